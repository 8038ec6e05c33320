// Clipped-PPO loss head of one minibatch, forward and gradient in one pass.
//
// The reference computes it with ~40 PyTorch ops and their autograd backward
// (src/nesle/native_ppo.py:546-566): Categorical(logits) log-probability and
// entropy, ratio, normalised advantages, the clipped surrogate, the value
// loss and their means.  Here three kernels do all of it on the caller's
// stream, with no atomics and no memsets (so the sequence can be captured in
// a graph and gives the same bits on every run):
//
//   1. adv_stats: one workgroup, mean and unbiased standard deviation of the
//      advantages (Tensor.std's N - 1);
//   2. head_rows: one thread per row; log-softmax, entropy, ratio, clipped
//      objective, d loss / d logits and d loss / d value for grad_output = 1,
//      and per-workgroup partial sums (objective, entropy, squared value
//      error, clipped count), reduced in a fixed order;
//   3. head_final: one workgroup sums the partials in block order and writes
//      loss and clip fraction (and adds them to an optional accumulator).
//
// Gradient conventions follow PyTorch's: max(a, b) sends the gradient to
// the larger operand and half to each on a tie; clamp passes it inside
// [lo, hi], bounds included.
#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <string>

#include "nes_launch.h"
#include "../../include/nesle_ppo.h"

namespace {

constexpr unsigned kRows = 256;    // rows (threads) per head_rows workgroup
constexpr unsigned kStats = 1024;  // threads of adv_stats / head_final

// Fixed-order tree sum of one value per thread over the workgroup.
template <unsigned N>
__device__ float block_sum(float v, float* sh) {
    const unsigned t = threadIdx.x;
    sh[t] = v;
    __syncthreads();
    for (unsigned s = N / 2; s > 0; s >>= 1) {
        if (t < s) sh[t] += sh[t + s];
        __syncthreads();
    }
    const float r = sh[0];
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(kStats) adv_stats(const float* adv, std::uint32_t n, float* stats) {
    __shared__ float sh[kStats];
    float acc = 0.0f;
    for (std::uint32_t i = threadIdx.x; i < n; i += kStats) acc += adv[i];
    const float mean = block_sum<kStats>(acc, sh) / static_cast<float>(n);
    float dev = 0.0f;
    for (std::uint32_t i = threadIdx.x; i < n; i += kStats) {
        const float d = adv[i] - mean;
        dev += d * d;
    }
    const float ss = block_sum<kStats>(dev, sh);
    if (threadIdx.x == 0) {
        stats[0] = mean;
        stats[1] = sqrtf(ss / static_cast<float>(n - 1));   // n = 1: 0 / 0, as Tensor.std
    }
}

struct HeadArgs {
    const float* logits;       // [n, a]
    const float* value;        // [n]
    const std::int64_t* actions;
    const float* old_logprob;
    const float* adv;
    const float* ret;
    std::uint32_t n, a;
    float lo, hi, clip;        // 1 - clip, 1 + clip (rounded from double), clip
    float ent_scale, vf_scale; // ent_coef / n, vf_coef / n
    float inv_n;
    const float* stats;        // mean, std
    float* dlogits;            // [n, a]
    float* dvalue;             // [n]
    float* partials;           // [blocks][4]
};

__global__ void __launch_bounds__(kRows) head_rows(HeadArgs h) {
    __shared__ float sh[kRows];
    const std::uint32_t i = blockIdx.x * kRows + threadIdx.x;
    float pg = 0.0f, ent = 0.0f, sq = 0.0f, clipped = 0.0f;
    if (i < h.n) {
        const float* l = h.logits + static_cast<std::size_t>(i) * h.a;
        float* dl = h.dlogits + static_cast<std::size_t>(i) * h.a;
        float mx = -INFINITY;
        for (std::uint32_t j = 0; j < h.a; ++j) mx = fmaxf(mx, l[j]);
        float se = 0.0f;
        for (std::uint32_t j = 0; j < h.a; ++j) se += expf(l[j] - mx);
        const float lse = mx + logf(se);
        float H = 0.0f;
        for (std::uint32_t j = 0; j < h.a; ++j) {
            const float lp = l[j] - lse;
            H -= expf(lp) * lp;
        }
        const std::int64_t act = h.actions[i];
        const bool valid = act >= 0 && act < static_cast<std::int64_t>(h.a);
        const std::uint32_t ai = valid ? static_cast<std::uint32_t>(act) : 0u;
        const float ratio = valid ? expf((l[ai] - lse) - h.old_logprob[i]) : NAN;
        const float adv_n = (h.adv[i] - h.stats[0]) / (h.stats[1] + 1e-8f);
        const float na = -adv_n;
        const float pg1 = na * ratio;
        const float pg2 = na * fminf(fmaxf(ratio, h.lo), h.hi);
        pg = fmaxf(pg1, pg2);
        const float inside = (ratio >= h.lo && ratio <= h.hi) ? 1.0f : 0.0f;
        const float w = pg1 > pg2 ? 1.0f : (pg1 < pg2 ? inside : 0.5f * (1.0f + inside));
        const float g = na * w * ratio * h.inv_n;       // d loss / d log p(action)
        for (std::uint32_t j = 0; j < h.a; ++j) {
            const float lp = l[j] - lse;
            const float p = expf(lp);
            float d = -g * p + h.ent_scale * p * (lp + H);
            if (j == ai) d += g;
            dl[j] = d;
        }
        const float dv = h.value[i] - h.ret[i];
        h.dvalue[i] = h.vf_scale * dv;
        ent = H;
        sq = dv * dv;
        clipped = fabsf(ratio - 1.0f) > h.clip ? 1.0f : 0.0f;
    }
    const float s0 = block_sum<kRows>(pg, sh);
    const float s1 = block_sum<kRows>(ent, sh);
    const float s2 = block_sum<kRows>(sq, sh);
    const float s3 = block_sum<kRows>(clipped, sh);
    if (threadIdx.x == 0) {
        float* p = h.partials + 4 * blockIdx.x;
        p[0] = s0; p[1] = s1; p[2] = s2; p[3] = s3;
    }
}

__global__ void __launch_bounds__(kStats) head_final(const float* partials, std::uint32_t blocks, float inv_n,
                                                     float ent_coef, float vf_coef, float* loss, float* clipfrac,
                                                     float* accum) {
    __shared__ float sh[kStats];
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (std::uint32_t b = threadIdx.x; b < blocks; b += kStats)
        for (int k = 0; k < 4; ++k) v[k] += partials[4 * b + k];
    const float pg = block_sum<kStats>(v[0], sh) * inv_n;
    const float ent = block_sum<kStats>(v[1], sh) * inv_n;
    const float vl = 0.5f * (block_sum<kStats>(v[2], sh) * inv_n);
    const float cf = block_sum<kStats>(v[3], sh) * inv_n;
    if (threadIdx.x == 0) {
        const float total = pg - ent_coef * ent + vf_coef * vl;
        *loss = total;
        *clipfrac = cf;
        if (accum != nullptr) {
            accum[0] += total;
            accum[1] += cf;
        }
    }
}

std::uint32_t scratch_floats(std::uint32_t batch) { return 2u + 4u * ((batch + kRows - 1) / kRows); }

constexpr std::uint32_t kStaticScratchFloats = 2u + 4u * ((NESLE_PPO_STATIC_MAX_BATCH + kRows - 1) / kRows);

// Device address of `scratch` (defined below) on each device, looked up on
// the first call made with that device current (the array's name in host
// code is only a stand-in for the symbol).
constexpr int kMaxDevices = 64;
std::array<float*, kMaxDevices> g_scratch_ptr{};
std::mutex g_scratch_mu;

int check_args(const char* who, const float* logits, const float* value, const std::int64_t* actions,
               const float* old_logprob, const float* advantages, const float* returns, std::uint32_t batch,
               std::uint32_t num_actions, const float* dlogits, const float* dvalue, const float* loss,
               const float* clipfrac) {
    if (batch == 0 || num_actions == 0 || num_actions > NESLE_PPO_MAX_ACTIONS) {
        nesle::set_last_error(std::string(who) + ": batch must be >= 1 and num_actions in 1.." +
                              std::to_string(NESLE_PPO_MAX_ACTIONS));
        return NESLE_EINVAL;
    }
    if (!logits || !value || !actions || !old_logprob || !advantages || !returns || !dlogits || !dvalue || !loss ||
        !clipfrac) {
        nesle::set_last_error(std::string(who) + ": null device pointer");
        return NESLE_EINVAL;
    }
    return NESLE_OK;
}

int launch_head(const char* who, const float* logits, const float* value, const std::int64_t* actions,
                const float* old_logprob, const float* advantages, const float* returns, std::uint32_t batch,
                std::uint32_t num_actions, double clip_coef, double ent_coef, double vf_coef, float* dlogits,
                float* dvalue, float* scratch_buf, float* loss, float* clipfrac, float* accum, void* stream) {
    const auto s = static_cast<hipStream_t>(stream);
    const std::uint32_t blocks = (batch + kRows - 1) / kRows;
    const float inv_n = 1.0f / static_cast<float>(batch);
    HeadArgs h{logits, value, actions, old_logprob, advantages, returns, batch, num_actions,
               static_cast<float>(1.0 - clip_coef), static_cast<float>(1.0 + clip_coef), static_cast<float>(clip_coef),
               static_cast<float>(ent_coef) * inv_n, static_cast<float>(vf_coef) * inv_n, inv_n,
               scratch_buf, dlogits, dvalue, scratch_buf + 2};
    hipLaunchKernelGGL(adv_stats, dim3(1), dim3(kStats), 0, s, advantages, batch, scratch_buf);
    hipLaunchKernelGGL(head_rows, dim3(blocks), dim3(kRows), 0, s, h);
    hipLaunchKernelGGL(head_final, dim3(1), dim3(kStats), 0, s, scratch_buf + 2, blocks, inv_n,
                       static_cast<float>(ent_coef), static_cast<float>(vf_coef), loss, clipfrac, accum);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        nesle::set_last_error(std::string(who) + ": launch failed: " + hipGetErrorString(e));
        return NESLE_EDEVICE;
    }
    return NESLE_OK;
}

}  // namespace

// Scratch of the allocation-free entry point: the advantage statistics (2
// floats) and the per-workgroup partial sums (4 floats per 256 rows) of
// minibatches up to NESLE_PPO_STATIC_MAX_BATCH rows, about 64 KiB per
// device.  Every call writes all of the scratch it reads before reading it,
// so nothing needs clearing between calls.
static __device__ __align__(256) float scratch[kStaticScratchFloats];

extern "C" {

std::uint32_t nesle_ppo_head_scratch_floats(std::uint32_t batch) { return scratch_floats(batch); }

int nesle_ppo_head(const float* logits, const float* value, const std::int64_t* actions, const float* old_logprob,
                   const float* advantages, const float* returns, std::uint32_t batch, std::uint32_t num_actions,
                   double clip_coef, double ent_coef, double vf_coef, float* dlogits, float* dvalue,
                   float* scratch_buf, float* loss, float* clipfrac, float* accum, void* stream) {
    const int rc = check_args("nesle_ppo_head", logits, value, actions, old_logprob, advantages, returns, batch,
                              num_actions, dlogits, dvalue, loss, clipfrac);
    if (rc != NESLE_OK) return rc;
    if (scratch_buf == nullptr) {
        nesle::set_last_error("nesle_ppo_head: null device pointer");
        return NESLE_EINVAL;
    }
    return launch_head("nesle_ppo_head", logits, value, actions, old_logprob, advantages, returns, batch,
                       num_actions, clip_coef, ent_coef, vf_coef, dlogits, dvalue, scratch_buf, loss, clipfrac,
                       accum, stream);
}

int nesle_ppo_head_static(const float* logits, const float* value, const std::int64_t* actions,
                          const float* old_logprob, const float* advantages, const float* returns, std::uint32_t batch,
                          std::uint32_t num_actions, double clip_coef, double ent_coef, double vf_coef,
                          float* dlogits, float* dvalue, float* loss, float* clipfrac, float* accum, void* stream) {
    const char* who = "nesle_ppo_head_static";
    const int rc = check_args(who, logits, value, actions, old_logprob, advantages, returns, batch, num_actions,
                              dlogits, dvalue, loss, clipfrac);
    if (rc != NESLE_OK) return rc;
    if (batch > NESLE_PPO_STATIC_MAX_BATCH) {
        nesle::set_last_error(std::string(who) + ": batch " + std::to_string(batch) + " exceeds the static scratch (" +
                              std::to_string(NESLE_PPO_STATIC_MAX_BATCH) + " rows); use nesle_ppo_head with a workspace");
        return NESLE_EINVAL;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        nesle::set_last_error(std::string(who) + ": no usable current device" +
                              (e != hipSuccess ? std::string(": ") + hipGetErrorString(e) : std::string()));
        return NESLE_EDEVICE;
    }
    float* ptr = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ptr = g_scratch_ptr[dev];
        if (ptr == nullptr) {
            void* addr = nullptr;
            e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (e != hipSuccess || addr == nullptr) {
                nesle::set_last_error(std::string(who) + ": hipGetSymbolAddress(scratch) failed: " +
                                      hipGetErrorString(e));
                return NESLE_EDEVICE;
            }
            ptr = static_cast<float*>(addr);
            g_scratch_ptr[dev] = ptr;
        }
    }
    return launch_head(who, logits, value, actions, old_logprob, advantages, returns, batch, num_actions, clip_coef,
                       ent_coef, vf_coef, dlogits, dvalue, ptr, loss, clipfrac, accum, stream);
}

}  // extern "C"
