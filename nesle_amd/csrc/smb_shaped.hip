// smb_shaped.hip -- the trainer's shaped Super Mario Bros. reward, on the device.
//
// The reference trainer's reward_mode="smart" (src/nesle/native_ppo.py:
// 120-316, TorchSmartMarioReward) scores each env-step from the step's RAM,
// pad masks and done flags with about sixty PyTorch element-wise launches and
// boolean-mask assignments (host synchronisations).  Here it is one thread
// per console: the eleven tracking values live in a [11][n] word array (one
// coalesced row per value), the RAM bytes come from the env-major RAM view,
// and the terms are summed in the reference's order with every float32
// operation rounded as PyTorch rounds it (no fused multiply-adds), so the
// reward is bit-identical to the reference's float32 tensor arithmetic.
// Nothing is allocated and nothing synchronises: a rollout graph can hold it.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <exception>
#include <string>

#include "../../include/nesle_ppo.h"
#include "nes_launch.h"

// No multiply-add contraction anywhere in this file: each float32 product
// and sum is rounded on its own, as PyTorch's separate kernels round them.
#pragma clang fp contract(off)

namespace nesle {
namespace {

// RAM map of the game (native_ppo.py:123-133).
constexpr std::uint32_t kXPage = 0x006D, kXScreen = 0x0086, kYViewport = 0x00B5, kPlayerState = 0x000E;
constexpr std::uint32_t kLives = 0x075A, kWorld = 0x075F, kStage = 0x075C, kArea = 0x0760, kGameMode = 0x0770;
constexpr std::uint32_t kCoins = 0x07ED, kScore = 0x07DE;

// Rows of the tracking state.
enum : std::uint32_t {
    kLastX = 0, kMaxX, kCheckpoint, kLastScore, kLastCoins, kLastLives, kLastLevel, kStall, kJumpStreak,
    kFinishAwarded, kFlagAwarded
};
static_assert(kFlagAwarded + 1 == NESLE_SMB_SHAPED_STATE_WORDS, "state rows");

struct Track {
    std::uint32_t* w;   // [NESLE_SMB_SHAPED_STATE_WORDS][n]
    std::uint32_t n;
    __device__ std::uint32_t& at(std::uint32_t row, std::uint32_t e) const { return w[static_cast<std::size_t>(row) * n + e]; }
    __device__ float f(std::uint32_t row, std::uint32_t e) const { return __uint_as_float(at(row, e)); }
    __device__ std::int32_t i(std::uint32_t row, std::uint32_t e) const { return static_cast<std::int32_t>(at(row, e)); }
    __device__ void set_f(std::uint32_t row, std::uint32_t e, float v) const { at(row, e) = __float_as_uint(v); }
    __device__ void set_i(std::uint32_t row, std::uint32_t e, std::int32_t v) const { at(row, e) = static_cast<std::uint32_t>(v); }
};

// Decimal digits, one per RAM byte (low nibble), most significant first.
__device__ std::int32_t bcd(const std::uint8_t* ram, std::uint32_t at, std::uint32_t digits) {
    std::int32_t v = 0;
    for (std::uint32_t k = 0; k < digits; ++k) v = v * 10 + (ram[at + k] & 0x0F);
    return v;
}

// Float32 operations rounded one at a time, as PyTorch's element-wise
// kernels do (a Python scalar operand is a float32 constant); written here,
// under the pragma above, so that no product fuses with a sum.
__device__ __forceinline__ float mul(float a, float b) { return a * b; }
__device__ __forceinline__ float add(float a, float b) { return a + b; }
__device__ __forceinline__ float sub(float a, float b) { return a - b; }
__device__ __forceinline__ float div(float a, float b) { return a / b; }

struct Ram {
    const std::uint8_t* row;
    __device__ float x() const { return add(mul(static_cast<float>(row[kXPage]), 256.0f), static_cast<float>(row[kXScreen])); }
    __device__ std::int32_t coins() const { return bcd(row, kCoins, 2); }
    __device__ float score() const { return static_cast<float>(bcd(row, kScore, 6)); }
    __device__ std::int32_t lives() const { return row[kLives]; }
    __device__ std::int32_t level() const { return row[kWorld] * 65536 + row[kStage] * 256 + row[kArea]; }
    __device__ bool death() const {
        const std::uint32_t s = row[kPlayerState];
        return s == 0x0B || s == 0x06 || row[kYViewport] > 1 || row[kLives] == 0xFF;
    }
};

// reset_where (native_ppo.py:174-207): start an episode from the RAM.
__global__ void __launch_bounds__(256) shaped_reset_kernel(const std::uint8_t* ram, const std::uint8_t* mask,
                                                          std::uint32_t n, Track t) {
    const std::uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e >= n || (mask != nullptr && mask[e] == 0)) return;
    const Ram r{ram + static_cast<std::size_t>(e) * 2048};
    const float x = r.x();
    t.set_f(kLastX, e, x);
    t.set_f(kMaxX, e, x);
    t.set_i(kCheckpoint, e, 0);
    t.set_f(kLastScore, e, r.score());
    t.set_i(kLastCoins, e, r.coins());
    t.set_i(kLastLives, e, r.lives());
    t.set_i(kLastLevel, e, r.level());
    t.set_i(kStall, e, 0);
    t.set_i(kJumpStreak, e, 0);
    t.set_i(kFinishAwarded, e, 0);
    t.set_i(kFlagAwarded, e, 0);
}

// compute (native_ppo.py:209-278) and _action_reward (:296-316).
__global__ void __launch_bounds__(256) shaped_reward_kernel(const std::uint8_t* ram, const std::uint8_t* pads,
                                                           const std::uint8_t* dones, std::uint32_t n,
                                                           nesle_smb_shaped_params p, Track t, float* out) {
    const std::uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const Ram r{ram + static_cast<std::size_t>(e) * 2048};
    const bool done = dones[e] != 0;

    // Forward progress and backtracking; stall counter.
    const float x = r.x();
    const float dx = sub(x, t.f(kLastX, e));
    const bool forward = dx > 0.0f;
    const float progress = forward ? mul(fminf(dx, 16.0f), p.progress_scale) : mul(fmaxf(dx, -16.0f), p.backtrack_scale);
    const std::int32_t stall = forward ? 0 : t.i(kStall, e) + 1;
    t.set_i(kStall, e, stall);
    // Checkpoints every checkpoint_width pixels of the furthest x.
    const float max_x = fmaxf(t.f(kMaxX, e), x);
    t.set_f(kMaxX, e, max_x);
    const std::int32_t ci_new = static_cast<std::int32_t>(floorf(div(max_x, p.checkpoint_width)));
    const std::int32_t ci_old = t.i(kCheckpoint, e);
    const std::int32_t ci_delta = ci_new - ci_old > 0 ? ci_new - ci_old : 0;
    const float checkpoint = mul(static_cast<float>(ci_delta), p.checkpoint_bonus);
    t.set_i(kCheckpoint, e, ci_new > ci_old ? ci_new : ci_old);

    // Score, coins, kills.
    const float score = r.score();
    const float score_delta = fmaxf(sub(score, t.f(kLastScore, e)), 0.0f);
    const std::int32_t coins = r.coins();
    std::int32_t coin_delta = coins - t.i(kLastCoins, e);
    if (coin_delta < 0) coin_delta += 100;
    if (coin_delta < 0) coin_delta = 0;
    const float score_reward = mul(score_delta, p.score_scale);
    const float kill_score = sub(score_delta, mul(static_cast<float>(coin_delta), 200.0f));
    const float kill_reward = kill_score >= 100.0f ? p.kill_bonus : 0.0f;
    const float coin_reward = mul(static_cast<float>(coin_delta), p.coin_bonus);

    // Finish zone and flag, once per episode each.
    const bool finish_hit = t.i(kFinishAwarded, e) == 0 && max_x >= p.finish_zone_x;
    const float finish_reward = finish_hit ? p.finish_zone_bonus : 0.0f;
    if (finish_hit) t.set_i(kFinishAwarded, e, 1);
    const bool death = r.death();
    const bool flag_hit = t.i(kFlagAwarded, e) == 0 &&
                          (r.row[kGameMode] == 2 || (max_x >= p.flag_zone_x && done && !death));
    const float flag_reward = flag_hit ? p.flag_bonus : 0.0f;
    if (flag_hit) t.set_i(kFlagAwarded, e, 1);

    // Stalling.
    const float stall_over = fmaxf(static_cast<float>(stall - p.stall_window + 1), 0.0f);
    const float stall_reward = -fminf(mul(stall_over, p.stall_penalty), p.max_stall_penalty);

    // Buttons: A (jump), Right, Left, Start, Select.
    const std::uint32_t pad = pads[e];
    const bool jump = pad & 0x01, right = pad & 0x80, left = pad & 0x40, start = pad & 0x08, select = pad & 0x04;
    const std::int32_t streak = jump ? t.i(kJumpStreak, e) + 1 : 0;
    t.set_i(kJumpStreak, e, streak);
    float action = 0.0f;
    action = sub(action, mul(jump ? 1.0f : 0.0f, p.jump_penalty));
    action = sub(action, mul((jump && !right) ? 1.0f : 0.0f, p.neutral_jump_penalty));
    const float repeated = fmaxf(static_cast<float>(streak - p.repeated_jump_window), 0.0f);
    action = sub(action, fminf(mul(repeated, p.repeated_jump_penalty), p.max_repeated_jump_penalty));
    action = sub(action, mul(left ? 1.0f : 0.0f, p.left_penalty));
    action = sub(action, mul((left && right) ? 1.0f : 0.0f, p.bad_button_penalty));
    action = sub(action, mul((start || select) ? 1.0f : 0.0f, p.bad_button_penalty));

    const float death_reward = (done && death) ? -p.death_penalty : 0.0f;
    const float time_reward = -p.time_penalty;

    t.set_f(kLastX, e, x);
    t.set_f(kLastScore, e, score);
    t.set_i(kLastCoins, e, coins);
    t.set_i(kLastLives, e, r.lives());
    t.set_i(kLastLevel, e, r.level());

    float total = add(progress, checkpoint);
    total = add(total, score_reward);
    total = add(total, kill_reward);
    total = add(total, coin_reward);
    total = add(total, finish_reward);
    total = add(total, flag_reward);
    total = add(total, stall_reward);
    total = add(total, action);
    total = add(total, death_reward);
    total = add(total, time_reward);
    out[e] = total;
}

int fail(int code, const std::string& msg) {
    set_last_error(msg);
    return code;
}

}  // namespace
}  // namespace nesle

extern "C" {

void nesle_smb_shaped_defaults(nesle_smb_shaped_params* p) {
    if (p == nullptr) return;
    *p = nesle_smb_shaped_params{};
    p->progress_scale = 0.18f;
    p->backtrack_scale = 0.03f;
    p->checkpoint_bonus = 3.0f;
    p->checkpoint_width = 128.0f;
    p->score_scale = 0.04f;
    p->coin_bonus = 3.0f;
    p->kill_bonus = 8.0f;
    p->finish_zone_x = 3100.0f;
    p->finish_zone_bonus = 100.0f;
    p->flag_zone_x = 3300.0f;
    p->flag_bonus = 100.0f;
    p->death_penalty = 75.0f;
    p->time_penalty = 0.005f;
    p->stall_penalty = 0.02f;
    p->max_stall_penalty = 0.5f;
    p->jump_penalty = 0.005f;
    p->neutral_jump_penalty = 0.02f;
    p->repeated_jump_penalty = 0.02f;
    p->max_repeated_jump_penalty = 0.25f;
    p->left_penalty = 0.01f;
    p->bad_button_penalty = 0.25f;
    p->stall_window = 40;
    p->repeated_jump_window = 6;
}

int nesle_smb_shaped_reset(const std::uint8_t* ram, const std::uint8_t* mask, std::uint32_t n, void* state,
                           void* stream) {
    if (n == 0 || ram == nullptr || state == nullptr) return nesle::fail(NESLE_EINVAL, "nesle_smb_shaped_reset: null pointer or n = 0");
    const nesle::Track t{static_cast<std::uint32_t*>(state), n};
    nesle::shaped_reset_kernel<<<dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(ram, mask, n, t);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? NESLE_OK : nesle::fail(NESLE_EDEVICE, std::string("shaped_reset_kernel: ") + hipGetErrorString(e));
}

int nesle_smb_shaped_reward(const std::uint8_t* ram, const std::uint8_t* pads, const std::uint8_t* dones,
                            std::uint32_t n, const nesle_smb_shaped_params* params, void* state, float* reward,
                            void* stream) {
    if (n == 0 || ram == nullptr || pads == nullptr || dones == nullptr || params == nullptr || state == nullptr ||
        reward == nullptr)
        return nesle::fail(NESLE_EINVAL, "nesle_smb_shaped_reward: null pointer or n = 0");
    if (params->checkpoint_width <= 0.0f) return nesle::fail(NESLE_EINVAL, "checkpoint_width must be positive");
    const nesle::Track t{static_cast<std::uint32_t*>(state), n};
    nesle::shaped_reward_kernel<<<dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        ram, pads, dones, n, *params, t, reward);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? NESLE_OK : nesle::fail(NESLE_EDEVICE, std::string("shaped_reward_kernel: ") + hipGetErrorString(e));
}

}  // extern "C"
