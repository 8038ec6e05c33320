// nes_kernels.hip -- utility kernels of libnesle_hip.so: masked restore of
// consoles from the snapshot bank, from one blob, or to power-on (the
// reference's reset kernels, cpp/src/cuda/kernels.cu:177-203, and the
// auto-reset that follows a step), full-state save of one console,
// the env-major RAM observation, int64 action ingestion
// (cpp/bindings/cuda_module.cu:310-317) and RAM poke (cuda_module.cu:356-364).
// The console step kernel lives in nes_step.hip.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "nes_device.h"
#include "nes_launch.h"
#include "nes_layout.h"

namespace nesle {
namespace {

constexpr std::uint32_t kBlock = 256;

// Masked restore, tiled for the address-major layout: blockIdx.x picks 64
// consecutive consoles (one wave, lane = console), blockIdx.y one share of
// the work — a run of kRestoreRows interleaved RAM/PRG-RAM rows, a run of
// CHR-RAM rows, or (the last y) the scalars, video memory and reward
// baselines.  A tile without a selected console leaves at once.  The
// consoles' sources are the bank slot of their level, one fixed blob, or
// power-on zeros; the baselines are seeded from the source blob's RAM, so
// no block reads rows another block writes.  A restore of a few consoles
// thus costs about one row run's byte stores, spread over many waves.
constexpr std::uint32_t kRestoreRows = 512;
constexpr std::uint32_t kRamRowBlocks = (kRamBytes + kPrgRamBytes) / kRestoreRows;   // 20
constexpr std::uint32_t kChrRowBlocks = kChrRamBytes / kRestoreRows;                  // 16

__global__ void __launch_bounds__(64) restore_kernel(DeviceState s, const std::uint8_t* mask,
                                                     const std::uint8_t* fixed_blob) {
    const std::uint32_t env = blockIdx.x * 64 + threadIdx.x;
    const bool mine = env < s.n && (mask == nullptr || mask[env] != 0);
    if (__ballot(mine) == 0) return;
    // Source of console e: the fixed blob, its level's bank slot, or null
    // (power-on).
    auto source = [&](std::uint32_t e) -> const std::uint8_t* {
        if (fixed_blob != nullptr) return fixed_blob;
        if (s.bank == nullptr) return nullptr;
        return s.bank + static_cast<std::size_t>(s.env_to_level[e]) * blob::kBytes;
    };
    const std::uint8_t* src = mine ? source(env) : nullptr;
    const std::uint32_t y = blockIdx.y, pitch = s.pitch;
    if (y < kRamRowBlocks) {
        if (!mine) return;
        std::uint8_t* dst = s.ram + static_cast<std::size_t>(y * kRestoreRows) * pitch + env;
        if (src != nullptr) {
            blob_rows(dst, pitch, src + blob::kRam + y * kRestoreRows, kRestoreRows);
        } else {
            zero_rows(dst, pitch, kRestoreRows);
        }
        return;
    }
    if (y < kRamRowBlocks + kChrRowBlocks) {
        if (!mine || s.chr_ram == nullptr) return;
        const std::uint32_t r0 = (y - kRamRowBlocks) * kRestoreRows;
        std::uint8_t* dst = s.chr_ram + static_cast<std::size_t>(r0) * pitch + env;
        if (src != nullptr) {
            blob_rows(dst, pitch, src + blob::kChrRam + r0, kRestoreRows);
        } else {
            zero_rows(dst, pitch, kRestoreRows);
        }
        return;
    }
    // Scalars and baselines per console; video memory by the whole wave, one
    // selected console at a time (contiguous 16-byte runs).
    if (mine) {
        if (src != nullptr) {
            blob_scalars(s, env, src);
            reward_seed(s, env, [&](std::uint32_t a) -> std::uint32_t { return src[blob::kRam + (a & 0x7FF)]; });
        } else {
            power_on_scalars(s, env);
            reward_seed(s, env, [](std::uint32_t) -> std::uint32_t { return 0; });
        }
    }
    const std::uint32_t lane = threadIdx.x;
    std::uint64_t todo = __ballot(mine);
    while (todo != 0) {
        const std::uint32_t k = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(todo)) - 1);
        todo &= todo - 1;
        const std::uint32_t e = blockIdx.x * 64 + k;   // wave-uniform
        const std::uint8_t* from = source(e);
        uint4* vm = reinterpret_cast<uint4*>(vram_of(s, e));
        // Video memory block: palette (2 x 16 B), OAM (16), nametables (128 or 256).
        const std::uint32_t words = s.vram_stride / 16;
        for (std::uint32_t i = lane; i < words; i += 64) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (from != nullptr) {
                const std::uint32_t o = 16 * i;
                const std::uint32_t at = o < vram::kOam ? blob::kPalette + o
                                       : o < vram::kNametable ? blob::kOam + (o - vram::kOam)
                                                              : blob::kNametable + (o - vram::kNametable);
                v = *reinterpret_cast<const uint4*>(from + at);
            }
            vm[i] = v;
        }
    }
}

// Gather console `env` into a canonical blob, one byte per thread.
__global__ void __launch_bounds__(kBlock) save_blob_kernel(DeviceState s, std::uint32_t env, std::uint8_t* out) {
    using namespace blob;
    const std::uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= kBytes) return;
    const std::size_t pitch = s.pitch;
    auto byte_of = [](std::uint64_t v, std::uint32_t k) { return static_cast<std::uint8_t>(v >> (8 * k)); };
    std::uint8_t v = 0;
    if (i < 4) {
        v = static_cast<std::uint8_t>("NST1"[i]);
    } else if (i < kA) {
        v = byte_of(s.pc[env], i - kPc);
    } else if (i < kCycles) {
        const std::uint8_t regs[6] = {s.a[env], s.x[env], s.y[env], s.sp[env], s.p[env], s.nmi_pending[env]};
        v = regs[i - kA];
    } else if (i < kFrame) {
        v = byte_of(s.cycles[env], i - kCycles);
    } else if (i < kFrameDot) {
        v = byte_of(s.frame[env], i - kFrame);
    } else if (i < kCtrl) {
        v = byte_of(s.frame_dot[env], i - kFrameDot);
    } else if (i < kV) {
        const std::uint8_t r[6] = {s.ctrl[env], s.mask[env], s.status[env], s.oam_addr[env], s.open_bus[env],
                                   s.read_buffer[env]};
        v = r[i - kCtrl];
    } else if (i < kT) {
        v = byte_of(s.v[env], i - kV);
    } else if (i < kFineX) {
        v = byte_of(s.t[env], i - kT);
    } else if (i < kPendingDma) {
        const std::uint8_t r[10] = {s.fine_x[env], s.w[env], s.scroll_x[env], s.scroll_y[env], s.c1_buttons[env],
                                    s.c1_shift[env], s.c1_count[env], s.strobe[env], s.c2_count[env], s.fault[env]};
        v = r[i - kFineX];
    } else if (i < kApuIo) {
        v = 0;  // no DMA stall is ever owed between instructions
    } else if (i < kRam) {
        v = s.apu_io[(i - kApuIo) * pitch + env];
    } else if (i < kPrgRam) {
        v = s.ram[(i - kRam) * pitch + env];
    } else if (i < kOam) {
        v = s.prg_ram[(i - kPrgRam) * pitch + env];
    } else if (i < kPalette) {
        v = vram_of(s, env)[vram::kOam + i - kOam];
    } else if (i < kNametable) {
        v = vram_of(s, env)[vram::kPalette + i - kPalette];
    } else if (i < kChrRam) {
        const std::uint32_t k = i - kNametable;
        v = k < s.nt_bytes ? vram_of(s, env)[vram::kNametable + k] : 0;
    } else {
        v = s.chr_ram != nullptr ? s.chr_ram[(i - kChrRam) * pitch + env] : 0;
    }
    out[i] = v;
}

// RAM observation: [2048][pitch] interleaved -> [n][2048] env-major.  A
// workgroup moves a tile of 256 consoles x 64 addresses in dwords: each lane
// loads four consoles' bytes at four consecutive addresses (four coalesced
// dword rows), transposes that 4x4 byte block in registers, and writes one
// dword per console (four addresses) into the LDS tile; the tile is then
// stored as dwords, 16 lanes per console row.  Loads stay inside the
// console pitch (a multiple of 256); stores stop at the last console.
constexpr std::uint32_t kObsEnvs = 256, kObsAddrs = 64;
constexpr std::uint32_t kObsRow = kObsAddrs / 4 + 1;   // dwords per console row in LDS (odd: bank spread)

__global__ void __launch_bounds__(kBlock) ram_obs_kernel(const std::uint8_t* __restrict__ ram,
                                                         std::uint8_t* __restrict__ obs, std::uint32_t n,
                                                         std::uint32_t pitch) {
    __shared__ std::uint32_t tile[kObsEnvs * kObsRow];
    const std::uint32_t env0 = blockIdx.x * kObsEnvs, addr0 = blockIdx.y * kObsAddrs;
    const std::uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Wave w takes addresses addr0 + 16w .. +15, four at a time; lane l takes
    // consoles env0 + 4l .. 4l + 3.
    const std::uint8_t* src = ram + static_cast<std::size_t>(addr0 + 16 * wave) * pitch + env0 + 4 * lane;
#pragma unroll
    for (std::uint32_t g = 0; g < 4; ++g) {
        const std::uint8_t* at = src + static_cast<std::size_t>(4 * g) * pitch;
        const std::uint32_t w0 = *reinterpret_cast<const std::uint32_t*>(at);
        const std::uint32_t w1 = *reinterpret_cast<const std::uint32_t*>(at + pitch);
        const std::uint32_t w2 = *reinterpret_cast<const std::uint32_t*>(at + 2 * static_cast<std::size_t>(pitch));
        const std::uint32_t w3 = *reinterpret_cast<const std::uint32_t*>(at + 3 * static_cast<std::size_t>(pitch));
        // w_a holds byte j = console 4l + j at address a; c_j holds console
        // 4l + j's bytes at the four addresses.
        const std::uint32_t t0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);
        const std::uint32_t t1 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);
        const std::uint32_t t2 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
        const std::uint32_t t3 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
        const std::uint32_t c[4] = {__builtin_amdgcn_perm(t2, t0, 0x05040100u), __builtin_amdgcn_perm(t2, t0, 0x07060302u),
                                    __builtin_amdgcn_perm(t3, t1, 0x05040100u), __builtin_amdgcn_perm(t3, t1, 0x07060302u)};
        // Write order rotated by lane >> 3, so that the 32 lanes of a
        // half-wave hit 32 different banks.
        const std::uint32_t col = 4 * wave + g;
#pragma unroll
        for (std::uint32_t i = 0; i < 4; ++i) {
            const std::uint32_t j = (i + (lane >> 3)) & 3;
            const std::uint32_t v = j == 0 ? c[0] : j == 1 ? c[1] : j == 2 ? c[2] : c[3];
            tile[(4 * lane + j) * kObsRow + col] = v;
        }
    }
    __syncthreads();
    const std::uint32_t c16 = threadIdx.x & 15;
#pragma unroll 4
    for (std::uint32_t e = threadIdx.x >> 4; e < kObsEnvs; e += kBlock / 16) {
        const std::uint32_t env = env0 + e;
        if (env < n)
            *reinterpret_cast<std::uint32_t*>(obs + static_cast<std::size_t>(env) * kRamBytes + addr0 + 4 * c16) =
                tile[e * kObsRow + c16];
    }
}

__global__ void __launch_bounds__(kBlock) actions_i64_kernel(std::uint8_t* dst, const long long* src, std::uint32_t n) {
    const std::uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) dst[i] = static_cast<std::uint8_t>(src[i] & 0xFF);
}

__global__ void __launch_bounds__(kBlock) poke_ram_kernel(DeviceState s, std::uint32_t addr, std::uint32_t value) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env < s.n) s.ram[static_cast<std::size_t>(addr & 0x7FF) * s.pitch + env] = static_cast<std::uint8_t>(value);
}

__global__ void __launch_bounds__(kBlock) poke_ram_envs_kernel(DeviceState s, std::uint32_t addr,
                                                               const std::uint8_t* values) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env < s.n) s.ram[static_cast<std::size_t>(addr & 0x7FF) * s.pitch + env] = values[env];
}

// Zero fill of n 64-bit words: a kernel rather than hipMemsetAsync, so that a
// step that clears its profile histograms can be captured in a HIP graph.
__global__ void __launch_bounds__(kBlock) zero_u64_kernel(unsigned long long* p, std::uint32_t n) {
    const std::uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) p[i] = 0ull;
}

__global__ void __launch_bounds__(kBlock) seed_kernel(DeviceState s) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env < s.n) reward_seed(s, env, GlobalRam{s, env});
}

// Presentation records from live state: frame-start and frame-end
// scroll/ctrl both the current ones, the mask and a copy of the video memory
// block; one workgroup per console (selected by mask, null = all).  Into the
// presentation snapshot (with the pre-render latch) after full resets and
// state loads, so a render right after them is coherent (cuda_module.cu:
// 1440-1463); or into a separate buffer for a render of live state.
__global__ void __launch_bounds__(kBlock) record_kernel(DeviceState s, const std::uint8_t* mask, std::uint8_t* out,
                                                        std::uint32_t latch) {
    const std::uint32_t env = blockIdx.x;
    if (mask != nullptr && mask[env] == 0) return;
    const std::uint32_t vs = s.vram_stride;
    std::uint8_t* rec = out + static_cast<std::size_t>(env) * (present::kHeader + vs);
    const std::uint32_t t = threadIdx.x;
    if (t < present::kHeader) {
        const std::uint32_t sx = s.scroll_x[env], sy = s.scroll_y[env], ctrl = s.ctrl[env];
        const std::uint32_t k = t % 3;
        const std::uint32_t v = t == present::kMask ? s.mask[env] : t > present::kMask ? 0u : (k == 0 ? sx : k == 1 ? sy : ctrl);
        rec[t] = static_cast<std::uint8_t>(v);
        if (t == 0 && latch != 0) {
            s.lat_sx[env] = static_cast<std::uint8_t>(sx);
            s.lat_sy[env] = static_cast<std::uint8_t>(sy);
            s.lat_ctrl[env] = static_cast<std::uint8_t>(ctrl);
        }
    }
    const auto* from = reinterpret_cast<const std::uint32_t*>(vram_of(s, env));
    auto* to = reinterpret_cast<std::uint32_t*>(rec + present::kHeader);
    for (std::uint32_t i = t; i < vs / 4; i += kBlock) to[i] = from[i];
}

inline std::uint32_t blocks_for(std::uint32_t n) { return (n + kBlock - 1) / kBlock; }

// ---- the ROM-less synthetic batch (CudaBatch(num_envs, frameskip)) ----------
// Not a console: RAM holds only the bytes the SMB reward rule reads, moved
// by the pad (cpp/bindings/cuda_module.cu:319-354) and scored by that rule
// (cpp/src/cuda/kernels.cu:12-17).  One thread per console, RAM rows
// interleaved as everywhere else (row * pitch + env, coalesced over a wave).
constexpr std::uint32_t kSynthXPage = 0x6D, kSynthXScreen = 0x86, kSynthYViewport = 0xB5, kSynthLives = 0x75A;
constexpr std::uint32_t kSynthState = 0x0E, kSynthTime = 0x7F8;

// Power-on of the synthetic console (batch_step.cuh:244-260): RAM cleared,
// then x = $0102, y viewport 1, 2 lives, time 400; reward baselines to match.
// A full reset (mask null) also clears rewards, dones and step counts, as the
// reference's reset() does (cuda_module.cu:469-512); a masked reset leaves
// the step's rewards and dones readable (they are the last_* values).
__global__ void __launch_bounds__(kBlock) synthetic_reset_kernel(DeviceState s, const std::uint8_t* mask,
                                                                 std::uint32_t* step_counts) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env >= s.n || (mask != nullptr && mask[env] == 0)) return;
    std::uint8_t* ram = s.ram + env;
    const std::size_t P = s.pitch;
    for (std::uint32_t a = 0; a < kRamBytes; ++a) ram[a * P] = 0;
    ram[kSynthXPage * P] = 1;
    ram[kSynthXScreen * P] = 2;
    ram[kSynthYViewport * P] = 1;
    ram[kSynthLives * P] = 2;
    ram[kSynthTime * P] = 4;   // BCD digits 4, 0, 0
    s.prev_x[env] = 0x102;
    s.prev_time[env] = 400;
    if (mask == nullptr) {
        s.rewards[env] = 0.0f;
        s.done[env] = 0;
        step_counts[env] = 0;
    }
}

// One env-step.  With `apply_actions` (the reference's step()) the pad moves
// x first -- Right +1, +1 more with B, Left -1, clamped to 0..$FFFF -- and
// every max(1, 24 / frameskip)-th step of the console (from its first)
// takes one from the 3-digit BCD time (not below 0); then the SMB rule
// scores the RAM against the baselines.  step_device() runs the rule alone
// (cuda_module.cu:620-633 launches only the reward kernel without a ROM).
__global__ void __launch_bounds__(kBlock) synthetic_step_kernel(DeviceState s, std::uint32_t frameskip,
                                                                std::uint32_t* step_counts,
                                                                std::uint32_t apply_actions) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env >= s.n) return;
    std::uint8_t* ram = s.ram + env;
    const std::size_t P = s.pitch;
    if (apply_actions != 0) {
        const std::uint32_t pad = s.actions[env];
        std::int32_t dx = (pad & 0x80) ? 1 + ((pad & 0x02) ? 1 : 0) : 0;
        dx -= (pad & 0x40) ? 1 : 0;
        std::int32_t x = static_cast<std::int32_t>(ram[kSynthXPage * P]) * 256 + ram[kSynthXScreen * P] + dx;
        x = x < 0 ? 0 : (x > 0xFFFF ? 0xFFFF : x);
        ram[kSynthXPage * P] = static_cast<std::uint8_t>(x >> 8);
        ram[kSynthXScreen * P] = static_cast<std::uint8_t>(x);
        const std::uint32_t fs = frameskip == 0 ? 1u : frameskip;
        const std::uint32_t cadence = 24u / fs == 0 ? 1u : 24u / fs;
        const std::uint32_t k = step_counts[env];
        step_counts[env] = k + 1;
        if (k % cadence == 0) {
            std::int32_t t = (ram[kSynthTime * P] & 15) * 100 + (ram[(kSynthTime + 1) * P] & 15) * 10 +
                             (ram[(kSynthTime + 2) * P] & 15);
            t = t > 0 ? t - 1 : 0;
            ram[kSynthTime * P] = static_cast<std::uint8_t>(t / 100);
            ram[(kSynthTime + 1) * P] = static_cast<std::uint8_t>((t / 10) % 10);
            ram[(kSynthTime + 2) * P] = static_cast<std::uint8_t>(t % 10);
        }
    }
    float reward = 0.0f;
    std::uint32_t done = 0;
    reward_apply(s, env, GlobalRam{s, env}, &reward, &done);
    s.rewards[env] = reward;
    s.done[env] = static_cast<std::uint8_t>(done);
}

}  // namespace

hipError_t launch_synthetic_reset(const DeviceState& s, const std::uint8_t* mask, std::uint32_t* step_counts,
                                  hipStream_t stream) {
    synthetic_reset_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s, mask, step_counts);
    return hipGetLastError();
}

hipError_t launch_synthetic_step(const DeviceState& s, std::uint32_t frameskip, std::uint32_t* step_counts,
                                 bool apply_actions, hipStream_t stream) {
    synthetic_step_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s, frameskip, step_counts,
                                                                                apply_actions ? 1u : 0u);
    return hipGetLastError();
}

hipError_t launch_restore(const DeviceState& s, const std::uint8_t* mask, const std::uint8_t* fixed_blob,
                          hipStream_t stream) {
    const dim3 grid((s.n + 63) / 64, kRamRowBlocks + kChrRowBlocks + 1);
    restore_kernel<<<grid, dim3(64), 0, stream>>>(s, mask, fixed_blob);
    return hipGetLastError();
}

hipError_t launch_reset(const DeviceState& s, const std::uint8_t* mask, hipStream_t stream) {
    return launch_restore(s, mask, nullptr, stream);
}

hipError_t launch_load_blob(const DeviceState& s, const std::uint8_t* blob_src, const std::uint8_t* mask,
                            hipStream_t stream) {
    return launch_restore(s, mask, blob_src, stream);
}

hipError_t launch_save_blob(const DeviceState& s, std::uint32_t env, std::uint8_t* out, hipStream_t stream) {
    save_blob_kernel<<<dim3(blocks_for(blob::kBytes)), dim3(kBlock), 0, stream>>>(s, env, out);
    return hipGetLastError();
}

hipError_t launch_ram_obs(const DeviceState& s, std::uint8_t* obs, hipStream_t stream) {
    // The loads cover whole 256-console groups: the pitch is a multiple of 256.
    if (s.pitch % kObsEnvs != 0 || s.pitch < s.n) return hipErrorInvalidValue;
    const dim3 grid((s.n + kObsEnvs - 1) / kObsEnvs, kRamBytes / kObsAddrs);
    ram_obs_kernel<<<grid, dim3(kBlock), 0, stream>>>(s.ram, obs, s.n, s.pitch);
    return hipGetLastError();
}

hipError_t launch_actions_i64(std::uint8_t* dst, const long long* src, std::uint32_t n, hipStream_t stream) {
    actions_i64_kernel<<<dim3(blocks_for(n)), dim3(kBlock), 0, stream>>>(dst, src, n);
    return hipGetLastError();
}

hipError_t launch_poke_ram(const DeviceState& s, std::uint32_t addr, std::uint32_t value, hipStream_t stream) {
    poke_ram_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s, addr, value);
    return hipGetLastError();
}

hipError_t launch_poke_ram_envs(const DeviceState& s, std::uint32_t addr, const std::uint8_t* values,
                                hipStream_t stream) {
    poke_ram_envs_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s, addr, values);
    return hipGetLastError();
}

hipError_t launch_seed_present(const DeviceState& s, const std::uint8_t* mask, hipStream_t stream) {
    if (s.n == 0 || s.present == nullptr) return hipSuccess;
    record_kernel<<<dim3(s.n), dim3(kBlock), 0, stream>>>(s, mask, s.present, 1u);
    return hipGetLastError();
}

hipError_t launch_live_records(const DeviceState& s, std::uint8_t* out, hipStream_t stream) {
    if (s.n == 0) return hipSuccess;
    record_kernel<<<dim3(s.n), dim3(kBlock), 0, stream>>>(s, nullptr, out, 0u);
    return hipGetLastError();
}

hipError_t launch_zero_u64(unsigned long long* p, std::uint32_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    zero_u64_kernel<<<dim3(blocks_for(n)), dim3(kBlock), 0, stream>>>(p, n);
    return hipGetLastError();
}

hipError_t launch_seed_baselines(const DeviceState& s, hipStream_t stream) {
    seed_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s);
    return hipGetLastError();
}

}  // namespace nesle
