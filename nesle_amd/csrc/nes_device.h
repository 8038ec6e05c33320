// nes_device.h -- device helpers shared by the step kernel (nes_step.hip) and
// the utility kernels (nes_kernels.hip): RAM access in HBM, the reward/done
// rules, and whole-console state moves (snapshot restore, power-on).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "nes_layout.h"

namespace nesle {

// Console RAM straight from HBM.  `State` is DeviceState, or the step
// kernel's view of it in the kernel-argument segment.
template <typename State>
struct GlobalRamOf {
    const State& s;
    std::uint32_t env;
    __device__ __forceinline__ std::uint32_t operator()(std::uint32_t a) const {
        return s.ram[static_cast<std::size_t>(a & 0x7FF) * s.pitch + env];
    }
};
using GlobalRam = GlobalRamOf<DeviceState>;

// ---- reward / done (batch_step.cuh:41-106; x-delta rule documented in
//      nes_layout.h).  `ram` is any callable returning console RAM bytes.
template <typename Ram>
__device__ __forceinline__ void smb_track(const Ram& ram, std::int32_t* x, std::int32_t* time) {
    *x = static_cast<std::int32_t>(ram(0x6D) * 256 + ram(0x86));
    *time = static_cast<std::int32_t>((ram(0x7F8) & 15) * 100 + (ram(0x7F9) & 15) * 10 + (ram(0x7FA) & 15));
}

template <typename Ram>
__device__ __forceinline__ void reward_seed(const DeviceState& s, std::uint32_t e, const Ram& ram) {
    if (s.reward_kind == kRewardSmb) {
        std::int32_t x, t;
        smb_track(ram, &x, &t);
        s.prev_x[e] = x;
        s.prev_time[e] = t;
    } else {
        s.prev_x[e] = static_cast<std::int32_t>(ram(s.x_lo) | (ram(s.x_hi) << 8));
        s.prev_time[e] = 0;
    }
}

template <typename State, typename Ram>
__device__ __forceinline__ void reward_apply(const State& s, std::uint32_t e, const Ram& ram, float* reward,
                                             std::uint32_t* done) {
    if (s.reward_kind == kRewardSmb) {
        std::int32_t x, t;
        smb_track(ram, &x, &t);
        std::int32_t dx = x - s.prev_x[e];
        if (dx < -5 || dx > 5) dx = 0;
        std::int32_t dt = t - s.prev_time[e];
        if (dt > 0) dt = 0;
        const std::uint32_t pstate = ram(0x0E);
        const bool dying = pstate == 0x0B || ram(0xB5) > 1;
        const bool dead = pstate == 0x06;
        const bool over = ram(0x75A) == 0xFF;
        bool flag_get = ram(0x770) == 2;
        const bool floating = ram(0x1D) == 3;
        for (std::uint32_t i = 0; i < 5; ++i) {
            const std::uint32_t en = ram(0x16 + i);
            if ((en == 0x2D || en == 0x31) && floating) flag_get = true;
        }
        *reward = static_cast<float>(dx + dt + ((dying || dead) ? -25 : 0));
        *done = (flag_get || dying || dead || over) ? 1u : 0u;
        s.prev_x[e] = x;
        s.prev_time[e] = t;
    } else {
        const std::int32_t x = static_cast<std::int32_t>(ram(s.x_lo) | (ram(s.x_hi) << 8));
        std::int32_t dx = static_cast<std::int16_t>(static_cast<std::uint16_t>(x - s.prev_x[e]));
        const std::int32_t c = static_cast<std::int32_t>(s.clip);
        dx = dx < -c ? -c : (dx > c ? c : dx);
        *reward = static_cast<float>(dx) - s.time_penalty;
        *done = ram(s.done_addr) == 0 ? 1u : 0u;
        s.prev_x[e] = x;
    }
}

// ---- whole-console state moves ------------------------------------------------
__device__ __forceinline__ std::uint32_t le16(const std::uint8_t* b, std::uint32_t o) { return b[o] | (b[o + 1] << 8); }
__device__ __forceinline__ std::uint32_t le32(const std::uint8_t* b, std::uint32_t o) {
    return b[o] | (b[o + 1] << 8) | (b[o + 2] << 16) | (static_cast<std::uint32_t>(b[o + 3]) << 24);
}
__device__ __forceinline__ std::uint64_t le64(const std::uint8_t* b, std::uint32_t o) {
    return le32(b, o) | (static_cast<std::uint64_t>(le32(b, o + 4)) << 32);
}

// Console `env`'s video memory block (palette, OAM, nametables; vram::*).
__device__ __forceinline__ std::uint8_t* vram_of(const DeviceState& s, std::uint32_t env) {
    return s.vram + static_cast<std::size_t>(env) * s.vram_stride;
}

// 16-byte copies and fills; every video memory section and blob field they
// are used on starts on a 16-byte boundary and is a multiple of 16 long.
__device__ __forceinline__ void copy16(std::uint8_t* dst, const std::uint8_t* src, std::uint32_t bytes) {
    for (std::uint32_t i = 0; i < bytes / 16; ++i) reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
}
__device__ __forceinline__ void zero16(std::uint8_t* dst, std::uint32_t bytes) {
    for (std::uint32_t i = 0; i < bytes / 16; ++i) reinterpret_cast<uint4*>(dst)[i] = make_uint4(0, 0, 0, 0);
}

// Byte `k` (a compile-time index after unrolling) of a run of dwords.
__device__ __forceinline__ std::uint32_t byte_at(const std::uint32_t* w, std::uint32_t k) {
    return (w[k >> 2] >> (8 * (k & 3))) & 0xFF;
}

// `rows` bytes of a blob (16-byte aligned, rows a multiple of 16) into
// consecutive rows of an address-major array at `dst` (= array + row0 *
// pitch + env).  The blob is read 16 bytes at a time, four loads ahead of
// the stores, so the copy waits on about one load round trip in all; the
// byte stores are independent of each other.
__device__ __forceinline__ void blob_rows(std::uint8_t* dst, std::uint32_t pitch, const std::uint8_t* src,
                                          std::uint32_t rows) {
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    const std::uint32_t chunks = rows / 16;
    const std::uint32_t last = chunks - 1;
    uint4 q0 = s4[0], q1 = s4[1 < last ? 1 : last], q2 = s4[2 < last ? 2 : last], q3 = s4[3 < last ? 3 : last];
    std::uint32_t at = 0;
#pragma unroll 1
    for (std::uint32_t c = 0; c < chunks; ++c) {
        const std::uint32_t w[4] = {q0.x, q0.y, q0.z, q0.w};
        q0 = q1;
        q1 = q2;
        q2 = q3;
        q3 = s4[c + 4 < last ? c + 4 : last];
#pragma unroll
        for (std::uint32_t k = 0; k < 16; ++k) {
            dst[at] = static_cast<std::uint8_t>(byte_at(w, k));
            at += pitch;
        }
    }
}

__device__ __forceinline__ void zero_rows(std::uint8_t* dst, std::uint32_t pitch, std::uint32_t rows) {
    std::uint32_t at = 0;
#pragma unroll 16
    for (std::uint32_t r = 0; r < rows; ++r) {
        dst[at] = 0;
        at += pitch;
    }
}

// The scalar fields and $4000-$4017 of a canonical blob into console `env`.
__device__ inline void blob_scalars(const DeviceState& s, std::uint32_t env, const std::uint8_t* b) {
    using namespace blob;
    s.pc[env] = static_cast<std::uint16_t>(le16(b, kPc));
    s.a[env] = b[kA]; s.x[env] = b[kX]; s.y[env] = b[kY]; s.sp[env] = b[kSp]; s.p[env] = b[kP];
    s.nmi_pending[env] = b[kNmi];
    s.cycles[env] = le64(b, kCycles);
    s.frame[env] = le64(b, kFrame);
    s.frame_dot[env] = le32(b, kFrameDot);
    s.ctrl[env] = b[kCtrl]; s.mask[env] = b[kMask]; s.status[env] = b[kStatus];
    s.oam_addr[env] = b[kOamAddr]; s.open_bus[env] = b[kOpenBus]; s.read_buffer[env] = b[kReadBuffer];
    s.v[env] = static_cast<std::uint16_t>(le16(b, kV)); s.t[env] = static_cast<std::uint16_t>(le16(b, kT));
    s.fine_x[env] = b[kFineX]; s.w[env] = b[kW]; s.scroll_x[env] = b[kScrollX]; s.scroll_y[env] = b[kScrollY];
    s.c1_buttons[env] = b[kC1Buttons]; s.c1_shift[env] = b[kC1Shift]; s.c1_count[env] = b[kC1Count];
    s.strobe[env] = b[kStrobe]; s.c2_count[env] = b[kC2Count]; s.fault[env] = b[kFault];
    for (std::uint32_t i = 0; i < kApuIoBytes; ++i) s.apu_io[i * s.pitch + env] = b[kApuIo + i];
}

// Power-on scalars: the reference CPU core after construction + reset_cpu
// (console.hpp:38-47,103-106; cpu.hpp:84-92), identical to the reference's
// cold reset of a batched console (batch_step.cuh:109-172); every array of
// the console is zero at power-on.
__device__ inline void power_on_scalars(const DeviceState& s, std::uint32_t env) {
    const std::uint8_t* prg = s.prg_rom;
    s.pc[env] = static_cast<std::uint16_t>(prg[0xFFFC & s.prg_mask] | (prg[0xFFFD & s.prg_mask] << 8));
    s.a[env] = 0; s.x[env] = 0; s.y[env] = 0; s.sp[env] = 0xFD; s.p[env] = 0x24;
    s.nmi_pending[env] = 0; s.cycles[env] = 7; s.frame[env] = 0; s.frame_dot[env] = 0;
    s.ctrl[env] = 0; s.mask[env] = 0; s.status[env] = 0; s.oam_addr[env] = 0; s.open_bus[env] = 0;
    s.read_buffer[env] = 0; s.v[env] = 0; s.t[env] = 0; s.fine_x[env] = 0; s.w[env] = 0;
    s.scroll_x[env] = 0; s.scroll_y[env] = 0;
    s.c1_buttons[env] = 0; s.c1_shift[env] = 0; s.c1_count[env] = 8; s.strobe[env] = 0; s.c2_count[env] = 8;
    s.fault[env] = 0;
    for (std::uint32_t i = 0; i < kApuIoBytes; ++i) s.apu_io[i * s.pitch + env] = 0;
}

}  // namespace nesle
