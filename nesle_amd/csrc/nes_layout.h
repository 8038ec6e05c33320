// nes_layout.h -- device state layout shared by the HIP kernels
// (nes_step.hip, nes_kernels.hip) and the host library (nes_host.hip).
//
// HBM layout.  CPU-side byte arrays (RAM, PRG RAM, APU/IO registers, CHR RAM)
// are interleaved "address-major": element (addr, env) lives at
// base[addr * pitch + env], with pitch = num_envs rounded up to 256.  Lanes of
// a wave64 are consecutive envs, so when they touch the same NES address (same
// code path, same zero-page variable) the wave issues one 64-byte access
// instead of 64 scattered ones, and a 128-byte cache line holds one NES
// address for 128 consecutive consoles.  Per-env scalars are plain SoA arrays
// indexed by env.  The env-major RAM observation that callers see
// ([num_envs][2048], the reference's layout at cpp/bindings/cuda_module.cu:
// 854-863) is produced by a transpose kernel.
//
// Video memory (palette, OAM, nametables) is env-major instead: one block of
// vram_stride bytes per console (vram::*).  Only the I/O paths touch it, one
// console at a time, and the vblank presentation snapshot copies a whole
// block, which is then one contiguous run per console.
#pragma once

#include <cstdint>

namespace nesle {

constexpr std::uint32_t kRamBytes = 2048;
constexpr std::uint32_t kPrgRamBytes = 8192;
constexpr std::uint32_t kOamBytes = 256;
constexpr std::uint32_t kPaletteBytes = 32;
constexpr std::uint32_t kChrRamBytes = 8192;
constexpr std::uint32_t kApuIoBytes = 24;
constexpr std::uint32_t kPrgRomMax = 32768;

// PPU timing (the reference's ppu.hpp:19-25 / batch_ppu.cuh:15-21): 341 dots
// per scanline, 262 scanlines, events at dot 1 of scanlines 30, 241, 261.
constexpr std::uint32_t kDotsPerLine = 341;
constexpr std::uint32_t kFrameDots = 341u * 262u;            // 89,342
constexpr std::uint32_t kSprite0Dot = 30u * 341u + 1u;       // 10,231
constexpr std::uint32_t kVblankDot = 241u * 341u + 1u;       // 82,182
constexpr std::uint32_t kPreRenderDot = 261u * 341u + 1u;    // 89,002

// Canonical full-state blob (one console), little endian.  Identical to the
// layout documented in oracle/nes_oracle.cpp so states compare byte for byte.
namespace blob {
constexpr std::uint32_t kPc = 4, kA = 6, kX = 7, kY = 8, kSp = 9, kP = 10, kNmi = 11;
constexpr std::uint32_t kCycles = 12, kFrame = 20, kFrameDot = 28;
constexpr std::uint32_t kCtrl = 32, kMask = 33, kStatus = 34, kOamAddr = 35, kOpenBus = 36;
constexpr std::uint32_t kReadBuffer = 37, kV = 38, kT = 40, kFineX = 42, kW = 43;
constexpr std::uint32_t kScrollX = 44, kScrollY = 45, kC1Buttons = 46, kC1Shift = 47;
constexpr std::uint32_t kC1Count = 48, kStrobe = 49, kC2Count = 50, kFault = 51, kPendingDma = 52;
constexpr std::uint32_t kApuIo = 56, kRam = 80, kPrgRam = 2128, kOam = 10320, kPalette = 10576;
constexpr std::uint32_t kNametable = 10608, kChrRam = 14704, kBytes = 22896;
constexpr std::uint32_t kNametableBytes = 4096;
}  // namespace blob

// Reward rules applied once per env-step after the last frame.
enum RewardKind : std::uint32_t {
    kRewardSmb = 0,     // the reference's SMB rule (cpp/include/nesle/cuda/batch_step.cuh:61-106)
    kRewardXDelta = 1,  // clip(int16(x - x_prev), -clip, clip) - time_penalty; done = RAM[done_addr] == 0
};

struct DeviceState {
    std::uint32_t n;           // consoles
    std::uint32_t pitch;       // interleave pitch (multiple of 256, >= n)
    std::uint32_t nt_bytes;    // 2048, or 4096 for four-screen carts
    std::uint32_t nt_mode;     // 0 vertical, 1 horizontal, 2 four-screen
    std::uint32_t prg_mask;    // 0x3FFF (16 KB PRG) or 0x7FFF (32 KB)
    std::uint32_t chr_size;    // 0 => CHR RAM
    const std::uint8_t* prg_rom;
    const std::uint8_t* chr_rom;

    // CPU scalars.
    std::uint16_t* pc;
    std::uint8_t* a;
    std::uint8_t* x;
    std::uint8_t* y;
    std::uint8_t* sp;
    std::uint8_t* p;
    std::uint8_t* fault;       // bit 0: illegal opcode (console frozen)
    std::uint64_t* cycles;
    // PPU scalars.
    std::uint32_t* frame_dot;  // scanline * 341 + dot
    std::uint64_t* frame;
    std::uint8_t* ctrl;
    std::uint8_t* mask;
    std::uint8_t* status;
    std::uint8_t* nmi_pending;
    std::uint8_t* oam_addr;
    std::uint8_t* open_bus;
    std::uint8_t* read_buffer;
    std::uint16_t* v;
    std::uint16_t* t;
    std::uint8_t* fine_x;
    std::uint8_t* w;
    std::uint8_t* scroll_x;
    std::uint8_t* scroll_y;
    // Controllers (pad 2 never has buttons pressed; it shares the strobe).
    std::uint8_t* c1_buttons;
    std::uint8_t* c1_shift;
    std::uint8_t* c1_count;
    std::uint8_t* strobe;
    std::uint8_t* c2_count;
    // Interleaved byte arrays ([bytes][pitch]).
    std::uint8_t* apu_io;
    std::uint8_t* ram;
    std::uint8_t* prg_ram;     // = ram + 2048 * pitch (RAM and PRG RAM are one array)
    std::uint8_t* chr_ram;     // null when the cart has CHR ROM
    // Env-major video memory: [n][vram_stride] (vram::* offsets).
    std::uint8_t* vram;
    std::uint32_t vram_stride;

    // Step inputs/outputs.
    const std::uint8_t* actions;   // [n] controller masks for this step
    float* rewards;                // [n]
    std::uint8_t* done;            // [n]
    std::int32_t* prev_x;          // [n] reward baselines
    std::int32_t* prev_time;       // [n]
    std::uint32_t reward_kind;
    std::uint32_t x_lo, x_hi, done_addr, clip;
    float time_penalty;

    // Optional statistics (null when not collected).
    std::uint64_t* stat_instructions;
    std::uint32_t* stat_frames;
    std::uint32_t* stat_budget_hits;
    unsigned long long* prof_opcodes;  // [256]
    unsigned long long* prof_pcs;      // [65536]
    unsigned long long* census;        // [census::kCount] (stats mode 3)

    // Snapshot bank: num_levels canonical blobs, env_to_level[n].
    const std::uint8_t* bank;
    const std::uint8_t* env_to_level;
    std::uint32_t num_levels;

    // Presentation snapshot (null when frames are off): one record of
    // present::kHeader + vram_stride bytes per console, frozen at a vblank,
    // and the scroll/ctrl latched at the pre-render line (batch_ppu.cuh:
    // 215-260).
    std::uint8_t* present;     // [n][present::kHeader + vram_stride]
    std::uint8_t* lat_sx;      // [n]
    std::uint8_t* lat_sy;      // [n]
    std::uint8_t* lat_ctrl;    // [n]
};

// Step-kernel census (stats mode 3): what the waves of one launch did, summed
// over waves.  A "wave-iteration" is one trip of the step loop (one emulated
// instruction or NMI entry for each lane of the wave); a cause counts a
// wave-iteration when at least one lane of the wave has it.  Cycle counts
// come from the shader clock read at the ends of each section, so they
// include the waits those reads add.
namespace census {
enum : std::uint32_t {
    kWaves = 0,          // waves that ran the loop
    kIterations,         // wave-iterations
    kRare,               // ... that took the rare path (any cause below)
    kRareIoWrite,        // I/O register or PRG RAM write
    kRareSide,           // JMP ($xxxx), or stack bytes outside the LDS window
    kRareIdle,           // JMP to itself (idle-loop fast-forward)
    kRareIllegal,        // illegal opcode
    kRareTiming,         // PPU timing event crossed
    kRareBudget,         // per-frame instruction budget reached
    kRareOutside,        // next instruction outside PRG ROM
    kRareOnlyIoWrite,    // rare wave-iterations whose only cause is I/O writes
    kDma,                // wave-iterations with an OAM DMA copy
    kPresent,            // wave-iterations with a presentation capture
    kIoRead,             // wave-iterations with an I/O or PRG RAM read
    kIoReadSlow,         // ... through the branchy register read (not $2002/$4016)
    kActiveLanes,        // sum over wave-iterations of lanes still running frames
    kDistinctEntries,    // sum over sampled wave-iterations (every 16th) of distinct microcode entries among those lanes
    kCyclesLoop,         // shader clock, loop entry to exit, summed over waves
    kCyclesRare,         // ... inside the rare path (including the decode redone after it)
    kCyclesIoRead,       // ... inside the I/O read side path
    kLanesIoWrite,       // lane events: I/O writes
    kLanesTiming,        // lane events: timing events crossed
    kLanesIoRead,        // lane events: I/O reads
    kLanesIoReadSlow,    // lane events: I/O reads through the branchy path
    kExits,              // rare wave-iterations after which the wave left the loop
    kDistinctSamples,    // wave-iterations sampled for kDistinctEntries
    kCyclesIoWrite,      // shader clock inside the rare path: I/O and PRG RAM writes
    kCyclesSettle,       // ... PPU settlement after timing events and the budget
    kCyclesDma,          // ... OAM DMA copies
    kCyclesPresent,      // ... presentation captures
    kCyclesRedo,         // ... the decode of the next instruction, when redone
    kRedo,               // rare wave-iterations after which the decode was redone
    kCount = 32
};
}  // namespace census

// Video memory block of one console: palette, OAM, then 2 KB of nametable
// RAM (4 KB on four-screen carts).  vram_stride = kNametable + nt_bytes.
namespace vram {
constexpr std::uint32_t kPalette = 0, kOam = 32, kNametable = 288;
constexpr std::uint32_t stride(std::uint32_t nt_bytes) { return kNametable + nt_bytes; }
}  // namespace vram

// Presentation record: scroll/ctrl at frame start (latched at the previous
// pre-render line) and end (at vblank), the mask, then the console's video
// memory block as it was at vblank.
namespace present {
constexpr std::uint32_t kSxStart = 0, kSyStart = 1, kCtrlStart = 2, kSxEnd = 3, kSyEnd = 4, kCtrlEnd = 5, kMask = 6;
constexpr std::uint32_t kHeader = 16;
constexpr std::uint32_t kPalette = kHeader + vram::kPalette, kOam = kHeader + vram::kOam;
constexpr std::uint32_t kNametable = kHeader + vram::kNametable;
constexpr std::uint32_t bytes(std::uint32_t nt_bytes) { return kHeader + vram::stride(nt_bytes); }
constexpr std::uint32_t kMaxBytes = kHeader + vram::kNametable + 4096;   // 4,400
}  // namespace present

}  // namespace nesle
