// nes_step.hip -- the batched NROM console step for gfx950 (MI355X).
//
// One lane per console.  Per launch a lane runs `frameskip` NES frames: NMI
// entry, the 6502 instruction, OAM DMA, lazy PPU settlement at the timing
// events, then the reward/done rule.  The auto-reset of done consoles is the
// restore kernel (nes_kernels.hip) launched right after on the same stream:
// kept out of this kernel, its code cannot change how the main loop is
// compiled, and it spreads a reset over many waves instead of one lane's
// serial copy.  Semantics follow the reference's CPU core
// (cpp/include/nesle/console.hpp:49-150, cpu.hpp:84-730, ppu.hpp:46-395,
// controller.hpp:18-67); the launch mirrors the reference's console_step_kernel
// (cpp/src/cuda/kernels.cu:19-104) and its snapshot reset (kernels.cu:195-203).
//
// Cost model on MI355X (measured): one wave issues one instruction every ~4.3
// cycles, an LDS round trip takes ~84 cycles and a global one ~250.  At 65,536
// consoles there is exactly one wave per SIMD, so the kernel is bound by the
// instructions a wave issues per emulated 6502 instruction and by the memory
// round trips on that path.  Hence:
//  * Geometry: 4 waves per workgroup, L = N/1024 (rounded up to a power of
//    two, at most 64) consoles per wave, so every SIMD holds one wave however
//    small the batch.
//  * LDS (a static 160 KB array) holds the PRG ROM (32 KB), the microcode
//    (nes_micro.h) and console RAM: all 2 KB of it when 4L consoles fit
//    (L <= 8), otherwise the zero page and $0180-$01FF.  Other RAM rows and
//    PRG RAM are address-major interleaved in HBM (row * pitch + env).
//  * Registers A/X/Y/SP are packed in one VGPR; the microcode drives one
//    branch-free datapath (addressing, stack window, next PC, ALU, flags).
//    Finished lanes and NMI entry run as virtual opcodes, so nothing needs a
//    commit select.  The registers that I/O reads touch ($2002, $4016/7:
//    status, open bus, write toggle, pads; for $2004 the OAM byte at
//    OAMADDR) are packed into VGPRs, so those reads take no memory round
//    trip; the other PPU registers live in a per-console LDS area.
//  * With RAM split between LDS and HBM, the next instruction is decoded one
//    iteration ahead: its effective address is computed and its HBM operand
//    load issued at the end of the current iteration, so the load has a
//    whole iteration to arrive.  HBM operand loads and stores are branch-free
//    (lanes without one read row 0 and write a spare row).
//  * Only the I/O register read branches inside the loop (PPUSTATUS and pad 1
//    reads by selects, the rest behind a branch); everything rare (I/O
//    writes, JMP indirect, stack wrap, idle loops, illegal opcodes, PPU
//    events, OAM DMA, code outside ROM) sits behind one wave-uniform test.
//  * With RAM split, a console that reaches vblank waits for the rest of its
//    wave (the vblank rendezvous), so the NMI handlers, which hold the I/O
//    writes, OAM DMA and the frame capture, run in step and share rare-path
//    entries.  OAM DMA and the capture are then copied by each lane for its
//    own console; otherwise the whole wave copies one console at a time
//    instead of a 256-iteration loop in one lane.
//  * The launch state's fields that only the rare work and the write-back
//    read come through a reloaded pointer to the kernel arguments (`reload`),
//    so the loop's scalar registers stay with its constants.
//  * The CPU cycle counter is not updated per instruction: every cycle is 3
//    PPU dots, so cycles advance by (dots advanced) / 3 at the end.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>

#include "nes_device.h"
#include "nes_launch.h"
#include "nes_layout.h"
#include "nes_micro.h"

namespace nesle {
namespace {

__constant__ mc::Table c_micro_split = mc::kTableSplit;
__constant__ mc::Table c_micro_full = mc::kTableFull;

// The whole 160 KB of a CU's LDS, statically: one workgroup per CU, and a
// static array has a known address (0), so LDS addresses need no base add.
constexpr std::uint32_t kLdsLimit = 160u * 1024u;
__shared__ __attribute__((aligned(16))) std::uint8_t lds[kLdsLimit];

constexpr std::uint32_t kMaxBlock = 1024;       // up to 16 waves per workgroup
// Microcode in LDS as five tables of 16-byte slices (dwords 0-3, 4-7, ...,
// 16-19 of every entry): lanes reading different entries then spread over the
// banks as with 16-byte entries, where 80-byte entries would pile onto few.
constexpr std::uint32_t kMicroBytes = 4 * mc::kDwords;                   // 80 B per entry
constexpr std::uint32_t kMicroSlices = mc::kDwords / 4;
constexpr std::uint32_t kMicroQuarter = 16 * mc::kEntries;               // bytes per table
constexpr std::uint32_t kLdsMicro = 32768;                               // after the PRG image
constexpr std::uint32_t kLdsRam = kLdsMicro + mc::kEntries * kMicroBytes; // console RAM blocks
// Per-console LDS block: RAM rows, 4 spare bytes, then a 40-byte register
// area (PPU/pad registers and the rarely touched loop state).  Strides are an
// odd number of dwords, so lanes at equal offsets hit distinct banks.
constexpr std::uint32_t kSplitStride = 428;     // $0180-$01FF, $0000-$00FF, spare, registers
constexpr std::uint32_t kFullStride = 2092;     // $0000-$07FF, spare, registers
// Register area offsets (bytes from the start of the area).  Bytes 2, 4, 7
// and 10-14 are unused: PPUSTATUS, open bus, the write toggle and the pad
// registers stay in VGPRs for the whole launch.
namespace reg {
constexpr std::uint32_t kCtrl = 0, kMask = 1, kOamAddr = 3, kReadBuffer = 5;
constexpr std::uint32_t kFineX = 6, kScrollX = 8, kScrollY = 9, kDmaPage = 15, kV = 16, kT = 18;
constexpr std::uint32_t kFrameDot = 20, kHorizon = 24, kFramesLeft = 28, kFrames = 32, kBudgetHits = 36;
}  // namespace reg

// Bits of a console's `flags` VGPR.
constexpr std::uint32_t kDmaPending = 1, kNmiPending = 2, kFault = 4, kPresentPending = 8;
// The microcode's clear-NMI bit is the flag's own bit, so the commit clears it
// with one and-not.
static_assert(kNmiPending == mc::kClearNmi, "NMI flag and clear bit must match");
// The PPU and pad registers every I/O read touches live in VGPRs: the write
// toggle and pad strobe as `flags` bits, pad 1's buttons in `flags` bits
// 8-15, the OAM byte at OAMADDR (what a `$2004` read returns) in `flags`
// bits 16-23, and `io` = open bus (bits 0-7) | PPUSTATUS (8-15) | pad 1
// shift register (16-23) | pad 1 reads (24-27) | pad 2 reads (28-31).
constexpr std::uint32_t kWToggle = 16, kStrobeBit = 32;

// Row of the interleaved RAM/PRG-RAM array that lanes with nothing to store
// write to (one spare byte per console after PRG RAM; lanes without a console
// use console 0's), so the operand store needs no branch.
constexpr std::uint32_t kTrashRow = kRamBytes + kPrgRamBytes;

// Lanes without a console run the datapath on a dummy block after the last
// console's (they write only their own stack window and spare byte).  The
// operand candidate read from a split block can reach 0x1FF bytes into a
// 428-byte block; the slack keeps the dummy block's reads in bounds.
constexpr std::uint32_t kLdsSlack = 128;
constexpr std::uint32_t lds_bytes(std::uint32_t consoles, bool full) {
    return kLdsRam + (consoles + 1) * (full ? kFullStride : kSplitStride) + kLdsSlack;
}

// XCD k (workgroups dispatched round-robin, b % 8 == k) owns one contiguous
// range of consoles, so interleaved cache lines stay in one L2.
__device__ __forceinline__ std::uint32_t xcd_block(std::uint32_t b, std::uint32_t nb) {
    const std::uint32_t q = nb >> 3, r = nb & 7, xcd = b & 7;
    return xcd * q + (xcd < r ? xcd : r) + (b >> 3);
}

// Wait for this wave's outstanding vector-memory operations (s_waitcnt
// vmcnt(0), gfx9 encoding with expcnt and lgkmcnt left open).  A side path
// that loads from HBM ends with it, so values it hands to the hot loop are
// complete there and the loop header carries no vmcnt wait, which would
// also wait for the store the previous iteration just issued.
__device__ __forceinline__ void vmem_settled() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The kernel's DeviceState where the launch placed it, in the kernel-argument
// segment (constant address space): a field read through it is a scalar load.
using KState = const __attribute__((address_space(4))) DeviceState;

// The same pointer, opaque to the optimiser.  Fields read through the result
// are loaded where they are used instead of being held in scalar registers
// across the loop: the rare work and the write-back read about forty of them,
// and held for the whole loop they took the registers of the hot path's
// constants, which were then materialised again on every iteration.
__device__ __forceinline__ KState* reload(KState* p) {
    asm volatile("" : "+s"(p));
    return p;
}

// Bitwise select: bits of `a` where `m` is set, else bits of `b` (v_bfi_b32).
__device__ __forceinline__ std::uint32_t sel(std::uint32_t m, std::uint32_t a, std::uint32_t b) {
    return (a & m) | (b & ~m);
}


__device__ __forceinline__ std::uint32_t ubfe(std::uint32_t v, std::uint32_t off, std::uint32_t w) {
    return __builtin_amdgcn_ubfe(v, off, w);
}

// Dots from `fd` to the next timing event: sprite-0 dot, vblank, pre-render
// line, frame end (ppu.hpp:19-25,136-147).  Signed differences keep every
// candidate comparison a plain select.  `through`: the frame end changes
// nothing a program can observe (the frame count and the dot counter's wrap,
// which settle() applies when it crosses it), so when it is not the launch's
// last, the countdown runs on to the next frame's sprite-0 dot, one rare-work
// entry per frame fewer.
__device__ __forceinline__ std::uint32_t to_event(std::uint32_t fd, bool through) {
    const std::int32_t c = static_cast<std::int32_t>(fd);
    std::int32_t d = static_cast<std::int32_t>(through ? kFrameDots + kSprite0Dot : kFrameDots) - c;
    const std::int32_t s0 = static_cast<std::int32_t>(kSprite0Dot) - c;
    const std::int32_t vb = static_cast<std::int32_t>(kVblankDot) - c;
    const std::int32_t pr = static_cast<std::int32_t>(kPreRenderDot) - c;
    d = (s0 > 0 && s0 < d) ? s0 : d;
    d = (vb > 0 && vb < d) ? vb : d;
    d = (pr > 0 && pr < d) ? pr : d;
    return static_cast<std::uint32_t>(d);
}

template <bool kFull>
struct Console {
    static constexpr std::uint32_t kStride = kFull ? kFullStride : kSplitStride;
    static constexpr std::uint32_t kSpare = kFull ? 2048u : 384u;  // dummy store target
    static constexpr std::uint32_t kRegs = kSpare + 4;              // register area
    static constexpr std::uint32_t kZp = kFull ? 0u : 0x80u;       // offset of $0000 in the block
    // Offset of stack byte $0100 + SP - 2 is SP + kStk (SP >= 0x82 in split mode).
    static constexpr std::uint32_t kStk = kFull ? 0xFEu : static_cast<std::uint32_t>(-0x82);

    // The launch's state: reloaded (`reload`) at the start of the rare work, so
    // the side paths and the rare work read its fields where they use them.
    KState* s;
    std::uint32_t env, base, pitch;
    std::uint32_t nmi_vec, brk_vec;
    // Split layout: this console's video memory block, held for the loop
    // (the I/O side path's `$2004` and `$2007` reads then need no scalar
    // loads; with all RAM in LDS it is computed where it is used, which
    // measured faster there).
    std::uint8_t* vm = nullptr;
    // Hot state in VGPRs: CPU registers, `flags` (NMI latch, pending OAM DMA,
    // fault, write toggle, strobe, pad 1 buttons) and `io` (open bus, status,
    // pad shift state).  The other PPU registers live in the console's LDS
    // register area (reg::*): only the I/O paths, PPU settlement and NMI entry
    // touch them.
    std::uint32_t pc, regs, p, flags, io;

    // ---- VGPR-resident I/O registers ------------------------------------------------
    __device__ __forceinline__ std::uint32_t open_bus() const { return io & 0xFF; }
    __device__ __forceinline__ void set_open_bus(std::uint32_t v) { io = (io & ~0xFFu) | (v & 0xFF); }
    __device__ __forceinline__ std::uint32_t status() const { return ubfe(io, 8, 8); }
    __device__ __forceinline__ void set_status(std::uint32_t v) { io = (io & ~0xFF00u) | ((v & 0xFF) << 8); }
    __device__ __forceinline__ std::uint32_t c1_shift() const { return ubfe(io, 16, 8); }
    __device__ __forceinline__ std::uint32_t c1_count() const { return ubfe(io, 24, 4); }
    __device__ __forceinline__ std::uint32_t c2_count() const { return io >> 28; }
    __device__ __forceinline__ void set_c1(std::uint32_t shift, std::uint32_t count) {
        io = (io & 0xF000FFFFu) | ((shift & 0xFF) << 16) | ((count & 0xF) << 24);
    }
    __device__ __forceinline__ void set_c2_count(std::uint32_t n) { io = (io & 0x0FFFFFFFu) | (n << 28); }
    __device__ __forceinline__ std::uint32_t buttons() const { return ubfe(flags, 8, 8); }
    // OAM and OAMADDR change only in the rare work (`$2003`/`$2004` writes,
    // OAM DMA) and between launches, so the byte a `$2004` read returns
    // (ppu.hpp:88-89: no side effects) is kept up to date there.
    __device__ __forceinline__ std::uint32_t oam_data() const { return ubfe(flags, 16, 8); }
    __device__ __forceinline__ void set_oam_data(std::uint32_t v) { flags = (flags & ~0xFF0000u) | ((v & 0xFF) << 16); }

    // ---- LDS register area ----------------------------------------------------------
    __device__ __forceinline__ std::uint32_t r8(std::uint32_t f) const { return lds[base + kRegs + f]; }
    __device__ __forceinline__ void w8(std::uint32_t f, std::uint32_t v) const {
        lds[base + kRegs + f] = static_cast<std::uint8_t>(v);
    }
    __device__ __forceinline__ std::uint32_t r16(std::uint32_t f) const {
        return *reinterpret_cast<const std::uint16_t*>(lds + base + kRegs + f);
    }
    __device__ __forceinline__ void w16(std::uint32_t f, std::uint32_t v) const {
        *reinterpret_cast<std::uint16_t*>(lds + base + kRegs + f) = static_cast<std::uint16_t>(v);
    }
    __device__ __forceinline__ std::uint32_t r32(std::uint32_t f) const {
        return *reinterpret_cast<const std::uint32_t*>(lds + base + kRegs + f);
    }
    __device__ __forceinline__ void w32(std::uint32_t f, std::uint32_t v) const {
        *reinterpret_cast<std::uint32_t*>(lds + base + kRegs + f) = v;
    }

    // ---- console RAM ($0000-$07FF, mirrored to $1FFF) -------------------------
    __device__ __forceinline__ static bool ram_in_lds(std::uint32_t ra) {
        return kFull || ((0xBu >> (ra >> 7)) & 1u);  // rows $000-$0FF and $180-$1FF
    }
    // Block offset of an LDS-resident RAM byte: split mode keeps $0180-$01FF
    // at 0x000-0x07F and the zero page at 0x080-0x17F, so the offset is one
    // add and mask; for other rows the result is an in-block byte that is
    // read and never written.
    __device__ __forceinline__ static std::uint32_t ram_lds_off(std::uint32_t ra) {
        return kFull ? (ra & 0x7FFu) : ((ra + 0x80u) & 0x1FFu);
    }
    // Offset of (row, this console) in an address-major interleaved array.
    __device__ __forceinline__ std::uint32_t goff(std::uint32_t row) const { return __umul24(row, pitch) + env; }
    // This console's video memory block (env-major).
    __device__ __forceinline__ std::uint8_t* vmem() const {
        if constexpr (kFull) return s->vram + static_cast<std::size_t>(env) * s->vram_stride;
        return vm;
    }
    __device__ __forceinline__ std::uint32_t ram_rd(std::uint32_t ra) const {
        if (ram_in_lds(ra)) return lds[base + ram_lds_off(ra)];
        return s->ram[goff(ra)];
    }
    __device__ __forceinline__ void ram_wr(std::uint32_t ra, std::uint32_t val) const {
        if (ram_in_lds(ra)) {
            lds[base + ram_lds_off(ra)] = static_cast<std::uint8_t>(val);
        } else {
            s->ram[goff(ra)] = static_cast<std::uint8_t>(val);
        }
    }

    // ---- PPU memory (ppu.hpp:280-338) -------------------------------------------
    __device__ std::uint32_t nt_index(std::uint32_t addr) const {
        const std::uint32_t i = (addr - 0x2000) & 0x0FFF;
        if (s->nt_mode == 2) return i;
        if (s->nt_mode == 0) return i & 0x07FF;
        return (i & 0x03FF) | ((i & 0x0800) >> 1);
    }
    __device__ static std::uint32_t pal_index(std::uint32_t addr) {
        const std::uint32_t i = addr & 0x1F;
        return ((i & 0x13) == 0x10) ? (i & 0x0F) : i;
    }
    __device__ std::uint32_t vram_rd(std::uint32_t addr) const {
        addr &= 0x3FFF;
        if (addr < 0x2000) {
            if (s->chr_size != 0) return s->chr_rom[addr % s->chr_size];
            return s->chr_ram[goff(addr & 0x1FFF)];
        }
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            return vmem()[vram::kNametable + nt_index(addr)];
        }
        return vmem()[vram::kPalette + pal_index(addr)];
    }
    __device__ void vram_wr(std::uint32_t addr, std::uint32_t val) const {
        addr &= 0x3FFF;
        if (addr < 0x2000) {
            if (s->chr_size == 0) s->chr_ram[goff(addr & 0x1FFF)] = static_cast<std::uint8_t>(val);
            return;
        }
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            vmem()[vram::kNametable + nt_index(addr)] = static_cast<std::uint8_t>(val);
            return;
        }
        vmem()[vram::kPalette + pal_index(addr)] = static_cast<std::uint8_t>(val);
    }

    // An I/O read: PPUSTATUS (and mirrors) and pad 1, the common ones, by
    // selects for every lane of the side path; the others through io_rd.
    __device__ std::uint32_t io_read(std::uint32_t addr) {
        const bool r2002 = (addr & 0xE007) == 0x2002;
        const bool r4016 = addr == 0x4016;
        const std::uint32_t v2002 = (status() & 0xE0) | (io & 0x1F);
        const bool strobe = (flags & kStrobeBit) != 0;
        const std::uint32_t n = c1_count(), sh = c1_shift();
        const bool shifting = r4016 && !strobe && n < 8;
        const std::uint32_t bit = strobe ? (buttons() & 1) : (n < 8 ? (sh & 1) : 1u);
        std::uint32_t io_n = r2002 ? ((io & ~0x80FFu) | v2002) : io;
        io = shifting ? ((io_n & 0xF000FFFFu) | ((sh >> 1) << 16) | ((n + 1) << 24)) : io_n;
        flags = r2002 ? (flags & ~(kNmiPending | kWToggle)) : flags;
        std::uint32_t v = r2002 ? v2002 : (0x40 | bit);
        if (!r2002 && !r4016) v = io_rd(addr);   // the compiler waits for its load where v is used
        return v;
    }

    // ---- I/O space $2000-$5FFF (console.hpp:49-101, ppu.hpp:84-134,340-396,
    //      controller.hpp:20-47) ----------------------------------------------------
    __device__ std::uint32_t io_rd(std::uint32_t addr) {
        // Split layout: OAMDATA, the benchmark ROM's most common read here,
        // is tested first (2.6 % faster at 65,536 consoles; the all-RAM-in-LDS
        // layout, which enters this path in 1 % of its iterations, is no
        // faster that way).
        if constexpr (!kFull) {
            if ((addr & 0xE007) == 0x2004) return oam_data();
        }
        if (addr >= 0x6000) return s->ram[goff(addr - 0x5800)];   // PRG RAM
        if (addr < 0x4000) {
            const std::uint32_t reg = addr & 7;
            if (reg == 2) {
                const std::uint32_t val = (status() & 0xE0) | (io & 0x1F);
                io = (io & ~0x80FFu) | val;   // vblank flag cleared, open bus = the value read
                flags &= ~(kNmiPending | kWToggle);
                return val;
            }
            if (reg == 4) return oam_data();
            if (reg == 7) {
                const std::uint32_t v = r16(reg::kV);
                const std::uint32_t va = v & 0x3FFF;
                std::uint32_t val;
                if (va >= 0x3F00) {
                    val = vram_rd(va);
                    w8(reg::kReadBuffer, vram_rd(va - 0x1000));
                } else {
                    val = r8(reg::kReadBuffer);
                    w8(reg::kReadBuffer, vram_rd(va));
                }
                w16(reg::kV, v + ((r8(reg::kCtrl) & 0x04) ? 32u : 1u));
                set_open_bus(val);
                return val;
            }
            return open_bus();
        }
        if (addr == 0x4016) {
            if (flags & kStrobeBit) return 0x40 | (buttons() & 1);
            std::uint32_t bit = 1;
            const std::uint32_t n = c1_count();
            if (n < 8) {
                const std::uint32_t sh = c1_shift();
                bit = sh & 1;
                set_c1(sh >> 1, n + 1);
            }
            return 0x40 | bit;
        }
        if (addr == 0x4017) {
            if (flags & kStrobeBit) return 0x40;
            const std::uint32_t n = c2_count();
            if (n < 8) {
                set_c2_count(n + 1);
                return 0x40;
            }
            return 0x41;
        }
        if (addr < 0x4018) return s->apu_io[goff(addr - 0x4000)];
        return 0;
    }

    __device__ void ppu_wr(std::uint32_t r, std::uint32_t val) {
        set_open_bus(val);
        if (r == 0) {
            const std::uint32_t ctrl = r8(reg::kCtrl);
            if ((val & 0x80) && !(ctrl & 0x80) && (status() & 0x80)) flags |= kNmiPending;
            w8(reg::kCtrl, val);
            w16(reg::kT, (r16(reg::kT) & 0xF3FF) | ((val & 0x03) << 10));
        } else if (r == 1) {
            w8(reg::kMask, val);
        } else if (r == 3) {
            w8(reg::kOamAddr, val);
            set_oam_data(vmem()[vram::kOam + (val & 0xFF)]);
        } else if (r == 4) {
            const std::uint32_t oa = r8(reg::kOamAddr);
            vmem()[vram::kOam + oa] = static_cast<std::uint8_t>(val);
            w8(reg::kOamAddr, oa + 1);
            set_oam_data(vmem()[vram::kOam + ((oa + 1) & 0xFF)]);
        } else if (r == 5) {
            const std::uint32_t t = r16(reg::kT);
            if (!(flags & kWToggle)) {
                w8(reg::kFineX, val & 7);
                w16(reg::kT, (t & 0xFFE0) | (val >> 3));
                w8(reg::kScrollX, val);
            } else {
                w16(reg::kT, (((t & 0x8FFF) | ((val & 0x07) << 12)) & 0xFC1F) | ((val & 0xF8) << 2));
                w8(reg::kScrollY, val);
            }
            flags ^= kWToggle;
        } else if (r == 6) {
            const std::uint32_t t = r16(reg::kT);
            if (!(flags & kWToggle)) {
                w16(reg::kT, (t & 0x00FF) | ((val & 0x3F) << 8));
            } else {
                const std::uint32_t nt = (t & 0x7F00) | val;
                w16(reg::kT, nt);
                w16(reg::kV, nt);
            }
            flags ^= kWToggle;
        } else if (r == 7) {
            const std::uint32_t v = r16(reg::kV);
            vram_wr(v, val);
            w16(reg::kV, v + ((r8(reg::kCtrl) & 0x04) ? 32u : 1u));
        }
    }

    // Returns the extra PPU dots the write costs (OAM DMA: 513 CPU cycles).
    __device__ std::uint32_t io_wr(std::uint32_t addr, std::uint32_t val) {
        if (addr >= 0x6000) {   // PRG RAM
            s->ram[goff(addr - 0x5800)] = static_cast<std::uint8_t>(val);
            return 0;
        }
        if (addr < 0x4000) {
            ppu_wr(addr & 7, val);
            return 0;
        }
        if (addr >= 0x4018) return 0;
        s->apu_io[goff(addr - 0x4000)] = static_cast<std::uint8_t>(val);
        if (addr == 0x4014) {  // copied by the wave right after this instruction
            w8(reg::kDmaPage, val);
            flags |= kDmaPending;
            return 3 * 513;
        }
        if (addr == 0x4016) {
            const std::uint32_t next = val & 1;
            if (next || (flags & kStrobeBit)) {
                set_c1(buttons(), 0);
                set_c2_count(0);
            }
            flags = next ? (flags | kStrobeBit) : (flags & ~kStrobeBit);
        }
        return 0;
    }

    // ---- CPU bus (console.hpp:49-101) --------------------------------------------
    __device__ std::uint32_t bus_rd(std::uint32_t addr) {
        if (addr < 0x2000) return ram_rd(addr & 0x7FF);
        if (addr >= 0x8000) return lds[addr & 0x7FFF];
        if (addr >= 0x6000) return s->ram[goff(addr - 0x5800)];
        return io_rd(addr) & 0xFF;
    }

    // ---- PPU timing (ppu.hpp:46-76) -------------------------------------------------
    // Advance by `dots` (less than one frame past the next frame end), applying
    // every event crossed in order.  Returns frames completed (0 or 1).  Only
    // the last vblank of the step reaches the presentation snapshot that a
    // render after the step sees, so earlier ones are not captured unless
    // `every_vblank` (frames cut short by the instruction budget, a console
    // that stopped).
    __device__ std::uint32_t settle(std::uint32_t dots, bool every_vblank, bool* vblank = nullptr) {
        const std::uint32_t start = r32(reg::kFrameDot), end = start + dots;
        const std::uint32_t fc = end >= kFrameDots ? 1u : 0u;
        std::uint32_t status = this->status();
        const std::uint32_t mask = r8(reg::kMask), ctrl = r8(reg::kCtrl);
        for (std::uint32_t fo = 0; fo <= fc; ++fo) {
            const std::uint32_t off = fo * kFrameDots;
            auto crossed = [&](std::uint32_t ev) { return start < off + ev && off + ev <= end; };
            if (crossed(kSprite0Dot) && (mask & 0x18)) status |= 0x40;
            if (crossed(kVblankDot)) {
                if (vblank != nullptr) *vblank = true;
                if (!(status & 0x80) && (ctrl & 0x80)) flags |= kNmiPending;
                status |= 0x80;
                if (s->present != nullptr && (every_vblank || r32(reg::kFramesLeft) <= fo + 1))
                    flags |= kPresentPending;   // captured after the instruction
            }
            if (crossed(kPreRenderDot)) {
                status &= 0x1F;
                flags &= ~kNmiPending;
                if (s->present != nullptr) {   // frame-start scroll/ctrl of the next snapshot
                    s->lat_sx[env] = static_cast<std::uint8_t>(r8(reg::kScrollX));
                    s->lat_sy[env] = static_cast<std::uint8_t>(r8(reg::kScrollY));
                    s->lat_ctrl[env] = static_cast<std::uint8_t>(ctrl);
                }
            }
        }
        set_status(status);
        w32(reg::kFrameDot, end - fc * kFrameDots);
        return fc;
    }

    // Presentation record of this console (batch_ppu.cuh:224-249): scroll and
    // ctrl latched at the last pre-render line, the current ones, the mask,
    // then the video memory block.  `lane`/`lanes`: the copy is shared by
    // `lanes` cooperating lanes (1 when the console's own lane does it alone).
    __device__ static void capture(KState* s, std::uint32_t e_env, std::uint32_t e_regs,
                                   std::uint32_t lane, std::uint32_t lanes) {
        const std::uint32_t vs = s->vram_stride;
        std::uint8_t* rec = s->present + static_cast<std::size_t>(e_env) * (present::kHeader + vs);
        for (std::uint32_t k = lane; k < 7; k += lanes) {
            std::uint32_t v;
            switch (k) {
                case 0: v = s->lat_sx[e_env]; break;
                case 1: v = s->lat_sy[e_env]; break;
                case 2: v = s->lat_ctrl[e_env]; break;
                case 3: v = lds[e_regs + reg::kScrollX]; break;
                case 4: v = lds[e_regs + reg::kScrollY]; break;
                case 5: v = lds[e_regs + reg::kCtrl]; break;
                default: v = lds[e_regs + reg::kMask]; break;
            }
            rec[k] = static_cast<std::uint8_t>(v);
        }
        // 16-byte copies (the block and record strides and the record
        // header are multiples of 16).  With all RAM in LDS a whole wave
        // loads its share (at most five pieces per lane) before it stores
        // any, one memory round trip per console; the split layout, whose
        // waves capture together at the vblank rendezvous (capture_own),
        // keeps the plain loop for the few consoles that capture alone.
        using u32x4 = std::uint32_t __attribute__((ext_vector_type(4)));
        const auto* from = reinterpret_cast<const u32x4*>(s->vram + static_cast<std::size_t>(e_env) * vs);
        auto* to = reinterpret_cast<u32x4*>(rec + present::kHeader);
        const std::uint32_t n = vs / 16;
        if (kFull && lanes == 64) {
            static_assert((present::kMaxBytes - present::kHeader) / 16 <= 5 * 64, "five 16-byte loads per lane");
            const u32x4 zero = {0u, 0u, 0u, 0u};
            const u32x4 v0 = lane < n ? from[lane] : zero;
            const u32x4 v1 = lane + 64 < n ? from[lane + 64] : zero;
            const u32x4 v2 = lane + 128 < n ? from[lane + 128] : zero;
            const u32x4 v3 = lane + 192 < n ? from[lane + 192] : zero;
            const u32x4 v4 = lane + 256 < n ? from[lane + 256] : zero;
            if (lane < n) to[lane] = v0;
            if (lane + 64 < n) to[lane + 64] = v1;
            if (lane + 128 < n) to[lane + 128] = v2;
            if (lane + 192 < n) to[lane + 192] = v3;
            if (lane + 256 < n) to[lane + 256] = v4;
        } else {
            for (std::uint32_t i = lane; i < n; i += lanes) to[i] = from[i];
        }
    }

    // The same record, copied by the console's own lane with eight 16-byte
    // loads in flight at a time: for the split layout's waves, whose
    // consoles reach vblank together and capture in the same iteration.
    __device__ static void capture_own(KState* s, std::uint32_t e_env, std::uint32_t e_regs) {
        const std::uint32_t vs = s->vram_stride;
        std::uint8_t* rec = s->present + static_cast<std::size_t>(e_env) * (present::kHeader + vs);
        rec[0] = s->lat_sx[e_env];
        rec[1] = s->lat_sy[e_env];
        rec[2] = s->lat_ctrl[e_env];
        rec[3] = lds[e_regs + reg::kScrollX];
        rec[4] = lds[e_regs + reg::kScrollY];
        rec[5] = lds[e_regs + reg::kCtrl];
        rec[6] = lds[e_regs + reg::kMask];
        using u32x4 = std::uint32_t __attribute__((ext_vector_type(4)));
        const auto* from = reinterpret_cast<const u32x4*>(s->vram + static_cast<std::size_t>(e_env) * vs);
        auto* to = reinterpret_cast<u32x4*>(rec + present::kHeader);
        const std::uint32_t n = vs / 16;
        constexpr std::uint32_t kPer = 8;
        for (std::uint32_t i = 0; i < n; i += kPer) {
            u32x4 v[kPer];
#pragma unroll
            for (std::uint32_t k = 0; k < kPer; ++k) v[k] = from[i + k < n ? i + k : n - 1];
#pragma unroll
            for (std::uint32_t k = 0; k < kPer; ++k)
                if (i + k < n) to[i + k] = v[k];
        }
    }
};

// Census of one wave (stats mode 3): wave-uniform counters built from ballots
// and the shader clock, added to the launch's totals when the wave is done.
struct WaveCensus {
    std::uint64_t v[census::kCount] = {};
    __device__ __forceinline__ void count(std::uint32_t k, bool any_lane) {
        v[k] += __builtin_amdgcn_ballot_w64(any_lane) != 0 ? 1u : 0u;
    }
    __device__ __forceinline__ void lanes(std::uint32_t k, bool lane_has) {
        v[k] += static_cast<std::uint64_t>(__popcll(__builtin_amdgcn_ballot_w64(lane_has)));
    }
    // Distinct values of `key` among the lanes in `who`.
    __device__ __forceinline__ static std::uint32_t distinct(std::uint32_t key, bool who) {
        std::uint64_t rem = __builtin_amdgcn_ballot_w64(who);
        std::uint32_t k = 0;
        while (rem != 0) {
            const std::uint32_t first = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(rem)) - 1);
            const std::uint32_t pick = __builtin_amdgcn_readlane(key, first);
            rem &= ~__builtin_amdgcn_ballot_w64(key == pick);
            ++k;
        }
        return k;
    }
    __device__ void flush(unsigned long long* out, std::uint32_t lane) const {
        if (out == nullptr || lane != 0) return;
        for (std::uint32_t k = 0; k < census::kCount; ++k)
            if (v[k] != 0) atomicAdd(out + k, static_cast<unsigned long long>(v[k]));
    }
};

// ---- the step kernel ---------------------------------------------------------------
// kStats: 0 none, 1 per-console counters, 2 counters + opcode/PC histograms,
// 3 counters + the census of the launch (WaveCensus).
// kFull: all console RAM in LDS.  kBudget: the per-frame instruction budget can
// bind (a frame always completes within 14,891 instructions, since every
// instruction advances the PPU by at least 6 dots).
// The all-RAM-in-LDS variant (small batches) always runs 4 waves, and the
// tighter launch bound makes it about 1 % faster; the split variant keeps the
// bound of the 8- and 16-wave workgroups (with the tighter one it is 3 % slower).
template <int kStats, bool kFull, bool kBudget>
__global__ void __launch_bounds__(kFull ? 256 : kMaxBlock) step_kernel(DeviceState s, std::uint32_t frameskip, std::uint32_t max_instr,
                                                         std::uint32_t lane_bits) {
    using C = Console<kFull>;
    const std::uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, T = blockDim.x;
    const std::uint32_t L = 1u << lane_bits;
    const std::uint32_t slot = wave * L + lane;
    const std::uint32_t env = xcd_block(blockIdx.x, gridDim.x) * ((T >> 6) * L) + slot;
    const bool mine = lane < L && env < s.n;

    {   // PRG ROM (a 16 KB image mirrored to 32 KB) and the microcode table.
        const std::uint32_t words = (s.prg_mask + 1) / 16;
        const uint4* src = reinterpret_cast<const uint4*>(s.prg_rom);
        uint4* dst = reinterpret_cast<uint4*>(lds);
        for (std::uint32_t i = tid; i < kPrgRomMax / 16; i += T) dst[i] = src[i & (words - 1)];
        // Microcode, with the BRK and NMI vectors (dword 7 of their entries)
        // taken from the PRG image.
        const uint4* tab = reinterpret_cast<const uint4*>(kFull ? &c_micro_full : &c_micro_split);
        const auto vec = [&](std::uint32_t a) {
            return s.prg_rom[a & s.prg_mask] | (static_cast<std::uint32_t>(s.prg_rom[(a + 1) & s.prg_mask]) << 8);
        };
        for (std::uint32_t i = tid; i < mc::kEntries * kMicroBytes / 16; i += T) {
            uint4 v = tab[i];
            if (i == kMicroSlices * 0x00 + 1) v.w = vec(0x7FFE);
            if (i == kMicroSlices * mc::kNmiEntry + 1) v.w = vec(0x7FFA);
            reinterpret_cast<uint4*>(lds + kLdsMicro + (i % kMicroSlices) * kMicroQuarter)[i / kMicroSlices] = v;
        }
    }
    const std::uint32_t base = kLdsRam + (mine ? slot : (T >> 6) * L) * C::kStride;
    const std::uint32_t P = s.pitch;
    // `s` is the kernel's first argument: it starts the kernel-argument segment.
    C c{(KState*)__builtin_amdgcn_kernarg_segment_ptr(), mine ? env : 0u, base, P};
    if constexpr (!kFull) c.vm = s.vram + static_cast<std::size_t>(c.env) * s.vram_stride;
    std::uint32_t fd0 = 0, horizon0 = 0;
    // The countdown may run through a frame end (to_event) unless the frame
    // budget can bind: the frame's instruction count then starts again only at
    // the next event, at most 1,762 instructions later (10,571 dots at six or
    // more per instruction), so a budget of 32,768 or more never binds early.
    const bool through_ok = !kBudget || max_instr >= 32768;
    if (mine) {
        // This console's RAM rows that live in LDS.
        const std::uint8_t* g = s.ram + env;
        auto stage = [&](std::uint32_t ra, std::uint32_t at) {
            const std::size_t r = ra;
            reinterpret_cast<std::uint32_t*>(lds + base + at)[0] =
                g[r * P] | (g[(r + 1) * P] << 8) | (g[(r + 2) * P] << 16) | (static_cast<std::uint32_t>(g[(r + 3) * P]) << 24);
        };
        if (kFull) {
            for (std::uint32_t ra = 0; ra < kRamBytes; ra += 4) stage(ra, ra);
        } else {
            for (std::uint32_t ra = 0; ra < 0x100; ra += 4) stage(ra, C::ram_lds_off(ra));
            for (std::uint32_t ra = 0x180; ra < 0x200; ra += 4) stage(ra, C::ram_lds_off(ra));
        }
        // PPU and pad registers, and the loop state kept off the hot path.
        c.w8(reg::kCtrl, s.ctrl[env]); c.w8(reg::kMask, s.mask[env]);
        c.w8(reg::kOamAddr, s.oam_addr[env]);
        c.w8(reg::kReadBuffer, s.read_buffer[env]); c.w8(reg::kFineX, s.fine_x[env]);
        c.w8(reg::kScrollX, s.scroll_x[env]); c.w8(reg::kScrollY, s.scroll_y[env]);
        c.w16(reg::kV, s.v[env]); c.w16(reg::kT, s.t[env]);
        fd0 = s.frame_dot[env];
        horizon0 = to_event(fd0, frameskip > 1 && through_ok);
        c.w32(reg::kFrameDot, fd0);
        c.w32(reg::kHorizon, horizon0);
        // The pad reads this step's mask; a high strobe re-latches (controller.hpp:20-25).
        const std::uint32_t buttons = s.actions[env], strobe = s.strobe[env];
        c.io = s.open_bus[env] | (s.status[env] << 8) | ((strobe ? buttons : s.c1_shift[env]) << 16) |
               ((strobe ? 0u : s.c1_count[env] & 0xFu) << 24) | (static_cast<std::uint32_t>(s.c2_count[env] & 0xF) << 28);
        c.pc = s.pc[env];
        c.regs = s.a[env] | (s.x[env] << 8) | (s.y[env] << 16) | (static_cast<std::uint32_t>(s.sp[env]) << 24);
        c.p = s.p[env];
        c.flags = (s.nmi_pending[env] ? kNmiPending : 0u) | (s.fault[env] ? kFault : 0u) | (s.w[env] ? kWToggle : 0u) |
                  (strobe ? kStrobeBit : 0u) | (buttons << 8);
        c.set_oam_data(c.vmem()[vram::kOam + s.oam_addr[env]]);
        c.w32(reg::kFramesLeft, (c.flags & kFault) ? 0u : frameskip);
        c.w32(reg::kFrames, 0);
        c.w32(reg::kBudgetHits, 0);
    } else {
        c.pc = 0x8000; c.regs = 0; c.p = 0x20; c.flags = 0; c.io = 0;
    }
    __syncthreads();
    c.nmi_vec = lds[0x7FFA] | (lds[0x7FFB] << 8);
    c.brk_vec = lds[0x7FFE] | (lds[0x7FFF] << 8);
    std::int32_t left = static_cast<std::int32_t>(horizon0);
    std::uint32_t in_frame = 0, instructions = 0;
    bool active = mine && !(c.flags & kFault) && frameskip != 0;
    [[maybe_unused]] bool parked = false;   // waiting at vblank for the rest of the wave
    const std::uint32_t spare = base + C::kSpare;
    // The next instruction's bytes, fetched as soon as its PC is known.
    std::uint32_t op, b1, b2;
    {
        const std::uint32_t off = c.pc & 0x7FFF;
        op = lds[off]; b1 = lds[off + 1]; b2 = lds[off + 2];
    }
    // Code outside PRG ROM: the bytes come through the bus, in order.
    auto fetch_bus = [&]() {
        const std::uint32_t pc = c.pc;
        op = c.bus_rd(pc);
        const std::uint32_t len = (lds[kLdsMicro + 16 * op + 1] >> 4) & 3;  // d0 bits 12-13
        b1 = len >= 2 ? c.bus_rd((pc + 1) & 0xFFFF) : 0u;
        b2 = len >= 3 ? c.bus_rd((pc + 2) & 0xFFFF) : 0u;
        vmem_settled();
    };
    if (active && !(c.flags & kNmiPending) && (c.pc - 0x8000u) > 0x7FFDu) fetch_bus();
    // A pending NMI is taken before the next instruction: its entry stands in
    // for the fetched opcode (the opcode is fetched again after RTI).
    if (c.flags & kNmiPending) op = mc::kNmiEntry;

    // Every lane runs the whole datapath each iteration.  A lane that has
    // finished its frames runs the NOP entry (changes nothing) and a pending
    // NMI runs as its own entry, so the commit needs no selects; only memory
    // and I/O side paths and the rare control cases branch.
    vmem_settled();  // the state loads above complete before the loop

    // Decode of the instruction about to run: microcode slices 0 and 4
    // (addressing, operand and ALU control), effective address, page-cross
    // flag and, in the split layout, the HBM operand.  The split layout
    // decodes one iteration ahead: at the end of an iteration (after its
    // memory writes, on which the decode may depend) or after rare work, so
    // the HBM operand load has a whole iteration to arrive and the operand
    // LDS reads go out with the microcode reads.  With all RAM in LDS (no HBM
    // operand) the decode at the top of the iteration measured faster.
    uint4 ma_c, me_c;
    std::uint32_t ea_c = 0, cross_c = 0, gval_c = 0;
    auto slices = [&](std::uint32_t mi) {
        const std::uint8_t* mw = lds + kLdsMicro + 16 * mi;
        ma_c = *reinterpret_cast<const uint4*>(mw);
        me_c = *reinterpret_cast<const uint4*>(mw + 4 * kMicroQuarter);
    };
    // Zero-page pointer of (zp,X) / (zp),Y (opcode bits select X).
    auto zp_pointer = [&](std::uint32_t o, std::uint32_t lo, std::uint32_t regs) {
        const std::uint32_t pz = (lo + (((o & 0x1F) == 0x01) ? ubfe(regs, 8, 8) : 0u)) & 0xFF;
        return lds[base + C::kZp + pz] | (lds[base + C::kZp + ((pz + 1) & 0xFF)] << 8);
    };
    auto address_at = [&](std::uint32_t ptr, std::uint32_t lo, std::uint32_t hi, std::uint32_t regs) {
        const std::uint32_t abs = lo | (hi << 8);
        const std::uint32_t ebase = sel(me_c.x, ptr, abs);
        const std::uint32_t ea_full = ebase + ubfe(regs, ma_c.x, ma_c.y);
        ea_c = ea_full & me_c.y;
        cross_c = ((ea_full ^ ebase) >> 8) & (ma_c.x >> 7) & 1;
        if constexpr (!kFull) {
            // Every lane loads (no branch); lanes without an HBM operand read
            // row 0, one cache line for the wave, and ignore the byte.
            const bool g = (ma_c.x & 0x100) && ea_c < 0x2000 && !C::ram_in_lds(ea_c & 0x7FF);
            gval_c = s.ram[c.goff(g ? (ea_c & 0x7FF) : 0u)];
        }
    };
    auto address = [&](std::uint32_t o, std::uint32_t lo, std::uint32_t hi, std::uint32_t regs) {
        address_at(zp_pointer(o, lo, regs), lo, hi, regs);
    };
    // Split layout: the decode also leaves the next iteration's microcode
    // row (offset in the slice tables) and stack-window address, and reads
    // the window itself (after this iteration's LDS writes), so the loop top
    // issues its LDS reads without computing their addresses first and the
    // next-PC unit has the window bytes at once.
    [[maybe_unused]] std::uint32_t mwo_c = 0, wb_c = 0;
    [[maybe_unused]] std::uint64_t wq_c = 0;
    auto window_at = [&](std::uint32_t regs) {
        const std::uint32_t sp = regs >> 24;
        return sp >= 0x82u ? base + C::kStk + sp : spare;   // below $0180 (not in LDS): the spare bytes
    };
    if constexpr (!kFull) {
        slices(active ? op : mc::kNopEntry);
        address(op, b1, b2, c.regs);
        mwo_c = 16 * (active ? op : mc::kNopEntry);
        wb_c = window_at(c.regs);
        __builtin_memcpy(&wq_c, lds + wb_c, 8);
    }
    [[maybe_unused]] WaveCensus cz;
    [[maybe_unused]] std::uint64_t t_loop = 0, t_rare = 0;
    if constexpr (kStats == 3) {
        t_loop = clock64();
        cz.count(census::kWaves, active);
    }
    // The loop ends when no lane is active; lanes only stop in the rare work,
    // so only that path tests it.
    if (__builtin_amdgcn_ballot_w64(active) != 0) for (;;) {
        const std::uint32_t pc0 = c.pc, regs0 = c.regs, p0 = c.p;
        const std::uint32_t mi = active ? op : mc::kNopEntry;
        const std::uint8_t* mw = lds + kLdsMicro + (kFull ? 16 * mi : mwo_c);
        if constexpr (kFull) {
            slices(mi);
            address(op, b1, b2, regs0);
        }
        const uint4 ma = ma_c, me = me_c;
        const uint4 mb = *reinterpret_cast<const uint4*>(mw + kMicroQuarter);
        const uint4 mcw = *reinterpret_cast<const uint4*>(mw + 2 * kMicroQuarter);
        const uint4 md = *reinterpret_cast<const uint4*>(mw + 3 * kMicroQuarter);
        const std::uint32_t d0 = ma.x, d1 = ma.y, d2 = ma.z, d3 = ma.w;
        const std::uint32_t d4 = mb.x, d5 = mb.y, d6 = mb.z, d7 = mb.w;
        const std::uint32_t d8 = mcw.x, d9 = mcw.y, d10 = mcw.z, d11 = mcw.w;
        const std::uint32_t d12 = md.x, d13 = md.y, d14 = md.z, d15 = md.w;
        const std::uint32_t d16 = me.x, d18 = me.z, d19 = me.w;   // d17: the address mask, used by the decode

        // Stack window $0100+SP-2 .. $0100+SP+3 (split mode: only when it lies
        // in the LDS half of the page, else a harmless spare area).
        const std::uint32_t sp = regs0 >> 24;
        std::uint32_t wb = base + C::kStk + sp;
        if (!kFull) wb = wb_c;
        // One unaligned 8-byte read; the last two bytes, unused, lie inside
        // the console's block (or its spare and register bytes).
        std::uint64_t wq;
        if constexpr (kFull) {
            __builtin_memcpy(&wq, lds + wb, 8);
        } else {
            wq = wq_c;   // read by the decode
        }
        const std::uint32_t wlo = static_cast<std::uint32_t>(wq), whi = static_cast<std::uint32_t>(wq >> 32);
        const std::uint32_t o2 = wlo & 0xFF, o1 = (wlo >> 8) & 0xFF, o0 = (wlo >> 16) & 0xFF;
        const std::uint32_t w1 = wlo >> 24, w2 = whi & 0xFF, w3 = (whi >> 8) & 0xFF;

        // Effective address and the operand candidates in LDS.
        const std::uint32_t abs = b1 | (b2 << 8);
        const std::uint32_t ea = ea_c, cross = cross_c;
        const std::uint32_t rom_v = lds[ea & 0x7FFF];
        const std::uint32_t ram_a = base + C::ram_lds_off(ea);
        const std::uint32_t ram_v = lds[ram_a];
        // Operand classes.  HBM operands (split layout: RAM rows outside LDS)
        // were loaded by the decode and are merged after the I/O side path.
        // PRG RAM ($6000-$7FFF) goes with the I/O registers through the side
        // path.
        const bool is_ram = ea < 0x2000, rom = ea >= 0x8000;
        const bool ram_lds = is_ram && C::ram_in_lds(ea & 0x7FF);
        const bool glob = is_ram && !ram_lds;
        const bool io = !is_ram && !rom;
        const bool rd = d0 & 0x100, wr = d0 & 0x200;
        const std::uint32_t row = ea & 0x7FF;
        const std::uint32_t gval = gval_c;

        // Next PC: fall through, branch, absolute (JMP/JSR), pulled return
        // address (RTS/RTI) or vector (BRK/NMI); its bytes are fetched now.
        const std::uint32_t fall = (pc0 + ((d0 >> 12) & 3)) & 0xFFFF;
        const std::uint32_t taken = ubfe(p0 ^ ((d2 >> 8) & 0xFF), d2, d3);
        const std::uint32_t target = (fall + static_cast<std::uint32_t>(static_cast<std::int32_t>(static_cast<std::int8_t>(b1)))) & 0xFFFF;
        const std::uint32_t bcyc = ((fall ^ target) & 0xFF00) ? 2u : 1u;
        std::uint32_t next = taken ? target : fall;
        const std::uint32_t wpull = w1 | (w2 << 8) | (w3 << 16);
        const std::uint32_t ret_pc = ((wpull >> d12) + ((d12 >> 16) & 1)) & 0xFFFF;
        next = sel(d9, abs, next);
        next = sel(d10, ret_pc, next);
        next = sel(d11, d7, next);
        std::uint32_t op_n, b1_n, b2_n;
        {
            const std::uint32_t off = next & 0x7FFF;
            // One unaligned 4-byte read; the fourth byte, unused, may lie
            // past the PRG image in the microcode area.
            std::uint32_t ins;
            __builtin_memcpy(&ins, lds + off, 4);
            op_n = ins & 0xFF; b1_n = (ins >> 8) & 0xFF; b2_n = (ins >> 16) & 0xFF;
        }

        // Pushed bytes in window order (SP-2, SP-1, SP), merged with the old
        // window contents.
        const std::uint32_t ret = pc0 + ((d12 >> 24) & 3);
        const std::uint32_t pb = (p0 & 0xEF) | ((d15 >> 8) & 0xFF);
        const std::uint32_t pw = __builtin_amdgcn_perm((regs0 << 8) | pb, ret, d5);
        const std::uint32_t win = sel(d4, pw, o2 | (o1 << 8) | (o0 << 16));
        const bool stack_side = (sp - ((d13 >> 8) & 0xFF)) > ((d13 >> 16) & 0xFF);

        // Operand: LDS (zero page, stack top, PRG ROM), HBM (other RAM rows,
        // PRG RAM), I/O registers, the immediate byte or the pulled byte.
        const std::uint32_t m_lds = rom ? rom_v : ram_v;
        std::uint32_t M = (rd && (rom || ram_lds)) ? m_lds : b1;
        M = sel(d13, w1, M);
        if constexpr (kStats == 3) {
            const bool slow = rd && io && (ea & 0xE007) != 0x2002 && ea != 0x4016;
            cz.count(census::kIoRead, rd && io);
            cz.count(census::kIoReadSlow, slow);
            cz.lanes(census::kLanesIoRead, rd && io);
            cz.lanes(census::kLanesIoReadSlow, slow);
        }
        [[maybe_unused]] std::uint64_t t_io = 0;
        if constexpr (kStats == 3) t_io = clock64();
        if (kFull) {
            if (rd && io) M = c.io_read(ea);   // all RAM is in LDS: no HBM operand
        } else {
            // The side path's result has a register of its own: were it
            // written into M, which shares the HBM load's register, the
            // compiler would wait for that load before the side path.
            std::uint32_t mio = 0;
            if (rd && io) mio = c.io_read(ea);
            M = (rd && io) ? mio : M;
            M = (rd && glob) ? gval : M;
        }
        if constexpr (kStats == 3) {
            if (__builtin_amdgcn_ballot_w64(rd && io) != 0) cz.v[census::kCyclesIoRead] += clock64() - t_io;
        }

        // Adder, logic unit and right shifter.
        const std::uint32_t R = ubfe(regs0, d2, 8);
        const std::uint32_t xa = sel(d18, M, R);
        const std::uint32_t bsrc = (d1 & 0x40) ? xa : M;
        const std::uint32_t xb = (bsrc & ((d1 >> 16) & 0xFF)) ^ (d1 >> 24);
        const std::uint32_t cf = p0 & 1;
        const std::uint32_t sum = xa + xb + ((cf & (d18 >> 8)) | ((d18 >> 16) & 1));
        const std::uint32_t lres = (R & M & ((d2 >> 8) & 0xFF)) | ((R ^ M) & ((d2 >> 16) & 0xFF));
        const std::uint32_t sr = (xa >> 1) | ((cf & (d1 >> 10)) << 7);
        const std::uint32_t ar = (sum & (d2 >> 24)) | lres;
        const std::uint32_t r = sel(d19, sr, ar);
        const std::uint32_t carry = sel(d19, xa, sum >> 8) & 1;
        const std::uint32_t ovf = ((~(xa ^ xb) & (xa ^ sum)) >> 1) & 0x40;
        const std::uint32_t nv_bit = M & 0xC0, nv_alu = (r & 0x80) | ovf;
        // Z by bit arithmetic (r is a byte, so ((r - 1) >> 30) & 2 is 2 exactly
        // when r is 0): a compare and a select on the fresh compare result
        // cost the wave a hazard stall (`s_nop`).  With all RAM in LDS the
        // N/V choice too; the split layout measured 0.6 % slower with it and
        // keeps that select.
        std::uint32_t f;
        if constexpr (kFull) {
            std::uint32_t nvm = static_cast<std::uint32_t>(static_cast<std::int32_t>(d0 << 8) >> 31);
            asm("" : "+v"(nvm));   // keeps the mask a bitwise select
            f = sel(nvm, nv_bit, nv_alu) | (((r - 1u) >> 30) & 2u) | carry;
        } else {
            const std::uint32_t nv = (d0 & 0x800000) ? nv_bit : nv_alu;
            f = nv | (((r - 1u) >> 30) & 2u) | carry;
        }
        const std::uint32_t fm = d0 >> 24;
        const std::uint32_t p1 = (p0 & ~fm) | (f & fm);
        const std::uint32_t pn = sel(d15, (M & 0xCF) | 0x20, (p1 & ((d3 >> 16) & 0xFF)) | (d3 >> 24));
        const std::uint32_t regs_n = sel(d8, r << ((d3 >> 5) & 31), regs0) + d6;

        // Memory writes: the stack window (pushed or old bytes), then the
        // operand to LDS (non-writers store to their spare byte).
        {   // one unaligned 4-byte write: the window bytes and SP+1 as read
            std::uint32_t win4 = (win & 0xFFFFFFu) | (w1 << 24);
            // All RAM in LDS: a push that wraps below $0100 is the stack side
            // path's, and the window's first bytes then lie in the zero page
            // ($00FE-$00FF): they get back what was read.  (The split layout
            // moves the window to the spare bytes before it can leave page 1.)
            if constexpr (kFull) win4 = stack_side ? wlo : win4;
            __builtin_memcpy(lds + wb, &win4, 4);
        }
        const std::uint32_t waddr = (wr && ram_lds) ? ram_a : spare;
        lds[waddr] = static_cast<std::uint8_t>(r);
        // Split layout: the next instruction's zero-page pointer, read right
        // after this instruction's LDS writes (its latency overlaps the
        // commit and the rare-work test).
        std::uint32_t ptr_n = 0;
        uint4 ma_n = ma, me_n = me;
        if constexpr (!kFull) {
            ptr_n = zp_pointer(op_n, b1_n, regs_n);
            // Slices 0 and 4 of the next instruction's microcode, read
            // together with its pointer.
            mwo_c = 16 * (active ? op_n : mc::kNopEntry);
            const std::uint8_t* mw_n = lds + kLdsMicro + mwo_c;
            wb_c = window_at(regs_n);
            __builtin_memcpy(&wq_c, lds + wb_c, 8);
            ma_n = *reinterpret_cast<const uint4*>(mw_n);
            me_n = *reinterpret_cast<const uint4*>(mw_n + 4 * kMicroQuarter);
        }

        // Commit.  The NOP entry leaves everything as it was.
        c.pc = next;
        c.regs = regs_n;
        c.p = pn;
        c.flags &= ~(d14 & mc::kClearNmi);
        op = op_n; b1 = b1_n; b2 = b2_n;
        std::uint32_t dots = 3 * ((d16 >> 16) + cross + (taken ? bcyc : 0u));
        const std::uint32_t counted = d14 & mc::kCount;
        in_frame += counted;
        instructions += counted;
        if constexpr (kStats == 2) {
            if (counted) {
                atomicAdd(&s.prof_opcodes[mi], 1ull);
                atomicAdd(&s.prof_pcs[pc0], 1ull);
            }
        }
        // Rare work, tested once per iteration: I/O register writes, JMP
        // ($xxxx), stack bytes outside the LDS window, the idle loop, illegal
        // opcodes, PPU timing events, the frame budget, OAM DMA and code
        // outside PRG ROM.
        const bool io_write = wr && io;
        const bool side = (d14 & mc::kJmpInd) || stack_side;
        const bool idle = (d14 & mc::kJmpAbs) && abs == pc0;
        const bool timing = counted && (left - static_cast<std::int32_t>(dots)) <= 0;
        const bool budget = kBudget && counted && in_frame >= max_instr;
        // All RAM in LDS: the terms or-ed without short-circuit (no branch
        // in the test; 1.6 % faster there); the split layout measured 4.5 %
        // slower that way and keeps the short-circuit form.
        bool rare;
        if constexpr (kFull) {
            rare = io_write | side | idle | ((d14 & mc::kIllegal) != 0) | timing | budget |
                   ((next - 0x8000u) > 0x7FFDu);
        } else {
            rare = io_write || side || idle || (d14 & mc::kIllegal) || timing || budget ||
                   (next - 0x8000u) > 0x7FFDu;
        }
        if constexpr (kStats == 3) {
            cz.v[census::kIterations] += 1;
            cz.lanes(census::kActiveLanes, active);
            if ((cz.v[census::kIterations] & 15) == 0) {   // sampled: the count costs a loop of ballots
                cz.v[census::kDistinctEntries] += WaveCensus::distinct(mi, active);
                cz.v[census::kDistinctSamples] += 1;
            }
            cz.count(census::kRare, rare);
            cz.count(census::kRareIoWrite, io_write);
            cz.count(census::kRareSide, side);
            cz.count(census::kRareIdle, idle);
            cz.count(census::kRareIllegal, (d14 & mc::kIllegal) != 0);
            cz.count(census::kRareTiming, timing);
            cz.count(census::kRareBudget, budget);
            cz.count(census::kRareOutside, (next - 0x8000u) > 0x7FFDu);
            const bool others = side || idle || (d14 & mc::kIllegal) || timing || budget || (next - 0x8000u) > 0x7FFDu;
            if (__builtin_amdgcn_ballot_w64(others) == 0) cz.count(census::kRareOnlyIoWrite, io_write);
            cz.lanes(census::kLanesIoWrite, io_write);
            cz.lanes(census::kLanesTiming, timing);
        }
        if constexpr (!kFull) s.ram[c.goff((wr && glob) ? row : kTrashRow)] = static_cast<std::uint8_t>(r);
        if constexpr (!kFull) {   // decode of the next instruction
            ma_c = ma_n; me_c = me_n;
            address_at(ptr_n, b1_n, b2_n, regs_n);
        }
        if (__builtin_amdgcn_ballot_w64(rare) == 0) {
            left -= static_cast<std::int32_t>(dots);
            continue;
        }
        c.s = reload(c.s);
        if constexpr (kStats == 3) t_rare = clock64();
        [[maybe_unused]] std::uint64_t t_sub = 0;
        if constexpr (kStats == 3) t_sub = clock64();
        if (io_write) dots += c.io_wr(ea, r);
        if constexpr (kStats == 3) {
            const std::uint64_t t = clock64();
            cz.v[census::kCyclesIoWrite] += t - t_sub;
            t_sub = t;
        }
        if (side) {
            std::uint32_t npc = next;
            if (d14 & mc::kJmpInd) {
                const std::uint32_t l = c.bus_rd(abs);
                npc = l | (c.bus_rd((abs & 0xFF00) | ((abs + 1) & 0xFF)) << 8);
            } else {
                const std::uint32_t npush = (d4 >> 16 & 1) + (d4 >> 8 & 1) + (d4 & 1);
                for (std::uint32_t k = 0; k < npush; ++k)
                    c.ram_wr(0x100 | ((sp - k) & 0xFF), (pw >> (8 * (2 - k))) & 0xFF);
                const std::uint32_t v1 = c.ram_rd(0x100 | ((sp + 1) & 0xFF));
                const std::uint32_t v2 = c.ram_rd(0x100 | ((sp + 2) & 0xFF));
                const std::uint32_t v3 = c.ram_rd(0x100 | ((sp + 3) & 0xFF));
                const std::uint32_t vp = v1 | (v2 << 8) | (v3 << 16);
                const std::uint32_t vret = ((vp >> d12) + ((d12 >> 16) & 1)) & 0xFFFF;
                npc = sel(d10, vret, next);
                // PLA: A = pulled byte with N and Z; PLP / RTI: P = pulled byte.
                const std::uint32_t pa = (p0 & ((d3 >> 16) & 0xFF)) | (d3 >> 24);
                std::uint32_t np = sel(d15, (v1 & 0xCF) | 0x20, pa);
                std::uint32_t nregs = regs0 + d6;
                if (d8 & 0xFF) {
                    nregs = (nregs & ~0xFFu) | v1;
                    np = (np & 0x7D) | (v1 & 0x80) | (v1 == 0 ? 2u : 0u);
                }
                c.regs = nregs;
                c.p = np;
            }
            vmem_settled();
            c.pc = npc;
            const std::uint32_t off = npc & 0x7FFF;
            op = lds[off]; b1 = lds[off + 1]; b2 = lds[off + 2];
        }
        // Idle loop (JMP to itself): the console repeats 3-cycle jumps until
        // the next timing event; account for them in one go.
        const std::int32_t gap = left - static_cast<std::int32_t>(dots);
        if (idle && gap > 0) {
            std::int32_t k = (gap + 8) / 9;
            if (kBudget) {
                const std::int32_t room = static_cast<std::int32_t>(max_instr) - static_cast<std::int32_t>(in_frame);
                k = k < room ? k : room;
            }
            dots += 9u * static_cast<std::uint32_t>(k);
            in_frame += static_cast<std::uint32_t>(k);
            instructions += static_cast<std::uint32_t>(k);
            if constexpr (kStats == 2) {
                atomicAdd(&c.s->prof_opcodes[0x4C], static_cast<unsigned long long>(k));
                atomicAdd(&c.s->prof_pcs[pc0], static_cast<unsigned long long>(k));
            }
        }
        // An illegal opcode freezes the console (the NOP-like entry changed nothing).
        if (d14 & mc::kIllegal) {
            c.flags |= kFault;
            active = false;
        }
        left -= static_cast<std::int32_t>(dots);
        if constexpr (kStats == 3) t_sub = clock64();
        bool at_vblank = false;
        if (counted && left <= 0) {  // a timing event was crossed: settle the PPU
            const std::uint32_t fc = c.settle(c.r32(reg::kHorizon) - static_cast<std::uint32_t>(left), kBudget, &at_vblank);
            std::uint32_t fl = c.r32(reg::kFramesLeft);
            if (fc) {
                c.w32(reg::kFrames, c.r32(reg::kFrames) + 1);
                in_frame = 0;
                fl -= 1;
                c.w32(reg::kFramesLeft, fl);
                if (fl == 0) active = false;
            }
            const std::uint32_t h = to_event(c.r32(reg::kFrameDot), fl > 1 && through_ok);
            c.w32(reg::kHorizon, h);
            left = static_cast<std::int32_t>(h);
        }
        if constexpr (!kFull) {
            // Vblank rendezvous: a console that has just reached vblank waits
            // (runs the NOP entry, its time stopped) until every running
            // console of its wave has reached it too; then all take their NMI
            // together, so the handler's I/O writes, OAM DMA and captures
            // share rare-path entries instead of each console entering alone.
            // Waiting changes no console's results.  Every running console
            // reaches its next vblank within a frame of PPU time (a frame the
            // instruction budget ends early leaves the PPU running), or
            // finishes its frames, and the wave resumes as soon as none is
            // left running, so the wait always ends.  (With
            // all RAM in LDS a wave holds at most 32 consoles and waiting
            // costs more than it saves: 15.28 vs 15.06 ms at 4,096.)
            if (at_vblank && active) {
                parked = true;
                active = false;
            }
            if (__builtin_amdgcn_ballot_w64(active) == 0 && __builtin_amdgcn_ballot_w64(parked) != 0) {
                active = active || parked;
                parked = false;
            }
        }
        if (kBudget && counted && active && in_frame >= max_instr) {  // per-frame budget (cuda_module.cu:1467)
            const std::uint32_t fc = c.settle(c.r32(reg::kHorizon) - static_cast<std::uint32_t>(left), true);
            const std::uint32_t h = to_event(c.r32(reg::kFrameDot), false);
            c.w32(reg::kHorizon, h);
            left = static_cast<std::int32_t>(h);
            c.w32(reg::kFrames, c.r32(reg::kFrames) + fc);
            c.w32(reg::kBudgetHits, c.r32(reg::kBudgetHits) + (fc ? 0u : 1u));
            in_frame = 0;
            const std::uint32_t fl = c.r32(reg::kFramesLeft) - 1;
            c.w32(reg::kFramesLeft, fl);
            if (fl == 0) active = false;
        }
        // OAM DMA ($4014, console.hpp:191-197): the whole wave copies one
        // console's 256 bytes at a time, 4 per lane.  RAM, PRG RAM and PRG ROM
        // pages have no read side effects; I/O pages are read by the console's
        // own lane through the bus, in order.
        if constexpr (kStats == 3) {
            const std::uint64_t t = clock64();
            cz.v[census::kCyclesSettle] += t - t_sub;
            t_sub = t;
        }
        std::uint64_t req = __ballot((c.flags & kDmaPending) != 0);
        if constexpr (kStats == 3) cz.v[census::kDma] += req != 0 ? 1u : 0u;
        if constexpr (!kFull) {
            // Split layout: the vblank rendezvous starts a wave's NMI handlers,
            // and with them their DMAs, in the same iteration.  When eight or
            // more consoles copy pages that live in HBM rows (RAM outside the
            // LDS rows, PRG RAM), each lane copies its own console's page: a
            // row's byte for 64 consoles is one coalesced load.
            const bool dma = (c.flags & kDmaPending) != 0;
            const std::uint32_t page = lds[c.base + C::kRegs + reg::kDmaPage];
            const bool hbm_page = (page < 0x20 && (page & 7) >= 2) || (page >= 0x60 && page < 0x80);
            if (__popcll(req) >= 8 && __builtin_amdgcn_ballot_w64(dma && !hbm_page) == 0) {
                if (dma) {
                    const std::uint32_t row0 = page < 0x20 ? ((page & 7) << 8) : ((page << 8) - 0x5800);
                    const std::uint32_t oa = c.r8(reg::kOamAddr);
                    std::uint8_t* oam = c.vmem() + vram::kOam;
                    std::uint32_t first = 0;
                    for (std::uint32_t i = 0; i < 256; i += 16) {   // 16 loads in flight
                        std::uint32_t v[16];
#pragma unroll
                        for (std::uint32_t k = 0; k < 16; ++k) v[k] = s.ram[c.goff(row0 + i + k)];
#pragma unroll
                        for (std::uint32_t k = 0; k < 16; ++k) oam[(oa + i + k) & 0xFF] = static_cast<std::uint8_t>(v[k]);
                        if (i == 0) first = v[0];
                    }
                    c.set_oam_data(first);   // OAM[OAMADDR] is now the page's first byte
                }
                req = 0;
            }
        }
        while (req != 0) {
            const std::uint32_t src = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(req)) - 1);
            req &= req - 1;
            const std::uint32_t e_env = __builtin_amdgcn_readlane(c.env, src);
            const std::uint32_t e_regs = __builtin_amdgcn_readlane(c.base, src) + C::kRegs;
            const std::uint32_t page = lds[e_regs + reg::kDmaPage];
            const std::uint32_t oa = lds[e_regs + reg::kOamAddr];
            const std::uint32_t e_base = e_regs - C::kRegs;
            std::uint8_t* e_oam = c.s->vram + static_cast<std::size_t>(e_env) * c.s->vram_stride + vram::kOam;
            if (page < 0x20 || page >= 0x60) {
                // All four loads go out before the stores (one round trip).
                std::uint32_t val[4];
#pragma unroll
                for (std::uint32_t k = 0; k < 4; ++k) {
                    const std::uint32_t addr = (page << 8) | (4 * lane + k);
                    if (page < 0x20) {
                        const std::uint32_t ra2 = addr & 0x7FF;
                        val[k] = C::ram_in_lds(ra2) ? lds[e_base + C::ram_lds_off(ra2)] : c.s->ram[__umul24(ra2, P) + e_env];
                    } else if (page < 0x80) {
                        val[k] = c.s->ram[__umul24(addr - 0x5800, P) + e_env];
                    } else {
                        val[k] = lds[addr & 0x7FFF];
                    }
                }
                const std::uint32_t word = val[0] | (val[1] << 8) | (val[2] << 16) | (val[3] << 24);
                if (false) {
                    reinterpret_cast<std::uint32_t*>(e_oam)[((oa >> 2) + lane) & 63] = word;
                } else {
#pragma unroll
                    for (std::uint32_t k = 0; k < 4; ++k)
                        e_oam[(oa + 4 * lane + k) & 0xFF] = static_cast<std::uint8_t>(val[k]);
                }
                // OAM[OAMADDR] is now the page's first byte, lane 0's first.
                const std::uint32_t first = __builtin_amdgcn_readlane(val[0], 0);
                if (lane == src) c.set_oam_data(first);
            } else if (lane == src) {
                // OAMADDR advances with every byte (ppu.hpp:131-134), which a
                // $2004 read inside the copy observes; it wraps back to `oa`.
                std::uint32_t first = 0;
                for (std::uint32_t i = 0; i < 256; ++i) {
                    const std::uint32_t at = (oa + i) & 0xFF;
                    c.w8(reg::kOamAddr, at);
                    c.set_oam_data(e_oam[at]);   // what a $2004 read in the page returns now
                    const std::uint32_t val = c.bus_rd((page << 8) | i);
                    e_oam[at] = static_cast<std::uint8_t>(val);
                    if (i == 0) first = val;
                }
                c.w8(reg::kOamAddr, oa);
                c.set_oam_data(first);
            }
        }
        c.flags &= ~kDmaPending;
        if constexpr (kStats == 3) {
            const std::uint64_t t = clock64();
            cz.v[census::kCyclesDma] += t - t_sub;
            t_sub = t;
        }
        // Presentation snapshot at vblank (batch_ppu.cuh:219-249), after the
        // OAM DMA of the same instruction: the wave copies one console's
        // video memory block at a time (contiguous 16-byte pieces) into its
        // record.  Split layout: a console waiting at the vblank rendezvous
        // captures when the wave resumes (it runs nothing while it waits, so
        // its video memory is what it was at vblank), and when eight or more
        // capture together each lane copies its own console's record.
        if constexpr (kFull) {
            std::uint64_t preq = __ballot((c.flags & kPresentPending) != 0);
            if constexpr (kStats == 3) cz.v[census::kPresent] += preq != 0 ? 1u : 0u;
            while (preq != 0) {
                const std::uint32_t src = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(preq)) - 1);
                preq &= preq - 1;
                const std::uint32_t e_env = __builtin_amdgcn_readlane(c.env, src);
                const std::uint32_t e_regs = __builtin_amdgcn_readlane(c.base, src) + C::kRegs;
                C::capture(c.s, e_env, e_regs, lane, 64);
            }
            c.flags &= ~kPresentPending;
        } else {
            const bool want = (c.flags & kPresentPending) != 0 && !parked;
            std::uint64_t preq = __ballot(want);
            if constexpr (kStats == 3) cz.v[census::kPresent] += preq != 0 ? 1u : 0u;
            if (__popcll(preq) >= 8) {
                if (want) C::capture_own(c.s, env, base + C::kRegs);
            } else {
                while (preq != 0) {
                    const std::uint32_t src = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(preq)) - 1);
                    preq &= preq - 1;
                    const std::uint32_t e_env = __builtin_amdgcn_readlane(c.env, src);
                    const std::uint32_t e_regs = __builtin_amdgcn_readlane(c.base, src) + C::kRegs;
                    C::capture(c.s, e_env, e_regs, lane, 64);
                }
            }
            if (want) c.flags &= ~kPresentPending;
        }
        if constexpr (kStats == 3) cz.v[census::kCyclesPresent] += clock64() - t_sub;
        // Code outside PRG ROM (RAM, PRG RAM, I/O) is fetched through the bus,
        // in order, once the PPU has settled.  NMI pending (set only here, by
        // a $2000 write or the vblank event): its entry runs next.
        if (active && !(c.flags & kNmiPending) && (c.pc - 0x8000u) > 0x7FFDu) fetch_bus();
        if (c.flags & kNmiPending) op = mc::kNmiEntry;
        if (__builtin_amdgcn_ballot_w64(active) == 0) {
            if constexpr (kStats == 3) {
                cz.v[census::kExits] += 1;
                cz.v[census::kCyclesRare] += clock64() - t_rare;
            }
            break;
        }
        if constexpr (!kFull) {
            // The rare work may have changed the next instruction, the
            // registers or RAM: decode again.  (Redoing it only in waves
            // where some lane's instruction, registers or activity changed
            // measured slower.)
            if constexpr (kStats == 3) {
                cz.v[census::kRedo] += 1;
                t_sub = clock64();
            }
            slices(active ? op : mc::kNopEntry);
            address(op, b1, b2, c.regs);
            mwo_c = 16 * (active ? op : mc::kNopEntry);
            wb_c = window_at(c.regs);
            __builtin_memcpy(&wq_c, lds + wb_c, 8);
            if constexpr (kStats == 3) cz.v[census::kCyclesRedo] += clock64() - t_sub;
        }
        if constexpr (kStats == 3) cz.v[census::kCyclesRare] += clock64() - t_rare;
    }
    // The write-back reads the state's fields after the loop.
    c.s = reload(c.s);
    KState& es = *c.s;
    if constexpr (kStats == 3) {
        cz.v[census::kCyclesLoop] += clock64() - t_loop;
        cz.flush(es.census, lane);
    }

    if (!mine) return;
    // Settle the dots of instructions executed since the last event (only a
    // console that faulted stops between events).
    if (left != static_cast<std::int32_t>(c.r32(reg::kHorizon))) {
        c.w32(reg::kFrames,
              c.r32(reg::kFrames) + c.settle(c.r32(reg::kHorizon) - static_cast<std::uint32_t>(left), true));
        if (c.flags & kPresentPending) C::capture(c.s, env, base + C::kRegs, 0, 1);
    }

    // Write the LDS-resident RAM rows and registers back to HBM.
    {
        std::uint8_t* g = es.ram + env;
        auto unstage = [&](std::uint32_t ra, std::uint32_t at) {
            const std::uint32_t v4 = reinterpret_cast<const std::uint32_t*>(lds + base + at)[0];
            const std::size_t r = ra;
            g[r * P] = static_cast<std::uint8_t>(v4);
            g[(r + 1) * P] = static_cast<std::uint8_t>(v4 >> 8);
            g[(r + 2) * P] = static_cast<std::uint8_t>(v4 >> 16);
            g[(r + 3) * P] = static_cast<std::uint8_t>(v4 >> 24);
        };
        if (kFull) {
            for (std::uint32_t ra = 0; ra < kRamBytes; ra += 4) unstage(ra, ra);
        } else {
            for (std::uint32_t ra = 0; ra < 0x100; ra += 4) unstage(ra, C::ram_lds_off(ra));
            for (std::uint32_t ra = 0x180; ra < 0x200; ra += 4) unstage(ra, C::ram_lds_off(ra));
        }
    }
    const std::uint32_t fd = c.r32(reg::kFrameDot);
    const std::uint32_t frames = c.r32(reg::kFrames);
    es.pc[env] = static_cast<std::uint16_t>(c.pc);
    es.a[env] = static_cast<std::uint8_t>(c.regs);
    es.x[env] = static_cast<std::uint8_t>(c.regs >> 8);
    es.y[env] = static_cast<std::uint8_t>(c.regs >> 16);
    es.sp[env] = static_cast<std::uint8_t>(c.regs >> 24);
    es.p[env] = static_cast<std::uint8_t>(c.p);
    // Every CPU cycle is 3 PPU dots.
    const std::uint64_t advanced = static_cast<std::uint64_t>(frames) * kFrameDots + fd - fd0;
    es.cycles[env] += advanced / 3;
    es.frame[env] += frames;
    es.frame_dot[env] = fd;
    es.nmi_pending[env] = static_cast<std::uint8_t>((c.flags & kNmiPending) ? 1 : 0);
    es.status[env] = static_cast<std::uint8_t>(c.status());
    es.ctrl[env] = static_cast<std::uint8_t>(c.r8(reg::kCtrl));
    es.mask[env] = static_cast<std::uint8_t>(c.r8(reg::kMask));
    es.oam_addr[env] = static_cast<std::uint8_t>(c.r8(reg::kOamAddr));
    es.open_bus[env] = static_cast<std::uint8_t>(c.open_bus());
    es.read_buffer[env] = static_cast<std::uint8_t>(c.r8(reg::kReadBuffer));
    es.v[env] = static_cast<std::uint16_t>(c.r16(reg::kV));
    es.t[env] = static_cast<std::uint16_t>(c.r16(reg::kT));
    es.fine_x[env] = static_cast<std::uint8_t>(c.r8(reg::kFineX));
    es.w[env] = static_cast<std::uint8_t>((c.flags & kWToggle) ? 1 : 0);
    es.scroll_x[env] = static_cast<std::uint8_t>(c.r8(reg::kScrollX));
    es.scroll_y[env] = static_cast<std::uint8_t>(c.r8(reg::kScrollY));
    es.c1_buttons[env] = static_cast<std::uint8_t>(c.buttons());
    es.c1_shift[env] = static_cast<std::uint8_t>(c.c1_shift());
    es.c1_count[env] = static_cast<std::uint8_t>(c.c1_count());
    es.strobe[env] = static_cast<std::uint8_t>((c.flags & kStrobeBit) ? 1 : 0);
    es.c2_count[env] = static_cast<std::uint8_t>(c.c2_count());
    const bool fault = (c.flags & kFault) != 0;
    es.fault[env] = static_cast<std::uint8_t>(fault ? 1 : 0);

    float reward = 0.0f;
    std::uint32_t done = 1;
    if (!fault) reward_apply(es, env, GlobalRamOf<KState>{es, env}, &reward, &done);
    es.rewards[env] = reward;
    es.done[env] = static_cast<std::uint8_t>(done);
    if constexpr (kStats != 0) {
        es.stat_instructions[env] = instructions;
        es.stat_frames[env] = frames;
        es.stat_budget_hits[env] = c.r32(reg::kBudgetHits);
    }
}

// Which of the step kernel's translation units this is (see launch_step).
#ifndef NESLE_STEP_PART
#define NESLE_STEP_PART 0
#endif
// Split-layout launches with at most 2^5 consoles per wave take the
// nes_step_narrow.hip instances.
constexpr std::uint32_t kNarrowLaneBits = 5;

struct Geometry {
    std::uint32_t waves, lane_bits, consoles, blocks, lds;
    bool full;
};

// W waves per workgroup (one workgroup per CU), L consoles per wave: the
// smallest power-of-two L with 256 CUs x W x L >= n.  W trades issue slots for
// latency hiding: W/4 waves share each SIMD.
Geometry geometry(std::uint32_t n, std::uint32_t waves) {
    // More consoles per wave while the batch needs them and the workgroup's
    // consoles still fit in LDS with at least the split layout.
    std::uint32_t lane_bits = 0;
    while (lane_bits < 6 && ((256u * waves) << lane_bits) < n &&
           lds_bytes(waves << (lane_bits + 1), false) <= kLdsLimit)
        ++lane_bits;
    Geometry g{};
    g.waves = waves;
    g.lane_bits = lane_bits;
    g.consoles = waves << lane_bits;
    g.blocks = (n + g.consoles - 1) / g.consoles;
    g.full = lds_bytes(g.consoles, true) <= kLdsLimit;
    g.lds = lds_bytes(g.consoles, g.full);
    return g;
}

template <int kStats, bool kFull, bool kBudget>
hipError_t launch_variant(const DeviceState& s, const Geometry& g, std::uint32_t frameskip, std::uint32_t max_instr,
                          hipStream_t stream) {
    step_kernel<kStats, kFull, kBudget><<<dim3(g.blocks), dim3(64 * g.waves), 0, stream>>>(
        s, frameskip, max_instr, g.lane_bits);
    return hipGetLastError();
}

// One layout's kernels, for every statistics mode and frame budget.
template <bool kFull>
hipError_t launch_layout(const DeviceState& s, const Geometry& g, std::uint32_t frameskip, std::uint32_t max_instr,
                         int stats_mode, hipStream_t stream) {
    // A frame needs at most ceil(89,342 / 6) = 14,891 instructions.
    const bool budget = max_instr < 15000;
    if (stats_mode == 3) return launch_variant<3, kFull, true>(s, g, frameskip, max_instr, stream);
    if (stats_mode == 2) return launch_variant<2, kFull, true>(s, g, frameskip, max_instr, stream);
    if (stats_mode == 1) return launch_variant<1, kFull, true>(s, g, frameskip, max_instr, stream);
    return budget ? launch_variant<0, kFull, true>(s, g, frameskip, max_instr, stream)
                  : launch_variant<0, kFull, false>(s, g, frameskip, max_instr, stream);
}

#if NESLE_STEP_PART == 0
// Waves per workgroup: NESLE_WAVES_PER_GROUP (4, 8 or 16) overrides the default.
std::uint32_t waves_per_group() {
    static const std::uint32_t w = [] {
        const char* e = std::getenv("NESLE_WAVES_PER_GROUP");
        const long v = e != nullptr ? std::strtol(e, nullptr, 10) : 0;
        return (v == 4 || v == 8 || v == 16) ? static_cast<std::uint32_t>(v) : 4u;
    }();
    return w;
}
#endif

}  // namespace

// The step kernel's instances come from three translation units, each built
// with its own scheduler flags (nesle_amd/build.py): this file's own
// (NESLE_STEP_PART 0: the split layout at 64 consoles per wave, and
// launch_step), nes_step_full.hip (1: all RAM in LDS) and
// nes_step_narrow.hip (2: the split layout at 16 or 32 consoles per wave).
// Each part recomputes the geometry from the console count and waves per
// workgroup, as launch_step does.
hipError_t launch_step_full(const DeviceState& s, std::uint32_t frameskip, std::uint32_t max_instr, int stats_mode,
                            hipStream_t stream);
hipError_t launch_step_narrow(const DeviceState& s, std::uint32_t waves, std::uint32_t frameskip,
                              std::uint32_t max_instr, int stats_mode, hipStream_t stream);

#if NESLE_STEP_PART == 1
hipError_t launch_step_full(const DeviceState& s, std::uint32_t frameskip, std::uint32_t max_instr, int stats_mode,
                            hipStream_t stream) {
    const Geometry g = geometry(s.n, 4);   // the all-in-LDS kernel is built for 4 waves
    if (!g.full || g.lds > kLdsLimit) return hipErrorInvalidConfiguration;
    return launch_layout<true>(s, g, frameskip, max_instr, stats_mode, stream);
}
#elif NESLE_STEP_PART == 2
hipError_t launch_step_narrow(const DeviceState& s, std::uint32_t waves, std::uint32_t frameskip,
                              std::uint32_t max_instr, int stats_mode, hipStream_t stream) {
    const Geometry g = geometry(s.n, waves);
    if (g.full || g.lane_bits > kNarrowLaneBits || g.lds > kLdsLimit) return hipErrorInvalidConfiguration;
    return launch_layout<false>(s, g, frameskip, max_instr, stats_mode, stream);
}
#else
hipError_t launch_step(const DeviceState& s, std::uint32_t frameskip, std::uint32_t max_instr, int stats_mode,
                       hipStream_t stream) {
    const std::uint32_t waves = waves_per_group();
    const Geometry g = geometry(s.n, waves);
    if (g.full) return launch_step_full(s, frameskip, max_instr, stats_mode, stream);
    if (g.lds > kLdsLimit) return hipErrorInvalidConfiguration;
    if (g.lane_bits <= kNarrowLaneBits) return launch_step_narrow(s, waves, frameskip, max_instr, stats_mode, stream);
    return launch_layout<false>(s, g, frameskip, max_instr, stats_mode, stream);
}
#endif

}  // namespace nesle
