// nes_kernels.hip -- the batched NROM console step for gfx950 (MI355X).
//
// One wave64 lane per console.  Per launch a lane runs `frameskip` NES frames:
// NMI entry, the 6502 instruction, OAM DMA stall, lazy PPU settlement at the
// timing events, then the reward/done rule and, if asked, a fused auto-reset
// from the snapshot bank.  Semantics follow the reference's CPU core
// (cpp/include/nesle/console.hpp:108-150, cpu.hpp:377-730, ppu.hpp:46-395);
// the launch structure mirrors the reference's console_step_kernel
// (cpp/src/cuda/kernels.cu:19-104) and reset kernels (kernels.cu:177-203).
//
// MI355X-specific choices:
//  * PRG ROM (<= 32 KB) and the 256-entry microcode table are staged into LDS
//    once per workgroup; every opcode/operand fetch is an LDS read.
//  * Instructions execute on one branch-free microcoded datapath
//    (nes_layout.h): a wave's cost does not grow with the number of distinct
//    opcodes its 64 lanes hold; only control-transfer/stack opcodes and I/O
//    registers take divergent paths.
//  * CPU registers and the per-instruction PPU scalars (frame_dot, status,
//    ctrl, mask, nmi) live in VGPRs for the whole launch.
//  * Console RAM and the other per-console arrays are address-major
//    interleaved ([addr][env]) so lanes on the same code path coalesce.
//  * Workgroups are remapped so that each XCD (blockIdx % 8 on MI355X) owns a
//    contiguous range of consoles: interleaved cache lines stay in one L2.
//  * The PPU is settled lazily: only at a timing event (sprite-0 dot, vblank,
//    pre-render, frame end).  The sprite-0 dot is always an event, so the
//    rendering-enable test sees the mask exactly as the reference CPU core's
//    per-dot PPU does.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "nes_launch.h"
#include "nes_layout.h"

namespace nesle {
namespace {

__constant__ std::uint64_t c_micro[256] = {
#define NESLE_E(i) mc::kTable.e[i]
#define NESLE_E8(i) NESLE_E(i), NESLE_E(i + 1), NESLE_E(i + 2), NESLE_E(i + 3), NESLE_E(i + 4), \
                    NESLE_E(i + 5), NESLE_E(i + 6), NESLE_E(i + 7)
#define NESLE_E64(i) NESLE_E8(i), NESLE_E8(i + 8), NESLE_E8(i + 16), NESLE_E8(i + 24), \
                     NESLE_E8(i + 32), NESLE_E8(i + 40), NESLE_E8(i + 48), NESLE_E8(i + 56)
    NESLE_E64(0), NESLE_E64(64), NESLE_E64(128), NESLE_E64(192)
#undef NESLE_E64
#undef NESLE_E8
#undef NESLE_E
};

constexpr std::uint32_t kBlock = 256;

// Maps the hardware block index to the logical console block so that XCD k
// (blocks dispatched round-robin, b % 8 == k) owns one contiguous range.
__device__ __forceinline__ std::uint32_t xcd_block(std::uint32_t b, std::uint32_t nb) {
    const std::uint32_t q = nb >> 3, r = nb & 7, xcd = b & 7;
    return xcd * q + (xcd < r ? xcd : r) + (b >> 3);
}

struct Lane {
    const DeviceState& s;
    const std::uint8_t* prg;   // LDS copy of PRG ROM
    std::uint32_t env;
    std::uint32_t pitch;
    // CPU registers.
    std::uint32_t pc, a, x, y, sp, p;
    std::uint64_t cycles;
    // Per-instruction PPU scalars.
    std::uint32_t frame_dot, status, ctrl, mask, nmi;
    std::uint32_t frames;      // frames completed in this launch
    std::uint32_t dma;         // DMA stall cycles owed by the current instruction
    std::uint32_t fault;

    __device__ __forceinline__ std::uint8_t* cell(std::uint8_t* base, std::uint32_t addr) const {
        return base + (static_cast<std::size_t>(addr) * pitch + env);
    }

    // ---- console RAM ($0000-$1FFF) -------------------------------------------
    __device__ __forceinline__ std::uint32_t ram_rd(std::uint32_t addr) const { return *cell(s.ram, addr & 0x7FF); }
    __device__ __forceinline__ void ram_wr(std::uint32_t addr, std::uint32_t v) const {
        *cell(s.ram, addr & 0x7FF) = static_cast<std::uint8_t>(v);
    }

    // ---- PPU memory (ppu.hpp:280-338) ----------------------------------------
    __device__ std::uint32_t nt_index(std::uint32_t addr) const {
        const std::uint32_t i = (addr - 0x2000) & 0x0FFF;
        if (s.nt_mode == 2) return i;
        if (s.nt_mode == 0) return i & 0x07FF;
        return (i & 0x03FF) | ((i & 0x0800) >> 1);
    }
    __device__ static std::uint32_t pal_index(std::uint32_t addr) {
        std::uint32_t i = addr & 0x1F;
        return ((i & 0x13) == 0x10) ? (i & 0x0F) : i;
    }
    __device__ std::uint32_t vram_rd(std::uint32_t addr) const {
        addr &= 0x3FFF;
        if (addr < 0x2000) {
            if (s.chr_size != 0) return s.chr_rom[addr % s.chr_size];
            return *cell(s.chr_ram, addr & 0x1FFF);
        }
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            return *cell(s.nametable, nt_index(addr));
        }
        return *cell(s.palette, pal_index(addr));
    }
    __device__ void vram_wr(std::uint32_t addr, std::uint32_t v) const {
        addr &= 0x3FFF;
        if (addr < 0x2000) {
            if (s.chr_size == 0) *cell(s.chr_ram, addr & 0x1FFF) = static_cast<std::uint8_t>(v);
            return;
        }
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            *cell(s.nametable, nt_index(addr)) = static_cast<std::uint8_t>(v);
            return;
        }
        *cell(s.palette, pal_index(addr)) = static_cast<std::uint8_t>(v);
    }

    // ---- I/O space $2000-$7FFF (console.hpp:49-101, ppu.hpp:84-134,340-396,
    //      controller.hpp:20-47) -------------------------------------------------
    __device__ std::uint32_t io_rd(std::uint32_t addr) {
        const std::uint32_t e = env;
        if (addr < 0x4000) {
            switch (addr & 7) {
                case 2: {
                    const std::uint32_t val = (status & 0xE0) | (s.open_bus[e] & 0x1F);
                    status &= 0x7F;
                    nmi = 0;
                    s.w[e] = 0;
                    s.open_bus[e] = static_cast<std::uint8_t>(val);
                    return val;
                }
                case 4:
                    return *cell(s.oam, s.oam_addr[e]);
                case 7: {
                    const std::uint32_t va = s.v[e] & 0x3FFF;
                    std::uint32_t val;
                    if (va >= 0x3F00) {
                        val = vram_rd(va);
                        s.read_buffer[e] = static_cast<std::uint8_t>(vram_rd(va - 0x1000));
                    } else {
                        val = s.read_buffer[e];
                        s.read_buffer[e] = static_cast<std::uint8_t>(vram_rd(va));
                    }
                    s.v[e] = static_cast<std::uint16_t>(s.v[e] + ((ctrl & 0x04) ? 32 : 1));
                    s.open_bus[e] = static_cast<std::uint8_t>(val);
                    return val;
                }
                default:
                    return s.open_bus[e];
            }
        }
        if (addr == 0x4016) {
            if (s.strobe[e]) return 0x40 | (s.c1_buttons[e] & 1);
            std::uint32_t bit = 1;
            const std::uint32_t n = s.c1_count[e];
            if (n < 8) {
                const std::uint32_t sh = s.c1_shift[e];
                bit = sh & 1;
                s.c1_shift[e] = static_cast<std::uint8_t>(sh >> 1);
                s.c1_count[e] = static_cast<std::uint8_t>(n + 1);
            }
            return 0x40 | bit;
        }
        if (addr == 0x4017) {
            if (s.strobe[e]) return 0x40;
            const std::uint32_t n = s.c2_count[e];
            if (n < 8) {
                s.c2_count[e] = static_cast<std::uint8_t>(n + 1);
                return 0x40;
            }
            return 0x41;
        }
        if (addr < 0x4018) return *cell(s.apu_io, addr - 0x4000);
        if (addr >= 0x6000) return *cell(s.prg_ram, addr - 0x6000);
        return 0;
    }

    __device__ void ppu_wr(std::uint32_t reg, std::uint32_t val) {
        const std::uint32_t e = env;
        s.open_bus[e] = static_cast<std::uint8_t>(val);
        switch (reg) {
            case 0:
                if ((val & 0x80) && !(ctrl & 0x80) && (status & 0x80)) nmi = 1;
                ctrl = val;
                s.t[e] = static_cast<std::uint16_t>((s.t[e] & 0xF3FF) | ((val & 0x03) << 10));
                break;
            case 1:
                mask = val;
                break;
            case 3:
                s.oam_addr[e] = static_cast<std::uint8_t>(val);
                break;
            case 4: {
                const std::uint32_t oa = s.oam_addr[e];
                *cell(s.oam, oa) = static_cast<std::uint8_t>(val);
                s.oam_addr[e] = static_cast<std::uint8_t>(oa + 1);
                break;
            }
            case 5:
                if (!s.w[e]) {
                    s.fine_x[e] = static_cast<std::uint8_t>(val & 7);
                    s.t[e] = static_cast<std::uint16_t>((s.t[e] & 0xFFE0) | (val >> 3));
                    s.scroll_x[e] = static_cast<std::uint8_t>(val);
                    s.w[e] = 1;
                } else {
                    std::uint32_t t = (s.t[e] & 0x8FFF) | ((val & 0x07) << 12);
                    t = (t & 0xFC1F) | ((val & 0xF8) << 2);
                    s.t[e] = static_cast<std::uint16_t>(t);
                    s.scroll_y[e] = static_cast<std::uint8_t>(val);
                    s.w[e] = 0;
                }
                break;
            case 6:
                if (!s.w[e]) {
                    s.t[e] = static_cast<std::uint16_t>((s.t[e] & 0x00FF) | ((val & 0x3F) << 8));
                    s.w[e] = 1;
                } else {
                    const std::uint16_t t = static_cast<std::uint16_t>((s.t[e] & 0x7F00) | val);
                    s.t[e] = t;
                    s.v[e] = t;
                    s.w[e] = 0;
                }
                break;
            case 7: {
                const std::uint32_t va = s.v[e];
                vram_wr(va, val);
                s.v[e] = static_cast<std::uint16_t>(va + ((ctrl & 0x04) ? 32 : 1));
                break;
            }
            default:
                break;
        }
    }

    // OAM DMA ($4014): 256 bus reads into OAM from OAMADDR, +513 CPU cycles
    // after the instruction (console.hpp:191-197).  Pages below $20 are plain
    // RAM; higher pages go through the full bus with its side effects.
    __device__ void oam_dma(std::uint32_t page) {
        const std::uint32_t oa = s.oam_addr[env];
        const std::uint32_t base = page << 8;
        if (page < 0x20) {
            for (std::uint32_t i = 0; i < 256; ++i) *cell(s.oam, (oa + i) & 0xFF) = static_cast<std::uint8_t>(ram_rd(base + i));
        } else {
            for (std::uint32_t i = 0; i < 256; ++i) {
                const std::uint32_t ad = (base + i) & 0xFFFF;
                std::uint32_t v;
                if (ad < 0x2000) v = ram_rd(ad);
                else if (ad >= 0x8000) v = prg[ad & s.prg_mask];
                else v = io_rd(ad);
                *cell(s.oam, (oa + i) & 0xFF) = static_cast<std::uint8_t>(v);
            }
        }
        dma += 513;
    }

    __device__ void io_wr(std::uint32_t addr, std::uint32_t val) {
        const std::uint32_t e = env;
        if (addr < 0x4000) {
            ppu_wr(addr & 7, val);
            return;
        }
        if (addr == 0x4014) {
            *cell(s.apu_io, 0x14) = static_cast<std::uint8_t>(val);
            oam_dma(val);
            return;
        }
        if (addr == 0x4016) {
            *cell(s.apu_io, 0x16) = static_cast<std::uint8_t>(val);
            const std::uint32_t next = val & 1;
            if (next || s.strobe[e]) {
                s.c1_shift[e] = s.c1_buttons[e];
                s.c1_count[e] = 0;
                s.c2_count[e] = 0;
            }
            s.strobe[e] = static_cast<std::uint8_t>(next);
            return;
        }
        if (addr < 0x4018) {
            *cell(s.apu_io, addr - 0x4000) = static_cast<std::uint8_t>(val);
            return;
        }
        if (addr >= 0x6000) *cell(s.prg_ram, addr - 0x6000) = static_cast<std::uint8_t>(val);
    }

    // ---- CPU bus -------------------------------------------------------------
    __device__ __forceinline__ std::uint32_t rd(std::uint32_t addr) {
        if (addr < 0x2000) return ram_rd(addr);
        if (addr >= 0x8000) return prg[addr & s.prg_mask];
        return io_rd(addr);
    }
    __device__ __forceinline__ void wr(std::uint32_t addr, std::uint32_t v) {
        if (addr < 0x2000) {
            ram_wr(addr, v);
        } else if (addr < 0x8000) {
            io_wr(addr, v);
        }
    }
    __device__ __forceinline__ void push(std::uint32_t v) {
        ram_wr(0x100 | sp, v);
        sp = (sp - 1) & 0xFF;
    }
    __device__ __forceinline__ std::uint32_t pull() {
        sp = (sp + 1) & 0xFF;
        return ram_rd(0x100 | sp);
    }

    // ---- one instruction (console.hpp:108-135 + cpu.hpp:377-730) -------------
    // Returns the PPU dots it accounts for (3 per CPU cycle, NMI and DMA
    // included); `op_out`/`pc_out` identify the executed opcode.
    __device__ __forceinline__ std::uint32_t exec(const std::uint64_t* micro, std::uint32_t& op_out,
                                                  std::uint32_t& pc_out) {
        std::uint32_t cyc = 0;
        if (nmi) {  // cpu.hpp:112-123, taken before the instruction
            nmi = 0;
            push(pc >> 8);
            push(pc & 0xFF);
            push((p & ~0x10u) | 0x20u);
            p |= 0x24;
            pc = prg[0xFFFA & s.prg_mask] | (prg[0xFFFB & s.prg_mask] << 8);
            cyc = 7;
        }
        pc_out = pc;

        // Fetch opcode and up to two operand bytes.
        std::uint32_t op, b1 = 0, b2 = 0;
        std::uint64_t m;
        if (pc >= 0x8000u && pc <= 0xFFFDu) {
            const std::uint32_t pm = s.prg_mask;
            op = prg[pc & pm];
            b1 = prg[(pc + 1) & pm];
            b2 = prg[(pc + 2) & pm];
            m = micro[op];
        } else {
            op = rd(pc);
            m = micro[op];
            const std::uint32_t len = static_cast<std::uint32_t>(m >> 58) & 3;
            if (len >= 2) b1 = rd((pc + 1) & 0xFFFF);
            if (len >= 3) b2 = rd((pc + 2) & 0xFFFF);
        }
        op_out = op;
        const std::uint32_t lo = static_cast<std::uint32_t>(m);
        const std::uint32_t hi = static_cast<std::uint32_t>(m >> 32);
        const std::uint32_t mode = lo & 15;
        const std::uint32_t kind = (lo >> 8) & 3;
        if (kind == mc::KILLEGAL) {
            fault |= 1;
            return 0;
        }
        cyc += (lo >> 4) & 7;

        // Effective address.
        std::uint32_t base = b1 | (b2 << 8);
        if (mode == mc::INDX || mode == mc::INDY) {
            const std::uint32_t ptr = (b1 + (mode == mc::INDX ? x : 0u)) & 0xFF;
            base = ram_rd(ptr) | (ram_rd((ptr + 1) & 0xFF) << 8);
        }
        constexpr std::uint32_t kUsesX = (1u << mc::ZPX) | (1u << mc::ABSX);
        constexpr std::uint32_t kUsesY = (1u << mc::ZPY) | (1u << mc::ABSY) | (1u << mc::INDY);
        constexpr std::uint32_t kZeroPage = (1u << mc::ZP) | (1u << mc::ZPX) | (1u << mc::ZPY);
        const std::uint32_t idx = ((kUsesX >> mode) & 1) ? x : (((kUsesY >> mode) & 1) ? y : 0u);
        std::uint32_t addr;
        if ((kZeroPage >> mode) & 1) {
            addr = (b1 + idx) & 0xFF;
        } else {
            addr = (base + idx) & 0xFFFF;
            cyc += ((lo >> 7) & 1) & (((base ^ addr) >> 8) != 0 ? 1u : 0u);
        }

        // Operand.
        std::uint32_t M = b1;
        if ((lo >> 13) & 1) M = rd(addr);

        // Datapath: adder / logic / shifter.
        const std::uint32_t rsel = (lo >> 10) & 3;
        const std::uint32_t R = rsel == 0 ? a : (rsel == 1 ? x : (rsel == 2 ? y : sp));
        const std::uint32_t xa = ((lo >> 12) & 1) ? M : R;
        const std::uint32_t xb = ((lo >> 19) & 1) ? (M ^ (((lo >> 20) & 1) ? 0xFFu : 0u))
                                                  : (((lo >> 21) & 1) ? 0xFFu : 0u);
        const std::uint32_t csel = (lo >> 22) & 3;
        const std::uint32_t cf = p & 1;
        const std::uint32_t cin = csel == mc::CFLAG ? cf : csel;
        const std::uint32_t sum = xa + xb + cin;
        const std::uint32_t land = R & M, lxor = R ^ M;
        const std::uint32_t lsel = (lo >> 17) & 3;
        const std::uint32_t lres = lsel == mc::LAND ? land : (lsel == mc::LOR ? (land | lxor) : lxor);
        const bool rot = (lo >> 25) & 1;
        const bool right = (lo >> 24) & 1;
        const std::uint32_t sres = right ? ((xa >> 1) | (rot ? cf << 7 : 0u)) : (((xa << 1) | (rot ? cf : 0u)) & 0xFF);
        const std::uint32_t scarry = right ? (xa & 1) : (xa >> 7);
        const std::uint32_t unit = (lo >> 15) & 3;
        const std::uint32_t r = unit == mc::UADD ? (sum & 0xFF) : (unit == mc::ULOGIC ? lres : sres);
        const std::uint32_t carry = unit == mc::USHIFT ? scarry : ((sum >> 8) & 1);
        const std::uint32_t ovf = ((~(xa ^ xb) & (xa ^ sum)) >> 1) & 0x40;
        const bool bit_rule = (lo >> 29) & 1;
        const std::uint32_t f = ((bit_rule ? M : r) & 0x80) | (bit_rule ? (M & 0x40) : ovf) | (r == 0 ? 2u : 0u) | carry;
        const std::uint32_t fmask = ((lo >> 30) | (hi << 2)) & 0xFF;
        const std::uint32_t pand = (hi >> 6) & 0xFF;
        const std::uint32_t por = (hi >> 14) & 0xFF;
        p = ((((p & ~fmask) | (f & fmask)) & pand) | por | 0x20) & 0xFF;

        // Register write-back and memory write.
        const std::uint32_t dst = (lo >> 26) & 7;
        a = dst == mc::DA ? r : a;
        x = dst == mc::DX ? r : x;
        y = dst == mc::DY ? r : y;
        sp = dst == mc::DSP ? r : sp;
        if ((lo >> 14) & 1) wr(addr, r);

        // Next PC: fall through, branch, or control transfer.
        std::uint32_t next = (pc + ((hi >> 26) & 3)) & 0xFFFF;
        if (kind == mc::KBRANCH) {
            const std::uint32_t pos = (0x1067u >> ((op >> 6) * 4)) & 0xF;
            const bool taken = ((p >> pos) & 1) == ((op >> 5) & 1);
            const std::uint32_t target = (next + static_cast<std::uint32_t>(static_cast<std::int32_t>(static_cast<std::int8_t>(b1)))) & 0xFFFF;
            cyc += taken ? (1u + (((next ^ target) >> 8) != 0 ? 1u : 0u)) : 0u;
            next = taken ? target : next;
        } else if (kind == mc::KCTRL) {
            const std::uint32_t abs = b1 | (b2 << 8);
            switch ((hi >> 22) & 15) {
                case mc::JMPA:
                    next = abs;
                    break;
                case mc::JMPI: {
                    const std::uint32_t l = rd(abs);
                    next = l | (rd((abs & 0xFF00) | ((abs + 1) & 0xFF)) << 8);
                    break;
                }
                case mc::JSR: {
                    const std::uint32_t ret = (pc + 2) & 0xFFFF;
                    push(ret >> 8);
                    push(ret & 0xFF);
                    next = abs;
                    break;
                }
                case mc::RTS: {
                    const std::uint32_t l = pull();
                    next = ((l | (pull() << 8)) + 1) & 0xFFFF;
                    break;
                }
                case mc::RTI: {
                    p = (pull() | 0x20) & ~0x10u;
                    const std::uint32_t l = pull();
                    next = l | (pull() << 8);
                    break;
                }
                case mc::BRK: {
                    const std::uint32_t ret = (pc + 2) & 0xFFFF;
                    push(ret >> 8);
                    push(ret & 0xFF);
                    push(p | 0x30);
                    p |= 0x24;
                    next = prg[0xFFFE & s.prg_mask] | (prg[0xFFFF & s.prg_mask] << 8);
                    break;
                }
                case mc::PHA:
                    push(a);
                    break;
                case mc::PHP:
                    push(p | 0x30);
                    break;
                case mc::PLA:
                    a = pull();
                    p = (p & 0x7D) | (a & 0x80) | (a == 0 ? 2u : 0u) | 0x20;
                    break;
                default:  // PLP
                    p = (pull() | 0x20) & ~0x10u;
                    break;
            }
        }
        pc = next;
        cyc += dma;
        dma = 0;
        cycles += cyc;
        return cyc * 3;
    }

    // ---- PPU timing (ppu.hpp:46-76, 136-147) ---------------------------------
    // Dots until the next timing event (sprite-0 dot, vblank, pre-render, frame
    // end) from the current position.  Written with unconditional signed
    // differences: the form with unsigned subtractions guarded by `ev > c` is
    // mis-compiled for gfx950 by ROCm 7.2's clang (the guarded pre-render term
    // is dropped), which the parity tests caught.
    __device__ __forceinline__ std::uint32_t to_event() const {
        const std::int32_t c = static_cast<std::int32_t>(frame_dot);
        std::int32_t d = static_cast<std::int32_t>(kFrameDots) - c;
        const std::int32_t s0 = static_cast<std::int32_t>(kSprite0Dot) - c;
        const std::int32_t vb = static_cast<std::int32_t>(kVblankDot) - c;
        const std::int32_t pr = static_cast<std::int32_t>(kPreRenderDot) - c;
        d = (s0 > 0 && s0 < d) ? s0 : d;
        d = (vb > 0 && vb < d) ? vb : d;
        d = (pr > 0 && pr < d) ? pr : d;
        return static_cast<std::uint32_t>(d);
    }

    // Advance the PPU by `dots` (< one frame past the next frame end) and apply
    // every event crossed, in order.  Returns frames completed (0 or 1).
    __device__ __forceinline__ std::uint32_t settle(std::uint32_t dots) {
        const std::uint32_t start = frame_dot, end = start + dots;
        const std::uint32_t fc = end >= kFrameDots ? 1u : 0u;
        for (std::uint32_t fo = 0; fo <= fc; ++fo) {
            const std::uint32_t off = fo * kFrameDots;
            auto crossed = [&](std::uint32_t ev) { return start < off + ev && off + ev <= end; };
            if (crossed(kSprite0Dot) && (mask & 0x18)) status |= 0x40;
            if (crossed(kVblankDot)) {
                if (!(status & 0x80) && (ctrl & 0x80)) nmi = 1;
                status |= 0x80;
            }
            if (crossed(kPreRenderDot)) {
                status &= 0x1F;
                nmi = 0;
            }
        }
        frame_dot = end - fc * kFrameDots;
        frames += fc;
        return fc;
    }
};

// ---- reward / done (batch_step.cuh:41-106; x-delta rule documented in
//      nes_layout.h) ----------------------------------------------------------
__device__ __forceinline__ void smb_track(const Lane& L, std::int32_t* x, std::int32_t* time) {
    *x = static_cast<std::int32_t>(L.ram_rd(0x6D) * 256 + L.ram_rd(0x86));
    *time = static_cast<std::int32_t>((L.ram_rd(0x7F8) & 15) * 100 + (L.ram_rd(0x7F9) & 15) * 10 + (L.ram_rd(0x7FA) & 15));
}

__device__ __forceinline__ void reward_seed(const Lane& L) {
    const DeviceState& s = L.s;
    if (s.reward_kind == kRewardSmb) {
        std::int32_t x, t;
        smb_track(L, &x, &t);
        s.prev_x[L.env] = x;
        s.prev_time[L.env] = t;
    } else {
        s.prev_x[L.env] = static_cast<std::int32_t>(L.ram_rd(s.x_lo) | (L.ram_rd(s.x_hi) << 8));
        s.prev_time[L.env] = 0;
    }
}

__device__ __forceinline__ void reward_apply(const Lane& L, float* reward, std::uint32_t* done) {
    const DeviceState& s = L.s;
    const std::uint32_t e = L.env;
    if (s.reward_kind == kRewardSmb) {
        std::int32_t x, t;
        smb_track(L, &x, &t);
        std::int32_t dx = x - s.prev_x[e];
        if (dx < -5 || dx > 5) dx = 0;
        std::int32_t dt = t - s.prev_time[e];
        if (dt > 0) dt = 0;
        const std::uint32_t pstate = L.ram_rd(0x0E);
        const bool dying = pstate == 0x0B || L.ram_rd(0xB5) > 1;
        const bool dead = pstate == 0x06;
        const bool over = L.ram_rd(0x75A) == 0xFF;
        bool flag_get = L.ram_rd(0x770) == 2;
        const bool floating = L.ram_rd(0x1D) == 3;
        for (std::uint32_t i = 0; i < 5; ++i) {
            const std::uint32_t en = L.ram_rd(0x16 + i);
            if ((en == 0x2D || en == 0x31) && floating) flag_get = true;
        }
        *reward = static_cast<float>(dx + dt + ((dying || dead) ? -25 : 0));
        *done = (flag_get || dying || dead || over) ? 1u : 0u;
        s.prev_x[e] = x;
        s.prev_time[e] = t;
    } else {
        const std::int32_t x = static_cast<std::int32_t>(L.ram_rd(s.x_lo) | (L.ram_rd(s.x_hi) << 8));
        std::int32_t dx = static_cast<std::int16_t>(static_cast<std::uint16_t>(x - s.prev_x[e]));
        const std::int32_t c = static_cast<std::int32_t>(s.clip);
        dx = dx < -c ? -c : (dx > c ? c : dx);
        *reward = static_cast<float>(dx) - s.time_penalty;
        *done = L.ram_rd(s.done_addr) == 0 ? 1u : 0u;
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

// Load a canonical blob into console `env` (all fields, arrays included).
__device__ void load_blob(const DeviceState& s, std::uint32_t env, const std::uint8_t* b) {
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
    const std::size_t pitch = s.pitch;
    for (std::uint32_t i = 0; i < kApuIoBytes; ++i) s.apu_io[i * pitch + env] = b[kApuIo + i];
    for (std::uint32_t i = 0; i < kRamBytes; ++i) s.ram[i * pitch + env] = b[kRam + i];
    for (std::uint32_t i = 0; i < kPrgRamBytes; ++i) s.prg_ram[i * pitch + env] = b[kPrgRam + i];
    for (std::uint32_t i = 0; i < kOamBytes; ++i) s.oam[i * pitch + env] = b[kOam + i];
    for (std::uint32_t i = 0; i < kPaletteBytes; ++i) s.palette[i * pitch + env] = b[kPalette + i];
    for (std::uint32_t i = 0; i < s.nt_bytes; ++i) s.nametable[i * pitch + env] = b[kNametable + i];
    if (s.chr_ram != nullptr)
        for (std::uint32_t i = 0; i < kChrRamBytes; ++i) s.chr_ram[i * pitch + env] = b[kChrRam + i];
}

// Power-on state: the reference CPU core after construction + reset_cpu
// (console.hpp:38-47,103-106; cpu.hpp:84-92); identical to the reference's
// cold reset of a batched console (batch_step.cuh:109-172).
__device__ void cold_reset(const DeviceState& s, std::uint32_t env, const std::uint8_t* prg) {
    s.pc[env] = static_cast<std::uint16_t>(prg[0xFFFC & s.prg_mask] | (prg[0xFFFD & s.prg_mask] << 8));
    s.a[env] = 0; s.x[env] = 0; s.y[env] = 0; s.sp[env] = 0xFD; s.p[env] = 0x24;
    s.nmi_pending[env] = 0; s.cycles[env] = 7; s.frame[env] = 0; s.frame_dot[env] = 0;
    s.ctrl[env] = 0; s.mask[env] = 0; s.status[env] = 0; s.oam_addr[env] = 0; s.open_bus[env] = 0;
    s.read_buffer[env] = 0; s.v[env] = 0; s.t[env] = 0; s.fine_x[env] = 0; s.w[env] = 0;
    s.scroll_x[env] = 0; s.scroll_y[env] = 0;
    s.c1_buttons[env] = 0; s.c1_shift[env] = 0; s.c1_count[env] = 8; s.strobe[env] = 0; s.c2_count[env] = 8;
    s.fault[env] = 0;
    const std::size_t pitch = s.pitch;
    for (std::uint32_t i = 0; i < kApuIoBytes; ++i) s.apu_io[i * pitch + env] = 0;
    for (std::uint32_t i = 0; i < kRamBytes; ++i) s.ram[i * pitch + env] = 0;
    for (std::uint32_t i = 0; i < kPrgRamBytes; ++i) s.prg_ram[i * pitch + env] = 0;
    for (std::uint32_t i = 0; i < kOamBytes; ++i) s.oam[i * pitch + env] = 0;
    for (std::uint32_t i = 0; i < kPaletteBytes; ++i) s.palette[i * pitch + env] = 0;
    for (std::uint32_t i = 0; i < s.nt_bytes; ++i) s.nametable[i * pitch + env] = 0;
    if (s.chr_ram != nullptr)
        for (std::uint32_t i = 0; i < kChrRamBytes; ++i) s.chr_ram[i * pitch + env] = 0;
}

// Rewards/dones of the terminal step stay visible after the reset, as the
// reference's last_rewards/last_done copies do (cuda_module.cu:635-656).
__device__ __forceinline__ void reset_env(const DeviceState& s, std::uint32_t env, const std::uint8_t* prg) {
    if (s.bank != nullptr) {
        load_blob(s, env, s.bank + static_cast<std::size_t>(s.env_to_level[env]) * blob::kBytes);
    } else {
        cold_reset(s, env, prg);
    }
}

// Reward baselines from the console's current RAM.
__device__ void seed_baselines(const DeviceState& s, std::uint32_t env) {
    Lane L{s, nullptr, env, s.pitch};
    reward_seed(L);
}

// ---- the step kernel ------------------------------------------------------------
template <int kStats>
__global__ void __launch_bounds__(kBlock) step_kernel(DeviceState s, std::uint32_t frameskip,
                                                      std::uint32_t max_instr, std::uint32_t auto_reset) {
    __shared__ __attribute__((aligned(16))) std::uint8_t lds_prg[kPrgRomMax];
    __shared__ std::uint64_t lds_micro[256];
    {
        const std::uint32_t bytes = s.prg_mask + 1;
        const uint4* src = reinterpret_cast<const uint4*>(s.prg_rom);
        uint4* dst = reinterpret_cast<uint4*>(lds_prg);
        for (std::uint32_t i = threadIdx.x; i < bytes / 16; i += kBlock) dst[i] = src[i];
        lds_micro[threadIdx.x] = c_micro[threadIdx.x];
        __syncthreads();
    }
    const std::uint32_t env = xcd_block(blockIdx.x, gridDim.x) * kBlock + threadIdx.x;
    if (env >= s.n) return;

    Lane L{s, lds_prg, env, s.pitch};
    L.pc = s.pc[env]; L.a = s.a[env]; L.x = s.x[env]; L.y = s.y[env]; L.sp = s.sp[env]; L.p = s.p[env];
    L.cycles = s.cycles[env];
    L.frame_dot = s.frame_dot[env]; L.status = s.status[env]; L.ctrl = s.ctrl[env]; L.mask = s.mask[env];
    L.nmi = s.nmi_pending[env];
    L.frames = 0; L.dma = 0; L.fault = s.fault[env];

    // The pad reads this step's mask; a high strobe re-latches immediately
    // (controller.hpp:20-25).
    const std::uint32_t buttons = s.actions[env];
    s.c1_buttons[env] = static_cast<std::uint8_t>(buttons);
    if (s.strobe[env]) {
        s.c1_shift[env] = static_cast<std::uint8_t>(buttons);
        s.c1_count[env] = 0;
    }

    std::uint32_t frames_left = L.fault ? 0u : frameskip;
    std::uint32_t in_frame = 0, pending = 0, horizon = L.to_event();
    std::uint64_t instructions = 0;
    std::uint32_t budget_hits = 0;
    while (frames_left != 0) {
        if (pending >= horizon) {
            const std::uint32_t fc = L.settle(pending);
            pending = 0;
            horizon = L.to_event();
            if (fc) {
                --frames_left;
                in_frame = 0;
                continue;
            }
        }
        std::uint32_t op, pc0;
        const std::uint32_t dots = L.exec(lds_micro, op, pc0);
        if (L.fault) break;
        pending += dots;
        ++in_frame;
        ++instructions;
        if constexpr (kStats == 2) {
            atomicAdd(&s.prof_opcodes[op], 1ull);
            atomicAdd(&s.prof_pcs[pc0], 1ull);
        }
        // Idle loop (JMP to itself): the console repeats 3-cycle jumps until the
        // next timing event is crossed; account for them in one go.
        const std::int32_t gap = static_cast<std::int32_t>(horizon) - static_cast<std::int32_t>(pending);
        if (op == 0x4C && L.pc == pc0 && gap > 0) {
            const std::int32_t room = static_cast<std::int32_t>(max_instr) - static_cast<std::int32_t>(in_frame);
            const std::int32_t want = (gap + 8) / 9;
            const std::uint32_t k = static_cast<std::uint32_t>(want < room ? want : room);
            pending += 9 * k;
            L.cycles += 3ull * k;
            in_frame += k;
            instructions += k;
            if constexpr (kStats == 2) {
                atomicAdd(&s.prof_opcodes[0x4C], static_cast<unsigned long long>(k));
                atomicAdd(&s.prof_pcs[pc0], static_cast<unsigned long long>(k));
            }
        }
        if (in_frame >= max_instr) {  // per-frame budget (cuda_module.cu:1467)
            const std::uint32_t fc = L.settle(pending);
            pending = 0;
            horizon = L.to_event();
            budget_hits += fc ? 0u : 1u;
            --frames_left;
            in_frame = 0;
        }
    }
    if (pending != 0) L.settle(pending);

    s.pc[env] = static_cast<std::uint16_t>(L.pc); s.a[env] = static_cast<std::uint8_t>(L.a);
    s.x[env] = static_cast<std::uint8_t>(L.x); s.y[env] = static_cast<std::uint8_t>(L.y);
    s.sp[env] = static_cast<std::uint8_t>(L.sp); s.p[env] = static_cast<std::uint8_t>(L.p);
    s.cycles[env] = L.cycles;
    s.frame_dot[env] = L.frame_dot; s.frame[env] += L.frames;
    s.status[env] = static_cast<std::uint8_t>(L.status); s.ctrl[env] = static_cast<std::uint8_t>(L.ctrl);
    s.mask[env] = static_cast<std::uint8_t>(L.mask); s.nmi_pending[env] = static_cast<std::uint8_t>(L.nmi);
    s.fault[env] = static_cast<std::uint8_t>(L.fault);

    float reward = 0.0f;
    std::uint32_t done = 1;
    if (!L.fault) reward_apply(L, &reward, &done);
    s.rewards[env] = reward;
    s.done[env] = static_cast<std::uint8_t>(done);
    if constexpr (kStats != 0) {
        s.stat_instructions[env] = instructions;
        s.stat_frames[env] = L.frames;
        s.stat_budget_hits[env] = budget_hits;
    }
    if (auto_reset && done) {
        reset_env(s, env, lds_prg);
        seed_baselines(s, env);
    }
}

// Masked reset: snapshot bank when present, else power-on.
__global__ void __launch_bounds__(kBlock) reset_kernel(DeviceState s, const std::uint8_t* mask) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env >= s.n || (mask != nullptr && mask[env] == 0)) return;
    reset_env(s, env, s.prg_rom);
    seed_baselines(s, env);
}

// Load one blob into every console selected by mask (null = all).
__global__ void __launch_bounds__(kBlock) load_blob_kernel(DeviceState s, const std::uint8_t* blob_src,
                                                           const std::uint8_t* mask) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env >= s.n || (mask != nullptr && mask[env] == 0)) return;
    load_blob(s, env, blob_src);
    seed_baselines(s, env);
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
        v = s.oam[(i - kOam) * pitch + env];
    } else if (i < kNametable) {
        v = s.palette[(i - kPalette) * pitch + env];
    } else if (i < kChrRam) {
        const std::uint32_t k = i - kNametable;
        v = k < s.nt_bytes ? s.nametable[k * pitch + env] : 0;
    } else {
        v = s.chr_ram != nullptr ? s.chr_ram[(i - kChrRam) * pitch + env] : 0;
    }
    out[i] = v;
}

// RAM observation: [2048][pitch] interleaved -> [n][2048] env-major, through
// a 64x64 LDS tile (coalesced on both sides).
__global__ void __launch_bounds__(kBlock) ram_obs_kernel(const std::uint8_t* __restrict__ ram,
                                                         std::uint8_t* __restrict__ obs, std::uint32_t n,
                                                         std::uint32_t pitch) {
    __shared__ std::uint8_t tile[64][65];
    const std::uint32_t env0 = blockIdx.x * 64, addr0 = blockIdx.y * 64;
    const std::uint32_t tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (std::uint32_t r = ty; r < 64; r += 4) {
        const std::uint32_t env = env0 + tx;
        tile[r][tx] = env < pitch ? ram[static_cast<std::size_t>(addr0 + r) * pitch + env] : 0;
    }
    __syncthreads();
    for (std::uint32_t r = ty; r < 64; r += 4) {
        const std::uint32_t env = env0 + r;
        if (env < n) obs[static_cast<std::size_t>(env) * kRamBytes + addr0 + tx] = tile[tx][r];
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

__global__ void __launch_bounds__(kBlock) seed_kernel(DeviceState s) {
    const std::uint32_t env = blockIdx.x * kBlock + threadIdx.x;
    if (env < s.n) seed_baselines(s, env);
}

inline std::uint32_t blocks_for(std::uint32_t n) { return (n + kBlock - 1) / kBlock; }

}  // namespace

hipError_t launch_step(const DeviceState& s, std::uint32_t frameskip, std::uint32_t max_instr,
                       bool auto_reset, int stats_mode, hipStream_t stream) {
    const dim3 grid(blocks_for(s.n)), block(kBlock);
    if (stats_mode == 2) {
        step_kernel<2><<<grid, block, 0, stream>>>(s, frameskip, max_instr, auto_reset ? 1u : 0u);
    } else if (stats_mode == 1) {
        step_kernel<1><<<grid, block, 0, stream>>>(s, frameskip, max_instr, auto_reset ? 1u : 0u);
    } else {
        step_kernel<0><<<grid, block, 0, stream>>>(s, frameskip, max_instr, auto_reset ? 1u : 0u);
    }
    return hipGetLastError();
}

hipError_t launch_reset(const DeviceState& s, const std::uint8_t* mask, hipStream_t stream) {
    reset_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s, mask);
    return hipGetLastError();
}

hipError_t launch_load_blob(const DeviceState& s, const std::uint8_t* blob_src, const std::uint8_t* mask,
                            hipStream_t stream) {
    load_blob_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s, blob_src, mask);
    return hipGetLastError();
}

hipError_t launch_save_blob(const DeviceState& s, std::uint32_t env, std::uint8_t* out, hipStream_t stream) {
    save_blob_kernel<<<dim3(blocks_for(blob::kBytes)), dim3(kBlock), 0, stream>>>(s, env, out);
    return hipGetLastError();
}

hipError_t launch_ram_obs(const DeviceState& s, std::uint8_t* obs, hipStream_t stream) {
    const dim3 grid((s.n + 63) / 64, kRamBytes / 64);
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

hipError_t launch_seed_baselines(const DeviceState& s, hipStream_t stream) {
    seed_kernel<<<dim3(blocks_for(s.n)), dim3(kBlock), 0, stream>>>(s);
    return hipGetLastError();
}

}  // namespace nesle
