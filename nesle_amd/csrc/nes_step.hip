// nes_step.hip -- the batched NROM console step for gfx950 (MI355X).
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

#include "nes_device.h"
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

constexpr std::uint32_t kMaxBlock = 256;

// Dynamic LDS layout of the step kernel (bytes):
//   [0, 32768)            PRG ROM, a 16 KB image mirrored to fill 32 KB
//   [32768, 32784)        padding read by the two-dword instruction fetch
//   [32784, 34832)        microcode table (256 x 8 B)
//   [34832, +256*T)       zero page of the block's T consoles
//   [.., +128*T)          top of the stack page ($0180-$01FF)
// Console bytes are dword-interleaved: byte `a` of lane t lives in dword
// (a >> 2) * T + t at byte a & 3, so a wave's 64 lanes always touch 64
// different banks whatever addresses they hold.
constexpr std::uint32_t kLdsMicro = 32784;
constexpr std::uint32_t kLdsZp = kLdsMicro + 256 * 8;
constexpr std::uint32_t kZpBytes = 256;
constexpr std::uint32_t kStackLo = 0x180;      // stack bytes $0180-$01FF live in LDS
constexpr std::uint32_t kStackBytes = 128;

constexpr std::uint32_t lds_bytes(std::uint32_t threads) {
    return kLdsZp + (kZpBytes + kStackBytes) * threads;
}

// Maps the hardware block index to the logical console block so that XCD k
// (blocks dispatched round-robin, b % 8 == k) owns one contiguous range.
__device__ __forceinline__ std::uint32_t xcd_block(std::uint32_t b, std::uint32_t nb) {
    const std::uint32_t q = nb >> 3, r = nb & 7, xcd = b & 7;
    return xcd * q + (xcd < r ? xcd : r) + (b >> 3);
}

struct Lane {
    const DeviceState& s;
    std::uint8_t* lds;         // generic pointer to the block's dynamic LDS
    std::uint8_t* ram_lane;    // s.ram + env (generic pointer into HBM)
    std::uint32_t env;
    std::uint32_t pitch;
    std::uint32_t row;         // 4 * threads per block: one dword row of LDS
    std::uint32_t lane4;       // 4 * thread index
    std::uint32_t stk_base;    // LDS offset of the stack rows
    std::uint32_t nmi_vec, brk_vec;
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

    // Generic pointer for a CPU address in RAM ($0000-$1FFF) or PRG ROM
    // ($8000-$FFFF): PRG, zero page and the stack top resolve to LDS, the
    // rest of RAM to HBM.  One FLAT access then serves every lane.
    __device__ __forceinline__ std::uint8_t* gptr(std::uint32_t addr) const {
        const std::uint32_t ra = addr & 0x7FF;
        const bool rom = addr >= 0x8000;
        const bool zp = ra < kZpBytes;
        const bool stk = (ra >> 7) == (kStackLo >> 7);
        const std::uint32_t sub = zp ? ra : (ra & 0x7F);
        const std::uint32_t rowoff = (sub >> 2) * row + lane4 + (sub & 3);
        const std::uint32_t loff = rom ? (addr & 0x7FFF) : (zp ? kLdsZp : stk_base) + rowoff;
        std::uint8_t* lp = lds + loff;
        std::uint8_t* gp = ram_lane + static_cast<std::size_t>(ra) * pitch;
        return (rom || zp || stk) ? lp : gp;
    }

    // ---- console RAM ($0000-$1FFF) -------------------------------------------
    __device__ __forceinline__ std::uint32_t ram_rd(std::uint32_t addr) const { return *gptr(addr & 0x7FF); }
    __device__ __forceinline__ void ram_wr(std::uint32_t addr, std::uint32_t v) const {
        *gptr(addr & 0x7FF) = static_cast<std::uint8_t>(v);
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
                v = rd(ad);
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
    __device__ __forceinline__ static bool is_io(std::uint32_t addr) { return addr >= 0x2000 && addr < 0x8000; }
    __device__ __forceinline__ std::uint32_t rd(std::uint32_t addr) {
        if (is_io(addr)) return io_rd(addr);
        return *gptr(addr);
    }
    __device__ __forceinline__ void wr(std::uint32_t addr, std::uint32_t v) {
        if (addr < 0x2000) {
            ram_wr(addr, v);
        } else if (addr < 0x8000) {
            io_wr(addr, v);
        }
    }

    // ---- one instruction (console.hpp:108-135 + cpu.hpp:377-730) -------------
    // Returns the PPU dots it accounts for (3 per CPU cycle, NMI and DMA
    // included); `op_out`/`pc_out` identify the executed opcode.
    __device__ __forceinline__ std::uint32_t exec(std::uint32_t& op_out, std::uint32_t& pc_out) {
        std::uint32_t cyc = 0;
        if (nmi) {  // cpu.hpp:112-123, taken before the instruction
            nmi = 0;
            *gptr(0x100 | sp) = static_cast<std::uint8_t>(pc >> 8);
            *gptr(0x100 | ((sp - 1) & 0xFF)) = static_cast<std::uint8_t>(pc);
            *gptr(0x100 | ((sp - 2) & 0xFF)) = static_cast<std::uint8_t>((p & ~0x10u) | 0x20u);
            sp = (sp - 3) & 0xFF;
            p |= 0x24;
            pc = nmi_vec;
            cyc = 7;
        }
        pc_out = pc;

        // Fetch the opcode and two operand bytes: two aligned LDS dwords.
        std::uint32_t op, b1, b2;
        if (pc >= 0x8000u && pc <= 0xFFFDu) {
            const std::uint32_t off = pc & 0x7FFF;
            const std::uint32_t* w = reinterpret_cast<const std::uint32_t*>(lds);
            const std::uint32_t bytes = __builtin_amdgcn_alignbyte(w[(off >> 2) + 1], w[off >> 2], off & 3);
            op = bytes & 0xFF;
            b1 = (bytes >> 8) & 0xFF;
            b2 = (bytes >> 16) & 0xFF;
        } else {  // code outside PRG ROM: exact bus reads, in order
            op = rd(pc);
            const std::uint32_t len = static_cast<std::uint32_t>(
                reinterpret_cast<const std::uint64_t*>(lds + kLdsMicro)[op] >> 58) & 3;
            b1 = len >= 2 ? rd((pc + 1) & 0xFFFF) : 0u;
            b2 = len >= 3 ? rd((pc + 2) & 0xFFFF) : 0u;
        }
        op_out = op;
        const std::uint64_t m = reinterpret_cast<const std::uint64_t*>(lds + kLdsMicro)[op];
        // Zero-page pointers for (zp,X) and (zp),Y, read before the decode is known.
        const std::uint32_t px = (b1 + x) & 0xFF;
        const std::uint32_t ptr_x = ram_rd(px) | (ram_rd((px + 1) & 0xFF) << 8);
        const std::uint32_t ptr_y = ram_rd(b1) | (ram_rd((b1 + 1) & 0xFF) << 8);

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
        const std::uint32_t abs = b1 | (b2 << 8);
        const std::uint32_t base = mode == mc::INDX ? ptr_x : (mode == mc::INDY ? ptr_y : abs);
        constexpr std::uint32_t kUsesX = (1u << mc::ZPX) | (1u << mc::ABSX);
        constexpr std::uint32_t kUsesY = (1u << mc::ZPY) | (1u << mc::ABSY) | (1u << mc::INDY);
        constexpr std::uint32_t kZeroPage = (1u << mc::ZP) | (1u << mc::ZPX) | (1u << mc::ZPY);
        const std::uint32_t idx = ((kUsesX >> mode) & 1) ? x : (((kUsesY >> mode) & 1) ? y : 0u);
        const bool zpm = (kZeroPage >> mode) & 1;
        const std::uint32_t addr = zpm ? ((b1 + idx) & 0xFF) : ((base + idx) & 0xFFFF);
        cyc += ((lo >> 7) & 1) & ((!zpm && ((base ^ addr) >> 8) != 0) ? 1u : 0u);

        // Operand: one FLAT load for RAM/PRG lanes, the I/O path for the rest.
        const bool rd_op = (lo >> 13) & 1;
        const bool io = is_io(addr);
        std::uint8_t* const ap = gptr(addr);
        std::uint32_t M = b1;
        if (rd_op && !io) M = *ap;
        if (rd_op && io) M = io_rd(addr);

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
        const bool wr_op = (lo >> 14) & 1;
        if (wr_op && addr < 0x2000) *ap = static_cast<std::uint8_t>(r);
        if (wr_op && io) io_wr(addr, r);

        // Next PC: fall through, branch, or control transfer.
        std::uint32_t next = (pc + ((hi >> 26) & 3)) & 0xFFFF;
        if (kind == mc::KBRANCH) {
            const std::uint32_t pos = (0x1067u >> ((op >> 6) * 4)) & 0xF;
            const bool taken = ((p >> pos) & 1) == ((op >> 5) & 1);
            const std::uint32_t target = (next + static_cast<std::uint32_t>(static_cast<std::int32_t>(static_cast<std::int8_t>(b1)))) & 0xFFFF;
            cyc += taken ? (1u + (((next ^ target) >> 8) != 0 ? 1u : 0u)) : 0u;
            next = taken ? target : next;
        } else if (kind == mc::KCTRL) {
            // Stack unit: JSR/BRK/PHA/PHP push, RTS/RTI/PLA/PLP pull
            // (cpu.hpp:394-402, 603-606, 666-694).
            const std::uint32_t c = (hi >> 22) & 15;
            constexpr std::uint32_t kPushes =
                (2u << (2 * mc::JSR)) | (3u << (2 * mc::BRK)) | (1u << (2 * mc::PHA)) | (1u << (2 * mc::PHP));
            constexpr std::uint32_t kPulls =
                (2u << (2 * mc::RTS)) | (3u << (2 * mc::RTI)) | (1u << (2 * mc::PLA)) | (1u << (2 * mc::PLP));
            const std::uint32_t npush = (kPushes >> (2 * c)) & 3;
            const std::uint32_t npull = (kPulls >> (2 * c)) & 3;
            const std::uint32_t ret = (pc + 2) & 0xFFFF;
            const std::uint32_t pb = p | 0x30;
            const std::uint32_t v0 = c == mc::PHA ? a : (c == mc::PHP ? pb : (ret >> 8));
            if (npush >= 1) *gptr(0x100 | sp) = static_cast<std::uint8_t>(v0);
            if (npush >= 2) *gptr(0x100 | ((sp - 1) & 0xFF)) = static_cast<std::uint8_t>(ret);
            if (npush >= 3) *gptr(0x100 | ((sp - 2) & 0xFF)) = static_cast<std::uint8_t>(pb);
            std::uint32_t w0 = 0, w1 = 0, w2 = 0;
            if (npull >= 1) w0 = *gptr(0x100 | ((sp + 1) & 0xFF));
            if (npull >= 2) w1 = *gptr(0x100 | ((sp + 2) & 0xFF));
            if (npull >= 3) w2 = *gptr(0x100 | ((sp + 3) & 0xFF));
            sp = (sp - npush + npull) & 0xFF;
            const std::uint32_t pulled_p = (w0 | 0x20) & ~0x10u;
            p = (c == mc::RTI || c == mc::PLP) ? pulled_p : (c == mc::BRK ? (p | 0x24) : p);
            if (c == mc::PLA) {
                a = w0;
                p = (p & 0x7D) | (a & 0x80) | (a == 0 ? 2u : 0u) | 0x20;
            }
            next = (c == mc::JMPA || c == mc::JSR) ? abs
                 : c == mc::RTS ? (((w0 | (w1 << 8)) + 1) & 0xFFFF)
                 : c == mc::RTI ? (w1 | (w2 << 8))
                 : c == mc::BRK ? brk_vec : next;
            if (c == mc::JMPI) {  // JMP ($xxxx) with the page-wrap fetch
                const std::uint32_t l = rd(abs);
                next = l | (rd((abs & 0xFF00) | ((abs + 1) & 0xFF)) << 8);
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

// ---- the step kernel ------------------------------------------------------------
// Launched with T = blockDim.x threads (64 or 256) and lds_bytes(T) bytes of
// dynamic LDS.
template <int kStats>
__global__ void __launch_bounds__(kMaxBlock) step_kernel(DeviceState s, std::uint32_t frameskip,
                                                         std::uint32_t max_instr, std::uint32_t auto_reset) {
    extern __shared__ __attribute__((aligned(16))) std::uint8_t lds_raw[];
    const std::uint32_t T = blockDim.x, tid = threadIdx.x;
    {
        // PRG ROM (16 KB images are mirrored so every fetch can use & 0x7FFF)
        // and the microcode table.
        const std::uint32_t bytes = s.prg_mask + 1;
        const uint4* src = reinterpret_cast<const uint4*>(s.prg_rom);
        uint4* dst = reinterpret_cast<uint4*>(lds_raw);
        for (std::uint32_t i = tid; i < kPrgRomMax / 16; i += T) dst[i] = src[i & ((bytes / 16) - 1)];
        if (tid < 1) dst[kPrgRomMax / 16] = src[0];
        std::uint64_t* micro = reinterpret_cast<std::uint64_t*>(lds_raw + kLdsMicro);
        for (std::uint32_t i = tid; i < 256; i += T) micro[i] = c_micro[i];
    }
    const std::uint32_t env = xcd_block(blockIdx.x, gridDim.x) * T + tid;
    const bool live = env < s.n;
    const std::uint32_t stk_base = kLdsZp + kZpBytes * T;
    std::uint32_t* lds32 = reinterpret_cast<std::uint32_t*>(lds_raw);
    if (live) {
        // Stage this console's zero page and stack top into LDS.
        const std::uint8_t* g = s.ram + env;
        const std::size_t P = s.pitch;
        for (std::uint32_t k = 0; k < kZpBytes / 4; ++k) {
            const std::size_t a0 = 4 * k;
            lds32[kLdsZp / 4 + k * T + tid] = g[a0 * P] | (g[(a0 + 1) * P] << 8) | (g[(a0 + 2) * P] << 16) |
                                              (static_cast<std::uint32_t>(g[(a0 + 3) * P]) << 24);
        }
        for (std::uint32_t k = 0; k < kStackBytes / 4; ++k) {
            const std::size_t a0 = kStackLo + 4 * k;
            lds32[stk_base / 4 + k * T + tid] = g[a0 * P] | (g[(a0 + 1) * P] << 8) | (g[(a0 + 2) * P] << 16) |
                                                (static_cast<std::uint32_t>(g[(a0 + 3) * P]) << 24);
        }
    }
    __syncthreads();
    if (!live) return;

    Lane L{s, lds_raw, s.ram + env, env, s.pitch, 4 * T, 4 * tid, stk_base};
    L.nmi_vec = lds_raw[0x7FFA] | (lds_raw[0x7FFB] << 8);
    L.brk_vec = lds_raw[0x7FFE] | (lds_raw[0x7FFF] << 8);
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
        const std::uint32_t dots = L.exec(op, pc0);
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

    // Write the staged zero page and stack top back to HBM.
    {
        std::uint8_t* g = s.ram + env;
        const std::size_t P = s.pitch;
        for (std::uint32_t k = 0; k < kZpBytes / 4; ++k) {
            const std::uint32_t v = lds32[kLdsZp / 4 + k * T + tid];
            const std::size_t a0 = 4 * k;
            g[a0 * P] = static_cast<std::uint8_t>(v);
            g[(a0 + 1) * P] = static_cast<std::uint8_t>(v >> 8);
            g[(a0 + 2) * P] = static_cast<std::uint8_t>(v >> 16);
            g[(a0 + 3) * P] = static_cast<std::uint8_t>(v >> 24);
        }
        for (std::uint32_t k = 0; k < kStackBytes / 4; ++k) {
            const std::uint32_t v = lds32[stk_base / 4 + k * T + tid];
            const std::size_t a0 = kStackLo + 4 * k;
            g[a0 * P] = static_cast<std::uint8_t>(v);
            g[(a0 + 1) * P] = static_cast<std::uint8_t>(v >> 8);
            g[(a0 + 2) * P] = static_cast<std::uint8_t>(v >> 16);
            g[(a0 + 3) * P] = static_cast<std::uint8_t>(v >> 24);
        }
    }

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
    if (!L.fault) reward_apply(s, env, GlobalRam{s, env}, &reward, &done);
    s.rewards[env] = reward;
    s.done[env] = static_cast<std::uint8_t>(done);
    if constexpr (kStats != 0) {
        s.stat_instructions[env] = instructions;
        s.stat_frames[env] = L.frames;
        s.stat_budget_hits[env] = budget_hits;
    }
    if (auto_reset && done) {
        reset_env(s, env, lds_raw);
        seed_baselines(s, env);
    }
}

}  // namespace

std::uint32_t step_block_size(std::uint32_t n) {
    // Small batches: one wave per workgroup spreads consoles over more CUs
    // (each with its own LDS copy of PRG); large batches: 256-thread groups
    // share one copy, keeping 4 groups' LDS under 160 KB per CU.
    return n <= 32768 ? 64u : 256u;
}

hipError_t launch_step(const DeviceState& s, std::uint32_t frameskip, std::uint32_t max_instr,
                       bool auto_reset, int stats_mode, hipStream_t stream) {
    const std::uint32_t T = step_block_size(s.n);
    const std::uint32_t lds = lds_bytes(T);
    const dim3 grid((s.n + T - 1) / T), block(T);
    const std::uint32_t ar = auto_reset ? 1u : 0u;
    if (stats_mode == 2) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&step_kernel<2>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        step_kernel<2><<<grid, block, lds, stream>>>(s, frameskip, max_instr, ar);
    } else if (stats_mode == 1) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&step_kernel<1>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        step_kernel<1><<<grid, block, lds, stream>>>(s, frameskip, max_instr, ar);
    } else {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&step_kernel<0>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        step_kernel<0><<<grid, block, lds, stream>>>(s, frameskip, max_instr, ar);
    }
    return hipGetLastError();
}


}  // namespace nesle
