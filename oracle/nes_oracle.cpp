// nes_oracle.cpp -- CPU restatement of the reference's NES CPU core.
//
// TEST INFRASTRUCTURE ONLY.  This file is the parity oracle: tests/, the smoke
// check in __graft_entry__.py and the cpu_baseline leg of bench.py load it as a
// checker or as the timed CPU baseline.  The product (nesle_amd/, the HIP
// library) never links, loads or calls it.
//
// It restates, in plain C++ written for this repository, the semantics of the
// reference's scalar console (the "reference C++ CPU core"):
//   * 6502/2A03 interpreter          cpp/include/nesle/cpu.hpp:84-730
//   * console bus + step loop        cpp/include/nesle/console.hpp:49-197
//   * PPU registers, eager per-dot   cpp/include/nesle/ppu.hpp:46-147,280-395
//     timing and VRAM mirroring
//   * standard controller            cpp/include/nesle/controller.hpp:18-67
//   * iNES parse                     cpp/src/rom.cpp:110-166
// plus the reward/done rule of the batched device core
// (cpp/include/nesle/cuda/batch_step.cuh:41-106) and a warm reset from an FCS
// snapshot (batch_step.cuh:174-242).  Each function cites the lines it follows.
//
// Canonical state blob (shared with the HIP library's nesle_read_state and the
// reference harness in oracle/ref_harness.cpp), little endian:
//   0 magic "NST1" | 4 pc u16 | 6 a | 7 x | 8 y | 9 sp | 10 p | 11 nmi_pending
//  12 cycles u64 | 20 frame u64 | 28 frame_dot u32 (scanline*341+dot)
//  32 ctrl | 33 mask | 34 status | 35 oam_addr | 36 open_bus | 37 read_buffer
//  38 v u16 | 40 t u16 | 42 fine_x | 43 w | 44 scroll_x | 45 scroll_y
//  46 c1_buttons | 47 c1_shift | 48 c1_count | 49 strobe | 50 c2_count
//  51 fault flags | 52 pending_dma u32 | 56 apu_io[24] | 80 ram[2048]
//  2128 prg_ram[8192] | 10320 oam[256] | 10576 palette[32]
//  10608 nametable[4096] | 14704 chr_ram[8192] | 22896 end
#include <algorithm>
#include <cmath>
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

constexpr std::size_t kStateBytes = 22896;
constexpr int kDotsPerLine = 341;
constexpr int kLinesPerFrame = 262;

enum : std::uint8_t { kC = 1, kZ = 2, kI = 4, kD = 8, kB = 16, kU = 32, kV = 64, kN = 128 };

struct Cart {
    std::vector<std::uint8_t> prg;
    std::vector<std::uint8_t> chr;
    int nt_mode = 0;  // 0 vertical, 1 horizontal, 2 four-screen
};

// iNES header parse: rom.cpp:110-166 (mapper 0 with one or two PRG banks only,
// console.hpp:38-47).
Cart parse_ines(const std::uint8_t* b, std::size_t n) {
    if (n < 16) throw std::invalid_argument("iNES data is shorter than the 16-byte header");
    if (b[0] != 'N' || b[1] != 'E' || b[2] != 'S' || b[3] != 0x1A)
        throw std::invalid_argument("iNES header magic must be NES<EOF>");
    const bool nes2 = (b[7] & 0x0C) == 0x08;
    if (nes2 && b[9] != 0) throw std::invalid_argument("NES 2.0 extended sizes are not supported");
    unsigned mapper = (b[6] >> 4) | (b[7] & 0xF0);
    if (nes2) mapper |= static_cast<unsigned>(b[8] & 0x0F) << 8;
    const unsigned prg_banks = b[4];
    if (mapper != 0 || (prg_banks != 1 && prg_banks != 2))
        throw std::invalid_argument("only mapper 0/NROM ROMs are supported");
    std::size_t off = 16 + ((b[6] & 0x04) ? 512 : 0);
    const std::size_t prg_n = prg_banks * 16384u, chr_n = b[5] * 8192u;
    if (n < off + prg_n + chr_n) throw std::invalid_argument("iNES data is truncated");
    Cart c;
    c.prg.assign(b + off, b + off + prg_n);
    c.chr.assign(b + off + prg_n, b + off + prg_n + chr_n);
    c.nt_mode = (b[6] & 0x08) ? 2 : ((b[6] & 0x01) ? 0 : 1);
    return c;
}

struct Machine {
    const Cart* cart = nullptr;
    // CPU (cpu.hpp:31-40).
    std::uint16_t pc = 0;
    std::uint8_t a = 0, x = 0, y = 0, sp = 0xFD, p = kU | kI;
    std::uint64_t cycles = 0;
    std::uint8_t fault = 0;
    // Console (console.hpp:199-206).
    std::uint8_t ram[2048] = {};
    std::uint8_t prg_ram[8192] = {};
    std::uint8_t apu_io[24] = {};
    std::uint32_t pending_dma = 0;
    // Controllers (controller.hpp:63-66); pad 2 never has buttons pressed and
    // shares the strobe line with pad 1.
    std::uint8_t c1_buttons = 0, c1_shift = 0, c1_count = 8, strobe = 0, c2_count = 8;
    // PPU (ppu.hpp:547-568).
    std::uint8_t ctrl = 0, mask = 0, status = 0, oam_addr = 0, open_bus = 0, read_buffer = 0;
    std::uint16_t v = 0, t = 0;
    std::uint8_t fine_x = 0, w = 0, nmi_pending = 0, scroll_x = 0, scroll_y = 0;
    int scanline = 0, dot = 0;
    std::uint64_t frame = 0;
    std::uint8_t oam[256] = {};
    std::uint8_t nt[4096] = {};
    std::uint8_t palette[32] = {};
    std::uint8_t chr_ram[8192] = {};
    // Presentation snapshot of the batched core (batch_ppu.cuh:215-260,
    // cuda_module.cu seed_presentation_snapshot): what a rendered frame shows
    // is frozen at every vblank (OAM, nametables, palette and end-of-frame
    // scroll/ctrl/mask); scroll and ctrl are latched at every pre-render line
    // and become the frame-start values of the next snapshot.
    struct Presentation {
        std::uint8_t sx_start = 0, sy_start = 0, ctrl_start = 0, sx_end = 0, sy_end = 0, ctrl_end = 0, mask = 0;
        std::uint8_t oam[256] = {}, nt[4096] = {}, palette[32] = {};
    } snap;
    std::uint8_t lat_sx = 0, lat_sy = 0, lat_ctrl = 0;

    void seed_presentation() {
        std::memcpy(snap.oam, oam, 256);
        std::memcpy(snap.nt, nt, 4096);
        std::memcpy(snap.palette, palette, 32);
        snap.mask = mask;
        lat_sx = snap.sx_start = snap.sx_end = scroll_x;
        lat_sy = snap.sy_start = snap.sy_end = scroll_y;
        lat_ctrl = snap.ctrl_start = snap.ctrl_end = ctrl;
    }
    void capture_presentation() {
        snap.sx_start = lat_sx; snap.sy_start = lat_sy; snap.ctrl_start = lat_ctrl;
        snap.sx_end = scroll_x; snap.sy_end = scroll_y; snap.ctrl_end = ctrl; snap.mask = mask;
        std::memcpy(snap.oam, oam, 256);
        std::memcpy(snap.nt, nt, 4096);
        std::memcpy(snap.palette, palette, 32);
    }

    // ---- PPU memory (ppu.hpp:280-338) -------------------------------------
    static std::uint16_t pal_index(std::uint16_t addr) {
        std::uint16_t i = addr & 0x1F;
        if ((i & 0x13) == 0x10) i &= 0x0F;  // $10/$14/$18/$1C alias $00/$04/$08/$0C
        return i;
    }
    std::uint16_t nt_index(std::uint16_t addr) const {
        const std::uint16_t i = (addr - 0x2000) & 0x0FFF;
        if (cart->nt_mode == 2) return i;
        if (cart->nt_mode == 0) return i & 0x07FF;
        return (i & 0x03FF) | ((i & 0x0800) >> 1);
    }
    std::uint8_t vram_read(std::uint16_t addr) const {
        addr &= 0x3FFF;
        if (addr < 0x2000) {
            if (!cart->chr.empty()) return cart->chr[addr % cart->chr.size()];
            return chr_ram[addr & 0x1FFF];
        }
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            return nt[nt_index(addr)];
        }
        return palette[pal_index(addr)];
    }
    void vram_write(std::uint16_t addr, std::uint8_t val) {
        addr &= 0x3FFF;
        if (addr < 0x2000) {
            if (cart->chr.empty()) chr_ram[addr & 0x1FFF] = val;
            return;
        }
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            nt[nt_index(addr)] = val;
            return;
        }
        palette[pal_index(addr)] = val;
    }

    // ---- PPU registers (ppu.hpp:84-134, 340-396) ---------------------------
    std::uint8_t ppu_reg_read(unsigned reg) {
        switch (reg & 7) {
            case 2: {
                const std::uint8_t val = (status & 0xE0) | (open_bus & 0x1F);
                status &= 0x7F;
                nmi_pending = 0;
                w = 0;
                open_bus = val;
                return val;
            }
            case 4:
                return oam[oam_addr];
            case 7: {
                const std::uint16_t addr = v & 0x3FFF;
                std::uint8_t val;
                if (addr >= 0x3F00) {
                    val = vram_read(addr);
                    read_buffer = vram_read(addr - 0x1000);
                } else {
                    val = read_buffer;
                    read_buffer = vram_read(addr);
                }
                v = static_cast<std::uint16_t>(v + ((ctrl & 0x04) ? 32 : 1));
                open_bus = val;
                return val;
            }
            default:
                return open_bus;
        }
    }
    void ppu_reg_write(unsigned reg, std::uint8_t val) {
        open_bus = val;
        switch (reg & 7) {
            case 0:
                if ((val & 0x80) && !(ctrl & 0x80) && (status & 0x80)) nmi_pending = 1;
                ctrl = val;
                t = static_cast<std::uint16_t>((t & 0xF3FF) | ((val & 0x03) << 10));
                break;
            case 1: mask = val; break;
            case 3: oam_addr = val; break;
            case 4: oam[oam_addr++] = val; break;
            case 5:
                if (!w) {
                    fine_x = val & 7;
                    t = static_cast<std::uint16_t>((t & 0xFFE0) | (val >> 3));
                    scroll_x = val;
                    w = 1;
                } else {
                    t = static_cast<std::uint16_t>((t & 0x8FFF) | ((val & 0x07) << 12));
                    t = static_cast<std::uint16_t>((t & 0xFC1F) | ((val & 0xF8) << 2));
                    scroll_y = val;
                    w = 0;
                }
                break;
            case 6:
                if (!w) {
                    t = static_cast<std::uint16_t>((t & 0x00FF) | ((val & 0x3F) << 8));
                    w = 1;
                } else {
                    t = static_cast<std::uint16_t>((t & 0x7F00) | val);
                    v = t;
                    w = 0;
                }
                break;
            case 7:
                vram_write(v, val);
                v = static_cast<std::uint16_t>(v + ((ctrl & 0x04) ? 32 : 1));
                break;
            default: break;
        }
    }

    // ---- PPU timing, one dot at a time (ppu.hpp:46-76, 136-147) ------------
    // Returns frames completed.
    std::uint32_t ppu_run(std::uint32_t dots) {
        std::uint32_t frames = 0;
        for (std::uint32_t i = 0; i < dots; ++i) {
            if (++dot >= kDotsPerLine) {
                dot = 0;
                if (++scanline >= kLinesPerFrame) {
                    scanline = 0;
                    ++frame;
                    ++frames;
                }
            }
            if (dot != 1) continue;
            if (scanline == 241) {
                if (!(status & 0x80) && (ctrl & 0x80)) nmi_pending = 1;
                status |= 0x80;
                capture_presentation();
            } else if (scanline == 30 && (mask & 0x18)) {
                status |= 0x40;
            } else if (scanline == 261) {
                status &= 0x1F;   // clears vblank, sprite 0 and overflow
                nmi_pending = 0;
                lat_sx = scroll_x; lat_sy = scroll_y; lat_ctrl = ctrl;
            }
        }
        return frames;
    }

    // ---- controllers (controller.hpp:20-47) --------------------------------
    void set_buttons(std::uint8_t m) {
        c1_buttons = m;
        if (strobe) { c1_shift = m; c1_count = 0; }
    }
    void write_strobe(std::uint8_t val) {
        const std::uint8_t next = val & 1;
        if (next || strobe) {
            c1_shift = c1_buttons; c1_count = 0;
            c2_count = 0;           // pad 2 latches its (empty) buttons
        }
        strobe = next;
    }
    std::uint8_t read_pad1() {
        if (strobe) return 0x40 | (c1_buttons & 1);
        std::uint8_t bit = 1;
        if (c1_count < 8) { bit = c1_shift & 1; c1_shift >>= 1; ++c1_count; }
        return 0x40 | bit;
    }
    std::uint8_t read_pad2() {
        if (strobe) return 0x40;
        std::uint8_t bit = 1;
        if (c2_count < 8) { bit = 0; ++c2_count; }
        return 0x40 | bit;
    }

    // ---- CPU bus (console.hpp:49-101, 181-197) -----------------------------
    std::uint8_t read(std::uint16_t addr) {
        if (addr < 0x2000) return ram[addr & 0x7FF];
        if (addr < 0x4000) return ppu_reg_read(addr & 7);
        if (addr == 0x4016) return read_pad1();
        if (addr == 0x4017) return read_pad2();
        if (addr < 0x4018) return apu_io[addr - 0x4000];
        if (addr >= 0x6000 && addr < 0x8000) return prg_ram[addr - 0x6000];
        if (addr >= 0x8000) {
            const std::size_t m = cart->prg.size() == 16384 ? 0x3FFF : 0x7FFF;
            return cart->prg[(addr - 0x8000) & m];
        }
        return 0;
    }
    void write(std::uint16_t addr, std::uint8_t val) {
        if (addr < 0x2000) { ram[addr & 0x7FF] = val; return; }
        if (addr < 0x4000) { ppu_reg_write(addr & 7, val); return; }
        if (addr == 0x4014) {
            apu_io[0x14] = val;
            const std::uint16_t base = static_cast<std::uint16_t>(val << 8);
            for (unsigned i = 0; i < 256; ++i) oam[oam_addr++] = read(static_cast<std::uint16_t>(base + i));
            pending_dma += 513;
            return;
        }
        if (addr == 0x4016) { apu_io[0x16] = val; write_strobe(val); return; }
        if (addr < 0x4018) { apu_io[addr - 0x4000] = val; return; }
        if (addr >= 0x6000 && addr < 0x8000) prg_ram[addr - 0x6000] = val;
    }

    // ---- CPU (cpu.hpp:84-123, 377-730) ---------------------------------------
    void flag(std::uint8_t f, bool on) { p = static_cast<std::uint8_t>(on ? (p | f) : (p & ~f)) | kU; }
    void zn(std::uint8_t val) { flag(kZ, val == 0); flag(kN, val & 0x80); }
    void push(std::uint8_t val) { write(0x0100 | sp, val); --sp; }
    std::uint8_t pull() { ++sp; return read(0x0100 | sp); }
    std::uint16_t read16(std::uint16_t addr) {
        const std::uint16_t lo = read(addr);
        return static_cast<std::uint16_t>(lo | (read(static_cast<std::uint16_t>(addr + 1)) << 8));
    }

    void power_on() {
        // Console construction + reset_cpu (console.hpp:38-47, 103-106; cpu.hpp:84-92).
        a = x = y = 0;
        sp = 0xFD;
        p = kU | kI;
        pc = read16(0xFFFC);
        cycles = 7;
        seed_presentation();   // the batched core seeds it at every full reset
    }

    void nmi() {
        push(pc >> 8);
        push(pc & 0xFF);
        push(static_cast<std::uint8_t>((p & ~kB) | kU));
        flag(kI, true);
        pc = read16(0xFFFA);
        cycles += 7;
    }

    void adc(std::uint8_t m) {
        const unsigned sum = a + m + (p & kC);
        const std::uint8_t r = static_cast<std::uint8_t>(sum);
        flag(kV, (~(a ^ m) & (a ^ r) & 0x80) != 0);
        flag(kC, sum > 0xFF);
        a = r;
        zn(a);
    }
    void cmp(std::uint8_t reg, std::uint8_t m) {
        flag(kC, reg >= m);
        zn(static_cast<std::uint8_t>(reg - m));
    }

    // One instruction; returns its cycle count (without DMA).
    unsigned step() {
        const std::uint8_t op = read(pc++);
        const unsigned hi = op >> 5, mid = (op >> 2) & 7, lo = op & 3;
        unsigned cyc = 0;
        std::uint16_t addr = 0;
        auto fetch = [&]() { return read(pc++); };
        auto fetch16 = [&]() {
            const std::uint16_t l = fetch();
            return static_cast<std::uint16_t>(l | (fetch() << 8));
        };
        auto zp16 = [&](std::uint8_t z) {
            const std::uint16_t l = read(z);
            return static_cast<std::uint16_t>(l | (read(static_cast<std::uint8_t>(z + 1)) << 8));
        };
        auto indexed = [&](std::uint16_t base, std::uint8_t idx, bool penalty) {
            const std::uint16_t e = static_cast<std::uint16_t>(base + idx);
            if (penalty && ((base ^ e) & 0xFF00)) ++cyc;
            return e;
        };
        auto branch = [&](bool take) {
            const std::int8_t off = static_cast<std::int8_t>(fetch());
            cyc = 2;
            if (take) {
                const std::uint16_t dst = static_cast<std::uint16_t>(pc + off);
                cyc += ((pc ^ dst) & 0xFF00) ? 2 : 1;
                pc = dst;
            }
        };
        auto rmw = [&](std::uint8_t (Machine::*fn)(std::uint8_t), unsigned base_cycles) {
            write(addr, (this->*fn)(read(addr)));
            cyc = base_cycles;
        };

        // Branches: xxy10000 (cpu.hpp:695-707).
        if ((op & 0x1F) == 0x10) {
            static const std::uint8_t sel[4] = {kN, kV, kC, kZ};
            branch(((p & sel[op >> 6]) != 0) == ((op & 0x20) != 0));
            return cyc;
        }
        switch (op) {
            // ---- implied / stack / control ----
            case 0x00:  // BRK (cpu.hpp:687-694)
                ++pc;
                push(pc >> 8); push(pc & 0xFF);
                push(p | kB | kU);
                flag(kI, true);
                pc = read16(0xFFFE);
                return 7;
            case 0x20: {  // JSR
                const std::uint16_t target = fetch16();
                const std::uint16_t ret = static_cast<std::uint16_t>(pc - 1);
                push(ret >> 8); push(ret & 0xFF);
                pc = target;
                return 6;
            }
            case 0x40: {  // RTI
                p = static_cast<std::uint8_t>((pull() | kU) & ~kB);
                const std::uint16_t l = pull();
                pc = static_cast<std::uint16_t>(l | (pull() << 8));
                return 6;
            }
            case 0x60: {  // RTS
                const std::uint16_t l = pull();
                pc = static_cast<std::uint16_t>((l | (pull() << 8)) + 1);
                return 6;
            }
            case 0x4C: pc = fetch16(); return 3;
            case 0x6C: {  // JMP (ind) with the page-wrap fetch
                const std::uint16_t ptr = fetch16();
                const std::uint16_t l = read(ptr);
                pc = static_cast<std::uint16_t>(l | (read((ptr & 0xFF00) | ((ptr + 1) & 0xFF)) << 8));
                return 5;
            }
            case 0x08: push(p | kB | kU); return 3;                                  // PHP
            case 0x28: p = static_cast<std::uint8_t>((pull() | kU) & ~kB); return 4;  // PLP
            case 0x48: push(a); return 3;                                            // PHA
            case 0x68: a = pull(); zn(a); return 4;                                  // PLA
            case 0x18: flag(kC, false); return 2;
            case 0x38: flag(kC, true); return 2;
            case 0x58: flag(kI, false); return 2;
            case 0x78: flag(kI, true); return 2;
            case 0xB8: flag(kV, false); return 2;
            case 0xD8: flag(kD, false); return 2;
            case 0xF8: flag(kD, true); return 2;
            case 0xAA: x = a; zn(x); return 2;   // TAX
            case 0xA8: y = a; zn(y); return 2;   // TAY
            case 0x8A: a = x; zn(a); return 2;   // TXA
            case 0x98: a = y; zn(a); return 2;   // TYA
            case 0xBA: x = sp; zn(x); return 2;  // TSX
            case 0x9A: sp = x; return 2;         // TXS
            case 0xE8: ++x; zn(x); return 2;
            case 0xC8: ++y; zn(y); return 2;
            case 0xCA: --x; zn(x); return 2;
            case 0x88: --y; zn(y); return 2;
            case 0xEA: return 2;
            case 0x0A: a = asl(a); return 2;
            case 0x4A: a = lsr(a); return 2;
            case 0x2A: a = rol(a); return 2;
            case 0x6A: a = ror(a); return 2;
            default: break;
        }

        // Remaining official opcodes are the aaabbbcc grid.
        if (lo == 1) {
            // ORA AND EOR ADC STA LDA CMP SBC over (zp,X) zp # abs (zp),Y zp,X abs,Y abs,X.
            const bool store = hi == 4;
            switch (mid) {
                case 0: addr = zp16(static_cast<std::uint8_t>(fetch() + x)); cyc = 6; break;
                case 1: addr = fetch(); cyc = 3; break;
                case 2: addr = pc++; cyc = 2; break;
                case 3: addr = fetch16(); cyc = 4; break;
                case 4: addr = indexed(zp16(fetch()), y, !store); cyc += store ? 6 : 5; break;
                case 5: addr = static_cast<std::uint8_t>(fetch() + x); cyc = 4; break;
                case 6: addr = indexed(fetch16(), y, !store); cyc += store ? 5 : 4; break;
                case 7: addr = indexed(fetch16(), x, !store); cyc += store ? 5 : 4; break;
            }
            if (store && mid == 2) return illegal(op);
            switch (hi) {
                case 0: a |= read(addr); zn(a); break;
                case 1: a &= read(addr); zn(a); break;
                case 2: a ^= read(addr); zn(a); break;
                case 3: adc(read(addr)); break;
                case 4: write(addr, a); break;
                case 5: a = read(addr); zn(a); break;
                case 6: cmp(a, read(addr)); break;
                case 7: adc(static_cast<std::uint8_t>(read(addr) ^ 0xFF)); break;
            }
            return cyc;
        }
        if (lo == 2) {
            // ASL ROL LSR ROR (RMW), STX LDX (zp,Y / abs,Y forms), DEC INC.
            const bool xy = hi == 4 || hi == 5;  // STX/LDX index with Y
            switch (mid) {
                case 0: if (hi != 5) return illegal(op); addr = pc++; cyc = 2; break;  // LDX #
                case 1: addr = fetch(); cyc = 3; break;
                case 3: addr = fetch16(); cyc = 4; break;
                case 5: addr = static_cast<std::uint8_t>(fetch() + (xy ? y : x)); cyc = 4; break;
                case 7:
                    if (hi == 4) return illegal(op);
                    addr = indexed(fetch16(), xy ? y : x, hi == 5);
                    cyc += hi == 5 ? 4 : 5;
                    break;
                default: return illegal(op);
            }
            switch (hi) {
                case 0: rmw(&Machine::asl, cyc + 2); break;
                case 1: rmw(&Machine::rol, cyc + 2); break;
                case 2: rmw(&Machine::lsr, cyc + 2); break;
                case 3: rmw(&Machine::ror, cyc + 2); break;
                case 4: write(addr, x); break;
                case 5: x = read(addr); zn(x); break;
                case 6: rmw(&Machine::dec, cyc + 2); break;
                case 7: rmw(&Machine::inc, cyc + 2); break;
            }
            return cyc;
        }
        if (lo == 0) {
            // BIT (zp/abs), STY, LDY, CPY, CPX.
            if (hi < 1 || hi == 2 || hi == 3) return illegal(op);
            switch (mid) {
                case 0: if (hi < 5) return illegal(op); addr = pc++; cyc = 2; break;
                case 1: addr = fetch(); cyc = 3; break;
                case 3: addr = fetch16(); cyc = 4; break;
                case 5: if (hi != 4 && hi != 5) return illegal(op);
                        addr = static_cast<std::uint8_t>(fetch() + x); cyc = 4; break;
                case 7: if (hi != 5) return illegal(op);
                        addr = indexed(fetch16(), x, true); cyc += 4; break;
                default: return illegal(op);
            }
            switch (hi) {
                case 1: {  // BIT
                    const std::uint8_t m = read(addr);
                    flag(kZ, (a & m) == 0);
                    flag(kN, m & 0x80);
                    flag(kV, m & 0x40);
                    break;
                }
                case 4: write(addr, y); break;
                case 5: y = read(addr); zn(y); break;
                case 6: cmp(y, read(addr)); break;
                case 7: cmp(x, read(addr)); break;
            }
            return cyc;
        }
        return illegal(op);
    }

    unsigned illegal(std::uint8_t) {
        fault |= 1;
        throw std::runtime_error("illegal 6502 opcode");
    }

    std::uint8_t asl(std::uint8_t m) { flag(kC, m & 0x80); m <<= 1; zn(m); return m; }
    std::uint8_t lsr(std::uint8_t m) { flag(kC, m & 1); m >>= 1; zn(m); return m; }
    std::uint8_t rol(std::uint8_t m) {
        const std::uint8_t c = p & kC;
        flag(kC, m & 0x80);
        m = static_cast<std::uint8_t>((m << 1) | c);
        zn(m);
        return m;
    }
    std::uint8_t ror(std::uint8_t m) {
        const std::uint8_t c = p & kC;
        flag(kC, m & 1);
        m = static_cast<std::uint8_t>((m >> 1) | (c << 7));
        zn(m);
        return m;
    }
    std::uint8_t inc(std::uint8_t m) { ++m; zn(m); return m; }
    std::uint8_t dec(std::uint8_t m) { --m; zn(m); return m; }

    // console.hpp:108-135: NMI is taken before the instruction, DMA stall is
    // added after it, then the PPU runs 3 dots per CPU cycle.
    std::uint32_t step_instruction() {
        const std::uint64_t before = cycles;
        if (nmi_pending) { nmi_pending = 0; nmi(); }
        cycles += step();
        if (pending_dma) { cycles += pending_dma; pending_dma = 0; }
        return ppu_run(static_cast<std::uint32_t>(cycles - before) * 3u);
    }

    // console.hpp:137-150.
    std::uint64_t step_frame(std::uint64_t max_instructions) {
        std::uint64_t n = 0;
        std::uint32_t frames = 0;
        while (n < max_instructions) {
            frames += step_instruction();
            ++n;
            if (frames) break;
        }
        return n;
    }

    // ---- frame rendering (batch_render.cuh:161-440, ppu.hpp:213-230,397-545) --
    // The state one frame is drawn from.
    struct View {
        std::uint8_t ctrl, mask, sx, sy;
        const std::uint8_t *nt, *pal, *oam;
    };
    // Two rule sets.  `cpu`: the reference CPU core's renderer (live state,
    // a background pixel is opaque when its pattern colour is non-zero, CHR
    // RAM is read).  Otherwise the batched core's renderer: a background pixel
    // counts as transparent when its palette value is 0, CHR RAM reads as 0,
    // and the frame comes from the presentation snapshot when `snapshot`.
    std::uint8_t ppu_view_read(const View& w, std::uint16_t addr, bool cpu) const {
        addr &= 0x3FFF;
        if (addr < 0x2000) {
            if (!cart->chr.empty()) return cart->chr[addr % cart->chr.size()];
            return cpu ? chr_ram[addr & 0x1FFF] : 0;
        }
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            return w.nt[nt_index(addr)];
        }
        return w.pal[pal_index(addr)];
    }
    std::uint8_t palette_value(const View& w, unsigned index, bool cpu) const {
        std::uint8_t v = ppu_view_read(w, static_cast<std::uint16_t>(0x3F00 + index), cpu);
        if (w.mask & 0x01) v &= 0x30;
        return v & 0x3F;
    }
    unsigned pattern_colour(const View& w, unsigned tile_base, unsigned fx, unsigned fy, bool cpu) const {
        const unsigned lo = ppu_view_read(w, static_cast<std::uint16_t>(tile_base + fy), cpu);
        const unsigned hi = ppu_view_read(w, static_cast<std::uint16_t>(tile_base + fy + 8), cpu);
        const unsigned bit = 7 - fx;
        return ((lo >> bit) & 1) | (((hi >> bit) & 1) << 1);
    }
    // Background at (x, y): *colour = pattern colour (0 transparent), returns
    // the palette value (0 when transparent).
    std::uint8_t background(const View& w, unsigned x, unsigned y, unsigned* colour, bool cpu) const {
        *colour = 0;
        if (!(w.mask & 0x08) || (!(w.mask & 0x02) && x < 8)) return 0;
        const unsigned wy = w.sy + y, wx = w.sx + x;
        const unsigned coarse_y = (wy % 240) / 8, fine_y = wy & 7;
        const unsigned base_nt = w.ctrl & 3;
        const unsigned nt_y = ((base_nt >> 1) + wy / 240) & 1;
        const unsigned coarse_x = (wx & 0xFF) / 8, fine_x = wx & 7;
        const unsigned nt_x = ((base_nt & 1) + wx / 256) & 1;
        const unsigned nt_base = 0x2000 + (nt_x | (nt_y << 1)) * 0x400;
        const unsigned pattern_base = (w.ctrl & 0x10) ? 0x1000 : 0;
        const unsigned tile = ppu_view_read(w, static_cast<std::uint16_t>(nt_base + coarse_y * 32 + coarse_x), cpu);
        const unsigned c = pattern_colour(w, pattern_base + tile * 16, fine_x, fine_y, cpu);
        if (c == 0) return 0;
        *colour = c;
        const unsigned attr = ppu_view_read(w, static_cast<std::uint16_t>(nt_base + 0x3C0 + (coarse_y / 4) * 8 + coarse_x / 4), cpu);
        const unsigned shift = ((coarse_y & 2) << 1) | (coarse_x & 2);
        return palette_value(w, ((attr >> shift) & 3) * 4 + c, cpu);
    }
    unsigned sprite_colour(const View& w, unsigned tile, unsigned attr, unsigned px, unsigned py, bool cpu) const {
        if (attr & 0x40) px = 7 - px;
        if (w.ctrl & 0x20) {
            if (attr & 0x80) py = 15 - py;
            const unsigned base = (tile & 1) ? 0x1000 : 0;
            const unsigned t = ((tile & 0xFE) + py / 8) & 0xFF;
            return pattern_colour(w, base + t * 16, px, py & 7, cpu);
        }
        if (attr & 0x80) py = 7 - py;
        const unsigned base = (w.ctrl & 0x08) ? 0x1000 : 0;
        return pattern_colour(w, base + tile * 16, px, py, cpu);
    }
    // One frame of palette values (0..63), 240 rows x 256.
    void render(std::uint8_t* out, bool snapshot, bool cpu) const {
        const View live{ctrl, mask, scroll_x, scroll_y, nt, palette, oam};
        View play = live, hud = live;
        int split = 0;
        if (snapshot && !cpu) {
            play = View{snap.ctrl_end, snap.mask, snap.sx_end, snap.sy_end, snap.nt, snap.palette, snap.oam};
            hud = View{snap.ctrl_start, snap.mask, snap.sx_start, snap.sy_start, snap.nt, snap.palette, snap.oam};
            split = snap.oam[0] + 1 + ((play.ctrl & 0x20) ? 16 : 8);
            if (split >= 240) { play = hud; split = 0; }
        }
        for (unsigned y = 0; y < 240; ++y) {
            for (unsigned x = 0; x < 256; ++x) {
                unsigned c = 0;
                const View& bs = static_cast<int>(y) < split ? hud : play;
                const std::uint8_t bgv = background(bs, x, y, &c, cpu);
                const bool bg_opaque = cpu ? (c != 0) : (bgv != 0);
                std::uint8_t colour = bg_opaque ? bgv : palette_value(play, 0, cpu);
                if ((play.mask & 0x10) && ((play.mask & 0x04) || x >= 8)) {
                    const unsigned h = (play.ctrl & 0x20) ? 16 : 8;
                    for (unsigned sp = 0; sp < 64; ++sp) {
                        const int sy = static_cast<int>(y) - (play.oam[4 * sp] + 1);
                        const int sx = static_cast<int>(x) - play.oam[4 * sp + 3];
                        if (sy < 0 || sy >= static_cast<int>(h) || sx < 0 || sx >= 8) continue;
                        const unsigned attr = play.oam[4 * sp + 2];
                        if (attr & 0x20) {   // behind the background
                            unsigned c2 = 0;
                            const std::uint8_t v2 = background(play, x, y, &c2, cpu);
                            if (cpu ? (c2 != 0) : (v2 != 0)) continue;
                        }
                        const unsigned sc = sprite_colour(play, play.oam[4 * sp + 1], attr, sx, sy, cpu);
                        if (sc == 0) continue;
                        colour = palette_value(play, 0x10 + (attr & 3) * 4 + sc, cpu);
                        break;
                    }
                }
                out[y * 256 + x] = colour;
            }
        }
    }

    // ---- canonical state blob ------------------------------------------------
    void save(std::uint8_t* o) const {
        std::memset(o, 0, kStateBytes);
        std::memcpy(o, "NST1", 4);
        auto u16 = [&](std::size_t off, std::uint16_t val) { o[off] = val & 0xFF; o[off + 1] = val >> 8; };
        auto u32 = [&](std::size_t off, std::uint32_t val) { for (int i = 0; i < 4; ++i) o[off + i] = (val >> (8 * i)) & 0xFF; };
        auto u64 = [&](std::size_t off, std::uint64_t val) { for (int i = 0; i < 8; ++i) o[off + i] = (val >> (8 * i)) & 0xFF; };
        u16(4, pc); o[6] = a; o[7] = x; o[8] = y; o[9] = sp; o[10] = p; o[11] = nmi_pending;
        u64(12, cycles); u64(20, frame); u32(28, static_cast<std::uint32_t>(scanline * kDotsPerLine + dot));
        o[32] = ctrl; o[33] = mask; o[34] = status; o[35] = oam_addr; o[36] = open_bus; o[37] = read_buffer;
        u16(38, v); u16(40, t); o[42] = fine_x; o[43] = w; o[44] = scroll_x; o[45] = scroll_y;
        o[46] = c1_buttons; o[47] = c1_shift; o[48] = c1_count; o[49] = strobe; o[50] = c2_count;
        o[51] = fault; u32(52, pending_dma);
        std::memcpy(o + 56, apu_io, 24);
        std::memcpy(o + 80, ram, 2048);
        std::memcpy(o + 2128, prg_ram, 8192);
        std::memcpy(o + 10320, oam, 256);
        std::memcpy(o + 10576, palette, 32);
        std::memcpy(o + 10608, nt, 4096);
        std::memcpy(o + 14704, chr_ram, 8192);
    }
    void load(const std::uint8_t* s) {
        auto u16 = [&](std::size_t off) { return static_cast<std::uint16_t>(s[off] | (s[off + 1] << 8)); };
        auto u32 = [&](std::size_t off) { std::uint32_t r = 0; for (int i = 0; i < 4; ++i) r |= std::uint32_t(s[off + i]) << (8 * i); return r; };
        auto u64 = [&](std::size_t off) { std::uint64_t r = 0; for (int i = 0; i < 8; ++i) r |= std::uint64_t(s[off + i]) << (8 * i); return r; };
        pc = u16(4); a = s[6]; x = s[7]; y = s[8]; sp = s[9]; p = s[10]; nmi_pending = s[11];
        cycles = u64(12); frame = u64(20);
        const std::uint32_t fd = u32(28);
        scanline = static_cast<int>(fd / kDotsPerLine); dot = static_cast<int>(fd % kDotsPerLine);
        ctrl = s[32]; mask = s[33]; status = s[34]; oam_addr = s[35]; open_bus = s[36]; read_buffer = s[37];
        v = u16(38); t = u16(40); fine_x = s[42]; w = s[43]; scroll_x = s[44]; scroll_y = s[45];
        c1_buttons = s[46]; c1_shift = s[47]; c1_count = s[48]; strobe = s[49]; c2_count = s[50];
        fault = s[51]; pending_dma = u32(52);
        std::memcpy(apu_io, s + 56, 24);
        std::memcpy(ram, s + 80, 2048);
        std::memcpy(prg_ram, s + 2128, 8192);
        std::memcpy(oam, s + 10320, 256);
        std::memcpy(palette, s + 10576, 32);
        std::memcpy(nt, s + 10608, 4096);
        std::memcpy(chr_ram, s + 14704, 8192);
    }
};

// Reward/done rules (one per env-step, after the last frame).
//   kind 0: the reference's SMB rule, batch_step.cuh:41-106.
//   kind 1: x-delta rule: clip(int16(x - x_prev), -clip, clip) - time_penalty,
//           done when RAM[done_addr] == 0.
struct RewardSpec {
    std::uint32_t kind = 0;
    std::uint32_t x_lo = 0x86, x_hi = 0x6D, done_addr = 0x14, clip = 15;
    float time_penalty = 0.0f;
};

struct RewardState { std::int32_t prev_x = 0, prev_time = 0; };

int bcd3(const std::uint8_t* ram, unsigned at) {
    int r = 0;
    for (unsigned i = 0; i < 3; ++i) r = r * 10 + (ram[at + i] & 0x0F);
    return r;
}

void smb_track(const std::uint8_t* ram, int* x, int* time) {
    *x = ram[0x6D] * 256 + ram[0x86];
    *time = bcd3(ram, 0x7F8);
}

void reward_apply(const RewardSpec& spec, const std::uint8_t* ram, RewardState& st, float* reward, std::uint8_t* done) {
    if (spec.kind == 0) {
        int x, time;
        smb_track(ram, &x, &time);
        int dx = x - st.prev_x;
        if (dx < -5 || dx > 5) dx = 0;
        int dt = time - st.prev_time;
        if (dt > 0) dt = 0;
        const bool dying = ram[0x0E] == 0x0B || ram[0xB5] > 1;
        const bool dead = ram[0x0E] == 0x06;
        const bool over = ram[0x75A] == 0xFF;
        bool flag_get = ram[0x770] == 2;
        for (unsigned i = 0; i < 5; ++i) {
            const std::uint8_t e = ram[0x16 + i];
            if ((e == 0x2D || e == 0x31) && ram[0x1D] == 3) flag_get = true;
        }
        *reward = static_cast<float>(dx + dt + ((dying || dead) ? -25 : 0));
        *done = (flag_get || dying || dead || over) ? 1 : 0;
        st.prev_x = x;
        st.prev_time = time;
        return;
    }
    const int x = ram[spec.x_lo & 0x7FF] | (ram[spec.x_hi & 0x7FF] << 8);
    int dx = static_cast<std::int16_t>(static_cast<std::uint16_t>(x - st.prev_x));
    const int c = static_cast<int>(spec.clip);
    dx = std::max(-c, std::min(c, dx));
    *reward = static_cast<float>(dx) - spec.time_penalty;
    *done = ram[spec.done_addr & 0x7FF] == 0 ? 1 : 0;
    st.prev_x = x;
}

void reward_seed(const RewardSpec& spec, const std::uint8_t* ram, RewardState& st) {
    if (spec.kind == 0) {
        smb_track(ram, &st.prev_x, &st.prev_time);
    } else {
        st.prev_x = ram[spec.x_lo & 0x7FF] | (ram[spec.x_hi & 0x7FF] << 8);
        st.prev_time = 0;
    }
}

std::uint64_t fnv1a(const std::uint8_t* d, std::size_t n, std::uint64_t h = 0xCBF29CE484222325ull) {
    for (std::size_t i = 0; i < n; ++i) { h ^= d[i]; h *= 0x100000001B3ull; }
    return h;
}

std::uint64_t splitmix64(std::uint64_t x) {
    std::uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// ---- 84x84 grayscale --------------------------------------------------------
// The pixel observation of the vendored project's PixelPreprocess
// (project/mario-rl-ram/src/mario_rl/wrappers.py:209-215) applied to the
// batched core's RGB frame (batch_render.cuh palette):
//   gray = uint8(np.dot(float32 RGB, [0.299, 0.587, 0.114]))  -- numpy 2.2
//     (OpenBLAS dgemv) evaluates the length-3 dot as fma(b, .114, fma(g, .587,
//     r * .299)) in double; the cast truncates;
//   Image.fromarray(gray).resize((84, 84), Image.BILINEAR)  -- Pillow 12's
//     separable resample (libImaging/Resample.c): horizontal pass first into
//     an 8-bit image, then vertical; triangle filter of support 1 widened by
//     the scale, weights normalised and rounded to 22-bit fixed point, each
//     output = clip8((2^21 + sum in * w) >> 22).
constexpr std::uint8_t kNesRgb[192] = {
    0x54, 0x54, 0x54, 0x00, 0x1E, 0x74, 0x08, 0x10, 0x90, 0x30, 0x00, 0x88,
    0x44, 0x00, 0x64, 0x5C, 0x00, 0x30, 0x54, 0x04, 0x00, 0x3C, 0x18, 0x00,
    0x20, 0x2A, 0x00, 0x08, 0x3A, 0x00, 0x00, 0x40, 0x00, 0x00, 0x3C, 0x00,
    0x00, 0x32, 0x3C, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0x98, 0x96, 0x98, 0x08, 0x4C, 0xC4, 0x30, 0x32, 0xEC, 0x5C, 0x1E, 0xE4,
    0x88, 0x14, 0xB0, 0xA0, 0x14, 0x64, 0x98, 0x22, 0x20, 0x78, 0x3C, 0x00,
    0x54, 0x5A, 0x00, 0x28, 0x72, 0x00, 0x08, 0x7C, 0x00, 0x00, 0x76, 0x28,
    0x00, 0x66, 0x78, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0xEC, 0xEE, 0xEC, 0x4C, 0x9A, 0xEC, 0x78, 0x7C, 0xEC, 0xB0, 0x62, 0xEC,
    0xE4, 0x54, 0xEC, 0xEC, 0x58, 0xB4, 0xEC, 0x6A, 0x64, 0xD4, 0x88, 0x20,
    0xA0, 0xAA, 0x00, 0x74, 0xC4, 0x00, 0x4C, 0xD0, 0x20, 0x38, 0xCC, 0x6C,
    0x38, 0xB4, 0xCC, 0x3C, 0x3C, 0x3C, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0xEC, 0xEE, 0xEC, 0xA8, 0xCC, 0xEC, 0xBC, 0xBC, 0xEC, 0xD4, 0xB2, 0xEC,
    0xEC, 0xAE, 0xEC, 0xEC, 0xAE, 0xD4, 0xEC, 0xB4, 0xB0, 0xE4, 0xC4, 0x90,
    0xCC, 0xD2, 0x78, 0xB4, 0xDE, 0x78, 0xA8, 0xE2, 0x90, 0x98, 0xE2, 0xB4,
    0xA0, 0xD6, 0xE4, 0xA0, 0xA2, 0xA0, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
};

std::uint8_t gray_of(unsigned index) {
    const double r = kNesRgb[3 * index], g = kNesRgb[3 * index + 1], b = kNesRgb[3 * index + 2];
    return static_cast<std::uint8_t>(static_cast<int>(std::fma(b, 0.114, std::fma(g, 0.587, r * 0.299))));
}

struct Resample {
    int ksize = 0;
    std::vector<int> lo, n, k;   // per output: first input, input count, ksize weights
};

Resample pil_bilinear(int in_size, int out_size) {
    constexpr int kPrecision = 22;
    Resample rs;
    const double scale = static_cast<double>(in_size) / out_size;
    const double filterscale = scale < 1.0 ? 1.0 : scale;
    const double support = 1.0 * filterscale;
    rs.ksize = static_cast<int>(std::ceil(support)) * 2 + 1;
    rs.k.assign(static_cast<std::size_t>(out_size * rs.ksize), 0);
    for (int xx = 0; xx < out_size; ++xx) {
        const double center = (xx + 0.5) * scale;
        const double ss = 1.0 / filterscale;
        int xmin = static_cast<int>(center - support + 0.5);
        if (xmin < 0) xmin = 0;
        int xmax = static_cast<int>(center + support + 0.5);
        if (xmax > in_size) xmax = in_size;
        xmax -= xmin;
        std::vector<double> w(static_cast<std::size_t>(xmax));
        double ww = 0.0;
        for (int x = 0; x < xmax; ++x) {
            double t = (x + xmin - center + 0.5) * ss;
            if (t < 0.0) t = -t;
            w[x] = t < 1.0 ? 1.0 - t : 0.0;
            ww += w[x];
        }
        for (int x = 0; x < xmax; ++x) {
            if (ww != 0.0) w[x] /= ww;
            rs.k[xx * rs.ksize + x] = w[x] < 0 ? static_cast<int>(-0.5 + w[x] * (1 << kPrecision))
                                              : static_cast<int>(0.5 + w[x] * (1 << kPrecision));
        }
        rs.lo.push_back(xmin);
        rs.n.push_back(xmax);
    }
    return rs;
}

std::uint8_t clip8(std::int64_t v) {
    v >>= 22;
    return static_cast<std::uint8_t>(v < 0 ? 0 : (v > 255 ? 255 : v));
}

// 240x256 palette values -> 84x84 gray.
void gray84(const std::uint8_t* frame, std::uint8_t* out) {
    static const Resample h = pil_bilinear(256, 84), v = pil_bilinear(240, 84);
    std::vector<std::uint8_t> gray(240 * 256), mid(240 * 84);
    for (int i = 0; i < 240 * 256; ++i) gray[i] = gray_of(frame[i] & 0x3F);
    for (int y = 0; y < 240; ++y)
        for (int x = 0; x < 84; ++x) {
            std::int64_t acc = 1 << 21;
            for (int j = 0; j < h.n[x]; ++j) acc += static_cast<std::int64_t>(gray[y * 256 + h.lo[x] + j]) * h.k[x * h.ksize + j];
            mid[y * 84 + x] = clip8(acc);
        }
    for (int y = 0; y < 84; ++y)
        for (int x = 0; x < 84; ++x) {
            std::int64_t acc = 1 << 21;
            for (int j = 0; j < v.n[y]; ++j) acc += static_cast<std::int64_t>(mid[(v.lo[y] + j) * 84 + x]) * v.k[y * v.ksize + j];
            out[y * 84 + x] = clip8(acc);
        }
}

struct Env {
    Cart cart;
    Machine m;
    RewardSpec spec;
    RewardState rs;
};

thread_local std::string g_error;

}  // namespace

extern "C" {

const char* oracle_last_error() { return g_error.c_str(); }
std::size_t oracle_state_bytes() { return kStateBytes; }

void* oracle_create(const std::uint8_t* ines, std::size_t len) {
    try {
        auto* e = new Env();
        e->cart = parse_ines(ines, len);
        e->m.cart = &e->cart;
        e->m.power_on();
        return e;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return nullptr;
    }
}

void oracle_destroy(void* h) { delete static_cast<Env*>(h); }

void oracle_set_reward(void* h, std::uint32_t kind, std::uint32_t x_lo, std::uint32_t x_hi,
                       std::uint32_t done_addr, std::uint32_t clip, float time_penalty) {
    auto* e = static_cast<Env*>(h);
    e->spec = RewardSpec{kind, x_lo, x_hi, done_addr, clip, time_penalty};
    reward_seed(e->spec, e->m.ram, e->rs);
}

// One env-step: set the pad, run `frameskip` frames (console.hpp:137-150),
// then apply the reward rule.  Returns instructions executed, or -1 on fault.
std::int64_t oracle_step(void* h, std::uint8_t buttons, std::uint32_t frameskip,
                         std::uint64_t max_instructions, float* reward, std::uint8_t* done) {
    auto* e = static_cast<Env*>(h);
    try {
        e->m.set_buttons(buttons);
        std::uint64_t n = 0;
        for (std::uint32_t f = 0; f < frameskip; ++f) n += e->m.step_frame(max_instructions);
        float r = 0.0f;
        std::uint8_t d = 0;
        reward_apply(e->spec, e->m.ram, e->rs, &r, &d);
        if (reward) *reward = r;
        if (done) *done = d;
        return static_cast<std::int64_t>(n);
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

// One console instruction (console.hpp:108-135): NMI entry, the instruction,
// DMA stall, PPU dots.  Returns the CPU cycles it took (NMI and DMA included)
// and stores the frames it completed in *frames; -1 on an illegal opcode.
std::int64_t oracle_step_instruction(void* h, std::uint32_t* frames) {
    auto* e = static_cast<Env*>(h);
    try {
        const std::uint64_t before = e->m.cycles;
        const std::uint32_t f = e->m.step_instruction();
        if (frames) *frames = f;
        return static_cast<std::int64_t>(e->m.cycles - before);
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

// CPU bus accesses with their side effects (console.hpp:49-101): the
// known-answer tests drive registers, mirrors, DMA and the pads through these.
std::uint32_t oracle_bus_read(void* h, std::uint32_t addr) {
    return static_cast<Env*>(h)->m.read(static_cast<std::uint16_t>(addr));
}
void oracle_bus_write(void* h, std::uint32_t addr, std::uint32_t value) {
    static_cast<Env*>(h)->m.write(static_cast<std::uint16_t>(addr), static_cast<std::uint8_t>(value));
}

// PPU memory space read ($0000-$3FFF, ppu.hpp:280-338) without side effects.
std::uint32_t oracle_ppu_peek(void* h, std::uint32_t addr) {
    return static_cast<Env*>(h)->m.vram_read(static_cast<std::uint16_t>(addr));
}

// Advance the PPU alone by `dots` (ppu.hpp:46-76); returns frames completed.
std::uint32_t oracle_ppu_run(void* h, std::uint32_t dots) { return static_cast<Env*>(h)->m.ppu_run(dots); }

void oracle_save(void* h, std::uint8_t* out) { static_cast<Env*>(h)->m.save(out); }

// Restore a full-state blob; reward baselines are re-seeded from its RAM.
void oracle_load(void* h, const std::uint8_t* in) {
    auto* e = static_cast<Env*>(h);
    e->m.load(in);
    reward_seed(e->spec, e->m.ram, e->rs);
}

std::uint64_t oracle_fnv1a(const std::uint8_t* d, std::size_t n) { return fnv1a(d, n); }

// One frame of palette values (240 x 256).  mode bit 0: from the presentation
// snapshot (batched core); bit 1: the CPU core's renderer rules (live state).
void oracle_render(void* h, std::uint32_t mode, std::uint8_t* out) {
    static_cast<Env*>(h)->m.render(out, (mode & 1) != 0, (mode & 2) != 0);
}
// Re-seed the presentation snapshot from live state (a full reset does this).
void oracle_seed_presentation(void* h) { static_cast<Env*>(h)->m.seed_presentation(); }
// Overwrite the snapshot's scroll/ctrl/mask: start x, start y, start ctrl,
// end x, end y, end ctrl, mask (test hook for the HUD/play split).
void oracle_set_presentation(void* h, const std::uint8_t* f) {
    auto& p = static_cast<Env*>(h)->m.snap;
    p.sx_start = f[0]; p.sy_start = f[1]; p.ctrl_start = f[2];
    p.sx_end = f[3]; p.sy_end = f[4]; p.ctrl_end = f[5]; p.mask = f[6];
}
// The presentation state, laid out as the reference harness's
// ref_present_get: [0..6] frame-start x, y, ctrl, frame-end x, y, ctrl, mask;
// [7..9] the pre-render latch x, y, ctrl; [16..271] OAM; [272..303] palette;
// [304..2351] the first 2,048 bytes of nametable RAM.
void oracle_present_get(void* h, std::uint8_t* out) {
    const auto& m = static_cast<Env*>(h)->m;
    const auto& p = m.snap;
    const std::uint8_t head[10] = {p.sx_start, p.sy_start, p.ctrl_start, p.sx_end, p.sy_end,
                                   p.ctrl_end, p.mask, m.lat_sx, m.lat_sy, m.lat_ctrl};
    std::memset(out, 0, 16);
    std::memcpy(out, head, 10);
    std::memcpy(out + 16, p.oam, 256);
    std::memcpy(out + 272, p.palette, 32);
    std::memcpy(out + 304, p.nt, 2048);
}
void oracle_palette_rgb(std::uint8_t* out) { std::memcpy(out, kNesRgb, sizeof(kNesRgb)); }
void oracle_gray84(const std::uint8_t* frame, std::uint8_t* out) { gray84(frame, out); }
std::uint64_t oracle_splitmix64(std::uint64_t x) { return splitmix64(x); }

// CPU baseline: n_envs consoles, each on its own controller stream
// mask = splitmix64(seed ^ (env << 32) ^ step) & 0xFF, run for `steps` env-steps
// of `frameskip` frames on `threads` std::threads (envs statically partitioned).
// Returns wall seconds; *checksum = XOR of per-env FNV-1a RAM hashes, and
// *instructions = total instructions executed.
double oracle_run_batch(const std::uint8_t* ines, std::size_t len, std::uint32_t n_envs,
                        std::uint32_t steps, std::uint32_t frameskip, std::uint64_t seed,
                        std::uint32_t threads, std::uint64_t* checksum, std::uint64_t* instructions) {
    Cart cart;
    try {
        cart = parse_ines(ines, len);
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1.0;
    }
    threads = std::max(1u, std::min(threads, n_envs));
    std::atomic<std::uint64_t> sum{0}, instr{0};
    std::atomic<bool> failed{false};
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::thread> pool;
    for (std::uint32_t t = 0; t < threads; ++t) {
        pool.emplace_back([&, t]() {
            const std::uint32_t lo = static_cast<std::uint32_t>(std::uint64_t(n_envs) * t / threads);
            const std::uint32_t hi = static_cast<std::uint32_t>(std::uint64_t(n_envs) * (t + 1) / threads);
            std::uint64_t local = 0, li = 0;
            try {
                for (std::uint32_t env = lo; env < hi; ++env) {
                    Machine m;
                    m.cart = &cart;
                    m.power_on();
                    for (std::uint32_t k = 0; k < steps; ++k) {
                        m.set_buttons(static_cast<std::uint8_t>(splitmix64(seed ^ (std::uint64_t(env) << 32) ^ k) & 0xFF));
                        for (std::uint32_t f = 0; f < frameskip; ++f) li += m.step_frame(200000);
                    }
                    local ^= fnv1a(m.ram, 2048);
                }
            } catch (...) {
                failed = true;
            }
            sum ^= local;
            instr += li;
        });
    }
    for (auto& th : pool) th.join();
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (failed) {
        g_error = "illegal opcode during batch run";
        return -1.0;
    }
    if (checksum) *checksum = sum.load();
    if (instructions) *instructions = instr.load();
    return secs;
}

// The snapshot workload on the CPU: console `env` starts from blob
// levels[env] with RAM[done_addr] = done_init[env], takes the pad stream
// splitmix64(seed ^ env << 32 ^ (step0 + k)) & 0xFF, and is re-loaded from its
// blob after every env-step that leaves RAM[done_addr] == 0 (the auto-reset of
// the HIP batch).  Returns seconds; RAM checksum, instructions and resets out.
double oracle_run_levels(const std::uint8_t* ines, std::size_t len, const std::uint8_t* blobs, std::uint32_t n_levels,
                         const std::uint8_t* levels, const std::uint8_t* done_init, std::uint32_t done_addr,
                         std::uint32_t n_envs, std::uint32_t steps, std::uint32_t frameskip, std::uint64_t seed,
                         std::uint64_t step0, std::uint32_t threads, std::uint64_t* checksum,
                         std::uint64_t* instructions, std::uint64_t* resets) {
    Cart cart;
    try {
        cart = parse_ines(ines, len);
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1.0;
    }
    for (std::uint32_t e = 0; e < n_envs; ++e)
        if (levels[e] >= n_levels) {
            g_error = "level out of range";
            return -1.0;
        }
    threads = std::max(1u, std::min(threads, n_envs));
    done_addr &= 0x7FF;
    std::atomic<std::uint64_t> sum{0}, instr{0}, rs{0};
    std::atomic<bool> failed{false};
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::thread> pool;
    for (std::uint32_t t = 0; t < threads; ++t) {
        pool.emplace_back([&, t]() {
            const std::uint32_t lo = static_cast<std::uint32_t>(std::uint64_t(n_envs) * t / threads);
            const std::uint32_t hi = static_cast<std::uint32_t>(std::uint64_t(n_envs) * (t + 1) / threads);
            std::uint64_t local = 0, li = 0, lr = 0;
            try {
                for (std::uint32_t env = lo; env < hi; ++env) {
                    const std::uint8_t* b = blobs + static_cast<std::size_t>(levels[env]) * kStateBytes;
                    Machine m;
                    m.cart = &cart;
                    m.load(b);
                    m.ram[done_addr] = done_init[env];
                    for (std::uint32_t k = 0; k < steps; ++k) {
                        m.set_buttons(static_cast<std::uint8_t>(
                            splitmix64(seed ^ (std::uint64_t(env) << 32) ^ (step0 + k)) & 0xFF));
                        for (std::uint32_t f = 0; f < frameskip; ++f) li += m.step_frame(200000);
                        if (m.ram[done_addr] == 0) {
                            m.load(b);
                            ++lr;
                        }
                    }
                    local ^= fnv1a(m.ram, 2048);
                }
            } catch (...) {
                failed = true;
            }
            sum ^= local;
            instr += li;
            rs += lr;
        });
    }
    for (auto& th : pool) th.join();
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (failed) {
        g_error = "illegal opcode during batch run";
        return -1.0;
    }
    if (checksum) *checksum = sum.load();
    if (instructions) *instructions = instr.load();
    if (resets) *resets = rs.load();
    return secs;
}

}  // extern "C"
