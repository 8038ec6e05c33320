// nes_layout.h -- device state layout and 6502 microcode shared by the HIP
// kernels (nes_kernels.hip) and the host library (nes_host.hip).
//
// HBM layout.  Every per-console byte array is interleaved "address-major":
// element (addr, env) lives at base[addr * pitch + env], with pitch = num_envs
// rounded up to 256.  Lanes of a wave64 are consecutive envs, so when they
// touch the same NES address (same code path, same zero-page variable) the
// wave issues one 64-byte access instead of 64 scattered ones, and a 128-byte
// cache line holds one NES address for 128 consecutive consoles.  Per-env
// scalars are plain SoA arrays indexed by env.  The env-major RAM observation
// that callers see ([num_envs][2048], the reference's layout at
// cpp/bindings/cuda_module.cu:854-863) is produced by a transpose kernel.
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
    std::uint8_t* prg_ram;
    std::uint8_t* oam;
    std::uint8_t* palette;
    std::uint8_t* nametable;
    std::uint8_t* chr_ram;     // null when the cart has CHR ROM

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

    // Snapshot bank: num_levels canonical blobs, env_to_level[n].
    const std::uint8_t* bank;
    const std::uint8_t* env_to_level;
    std::uint32_t num_levels;
};

// ---------------------------------------------------------------------------
// 6502 microcode.
//
// One 64-bit word per opcode drives a single branch-free datapath: operand
// fetch, effective address, memory read, an 8-bit adder / logic unit /
// shifter, flag merge and register write-back.  Control-transfer and stack
// opcodes take a separate path.  Field layout:
//   0-3  addressing mode          4-6  base cycles        7  page-cross penalty
//   8-9  kind (alu/branch/ctrl/illegal)                  10-11 R input (A X Y SP)
//   12   primary input is M        13   reads memory       14  writes memory
//   15-16 unit (adder/logic/shift) 17-18 logic op (and/or/eor)
//   19   adder B from M            20   B ^= 0xFF          21  B constant 0xFF
//   22-23 carry in (0, 1, C)       24   shift right        25  rotate through C
//   26-28 destination (none A X Y SP)                    29  BIT flag rule
//   30-37 flag mask merged from the datapath (N V . . . . Z C)
//   38-45 P AND mask               46-53 P OR mask
//   54-57 control op               58-59 instruction length
// ---------------------------------------------------------------------------
namespace mc {

enum Mode : std::uint32_t { IMP = 0, ACC, IMM, ZP, ZPX, ZPY, ABS, ABSX, ABSY, INDX, INDY, IND, REL };
enum Kind : std::uint32_t { KALU = 0, KBRANCH = 1, KCTRL = 2, KILLEGAL = 3 };
enum Reg : std::uint32_t { RA = 0, RX = 1, RY = 2, RSP = 3 };
enum Unit : std::uint32_t { UADD = 0, ULOGIC = 1, USHIFT = 2 };
enum Logic : std::uint32_t { LAND = 0, LOR = 1, LEOR = 2 };
enum Cin : std::uint32_t { CZERO = 0, CONE = 1, CFLAG = 2 };
enum Dst : std::uint32_t { DNONE = 0, DA = 1, DX = 2, DY = 3, DSP = 4 };
enum Ctrl : std::uint32_t { JMPA = 0, JMPI, JSR, RTS, RTI, BRK, PHA, PHP, PLA, PLP };

constexpr std::uint32_t kFlagN = 0x80, kFlagV = 0x40, kFlagZ = 0x02, kFlagC = 0x01;

constexpr std::uint32_t mode_len(std::uint32_t m) {
    return (m == IMP || m == ACC) ? 1u : ((m == ABS || m == ABSX || m == ABSY || m == IND) ? 3u : 2u);
}

struct Word {
    std::uint64_t v = 0;
    constexpr Word& set(std::uint32_t lo, std::uint32_t bits, std::uint64_t val) {
        const std::uint64_t m = ((std::uint64_t{1} << bits) - 1) << lo;
        v = (v & ~m) | ((val << lo) & m);
        return *this;
    }
};

constexpr std::uint64_t base_word(std::uint32_t mode, std::uint32_t cycles, bool penalty, std::uint32_t kind) {
    Word w;
    w.set(0, 4, mode).set(4, 3, cycles).set(7, 1, penalty ? 1 : 0).set(8, 2, kind);
    w.set(38, 8, 0xFF).set(46, 8, 0).set(58, 2, mode_len(mode));
    return w.v;
}

// Field helpers over a word.
constexpr std::uint64_t with(std::uint64_t v, std::uint32_t lo, std::uint32_t bits, std::uint64_t val) {
    Word w{v};
    w.set(lo, bits, val);
    return w.v;
}

struct Table {
    std::uint64_t e[256];
};

// Loads: R <- M.
constexpr std::uint64_t load(std::uint32_t mode, std::uint32_t cyc, bool pen, std::uint32_t dst) {
    std::uint64_t v = base_word(mode, cyc, pen, KALU);
    v = with(v, 12, 1, 1);                   // primary input M
    v = with(v, 13, 1, mode == IMM ? 0 : 1); // immediate operand comes from the fetch
    v = with(v, 26, 3, dst);
    v = with(v, 30, 8, kFlagN | kFlagZ);
    return v;
}
// Stores: M <- R.
constexpr std::uint64_t store(std::uint32_t mode, std::uint32_t cyc, std::uint32_t reg) {
    std::uint64_t v = base_word(mode, cyc, false, KALU);
    v = with(v, 10, 2, reg);
    v = with(v, 14, 1, 1);
    return v;
}
// Register transfer / increment: dst <- R (+ const).
constexpr std::uint64_t regop(std::uint32_t reg, std::uint32_t dst, std::uint32_t b_ff, std::uint32_t cin, bool flags) {
    std::uint64_t v = base_word(IMP, 2, false, KALU);
    v = with(v, 10, 2, reg);
    v = with(v, 21, 1, b_ff);
    v = with(v, 22, 2, cin);
    v = with(v, 26, 3, dst);
    v = with(v, 30, 8, flags ? (kFlagN | kFlagZ) : 0);
    return v;
}
// Two-operand ALU ops against a register: ORA/AND/EOR/ADC/SBC/CMP/CPX/CPY/BIT.
constexpr std::uint64_t binop(std::uint32_t mode, std::uint32_t cyc, bool pen, std::uint32_t reg,
                              std::uint32_t unit, std::uint32_t logic, bool invert, std::uint32_t cin,
                              std::uint32_t dst, std::uint32_t flags, bool bit_rule) {
    std::uint64_t v = base_word(mode, cyc, pen, KALU);
    v = with(v, 10, 2, reg);
    v = with(v, 13, 1, mode == IMM ? 0 : 1);
    v = with(v, 15, 2, unit);
    v = with(v, 17, 2, logic);
    v = with(v, 19, 1, unit == UADD ? 1 : 0);
    v = with(v, 20, 1, invert ? 1 : 0);
    v = with(v, 22, 2, cin);
    v = with(v, 26, 3, dst);
    v = with(v, 29, 1, bit_rule ? 1 : 0);
    v = with(v, 30, 8, flags);
    return v;
}
// Shifts and INC/DEC on A (mode ACC) or memory (read-modify-write).
constexpr std::uint64_t rmw(std::uint32_t mode, std::uint32_t cyc, std::uint32_t unit, bool right, bool rot,
                            std::uint32_t b_ff, std::uint32_t cin) {
    std::uint64_t v = base_word(mode, cyc, false, KALU);
    const bool mem = mode != ACC;
    v = with(v, 10, 2, RA);
    v = with(v, 12, 1, mem ? 1 : 0);
    v = with(v, 13, 1, mem ? 1 : 0);
    v = with(v, 14, 1, mem ? 1 : 0);
    v = with(v, 15, 2, unit);
    v = with(v, 21, 1, b_ff);
    v = with(v, 22, 2, cin);
    v = with(v, 24, 1, right ? 1 : 0);
    v = with(v, 25, 1, rot ? 1 : 0);
    v = with(v, 26, 3, mem ? DNONE : DA);
    v = with(v, 30, 8, unit == USHIFT ? (kFlagN | kFlagZ | kFlagC) : (kFlagN | kFlagZ));
    return v;
}
constexpr std::uint64_t flagop(std::uint32_t and_mask, std::uint32_t or_mask) {
    std::uint64_t v = base_word(IMP, 2, false, KALU);
    v = with(v, 38, 8, and_mask);
    v = with(v, 46, 8, or_mask);
    return v;
}
constexpr std::uint64_t ctrl(std::uint32_t op, std::uint32_t mode, std::uint32_t cyc) {
    return with(base_word(mode, cyc, false, KCTRL), 54, 4, op);
}

// Opcode table: the official 151 opcodes with the cycle counts of the
// reference's decode table (cpp/include/nesle/cpu.hpp:190-353); the rest are
// illegal.
constexpr Table make_table() {
    Table t{};
    for (auto& e : t.e) e = base_word(IMP, 0, false, KILLEGAL);
    // Two-operand groups over the eight cc=01 addressing modes.
    struct G { std::uint32_t base; std::uint32_t reg, unit, logic; bool inv; std::uint32_t cin, dst, flags; bool store; };
    constexpr std::uint32_t NZ = kFlagN | kFlagZ, NZC = NZ | kFlagC, NZCV = NZC | kFlagV;
    const G groups[8] = {
        {0x00, RA, ULOGIC, LOR, false, CZERO, DA, NZ, false},    // ORA
        {0x20, RA, ULOGIC, LAND, false, CZERO, DA, NZ, false},   // AND
        {0x40, RA, ULOGIC, LEOR, false, CZERO, DA, NZ, false},   // EOR
        {0x60, RA, UADD, 0, false, CFLAG, DA, NZCV, false},      // ADC
        {0x80, RA, 0, 0, false, 0, 0, 0, true},                  // STA
        {0xA0, 0, 0, 0, false, 0, DA, NZ, false},                // LDA
        {0xC0, RA, UADD, 0, true, CONE, DNONE, NZC, false},      // CMP
        {0xE0, RA, UADD, 0, true, CFLAG, DA, NZCV, false},       // SBC
    };
    const std::uint32_t modes[8] = {INDX, ZP, IMM, ABS, INDY, ZPX, ABSY, ABSX};
    const std::uint32_t cycles[8] = {6, 3, 2, 4, 5, 4, 4, 4};
    const std::uint32_t store_cycles[8] = {6, 3, 0, 4, 6, 4, 5, 5};
    const bool penalty[8] = {false, false, false, false, true, false, true, true};
    for (const auto& g : groups) {
        for (std::uint32_t i = 0; i < 8; ++i) {
            const std::uint32_t op = g.base | (i << 2) | 1u;
            if (g.store) {
                if (modes[i] != IMM) t.e[op] = store(modes[i], store_cycles[i], RA);
            } else if (g.base == 0xA0) {
                t.e[op] = load(modes[i], cycles[i], penalty[i], DA);
            } else {
                t.e[op] = binop(modes[i], cycles[i], penalty[i], g.reg, g.unit, g.logic, g.inv, g.cin,
                                g.dst, g.flags, false);
            }
        }
    }
    // LDX / LDY / STX / STY.
    t.e[0xA2] = load(IMM, 2, false, DX); t.e[0xA6] = load(ZP, 3, false, DX);
    t.e[0xB6] = load(ZPY, 4, false, DX); t.e[0xAE] = load(ABS, 4, false, DX);
    t.e[0xBE] = load(ABSY, 4, true, DX);
    t.e[0xA0] = load(IMM, 2, false, DY); t.e[0xA4] = load(ZP, 3, false, DY);
    t.e[0xB4] = load(ZPX, 4, false, DY); t.e[0xAC] = load(ABS, 4, false, DY);
    t.e[0xBC] = load(ABSX, 4, true, DY);
    t.e[0x86] = store(ZP, 3, RX); t.e[0x96] = store(ZPY, 4, RX); t.e[0x8E] = store(ABS, 4, RX);
    t.e[0x84] = store(ZP, 3, RY); t.e[0x94] = store(ZPX, 4, RY); t.e[0x8C] = store(ABS, 4, RY);
    // CPX / CPY / BIT.
    t.e[0xE0] = binop(IMM, 2, false, RX, UADD, 0, true, CONE, DNONE, NZC, false);
    t.e[0xE4] = binop(ZP, 3, false, RX, UADD, 0, true, CONE, DNONE, NZC, false);
    t.e[0xEC] = binop(ABS, 4, false, RX, UADD, 0, true, CONE, DNONE, NZC, false);
    t.e[0xC0] = binop(IMM, 2, false, RY, UADD, 0, true, CONE, DNONE, NZC, false);
    t.e[0xC4] = binop(ZP, 3, false, RY, UADD, 0, true, CONE, DNONE, NZC, false);
    t.e[0xCC] = binop(ABS, 4, false, RY, UADD, 0, true, CONE, DNONE, NZC, false);
    t.e[0x24] = binop(ZP, 3, false, RA, ULOGIC, LAND, false, CZERO, DNONE, kFlagN | kFlagV | kFlagZ, true);
    t.e[0x2C] = binop(ABS, 4, false, RA, ULOGIC, LAND, false, CZERO, DNONE, kFlagN | kFlagV | kFlagZ, true);
    // Shifts: ASL ROL LSR ROR over acc/zp/abs/zp,X/abs,X.
    struct S { std::uint32_t base; bool right, rot; };
    const S shifts[4] = {{0x00, false, false}, {0x20, false, true}, {0x40, true, false}, {0x60, true, true}};
    for (const auto& s : shifts) {
        t.e[s.base | 0x0A] = rmw(ACC, 2, USHIFT, s.right, s.rot, 0, CZERO);
        t.e[s.base | 0x06] = rmw(ZP, 5, USHIFT, s.right, s.rot, 0, CZERO);
        t.e[s.base | 0x0E] = rmw(ABS, 6, USHIFT, s.right, s.rot, 0, CZERO);
        t.e[s.base | 0x16] = rmw(ZPX, 6, USHIFT, s.right, s.rot, 0, CZERO);
        t.e[s.base | 0x1E] = rmw(ABSX, 7, USHIFT, s.right, s.rot, 0, CZERO);
    }
    // INC / DEC memory.
    t.e[0xE6] = rmw(ZP, 5, UADD, false, false, 0, CONE);  t.e[0xF6] = rmw(ZPX, 6, UADD, false, false, 0, CONE);
    t.e[0xEE] = rmw(ABS, 6, UADD, false, false, 0, CONE); t.e[0xFE] = rmw(ABSX, 7, UADD, false, false, 0, CONE);
    t.e[0xC6] = rmw(ZP, 5, UADD, false, false, 1, CZERO);  t.e[0xD6] = rmw(ZPX, 6, UADD, false, false, 1, CZERO);
    t.e[0xCE] = rmw(ABS, 6, UADD, false, false, 1, CZERO); t.e[0xDE] = rmw(ABSX, 7, UADD, false, false, 1, CZERO);
    // Register transfers and increments.
    t.e[0xAA] = regop(RA, DX, 0, CZERO, true);   // TAX
    t.e[0xA8] = regop(RA, DY, 0, CZERO, true);   // TAY
    t.e[0x8A] = regop(RX, DA, 0, CZERO, true);   // TXA
    t.e[0x98] = regop(RY, DA, 0, CZERO, true);   // TYA
    t.e[0xBA] = regop(RSP, DX, 0, CZERO, true);  // TSX
    t.e[0x9A] = regop(RX, DSP, 0, CZERO, false); // TXS
    t.e[0xE8] = regop(RX, DX, 0, CONE, true);    // INX
    t.e[0xC8] = regop(RY, DY, 0, CONE, true);    // INY
    t.e[0xCA] = regop(RX, DX, 1, CZERO, true);   // DEX
    t.e[0x88] = regop(RY, DY, 1, CZERO, true);   // DEY
    t.e[0xEA] = base_word(IMP, 2, false, KALU);  // NOP
    // Flag set/clear.
    t.e[0x18] = flagop(0xFE, 0x00); t.e[0x38] = flagop(0xFF, 0x01);  // CLC SEC
    t.e[0x58] = flagop(0xFB, 0x00); t.e[0x78] = flagop(0xFF, 0x04);  // CLI SEI
    t.e[0xB8] = flagop(0xBF, 0x00);                                  // CLV
    t.e[0xD8] = flagop(0xF7, 0x00); t.e[0xF8] = flagop(0xFF, 0x08);  // CLD SED
    // Branches: opcode xxy10000 tests N, V, C, Z (bits 7-6), taken when equal
    // to y; the datapath derives the tested flag from the opcode itself.
    for (std::uint32_t i = 0; i < 8; ++i) t.e[(i << 5) | 0x10u] = base_word(REL, 2, false, KBRANCH);
    // Control transfer and stack.
    t.e[0x4C] = ctrl(JMPA, ABS, 3);
    t.e[0x6C] = ctrl(JMPI, IND, 5);
    t.e[0x20] = ctrl(JSR, ABS, 6);
    t.e[0x60] = ctrl(RTS, IMP, 6);
    t.e[0x40] = ctrl(RTI, IMP, 6);
    t.e[0x00] = ctrl(BRK, IMP, 7);
    t.e[0x48] = ctrl(PHA, IMP, 3);
    t.e[0x08] = ctrl(PHP, IMP, 3);
    t.e[0x68] = ctrl(PLA, IMP, 4);
    t.e[0x28] = ctrl(PLP, IMP, 4);
    return t;
}

inline constexpr Table kTable = make_table();

}  // namespace mc
}  // namespace nesle
