// nes_micro.h -- the 6502 microcode of the step kernel (nes_step.hip).
//
// One 128-bit word per opcode (four dwords d[0..3]) drives a single
// branch-free datapath: effective address, operand, an adder / logic unit /
// right shifter, flag merge, register write-back and next PC.  Stack and
// control-transfer opcodes set kind = CTRL and take the kernel's stack path.
//
// CPU registers live packed in one VGPR: A bits 0-7, X 8-15, Y 16-23, SP
// 24-31.  Register operands are read with a bitfield extract whose offset and
// width come straight from a microcode dword: the hardware uses only the low
// five bits of those operands, so fields placed at bit 0 of a dword cost no
// extraction.
//
// Field map:
//   d0  0-4  index-register offset in the packed registers (X 8, Y 16)
//       5    base is the zero-page pointer ((zp,X) / (zp),Y)
//       6    wrap the effective address to the zero page
//       7    +1 cycle when indexing crosses a page
//       8    reads the memory operand         9  writes the memory operand
//       10-11 kind (ALU, BRANCH, CTRL, ILLEGAL)
//       12-13 length in bytes               14-18 base cycles x 3 (PPU dots)
//       19-22 control op                    23   BIT flag rule
//       24-31 flags taken from the datapath (N V . . . . Z C)
//   d1  0-4  index width (8 when indexed, else 0)
//       5    adder input A is the operand M (else register R)
//       6    adder input B is taken from A (left shifts: A + A + c)
//       7    carry in 1                      8   carry in = C flag
//       9    unit: right shifter             10  rotate (shift in C)
//       16-23 mask on B                      24-31 xor on B
//   d2  0-4  register R offset (A 0, X 8, Y 16, SP 24); for branches the
//            bit position of the tested flag
//       8-15 mask of R & M (logic AND term); for branches the pattern XORed
//            into P before the test (the tested bit set when the branch is
//            taken on a clear flag)
//       16-23 mask of R ^ M (XOR term)       24-31 result mask of the adder
//   d3  0-4  branch test width (1 for branches, 0 otherwise)
//       5-9  destination offset in the packed registers
//       10-14 destination width (8, or 0 for none)
//       16-23 flags AND mask                 24-31 flags OR mask (| 0x20)
#pragma once

#include <cstdint>

namespace nesle {
namespace mc {

enum Kind : std::uint32_t { KALU = 0, KBRANCH = 1, KCTRL = 2, KILLEGAL = 3 };
enum Ctrl : std::uint32_t { JMPA = 0, JMPI, JSR, RTS, RTI, BRK, PHA, PHP, PLA, PLP };
enum Mode : std::uint32_t { IMP = 0, ACC, IMM, ZP, ZPX, ZPY, ABS, ABSX, ABSY, INDX, INDY, IND, REL };
enum Reg : std::uint32_t { RA = 0, RX = 1, RY = 2, RSP = 3, RNONE = 4 };

constexpr std::uint32_t kN = 0x80, kV = 0x40, kZ = 0x02, kC = 0x01;

struct Word {
    std::uint32_t d[4] = {0, 0, 0, 0};
    constexpr Word& set(int dw, int lo, int bits, std::uint32_t v) {
        const std::uint32_t m = (bits == 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u)) << lo;
        d[dw] = (d[dw] & ~m) | ((v << lo) & m);
        return *this;
    }
};

constexpr std::uint32_t mode_len(std::uint32_t m) {
    return (m == IMP || m == ACC) ? 1u : ((m == ABS || m == ABSX || m == ABSY || m == IND) ? 3u : 2u);
}

constexpr std::uint32_t reg_off(std::uint32_t r) { return r == RNONE ? 0u : 8u * r; }

// Common part: addressing mode, kind, length, cycles.
constexpr Word base(std::uint32_t mode, std::uint32_t cycles, bool penalty, std::uint32_t kind) {
    Word w;
    const bool idx_x = mode == ZPX || mode == ABSX;
    const bool idx_y = mode == ZPY || mode == ABSY || mode == INDY;
    w.set(0, 0, 5, idx_x ? 8u : (idx_y ? 16u : 0u));
    w.set(1, 0, 5, (idx_x || idx_y) ? 8u : 0u);
    w.set(0, 5, 1, (mode == INDX || mode == INDY) ? 1u : 0u);
    w.set(0, 6, 1, (mode == ZP || mode == ZPX || mode == ZPY) ? 1u : 0u);
    w.set(0, 7, 1, penalty ? 1u : 0u);
    w.set(0, 10, 2, kind);
    w.set(0, 12, 2, mode_len(mode));
    w.set(0, 14, 5, 3u * cycles);
    w.set(3, 16, 8, 0xFF);   // flags AND mask: keep
    w.set(3, 24, 8, 0x20);   // flags OR mask: the unused bit reads as 1
    return w;
}

// Adder configuration: r = (A + B + cin) & 0xFF.
constexpr Word adder(Word w, bool a_is_m, std::uint32_t reg, bool b_from_a, std::uint32_t b_mask, std::uint32_t b_xor,
                     bool cin_1, bool cin_c) {
    w.set(1, 5, 1, a_is_m ? 1u : 0u);
    w.set(2, 0, 5, reg_off(reg));
    w.set(1, 6, 1, b_from_a ? 1u : 0u);
    w.set(1, 16, 8, b_mask);
    w.set(1, 24, 8, b_xor);
    w.set(1, 7, 1, cin_1 ? 1u : 0u);
    w.set(1, 8, 1, cin_c ? 1u : 0u);
    w.set(2, 24, 8, 0xFF);
    return w;
}

constexpr Word dest(Word w, std::uint32_t reg, std::uint32_t flags) {
    if (reg != RNONE) {
        w.set(3, 5, 5, reg_off(reg));
        w.set(3, 10, 5, 8);
    }
    w.set(0, 24, 8, flags);
    return w;
}

constexpr Word memops(Word w, bool rd, bool wr) {
    w.set(0, 8, 1, rd ? 1u : 0u);
    w.set(0, 9, 1, wr ? 1u : 0u);
    return w;
}

// R <- M (LDA/LDX/LDY).
constexpr Word load(std::uint32_t mode, std::uint32_t cyc, bool pen, std::uint32_t dst) {
    Word w = base(mode, cyc, pen, KALU);
    w = memops(w, mode != IMM, false);
    w = adder(w, true, RNONE, false, 0, 0, false, false);
    return dest(w, dst, kN | kZ);
}

// M <- R (STA/STX/STY).
constexpr Word store(std::uint32_t mode, std::uint32_t cyc, std::uint32_t reg) {
    Word w = base(mode, cyc, false, KALU);
    w = memops(w, false, true);
    return adder(w, false, reg, false, 0, 0, false, false);
}

// Register transfers, increments and decrements: dst <- R + B + cin.
constexpr Word regop(std::uint32_t reg, std::uint32_t dst, std::uint32_t b_xor, bool cin_1, bool flags) {
    Word w = base(IMP, 2, false, KALU);
    w = adder(w, false, reg, false, 0, b_xor, cin_1, false);
    return dest(w, dst, flags ? (kN | kZ) : 0u);
}

// ADC / SBC / CMP / CPX / CPY.
constexpr Word arith(std::uint32_t mode, std::uint32_t cyc, bool pen, std::uint32_t reg, bool subtract, bool compare) {
    Word w = base(mode, cyc, pen, KALU);
    w = memops(w, mode != IMM, false);
    w = adder(w, false, reg, false, 0xFF, subtract ? 0xFFu : 0u, compare, !compare);
    return dest(w, compare ? RNONE : RA, compare ? (kN | kZ | kC) : (kN | kZ | kC | kV));
}

// ORA / AND / EOR / BIT: r = (R & M & and_mask) | ((R ^ M) & xor_mask).
constexpr Word logic(std::uint32_t mode, std::uint32_t cyc, bool pen, std::uint32_t and_mask, std::uint32_t xor_mask,
                     bool bit_rule) {
    Word w = base(mode, cyc, pen, KALU);
    w = memops(w, mode != IMM, false);
    w.set(2, 0, 5, 0);        // R = A
    w.set(2, 8, 8, and_mask);
    w.set(2, 16, 8, xor_mask);
    w.set(0, 23, 1, bit_rule ? 1u : 0u);
    return dest(w, bit_rule ? RNONE : RA, bit_rule ? (kN | kV | kZ) : (kN | kZ));
}

// ASL / ROL (adder: A + A + c), LSR / ROR (right shifter), on A or memory.
constexpr Word shift(std::uint32_t mode, std::uint32_t cyc, bool right, bool rot) {
    Word w = base(mode, cyc, false, KALU);
    const bool mem = mode != ACC;
    w = memops(w, mem, mem);
    if (right) {
        w.set(1, 5, 1, mem ? 1u : 0u);
        w.set(2, 0, 5, 0);
        w.set(1, 9, 1, 1);
        w.set(1, 10, 1, rot ? 1u : 0u);
    } else {
        w = adder(w, mem, RA, true, 0xFF, 0, false, rot);
    }
    return dest(w, mem ? RNONE : RA, kN | kZ | kC);
}

// INC / DEC memory: M + 0 + 1 or M + 0xFF + 0.
constexpr Word incdec(std::uint32_t mode, std::uint32_t cyc, bool dec) {
    Word w = base(mode, cyc, false, KALU);
    w = memops(w, true, true);
    w = adder(w, true, RNONE, false, 0, dec ? 0xFFu : 0u, !dec, false);
    return dest(w, RNONE, kN | kZ);
}

constexpr Word flagop(std::uint32_t and_mask, std::uint32_t or_mask) {
    Word w = base(IMP, 2, false, KALU);
    w.set(3, 16, 8, and_mask);
    w.set(3, 24, 8, or_mask | 0x20u);
    return w;
}

constexpr Word branch(std::uint32_t op) {
    Word w = base(REL, 2, false, KBRANCH);
    // Opcode xxy10000 tests N, V, C, Z (bits 7-6) and is taken when the flag
    // equals y: XOR the flag with !y, then the tested bit is 1 when taken.
    constexpr std::uint32_t pos[4] = {7, 6, 0, 1};
    const std::uint32_t fp = pos[op >> 6];
    const bool want = (op >> 5) & 1u;
    w.set(2, 0, 5, fp);
    w.set(3, 0, 5, 1);
    w.set(2, 8, 8, want ? 0u : (1u << fp));
    return w;
}

constexpr Word ctrl(std::uint32_t op, std::uint32_t mode, std::uint32_t cyc) {
    Word w = base(mode, cyc, false, KCTRL);
    w.set(0, 19, 4, op);
    return w;
}

struct Table {
    Word e[256];
};

// The official 151 opcodes with the reference's cycle counts
// (cpp/include/nesle/cpu.hpp:190-353); the rest are illegal.
constexpr Table make_table() {
    Table t{};
    for (auto& e : t.e) e = base(IMP, 0, false, KILLEGAL);
    // cc=01 group over its eight addressing modes.
    const std::uint32_t modes[8] = {INDX, ZP, IMM, ABS, INDY, ZPX, ABSY, ABSX};
    const std::uint32_t cyc[8] = {6, 3, 2, 4, 5, 4, 4, 4};
    const std::uint32_t st_cyc[8] = {6, 3, 0, 4, 6, 4, 5, 5};
    const bool pen[8] = {false, false, false, false, true, false, true, true};
    for (std::uint32_t i = 0; i < 8; ++i) {
        const std::uint32_t m = modes[i];
        t.e[0x01 | (i << 2)] = logic(m, cyc[i], pen[i], 0xFF, 0xFF, false);  // ORA
        t.e[0x21 | (i << 2)] = logic(m, cyc[i], pen[i], 0xFF, 0x00, false);  // AND
        t.e[0x41 | (i << 2)] = logic(m, cyc[i], pen[i], 0x00, 0xFF, false);  // EOR
        t.e[0x61 | (i << 2)] = arith(m, cyc[i], pen[i], RA, false, false);   // ADC
        if (m != IMM) t.e[0x81 | (i << 2)] = store(m, st_cyc[i], RA);        // STA
        t.e[0xA1 | (i << 2)] = load(m, cyc[i], pen[i], RA);                  // LDA
        t.e[0xC1 | (i << 2)] = arith(m, cyc[i], pen[i], RA, true, true);     // CMP
        t.e[0xE1 | (i << 2)] = arith(m, cyc[i], pen[i], RA, true, false);    // SBC
    }
    t.e[0xA2] = load(IMM, 2, false, RX); t.e[0xA6] = load(ZP, 3, false, RX);
    t.e[0xB6] = load(ZPY, 4, false, RX); t.e[0xAE] = load(ABS, 4, false, RX);
    t.e[0xBE] = load(ABSY, 4, true, RX);
    t.e[0xA0] = load(IMM, 2, false, RY); t.e[0xA4] = load(ZP, 3, false, RY);
    t.e[0xB4] = load(ZPX, 4, false, RY); t.e[0xAC] = load(ABS, 4, false, RY);
    t.e[0xBC] = load(ABSX, 4, true, RY);
    t.e[0x86] = store(ZP, 3, RX); t.e[0x96] = store(ZPY, 4, RX); t.e[0x8E] = store(ABS, 4, RX);
    t.e[0x84] = store(ZP, 3, RY); t.e[0x94] = store(ZPX, 4, RY); t.e[0x8C] = store(ABS, 4, RY);
    t.e[0xE0] = arith(IMM, 2, false, RX, true, true); t.e[0xE4] = arith(ZP, 3, false, RX, true, true);
    t.e[0xEC] = arith(ABS, 4, false, RX, true, true);
    t.e[0xC0] = arith(IMM, 2, false, RY, true, true); t.e[0xC4] = arith(ZP, 3, false, RY, true, true);
    t.e[0xCC] = arith(ABS, 4, false, RY, true, true);
    t.e[0x24] = logic(ZP, 3, false, 0xFF, 0x00, true);
    t.e[0x2C] = logic(ABS, 4, false, 0xFF, 0x00, true);
    const struct { std::uint32_t base; bool right, rot; } sh[4] = {
        {0x00, false, false}, {0x20, false, true}, {0x40, true, false}, {0x60, true, true}};
    for (const auto& s : sh) {
        t.e[s.base | 0x0A] = shift(ACC, 2, s.right, s.rot);
        t.e[s.base | 0x06] = shift(ZP, 5, s.right, s.rot);
        t.e[s.base | 0x0E] = shift(ABS, 6, s.right, s.rot);
        t.e[s.base | 0x16] = shift(ZPX, 6, s.right, s.rot);
        t.e[s.base | 0x1E] = shift(ABSX, 7, s.right, s.rot);
    }
    t.e[0xE6] = incdec(ZP, 5, false); t.e[0xF6] = incdec(ZPX, 6, false);
    t.e[0xEE] = incdec(ABS, 6, false); t.e[0xFE] = incdec(ABSX, 7, false);
    t.e[0xC6] = incdec(ZP, 5, true); t.e[0xD6] = incdec(ZPX, 6, true);
    t.e[0xCE] = incdec(ABS, 6, true); t.e[0xDE] = incdec(ABSX, 7, true);
    t.e[0xAA] = regop(RA, RX, 0, false, true);    // TAX
    t.e[0xA8] = regop(RA, RY, 0, false, true);    // TAY
    t.e[0x8A] = regop(RX, RA, 0, false, true);    // TXA
    t.e[0x98] = regop(RY, RA, 0, false, true);    // TYA
    t.e[0xBA] = regop(RSP, RX, 0, false, true);   // TSX
    t.e[0x9A] = regop(RX, RSP, 0, false, false);  // TXS
    t.e[0xE8] = regop(RX, RX, 0, true, true);     // INX
    t.e[0xC8] = regop(RY, RY, 0, true, true);     // INY
    t.e[0xCA] = regop(RX, RX, 0xFF, false, true); // DEX
    t.e[0x88] = regop(RY, RY, 0xFF, false, true); // DEY
    t.e[0xEA] = base(IMP, 2, false, KALU);        // NOP
    t.e[0x18] = flagop(0xFE, 0x00); t.e[0x38] = flagop(0xFF, 0x01);  // CLC SEC
    t.e[0x58] = flagop(0xFB, 0x00); t.e[0x78] = flagop(0xFF, 0x04);  // CLI SEI
    t.e[0xB8] = flagop(0xBF, 0x00);                                  // CLV
    t.e[0xD8] = flagop(0xF7, 0x00); t.e[0xF8] = flagop(0xFF, 0x08);  // CLD SED
    for (std::uint32_t i = 0; i < 8; ++i) t.e[(i << 5) | 0x10u] = branch((i << 5) | 0x10u);
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
