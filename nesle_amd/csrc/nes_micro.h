// nes_micro.h -- the 6502 microcode of the step kernel (nes_step.hip).
//
// One 80-byte word (twenty dwords d[0..19]) per opcode drives a single
// branch-free datapath: effective address, operand, an adder / logic unit /
// right shifter, flag merge, register write-back, a three-byte stack window
// (pushes, pulls, stack-pointer change) and the next-PC selection.  Besides
// the 256 opcodes there are two virtual entries: kNopEntry (a lane that has
// finished its frames: changes nothing) and kNmiEntry (NMI entry: pushes PC
// and P like BRK and is counted as no instruction).
//
// CPU registers live packed in one VGPR: A bits 0-7, X 8-15, Y 16-23, SP
// 24-31.  Register operands are read with a bitfield extract whose offset and
// width come straight from a microcode dword: the hardware uses only the low
// five bits of those operands, so fields placed at bit 0 of a dword cost no
// extraction.  Masks that select between 8- or 16-bit values only need their
// low bits; whole-dword fields (push mask, perm selector, SP delta, register
// mask) are used as they are.
//
// Field map:
//   d0  0-4  index-register offset in the packed registers (X 8, Y 16)
//       5    base is the zero-page pointer ((zp,X) / (zp),Y)
//       6    wrap the effective address to the zero page
//       7    +1 cycle when indexing crosses a page
//       8    reads the memory operand         9  writes the memory operand
//       12-13 length in bytes               14-18 base CPU cycles
//       23   BIT flag rule                  24-31 flags taken from the datapath
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
//       16-23 flags AND mask                 24-31 flags OR mask (| 0x20)
//   d4  push mask over the window bytes in memory order (byte 0 = $0100+SP-2,
//       byte 1 = SP-1, byte 2 = SP)
//   d5  v_perm selector building the pushed bytes from
//       {src0 = (registers << 8) | pushed P, src1 = return address}
//   d6  stack-pointer change << 24
//   d7  interrupt vector (BRK, NMI; filled in from the PRG image at launch)
//   d8  destination register mask in the packed registers
//   d9  next PC := absolute operand (JMP, JSR)            0xFFFF or 0
//   d10 next PC := pulled return address (RTS, RTI)       0xFFFF or 0
//   d11 next PC := vector (BRK, NMI)                      0xFFFF or 0
//   d12 0-4 shift of the pulled bytes (RTI 8), 16 +1 (RTS), 24-25 return
//       address offset from the opcode (JSR, BRK 2)
//   d13 0-7 operand := first pulled byte (PLA, PLP, RTI)
//       8-15 lowest SP the window serves, 16-23 SP range above it: outside
//       it the stack bytes leave the LDS window and the opcode takes the
//       kernel's stack side path
//   d14 0 counts as an instruction, 1 clears the pending NMI,
//       2 JMP absolute (idle-loop check), 3 JMP indirect (side path),
//       4 illegal opcode
//   d15 0-7 P := pulled byte (PLP, RTI), 8-15 B/U bits of a pushed P
//   d16 0-15 base is the zero-page pointer (0xFFFF or 0); 16-23 base CPU
//       cycles
//   d17 effective-address mask (0xFF zero page, 0xFFFF otherwise)
//   d18 0-7 adder input A is the operand M (0xFF or 0); 8 carry in = C flag;
//       16 carry in 1
//   d19 0-7 unit: right shifter (0xFF or 0)
#pragma once

#include <cstdint>

namespace nesle {
namespace mc {

constexpr std::uint32_t kDwords = 20;
constexpr std::uint32_t kNopEntry = 256, kNmiEntry = 257, kEntries = 258;
// d14 bits.
constexpr std::uint32_t kCount = 1, kClearNmi = 2, kJmpAbs = 4, kJmpInd = 8, kIllegal = 16;

enum Mode : std::uint32_t { IMP = 0, ACC, IMM, ZP, ZPX, ZPY, ABS, ABSX, ABSY, INDX, INDY, IND, REL };
enum Reg : std::uint32_t { RA = 0, RX = 1, RY = 2, RSP = 3, RNONE = 4 };

constexpr std::uint32_t kN = 0x80, kV = 0x40, kZ = 0x02, kC = 0x01;

struct Word {
    std::uint32_t d[kDwords] = {};
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

// Stack window range: the opcode's pushed and pulled bytes stay inside the
// console's LDS copy of the stack page ($0100-$01FF when all RAM is in LDS,
// $0180-$01FF otherwise) without wrapping.
constexpr Word window(Word w, std::uint32_t npush, std::uint32_t npull, bool full) {
    const std::uint32_t lo = full ? (npush ? npush - 1u : 0u) : 0x82u;
    const std::uint32_t hi = 0xFFu - npull;
    w.set(13, 8, 8, lo);
    w.set(13, 16, 8, hi - lo);
    return w;
}

constexpr Word make_nop() {
    Word w;
    w.set(3, 16, 8, 0xFF);   // flags AND mask: keep
    w.set(3, 24, 8, 0x20);   // flags OR mask: the unused bit reads as 1
    w.set(13, 16, 8, 0xFF);  // any SP is served
    return w;
}

// Common part: addressing mode, length, cycles; no stack use.
constexpr Word base(std::uint32_t mode, std::uint32_t cycles, bool penalty) {
    Word w = make_nop();
    const bool idx_x = mode == ZPX || mode == ABSX;
    const bool idx_y = mode == ZPY || mode == ABSY || mode == INDY;
    w.set(0, 0, 5, idx_x ? 8u : (idx_y ? 16u : 0u));
    w.set(1, 0, 5, (idx_x || idx_y) ? 8u : 0u);
    w.set(0, 5, 1, (mode == INDX || mode == INDY) ? 1u : 0u);
    w.set(0, 6, 1, (mode == ZP || mode == ZPX || mode == ZPY) ? 1u : 0u);
    w.set(0, 7, 1, penalty ? 1u : 0u);
    w.set(0, 12, 2, mode_len(mode));
    w.set(0, 14, 5, cycles);
    w.set(14, 0, 5, kCount);
    w.set(16, 0, 16, (mode == INDX || mode == INDY) ? 0xFFFFu : 0u);
    w.set(16, 16, 8, cycles);
    w.set(17, 0, 32, (mode == ZP || mode == ZPX || mode == ZPY) ? 0xFFu : 0xFFFFu);
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
    w.set(18, 0, 8, a_is_m ? 0xFFu : 0u);
    w.set(18, 8, 1, cin_c ? 1u : 0u);
    w.set(18, 16, 1, cin_1 ? 1u : 0u);
    return w;
}

constexpr Word dest(Word w, std::uint32_t reg, std::uint32_t flags) {
    if (reg != RNONE) {
        w.set(3, 5, 5, reg_off(reg));
        w.set(8, 0, 32, 0xFFu << reg_off(reg));
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
    Word w = base(mode, cyc, pen);
    w = memops(w, mode != IMM, false);
    w = adder(w, true, RNONE, false, 0, 0, false, false);
    return dest(w, dst, kN | kZ);
}

// M <- R (STA/STX/STY).
constexpr Word store(std::uint32_t mode, std::uint32_t cyc, std::uint32_t reg) {
    Word w = base(mode, cyc, false);
    w = memops(w, false, true);
    return adder(w, false, reg, false, 0, 0, false, false);
}

// Register transfers, increments and decrements: dst <- R + B + cin.
constexpr Word regop(std::uint32_t reg, std::uint32_t dst, std::uint32_t b_xor, bool cin_1, bool flags) {
    Word w = base(IMP, 2, false);
    w = adder(w, false, reg, false, 0, b_xor, cin_1, false);
    return dest(w, dst, flags ? (kN | kZ) : 0u);
}

// ADC / SBC / CMP / CPX / CPY.
constexpr Word arith(std::uint32_t mode, std::uint32_t cyc, bool pen, std::uint32_t reg, bool subtract, bool compare) {
    Word w = base(mode, cyc, pen);
    w = memops(w, mode != IMM, false);
    w = adder(w, false, reg, false, 0xFF, subtract ? 0xFFu : 0u, compare, !compare);
    return dest(w, compare ? RNONE : RA, compare ? (kN | kZ | kC) : (kN | kZ | kC | kV));
}

// ORA / AND / EOR / BIT: r = (R & M & and_mask) | ((R ^ M) & xor_mask).
constexpr Word logic(std::uint32_t mode, std::uint32_t cyc, bool pen, std::uint32_t and_mask, std::uint32_t xor_mask,
                     bool bit_rule) {
    Word w = base(mode, cyc, pen);
    w = memops(w, mode != IMM, false);
    w.set(2, 0, 5, 0);        // R = A
    w.set(2, 8, 8, and_mask);
    w.set(2, 16, 8, xor_mask);
    w.set(0, 23, 1, bit_rule ? 1u : 0u);
    return dest(w, bit_rule ? RNONE : RA, bit_rule ? (kN | kV | kZ) : (kN | kZ));
}

// ASL / ROL (adder: A + A + c), LSR / ROR (right shifter), on A or memory.
constexpr Word shift(std::uint32_t mode, std::uint32_t cyc, bool right, bool rot) {
    Word w = base(mode, cyc, false);
    const bool mem = mode != ACC;
    w = memops(w, mem, mem);
    if (right) {
        w.set(1, 5, 1, mem ? 1u : 0u);
        w.set(2, 0, 5, 0);
        w.set(1, 9, 1, 1);
        w.set(1, 10, 1, rot ? 1u : 0u);
        w.set(18, 0, 8, mem ? 0xFFu : 0u);
        w.set(19, 0, 8, 0xFF);
    } else {
        w = adder(w, mem, RA, true, 0xFF, 0, false, rot);
    }
    return dest(w, mem ? RNONE : RA, kN | kZ | kC);
}

// INC / DEC memory: M + 0 + 1 or M + 0xFF + 0.
constexpr Word incdec(std::uint32_t mode, std::uint32_t cyc, bool dec) {
    Word w = base(mode, cyc, false);
    w = memops(w, true, true);
    w = adder(w, true, RNONE, false, 0, dec ? 0xFFu : 0u, !dec, false);
    return dest(w, RNONE, kN | kZ);
}

constexpr Word flagop(std::uint32_t and_mask, std::uint32_t or_mask) {
    Word w = base(IMP, 2, false);
    w.set(3, 16, 8, and_mask);
    w.set(3, 24, 8, or_mask | 0x20u);
    return w;
}

constexpr Word branch(std::uint32_t op) {
    Word w = base(REL, 2, false);
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

// Stack and control transfer (cpu.hpp:394-402,603-606,666-694 and the NMI
// entry cpu.hpp:112-123).  Pushes go to SP, SP-1, SP-2; pulls come from
// SP+1, SP+2, SP+3.
constexpr std::uint32_t kPermZero = 0x0C;  // v_perm selector byte for 0x00
constexpr std::uint32_t perm_sel(std::uint32_t b0, std::uint32_t b1, std::uint32_t b2) {
    return b0 | (b1 << 8) | (b2 << 16) | (kPermZero << 24);
}
// Selector bytes: 0 return address low, 1 return address high, 4 pushed P, 5 A.
constexpr Word pushes(Word w, std::uint32_t n, std::uint32_t sel, std::uint32_t ret_off, std::uint32_t bflags,
                      bool full) {
    w.set(4, 0, 32, n == 1 ? 0x00FF0000u : (n == 2 ? 0x00FFFF00u : 0x00FFFFFFu));
    w.set(5, 0, 32, sel);
    w.set(6, 0, 32, static_cast<std::uint32_t>(-static_cast<std::int32_t>(n)) << 24);
    w.set(12, 24, 2, ret_off);
    w.set(15, 8, 8, bflags);
    return window(w, n, 0, full);
}
constexpr Word pulls(Word w, std::uint32_t n, bool full) {
    w.set(6, 0, 32, n << 24);
    w.set(13, 0, 8, 0xFF);   // operand := first pulled byte
    return window(w, 0, n, full);
}

struct Table {
    Word e[kEntries];
};

// The official 151 opcodes with the reference's cycle counts
// (cpp/include/nesle/cpu.hpp:190-353); the rest are illegal.  `full`: all of
// the console's RAM is in LDS (selects the stack window range).
constexpr Table make_table(bool full) {
    Table t{};
    for (auto& e : t.e) e = make_nop().set(14, 0, 5, kIllegal);
    t.e[kNopEntry] = make_nop();
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
    t.e[0xEA] = base(IMP, 2, false);              // NOP
    t.e[0x18] = flagop(0xFE, 0x00); t.e[0x38] = flagop(0xFF, 0x01);  // CLC SEC
    t.e[0x58] = flagop(0xFB, 0x00); t.e[0x78] = flagop(0xFF, 0x04);  // CLI SEI
    t.e[0xB8] = flagop(0xBF, 0x00);                                  // CLV
    t.e[0xD8] = flagop(0xF7, 0x00); t.e[0xF8] = flagop(0xFF, 0x08);  // CLD SED
    for (std::uint32_t i = 0; i < 8; ++i) t.e[(i << 5) | 0x10u] = branch((i << 5) | 0x10u);

    // JMP abs: next PC = operand (and the idle-loop check).
    t.e[0x4C] = base(ABS, 3, false).set(9, 0, 32, 0xFFFF).set(14, 0, 5, kCount | kJmpAbs);
    // JMP (ind): the kernel's side path reads the pointer with the page-wrap bug.
    t.e[0x6C] = base(IND, 5, false).set(14, 0, 5, kCount | kJmpInd);
    // JSR: push PC+2 (high at SP, low at SP-1), next PC = operand.
    t.e[0x20] = pushes(base(ABS, 6, false), 2, perm_sel(kPermZero, 0, 1), 2, 0, full).set(9, 0, 32, 0xFFFF);
    // RTS: pull low, high; next PC = pulled + 1.
    t.e[0x60] = pulls(base(IMP, 6, false), 2, full).set(10, 0, 32, 0xFFFF).set(12, 16, 1, 1).set(13, 0, 8, 0);
    // RTI: pull P, low, high.
    t.e[0x40] = pulls(base(IMP, 6, false), 3, full).set(10, 0, 32, 0xFFFF).set(12, 0, 5, 8).set(15, 0, 8, 0xFF);
    // BRK: push PC+2 and P|B|U, set I, next PC = IRQ/BRK vector.
    t.e[0x00] = pushes(base(IMP, 7, false), 3, perm_sel(4, 0, 1), 2, 0x30, full).set(11, 0, 32, 0xFFFF)
                    .set(3, 24, 8, 0x24);
    // PHA, PHP (P|B|U).
    t.e[0x48] = pushes(base(IMP, 3, false), 1, perm_sel(kPermZero, kPermZero, 5), 0, 0, full);
    t.e[0x08] = pushes(base(IMP, 3, false), 1, perm_sel(kPermZero, kPermZero, 4), 0, 0x30, full);
    // PLA: A = pulled byte, N and Z.
    {
        Word w = pulls(base(IMP, 4, false), 1, full);
        w = adder(w, true, RNONE, false, 0, 0, false, false);
        t.e[0x68] = dest(w, RA, kN | kZ);
    }
    // PLP: P = pulled byte (B clear, U set).
    t.e[0x28] = pulls(base(IMP, 4, false), 1, full).set(15, 0, 8, 0xFF);
    // NMI entry: push PC and P with B clear, set I, next PC = NMI vector; not
    // an instruction of its own (console.hpp:108-135).
    t.e[kNmiEntry] = pushes(base(IMP, 7, false), 3, perm_sel(4, 0, 1), 0, 0x20, full).set(11, 0, 32, 0xFFFF)
                         .set(3, 24, 8, 0x24).set(0, 12, 2, 0).set(14, 0, 5, kClearNmi);
    return t;
}

inline constexpr Table kTableSplit = make_table(false);
inline constexpr Table kTableFull = make_table(true);

}  // namespace mc
}  // namespace nesle
