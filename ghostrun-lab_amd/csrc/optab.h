// Host-side construction of the 6502 opcode descriptors the device interpreter reads (nes_dev.h): the 151 official
// opcodes, derived from the 6502's operation classes and addressing modes; every other byte is a fault.
#pragma once
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <stdint.h>
#endif

#include "nes_dev.h"

namespace nd {

enum Mn { ORA, AND, EOR, ADC, STA, LDA, CMP, SBC, ASL, ROL, LSR, ROR, STX, LDX, DEC, INC, BIT, STY, LDY, CPY, CPX,
          BPL, BMI, BVC, BVS, BCC, BCS, BNE, BEQ, CLC, SEC, CLI, SEI, CLV, CLD, SED, TAX, TAY, TXA, TYA, TSX, TXS,
          INX, INY, DEX, DEY, NOP, PHA, PHP, PLA, PLP, JMP, JSR, RTS, RTI, BRK };

constexpr uint32_t rw_cycles(bool store, uint32_t mode) {
    switch (mode) {
        case M_IMM: return 2;
        case M_ZP: return 3;
        case M_ZPX: case M_ZPY: case M_ABS: return 4;
        case M_ABX: case M_ABY: return store ? 5 : 4;
        case M_IZX: return 6;
        default: return store ? 6 : 5;   // M_IZY
    }
}

constexpr uint32_t descriptor(Mn mn, uint32_t mode) {
    const uint32_t pen = (mode == M_ABX || mode == M_ABY || mode == M_IZY) ? D_PEN : 0u;
    const uint32_t rd = mode == M_IMM ? 0u : D_READ;
    switch (mn) {
        case ORA: case AND: case EOR: case ADC: case SBC: {
            const uint32_t sub = mn == ORA ? 0 : mn == AND ? 1 : mn == EOR ? 2 : mn == ADC ? 3 : 4;
            return desc(mode, rw_cycles(false, mode), G_ALU, sub, 0, 0, rd | pen);
        }
        case CMP: case CPX: case CPY:
            return desc(mode, rw_cycles(false, mode), G_ALU, 5, mn == CMP ? R_A : mn == CPX ? R_X : R_Y, 0, rd | pen);
        case BIT: return desc(mode, rw_cycles(false, mode), G_ALU, 6, 0, 0, D_READ);
        case LDA: case LDX: case LDY:
            return desc(mode, rw_cycles(false, mode), G_LD, 0, R_OPD, mn == LDA ? R_A : mn == LDX ? R_X : R_Y, rd | pen);
        case STA: case STX: case STY:
            return desc(mode, rw_cycles(true, mode), G_ST, 0, mn == STA ? R_A : mn == STX ? R_X : R_Y, 0, D_WRITE);
        case ASL: case ROL: case LSR: case ROR: {
            const uint32_t sub = mn == ASL ? 0 : mn == LSR ? 1 : mn == ROL ? 2 : 3;
            if (mode == M_IMP) return desc(M_IMP, 2, G_SHIFT, sub, R_A, R_A, 0);
            const uint32_t cyc = mode == M_ZP ? 5 : mode == M_ABX ? 7 : 6;
            return desc(mode, cyc, G_SHIFT, sub, R_OPD, R_OPD, D_READ | D_WRITE);
        }
        case INC: case DEC: {
            const uint32_t cyc = mode == M_ZP ? 5 : mode == M_ABX ? 7 : 6;
            return desc(mode, cyc, G_INCDEC, mn == DEC ? 1 : 0, R_OPD, R_OPD, D_READ | D_WRITE);
        }
        case INX: return desc(M_IMP, 2, G_INCDEC, 0, R_X, R_X, 0);
        case INY: return desc(M_IMP, 2, G_INCDEC, 0, R_Y, R_Y, 0);
        case DEX: return desc(M_IMP, 2, G_INCDEC, 1, R_X, R_X, 0);
        case DEY: return desc(M_IMP, 2, G_INCDEC, 1, R_Y, R_Y, 0);
        case BPL: return desc(M_REL, 2, G_BR, 7, 0, 0, 0);
        case BMI: return desc(M_REL, 2, G_BR, 7 | 8, 0, 0, 0);
        case BVC: return desc(M_REL, 2, G_BR, 6, 0, 0, 0);
        case BVS: return desc(M_REL, 2, G_BR, 6 | 8, 0, 0, 0);
        case BCC: return desc(M_REL, 2, G_BR, 0, 0, 0, 0);
        case BCS: return desc(M_REL, 2, G_BR, 0 | 8, 0, 0, 0);
        case BNE: return desc(M_REL, 2, G_BR, 1, 0, 0, 0);
        case BEQ: return desc(M_REL, 2, G_BR, 1 | 8, 0, 0, 0);
        case CLC: return desc(M_IMP, 2, G_FLAG, 0, 0, 0, 0);
        case SEC: return desc(M_IMP, 2, G_FLAG, 0 | 8, 0, 0, 0);
        case CLI: return desc(M_IMP, 2, G_FLAG, 2, 0, 0, 0);
        case SEI: return desc(M_IMP, 2, G_FLAG, 2 | 8, 0, 0, 0);
        case CLV: return desc(M_IMP, 2, G_FLAG, 6, 0, 0, 0);
        case CLD: return desc(M_IMP, 2, G_FLAG, 3, 0, 0, 0);
        case SED: return desc(M_IMP, 2, G_FLAG, 3 | 8, 0, 0, 0);
        case TAX: return desc(M_IMP, 2, G_LD, 0, R_A, R_X, 0);
        case TAY: return desc(M_IMP, 2, G_LD, 0, R_A, R_Y, 0);
        case TXA: return desc(M_IMP, 2, G_LD, 0, R_X, R_A, 0);
        case TYA: return desc(M_IMP, 2, G_LD, 0, R_Y, R_A, 0);
        case TSX: return desc(M_IMP, 2, G_LD, 0, R_SP, R_X, 0);
        case TXS: return desc(M_IMP, 2, G_LD, 0, R_X, R_SP, 0);
        case NOP: return desc(M_IMP, 2, G_NOP, 0, 0, 0, 0);
        case PHA: return desc(M_IMP, 3, G_PUSH, 0, R_A, 0, 0);
        case PHP: return desc(M_IMP, 3, G_PUSH, 0, R_X, 0, 0);   // src != A: the status byte
        case PLA: return desc(M_IMP, 4, G_PULL, 0, 0, R_A, 0);
        case PLP: return desc(M_IMP, 4, G_PULL, 0, 0, R_X, 0);   // dst != A: the status byte
        case JMP: return desc(mode, mode == M_IND ? 5 : 3, G_JMP, 0, 0, 0, 0);
        case JSR: return desc(M_ABS, 6, G_JSR, 0, 0, 0, 0);
        case RTS: return desc(M_IMP, 6, G_RTS, 0, 0, 0, 0);
        case RTI: return desc(M_IMP, 6, G_RTI, 0, 0, 0, 0);
        default: return desc(M_IMP, 7, G_BRK, 0, 0, 0, 0);   // BRK
    }
}

struct OpRow { uint8_t op; Mn mn; uint32_t mode; };
// column-group instructions: opcode = aaa << 5 | bbb << 2 | 01
constexpr uint32_t kG1Mode[8] = {M_IZX, M_ZP, M_IMM, M_ABS, M_IZY, M_ZPX, M_ABY, M_ABX};
constexpr Mn kG1[8] = {ORA, AND, EOR, ADC, STA, LDA, CMP, SBC};
// read-modify-write shifts and INC/DEC: opcode = aaa << 5 | bbb << 2 | 10
constexpr Mn kG2[8] = {ASL, ROL, LSR, ROR, STX, LDX, DEC, INC};
constexpr OpRow kRest[] = {
    {0x86, STX, M_ZP}, {0x8E, STX, M_ABS}, {0x96, STX, M_ZPY},
    {0xA2, LDX, M_IMM}, {0xA6, LDX, M_ZP}, {0xAE, LDX, M_ABS}, {0xB6, LDX, M_ZPY}, {0xBE, LDX, M_ABY},
    {0x84, STY, M_ZP}, {0x8C, STY, M_ABS}, {0x94, STY, M_ZPX},
    {0xA0, LDY, M_IMM}, {0xA4, LDY, M_ZP}, {0xAC, LDY, M_ABS}, {0xB4, LDY, M_ZPX}, {0xBC, LDY, M_ABX},
    {0xC0, CPY, M_IMM}, {0xC4, CPY, M_ZP}, {0xCC, CPY, M_ABS},
    {0xE0, CPX, M_IMM}, {0xE4, CPX, M_ZP}, {0xEC, CPX, M_ABS},
    {0x24, BIT, M_ZP}, {0x2C, BIT, M_ABS},
    {0x10, BPL, M_REL}, {0x30, BMI, M_REL}, {0x50, BVC, M_REL}, {0x70, BVS, M_REL},
    {0x90, BCC, M_REL}, {0xB0, BCS, M_REL}, {0xD0, BNE, M_REL}, {0xF0, BEQ, M_REL},
    {0x18, CLC, M_IMP}, {0x38, SEC, M_IMP}, {0x58, CLI, M_IMP}, {0x78, SEI, M_IMP}, {0xB8, CLV, M_IMP},
    {0xD8, CLD, M_IMP}, {0xF8, SED, M_IMP},
    {0xAA, TAX, M_IMP}, {0xA8, TAY, M_IMP}, {0x8A, TXA, M_IMP}, {0x98, TYA, M_IMP}, {0xBA, TSX, M_IMP},
    {0x9A, TXS, M_IMP}, {0xE8, INX, M_IMP}, {0xC8, INY, M_IMP}, {0xCA, DEX, M_IMP}, {0x88, DEY, M_IMP},
    {0xEA, NOP, M_IMP}, {0x48, PHA, M_IMP}, {0x08, PHP, M_IMP}, {0x68, PLA, M_IMP}, {0x28, PLP, M_IMP},
    {0x4C, JMP, M_ABS}, {0x6C, JMP, M_IND}, {0x20, JSR, M_ABS}, {0x60, RTS, M_IMP}, {0x40, RTI, M_IMP},
    {0x00, BRK, M_IMP},
};

struct Optab { uint32_t t[256]; };

constexpr Optab make_optab() {
    Optab o{};   // all G_ILL
    for (uint32_t a = 0; a < 8; ++a)
        for (uint32_t b = 0; b < 8; ++b) {
            if (kG1[a] == STA && kG1Mode[b] == M_IMM) continue;
            o.t[(a << 5) | (b << 2) | 1u] = descriptor(kG1[a], kG1Mode[b]);
        }
    for (uint32_t a = 0; a < 8; ++a) {
        const Mn mn = kG2[a];
        if (mn == STX || mn == LDX) continue;
        o.t[(a << 5) | (1u << 2) | 2u] = descriptor(mn, M_ZP);
        o.t[(a << 5) | (3u << 2) | 2u] = descriptor(mn, M_ABS);
        o.t[(a << 5) | (5u << 2) | 2u] = descriptor(mn, M_ZPX);
        o.t[(a << 5) | (7u << 2) | 2u] = descriptor(mn, M_ABX);
        if (a < 4) o.t[(a << 5) | (2u << 2) | 2u] = descriptor(mn, M_IMP);   // accumulator
    }
    for (const OpRow& r : kRest) o.t[r.op] = descriptor(r.mn, r.mode);
    return o;
}

// The descriptor table at compile time: the wave interpreter specialises each opcode's code on its entry.
constexpr Optab kOptab = make_optab();

inline void build_optab(uint32_t* t) {
    for (int i = 0; i < 256; ++i) t[i] = kOptab.t[i];
}

}  // namespace nd
