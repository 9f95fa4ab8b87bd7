// Wave-uniform fast path of the 6502 interpreter (gfx950).
//
// A console owned by a whole wavefront has wave-uniform state, so the compiler keeps it in SGPRs and runs it on the
// scalar unit with uniform branches. This header adds the fast path that makes that cheap: `switch (opcode)` where
// each case is the generic step (nes_dev.h cpu_step) specialised at compile time on that opcode's descriptor
// (optab.h kOptab), so an instruction is straight-line scalar code with no table decode. Instruction bytes come
// through the scalar data cache (constant address space loads of the widened PRG image).
//
// The fast path covers every official opcode whose memory operands are CPU RAM ($0000-$1FFF) or, for reads, PRG
// ($8000-$FFFF). Anything else - I/O registers, PRG RAM, open bus, a store or read-modify-write at $8000+ (a mapper
// write), BRK, an opcode outside the official set, a pending NMI or IRQ, code outside PRG - returns 0 before any
// state changes and the caller runs the generic step instead, so the semantics are exactly cpu_step's
// (third_party/nesle-extensions.patch:823-862 and rl/csrc/nes_machine.cuh:67-103 in kdcyberdude/ghostrun-lab).
#pragma once
#include "nes_dev.h"
#include "optab.h"

namespace nd {

typedef __attribute__((address_space(4))) const uint32_t ConstU32;
typedef __attribute__((address_space(4))) const uint8_t ConstU8;

// Registers the fast loop keeps live: the CPU registers, the cycle counter and the PRG page offsets. Everything
// else about the console (PPU, controller, DMC, mapper) stays in the console state in LDS and only the generic
// step, the PPU settle and the idle fast-forward touch it, so the loop's live set is small enough to stay in SGPRs.
// N and Z are kept lazily in one value nz: N = (nz >= $80), Z = (low byte of nz == 0). An instruction that sets both
// from a result r stores r itself; BIT, whose N comes from the operand, adds the operand's bit 7 as bit 8. The N and
// Z bits of p are stale in between and are rebuilt when p is stored or pushed.
// pc is held as pcs, the byte offset of its fetch-table entry (8 bytes an entry), so the fetch needs no address
// arithmetic. On NROM the table is by CPU address and pcs = pc * 8; it may run one past $FFFF after the last
// instruction of the address space and is wrapped when stored (the fast path sends such a pc to the generic step).
// On the banked boards the table is by PRG offset, pcs = (PRG offset of pc) * 8 and pd = that offset - pc (mod 2^32),
// so pc = pcs / 8 - pd. Within an 8 KB page the offset moves with pc: the table sends every instruction that ends on
// the last byte of its page to the generic step, so sequential flow never leaves a page in the fast path, a branch to
// another page goes to the generic step, and every jump, call and return maps its target again (hot_pcs), as does
// the reload after the generic step, which is the only place the PRG mapping changes.
struct Hot {
    uint32_t pc, a, x, y, sp, p, nz;
    uint32_t c, v;  // the carry (0 or 1) and V in bit 7 (lazy, as N and Z in nz); p's own C and V bits are stale
    uint32_t ctl;   // controller 1: shift register | strobe << 8
    uint64_t cycles;
    uint32_t prg0, prg1, prg2, prg3;
    uint32_t pd;
};
constexpr uint32_t kPcShift = 3u;
// The banked boards' stand-in for a pc outside PRG ($0000-$7FFF, or one past $FFFF): the entry of the last byte of
// PRG page 0, which holds the generic step's key (no instruction that starts there ends inside the page).
constexpr uint32_t kOffPrg = 0x1FFFu;

// (uni(): a wave-uniform value read from LDS, as a scalar - replay_dev.h. An LDS load lands in a VGPR; without it the
// compiler moves every use of the value to the vector unit, with lane-mask compares instead of SCC branches.)

// The lazy N and Z of a status byte p: bit 8 = N, and a low byte that is 0 exactly when Z is set.
__device__ __forceinline__ uint32_t nz_of_p(uint32_t p) {
    return ((p & FL_N) << 1) | ((p & FL_Z) ? 0u : 1u);
}

// p with N, Z, C and V rebuilt from the values kept apart.
__device__ __forceinline__ uint32_t hflags(const Hot& h) {
    return (h.p & ~(FL_N | FL_Z | FL_C | FL_V)) | (h.nz >= 0x80u ? FL_N : 0u) | ((h.nz & 0xFFu) ? 0u : FL_Z) | h.c |
           ((h.v >> 1) & FL_V);
}
// C and V kept apart from a status byte p.
__device__ __forceinline__ void hcv(Hot& h, uint32_t p) {
    h.c = p & FL_C;
    h.v = (p & FL_V) << 1;
}

// pcs of CPU address `pc` (on the banked boards also pd, from the PRG offsets in h).
template <uint32_t B>
__device__ __forceinline__ uint32_t hot_pcs(Hot& h, uint32_t pc) {
    if constexpr (B == NES_BOARD_NROM) {
        return pc << kPcShift;
    } else {
        if (pc - 0x8000u >= 0x8000u) {
            h.pd = kOffPrg - pc;
            return kOffPrg << kPcShift;
        }
        const uint32_t page = sel4((pc >> 13) & 3u, h.prg0, h.prg1, h.prg2, h.prg3);
        h.pd = page - (pc & 0xE000u);
        return (page + (pc & 0x1FFFu)) << kPcShift;
    }
}
// The CPU address of pcs (not wrapped).
template <uint32_t B>
__device__ __forceinline__ uint32_t hot_cpu(const Hot& h, uint32_t pcs) {
    if constexpr (B == NES_BOARD_NROM) return pcs >> kPcShift;
    else return (pcs >> kPcShift) - h.pd;
}

template <uint32_t B>
__device__ __forceinline__ void hot_load(Hot& h, const Con& c) {
    h.a = uni(c.a); h.x = uni(c.x); h.y = uni(c.y); h.sp = uni(c.sp); h.p = uni(c.p);
    h.nz = nz_of_p(h.p);
    hcv(h, h.p);
    h.cycles = uni64(c.cycles);
    h.prg0 = uni(c.prg0); h.prg1 = uni(c.prg1); h.prg2 = uni(c.prg2); h.prg3 = uni(c.prg3);
    h.pd = 0;
    h.pc = hot_pcs<B>(h, uni(c.pc));
    h.ctl = uni(c.shift) | (uni(c.strobe) << 8);
}
// (the PRG offsets change only in the generic step and map_write_fast, which write them to the console state)
template <uint32_t B>
__device__ __forceinline__ void hot_store(const Hot& h, Con& c) {
    c.pc = hot_cpu<B>(h, h.pc) & 0xFFFFu; c.a = h.a; c.x = h.x; c.y = h.y; c.sp = h.sp; c.p = hflags(h);
    c.cycles = h.cycles;
    c.shift = h.ctl & 0xFFu;
    c.strobe = h.ctl >> 8;
}

__device__ __forceinline__ uint32_t hget(const Hot& h, uint32_t code, uint32_t opd) {
    return code == R_A ? h.a : code == R_X ? h.x : code == R_Y ? h.y : code == R_SP ? h.sp : opd;
}
__device__ __forceinline__ void hset(Hot& h, uint32_t code, uint32_t v) {
    if (code == R_A) h.a = v;
    else if (code == R_X) h.x = v;
    else if (code == R_Y) h.y = v;
    else if (code == R_SP) h.sp = v;
}
__device__ __forceinline__ void hnz(Hot& h, uint32_t v) {   // v < 256
    h.nz = v;
}
// A CPU RAM byte (LDS) as a scalar: the value is wave-uniform, and in an SGPR the code that uses it stays on the
// scalar unit (SCC branches instead of VALU compares and VCC branches).
__device__ __forceinline__ uint32_t rd8(const Mem& m, uint32_t a) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)m.ram[a]);
}

__device__ __forceinline__ void hpush(Hot& h, const Mem& m, uint32_t v) {
    m.ram[0x100u | h.sp] = (uint8_t)v;
    h.sp = (h.sp - 1u) & 0xFFu;
}
__device__ __forceinline__ uint32_t hpull(Hot& h, const Mem& m) {
    h.sp = (h.sp + 1u) & 0xFFu;
    return rd8(m, 0x100u | h.sp);
}

// Controller port 1 ($4016), one of the two I/O registers the fast path serves itself: the same read and write as
// the bus (nes_dev.h io_read / io_write), on the console state in LDS.
__device__ __forceinline__ uint32_t port_read(Hot& h, const Con& cs) {
    uint32_t bit;
    if (h.ctl >> 8) {
        bit = uni(cs.pad) & 1u;
    } else {
        bit = h.ctl & 1u;
        h.ctl = (h.ctl >> 1) | 0x80u;
    }
    return 0x40u | bit;
}
// PPU status ($2002 and its mirrors): the bus's read (nes_dev.h io_read) - the value, then vblank and the write
// toggle cleared. Status bits change only at PPU events, and the fast path runs only short of the next one, so the
// status in the console state is the one the read sees.
__device__ __forceinline__ uint32_t status_read(Con& cs) {
    const uint32_t st = uni(cs.status);
    const uint32_t v = (st & 0xE0u) | (uni(cs.open_bus) & 0x1Fu);
    cs.status = st & 0x7Fu;
    cs.w = 0;
    cs.open_bus = v;
    return v;
}
__device__ __forceinline__ void port_write(Hot& h, const Con& cs, uint32_t v) {
    h.ctl = (v & 1u) ? (uni(cs.pad) | 0x100u) : (h.ctl & 0xFFu);
}
// PPU register writes ($2000-$3FFF) in a burst that starts between vblank and the pre-render line (cs.b_quiet): the
// frame log is off from vblank to the pre-render line (nes_dev.h cpu_step's log_on), a burst ends short of the next
// PPU event (vblank, the $2002 clear, the pre-render line, the sprite-0 check, an MMC3 clock: dots_to_event), and
// what the writes feed - the log header, the sprite-0 schedule, MMC3's clocks, which fall on visible lines and the
// pre-render line - is taken at those events, so such a write is the bus's own (nes_dev.h ppu_reg_write) with nothing
// logged. Whether the fast path can take it, decided before any state changes: not a $2000 write that raises an NMI
// (the NMI is taken before the next instruction, by the generic step), not MMC2's $2006 / $2007 (the VRAM address
// flips its latches).
template <uint32_t B>
__device__ __forceinline__ bool ppu_write_quiet(const Mem& m, const Con& cs, uint32_t reg, uint32_t v) {
    if (!uni(cs.b_quiet)) return false;
    if (reg == 0u && !(uni(cs.ctrl) & 0x80u) && (v & 0x80u) && (uni(cs.status) & 0x80u)) return false;
    if constexpr (B != NES_BOARD_NROM)
        if (m.cart.board == NES_BOARD_MMC2 && reg >= 6u) return false;
    return true;
}
__device__ __forceinline__ void ppu_write(const Mem& m, Con& cs, uint32_t reg, uint32_t v) {
    Access ac;
    ac.now = 0;
    ac.log_on = false;
    ac.dma = false;
    ppu_reg_write(cs, m, ac, reg, v);
}

// Byte offset in the PRG image of CPU address `addr` ($8000-$FFFF). NROM maps the image linearly (mirrored).
template <uint32_t B>
__device__ __forceinline__ uint32_t prg_index(const Hot& h, const Mem& m, uint32_t addr) {
    if constexpr (B == NES_BOARD_NROM) return addr & 0x7FFFu;   // the NROM image is 32 KB (16 KB mirrored)
    else return sel4((addr >> 13) & 3u, h.prg0, h.prg1, h.prg2, h.prg3) + (addr & 0x1FFFu);
}

// Mapper writes the fast path takes (nes_dev.h map_write and map_sync restate the boards): those that change no CHR
// page, no mirroring and no IRQ state, and switch no PRG page that the instruction runs in (the next one is on the
// same page: kFetchWords), so nothing is logged for the renderer:
//   - MMC3: a bank select ($8000, even) that keeps the PRG and CHR modes (bits 6-7), a bank data write ($8001, odd)
//     to R6 or R7 (patch:3158-3162 the registers, 3037-3048 the pages);
//   - MMC1: a serial-port write that only shifts a bit in (a reset, and the fifth write, which loads a register, go
//     to the generic step; patch:3128-3145);
//   - UxROM: the 16 KB bank at $8000, ANDed with the byte under the write when the cart declares bus conflicts;
//   - MMC2: the 8 KB bank at $8000 ($A000-$AFFF; patch:3147-3149).
// map_write_ok only decides (no state change); map_write_fast writes the register to the record and the PRG pages
// through to the console state, the record and h. What the decision needs is in the console state (Con::map_fast),
// not a global load away.
template <uint32_t B>
__device__ __forceinline__ uint32_t map_rom_byte(const Hot& h, const Mem& m, uint32_t ea) {
    return prg_wide(m, prg_index<B>(h, m, ea)) & 0xFFu;
}
// The PRG slots (bit i: the 8 KB page at $8000 + i * $2000) a write of v at ea that the fast path takes switches.
__device__ __forceinline__ uint32_t map_fast_slots(const Mem& m, const Con& cs, uint32_t ea) {
    const uint32_t board = m.cart.board;
    if (board == NES_BOARD_MMC3) {
        const uint32_t sel = uni(cs.map_fast);
        return (ea & 1u) == 0u ? 0u : (sel & 7u) == 7u ? 2u : (sel & 0x40u) ? 4u : 1u;
    }
    return board == NES_BOARD_UXROM ? 3u : board == NES_BOARD_MMC2 ? 1u : 0u;
}
template <uint32_t B>
__device__ __forceinline__ bool map_write_ok(const Hot& h, const Mem& m, const Con& cs, uint32_t ea, uint32_t v,
                                             uint32_t pcs) {
    const uint32_t board = m.cart.board;
    if (board == NES_BOARD_MMC3) {
        const uint32_t k = ea & 0xE001u, sel = uni(cs.map_fast);
        if (k == 0x8000u) {
            if ((sel ^ v) & 0xC0u) return false;
        } else if (k != 0x8001u || (sel & 7u) < 6u) {
            return false;
        }
    } else if (board == NES_BOARD_MMC1) {
        return (v & 0x80u) == 0u && (uni(cs.map_fast) >> 8) < 4u;
    } else if (board == NES_BOARD_MMC2) {
        if ((ea & 0xF000u) != 0xA000u) return false;
    } else if (board != NES_BOARD_UXROM) {
        return false;
    }
    const uint32_t cpu = hot_cpu<B>(h, pcs);
    return cpu < 0x8000u || ((map_fast_slots(m, cs, ea) >> ((cpu >> 13) & 3u)) & 1u) == 0u;
}
template <uint32_t B>
__device__ __forceinline__ void map_set_prg_fast(Hot& h, const Mem& m, Con& cs, uint32_t slot, uint32_t page) {
    const uint32_t off = (page & (m.cart.prg_pages8 - 1u)) * 8192u;   // map_set_prg
    m.rec->prg_off[slot] = off;
    if (slot == 0u) {
        h.prg0 = off;
        cs.prg0 = off;
    } else if (slot == 1u) {
        h.prg1 = off;
        cs.prg1 = off;
    } else {
        h.prg2 = off;
        cs.prg2 = off;
    }
}
template <uint32_t B>
__device__ __forceinline__ void map_write_fast(Hot& h, const Mem& m, Con& cs, uint32_t ea, uint32_t v) {
    uint8_t* r = m.rec->mreg;
    const uint32_t board = m.cart.board;
    if (board == NES_BOARD_MMC3) {
        const uint32_t sel = uni(cs.map_fast);
        if ((ea & 1u) == 0u) {
            r[8] = (uint8_t)v;
            cs.map_fast = v;
        } else {
            r[sel & 7u] = (uint8_t)v;
            map_set_prg_fast<B>(h, m, cs, (sel & 7u) == 7u ? 1u : (sel & 0x40u) ? 2u : 0u, v);
        }
    } else if (board == NES_BOARD_MMC1) {
        const uint32_t sr = uni(cs.map_fast), n = sr >> 8, bits = (sr & 0xFFu) | ((v & 1u) << n);
        r[4] = (uint8_t)bits;
        r[5] = (uint8_t)(n + 1u);
        cs.map_fast = bits | ((n + 1u) << 8);
    } else if (board == NES_BOARD_MMC2) {
        r[4] = (uint8_t)(v & 0x0Fu);
        map_set_prg_fast<B>(h, m, cs, 0u, v & 0x0Fu);
    } else {   // UxROM
        const uint32_t b = m.cart.bus_conflicts ? (v & map_rom_byte<B>(h, m, ea)) : v;
        r[0] = (uint8_t)b;
        map_set_prg_fast<B>(h, m, cs, 0u, b * 2u);
        map_set_prg_fast<B>(h, m, cs, 1u, b * 2u + 1u);
    }
}

// A PRG RAM byte ($6000-$7FFF, in the console record), as a scalar; the bus's read (nes_dev.h io_read) with the RAM
// on, which it is on every board but MMC1 (the fast path leaves MMC1's to the generic step).
__device__ __forceinline__ uint32_t prg_ram_read(const Mem& m, uint32_t a) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)m.rec->prg_ram[a - 0x6000u]);
}

// Widened PRG word at `idx` (bytes idx, idx+1, idx+2) through a scalar load: the image is read-only for the
// whole kernel.
__device__ __forceinline__ uint32_t prg_wide(const Mem& m, uint32_t idx) {
    return ((ConstU32*)m.cart.prgw)[idx];
}

// A fast-path result: the instruction needs the generic step (nothing changed). As a take off the burst counter
// (cycles << 14) - 1 it stands for 0 cycles.
constexpr uint32_t kGeneric = 0xFFFFFFFFu;

// One instruction of opcode descriptor D at pcs (operand bytes lo, hi). Returns what it takes
// off the burst counter, (CPU cycles << 14) - 1, or kGeneric with nothing changed when the generic step must run it.
// The operand word comes decoded from the fetch table (kFetchWords): the operand byte of a two-byte instruction; a
// branch's target times 8 (NROM) or its sign-extended offset times 8 (banked boards); JMP's and JSR's target (times 8
// on NROM);
// else lo | hi << 8. HOT: a hot key (a branch that stays on its page).
// Whether the conditional branch of descriptor D is taken: its flag (N and Z from the lazy nz, the others from p) has
// the value the branch tests for.
template <uint32_t D>
__device__ __forceinline__ bool br_taken(const Hot& h) {
    constexpr uint32_t sub = (D >> 12) & 15u, bit = sub & 7u;
    bool set;
    if constexpr (bit == 7u) set = h.nz >= 0x80u;
    else if constexpr (bit == 1u) set = (h.nz & 0xFFu) == 0u;
    else if constexpr (bit == 0u) set = h.c != 0u;
    else if constexpr (bit == 6u) set = (h.v & 0x80u) != 0u;
    else set = ((h.p >> bit) & 1u) != 0;
    return set == ((sub & 8u) != 0);
}

// PPU: absolute PPU register writes of a quiet burst here too (ppu_write_quiet; the translated blocks' instructions,
// whose register is known when the block is compiled; other stores there and elsewhere: the generic step).
template <uint32_t B, uint32_t D, bool HOT = false, bool PPU = false>
__device__ __forceinline__ uint32_t fx(Hot& h, const Mem& m, Con& cs, uint32_t pcs, uint32_t base) {
    constexpr uint32_t PS = kPcShift;
    constexpr bool nrom = B == NES_BOARD_NROM;
    constexpr uint32_t mode = D & 15u, grp = (D >> 8) & 15u, sub = (D >> 12) & 15u;
    constexpr uint32_t src = (D >> 16) & 7u, dst = (D >> 19) & 7u;
    constexpr bool rd = (D & D_READ) != 0, wr = (D & D_WRITE) != 0, pen = (D & D_PEN) != 0;
    constexpr bool zpage = mode == M_ZP || mode == M_ZPX || mode == M_ZPY;
    if constexpr (grp == G_ILL || grp == G_BRK) {
        return kGeneric;
    } else {
        uint32_t cyc = (D >> 4) & 15u;
        constexpr bool two = mode == M_IMM || mode == M_ZP || mode == M_ZPX || mode == M_ZPY || mode == M_IZX ||
                             mode == M_IZY;
        const uint32_t lo = two ? base : (base & 0xFFu);
        uint32_t ea = 0;
        if constexpr (mode == M_ZP) {
            ea = lo;
        } else if constexpr (mode == M_ZPX) {
            ea = (lo + h.x) & 0xFFu;
        } else if constexpr (mode == M_ZPY) {
            ea = (lo + h.y) & 0xFFu;
        } else if constexpr (mode == M_ABS || mode == M_IND) {
            ea = base;
        } else if constexpr (mode == M_ABX || mode == M_ABY) {
            ea = (base + (mode == M_ABX ? h.x : h.y)) & 0xFFFFu;
            if constexpr (pen) cyc += ((base ^ ea) & 0xFF00u) ? 1u : 0u;
        } else if constexpr (mode == M_IZX) {
            const uint32_t ptr = (lo + h.x) & 0xFFu;
            ea = rd8(m, ptr) | (rd8(m, (ptr + 1u) & 0xFFu) << 8);
        } else if constexpr (mode == M_IZY) {
            const uint32_t b2 = rd8(m, lo) | (rd8(m, (lo + 1u) & 0xFFu) << 8);
            ea = (b2 + h.y) & 0xFFFFu;
            if constexpr (pen) cyc += ((b2 ^ ea) & 0xFF00u) ? 1u : 0u;
        }
        // Memory class, decided before any side effect (every check below comes before the first state change):
        // RAM, PRG RAM ($6000-$7FFF; on MMC1, whose register can disable it, the generic step), PRG reads, the
        // controller port and PPU status reads run here; any other I/O register, a read-modify-write elsewhere and
        // any write at $8000+ (a mapper) but the bank writes of map_write_ok go to the generic step. Written
        // as chains of single compares: boolean
        // combinations of uniform conditions become lane-mask arithmetic.
        if constexpr (!zpage && rd && wr) {
            if (ea >= 0x2000u) {
                if (ea < 0x6000u) return kGeneric;
                if (ea >= 0x8000u) return kGeneric;
                if (m.cart.board == NES_BOARD_MMC1) return kGeneric;
            }
        }
        if constexpr (!zpage && wr && !rd) {
            if (ea >= 0x2000u) {
                if (ea != 0x4016u) {
                    if (ea < 0x4000u) {
                        if constexpr (!PPU || mode != M_ABS) return kGeneric;
                        else if (!ppu_write_quiet<B>(m, cs, ea & 7u, hget(h, src, 0))) return kGeneric;
                    } else if (ea < 0x6000u) return kGeneric;
                    if (ea >= 0x8000u) {   // (a bank write is an absolute store; an indexed one: the generic step)
                        if constexpr (nrom || mode != M_ABS) return kGeneric;
                        else if (!map_write_ok<B>(h, m, cs, ea, hget(h, src, 0), pcs)) return kGeneric;
                    } else if (m.cart.board == NES_BOARD_MMC1) {
                        return kGeneric;
                    }
                }
            }
        }
        uint32_t opd = lo;
        if constexpr (rd) {
            if constexpr (mode == M_ZP) {
                opd = rd8(m, ea);   // the fetch table's operand byte: < $100
            } else if constexpr (zpage) {
                opd = rd8(m, ea & 0x7FFu);
            } else if constexpr (wr) {
                opd = ea < 0x2000u ? rd8(m, ea & 0x7FFu) : prg_ram_read(m, ea);
            } else {
                if (ea < 0x2000u) opd = rd8(m, ea & 0x7FFu);
                else if (ea >= 0x8000u) opd = prg_wide(m, prg_index<B>(h, m, ea)) & 0xFFu;
                else if (ea == 0x4016u) opd = port_read(h, cs);
                else if ((ea & 0xE007u) == 0x2002u) opd = status_read(cs);
                else if (ea >= 0x6000u && m.cart.board != NES_BOARD_MMC1) opd = prg_ram_read(m, ea);
                else return kGeneric;
            }
        }
        constexpr uint32_t len = instr_len(mode);
        uint32_t npc = pcs + (len << PS), res = 0;   // pc <= $FFFD here; $10000 is wrapped when stored
        if constexpr (grp == G_LD) {
            res = hget(h, src, opd);
            hset(h, dst, res);
            if constexpr (dst != R_SP) hnz(h, res);
        } else if constexpr (grp == G_ST) {
            res = hget(h, src, 0);
        } else if constexpr (grp == G_INCDEC) {
            res = (hget(h, src, opd) + (sub ? 0xFFu : 1u)) & 0xFFu;
            hset(h, dst, res);
            hnz(h, res);
        } else if constexpr (grp == G_ALU) {
            if constexpr (sub <= 2) {
                h.a = sub == 0 ? (h.a | opd) : sub == 1 ? (h.a & opd) : (h.a ^ opd);
                hnz(h, h.a);
            } else if constexpr (sub <= 4) {
                const uint32_t mv = sub == 4 ? (opd ^ 0xFFu) : opd;
                const uint32_t sum = h.a + mv + h.c;
                h.v = ~(h.a ^ mv) & (h.a ^ sum);   // bit 7: the signed overflow
                h.c = sum >> 8;
                h.a = sum & 0xFFu;
                hnz(h, h.a);
            } else if constexpr (sub == 5) {
                const uint32_t r = hget(h, src, 0);
                h.c = r >= opd ? 1u : 0u;
                hnz(h, (r - opd) & 0xFFu);
            } else {
                h.v = opd << 1;                               // V from the operand's bit 6
                h.nz = (h.a & opd) | ((opd & 0x80u) << 1);   // N from the operand, Z from A & operand
            }
        } else if constexpr (grp == G_SHIFT) {
            const uint32_t in = hget(h, src, opd), cin = h.c;
            uint32_t cout;
            if constexpr (sub == 0) { res = (in << 1) & 0xFFu; cout = in >> 7; }
            else if constexpr (sub == 1) { res = in >> 1; cout = in & 1u; }
            else if constexpr (sub == 2) { res = ((in << 1) | cin) & 0xFFu; cout = in >> 7; }
            else { res = (in >> 1) | (cin << 7); cout = in & 1u; }
            h.c = cout;
            hset(h, dst, res);
            hnz(h, res);
        } else if constexpr (grp == G_BR) {
            if (br_taken<D>(h)) {
                const uint32_t tgt = nrom ? base : npc + base;   // wrapped when stored
                if constexpr (!nrom && !HOT) {
                    if ((npc ^ tgt) >> 16) return kGeneric;   // to another 8 KB page: bits 13+ of the PRG offset
                }
                if constexpr (HOT) cyc += 1u;
                else cyc += ((npc ^ tgt) & (0xFF00u << PS)) ? 2u : 1u;
                npc = tgt;
            }
        } else if constexpr (grp == G_FLAG) {
            constexpr uint32_t bit = sub & 7u, bitm = 1u << bit;
            if constexpr (bit == 0u) h.c = (sub & 8u) ? 1u : 0u;
            else if constexpr (bit == 6u) h.v = (sub & 8u) ? 0x80u : 0u;
            else h.p = (sub & 8u) ? (h.p | bitm) : (h.p & ~bitm);
        } else if constexpr (grp == G_PUSH) {
            hpush(h, m, src == R_A ? h.a : (hflags(h) | FL_B | FL_U));
        } else if constexpr (grp == G_PULL) {
            const uint32_t v = hpull(h, m);
            if constexpr (dst == R_A) {
                h.a = v;
                hnz(h, v);
            } else {
                h.p = (v & ~FL_B) | FL_U;
                h.nz = nz_of_p(h.p);
                hcv(h, h.p);
            }
        } else if constexpr (grp == G_JMP) {
            if constexpr (mode == M_IND) {
                const uint32_t a1 = (base & 0xFF00u) | ((base + 1u) & 0xFFu);
                if ((base >= 0x2000u && base < 0x8000u) || (a1 >= 0x2000u && a1 < 0x8000u)) return kGeneric;
                const uint32_t l8 = base < 0x2000u ? rd8(m, base & 0x7FFu)
                                                   : (prg_wide(m, prg_index<B>(h, m, base)) & 0xFFu);
                const uint32_t h8 = a1 < 0x2000u ? rd8(m, a1 & 0x7FFu)
                                                 : (prg_wide(m, prg_index<B>(h, m, a1)) & 0xFFu);
                npc = hot_pcs<B>(h, l8 | (h8 << 8));
            } else {
                // the idle loop (a jump to itself): the generic step runs it, then the fast-forward
                if constexpr (nrom) {
                    npc = base;
                    if (npc == pcs) return kGeneric;
                } else {
                    if (base == hot_cpu<B>(h, pcs)) return kGeneric;
                    npc = hot_pcs<B>(h, base);
                }
            }
        } else if constexpr (grp == G_JSR) {
            const uint32_t ret = hot_cpu<B>(h, pcs) + 2u;   // <= $FFFF
            hpush(h, m, ret >> 8);
            hpush(h, m, ret & 0xFFu);
            npc = nrom ? base : hot_pcs<B>(h, base);
        } else if constexpr (grp == G_RTS) {
            const uint32_t l8 = hpull(h, m), h8 = hpull(h, m);
            npc = hot_pcs<B>(h, ((h8 << 8) | l8) + 1u);
        } else if constexpr (grp == G_RTI) {
            h.p = (hpull(h, m) & ~FL_B) | FL_U;
            h.nz = nz_of_p(h.p);
            hcv(h, h.p);
            const uint32_t l8 = hpull(h, m), h8 = hpull(h, m);
            npc = hot_pcs<B>(h, (h8 << 8) | l8);
        }
        if constexpr (wr) {
            if constexpr (mode == M_ZP) m.ram[ea] = (uint8_t)res;
            else if constexpr (zpage) m.ram[ea & 0x7FFu] = (uint8_t)res;
            else if (ea < 0x2000u) m.ram[ea & 0x7FFu] = (uint8_t)res;
            else if (PPU && mode == M_ABS && !rd && ea < 0x4000u) ppu_write(m, cs, ea & 7u, res);
            else if (!nrom && !rd && mode == M_ABS && ea >= 0x8000u) map_write_fast<B>(h, m, cs, ea, res);
            else if (ea >= 0x6000u) m.rec->prg_ram[ea - 0x6000u] = (uint8_t)res;   // (a read-modify-write: here)
            else port_write(h, cs, res);
        }
        h.pc = npc;
        return (cyc << 14) - 1u;   // the caller adds the cycles and services the DMC, as cpu_step does after its count
    }
}

// (a hot opcode other than a branch never reaches the switch over all opcodes: its case merges into the default; a
// branch to another page comes here with its opcode)
#define ND_FX(n)                                                                              \
    case n:                                                                                   \
        if constexpr (is_hot(n) && (kOptab.t[n] & 15u) != M_REL)                              \
            return kGeneric;                                                                  \
        else                                                                                  \
            return fx<B, kOptab.t[n]>(h, m, cs, pcs, base);
#define ND_HOT(i) \
    case kHotKey + i: return fx<B, kOptab.t[kHotOps[i]], true>(h, m, cs, pcs, base);
#define ND_HOT8(i) ND_HOT(i) ND_HOT(i + 1) ND_HOT(i + 2) ND_HOT(i + 3) ND_HOT(i + 4) ND_HOT(i + 5) ND_HOT(i + 6) ND_HOT(i + 7)
#define ND_FX16(h)                                                                                                    \
    ND_FX(h + 0x0) ND_FX(h + 0x1) ND_FX(h + 0x2) ND_FX(h + 0x3) ND_FX(h + 0x4) ND_FX(h + 0x5) ND_FX(h + 0x6)          \
    ND_FX(h + 0x7) ND_FX(h + 0x8) ND_FX(h + 0x9) ND_FX(h + 0xA) ND_FX(h + 0xB) ND_FX(h + 0xC) ND_FX(h + 0xD)          \
    ND_FX(h + 0xE) ND_FX(h + 0xF)

// The opcodes' switch (without the hot ones, which never reach it).
template <uint32_t B>
__device__ __forceinline__ uint32_t fx_all(Hot& h, const Mem& m, Con& cs, uint32_t pcs, uint32_t op, uint32_t base) {
    switch (op) {
        ND_FX16(0x00) ND_FX16(0x10) ND_FX16(0x20) ND_FX16(0x30) ND_FX16(0x40) ND_FX16(0x50) ND_FX16(0x60)
        ND_FX16(0x70) ND_FX16(0x80) ND_FX16(0x90) ND_FX16(0xA0) ND_FX16(0xB0) ND_FX16(0xC0) ND_FX16(0xD0)
        ND_FX16(0xE0) ND_FX16(0xF0)
        default: return kGeneric;
    }
}

// The hot keys' switch.
template <uint32_t B>
__device__ __forceinline__ uint32_t fx_hot(Hot& h, const Mem& m, Con& cs, uint32_t pcs, uint32_t op, uint32_t base) {
    switch (op) {
        ND_HOT8(0) ND_HOT8(8) ND_HOT8(16) ND_HOT8(24)
        default: __builtin_unreachable();   // the fetch table holds no other key >= kHotKey
    }
}

// The fast path for the instruction at h.pc: (its cycles << 14) - 1, or kGeneric (nothing changed) for the generic
// step. The instruction comes decoded from the fetch table at byte offset pcs, a scalar load with an SGPR offset: on
// NROM pcs = pc * 8 (pc <= $1007E, a branch just past $FFFF; $02 outside PRG), on the banked boards the PRG offset
// of pc times 8 ($02 where an instruction would end on the last byte of its 8 KB page, and kOffPrg for a pc outside
// PRG).
template <uint32_t B>
__device__ __forceinline__ uint32_t fast_step(Hot& h, const Mem& m, Con& cs, uint32_t op, uint32_t base) {
    const uint32_t pcs = h.pc;
    if (__builtin_expect(op >= kHotKey, 1)) return fx_hot<B>(h, m, cs, pcs, op, base);
    // (read back as an opaque scalar: with the range op < $100 known the compiler narrows the switch to 8 bits and
    // widens it again with two masks)
    return fx_all<B>(h, m, cs, pcs, uni(op), base);
}
// The same, fetching the entry itself.
template <uint32_t B>
__device__ __forceinline__ uint32_t fast_step(Hot& h, const Mem& m, Con& cs, uint32_t* op_out) {
    // (two 32-bit loads, which the compiler pairs into one 64-bit load: read as the halves of a 64-bit value,
    // base's compares would become 64-bit ones, which the scalar unit has only for equality)
    ConstU32* e = (ConstU32*)((ConstU8*)m.cart.fetchw + h.pc);
    const uint32_t op = e[0], base = e[1];
    *op_out = op;
    return fast_step<B>(h, m, cs, op, base);
}
#undef ND_FX16
#undef ND_FX
#undef ND_HOT8
#undef ND_HOT

// Cycles from `now` until the DMC's next event, saturated to 32 bits (an idle DMC is never reached within a frame).
__device__ __forceinline__ uint32_t dmc_distance(uint64_t now, uint64_t event) {
    if (event <= now) return 0;
    const uint64_t d = event - now;
    return d > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)d;
}

#ifdef RLENV_JIT_INC
// The most a translated block's instruction can take off the burst counter: its cycles with the page-crossing
// penalty and a taken branch to another page.
constexpr uint32_t jit_maxtake(uint32_t op) {
    return ((((kOptab.t[op] >> 4) & 15u) + ((kOptab.t[op] & D_PEN) ? 1u : 0u) +
             (((kOptab.t[op] >> 8) & 15u) == G_BR ? 2u : 0u)) << 14) - 1u;
}
// One instruction of a block (inside the block's room), and the block's first instruction alone (no room for the
// block: the interpreter's own test ends the burst).
#define JIT_STEP(op, pcs, base)                              \
    t = fx<B, kOptab.t[op], false, true>(h, m, cs, pcs, base); \
    if (t == kGeneric) { take = t; goto burst_end; }          \
    v -= t;
#define JIT_ONE(op, pcs, base)                               \
    t = fx<B, kOptab.t[op], false, true>(h, m, cs, pcs, base); \
    if (v < t) { take = t; goto burst_end; }                  \
    v -= t;                                                   \
    continue;
#endif

// The frame loop (rl/csrc/nes_machine.cuh:67-103) for a console whose state `cs` lives in LDS: instructions until a
// settle reaches absolute dot `target`, the PPU settled lazily when the unsettled dots reach the event horizon and
// after an idle jump (then fast-forwarded), within the instruction budget, stopping on a fault. Fast instructions run
// in bursts that keep only Hot and a few scalars live, counting CPU cycles in 32 bits since the last flush into
// h.cycles (a frame is ~30k cycles); the generic step and the settle work on `cs` (registers written back before and
// reloaded after the generic step; the settle touches no CPU register). Every settle goes through the one call of
// ppu_step at the top of the loop, so its replays are inlined once.
template <uint32_t B>
__device__ __forceinline__ uint32_t run_until_wave(Con& cs, const Mem& m, const uint32_t* optab, uint64_t target,
                                                   uint32_t budget = NES_BUDGET) {
    uint32_t instructions = 0, fault = 0, pending = 0;
    uint32_t to_event = uni(dots_to_event(cs, m));
    Hot h;
    hot_load<B>(h, cs);
    uint64_t dmc_event = uni64(cs.dmc_event);
    uint32_t ecyc = 0;                                     // cycles not yet added to h.cycles
    uint32_t dmc_in = dmc_distance(h.cycles, dmc_event);   // from h.cycles to the DMC event; ecyc <= dmc_in here
    uint32_t nmi = uni(cs.nmi_pending), irq = uni(cs.irq_line);
    // why a settle is due besides the horizon: 1 after an idle jump (then the fast-forward), 2 before leaving
    uint32_t why = 0;
    // The last fast instruction took the cycle count to the DMC event: service it, then count the instruction with
    // the stolen cycles (cpu_step's order).
    auto dmc_due = [&](uint32_t cyc) {
        h.cycles += ecyc;
        ecyc = 0;
        const uint32_t s = dmc_service(m.rec, h.cycles, 1);
        dmc_event = uni64(m.rec->dmc_event);
        h.cycles += s;
        dmc_in = dmc_distance(h.cycles, dmc_event);
        pending += 3u * (cyc + s);
        ++instructions;
    };
    for (;;) {
        if (why == 0 && instructions >= budget) why = 2;
        if (why != 0 || pending >= to_event) {
            ppu_step<B>(cs, m, pending);   // touches no CPU register
            pending = 0;
            nmi = uni(cs.nmi_pending);
            irq = uni(cs.irq_line);
            if (why == 2) break;
            if (why == 1) {
                why = 0;
                if (abs_dot(cs) >= target) break;
                // The idle JMP-to-self loop (patch:866-893): whole 3-cycle jumps up to the next PPU event, settled at
                // once; not with an NMI raised by the settle before it. (h is current: the generic step stored it.)
                if (!nmi) {
                    const uint32_t jumps = (uni(dots_to_event(cs, m, true)) + 8u) / 9u;
                    if (jumps) {
                        h.cycles += 3u * jumps;
                        if (h.cycles >= dmc_event) {
                            (void)dmc_service(m.rec, h.cycles, 0);
                            dmc_event = uni64(m.rec->dmc_event);
                        }
                        dmc_in = dmc_distance(h.cycles, dmc_event);
                        pending = 9u * jumps;
                        to_event = 0;
                        continue;
                    }
                }
                to_event = uni(dots_to_event(cs, m));
                continue;
            }
            to_event = uni(dots_to_event(cs, m));
            if (abs_dot(cs) >= target) break;
        }
        uint32_t op = 0, pc0 = 0, cyc = 0;
        if (((nmi | (irq & ~(h.p >> 2))) & 1u) == 0u) {   // no NMI, and no IRQ unless the I flag masks it
            // Fast instructions. With no IRQ asserted (a masked one is taken as soon as CLI, PLP or RTI clears the I
            // flag) this is a burst: they run back to back until one needs the generic step (cyc = 0, nothing
            // changed) or the cycles used reach `room`, the nearest of the DMC event, the PPU event horizon (3 dots a
            // cycle) and the instruction budget (every instruction takes at least 2 cycles, so a burst never passes
            // it). Otherwise one instruction runs. lm1 = room - 1 (< 2^15: the horizon is less than a frame, 89342
            // dots, away). One register counts both: v = lm1 << 14 | instructions run (< 2^14: half the room at
            // most), and each instruction takes (cyc << 14) - 1 off it (a constant for most handlers). v < take
            // exactly when cyc > lm1, "cyc == 0 or cyc >= room" (kGeneric stands for a cyc of 0).
            uint32_t lm1 = 0;
            if ((irq & 1u) == 0u)
                lm1 = uni(max(min(min(dmc_in - ecyc, (to_event - pending + 2u) / 3u), 2u * (budget - instructions)),
                              1u) - 1u);
            const uint32_t lm1_0 = lm1;
            uint32_t v = lm1 << 14, take;
            // The wave's issue priority from the dots left to the frame's target (half a frame or more, a quarter,
            // an eighth, less): the arbiter takes the oldest wave first among equals, so without this the waves of a
            // CU finish far apart and the last ones run with too few others to hide their latency; the steps halve
            // toward the end, where the spread is left.
            {
                const uint64_t left = target - abs_dot(cs);
                if (left >= NES_FRAME_DOTS / 2u) __builtin_amdgcn_s_setprio(3);
                else if (left >= NES_FRAME_DOTS / 4u) __builtin_amdgcn_s_setprio(2);
                else if (left >= NES_FRAME_DOTS / 8u) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
            }
            // What no instruction of the burst touches waits in LDS until the burst ends: left in registers it would
            // crowd the burst's own values (the 6502 registers and flags) out of the scalar registers and into
            // vector-register lanes.
            cs.b_dmc_event = dmc_event;
            cs.b_target = target;
            cs.b_instructions = instructions;
            cs.b_pending = pending;
            cs.b_to_event = to_event;
            cs.b_ecyc = ecyc;
            cs.b_dmc_in = dmc_in;
            cs.b_why = why;
            cs.b_budget = budget;
            cs.b_nmi = nmi;
            cs.b_irq = irq;
            {
                const uint32_t d0 = uni(cs.frame_dot) + pending;   // the burst's first dot (< the next event)
                cs.b_quiet = d0 >= NES_VBLANK_DOT && d0 < NES_PRERENDER_DOT ? 1u : 0u;
            }
            for (;;) {
#ifdef RLENV_JIT_INC
                ConstU32* e = (ConstU32*)((ConstU8*)m.cart.fetchw + h.pc);
                const uint32_t fop = e[0], fbase = e[1];
                if (fop >= kBlockKey) {   // a translated block starts here (jit.h)
                    uint32_t t;
                    switch (fop) {
#include RLENV_JIT_INC
                        default: __builtin_unreachable();
                    }
                }
                take = fast_step<B>(h, m, cs, fop, fbase);
#else
                take = fast_step<B>(h, m, cs, &op);
#endif
                if (v < take) break;
                v -= take;
            }
#ifdef RLENV_JIT_INC
        burst_end:
#endif
            dmc_event = uni64(cs.b_dmc_event);
            target = uni64(cs.b_target);
            instructions = uni(cs.b_instructions);
            pending = uni(cs.b_pending);
            to_event = uni(cs.b_to_event);
            ecyc = uni(cs.b_ecyc);
            dmc_in = uni(cs.b_dmc_in);
            why = uni(cs.b_why);
            budget = uni(cs.b_budget);
            nmi = uni(cs.b_nmi);
            irq = uni(cs.b_irq);
            cyc = (take + 1u) >> 14;               // 0 for kGeneric
            lm1 = v >> 14;
            const uint32_t n = (v & 0x3FFFu) + 1u;
            const uint32_t used = lm1_0 - lm1 + cyc;   // cycles of the n instructions
            ecyc += used;
            if (cyc != 0u) {
                if (ecyc >= dmc_in) {   // the last one took the cycle count to the DMC event
                    pending += 3u * (used - cyc);
                    instructions += n - 1u;
                    dmc_due(cyc);
                } else {                // the event horizon or the budget: back to the top
                    pending += 3u * used;
                    instructions += n;
                }
                continue;
            }
            pending += 3u * used;       // the last one needs the generic step
            instructions += n - 1u;
        }
        // the generic step: I/O, interrupts, the idle loop, BRK, faults, code outside PRG
        h.cycles += ecyc;
        ecyc = 0;
        if constexpr (B != NES_BOARD_NROM) {
            // MMC3: the counter's clocks up to the instruction first (its horizon is only the IRQ's clock)
            if (m.cart.board == NES_BOARD_MMC3 && pending != 0u) {
                mmc3_presettle(cs, m, pending);
                pending = 0;
            }
        }
        hot_store<B>(h, cs);
        cs.dmc_event = dmc_event;
        cyc = cpu_step(cs, m, optab, uni(cs.frame_dot) + pending, &fault, &op, &pc0);
        hot_load<B>(h, cs);
        dmc_event = uni64(cs.dmc_event);
        dmc_in = dmc_distance(h.cycles, dmc_event);
        nmi = uni(cs.nmi_pending);
        irq = uni(cs.irq_line);
        if (fault) {
            why = 2;
            continue;
        }
        if constexpr (B != NES_BOARD_NROM) {
            // the instruction may have moved the IRQ's clock (a mapper or PPU register write); pending is 0 here
            if (m.cart.board == NES_BOARD_MMC3) to_event = uni(dots_to_event(cs, m));
        }
        pending += 3u * cyc;
        ++instructions;
        if (op == 0x4Cu && hot_cpu<B>(h, h.pc) == pc0) why = 1;
    }
    h.cycles += ecyc;
    hot_store<B>(h, cs);
    cs.dmc_event = dmc_event;
    cs.instr += instructions;
    return fault;
}

}  // namespace nd
