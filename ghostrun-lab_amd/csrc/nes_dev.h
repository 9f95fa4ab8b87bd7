// Device-side NES console for gfx950: one console per lane, hot registers in VGPRs, the 2 KB CPU RAM in LDS,
// everything else in the console record in HBM (include/nesrec.h).
//
// The 6502 is table-driven: one 32-bit descriptor per opcode (addressing mode, cycles, operation group and its
// parameters, read/write/penalty flags) held in LDS. Every instruction runs the same fetch -> effective address
// -> bus read -> group -> bus write sequence, so lanes on different opcodes diverge only inside the short group
// switch and inside the bus decode. Instruction fetch is one 32-bit load from a widened PRG image (word i holds
// PRG bytes i, i+1, i+2), so opcode and both operand bytes arrive in one memory access.
//
// Semantics are those of the reference env's NES machine (kdcyberdude/ghostrun-lab): frame loop
// rl/csrc/nes_machine.cuh:67-103, instruction step third_party/nesle-extensions.patch:823-862, bus side effects
// patch:570-779, PPU events patch:1822-2240, frame log patch:894-1185, mappers patch:2841-3367, DMC patch:430-565.
#pragma once
#ifndef ND_HOST_BUILD
#include <hip/hip_runtime.h>
#endif
#include <stdint.h>

#include "nesrec.h"

namespace nd {

constexpr uint32_t kRamStride = 2052;   // LDS bytes per console: 513 words, so equal offsets of 64 consoles hit 64 banks
constexpr uint32_t kNoHit = 0x7FFFFFFFu;
constexpr uint64_t kDmcIdle = ~0ull;
constexpr uint32_t FL_C = 1, FL_Z = 2, FL_I = 4, FL_D = 8, FL_B = 16, FL_U = 32, FL_V = 64, FL_N = 128;

// ---------------------------------------------------------------------------------- opcode descriptors
enum : uint32_t { M_IMP = 0, M_IMM, M_ZP, M_ZPX, M_ZPY, M_ABS, M_ABX, M_ABY, M_IZX, M_IZY, M_REL, M_IND };
enum : uint32_t {
    G_ILL = 0, G_LD, G_ST, G_INCDEC, G_ALU, G_SHIFT, G_BR, G_FLAG, G_NOP, G_PUSH, G_PULL, G_JMP, G_JSR, G_RTS,
    G_RTI, G_BRK
};
enum : uint32_t { R_OPD = 0, R_A = 1, R_X = 2, R_Y = 3, R_SP = 4 };   // register codes of src/dst fields
// descriptor bits: mode 0-3 | cycles 4-7 | group 8-11 | sub 12-15 | src 16-18 | dst 19-21 | read 22 | write 23 |
// page-cross penalty 24
constexpr uint32_t D_READ = 1u << 22, D_WRITE = 1u << 23, D_PEN = 1u << 24;
__host__ __device__ constexpr uint32_t desc(uint32_t mode, uint32_t cyc, uint32_t grp, uint32_t sub, uint32_t src,
                                            uint32_t dst, uint32_t flags) {
    return mode | (cyc << 4) | (grp << 8) | (sub << 12) | (src << 16) | (dst << 19) | flags;
}

// ----------------------------------------------------------------------------------- per-lane state
struct Con {
    uint32_t pc, a, x, y, sp, p;
    uint32_t irq_line, nmi_pending;
    uint64_t cycles;
    uint32_t pad, shift, strobe, instr;
    uint32_t frame_dot, frame;
    uint32_t v, t, ctrl, mask, status, oam_addr, fx, w, read_buf, open_bus;
    int32_t s0_dot;
    uint32_t log_frame, log_n, s0_valid;
    uint64_t dmc_event;
    uint32_t prg0, prg1, prg2, prg3;   // PRG byte offsets of $8000/$A000/$C000/$E000
    uint32_t nt_map;                   // 4 x 2 bits
};

struct Cart {
    const uint32_t* prgw;   // widened PRG
    const uint32_t* fetchw; // decoded instructions: NROM by CPU address (kFetchWords x 2 words), else by PRG offset
    const uint8_t* chr;     // CHR ROM, nullptr = CHR RAM in the record
    uint32_t prg_pages8;    // 8 KB pages (power of two)
    uint32_t chr_pages1;    // 1 KB pages (power of two)
    uint32_t board;
    uint32_t mirroring;     // header: 0 horizontal, 1 vertical
    uint32_t bus_conflicts; // UxROM / CNROM declared with AND-type bus conflicts (NES 2.0 submapper 2)
};

// Instruction-fetch table (fast path): entry = {dispatch key, operand word}, two dwords: the opcode, or its hot key
// for the opcodes of kHotOps, and the decoded operand. NROM and CNROM (fixed PRG): entry a for CPU address a, for
// $8000 <= a <= $FFFD; every other entry (RAM, I/O, the last two bytes, and a pc just past $FFFF) holds opcode $02,
// which no fast-path handler runs, so the generic step fetches it. Banked boards: one entry per PRG byte offset (the
// last two of each 8 KB page hold $02: an instruction there runs into the next CPU page).
constexpr uint32_t kFetchWords = 0x10100u;

// Opcodes the NROM fetch table stores as hot keys $100 + i (i = index here) instead of the opcode: the interpreter
// dispatches a hot key through a switch of 32 cases (5 compares) after one range check, and every other opcode
// through the switch over all 256 (8 compares). The list is the common core of 6502 game code: loads and stores of
// A, the conditional branches, subroutine calls, counters, and the immediate-operand arithmetic and shifts.
constexpr uint32_t kHotOps[32] = {
    0xA9u, 0xA5u, 0xADu, 0xBDu, 0xB9u, 0xB1u, 0xA2u, 0xA6u, 0xA0u,   // LDA #, zp, abs, abs,X, abs,Y, (zp),Y; LDX #, zp; LDY #
    0x85u, 0x8Du, 0x9Du, 0x99u,                                      // STA zp, abs, abs,X, abs,Y
    0xD0u, 0xF0u, 0x10u, 0x90u, 0xB0u,                               // BNE BEQ BPL BCC BCS
    0x20u, 0x60u, 0x4Cu,                                             // JSR RTS JMP
    0xE8u, 0xCAu, 0xC8u, 0x88u,                                      // INX DEX INY DEY
    0xC9u, 0x29u, 0x18u, 0x69u, 0x4Au, 0x0Au, 0xAAu};                // CMP # AND # CLC ADC # LSR A ASL A TAX
constexpr uint32_t kHotKey = 0x100u;
constexpr bool is_hot(uint32_t op) {
    for (uint32_t i = 0; i < 32u; ++i)
        if (kHotOps[i] == op) return true;
    return false;
}

struct Mem {
    NesRec* rec;
    uint8_t* ram;           // this console's 2 KB CPU RAM (LDS)
    uint8_t* nt;            // 2 KB nametable RAM, 256 B OAM, 32 B palette: the record's, or LDS copies of them
    uint8_t* oam;
    uint8_t* pal;
    Cart cart;
};

// The memories of a console record, with the CPU RAM at `ram`.
__device__ __forceinline__ Mem mem_of(NesRec* rec, uint8_t* ram, const Cart& cart) {
    return Mem{rec, ram, rec->nt, rec->oam, rec->pal, cart};
}

__device__ __forceinline__ uint32_t sel4(uint32_t i, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return i & 2u ? (i & 1u ? d : c) : (i & 1u ? b : a);
}
__device__ __forceinline__ uint32_t prg_off(const Con& c, uint32_t addr) {
    return sel4((addr >> 13) & 3u, c.prg0, c.prg1, c.prg2, c.prg3);
}
__device__ __forceinline__ uint32_t prg_byte(const Con& c, const Mem& m, uint32_t addr) {
    return m.cart.prgw[prg_off(c, addr) + (addr & 0x1FFFu)] & 0xFFu;
}
__device__ __forceinline__ bool prg_ram_on(const Mem& m) {
    return m.cart.board != NES_BOARD_MMC1 || (m.rec->mreg[3] & 0x10u) == 0;
}
__device__ __forceinline__ uint32_t nt_index(uint32_t nt_map, uint32_t addr) {
    return ((nt_map >> (((addr >> 10) & 3u) * 2u)) & 1u) * 1024u + (addr & 0x3FFu);
}
__device__ __forceinline__ uint32_t chr_byte(const Mem& m, const uint32_t* chr_off, uint32_t a) {
    const uint32_t off = chr_off[(a >> 10) & 7u] + (a & 0x3FFu);
    return m.cart.chr ? m.cart.chr[off] : m.rec->chr_ram[off & (NES_CHRRAM_BYTES - 1u)];
}
// CHR byte through packed page numbers (replay state)
__device__ __forceinline__ uint32_t chr_byte_pk(const Mem& m, uint32_t lo, uint32_t hi, uint32_t a) {
    const uint32_t slot = (a >> 10) & 7u;
    const uint32_t page = ((slot & 4u ? hi : lo) >> ((slot & 3u) * 8u)) & 0xFFu;
    const uint32_t off = page * 1024u + (a & 0x3FFu);
    return m.cart.chr ? m.cart.chr[off] : m.rec->chr_ram[off & (NES_CHRRAM_BYTES - 1u)];
}

// ----------------------------------------------------------------------------------------- mappers
__device__ inline void map_set_prg(Con& c, const Mem& m, uint32_t slot, uint32_t page) {
    const uint32_t off = (page & (m.cart.prg_pages8 - 1u)) * 8192u;
    if (slot == 0) c.prg0 = off; else if (slot == 1) c.prg1 = off; else if (slot == 2) c.prg2 = off; else c.prg3 = off;
    m.rec->prg_off[slot] = off;
}
__device__ inline void map_set_chr(const Mem& m, uint32_t slot, uint32_t page) {
    m.rec->chr_off[slot] = (page & (m.cart.chr_pages1 - 1u)) * 1024u;
}
__device__ inline uint32_t nt_map_of(uint32_t kind) {   // 0 horizontal, 1 vertical, 2 single low, 3 single high
    return kind == 0 ? 0x50u : kind == 1 ? 0x44u : kind == 2 ? 0x00u : 0x55u;
}
__device__ inline void map_set_nt(Con& c, const Mem& m, uint32_t kind) {
    c.nt_map = nt_map_of(kind);
    for (uint32_t k = 0; k < 4; ++k) m.rec->nt_map[k] = (uint8_t)((c.nt_map >> (2 * k)) & 3u);
}

// MMC2: an address in $0FD0-$0FEF / $1FD0-$1FEF flips the latch of its half (FCEUmm's PPU_hook ranges,
// patch:3196-3220, 1390-1402). 0 = none, else the latch value + 1 | half << 2.
__device__ __forceinline__ uint32_t mmc2_trigger(uint32_t a) {
    const uint32_t high = (a >> 8) & 0x3Fu, low = a & 0xF0u;
    if (high >= 0x20u || (high & 0x0Fu) != 0x0Fu || (low != 0xD0u && low != 0xE0u)) return 0;
    return (low == 0xE0u ? 2u : 1u) | (high < 0x10u ? 0u : 4u);
}

// Page tables from the board registers (MMC1: control, CHR0, CHR1, PRG; MMC3: R0-R7, select, mirroring, ...;
// MMC2: CHR $FD/$0000, $FE/$0000, $FD/$1000, $FE/$1000, PRG, mirroring, latch 0, latch 1).
__device__ inline void map_sync(Con& c, const Mem& m) {
    const uint8_t* r = m.rec->mreg;
    if (m.cart.board == NES_BOARD_MMC1) {
        const uint32_t ctl = r[0], outer = r[1] & 0x10u, bank = r[3] & 0x0Fu;
        const uint32_t mode = (ctl >> 2) & 3u;
        const uint32_t lo = mode == 3 ? bank + outer : mode == 2 ? outer : (bank & ~1u) + outer;
        const uint32_t hi = mode == 3 ? 0x0Fu + outer : mode == 2 ? bank + outer : lo + 1u;
        map_set_prg(c, m, 0, 2u * lo);
        map_set_prg(c, m, 1, 2u * lo + 1u);
        map_set_prg(c, m, 2, 2u * hi);
        map_set_prg(c, m, 3, 2u * hi + 1u);
        const bool four = (ctl & 0x10u) != 0;
        const uint32_t c0 = four ? r[1] : (r[1] & 0xFEu), c1 = four ? r[2] : (r[1] | 1u);
        for (uint32_t i = 0; i < 4; ++i) {
            map_set_chr(m, i, 4u * c0 + i);
            map_set_chr(m, 4u + i, 4u * c1 + i);
        }
        const uint32_t mir = ctl & 3u;   // 0 one-screen low, 1 one-screen high, 2 vertical, 3 horizontal
        map_set_nt(c, m, mir == 0 ? 2u : mir == 1 ? 3u : mir == 2 ? 1u : 0u);
    } else if (m.cart.board == NES_BOARD_MMC3) {
        const uint32_t s = r[8];
        const bool swap = (s & 0x40u) != 0;
        map_set_prg(c, m, 0, swap ? 0x7Eu : r[6]);
        map_set_prg(c, m, 1, r[7]);
        map_set_prg(c, m, 2, swap ? r[6] : 0x7Eu);
        map_set_prg(c, m, 3, 0x7Fu);
        const uint32_t f = (s & 0x80u) ? 4u : 0u;
        map_set_chr(m, 0u ^ f, r[0] & 0xFEu);
        map_set_chr(m, 1u ^ f, r[0] | 1u);
        map_set_chr(m, 2u ^ f, r[1] & 0xFEu);
        map_set_chr(m, 3u ^ f, r[1] | 1u);
        for (uint32_t i = 0; i < 4; ++i) map_set_chr(m, (4u + i) ^ f, r[2 + i]);
        map_set_nt(c, m, (r[9] & 1u) ? 0u : 1u);
    } else if (m.cart.board == NES_BOARD_MMC2) {   // the 8 KB bank at $8000, the last three fixed (patch:3027-3035)
        map_set_prg(c, m, 0, r[4]);
        map_set_prg(c, m, 1, ~2u);
        map_set_prg(c, m, 2, ~1u);
        map_set_prg(c, m, 3, ~0u);
        for (uint32_t i = 0; i < 4; ++i) {
            map_set_chr(m, i, 4u * r[r[6] & 1u] + i);
            map_set_chr(m, 4u + i, 4u * r[2u + (r[7] & 1u)] + i);
        }
        map_set_nt(c, m, r[5] ? 1u : 0u);
    } else if (m.cart.board == NES_BOARD_UXROM) {   // the 16 KB bank in register 0, the last one fixed at $C000
        const uint32_t last = m.cart.prg_pages8 / 2u - 1u;
        map_set_prg(c, m, 0, r[0] * 2u);
        map_set_prg(c, m, 1, r[0] * 2u + 1u);
        map_set_prg(c, m, 2, last * 2u);
        map_set_prg(c, m, 3, last * 2u + 1u);
        for (uint32_t i = 0; i < 8; ++i) map_set_chr(m, i, i);
        map_set_nt(c, m, m.cart.mirroring ? 1u : 0u);
    } else {   // NROM; CNROM: the 8 KB CHR bank in register 0 (patch:2982-2990)
        const uint32_t chr8 = m.cart.board == NES_BOARD_CNROM ? r[0] : 0u;
        for (uint32_t i = 0; i < 4; ++i) map_set_prg(c, m, i, i);
        for (uint32_t i = 0; i < 8; ++i) map_set_chr(m, i, chr8 * 8u + i);
        map_set_nt(c, m, m.cart.mirroring ? 1u : 0u);
    }
}

__device__ inline void map_write(Con& c, const Mem& m, uint32_t addr, uint32_t v) {
    uint8_t* r = m.rec->mreg;
    if (m.cart.board == NES_BOARD_MMC1) {
        if (v & 0x80u) {
            r[0] |= 0x0Cu;
            r[4] = 0;
            r[5] = 0;
        } else {
            const uint32_t n = r[5];
            r[4] = (uint8_t)(r[4] | ((v & 1u) << n));
            if (n + 1u < 5u) {
                r[5] = (uint8_t)(n + 1u);
                return;
            }
            r[(addr >> 13) & 3u] = r[4];
            r[4] = 0;
            r[5] = 0;
        }
        map_sync(c, m);
    } else if (m.cart.board == NES_BOARD_MMC3) {
        const uint32_t k = addr & 0xE001u;
        if (k == 0x8000u) r[8] = (uint8_t)v;
        else if (k == 0x8001u) r[r[8] & 7u] = (uint8_t)v;
        else if (k == 0xA000u) r[9] = (uint8_t)v;
        else {
            if (k == 0xA001u) r[10] = (uint8_t)v;
            else if (k == 0xC000u) r[11] = (uint8_t)v;
            else if (k == 0xC001u) r[14] = 1;
            else if (k == 0xE000u) { r[13] = 0; c.irq_line = 0; }
            else r[13] = 1;
            return;
        }
        map_sync(c, m);
    } else if (m.cart.board == NES_BOARD_MMC2) {   // patch:3147-3156
        const uint32_t k = addr & 0xF000u;
        if (k == 0xA000u) r[4] = (uint8_t)(v & 0x0Fu);
        else if (k >= 0xB000u && k <= 0xE000u) r[(k >> 12) - 0xBu] = (uint8_t)(v & 0x1Fu);
        else if (k == 0xF000u) r[5] = (uint8_t)((v & 1u) ^ 1u);
        else return;   // $8000-$9FFF: no register
        map_sync(c, m);
    } else if (m.cart.board == NES_BOARD_CNROM || m.cart.board == NES_BOARD_UXROM) {
        // the bank latch, ANDed with the ROM byte under a bus conflict
        const uint32_t rom = m.cart.prgw[m.rec->prg_off[(addr >> 13) & 3u] + (addr & 0x1FFFu)] & 0xFFu;
        r[0] = (uint8_t)(m.cart.bus_conflicts ? (v & rom) : v);
        map_sync(c, m);
    }
}

__device__ inline void mmc3_clock(Con& c, const Mem& m) {
    uint8_t* r = m.rec->mreg;
    uint32_t cnt = r[12];
    if (cnt == 0 || r[14] != 0) {
        cnt = r[11];
        r[14] = 0;
    } else {
        --cnt;
    }
    r[12] = (uint8_t)cnt;
    if (cnt == 0 && r[13] != 0) c.irq_line = 1;
}

// ---------------------------------------------------------------------------------------------- DMC
__device__ __forceinline__ uint32_t dmc_period(uint32_t rate) {
    // NTSC CPU cycles per output bit, $4010 bits 0-3
    const uint32_t lo4 = rate & 15u;
    uint32_t p = 54;
    switch (lo4) {
        case 0: p = 428; break; case 1: p = 380; break; case 2: p = 340; break; case 3: p = 320; break;
        case 4: p = 286; break; case 5: p = 254; break; case 6: p = 226; break; case 7: p = 214; break;
        case 8: p = 190; break; case 9: p = 160; break; case 10: p = 142; break; case 11: p = 128; break;
        case 12: p = 106; break; case 13: p = 84; break; case 14: p = 72; break; default: p = 54; break;
    }
    return p;
}

// Service of the sample channel at CPU cycle `now`: drains the buffered byte on its clock, fetches the next at once
// (4 stolen cycles each when `steal`), skips silent whole bytes, applies a rate change from the next bit clock.
__device__ __forceinline__ uint32_t dmc_service(NesRec* r, uint64_t now, int steal) {
    const uint64_t byte_cycles = 8ull * dmc_period(r->dmc_rate);
    uint64_t end = r->dmc_byte_end;
    uint32_t full = r->dmc_full, left = r->dmc_left, stolen = 0;
    const uint32_t control = r->dmc_control;
    if (!full && end <= now) end += ((now - end) / byte_cycles + 1u) * byte_cycles;
    while (true) {
        if (full) {
            if (end > now) break;
            full = 0;
            end += byte_cycles;
            if (left == 0) {
                if (end <= now) end += ((now - end) / byte_cycles + 1u) * byte_cycles;
                break;
            }
        }
        if (left == 0) break;
        full = 1;
        --left;
        if (left == 0 && (control & 0x40u)) left = r->dmc_length * 16u + 1u;
        if (steal) {
            stolen += 4;
            now += 4;
        }
    }
    const uint32_t rate = control & 15u;
    if (rate != r->dmc_rate) {
        const uint64_t oldp = dmc_period(r->dmc_rate);
        const uint64_t later = (end - now - 1u) / oldp;
        end = end - later * oldp + later * dmc_period(rate);
        r->dmc_rate = (uint8_t)rate;
    }
    r->dmc_byte_end = end;
    r->dmc_full = (uint8_t)full;
    r->dmc_left = (uint16_t)left;
    r->dmc_event = full ? end : kDmcIdle;
    return stolen;
}

// ------------------------------------------------------------------------------- line replay (frame log)
// Renderer state of one line: the PPU state at dot 320 of the line before (the first tile prefetch).
struct Replay {
    uint32_t v, t, fx, ctrl, mask;
    uint32_t chr_lo, chr_hi;   // 1 KB CHR page of slots 0-3 / 4-7, 8 bits each
    uint32_t nt_map;
    uint32_t creg, latch;      // MMC2: the 4 CHR registers (8 bits each), latch 0 | latch 1 << 8
    uint32_t mmc2_pages;       // MMC2: the cart's 1 KB CHR pages; 0 on other boards
    uint32_t ev, count;
    int32_t next;              // time of event ev (INT32_MAX when none is left)
    const uint32_t* events;
};

// MMC2: half `half`'s slots from its register and latch (patch:1385-1388)
__device__ __forceinline__ void rp_mmc2_select(Replay& s, uint32_t half) {
    const uint32_t reg = 2u * half + ((s.latch >> (8u * half)) & 1u);
    const uint32_t bank = (s.creg >> (8u * reg)) & 0xFFu;
    uint32_t pk = 0;
    for (uint32_t i = 0; i < 4u; ++i) pk |= ((bank * 4u + i) & (s.mmc2_pages - 1u)) << (8u * i);
    if (half) s.chr_hi = pk;
    else s.chr_lo = pk;
}
// MMC2: the latch hook of a pattern fetch at a (patch:1390-1402)
__device__ __forceinline__ void rp_hook(Replay& s, uint32_t a) {
    const uint32_t t = mmc2_trigger(a);
    if (t == 0) return;
    const uint32_t half = t >> 2;
    s.latch = (s.latch & ~(0xFFu << (8u * half))) | (((t & 3u) - 1u) << (8u * half));
    rp_mmc2_select(s, half);
}

__device__ __forceinline__ int32_t rp_time(const Replay& s, uint32_t i) {
    return (int32_t)(s.events[2u * i] & 0xFFFFFFu) - NES_LOG_TIME_BIAS;
}

// Applies event i. Palette writes go to `pal` (nullptr: ignored, as in the sprite-0 scan).
__device__ inline void rp_apply(Replay& s, uint32_t i, uint8_t* pal) {
    const uint32_t w0 = s.events[2u * i], w1 = s.events[2u * i + 1u];
    const uint32_t kind = w0 >> 24, val = w1 & 0xFFu, aux = (w1 >> 8) & 0xFFu;
    const uint32_t step = (s.ctrl & 4u) ? 32u : 1u;
    if (kind == NES_EV_CTRL) {
        s.ctrl = val;
        s.t = (s.t & 0xF3FFu) | ((val & 3u) << 10);
    } else if (kind == NES_EV_MASK) {
        s.mask = val;
    } else if (kind == NES_EV_SCROLL) {
        if (aux == 0) {
            s.t = (s.t & 0xFFE0u) | (val >> 3);
            s.fx = val & 7u;
        } else {
            s.t = (s.t & 0x0C1Fu) | ((val & 7u) << 12) | ((val & 0xF8u) << 2);
        }
    } else if (kind == NES_EV_ADDR) {
        if (aux == 0) {
            s.t = (s.t & 0x00FFu) | ((val & 0x3Fu) << 8);
        } else {
            s.t = (s.t & 0xFF00u) | val;
            s.v = s.t;
        }
    } else if (kind == NES_EV_DATA) {
        s.v = (s.v + aux * step) & 0x7FFFu;
    } else if (kind == NES_EV_PAL) {
        if (pal) pal[aux & 31u] = (uint8_t)val;
        s.v = (s.v + step) & 0x7FFFu;
    } else if (kind == NES_EV_CHR) {
        const uint32_t sh = (aux & 3u) * 8u, keep = ~(0xFFu << sh);
        if (aux & 4u) s.chr_hi = (s.chr_hi & keep) | (val << sh);
        else s.chr_lo = (s.chr_lo & keep) | (val << sh);
    } else if (kind == NES_EV_MIRROR) {
        s.nt_map = val;
    } else if (kind == NES_EV_MMC2) {   // patch:1471-1478
        if (aux < 4u) {
            s.creg = (s.creg & ~(0xFFu << (8u * aux))) | (val << (8u * aux));
            rp_mmc2_select(s, aux >> 1);
        } else if (aux == 6u || aux == 7u) {
            const uint32_t h = aux - 6u;
            s.latch = (s.latch & ~(0xFFu << (8u * h))) | ((val & 1u) << (8u * h));
            rp_mmc2_select(s, h);
        }
    }
}

__device__ __forceinline__ void rp_next(Replay& s) {
    s.next = s.ev < s.count ? rp_time(s, s.ev) : INT32_MAX;
}

// Applies the events before `time`; the time of the next one is kept in a register, so a check with nothing to apply
// reads no memory.
__device__ inline void rp_until(Replay& s, int32_t time, uint8_t* pal) {
    while (s.next < time) {
        rp_apply(s, s.ev, pal);
        ++s.ev;
        rp_next(s);
    }
}

__device__ inline void rp_yinc(Replay& s) {
    if ((s.v & 0x7000u) != 0x7000u) {
        s.v += 0x1000u;
        return;
    }
    s.v &= ~0x7000u;
    uint32_t cy = (s.v >> 5) & 31u;
    if (cy == 29u) {
        cy = 0;
        s.v ^= 0x0800u;
    } else if (cy == 31u) {
        cy = 0;
    } else {
        ++cy;
    }
    s.v = (s.v & ~0x03E0u) | (cy << 5);
}

// After line l's pixels: Y increment (dot 256), horizontal copy (257), on the pre-render line (l = -1) the vertical
// copy (304); the state at dot 320 is the next line's.
__device__ inline void rp_line_end(Replay& s, int l, uint8_t* pal) {
    const int32_t base = l * 341;
    rp_until(s, base + 256, pal);
    if (s.mask & 0x18u) rp_yinc(s);
    rp_until(s, base + 257, pal);
    if (s.mask & 0x18u) s.v = (s.v & ~0x041Fu) | (s.t & 0x041Fu);
    if (l < 0) {
        rp_until(s, base + 304, pal);
        if (s.mask & 0x18u) s.v = (s.v & ~0x7BE0u) | (s.t & 0x7BE0u);
    }
    rp_until(s, base + 320, pal);
}

// events: the log's event words (from `log` + NES_LOG_HDR_WORDS on), in place or a copy of them. mmc2_pages: the
// cart's 1 KB CHR pages on MMC2, else 0.
__device__ inline void rp_begin(Replay& s, const uint32_t* log, uint32_t log_n, uint8_t* pal, const uint32_t* events,
                                uint32_t mmc2_pages) {
    const uint32_t h1 = log[1], h2 = log[2], h3 = log[3], h4 = log[4];
    s.creg = log[14];
    s.latch = log[15];
    s.mmc2_pages = mmc2_pages;
    s.ctrl = h1 & 0xFFu;
    s.mask = (h1 >> 8) & 0xFFu;
    s.fx = (h1 >> 16) & 7u;
    s.v = h2 & 0xFFFFu;
    s.t = h2 >> 16;
    s.chr_lo = h3;
    s.chr_hi = h4;
    s.nt_map = log[5] & 0xFFu;
    if (pal)
        for (uint32_t i = 0; i < 8; ++i) {
            const uint32_t w = log[6 + i];
            pal[4 * i] = (uint8_t)w; pal[4 * i + 1] = (uint8_t)(w >> 8);
            pal[4 * i + 2] = (uint8_t)(w >> 16); pal[4 * i + 3] = (uint8_t)(w >> 24);
        }
    s.events = events;
    s.count = log_n < NES_LOG_EVENTS ? log_n : NES_LOG_EVENTS;
    s.ev = 0;
    rp_next(s);
    rp_line_end(s, -1, pal);
}

// Background 2-bit value at pixel x of a line drawn with state s (nametables/CHR read through the record), the
// pattern bytes through the slot pages lo/hi.
__device__ inline uint32_t rp_bg(const Replay& s, const Mem& m, uint32_t x, uint32_t* pal_sel, uint32_t lo_pk,
                                 uint32_t hi_pk) {
    const uint32_t pos = x + s.fx, bit = pos & 7u;
    uint32_t cx = (s.v & 31u) + (pos >> 3), nth = (s.v >> 10) & 1u;
    if (cx >= 32u) {
        cx -= 32u;
        nth ^= 1u;
    }
    const uint32_t cy = (s.v >> 5) & 31u, fy = (s.v >> 12) & 7u;
    const uint32_t base = 0x2000u | ((nth | (((s.v >> 11) & 1u) << 1)) << 10);
    const uint32_t tile = m.nt[nt_index(s.nt_map, base | (cy << 5) | cx)];
    const uint32_t at = m.nt[nt_index(s.nt_map, base | 0x3C0u | ((cy >> 2) << 3) | (cx >> 2))];
    *pal_sel = (at >> (((cy & 2u) << 1) | (cx & 2u))) & 3u;
    const uint32_t pa = ((s.ctrl & 0x10u) << 8) + tile * 16u + fy;
    const uint32_t lo = chr_byte_pk(m, lo_pk, hi_pk, pa), hi = chr_byte_pk(m, lo_pk, hi_pk, pa + 8u);
    return ((lo >> (7u - bit)) & 1u) | (((hi >> (7u - bit)) & 1u) << 1);
}

__device__ inline uint32_t sprite_row_addr(uint32_t ctrl, uint32_t tile, uint32_t attr, uint32_t row) {
    const uint32_t h = (ctrl & 0x20u) ? 16u : 8u;
    if (attr & 0x80u) row = h - 1u - row;
    if (h == 8u) return ((ctrl & 0x08u) << 9) + tile * 16u + row;
    return ((tile & 1u) << 12) + (tile & 0xFEu) * 16u + (row & 7u) + ((row & 8u) << 1);
}

// MMC2: the pattern fetches of line l in order, each through the slot pages of the moment and then the latch hook
// (patch:1496-1560, 1660-1700): the sprites of line l, fetched at the end of line l - 1 (l >= 1), then, unless
// sprites_only, the line's 34 background tile slots. sink(kind, index, chr_lo, chr_hi, pa) gets the pages each
// fetch read through and its pattern address (kind 0: sprite rank, 1: tile slot). Fetches happen only while
// rendering is on. Wave-uniform.
template <class Sink>
__device__ __forceinline__ void rp_mmc2_line(Replay& s, const uint8_t* nt, const uint8_t* oam, int l, bool sprites_only,
                                    Sink&& sink) {
    if (s.mmc2_pages == 0 || (s.mask & 0x18u) == 0) return;
    if (l >= 1) {
        const int h = (s.ctrl & 0x20u) ? 16 : 8;
        uint32_t n = 0;
        for (uint32_t i = 0; i < 64u && n < 8u; ++i) {
            const int row = l - (int)oam[4u * i] - 1;
            if (row < 0 || row >= h) continue;
            const uint32_t pa = sprite_row_addr(s.ctrl, oam[4u * i + 1u], oam[4u * i + 2u], (uint32_t)row);
            sink(0u, n, s.chr_lo, s.chr_hi, pa);
            rp_hook(s, pa);
            ++n;
        }
    }
    if (sprites_only) return;
    const uint32_t cy = (s.v >> 5) & 31u, fy = (s.v >> 12) & 7u, ntv = (s.v >> 11) & 1u;
    for (uint32_t t = 0; t < 34u; ++t) {   // one tile right per slot, the nametable switching at each wrap
        const uint32_t cc = (s.v & 31u) + t, nth = ((s.v >> 10) & 1u) ^ ((cc >> 5) & 1u);
        const uint32_t base = 0x2000u | ((nth | (ntv << 1)) << 10);
        const uint32_t pa = ((s.ctrl & 0x10u) << 8) + nt[nt_index(s.nt_map, base | (cy << 5) | (cc & 31u))] * 16u + fy;
        sink(1u, t, s.chr_lo, s.chr_hi, pa);
        rp_hook(s, pa);
    }
}

// First sprite-0 hit of the logged frame on MMC2 (the scan below, with each line's fetches moving the latches):
// sprite 0 and the two tile slots under it read through the pages of their own fetches.
__device__ inline int32_t sprite0_scan_mmc2(const Mem m, uint32_t log_n) {
    const uint8_t* oam = m.oam;
    const int y0 = oam[0], x0 = oam[3];
    if (y0 >= 239) return (int32_t)kNoHit;
    const uint32_t tile = oam[1], attr = oam[2];
    Replay s;
    rp_begin(s, m.rec->log, log_n, nullptr, m.rec->log + NES_LOG_HDR_WORDS, m.cart.chr_pages1);
    for (int l = 0; l < 240; ++l) {
        const uint32_t slot_a = ((uint32_t)x0 + s.fx) >> 3;
        uint32_t s0lo = s.chr_lo, s0hi = s.chr_hi, alo = s.chr_lo, ahi = s.chr_hi, blo = s.chr_lo, bhi = s.chr_hi;
        rp_mmc2_line(s, m.nt, oam, l, false, [&](uint32_t kind, uint32_t i, uint32_t lo, uint32_t hi, uint32_t) {
            if (kind == 0u && i == 0u) { s0lo = lo; s0hi = hi; }
            if (kind == 1u && i == slot_a) { alo = lo; ahi = hi; }
            if (kind == 1u && i == slot_a + 1u) { blo = lo; bhi = hi; }
        });
        const int h = (s.ctrl & 0x20u) ? 16 : 8;
        const int row = l - y0 - 1;
        if ((s.mask & 0x18u) == 0x18u && row >= 0 && row < h) {
            const uint32_t pa = sprite_row_addr(s.ctrl, tile, attr, (uint32_t)row);
            const uint32_t lo = chr_byte_pk(m, s0lo, s0hi, pa), hi = chr_byte_pk(m, s0lo, s0hi, pa + 8u);
            for (int col = 0; col < 8; ++col) {
                const int x = x0 + col;
                if (x >= 255) break;
                if (x < 8 && (s.mask & 0x06u) != 0x06u) continue;
                const uint32_t b = (attr & 0x40u) ? (uint32_t)col : 7u - (uint32_t)col;
                if ((((lo >> b) & 1u) | ((hi >> b) & 1u)) == 0) continue;
                uint32_t ps;
                const bool in_a = (((uint32_t)x + s.fx) >> 3) == slot_a;
                if (rp_bg(s, m, (uint32_t)x, &ps, in_a ? alo : blo, in_a ? ahi : bhi)) return l * 341 + x + 1;
            }
        }
        if (l >= y0 + 16) break;
        rp_line_end(s, l, nullptr);
    }
    return (int32_t)kNoHit;
}

// First sprite-0 hit of the logged frame from the events logged so far (frame dot), kNoHit if none.
__device__ __forceinline__ int32_t sprite0_scan(const Mem m, uint32_t log_n) {
    if (m.cart.board == NES_BOARD_MMC2) return sprite0_scan_mmc2(m, log_n);
    const uint8_t* oam = m.oam;
    const int y0 = oam[0], x0 = oam[3];
    if (y0 >= 239) return (int32_t)kNoHit;
    const uint32_t tile = oam[1], attr = oam[2];
    Replay s;
    rp_begin(s, m.rec->log, log_n, nullptr, m.rec->log + NES_LOG_HDR_WORDS, 0u);
    for (int l = 0; l < 240; ++l) {
        const int h = (s.ctrl & 0x20u) ? 16 : 8;
        const int row = l - y0 - 1;
        if ((s.mask & 0x18u) == 0x18u && row >= 0 && row < h) {
            const uint32_t pa = sprite_row_addr(s.ctrl, tile, attr, (uint32_t)row);
            const uint32_t lo = chr_byte_pk(m, s.chr_lo, s.chr_hi, pa), hi = chr_byte_pk(m, s.chr_lo, s.chr_hi, pa + 8u);
            for (int col = 0; col < 8; ++col) {
                const int x = x0 + col;
                if (x >= 255) break;
                if (x < 8 && (s.mask & 0x06u) != 0x06u) continue;
                const uint32_t b = (attr & 0x40u) ? (uint32_t)col : 7u - (uint32_t)col;
                if ((((lo >> b) & 1u) | ((hi >> b) & 1u)) == 0) continue;
                uint32_t ps;
                if (rp_bg(s, m, (uint32_t)x, &ps, s.chr_lo, s.chr_hi)) return l * 341 + x + 1;
            }
        }
        if (l >= y0 + 16) break;
        rp_line_end(s, l, nullptr);
    }
    return (int32_t)kNoHit;
}

// ------------------------------------------------------------------------------------- PPU timing events
__device__ __forceinline__ uint64_t abs_dot(const Con& c) { return (uint64_t)c.frame * NES_FRAME_DOTS + c.frame_dot; }

__device__ inline void s0_refresh(Con& c, const Mem& m) {
    if (c.s0_valid || c.frame != c.log_frame) return;
    c.s0_valid = 1;
    c.s0_dot = (int32_t)kNoHit;
    if ((c.status & 0x40u) || c.frame_dot >= 240u * 341u) return;
    int32_t hit = sprite0_scan(m, c.log_n);
    if (hit != (int32_t)kNoHit && hit <= (int32_t)c.frame_dot) hit = (int32_t)c.frame_dot + 1;
    c.s0_dot = hit;
}

// Dots from the current frame dot to the next PPU event. Written as a search for the nearest absolute event dot
// (every candidate is compared, never subtracted, before the one final difference): the min-of-differences form
// `if (fd < E) best = min(best, E - fd)` is folded by the gfx950 compiler into an unguarded min, which returns 0 when
// fd == E and stalls ppu_advance.
__device__ inline uint32_t dots_to_event(Con& c, const Mem& m) {
    const uint32_t fd = c.frame_dot;
    uint32_t next = NES_FRAME_DOTS;
    if (fd < NES_PRERENDER_DOT) next = NES_PRERENDER_DOT;
    if (fd < NES_VBLANK_DOT) next = NES_VBLANK_DOT;
    if (m.cart.board == NES_BOARD_MMC3) {
        // clocks: dot 266 of lines 0..239, dot 256 of the pre-render line
        const uint32_t line = fd / 341u, d = fd - line * 341u;
        uint32_t clk = next;
        if (line < 239u) clk = d < 266u ? line * 341u + 266u : line * 341u + 341u + 266u;
        else if (line == 239u) clk = d < 266u ? line * 341u + 266u : 261u * 341u + 256u;
        else if (line < 261u || d < 256u) clk = 261u * 341u + 256u;
        if (clk > fd && clk < next) next = clk;
    }
    s0_refresh(c, m);
    if (c.frame == c.log_frame && c.s0_dot != (int32_t)kNoHit) {
        const uint32_t s0 = (uint32_t)c.s0_dot;
        if (s0 > fd && s0 < next) next = s0;
    }
    return next - fd;
}

__device__ inline void log_capture(Con& c, const Mem& m) {
    uint32_t* h = m.rec->log;
    const uint32_t* co = m.rec->chr_off;
    uint32_t p0 = 0, p1 = 0;
    for (uint32_t i = 0; i < 4; ++i) {
        p0 |= ((co[i] >> 10) & 0xFFu) << (8 * i);
        p1 |= ((co[4 + i] >> 10) & 0xFFu) << (8 * i);
    }
    const uint32_t* pal = reinterpret_cast<const uint32_t*>(m.pal);
    h[0] = 0;
    h[1] = c.ctrl | (c.mask << 8) | (c.fx << 16);
    h[2] = c.v | (c.t << 16);
    h[3] = p0;
    h[4] = p1;
    h[5] = c.nt_map;
    for (uint32_t i = 0; i < 8; ++i) h[6 + i] = pal[i];
    const uint8_t* r = m.rec->mreg;
    const bool mmc2 = m.cart.board == NES_BOARD_MMC2;
    h[14] = mmc2 ? (r[0] | ((uint32_t)r[1] << 8) | ((uint32_t)r[2] << 16) | ((uint32_t)r[3] << 24)) : 0u;
    h[15] = mmc2 ? (r[6] | ((uint32_t)r[7] << 8)) : 0u;
    c.log_n = 0;
    c.log_frame = c.frame + 1u;
    c.s0_valid = 0;
    c.s0_dot = (int32_t)kNoHit;
}

// MMC2 at vblank: the latches this frame's own fetches leave, from a latches-only replay of its log over the
// nametables and OAM as they are now (NeSLE's frame_resolve_mmc2, patch:1790-1812; rl/csrc/nes_machine.cuh:110-131
// runs the same replay after the vblank stop, before any further instruction). Every frame the kernels run ends at
// the vblank dot, so they call it at each frame's stop (the vblank just processed, no instruction after it).
__device__ inline void mmc2_resolve(NesRec* rec, const uint8_t* nt, const uint8_t* oam, uint32_t log_n,
                                    uint32_t chr_pages) {
    Replay s;
    rp_begin(s, rec->log, log_n, nullptr, rec->log + NES_LOG_HDR_WORDS, chr_pages);
    const auto none = [](uint32_t, uint32_t, uint32_t, uint32_t, uint32_t) {};
    for (int l = 0; l < 240; ++l) {
        rp_mmc2_line(s, nt, oam, l, false, none);
        rp_line_end(s, l, nullptr);
    }
    rp_mmc2_line(s, nt, oam, 240, true, none);
    rp_until(s, INT32_MAX, nullptr);
    const uint32_t l0 = s.latch & 1u, l1 = (s.latch >> 8) & 1u;
    rec->mreg[6] = (uint8_t)l0;
    rec->mreg[7] = (uint8_t)l1;
    for (uint32_t i = 0; i < 4; ++i) {   // the halves' pages, as the board's page sync sets them
        rec->chr_off[i] = ((4u * rec->mreg[l0] + i) & (chr_pages - 1u)) * 1024u;
        rec->chr_off[4u + i] = ((4u * rec->mreg[2u + l1] + i) & (chr_pages - 1u)) * 1024u;
    }
}

__device__ inline void process_events(Con& c, const Mem& m) {
    const uint32_t d = c.frame_dot;
    if (d == NES_FRAME_DOTS) {
        c.frame_dot = 0;
        ++c.frame;
        return;
    }
    if (d == NES_VBLANK_DOT) {
        c.status |= 0x80u;
        if (c.ctrl & 0x80u) c.nmi_pending = 1;
    }
    if (d == NES_PRERENDER_DOT) {
        c.status &= 0x1Fu;
        log_capture(c, m);
    }
    if (m.cart.board == NES_BOARD_MMC3 && (c.mask & 0x18u) &&
        ((d < 240u * 341u && d % 341u == 266u) || d == 261u * 341u + 256u))
        mmc3_clock(c, m);
    if (c.frame == c.log_frame && c.s0_dot != (int32_t)kNoHit && d == (uint32_t)c.s0_dot) {
        c.status |= 0x40u;
        c.s0_dot = (int32_t)kNoHit;
    }
}

__device__ inline void ppu_advance(Con& c, const Mem& m, uint32_t dots) {
    while (dots > 0) {
        const uint32_t to = dots_to_event(c, m);
        if (dots < to) {
            c.frame_dot += dots;
            return;
        }
        c.frame_dot += to;
        dots -= to;
        process_events(c, m);
    }
}

// ------------------------------------------------------------------------------------------------ bus
struct Access {
    int32_t ev_time;   // log time of this instruction's PPU accesses (its last cycle)
    bool log_on;       // the instruction started inside the log window
    bool dma;          // a $4014 write happened
};

__device__ inline void log_event(Con& c, const Mem& m, const Access& ac, uint32_t kind, uint32_t value, uint32_t aux) {
    if (kind != NES_EV_PAL) c.s0_valid = 0;
    if (!ac.log_on) return;
    uint32_t* h = m.rec->log;
    uint32_t* ev = h + NES_LOG_HDR_WORDS;
    if (kind == NES_EV_DATA && (c.mask & 0x18u) == 0 && c.log_n > 0) {
        uint32_t* last = ev + 2u * (c.log_n - 1u);
        if ((last[0] >> 24) == NES_EV_DATA && (last[1] >> 8) < 0xFFu) {
            last[1] += 0x100u;
            return;
        }
    }
    if (c.log_n >= NES_LOG_EVENTS) {
        h[0] |= NES_LOG_OVERFLOW;
        return;
    }
    ev[2u * c.log_n] = ((uint32_t)(ac.ev_time + NES_LOG_TIME_BIAS) & 0xFFFFFFu) | (kind << 24);
    ev[2u * c.log_n + 1u] = (value & 0xFFu) | ((aux & 0xFFu) << 8);
    ++c.log_n;
    h[0] = (h[0] & NES_LOG_OVERFLOW) | c.log_n;
}

__device__ inline uint32_t ppu_mem_read(const Con& c, const Mem& m, uint32_t a) {
    a &= 0x3FFFu;
    if (a < 0x2000u) return chr_byte(m, m.rec->chr_off, a);
    if (a < 0x3F00u) return m.nt[nt_index(c.nt_map, a)];
    uint32_t i = a & 0x1Fu;
    if ((i & 0x13u) == 0x10u) i &= 0x0Fu;
    return m.pal[i];
}

__device__ __forceinline__ uint32_t vinc(const Con& c) { return (c.ctrl & 4u) ? 32u : 1u; }

// MMC2: the VRAM address the CPU drives through $2006/$2007 flips a latch; a change is logged for the renderer
// (patch:615-636, 3196-3220).
__device__ inline void mmc2_ppu_address(Con& c, const Mem& m, const Access& ac, uint32_t a) {
    const uint32_t t = m.cart.board == NES_BOARD_MMC2 ? mmc2_trigger(a) : 0u;
    if (t == 0) return;
    const uint32_t half = t >> 2, latch = (t & 3u) - 1u;
    uint8_t* r = m.rec->mreg;
    if (r[6 + half] == latch) return;
    r[6 + half] = (uint8_t)latch;
    for (uint32_t i = 0; i < 4; ++i) map_set_chr(m, 4u * half + i, 4u * r[2u * half + latch] + i);   // the half's pages
    log_event(c, m, ac, NES_EV_MMC2, latch, 6 + half);
}

__device__ inline uint32_t io_read(Con& c, const Mem& m, const Access& ac, uint32_t a) {
    if (a < 0x4000u) {
        const uint32_t reg = a & 7u;
        uint32_t v;
        if (reg == 2) {
            v = (c.status & 0xE0u) | (c.open_bus & 0x1Fu);
            c.status &= 0x7Fu;
            c.w = 0;
        } else if (reg == 4) {
            v = m.oam[c.oam_addr];
        } else if (reg == 7) {
            const uint32_t pa = c.v & 0x3FFFu;
            if (pa < 0x3F00u) {
                v = c.read_buf;
                mmc2_ppu_address(c, m, ac, pa);
                c.read_buf = ppu_mem_read(c, m, pa);
            } else {
                v = ppu_mem_read(c, m, pa);
                c.read_buf = ppu_mem_read(c, m, pa - 0x1000u);
                mmc2_ppu_address(c, m, ac, pa);
            }
            c.v = (c.v + vinc(c)) & 0x7FFFu;
            log_event(c, m, ac, NES_EV_DATA, 0, 1);
            mmc2_ppu_address(c, m, ac, c.v & 0x3FFFu);
        } else {
            return c.open_bus;
        }
        c.open_bus = v;
        return v;
    }
    if (a == 0x4015u) return m.rec->dmc_left ? 0x10u : 0u;
    if (a == 0x4016u) {
        uint32_t bit;
        if (c.strobe) {
            bit = c.pad & 1u;
        } else {
            bit = c.shift & 1u;
            c.shift = (c.shift >> 1) | 0x80u;
        }
        return 0x40u | bit;
    }
    if (a >= 0x6000u) return prg_ram_on(m) ? m.rec->prg_ram[a - 0x6000u] : (a >> 8);
    return a >> 8;
}

__device__ __forceinline__ uint32_t bus_read(Con& c, const Mem& m, const Access& ac, uint32_t a) {
    if (a < 0x2000u) return m.ram[a & 0x7FFu];
    if (a >= 0x8000u) return prg_byte(c, m, a);
    return io_read(c, m, ac, a);
}

__device__ inline void io_write(Con& c, const Mem& m, Access& ac, uint32_t a, uint32_t v);

__device__ __forceinline__ void bus_write(Con& c, const Mem& m, Access& ac, uint32_t a, uint32_t v) {
    if (a < 0x2000u) m.ram[a & 0x7FFu] = (uint8_t)v;
    else io_write(c, m, ac, a, v);
}

__device__ inline void ppu_reg_write(Con& c, const Mem& m, const Access& ac, uint32_t reg, uint32_t v) {
    c.open_bus = v;
    if (reg == 0) {
        if (!(c.ctrl & 0x80u) && (v & 0x80u) && (c.status & 0x80u)) c.nmi_pending = 1;
        c.ctrl = v;
        c.t = (c.t & 0xF3FFu) | ((v & 3u) << 10);
        log_event(c, m, ac, NES_EV_CTRL, v, 0);
    } else if (reg == 1) {
        c.mask = v;
        log_event(c, m, ac, NES_EV_MASK, v, 0);
    } else if (reg == 3) {
        c.oam_addr = v;
    } else if (reg == 4) {
        m.oam[c.oam_addr] = (uint8_t)v;
        c.oam_addr = (c.oam_addr + 1u) & 0xFFu;
        c.s0_valid = 0;
    } else if (reg == 5) {
        log_event(c, m, ac, NES_EV_SCROLL, v, c.w);
        if (c.w == 0) {
            c.t = (c.t & 0xFFE0u) | (v >> 3);
            c.fx = v & 7u;
            c.w = 1;
        } else {
            c.t = (c.t & 0x0C1Fu) | ((v & 7u) << 12) | ((v & 0xF8u) << 2);
            c.w = 0;
        }
    } else if (reg == 6) {
        log_event(c, m, ac, NES_EV_ADDR, v, c.w);
        if (c.w == 0) {
            c.t = (c.t & 0x00FFu) | ((v & 0x3Fu) << 8);
            c.w = 1;
        } else {
            c.t = (c.t & 0xFF00u) | v;
            c.v = c.t;
            c.w = 0;
            mmc2_ppu_address(c, m, ac, c.v);
        }
    } else if (reg == 7) {
        const uint32_t pa = c.v & 0x3FFFu;
        if (pa < 0x2000u) {
            if (!m.cart.chr) {
                m.rec->chr_ram[(m.rec->chr_off[(pa >> 10) & 7u] + (pa & 0x3FFu)) & (NES_CHRRAM_BYTES - 1u)] = (uint8_t)v;
                c.s0_valid = 0;
            }
            log_event(c, m, ac, NES_EV_DATA, 0, 1);
        } else if (pa < 0x3F00u) {
            m.nt[nt_index(c.nt_map, pa)] = (uint8_t)v;
            log_event(c, m, ac, NES_EV_DATA, 0, 1);
        } else {
            uint32_t i = pa & 0x1Fu;
            if ((i & 0x13u) == 0x10u) i &= 0x0Fu;
            m.pal[i] = (uint8_t)(v & 0x3Fu);
            log_event(c, m, ac, NES_EV_PAL, v & 0x3Fu, i);
        }
        c.v = (c.v + vinc(c)) & 0x7FFFu;
        mmc2_ppu_address(c, m, ac, c.v & 0x3FFFu);
    }
}

__device__ inline void io_write(Con& c, const Mem& m, Access& ac, uint32_t a, uint32_t v) {
    if (a < 0x4000u) {
        ppu_reg_write(c, m, ac, a & 7u, v);
    } else if (a == 0x4014u) {
        // OAM DMA: 256 bytes of CPU page v through the bus (normally RAM in LDS)
        uint8_t* oam = m.oam;
        for (uint32_t i = 0; i < 256u; ++i) {
            const uint32_t src = (v << 8) | i;
            const uint32_t b = src < 0x2000u ? m.ram[src & 0x7FFu] : bus_read(c, m, ac, src);
            oam[(c.oam_addr + i) & 0xFFu] = (uint8_t)b;
        }
        c.s0_valid = 0;
        ac.dma = true;
    } else if (a == 0x4016u) {
        c.strobe = v & 1u;
        if (c.strobe) c.shift = c.pad;
    } else if (a == 0x4010u || a == 0x4013u || a == 0x4015u) {
        NesRec* r = m.rec;
        if (a == 0x4010u) r->dmc_control = (uint8_t)v;
        else if (a == 0x4013u) r->dmc_length = (uint8_t)v;
        else if ((v & 0x10u) == 0) r->dmc_left = 0;
        else if (r->dmc_left == 0) r->dmc_left = (uint16_t)(r->dmc_length * 16u + 1u);
        c.dmc_event = 0;
    } else if (a >= 0x8000u) {
        if (m.cart.board == NES_BOARD_NROM) return;
        uint32_t before[8];
        const uint32_t* co = m.rec->chr_off;
        for (uint32_t i = 0; i < 8; ++i) before[i] = co[i];
        const uint32_t map_before = c.nt_map;
        const uint32_t creg_before = *reinterpret_cast<const uint32_t*>(m.rec->mreg);
        map_write(c, m, a, v);
        for (uint32_t i = 0; i < 8; ++i)
            if (co[i] != before[i]) log_event(c, m, ac, NES_EV_CHR, co[i] >> 10, i);
        if (c.nt_map != map_before) log_event(c, m, ac, NES_EV_MIRROR, c.nt_map, 0);
        if (m.cart.board == NES_BOARD_MMC2)   // patch:661-664
            for (uint32_t i = 0; i < 4; ++i) {
                const uint32_t now = m.rec->mreg[i];
                if (now != ((creg_before >> (8u * i)) & 0xFFu)) log_event(c, m, ac, NES_EV_MMC2, now, i);
            }
    } else if (a >= 0x6000u) {
        if (prg_ram_on(m)) m.rec->prg_ram[a - 0x6000u] = (uint8_t)v;
    }
}

// Instruction-stream bytes without side effects (RAM, PRG RAM, PRG; open bus elsewhere).
__device__ inline uint32_t fetch_slow(const Con& c, const Mem& m, uint32_t a) {
    a &= 0xFFFFu;
    if (a < 0x2000u) return m.ram[a & 0x7FFu];
    if (a >= 0x8000u) return prg_byte(c, m, a);
    if (a >= 0x6000u && prg_ram_on(m)) return m.rec->prg_ram[a - 0x6000u];
    return a >> 8;
}

// ------------------------------------------------------------------------------------------------ 6502
__device__ __forceinline__ void set_nz(Con& c, uint32_t v) {
    c.p = (c.p & ~(FL_N | FL_Z)) | (v & 0x80u) | ((v & 0xFFu) ? 0u : FL_Z);
}
__device__ __forceinline__ void push8(Con& c, const Mem& m, uint32_t v) {
    m.ram[0x100u | c.sp] = (uint8_t)v;
    c.sp = (c.sp - 1u) & 0xFFu;
}
__device__ __forceinline__ uint32_t pull8(Con& c, const Mem& m) {
    c.sp = (c.sp + 1u) & 0xFFu;
    return m.ram[0x100u | c.sp];
}
__device__ __forceinline__ uint32_t reg_get(const Con& c, uint32_t code, uint32_t opd) {
    return code == R_A ? c.a : code == R_X ? c.x : code == R_Y ? c.y : code == R_SP ? c.sp : opd;
}
__device__ __forceinline__ void reg_set(Con& c, uint32_t code, uint32_t v) {
    if (code == R_A) c.a = v;
    else if (code == R_X) c.x = v;
    else if (code == R_Y) c.y = v;
    else if (code == R_SP) c.sp = v;
}

__device__ inline void interrupt(Con& c, const Mem& m, uint32_t vector) {
    push8(c, m, c.pc >> 8);
    push8(c, m, c.pc & 0xFFu);
    push8(c, m, (c.p & ~FL_B) | FL_U);
    c.p |= FL_I;
    c.pc = fetch_slow(c, m, vector) | (fetch_slow(c, m, vector + 1u) << 8);
}

// One step: a pending NMI (or the asserted cartridge IRQ with I clear), then one instruction, the OAM-DMA stall and
// the DMC service. `start_rel` = log time of the step's first dot. Returns the CPU cycles, 0 with *fault set.
__device__ inline uint32_t cpu_step(Con& c, const Mem& m, const uint32_t* optab, int32_t start_rel, uint32_t* fault,
                                    uint32_t* op_out, uint32_t* pc_out) {
    uint32_t cyc = 0;
    if (c.nmi_pending) {
        c.nmi_pending = 0;
        interrupt(c, m, 0xFFFAu);
        cyc = 7;
    } else if (c.irq_line && !(c.p & FL_I)) {
        interrupt(c, m, 0xFFFEu);
        cyc = 7;
    }
    const int32_t rel = start_rel + 3 * (int32_t)cyc;
    Access ac;
    ac.log_on = rel >= -340 && rel < (int32_t)NES_VBLANK_DOT;
    ac.dma = false;
    // fetch opcode + operands
    const uint32_t pc = c.pc;
    uint32_t word;
    if (pc >= 0x8000u && (pc & 0x1FFFu) <= 0x1FFDu) {
        word = m.cart.prgw[prg_off(c, pc) + (pc & 0x1FFFu)];
    } else {
        word = fetch_slow(c, m, pc) | (fetch_slow(c, m, pc + 1u) << 8) | (fetch_slow(c, m, pc + 2u) << 16);
    }
    const uint32_t op = word & 0xFFu, lo = (word >> 8) & 0xFFu, hi = (word >> 16) & 0xFFu;
    *op_out = op;
    *pc_out = pc;
    const uint32_t d = optab[op];
    const uint32_t mode = d & 15u, grp = (d >> 8) & 15u, sub = (d >> 12) & 15u;
    const uint32_t src = (d >> 16) & 7u, dst = (d >> 19) & 7u;
    uint32_t icyc = (d >> 4) & 15u;
    if (grp == G_ILL) {
        *fault = (pc << 8) | op;
        return 0;
    }
    // effective address
    uint32_t base = lo | (hi << 8), idx = 0;
    if (mode == M_ZPX || mode == M_ABX) idx = c.x;
    else if (mode == M_ZPY || mode == M_ABY) idx = c.y;
    if (mode == M_IZX || mode == M_IZY) {
        const uint32_t ptr = mode == M_IZX ? ((lo + c.x) & 0xFFu) : lo;
        base = m.ram[ptr] | ((uint32_t)m.ram[(ptr + 1u) & 0xFFu] << 8);
        idx = mode == M_IZY ? c.y : 0u;
    }
    uint32_t ea;
    if (mode == M_ZP || mode == M_ZPX || mode == M_ZPY) {
        ea = (lo + idx) & 0xFFu;
    } else {
        ea = (base + idx) & 0xFFFFu;
        if ((d & D_PEN) && ((base ^ ea) & 0xFF00u)) ++icyc;
    }
    ac.ev_time = rel + 3 * (int32_t)icyc;
    uint32_t opd = lo;
    if (d & D_READ) opd = bus_read(c, m, ac, ea);
    uint32_t res = 0, npc = (pc + (mode == M_IMP ? 1u : (mode >= M_ABS && mode <= M_ABY) || mode == M_IND ? 3u : 2u)) & 0xFFFFu;
    switch (grp) {
        case G_LD: {   // LDA LDX LDY, TAX TAY TXA TYA TSX TXS
            res = reg_get(c, src, opd);
            reg_set(c, dst, res);
            if (dst != R_SP) set_nz(c, res);
            break;
        }
        case G_ST: res = reg_get(c, src, 0); break;
        case G_INCDEC: {   // sub 0 = +1, 1 = -1; src/dst a register, or the operand (memory)
            res = (reg_get(c, src, opd) + (sub ? 0xFFu : 1u)) & 0xFFu;
            reg_set(c, dst, res);
            set_nz(c, res);
            break;
        }
        case G_ALU: {   // sub: 0 ORA 1 AND 2 EOR 3 ADC 4 SBC 5 CMP(src) 6 BIT
            if (sub <= 2) {
                c.a = sub == 0 ? (c.a | opd) : sub == 1 ? (c.a & opd) : (c.a ^ opd);
                set_nz(c, c.a);
            } else if (sub <= 4) {
                const uint32_t mv = sub == 4 ? (opd ^ 0xFFu) : opd;
                const uint32_t sum = c.a + mv + (c.p & FL_C);
                const uint32_t ov = (~(c.a ^ mv) & (c.a ^ sum) & 0x80u) ? FL_V : 0u;
                c.p = (c.p & ~(FL_C | FL_V)) | (sum >> 8) | ov;
                c.a = sum & 0xFFu;
                set_nz(c, c.a);
            } else if (sub == 5) {
                const uint32_t r = reg_get(c, src, 0);
                c.p = (c.p & ~FL_C) | (r >= opd ? FL_C : 0u);
                set_nz(c, (r - opd) & 0xFFu);
            } else {
                c.p = (c.p & ~(FL_N | FL_V | FL_Z)) | (opd & 0xC0u) | ((c.a & opd) ? 0u : FL_Z);
            }
            break;
        }
        case G_SHIFT: {   // sub: 0 ASL 1 LSR 2 ROL 3 ROR; src/dst A or the operand
            const uint32_t in = reg_get(c, src, opd), cin = c.p & FL_C;
            uint32_t cout;
            if (sub == 0) { res = (in << 1) & 0xFFu; cout = in >> 7; }
            else if (sub == 1) { res = in >> 1; cout = in & 1u; }
            else if (sub == 2) { res = ((in << 1) | cin) & 0xFFu; cout = in >> 7; }
            else { res = (in >> 1) | (cin << 7); cout = in & 1u; }
            c.p = (c.p & ~FL_C) | cout;
            reg_set(c, dst, res);
            set_nz(c, res);
            break;
        }
        case G_BR: {   // sub: flag bit index (0 C, 1 Z, 6 V, 7 N) in bits 0-2, want-set in bit 3
            const bool set = ((c.p >> (sub & 7u)) & 1u) != 0;
            if (set == ((sub & 8u) != 0)) {
                const uint32_t target = (npc + (uint32_t)(int32_t)(int8_t)lo) & 0xFFFFu;
                icyc += ((npc ^ target) & 0xFF00u) ? 2u : 1u;
                npc = target;
            }
            break;
        }
        case G_FLAG: {   // sub: bit index in bits 0-2, set in bit 3
            const uint32_t bitm = 1u << (sub & 7u);
            c.p = (sub & 8u) ? (c.p | bitm) : (c.p & ~bitm);
            break;
        }
        case G_PUSH: push8(c, m, src == R_A ? c.a : (c.p | FL_B | FL_U)); break;
        case G_PULL: {
            const uint32_t v = pull8(c, m);
            if (dst == R_A) {
                c.a = v;
                set_nz(c, v);
            } else {
                c.p = (v & ~FL_B) | FL_U;
            }
            break;
        }
        case G_JMP: {
            if (mode == M_IND) {
                const uint32_t l8 = bus_read(c, m, ac, base);
                const uint32_t h8 = bus_read(c, m, ac, (base & 0xFF00u) | ((base + 1u) & 0xFFu));
                npc = l8 | (h8 << 8);
            } else {
                npc = base;
            }
            break;
        }
        case G_JSR: {
            const uint32_t ret = (pc + 2u) & 0xFFFFu;
            push8(c, m, ret >> 8);
            push8(c, m, ret & 0xFFu);
            npc = base;
            break;
        }
        case G_RTS: {
            const uint32_t l8 = pull8(c, m), h8 = pull8(c, m);
            npc = (((h8 << 8) | l8) + 1u) & 0xFFFFu;
            break;
        }
        case G_RTI: {
            c.p = (pull8(c, m) & ~FL_B) | FL_U;
            const uint32_t l8 = pull8(c, m), h8 = pull8(c, m);
            npc = (h8 << 8) | l8;
            break;
        }
        case G_BRK: {
            const uint32_t ret = (pc + 2u) & 0xFFFFu;
            push8(c, m, ret >> 8);
            push8(c, m, ret & 0xFFu);
            push8(c, m, c.p | FL_B | FL_U);
            c.p |= FL_I;
            npc = fetch_slow(c, m, 0xFFFEu) | (fetch_slow(c, m, 0xFFFFu) << 8);
            break;
        }
        default: break;   // G_NOP
    }
    if (d & D_WRITE) bus_write(c, m, ac, ea, res);
    c.pc = npc;
    cyc += icyc;
    c.cycles += cyc;
    if (ac.dma) {
        const uint32_t stall = 513u + (uint32_t)(c.cycles & 1u);
        c.cycles += stall;
        cyc += stall;
    }
    if (c.cycles >= c.dmc_event) {
        const uint32_t s = dmc_service(m.rec, c.cycles, 1);
        c.dmc_event = m.rec->dmc_event;
        c.cycles += s;
        cyc += s;
    }
    return cyc;
}

// Skip whole 3-cycle jumps of a JMP-to-self idle loop up to the next PPU event; not while an interrupt waits.
__device__ inline void fast_forward(Con& c, const Mem& m) {
    if (c.nmi_pending || (c.irq_line && !(c.p & FL_I))) return;
    const uint32_t to = dots_to_event(c, m);
    const uint32_t jumps = (to + 8u) / 9u;
    if (jumps == 0) return;
    c.cycles += 3u * jumps;
    if (c.cycles >= c.dmc_event) {
        (void)dmc_service(m.rec, c.cycles, 0);
        c.dmc_event = m.rec->dmc_event;
    }
    ppu_advance(c, m, 9u * jumps);
}

// Runs the console until the PPU reaches absolute dot `target` (rl/csrc/nes_machine.cuh:67-103). Returns the fault.
__device__ inline uint32_t run_until(Con& c, const Mem& m, const uint32_t* optab, uint64_t target,
                                     uint32_t budget = NES_BUDGET) {
    uint32_t instructions = 0, fault = 0, pending = 0;
    uint32_t to_event = dots_to_event(c, m);
    while (instructions < budget) {
        if (pending >= to_event) {
            ppu_advance(c, m, pending);
            pending = 0;
            if (abs_dot(c) >= target) break;
            to_event = dots_to_event(c, m);
        }
        const int32_t start_rel =
            (int32_t)((int64_t)abs_dot(c) + pending - (int64_t)c.log_frame * NES_FRAME_DOTS);
        uint32_t op, pc0;
        const uint32_t cyc = cpu_step(c, m, optab, start_rel, &fault, &op, &pc0);
        if (fault) break;
        pending += 3u * cyc;
        ++instructions;
        ++c.instr;
        if (!c.s0_valid) to_event = dots_to_event(c, m);
        if (op == 0x4Cu && c.pc == pc0) {
            ppu_advance(c, m, pending);
            pending = 0;
            if (abs_dot(c) >= target) break;
            fast_forward(c, m);
            to_event = dots_to_event(c, m);
            if (abs_dot(c) >= target) break;
        }
    }
    if (pending) ppu_advance(c, m, pending);
    return fault;
}

// Power-on of one console record: cold reset, RAM 0xFF, frame 0's log from the power-on PPU state.
__device__ inline void power_on(NesRec* rec, const Cart& cart) {
    // zero through a character type: typed field stores below may not be reordered before it
    uint8_t* bytes = reinterpret_cast<uint8_t*>(rec);
    for (uint32_t i = 0; i < NES_REC_BYTES; ++i) bytes[i] = 0;
    rec->board = (uint8_t)cart.board;
    Con c = {};
    const Mem m = mem_of(rec, nullptr, cart);
    uint8_t* r = rec->mreg;
    if (cart.board == NES_BOARD_MMC1) {
        r[0] = 0x0C;
    } else if (cart.board == NES_BOARD_MMC3) {
        r[1] = 2; r[2] = 4; r[3] = 5; r[4] = 6; r[5] = 7; r[7] = 1;
        r[9] = cart.mirroring ? 0 : 1;
    } else if (cart.board == NES_BOARD_MMC2) {
        r[6] = 1;   // both latches on the $FE bank (patch:3080-3083)
        r[7] = 1;
    }
    map_sync(c, m);
    for (uint32_t i = 0; i < NES_RAM_BYTES; ++i) rec->ram[i] = 0xFF;
    rec->sp = 0xFD;
    rec->p = FL_I | FL_U;
    const uint32_t vec = rec->prg_off[3] + 0x1FFCu;
    rec->pc = (uint16_t)((cart.prgw[vec] & 0xFFu) | ((cart.prgw[vec + 1] & 0xFFu) << 8));
    rec->cycles = 7;
    rec->s0_dot = (int32_t)kNoHit;
    rec->s0_valid = 0;
    rec->dmc_byte_end = 7u + 1u + 7u * 428u;
    rec->dmc_event = kDmcIdle;
    uint32_t* h = rec->log;
    for (uint32_t i = 0; i < 4; ++i) {
        h[3] |= ((rec->chr_off[i] >> 10) & 0xFFu) << (8 * i);
        h[4] |= ((rec->chr_off[4 + i] >> 10) & 0xFFu) << (8 * i);
    }
    h[5] = c.nt_map;
    rec->log_frame = 0;
}

// ------------------------------------------------------------------------------------ record <-> lane
__device__ inline void con_load(Con& c, const NesRec* r) {
    c.pc = r->pc; c.a = r->a; c.x = r->x; c.y = r->y; c.sp = r->sp; c.p = r->p;
    c.irq_line = r->irq_line; c.nmi_pending = r->nmi_pending; c.cycles = r->cycles;
    c.pad = r->pad; c.shift = r->shift; c.strobe = r->strobe; c.instr = r->instr_lo;
    c.frame_dot = r->frame_dot; c.frame = r->frame;
    c.v = r->v; c.t = r->t; c.ctrl = r->ctrl; c.mask = r->mask; c.status = r->status; c.oam_addr = r->oam_addr;
    c.fx = r->fx; c.w = r->w; c.read_buf = r->read_buf; c.open_bus = r->open_bus;
    c.s0_dot = r->s0_dot; c.log_frame = r->log_frame; c.log_n = r->log_n; c.s0_valid = r->s0_valid;
    c.dmc_event = r->dmc_event;
    c.prg0 = r->prg_off[0]; c.prg1 = r->prg_off[1]; c.prg2 = r->prg_off[2]; c.prg3 = r->prg_off[3];
    c.nt_map = r->nt_map[0] | (r->nt_map[1] << 2) | (r->nt_map[2] << 4) | ((uint32_t)r->nt_map[3] << 6);
}

__device__ inline void con_store(const Con& c, NesRec* r) {
    r->pc = (uint16_t)c.pc; r->a = (uint8_t)c.a; r->x = (uint8_t)c.x; r->y = (uint8_t)c.y; r->sp = (uint8_t)c.sp;
    r->p = (uint8_t)c.p; r->irq_line = (uint8_t)c.irq_line; r->nmi_pending = (uint8_t)c.nmi_pending;
    r->cycles = c.cycles; r->pad = (uint8_t)c.pad; r->shift = (uint8_t)c.shift; r->strobe = (uint8_t)c.strobe;
    r->instr_lo = c.instr; r->frame_dot = c.frame_dot; r->frame = c.frame;
    r->v = (uint16_t)c.v; r->t = (uint16_t)c.t; r->ctrl = (uint8_t)c.ctrl; r->mask = (uint8_t)c.mask;
    r->status = (uint8_t)c.status; r->oam_addr = (uint8_t)c.oam_addr; r->fx = (uint8_t)c.fx; r->w = (uint8_t)c.w;
    r->read_buf = (uint8_t)c.read_buf; r->open_bus = (uint8_t)c.open_bus;
    r->s0_dot = c.s0_dot; r->log_frame = c.log_frame; r->log_n = (uint16_t)c.log_n; r->s0_valid = (uint8_t)c.s0_valid;
    r->dmc_event = c.dmc_event;
    // prg_off and nt_map are written through to the record whenever they change (map_set_*)
}

}  // namespace nd
