// Device-side NES console for gfx950, one console per wavefront: its registers wave-uniform (scalar registers), its
// 2 KB CPU RAM, nametables, OAM and palette in the wave's LDS, everything else in the console record in HBM
// (include/nesrec.h). This file holds the console's generic step and what the fast paths share with it: the bus, the
// PPU's timing events and frame log, the mappers and the DMC (the fast paths: wave_dev.h, jit.h).
//
// The generic 6502 step is table-driven: one 32-bit descriptor per opcode (addressing mode, cycles, operation group
// and its parameters, read/write/penalty flags) in constant memory, read through the scalar cache. Every instruction
// runs the same fetch -> effective address -> bus read -> group -> bus write sequence. Instruction fetch is one
// 32-bit load from a widened PRG image (word i holds PRG bytes i, i+1, i+2), so the opcode and both operand bytes
// arrive in one memory access.
//
// Semantics are those of the reference env's NES machine (kdcyberdude/ghostrun-lab): frame loop
// rl/csrc/nes_machine.cuh:67-103, instruction step third_party/nesle-extensions.patch:823-862, bus side effects
// patch:570-779, PPU events patch:1822-2240, frame log patch:894-1185, mappers patch:2841-3367, DMC patch:430-565.
#pragma once
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#ifndef ND_HOST_BUILD
#include <hip/hip_runtime.h>
#endif
#include <stdint.h>
#endif

#include "nesrec.h"
#include "replay_dev.h"

namespace nd {

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
    uint32_t s0_sched;
    uint32_t log_frame, log_n, log_flags;
    uint64_t dmc_event;
    uint32_t prg0, prg1, prg2, prg3;   // PRG byte offsets of $8000/$A000/$C000/$E000
    uint32_t nt_map;                   // 4 x 2 bits
    uint32_t map_fast;                 // what the fast path's mapper writes decide on (wave_dev.h map_write_ok), as
                                       // in the record's mreg: MMC3 the bank select, MMC1 the shift register | count << 8
    // wave_dev.h run_until_wave's own state, parked here while a burst of fast instructions runs; b_quiet: the burst
    // starts between vblank and the pre-render line (wave_dev.h ppu_write_quiet)
    uint64_t b_dmc_event, b_target;
    uint32_t b_instructions, b_pending, b_to_event, b_ecyc, b_dmc_in, b_why, b_budget, b_nmi, b_irq, b_quiet;
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
    // CHR ROM again with each tile row's two plane bytes side by side (16-bit word page * 512 + (a & $3F0) / 2 +
    // (a & 7) holds the bytes at a and a + 8), for the renderer's one-load pattern fetch; nullptr = CHR RAM
    const uint16_t* chr_pairs;
};

// Instruction-fetch table (fast path): entry = {dispatch key, operand word}, two dwords: the opcode, or its hot key
// for the opcodes of kHotOps, and the decoded operand. NROM and CNROM (fixed PRG): entry a for CPU address a, for
// $8000 <= a <= $FFFD; every other entry (RAM, I/O, the last two bytes, and a pc just past $FFFF) holds opcode $02,
// which no fast-path handler runs, so the generic step fetches it. Banked boards: one entry per PRG byte offset, $02
// where the instruction would end on the last byte of its 8 KB page or beyond it, so that every instruction the
// fast path runs leaves the next pc on the same page (the next CPU page may map another bank).
constexpr uint32_t kFetchWords = 0x10100u;

// Bytes of an instruction of addressing mode `mode`.
constexpr uint32_t instr_len(uint32_t mode) {
    return mode == M_IMP ? 1u : ((mode >= M_ABS && mode <= M_ABY) || mode == M_IND) ? 3u : 2u;
}

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
constexpr uint32_t kBlockKey = 0x200u;   // translated blocks (jit.h): keys kBlockKey + block index
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
    uint32_t* scratch;      // 34 words of LDS for the sprite-0 check's MMC2 pages
};

// The memories of a console record, with the CPU RAM at `ram`.
__device__ __forceinline__ Mem mem_of(NesRec* rec, uint8_t* ram, const Cart& cart) {
    return Mem{rec, ram, rec->nt, rec->oam, rec->pal, cart, nullptr};
}

// One of four wave-uniform values by index i (0-3), as one scalar sequence. Written as C (nested selects), the
// compiler splits it into a branch on bit 1 and an s_cselect on bit 0 at the join, with SCC live across the branch;
// in a kernel large enough that the branch is relaxed into an s_getpc / s_add_u32 / s_addc_u32 / s_setpc jump, the
// jump's adds overwrite SCC and the join selects the wrong value (seen in translated kernels of banked carts: a read
// of $8000-$9FFF through the $A000 window). Here SCC lives only inside the statement. A constant index folds. The
// operands are scalar registers: wave-uniform values, read from LDS through uni() where they come from there.
__device__ __forceinline__ uint32_t sel4(uint32_t i, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    if (__builtin_constant_p(i)) return i & 2u ? (i & 1u ? d : c) : (i & 1u ? b : a);
    uint32_t r, t;
    asm("s_bitcmp1_b32 %2, 0\n\t"
        "s_cselect_b32 %0, %4, %3\n\t"
        "s_cselect_b32 %1, %6, %5\n\t"
        "s_bitcmp1_b32 %2, 1\n\t"
        "s_cselect_b32 %0, %1, %0"
        : "=&s"(r), "=&s"(t)
        : "s"(i), "s"(a), "s"(b), "s"(c), "s"(d)
        : "scc");
    return r;
}
__device__ __forceinline__ uint32_t prg_off(const Con& c, uint32_t addr) {
    return sel4(uni((addr >> 13) & 3u), uni(c.prg0), uni(c.prg1), uni(c.prg2), uni(c.prg3));
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
                c.map_fast = r[4] | ((n + 1u) << 8);
                return;
            }
            r[(addr >> 13) & 3u] = r[4];
            r[4] = 0;
            r[5] = 0;
        }
        c.map_fast = 0;
        map_sync(c, m);
    } else if (m.cart.board == NES_BOARD_MMC3) {
        const uint32_t k = addr & 0xE001u;
        if (k == 0x8000u) r[8] = (uint8_t)(c.map_fast = v);
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

// The MMC3 scanline counter (patch:1881-1903): a clock reloads the counter from the latch when it is 0 or a reload
// was asked for ($C001), else decrements it, and raises the IRQ line when it is then 0 with the IRQ enabled. Registers:
// mreg[11] latch, [12] counter, [13] IRQ enabled, [14] reload asked for.
//
// The counter of n >= 1 clocks in closed form: the first clock leaves c1 (the latch after a reload or from 0, else the
// counter less one); the counter then counts down to 0, which it reaches at clock c1 + 1, and runs the cycle latch,
// latch - 1, ..., 0 of latch + 1 clocks from there. *zero: whether some clock of the n left it at 0 (the IRQ).
__host__ __device__ __forceinline__ uint32_t mmc3_after_clocks(uint32_t cnt, uint32_t reload, uint32_t latch,
                                                                 uint32_t n, bool* zero) {
    const uint32_t c1 = (cnt == 0u || reload != 0u) ? latch : cnt - 1u;
    *zero = n >= c1 + 1u;
    if (n - 1u <= c1) return c1 - (n - 1u);
    return latch - (n - 2u - c1) % (latch + 1u);
}

// MMC3 clock dots of one frame: lines 0-239 at dot 266, the pre-render line (261) at dot 256. The number of them at
// frame dots <= x (x < NES_FRAME_DOTS, the dots of a frame that is not short).
__host__ __device__ __forceinline__ uint32_t mmc3_clocks_upto(uint32_t x) {
    const uint32_t line = x / 341u, d = x - line * 341u;
    if (line < 240u) return line + (d >= 266u ? 1u : 0u);
    if (line < 261u) return 240u;
    return 240u + (d >= 256u ? 1u : 0u);
}

// The clocks of the dots (start, end] (ppu_step's dots: the skipped last dot of a short frame counted) at once. The
// device settles the PPU lazily (dots_to_event), so a span holds many clocks; nothing reads the counter between them,
// and what decides them - the mask, the control register and the board's IRQ registers - changes only in the generic
// step, before which wave_dev.h settles, so applying them together leaves the state of applying them one by one.
__device__ inline void mmc3_clock_span(Con& c, const Mem& m, uint32_t start, uint32_t end) {
    const uint32_t n = (end / NES_FRAME_DOTS) * 241u + mmc3_clocks_upto(end % NES_FRAME_DOTS) -
                       (start / NES_FRAME_DOTS) * 241u - mmc3_clocks_upto(start % NES_FRAME_DOTS);
    if (n == 0u) return;
    uint8_t* r = m.rec->mreg;
    bool zero = false;
    r[12] = (uint8_t)mmc3_after_clocks(r[12], r[14], r[11], n, &zero);
    r[14] = 0;
    if (zero && r[13] != 0) c.irq_line = 1;
}

// The frame dot of the clock that will raise the IRQ line, if it comes in this frame after frame dot `cur` (clocks
// on, IRQ enabled, the line not already raised), else NES_FRAME_DOTS.
__device__ __forceinline__ uint32_t mmc3_irq_dot(const Con& c, const Mem& m, uint32_t cur) {
    if (!(uni(c.mask) & 0x18u) || (uni(c.ctrl) & 0x38u) == 0x18u || uni(c.irq_line)) return NES_FRAME_DOTS;
    const uint8_t* r = m.rec->mreg;
    if (r[13] == 0) return NES_FRAME_DOTS;
    const uint32_t cnt = r[12];
    const uint32_t k = (cnt == 0u || r[14] != 0) ? r[11] + 1u : cnt;   // the clock (1st, 2nd, ...) that leaves 0
    const uint32_t i = mmc3_clocks_upto(cur) + k - 1u;                     // its index in the frame
    return i < 240u ? i * 341u + 266u : i == 240u ? 261u * 341u + 256u : NES_FRAME_DOTS;
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

// ------------------------------------------------------------------------------------- PPU timing events
__device__ __forceinline__ uint64_t abs_dot(const Con& c) {
    return (uint64_t)uni(c.frame) * NES_FRAME_DOTS + uni(c.frame_dot);
}

// Dots from frame dot `cur` to the next MMC3 counter clock (dot 266 of lines 0-239, dot 256 of the pre-render line),
// strictly after it (patch:1881-1903).
__device__ __forceinline__ uint32_t dots_to_mmc3_clock(uint32_t cur) {
    const uint32_t line = cur / 341u, d = cur - line * 341u;
    if (line < 240u) {
        if (d < 266u) return 266u - d;
        if (line + 1u < 240u) return 341u - d + 266u;
        return (261u - line) * 341u + 256u - d;
    }
    if (line < 261u) return (261u - line) * 341u + 256u - d;
    if (d < 256u) return 256u - d;
    return 341u - d + 266u;
}

// Before a generic step on MMC3: the counter's clocks in the `dots` since the last settle, and the frame dot moved on
// by them (the caller's pending dots become 0). No other event lies in them (the caller settles at its horizon), and
// the generic step may change what decides the clocks (the mask, the control register, the IRQ registers), so the
// clocks before the instruction take the values before it, as they do when every clock is settled at its own dot.
__device__ inline void mmc3_presettle(Con& c, const Mem& m, uint32_t dots) {
    const uint32_t start = uni(c.frame_dot);
    if ((uni(c.mask) & 0x18u) && (uni(c.ctrl) & 0x38u) != 0x18u) mmc3_clock_span(c, m, start, start + dots);
    c.frame_dot = start + dots;
}

// Dots from the current frame dot to the next PPU event (patch:2001-2037): the frame wrap, vblank, the pre-render
// line, the $2002 flag set and clear dots, the scheduled sprite-0 check and, on MMC3, the counter clocks. A short
// frame ends a dot early. Written as a search for the nearest event at an absolute dot (events at or before the
// current dot count from the next frame), then one difference. On MMC3 the reference stops at every clock; with
// every_clock false only the clock that raises the IRQ is an event (mmc3_clock_span applies the others in a span),
// which changes nothing the CPU can see while it runs instructions; the idle loop's fast-forward stops at every clock
// as the reference's does (each stop runs one JMP as an instruction, with the DMC's cycle steal).
__device__ inline uint32_t dots_to_event(const Con& c, const Mem& m, bool every_clock = false) {
    const uint32_t cur = uni(c.frame_dot), skip = (uni(c.log_flags) & NES_LOG_SHORT) ? 1u : 0u;
    const uint32_t frame = NES_FRAME_DOTS - skip;
    uint32_t next = frame;
    auto cand = [&](uint32_t e) {
        const uint32_t at = e > cur ? e : frame + e;
        if (at < next) next = at;
    };
    cand(NES_VFLAG_DOT);
    cand(NES_VBLANK_DOT);
    cand(NES_SCLR_DOT);
    cand(NES_PRERENDER_DOT);
    const uint32_t s0 = uni(c.s0_sched) & NES_S0_DOT;
    if (s0 != 0) cand(s0);
    if (m.cart.board == NES_BOARD_MMC3) {
        uint32_t at;
        if (every_clock) {
            at = cur + dots_to_mmc3_clock(cur);
            if (at >= NES_FRAME_DOTS) at -= skip;
        } else {
            at = mmc3_irq_dot(c, m, cur);
        }
        if (at < next) next = at;
    }
    return next - cur;
}

// The frame log's header from the live state (patch:1073-1105): taken at the pre-render line, and at power-on.
__device__ inline void log_header(const Con& c, const Mem& m, uint32_t kook) {
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
    h[5] = c.nt_map | (kook ? NES_LOG_KOOK : 0u);
    for (uint32_t i = 0; i < 8; ++i) h[6 + i] = pal[i];
    const uint8_t* r = m.rec->mreg;
    const bool mmc2 = m.cart.board == NES_BOARD_MMC2;
    h[14] = mmc2 ? (r[0] | ((uint32_t)r[1] << 8) | ((uint32_t)r[2] << 16) | ((uint32_t)r[3] << 24)) : 0u;
    h[15] = mmc2 ? (r[6] | ((uint32_t)r[7] << 8)) : 0u;
}

// The pre-render line: the log starts over for the next frame; every other frame is a kook frame, whose pre-render
// line is a dot short (patch:1111-1122).
__device__ inline void log_capture(Con& c, const Mem& m) {
    const uint32_t flags = uni(c.log_flags), kook = flags & NES_LOG_NEXT_KOOK;
    log_header(c, m, kook);
    c.log_n = 0;
    c.log_frame = uni(c.frame) + 1u;
    c.log_flags = ((flags ^ NES_LOG_NEXT_KOOK) & ~NES_LOG_SHORT) | (kook ? NES_LOG_SHORT : 0u);
}

// MMC2 at vblank: the latches the frame's own pattern fetches leave, and the halves' pages they select.
__device__ inline void mmc2_resolve(Con& c, const Mem& m) {
    const uint32_t lat = mmc2_latches(m.rec->log, uni(c.log_n), m.nt, m.oam, m.cart.chr_pages1);
    NesRec* rec = m.rec;
    const uint32_t l0 = lat & 1u, l1 = (lat >> 8) & 1u;
    rec->mreg[6] = (uint8_t)l0;
    rec->mreg[7] = (uint8_t)l1;
    const uint32_t b0 = rec->mreg[l0], b1 = rec->mreg[2u + l1];
    for (uint32_t i = 0; i < 4; ++i) {   // the halves' pages, as the board's page sync sets them
        map_set_chr(m, i, 4u * b0 + i);
        map_set_chr(m, 4u + i, 4u * b1 + i);
    }
}

// The PPU over `dots` dots from the current frame dot (NeSLE's settle, patch:2040-2156): every event in the span,
// per frame in this order - the sprite-0 check, the $2002 vblank flag, vblank (NMI 12 dots after the flag, whether
// or not a read took it; MMC2's latch resolve), the $2002 clear, the pre-render line (log capture, this frame's
// sprite-0 check scheduled for sprite 0's first line) - then the span's MMC3 clocks. B: the emulator's board class
// (the fixed-PRG instantiation has neither MMC2 nor MMC3).
template <uint32_t B>
__device__ inline void ppu_step(Con& c, const Mem& m, uint32_t dots) {
    const uint32_t start = uni(c.frame_dot);
    uint32_t end = start + dots;
    if ((uni(c.log_flags) & NES_LOG_SHORT) && end >= NES_FRAME_DOTS - 1u) end += 1u;   // the skipped last dot
    const uint32_t frames = end / NES_FRAME_DOTS;
    for (uint32_t f = 0; f <= frames; ++f) {
        const uint32_t base = f * NES_FRAME_DOTS;
        auto crossed = [&](uint32_t e) { return base + e > start && base + e <= end; };
        const uint32_t sched = uni(c.s0_sched), s0 = sched & NES_S0_DOT;
        if (s0 != 0 && crossed(s0)) {
            // worked out again with the writes logged so far, unless nothing was logged since the last answer
            const uint32_t log_n = uni(c.log_n);
            uint32_t hit, dot;
            if ((sched & NES_S0_KNOWN) && ((sched >> 20) & 0x1FFu) == log_n) {
                dot = s0;
                hit = (sched & NES_S0_HIT) ? 1u : 0u;
            } else {
                dot = sprite0_hit(m.rec->log, log_n, m.nt, m.oam, m.cart.chr, m.rec->chr_ram,
                                  m.cart.board == NES_BOARD_MMC2 ? m.cart.chr_pages1 : 0u, m.scratch, &hit);
                dot = uni(dot);
                hit = uni(hit);
            }
            const bool reached = base + dot <= end;
            if (hit && reached) c.status = uni(c.status) | 0x40u;
            c.s0_sched = dot != 0 && !reached ? dot | NES_S0_KNOWN | (hit ? NES_S0_HIT : 0u) | (log_n << 20) : 0u;
        }
        if (crossed(NES_VFLAG_DOT)) c.status = uni(c.status) | 0x80u;
        if (crossed(NES_VBLANK_DOT)) {
            if (uni(c.ctrl) & 0x80u) c.nmi_pending = 1;
            if constexpr (B != NES_BOARD_NROM)
                if (m.cart.board == NES_BOARD_MMC2) mmc2_resolve(c, m);
        }
        if (crossed(NES_SCLR_DOT)) c.status = uni(c.status) & 0x1Fu;
        if (crossed(NES_PRERENDER_DOT)) {
            c.status = uni(c.status) & 0x1Fu;
            log_capture(c, m);
            const uint32_t y = uni(m.oam[0]);
            c.s0_sched = y < 239u ? (y + 1u) * 341u - 20u - NES_FCEU_LAG : 0u;
        }
    }
    if constexpr (B != NES_BOARD_NROM) {
        // FCEUmm clocks the counter while rendering, unless both pattern tables are at $1000 with 8x8 sprites
        if (m.cart.board == NES_BOARD_MMC3 && (uni(c.mask) & 0x18u) && (uni(c.ctrl) & 0x38u) != 0x18u)
            mmc3_clock_span(c, m, start, end);
    }
    c.frame_dot = end % NES_FRAME_DOTS;
    c.frame = uni(c.frame) + frames;
    if (frames) c.log_flags = uni(c.log_flags) & ~NES_LOG_SHORT;
}

// ------------------------------------------------------------------------------------------------ bus
struct Access {
    uint32_t now;      // NeSLE frame dot at which the instruction starts: the stamp of its log events
    bool log_on;       // the instruction starts while a frame is logged (before vblank or from the pre-render line)
    bool dma;          // a $4014 write happened
};

__device__ inline void log_event(Con& c, const Mem& m, const Access& ac, uint32_t kind, uint32_t value, uint32_t aux) {
    if (!ac.log_on) return;
    uint32_t* h = m.rec->log;
    uint32_t* ev = h + NES_LOG_HDR_WORDS;
    if (kind == NES_EV_DATA && (c.mask & 0x18u) == 0 && c.log_n > 0) {
        uint32_t* last = ev + 2u * (c.log_n - 1u);
        if ((last[0] & 15u) == NES_EV_DATA && (last[1] >> 8) < 0xFFu) {
            last[1] += 0x100u;
            return;
        }
    }
    if (c.log_n >= NES_LOG_EVENTS) {
        h[0] |= NES_LOG_OVERFLOW;
        return;
    }
    ev[2u * c.log_n] = NES_EV_WORD0(kind, ac.now & 0x1FFFFu);
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
            log_event(c, m, ac, NES_EV_DREAD, 0, 0);
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
            }
            log_event(c, m, ac, NES_EV_DATA, 0, 0);
        } else if (pa < 0x3F00u) {
            m.nt[nt_index(c.nt_map, pa)] = (uint8_t)v;
            log_event(c, m, ac, NES_EV_DATA, 0, 0);
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
        if (v < 0x20u && (c.oam_addr & 15u) == 0u && ((unsigned long long)oam & 15u) == 0u && ((unsigned long long)m.ram & 15u) == 0u) {
            // a RAM page (no side effect on the bus) to a 16-byte-aligned OAM address: 16 moves of 16 bytes, OAM
            // wrapping at its end, instead of 256 of one byte
            const uint4* from = reinterpret_cast<const uint4*>(m.ram + ((v << 8) & 0x7FFu));
            uint4* to = reinterpret_cast<uint4*>(oam);
            const uint32_t d0 = c.oam_addr >> 4;
            for (uint32_t j = 0; j < 16u; ++j) to[(d0 + j) & 15u] = from[j];
        } else {
            for (uint32_t i = 0; i < 256u; ++i) {
                const uint32_t src = (v << 8) | i;
                const uint32_t b = src < 0x2000u ? m.ram[src & 0x7FFu] : bus_read(c, m, ac, src);
                oam[(c.oam_addr + i) & 0xFFu] = (uint8_t)b;
            }
        }
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
// the DMC service. `now0` = the frame dot of the step's first dot (the settled frame dot plus the dots not settled
// yet): the instruction's log events are stamped with its start, and with its cycles once it has run (patch:829-836,
// 1166-1185). Returns the CPU cycles, 0 with *fault set.
__device__ inline uint32_t cpu_step(Con& c, const Mem& m, const uint32_t* optab, uint32_t now0, uint32_t* fault,
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
    Access ac;
    ac.now = now0 + 3u * cyc;
    ac.log_on = ac.now < NES_VBLANK_DOT || ac.now >= NES_PRERENDER_DOT;
    ac.dma = false;
    const uint32_t logged = c.log_n;
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
    uint32_t opd = lo;
    if (d & D_READ) opd = bus_read(c, m, ac, ea);
    uint32_t res = 0, npc = (pc + instr_len(mode)) & 0xFFFFu;
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
    for (uint32_t i = logged; i < c.log_n && i < NES_LOG_EVENTS; ++i)
        m.rec->log[NES_LOG_HDR_WORDS + 2u * i] |= (icyc > 15u ? 15u : icyc) << 4;
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
    rec->dmc_byte_end = 7u + 1u + 7u * 428u;
    rec->dmc_event = kDmcIdle;
    c.ctrl = c.mask = c.fx = c.v = c.t = 0;
    log_header(c, m, 0);   // frame 0 is logged from the power-on state (patch:1160-1166)
}

// ------------------------------------------------------------------------------------ record <-> lane
__device__ inline void con_load(Con& c, const NesRec* r) {
    c.pc = r->pc; c.a = r->a; c.x = r->x; c.y = r->y; c.sp = r->sp; c.p = r->p;
    c.irq_line = r->irq_line; c.nmi_pending = r->nmi_pending; c.cycles = r->cycles;
    c.pad = r->pad; c.shift = r->shift; c.strobe = r->strobe; c.instr = r->instr_lo;
    c.frame_dot = r->frame_dot; c.frame = r->frame;
    c.v = r->v; c.t = r->t; c.ctrl = r->ctrl; c.mask = r->mask; c.status = r->status; c.oam_addr = r->oam_addr;
    c.fx = r->fx; c.w = r->w; c.read_buf = r->read_buf; c.open_bus = r->open_bus;
    c.s0_sched = r->s0_sched; c.log_frame = r->log_frame; c.log_n = r->log_n; c.log_flags = r->log_flags;
    c.dmc_event = r->dmc_event;
    c.prg0 = r->prg_off[0]; c.prg1 = r->prg_off[1]; c.prg2 = r->prg_off[2]; c.prg3 = r->prg_off[3];
    c.nt_map = r->nt_map[0] | (r->nt_map[1] << 2) | (r->nt_map[2] << 4) | ((uint32_t)r->nt_map[3] << 6);
    c.map_fast = r->board == NES_BOARD_MMC3   ? r->mreg[8]
                 : r->board == NES_BOARD_MMC1 ? r->mreg[4] | (r->mreg[5] << 8)
                                              : 0u;
}

__device__ inline void con_store(const Con& c, NesRec* r) {
    r->pc = (uint16_t)c.pc; r->a = (uint8_t)c.a; r->x = (uint8_t)c.x; r->y = (uint8_t)c.y; r->sp = (uint8_t)c.sp;
    r->p = (uint8_t)c.p; r->irq_line = (uint8_t)c.irq_line; r->nmi_pending = (uint8_t)c.nmi_pending;
    r->cycles = c.cycles; r->pad = (uint8_t)c.pad; r->shift = (uint8_t)c.shift; r->strobe = (uint8_t)c.strobe;
    r->instr_lo = c.instr; r->frame_dot = c.frame_dot; r->frame = c.frame;
    r->v = (uint16_t)c.v; r->t = (uint16_t)c.t; r->ctrl = (uint8_t)c.ctrl; r->mask = (uint8_t)c.mask;
    r->status = (uint8_t)c.status; r->oam_addr = (uint8_t)c.oam_addr; r->fx = (uint8_t)c.fx; r->w = (uint8_t)c.w;
    r->read_buf = (uint8_t)c.read_buf; r->open_bus = (uint8_t)c.open_bus;
    r->s0_sched = c.s0_sched; r->log_frame = c.log_frame; r->log_n = (uint16_t)c.log_n;
    r->log_flags = (uint8_t)c.log_flags;
    r->dmc_event = c.dmc_event;
    // prg_off and nt_map are written through to the record whenever they change (map_set_*)
}

}  // namespace nd
