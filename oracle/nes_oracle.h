/* ORACLE — test infrastructure only.
 *
 * Scalar CPU restatement of one NES console on the env's hot path: 6502 (official opcodes; any other
 * opcode is a fault), bus, PPU timing with the frame log, the line-replay renderer, sprite-0 hit,
 * NROM/MMC1/UxROM/CNROM/MMC3/MMC2, DMC, controller port. It exists to check the HIP library bit for bit; nothing in the
 * product links it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Reference behaviour followed (file:line in kdcyberdude/ghostrun-lab):
 *   frame loop ............ rl/csrc/nes_machine.cuh:67-103 (step_until: lazy PPU settle, JMP-to-self
 *                           fast-forward, 200k budget, fault = pc << 8 | opcode)
 *   instruction step ...... third_party/nesle-extensions.patch:823-862 (NMI, then level IRQ, instruction,
 *                           DMA stall, DMC service)
 *   fast-forward .......... patch:866-893 ((dots_to_event + 8) / 9 skipped 3-cycle jumps, DMC without steal)
 *   bus side effects ...... patch:570-779 ($2000-$2007, $4014, $4015, $4016, $6000 PRG RAM, $8000 mapper)
 *   DMC ................... patch:430-565 (rate table, 4-cycle fetch steal, loop, rate change at next clock)
 *   PPU events ............ patch:1822-2240 (NeSLE's settle over a span: the scheduled sprite-0 check, $2002 bit 7
 *                           12 dots before the vblank NMI, status cleared 12 dots before the pre-render line, log
 *                           capture, MMC3 clocks at dot 266 of lines 0-239 and dot 256 of the pre-render line while
 *                           rendering and not both pattern tables at $1000 with 8x8 sprites; kook frames a dot short)
 *   frame log ............. patch:900-1185 (header at pre-render, events stamped with their instruction's start dot
 *                           and cycles, $2007 writes merged while rendering is off, 256 events)
 *   line replay ........... patch:1243-1730 (FCEUmm's line renderer: writes applied at their dot mid-line, 34 tile
 *                           slots with the two-tile shift registers, Fixit1/Fixit2, sprite lines fetched at the end
 *                           of the line before and latched at RefreshSprites, CopySprites, greyscale while rendering,
 *                           emphasis from the mask at the line's end)
 *   sprite-0 hit .......... patch:1732-1788 (frame_sprite0_hit: the first line position from which a $2002 read
 *                           sees the hit, minus 12 dots for the read's own cycles)
 *   mappers ............... patch:2841-3367 (MMC1 serial port/modes, MMC3 R0-R7/modes/IRQ rev B, WRAM enable,
 *                           CNROM/UxROM latches, MMC2 registers)
 *   MMC2 latches .......... patch:615-664, 3196-3220 (CPU-driven flips), 1390-1402 and the fetch order of the line
 *                           replay (the hook after each pattern fetch), 1790-1812 (the vblank resolve)
 *   obs crop .............. rl/csrc/nes_machine.cuh:133-155 (lines 8..231, x 8..247, & 0x3F, emph = mask>>5&7)
 * The 6502 core itself is upstream NeSLE (not in the reference tree): parity with it is unpinned; the oracle is pinned
 * by datasheet known-answer tests instead (tests/test_oracle_cpu6502.py). The line replay, the sprite-0 dot and the
 * PPU event timing are pinned by hand-derived known-answer tests (tests/test_oracle_ppu.py); FCEUmm's 11-dot grid lag
 * and its kook frames are followed as the patch states them, and no reference golden vector pins them.
 * MMC2: registers, CPU-driven flips and the fetch-then-flip order along a line are pinned by known-answer tests
 * (tests/test_oracle_mappers.py); the vblank resolve is parity unpinned (no golden vector of the reference covers it).
 */
#ifndef NES_ORACLE_H
#define NES_ORACLE_H
#include <stdint.h>

#include "nesrec.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct NesCart {
    const uint8_t* prg;    /* PRG image, size a power of two */
    uint32_t prg_size;
    const uint8_t* chr;    /* CHR ROM, NULL = 8 KB CHR RAM in the console record */
    uint32_t chr_size;
    uint8_t board;         /* NES_BOARD_* */
    uint8_t mirroring;     /* header arrangement: 0 horizontal, 1 vertical */
    uint8_t bus_conflicts; /* UxROM / CNROM declared with AND-type bus conflicts (NES 2.0 submapper 2) */
} NesCart;

/* iNES parse into a cart view over `rom` (PRG copied into `prg_buf` padded to a power of two).
 * Returns 0, or -1 with a message in err. */
int orc_parse_ines(const uint8_t* rom, uint32_t size, uint8_t* prg_buf, uint32_t prg_buf_size, NesCart* cart,
                   char* err, int err_len);

void orc_power_on(NesRec* r, const NesCart* c);
/* Runs until the PPU reaches absolute dot `target` (frame * 89342 + frame_dot). Returns the fault code
 * (pc << 8 | opcode of an unimplemented opcode), 0 = fine. */
uint32_t orc_run_until(NesRec* r, const NesCart* c, uint64_t target);
/* One step (pending interrupt + one instruction) with the PPU settled after it. Returns CPU cycles, or 0
 * with *fault set. For known-answer tests. */
uint32_t orc_step(NesRec* r, const NesCart* c, uint32_t* fault);
/* The picture of the logged frame: 240 lines x 256 colour indices and each line's emphasis. */
void orc_render_full(const NesRec* r, const NesCart* c, uint8_t* pix /* 240*256 */, uint8_t* emph /* 240 */);
/* The env's 224 x 240 crop (rl/csrc/nes_machine.cuh:133-155). */
void orc_render_obs(const NesRec* r, const NesCart* c, uint8_t* obs /* 224*240 */, uint8_t* emph /* 224 */);
/* CPU bus access with side effects (tests). */
uint8_t orc_bus_read(NesRec* r, const NesCart* c, uint16_t addr);
void orc_bus_write(NesRec* r, const NesCart* c, uint16_t addr, uint8_t v);
/* DMC service at CPU cycle `now` (tests). Returns the stolen cycles. */
uint32_t orc_dmc_service(NesRec* r, uint64_t now, int steal);
void orc_dmc_reset(NesRec* r, uint64_t now);
/* FCEUmm's sprite-0 hit of the logged frame from the log so far (tests): the frame dot from which an instruction
 * sees the flag (*hit = 1), else the end of sprite 0's lines, or 0 with sprite 0 below the picture. */
uint32_t orc_sprite0_hit(const NesRec* r, const NesCart* c, int* hit);
/* MMC2's vblank resolve (tests): the latches the logged frame's own pattern fetches leave, written to the board's
 * latch registers with the CHR pages they select (patch:1790-1812). */
void orc_mmc2_resolve(NesRec* r, const NesCart* c);
/* orc_run_until with an instruction budget other than NES_BUDGET (tests of the budget exit). */
uint32_t orc_run_until_budget(NesRec* r, const NesCart* c, uint64_t target, uint32_t budget);
/* Hash of the 2 KB CPU RAM: sum over 32-bit words k of splitmix64(k << 32 | word_k) mod 2^64. */
uint64_t orc_ram_hash(const uint8_t* ram);
uint64_t orc_splitmix64(uint64_t x);

#ifdef __cplusplus
}
#endif
#endif
