/* Console record: the complete state of one emulated NES console, as one contiguous block.
 *
 * Both the CPU oracle (oracle/) and the HIP library keep every console in this layout, so a
 * whole console can be compared byte for byte between the two builds, restored from a boot
 * snapshot with one copy, and saved/loaded for an exact resume.
 *
 * The reference keeps the same information as ~40 separate per-env arrays (rl/csrc/nes_machine.cuh:37-64,
 * `bind_arrays`); the fields below cover the ones on the NROM/MMC1/MMC3 path.
 *
 * Layout rules: little-endian, no implicit padding (checked below), every memory block 256-byte aligned.
 * Plain C so that gcc (oracle) and hipcc (device + host) read it identically.
 */
#ifndef NESREC_H
#define NESREC_H
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <stddef.h>
#include <stdint.h>
#endif

#define NES_RAM_BYTES 2048u
#define NES_NT_BYTES 2048u
#define NES_OAM_BYTES 256u
#define NES_PAL_BYTES 32u
#define NES_PRGRAM_BYTES 8192u
#define NES_CHRRAM_BYTES 8192u
#define NES_LOG_HDR_WORDS 16u
#define NES_LOG_EVENTS 256u
#define NES_LOG_WORDS (NES_LOG_HDR_WORDS + 2u * NES_LOG_EVENTS)

/* Frame timing (PPU dots). A frame is 262 lines of 341 dots; a decision frame ends at the vblank dot. */
#define NES_DOTS_PER_LINE 341u
#define NES_FRAME_DOTS (341u * 262u)          /* 89342 (rl/csrc/nes_machine.cuh:28) */
#define NES_VBLANK_DOT (241u * 341u + 1u)     /* 82182 (rl/csrc/nes_machine.cuh:29) */
#define NES_PRERENDER_DOT (261u * 341u + 1u)  /* 89002: flags cleared, frame log header captured */
#define NES_BUDGET 200000u                    /* instructions per frame (rl/csrc/nes_machine.cuh:30) */
#define NES_NO_HIT 0x7FFFFFFF

/* Boards. */
#define NES_BOARD_NROM 0u
#define NES_BOARD_MMC1 1u
#define NES_BOARD_UXROM 2u                    /* 16 KB PRG bank at $8000, the last 16 KB fixed at $C000 */
#define NES_BOARD_CNROM 3u                    /* 32 KB PRG fixed, 8 KB CHR bank latch (patch:3418) */
#define NES_BOARD_MMC3 4u
#define NES_BOARD_MMC2 5u                     /* mapper 9: 8 KB PRG bank at $8000, 4 KB CHR halves picked by the
                                                 $FD/$FE latches (patch:3027-3035, 3147-3156) */

/* Frame timing of the renderer's line grid (FCEUmm's, which the reference replays the log on,
 * third_party/nesle-extensions.patch:940-965). A log event is stamped with the NeSLE frame dot at which its
 * instruction starts and the instruction's cycles; on the replay grid it sits NES_FCEU_LAG dots later, and the
 * pre-render line's writes are counted back from line 0 (one dot more on a "kook" frame, whose pre-render line is a
 * dot short). Line l of the replay starts NES_LINE_LEAD dots before the line's dot 0. */
#define NES_FCEU_LAG 11
#define NES_LINE_LEAD 16
#define NES_VFLAG_DOT (NES_VBLANK_DOT - 12u)      /* 82170: $2002 bit 7 set (patch:1940-1945) */
#define NES_SCLR_DOT (NES_PRERENDER_DOT - 12u)    /* 88990: $2002 bits 5-7 cleared */

/* Frame-log events: two words each. Word 0: kind (bits 0-3) | instruction cycles, at most 15 (bits 4-7) |
 * NeSLE frame dot of the instruction's start (bits 8-24). Word 1: value | aux << 8. */
#define NES_EV_CTRL 1u    /* $2000 */
#define NES_EV_MASK 2u    /* $2001 */
#define NES_EV_SCROLL 3u  /* $2005, aux = write toggle before the write */
#define NES_EV_ADDR 4u    /* $2006, aux = write toggle before the write */
#define NES_EV_DATA 5u    /* $2007 write below the palette: address increment; aux = further writes merged into it */
#define NES_EV_PAL 6u     /* $2007 palette write: value, aux = palette index (after mirroring); address increment */
#define NES_EV_CHR 7u     /* CHR 1 KB page change: value = page, aux = slot 0..7 */
#define NES_EV_MIRROR 8u  /* nametable map change: value = nt_map packed 4 x 2 bits */
#define NES_EV_MMC2 9u    /* MMC2 register change: value, aux = register (0-3 CHR banks, 6-7 latches) */
#define NES_EV_DREAD 10u  /* $2007 read: address increment (a vertical step while a line is drawn) */
#define NES_EV_WORD0(kind, dot) ((uint32_t)(kind) | ((uint32_t)(dot) << 8))

/* Log header words: 0 count | overflow << 31, 1 ctrl | mask << 8 | fine x << 16, 2 v | t << 16,
 * 3-4 CHR 1 KB page of each slot (8 bits each), 5 nt_map packed | kook frame << 8, 6-13 palette RAM,
 * 14 MMC2 CHR registers (8 bits each), 15 MMC2 latch 0 | latch 1 << 8 (zero on other boards). */
#define NES_LOG_KOOK 0x100u

/* s0_sched: the frame dot of the next sprite-0 check (bits 0-16), 0 = none this frame; once a check has run and
 * left a later dot: the answer it found (NES_S0_KNOWN, NES_S0_HIT) and the log length it saw (bits 20-28). */
#define NES_S0_DOT 0x1FFFFu
#define NES_S0_HIT 0x20000000u
#define NES_S0_KNOWN 0x40000000u

/* log_flags */
#define NES_LOG_NEXT_KOOK 1u   /* the next frame captured is a kook frame */
#define NES_LOG_SHORT 2u       /* this frame's pre-render line is a dot short (from its capture to the wrap) */

#define NES_LOG_OVERFLOW 0x80000000u

typedef struct NesRec {
    /* ---- CPU, controller (0x00) ---- */
    uint16_t pc;
    uint8_t a, x, y, sp, p;
    uint8_t irq_line;     /* cartridge IRQ line (MMC3) */
    uint64_t cycles;      /* CPU cycles since power-on */
    uint8_t nmi_pending;
    uint8_t pad;          /* pad byte of the current frame (bit0 A .. bit7 Right) */
    uint8_t shift;        /* controller 1 shift register */
    uint8_t strobe;
    uint32_t instr_lo;    /* emulated instructions since power-on (low 32 bits) */
    /* ---- PPU (0x18) ---- */
    uint32_t frame_dot;   /* 0..89341, 0 = line 0 dot 0 */
    uint32_t frame;
    uint16_t v, t;
    uint8_t ctrl, mask, status, oam_addr;
    uint8_t fx, w, read_buf, open_bus;
    uint32_t s0_sched;    /* next sprite-0 check (NES_S0_*) */
    uint32_t log_frame;   /* frame whose lines the log describes */
    uint16_t log_n;
    uint8_t log_flags;    /* NES_LOG_NEXT_KOOK, NES_LOG_SHORT */
    uint8_t board;
    uint64_t _ppu_res;
    /* ---- DMC (0x40) ---- */
    uint64_t dmc_byte_end;
    uint64_t dmc_event;
    uint16_t dmc_left;
    uint8_t dmc_control, dmc_length, dmc_rate, dmc_full, _dmc0, _dmc1;
    /* ---- mapper (0x58) ---- */
    uint8_t mreg[16];
    uint32_t prg_off[4];  /* byte offset in PRG of the 8 KB page at $8000/$A000/$C000/$E000 */
    uint32_t chr_off[8];  /* byte offset in CHR of each 1 KB slot of $0000-$1FFF */
    uint8_t nt_map[4];    /* physical 1 KB nametable (0/1) of each logical nametable */
    uint32_t _res[25];    /* pad to 0x100 */
    /* ---- memories ---- */
    uint8_t ram[NES_RAM_BYTES];         /* 0x100 */
    uint8_t nt[NES_NT_BYTES];           /* 0x900 */
    uint8_t oam[NES_OAM_BYTES];         /* 0x1100 */
    uint8_t pal[256];                   /* 0x1200: 32 used */
    uint32_t log[NES_LOG_WORDS + 48];   /* 0x1300: header + events, padded to 256 B */
    uint8_t prg_ram[NES_PRGRAM_BYTES];  /* 0x1C00 */
    uint8_t chr_ram[NES_CHRRAM_BYTES];  /* 0x3C00 */
} NesRec;                               /* 0x5C00 = 23552 bytes */

#define NES_REC_BYTES 23552u

#ifdef __cplusplus
#define NESREC_ASSERT static_assert
#else
#define NESREC_ASSERT _Static_assert
#endif
NESREC_ASSERT(offsetof(NesRec, frame_dot) == 0x18, "layout");
NESREC_ASSERT(offsetof(NesRec, dmc_byte_end) == 0x40, "layout");
NESREC_ASSERT(offsetof(NesRec, mreg) == 0x58, "layout");
NESREC_ASSERT(offsetof(NesRec, ram) == 0x100, "layout");
NESREC_ASSERT(offsetof(NesRec, nt) == 0x900, "layout");
NESREC_ASSERT(offsetof(NesRec, oam) == 0x1100, "layout");
NESREC_ASSERT(offsetof(NesRec, pal) == 0x1200, "layout");
NESREC_ASSERT(offsetof(NesRec, log) == 0x1300, "layout");
NESREC_ASSERT(offsetof(NesRec, prg_ram) == 0x1C00, "layout");
NESREC_ASSERT(offsetof(NesRec, chr_ram) == 0x3C00, "layout");
NESREC_ASSERT(sizeof(NesRec) == NES_REC_BYTES, "layout");

#endif
