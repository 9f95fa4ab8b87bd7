/* ORACLE — test infrastructure only (see nes_oracle.h). Scalar C, one console at a time, written for
 * clarity: a switch-per-opcode 6502, a pixel-by-pixel line replay. */
#include "nes_oracle.h"

#include <stdio.h>
#include <string.h>

#define FL_C 0x01u
#define FL_Z 0x02u
#define FL_I 0x04u
#define FL_D 0x08u
#define FL_B 0x10u
#define FL_U 0x20u
#define FL_V 0x40u
#define FL_N 0x80u


uint64_t orc_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

uint64_t orc_ram_hash(const uint8_t* ram) {
    uint64_t h = 0;
    for (uint32_t k = 0; k < NES_RAM_BYTES / 4u; ++k) {
        const uint32_t w = (uint32_t)ram[4 * k] | ((uint32_t)ram[4 * k + 1] << 8) | ((uint32_t)ram[4 * k + 2] << 16) |
                           ((uint32_t)ram[4 * k + 3] << 24);
        h += orc_splitmix64(((uint64_t)k << 32) | w);
    }
    return h;
}

/* ------------------------------------------------------------------------------------------ cartridge */

int orc_parse_ines(const uint8_t* rom, uint32_t size, uint8_t* prg_buf, uint32_t prg_buf_size, NesCart* cart,
                   char* err, int err_len) {
    memset(cart, 0, sizeof(*cart));
    if (size < 16 || rom[0] != 'N' || rom[1] != 'E' || rom[2] != 'S' || rom[3] != 0x1A) {
        snprintf(err, err_len, "not an iNES image");
        return -1;
    }
    const uint32_t prg = (uint32_t)rom[4] * 16384u, chr = (uint32_t)rom[5] * 8192u;
    const uint32_t mapper = (rom[6] >> 4) | (rom[7] & 0xF0u);
    const uint32_t trainer = (rom[6] & 4u) ? 512u : 0u;
    if (rom[6] & 8u) {
        snprintf(err, err_len, "four-screen nametables are not supported");
        return -1;
    }
    if (mapper > 4u && mapper != 9u) {
        snprintf(err, err_len, "unsupported mapper %u (supported: 0 NROM, 1 MMC1, 2 UxROM, 3 CNROM, 4 MMC3, 9 MMC2)",
                 mapper);
        return -1;
    }
    if (mapper == 9u && chr == 0) {
        snprintf(err, err_len, "MMC2 needs CHR ROM");
        return -1;
    }
    if (prg == 0 || 16u + trainer + prg + chr > size) {
        snprintf(err, err_len, "truncated iNES image");
        return -1;
    }
    uint32_t padded = 8192u;
    while (padded < prg) padded <<= 1;
    if (padded > prg_buf_size) {
        snprintf(err, err_len, "PRG too large");
        return -1;
    }
    memset(prg_buf, 0, padded);
    memcpy(prg_buf, rom + 16 + trainer, prg);
    if (prg < padded) { /* mirror a short image (16 KB NROM) across the padded space */
        for (uint32_t o = prg; o < padded; o += prg) memcpy(prg_buf + o, rom + 16 + trainer, prg);
    }
    cart->prg = prg_buf;
    cart->prg_size = padded;
    cart->chr = chr ? rom + 16 + trainer + prg : NULL;
    cart->chr_size = chr ? chr : NES_CHRRAM_BYTES;
    cart->board = (uint8_t)(mapper == 9u ? NES_BOARD_MMC2 : mapper);
    cart->mirroring = (uint8_t)(rom[6] & 1u);
    /* UxROM / CNROM bus conflicts only when the header declares them: NES 2.0 (byte 7 bits 2-3 = 2), submapper 2
     * (patch:4008, layout.bus_conflicts = mapper 3 && declared) */
    cart->bus_conflicts =
        (uint8_t)((mapper == 2u || mapper == 3u) && (rom[7] & 0x0Cu) == 0x08u && (rom[8] >> 4) == 2u);
    return 0;
}

static void set_nt_map(NesRec* r, uint32_t kind) { /* 0 horizontal, 1 vertical, 2 single low, 3 single high */
    static const uint8_t maps[4][4] = {{0, 0, 1, 1}, {0, 1, 0, 1}, {0, 0, 0, 0}, {1, 1, 1, 1}};
    memcpy(r->nt_map, maps[kind & 3u], 4);
}

static uint32_t nt_map_packed(const NesRec* r) {
    return r->nt_map[0] | (r->nt_map[1] << 2) | (r->nt_map[2] << 4) | ((uint32_t)r->nt_map[3] << 6);
}

static void set_prg8(NesRec* r, const NesCart* c, int slot, uint32_t page) {
    r->prg_off[slot] = (page & (c->prg_size / 8192u - 1u)) * 8192u;
}
static void set_chr1(NesRec* r, const NesCart* c, int slot, uint32_t page) {
    r->chr_off[slot] = (page & (c->chr_size / 1024u - 1u)) * 1024u;
}

/* MMC1 registers: 0 control, 1 CHR0, 2 CHR1, 3 PRG, 4 shift, 5 shift count.
 * UxROM register: 0 the 16 KB PRG bank at $8000. CNROM register: 0 the 8 KB CHR bank.
 * MMC3 registers: 0-7 R0-R7, 8 bank select, 9 mirroring, 10 PRG RAM protect, 11 IRQ latch, 12 IRQ counter,
 * 13 IRQ enabled, 14 IRQ reload. (patch:2917-2919, 2991-3063)
 * MMC2 registers: 0-3 the CHR banks ($FD/$0000, $FE/$0000, $FD/$1000, $FE/$1000), 4 PRG, 5 mirroring (1 vertical),
 * 6-7 the latches of the two halves (0 = $FD bank, 1 = $FE bank) (patch:2916, 3027-3035). */
static void mapper_sync(NesRec* r, const NesCart* c) {
    const uint8_t* m = r->mreg;
    if (c->board == NES_BOARD_MMC1) {
        const uint32_t control = m[0], offs = m[1] & 0x10u, prg = m[3] & 0x0Fu;
        uint32_t lo, hi;
        switch (control & 0x0Cu) {
            case 0x0Cu: lo = prg + offs; hi = 0x0Fu + offs; break;
            case 0x08u: lo = offs; hi = prg + offs; break;
            default: lo = (prg & ~1u) + offs; hi = lo + 1u; break;
        }
        set_prg8(r, c, 0, lo * 2u);
        set_prg8(r, c, 1, lo * 2u + 1u);
        set_prg8(r, c, 2, hi * 2u);
        set_prg8(r, c, 3, hi * 2u + 1u);
        const uint32_t c0 = (control & 0x10u) ? m[1] : (m[1] & 0xFEu);
        const uint32_t c1 = (control & 0x10u) ? m[2] : (m[1] | 0x01u);
        for (int i = 0; i < 4; ++i) {
            set_chr1(r, c, i, c0 * 4u + (uint32_t)i);
            set_chr1(r, c, 4 + i, c1 * 4u + (uint32_t)i);
        }
        switch (control & 3u) {
            case 0: set_nt_map(r, 2); break;
            case 1: set_nt_map(r, 3); break;
            case 2: set_nt_map(r, 1); break;
            default: set_nt_map(r, 0); break;
        }
    } else if (c->board == NES_BOARD_MMC3) {
        const uint32_t sel = m[8];
        if (sel & 0x40u) {
            set_prg8(r, c, 0, 0x7Eu);
            set_prg8(r, c, 2, m[6]);
        } else {
            set_prg8(r, c, 0, m[6]);
            set_prg8(r, c, 2, 0x7Eu);
        }
        set_prg8(r, c, 1, m[7]);
        set_prg8(r, c, 3, 0x7Fu);
        const int f = (sel & 0x80u) ? 4 : 0;
        set_chr1(r, c, 0 ^ f, m[0] & 0xFEu);
        set_chr1(r, c, 1 ^ f, m[0] | 1u);
        set_chr1(r, c, 2 ^ f, m[1] & 0xFEu);
        set_chr1(r, c, 3 ^ f, m[1] | 1u);
        set_chr1(r, c, 4 ^ f, m[2]);
        set_chr1(r, c, 5 ^ f, m[3]);
        set_chr1(r, c, 6 ^ f, m[4]);
        set_chr1(r, c, 7 ^ f, m[5]);
        set_nt_map(r, (m[9] & 1u) ? 0u : 1u);
    } else if (c->board == NES_BOARD_MMC2) { /* the 8 KB bank at $8000, the last three fixed */
        set_prg8(r, c, 0, m[4]);
        set_prg8(r, c, 1, ~2u);
        set_prg8(r, c, 2, ~1u);
        set_prg8(r, c, 3, ~0u);
        for (int i = 0; i < 4; ++i) {
            set_chr1(r, c, i, m[m[6] & 1u] * 4u + (uint32_t)i);
            set_chr1(r, c, 4 + i, m[2u + (m[7] & 1u)] * 4u + (uint32_t)i);
        }
        set_nt_map(r, m[5] ? 1u : 0u);
    } else if (c->board == NES_BOARD_UXROM) { /* the 16 KB bank in register 0, the last one fixed at $C000 */
        const uint32_t last = c->prg_size / 16384u - 1u;
        set_prg8(r, c, 0, m[0] * 2u);
        set_prg8(r, c, 1, m[0] * 2u + 1u);
        set_prg8(r, c, 2, last * 2u);
        set_prg8(r, c, 3, last * 2u + 1u);
        for (int i = 0; i < 8; ++i) set_chr1(r, c, i, (uint32_t)i);
        set_nt_map(r, c->mirroring ? 1u : 0u);
    } else { /* NROM; CNROM: the 8 KB CHR bank in register 0 (patch:2982-2990) */
        const uint32_t chr8 = c->board == NES_BOARD_CNROM ? m[0] : 0u;
        for (int i = 0; i < 4; ++i) set_prg8(r, c, i, (uint32_t)i);
        for (int i = 0; i < 8; ++i) set_chr1(r, c, i, chr8 * 8u + (uint32_t)i);
        set_nt_map(r, c->mirroring ? 1u : 0u);
    }
}

static void mapper_power_on(NesRec* r, const NesCart* c) {
    memset(r->mreg, 0, sizeof(r->mreg));
    if (c->board == NES_BOARD_MMC1) {
        r->mreg[0] = 0x0C;
    } else if (c->board == NES_BOARD_MMC3) {
        r->mreg[1] = 2; r->mreg[2] = 4; r->mreg[3] = 5; r->mreg[4] = 6; r->mreg[5] = 7; r->mreg[7] = 1;
        r->mreg[9] = c->mirroring ? 0 : 1;
    } else if (c->board == NES_BOARD_MMC2) {
        r->mreg[6] = 1;   /* both latches on the $FE bank (patch:3080-3083) */
        r->mreg[7] = 1;
    }
    mapper_sync(r, c);
}

/* A CPU write to $8000-$FFFF (patch:3124-3180). */
static void mapper_write(NesRec* r, const NesCart* c, uint16_t addr, uint8_t v) {
    uint8_t* m = r->mreg;
    if (c->board == NES_BOARD_MMC1) {
        if (v & 0x80u) {
            m[0] |= 0x0Cu;
            m[4] = 0;
            m[5] = 0;
        } else {
            m[4] = (uint8_t)(m[4] | ((v & 1u) << m[5]));
            if (++m[5] < 5u) return;
            m[(addr >> 13) & 3u] = m[4];
            m[4] = 0;
            m[5] = 0;
        }
        mapper_sync(r, c);
    } else if (c->board == NES_BOARD_MMC3) {
        switch (addr & 0xE001u) {
            case 0x8000u: m[8] = v; break;
            case 0x8001u: m[m[8] & 7u] = v; break;
            case 0xA000u: m[9] = v; break;
            case 0xA001u: m[10] = v; return;
            case 0xC000u: m[11] = v; return;
            case 0xC001u: m[14] = 1; return;
            case 0xE000u: m[13] = 0; r->irq_line = 0; return;
            default: m[13] = 1; return;
        }
        mapper_sync(r, c);
    } else if (c->board == NES_BOARD_MMC2) {
        switch (addr & 0xF000u) {
            case 0xA000u: m[4] = v & 0x0Fu; break;
            case 0xB000u: m[0] = v & 0x1Fu; break;
            case 0xC000u: m[1] = v & 0x1Fu; break;
            case 0xD000u: m[2] = v & 0x1Fu; break;
            case 0xE000u: m[3] = v & 0x1Fu; break;
            case 0xF000u: m[5] = (v & 1u) ^ 1u; break;
            default: return;   /* $8000-$9FFF: no register */
        }
        mapper_sync(r, c);
    } else if (c->board == NES_BOARD_CNROM || c->board == NES_BOARD_UXROM) {
        /* the bank latch, ANDed with the ROM byte under a bus conflict (patch:3124-3127, 3281-3283) */
        const uint8_t rom = c->prg[r->prg_off[(addr >> 13) & 3u] + (addr & 0x1FFFu)];
        m[0] = c->bus_conflicts ? (uint8_t)(v & rom) : v;
        mapper_sync(r, c);
    }
}

static void mmc3_clock(NesRec* r) { /* revision B counter (patch:3182-3193) */
    uint8_t* m = r->mreg;
    if (m[12] == 0 || m[14] != 0) {
        m[12] = m[11];
        m[14] = 0;
    } else {
        --m[12];
    }
    if (m[12] == 0 && m[13] != 0) r->irq_line = 1;
}

/* MMC2: a pattern fetch or CPU-driven VRAM address in $0FD0-$0FEF / $1FD0-$1FEF flips the latch of its half
 * (FCEUmm's PPU_hook ranges, patch:3196-3220, 1390-1402). 0 = none, else the latch value + 1 | half << 2. */
static uint32_t mmc2_trigger(uint32_t a) {
    const uint32_t high = (a >> 8) & 0x3Fu, low = a & 0xF0u;
    if (high >= 0x20u || (high & 0x0Fu) != 0x0Fu || (low != 0xD0u && low != 0xE0u)) return 0;
    return (low == 0xE0u ? 2u : 1u) | (high < 0x10u ? 0u : 4u);
}

static int prg_ram_enabled(const NesRec* r, const NesCart* c) {
    return c->board != NES_BOARD_MMC1 || (r->mreg[3] & 0x10u) == 0;
}

static uint8_t chr_read(const NesRec* r, const NesCart* c, const uint32_t* chr_off, uint32_t a) {
    const uint32_t off = chr_off[(a >> 10) & 7u] + (a & 0x3FFu);
    return c->chr ? c->chr[off] : r->chr_ram[off & (NES_CHRRAM_BYTES - 1u)];
}

/* ------------------------------------------------------------------------------------------------ DMC */

static uint32_t dmc_period(uint32_t rate) {
    static const uint16_t t[16] = {428, 380, 340, 320, 286, 254, 226, 214, 190, 160, 142, 128, 106, 84, 72, 54};
    return t[rate & 15u];
}

#define DMC_IDLE 0xFFFFFFFFFFFFFFFFull

void orc_dmc_reset(NesRec* r, uint64_t now) {
    r->dmc_left = 0;
    r->dmc_control = r->dmc_length = r->dmc_rate = r->dmc_full = 0;
    r->dmc_byte_end = now + 1u + 7u * dmc_period(0);
    r->dmc_event = DMC_IDLE;
}

/* Brings the sample channel up to CPU cycle `now` (patch:430-520): a buffered byte drains on its bit clocks,
 * then the next byte is fetched at once (4 stolen cycles unless `steal` is 0); silent time is skipped in
 * whole bytes; a rate change keeps the clock already counting. */
uint32_t orc_dmc_service(NesRec* r, uint64_t now, int steal) {
    const uint64_t byte_cycles = 8ull * dmc_period(r->dmc_rate);
    uint32_t stolen = 0;
    if (!r->dmc_full && r->dmc_byte_end <= now)
        r->dmc_byte_end += ((now - r->dmc_byte_end) / byte_cycles + 1u) * byte_cycles;
    for (;;) {
        if (r->dmc_full) {
            if (r->dmc_byte_end > now) break;
            r->dmc_full = 0;
            r->dmc_byte_end += byte_cycles;
            if (r->dmc_left == 0) {
                if (r->dmc_byte_end <= now)
                    r->dmc_byte_end += ((now - r->dmc_byte_end) / byte_cycles + 1u) * byte_cycles;
                break;
            }
        }
        if (r->dmc_left == 0) break;
        r->dmc_full = 1;
        if (--r->dmc_left == 0 && (r->dmc_control & 0x40u)) r->dmc_left = (uint16_t)(r->dmc_length * 16u + 1u);
        if (steal) {
            stolen += 4;
            now += 4;
        }
    }
    const uint32_t rate = r->dmc_control & 0x0Fu;
    if (rate != r->dmc_rate) {
        const uint64_t oldp = dmc_period(r->dmc_rate);
        const uint64_t later = (r->dmc_byte_end - now - 1u) / oldp;
        r->dmc_byte_end = r->dmc_byte_end - later * oldp + later * dmc_period(rate);
        r->dmc_rate = (uint8_t)rate;
    }
    r->dmc_event = r->dmc_full ? r->dmc_byte_end : DMC_IDLE;
    return stolen;
}

static void dmc_write(NesRec* r, uint16_t addr, uint8_t v) {
    if (addr == 0x4010) {
        r->dmc_control = v;
    } else if (addr == 0x4013) {
        r->dmc_length = v;
    } else if ((v & 0x10u) == 0) {
        r->dmc_left = 0;
    } else if (r->dmc_left == 0) {
        r->dmc_left = (uint16_t)(r->dmc_length * 16u + 1u);
    }
    r->dmc_event = 0;
}

/* ------------------------------------------------------------------------------------------- power-on */

static void log_header(NesRec* r, int kook);


void orc_power_on(NesRec* r, const NesCart* c) {
    memset(r, 0, sizeof(*r));
    r->board = c->board;
    mapper_power_on(r, c);
    memset(r->ram, 0xFF, NES_RAM_BYTES); /* power-on RAM 0xFF (rl/csrc/rlenv_build.hpp:243) */
    r->sp = 0xFD;
    r->p = FL_I | FL_U;
    const uint32_t lo = c->prg[r->prg_off[3] + 0x1FFCu], hi = c->prg[r->prg_off[3] + 0x1FFDu];
    r->pc = (uint16_t)(lo | (hi << 8));
    r->cycles = 7;
    orc_dmc_reset(r, r->cycles);
    log_header(r, 0);   /* frame 0 is logged from the power-on state (patch:1160-1166) */
}

/* ------------------------------------------------------------------------------------- frame log + replay */

/* The frame log's header from the live PPU and board state (patch:1073-1105): taken at the pre-render line, and
 * at power-on for the first frame. */
static void log_header(NesRec* r, int kook) {
    uint32_t* h = r->log;
    memset(h, 0, NES_LOG_HDR_WORDS * 4u);
    h[1] = r->ctrl | ((uint32_t)r->mask << 8) | ((uint32_t)r->fx << 16);
    h[2] = r->v | ((uint32_t)r->t << 16);
    for (int i = 0; i < 8; ++i) h[3 + (i >> 2)] |= ((r->chr_off[i] >> 10) & 0xFFu) << ((i & 3) * 8);
    h[5] = nt_map_packed(r) | (kook ? NES_LOG_KOOK : 0u);
    for (int i = 0; i < 8; ++i)
        h[6 + i] = r->pal[4 * i] | ((uint32_t)r->pal[4 * i + 1] << 8) | ((uint32_t)r->pal[4 * i + 2] << 16) |
                   ((uint32_t)r->pal[4 * i + 3] << 24);
    if (r->board == NES_BOARD_MMC2) {
        h[14] = r->mreg[0] | ((uint32_t)r->mreg[1] << 8) | ((uint32_t)r->mreg[2] << 16) | ((uint32_t)r->mreg[3] << 24);
        h[15] = r->mreg[6] | ((uint32_t)r->mreg[7] << 8);
    }
}

/* Pre-render line: the log starts over for the next frame; every other frame is a kook frame, whose pre-render
 * line is a dot short (patch:1111-1122). */
static void log_capture(NesRec* r) {
    const int kook = (r->log_flags & NES_LOG_NEXT_KOOK) != 0;
    log_header(r, kook);
    r->log_n = 0;
    r->log_frame = r->frame + 1u;
    r->log_flags = (uint8_t)(((r->log_flags ^ NES_LOG_NEXT_KOOK) & ~NES_LOG_SHORT) | (kook ? NES_LOG_SHORT : 0u));
}

/* Replay time of NeSLE frame dot `dot`: line 0 dot 0 is 0, the pre-render line negative (patch:950-956). */
static int32_t fceu_time(uint32_t dot, int kook) {
    return dot >= NES_PRERENDER_DOT ? (int32_t)dot - (int32_t)NES_FRAME_DOTS + NES_FCEU_LAG + kook
                                    : (int32_t)dot + NES_FCEU_LAG;
}

/* Up to eight sprites of one line: pattern bytes, attributes and x (FCEUmm's sprite line buffer). */
typedef struct SprLine {
    uint32_t n;
    uint8_t lo[8], hi[8], attr[8], x[8];
} SprLine;

/* The renderer's state between lines (patch:1289-1313): the PPU registers it has replayed, the board's CHR and
 * nametable wiring, the background shift registers, the sprite line fetched for the next line and the one it
 * draws, and the sprite-0 check. */
typedef struct Replay {
    const NesRec* r;
    const NesCart* c;
    const uint32_t* ev;
    uint32_t count, cur;
    int kook;
    uint32_t v, t, fx, ctrl, mask;
    uint32_t chr_off[8];
    uint8_t nt_map[4];
    int mmc2;
    uint32_t creg[4], latch[2], chr_pages;
    uint8_t pal[32];
    uint32_t sh_lo, sh_hi, at;       /* pattern shift registers (last two tiles fetched), attribute latch */
    SprLine fetched, drawn;
    uint8_t spal[16];
    int blurp;                       /* sprite 0 is in the fetched line */
    int spork;                       /* a sprite line waits to be drawn */
    int hit, hit_x;                  /* $2002 bit 6 of the replay and the pixel where it was found */
    int sphitx;                      /* x of sprite 0 on this line, NO_CHECK = no check */
    uint32_t sphit_bits;             /* its opaque pixels, leftmost in bit 7 */
} Replay;
#define NO_CHECK 0x100

/* One line's pixels: the palette value, 0x40 | backdrop where the background is transparent, 0xFF not drawn yet;
 * the next tile slot, the output position and whether the line's vertical step is still due. */
typedef struct Line {
    uint8_t px[256];
    int tile, out, fix;
} Line;

static uint32_t ev_kind(const Replay* s, uint32_t i) { return s->ev[2u * i] & 15u; }
static int32_t ev_start(const Replay* s, uint32_t i) {
    return fceu_time((s->ev[2u * i] >> 8) & 0x1FFFFu, s->kook);
}
/* The end of the event's instruction: its accesses are stamped there (patch:1336-1338). */
static int32_t ev_end(const Replay* s, uint32_t i) { return ev_start(s, i) + 3 * (int32_t)((s->ev[2u * i] >> 4) & 15u); }

static int rendering(const Replay* s) { return (s->mask & 0x18u) != 0; }
static uint32_t inc_of(const Replay* s) { return (s->ctrl & 4u) ? 32u : 1u; }

static void replay_mmc2_select(Replay* s, uint32_t half) { /* patch:1385-1388 */
    const uint32_t bank = s->creg[2u * half + s->latch[half]];
    for (uint32_t i = 0; i < 4u; ++i) s->chr_off[4u * half + i] = ((bank * 4u + i) & (s->chr_pages - 1u)) * 1024u;
}

static void replay_hook(Replay* s, uint32_t a) { /* a pattern fetch at a (patch:1390-1402) */
    const uint32_t t = s->mmc2 ? mmc2_trigger(a) : 0u;
    if (t == 0) return;
    s->latch[t >> 2] = (t & 3u) - 1u;
    replay_mmc2_select(s, t >> 2);
}

static uint8_t rp_chr(const Replay* s, uint32_t a) { return chr_read(s->r, s->c, s->chr_off, a & 0x1FFFu); }
static uint8_t rp_nt(const Replay* s, uint32_t a) {
    return s->r->nt[(s->nt_map[(a >> 10) & 3u] & 1u) * 1024u + (a & 0x3FFu)];
}

/* v one row down (FCEUmm's Fixit1, and a $2007 read while a line is drawn; patch:1410-1422). */
static void y_step(Replay* s) {
    uint32_t v = s->v;
    if ((v & 0x7000u) != 0x7000u) {
        v += 0x1000u;
    } else {
        v &= ~0x7000u;
        const uint32_t row = (v >> 5) & 31u;
        if (row == 29u) v = (v & ~0x03E0u) ^ 0x0800u;
        else if (row == 31u) v &= ~0x03E0u;
        else v += 0x20u;
    }
    s->v = v & 0x7FFFu;
}

/* Event i on the replay state (patch:1424-1481). `drawing`: a line is being drawn. */
static void replay_apply(Replay* s, uint32_t i, int drawing) {
    const uint32_t w1 = s->ev[2u * i + 1u], val = w1 & 0xFFu, aux = (w1 >> 8) & 0xFFu;
    switch (ev_kind(s, i)) {
        case NES_EV_CTRL: s->ctrl = val; s->t = (s->t & 0xF3FFu) | ((val & 3u) << 10); break;
        case NES_EV_MASK: s->mask = val; break;
        case NES_EV_SCROLL:
            if (aux == 0) {
                s->t = (s->t & 0xFFE0u) | (val >> 3);
                s->fx = val & 7u;
            } else {
                s->t = (s->t & 0x0C1Fu) | ((val & 7u) << 12) | ((val & 0xF8u) << 2);
            }
            break;
        case NES_EV_ADDR:
            if (aux == 0) {
                s->t = (s->t & 0x00FFu) | ((val & 0x3Fu) << 8);
            } else {
                s->t = (s->t & 0xFF00u) | val;
                s->v = s->t;
            }
            break;
        case NES_EV_DATA: s->v = (s->v + (aux + 1u) * inc_of(s)) & 0x7FFFu; break;
        case NES_EV_DREAD:
            if (drawing && rendering(s)) y_step(s);
            else s->v = (s->v + inc_of(s)) & 0x7FFFu;
            break;
        case NES_EV_PAL:
            s->pal[aux & 31u] = (uint8_t)val;
            s->v = (s->v + inc_of(s)) & 0x7FFFu;
            break;
        case NES_EV_CHR: s->chr_off[aux & 7u] = val * 1024u; break;
        case NES_EV_MIRROR:
            for (int k = 0; k < 4; ++k) s->nt_map[k] = (uint8_t)((val >> (2 * k)) & 3u);
            break;
        case NES_EV_MMC2:
            if (aux < 4u) {
                s->creg[aux] = val;
                replay_mmc2_select(s, aux >> 1);
            } else if (aux == 6u || aux == 7u) {
                s->latch[aux - 6u] = val & 1u;
                replay_mmc2_select(s, aux - 6u);
            }
            break;
        default: break;
    }
}

/* The replay of the console's logged frame, from its header (patch:1361-1383), over the console's nametables and
 * OAM as they are now; `n` events of the log. */
static void replay_load(Replay* s, const NesRec* r, const NesCart* c, uint32_t n) {
    memset(s, 0, sizeof(*s));
    const uint32_t* h = r->log;
    s->r = r;
    s->c = c;
    s->ev = h + NES_LOG_HDR_WORDS;
    s->count = n < NES_LOG_EVENTS ? n : NES_LOG_EVENTS;
    s->kook = (h[5] & NES_LOG_KOOK) != 0;
    s->ctrl = h[1] & 0xFFu;
    s->mask = (h[1] >> 8) & 0xFFu;
    s->fx = (h[1] >> 16) & 7u;
    s->v = h[2] & 0x7FFFu;
    s->t = (h[2] >> 16) & 0x7FFFu;
    for (int i = 0; i < 8; ++i) s->chr_off[i] = ((h[3 + (i >> 2)] >> ((i & 3) * 8)) & 0xFFu) * 1024u;
    for (int k = 0; k < 4; ++k) s->nt_map[k] = (uint8_t)((h[5] >> (2 * k)) & 3u);
    for (int i = 0; i < 32; ++i) s->pal[i] = (uint8_t)(h[6 + (i >> 2)] >> ((i & 3) * 8));
    s->mmc2 = c->board == NES_BOARD_MMC2;
    s->chr_pages = c->chr_size / 1024u;
    for (int i = 0; i < 4; ++i) s->creg[i] = (h[14] >> (8 * i)) & 0xFFu;
    s->latch[0] = h[15] & 1u;
    s->latch[1] = (h[15] >> 8) & 1u;
    s->sphitx = NO_CHECK;
    s->hit_x = -1;
}

/* The pre-render line: the writes before line 0's lead-in, then v = t while rendering (patch:1483-1490). */
static void replay_begin_frame(Replay* s) {
    while (s->cur < s->count && ev_start(s, s->cur) < -NES_LINE_LEAD) replay_apply(s, s->cur++, 0);
    if (rendering(s)) s->v = s->t;
}

/* Tile slots [ln->tile, last) of the current line (FCEUmm's tile loop, patch:1496-1577). Slot k >= 2 first
 * shifts out 8 pixels of the two tiles fetched before it at the output position, then slot k's tile is fetched at
 * v and v steps one tile right. With rendering off the slots draw the backdrop and still move the output position,
 * the two prefetch slots included. The oracle fetches every slot also without pixels: only the last two fetches of
 * a run and the MMC2 latches outlast it, and both come out the same. */
static void replay_tiles(Replay* s, Line* ln, int last, int pixels) {
    const int first = ln->tile;
    const uint8_t back = (uint8_t)((s->pal[0] & 0x3Fu) | 0x40u);
    if (!rendering(s)) {
        if (pixels)
            for (int p = ln->out; p < ln->out + 8 * (last - first) && p < 256; ++p) ln->px[p] = back;
        ln->out += 8 * (last - first);
        ln->tile = last;
        return;
    }
    for (int k = first; k < last; ++k) {
        if (k >= 2) {
            if (pixels && ln->out < 256) {
                const uint32_t lo = (s->sh_lo >> (8u - s->fx)) & 0xFFu, hi = (s->sh_hi >> (8u - s->fx)) & 0xFFu;
                for (uint32_t q = 0; q < 8u; ++q) {
                    const uint32_t val = ((lo >> (7u - q)) & 1u) | (((hi >> (7u - q)) & 1u) << 1);
                    const uint32_t sel = q + s->fx < 8u ? (s->at & 3u) : ((s->at >> 2) & 3u);
                    ln->px[ln->out + (int)q] = val ? (uint8_t)(s->pal[sel * 4u + val] & 0x3Fu) : back;
                }
            }
            ln->out += 8;
        }
        const uint32_t v = s->v, base = 0x2000u | (v & 0x0C00u);
        const uint32_t tile = rp_nt(s, base | (v & 0x3FFu));
        const uint32_t col = v & 0x1Fu;
        const uint32_t attr = rp_nt(s, base | 0x3C0u | (col >> 2) | ((v & 0x380u) >> 4));
        const uint32_t sel = (attr >> ((col & 2u) | ((v & 0x40u) >> 4))) & 3u;
        const uint32_t pa = tile * 16u + ((s->ctrl & 0x10u) << 8) + ((v >> 12) & 7u);
        const uint32_t p0 = rp_chr(s, pa), p1 = rp_chr(s, pa + 8u);   /* both through the bank before the hook */
        replay_hook(s, pa);
        s->at = (s->at >> 2) | (sel << 2);
        s->sh_lo = (s->sh_lo << 8) | p0;
        s->sh_hi = (s->sh_hi << 8) | p1;
        s->v = col == 0x1Fu ? (v ^ 0x41Fu) : (v + 1u);
    }
    if (pixels) {
        if (first <= 2 && last > 2 && !(s->mask & 0x02u))   /* left column of the background hidden */
            for (int p = 0; p < 8; ++p) ln->px[p] = back;
        if (!(s->mask & 0x08u)) {                            /* background off (sprites on) */
            int from = first - 2, n = last - first;
            if (from < 0) {
                n += from;
                from = 0;
            }
            for (int p = 8 * from; p < 8 * (from + n) && p < 256; ++p) ln->px[p] = back;
        }
    }
    ln->tile = last;
}

/* The sprite-0 check against the background drawn left of line position p - 16 (patch:1583-1594). */
static void replay_check_hit(Replay* s, const Line* ln, int p) {
    if (s->sphitx == NO_CHECK) return;
    for (int x = s->sphitx; x < s->sphitx + 8 && x < p - 16 && x < 255; ++x) {
        if ((s->sphit_bits & (0x80u >> (x - s->sphitx))) && !(ln->px[x] & 0x40u)) {
            s->hit = 1;
            s->hit_x = x;
            s->sphitx = NO_CHECK;
            return;
        }
    }
}

/* The line drawn up to position p (FCEUmm's RefreshLine for an access at p, patch:1596-1613): the tile slots up
 * to p / 8, one more while the sprite-0 check waits on the slot being drawn, the line's vertical step once p
 * reaches 268, then the check. */
static void replay_update(Replay* s, Line* ln, int p, int pixels) {
    int last = p >> 3;
    if (pixels && s->sphitx != NO_CHECK && s->sphitx < p - 16 && s->sphitx >= (last - 2) * 8) ++last;
    if (last > 34) last = 34;
    if (last <= ln->tile) return;
    replay_tiles(s, ln, last, pixels);
    if (p >= 268 && ln->fix) {
        if (rendering(s)) y_step(s);
        ln->fix = 0;
    }
    if (pixels) replay_check_hit(s, ln, p);
}

/* Line l: its pixels with every write that lands while it is drawn, each at the end of its instruction; $2007
 * writes draw nothing first (patch:1617-1634). */
static void replay_line(Replay* s, Line* ln, int l, int pixels) {
    const int start = l * 341 - NES_LINE_LEAD;
    ln->tile = 0;
    ln->out = 0;
    ln->fix = 1;
    if (pixels) memset(ln->px, 0xFF, sizeof(ln->px));
    while (s->cur < s->count && ev_start(s, s->cur) < start + 272) {
        const uint32_t kind = ev_kind(s, s->cur);
        if (kind != NES_EV_DATA && kind != NES_EV_PAL) replay_update(s, ln, ev_end(s, s->cur) - start, pixels);
        replay_apply(s, s->cur++, 1);
    }
    replay_update(s, ln, 272, pixels);
    if (ln->fix) {
        if (rendering(s)) y_step(s);
        ln->fix = 0;
    }
    if (pixels) replay_check_hit(s, ln, 272);
}

/* The sprites of the line (if sprites are on at its end), then greyscale; returns the line's emphasis bits
 * (patch:1637-1661). Each pixel takes the lowest-numbered opaque sprite on it, drawn over a transparent background
 * or when in front. */
static uint32_t replay_compose(Replay* s, Line* ln) {
    if ((s->mask & 0x10u) && s->spork) {
        s->spork = 0;
        const SprLine* d = &s->drawn;
        for (uint32_t x = (s->mask & 0x04u) ? 0u : 8u; x < 256u; ++x) {
            for (uint32_t n = 0; n < d->n; ++n) {
                const uint32_t col = x - d->x[n];
                if (col >= 8u) continue;
                const uint32_t b = (d->attr[n] & 0x40u) ? col : 7u - col;
                const uint32_t val = ((d->lo[n] >> b) & 1u) | (((d->hi[n] >> b) & 1u) << 1);
                if (val == 0) continue;
                if (!(d->attr[n] & 0x20u) || (ln->px[x] & 0x40u)) ln->px[x] = s->spal[(d->attr[n] & 3u) * 4u + val];
                break;
            }
        }
    }
    const uint8_t keep = (s->mask & 0x01u) && rendering(s) ? 0x30u : 0x3Fu;
    for (int x = 0; x < 256; ++x) ln->px[x] &= keep;
    return s->mask >> 5;
}

/* After line l's pixels (patch:1666-1730): the sprites of line l + 1 fetched with the state of that moment (up to
 * eight, OAM order), the writes up to dot 262 of the line grid, the horizontal copy from t, the writes up to its end,
 * and, with sprites on, the fetched line becomes the one drawn next, with its palette and sprite-0 check. `sprites`
 * 0 skips the fetch where no later line can need it (not on MMC2, whose latches every fetch moves). */
static void replay_end_of_line(Replay* s, int l, int sprites) {
    const int start = l * 341 - NES_LINE_LEAD;
    s->sphitx = NO_CHECK;
    if (rendering(s) && (sprites || s->mmc2)) {
        const uint32_t ctrl = s->ctrl, h = (ctrl & 0x20u) ? 16u : 8u;
        const uint32_t table8 = (ctrl & 0x08u) && !(ctrl & 0x20u) ? 0x1000u : 0u;
        SprLine* f = &s->fetched;
        f->n = 0;
        s->blurp = 0;
        for (uint32_t i = 0; i < 64u; ++i) {
            const uint8_t* o = s->r->oam + 4u * i;
            const uint32_t row = (uint32_t)(l - (int)o[0]);
            if (row >= h) continue;
            if (f->n >= 8u) break;
            if (i == 0) s->blurp = 1;
            uint32_t pa = h == 16u ? ((o[1] & 1u) << 12) + ((o[1] & 0xFEu) << 4) : ((uint32_t)o[1] << 4) + table8;
            if (o[2] & 0x80u) pa += 7u - row + ((ctrl & 0x20u) >> 1) - (row & 8u);   /* vertical flip */
            else pa += row + (row & 8u);
            pa &= 0x1FFFu;
            f->lo[f->n] = rp_chr(s, pa);
            f->hi[f->n] = rp_chr(s, pa + 8u);
            replay_hook(s, pa);
            f->attr[f->n] = o[2];
            f->x[f->n] = o[3];
            ++f->n;
        }
    }
    while (s->cur < s->count && ev_start(s, s->cur) < start + 278) replay_apply(s, s->cur++, 1);
    if (rendering(s)) s->v = (s->v & 0xFBE0u) | (s->t & 0x041Fu);
    while (s->cur < s->count && ev_start(s, s->cur) < start + 341) replay_apply(s, s->cur++, 1);
    if (s->mask & 0x10u) {
        s->spork = 0;
        if (s->fetched.n != 0) {
            s->drawn = s->fetched;
            for (int i = 0; i < 16; ++i) s->spal[i] = (uint8_t)(s->pal[16 + i] & 0x3Fu);
            const uint32_t bits = s->drawn.lo[0] | s->drawn.hi[0];
            if (s->blurp && !s->hit && bits) {
                uint32_t b = bits;
                if (s->drawn.attr[0] & 0x40u) {   /* flipped: mirror the byte */
                    b = 0;
                    for (int k = 0; k < 8; ++k) b |= ((bits >> k) & 1u) << (7 - k);
                }
                s->sphitx = s->drawn.x[0];
                s->sphit_bits = b;
            }
            s->spork = 1;
        }
    }
}

void orc_render_full(const NesRec* r, const NesCart* c, uint8_t* pix, uint8_t* emph) {
    Replay s;
    Line ln;
    replay_load(&s, r, c, r->log_n);
    replay_begin_frame(&s);
    for (int l = 0; l < 240; ++l) {
        replay_line(&s, &ln, l, 1);
        emph[l] = (uint8_t)(replay_compose(&s, &ln) & 7u);
        memcpy(pix + 256 * l, ln.px, 256);
        replay_end_of_line(&s, l, 1);
    }
}

/* The env's picture (rl/csrc/nes_machine.cuh:133-155): lines 8..231, x 8..247. */
void orc_render_obs(const NesRec* r, const NesCart* c, uint8_t* obs, uint8_t* emph) {
    Replay s;
    Line ln;
    replay_load(&s, r, c, r->log_n);
    replay_begin_frame(&s);
    for (int l = 0; l < 232; ++l) {
        replay_line(&s, &ln, l, 1);
        const uint32_t e = replay_compose(&s, &ln);
        if (l >= 8) {
            for (int x = 0; x < 240; ++x) obs[(l - 8) * 240 + x] = ln.px[8 + x] & 0x3Fu;
            emph[l - 8] = (uint8_t)(e & 7u);
        }
        replay_end_of_line(&s, l, 1);
    }
}

/* The first line position >= x + 17 whose RefreshLine has drawn pixel x (patch:1743-1750): the position from which
 * an access sees a hit found at x. */
static int first_seen(int x, int sphitx) {
    for (int p = x + 17;; ++p) {
        int last = p >> 3;
        if (sphitx < p - 16 && sphitx >= (last - 2) * 8) ++last;
        if (last > 34) last = 34;
        if (x < (last - 2) * 8) return p;
    }
}

/* The frame's sprite-0 hit from the log so far (patch:1752-1788): replays up to sprite 0's last line (pixels from
 * its first) and returns the NeSLE frame dot from which an instruction sees the flag, *hit = 1. An access is stamped
 * with its instruction's end, so a 4-cycle $2002 read that starts 12 dots earlier sees it. With no hit: the dot
 * after which no write can add one (the end of sprite 0's lines), or 0 when sprite 0 is below the picture. */
uint32_t orc_sprite0_hit(const NesRec* r, const NesCart* c, int* hit) {
    *hit = 0;
    const int first = (int)r->oam[0] + 1;
    if (first >= 240) return 0;
    Replay s;
    Line ln;
    replay_load(&s, r, c, r->log_n);
    replay_begin_frame(&s);
    const int last = first + 15 < 239 ? first + 15 : 239;
    for (int l = 0; l <= last; ++l) {
        const int sphitx = s.sphitx;
        replay_line(&s, &ln, l, l >= first);
        if (s.hit) {
            *hit = 1;
            return (uint32_t)(l * 341 - NES_LINE_LEAD + first_seen(s.hit_x, sphitx) - 12 - NES_FCEU_LAG);
        }
        s.spork = 0;
        replay_end_of_line(&s, l, l >= first - 1);
    }
    return (uint32_t)(last * 341 + 256 - NES_FCEU_LAG);
}

/* MMC2 at vblank: the latches this frame's own pattern fetches leave (NeSLE's frame_resolve_mmc2, patch:1790-1812,
 * which the reference env runs right after the vblank stop, rl/csrc/nes_machine.cuh:110-131). */
static void mmc2_resolve(NesRec* r, const NesCart* c) {
    Replay s;
    Line ln;
    replay_load(&s, r, c, r->log_n);
    replay_begin_frame(&s);
    for (int l = 0; l < 240; ++l) {
        replay_line(&s, &ln, l, 0);
        replay_end_of_line(&s, l, 1);
    }
    while (s.cur < s.count) replay_apply(&s, s.cur++, 0);
    r->mreg[6] = (uint8_t)s.latch[0];
    r->mreg[7] = (uint8_t)s.latch[1];
    mapper_sync(r, c);
}

void orc_mmc2_resolve(NesRec* r, const NesCart* c) { mmc2_resolve(r, c); }

/* ------------------------------------------------------------------------------------------ PPU events */

static uint64_t abs_dot(const NesRec* r) { return (uint64_t)r->frame * NES_FRAME_DOTS + r->frame_dot; }

/* Dots from the current frame dot to the next MMC3 counter clock (dot 266 of lines 0-239, dot 256 of the
 * pre-render line), strictly after it (patch:1881-1903). */
static uint32_t dots_to_mmc3_clock(uint32_t cur) {
    const uint32_t line = cur / 341u, d = cur % 341u;
    if (line < 240u) {
        if (d < 266u) return 266u - d;
        if (line + 1u < 240u) return 341u - d + 266u;
        return (261u - line) * 341u + 256u - d;
    }
    if (line < 261u) return (261u - line) * 341u + 256u - d;
    if (d < 256u) return 256u - d;
    return 341u - d + 266u;
}

/* Dots to the next PPU event (patch:2001-2037): the frame wrap, vblank, pre-render, the $2002 flag set and clear
 * dots, the scheduled sprite-0 check and the MMC3 clocks. A short frame ends a dot early. */
static uint32_t dots_to_event(const NesRec* r, const NesCart* c) {
    const uint32_t cur = r->frame_dot, skip = (r->log_flags & NES_LOG_SHORT) ? 1u : 0u;
    const uint32_t frame = NES_FRAME_DOTS - skip;
#define DIST(e) ((e) > cur ? (e) - cur : frame - cur + (e))
    uint32_t next = frame - cur, d;
    if ((d = DIST(NES_VBLANK_DOT)) < next) next = d;
    if ((d = DIST(NES_PRERENDER_DOT)) < next) next = d;
    if ((d = DIST(NES_VFLAG_DOT)) < next) next = d;
    if ((d = DIST(NES_SCLR_DOT)) < next) next = d;
    const uint32_t s0 = r->s0_sched & NES_S0_DOT;
    if (s0 != 0 && (d = DIST(s0)) < next) next = d;
#undef DIST
    if (c->board == NES_BOARD_MMC3) {
        uint32_t clk = dots_to_mmc3_clock(cur);
        if (cur + clk >= NES_FRAME_DOTS) clk -= skip;
        if (clk < next) next = clk;
    }
    return next;
}

/* The PPU over `dots` dots from the current frame dot (NeSLE's settle, patch:2040-2156): every event in the span,
 * per frame in this order: the sprite-0 check, the $2002 vblank flag, vblank (NMI; MMC2's latch resolve), the $2002
 * clear, the pre-render line (log capture, the frame's sprite-0 check scheduled at sprite 0's first line); then the
 * span's MMC3 clocks. */
static void ppu_step(NesRec* r, const NesCart* c, uint32_t dots) {
    const uint32_t start = r->frame_dot;
    uint32_t end = start + dots;
    if ((r->log_flags & NES_LOG_SHORT) && end >= NES_FRAME_DOTS - 1u) end += 1u;   /* the skipped last dot */
    const uint32_t frames = end / NES_FRAME_DOTS;
    for (uint32_t f = 0; f <= frames; ++f) {
        const uint32_t base = f * NES_FRAME_DOTS;
#define CROSSED(e) (base + (e) > start && base + (e) <= end)
        const uint32_t sched = r->s0_sched, s0 = sched & NES_S0_DOT;
        if (s0 != 0 && CROSSED(s0)) {
            /* worked out again with the writes logged so far, unless nothing was logged since the last answer */
            int hit;
            uint32_t dot;
            if ((sched & NES_S0_KNOWN) && ((sched >> 20) & 0x1FFu) == r->log_n) {
                dot = s0;
                hit = (sched & NES_S0_HIT) != 0;
            } else {
                dot = orc_sprite0_hit(r, c, &hit);
            }
            const int reached = base + dot <= end;
            if (hit && reached) r->status |= 0x40u;
            r->s0_sched = dot != 0 && !reached
                              ? dot | NES_S0_KNOWN | (hit ? NES_S0_HIT : 0u) | ((uint32_t)r->log_n << 20)
                              : 0u;
        }
        if (CROSSED(NES_VFLAG_DOT)) r->status |= 0x80u;
        if (CROSSED(NES_VBLANK_DOT)) {   /* NMI 12 dots after the flag, whether or not a read took it */
            if (r->ctrl & 0x80u) r->nmi_pending = 1;
            if (c->board == NES_BOARD_MMC2) mmc2_resolve(r, c);
        }
        if (CROSSED(NES_SCLR_DOT)) r->status &= 0x1Fu;
        if (CROSSED(NES_PRERENDER_DOT)) {
            r->status &= 0x1Fu;
            log_capture(r);
            const uint32_t y = r->oam[0];
            r->s0_sched = y < 239u ? (y + 1u) * 341u - 20u - NES_FCEU_LAG : 0u;
        }
#undef CROSSED
    }
    if (c->board == NES_BOARD_MMC3 && (r->mask & 0x18u) && (r->ctrl & 0x38u) != 0x18u) {
        /* FCEUmm clocks the counter while rendering, unless both pattern tables are at $1000 with 8x8 sprites */
        for (uint32_t la = start / 341u; la <= end / 341u; ++la) {
            const uint32_t line = la % 262u;
            uint32_t at;
            if (line < 240u) at = 266u;
            else if (line == 261u) at = 256u;
            else continue;
            const uint32_t d = la * 341u + at;
            if (d > start && d <= end) mmc3_clock(r);
        }
    }
    r->frame_dot = end % NES_FRAME_DOTS;
    r->frame += frames;
    if (frames) r->log_flags &= (uint8_t)~NES_LOG_SHORT;
}

/* ------------------------------------------------------------------------------------------------- bus */

typedef struct Bus {
    NesRec* r;
    const NesCart* c;
    uint32_t now;    /* NeSLE frame dot at which this instruction starts (its log stamp) */
    int log_on;      /* the instruction starts while a frame is logged: before vblank or from the pre-render line */
    int dma;         /* a $4014 write happened */
} Bus;

static void log_event(Bus* b, uint32_t kind, uint32_t value, uint32_t aux) {
    NesRec* r = b->r;
    if (!b->log_on) return;
    uint32_t* h = r->log;
    uint32_t* ev = h + NES_LOG_HDR_WORDS;
    if (kind == NES_EV_DATA && (r->mask & 0x18u) == 0 && r->log_n > 0) {
        uint32_t* last = ev + 2u * (r->log_n - 1u);
        if ((last[0] & 15u) == NES_EV_DATA && (last[1] >> 8) < 0xFFu) {
            last[1] += 0x100u;
            return;
        }
    }
    if (r->log_n >= NES_LOG_EVENTS) {
        h[0] |= NES_LOG_OVERFLOW;
        return;
    }
    ev[2u * r->log_n] = NES_EV_WORD0(kind, b->now & 0x1FFFFu);
    ev[2u * r->log_n + 1u] = (value & 0xFFu) | ((aux & 0xFFu) << 8);
    ++r->log_n;
    h[0] = (h[0] & NES_LOG_OVERFLOW) | r->log_n;
}

static uint8_t ppu_mem_read(const NesRec* r, const NesCart* c, uint32_t a) {
    a &= 0x3FFFu;
    if (a < 0x2000u) return chr_read(r, c, r->chr_off, a);
    if (a < 0x3F00u) return r->nt[(r->nt_map[(a >> 10) & 3u] & 1u) * 1024u + (a & 0x3FFu)];
    uint32_t i = a & 0x1Fu;
    if ((i & 0x13u) == 0x10u) i &= 0x0Fu;
    return r->pal[i];
}

static void ppu_mem_write(Bus* b, uint32_t a, uint8_t v) {
    NesRec* r = b->r;
    a &= 0x3FFFu;
    if (a < 0x2000u) {
        if (!b->c->chr) {
            r->chr_ram[(r->chr_off[(a >> 10) & 7u] + (a & 0x3FFu)) & (NES_CHRRAM_BYTES - 1u)] = v;
        }
        log_event(b, NES_EV_DATA, 0, 0);
    } else if (a < 0x3F00u) {
        r->nt[(r->nt_map[(a >> 10) & 3u] & 1u) * 1024u + (a & 0x3FFu)] = v;
        log_event(b, NES_EV_DATA, 0, 0);
    } else {
        uint32_t i = a & 0x1Fu;
        if ((i & 0x13u) == 0x10u) i &= 0x0Fu;
        r->pal[i] = v & 0x3Fu;
        log_event(b, NES_EV_PAL, v & 0x3Fu, i);
    }
}

/* MMC2: the VRAM address the CPU drives through $2006/$2007 flips a latch; a change is logged for the renderer
 * (patch:615-636, 3196-3220). */
static void mmc2_ppu_address(Bus* b, uint32_t a) {
    NesRec* r = b->r;
    const uint32_t t = b->c->board == NES_BOARD_MMC2 ? mmc2_trigger(a) : 0u;
    if (t == 0) return;
    const uint32_t half = t >> 2, latch = (t & 3u) - 1u;
    if (r->mreg[6 + half] == latch) return;
    r->mreg[6 + half] = (uint8_t)latch;
    mapper_sync(r, b->c);
    log_event(b, NES_EV_MMC2, latch, 6 + half);
}

static uint8_t ppu_reg_read(Bus* b, uint32_t reg) {
    NesRec* r = b->r;
    uint8_t v;
    switch (reg) {
        case 2:
            v = (uint8_t)((r->status & 0xE0u) | (r->open_bus & 0x1Fu));
            r->status &= 0x7Fu;
            r->w = 0;
            break;
        case 4: v = r->oam[r->oam_addr]; break;
        case 7: {
            const uint32_t a = r->v & 0x3FFFu;
            if (a < 0x3F00u) {
                v = r->read_buf;
                mmc2_ppu_address(b, a);
                r->read_buf = ppu_mem_read(r, b->c, a);
            } else {
                v = ppu_mem_read(r, b->c, a);
                r->read_buf = ppu_mem_read(r, b->c, a - 0x1000u);
                mmc2_ppu_address(b, a);
            }
            r->v = (uint16_t)((r->v + ((r->ctrl & 4u) ? 32u : 1u)) & 0x7FFFu);
            log_event(b, NES_EV_DREAD, 0, 0);
            mmc2_ppu_address(b, r->v & 0x3FFFu);
            break;
        }
        default: return r->open_bus;
    }
    r->open_bus = v;
    return v;
}

static void ppu_reg_write(Bus* b, uint32_t reg, uint8_t v) {
    NesRec* r = b->r;
    r->open_bus = v;
    switch (reg) {
        case 0:
            if (!(r->ctrl & 0x80u) && (v & 0x80u) && (r->status & 0x80u)) r->nmi_pending = 1;
            r->ctrl = v;
            r->t = (uint16_t)((r->t & 0xF3FFu) | ((v & 3u) << 10));
            log_event(b, NES_EV_CTRL, v, 0);
            break;
        case 1:
            r->mask = v;
            log_event(b, NES_EV_MASK, v, 0);
            break;
        case 3: r->oam_addr = v; break;
        case 4:
            r->oam[r->oam_addr++] = v;
            break;
        case 5:
            log_event(b, NES_EV_SCROLL, v, r->w);
            if (r->w == 0) {
                r->t = (uint16_t)((r->t & 0xFFE0u) | (v >> 3));
                r->fx = v & 7u;
                r->w = 1;
            } else {
                r->t = (uint16_t)((r->t & 0x0C1Fu) | ((v & 7u) << 12) | ((v & 0xF8u) << 2));
                r->w = 0;
            }
            break;
        case 6:
            log_event(b, NES_EV_ADDR, v, r->w);
            if (r->w == 0) {
                r->t = (uint16_t)((r->t & 0x00FFu) | ((v & 0x3Fu) << 8));
                r->w = 1;
            } else {
                r->t = (uint16_t)((r->t & 0xFF00u) | v);
                r->v = r->t;
                r->w = 0;
                mmc2_ppu_address(b, r->v);
            }
            break;
        case 7:
            ppu_mem_write(b, r->v, v);
            r->v = (uint16_t)((r->v + ((r->ctrl & 4u) ? 32u : 1u)) & 0x7FFFu);
            mmc2_ppu_address(b, r->v & 0x3FFFu);
            break;
        default: break;
    }
}

static uint8_t bus_read(Bus* b, uint16_t a) {
    NesRec* r = b->r;
    if (a < 0x2000u) return r->ram[a & 0x7FFu];
    if (a >= 0x8000u) return b->c->prg[r->prg_off[(a >> 13) & 3u] + (a & 0x1FFFu)];
    if (a < 0x4000u) return ppu_reg_read(b, a & 7u);
    if (a == 0x4015u) return r->dmc_left ? 0x10u : 0x00u;
    if (a == 0x4016u) {
        uint32_t bit;
        if (r->strobe) {
            bit = r->pad & 1u;
        } else {
            bit = r->shift & 1u;
            r->shift = (uint8_t)((r->shift >> 1) | 0x80u);
        }
        return (uint8_t)(0x40u | bit);
    }
    if (a >= 0x6000u) return prg_ram_enabled(r, b->c) ? r->prg_ram[a - 0x6000u] : (uint8_t)(a >> 8);
    return (uint8_t)(a >> 8); /* $4000-$5FFF open bus */
}

static void bus_write(Bus* b, uint16_t a, uint8_t v) {
    NesRec* r = b->r;
    if (a < 0x2000u) {
        r->ram[a & 0x7FFu] = v;
    } else if (a < 0x4000u) {
        ppu_reg_write(b, a & 7u, v);
    } else if (a == 0x4014u) {
        for (uint32_t i = 0; i < 256u; ++i) r->oam[(r->oam_addr + i) & 0xFFu] = bus_read(b, (uint16_t)((v << 8) | i));
        b->dma = 1;
    } else if (a == 0x4016u) {
        r->strobe = v & 1u;
        if (r->strobe) r->shift = r->pad;
    } else if (a == 0x4010u || a == 0x4013u || a == 0x4015u) {
        dmc_write(r, a, v);
    } else if (a >= 0x8000u) {
        uint32_t before[8];
        uint8_t map_before[4], creg_before[4];
        memcpy(before, r->chr_off, sizeof(before));
        memcpy(map_before, r->nt_map, 4);
        memcpy(creg_before, r->mreg, 4);
        mapper_write(r, b->c, a, v);
        for (uint32_t i = 0; i < 8u; ++i)
            if (r->chr_off[i] != before[i]) log_event(b, NES_EV_CHR, r->chr_off[i] >> 10, i);
        if (memcmp(map_before, r->nt_map, 4) != 0) log_event(b, NES_EV_MIRROR, nt_map_packed(r), 0);
        if (b->c->board == NES_BOARD_MMC2)   /* patch:661-664 */
            for (uint32_t i = 0; i < 4u; ++i)
                if (r->mreg[i] != creg_before[i]) log_event(b, NES_EV_MMC2, r->mreg[i], i);
    } else if (a >= 0x6000u) {
        if (prg_ram_enabled(r, b->c)) r->prg_ram[a - 0x6000u] = v;
    }
}

uint8_t orc_bus_read(NesRec* r, const NesCart* c, uint16_t addr) {
    Bus b = {r, c, 0, 0, 0};
    return bus_read(&b, addr);
}
void orc_bus_write(NesRec* r, const NesCart* c, uint16_t addr, uint8_t v) {
    Bus b = {r, c, 0, 0, 0};
    bus_write(&b, addr, v);
}

/* ------------------------------------------------------------------------------------------------ 6502 */

/* Base cycles of the 151 official opcodes; 0 = not implemented (fault). */
static const uint8_t kCycles[256] = {
    /*        0  1  2  3  4  5  6  7  8  9  A  B  C  D  E  F */
    /* 0 */ 7, 6, 0, 0, 0, 3, 5, 0, 3, 2, 2, 0, 0, 4, 6, 0,
    /* 1 */ 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    /* 2 */ 6, 6, 0, 0, 3, 3, 5, 0, 4, 2, 2, 0, 4, 4, 6, 0,
    /* 3 */ 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    /* 4 */ 6, 6, 0, 0, 0, 3, 5, 0, 3, 2, 2, 0, 3, 4, 6, 0,
    /* 5 */ 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    /* 6 */ 6, 6, 0, 0, 0, 3, 5, 0, 4, 2, 2, 0, 5, 4, 6, 0,
    /* 7 */ 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    /* 8 */ 0, 6, 0, 0, 3, 3, 3, 0, 2, 0, 2, 0, 4, 4, 4, 0,
    /* 9 */ 2, 6, 0, 0, 4, 4, 4, 0, 2, 5, 2, 0, 0, 5, 0, 0,
    /* A */ 2, 6, 2, 0, 3, 3, 3, 0, 2, 2, 2, 0, 4, 4, 4, 0,
    /* B */ 2, 5, 0, 0, 4, 4, 4, 0, 2, 4, 2, 0, 4, 4, 4, 0,
    /* C */ 2, 6, 0, 0, 3, 3, 5, 0, 2, 2, 2, 0, 4, 4, 6, 0,
    /* D */ 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    /* E */ 2, 6, 0, 0, 3, 3, 5, 0, 2, 2, 2, 0, 4, 4, 6, 0,
    /* F */ 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
};

typedef struct Cpu {
    Bus* b;
    NesRec* r;
    uint32_t cycles; /* this instruction */
    uint8_t lo, hi;  /* the two bytes after the opcode */
} Cpu;

/* Instruction-stream bytes (opcode, operands, vectors) are fetched without side effects: RAM, PRG RAM and
 * PRG ROM as memory, anything else as open bus (the high address byte). */
static uint8_t fetch(const NesRec* r, const NesCart* c, uint16_t a) {
    if (a < 0x2000u) return r->ram[a & 0x7FFu];
    if (a >= 0x8000u) return c->prg[r->prg_off[(a >> 13) & 3u] + (a & 0x1FFFu)];
    if (a >= 0x6000u && prg_ram_enabled(r, c)) return r->prg_ram[a - 0x6000u];
    return (uint8_t)(a >> 8);
}

static uint8_t rd(Cpu* k, uint16_t a) { return bus_read(k->b, a); }
static void wr(Cpu* k, uint16_t a, uint8_t v) { bus_write(k->b, a, v); }
static void push(Cpu* k, uint8_t v) { k->r->ram[0x100u | k->r->sp] = v; k->r->sp--; }
static uint8_t pull(Cpu* k) { k->r->sp++; return k->r->ram[0x100u | k->r->sp]; }
static void nz(NesRec* r, uint32_t v) {
    r->p = (uint8_t)((r->p & ~(FL_N | FL_Z)) | (v & 0x80u) | ((v & 0xFFu) ? 0 : FL_Z));
}

static void interrupt(Cpu* k, uint16_t vector) {
    NesRec* r = k->r;
    push(k, (uint8_t)(r->pc >> 8));
    push(k, (uint8_t)r->pc);
    push(k, (uint8_t)((r->p & ~FL_B) | FL_U));
    r->p |= FL_I;
    r->pc = (uint16_t)(fetch(r, k->b->c, vector) | (fetch(r, k->b->c, (uint16_t)(vector + 1)) << 8));
}

/* addressing modes, from the fetched operand bytes */
static uint16_t ea_zp(Cpu* k) { return k->lo; }
static uint16_t ea_zpx(Cpu* k) { return (uint16_t)((k->lo + k->r->x) & 0xFFu); }
static uint16_t ea_zpy(Cpu* k) { return (uint16_t)((k->lo + k->r->y) & 0xFFu); }
static uint16_t ea_abs(Cpu* k) { return (uint16_t)(k->lo | (k->hi << 8)); }
static uint16_t ea_abi(Cpu* k, uint8_t idx, int penalty) {
    const uint16_t base = ea_abs(k), a = (uint16_t)(base + idx);
    if (penalty && ((base ^ a) & 0xFF00u)) k->cycles++;
    return a;
}
static uint16_t ea_izx(Cpu* k) {
    const uint32_t p = (k->lo + k->r->x) & 0xFFu;
    return (uint16_t)(k->r->ram[p] | (k->r->ram[(p + 1u) & 0xFFu] << 8));
}
static uint16_t ea_izy(Cpu* k, int penalty) {
    const uint32_t p = k->lo;
    const uint16_t base = (uint16_t)(k->r->ram[p] | (k->r->ram[(p + 1u) & 0xFFu] << 8));
    const uint16_t a = (uint16_t)(base + k->r->y);
    if (penalty && ((base ^ a) & 0xFF00u)) k->cycles++;
    return a;
}

static void adc(NesRec* r, uint32_t m) {
    const uint32_t s = r->a + m + (r->p & FL_C);
    const uint32_t v = (~(r->a ^ m) & (r->a ^ s) & 0x80u) ? FL_V : 0;
    r->p = (uint8_t)((r->p & ~(FL_C | FL_V)) | (s > 0xFFu ? FL_C : 0) | v);
    r->a = (uint8_t)s;
    nz(r, r->a);
}
static void cmp(NesRec* r, uint32_t reg, uint32_t m) {
    r->p = (uint8_t)((r->p & ~FL_C) | (reg >= m ? FL_C : 0));
    nz(r, (reg - m) & 0xFFu);
}

/* read-modify-write kinds */
enum { RMW_ASL, RMW_LSR, RMW_ROL, RMW_ROR, RMW_INC, RMW_DEC };
static uint8_t rmw(NesRec* r, int kind, uint32_t m) {
    uint32_t out;
    switch (kind) {
        case RMW_ASL: r->p = (uint8_t)((r->p & ~FL_C) | (m >> 7)); out = (m << 1) & 0xFFu; break;
        case RMW_LSR: r->p = (uint8_t)((r->p & ~FL_C) | (m & 1u)); out = m >> 1; break;
        case RMW_ROL: out = ((m << 1) | (r->p & FL_C)) & 0xFFu; r->p = (uint8_t)((r->p & ~FL_C) | (m >> 7)); break;
        case RMW_ROR: out = (m >> 1) | ((r->p & FL_C) << 7); r->p = (uint8_t)((r->p & ~FL_C) | (m & 1u)); break;
        case RMW_INC: out = (m + 1u) & 0xFFu; break;
        default: out = (m - 1u) & 0xFFu; break;
    }
    nz(r, out);
    return (uint8_t)out;
}

static void branch(Cpu* k, int cond) {
    NesRec* r = k->r;
    const uint16_t next = (uint16_t)(r->pc + 2);
    if (cond) {
        const uint16_t target = (uint16_t)(next + (int8_t)k->lo);
        k->cycles += ((next ^ target) & 0xFF00u) ? 2u : 1u;
        r->pc = target;
    } else {
        r->pc = next;
    }
}

/* The effective address of a memory operand by (opcode) for read-modify-write. */
static uint16_t ea_rmw(Cpu* k, uint8_t op, uint16_t* len) {
    switch (op & 0x1Cu) {
        case 0x04: *len = 2; return ea_zp(k);
        case 0x0C: *len = 3; return ea_abs(k);
        case 0x14: *len = 2; return ea_zpx(k);
        default: *len = 3; return ea_abi(k, k->r->x, 0); /* 0x1C */
    }
}

/* Executes instruction `op` at pc. Returns 0 on an unimplemented opcode. Data accesses that the frame log
 * may record are stamped with the instruction's end: every penalty cycle is known before them. */
static int execute(Cpu* k, uint8_t op) {
    NesRec* r = k->r;
    Bus* b = k->b;
    const uint32_t base = kCycles[op];
    if (base == 0) return 0;
    k->cycles = base;
    uint16_t len = 1, a;
    uint8_t m;
    switch (op) {
        /* ---- group 1: ORA AND EOR ADC LDA CMP SBC (STA below) ---- */
        case 0x01: case 0x05: case 0x09: case 0x0D: case 0x11: case 0x15: case 0x19: case 0x1D:
        case 0x21: case 0x25: case 0x29: case 0x2D: case 0x31: case 0x35: case 0x39: case 0x3D:
        case 0x41: case 0x45: case 0x49: case 0x4D: case 0x51: case 0x55: case 0x59: case 0x5D:
        case 0x61: case 0x65: case 0x69: case 0x6D: case 0x71: case 0x75: case 0x79: case 0x7D:
        case 0xA1: case 0xA5: case 0xA9: case 0xAD: case 0xB1: case 0xB5: case 0xB9: case 0xBD:
        case 0xC1: case 0xC5: case 0xC9: case 0xCD: case 0xD1: case 0xD5: case 0xD9: case 0xDD:
        case 0xE1: case 0xE5: case 0xE9: case 0xED: case 0xF1: case 0xF5: case 0xF9: case 0xFD: {
            switch ((op >> 2) & 7u) {
                case 0: m = rd(k, ea_izx(k)); len = 2; break;
                case 1: m = rd(k, ea_zp(k)); len = 2; break;
                case 2: m = k->lo; len = 2; break;
                case 3: m = rd(k, ea_abs(k)); len = 3; break;
                case 4: a = ea_izy(k, 1); m = rd(k, a); len = 2; break;
                case 5: m = rd(k, ea_zpx(k)); len = 2; break;
                case 6: a = ea_abi(k, r->y, 1); m = rd(k, a); len = 3; break;
                default: a = ea_abi(k, r->x, 1); m = rd(k, a); len = 3; break;
            }
            switch (op >> 5) {
                case 0: r->a |= m; nz(r, r->a); break;
                case 1: r->a &= m; nz(r, r->a); break;
                case 2: r->a ^= m; nz(r, r->a); break;
                case 3: adc(r, m); break;
                case 5: r->a = m; nz(r, m); break;
                case 6: cmp(r, r->a, m); break;
                default: adc(r, m ^ 0xFFu); break;
            }
            break;
        }
        /* ---- stores ---- */
        case 0x81: wr(k, ea_izx(k), r->a); len = 2; break;
        case 0x85: wr(k, ea_zp(k), r->a); len = 2; break;
        case 0x8D: wr(k, ea_abs(k), r->a); len = 3; break;
        case 0x91: wr(k, ea_izy(k, 0), r->a); len = 2; break;
        case 0x95: wr(k, ea_zpx(k), r->a); len = 2; break;
        case 0x99: wr(k, ea_abi(k, r->y, 0), r->a); len = 3; break;
        case 0x9D: wr(k, ea_abi(k, r->x, 0), r->a); len = 3; break;
        case 0x86: wr(k, ea_zp(k), r->x); len = 2; break;
        case 0x8E: wr(k, ea_abs(k), r->x); len = 3; break;
        case 0x96: wr(k, ea_zpy(k), r->x); len = 2; break;
        case 0x84: wr(k, ea_zp(k), r->y); len = 2; break;
        case 0x8C: wr(k, ea_abs(k), r->y); len = 3; break;
        case 0x94: wr(k, ea_zpx(k), r->y); len = 2; break;
        /* ---- loads X/Y, compares X/Y, BIT ---- */
        case 0xA2: case 0xA6: case 0xAE: case 0xB6: case 0xBE:
        case 0xA0: case 0xA4: case 0xAC: case 0xB4: case 0xBC:
        case 0xE0: case 0xE4: case 0xEC: case 0xC0: case 0xC4: case 0xCC:
        case 0x24: case 0x2C: {
            switch (op) {
                case 0xA2: case 0xA0: case 0xE0: case 0xC0: m = k->lo; len = 2; break;
                case 0xA6: case 0xA4: case 0xE4: case 0xC4: case 0x24: m = rd(k, ea_zp(k)); len = 2; break;
                case 0xAE: case 0xAC: case 0xEC: case 0xCC: case 0x2C: m = rd(k, ea_abs(k)); len = 3; break;
                case 0xB6: m = rd(k, ea_zpy(k)); len = 2; break;
                case 0xB4: m = rd(k, ea_zpx(k)); len = 2; break;
                case 0xBE: a = ea_abi(k, r->y, 1); m = rd(k, a); len = 3; break;
                default: a = ea_abi(k, r->x, 1); m = rd(k, a); len = 3; break;
            }
            switch (op) {
                case 0xA2: case 0xA6: case 0xAE: case 0xB6: case 0xBE: r->x = m; nz(r, m); break;
                case 0xA0: case 0xA4: case 0xAC: case 0xB4: case 0xBC: r->y = m; nz(r, m); break;
                case 0xE0: case 0xE4: case 0xEC: cmp(r, r->x, m); break;
                case 0xC0: case 0xC4: case 0xCC: cmp(r, r->y, m); break;
                default:
                    r->p = (uint8_t)((r->p & ~(FL_N | FL_V | FL_Z)) | (m & 0xC0u) | ((r->a & m) ? 0 : FL_Z));
                    break;
            }
            break;
        }
        /* ---- read-modify-write on memory ---- */
        case 0x06: case 0x0E: case 0x16: case 0x1E: case 0x26: case 0x2E: case 0x36: case 0x3E:
        case 0x46: case 0x4E: case 0x56: case 0x5E: case 0x66: case 0x6E: case 0x76: case 0x7E:
        case 0xC6: case 0xCE: case 0xD6: case 0xDE: case 0xE6: case 0xEE: case 0xF6: case 0xFE: {
            static const int kinds[8] = {RMW_ASL, RMW_ROL, RMW_LSR, RMW_ROR, 0, 0, RMW_DEC, RMW_INC};
            a = ea_rmw(k, op, &len);
            m = rd(k, a);
            wr(k, a, rmw(r, kinds[op >> 5], m));
            break;
        }
        case 0x0A: r->a = rmw(r, RMW_ASL, r->a); break;
        case 0x2A: r->a = rmw(r, RMW_ROL, r->a); break;
        case 0x4A: r->a = rmw(r, RMW_LSR, r->a); break;
        case 0x6A: r->a = rmw(r, RMW_ROR, r->a); break;
        /* ---- branches ---- */
        case 0x10: branch(k, !(r->p & FL_N)); return 1;
        case 0x30: branch(k, (r->p & FL_N) != 0); return 1;
        case 0x50: branch(k, !(r->p & FL_V)); return 1;
        case 0x70: branch(k, (r->p & FL_V) != 0); return 1;
        case 0x90: branch(k, !(r->p & FL_C)); return 1;
        case 0xB0: branch(k, (r->p & FL_C) != 0); return 1;
        case 0xD0: branch(k, !(r->p & FL_Z)); return 1;
        case 0xF0: branch(k, (r->p & FL_Z) != 0); return 1;
        /* ---- flags, transfers, register inc/dec ---- */
        case 0x18: r->p &= (uint8_t)~FL_C; break;
        case 0x38: r->p |= FL_C; break;
        case 0x58: r->p &= (uint8_t)~FL_I; break;
        case 0x78: r->p |= FL_I; break;
        case 0xB8: r->p &= (uint8_t)~FL_V; break;
        case 0xD8: r->p &= (uint8_t)~FL_D; break;
        case 0xF8: r->p |= FL_D; break;
        case 0xAA: r->x = r->a; nz(r, r->x); break;
        case 0xA8: r->y = r->a; nz(r, r->y); break;
        case 0x8A: r->a = r->x; nz(r, r->a); break;
        case 0x98: r->a = r->y; nz(r, r->a); break;
        case 0xBA: r->x = r->sp; nz(r, r->x); break;
        case 0x9A: r->sp = r->x; break;
        case 0xE8: r->x++; nz(r, r->x); break;
        case 0xC8: r->y++; nz(r, r->y); break;
        case 0xCA: r->x--; nz(r, r->x); break;
        case 0x88: r->y--; nz(r, r->y); break;
        case 0xEA: break;
        /* ---- stack ---- */
        case 0x48: push(k, r->a); break;
        case 0x08: push(k, (uint8_t)(r->p | FL_B | FL_U)); break;
        case 0x68: r->a = pull(k); nz(r, r->a); break;
        case 0x28: r->p = (uint8_t)((pull(k) & ~FL_B) | FL_U); break;
        /* ---- jumps and calls ---- */
        case 0x4C: r->pc = ea_abs(k); return 1;
        case 0x6C: {
            const uint16_t p = ea_abs(k);
            const uint32_t lo = rd(k, p);
            r->pc = (uint16_t)(lo | (rd(k, (uint16_t)((p & 0xFF00u) | ((p + 1u) & 0xFFu))) << 8));
            return 1;
        }
        case 0x20: {
            const uint16_t ret = (uint16_t)(r->pc + 2);
            push(k, (uint8_t)(ret >> 8));
            push(k, (uint8_t)ret);
            r->pc = ea_abs(k);
            return 1;
        }
        case 0x60: {
            const uint32_t lo = pull(k), hi = pull(k);
            r->pc = (uint16_t)(((hi << 8) | lo) + 1u);
            return 1;
        }
        case 0x40: {
            r->p = (uint8_t)((pull(k) & ~FL_B) | FL_U);
            const uint32_t lo = pull(k), hi = pull(k);
            r->pc = (uint16_t)((hi << 8) | lo);
            return 1;
        }
        case 0x00: {
            const uint16_t ret = (uint16_t)(r->pc + 2);
            push(k, (uint8_t)(ret >> 8));
            push(k, (uint8_t)ret);
            push(k, (uint8_t)(r->p | FL_B | FL_U));
            r->p |= FL_I;
            r->pc = (uint16_t)(fetch(r, b->c, 0xFFFE) | (fetch(r, b->c, 0xFFFF) << 8));
            return 1;
        }
        default: return 0;
    }
    r->pc = (uint16_t)(r->pc + len);
    return 1;
}

/* One step: pending NMI (or an asserted cartridge IRQ with I clear), then one instruction, then the OAM-DMA
 * stall and the DMC service (patch:823-862). `pending` = dots not yet settled. The frame-log events the
 * instruction makes are stamped with its start dot, and with its cycles once it has run (patch:829-836,
 * 1166-1185). */
static uint32_t step(NesRec* r, const NesCart* c, uint32_t pending, uint32_t* fault, uint8_t* op_out,
                     uint16_t* pc_out) {
    Bus b = {r, c, 0, 0, 0};
    Cpu k = {&b, r, 0, 0, 0};
    uint32_t cyc = 0;
    if (r->nmi_pending) {
        r->nmi_pending = 0;
        interrupt(&k, 0xFFFA);
        cyc = 7;
    } else if (r->irq_line && !(r->p & FL_I)) {
        interrupt(&k, 0xFFFE);
        cyc = 7;
    }
    b.now = r->frame_dot + pending + 3u * cyc;
    b.log_on = b.now < NES_VBLANK_DOT || b.now >= NES_PRERENDER_DOT;
    const uint32_t logged = r->log_n;
    *pc_out = r->pc;
    *op_out = fetch(r, c, r->pc);
    k.lo = fetch(r, c, (uint16_t)(r->pc + 1));
    k.hi = fetch(r, c, (uint16_t)(r->pc + 2));
    if (!execute(&k, *op_out)) {
        *fault = ((uint32_t)r->pc << 8) | *op_out;
        return 0;
    }
    for (uint32_t i = logged; i < r->log_n && i < NES_LOG_EVENTS; ++i)
        r->log[NES_LOG_HDR_WORDS + 2u * i] |= (k.cycles > 15u ? 15u : k.cycles) << 4;
    cyc += k.cycles;
    r->cycles += cyc;
    if (b.dma) {
        const uint32_t stall = 513u + (uint32_t)(r->cycles & 1u);
        r->cycles += stall;
        cyc += stall;
    }
    if (r->cycles >= r->dmc_event) {
        const uint32_t s = orc_dmc_service(r, r->cycles, 1);
        r->cycles += s;
        cyc += s;
    }
    return cyc;
}

uint32_t orc_step(NesRec* r, const NesCart* c, uint32_t* fault) {
    uint8_t op;
    uint16_t pc;
    *fault = 0;
    const uint32_t cyc = step(r, c, 0, fault, &op, &pc);
    if (*fault) return 0;
    ppu_step(r, c, 3u * cyc);
    return cyc;
}

/* The JMP-to-self idle loop: skip whole 3-cycle jumps up to the next PPU event (patch:866-893); not with an NMI
 * raised by the settle before it. */
static void fast_forward(NesRec* r, const NesCart* c) {
    if (r->nmi_pending) return;
    const uint32_t to = dots_to_event(r, c);
    const uint32_t jumps = (to + 8u) / 9u;
    if (jumps == 0) return;
    r->cycles += 3u * jumps;
    if (r->cycles >= r->dmc_event) (void)orc_dmc_service(r, r->cycles, 0);
    ppu_step(r, c, 9u * jumps);
}

/* rl/csrc/nes_machine.cuh:67-103: instructions until a settle reaches absolute dot `target`, with the PPU settled
 * lazily at its event horizon and after an idle jump. */
uint32_t orc_run_until_budget(NesRec* r, const NesCart* c, uint64_t target, uint32_t budget) {
    uint32_t instructions = 0, fault = 0, pending = 0;
    uint32_t to_event = dots_to_event(r, c);
    int done = 0;
    while (instructions < budget && !done) {
        if (pending >= to_event) {
            ppu_step(r, c, pending);
            pending = 0;
            to_event = dots_to_event(r, c);
            if (abs_dot(r) >= target) break;
        }
        uint8_t op;
        uint16_t pc0;
        const uint32_t cyc = step(r, c, pending, &fault, &op, &pc0);
        if (fault) break;
        pending += 3u * cyc;
        ++instructions;
        ++r->instr_lo;
        if (op == 0x4C && r->pc == pc0) {
            ppu_step(r, c, pending);
            pending = 0;
            if (abs_dot(r) >= target) break;
            fast_forward(r, c);
            to_event = dots_to_event(r, c);
            done = abs_dot(r) >= target;
        }
    }
    if (pending) ppu_step(r, c, pending);
    return fault;
}

uint32_t orc_run_until(NesRec* r, const NesCart* c, uint64_t target) {
    return orc_run_until_budget(r, c, target, NES_BUDGET);
}
