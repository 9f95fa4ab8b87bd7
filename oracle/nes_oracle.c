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

#define PRE_LINE_START (-341)
#define LOG_WINDOW_START (-340) /* pre-render dot 1 */

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
    r->s0_dot = NES_NO_HIT;
    r->s0_valid = 0;
    orc_dmc_reset(r, r->cycles);
    /* the log of frame 0 starts from the power-on PPU state */
    uint32_t* h = r->log;
    h[1] = 0;
    h[2] = 0;
    for (int i = 0; i < 8; ++i) h[3 + (i >> 2)] |= ((r->chr_off[i] >> 10) & 0xFFu) << ((i & 3) * 8);
    h[5] = nt_map_packed(r);
    r->log_frame = 0;
}

/* ------------------------------------------------------------------------------------- frame log + replay */

static void log_capture(NesRec* r) {
    uint32_t* h = r->log;
    memset(h, 0, NES_LOG_HDR_WORDS * 4u);
    h[1] = r->ctrl | ((uint32_t)r->mask << 8) | ((uint32_t)r->fx << 16);
    h[2] = r->v | ((uint32_t)r->t << 16);
    for (int i = 0; i < 8; ++i) h[3 + (i >> 2)] |= ((r->chr_off[i] >> 10) & 0xFFu) << ((i & 3) * 8);
    h[5] = nt_map_packed(r);
    if (r->board == NES_BOARD_MMC2) {
        h[14] = r->mreg[0] | ((uint32_t)r->mreg[1] << 8) | ((uint32_t)r->mreg[2] << 16) | ((uint32_t)r->mreg[3] << 24);
        h[15] = r->mreg[6] | ((uint32_t)r->mreg[7] << 8);
    }
    for (int i = 0; i < 8; ++i)
        h[6 + i] = r->pal[4 * i] | ((uint32_t)r->pal[4 * i + 1] << 8) | ((uint32_t)r->pal[4 * i + 2] << 16) |
                   ((uint32_t)r->pal[4 * i + 3] << 24);
    r->log_n = 0;
    r->log_frame = r->frame + 1u;
    r->s0_valid = 0;
    r->s0_dot = NES_NO_HIT;
}

typedef struct Replay {
    uint32_t v, t, fx, ctrl, mask;
    uint8_t pal[32];
    uint32_t chr_off[8];
    uint8_t nt_map[4];
    uint32_t ev, count;
    const uint32_t* events;
    int mmc2;                        /* MMC2: the CHR halves follow creg and the latches */
    uint32_t creg[4], latch[2], chr_pages;
} Replay;

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

static int32_t ev_time(const Replay* s, uint32_t i) {
    return (int32_t)(s->events[2 * i] & 0xFFFFFFu) - NES_LOG_TIME_BIAS;
}

static void replay_apply(Replay* s, uint32_t i) {
    const uint32_t kind = s->events[2 * i] >> 24, w1 = s->events[2 * i + 1];
    const uint32_t val = w1 & 0xFFu, aux = (w1 >> 8) & 0xFFu;
    const uint32_t inc = (s->ctrl & 4u) ? 32u : 1u;
    switch (kind) {
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
        case NES_EV_DATA: s->v = (s->v + aux * inc) & 0x7FFFu; break;
        case NES_EV_PAL:
            s->pal[aux & 31u] = (uint8_t)val;
            s->v = (s->v + inc) & 0x7FFFu;
            break;
        case NES_EV_CHR: s->chr_off[aux & 7u] = val * 1024u; break;
        case NES_EV_MIRROR:
            for (int k = 0; k < 4; ++k) s->nt_map[k] = (uint8_t)((val >> (2 * k)) & 3u);
            break;
        case NES_EV_MMC2: /* patch:1471-1478 */
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

static void replay_until(Replay* s, int32_t time) { /* events strictly before `time` */
    while (s->ev < s->count && ev_time(s, s->ev) < time) replay_apply(s, s->ev++);
}

static int rendering(const Replay* s) { return (s->mask & 0x18u) != 0; }

static void y_increment(Replay* s) {
    if ((s->v & 0x7000u) != 0x7000u) {
        s->v += 0x1000u;
    } else {
        s->v &= ~0x7000u;
        uint32_t y = (s->v >> 5) & 31u;
        if (y == 29u) {
            y = 0;
            s->v ^= 0x0800u;
        } else if (y == 31u) {
            y = 0;
        } else {
            ++y;
        }
        s->v = (s->v & ~0x03E0u) | (y << 5);
    }
}

/* Line l's internal operations after its pixels: Y increment at dot 256, horizontal copy at 257; on the
 * pre-render line (l = -1) also the vertical copy (taken at dot 304); then the state at dot 320 is the one
 * line l + 1 is drawn with. */
static void replay_line_end(Replay* s, int l) {
    const int32_t base = l * 341;
    replay_until(s, base + 256);
    if (rendering(s)) y_increment(s);
    replay_until(s, base + 257);
    if (rendering(s)) s->v = (s->v & ~0x041Fu) | (s->t & 0x041Fu);
    if (l < 0) {
        replay_until(s, base + 304);
        if (rendering(s)) s->v = (s->v & ~0x7BE0u) | (s->t & 0x7BE0u);
    }
    replay_until(s, base + 320);
}

static void replay_begin(Replay* s, const NesRec* r, const NesCart* c) {
    const uint32_t* h = r->log;
    s->mmc2 = c->board == NES_BOARD_MMC2;
    s->chr_pages = c->chr_size / 1024u;
    for (int i = 0; i < 4; ++i) s->creg[i] = (h[14] >> (8 * i)) & 0xFFu;
    s->latch[0] = h[15] & 1u;
    s->latch[1] = (h[15] >> 8) & 1u;
    s->ctrl = h[1] & 0xFFu;
    s->mask = (h[1] >> 8) & 0xFFu;
    s->fx = (h[1] >> 16) & 7u;
    s->v = h[2] & 0xFFFFu;
    s->t = h[2] >> 16;
    for (int i = 0; i < 8; ++i) s->chr_off[i] = ((h[3 + (i >> 2)] >> ((i & 3) * 8)) & 0xFFu) * 1024u;
    for (int k = 0; k < 4; ++k) s->nt_map[k] = (uint8_t)((h[5] >> (2 * k)) & 3u);
    for (int i = 0; i < 32; ++i) s->pal[i] = (uint8_t)(h[6 + (i >> 2)] >> ((i & 3) * 8));
    s->events = h + NES_LOG_HDR_WORDS;
    s->count = r->log_n < NES_LOG_EVENTS ? r->log_n : NES_LOG_EVENTS;
    s->ev = 0;
    replay_line_end(s, -1);
}

static uint8_t nt_read(const NesRec* r, const Replay* s, uint32_t addr) { /* addr in $2000-$2FFF */
    const uint32_t n = (addr >> 10) & 3u;
    return r->nt[(s->nt_map[n] & 1u) * 1024u + (addr & 0x3FFu)];
}

/* Pattern address (low plane) of background tile slot `slot` (0..33) of the line drawn with state s. */
static uint32_t bg_slot_pa(const NesRec* r, const Replay* s, uint32_t slot) {
    /* the fetch address moves right one tile per slot, switching nametables at each wrap (twice for slot 33
     * from column 31) */
    const uint32_t cc = (s->v & 31u) + slot, cx = cc & 31u, nth = ((s->v >> 10) & 1u) ^ ((cc >> 5) & 1u);
    const uint32_t cy = (s->v >> 5) & 31u, fy = (s->v >> 12) & 7u, ntv = (s->v >> 11) & 1u;
    const uint32_t base = 0x2000u | ((nth | (ntv << 1)) << 10);
    return ((s->ctrl & 0x10u) << 8) + nt_read(r, s, base | (cy << 5) | cx) * 16u + fy;
}

/* Pattern address (low plane) of a sprite's row `row` (0..h-1, before the vertical flip). */
static uint32_t sprite_row_pa(uint32_t ctrl, uint32_t tile, uint32_t attr, uint32_t row) {
    const uint32_t h = (ctrl & 0x20u) ? 16u : 8u;
    if (attr & 0x80u) row = h - 1u - row;
    if (h == 8u) return ((ctrl & 0x08u) << 9) + tile * 16u + row;
    return ((tile & 1u) << 12) + (tile & 0xFEu) * 16u + (row & 7u) + ((row & 8u) << 1);
}

/* MMC2: the pattern fetches of line l in order, each through the bank of the moment and then the latch hook
 * (patch:1496-1560, 1660-1700): the sprites of line l, fetched at the end of line l - 1 (l >= 1), then, unless
 * sprites_only, the line's 34 background tile slots. sp_chr[k] / bg_chr[t] receive the CHR offset of the 4 KB
 * half each fetch read (slot 0 of the half); either may be NULL. Fetches happen only while rendering is on. */
static void mmc2_line_fetches(Replay* s, const NesRec* r, int l, int sprites_only, uint32_t* sp_chr,
                              uint32_t* bg_chr) {
    if (!s->mmc2 || (s->mask & 0x18u) == 0) return;
    if (l >= 1) {
        const int h = (s->ctrl & 0x20u) ? 16 : 8;
        uint32_t n = 0;
        for (uint32_t i = 0; i < 64u && n < 8u; ++i) {
            const uint8_t* o = r->oam + 4u * i;
            const int row = l - (int)o[0] - 1;
            if (row < 0 || row >= h) continue;
            const uint32_t pa = sprite_row_pa(s->ctrl, o[1], o[2], (uint32_t)row);
            if (sp_chr) sp_chr[n] = s->chr_off[4u * (pa >> 12)];
            replay_hook(s, pa);
            ++n;
        }
    }
    if (sprites_only) return;
    for (uint32_t t = 0; t < 34u; ++t) {
        const uint32_t pa = bg_slot_pa(r, s, t);
        if (bg_chr) bg_chr[t] = s->chr_off[4u * (pa >> 12)];
        replay_hook(s, pa);
    }
}

/* A pattern byte through the 1 KB slot table, or (base4 != ~0) from the 4 KB CHR half at byte offset base4. */
static uint32_t pat_read(const NesRec* r, const NesCart* c, const Replay* s, uint32_t base4, uint32_t a) {
    return base4 != ~0u ? c->chr[base4 + (a & 0xFFFu)] : chr_read(r, c, s->chr_off, a);
}

/* Background pixel x (0..255) of a line drawn with state s: 2-bit value and palette select. bg_chr: the MMC2
 * fetch banks of the line's tile slots, or NULL. */
static uint32_t bg_pixel(const NesRec* r, const NesCart* c, const Replay* s, uint32_t x, uint32_t* attr_out,
                         const uint32_t* bg_chr) {
    const uint32_t pos = x + s->fx, slot = pos >> 3, bit = pos & 7u;
    uint32_t cx = (s->v & 31u) + slot, nth = (s->v >> 10) & 1u;
    if (cx >= 32u) {
        cx -= 32u;
        nth ^= 1u;
    }
    const uint32_t cy = (s->v >> 5) & 31u, fy = (s->v >> 12) & 7u, ntv = (s->v >> 11) & 1u;
    const uint32_t base = 0x2000u | ((nth | (ntv << 1)) << 10);
    const uint32_t tile = nt_read(r, s, base | (cy << 5) | cx);
    const uint32_t at = nt_read(r, s, base | 0x3C0u | ((cy >> 2) << 3) | (cx >> 2));
    *attr_out = (at >> (((cy & 2u) << 1) | (cx & 2u))) & 3u;
    const uint32_t pa = ((s->ctrl & 0x10u) << 8) + tile * 16u + fy;
    const uint32_t b4 = bg_chr ? bg_chr[slot] : ~0u;
    const uint32_t lo = pat_read(r, c, s, b4, pa), hi = pat_read(r, c, s, b4, pa + 8u);
    return ((lo >> (7u - bit)) & 1u) | (((hi >> (7u - bit)) & 1u) << 1);
}

/* Pixel of sprite i at screen x on line l (0 transparent / outside), `row` = l - y - 1. base4: the MMC2 fetch
 * bank of the sprite's row (~0 = the slot table). */
static uint32_t sprite_pixel(const NesRec* r, const NesCart* c, const Replay* s, uint32_t i, uint32_t row,
                             uint32_t col, uint32_t base4) {
    const uint8_t* o = r->oam + 4u * i;
    if (o[2] & 0x40u) col = 7u - col;
    const uint32_t pa = sprite_row_pa(s->ctrl, o[1], o[2], row);
    const uint32_t lo = pat_read(r, c, s, base4, pa), hi = pat_read(r, c, s, base4, pa + 8u);
    return ((lo >> (7u - col)) & 1u) | (((hi >> (7u - col)) & 1u) << 1);
}

static void render_line(const NesRec* r, const NesCart* c, const Replay* s, int l, uint8_t* px,
                        const uint32_t* bg_chr, const uint32_t* sp_chr) {
    const int bg_on = (s->mask & 0x08u) != 0, sp_on = (s->mask & 0x10u) != 0;
    const uint32_t h = (s->ctrl & 0x20u) ? 16u : 8u;
    uint32_t sel[8], nsel = 0;
    if (sp_on) {
        for (uint32_t i = 0; i < 64u && nsel < 8u; ++i) {
            const int row = l - (int)r->oam[4 * i] - 1;
            if (row >= 0 && row < (int)h) sel[nsel++] = i;
        }
    }
    for (uint32_t x = 0; x < 256u; ++x) {
        uint32_t bg = 0, bga = 0;
        if (bg_on && (x >= 8u || (s->mask & 0x02u))) bg = bg_pixel(r, c, s, x, &bga, bg_chr);
        uint32_t sp = 0, spa = 0, behind = 0;
        if (x >= 8u || (s->mask & 0x04u)) {
            for (uint32_t k = 0; k < nsel; ++k) {
                const uint8_t* o = r->oam + 4u * sel[k];
                const uint32_t col = x - o[3];
                if (x < o[3] || col >= 8u) continue;
                const uint32_t p = sprite_pixel(r, c, s, sel[k], (uint32_t)(l - o[0] - 1), col,
                                                sp_chr ? sp_chr[k] : ~0u);
                if (p) {
                    sp = p;
                    spa = o[2] & 3u;
                    behind = (o[2] >> 5) & 1u;
                    break;
                }
            }
        }
        uint32_t colour;
        if (bg && (!sp || behind)) colour = s->pal[bga * 4u + bg];
        else if (sp) colour = s->pal[16u + spa * 4u + sp];
        else colour = s->pal[0];
        colour &= 0x3Fu;
        if (s->mask & 1u) colour &= 0x30u;
        px[x] = (uint8_t)colour;
    }
}

void orc_render_full(const NesRec* r, const NesCart* c, uint8_t* pix, uint8_t* emph) {
    Replay s;
    replay_begin(&s, r, c);
    for (int l = 0; l < 240; ++l) {
        uint32_t bgc[34], spc[8];
        mmc2_line_fetches(&s, r, l, 0, spc, bgc);
        render_line(r, c, &s, l, pix + l * 256, s.mmc2 ? bgc : NULL, s.mmc2 ? spc : NULL);
        emph[l] = (uint8_t)((s.mask >> 5) & 7u);
        replay_line_end(&s, l);
    }
}

void orc_render_obs(const NesRec* r, const NesCart* c, uint8_t* obs, uint8_t* emph) {
    Replay s;
    uint8_t line[256];
    replay_begin(&s, r, c);
    for (int l = 0; l < 232; ++l) {
        uint32_t bgc[34], spc[8];
        mmc2_line_fetches(&s, r, l, 0, spc, bgc);
        if (l >= 8) {
            render_line(r, c, &s, l, line, s.mmc2 ? bgc : NULL, s.mmc2 ? spc : NULL);
            memcpy(obs + (l - 8) * 240, line + 8, 240);
            emph[l - 8] = (uint8_t)((s.mask >> 5) & 7u);
        }
        replay_line_end(&s, l);
    }
}

/* First sprite-0 hit of the logged frame (frame dot), from the log so far: sprite 0's opaque pixels against
 * opaque background pixels, both layers on, not at x = 255, not in a clipped left column. */
int32_t orc_sprite0_scan(const NesRec* r, const NesCart* c) {
    Replay s;
    const int y0 = r->oam[0], x0 = r->oam[3];
    if (y0 >= 239) return NES_NO_HIT;
    replay_begin(&s, r, c);
    for (int l = 0; l < 240; ++l) {
        uint32_t bgc[34], spc[8];
        mmc2_line_fetches(&s, r, l, 0, spc, bgc);
        const uint32_t* bg_chr = s.mmc2 ? bgc : NULL;
        const uint32_t h = (s.ctrl & 0x20u) ? 16u : 8u;
        const int row = l - y0 - 1;
        if ((s.mask & 0x18u) == 0x18u && row >= 0 && row < (int)h) {
            for (int col = 0; col < 8; ++col) {
                const int x = x0 + col;
                if (x >= 255) break;
                if (x < 8 && (s.mask & 0x06u) != 0x06u) continue;
                uint32_t a;
                if (sprite_pixel(r, c, &s, 0, (uint32_t)row, (uint32_t)col, s.mmc2 ? spc[0] : ~0u) &&
                    bg_pixel(r, c, &s, (uint32_t)x, &a, bg_chr))
                    return l * 341 + x + 1;
            }
        }
        if (l >= y0 + 16) break; /* past sprite 0 at any size: no later hit possible */
        replay_line_end(&s, l);
    }
    return NES_NO_HIT;
}

/* ------------------------------------------------------------------------------------------ PPU events */

static uint64_t abs_dot(const NesRec* r) { return (uint64_t)r->frame * NES_FRAME_DOTS + r->frame_dot; }

static void s0_update(NesRec* r, const NesCart* c) {
    if (r->s0_valid || r->frame != r->log_frame) return;
    r->s0_valid = 1;
    r->s0_dot = NES_NO_HIT;
    if ((r->status & 0x40u) || r->frame_dot >= 240u * 341u) return;
    int32_t hit = orc_sprite0_scan(r, c);
    if (hit != NES_NO_HIT && hit <= (int32_t)r->frame_dot) hit = (int32_t)r->frame_dot + 1;
    r->s0_dot = hit;
}

static int is_mmc3_clock_dot(uint32_t d) {
    if (d == 261u * 341u + 256u) return 1;
    return d < 240u * 341u && d % 341u == 266u;
}

static uint32_t dots_to_event(NesRec* r, const NesCart* c) {
    const uint32_t fd = r->frame_dot;
    uint32_t best = NES_FRAME_DOTS - fd;
    if (fd < NES_VBLANK_DOT && NES_VBLANK_DOT - fd < best) best = NES_VBLANK_DOT - fd;
    if (fd < NES_PRERENDER_DOT && NES_PRERENDER_DOT - fd < best) best = NES_PRERENDER_DOT - fd;
    if (c->board == NES_BOARD_MMC3) {
        const uint32_t line = fd / 341u, d = fd % 341u;
        uint32_t next;
        if (line < 240u) next = d < 266u ? line * 341u + 266u : (line < 239u ? (line + 1u) * 341u + 266u : 261u * 341u + 256u);
        else if (line < 261u) next = 261u * 341u + 256u;
        else next = d < 256u ? 261u * 341u + 256u : 0xFFFFFFFFu;
        if (next != 0xFFFFFFFFu && next - fd < best) best = next - fd;
    }
    s0_update(r, c);
    if (r->frame == r->log_frame && r->s0_dot != NES_NO_HIT && (uint32_t)r->s0_dot > fd &&
        (uint32_t)r->s0_dot - fd < best)
        best = (uint32_t)r->s0_dot - fd;
    return best;
}

/* MMC2 at vblank: the latches this frame's own fetches leave, from a latches-only replay of its log over the
 * nametables and OAM as they are now (NeSLE's frame_resolve_mmc2, patch:1790-1812; rl/csrc/nes_machine.cuh:110-131
 * runs the same replay after the vblank stop, before any further instruction). */
static void mmc2_resolve(NesRec* r, const NesCart* c) {
    if (r->frame != r->log_frame) return;   /* no log of this frame (the first one after power-on) */
    Replay s;
    replay_begin(&s, r, c);
    for (int l = 0; l < 240; ++l) {
        mmc2_line_fetches(&s, r, l, 0, NULL, NULL);
        replay_line_end(&s, l);
    }
    mmc2_line_fetches(&s, r, 240, 1, NULL, NULL);
    replay_until(&s, INT32_MAX);
    r->mreg[6] = (uint8_t)s.latch[0];
    r->mreg[7] = (uint8_t)s.latch[1];
    mapper_sync(r, c);
}

static void process_events(NesRec* r, const NesCart* c) {
    const uint32_t d = r->frame_dot;
    if (d == NES_FRAME_DOTS) {
        r->frame_dot = 0;
        ++r->frame;
        return;
    }
    if (d == NES_VBLANK_DOT) {
        r->status |= 0x80u;
        if (r->ctrl & 0x80u) r->nmi_pending = 1;
        if (c->board == NES_BOARD_MMC2) mmc2_resolve(r, c);
    }
    if (d == NES_PRERENDER_DOT) {
        r->status &= 0x1Fu;
        log_capture(r);
    }
    if (c->board == NES_BOARD_MMC3 && is_mmc3_clock_dot(d) && (r->mask & 0x18u)) mmc3_clock(r);
    if (r->frame == r->log_frame && r->s0_dot != NES_NO_HIT && d == (uint32_t)r->s0_dot) {
        r->status |= 0x40u;
        r->s0_dot = NES_NO_HIT;
    }
}

static void ppu_advance(NesRec* r, const NesCart* c, uint32_t dots) {
    while (dots > 0) {
        const uint32_t to = dots_to_event(r, c);
        if (dots < to) {
            r->frame_dot += dots;
            return;
        }
        r->frame_dot += to;
        dots -= to;
        process_events(r, c);
    }
}

/* ------------------------------------------------------------------------------------------------- bus */

typedef struct Bus {
    NesRec* r;
    const NesCart* c;
    int32_t ev_time; /* log time of this instruction's accesses (its end) */
    int log_on;      /* the instruction started inside the log window */
    int dma;         /* a $4014 write happened */
} Bus;

static void log_event(Bus* b, uint32_t kind, uint32_t value, uint32_t aux) {
    NesRec* r = b->r;
    if (kind != NES_EV_PAL) r->s0_valid = 0;
    if (!b->log_on) return;
    uint32_t* h = r->log;
    uint32_t* ev = h + NES_LOG_HDR_WORDS;
    if (kind == NES_EV_DATA && (r->mask & 0x18u) == 0 && r->log_n > 0) {
        uint32_t* last = ev + 2u * (r->log_n - 1u);
        if ((last[0] >> 24) == NES_EV_DATA && (last[1] >> 8) < 0xFFu) {
            last[1] += 0x100u;
            return;
        }
    }
    if (r->log_n >= NES_LOG_EVENTS) {
        h[0] |= NES_LOG_OVERFLOW;
        return;
    }
    ev[2u * r->log_n] = ((uint32_t)(b->ev_time + NES_LOG_TIME_BIAS) & 0xFFFFFFu) | (kind << 24);
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
            r->s0_valid = 0;
        }
        log_event(b, NES_EV_DATA, 0, 1);
    } else if (a < 0x3F00u) {
        r->nt[(r->nt_map[(a >> 10) & 3u] & 1u) * 1024u + (a & 0x3FFu)] = v;
        log_event(b, NES_EV_DATA, 0, 1);
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
            log_event(b, NES_EV_DATA, 0, 1);
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
            r->s0_valid = 0;
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
        r->s0_valid = 0;
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
static int execute(Cpu* k, uint8_t op, int32_t abs_start_rel, int log_on) {
    NesRec* r = k->r;
    Bus* b = k->b;
    const uint32_t base = kCycles[op];
    if (base == 0) return 0;
    k->cycles = base;
    uint16_t len = 1, a;
    uint8_t m;
    b->log_on = log_on;
    b->ev_time = abs_start_rel + 3 * (int32_t)base;
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
                case 4: a = ea_izy(k, 1); b->ev_time = abs_start_rel + 3 * (int32_t)k->cycles; m = rd(k, a); len = 2; break;
                case 5: m = rd(k, ea_zpx(k)); len = 2; break;
                case 6: a = ea_abi(k, r->y, 1); b->ev_time = abs_start_rel + 3 * (int32_t)k->cycles; m = rd(k, a); len = 3; break;
                default: a = ea_abi(k, r->x, 1); b->ev_time = abs_start_rel + 3 * (int32_t)k->cycles; m = rd(k, a); len = 3; break;
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
                case 0xBE: a = ea_abi(k, r->y, 1); b->ev_time = abs_start_rel + 3 * (int32_t)k->cycles; m = rd(k, a); len = 3; break;
                default: a = ea_abi(k, r->x, 1); b->ev_time = abs_start_rel + 3 * (int32_t)k->cycles; m = rd(k, a); len = 3; break;
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
 * stall and the DMC service (patch:823-862). `pending` = dots not yet settled. */
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
    const int64_t start = (int64_t)abs_dot(r) + pending + 3 * cyc - (int64_t)r->log_frame * NES_FRAME_DOTS;
    const int log_on = start >= LOG_WINDOW_START && start < (int64_t)NES_VBLANK_DOT;
    *pc_out = r->pc;
    *op_out = fetch(r, c, r->pc);
    k.lo = fetch(r, c, (uint16_t)(r->pc + 1));
    k.hi = fetch(r, c, (uint16_t)(r->pc + 2));
    if (!execute(&k, *op_out, (int32_t)start, log_on)) {
        *fault = ((uint32_t)r->pc << 8) | *op_out;
        return 0;
    }
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
    (void)dots_to_event(r, c);
    const uint32_t cyc = step(r, c, 0, fault, &op, &pc);
    if (*fault) return 0;
    ppu_advance(r, c, 3u * cyc);
    return cyc;
}

/* The JMP-to-self idle loop: skip whole 3-cycle jumps up to the next PPU event (patch:866-893). Not while an
 * interrupt waits to be taken. */
static void fast_forward(NesRec* r, const NesCart* c) {
    if (r->nmi_pending || (r->irq_line && !(r->p & FL_I))) return;
    const uint32_t to = dots_to_event(r, c);
    const uint32_t jumps = (to + 8u) / 9u;
    if (jumps == 0) return;
    r->cycles += 3u * jumps;
    if (r->cycles >= r->dmc_event) (void)orc_dmc_service(r, r->cycles, 0);
    ppu_advance(r, c, 9u * jumps);
}

uint32_t orc_run_until(NesRec* r, const NesCart* c, uint64_t target) {
    uint32_t instructions = 0, fault = 0, pending = 0;
    uint32_t to_event = dots_to_event(r, c);
    while (instructions < NES_BUDGET) {
        if (pending >= to_event) {
            ppu_advance(r, c, pending);
            pending = 0;
            if (abs_dot(r) >= target) break;
            to_event = dots_to_event(r, c);
        }
        uint8_t op;
        uint16_t pc0;
        const uint32_t cyc = step(r, c, pending, &fault, &op, &pc0);
        if (fault) break;
        pending += 3u * cyc;
        ++instructions;
        ++r->instr_lo;
        if (!r->s0_valid) to_event = dots_to_event(r, c);
        if (op == 0x4C && r->pc == pc0) {
            ppu_advance(r, c, pending);
            pending = 0;
            if (abs_dot(r) >= target) break;
            fast_forward(r, c);
            to_event = dots_to_event(r, c);
            if (abs_dot(r) >= target) break;
        }
    }
    if (pending) ppu_advance(r, c, pending);
    return fault;
}
