/* reward10 game readers other than SMB: RAM -> Signals for Pac-Man, Excitebike, Contra, Castlevania, Gradius,
 * Zelda, Tetris, Tecmo Bowl, Kage, Final Mission and Punch-Out (rl/csrc/reward10.cuh:160-524), the per-game tracker
 * constants (rl/csrc/reward10_consts.h:11-37) and the per-env key sets two readers keep (reward10.cuh:26-56).
 *
 * One source for the CPU oracle (C) and the HIP library (device code): the readers are pure functions of the RAM
 * and the reader state, and their parity is pinned against the reference's own compiled rl10_replay
 * (rl/csrc/host_api.cpp:13-31) on seeded RAM trajectories (tests/golden/gen_golden.py), for each build separately.
 * Arithmetic is double in the reference's (Python's) order; build with -ffp-contract=off.
 *
 * Tables and constants that must equal the reference's bit for bit (Kage routes, bosses, Zelda items, game units)
 * are its values, written as hexadecimal floats.
 */
#ifndef RL10_GAMES_H
#define RL10_GAMES_H
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <math.h>
#include <stdint.h>
#endif

#include "rlenv_state.h"

#if defined(__HIPCC__)
#define RL10G_FN static __device__ __forceinline__
#define RL10G_HD static __host__ __device__ __forceinline__
#define RL10G_TAB static __constant__ const
#else
#define RL10G_FN static inline
#define RL10G_HD static inline
#define RL10G_TAB static const
#endif

/* game ids (reward10_consts.h:11-23) */
enum { RL10_SMB = 0, RL10_PACMAN, RL10_EXCITEBIKE, RL10_CONTRA, RL10_CASTLEVANIA, RL10_GRADIUS, RL10_ZELDA, RL10_TETRIS,
       RL10_TECMOBOWL, RL10_KAGE, RL10_FINALMISSION, RL10_PUNCHOUT, RL10_NUM_GAMES };

/* One game's tracker constants (reward10_consts.h:25-37). */
typedef struct Rl10Game {
    double progress_unit, score_unit, stall_frames, idle_per_frame;
    int death_from_lives, start_ok, select_ok;
} Rl10Game;

RL10G_HD Rl10Game rl10_game(int game) {
    Rl10Game g = {0x1.7700000000000p+11, 0x1.9000000000000p+7, 0x1.c200000000000p+12, -0x1.0624dd2f1a9fcp-12, 0, 0, 0};
    switch (game) {
        case RL10_PACMAN: g.progress_unit = 0x1.8p+7; g.score_unit = 0x1.f4p+9; break;
        case RL10_EXCITEBIKE: g.progress_unit = 0x1.57cp+13; g.score_unit = 0x1p+0; break;
        case RL10_CONTRA: g.progress_unit = 0x1.77p+12; g.score_unit = 0x1.9p+7; break;
        case RL10_CASTLEVANIA: g.progress_unit = 0x1.77p+11; g.score_unit = 0x1.2cp+8; break;
        case RL10_GRADIUS: g.progress_unit = 0x1.ap+11; g.score_unit = 0x1.f4p+10; break;
        case RL10_ZELDA: g.progress_unit = 0x1.4p+4; g.score_unit = 0x1.4p+2; g.start_ok = 1; break;
        case RL10_TETRIS: g.progress_unit = 0x1.4p+3; g.score_unit = 0x1.4p+5; break;
        case RL10_TECMOBOWL:
            g.progress_unit = 0x1.9p+6; g.score_unit = 0x1.cp+2; g.stall_frames = 0x1.194p+14;
            g.idle_per_frame = -0x1.a36e2eb1c432dp-14;
            break;
        case RL10_KAGE: g.progress_unit = 0x1.f4p+9; g.score_unit = 0x1p+0; break;
        case RL10_FINALMISSION: g.progress_unit = 0x1.e8p+9; g.score_unit = 0x1.f4p+9; break;
        case RL10_PUNCHOUT: g.progress_unit = 0x1.2p+8; g.score_unit = 0x1.9p+6; g.start_ok = 1; g.select_ok = 1; break;
        default: break;   /* SMB */
    }
    return g;
}

/* Entries of a game's per-env key set (reward10.cuh:527-529); 0 = none. */
RL10G_HD uint32_t rl10_keyset_capacity(int game) {
    return game == RL10_ZELDA ? 16384u : game == RL10_CASTLEVANIA ? 4096u : 0u;
}

/* ------------------------------------------------------------------------------------------------ key sets */
/* Open addressing with linear probing over `cap` (a power of two) slots; a slot holds key + 1, 0 = empty. Returns
 * 1 inserted, 0 present, -1 full (load kept <= 3/4; the caller flags an overflow). */
RL10G_FN uint32_t rl10_mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

RL10G_FN int rl10_keyset_insert(uint32_t* slots, uint32_t cap, uint32_t* count, uint32_t key) {
    if (cap == 0u) return -1;
    const uint32_t stored = key + 1u;
    uint32_t i = rl10_mix32(key) & (cap - 1u);
    for (uint32_t n = 0; n < cap; ++n, i = (i + 1u) & (cap - 1u)) {
        const uint32_t v = slots[i];
        if (v == stored) return 0;
        if (v == 0u) {
            if ((*count + 1u) * 4u > cap * 3u) return -1;
            slots[i] = stored;
            *count += 1u;
            return 1;
        }
    }
    return -1;
}

RL10G_FN void rl10_keyset_clear(uint32_t* slots, uint32_t cap) {
    for (uint32_t i = 0; i < cap; ++i) slots[i] = 0u;
}

/* ------------------------------------------------------------------------------------------------ helpers */
RL10G_FN int rl10_u8(const uint8_t* r, int a) { return (int)r[a]; }

RL10G_FN int64_t rl10_bcd(const uint8_t* r, const int* addrs, int n) {   /* two decimal digits per byte */
    int64_t v = 0;
    for (int i = 0; i < n; ++i) {
        const int x = r[addrs[i]];
        v = v * 100 + (x >> 4) * 10 + (x & 15);
    }
    return v;
}

RL10G_FN int64_t rl10_digits(const uint8_t* r, int first, int last_excl) {   /* one decimal digit per byte */
    int64_t v = 0;
    for (int a = first; a < last_excl; ++a) v = v * 10 + r[a];
    return v;
}

RL10G_FN int rl10_popcount8(int x) {
    int c = 0;
    for (; x; x >>= 1) c += x & 1;
    return c;
}

/* sqrt(x^2 + y^2) correctly rounded, as Python's math.hypot on these inputs (reward10.cuh:124-139): the exact sum
 * of squares as a double-double (products by fma, the sum by two-sum), then one Newton step of the root. */
RL10G_FN double rl10_hypot(double x, double y) {
    x = fabs(x);
    y = fabs(y);
    if (x < y) {
        const double t = x;
        x = y;
        y = t;
    }
    if (y == 0.0) return x;
    const double xx = x * x, yy = y * y;
    const double ex = fma(x, x, -xx), ey = fma(y, y, -yy);
    const double hi = xx + yy;
    const double b = hi - xx;
    const double lo = (xx - (hi - b)) + (yy - b) + ex + ey;
    const double s = sqrt(hi);
    const double res = fma(-s, s, hi) + lo;
    return s + res / (2.0 * s);
}

RL10G_FN Rl10Signals rl10_blank(void) {
    Rl10Signals s;
    s.in_play = s.progress_valid = s.dying = s.has_lives = s.has_health = s.has_score = s.game_over = s.won = 0;
    s.level = s.lives = 0;
    s.progress = s.health = 0.0;
    s.score = 0;
    return s;
}

/* ------------------------------------------------------------------------------------------------ readers */
/* Pac-Man (reward10.cuh:160-176) */
RL10G_FN Rl10Signals rl10_pacman(const uint8_t* r) {
    const int state = rl10_u8(r, 0x3F), remaining = rl10_u8(r, 0x6A);
    const int game = rl10_u8(r, 0x48) == 0 && rl10_u8(r, 0x47) == 0;
    const int playing = game && (state == 4 || state == 6 || state == 12) && !(rl10_u8(r, 0x4A) & 1);
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)playing;
    s.level = rl10_u8(r, 0x68);
    s.progress = remaining <= 192 ? (double)(192 - remaining) : 0.0;
    s.progress_valid = (uint8_t)(playing && remaining <= 192);
    s.dying = (uint8_t)(game && state == 8);
    s.has_lives = 1;
    s.lives = rl10_u8(r, 0x67);
    int64_t sc = 0, p10 = 1;
    for (int i = 0; i < 6; ++i, p10 *= 10) sc += rl10_u8(r, 0x70 + i) * p10;
    s.has_score = 1;
    s.score = 10 * sc;
    s.game_over = (uint8_t)(game && state == 10);
    return s;
}

/* Excitebike (reward10.cuh:178-207): the distance is the camera's travel, unwrapped, while racing */
RL10G_FN Rl10Signals rl10_excitebike(const uint8_t* r, Rl10Reader* e) {
    const int level = rl10_u8(r, 0x43) + rl10_u8(r, 0x46);
    const int racing = rl10_u8(r, 0x47) == 1 && rl10_u8(r, 0x4F) == 1 && rl10_u8(r, 0x52) == 0;
    const int cam = rl10_u8(r, 0x12) + 256 * (rl10_u8(r, 0x4D) & 1);
    const int k4f = rl10_u8(r, 0x4F);
    if (!e->has_key || e->key_a != level || e->key_b != k4f) {
        e->has_key = 1;
        e->key_a = level;
        e->key_b = k4f;
        e->has_cam = 0;
        e->dist = 0.0;
    }
    if (racing) {
        if (e->has_cam) e->dist += ((cam - e->cam + 256) % 512 + 512) % 512 - 256;   /* a non-negative modulo */
        e->has_cam = 1;
        e->cam = cam;
    } else {
        e->has_cam = 0;
    }
    const int k9c = rl10_u8(r, 0x9C);
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)(racing && rl10_u8(r, 0x3B1) == 0);
    s.level = level;
    s.progress = e->dist;
    s.progress_valid = (uint8_t)racing;
    s.dying = (uint8_t)(racing && (rl10_u8(r, 0xF2) == 1 || (1 <= k9c && k9c <= 4)));
    s.has_health = 1;
    s.health = rl10_u8(r, 0x3B6) >= 32 ? 0.0 : 1.0;
    s.game_over = (uint8_t)(rl10_u8(r, 0x41) == 0 || rl10_u8(r, 0x41) == 1);
    s.won = (uint8_t)(rl10_u8(r, 0x3F3) >= 2);
    return s;
}

#define RL10_CONTRA_ROOM 0x1.f4p+9   /* 1000 */
#define RL10_CONTRA_BOSS 0x1.77p+11  /* 3000 */

/* Contra (reward10.cuh:209-250): screen position; base rooms by screen plus the core's damage; stage 1's boss */
RL10G_FN Rl10Signals rl10_contra(const uint8_t* r, Rl10Reader* e) {
    const int game = rl10_u8(r, 0x18) == 5 && rl10_u8(r, 0x1C) == 0;
    const int running = game && rl10_u8(r, 0x2C) == 4;
    const int over = game && rl10_u8(r, 0x38) == 1;
    const int level = rl10_u8(r, 0x30), screen = rl10_u8(r, 0x64);
    double progress = (double)(screen * 256 + rl10_u8(r, 0x65));
    if (rl10_u8(r, 0x40) == 1) {
        progress = screen * RL10_CONTRA_ROOM;
        int slot = -1;
        for (int i = 0; i < 16 && slot < 0; ++i)
            if (rl10_u8(r, 0x528 + i) == 0x14) slot = i;
        if (slot >= 0) {
            if (!e->has_key || e->key_a != level || e->key_b != screen) {
                e->has_key = 1;
                e->key_a = level;
                e->key_b = screen;
                e->core_max = 0;
            }
            const int hp = rl10_u8(r, 0x578 + slot);
            if (hp > e->core_max) e->core_max = hp;
            if (e->core_max >= 2) progress += 0.5 * RL10_CONTRA_ROOM * (1 - (double)hp / e->core_max);
        }
    } else if (level == 0) {
        int slot = -1;
        for (int i = 0; i < 16 && slot < 0; ++i)
            if (rl10_u8(r, 0x528 + i) == 0x11) slot = i;
        if (slot >= 0) {
            const int hp = rl10_u8(r, 0x578 + slot);
            progress += RL10_CONTRA_BOSS * ((double)(32 - (hp < 32 ? hp : 32)) / 32);
        }
    }
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)(running && rl10_u8(r, 0x25) == 0 && !over);
    s.level = level;
    s.progress = progress;
    s.progress_valid = (uint8_t)(running && rl10_u8(r, 0x90) == 1);
    s.dying = (uint8_t)(game && rl10_u8(r, 0x90) == 2);
    s.has_lives = 1;
    s.lives = over ? -1 : rl10_u8(r, 0x32);
    s.has_score = 1;
    s.score = (int64_t)(rl10_u8(r, 0x7E2) | (rl10_u8(r, 0x7E3) << 8)) * 100;
    s.game_over = (uint8_t)over;
    return s;
}

#define RL10_CASTLE_BOSS 0x1.77p+10  /* 1500 */

/* Castlevania (reward10.cuh:252-280): 32-px cells visited per floor band on the stage, plus the stage boss */
RL10G_FN Rl10Signals rl10_castlevania(const uint8_t* r, Rl10State* t, Rl10Reader* e, uint32_t* keys, uint32_t cap) {
    const int state = rl10_u8(r, 0x18);
    const int play = state == 5 && rl10_u8(r, 0x19) == 6;
    const int hp = rl10_u8(r, 0x45);
    const int stage = rl10_u8(r, 0x28), x = rl10_u8(r, 0x41) * 256 + rl10_u8(r, 0x40), y = rl10_u8(r, 0x3F);
    if (!e->has_stage || stage != e->stage) {
        e->has_stage = 1;
        e->stage = stage;
        rl10_keyset_clear(keys, cap);
        e->cells = 0;
        e->has_floor = 0;
    }
    if (play && hp > 0) {
        const int dy = y - e->floor_y;
        if (!e->has_floor || (dy < 0 ? -dy : dy) >= 40) {
            e->has_floor = 1;
            e->floor_y = y;
        }
        if (rl10_keyset_insert(keys, cap, &e->cells, (uint32_t)((x / 32) * 8 + e->floor_y / 40)) < 0) t->overflow = 1;
    }
    const int boss_stage = stage == 3 || stage == 6 || stage == 9 || stage == 12 || stage == 15 || stage == 18;
    const int eb = rl10_u8(r, 0x1A9);
    const double boss = boss_stage ? (double)(64 - (eb < 64 ? eb : 64)) / 64.0 : 0.0;
    const int kScore[3] = {0x7FE, 0x7FD, 0x7FC};
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)(play && rl10_u8(r, 0x22) == 0);
    s.level = stage;
    s.progress = (double)(32LL * e->cells) + boss * RL10_CASTLE_BOSS;
    s.progress_valid = (uint8_t)(play && hp > 0);
    s.dying = (uint8_t)((state == 5 || state == 6 || state == 7) && (hp == 0 || rl10_u8(r, 0x46C) == 8));
    s.has_lives = 1;
    s.lives = rl10_u8(r, 0x2A);
    s.has_health = 1;
    s.health = hp / 64.0;
    s.has_score = 1;
    s.score = rl10_bcd(r, kScore, 3);
    s.game_over = (uint8_t)(state == 7 || state == 13);
    return s;
}

/* Gradius (reward10.cuh:282-297) */
RL10G_FN Rl10Signals rl10_gradius(const uint8_t* r) {
    const int game = rl10_u8(r, 0x00) == 5 && rl10_u8(r, 0x0A) == 1;
    const int state = rl10_u8(r, 0x1B), lives = rl10_u8(r, 0x20);
    const int playing = game && (state & 0xE0) == 0x80 && rl10_u8(r, 0x15) == 0;
    const int kScore[3] = {0x7E6, 0x7E5, 0x7E4};
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)playing;
    s.level = rl10_u8(r, 0x19);
    s.progress = (double)(rl10_u8(r, 0x3F) * 256 + rl10_u8(r, 0x3E));
    s.progress_valid = (uint8_t)playing;
    s.dying = (uint8_t)(game && (state & 0xE0) == 0xA0);
    s.has_lives = 1;
    s.lives = lives > 127 ? lives - 256 : lives;
    s.has_score = 1;
    s.score = rl10_bcd(r, kScore, 3) * 10;
    s.game_over = (uint8_t)(rl10_u8(r, 0x00) == 5 && state == 192);
    return s;
}

RL10G_TAB int kRl10ZeldaItem[16] = {0x657, 0x659, 0x65A, 0x65B, 0x65C, 0x65F, 0x660, 0x661,
                                    0x662, 0x663, 0x664, 0x665, 0x666, 0x674, 0x675, 0x676};
RL10G_TAB int kRl10ZeldaCap[16] = {3, 2, 1, 2, 1, 1, 1, 1, 2, 1, 1, 1, 1, 1, 1, 1};

/* Zelda (reward10.cuh:299-335): rooms and 32-px cells visited (one key set, rooms tagged by bit 31), items and heart
 * containers gained since the first time in play */
RL10G_FN Rl10Signals rl10_zelda(const uint8_t* r, Rl10State* t, Rl10Reader* e, uint32_t* keys, uint32_t cap) {
    const int mode = rl10_u8(r, 0x12);
    const int play = mode == 5 || mode == 0xB;
    int items = 0;
    for (int i = 0; i < 16; ++i) {
        const int v = rl10_u8(r, kRl10ZeldaItem[i]);
        items += v < kRl10ZeldaCap[i] ? v : kRl10ZeldaCap[i];
    }
    const int hpb = rl10_u8(r, 0x66F), part = rl10_u8(r, 0x670);
    const double h = (hpb & 0xF) + (part >= 0x80 ? 1.0 : part > 0 ? 0.5 : 0.0);
    const int containers = (hpb >> 4) + 1;
    if (play) {
        const uint32_t d = (uint32_t)rl10_u8(r, 0x10), room = (uint32_t)rl10_u8(r, 0xEB);
        if (rl10_keyset_insert(keys, cap, &e->rooms, 0x80000000u | (d << 8) | room) < 0) t->overflow = 1;
        const uint32_t cell = (d << 16) | (room << 8) | ((uint32_t)(mode == 0xB) << 6) |
                              ((uint32_t)(rl10_u8(r, 0x70) / 32) << 3) | (uint32_t)(rl10_u8(r, 0x84) / 32);
        if (rl10_keyset_insert(keys, cap, &e->cells, cell) < 0) t->overflow = 1;
        if (!e->has_base) {
            e->has_base = 1;
            e->base_items = items;
            e->base_containers = containers;
        }
    }
    int gained = 0;
    if (e->has_base) {
        const int gi = items - e->base_items, gc = containers - e->base_containers;
        gained = (gi > 0 ? gi : 0) + (gc > 0 ? gc : 0);
    }
    const double hf = h / containers;
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)play;
    s.level = rl10_popcount8(rl10_u8(r, 0x671));
    s.progress = ((double)e->rooms + 0.02 * e->cells) + (double)(10 * gained);
    s.progress_valid = (uint8_t)play;
    s.dying = (uint8_t)(mode == 0x11);
    s.has_health = 1;
    s.health = hf < 1.0 ? hf : 1.0;
    s.has_score = 1;
    s.score = rl10_u8(r, 0x66D);
    s.game_over = (uint8_t)(mode == 0x11);
    return s;
}

/* Tetris (reward10.cuh:337-355) */
RL10G_FN Rl10Signals rl10_tetris(const uint8_t* r) {
    const int mode = rl10_u8(r, 0xC0), ps = rl10_u8(r, 0x48), render = rl10_u8(r, 0xBD);
    const int kLines[2] = {0x51, 0x50};
    const int kScore[3] = {0x55, 0x54, 0x53};
    const int64_t lines = rl10_bcd(r, kLines, 2);
    const int level = rl10_u8(r, 0x64);
    const int playing = mode == 4 && 1 <= ps && ps <= 8 && render == 3;
    const int topout = mode == 4 && ps == 10;
    const int64_t pl = lines - 10LL * level;
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)playing;
    s.level = level;
    s.progress = (double)(pl > 0 ? pl : 0);
    s.progress_valid = (uint8_t)playing;
    s.dying = (uint8_t)topout;
    s.has_score = 1;
    s.score = rl10_bcd(r, kScore, 3);
    s.game_over = (uint8_t)(topout && rl10_u8(r, 0x58) == 20);
    return s;
}

#define RL10_TECMO_GOAL_X 1456
#define RL10_TECMO_PX_PER_YARD 0x1.999999999999ap+3   /* 12.8 */

/* Tecmo Bowl (reward10.cuh:357-416): points, plus the yards the current drive has gained on the field */
RL10G_FN Rl10Signals rl10_tecmobowl(const uint8_t* r, Rl10Reader* e) {
    const int kOwn[1] = {0x43}, kOpp[1] = {0x48};
    const int own = (int)rl10_bcd(r, kOwn, 1), opp = (int)rl10_bcd(r, kOpp, 1);
    const int s0 = rl10_u8(r, 0x2C), s1 = rl10_u8(r, 0x2D);
    const int ended = rl10_u8(r, 0x8D) >= 4 && rl10_u8(r, 0x8B) == 0 && rl10_u8(r, 0x8A) == 0;
    const int on_screen = (s0 == 8 && s1 == 0) || (s0 == 9 && s1 == 9) || (s0 == 12 && s1 == 12);
    const int playing = on_screen && rl10_u8(r, 0x8D) <= 4 && !ended;
    if (playing) {
        e->has_week = 1;
        e->week = rl10_u8(r, 0x8F);
    }
    const int state = rl10_u8(r, 0x49);
    const int los = rl10_u8(r, 0xFB) + 256 * rl10_u8(r, 0xFC);
    const double yard = (los - RL10_TECMO_GOAL_X) / RL10_TECMO_PX_PER_YARD;
    const int scored = e->has_own && opp - e->opp >= 2;
    if (e->has_own && own != e->own) e->has_drive = 0;
    if (playing && state == 1) {
        e->has_drive = 0;
    } else if (playing && state == 0 && s0 == 9 && s1 == 9) {
        if (!e->has_drive) {
            e->has_drive = 1;
            e->drive_start = yard;
            e->drive_best = yard;
        }
        e->drive_best = yard > e->drive_best ? yard : e->drive_best;
    }
    e->has_own = 1;
    e->own = own;
    e->opp = opp;
    double gain = 0.0;
    if (e->has_drive) {
        const double g = e->drive_best - e->drive_start;
        gain = 0.0 >= g ? 0.0 : g;
    }
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)playing;
    s.level = rl10_u8(r, 0x8F);
    s.progress = 100.0 / 7.0 * own + gain;
    s.progress_valid = (uint8_t)playing;
    s.dying = (uint8_t)scored;
    s.has_score = 1;
    s.score = own;
    s.game_over = (uint8_t)(ended && opp > own);
    s.won = (uint8_t)(ended && own > opp && e->has_week && e->week == 10);
    return s;
}

/* Kage routes (reward10_consts.h:40-103): per stage, polyline segments {x0, y0, x1, y1, length, arc length before}
 * and the route's total length; the bosses {stage, kind, selector, hit points}. */
typedef struct Rl10KageSeg { double x0, y0, x1, y1, len, acc; } Rl10KageSeg;
typedef struct Rl10KageRoute { int stage, first, count; double total; } Rl10KageRoute;
typedef struct Rl10KageBoss { int stage, kind, sel, max_hp; } Rl10KageBoss;
#define RL10_KAGE_LOOKAHEAD 0x1.9p+8   /* 400 */
#define RL10_KAGE_MAX_OFF 0x1.8p+7     /* 192 */

RL10G_TAB Rl10KageSeg kRl10KageSegs[45] = {
    {0x1p+8, 0x1.9p+8, 0x1.fep+10, 0x1.9p+8, 0x1.bep+10, 0x0p+0},
    {0x1.4p+11, 0x1p+9, 0x1.9c2p+11, 0x1p+9, 0x1.708p+9, 0x0p+0},
    {0x1.9c2p+11, 0x1p+9, 0x1.a02p+11, 0x1.cep+8, 0x1.dae803b4bc0c4p+5, 0x1.708p+9},
    {0x1.a02p+11, 0x1.cep+8, 0x1.a02p+11, 0x1.26p+8, 0x1.5p+7, 0x1.8e2e803b4bc0cp+9},
    {0x1.a02p+11, 0x1.26p+8, 0x1.c02p+11, 0x1.0ep+8, 0x1.011f5eb54147p+8, 0x1.e22e803b4bc0cp+9},
    {0x1p+8, 0x1p+10, 0x1p+11, 0x1p+10, 0x1.cp+10, 0x0p+0},
    {0x1p+9, 0x1.8p+9, 0x1.b44p+10, 0x1.8p+9, 0x1.344p+10, 0x0p+0},
    {0x1.b44p+10, 0x1.8p+9, 0x1.c04p+10, 0x1.67p+9, 0x1.153e5af20e11ap+6, 0x1.344p+10},
    {0x1.c04p+10, 0x1.67p+9, 0x1.c04p+10, 0x1.13p+9, 0x1.5p+7, 0x1.4593e5af20e12p+10},
    {0x1.c04p+10, 0x1.13p+9, 0x1.cc4p+10, 0x1.fep+8, 0x1.f3db2174e7468p+5, 0x1.6f93e5af20e12p+10},
    {0x1.cc4p+10, 0x1.fep+8, 0x1.ap+11, 0x1.fep+8, 0x1.73cp+10, 0x1.7f32bebac81b5p+10},
    {0x1p+9, 0x1p+11, 0x1.364p+10, 0x1p+11, 0x1.6c8p+9, 0x0p+0},
    {0x1.364p+10, 0x1p+11, 0x1.404p+10, 0x1.f38p+10, 0x1.001ffe003ff6p+6, 0x1.6c8p+9},
    {0x1.404p+10, 0x1.f38p+10, 0x1.404p+10, 0x1.838p+10, 0x1.cp+8, 0x1.8c83ffc007fecp+9},
    {0x1.404p+10, 0x1.838p+10, 0x1.804p+10, 0x1.838p+10, 0x1p+8, 0x1.3641ffe003ff6p+10},
    {0x1p+8, 0x1.4p+10, 0x1.f9p+9, 0x1.4p+10, 0x1.79p+9, 0x0p+0},
    {0x1.f9p+9, 0x1.4p+10, 0x1.004p+10, 0x1.87p+9, 0x1.f239d17680fcep+8, 0x1.79p+9},
    {0x1.004p+10, 0x1.87p+9, 0x1.8p+10, 0x1.87p+9, 0x1.ffp+8, 0x1.390e745da03f4p+10},
    {0x1.8p+10, 0x1.87p+9, 0x1.002p+11, 0x1.87p+9, 0x1.008p+9, 0x0p+0},
    {0x1.002p+11, 0x1.87p+9, 0x1.002p+11, 0x1.17p+9, 0x1.cp+7, 0x1.008p+9},
    {0x1.002p+11, 0x1.17p+9, 0x1.072p+11, 0x1.07p+9, 0x1.01fe03f61bad0p+6, 0x1.708p+9},
    {0x1.072p+11, 0x1.07p+9, 0x1.3c2p+11, 0x1.07p+9, 0x1.a8p+8, 0x1.90bfc07ec375ap+9},
    {0x1.3c2p+11, 0x1.07p+9, 0x1.402p+11, 0x1.2ep+8, 0x1.c48c6001f0acp+7, 0x1.325fe03f61badp+10},
    {0x1.402p+11, 0x1.2ep+8, 0x1.472p+11, 0x1.06p+8, 0x1.13463fa37014ep+6, 0x1.6af16c3f9fd05p+10},
    {0x1.472p+11, 0x1.06p+8, 0x1.902p+11, 0x1.06p+8, 0x1.24p+9, 0x1.7c25d039d6d1ap+10},
    {0x1p+8, 0x1p+10, 0x1.008p+9, 0x1p+10, 0x1.01p+8, 0x0p+0},
    {0x1.008p+9, 0x1p+10, 0x1.008p+9, 0x1.2ep+8, 0x1.69p+9, 0x1.01p+8},
    {0x1.008p+9, 0x1.2ep+8, 0x1.1cp+9, 0x1.0ep+8, 0x1.fd0dd48f04c64p+5, 0x1.e98p+9},
    {0x1.1cp+9, 0x1.0ep+8, 0x1.3f2p+11, 0x1.0ep+8, 0x1.f04p+10, 0x1.04a86ea478263p+10},
    {0x1p+8, 0x1.8p+10, 0x1.fp+9, 0x1.8p+10, 0x1.7p+9, 0x0p+0},
    {0x1.fp+9, 0x1.8p+10, 0x1p+10, 0x1.b8p+10, 0x1.c48c6001f0acp+7, 0x1.7p+9},
    {0x1p+10, 0x1.b8p+10, 0x1.0c4p+10, 0x1.cp+10, 0x1.d4302088b1658p+5, 0x1.e12318007c2bp+9},
    {0x1.0c4p+10, 0x1.cp+10, 0x1.7bp+11, 0x1.cp+10, 0x1.e9cp+10, 0x1.fe661a0907416p+9},
    {0x1.7bp+11, 0x1.cp+10, 0x1.8p+11, 0x1.b38p+10, 0x1.001ffe003ff6p+6, 0x1.7479868241d06p+11},
    {0x1.8p+11, 0x1.b38p+10, 0x1.8p+11, 0x1.458p+10, 0x1.b8p+8, 0x1.7c7a867243d01p+11},
    {0x1p+8, 0x1.8p+9, 0x1.fcp+9, 0x1.8p+9, 0x1.7cp+9, 0x0p+0},
    {0x1.fcp+9, 0x1.8p+9, 0x1.004p+10, 0x1.0ep+8, 0x1.f214d14cc1837p+8, 0x1.7cp+9},
    {0x1.004p+10, 0x1.0ep+8, 0x1.0ep+10, 0x1.06p+8, 0x1.bca153b3343fp+5, 0x1.3a8534533060ep+10},
    {0x1.0ep+10, 0x1.06p+8, 0x1.f8p+10, 0x1.06p+8, 0x1.d4p+9, 0x1.486a3ef0ca02ep+10},
    {0x1.f8p+10, 0x1.06p+8, 0x1p+11, 0x1.38p+8, 0x1.dae803b4bc0c4p+5, 0x1.19351f7865017p+11},
    {0x1p+11, 0x1.38p+8, 0x1p+11, 0x1.ep+8, 0x1.5p+7, 0x1.20a0bf8737f1ap+11},
    {0x1p+11, 0x1.ep+8, 0x1.072p+11, 0x1p+9, 0x1.057906452f4c8p+6, 0x1.35a0bf8737f1ap+11},
    {0x1.072p+11, 0x1p+9, 0x1.a02p+11, 0x1p+9, 0x1.32p+10, 0x1.3dcc87b9616cp+11},
    {0x1p+8, 0x1.8p+10, 0x1.f88p+9, 0x1.8p+10, 0x1.788p+9, 0x0p+0},
    {0x1.f88p+9, 0x1.8p+10, 0x1.004p+10, 0x1.08p+8, 0x1.3e0670a3a21efp+10, 0x1.788p+9},
};
RL10G_TAB Rl10KageRoute kRl10KageRoutes[11] = {
    {0, 0, 1, 0x1.bep+10},           {1, 1, 4, 0x1.315f17caf6322p+10}, {2, 5, 1, 0x1.cp+10},
    {4, 6, 5, 0x1.79795f5d640dap+11}, {5, 11, 4, 0x1.7641ffe003ff6p+10}, {7, 15, 3, 0x1.b8ce745da03f4p+10},
    {8, 18, 7, 0x1.0712e81ceb68dp+11}, {10, 25, 4, 0x1.7a7437523c132p+11}, {11, 29, 6, 0x1.b37a867243d01p+11},
    {13, 35, 8, 0x1.d6cc87b9616cp+11}, {14, 43, 2, 0x1.fa4670a3a21efp+10},
};
RL10G_TAB Rl10KageBoss kRl10KageBosses[6] = {{0, 129, 20, 16}, {3, 128, 16, 16}, {6, 130, 31, 16},
                                              {9, 133, 51, 32}, {12, 132, 69, 28}, {14, 136, 79, 100}};

/* The route fraction of Kage at (cx, cy): the nearest point on the segments up to a lookahead past the best arc so
 * far (reward10.cuh:393-416). Returns 0 for Python's None (nothing within the allowed offset). */
RL10G_FN int rl10_kage_frac(Rl10Reader* e, int route, double cx, double cy, double* frac) {
    const Rl10KageRoute rt = kRl10KageRoutes[route];
    int have = 0;
    double bd = 0.0, barc = 0.0;
    for (int k = 0; k < rt.count; ++k) {
        const Rl10KageSeg g = kRl10KageSegs[rt.first + k];
        if (g.acc > e->best_arc + RL10_KAGE_LOOKAHEAD) break;
        double t = 0.0;
        if (g.len != 0.0) {
            const double num = (cx - g.x0) * (g.x1 - g.x0) + (cy - g.y0) * (g.y1 - g.y0);
            const double q = num / (g.len * g.len);
            const double m = 1.0 < q ? 1.0 : q;
            t = 0.0 < m ? m : 0.0;
        }
        const double d = rl10_hypot(g.x0 + t * (g.x1 - g.x0) - cx, g.y0 + t * (g.y1 - g.y0) - cy);
        if (!have || d < bd) {
            have = 1;
            bd = d;
            barc = g.acc + t * g.len;
        }
    }
    if (bd > RL10_KAGE_MAX_OFF) return 0;
    e->best_arc = e->best_arc >= barc ? e->best_arc : barc;
    *frac = barc / rt.total;
    return 1;
}

/* Kage (reward10.cuh:418-453): the fraction of the stage's route, and the boss's damage on boss stages */
RL10G_FN Rl10Signals rl10_kage(const uint8_t* r, Rl10Reader* e) {
    const int mode = rl10_u8(r, 2), stage = rl10_u8(r, 0x40), hp = rl10_u8(r, 0x6F0);
    if (!e->has_stage || stage != e->stage) {
        e->has_stage = 1;
        e->stage = stage;
        e->best_arc = 0.0;
    }
    const double cx = ((rl10_u8(r, 0x23) << 8) | rl10_u8(r, 0x22)) / 16.0;
    const double cy = ((rl10_u8(r, 0x25) << 8) | rl10_u8(r, 0x24)) / 16.0;
    const int play = mode == 0 && stage < 15;
    double progress = 0.0;
    int valid = play && hp > 0 && rl10_u8(r, 0x6A1) != 8;
    int route = -1, boss = -1;
    for (int i = 0; i < 11; ++i)
        if (route < 0 && kRl10KageRoutes[i].stage == stage) route = i;
    for (int i = 0; i < 6; ++i)
        if (kRl10KageBosses[i].stage == stage) boss = i;
    const double route_w = route < 0 ? 0.0 : (boss >= 0 ? 500.0 : 1000.0);
    if (play && route >= 0) {
        double f = 0.0;
        if (!rl10_kage_frac(e, route, cx, cy, &f)) valid = 0;
        else progress = route_w * f;
    }
    if (play && boss >= 0) {
        const Rl10KageBoss b = kRl10KageBosses[boss];
        if (rl10_u8(r, 0x708) == b.kind && rl10_u8(r, 0x798) == b.sel) {
            const int v = rl10_u8(r, 0x7F8), mx = b.max_hp;
            progress = route_w + (1000.0 - route_w) * ((double)(mx - (v < mx ? v : mx)) / mx);
        }
    }
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)(play && hp > 0 && rl10_u8(r, 0xD1) == 0);
    s.level = stage;
    s.progress = progress;
    s.progress_valid = (uint8_t)valid;
    s.dying = (uint8_t)(hp == 0 && stage < 15);
    s.has_health = 1;
    s.health = hp / 16.0;
    s.game_over = (uint8_t)(hp == 0 && mode != 0);
    s.won = (uint8_t)(stage == 0 && mode == 0x6B && rl10_u8(r, 0xAE) == 0xFF && rl10_u8(r, 0x708) == 0x88 &&
                      rl10_u8(r, 0x798) == 0x4F && rl10_u8(r, 0x7F8) == 0 && rl10_u8(r, 0x758) == 0x10 && hp > 0);
    return s;
}

#define RL10_FINAL_BOSS 0x1.2cp+8   /* 300 */

/* Final Mission (reward10.cuh:455-484): stage scroll, plus the boss's damage at the end of a stage */
RL10G_FN Rl10Signals rl10_finalmission(const uint8_t* r, Rl10Reader* e) {
    const int game = rl10_u8(r, 0x02) == 4 && rl10_u8(r, 0x03) == 0;
    const int routine = rl10_u8(r, 0x38);
    const int playing = game && routine == 4 && rl10_u8(r, 0x4F) >= 1 && rl10_u8(r, 0x85) == 0 &&
                        rl10_u8(r, 0x0E) == 0;
    const int level = rl10_u8(r, 0x1E);
    double progress = (double)(rl10_u8(r, 0x4F) * 32 + rl10_u8(r, 0x4E));
    if (game && routine == 4 && rl10_u8(r, 0x4D) == 0 && rl10_u8(r, 0x4F) >= 1) {
        int hp = 0;
        for (int a = 0x4A0; a < 0x4C0; ++a) hp = rl10_u8(r, a) > hp ? rl10_u8(r, a) : hp;
        if (!e->has_key || e->key_a != level || e->key_d != progress) {
            e->has_key = 1;
            e->key_a = level;
            e->key_d = progress;
            e->core_max = 0;
        }
        if (hp > e->core_max) e->core_max = hp;
        if (e->core_max >= 20) progress += RL10_FINAL_BOSS * ((double)(e->core_max - hp) / e->core_max);
    }
    const int pips = rl10_u8(r, 0x1C);
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)playing;
    s.level = level;
    s.progress = progress;
    s.progress_valid = (uint8_t)playing;
    s.dying = (uint8_t)(game && rl10_u8(r, 0x85) != 0);
    s.has_health = 1;
    s.health = (pips < 4 ? pips : 4) / 4.0;
    s.has_score = 1;
    s.score = 10LL * (rl10_u8(r, 0x8A) | (rl10_u8(r, 0x8B) << 8) | (rl10_u8(r, 0x8C) << 16));
    s.game_over = (uint8_t)(game && (routine == 7 || routine == 8));
    return s;
}

#define RL10_PUNCH_UNIT 0x1.2p+8   /* 288 */

/* Punch-Out (reward10.cuh:486-507): damage dealt in the current fight */
RL10G_FN Rl10Signals rl10_punchout(const uint8_t* r, Rl10Reader* e) {
    const int state = rl10_u8(r, 0x00), scene = rl10_u8(r, 0x05), fight = rl10_u8(r, 0x01);
    const int hp = rl10_u8(r, 0x398);
    if (!e->has_fight || fight != e->fight) {
        e->has_fight = 1;
        e->fight = fight;
        e->damage = 0;
        e->has_prev_hp = 0;
    }
    if (state == 1 && e->has_prev_hp && hp < e->prev_hp) e->damage += e->prev_hp - hp;
    e->has_prev_hp = 1;
    e->prev_hp = hp;
    const int playing = state == 1 && (scene == 0 || scene == 1) && rl10_u8(r, 0x300) == 1;
    const int loss = state == 249 || state == 251 || state == 253;
    const int winst = state == 250 || state == 252 || state == 254;
    const double hf = rl10_u8(r, 0x391) / 96.0;
    Rl10Signals s = rl10_blank();
    s.in_play = (uint8_t)playing;
    s.level = fight;
    s.progress = e->damage < RL10_PUNCH_UNIT ? (double)e->damage : RL10_PUNCH_UNIT;
    s.progress_valid = (uint8_t)playing;
    s.dying = (uint8_t)((state == 1 && scene == 2) || (loss && scene != 2));
    s.has_health = 1;
    s.health = hf < 1.0 ? hf : 1.0;
    s.has_score = 1;
    s.score = rl10_digits(r, 0x3E8, 0x3EE);
    s.game_over = (uint8_t)(loss || rl10_u8(r, 0x172) * 10 + rl10_u8(r, 0x173) > 0);
    s.won = (uint8_t)(winst && fight == 13);
    return s;
}

/* The signals of a game other than SMB from its 2 KB RAM (reward10.cuh:509-524). t: the tracker (its overflow flag),
 * e: the reader state, keys/cap: the env's key set. */
RL10G_FN Rl10Signals rl10_observe(int game, const uint8_t* r, Rl10State* t, Rl10Reader* e, uint32_t* keys,
                                  uint32_t cap) {
    switch (game) {
        case RL10_PACMAN: return rl10_pacman(r);
        case RL10_EXCITEBIKE: return rl10_excitebike(r, e);
        case RL10_CONTRA: return rl10_contra(r, e);
        case RL10_CASTLEVANIA: return rl10_castlevania(r, t, e, keys, cap);
        case RL10_GRADIUS: return rl10_gradius(r);
        case RL10_ZELDA: return rl10_zelda(r, t, e, keys, cap);
        case RL10_TETRIS: return rl10_tetris(r);
        case RL10_TECMOBOWL: return rl10_tecmobowl(r, e);
        case RL10_KAGE: return rl10_kage(r, e);
        case RL10_FINALMISSION: return rl10_finalmission(r, e);
        default: return rl10_punchout(r, e);
    }
}

#endif
