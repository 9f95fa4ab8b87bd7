/* ORACLE — test infrastructure only.
 *
 * CPU restatement of the env step around the emulator: controller/turbo/sticky/dropout (counter RNG), the
 * reward10 tracker with the SMB reader, the per-env phase order, boot snapshots and idle templates, and
 * the same C ABI as the HIP library (include/rlenv_api.h) over host memory, OpenMP over envs with
 * schedule(dynamic, 1) as the reference's CPU build does (rl/csrc/rlenv_cpu.cpp:34-45).
 *
 * Followed (kdcyberdude/ghostrun-lab):
 *   controller/RNG/dropout .. rl/csrc/controller.cuh:41-189
 *   reward10 tracker ........ rl/csrc/reward10.cuh:546-632, SMB reader 143-158, consts reward10_consts.h:24-39
 *   phases .................. rl/csrc/rlenv_core.cuh:138-414 (ph_frame, ph_render, reset_state, ph_finish,
 *                             ph_reset_idle, ph_reset_frame, ph_reset_finish_controls, env_start, env_step)
 *   build ................... rl/csrc/rlenv_build.hpp:193-366 (boot on the host, slot n = snapshot, idle
 *                             templates, episode counters start at 0xFFFFFFFF)
 *   resume blob order ....... rl/csrc/rlenv_build.hpp:253-280
 *   pack6 ................... rl/csrc/rlenv.cu:127-142
 */
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nes_oracle.h"
#include "rlenv_api.h"
#include "rl10_games.h"
#include "rlenv_state.h"

static __thread char g_err[256];

/* ------------------------------------------------------------------------------------- controller */

enum { BIT_A = 1, BIT_B = 2, BIT_SELECT = 4, BIT_START = 8, BIT_UP = 16, BIT_DOWN = 32, BIT_LEFT = 64, BIT_RIGHT = 128 };
enum { DROP_UP, DROP_DOWN, DROP_LEFT, DROP_RIGHT, DROP_AHOLD, DROP_BHOLD, DROP_TURBOA, DROP_TURBOB };

typedef struct Move { int dpad, a, b, start, select; } Move;

static uint32_t dpad_bits(int d) {
    static const uint8_t t[9] = {0, BIT_UP, BIT_UP | BIT_RIGHT, BIT_RIGHT, BIT_DOWN | BIT_RIGHT, BIT_DOWN,
                                 BIT_DOWN | BIT_LEFT, BIT_LEFT, BIT_UP | BIT_LEFT};
    return (d >= 0 && d < 9) ? t[d] : 0u;
}
static int dpad_from_bits(uint32_t bits) {
    for (int d = 0; d < 9; ++d)
        if (dpad_bits(d) == bits) return d;
    return 0;
}
static int move_pack(Move m) { return m.dpad + 9 * (m.a + 3 * (m.b + 3 * (m.start + 2 * m.select))); }
static Move move_unpack(int id) {
    Move m;
    m.dpad = id % 9; id /= 9;
    m.a = id % 3; id /= 3;
    m.b = id % 3; id /= 3;
    m.start = id % 2; id /= 2;
    m.select = id % 2;
    return m;
}
static uint8_t pad_byte(Move m, uint64_t frame) {
    const int even = (frame & 1u) == 0;
    uint32_t p = dpad_bits(m.dpad);
    if (m.a == 1 || (m.a == 2 && even)) p |= BIT_A;
    if (m.b == 1 || (m.b == 2 && even)) p |= BIT_B;
    if (m.start) p |= BIT_START;
    if (m.select) p |= BIT_SELECT;
    return (uint8_t)p;
}
static Move restrict_move(Move m, int dropped, int start_ok, int select_ok) {
    uint32_t bits = dpad_bits(m.dpad);
    if (dropped == DROP_UP) bits &= ~(uint32_t)BIT_UP;
    if (dropped == DROP_DOWN) bits &= ~(uint32_t)BIT_DOWN;
    if (dropped == DROP_LEFT) bits &= ~(uint32_t)BIT_LEFT;
    if (dropped == DROP_RIGHT) bits &= ~(uint32_t)BIT_RIGHT;
    m.dpad = dpad_from_bits(bits);
    if ((dropped == DROP_AHOLD && m.a == 1) || (dropped == DROP_TURBOA && m.a == 2)) m.a = 0;
    if ((dropped == DROP_BHOLD && m.b == 1) || (dropped == DROP_TURBOB && m.b == 2)) m.b = 0;
    if (!start_ok) m.start = 0;
    if (!select_ok) m.select = 0;
    return m;
}
/* raw pad mode: a dropped input clears its button */
static uint8_t restrict_pad(uint32_t p, int dropped) {
    static const uint8_t clear[8] = {BIT_UP, BIT_DOWN, BIT_LEFT, BIT_RIGHT, BIT_A, BIT_B, BIT_A, BIT_B};
    if (dropped >= 0 && dropped < 8) p &= ~(uint32_t)clear[dropped];
    return (uint8_t)p;
}

typedef struct Masks { uint32_t dpad, a, b, start, select; } Masks;
static Masks legal(int dropped, int start_ok, int select_ok) {
    Masks k = {0x1FF, 7, 7, start_ok ? 3u : 1u, select_ok ? 3u : 1u};
    uint32_t gone = 0;
    if (dropped == DROP_UP) gone = BIT_UP;
    if (dropped == DROP_DOWN) gone = BIT_DOWN;
    if (dropped == DROP_LEFT) gone = BIT_LEFT;
    if (dropped == DROP_RIGHT) gone = BIT_RIGHT;
    if (gone)
        for (int d = 0; d < 9; ++d)
            if (dpad_bits(d) & gone) k.dpad &= ~(1u << d);
    if (dropped == DROP_AHOLD) k.a &= ~2u;
    if (dropped == DROP_TURBOA) k.a &= ~4u;
    if (dropped == DROP_BHOLD) k.b &= ~2u;
    if (dropped == DROP_TURBOB) k.b &= ~4u;
    return k;
}

static uint64_t smix(uint64_t x) { return orc_splitmix64(x); }
static uint32_t rand_u32(uint64_t seed, uint64_t* counter) {
    const uint64_t c = (*counter)++;
    return (uint32_t)(smix(seed ^ smix(c)) >> 32);
}
static uint32_t rand_below(uint64_t seed, uint64_t* counter, uint32_t n) {
    return (uint32_t)(((uint64_t)rand_u32(seed, counter) * n) >> 32);
}
static uint64_t episode_seed(uint64_t run_seed, uint32_t env, uint64_t episode) {
    return smix(smix(run_seed ^ 0xD20F0D20F0ull) ^ ((uint64_t)env << 40) ^ episode);
}

static int32_t draw_gap(Dropout* s, uint32_t gap_p32) { /* Geometric on {1, 2, ...} by Bernoulli trials */
    int32_t k = 1;
    while (rand_u32(s->seed, &s->counter) >= gap_p32) ++k;
    return k;
}
static int8_t next_column(Dropout* s, uint32_t gap_p32) {
    if (s->drop_left > 0) {
        const int8_t out = (int8_t)s->drop_input;
        if (--s->drop_left == 0) s->gap_left = draw_gap(s, gap_p32);
        return out;
    }
    if (--s->gap_left == 0) {
        s->drop_input = (int32_t)rand_below(s->seed, &s->counter, RLE_DROP_INPUTS);
        s->drop_left = 8 + (int32_t)rand_below(s->seed, &s->counter, 22 - 8 + 1);
    }
    return -1;
}
static void dropout_reset(Dropout* s, uint64_t seed, int enabled, uint32_t gap_p32) {
    s->seed = seed;
    s->counter = 0;
    s->drop_left = 0;
    s->drop_input = -1;
    s->head = 0;
    s->gap_left = enabled ? draw_gap(s, gap_p32) : 0x7FFFFFFF;
    for (int j = 0; j < RLC_RING; ++j) s->ring[j] = -1;
    for (int j = 0; j < RLE_TIMELINE; ++j) s->ring[j] = enabled ? next_column(s, gap_p32) : (int8_t)-1;
}
static int dropped_now(const Dropout* s) { return s->ring[s->head % RLC_RING]; }
static void dropout_advance(Dropout* s, int enabled, uint32_t gap_p32) {
    s->ring[s->head % RLC_RING] = -1;
    ++s->head;
    s->ring[(s->head + RLE_TIMELINE - 1) % RLC_RING] = enabled ? next_column(s, gap_p32) : (int8_t)-1;
}
static void timeline(const Dropout* s, uint8_t* out) {
    memset(out, 0, RLE_TIMELINE_BYTES);
    for (int j = 0; j < RLE_TIMELINE; ++j) {
        const int b = s->ring[(s->head + (uint32_t)j) % RLC_RING];
        if (b >= 0) out[b * RLE_TIMELINE + j] = 1;
    }
}

/* ------------------------------------------------------------------------------------- reward10 (SMB) */

#define W_PROGRESS 0x1.0000000000000p+0
#define W_LEVEL 0x1.0000000000000p+0
#define W_DEATH -0x1.999999999999ap-4
#define W_STALL -0x1.999999999999ap-4
#define W_SCORE 0x1.47ae147ae147bp-6
#define SCORE_CAP 0x1.999999999999ap-4
#define SCORE_LEVEL_BUDGET 0x1.999999999999ap-3
#define W_WIN 0x1.4000000000000p+2
#define W_ROLLBACK -0x1.47ae147ae147bp-6
#define ROLLBACK_DROP 0x1.0000000000000p-2
#define SMB_PROGRESS_UNIT 0x1.7700000000000p+11 /* 3000 */
#define SMB_SCORE_UNIT 0x1.9000000000000p+7     /* 200 */
#define SMB_STALL_FRAMES 0x1.c200000000000p+12  /* 7200 */
#define SMB_IDLE_PER_FRAME -0x1.0624dd2f1a9fcp-12

enum { EV_SKIP = 1, EV_LEVEL = 2, EV_DEATH = 4, EV_WON = 8, EV_GAMEOVER = 16, EV_STALL = 32, EV_ROLLBACK = 64 };
enum { END_NONE = 0, END_GAMEOVER = 1, END_WON = 2, END_SKIP = 3, END_STALL = 4 };
enum { P_PROGRESS, P_LEVEL, P_DEATH, P_DAMAGE, P_SCORE, P_WIN, P_STALL };

typedef struct Rl10Update {
    double reward;
    int done;
    uint32_t events;
    int event_level;
    double part[RLE_PARTS];
} Rl10Update;

/* the 15 bytes the SMB reader reads, in the packed order of rl10_smb_run */
static const uint16_t kSmbAddr[15] = {0x0E, 0x6D, 0x86, 0xB5, 0x75A, 0x75C, 0x75F, 0x770, 0x772,
                                      0x7DD, 0x7DE, 0x7DF, 0x7E0, 0x7E1, 0x7E2};

static Rl10Signals observe_smb(const uint8_t* b15) { /* b15: bytes in kSmbAddr order */
    const int routine = b15[0], page = b15[1], x = b15[2], b5 = b15[3], lives = b15[4], lv = b15[5], world = b15[6],
              mode = b15[7], task = b15[8];
    Rl10Signals s;
    memset(&s, 0, sizeof(s));
    s.in_play = mode == 1 && task == 3;
    s.level = world * 4 + lv;
    s.progress = (double)((page > 127 ? page - 256 : page) * 256 + x);
    s.progress_valid = mode == 1 && task == 3 && routine == 8;
    s.dying = mode == 1 && (routine == 6 || routine == 0xB || (routine == 8 && b5 >= 2));
    s.has_lives = 1;
    s.lives = lives > 127 ? lives - 256 : lives;
    s.has_score = 1;
    int64_t v = 0;
    for (int i = 9; i < 15; ++i) v = v * 10 + b15[i];
    s.score = v * 10;
    s.game_over = mode == 3;
    s.won = mode == 2 && world == 7;
    return s;
}

static void rl10_reset(Rl10State* e) { memset(e, 0, sizeof(*e)); }

typedef struct Rl10Consts {  /* one game's row of kGameConsts (reward10_consts.h:23-37) */
    double progress_unit, score_unit, stall_frames /* < 0: no stall limit */, idle_per_frame;
    int death_from_lives;
} Rl10Consts;
static const Rl10Consts kSmbConsts = {SMB_PROGRESS_UNIT, SMB_SCORE_UNIT, SMB_STALL_FRAMES, SMB_IDLE_PER_FRAME, 0};
#define W_DAMAGE -0x1.0000000000000p-2

/* RewardTracker.update (rl/csrc/reward10.cuh:546-632): doubles in Python's evaluation order. */
static Rl10Update rl10_update_sig(const Rl10Signals* sp, int frames, Rl10State* e, const Rl10Consts* G) {
    const Rl10Signals s = *sp;
    const int has_p = e->has_prev;
    const Rl10Signals p = e->prev;
    double r = 0.0;
    uint32_t ev = 0;
    int ev_level = 0, fresh = 0;
    double part[RLE_PARTS] = {0, 0, 0, 0, 0, 0, 0};
    Rl10Update out;
    memset(&out, 0, sizeof(out));
    out.done = 1;
    e->has_prev = 1;
    e->prev = s;
    if (e->done) return out;
    if (s.in_play) {
        if (!e->has_best_level) {
            e->has_best_level = 1;
            e->best_level = s.level;
            e->has_best_progress = 0;
            e->score_used = 0.0;
        } else if (s.level > e->best_level + 1) {
            ev |= EV_SKIP;
            ev_level = s.level;
            e->done = 1;
            e->end_reason = END_SKIP;
        } else if (s.level > e->best_level) {
            r += W_LEVEL;
            part[P_LEVEL] += W_LEVEL;
            ev |= EV_LEVEL;
            ev_level = s.level;
            e->best_level = s.level;
            e->has_best_progress = 0;
            e->score_used = 0.0;
            fresh = 1;
        }
        if (s.level == e->best_level && s.progress_valid) {
            if (!e->has_best_progress) {
                e->has_best_progress = 1;
                e->best_progress = s.progress;
            } else if (s.progress > e->best_progress) {
                const double rp = W_PROGRESS * (s.progress - e->best_progress) / G->progress_unit;
                r += rp;
                part[P_PROGRESS] += rp;
                e->best_progress = s.progress;
                fresh = 1;
            }
        }
    }
    int death = 0;
    if (has_p) {
        if (!G->death_from_lives) death = s.dying && !p.dying;
        else death = s.has_lives && p.has_lives && s.lives < p.lives;
        if (death && (s.in_play || p.in_play)) {
            r += W_DEATH;
            part[P_DEATH] += W_DEATH;
            e->deaths += 1;
            ev |= EV_DEATH;
            fresh = 1;
        }
        if (s.in_play && p.in_play && s.has_health && p.has_health && s.health < p.health) {
            const double rd = W_DAMAGE * (p.health - s.health);
            r += rd;
            part[P_DAMAGE] += rd;
        }
        if (s.in_play && p.in_play && s.has_score && p.has_score && s.score > p.score) {
            double sr = W_SCORE * (double)(s.score - p.score) / G->score_unit;
            if (SCORE_CAP < sr) sr = SCORE_CAP;
            const double left = SCORE_LEVEL_BUDGET - e->score_used;
            if (left < sr) sr = left;
            if (sr > 0) {
                r += sr;
                part[P_SCORE] += sr;
                e->score_used += sr;
            }
        }
    }
    if (has_p && !e->done && !death && !s.dying && !p.dying && !s.won && !s.game_over && s.in_play && p.in_play &&
        s.progress_valid && p.progress_valid && s.level == p.level && s.level == e->best_level &&
        p.progress - s.progress >= ROLLBACK_DROP * G->progress_unit) {
        r += W_ROLLBACK;
        part[P_STALL] += W_ROLLBACK;
        ev |= EV_ROLLBACK;
    }
    if (!fresh && !e->done && has_p && s.in_play && p.in_play && s.progress_valid && p.progress_valid &&
        s.progress <= p.progress) {
        const double ci = G->idle_per_frame * frames;
        r += ci;
        part[P_STALL] += ci;
    }
    e->idle_frames = (fresh || !has_p) ? 0 : e->idle_frames + frames;
    if (s.won) {
        r += W_WIN;
        part[P_WIN] += W_WIN;
        ev |= EV_WON;
        e->done = 1;
        e->end_reason = END_WON;
    } else if (s.game_over) {
        ev |= EV_GAMEOVER;
        e->done = 1;
        e->end_reason = END_GAMEOVER;
    } else if (!e->done && G->stall_frames >= 0.0 && (double)e->idle_frames >= G->stall_frames) {
        r += W_STALL;
        part[P_STALL] += W_STALL;
        ev |= EV_STALL;
        e->done = 1;
        e->end_reason = END_STALL;
    }
    out.reward = r;
    out.done = e->done;
    out.events = ev;
    out.event_level = ev_level;
    memcpy(out.part, part, sizeof(part));
    return out;
}

static Rl10Update rl10_update(const uint8_t* b15, int frames, Rl10State* e) {
    const Rl10Signals s = observe_smb(b15);
    return rl10_update_sig(&s, frames, e, &kSmbConsts);
}

/* RewardTracker.update for any game (rl/csrc/reward10.cuh:546-548): the game's reader on the 2 KB RAM (SMB's own
 * above, the others in include/rl10_games.h), then the tracker with the game's constants. rd/keys/cap: the env's
 * reader state and key set (unused by SMB). */
static Rl10Update rl10_update_game(int game, const uint8_t* ram, int frames, Rl10State* e, Rl10Reader* rd,
                                   uint32_t* keys, uint32_t cap) {
    if (game == RL10_SMB) {
        uint8_t b15[15];
        for (int i = 0; i < 15; ++i) b15[i] = ram[kSmbAddr[i]];
        return rl10_update(b15, frames, e);
    }
    const Rl10Game gc = rl10_game(game);
    const Rl10Consts G = {gc.progress_unit, gc.score_unit, gc.stall_frames, gc.idle_per_frame, gc.death_from_lives};
    const Rl10Signals s = rl10_observe(game, ram, e, rd, keys, cap);
    return rl10_update_sig(&s, frames, e, &G);
}

static void gather15(const uint8_t* ram, uint8_t* b15) {
    for (int i = 0; i < 15; ++i) b15[i] = ram[kSmbAddr[i]];
}

/* --------------------------------------------------------------------------------------------- env */

typedef struct Game {
    NesCart cart;
    uint8_t* prg;      /* padded PRG image */
    uint8_t* rom;      /* iNES copy (CHR points into it) */
    int game, n, offset, start_ok, select_ok;
    uint32_t kcap;     /* key-set entries per env (rl10_keyset_capacity) */
    uint32_t* keys;    /* [n * kcap] */
    NesRec* recs;      /* n + 1 records; slot n = boot snapshot */
    NesRec* idle;      /* idle_max templates: the snapshot after k = 1..idle_max neutral frames */
    uint64_t tmpl_target;
    /* level starts / places (rl/csrc/rlenv_core.cuh:60-74; lv_cap = 0: off): slot s < lv_levels is level s, saved on
     * the level event; slots lv_levels..lv_cap-1 are places, saved on request. One saved console is a whole record. */
    int lv_cap, lv_levels;
    NesRec* lv_rec;           /* [lv_cap] */
    Rl10Saved* lv_st;         /* [lv_cap] tracker + reader per slot */
    uint32_t* lv_keys;        /* [lv_cap * kcap] */
    uint64_t* lv_target;      /* [lv_cap] */
    uint32_t* lv_frame;       /* [lv_cap] */
    int32_t* lv_deaths;       /* [lv_cap], -1 = nothing saved */
    uint64_t* lv_claim;       /* [lv_cap] (deaths << 32 | env) of this decision's best arrival, ~0 = none */
    uint32_t* lv_cdf;         /* [lv_cap] cumulative level weights * 2^32 */
    uint32_t lv_thresh;       /* P(a new episode starts from a saved level) * 2^32 */
    int lv_weighted;
} Game;

typedef struct Env {
    int ngames, total;
    Game* games;
    int idle_tmpl;
    /* per env */
    Rl10State* st;
    Rl10Reader* rd;
    Dropout* drop;
    uint64_t *target, *sticky_seed, *sticky_ctr;
    uint32_t *ep_frame, *episode, *fault;
    int16_t* prev_applied;
    float* ep_ret;
    int32_t *ep_len, *ep_maxlvl, *ep_idle;
    uint8_t* resetting;
    int lv_cap;               /* level starts on (every game has the same cap) */
    int32_t* ep_start;        /* [N] slot the current episode started from, -1 = boot snapshot (with lv_cap) */
    /* bound buffers */
    const int16_t* actions;
    uint8_t *obs, *emph, *done, *masks, *tl, *pads;
    float *reward, *info, *parts;
    uint32_t* events;
    uint64_t* ram_hash;
    int32_t *start_out, *level_out;
    float* progress_out;
    /* settings */
    uint64_t run_seed;
    int sticky, idle_max, dropout, no_render, episode_level_end, pad_mode;
    uint32_t end_p32, gap_p32;
    uint32_t budget;          /* instructions per frame: NES_BUDGET, or RLENV_BUDGET (diagnostics of the budget exit) */
} Env;

static void emu_frame(Env* E, Game* g, int e, int ge, uint8_t pad) {
    NesRec* r = &g->recs[e];
    r->pad = pad;
    if (E->fault[ge] == 0) {
        const uint32_t f = orc_run_until_budget(r, &g->cart, E->target[ge], E->budget);
        if (f) E->fault[ge] = f;
    }
    E->target[ge] += NES_FRAME_DOTS;
    ++E->ep_frame[ge];
}

static void ph_frame(Env* E, Game* g, int e, int f) {
    const int ge = g->offset + e;
    const int d = dropped_now(&E->drop[ge]);
    uint8_t pad;
    if (E->pad_mode) {
        uint32_t p = (uint16_t)E->actions[ge] & 0xFFu;
        if (E->sticky && rand_u32(E->sticky_seed[ge], &E->sticky_ctr[ge]) < RLC_STICKY_P32)
            p = (uint16_t)E->prev_applied[ge] & 0xFFu;
        pad = restrict_pad(p, d);
        E->prev_applied[ge] = pad;
    } else {
        Move m = move_unpack(E->actions[ge]);
        if (E->sticky && rand_u32(E->sticky_seed[ge], &E->sticky_ctr[ge]) < RLC_STICKY_P32)
            m = restrict_move(move_unpack(E->prev_applied[ge]), d, g->start_ok, g->select_ok);
        E->prev_applied[ge] = (int16_t)move_pack(m);
        pad = pad_byte(m, E->ep_frame[ge]);
    }
    E->pads[(size_t)ge * RLE_FRAMES + f] = pad;
    emu_frame(E, g, e, ge, pad);
}

static void ph_render(Env* E, Game* g, int e, int f, int restart_pass) {
    const int ge = g->offset + e;
    if (restart_pass && E->resetting[ge] == 0) return;
    if (E->no_render) return;
    orc_render_obs(&g->recs[e], &g->cart, E->obs + ((size_t)ge * RLE_FRAMES + f) * RLE_OBS_PIXELS,
                   E->emph + ((size_t)ge * RLE_FRAMES + f) * RLE_OBS_H);
}

static void reset_state(Env* E, Game* g, int e) {
    const int ge = g->offset + e;
    const uint32_t ep = ++E->episode[ge];
    const uint64_t seed = episode_seed(E->run_seed, (uint32_t)ge, ep);
    E->sticky_seed[ge] = smix(seed ^ 0x5717C4A55EEDull);
    E->sticky_ctr[ge] = 0;
    int idle = 0;
    if (E->idle_max > 0) idle = (int)rand_below(E->sticky_seed[ge], &E->sticky_ctr[ge], (uint32_t)(E->idle_max + 1));
    /* a level start? (rlenv_core.cuh:220-236; drawn only when level starts are on) */
    int lv = -1;
    if (g->lv_cap > 0 && g->lv_thresh != 0 && rand_u32(E->sticky_seed[ge], &E->sticky_ctr[ge]) < g->lv_thresh) {
        uint32_t saved = 0;
        for (int s = 0; s < g->lv_cap; ++s) saved += g->lv_deaths[s] >= 0 ? 1u : 0u;
        if (g->lv_weighted) {
            const uint32_t u = rand_u32(E->sticky_seed[ge], &E->sticky_ctr[ge]);
            for (int s = 0; s < g->lv_cap && lv < 0; ++s)
                if (u < g->lv_cdf[s]) lv = s;
        } else if (saved > 0) {
            uint32_t pick = rand_below(E->sticky_seed[ge], &E->sticky_ctr[ge], saved);
            for (int s = 0; s < g->lv_cap && lv < 0; ++s)
                if (g->lv_deaths[s] >= 0 && pick-- == 0) lv = s;
        }
    }
    const int k = lv < 0 && idle <= E->idle_tmpl ? idle : 0;
    memcpy(&g->recs[e], lv >= 0 ? &g->lv_rec[lv] : k == 0 ? &g->recs[g->n] : &g->idle[k - 1], sizeof(NesRec));
    uint32_t* keys = g->keys + (size_t)e * g->kcap;
    if (lv >= 0) {
        E->target[ge] = g->lv_target[lv];
        E->ep_frame[ge] = g->lv_frame[lv];
        E->st[ge] = g->lv_st[lv].st;
        E->rd[ge] = g->lv_st[lv].rd;
        memcpy(keys, g->lv_keys + (size_t)lv * g->kcap, (size_t)g->kcap * 4u);
    } else {
        E->target[ge] = g->tmpl_target + (uint64_t)k * NES_FRAME_DOTS;
        E->ep_frame[ge] = (uint32_t)k;
        rl10_reset(&E->st[ge]);   /* and the reader and its key set (reward10.cuh:531-532) */
        memset(&E->rd[ge], 0, sizeof(Rl10Reader));
        memset(keys, 0, (size_t)g->kcap * 4u);
    }
    if (E->ep_start) E->ep_start[ge] = lv;
    E->fault[ge] = 0;
    dropout_reset(&E->drop[ge], seed, E->dropout != 0, E->gap_p32);
    E->prev_applied[ge] = 0;
    E->ep_idle[ge] = idle;
    E->resetting[ge] = 1;
}

static void write_controls(Env* E, Game* g, int ge) {
    const int d = dropped_now(&E->drop[ge]);
    const Masks k = legal(d, g->start_ok, g->select_ok);
    uint8_t* m = E->masks + (size_t)ge * RLE_MASK_BYTES;
    for (int i = 0; i < 9; ++i) m[i] = (k.dpad >> i) & 1u;
    for (int i = 0; i < 3; ++i) m[9 + i] = (k.a >> i) & 1u;
    for (int i = 0; i < 3; ++i) m[12 + i] = (k.b >> i) & 1u;
    for (int i = 0; i < 2; ++i) m[15 + i] = (k.start >> i) & 1u;
    for (int i = 0; i < 2; ++i) m[17 + i] = (k.select >> i) & 1u;
    timeline(&E->drop[ge], E->tl + (size_t)ge * RLE_TIMELINE_BYTES);
}

static void ph_finish(Env* E, Game* g, int e) {
    const int ge = g->offset + e;
    const Rl10Update u = rl10_update_game(g->game, g->recs[e].ram, RLE_FRAMES, &E->st[ge], &E->rd[ge],
                                          g->keys + (size_t)e * g->kcap, g->kcap);
    const int faulted = E->fault[ge] != 0;
    const int level_clear = !u.done && !faulted && E->episode_level_end >= 0 && (u.events & EV_LEVEL) &&
                            u.event_level == E->episode_level_end + 1;
    int synthetic = 0;
    if (E->end_p32 != 0 && !u.done && !faulted && !level_clear) {
        uint64_t ctr = (uint64_t)(uint32_t)E->ep_len[ge];
        const uint64_t es = smix(episode_seed(E->run_seed, (uint32_t)ge, E->episode[ge]) ^ 0xE9D5EEDull);
        synthetic = rand_u32(es, &ctr) < E->end_p32;
    }
    const int done = u.done || faulted || level_clear || synthetic;
    const float r = faulted ? 0.0f : (float)u.reward;
    E->reward[ge] = r;
    if (E->parts)
        for (int k = 0; k < RLE_PARTS; ++k) E->parts[(size_t)ge * RLE_PARTS + k] = faulted ? 0.0f : (float)u.part[k];
    E->done[ge] = (uint8_t)(done ? 1 : 0);
    E->events[ge] = u.events;
    E->ep_ret[ge] += r;
    ++E->ep_len[ge];
    if (u.event_level > E->ep_maxlvl[ge]) E->ep_maxlvl[ge] = u.event_level;
    dropout_advance(&E->drop[ge], E->dropout != 0, E->gap_p32);
    /* level-start claim: the arrival with the fewest deaths, then the lowest env index (rlenv_core.cuh:288-291) */
    if (g->lv_cap > 0 && !done && (u.events & EV_LEVEL) && u.event_level >= 0 && u.event_level < g->lv_levels) {
        const uint64_t d = (uint64_t)(uint32_t)(E->st[ge].deaths < 0 ? 0 : E->st[ge].deaths);
        const uint64_t v = (d << 32) | (uint32_t)e;
        uint64_t cur = __atomic_load_n(&g->lv_claim[u.event_level], __ATOMIC_RELAXED);
        while (v < cur && !__atomic_compare_exchange_n(&g->lv_claim[u.event_level], &cur, v, 1, __ATOMIC_RELAXED,
                                                       __ATOMIC_RELAXED)) {
        }
    }
    if (E->level_out) E->level_out[ge] = E->st[ge].has_best_level ? E->st[ge].best_level : -1;
    if (E->progress_out)
        E->progress_out[ge] = E->st[ge].has_prev && E->st[ge].prev.progress_valid
                                  ? (float)(E->st[ge].prev.progress / rl10_game(g->game).progress_unit) : NAN;
    if (done) {
        if (E->start_out) E->start_out[ge] = E->ep_start ? E->ep_start[ge] : -1;
        float* inf = E->info + (size_t)ge * RLE_INFO;
        inf[0] = E->ep_ret[ge];
        inf[1] = (float)E->ep_len[ge];
        inf[2] = (float)(faulted ? RLE_END_FAULT
                                 : level_clear ? RLE_END_LEVEL_CLEAR
                                               : synthetic ? RLE_END_SYNTHETIC : E->st[ge].end_reason);
        inf[3] = (float)E->st[ge].deaths;
        inf[4] = (float)E->ep_maxlvl[ge];
        inf[5] = E->st[ge].overflow ? 1.0f : 0.0f;
        inf[6] = (float)E->ep_idle[ge];
        inf[7] = (float)E->episode[ge];
        reset_state(E, g, e);
    }
}

static void ph_reset_idle(Env* E, Game* g, int e) {
    const int ge = g->offset + e;
    if (E->resetting[ge] == 0) return;
    const int lv = E->ep_start && E->ep_start[ge] >= 0;   /* a level start: every idle frame is emulated */
    const int done = !lv && E->ep_idle[ge] <= E->idle_tmpl ? E->ep_idle[ge] : 0;
    for (int i = done; i < E->ep_idle[ge]; ++i) emu_frame(E, g, e, ge, 0);
}

static void ph_reset_frame(Env* E, Game* g, int e) {
    const int ge = g->offset + e;
    if (E->resetting[ge] == 0) return;
    emu_frame(E, g, e, ge, 0);
}

static void ph_reset_finish_controls(Env* E, Game* g, int e) {
    const int ge = g->offset + e;
    if (E->resetting[ge] != 0) {
        (void)rl10_update_game(g->game, g->recs[e].ram, E->ep_idle[ge] + RLE_FRAMES, &E->st[ge], &E->rd[ge],
                               g->keys + (size_t)e * g->kcap, g->kcap);
        E->ep_ret[ge] = 0.0f;
        E->ep_len[ge] = 0;
        const int sl = E->ep_start ? E->ep_start[ge] : -1;   /* a place: its level is the tracker's */
        E->ep_maxlvl[ge] = sl >= g->lv_levels ? (E->st[ge].has_best_level ? E->st[ge].best_level : 0) : sl > 0 ? sl : 0;
        E->resetting[ge] = 0;
    }
    write_controls(E, g, ge);
}

static void restart_phases(Env* E, Game* g, int e) {
    ph_reset_idle(E, g, e);
    for (int f = 0; f < RLE_FRAMES; ++f) {
        ph_reset_frame(E, g, e);
        ph_render(E, g, e, f, 1);
    }
    ph_reset_finish_controls(E, g, e);
}

static void env_step_one(Env* E, Game* g, int e) {
    const int ge = g->offset + e;
    for (int f = 0; f < RLE_FRAMES; ++f) {
        ph_frame(E, g, e, f);
        ph_render(E, g, e, f, 0);
    }
    if (E->ram_hash) E->ram_hash[ge] = orc_ram_hash(g->recs[e].ram);
    ph_finish(E, g, e);
    restart_phases(E, g, e);
}

static Game* game_of(Env* E, int k, int* e) {
    int gi = 0;
    while (k >= E->games[gi].offset + E->games[gi].n) ++gi;
    *e = k - E->games[gi].offset;
    return &E->games[gi];
}

/* ------------------------------------------------------------------------------------------- build */

static void* xcalloc(size_t n, size_t sz) {
    void* p = calloc(n ? n : 1, sz ? sz : 1);
    if (!p) {
        fprintf(stderr, "oracle: out of memory\n");
        abort();
    }
    return p;
}

static void env_free(Env* E) {
    if (!E) return;
    for (int i = 0; i < E->ngames; ++i) {
        free(E->games[i].prg);
        free(E->games[i].rom);
        free(E->games[i].recs);
        free(E->games[i].idle);
        free(E->games[i].lv_rec); free(E->games[i].lv_st); free(E->games[i].lv_target); free(E->games[i].lv_frame);
        free(E->games[i].lv_deaths); free(E->games[i].lv_claim); free(E->games[i].lv_cdf);
        free(E->games[i].lv_keys); free(E->games[i].keys);
    }
    free(E->games);
    free(E->st); free(E->rd); free(E->drop); free(E->target); free(E->sticky_seed); free(E->sticky_ctr);
    free(E->ep_frame); free(E->episode); free(E->fault); free(E->prev_applied); free(E->ep_ret);
    free(E->ep_len); free(E->ep_maxlvl); free(E->ep_idle); free(E->resetting); free(E->ep_start);
    free(E);
}

void* rlenv_create(int ngames, const int* game_ids, const uint8_t* const* roms, const size_t* rom_sizes,
                   const uint8_t* const* boot_pads, const size_t* boot_sizes, const int* n_envs, uint64_t run_seed,
                   int sticky, int idle_max, int dropout, int device) {
    (void)device;
    Env* E = (Env*)xcalloc(1, sizeof(Env));
    E->ngames = ngames;
    E->games = (Game*)xcalloc((size_t)ngames, sizeof(Game));
    E->run_seed = run_seed;
    E->sticky = sticky;
    E->idle_max = idle_max;
    E->dropout = dropout;
    E->idle_tmpl = idle_max > 0 ? idle_max : 0;
    E->episode_level_end = -1;
    E->gap_p32 = RLC_GAP_P32;
    E->budget = NES_BUDGET;
    {   /* the HIP library's diagnostic knob, read the same way */
        const char* v = getenv("RLENV_BUDGET");
        if (v) {
            const int b = atoi(v);
            E->budget = (uint32_t)(b < 1 ? 1 : b > (int)NES_BUDGET ? (int)NES_BUDGET : b);
        }
    }
    for (int i = 0; i < ngames; ++i) {
        Game* g = &E->games[i];
        if (game_ids[i] < 0 || game_ids[i] >= RL10_NUM_GAMES) {
            snprintf(g_err, sizeof(g_err), "game id %d: the reward10 games are 0..%d", game_ids[i],
                     RL10_NUM_GAMES - 1);
            env_free(E);
            return NULL;
        }
        g->game = game_ids[i];
        g->kcap = rl10_keyset_capacity(g->game);
        g->keys = (uint32_t*)xcalloc((size_t)n_envs[i] * g->kcap + 1u, 4);
        g->n = n_envs[i];
        g->offset = E->total;
        E->total += n_envs[i];
        g->rom = (uint8_t*)xcalloc(rom_sizes[i], 1);
        memcpy(g->rom, roms[i], rom_sizes[i]);
        g->prg = (uint8_t*)xcalloc(1u << 20, 1);
        if (orc_parse_ines(g->rom, (uint32_t)rom_sizes[i], g->prg, 1u << 20, &g->cart, g_err, sizeof(g_err)) != 0) {
            env_free(E);
            return NULL;
        }
        g->recs = (NesRec*)xcalloc((size_t)g->n + 1, sizeof(NesRec));
        g->idle = (NesRec*)xcalloc((size_t)(E->idle_tmpl ? E->idle_tmpl : 1), sizeof(NesRec));
        NesRec* boot = &g->recs[g->n];
        orc_power_on(boot, &g->cart);
        uint64_t target = NES_VBLANK_DOT;
        for (size_t f = 0; f < boot_sizes[i]; ++f) {
            boot->pad = boot_pads[i][f];
            if (orc_run_until_budget(boot, &g->cart, target, E->budget) != 0) {
                snprintf(g_err, sizeof(g_err), "emulator fault during boot of game %d", g->game);
                env_free(E);
                return NULL;
            }
            target += NES_FRAME_DOTS;
        }
        g->tmpl_target = target;
        NesRec tmp = *boot;
        for (int k = 1; k <= E->idle_tmpl; ++k) {
            tmp.pad = 0;
            if (orc_run_until_budget(&tmp, &g->cart, target, E->budget) != 0) {
                snprintf(g_err, sizeof(g_err), "emulator fault in idle frames of game %d", g->game);
                env_free(E);
                return NULL;
            }
            target += NES_FRAME_DOTS;
            g->idle[k - 1] = tmp;
        }
        g->start_ok = rl10_game(g->game).start_ok;   /* reward10_consts.h:25-37 */
        g->select_ok = rl10_game(g->game).select_ok;
    }
    const size_t N = (size_t)E->total;
    E->st = (Rl10State*)xcalloc(N, sizeof(Rl10State));
    E->rd = (Rl10Reader*)xcalloc(N, sizeof(Rl10Reader));
    E->drop = (Dropout*)xcalloc(N, sizeof(Dropout));
    E->target = (uint64_t*)xcalloc(N, 8);
    E->sticky_seed = (uint64_t*)xcalloc(N, 8);
    E->sticky_ctr = (uint64_t*)xcalloc(N, 8);
    E->ep_frame = (uint32_t*)xcalloc(N, 4);
    E->episode = (uint32_t*)xcalloc(N, 4);
    for (size_t i = 0; i < N; ++i) E->episode[i] = 0xFFFFFFFFu;
    E->fault = (uint32_t*)xcalloc(N, 4);
    E->prev_applied = (int16_t*)xcalloc(N, 2);
    E->ep_ret = (float*)xcalloc(N, 4);
    E->ep_len = (int32_t*)xcalloc(N, 4);
    E->ep_maxlvl = (int32_t*)xcalloc(N, 4);
    E->ep_idle = (int32_t*)xcalloc(N, 4);
    E->resetting = (uint8_t*)xcalloc(N, 1);
    return E;
}

int rlenv_num_envs(void* h) { return ((Env*)h)->total; }
int rlenv_num_games(void* h) { return ((Env*)h)->ngames; }
void rlenv_set_episode_level_end(void* h, int level) { ((Env*)h)->episode_level_end = level; }
void rlenv_set_no_render(void* h, int v) { ((Env*)h)->no_render = v; }
void rlenv_set_pad_mode(void* h, int raw) { ((Env*)h)->pad_mode = raw; }
void rlenv_set_end_prob(void* h, uint32_t p) { ((Env*)h)->end_p32 = p; }
void rlenv_set_dropout_gap(void* h, uint32_t p) { ((Env*)h)->gap_p32 = p; }
void rlenv_bind_ram_hash(void* h, uint64_t* out) { ((Env*)h)->ram_hash = out; }

void rlenv_bind(void* h, const int16_t* actions, uint8_t* obs, uint8_t* emph, float* reward, uint8_t* done,
                uint8_t* masks, uint8_t* tl, uint8_t* pads, uint32_t* events, float* info) {
    Env* E = (Env*)h;
    E->actions = actions; E->obs = obs; E->emph = emph; E->reward = reward; E->done = done; E->masks = masks;
    E->tl = tl; E->pads = pads; E->events = events; E->info = info;
}
void rlenv_bind_parts(void* h, float* parts) { ((Env*)h)->parts = parts; }
void rlenv_bind_obs(void* h, uint8_t* obs, uint8_t* emph) {
    ((Env*)h)->obs = obs;
    ((Env*)h)->emph = emph;
}

int rlenv_start(void* h, void* stream) {
    (void)stream;
    Env* E = (Env*)h;
#pragma omp parallel for schedule(dynamic, 1)
    for (int k = 0; k < E->total; ++k) {
        int e;
        Game* g = game_of(E, k, &e);
        reset_state(E, g, e);
        restart_phases(E, g, e);
    }
    return 0;
}

/* Level-start saves of game g after its envs' finish (rlenv_core.cuh:343-387, rl/csrc/rlenv_cpu.cpp:108-117). */
static void level_saves(Env* E, Game* g) {
    for (int s = 0; s < g->lv_levels; ++s) {
        const uint64_t cl = g->lv_claim[s];
        if (cl == ~0ull) continue;
        const int take = g->lv_deaths[s] < 0 || (int32_t)(cl >> 32) <= g->lv_deaths[s];
        if (take) {
            const int e = (int)(cl & 0xFFFFFFFFull), ge = g->offset + e;
            g->lv_rec[s] = g->recs[e];
            g->lv_st[s].st = E->st[ge];
            g->lv_st[s].rd = E->rd[ge];
            memcpy(g->lv_keys + (size_t)s * g->kcap, g->keys + (size_t)e * g->kcap, (size_t)g->kcap * 4u);
            g->lv_target[s] = E->target[ge];
            g->lv_frame[s] = E->ep_frame[ge];
            g->lv_deaths[s] = (int32_t)(cl >> 32);
        }
        g->lv_claim[s] = ~0ull;
    }
}

int rlenv_step(void* h, void* stream) {
    (void)stream;
    Env* E = (Env*)h;
#pragma omp parallel for schedule(dynamic, 1)
    for (int k = 0; k < E->total; ++k) {
        int e;
        Game* g = game_of(E, k, &e);
        env_step_one(E, g, e);
    }
    /* level-start saves after every env's finish; restarts read the saves only in reset_state, so doing them after
     * the whole step equals the GPU's order (rlenv_core.cuh:343-387, rl/csrc/rlenv_cpu.cpp:108-117) */
    for (int i = 0; i < E->ngames; ++i) level_saves(E, &E->games[i]);
    return 0;
}

/* One decision of envs [start, start + count) of game gi, their pictures into obs / emph (whole-batch buffers; these
 * envs write only their own rows): the GPU extras rlenv_step_game / rlenv_step_range of rl/csrc/rlenv.cu:247-268,
 * for the checker. */
int rlenv_step_range(void* h, int gi, int start, int count, uint8_t* obs, uint8_t* emph, void* stream) {
    (void)stream;
    Env* E = (Env*)h;
    if (gi < 0 || gi >= E->ngames) {
        snprintf(g_err, sizeof(g_err), "step_range: bad game");
        return 1;
    }
    Game* g = &E->games[gi];
    if (start < 0 || count <= 0 || start + count > g->n) {
        snprintf(g_err, sizeof(g_err), "step_range: bad range");
        return 1;
    }
    uint8_t *obs0 = E->obs, *emph0 = E->emph;
    E->obs = obs;
    E->emph = emph;
#pragma omp parallel for schedule(dynamic, 1)
    for (int e = start; e < start + count; ++e) env_step_one(E, g, e);
    level_saves(E, g);
    E->obs = obs0;
    E->emph = emph0;
    return 0;
}

int rlenv_step_game(void* h, int gi, uint8_t* obs, uint8_t* emph, void* stream) {
    Env* E = (Env*)h;
    if (gi < 0 || gi >= E->ngames) {
        snprintf(g_err, sizeof(g_err), "step_game: bad game");
        return 1;
    }
    return rlenv_step_range(h, gi, 0, E->games[gi].n, obs, emph, stream);
}

/* ---------------------------------------------------------------------------- level starts / places
 * rl/csrc/rlenv_api.h:22-39, rl/csrc/rlenv_build.hpp:210-251, rl/csrc/rlenv_cpu.cpp:119-170. */
int rlenv_enable_places(void* h, int cap, int levels) {
    Env* E = (Env*)h;
    if (E->lv_cap != 0 || cap <= 0 || levels <= 0 || levels > cap) {
        snprintf(g_err, sizeof(g_err), "level starts: enable once, 0 < levels <= cap");
        return 1;
    }
    for (int i = 0; i < E->ngames; ++i) {
        Game* g = &E->games[i];
        g->lv_cap = cap;
        g->lv_levels = levels;
        g->lv_rec = (NesRec*)xcalloc((size_t)cap, sizeof(NesRec));
        g->lv_st = (Rl10Saved*)xcalloc((size_t)cap, sizeof(Rl10Saved));
        g->lv_keys = (uint32_t*)xcalloc((size_t)cap * g->kcap + 1u, 4);
        g->lv_target = (uint64_t*)xcalloc((size_t)cap, 8);
        g->lv_frame = (uint32_t*)xcalloc((size_t)cap, 4);
        g->lv_deaths = (int32_t*)xcalloc((size_t)cap, 4);
        g->lv_claim = (uint64_t*)xcalloc((size_t)cap, 8);
        g->lv_cdf = (uint32_t*)xcalloc((size_t)cap, 4);
        for (int s = 0; s < cap; ++s) {
            g->lv_deaths[s] = -1;
            g->lv_claim[s] = ~0ull;
        }
    }
    E->ep_start = (int32_t*)xcalloc((size_t)E->total, 4);
    for (int k = 0; k < E->total; ++k) E->ep_start[k] = -1;
    E->lv_cap = cap;
    return 0;
}
int rlenv_enable_level_starts(void* h, int cap) { return rlenv_enable_places(h, cap, cap); }
void rlenv_set_level_plan(void* h, int gi, double p, const uint32_t* cdf) {
    Game* g = &((Env*)h)->games[gi];
    if (g->lv_cap == 0) return;
    g->lv_thresh = (uint32_t)(p <= 0.0 ? 0.0 : p >= 1.0 ? 4294967295.0 : p * 4294967296.0);
    g->lv_weighted = cdf != NULL;
    if (cdf) memcpy(g->lv_cdf, cdf, (size_t)g->lv_cap * 4);
}
void rlenv_bind_start(void* h, int32_t* out) { ((Env*)h)->start_out = out; }
void rlenv_bind_level(void* h, int32_t* out) { ((Env*)h)->level_out = out; }
void rlenv_bind_progress(void* h, float* out) { ((Env*)h)->progress_out = out; }
int rlenv_level_deaths(void* h, int gi, int32_t* out, void* stream) {
    (void)stream;
    const Game* g = &((Env*)h)->games[gi];
    if (g->lv_cap) memcpy(out, g->lv_deaths, (size_t)g->lv_cap * 4);
    return 0;
}
/* env_idx[j] -> slot_idx[j] (skipped where the slot is a level slot or out of range); host arrays here */
int rlenv_place_save(void* h, int gi, const int32_t* env_idx, const int32_t* slot_idx, int count, void* stream) {
    (void)stream;
    Env* E = (Env*)h;
    Game* g = &E->games[gi];
    for (int j = 0; j < count && g->lv_cap > 0; ++j) {
        const int s = slot_idx[j], e = env_idx[j];
        if (s < g->lv_levels || s >= g->lv_cap || e < 0 || e >= g->n) continue;
        const int ge = g->offset + e;
        g->lv_rec[s] = g->recs[e];
        g->lv_st[s].st = E->st[ge];
        g->lv_st[s].st.idle_frames = 0;   /* the no-progress clock restarts at a place (rlenv_core.cuh:366-375) */
        g->lv_st[s].rd = E->rd[ge];
        memcpy(g->lv_keys + (size_t)s * g->kcap, g->keys + (size_t)e * g->kcap, (size_t)g->kcap * 4u);
        g->lv_target[s] = E->target[ge];
        g->lv_frame[s] = E->ep_frame[ge];
        g->lv_deaths[s] = 0;
    }
    return 0;
}
int rlenv_place_copy(void* h, int gi, const int32_t* src, const int32_t* dst, int count, void* stream) {
    (void)stream;
    Game* g = &((Env*)h)->games[gi];
    for (int j = 0; j < count; ++j) {
        if (src[j] < 0 || dst[j] < 0 || src[j] >= g->lv_cap || dst[j] >= g->lv_cap) {
            snprintf(g_err, sizeof(g_err), "place_copy: bad slot");
            return 1;
        }
        const int a = src[j], b = dst[j];
        g->lv_rec[b] = g->lv_rec[a];
        g->lv_st[b] = g->lv_st[a];
        memmove(g->lv_keys + (size_t)b * g->kcap, g->lv_keys + (size_t)a * g->kcap, (size_t)g->kcap * 4u);
        g->lv_target[b] = g->lv_target[a];
        g->lv_frame[b] = g->lv_frame[a];
        g->lv_deaths[b] = g->lv_deaths[a];
    }
    return 0;
}
/* stride of one saved console, key words per env (the game's key set), sizeof(Rl10State), cap, levels */
void rlenv_level_layout(void* h, int gi, uint32_t* out) {
    const Game* g = &((Env*)h)->games[gi];
    out[0] = (uint32_t)sizeof(NesRec);
    out[1] = g->kcap;
    out[2] = (uint32_t)sizeof(Rl10Saved);   /* tracker + reader per slot */
    out[3] = (uint32_t)g->lv_cap;
    out[4] = (uint32_t)g->lv_levels;
}

/* Resume blob: per game every console record (n + 1, snapshot slot included), then the per-env arrays in
 * the reference's order (rl/csrc/rlenv_build.hpp:253-268). */
typedef void (*visit_fn)(void* p, size_t bytes, void* ctx);
static void for_each_state(Env* E, visit_fn f, void* ctx) {
    for (int i = 0; i < E->ngames; ++i) {
        f(E->games[i].recs, sizeof(NesRec) * ((size_t)E->games[i].n + 1), ctx);
        f(E->games[i].keys, (size_t)E->games[i].n * E->games[i].kcap * 4u, ctx);
    }
    const size_t N = (size_t)E->total;
    f(E->st, N * sizeof(Rl10State), ctx);
    f(E->rd, N * sizeof(Rl10Reader), ctx);
    f(E->drop, N * sizeof(Dropout), ctx);
    f(E->target, N * 8, ctx); f(E->ep_frame, N * 4, ctx); f(E->prev_applied, N * 2, ctx);
    f(E->sticky_seed, N * 8, ctx); f(E->sticky_ctr, N * 8, ctx); f(E->episode, N * 4, ctx);
    f(E->ep_ret, N * 4, ctx); f(E->ep_len, N * 4, ctx); f(E->ep_maxlvl, N * 4, ctx);
    f(E->ep_idle, N * 4, ctx); f(E->fault, N * 4, ctx);
    /* level starts last, so a state saved without them is a prefix (rl/csrc/rlenv_build.hpp:269-279) */
    if (E->lv_cap > 0) {
        f(E->ep_start, N * 4, ctx);
        for (int i = 0; i < E->ngames; ++i) {
            Game* g = &E->games[i];
            const size_t L = (size_t)g->lv_cap;
            f(g->lv_rec, L * sizeof(NesRec), ctx);
            f(g->lv_st, L * sizeof(Rl10Saved), ctx);
            f(g->lv_keys, L * g->kcap * 4u, ctx);
            f(g->lv_target, L * 8, ctx); f(g->lv_frame, L * 4, ctx); f(g->lv_deaths, L * 4, ctx);
        }
    }
}
static void v_count(void* p, size_t b, void* ctx) { (void)p; *(size_t*)ctx += b; }
static void v_save(void* p, size_t b, void* ctx) { uint8_t** o = (uint8_t**)ctx; memcpy(*o, p, b); *o += b; }
static void v_load(void* p, size_t b, void* ctx) { const uint8_t** i = (const uint8_t**)ctx; memcpy(p, *i, b); *i += b; }

size_t rlenv_state_bytes(void* h) {
    size_t n = 0;
    for_each_state((Env*)h, v_count, &n);
    return n;
}
int rlenv_save(void* h, uint8_t* out, void* stream) {
    (void)stream;
    for_each_state((Env*)h, v_save, &out);
    return 0;
}
int rlenv_load(void* h, const uint8_t* in, void* stream) {
    (void)stream;
    for_each_state((Env*)h, v_load, &in);
    return 0;
}
int rlenv_read_consoles(void* h, int gi, int first, int count, uint8_t* out, void* stream) {
    (void)stream;
    Env* E = (Env*)h;
    if (gi < 0 || gi >= E->ngames || first < 0 || count < 0 || first + count > E->games[gi].n + 1) {
        snprintf(g_err, sizeof(g_err), "read_consoles: bad range");
        return 1;
    }
    memcpy(out, &E->games[gi].recs[first], sizeof(NesRec) * (size_t)count);
    return 0;
}
const char* rlenv_error(void) { return g_err; }
void rlenv_destroy(void* h) { env_free((Env*)h); }

/* ---------------------------------------------------------------------------------- codecs / hooks */

int rl_pack6(const void* src, void* dst, size_t pixels, void* stream) {
    (void)stream;
    if (pixels % 4) {
        snprintf(g_err, sizeof(g_err), "pack6: pixel count must be divisible by four");
        return 1;
    }
    const uint8_t* s = (const uint8_t*)src;
    uint8_t* d = (uint8_t*)dst;
    for (size_t i = 0; i < pixels / 4; ++i) {
        const uint32_t v = s[4 * i] | ((uint32_t)s[4 * i + 1] << 6) | ((uint32_t)s[4 * i + 2] << 12) |
                           ((uint32_t)s[4 * i + 3] << 18);
        d[3 * i] = (uint8_t)v;
        d[3 * i + 1] = (uint8_t)(v >> 8);
        d[3 * i + 2] = (uint8_t)(v >> 16);
    }
    return 0;
}
int rl_unpack6(const void* src, void* dst, size_t pixels, void* stream) {
    (void)stream;
    if (pixels % 4) {
        snprintf(g_err, sizeof(g_err), "unpack6: pixel count must be divisible by four");
        return 1;
    }
    const uint8_t* s = (const uint8_t*)src;
    uint8_t* d = (uint8_t*)dst;
    for (size_t i = 0; i < pixels / 4; ++i) {
        const uint32_t v = s[3 * i] | ((uint32_t)s[3 * i + 1] << 8) | ((uint32_t)s[3 * i + 2] << 16);
        d[4 * i] = v & 63u;
        d[4 * i + 1] = (v >> 6) & 63u;
        d[4 * i + 2] = (v >> 12) & 63u;
        d[4 * i + 3] = (v >> 18) & 63u;
    }
    return 0;
}

/* The standalone tracker over packed 15-byte RAM views (the oracle of rl10_smb_run). */
int rl10_smb_run(const uint8_t* ram15, int T, int N, int frames, void* state, float* reward, uint8_t* done,
                 void* stream) {
    (void)stream;
    Rl10State* st = (Rl10State*)state;
#pragma omp parallel for schedule(static)
    for (int e = 0; e < N; ++e)
        for (int t = 0; t < T; ++t) {
            const Rl10Update u = rl10_update(ram15 + ((size_t)t * N + e) * 16u, frames, &st[e]);
            reward[(size_t)t * N + e] = (float)u.reward;
            done[(size_t)t * N + e] = (uint8_t)u.done;
        }
    return 0;
}

/* The tracker of any game over T steps of N envs (include/rlenv_api.h rl10_run), host buffers. */
int rl10_run(int game, const uint8_t* ram, int T, int N, const int32_t* frames, void* state, void* reader,
             uint32_t* keys, double* reward, uint8_t* done, uint32_t* events, int32_t* event_level, int32_t* deaths,
             uint8_t* end_reason, void* stream) {
    (void)stream;
    const uint32_t cap = game >= 0 && game < RL10_NUM_GAMES ? rl10_keyset_capacity(game) : 0u;
    if (game < 0 || game >= RL10_NUM_GAMES || T < 0 || N < 0 ||
        (N > 0 && T > 0 && (!ram || !frames || !state || !reader || (cap > 0 && !keys)))) {
        snprintf(g_err, sizeof(g_err), "rl10_run: bad game id, size or buffer");
        return 1;
    }
    Rl10State* st = (Rl10State*)state;
    Rl10Reader* rd = (Rl10Reader*)reader;
#pragma omp parallel for schedule(static)
    for (int e = 0; e < N; ++e)
        for (int t = 0; t < T; ++t) {
            const size_t i = (size_t)t * N + e;
            const Rl10Update u = rl10_update_game(game, ram + i * 2048u, frames[i], &st[e], &rd[e],
                                                  keys ? keys + (size_t)e * cap : NULL, cap);
            if (reward) reward[i] = u.reward;
            if (done) done[i] = (uint8_t)u.done;
            if (events) events[i] = u.events;
            if (event_level) event_level[i] = u.event_level;
            if (deaths) deaths[i] = st[e].deaths;
            if (end_reason) end_reason[i] = st[e].end_reason;
        }
    return 0;
}

/* Test hooks with the signatures of the reference's rl/csrc/host_api.cpp:13-66. */
int orc_rl10_replay(int game, const uint8_t* ram, int n, const int* frames, double* reward, uint8_t* done,
                    uint32_t* events, int* event_level, int* deaths, uint8_t* end_reason) {
    if (game < 0 || game >= RL10_NUM_GAMES) return -1;
    Rl10State e;
    Rl10Reader rd;
    rl10_reset(&e);
    memset(&rd, 0, sizeof(rd));
    const uint32_t cap = rl10_keyset_capacity(game);
    uint32_t* keys = (uint32_t*)xcalloc(cap + 1u, 4);
    for (int i = 0; i < n; ++i) {
        const Rl10Update u = rl10_update_game(game, ram + (size_t)i * 2048u, frames[i], &e, &rd, keys, cap);
        reward[i] = u.reward;
        done[i] = (uint8_t)u.done;
        events[i] = u.events;
        event_level[i] = u.event_level;
        deaths[i] = e.deaths;
        end_reason[i] = e.end_reason;
    }
    free(keys);
    return e.overflow ? 1 : 0;
}
void orc_pad_table(uint8_t* out) {
    for (int id = 0; id < RLC_MOVES; ++id)
        for (int f = 0; f < 2; ++f) out[2 * id + f] = pad_byte(move_unpack(id), (uint64_t)f);
}
void orc_legal_table(int start_ok, int select_ok, uint8_t* out, int32_t* rest) {
    for (int d = -1; d < RLE_DROP_INPUTS; ++d) {
        const Masks k = legal(d, start_ok != 0, select_ok != 0);
        for (int id = 0; id < RLC_MOVES; ++id) {
            const Move m = move_unpack(id);
            const int ok = ((k.dpad >> m.dpad) & 1) && ((k.a >> m.a) & 1) && ((k.b >> m.b) & 1) &&
                           ((k.start >> m.start) & 1) && ((k.select >> m.select) & 1);
            out[(d + 1) * RLC_MOVES + id] = (uint8_t)ok;
            rest[(d + 1) * RLC_MOVES + id] = move_pack(restrict_move(m, d, start_ok != 0, select_ok != 0));
        }
    }
}
void orc_schedule(uint64_t seed, int enabled, int n, int8_t* dropped, uint8_t* timelines, uint32_t gap_p32) {
    Dropout s;
    dropout_reset(&s, seed, enabled != 0, gap_p32);
    for (int t = 0; t < n; ++t) {
        dropped[t] = (int8_t)dropped_now(&s);
        if (timelines) timeline(&s, timelines + (size_t)t * RLE_TIMELINE_BYTES);
        dropout_advance(&s, enabled != 0, gap_p32);
    }
}
uint64_t orc_episode_seed(uint64_t run_seed, uint32_t env, uint64_t episode) {
    return episode_seed(run_seed, env, episode);
}
int orc_num_threads(void) { return omp_get_max_threads(); }

/* One tracker update from given signals and game constants {progress_unit, score_unit, stall_frames (< 0 none),
 * idle_per_frame}: the closed-form tracker tests drive this. out: reward, done, events, event_level, parts[7]. */
void orc_rl10_step(void* state, const void* signals, int frames, const double* consts, int death_from_lives,
                   double* out) {
    const Rl10Consts G = {consts[0], consts[1], consts[2], consts[3], death_from_lives};
    const Rl10Update u = rl10_update_sig((const Rl10Signals*)signals, frames, (Rl10State*)state, &G);
    out[0] = u.reward;
    out[1] = u.done;
    out[2] = u.events;
    out[3] = u.event_level;
    for (int k = 0; k < RLE_PARTS; ++k) out[4 + k] = u.part[k];
}
void orc_smb_observe(const uint8_t* ram, void* signals_out) {
    uint8_t b15[15];
    gather15(ram, b15);
    *(Rl10Signals*)signals_out = observe_smb(b15);
}
/* OpenMP threads of the oracle's parallel loops (the CPU baseline times 1 and all host threads). */
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
/* The oracle has no device work to time: the per-kernel clock reads zero launches. */
void rlenv_set_kernel_timing(void* h, int on) { (void)h; (void)on; }
int rlenv_kernel_times(void* h, double* ms, int64_t* count, int n) {
    (void)h;
    for (int i = 0; i < n; ++i) { ms[i] = 0.0; count[i] = 0; }
    return 0;
}
/* The oracle runs no translated kernels: nothing to wait for, no translation per game. */
int rlenv_jit_wait(void* h) { (void)h; return 0; }
int rlenv_jit_status(void* h, int gi, int32_t* out) {
    (void)h; (void)gi;
    out[0] = 0; out[1] = 0; out[2] = 0; out[3] = -1; out[4] = 0; out[5] = -1;
    return 0;
}
