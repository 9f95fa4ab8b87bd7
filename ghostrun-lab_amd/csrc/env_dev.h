// Device side of the env around the console: controller moves and pad bytes, the counter RNG, the button-dropout
// schedule (rl/csrc/controller.cuh:41-189) and the reward10 tracker with the game readers (SMB's here, the other
// eleven shared with the CPU build in include/rl10_games.h; rl/csrc/reward10.cuh:143-524, 546-632; constants
// rl/csrc/reward10_consts.h:11-39). Integer-only where the
// reference is, double in Python's evaluation order for the reward (built with -ffp-contract=off).
#pragma once
#ifndef ND_HOST_BUILD
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <hip/hip_runtime.h>
#endif
#endif
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <stdint.h>
#endif

#include "rlenv_state.h"
#include "rl10_games.h"

namespace ev {

// ------------------------------------------------------------------------------------- controller
constexpr uint32_t B_A = 1, B_B = 2, B_SELECT = 4, B_START = 8, B_UP = 16, B_DOWN = 32, B_LEFT = 64, B_RIGHT = 128;

// d-pad choice (0 none, 1 U, 2 UR, 3 R, 4 DR, 5 D, 6 DL, 7 L, 8 UL) -> pad bits. Nibble k of the table holds choice
// k's directions as (Up, Down, Left, Right) in bits 0..3, which are the pad's bits 4..7.
__device__ __forceinline__ uint32_t dpad_bits(uint32_t d) {
    constexpr uint64_t kTable = 0x5462A8910ull;
    return d < 9u ? (uint32_t)((kTable >> (4u * d)) & 15u) << 4 : 0u;
}
__device__ __forceinline__ uint32_t dpad_from_bits(uint32_t bits) {
    uint32_t out = 0;
    for (uint32_t d = 8; d >= 1u; --d)
        if (dpad_bits(d) == bits) out = d;
    return out;
}

struct Move { uint32_t dpad, a, b, start, select; };
__device__ __forceinline__ Move unpack(uint32_t id) {
    Move m;
    m.dpad = id % 9u; id /= 9u;
    m.a = id % 3u; id /= 3u;
    m.b = id % 3u; id /= 3u;
    m.start = id % 2u; id /= 2u;
    m.select = id % 2u;
    return m;
}
__device__ __forceinline__ uint32_t pack(const Move& m) {
    return m.dpad + 9u * (m.a + 3u * (m.b + 3u * (m.start + 2u * m.select)));
}
__device__ __forceinline__ uint32_t pad_of(const Move& m, uint32_t frame) {
    const bool even = (frame & 1u) == 0;
    uint32_t p = dpad_bits(m.dpad);
    if (m.a == 1u || (m.a == 2u && even)) p |= B_A;
    if (m.b == 1u || (m.b == 2u && even)) p |= B_B;
    if (m.start) p |= B_START;
    if (m.select) p |= B_SELECT;
    return p;
}
// dropped input: 0 Up 1 Down 2 Left 3 Right 4 A-hold 5 B-hold 6 TurboA 7 TurboB
__device__ __forceinline__ Move restrict_move(Move m, int dropped, bool start_ok, bool select_ok) {
    uint32_t bits = dpad_bits(m.dpad);
    if (dropped >= 0 && dropped < 4) bits &= ~(B_UP << (uint32_t)dropped);   // Up, Down, Left, Right are bits 4..7
    m.dpad = dpad_from_bits(bits);
    if ((dropped == 4 && m.a == 1u) || (dropped == 6 && m.a == 2u)) m.a = 0;
    if ((dropped == 5 && m.b == 1u) || (dropped == 7 && m.b == 2u)) m.b = 0;
    if (!start_ok) m.start = 0;
    if (!select_ok) m.select = 0;
    return m;
}
__device__ __forceinline__ uint32_t restrict_pad(uint32_t p, int dropped) {
    if (dropped >= 0 && dropped < 4) p &= ~(B_UP << (uint32_t)dropped);
    else if (dropped == 4 || dropped == 6) p &= ~B_A;
    else if (dropped == 5 || dropped == 7) p &= ~B_B;
    return p & 0xFFu;
}

// ------------------------------------------------------------------------------------------- RNG
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint32_t rnd32(uint64_t seed, uint64_t& ctr) {
    return (uint32_t)(mix64(seed ^ mix64(ctr++)) >> 32);
}
__device__ __forceinline__ uint32_t rnd_below(uint64_t seed, uint64_t& ctr, uint32_t n) {
    return (uint32_t)(((uint64_t)rnd32(seed, ctr) * n) >> 32);
}
__device__ __forceinline__ uint64_t ep_seed(uint64_t run_seed, uint32_t env, uint64_t episode) {
    return mix64(mix64(run_seed ^ 0xD20F0D20F0ull) ^ ((uint64_t)env << 40) ^ episode);
}

// --------------------------------------------------------------------------------------- dropout
__device__ inline int32_t gap_draw(Dropout& s, uint32_t p32) {
    int32_t k = 1;
    while (rnd32(s.seed, s.counter) >= p32) ++k;
    return k;
}
__device__ inline int32_t column_next(Dropout& s, uint32_t p32) {
    if (s.drop_left > 0) {
        const int32_t out = s.drop_input;
        if (--s.drop_left == 0) s.gap_left = gap_draw(s, p32);
        return out;
    }
    if (--s.gap_left == 0) {
        s.drop_input = (int32_t)rnd_below(s.seed, s.counter, 8u);
        s.drop_left = 8 + (int32_t)rnd_below(s.seed, s.counter, 15u);
    }
    return -1;
}
__device__ inline void drop_reset(Dropout& s, uint64_t seed, bool on, uint32_t p32) {
    s.seed = seed;
    s.counter = 0;
    s.drop_left = 0;
    s.drop_input = -1;
    s.head = 0;
    s.gap_left = on ? gap_draw(s, p32) : 0x7FFFFFFF;
    for (int j = 0; j < RLC_RING; ++j) s.ring[j] = -1;
    for (int j = 0; j < RLE_TIMELINE; ++j) s.ring[j] = (int8_t)(on ? column_next(s, p32) : -1);
}
__device__ __forceinline__ int dropped_now(const Dropout* s) { return s->ring[s->head & (RLC_RING - 1)]; }
__device__ inline void drop_advance(Dropout& s, bool on, uint32_t p32) {
    s.ring[s.head & (RLC_RING - 1)] = -1;
    ++s.head;
    s.ring[(s.head + RLE_TIMELINE - 1) & (RLC_RING - 1)] = (int8_t)(on ? column_next(s, p32) : -1);
}

// ------------------------------------------------------------------------------------- reward10 tracker
constexpr double kWProgress = 0x1.0000000000000p+0, kWLevel = 0x1.0000000000000p+0;
constexpr double kWDeath = -0x1.999999999999ap-4, kWStall = -0x1.999999999999ap-4;
constexpr double kWScore = 0x1.47ae147ae147bp-6, kScoreCap = 0x1.999999999999ap-4;
constexpr double kScoreBudget = 0x1.999999999999ap-3, kWWin = 0x1.4000000000000p+2;
constexpr double kWRollback = -0x1.47ae147ae147bp-6, kRollbackDrop = 0x1.0000000000000p-2;
constexpr double kWDamage = -0x1.0000000000000p-2;
enum : uint32_t { EV_SKIP = 1, EV_LEVEL = 2, EV_DEATH = 4, EV_WON = 8, EV_GAMEOVER = 16, EV_STALL = 32, EV_ROLLBACK = 64 };

struct Out {
    double reward;
    bool done;
    uint32_t events;
    int event_level;
    double part[RLE_PARTS];
};

// b: the 15 bytes in the order 0x0E 0x6D 0x86 0xB5 0x75A 0x75C 0x75F 0x770 0x772 0x7DD..0x7E2
__device__ inline Rl10Signals smb_signals(const uint8_t* b) {
    Rl10Signals s = {};
    const int routine = b[0], page = b[1], world = b[6], mode = b[7];
    s.in_play = mode == 1 && b[8] == 3;
    s.level = world * 4 + b[5];
    s.progress = (double)(((page ^ 0x80) - 0x80) * 256 + b[2]);
    s.progress_valid = s.in_play && routine == 8;
    s.dying = mode == 1 && (routine == 6 || routine == 11 || (routine == 8 && b[3] >= 2));
    s.has_lives = 1;
    s.lives = ((int)b[4] ^ 0x80) - 0x80;
    s.has_score = 1;
    int64_t sc = 0;
    for (int i = 9; i < 15; ++i) sc = sc * 10 + b[i];
    s.score = sc * 10;
    s.game_over = mode == 3;
    s.won = mode == 2 && world == 7;
    return s;
}

// RewardTracker.update (rl/csrc/reward10.cuh:546-632) with one game's constants G (reward10_consts.h:24-37).
__device__ inline Out update(const Rl10Signals& s, int frames, Rl10State& e, const Rl10Game& G) {
    Out o = {};
    const bool had = e.has_prev != 0;
    const Rl10Signals p = e.prev;
    e.has_prev = 1;
    e.prev = s;
    o.done = true;
    if (e.done) return o;
    double r = 0.0;
    uint32_t evs = 0;
    int lvl = 0;
    bool fresh = false;
    if (s.in_play) {
        if (!e.has_best_level) {
            e.has_best_level = 1;
            e.best_level = s.level;
            e.has_best_progress = 0;
            e.score_used = 0.0;
        } else if (s.level > e.best_level + 1) {
            evs |= EV_SKIP;
            lvl = s.level;
            e.done = 1;
            e.end_reason = 3;
        } else if (s.level > e.best_level) {
            r += kWLevel;
            o.part[1] += kWLevel;
            evs |= EV_LEVEL;
            lvl = s.level;
            e.best_level = s.level;
            e.has_best_progress = 0;
            e.score_used = 0.0;
            fresh = true;
        }
        if (s.level == e.best_level && s.progress_valid) {
            if (!e.has_best_progress) {
                e.has_best_progress = 1;
                e.best_progress = s.progress;
            } else if (s.progress > e.best_progress) {
                const double gain = kWProgress * (s.progress - e.best_progress) / G.progress_unit;
                r += gain;
                o.part[0] += gain;
                e.best_progress = s.progress;
                fresh = true;
            }
        }
    }
    bool death = false;
    if (had) {
        death = G.death_from_lives ? s.has_lives && p.has_lives && s.lives < p.lives : s.dying && !p.dying;
        if (death && (s.in_play || p.in_play)) {
            r += kWDeath;
            o.part[2] += kWDeath;
            e.deaths += 1;
            evs |= EV_DEATH;
            fresh = true;
        }
        if (s.in_play && p.in_play && s.has_health && p.has_health && s.health < p.health) {
            const double rd = kWDamage * (p.health - s.health);
            r += rd;
            o.part[3] += rd;
        }
        if (s.in_play && p.in_play && s.has_score && p.has_score && s.score > p.score) {
            double sr = kWScore * (double)(s.score - p.score) / G.score_unit;
            if (kScoreCap < sr) sr = kScoreCap;
            const double left = kScoreBudget - e.score_used;
            if (left < sr) sr = left;
            if (sr > 0) {
                r += sr;
                o.part[4] += sr;
                e.score_used += sr;
            }
        }
    }
    if (had && !e.done && !death && !s.dying && !p.dying && !s.won && !s.game_over && s.in_play && p.in_play &&
        s.progress_valid && p.progress_valid && s.level == p.level && s.level == e.best_level &&
        p.progress - s.progress >= kRollbackDrop * G.progress_unit) {
        r += kWRollback;
        o.part[6] += kWRollback;
        evs |= EV_ROLLBACK;
    }
    if (!fresh && !e.done && had && s.in_play && p.in_play && s.progress_valid && p.progress_valid &&
        s.progress <= p.progress) {
        const double idle = G.idle_per_frame * frames;
        r += idle;
        o.part[6] += idle;
    }
    e.idle_frames = (fresh || !had) ? 0 : e.idle_frames + frames;
    if (s.won) {
        r += kWWin;
        o.part[5] += kWWin;
        evs |= EV_WON;
        e.done = 1;
        e.end_reason = 2;
    } else if (s.game_over) {
        evs |= EV_GAMEOVER;
        e.done = 1;
        e.end_reason = 1;
    } else if (!e.done && G.stall_frames >= 0.0 && (double)e.idle_frames >= G.stall_frames) {
        r += kWStall;
        o.part[6] += kWStall;
        evs |= EV_STALL;
        e.done = 1;
        e.end_reason = 4;
    }
    o.reward = r;
    o.done = e.done != 0;
    o.events = evs;
    o.event_level = lvl;
    return o;
}

__device__ __forceinline__ void smb_gather(const uint8_t* ram, uint8_t* b) {
    b[0] = ram[0x0E]; b[1] = ram[0x6D]; b[2] = ram[0x86]; b[3] = ram[0xB5];
    b[4] = ram[0x75A]; b[5] = ram[0x75C]; b[6] = ram[0x75F]; b[7] = ram[0x770]; b[8] = ram[0x772];
    for (int i = 0; i < 6; ++i) b[9 + i] = ram[0x7DD + i];
}

// The game's reader on one env's 2 KB RAM (rl/csrc/reward10.cuh:546-548), then the tracker. rd and keys (cap
// entries) are the env's reader state and key set; SMB keeps neither. The game id is uniform over a launch.
__device__ inline Out observe_update(int game, const uint8_t* ram, int frames, Rl10State& st, Rl10Reader* rd,
                                     uint32_t* keys, uint32_t cap) {
    Rl10Signals sig;
    if (game == RL10_SMB) {
        uint8_t b15[15];
        smb_gather(ram, b15);
        sig = smb_signals(b15);
    } else {
        sig = rl10_observe(game, ram, &st, rd, keys, cap);   // the reader in place
    }
    return update(sig, frames, st, rl10_game(game));
}

}  // namespace ev
