// The reward10 SMB tracker on its own (rl10_smb_run), in three passes over T x N env-steps.
//
// RewardTracker.update (rl/csrc/reward10.cuh:546-632, env_dev.h ev::update) carries a small state from step to step;
// one env's steps are a chain. Run as one env per lane that chain is all there is to do, and with 8192 envs (128 waves
// for 1024 SIMDs) nothing hides its latency: each instruction of a step issues once every 4 cycles. So the chain is cut
// down to the state and nothing else:
//
// 1. k_smb_signals, all env-steps in parallel: the SMB signals of step t (rl/csrc/reward10.cuh:143-158) and of step
//    t - 1 (or the tracker's saved ones for the first step), and everything that depends only on them - the death,
//    the capped score reward, the rollback and idle conditions - into a 16-byte SmbStep per env-step.
// 2. k_smb_chain, one env per lane, its T steps in order: the tracker state alone (best level, best progress, score
//    budget, deaths, idle frames, the end), without branches, with sentinels for the "not seen yet" flags. It writes
//    over each SmbStep what the step's reward needs of the state (SmbDec: the step's flags as the tracker saw them,
//    and whether it entered a level, gained progress, skipped a level, was at the best level, stalled, was done
//    after it, scored; the score term; the best progress before a gain) and leaves the tracker's state, its end
//    reason worked out once from the flags of the step that ended the episode. About 80 instructions a step.
// 3. k_smb_reward, all env-steps in parallel: the reward, summed in update's order from those terms (so the same
//    doubles are added in the same order: bit-exact), and the done flag.
#pragma once
#include "env_dev.h"

namespace ev {

struct SmbStep {
    double score_r;     // min(kScoreCap, kWScore * (score - previous score) / score_unit), with ST_SCORE
    int32_t progress;   // the signed page * 256 + x (an integer-valued double in the signals)
    int16_t level;
    uint16_t flags;
};
enum : uint32_t {
    ST_IN_PLAY = 1, ST_VALID = 2, ST_WON = 4, ST_OVER = 8, ST_DEATH = 16, ST_SCORE = 32, ST_ROLLBACK = 64,
    ST_IDLE = 128, ST_HAD = 256
};
struct SmbDec {
    double score;         // the score term (min of the capped score reward and the budget left), with DC_SCORE
    int32_t best_before;  // the best progress before a gain, with DC_GAIN
    int16_t progress;
    uint16_t flags;       // the step's ST_ flags as the tracker saw them (none once it is done), then DC_ bits
};
enum : uint32_t {
    DC_LEVEL = 1u << 9, DC_GAIN = 1u << 10, DC_SKIP = 1u << 11, DC_AT_BEST = 1u << 12, DC_STALL = 1u << 13,
    DC_DONE = 1u << 14, DC_SCORE = 1u << 15
};
static_assert(sizeof(SmbStep) == 16 && sizeof(SmbDec) == 16, "16-byte records, one overwritten by the other");

// Step 1 for one env-step: signals s, the previous step's p (had: there was one).
__device__ __forceinline__ SmbStep smb_step_record(const Rl10Signals& s, const Rl10Signals& p, bool had,
                                                   const Rl10Game& G) {
    uint32_t f = had ? ST_HAD : 0u;
    if (s.in_play) f |= ST_IN_PLAY;
    if (s.progress_valid) f |= ST_VALID;
    if (s.won) f |= ST_WON;
    if (s.game_over) f |= ST_OVER;
    // update's death, before its in-play test (the rollback condition uses it as is)
    const bool death = had && (G.death_from_lives ? s.has_lives && p.has_lives && s.lives < p.lives : s.dying && !p.dying);
    if (death && (s.in_play || p.in_play)) f |= ST_DEATH;
    double sr = 0.0;
    if (had && s.in_play && p.in_play && s.has_score && p.has_score && s.score > p.score) {
        sr = kWScore * (double)(s.score - p.score) / G.score_unit;
        if (kScoreCap < sr) sr = kScoreCap;
        f |= ST_SCORE;
    }
    if (had && !death && !s.dying && !p.dying && !s.won && !s.game_over && s.in_play && p.in_play && s.progress_valid &&
        p.progress_valid && s.level == p.level && p.progress - s.progress >= kRollbackDrop * G.progress_unit)
        f |= ST_ROLLBACK;
    if (had && s.in_play && p.in_play && s.progress_valid && p.progress_valid && s.progress <= p.progress) f |= ST_IDLE;
    return SmbStep{sr, (int32_t)s.progress, (int16_t)s.level, (uint16_t)f};
}

// The tracker state of step 2 in registers: no best level = -1, no best progress = kNoBest (below every progress, so
// that "progress > best" also covers the first setting). update leaves best_progress as it was when a new level
// clears has_best_progress, so the value last assigned is kept apart (last_progress, kNoBest: none in this run) for
// the state written back.
struct SmbChain {
    uint32_t done, end_flags;
    int32_t best_level, best_progress, last_progress, deaths;
    int64_t idle;
    double score_used;
};
constexpr int32_t kNoBest = (int32_t)0x80000000u;

// One step of update's state logic (the damage term is absent: SMB has no health). stall: the stall limit in frames
// (an integer-valued double in the game constants, so (double)idle >= limit is idle >= stall), -1 for none.
__device__ __forceinline__ SmbDec smb_chain_step(const SmbStep& q, int frames, SmbChain& s, int64_t stall) {
    const uint32_t alive = s.done ^ 1u;
    const uint32_t f = q.flags & (0u - alive);                // a finished tracker sees no flag
    const int32_t level = q.level, progress = q.progress;
    const bool ip = (f & ST_IN_PLAY) != 0;
    const int32_t bl = s.best_level;
    const bool have = bl >= 0;
    const bool skip = ip && have && level > bl + 1;
    const bool up = ip && have && level == bl + 1;
    const bool reset = ip && (!have || level == bl + 1);
    s.best_level = reset ? level : bl;
    const int32_t bp = reset ? kNoBest : s.best_progress;
    s.score_used = reset ? 0.0 : s.score_used;
    const bool at_best = level == s.best_level;
    const bool better = ip && at_best && (f & ST_VALID) && progress > bp;   // a first setting or a gain
    const bool gain = better && bp != kNoBest;
    s.best_progress = better ? progress : bp;
    s.last_progress = better ? progress : s.last_progress;
    const uint32_t death = (f >> 4) & 1u;       // ST_DEATH
    s.deaths += (int32_t)death;
    const bool fresh = up || gain || death;
    const double sr = __builtin_fmin(kScoreBudget - s.score_used, q.score_r);   // (both finite)
    const bool score = (f & ST_SCORE) && sr > 0;
    s.score_used = score ? s.score_used + sr : s.score_used;
    const int64_t idle = (fresh || !(f & ST_HAD)) ? 0 : s.idle + frames;
    s.idle = alive ? idle : s.idle;
    const bool win = (f & ST_WON) != 0;
    const bool over = !win && (f & ST_OVER);
    const bool stall_end = alive && !win && !over && !skip && stall >= 0 && idle >= stall;
    const bool ends = skip || win || over || stall_end;   // (only while alive: f is 0 after the end)
    s.done = s.done | (ends ? 1u : 0u);
    const uint32_t o = f | (up ? DC_LEVEL : 0u) | (gain ? DC_GAIN : 0u) | (skip ? DC_SKIP : 0u) |
                       (at_best ? DC_AT_BEST : 0u) | (stall_end ? DC_STALL : 0u) | (s.done << 14) |
                       (score ? DC_SCORE : 0u);
    s.end_flags = ends ? o : s.end_flags;   // the ending step's flags: the end reason, worked out once at the end
    return SmbDec{sr, bp, (int16_t)progress, (uint16_t)o};
}

// update's end reason from the flags of the step that ended the episode: 2 won, 1 game over, 4 stalled, 3 skipped a
// level (checked in update's order).
__device__ __forceinline__ uint32_t smb_end_reason(uint32_t f) {
    return (f & ST_WON) ? 2u : (f & ST_OVER) ? 1u : (f & DC_STALL) ? 4u : 3u;
}

// Step 3 for one env-step: update's reward, its terms added in update's order.
__device__ __forceinline__ double smb_reward(const SmbDec& d, int frames, const Rl10Game& G) {
    const uint32_t f = d.flags;
    const bool death = (f & ST_DEATH) != 0, skip = (f & DC_SKIP) != 0;
    const bool fresh = (f & (DC_LEVEL | DC_GAIN)) != 0 || death;
    double r = 0.0;
    if (f & DC_LEVEL) r += kWLevel;
    if (f & DC_GAIN) r += kWProgress * ((double)d.progress - (double)d.best_before) / G.progress_unit;
    if (death) r += kWDeath;
    if (f & DC_SCORE) r += d.score;
    if ((f & ST_ROLLBACK) && !skip && (f & DC_AT_BEST)) r += kWRollback;
    if (!fresh && !skip && (f & ST_IDLE)) r += G.idle_per_frame * frames;
    if (f & ST_WON) r += kWWin;
    else if (f & DC_STALL) r += kWStall;
    return r;
}

}  // namespace ev
