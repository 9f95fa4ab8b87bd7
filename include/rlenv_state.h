/* Per-env RL state kept beside each console: the reward tracker and the button-dropout schedule. Shared
 * layout of the CPU oracle and the HIP library (it is part of the saved state blob).
 *
 * Rl10State holds what the reference's rl10::EnvState holds for the SMB reader (rl/csrc/reward10.cuh:63-103);
 * Dropout is the reference's rlc::Dropout (rl/csrc/controller.cuh:138-145).
 */
#ifndef RLENV_STATE_H
#define RLENV_STATE_H
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <stdint.h>
#endif

typedef struct Rl10Signals {      /* reward.Signals with explicit "has" flags for Python's None */
    uint8_t in_play, progress_valid, dying, has_lives, has_health, has_score, game_over, won;
    int32_t level, lives;
    double progress, health;
    int64_t score;
} Rl10Signals;                    /* 40 bytes */

typedef struct Rl10State {        /* RewardTracker */
    uint8_t has_prev, has_best_level, has_best_progress, done, end_reason, overflow, _p0, _p1;
    int32_t best_level, deaths;
    int64_t idle_frames;
    double best_progress, score_used;
    Rl10Signals prev;
} Rl10State;                      /* 80 bytes */

/* The game readers' own state (rl/csrc/reward10.cuh:87-101, the reader part of rl10::EnvState): what the Castlevania,
 * Zelda, Excitebike, Contra, Final Mission, Kage, Tecmo Bowl and Punch-Out readers carry between updates. */
typedef struct Rl10Reader {
    uint8_t has_stage, has_floor, has_base, has_key, has_cam, has_own, has_drive, has_week;
    uint8_t has_fight, has_prev_hp, _p0[6];
    int32_t stage, floor_y, base_items, base_containers;
    int32_t key_a, key_b, cam, core_max;
    int32_t own, opp, week, fight;
    int32_t damage, prev_hp;
    uint32_t cells, rooms;
    double key_d, dist, best_arc, drive_start, drive_best;
} Rl10Reader;                     /* 120 bytes */

/* One archive slot's tracker state: the tracker and its game reader, saved, restored and copied together. It is the
 * per-slot block whose size rlenv_level_layout reports (the sizeof(rl10::EnvState) of rl/csrc/rlenv_build.hpp:275),
 * so a state blob's archive tail has the reference's six parts per game. */
typedef struct Rl10Saved {
    Rl10State st;
    Rl10Reader rd;
} Rl10Saved;                      /* 200 bytes */

#define RLC_RING 64
typedef struct Dropout {
    uint64_t seed, counter;       /* the schedule's own generator */
    int32_t gap_left;             /* healthy decisions left before the next dropout */
    int32_t drop_left;            /* decisions left in the current dropout */
    int32_t drop_input;           /* input of the current dropout */
    uint32_t head;                /* decision index of ring column "now" */
    int8_t ring[RLC_RING];        /* ring[(head + j) % 64] = input off at decision head + j, -1 none */
} Dropout;                        /* 96 bytes */

#ifdef __cplusplus
static_assert(sizeof(Rl10Signals) == 40 && sizeof(Rl10State) == 80 && sizeof(Dropout) == 96 &&
              sizeof(Rl10Reader) == 120, "layout");
#else
_Static_assert(sizeof(Rl10Signals) == 40 && sizeof(Rl10State) == 80 && sizeof(Dropout) == 96 &&
               sizeof(Rl10Reader) == 120, "layout");
#endif

/* Env constants (rl/rlenv.py:34-38, rl/csrc/rlenv_core.cuh:33-38, rl/csrc/controller.cuh:24-32). */
#define RLE_FRAMES 4
#define RLE_OBS_H 224
#define RLE_OBS_W 240
#define RLE_OBS_PIXELS (RLE_OBS_H * RLE_OBS_W)
#define RLE_MASK_BYTES 19
#define RLE_TIMELINE 45
#define RLE_DROP_INPUTS 8
#define RLE_TIMELINE_BYTES (RLE_DROP_INPUTS * RLE_TIMELINE)
#define RLE_INFO 8
#define RLE_PARTS 7
#define RLE_END_FAULT 5
#define RLE_END_LEVEL_CLEAR 6
#define RLE_END_SYNTHETIC 7       /* this build's configurable Geometric episode end */
#define RLC_MOVES 324
#define RLC_GAP_P32 122713351u    /* floor(2^32 / 35) */
#define RLC_STICKY_P32 0x40000000u

#endif
