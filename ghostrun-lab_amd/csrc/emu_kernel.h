// The console-frame kernel's arguments and body, shared by the library's own emulator kernel (rlenv_hip.hip k_emu_w)
// and the kernels compiled at run time from a cartridge's translated blocks (jit.h): the env's device-side arrays,
// outputs and settings, a game's console records and cartridge, and emu_body, one emulated frame of one console
// per wavefront.
#pragma once
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

#include "env_dev.h"
#include "nes_dev.h"
#include "optab.h"
#include "render_dev.h"
#include "rlenv_state.h"
#include "wave_dev.h"

namespace nd {

struct EnvArrays {
    Rl10State* st;
    Rl10Reader* rd;        // [N] reader state of the game's reader (unused by SMB)
    Dropout* drop;
    uint64_t *target, *sticky_seed, *sticky_ctr;
    uint32_t *ep_frame, *episode, *fault;
    int16_t* prev_applied;
    float* ep_ret;
    int32_t *ep_len, *ep_maxlvl, *ep_idle;
    uint8_t* resetting;
    int32_t* ep_start;     // [N] slot the episode started from, -1 = boot snapshot; nullptr without level starts
};

struct Outs {
    const int16_t* actions;
    uint8_t *obs, *emph, *done, *masks, *tl, *pads;
    float *reward, *info, *parts;
    uint32_t* events;
    uint64_t* ram_hash;
    int32_t *start_out, *level_out;   // level starts: start slot of a finished episode, level after the decision
    float* progress_out;              // within-level progress / progress unit, NaN = not valid
};

struct Settings {
    uint64_t run_seed;
    int sticky, idle_max, idle_tmpl, dropout, no_render, episode_level_end, pad_mode;
    uint32_t end_p32, gap_p32;
};

// Saved level starts and places of one game (rl/csrc/rlenv_core.cuh:60-74): slot s < levels is level s, saved on the
// tracker's level event; slots levels..cap-1 are places, saved on request. A saved console is a whole record.
struct LevelK {
    int cap, levels;                 // cap 0: off
    NesRec* rec;                     // [cap]
    Rl10Saved* st;                   // [cap] tracker + reader per slot
    uint32_t* keys;                  // [cap * kcap]
    uint64_t* target;                // [cap]
    uint32_t* frame;                 // [cap]
    int32_t* deaths;                 // [cap], -1 = nothing saved
    unsigned long long* claim;       // [cap] (deaths << 32 | env) of this decision's best arrival, ~0 = none
    uint32_t* cdf;                   // [cap] cumulative slot weights * 2^32
    uint32_t thresh;                 // P(a new episode starts from a saved slot) * 2^32
    int weighted;                    // 1: pick by cdf, 0: uniform over the saved slots
};

// What the renderer needs of one console-frame, copied out of the record by the emulator kernel at the frame's vblank
// stop: the frame log and its event count, the nametables and the OAM (CHR RAM, on carts that have it, in a parallel
// array). One bank per frame of a decision, so that frame f is drawn from its bank while the frames after it are
// emulated.
struct FrameBank {
    uint32_t log[NES_LOG_WORDS];
    uint32_t log_n, unused[3];
    uint8_t nt[NES_NT_BYTES];
    uint8_t oam[NES_OAM_BYTES];
};
static_assert(sizeof(FrameBank) % 16 == 0 && (NES_LOG_WORDS * 4) % 16 == 0, "16-byte copies");

struct GameK {
    NesRec* recs;          // n + 1 records, slot n = boot snapshot
    const NesRec* idle;    // idle templates
    // Restart templates, one per idle count k = 0..idle_tmpl: the record after a restart's 4 neutral frames from
    // the boot snapshot (k = 0) or idle template k, those frames' pictures and emphasis, and the fault code they
    // leave (0 = none). A restart from the boot snapshot copies one instead of emulating the frames.
    const NesRec* rst;
    const uint8_t* rst_obs;     // [idle_tmpl + 1][RLE_FRAMES][RLE_OBS_PIXELS]
    const uint8_t* rst_emph;    // [idle_tmpl + 1][RLE_FRAMES][RLE_OBS_H]
    const uint32_t* rst_fault;  // [idle_tmpl + 1]
    Cart cart;
    int n, offset, start_ok, select_ok, game;
    uint32_t kcap;         // key-set entries per env (rl10_keyset_capacity; 0 for most games)
    uint32_t* keys;        // [n * kcap] per-env key sets
    uint64_t tmpl_target;
    int32_t* list;         // restart list (env index within the game)
    uint32_t* list_count;
    LevelK lv;
    FrameBank* bank[RLE_FRAMES];     // [n] per frame of a decision
    uint8_t* bank_chr[RLE_FRAMES];   // [n][NES_CHRRAM_BYTES] per frame, CHR RAM carts only (else nullptr)
};

// EMU_TEMPLATE: one frame of every restart template (block k = template k, pad 0, target boot_target + k frames,
// fault word boot_fault[k]); the GameK's recs point at the templates.
enum : int { EMU_DECISION = 0, EMU_RESTART = 1, EMU_BOOT = 2, EMU_IDLE = 3, EMU_TEMPLATE = 4 };

struct EmuArgs {
    GameK g;
    EnvArrays e;
    Outs o;
    Settings s;
    const uint32_t* optab;
    int mode, f, use_list, e0, e1;
    uint32_t boot_pad;
    uint64_t boot_target;
    uint32_t* boot_fault;
    uint32_t budget;       // instructions per frame (NES_BUDGET; smaller only for diagnostics)
    FrameBank* bank;       // decision frames drawn from a bank: the bank this frame's render state goes to
    uint8_t* bank_chr;
    int finish;            // the decision's last frame, with kDraw: its waves also do the finish (finish_env)
};

__device__ __forceinline__ int slot_count(const GameK& g, int use_list, int e0, int e1) {
    return use_list ? (int)*g.list_count : e1 - e0;
}
__device__ __forceinline__ int slot_env(const GameK& g, int use_list, int e0, int k) {
    return use_list ? g.list[k] : e0 + k;
}

__device__ __forceinline__ uint64_t ram_hash(const uint8_t* ram) {
    const uint4* w = reinterpret_cast<const uint4*>(ram);
    uint64_t h = 0;
    for (uint32_t k = 0; k < 128u; ++k) {
        const uint4 q = w[k];
        h += ev::mix64(((uint64_t)(4u * k) << 32) | q.x);
        h += ev::mix64(((uint64_t)(4u * k + 1u) << 32) | q.y);
        h += ev::mix64(((uint64_t)(4u * k + 2u) << 32) | q.z);
        h += ev::mix64(((uint64_t)(4u * k + 3u) << 32) | q.w);
    }
    return h;
}

// RL part of the restart (rl/csrc/rlenv_core.cuh:208-263 without the record copy, which k_reset_copy does).
__device__ __forceinline__ void reset_rl(const GameK& g, const EnvArrays& e, const Settings& s, int ge) {
    const uint32_t ep = ++e.episode[ge];
    const uint64_t seed = ev::ep_seed(s.run_seed, (uint32_t)ge, ep);
    const uint64_t sseed = ev::mix64(seed ^ 0x5717C4A55EEDull);
    uint64_t ctr = 0;
    int idle = 0;
    if (s.idle_max > 0) idle = (int)ev::rnd_below(sseed, ctr, (uint32_t)(s.idle_max + 1));
    // a level start? (rl/csrc/rlenv_core.cuh:220-236: drawn only when level starts are on, after the idle count)
    int lv = -1;
    const LevelK& L = g.lv;
    if (L.cap > 0 && L.thresh != 0 && ev::rnd32(sseed, ctr) < L.thresh) {
        uint32_t saved = 0;
        for (int q = 0; q < L.cap; ++q) saved += L.deaths[q] >= 0 ? 1u : 0u;
        if (L.weighted) {
            const uint32_t u = ev::rnd32(sseed, ctr);
            for (int q = 0; q < L.cap && lv < 0; ++q)
                if (u < L.cdf[q]) lv = q;
        } else if (saved > 0) {
            uint32_t pick = ev::rnd_below(sseed, ctr, saved);
            for (int q = 0; q < L.cap && lv < 0; ++q)
                if (L.deaths[q] >= 0 && pick-- == 0) lv = q;
        }
    }
    e.sticky_seed[ge] = sseed;
    e.sticky_ctr[ge] = ctr;
    if (lv >= 0) {
        e.target[ge] = L.target[lv];
        e.ep_frame[ge] = L.frame[lv];
        e.st[ge] = L.st[lv].st;
        e.rd[ge] = L.st[lv].rd;
    } else {
        const int k = idle <= s.idle_tmpl ? idle : 0;
        e.target[ge] = g.tmpl_target + (uint64_t)k * NES_FRAME_DOTS;
        e.ep_frame[ge] = (uint32_t)k;
        e.st[ge] = Rl10State{};
        e.rd[ge] = Rl10Reader{};   // the reader and its key set restart too (rl/csrc/reward10.cuh:531-532)
    }
    if (e.ep_start) e.ep_start[ge] = lv;
    e.fault[ge] = 0;
    ev::drop_reset(e.drop[ge], seed, s.dropout != 0, s.gap_p32);   // in place: a local copy of the ring spills
    e.prev_applied[ge] = 0;
    e.ep_idle[ge] = idle;
    e.resetting[ge] = 1;
}

// ram_hash by the 64 lanes of a wave (RAM in LDS): lane j hashes words 8j..8j+7, and the sums are added across the
// lanes (the hash is a sum, so the order does not matter). Every lane returns the hash.
__device__ __forceinline__ uint64_t ram_hash_wave(const uint8_t* ram, int lane) {
    const uint4* w = reinterpret_cast<const uint4*>(ram) + 2 * lane;
    uint64_t h = 0;
    for (uint32_t i = 0; i < 2u; ++i) {
        const uint4 q = w[i];
        const uint32_t k = 8u * (uint32_t)lane + 4u * i;
        h += ev::mix64(((uint64_t)k << 32) | q.x);
        h += ev::mix64(((uint64_t)(k + 1u) << 32) | q.y);
        h += ev::mix64(((uint64_t)(k + 2u) << 32) | q.z);
        h += ev::mix64(((uint64_t)(k + 3u) << 32) | q.w);
    }
    for (int d = 32; d >= 1; d >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)h, d), hi = (uint32_t)__shfl_xor((int)(uint32_t)(h >> 32), d);
        h += (uint64_t)lo | ((uint64_t)hi << 32);
    }
    return h;
}

// The finish of one env's decision (rl/csrc/rlenv_core.cuh:267-310): the tracker over the console's RAM as the
// decision left it, the outputs, the episode end (done, synthetic ends, level clear, fault) and the RL part of a
// restart. True when the env restarts (the caller adds it to the restart list). The RAM hash is the caller's.
template <class A>
__device__ __forceinline__ bool finish_env(const A& a, int e, int ge, const uint8_t* ram) {
    Rl10State& st = a.e.st[ge];   // in place (a copy in registers spills under the console-frame kernel's 64 VGPRs)
    const ev::Out u = ev::observe_update(a.g.game, ram, RLE_FRAMES, st, &a.e.rd[ge],
                                         a.g.keys + (size_t)e * a.g.kcap, a.g.kcap);
    const bool faulted = a.e.fault[ge] != 0;
    const bool level_clear = !u.done && !faulted && a.s.episode_level_end >= 0 && (u.events & ev::EV_LEVEL) &&
                             u.event_level == a.s.episode_level_end + 1;
    bool synthetic = false;
    if (a.s.end_p32 != 0 && !u.done && !faulted && !level_clear) {
        uint64_t ctr = (uint64_t)(uint32_t)a.e.ep_len[ge];
        const uint64_t es = ev::mix64(ev::ep_seed(a.s.run_seed, (uint32_t)ge, a.e.episode[ge]) ^ 0xE9D5EEDull);
        synthetic = ev::rnd32(es, ctr) < a.s.end_p32;
    }
    const bool done = u.done || faulted || level_clear || synthetic;
    const float r = faulted ? 0.0f : (float)u.reward;
    a.o.reward[ge] = r;
    if (a.o.parts)
        for (int q = 0; q < RLE_PARTS; ++q) a.o.parts[(size_t)ge * RLE_PARTS + q] = faulted ? 0.0f : (float)u.part[q];
    a.o.done[ge] = done ? 1 : 0;
    a.o.events[ge] = u.events;
    const float ret = a.e.ep_ret[ge] + r;
    a.e.ep_ret[ge] = ret;
    const int32_t len = a.e.ep_len[ge] + 1;
    a.e.ep_len[ge] = len;
    if (u.event_level > a.e.ep_maxlvl[ge]) a.e.ep_maxlvl[ge] = u.event_level;
    ev::drop_advance(a.e.drop[ge], a.s.dropout != 0, a.s.gap_p32);   // in place (no local copy of the ring)
    // level-start claim: the arrival with the fewest deaths, then the lowest env index (rlenv_core.cuh:288-291)
    if (a.g.lv.cap > 0 && !done && (u.events & ev::EV_LEVEL) && u.event_level >= 0 && u.event_level < a.g.lv.levels) {
        const unsigned long long dd = (unsigned long long)(uint32_t)(st.deaths < 0 ? 0 : st.deaths);
        atomicMin(&a.g.lv.claim[u.event_level], (dd << 32) | (uint32_t)e);
    }
    if (a.o.level_out) a.o.level_out[ge] = st.has_best_level ? st.best_level : -1;
    if (a.o.progress_out)
        a.o.progress_out[ge] = st.has_prev && st.prev.progress_valid ? (float)(st.prev.progress / rl10_game(a.g.game).progress_unit)
                                                                      : __builtin_nanf("");
    if (done) {
        if (a.o.start_out) a.o.start_out[ge] = a.e.ep_start ? a.e.ep_start[ge] : -1;
        float* inf = a.o.info + (size_t)ge * RLE_INFO;
        inf[0] = ret;
        inf[1] = (float)len;
        inf[2] = (float)(faulted ? RLE_END_FAULT : level_clear ? RLE_END_LEVEL_CLEAR
                                                               : synthetic ? RLE_END_SYNTHETIC : st.end_reason);
        inf[3] = (float)st.deaths;
        inf[4] = (float)a.e.ep_maxlvl[ge];
        inf[5] = st.overflow ? 1.0f : 0.0f;
        inf[6] = (float)a.e.ep_idle[ge];
        inf[7] = (float)a.e.episode[ge];
        reset_rl(a.g, a.e, a.s, ge);
        return true;
    }
    return false;
}

// Per-frame pad byte of a decision frame (rl/csrc/rlenv_core.cuh:181-191): sticky repeat, dropout, turbo phase.
template <class Args>
__device__ __forceinline__ uint32_t decision_pad(const Args& a, int ge, int f) {
    const int d = ev::dropped_now(&a.e.drop[ge]);
    uint64_t ctr = a.e.sticky_ctr[ge];
    const uint64_t seed = a.e.sticky_seed[ge];
    uint32_t pad;
    if (a.s.pad_mode) {
        uint32_t p = (uint16_t)a.o.actions[ge] & 0xFFu;
        if (a.s.sticky && ev::rnd32(seed, ctr) < RLC_STICKY_P32) p = (uint16_t)a.e.prev_applied[ge] & 0xFFu;
        pad = ev::restrict_pad(p, d);
        a.e.prev_applied[ge] = (int16_t)pad;
    } else {
        ev::Move mv = ev::unpack((uint32_t)(int32_t)a.o.actions[ge]);
        if (a.s.sticky && ev::rnd32(seed, ctr) < RLC_STICKY_P32)
            mv = ev::restrict_move(ev::unpack((uint32_t)(int32_t)a.e.prev_applied[ge]), d, a.g.start_ok != 0,
                                   a.g.select_ok != 0);
        a.e.prev_applied[ge] = (int16_t)ev::pack(mv);
        pad = ev::pad_of(mv, a.e.ep_frame[ge]);
    }
    a.e.sticky_ctr[ge] = ctr;
    a.o.pads[(size_t)ge * RLE_FRAMES + f] = (uint8_t)pad;
    return pad;
}

// The opcode descriptors in constant memory: the wave-uniform generic step reads them through the scalar cache.
static __constant__ Optab c_optab = kOptab;

// Copies n bytes (a multiple of 16, 16-byte aligned) with the 64 lanes of the wavefront.
__device__ __forceinline__ void wave_copy16(void* dst, const void* src, uint32_t n, int lane) {
    uint4* d = static_cast<uint4*>(dst);
    const uint4* s = static_cast<const uint4*>(src);
    for (uint32_t i = (uint32_t)lane; i < n / 16u; i += 64u) d[i] = s[i];
}

// Per-wavefront LDS of one console: CPU RAM, nametables, OAM, palette and the console state.
struct WaveLds {
    uint8_t ram[NES_RAM_BYTES];
    uint8_t nt[NES_NT_BYTES];
    uint8_t oam[NES_OAM_BYTES];
    uint8_t pal[NES_PAL_BYTES];
    Con cs;
    uint32_t scratch[34];   // the sprite-0 check's MMC2 pages
};
static_assert(sizeof(RenderScratch) <= NES_RAM_BYTES && offsetof(WaveLds, ram) % 16 == 0,
              "the render's scratch fits over the CPU RAM");

// The kernel's arguments for what runs after the emulation, read there from the kernel-argument segment (every
// kernel that runs emu_body takes its EmuArgs as its only parameter, so they start the segment) through an address
// the compiler cannot see through. Read from the parameter, they are loaded at the kernel's start and held through
// the emulation in scalar registers that the burst loop needs (the decision's finish pushed the translated
// emulate-and-draw kernel into scratch; the frame bank's pointers cost the translated frame 1 %).
__device__ __forceinline__ const EmuArgs& late_args() {
    const EmuArgs* p = (const EmuArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *p;
}
// The check, where each kernel that runs emu_body is defined: its type is void (EmuArgs), so its one explicit argument
// is the EmuArgs at offset 0 of the kernel-argument segment that late_args reads (a second parameter, or one before
// it, would make late_args read other bytes without any error).
#define ND_EMU_KERNEL_ARGS(...)                                                             \
    static_assert(__is_same(decltype(&__VA_ARGS__), void (*)(nd::EmuArgs)),                 \
                  "a kernel that runs emu_body takes its EmuArgs as its only parameter (late_args)")

// One console per wavefront (blockDim 64): the console index comes from blockIdx only, so every emulator value is
// wave-uniform; lane 0 (every lane on MMC2) runs the 6502 on the scalar unit (SGPRs, uniform branches) with the
// console's memories in LDS, the 64 lanes copy them in and out. Eight waves per SIMD: 8192 consoles fill 256 CUs x 4
// SIMDs x 8 in one
// round (left to itself the compiler takes 71 VGPRs, 7 waves, and the eighth wave of every SIMD runs after the
// others).
// kBank: a decision frame whose picture is drawn from a frame bank (its render state is copied there at the end).
// kDraw: a decision frame whose picture the same wave draws once the frame is emulated and the console copied out
// (render_dev.h, the render's scratch laid over the CPU RAM in LDS, the nametables and OAM where the frame left them);
// for the decision's last frame (a.finish) the wave also does the env's finish first.
template <uint32_t B, bool kBank, bool kDraw = false>
__device__ __forceinline__ void emu_body(const EmuArgs& a) {
    __shared__ __align__(16) WaveLds L;
    const int count = a.mode == EMU_BOOT ? 1 : slot_count(a.g, a.use_list, a.e0, a.e1);
    const int k = (int)blockIdx.x;
    if (k >= count) return;
    const int lane = (int)threadIdx.x;
    const int e = a.mode == EMU_BOOT ? a.e0 : slot_env(a.g, a.use_list, a.e0, k);
    const int ge = a.g.offset + e;
    if (a.mode == EMU_RESTART && a.e.resetting[ge] != 1) return;   // 2: copied from a restart template
    // EMU_IDLE: a restart from a saved level start emulates all of its idle frames (pad 0) in this one launch; a
    // restart from the boot snapshot copied a template that holds them (rl/csrc/rlenv_core.cuh:312-318)
    int frames = 1;
    if (a.mode == EMU_IDLE) {
        if (a.e.resetting[ge] == 0 || a.e.ep_start == nullptr || a.e.ep_start[ge] < 0) return;
        frames = a.e.ep_idle[ge];
        if (frames <= 0) return;
    }
    NesRec* rec = &a.g.recs[e];
    wave_copy16(L.ram, rec->ram, NES_RAM_BYTES, lane);
    wave_copy16(L.nt, rec->nt, NES_NT_BYTES, lane);
    wave_copy16(L.oam, rec->oam, NES_OAM_BYTES, lane);
    wave_copy16(L.pal, rec->pal, NES_PAL_BYTES, lane);
    __syncthreads();
    // An MMC2 console is emulated on all 64 lanes, every lane doing the same (every value is wave-uniform, and every
    // store writes the same value to the same place), so that the line replays of its sprite-0 check and vblank
    // latch resolve can spread a run's pattern fetches over the lanes (replay_dev.h rs_mmc2_fetches); any other
    // console on lane 0.
    const bool wide = B != NES_BOARD_NROM && a.g.cart.board == NES_BOARD_MMC2;
    if (lane == 0 || wide) {
        uint32_t pad = 0, fault = 0;
        uint64_t target;
        if (a.mode == EMU_BOOT) {
            pad = a.boot_pad;
            target = a.boot_target;
        } else if (a.mode == EMU_TEMPLATE) {
            target = a.boot_target + (uint64_t)e * NES_FRAME_DOTS;
            fault = a.boot_fault[e];
        } else {
            if (a.mode == EMU_DECISION) pad = decision_pad(a, ge, a.f);
            target = a.e.target[ge];
            fault = a.e.fault[ge];
        }
        Con& cs = L.cs;
        con_load(cs, rec);
        const Mem m{rec, L.ram, L.nt, L.oam, L.pal, a.g.cart, L.scratch};
        for (int i = 0; i < frames; ++i) {   // a faulted console stays put; its target and frame still advance
            cs.pad = pad;
            if (fault == 0) {
                const uint32_t f = run_until_wave<B>(cs, m, c_optab.t, target, a.budget);
                if (f != 0) {
                    if (a.mode == EMU_BOOT) atomicOr(a.boot_fault, 1u);
                    else if (a.mode == EMU_TEMPLATE) a.boot_fault[e] = f;
                    else a.e.fault[ge] = f;
                    fault = f;
                }
            }
            target += NES_FRAME_DOTS;
        }
        con_store(cs, rec);
        if (a.mode != EMU_BOOT && a.mode != EMU_TEMPLATE) {
            a.e.target[ge] = target;
            a.e.ep_frame[ge] += (uint32_t)frames;
        }
    }
    __syncthreads();
    wave_copy16(rec->ram, L.ram, NES_RAM_BYTES, lane);
    wave_copy16(rec->nt, L.nt, NES_NT_BYTES, lane);
    wave_copy16(rec->oam, L.oam, NES_OAM_BYTES, lane);
    wave_copy16(rec->pal, L.pal, NES_PAL_BYTES, lane);
    if constexpr (kBank) {   // the frame's render state (the log lane 0 wrote before the sync above)
        const EmuArgs& la = late_args();
        FrameBank* b = &la.bank[e];
        wave_copy16(b->log, rec->log, NES_LOG_WORDS * 4u, lane);
        wave_copy16(b->nt, L.nt, NES_NT_BYTES, lane);
        wave_copy16(b->oam, L.oam, NES_OAM_BYTES, lane);
        if (lane == 0) b->log_n = L.cs.log_n;
        if (la.bank_chr) wave_copy16(la.bank_chr + (size_t)e * NES_CHRRAM_BYTES, rec->chr_ram, NES_CHRRAM_BYTES, lane);
    }
    if constexpr (kDraw) {
        const bool draw = a.mode == EMU_DECISION && !a.s.no_render, finish = a.mode == EMU_DECISION && a.finish;
        if (draw || finish) {
            // the frame log, CHR RAM and RAM written above are read after this sync, and the copy-out's reads of the
            // RAM are done before the scratch overwrites it
            const uint32_t log_n = uni(L.cs.log_n);
            __syncthreads();
            if (finish) {   // the decision's finish (k_finish's work), in the waves of its last frame
                const uint64_t h = a.o.ram_hash ? ram_hash_wave(L.ram, lane) : 0;
                if (lane == 0) {
                    const EmuArgs& fa = late_args();
                    if (fa.o.ram_hash) fa.o.ram_hash[ge] = h;
                    if (finish_env(fa, e, ge, rec->ram)) fa.g.list[atomicAdd(fa.g.list_count, 1u)] = e;
                }
                __syncthreads();   // (the hash has read the RAM before the scratch overwrites it)
            }
            if (draw) {
                uint8_t* obs = a.o.obs + ((size_t)ge * RLE_FRAMES + a.f) * RLE_OBS_PIXELS;
                uint8_t* emph = a.o.emph + ((size_t)ge * RLE_FRAMES + a.f) * RLE_OBS_H;
                draw_frame<false>(reinterpret_cast<RenderScratch*>(L.ram), L.nt, L.oam, rec->log, log_n, a.g.cart,
                                  rec->chr_ram, obs, emph, lane);
            }
        }
    }
}

}  // namespace nd
