// HIP build of the batched NES environment step for MI355X (gfx950), behind the C ABI of include/rlenv_api.h.
//
// One decision of one game is this launch sequence on the caller's stream (the reference's phase order,
// rl/csrc/rlenv_core.cuh:389-414 and rl/csrc/rlenv.cu:145-170):
//   4 x k_emu_w: one emulated frame of every console and its picture into obs slot f - drawn by the same waves
//     (emu_kernel.h, kDraw), or for frames 0-1 of a one-game env of one round of waves by k_render on a render
//     stream from a frame bank (kBank); the last frame's waves also do the finish (finish_env: reward10 update,
//     outputs, dropout advance; finished episodes reset their RL state and join the restart list)
//   k_reset_copy: boot snapshot (or idle template) -> console record, one workgroup per listed console
//   4 x (k_emu_w, k_render) over the restart list only (neutral frames of the new episode)
//   k_reset_finish: first tracker update of new episodes; masks and dropout timeline of every env
//
// k_emu_w (the default) gives each console a whole wavefront: the console index comes from blockIdx, so its state
// is wave-uniform and the 6502 runs on the scalar unit (uniform branches, SGPRs) with a per-opcode fast path
// (wave_dev.h); the console's RAM, nametables, OAM, palette and cold state live in LDS for the launch. 8192 consoles
// are 8192 waves, 8 per SIMD.
// k_render draws one console-frame per wavefront: the log is replayed through FCEUmm's line renderer (replay_dev.h),
// its scalar walk wave-uniform, each run of tile slots fetched and shifted out by the lanes into a line buffer in LDS,
// sprites selected with one ballot per line, and each output row is one coalesced 240-byte store.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <ctime>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "emu_kernel.h"
#include "env_dev.h"
#include "jit.h"
#include "jit_check.h"
#include "smb_tracker.h"
#include "nes_dev.h"
#include "optab.h"
#include "render_dev.h"
#include "rlenv_api.h"
#include "rlenv_state.h"
#include "wave_dev.h"

using namespace nd;

namespace {

thread_local std::string g_error;

// ============================================================================================ kernels
// (the console-frame kernel's arguments and body: emu_kernel.h, shared with the translated kernels of jit.h)
template <uint32_t B, bool kBank, bool kDraw>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_emu_w(EmuArgs a) {
    emu_body<B, kBank, kDraw>(a);
}
ND_EMU_KERNEL_ARGS(k_emu_w<NES_BOARD_NROM, false, false>);

// Power-on of one console record.
__global__ void k_power_on(NesRec* rec, Cart cart) {
    if (threadIdx.x == 0 && blockIdx.x == 0) power_on(rec, cart);
}

// ----------------------------------------------------------------------------------------- render
struct RenderArgs {
    GameK g;
    EnvArrays e;
    Outs o;
    Settings s;
    int f, use_list, restart_pass, e0, e1;
    const FrameBank* bank;       // draw from this bank (nullptr: from the record)
    const uint8_t* bank_chr;
};

// One console-frame per wavefront (blockDim 64): the picture of the frame the console has logged, drawn from its
// nametables and OAM as of the frame's vblank stop (render_dev.h draw_frame).
template <bool kBank>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_render(RenderArgs a) {
    __shared__ __align__(16) struct {
        uint8_t nt[NES_NT_BYTES];
        uint8_t oam[NES_OAM_BYTES];
        RenderScratch r;
    } L;
    const int count = slot_count(a.g, a.use_list, a.e0, a.e1);
    const int k = (int)blockIdx.x;
    if (k >= count) return;
    const int e = slot_env(a.g, a.use_list, a.e0, k);
    const int ge = a.g.offset + e;
    if (a.restart_pass && a.e.resetting[ge] != 1) return;   // 2: copied from a restart template
    if (a.s.no_render) return;
    const int lane = (int)threadIdx.x;
    const NesRec* rec = &a.g.recs[e];
    const FrameBank* bk = kBank ? &a.bank[e] : nullptr;
    const uint32_t* log = kBank ? bk->log : rec->log;
    const uint32_t log_n = kBank ? bk->log_n : rec->log_n;
    const uint8_t* chr_ram = kBank && a.bank_chr ? a.bank_chr + (size_t)e * NES_CHRRAM_BYTES : rec->chr_ram;
    wave_copy16(L.nt, kBank ? bk->nt : rec->nt, NES_NT_BYTES, lane);
    wave_copy16(L.oam, kBank ? bk->oam : rec->oam, NES_OAM_BYTES, lane);
    uint8_t* obs = a.o.obs + ((size_t)ge * RLE_FRAMES + a.f) * RLE_OBS_PIXELS;
    uint8_t* emph = a.o.emph + ((size_t)ge * RLE_FRAMES + a.f) * RLE_OBS_H;
    draw_frame<true>(&L.r, L.nt, L.oam, log, log_n, a.g.cart, chr_ram, obs, emph, lane);
}

// ----------------------------------------------------------------------------------------- finish
struct FinishArgs {
    GameK g;
    EnvArrays e;
    Outs o;
    Settings s;
    int e0, e1;
};

__device__ __forceinline__ void list_append(const GameK& g, bool want, int e) {
    // one atomic per wavefront: the lanes that restart take consecutive list entries
    const uint64_t b = __ballot(want);
    if (b == 0) return;
    const int lane = (int)(threadIdx.x & 63u);
    const int leader = __builtin_ctzll(b);
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(g.list_count, (uint32_t)__popcll(b));
    base = __shfl(base, leader);
    if (want) g.list[base + (uint32_t)__popcll(b & ((1ull << lane) - 1ull))] = e;
}

// Start: every env of the range restarts (rl/csrc/rlenv_core.cuh:400-404).
__global__ __launch_bounds__(256) void k_start(FinishArgs a) {
    const int k = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    const bool valid = k < a.e1 - a.e0;
    const int e = a.e0 + (valid ? k : 0);
    if (valid) reset_rl(a.g, a.e, a.s, a.g.offset + e);
    list_append(a.g, valid, e);
}

// A listed restart, one workgroup per entry. From a saved level start: the slot's record and key set (its idle and
// restart frames are emulated next). From the boot snapshot: restart template k (k = the idle count) - the record
// after the 4 neutral frames, their pictures, emphasis and fault - with the target and frame counter moved past
// those frames; the env is marked 2 (copied) so that the restart passes leave it alone. Empty key set.
__global__ __launch_bounds__(256) void k_reset_copy(FinishArgs a) {
    const uint32_t count = *a.g.list_count;
    for (uint32_t k = blockIdx.x; k < count; k += gridDim.x) {
        const int e = a.g.list[k], ge = a.g.offset + e;
        const int idle = a.e.ep_idle[ge];
        const int lv = a.e.ep_start ? a.e.ep_start[ge] : -1;
        const int t = idle <= a.s.idle_tmpl ? idle : 0;
        const uint4* src = reinterpret_cast<const uint4*>(lv >= 0 ? &a.g.lv.rec[lv] : &a.g.rst[t]);
        uint4* dst = reinterpret_cast<uint4*>(&a.g.recs[e]);
        for (uint32_t i = threadIdx.x; i < NES_REC_BYTES / 16u; i += blockDim.x) dst[i] = src[i];
        uint32_t* kd = a.g.keys + (size_t)e * a.g.kcap;
        const uint32_t* ks = lv >= 0 ? a.g.lv.keys + (size_t)lv * a.g.kcap : nullptr;
        for (uint32_t i = threadIdx.x; i < a.g.kcap; i += blockDim.x) kd[i] = ks ? ks[i] : 0u;
        if (lv >= 0) continue;
        if (!a.s.no_render) {
            constexpr uint32_t kObs = RLE_FRAMES * RLE_OBS_PIXELS / 16u, kEmph = RLE_FRAMES * RLE_OBS_H / 16u;
            const uint4* so = reinterpret_cast<const uint4*>(a.g.rst_obs + (size_t)t * RLE_FRAMES * RLE_OBS_PIXELS);
            uint4* d = reinterpret_cast<uint4*>(a.o.obs + (size_t)ge * RLE_FRAMES * RLE_OBS_PIXELS);
            for (uint32_t i = threadIdx.x; i < kObs; i += blockDim.x) d[i] = so[i];
            const uint4* se = reinterpret_cast<const uint4*>(a.g.rst_emph + (size_t)t * RLE_FRAMES * RLE_OBS_H);
            uint4* de = reinterpret_cast<uint4*>(a.o.emph + (size_t)ge * RLE_FRAMES * RLE_OBS_H);
            for (uint32_t i = threadIdx.x; i < kEmph; i += blockDim.x) de[i] = se[i];
        }
        if (threadIdx.x == 0) {
            a.e.fault[ge] = a.g.rst_fault[t];
            a.e.target[ge] += (uint64_t)RLE_FRAMES * NES_FRAME_DOTS;
            a.e.ep_frame[ge] += RLE_FRAMES;
            a.e.resetting[ge] = 2;
        }
    }
}

// First tracker update of restarted envs; masks and dropout timeline of every env (rl/csrc/rlenv_core.cuh:138-148,
// 327-342). Thread 0 empties the restart list for the next decision's finish: every kernel that reads it (the copy,
// the restart frames) ran before this one, and this one does not.
__global__ __launch_bounds__(256) void k_reset_finish(FinishArgs a) {
    const int k = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (k == 0) *a.g.list_count = 0;
    if (k < a.e1 - a.e0) {
        const int e = a.e0 + k, ge = a.g.offset + e;
        if (a.e.resetting[ge]) {
            Rl10State st = a.e.st[ge];
            (void)ev::observe_update(a.g.game, a.g.recs[e].ram, a.e.ep_idle[ge] + RLE_FRAMES, st, &a.e.rd[ge],
                                     a.g.keys + (size_t)e * a.g.kcap, a.g.kcap);
            a.e.st[ge] = st;
            a.e.ep_ret[ge] = 0.0f;
            a.e.ep_len[ge] = 0;
            const int sl = a.e.ep_start ? a.e.ep_start[ge] : -1;   // a place: its level is the tracker's
            a.e.ep_maxlvl[ge] = sl >= a.g.lv.levels ? (st.has_best_level ? st.best_level : 0) : sl > 0 ? sl : 0;
            a.e.resetting[ge] = 0;
        }
        const Dropout* d = &a.e.drop[ge];
        const int dr = ev::dropped_now(d);
        uint8_t* mk = a.o.masks + (size_t)ge * RLE_MASK_BYTES;
        for (uint32_t i = 0; i < 9; ++i) mk[i] = (dr >= 0 && dr < 4 && (ev::dpad_bits(i) & (ev::B_UP << dr))) ? 0 : 1;
        mk[9] = 1;
        mk[10] = dr == 4 ? 0 : 1;
        mk[11] = dr == 6 ? 0 : 1;
        mk[12] = 1;
        mk[13] = dr == 5 ? 0 : 1;
        mk[14] = dr == 7 ? 0 : 1;
        mk[15] = 1;
        mk[16] = a.g.start_ok ? 1 : 0;
        mk[17] = 1;
        mk[18] = a.g.select_ok ? 1 : 0;
        uint32_t* tl = reinterpret_cast<uint32_t*>(a.o.tl + (size_t)ge * RLE_TIMELINE_BYTES);
        for (int i = 0; i < RLE_TIMELINE_BYTES / 4; ++i) tl[i] = 0;
        uint8_t* tb = a.o.tl + (size_t)ge * RLE_TIMELINE_BYTES;
        for (uint32_t j = 0; j < RLE_TIMELINE; ++j) {
            const int b = d->ring[(d->head + j) & (RLC_RING - 1)];
            if (b >= 0) tb[b * RLE_TIMELINE + j] = 1;
        }
    }
}

__global__ void k_list_clear(uint32_t* count) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *count = 0;
}

// Level-start saves after a decision's finish, one workgroup per level slot (rl/csrc/rlenv_core.cuh:343-387): the
// claimed arrival replaces the saved one when nothing is saved yet or it has no more deaths (the newest on ties).
// The claim is wave-uniform per workgroup, so every thread takes the same branch.
__global__ __launch_bounds__(256) void k_archive(FinishArgs a) {
    const int q = (int)blockIdx.x;
    const LevelK& L = a.g.lv;
    const unsigned long long cl = L.claim[q];
    if (cl == ~0ull) return;
    const bool take = L.deaths[q] < 0 || (int32_t)(cl >> 32) <= L.deaths[q];
    const int e = (int)(cl & 0xFFFFFFFFull);
    if (take) {
        const uint4* src = reinterpret_cast<const uint4*>(&a.g.recs[e]);
        uint4* dst = reinterpret_cast<uint4*>(&L.rec[q]);
        for (uint32_t i = threadIdx.x; i < NES_REC_BYTES / 16u; i += blockDim.x) dst[i] = src[i];
        const uint32_t* ks = a.g.keys + (size_t)e * a.g.kcap;
        uint32_t* kd = L.keys + (size_t)q * a.g.kcap;
        for (uint32_t i = threadIdx.x; i < a.g.kcap; i += blockDim.x) kd[i] = ks[i];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (take) {
            const int ge = a.g.offset + e;
            L.st[q].st = a.e.st[ge];
            L.st[q].rd = a.e.rd[ge];
            L.target[q] = a.e.target[ge];
            L.frame[q] = a.e.ep_frame[ge];
            L.deaths[q] = (int32_t)(cl >> 32);
        }
        L.claim[q] = ~0ull;
    }
}

// Place saves (rl/csrc/rlenv.cu:100-108): workgroup j copies env env[j] of the game into slot slot[j], skipped where
// the slot is a level slot or out of range. The no-progress clock restarts at a place (rlenv_core.cuh:366-375).
__global__ __launch_bounds__(256) void k_place_save(FinishArgs a, const int32_t* env, const int32_t* slot) {
    const int q = slot[blockIdx.x], e = env[blockIdx.x];
    const LevelK& L = a.g.lv;
    if (q < L.levels || q >= L.cap || e < 0 || e >= a.g.n) return;
    const uint4* src = reinterpret_cast<const uint4*>(&a.g.recs[e]);
    uint4* dst = reinterpret_cast<uint4*>(&L.rec[q]);
    for (uint32_t i = threadIdx.x; i < NES_REC_BYTES / 16u; i += blockDim.x) dst[i] = src[i];
    const uint32_t* ks = a.g.keys + (size_t)e * a.g.kcap;
    uint32_t* kd = L.keys + (size_t)q * a.g.kcap;
    for (uint32_t i = threadIdx.x; i < a.g.kcap; i += blockDim.x) kd[i] = ks[i];
    __syncthreads();
    if (threadIdx.x == 0) {
        const int ge = a.g.offset + e;
        Rl10State st = a.e.st[ge];
        st.idle_frames = 0;
        L.st[q].st = st;
        L.st[q].rd = a.e.rd[ge];
        L.target[q] = a.e.target[ge];
        L.frame[q] = a.e.ep_frame[ge];
        L.deaths[q] = 0;
    }
}


// ------------------------------------------------------------------------------------- codec, gathers
// pack6: 4 colour indices (6 bits) -> 3 bytes, little-endian v = p0 | p1 << 6 | p2 << 12 | p3 << 18
// (rl/csrc/rlenv.cu:127-134). Each thread packs 16 pixels: one 16-byte load, one 12-byte store.
__global__ __launch_bounds__(256) void k_pack6(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, size_t groups) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t g0 = t * 4u;
    if (g0 >= groups) return;
    if (g0 + 4u <= groups) {
        const uint4 q = reinterpret_cast<const uint4*>(src)[t];
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        uint32_t v[4];
        for (int i = 0; i < 4; ++i)
            v[i] = (w[i] & 0x3Fu) | ((w[i] >> 2) & 0xFC0u) | ((w[i] >> 4) & 0x3F000u) | ((w[i] >> 6) & 0xFC0000u);
        uint32_t* o = reinterpret_cast<uint32_t*>(dst + 12u * t);
        o[0] = v[0] | (v[1] << 24);
        o[1] = (v[1] >> 8) | (v[2] << 16);
        o[2] = (v[2] >> 16) | (v[3] << 8);
    } else {
        for (size_t g = g0; g < groups; ++g) {
            const uint32_t v = src[4 * g] | ((uint32_t)src[4 * g + 1] << 6) | ((uint32_t)src[4 * g + 2] << 12) |
                               ((uint32_t)src[4 * g + 3] << 18);
            dst[3 * g] = (uint8_t)v;
            dst[3 * g + 1] = (uint8_t)(v >> 8);
            dst[3 * g + 2] = (uint8_t)(v >> 16);
        }
    }
}

__global__ __launch_bounds__(256) void k_unpack6(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, size_t groups) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t g0 = t * 4u;
    if (g0 >= groups) return;
    if (g0 + 4u <= groups) {
        const uint32_t* in = reinterpret_cast<const uint32_t*>(src + 12u * t);
        const uint32_t a0 = in[0], a1 = in[1], a2 = in[2];
        const uint32_t v[4] = {a0 & 0xFFFFFFu, (a0 >> 24) | ((a1 & 0xFFFFu) << 8), (a1 >> 16) | ((a2 & 0xFFu) << 16),
                               a2 >> 8};
        uint32_t w[4];
        for (int i = 0; i < 4; ++i)
            w[i] = (v[i] & 63u) | (((v[i] >> 6) & 63u) << 8) | (((v[i] >> 12) & 63u) << 16) | (((v[i] >> 18) & 63u) << 24);
        reinterpret_cast<uint4*>(dst)[t] = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        for (size_t g = g0; g < groups; ++g) {
            const uint32_t v = src[3 * g] | ((uint32_t)src[3 * g + 1] << 8) | ((uint32_t)src[3 * g + 2] << 16);
            dst[4 * g] = v & 63u;
            dst[4 * g + 1] = (v >> 6) & 63u;
            dst[4 * g + 2] = (v >> 12) & 63u;
            dst[4 * g + 3] = (v >> 18) & 63u;
        }
    }
}

__global__ void k_gather_rows(uint4* __restrict__ dst, const uint4* __restrict__ src, const int64_t* rows, size_t row_vecs) {
    const size_t j = blockIdx.x;
    const uint4* s = src + (size_t)rows[j] * row_vecs;
    uint4* d = dst + j * row_vecs;
    for (size_t i = blockIdx.y * blockDim.x + threadIdx.x; i < row_vecs; i += (size_t)gridDim.y * blockDim.x) d[i] = s[i];
}

// Standalone reward10 SMB tracker (smb_tracker.h): the signals and what depends only on them for every env-step in
// parallel, the tracker state env by env, the rewards in parallel.
// 1. Four consecutive steps of one env per thread (rows t-1 .. t+3 of ram15 read once).
__global__ __launch_bounds__(256) void k_smb_signals(const uint8_t* __restrict__ ram15, int T, int N,
                                                      const Rl10State* __restrict__ state, ev::SmbStep* __restrict__ rec) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t groups = (size_t)((T + 3) / 4) * (size_t)N;
    if (i >= groups) return;
    const int e = (int)(i % (size_t)N), t0 = (int)(i / (size_t)N) * 4;
    const uint4* src = reinterpret_cast<const uint4*>(ram15);
    const Rl10Game G = rl10_game(RL10_SMB);
    auto signals = [&](int t) {
        const uint4 q = src[(size_t)t * N + e];
        uint8_t b[16];
        memcpy(b, &q, 16);
        return ev::smb_signals(b);
    };
    Rl10Signals p;
    bool had;
    if (t0 > 0) {
        p = signals(t0 - 1);
        had = true;
    } else {
        p = state[e].prev;
        had = state[e].has_prev != 0;
    }
    for (int k = 0; k < 4 && t0 + k < T; ++k) {
        const Rl10Signals s = signals(t0 + k);
        rec[(size_t)(t0 + k) * N + e] = ev::smb_step_record(s, p, had, G);
        p = s;
        had = true;
    }
}
// 2. One env per lane (64-lane blocks: as many CUs as waves), its steps in order; the records of kAhead steps are
// loaded ahead in two register buffers, through row bases that are the same for the whole wave (the buffer holds
// kAhead rows past the last, which the last loads read and nothing uses).
constexpr int kAhead = 4;
__global__ __launch_bounds__(64) void k_smb_chain(ev::SmbStep* __restrict__ rec, const uint8_t* __restrict__ ram15,
                                                   int T, int N, int frames, Rl10State* __restrict__ state) {
    const int e = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (e >= N) return;
    const Rl10Game G = rl10_game(RL10_SMB);
    const int64_t stall = G.stall_frames >= 0.0 ? (int64_t)__builtin_ceil(G.stall_frames) : -1;
    auto row = [&](int t) { return rec + (size_t)(uint32_t)t * (uint32_t)N; };
    auto put = [&](int t, const ev::SmbDec& d) { reinterpret_cast<ev::SmbDec*>(row(t))[e] = d; };
    Rl10State st = state[e];
    ev::SmbChain c{st.done ? 1u : 0u, 0u, st.has_best_level ? st.best_level : -1,
                   st.has_best_progress ? (int32_t)st.best_progress : ev::kNoBest, ev::kNoBest, st.deaths,
                   st.idle_frames, st.score_used};
    ev::SmbStep a[kAhead], b[kAhead];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) a[j] = row(j)[e];
    int t = 0;
    for (; t + 2 * kAhead <= T; t += 2 * kAhead) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) b[j] = row(t + kAhead + j)[e];
#pragma unroll
        for (int j = 0; j < kAhead; ++j) put(t + j, ev::smb_chain_step(a[j], frames, c, stall));
#pragma unroll
        for (int j = 0; j < kAhead; ++j) a[j] = row(t + 2 * kAhead + j)[e];
#pragma unroll
        for (int j = 0; j < kAhead; ++j) put(t + kAhead + j, ev::smb_chain_step(b[j], frames, c, stall));
    }
    for (; t < T; ++t) put(t, ev::smb_chain_step(row(t)[e], frames, c, stall));   // the last T % 8 steps
    st.done = (uint8_t)c.done;
    if (c.end_flags) st.end_reason = (uint8_t)ev::smb_end_reason(c.end_flags);   // ended in this call
    st.has_best_level = c.best_level >= 0 ? 1 : 0;
    if (c.best_level >= 0) st.best_level = c.best_level;
    st.has_best_progress = c.best_progress != ev::kNoBest ? 1 : 0;
    if (c.last_progress != ev::kNoBest) st.best_progress = (double)c.last_progress;
    st.deaths = c.deaths;
    st.idle_frames = c.idle;
    st.score_used = c.score_used;
    if (T > 0) {   // update's prev: the signals of the last step
        const uint4 q = reinterpret_cast<const uint4*>(ram15)[(size_t)(T - 1) * N + e];
        uint8_t bb[16];
        memcpy(bb, &q, 16);
        st.has_prev = 1;
        st.prev = ev::smb_signals(bb);
    }
    state[e] = st;
}
// 3. The rewards and done flags of every env-step.
__global__ __launch_bounds__(256) void k_smb_reward(const ev::SmbDec* __restrict__ dec, size_t n, int frames,
                                                     float* __restrict__ reward, uint8_t* __restrict__ done) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const ev::SmbDec d = dec[i];
    reward[i] = (float)ev::smb_reward(d, frames, rl10_game(RL10_SMB));
    done[i] = (d.flags & ev::DC_DONE) ? 1 : 0;
}

// The per-step records of rl10_smb_run come from a stream-ordered pool of the device (allocated and freed on the
// caller's stream, so calls on different streams never share one), which keeps its memory for the next call.
hipMemPool_t smb_pool(int device) {
    static std::mutex lock;
    static std::map<int, hipMemPool_t> pools;
    std::lock_guard<std::mutex> hold(lock);
    auto it = pools.find(device);
    if (it != pools.end()) return it->second;
    hipMemPoolProps props{};
    props.allocType = hipMemAllocationTypePinned;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = device;
    hipMemPool_t pool = nullptr;
    if (hipMemPoolCreate(&pool, &props) != hipSuccess) throw std::runtime_error("hipMemPoolCreate failed");
    uint64_t keep = ~0ull;
    (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
    pools.emplace(device, pool);
    return pool;
}

// Standalone reward10 tracker of any game: one env per thread, T steps over the 2 KB RAM of each env-step.
struct Rl10RunArgs {
    const uint8_t* ram;
    const int32_t* frames;
    Rl10State* state;
    Rl10Reader* reader;
    uint32_t* keys;
    double* reward;
    uint8_t *done, *end_reason;
    uint32_t* events;
    int32_t *event_level, *deaths;
    int game, T, N;
    uint32_t cap;
};
__global__ __launch_bounds__(256) void k_rl10_run(Rl10RunArgs a) {
    const int e = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (e >= a.N) return;
    Rl10State st = a.state[e];
    uint32_t* keys = a.keys ? a.keys + (size_t)e * a.cap : nullptr;
    for (int t = 0; t < a.T; ++t) {
        const size_t i = (size_t)t * a.N + e;
        const ev::Out u = ev::observe_update(a.game, a.ram + i * 2048u, a.frames[i], st, &a.reader[e], keys, a.cap);
        if (a.reward) a.reward[i] = u.reward;
        if (a.done) a.done[i] = u.done ? 1 : 0;
        if (a.events) a.events[i] = u.events;
        if (a.event_level) a.event_level[i] = u.event_level;
        if (a.deaths) a.deaths[i] = st.deaths;
        if (a.end_reason) a.end_reason[i] = st.end_reason;
    }
    a.state[e] = st;
}

// rlenv_step_static's restart queues, per GPU: the counts of up to kStaticGames games, then the queued env indices
// of up to kStaticEnvs envs in all (each game's at its env offset). In host code the name stands for no device address:
// the library takes the address once per device at rlenv_create (hipGetSymbolAddress) and uses only that.
constexpr uint32_t kStaticGames = 64u, kStaticEnvs = 1u << 18;
static __device__ __align__(256) uint32_t scratch[kStaticGames + kStaticEnvs];

// ============================================================================================== host
struct DevMem {
    std::vector<void*> blocks;
    void* alloc(size_t n) {
        void* p = nullptr;
        if (hipMalloc(&p, n ? n : 1) != hipSuccess) throw std::runtime_error("hipMalloc failed");
        blocks.push_back(p);
        return p;
    }
    template <class T> T* zeros(size_t count) {
        T* p = static_cast<T*>(alloc(sizeof(T) * count));
        if (hipMemset(p, 0, sizeof(T) * count) != hipSuccess) throw std::runtime_error("hipMemset failed");
        return p;
    }
    void upload(void* dst, const void* src, size_t n) {
        if (hipMemcpy(dst, src, n, hipMemcpyHostToDevice) != hipSuccess) throw std::runtime_error("upload failed");
    }
    ~DevMem() {
        for (void* p : blocks) (void)hipFree(p);
    }
};

// ------------------------------------------------------------------------------- translated kernels (jit.h)
// The device headers the translated kernels are compiled from, embedded by the Makefile.
struct JitHeader { const char* name; const char* text; };
const JitHeader kJitHeaders[] = {
#include "jit_headers.inc"
};
// hiprtc options: the Makefile's device flags, then the words of RLENV_JIT_EXTRA (diagnostics; tests pass
// "-mllvm -amdgpu-s-branch-bits=5", which relaxes nearly every branch into a far jump, to check that the kernels
// hold no far-jump hazard whatever the layout).
const char* const kJitOptions[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm",
                                   "-structurizecfg-skip-uniform-regions=true", "-mllvm", "-enable-tail-merge=false"};
std::vector<std::string> jit_options() {
    std::vector<std::string> o(std::begin(kJitOptions), std::end(kJitOptions));
    if (const char* extra = std::getenv("RLENV_JIT_EXTRA")) {
        std::string w;
        for (const char* c = extra;; ++c) {
            if (*c == 0 || *c == ' ') {
                if (!w.empty()) o.push_back(w);
                w.clear();
                if (*c == 0) break;
            } else {
                w += *c;
            }
        }
    }
    return o;
}

// One translation compiled for gfx950, shared by every env of the process whose translation has the same text; with
// RLENV_JIT_CACHE=<directory> the code object is also kept there, named by a hash of everything it is built from.
struct JitJob {
    std::string blocks, source;
    std::atomic<int> state{0};   // 0 compiling, 1 compiled, 2 failed
    std::vector<char> code;
    std::string error;
    double seconds = 0;
    int far_jumps = 0, hazards = 0;   // jit_check.h: far jumps in the code object, and those into live SCC
};

// A game's translated kernel: its job, the fetch table with the blocks' keys, the variant it was built for (decision
// frames drawn from frame banks or not), and its module once loaded on the env's device.
struct JitSlot {
    std::shared_ptr<JitJob> job;
    const uint32_t* fetchw = nullptr;
    bool bank = false, banked = false;   // built for frames drawn from frame banks; for a banked-PRG board
    uint32_t blocks = 0, instructions = 0;
    hipModule_t mod = nullptr;
    hipFunction_t fn = nullptr;        // k_emu_jit: frames drawn from frame banks (a bank translation only)
    hipFunction_t fn_draw = nullptr;   // k_emu_jit_draw: frames the emulator's waves draw themselves
    bool failed = false;
};

uint64_t fnv1a(const char* p, size_t n, uint64_t h = 0xcbf29ce484222325ull) {
    for (size_t i = 0; i < n; ++i) h = (h ^ (uint8_t)p[i]) * 0x100000001b3ull;
    return h;
}

// A compiled code object is used only when jit_check.h finds no far jump into live SCC in it (a miscompile that
// gives wrong results silently); otherwise the job fails and its game keeps the library's own kernel.
bool jit_validate(JitJob& job) {
    std::string where;
    job.hazards = jit_far_branch_hazards(job.code, &job.far_jumps, &where);
    if (job.hazards == 0) return true;
    job.error = job.hazards < 0 ? std::string("jit check: the code object could not be disassembled")
                                : "jit check: " + std::to_string(job.hazards) + " of " +
                                      std::to_string(job.far_jumps) + " far jumps land where SCC is live (" + where +
                                      ")";
    return false;
}

void jit_compile(JitJob& job) {
    const auto t0 = std::chrono::steady_clock::now();
    const std::vector<std::string> opts = jit_options();
    std::string path;
    if (const char* dir = std::getenv("RLENV_JIT_CACHE"); dir && *dir) {
        uint64_t h = fnv1a(job.source.data(), job.source.size());
        h = fnv1a(job.blocks.data(), job.blocks.size(), h);
        for (const JitHeader& hd : kJitHeaders) h = fnv1a(hd.text, strlen(hd.text), h);
        for (const std::string& o : opts) h = fnv1a(o.c_str(), o.size(), h);
        char name[48];
        snprintf(name, sizeof name, "/rlenv_jit_%016llx.hsaco", (unsigned long long)h);
        path = std::string(dir) + name;
        if (FILE* f = fopen(path.c_str(), "rb")) {
            char buf[65536];
            size_t n;
            while ((n = fread(buf, 1, sizeof buf, f)) > 0) job.code.insert(job.code.end(), buf, buf + n);
            fclose(f);
            if (!job.code.empty()) {
                const bool ok = jit_validate(job);
                job.seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
                job.state.store(ok ? 1 : 2, std::memory_order_release);
                return;
            }
        }
    }
    std::vector<const char*> texts, names;
    for (const JitHeader& hd : kJitHeaders) {
        texts.push_back(hd.text);
        names.push_back(hd.name);
    }
    texts.push_back(job.blocks.c_str());
    names.push_back("jit_blocks.inc");
    hiprtcProgram prog = nullptr;
    hiprtcResult r = hiprtcCreateProgram(&prog, job.source.c_str(), "rlenv_jit.hip", (int)texts.size(), texts.data(),
                                         names.data());
    if (r == HIPRTC_SUCCESS) {
        std::vector<const char*> o;
        for (const std::string& w : opts) o.push_back(w.c_str());
        r = hiprtcCompileProgram(prog, (int)o.size(), o.data());
    }
    bool ok = r == HIPRTC_SUCCESS;
    if (ok) {
        size_t n = 0;
        ok = hiprtcGetCodeSize(prog, &n) == HIPRTC_SUCCESS && n > 0;
        job.code.resize(n);
        ok = ok && hiprtcGetCode(prog, job.code.data()) == HIPRTC_SUCCESS;
    }
    if (!ok) {
        job.error = std::string("hiprtc: ") + hiprtcGetErrorString(r);
        size_t n = 0;
        if (prog && hiprtcGetProgramLogSize(prog, &n) == HIPRTC_SUCCESS && n > 1) {
            std::string log(n, '\0');
            if (hiprtcGetProgramLog(prog, &log[0]) == HIPRTC_SUCCESS) job.error += "\n" + log.substr(0, 4000);
        }
    }
    if (prog) hiprtcDestroyProgram(&prog);
    ok = ok && jit_validate(job);
    if (ok && !path.empty()) {   // written aside, then renamed: a reader never sees half a file
        const std::string tmp = path + ".tmp" + std::to_string((unsigned long long)std::hash<std::thread::id>{}(
                                                    std::this_thread::get_id()));
        if (FILE* f = fopen(tmp.c_str(), "wb")) {
            const bool written = fwrite(job.code.data(), 1, job.code.size(), f) == job.code.size();
            fclose(f);
            if (!written || rename(tmp.c_str(), path.c_str()) != 0) remove(tmp.c_str());
        }
    }
    job.seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    job.state.store(ok ? 1 : 2, std::memory_order_release);
}

// The compile queue: one worker thread per process compiles the translations in the order they were asked for
// (hiprtc runs one compile at a time in a process anyway), so rlenv_create returns once its games are booted and a
// game's decision frames switch to the translated kernel at a call boundary after its compile (jit_refresh). The
// thread is started on first use and detached; a handler registered with atexit at that point (after the compiler
// library's own initialisation, so it runs before its teardown) drops the jobs not started and waits for the one in
// flight, so that no compile runs while the process tears down.
struct JitQueue {
    std::mutex lock;
    std::condition_variable cv;
    std::deque<std::shared_ptr<JitJob>> jobs;
    bool started = false, stopping = false, busy = false;
};
JitQueue& jit_queue() {
    static JitQueue* q = new JitQueue();   // never destroyed: the worker may use it during exit
    return *q;
}
void jit_worker() {
    JitQueue& q = jit_queue();
    std::unique_lock<std::mutex> hold(q.lock);
    for (;;) {
        q.cv.wait(hold, [&] { return q.stopping || !q.jobs.empty(); });
        if (q.stopping) return;
        std::shared_ptr<JitJob> job = q.jobs.front();
        q.jobs.pop_front();
        q.busy = true;
        hold.unlock();
        jit_compile(*job);
        hold.lock();
        q.busy = false;
        q.cv.notify_all();
    }
}
void jit_drain_at_exit() {
    JitQueue& q = jit_queue();
    std::unique_lock<std::mutex> hold(q.lock);
    q.stopping = true;
    for (const auto& job : q.jobs) {
        job->error = "the process exited before the compile";
        job->state.store(2, std::memory_order_release);
    }
    q.jobs.clear();
    q.cv.notify_all();
    q.cv.wait(hold, [&] { return !q.busy; });
}
void jit_enqueue(const std::shared_ptr<JitJob>& job) {
    JitQueue& q = jit_queue();
    std::lock_guard<std::mutex> hold(q.lock);
    if (q.stopping) {
        job->error = "the process is exiting";
        job->state.store(2, std::memory_order_release);
        return;
    }
    if (!q.started) {
        q.started = true;
        std::atexit(jit_drain_at_exit);
        std::thread(jit_worker).detach();
    }
    q.jobs.push_back(job);
    q.cv.notify_all();
}

// The job of (blocks, source): this process's existing one (fresh = false), or a new one the caller compiles.
constexpr int kJitMinEnvs = 1024;   // games of fewer envs run the library's kernel unless RLENV_JIT=sync

std::shared_ptr<JitJob> jit_job(std::string blocks, std::string source, bool& fresh) {
    static std::mutex lock;
    static std::map<std::string, std::shared_ptr<JitJob>> jobs;
    std::lock_guard<std::mutex> hold(lock);
    std::string key = source + blocks;
    auto it = jobs.find(key);
    fresh = it == jobs.end();
    if (!fresh) return it->second;
    auto job = std::make_shared<JitJob>();
    job->blocks = std::move(blocks);
    job->source = std::move(source);
    jobs.emplace(std::move(key), job);
    return job;
}

struct GameH {
    GameK k;
    int game;
    std::shared_ptr<JitSlot> jit;   // fixed-PRG carts: the translated kernel (nullptr: none)
};

// Kernel classes of a decision, for the per-kernel clock (rlenv_kernel_times).
enum KClass : int {
    KC_EMU = 0, KC_RENDER, KC_FINISH, KC_RESET_COPY, KC_EMU_RESTART, KC_RENDER_RESTART, KC_RESET_FINISH, KC_EMU_IDLE,
    KC_ARCHIVE, KC_EMU_DRAW, KC_COUNT
};

// Optional per-launch HIP-event clock: when on, every launch of a decision is bracketed by two events on its
// stream; the durations are summed per kernel class when read. Events are recycled through a pool.
struct KernelClock {
    bool on = false;
    struct Mark { int cls; hipEvent_t a, b; };
    std::vector<hipEvent_t> pool;
    std::vector<Mark> marks;
    hipEvent_t take() {
        if (!pool.empty()) {
            hipEvent_t ev = pool.back();
            pool.pop_back();
            return ev;
        }
        // (timing only: no system-scope fence when the event is reached - the cache writeback and invalidation it
        // costs slowed the decision step by 0.9 % with two events a launch)
        hipEvent_t ev = nullptr;
        if (hipEventCreateWithFlags(&ev, hipEventDisableSystemFence) != hipSuccess)
            throw std::runtime_error("hipEventCreate failed");
        return ev;
    }
    template <class F> void run(int cls, hipStream_t st, F&& launch) {
        if (!on) {
            launch();
            return;
        }
        Mark m{cls, take(), take()};
        (void)hipEventRecord(m.a, st);
        launch();
        (void)hipEventRecord(m.b, st);
        marks.push_back(m);
    }
    // Sums and forgets the recorded launches (waits for them). Returns 0, or 1 on a HIP error.
    int drain(double* ms, int64_t* count) {
        int bad = 0;
        for (const Mark& m : marks) {
            float t = 0.f;
            bad |= hipEventSynchronize(m.b) != hipSuccess;
            bad |= hipEventElapsedTime(&t, m.a, m.b) != hipSuccess;
            ms[m.cls] += t;
            count[m.cls] += 1;
            pool.push_back(m.a);
            pool.push_back(m.b);
        }
        marks.clear();
        return bad;
    }
    ~KernelClock() {
        for (const Mark& m : marks) {
            (void)hipEventDestroy(m.a);
            (void)hipEventDestroy(m.b);
        }
        for (hipEvent_t ev : pool) (void)hipEventDestroy(ev);
    }
};

// Streams and events, all at the default priority and created with the env (a call allocates nothing):
// * with more than one game, one stream per game and the events that fork a call's work from the caller's stream
//   onto them and join it back (rl/csrc/rlenv.cu:38-40, 173-182): the games step concurrently, so a batch of many
//   small games fills the GPU as one large game does;
// * with one game, a render stream, per decision frame f an "emulated" event and one "drawn" event: frames 0 and 1
//   are drawn on the render stream from their frame banks while the frames after them are emulated on the caller's
//   stream.
struct RenderPipe {
    hipStream_t stream = nullptr;
    hipEvent_t emulated[RLE_FRAMES] = {}, drawn = nullptr;
};
struct GameStreams {
    std::vector<hipStream_t> s;
    std::vector<hipEvent_t> done;
    std::vector<RenderPipe> render;
    hipEvent_t fork = nullptr;
    static hipEvent_t event() {
        hipEvent_t ev = nullptr;
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) throw std::runtime_error("hipEventCreate failed");
        return ev;
    }
    static hipStream_t stream() {
        hipStream_t st = nullptr;
        if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) throw std::runtime_error("hipStreamCreate failed");
        return st;
    }
    void create(size_t n) {
        render.resize(n);
        if (n == 1) {
            render[0].stream = stream();
            for (int f = 0; f < RLE_FRAMES; ++f) render[0].emulated[f] = event();
            render[0].drawn = event();
            return;
        }
        fork = event();
        for (size_t i = 0; i < n; ++i) {
            s.push_back(stream());
            done.push_back(event());
        }
    }
    ~GameStreams() {
        for (hipEvent_t ev : done) (void)hipEventDestroy(ev);
        for (hipStream_t st : s) (void)hipStreamDestroy(st);
        for (RenderPipe& p : render) {
            for (int f = 0; f < RLE_FRAMES; ++f)
                if (p.emulated[f]) (void)hipEventDestroy(p.emulated[f]);
            if (p.drawn) (void)hipEventDestroy(p.drawn);
            if (p.stream) (void)hipStreamDestroy(p.stream);
        }
        if (fork) (void)hipEventDestroy(fork);
    }
};

struct Env {
    DevMem mem;
    GameStreams gs;          // per-game streams (with more than one game) and render pipes
    int one_round = 8192;    // one-console waves the GPU holds at once: CUs x 4 SIMDs x 8 waves
    int device = 0;
    int total = 0;
    std::vector<GameH> games;
    EnvArrays e{};
    Outs o{};
    Settings s{};
    uint32_t* optab = nullptr;
    uint32_t budget = NES_BUDGET;
    int lv_cap = 0;          // level starts / places per game (0 = off)
    uint32_t* scratch = nullptr;   // this device's static restart-queue scratch (rlenv_step_static)
    mutable KernelClock clock;
    ~Env() {
        bool loaded = false;
        for (const GameH& gh : games) loaded = loaded || (gh.jit && gh.jit->mod);
        if (loaded) {   // no launch of a translated kernel may be left in flight when its module goes
            (void)hipSetDevice(device);
            (void)hipDeviceSynchronize();
            for (const GameH& gh : games)
                if (gh.jit && gh.jit->mod) (void)hipModuleUnload(gh.jit->mod);
        }
    }
};

// The translated kernel of the game whose device arguments are g (found by its first env, which copies keep).
JitSlot* jit_slot(const Env& env, const GameK& g) {
    for (const GameH& gh : env.games)
        if (gh.jit && gh.k.offset == g.offset && gh.k.n == g.n) return gh.jit.get();
    return nullptr;
}

// Whether the translated kernel can be launched: loads its module on the env's device the first time its job has
// compiled. A failed compile or load leaves the game on the library's own kernel (the results are the same). Called
// only between decisions (jit_refresh, jit_wait, jit_status), so that the frames of one decision run one kernel.
bool jit_ready(const Env& env, JitSlot& j) {
    if (j.fn_draw) return true;
    if (j.failed || !j.job) return false;
    const int st = j.job->state.load(std::memory_order_acquire);
    if (st == 0) return false;
    if (st == 2) {
        j.failed = true;
        return false;
    }
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (cur != env.device) (void)hipSetDevice(env.device);
    const bool ok = hipModuleLoadData(&j.mod, j.job->code.data()) == hipSuccess &&
                    (!j.bank || hipModuleGetFunction(&j.fn, j.mod, "k_emu_jit") == hipSuccess) &&
                    hipModuleGetFunction(&j.fn_draw, j.mod, "k_emu_jit_draw") == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        if (j.mod) (void)hipModuleUnload(j.mod);
        j.mod = nullptr;
        j.fn = j.fn_draw = nullptr;
        j.failed = true;
    }
    if (cur >= 0 && cur != env.device) (void)hipSetDevice(cur);
    return ok;
}

// At the start of a call that launches decision frames: the games whose compile has finished since switch to their
// translated kernels.
void jit_refresh(const Env& env) {
    for (const GameH& gh : env.games)
        if (gh.jit && !gh.jit->fn_draw && !gh.jit->failed) (void)jit_ready(env, *gh.jit);
}

// The address of `scratch` on each device, taken once with that device current.
uint32_t* scratch_of(int device) {
    static std::mutex lock;
    static uint32_t* ptr[64] = {};
    if (device < 0 || device >= 64) throw std::runtime_error("device index out of range");
    std::lock_guard<std::mutex> hold(lock);
    if (!ptr[device]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
            throw std::runtime_error("hipGetSymbolAddress(scratch) failed");
        ptr[device] = static_cast<uint32_t*>(p);
    }
    return ptr[device];
}

// Runs f(game index, stream) for every game: on the caller's stream for a one-game env; otherwise each game on its
// own stream, forked from and joined back to the caller's stream. Returns 0, or 1 with g_error set.
// The runtime maps more streams than it has hardware queues (4 by default) onto shared queues, which run what they
// hold in order, and a wait enqueued on the caller's stream becomes a barrier in its queue. So every game's work is
// enqueued before the caller's stream waits on any game: joined one by one, the games that share the caller's queue
// would wait behind the join of every game enqueued before them.
template <class F>
int for_games(Env& env, hipStream_t st, F&& f) {
    const size_t n = env.games.size();
    if (n == 1) {
        f(0, st);
        return 0;
    }
    bool bad = hipEventRecord(env.gs.fork, st) != hipSuccess;
    for (size_t gi = 0; gi < n; ++gi) {
        const hipStream_t gst = env.gs.s[gi];
        bad |= hipStreamWaitEvent(gst, env.gs.fork, 0) != hipSuccess;
        f(gi, gst);
        bad |= hipEventRecord(env.gs.done[gi], gst) != hipSuccess;
    }
    for (size_t gi = 0; gi < n; ++gi) bad |= hipStreamWaitEvent(st, env.gs.done[gi], 0) != hipSuccess;
    if (bad) g_error = "fork/join of the game streams failed";
    return bad ? 1 : 0;
}

// iNES -> cart description; the PRG is padded to a power of two by repeating a short image (NROM-128).
struct Parsed {
    std::vector<uint8_t> prg, chr;
    uint32_t board = 0, mirroring = 0, bus_conflicts = 0;
};

Parsed parse_ines(const uint8_t* rom, size_t size) {
    if (size < 16 || std::memcmp(rom, "NES\x1A", 4) != 0) throw std::runtime_error("not an iNES image");
    const size_t prg = (size_t)rom[4] * 16384u, chr = (size_t)rom[5] * 8192u;
    const uint32_t mapper = (rom[6] >> 4) | (rom[7] & 0xF0u);
    const size_t skip = 16u + ((rom[6] & 4u) ? 512u : 0u);
    if (rom[6] & 8u) throw std::runtime_error("four-screen nametables are not supported");
    if (mapper > 4u && mapper != 9u)
        throw std::runtime_error("unsupported mapper " + std::to_string(mapper) +
                                 " (supported: 0 NROM, 1 MMC1, 2 UxROM, 3 CNROM, 4 MMC3, 9 MMC2)");
    if (mapper == 9u && chr == 0) throw std::runtime_error("MMC2 needs CHR ROM");
    if (prg == 0 || skip + prg + chr > size) throw std::runtime_error("truncated iNES image");
    Parsed p;
    size_t padded = 8192;
    while (padded < prg) padded <<= 1;
    p.prg.resize(padded);
    for (size_t o = 0; o < padded; o += prg) std::memcpy(p.prg.data() + o, rom + skip, std::min(prg, padded - o));
    p.chr.assign(rom + skip + prg, rom + skip + prg + chr);
    p.board = mapper == 9u ? NES_BOARD_MMC2 : mapper;
    p.mirroring = rom[6] & 1u;
    // UxROM / CNROM bus conflicts only when the header declares them: NES 2.0, submapper 2 (patch:4008)
    p.bus_conflicts = (mapper == 2u || mapper == 3u) && (rom[7] & 0x0Cu) == 0x08u && (rom[8] >> 4) == 2u;
    return p;
}

// RLENV_TRACE=1: synchronise after every launch and print its name and time (diagnostics).
bool trace_on() {
    static const bool on = std::getenv("RLENV_TRACE") != nullptr;
    return on;
}
void trace(const char* what, hipStream_t st) {
    if (!trace_on()) return;
    static double t0 = 0;
    const hipError_t e = hipStreamSynchronize(st);
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    const double now = ts.tv_sec + ts.tv_nsec * 1e-9;
    std::fprintf(stderr, "[rlenv] %-14s %s %.3f ms\n", what, hipGetErrorString(e), t0 ? (now - t0) * 1e3 : 0.0);
    std::fflush(stderr);
    t0 = now;
}

int check(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        g_error = std::string(what) + ": " + hipGetErrorString(err);
        return 1;
    }
    return 0;
}

FinishArgs finish_args(const Env& env, const GameK& g, int e0, int e1, const Outs& o) {
    return FinishArgs{g, env.e, o, env.s, e0, e1};
}

// bank >= 0: a decision frame whose picture is drawn from frame bank `bank`; draw: a decision frame the emulator's
// waves draw themselves, and with finish the decision's last, whose waves also do the finish.
void launch_emu(const Env& env, const GameK& g, const Outs& o, int mode, int f, bool use_list, int e0, int e1,
                hipStream_t st, int bank = -1, bool draw = false, bool finish = false) {
    EmuArgs a{g, env.e, o, env.s, env.optab, mode, f, use_list ? 1 : 0, e0, e1, 0, 0, nullptr, env.budget,
              bank >= 0 ? g.bank[bank] : nullptr, bank >= 0 ? g.bank_chr[bank] : nullptr, finish ? 1 : 0};
    const int blocks = use_list ? g.n : e1 - e0;
    const int cls = mode == EMU_DECISION ? (draw ? KC_EMU_DRAW : KC_EMU) : mode == EMU_IDLE ? KC_EMU_IDLE
                                                                                             : KC_EMU_RESTART;
    // decision frames of a fixed-PRG cart run its translated kernel once that is compiled and loaded, when it was
    // built for the way this launch's frame is drawn
    JitSlot* js = mode == EMU_DECISION && blocks > 0 ? jit_slot(env, g) : nullptr;
    hipFunction_t fn = nullptr;
    if (js && js->fn_draw) fn = draw ? js->fn_draw : a.bank ? js->fn : nullptr;
    if (fn) {
        a.g.cart.fetchw = js->fetchw;
        void* args[] = {&a};
        env.clock.run(cls, st, [&] {
            (void)hipModuleLaunchKernel(fn, (unsigned)blocks, 1, 1, 64, 1, 1, 0, st, args, nullptr);
        });
        trace("emu_jit", st);
        return;
    }
    if (blocks > 0)
        env.clock.run(cls, st, [&] {
            // the fast path knows two kinds of board: fixed 32 KB PRG (NROM, CNROM) and banked PRG (the rest)
            const bool nrom = g.cart.board == NES_BOARD_NROM || g.cart.board == NES_BOARD_CNROM;
            if (a.bank) {
                if (nrom) hipLaunchKernelGGL((k_emu_w<NES_BOARD_NROM, true, false>), dim3(blocks), dim3(64), 0, st, a);
                else hipLaunchKernelGGL((k_emu_w<NES_BOARD_MMC3, true, false>), dim3(blocks), dim3(64), 0, st, a);
            } else if (draw) {
                if (nrom) hipLaunchKernelGGL((k_emu_w<NES_BOARD_NROM, false, true>), dim3(blocks), dim3(64), 0, st, a);
                else hipLaunchKernelGGL((k_emu_w<NES_BOARD_MMC3, false, true>), dim3(blocks), dim3(64), 0, st, a);
            } else {
                if (nrom) hipLaunchKernelGGL((k_emu_w<NES_BOARD_NROM, false, false>), dim3(blocks), dim3(64), 0, st, a);
                else hipLaunchKernelGGL((k_emu_w<NES_BOARD_MMC3, false, false>), dim3(blocks), dim3(64), 0, st, a);
            }
        });
    trace(mode == EMU_DECISION ? "emu" : mode == EMU_IDLE ? "emu_idle" : "emu_restart", st);
}

void launch_render(const Env& env, const GameK& g, const Outs& o, int f, bool use_list, bool restart, int e0, int e1,
                   hipStream_t st, int bank = -1) {
    RenderArgs a{g, env.e, o, env.s, f, use_list ? 1 : 0, restart ? 1 : 0, e0, e1,
                 bank >= 0 ? g.bank[bank] : nullptr, bank >= 0 ? g.bank_chr[bank] : nullptr};
    const int n = use_list ? g.n : e1 - e0;
    if (n > 0)
        env.clock.run(restart ? KC_RENDER_RESTART : KC_RENDER, st,
                      [&] {
                          if (a.bank) hipLaunchKernelGGL(k_render<true>, dim3(n), dim3(64), 0, st, a);
                          else hipLaunchKernelGGL(k_render<false>, dim3(n), dim3(64), 0, st, a);
                      });
    trace(restart ? "render_restart" : "render", st);
}

// The restart half of a decision / start: snapshot copy, 4 neutral frames with pictures, first tracker update.
void restart_phases(const Env& env, const GameK& g, const Outs& o, int e0, int e1, hipStream_t st) {
    const FinishArgs fa = finish_args(env, g, e0, e1, o);
    const int n = e1 - e0;
    env.clock.run(KC_RESET_COPY, st, [&] {
        hipLaunchKernelGGL(k_reset_copy, dim3(std::min(std::max(n, 1), 2048)), dim3(256), 0, st, fa);
    });
    trace("reset_copy", st);
    // Idle frames: a restart from the boot snapshot copied the template that holds them (the template count equals
    // idle_max); one from a saved level start emulates them here.
    // Only a restart from a saved level start emulates; one from the boot snapshot was a copy.
    if (g.lv.cap > 0) {
        if (env.s.idle_max > 0) launch_emu(env, g, o, EMU_IDLE, 0, true, e0, e1, st);
        for (int f = 0; f < RLE_FRAMES; ++f) {
            launch_emu(env, g, o, EMU_RESTART, f, true, e0, e1, st);
            launch_render(env, g, o, f, true, true, e0, e1, st);
        }
    }
    env.clock.run(KC_RESET_FINISH, st,
                  [&] { hipLaunchKernelGGL(k_reset_finish, dim3((n + 255) / 256), dim3(256), 0, st, fa); });
    trace("reset_finish", st);
}


// A decision of envs [e0, e1) of game g: 4 frames, then the finish, the level saves and the restart pass.
// Pipelined (a one-game env whose frame launch fits in one round of waves, so that waves retiring from the
// emulator leave CU slots idle): frames 0 and 1 are drawn on the game's render stream from frame banks 0 and 1 while
// the frames after them are emulated on `st`, frames 2 and 3 by the waves that emulate them (drawn on the render
// stream too, frame 2 left the render stream's last launch running alone after the emulation: 3.42 against 3.33
// ms per decision of 8192 consoles), and the restart pass, which writes the pictures of restarted envs, waits until
// every frame is drawn (so does the next decision, which refills the banks, through it). Otherwise each frame is
// drawn on `st` after it is emulated: with several rounds of waves, or with other games' streams, the CUs are
// already kept busy.
constexpr int kBankFrames = 2;   // decision frames drawn on the render stream when pipelined: 0 .. kBankFrames - 1
void decision_phases(const Env& env, const GameK& g, const RenderPipe& p, const Outs& o, int e0, int e1,
                     hipStream_t st) {
    const int n = e1 - e0;
    if (n <= 0) return;
    const bool draw = !env.s.no_render;
    const bool pipelined = draw && env.games.size() == 1 && n <= env.one_round;
    for (int f = 0; f < RLE_FRAMES; ++f) {
        if (!pipelined || f >= kBankFrames) {   // emulated and drawn by the same waves; the last one finishes too
            launch_emu(env, g, o, EMU_DECISION, f, false, e0, e1, st, -1, true, f == RLE_FRAMES - 1);
            continue;
        }
        launch_emu(env, g, o, EMU_DECISION, f, false, e0, e1, st, f);
        (void)hipEventRecord(p.emulated[f], st);
        (void)hipStreamWaitEvent(p.stream, p.emulated[f], 0);
        launch_render(env, g, o, f, false, false, e0, e1, p.stream, f);
    }
    if (pipelined) (void)hipEventRecord(p.drawn, p.stream);
    const FinishArgs fa = finish_args(env, g, e0, e1, o);   // (the finish itself ran in the last frame's waves)
    if (g.lv.cap > 0) {   // level-start saves, before any restart (restarts read the saves of earlier decisions)
        env.clock.run(KC_ARCHIVE, st,
                      [&] { hipLaunchKernelGGL(k_archive, dim3(g.lv.levels), dim3(256), 0, st, fa); });
        trace("archive", st);
    }
    if (pipelined) (void)hipStreamWaitEvent(st, p.drawn, 0);
    restart_phases(env, g, o, e0, e1, st);
}

// Fetch-table entry of the instruction at a (NROM: a CPU address; banked boards: a PRG byte offset, whose low 13
// bits are those of the CPU address wherever its 8 KB page is mapped), opcode op, next bytes b1 b2: the dispatch key
// (a hot key for the opcodes of kHotOps, except a branch whose target is on another page) and the decoded operand
// word the handlers take (wave_dev.h fx): the operand byte of a two-byte instruction; a branch's target times 8
// (NROM; pc past $FFFF not wrapped, as the interpreter counts it) or its sign-extended offset (banked); JMP's and
// JSR's target (times 8 on NROM); else b1 | b2 << 8.
void fetch_entry(uint32_t* e, uint32_t a, uint32_t op, uint32_t b1, uint32_t b2, bool nrom) {
    const uint32_t d = kOptab.t[op], mode = d & 15u, grp = (d >> 8) & 15u;
    uint32_t base = b1 | (b2 << 8);
    bool cross = false;
    if (grp == G_ILL || grp == G_BRK) {
        e[0] = op;   // the generic step runs (and faults on) it
        e[1] = base;
        return;
    }
    if (mode == M_IMM || mode == M_ZP || mode == M_ZPX || mode == M_ZPY || mode == M_IZX || mode == M_IZY) {
        base = b1;
    } else if (mode == M_REL) {
        const uint32_t off = (uint32_t)(int32_t)(int8_t)b1, tgt = a + 2u + off;
        cross = ((a + 2u) ^ tgt) & 0xFF00u;   // the page of pc + 2 and of the target (low bits of a suffice)
        base = nrom ? tgt << 3 : off << 3;
    } else if (nrom && (op == 0x4Cu || op == 0x20u)) {
        base <<= 3;
    }
    uint32_t hot = 0;
    while (hot < 32u && kHotOps[hot] != op) ++hot;
    e[0] = hot < 32u && !cross ? kHotKey + hot : op;
    e[1] = base;
}

// The restart templates of a game (GameK::rst): the snapshot and every idle template, each run through a restart's
// 4 neutral frames (rl/csrc/rlenv_core.cuh:320-326, ph_reset_frame, and the restart pass of ph_render) - one
// launch per frame over all templates, each drawn into its own pictures. A fault in those frames is recorded, not an
// error: the episode that copies the template ends with it at its first decision, as one that emulated them would.
void build_restart_templates(Env& env, GameK& g) {
    const int count = env.s.idle_tmpl + 1;
    NesRec* rst = const_cast<NesRec*>(g.rst);
    if (hipMemcpy(&rst[0], &g.recs[g.n], sizeof(NesRec), hipMemcpyDeviceToDevice) != hipSuccess ||
        (count > 1 && hipMemcpy(&rst[1], g.idle, sizeof(NesRec) * (size_t)(count - 1), hipMemcpyDeviceToDevice) !=
                          hipSuccess))
        throw std::runtime_error("restart template copy failed");
    GameK t = g;
    t.recs = rst;
    t.offset = 0;
    Outs o = env.o;
    o.obs = const_cast<uint8_t*>(g.rst_obs);
    o.emph = const_cast<uint8_t*>(g.rst_emph);
    Settings s = env.s;
    s.no_render = 0;
    for (int f = 0; f < RLE_FRAMES; ++f) {
        const EmuArgs a{t, env.e, o, s, env.optab, EMU_TEMPLATE, f, 0, 0, count, 0,
                        g.tmpl_target + (uint64_t)f * NES_FRAME_DOTS, const_cast<uint32_t*>(g.rst_fault), env.budget};
        if (g.cart.board == NES_BOARD_NROM || g.cart.board == NES_BOARD_CNROM)
            hipLaunchKernelGGL((k_emu_w<NES_BOARD_NROM, false, false>), dim3(count), dim3(64), 0, 0, a);
        else
            hipLaunchKernelGGL((k_emu_w<NES_BOARD_MMC3, false, false>), dim3(count), dim3(64), 0, 0, a);
        const RenderArgs r{t, env.e, o, s, f, 0, 0, 0, count};
        hipLaunchKernelGGL(k_render<false>, dim3(count), dim3(64), 0, 0, r);
    }
    if (hipDeviceSynchronize() != hipSuccess || check("restart templates")) throw std::runtime_error(g_error);
}

void boot_game(Env& env, GameH& gh, const uint8_t* pads, size_t npads) {
    GameK& g = gh.k;
    hipLaunchKernelGGL(k_power_on, dim3(1), dim3(1), 0, 0, &g.recs[g.n], g.cart);
    trace("power_on", 0);
    uint32_t* fault = env.mem.zeros<uint32_t>(1);
    uint64_t target = NES_VBLANK_DOT;
    auto frame = [&](NesRec* base, int index, uint32_t pad) {
        GameK one = g;
        one.recs = base;
        EmuArgs a{one, env.e, env.o, env.s, env.optab, EMU_BOOT, 0, 0, index, index + 1, pad, target, fault,
                  env.budget};
        if (g.cart.board == NES_BOARD_NROM || g.cart.board == NES_BOARD_CNROM)
            hipLaunchKernelGGL((k_emu_w<NES_BOARD_NROM, false, false>), dim3(1), dim3(64), 0, 0, a);
        else
            hipLaunchKernelGGL((k_emu_w<NES_BOARD_MMC3, false, false>), dim3(1), dim3(64), 0, 0, a);
        target += NES_FRAME_DOTS;
    };
    for (size_t i = 0; i < npads; ++i) frame(g.recs, g.n, pads[i]);
    g.tmpl_target = target;
    NesRec* idle = const_cast<NesRec*>(g.idle);
    for (int k = 1; k <= env.s.idle_tmpl; ++k) {
        const NesRec* src = k == 1 ? &g.recs[g.n] : &idle[k - 2];
        if (hipMemcpy(&idle[k - 1], src, sizeof(NesRec), hipMemcpyDeviceToDevice) != hipSuccess)
            throw std::runtime_error("idle template copy failed");
        frame(idle, k - 1, 0);
    }
    uint32_t host_fault = 0;
    if (hipMemcpy(&host_fault, fault, 4, hipMemcpyDeviceToHost) != hipSuccess) throw std::runtime_error("boot sync failed");
    if (check("boot")) throw std::runtime_error(g_error);
    if (host_fault) throw std::runtime_error("emulator fault during boot of game " + std::to_string(gh.game));
    build_restart_templates(env, g);
}

template <class F>
void for_each_state(Env& env, F&& f) {
    for (auto& gh : env.games) {
        f(gh.k.recs, sizeof(NesRec) * ((size_t)gh.k.n + 1));
        f(gh.k.keys, (size_t)gh.k.n * gh.k.kcap * 4u);
    }
    const size_t N = (size_t)env.total;
    f(env.e.st, N * sizeof(Rl10State));
    f(env.e.rd, N * sizeof(Rl10Reader));
    f(env.e.drop, N * sizeof(Dropout));
    f(env.e.target, N * 8); f(env.e.ep_frame, N * 4); f(env.e.prev_applied, N * 2); f(env.e.sticky_seed, N * 8);
    f(env.e.sticky_ctr, N * 8); f(env.e.episode, N * 4); f(env.e.ep_ret, N * 4); f(env.e.ep_len, N * 4);
    f(env.e.ep_maxlvl, N * 4); f(env.e.ep_idle, N * 4); f(env.e.fault, N * 4);
    // level starts last, so a state saved without them is a prefix (rl/csrc/rlenv_build.hpp:269-279)
    if (env.lv_cap > 0) {
        f(env.e.ep_start, N * 4);
        for (auto& gh : env.games) {
            const LevelK& L = gh.k.lv;
            const size_t C = (size_t)L.cap;
            f(L.rec, C * sizeof(NesRec));
            f(L.st, C * sizeof(Rl10Saved));
            f(L.keys, C * gh.k.kcap * 4u);
            f(L.target, C * 8); f(L.frame, C * 4); f(L.deaths, C * 4);
        }
    }
}

}  // namespace

// ============================================================================================ C ABI
extern "C" {

void* rlenv_create(int ngames, const int* game_ids, const uint8_t* const* roms, const size_t* rom_sizes,
                   const uint8_t* const* boot_pads, const size_t* boot_sizes, const int* n_envs, uint64_t run_seed,
                   int sticky, int idle_max, int dropout, int device) {
    Env* env = nullptr;
    try {
        if (hipSetDevice(device) != hipSuccess) throw std::runtime_error("hipSetDevice failed");
        env = new Env();
        env->device = device;
        env->scratch = scratch_of(device);
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
            env->one_round = cus * 32;
        if (const char* v = std::getenv("RLENV_BUDGET")) env->budget = (uint32_t)std::max(1, std::min((int)NES_BUDGET, std::atoi(v)));
        env->s.run_seed = run_seed;
        env->s.sticky = sticky;
        env->s.idle_max = idle_max;
        env->s.idle_tmpl = idle_max > 0 ? idle_max : 0;
        env->s.dropout = dropout;
        env->s.episode_level_end = -1;
        env->s.gap_p32 = RLC_GAP_P32;
        uint32_t tab[256];
        build_optab(tab);
        env->optab = static_cast<uint32_t*>(env->mem.alloc(sizeof(tab)));
        env->mem.upload(env->optab, tab, sizeof(tab));
        for (int i = 0; i < ngames; ++i) env->total += n_envs[i];
        const size_t N = (size_t)env->total;
        EnvArrays& e = env->e;
        e.st = env->mem.zeros<Rl10State>(N);
        e.rd = env->mem.zeros<Rl10Reader>(N);
        e.drop = env->mem.zeros<Dropout>(N);
        e.target = env->mem.zeros<uint64_t>(N);
        e.sticky_seed = env->mem.zeros<uint64_t>(N);
        e.sticky_ctr = env->mem.zeros<uint64_t>(N);
        e.ep_frame = env->mem.zeros<uint32_t>(N);
        e.episode = env->mem.zeros<uint32_t>(N);
        {
            std::vector<uint32_t> init(N, 0xFFFFFFFFu);
            env->mem.upload(e.episode, init.data(), N * 4);
        }
        e.fault = env->mem.zeros<uint32_t>(N);
        e.prev_applied = env->mem.zeros<int16_t>(N);
        e.ep_ret = env->mem.zeros<float>(N);
        e.ep_len = env->mem.zeros<int32_t>(N);
        e.ep_maxlvl = env->mem.zeros<int32_t>(N);
        e.ep_idle = env->mem.zeros<int32_t>(N);
        e.resetting = env->mem.zeros<uint8_t>(N);
        // translated kernels (jit.h): by default every game of at least kJitMinEnvs envs (a smaller one gains less
        // than the compile takes), compiled in the background; RLENV_JIT=fixed: only the fixed-PRG games of that
        // size (a banked cart's translation is larger, tens of seconds of compile); sync: every game, compiled
        // before rlenv_create returns; 0 (or off): none
        const char* jv = std::getenv("RLENV_JIT");
        const int jit_mode = !jv ? 2 : (!strcmp(jv, "0") || !strcmp(jv, "off")) ? 0 : !strcmp(jv, "sync") ? 3
                             : !strcmp(jv, "fixed") ? 1 : 2;
        std::vector<std::string> jit_cases((size_t)ngames);
        int offset = 0;
        for (int i = 0; i < ngames; ++i) {
            if (game_ids[i] < 0 || game_ids[i] >= RL10_NUM_GAMES)
                throw std::runtime_error("game id " + std::to_string(game_ids[i]) + ": the reward10 games are 0.." +
                                         std::to_string(RL10_NUM_GAMES - 1));
            const Parsed p = parse_ines(roms[i], rom_sizes[i]);
            GameH gh{};
            gh.game = game_ids[i];
            GameK& g = gh.k;
            g.n = n_envs[i];
            g.offset = offset;
            offset += g.n;
            g.game = game_ids[i];
            g.kcap = rl10_keyset_capacity(g.game);
            g.keys = env->mem.zeros<uint32_t>((size_t)g.n * g.kcap + 1u);
            g.start_ok = rl10_game(g.game).start_ok;   // rl/csrc/reward10_consts.h:25-37
            g.select_ok = rl10_game(g.game).select_ok;
            // widened PRG: word i = bytes i, i+1, i+2 (the instruction window at i); a fixed NROM or CNROM image is
            // widened to 32 KB (a 16 KB one mirrored, as the CPU sees it), so that the fast path (the NROM one for
            // both: CNROM switches only CHR) indexes it by address & $7FFF
            std::vector<uint8_t> img(p.prg);
            const bool fixed32 = p.board == NES_BOARD_NROM || p.board == NES_BOARD_CNROM;   // the NROM fast path
            if (fixed32) {
                img.resize(32768u);
                for (size_t k = p.prg.size(); k < img.size(); ++k) img[k] = p.prg[k % p.prg.size()];
            }
            std::vector<uint32_t> wide(img.size());
            for (size_t k = 0; k < img.size(); ++k) {
                const size_t k1 = std::min(k + 1, img.size() - 1), k2 = std::min(k + 2, img.size() - 1);
                wide[k] = img[k] | ((uint32_t)img[k1] << 8) | ((uint32_t)img[k2] << 16);
            }
            uint32_t* prgw = static_cast<uint32_t*>(env->mem.alloc(wide.size() * 4));
            env->mem.upload(prgw, wide.data(), wide.size() * 4);
            uint8_t* chr = nullptr;
            uint16_t* chr_pairs = nullptr;
            if (!p.chr.empty()) {
                chr = static_cast<uint8_t*>(env->mem.alloc(p.chr.size()));
                env->mem.upload(chr, p.chr.data(), p.chr.size());
                std::vector<uint16_t> pairs(p.chr.size() / 2);   // per 16-byte tile: row r = plane 0 | plane 1 << 8
                for (size_t t = 0; t < p.chr.size(); t += 16)
                    for (size_t r = 0; r < 8; ++r)
                        pairs[t / 2 + r] = (uint16_t)(p.chr[t + r] | (p.chr[t + 8 + r] << 8));
                chr_pairs = static_cast<uint16_t*>(env->mem.alloc(p.chr.size()));
                env->mem.upload(chr_pairs, pairs.data(), p.chr.size());
            }
            uint32_t chr_pages = p.chr.empty() ? 8u : (uint32_t)(p.chr.size() / 1024u);
            if (chr_pages & (chr_pages - 1u)) throw std::runtime_error("CHR size must be a power of two");
            std::vector<uint32_t> f;
            if (fixed32) {   // by CPU address
                f.assign(2u * kFetchWords, 0u);
                for (uint32_t a = 0; a < kFetchWords; ++a) f[2u * a] = 0x02u;
                const size_t mask = (p.prg.size() - 1u) & 0x7FFFu;
                for (uint32_t a = 0x8000u; a <= 0xFFFDu; ++a)
                    fetch_entry(&f[2u * a], a, p.prg[a & mask], p.prg[(a + 1u) & mask], p.prg[(a + 2u) & mask],
                                true);
            } else {   // by PRG offset; $02 where an instruction would end on the last byte of its 8 KB page
                f.assign(2u * p.prg.size(), 0u);
                const auto at = [&](uint32_t k) { return k < p.prg.size() ? (uint32_t)p.prg[k] : 0u; };
                for (uint32_t o = 0; o < p.prg.size(); ++o) {
                    const uint32_t op = p.prg[o];
                    if ((o & 0x1FFFu) + instr_len(kOptab.t[op] & 15u) >= 0x2000u) f[2u * o] = 0x02u;
                    else fetch_entry(&f[2u * o], o, op, at(o + 1u), at(o + 2u), false);
                }
            }
            // the translation, and a fetch table with its blocks' keys (by CPU address, or by PRG offset)
            if (jit_mode == 3 || (jit_mode >= 1 && g.n >= kJitMinEnvs && (fixed32 || jit_mode == 2))) {
                JitProgram jp = fixed32 ? jit_translate_fixed(img) : jit_translate_banked(p.prg, p.board);
                if (!jp.leader_addr.empty()) {
                    std::vector<uint32_t> fj(f);
                    for (size_t b = 0; b < jp.leader_addr.size(); ++b)
                        fj[2u * jp.leader_addr[b]] = kBlockKey + (uint32_t)b;
                    auto js = std::make_shared<JitSlot>();
                    uint32_t* fjw = static_cast<uint32_t*>(env->mem.alloc(fj.size() * 4));
                    env->mem.upload(fjw, fj.data(), fj.size() * 4);
                    js->fetchw = fjw;
                    js->banked = !fixed32;
                    js->blocks = (uint32_t)jp.leader_addr.size();
                    js->instructions = jp.instructions;
                    gh.jit = js;
                    jit_cases[i] = std::move(jp.cases);
                }
            }
            uint32_t* fetchw = static_cast<uint32_t*>(env->mem.alloc(f.size() * 4));
            env->mem.upload(fetchw, f.data(), f.size() * 4);
            g.cart = Cart{prgw, fetchw, chr, (uint32_t)(p.prg.size() / 8192u), chr_pages, p.board, p.mirroring,
                          p.bus_conflicts, chr_pairs};
            g.recs = env->mem.zeros<NesRec>((size_t)g.n + 1);
            g.idle = env->mem.zeros<NesRec>((size_t)std::max(env->s.idle_tmpl, 1));
            const size_t tmpl = (size_t)env->s.idle_tmpl + 1;
            g.rst = env->mem.zeros<NesRec>(tmpl);
            g.rst_obs = env->mem.zeros<uint8_t>(tmpl * RLE_FRAMES * RLE_OBS_PIXELS);
            g.rst_emph = env->mem.zeros<uint8_t>(tmpl * RLE_FRAMES * RLE_OBS_H);
            g.rst_fault = env->mem.zeros<uint32_t>(tmpl);
            for (int b = 0; b < kBankFrames; ++b) {   // (the banks of the frames drawn on the render stream)
                g.bank[b] = env->mem.zeros<FrameBank>((size_t)std::max(g.n, 1));
                g.bank_chr[b] = g.cart.chr ? nullptr : env->mem.zeros<uint8_t>((size_t)g.n * NES_CHRRAM_BYTES);
            }
            g.list = env->mem.zeros<int32_t>((size_t)std::max(g.n, 1));
            g.list_count = env->mem.zeros<uint32_t>(1);
            env->games.push_back(gh);
            boot_game(*env, env->games.back(), boot_pads[i], boot_sizes[i]);
        }
        env->gs.create(env->games.size());
        if (hipDeviceSynchronize() != hipSuccess || check("create")) throw std::runtime_error(g_error);
        // the translations' kernels: queued for the process's compile thread (a translation another env already
        // asked for is not compiled again); with RLENV_JIT=sync compiled and loaded before the env is returned
        for (size_t i = 0; i < env->games.size(); ++i) {
            GameH& gh = env->games[i];
            if (!gh.jit) continue;
            // the variant the decision frames use: drawn from frame banks in a one-game env of one round of waves
            gh.jit->bank = env->games.size() == 1 && gh.k.n <= env->one_round;
            bool is_new = false;
            gh.jit->job = jit_job(std::move(jit_cases[i]), jit_module_source(gh.jit->bank, gh.jit->banked), is_new);
            if (is_new) jit_enqueue(gh.jit->job);
        }
        if (jit_mode == 3)
            for (GameH& gh : env->games)
                if (gh.jit) {
                    while (gh.jit->job->state.load(std::memory_order_acquire) == 0)
                        std::this_thread::sleep_for(std::chrono::milliseconds(5));
                    (void)jit_ready(*env, *gh.jit);
                }
        return env;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        delete env;
        return nullptr;
    }
}

int rlenv_num_envs(void* h) { return static_cast<Env*>(h)->total; }
int rlenv_num_games(void* h) { return (int)static_cast<Env*>(h)->games.size(); }
void rlenv_set_episode_level_end(void* h, int level) { static_cast<Env*>(h)->s.episode_level_end = level; }
void rlenv_set_no_render(void* h, int v) { static_cast<Env*>(h)->s.no_render = v; }
void rlenv_set_pad_mode(void* h, int raw) { static_cast<Env*>(h)->s.pad_mode = raw; }
void rlenv_set_end_prob(void* h, uint32_t p) { static_cast<Env*>(h)->s.end_p32 = p; }
void rlenv_set_dropout_gap(void* h, uint32_t p) { static_cast<Env*>(h)->s.gap_p32 = p; }
void rlenv_bind_ram_hash(void* h, uint64_t* out) { static_cast<Env*>(h)->o.ram_hash = out; }

void rlenv_bind(void* h, const int16_t* actions, uint8_t* obs, uint8_t* emph, float* reward, uint8_t* done,
                uint8_t* masks, uint8_t* tl, uint8_t* pads, uint32_t* events, float* info) {
    Outs& o = static_cast<Env*>(h)->o;
    o.actions = actions; o.obs = obs; o.emph = emph; o.reward = reward; o.done = done; o.masks = masks;
    o.tl = tl; o.pads = pads; o.events = events; o.info = info;
}
void rlenv_bind_parts(void* h, float* parts) { static_cast<Env*>(h)->o.parts = parts; }
void rlenv_bind_obs(void* h, uint8_t* obs, uint8_t* emph) {
    Outs& o = static_cast<Env*>(h)->o;
    o.obs = obs;
    o.emph = emph;
}

int rlenv_start(void* h, void* stream) {
    Env& env = *static_cast<Env*>(h);
    const int bad = for_games(env, static_cast<hipStream_t>(stream), [&](size_t gi, hipStream_t st) {
        const GameK& g = env.games[gi].k;
        const FinishArgs fa = finish_args(env, g, 0, g.n, env.o);
        hipLaunchKernelGGL(k_start, dim3((g.n + 255) / 256), dim3(256), 0, st, fa);
        trace("start", st);
        restart_phases(env, g, env.o, 0, g.n, st);
    });
    return bad ? 1 : check("start");
}

int rlenv_step(void* h, void* stream) {
    Env& env = *static_cast<Env*>(h);
    jit_refresh(env);
    const int bad = for_games(env, static_cast<hipStream_t>(stream), [&](size_t gi, hipStream_t st) {
        decision_phases(env, env.games[gi].k, env.gs.render[gi], env.o, 0, env.games[gi].k.n, st);
    });
    return bad ? 1 : check("step");
}

// (a translation whose compile finished is not loaded here: loading a module allocates; rlenv_step, rlenv_jit_wait
// and rlenv_jit_status load it)
int rlenv_step_static(void* h, void* stream) {
    Env& env = *static_cast<Env*>(h);
    if (env.games.size() > kStaticGames || (uint32_t)env.total > kStaticEnvs) {
        g_error = "step_static: at most " + std::to_string(kStaticGames) + " games and " + std::to_string(kStaticEnvs) +
                  " envs";
        return 1;
    }
    const int bad = for_games(env, static_cast<hipStream_t>(stream), [&](size_t gi, hipStream_t st) {
        GameK g = env.games[gi].k;
        g.list = reinterpret_cast<int32_t*>(env.scratch + kStaticGames + g.offset);
        g.list_count = env.scratch + gi;
        hipLaunchKernelGGL(k_list_clear, dim3(1), dim3(1), 0, st, g.list_count);   // the last call's count
        decision_phases(env, g, env.gs.render[gi], env.o, 0, g.n, st);
    });
    return bad ? 1 : check("step_static");
}

int rlenv_step_game(void* h, int gi, uint8_t* obs, uint8_t* emph, void* stream) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size()) { g_error = "step_game: bad game"; return 1; }
    jit_refresh(env);
    Outs o = env.o;
    o.obs = obs;
    o.emph = emph;
    decision_phases(env, env.games[gi].k, env.gs.render[gi], o, 0, env.games[gi].k.n, static_cast<hipStream_t>(stream));
    return check("step_game");
}

int rlenv_step_range(void* h, int gi, int start, int count, uint8_t* obs, uint8_t* emph, void* stream) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size()) { g_error = "step_range: bad game"; return 1; }
    const GameK& g = env.games[gi].k;
    if (start < 0 || count <= 0 || start + count > g.n) { g_error = "step_range: bad range"; return 1; }
    jit_refresh(env);
    Outs o = env.o;
    o.obs = obs;
    o.emph = emph;
    decision_phases(env, g, env.gs.render[gi], o, start, start + count, static_cast<hipStream_t>(stream));
    return check("step_range");
}

size_t rlenv_state_bytes(void* h) {
    size_t n = 0;
    for_each_state(*static_cast<Env*>(h), [&](void*, size_t b) { n += b; });
    return n;
}

int rlenv_save(void* h, uint8_t* out, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int bad = 0;
    for_each_state(*static_cast<Env*>(h), [&](void* p, size_t b) {
        bad |= hipMemcpyAsync(out, p, b, hipMemcpyDeviceToHost, s) != hipSuccess;
        out += b;
    });
    bad |= hipStreamSynchronize(s) != hipSuccess;
    if (bad) g_error = "save failed";
    return bad;
}

int rlenv_load(void* h, const uint8_t* in, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int bad = 0;
    for_each_state(*static_cast<Env*>(h), [&](void* p, size_t b) {
        bad |= hipMemcpyAsync(p, in, b, hipMemcpyHostToDevice, s) != hipSuccess;
        in += b;
    });
    bad |= hipStreamSynchronize(s) != hipSuccess;
    if (bad) g_error = "load failed";
    return bad;
}

// ---------------------------------------------------------------- level starts / places (rl/csrc/rlenv.cu:300-362)
int rlenv_enable_places(void* h, int cap, int levels) {
    Env& env = *static_cast<Env*>(h);
    if (env.lv_cap != 0 || cap <= 0 || levels <= 0 || levels > cap) {
        g_error = "level starts: enable once, 0 < levels <= cap";
        return 1;
    }
    try {
        for (auto& gh : env.games) {
            LevelK& L = gh.k.lv;
            L.cap = cap;
            L.levels = levels;
            L.rec = env.mem.zeros<NesRec>((size_t)cap);
            L.st = env.mem.zeros<Rl10Saved>((size_t)cap);
            L.keys = env.mem.zeros<uint32_t>((size_t)cap * gh.k.kcap + 1u);
            L.target = env.mem.zeros<uint64_t>((size_t)cap);
            L.frame = env.mem.zeros<uint32_t>((size_t)cap);
            L.deaths = env.mem.zeros<int32_t>((size_t)cap);
            L.claim = env.mem.zeros<unsigned long long>((size_t)cap);
            L.cdf = env.mem.zeros<uint32_t>((size_t)cap);
            const std::vector<int32_t> none((size_t)cap, -1);
            const std::vector<unsigned long long> free_((size_t)cap, ~0ull);
            env.mem.upload(L.deaths, none.data(), (size_t)cap * 4);
            env.mem.upload(L.claim, free_.data(), (size_t)cap * 8);
            L.thresh = 0;
            L.weighted = 0;
        }
        env.e.ep_start = env.mem.zeros<int32_t>((size_t)env.total);
        const std::vector<int32_t> boot((size_t)env.total, -1);
        env.mem.upload(env.e.ep_start, boot.data(), (size_t)env.total * 4);
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return 1;
    }
    env.lv_cap = cap;
    return 0;
}
int rlenv_enable_level_starts(void* h, int cap) { return rlenv_enable_places(h, cap, cap); }
void rlenv_set_level_plan(void* h, int gi, double p, const uint32_t* cdf) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size()) return;
    LevelK& L = env.games[gi].k.lv;
    if (L.cap == 0) return;
    L.thresh = (uint32_t)(p <= 0.0 ? 0.0 : p >= 1.0 ? 4294967295.0 : p * 4294967296.0);
    L.weighted = cdf != nullptr;
    if (cdf) env.mem.upload(L.cdf, cdf, (size_t)L.cap * 4);
}
void rlenv_bind_start(void* h, int32_t* out) { static_cast<Env*>(h)->o.start_out = out; }
void rlenv_bind_level(void* h, int32_t* out) { static_cast<Env*>(h)->o.level_out = out; }
void rlenv_bind_progress(void* h, float* out) { static_cast<Env*>(h)->o.progress_out = out; }
int rlenv_level_deaths(void* h, int gi, int32_t* out, void* stream) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size()) { g_error = "level_deaths: bad game"; return 1; }
    const LevelK& L = env.games[gi].k.lv;
    if (L.cap == 0) return 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(out, L.deaths, (size_t)L.cap * 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        g_error = "level_deaths failed";
        return 1;
    }
    return 0;
}
int rlenv_place_save(void* h, int gi, const int32_t* env_idx, const int32_t* slot_idx, int count, void* stream) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size()) { g_error = "place_save: bad game"; return 1; }
    const GameK& g = env.games[gi].k;
    if (g.lv.cap == 0 || count <= 0) return 0;
    const FinishArgs fa = finish_args(env, g, 0, g.n, env.o);
    hipLaunchKernelGGL(k_place_save, dim3(count), dim3(256), 0, static_cast<hipStream_t>(stream), fa, env_idx, slot_idx);
    return check("place_save");
}
int rlenv_place_copy(void* h, int gi, const int32_t* src, const int32_t* dst, int count, void* stream) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size()) { g_error = "place_copy: bad game"; return 1; }
    const GameK& g = env.games[gi].k;
    const LevelK& L = g.lv;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int bad = 0;
    for (int i = 0; i < count; ++i) {
        if (src[i] < 0 || dst[i] < 0 || src[i] >= L.cap || dst[i] >= L.cap) {
            g_error = "place_copy: bad slot";
            return 1;
        }
        const size_t a = (size_t)src[i], b = (size_t)dst[i];
        const auto d2d = [&](void* to, const void* from, size_t n) {
            bad |= hipMemcpyAsync(to, from, n, hipMemcpyDeviceToDevice, s) != hipSuccess;
        };
        d2d(L.rec + b, L.rec + a, sizeof(NesRec));
        d2d(L.st + b, L.st + a, sizeof(Rl10Saved));
        if (g.kcap) d2d(L.keys + b * g.kcap, L.keys + a * g.kcap, (size_t)g.kcap * 4u);
        d2d(L.target + b, L.target + a, 8);
        d2d(L.frame + b, L.frame + a, 4);
        d2d(L.deaths + b, L.deaths + a, 4);
    }
    bad |= hipStreamSynchronize(s) != hipSuccess;
    if (bad) g_error = "place_copy failed";
    return bad;
}
void rlenv_level_layout(void* h, int gi, uint32_t* out) {
    const Env& env = *static_cast<Env*>(h);
    const LevelK& L = env.games[gi].k.lv;
    out[0] = (uint32_t)sizeof(NesRec);
    out[1] = env.games[gi].k.kcap;   // key words per env (the game's key set)
    out[2] = (uint32_t)sizeof(Rl10Saved);   // tracker + reader per slot
    out[3] = (uint32_t)L.cap;
    out[4] = (uint32_t)L.levels;
}

int rlenv_read_consoles(void* h, int gi, int first, int count, uint8_t* out, void* stream) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size() || first < 0 || count < 0 || first + count > env.games[gi].k.n + 1) {
        g_error = "read_consoles: bad range";
        return 1;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(out, &env.games[gi].k.recs[first], sizeof(NesRec) * (size_t)count, hipMemcpyDeviceToHost, s) !=
            hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        g_error = "read_consoles failed";
        return 1;
    }
    return 0;
}

void rlenv_set_kernel_timing(void* h, int on) { static_cast<Env*>(h)->clock.on = on != 0; }

int rlenv_jit_wait(void* h) {
    Env& env = *static_cast<Env*>(h);
    std::string err;
    for (size_t gi = 0; gi < env.games.size(); ++gi) {
        JitSlot* j = env.games[gi].jit.get();
        if (!j || !j->job) continue;
        while (j->job->state.load(std::memory_order_acquire) == 0)
            std::this_thread::sleep_for(std::chrono::milliseconds(5));
        if (!jit_ready(env, *j))
            err += "game " + std::to_string(gi) + ": " +
                   (j->job->error.empty() ? std::string("loading the translated kernel failed") : j->job->error) + "\n";
    }
    if (!err.empty()) {
        g_error = "jit: " + err;
        return 1;
    }
    return 0;
}

int rlenv_jit_translate(const uint8_t* rom, size_t rom_size, int compile, int32_t* out, char* text, size_t text_cap) {
    try {
        const Parsed p = parse_ines(rom, rom_size);
        const bool fixed32 = p.board == NES_BOARD_NROM || p.board == NES_BOARD_CNROM;
        std::vector<uint8_t> img(32768u);   // a fixed image as the CPU sees it: 16 KB mirrored
        for (size_t k = 0; k < img.size(); ++k) img[k] = p.prg[k % p.prg.size()];
        JitProgram jp = fixed32 ? jit_translate_fixed(img) : jit_translate_banked(p.prg, p.board);
        out[0] = (int32_t)jp.leader_addr.size();
        out[1] = (int32_t)jp.instructions;
        out[2] = -1;
        out[3] = 0;
        out[4] = 0;
        out[5] = 0;
        if (text && text_cap) {
            const size_t n = std::min(text_cap - 1, jp.cases.size());
            memcpy(text, jp.cases.data(), n);
            text[n] = 0;
        }
        if (compile) {
            JitJob job;
            job.blocks = std::move(jp.cases);
            job.source = jit_module_source(compile >= 2, !fixed32);   // 2: with the frame-bank kernel
            jit_compile(job);
            out[2] = (int32_t)(job.seconds * 1000.0);
            out[3] = (int32_t)job.code.size();
            out[4] = job.far_jumps;
            out[5] = job.hazards;
            if (job.state.load() != 1) {
                g_error = job.error;
                return 1;
            }
        }
        return 0;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return 1;
    }
}

int rlenv_jit_check(const char* code, size_t size, int32_t* out, char* where, size_t where_cap) {
    const std::vector<char> co(code, code + size);
    std::string w;
    int far = 0;
    out[1] = jit_far_branch_hazards(co, &far, &w);
    out[0] = far;
    if (where && where_cap) {
        const size_t n = std::min(where_cap - 1, w.size());
        memcpy(where, w.data(), n);
        where[n] = 0;
    }
    return 0;
}

int rlenv_jit_status(void* h, int gi, int32_t* out) {
    Env& env = *static_cast<Env*>(h);
    if (gi < 0 || gi >= (int)env.games.size()) { g_error = "jit_status: bad game"; return 1; }
    JitSlot* j = env.games[gi].jit.get();
    if (j && !j->fn_draw && !j->failed) (void)jit_ready(env, *j);
    const int st = !j ? 0 : j->fn_draw ? 2 : (j->failed || (j->job && j->job->state.load() == 2)) ? 3 : 1;
    out[0] = st;
    out[1] = j ? (int32_t)j->blocks : 0;
    out[2] = j ? (int32_t)j->instructions : 0;
    out[3] = j && j->job && j->job->state.load() != 0 ? (int32_t)(j->job->seconds * 1000.0) : -1;
    out[4] = (j && j->bank ? 1 : 0) | (j && j->banked ? 2 : 0);
    out[5] = j && j->job && j->job->state.load() != 0 ? j->job->far_jumps : -1;
    return 0;
}

int rlenv_kernel_times(void* h, double* ms, int64_t* count, int n) {
    if (n < KC_COUNT) { g_error = "kernel_times: need room for every kernel class (10)"; return 1; }
    for (int i = 0; i < n; ++i) { ms[i] = 0.0; count[i] = 0; }
    if (static_cast<Env*>(h)->clock.drain(ms, count)) { g_error = "kernel_times: event query failed"; return 1; }
    return 0;
}

const char* rlenv_error(void) { return g_error.c_str(); }
void rlenv_destroy(void* h) { delete static_cast<Env*>(h); }

void* rl_host_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocPortable) != hipSuccess) {
        g_error = "hipHostMalloc failed";
        return nullptr;
    }
    return p;
}
void rl_host_free(void* p) { (void)hipHostFree(p); }

int rl_pack6(const void* src, void* dst, size_t pixels, void* stream) {
    if (pixels % 4) { g_error = "pack6: pixel count must be divisible by four"; return 1; }
    const size_t groups = pixels / 4, threads = (groups + 3) / 4;
    if (groups)
        hipLaunchKernelGGL(k_pack6, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), groups);
    return check("pack6");
}
int rl_unpack6(const void* src, void* dst, size_t pixels, void* stream) {
    if (pixels % 4) { g_error = "unpack6: pixel count must be divisible by four"; return 1; }
    const size_t groups = pixels / 4, threads = (groups + 3) / 4;
    if (groups)
        hipLaunchKernelGGL(k_unpack6, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), groups);
    return check("unpack6");
}
int rl_memcpy_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, static_cast<hipStream_t>(stream)) != hipSuccess)
        return check("memcpy");
    return 0;
}
int rl_gather_rows(void* dst, const void* src, const int64_t* rows, int nrows, size_t row_bytes, void* stream) {
    if (row_bytes % 16) { g_error = "gather_rows: row bytes must be a multiple of 16"; return 1; }
    if (nrows > 0)
        hipLaunchKernelGGL(k_gather_rows, dim3(nrows, 32), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<uint4*>(dst), static_cast<const uint4*>(src), rows, row_bytes / 16);
    return check("gather");
}
int rl_gather_envs(void* dst, const void* src, const int64_t* envs, int n, int T, int N, size_t row_bytes, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int j = 0; j < n; ++j) {
        if (hipMemcpy2DAsync(static_cast<char*>(dst) + (size_t)j * row_bytes, (size_t)n * row_bytes,
                             static_cast<const char*>(src) + (size_t)envs[j] * row_bytes, (size_t)N * row_bytes,
                             row_bytes, (size_t)T, hipMemcpyDefault, s) != hipSuccess)
            return check("gather2d");
    }
    return 0;
}

int rl_stream_create(void** stream) {
    hipStream_t s = nullptr;
    if (!stream) { g_error = "stream_create: null output"; return 1; }
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        g_error = std::string("stream_create: ") + hipGetErrorString(e);
        return 1;
    }
    *stream = s;
    return 0;
}
int rl_stream_destroy(void* stream) {
    if (!stream) { g_error = "stream_destroy: null stream"; return 1; }
    const hipError_t e = hipStreamDestroy(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        g_error = std::string("stream_destroy: ") + hipGetErrorString(e);
        return 1;
    }
    return 0;
}

int rl10_smb_run(const uint8_t* ram15, int T, int N, int frames, void* state, float* reward, uint8_t* done,
                 void* stream) {
    if (N <= 0 || T <= 0) return check("rl10_smb_run");
    try {
        const hipStream_t st = static_cast<hipStream_t>(stream);
        int device = 0;
        if (hipGetDevice(&device) != hipSuccess) throw std::runtime_error("hipGetDevice failed");
        const size_t n = (size_t)T * (size_t)N;
        void* rec = nullptr;   // (kAhead rows past the last: k_smb_chain's last loads)
        if (hipMallocFromPoolAsync(&rec, (n + (size_t)kAhead * (size_t)N) * sizeof(ev::SmbStep), smb_pool(device), st) !=
            hipSuccess)
            throw std::runtime_error("rl10_smb_run: no device memory for the per-step records");
        const size_t groups = (size_t)((T + 3) / 4) * (size_t)N;
        hipLaunchKernelGGL(k_smb_signals, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, ram15, T, N,
                           static_cast<const Rl10State*>(state), static_cast<ev::SmbStep*>(rec));
        hipLaunchKernelGGL(k_smb_chain, dim3((N + 63) / 64), dim3(64), 0, st, static_cast<ev::SmbStep*>(rec), ram15, T,
                           N, frames, static_cast<Rl10State*>(state));
        hipLaunchKernelGGL(k_smb_reward, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           static_cast<const ev::SmbDec*>(rec), n, frames, reward, done);
        const int bad = check("rl10_smb_run");
        (void)hipFreeAsync(rec, st);
        return bad;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return 1;
    }
}

int rl10_run(int game, const uint8_t* ram, int T, int N, const int32_t* frames, void* state, void* reader,
             uint32_t* keys, double* reward, uint8_t* done, uint32_t* events, int32_t* event_level, int32_t* deaths,
             uint8_t* end_reason, void* stream) {
    if (game < 0 || game >= RL10_NUM_GAMES || T < 0 || N < 0 || (N > 0 && T > 0 && (!ram || !frames || !state ||
        !reader || (rl10_keyset_capacity(game) > 0 && !keys)))) {
        g_error = "rl10_run: bad game id, size or buffer";
        return 1;
    }
    if (N > 0 && T > 0) {
        const Rl10RunArgs a{ram, frames, static_cast<Rl10State*>(state), static_cast<Rl10Reader*>(reader), keys,
                            reward, done, end_reason, events, event_level, deaths, game, T, N,
                            rl10_keyset_capacity(game)};
        hipLaunchKernelGGL(k_rl10_run, dim3((N + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), a);
    }
    return check("rl10_run");
}

}  // extern "C"
