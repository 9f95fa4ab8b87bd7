/* C ABI of the batched NES environment step (HIP build: ghostrun-lab_amd/csrc -> librlenv_hip.so).
 *
 * A drop-in for the reference's rl/csrc/rlenv_api.h:8-47 and the GPU extras of rl/csrc/rlenv.cu:186-427: the
 * same names, argument meanings and error behaviour, so rl/rlenv.py's ctypes loader (rl/rlenv.py:76-121) binds
 * it unchanged. All buffers are device pointers; `stream` is a hipStream_t passed as void* (torch's current
 * stream). Plain C types only. The CPU oracle (oracle/) exports the same entry points for tests, with host
 * pointers, ignoring `stream`.
 *
 * Errors: int 0 = ok, non-zero = error with the message in rlenv_error(); rlenv_create returns NULL on error.
 * Emulator faults are data (episode end 5), not errors.
 */
#ifndef RLENV_API_H
#define RLENV_API_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Builds every game's boot snapshot (power-on, RAM 0xFF, the boot pad bytes frame by frame) and idle
 * templates, and allocates n+1 console records per game (slot n = boot snapshot).
 * Replaces rl/csrc/rlenv_api.h:10-12 (rlenv.cu:188-217). game_ids: reward10 game ids 0..11 (smb, pacman,
 * excitebike, contra, castlevania, gradius, zelda, tetris, tecmobowl, kage, finalmission, punchout; the order of
 * rl/games_manifest.json), each choosing the reward reader and the Start/Select legality. roms: iNES images
 * (mappers 0-4 and 9). device: HIP device index. */
void* rlenv_create(int ngames, const int* game_ids, const uint8_t* const* roms, const size_t* rom_sizes,
                   const uint8_t* const* boot_pads, const size_t* boot_sizes, const int* n_envs, uint64_t run_seed,
                   int sticky, int idle_max, int dropout, int device);
int rlenv_num_envs(void* h);                                   /* rlenv_api.h:13 */
void rlenv_set_episode_level_end(void* h, int level);          /* rlenv_api.h:15 */
/* rlenv_api.h:16-18: actions int16 [N], obs u8 [N,4,224,240], emph u8 [N,4,224], reward f32 [N], done u8 [N],
 * masks u8 [N,19], timeline u8 [N,8,45], pads u8 [N,4], events u32 [N], info f32 [N,8]. */
void rlenv_bind(void* h, const int16_t* actions, uint8_t* obs, uint8_t* emph, float* reward, uint8_t* done,
                uint8_t* masks, uint8_t* timeline, uint8_t* pads, uint32_t* events, float* info);
void rlenv_bind_parts(void* h, float* parts);                  /* rlenv_api.h:20: [N,7] */
void rlenv_bind_obs(void* h, uint8_t* obs, uint8_t* emph);     /* rlenv_api.h:22 */
/* Level starts and places (rlenv_api.h:22-39; rl/csrc/rlenv_core.cuh:14-20). enable: room for `cap` saved starts
 * per game, the first `levels` of them level starts (saved on the tracker's level event, the arrival with the fewest
 * deaths kept, the newest on ties), the rest places (saved by place_save); call once, before start/load; error if
 * called twice or 0 < levels <= cap does not hold. set_level_plan: game gi's chance p that a new episode starts from
 * a saved slot, and its cumulative slot weights * 2^32 (cap entries; NULL = uniform over the saved slots); call
 * between decisions. bind_start/level/progress: outputs [N] int32 start slot of a finished episode (-1 = boot
 * snapshot; valid where done), [N] int32 level after each decision (-1 = unknown), [N] float within-level progress /
 * progress unit (NaN = not valid). level_deaths: deaths of game gi's saves (-1 = empty), cap entries, to host memory
 * (synchronous). place_save: env_idx[j] (index within game gi) -> slot_idx[j] (skipped where < levels), device
 * arrays, on `stream` after a step. place_copy: slot src[j] -> dst[j], host arrays, synchronous. level_layout: out[5]
 * = bytes of one saved console, key words per env, bytes of one slot's tracker state (sizeof(Rl10Saved): the tracker and
 * its game reader), cap, levels. */
int rlenv_enable_level_starts(void* h, int cap);                                       /* rlenv_api.h:26 */
int rlenv_enable_places(void* h, int cap, int levels);                                 /* rlenv_api.h:36 */
void rlenv_set_level_plan(void* h, int gi, double p, const uint32_t* cdf);             /* rlenv_api.h:27 */
void rlenv_bind_start(void* h, int32_t* start_out);                                    /* rlenv_api.h:28 */
void rlenv_bind_level(void* h, int32_t* level_out);                                    /* rlenv_api.h:29 */
void rlenv_bind_progress(void* h, float* progress_out);                                /* rlenv_api.h:30 */
int rlenv_level_deaths(void* h, int gi, int32_t* host_out, void* stream);              /* rlenv_api.h:31 */
int rlenv_place_save(void* h, int gi, const int32_t* env_idx, const int32_t* slot_idx, int count,
                     void* stream);                                                    /* rlenv_api.h:37 */
int rlenv_place_copy(void* h, int gi, const int32_t* src, const int32_t* dst, int count,
                     void* stream);                                                    /* rlenv_api.h:38 */
void rlenv_level_layout(void* h, int gi, uint32_t* out);                               /* rlenv_api.h:39 */
int rlenv_start(void* h, void* stream);                        /* rlenv_api.h:40 */
int rlenv_step(void* h, void* stream);                         /* rlenv_api.h:41 */
size_t rlenv_state_bytes(void* h);                             /* rlenv_api.h:42 */
int rlenv_save(void* h, uint8_t* host_out, void* stream);      /* rlenv_api.h:43 (synchronous) */
int rlenv_load(void* h, const uint8_t* host_in, void* stream); /* rlenv_api.h:44 (synchronous) */
const char* rlenv_error(void);                                 /* rlenv_api.h:45 (thread-local) */
void rlenv_destroy(void* h);                                   /* rlenv_api.h:46 */

/* GPU extras of rl/csrc/rlenv.cu. */
int rlenv_num_games(void* h);                                                      /* rlenv.cu:249 */
int rlenv_step_game(void* h, int gi, uint8_t* obs, uint8_t* emph, void* stream);    /* rlenv.cu:250-256 */
int rlenv_step_range(void* h, int gi, int start, int count, uint8_t* obs, uint8_t* emph,
                     void* stream);                                                /* rlenv.cu:258-268 */
void rlenv_set_no_render(void* h, int v);                                          /* rlenv.cu:364-366 */
void* rl_host_alloc(size_t bytes);                                                 /* rlenv.cu:371-378 */
void rl_host_free(void* p);                                                        /* rlenv.cu:379 */
int rl_pack6(const void* src, void* dst, size_t pixels, void* stream);             /* rlenv.cu:380-386 */
int rl_unpack6(const void* src, void* dst, size_t pixels, void* stream);           /* rlenv.cu:387-393 */
int rl_memcpy_async(void* dst, const void* src, size_t bytes, void* stream);       /* rlenv.cu:394-398 */
int rl_gather_rows(void* dst, const void* src, const int64_t* rows, int nrows, size_t row_bytes,
                   void* stream);                                                  /* rlenv.cu:400-409 */
int rl_gather_envs(void* dst, const void* src, const int64_t* envs, int n, int T, int N, size_t row_bytes,
                   void* stream);                                                  /* rlenv.cu:411-421 */
/* Streams for the rollout store's copies (no reference counterpart; the reference trainer's streams are torch's):
 * a stream at the default priority that does not wait for the null stream, and its release. torch's own streams
 * are never destroyed, and the runtime spreads streams over its hardware queues by how many each already serves, so
 * a store whose streams outlive it changes where every later stream of the process runs. */
int rl_stream_create(void** stream);
int rl_stream_destroy(void* stream);

/* Additions of this build for the benchmark workloads (no reference counterpart):
 *  pad mode 1: actions hold raw pad bytes (0..255) instead of move ids; sticky repeats the previous frame's
 *    byte; a dropped input clears its button bit.
 *  end_p32: per decision, an episode also ends with probability end_p32 / 2^32 (end reason 7), drawn from
 *    the env's own counter stream (seed of the episode, decision index).
 *  gap_p32: P(a healthy dropout gap ends) per decision, default floor(2^32/35) as the reference's kGapP32.
 *  ram hash: u64 [N], per decision the hash of the console's 2 KB RAM after its 4 frames.
 *  read_consoles: console records (include/nesrec.h) of game gi, envs [first, first+count), to host memory
 *    (synchronous). */
void rlenv_set_pad_mode(void* h, int raw);
void rlenv_set_end_prob(void* h, uint32_t end_p32);
void rlenv_set_dropout_gap(void* h, uint32_t gap_p32);
void rlenv_bind_ram_hash(void* h, uint64_t* ram_hash);
int rlenv_read_consoles(void* h, int gi, int first, int count, uint8_t* host_out, void* stream);
/* Per-kernel clock (no reference counterpart; the measurement harness reads it): when on, every launch of a
 * start/step is bracketed by two HIP events on its stream. rlenv_kernel_times waits for the recorded launches,
 * writes the summed milliseconds and launch counts per kernel class into ms[n] / count[n] (n >= 10; classes:
 * 0 emu (decision frames drawn by another kernel, from frame banks), 1 render, 2 finish, 3 reset_copy, 4 emu_restart,
 * 5 render_restart, 6 reset_finish, 7 emu_idle (idle frames of level starts), 8 archive (level-start saves), 9
 * emu_draw (decision frames emulated and drawn by the same waves, the decision's last one with its finish)) and
 * forgets them. */
void rlenv_set_kernel_timing(void* h, int on);
int rlenv_kernel_times(void* h, double* ms, int64_t* count, int n);
/* Translated kernels (no reference counterpart: an acceleration inside this library). rlenv_create translates the
 * cart's 6502 code into blocks of the interpreter's per-opcode handlers with constant operands (by CPU address on
 * NROM and CNROM, by PRG offset on the banked boards) and compiles them at run time (hiprtc; the games' compiles in
 * parallel, each translation once per process) into a copy of the console-frame kernel that the game's decision
 * frames then use; a console's results are the same on either kernel. Which games: by default every game of at least
 * 1024 envs; RLENV_JIT=fixed: only the fixed-PRG games of that size; RLENV_JIT=sync: every game; RLENV_JIT=0 (or off):
 * none. The compiles run on one thread of the process, one at a time, in the order asked for, while rlenv_create
 * returns at once (RLENV_JIT=sync: after them); a game's decision frames switch to its translated kernel at the first
 * rlenv_step, rlenv_step_game, rlenv_step_range, rlenv_jit_wait or rlenv_jit_status after its compile (never in the
 * middle of a decision; rlenv_step_static allocates nothing and so loads nothing). A compiled code object is used
 * only if it holds no far jump into live SCC (a compiler fault, see rlenv_jit_check); else that game keeps the
 * library's kernel. RLENV_JIT_CACHE=<directory>: compiled code objects are also kept there, for later processes.
 * RLENV_JIT_EXTRA: further compile options, separated by spaces (diagnostics).
 *  jit_wait: waits for the env's compiles; 0 when every translated game runs translated decision frames (those drawn
 *    the way its translation was built for: from frame banks in a one-game env of one round of waves, from the
 *    records otherwise); non-zero, with the compile error in rlenv_error, when a compile, its check or its load
 *    failed (that game keeps the library's own kernel).
 *  jit_status: out[6] = state (0 no translation, 1 compiling, 2 loaded, 3 failed), blocks, instructions, compile
 *    milliseconds (-1 while compiling), flags (1: built for frames drawn from frame banks, 2: a banked-PRG
 *    translation, whose blocks are keyed by their PRG bank too), far jumps in the code object (-1 while compiling).
 *  jit_translate: the translation of an iNES image (needs no GPU): out[6] = blocks, instructions, compile
 *    milliseconds, code-object bytes, far jumps and far jumps into live SCC (-1 and 0s without compile); text (if
 *    not null): the generated blocks, NUL-terminated, cut at text_cap. compile: 0 none, 1 the kernel of decision
 *    frames drawn by the emulator's waves (the variant of several games or several rounds of waves), 2 with the
 *    frame-bank kernel too (a one-game env of one round of waves); with RLENV_JIT_CACHE the code object is kept there
 *    as rlenv_create would keep it, so a later create finds it. Non-zero for an image that does not parse, a failed
 *    compile or a code object that fails the check.
 *  jit_check: the far-jump check of a gfx950 code object (an ELF as hiprtc returns it): a branch too far for its
 *    16-bit offset is compiled to s_getpc_b64 / s_add_u32 / s_addc_u32 / s_setpc_b64, whose adds overwrite SCC,
 *    and the compiler does not make sure that the code at the target does not read SCC first. out[2] = far jumps,
 *    those whose target reads SCC before writing it (-1: not a code object it can disassemble); where (if not
 *    null): the first such target, NUL-terminated. */
int rlenv_jit_wait(void* h);
int rlenv_jit_status(void* h, int gi, int32_t* out);
int rlenv_jit_translate(const uint8_t* rom, size_t rom_size, int compile, int32_t* out, char* text, size_t text_cap);
int rlenv_jit_check(const char* code, size_t size, int32_t* out, char* where, size_t where_cap);

/* The reward10 SMB tracker on its own (benchmark config "reward10 standalone"): T steps of N envs.
 * ram15: u8 [T, N, 16], per env-step the 15 RAM bytes the SMB reader reads, in the order
 *   0x0E, 0x6D, 0x86, 0xB5, 0x75A, 0x75C, 0x75F, 0x770, 0x772, 0x7DD..0x7E2 (byte 15 unused);
 * state: Rl10State [N] (include/rlenv_state.h), updated in place; reward f32 [T, N]; done u8 [T, N].
 * frames = emulated frames per step. Follows rl/csrc/host_api.cpp:13-31 (rl10_replay) for game smb. */
int rl10_smb_run(const uint8_t* ram15, int T, int N, int frames, void* state, float* reward, uint8_t* done,
                 void* stream);

/* The reward10 tracker of any game (ids as in rlenv_create) on device RAM: T steps of N envs, one env per thread.
 * ram: u8 [T, N, 2048] device, the 2 KB RAM of each env-step; frames: i32 [T, N] emulated frames per step;
 * state: Rl10State [N], reader: Rl10Reader [N] (include/rlenv_state.h) and keys: u32 [N * cap], cap =
 * rl10_keyset_capacity(game) (include/rl10_games.h; keys may be null when it is 0), all zeroed for a fresh env and
 * updated in place; a key set that fills sets state.overflow, as rl10_replay's nonzero return.
 * Outputs [T, N]: reward f64, done u8, events u32, event_level i32, deaths i32 and end_reason u8 (the tracker's
 * after each step; any output may be null). Follows rl/csrc/host_api.cpp:13-31 (rl10_replay) for N envs at once. */
int rl10_run(int game, const uint8_t* ram, int T, int N, const int32_t* frames, void* state, void* reader,
             uint32_t* keys, double* reward, uint8_t* done, uint32_t* events, int32_t* event_level, int32_t* deaths,
             uint8_t* end_reason, void* stream);

/* rlenv_step with every game's restart queue (the indices of the envs whose episode ended this decision, and their
 * count) in the library's static device scratch instead of the buffers rlenv_create allocated for it: the call
 * allocates nothing (no hipMalloc, hipFree or allocating library routine). No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Limits: at most 64 games and 262,144 envs per env (larger envs are refused with an error). Every
 * call on one GPU shares that GPU's scratch, so calls that overlap on one GPU (two streams, two envs) race. */
int rlenv_step_static(void* h, void* stream);

#ifdef __cplusplus
}
#endif
#endif
