"""`RlEnv`: the Python face of the batched NES environment step on one GPU, a drop-in for the reference's
rl/rlenv.py:172-389 (constructor arguments, bound tensors with their shapes and dtypes, method names and what they
do), over this repository's HIP library `librlenv_hip.so` (C ABI: include/rlenv_api.h).

    env = RlEnv({'smb': 8192}, device='cuda', seed=1, roms={'smb': cart_bytes})
    env.start()                       # pictures of the first decision, legal parts in env.masks
    env.actions.copy_(moves)          # int16 move ids (or raw pad bytes with pad_mode=True)
    env.step()                        # every bound output rewritten in place, on torch's current stream

How it is put together:
  * `bind_library` attaches ctypes signatures to a library from one table (`_ABI`); entries marked optional are
    bound only where the library exports them (the CPU oracle has no host-memory helpers).
  * The outputs are allocated from one spec table (`_OUTPUTS`) on the env's device and handed to the library once;
    the library writes into them on every call. Nothing is copied to the host per decision.
  * Every library call goes through `_check`, which turns a non-zero return into a RuntimeError carrying
    `rlenv_error()`.

On a GPU device the HIP library is the only implementation: it must be built (`python __graft_entry__.py`), and a
missing build is an error. `device='cpu'` needs `lib_path` to a library with the same C ABI (the tests pass the CPU
oracle's).

Keyword arguments beyond the reference's: ``roms`` may hold iNES bytes; ``boot`` maps a game to its boot pad bytes
(default none: the episode starts at power-on); ``pad_mode`` makes actions raw pad bytes; ``end_prob`` adds a
Geometric episode end per decision (end reason 7); ``dropout_gap`` sets P(a dropout gap ends) per decision;
``ram_hash`` binds a per-decision hash of each console's RAM.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np
import torch

PKG = Path(__file__).resolve().parents[1]          # ghostrun-lab_amd/
HIP_LIB = Path(os.environ.get('RL_HIP_LIB', PKG / 'csrc' / '_build' / 'librlenv_hip.so'))

# The twelve games in reward10 id order (rl/games_manifest.json; rl/rlenv.py:30-31).
GAMES = ['smb', 'pacman', 'excitebike', 'contra', 'castlevania', 'gradius', 'zelda', 'tetris', 'tecmobowl', 'kage',
         'finalmission', 'punchout']
OBS_H, OBS_W, FRAMES = 224, 240, 4
FRAME_BYTES = FRAMES * OBS_H * OBS_W
MASK_BYTES, TIMELINE, INFO = 19, 8 * 45, 8
PART_NAMES = ('progress', 'level', 'death', 'damage', 'score', 'win', 'stall')   # columns of env.parts
NUM_PARTS = len(PART_NAMES)
END_NAMES = {0: 'none', 1: 'game_over', 2: 'won', 3: 'skip', 4: 'stall', 5: 'fault', 6: 'level_clear', 7: 'synthetic'}
NES_REC_BYTES = 23552   # one console record, include/nesrec.h

_P, _I, _U32, _U64, _SZ, _F64 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t,
                                 ctypes.c_double)
_VOID = None
# name: (restype, argtypes, optional). Entry points returning int return 0, or non-zero with rlenv_error() set.
_ABI = {
    'rlenv_create': (_P, [_I, _P, _P, _P, _P, _P, _P, _U64, _I, _I, _I, _I], False),
    'rlenv_destroy': (_VOID, [_P], False),
    'rlenv_error': (ctypes.c_char_p, [], False),
    'rlenv_num_envs': (_I, [_P], False),
    'rlenv_num_games': (_I, [_P], False),
    'rlenv_bind': (_VOID, [_P] * 11, False),
    'rlenv_bind_parts': (_VOID, [_P, _P], False),
    'rlenv_bind_obs': (_VOID, [_P, _P, _P], False),
    'rlenv_start': (_I, [_P, _P], False),
    'rlenv_step': (_I, [_P, _P], False),
    'rlenv_state_bytes': (_SZ, [_P], False),
    'rlenv_save': (_I, [_P, _P, _P], False),
    'rlenv_load': (_I, [_P, _P, _P], False),
    'rlenv_set_episode_level_end': (_VOID, [_P, _I], False),
    'rlenv_set_no_render': (_VOID, [_P, _I], False),
    'rlenv_enable_level_starts': (_I, [_P, _I], False),
    'rlenv_enable_places': (_I, [_P, _I, _I], False),
    'rlenv_set_level_plan': (_VOID, [_P, _I, _F64, _P], False),
    'rlenv_bind_start': (_VOID, [_P, _P], False),
    'rlenv_bind_level': (_VOID, [_P, _P], False),
    'rlenv_bind_progress': (_VOID, [_P, _P], False),
    'rlenv_level_deaths': (_I, [_P, _I, _P, _P], False),
    'rlenv_place_save': (_I, [_P, _I, _P, _P, _I, _P], False),
    'rlenv_place_copy': (_I, [_P, _I, _P, _P, _I, _P], False),
    'rlenv_level_layout': (_VOID, [_P, _I, _P], False),
    'rlenv_set_pad_mode': (_VOID, [_P, _I], False),
    'rlenv_set_end_prob': (_VOID, [_P, _U32], False),
    'rlenv_set_dropout_gap': (_VOID, [_P, _U32], False),
    'rlenv_bind_ram_hash': (_VOID, [_P, _P], False),
    'rlenv_read_consoles': (_I, [_P, _I, _I, _I, _P, _P], False),
    'rl_pack6': (_I, [_P, _P, _SZ, _P], False),
    'rl_unpack6': (_I, [_P, _P, _SZ, _P], False),
    'rl10_smb_run': (_I, [_P, _I, _I, _I, _P, _P, _P, _P], False),
    'rl10_run': (_I, [_I, _P, _I, _I] + [_P] * 11, False),
    'rlenv_step_game': (_I, [_P, _I, _P, _P, _P], True),
    'rlenv_step_range': (_I, [_P, _I, _I, _I, _P, _P, _P], True),
    'rlenv_step_static': (_I, [_P, _P], True),
    'rlenv_jit_wait': (_I, [_P], True),
    'rlenv_jit_status': (_I, [_P, _I, _P], True),
    'rlenv_jit_translate': (_I, [_P, _SZ, _I, _P, _P, _SZ], True),
    'rlenv_jit_check': (_I, [_P, _SZ, _P, _P, _SZ], True),
    'rl_host_alloc': (_P, [_SZ], True),
    'rl_host_free': (_VOID, [_P], True),
    'rl_memcpy_async': (_I, [_P, _P, _SZ, _P], True),
    'rl_gather_rows': (_I, [_P, _P, _P, _I, _SZ, _P], True),
    'rl_gather_envs': (_I, [_P, _P, _P, _I, _I, _I, _SZ, _P], True),
    'rl_stream_create': (_I, [_P], True),
    'rl_stream_destroy': (_I, [_P], True),
}


def bind_library(path) -> ctypes.CDLL:
    """Load a library with the env's C ABI and attach the signatures of `_ABI` (the bindings of the reference's
    rl/rlenv.py:76-121, plus this library's additions)."""
    lib = ctypes.CDLL(str(path))
    for name, (res, args, optional) in _ABI.items():
        if optional and not hasattr(lib, name):
            continue
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def hip_library() -> Path:
    """The built HIP library; an error when it is missing (there is no other GPU implementation)."""
    if not HIP_LIB.exists():
        raise RuntimeError(f'{HIP_LIB} is not built: run `python __graft_entry__.py` (the HIP build) first')
    return HIP_LIB


def _addr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _carray(ctype, values):
    return (ctype * len(values))(*values)


# Bound outputs: attribute, per-env shape, dtype, in rlenv_bind's argument order after `actions`
# (include/rlenv_api.h; rl/rlenv.py:208-220).
_OUTPUTS = (('obs', (FRAMES, OBS_H, OBS_W), torch.uint8), ('emph', (FRAMES, OBS_H), torch.uint8),
            ('reward', (), torch.float32), ('done', (), torch.uint8), ('masks', (MASK_BYTES,), torch.uint8),
            ('timeline', (8, 45), torch.uint8), ('pads', (FRAMES,), torch.uint8), ('events', (), torch.int32),
            ('info', (INFO,), torch.float32))

# Per-slot widths of the archive tail of a state blob, per game (rl/csrc/rlenv_build.hpp:269-279): a saved console,
# its tracker block (level_layout 'st'), its key words, target, frame and deaths. Empty slots hold zeros, except
# deaths, which hold -1.
_TAIL_FILL = (0, 0, 0, 0, 0, 0xFF)


class RlEnv:
    def __init__(self, counts: dict, device='cuda', seed=0, sticky=True, idle_max=30, dropout=True, roms=None,
                 lib_path=None, level_cap=0, level_slots=None, boot=None, pad_mode=False, end_prob=0.0,
                 dropout_gap=None, ram_hash=False):
        """counts: game slug -> number of envs; the envs of the games are laid out in GAMES order. roms: slug ->
        iNES bytes or a path. level_cap > 0 keeps a per-game archive of level starts (slots 0..level_cap-1); new
        episodes begin from it with the chance set_level_prob / set_level_plan give (0 until set). With level_slots
        below level_cap, slots level_slots..level_cap-1 are places, filled by place_save. start_level: the slot the
        episode that just ended began from (-1 = the boot snapshot; read where done). level_now / progress_now: the
        level and within-level progress after each decision."""
        self.device = torch.device(device)
        self.games = [g for g in GAMES if counts.get(g, 0) > 0]
        self.counts = [int(counts[g]) for g in self.games]
        self.n = sum(self.counts)
        self.game_of_env = torch.repeat_interleave(torch.tensor([GAMES.index(g) for g in self.games], dtype=torch.long),
                                                   torch.tensor(self.counts)).to(self.device)
        on_gpu = self.device.type == 'cuda'
        if lib_path is None and not on_gpu:
            raise RuntimeError("device='cpu' needs lib_path (a CPU library with the same C ABI)")
        self.lib_path = Path(lib_path) if lib_path is not None else hip_library()
        self.lib = bind_library(self.lib_path)
        self.h = None
        self.h = self._create(roms or {}, boot or {}, seed, sticky, idle_max, dropout, on_gpu)

        N, dev = self.n, self.device
        self.actions = torch.zeros(N, dtype=torch.int16, device=dev)
        for name, shape, dtype in _OUTPUTS:
            setattr(self, name, torch.zeros((N,) + shape, dtype=dtype, device=dev))
        self.lib.rlenv_bind(self.h, _addr(self.actions), *(_addr(getattr(self, o[0])) for o in _OUTPUTS))
        self.parts = torch.zeros(N, NUM_PARTS, dtype=torch.float32, device=dev)   # the reward split by source
        self.lib.rlenv_bind_parts(self.h, _addr(self.parts))

        self.level_cap = int(level_cap)
        self.level_slots = self.level_cap if level_slots is None else int(level_slots)
        self.start_level = torch.full((N,), -1, dtype=torch.int32, device=dev)
        if self.level_cap > 0:
            self._enable_archive()
        self.lib.rlenv_set_pad_mode(self.h, int(bool(pad_mode)))
        if end_prob:
            self.lib.rlenv_set_end_prob(self.h, self._p32(end_prob))
        if dropout_gap is not None:
            self.lib.rlenv_set_dropout_gap(self.h, self._p32(dropout_gap))
        self.ram_hash = torch.zeros(N, dtype=torch.int64, device=dev) if ram_hash else None
        if ram_hash:
            self.lib.rlenv_bind_ram_hash(self.h, _addr(self.ram_hash))

    # ------------------------------------------------------------------ construction
    def _create(self, roms, boot, seed, sticky, idle_max, dropout, on_gpu):
        absent = [g for g in self.games if g not in roms]
        if absent:
            raise RuntimeError(f'no ROM given for {absent} (pass roms=..., e.g. rl.synth.nrom_cart(seed))')
        images = [bytes(roms[g]) if isinstance(roms[g], (bytes, bytearray)) else Path(roms[g]).read_bytes()
                  for g in self.games]
        pads = [bytes(boot.get(g, b'')) for g in self.games]
        image_ptrs, pad_ptrs = _carray(ctypes.c_char_p, images), _carray(ctypes.c_char_p, pads)
        self._host_inputs = (images, pads, image_ptrs, pad_ptrs)   # alive for as long as the env
        if on_gpu:
            index = self.device.index if self.device.index is not None else torch.cuda.current_device()
            torch.cuda.set_device(index)
            torch.zeros(1, device=self.device)   # torch's HIP context exists before the library's first call
        else:
            index = 0
        h = self.lib.rlenv_create(len(self.games), _carray(ctypes.c_int, [GAMES.index(g) for g in self.games]),
                                  image_ptrs, _carray(ctypes.c_size_t, [len(b) for b in images]), pad_ptrs,
                                  _carray(ctypes.c_size_t, [len(b) for b in pads]), _carray(ctypes.c_int, self.counts),
                                  int(seed) % 2 ** 64, int(sticky), int(idle_max), int(dropout), index)
        if not h:
            raise RuntimeError(f'rlenv_create: {self.lib.rlenv_error().decode()}')
        return h

    def _enable_archive(self):
        if self.level_slots < self.level_cap:
            self._check(self.lib.rlenv_enable_places(self.h, self.level_cap, self.level_slots))
        else:
            self._check(self.lib.rlenv_enable_level_starts(self.h, self.level_cap))
        self.level_now = torch.full((self.n,), -1, dtype=torch.int32, device=self.device)
        self.progress_now = torch.full((self.n,), float('nan'), dtype=torch.float32, device=self.device)
        self.lib.rlenv_bind_start(self.h, _addr(self.start_level))
        self.lib.rlenv_bind_level(self.h, _addr(self.level_now))
        self.lib.rlenv_bind_progress(self.h, _addr(self.progress_now))

    @staticmethod
    def _p32(p):
        """A probability as the library's 32-bit fixed point (p * 2^32, saturated)."""
        return min(int(float(p) * 2 ** 32), 2 ** 32 - 1)

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def _stream(self):
        """torch's current stream on the env's device (0 = none, on the CPU)."""
        if self.device.type != 'cuda':
            return ctypes.c_void_p(0)
        return ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def _sync(self):
        if self.device.type == 'cuda':
            torch.cuda.synchronize(self.device)

    # ------------------------------------------------------------------ decisions
    def start(self):
        """Boot every env from its game's snapshot and draw the first observation."""
        self._check(self.lib.rlenv_start(self.h, self._stream()))

    def step(self):
        """One decision of every env: 4 frames under the moves in `actions`, then rewards, ends and restarts."""
        self._check(self.lib.rlenv_step(self.h, self._stream()))

    def step_game(self, gi, obs, emph):
        """One decision of the envs of game gi (an index into self.games) only, pictures into obs / emph (tensors of
        the whole batch's shape)."""
        self._check(self.lib.rlenv_step_game(self.h, gi, _addr(obs), _addr(emph), self._stream()))

    def step_range(self, gi, start, count, obs, emph):
        """step_game restricted to envs start..start+count-1 of game gi."""
        self._check(self.lib.rlenv_step_range(self.h, gi, start, count, _addr(obs), _addr(emph), self._stream()))

    # ------------------------------------------------------------------ translated kernels
    def jit_wait(self):
        """Wait until the translated kernel of every translated game (include/rlenv_api.h rlenv_jit_wait) is compiled
        and loaded; an error if a compile, its far-jump check or its load failed."""
        self._check(self.lib.rlenv_jit_wait(self.h))

    def jit_status(self, gi=0) -> dict:
        """State of game gi's translated kernel: state ('none', 'compiling', 'loaded', 'failed'), blocks,
        instructions, compile_ms (-1 while compiling), frame_bank (built for frames drawn from frame banks), banked
        (a banked-PRG translation: blocks keyed by their PRG bank too), far_jumps (in its code object; -1 while
        compiling)."""
        out = (ctypes.c_int32 * 6)()
        self._check(self.lib.rlenv_jit_status(self.h, gi, out))
        return dict(state=('none', 'compiling', 'loaded', 'failed')[out[0]], blocks=out[1], instructions=out[2],
                    compile_ms=out[3], frame_bank=bool(out[4] & 1), banked=bool(out[4] & 2),
                    far_jumps=out[5])

    def set_episode_level_end(self, level):
        """End episodes (reason level_clear) on reaching level `level` + 1 (0: on reaching level 1); -1 = never, the
        default (rl/rlenv.py:323-324)."""
        self.lib.rlenv_set_episode_level_end(self.h, int(level))

    def set_no_render(self, v: bool):
        """Skip drawing the pictures (the emulation and rewards still run)."""
        self.lib.rlenv_set_no_render(self.h, int(bool(v)))

    def drop_obs_buffers(self):
        """Release the default picture tensors, for a caller that binds its own with bind_obs."""
        self.obs = self.emph = None

    def bind_obs(self, obs, emph):
        """Draw the next pictures into obs [N, 4, 224, 240] / emph [N, 4, 224] (uint8, contiguous, on the env's
        device). The env keeps a reference to both until the next bind."""
        if obs.shape != (self.n, FRAMES, OBS_H, OBS_W) or emph.shape != (self.n, FRAMES, OBS_H):
            raise ValueError(f'bind_obs: shapes {tuple(obs.shape)} / {tuple(emph.shape)}')
        if not (obs.is_contiguous() and emph.is_contiguous()):
            raise ValueError('bind_obs: tensors must be contiguous')
        self._bound_pictures = (obs, emph)
        self.lib.rlenv_bind_obs(self.h, _addr(obs), _addr(emph))

    def game_slices(self):
        """The env rows of each game, in self.games order."""
        ends = np.cumsum([0] + self.counts)
        return [slice(int(a), int(b)) for a, b in zip(ends[:-1], ends[1:])]

    def consoles(self, gi=0, first=0, count=None) -> np.ndarray:
        """Console records (include/nesrec.h) of envs first..first+count-1 of game gi, as uint8 [count, 23552]
        (synchronous)."""
        count = self.counts[gi] - first if count is None else count
        out = np.empty((count, NES_REC_BYTES), np.uint8)
        self._sync()
        self._check(self.lib.rlenv_read_consoles(self.h, gi, first, count, out.ctypes.data_as(_P), self._stream()))
        return out

    # ------------------------------------------------------------------ level starts and places
    def set_level_prob(self, prob: float):
        """Chance that a new episode begins from a saved level start, uniform over each game's saved slots."""
        if prob and self.level_cap == 0:
            raise ValueError('set_level_prob: the env keeps no level starts (level_cap=0)')
        for gi in range(len(self.games)):
            self.set_level_plan(gi, prob)

    def set_level_plan(self, gi, prob, weights=None):
        """Game gi's chance of a level start and the weights of its slots ([level_cap], non-zero only on saved
        slots, summing to 1; None = uniform over the saved slots). Takes effect from the next decision."""
        if self.level_cap == 0:
            return
        cdf = None
        if weights is not None:
            w = np.asarray(weights, np.float64)
            top = 2.0 ** 32 - 1
            cdf = np.minimum(np.cumsum(w) * 2.0 ** 32, top)
            cdf[np.nonzero(w)[0].max():] = top   # rounding never leaves the last weighted slot unreachable
            cdf = cdf.astype(np.uint32)
        self._sync()
        self.lib.rlenv_set_level_plan(self.h, gi, float(prob), None if cdf is None else cdf.ctypes.data_as(_P))

    def saved_levels(self):
        """Per game: {slot: deaths of the arrival that was saved} for the level-start slots that hold one
        (synchronous)."""
        out = {}
        for gi, g in enumerate(self.games):
            deaths = np.full(max(self.level_cap, 1), -1, np.int32)
            if self.level_cap > 0:
                self._sync()
                self._check(self.lib.rlenv_level_deaths(self.h, gi, deaths.ctypes.data_as(_P), self._stream()))
            held = np.nonzero(deaths[:self.level_slots] >= 0)[0]
            out[g] = {int(s): int(deaths[s]) for s in held}
        return out

    def place_save(self, gi, env_idx, slot_idx):
        """After a decision, on the current stream: save env env_idx[j] of game gi into place slot slot_idx[j]
        (slots below level_slots are level starts and are left alone). int32 tensors on the env's device."""
        if env_idx.dtype != torch.int32 or slot_idx.dtype != torch.int32 or env_idx.numel() != slot_idx.numel():
            raise ValueError('place_save: two int32 tensors of one length')
        env_idx, slot_idx = env_idx.contiguous(), slot_idx.contiguous()
        self._check(self.lib.rlenv_place_save(self.h, gi, _addr(env_idx), _addr(slot_idx), int(env_idx.numel()),
                                              self._stream()))

    def place_copy(self, gi, src, dst):
        """Copy slot src[j] over slot dst[j] of game gi, the whole saved state (synchronous)."""
        a, b = np.ascontiguousarray(src, np.int32), np.ascontiguousarray(dst, np.int32)
        if a.shape != b.shape:
            raise ValueError('place_copy: src and dst differ in length')
        if a.size:
            self._check(self.lib.rlenv_place_copy(self.h, gi, a.ctypes.data_as(_P), b.ctypes.data_as(_P), a.size,
                                                  self._stream()))

    def level_layout(self, gi):
        """Sizes of game gi's archive slot: stride (console bytes), key_cap (key words), st (tracker block bytes),
        cap (slots) and levels."""
        out = np.zeros(5, np.uint32)
        self.lib.rlenv_level_layout(self.h, gi, out.ctypes.data_as(_P))
        return dict(zip(('stride', 'key_cap', 'st', 'cap', 'levels'), map(int, out)))

    def _tail_widths(self):
        """Per game, the per-slot byte width of each of the six parts of the archive tail."""
        out = []
        for gi in range(len(self.games)):
            lay = self.level_layout(gi)
            out.append((lay['stride'], lay['st'], 4 * lay['key_cap'], 8, 4, 4))
        return out

    def _grow_archive(self, buf, old_cap, need):
        """Re-lay a blob saved with old_cap archive slots per game for this env's level_cap: each part keeps its
        old slots and gains empty ones. None when buf is not such a blob."""
        widths = self._tail_widths()
        old_tail = old_cap * sum(map(sum, widths))
        if len(buf) - old_tail + self.level_cap * sum(map(sum, widths)) != need:
            return None
        pieces, o = [buf[:len(buf) - old_tail]], len(buf) - old_tail
        for game in widths:
            for w, fill in zip(game, _TAIL_FILL):
                pieces.append(buf[o:o + old_cap * w])
                pieces.append(np.full((self.level_cap - old_cap) * w, fill, np.uint8))
                o += old_cap * w
        return np.concatenate(pieces)

    # ------------------------------------------------------------------ exact resume
    def state_dict(self) -> dict:
        """Everything an exact resume needs: the library's state blob (consoles, trackers, dropout, counters, the
        archive) and the outputs a caller reads between decisions."""
        blob = np.empty(self.lib.rlenv_state_bytes(self.h), np.uint8)
        self._sync()
        self._check(self.lib.rlenv_save(self.h, blob.ctypes.data_as(_P), self._stream()))
        outs = {k: getattr(self, k).cpu() for k in ('obs', 'emph', 'masks', 'timeline', 'done', 'reward')
                if getattr(self, k) is not None}
        return dict(env=blob, outputs=outs, games=self.games, counts=self.counts, level_cap=self.level_cap)

    def load_state_dict(self, sd):
        """Resume from state_dict(). A blob saved with fewer archive slots grows into this env's (the new slots
        empty); one saved with no archive takes this env's empty one."""
        if sd['games'] != self.games or sd['counts'] != self.counts:
            raise ValueError('load_state_dict: the env was saved with other games or counts')
        blob = np.ascontiguousarray(sd['env'])
        need = self.lib.rlenv_state_bytes(self.h)
        old_cap = int(sd.get('level_cap', 0))
        if len(blob) < need and self.level_cap > 0:
            if old_cap == 0:
                blob = np.concatenate([blob, self.state_dict()['env'][len(blob):]])
            elif old_cap < self.level_cap:
                grown = self._grow_archive(blob, old_cap, need)
                blob = blob if grown is None else grown
        if len(blob) != need:
            raise ValueError(f'load_state_dict: a {len(blob)}-byte state for a {need}-byte env')
        self._check(self.lib.rlenv_load(self.h, blob.ctypes.data_as(_P), self._stream()))
        for k, v in sd['outputs'].items():
            if getattr(self, k) is not None:
                getattr(self, k).copy_(v)

    def __del__(self):
        if getattr(self, 'h', None):
            self.lib.rlenv_destroy(self.h)
            self.h = None
