"""Python side of the batched NES environment step: the drop-in for the reference's rl/rlenv.py.

    env = RlEnv({'smb': 8192}, device='cuda', seed=1, roms={'smb': cart_bytes})
    env.start()                       # first observation in env.obs / env.emph, legal parts in env.masks
    env.actions.copy_(moves)          # int16 packed move ids (controller.cuh), legal under env.masks
    env.step()                        # env.obs, reward, done, masks, timeline, pads, events, info updated in place

Same constructor, tensors, dtypes, shapes and methods as rl/rlenv.py:172-389 (RlEnv), over this repo's HIP library
(ghostrun-lab_amd/csrc -> librlenv_hip.so, loaded with ctypes exactly as rl/rlenv.py:76-121 loads the CUDA one).
Everything stays on the device; nothing is copied to the host per step. Calls go on torch's current stream.

device='cpu' has no product build here: pass ``lib_path`` to a library with the same C ABI (the tests pass the
CPU oracle's). On a GPU device the HIP library must be built (``python __graft_entry__.py`` or
``make -C ghostrun-lab_amd/csrc``); a missing library is an error, never a silent fallback.

Additions for the benchmark workloads (no reference counterpart): ``roms`` may map a slug to iNES bytes (the
seed-generated carts of rl.synth); ``boot`` maps a slug to its boot pad bytes (default: none, start at power-on);
``pad_mode=True`` makes actions raw pad bytes; ``end_prob`` adds a Geometric episode end per decision;
``dropout_gap`` sets P(a dropout gap ends) per decision; ``ram_hash=True`` binds a per-decision RAM hash output.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np
import torch

PKG = Path(__file__).resolve().parents[1]          # ghostrun-lab_amd/
HIP_LIB = Path(os.environ.get('RL_HIP_LIB', PKG / 'csrc' / '_build' / 'librlenv_hip.so'))

# rl/games_manifest.json order = reward10 game ids (rl/rlenv.py:30-31)
GAMES = ['smb', 'pacman', 'excitebike', 'contra', 'castlevania', 'gradius', 'zelda', 'tetris', 'tecmobowl', 'kage',
         'finalmission', 'punchout']
OBS_H, OBS_W, FRAMES = 224, 240, 4
FRAME_BYTES = FRAMES * OBS_H * OBS_W
MASK_BYTES, TIMELINE, INFO = 19, 8 * 45, 8
PART_NAMES = ('progress', 'level', 'death', 'damage', 'score', 'win', 'stall')  # rlenv.parts columns
NUM_PARTS = len(PART_NAMES)
END_NAMES = {0: 'none', 1: 'game_over', 2: 'won', 3: 'skip', 4: 'stall', 5: 'fault', 6: 'level_clear', 7: 'synthetic'}
NES_REC_BYTES = 23552   # include/nesrec.h
READER_BYTES = 120      # sizeof(Rl10Reader), include/rlenv_state.h


def _load(path: Path):
    """ctypes binding of the C ABI (include/rlenv_api.h; the reference's rl/rlenv.py:76-121)."""
    lib = ctypes.CDLL(str(path))
    P, I, U64, U32, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_size_t
    lib.rlenv_create.restype = P
    lib.rlenv_create.argtypes = [I, P, P, P, P, P, P, U64, I, I, I, I]
    lib.rlenv_num_envs.argtypes = [P]
    lib.rlenv_bind.argtypes = [P] * 11
    lib.rlenv_bind_parts.argtypes = [P, P]
    lib.rlenv_bind_obs.argtypes = [P, P, P]
    lib.rlenv_start.argtypes = [P, P]
    lib.rlenv_step.argtypes = [P, P]
    lib.rlenv_state_bytes.restype = SZ
    lib.rlenv_state_bytes.argtypes = [P]
    lib.rlenv_save.argtypes = [P, P, P]
    lib.rlenv_load.argtypes = [P, P, P]
    lib.rlenv_error.restype = ctypes.c_char_p
    lib.rlenv_destroy.argtypes = [P]
    lib.rlenv_set_episode_level_end.argtypes = [P, I]
    lib.rlenv_num_games.argtypes = [P]
    lib.rlenv_set_no_render.argtypes = [P, I]
    lib.rlenv_set_pad_mode.argtypes = [P, I]
    lib.rlenv_set_end_prob.argtypes = [P, U32]
    lib.rlenv_set_dropout_gap.argtypes = [P, U32]
    lib.rlenv_bind_ram_hash.argtypes = [P, P]
    lib.rlenv_read_consoles.argtypes = [P, I, I, I, P, P]
    lib.rlenv_enable_level_starts.argtypes = [P, I]
    lib.rlenv_enable_places.argtypes = [P, I, I]
    lib.rlenv_set_level_plan.argtypes = [P, I, ctypes.c_double, P]
    lib.rlenv_bind_start.argtypes = lib.rlenv_bind_level.argtypes = lib.rlenv_bind_progress.argtypes = [P, P]
    lib.rlenv_level_deaths.argtypes = [P, I, P, P]
    lib.rlenv_place_save.argtypes = lib.rlenv_place_copy.argtypes = [P, I, P, P, I, P]
    lib.rlenv_level_layout.argtypes = [P, I, P]
    lib.rl_pack6.argtypes = [P, P, SZ, P]
    lib.rl_unpack6.argtypes = [P, P, SZ, P]
    lib.rl10_smb_run.argtypes = [P, I, I, I, P, P, P, P]
    lib.rl10_run.argtypes = [I, P, I, I] + [P] * 11
    if hasattr(lib, 'rl_gather_rows'):  # GPU build only
        lib.rl_host_alloc.restype = P
        lib.rl_host_alloc.argtypes = [SZ]
        lib.rl_host_free.argtypes = [P]
        lib.rl_memcpy_async.argtypes = [P, P, SZ, P]
        lib.rl_gather_rows.argtypes = [P, P, P, I, SZ, P]
        lib.rl_gather_envs.argtypes = [P, P, P, I, I, I, SZ, P]
    if hasattr(lib, 'rlenv_step_range'):
        lib.rlenv_step_game.argtypes = [P, I, P, P, P]
        lib.rlenv_step_range.argtypes = [P, I, I, I, P, P, P]
    return lib


def hip_library() -> Path:
    if not HIP_LIB.exists():
        raise RuntimeError(f'{HIP_LIB} is not built: run `python __graft_entry__.py` (the HIP build) first')
    return HIP_LIB


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


class RlEnv:
    def __init__(self, counts: dict, device='cuda', seed=0, sticky=True, idle_max=30, dropout=True, roms=None,
                 lib_path=None, level_cap=0, level_slots=None, boot=None, pad_mode=False, end_prob=0.0,
                 dropout_gap=None, ram_hash=False):
        """counts: game slug -> number of envs (envs are laid out in GAMES order). roms: slug -> iNES path or bytes.
        level_cap > 0: save level starts (levels 0..level_cap-1 of each game), used by new episodes with the chance
        set by set_level_prob / set_level_plan (default 0); self.start_level: the slot a finished episode started
        from (-1 = boot snapshot, valid where done); self.level_now / self.progress_now: the level and within-level
        progress after each decision. level_slots < level_cap: only slots 0..level_slots-1 are level starts, the rest
        are places filled by place_save (rl/rlenv.py:172-238 of the reference)."""
        self.device = torch.device(device)
        self.games = [g for g in GAMES if counts.get(g, 0) > 0]
        self.counts = [int(counts[g]) for g in self.games]
        self.n = sum(self.counts)
        self.game_of_env = torch.tensor(sum(([GAMES.index(g)] * c for g, c in zip(self.games, self.counts)), []),
                                        dtype=torch.long, device=self.device)
        gpu = self.device.type == 'cuda'
        if lib_path is None:
            if not gpu:
                raise RuntimeError("device='cpu' needs lib_path (a CPU library with the same C ABI)")
            lib_path = hip_library()
        self.lib_path = Path(lib_path)
        self.lib = _load(self.lib_path)
        roms, boot = roms or {}, boot or {}
        missing = [g for g in self.games if g not in roms]
        if missing:
            raise RuntimeError(f'no ROM given for {missing} (pass roms=..., e.g. rl.synth.nrom_cart(seed))')
        rom_bytes = [bytes(roms[g]) if isinstance(roms[g], (bytes, bytearray)) else Path(roms[g]).read_bytes()
                     for g in self.games]
        boots = [bytes(boot.get(g, b'')) for g in self.games]
        self._keep = [rom_bytes, boots]
        arr = lambda T, xs: (T * len(xs))(*xs)  # noqa: E731
        rom_p = arr(ctypes.c_char_p, rom_bytes)
        boot_p = arr(ctypes.c_char_p, boots)
        self._keep += [rom_p, boot_p]
        dev_index = self.device.index if self.device.index is not None else (torch.cuda.current_device() if gpu else 0)
        if gpu:
            torch.cuda.set_device(dev_index)
            torch.zeros(1, device=self.device)  # torch's HIP context first
        self.h = self.lib.rlenv_create(
            len(self.games), arr(ctypes.c_int, [GAMES.index(g) for g in self.games]), rom_p,
            arr(ctypes.c_size_t, [len(r) for r in rom_bytes]), boot_p, arr(ctypes.c_size_t, [len(b) for b in boots]),
            arr(ctypes.c_int, self.counts), int(seed) & (2 ** 64 - 1), int(sticky), int(idle_max), int(dropout),
            dev_index)
        if not self.h:
            raise RuntimeError(f'rlenv_create: {self.lib.rlenv_error().decode()}')
        N, d = self.n, self.device
        self.actions = torch.zeros(N, dtype=torch.int16, device=d)
        self.obs = torch.zeros(N, FRAMES, OBS_H, OBS_W, dtype=torch.uint8, device=d)
        self.emph = torch.zeros(N, FRAMES, OBS_H, dtype=torch.uint8, device=d)
        self.reward = torch.zeros(N, dtype=torch.float32, device=d)
        self.done = torch.zeros(N, dtype=torch.uint8, device=d)
        self.masks = torch.zeros(N, MASK_BYTES, dtype=torch.uint8, device=d)
        self.timeline = torch.zeros(N, 8, 45, dtype=torch.uint8, device=d)
        self.pads = torch.zeros(N, FRAMES, dtype=torch.uint8, device=d)
        self.events = torch.zeros(N, dtype=torch.int32, device=d)
        self.info = torch.zeros(N, INFO, dtype=torch.float32, device=d)
        self.lib.rlenv_bind(self.h, _ptr(self.actions), _ptr(self.obs), _ptr(self.emph), _ptr(self.reward),
                            _ptr(self.done), _ptr(self.masks), _ptr(self.timeline), _ptr(self.pads),
                            _ptr(self.events), _ptr(self.info))
        self.parts = torch.zeros(N, NUM_PARTS, dtype=torch.float32, device=d)
        self.lib.rlenv_bind_parts(self.h, _ptr(self.parts))
        self.level_cap = int(level_cap)
        self.level_slots = int(level_slots if level_slots is not None else level_cap)
        self.start_level = torch.full((N,), -1, dtype=torch.int32, device=d)
        if self.level_cap > 0:
            ok = (self.lib.rlenv_enable_places(self.h, self.level_cap, self.level_slots)
                  if self.level_slots < self.level_cap else self.lib.rlenv_enable_level_starts(self.h, self.level_cap))
            if ok != 0:
                raise RuntimeError(self.lib.rlenv_error().decode())
            self.lib.rlenv_bind_start(self.h, _ptr(self.start_level))
            self.level_now = torch.full((N,), -1, dtype=torch.int32, device=d)
            self.lib.rlenv_bind_level(self.h, _ptr(self.level_now))
            self.progress_now = torch.full((N,), float('nan'), dtype=torch.float32, device=d)
            self.lib.rlenv_bind_progress(self.h, _ptr(self.progress_now))
        self.lib.rlenv_set_pad_mode(self.h, int(bool(pad_mode)))
        if end_prob:
            self.lib.rlenv_set_end_prob(self.h, min(int(float(end_prob) * 2 ** 32), 2 ** 32 - 1))
        if dropout_gap is not None:
            self.lib.rlenv_set_dropout_gap(self.h, min(int(float(dropout_gap) * 2 ** 32), 2 ** 32 - 1))
        self.ram_hash = None
        if ram_hash:
            self.ram_hash = torch.zeros(N, dtype=torch.int64, device=d)
            self.lib.rlenv_bind_ram_hash(self.h, _ptr(self.ram_hash))

    def set_level_prob(self, prob: float):
        """Chance that a new episode starts from a saved level start (uniform over each game's saved slots)."""
        assert self.level_cap > 0 or prob == 0
        for gi in range(len(self.games)):
            self.set_level_plan(gi, prob)

    def set_level_plan(self, gi, prob, weights=None):
        """Game gi's chance of a level start and its slot weights ([level_cap], weight only on saved slots, sum 1;
        None = uniform over the saved slots). Call between decisions."""
        if self.level_cap == 0:
            return
        cdf = None
        if weights is not None:
            w = np.asarray(weights, np.float64)
            cdf = np.minimum(np.cumsum(w) * 2.0 ** 32, 2.0 ** 32 - 1).astype(np.uint32)
            cdf[np.flatnonzero(w)[-1]:] = 2 ** 32 - 1   # the last weighted slot takes the rounding remainder
        self._sync()
        self.lib.rlenv_set_level_plan(self.h, gi, float(prob),
                                      None if cdf is None else cdf.ctypes.data_as(ctypes.c_void_p))

    def saved_levels(self):
        """game slug -> {slot: deaths of the saved arrival} over the level slots (synchronous)."""
        out = {}
        for gi, g in enumerate(self.games):
            buf = np.full(max(self.level_cap, 1), -1, np.int32)
            if self.level_cap > 0:
                self._sync()
                if self.lib.rlenv_level_deaths(self.h, gi, buf.ctypes.data_as(ctypes.c_void_p), self._stream()) != 0:
                    raise RuntimeError(self.lib.rlenv_error().decode())
            out[g] = {int(s): int(v) for s, v in enumerate(buf[:self.level_slots]) if v >= 0}
        return out

    def place_save(self, gi, env_idx, slot_idx):
        """After a step, on the current stream: env env_idx[j] (index within game gi) -> place slot slot_idx[j]
        (skipped where < level_slots). int32 tensors on the env's device."""
        assert env_idx.dtype == torch.int32 and slot_idx.dtype == torch.int32
        assert env_idx.is_contiguous() and slot_idx.is_contiguous() and env_idx.numel() == slot_idx.numel()
        if self.lib.rlenv_place_save(self.h, gi, _ptr(env_idx), _ptr(slot_idx), int(env_idx.numel()),
                                     self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def place_copy(self, gi, src, dst):
        """Slot src[j] -> slot dst[j] of game gi (the whole saved state), synchronous."""
        a, b = np.ascontiguousarray(src, np.int32), np.ascontiguousarray(dst, np.int32)
        if len(a) != len(b):
            raise ValueError('place_copy: src and dst differ in length')
        if len(a) and self.lib.rlenv_place_copy(self.h, gi, a.ctypes.data_as(ctypes.c_void_p),
                                                b.ctypes.data_as(ctypes.c_void_p), len(a), self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def level_layout(self, gi):
        out = np.zeros(5, np.uint32)
        self.lib.rlenv_level_layout(self.h, gi, out.ctypes.data_as(ctypes.c_void_p))
        return dict(stride=int(out[0]), key_cap=int(out[1]), st=int(out[2]), cap=int(out[3]), levels=int(out[4]))

    def _archive_sizes(self, cap):
        """Byte sizes of the level-start tail of the state blob per game for `cap` slots: saved consoles, trackers,
        reader states, key words, targets, frames, deaths (the order the library saves them in)."""
        out = []
        for gi in range(len(self.games)):
            lay = self.level_layout(gi)
            out.append([cap * lay['stride'], cap * lay['st'], cap * READER_BYTES, cap * lay['key_cap'] * 4, cap * 8,
                        cap * 4, cap * 4])
        return out

    def _grow_archive(self, buf, old_cap, need):
        """A state saved with old_cap slots per game -> this env's level_cap (the new slots empty); None when buf is
        not such a state."""
        old, new = self._archive_sizes(old_cap), self._archive_sizes(self.level_cap)
        old_tail = sum(map(sum, old))
        if len(buf) - old_tail + sum(map(sum, new)) != need:
            return None
        parts, o = [buf[:len(buf) - old_tail]], len(buf) - old_tail
        for so, sn in zip(old, new):
            for k, (a, b) in enumerate(zip(so, sn)):
                parts.append(buf[o:o + a])
                o += a
                parts.append(np.full(b - a, 0xFF if k == 6 else 0, np.uint8))   # deaths -1 = empty
        return np.concatenate(parts)

    def _sync(self):
        if self.device.type == 'cuda':
            torch.cuda.synchronize(self.device)

    def drop_obs_buffers(self):
        """Free the default picture outputs (a caller that always binds its own via bind_obs)."""
        self.obs = self.emph = None

    def bind_obs(self, obs, emph):
        """Write the next pictures into these tensors ([N,4,224,240] / [N,4,224] uint8, contiguous, same device)."""
        assert obs.is_contiguous() and emph.is_contiguous() and obs.shape == (self.n, FRAMES, OBS_H, OBS_W)
        self._obs_keep = (obs, emph)
        self.lib.rlenv_bind_obs(self.h, _ptr(obs), _ptr(emph))

    def _stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream if self.device.type == 'cuda' else 0)

    def set_episode_level_end(self, level):
        self.lib.rlenv_set_episode_level_end(self.h, int(level))

    def set_no_render(self, v: bool):
        self.lib.rlenv_set_no_render(self.h, int(bool(v)))

    def start(self):
        if self.lib.rlenv_start(self.h, self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def step(self):
        if self.lib.rlenv_step(self.h, self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def step_game(self, gi, obs, emph):
        """Step only the gi-th game (of self.games) on the current stream, its pictures into obs/emph."""
        if self.lib.rlenv_step_game(self.h, gi, _ptr(obs), _ptr(emph), self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def step_range(self, gi, start, count, obs, emph):
        """Like step_game, for envs [start, start+count) of the gi-th game only."""
        if self.lib.rlenv_step_range(self.h, gi, start, count, _ptr(obs), _ptr(emph), self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def game_slices(self):
        out, a = [], 0
        for c in self.counts:
            out.append(slice(a, a + c))
            a += c
        return out

    def consoles(self, gi=0, first=0, count=None) -> np.ndarray:
        """Console records (include/nesrec.h) of game gi, envs [first, first+count), as uint8 [count, 23552]."""
        count = self.counts[gi] - first if count is None else count
        out = np.empty((count, NES_REC_BYTES), np.uint8)
        if self.device.type == 'cuda':
            torch.cuda.synchronize(self.device)
        if self.lib.rlenv_read_consoles(self.h, gi, first, count, out.ctypes.data_as(ctypes.c_void_p),
                                        self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())
        return out

    def state_dict(self) -> dict:
        """Exact resume state of every env (emulators, rewards, dropout, RNG counters) plus the observation outputs."""
        buf = np.empty(self.lib.rlenv_state_bytes(self.h), np.uint8)
        if self.device.type == 'cuda':
            torch.cuda.synchronize(self.device)
        if self.lib.rlenv_save(self.h, buf.ctypes.data_as(ctypes.c_void_p), self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())
        outs = {k: getattr(self, k).cpu() for k in ('obs', 'emph', 'masks', 'timeline', 'done', 'reward')
                if getattr(self, k) is not None}
        return dict(env=buf, outputs=outs, games=self.games, counts=self.counts, level_cap=self.level_cap)

    def load_state_dict(self, sd):
        """Exact resume. A state saved with fewer level slots grows into this env's (new slots empty); a state
        saved without level starts gets an empty archive (its level-start tail is this fresh env's)."""
        assert sd['games'] == self.games and sd['counts'] == self.counts, 'env layout changed'
        buf = np.ascontiguousarray(sd['env'])
        need = self.lib.rlenv_state_bytes(self.h)
        old_cap = int(sd.get('level_cap', 0))
        if len(buf) < need and self.level_cap > old_cap > 0:
            grown = self._grow_archive(buf, old_cap, need)
            buf = buf if grown is None else grown
        if len(buf) < need and self.level_cap > 0 and old_cap == 0:
            buf = np.concatenate([buf, self.state_dict()['env'][len(buf):]])
        assert len(buf) == need, 'env state size changed'
        if self.lib.rlenv_load(self.h, buf.ctypes.data_as(ctypes.c_void_p), self._stream()) != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())
        for k, v in sd['outputs'].items():
            if getattr(self, k) is not None:
                getattr(self, k).copy_(v)

    def __del__(self):
        if getattr(self, 'h', None):
            self.lib.rlenv_destroy(self.h)
            self.h = None
