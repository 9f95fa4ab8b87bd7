"""`RolloutStore`: a rollout's pictures in pinned host memory, the consumer of the env's pictures in a training loop
(the role of the reference trainer's host store, rl/train.py:174-294), over this library's pack6 / memcpy / gather
entry points (include/rlenv_api.h).

At the reference's sizes the pictures of a T-decision rollout of N envs do not fit beside a learner in HBM, so they
live in host memory and come back one minibatch at a time. The design:

  * Host memory: `regions` blocks of (T + 1) rows x N envs x row_bytes (row 0 of a region is the observation the
    rollout starts from). With pack6 a row is 6 bits per pixel (3/4 of the bytes).
  * Device ring: `ring` picture tensors that the env draws into in turn (decision t into `target(t)`), each with its
    own packed staging buffer and a `drained` event: the ring slot is free again once its copy to the host is done.
    `target(t)` makes torch's current stream wait for that before it hands the slot out, so the env never
    overwrites pictures that are still being copied, and the host never blocks.
  * `commit(region, t)` packs the slot on the current stream (right behind the env's decision), then copies it to
    host row t of the region on a copy stream, so the copy overlaps the next decision.
  * `minibatches(region, perm, mb)` yields the learner [T * mb, 4, 224, 240] device tensors (row t * mb + j =
    decision t of env perm[i * mb + j]): a strided host-to-device copy per env (rl_gather_envs) into one of two
    device buffers, unpacked there, on a gather stream that runs one minibatch ahead; a buffer is reused once the
    caller has asked for the minibatch after the one it held. The gather stream first waits for the copy stream, so
    the rollout's copies are complete without a host synchronisation.

The copy and gather streams are the library's (rl_stream_create: default priority, not synchronised with the null
stream), used through torch as external streams and destroyed by close(). torch's own streams live until the process
ends, and the runtime places each stream on the hardware queue that serves the fewest, so streams kept alive after
the store is done would move every later stream of the process (a twelve-game env's game streams stepped at 1.28 M
decisions/s after a store on torch streams, 1.53 M after one on these). Ordering is by torch events only.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

FRAME_BYTES = 4 * 224 * 240
PACKED_BYTES = FRAME_BYTES * 3 // 4


def _vp(x):
    return ctypes.c_void_p(x if isinstance(x, int) else x.data_ptr())


class RolloutStore:
    def __init__(self, lib, decisions, envs, device, minibatch_envs, regions=1, ring=2, pack6=True):
        """lib: the env's library (RlEnv.lib). decisions: T, rows per region after the start row. envs: N.
        minibatch_envs: the largest minibatch `minibatches` will be asked for."""
        self.lib, self.T, self.N = lib, int(decisions), int(envs)
        self.dev = torch.device(device)
        self.pack6 = bool(pack6)
        self.row_bytes = PACKED_BYTES if self.pack6 else FRAME_BYTES
        self.region_bytes = (self.T + 1) * self.N * self.row_bytes
        self.regions = int(regions)
        self.base = lib.rl_host_alloc(self.region_bytes * self.regions)
        if not self.base:
            raise RuntimeError(f'pinned host allocation of {self.region_bytes * self.regions / 2 ** 30:.2f} GiB '
                               f'failed: {lib.rlenv_error().decode()}')
        new = lambda *shape: torch.empty(shape, dtype=torch.uint8, device=self.dev)  # noqa: E731
        self.ring = [new(self.N, 4, 224, 240).zero_() for _ in range(int(ring))]
        self.staging = [new(self.N, self.row_bytes) for _ in self.ring] if self.pack6 else None
        self.drained = [torch.cuda.Event() for _ in self.ring]
        self._streams = []
        self.copy_stream, self.gather_stream = self._stream(), self._stream()
        self.mb_cap = int(minibatch_envs)
        self.batches = [new(self.T * self.mb_cap, 4, 224, 240) for _ in range(2)]
        self.packed_batches = [new(self.T * self.mb_cap, self.row_bytes) for _ in range(2)] if self.pack6 else None
        self.ready = [torch.cuda.Event() for _ in range(2)]
        self.released = [torch.cuda.Event() for _ in range(2)]

    def _stream(self):
        """A stream of the library's (default priority), which close() destroys, as a torch external stream."""
        h = ctypes.c_void_p()
        self._check(self.lib.rl_stream_create(ctypes.byref(h)))
        self._streams.append(h.value)
        return torch.cuda.ExternalStream(h.value, device=self.dev)

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def row_address(self, region, t):
        """Host address of row t of a region (N consecutive env rows of row_bytes)."""
        if not (0 <= region < self.regions and 0 <= t <= self.T):
            raise IndexError(f'row {t} of region {region}')
        return self.base + region * self.region_bytes + t * self.N * self.row_bytes

    # ----------------------------------------------------------------- rollout side
    def target(self, t):
        """The ring slot decision t is drawn into (bind it with RlEnv.bind_obs), free once torch's current stream
        reaches this point: the stream waits for the slot's last copy to the host."""
        k = t % len(self.ring)
        torch.cuda.current_stream(self.dev).wait_event(self.drained[k])
        return self.ring[k]

    def commit(self, region, t, rows=None):
        """Decision t is in its ring slot: pack it (pack6) on the current stream and copy it, or the env rows
        `rows` (a slice) of it, to host row t of the region on the copy stream."""
        k = t % len(self.ring)
        rows = rows or slice(0, self.N)
        current = torch.cuda.current_stream(self.dev)
        src = self.ring[k][rows]
        if self.pack6:
            dst = self.staging[k][rows]
            self._check(self.lib.rl_pack6(_vp(src), _vp(dst), src.numel(), _vp(current.cuda_stream)))
            src = dst
        self.copy_stream.wait_stream(current)
        self._check(self.lib.rl_memcpy_async(_vp(self.row_address(region, t) + rows.start * self.row_bytes),
                                             _vp(src), src.numel(),
                                             _vp(self.copy_stream.cuda_stream)))
        self.drained[k].record(self.copy_stream)

    # ----------------------------------------------------------------- learner side
    def minibatches(self, region, perm, mb):
        """Iterate over the region's decisions 0..T-1 in minibatches of mb envs taken in the order of perm (env
        indices); each item is ready on torch's current stream when it is returned."""
        envs = np.ascontiguousarray(torch.as_tensor(perm).cpu().numpy(), dtype=np.int64)
        if envs.size and (envs.min() < 0 or envs.max() >= self.N):
            raise ValueError('minibatches: env index out of range')
        if not 0 < mb <= self.mb_cap:
            raise ValueError(f'minibatches: {mb} envs per minibatch, the buffers hold {self.mb_cap}')
        count = len(envs) // mb
        src = self.row_address(region, 0)
        self.gather_stream.wait_stream(self.copy_stream)
        self.gather_stream.wait_stream(torch.cuda.current_stream(self.dev))

        def fetch(i):
            k = i % 2
            self.gather_stream.wait_event(self.released[k])
            chunk = envs[i * mb:(i + 1) * mb]
            staged = self.packed_batches[k] if self.pack6 else self.batches[k]
            self._check(self.lib.rl_gather_envs(_vp(staged), _vp(src), chunk.ctypes.data_as(ctypes.c_void_p), mb,
                                                self.T, self.N, self.row_bytes, _vp(self.gather_stream.cuda_stream)))
            if self.pack6:
                self._check(self.lib.rl_unpack6(_vp(staged), _vp(self.batches[k]), self.T * mb * FRAME_BYTES,
                                                _vp(self.gather_stream.cuda_stream)))
            self.ready[k].record(self.gather_stream)

        return self._iterate(count, mb, fetch)

    def _iterate(self, count, mb, fetch):
        if count:
            fetch(0)
        for i in range(count):
            if i + 1 < count:
                fetch(i + 1)
            current = torch.cuda.current_stream(self.dev)
            current.wait_event(self.ready[i % 2])
            yield self.batches[i % 2][:self.T * mb]
            self.released[i % 2].record(torch.cuda.current_stream(self.dev))

    def close(self):
        """Wait for the device, then free the pinned host memory and destroy the store's streams."""
        if getattr(self, 'base', None) or getattr(self, '_streams', None):
            torch.cuda.synchronize(self.dev)
        if getattr(self, 'base', None):
            self.lib.rl_host_free(ctypes.c_void_p(self.base))
            self.base = None
        for h in getattr(self, '_streams', None) or ():
            self.lib.rl_stream_destroy(ctypes.c_void_p(h))
        self._streams = []

    def __del__(self):
        self.close()
