"""Rollout pictures in pinned host memory: the consumer of the environment's pictures in the reference trainer
(rl/train.py:174-294, class HostObs), over this library's entry points.

A rollout of T decisions of N envs does not fit next to the learner in HBM at the reference's sizes, so the pictures
go to pinned host memory and come back per minibatch:

  * the env draws decision t into device slot t % nslots (`slot`, bound with RlEnv.bind_obs);
  * `saved(r, t)` packs the slot 6 bits per pixel on the device (pack6, 3/4 of the bytes) and copies it into row t of
    host region r on a side stream, so the copy overlaps the next decision;
  * `before_write(t)` makes the env wait until the slot it draws next has been copied out;
  * `epoch(r, perm, mb)` / `batch(i)` / `done_with(i)` hand the learner whole T-row sequences of mb envs: a 2-D copy per
    env (rl_gather_envs, the copy engines) into one of two device buffers, unpacked (rl_unpack6) on a gather stream,
    one minibatch ahead of the learner.

Streams are torch streams at the default priority; ordering is by torch events only (no host synchronisation
except where the docstrings say so). Region r holds T + 1 rows: row 0 is the observation the rollout starts from.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

FRAME_BYTES = 4 * 224 * 240


class HostObs:
    def __init__(self, lib, T, N, dev, mb, regions, nslots=2, pack6=False):
        if nslots not in (1, 2) or T % nslots:
            raise ValueError('nslots must be 1 or 2 and divide T (the next rollout starts in slot 0)')
        self.lib, self.T, self.N, self.dev, self.nslots = lib, int(T), int(N), torch.device(dev), int(nslots)
        self.pack6 = bool(pack6)
        self.row_bytes = FRAME_BYTES * 3 // 4 if self.pack6 else FRAME_BYTES
        self.region_bytes = (self.T + 1) * self.N * self.row_bytes
        self.ptr = lib.rl_host_alloc(self.region_bytes * int(regions))
        if not self.ptr:
            raise RuntimeError(f'pinned host allocation of {self.region_bytes * regions / 2 ** 30:.2f} GiB failed: '
                               f'{lib.rlenv_error().decode()}')
        self.slots = [torch.zeros(N, 4, 224, 240, dtype=torch.uint8, device=self.dev) for _ in range(self.nslots)]
        self.packed = torch.empty(N, self.row_bytes, dtype=torch.uint8, device=self.dev) if self.pack6 else None
        self.d2h = torch.cuda.Stream(self.dev)
        self.gather = torch.cuda.Stream(self.dev)
        self.copied = [torch.cuda.Event() for _ in range(2)]     # slot k's last copy-out has finished
        self.mbuf = [torch.empty(self.T * mb, 4, 224, 240, dtype=torch.uint8, device=self.dev) for _ in range(2)]
        self.pmbuf = ([torch.empty(self.T * mb, self.row_bytes, dtype=torch.uint8, device=self.dev) for _ in range(2)]
                      if self.pack6 else self.mbuf)
        self.mb_cap = int(mb)
        self.fetched = [torch.cuda.Event() for _ in range(2)]    # minibatch buffer k is filled
        self.used = [torch.cuda.Event() for _ in range(2)]       # the learner is done with minibatch buffer k
        self.d2h_g, self.copied_g = [], []

    def close(self):
        if getattr(self, 'ptr', None):
            torch.cuda.synchronize(self.dev)
            self.lib.rl_host_free(ctypes.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        self.close()

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.rlenv_error().decode())

    def host_row(self, r, t):
        """Address of row t of region r (N rows of row_bytes)."""
        return self.ptr + r * self.region_bytes + t * self.N * self.row_bytes

    def slot(self, r, t):
        return self.slots[t % self.nslots]

    def before_write(self, t):
        """The env is about to draw decision t + 1 into its slot: that slot's previous copy-out must have finished."""
        torch.cuda.current_stream(self.dev).wait_event(self.copied[(t + 1) % self.nslots])

    def _copy_out(self, src, dst, nbytes, stream, done_event):
        current = torch.cuda.current_stream(self.dev)
        stream.wait_stream(current)
        self._check(self.lib.rl_memcpy_async(ctypes.c_void_p(dst), ctypes.c_void_p(src.data_ptr()), nbytes,
                                             ctypes.c_void_p(stream.cuda_stream)))
        done_event.record(stream)

    def saved(self, r, t):
        """Slot t % nslots holds decision t: copy it (packed when pack6) into row t of region r."""
        current = torch.cuda.current_stream(self.dev)
        src = self.slots[t % self.nslots]
        if self.pack6:
            current.wait_event(self.copied[(t - 1) % self.nslots])   # one packed staging row: its last copy is out
            self._check(self.lib.rl_pack6(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(self.packed.data_ptr()),
                                          self.N * FRAME_BYTES, ctypes.c_void_p(current.cuda_stream)))
            src = self.packed
        self._copy_out(src, self.host_row(r, t), self.N * self.row_bytes, self.d2h, self.copied[t % self.nslots])

    def handoff(self, src, dst):
        """Decision T sits in device slot T % nslots == 0, where the next rollout starts: nothing to move."""

    def _game_streams(self, gi):
        while len(self.d2h_g) <= gi:
            self.d2h_g.append(torch.cuda.Stream(self.dev))
            self.copied_g.append([torch.cuda.Event(), torch.cuda.Event()])
        return self.d2h_g[gi], self.copied_g[gi]

    def before_write_game(self, gi, t):
        torch.cuda.current_stream(self.dev).wait_event(self._game_streams(gi)[1][(t + 1) % self.nslots])

    def saved_game(self, r, t, gi, rows):
        """Like saved, for the env rows `rows` (a slice) of game gi, on that game's own copy stream."""
        stream, events = self._game_streams(gi)
        current = torch.cuda.current_stream(self.dev)
        src = self.slots[t % self.nslots][rows]
        if self.pack6:
            current.wait_event(events[(t - 1) % self.nslots])
            packed = self.packed[rows]
            self._check(self.lib.rl_pack6(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(packed.data_ptr()),
                                          src.numel(), ctypes.c_void_p(current.cuda_stream)))
            src = packed
        self._copy_out(src, self.host_row(r, t) + rows.start * self.row_bytes, (rows.stop - rows.start) * self.row_bytes,
                       stream, events[t % self.nslots])

    def epoch(self, r, perm, mb):
        """This epoch's minibatches: whole T-row sequences of mb envs of region r, in the order of perm (env
        indices); starts fetching the first. Every copy-out of region r must have finished (the caller synchronises
        between rollout and learning)."""
        self.base = self.host_row(r, 0)
        self.perm_host = np.ascontiguousarray(torch.as_tensor(perm).cpu().numpy().astype(np.int64))
        if self.perm_host.size and (self.perm_host.min() < 0 or self.perm_host.max() >= self.N):
            raise ValueError('epoch: env index out of range')
        self.mb = int(mb)
        if not 0 < self.mb <= self.mb_cap:
            raise ValueError(f'epoch: minibatch of {mb} envs, the buffers hold {self.mb_cap}')
        self.nmb = len(self.perm_host) // self.mb
        self.gather.wait_stream(torch.cuda.current_stream(self.dev))
        if self.nmb:
            self._fetch(0)

    def _fetch(self, i):
        k = i % 2
        self.gather.wait_event(self.used[k])
        envs = self.perm_host[i * self.mb:(i + 1) * self.mb]
        self._check(self.lib.rl_gather_envs(ctypes.c_void_p(self.pmbuf[k].data_ptr()), ctypes.c_void_p(self.base),
                                            envs.ctypes.data_as(ctypes.c_void_p), self.mb, self.T, self.N,
                                            self.row_bytes, ctypes.c_void_p(self.gather.cuda_stream)))
        if self.pack6:
            self._check(self.lib.rl_unpack6(ctypes.c_void_p(self.pmbuf[k].data_ptr()),
                                            ctypes.c_void_p(self.mbuf[k].data_ptr()), self.T * self.mb * FRAME_BYTES,
                                            ctypes.c_void_p(self.gather.cuda_stream)))
        self.fetched[k].record(self.gather)

    def batch(self, i):
        """Minibatch i as [T * mb, 4, 224, 240] uint8 (row t * mb + j = decision t of env perm[i * mb + j]), ready on
        the current stream; the next one is fetched meanwhile."""
        if i + 1 < self.nmb:
            self._fetch(i + 1)
        torch.cuda.current_stream(self.dev).wait_event(self.fetched[i % 2])
        return self.mbuf[i % 2]

    def done_with(self, i):
        self.used[i % 2].record(torch.cuda.current_stream(self.dev))
