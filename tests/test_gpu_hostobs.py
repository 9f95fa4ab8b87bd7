"""The pinned-host rollout store (rl/hostobs.py; the reference trainer's host store, rl/train.py:174-294) over the
library's pack6 / memcpy / gather entry points (rl/csrc/rlenv.cu:366-421): every picture of a rollout written by the
env into the two device slots comes back bit-exact through the host region, both through the copy-engine minibatch
gather + unpack6 and through the kernel row gather, and the packed host rows are the oracle's pack6 of the
pictures."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import HIP_LIB, oracle, ptr
from rl import synth
from rl.hostobs import FRAME_BYTES, RolloutStore
from rl.rlenv import RlEnv


def host_bytes(addr, n):
    return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(addr)).copy()


@pytest.mark.gpu
@pytest.mark.parametrize('pack6', [True, False])
def test_rollout_round_trip_through_pinned_host(pack6):
    N, T, mb, r = 24, 6, 8, 1
    print(f'case: RolloutStore pack6={pack6}, {N} envs x {T} decisions, minibatches of {mb}, region {r} of 2',
          flush=True)
    env = RlEnv({'smb': N}, device='cuda', lib_path=HIP_LIB, roms={'smb': synth.smb_like_cart(3)}, seed=9,
                pad_mode=True, end_prob=1 / 4, idle_max=2)
    store = RolloutStore(env.lib, T, N, 'cuda', mb, regions=2, pack6=pack6)
    emph = torch.zeros(N, 4, 224, dtype=torch.uint8, device='cuda')
    g = torch.Generator().manual_seed(1)
    truth = []
    env.bind_obs(store.target(0), emph)
    env.start()
    truth.append(store.ring[0].clone())
    store.commit(r, 0)
    for t in range(1, T + 1):
        env.bind_obs(store.target(t), emph)
        env.actions.copy_(torch.randint(0, 256, (N,), generator=g, dtype=torch.int16).cuda())
        env.step()
        truth.append(store.ring[t % 2].clone())
        if t == T:   # the last decision in two halves (a caller copying game by game)
            store.commit(r, t, slice(0, 10))
            store.commit(r, t, slice(10, N))
        else:
            store.commit(r, t)
    torch.cuda.synchronize()
    assert any(not torch.equal(truth[t], truth[t + 1]) for t in range(T))
    # host rows: the (packed) pictures
    for t in range(T + 1):
        want = truth[t].cpu().numpy().reshape(-1)
        if pack6:
            packed = np.zeros(want.size // 4 * 3, np.uint8)
            assert oracle().rl_pack6(ptr(want), ptr(packed), want.size, None) == 0
            want = packed
        assert np.array_equal(host_bytes(store.row_address(r, t), N * store.row_bytes), want), t
    # minibatches: copy-engine gather (+ unpack6), one minibatch ahead
    perm = torch.randperm(N, generator=g)
    seen = 0
    for i, b in enumerate(store.minibatches(r, perm, mb)):
        b = b.cpu()
        for t in range(T):
            for j in range(mb):
                assert torch.equal(b[t * mb + j], truth[t][perm[i * mb + j]].cpu()), (i, t, j)
        seen += 1
    assert seen == N // mb
    # kernel gather of host rows over PCIe
    rows = torch.tensor([0, 5, N * 3 + 7, N * T + N - 1, 11], dtype=torch.int64)
    rows_d = rows.cuda()
    dst = torch.empty(len(rows), store.row_bytes, dtype=torch.uint8, device='cuda')
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert env.lib.rl_gather_rows(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(store.row_address(r, 0)),
                                  ctypes.c_void_p(rows_d.data_ptr()), len(rows), store.row_bytes, s) == 0
    torch.cuda.synchronize()
    region = host_bytes(store.row_address(r, 0), (T + 1) * N * store.row_bytes).reshape(-1, store.row_bytes)
    assert np.array_equal(dst.cpu().numpy(), region[rows.numpy()])
    assert env.lib.rl_gather_rows(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(store.row_address(r, 0)),
                                  ctypes.c_void_p(rows_d.data_ptr()), len(rows), 24, s) != 0
    with pytest.raises(ValueError):
        next(store.minibatches(r, perm, mb * 2))
    with pytest.raises(IndexError):
        store.row_address(2, 0)
    store.close()
    assert FRAME_BYTES == 4 * 224 * 240
