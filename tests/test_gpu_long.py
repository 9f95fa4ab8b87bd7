"""Parity at the lengths the reference and the benchmark configurations state, each run once:

* the reference's own equality gate (rl/tests/gpu_check.py:28-53): all twelve games, 4 consoles each, sticky moves,
  button dropout, idle_max 30 (rl/rlenv.py:173, the default: 31 restart templates a game), moves drawn by
  random_legal from the masks, 300 decisions, every output every decision and `info` at every done;
* the CPU build's configuration (64 NROM consoles, raw pads, sticky) for its 500 decisions, every console every 50
  decisions;
* the GPU configuration (8192 NROM consoles, raw pads, sticky) for its 1024 decisions, consoles 0-63 and 8128-8191
  every 64 decisions;
* the divergence/mapper stress configuration (16384 MMC3 consoles, two rounds of waves, translated) for its 512
  decisions with its frames 6-bit packed on the device every decision, the packed bytes of consoles 0-31 and
  16352-16383 compared with the oracle's packer on the oracle's frames every 64 decisions;
* the rollout configuration (8192 NROM consoles, Geometric(1/2000) ends, 20 % dropped inputs) for its 128 decisions
  through the pinned-host rollout store (rl/hostobs.py): each decision packed and copied to pinned host rows, and
  the host rows of consoles 0-63 and 4096-4159 unpacked and compared with the oracle's frames.

The synthetic carts count frames in 8-bit RAM counters that wrap every 64 decisions, so these lengths reach states
(IRQ lines, CHR bank sequences, restart templates deep in the idle range) that the shorter tests sample once."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import HIP_LIB, ORACLE_LIB, oracle, ptr
from rl import synth
from rl.actions import random_legal
from rl.hostobs import RolloutStore
from rl.rlenv import GAMES, RlEnv
from test_env_games import roms
from test_gpu_parity import OUTS
from test_gpu_paths import subset_run, tptr


@pytest.mark.gpu
def test_reference_equality_gate_shape():
    """rl/tests/gpu_check.py equality(steps=300, per_game=4): the reference compares obs, emph, reward, done, masks,
    timeline, pads, events and parts every step, and info at each done; this also compares the RAM hash and the
    console records every 50 decisions."""
    print('case: 12 games x 4 consoles, sticky, dropout, idle_max 30, random_legal moves, 300 decisions', flush=True)
    kw = dict(seed=11, sticky=True, idle_max=30, dropout=True, ram_hash=True, roms=roms())
    counts = {g: 4 for g in GAMES}
    gpu = RlEnv(counts, device='cuda', lib_path=HIP_LIB, **kw)
    cpu = RlEnv(counts, device='cpu', lib_path=ORACLE_LIB, **kw)
    gpu.start()
    cpu.start()
    gen = torch.Generator().manual_seed(11)
    dones = 0
    for t in range(301):
        torch.cuda.synchronize()
        for k in OUTS:
            a, b = getattr(cpu, k).numpy(), getattr(gpu, k).cpu().numpy()
            if not np.array_equal(a, b):
                envs = np.unique(np.argwhere(a != b)[:, 0])
                raise AssertionError(f'decision {t}: {k} differs in envs {envs[:8].tolist()}')
        d = cpu.done.numpy().astype(bool)
        if t and d.any():
            dones += int(d.sum())
            assert np.array_equal(cpu.info.numpy()[d], gpu.info.cpu().numpy()[d]), f'decision {t}: info'
        if t % 50 == 0:
            for gi in range(len(GAMES)):
                assert np.array_equal(cpu.consoles(gi), gpu.consoles(gi)), (t, GAMES[gi])
        if t == 300:
            break
        act = random_legal(cpu.masks, gen)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        cpu.step()
        gpu.step()
    print(f'  {dones} finished episodes', flush=True)
    assert dones > 0


@pytest.mark.gpu
def test_cpu_config_full_length():
    print('case: NROM seed 1, 64 consoles, raw pads, sticky, 500 decisions, every console every 50', flush=True)
    from test_gpu_parity import pair, run
    cpu, gpu = pair(64, synth.nrom_cart(1), seed=1, sticky=True, idle_max=0, dropout=False, pad_mode=True)
    run(cpu, gpu, 500, 72, True, check_every=50)


@pytest.mark.gpu
def test_gpu_config_full_length():
    print('case: NROM seed 1, 8192 consoles, sticky, 1024 decisions, consoles 0-63 and 8128-8191 every 64',
          flush=True)
    subset_run(8192, synth.nrom_cart(1), [(0, 64), (8128, 8192)], 1024, 71, check_every=64, seed=1, sticky=True,
               idle_max=0, dropout=False, pad_mode=True)


@pytest.mark.gpu
def test_mmc3_stress_config_full_length_packed():
    print('case: MMC3 seed 1, 16384 consoles, translated, 512 decisions packed every decision, consoles 0-31 and '
          '16352-16383 every 64', flush=True)
    n, ranges = 16384, [(0, 32), (16352, 16384)]
    kw = dict(seed=3, sticky=False, idle_max=0, dropout=False, pad_mode=True, ram_hash=True,
              roms={'smb': synth.mmc3_cart(1)})
    gpu = RlEnv({'smb': n}, device='cuda', lib_path=HIP_LIB, **kw)
    gpu.jit_wait()
    assert gpu.jit_status(0)['state'] == 'loaded'
    cpu = RlEnv({'smb': n}, device='cpu', lib_path=ORACLE_LIB, **kw)
    per = 4 * 224 * 240 * 3 // 4
    packed = torch.empty(n * per, dtype=torch.uint8, device='cuda')
    rows = torch.cat([torch.arange(a, b) for a, b in ranges])
    g = torch.Generator().manual_seed(72)
    gpu.start()
    cpu.start()
    for t in range(512):
        act = torch.randint(0, 256, (n,), generator=g, dtype=torch.int16)
        gpu.actions.copy_(act.cuda())
        cpu.actions.copy_(act)
        gpu.step()
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert gpu.lib.rl_pack6(tptr(gpu.obs), tptr(packed), gpu.obs.numel(), s) == 0
        for a, b in ranges:
            cpu.step_range(0, a, b - a, cpu.obs, cpu.emph)
        if (t + 1) % 64:
            continue
        torch.cuda.synchronize()
        src = np.ascontiguousarray(cpu.obs[rows].numpy())
        want = np.empty(src.size * 3 // 4, np.uint8)
        assert oracle().rl_pack6(ptr(src), ptr(want), src.size, None) == 0
        got = packed.view(n, per)[rows.cuda()].cpu().numpy().reshape(-1)
        assert np.array_equal(got, want), f'decision {t}: packed frames differ'
        for k in OUTS:
            assert np.array_equal(getattr(cpu, k)[rows].numpy(), getattr(gpu, k)[rows.cuda()].cpu().numpy()), (t, k)
    for a, b in ranges:
        assert np.array_equal(cpu.consoles(0, a, b - a), gpu.consoles(0, a, b - a)), (a, b)


@pytest.mark.gpu
def test_rollout_config_full_length_through_pinned_host():
    print('case: NROM seed 1, 8192 consoles, ends 1/2000, dropout 20%, 128 decisions through the pinned-host store, '
          'consoles 0-63 and 4096-4159 every decision', flush=True)
    n, ranges = 8192, [(0, 64), (4096, 4160)]
    kw = dict(seed=2, sticky=True, idle_max=0, dropout=True, pad_mode=True, end_prob=1 / 2000, dropout_gap=1 / 60,
              ram_hash=True, roms={'smb': synth.nrom_cart(1)})
    gpu = RlEnv({'smb': n}, device='cuda', lib_path=HIP_LIB, **kw)
    gpu.jit_wait()
    cpu = RlEnv({'smb': n}, device='cpu', lib_path=ORACLE_LIB, **kw)
    store = RolloutStore(gpu.lib, 1, n, 'cuda', 1, regions=1, ring=2, pack6=True)   # host rows 0 and 1, in turn
    emph = torch.zeros(n, 4, 224, dtype=torch.uint8, device='cuda')
    rows = torch.cat([torch.arange(a, b) for a, b in ranges]).numpy()
    g = torch.Generator().manual_seed(73)
    gpu.bind_obs(store.target(0), emph)
    gpu.start()
    cpu.start()
    ends = 0
    for t in range(128):
        act = torch.randint(0, 256, (n,), generator=g, dtype=torch.int16)
        gpu.bind_obs(store.target(t), emph)
        gpu.actions.copy_(act.cuda())
        cpu.actions.copy_(act)
        gpu.step()
        store.commit(0, t % 2)
        for a, b in ranges:
            cpu.step_range(0, a, b - a, cpu.obs, cpu.emph)
        torch.cuda.synchronize()
        host = np.ctypeslib.as_array((ctypes.c_uint8 * (n * store.row_bytes)).from_address(store.row_address(0, t % 2)))
        got_packed = np.ascontiguousarray(host.reshape(n, store.row_bytes)[rows]).reshape(-1)
        got = np.empty(got_packed.size // 3 * 4, np.uint8)
        assert oracle().rl_unpack6(ptr(got_packed), ptr(got), got.size, None) == 0
        assert np.array_equal(got, cpu.obs[torch.from_numpy(rows)].numpy().reshape(-1)), f'decision {t}: host rows'
        for k in ('emph', 'reward', 'done', 'masks', 'timeline', 'pads', 'events', 'info', 'parts', 'ram_hash'):
            want = getattr(cpu, k)[torch.from_numpy(rows)].numpy()
            got_k = (emph if k == 'emph' else getattr(gpu, k))[torch.from_numpy(rows).cuda()].cpu().numpy()
            assert np.array_equal(want, got_k), (t, k)
        ends += int(cpu.done[torch.from_numpy(rows)].sum())
    store.close()
    for a, b in ranges:
        assert np.array_equal(cpu.consoles(0, a, b - a), gpu.consoles(0, a, b - a)), (a, b)
