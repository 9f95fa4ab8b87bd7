"""The reward10 readers of all twelve games in the HIP library: the device tracker (rl10_run) against the reference's
own rl10_replay outputs (tests/golden/reward10_games.npz, reward10_smb.npz), and whole env steps of every game at
once, GPU vs the oracle bit for bit, with level starts and places carrying the readers' state and key sets
(k_finish, k_reset_copy, k_reset_finish, k_archive, k_place_save)."""
import ctypes
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import GOLDEN, HIP_LIB
from rl import synth
from rl.rlenv import GAMES, RlEnv
from test_env_games import KEY_CAP, all_games, roms
from test_gpu_parity import OUTS

sys.path.insert(0, str(Path(__file__).resolve().parent / 'golden'))
from reward10_ram import trajectory  # noqa: E402

FIX = np.load(GOLDEN / 'reward10_games.npz')


def tptr(t):
    return ctypes.c_void_p(t.data_ptr())


def hip():
    lib = ctypes.CDLL(str(HIP_LIB))
    lib.rl10_run.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 11
    return lib


def device_run(lib, gi, ram, frames, cap):
    """rl10_run on the GPU over ram [T, N, 2048] / frames [T, N]; outputs [N, T] like the fixtures."""
    T, N = frames.shape
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()   # noqa: E731
    ram_d, fr_d = d(ram), d(frames)
    st = torch.zeros(N * 80, dtype=torch.uint8, device='cuda')
    rd = torch.zeros(N * 120, dtype=torch.uint8, device='cuda')
    keys = torch.zeros(N * cap + 1, dtype=torch.int32, device='cuda')
    out = dict(reward=torch.zeros(T, N, dtype=torch.float64, device='cuda'),
               done=torch.zeros(T, N, dtype=torch.uint8, device='cuda'),
               events=torch.zeros(T, N, dtype=torch.int32, device='cuda'),
               level=torch.zeros(T, N, dtype=torch.int32, device='cuda'),
               deaths=torch.zeros(T, N, dtype=torch.int32, device='cuda'),
               end=torch.zeros(T, N, dtype=torch.uint8, device='cuda'))
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.rl10_run(gi, tptr(ram_d), T, N, tptr(fr_d), tptr(st), tptr(rd), tptr(keys), tptr(out['reward']),
                        tptr(out['done']), tptr(out['events']), tptr(out['level']), tptr(out['deaths']),
                        tptr(out['end']), s) == 0
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy().T for k, v in out.items()}
    res['events'] = res['events'].view(np.uint32)
    return res


@pytest.mark.gpu
def test_device_readers_match_reference_replay():
    print('case: rl10_run on the GPU, 11 games x 24 episodes x 40 steps and SMB 16 x 1024', flush=True)
    lib = hip()
    E, T = int(FIX['episodes']), int(FIX['steps'])
    for game in GAMES[1:]:
        tr = [trajectory(game, ep, T) for ep in range(E)]
        ram = np.stack([r for r, _ in tr], 1)
        frames = np.stack([f for _, f in tr], 1).astype(np.int32)
        out = device_run(lib, GAMES.index(game), ram, frames, KEY_CAP.get(game, 0))
        for k in out:
            np.testing.assert_array_equal(out[k], FIX[f'{game}_{k}'], err_msg=f'{game}: {k}')
    gold = np.load(GOLDEN / 'reward10_smb.npz')
    ram = synth.expand_ram(gold['traj'])
    frames = np.repeat(gold['frames'][:, None], ram.shape[1], 1).astype(np.int32)
    out = device_run(lib, 0, ram, frames, 0)
    for k in ('reward', 'done', 'events', 'level', 'deaths', 'end'):
        np.testing.assert_array_equal(out[k].T, gold[k], err_msg=f'smb: {k}')
    assert lib.rl10_run(12, None, 1, 1, None, None, None, None, None, None, None, None, None, None, None) != 0


def gpu_all_games(n, **kw):
    kw.setdefault('seed', 3)
    return RlEnv({g: n for g in GAMES}, device='cuda', lib_path=HIP_LIB, roms=roms(), **kw)


def compare(cpu, gpu, where):
    torch.cuda.synchronize()
    for k in OUTS + ('start_level', 'level_now'):
        a, b = getattr(cpu, k).numpy(), getattr(gpu, k).cpu().numpy()
        if not np.array_equal(a, b):
            bad = np.argwhere(a != b)
            raise AssertionError(f'{where}: {k} differs at {len(bad)} places, first {bad[:3].tolist()}')
    a, b = cpu.progress_now.numpy(), gpu.progress_now.cpu().numpy()
    assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)]), where
    for gi in range(len(GAMES)):
        if not np.array_equal(cpu.consoles(gi), gpu.consoles(gi)):
            raise AssertionError(f'{where}: console records of {GAMES[gi]} differ')


def run_pair(cpu, gpu, steps, g, check_every=1):
    """Random move ids to both; returns how many finished episodes had started from a saved slot."""
    starts = 0
    for t in range(steps):
        act = torch.randint(0, 324, (cpu.n,), generator=g, dtype=torch.int16)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        cpu.step()
        gpu.step()
        if (t + 1) % check_every == 0 or t == steps - 1:
            compare(cpu, gpu, f'step {t}')
        starts += int((cpu.start_level.numpy() >= 0).sum())
    return starts


@pytest.mark.gpu
def test_all_games_env_parity_with_level_starts_and_places():
    print('case: 12 games x 4 consoles on spec carts, level_cap 4 / level slots 2, idle 0..2, dropout, 30 '
          'decisions, places saved and copied in zelda and kage, p(level start) 0.6 for 20 decisions', flush=True)
    kw = dict(sticky=True, idle_max=2, dropout=True, ram_hash=True, level_cap=4, level_slots=2)
    cpu = all_games(4, **kw)
    gpu = gpu_all_games(4, **kw)
    g = torch.Generator().manual_seed(11)
    cpu.start()
    gpu.start()
    compare(cpu, gpu, 'start')
    run_pair(cpu, gpu, 30, g, check_every=5)
    for game in ('zelda', 'kage'):
        gi = GAMES.index(game)
        env_idx, slot_idx = [1, 3], [2, 3]
        cpu.place_save(gi, torch.tensor(env_idx, dtype=torch.int32), torch.tensor(slot_idx, dtype=torch.int32))
        gpu.place_save(gi, torch.tensor(env_idx, dtype=torch.int32, device='cuda'),
                       torch.tensor(slot_idx, dtype=torch.int32, device='cuda'))
        for e in (cpu, gpu):
            e.place_copy(gi, [3], [2])
    for e in (cpu, gpu):
        e.set_level_prob(0.6)
    assert np.array_equal(cpu.state_dict()['env'], gpu.state_dict()['env'])
    assert run_pair(cpu, gpu, 20, g) > 0, 'no episode started from a saved slot'
    assert np.array_equal(cpu.state_dict()['env'], gpu.state_dict()['env'])
