"""Level starts and places, HIP library vs the CPU oracle, bit for bit: the level-event claims and saves
(k_finish + k_archive), restarts from saved level starts with their idle frames emulated (k_reset_copy + the idle
pass of k_emu_w), weighted plans over places, and the start/level/progress outputs; the archive is compared through
the exact-resume blob."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import HIP_LIB, ORACLE_LIB
from rl import synth
from rl.rlenv import RlEnv
from test_gpu_parity import OUTS

RIGHT, DOWN, A = 128, 32, 1


def pair(n, **kw):
    cart = synth.smb_like_cart(2)
    cpu = RlEnv({'smb': n}, device='cpu', roms={'smb': cart}, lib_path=ORACLE_LIB, ram_hash=True, **kw)
    gpu = RlEnv({'smb': n}, device='cuda', roms={'smb': cart}, lib_path=HIP_LIB, ram_hash=True, **kw)
    return cpu, gpu


def compare(cpu, gpu, where):
    torch.cuda.synchronize()
    for k in OUTS + ('start_level', 'level_now'):
        a, b = getattr(cpu, k).numpy(), getattr(gpu, k).cpu().numpy()
        if not np.array_equal(a, b):
            bad = np.argwhere(a != b)
            raise AssertionError(f'{where}: {k} differs at {len(bad)} places, first {bad[:3].tolist()}')
    a, b = cpu.progress_now.numpy(), gpu.progress_now.cpu().numpy()
    assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)]), where
    ca, cb = cpu.consoles(0), gpu.consoles(0)
    if not np.array_equal(ca, cb):
        env, off = np.argwhere(ca != cb)[0]
        raise AssertionError(f'{where}: console record {env} differs first at byte 0x{off:x}')


def set_end(env, p):
    env.lib.rlenv_set_end_prob.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
    env.lib.rlenv_set_end_prob(env.h, min(int(p * 2 ** 32), 2 ** 32 - 1))


def pads(n, t, g):
    """Mostly Right (A now and then); every third env holds Down for decisions 2..7 first (a death)."""
    p = torch.full((n,), RIGHT, dtype=torch.int16) | (torch.rand(n, generator=g) < 0.3).to(torch.int16) * A
    for k in range(0, n, 3):
        if 2 <= t < 8:
            p[k] = DOWN
    return p


def run_pair(cpu, gpu, t0, steps, g, check_every=1):
    for t in range(t0, t0 + steps):
        act = pads(cpu.n, t, g)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        cpu.step()
        gpu.step()
        if (t + 1) % check_every == 0:
            compare(cpu, gpu, f'step {t}')


@pytest.mark.gpu
def test_level_starts_claims_restarts_and_idle_frames():
    print('case: SMB-like cart seed 2, 12 consoles, level_cap 4, idle 0..3, 110 decisions to level 1, then '
          'p(level start) 0.7 with Geometric(1/5) ends for 30 decisions', flush=True)
    cpu, gpu = pair(12, seed=31, sticky=True, idle_max=3, dropout=True, pad_mode=True, level_cap=4)
    g = torch.Generator().manual_seed(4)
    cpu.start()
    gpu.start()
    compare(cpu, gpu, 'start')
    run_pair(cpu, gpu, 0, 110, g, check_every=10)
    assert cpu.saved_levels() == gpu.saved_levels() and 1 in cpu.saved_levels()['smb']
    for e in (cpu, gpu):
        e.set_level_prob(0.7)
        set_end(e, 1 / 5)
    run_pair(cpu, gpu, 110, 30, g)
    assert (cpu.start_level.numpy() >= 0).any(), 'no episode started from a level start'
    assert np.array_equal(cpu.state_dict()['env'], gpu.state_dict()['env'])


@pytest.mark.gpu
def test_places_weighted_plan():
    print('case: SMB-like cart seed 2, 8 consoles, level_cap 5 / level slots 2, place saves, weighted plan over '
          'places, Geometric(1/4) ends, 24 decisions', flush=True)
    cpu, gpu = pair(8, seed=32, sticky=False, idle_max=2, dropout=False, pad_mode=True, level_cap=5, level_slots=2)
    g = torch.Generator().manual_seed(5)
    cpu.start()
    gpu.start()
    run_pair(cpu, gpu, 10, 12, g, check_every=4)
    env_idx = [1, 6, 3]
    slot_idx = [2, 4, 0]                                  # slot 0 is a level slot: skipped
    cpu.place_save(0, torch.tensor(env_idx, dtype=torch.int32), torch.tensor(slot_idx, dtype=torch.int32))
    env_d = torch.tensor(env_idx, dtype=torch.int32, device='cuda')
    slot_d = torch.tensor(slot_idx, dtype=torch.int32, device='cuda')
    gpu.place_save(0, env_d, slot_d)
    for e in (cpu, gpu):
        e.place_copy(0, [4], [3])
        e.set_level_plan(0, 0.9, np.array([0, 0, 0.25, 0.25, 0.5]))
        set_end(e, 1 / 4)
    assert np.array_equal(cpu.state_dict()['env'], gpu.state_dict()['env'])
    run_pair(cpu, gpu, 22, 24, g)
    assert set(cpu.start_level.numpy()[cpu.done.numpy() == 1]) <= {-1, 2, 3, 4}
    assert np.array_equal(cpu.state_dict()['env'], gpu.state_dict()['env'])


@pytest.mark.gpu
def test_grown_archive_resumes_on_both_builds():
    """A HIP blob saved with 2 archive slots per game (SMB-like and a Castlevania env with its key sets), grown to 4
    by the reference's six-part formula (rl/rlenv.py:293-310), loads into a HIP env and an oracle env of 4 slots;
    both then step bit-exactly alike, with level starts drawn from the grown archive."""
    from test_env_levels import reference_grow
    print('case: smb 3 + castlevania 2 envs, archive 2 -> 4 slots, 95 + 12 decisions', flush=True)
    roms = {'smb': synth.smb_like_cart(1), 'castlevania': synth.nrom_cart(2)}
    kw = dict(roms=roms, seed=6, sticky=False, idle_max=0, dropout=False, pad_mode=True, ram_hash=True)
    a = RlEnv({'smb': 3, 'castlevania': 2}, device='cuda', lib_path=HIP_LIB, level_cap=2, **kw)
    a.start()
    for t in range(95):
        a.actions.copy_(torch.tensor([RIGHT, RIGHT | A, RIGHT, 0, RIGHT], dtype=torch.int16, device='cuda'))
        a.step()
    assert 1 in a.saved_levels()['smb']
    sd = a.state_dict()
    lays = [a.level_layout(g) for g in range(2)]
    cpu = RlEnv({'smb': 3, 'castlevania': 2}, device='cpu', lib_path=ORACLE_LIB, level_cap=4, **kw)
    gpu = RlEnv({'smb': 3, 'castlevania': 2}, device='cuda', lib_path=HIP_LIB, level_cap=4, **kw)
    grown = reference_grow(sd['env'], lays, 2, 4)
    for x in (cpu, gpu):
        x.load_state_dict(dict(sd, env=grown, level_cap=4))
        x.set_level_prob(0.5)
        set_end(x, 1 / 3)
    assert np.array_equal(cpu.state_dict()['env'], gpu.state_dict()['env'])
    g = torch.Generator().manual_seed(7)
    starts = 0
    for t in range(12):
        act = torch.randint(0, 256, (5,), generator=g, dtype=torch.int16)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        cpu.step()
        gpu.step()
        torch.cuda.synchronize()
        for k in OUTS + ('start_level', 'level_now'):
            assert np.array_equal(getattr(cpu, k).numpy(), getattr(gpu, k).cpu().numpy()), (t, k)
        starts += int(((cpu.start_level >= 0) & (cpu.done > 0)).sum())
    assert starts > 0
    assert np.array_equal(cpu.state_dict()['env'], gpu.state_dict()['env'])
