"""More HIP-vs-oracle parity: rewards and restarts, full-size console independence, the GPU extras of the ABI
(step_range, pack6/unpack6) and the standalone reward10 kernel against the reference's golden fixture."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import GOLDEN, HIP_LIB, ORACLE_LIB, oracle, ptr
from rl import synth
from rl.rlenv import RlEnv
from test_gpu_parity import compare, pair, run


def tptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.gpu
def test_smb_like_rewards_restarts_moves():
    print('case: SMB-like cart seed 1, 16 consoles, move ids, sticky, dropout, idle 0..6, 40 decisions', flush=True)
    cpu, gpu = pair(16, synth.smb_like_cart(1), seed=11, sticky=True, idle_max=6, dropout=True)
    run(cpu, gpu, 40, 3, False)


@pytest.mark.gpu
def test_smb_like_raw_pads_level_end_and_ends():
    print('case: SMB-like cart seed 2, 24 consoles, raw pads, level end 0, Geometric(1/16) ends, 40 decisions',
          flush=True)
    cpu, gpu = pair(24, synth.smb_like_cart(2), seed=12, sticky=True, idle_max=3, dropout=True, pad_mode=True,
                    end_prob=1 / 16, dropout_gap=0.05)
    cpu.set_episode_level_end(0)
    gpu.set_episode_level_end(0)
    run(cpu, gpu, 40, 4, True)


@pytest.mark.gpu
def test_boot_sequence_snapshot_and_restarts():
    """Boot pads run on the device before the snapshot (rl/csrc/rlenv_build.hpp:193-209): restarts resume after the
    cart's 4-frame boot, as the reference's recorded boot sequences do."""
    print('case: NROM seed 5, 16 consoles, boot 4 neutral + 2 pressed frames, Geometric(1/6) ends, 24 decisions',
          flush=True)
    cpu, gpu = pair(16, synth.nrom_cart(5), seed=13, sticky=True, idle_max=2, dropout=True, pad_mode=True,
                    end_prob=1 / 6, boot={'smb': bytes(4) + bytes((0x80, 0x81))})
    run(cpu, gpu, 24, 5, True)


@pytest.mark.gpu
def test_full_size_console_independence():
    """8192 consoles; with no per-console randomness (no sticky, dropout, idle or synthetic ends) a console's
    outputs depend only on its own pad stream, so consoles 0, 4095 and 8191 must equal an oracle run of those
    streams."""
    print('case: NROM seed 1, 8192 consoles x 8 decisions, consoles 0/4095/8191 vs oracle', flush=True)
    cart = synth.nrom_cart(1)
    kw = dict(seed=1, sticky=False, idle_max=0, dropout=False, pad_mode=True, ram_hash=True, roms={'smb': cart})
    gpu = RlEnv({'smb': 8192}, device='cuda', lib_path=HIP_LIB, **kw)
    gpu.jit_wait()
    cpu = RlEnv({'smb': 3}, device='cpu', lib_path=ORACLE_LIB, **kw)
    pick = torch.tensor([0, 4095, 8191])
    g = torch.Generator().manual_seed(0)
    gpu.start()
    cpu.start()
    for t in range(8):
        act = torch.randint(0, 256, (8192,), generator=g, dtype=torch.int16)
        gpu.actions.copy_(act.cuda())
        cpu.actions.copy_(act[pick])
        gpu.step()
        cpu.step()
        torch.cuda.synchronize()
        for k in ('obs', 'emph', 'reward', 'done', 'ram_hash', 'pads'):
            assert torch.equal(getattr(gpu, k)[pick.cuda()].cpu(), getattr(cpu, k)), (t, k)


@pytest.mark.gpu
def test_resume_blob_equals_oracle_and_cross_loads():
    """The exact-resume blob (rlenv_save) of the HIP build equals the oracle's byte for byte, and an oracle blob
    loaded into a fresh HIP env continues exactly as the oracle does (the reference's resume check is
    rl/tests/gpu_check.py:56-74)."""
    print('case: SMB-like cart seed 4, 12 consoles, ends + dropout + idle, save after 10, 10 more decisions',
          flush=True)
    kw = dict(seed=21, sticky=True, idle_max=3, dropout=True, pad_mode=True, end_prob=0.1)
    cart = synth.smb_like_cart(4)
    cpu, gpu = pair(12, cart, **kw)
    run(cpu, gpu, 10, 6, True)
    sd_cpu, sd_gpu = cpu.state_dict(), gpu.state_dict()
    assert sd_cpu['env'].shape == sd_gpu['env'].shape
    assert np.array_equal(sd_cpu['env'], sd_gpu['env'])
    fresh = RlEnv({'smb': 12}, device='cuda', roms={'smb': cart}, lib_path=HIP_LIB, ram_hash=True, **kw)
    fresh.load_state_dict(sd_cpu)
    g = torch.Generator().manual_seed(8)
    for t in range(10):
        act = torch.randint(0, 256, (12,), generator=g, dtype=torch.int16)
        cpu.actions.copy_(act)
        fresh.actions.copy_(act.cuda())
        cpu.step()
        fresh.step()
        torch.cuda.synchronize()
        for k in ('obs', 'emph', 'reward', 'done', 'masks', 'timeline', 'pads', 'events', 'parts', 'ram_hash'):
            assert torch.equal(getattr(cpu, k), getattr(fresh, k).cpu()), (t, k)
        d = cpu.done.bool()                              # info is written at episode end and is not in the blob
        assert torch.equal(cpu.info[d], fresh.info.cpu()[d]), t
        assert np.array_equal(cpu.consoles(0), fresh.consoles(0)), t


@pytest.mark.gpu
def test_step_range_equals_step():
    print('case: SMB-like cart, 16 consoles, step vs two step_range halves, 12 decisions', flush=True)
    kw = dict(seed=5, sticky=True, idle_max=2, dropout=True, pad_mode=True, roms={'smb': synth.smb_like_cart(3)})
    a = RlEnv({'smb': 16}, device='cuda', lib_path=HIP_LIB, **kw)
    b = RlEnv({'smb': 16}, device='cuda', lib_path=HIP_LIB, **kw)
    a.start()
    b.start()
    g = torch.Generator().manual_seed(1)
    for t in range(12):
        act = torch.randint(0, 256, (16,), generator=g, dtype=torch.int16).cuda()
        a.actions.copy_(act)
        b.actions.copy_(act)
        a.step()
        b.step_range(0, 0, 5, b.obs, b.emph)
        b.step_range(0, 5, 11, b.obs, b.emph)
        torch.cuda.synchronize()
        for k in ('obs', 'emph', 'reward', 'done', 'masks', 'timeline', 'pads', 'events'):
            assert torch.equal(getattr(a, k), getattr(b, k)), (t, k)


@pytest.mark.gpu
def test_pack6_unpack6_on_device():
    print('case: pack6/unpack6, 2 x 4 x 224 x 240 frames + odd count', flush=True)
    lib = ctypes.CDLL(str(HIP_LIB))
    lib.rl_pack6.argtypes = lib.rl_unpack6.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                                       ctypes.c_void_p]
    g = torch.Generator().manual_seed(0)
    for n in (2 * 4 * 224 * 240, 4 * 13):
        px = torch.randint(0, 64, (n,), generator=g, dtype=torch.uint8)
        d = px.cuda()
        packed = torch.empty(n // 4 * 3, dtype=torch.uint8, device='cuda')
        back = torch.empty(n, dtype=torch.uint8, device='cuda')
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.rl_pack6(tptr(d), tptr(packed), n, s) == 0
        assert lib.rl_unpack6(tptr(packed), tptr(back), n, s) == 0
        torch.cuda.synchronize()
        want = np.zeros(n // 4 * 3, np.uint8)
        pxn = px.numpy()
        assert oracle().rl_pack6(ptr(pxn), ptr(want), n, None) == 0
        assert np.array_equal(packed.cpu().numpy(), want) and torch.equal(back.cpu(), px)
    assert lib.rl_pack6(tptr(d), tptr(packed), 6, s) != 0


@pytest.mark.gpu
def test_reward10_kernel_matches_reference_fixture_and_oracle():
    print('case: rl10_smb_run, golden 16 x 1024 and synthetic 512 x 256', flush=True)
    lib = ctypes.CDLL(str(HIP_LIB))
    lib.rl10_smb_run.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    gold = np.load(GOLDEN / 'reward10_smb.npz')
    traj = torch.from_numpy(gold['traj']).cuda()        # [1024, 16, 16]; the first step covers 8 frames
    T, N = traj.shape[:2]
    state = torch.zeros(N * 80, dtype=torch.uint8, device='cuda')
    rew = torch.zeros(T, N, dtype=torch.float32, device='cuda')
    done = torch.zeros(T, N, dtype=torch.uint8, device='cuda')
    assert lib.rl10_smb_run(tptr(traj[:1].contiguous()), 1, N, 8, tptr(state), tptr(rew), tptr(done), s) == 0
    assert lib.rl10_smb_run(tptr(traj[1:].contiguous()), T - 1, N, 4, tptr(state), tptr(rew[1:]), tptr(done[1:]),
                            s) == 0
    torch.cuda.synchronize()
    assert np.array_equal(rew.cpu().numpy(), gold['reward'].astype(np.float32))
    assert np.array_equal(done.cpu().numpy(), gold['done'])
    ram = synth.smb_ram15(21, 512, 256)
    T, N = ram.shape[:2]
    want_r = np.zeros((T, N), np.float32)
    want_d = np.zeros((T, N), np.uint8)
    st = np.zeros(N * 80, np.uint8)
    assert oracle().rl10_smb_run(ptr(ram), T, N, 4, ptr(st), ptr(want_r), ptr(want_d), None) == 0
    d_ram = torch.from_numpy(ram).cuda()
    state = torch.zeros(N * 80, dtype=torch.uint8, device='cuda')
    rew = torch.zeros(T, N, dtype=torch.float32, device='cuda')
    done = torch.zeros(T, N, dtype=torch.uint8, device='cuda')
    assert lib.rl10_smb_run(tptr(d_ram), T, N, 4, tptr(state), tptr(rew), tptr(done), s) == 0
    torch.cuda.synchronize()
    assert np.array_equal(rew.cpu().numpy(), want_r) and np.array_equal(done.cpu().numpy(), want_d)
    assert np.array_equal(state.cpu().numpy(), st)


def stress_ram15(seed, n, steps, level_up_at):
    """SMB RAM trajectories that reach every path of the tracker: synth.smb_ram15 with seeded overlays - a fifth of
    the envs with a stuck position (idle frames up to the stall end), level steps and skips (end reason 3), wins (2)
    and game overs (1), dying routines and pits, lives lost, score jumps past the cap and the level's budget, steps
    out of play, and at step `level_up_at` a level step with the position invalid (the best progress left unset, as
    update leaves it, at the end of a call)."""
    ram = synth.smb_ram15(seed, n, steps)
    rng = np.random.default_rng([0x53545245, seed])
    stuck = rng.random(n) < 0.2
    ram[:, stuck, 1:3] = ram[:1, stuck, 1:3]
    u = rng.random((steps, n, 8))
    lvl = ram[:, :, 5].astype(np.int64) + np.cumsum((u[:, :, 0] < 4e-3) + 2 * (u[:, :, 1] < 5e-4), axis=0)
    ram[:, :, 5] = (lvl & 3).astype(np.uint8)
    ram[:, :, 6] = np.minimum(ram[:, :, 6].astype(np.int64) + (lvl >> 2), 7).astype(np.uint8)
    win = u[:, :, 2] < 2e-4                                     # mode 2 in world 8 (index 7)
    ram[:, :, 7] = np.where(win, 2, np.where(u[:, :, 2] > 1 - 3e-4, 3, ram[:, :, 7]))
    ram[:, :, 6] = np.where(win, 7, ram[:, :, 6])
    ram[:, :, 0] = np.where(u[:, :, 3] < 0.02, 6, np.where(u[:, :, 3] > 0.99, 11, ram[:, :, 0]))
    ram[:, :, 3] = np.where(u[:, :, 4] < 0.01, 2, ram[:, :, 3])
    ram[:, :, 4] = (ram[:, :, 4].astype(np.int64) - (u[:, :, 5] < 2e-3)).astype(np.uint8)
    ram[:, :, 8] = np.where(u[:, :, 6] < 0.01, 1, ram[:, :, 8])
    jump = u[:, :, 7] < 5e-3
    ram[:, :, 9:11] = np.where(jump[:, :, None], rng.integers(0, 10, (steps, n, 2)), ram[:, :, 9:11])
    ram[level_up_at, :, 5] = (ram[level_up_at, :, 5] + 1) & 3
    ram[level_up_at, :, 0] = 0
    return ram


@pytest.mark.gpu
def test_reward10_kernel_every_path_over_split_calls():
    """rl10_smb_run (the tracker in three passes: signals in parallel, the state env by env, the rewards in
    parallel) against the oracle's tracker on trajectories that reach every end (level skip, win, game over, stall),
    deaths, score budgets and rollbacks, over calls of 37, 1, 100 and 118 steps (the state carried between them, a
    call ending right after a level step that left the best progress unset), 300 envs (a partial wave), 64 frames a
    step (the stall limit within reach)."""
    print('case: rl10_smb_run, 300 envs x 256 steps in calls of 37/1/100/118, every tracker path', flush=True)
    lib = ctypes.CDLL(str(HIP_LIB))
    lib.rl10_smb_run.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    N, T, frames = 300, 256, 64
    ram = stress_ram15(5, N, T, level_up_at=36)
    st_c = np.zeros(N * 80, np.uint8)
    st_g = torch.zeros(N * 80, dtype=torch.uint8, device='cuda')
    t0 = 0
    for n_steps in (37, 1, 100, 118):
        part = np.ascontiguousarray(ram[t0:t0 + n_steps])
        want_r = np.zeros((n_steps, N), np.float32)
        want_d = np.zeros((n_steps, N), np.uint8)
        assert oracle().rl10_smb_run(ptr(part), n_steps, N, frames, ptr(st_c), ptr(want_r), ptr(want_d), None) == 0
        rew = torch.zeros(n_steps, N, dtype=torch.float32, device='cuda')
        done = torch.zeros(n_steps, N, dtype=torch.uint8, device='cuda')
        assert lib.rl10_smb_run(tptr(torch.from_numpy(part).cuda()), n_steps, N, frames, tptr(st_g), tptr(rew),
                                tptr(done), s) == 0
        torch.cuda.synchronize()
        assert np.array_equal(rew.cpu().numpy(), want_r), (t0, n_steps)
        assert np.array_equal(done.cpu().numpy(), want_d), (t0, n_steps)
        assert np.array_equal(st_g.cpu().numpy(), st_c), (t0, n_steps)
        t0 += n_steps
    ends = st_c.reshape(N, 80)[:, 4]          # Rl10State.end_reason
    assert set(np.unique(ends).tolist()) >= {1, 2, 3, 4}, np.unique(ends, return_counts=True)
