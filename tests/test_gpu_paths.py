"""HIP library vs the CPU oracle on the paths the other parity tests leave out: the DMC sample channel, the emulator
fault end, the instruction-budget exit, rlenv_step_game on a two-game env, and the benchmark shapes at full size
(8192 NROM consoles with sticky moves; the rollout shape with Geometric ends and button dropout; 16384 MMC3
consoles, two rounds of waves; twelve games of 3072 consoles on their own carts and streams), checked on console
subsets that the oracle steps with rlenv_step_range."""
import ctypes
import os

import numpy as np
import pytest
import torch

from helpers import HIP_LIB, ORACLE_LIB, oracle, ptr
from rl import synth
from rl.rlenv import RlEnv
from test_gpu_parity import OUTS, compare, pair, run


@pytest.mark.gpu
def test_dmc_channel():
    print('case: DMC cart seed 1, 16 consoles, raw pads, sticky, 24 decisions', flush=True)
    cpu, gpu = pair(16, synth.dmc_cart(1), seed=31, sticky=True, idle_max=2, dropout=False, pad_mode=True)
    run(cpu, gpu, 24, 31, True)


@pytest.mark.gpu
def test_fault_ends_episodes():
    """The fault cart faults after 3 frames of every episode: end reason 5 with reward 0, then a restart from the
    boot snapshot (rl/csrc/rlenv_core.cuh:273-301; rl/csrc/nes_machine.cuh:84-87)."""
    print('case: fault cart, 8 consoles, 12 decisions', flush=True)
    cpu, gpu = pair(8, synth.fault_cart(3), seed=32, sticky=False, idle_max=0, dropout=False, pad_mode=True)
    g = torch.Generator().manual_seed(32)
    cpu.start()
    gpu.start()
    compare(cpu, gpu, 'start')
    ends = 0
    for t in range(12):
        act = torch.randint(0, 256, (8,), generator=g, dtype=torch.int16)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        cpu.step()
        gpu.step()
        compare(cpu, gpu, f'step {t}')
        done = cpu.done.numpy().astype(bool)
        if done.any():
            assert (cpu.info.numpy()[done, 2] == 5).all() and (cpu.reward.numpy()[done] == 0).all()
            ends += int(done.sum())
    assert ends >= 8


@pytest.mark.gpu
def test_instruction_budget_exit():
    """A frame stops when its instructions reach the budget (rl/csrc/nes_machine.cuh:30, 76). The 200,000 of the
    reference is out of reach (an instruction takes at least 6 dots, a frame 89,342), so the budget is lowered
    through RLENV_BUDGET in both builds: frames end before vblank and the console falls behind its target. On the
    NROM and MMC2 carts."""
    print('case: RLENV_BUDGET 3000, NROM seed 3 and MMC2 seed 1, 8 consoles each, 10 decisions', flush=True)
    os.environ['RLENV_BUDGET'] = '3000'
    try:
        pairs = [pair(8, synth.nrom_cart(3), seed=33, sticky=True, idle_max=0, dropout=False, pad_mode=True),
                 pair(8, synth.mmc2_cart(1), seed=34, sticky=True, idle_max=0, dropout=False, pad_mode=True)]
    finally:
        del os.environ['RLENV_BUDGET']
    for cpu, gpu in pairs:
        run(cpu, gpu, 10, 33, True)
        fd = cpu.consoles(0)[:, 0x18:0x1C].copy().view(np.uint32)[:, 0]
        assert (fd != 82182).any()                       # some frames stopped short of vblank


@pytest.mark.gpu
def test_step_game_two_games():
    """rlenv_step_game (rl/csrc/rlenv.cu:247-256) on a two-game env, each game stepped on its own, its pictures into
    the whole-batch buffers."""
    print('case: games smb (SMB-like cart) + tetris (NROM cart), 8 + 8 consoles, step_game each, 12 decisions',
          flush=True)
    roms = {'smb': synth.smb_like_cart(5), 'tetris': synth.nrom_cart(6)}
    kw = dict(seed=35, sticky=True, idle_max=2, dropout=True, pad_mode=True, ram_hash=True, roms=roms)
    cpu = RlEnv({'smb': 8, 'tetris': 8}, device='cpu', lib_path=ORACLE_LIB, **kw)
    gpu = RlEnv({'smb': 8, 'tetris': 8}, device='cuda', lib_path=HIP_LIB, **kw)
    g = torch.Generator().manual_seed(35)
    cpu.start()
    gpu.start()
    for t in range(12):
        act = torch.randint(0, 256, (16,), generator=g, dtype=torch.int16)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        for gi in (1, 0) if t % 2 else (0, 1):
            cpu.step_game(gi, cpu.obs, cpu.emph)
            gpu.step_game(gi, gpu.obs, gpu.emph)
        torch.cuda.synchronize()
        for k in OUTS:
            assert np.array_equal(getattr(cpu, k).numpy(), getattr(gpu, k).cpu().numpy()), (t, k)
        for gi in (0, 1):
            assert np.array_equal(cpu.consoles(gi), gpu.consoles(gi)), (t, gi)


def tptr(t):
    return ctypes.c_void_p(t.data_ptr())


def subset_run(n, cart, ranges, decisions, act_seed, check_every=1, banked=None, **kw):
    """n consoles on the GPU, every decision of all of them; the oracle steps only the console ranges (with their own
    env indices, so their seeds and streams are the same) and every output of those consoles is compared (every
    check_every decisions, and at the last). A game of this size is translated (compiled in the background): the
    run starts once the translated kernel is loaded, so every decision runs it."""
    kw = dict(kw, ram_hash=True, roms={'smb': cart})
    gpu = RlEnv({'smb': n}, device='cuda', lib_path=HIP_LIB, **kw)
    gpu.jit_wait()
    st = gpu.jit_status(0)
    assert st['state'] == 'loaded', st
    assert banked is None or st['banked'] == banked, st
    print(f'  translated: {st["blocks"]} blocks, {st["instructions"]} instructions, compiled in {st["compile_ms"]} '
          f'ms, {st["far_jumps"]} far jumps', flush=True)
    cpu = RlEnv({'smb': n}, device='cpu', lib_path=ORACLE_LIB, **kw)
    g = torch.Generator().manual_seed(act_seed)
    gpu.start()
    cpu.start()
    rows = torch.cat([torch.arange(a, b) for a, b in ranges])
    ends = 0
    for t in range(decisions):
        act = torch.randint(0, 256, (n,), generator=g, dtype=torch.int16)
        gpu.actions.copy_(act.cuda())
        cpu.actions.copy_(act)
        gpu.step()
        for a, b in ranges:
            cpu.step_range(0, a, b - a, cpu.obs, cpu.emph)
        if (t + 1) % check_every and t != decisions - 1:
            continue
        torch.cuda.synchronize()
        for k in OUTS:
            want, got = getattr(cpu, k)[rows].numpy(), getattr(gpu, k)[rows.cuda()].cpu().numpy()
            if not np.array_equal(want, got):
                bad = np.argwhere(want != got)
                raise AssertionError(f'decision {t}: {k} differs at {len(bad)} places, first {bad[:3].tolist()}')
        ends += int(cpu.done[rows].sum())
    for a, b in ranges:
        assert np.array_equal(cpu.consoles(0, a, b - a), gpu.consoles(0, a, b - a)), (a, b)
    return gpu, cpu, ends


@pytest.mark.gpu
def test_full_size_nrom_sticky_subset():
    """The benchmark's shape: 8192 NROM consoles, raw pads uniform over 256 values, sticky p = 0.25; consoles 0-63
    and 8128-8191 against the oracle for 64 decisions."""
    print('case: NROM seed 1, 8192 consoles, sticky, 64 decisions, consoles 0-63 and 8128-8191', flush=True)
    subset_run(8192, synth.nrom_cart(1), [(0, 64), (8128, 8192)], 64, 41, seed=1, sticky=True, idle_max=0,
               dropout=False, pad_mode=True)


@pytest.mark.gpu
def test_full_size_rollout_shape_subset():
    """The rollout shape: 8192 NROM consoles, episode ends Geometric(1/2000) a decision, button dropout with a 20%
    dropped share, restarts from the boot snapshot; consoles 0-63 and 4096-4159, 48 decisions. The packed frames of
    those consoles equal the oracle's packer on the oracle's frames."""
    print('case: NROM seed 1, 8192 consoles, ends 1/2000, dropout 20%, 48 decisions, 128 consoles', flush=True)
    gpu, cpu, _ = subset_run(8192, synth.nrom_cart(1), [(0, 64), (4096, 4160)], 48, 42, seed=2, sticky=True,
                             idle_max=0, dropout=True, pad_mode=True, end_prob=1 / 2000, dropout_gap=1 / 60)
    rows = torch.cat([torch.arange(0, 64), torch.arange(4096, 4160)])
    packed = torch.empty(gpu.obs.numel() * 3 // 4, dtype=torch.uint8, device='cuda')
    assert gpu.lib.rl_pack6(tptr(gpu.obs), tptr(packed), gpu.obs.numel(), None) == 0
    torch.cuda.synchronize()
    per = gpu.obs[0].numel() * 3 // 4
    got = packed.view(-1, per)[rows.cuda()].cpu().numpy()
    src = np.ascontiguousarray(cpu.obs[rows].numpy())
    want = np.empty(src.size * 3 // 4, np.uint8)
    assert oracle().rl_pack6(ptr(src), ptr(want), src.size, None) == 0
    assert np.array_equal(got.reshape(-1), want)


@pytest.mark.gpu
def test_full_size_mmc3_two_wave_rounds_subset():
    """The stress shape: 16384 MMC3 consoles (two rounds of waves on one GPU) on the translated kernel of the full-size
    cart (its far jumps checked), independent random pads; consoles 0-31 (first round) and 16352-16383 (second round)
    against the oracle for 16 decisions."""
    print('case: MMC3 seed 1, 16384 consoles, translated, 16 decisions, consoles 0-31 and 16352-16383', flush=True)
    subset_run(16384, synth.mmc3_cart(1), [(0, 32), (16352, 16384)], 16, 43, banked=True, seed=3, sticky=False,
               idle_max=0, dropout=False, pad_mode=True)


# The twelve-games workload's carts: the SMB-like cart for the first game, then a board per game in turn, seeds 1..12.
TWELVE_BOARDS = ('smb_like', 'nrom', 'mmc1', 'uxrom', 'cnrom', 'mmc3', 'mmc2', 'nrom', 'mmc1', 'uxrom', 'cnrom', 'mmc3')


@pytest.mark.gpu
def test_full_size_twelve_games_subset():
    """The multi-game shape: 12 games x 3072 consoles, each game on its own full-size seed-generated cart and its own
    translated kernel (banked boards included), every game stepping on its own stream; in every game consoles 0-7 and
    3064-3071 against the oracle (rlenv_step_range per game) for 40 decisions (the SMB-like game's episodes end and
    restart among them), every output and, at the end, every console record. The compiled translations come from the translation cache in the build folder when it holds
    them (a compile otherwise)."""
    from rl.rlenv import GAMES
    print('case: twelve games x 3072 consoles (full-size carts, all translated), sticky, consoles 0-7 '
          'and 3064-3071 of every game, 40 decisions', flush=True)
    cache = os.path.join(os.path.dirname(HIP_LIB), 'jit_cache')
    own_cache = 'RLENV_JIT_CACHE' not in os.environ and os.path.isdir(cache)
    make = dict(smb_like=synth.smb_like_cart, nrom=synth.nrom_cart, mmc1=synth.mmc1_cart, uxrom=synth.uxrom_cart,
                cnrom=synth.cnrom_cart, mmc3=synth.mmc3_cart, mmc2=synth.mmc2_cart)
    roms = {g: make[b](1 + i) for i, (g, b) in enumerate(zip(GAMES, TWELVE_BOARDS))}
    n = 3072
    counts = {g: n for g in GAMES}
    kw = dict(seed=1, sticky=True, idle_max=0, dropout=False, pad_mode=True, ram_hash=True, roms=roms,
              boot={g: bytes(4) for g in GAMES})
    if own_cache:
        os.environ['RLENV_JIT_CACHE'] = cache
    try:
        gpu = RlEnv(counts, device='cuda', lib_path=HIP_LIB, **kw)
        gpu.jit_wait()
    finally:
        if own_cache:
            del os.environ['RLENV_JIT_CACHE']
    for gi, g in enumerate(GAMES):
        st = gpu.jit_status(gi)
        assert st['state'] == 'loaded', (g, st)
    cpu = RlEnv(counts, device='cpu', lib_path=ORACLE_LIB, **kw)
    ranges = [(0, 8), (n - 8, n)]
    rows = torch.cat([torch.arange(gi * n + a, gi * n + b) for gi in range(len(GAMES)) for a, b in ranges])
    g = torch.Generator().manual_seed(44)
    gpu.start()
    cpu.start()
    ends = 0
    for t in range(40):
        act = torch.randint(0, 256, (len(GAMES) * n,), generator=g, dtype=torch.int16)
        gpu.actions.copy_(act.cuda())
        cpu.actions.copy_(act)
        gpu.step()
        for gi in range(len(GAMES)):
            for a, b in ranges:
                cpu.step_range(gi, a, b - a, cpu.obs, cpu.emph)
        torch.cuda.synchronize()
        for k in OUTS:
            want, got = getattr(cpu, k)[rows].numpy(), getattr(gpu, k)[rows.cuda()].cpu().numpy()
            if not np.array_equal(want, got):
                bad = np.argwhere(want != got)
                raise AssertionError(f'decision {t}: {k} differs at {len(bad)} places, first {bad[:3].tolist()}')
        ends += int(cpu.done[rows].sum())
    assert ends > 0, 'no episode ended in the checked consoles'
    for gi in range(len(GAMES)):
        for a, b in ranges:
            assert np.array_equal(cpu.consoles(gi, a, b - a), gpu.consoles(gi, a, b - a)), (GAMES[gi], a, b)
