"""Translated kernels (ghostrun-lab_amd/csrc/jit.h) against the CPU oracle: the decision frames of a fixed-PRG cart
run the kernel compiled from its translated blocks, and every output and every console record must still equal the
oracle's, bit for bit (the reference's own check is rl/tests/gpu_check.py:28-53: every output every step). Each case
forces the translation (RLENV_JIT=sync) on a small env and asserts that it was loaded; the carts cover what ends a
block early or keeps an instruction out of one: the idle JMP-to-self loop and NMI-driven logic (SMB-like cart), DMC
events inside bursts, an unofficial opcode (the fault end), writes to ROM (CNROM bank switches, with and without bus
conflicts), instruction-budget stops, and the two variants (frames drawn from frame banks in a one-game env, from
the records in a two-game env)."""
import os

import numpy as np
import pytest
import torch

from helpers import HIP_LIB, ORACLE_LIB
from rl import synth
from rl.rlenv import RlEnv
from test_gpu_parity import compare, pair, run


def translated_pair(n, cart, **kw):
    os.environ['RLENV_JIT'] = 'sync'
    try:
        cpu, gpu = pair(n, cart, **kw)
    finally:
        del os.environ['RLENV_JIT']
    st = gpu.jit_status(0)
    assert st['state'] == 'loaded' and st['blocks'] > 0 and st['instructions'] > 0, st
    gpu.jit_wait()
    return cpu, gpu, st


@pytest.mark.gpu
def test_translated_benchmark_cart():
    print('case: translated NROM seed 1 (the benchmark cart), 16 consoles, raw pads, sticky, 24 decisions',
          flush=True)
    cpu, gpu, st = translated_pair(16, synth.nrom_cart(1), seed=5, sticky=True, idle_max=0, dropout=False,
                                   pad_mode=True)
    assert st['frame_bank'] and not st['banked']   # one game, one round of waves: frames drawn from frame banks
    run(cpu, gpu, 24, 0, True)


@pytest.mark.gpu
def test_translated_modes_cart():
    print('case: translated modes cart seed 2, 16 consoles, raw pads, sticky, 20 decisions (every sprite and mask '
          'mode, one a frame)', flush=True)
    cpu, gpu, st = translated_pair(16, synth.modes_cart(2), seed=12, sticky=True, idle_max=0, dropout=False,
                                   pad_mode=True)
    assert st['frame_bank'] and not st['banked']
    run(cpu, gpu, 20, 6, True)


@pytest.mark.gpu
def test_translated_vblank_io_cart():
    print('case: translated vblank I/O cart seed 2, 16 consoles, raw pads, sticky, 20 decisions (every PPU register '
          'written between vblank and the pre-render line, nested NMIs)', flush=True)
    cpu, gpu, st = translated_pair(16, synth.vblank_io_cart(2), seed=14, sticky=True, idle_max=0, dropout=False,
                                   pad_mode=True)
    assert st['frame_bank'] and not st['banked']
    run(cpu, gpu, 20, 6, True)


@pytest.mark.gpu
def test_translated_smb_like_idle_loop_and_ends():
    print('case: translated SMB-like seed 2, 24 consoles, raw pads, level end 0, Geometric(1/16) ends, idle 0..3, '
          '40 decisions', flush=True)
    cpu, gpu, _ = translated_pair(24, synth.smb_like_cart(2), seed=12, sticky=True, idle_max=3, dropout=True,
                                  pad_mode=True, end_prob=1 / 16, dropout_gap=0.05)
    cpu.set_episode_level_end(0)
    gpu.set_episode_level_end(0)
    run(cpu, gpu, 40, 4, True)


@pytest.mark.gpu
def test_translated_dmc_cart():
    print('case: translated DMC cart seed 1, 16 consoles, raw pads, sticky, 24 decisions', flush=True)
    cpu, gpu, _ = translated_pair(16, synth.dmc_cart(1), seed=31, sticky=True, idle_max=2, dropout=False,
                                  pad_mode=True)
    run(cpu, gpu, 24, 31, True)


@pytest.mark.gpu
def test_translated_fault_cart():
    print('case: translated fault cart, 8 consoles, 12 decisions (end reason 5 every episode)', flush=True)
    cpu, gpu, _ = translated_pair(8, synth.fault_cart(3), seed=32, sticky=False, idle_max=0, dropout=False,
                                  pad_mode=True)
    run(cpu, gpu, 12, 32, True)


@pytest.mark.gpu
@pytest.mark.parametrize('conflicts', [False, True])
def test_translated_cnrom_bank_switches(conflicts):
    print(f'case: translated CNROM seed 2, bus conflicts {conflicts}, 16 consoles, Geometric(1/8) ends, 16 decisions',
          flush=True)
    cpu, gpu, _ = translated_pair(16, synth.cnrom_cart(2, conflicts=conflicts), seed=19, sticky=True, idle_max=1,
                                  dropout=True, pad_mode=True, end_prob=1 / 8)
    run(cpu, gpu, 16, 5, True)


@pytest.mark.gpu
def test_translated_status_polls():
    """The poll cart (NMI off) waits every frame for vblank and for the sprite-0 flag to clear and to be set by polling
    $2002; the translation takes each poll's repeated iterations within a burst at once (jit.h jit_poll_skip), and
    the consoles, instruction counter and cycles included, must still equal the oracle's."""
    print('case: translated poll cart seed 1, 16 consoles, raw pads, sticky, Geometric(1/8) ends, 20 decisions',
          flush=True)
    cpu, gpu, _ = translated_pair(16, synth.poll_cart(1), seed=53, sticky=True, idle_max=1, dropout=True,
                                  pad_mode=True, end_prob=1 / 8)
    run(cpu, gpu, 20, 53, True)


@pytest.mark.gpu
def test_translated_bmi_status_poll():
    """The poll cart's BMI variant: a pad-dependent delay ends before, inside or after vblank, then BIT $2002 / BMI
    back to itself; inside vblank the first read clears the flag and branches and the second falls through (a pass
    in about nine on the oracle). Taken at once, the repeated iterations would run the console past the next PPU
    event."""
    print('case: translated poll cart seed 1 with the BMI poll, 16 consoles, raw pads, 24 decisions', flush=True)
    cpu, gpu, _ = translated_pair(16, synth.poll_cart(1, bmi=True), seed=54, sticky=False, idle_max=0,
                                  dropout=False, pad_mode=True)
    run(cpu, gpu, 24, 54, True)


@pytest.mark.gpu
def test_translated_instruction_budget_exit():
    print('case: translated NROM seed 3, RLENV_BUDGET 3000, 8 consoles, 10 decisions', flush=True)
    os.environ['RLENV_BUDGET'] = '3000'
    try:
        cpu, gpu, _ = translated_pair(8, synth.nrom_cart(3), seed=33, sticky=True, idle_max=0, dropout=False,
                                      pad_mode=True)
    finally:
        del os.environ['RLENV_BUDGET']
    run(cpu, gpu, 10, 33, True)
    fd = cpu.consoles(0)[:, 0x18:0x1C].copy().view(np.uint32)[:, 0]
    assert (fd != 82182).any()   # some frames stopped short of vblank


@pytest.mark.gpu
def test_translated_two_games_from_the_records():
    """Two games: each game's decision frames are drawn from the records (no frame banks), the other variant."""
    print('case: translated tetris (NROM seed 6) + smb (SMB-like seed 5), 8 + 8 consoles, 16 decisions', flush=True)
    roms = {'smb': synth.smb_like_cart(5), 'tetris': synth.nrom_cart(6)}
    kw = dict(seed=35, sticky=True, idle_max=2, dropout=True, pad_mode=True, ram_hash=True, roms=roms)
    os.environ['RLENV_JIT'] = 'sync'
    try:
        gpu = RlEnv({'smb': 8, 'tetris': 8}, device='cuda', lib_path=HIP_LIB, **kw)
    finally:
        del os.environ['RLENV_JIT']
    cpu = RlEnv({'smb': 8, 'tetris': 8}, device='cpu', lib_path=ORACLE_LIB, **kw)
    for gi in range(2):
        st = gpu.jit_status(gi)
        assert st['state'] == 'loaded' and not st['frame_bank'], st
    g = torch.Generator().manual_seed(35)
    cpu.start()
    gpu.start()
    compare(cpu, gpu, 'start')
    for t in range(16):
        act = torch.randint(0, 256, (16,), generator=g, dtype=torch.int16)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        cpu.step()
        gpu.step()
        compare(cpu, gpu, f'step {t}')
    for gi in range(2):
        assert np.array_equal(cpu.consoles(gi), gpu.consoles(gi)), gi


@pytest.mark.gpu
def test_translated_equals_interpreter_at_full_size():
    """8192 consoles of the benchmark cart, sticky: the env that runs the translated kernel (a game this size is
    translated by default) and one that does not (RLENV_JIT=0) give the same outputs and records, every decision."""
    print('case: NROM seed 1, 8192 consoles, translated vs the library kernel, 12 decisions', flush=True)
    kw = dict(seed=1, sticky=True, idle_max=0, dropout=False, pad_mode=True, ram_hash=True,
              roms={'smb': synth.nrom_cart(1)})
    fast = RlEnv({'smb': 8192}, device='cuda', lib_path=HIP_LIB, **kw)
    fast.jit_wait()
    assert fast.jit_status(0)['state'] == 'loaded'
    os.environ['RLENV_JIT'] = '0'
    try:
        slow = RlEnv({'smb': 8192}, device='cuda', lib_path=HIP_LIB, **kw)
    finally:
        del os.environ['RLENV_JIT']
    assert slow.jit_status(0)['state'] == 'none'
    g = torch.Generator().manual_seed(41)
    fast.start()
    slow.start()
    for t in range(12):
        act = torch.randint(0, 256, (8192,), generator=g, dtype=torch.int16).cuda()
        fast.actions.copy_(act)
        slow.actions.copy_(act)
        fast.step()
        slow.step()
        torch.cuda.synchronize()
        for k in ('obs', 'emph', 'reward', 'done', 'ram_hash', 'pads'):
            assert torch.equal(getattr(fast, k), getattr(slow, k)), (t, k)
    assert np.array_equal(fast.consoles(0), slow.consoles(0))


@pytest.mark.gpu
@pytest.mark.parametrize('board', ['seam', 'mmc3', 'mmc1', 'uxrom', 'mmc2'])
def test_translated_banked_boards(board):
    """Banked PRG (blocks by PRG offset, a run of one 8 KB page each; jumps, calls and returns mapped at run time):
    the seam cart (code running off windows, branches across them, JMP ($04FF), code in RAM), MMC3 (scanline IRQ,
    sprite-0 split, PRG RAM), MMC1 from power-on (serial writes, CHR RAM), UxROM with bus conflicts, MMC2 latches.
    Smaller seed-generated carts than the benchmark's keep the compiles short."""
    carts = {'seam': lambda: synth.seam_cart(1, blocks=4, sub_blocks=3),
             'mmc3': lambda: synth.mmc3_cart(3, blocks=6, sub_blocks=4),
             'mmc1': lambda: synth.mmc1_cart(3, blocks=6, sub_blocks=4),
             'uxrom': lambda: synth.uxrom_cart(2, blocks=6, sub_blocks=4, conflicts=True),
             'mmc2': lambda: synth.mmc2_cart(1, blocks=6, sub_blocks=4)}
    print(f'case: translated {board} (small seed-generated cart), 16 consoles, raw pads, sticky, Geometric(1/8) '
          'ends, 16 decisions', flush=True)
    cpu, gpu, st = translated_pair(16, carts[board](), seed=50, sticky=True, idle_max=1, dropout=True, pad_mode=True,
                                   end_prob=1 / 8)
    print(f'  {st["blocks"]} blocks, {st["instructions"]} instructions, compiled in {st["compile_ms"]} ms', flush=True)
    run(cpu, gpu, 16, 51, True)


@pytest.mark.gpu
@pytest.mark.parametrize('cart', ['nrom', 'cnrom', 'smb_like', 'poll', 'modes', 'vblank_io', 'mmc3', 'mmc1', 'uxrom',
                                  'mmc2', 'seam'])
def test_translated_seed_sweep(cart):
    """Every cart generator at a seed no other translated test uses, translated (the banked boards at a smaller size,
    to keep the compiles short): sticky repeats, button dropout, idle frames and Geometric(1/10) episode ends, every
    output and record against the oracle every third decision."""
    small = dict(blocks=6, sub_blocks=4)
    make = {'nrom': lambda: synth.nrom_cart(21), 'cnrom': lambda: synth.cnrom_cart(21),
            'smb_like': lambda: synth.smb_like_cart(21), 'poll': lambda: synth.poll_cart(21),
            'modes': lambda: synth.modes_cart(21), 'vblank_io': lambda: synth.vblank_io_cart(21),
            'mmc3': lambda: synth.mmc3_cart(21, **small), 'mmc1': lambda: synth.mmc1_cart(21, **small),
            'uxrom': lambda: synth.uxrom_cart(21, **small), 'mmc2': lambda: synth.mmc2_cart(21, **small),
            'seam': lambda: synth.seam_cart(21, blocks=4, sub_blocks=3)}
    print(f'case: translated {cart} cart seed 21, 16 consoles, sticky, dropout, idle 0..1, ends 1/10, 12 decisions',
          flush=True)
    cpu, gpu, st = translated_pair(16, make[cart](), seed=21, sticky=True, idle_max=1, dropout=True, pad_mode=True,
                                   end_prob=1 / 10, dropout_gap=1 / 8)
    print(f'  {st["blocks"]} blocks, {st["instructions"]} instructions, compiled in {st["compile_ms"]} ms', flush=True)
    run(cpu, gpu, 12, 121, True, check_every=3)
