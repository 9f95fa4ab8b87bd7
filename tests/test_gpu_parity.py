"""HIP library vs the CPU oracle, every output of every decision, bit for bit (the reference's own check is
rl/tests/gpu_check.py:28-53: GPU vs CPU build, every output every step)."""
import numpy as np
import pytest
import torch

from helpers import HIP_LIB, ORACLE_LIB, REC_BYTES
from rl import synth
from rl.rlenv import RlEnv

OUTS = ('obs', 'emph', 'reward', 'done', 'masks', 'timeline', 'pads', 'events', 'info', 'parts', 'ram_hash')


def pair(n, cart, **kw):
    cpu = RlEnv({'smb': n}, device='cpu', roms={'smb': cart}, lib_path=ORACLE_LIB, ram_hash=True, **kw)
    gpu = RlEnv({'smb': n}, device='cuda', roms={'smb': cart}, lib_path=HIP_LIB, ram_hash=True, **kw)
    return cpu, gpu


def compare(cpu, gpu, where):
    torch.cuda.synchronize()
    for k in OUTS:
        a, b = getattr(cpu, k).numpy(), getattr(gpu, k).cpu().numpy()
        if not np.array_equal(a, b):
            bad = np.argwhere(a != b)
            raise AssertionError(f'{where}: {k} differs at {len(bad)} places, first {bad[:3].tolist()}')
    ca, cb = cpu.consoles(0), gpu.consoles(0)
    if not np.array_equal(ca, cb):
        env, off = np.argwhere(ca != cb)[0]
        raise AssertionError(f'{where}: console record {env} differs first at byte 0x{off:x}')


def run(cpu, gpu, steps, seed, pad_mode, check_every=1):
    g = torch.Generator().manual_seed(seed)
    cpu.start()
    gpu.start()
    compare(cpu, gpu, 'start')
    for t in range(steps):
        hi = 256 if pad_mode else 324
        act = torch.randint(0, hi, (cpu.n,), generator=g, dtype=torch.int16)
        cpu.actions.copy_(act)
        gpu.actions.copy_(act.cuda())
        cpu.step()
        gpu.step()
        if (t + 1) % check_every == 0 or t == steps - 1:
            compare(cpu, gpu, f'step {t}')


@pytest.mark.gpu
def test_nrom_raw_pads_sticky():
    print('case: NROM seed 1, 16 consoles, raw pads, sticky, 24 decisions', flush=True)
    cpu, gpu = pair(16, synth.nrom_cart(1), seed=5, sticky=True, idle_max=0, dropout=False, pad_mode=True)
    run(cpu, gpu, 24, 0, True)


@pytest.mark.gpu
def test_nrom_moves_dropout_idle_ends():
    print('case: NROM seed 2, 16 consoles, move ids, dropout, idle 0..6, Geometric(1/8) ends', flush=True)
    cpu, gpu = pair(16, synth.nrom_cart(2), seed=7, sticky=True, idle_max=6, dropout=True, end_prob=1 / 8)
    run(cpu, gpu, 24, 1, False)


@pytest.mark.gpu
def test_modes_cart_every_sprite_and_mask_mode():
    print('case: modes cart seed 1, 16 consoles, raw pads, sticky, 20 decisions (8x8 / 8x16 sprites, sprites or '
          'background off, clipped left columns, greyscale, emphasis, one mode a frame)', flush=True)
    cpu, gpu = pair(16, synth.modes_cart(1), seed=11, sticky=True, idle_max=0, dropout=False, pad_mode=True)
    run(cpu, gpu, 20, 5, True)


@pytest.mark.gpu
def test_vblank_io_cart_every_ppu_register_in_vblank():
    print('case: vblank I/O cart seed 1, 16 consoles, raw pads, sticky, 20 decisions (OAM through $2003/$2004, palette '
          'mirrors, a column with the increment of 32, register mirrors, an indexed store, nested NMIs)', flush=True)
    cpu, gpu = pair(16, synth.vblank_io_cart(1), seed=13, sticky=True, idle_max=0, dropout=False, pad_mode=True)
    run(cpu, gpu, 20, 5, True)


@pytest.mark.gpu
def test_mmc3_stress():
    print('case: MMC3 seed 3, 16 consoles, raw pads, IRQ + sprite-0 + bank switches', flush=True)
    cpu, gpu = pair(16, synth.mmc3_cart(3), seed=9, sticky=True, idle_max=0, dropout=False, pad_mode=True)
    run(cpu, gpu, 16, 2, True)


@pytest.mark.gpu
def test_mmc1_chr_ram_bank_switches():
    print('case: MMC1 seed 2, 16 consoles, 8-frame boot, raw pads, sticky, Geometric(1/8) ends, 20 decisions',
          flush=True)
    cpu, gpu = pair(16, synth.mmc1_cart(2), seed=17, sticky=True, idle_max=2, dropout=True, pad_mode=True,
                    end_prob=1 / 8, boot={'smb': bytes(8)})
    run(cpu, gpu, 20, 3, True)


@pytest.mark.gpu
@pytest.mark.parametrize('conflicts', [False, True])
def test_cnrom_chr_bank_switches(conflicts):
    print(f'case: CNROM seed 2, bus conflicts {conflicts}, 16 consoles, raw pads, sticky, Geometric(1/8) ends, '
          '16 decisions', flush=True)
    cpu, gpu = pair(16, synth.cnrom_cart(2, conflicts=conflicts), seed=19, sticky=True, idle_max=1, dropout=True,
                    pad_mode=True, end_prob=1 / 8)
    run(cpu, gpu, 16, 5, True)


@pytest.mark.gpu
@pytest.mark.parametrize('conflicts', [False, True])
def test_uxrom_prg_bank_switches(conflicts):
    print(f'case: UxROM seed 2, bus conflicts {conflicts}, 16 consoles, raw pads, sticky, Geometric(1/8) ends, '
          '16 decisions', flush=True)
    cpu, gpu = pair(16, synth.uxrom_cart(2, conflicts=conflicts), seed=23, sticky=True, idle_max=1, dropout=True,
                    pad_mode=True, end_prob=1 / 8)
    run(cpu, gpu, 16, 6, True)


@pytest.mark.gpu
def test_mmc1_from_power_on():
    print('case: MMC1 seed 3, 8 consoles, boot from power-on (CHR RAM upload in the decisions), 12 decisions',
          flush=True)
    cpu, gpu = pair(8, synth.mmc1_cart(3), seed=18, sticky=False, idle_max=0, dropout=False, pad_mode=True)
    run(cpu, gpu, 12, 4, True)


@pytest.mark.gpu
@pytest.mark.parametrize('seed', [1, 2])
def test_mmc2_latches_follow_the_fetches(seed):
    print(f'case: MMC2 seed {seed}, 16 consoles, raw pads, $FD/$FE tiles in nametables and sprites, CHR bank and '
          'mirroring rewrites, CPU-driven latch flips, 16 decisions', flush=True)
    cpu, gpu = pair(16, synth.mmc2_cart(seed), seed=20 + seed, sticky=True, idle_max=2, dropout=False, pad_mode=True)
    run(cpu, gpu, 16, 7 + seed, True)


@pytest.mark.gpu
@pytest.mark.parametrize('seed', [0, 1])
def test_mmc3_code_across_prg_windows(seed):
    print(f'case: seam cart seed {seed} (MMC3), 16 consoles, raw pads, sticky, code running off 8 KB windows, '
          'branches across them, JMP ($04FF), code in RAM, 16 decisions', flush=True)
    cpu, gpu = pair(16, synth.seam_cart(seed), seed=30 + seed, sticky=True, idle_max=1, dropout=False, pad_mode=True)
    run(cpu, gpu, 16, 11 + seed, True)


SWEEP = {'nrom': synth.nrom_cart, 'cnrom': synth.cnrom_cart, 'uxrom': synth.uxrom_cart, 'mmc1': synth.mmc1_cart,
         'mmc3': synth.mmc3_cart, 'mmc2': synth.mmc2_cart, 'smb_like': synth.smb_like_cart, 'seam': synth.seam_cart,
         'poll': synth.poll_cart, 'modes': synth.modes_cart, 'vblank_io': synth.vblank_io_cart}


@pytest.mark.gpu
@pytest.mark.parametrize('seed', [21, 22])
@pytest.mark.parametrize('cart', sorted(SWEEP))
def test_seed_sweep_every_cart_generator(cart, seed):
    """Every cart generator at two seeds no other test uses, at its default size, on the library's kernels (16
    consoles are below the translation threshold): raw pads with sticky repeats, button dropout, idle frames and
    Geometric(1/10) episode ends, every output and record against the oracle every third decision."""
    print(f'case: {cart} cart seed {seed}, 16 consoles, sticky, dropout, idle 0..1, ends 1/10, 12 decisions',
          flush=True)
    cpu, gpu = pair(16, SWEEP[cart](seed), seed=seed, sticky=True, idle_max=1, dropout=True, pad_mode=True,
                    end_prob=1 / 10, dropout_gap=1 / 8)
    run(cpu, gpu, 12, seed + 100, True, check_every=3)
