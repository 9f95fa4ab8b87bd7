"""rlenv_step_static: rlenv_step with every game's restart queue in the library's static device scratch (an entry
point that allocates nothing) gives the same outputs and console records as rlenv_step, on two envs in a row, the
second smaller (the scratch keeps the first one's queue)."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import HIP_LIB
from rl import synth
from rl.rlenv import RlEnv
from test_gpu_parity import OUTS


@pytest.mark.gpu
def test_step_static_equals_step():
    lib = ctypes.CDLL(str(HIP_LIB))
    lib.rlenv_step_static.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    for n, cart, seed in ((48, synth.nrom_cart(1), 61), (16, synth.smb_like_cart(2), 62)):
        print(f'case: {n} consoles, seed {seed}, Geometric(1/4) ends, rlenv_step vs rlenv_step_static', flush=True)
        kw = dict(seed=seed, sticky=True, idle_max=2, dropout=True, pad_mode=True, end_prob=1 / 4, ram_hash=True,
                  roms={'smb': cart})
        a = RlEnv({'smb': n}, device='cuda', lib_path=HIP_LIB, **kw)
        b = RlEnv({'smb': n}, device='cuda', lib_path=HIP_LIB, **kw)
        g = torch.Generator().manual_seed(seed)
        a.start()
        b.start()
        ends = 0
        for t in range(8):
            act = torch.randint(0, 256, (n,), generator=g, dtype=torch.int16).cuda()
            a.actions.copy_(act)
            b.actions.copy_(act)
            a.step()
            assert lib.rlenv_step_static(ctypes.c_void_p(b.h), b._stream()) == 0, lib.rlenv_error()
            torch.cuda.synchronize()
            for k in OUTS:
                assert torch.equal(getattr(a, k), getattr(b, k)), (n, t, k)
            ends += int(a.done.sum())
        assert np.array_equal(a.consoles(0), b.consoles(0))
        assert ends > 0
