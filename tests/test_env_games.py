"""The twelve reward10 games inside the oracle's env: every game's reader runs on its own cartridge (a spec cart that
writes the reader's RAM bytes, rl.synth.spec_cart with tests/golden/reward10_ram.py's specs), several games in one
env (envs laid out in game order, rl/rlenv.py:107-120), Start/Select legality per game (reward10_consts.h:25-37),
the key-set size in the level layout, and exact resume with the readers' state, key sets and saved level starts in
the blob (rl/tests/gpu_check.py:56-74 restated per game)."""
import sys
from pathlib import Path

import numpy as np
import torch

from helpers import ORACLE_LIB
from rl import synth
from rl.rlenv import GAMES, RlEnv

sys.path.insert(0, str(Path(__file__).resolve().parent / 'golden'))
from reward10_ram import SPECS  # noqa: E402

KEY_CAP = {'castlevania': 4096, 'zelda': 16384}   # rl10_keyset_capacity (reward10.cuh:527-529)


def roms():
    out = {g: synth.spec_cart(SPECS[g], 1) for g in GAMES[1:]}
    out['smb'] = synth.smb_like_cart(1)
    return out


def all_games(n=4, **kw):
    kw.setdefault('seed', 3)
    return RlEnv({g: n for g in GAMES}, device='cpu', lib_path=ORACLE_LIB, roms=roms(), **kw)


def drive(e, steps, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(steps):
        e.actions.copy_(torch.randint(0, 324, (e.n,), generator=g, dtype=torch.int16))
        e.step()
        out.append({k: getattr(e, k).clone() for k in ('obs', 'reward', 'done', 'masks', 'events', 'parts')})
    return out


def test_every_game_rewards_and_ends_in_the_env():
    e = all_games(n=4, idle_max=0, sticky=True, dropout=False)
    e.start()
    out = drive(e, 80, 0)
    r = torch.stack([o['reward'] for o in out]).reshape(80, len(GAMES), 4)
    d = torch.stack([o['done'] for o in out]).reshape(80, len(GAMES), 4)
    ev = torch.stack([o['events'] for o in out]).reshape(80, len(GAMES), 4)
    for gi, g in enumerate(GAMES):
        assert (r[:, gi] > 0).any() and (r[:, gi] < 0).any(), g
    ended = [g for gi, g in enumerate(GAMES) if d[:, gi].any()]
    died = [g for gi, g in enumerate(GAMES) if ((ev[:, gi] & 4) | (ev[:, gi] & 16)).any()]
    assert len(ended) >= 8 and len(died) >= 8, (ended, died)
    parts = torch.stack([o['parts'] for o in out])
    assert torch.allclose(parts.sum(-1), torch.stack([o['reward'] for o in out]), atol=1e-5)


def test_start_select_legality_and_key_layout():
    e = all_games(n=1, dropout=False)
    e.start()
    masks = e.masks.numpy()
    for gi, g in enumerate(GAMES):
        # mask bytes 16 and 18: Start and Select usable (the move set's Start/Select entries)
        assert masks[gi, 16] == (1 if g in ('zelda', 'punchout') else 0), g
        assert masks[gi, 18] == (1 if g == 'punchout' else 0), g
    lev = all_games(n=1, level_cap=2)
    for gi, g in enumerate(GAMES):
        assert lev.level_layout(gi)['key_cap'] == KEY_CAP.get(g, 0), g


def test_exact_resume_with_readers_and_level_starts():
    kw = dict(sticky=True, idle_max=2, dropout=True, level_cap=3)
    a = all_games(**kw)
    a.start()
    drive(a, 30, 1)
    a.set_level_prob(0.6)
    sd = a.state_dict()
    tail_a = drive(a, 20, 2)
    b = all_games(**kw)
    b.load_state_dict(sd)
    b.set_level_prob(0.6)
    tail_b = drive(b, 20, 2)
    for x, y in zip(tail_a, tail_b):
        for k in x:
            assert torch.equal(x[k], y[k]), k
    saved = a.saved_levels()
    assert sum(len(v) for v in saved.values()) >= 4, saved
    assert np.array_equal(a.state_dict()['env'], b.state_dict()['env'])
