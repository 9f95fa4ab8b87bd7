"""The oracle's reward10 readers of the eleven games other than SMB (include/rl10_games.h, the same source as the HIP
library's) against the reference's own compiled rl10_replay (rl/csrc/host_api.cpp:13-31): every update of 24 seeded
RAM episodes per game, reward bit for bit, done, events, event level, deaths and end reason
(tests/golden/reward10_games.npz, written by gen_golden.py from oracle/_ref; the RAM comes from reward10_ram.py)."""
import ctypes
import sys
from pathlib import Path

import numpy as np
import pytest

from helpers import GOLDEN, oracle

sys.path.insert(0, str(Path(__file__).resolve().parent / 'golden'))
from reward10_ram import GAMES, trajectory  # noqa: E402

FIX = np.load(GOLDEN / 'reward10_games.npz')


def p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def oracle_replay(game, rams, frames):
    lib = oracle()
    n = len(rams)
    out = dict(reward=np.zeros(n, np.float64), done=np.zeros(n, np.uint8), events=np.zeros(n, np.uint32),
               level=np.zeros(n, np.int32), deaths=np.zeros(n, np.int32), end=np.zeros(n, np.uint8))
    ov = lib.orc_rl10_replay(game, p(np.ascontiguousarray(rams)), n, p(np.ascontiguousarray(frames, np.int32)),
                             p(out['reward']), p(out['done']), p(out['events']), p(out['level']), p(out['deaths']),
                             p(out['end']))
    return out, ov


@pytest.mark.parametrize('game', GAMES[1:])
def test_reader_matches_reference_replay(game):
    gi = GAMES.index(game)
    for ep in range(int(FIX['episodes'])):
        rams, frames = trajectory(game, ep, int(FIX['steps']))
        out, ov = oracle_replay(gi, rams, frames)
        for k in ('reward', 'done', 'events', 'level', 'deaths', 'end'):
            np.testing.assert_array_equal(out[k], FIX[f'{game}_{k}'][ep], err_msg=f'{game} episode {ep}: {k}')
        assert ov == FIX[f'{game}_overflow'][ep]


def test_fixtures_exercise_the_readers():
    """The seeded trajectories reach the tracker's paths: progress and level rewards, deaths, and episode ends of
    more than one kind, in every game (a trajectory that never leaves one state would pin little)."""
    for game in GAMES[1:]:
        r, ev, end = FIX[f'{game}_reward'], FIX[f'{game}_events'], FIX[f'{game}_end']
        assert (r > 0).any() and (r < 0).any(), game
        assert (ev & 4).any(), f'{game}: no death event'        # kEvDeath
        assert len(set(end[:, -1].tolist())) >= 2, f'{game}: one end kind only'
