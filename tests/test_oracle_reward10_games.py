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


STATE_BYTES, READER_BYTES = 80, 120   # sizeof(Rl10State), sizeof(Rl10Reader) (include/rlenv_state.h)


def batch(game):
    """The fixture's episodes of `game` as one batch: RAM [T, N, 2048], frames [T, N]."""
    E, T = int(FIX['episodes']), int(FIX['steps'])
    tr = [trajectory(game, ep, T) for ep in range(E)]
    return (np.ascontiguousarray(np.stack([r for r, _ in tr], 1)),
            np.ascontiguousarray(np.stack([f for _, f in tr], 1).astype(np.int32)))


def run_batched(lib, gi, ram, frames, cap):
    """rl10_run over [T, N] of host arrays; outputs transposed to [N, T] like the fixtures."""
    T, N = frames.shape
    st = np.zeros(N * STATE_BYTES, np.uint8)
    rd = np.zeros(N * READER_BYTES, np.uint8)
    keys = np.zeros(N * cap + 1, np.uint32)
    out = dict(reward=np.zeros((T, N), np.float64), done=np.zeros((T, N), np.uint8),
               events=np.zeros((T, N), np.uint32), level=np.zeros((T, N), np.int32),
               deaths=np.zeros((T, N), np.int32), end=np.zeros((T, N), np.uint8))
    assert lib.rl10_run(gi, p(ram), T, N, p(frames), p(st), p(rd), p(keys), p(out['reward']), p(out['done']),
                        p(out['events']), p(out['level']), p(out['deaths']), p(out['end']), None) == 0
    return {k: v.T for k, v in out.items()}


KEY_CAP = {'castlevania': 4096, 'zelda': 16384}   # rl10_keyset_capacity (reward10.cuh:527-529)


def test_batched_run_matches_reference_replay():
    """rl10_run (one env per episode, all episodes of a game in one call) equals the reference's per-episode
    rl10_replay outputs for every game, and rejects a bad game id and a missing key buffer."""
    lib = oracle()
    lib.rl10_run.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 11
    for game in GAMES[1:]:
        gi = GAMES.index(game)
        ram, frames = batch(game)
        out = run_batched(lib, gi, ram, frames, KEY_CAP.get(game, 0))
        for k in out:
            np.testing.assert_array_equal(out[k], FIX[f'{game}_{k}'], err_msg=f'{game}: {k}')
    ram, frames = batch('pacman')
    z = np.zeros(4096, np.uint8)
    assert lib.rl10_run(12, p(ram), 1, 1, p(frames), p(z), p(z), None, None, None, None, None, None, None, None) != 0
    assert lib.rl10_run(GAMES.index('zelda'), p(ram), 1, 1, p(frames), p(z), p(z), None, None, None, None, None, None,
                        None, None) != 0


def test_batched_run_smb_matches_reference_fixture():
    """SMB through rl10_run on the full 2 KB RAM equals the reference's SMB replay fixture."""
    from rl import synth
    lib = oracle()
    lib.rl10_run.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 11
    gold = np.load(GOLDEN / 'reward10_smb.npz')
    ram = np.ascontiguousarray(synth.expand_ram(gold['traj']))            # [T, N, 2048]
    T, N = ram.shape[:2]
    frames = np.ascontiguousarray(np.repeat(gold['frames'][:, None], N, 1).astype(np.int32))
    out = run_batched(lib, 0, ram, frames, 0)
    for k, g in (('reward', 'reward'), ('done', 'done'), ('events', 'events'), ('level', 'level'),
                 ('deaths', 'deaths'), ('end', 'end')):
        np.testing.assert_array_equal(out[k].T, gold[g], err_msg=k)
