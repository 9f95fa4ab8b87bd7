"""The oracle's reward10 tracker (rl/csrc/reward10.cuh:546-632, Python source of truth scripts/reward10/reward.py).

Pinned three ways:
  * the reference's compiled host library (rl/csrc/host_api.cpp rl10_replay) on the nine SMB rollback boundary
    cases of rl/tests/test_reward_replay.py:122-143 and on seeded SMB-style RAM trajectories (16 envs x 1024
    steps): rewards equal as doubles, dones, event bits, event levels, deaths and end reasons equal
    (tests/golden/reward10_smb.npz);
  * the closed-form cases of the reference's tests/test_reward10.py restated against the oracle's tracker with
    the FakeGame constants (progress unit 100, score unit 10, no waiting cost unless a case sets one);
  * the standalone batched entry point rl10_smb_run equals a per-env replay.
"""
import ctypes

import numpy as np

from helpers import GOLDEN, oracle, ptr

W_LEVEL, W_DEATH, W_STALL, W_WIN, W_ROLLBACK = 1.0, -0.1, -0.1, 5.0, -0.02
W_IDLE, SCORE_CAP, SCORE_LEVEL_BUDGET = -1.8, 0.1, 0.2
EV = dict(skip=1, level=2, death=4, won=8, game_over=16, stall=32, rollback=64)


class Signals(ctypes.Structure):
    _fields_ = [('in_play', ctypes.c_uint8), ('progress_valid', ctypes.c_uint8), ('dying', ctypes.c_uint8),
                ('has_lives', ctypes.c_uint8), ('has_health', ctypes.c_uint8), ('has_score', ctypes.c_uint8),
                ('game_over', ctypes.c_uint8), ('won', ctypes.c_uint8), ('level', ctypes.c_int32),
                ('lives', ctypes.c_int32), ('progress', ctypes.c_double), ('health', ctypes.c_double),
                ('score', ctypes.c_int64)]


class State(ctypes.Structure):
    _fields_ = [('has_prev', ctypes.c_uint8), ('has_best_level', ctypes.c_uint8),
                ('has_best_progress', ctypes.c_uint8), ('done', ctypes.c_uint8), ('end_reason', ctypes.c_uint8),
                ('overflow', ctypes.c_uint8), ('_p0', ctypes.c_uint8), ('_p1', ctypes.c_uint8),
                ('best_level', ctypes.c_int32), ('deaths', ctypes.c_int32), ('idle_frames', ctypes.c_int64),
                ('best_progress', ctypes.c_double), ('score_used', ctypes.c_double), ('prev', Signals)]


assert ctypes.sizeof(Signals) == 40 and ctypes.sizeof(State) == 80


def S(in_play=True, level=0, progress=0.0, progress_valid=True, dying=False, lives=None, score=None, game_over=False,
      won=False):
    s = Signals(in_play=in_play, progress_valid=progress_valid, dying=dying, game_over=game_over, won=won,
                level=level, progress=float(progress))
    if lives is not None:
        s.has_lives, s.lives = 1, lives
    if score is not None:
        s.has_score, s.score = 1, score
    return s


class Tracker:
    """The oracle's tracker with one game's constants (FakeGame of the reference's tests by default)."""

    def __init__(self, progress_unit=100.0, score_unit=10.0, stall_seconds=120.0, idle_scale=0.0, lives=False):
        stall_frames = stall_seconds * 60.0
        self.consts = (ctypes.c_double * 4)(progress_unit, score_unit, stall_frames, W_IDLE * idle_scale / stall_frames)
        self.lives = int(lives)
        self.st = State()

    def update(self, s, frames=8):
        out = (ctypes.c_double * 11)()
        oracle().orc_rl10_step(ctypes.byref(self.st), ctypes.byref(s), frames, self.consts, self.lives, out)
        return out[0], bool(out[1]), int(out[2]), int(out[3])


def run(seq, **kw):
    tr = Tracker(**kw)
    return [tr.update(s) for s in seq], tr


def test_progress_is_high_water_only():
    out, _ = run([S(progress=0), S(progress=50), S(progress=30), S(progress=50), S(progress=60)])
    assert [round(o[0], 9) for o in out] == [0, 0.5, 0, 0, 0.1]


def test_next_level_bonus_and_stale_progress_ignored():
    out, _ = run([S(progress=10), S(level=1, progress=2900, progress_valid=False), S(level=1, progress=40),
                  S(level=1, progress=90)])
    assert out[1][0] == W_LEVEL and out[2][0] == 0 and abs(out[3][0] - 0.5) < 1e-9


def test_level_skip_ends_episode_without_bonus():
    out, tr = run([S(progress=10), S(level=3, progress=40), S(level=3, progress=90)])
    assert out[1] == (0.0, True, EV['skip'], 3)
    assert out[2] == (0.0, True, 0, 0) and tr.st.best_level == 0 and tr.st.end_reason == 3


def test_death_edge_counts_once():
    out, tr = run([S(), S(dying=True), S(dying=True), S(in_play=False, dying=True), S()])
    assert tr.st.deaths == 1 and out[1][0] == W_DEATH and out[1][2] == EV['death']


def test_lives_mode_and_game_over():
    out, tr = run([S(lives=2), S(lives=1), S(lives=1, game_over=True), S(lives=1)], lives=True)
    assert tr.st.deaths == 1 and out[2][1] is True and out[3] == (0.0, True, 0, 0) and tr.st.end_reason == 1


def test_score_capped_and_win():
    out, tr = run([S(score=0), S(score=10_000), S(score=10_000, won=True)])
    assert out[1][0] == SCORE_CAP and out[2][0] == W_WIN and tr.st.done and tr.st.end_reason == 2


def test_score_budget_per_level_not_reset_by_death():
    out, _ = run([S(score=0), S(score=1000), S(score=2000), S(score=3000), S(score=4000, dying=True),
                  S(level=1, score=5000)])
    assert [o[0] for o in out[1:4]] == [SCORE_CAP, SCORE_CAP, 0.0] and 2 * SCORE_CAP == SCORE_LEVEL_BUDGET
    assert out[4][0] == W_DEATH and out[5][0] == W_LEVEL + SCORE_CAP


def test_stall_ends_episode_with_penalty_and_waiting_costs():
    tr = Tracker(stall_seconds=2.0, idle_scale=1.0)             # 120 frames = 15 decisions of 8 frames
    out = [tr.update(S(progress=10)) for _ in range(16)]
    assert [o[1] for o in out[:15]] == [False] * 15
    per = W_IDLE * 8 / 120
    assert out[0][0] == 0 and all(abs(o[0] - per) < 1e-12 for o in out[1:15])
    assert abs(out[15][0] - (per + W_STALL)) < 1e-12 and out[15][1] and out[15][2] == EV['stall']
    assert tr.st.end_reason == 4
    assert abs(sum(o[0] for o in out) - (W_IDLE + W_STALL)) < 1e-9


def test_waiting_cost_only_when_not_moving_forward_in_play():
    tr = Tracker(idle_scale=1.0)
    seq = [S(progress=30), S(progress=10), S(progress=20), S(progress=20), S(progress=20, in_play=False),
           S(progress=20, in_play=False)]
    r = [tr.update(s)[0] for s in seq]
    per = W_IDLE * 8 / (120 * 60)
    assert r[0] == 0 and abs(r[1] - per) < 1e-12 and r[2] == 0 and abs(r[3] - per) < 1e-12 and r[4] == 0 and r[5] == 0


def test_stall_clock_restarts_on_progress_and_counts_pause():
    tr = Tracker(stall_seconds=2.0)
    seq = [S(progress=0)] * 11 + [S(progress=5)] + [S(progress=5, in_play=False)] * 15
    out = [tr.update(s) for s in seq]
    assert not any(o[1] for o in out[:26]) and out[26][2] == EV['stall']
    tr = Tracker(stall_seconds=2.0)
    tr.update(S())
    tr.st.idle_frames = 100
    tr.update(S(dying=True))
    assert tr.st.idle_frames == 0                               # a death restarts it
    tr.update(S(dying=False))
    tr.st.idle_frames = 100
    tr.update(S(level=1))
    assert tr.st.idle_frames == 0                               # so does a new level


def test_rollback_penalty_once_per_abrupt_drop():
    out, tr = run([S(progress=80), S(progress=40), S(progress=60), S(progress=20), S(progress=90)])
    assert [round(o[0], 9) for o in out] == [0, W_ROLLBACK, 0, W_ROLLBACK, 0.1]
    assert out[1][2] == EV['rollback'] and tr.st.best_progress == 90
    gradual, _ = run([S(progress=x) for x in (80, 60, 40, 20)])
    assert all(o[0] == 0 and o[2] == 0 for o in gradual)


def test_rollback_ignores_deaths_and_invalid_or_changed_level_positions():
    for before, after in [
        (S(progress=80), S(progress=0, dying=True)), (S(progress=80, dying=True), S(progress=0)),
        (S(progress=80), S(progress=0, progress_valid=False)), (S(progress=80, progress_valid=False), S(progress=0)),
        (S(progress=80), S(progress=0, in_play=False)), (S(progress=80), S(progress=0, level=1)),
        (S(progress=80), S(progress=0, won=True)), (S(progress=80), S(progress=0, game_over=True)),
    ]:
        out, _ = run([before, after])
        assert not out[1][2] & EV['rollback']
    out, _ = run([S(progress=80, lives=2), S(progress=0, lives=1)], lives=True)
    assert out[1][2] == EV['death'] and out[1][0] == W_DEATH


def test_smb_page_is_signed():
    ram = np.zeros(2048, np.uint8)
    ram[0x770], ram[0x772], ram[0x0E], ram[0x86], ram[0x6D] = 1, 3, 8, 222, 3
    s = Signals()
    oracle().orc_smb_observe(ptr(ram), ctypes.byref(s))
    assert s.progress == 3 * 256 + 222 and s.progress_valid and s.in_play
    ram[0x6D] = 255
    oracle().orc_smb_observe(ptr(ram), ctypes.byref(s))
    assert s.progress == -256 + 222


def replay(rams, frames):
    n = len(rams)
    rams = np.ascontiguousarray(rams, np.uint8)
    frames = np.ascontiguousarray(frames, np.int32)
    out = dict(reward=np.zeros(n, np.float64), done=np.zeros(n, np.uint8), events=np.zeros(n, np.uint32),
               level=np.zeros(n, np.int32), deaths=np.zeros(n, np.int32), end=np.zeros(n, np.uint8))
    ov = oracle().orc_rl10_replay(0, ptr(rams), n, ptr(frames), ptr(out['reward']), ptr(out['done']),
                                  ptr(out['events']), ptr(out['level']), ptr(out['deaths']), ptr(out['end']))
    assert ov == 0
    return out


def test_rollback_boundaries_match_reference():
    g = np.load(GOLDEN / 'reward10_smb.npz')
    for i in range(len(g['rollback_flags'])):
        out = replay(g['rollback_rams'][i], np.full(2, 4, np.int32))
        assert np.array_equal(out['reward'], g['rollback_reward'][i]), i
        assert np.array_equal(out['events'], g['rollback_events'][i]), i
        assert np.array_equal(out['done'], g['rollback_done'][i]), i
        assert bool(out['events'][1] & EV['rollback']) == bool(g['rollback_flags'][i]), i


def test_trajectories_match_reference():
    import sys
    from rl import synth  # noqa: F401  (package on sys.path through conftest)
    g = np.load(GOLDEN / 'reward10_smb.npz')
    traj = g['traj']
    for e in range(traj.shape[1]):
        out = replay(synth.expand_ram(traj[:, e]), g['frames'])
        for k in ('reward', 'done', 'events', 'level', 'deaths', 'end'):
            assert np.array_equal(out[k], g[k][:, e]), (e, k)
    assert 'rl' in sys.modules
    assert (g['events'] != 0).any() and (g['reward'] != 0).any(), 'the fixture exercises the tracker'


def test_batched_entry_equals_replay():
    from rl import synth
    T, N = 256, 12
    traj = synth.smb_ram15(11, N, T)
    state = np.zeros(N * 80, np.uint8)
    reward = np.zeros((T, N), np.float32)
    done = np.zeros((T, N), np.uint8)
    assert oracle().rl10_smb_run(ptr(traj), T, N, 4, ptr(state), ptr(reward), ptr(done), None) == 0
    for e in range(N):
        out = replay(synth.expand_ram(traj[:, e]), np.full(T, 4, np.int32))
        assert np.array_equal(reward[:, e], out['reward'].astype(np.float32)), e
        assert np.array_equal(done[:, e], out['done']), e
