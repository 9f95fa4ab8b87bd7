"""The oracle's controller, counter RNG and dropout schedule.

Pinned two ways:
  * golden fixtures written by the reference's own host library (rl/csrc/host_api.cpp, compiled from its sources
    by oracle/Makefile.ref; tests/golden/gen_golden.py): pad table, legality/restrict tables, schedules, episode
    seeds must equal them exactly;
  * an independent Python reading of the contract, restating rl/tests/test_controller.py:33-152 (move packing,
    turbo phase, a dropped input masks exactly the moves that use it, a sticky repeat never adds a button, the
    schedule's run lengths and shares, the timeline is the future).
"""
import numpy as np

from helpers import GOLDEN, oracle, ptr

UP, DOWN, LEFT, RIGHT, A, B, SELECT, START = 16, 32, 64, 128, 1, 2, 4, 8
DPAD = [0, UP, UP | RIGHT, RIGHT, DOWN | RIGHT, DOWN, DOWN | LEFT, LEFT, UP | LEFT]
NM = 324


def ref_unpack(i):
    d, i = i % 9, i // 9
    a, i = i % 3, i // 3
    b, i = i % 3, i // 3
    s, i = i % 2, i // 2
    return d, a, b, s, i % 2


def ref_pad(i, frame):
    d, a, b, s, sel = ref_unpack(i)
    even = frame % 2 == 0
    return (DPAD[d] | (A if a == 1 or (a == 2 and even) else 0) | (B if b == 1 or (b == 2 and even) else 0)
            | (START if s else 0) | (SELECT if sel else 0))


def ref_uses(i, drop):
    d, a, b, s, sel = ref_unpack(i)
    return {0: DPAD[d] & UP, 1: DPAD[d] & DOWN, 2: DPAD[d] & LEFT, 3: DPAD[d] & RIGHT,
            4: a == 1, 5: b == 1, 6: a == 2, 7: b == 2}[drop]


def tables(start_ok, select_ok):
    legal = np.zeros(9 * NM, np.uint8)
    rest = np.zeros(9 * NM, np.int32)
    oracle().orc_legal_table(start_ok, select_ok, ptr(legal), ptr(rest))
    return legal, rest


def schedule(seed, n, enabled=True, with_timeline=False, gap_p32=122713351):
    dropped = np.zeros(n, np.int8)
    tl = np.zeros((n, 8 * 45), np.uint8) if with_timeline else None
    oracle().orc_schedule(int(seed), int(enabled), n, ptr(dropped), ptr(tl) if with_timeline else None, gap_p32)
    return dropped, tl


def test_pad_table_matches_reference_and_spec():
    out = np.zeros(2 * NM, np.uint8)
    oracle().orc_pad_table(ptr(out))
    gold = np.load(GOLDEN / 'controller.npz')
    assert np.array_equal(out, gold['pad_table'])
    out = out.reshape(NM, 2)
    for i in range(NM):
        for f in (0, 1):
            assert out[i, f] == ref_pad(i, f), (i, f)
        p = out[i, 0] | out[i, 1]
        assert not (p & UP and p & DOWN) and not (p & LEFT and p & RIGHT)


def test_legal_and_restrict_tables_match_reference_and_spec():
    gold = np.load(GOLDEN / 'controller.npz')
    for so, se in ((0, 0), (1, 0), (1, 1)):
        legal, rest = tables(so, se)
        assert np.array_equal(legal, gold[f'out_{so}{se}']), (so, se)
        assert np.array_equal(rest, gold[f'rest_{so}{se}']), (so, se)
        legal, rest = legal.reshape(9, NM), rest.reshape(9, NM)
        for i in range(NM):
            d, a, b, s, sel = ref_unpack(i)
            allowed = (not s or so) and (not sel or se)
            assert legal[0, i] == allowed
            for drop in range(8):
                assert legal[drop + 1, i] == (allowed and not ref_uses(i, drop)), (i, drop)
                r = rest[drop + 1, i]
                assert legal[drop + 1, r]
                pr, pi = ref_pad(r, 0) | ref_pad(r, 1), ref_pad(i, 0) | ref_pad(i, 1)
                assert pr & ~pi == 0, 'a sticky repeat never adds a button'
        assert legal[0].sum() == {(0, 0): 81, (1, 0): 162, (1, 1): 324}[(so, se)]


def test_schedule_matches_reference():
    gold = np.load(GOLDEN / 'dropout.npz')
    for i, seed in enumerate(gold['seeds']):
        d, _ = schedule(int(seed), gold['dropped'].shape[1])
        assert np.array_equal(d, gold['dropped'][i]), i
        d2, tl = schedule(int(seed), gold['timelines'].shape[1], with_timeline=True)
        assert np.array_equal(tl, gold['timelines'][i]), i
    off, _ = schedule(99, 50, enabled=False)
    assert np.array_equal(off, gold['disabled'])


def test_episode_seed_matches_reference():
    gold = np.load(GOLDEN / 'dropout.npz')
    lib = oracle()
    got = np.array([lib.orc_episode_seed(int(a), int(b), int(c)) for a, b, c in gold['triples']], np.uint64)
    assert np.array_equal(got, gold['episode_seed'])
    assert len({lib.orc_episode_seed(1, e, k) for e in range(64) for k in range(64)}) == 64 * 64


def runs(x):
    edges = np.flatnonzero(np.diff(x)) + 1
    starts = np.r_[0, edges]
    return x[starts], np.diff(np.r_[starts, len(x)])


def test_schedule_statistics():
    n = 15 * 3600 * 20
    d, _ = schedule(oracle().orc_episode_seed(7, 3, 11), n)
    vals, lens = runs(d)
    inner_v, inner_l = vals[1:-1], lens[1:-1]
    on = inner_v >= 0
    assert not np.any(on[1:] & on[:-1]), 'two dropouts without a healthy gap'
    assert inner_l[on].min() >= 8 and inner_l[on].max() <= 22
    assert inner_l[~on].min() >= 1 and abs(inner_l[~on].mean() - 35) < 1.0
    assert 0.29 < (d >= 0).mean() < 0.31
    share = np.bincount(d[d >= 0], minlength=8) / n
    assert np.all(np.abs(share - 0.0375) < 0.003)


def test_schedule_with_configured_gap_gives_twenty_percent():
    """The full-rollout workload's 20 % dropped share: mean run 15 decisions, so the healthy gap mean is 60, i.e.
    P(a gap ends) = 1/60 per decision (the same Geometric gap draw with another p)."""
    d, _ = schedule(12345, 400_000, gap_p32=int(2 ** 32 / 60))
    assert 0.19 < (d >= 0).mean() < 0.21


def test_timeline_is_the_future():
    n = 3000
    d, tl = schedule(12345, n, with_timeline=True)
    tl = tl.reshape(n, 8, 45)
    for t in range(n - 45):
        want = np.zeros((8, 45), np.uint8)
        for j in range(45):
            if d[t + j] >= 0:
                want[d[t + j], j] = 1
        assert np.array_equal(tl[t], want), t


def test_seeds_and_disable():
    a, _ = schedule(99, 5000)
    b, _ = schedule(99, 5000)
    c, _ = schedule(100, 5000)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    off, tl = schedule(99, 500, enabled=False, with_timeline=True)
    assert (off == -1).all() and tl.sum() == 0


def test_move_id_codec_and_random_legal():
    """rl/actions.py's mixed-radix move ids (d-pad 9, A 3, B 3, Start 2, Select 2, least significant first): every
    one of the 324 ids round-trips, the place values are the running products of the radices, the mask columns are
    the parts side by side, and random_legal draws only legal choices, every legal choice of a part with about
    equal frequency."""
    import torch
    from rl import actions
    ids = torch.arange(324, dtype=torch.int16)
    parts = actions.unpack(ids)
    assert [int(p.max()) + 1 for p in parts] == [9, 3, 3, 2, 2]
    assert torch.equal(actions.pack(parts), ids)
    assert actions.MULT == [1, 9, 27, 81, 162] and actions.NUM_MOVES == 324
    assert actions.PARTS == [(0, 9), (9, 12), (12, 15), (15, 17), (17, 19)]
    # brute force: the id of (d, a, b, s, t) is d + 9a + 27b + 81s + 162t
    want = [d + 9 * a + 27 * b + 81 * s + 162 * t for t in range(2) for s in range(2) for b in range(3)
            for a in range(3) for d in range(9)]
    assert want == list(range(324))
    g = torch.Generator().manual_seed(3)
    masks = torch.zeros(4000, 19, dtype=torch.uint8)
    masks[:, [0, 4, 8]] = 1            # d-pad: none, left-ish, right-ish only
    masks[:, 9] = 1                    # A: only "off"
    masks[:, 12:15] = 1                # B: all three
    masks[:2000, 15] = 1               # Start: off for half the envs, on for the other half
    masks[2000:, 16] = 1
    masks[:, 17:19] = 1
    got = actions.unpack(actions.random_legal(masks, g))
    for k, (a, b) in enumerate(actions.PARTS):
        assert bool(masks[torch.arange(4000), a + got[k]].all())
    counts = torch.bincount(got[0], minlength=9)
    assert set(torch.nonzero(counts).flatten().tolist()) == {0, 4, 8}
    assert all(abs(int(counts[c]) - 4000 / 3) < 200 for c in (0, 4, 8))
    assert (got[3][:2000] == 0).all() and (got[3][2000:] == 1).all()
