"""Level starts and places on the oracle (rl/csrc/rlenv_core.cuh:14-20, 208-263, 288-291, 343-387; the reference's
rl/rlenv.py:240-324 surface), restated without NeSLE or ROMs on the SMB-like synthetic cart: holding Right for 91
decisions reaches page 3, the next level (the tracker's level 1); holding Down for 6 decisions starts dying (a death).

  * the level-1 save is the arrival with the fewest deaths; among equal deaths in one decision the lowest env
    index; a later arrival with no more deaths replaces it (the newest on ties);
  * a level start is the saved console plus 4 neutral frames: checked against the emulator run directly on the
    saved record (orc_run_until / orc_render_obs), not through the env code;
  * start_level reports the slot an episode started from, level_now / progress_now the tracker after a decision;
  * places: place_save / place_copy / level_deaths / level_layout, a restart from a weighted place;
  * the archive is part of the exact-resume state, and a state saved with fewer slots grows into more.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import ORACLE_LIB, Console, ptr
from rl import synth
from rl.rlenv import RlEnv

RIGHT, LEFT, DOWN, A = 128, 64, 32, 1
REC = 23552
FRAME_DOTS = 341 * 262


def env(n, **kw):
    kw.setdefault('seed', 3)
    kw.setdefault('level_cap', 4)
    return RlEnv({'smb': n}, device='cpu', lib_path=ORACLE_LIB, roms={'smb': synth.smb_like_cart(1)},
                 sticky=False, idle_max=0, dropout=False, pad_mode=True, **kw)


def tail_sizes(lay, cap):
    """The reference's six archive parts of one game for `cap` slots (rl/rlenv.py:293-310 _grow_archive,
    rl/csrc/rlenv_build.hpp:274-278): consoles, tracker blocks, key words, targets, frames, deaths."""
    return [cap * lay['stride'], cap * lay['st'], cap * lay['key_cap'] * 4, cap * 8, cap * 4, cap * 4]


def archive(e, gi=0):
    """Game gi's part of the level-start tail of the state blob: (records [cap, REC], tracker blocks [cap, st] =
    Rl10State then Rl10Reader, targets, frames, deaths), parsed with the reference's six-part layout."""
    lays = [e.level_layout(g) for g in range(len(e.games))]
    blob = e.state_dict()['env']
    o = len(blob) - sum(sum(tail_sizes(l, l['cap'])) for l in lays)
    for g in range(gi):
        o += sum(tail_sizes(lays[g], lays[g]['cap']))
    lay, cap = lays[gi], lays[gi]['cap']
    parts = []
    for s_ in tail_sizes(lay, cap):
        parts.append(blob[o:o + s_])
        o += s_
    return (parts[0].reshape(cap, lay['stride']), parts[1].reshape(cap, lay['st']),
            parts[3].view(np.uint64), parts[4].view(np.uint32), parts[5].view(np.int32))


def drive(e, pads_of, steps):
    for t in range(steps):
        e.actions.copy_(torch.tensor(pads_of(t), dtype=torch.int16))
        e.step()


def force_end(e, on=True):
    e.lib.rlenv_set_end_prob.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
    e.lib.rlenv_set_end_prob(e.h, 2 ** 32 - 1 if on else 0)


def test_layout_enable_errors_and_empty_archive():
    e = env(4, level_cap=6, level_slots=2)
    assert e.level_layout(0) == dict(stride=REC, key_cap=0, st=80 + 120, cap=6, levels=2)   # tracker + reader
    assert e.saved_levels() == {'smb': {}}
    assert e.lib.rlenv_enable_places(e.h, 4, 4) != 0 and b'once' in e.lib.rlenv_error()
    f = RlEnv({'smb': 2}, device='cpu', lib_path=ORACLE_LIB, roms={'smb': synth.smb_like_cart(1)})
    assert f.lib.rlenv_enable_places(f.h, 4, 5) != 0
    recs, st, tgt, frm, deaths = archive(e)
    assert (deaths == -1).all() and (recs == 0).all()


def test_claim_fewest_deaths_lowest_index_then_newest():
    """env 0 dies once then runs; envs 1 and 2 run at once (2 also scores, so the two saves differ); env 3 starts
    4 decisions late. Level 1: env 1 (deaths 0, index 1 < 2), then env 3 (deaths 0, a later decision), never env 0."""
    e = env(4)
    e.start()

    def pads(t):
        p0 = DOWN if t < 6 else (0 if t < 16 else RIGHT)
        return [p0, RIGHT, RIGHT | A, RIGHT if t >= 4 else 0]

    level_seen = None
    for t in range(120):
        drive(e, lambda _: pads(t), 1)
        saved = e.saved_levels()['smb']
        if 1 in saved and level_seen is None:
            level_seen = t
            recs, st, tgt, frm, deaths = archive(e)
            assert deaths[1] == 0
            cons = e.consoles(0)
            assert np.array_equal(recs[1], cons[1]) and not np.array_equal(recs[1], cons[2])
            assert int(e.level_now[1]) == 1 and int(e.level_now[2]) == 1 and int(e.level_now[3]) == 0
        if level_seen is not None and t == level_seen + 4:
            # env 3 arrived exactly 4 decisions later with 0 deaths: its console replaced env 1's
            recs, st, tgt, frm, deaths = archive(e)
            assert deaths[1] == 0 and int(e.level_now[3]) == 1
            assert np.array_equal(recs[1], e.consoles(0)[3])
            saved_after_3 = recs[1].copy()
    assert level_seen is not None
    assert int(e.level_now[0]) == 1                     # env 0 arrived too, with a death: the save stayed env 3's
    recs, st, tgt, frm, deaths = archive(e)
    assert deaths[1] == 0 and np.array_equal(recs[1], saved_after_3) and e.saved_levels()['smb'] == {1: 0}


def test_newest_arrival_with_equal_deaths_replaces_the_save():
    e = env(2)
    e.start()
    cons_at = {}
    for t in range(110):
        drive(e, lambda _: [RIGHT, RIGHT | A if t >= 3 else 0], 1)
        now = e.level_now.numpy().copy()
        if now[0] == 1 and 0 not in cons_at:
            cons_at[0] = e.consoles(0)[0].copy()
            assert np.array_equal(archive(e)[0][1], cons_at[0])
        if now[1] == 1 and 1 not in cons_at:
            cons_at[1] = e.consoles(0)[1].copy()
            assert np.array_equal(archive(e)[0][1], cons_at[1])     # the later arrival, deaths 0 <= 0
    assert set(cons_at) == {0, 1}


def emulate_from(cart_bytes, rec, target):
    """4 neutral frames from a saved record, run with the emulator's own entry points (no env code): pictures and
    the final record."""
    con = Console(cart_bytes)
    con.rec[:] = rec
    obs = np.zeros((4, 224, 240), np.uint8)
    emph = np.zeros((4, 224), np.uint8)
    for f in range(4):
        con.set('pad', 0)
        assert con.run_until(target + f * FRAME_DOTS) == 0
        con.lib.orc_render_obs(ptr(con.rec), con.cart_ptr(), ptr(obs[f]), ptr(emph[f]))
    return obs, emph, con.rec.copy()


def test_level_start_is_the_saved_console_plus_four_neutral_frames():
    cart = synth.smb_like_cart(1)
    e = env(3)
    e.start()
    drive(e, lambda t: [RIGHT, RIGHT, RIGHT], 95)
    assert e.saved_levels()['smb'] == {1: 0}
    recs, st, tgt, frm, deaths = archive(e)
    want_obs, want_emph, want_rec = emulate_from(cart, recs[1], int(tgt[1]))
    e.set_level_prob(1.0)
    force_end(e)
    drive(e, lambda t: [0, 0, 0], 1)
    force_end(e, False)
    assert e.done.all()
    assert (e.start_level == -1).all()                 # the finished episodes started at the boot snapshot
    cons = e.consoles(0)
    for k in range(3):
        assert np.array_equal(e.obs[k].numpy(), want_obs) and np.array_equal(e.emph[k].numpy(), want_emph)
        assert np.array_equal(cons[k], want_rec)
    # the tracker continues from the saved one: level 1 is not a new level event, so no level reward
    drive(e, lambda t: [RIGHT, RIGHT, RIGHT], 3)
    assert not (e.events.numpy() & 2).any() and (e.level_now == 1).all()
    force_end(e)
    drive(e, lambda t: [0, 0, 0], 1)
    assert (e.start_level == 1).all() and (e.info[:, 4] >= 1).all()   # started from slot 1; max level >= 1


def test_progress_and_level_outputs():
    e = env(2)
    e.start()
    drive(e, lambda t: [RIGHT, LEFT], 5)
    cons = e.consoles(0)
    for k in range(2):
        ram = cons[k][0x100:0x900]
        page, x = int(ram[0x6D]), int(ram[0x86])
        page = page - 256 if page > 127 else page
        assert e.progress_now[k].item() == np.float32((page * 256 + x) / 3000.0)
        assert int(e.level_now[k]) == 0
    drive(e, lambda t: [DOWN, 0], 6)                    # env 0 starts dying: progress not valid while dying
    assert np.isnan(e.progress_now[0].item()) and not np.isnan(e.progress_now[1].item())


def test_places_save_copy_and_weighted_restart():
    e = env(3, level_cap=5, level_slots=2)
    e.start()
    drive(e, lambda t: [RIGHT, RIGHT | A, 0], 10)
    e.place_save(0, torch.tensor([1, 0, 2], dtype=torch.int32), torch.tensor([3, 1, 4], dtype=torch.int32))
    recs, st, tgt, frm, deaths = archive(e)
    cons = e.consoles(0)
    assert list(deaths) == [-1, -1, -1, 0, 0]          # slot 1 is a level slot: skipped
    assert np.array_equal(recs[3], cons[1]) and np.array_equal(recs[4], cons[2])
    e.place_copy(0, [3], [2])
    recs2, st2, tgt2, frm2, deaths2 = archive(e)
    assert list(deaths2) == [-1, -1, 0, 0, 0] and np.array_equal(recs2[2], recs2[3]) and tgt2[2] == tgt2[3]
    with pytest.raises(RuntimeError):
        e.place_copy(0, [5], [0])
    assert e.saved_levels()['smb'] == {}                 # saved_levels covers the level slots only
    # all weight on place 4 (env 2's idle console): every restart starts there
    w = np.zeros(5)
    w[4] = 1.0
    e.set_level_plan(0, 1.0, w)
    want_obs, _, want_rec = emulate_from(synth.smb_like_cart(1), recs[4], int(tgt[4]))
    force_end(e)
    drive(e, lambda t: [0, 0, 0], 1)
    force_end(e, False)
    cons = e.consoles(0)
    for k in range(3):
        assert np.array_equal(e.obs[k].numpy(), want_obs) and np.array_equal(cons[k], want_rec)
    force_end(e)
    drive(e, lambda t: [0, 0, 0], 1)
    assert (e.start_level == 4).all()


def test_archive_resumes_exactly_and_grows():
    kw = dict(level_cap=4)
    a = env(3, **kw)
    a.start()
    drive(a, lambda t: [RIGHT, RIGHT, RIGHT | A], 95)
    a.set_level_prob(0.5)
    sd = a.state_dict()
    b = env(3, **kw)
    b.load_state_dict(sd)
    b.set_level_prob(0.5)
    a.lib.rlenv_set_end_prob.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
    for x in (a, b):
        x.lib.rlenv_set_end_prob(x.h, 2 ** 30)
    g = torch.Generator().manual_seed(0)
    for t in range(12):
        act = torch.randint(0, 256, (3,), generator=g, dtype=torch.int16)
        a.actions.copy_(act)
        b.actions.copy_(act)
        a.step()
        b.step()
        for k in ('obs', 'reward', 'done', 'start_level', 'level_now'):
            assert torch.equal(getattr(a, k), getattr(b, k)), (t, k)
        assert torch.equal(a.progress_now.nan_to_num(-1), b.progress_now.nan_to_num(-1))
    assert np.array_equal(a.state_dict()['env'], b.state_dict()['env'])
    # a state saved with 4 slots loads into an env with 6: the first 4 slots as saved, the new ones empty
    c = env(3, level_cap=6)
    c.load_state_dict(a.state_dict())
    ra, rc = archive(a), archive(c)
    assert np.array_equal(rc[0][:4], ra[0]) and list(rc[4][4:]) == [-1, -1] and np.array_equal(rc[4][:4], ra[4])
    # a state saved without level starts loads with an empty archive
    d0 = RlEnv({'smb': 3}, device='cpu', lib_path=ORACLE_LIB, roms={'smb': synth.smb_like_cart(1)}, seed=3,
               sticky=False, idle_max=0, dropout=False, pad_mode=True)
    d0.start()
    d = env(3)
    d.load_state_dict(d0.state_dict())
    assert (archive(d)[4] == -1).all()


def reference_grow(buf, lays, old_cap, new_cap):
    """The reference's archive growth (rl/rlenv.py:293-310), restated: the blob's prefix, then per game each of the
    six parts with its old slots followed by the new empty ones (zeros; deaths 0xFF bytes = -1)."""
    old_tail = sum(sum(tail_sizes(l, old_cap)) for l in lays)
    out, o = [buf[:len(buf) - old_tail]], len(buf) - old_tail
    for l in lays:
        for k, (a, b) in enumerate(zip(tail_sizes(l, old_cap), tail_sizes(l, new_cap))):
            out += [buf[o:o + a], np.full(b - a, 0xFF if k == 5 else 0, np.uint8)]
            o += a
    return np.concatenate(out)


def test_reference_formula_grows_a_two_game_archive():
    """A blob saved with 2 slots per game, on an SMB env and a Castlevania env (a 4,096-word key set per env and
    slot), grown to 4 slots by the reference's own six-part formula: RlEnv's growth gives the same bytes, the
    grown blob loads, the saved slots keep their contents, and the resumed env steps exactly as the saved one."""
    roms = {'smb': synth.smb_like_cart(1), 'castlevania': synth.nrom_cart(2)}
    mk = lambda cap: RlEnv({'smb': 2, 'castlevania': 2}, device='cpu', lib_path=ORACLE_LIB, roms=roms, seed=5,  # noqa
                           sticky=False, idle_max=0, dropout=False, pad_mode=True, level_cap=cap)
    a = mk(2)
    a.start()
    drive(a, lambda t: [RIGHT, RIGHT | A, RIGHT, 0], 95)
    assert 1 in a.saved_levels()['smb']
    sd = a.state_dict()
    lays = [a.level_layout(g) for g in range(2)]
    assert lays[1]['key_cap'] == 4096 and lays[0]['st'] == lays[1]['st'] == 200
    grown = reference_grow(sd['env'], lays, 2, 4)
    b = mk(4)
    assert len(grown) == b.lib.rlenv_state_bytes(b.h)
    assert np.array_equal(b._grow_archive(sd['env'], 2, len(grown)), grown)
    b.load_state_dict(sd)
    assert np.array_equal(b.state_dict()['env'], grown)
    for gi in range(2):
        ra, rb = archive(a, gi), archive(b, gi)
        for x, y in zip(ra, rb):
            assert np.array_equal(y[:2], x)
        assert list(rb[4][2:]) == [-1, -1] and not rb[0][2:].any()
    g = torch.Generator().manual_seed(4)
    for t in range(10):
        act = torch.randint(0, 256, (4,), generator=g, dtype=torch.int16)
        for x in (a, b):
            x.actions.copy_(act)
            x.step()
        for k in ('obs', 'reward', 'done', 'masks', 'level_now'):
            assert torch.equal(getattr(a, k), getattr(b, k)), (t, k)
