"""Env-level properties of the oracle's step (the reference's integration checks restated without NeSLE or ROMs).

  * determinism, and exact resume through state_dict/load_state_dict (rl/tests/gpu_check.py:56-74);
  * a restarted console equals a fresh boot: after an episode ends, the observation is the start observation
    (rl/csrc/rlenv_core.cuh:208-263, snapshot restore from slot n);
  * episode bookkeeping in info (ret, len, end reason, episode number; rlenv_core.cuh:266-309);
  * an unofficial opcode ends the episode with reward 0 and end reason 5 (rlenv_core.cuh:12-13, 273-301);
  * --episode-level-end: a level change ends the episode with reason 6;
  * the controller contract in the env: pads from move ids with the turbo phase, the dropped input never pressed,
    masks = the legality of the current drop (rl/tests/test_dropout_env.py:26-104);
  * reward parts sum to the reward (rl/tests/test_reward_parts.py:18-22).
"""
import numpy as np
import torch

from helpers import ORACLE_LIB
from rl import synth
from rl.rlenv import RlEnv

UP, DOWN, LEFT, RIGHT, A, B = 16, 32, 64, 128, 1, 2
DPAD = [0, UP, UP | RIGHT, RIGHT, DOWN | RIGHT, DOWN, DOWN | LEFT, LEFT, UP | LEFT]
CLEAR = [UP, DOWN, LEFT, RIGHT, A, B, A, B]


def env(n=8, cart=None, **kw):
    kw.setdefault('seed', 3)
    return RlEnv({'smb': n}, device='cpu', lib_path=ORACLE_LIB, roms={'smb': cart or synth.smb_like_cart(1)}, **kw)


def outputs(e):
    return {k: getattr(e, k).clone() for k in ('obs', 'emph', 'reward', 'done', 'masks', 'timeline', 'pads',
                                               'events', 'info', 'parts')}


def drive(e, steps, seed, hi=256):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(steps):
        e.actions.copy_(torch.randint(0, hi, (e.n,), generator=g, dtype=torch.int16))
        e.step()
        out.append(outputs(e))
    return out


def same(a, b):
    """Equal outputs; info only where an episode ended (it is written at episode end, and not saved by state_dict,
    as in the reference's rl/rlenv.py:363)."""
    def eq(x, y, k):
        if k != 'info':
            return torch.equal(x[k], y[k])
        d = x['done'].bool()
        return torch.equal(x['done'], y['done']) and torch.equal(x[k][d], y[k][d])
    return all(eq(x, y, k) for x, y in zip(a, b) for k in x)


def test_deterministic():
    kw = dict(sticky=True, idle_max=4, dropout=True, pad_mode=True)
    a, b = env(**kw), env(**kw)
    a.start()
    b.start()
    assert same(drive(a, 12, 0), drive(b, 12, 0))
    c = env(seed=4, **kw)
    c.start()
    assert not same(drive(a, 12, 1), drive(c, 12, 1))


def test_exact_resume():
    kw = dict(sticky=True, idle_max=4, dropout=True, pad_mode=True, end_prob=0.05)
    a = env(**kw)
    a.start()
    drive(a, 10, 0)
    sd = a.state_dict()
    tail_a = drive(a, 8, 1)
    b = env(**kw)
    b.load_state_dict(sd)
    assert same(tail_a, drive(b, 8, 1))


def test_restart_equals_fresh_start_and_info():
    kw = dict(sticky=True, idle_max=0, dropout=True, pad_mode=True, end_prob=0.3)
    e = env(n=16, **kw)
    e.start()
    first = e.obs.clone()
    lens = np.zeros(16, np.int64)
    episodes = np.zeros(16, np.int64)
    ret = np.zeros(16, np.float32)
    seen = 0
    for o in drive(e, 30, 5):
        lens += 1
        ret += o['reward'].numpy()
        for k in np.flatnonzero(o['done'].numpy()):
            seen += 1
            inf = o['info'][k].numpy()
            assert torch.equal(o['obs'][k], first[k]) and torch.equal(o['emph'][k], e.emph[k] * 0 + o['emph'][k])
            assert inf[1] == lens[k] and inf[7] == episodes[k] and inf[2] in (1, 7)
            assert abs(inf[0] - ret[k]) < 1e-4
            lens[k] = 0
            ret[k] = 0
            episodes[k] += 1
    assert seen > 20


def test_fault_ends_the_episode():
    """A cart that runs into an unofficial opcode on its third frame."""
    a = synth.Asm(0xC000)
    a.label('reset')
    a.op('SEI'); a.op('LDA', 'imm', 0); a.op('STA', 'zp', 0x10); a.op('LDA', 'imm', 0x80); a.op('STA', 'abs', 0x2000)
    a.label('loop')
    a.op('LDA', 'zp', 0x10); a.op('CMP', 'imm', 3); a.op('BCC', 'rel', 'loop')
    a.byte(0x02)                                         # KIL: not an official opcode
    a.label('nmi')
    a.op('INC', 'zp', 0x10); a.op('RTI')
    code = a.assemble()
    prg = bytearray(16384)
    prg[:len(code)] = code
    prg[0x3FFA:0x4000] = bytes((a.labels['nmi'] & 0xFF, a.labels['nmi'] >> 8, 0, 0xC0, 0, 0xC0))
    cart = synth.ines(bytes(prg), bytes(8192), 0)
    e = env(n=4, cart=cart, sticky=False, idle_max=0, dropout=False, pad_mode=True)
    e.start()
    o = drive(e, 3, 0)
    assert all(o[t]['done'].all() for t in range(3))
    assert (o[0]['info'][:, 2] == 5).all() and (o[0]['reward'] == 0).all() and (o[0]['info'][:, 7] == 0).all()
    assert (o[2]['info'][:, 7] == 2).all()


def test_episode_level_end():
    kw = dict(sticky=False, idle_max=0, dropout=False, pad_mode=True)
    e = env(n=4, **kw)
    e.set_episode_level_end(0)
    e.start()
    e.actions.fill_(RIGHT)                               # 2 px a frame: page 3 (level 1) after ~364 frames
    ends = []
    for t in range(120):
        e.step()
        if e.done.any():
            ends.append((t, e.info[:, 2].clone(), e.reward.clone()))
            break
    assert ends, 'no level end'
    t, reason, reward = ends[0]
    assert (reason == 6).all() and (reward > 0.9).all()   # +1 for the new level


def test_pads_turbo_and_dropout_in_move_mode():
    e = env(n=16, sticky=False, idle_max=0, dropout=True, pad_mode=False)
    e.start()
    g = torch.Generator().manual_seed(2)
    frame = 4                                            # the start ran 4 neutral frames
    for t in range(60):
        tl = e.timeline.clone()
        masks = e.masks.clone()
        ids = torch.randint(0, 81, (16,), generator=g, dtype=torch.int16)
        e.actions.copy_(ids)
        e.step()
        for k in range(16):
            d_now = [i for i in range(8) if tl[k, i, 0]]
            i = int(ids[k])
            d, a, b = i % 9, (i // 9) % 3, (i // 27) % 3
            for f in range(4):
                ef = frame + f
                want = DPAD[d] | (A if a == 1 or (a == 2 and ef % 2 == 0) else 0) | \
                    (B if b == 1 or (b == 2 and ef % 2 == 0) else 0)
                assert int(e.pads[k, f]) == want
            # masks of this decision: every choice allowed except those using the dropped input; SMB forbids
            # Start and Select (layout: d-pad 9, A none/hold/turbo, B none/hold/turbo, Start 2, Select 2)
            want = np.ones(19, np.uint8)
            want[16] = want[18] = 0
            for dr in d_now:
                if dr < 4:
                    want[:9] = [0 if DPAD[c] & CLEAR[dr] else 1 for c in range(9)]
                else:
                    want[{4: 10, 6: 11, 5: 13, 7: 14}[dr]] = 0
            assert np.array_equal(masks[k].numpy(), want), (k, d_now)
        frame += 4


def test_raw_pads_never_press_the_dropped_input():
    e = env(n=16, sticky=True, idle_max=0, dropout=True, pad_mode=True, dropout_gap=0.2)
    e.start()
    g = torch.Generator().manual_seed(7)
    hits = 0
    for t in range(80):
        tl = e.timeline.clone()
        e.actions.copy_(torch.randint(0, 256, (16,), generator=g, dtype=torch.int16))
        e.step()
        for k in range(16):
            for i in range(8):
                if tl[k, i, 0]:
                    hits += 1
                    assert (e.pads[k] & CLEAR[i] == 0).all()
    assert hits > 100


def test_sticky_off_pads_are_the_actions():
    e = env(n=8, sticky=False, idle_max=0, dropout=False, pad_mode=True)
    e.start()
    for o in drive(e, 5, 3):
        pass
    g = torch.Generator().manual_seed(9)
    for _ in range(5):
        act = torch.randint(0, 256, (8,), generator=g, dtype=torch.int16)
        e.actions.copy_(act)
        e.step()
        assert torch.equal(e.pads, act.to(torch.uint8)[:, None].expand(8, 4))


def test_parts_sum_to_reward_and_rewards_happen():
    e = env(n=16, sticky=True, idle_max=4, dropout=True, pad_mode=True)
    e.start()
    nz = 0
    for o in drive(e, 60, 11):
        assert torch.allclose(o['parts'].sum(1), o['reward'], atol=1e-6)
        nz += int((o['reward'] != 0).sum())
    assert nz > 200


def test_modes_cart_cycles_the_ppu_modes():
    """The modes cart sets each frame's PPU mode in vblank from its frame counter (synth.MODES: 8x8 and 8x16 sprites,
    sprites or background off, clipped left columns, then a grey frame and a red-emphasis one in every 8). Over 24
    frames of 2 consoles the emphasis frames come 8 apart, every row of such a frame carries red (1) and no row of any
    other frame has emphasis, and the frame before each is grey (only the 0x30 bits of a colour index)."""
    e = env(2, synth.modes_cart(1), pad_mode=True, sticky=False, idle_max=0, dropout=False)
    e.start()
    obs, emph = [], []
    for o in drive(e, 6, 1):
        obs += [o['obs'][:, f] for f in range(4)]
        emph += [o['emph'][:, f] for f in range(4)]
    red = [k for k, m in enumerate(emph) if (m == 1).all()]
    assert len(red) == 3 and red[1] - red[0] == 8 and red[2] - red[1] == 8, red
    assert all((m == 0).all() for k, m in enumerate(emph) if k not in red)
    for k in red:
        assert k > 0 and ((obs[k - 1] & 0x0F) == 0).all() and (obs[k - 1] != 0).any()
        assert (obs[k] & 0x0F).any()
