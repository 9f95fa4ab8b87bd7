#!/usr/bin/env python3
"""Throughput of the batched NES environment step on one MI355X (emulated frames/s and decisions/s).

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--only] [--no-cpu]

A step is one decision of every console: 4 emulated frames each (6502 + PPU + mapper), each frame's 224x240
colour-index picture and emphasis written to HBM, then the reward10 tracker, the outputs and the restart pass
(rl/csrc/rlenv.cu:145-170 is the reference's launch order for one decision).

Workloads (synthetic data; the reference ships no ROMs):
  nrom128-raw-frames (the headline line): 8192 consoles of the seed-generated NROM-128 cartridge
      (rl.synth.nrom_cart: 16 KB PRG of generated 6502 code, 8 KB random CHR), per console and decision a pad byte
      uniform over 0..255, sticky repeat p = 0.25 per frame, no dropout, no idle frames, raw uint8 frames
      [N, 4, 224, 240] + emphasis + a 2 KB RAM hash per console to HBM. The SMB reward reader sees RAM bytes the
      cart never writes, so no episode ends: the restart kernels find nothing to restart.
  rollout-pack6: 8192 NROM consoles, episode ends drawn with p = 1/2000 per decision, finished consoles restored
      from the boot snapshot, 20 % of decisions with a dropped input, and every decision's frames 6-bit packed on
      the device and copied into a ring of pinned host slots on a second stream (the trainer's obs-pack6 store).
  mmc3-stress: 16384 consoles of the seed-generated MMC3 cartridge (256 KB PRG, 128 KB CHR, bank switches,
      scanline IRQ at a varying line, sprite-0 split), independent random pads, frames 6-bit packed on the device.
  twelve-games: the twelve reward10 games, 3072 consoles each (36,864), each on its own seed-generated cartridge
      (the SMB-like cart for smb; NROM, MMC1, UxROM, CNROM, MMC3 and MMC2 carts for the others), raw pads with
      sticky repeat, raw frames; the games step concurrently, one stream each.
  reward10: the SMB reward tracker alone, 8192 envs x 1024 steps of seed-generated SMB RAM trajectories
      (rl.synth.smb_ram15); value in env-steps/s.

One invocation measures the chosen workload (the headline by default) with its parity check and CPU baseline, then,
unless --only, every other workload with a parity check, each under "workloads" in the same JSON line.

Timing: W untimed decisions, then K decisions between device synchronisations; value = consoles * K / seconds.
Inputs (pad bytes) are resident in HBM before the timed region. The library's per-kernel clock brackets every
launch with HIP events on the stream it runs on, which gives each kernel's average duration over the same timed
region; the roofline is computed for the kernel that takes the most time, and for the whole step.

Parity: after the warmup the first 64 consoles' outputs are compared with the CPU oracle run on the same seeds and
pad bytes; for the chosen workload the oracle then continues as the timed CPU baseline (a bounded sample of the same
workload on the host's cores, plus a 1-thread sample).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / 'ghostrun-lab_amd'))

ORACLE_LIB = ROOT / 'oracle' / '_build' / 'liboracle_rlenv.so'
# Compiled translations of the workloads' carts (RLENV_JIT_CACHE): a cold cache adds their compiles (tens of seconds
# each, one at a time) to the env creation, never to the timed region; `bench.py --precompile` fills it on the CPU.
JIT_CACHE = ROOT / 'ghostrun-lab_amd' / 'csrc' / '_build' / 'jit_cache'
ONE_ROUND = 256 * 32                       # consoles the MI355X holds in one round of one-console waves
COUNTERS = ROOT / 'profiles' / 'counters.json'
HBM_PEAK_GBPS = 8000.0
CLOCK_HZ = 2.4e9                           # MI355X peak engine clock
CUS = 256
SALU_PEAK = CUS * CLOCK_HZ                 # one scalar instruction per CU per clock
VALU_PEAK = CUS * CLOCK_HZ                 # one wave64 vector instruction per CU per clock (4 SIMDs x 1/4)
# The library's kernel classes (include/rlenv_api.h rlenv_kernel_times), in its order.
KERNELS = ('k_emu', 'k_render', 'k_finish', 'k_reset_copy', 'k_emu_restart', 'k_render_restart', 'k_reset_finish',
           'k_emu_idle', 'k_archive', 'k_emu_draw')

# Algorithmic bytes per console per decision (outputs written + inputs read by the path, not state traffic).
PICTURE_BYTES = 224 * 240 + 224            # one frame's colour indices + emphasis
PAD_BYTES = 2 + 1                          # a frame's action read and pad byte written
FINISH_BYTES = 4 + 1 + 4 + 28 + 8          # reward, done, events, parts, RAM hash
DECISION_BYTES = 4 * (PICTURE_BYTES + 1) + 2 + 4 + 1 + 4 + 28 + 19 + 360   # 216,358 B per console per decision
PACK6_BYTES = 4 * 224 * 240 * 3 // 4 + 896 + 420                       # 162,596 B per console per decision
RL10_STEP_BYTES = 20                                                      # 15 RAM bytes read + f32 reward + done
# Algorithmic bytes each kernel class writes or reads itself, per console per launch, and per console per decision
# on top of that (the decision's finish, in the last frame's launch).
ALG_BYTES = {
    'k_emu': (PAD_BYTES, 0),                        # frames drawn elsewhere: the emulation's own inputs and outputs
    'k_emu_draw': (PICTURE_BYTES + PAD_BYTES, FINISH_BYTES),   # emulated and drawn; the last frame also finishes
    'k_render': (PICTURE_BYTES, 0),
    'k_finish': (FINISH_BYTES, 0),
    'k_reset_copy': (0, 0),
    'k_emu_restart': (0, 0),
    'k_render_restart': (0, 0),
    'k_reset_finish': (19 + 360, 0),                 # masks, timeline
    'k_emu_idle': (0, 0),
    'k_archive': (0, 0),
}


def metric(consoles):
    """BASELINE's metric, at the workload's console count."""
    return f'emulated NES frames/sec and decisions/sec at {consoles} consoles, 1 MI355X'

WORKLOADS = {
    'nrom128-raw-frames': dict(consoles=8192, cart='nrom', sticky=True, dropout=False, end_prob=0.0, pack6=None),
    'rollout-pack6': dict(consoles=8192, cart='nrom', sticky=True, dropout=True, end_prob=1 / 2000, pack6='host'),
    'mmc3-stress': dict(consoles=16384, cart='mmc3', sticky=False, dropout=False, end_prob=0.0, pack6='device'),
    'twelve-games': dict(consoles=12 * 3072, cart='twelve', sticky=True, dropout=False, end_prob=0.0, pack6=None),
    'reward10': dict(consoles=8192),
}
HEADLINE = 'nrom128-raw-frames'
EXTRA_STEPS = 16                            # timed decisions of each additional workload


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=64)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--workload', choices=sorted(WORKLOADS), default=HEADLINE)
    ap.add_argument('--only', action='store_true', help='measure the chosen workload only')
    ap.add_argument('--consoles', type=int, default=0, help='override the workload console count')
    ap.add_argument('--cart-seed', type=int, default=1)
    ap.add_argument('--seed', type=int, default=1)
    ap.add_argument('--host-slots', type=int, default=4, help='pinned host ring slots of rollout-pack6')
    ap.add_argument('--cpu-seconds', type=float, default=10.0)
    ap.add_argument('--no-cpu', action='store_true', help='skip the parity checks and the CPU baseline')
    ap.add_argument('--no-kernel-clock', action='store_true')
    ap.add_argument('--precompile', action='store_true',
                    help='compile the workloads\' translated kernels into the translation cache (CPU only) and exit')
    return ap.parse_args()


def main():
    args = parse()
    os.environ.setdefault('RLENV_JIT_CACHE', str(JIT_CACHE))
    Path(os.environ['RLENV_JIT_CACHE']).mkdir(parents=True, exist_ok=True)
    if args.precompile:
        precompile(args)
        return
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print('bench.py measures one GPU: the environment step runs on a single MI355X and has no multi-GPU path '
              '(consoles are independent, so a multi-GPU run is one process per GPU over disjoint console ranges, '
              'with no communication). Run with --gpus 1.', file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 1:
        sys.exit('need --steps >= 1 and --warmup >= 1')
    import torch
    if not torch.cuda.is_available():
        sys.exit('bench.py needs a HIP device')
    out = run_workload(args, args.workload, args.steps, args.warmup, baseline=True)
    if not args.only:
        out['workloads'] = {}
        for name in WORKLOADS:
            if name == args.workload:
                continue
            res = run_workload(args, name, min(args.steps, EXTRA_STEPS), min(args.warmup, 6), baseline=False)
            out['workloads'][name] = {k: res[k] for k in ('metric', 'value', 'unit', 'ms_per_step', 'steps', 'warmup',
                                                          'dtype', 'config', 'roofline', 'parity', 'kernels',
                                                          'frames_per_s', 'emulated_instructions_per_s',
                                                          'step_output_gbps', 'translated') if k in res}
            torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)
    bad = [n for n, r in [(args.workload, out)] + list(out.get('workloads', {}).items())
           if 'parity' in r and not r['parity']['bit_exact']]
    if bad:
        print(f'[bench] parity FAILED for {bad}', file=sys.stderr, flush=True)
        sys.exit(3)


def _compile_one(job):
    """One translation through the library, into the cache (a process of its own: compiles in one process run one
    at a time)."""
    rom, mode = job
    from rl.rlenv import bind_library, hip_library
    lib = bind_library(hip_library())
    lib.rlenv_error.restype = ctypes.c_char_p
    out = (ctypes.c_int32 * 6)()
    t = time.perf_counter()
    rc = lib.rlenv_jit_translate(rom, len(rom), mode, out, None, 0)
    return rc, list(out), time.perf_counter() - t, (lib.rlenv_error() or b'').decode()[:300]


def precompile(args):
    """The translations every env workload creates (the frame-bank variant for a one-game env of one round of waves),
    compiled in parallel processes into RLENV_JIT_CACHE."""
    from concurrent.futures import ProcessPoolExecutor
    jobs = {}
    for name, w in WORKLOADS.items():
        if name == 'reward10':
            continue
        carts = carts_of(w, args.cart_seed)
        bank = len(carts) == 1 and w['consoles'] <= ONE_ROUND
        for rom in carts.values():
            jobs[(rom, 2 if bank else 1)] = name
    workers = max(1, min(len(jobs), (os.cpu_count() or 2) // 2, 8))
    print(f'[bench] compiling {len(jobs)} translations into {os.environ["RLENV_JIT_CACHE"]} ({workers} processes)',
          file=sys.stderr, flush=True)
    with ProcessPoolExecutor(workers) as pool:
        for (job, name), (rc, out, sec, err) in zip(jobs.items(), pool.map(_compile_one, list(jobs))):
            print(f'[bench] {name}: {out[0]} blocks, {out[1]} instructions, {sec:.1f} s, {out[4]} far jumps' +
                  (f' FAILED: {err}' if rc else ''), file=sys.stderr, flush=True)


def run_workload(args, name, steps, warmup, baseline):
    if name == 'reward10':
        return bench_reward10(args, steps, warmup, baseline)
    return bench_env(args, name, steps, warmup, baseline)


# ------------------------------------------------------------------------------------------------ env


# The twelve-games batch: a cart per game, in GAMES order (the SMB-like cart for smb, the boards in turn after it).
TWELVE_BOARDS = ('smb_like', 'nrom', 'mmc1', 'uxrom', 'cnrom', 'mmc3', 'mmc2', 'nrom', 'mmc1', 'uxrom', 'cnrom', 'mmc3')


def carts_of(w, seed):
    """game slug -> cart bytes of a workload."""
    from rl import synth
    from rl.rlenv import GAMES
    if w['cart'] != 'twelve':
        return {'smb': synth.nrom_cart(seed) if w['cart'] == 'nrom' else synth.mmc3_cart(seed)}
    make = dict(smb_like=synth.smb_like_cart, nrom=synth.nrom_cart, mmc1=synth.mmc1_cart, uxrom=synth.uxrom_cart,
                cnrom=synth.cnrom_cart, mmc3=synth.mmc3_cart, mmc2=synth.mmc2_cart)
    return {g: make[b](seed + i) for i, (g, b) in enumerate(zip(GAMES, TWELVE_BOARDS))}


# Boot: the reference records each game's boot pad bytes from power-on through its boot sequence and takes the
# boot snapshot after them (rl/rlenv.py:142-170, rl/csrc/rlenv_build.hpp:193-209), so a restart resumes at the end of
# the boot, never at power-on. The seed-generated carts boot in 4 frames (two vblank waits, RAM clear, palette and
# nametable upload); their boot sequence is 4 neutral pad bytes.
BOOT_FRAMES = 4


def env_kwargs(w, args, carts):
    kw = dict(seed=args.seed, sticky=w['sticky'], idle_max=0, dropout=w['dropout'], pad_mode=True, ram_hash=True,
              roms=carts, end_prob=w['end_prob'], boot={g: bytes(BOOT_FRAMES) for g in carts})
    if w['dropout']:
        kw['dropout_gap'] = 1 / 60   # mean gap 60 decisions, mean run 15: 20 % of decisions with a dropped input
    return kw


class Pack6Sink:
    """Where each decision's pictures go. 'device': packed 6 bits per pixel on the device (3/4 of the bytes) into a
    staging buffer. 'host': the pinned-host rollout store (rl.hostobs.RolloutStore; the trainer's store of
    rl/train.py:174-294): the env draws into a ring of two device slots, each packed and copied into a ring of pinned
    host rows on a copy stream while the next decision runs."""

    def __init__(self, env, mode, slots):
        import torch
        self.env, self.mode = env, mode
        self.lib = env.lib
        self.t = 0
        if mode == 'host':
            from rl.hostobs import RolloutStore
            self.rows = slots
            self.store = RolloutStore(env.lib, slots - 1, env.n, env.device, 1, regions=1, ring=2, pack6=True)
            self.emph = env.emph
        else:
            self.px = env.n * 4 * 224 * 240
            self.staging = torch.empty(self.px // 4 * 3, dtype=torch.uint8, device=env.device)

    def before(self):
        """Ahead of a decision: point the env's pictures at the ring slot it draws into."""
        if self.mode == 'host':
            self.env.bind_obs(self.store.target(self.t), self.emph)

    def after(self):
        import torch
        if self.mode == 'host':
            self.store.commit(0, self.t % self.rows)
        else:
            st = ctypes.c_void_p(torch.cuda.current_stream(self.env.device).cuda_stream)
            if self.lib.rl_pack6(ctypes.c_void_p(self.env.obs.data_ptr()), ctypes.c_void_p(self.staging.data_ptr()),
                                 self.px, st) != 0:
                raise RuntimeError(self.lib.rlenv_error().decode())
        self.t += 1

    def obs(self):
        """The pictures of the last decision."""
        return self.store.ring[(self.t - 1) % 2] if self.mode == 'host' else self.env.obs

    def close(self):
        if self.mode == 'host':
            self.store.close()


def bench_env(args, name, K, W, baseline):
    import torch
    from rl.rlenv import GAMES, RlEnv
    w = WORKLOADS[name]
    dev = torch.device('cuda:0')
    N = (args.consoles if name == args.workload else 0) or w['consoles']
    carts = carts_of(w, args.cart_seed)
    counts = {g: N // len(carts) for g in carts}
    N = sum(counts.values())
    kw = env_kwargs(w, args, carts)
    gen = torch.Generator().manual_seed(args.seed)
    pads_host = torch.randint(0, 256, (W + K, N), generator=gen, dtype=torch.int16)
    pads = pads_host.to(dev)

    print(f'[bench] workload {name}: {N} consoles, warmup {W}, timed {K} decisions', file=sys.stderr, flush=True)
    env = RlEnv(counts, device=dev, **kw)
    # the translated kernels (compiled on the library's compile thread, or found in the translation cache): warmup,
    # parity and the timed region all run them; a translation that failed (its compile or its far-jump check)
    # leaves its game on the library's kernel, as in any env
    t_jit = time.perf_counter()
    try:
        env.jit_wait()
    except RuntimeError as ex:
        print(f'[bench] {ex}', file=sys.stderr, flush=True)
    translated = [dict(game=g, **env.jit_status(gi)) for gi, g in enumerate(counts)]
    translated = [t for t in translated if t['state'] != 'none']
    if translated:
        print(f'[bench] translated kernels ready after {time.perf_counter() - t_jit:.1f} s: ' +
              ', '.join(f'{t["game"]} {t["blocks"]} blocks / {t["instructions"]} instructions' for t in translated),
              file=sys.stderr, flush=True)
    sink = Pack6Sink(env, w['pack6'], args.host_slots) if w['pack6'] else None
    env.start()
    for t in range(W):
        env.actions.copy_(pads[t])
        if sink:
            sink.before()
        env.step()
        if sink:
            sink.after()
    torch.cuda.synchronize()
    first = env.games[0]
    ncmp = min(64, counts[first])
    snap = {k: getattr(env, k)[:ncmp].cpu().numpy() for k in ('emph', 'reward', 'done', 'ram_hash')}
    snap['obs'] = (sink.obs() if sink else env.obs)[:ncmp].cpu().numpy()
    instr0 = _instructions(env)
    print('[bench] warmup done', file=sys.stderr, flush=True)

    clock = not args.no_kernel_clock
    if clock:
        env.lib.rlenv_set_kernel_timing.argtypes = [ctypes.c_void_p, ctypes.c_int]
        env.lib.rlenv_kernel_times.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        env.lib.rlenv_set_kernel_timing(env.h, 1)
    ends = torch.zeros((), dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(W, W + K):
        env.actions.copy_(pads[t])
        if sink:
            sink.before()
        env.step()
        if sink:
            sink.after()
        if w['end_prob']:
            ends += env.done.sum()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    kern = _kernel_times(env, N, K, dt) if clock else {}
    instr1 = _instructions(env)
    ends_timed = int(ends.item()) if w['end_prob'] else int(env.done.sum().item())
    if sink:
        sink.close()
    print(f'[bench] timed region {dt:.3f} s', file=sys.stderr, flush=True)

    decisions = N * K / dt
    out_bytes = PACK6_BYTES if w['pack6'] else DECISION_BYTES
    cart = (f'rl.synth.{w["cart"]}_cart({args.cart_seed})' if w['cart'] != 'twelve' else
            'per game: ' + ', '.join(f'{g}={b}({args.cart_seed + i})' for i, (g, b) in enumerate(zip(GAMES,
                                                                                                    TWELVE_BOARDS))))
    cfg = dict(workload=name, consoles=N, games=len(counts), frames_per_decision=4, cart=cart,
               pads='uniform 0..255' + (', sticky p=0.25' if w['sticky'] else ''), dropout=w['dropout'],
               end_prob=w['end_prob'], idle_max=0,
               outputs=('raw u8 frames [N,4,224,240]' if not w['pack6'] else
                        'frames 6-bit packed on the device' + (
                            f', copied to {args.host_slots} pinned host slots' if w['pack6'] == 'host' else '')) +
               ' + emphasis + RAM hash',
               episode_ends_in_timed_region=ends_timed)
    out = dict(metric=metric(N), value=round(decisions, 1), unit='decisions/s', frames_per_s=round(4 * decisions, 1),
               n_gpus=1, steps=K, warmup=W, ms_per_step=round(dt * 1e3 / K, 3), higher_is_better=True,
               scaling='weak', vs_baseline=None, dtype='u8',
               data='synthetic: seed-generated cartridges (rl.synth), uniform random pad bytes', config=cfg,
               emulated_instructions_per_s=round(float(instr1 - instr0) / dt, 1),
               step_output_gbps=round(out_bytes * N * K / dt / 1e9, 3))
    if translated:   # games whose decision frames ran their translated kernel (state 'loaded')
        out['translated'] = translated
    if kern:
        out['roofline'] = _roofline(name, kern, N, K, dt, out_bytes, games=len(counts))
        out['kernels'] = kern
        counters = _counters(name)
        if counters:
            out['counters_profiling_session'] = counters
    if not args.no_cpu:
        cpu_kw = dict(kw, roms={first: carts[first]}, boot={first: bytes(BOOT_FRAMES)})
        parity, base, one = _cpu_env(args, w, first, cpu_kw, pads_host, snap, ncmp, W, baseline)
        out['parity'] = parity
        if baseline:
            out['cpu_baseline'], out['cpu_baseline_1thread'] = base, one
    del env
    return out


def _kernel_times(env, N, K, dt):
    ms = np.zeros(len(KERNELS), np.float64)
    cnt = np.zeros(len(KERNELS), np.int64)
    if env.lib.rlenv_kernel_times(env.h, ms.ctypes.data, cnt.ctypes.data, len(KERNELS)) != 0:
        raise RuntimeError(env.lib.rlenv_error().decode())
    env.lib.rlenv_set_kernel_timing(env.h, 0)
    games = len(env.games)
    kern = {}
    for name, m, c in zip(KERNELS, ms, cnt):
        if c == 0:
            continue
        per = m / c
        per_launch, per_decision = ALG_BYTES[name]
        # a launch covers one game's consoles; the per-decision bytes spread over the class's launches of a decision
        alg = (per_launch + per_decision * K / c) * N / games
        kern[name] = dict(ms_per_launch=round(per, 4), launches_per_step=round(c / K, 3), ms_per_step=round(m / K, 3),
                          share=round(m / (dt * 1e3), 4), alg_bytes_per_launch=round(alg),
                          achieved_gbps=round(alg / (per * 1e-3) / 1e9, 3))
    return kern


def _roofline(name, kern, n, K, dt, out_bytes, games=1):
    """The dominant kernel (the most time per step): its algorithmic bytes per launch over its average launch time
    against HBM (the `bound`/`frac` of the line), and the whole step against HBM. Where the committed counter run of
    the same workload (profiles/counters.json, a deterministic workload) covers the kernels, what actually limits
    them: `issue` gives the dominant kernel's SALU and VALU instructions per launch over this run's average launch time,
    `step_issue` every profiled kernel's instructions per step over this run's step time, each against one instruction
    per CU per clock (256 CUs at 2.4 GHz), and `limiter` names the largest of the step's scalar issue, vector issue and
    HBM fractions."""
    dom = max(kern, key=lambda k: kern[k]['ms_per_step'])
    d = kern[dom]
    step_gbps = out_bytes * n * K / dt / 1e9
    hbm_frac = d['achieved_gbps'] / HBM_PEAK_GBPS
    r = dict(kernel=dom, bound='hbm', achieved=d['achieved_gbps'], peak=HBM_PEAK_GBPS, unit='GB/s',
             frac=round(hbm_frac, 6), traffic=_traffic(name, dom, n),
             step_achieved_gbps=round(step_gbps, 3),
             step_frac=round(step_gbps / HBM_PEAK_GBPS, 6))
    cs = _counters(name) or {}
    c = cs.get(dom)
    if c and c.get('insts_salu') and c.get('dispatches'):
        per_s = d['ms_per_launch'] * 1e-3
        r['issue'] = dict(salu_frac=round(c['insts_salu'] / per_s / SALU_PEAK, 4),
                          valu_frac=round(c['insts_valu'] / per_s / VALU_PEAK, 4), hbm_frac=round(hbm_frac, 6),
                          salu_per_launch=c['insts_salu'], valu_per_launch=c['insts_valu'],
                          salu_per_emulated_instruction=(c.get('per_emulated_instruction') or {}).get('salu'),
                          counter_SALUBusy_pct=c.get('SALUBusy_pct'), counter_VALUBusy_pct=c.get('VALUBusy_pct'),
                          counter_VALUUtilization_pct=c.get('VALUUtilization_pct'),
                          alone_ms_per_launch=c.get('ms_per_dispatch'))
        if c.get('ms_per_dispatch'):     # the kernel alone (the counter runs serialise launches)
            alone_s = c['ms_per_dispatch'] * 1e-3
            r['issue'].update(salu_frac_alone=round(c['insts_salu'] / alone_s / SALU_PEAK, 4),
                              valu_frac_alone=round(c['insts_valu'] / alone_s / VALU_PEAK, 4))
    prof = [k for k in kern if k in cs and cs[k].get('insts_salu')]
    if prof:
        step_s = dt / K
        salu = sum(cs[k]['insts_salu'] * kern[k]['launches_per_step'] for k in prof) / step_s / SALU_PEAK
        valu = sum(cs[k]['insts_valu'] * kern[k]['launches_per_step'] for k in prof) / step_s / VALU_PEAK
        step_hbm = r['step_frac']
        r['step_issue'] = dict(salu_frac=round(salu, 4), valu_frac=round(valu, 4), hbm_frac=step_hbm,
                               kernels=prof)
        r['limiter'] = 'salu' if salu >= max(valu, step_hbm) else 'valu' if valu >= step_hbm else 'hbm'
        r['note'] = ('one console per wavefront: the 6502 and the PPU event logic run on the scalar unit, which the '
                     'renderer\'s per-line control flow shares; the emulator\'s memory traffic is console state staged '
                     'through LDS, not algorithmic bytes')
    if games > 1:
        r['note'] = ('the games step on streams of their own, which share the runtime\'s hardware queues, so a launch\'s '
                     'event-clock time includes other games\' launches queued between its events: the kernel\'s '
                     'achieved figure is a lower bound, the step figures are exact')
    if name == 'rollout-pack6':
        r['host_link_gbps'] = round(PACK6_BYTES * n * K / dt / 1e9, 3)
        r['limiter'] = 'host link'
        r['note'] = 'every decision\'s packed frames cross the host link (PCIe 5 x16, about 63 GB/s each way)'
    return r


def _summary():
    return json.loads(COUNTERS.read_text()) if COUNTERS.exists() else {}


def _counters(workload):
    """Issue and utilisation figures of the workload's kernels from the committed counter summary, if present
    (figures of the profiling session, each kernel alone, not of this run)."""
    keep = ('kernel', 'dispatches', 'ms_per_dispatch', 'insts_salu', 'insts_valu', 'SALUBusy_pct', 'VALUBusy_pct',
            'VALUUtilization_pct', 'per_emulated_instruction', 'wave_state_pct')   # instructions: per launch
    w = _summary().get('workloads', {}).get(workload)
    return {k: {f: v[f] for f in keep if f in v} for k, v in w.items()} if w else None


def _traffic(workload, kernel, n):
    """HBM bytes per launch of `kernel` on `workload` from the committed counter summary (FETCH_SIZE + WRITE_SIZE
    scaled by the copy-kernel calibration), scaled to n consoles; None when it does not cover them."""
    t = _summary().get('traffic', {}).get(workload, {}).get(kernel)
    return round(t['bytes_per_console_launch'] * n) if t and 'consoles' in t else None


def _rl10_traffic(env_steps):
    """HBM bytes of one tracker run (its three kernels) from the committed counter summary, scaled to env_steps."""
    t = _summary().get('traffic', {}).get('reward10')
    if not t or not all('env_steps' in v for v in t.values()):
        return None
    return round(sum((v['fetch_bytes_per_launch'] + v['write_bytes_per_launch']) / v['env_steps'] for v in t.values())
                 * env_steps)


def _instructions(env) -> int:
    """Emulated 6502 instructions of every console so far (record field instr_lo, u32 at 0x14)."""
    import torch
    torch.cuda.synchronize()
    total = 0
    for gi in range(len(env.games)):
        rec = env.consoles(gi)
        total += int(np.frombuffer(np.ascontiguousarray(rec[:, 0x14:0x18]).tobytes(), np.uint32).astype(np.int64).sum())
    return total


def _oracle():
    lib = ctypes.CDLL(str(ORACLE_LIB))
    lib.orc_set_threads.argtypes = [ctypes.c_int]
    return lib


def _host_cpus():
    """Threads the CPU baseline uses (OMP_NUM_THREADS, else the CPUs this process may run on, at most 16: the GPU
    box's CPU share), and the host's logical and physical core counts."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    phys = set()
    try:
        cur = {}
        for line in Path('/proc/cpuinfo').read_text().splitlines() + ['']:
            if not line.strip():
                if 'core id' in cur:
                    phys.add((cur.get('physical id'), cur['core id']))
                cur = {}
            elif ':' in line:
                k, v = line.split(':', 1)
                cur[k.strip()] = v.strip()
    except OSError:
        pass
    threads = int(os.environ.get('OMP_NUM_THREADS', '0')) or min(allowed, 16)
    return threads, dict(nproc=os.cpu_count(), affinity=allowed, physical_cores=len(phys) or None)


def _cpu_env(args, w, game, kw, pads_host, snap, ncmp, W, baseline):
    """Parity of the first ncmp consoles after the warmup; with `baseline`, the CPU baseline (oracle) on the same
    workload: max(64, 4 x threads) consoles on the baseline threads, then 64 consoles on 1 thread."""
    import torch
    from rl.rlenv import RlEnv
    lib = _oracle()
    lib.rl_pack6.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    threads, host = _host_cpus()
    lib.orc_set_threads(threads)
    cpu = RlEnv({game: ncmp}, device='cpu', lib_path=ORACLE_LIB, **kw)
    cpu.start()
    for t in range(W):
        cpu.actions.copy_(pads_host[t, :ncmp])
        cpu.step()
    bad = [k for k in snap if not np.array_equal(snap[k], getattr(cpu, k).numpy())]
    parity = dict(consoles=ncmp, decisions=W, bit_exact=not bad, differs=bad, outputs=sorted(snap))
    print(f'[bench] parity vs oracle on {ncmp} consoles x {W} decisions: '
          f'{"bit-exact" if not bad else "DIFFERS in " + ",".join(bad)}', file=sys.stderr, flush=True)
    del cpu
    if not baseline:
        return parity, None, None
    res = {}
    for label, nthr, n, budget in (('all', threads, max(64, 4 * threads), args.cpu_seconds),
                                   ('one', 1, 64, max(2.0, args.cpu_seconds / 3))):
        lib.orc_set_threads(nthr)
        cpu = RlEnv({game: n}, device='cpu', lib_path=ORACLE_LIB, **kw)
        packed = np.empty(n * 4 * 224 * 240 // 4 * 3, np.uint8)
        cpu.start()
        gen = np.random.default_rng(args.seed + 7)
        t0 = time.perf_counter()
        d = 0
        while True:
            cpu.actions.copy_(torch.from_numpy(gen.integers(0, 256, n).astype(np.int16)))
            cpu.step()
            if w['pack6']:
                obs = cpu.obs.numpy()
                lib.rl_pack6(obs.ctypes.data, packed.ctypes.data, obs.size, None)
            d += 1
            el = time.perf_counter() - t0
            if el >= budget and d >= 2:
                break
        res[label] = dict(value=round(n * d / el, 2), unit='decisions/s', cores=nthr, kind='port', **host,
                          sample=f'CPU oracle (oracle/, C, OpenMP over consoles) on {n} consoles of the same '
                                 f'cartridge, settings and pad distribution{" with pack6" if w["pack6"] else ""}, '
                                 f'{d} decisions x 4 frames in {el:.1f} s, {nthr} thread(s)')
        del cpu
    return parity, res['all'], res['one']


# ------------------------------------------------------------------------------------------- reward10


def bench_reward10(args, K, W, baseline):
    """The SMB reward tracker alone (rl10_smb_run): T steps of N envs over seed-generated RAM trajectories, timed per
    call (its three kernels); value in env-steps/s."""
    import torch
    from rl import synth
    from rl.rlenv import hip_library
    N = (args.consoles if args.workload == 'reward10' else 0) or WORKLOADS['reward10']['consoles']
    T = 1024
    print(f'[bench] workload reward10: {N} envs x {T} steps, warmup {W}, timed {K} runs', file=sys.stderr,
          flush=True)
    ram = synth.smb_ram15(args.seed, N, T)                   # [T, N, 16]
    lib = ctypes.CDLL(str(hip_library()))
    lib.rl10_smb_run.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    d_ram = torch.from_numpy(ram).cuda()
    state = torch.zeros(N * 80, dtype=torch.uint8, device='cuda')
    rew = torch.zeros(T, N, dtype=torch.float32, device='cuda')
    done = torch.zeros(T, N, dtype=torch.uint8, device='cuda')
    cur = torch.cuda.current_stream()
    st = ctypes.c_void_p(cur.cuda_stream)

    def p(t):
        return ctypes.c_void_p(t.data_ptr())

    def run():
        state.zero_()
        if lib.rl10_smb_run(p(d_ram), T, N, 4, p(state), p(rew), p(done), st) != 0:
            raise RuntimeError('rl10_smb_run failed')

    for _ in range(W):
        run()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    t0 = time.perf_counter()
    for a, b in evs:
        state.zero_()
        a.record(cur)
        if lib.rl10_smb_run(p(d_ram), T, N, 4, p(state), p(rew), p(done), st) != 0:
            raise RuntimeError('rl10_smb_run failed')
        b.record(cur)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    kms = sum(a.elapsed_time(b) for a, b in evs) / K
    steps_s = N * T * K / dt
    alg = RL10_STEP_BYTES * N * T
    achieved = alg / (kms * 1e-3) / 1e9
    out = dict(metric='reward10 SMB env-steps/sec at 8192 envs, 1 MI355X (standalone tracker)',
               value=round(steps_s, 1), unit='env-steps/s', n_gpus=1, steps=K, warmup=W,
               ms_per_step=round(dt * 1e3 / K, 3), higher_is_better=True, scaling='weak', vs_baseline=None,
               dtype='f64', data='synthetic: seed-generated SMB RAM trajectories (rl.synth.smb_ram15)',
               config=dict(workload='reward10', envs=N, steps_per_run=T, frames_per_step=4),
               kernels=dict(rl10_smb_run=dict(ms_per_launch=round(kms, 4), alg_bytes_per_launch=alg,
                                              achieved_gbps=round(achieved, 3),
                                              clocks_per_step=round(kms * 1e-3 * CLOCK_HZ / T, 1),
                                              launches='k_smb_signals, k_smb_chain, k_smb_reward')),
               roofline=dict(kernel='rl10_smb_run', bound='hbm', achieved=round(achieved, 3), peak=HBM_PEAK_GBPS,
                             unit='GB/s', frac=round(achieved / HBM_PEAK_GBPS, 6), traffic=_rl10_traffic(N * T),
                             limiter='issue latency',
                             note='k_smb_chain, one env per lane for T steps in order, issues one instruction of a '
                                  'step every 4 cycles (one wave per SIMD on 128 of them); the signals and the '
                                  'rewards run over all env-steps in parallel'))
    if not args.no_cpu:
        got_r, got_d = rew.cpu().numpy(), done.cpu().numpy()
        lib_o = _oracle()
        lib_o.rl10_smb_run.argtypes = lib.rl10_smb_run.argtypes
        ncmp = min(64, N)
        sub = np.ascontiguousarray(ram[:, :ncmp])
        want_r = np.zeros((T, ncmp), np.float32)
        want_d = np.zeros((T, ncmp), np.uint8)
        st0 = np.zeros(ncmp * 80, np.uint8)
        lib_o.rl10_smb_run(sub.ctypes.data, T, ncmp, 4, st0.ctypes.data, want_r.ctypes.data, want_d.ctypes.data, None)
        ok = np.array_equal(got_r[:, :ncmp], want_r) and np.array_equal(got_d[:, :ncmp], want_d)
        out['parity'] = dict(envs=ncmp, steps=T, bit_exact=bool(ok), outputs=['reward', 'done'])
        if baseline:
            threads, host = _host_cpus()
            res = {}
            for label, nthr in (('all', threads), ('one', 1)):
                lib_o.orc_set_threads(nthr)
                n = N if nthr > 1 else N // 8
                sub = np.ascontiguousarray(ram[:, :n])
                r = np.zeros((T, n), np.float32)
                dd = np.zeros((T, n), np.uint8)
                s = np.zeros(n * 80, np.uint8)
                t0 = time.perf_counter()
                lib_o.rl10_smb_run(sub.ctypes.data, T, n, 4, s.ctypes.data, r.ctypes.data, dd.ctypes.data, None)
                el = time.perf_counter() - t0
                res[label] = dict(value=round(n * T / el, 1), unit='env-steps/s', cores=nthr, kind='port', **host,
                                  sample=f'CPU oracle rl10_smb_run (C, OpenMP over envs) on {n} envs x {T} steps of '
                                         f'the same trajectories, {el:.2f} s, {nthr} thread(s)')
            out['cpu_baseline'], out['cpu_baseline_1thread'] = res['all'], res['one']
    return out


if __name__ == '__main__':
    main()
