#!/usr/bin/env python3
"""Throughput of the batched NES environment step on one MI355X (emulated frames/s and decisions/s).

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

A step is one decision of every console: 4 emulated frames each (6502 + PPU + mapper), each frame's 224x240
colour-index picture and emphasis written to HBM, then the reward10 tracker, the outputs and the restart pass
(rl/csrc/rlenv.cu:145-170 is the reference's launch order for one decision).

Workloads (synthetic data; the reference ships no ROMs):
  nrom128-raw-frames (default, the headline): 8192 consoles of the seed-generated NROM-128 cartridge
      (rl.synth.nrom_cart: 16 KB PRG of generated 6502 code, 8 KB random CHR), per console and decision a pad byte
      uniform over 0..255, sticky repeat p = 0.25 per frame, no dropout, no idle frames, raw uint8 frames
      [N, 4, 224, 240] + emphasis + a 2 KB RAM hash per console to HBM. The SMB reward reader sees RAM bytes the
      cart never writes, so no episode ends within 1800 decisions: the restart kernels find nothing to restart.
  rollout-pack6: 8192 NROM consoles, episode ends drawn with p = 1/2000 per decision, finished consoles restored
      from the boot snapshot, 20 % of decisions with a dropped input, and every decision's frames 6-bit packed on
      the device and copied into a ring of pinned host slots on a second stream (the trainer's obs-pack6 store).
  mmc3-stress: 16384 consoles of the seed-generated MMC3 cartridge (256 KB PRG, 128 KB CHR, bank switches,
      scanline IRQ at a varying line, sprite-0 split), independent random pads, frames 6-bit packed on the device.
  reward10: the SMB reward tracker alone, 8192 envs x 1024 steps of seed-generated SMB RAM trajectories
      (rl.synth.smb_ram15); value in env-steps/s.

Timing: W untimed decisions, then K decisions between device synchronisations; value = consoles * K / seconds.
Inputs (pad bytes) are resident in HBM before the timed region. The library's per-kernel clock brackets every
launch with HIP events on the stream it runs on, which gives each kernel's average duration over the same timed
region; the roofline is computed for the kernel that takes the most time.

Parity: after the warmup the first 64 consoles' outputs are compared with the CPU oracle run on the same seeds and
pad bytes; the oracle then continues as the timed CPU baseline (a bounded sample of the same workload on the
host's cores, plus a 1-thread sample).
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

METRIC = 'emulated NES frames/sec and decisions/sec at 8192 consoles, 1 MI355X'
ORACLE_LIB = ROOT / 'oracle' / '_build' / 'liboracle_rlenv.so'
COUNTERS = ROOT / 'profiles' / 'counters.json'
HBM_PEAK_GBPS = 8000.0
SALU_PEAK = 256 * 2.4e9                    # one scalar ALU per CU (256 CUs) at the 2.4 GHz peak engine clock
KERNELS = ('k_emu', 'k_render', 'k_finish', 'k_reset_copy', 'k_emu_restart', 'k_render_restart', 'k_reset_finish',
           'k_emu_idle', 'k_archive')

# Algorithmic bytes per console per launch (outputs written + inputs read by the path, not state traffic).
PICTURE_BYTES = 224 * 240 + 224            # one frame's colour indices + emphasis
ALG_BYTES = {
    'k_emu': 2 + 1,                         # the action (int16) read, the frame's pad byte written
    'k_render': PICTURE_BYTES,
    'k_finish': 4 + 1 + 4 + 28 + 8,         # reward, done, events, parts, RAM hash
    'k_reset_copy': 0,
    'k_emu_restart': 0,
    'k_render_restart': 0,
    'k_reset_finish': 19 + 360,             # masks, timeline
    'k_emu_idle': 0,
    'k_archive': 0,
}
DECISION_BYTES = 4 * (PICTURE_BYTES + 1) + 2 + 4 + 1 + 4 + 28 + 19 + 360   # 216,358 B per console per decision
PACK6_BYTES = 4 * 224 * 240 * 3 // 4 + 896 + 420                       # 162,596 B per console per decision
RL10_STEP_BYTES = 20                                                      # 15 RAM bytes read + f32 reward + done

WORKLOADS = {
    'nrom128-raw-frames': dict(consoles=8192, cart='nrom', sticky=True, dropout=False, end_prob=0.0, pack6=None),
    'rollout-pack6': dict(consoles=8192, cart='nrom', sticky=True, dropout=True, end_prob=1 / 2000, pack6='host'),
    'mmc3-stress': dict(consoles=16384, cart='mmc3', sticky=False, dropout=False, end_prob=0.0, pack6='device'),
    'reward10': dict(consoles=8192),
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=64)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--workload', choices=sorted(WORKLOADS), default='nrom128-raw-frames')
    ap.add_argument('--consoles', type=int, default=0, help='override the workload console count')
    ap.add_argument('--cart-seed', type=int, default=1)
    ap.add_argument('--seed', type=int, default=1)
    ap.add_argument('--host-slots', type=int, default=4, help='pinned host ring slots of rollout-pack6')
    ap.add_argument('--cpu-seconds', type=float, default=10.0)
    ap.add_argument('--cpu-consoles', type=int, default=64)
    ap.add_argument('--no-cpu', action='store_true', help='skip the parity check and the CPU baseline')
    ap.add_argument('--no-kernel-clock', action='store_true')
    return ap.parse_args()


def main():
    args = parse()
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
    out = bench_reward10(args) if args.workload == 'reward10' else bench_env(args)
    print(json.dumps(out), flush=True)
    if 'parity' in out and not out['parity']['bit_exact']:
        sys.exit(3)


# ------------------------------------------------------------------------------------------------ env


def cart_of(w, seed):
    from rl import synth
    return synth.nrom_cart(seed) if w['cart'] == 'nrom' else synth.mmc3_cart(seed)


# Boot: the reference records each game's boot pad bytes from power-on through its boot sequence and takes the
# boot snapshot after them (rl/rlenv.py:142-170, rl/csrc/rlenv_build.hpp:193-209), so a restart resumes at the end of
# the boot, never at power-on. The seed-generated carts boot in 4 frames (two vblank waits, RAM clear, palette and
# nametable upload); their boot sequence is 4 neutral pad bytes.
BOOT_FRAMES = 4


def env_kwargs(w, args, cart):
    kw = dict(seed=args.seed, sticky=w['sticky'], idle_max=0, dropout=w['dropout'], pad_mode=True, ram_hash=True,
              roms={'smb': cart}, end_prob=w['end_prob'], boot={'smb': bytes(BOOT_FRAMES)})
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


def bench_env(args):
    import torch
    from rl.rlenv import RlEnv
    w = WORKLOADS[args.workload]
    dev = torch.device('cuda:0')
    N = args.consoles or w['consoles']
    W, K = args.warmup, args.steps
    cart = cart_of(w, args.cart_seed)
    kw = env_kwargs(w, args, cart)
    gen = torch.Generator().manual_seed(args.seed)
    pads_host = torch.randint(0, 256, (W + K, N), generator=gen, dtype=torch.int16)
    pads = pads_host.to(dev)

    print(f'[bench] workload {args.workload}: {N} consoles, warmup {W}, timed {K} decisions', file=sys.stderr,
          flush=True)
    env = RlEnv({'smb': N}, device=dev, **kw)
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
    ncmp = min(args.cpu_consoles, N)
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
    cfg = dict(workload=args.workload, consoles=N, frames_per_decision=4,
               cart=f'rl.synth.{w["cart"]}_cart({args.cart_seed})',
               pads='uniform 0..255' + (', sticky p=0.25' if w['sticky'] else ''), dropout=w['dropout'],
               end_prob=w['end_prob'], idle_max=0,
               outputs=('raw u8 frames [N,4,224,240]' if not w['pack6'] else
                        'frames 6-bit packed on the device' + (
                            f', copied to {args.host_slots} pinned host slots' if w['pack6'] == 'host' else '')) +
               ' + emphasis + RAM hash',
               episode_ends_in_timed_region=ends_timed)
    out = dict(metric=METRIC, value=round(decisions, 1), unit='decisions/s', frames_per_s=round(4 * decisions, 1),
               n_gpus=1, steps=K, warmup=W, ms_per_step=round(dt * 1e3 / K, 3), higher_is_better=True,
               scaling='weak', vs_baseline=None, dtype='u8',
               data='synthetic: seed-generated cartridge (rl.synth), uniform random pad bytes', config=cfg,
               emulated_instructions_per_s=round(float(instr1 - instr0) / dt, 1),
               step_output_gbps=round(out_bytes * N * K / dt / 1e9, 3))
    if kern:
        out['roofline'] = _roofline(kern, N)
        iss = _issue_roofline(args.workload, kern, K, dt, out['emulated_instructions_per_s'])
        if iss:
            out['issue_roofline'] = iss
        out['kernels'] = kern
        counters = _counters(args.workload)
        if counters:
            out['counters'] = counters
    if not args.no_cpu:
        out['parity'], out['cpu_baseline'], out['cpu_baseline_1thread'] = _cpu_env(args, w, kw, pads_host, snap,
                                                                                 ncmp)
    return out


def _kernel_times(env, N, K, dt):
    ms = np.zeros(len(KERNELS), np.float64)
    cnt = np.zeros(len(KERNELS), np.int64)
    if env.lib.rlenv_kernel_times(env.h, ms.ctypes.data, cnt.ctypes.data, len(KERNELS)) != 0:
        raise RuntimeError(env.lib.rlenv_error().decode())
    env.lib.rlenv_set_kernel_timing(env.h, 0)
    kern = {}
    for name, m, c in zip(KERNELS, ms, cnt):
        if c == 0:
            continue
        per = m / c
        alg = ALG_BYTES[name] * N
        kern[name] = dict(ms_per_launch=round(per, 4), launches_per_step=round(c / K, 3), ms_per_step=round(m / K, 3),
                          share=round(m / (dt * 1e3), 4), alg_bytes_per_launch=alg,
                          achieved_gbps=round(alg / (per * 1e-3) / 1e9, 3))
    return kern


def _roofline(kern, n):
    dom = max(kern, key=lambda k: kern[k]['ms_per_step'])
    d = kern[dom]
    r = dict(kernel=dom, bound='hbm', achieved=d['achieved_gbps'], peak=HBM_PEAK_GBPS, unit='GB/s',
             frac=round(d['achieved_gbps'] / HBM_PEAK_GBPS, 6), traffic=_traffic(dom, n))
    if dom in ('k_emu', 'k_emu_restart'):
        r['note'] = ('the 6502 interpreter: one console per wavefront on the scalar unit, bound by scalar issue '
                     '(issue_roofline), not by HBM; its algorithmic bytes are the action read and the pad byte written')
    return r


def _issue_roofline(workload, kern, K, dt, ips):
    """Scalar-issue roofline of the emulator kernel: SALU instructions per second against one scalar ALU per CU at
    the peak engine clock. SALU instructions per emulated instruction come from the committed counter run of the same
    workload (SQ_INSTS_SALU); the emulated instructions and the kernel's time are measured in this run. VALU
    utilisation of the two frame kernels is reported beside it from the same counter run."""
    c = _counters(workload) or {}
    e = c.get('k_emu')
    if not e or 'k_emu' not in kern:
        return None
    restart = kern.get('k_emu_restart', {}).get('ms_per_step', 0.0)
    if restart > 0.05 * kern['k_emu']['ms_per_step']:
        return None                          # restart frames would count in the instructions but not in k_emu time
    salu = e['per_emulated_instruction']['salu']
    emu_s = kern['k_emu']['ms_per_step'] * K / 1e3
    achieved = ips * dt / emu_s * salu
    out = dict(kernel='k_emu', bound='salu', unit='SALU instr/s', achieved=round(achieved / 1e9, 1) * 1e9,
               peak=SALU_PEAK, frac=round(achieved / SALU_PEAK, 4), salu_per_emulated_instruction=salu,
               counter_SALUBusy_pct=e.get('SALUBusy_pct'))
    out['valu_busy_pct'] = {k: v.get('VALUBusy_pct') for k, v in c.items() if isinstance(v, dict)}
    return out


def _summary():
    return json.loads(COUNTERS.read_text()) if COUNTERS.exists() else {}


def _counters(workload):
    """Issue and utilisation figures of the frame kernels from the committed counter summary, if present."""
    keep = ('kernel', 'SALUBusy_pct', 'VALUBusy_pct', 'VALUUtilization_pct', 'per_emulated_instruction',
            'wave_state_pct')
    w = _summary().get('workloads', {}).get(workload)
    return {k: {f: v[f] for f in keep if f in v} for k, v in w.items()} if w else None


def _traffic(kernel, n):
    """HBM bytes per launch of `kernel` from the committed counter summary (FETCH_SIZE + WRITE_SIZE scaled by the
    copy-kernel calibration), scaled to n consoles; None when no summary covers it."""
    t = _summary().get('traffic', {}).get(kernel)
    return round(t['bytes_per_console_launch'] * n) if t else None


def _instructions(env) -> int:
    """Emulated 6502 instructions of every console so far (record field instr_lo, u32 at 0x14)."""
    import torch
    torch.cuda.synchronize()
    rec = env.consoles(0)
    return int(np.frombuffer(np.ascontiguousarray(rec[:, 0x14:0x18]).tobytes(), np.uint32).astype(np.int64).sum())


def _oracle():
    lib = ctypes.CDLL(str(ORACLE_LIB))
    lib.orc_set_threads.argtypes = [ctypes.c_int]
    return lib


def _threads():
    return int(os.environ.get('OMP_NUM_THREADS', '0')) or min(os.cpu_count() or 1, 16)


def _cpu_env(args, w, kw, pads_host, snap, ncmp):
    """Parity of the first ncmp consoles after the warmup, then the CPU baseline (oracle) on the same workload."""
    import torch
    from rl.rlenv import RlEnv
    lib = _oracle()
    lib.rl_pack6.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    W = args.warmup
    res = {}
    parity = None
    for label, nthr, budget in (('all', _threads(), args.cpu_seconds), ('one', 1, max(2.0, args.cpu_seconds / 3))):
        lib.orc_set_threads(nthr)
        cpu = RlEnv({'smb': ncmp}, device='cpu', lib_path=ORACLE_LIB, **kw)
        packed = np.empty(ncmp * 4 * 224 * 240 // 4 * 3, np.uint8)
        cpu.start()
        for t in range(W):
            cpu.actions.copy_(pads_host[t, :ncmp])
            cpu.step()
        if label == 'all':
            bad = [k for k in snap if not np.array_equal(snap[k], getattr(cpu, k).numpy())]
            parity = dict(consoles=ncmp, decisions=W, bit_exact=not bad, differs=bad, outputs=sorted(snap))
            print(f'[bench] parity vs oracle on {ncmp} consoles x {W} decisions: '
                  f'{"bit-exact" if not bad else "DIFFERS in " + ",".join(bad)}', file=sys.stderr, flush=True)
        gen = np.random.default_rng(args.seed + 7)
        t0 = time.perf_counter()
        d = 0
        while True:
            cpu.actions.copy_(torch.from_numpy(gen.integers(0, 256, ncmp).astype(np.int16)))
            cpu.step()
            if w['pack6']:
                obs = cpu.obs.numpy()
                lib.rl_pack6(obs.ctypes.data, packed.ctypes.data, obs.size, None)
            d += 1
            el = time.perf_counter() - t0
            if el >= budget and d >= 2:
                break
        res[label] = dict(value=round(ncmp * d / el, 2), unit='decisions/s', cores=nthr, kind='port',
                          sample=f'CPU oracle (oracle/, C, OpenMP over consoles) on {ncmp} consoles of the same '
                                 f'cartridge, settings and pad distribution{" with pack6" if w["pack6"] else ""}, '
                                 f'{d} decisions x 4 frames in {el:.1f} s, {nthr} thread(s)')
        del cpu
    return parity, res['all'], res['one']


# ------------------------------------------------------------------------------------------- reward10


def bench_reward10(args):
    """The SMB reward tracker alone (rl10_smb_run): T steps of N envs over seed-generated RAM trajectories, one
    env per lane; value in env-steps/s."""
    import torch
    from rl import synth
    from rl.rlenv import hip_library
    N = args.consoles or WORKLOADS['reward10']['consoles']
    T = 1024
    K, W = args.steps, args.warmup
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
               kernels=dict(k_rl10_smb=dict(ms_per_launch=round(kms, 4), alg_bytes_per_launch=alg,
                                            achieved_gbps=round(achieved, 3))),
               roofline=dict(kernel='k_rl10_smb', bound='hbm', achieved=round(achieved, 3), peak=HBM_PEAK_GBPS,
                             unit='GB/s', frac=round(achieved / HBM_PEAK_GBPS, 6), traffic=_traffic('k_rl10_smb', 1)))
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
        res = {}
        for label, nthr in (('all', _threads()), ('one', 1)):
            lib_o.orc_set_threads(nthr)
            n = N if nthr > 1 else N // 8
            sub = np.ascontiguousarray(ram[:, :n])
            r = np.zeros((T, n), np.float32)
            dd = np.zeros((T, n), np.uint8)
            s = np.zeros(n * 80, np.uint8)
            t0 = time.perf_counter()
            lib_o.rl10_smb_run(sub.ctypes.data, T, n, 4, s.ctypes.data, r.ctypes.data, dd.ctypes.data, None)
            el = time.perf_counter() - t0
            res[label] = dict(value=round(n * T / el, 1), unit='env-steps/s', cores=nthr, kind='port',
                              sample=f'CPU oracle rl10_smb_run (C, OpenMP over envs) on {n} envs x {T} steps of '
                                     f'the same trajectories, {el:.2f} s, {nthr} thread(s)')
        out['cpu_baseline'], out['cpu_baseline_1thread'] = res['all'], res['one']
    return out


if __name__ == '__main__':
    main()
