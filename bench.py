#!/usr/bin/env python3
"""Throughput of the batched NES environment step on one MI355X (emulated frames/s and decisions/s).

    python bench.py [--steps K] [--warmup W] [--consoles 8192] [--no-cpu]

A step is one decision of every console: 4 emulated frames each (6502 + PPU + mapper), each frame's 224x240
colour-index picture and emphasis written to HBM, then the reward10 tracker, the outputs and the restart pass
(rl/csrc/rlenv.cu:145-170 is the reference's launch order for one decision).

Workload "nrom128-raw-frames" (the headline one): 8192 consoles of the seed-generated NROM-128 cartridge
(rl.synth.nrom_cart(1): 16 KB PRG of generated 6502 code, 8 KB random CHR), per console and decision a pad byte
uniform over 0..255, sticky repeat with p = 0.25 per frame, no dropout, no idle frames, raw uint8 frames
[N, 4, 224, 240] plus emphasis and a 2 KB RAM hash per console to HBM. The SMB reward reader sees RAM bytes the cart
never writes, so no episode ends within 1800 decisions (the stall clock needs 7200 frames): the restart kernels
launch but find no console to restart.

Timing: W untimed decisions, then K decisions between two device synchronisations; value = consoles * K / seconds.
Inputs (the pad bytes of every decision) are resident in HBM before the timed region. With --kernel-clock (default
on) the library brackets every launch with HIP events on the stream it runs on, which gives each kernel's average
duration over the same timed region; the roofline is computed for the kernel that takes the most time.

Parity: after the warmup the first 64 consoles' pictures, emphasis, rewards, dones and RAM hashes are compared with
the CPU oracle run on the same seeds and pad bytes; the oracle's run then continues as the timed CPU baseline
(a bounded sample of the same workload: 64 consoles, about --cpu-seconds of wall time, all host threads; plus a
1-thread sample).
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
TRAFFIC = ROOT / 'profiles' / 'traffic.json'
HBM_PEAK_GBPS = 8000.0
KERNELS = ('k_emu', 'k_render', 'k_finish', 'k_reset_copy', 'k_emu_restart', 'k_render_restart', 'k_reset_finish',
           'k_decision')

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
}
DECISION_BYTES = 4 * (PICTURE_BYTES + 1) + 2 + 4 + 1 + 4 + 28 + 19 + 360   # 216,358 B per console per decision
ALG_BYTES['k_decision'] = DECISION_BYTES + 8                          # the fused decision, RAM hash included


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=64)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--consoles', type=int, default=8192)
    ap.add_argument('--cart-seed', type=int, default=1)
    ap.add_argument('--seed', type=int, default=1)
    ap.add_argument('--cpw', type=int, default=0, help='consoles per wavefront of k_emu (0 = library default)')
    ap.add_argument('--emu', choices=('lane', 'wave'), default=None,
                    help='emulation kernel: one console per lane (k_emu) or per wavefront (k_emu_w)')
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
    if args.cpw:
        os.environ['RLENV_CPW'] = str(args.cpw)
    if args.emu:
        os.environ['RLENV_EMU'] = args.emu

    import torch
    from rl import synth
    from rl.rlenv import RlEnv

    if not torch.cuda.is_available():
        sys.exit('bench.py needs a HIP device')
    dev = torch.device('cuda:0')
    N, W, K = args.consoles, args.warmup, args.steps
    cart = synth.nrom_cart(args.cart_seed)
    kw = dict(seed=args.seed, sticky=True, idle_max=0, dropout=False, pad_mode=True, ram_hash=True,
              roms={'smb': cart})
    gen = torch.Generator().manual_seed(args.seed)
    pads_host = torch.randint(0, 256, (W + K, N), generator=gen, dtype=torch.int16)
    pads = pads_host.to(dev)

    print(f'[bench] workload nrom128-raw-frames: {N} consoles, warmup {W}, timed {K} decisions', file=sys.stderr,
          flush=True)
    env = RlEnv({'smb': N}, device=dev, **kw)
    env.start()
    for t in range(W):
        env.actions.copy_(pads[t])
        env.step()
    torch.cuda.synchronize()
    ncmp = min(args.cpu_consoles, N)
    snap = {k: getattr(env, k)[:ncmp].cpu().numpy() for k in ('obs', 'emph', 'reward', 'done', 'ram_hash')}
    instr0 = _instructions(env)
    print('[bench] warmup done', file=sys.stderr, flush=True)

    clock = not args.no_kernel_clock
    if clock:
        env.lib.rlenv_set_kernel_timing.argtypes = [ctypes.c_void_p, ctypes.c_int]
        env.lib.rlenv_kernel_times.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        env.lib.rlenv_set_kernel_timing(env.h, 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(W, W + K):
        env.actions.copy_(pads[t])
        env.step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    kern = {}
    if clock:
        ms = np.zeros(len(KERNELS), np.float64)
        cnt = np.zeros(len(KERNELS), np.int64)
        if env.lib.rlenv_kernel_times(env.h, ms.ctypes.data, cnt.ctypes.data, len(KERNELS)) != 0:
            raise RuntimeError(env.lib.rlenv_error().decode())
        env.lib.rlenv_set_kernel_timing(env.h, 0)
        for name, m, c in zip(KERNELS, ms, cnt):
            if c == 0:
                continue
            per = m / c
            alg = ALG_BYTES[name] * N
            kern[name] = dict(ms_per_launch=round(per, 4), launches_per_step=round(c / K, 3),
                              ms_per_step=round(m / K, 3), share=round(m / (dt * 1e3), 4),
                              alg_bytes_per_launch=alg, achieved_gbps=round(alg / (per * 1e-3) / 1e9, 3))
    instr1 = _instructions(env)
    done_any = int(env.done.sum().item())
    print(f'[bench] timed region {dt:.3f} s', file=sys.stderr, flush=True)

    decisions = N * K / dt
    out = dict(metric=METRIC, value=round(decisions, 1), unit='decisions/s', frames_per_s=round(4 * decisions, 1),
               n_gpus=1, steps=K, warmup=W, ms_per_step=round(dt * 1e3 / K, 3), higher_is_better=True,
               scaling='weak', vs_baseline=None, dtype='u8',
               data='synthetic: seed-generated NROM-128 cartridge (rl.synth.nrom_cart), uniform random pad bytes',
               config=dict(workload='nrom128-raw-frames', consoles=N, frames_per_decision=4,
                           cart=f'rl.synth.nrom_cart({args.cart_seed})', pads='uniform 0..255, sticky p=0.25',
                           dropout=False, idle_max=0, outputs='raw u8 frames [N,4,224,240] + emphasis + RAM hash',
                           episode_ends_in_timed_region=done_any),
               emulated_instructions_per_s=round(float(instr1 - instr0) / dt, 1),
               step_hbm_gbps=round(DECISION_BYTES * N * K / dt / 1e9, 3))
    if kern:
        dom = max(kern, key=lambda k: kern[k]['ms_per_step'])
        d = kern[dom]
        achieved = d['achieved_gbps']
        out['roofline'] = dict(kernel=dom, bound='hbm', achieved=achieved, peak=HBM_PEAK_GBPS, unit='GB/s',
                               frac=round(achieved / HBM_PEAK_GBPS, 6), traffic=_traffic(dom, N))
        if dom == 'k_emu':
            out['roofline']['note'] = ('k_emu interprets 6502 code one console per lane: it is bound by VALU issue '
                                       'and divergence, not HBM; its algorithmic bytes are the pad byte and action')
        out['kernels'] = kern
    if not args.no_cpu:
        out['parity'], out['cpu_baseline'], out['cpu_baseline_1thread'] = _cpu(args, cart, kw, pads_host, snap, ncmp)
    print(json.dumps(out), flush=True)
    if not args.no_cpu and not out['parity']['bit_exact']:
        sys.exit(3)


def _instructions(env) -> int:
    """Emulated 6502 instructions of every console so far (record field instr_lo, u32 at 0x14)."""
    import torch
    torch.cuda.synchronize()
    rec = env.consoles(0)
    return int(np.frombuffer(np.ascontiguousarray(rec[:, 0x14:0x18]).tobytes(), np.uint32).astype(np.int64).sum())


def _traffic(kernel, n):
    """HBM bytes per launch of `kernel` from the committed counter summary (FETCH_SIZE + WRITE_SIZE, scaled by the
    copy-kernel calibration), scaled to n consoles; None when no summary covers it."""
    if not TRAFFIC.exists():
        return None
    t = json.loads(TRAFFIC.read_text()).get(kernel)
    if not t:
        return None
    return round(t['bytes_per_console_launch'] * n)


def _cpu(args, cart, kw, pads_host, snap, ncmp):
    """Parity of the first ncmp consoles after the warmup, then the CPU baseline (oracle) on the same workload."""
    from rl.rlenv import RlEnv
    lib = ctypes.CDLL(str(ORACLE_LIB))
    lib.orc_set_threads.argtypes = [ctypes.c_int]
    threads = int(os.environ.get('OMP_NUM_THREADS', '0')) or min(os.cpu_count() or 1, 16)
    W = args.warmup
    res = {}
    for label, nthr, budget in (('all', threads, args.cpu_seconds), ('one', 1, max(2.0, args.cpu_seconds / 3))):
        lib.orc_set_threads(nthr)
        cpu = RlEnv({'smb': ncmp}, device='cpu', lib_path=ORACLE_LIB, **kw)
        cpu.start()
        t = 0
        for t in range(W):
            cpu.actions.copy_(pads_host[t, :ncmp])
            cpu.step()
        if label == 'all':
            bad = [k for k in snap if not np.array_equal(snap[k], getattr(cpu, k).numpy())]
            parity = dict(consoles=ncmp, decisions=W, bit_exact=not bad, differs=bad,
                          outputs=sorted(snap))
            print(f'[bench] parity vs oracle on {ncmp} consoles x {W} decisions: '
                  f'{"bit-exact" if not bad else "DIFFERS in " + ",".join(bad)}', file=sys.stderr, flush=True)
        gen = np.random.default_rng(args.seed + 7)
        t0 = time.perf_counter()
        d = 0
        while True:
            cpu.actions.copy_(torch_int16(gen.integers(0, 256, ncmp)))
            cpu.step()
            d += 1
            el = time.perf_counter() - t0
            if el >= budget and d >= 2:
                break
        res[label] = dict(value=round(ncmp * d / el, 2), unit='decisions/s', cores=nthr, kind='port',
                          sample=f'CPU oracle (oracle/, C, OpenMP over consoles) on {ncmp} consoles of the same '
                                 f'NROM-128 cart and pad distribution, {d} decisions x 4 frames in {el:.1f} s, '
                                 f'{nthr} thread(s)')
        del cpu
    return parity, res['all'], res['one']


def torch_int16(a):
    import torch
    return torch.from_numpy(np.asarray(a, np.int16))


if __name__ == '__main__':
    main()
