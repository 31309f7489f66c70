"""Benchmark: world physics substeps/s of the MI355X world-local control step on one GPU.

A "step" is one control step of every world: ``substeps`` (25) physics substeps, one kernel launch,
inputs already resident in HBM.  ``value`` = nworld x substeps x steps / elapsed (whole job).
The roofline object prices the dominant kernel with the algorithmic bytes of the reference's
materialized dataflow per world-substep (formula B_alg in DESIGN.md) over the kernel's average
duration measured with HIP events on the launch stream.  ``cpu_baseline`` times the CPU FP64
oracle on the host cores on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--nworld N]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / 'gpu-libero_amd'))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
WORKLOADS = {'c2': 1024, 'c1': 2, 'c3': 4096, 'c4': 8192, 'c5': 16384}


def balg_bytes(m, rows=0, contacts=0, candidates=0, iterations=0):
    """Algorithmic bytes per world-substep of the reference dataflow (SURVEY section 8(d) formula):
    every array of the reference's materialized stages counted once per producer write and once per
    consumer read, in 4-byte words."""
    nq, nv, nb, ng, ns, nj = m.nq, m.nv, m.nbody, m.ngeom, m.nsite, m.njnt
    nC = m.nMpair
    P = (nv + 3) // 4 * 4
    R, C, K, it = rows, contacts, candidates, iterations
    words = (nq + 57 * nb + 12 * (ng + ns) + 6 * nj + 6 * nv + nC
             + 2 * nC + nv
             + (12 * ng + 5 * K * 2 + 24 * K + 42 * C * 3 if (R or C) else 0)
             + R * P + 8 * R + R * P
             + nv + 6 * nv + 10 * nb + 24 * nb + 10 * nv
             + 49 + 12 * nv + 60 + 6 * nv + 600
             + it * (3 * R * P + (2 + 2 * (nv > 32)) * P * P + 14 * R + 6 * nv + nC)
             + 24 * nb + 14 * nv + 2 * nC + nq)
    return 4 * words


def cpu_baseline(config, nworld_gpu, substeps, seed, budget_s=12.0):
    """Oracle (CPU FP64) world-substeps/s on all host cores, on a bounded sample of worlds."""
    from libero_hip import scene as S
    from libero_hip.model import Model
    from tests.helpers import make_oracle
    cores = len(os.sched_getaffinity(0))
    cores = min(cores, 16)
    sample = min(nworld_gpu, max(cores * 8, 64))
    sc = S.make_scene(config, sample, seed=seed, substeps=substeps)
    m = Model(sc)
    om, od = make_oracle(m, sample)
    od['qpos'][:] = sc.init_qpos
    od.forward(None, 8 | 2, threads=cores)
    acts = S.make_actions(sample, 64, seed=seed)
    done, t0 = 0, time.perf_counter()
    while True:
        od['osc_action'][:] = acts[done % 64]
        od.control_step(substeps, 1, threads=cores, pin=True)
        done += 1
        el = time.perf_counter() - t0
        if el > budget_s or done >= 64:
            break
    rate = sample * substeps * done / el
    return dict(value=rate, unit='world-substeps/s', cores=cores, kind='port',
                sample='%d worlds x %d control steps x %d substeps of %s (oracle FP64, %d threads)'
                       % (sample, done, substeps, config, cores))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--config', default='c2')
    ap.add_argument('--nworld', type=int, default=0)
    ap.add_argument('--substeps', type=int, default=25)
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--no-cpu', action='store_true')
    args = ap.parse_args()
    if args.gpus != 1:
        print('bench.py: this backend runs on one GPU per process; --gpus %d is not provided '
              '(worlds shard by contiguous ranges, one process per GPU; see DESIGN.md)' % args.gpus)
        sys.exit(2)
    import torch
    from libero_hip import scene as S, native
    from libero_hip.model import Model
    if not torch.cuda.is_available():
        print('bench.py needs a ROCm GPU', file=sys.stderr)
        sys.exit(1)
    nworld = args.nworld or WORKLOADS[args.config]
    sc = S.make_scene(args.config, nworld, seed=args.seed, substeps=args.substeps)
    m = Model(sc)
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, nworld)
    dd['qpos'].copy_(torch.from_numpy(sc.init_qpos))
    dd['osc_gains'].copy_(torch.from_numpy(np.tile(np.r_[sc.osc['kp'], sc.osc['kd']], (nworld, 1))))
    dd['osc_q0'].copy_(torch.from_numpy(np.tile(sc.osc['q0'], (nworld, 1))))
    dd['body_active'].fill_(1)
    stream = torch.cuda.Stream()
    ncontrol = args.warmup + args.steps
    acts = torch.from_numpy(S.make_actions(nworld, ncontrol, seed=args.seed)).to('cuda')
    with torch.cuda.stream(stream):
        dd.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL, stream)
        for k in range(args.warmup):
            dd['osc_action'].copy_(acts[k])
            dd.control_step(args.substeps, native.FLAG_POLICY_FIRST, stream)
    stream.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for k in range(args.steps):
            dd['osc_action'].copy_(acts[args.warmup + k])
            starts[k].record(stream)
            dd.control_step(args.substeps, native.FLAG_POLICY_FIRST, stream)
            ends[k].record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    errors = dd['osc_error'].cpu().numpy()
    if errors.any():
        print('controller errors in %d worlds' % int((errors != 0).sum()), file=sys.stderr)
    kavg = float(np.mean(kernel_ms))
    value = nworld * args.substeps * args.steps / elapsed
    # per-world rows R, contacts C and Newton iterations `it` of the last substep, read back from
    # the device counters; candidates K counted as C (a lower bound, so B_alg is not inflated)
    if m.njmax > 0:
        R = dd['nefc'].cpu().numpy()[:, 0].astype(float)
        C = dd['ncon'].cpu().numpy()[:, 0].astype(float)
        it = dd['solver_niter'].cpu().numpy()[:, 0].astype(float)
        balg = float(np.mean([balg_bytes(m, r, c, c, i) for r, c, i in zip(R, C, it)]))
        counters = {'rows_mean': float(R.mean()), 'contacts_mean': float(C.mean()),
                    'newton_iterations_mean': float(it.mean())}
    else:
        balg = balg_bytes(m)
        counters = {}
    per_launch = balg * nworld * args.substeps
    achieved = per_launch / (kavg * 1e-3) / 1e9
    traffic = None
    tfile = ROOT / 'profiles' / ('traffic_%s.json' % args.config)
    if tfile.exists():
        try:
            t = json.loads(tfile.read_text())
            if t.get('nworld') == nworld and t.get('substeps') == args.substeps:
                traffic = t.get('bytes_per_launch')
        except ValueError:
            traffic = None
    out = {
        'metric': 'world physics substeps/sec at N worlds on 1 MI355X; % HBM roofline',
        'value': value, 'unit': 'world-substeps/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': elapsed / args.steps * 1e3, 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32 (FP64 OSC)', 'data': 'synthetic',
        'config': {'workload': '%s: %s' % (args.config, m.summary()), 'nworld': nworld,
                   'substeps_per_step': args.substeps, 'scene_seed': args.seed,
                   'kernel_ms_avg': kavg, 'lds_bytes_per_world': dm.lds_bytes(), **counters,
                   'parallelism': 'one wavefront per world, world-local'},
        'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': achieved / HBM_PEAK_GBS, 'traffic': traffic,
                     'balg_bytes_per_world_substep': balg},
    }
    if not args.no_cpu:
        out['cpu_baseline'] = cpu_baseline(args.config, nworld, args.substeps, args.seed)
    print(json.dumps(out))


if __name__ == '__main__':
    main()
