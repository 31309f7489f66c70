"""Benchmark: world physics substeps/s of the MI355X world-local control step on one GPU.

A "step" is one control step of every world: ``substeps`` (25) physics substeps, one kernel launch,
inputs already resident in HBM.  ``value`` = nworld x substeps x steps / elapsed (whole job).
The roofline object prices the dominant kernel with the algorithmic bytes of the reference's
materialized dataflow per world-substep (``balg_bytes``) over the kernel's average duration
measured with HIP events on the launch stream.  ``cpu_baseline`` times the CPU FP64
oracle on the host cores on a bounded sample of the same workload.

The default workload is config 3 (4096 contact-rich worlds: arm, table, 2 boxes, 2 capsules, 2
hulls), the configuration the metric's target is quoted on; configs 1, 2, 4 and 5 are selected
with --config c1 | c2 | c4 | c5.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3] [--nworld N]
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
# per-world overflow bits (include/mx_physics.h); the solver's iteration limits are legal exits,
# every other bit means a launch computed nothing or dropped contacts or rows
OVERFLOW_BITS = {'nefc': 1 << 0, 'broadphase': 1 << 2, 'narrowphase': 1 << 3, 'ccd': 1 << 4,
                 'epa_horizon': 1 << 8, 'iterations': 1 << 9, 'ls_iterations': 1 << 10, 'launch': 1 << 12}
LEGAL_EXITS = OVERFLOW_BITS['iterations'] | OVERFLOW_BITS['ls_iterations']


def launch_health(dd):
    """Worlds per overflow bit and worlds with a controller error, read after the timed launches
    (capacity and failure bits are sticky on the device, so one read covers every launch)."""
    ovf = dd['overflow'].cpu().numpy()[:, 0]
    err = dd['osc_error'].cpu().numpy()[:, 0]
    counts = {name: int(((ovf & bit) != 0).sum()) for name, bit in OVERFLOW_BITS.items()}
    counts['controller_error'] = int((err != 0).sum())
    bad = int(((ovf & ~LEGAL_EXITS) != 0).sum()) + counts['controller_error']
    return counts, bad


def padded_nv(nv):
    """The reference's padded dof count of its dense Newton arrays
    (gpu/host/backends/cuda_fp32/model.py:27): multiples of 4 up to 32 dofs, else of 16 with one
    spare column."""
    return ((nv + int(nv > 32) + 15) // 16) * 16 if nv > 32 else ((nv + 3) // 4) * 4


def balg_bytes(m, rows=0, contacts=0, candidates=0, iterations=0, iter_rows=None):
    """Algorithmic bytes per world-substep of the reference's materialized dataflow: every array
    of the reference's stages (one leaf kernel each, state through HBM in between) counted once per
    producer write and once per consumer read, in 4-byte words.  The figure is linear in rows R,
    contacts C, candidates K, iterations it and their product it R (iter_rows, default it x R), so
    the means of these over many world-substeps give the mean figure."""
    nq, nv, nb, ng, ns, nj = m.nq, m.nv, m.nbody, m.ngeom, m.nsite, m.njnt
    nC = m.nMpair
    P = padded_nv(nv)
    R, C, K, it = (np.asarray(x, float) for x in (rows, contacts, candidates, iterations))
    itR = it * R if iter_rows is None else np.asarray(iter_rows, float)
    words = (nq + 57 * nb + 12 * (ng + ns) + 6 * nj + 6 * nv + nC
             + 2 * nC + nv
             + np.where((R > 0) | (C > 0), 12 * ng + 5 * K * 2 + 24 * K + 42 * C * 3, 0)
             + R * P + 8 * R + R * P
             + nv + 6 * nv + 10 * nb + 24 * nb + 10 * nv
             + 49 + 12 * nv + 60 + 6 * nv + 600
             + itR * (3 * P + 14) + it * ((2 + 2 * (nv > 32)) * P * P + 6 * nv + nC)
             + 24 * nb + 14 * nv + 2 * nC + nq)
    return 4 * words


def cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def _oracle_rate(config, sample, substeps, seed, threads, budget_s):
    from libero_hip import scene as S
    from libero_hip.model import Model
    from tests.helpers import make_oracle
    sc = S.make_scene(config, sample, seed=seed, substeps=substeps)
    m = Model(sc)
    om, od = make_oracle(m, sample)
    od['qpos'][:] = sc.init_qpos
    od.forward(None, 8 | 2, threads=threads)
    acts = S.make_actions(sample, 64, seed=seed)
    done, t0 = 0, time.perf_counter()
    while True:
        od['osc_action'][:] = acts[done % 64]
        od.control_step(substeps, 1, threads=threads, pin=True)
        done += 1
        el = time.perf_counter() - t0
        if el > budget_s or done >= 64:
            break
    return sample * substeps * done / el, done


def cpu_baseline(config, nworld_gpu, substeps, seed, budget_s=12.0):
    """Oracle (CPU FP64) world-substeps/s with one pinned thread per core over the host cores this
    process may use (at most 16, the GPU box's share), on a bounded sample of worlds; a one-core
    figure on a smaller sample beside it."""
    cores = min(len(os.sched_getaffinity(0)), 16)
    sample = min(nworld_gpu, max(cores * 8, 64))
    rate, done = _oracle_rate(config, sample, substeps, seed, cores, budget_s)
    one_sample = min(nworld_gpu, 8)
    rate1, done1 = _oracle_rate(config, one_sample, substeps, seed, 1, budget_s / 3)
    return dict(value=rate, unit='world-substeps/s', cores=cores, kind='port',
                sample='%d worlds x %d control steps x %d substeps of %s (oracle FP64, %d pinned threads)'
                       % (sample, done, substeps, config, cores),
                one_core=rate1,
                one_core_sample='%d worlds x %d control steps, 1 thread' % (one_sample, done1),
                cpu_model=cpu_model(), nproc=os.cpu_count(),
                smt=_smt())


def _smt():
    try:
        return int(open('/sys/devices/system/cpu/smt/active').read().strip()) == 1
    except (OSError, ValueError):
        return None


def copy_bandwidth_gbs(torch, nbytes=1 << 30, reps=10):
    """Measured device-to-device copy bandwidth (read + write bytes over time), for the roofline's
    achieved-HBM denominator beside the datasheet figure."""
    a = torch.empty(nbytes // 4, dtype=torch.float32, device='cuda')
    b = torch.empty_like(a)
    a.fill_(1.0)
    b.copy_(a)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        b.copy_(a)
    t1.record()
    torch.cuda.synchronize()
    gbs = 2 * nbytes * reps / (t0.elapsed_time(t1) * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return gbs


def timed_launches(dispatches, warmup, steps):
    """The timed control steps among a run's control_step_kernel dispatches, in launch order: after
    the bootstrap forward pass and the warm-up steps, before the c5 split's standalone-controller
    and controller-off launches."""
    return dispatches[1 + warmup:1 + warmup + steps]


def _counter_rows(folder, counter):
    import csv
    rows = []
    for f in sorted(Path(folder).rglob('*_counter_collection.csv')):
        for r in csv.DictReader(open(f)):
            if r['Counter_Name'] == counter:
                rows.append(r)
    rows.sort(key=lambda r: int(r['Dispatch_Id']))
    return rows


def traffic_from(config, nworld, substeps, steps, warmup, fetch_dir, write_dir):
    """HBM bytes per launch of control_step_kernel from two rocprofv3 --pmc runs of this script
    (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled by what the same counter reads for
    the 1 GiB device copies of copy_bandwidth_gbs in the same run.  Writes
    profiles/traffic_<config>.json, which later bench lines report as roofline.traffic."""
    out = {'config': config, 'nworld': nworld, 'substeps': substeps}
    total = 0.0
    for name, folder in (('FETCH_SIZE', fetch_dir), ('WRITE_SIZE', write_dir)):
        rows = _counter_rows(folder, name)
        kern = timed_launches([float(r['Counter_Value']) for r in rows if 'control_step_kernel' in r['Kernel_Name']],
                              warmup, steps)
        copies = [r for r in rows if 'copy' in r['Kernel_Name'].lower()]
        big = max(int(r['Grid_Size']) for r in copies)
        copy_kib = [float(r['Counter_Value']) for r in copies if int(r['Grid_Size']) == big]
        factor = (1 << 20) / float(np.median(copy_kib))      # a 1 GiB copy reads and writes 2^20 KiB
        per = float(np.mean(kern)) * 1024 * factor
        out[name.lower()] = {'kib_per_dispatch_raw': float(np.mean(kern)), 'dispatches': len(kern),
                             'copy_kib_raw': float(np.median(copy_kib)), 'copy_grid': big,
                             'scale': factor, 'bytes_per_launch': per}
        total += per
    out['bytes_per_launch'] = total
    out['commands'] = ['cd /tmp && rocprofv3 --pmc %s -d <dir> -o %s --output-format csv -- python3 '
                       '$GRAFT_REPO_ROOT/bench.py --config %s --steps %d --warmup %d --no-cpu'
                       % (c, c[0].lower(), config, steps, warmup) for c in ('FETCH_SIZE', 'WRITE_SIZE')]
    out['derived_by'] = ('python bench.py --config %s --steps %d --warmup %d --traffic-from <FETCH_SIZE dir> '
                         '<WRITE_SIZE dir>' % (config, steps, warmup))
    path = ROOT / 'profiles' / ('traffic_%s.json' % config)
    path.write_text(json.dumps(out, indent=1) + '\n')
    print(json.dumps(out))


def trace_from(config, nworld, substeps, steps, warmup, folder):
    """Summary of a rocprofv3 --kernel-trace --stats run of this script (the kernel statistics, the
    launch shape and every control_step_kernel launch's duration); writes
    profiles/control_step_kernel_<config>_n<nworld>.md."""
    import csv
    folder = Path(folder)
    stats = next(folder.rglob('*_kernel_stats.csv'))
    trace = next(folder.rglob('*_kernel_trace.csv'))
    rows = list(csv.DictReader(open(trace)))
    rows.sort(key=lambda r: int(r['Start_Timestamp']))
    kern = [r for r in rows if 'control_step_kernel' in r['Kernel_Name']]
    ms = [(int(r['End_Timestamp']) - int(r['Start_Timestamp'])) * 1e-6 for r in kern]
    timed = timed_launches(ms, warmup, steps)
    k = kern[-1]
    cmd = ('cd /tmp && rocprofv3 --kernel-trace --stats -d <dir> -o %s --output-format csv -- python3 '
           '$GRAFT_REPO_ROOT/bench.py --config %s --no-cpu' % (config, config))
    lines = ['# control_step_kernel, workload %s (N=%d, %d substeps per launch)' % (config, nworld, substeps), '',
             'Command (on the MI355X box, repository at $GRAFT_REPO_ROOT):', '', '```', cmd, '```', '',
             'Derived by `python bench.py --config %s --trace-from <dir>`.' % config, '',
             'Launch shape: %s, grid %s threads in workgroups of %s (%s per world), arch VGPR %s, AGPR %s, '
             'SGPR %s, scratch %s B/lane (dynamic LDS is not shown by the trace).'
             % (k['Kernel_Name'], k['Grid_Size_X'], k['Workgroup_Size_X'],
                'one 64-lane wave' if int(k['Workgroup_Size_X']) == 64 else
                '%d 64-lane waves' % (int(k['Workgroup_Size_X']) // 64),
                k['VGPR_Count'], k['Accum_VGPR_Count'], k['SGPR_Count'], k['Scratch_Size']), '',
             '## --stats (kernel_stats.csv)', '',
             '| kernel | calls | avg ns | min ns | max ns | % |', '|---|---|---|---|---|---|']
    for r in csv.DictReader(open(stats)):
        lines.append('| %s | %s | %.0f | %s | %s | %s |' % (r['Name'][:60], r['Calls'], float(r['AverageNs']), r['MinNs'],
                                                          r['MaxNs'], r['Percentage']))
    lines += ['', '## control_step_kernel launches (kernel_trace.csv, ms)', '',
              'The first launch is the bootstrap forward (1 substep, no integration), then %d warmup steps '
              'and the %d timed control steps of %d substeps (for c5, the controller-off launches of its '
              'split follow).' % (warmup, steps, substeps), '',
              ' '.join('%.3f' % x for x in ms), '',
              '**Average over the %d timed launches: %.3f ms** (median %.3f, min %.3f, max %.3f)'
              % (len(timed), float(np.mean(timed)), float(np.median(timed)), min(timed), max(timed)), '']
    path = ROOT / 'profiles' / ('control_step_kernel_%s_n%d.md' % (config, nworld))
    path.write_text('\n'.join(lines))
    print('\n'.join(lines))


# SQ / GRBM counter passes of control_step_kernel (each within one run's hardware limits: at most 8
# SQ and 2 GRBM counters), and how the summary derives its figures from them
COUNTER_PASSES = (
    ('SQ_WAVES', 'SQ_WAVE_CYCLES', 'SQ_BUSY_CYCLES', 'SQ_WAIT_ANY', 'SQ_WAIT_INST_ANY', 'SQ_ACTIVE_INST_ANY',
     'GRBM_GUI_ACTIVE', 'GRBM_COUNT'),
    ('SQ_INSTS_VALU', 'SQ_INSTS_SALU', 'SQ_INSTS_LDS', 'SQ_INSTS_VMEM_RD', 'SQ_INSTS_VMEM_WR', 'SQ_INSTS_SMEM',
     'SQ_ACTIVE_INST_VALU', 'SQ_THREAD_CYCLES_VALU'),
    ('SQ_LDS_BANK_CONFLICT', 'SQ_LDS_ADDR_CONFLICT', 'SQ_LDS_UNALIGNED_STALL', 'SQ_ACTIVE_INST_LDS',
     'SQ_WAIT_INST_LDS', 'SQ_INSTS_FLAT', 'SQ_INSTS_VALU_FLOPS_FP64', 'SQ_INSTS_VALU_FLOPS_FP32'),
)
# GRBM counters sum over the 8 XCDs; SQ cycle counters are in units of 4 cycles
XCDS, CUS, SIMDS_PER_CU = 8, 256, 4


def counters_from(config, nworld, substeps, steps, warmup, folders):
    """Summary of the SQ counter passes (rocprofv3 --pmc runs of this script, one folder per pass
    of COUNTER_PASSES, in order) for the timed control_step_kernel launches: instruction mix per
    wave, VALU busy and lane utilisation, wave-slot occupancy, the fraction of wave cycles waiting,
    LDS bank conflicts.  Writes profiles/counters_<config>.md."""
    vals = {}
    for names, folder in zip(COUNTER_PASSES, folders):
        for name in names:
            rows = timed_launches([r for r in _counter_rows(folder, name) if 'control_step_kernel' in r['Kernel_Name']],
                                  warmup, steps)
            if rows:
                vals[name] = float(np.mean([float(r['Counter_Value']) for r in rows]))
    g = lambda k: vals.get(k, float('nan'))
    waves = g('SQ_WAVES')
    cycles = g('GRBM_GUI_ACTIVE') / XCDS          # GPU-active cycles of the launch
    lines = ['# SQ counters: control_step_kernel, workload %s (N=%d, %d substeps per launch)' % (config, nworld, substeps), '',
             'Averages over the %d timed launches of `python3 bench.py --config %s --no-cpu` (one launch = one' % (steps, config),
             'control step of every world). Commands, one pass each (run from /tmp):', '', '```']
    for names in COUNTER_PASSES:
        lines.append('rocprofv3 --pmc %s -d <dir> -o pmc --output-format csv -- python3 $GRAFT_REPO_ROOT/bench.py '
                     '--config %s --no-cpu' % (' '.join(names), config))
    lines += ['```', '', 'Derived by `python bench.py --config %s --counters-from <pass dirs>`.' % config, '',
              '| figure | value | from |', '|---|---|---|']
    rows = [
        ('waves per launch', '%.0f' % waves, 'SQ_WAVES'),
        ('VALU instructions per wave', '%.0f' % (g('SQ_INSTS_VALU') / waves), 'SQ_INSTS_VALU / SQ_WAVES'),
        ('SALU instructions per wave', '%.0f' % (g('SQ_INSTS_SALU') / waves), 'SQ_INSTS_SALU / SQ_WAVES'),
        ('LDS instructions per wave', '%.0f' % (g('SQ_INSTS_LDS') / waves), 'SQ_INSTS_LDS / SQ_WAVES'),
        ('vector memory reads / writes per wave', '%.0f / %.0f' % (g('SQ_INSTS_VMEM_RD') / waves, g('SQ_INSTS_VMEM_WR') / waves),
         'SQ_INSTS_VMEM_RD, _WR / SQ_WAVES'),
        ('scalar memory instructions per wave', '%.0f' % (g('SQ_INSTS_SMEM') / waves), 'SQ_INSTS_SMEM / SQ_WAVES'),
        ('wave cycles waiting on a dependency', '%.1f %%' % (100 * g('SQ_WAIT_ANY') / g('SQ_WAVE_CYCLES')),
         'SQ_WAIT_ANY / SQ_WAVE_CYCLES'),
        ('wave cycles waiting for an instruction to issue', '%.1f %%' % (100 * g('SQ_WAIT_INST_ANY') / g('SQ_WAVE_CYCLES')),
         'SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES'),
        ('VALU busy (per SIMD, of GPU-active cycles)',
         '%.1f %%' % (100 * 4 * g('SQ_ACTIVE_INST_VALU') / (SIMDS_PER_CU * CUS) / cycles),
         '4 x SQ_ACTIVE_INST_VALU / (1024 SIMDs x GRBM_GUI_ACTIVE / 8)'),
        ('VALU lane utilisation', '%.1f %%' % (100 * g('SQ_THREAD_CYCLES_VALU') / (64 * g('SQ_ACTIVE_INST_VALU'))),
         'SQ_THREAD_CYCLES_VALU / (64 x SQ_ACTIVE_INST_VALU)'),
        ('mean resident waves per CU', '%.1f' % (4 * g('SQ_WAVE_CYCLES') / cycles / CUS),
         '4 x SQ_WAVE_CYCLES / (GRBM_GUI_ACTIVE / 8) / 256'),
        ('LDS bank-conflict cycles per LDS-active cycle', '%.2f %%' % (100 * g('SQ_LDS_BANK_CONFLICT') / g('SQ_ACTIVE_INST_LDS')),
         'SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS'),
        ('wave cycles waiting on LDS', '%.1f %%' % (100 * g('SQ_WAIT_INST_LDS') / g('SQ_WAVE_CYCLES')),
         'SQ_WAIT_INST_LDS / SQ_WAVE_CYCLES'),
        ('flat (generic address) instructions per wave', '%.0f' % (g('SQ_INSTS_FLAT') / waves), 'SQ_INSTS_FLAT / SQ_WAVES'),
        ('FP32 / FP64 VALU FLOP counters per launch (FLOPs per instruction, MFMA excluded)',
         '%.3g / %.3g' % (g('SQ_INSTS_VALU_FLOPS_FP32'), g('SQ_INSTS_VALU_FLOPS_FP64')), 'SQ_INSTS_VALU_FLOPS_FP32, _FP64'),
        ('VALU lane-cycles used, of the VALU peak (busy x lane utilisation)',
         '%.1f %%' % (100 * g('SQ_THREAD_CYCLES_VALU') / 64 * 4 / (SIMDS_PER_CU * CUS) / cycles),
         'SQ_THREAD_CYCLES_VALU / 64 x 4 / (1024 SIMDs x GRBM_GUI_ACTIVE / 8)'),
    ]
    for r in rows:
        lines.append('| %s | %s | %s |' % r)
    lines += ['', 'Raw per-launch averages: ' + ', '.join('%s %.4g' % (k, v) for k, v in sorted(vals.items())), '']
    path = ROOT / 'profiles' / ('counters_%s.md' % config)
    path.write_text('\n'.join(lines))
    print('\n'.join(lines))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--config', default='c3')
    ap.add_argument('--nworld', type=int, default=0)
    ap.add_argument('--substeps', type=int, default=25)
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--precision', choices=('fp32', 'fp64'), default='fp32',
                    help='fp64: the FP64 route (physics in double, working set in LDS); a report beside the '
                         'FP32 line, not the metric')
    ap.add_argument('--traffic-from', nargs=2, metavar=('FETCH_DIR', 'WRITE_DIR'),
                    help='write profiles/traffic_<config>.json from two --pmc runs of this script')
    ap.add_argument('--trace-from', metavar='TRACE_DIR',
                    help='write profiles/control_step_kernel_<config>_n<N>.md from a --kernel-trace --stats run')
    ap.add_argument('--counters-from', nargs=len(COUNTER_PASSES), metavar='PASS_DIR',
                    help='write profiles/counters_<config>.md from the --pmc runs of COUNTER_PASSES')
    args = ap.parse_args()
    if args.traffic_from:
        traffic_from(args.config, args.nworld or WORKLOADS[args.config], args.substeps, args.steps, args.warmup,
                     *args.traffic_from)
        return
    if args.trace_from:
        trace_from(args.config, args.nworld or WORKLOADS[args.config], args.substeps, args.steps, args.warmup,
                   args.trace_from)
        return
    if args.counters_from:
        counters_from(args.config, args.nworld or WORKLOADS[args.config], args.substeps, args.steps, args.warmup,
                      args.counters_from)
        return
    if args.gpus != 1:
        print('bench.py: this backend runs on one GPU per process; --gpus %d is not provided '
              '(worlds shard by contiguous ranges, one process per GPU)' % args.gpus)
        sys.exit(2)
    import torch
    from libero_hip import scene as S, native, layout
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
    if m.body_active is None:
        dd['body_active'].fill_(1)
    else:                               # heterogeneous batch: parked object slots are masked
        dd['body_active'].copy_(torch.from_numpy(m.body_active))
    fp64 = args.precision == 'fp64'
    route = native.FLAG_FP64 if fp64 else 0
    if fp64 and dm.lds_bytes_fp64() > layout.LDS_BUDGET:
        print('bench.py: %s has no FP64 route (%d bytes of LDS per world)' % (args.config, dm.lds_bytes_fp64()),
              file=sys.stderr)
        sys.exit(2)
    stream = torch.cuda.Stream()
    ncontrol = args.warmup + args.steps
    toggle = 10 if args.config == 'c5' else 0    # C5 toggles the gripper every 10 controls
    acts = torch.from_numpy(S.make_actions(nworld, ncontrol, seed=args.seed, gripper_toggle=toggle)).to('cuda')
    with torch.cuda.stream(stream):
        dd.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL | route, stream)
        for k in range(args.warmup):
            dd['osc_action'].copy_(acts[k])
            dd.control_step(args.substeps, native.FLAG_POLICY_FIRST | route, stream)
    stream.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    dd['stat_sums'].zero_()             # row, contact and iteration sums of the timed substeps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for k in range(args.steps):
            dd['osc_action'].copy_(acts[args.warmup + k])
            starts[k].record(stream)
            dd.control_step(args.substeps, native.FLAG_POLICY_FIRST | route, stream)
            ends[k].record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    health, bad = launch_health(dd)
    kavg = float(np.mean(kernel_ms))
    value = nworld * args.substeps * args.steps / elapsed
    # rows R, contacts C, Newton iterations `it` and it x R over every timed world-substep, from the
    # kernel's per-world sums (candidates K counted as C, a lower bound)
    if m.njmax > 0:
        R, C, it, itR = (dd['stat_sums'].cpu().numpy() / (args.steps * args.substeps)).mean(axis=0)
        balg = float(balg_bytes(m, R, C, C, it, itR))
        counters = {'rows_mean': float(R), 'contacts_mean': float(C), 'newton_iterations_mean': float(it),
                    'counters_from': 'stat_sums over every timed world-substep'}
    else:
        balg = float(balg_bytes(m))
        counters = {}
    per_launch = balg * nworld * args.substeps
    achieved = per_launch / (kavg * 1e-3) / 1e9
    traffic = None
    tfile = ROOT / 'profiles' / ('traffic_%s.json' % args.config)
    if tfile.exists() and not fp64:
        try:
            t = json.loads(tfile.read_text())
            if t.get('nworld') == nworld and t.get('substeps') == args.substeps:
                traffic = t.get('bytes_per_launch')
        except ValueError:
            traffic = None
    split = {}
    if args.config == 'c5' and not fp64:
        # the FP64 OSC timed apart: its own kernel (mx_osc, every world's controller from the inputs
        # the last substep published, once per launch), and the same control steps once more with
        # the controller off (ctrl held), whose kernel time is the FP32 physics alone
        with torch.cuda.stream(stream):
            dd.osc(0, stream)              # untimed first call: loads the controller's code object
        stream.synchronize()
        with torch.cuda.stream(stream):
            for k in range(args.steps):
                starts[k].record(stream)
                dd.osc(0, stream)
                ends[k].record(stream)
        stream.synchronize()
        oavg = float(np.mean([s.elapsed_time(e) for s, e in zip(starts, ends)]))
        with torch.cuda.stream(stream):
            for k in range(args.steps):
                starts[k].record(stream)
                dd.control_step(args.substeps, native.FLAG_NO_CONTROL, stream)
                ends[k].record(stream)
        stream.synchronize()
        phys = [s.elapsed_time(e) for s, e in zip(starts, ends)]
        pavg = float(np.mean(phys))
        health_off, bad_off = launch_health(dd)
        bad += bad_off
        split = {'physics_kernel_ms_avg': pavg, 'osc_kernel_ms_avg': oavg,
                 'osc_solves_per_s': nworld / (oavg * 1e-3),
                 'physics_world_substeps_per_s': nworld * args.substeps / (pavg * 1e-3)}
    copy_gbs = copy_bandwidth_gbs(torch)
    per_control = np.array(kernel_ms)
    timing = {'control_steps_per_s': args.steps / elapsed, 'control_ms_p50': float(np.percentile(per_control, 50)),
              'control_ms_p95': float(np.percentile(per_control, 95))}
    out = {
        'metric': 'world physics substeps/sec at N worlds on 1 MI355X; % HBM roofline',
        'value': value, 'unit': 'world-substeps/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': elapsed / args.steps * 1e3, 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f64 (FP64 route)' if fp64 else 'f32 (FP64 OSC)', 'data': 'synthetic',
        'config': {'workload': '%s: %s' % (args.config, m.summary()), 'nworld': nworld,
                   'substeps_per_step': args.substeps, 'scene_seed': args.seed,
                   'kernel_ms_avg': kavg, 'lds_bytes_per_world': dm.lds_bytes_fp64() if fp64 else dm.lds_bytes(),
                   **counters, **split, **timing,
                   'overflow_worlds': health,
                   'parallelism': ('two wavefronts per world (LDS route, smooth path), world-local'
                                   if m.njmax == 0 and (fp64 or dd.struct.workspace_doubles == 0)
                                   else 'one wavefront per world, world-local'),
                   'route': 'fp64 (LDS)' if fp64 else ('workspace' if m.njmax > 0 and dd.struct.workspace_doubles else 'lds')},
        'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': achieved / HBM_PEAK_GBS, 'traffic': traffic,
                     'balg_bytes_per_world_substep': balg, 'copy_gbs_measured': copy_gbs,
                     'frac_of_measured_copy': achieved / copy_gbs},
    }
    if bad:
        # a launch that set a capacity or failure bit (or a controller error) has no valid rate
        print('bench.py: %d worlds ended the timed launches with an overflow bit other than the solver '
              'iteration limits, or a controller error: %s' % (bad, json.dumps(health)), file=sys.stderr)
        print(json.dumps(out), file=sys.stderr)
        sys.exit(3)
    if not args.no_cpu:
        out['cpu_baseline'] = cpu_baseline(args.config, nworld, args.substeps, args.seed)
    print(json.dumps(out))


if __name__ == '__main__':
    main()
