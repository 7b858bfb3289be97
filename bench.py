"""SpMM benchmark: boo_matmul on the 3-D 27-point stencil (64^3, K=64, fp32).

Metric: SpMM GFLOP/s = 2*nnz*K/t, with the achieved HBM GB/s
of the algorithmic bytes 4(2nnz + m + 1) + 4K(x_rows + m) against MI355X's
8 TB/s.  One step = one boo_matmul of the whole matrix against one X.

Inputs are resident in HBM before timing starts, and the timed loop rotates
over NROT independent copies (matrix staging, X, Y) whose combined size is
well beyond the 256 MB Infinity Cache, so a step cannot be served from the
previous step's cached data.  Steps are issued through the C ABI with
preallocated outputs (the reference's timed-harness scope,
bindings/bindings_boo_timed.cu); the Python-API cost per call is reported
beside it.

Output: one JSON line on stdout (rank 0), as the driver expects.
    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config 2]
    python bench.py --calibrate-copy   # plain copy of known size, for rocprof scaling
    python bench.py --steps 5 --warmup 2 --no-pbr --no-cpu-baseline   # BOO only (counter runs)
    python bench.py --steps 5 --warmup 2 --no-boo --no-cpu-baseline   # PBR only (counter runs)
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PEAK_HBM_GBS = 8000.0
NROT = 4


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def bytes_alg(A, K):
    """4(2 nnz + m + 1) + 4K(x_rows_referenced + m): fp32 values, int32
    indices (reports/agent_loop/BENCH_SCHEMA.md:104 of the reference)."""
    m = A.shape[0]
    x_rows = int(np.unique(A.indices).size)
    return 4 * (2 * A.nnz + m + 1) + 4 * K * (x_rows + m)


def time_steps(fns, steps, warmup, torch):
    """Exactly `steps` calls (rotating over fns), bracketed by synchronize on
    both sides.  Returns (wall ms per step, GPU ms per step): the second is
    one HIP event pair on the launch stream around the whole timed region,
    divided by the step count, so no per-step marker sits between kernels."""
    for i in range(warmup):
        fns[i % len(fns)]()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        fns[i % len(fns)]()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall / steps * 1e3, e0.elapsed_time(e1) / steps


def cpu_baseline(A, spec, cfg, fmt, y_gpu):
    """The reference's own CPU ops, compiled from its sources into
    oracle/_ref, on the same matrix and X (seed 0), single-threaded:
    boo_batched_matmul_cpu (boo_matrix.cpp:336-396), pbr_batched_matmul_cpu
    (pbr_matrix.cpp:17-68) and the CSR row loop (boo_matrix.cpp:374-383, run
    over the whole matrix by building the BOO with every entry in the
    remainder).  `value` is the measured format's op; the GPU's Y for the
    same X (y_gpu: {'boo': .., 'pbr': ..}) is compared with the reference
    op's Y under the north star's bar, max |Y_gpu - Y_ref| / (|A||X|)."""
    import importlib
    import torch
    ref_dir = ROOT / 'oracle' / '_ref'
    if not any(ref_dir.glob('torch_fast_spdmm_core*.so')):
        return None
    sys.path.insert(0, str(ref_dir))
    ref = importlib.import_module('torch_fast_spdmm_core')
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O
    from spmm_amd import matrices as M
    K = spec['K']
    x = torch.from_numpy(M.dense_x(A.shape[1], K))
    rl = O.identity_labels(A.shape[0], 32)
    cl = O.identity_labels(A.shape[1], 32)
    thr = spec.get('pbr_threshold', 4)
    builds = {
        'boo': lambda: ref.csr_to_boo(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], rl, cl, 2, 4, 0),
        'pbr': lambda: ref.csr_to_pbr(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], 8, 8, thr),
        # threshold above any block's count: every entry goes to the remainder CSR
        'csr': lambda: ref.csr_to_boo(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], rl, cl, 2,
                                      1 << 30, 0),
    }
    ops = {'boo': ref.boo_batched_matmul_cpu, 'pbr': ref.pbr_batched_matmul_cpu, 'csr': ref.boo_batched_matmul_cpu}
    names = {'boo': 'boo_batched_matmul_cpu', 'pbr': 'pbr_batched_matmul_cpu',
             'csr': 'CSR row loop (boo_batched_matmul_cpu, all entries in the remainder)'}
    _, bound = O.spmm_reference(A, x.numpy())
    nthreads = torch.get_num_threads()
    torch.set_num_threads(1)
    res = {}
    # all three ops on configs up to ~8M nonzeros (about 10 s of CPU work);
    # above that only the measured format's op keeps the run bounded
    which = ('boo', 'pbr', 'csr') if A.nnz <= 8_000_000 else (fmt,)
    try:
        for k in which:
            b = builds[k]()
            y = ops[k](b, x)                                    # warmup, and the reference's Y
            ts = []
            for _ in range(3):
                t0 = time.perf_counter()
                ops[k](b, x)
                ts.append(time.perf_counter() - t0)
            t = sorted(ts)[1]
            r = {'gflops': round(2.0 * A.nnz * K / t / 1e9, 3), 'ms_per_call': round(t * 1e3, 1), 'op': names[k]}
            yg = y_gpu.get(k)
            if yg is not None:
                err = np.abs(np.asarray(yg, np.float64) - y.numpy()[0].astype(np.float64))
                with np.errstate(divide='ignore', invalid='ignore'):
                    ratio = np.where(bound > 0, err / np.where(bound > 0, bound, 1), np.where(err > 0, np.inf, 0))
                r['gpu_vs_reference_max_ratio'] = float(f'{float(ratio.max()):.3e}')
                r['gpu_vs_reference_ok'] = bool(np.all(err <= 1e-5 * bound))
            res[k] = r
            del b
    finally:
        torch.set_num_threads(nthreads)
    cpu_model = platform.processor() or 'x86_64'
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    cpu_model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    main = res[fmt]
    return {'value': main['gflops'], 'unit': 'GFLOP/s', 'cores': 1, 'kind': 'reference',
            'sample': f'full config-{cfg} matrix, K={K}, X seed 0: {names[fmt]}, 1 warmup + median of 3 '
                      f'({main["ms_per_call"]:.0f} ms/call), single thread',
            'ops': res, 'host_cpu': cpu_model, 'host_cores_available': len(os.sched_getaffinity(0))}


def vendor_baseline(S, A, K, Xs, steps, warmup, O, torch):
    """The vendor library on the same CSR and X: a persistent rocSPARSE SpMM
    plan per algorithm (spmm_amd.DirectSpMM, the reference's DirectSpMM over
    cuSPARSE, bindings/bindings_cusparse.cu:21-160), each call timed by its
    own native event pair (timed_run) and checked against the same fp64
    bound; the fastest algorithm that passes is the baseline."""
    crow = torch.from_numpy(A.indptr.astype(np.int32)).cuda()
    col = torch.from_numpy(A.indices.astype(np.int32)).cuda()
    val = torch.from_numpy(A.data.astype(np.float32)).cuda()
    x = Xs[0]
    per_alg = {}
    for alg in ('DEFAULT', 'csr', 'csr_row_split', 'csr_nnz_split', 'csr_merge_path'):
        try:
            plan = S.DirectSpMM(crow, col, val, x, alg)
            if not plan.info()['supported']:
                per_alg[alg] = {'supported': False}
                continue
            y = plan.run()
            torch.cuda.synchronize()
            ratio, ok = O.within_bound(y.cpu().numpy(), A, x.cpu().numpy(), 1e-5)
            for _ in range(warmup):
                plan.timed_run()
            ms = float(np.median([plan.timed_run() for _ in range(steps)]))
            per_alg[alg] = {'kernel_ms_median': round(ms, 5), 'parity_ratio': float(f'{ratio:.3e}'),
                            'parity_ok': bool(ok), 'workspace_bytes': int(plan.info()['workspace_bytes'])}
            del plan
        except Exception as exc:             # an algorithm this build cannot run: say so
            per_alg[alg] = {'error': f'{type(exc).__name__}: {exc}'[:160]}
    good = {a: r for a, r in per_alg.items() if r.get('parity_ok')}
    if not good:
        return {'error': 'no rocSPARSE algorithm ran within the bound', 'algorithms': per_alg}
    best = min(good, key=lambda a: good[a]['kernel_ms_median'])
    ms = good[best]['kernel_ms_median']
    return {'value': round(2.0 * A.nnz * K / (ms * 1e-3) / 1e9, 2), 'unit': 'GFLOP/s', 'kernel_ms': ms,
            'library': f'rocSPARSE generic SpMM, CSR int32 fp32, algorithm {best} (spmm_amd.DirectSpMM)',
            'parity_ratio': good[best]['parity_ratio'], 'parity_ok': True, 'algorithms': per_alg,
            'note': f'median of {steps} natively timed calls per algorithm; one X/CSR copy (MALL-resident)'}


def cpp_timed_boo(S, A, K, x, calls, torch):
    """One boo_matmul call between two native events on the construction
    stream (spmm_amd.BOOTimedSpMM.timed_run, the reference's C++-only timing
    scope, bindings/bindings_boo_timed.cu:254-270): the median of `calls`
    calls on one MALL-resident copy."""
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to(x.device)
    m = boo._gpu_meta
    timed = S.BOOTimedSpMM(boo.rows, boo.cols, boo.max_nr, boo.max_nc, boo.max_nnz_blk, m.row_grp_ptr,
                           m.row_ids, m.col_grp_ptr, m.col_ids, m.blk_row_grp, m.blk_col_grp, m.blk_nz_ptr,
                           m.blk_shift, m.nz_idx, m.nz_val, m.rem_indptr, m.rem_col_ind, m.rem_vals,
                           m.tail_row, m.tail_col, m.tail_val, x)
    for _ in range(3):
        timed.timed_run()
    ms = float(np.median([timed.timed_run() for _ in range(calls)]))
    return {'boo_us_median': round(ms * 1e3, 2), 'calls': calls,
            'scope': 'BOOTimedSpMM.timed_run: one boo_matmul call between two events, one MALL-resident copy'}


def traffic_from_profiles(workload):
    p = ROOT / 'profiles' / f'{workload}_traffic.json'
    if p.exists():
        try:
            return json.loads(p.read_text())
        except ValueError:
            return None
    return None


def calibrate_copy(torch):
    """A plain device copy of known size, for scaling FETCH_SIZE/WRITE_SIZE."""
    n = 128 * 1024 * 1024                                   # 512 MiB of fp32
    a = torch.ones(n, device='cuda')
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({'calibrate_copy_bytes_each_way': 4 * n, 'reps': 5}))


def bench_boo(S, A, K, Xs, Ys, dev, stream, args, O, torch):
    """Time boo_matmul's entry point over rotating copies; returns (wall ms,
    GPU ms per step, Python-API ms per call, parity ratio)."""
    nrot = len(Xs)
    boos = []
    labels = {}
    if args.cluster != 'identity':            # cluster once, build every copy from the labels
        t0 = time.perf_counter()
        rl, cl = S.clustering.cluster_axes(A, args.cluster, 32, 32, 32, 32, feasible_first=True)
        labels = dict(row_labels=rl, col_labels=cl)
        _log(f'{args.cluster} clustering: {time.perf_counter() - t0:.1f} s, {int(rl.max()) + 1} row groups')
    for _ in range(nrot):
        t0 = time.perf_counter()
        if labels:
            boos.append(S.csr_to_boo(A, target_nr=32, target_nc=32, **labels).to(dev))
        else:
            boos.append(S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to(dev))
        d = boos[-1]._gpu_meta.desc
        _log(f'BOO staged in {time.perf_counter() - t0:.1f} s: {d["n_tiles"]} tiles, {d["n_waves"]} waves, '
             f'{d["n_crow"]} gather rows, {d["n_long"]} long rows, {d["n_splits"]} split slices')
    ws_bytes = int(S._core.boo_workspace_bytes(boos[0]._gpu_meta.desc, 0, 1, K))
    wss = [torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) for _ in range(nrot)]

    def boo_step(i):
        S._core.boo_matmul_gpu(boos[i]._gpu_meta.desc, 0, int(Xs[i].data_ptr()), int(Ys[i].data_ptr()),
                               1, K, int(wss[i].data_ptr()), ws_bytes, int(stream))
    boo_fns = [lambda i=i: boo_step(i) for i in range(nrot)]
    # parity of the timed entry point against the fp64 product before timing
    boo_step(0)
    torch.cuda.synchronize()
    ratio, ok = O.within_bound(Ys[0][0].cpu().numpy(), A, Xs[0].cpu().numpy(), 1e-5)
    if not ok:
        _log(f'PARITY FAILURE: max |err|/(|A||X|) = {ratio:.3e}')
        sys.exit(1)
    ms_wall, ms_ev_mean = time_steps(boo_fns, args.steps, args.warmup, torch)
    api_fns = [lambda i=i: S.boo_matmul(boos[i], Xs[i]) for i in range(nrot)]
    ms_api, _ = time_steps(api_fns, min(args.steps, 20), 3, torch)
    _log(f'BOO: wall {ms_wall * 1e3:.1f} us/step, GPU (events over the timed region) '
         f'{ms_ev_mean * 1e3:.1f} us/step; python API {ms_api * 1e3:.1f} us/call; '
         f'parity ratio {ratio:.2e}')
    return ms_wall, ms_ev_mean, ms_api, ratio


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=50)
    ap.add_argument('--warmup', type=int, default=10)
    ap.add_argument('--config', type=int, default=2)
    ap.add_argument('--cluster', default='identity', choices=('identity', 'hem'),
                    help='BOO clustering (the headline workload is identity)')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-pbr', action='store_true', help='skip the PBR line (profiling runs)')
    ap.add_argument('--no-boo', action='store_true',
                    help='skip BOO, so PBR is the measured path (PBR counter runs)')
    ap.add_argument('--calibrate-copy', action='store_true')
    ap.add_argument('--no-vendor', action='store_true', help='skip the rocSPARSE baseline')
    ap.add_argument('--no-cpp-timed', action='store_true',
                    help='skip the natively timed single-call BOO figure (keeps a kernel trace to the timed steps)')
    ap.add_argument('--pbr-slab-mb', type=float, default=0.0,
                    help='PBR launch knob: X above this many MiB runs its feature tiles one launch each (0: never)')
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print(f'bench.py: this build measures one GPU only (the SpMM path has no multi-GPU '
              f'component); got --gpus {args.gpus}', file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, str(ROOT))
    import spmm_amd as S
    from spmm_amd import matrices as M
    S.set_pbr_slab_bytes(int(args.pbr_slab_mb * (1 << 20)))

    if args.calibrate_copy:
        calibrate_copy(torch)
        return

    A, spec = M.make_config(args.config)
    K = spec['K']
    nnz, m = A.nnz, A.shape[0]
    balg = bytes_alg(A, K)
    flops = 2.0 * nnz * K
    _log(f'config {args.config}: {spec["name"]} {A.shape} nnz={nnz} K={K} bytes_alg={balg}')

    # Copies of matrix, X and Y rotate so that the 256 MB MALL cannot hold one
    # step's data for the next; a config above 512 MB of compulsory traffic
    # cannot stay in it anyway.
    nrot = NROT if balg < 512e6 else 1
    Xs = [torch.from_numpy(M.dense_x(A.shape[1], K, seed=s)).cuda() for s in range(nrot)]
    dev = torch.device('cuda', torch.cuda.current_device())
    Ys = [torch.empty((1, m, K), device=dev) for _ in range(nrot)]
    stream = torch.cuda.current_stream().cuda_stream
    from oracle import oracle as O
    has_boo = 'boo' in spec['formats'] and not args.no_boo
    run_pbr = 'pbr' in spec['formats'] and (not args.no_pbr or not has_boo)
    fmt = 'boo' if has_boo else 'pbr'
    ms_wall = ms_ev_mean = ms_api = ratio = None

    # ---- BOO (headline when the config has it)
    y_gpu = {}
    if has_boo:
        ms_wall, ms_ev_mean, ms_api, ratio = bench_boo(S, A, K, Xs, Ys, dev, stream, args, O, torch)
        y_gpu['boo'] = Ys[0][0].cpu().numpy()

    # ---- PBR on the same matrix
    pbr = {}
    if run_pbr:
        thr = spec.get('pbr_threshold', 4)
        pbrs = [S.csr_to_pbr(A, 8, 8, thr).to(dev) for _ in range(nrot)]

        # a scattered PBR matrix runs its CSR through the BOO gather pass, as
        # pbr_matmul does (spmm_amd.pbr.GATHER_MAX_BLOCK_SHARE)
        gather = pbrs[0]._gpu_meta.gather is not None
        pws_bytes = int(S._core.boo_workspace_bytes(pbrs[0]._gpu_meta.gather.desc, 0, 1, K)) if gather else 0
        pws = torch.empty(max(pws_bytes, 1), dtype=torch.uint8, device=dev)

        def pbr_step(i):
            if gather:
                S._core.boo_matmul_gpu(pbrs[i]._gpu_meta.gather.desc, 0, int(Xs[i].data_ptr()),
                                       int(Ys[i].data_ptr()), 1, K, int(pws.data_ptr()), pws_bytes, int(stream))
            else:
                S._core.pbr_matmul_gpu(pbrs[i]._gpu_meta.desc, 0, int(Xs[i].data_ptr()),
                                       int(Ys[i].data_ptr()), 1, K, int(stream))
        pbr_step(0)
        torch.cuda.synchronize()
        y_gpu['pbr'] = Ys[0][0].cpu().numpy()
        pratio, pok = O.within_bound(y_gpu['pbr'], A, Xs[0].cpu().numpy(), 1e-5)
        if not pok:
            _log(f'PBR PARITY FAILURE: {pratio:.3e}')
            sys.exit(1)
        p_wall, p_ev = time_steps([lambda i=i: pbr_step(i) for i in range(nrot)], args.steps,
                                     args.warmup, torch)
        pbr_workload = f'cfg{args.config}_{spec["name"]}_pbr8x8_thr{thr}_K{K}'
        pbr = {'kernels': 'BOO gather pass (scattered matrix)' if gather else 'stripe',
               'ms_per_step': round(p_wall, 5), 'kernel_ms_mean': round(p_ev, 5),
               'gflops': round(flops / (p_wall * 1e-3) / 1e9, 2),
               'hbm_gbs': round(balg / (p_ev * 1e-3) / 1e9, 1),
               'hbm_frac': round(balg / (p_ev * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
               'traffic': (traffic_from_profiles(pbr_workload) or {}).get('bytes_per_launch')}
        _log(f'PBR: wall {p_wall * 1e3:.1f} us/step, kernel {p_ev * 1e3:.1f} us')
        if not has_boo:                    # PBR is the measured path of this config
            ms_wall, ms_ev_mean, ratio = p_wall, p_ev, pratio

    gbs = balg / (ms_ev_mean * 1e-3) / 1e9
    if has_boo:
        workload = f'cfg{args.config}_{spec["name"]}_boo_{args.cluster}32_K{K}'
        fmt_desc = f'BOO {args.cluster} 32x32, remainder policy (threshold 4)'
    else:
        workload = f'cfg{args.config}_{spec["name"]}_pbr8x8_thr{spec.get("pbr_threshold", 4)}_K{K}'
        fmt_desc = f'PBR 8x8, min_nnz_per_block {spec.get("pbr_threshold", 4)}'
    cpu = None if args.no_cpu_baseline else cpu_baseline(A, spec, args.config, fmt, y_gpu)
    vendor = None if args.no_vendor else vendor_baseline(S, A, K, Xs, min(args.steps, 20), 3, O, torch)
    cpp_timed = (cpp_timed_boo(S, A, K, Xs[0], min(args.steps, 20), torch)
                 if has_boo and not args.no_cpp_timed else None)
    if vendor and 'kernel_ms' in vendor:
        _log(f'vendor: {vendor["library"]}: {vendor["kernel_ms"] * 1e3:.1f} us/call, '
             f'parity ok {vendor["parity_ok"]}')
    elif vendor:
        _log(f'vendor baseline failed: {vendor}')
    out = {
        'metric': f'SpMM GFLOP/s (2*nnz*K/t), {fmt}_matmul; HBM GB/s of algorithmic bytes vs 8 TB/s',
        'value': round(flops / (ms_wall * 1e-3) / 1e9, 2),
        'unit': 'GFLOP/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms_wall, 5),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic',
        'config': {'workload': workload, 'matrix': spec['name'], 'rows': m, 'nnz': nnz, 'K': K,
                   'format': fmt_desc, 'bytes_alg': balg, 'rotation_copies': nrot},
        'hbm_gbs': round(balg / (ms_wall * 1e-3) / 1e9, 1),
        'roofline': {'bound': 'hbm', 'achieved': round(gbs, 1), 'peak': PEAK_HBM_GBS, 'unit': 'GB/s',
                     'frac': round(gbs / PEAK_HBM_GBS, 4),
                     'traffic': (traffic_from_profiles(workload) or {}).get('bytes_per_launch')},
        'kernel_us_mean': round(ms_ev_mean * 1e3, 2),
        'python_api_us_per_call': round(ms_api * 1e3, 2) if ms_api is not None else None,
        'pbr': pbr,
        'cpu_baseline': cpu,
        'vendor_baseline': vendor,
        'cpp_timed': cpp_timed,
    }
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
