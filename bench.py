"""Benchmark of the WarpGBM hot path on one MI355X.

Metric: histogram GB/s (% HBM peak) + train/infer seconds,
1M x 1K, 100 trees, depth 5.

* value: whole-op throughput of the histogram build on config C2
  (1,000,000 rows x 1,000 int8 codes in [0, 32), float32 gradients, 1 era).
  One step = the root histogram (all rows) + the 16-node histogram (rows
  assigned uniformly at random to 16 depth-4 nodes), inputs resident in HBM.
  Algorithmic bytes per launch: R*F + 4R (gradients) + 4R (row indices, node
  case only) + nodes*F*B*8 (G and H written).
* Before the warm-up steps the step runs for --settle-ms of wall time: the
  GPU's clocks take tens of milliseconds of sustained load to settle, and a
  short run would otherwise time the ramp.
* roofline: the dominant kernel (hist_tiles), its average launch duration
  from HIP events recorded on its launch stream right before and right
  after every one of its dispatches in the timed region (wgbm_timer_enable(1):
  the interval is the kernel plus the dispatch of its packet, a few
  microseconds).  The same steps without events are timed too
  (ms_per_step_no_events): each event pair adds that dispatch time again.
* cpu_baseline: the CPU oracle (C loops on all OpenMP threads) running the
  same C2 step, 1 warm-up then the median of 5; plus C1 end to end (quantile
  edges, binning, 20 trees) on the CPU, median of 3; and estimates of the
  C3, C4 and C5 fits (edges + binning timed, one tree or round timed, times
  the trees or rounds of the config).
* dropin: the reference-shaped ops of node_kernel in the reference's call
  patterns: compute_histogram3 on C2 (root with sample_indices = all rows,
  then one call per node with that node's rows, raw [N, F] int8 codes);
  compute_split at a C4 node's shape; predict_forest of C3's 100 trees as
  flatten_tree tables; custom_cuda_binner once per C3 column.
* train_s / infer_s: end-to-end fit / predict wall seconds on config C3
  (1M x 1000 float32 features, 100 trees, depth 5, 32 bins, lr 0.01; predict
  on 1M held-out rows), including host->device copies and binning; C4 (era
  DES) and C5 (softmax) likewise, C1 fit seconds on the GPU.
* kernels: achieved HBM bandwidth of quantile edges, binning and inference on
  C3's held-out matrix resident on the device (algorithmic bytes / median
  call time); quantile_select_staged is the part of the edges that a fit runs
  after its upload (the column staging rides on the transfer).

* c4_des: the era path (DES) on C4 per depth: per-era gain kernel ("rows")
  and era sums + pick ("sums"), HIP-event times against algorithmic bytes
  counted from the fitted forest.
* roofline.hbm_read_probe: a pure 16-byte streaming read of the C2 codes
  buffer, the practical HBM ceiling of a read-bound kernel on this GPU.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-ms MS]
                       [--no-e2e] [--no-cpu] [--no-extra] [--no-dropin]
                       [--only-extra --extra c4 --c4-trees T]   (profiling driver)
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def c2_inputs(rows, feats, seed=0):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 32, (rows, feats), dtype=np.int8)
    grad = rng.standard_normal(rows, dtype=np.float32)
    node = rng.integers(0, 16, rows)
    return codes, grad, node


def c3_inputs(rows, feats, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((rows, feats), dtype=np.float32)
    w20 = np.random.default_rng(1000).standard_normal(20).astype(np.float32)
    y = X[:, :20] @ w20 + 0.5 * np.sin(X[:, 0] * X[:, 1]) + rng.normal(0, 0.5, rows).astype(np.float32)
    return X, y.astype(np.float32)


def c4_inputs(rows=500_000, feats=2000, eras=500, seed=0):
    """Config C4: int8 codes in {0..4}, 500 contiguous equal eras; target = per-era
    5-quantile bucket of a score built from 50 features, 25 of which flip sign in
    half of the eras."""
    rng = np.random.default_rng(seed)
    X = rng.integers(0, 5, (rows, feats), dtype=np.int8)
    era = np.repeat(np.arange(eras), rows // eras)
    c = rng.standard_normal(50)
    s = np.ones((eras, 50))
    flip = rng.random((eras, 25)) < 0.5
    s[:, 25:] = np.where(flip, -1.0, 1.0)
    score = ((X[:, :50].astype(np.float32) - 2) * (c * s[era])).sum(axis=1) + rng.standard_normal(rows)
    y = np.empty(rows, np.float32)
    for e in range(eras):
        sl = slice(e * (rows // eras), (e + 1) * (rows // eras))
        q = np.quantile(score[sl], [0.2, 0.4, 0.6, 0.8])
        y[sl] = np.digitize(score[sl], q) / 4.0
    return X, y, era


def c5_inputs(rows_per_class=20_000, feats=100, K=10, seed=0):
    """Config C5: 10 Gaussian clusters in 30 informative dims (means ~N(0, 1.5^2),
    unit variance) plus 70 noise dims."""
    means = np.random.default_rng(100).normal(0, 1.5, (K, 30))  # one distribution
    rng = np.random.default_rng(seed)
    lab = np.repeat(np.arange(K), rows_per_class)
    X = np.empty((len(lab), feats), np.float32)
    X[:, :30] = means[lab] + rng.standard_normal((len(lab), 30))
    X[:, 30:] = rng.standard_normal((len(lab), feats - 30))
    return X, lab


def c1_inputs(n=10000, f=50, seed=0):
    """Config C1: X ~ N(0,1) float32, y = X.w (10 nonzero) + 0.1 N(0,1)."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, f), dtype=np.float32)
    w = np.zeros(f, np.float32)
    idx = rng.choice(f, 10, replace=False)
    w[idx] = rng.standard_normal(10)
    y = (X @ w + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return X, y


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="wall time the step runs before the warm-up steps (clock ramp)")
    ap.add_argument("--rows", type=int, default=1_000_000)
    ap.add_argument("--feats", type=int, default=1000)
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--e2e-rows", type=int, default=1_000_000)
    ap.add_argument("--e2e-trees", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip C4 / C5 / C1 end to end")
    ap.add_argument("--runs", type=int, default=2, choices=(1, 2),
                    help="fit + predict runs per end-to-end config (the last is reported; "
                         "with 2 the first is reported as *_cold_s)")
    ap.add_argument("--extra", default="c1,c4,c5",
                    help="the end-to-end configs run after C3 (comma list of c1, c4, c5)")
    ap.add_argument("--no-dropin", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (calibrates HBM byte counters)")
    ap.add_argument("--only-extra", action="store_true",
                    help="run only the --extra configs (no C2 step, probes, drop-in, CPU or C3): "
                         "a short driver for profiling those fits")
    ap.add_argument("--c4-trees", type=int, default=100,
                    help="trees of the C4 fits (100 is the config; fewer for counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU path is design-only", file=sys.stderr)
        sys.exit(2)

    import torch

    from warpgbm_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        # a plain copy of known size: 2^30 bytes read, 2^30 bytes written
        src = torch.ones(1 << 30, dtype=torch.int8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    if args.only_extra:
        out = {"metric": "end-to-end fits of the --extra configs only (a profiling driver)",
               "config": {"workload": args.extra, "c4_trees": args.c4_trees}}
        for cfg in ("c1", "c4", "c5"):
            if cfg in args.extra.split(","):
                out.update(run_extra(cfg, args.runs, None, args.c4_trees))
        print(json.dumps(out))
        return
    N, F, B = args.rows, args.feats, 32
    log(f"generating C2 inputs {N}x{F}")
    codes_h, grad_h, node_h = c2_inputs(N, F)
    # the codes in the library's native layout, made by the pre-binned ingest
    # (what fit() does with int8 input): rows padded to a 128-byte multiple,
    # every byte in [0, B + 1]; algorithmic bytes still count F bytes per row
    from warpgbm_amd import device as D

    raw = torch.from_numpy(codes_h).to(dev)
    nat = D.codes_from_int8(raw, False, B)[0]
    codes, S = nat.rm, nat.stride
    grad = torch.from_numpy(grad_h).to(dev)
    order16_h = np.argsort(node_h, kind="stable").astype(np.int32)
    seg16_h = np.zeros(17, np.int64)
    seg16_h[1:] = np.cumsum(np.bincount(node_h, minlength=16))
    order16 = torch.from_numpy(order16_h).to(dev)
    seg16 = torch.from_numpy(seg16_h).to(dev)
    seg1 = torch.tensor([0, N], dtype=torch.int64, device=dev)
    G1 = torch.zeros((1, F, B), device=dev)
    H1 = torch.zeros_like(G1)
    G16 = torch.zeros((16, F, B), device=dev)
    H16 = torch.zeros_like(G16)
    stream = _lib.current_stream_ptr(dev)
    flags = _lib.CODES_NATIVE

    def step():
        _lib.check(lib.wgbm_histogram_segments(codes.data_ptr(), N, S, F, grad.data_ptr(), None,
                                               seg1.data_ptr(), 1, N, B, flags, G1.data_ptr(),
                                               H1.data_ptr(), stream), "hist root")
        _lib.check(lib.wgbm_histogram_segments(codes.data_ptr(), N, S, F, grad.data_ptr(),
                                               order16.data_ptr(), seg16.data_ptr(), 16, N, B,
                                               flags, G16.data_ptr(), H16.data_ptr(), stream),
                   "hist 16 nodes")

    # sanity first: exact counts.  Its first-use torch reductions load code
    # objects for ~0.1 s; done here, that idle time does not fall between the
    # settle and the timed region (the clocks ramp again after ~0.1 s idle).
    step()
    torch.cuda.synchronize()
    assert torch.all(H1.sum(dim=2) == N), "root histogram counts are wrong"
    assert torch.equal(H16.sum(dim=0), H1[0]), "16-node counts do not add up to the root"
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    torch.cuda.synchronize()
    # the clock ramp: the step runs for settle_ms of wall time (the clocks
    # reach their steady state after ~20 ms of sustained load), then the
    # warm-up steps lead straight into the timed region
    n_settle, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.settle_ms:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
        n_settle += 20
    settle_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    def run_steps(with_events):
        lib.wgbm_timer_reset()
        lib.wgbm_timer_enable(1 if with_events else 0)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        lib.wgbm_timer_enable(0)
        return e0.elapsed_time(e1) / args.steps

    # the timed region: every hist_tiles dispatch carries a HIP event pair
    mark("c2 timed")
    ms_step = run_steps(True)
    mark("c2 plain")
    tot = C.c_double()
    cnt = C.c_int64()
    lib.wgbm_timer_read(b"hist_tiles", C.byref(tot), C.byref(cnt))
    k_ms = tot.value / max(cnt.value, 1)
    assert cnt.value == 2 * args.steps, (cnt.value, args.steps)
    # the same steps with no events attached (their dispatch overhead)
    ms_step_plain = run_steps(False)
    mark("c2 end")
    bytes_root = N * F + 4 * N + 1 * F * B * 8
    bytes_16 = N * F + 4 * N + 4 * N + 16 * F * B * 8
    gbs = (bytes_root + bytes_16) / (ms_step * 1e-3) / 1e9
    k_achieved = ((bytes_root + bytes_16) / 2) / (k_ms * 1e-3) / 1e9
    log(f"histogram step {ms_step:.4f} ms ({gbs:.1f} GB/s), {ms_step_plain:.4f} ms without "
        f"events; hist_tiles {k_ms:.4f} ms/launch over {cnt.value} launches "
        f"({k_achieved:.1f} GB/s); settle {n_settle} steps in {settle_ms:.0f} ms")
    # ceiling of the kernel's LDS stage: 64-bit LDS atomic adds per second in
    # the same LDS layout with no global traffic (measured live, after the
    # timed region so that its heavy LDS load does not precede the timing)
    lds_peak = C.c_double(0.0)
    _lib.check(lib.wgbm_probe_lds_atomics(512, 500, C.byref(lds_peak), stream), "lds probe")
    lds_peak = lds_peak.value
    log(f"LDS atomic probe: {lds_peak:.3e} 64-bit adds/s")
    # achievable HBM read rate: 16-byte streaming loads over the same codes
    # buffer (N x S bytes), ten launches back to back
    hbm_probe = C.c_double(0.0)
    _lib.check(lib.wgbm_probe_hbm_read(codes.data_ptr(), N * S, 10, C.byref(hbm_probe), stream),
               "hbm probe")
    hbm_probe = hbm_probe.value / 1e9
    log(f"HBM read probe: {hbm_probe:.1f} GB/s ({N * S} bytes, 16-byte loads)")

    dropin = None
    if not args.no_dropin:
        dropin = {"compute_histogram3": dropin_leg(raw, grad, order16, seg16_h, N, F, B, dev)}
    del nat, codes, G16, H16, raw
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_leg(codes_h, grad_h, order16_h, seg16_h, N, F, B,
                               bytes_root + bytes_16, run_c1=not args.no_extra)
    del grad, order16

    e2e = {}
    if not args.no_e2e:
        from warpgbm_amd import WarpGBM

        n = args.e2e_rows
        log(f"generating C3 inputs {n}x{F}")
        X, y = c3_inputs(n, F, 0)
        Xt, yt = c3_inputs(n, F, 1)
        # two identical fits / predicts: the first in this process pays the
        # one-time costs (first large staged upload, first launch of each
        # kernel), the second is the steady state reported as train_s / infer_s
        runs = []
        for run in range(args.runs):
            m = WarpGBM(num_bins=32, max_depth=5, n_estimators=args.e2e_trees,
                        learning_rate=0.01)
            torch.cuda.synchronize()
            mark(f"c3 fit {run}")
            t0 = time.perf_counter()
            m.fit(X, y)
            torch.cuda.synchronize()
            tr = time.perf_counter() - t0
            mark(f"c3 predict {run}")
            t0 = time.perf_counter()
            p = m.predict(Xt)
            torch.cuda.synchronize()
            runs.append((tr, time.perf_counter() - t0, p))
            mark(f"c3 end {run}")
        if cpu is not None:
            cpu.update(cpu_train_estimate("c3", X, y))
        del X, y
        (train_cold, infer_cold, _), (train_s, infer_s, p) = runs[0], runs[-1]
        corr = float(np.corrcoef(p, yt)[0, 1])
        e2e = {"train_s": round(train_s, 3), "infer_s": round(infer_s, 3),
               "train_cold_s": round(train_cold, 3), "infer_cold_s": round(infer_cold, 3),
               "heldout_corr": round(corr, 4), "e2e_workload": f"C3 {n}x{F}, {args.e2e_trees} trees",
               "e2e_timing": "second of two identical fit + predict runs in this process "
                             "(the first, *_cold_s, includes one-time setup)"}
        log(f"C3 train {train_s:.3f} s (first run {train_cold:.3f}), infer {infer_s:.3f} s "
            f"(first run {infer_cold:.3f}), corr {corr:.4f}")
        e2e["kernels"] = c3_kernel_rooflines(m, Xt, dropin)
        del Xt

    # HBM bytes per hist_tiles launch from the committed rocprofv3 PMC summary
    # (FETCH_SIZE / WRITE_SIZE runs of this same workload, scaled by a copy of
    # known size); null when that summary is absent
    traffic = None
    tpath = ROOT / "profiles" / "hist_c2_traffic.json"
    if tpath.exists() and N == 1_000_000 and F == 1000:
        traffic = round(json.loads(tpath.read_text())["traffic_bytes_per_dispatch"])
    out = {
        "metric": "histogram GB/s (% HBM peak) + train/infer sec, 1M×1K 100 trees depth 5",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 codes / int64 exact sums",
        "data": "synthetic (numpy default_rng(0); C2 histogram and C3 end-to-end workloads)",
        "config": {"workload": f"C2 histogram: root + 16 nodes, {N}x{F} int8, 32 bins, 1 era",
                   "rows": N, "features": F, "bins": B, "nodes": [1, 16], "row_stride": S},
        "warmup_state": {"settle_ms": round(settle_ms, 1), "settle_steps": n_settle,
                         "warmup_steps": args.warmup},
        "ms_per_step_no_events": round(ms_step_plain, 4),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(k_achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(k_achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": "hist_tiles_kernel<4,0,32,*,true> (native codes)",
                     "kernel_ms": round(k_ms, 4),
                     "kernel_timing": f"HIP events recorded around all {cnt.value} launches "
                                      f"of the timed region ({args.steps} steps x 2) on the "
                                      f"kernel's stream",
                     # the binding unit in practice: one 64-bit LDS atomic per
                     # (row, feature); peak = wgbm_probe_lds_atomics, measured
                     # above on this GPU
                     # the practical HBM ceiling: a pure 16-byte streaming read
                     "hbm_read_probe": {"GB/s": round(hbm_probe, 1),
                                        "frac_of_peak": round(hbm_probe / HBM_PEAK_GBS, 4),
                                        "kernel_frac_of_probe": round(k_achieved / hbm_probe, 4)},
                     "lds_atomics": {"updates": N * F, "achieved_per_s": round(N * F / (k_ms * 1e-3)),
                                     "peak_per_s": round(lds_peak),
                                     "frac": round(N * F / (k_ms * 1e-3) / lds_peak, 4)}},
        "cpu_baseline": cpu,
        "dropin": dropin,
    }
    out.update(e2e)
    if not args.no_extra:
        for cfg in ("c1", "c4", "c5"):
            if cfg in args.extra.split(","):
                out.update(run_extra(cfg, args.runs, cpu, args.c4_trees))
    write_marks()
    print(json.dumps(out))


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Phase marks on CLOCK_MONOTONIC (the clock of rocprofv3's kernel
# timestamps), written to $WGBM_BENCH_MARKS as JSON when that is set, so a
# kernel trace of this run can be split into its legs.
_MARKS: list = []


def mark(label):
    _MARKS.append((label, time.clock_gettime_ns(time.CLOCK_MONOTONIC)))


def write_marks():
    path = os.environ.get("WGBM_BENCH_MARKS")
    if path:
        Path(path).write_text(json.dumps(_MARKS))


def dropin_leg(raw, grad, order16, seg16_h, N, F, B, dev):
    """The reference-shaped op in the reference's call pattern on C2:
    node_kernel.compute_histogram3 on the raw [N, F] int8 codes, once for the
    root (sample_indices = every row) and once per node (that node's rows),
    as warpgbm/core.py:543-563 calls it; the outputs accumulate (the
    reference's per-call torch.zeros is the caller's and is not timed).
    Two feature choices: every feature (colsample_bytree = 1, the reference's
    arange) and a random half (colsample_bytree = 0.5, the reference's
    randperm(F)[:k], core.py:722).  Median of 5 steps after one warm-up,
    torch events on the current stream."""
    import torch

    from warpgbm_amd import node_kernel as nk

    era = torch.zeros(N, dtype=torch.int32, device=dev)
    rows_all = torch.arange(N, dtype=torch.int32, device=dev)
    node_rows = [order16[int(seg16_h[k]):int(seg16_h[k + 1])] for k in range(16)]
    gen = torch.Generator(device="cpu").manual_seed(7)
    choices = {"all": torch.arange(F, dtype=torch.int32),
               "half": torch.randperm(F, generator=gen, dtype=torch.int32)[:F // 2]}
    out = {"calls_per_step": 17,
           "pattern": "root (sample_indices = all rows) + one call per node, raw [N, F] int8 "
                      "codes, 1 era"}
    for name, fsel in choices.items():
        feats = fsel.to(dev)
        k = feats.numel()
        G = torch.zeros((17, 1, k, B), device=dev)
        H = torch.zeros_like(G)

        def dstep():
            nk.compute_histogram3(raw, grad, rows_all, feats, era, G[0], H[0], B)
            for j in range(16):
                nk.compute_histogram3(raw, grad, node_rows[j], feats, era, G[j + 1], H[j + 1], B)

        dstep()
        ts = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            dstep()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        ms = sorted(ts)[2]
        # root and nodes: the selected codes, gradient and row id of every row; outputs
        nbytes = 2 * (N * k + 8 * N) + 17 * k * B * 8
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"drop-in compute_histogram3 ({name} features, {k}), C2 root + 16 per-node calls: "
            f"{ms:.3f} ms ({gbs:.0f} GB/s)")
        key = "" if name == "all" else "half_"
        out[key + "features"] = k
        out[key + "ms_per_step"] = round(ms, 4)
        out[key + "bytes"] = int(nbytes)
        out[key + "GB/s"] = round(gbs, 1)
        out[key + "frac"] = round(gbs / HBM_PEAK_GBS, 4)
    return out


def cpu_baseline_leg(codes_h, grad_h, order16_h, seg16_h, N, F, B, step_bytes, run_c1):
    """The CPU oracle (test infrastructure, the checker of the GPU path) on
    the host: the same C2 step (root + 16 nodes, exact sums) with its C loops
    on every OpenMP thread, 1 warm-up then the median of 5; C1 end to end
    (quantile edges, binning, 20 trees of depth 5) median of 3."""
    from oracle import clib, gbm, ops

    threads = clib.num_threads()
    feats = np.arange(F)
    qbits = ops.qbits_for_rows(N)

    def cstep():
        s = ops.shift_from_absmax(np.max(np.abs(grad_h)), qbits)
        q = ops.quantise(grad_h, s)
        clib.hist_exact_q(codes_h, q, None, feats, None, 1, B)
        for k in range(16):
            clib.hist_exact_q(codes_h, q, order16_h[seg16_h[k]:seg16_h[k + 1]], feats, None, 1, B)

    cstep()
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        cstep()
        ts.append(time.perf_counter() - t0)
    dt = sorted(ts)[2]
    cpu = {"value": round(step_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
           "kind": "port", "host_cpus": os.cpu_count(), "cpu_model": cpu_model(),
           "sample": f"the full C2 step (root + 16 nodes, {N}x{F} int8 codes, exact sums) by the "
                     f"oracle's C loops on {threads} OpenMP threads; 1 warm-up, median of 5: "
                     f"{dt:.3f} s per step"}
    log(f"cpu baseline {cpu['value']} GB/s ({dt:.3f} s per step, {threads} threads)")
    if run_c1:
        X, y = c1_inputs()

        def c1_fit():
            edges = clib.quantile_edges_matrix(X, 32)
            codes = clib.bin_matrix(X, edges)
            gbm.Forest(num_bins=32, max_depth=5, n_estimators=20, learning_rate=0.1).fit_codes(
                codes, y, hist=clib.hist_exact_q, scan=clib.split_scan_q)

        c1_fit()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            c1_fit()
            ts.append(time.perf_counter() - t0)
        cpu["c1_train_s"] = round(sorted(ts)[1], 3)
        cpu["c1_sample"] = ("C1 end to end: 10000x50 float32, edges + binning + 20 trees of depth 5 "
                            "(32 bins), oracle growth with the C loops; median of 3")
        log(f"cpu C1 train {cpu['c1_train_s']} s")
    return cpu


def cpu_train_estimate(cfg, X, y, era=None):
    """The CPU oracle on an end-to-end config: the
    one-time work (quantile edges and binning of the float32 matrix, none for
    C4's pre-binned codes) timed once, plus ONE tree (C3, C4) or one round
    of K class trees (C5) grown with the oracle's C loops on every OpenMP
    thread; the whole fit is estimated as one-time + trees x that (labelled
    as an estimate: the trees of a fit differ in size, the first is timed)."""
    from oracle import clib, gbm

    threads = clib.num_threads()
    t0 = time.perf_counter()
    if cfg == "c4":
        codes, prep = X, 0.0
        kw, n = dict(num_bins=5, max_depth=8, learning_rate=0.1), 100
    else:
        B = 32
        edges = clib.quantile_edges_matrix(X, B)
        codes = clib.bin_matrix(X, edges)
        prep = time.perf_counter() - t0
        kw, n = ((dict(num_bins=32, max_depth=5, learning_rate=0.01), 100) if cfg == "c3" else
                 (dict(objective="multiclass", num_bins=32, max_depth=6, learning_rate=0.1), 200))
    t1 = time.perf_counter()
    gbm.Forest(n_estimators=1, **kw).fit_codes(codes, y, era_id=era, hist=clib.hist_exact_q,
                                               scan=clib.split_scan_q)
    one = time.perf_counter() - t1
    unit = "round of 10 class trees" if cfg == "c5" else "tree"
    log(f"cpu {cfg.upper()}: one-time {prep:.2f} s, one {unit} {one:.2f} s "
        f"({threads} threads) -> estimated fit {prep + n * one:.1f} s")
    return {f"{cfg}_train_est_s": round(prep + n * one, 2),
            f"{cfg}_sample": f"{cfg.upper()} on the CPU oracle ({threads} threads): quantile edges + "
                             f"binning {prep:.2f} s (timed once) + {n} x one {unit} "
                             f"{one:.2f} s (the first {unit} of the fit, timed; the x{n} is an "
                             f"estimate)"}


def c3_kernel_rooflines(m, Xt, dropin=None):
    """Achieved HBM bandwidth of the other three operators on C3's held-out
    matrix (1M x 1000 float32, resident on the device): quantile edges,
    binning, and inference of the fitted 100 trees.  Each is timed with torch
    events on the current stream (the stream the library launches on), median
    of 5 calls after one warm-up; bytes are the algorithmic ones (every input
    byte read once, every output byte written once)."""
    import torch

    from warpgbm_amd import device as D

    dev = torch.device("cuda:0")
    Xd = D.upload_float(Xt, dev)
    n, F = Xd.shape
    B = m.num_bins

    def timed(fn):
        fn()
        ts = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return sorted(ts)[2]

    out = {}

    def put(name, ms, nbytes, what):
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "bytes": int(nbytes), "GB/s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_are": what}

    edges = D.quantile_edges(Xd, B)
    put("quantile_edges", timed(lambda: D.quantile_edges(Xd, B)), n * F * 4 + F * (B - 1) * 4,
        "X read once + edges (moved: X read and its values written transposed, then two scans of each transposed column)")
    # the fit's split of the same work: the staging (X's values transposed
    # into columns) runs block by block on the copy stream while the upload
    # is in flight, and only the selection over the staged columns follows
    # the transfer
    stq = D.QuantileStage(n, F, dev)
    stq.stage(Xd, 0, n)
    e2 = stq.edges(B)
    assert torch.equal(e2.view(torch.int32), edges.view(torch.int32)), "staged edges differ"
    put("quantile_select_staged", timed(lambda: stq.edges(B)), n * F * 4 + F * (B - 1) * 4,
        "X's values read once + edges (moved: two scans of each staged column; the fit stages "
        "the columns behind the PCIe upload, wgbm_quantile_stage_rows per row block)")
    del stq, e2
    put("bin_matrix", timed(lambda: D.bin_matrix(Xd, edges, with_cm=False)),
        n * F * 4 + n * F + F * (B - 1) * 4, "X + codes (row-major) + edges")
    codes = D.bin_matrix(Xd, edges, with_cm=False)
    if dropin is not None:
        dropin.update(dropin_ops_leg(m, Xd, codes))
    del Xd
    feat, bin_, leaf, nt = m._cached_heap()
    pred = torch.zeros((n, 1), dtype=torch.float32, device=dev)
    put("predict_heap", timed(lambda: D.predict_heap(codes, feat, bin_, leaf, nt, 1, m.max_depth,
                                                       m.learning_rate, pred)),
        n * F + 8 * n, "codes + predictions read and written (tables are in LDS)")
    for k, v in out.items():
        print(f"[bench] {k}: {v['ms']:.3f} ms, {v['GB/s']:.0f} GB/s ({100 * v['frac']:.1f}% of HBM)",
              file=sys.stderr, flush=True)
    return out


def dropin_ops_leg(m, Xd, codes):
    """The other three reference-shaped ops of warpgbm.cuda.node_kernel, each
    in the reference's own call pattern, timed like c3_kernel_rooflines
    (median of 5 after a warm-up, torch events on the current stream), with
    algorithmic bytes:
    * compute_split (best_split_kernel.cu:61-88) at a C4 node's shape, E=500
      eras x F=2000 features x B=5 bins: G and H read, per-era gain and
      direction written (E*F*B*8 + E*F*(B-1)*8 bytes);
    * predict_forest (predict.cu:48-76) of C3's 100 fitted trees as the
      reference's flatten_tree tables ([100, 2^(depth+1), 6], core.py:917-932)
      on C3's 1M held-out rows as raw [N, F] int8 codes (N*F + 8N bytes);
    * custom_cuda_binner (binner.cu:27-52) once per feature column, as the
      reference's quantile-binning loop calls it (core.py:527-537): F calls,
      each on one resident contiguous float32 column of C3's held-out matrix
      (N*F*4 + N*F bytes + edges)."""
    import torch

    from warpgbm_amd import node_kernel as nk

    dev = torch.device("cuda:0")

    def timed(fn):
        fn()
        ts = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return sorted(ts)[2]

    out = {}

    def put(name, ms, nbytes, shape):
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "bytes": int(nbytes), "GB/s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "shape": shape}
        log(f"drop-in {name} ({shape}): {ms:.3f} ms, {gbs:.0f} GB/s")

    # compute_split at a C4 node: a real-looking histogram (counts of 500,000
    # rows over 500 eras and 5 bins, residual sums)
    E, F4, B4 = 500, 2000, 5
    gen = torch.Generator(device="cpu").manual_seed(11)
    Hh = torch.randint(0, 400, (E, F4, B4), generator=gen).float().to(dev)
    Gh = (torch.randn((E, F4, B4), generator=gen) * Hh.cpu().sqrt()).to(dev)
    gain = torch.empty((E, F4, B4 - 1), device=dev)
    dirn = torch.empty_like(gain)
    put("compute_split", timed(lambda: nk.compute_split(Gh, Hh, 0.0, 20.0, 1e-6, gain, dirn)),
        E * F4 * B4 * 8 + E * F4 * (B4 - 1) * 8, "E=500 x F=2000 x B=5 (a C4 node)")
    del Gh, Hh, gain, dirn

    # predict_forest: the reference's flat tables of C3's forest
    n, F = Xd.shape
    M = 2 ** (m.max_depth + 1)
    tt = torch.stack([m.flatten_tree(t, M) for t in m.forest]).to(dev)
    raw = codes.rm[:, :F].contiguous()
    pred = torch.zeros(n, device=dev)
    put("predict_forest", timed(lambda: nk.predict_forest(raw, tt, m.learning_rate, pred)),
        n * F + 8 * n, f"{len(m.forest)} trees x {M} nodes on {n}x{F} int8 codes")
    del raw, pred

    # custom_cuda_binner per column
    XT = Xd.t().contiguous()
    edges = torch.as_tensor(m.bin_edges).to(dev)
    cols = torch.empty((F, n), dtype=torch.int8, device=dev)

    def bin_loop():
        for f in range(F):
            nk.custom_cuda_binner(XT[f], edges[f], cols[f])

    put("custom_cuda_binner", timed(bin_loop), n * F * 5 + F * (m.num_bins - 1) * 4,
        f"{F} per-column calls of {n} values, {m.num_bins} bins")
    del XT, cols
    torch.cuda.empty_cache()
    return out


def des_level_rooflines(lib, X, y, era, trees=100):
    """Achieved HBM bandwidth of the era path (DES) on C4, per depth: one
    more 100-tree fit with the library's event timers on ("des_rows_L<d>":
    the per-era gain kernel, pair codes or int8 codes; "des_sums_L<d>": era
    sums, pick and finish), against algorithmic bytes counted from the
    fitted forest by routing every row through each tree on the host:
    * rows kernel: every row of a live (node, era) segment (one that can
      hold a split: at least 2 x min_child_weight rows) read once -- its
      codes (F/2 bytes as pair codes on the levels that use them, F bytes
      as int8 codes) plus its row id and residual (8 bytes) -- and the
      segment's gains and directions staged (5 bytes per candidate);
    * sums: the staged values read once, each live 32-era block's float64
      sum and int8 direction count written and read (9 bytes per candidate
      each way); the criterion, agreement and pick stay on chip."""
    import torch

    from warpgbm_amd import WarpGBM

    kw = dict(num_bins=5, max_depth=8, n_estimators=trees, learning_rate=0.1)
    lib.wgbm_timer_reset()
    lib.wgbm_timer_enable(1)
    m = WarpGBM(**kw).fit(X, y, era_id=era)
    torch.cuda.synchronize()
    lib.wgbm_timer_enable(0)
    N, F = X.shape
    B, D, mcw = m.num_bins, m.max_depth, float(m.min_child_weight)
    eras = np.unique(era, return_inverse=True)[1].astype(np.int64)
    E = int(eras.max()) + 1
    W = (E + 31) // 32
    ncand = F * (B - 1)
    # the routing runs on the device with torch (bookkeeping for the byte
    # counts, outside every timed region)
    dev = torch.device("cuda:0")
    feat, bin_, _, _ = m._cached_heap()
    feat, bin_ = feat[:, 0].long(), bin_[:, 0].long()
    Xd = torch.from_numpy(X).to(dev)
    ed = torch.from_numpy(eras).to(dev)
    rows_alive = np.zeros(D, np.int64)
    segs_alive = np.zeros(D, np.int64)
    blocks_live = np.zeros(D, np.int64)
    present = np.zeros(D, np.int64)
    for t in range(feat.shape[0]):
        idx = torch.arange(N, device=dev)
        h = torch.zeros(N, dtype=torch.long, device=dev)
        for d in range(D):
            base = (1 << d) - 1
            key = (h - base) * E + ed[idx]
            cnt = torch.bincount(key, minlength=(1 << d) * E).reshape(1 << d, E)
            live = cnt >= 2.0 * mcw
            pad = torch.zeros((1 << d, W * 32), dtype=torch.bool, device=dev)
            pad[:, :E] = live
            st = torch.stack([(cnt * live).sum(), live.sum(),
                              pad.reshape(1 << d, W, 32).any(dim=2).sum(),
                              (cnt.sum(dim=1) > 0).sum()]).cpu().numpy()
            rows_alive[d] += int(st[0])
            segs_alive[d] += int(st[1])
            blocks_live[d] += int(st[2])
            present[d] += int(st[3])
            f = feat[t, h]
            keep = f >= 0
            idx, h, f = idx[keep], h[keep], f[keep]
            right = Xd[idx, f].long() > bin_[t, h]
            h = 2 * h + 1 + right.long()
    del Xd, ed
    levels = []
    tot_ms = tot_bytes = 0.0
    for d in range(D):
        pairs = N >= 96 * (1 << d) * E  # the engine's pair-code rule (kDesPairMinRows)
        rb = rows_alive[d] * ((F + 1) // 2 + 8 if pairs else F + 8) + segs_alive[d] * ncand * 5
        sb = segs_alive[d] * ncand * 5 + blocks_live[d] * ncand * 18
        ent = {"depth": d, "codes": "pair" if pairs else "int8"}
        for name, nbytes in (("rows", rb), ("sums", sb)):
            tot = C.c_double()
            cnt = C.c_int64()
            lib.wgbm_timer_read(f"des_{name}_L{d}".encode(), C.byref(tot), C.byref(cnt))
            ms = tot.value
            gbs = nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
            ent[name] = {"ms": round(ms, 3), "bytes": int(nbytes), "GB/s": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "launches": int(cnt.value)}
            tot_ms += ms
            tot_bytes += nbytes
        levels.append(ent)
        log(f"C4 DES depth {d} ({ent['codes']}): rows {ent['rows']['ms']:.2f} ms "
            f"{ent['rows']['GB/s']:.0f} GB/s, sums {ent['sums']['ms']:.2f} ms "
            f"{ent['sums']['GB/s']:.0f} GB/s")
    gbs = tot_bytes / (tot_ms * 1e-3) / 1e9
    log(f"C4 DES total {tot_ms:.1f} ms for {trees} trees, {gbs:.0f} GB/s")
    return {"ms": round(tot_ms, 2), "bytes": int(tot_bytes), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "trees": trees, "levels": levels,
            "bytes_are": "per depth, summed over the trees: live (node, era) segments' rows "
                         "(codes + row id + residual) and staged per-era gains (rows); staged "
                         "gains read, 32-era block sums written and read (sums); timed with "
                         "HIP events around the launches"}


def run_extra(cfg, n_runs=2, cpu=None, c4_trees=100):
    """End-to-end seconds of configs C1 (fit only), C4 (era-aware DES) and C5
    (softmax); with a cpu_baseline dict, the CPU oracle's estimate of the same
    fit is added to it."""
    import torch

    from warpgbm_amd import WarpGBM

    if cfg == "c1":
        X, y = c1_inputs()
        WarpGBM(num_bins=32, max_depth=5, n_estimators=20, learning_rate=0.1).fit(X, y)
        ts = []
        for _ in range(3):
            m = WarpGBM(num_bins=32, max_depth=5, n_estimators=20, learning_rate=0.1)
            t0 = time.perf_counter()
            m.fit(X, y)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        tr = sorted(ts)[1]
        log(f"C1 train {tr:.3f} s (median of 3)")
        return {"c1_train_s": round(tr, 3)}
    if cfg == "c4":
        print("[bench] generating C4 inputs", file=sys.stderr, flush=True)
        X, y, era = c4_inputs()
        runs = []
        for run in range(n_runs):  # the second run is the steady state (see the C3 leg)
            m = WarpGBM(num_bins=5, max_depth=8, n_estimators=c4_trees, learning_rate=0.1)
            torch.cuda.synchronize()
            mark(f"c4 fit {run}")
            t0 = time.perf_counter()
            m.fit(X, y, era_id=era)
            torch.cuda.synchronize()
            tr = time.perf_counter() - t0
            mark(f"c4 predict {run}")
            t0 = time.perf_counter()
            p = m.predict(X)
            runs.append((tr, time.perf_counter() - t0, p))
            mark(f"c4 end {run}")
        (tr0, inf0, _), (tr, inf, p) = runs[0], runs[-1]
        corr = float(np.corrcoef(p, y)[0, 1])
        if cpu is not None:
            cpu.update(cpu_train_estimate("c4", X, y, era))
        from warpgbm_amd import _lib
        des = des_level_rooflines(_lib.load(), X, y, era, c4_trees)
        print(f"[bench] C4 train {tr:.3f} s (first run {tr0:.3f}), infer {inf:.3f} s "
              f"(first run {inf0:.3f}), in-sample corr {corr:.4f}", file=sys.stderr, flush=True)
        return {"c4_train_s": round(tr, 3), "c4_infer_s": round(inf, 3),
                "c4_train_cold_s": round(tr0, 3), "c4_infer_cold_s": round(inf0, 3),
                "c4_corr": round(corr, 4), "c4_des": des}
    if cfg == "c5":
        print("[bench] generating C5 inputs", file=sys.stderr, flush=True)
        X, lab = c5_inputs()
        Xt, labt = c5_inputs(rows_per_class=100_000, seed=1)
        runs = []
        for run in range(n_runs):  # the second run is the steady state (see the C3 leg)
            m = WarpGBM(objective="multiclass", num_bins=32, max_depth=6, n_estimators=200,
                        learning_rate=0.1)
            torch.cuda.synchronize()
            mark(f"c5 fit {run}")
            t0 = time.perf_counter()
            m.fit(X, lab)
            torch.cuda.synchronize()
            tr = time.perf_counter() - t0
            mark(f"c5 predict {run}")
            t0 = time.perf_counter()
            proba = m.predict_proba(Xt)
            runs.append((tr, time.perf_counter() - t0, proba))
            mark(f"c5 end {run}")
        (tr0, inf0, _), (tr, inf, proba) = runs[0], runs[-1]
        acc = float((np.argmax(proba, axis=1) == labt).mean())
        if cpu is not None:
            cpu.update(cpu_train_estimate("c5", X, lab))
        print(f"[bench] C5 train {tr:.3f} s (first run {tr0:.3f}), predict_proba {inf:.3f} s "
              f"(first run {inf0:.3f}), acc {acc:.4f}", file=sys.stderr, flush=True)
        return {"c5_train_s": round(tr, 3), "c5_infer_s": round(inf, 3),
                "c5_train_cold_s": round(tr0, 3), "c5_infer_cold_s": round(inf0, 3),
                "c5_acc": round(acc, 4)}
    raise SystemExit(f"unknown extra config {cfg}")


if __name__ == "__main__":
    main()
