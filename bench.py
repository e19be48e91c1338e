#!/usr/bin/env python3
"""Benchmark of TinyGNN's sparse-inference hot path on one MI355X.

Metric: CSR SpMM GB/s and % of HBM peak; forward ms at the
232,965-node / 114,615,892-edge graph.

Default run (N=1):
  * headline ``value``: CSR SpMM (tinygnn::spmm, reference src/ops.cpp:198-297)
    on the config-D matrix -- 1,000,000 x 1,000,000, power-law out-degree
    (exponent 2.1, mean 50, clip 20,000; 50,000,000 nonzeros), values in
    (0,1] -- times a dense N(0,1) B of width F=128.  One "step" = one SpMM
    pass with the matrix and B already resident in HBM.  GB/s counts the
    algorithmic bytes 4(M+1) + 8 nnz + 4 F nnz + 4 F M (the reference's own
    cost model, ops.cpp:186-191);
  * the rest of the sweep (F = 32, 512) as ``sweep``;
  * ``cpu_baseline``: the reference's spmm compiled from its sources
    (oracle/_ref) or, where that library is absent, the oracle restatement,
    timed on the host cores over a bounded row sample of the same matrix.

``--gpus N`` with N > 1 exits: this build measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def spmm_bytes(m: int, nnz: int, f: int) -> int:
    """Algorithmic HBM bytes of one SpMM pass (reference ops.cpp:186-191)."""
    return 4 * (m + 1) + 8 * nnz + 4 * f * nnz + 4 * f * m


def csr_from_edges_host(src: np.ndarray, dst: np.ndarray, n: int):
    """edge_list_to_csr semantics (row = src, sorted destinations, duplicates
    kept) computed with numpy; used only to stage the benchmark input."""
    key = (src.astype(np.int64) << 32) | dst.astype(np.int64)
    key.sort()
    ci = (key & 0xFFFFFFFF).astype(np.int32)
    rp = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(src, minlength=n), out=rp[1:])
    return rp.astype(np.int32), ci


class StreamTimer:
    """HIP events recorded on the stream the kernels are launched on."""

    def __init__(self, torch, stream):
        self.torch = torch
        self.stream = stream
        self.pairs = []

    def start(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e

    def stop(self, e0):
        e1 = self.torch.cuda.Event(enable_timing=True)
        e1.record(self.stream)
        self.pairs.append((e0, e1))

    def ms(self):
        return [a.elapsed_time(b) for a, b in self.pairs]


def run_spmm_d(args, torch, tg):
    from tinygnn_amd import synth

    t0 = time.time()
    src, dst = synth.powerlaw_edges(synth.D_NODES, synth.D_EDGES, alpha=2.1, dmax=20000,
                                    seed=args.seed, shuffle=False)
    m = synth.D_NODES
    rp, ci = csr_from_edges_host(src, dst, m)
    del src, dst
    nnz = int(rp[-1])
    rng = np.random.default_rng(args.seed + 2)
    val = (1.0 - rng.random(nnz, dtype=np.float32)).astype(np.float32)  # (0, 1]
    deg = np.diff(rp)
    log(f"config D: m={m} nnz={nnz} max_deg={int(deg.max())} built in {time.time()-t0:.1f}s")

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    a = tg.DeviceCSR.from_numpy(m, m, rp, ci, val, device=dev)
    fs = sorted(set(args.f_sweep) | {args.f})
    fmax = max(fs)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 3)
    b_full = torch.randn((m, fmax), generator=gen, device=dev, dtype=torch.float32)
    plan = tg.SpmmPlan(a.row_ptr, m, nnz, fmax, stream=stream)
    info = plan.info()
    log(f"plan: {info}")

    results = {}
    for f in fs:
        b = b_full[:, :f].contiguous()
        c = torch.empty((m, f), device=dev, dtype=torch.float32)
        for _ in range(args.warmup):
            tg.spmm(a, b, plan=plan, out=c)
        torch.cuda.synchronize()
        timer = StreamTimer(torch, stream)
        t_start = time.perf_counter()
        for _ in range(args.steps):
            e0 = timer.start()
            tg.spmm(a, b, plan=plan, out=c)
            timer.stop(e0)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t_start) * 1e3 / args.steps
        ev = timer.ms()
        nbytes = spmm_bytes(m, nnz, f)
        avg = float(np.mean(ev))
        results[f] = dict(f=f, ms_per_step=wall, kernel_ms_avg=avg,
                          kernel_ms_median=float(np.median(ev)),
                          gbs=nbytes / (wall * 1e-3) / 1e9,
                          kernel_gbs=nbytes / (avg * 1e-3) / 1e9, bytes=nbytes,
                          gflops=2.0 * nnz * f / (avg * 1e-3) / 1e9)
        log(f"F={f}: {wall:.3f} ms/step, kernel avg {avg:.3f} ms, "
            f"{results[f]['kernel_gbs']:.0f} GB/s algorithmic")
        # Spot-check a few rows against an fp64 product (cheap sanity, the
        # parity tests are in tests/).
        rows = np.random.default_rng(1).integers(0, m, size=64)
        cb = c[torch.from_numpy(rows).to(dev)].cpu().numpy().astype(np.float64)
        bh = b_full[:, :f]
        for k, r in enumerate(rows):
            s, e = rp[r], rp[r + 1]
            cols = torch.from_numpy(ci[s:e].astype(np.int64)).to(dev)
            ref = (torch.from_numpy(val[s:e].astype(np.float64)).to(dev)[:, None] *
                   bh[cols].double()).sum(0).cpu().numpy()
            err = np.abs(cb[k] - ref).max() if e > s else np.abs(cb[k]).max()
            assert err <= 1e-3 * max(1.0, np.abs(ref).max() if e > s else 1.0), (r, err)
        del b, c

    head = results[args.f]
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_spmm(rp, ci, val, b_full[:, :args.f].contiguous().cpu().numpy(),
                                args)
    return dict(m=m, nnz=nnz, max_deg=int(deg.max()), plan=info, results=results,
                head=head, cpu=cpu)


def cpu_baseline_spmm(rp, ci, val, b, args):
    """The reference spmm on the host cores over rows [0, R) of the same
    matrix with the full B; R is sized for a few seconds per call."""
    import oracle

    f = b.shape[1]
    kind = "reference" if oracle.has_reference() else "port"
    lib = oracle.reference() if kind == "reference" else oracle.restate()
    cores = lib.num_threads()
    m = rp.shape[0] - 1
    target_nnz = min(int(rp[-1]), args.cpu_sample_nnz)
    r = int(np.searchsorted(rp, target_nnz))
    r = max(1, min(r, m))
    nnz_s = int(rp[r])
    sub = oracle.CSR(r, m, rp[:r + 1].copy(), ci[:nnz_s].copy(), val[:nnz_s].copy())
    times = []
    if kind == "reference":
        ta, tb = lib.csr(sub), lib.dense(b)
        out = np.zeros((r, f), np.float32)
        import ctypes
        t_end = time.time() + args.cpu_seconds
        while len(times) < 5 and (len(times) < 2 or time.time() < t_end):
            t0 = time.perf_counter()
            lib._check(lib.L.ref_spmm(ta.h, tb.h, out.ctypes.data_as(ctypes.c_void_p)))
            times.append(time.perf_counter() - t0)
    else:
        t_end = time.time() + args.cpu_seconds
        while len(times) < 5 and (len(times) < 2 or time.time() < t_end):
            t0 = time.perf_counter()
            lib.spmm(sub, b)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nbytes = spmm_bytes(r, nnz_s, f)
    log(f"cpu baseline ({kind}, {cores} threads): rows [0,{r}) nnz {nnz_s}: "
        f"{med*1e3:.1f} ms -> {nbytes/med/1e9:.1f} GB/s")
    return dict(value=nbytes / med / 1e9, unit="GB/s", cores=cores, kind=kind,
                sample=f"spmm rows [0,{r}) of the config-D matrix ({nnz_s} nnz) x full B "
                       f"(F={f}); median of {len(times)} calls, {med*1e3:.1f} ms each")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--f", type=int, default=128, help="headline feature width")
    ap.add_argument("--f-sweep", type=int, nargs="*", default=[32, 128, 512])
    ap.add_argument("--seed", type=int, default=2101)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-sample-nnz", type=int, default=10_000_000)
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(sharding is design-only, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch

    import tinygnn_amd as tg

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    tg.lib.load()
    torch.cuda.set_device(0)

    r = run_spmm_d(args, torch, tg)
    head = r["head"]
    line = {
        "metric": "CSR SpMM GB/s & % HBM peak; forward ms at 233K nodes / 114.6M edges",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded power-law CSR, N(0,1) features)",
        "config": {"workload": f"spmm config D: 1,000,000 x 1,000,000 CSR, {r['nnz']} nnz "
                               f"(power-law 2.1, max deg {r['max_deg']}), F={args.f}",
                   "m": r["m"], "nnz": r["nnz"], "f": args.f},
        "pct_hbm_peak": round(100.0 * head["gbs"] / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(head["kernel_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": "spmm pass (agg_chunk_kernel + agg_reduce_kernel)",
                     "kernel_ms_avg": round(head["kernel_ms_avg"], 4),
                     "bytes_per_launch": head["bytes"]},
        "sweep": [{"f": v["f"], "ms": round(v["kernel_ms_avg"], 4),
                   "gbs": round(v["kernel_gbs"], 1),
                   "pct_hbm_peak": round(100 * v["kernel_gbs"] / HBM_PEAK_GBS, 2)}
                  for v in r["results"].values()],
        "cpu_baseline": r["cpu"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
