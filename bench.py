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
    timed on the host cores over a bounded row sample of the same matrix;
  * ``forward``: the config-E forwards (232,965 nodes, 114,615,892 edges,
    602-d features): 2-layer GCN, SAGE-mean and GAT (4 x 64 heads), median
    ms with cached preprocessing and with the reference's semantics
    (gcn_norm / add_self_loops inside every forward), the reference's
    Model::forward timed once on the host cores, and the parity of the
    log-softmax logits against it (|err| <= 1e-5 + 1e-4|ref|, argmax).
  * ``cora``: configs A/B/C (Cora-synth GCN / SAGE / GAT): microseconds per
    forward, cached and with the reference's semantics, beside the compiled
    reference at all host threads and at one, and raw-output parity;
  * ``ingest``: GraphLoader's CSV parsing on the device -- a 20M-line edge
    list and a 50,000 x 602 feature table -- with the text in HBM and through
    the file path, against the compiled reference's parser on a sample.
Graphs are generated on the GPU from seeded power-law degrees and built into
CSR by the library's own edge_list_to_csr (its time is reported).

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
DEFAULT_SEED = 2101
PMC_SUMMARY = os.path.join(ROOT, "profiles", "spmm_configD_pmc.md")


def measure_copy(torch, reps: int = 10):
    """Achievable HBM bandwidth of a plain stream on this box, beside the
    8 TB/s peak: a 1 GiB device-to-device copy (1 GiB read + 1 GiB written),
    HIP events on the current stream, median of `reps` copies after 3
    warm-ups."""
    x = torch.ones(1 << 28, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        y.copy_(x)
        e1.record()
        ts.append((e0, e1))
    torch.cuda.synchronize()
    ms = float(np.median([a.elapsed_time(b) for a, b in ts]))
    nbytes = 2 * x.numel() * 4
    del x, y
    torch.cuda.empty_cache()
    print(f"[bench] device copy of 1 GiB: {ms:.3f} ms, {nbytes / ms / 1e6:.0f} GB/s",
          file=sys.stderr)
    return {"gbs": round(nbytes / ms / 1e6, 1), "ms": round(ms, 4), "bytes": nbytes,
            "kernel": "torch copy_ of 1 GiB (read + write)",
            "note": "a read + write stream; the SpMM pass reads almost only, and part of its "
                    "B gathers hit the MALL / L2, so its algorithmic rate can exceed this"}


def measured_traffic(f: int, seed: int):
    """Bytes per SpMM launch between L2 and the fabric (HBM and Infinity
    Cache), from the committed rocprofv3 summary: fetched = 32/64/128 x the
    per-size L2 read-request counters, written = WRITE_SIZE.  For the
    default workload only; None when no profile covers this configuration."""
    import re

    if seed != DEFAULT_SEED or not os.path.exists(PMC_SUMMARY):
        return None
    m = re.search(r'"spmm_configD_traffic_bytes":\s*(\{[^}]*\})', open(PMC_SUMMARY).read())
    if not m:
        return None
    v = json.loads(m.group(1)).get(str(f))
    return int(v) if v is not None else None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def spmm_bytes(m: int, nnz: int, f: int) -> int:
    """Algorithmic HBM bytes of one SpMM pass (reference ops.cpp:186-191)."""
    return 4 * (m + 1) + 8 * nnz + 4 * f * nnz + 4 * f * m


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


def build_graph_gpu(torch, tg, n, n_edges, seed, dev):
    """Seeded power-law edge list drawn on the GPU (synth.powerlaw_edges_device),
    then the device CSR build (edge_list_to_csr).  Returns the device CSR and
    the build time in ms."""
    from tinygnn_amd import synth

    src, dst = synth.powerlaw_edges_device(torch, n, n_edges, seed, dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a = tg.edge_list_to_csr(src, dst, n)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3
    del src, dst
    return a, ms


def run_spmm_d(args, torch, tg):
    from tinygnn_amd import synth

    t0 = time.time()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    m = synth.D_NODES
    a, csr_ms = build_graph_gpu(torch, tg, m, synth.D_EDGES, args.seed, dev)
    nnz = a.nnz
    gv = torch.Generator(device=dev)
    gv.manual_seed(args.seed + 2)
    a.val = 1.0 - torch.rand(nnz, generator=gv, device=dev)  # (0, 1]
    rp, ci, val = a.to_numpy()
    deg = np.diff(rp)
    log(f"config D: m={m} nnz={nnz} max_deg={int(deg.max())} built in {time.time()-t0:.1f}s "
        f"(device CSR build {csr_ms:.1f} ms)")
    fs = sorted(set(args.f_sweep) | {args.f})
    fmax = max(fs)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 3)
    b_full = torch.randn((m, fmax), generator=gen, device=dev, dtype=torch.float32)
    # the plan: its build (count, scans, one synchronisation for the sizes,
    # scatter) is a one-time cost per CSR structure, timed here apart from
    # the passes; the default plan sums in the reference's order
    plan_ms = []
    for _ in range(5):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        p_t = tg.SpmmPlan(a.row_ptr, m, nnz, fmax, stream=stream)
        torch.cuda.synchronize()
        plan_ms.append((time.perf_counter() - t1) * 1e3)
        p_t.close()
    plan_build_ms = float(np.median(plan_ms))
    plan = tg.SpmmPlan(a.row_ptr, m, nnz, fmax, stream=stream)
    plan_fast = tg.SpmmPlan(a.row_ptr, m, nnz, fmax, stream=stream,
                            precision=tg.PRECISION_FAST)
    info = plan.info()
    log(f"plan: {info}; built in {plan_build_ms:.2f} ms (median of 5)")

    def time_spmm(f, p):
        b = b_full[:, :f].contiguous()
        c = torch.empty((m, f), device=dev, dtype=torch.float32)
        for _ in range(args.warmup):
            tg.spmm(a, b, plan=p, out=c)
        torch.cuda.synchronize()
        timer = StreamTimer(torch, stream)
        t_start = time.perf_counter()
        for _ in range(args.steps):
            e0 = timer.start()
            tg.spmm(a, b, plan=p, out=c)
            timer.stop(e0)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t_start) * 1e3 / args.steps
        ev = timer.ms()
        nbytes = spmm_bytes(m, nnz, f)
        avg = float(np.mean(ev))
        return c, dict(f=f, ms_per_step=wall, kernel_ms_avg=avg,
                       kernel_ms_median=float(np.median(ev)),
                       gbs=nbytes / (wall * 1e-3) / 1e9,
                       kernel_gbs=nbytes / (avg * 1e-3) / 1e9, bytes=nbytes,
                       gflops=2.0 * nnz * f / (avg * 1e-3) / 1e9)

    results, results_fast = {}, {}
    for f in fs:
        _, results_fast[f] = time_spmm(f, plan_fast)
        c, results[f] = time_spmm(f, plan)
        log(f"F={f}: {results[f]['ms_per_step']:.3f} ms/step, kernel avg "
            f"{results[f]['kernel_ms_avg']:.3f} ms, {results[f]['kernel_gbs']:.0f} GB/s "
            f"algorithmic (exact: the reference's order); fast (per-chunk partials) "
            f"{results_fast[f]['kernel_ms_avg']:.3f} ms, "
            f"{results_fast[f]['kernel_gbs']:.0f} GB/s")
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
        del c

    head = results[args.f]
    cpp = None
    if not args.no_cpp_api:
        cpp = cpp_api_spmm(torch, tg, a, rp, ci, val, b_full[:, :args.f].contiguous(), plan,
                           args.steps)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_spmm(rp, ci, val, b_full[:, :args.f].contiguous().cpu().numpy(),
                                args)
    plan_fast.close()
    return dict(m=m, nnz=nnz, max_deg=int(deg.max()), plan=info, results=results,
                results_fast=results_fast, head=head, cpu=cpu, csr_build_ms=csr_ms,
                cpp_api=cpp, plan_build_ms=plan_build_ms)


def _tinygnn_pkg():
    """The reference's Python surface (package ``tinygnn``: pybind
    ``_tinygnn_core`` over this build's C++ API, libtinygnn.so)."""
    pkg = os.path.join(ROOT, "tinygnn_amd")
    if pkg not in sys.path:
        sys.path.insert(0, pkg)
    import tinygnn
    return tinygnn


def wall_ms_per_call(torch, fn, reps: int, warmup: int = 2) -> float:
    """Wall milliseconds per call of fn over reps calls, the device
    synchronised before and after the loop (each call's launches, host work
    and allocation included)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / reps


def _csr_view(n_rows, n_cols, rp, ci, val):
    """The attributes Tensor.from_scipy_csr reads (shape, indptr, indices, data)."""
    from types import SimpleNamespace
    return SimpleNamespace(shape=(n_rows, n_cols), indptr=rp, indices=ci, data=val)


def cpp_api_spmm(torch, tg, a, rp, ci, val, b, plan, reps):
    """tinygnn::spmm(A, B) (the reference's ops.hpp:112, this build's
    include/tinygnn/ops.hpp over libtinygnn.so) through the pybind module,
    against the C-ABI call tg_spmm_execute on the same device data: wall ms
    per call.  The C++ API returns a new tensor per call (value semantics);
    the C-ABI call writes into a preallocated output.  Both reuse a plan (the
    C++ API caches one per CSR tensor version).  The outputs must agree bit
    for bit."""
    T = _tinygnn_pkg()
    m = a.n_rows
    A = T.Tensor.from_scipy_csr(_csr_view(m, a.n_cols, rp, ci, val))
    B = T.from_torch(b)
    keep = [None]

    def cpp():
        keep[0] = T.spmm(A, B)

    c = torch.empty((m, b.shape[1]), device=b.device)
    cpp_ms = wall_ms_per_call(torch, cpp, reps)
    cabi_ms = wall_ms_per_call(torch, lambda: tg.spmm(a, b, plan=plan, out=c), reps)
    same = bool(torch.equal(T.to_torch(keep[0]).view(torch.int32), c.view(torch.int32)))
    log(f"C++ API spmm: {cpp_ms:.3f} ms/call, C-ABI {cabi_ms:.3f} ms/call, bit-identical {same}")
    del keep, A, B
    return dict(cpp_api_ms_per_call=round(cpp_ms, 4), c_abi_ms_per_call=round(cabi_ms, 4),
                ratio=round(cpp_ms / cabi_ms, 4), bit_identical=same, calls=reps)


def cpp_api_gcn_layer(torch, rp, ci, val, x, w, b, reps):
    """GCNLayer::forward (the reference's layers.hpp:172-214, layers.cpp:
    286-339) through the pybind module over libtinygnn.so at config E's layer
    1 (602 -> 256, ReLU) on gcn_norm(A): wall ms per call, against the same
    steps as separate C++ API calls (matmul, spmm, add_bias, relu_inplace --
    the reference's sequence, two more passes over the 238 MB output).  The
    layer fuses bias and ReLU into the SpMM's store; the two results must be
    bit-identical."""
    T = _tinygnn_pkg()
    n = rp.shape[0] - 1
    A = T.Tensor.from_scipy_csr(_csr_view(n, n, rp, ci, val))
    An = T.gcn_norm(A)
    H = T.from_torch(x)
    W = T.from_torch(w)
    B = T.from_torch(b.reshape(1, -1))
    layer = T.GCNLayer(w.shape[0], w.shape[1], True, T.Activation.RELU)
    layer.set_weight(W)
    layer.set_bias(B)
    keep = [None, None]

    def fused():
        keep[0] = layer.forward(An, H)

    def chain():
        out = T.spmm(An, T.matmul(H, W))
        T.add_bias(out, B)
        T.relu_inplace(out)
        keep[1] = out

    fused_ms = wall_ms_per_call(torch, fused, reps)
    chain_ms = wall_ms_per_call(torch, chain, reps)
    same = bool(torch.equal(T.to_torch(keep[0]).view(torch.int32),
                            T.to_torch(keep[1]).view(torch.int32)))
    log(f"C++ API GCNLayer::forward (602 -> 256, ReLU, unblocked): {fused_ms:.2f} ms/call fused, "
        f"{chain_ms:.2f} ms as separate calls, bit-identical {same}")
    del keep, A, An, H, W, B, layer
    return dict(gcn_layer_ms_per_call=round(fused_ms, 3),
                separate_calls_ms_per_call=round(chain_ms, 3), bit_identical=same, calls=reps,
                note="layer 1 of config E's GCN on gcn_norm(A) through libtinygnn.so: matmul, "
                     "then spmm with add_bias and relu fused into its store, against matmul, "
                     "spmm, add_bias, relu_inplace as separate calls")


def cpp_api_model(torch, tg, spec, w, adj, rp, ci, val, x, y_cabi, reps):
    """Model::forward (the reference's model.hpp:148) through the pybind
    module over libtinygnn.so, against tg_model_forward through ctypes on the
    same graph, features and weights (loaded from a TGNN weight file by the
    C++ side): wall ms per cached forward (the C++ Model reuses the derived
    adjacency while the tensor and its version are unchanged).  Outputs must
    agree bit for bit with the C-ABI forward's."""
    import tempfile
    T = _tinygnn_pkg()
    M = T.Model()
    post = {0: T.Model.InterActivation.NONE, 1: T.Model.InterActivation.RELU,
            2: T.Model.InterActivation.ELU}
    act = {0: T.Activation.NONE, 1: T.Activation.RELU}
    for l in spec:
        if l["type"] == "gcn":
            M.add_gcn_layer(l["in"], l["out"], True, act[l["act"]], post[l["post"]])
        elif l["type"] == "sage":
            M.add_sage_layer(l["in"], l["out"], T.SAGELayer.Aggregator.Mean, True,
                             act[l["act"]], post[l["post"]])
        else:
            M.add_gat_layer(l["in"], l["out"], l["heads"], l["concat"], l["slope"], True,
                            act[l["act"]], post[l["post"]])
    fd, path = tempfile.mkstemp(suffix=".tgnn")
    os.close(fd)
    try:
        tg.save_weight_file(path, w)
        M.load_weights(path)
    finally:
        os.remove(path)
    n = adj.n_rows
    A = T.Tensor.from_scipy_csr(_csr_view(n, n, rp, ci, val))
    X = T.from_torch(x)
    keep = [None]

    def cpp():
        keep[0] = M.forward(A, X)

    cpp_ms = wall_ms_per_call(torch, cpp, reps)
    same = bool(torch.equal(T.to_torch(keep[0]).view(torch.int32), y_cabi.view(torch.int32)))
    del keep, A, X, M
    return cpp_ms, same


def logit_parity(got, want):
    """|err| <= 1e-5 + 1e-4|want| elementwise, argmax agreement, and the
    number of nodes whose reference top-2 gap is within the largest error
    (near-ties, where any non-bit-exact path may flip the argmax).  Applied
    to raw Model::forward outputs and to log-softmax logits alike."""
    err = np.abs(got.astype(np.float64) - want)
    tol = 1e-5 + 1e-4 * np.abs(want.astype(np.float64))
    top2 = np.sort(want, axis=1)[:, -2:]
    ties = int(((top2[:, 1] - top2[:, 0]) <= float(err.max())).sum())
    return dict(max_abs_err=float(err.max()), within_tol=bool((err <= tol).all()),
                n_out_of_tol=int((err > tol).sum()),
                argmax_mismatch=int((got.argmax(1) != want.argmax(1)).sum()), near_ties=ties)


MFMA_PEAK_TFS = 157.3  # fp32 dense MFMA, MI355X


def _gemm_cost(m, k, n):
    """(bytes, flops) of C[m x n] = A[m x k] B[k x n], each operand once."""
    return 4 * (m * k + k * n + m * n), 2 * m * n * k


def _blocked_cost(n, nnz, f, nb, gc, values=False, self_term=False, score_heads=0):
    """Compulsory L2 fills of one blocked aggregation (all its passes) of
    width f over a structure of nnz entries cut into nb column blocks, with
    lane groups of gc columns (g = ceil(f / gc) groups):
      * the index stream once per column group: 2 nnz g for blocks of at
        most 65,536 rows (16-bit offsets in the block), else 4 nnz g; values
        4 nnz g more;
      * the chunk descriptors once per column group and block: 16 n nb g;
      * each block's slice of the gathered matrix once per XCD's L2:
        8 x 4 n f (with f padded to whole 32-column tiles);
      * the output read and written once per block after the first:
        4 n f (2 nb - 1);
      * a self term (SAGE) once: 4 n f;
      * GAT: the row's source score per column group and pass, 4 n g nb (the
        destination scores a_r . Wh_j are computed in the pass from the
        gathered rows), and the online softmax state (max, sum) per row and
        column group, read and written once per block after the first:
        8 n g (2 nb - 1).
    The gathers themselves (4 f bytes per entry) are served by L2 and are not
    counted here (gather_lines); they are what the passes spend their time
    on."""
    g = -(-f // gc)
    fpad = -(-f // 32) * 32
    idx = 2 if -(-n // nb) <= 65536 else 4
    b = (idx * nnz * g + (4 * nnz * g if values else 0) + 16 * n * nb * g + 8 * 4 * n * fpad +
         4 * n * f * (2 * nb - 1))
    if self_term:
        b += 4 * n * f
    if score_heads:
        b += 4 * n * g * nb + 8 * n * g * (2 * nb - 1)
    return b


def gather_lines(f, gc):
    """128-byte lines one entry's gather touches in a blocked aggregation of
    width f in lane groups of gc columns: one per 32-column tile (tile-major,
    gc = 32); a 64-column group's row-major 256-byte span covers
    ceil(4 c / 128) lines for its c valid columns."""
    if gc == 32:
        return -(-f // 32)
    return sum(-(-4 * min(gc, f - c0) // 128) for c0 in range(0, f, gc))


def forward_roofline(name, n, nnz_a, f_in, hidden, classes, heads, info, l2_gbs=None):
    """T_roof of the config-E cached forward in fast precision, over the
    kernels of the dataflow the library ran (info = Model.blocking_info()):
    sum over kernels of max(bytes / 8 TB/s, flops / 157.3 TFLOP/s), bytes as
    _gemm_cost / _blocked_cost (the reference's SpMM cost model,
    ops.cpp:186-191, where a pass is unblocked).  With l2_gbs (the measured
    rate of the aggregation kernel gathering L2-resident rows), a second sum
    adds the blocked passes' gathers as a third bound, gathered lines x 128
    bytes / l2_gbs.  Returns (ms, ms with the gather bound or None,
    per-kernel list)."""
    nnz_s = nnz_a + n
    ks = []

    def gemm(label, m, k, nn):
        b, fl = _gemm_cost(m, k, nn)
        ks.append((label, b, fl, 0))

    def agg(label, nnz, f, nb, gc, **kw):
        if nb > 0:
            ks.append((label, _blocked_cost(n, nnz, f, nb, gc, **kw), 2 * nnz * f,
                       128 * nnz * gather_lines(f, gc)))
        else:  # unblocked: the reference's cost model (gathers from HBM)
            v = 0 if kw.get("values") is False else 4 * nnz
            ks.append((label, 4 * (n + 1) + 4 * nnz + v + 4 * f * nnz + 4 * f * n, 2 * nnz * f,
                       0))

    if name == "gcn":
        nb, gc = info["blocks_sl"], info["cols_sl"]
        weighted = not (nb > 0 and gc == 32)  # factored GCN passes carry no values
        gemm("L1 transform", n, f_in, hidden)
        agg("L1 aggregation", nnz_s, hidden, nb, gc, values=weighted)
        gemm("L2 transform", n, hidden, classes)
        agg("L2 aggregation", nnz_s, classes, nb, gc, values=weighted)
    elif name == "sage":
        nb, gc = info["blocks_raw"], info["cols_raw"]
        gemm("L1 transform [Ws|Wn]", n, f_in, 2 * hidden)
        agg("L1 mean aggregation", nnz_a, hidden, nb, gc, values=False, self_term=True)
        gemm("L2 transform [Ws|Wn]", n, hidden, 2 * 64)  # 41 + 41 padded to 64 + 64
        agg("L2 mean aggregation", nnz_a, classes, nb, gc, values=False, self_term=True)
    else:
        # fast precision: the softmax rides along the blocked passes (a
        # running (max, sum) per row and column group, read and written per pass);
        # unblocked, one online-softmax pass
        nb, gc = info["blocks_sl"], info["cols_sl"]
        for li, (fi, fo, h) in enumerate(((f_in, hidden, heads), (hidden * heads, classes, 1))):
            gemm(f"L{li + 1} transform", n, fi, fo * h)
            ks.append((f"L{li + 1} scores", 4 * n * fo * h + 8 * n * h, 4 * n * fo * h, 0))
            agg(f"L{li + 1} attention aggregation", nnz_s, fo * h, nb, gc, values=False,
                score_heads=h)
    out, tot, tot_l2 = [], 0.0, 0.0
    for label, b, fl, gb in ks:
        t = max(b / (HBM_PEAK_GBS * 1e6), fl / (MFMA_PEAK_TFS * 1e9))
        tot += t
        k = dict(kernel=label, bytes=int(b), flops=int(fl), t_roof_ms=round(t, 4),
                 bound="hbm" if b / (HBM_PEAK_GBS * 1e6) >= fl / (MFMA_PEAK_TFS * 1e9)
                 else "mfma")
        if gb:
            k["gathered_bytes"] = int(gb)
            if l2_gbs:
                k["t_gather_ms"] = round(gb / (l2_gbs * 1e6), 4)
        tot_l2 += max(t, gb / (l2_gbs * 1e6)) if l2_gbs else t
        out.append(k)
    return tot, (tot_l2 if l2_gbs else None), out


def run_forward_e(args, torch, tg):
    """2-layer GCN / SAGE-mean / GAT forwards at config E, with the
    reference's Model::forward timed on the host cores and full-size
    parity of the logits."""
    from tinygnn_amd import synth

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    n = synth.E_NODES
    t0 = time.time()
    l2 = measure_l2_gather(torch, tg)
    l2_read = measure_l2_read(torch, tg)
    l2_rate = l2_read["rate_gbs"]
    adj, csr_ms = build_graph_gpu(torch, tg, n, synth.E_EDGES, args.seed + 10, dev)
    rng = np.random.default_rng(args.seed + 11)
    x_h = rng.standard_normal((n, synth.E_FEATURES), dtype=np.float32)
    x = torch.from_numpy(x_h).to(dev)
    # the one-time upload a caller with the graph in host memory pays
    rp_h, ci_h, val_h = adj.to_numpy()
    h2d = measure_h2d(torch, [rp_h, ci_h, val_h, x_h])
    del rp_h, ci_h, val_h
    log(f"config E upload (CSR + features, {h2d['bytes']} bytes): pageable "
        f"{h2d['pageable']['ms']} ms, pinned {h2d['pinned']['ms']} ms")
    log(f"config E: n={n} nnz={adj.nnz} built in {time.time()-t0:.1f}s "
        f"(device CSR build {csr_ms:.1f} ms)")
    specs = {"gcn": synth.spec_gcn(synth.E_FEATURES, 256, synth.E_CLASSES),
             "sage": synth.spec_sage(synth.E_FEATURES, 256, synth.E_CLASSES),
             "gat": synth.spec_gat(synth.E_FEATURES, 64, 4, synth.E_CLASSES)}
    ref = ref_tensors = None
    if not args.no_cpu:
        import oracle
        if oracle.has_reference():
            ref = oracle.reference()
            rp, ci, val = adj.to_numpy()
            t1 = time.time()
            ref_csr = oracle.CSR(n, n, rp, ci, val)
            ref_tensors = (ref.csr(ref_csr), ref.dense(x_h))
            log(f"reference tensors built in {time.time()-t1:.1f}s")
            del rp, ci, val
    out = {}
    rp_e = ci_e = val_e = None
    for name, spec in specs.items():
        w = synth.model_weights(spec, seed=args.seed + 20)
        model = tg.Model.from_spec(spec, w)
        y = torch.empty((n, model.output_cols()), device=dev)
        # the first cached forward of a new model: its one-time preprocessing
        # (gcn_norm / add_self_loops, row plans, blocked copies, buffers)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        model.forward(adj, x, mode=tg.FORWARD_CACHED, out=y)
        torch.cuda.synchronize()
        first_ms = (time.perf_counter() - t1) * 1e3
        for _ in range(args.fwd_warmup):
            model.forward(adj, x, mode=tg.FORWARD_CACHED, out=y)
        torch.cuda.synchronize()
        timer = StreamTimer(torch, stream)
        for _ in range(args.fwd_steps):
            e0 = timer.start()
            model.forward(adj, x, mode=tg.FORWARD_CACHED, out=y)
            timer.stop(e0)
        torch.cuda.synchronize()
        cached = float(np.median(timer.ms()))
        blocking = model.blocking_info()
        cpp = None
        if not args.no_cpp_api:
            reps = max(3, args.fwd_steps // 2)
            cabi_wall = wall_ms_per_call(
                torch, lambda: model.forward(adj, x, mode=tg.FORWARD_CACHED, out=y), reps)
            if rp_e is None:
                rp_e, ci_e, val_e = adj.to_numpy()
            cpp_ms, same = cpp_api_model(torch, tg, spec, w, adj, rp_e, ci_e, val_e, x, y, reps)
            cpp = dict(cpp_api_ms_per_call=round(cpp_ms, 3), c_abi_ms_per_call=round(cabi_wall, 3),
                       ratio=round(cpp_ms / cabi_wall, 4), bit_identical=same, calls=reps)
            if name == "gcn":
                torch.cuda.empty_cache()
                cpp["gcn_layer"] = cpp_api_gcn_layer(
                    torch, rp_e, ci_e, val_e, x,
                    torch.from_numpy(w["layer0.weight"]).to(dev),
                    torch.randn(w["layer0.bias"].shape[1], device=dev), 3)
            log(f"{name}: C++ API Model::forward {cpp_ms:.2f} ms/call, C-ABI {cabi_wall:.2f} "
                f"ms/call, bit-identical {same}")
        # the timed (cached) forward's raw outputs and logits are the ones checked
        raw = y.cpu().numpy()
        logits = tg.log_softmax_(y.clone()).cpu().numpy()
        # reference-semantics calls (the adjacency preprocessed in every
        # call), timed as the cached ones: untimed warm-up calls, then calls
        # back to back, each bracketed by events on the stream
        for _ in range(args.fwd_warmup):
            model.forward(adj, x, mode=tg.FORWARD_REFERENCE, out=y)
        torch.cuda.synchronize()
        timer = StreamTimer(torch, stream)
        for _ in range(args.fwd_steps):
            e0 = timer.start()
            model.forward(adj, x, mode=tg.FORWARD_REFERENCE, out=y)
            timer.stop(e0)
        torch.cuda.synchronize()
        refsem = float(np.median(timer.ms()))
        # and each from an idle GPU (a synchronisation before the call: the
        # host's time to its first launch included)
        timer = StreamTimer(torch, stream)
        for _ in range(5):
            torch.cuda.synchronize()
            e0 = timer.start()
            model.forward(adj, x, mode=tg.FORWARD_REFERENCE, out=y)
            timer.stop(e0)
        torch.cuda.synchronize()
        refsem_idle = float(np.median(timer.ms()))
        raw_r = y.cpu().numpy()
        logits_r = tg.log_softmax_(y.clone()).cpu().numpy()
        # the same model in exact precision (the reference's operation order)
        model.set_precision(tg.PRECISION_EXACT)
        model.forward(adj, x, mode=tg.FORWARD_CACHED, out=y)
        torch.cuda.synchronize()
        timer = StreamTimer(torch, stream)
        for _ in range(3):
            e0 = timer.start()
            model.forward(adj, x, mode=tg.FORWARD_CACHED, out=y)
            timer.stop(e0)
        torch.cuda.synchronize()
        exact_ms = float(np.median(timer.ms()))
        raw_x = y.cpu().numpy()
        logits_x = tg.log_softmax_(y.clone()).cpu().numpy()
        model.set_precision(tg.PRECISION_FAST)
        troof, troof_l2, kern = forward_roofline(name, n, adj.nnz, synth.E_FEATURES,
                                                 256 if name != "gat" else 64, synth.E_CLASSES,
                                                 4, blocking, l2_rate)
        r = dict(gpu_ms=round(cached, 3), gpu_ms_reference_semantics=round(refsem, 3),
                 gpu_ms_reference_semantics_from_idle=round(refsem_idle, 3),
                 first_forward_ms=round(first_ms, 2),
                 one_time_preprocessing_ms=round(first_ms - cached, 2),
                 cpp_api=cpp,
                 gpu_ms_exact=round(exact_ms, 3), blocking=blocking,
                 roofline_ms=round(troof, 4), roofline_frac=round(troof / cached, 4),
                 roofline_kernels=kern,
                 roofline_note="T_roof = sum over the dataflow's kernels of max(compulsory "
                               "bytes / 8 TB/s, flops / 157.3 TF/s); blocked passes count "
                               "their compulsory L2 fills, not the L2-served gathers",
                 gather_bound_ms=round(troof_l2, 4) if troof_l2 else None,
                 gather_bound_frac=round(troof_l2 / cached, 4) if troof_l2 else None,
                 gather_bound_note="the same sum with each blocked pass bounded also by its "
                                   "gathered lines x 128 B at the box's L2 read ceiling "
                                   "(l2_read: plain coalesced loads of an L2-resident buffer)")
        log(f"{name}: first forward {first_ms:.1f} ms; cached {cached:.2f} ms, reference "
            f"semantics {refsem:.2f} ms ({refsem_idle:.2f} from idle), exact {exact_ms:.2f} ms; roofline {troof:.3f} ms, "
            f"gather bound "
            f"{troof_l2 or 0:.3f} ms ({(troof_l2 or 0) / cached:.3f})")
        if ref is not None:
            rm = ref.model(spec, w)
            t1 = time.perf_counter()
            want_raw = rm.forward_handles(ref_tensors[0], ref_tensors[1], n)
            cpu_ms = (time.perf_counter() - t1) * 1e3
            want = ref.activation("log_softmax", want_raw)
            layers = ref_layer_only(ref, oracle.restate(), spec, w, ref_csr, x_h)
            cpu_layers_ms = cpu_median_ms(layers, 1, warmup=0)
            del layers
            r.update(cpu_ms=round(cpu_ms, 1), cpu_threads=ref.num_threads(),
                     cpu_ms_layers=round(cpu_layers_ms, 1),
                     speedup=round(cpu_ms / cached, 1),
                     parity_raw=logit_parity(raw, want_raw),
                     parity_raw_reference_semantics=logit_parity(raw_r, want_raw),
                     parity=logit_parity(logits, want),
                     parity_reference_semantics=logit_parity(logits_r, want),
                     parity_exact=dict(
                         logit_parity(logits_x, want),
                         forward_bit_identical_frac=float(
                             (raw_x.view(np.int32) == want_raw.view(np.int32)).mean())))
            log(f"{name}: cpu {cpu_ms:.0f} ms ({ref.num_threads()} thr), parity {r['parity']}, "
                f"exact {r['parity_exact']}")
            del rm, want, want_raw
        del raw, raw_r
        out[name] = r
        del model, y
    return dict(n=n, nnz=adj.nnz, csr_build_ms=round(csr_ms, 2), h2d=h2d, l2_read=l2_read,
                l2_gather=l2, models=out)


def measure_l2_read(torch, tg, sizes_mb=(1, 2, 4), workgroups: int = 8192, reps: int = 20):
    """The L2 read ceiling of this box (tg_probe_l2_read): workgroups x the
    buffer size of plain coalesced 16-byte loads from a buffer that every
    XCD's 4 MB L2 holds, no gathers, no index stream.  HIP events around
    `reps` launches on the current stream, after 3 warm-ups; the best of the
    sizes is the ceiling."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sink = torch.empty(workgroups * 256, device=dev)
    out = {}
    for mb in sizes_mb:
        nbytes = mb << 20
        buf = torch.randn(nbytes // 4, device=dev)
        for _ in range(3):
            tg.lib.check(tg.lib.tg_probe_l2_read(buf.data_ptr(), nbytes, workgroups,
                                                 sink.data_ptr(), tg.stream_handle(stream)))
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            tg.lib.check(tg.lib.tg_probe_l2_read(buf.data_ptr(), nbytes, workgroups,
                                                 sink.data_ptr(), tg.stream_handle(stream)))
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[f"{mb}MB"] = dict(ms=round(ms, 4), gbs=round(workgroups * nbytes / ms / 1e6, 1))
        del buf
    best = max(v["gbs"] for v in out.values())
    r = dict(rate_gbs=best, by_size=out, workgroups=workgroups,
             kernel="tg_probe_l2_read: coalesced 16-byte loads of an L2-resident buffer")
    log(f"L2 read ceiling: {best} GB/s ({out})")
    return r


def measure_h2d(torch, arrays):
    """One-time upload of host arrays (numpy) to the device: pageable
    (torch .to(device), the path a caller with ordinary host memory takes)
    and from pinned host memory; wall time with synchronisation, best of 3."""
    dev = torch.device("cuda:0")
    nbytes = sum(a.nbytes for a in arrays)
    srcs = [torch.from_numpy(a) for a in arrays]
    pinned = [t.pin_memory() for t in srcs]
    res = {}
    for name, hs, nb in (("pageable", srcs, False), ("pinned", pinned, True)):
        best = None
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ds = [h.to(dev, non_blocking=nb) for h in hs]
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3
            best = ms if best is None else min(best, ms)
            del ds
        res[name] = dict(ms=round(best, 2), gbs=round(nbytes / best / 1e6, 1))
    del pinned
    return dict(bytes=int(nbytes), **res)


def measure_l2_gather(torch, tg, rows: int = 500_000, deg: int = 64, cols: int = 16384,
                      f: int = 32, reps: int = 50):
    """The aggregation kernel's gather rate when every gathered row is
    L2-resident: a SAGE-mean aggregation (unweighted, as the factored GCN
    and SAGE passes) of `rows` rows with `deg` sorted random columns each
    in [0, cols), B = cols x f floats (2 MB at the defaults: every line stays
    in each XCD's 4 MB L2).  Rate = gathered bytes (one 128-byte line per
    entry at f = 32) / HIP-event time per call, the mean over `reps` calls."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    rp = (torch.arange(rows + 1, device=dev, dtype=torch.int64) * deg).to(torch.int32)
    ci = torch.randint(0, cols, (rows, deg), generator=g, device=dev, dtype=torch.int32)
    ci = torch.sort(ci, dim=1)[0].reshape(-1).contiguous()
    a = tg.DeviceCSR(rows, cols, rp, ci, torch.ones(rows * deg, device=dev))
    b = torch.randn(cols, f, generator=g, device=dev)
    plan = tg.SpmmPlan(rp, rows, rows * deg, f)
    for _ in range(20):
        tg.sage_aggregate(plan, a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        tg.sage_aggregate(plan, a, b)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    gathered = rows * deg * 128 * (-(-f // 32))
    del a, b, plan, ci, rp
    torch.cuda.empty_cache()
    r = dict(rate_gbs=round(gathered / ms / 1e6, 1), ms=round(ms, 4), rows=rows, entries=rows * deg,
             cols=cols, f=f, gathered_bytes=gathered)
    log(f"L2-resident gather rate: {r['rate_gbs']} GB/s ({r})")
    return r


def run_calib_gather(torch, tg, rows: int = 1 << 23):
    """Calibration dispatches for rocprofv3 FETCH_SIZE on gather-shaped
    traffic: SpMM by a permutation matrix (one entry per row, every column
    once), so every row of B is gathered exactly once, in random order:
    F = 32 (one 128-byte line per gather, B 1 GiB) and F = 16 (64-byte
    gathers, half lines, B 512 MB), both beyond the MALL.  A dispatch's unique
    bytes are B + 12 rows (column, value, row pointer) read and 4 F rows
    written; its FETCH_SIZE against that figure gives the counter's scale for
    gathers of that size."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    perm = torch.randperm(rows, generator=g, device=dev).to(torch.int32)
    rp = torch.arange(rows + 1, device=dev, dtype=torch.int32)
    a = tg.DeviceCSR(rows, rows, rp, perm, torch.ones(rows, device=dev))
    out = {}
    for f in (32, 16):
        b = torch.randn(rows, f, generator=g, device=dev)
        c = torch.empty(rows, f, device=dev)
        plan = tg.SpmmPlan(rp, rows, rows, f)
        for _ in range(2):
            tg.spmm(a, b, plan=plan, out=c)
        torch.cuda.synchronize()
        out[f] = dict(rows=rows, read_bytes=4 * rows * f + 12 * rows, written_bytes=4 * rows * f)
        del b, c, plan
    del a, perm, rp
    torch.cuda.empty_cache()
    log(f"gather calibration dispatches: {out}")
    return out


def host_info():
    """The CPU the baselines ran on: model name, logical CPUs, the CPUs this
    process may use, and OMP_NUM_THREADS."""
    model = "?"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(cpu_model=model, nproc=os.cpu_count(), affinity=len(os.sched_getaffinity(0)),
                omp_num_threads=os.environ.get("OMP_NUM_THREADS"))


def cpu_median_ms(fn, reps: int, warmup: int = 1):
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return float(np.median(ts))


def ref_layer_only(ref, restate, spec, w, a, x):
    """A closure timing only the reference's layer forwards of a 2-layer
    model (layers.cpp:286-339, :538-752, :945-1129): the normalised / self-looped
    adjacency, every layer's input and the weights are prepared beforehand, so
    the per-call gcn_norm / add_self_loops and feature copy of Model::forward
    (model.cpp:373-391) and the head concat are left out."""
    import oracle
    kinds = {l["type"] for l in spec}
    a_gcn = ref.csr(restate.gcn_norm(a)) if "gcn" in kinds else None
    a_sl = ref.csr(restate.add_self_loops(a)) if "gat" in kinds else None
    a_raw = ref.csr(a)
    calls, h = [], x
    acsr = {"gcn": restate.gcn_norm(a) if a_gcn else None,
            "gat": restate.add_self_loops(a) if a_sl else None}
    for li, l in enumerate(spec):
        p = f"layer{li}"
        th = ref.dense(h)
        if l["type"] == "gcn":
            wt, b = oracle._f(w[p + ".weight"]), oracle._f(w[p + ".bias"])
            out = np.zeros((a.n_rows, l["out"]), np.float32)
            calls.append((ref.L.ref_gcn_layer, (a_gcn.h, th.h, l["in"], l["out"],
                                                 oracle._ptr(wt), oracle._ptr(b), 1,
                                                 l.get("act", 1), oracle._ptr(out)), (th, wt, b)))
            h = restate.gcn_layer(acsr["gcn"], h, wt, b, l.get("act", 1))
        elif l["type"] == "sage":
            wn, ws = oracle._f(w[p + ".weight_neigh"]), oracle._f(w[p + ".weight_self"])
            b = oracle._f(w[p + ".bias"])
            out = np.zeros((a.n_rows, l["out"]), np.float32)
            calls.append((ref.L.ref_sage_layer, (a_raw.h, th.h, l["in"], l["out"], 0,
                                                  oracle._ptr(wn), oracle._ptr(ws),
                                                  oracle._ptr(b), 1, l.get("act", 1),
                                                  oracle._ptr(out)), (th, wn, ws, b)))
            h = restate.sage_layer(a, h, wn, ws, b, l.get("act", 1))
        else:
            heads = []
            for hd in range(l.get("heads", 1)):
                hp = f"{p}.head{hd}"
                wt, al, ar = (oracle._f(w[hp + k]) for k in (".weight", ".attn_left",
                                                               ".attn_right"))
                b = oracle._f(w[hp + ".bias"])
                out = np.zeros((a.n_rows, l["out"]), np.float32)
                calls.append((ref.L.ref_gat_layer, (a_sl.h, th.h, l["in"], l["out"],
                                                     oracle._ptr(wt), oracle._ptr(al),
                                                     oracle._ptr(ar), oracle._ptr(b),
                                                     l.get("slope", 0.2), 1, l.get("act", 0),
                                                     oracle._ptr(out)), (th, wt, al, ar, b)))
                heads.append(restate.gat_layer(acsr["gat"], h, wt, al, ar, b,
                                               l.get("slope", 0.2), l.get("act", 0)))
            h = np.ascontiguousarray(np.concatenate(heads, axis=1)) if len(heads) > 1 else heads[0]
            if l.get("post", 0) == 2:
                h = restate.activation("elu", h, 1.0)
    keep = (a_gcn, a_sl, a_raw)

    def run():
        for fn, argv, _ in calls:
            ref._check(fn(*argv))
    run.keep = (keep, calls)
    return run


def run_cora(args, torch, tg):
    """Configs A/B/C: 2-layer GCN / SAGE-mean / GAT on the Cora-synth graph
    (2,708 nodes, 10,858 entries, 1,433 features).  GPU: microseconds per
    forward with cached preprocessing and with the reference's semantics
    (HIP events on the stream around each forward, median of args.cora_steps
    after 3 warm-ups).  Host: the compiled reference's Model::forward plus
    the caller's log_softmax (test_e2e.cpp:316) at all OpenMP threads and at
    one, and its layer-only time (median of 5).  Parity of the raw outputs
    and of the logits against the reference's."""
    from tinygnn_amd import synth
    import oracle

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    src, dst, x_h = synth.cora_synth()
    n = synth.CORA_NODES
    adj = tg.edge_list_to_csr(torch.from_numpy(src).to(dev), torch.from_numpy(dst).to(dev), n)
    x = torch.from_numpy(x_h).to(dev)
    ref = restate = None
    if not args.no_cpu and oracle.has_reference():
        ref, restate = oracle.reference(), oracle.restate()
        rp, ci, val = adj.to_numpy()
        a = oracle.CSR(n, n, rp, ci, val)
        ta, tx = ref.csr(a), ref.dense(x_h)
    out = {}
    for name, (spec, w) in synth.cora_models().items():
        m = tg.Model.from_spec(spec, w)
        y = torch.empty((n, m.output_cols()), device=dev)
        r = {}
        for mode, key in ((tg.FORWARD_CACHED, "gpu_us"),
                          (tg.FORWARD_REFERENCE, "gpu_us_reference_semantics")):
            for _ in range(3):
                m.forward(adj, x, mode=mode, out=y)
            torch.cuda.synchronize()
            timer = StreamTimer(torch, stream)
            for _ in range(args.cora_steps):
                e0 = timer.start()
                m.forward(adj, x, mode=mode, out=y)
                timer.stop(e0)
            torch.cuda.synchronize()
            r[key] = round(float(np.median(timer.ms())) * 1e3, 1)
        raw = y.cpu().numpy()
        logits = tg.log_softmax_(y.clone()).cpu().numpy()
        if ref is not None:
            rm = ref.model(spec, w)
            threads = ref.num_threads()

            def fwd():
                return ref.activation("log_softmax", rm.forward_handles(ta, tx, n))

            r["cpu_us"] = round(cpu_median_ms(fwd, 5) * 1e3, 1)
            ref.set_num_threads(1)
            r["cpu_us_1thread"] = round(cpu_median_ms(fwd, 5) * 1e3, 1)
            layers = ref_layer_only(ref, restate, spec, w, a, x_h)
            r["cpu_us_layers_1thread"] = round(cpu_median_ms(layers, 5) * 1e3, 1)
            ref.set_num_threads(threads)
            r["cpu_us_layers"] = round(cpu_median_ms(layers, 5) * 1e3, 1)
            r["cpu_threads"] = threads
            r["speedup"] = round(r["cpu_us"] / r["gpu_us"], 1)
            r["speedup_reference_semantics"] = round(r["cpu_us"] /
                                                     r["gpu_us_reference_semantics"], 1)
            want_raw = rm.forward_handles(ta, tx, n)
            r["parity_raw"] = logit_parity(raw, want_raw)
            r["raw_bit_identical_frac"] = float((raw.view(np.int32) ==
                                                 want_raw.view(np.int32)).mean())
            r["parity"] = logit_parity(logits, ref.activation("log_softmax", want_raw))
            del rm, layers
        log(f"cora {name}: gpu {r['gpu_us']} us cached, {r['gpu_us_reference_semantics']} us "
            f"reference semantics; cpu {r.get('cpu_us')} us ({r.get('cpu_threads')} thr), "
            f"{r.get('cpu_us_1thread')} us (1 thr); raw bit-identical "
            f"{r.get('raw_bit_identical_frac')}")
        out[name] = r
        del m, y
    return dict(n=n, nnz=adj.nnz, features=synth.CORA_FEATURES, models=out)


def run_ingest(args, torch, tg):
    """GraphLoader on the device (graph_loader.cpp:61-206): CSV parse time
    with the text already in HBM (the index and parse kernels), the file path
    end to end (read into pinned staging, copy, parse), and the compiled
    reference's parse_edges / parse_features timed on a bounded sample of the
    same texts, whose results must equal the device's bit for bit."""
    import tempfile

    from tinygnn_amd import synth

    rng = np.random.default_rng(args.seed + 7)
    n_nodes, f_in = 232_965, 602
    ne, nr = args.ingest_edges, args.ingest_rows
    src = rng.integers(0, n_nodes, ne)
    dst = rng.integers(0, n_nodes, ne)
    text_e = synth.edges_csv(src, dst)
    text_f, kf = synth.features_csv(nr, f_in, seed=args.seed + 8)
    ref = None
    if not args.no_cpu:
        import oracle
        ref = oracle.reference() if oracle.has_reference() else None
    tmp = tempfile.mkdtemp(prefix="tg_ingest_")
    out = {}
    for kind, text in (("edges", text_e), ("features", text_f)):
        dev_text = torch.from_numpy(np.frombuffer(text, np.uint8).copy()).cuda()

        def parse_dev():
            c = tg.CsvText.from_device(dev_text, kind)
            r = c.parse_edges()[:2] if kind == "edges" else c.parse_features()
            c.close()
            return r

        parse_dev()
        torch.cuda.synchronize()
        ms = []
        for _ in range(args.ingest_steps):
            t0 = time.perf_counter()
            res = parse_dev()
            torch.cuda.synchronize()
            ms.append((time.perf_counter() - t0) * 1e3)
        gpu_ms = float(np.median(ms))
        if kind == "edges":
            exact = bool(np.array_equal(res[0].cpu().numpy(), src) and
                         np.array_equal(res[1].cpu().numpy(), dst))
        else:  # decimal fields d.dddddd: within half an ulp of k / 1e6
            want = kf / 1e6
            got = res.cpu().numpy().astype(np.float64)
            exact = bool(np.all(np.abs(got - want) <= np.spacing(np.abs(want).astype(np.float32))
                                .astype(np.float64) / 2 + 1e-12))
        del res
        path = os.path.join(tmp, kind + ".csv")
        with open(path, "wb") as fh:
            fh.write(text)
        fms = []
        for _ in range(3):
            t0 = time.perf_counter()
            r2 = tg.parse_edges(path) if kind == "edges" else tg.parse_features(path)
            torch.cuda.synchronize()
            fms.append((time.perf_counter() - t0) * 1e3)
            del r2
        lines = ne if kind == "edges" else nr
        e = dict(bytes=len(text), lines=lines, gpu_ms=round(gpu_ms, 3),
                 gbs=round(len(text) / gpu_ms / 1e6, 1),
                 lines_per_s=round(lines / gpu_ms * 1e3, 0), values_ok=exact,
                 file_ms=round(float(np.median(fms)), 2),
                 file_gbs=round(len(text) / float(np.median(fms)) / 1e6, 2))
        log(f"ingest {kind}: {len(text) / 1e6:.0f} MB, device parse {gpu_ms:.2f} ms "
            f"({e['gbs']} GB/s), file path {e['file_ms']} ms, values ok {exact}")
        if ref is not None:
            # a bounded sample: the first lines of the same text
            n_s = min(lines, 2_000_000 if kind == "edges" else 3_000)
            cut = 0
            for _ in range(n_s + 1):  # header + n_s lines
                cut = text.index(b"\n", cut) + 1
            sample = os.path.join(tmp, kind + "_sample.csv")
            with open(sample, "wb") as fh:
                fh.write(text[:cut])
            t0 = time.perf_counter()
            want = (ref.parse_edges_file(sample) if kind == "edges"
                    else ref.parse_features_file(sample))
            cpu_ms = (time.perf_counter() - t0) * 1e3
            got = tg.parse_edges(sample) if kind == "edges" else tg.parse_features(sample)
            if kind == "edges":
                par = bool(np.array_equal(got[0].cpu().numpy(), want[0]) and
                           np.array_equal(got[1].cpu().numpy(), want[1]))
            else:
                par = bool(np.array_equal(got.cpu().numpy().view(np.int32), want.view(np.int32)))
            e["cpu_baseline"] = dict(value=round(cut / cpu_ms / 1e6, 3), unit="GB/s", cores=1,
                                     kind="reference", ms=round(cpu_ms, 1),
                                     sample=f"first {n_s} data lines ({cut} bytes)")
            e["parity_sample_bit_exact"] = par
            e["speedup_vs_reference"] = round(e["gbs"] / (cut / cpu_ms / 1e6), 1)
            log(f"ingest {kind}: reference {cut / cpu_ms / 1e6:.3f} GB/s on the sample, "
                f"bit-exact {par}")
        out[kind] = e
        del dev_text
    for fn in os.listdir(tmp):
        os.remove(os.path.join(tmp, fn))
    os.rmdir(tmp)
    return out


def cpu_baseline_spmm(rp, ci, val, b, args):
    """The reference's spmm (ops.cpp:198-297, compiled from its sources:
    oracle/_ref) on the host cores over the whole config-D matrix with the
    whole B, timed per call as the reference's own benchmark does
    (benchmarks/bench_datasets.cpp:57-69: one warm-up, then the median of
    the timed calls): at all OpenMP threads, the median of 5 calls; on one
    thread, one call.  --cpu-sample-nnz > 0 bounds the rows (a prefix of the
    matrix) for quick runs.  Where the compiled reference is absent the C
    restatement (single-threaded) is timed instead (kind "port")."""
    import ctypes

    import oracle

    f = b.shape[1]
    kind = "reference" if oracle.has_reference() else "port"
    lib = oracle.reference() if kind == "reference" else oracle.restate()
    cores = lib.num_threads()
    m = rp.shape[0] - 1
    target_nnz = int(rp[-1]) if args.cpu_sample_nnz <= 0 else min(int(rp[-1]),
                                                                   args.cpu_sample_nnz)
    r = m if target_nnz >= int(rp[-1]) else max(1, min(int(np.searchsorted(rp, target_nnz)), m))
    nnz_s = int(rp[r])
    sub = oracle.CSR(r, m, rp[:r + 1], ci[:nnz_s], val[:nnz_s])
    whole = r == m
    if kind == "reference":
        ta, tb = lib.csr(sub), lib.dense(b)
        out = np.zeros((r, f), np.float32)

        def call():
            lib._check(lib.L.ref_spmm(ta.h, tb.h, out.ctypes.data_as(ctypes.c_void_p)))
    else:
        def call():
            lib.spmm(sub, b)
    med = cpu_median_ms(call, 5, warmup=1) / 1e3
    nbytes = spmm_bytes(r, nnz_s, f)
    what = "the whole config-D matrix" if whole else f"rows [0,{r}) of the config-D matrix"
    log(f"cpu baseline ({kind}, {cores} threads): {what}, nnz {nnz_s}: "
        f"{med*1e3:.1f} ms -> {nbytes/med/1e9:.1f} GB/s")
    lib.set_num_threads(1)
    try:
        t0 = time.perf_counter()
        call()
        one = time.perf_counter() - t0
    finally:
        lib.set_num_threads(cores)
    g1 = nbytes / one / 1e9
    log(f"cpu baseline ({kind}, 1 thread): {what}: {one*1e3:.1f} ms -> {g1:.2f} GB/s")
    return dict(value=round(nbytes / med / 1e9, 3), unit="GB/s", cores=cores, kind=kind,
                ms=round(med * 1e3, 2),
                sample=f"spmm over {what} ({nnz_s} nnz) x the whole B (F={f}); one warm-up, "
                       f"median of 5 calls, {med*1e3:.1f} ms each",
                one_thread=dict(value=round(g1, 3), unit="GB/s", cores=1, ms=round(one * 1e3, 1),
                                sample=f"{what}, one call"),
                host=host_info())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--f", type=int, default=128, help="headline feature width")
    ap.add_argument("--f-sweep", type=int, nargs="*", default=[32, 128, 512])
    ap.add_argument("--seed", type=int, default=DEFAULT_SEED)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-sample-nnz", type=int, default=0,
                    help="time the CPU baseline over a row prefix of about this many "
                         "nonzeros (0 = the whole config-D matrix)")
    ap.add_argument("--no-spmm", action="store_true",
                    help="skip the config-D SpMM leg (profiling the forwards or ingestion "
                         "alone); the line then carries no headline value")
    ap.add_argument("--no-forward", action="store_true", help="skip the config-E forwards")
    ap.add_argument("--fwd-steps", type=int, default=10)
    ap.add_argument("--fwd-warmup", type=int, default=2)
    ap.add_argument("--no-ingest", action="store_true", help="skip the CSV ingestion leg")
    ap.add_argument("--no-cora", action="store_true", help="skip the Cora-synth (A/B/C) leg")
    ap.add_argument("--no-cpp-api", action="store_true",
                    help="skip timing the C++ API (tinygnn::spmm, Model::forward) beside the C-ABI")
    ap.add_argument("--cora-steps", type=int, default=20)
    ap.add_argument("--ingest-edges", type=int, default=20_000_000)
    ap.add_argument("--ingest-rows", type=int, default=50_000)
    ap.add_argument("--ingest-steps", type=int, default=5)
    ap.add_argument("--calib-gather", action="store_true",
                    help="also run permutation SpMMs (every B row gathered once; F=32, 16), the "
                         "gather-shaped dispatches for scaling rocprofv3 FETCH_SIZE")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 1 GiB copy kernel (out = x * 1), the reference "
                         "dispatch for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this build runs on one GPU; sharding across GPUs is not implemented)", file=sys.stderr)
        sys.exit(2)

    import torch

    import tinygnn_amd as tg

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    tg.lib.load()
    torch.cuda.set_device(0)

    r = None if args.no_spmm else run_spmm_d(args, torch, tg)
    torch.cuda.empty_cache()
    copy = measure_copy(torch)
    if args.calib_copy:
        xc = torch.ones(1 << 28, device="cuda:0")  # 1 GiB read, 1 GiB written
        yc = torch.empty_like(xc)
        for _ in range(3):
            torch.mul(xc, 1.0, out=yc)
        torch.cuda.synchronize()
        del xc, yc
    if args.calib_gather:
        run_calib_gather(torch, tg)
    fwd = None if args.no_forward else run_forward_e(args, torch, tg)
    torch.cuda.empty_cache()
    cora = None if args.no_cora else run_cora(args, torch, tg)
    ingest = None if args.no_ingest else run_ingest(args, torch, tg)
    if r is None:
        print(json.dumps({"metric": "CSR SpMM GB/s & % HBM peak; forward ms at 233K nodes / "
                                    "114.6M edges", "value": None, "unit": "GB/s",
                          "note": "--no-spmm: the SpMM leg was skipped", "forward": fwd,
                          "cora": cora, "ingest": ingest, "host": host_info()}), flush=True)
        return
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
        # achievable bandwidth of a plain copy on this box, beside the peak
        "hbm_copy": copy,
        "roofline": {"bound": "hbm", "achieved": round(head["kernel_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.f, args.seed),
                     "traffic_source": "profiles/spmm_configD_pmc.md (TCC_EA0_RDREQ "
                                       "32B/64B/128B x size + WRITE_SIZE, checked on a "
                                       "permutation SpMM and a 1 GiB copy)",
                     "kernel": "spmm pass, reference order (agg_long_kernel + agg_chunk_kernel)",
                     "kernel_ms_avg": round(head["kernel_ms_avg"], 4),
                     "bytes_per_launch": head["bytes"]},
        # the default plan: every row one fma chain in nonzero order (the
        # reference's order; the output is bit-identical to the reference)
        "sweep_exact": [{"f": v["f"], "ms": round(v["kernel_ms_avg"], 4),
                         "gbs": round(v["kernel_gbs"], 1),
                         "pct_hbm_peak": round(100 * v["kernel_gbs"] / HBM_PEAK_GBS, 2)}
                        for v in r["results"].values()],
        # TG_PRECISION_FAST plans: rows of more than 1,024 nonzeros summed
        # from per-chunk partials (agg_chunk_kernel + agg_reduce_kernel)
        "sweep_fast": [{"f": v["f"], "ms": round(v["kernel_ms_avg"], 4),
                        "gbs": round(v["kernel_gbs"], 1),
                        "pct_hbm_peak": round(100 * v["kernel_gbs"] / HBM_PEAK_GBS, 2)}
                       for v in r["results_fast"].values()],
        "plan_build_ms": round(r["plan_build_ms"], 3),
        "cpu_baseline": r["cpu"],
        "cpp_api_spmm": r["cpp_api"],
        "csr_build_ms": round(r["csr_build_ms"], 2),
        "forward": fwd,
        "cora": cora,
        "ingest": ingest,
        "host": host_info(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
