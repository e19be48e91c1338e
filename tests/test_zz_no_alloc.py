"""tg_spmm_noalloc, the SpMM entry point that allocates nothing, against the
entry point it varies, tg_spmm (reference spmm, src/ops.cpp:198-297), both
called through the C-ABI.

Two calls in a row, the second on a smaller input, so that the second runs
over the scratch the first left behind: each output must equal tg_spmm's
bit for bit (the same plan and kernels) and the oracle's, every row
included (both sum each row as one chain in the reference's order).
Outputs start as NaN, so an element left unwritten fails.  Also: the call
captured into HIP graphs and replayed, a first call under capture refused,
the device array held only by processes that call the entry, and the NaN
fill for a row_ptr whose last entry exceeds nnz.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import bits, random_csr

pytestmark = pytest.mark.gpu


def _spmm(gpu, fn, a, b):
    """One call of tg_spmm / tg_spmm_noalloc on fresh device copies."""
    from tinygnn_amd import _lib
    import tinygnn_amd as tg
    L = _lib.lib.load()
    rp = gpu.from_numpy(a.row_ptr).cuda()
    ci = gpu.from_numpy(a.col_ind).cuda()
    v = gpu.from_numpy(a.val).cuda()
    db = gpu.from_numpy(b).cuda()
    c = gpu.full((a.n_rows, b.shape[1]), float("nan"), device="cuda:0")
    rc = getattr(L, fn)(a.n_rows, a.n_cols, b.shape[1], a.nnz, rp.data_ptr(), ci.data_ptr(),
                        v.data_ptr(), db.data_ptr(), b.shape[1], c.data_ptr(), b.shape[1],
                        C.c_void_p(tg.stream_handle()))
    assert rc == 0, L.tg_last_error().decode()
    gpu.cuda.synchronize()
    return c.cpu().numpy()


def _check_oracle(restate, a, b, got):
    """Every row bit-identical to the oracle's chain; returns the number of
    rows longer than the plan's 1,024-entry chunk (the workgroup-per-row
    path)."""
    np.testing.assert_array_equal(bits(got), bits(restate.spmm(a, b)))
    return int((np.diff(a.row_ptr) > 1024).sum())


def test_spmm_noalloc_two_calls(gpu, restate):
    rng = np.random.default_rng(77)
    big = random_csr(rng, 30_000, 26_000, avg_deg=40, max_deg=6000, empty_frac=0.05)
    b_big = rng.standard_normal((26_000, 72)).astype(np.float32)
    small = random_csr(rng, 4_000, 5_000, avg_deg=9, max_deg=2500, empty_frac=0.2)
    b_small = rng.standard_normal((5_000, 24)).astype(np.float32)
    n_split = []
    for a, b in ((big, b_big), (small, b_small)):
        got = _spmm(gpu, "tg_spmm_noalloc", a, b)
        ref = _spmm(gpu, "tg_spmm", a, b)
        assert np.isfinite(got).all()
        np.testing.assert_array_equal(bits(got), bits(ref))
        n_split.append(_check_oracle(restate, a, b, got))
    assert n_split[0] > 0 and n_split[1] > 0  # both calls have rows longer than a chunk


def test_spmm_noalloc_edges(gpu, restate):
    """No nonzeros (a zero result), a single row longer than several chunks,
    and a width that is not a multiple of 4."""
    import oracle
    z = oracle.CSR(7, 5, np.zeros(8, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    got = _spmm(gpu, "tg_spmm_noalloc", z, np.ones((5, 3), np.float32))
    assert got.shape == (7, 3) and not got.any()
    rng = np.random.default_rng(5)
    n = 5000
    ci = np.sort(rng.integers(0, n, 4500)).astype(np.int32)
    rp = np.zeros(3, np.int32)
    rp[1:] = [4500, 4500]
    a = oracle.CSR(2, n, rp, ci, rng.random(4500).astype(np.float32))
    b = rng.standard_normal((n, 41)).astype(np.float32)
    got = _spmm(gpu, "tg_spmm_noalloc", a, b)
    np.testing.assert_array_equal(bits(got), bits(_spmm(gpu, "tg_spmm", a, b)))
    assert _check_oracle(restate, a, b, got) == 1


def _device_args(gpu, a, b):
    rp = gpu.from_numpy(a.row_ptr).cuda()
    ci = gpu.from_numpy(a.col_ind).cuda()
    v = gpu.from_numpy(a.val).cuda()
    db = gpu.from_numpy(b).cuda()
    c = gpu.full((a.n_rows, b.shape[1]), float("nan"), device="cuda:0")
    return rp, ci, v, db, c


def test_spmm_noalloc_nan_on_inconsistent_row_ptr(gpu):
    """row_ptr[m] larger than the nnz passed: where that overflows the plan's
    capacities (here a row longer than a chunk while nnz admits none), the
    call still returns TG_OK and fills C with NaN, so the misuse shows."""
    import oracle
    import tinygnn_amd as tg
    from tinygnn_amd import _lib
    L = _lib.lib.load()
    rng = np.random.default_rng(9)
    n = 3000
    ci = np.sort(rng.integers(0, n, 2500)).astype(np.int32)
    a = oracle.CSR(4, n, np.array([0, 0, 2500, 2500, 2500], np.int32), ci,
                   rng.random(2500).astype(np.float32))
    b = rng.standard_normal((n, 8)).astype(np.float32)
    rp, ci_d, v, db, c = _device_args(gpu, a, b)
    c.zero_()
    rc = L.tg_spmm_noalloc(4, n, 8, 10, rp.data_ptr(), ci_d.data_ptr(), v.data_ptr(),
                           db.data_ptr(), 8, c.data_ptr(), 8, C.c_void_p(tg.stream_handle()))
    assert rc == 0, L.tg_last_error().decode()
    gpu.cuda.synchronize()
    assert np.isnan(c.cpu().numpy()).all()


def test_spmm_noalloc_graph_capture(gpu):
    """A call made once outside capture, then captured on a side stream into
    a HIP graph -- one graph per input, a large and a smaller one, sharing the
    device array -- and each graph replayed twice in alternation, with eager
    work and synchronisations between replays: every replay equals tg_spmm
    bit for bit."""
    import tinygnn_amd as tg
    from tinygnn_amd import _lib
    L = _lib.lib.load()
    rng = np.random.default_rng(31)
    cases = [(random_csr(rng, 20_000, 20_000, avg_deg=30, max_deg=5000, empty_frac=0.05), 64),
             (random_csr(rng, 3_000, 4_000, avg_deg=8, max_deg=2000, empty_frac=0.2), 20)]
    side = gpu.cuda.Stream()
    graphs = []
    for a, f in cases:
        b = rng.standard_normal((a.n_cols, f)).astype(np.float32)
        args = _device_args(gpu, a, b)
        rp, ci, v, db, c = args

        def call(stream, a=a, f=f, args=args):
            rp, ci, v, db, c = args
            return L.tg_spmm_noalloc(a.n_rows, a.n_cols, f, a.nnz, rp.data_ptr(), ci.data_ptr(),
                                     v.data_ptr(), db.data_ptr(), f, c.data_ptr(), f,
                                     C.c_void_p(stream.cuda_stream))

        with gpu.cuda.stream(side):
            assert call(side) == 0, L.tg_last_error().decode()  # outside capture
        gpu.cuda.synchronize()
        want = _spmm(gpu, "tg_spmm", a, b)
        np.testing.assert_array_equal(bits(c.cpu().numpy()), bits(want))
        g = gpu.cuda.CUDAGraph()
        with gpu.cuda.graph(g, stream=side):
            rc = call(side)
        assert rc == 0, L.tg_last_error().decode()
        # the graph holds the inputs' addresses: keep them alive
        graphs.append((g, c, want, args))
    for _ in range(2):
        for g, c, want, _args in graphs:
            c.fill_(float("nan"))
            gpu.cuda.synchronize()
            g.replay()
            gpu.cuda.synchronize()
            np.testing.assert_array_equal(bits(c.cpu().numpy()), bits(want))
            # eager work between replays
            x = gpu.randn(1 << 20, device="cuda:0")
            float((x * x).sum())


FRESH_PROCESS = r"""
import ctypes as C, sys
import numpy as np, torch
sys.path.insert(0, sys.argv[1])
import tinygnn_amd as tg
from tinygnn_amd import _lib
L = _lib.lib.load()
torch.cuda.init()
n, f = 2000, 16
rng = np.random.default_rng(1)
rp = torch.arange(0, 10 * (n + 1), 10, dtype=torch.int32, device="cuda")
ci = torch.from_numpy(rng.integers(0, n, 10 * n).astype(np.int32)).cuda()
v = torch.ones(10 * n, device="cuda")
b = torch.randn(n, f, device="cuda")
c = torch.empty(n, f, device="cuda")
args = (n, n, f, 10 * n, rp.data_ptr(), ci.data_ptr(), v.data_ptr(), b.data_ptr(), f,
        c.data_ptr(), f)
s = torch.cuda.Stream()
assert L.tg_spmm(*args, C.c_void_p(s.cuda_stream)) == 0
torch.cuda.synchronize()
free0 = torch.cuda.mem_get_info()[0]
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    rc = L.tg_spmm_noalloc(*args, C.c_void_p(s.cuda_stream))
    msg = L.tg_last_error().decode()
torch.cuda.synchronize()
free1 = torch.cuda.mem_get_info()[0]
assert L.tg_spmm_noalloc(*args, C.c_void_p(s.cuda_stream)) == 0
torch.cuda.synchronize()
free2 = torch.cuda.mem_get_info()[0]
print(rc, free0, free1, free2)
print(msg)
"""


def test_spmm_noalloc_fresh_process(gpu):
    """In a process that has not called it: the first call under stream
    capture is refused (TG_ERR_INVALID_ARGUMENT, the device array's address
    must be resolved outside capture), the array is not held before the first
    call (tg_spmm, in the same library, does not load it), and the first call
    outside capture makes the GPU hold it."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", FRESH_PROCESS, root], capture_output=True,
                       text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.strip().splitlines()
    rc, free0, free1, free2 = (int(x) for x in lines[-2].split())
    assert rc == 1, lines  # TG_ERR_INVALID_ARGUMENT
    assert "outside stream capture" in lines[-1]
    mib = 1 << 20
    assert abs(free0 - free1) < 16 * mib, (free0, free1)
    assert free1 - free2 >= 120 * mib, (free1, free2)
