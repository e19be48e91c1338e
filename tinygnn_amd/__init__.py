"""tinygnn_amd -- TinyGNN's sparse-inference path on MI355X (gfx950).

The product is the C-ABI library ``_build/libtinygnn_amd.so`` (hand-written
HIP kernels, declared in ``include/tinygnn_amd.h``) and the C++ API over it
(``include/tinygnn/*.hpp``).  This Python module is a thin ctypes front end
used by the tests and the benchmark: it takes torch tensors for device
memory and the current torch stream for ordering, and passes raw pointers
through the C-ABI.  There is no CPU fallback: without the library or a GPU
every call raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

from ._lib import InvalidArgument, NativeLibraryMissing, OutOfRange, TgError, lib  # noqa: F401

ACT_NONE, ACT_RELU = 0, 1
POST_NONE, POST_RELU, POST_ELU = 0, 1, 2
AGG_MEAN, AGG_MAX = 0, 1
GEMM_AUTO, GEMM_INORDER, GEMM_MFMA = 0, 1, 2
EPI_NONE, EPI_RELU, EPI_ELU = 0, 1, 2
SAGE_AUTO, SAGE_CONCAT, SAGE_TRANSFORM_FIRST = 0, 1, 2
FORWARD_REFERENCE, FORWARD_CACHED = 0, 1
PRECISION_FAST, PRECISION_EXACT = 0, 1


def _torch():
    import torch
    return torch


def stream_handle(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def dptr(t, dtype=None) -> int:
    """Device pointer of a CUDA/HIP torch tensor (0 for None): contiguous, or
    a row-major 2-D view with unit column stride (its row stride is passed as
    the leading dimension)."""
    if t is None:
        return 0
    if not t.is_cuda:
        raise ValueError("tinygnn_amd expects device (cuda) tensors")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {t.dtype}")
    if not (t.is_contiguous() or (t.dim() == 2 and t.stride(1) == 1)):
        raise ValueError("tinygnn_amd expects contiguous tensors or row-major 2-D views")
    return int(t.data_ptr())


@dataclass
class DeviceCSR:
    """CSR matrix resident on the device (row = source node)."""
    n_rows: int
    n_cols: int
    row_ptr: "object"   # torch.int32 [n_rows + 1]
    col_ind: "object"   # torch.int32 [nnz]
    val: "object"       # torch.float32 [nnz]

    @property
    def nnz(self) -> int:
        return int(self.col_ind.numel())

    @staticmethod
    def from_numpy(n_rows, n_cols, row_ptr, col_ind, val, device="cuda"):
        torch = _torch()
        return DeviceCSR(n_rows, n_cols,
                         torch.from_numpy(row_ptr).to(device=device, dtype=torch.int32),
                         torch.from_numpy(col_ind).to(device=device, dtype=torch.int32),
                         torch.from_numpy(val).to(device=device, dtype=torch.float32))

    def to_numpy(self):
        return (self.row_ptr.cpu().numpy(), self.col_ind.cpu().numpy(), self.val.cpu().numpy())


class SpmmPlan:
    """Degree-binned row schedule of one CSR structure (tg_spmm_plan_*)."""

    def __init__(self, row_ptr, n_rows: int, nnz_bound: int, max_f: int, chunk_nnz: int = 0,
                 stream=None, precision: int = PRECISION_EXACT):
        h = C.c_void_p()
        lib.check(lib.tg_spmm_plan_create(n_rows, nnz_bound, dptr(row_ptr), max_f, chunk_nnz,
                                          stream_handle(stream), C.byref(h)))
        self.h = h
        self.row_ptr = row_ptr
        self.n_rows = n_rows
        if precision != PRECISION_EXACT:
            self.set_precision(precision)

    def set_precision(self, precision: int) -> None:
        """PRECISION_EXACT: every row one fma chain in nonzero order (the
        reference's order, bit-identical output); PRECISION_FAST: rows longer
        than the chunk summed from per-chunk partials."""
        lib.check(lib.tg_spmm_plan_set_precision(self.h, precision))

    @property
    def handle(self):
        return self.h

    def info(self):
        a, b, c = C.c_int64(), C.c_int64(), C.c_int64()
        lib.check(lib.tg_spmm_plan_info(self.h, C.byref(a), C.byref(b), C.byref(c)))
        return dict(n_chunks=a.value, n_split_rows=b.value, n_partials=c.value)

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            lib.tg_spmm_plan_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _check_spmm_shapes(a: DeviceCSR, b):
    # ops.cpp:219-229
    if a.n_cols != b.shape[0]:
        raise InvalidArgument(1, f"spmm: dimension mismatch — A is ({a.n_rows}×{a.n_cols}, "
                                 f"SparseCSR) but B is ({b.shape[0]}×{b.shape[1]}, Dense). "
                                 f"Required: A.cols() == B.rows() ({a.n_cols} vs {b.shape[0]}).")


def spmm_epilogue(a: DeviceCSR, b, plan: SpmmPlan, bias=None, epilogue: int = EPI_NONE,
                  out=None, stream=None):
    """act(A * B + bias) in one pass (tg_spmm_execute_epilogue): the SpMM of
    GCNLayer::forward with add_bias and the activation fused into its store
    (reference layers.cpp:319-336); bit-identical to spmm, add_bias_, then
    relu_ / elu_."""
    torch = _torch()
    _check_spmm_shapes(a, b)
    f = b.shape[1]
    if out is None:
        out = torch.empty((a.n_rows, f), dtype=torch.float32, device=b.device)
    lib.check(lib.tg_spmm_execute_epilogue(plan.h, a.n_cols, f, dptr(a.row_ptr),
                                           dptr(a.col_ind), dptr(a.val), dptr(b), b.stride(0),
                                           dptr(out), out.stride(0), dptr(bias), epilogue,
                                           stream_handle(stream)))
    return out


def spmm(a: DeviceCSR, b, plan: SpmmPlan | None = None, out=None, stream=None,
         precision: int = PRECISION_EXACT):
    """C = A * B (reference ops.cpp:198-297).  With a plan, the plan's
    precision applies; without one, `precision`: PRECISION_EXACT (the
    default) is the reference's summation order, bit-identical;
    PRECISION_FAST sums rows longer than 1,024 nonzeros from per-chunk
    partials."""
    torch = _torch()
    _check_spmm_shapes(a, b)
    f = b.shape[1]
    if out is None:
        out = torch.empty((a.n_rows, f), dtype=torch.float32, device=b.device)
    s = stream_handle(stream)
    if plan is None:
        lib.check(lib.tg_spmm_ex(a.n_rows, a.n_cols, f, a.nnz, dptr(a.row_ptr), dptr(a.col_ind),
                                 dptr(a.val), dptr(b), b.stride(0), dptr(out), out.stride(0),
                                 precision, s))
    else:
        lib.check(lib.tg_spmm_execute(plan.h, a.n_cols, f, dptr(a.row_ptr), dptr(a.col_ind),
                                      dptr(a.val), dptr(b), b.stride(0), dptr(out),
                                      out.stride(0), s))
    return out


# ---------------------------------------------------------------------------
# Graph preprocessing
# ---------------------------------------------------------------------------
def edge_list_to_csr(src, dst, n_nodes: int, stream=None) -> DeviceCSR:
    """GraphLoader::edge_list_to_csr (graph_loader.cpp:211-281) on the device."""
    torch = _torch()
    dev = src.device
    e = int(src.numel())
    rp = torch.empty(n_nodes + 1, dtype=torch.int32, device=dev)
    ci = torch.empty(max(e, 1), dtype=torch.int32, device=dev)[:e]
    v = torch.empty(max(e, 1), dtype=torch.float32, device=dev)[:e]
    lib.check(lib.tg_edge_list_to_csr(n_nodes, e, dptr(src, torch.int32), dptr(dst, torch.int32),
                                      dptr(rp), ci.data_ptr(), v.data_ptr(), None, 0,
                                      stream_handle(stream)))
    return DeviceCSR(n_nodes, n_nodes, rp, ci, v)


def csr_validate(a: DeviceCSR, stream=None) -> None:
    """The checks of Tensor::sparse_csr (tensor.cpp:46-86); raises InvalidArgument."""
    lib.check(lib.tg_csr_validate(a.n_rows, a.n_cols, a.nnz, dptr(a.row_ptr),
                                  a.col_ind.data_ptr() if a.nnz else None, stream_handle(stream)))


def _require_square(a: DeviceCSR, fn: str):
    if a.n_rows != a.n_cols:
        raise InvalidArgument(1, f"{fn}: A must be square — got ({a.n_rows}×{a.n_cols}).")


def _self_loop_outputs(a: DeviceCSR):
    torch = _torch()
    dev = a.row_ptr.device
    cap = a.nnz + a.n_rows
    return (torch.empty(a.n_rows + 1, dtype=torch.int32, device=dev),
            torch.empty(max(cap, 1), dtype=torch.int32, device=dev),
            torch.empty(max(cap, 1), dtype=torch.float32, device=dev))


def _trim(a: DeviceCSR, rp, ci, v) -> DeviceCSR:
    nnz = int(rp[-1].item()) if a.n_rows else 0
    return DeviceCSR(a.n_rows, a.n_cols, rp, ci[:nnz], v[:nnz])


def add_self_loops(a: DeviceCSR, stream=None) -> DeviceCSR:
    """add_self_loops (layers.cpp:71-144): A + I, bit-identical structure/values."""
    _require_square(a, "add_self_loops")
    rp, ci, v = _self_loop_outputs(a)
    lib.check(lib.tg_add_self_loops(a.n_rows, a.nnz, dptr(a.row_ptr), a.col_ind.data_ptr(),
                                    a.val.data_ptr(), dptr(rp), dptr(ci), dptr(v), None, 0,
                                    stream_handle(stream)))
    return _trim(a, rp, ci, v)


def gcn_norm(a: DeviceCSR, with_degrees: bool = False, stream=None):
    """gcn_norm (layers.cpp:158-208): D^-1/2 (A+I) D^-1/2."""
    torch = _torch()
    _require_square(a, "gcn_norm")
    rp, ci, v = _self_loop_outputs(a)
    deg = torch.empty(max(a.n_rows, 1), dtype=torch.float32, device=rp.device)
    dis = torch.empty_like(deg)
    lib.check(lib.tg_gcn_norm(a.n_rows, a.nnz, dptr(a.row_ptr), a.col_ind.data_ptr(),
                              a.val.data_ptr(), dptr(rp), dptr(ci), dptr(v), dptr(deg), dptr(dis),
                              None, 0, stream_handle(stream)))
    out = _trim(a, rp, ci, v)
    return (out, deg[:a.n_rows], dis[:a.n_rows]) if with_degrees else out


def edge_softmax(a: DeviceCSR, stream=None) -> DeviceCSR:
    """edge_softmax (layers.cpp:768-822)."""
    torch = _torch()
    v = torch.zeros_like(a.val)
    lib.check(lib.tg_edge_softmax(a.n_rows, dptr(a.row_ptr), a.val.data_ptr(), v.data_ptr(),
                                  stream_handle(stream)))
    return DeviceCSR(a.n_rows, a.n_cols, a.row_ptr, a.col_ind, v)


# ---------------------------------------------------------------------------
# Dense ops
# ---------------------------------------------------------------------------
def matmul(a, b, bias=None, epilogue: int = EPI_NONE, algo: int = GEMM_AUTO, out=None,
           stream=None):
    """matmul (ops.cpp:70-162) with an optional fused bias + activation."""
    torch = _torch()
    if a.shape[1] != b.shape[0]:
        # ops.cpp:90-97, the reference's text
        raise InvalidArgument(1, f"matmul: dimension mismatch — A is ({a.shape[0]}×{a.shape[1]})"
                                 f" but B is ({b.shape[0]}×{b.shape[1]}). Required: A.cols() == "
                                 f"B.rows() (both = {a.shape[1]} vs {b.shape[0]}).")
    m, k = a.shape
    n = b.shape[1]
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    lib.check(lib.tg_matmul(m, k, n, dptr(a), a.stride(0), dptr(b), b.stride(0), dptr(out),
                            out.stride(0), dptr(bias), epilogue, algo, stream_handle(stream)))
    return out


def _unary(name, x, *extra, stream=None):
    lib.check(getattr(lib, name)(x.numel(), dptr(x), *extra, stream_handle(stream)))
    return x


def relu_(x, stream=None):
    return _unary("tg_relu", x, stream=stream)


def leaky_relu_(x, alpha: float = 0.01, stream=None):
    return _unary("tg_leaky_relu", x, alpha, stream=stream)


def elu_(x, alpha: float = 1.0, stream=None):
    return _unary("tg_elu", x, alpha, stream=stream)


def sigmoid_(x, stream=None):
    return _unary("tg_sigmoid", x, stream=stream)


def tanh_(x, stream=None):
    return _unary("tg_tanh", x, stream=stream)


def gelu_(x, stream=None):
    return _unary("tg_gelu", x, stream=stream)


def softmax_(x, stream=None):
    lib.check(lib.tg_softmax(x.shape[0], x.shape[1], dptr(x), stream_handle(stream)))
    return x


def log_softmax_(x, stream=None):
    lib.check(lib.tg_log_softmax(x.shape[0], x.shape[1], dptr(x), stream_handle(stream)))
    return x


def add_bias_(x, bias, stream=None):
    n = x.shape[1]
    if bias.dim() != 2 or bias.shape[0] != 1 or bias.shape[1] != n:
        shp = tuple(bias.shape) if bias.dim() == 2 else (1, bias.numel())
        raise InvalidArgument(1, f"add_bias: bias must be shape (1×{n}) to match X columns, "
                                 f"but got ({shp[0]}×{shp[1]}).")
    lib.check(lib.tg_add_bias(x.shape[0], n, dptr(x), dptr(bias), stream_handle(stream)))
    return x


# ---------------------------------------------------------------------------
# Layers
# ---------------------------------------------------------------------------
def sage_aggregate(plan: SpmmPlan, a: DeviceCSR, h, agg: int = AGG_MEAN, stream=None):
    torch = _torch()
    out = torch.empty((a.n_rows, h.shape[1]), dtype=torch.float32, device=h.device)
    lib.check(lib.tg_sage_aggregate(plan.h, a.n_rows, h.shape[1], agg, dptr(a.row_ptr),
                                    a.col_ind.data_ptr(), dptr(h), h.stride(0), dptr(out),
                                    out.stride(0), stream_handle(stream)))
    return out


def sage_forward(plan: SpmmPlan, a: DeviceCSR, h, w_neigh, w_self, bias=None,
                 act: int = ACT_RELU, post: int = POST_NONE, agg: int = AGG_MEAN,
                 dataflow: int = SAGE_AUTO, stream=None):
    """SAGELayer::forward (layers.cpp:538-752)."""
    torch = _torch()
    f_in, f_out = w_neigh.shape
    out = torch.empty((a.n_rows, f_out), dtype=torch.float32, device=h.device)
    lib.check(lib.tg_sage_forward(plan.h, a.n_rows, f_in, f_out, agg, dptr(a.row_ptr),
                                  a.col_ind.data_ptr(), dptr(h), dptr(w_neigh), dptr(w_self),
                                  dptr(bias), act, post, dataflow, dptr(out), None, 0,
                                  stream_handle(stream)))
    return out


def gat_scores(wh, heads: int, f: int, att_l, att_r, stream=None):
    torch = _torch()
    n = wh.shape[0]
    src = torch.empty((n, heads), dtype=torch.float32, device=wh.device)
    dst = torch.empty_like(src)
    lib.check(lib.tg_gat_scores(n, heads, f, dptr(wh), wh.stride(0), dptr(att_l), dptr(att_r),
                                dptr(src), dptr(dst), stream_handle(stream)))
    return src, dst


def gat_aggregate(plan: SpmmPlan, a_sl: DeviceCSR, wh, heads: int, f: int, src, dst,
                  slope: float = 0.2, bias=None, act: int = ACT_NONE, post: int = POST_NONE,
                  concat: bool = True, stream=None):
    """All heads of GATLayer::forward's fused edge pass (layers.cpp:1052-1112)."""
    torch = _torch()
    cols = heads * f if (concat or heads == 1) else f
    out = torch.empty((a_sl.n_rows, cols), dtype=torch.float32, device=wh.device)
    lib.check(lib.tg_gat_aggregate(plan.h, a_sl.n_rows, heads, f, dptr(a_sl.row_ptr),
                                   a_sl.col_ind.data_ptr(), dptr(wh), wh.stride(0), dptr(src),
                                   dptr(dst), slope, dptr(bias), act, post, int(concat),
                                   dptr(out), out.stride(0), None, 0, stream_handle(stream)))
    return out


# ---------------------------------------------------------------------------
# Model
# ---------------------------------------------------------------------------
class Model:
    """tinygnn::Model (model.hpp:89-164) on the device, over tg_model_*."""

    def __init__(self):
        h = C.c_void_p()
        lib.check(lib.tg_model_create(C.byref(h)))
        self.h = h

    def add_gcn_layer(self, in_f, out_f, bias=True, act=ACT_RELU, post=POST_NONE) -> int:
        i = C.c_int64()
        lib.check(lib.tg_model_add_gcn_layer(self.h, in_f, out_f, int(bias), act, post,
                                             C.byref(i)))
        return i.value

    def add_sage_layer(self, in_f, out_f, agg=AGG_MEAN, bias=True, act=ACT_RELU,
                       post=POST_NONE) -> int:
        i = C.c_int64()
        lib.check(lib.tg_model_add_sage_layer(self.h, in_f, out_f, agg, int(bias), act, post,
                                              C.byref(i)))
        return i.value

    def add_gat_layer(self, in_f, out_f, num_heads=1, concat=True, neg_slope=0.2, bias=True,
                      act=ACT_NONE, post=POST_NONE) -> int:
        i = C.c_int64()
        lib.check(lib.tg_model_add_gat_layer(self.h, in_f, out_f, num_heads, int(concat),
                                             neg_slope, int(bias), act, post, C.byref(i)))
        return i.value

    def num_layers(self) -> int:
        n = C.c_int64()
        lib.check(lib.tg_model_num_layers(self.h, C.byref(n)))
        return n.value

    def output_cols(self) -> int:
        n = C.c_int64()
        lib.check(lib.tg_model_output_cols(self.h, C.byref(n)))
        return n.value

    def set_tensor(self, name: str, array) -> None:
        import numpy as np
        a = np.ascontiguousarray(array, dtype=np.float32)
        if a.ndim == 1:
            a = a.reshape(1, -1)
        lib.check(lib.tg_model_set_tensor(self.h, name.encode(), a.shape[0], a.shape[1],
                                          a.ctypes.data_as(C.c_void_p)))

    def load_weights(self, weights=None) -> None:
        """Model::load_weights (model.cpp:252-305).  ``weights`` is a dict of
        name -> array, a :class:`WeightFile`, or the path of a TGNN weight
        file (model.cpp:252-255).  Only the given tensors are looked up, as
        the reference looks up only the WeightFile it is given."""
        if isinstance(weights, (str, bytes)) or hasattr(weights, "__fspath__"):
            weights = load_weight_file(weights)
        if isinstance(weights, WeightFile):
            weights = weights.tensors
        lib.check(lib.tg_model_clear_tensors(self.h))
        for k, v in (weights or {}).items():
            self.set_tensor(k, v)
        lib.check(lib.tg_model_load_weights(self.h))

    def set_sage_dataflow(self, dataflow: int) -> None:
        lib.check(lib.tg_model_set_sage_dataflow(self.h, dataflow))

    def set_precision(self, precision: int) -> None:
        """PRECISION_FAST (default) or PRECISION_EXACT (the reference's
        operation order: bit-identical GCN / SAGE outputs)."""
        lib.check(lib.tg_model_set_precision(self.h, precision))

    def set_blocking(self, rows_per_block: int = -1) -> None:
        """Column blocking of the GCN / SAGE-mean / GAT aggregations (both
        forward modes; exact precision: only for rows in column order, keeping
        the reference's summation order): rows_per_block source nodes per
        block, 0 = off, -1 = the default (equal blocks of at most 23552 rows
        for weighted passes over A + I -- GAT, exact or weighted GCN -- and
        38912 for passes without values -- SAGE's mean over A, fast GCN over a
        unit-valued A + I -- on graphs dense enough to pay)."""
        lib.check(lib.tg_model_set_blocking(self.h, rows_per_block))

    def blocking_info(self) -> dict:
        """The column blocking the last forward used (tg_model_blocking_info):
        blocks and lane-group columns of A + I's and A's blocked copies,
        whether A + I's was split from A directly (sl_direct), and whether
        each copy is prepared for the output-resident passes (resident_sl,
        resident_raw)."""
        v = [C.c_int64() for _ in range(6)]
        lib.check(lib.tg_model_blocking_info(self.h, *[C.byref(x) for x in v]))
        return dict(blocks_sl=v[0].value, cols_sl=v[1].value, blocks_raw=v[2].value,
                    cols_raw=v[3].value, sl_direct=bool(v[4].value),
                    resident_sl=bool(v[5].value & 1), resident_raw=bool(v[5].value & 2))

    def set_self_loop_split(self, direct: bool = True) -> None:
        """Whether a fast GCN-only model splits its blocked A + I from A
        directly when A allows it (tg_model_set_self_loop_split; the same
        outputs bit for bit either way).  Drops the cached state."""
        self._adj_key = None
        lib.check(lib.tg_model_set_self_loop_split(self.h, 1 if direct else 0))

    def set_resident_passes(self, on: bool = True) -> None:
        """Whether the fast blocked aggregations without values (SAGE mean,
        the factored GCN) run as output-resident passes, one launch with the
        output tile in LDS, or one pass per column block
        (tg_model_set_resident_passes).  Drops the cached state."""
        self._adj_key = None
        lib.check(lib.tg_model_set_resident_passes(self.h, 1 if on else 0))

    def invalidate(self) -> None:
        """Forgets the cached adjacency state (tg_model_invalidate)."""
        self._adj_key = None
        lib.check(lib.tg_model_invalidate(self.h))

    @staticmethod
    def _adjacency_key(adj: DeviceCSR):
        return (adj.n_rows, adj.row_ptr, adj.col_ind, adj.val, adj.row_ptr._version,
                adj.col_ind._version, adj.val._version)

    def _cache_valid(self, key) -> bool:
        old = getattr(self, "_adj_key", None)
        if old is None:
            return False
        return (old[0] == key[0] and all(a is b for a, b in zip(old[1:4], key[1:4]))
                and old[4:] == key[4:])

    def forward(self, adj: DeviceCSR, x, mode: int = FORWARD_REFERENCE, out=None, stream=None):
        """Model::forward (model.cpp:359-439).

        ``mode=FORWARD_REFERENCE`` (the default) recomputes gcn_norm /
        add_self_loops and the row plans on every call, as the reference
        does (model.cpp:373-381).  ``mode=FORWARD_CACHED`` reuses them when
        ``adj`` holds the same ``row_ptr`` / ``col_ind`` / ``val`` tensor
        objects as the previous forward, at the same torch versions (an
        in-place edit through torch bumps the version; a new tensor is a
        different object).  The model keeps references to those three
        tensors, so their memory cannot be handed to another graph while the
        cache refers to it.  Writes that torch does not track (through raw
        device pointers) must be followed by :meth:`invalidate`."""
        torch = _torch()
        if out is None:
            out = torch.empty((adj.n_rows, self.output_cols()), dtype=torch.float32,
                              device=x.device)
        key = self._adjacency_key(adj)
        if mode == FORWARD_CACHED and not self._cache_valid(key):
            lib.check(lib.tg_model_invalidate(self.h))
        self._adj_key = None
        lib.check(lib.tg_model_forward(self.h, adj.n_rows, adj.nnz, dptr(adj.row_ptr),
                                       adj.col_ind.data_ptr(), adj.val.data_ptr(), x.shape[1],
                                       dptr(x), dptr(out), mode, stream_handle(stream)))
        self._adj_key = key
        return out

    @staticmethod
    def from_spec(spec, weights: dict | None = None) -> "Model":
        """Builds a model from layer dicts (see tinygnn_amd.synth.spec_*)."""
        m = Model()
        for l in spec:
            t = l["type"]
            if t == "gcn":
                m.add_gcn_layer(l["in"], l["out"], l.get("bias", True), l.get("act", ACT_RELU),
                                l.get("post", POST_NONE))
            elif t == "sage":
                m.add_sage_layer(l["in"], l["out"], l.get("agg", AGG_MEAN), l.get("bias", True),
                                 l.get("act", ACT_RELU), l.get("post", POST_NONE))
            elif t == "gat":
                m.add_gat_layer(l["in"], l["out"], l.get("heads", 1), l.get("concat", True),
                                l.get("slope", 0.2), l.get("bias", True), l.get("act", ACT_NONE),
                                l.get("post", POST_NONE))
            else:
                raise ValueError(t)
        if weights is not None:
            m.load_weights(weights)
        return m

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            lib.tg_model_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# Ingestion: CSV graphs (GraphLoader, graph_loader.cpp:61-326), the TGNN
# weight file (model.cpp:134-185) and the Cora binary (model.cpp:49-129).
# ---------------------------------------------------------------------------
class CsvText:
    """A CSV text indexed into lines on the device (tg_csv_open / tg_csv_index).

    ``CsvText.open(path)`` reads the file into device memory;
    ``CsvText.from_device(u8_tensor, name)`` indexes bytes already there (the
    tensor is kept alive with the handle)."""

    def __init__(self, handle, keep=None):
        self.h = handle
        self._keep = keep
        n, hdr = C.c_int64(), C.c_int()
        lib.check(lib.tg_csv_info(self.h, C.byref(n), C.byref(hdr)))
        self.n_lines, self.has_header = int(n.value), bool(hdr.value)

    @classmethod
    def open(cls, path, stream=None) -> "CsvText":
        h = C.c_void_p()
        lib.check(lib.tg_csv_open(os.fsencode(path), C.byref(h), stream_handle(stream)))
        return cls(h)

    @classmethod
    def from_device(cls, text, name: str = "", stream=None) -> "CsvText":
        torch = _torch()
        if text.dtype != torch.uint8 or not text.is_contiguous():
            raise ValueError("CsvText.from_device expects a contiguous uint8 device tensor")
        h = C.c_void_p()
        lib.check(lib.tg_csv_index(dptr(text), text.numel(), name.encode(), C.byref(h),
                                   stream_handle(stream)))
        return cls(h, keep=text)

    @property
    def n_data(self) -> int:
        return self.n_lines - int(self.has_header)

    def parse_edges(self, device=None, stream=None):
        """GraphLoader::parse_edges (graph_loader.cpp:61-107): (src, dst,
        max_id) with int32 device tensors of one entry per data line."""
        torch = _torch()
        device = device or torch.device("cuda", torch.cuda.current_device())
        n = max(self.n_data, 0)
        src = torch.empty(max(n, 1), dtype=torch.int32, device=device)[:n]
        dst = torch.empty(max(n, 1), dtype=torch.int32, device=device)[:n]
        mx = C.c_int64()
        lib.check(lib.tg_csv_parse_edges(self.h, src.data_ptr(), dst.data_ptr(), C.byref(mx),
                                         stream_handle(stream)))
        return src, dst, int(mx.value)

    def feature_shape(self, stream=None):
        rows, cols = C.c_int64(), C.c_int64()
        lib.check(lib.tg_csv_feature_shape(self.h, C.byref(rows), C.byref(cols),
                                           stream_handle(stream)))
        return int(rows.value), int(cols.value)

    def parse_features(self, n_rows: int | None = None, device=None, stream=None):
        """GraphLoader::parse_features (graph_loader.cpp:112-206): a
        [rows x cols] float32 device tensor (``n_rows`` > rows zero-pads)."""
        torch = _torch()
        device = device or torch.device("cuda", torch.cuda.current_device())
        rows, cols = self.feature_shape(stream)
        n_rows = rows if n_rows is None else int(n_rows)
        out = torch.empty((n_rows, cols), dtype=torch.float32, device=device)
        lib.check(lib.tg_csv_parse_features(self.h, out.data_ptr() if out.numel() else None,
                                            n_rows, cols, stream_handle(stream)))
        return out

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            lib.tg_csv_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def parse_edges(path, stream=None):
    """GraphLoader::parse_edges on the device: (src, dst) int32 tensors."""
    t = CsvText.open(path, stream)
    try:
        src, dst, _ = t.parse_edges(stream=stream)
        return src, dst
    finally:
        t.close()


def parse_features(path, stream=None):
    """GraphLoader::parse_features on the device: [rows x cols] float32."""
    t = CsvText.open(path, stream)
    try:
        return t.parse_features(stream=stream)
    finally:
        t.close()


@dataclass
class GraphData:
    """GraphData (graph_loader.hpp:17-23): adjacency (values 1.0) and
    features, both on the device."""
    adjacency: DeviceCSR
    node_features: object
    num_nodes: int
    num_edges: int
    num_features: int


def load_graph(edges_path, features_path, stream=None) -> GraphData:
    """GraphLoader::load (graph_loader.cpp:286-326): edges, then features,
    num_nodes = max(largest endpoint + 1, feature rows), the CSR built on the
    device and the features zero-padded to num_nodes rows."""
    te = CsvText.open(edges_path, stream)
    try:
        src, dst, max_id = te.parse_edges(stream=stream)
    finally:
        te.close()
    tf = CsvText.open(features_path, stream)
    try:
        rows, cols = tf.feature_shape(stream)
        n_edges = int(src.numel())
        num_nodes = max(max_id + 1 if n_edges else 0, rows)
        x = tf.parse_features(n_rows=num_nodes, stream=stream)
    finally:
        tf.close()
    adj = edge_list_to_csr(src, dst, num_nodes, stream=stream)
    return GraphData(adj, x, num_nodes, n_edges, cols)


@dataclass
class WeightFile:
    """WeightFile (model.hpp:76-79): test accuracy and named host tensors."""
    test_accuracy: float
    tensors: dict


def load_weight_file(path) -> WeightFile:
    """load_weight_file (model.cpp:134-185), read by the native library."""
    import numpy as np
    h = C.c_void_p()
    lib.check(lib.tg_weights_open(os.fsencode(path), C.byref(h)))
    try:
        n, acc = C.c_int64(), C.c_float()
        lib.check(lib.tg_weights_info(h, C.byref(n), C.byref(acc)))
        tensors = {}
        for i in range(n.value):
            name, nlen, rows, cols, data = (C.c_void_p(), C.c_int64(), C.c_int64(), C.c_int64(),
                                            C.c_void_p())
            lib.check(lib.tg_weights_tensor(h, i, C.byref(name), C.byref(nlen), C.byref(rows),
                                            C.byref(cols), C.byref(data)))
            key = C.string_at(name.value, nlen.value).decode("utf-8", "surrogateescape")
            count = rows.value * cols.value
            arr = np.empty((rows.value, cols.value), np.float32)
            if count:
                C.memmove(arr.ctypes.data, data.value, count * 4)
            tensors[key] = arr
        return WeightFile(float(acc.value), tensors)
    finally:
        lib.tg_weights_destroy(h)


def save_weight_file(path, tensors: dict, test_accuracy: float = 0.0) -> None:
    """Writes a TGNN weight file, version 1 (model.hpp:22-33): the format
    load_weight_file reads.  Tensors are 2-D float32 (1-D arrays are written
    as one row), in the dict's order."""
    import struct
    import numpy as np
    with open(path, "wb") as f:
        f.write(b"TGNN")
        f.write(struct.pack("<IfI", 1, float(test_accuracy), len(tensors)))
        for name, arr in tensors.items():
            a = np.ascontiguousarray(arr, dtype="<f4")
            if a.ndim == 1:
                a = a.reshape(1, -1)
            if a.ndim != 2:
                raise ValueError(f"{name}: expected a 1-D or 2-D array")
            nb = name.encode("utf-8", "surrogateescape")
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<II", *a.shape))
            f.write(a.tobytes())


@dataclass
class CoraData:
    """CoraData (model.hpp:50-62): the graph on the device, labels and masks
    on the host."""
    num_nodes: int
    num_features: int
    num_classes: int
    num_edges: int
    adjacency: DeviceCSR
    features: object
    labels: object
    train_mask: object
    val_mask: object
    test_mask: object


def load_cora_binary(path, stream=None) -> CoraData:
    """load_cora_binary (model.cpp:49-129): the file read by the native
    library, features uploaded, adjacency built on the device."""
    import numpy as np
    torch = _torch()
    dev = torch.device("cuda", torch.cuda.current_device())
    h = C.c_void_p()
    lib.check(lib.tg_cora_open(os.fsencode(path), C.byref(h)))
    try:
        n, f, c, e = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int64()
        lib.check(lib.tg_cora_info(h, C.byref(n), C.byref(f), C.byref(c), C.byref(e)))
        n, f, c, e = n.value, f.value, c.value, e.value
        x = torch.empty((n, f), dtype=torch.float32, device=dev)
        rp = torch.empty(n + 1, dtype=torch.int32, device=dev)
        ci = torch.empty(max(e, 1), dtype=torch.int32, device=dev)[:e]
        v = torch.empty(max(e, 1), dtype=torch.float32, device=dev)[:e]
        lib.check(lib.tg_cora_upload(h, x.data_ptr() if x.numel() else None, rp.data_ptr(),
                                     ci.data_ptr(), v.data_ptr(), stream_handle(stream)))
        ptrs = [C.c_void_p() for _ in range(4)]
        lib.check(lib.tg_cora_host(h, *[C.byref(p) for p in ptrs]))
        labels = np.empty(n, np.int32)
        masks = [np.empty(n, np.uint8) for _ in range(3)]
        if n:
            C.memmove(labels.ctypes.data, ptrs[0].value, n * 4)
            for m, p in zip(masks, ptrs[1:]):
                C.memmove(m.ctypes.data, p.value, n)
        return CoraData(n, f, c, e, DeviceCSR(n, n, rp, ci, v), x, labels, *masks)
    finally:
        lib.tg_cora_destroy(h)
