"""CPU oracle for TinyGNN's sparse-inference path -- TEST INFRASTRUCTURE ONLY.

Two ctypes-loaded libraries, both built by ``oracle/Makefile``:

* ``restate`` -- ``_build/libtgoracle.so``: the C restatement
  (``tg_oracle.c``), each function citing the reference file:line it follows.
* ``reference`` -- ``_ref/libtgref.so``: the real reference compiled from its
  own sources plus ``ref_shim.cpp``.  Present only where it was built (it is
  built in the development container and shipped prebuilt).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg import this package, and only as the checker or as the
timed CPU baseline.  The product library (``tinygnn_amd``) never imports it.

All arrays are numpy, C-contiguous; dense matrices are float32 row-major and
CSR matrices are ``(row_ptr int32[n+1], col_ind int32[nnz], val float32[nnz])``.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
RESTATE_SO = os.path.join(HERE, "_build", "libtgoracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtgref.so")

_i64 = C.c_int64
_i32 = C.c_int
_f32 = C.c_float
_p = C.c_void_p


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(_p)


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


class OracleError(Exception):
    """The reference would have thrown; ``kind`` names its exception type."""

    def __init__(self, kind: str, message: str):
        super().__init__(message)
        self.kind = kind


@dataclass
class CSR:
    n_rows: int
    n_cols: int
    row_ptr: np.ndarray
    col_ind: np.ndarray
    val: np.ndarray

    @property
    def nnz(self) -> int:
        return int(self.col_ind.shape[0])


# ---------------------------------------------------------------------------
# The C restatement
# ---------------------------------------------------------------------------
class _Restate:
    def __init__(self, path: str = RESTATE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: run `make -C oracle` (or __graft_entry__.build())")
        L = C.CDLL(path)
        self.L = L
        sig = {
            "or_last_error": (C.c_char_p, []),
            "or_set_num_threads": (None, [_i32]),
            "or_get_num_threads": (_i32, []),
            "or_edge_list_to_csr": (_i32, [_i64, _i64, _p, _p, _p, _p, _p]),
            "or_add_self_loops_nnz": (_i64, [_i64, _p, _p]),
            "or_add_self_loops": (None, [_i64, _p, _p, _p, _p, _p, _p]),
            "or_gcn_norm": (None, [_i64, _p, _p, _p, _p, _p, _p, _p, _p]),
            "or_spmm": (None, [_i64, _i64, _p, _p, _p, _p, _p]),
            "or_spmm_rows_f64": (None, [_i64, _p, _i64, _p, _p, _p, _p, _p, _p]),
            "or_matmul": (None, [_i64, _i64, _i64, _p, _p, _p]),
            "or_relu": (None, [_i64, _p]),
            "or_leaky_relu": (None, [_i64, _p, _f32]),
            "or_elu": (None, [_i64, _p, _f32]),
            "or_sigmoid": (None, [_i64, _p]),
            "or_tanh": (None, [_i64, _p]),
            "or_gelu": (None, [_i64, _p]),
            "or_softmax": (None, [_i64, _i64, _p]),
            "or_log_softmax": (None, [_i64, _i64, _p]),
            "or_add_bias": (None, [_i64, _i64, _p, _p]),
            "or_edge_softmax": (None, [_i64, _p, _p, _p]),
            "or_sage_max_aggregate": (None, [_i64, _i64, _p, _p, _p, _p]),
            "or_sage_forward": (None, [_i64, _i64, _i64, _i32, _p, _p, _p, _p, _p,
                                       _p, _i32, _i32, _p]),
            "or_gcn_forward": (None, [_i64, _i64, _i64, _p, _p, _p, _p, _p, _p,
                                      _i32, _i32, _p]),
            "or_gat_scores": (None, [_i64, _i64, _p, _p, _p, _p, _p]),
            "or_gat_forward": (None, [_i64, _i64, _i64, _p, _p, _p, _p, _p, _p,
                                      _p, _f32, _i32, _i32, _p]),
            "or_parse_edges": (_i32, [_p, _i64, C.c_char_p, _p, _p, _i64, C.POINTER(_i64)]),
            "or_parse_features": (_i32, [_p, _i64, C.c_char_p, _p, _i64, C.POINTER(_i64),
                                         C.POINTER(_i64)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    # -- CSV ingestion (graph_loader.cpp:61-206), over bytes ------------------
    def parse_edges(self, text: bytes, name: str = ""):
        """(src, dst) int32 arrays; raises OracleError('runtime_error', msg)."""
        t = np.frombuffer(bytes(text), np.uint8).copy()
        cap = int(text.count(b"\n")) + 1
        src = np.zeros(cap, np.int32)
        dst = np.zeros(cap, np.int32)
        cnt = _i64()
        rc = self.L.or_parse_edges(_ptr(t), len(text), name.encode(), _ptr(src), _ptr(dst), cap,
                                   C.byref(cnt))
        if rc:
            raise OracleError("runtime_error", self.L.or_last_error().decode("latin-1"))
        return src[:cnt.value].copy(), dst[:cnt.value].copy()

    def parse_features(self, text: bytes, name: str = "") -> np.ndarray:
        t = np.frombuffer(bytes(text), np.uint8).copy()
        rows, cols = _i64(), _i64()
        rc = self.L.or_parse_features(_ptr(t), len(text), name.encode(), None, 0, C.byref(rows),
                                      C.byref(cols))
        if rc:
            raise OracleError("runtime_error", self.L.or_last_error().decode("latin-1"))
        out = np.zeros((rows.value, cols.value), np.float32)
        self.L.or_parse_features(_ptr(t), len(text), name.encode(), _ptr(out), out.size,
                                 C.byref(rows), C.byref(cols))
        return out

    def set_num_threads(self, n: int) -> None:
        self.L.or_set_num_threads(int(n))

    def num_threads(self) -> int:
        return int(self.L.or_get_num_threads())

    # -- graph preprocessing ------------------------------------------------
    def edge_list_to_csr(self, src, dst, n_nodes: int) -> CSR:
        src, dst = _i(src), _i(dst)
        e = src.shape[0]
        rp = np.zeros(n_nodes + 1, np.int32)
        ci = np.zeros(e, np.int32)
        v = np.zeros(e, np.float32)
        rc = self.L.or_edge_list_to_csr(n_nodes, e, _ptr(src), _ptr(dst), _ptr(rp),
                                        _ptr(ci), _ptr(v))
        if rc:
            raise OracleError("invalid_argument", self.L.or_last_error().decode())
        return CSR(n_nodes, n_nodes, rp, ci, v)

    def add_self_loops(self, a: CSR) -> CSR:
        n = a.n_rows
        nnz2 = int(self.L.or_add_self_loops_nnz(n, _ptr(a.row_ptr), _ptr(a.col_ind)))
        rp = np.zeros(n + 1, np.int32)
        ci = np.zeros(nnz2, np.int32)
        v = np.zeros(nnz2, np.float32)
        self.L.or_add_self_loops(n, _ptr(a.row_ptr), _ptr(a.col_ind), _ptr(a.val),
                                 _ptr(rp), _ptr(ci), _ptr(v))
        return CSR(n, n, rp, ci, v)

    def gcn_norm(self, a: CSR, with_degrees: bool = False):
        n = a.n_rows
        nnz2 = int(self.L.or_add_self_loops_nnz(n, _ptr(a.row_ptr), _ptr(a.col_ind)))
        rp = np.zeros(n + 1, np.int32)
        ci = np.zeros(nnz2, np.int32)
        v = np.zeros(nnz2, np.float32)
        deg = np.zeros(n, np.float32)
        dis = np.zeros(n, np.float32)
        self.L.or_gcn_norm(n, _ptr(a.row_ptr), _ptr(a.col_ind), _ptr(a.val), _ptr(rp),
                           _ptr(ci), _ptr(v), _ptr(deg), _ptr(dis))
        out = CSR(n, n, rp, ci, v)
        return (out, deg, dis) if with_degrees else out

    def edge_softmax(self, a: CSR) -> CSR:
        v = np.zeros_like(a.val)
        self.L.or_edge_softmax(a.n_rows, _ptr(a.row_ptr), _ptr(a.val), _ptr(v))
        return CSR(a.n_rows, a.n_cols, a.row_ptr.copy(), a.col_ind.copy(), v)

    # -- ops ----------------------------------------------------------------
    def spmm(self, a: CSR, b) -> np.ndarray:
        b = _f(b)
        f = b.shape[1]
        c = np.zeros((a.n_rows, f), np.float32)
        self.L.or_spmm(a.n_rows, f, _ptr(a.row_ptr), _ptr(a.col_ind), _ptr(a.val),
                       _ptr(b), _ptr(c))
        return c

    def spmm_rows_f64(self, a: CSR, b, rows):
        """Checker (not a restatement): float64 ``(exact, absum)`` of the
        product's rows ``rows``: sum of val*B[col] and of |val*B[col]|."""
        b = _f(b)
        rows = _i(rows)
        f = b.shape[1]
        exact = np.zeros((rows.shape[0], f), np.float64)
        absum = np.zeros_like(exact)
        self.L.or_spmm_rows_f64(rows.shape[0], _ptr(rows), f, _ptr(a.row_ptr), _ptr(a.col_ind),
                                _ptr(a.val), _ptr(b), _ptr(exact), _ptr(absum))
        return exact, absum

    def matmul(self, a, b) -> np.ndarray:
        a, b = _f(a), _f(b)
        c = np.zeros((a.shape[0], b.shape[1]), np.float32)
        self.L.or_matmul(a.shape[0], a.shape[1], b.shape[1], _ptr(a), _ptr(b), _ptr(c))
        return c

    def activation(self, kind: str, x, alpha: float = 0.0) -> np.ndarray:
        x = _f(x).copy()
        n = x.size
        if kind == "relu":
            self.L.or_relu(n, _ptr(x))
        elif kind == "leaky_relu":
            self.L.or_leaky_relu(n, _ptr(x), alpha)
        elif kind == "elu":
            self.L.or_elu(n, _ptr(x), alpha)
        elif kind == "sigmoid":
            self.L.or_sigmoid(n, _ptr(x))
        elif kind == "tanh":
            self.L.or_tanh(n, _ptr(x))
        elif kind == "gelu":
            self.L.or_gelu(n, _ptr(x))
        elif kind == "softmax":
            self.L.or_softmax(x.shape[0], x.shape[1], _ptr(x))
        elif kind == "log_softmax":
            self.L.or_log_softmax(x.shape[0], x.shape[1], _ptr(x))
        else:
            raise ValueError(kind)
        return x

    def add_bias(self, x, bias) -> np.ndarray:
        x = _f(x).copy()
        self.L.or_add_bias(x.shape[0], x.shape[1], _ptr(x), _ptr(_f(bias)))
        return x

    # -- layers ---------------------------------------------------------------
    def sage_max_aggregate(self, a: CSR, h) -> np.ndarray:
        h = _f(h)
        out = np.zeros((a.n_rows, h.shape[1]), np.float32)
        self.L.or_sage_max_aggregate(a.n_rows, h.shape[1], _ptr(a.row_ptr),
                                     _ptr(a.col_ind), _ptr(h), _ptr(out))
        return out

    def gcn_layer(self, a_norm: CSR, h, w, b=None, act: int = 1) -> np.ndarray:
        h, w = _f(h), _f(w)
        out = np.zeros((a_norm.n_rows, w.shape[1]), np.float32)
        self.L.or_gcn_forward(a_norm.n_rows, w.shape[0], w.shape[1], _ptr(a_norm.row_ptr),
                              _ptr(a_norm.col_ind), _ptr(a_norm.val), _ptr(h), _ptr(w),
                              _ptr(None if b is None else _f(b)), int(b is not None),
                              act, _ptr(out))
        return out

    def sage_layer(self, a: CSR, h, wn, ws, b=None, act: int = 1,
                   agg: int = 0) -> np.ndarray:
        h, wn, ws = _f(h), _f(wn), _f(ws)
        out = np.zeros((a.n_rows, wn.shape[1]), np.float32)
        self.L.or_sage_forward(a.n_rows, wn.shape[0], wn.shape[1], agg, _ptr(a.row_ptr),
                               _ptr(a.col_ind), _ptr(h), _ptr(wn), _ptr(ws),
                               _ptr(None if b is None else _f(b)), int(b is not None),
                               act, _ptr(out))
        return out

    def gat_scores(self, wh, al, ar):
        wh = _f(wh)
        n, f = wh.shape
        s = np.zeros(n, np.float32)
        d = np.zeros(n, np.float32)
        self.L.or_gat_scores(n, f, _ptr(wh), _ptr(_f(al)), _ptr(_f(ar)), _ptr(s), _ptr(d))
        return s, d

    def gat_layer(self, a_sl: CSR, h, w, al, ar, b=None, slope: float = 0.2,
                  act: int = 0) -> np.ndarray:
        h, w = _f(h), _f(w)
        out = np.zeros((a_sl.n_rows, w.shape[1]), np.float32)
        self.L.or_gat_forward(a_sl.n_rows, w.shape[0], w.shape[1], _ptr(a_sl.row_ptr),
                              _ptr(a_sl.col_ind), _ptr(h), _ptr(w), _ptr(_f(al)),
                              _ptr(_f(ar)), _ptr(None if b is None else _f(b)), slope,
                              int(b is not None), act, _ptr(out))
        return out

    # -- Model::forward (model.cpp:359-439) -----------------------------------
    def model_forward(self, spec, weights: dict, adj: CSR, x) -> np.ndarray:
        """Restates model.cpp:359-439: gcn_norm if any GCN layer, add_self_loops
        if any GAT layer (both recomputed per call), layers in order, multi-head
        GAT concat (:312-332) or average (:335-354), then the post activation
        (:426-435).  ``spec`` is a list of layer dicts (see tinygnn_amd.models)."""
        a_gcn = self.gcn_norm(adj) if any(l["type"] == "gcn" for l in spec) else None
        a_sl = self.add_self_loops(adj) if any(l["type"] == "gat" for l in spec) else None
        h = _f(x).copy()
        for li, l in enumerate(spec):
            p = f"layer{li}"
            if l["type"] == "gcn":
                h = self.gcn_layer(a_gcn, h, weights[p + ".weight"],
                                   weights.get(p + ".bias") if l.get("bias", True) else None,
                                   l.get("act", 1))
            elif l["type"] == "sage":
                h = self.sage_layer(adj, h, weights[p + ".weight_neigh"],
                                    weights[p + ".weight_self"],
                                    weights.get(p + ".bias") if l.get("bias", True) else None,
                                    l.get("act", 1), l.get("agg", 0))
            elif l["type"] == "gat":
                heads = []
                for hd in range(l.get("heads", 1)):
                    hp = f"{p}.head{hd}"
                    heads.append(self.gat_layer(
                        a_sl, h, weights[hp + ".weight"], weights[hp + ".attn_left"],
                        weights[hp + ".attn_right"],
                        weights.get(hp + ".bias") if l.get("bias", True) else None,
                        l.get("slope", 0.2), l.get("act", 0)))
                if len(heads) == 1:
                    h = heads[0]
                elif l.get("concat", True):
                    h = np.ascontiguousarray(np.concatenate(heads, axis=1))
                else:
                    acc = np.zeros_like(heads[0])
                    for t in heads:
                        acc += t
                    h = acc * np.float32(1.0 / len(heads))
            post = l.get("post", 0)
            if post == 1:
                h = self.activation("relu", h)
            elif post == 2:
                h = self.activation("elu", h, 1.0)
        return h


# ---------------------------------------------------------------------------
# The real reference (compiled from its sources)
# ---------------------------------------------------------------------------
_KINDS = {1: "invalid_argument", 2: "runtime_error", 3: "out_of_range", 4: "exception"}
_ACT = {"relu": 0, "leaky_relu": 1, "elu": 2, "sigmoid": 3, "tanh": 4, "gelu": 5,
        "softmax": 6, "log_softmax": 7}


class _RefTensor:
    def __init__(self, lib, handle):
        self._lib = lib
        self.h = handle

    def __del__(self):
        if self.h:
            self._lib.L.ref_tensor_free(self.h)
            self.h = None

    def to_csr(self) -> CSR:
        L = self._lib.L
        r, c, nnz = L.ref_tensor_rows(self.h), L.ref_tensor_cols(self.h), L.ref_tensor_nnz(self.h)
        rp = np.zeros(r + 1, np.int32)
        ci = np.zeros(nnz, np.int32)
        v = np.zeros(nnz, np.float32)
        L.ref_tensor_read(self.h, _ptr(rp), _ptr(ci), _ptr(v))
        return CSR(r, c, rp, ci, v)


class _Reference:
    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is missing (built only where the reference is)")
        L = C.CDLL(path)
        self.L = L
        sig = {
            "ref_last_error": (C.c_char_p, []),
            "ref_set_num_threads": (None, [_i32]),
            "ref_get_num_threads": (_i32, []),
            "ref_tensor_csr": (_p, [_i64, _i64, _i64, _p, _p, _p]),
            "ref_tensor_dense": (_p, [_i64, _i64, _p]),
            "ref_tensor_free": (None, [_p]),
            "ref_tensor_rows": (_i64, [_p]),
            "ref_tensor_cols": (_i64, [_p]),
            "ref_tensor_nnz": (_i64, [_p]),
            "ref_tensor_read": (_i32, [_p, _p, _p, _p]),
            "ref_edge_list_to_csr": (_p, [_i64, _i64, _p, _p]),
            "ref_add_self_loops": (_p, [_p]),
            "ref_gcn_norm": (_p, [_p]),
            "ref_edge_softmax": (_p, [_p]),
            "ref_spmm": (_i32, [_p, _p, _p]),
            "ref_matmul": (_i32, [_p, _p, _p]),
            "ref_sage_max_aggregate": (_i32, [_p, _p, _p]),
            "ref_activation": (_i32, [_i32, _i64, _i64, _p, _f32]),
            "ref_add_bias": (_i32, [_i64, _i64, _p, _i64, _i64, _p]),
            "ref_gcn_layer": (_i32, [_p, _p, _i64, _i64, _p, _p, _i32, _i32, _p]),
            "ref_sage_layer": (_i32, [_p, _p, _i64, _i64, _i32, _p, _p, _p, _i32, _i32, _p]),
            "ref_gat_layer": (_i32, [_p, _p, _i64, _i64, _p, _p, _p, _p, _f32, _i32, _i32,
                                     _p]),
            "ref_model_create": (_p, []),
            "ref_model_free": (None, [_p]),
            "ref_model_add_gcn": (_i32, [_p, _i64, _i64, _i32, _i32, _i32]),
            "ref_model_add_sage": (_i32, [_p, _i64, _i64, _i32, _i32, _i32, _i32]),
            "ref_model_add_gat": (_i32, [_p, _i64, _i64, _i64, _i32, _f32, _i32, _i32,
                                         _i32]),
            "ref_model_set_tensor": (_i32, [_p, C.c_char_p, _i64, _i64, _p]),
            "ref_model_load_weights": (_i32, [_p]),
            "ref_model_forward": (_i32, [_p, _p, _p, C.POINTER(_i64), C.POINTER(_i64), _p,
                                         _i64]),
            "ref_parse_edges": (_p, [C.c_char_p, C.POINTER(_i32)]),
            "ref_edges_count": (_i64, [_p]),
            "ref_edges_read": (None, [_p, _p, _p]),
            "ref_edges_free": (None, [_p]),
            "ref_parse_features": (_p, [C.c_char_p, C.POINTER(_i32)]),
            "ref_graph_load": (_p, [C.c_char_p, C.c_char_p, C.POINTER(_i32)]),
            "ref_graph_adjacency": (_p, [_p]),
            "ref_graph_features": (_p, [_p]),
            "ref_graph_counts": (None, [_p, C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i64)]),
            "ref_graph_free": (None, [_p]),
            "ref_load_cora": (_p, [C.c_char_p, C.POINTER(_i32)]),
            "ref_cora_counts": (None, [_p] + [C.POINTER(_i64)] * 4),
            "ref_cora_adjacency": (_p, [_p]),
            "ref_cora_features": (_p, [_p]),
            "ref_cora_read": (None, [_p, _p, _p, _p, _p]),
            "ref_cora_free": (None, [_p]),
            "ref_load_weight_file": (_p, [C.c_char_p, C.POINTER(_i32)]),
            "ref_weights_accuracy": (_f32, [_p]),
            "ref_weights_names": (_i64, [_p, _p, _i64]),
            "ref_weights_tensor": (_p, [_p, C.c_char_p]),
            "ref_weights_free": (None, [_p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    def _check(self, rc):
        if rc:
            raise OracleError(_KINDS.get(rc, "exception"), self.L.ref_last_error().decode())

    def _opened(self, h, code):
        if not h:
            raise OracleError(_KINDS.get(code.value, "exception"),
                              self.L.ref_last_error().decode("latin-1"))
        return h

    def _dense_of(self, t) -> np.ndarray:
        """Copies a borrowed dense Tensor handle out."""
        L = self.L
        out = np.zeros((L.ref_tensor_rows(t), L.ref_tensor_cols(t)), np.float32)
        L.ref_tensor_read(t, None, None, _ptr(out))
        return out

    def _csr_of(self, t) -> CSR:
        L = self.L
        r, c, nnz = L.ref_tensor_rows(t), L.ref_tensor_cols(t), L.ref_tensor_nnz(t)
        rp, ci, v = np.zeros(r + 1, np.int32), np.zeros(nnz, np.int32), np.zeros(nnz, np.float32)
        L.ref_tensor_read(t, _ptr(rp), _ptr(ci), _ptr(v))
        return CSR(r, c, rp, ci, v)

    # -- file ingestion (graph_loader.cpp:61-326, model.cpp:49-185) ----------
    def parse_edges_file(self, path: str):
        code = _i32()
        h = self._opened(self.L.ref_parse_edges(path.encode(), C.byref(code)), code)
        n = self.L.ref_edges_count(h)
        src, dst = np.zeros(n, np.int32), np.zeros(n, np.int32)
        self.L.ref_edges_read(h, _ptr(src), _ptr(dst))
        self.L.ref_edges_free(h)
        return src, dst

    def parse_features_file(self, path: str) -> np.ndarray:
        code = _i32()
        h = self._opened(self.L.ref_parse_features(path.encode(), C.byref(code)), code)
        out = self._dense_of(h)
        self.L.ref_tensor_free(h)
        return out

    def load_graph(self, edges_path: str, features_path: str):
        """(adjacency CSR, features, (num_nodes, num_edges, num_features))."""
        code = _i32()
        g = self._opened(self.L.ref_graph_load(edges_path.encode(), features_path.encode(),
                                               C.byref(code)), code)
        n, e, f = _i64(), _i64(), _i64()
        self.L.ref_graph_counts(g, C.byref(n), C.byref(e), C.byref(f))
        adj = self._csr_of(self.L.ref_graph_adjacency(g))
        x = self._dense_of(self.L.ref_graph_features(g))
        self.L.ref_graph_free(g)
        return adj, x, (n.value, e.value, f.value)

    def load_cora(self, path: str) -> dict:
        code = _i32()
        h = self._opened(self.L.ref_load_cora(path.encode(), C.byref(code)), code)
        cnt = [_i64() for _ in range(4)]
        self.L.ref_cora_counts(h, *[C.byref(c) for c in cnt])
        n = cnt[0].value
        labels = np.zeros(n, np.int32)
        masks = [np.zeros(n, np.uint8) for _ in range(3)]
        self.L.ref_cora_read(h, _ptr(labels), *[_ptr(m) for m in masks])
        out = dict(num_nodes=n, num_features=cnt[1].value, num_classes=cnt[2].value,
                   num_edges=cnt[3].value, adjacency=self._csr_of(self.L.ref_cora_adjacency(h)),
                   features=self._dense_of(self.L.ref_cora_features(h)), labels=labels,
                   train_mask=masks[0], val_mask=masks[1], test_mask=masks[2])
        self.L.ref_cora_free(h)
        return out

    def load_weight_file(self, path: str):
        """(test_accuracy, {name: float32 array})."""
        code = _i32()
        h = self._opened(self.L.ref_load_weight_file(path.encode(), C.byref(code)), code)
        need = self.L.ref_weights_names(h, None, 0)
        buf = C.create_string_buffer(int(need))
        self.L.ref_weights_names(h, C.cast(buf, _p), need)
        names = ([s for s in buf.value.decode("utf-8", "surrogateescape").split("\n") if s]
                 if need > 1 else [])
        tensors = {nm: self._dense_of(self.L.ref_weights_tensor(h, nm.encode("utf-8", "surrogateescape")))
                   for nm in names}
        acc = float(self.L.ref_weights_accuracy(h))
        self.L.ref_weights_free(h)
        return acc, tensors

    def _handle(self, h):
        if not h:
            raise OracleError("invalid_argument", self.L.ref_last_error().decode())
        return _RefTensor(self, h)

    def set_num_threads(self, n: int) -> None:
        self.L.ref_set_num_threads(int(n))

    def num_threads(self) -> int:
        return int(self.L.ref_get_num_threads())

    def csr(self, a: CSR) -> _RefTensor:
        return self._handle(self.L.ref_tensor_csr(a.n_rows, a.n_cols, a.nnz, _ptr(_i(a.row_ptr)),
                                                  _ptr(_i(a.col_ind)), _ptr(_f(a.val))))

    def csr_raw(self, n_rows, n_cols, rp, ci, v) -> _RefTensor:
        rp, ci, v = _i(rp), _i(ci), _f(v)
        return self._handle(self.L.ref_tensor_csr(n_rows, n_cols, ci.shape[0], _ptr(rp),
                                                  _ptr(ci), _ptr(v)))

    def dense(self, x) -> _RefTensor:
        x = _f(x)
        if x.ndim == 1:
            x = x.reshape(1, -1)
        return self._handle(self.L.ref_tensor_dense(x.shape[0], x.shape[1], _ptr(x)))

    def edge_list_to_csr(self, src, dst, n_nodes) -> CSR:
        src, dst = _i(src), _i(dst)
        return self._handle(self.L.ref_edge_list_to_csr(n_nodes, src.shape[0], _ptr(src),
                                                        _ptr(dst))).to_csr()

    def add_self_loops(self, a: CSR) -> CSR:
        t = self.csr(a)
        return self._handle(self.L.ref_add_self_loops(t.h)).to_csr()

    def gcn_norm(self, a: CSR) -> CSR:
        t = self.csr(a)
        return self._handle(self.L.ref_gcn_norm(t.h)).to_csr()

    def edge_softmax(self, a: CSR) -> CSR:
        t = self.csr(a)
        return self._handle(self.L.ref_edge_softmax(t.h)).to_csr()

    def spmm(self, a: CSR, b) -> np.ndarray:
        b = _f(b)
        out = np.zeros((a.n_rows, b.shape[1]), np.float32)
        ta, tb = self.csr(a), self.dense(b)
        self._check(self.L.ref_spmm(ta.h, tb.h, _ptr(out)))
        return out

    def spmm_rows_f64(self, a: CSR, b, rows):
        """Checker (not a restatement): float64 ``(exact, absum)`` of the
        product's rows ``rows``: sum of val*B[col] and of |val*B[col]|."""
        b = _f(b)
        rows = _i(rows)
        f = b.shape[1]
        exact = np.zeros((rows.shape[0], f), np.float64)
        absum = np.zeros_like(exact)
        self.L.or_spmm_rows_f64(rows.shape[0], _ptr(rows), f, _ptr(a.row_ptr), _ptr(a.col_ind),
                                _ptr(a.val), _ptr(b), _ptr(exact), _ptr(absum))
        return exact, absum

    def matmul(self, a, b) -> np.ndarray:
        a, b = _f(a), _f(b)
        out = np.zeros((a.shape[0], b.shape[1]), np.float32)
        ta, tb = self.dense(a), self.dense(b)
        self._check(self.L.ref_matmul(ta.h, tb.h, _ptr(out)))
        return out

    def activation(self, kind: str, x, alpha: float = 0.0) -> np.ndarray:
        x = _f(x).copy()
        if x.ndim == 1:
            x = x.reshape(1, -1)
        self._check(self.L.ref_activation(_ACT[kind], x.shape[0], x.shape[1], _ptr(x), alpha))
        return x

    def add_bias(self, x, bias) -> np.ndarray:
        x = _f(x).copy()
        b = _f(bias)
        if b.ndim == 1:
            b = b.reshape(1, -1)
        self._check(self.L.ref_add_bias(x.shape[0], x.shape[1], _ptr(x), b.shape[0],
                                        b.shape[1], _ptr(b)))
        return x

    def sage_max_aggregate(self, a: CSR, h) -> np.ndarray:
        h = _f(h)
        out = np.zeros((a.n_rows, h.shape[1]), np.float32)
        ta, th = self.csr(a), self.dense(h)
        self._check(self.L.ref_sage_max_aggregate(ta.h, th.h, _ptr(out)))
        return out

    def gcn_layer(self, a_norm: CSR, h, w, b=None, act: int = 1) -> np.ndarray:
        h, w = _f(h), _f(w)
        out = np.zeros((a_norm.n_rows, w.shape[1]), np.float32)
        ta, th = self.csr(a_norm), self.dense(h)
        self._check(self.L.ref_gcn_layer(ta.h, th.h, w.shape[0],
                                         w.shape[1], _ptr(w),
                                         _ptr(None if b is None else _f(b)),
                                         int(b is not None), act, _ptr(out)))
        return out

    def sage_layer(self, a: CSR, h, wn, ws, b=None, act: int = 1, agg: int = 0) -> np.ndarray:
        h, wn, ws = _f(h), _f(wn), _f(ws)
        out = np.zeros((a.n_rows, wn.shape[1]), np.float32)
        ta, th = self.csr(a), self.dense(h)
        self._check(self.L.ref_sage_layer(ta.h, th.h, wn.shape[0],
                                          wn.shape[1], agg, _ptr(wn), _ptr(ws),
                                          _ptr(None if b is None else _f(b)),
                                          int(b is not None), act, _ptr(out)))
        return out

    def gat_layer(self, a_sl: CSR, h, w, al, ar, b=None, slope: float = 0.2,
                  act: int = 0) -> np.ndarray:
        h, w = _f(h), _f(w)
        out = np.zeros((a_sl.n_rows, w.shape[1]), np.float32)
        ta, th = self.csr(a_sl), self.dense(h)
        self._check(self.L.ref_gat_layer(ta.h, th.h, w.shape[0],
                                         w.shape[1], _ptr(w), _ptr(_f(al)), _ptr(_f(ar)),
                                         _ptr(None if b is None else _f(b)), slope,
                                         int(b is not None), act, _ptr(out)))
        return out

    def model(self, spec, weights: dict) -> "RefModel":
        return RefModel(self, spec, weights)


class RefModel:
    """The reference's ``Model`` built from a layer spec and named weights."""

    def __init__(self, lib: _Reference, spec, weights: dict):
        self.lib = lib
        L = lib.L
        self.h = L.ref_model_create()
        for l in spec:
            t = l["type"]
            if t == "gcn":
                lib._check(L.ref_model_add_gcn(self.h, l["in"], l["out"], int(l.get("bias", True)),
                                               l.get("act", 1), l.get("post", 0)))
            elif t == "sage":
                lib._check(L.ref_model_add_sage(self.h, l["in"], l["out"], l.get("agg", 0),
                                                int(l.get("bias", True)), l.get("act", 1),
                                                l.get("post", 0)))
            elif t == "gat":
                lib._check(L.ref_model_add_gat(self.h, l["in"], l["out"], l.get("heads", 1),
                                               int(l.get("concat", True)), l.get("slope", 0.2),
                                               int(l.get("bias", True)), l.get("act", 0),
                                               l.get("post", 0)))
        self.out_dim = spec[-1]["out"] * (spec[-1].get("heads", 1)
                                          if spec[-1]["type"] == "gat" and spec[-1].get("concat", True)
                                          else 1)
        for name, arr in weights.items():
            a = _f(arr)
            if a.ndim == 1:
                a = a.reshape(1, -1)
            lib._check(L.ref_model_set_tensor(self.h, name.encode(), a.shape[0], a.shape[1],
                                              _ptr(a)))
        lib._check(L.ref_model_load_weights(self.h))

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.L.ref_model_free(self.h)
            self.h = None

    def forward_handles(self, adj_t: _RefTensor, x_t: _RefTensor, n_rows: int) -> np.ndarray:
        out = np.zeros((n_rows, self.out_dim), np.float32)
        r, c = _i64(0), _i64(0)
        self.lib._check(self.lib.L.ref_model_forward(self.h, adj_t.h, x_t.h, C.byref(r),
                                                     C.byref(c), _ptr(out), out.size))
        assert (r.value, c.value) == out.shape
        return out

    def forward(self, adj: CSR, x) -> np.ndarray:
        ta, tx = self.lib.csr(adj), self.lib.dense(x)
        return self.forward_handles(ta, tx, adj.n_rows)


_restate = None
_reference = None


def restate() -> _Restate:
    global _restate
    if _restate is None:
        _restate = _Restate()
    return _restate


def reference() -> _Reference:
    global _reference
    if _reference is None:
        _reference = _Reference()
    return _reference


def has_reference() -> bool:
    return os.path.exists(REF_SO)
