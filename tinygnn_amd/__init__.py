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
from dataclasses import dataclass

from ._lib import InvalidArgument, NativeLibraryMissing, OutOfRange, TgError, lib  # noqa: F401

ACT_NONE, ACT_RELU = 0, 1
POST_NONE, POST_RELU, POST_ELU = 0, 1, 2
AGG_MEAN, AGG_MAX = 0, 1
GEMM_AUTO, GEMM_INORDER, GEMM_MFMA = 0, 1, 2
EPI_NONE, EPI_RELU, EPI_ELU = 0, 1, 2
SAGE_AUTO, SAGE_CONCAT, SAGE_TRANSFORM_FIRST = 0, 1, 2
FORWARD_REFERENCE, FORWARD_CACHED = 0, 1


def _torch():
    import torch
    return torch


def stream_handle(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def dptr(t, dtype=None) -> int:
    """Device pointer of a contiguous CUDA/HIP torch tensor (0 for None)."""
    if t is None:
        return 0
    torch = _torch()
    if not t.is_cuda:
        raise ValueError("tinygnn_amd expects device (cuda) tensors")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("tinygnn_amd expects contiguous tensors")
    del torch
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
                 stream=None):
        h = C.c_void_p()
        lib.check(lib.tg_spmm_plan_create(n_rows, nnz_bound, dptr(row_ptr), max_f, chunk_nnz,
                                          stream_handle(stream), C.byref(h)))
        self.h = h
        self.row_ptr = row_ptr
        self.n_rows = n_rows

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


def spmm(a: DeviceCSR, b, plan: SpmmPlan | None = None, out=None, stream=None):
    """C = A * B (reference ops.cpp:198-297)."""
    torch = _torch()
    f = b.shape[1]
    if out is None:
        out = torch.empty((a.n_rows, f), dtype=torch.float32, device=b.device)
    s = stream_handle(stream)
    if plan is None:
        lib.check(lib.tg_spmm(a.n_rows, a.n_cols, f, a.nnz, dptr(a.row_ptr), dptr(a.col_ind),
                              dptr(a.val), dptr(b), b.stride(0), dptr(out), out.stride(0), s))
    else:
        lib.check(lib.tg_spmm_execute(plan.h, a.n_cols, f, dptr(a.row_ptr), dptr(a.col_ind),
                                      dptr(a.val), dptr(b), b.stride(0), dptr(out),
                                      out.stride(0), s))
    return out
