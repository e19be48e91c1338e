"""ctypes binding of the C-ABI declared in include/tinygnn_amd.h.

The shared library is ``tinygnn_amd/_build/libtinygnn_amd.so`` (built in-tree
by ``tinygnn_amd.build``).  There is no fallback: if the library is missing,
every call raises ``NativeLibraryMissing``.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libtinygnn_amd.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "tinygnn_amd.h")

i64 = C.c_int64
i32 = C.c_int
f32 = C.c_float
vp = C.c_void_p
sz = C.c_size_t
pi64 = C.POINTER(C.c_int64)

TG_OK = 0
TG_ERR_INVALID_ARGUMENT = 1
TG_ERR_RUNTIME = 2
TG_ERR_OUT_OF_RANGE = 3
TG_ERR_HIP = 4
TG_ERR_ALLOC = 5


class NativeLibraryMissing(RuntimeError):
    pass


class TgError(RuntimeError):
    """A failed C-ABI call; ``kind`` names the reference exception type."""

    KINDS = {TG_ERR_INVALID_ARGUMENT: "invalid_argument", TG_ERR_RUNTIME: "runtime_error",
             TG_ERR_OUT_OF_RANGE: "out_of_range", TG_ERR_HIP: "hip_error",
             TG_ERR_ALLOC: "alloc_error"}

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status
        self.kind = self.KINDS.get(status, "unknown")


class InvalidArgument(TgError, ValueError):
    pass


class OutOfRange(TgError, IndexError):
    pass


# name -> (restype, argtypes)
SIGNATURES = {
    "tg_last_error": (C.c_char_p, []),
    "tg_version": (i32, []),
    "tg_edge_list_to_csr_workspace_size": (sz, [i64, i64]),
    "tg_edge_list_to_csr": (i32, [i64, i64, vp, vp, vp, vp, vp, vp, sz, vp]),
    "tg_csr_validate": (i32, [i64, i64, i64, vp, vp, vp]),
    "tg_coo_to_csr": (i32, [i64, i64, vp, vp, vp, vp, vp, C.c_char_p, vp]),
    "tg_self_loops_workspace_size": (sz, [i64]),
    "tg_add_self_loops": (i32, [i64, i64, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
    "tg_gcn_norm": (i32, [i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
    "tg_spmm_plan_create": (i32, [i64, i64, vp, i64, i64, vp, C.POINTER(vp)]),
    "tg_spmm_plan_destroy": (i32, [vp]),
    "tg_spmm_plan_info": (i32, [vp, pi64, pi64, pi64]),
    "tg_spmm_execute": (i32, [vp, i64, i64, vp, vp, vp, vp, i64, vp, i64, vp]),
    "tg_spmm_plan_set_precision": (i32, [vp, i32]),
    "tg_spmm_execute_epilogue": (i32, [vp, i64, i64, vp, vp, vp, vp, i64, vp, i64, vp, i32, vp]),
    "tg_probe_l2_read": (i32, [vp, i64, i64, vp, vp]),
    "tg_spmm": (i32, [i64, i64, i64, i64, vp, vp, vp, vp, i64, vp, i64, vp]),
    "tg_spmm_ex": (i32, [i64, i64, i64, i64, vp, vp, vp, vp, i64, vp, i64, i32, vp]),
    "tg_spmm_noalloc": (i32, [i64, i64, i64, i64, vp, vp, vp, vp, i64, vp, i64, vp]),
    "tg_matmul": (i32, [i64, i64, i64, vp, i64, vp, i64, vp, i64, vp, i32, i32, vp]),
    "tg_relu": (i32, [i64, vp, vp]),
    "tg_leaky_relu": (i32, [i64, vp, f32, vp]),
    "tg_elu": (i32, [i64, vp, f32, vp]),
    "tg_sigmoid": (i32, [i64, vp, vp]),
    "tg_tanh": (i32, [i64, vp, vp]),
    "tg_gelu": (i32, [i64, vp, vp]),
    "tg_softmax": (i32, [i64, i64, vp, vp]),
    "tg_log_softmax": (i32, [i64, i64, vp, vp]),
    "tg_add_bias": (i32, [i64, i64, vp, vp, vp]),
    "tg_edge_softmax": (i32, [i64, vp, vp, vp, vp]),
    "tg_sage_aggregate": (i32, [vp, i64, i64, i32, vp, vp, vp, i64, vp, i64, vp]),
    "tg_sage_forward_workspace_size": (sz, [i64, i64, i64, i32, i32, i64]),
    "tg_sage_forward": (i32, [vp, i64, i64, i64, i32, vp, vp, vp, vp, vp, vp, i32, i32, i32,
                              vp, vp, sz, vp]),
    "tg_gat_scores": (i32, [i64, i64, i64, vp, i64, vp, vp, vp, vp, vp]),
    "tg_gat_workspace_size": (sz, [vp, i64, i64, i64, i32]),
    "tg_gat_aggregate": (i32, [vp, i64, i64, i64, vp, vp, vp, i64, vp, vp, f32, vp, i32, i32,
                               i32, vp, i64, vp, sz, vp]),
    "tg_model_create": (i32, [C.POINTER(vp)]),
    "tg_model_destroy": (i32, [vp]),
    "tg_model_add_gcn_layer": (i32, [vp, i64, i64, i32, i32, i32, pi64]),
    "tg_model_add_sage_layer": (i32, [vp, i64, i64, i32, i32, i32, i32, pi64]),
    "tg_model_add_gat_layer": (i32, [vp, i64, i64, i64, i32, f32, i32, i32, i32, pi64]),
    "tg_model_num_layers": (i32, [vp, pi64]),
    "tg_model_output_cols": (i32, [vp, pi64]),
    "tg_model_set_tensor": (i32, [vp, C.c_char_p, i64, i64, vp]),
    "tg_model_clear_tensors": (i32, [vp]),
    "tg_model_load_weights": (i32, [vp]),
    "tg_model_set_sage_dataflow": (i32, [vp, i32]),
    "tg_model_set_precision": (i32, [vp, i32]),
    "tg_model_set_blocking": (i32, [vp, i64]),
    "tg_model_forward": (i32, [vp, i64, i64, vp, vp, vp, i64, vp, vp, i32, vp]),
    "tg_model_invalidate": (i32, [vp]),
    "tg_model_blocking_info": (i32, [vp, pi64, pi64, pi64, pi64, pi64, pi64]),
    "tg_model_set_self_loop_split": (i32, [vp, i32]),
    "tg_model_set_resident_passes": (i32, [vp, i32]),
    "tg_csv_open": (i32, [C.c_char_p, C.POINTER(vp), vp]),
    "tg_csv_index": (i32, [vp, i64, C.c_char_p, C.POINTER(vp), vp]),
    "tg_csv_destroy": (i32, [vp]),
    "tg_csv_info": (i32, [vp, pi64, C.POINTER(i32)]),
    "tg_csv_parse_edges": (i32, [vp, vp, vp, pi64, vp]),
    "tg_csv_feature_shape": (i32, [vp, pi64, pi64, vp]),
    "tg_csv_parse_features": (i32, [vp, vp, i64, i64, vp]),
    "tg_weights_open": (i32, [C.c_char_p, C.POINTER(vp)]),
    "tg_weights_info": (i32, [vp, pi64, C.POINTER(f32)]),
    "tg_weights_tensor": (i32, [vp, i64, C.POINTER(vp), pi64, pi64, pi64, C.POINTER(vp)]),
    "tg_weights_destroy": (i32, [vp]),
    "tg_cora_open": (i32, [C.c_char_p, C.POINTER(vp)]),
    "tg_cora_info": (i32, [vp, pi64, pi64, pi64, pi64]),
    "tg_cora_host": (i32, [vp, C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), C.POINTER(vp)]),
    "tg_cora_upload": (i32, [vp, vp, vp, vp, vp, vp]),
    "tg_cora_destroy": (i32, [vp]),
}


def header_symbols(path: str = HEADER) -> list[str]:
    """Function names declared in the C-ABI header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", text)))


class _Lib:
    def __init__(self):
        self._cdll = None

    def load(self):
        if self._cdll is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"{LIB_PATH} not found: build it with `python -m tinygnn_amd.build` "
                    "(there is no CPU fallback)")
            lib = C.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name, None)
                if fn is None:
                    continue
                fn.restype = res
                fn.argtypes = args
            self._cdll = lib
        return self._cdll

    def __getattr__(self, name):
        if name.startswith("tg_"):
            return getattr(self.load(), name)
        raise AttributeError(name)

    def check(self, status: int) -> None:
        if status != TG_OK:
            msg = self.load().tg_last_error().decode(errors="replace")
            if status == TG_ERR_INVALID_ARGUMENT:
                raise InvalidArgument(status, msg)
            if status == TG_ERR_OUT_OF_RANGE:
                raise OutOfRange(status, msg)
            raise TgError(status, msg)


lib = _Lib()
