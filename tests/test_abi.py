"""The C-ABI library on the CPU (no GPU calls): it loads, exports every
function include/tinygnn_amd.h declares, and maps argument errors to the
reference's exception kinds and messages before touching the device."""
import ctypes as C
import subprocess

import pytest

from tinygnn_amd import _lib


def test_exports_every_header_symbol():
    lib = _lib.lib.load()
    declared = _lib.header_symbols()
    assert len(declared) >= 40
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert set(declared) <= exported
    # the ctypes table covers exactly the header
    assert set(_lib.SIGNATURES) == set(declared)


def test_version_and_error_channel():
    lib = _lib.lib.load()
    assert lib.tg_version() >= 1
    assert isinstance(lib.tg_last_error(), bytes)


def test_argument_errors_without_device():
    L = _lib.lib.load()
    # softmax over 0 columns (ops.cpp:511-515) fails before any device work
    assert L.tg_softmax(3, 0, None, None) == _lib.TG_ERR_INVALID_ARGUMENT
    assert L.tg_last_error().decode() == ("softmax_inplace: tensor has 0 columns — softmax "
                                          "over an empty set is undefined.")
    assert L.tg_log_softmax(3, 0, None, None) == _lib.TG_ERR_INVALID_ARGUMENT
    assert b"log-softmax over an empty set" in L.tg_last_error()
    assert L.tg_matmul(-1, 2, 2, None, 2, None, 2, None, 2, None, 0, 0,
                       None) == _lib.TG_ERR_INVALID_ARGUMENT
    assert L.tg_spmm_plan_create(4, 4, None, 4, 0, None, None) == _lib.TG_ERR_INVALID_ARGUMENT
    assert b"plan_out is null" in L.tg_last_error()
    h = C.c_void_p()
    assert L.tg_model_create(C.byref(h)) == _lib.TG_OK
    n = C.c_int64(-1)
    assert L.tg_model_num_layers(h, C.byref(n)) == _lib.TG_OK and n.value == 0
    # Model::forward on an empty model is a runtime_error (model.cpp:360-362)
    assert L.tg_model_output_cols(h, C.byref(n)) == _lib.TG_ERR_RUNTIME
    assert L.tg_last_error() == b"Model::forward: no layers configured."
    assert L.tg_model_forward(h, 0, 0, None, None, None, 0, None, None, 0,
                              None) == _lib.TG_ERR_RUNTIME
    assert L.tg_model_load_weights(h) == _lib.TG_OK  # nothing to load
    assert L.tg_model_destroy(h) == _lib.TG_OK


def test_python_front_end_raises_typed_errors():
    import tinygnn_amd as tg
    with pytest.raises(tg.InvalidArgument):
        _lib.lib.check(_lib.TG_ERR_INVALID_ARGUMENT)
    with pytest.raises(tg.OutOfRange):
        _lib.lib.check(_lib.TG_ERR_OUT_OF_RANGE)
    with pytest.raises(tg.TgError) as e:
        _lib.lib.check(_lib.TG_ERR_RUNTIME)
    assert e.value.kind == "runtime_error"


def test_spmm_noalloc_rejects_oversize_before_device_work():
    """tg_spmm_noalloc checks the plan's size against its fixed scratch before
    any device call (so this runs without a GPU): config D's 10^6 x 10^6 /
    5 x 10^7 matrix fits up to f = 256 and not at f = 257."""
    L = _lib.lib.load()
    dummy = C.c_void_p(16)  # never dereferenced: the call fails on the host
    rc = L.tg_spmm_noalloc(1_000_000, 1_000_000, 257, 50_000_000, dummy, dummy, dummy, dummy,
                           257, dummy, 257, None)
    assert rc == _lib.TG_ERR_INVALID_ARGUMENT
    msg = L.tg_last_error().decode()
    assert msg.startswith("tg_spmm_noalloc: the plan for m=1000000, nnz=50000000, f=257 needs ")
    assert "the maximum is 134217728" in msg
    assert L.tg_spmm_noalloc(-1, 1, 1, 1, dummy, dummy, dummy, dummy, 1, dummy, 1,
                             None) == _lib.TG_ERR_INVALID_ARGUMENT
