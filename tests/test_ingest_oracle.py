"""Ingestion on the CPU: GraphLoader's CSV parsing (graph_loader.cpp:14-326),
the TGNN weight file (model.cpp:134-185) and the Cora binary
(model.cpp:49-129).

* The oracle's restatement against the reference's known answers
  (test_graph_loader.cpp) and, where the compiled reference is present,
  against the reference itself on the same files: outputs bit for bit and
  error messages verbatim, over the known cases, edge cases of the field
  splitting and conversions, and seeded valid and corrupted files.
* The device parser's number conversions (csrc/numparse.hpp), compiled for
  the host, against the C library the reference converts with (glibc strtof
  / strtol through std::stof / std::stoi).
* The library's host-side readers of the weight file and the Cora binary
  (no device call) against the compiled reference.
"""
import os
import subprocess

import numpy as np
import pytest

import oracle
from csv_cases import (EDGE_ERRORS, EDGE_EXTRA, EDGE_KNOWN, FEATURE_ERRORS, FEATURE_EXTRA,
                       FEATURE_KNOWN, LOAD_KNOWN, corrupt, random_edges_csv,
                       random_features_csv)

needs_ref = pytest.mark.skipif(not oracle.has_reference(),
                               reason="compiled reference not built here")


def _edge_result(fn):
    try:
        s, d = fn()
        return ("ok", s.tolist(), d.tolist())
    except oracle.OracleError as e:
        return ("err", e.kind, str(e))


def _feat_result(fn):
    try:
        x = fn()
        return ("ok", x.shape, np.ascontiguousarray(x).view(np.int32).tobytes())
    except oracle.OracleError as e:
        return ("err", e.kind, str(e))


def test_edges_known_answers(restate):
    for name, text, exp in EDGE_KNOWN:
        src, dst = restate.parse_edges(text, name)
        assert src.shape[0] == exp["count"], name
        for k, (s, d) in exp["at"].items():
            assert (src[k], dst[k]) == (s, d), (name, k)


def test_features_known_answers(restate):
    for name, text, exp in FEATURE_KNOWN:
        x = restate.parse_features(text, name)
        assert x.shape == exp["shape"], name
        for (r, c), v in exp["at"].items():
            assert x[r, c] == np.float32(v), (name, r, c)


def test_error_messages(restate):
    for text, msg in EDGE_ERRORS:
        with pytest.raises(oracle.OracleError, match=msg.replace("(", r"\(")) as ei:
            restate.parse_edges(text, "f.csv")
        assert ei.value.kind == "runtime_error"
    for text, msg in FEATURE_ERRORS:
        with pytest.raises(oracle.OracleError, match=msg) as ei:
            restate.parse_features(text, "f.csv")
        assert ei.value.kind == "runtime_error"


def _fuzz_texts(seed: int):
    rng = np.random.default_rng(seed)
    edges, feats = [], []
    for i in range(12):
        e = random_edges_csv(rng, int(rng.integers(1, 300)), int(rng.integers(1, 50)),
                             header=bool(i % 2), crlf=bool(i % 3 == 0),
                             blank_every=int(rng.integers(0, 7)))
        edges.append(e)
        edges.append(corrupt(rng, e, int(rng.integers(1, 4))))
        f = random_features_csv(rng, int(rng.integers(1, 60)), int(rng.integers(1, 9)),
                                header=bool(i % 2), dup_frac=0.2 * (i % 3), gaps=bool(i % 4 == 0))
        feats.append(f)
        feats.append(corrupt(rng, f, int(rng.integers(1, 4))))
    return edges, feats


@needs_ref
def test_restatement_matches_reference(restate, reference, tmp_path):
    edges, feats = _fuzz_texts(2024)
    edges += [t for _, t, _ in EDGE_KNOWN] + [t for t, _ in EDGE_ERRORS] + EDGE_EXTRA
    feats += [t for _, t, _ in FEATURE_KNOWN] + [t for t, _ in FEATURE_ERRORS] + FEATURE_EXTRA
    p = str(tmp_path / "g.csv")
    for text in edges:
        open(p, "wb").write(text)
        assert _edge_result(lambda: restate.parse_edges(text, p)) == \
            _edge_result(lambda: reference.parse_edges_file(p)), text[:200]
    for text in feats:
        open(p, "wb").write(text)
        assert _feat_result(lambda: restate.parse_features(text, p)) == \
            _feat_result(lambda: reference.parse_features_file(p)), text[:200]
    # a missing file (the reference's open message; not part of the restatement)
    with pytest.raises(oracle.OracleError, match="GraphLoader: cannot open file"):
        reference.parse_edges_file(str(tmp_path / "missing.csv"))


@needs_ref
def test_load_known_answers(reference, tmp_path):
    for name, et, ft, exp in LOAD_KNOWN:
        ep, fp = str(tmp_path / "e.csv"), str(tmp_path / "f.csv")
        open(ep, "wb").write(et)
        open(fp, "wb").write(ft)
        adj, x, (n, e, f) = reference.load_graph(ep, fp)
        assert (n, e, f) == (exp["nodes"], exp["edges"], exp["features"]), name
        assert adj.nnz == exp["nnz"] and x.shape[0] == exp["rows"], name
        for (r, c), v in exp["at"].items():
            assert x[r, c] == np.float32(v), name


def test_numparse_matches_c_library():
    """numparse.hpp (the device parser's conversions) on the host against
    glibc strtof / strtol: random and adversarial strings (midpoints,
    subnormals, the tininess boundary, overflow, hex, inf / nan payloads)."""
    from tinygnn_amd import build
    exe = build.NUMPARSE_TEST
    if not os.path.exists(exe):
        pytest.skip("test_numparse not built")
    r = subprocess.run([exe, "60000", "31"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:]
    assert "0 mismatches" in r.stdout


# -- binary formats ----------------------------------------------------------
def write_cora(path, n, f, c, x, labels, masks, src, dst):
    """The Cora export layout read by load_cora_binary (model.cpp:49-129)."""
    with open(path, "wb") as fh:
        fh.write(np.array([n, f, c, len(src)], "<u4").tobytes())
        fh.write(np.ascontiguousarray(x, "<f4").tobytes())
        fh.write(np.ascontiguousarray(labels, "<i4").tobytes())
        for m in masks:
            fh.write(np.ascontiguousarray(m, np.uint8).tobytes())
        fh.write(np.ascontiguousarray(src, "<i4").tobytes())
        fh.write(np.ascontiguousarray(dst, "<i4").tobytes())


def synthetic_cora(seed=3, n=300, f=20, c=5, e=1500):
    rng = np.random.default_rng(seed)
    x = (rng.random((n, f)) < 0.1).astype(np.float32)
    labels = rng.integers(0, c, n).astype(np.int32)
    masks = [(rng.random(n) < p).astype(np.uint8) for p in (0.1, 0.2, 0.3)]
    src = rng.integers(0, n, e).astype(np.int32)
    dst = rng.integers(0, n, e).astype(np.int32)
    return n, f, c, x, labels, masks, src, dst


def _native_weights(path):
    import tinygnn_amd as tg
    try:
        w = tg.load_weight_file(path)
        return ("ok", np.float32(w.test_accuracy), {k: v.tobytes() for k, v in w.tensors.items()})
    except tg.TgError as ex:
        return ("err", ex.kind, str(ex))


def _ref_weights(reference, path):
    try:
        acc, t = reference.load_weight_file(path)
        return ("ok", np.float32(acc), {k: v.tobytes() for k, v in t.items()})
    except oracle.OracleError as ex:
        return ("err", ex.kind, str(ex))


@needs_ref
def test_weight_file_matches_reference(reference, tmp_path):
    """save_weight_file -> the reference's load_weight_file and the native
    reader agree (tensors, accuracy), and so do their errors."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(5)
    tensors = {"layer0.weight": rng.standard_normal((7, 3)).astype(np.float32),
               "layer0.bias": rng.standard_normal((1, 3)).astype(np.float32),
               "layer1.head0.attn_left": rng.standard_normal(4).astype(np.float32),
               "empty": np.zeros((0, 5), np.float32), "é": np.ones((2, 2), np.float32)}
    p = str(tmp_path / "w.bin")
    tg.save_weight_file(p, tensors, test_accuracy=0.8125)
    got, want = _native_weights(p), _ref_weights(reference, p)
    assert got == want
    assert got[2]["layer1.head0.attn_left"] == tensors["layer1.head0.attn_left"].tobytes()
    blob = open(p, "rb").read()
    broken = {"magic": b"TGNX" + blob[4:], "version": blob[:4] + b"\x02\x00\x00\x00" + blob[8:],
              "truncated": blob[:-3], "header_only": blob[:10], "empty": b""}
    for name, b in broken.items():
        q = str(tmp_path / f"{name}.bin")
        open(q, "wb").write(b)
        assert _native_weights(q) == _ref_weights(reference, q), name
    assert _native_weights(str(tmp_path / "none.bin")) == \
        _ref_weights(reference, str(tmp_path / "none.bin"))


@needs_ref
def test_cora_binary_host_side_matches_reference(reference, tmp_path):
    """The native reader's host half (sizes, labels, masks) against
    load_cora_binary; the device half is tested on the GPU."""
    import ctypes as C
    from tinygnn_amd import lib
    n, f, c, x, labels, masks, src, dst = synthetic_cora()
    p = str(tmp_path / "cora.bin")
    write_cora(p, n, f, c, x, labels, masks, src, dst)
    want = reference.load_cora(p)
    h = C.c_void_p()
    lib.check(lib.tg_cora_open(p.encode(), C.byref(h)))
    try:
        cnt = [C.c_int64() for _ in range(4)]
        lib.check(lib.tg_cora_info(h, *[C.byref(v) for v in cnt]))
        assert [v.value for v in cnt] == [want["num_nodes"], want["num_features"],
                                          want["num_classes"], want["num_edges"]]
        ptrs = [C.c_void_p() for _ in range(4)]
        lib.check(lib.tg_cora_host(h, *[C.byref(q) for q in ptrs]))
        np.testing.assert_array_equal(np.ctypeslib.as_array(C.cast(ptrs[0], C.POINTER(C.c_int32)),
                                                            (n,)), want["labels"])
        for q, key in zip(ptrs[1:], ("train_mask", "val_mask", "test_mask")):
            np.testing.assert_array_equal(
                np.ctypeslib.as_array(C.cast(q, C.POINTER(C.c_uint8)), (n,)), want[key])
    finally:
        lib.tg_cora_destroy(h)
    # truncated and missing files: the reference's messages
    open(p, "wb").write(open(p, "rb").read()[:-5])
    with pytest.raises(oracle.OracleError) as ei:
        reference.load_cora(p)
    h = C.c_void_p()
    rc = lib.tg_cora_open(p.encode(), C.byref(h))
    assert rc != 0 and lib.tg_last_error().decode() == str(ei.value)
    rc = lib.tg_cora_open(str(tmp_path / "nope.bin").encode(), C.byref(h))
    assert rc != 0 and lib.tg_last_error().decode() == \
        "load_cora_binary: cannot open " + str(tmp_path / "nope.bin")
