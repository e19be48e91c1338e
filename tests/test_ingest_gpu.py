"""Ingestion on the GPU: GraphLoader's CSV parsing (csrc/ingest.hip), the
Cora binary and the TGNN weight file (csrc/loaders.hip) against the CPU
oracle (tg_oracle.c) and, where present, the compiled reference.

Bar: edges bit-identical, features bit-identical (floats compared as bits),
errors with the reference's message for the same first failing line; from
one-line files to millions of lines, lines spanning many 1 KB windows, text
at unaligned device addresses, and files with planted defects.
"""
import os

import numpy as np
import pytest

import oracle
from csv_cases import (EDGE_ERRORS, EDGE_EXTRA, EDGE_KNOWN, FEATURE_ERRORS, FEATURE_EXTRA,
                       FEATURE_KNOWN, LOAD_KNOWN, corrupt, random_edges_csv,
                       random_features_csv)
from test_ingest_oracle import synthetic_cora, write_cora

pytestmark = pytest.mark.gpu
needs_ref = pytest.mark.skipif(not oracle.has_reference(),
                               reason="compiled reference not built here")


def _device_text(gpu, text: bytes, offset: int = 0):
    """text as a uint8 device tensor starting `offset` bytes past an aligned
    allocation (a contiguous view)."""
    buf = np.zeros(len(text) + offset + 1, np.uint8)
    buf[offset:offset + len(text)] = np.frombuffer(text, np.uint8)
    t = gpu.from_numpy(buf).cuda()
    return t[offset:offset + len(text)]


def _gpu_edges(gpu, text, name="f.csv", offset=0):
    import tinygnn_amd as tg
    try:
        c = tg.CsvText.from_device(_device_text(gpu, text, offset), name)
        s, d, _ = c.parse_edges()
        return ("ok", s.cpu().numpy().tolist(), d.cpu().numpy().tolist())
    except tg.TgError as e:
        return ("err", e.kind, str(e))


def _ora_edges(restate, text, name="f.csv"):
    try:
        s, d = restate.parse_edges(text, name)
        return ("ok", s.tolist(), d.tolist())
    except oracle.OracleError as e:
        return ("err", e.kind, str(e))


def _gpu_feats(gpu, text, name="f.csv", offset=0):
    import tinygnn_amd as tg
    try:
        c = tg.CsvText.from_device(_device_text(gpu, text, offset), name)
        x = c.parse_features().cpu().numpy()
        return ("ok", x.shape, np.ascontiguousarray(x).view(np.int32).tobytes())
    except tg.TgError as e:
        return ("err", e.kind, str(e))


def _ora_feats(restate, text, name="f.csv"):
    try:
        x = restate.parse_features(text, name)
        return ("ok", x.shape, np.ascontiguousarray(x).view(np.int32).tobytes())
    except oracle.OracleError as e:
        return ("err", e.kind, str(e))


def _fuzz(seed, n=16):
    rng = np.random.default_rng(seed)
    edges, feats = [], []
    for i in range(n):
        e = random_edges_csv(rng, int(rng.integers(1, 2000)), int(rng.integers(1, 5000)),
                             header=bool(i % 2), crlf=bool(i % 3 == 0),
                             blank_every=int(rng.integers(0, 9)))
        edges += [e, corrupt(rng, e, int(rng.integers(1, 5)))]
        f = random_features_csv(rng, int(rng.integers(1, 300)), int(rng.integers(1, 40)),
                                header=bool(i % 2), dup_frac=0.15 * (i % 3), gaps=bool(i % 4 == 0))
        feats += [f, corrupt(rng, f, int(rng.integers(1, 5)))]
    return edges, feats


def test_edges_match_oracle(gpu, restate):
    edges, _ = _fuzz(11)
    texts = ([t for _, t, _ in EDGE_KNOWN] + [t for t, _ in EDGE_ERRORS] + EDGE_EXTRA + edges)
    for k, text in enumerate(texts):
        print(f"edges case {k} ({len(text)} bytes)", flush=True)
        assert _gpu_edges(gpu, text) == _ora_edges(restate, text), text[:300]


def test_features_match_oracle(gpu, restate):
    _, feats = _fuzz(12)
    texts = ([t for _, t, _ in FEATURE_KNOWN] + [t for t, _ in FEATURE_ERRORS] + FEATURE_EXTRA +
             feats)
    for k, text in enumerate(texts):
        print(f"features case {k} ({len(text)} bytes)", flush=True)
        assert _gpu_feats(gpu, text) == _ora_feats(restate, text), text[:300]


def test_known_answers_on_device(gpu):
    import tinygnn_amd as tg
    for name, text, exp in EDGE_KNOWN:
        s, d, _ = tg.CsvText.from_device(_device_text(gpu, text), name).parse_edges()
        s, d = s.cpu().numpy(), d.cpu().numpy()
        assert s.shape[0] == exp["count"], name
        for k, (a, b) in exp["at"].items():
            assert (s[k], d[k]) == (a, b), name
    for name, text, exp in FEATURE_KNOWN:
        x = tg.CsvText.from_device(_device_text(gpu, text), name).parse_features().cpu().numpy()
        assert x.shape == exp["shape"], name
        for (r, c), v in exp["at"].items():
            assert x[r, c] == np.float32(v), name


def test_unaligned_text(gpu, restate):
    rng = np.random.default_rng(3)
    e = random_edges_csv(rng, 700, 90, header=True, crlf=True)
    f = random_features_csv(rng, 120, 17, header=True, dup_frac=0.1)
    for off in (1, 3, 7, 8, 13, 15):
        assert _gpu_edges(gpu, e, offset=off) == _ora_edges(restate, e), off
        assert _gpu_feats(gpu, f, offset=off) == _ora_feats(restate, f), off
        bad = corrupt(np.random.default_rng(off), f)
        assert _gpu_feats(gpu, bad, offset=off) == _ora_feats(restate, bad), off


def test_long_lines(gpu, restate):
    """Feature lines of 2,000-5,000 fields (many 1 KB windows per line), a
    bad field deep inside one, and a count mismatch on the last line."""
    rng = np.random.default_rng(8)
    f = random_features_csv(rng, 40, 3000, header=True)
    assert _gpu_feats(gpu, f) == _ora_feats(restate, f)
    lines = f.split(b"\n")
    fields = lines[17].split(b",")
    fields[2345] = b"1.5.5e"
    lines[17] = b",".join(fields)
    bad = b"\n".join(lines)
    assert _gpu_feats(gpu, bad) == _ora_feats(restate, bad)
    fields = lines[17].split(b",")
    fields[2345] = b"zz"
    lines[17] = b",".join(fields)
    bad = b"\n".join(lines)
    assert _gpu_feats(gpu, bad)[0] == "err"
    assert _gpu_feats(gpu, bad) == _ora_feats(restate, bad)
    short = f.rstrip(b"\n") + b",1\n"
    assert _gpu_feats(gpu, short) == _ora_feats(restate, short)


def test_large_files(gpu, restate, tmp_path):
    """Millions of edge lines and a 30,000 x 100 feature table through the
    file path (pinned staging, overlapped copies), then a planted defect near
    the end of each."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(21)
    n = 3_000_000
    s = rng.integers(0, 1_000_000, n)
    d = rng.integers(0, 1_000_000, n)
    text = ("src,dst\n" + "\n".join(f"{a},{b}" for a, b in zip(s.tolist(), d.tolist())) +
            "\n").encode()
    p = str(tmp_path / "edges.csv")
    open(p, "wb").write(text)
    gs, gd = tg.parse_edges(p)
    np.testing.assert_array_equal(gs.cpu().numpy(), s.astype(np.int32))
    np.testing.assert_array_equal(gd.cpu().numpy(), d.astype(np.int32))
    bad = text[:-40] + b"12,-4\n" + text[-40:]
    open(p, "wb").write(bad)
    with pytest.raises(tg.TgError) as ei:
        tg.parse_edges(p)
    with pytest.raises(oracle.OracleError) as eo:
        restate.parse_edges(bad, p)
    assert str(ei.value) == str(eo.value)
    f = random_features_csv(rng, 30_000, 100, header=True, dup_frac=0.05)
    q = str(tmp_path / "feat.csv")
    open(q, "wb").write(f)
    got = tg.parse_features(q).cpu().numpy()
    want = restate.parse_features(f, q)
    np.testing.assert_array_equal(got.view(np.int32), want.view(np.int32))
    badf = f[:-300] + b",x" + f[-300:]
    open(q, "wb").write(badf)
    with pytest.raises(tg.TgError) as ei:
        tg.parse_features(q)
    with pytest.raises(oracle.OracleError) as eo:
        restate.parse_features(badf, q)
    assert str(ei.value) == str(eo.value)


def test_file_errors(gpu, tmp_path):
    import tinygnn_amd as tg
    missing = str(tmp_path / "missing.csv")
    with pytest.raises(tg.TgError, match="GraphLoader: cannot open file '" + missing + "'"):
        tg.parse_edges(missing)
    with pytest.raises(tg.TgError, match="GraphLoader: cannot open file"):
        tg.parse_features(missing)
    p = str(tmp_path / "empty.csv")
    open(p, "wb").write(b"\n \r\n")
    with pytest.raises(tg.TgError, match="GraphLoader::parse_edges: file is empty: '" + p + "'"):
        tg.parse_edges(p)
    with pytest.raises(tg.TgError, match="GraphLoader::parse_features: file is empty"):
        tg.parse_features(p)


@needs_ref
def test_load_graph_matches_reference(gpu, reference, tmp_path):
    import tinygnn_amd as tg
    rng = np.random.default_rng(4)
    pairs = [(et, ft) for _, et, ft, _ in LOAD_KNOWN]
    pairs.append((random_edges_csv(rng, 5000, 700), random_features_csv(rng, 500, 12)))
    pairs.append((random_edges_csv(rng, 100, 50), random_features_csv(rng, 900, 3, gaps=True)))
    pairs.append((b"src,dst\n", random_features_csv(rng, 30, 4)))
    pairs.append((random_edges_csv(rng, 10, 5), b"0,1\n0,x\n"))
    ep, fp = str(tmp_path / "e.csv"), str(tmp_path / "f.csv")
    for et, ft in pairs:
        open(ep, "wb").write(et)
        open(fp, "wb").write(ft)
        try:
            adj, x, cnt = reference.load_graph(ep, fp)
        except oracle.OracleError as e:
            with pytest.raises(tg.TgError) as ei:
                tg.load_graph(ep, fp)
            assert str(ei.value) == str(e)
            continue
        g = tg.load_graph(ep, fp)
        assert (g.num_nodes, g.num_edges, g.num_features) == cnt
        rp, ci, v = g.adjacency.to_numpy()
        np.testing.assert_array_equal(rp, adj.row_ptr)
        np.testing.assert_array_equal(ci, adj.col_ind)
        np.testing.assert_array_equal(v.view(np.int32), adj.val.view(np.int32))
        np.testing.assert_array_equal(g.node_features.cpu().numpy().view(np.int32),
                                      x.view(np.int32))


@needs_ref
def test_cora_binary_matches_reference(gpu, reference, tmp_path):
    import tinygnn_amd as tg
    n, f, c, x, labels, masks, src, dst = synthetic_cora(seed=9, n=2708, f=143, c=7, e=10858)
    p = str(tmp_path / "cora.bin")
    write_cora(p, n, f, c, x, labels, masks, src, dst)
    want = reference.load_cora(p)
    got = tg.load_cora_binary(p)
    assert (got.num_nodes, got.num_features, got.num_classes, got.num_edges) == \
        (want["num_nodes"], want["num_features"], want["num_classes"], want["num_edges"])
    rp, ci, v = got.adjacency.to_numpy()
    np.testing.assert_array_equal(rp, want["adjacency"].row_ptr)
    np.testing.assert_array_equal(ci, want["adjacency"].col_ind)
    np.testing.assert_array_equal(v.view(np.int32), want["adjacency"].val.view(np.int32))
    np.testing.assert_array_equal(got.features.cpu().numpy().view(np.int32),
                                  want["features"].view(np.int32))
    np.testing.assert_array_equal(got.labels, want["labels"])
    for k in ("train_mask", "val_mask", "test_mask"):
        np.testing.assert_array_equal(getattr(got, k), want[k])
    # an out-of-range destination: the CSR validation message, at its sorted position
    dst2 = dst.copy()
    dst2[123] = n + 5
    write_cora(p, n, f, c, x, labels, masks, src, dst2)
    with pytest.raises(oracle.OracleError) as eo:
        reference.load_cora(p)
    with pytest.raises(tg.InvalidArgument) as ei:
        tg.load_cora_binary(p)
    assert str(ei.value) == str(eo.value)
    # an out-of-range source (undefined behaviour in the reference): an error here
    src2 = src.copy()
    src2[7] = -1
    write_cora(p, n, f, c, x, labels, masks, src2, dst)
    with pytest.raises(tg.InvalidArgument, match=r"load_cora_binary: edge\[7\].src = -1"):
        tg.load_cora_binary(p)


def test_model_load_weights_from_file(gpu, restate, tmp_path):
    """Model.load_weights(path) (model.cpp:252-255) equals loading the same
    tensors from a dict, and a file missing a tensor raises the reference's
    message."""
    import tinygnn_amd as tg
    from tinygnn_amd import synth
    from helpers import random_csr
    rng = np.random.default_rng(6)
    n = 400
    a = random_csr(rng, n, n, avg_deg=6)
    da = tg.DeviceCSR.from_numpy(n, n, a.row_ptr, a.col_ind, a.val)
    x = gpu.from_numpy(rng.standard_normal((n, 20)).astype(np.float32)).cuda()
    spec = synth.spec_gat(20, 8, 3, 5)
    w = synth.model_weights(spec, seed=2)
    p = str(tmp_path / "w.bin")
    tg.save_weight_file(p, w, test_accuracy=0.5)
    m1 = tg.Model.from_spec(spec, w)
    m2 = tg.Model.from_spec(spec)
    m2.load_weights(p)
    np.testing.assert_array_equal(m1.forward(da, x).cpu().numpy(), m2.forward(da, x).cpu().numpy())
    w.pop("layer1.head0.attn_right")
    tg.save_weight_file(p, w)
    with pytest.raises(tg.TgError, match="Model::load_weights: missing tensor "
                                         "'layer1.head0.attn_right'"):
        m2.load_weights(p)
