#!/usr/bin/env python3
"""Writes tests/golden/*.npz from the REAL reference, compiled from its own
sources by oracle/Makefile into oracle/_ref/libtgref.so.  The reference's
sources exist only in the development container, so the fixtures are
written there and committed.  The compiled library itself travels to the GPU
box with the rest of the tree (it is git-ignored, not gpurun-ignored), where
tests and bench.py load it as a checker and CPU baseline; nothing there
compiles or reads the reference's sources.

Fixtures (inputs are regenerated from tinygnn_amd.synth by seed; each fixture
stores the SHA-256 of the inputs it was made from so a drifted generator
fails loudly instead of comparing different data):

* cora_synth.npz -- configs A/B/C: the 2,708-node / 10,858-entry graph,
  its CSR (edge_list_to_csr), add_self_loops and gcn_norm outputs, and the
  outputs of the 2-layer GCN / SAGE-mean / GAT Model::forward (reference
  src/model.cpp:359-439; the caller's log_softmax, ops.cpp:565-606, is
  pinned by ops_small.npz).
* ops_small.npz -- small seeded cases for spmm, matmul, activations,
  add_bias, edge_softmax, gat_scores (F = 1..17, 41, 64, 100), the three
  layers, SAGE-max, and self-loop edge cases (existing / duplicate diagonal,
  empty rows).

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tinygnn_amd import synth  # noqa: E402

from golden_inputs import cora_inputs, ops_inputs  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def make_cora(ref) -> dict:
    inp = cora_inputs()
    out = {"input_sha": np.array(sha(inp["src"], inp["dst"], inp["x"],
                                     *[inp["weights"][k][1][n] for k in sorted(inp["weights"])
                                       for n in sorted(inp["weights"][k][1])]))}
    a = ref.edge_list_to_csr(inp["src"], inp["dst"], synth.CORA_NODES)
    out["row_ptr"], out["col_ind"] = a.row_ptr, a.col_ind
    sl = ref.add_self_loops(a)
    out["sl_row_ptr"], out["sl_col_ind"], out["sl_val"] = sl.row_ptr, sl.col_ind, sl.val
    gn = ref.gcn_norm(a)
    out["norm_val"] = gn.val
    for name, (spec, w) in inp["weights"].items():
        model = ref.model(spec, w)
        logits = model.forward(a, inp["x"])
        out[f"{name}_forward"] = logits
    return out


def make_ops(ref) -> dict:
    inp = ops_inputs()
    out = {"input_sha": np.array(sha(*[inp[k] for k in sorted(inp) if isinstance(inp[k],
                                                                               np.ndarray)]))}
    a = oracle.CSR(inp["a_n"].item(), inp["a_k"].item(), inp["a_rp"], inp["a_ci"], inp["a_v"])
    out["spmm"] = ref.spmm(a, inp["b"])
    out["matmul"] = ref.matmul(inp["ma"], inp["mb"])
    for kind in ("relu", "sigmoid", "tanh", "gelu", "softmax", "log_softmax"):
        out[f"act_{kind}"] = ref.activation(kind, inp["x"])
    out["act_leaky_relu"] = ref.activation("leaky_relu", inp["x"], 0.2)
    out["act_elu"] = ref.activation("elu", inp["x"], 1.0)
    out["add_bias"] = ref.add_bias(inp["x"], inp["bias_x"])
    sq = oracle.CSR(inp["s_n"].item(), inp["s_n"].item(), inp["s_rp"], inp["s_ci"], inp["s_v"])
    out["edge_softmax"] = ref.edge_softmax(sq).val
    sl = ref.add_self_loops(sq)
    out["sl_row_ptr"], out["sl_col_ind"], out["sl_val"] = sl.row_ptr, sl.col_ind, sl.val
    out["norm_val"] = ref.gcn_norm(sq).val
    # GAT scores via a single-head layer forward is not observable on its
    # own; pin them through layers of every width instead.
    n = sq.n_rows
    for f in inp["gat_widths"]:
        rng = np.random.default_rng(int(f))
        h = rng.standard_normal((n, 5)).astype(np.float32)
        w = rng.standard_normal((5, int(f))).astype(np.float32)
        al = rng.standard_normal((1, int(f))).astype(np.float32)
        ar = rng.standard_normal((1, int(f))).astype(np.float32)
        b = rng.standard_normal((1, int(f))).astype(np.float32)
        out[f"gat_f{f}"] = ref.gat_layer(sl, h, w, al, ar, b, 0.2, 1)
    h = inp["lh"]
    out["gcn_layer"] = ref.gcn_layer(ref.gcn_norm(sq), h, inp["lw"], inp["lb"], 1)
    out["sage_mean"] = ref.sage_layer(sq, h, inp["lw"], inp["lw2"], inp["lb"], 1, 0)
    out["sage_max"] = ref.sage_layer(sq, h, inp["lw"], inp["lw2"], inp["lb"], 0, 1)
    out["sage_max_aggregate"] = ref.sage_max_aggregate(sq, h)
    return out


def main():
    if not oracle.has_reference():
        sys.exit("oracle/_ref/libtgref.so is missing: run `make -C oracle` where the "
                 "reference sources are")
    ref = oracle.reference()
    np.savez_compressed(os.path.join(HERE, "cora_synth.npz"), **make_cora(ref))
    np.savez_compressed(os.path.join(HERE, "ops_small.npz"), **make_ops(ref))
    for f in ("cora_synth.npz", "ops_small.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
