"""Seeded synthetic workloads for the benchmark configurations (A to E).

The reference ships no generator for these shapes, so these are this
package's own, fixed by seed and shared by the GPU path, the CPU oracle and
the benchmark:

* ``cora_synth``     -- 2,708 nodes; a Barabasi-Albert (m=2) graph topped up to
  exactly 5,429 undirected edges (10,858 directed CSR entries); 1,433-d
  Bernoulli(0.013) bag-of-words features, row-normalised.
* ``powerlaw_edges`` -- directed edge list with a discrete power-law
  out-degree (exponent, mean, clip) summing to an exact edge count and
  uniform destinations (never the source itself), in a shuffled order.
  Config D: 1,000,000 nodes, 50,000,000 edges, exponent 2.1, clip 20,000.
  Config E: 232,965 nodes, 114,615,892 edges (mean ~492), clip 20,000.
* ``glorot``         -- Glorot-uniform weights U(-a, a), a = sqrt(6/(fan_in+fan_out)).

All arrays are numpy; int32 indices, float32 values.
"""
from __future__ import annotations

import math

import numpy as np

CORA_NODES = 2708
CORA_UNDIRECTED_EDGES = 5429
CORA_FEATURES = 1433
CORA_CLASSES = 7

D_NODES = 1_000_000
D_EDGES = 50_000_000
E_NODES = 232_965
E_EDGES = 114_615_892
E_FEATURES = 602
E_CLASSES = 41


def _powerlaw_mean(xmin: float, alpha: float, dmax: int, u: np.ndarray) -> float:
    d = np.floor(xmin * (1.0 - u) ** (-1.0 / (alpha - 1.0)))
    return float(np.clip(d, 1, dmax).mean())


def powerlaw_degrees(n: int, total: int, alpha: float = 2.1, dmax: int = 20000,
                     seed: int = 0) -> np.ndarray:
    """Out-degrees of n nodes from a discrete power law with exponent alpha,
    clipped to [1, dmax], calibrated (x_min by bisection) and then adjusted by
    +-1 steps on random nodes so that they sum to exactly ``total``."""
    rng = np.random.default_rng(seed)
    u = rng.random(n)
    lo, hi = 0.5, float(dmax)
    for _ in range(60):
        mid = 0.5 * (lo + hi)
        if _powerlaw_mean(mid, alpha, dmax, u) * n < total:
            lo = mid
        else:
            hi = mid
    deg = np.clip(np.floor(hi * (1.0 - u) ** (-1.0 / (alpha - 1.0))), 1, dmax).astype(np.int64)
    diff = int(total - deg.sum())
    while diff != 0:
        idx = rng.integers(0, n, size=abs(diff))
        if diff > 0:
            ok = deg[idx] < dmax
            np.add.at(deg, idx[ok], 1)
        else:
            ok = deg[idx] > 1
            np.add.at(deg, idx[ok], -1)
            deg = np.maximum(deg, 1)
        diff = int(total - deg.sum())
    return deg.astype(np.int32)


def powerlaw_edges(n: int, total: int, alpha: float = 2.1, dmax: int = 20000,
                   seed: int = 0, shuffle: bool = True):
    """(src, dst) int32 arrays: power-law out-degrees, uniform destinations
    different from the source, duplicates possible, shuffled edge order."""
    deg = powerlaw_degrees(n, total, alpha, dmax, seed)
    rng = np.random.default_rng(seed + 1)
    src = np.repeat(np.arange(n, dtype=np.int32), deg)
    dst = rng.integers(0, n - 1, size=total, dtype=np.int32)
    dst += (dst >= src).astype(np.int32)  # skip the source: no self-loops
    if shuffle:
        perm = rng.permutation(total)
        src = src[perm]
        dst = dst[perm]
    return src, dst


def ba_edges(n: int, m: int, seed: int) -> set:
    """Undirected Barabasi-Albert edges (preferential attachment, m per node)."""
    rng = np.random.default_rng(seed)
    edges = set()
    targets = []  # multiset of endpoints (degree-proportional sampling)
    for i in range(m + 1):
        for j in range(i):
            edges.add((j, i))
            targets += [i, j]
    for v in range(m + 1, n):
        chosen = set()
        while len(chosen) < m:
            chosen.add(int(targets[int(rng.integers(0, len(targets)))]))
        for u in chosen:
            edges.add((min(u, v), max(u, v)))
            targets += [u, v]
    return edges


def cora_synth(seed: int = 2708):
    """(src, dst, X): 10,858 directed entries of 5,429 undirected edges and the
    2,708 x 1,433 row-normalised binary feature matrix."""
    n = CORA_NODES
    edges = ba_edges(n, 2, seed)
    rng = np.random.default_rng(seed + 7)
    while len(edges) < CORA_UNDIRECTED_EDGES:
        a, b = (int(x) for x in rng.integers(0, n, size=2))
        if a != b:
            edges.add((min(a, b), max(a, b)))
    assert len(edges) == CORA_UNDIRECTED_EDGES, len(edges)
    und = np.array(sorted(edges), dtype=np.int32)
    src = np.concatenate([und[:, 0], und[:, 1]]).astype(np.int32)
    dst = np.concatenate([und[:, 1], und[:, 0]]).astype(np.int32)
    x = (rng.random((n, CORA_FEATURES)) < 0.013).astype(np.float32)
    rs = x.sum(axis=1, keepdims=True)
    x = np.where(rs > 0, x / np.maximum(rs, 1), 0).astype(np.float32)
    return src, dst, x


def powerlaw_edges_device(torch, n: int, total: int, seed: int, device, alpha: float = 2.1,
                          dmax: int = 20000):
    """The benchmark's config-D / config-E edge list, drawn on the GPU:
    out-degrees from ``powerlaw_degrees(n, total, alpha, dmax, seed)`` (host),
    destinations uniform over the other nodes and a random edge order from a
    torch generator on ``device`` seeded with ``seed + 1``.  Returns int32
    device tensors ``(src, dst)`` of ``total`` entries; deterministic for a
    given seed and device type."""
    deg = powerlaw_degrees(n, total, alpha=alpha, dmax=dmax, seed=seed)
    g = torch.Generator(device=device)
    g.manual_seed(seed + 1)
    src = torch.repeat_interleave(torch.arange(n, dtype=torch.int32, device=device),
                                  torch.from_numpy(deg.astype(np.int64)).to(device))
    dst = torch.randint(0, n - 1, (total,), generator=g, device=device, dtype=torch.int32)
    dst += (dst >= src).to(torch.int32)  # no self-loops in the raw graph
    perm = torch.randperm(total, generator=g, device=device)
    src, dst = src[perm].contiguous(), dst[perm].contiguous()
    del perm
    return src, dst


def glorot(rng: np.random.Generator, fan_in: int, fan_out: int, shape=None) -> np.ndarray:
    a = math.sqrt(6.0 / (fan_in + fan_out))
    shape = shape or (fan_in, fan_out)
    return rng.uniform(-a, a, size=shape).astype(np.float32)


def model_weights(spec, seed: int = 0) -> dict:
    """Glorot weights (zero biases) named as Model::load_weights expects
    (reference include/tinygnn/model.hpp:131-135)."""
    rng = np.random.default_rng(seed)
    w = {}
    for li, l in enumerate(spec):
        p = f"layer{li}"
        fi, fo = l["in"], l["out"]
        if l["type"] == "gcn":
            w[p + ".weight"] = glorot(rng, fi, fo)
            w[p + ".bias"] = np.zeros((1, fo), np.float32)
        elif l["type"] == "sage":
            w[p + ".weight_neigh"] = glorot(rng, fi, fo)
            w[p + ".weight_self"] = glorot(rng, fi, fo)
            w[p + ".bias"] = np.zeros((1, fo), np.float32)
        elif l["type"] == "gat":
            for h in range(l.get("heads", 1)):
                hp = f"{p}.head{h}"
                w[hp + ".weight"] = glorot(rng, fi, fo)
                w[hp + ".attn_left"] = glorot(rng, fo, 1, shape=(1, fo))
                w[hp + ".attn_right"] = glorot(rng, fo, 1, shape=(1, fo))
                w[hp + ".bias"] = np.zeros((1, fo), np.float32)
    return w


# The benchmark model stacks (layer dicts as used by tinygnn_amd.Model and the
# oracle): act = layer activation, post = Model InterActivation.
def spec_gcn(f_in, hidden, classes):
    return [dict(type="gcn", **{"in": f_in}, out=hidden, act=1, post=0),
            dict(type="gcn", **{"in": hidden}, out=classes, act=0, post=0)]


def spec_sage(f_in, hidden, classes):
    return [dict(type="sage", **{"in": f_in}, out=hidden, act=1, post=0, agg=0),
            dict(type="sage", **{"in": hidden}, out=classes, act=0, post=0, agg=0)]


def spec_gat(f_in, hidden, heads, classes):
    return [dict(type="gat", **{"in": f_in}, out=hidden, heads=heads, concat=True, slope=0.2,
                 act=0, post=2),
            dict(type="gat", **{"in": hidden * heads}, out=classes, heads=1, concat=True,
                 slope=0.2, act=0, post=0)]


def cora_models() -> dict:
    """Configs A/B/C on the Cora-synth graph: name -> (spec, Glorot weights
    with zero biases), GCN 1433->16->7, SAGE-mean 1433->64->7, GAT 8 x 8
    concat + ELU -> 1 x 7 (the golden fixtures' seeds)."""
    f, c = CORA_FEATURES, CORA_CLASSES
    specs = {"gcn": spec_gcn(f, 16, c), "sage": spec_sage(f, 64, c), "gat": spec_gat(f, 8, 8, c)}
    return {k: (sp, model_weights(sp, seed=100 + i))
            for i, (k, sp) in enumerate(sorted(specs.items()))}


# ---------------------------------------------------------------------------
# CSV texts for the ingestion benchmark (GraphLoader's formats,
# graph_loader.hpp:26-35), generated with vectorised byte arithmetic.
# ---------------------------------------------------------------------------
def _digits(a):
    a = np.asarray(a, np.int64)
    nd = np.ones(a.shape, np.int64)
    t = a // 10
    while t.any():
        nd += t > 0
        t //= 10
    return nd


def edges_csv(src, dst, header: bool = True) -> bytes:
    """'src,dst' lines (non-negative ids, no padding), optional header.
    Built as fixed-width rows (right-aligned digits, NUL padding) and
    compacted by dropping the padding."""
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    n = src.shape[0]
    w = max(int(_digits(np.array([max(int(src.max(initial=0)), int(dst.max(initial=0)))]))[0]), 1)
    fixed = np.zeros((n, 2 * w + 2), np.uint8)
    top = max(int(src.max(initial=0)), int(dst.max(initial=0)))

    def right_aligned(a):  # (len(a), w) digits, NUL-padded on the left
        out = np.zeros((a.shape[0], w), np.uint8)
        v = a.copy()
        for k in range(w):
            out[:, w - 1 - k] = np.where((a >= 10 ** k) | (k == 0), v % 10 + 48, 0)
            v //= 10
        return out

    table = right_aligned(np.arange(top + 1, dtype=np.int64)) if top < (1 << 24) else None
    for a, col0 in ((src, 0), (dst, w + 1)):
        fixed[:, col0:col0 + w] = table[a] if table is not None else right_aligned(a)
    fixed[:, w] = ord(",")
    fixed[:, -1] = ord("\n")
    flat = fixed.ravel()
    head = b"src,dst\n" if header else b""
    return head + flat[flat != 0].tobytes()


def features_csv(n_rows: int, n_feat: int, seed: int = 0, header: bool = True):
    """A feature table of fixed-width fields: zero-padded 7-digit node ids
    (rows in random order) and values '-d.dddddd' / ' d.dddddd' (a leading
    space where there is no sign; the parser skips it).  Returns (text,
    values) with values[i] the row of node i as the decimal strings' exact
    integers k (value = k / 1e6)."""
    rng = np.random.default_rng(seed)
    k = rng.integers(-9_999_999, 10_000_000, size=(n_rows, n_feat), dtype=np.int64)
    order = rng.permutation(n_rows)
    w = 10  # ',' + sign + d + '.' + 6 digits
    row_len = 7 + n_feat * w + 1
    buf = np.empty((n_rows, row_len), np.uint8)
    ids = order.astype(np.int64)
    for j in range(7):
        buf[:, 6 - j] = (ids // 10 ** j % 10 + 48).astype(np.uint8)
    kk = k[order]
    mag = np.abs(kk)
    tok = buf[:, 7:7 + n_feat * w].reshape(n_rows, n_feat, w)
    tok[:, :, 0] = ord(",")
    tok[:, :, 1] = np.where(kk < 0, ord("-"), ord(" ")).astype(np.uint8)
    tok[:, :, 2] = (mag // 1_000_000 % 10 + 48).astype(np.uint8)
    tok[:, :, 3] = ord(".")
    for j in range(6):
        tok[:, :, 9 - j] = (mag // 10 ** j % 10 + 48).astype(np.uint8)
    buf[:, -1] = ord("\n")
    head = ("node_id," + ",".join(f"f{j}" for j in range(n_feat)) + "\n").encode() if header else b""
    return head + buf.tobytes(), k
