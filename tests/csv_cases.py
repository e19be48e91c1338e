"""CSV inputs for the GraphLoader tests: the reference's own known answers
(tests/test_graph_loader.cpp of the reference) and seeded generators of
valid and broken files.

Known answers are (text, expected) pairs; expected is a list of (src, dst)
for edge files, a {(row, col): value} dict plus the shape for feature files,
or the error message substring the reference's tests assert (they assert
only the exception type; the messages come from graph_loader.cpp)."""
from __future__ import annotations

import numpy as np

# test_graph_loader.cpp:151-223
EDGE_KNOWN = [
    ("with_header",  # :151-172
     b"src,dst\n0,1\n0,2\n1,0\n1,3\n2,0\n2,3\n2,4\n3,1\n3,2\n4,2\n",
     {"count": 10, "at": {0: (0, 1), 1: (0, 2), 6: (2, 4), 9: (4, 2)}}),
    ("no_header", b"0,1\n1,2\n2,0\n", {"count": 3, "at": {0: (0, 1), 1: (1, 2), 2: (2, 0)}}),
    ("crlf", b"src,dst\r\n0, 1\r\n1 ,0\r\n", {"count": 2, "at": {0: (0, 1), 1: (1, 0)}}),
    ("single", b"5,10\n", {"count": 1, "at": {0: (5, 10)}}),
    ("self_loop", b"0,0\n1,1\n0,1\n", {"count": 3, "at": {0: (0, 0), 1: (1, 1)}}),
    ("trailing_blanks", b"0,1\n2,3\n\n\n", {"count": 2, "at": {}}),
    ("header_only", b"src,dst\n", {"count": 0, "at": {}}),  # :1624-1630
]

# test_graph_loader.cpp:228-323
FEATURE_KNOWN = [
    ("with_header",  # :228-249
     b"node_id,feat_0,feat_1,feat_2\n0,1.0,0.0,0.5\n1,0.0,1.0,0.0\n2,0.5,0.5,1.0\n"
     b"3,0.0,0.0,1.0\n4,1.0,1.0,0.0\n",
     {"shape": (5, 3), "at": {(0, 0): 1.0, (0, 2): 0.5, (2, 1): 0.5, (4, 0): 1.0, (4, 2): 0.0}}),
    ("no_header", b"0,1.0,2.0\n1,3.0,4.0\n",  # :252-265
     {"shape": (2, 2), "at": {(0, 0): 1.0, (0, 1): 2.0, (1, 0): 3.0, (1, 1): 4.0}}),
    ("sparse_ids", b"node_id,f0\n0,10.0\n5,50.0\n",  # :268-283
     {"shape": (6, 1), "at": {(0, 0): 10.0, (1, 0): 0.0, (2, 0): 0.0, (5, 0): 50.0}}),
    ("single", b"0,42.0\n", {"shape": (1, 1), "at": {(0, 0): 42.0}}),  # :286-293
    ("unordered", b"node_id,f0,f1\n3,30.0,31.0\n1,10.0,11.0\n0, 0.0, 1.0\n2,20.0,21.0\n",
     {"shape": (4, 2), "at": {(0, 0): 0.0, (0, 1): 1.0, (1, 0): 10.0, (3, 0): 30.0,
                              (3, 1): 31.0}}),  # :296-313
    ("negative_values", b"0,-1.5,2.5\n1,3.0,-4.0\n",  # :316-323
     {"shape": (2, 2), "at": {(0, 0): -1.5, (1, 1): -4.0}}),
]

# GraphLoader::load (test_graph_loader.cpp:508-548, 644-663)
LOAD_KNOWN = [
    ("small_graph", EDGE_KNOWN[0][1], FEATURE_KNOWN[0][1],
     {"nodes": 5, "edges": 10, "features": 3, "nnz": 10, "rows": 5, "at": {(2, 2): 1.0}}),
    ("edge_expands_features", b"0,5\n5,0\n", b"node_id,f0\n0,1.0\n1,2.0\n",
     {"nodes": 6, "edges": 2, "features": 1, "nnz": 2, "rows": 6,
      "at": {(0, 0): 1.0, (1, 0): 2.0, (5, 0): 0.0}}),
]

# test_graph_loader.cpp:1558-1640 (exception type only there; the messages
# are graph_loader.cpp's)
EDGE_ERRORS = [
    (b"", "file is empty"),
    (b"0 1\n", "malformed line 1: '0 1'"),
    (b"0,abc\n", "invalid integer on line 1: '0,abc'"),
    (b"-1,2\n", "negative node ID on line 1: src=-1, dst=2"),
]
FEATURE_ERRORS = [
    (b"-1,1.0,2.0\n", "negative node_id on line 1"),
    (b"0,1.0,2.0\n1,3.0\n", "inconsistent feature count on line 2: expected 2 but got 1"),
    (b"node_id,f0,f1\n", "no data rows in"),
    (b"", "file is empty"),
]

# Edge cases of the field splitting and conversions beyond the reference's tests.
EDGE_EXTRA = [
    b"  \n 5,7 \n", b"1,2,3\n4,5x\n", b"2147483647,0\n", b"2147483648,1\n", b"1,-0\n",
    b"1,2\n3\n", b"x,y\n1,2\n", b"_a,b\n1,2\n", b"1\t,\t2\n", b"\x0b7,8\n", b"+3,+4\n",
    b"00012,0003\n", b"1,2\r\n\r\n3,4", b"1,2\n,\n", b"1,\n", b"1,2\n3,4\n-5,6\n7,x\n",
    b"9,9\n" * 5 + b"1,99999999999999999999\n", b"4,5\x00junk\n6,7\n", b"1 2,3\n",
]
FEATURE_EXTRA = [
    b"0,1,2,\n1,3,4\n", b"0,,1\n", b"0\n", b"0,\n", b"x,1\n0,1\n", b"0,1e-40\n",
    b"0, 1.5 ,\t2\r\n1,nan,inf\n", b"3,1\n3,2\n", b"0,0x1.8p1,-0,1e38\n1,.5,5.,-.5e-3\n",
    b"0,1.5abc,2\n", b"0,1,2\n1,1\n2,x\n", b"0,1\n1,2,3\n", b"abc,1\n", b"a,1\nb,2\n",
    b"1.5,2\n", b" 7 ,1\n", b"0,3.4028235e38\n1,3.4028236e38\n", b"0,nan(0x123),-nan\n",
    b"0,1e-45\n", b"0,0x1p-149\n", b"0,16777217,33554435\n", b"2147483648,1\n",
    b"0,1\n0,2\n0,3\n", b"0,1,2\n\n\n1,3,4\n   \n", b",1\n", b"0,1\n,\n",
    b"0,1.0\n1,1.0,\n", b"0," + b"1," * 300 + b"1\n1," + b"2," * 300 + b"2\n",
]


def _float_token(rng) -> str:
    k = int(rng.integers(0, 12))
    v = float(rng.standard_normal() * 10.0 ** int(rng.integers(-8, 8)))
    if k == 0:
        return repr(v)
    if k == 1:
        return f"{v:.3f}"
    if k == 2:
        return f"{v:.9g}"
    if k == 3:
        return f"{v:e}"
    if k == 4:
        return str(int(rng.integers(-5, 6)))
    if k == 5:
        return float.hex(v)
    if k == 6:
        return f" {v:.5g}\t"
    if k == 7:
        return f"{v:.20e}"
    if k == 8:
        return f"{float(np.float32(v)):.9e}"
    if k == 9:
        return "0.0"
    if k == 10:
        return f"{v:.1f}"
    return f"{v:.17g}"


def random_edges_csv(rng, n_lines: int, n_nodes: int, header: bool = True, crlf: bool = False,
                     blank_every: int = 0) -> bytes:
    """A valid edge list with assorted spacing, optional header, CRLF and
    blank lines."""
    s = rng.integers(0, n_nodes, n_lines)
    d = rng.integers(0, n_nodes, n_lines)
    eol = "\r\n" if crlf else "\n"
    out = ["src,dst" + eol] if header else []
    for i in range(n_lines):
        sp = rng.integers(0, 6)
        if sp == 0:
            out.append(f" {s[i]} , {d[i]} {eol}")
        elif sp == 1:
            out.append(f"{s[i]},\t{d[i]}{eol}")
        else:
            out.append(f"{s[i]},{d[i]}{eol}")
        if blank_every and i % blank_every == 0:
            out.append("  " + eol)
    return "".join(out).encode()


def random_features_csv(rng, n_rows: int, n_feat: int, header: bool = True,
                        shuffle: bool = True, dup_frac: float = 0.0, gaps: bool = False) -> bytes:
    """A valid feature table with mixed float spellings, shuffled and
    optionally repeated / missing node ids."""
    ids = np.arange(n_rows)
    if gaps:
        ids = np.sort(rng.choice(n_rows * 2, n_rows, replace=False))
    if dup_frac:
        extra = rng.choice(ids, int(n_rows * dup_frac))
        ids = np.concatenate([ids, extra])
    if shuffle:
        rng.shuffle(ids)
    lines = []
    if header:
        lines.append("node_id," + ",".join(f"f{j}" for j in range(n_feat)))
    for i in ids:
        lines.append(str(int(i)) + "," + ",".join(_float_token(rng) for _ in range(n_feat)))
    return ("\n".join(lines) + "\n").encode()


def corrupt(rng, text: bytes, n: int = 1) -> bytes:
    """Plants n random defects (bad tokens, dropped commas, negative ids,
    extra fields) at random lines."""
    lines = text.split(b"\n")
    bad = [b"abc", b"", b"-3", b"1e99", b"1e-60", b"0x", b"nan(", b"--1", b" ", b"1,2,3", b"2147483648"]
    for _ in range(n):
        i = int(rng.integers(0, max(len(lines) - 1, 1)))
        fields = lines[i].split(b",")
        j = int(rng.integers(0, len(fields)))
        op = int(rng.integers(0, 3))
        if op == 0:
            fields[j] = bad[int(rng.integers(0, len(bad)))]
            lines[i] = b",".join(fields)
        elif op == 1:
            lines[i] = lines[i].replace(b",", b" ", 1)
        else:
            lines[i] = lines[i] + b",7"
    return b"\n".join(lines)
