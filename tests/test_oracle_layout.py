"""Row-ownership mapping (common/kv_layout.h:26-57, kvc_common.h:81-89).

Three implementations must agree: the oracle's C restatement, kvx's
header include/kvx/kv_layout.h (compiled here with g++), and -- where the
reference is mounted -- the reference's own kv_layout.h compiled into
oracle/_ref/libkvref.so.  The known answers are the literals of the
reference's test/test_layout.py, kept in tests/golden/reference_kats.json.
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))["layout"]
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libkvref.so")


def test_layout_literals():
    for rows, n, want in KATS["per_layer_seg_rows"]:
        assert orc.per_layer_seg_rows(rows, n) == want
    for case in KATS["node_of"]:
        got = [orc.node_of(r, case["stripe"], case["nodes"]) for r in case["rows"]]
        assert got == case["expect"]
    for case in KATS["seg_row_of"]:
        got = [orc.seg_row_of(r, case["stripe"], case["nodes"]) for r in case["rows"]]
        assert got == case["expect"]
    cov = KATS["seg_row_cover"]
    seen = [orc.seg_row_of(r, cov["stripe"], cov["nodes"]) for r in range(cov["layer_rows"])]
    assert max(seen) == cov["max"]
    for v in range(cov["max"]):
        assert seen.count(v) == cov["each"]
    bal = KATS["balance"]
    for lo in bal["starts"]:
        nodes = [orc.node_of(r, bal["stripe"], bal["nodes"]) for r in range(lo, lo + bal["count"])]
        assert nodes.count(0) == bal["per_node"] and nodes.count(1) == bal["per_node"]
    for layer, row, s, n, plsr, rb, want in KATS["seg_offset"]:
        assert orc.seg_offset(layer, row, s, n, plsr, rb) == want
    for base, layer, row, s, n, plsr, rb, want in KATS["seg_addr"]:
        assert base + orc.seg_offset(layer, row, s, n, plsr, rb) == want


def test_validate_literals():
    # test_layout.py:52-59 calls validate(layer_num, layer_rows, row_bytes, stripe_rows, node_num)
    for layer_num, layer_rows, rb, s, n in KATS["validate_ok"]:
        assert orc.layout_validate(n, layer_num, layer_rows, orc.per_layer_seg_rows(layer_rows, n), rb, s) == 0
    for layer_num, layer_rows, rb, s, n in KATS["validate_bad"]:
        plsr = orc.per_layer_seg_rows(layer_rows, n) if n else 0
        assert orc.layout_validate(n, layer_num, layer_rows, plsr, rb, s) == -1
    # the C header also rejects a perLayerSegRows that is not ceil(rows/N) and N > 64
    assert orc.layout_validate(2, 2, 1024, 511, 1152, 1) == -1
    assert orc.layout_validate(65, 2, 1024, orc.per_layer_seg_rows(1024, 65), 1152, 1) == -1


_PROBE_SRC = r"""
#include <cstdio>
#include <cstdlib>
#include "kvx/kv_layout.h"
int main(int argc, char **argv) {
    unsigned S = (unsigned)atoi(argv[1]), N = (unsigned)atoi(argv[2]), rows = (unsigned)atoi(argv[3]);
    unsigned plsr = kvx_per_layer_seg_rows(rows, N);
    for (unsigned r = 0; r < rows; ++r)
        printf("%u %u %llu\n", kvx_node_of(r, S, N), kvx_seg_row_of(r, S, N),
               (unsigned long long)kvx_seg_offset(3, r, S, N, plsr, 1152));
    printf("%d %d\n", kvx_layout_validate(N, 2, rows, plsr, 1152, S), kvx_layout_validate(N, 2, rows, plsr, 1151, S));
    return 0;
}
"""


@pytest.fixture(scope="module")
def layout_probe(tmp_path_factory):
    d = tmp_path_factory.mktemp("layout")
    src = d / "probe.cpp"
    src.write_text(_PROBE_SRC)
    exe = d / "probe"
    subprocess.run(["g++", "-O1", "-std=c++17", "-I", os.path.join(ROOT, "include"), "-o", str(exe), str(src)],
                   check=True)
    return str(exe)


@pytest.mark.parametrize("S,N,rows", [(1, 2, 300), (1, 4, 257), (64, 4, 1000), (3, 7, 500), (0, 3, 50)])
def test_header_matches_oracle(layout_probe, S, N, rows):
    out = subprocess.run([layout_probe, str(S), str(N), str(rows)], check=True, capture_output=True,
                         text=True).stdout.split("\n")
    plsr = orc.per_layer_seg_rows(rows, N)
    for r in range(rows):
        node, seg_row, off = (int(x) for x in out[r].split())
        assert node == orc.node_of(r, S, N)
        assert seg_row == orc.seg_row_of(r, S, N)
        assert off == orc.seg_offset(3, r, S, N, plsr, 1152)
    ok, bad = (int(x) for x in out[rows].split())
    assert ok == orc.layout_validate(N, 2, rows, plsr, 1152, S)
    assert bad == -1


@pytest.mark.skipif(not os.path.exists(REF_LIB), reason="oracle/_ref not built (reference not mounted)")
def test_oracle_matches_reference_header():
    ref = ctypes.CDLL(REF_LIB)
    for f in ("kvref_per_layer_seg_rows", "kvref_node", "kvref_seg_row"):
        getattr(ref, f).restype = ctypes.c_uint32
        getattr(ref, f).argtypes = [ctypes.c_uint32] * (2 if f == "kvref_per_layer_seg_rows" else 3)
    ref.kvref_seg_offset.restype = ctypes.c_uint64
    ref.kvref_seg_offset.argtypes = [ctypes.c_uint32] * 6
    ref.kvref_validate.restype = ctypes.c_int
    ref.kvref_validate.argtypes = [ctypes.c_uint32] * 6
    rng = np.random.default_rng(5)
    for _ in range(2000):
        n = int(rng.integers(1, 65))
        s = int(rng.choice([1, 2, 3, 16, 64, 1000]))
        row = int(rng.integers(0, 1 << 32))
        layer = int(rng.integers(0, 128))
        rows = int(rng.integers(0, 1 << 22))
        plsr = orc.per_layer_seg_rows(rows, n)
        assert ref.kvref_per_layer_seg_rows(rows, n) == plsr
        assert ref.kvref_node(row, s, n) == orc.node_of(row, s, n)
        assert ref.kvref_seg_row(row, s, n) == orc.seg_row_of(row, s, n)
        assert ref.kvref_seg_offset(layer, row % (1 << 20), s, n, plsr, 1152) == \
            orc.seg_offset(layer, row % (1 << 20), s, n, plsr, 1152)
        rb = int(rng.choice([1152, 1151, 128, 0]))
        assert ref.kvref_validate(n, 2, rows, plsr, rb, s) == orc.layout_validate(n, 2, rows, plsr, rb, s)
