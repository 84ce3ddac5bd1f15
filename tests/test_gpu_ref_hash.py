"""The oracle's dropout hash against the reference's own hash, compiled from its
source lines (reference @ None: csrc/flash_attn_v100/fa_common.cuh:21-38) by
oracle/build_ref.py into oracle/_ref/libfa2ref_hash.so and run on the GPU.

This pins what the published-algorithm checks in test_oracle.py leave open:
which index takes which multiplier, the +1 offsets, and the fp32 threshold
compare, over 2^20 + edge (seed, row, col, bh, p) tuples.  Planted mistakes in
the oracle (row and col multipliers swapped, a dropped +1, a mistyped seed
multiplier, row and col exchanged) must disagree with the reference bits.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import fa2_oracle as orc

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "oracle", "_ref", "libfa2ref_hash.so")

pytestmark = pytest.mark.gpu


def _lib():
    if not os.path.exists(LIB):
        pytest.skip("oracle/_ref/libfa2ref_hash.so not built (the reference tree was absent at build time)")
    lib = ctypes.CDLL(LIB)
    P = ctypes.c_void_p
    lib.fa2ref_dropout_keep.argtypes = [P, P, P, P, P, P, ctypes.c_int64]
    lib.fa2ref_hash_u32.argtypes = [P, P, ctypes.c_int64]
    return lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _tuples(n=1 << 20, seed=7):
    rng = np.random.default_rng(seed)
    s = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    row = rng.integers(0, 70000, size=n).astype(np.int32)
    col = rng.integers(0, 70000, size=n).astype(np.int32)
    bh = rng.integers(0, 1 << 16, size=n).astype(np.uint32)
    # a quarter of the rows / cols over the whole 24-bit range, and edge values
    q = n // 4
    row[:q] = rng.integers(0, 1 << 24, size=q)
    col[q:2 * q] = rng.integers(0, 1 << 24, size=q)
    edge = np.array([0, 1, 63, 64, 65, 127, 128, 4095, 4096, 65535, (1 << 24) - 1], np.int32)
    row[:edge.size * edge.size] = np.repeat(edge, edge.size)
    col[:edge.size * edge.size] = np.tile(edge, edge.size)
    s[:4] = [0, 1, 0xFFFFFFFF, 0x80000000]
    bh[:3] = [0, 95, 0xFFFF]
    # p: fixed values including the smallest steps around 0 and 1, and random ones
    fixed = np.array([0.0, 2.0 ** -24, 0.1, 1 / 3, 0.5, 0.9, 1 - 2.0 ** -24, 0.999999], np.float32)
    p = rng.random(n, dtype=np.float32)
    p[: n // 2] = fixed[rng.integers(0, fixed.size, size=n // 2)]
    return s, row, col, bh, p


def _ref_keep(lib, s, row, col, bh, p):
    out = np.zeros(s.size, np.uint8)
    rc = lib.fa2ref_dropout_keep(_ptr(s), _ptr(row), _ptr(col), _ptr(bh), _ptr(p), _ptr(out), s.size)
    assert rc == 0, f"hip error {rc}"
    return out.astype(bool)


def _keep_from_hash(h, p):
    return (h >> np.uint64(8)).astype(np.float32) * np.float32(1.0 / 16777216.0) >= p


def test_oracle_keep_equals_reference_keep():
    lib = _lib()
    s, row, col, bh, p = _tuples()
    ref = _ref_keep(lib, s, row, col, bh, p)
    mine = orc.dropout_keep(s, row, col, bh, p)
    assert mine.shape == ref.shape
    print(f"{ref.size} tuples, keep rate {ref.mean():.4f}, mismatches {(mine != ref).sum()}", flush=True)
    assert np.array_equal(mine, ref)


def test_oracle_finaliser_equals_reference_hash_u32():
    lib = _lib()
    x = np.random.default_rng(3).integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x[:3] = [0, 1, 0xFFFFFFFF]
    out = np.zeros_like(x)
    assert lib.fa2ref_hash_u32(_ptr(x), _ptr(out), x.size) == 0
    assert np.array_equal(orc.hash_u32(x).astype(np.uint32), out)


def test_planted_wiring_mistakes_disagree_with_reference():
    lib = _lib()
    s, row, col, bh, p = _tuples(n=1 << 18, seed=11)
    p = np.full_like(p, 0.5)   # every wrong bit shows with probability 1/2
    ref = _ref_keep(lib, s, row, col, bh, p)
    R, C = orc.DROP_ROW_MUL, orc.DROP_COL_MUL
    variants = {
        "row/col multipliers swapped": orc.dropout_hash(s, row, col, bh, muls=(orc.DROP_SEED_MUL, C, R, orc.DROP_BH_MUL)),
        "row +1 dropped": orc.dropout_hash(s, row.astype(np.int64) - 1, col, bh),
        "col +1 dropped": orc.dropout_hash(s, row, col.astype(np.int64) - 1, bh),
        "bh +1 dropped": orc.dropout_hash(s, row, col, bh.astype(np.int64) - 1),
        "seed multiplier 0x9E3779B9": orc.dropout_hash(s, row, col, bh, muls=(0x9E3779B9, R, C, orc.DROP_BH_MUL)),
        "row and col exchanged": orc.dropout_hash(s, col, row, bh),
    }
    for name, h in variants.items():
        frac = (_keep_from_hash(h, p) != ref).mean()
        assert frac > 0.4, f"planted mistake not caught: {name} ({frac:.3f})"
    assert np.array_equal(_keep_from_hash(orc.dropout_hash(s, row, col, bh), p), ref)
