"""The synthetic-data generator's CPU definition (cx_oracle.c).  CPU only.
Its GPU twin is checked bit for bit in test_gpu_generator.py."""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).parent / "golden"


def test_normal_statistics(oracle):
    v = oracle.gen_normal(7, 3, 1 << 20, 1.0).astype(np.float64)
    assert abs(v.mean()) < 4e-3
    assert abs(v.std() - 1.0) < 4e-3
    kurt = ((v - v.mean()) ** 4).mean() / v.var() ** 2
    assert abs(kurt - 3.0) < 0.05
    # tail mass vs the Gaussian: P(|z| > 3) = 0.0027
    assert abs((np.abs(v) > 3).mean() - 0.0027) < 4e-4


def test_normal_is_deterministic_and_stream_separated(oracle):
    a = oracle.gen_normal(1, 2, 1000, 1.0)
    b = oracle.gen_normal(1, 2, 1000, 1.0)
    c = oracle.gen_normal(1, 3, 1000, 1.0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert not np.array_equal(a, c)
    assert abs(np.corrcoef(a, c)[0, 1]) < 0.1


def test_fp8_matrix_quantisation(oracle):
    rows, cols, blk = 256, 384, 128
    q, s = oracle.gen_fp8_matrix(5, 9, rows, cols, blk, blk, 0.02)
    v = oracle.gen_normal(5, 9, rows * cols, 0.02).reshape(rows, cols)
    for br in range(rows // blk):
        for bc in range(cols // blk):
            blkv = v[br * blk:(br + 1) * blk, bc * blk:(bc + 1) * blk]
            assert s[br, bc] == np.float32(np.abs(blkv).max() / np.float32(448.0))
            deq = oracle.fp8_lut[q[br * blk:(br + 1) * blk, bc * blk:(bc + 1) * blk]] * s[br, bc]
            # e4m3 RNE: relative error <= 2^-4 for normals, abs <= 2^-10*s for subnormals
            err = np.abs(deq - blkv)
            assert np.all(err <= np.maximum(np.abs(blkv) * 2.0 ** -4, s[br, bc] * 2.0 ** -10) * 1.0001)
            # the block max maps to +-448
            assert np.abs(oracle.fp8_lut[q[br * blk:(br + 1) * blk, bc * blk:(bc + 1) * blk]]).max() == 448.0


def test_generated_expert_matches_golden_checksums(oracle):
    g = np.load(GOLDEN / "seeded_expert.npz")
    ex = oracle.gen_expert(int(g["seed"]), int(g["stream_base"]))
    for k in ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down"):
        assert hashlib.sha256(np.ascontiguousarray(ex[k]).tobytes()).hexdigest() == str(g[f"sha_{k}"]), k
    x = oracle.gen_normal(int(g["seed"]), int(g["x_stream"]), 7168, 1.0, "bf16")
    assert np.array_equal(x, g["x_bf16"])
