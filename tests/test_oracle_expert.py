"""Pins the oracle's expert MLP and CPU-baseline port.  CPU only.

Checks, each chosen so a plausible slip (transposed matrix, wrong scale index,
swapped gate/up, missing SiLU, dropped block scale) fails one of them:
  * bit-exact h and encoded y against the reference's RunExpertReferenceV2
    (golden fixtures written by tests/golden/make_golden.py from oracle/_ref);
  * float64 dequantise-then-MLP restatement (numpy, independent code);
  * closed forms on hand-built experts (identity-like weights);
  * the baseline port is bit-exact with the reference CPU backend.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle.oracle import BF16, FP16, dummy_expert_np, expert_f64, rel_l2

GOLDEN = Path(__file__).parent / "golden"


def test_dummy_restatement_equals_reference_fixture(refcpu):
    a = dummy_expert_np()
    b = refcpu.dummy_expert()
    for k in ("w_up", "w_gate", "w_down"):
        assert np.array_equal(a[k], b[k]), k
    for k in ("s_up", "s_gate", "s_down"):
        assert np.array_equal(a[k].ravel().view(np.uint32), b[k].ravel().view(np.uint32)), k


@pytest.mark.parametrize("name,dt", [("fp16", FP16), ("bf16", BF16)])
def test_oracle_bit_exact_vs_reference_kat(oracle, name, dt):
    g = np.load(GOLDEN / "dummy_kat.npz")
    ex = dummy_expert_np()
    x = oracle.decode_act(g[f"x_{name}"], dt)
    h, y = oracle.expert_ref(ex, x)
    assert np.array_equal(h[0].view(np.uint32), g[f"h_{name}"].view(np.uint32))
    assert np.array_equal(oracle.encode_act(y[0], dt, "ref"), g[f"y_{name}"])


def test_oracle_bit_exact_vs_reference_seeded(oracle):
    g = np.load(GOLDEN / "seeded_expert.npz")
    ex = oracle.gen_expert(int(g["seed"]), int(g["stream_base"]))
    x = oracle.decode_act(g["x_bf16"], BF16)
    h, y = oracle.expert_ref(ex, x)
    assert np.array_equal(h[0].view(np.uint32), g["h"].view(np.uint32))
    assert np.array_equal(oracle.encode_act(y[0], BF16, "ref"), g["y_bf16"])


def test_oracle_vs_float64_restatement(oracle):
    g = np.load(GOLDEN / "seeded_expert.npz")
    ex = oracle.gen_expert(int(g["seed"]), int(g["stream_base"]))
    x = oracle.decode_act(g["x_bf16"], BF16)
    h, y = oracle.expert_ref(ex, x)
    h64, y64 = expert_f64(ex, x, oracle.fp8_lut)
    assert rel_l2(h, h64) < 1e-5
    assert rel_l2(y, y64) < 1e-5


def _tiny_expert(hidden, inter, rb=1, cb=1):
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 256, size=(3, max(hidden, inter) ** 2), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # avoid the NaN-code quirk here
    ex = dict(w_up=codes[0][: inter * hidden].reshape(inter, hidden),
              w_gate=codes[1][: inter * hidden].reshape(inter, hidden),
              w_down=codes[2][: hidden * inter].reshape(hidden, inter),
              hidden=hidden, inter=inter, rb=rb, cb=cb)
    nu = ((inter + rb - 1) // rb, (hidden + cb - 1) // cb)
    nd = ((hidden + rb - 1) // rb, (inter + cb - 1) // cb)
    ex["s_up"] = rng.uniform(0.001, 0.01, nu).astype(np.float32)
    ex["s_gate"] = rng.uniform(0.001, 0.01, nu).astype(np.float32)
    ex["s_down"] = rng.uniform(0.001, 0.01, nd).astype(np.float32)
    return ex


@pytest.mark.parametrize("shape", [(8, 4, 1, 1), (256, 128, 128, 128), (96, 40, 32, 16)])
def test_oracle_small_shapes_vs_float64(oracle, shape):
    H, I, rb, cb = shape
    ex = _tiny_expert(H, I, rb, cb)
    x = np.random.default_rng(4).normal(0, 1, (3, H)).astype(np.float32)
    h, y = oracle.expert_ref(ex, x)
    h64, y64 = expert_f64(ex, x, oracle.fp8_lut)
    assert rel_l2(h, h64) < 1e-5 and rel_l2(y, y64) < 1e-5


def test_oracle_closed_form_single_nonzero_weights(oracle):
    # up = gate = 1.0 * s at one column, down = identity-like: y[r] = s_d * h[r%I]
    H, I = 8, 4
    ex = dict(w_up=np.zeros((I, H), np.uint8), w_gate=np.zeros((I, H), np.uint8),
              w_down=np.zeros((H, I), np.uint8), hidden=H, inter=I, rb=1, cb=1)
    one = 0x38  # e4m3fn 1.0
    for r in range(I):
        ex["w_up"][r, r] = one
        ex["w_gate"][r, r + 4] = one
    for r in range(H):
        ex["w_down"][r, r % I] = one
    ex["s_up"] = np.full((I, H), 2.0, np.float32)
    ex["s_gate"] = np.full((I, H), 0.5, np.float32)
    ex["s_down"] = np.full((H, I), 3.0, np.float32)
    x = np.arange(1, H + 1, dtype=np.float32) / 4
    h, y = oracle.expert_ref(ex, x)
    up = 2.0 * x[:I]
    gate = 0.5 * x[4:8]
    hh = gate / (1 + np.exp(-gate)) * up
    assert np.allclose(h[0], hh, rtol=1e-6)
    assert np.allclose(y[0], 3.0 * hh[np.arange(H) % I], rtol=1e-6)


@pytest.mark.parametrize("dt", [FP16, BF16])
def test_baseline_port_bit_exact_vs_reference_cpu_backend(oracle, refcpu, dt):
    ex = dummy_expert_np(hidden=1024, inter=256)
    _, xe = refcpu.dummy_input(1024, dt)
    ours = oracle.expert_cpu_baseline(ex, xe, dt, dt, threads=4)
    ce = refcpu.cpu_expert(ex)
    theirs = ce.run(xe, dt, dt, threads=4)
    ce.close()
    assert np.array_equal(ours, theirs)
