"""Pins the oracle's codecs (cx_oracle.c) against the reference's own code,
closed forms and torch.  CPU only."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.oracle import BF16, FP16, fp8_decode_closed_form

GOLDEN = __import__("pathlib").Path(__file__).parent / "golden"


def test_fp8_decode_matches_closed_form(oracle):
    for code in range(256):
        assert oracle.fp8_lut[code] == np.float32(fp8_decode_closed_form(code)), code


def test_fp8_decode_matches_reference_lut_fixture(oracle):
    # DecodeFp8ByteV2(TORCH_E4M3FN, .) from the reference C++ (fp8_lut_v2.cc:47-66)
    ref = np.load(GOLDEN / "ref_fp8_lut.npy")
    assert np.array_equal(oracle.fp8_lut.view(np.uint32), ref.view(np.uint32))


def test_fp8_decode_matches_torch_except_nan_codes(oracle):
    codes = torch.arange(256, dtype=torch.uint8)
    tv = codes.view(torch.float8_e4m3fn).float().numpy()
    for c in range(256):
        if c in (0x7F, 0xFF):
            assert math.isnan(tv[c])                       # OCP: NaN
            assert oracle.fp8_lut[c] == (448.0 if c == 0x7F else -448.0)  # reference quirk
        else:
            assert tv[c] == oracle.fp8_lut[c], hex(c)


def test_fp8_quirk_codes_equal_their_canonical_neighbours(oracle):
    # the upload canonicalisation 0x7F->0x7E, 0xFF->0xFE preserves values
    assert oracle.fp8_lut[0x7F] == oracle.fp8_lut[0x7E] == 448.0
    assert oracle.fp8_lut[0xFF] == oracle.fp8_lut[0xFE] == -448.0


def test_fp8_encode_matches_torch_rne(oracle):
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.normal(0, 100, 4000), rng.normal(0, 1, 4000), rng.normal(0, 0.01, 2000),
        rng.uniform(-448, 448, 2000),
        # exact midpoints between representable values exercise ties-to-even
        (oracle.fp8_lut[1:0x7E].astype(np.float64) + oracle.fp8_lut[2:0x7F]) / 2,
        [0.0, -0.0, 448.0, -448.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11],
    ]).astype(np.float32)
    ours = oracle.fp8_encode(v)
    theirs = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)


def test_fp8_encode_saturates(oracle):
    assert oracle.fp8_encode(np.array([460.0, 1e6, -1e6], np.float32)).tolist() == [0x7E, 0x7E, 0xFE]


# --- activation codecs: reference KATs (test_activation_codec_v2.cc:26-84) ---
FP16_KAT = [(0x0000, 0.0), (0x8000, -0.0), (0x3C00, 1.0), (0xBC00, -1.0), (0x3800, 0.5),
            (0x3400, 0.25), (0x4000, 2.0)]
BF16_KAT = [(0x0000, 0.0), (0x8000, -0.0), (0x3F80, 1.0), (0xBF80, -1.0), (0x3F00, 0.5),
            (0x3E80, 0.25), (0x4000, 2.0)]


@pytest.mark.parametrize("bits,val", FP16_KAT)
def test_fp16_decode_kat(oracle, bits, val):
    got = oracle.L.cxo_fp16_decode(bits)
    assert got == val and math.copysign(1, got) == math.copysign(1, val)


@pytest.mark.parametrize("bits,val", BF16_KAT)
def test_bf16_decode_kat(oracle, bits, val):
    got = oracle.L.cxo_bf16_decode(bits)
    assert got == val and math.copysign(1, got) == math.copysign(1, val)


def test_fp16_decode_all_codes_vs_numpy(oracle):
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    ours = np.array([oracle.L.cxo_fp16_decode(int(c)) for c in codes[::7]], np.float32)
    r = ref[::7]
    finite = np.isfinite(r)
    assert np.array_equal(ours[finite].view(np.uint32), r[finite].view(np.uint32))


def test_rne_encoders_vs_numpy_and_torch(oracle):
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.normal(0, 3, 3000), rng.normal(0, 1e-5, 500),
                        [65504.0, 65520.0, 1e-8, 6.1e-5]]).astype(np.float32)
    f16 = oracle.encode_act(v, FP16, "rne")
    assert np.array_equal(f16, v.astype(np.float16).view(np.uint16))
    b16 = oracle.encode_act(v, BF16, "rne")
    assert np.array_equal(b16, torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


def test_reference_encoders_match_rne_on_sin_set(oracle, refcpu):
    # test_activation_codec_cuda_v2.cc:15-69: the reference's half-up CPU
    # encoder equals device RNE on x = sin(0.0005 i), i < 4096 (no ties).
    x = np.sin(np.float32(0.0005) * np.arange(4096, dtype=np.float32)).astype(np.float32)
    for dt in (FP16, BF16):
        ref_bits = np.array([refcpu.L.ref_encode(dt, float(a)) for a in x], np.uint16)
        assert np.array_equal(oracle.encode_act(x, dt, "ref"), ref_bits)
        assert np.array_equal(oracle.encode_act(x, dt, "rne"), ref_bits)


def test_reference_encoder_restatement_matches_reference(oracle, refcpu):
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.normal(0, 10, 2000), rng.normal(0, 1e-6, 200),
                        [65504.0, 70000.0, -0.0, 1e10, -1e10]]).astype(np.float32)
    for dt in (FP16, BF16):
        ref_bits = np.array([refcpu.L.ref_encode(dt, float(a)) for a in v], np.uint16)
        assert np.array_equal(oracle.encode_act(v, dt, "ref"), ref_bits)
