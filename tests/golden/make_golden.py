"""Writes the golden fixtures of tests/golden from the reference's own C++
(oracle/_ref/libcx_ref.so: expert_reference_v2.cc, dummy_expert_data_v2.cc,
fp8_lut_v2.cc and activation_codec_v2.h compiled from /root/reference).

    python tests/golden/make_golden.py

Fixtures (inputs and expected outputs only):
  ref_fp8_lut.npy     DecodeFp8ByteV2(TORCH_E4M3FN, 0..255)         (fp8_lut_v2.cc:47-66)
  dummy_kat.npz       reference KAT: dummy bundle + sin input, fp16 and bf16,
                      RunExpertReferenceV2 outputs (y bits, h fp32)  (expert_reference_v2.cc:146-178)
  seeded_expert.npz   config-0 expert from this repo's generator (seed 1234,
                      stream base 0x100): weight checksums, x bf16, reference y/h
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.oracle import BF16, FP16, Oracle, RefCpu  # noqa: E402

OUT = Path(__file__).resolve().parent

SEED, STREAM_BASE, X_STREAM = 1234, 0x100, 0x900


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> None:
    ref = RefCpu()
    o = Oracle()
    lut = np.array([ref.L.ref_fp8_decode(2, i) for i in range(256)], np.float32)
    np.save(OUT / "ref_fp8_lut.npy", lut)

    ex = ref.dummy_expert()
    d = {}
    for name, dt in (("fp16", FP16), ("bf16", BF16)):
        _, xe = ref.dummy_input(7168, dt)
        y, h = ref.expert_reference(ex, xe, dt, dt)
        d[f"x_{name}"] = xe
        d[f"y_{name}"] = y
        d[f"h_{name}"] = h
    np.savez_compressed(OUT / "dummy_kat.npz", **d)

    sx = o.gen_expert(SEED, STREAM_BASE)
    x = o.gen_normal(SEED, X_STREAM, 7168, 1.0, "bf16")
    y, h = ref.expert_reference(sx, x, BF16, BF16)
    np.savez_compressed(
        OUT / "seeded_expert.npz", seed=SEED, stream_base=STREAM_BASE, x_stream=X_STREAM,
        x_bf16=x, y_bf16=y, h=h,
        sha_w_up=sha(sx["w_up"]), sha_w_gate=sha(sx["w_gate"]), sha_w_down=sha(sx["w_down"]),
        sha_s_up=sha(sx["s_up"]), sha_s_gate=sha(sx["s_gate"]), sha_s_down=sha(sx["s_down"]))
    print("wrote", sorted(p.name for p in OUT.glob("*.np*")))


if __name__ == "__main__":
    main()
