"""The GPU generator reproduces the CPU definition bit for bit, and the
hardware fp8 converter used by the kernels decodes every canonical code like
the reference table."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,name", [(torch.float32, "f32"), (torch.bfloat16, "bf16"),
                                        (torch.float16, "fp16")])
def test_gen_normal_bit_exact(gpu, oracle, dtype, name):
    print(f"[gen] normal {name}", flush=True)
    n = 100_003
    t = gpu.gen_normal(17, 5, (n,), 0.37, dtype)
    torch.cuda.synchronize()
    ref = oracle.gen_normal(17, 5, n, 0.37, name)
    got = t.cpu().view(torch.int32 if name == "f32" else torch.int16).numpy()
    assert np.array_equal(got.view(ref.dtype), ref)


def test_gen_fp8_matrix_bit_exact(gpu, oracle):
    print("[gen] fp8 matrix", flush=True)
    from constellation_amd.engine import Expert
    e = Expert.generate(0, 3, 0x44, hidden=1024, inter=384)
    try:
        ex = e.download()
        cpu = oracle.gen_expert(3, 0x44, hidden=1024, inter=384)
        for k in ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down"):
            assert np.array_equal(np.ascontiguousarray(ex[k]).view(np.uint8),
                                  np.ascontiguousarray(cpu[k]).view(np.uint8)), k
    finally:
        e.free()


def test_upload_canonicalises_nan_codes(gpu):
    print("[gen] canonicalise", flush=True)
    from constellation_amd.engine import Expert
    H, I = 512, 128
    codes = (np.arange(I * H) % 256).astype(np.uint8).reshape(I, H)
    s = np.ones((1, 4), np.float32)
    sd = np.ones((4, 1), np.float32)
    e = Expert.upload(0, codes, s, codes, s, codes.T.copy(), sd)
    try:
        back = e.download()["w_up"]
        exp = codes.copy()
        exp[exp == 0x7F] = 0x7E
        exp[exp == 0xFF] = 0xFE
        assert np.array_equal(back, exp)
    finally:
        e.free()
