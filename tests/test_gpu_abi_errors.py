"""Argument errors at the C ABI on a device (ctypes calls, no Python-side
checks in between): each entry point refuses a bad argument with its error
code and a message in cx_last_error, before any launch, and the context then
serves a valid call whose output equals a fresh context's.  The router's
messages follow the reference's ValueErrors (server/moe_layer_runtime.py:
250-319: "num_experts=... not divisible by n_group=...", "invalid
topk_group=...", "invalid top_k=...").
"""
from __future__ import annotations

import ctypes as C

import pytest
import torch

from constellation_amd._lib import BF16, CX_EINVAL, CX_OK, F32, FP16, lib

pytestmark = pytest.mark.gpu


def _expect(rc, code, text):
    assert rc == code, (rc, code, text)
    msg = lib().cx_last_error() or b""
    assert text.encode() in msg, msg


def test_expert_run_argument_errors(gpu):
    from constellation_amd.engine import Context, Expert
    print("[abi] cx_expert_run errors", flush=True)
    H, I, T = 1024, 512, 2
    e = Expert.generate(0, 140, 0x700, hidden=H, inter=I)
    try:
        x = gpu.gen_normal(141, 1, (T, H), 1.0, torch.bfloat16)
        y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        s = gpu.stream()
        L = lib()
        d = C.byref(e.desc)
        _expect(L.cx_expert_run(None, d, x.data_ptr(), BF16, T, y.data_ptr(), BF16, None, s),
                CX_EINVAL, "NULL context")
        _expect(L.cx_expert_run(gpu.handle, None, x.data_ptr(), BF16, T, y.data_ptr(), BF16, None, s),
                CX_EINVAL, "descriptor is NULL")
        _expect(L.cx_expert_run(gpu.handle, d, x.data_ptr(), BF16, 0, y.data_ptr(), BF16, None, s),
                CX_EINVAL, "bad n_tokens")
        _expect(L.cx_expert_run(gpu.handle, d, x.data_ptr(), F32, T, y.data_ptr(), BF16, None, s),
                CX_EINVAL, "dtypes must be fp16/bf16")
        _expect(L.cx_expert_run(gpu.handle, d, None, BF16, T, y.data_ptr(), BF16, None, s),
                CX_EINVAL, "NULL buffer")
        bad = type(e.desc).from_buffer_copy(e.desc)
        bad.down_rb = 0
        _expect(L.cx_expert_run(gpu.handle, C.byref(bad), x.data_ptr(), BF16, T, y.data_ptr(), BF16,
                                None, s), CX_EINVAL, "block sizes must be > 0")
        # the context still serves a valid call, equal to a fresh context's
        assert L.cx_expert_run(gpu.handle, d, x.data_ptr(), BF16, T, y.data_ptr(), BF16, None, s) == CX_OK
        with Context(0) as fresh:
            y0 = fresh.expert_run(e, x)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y0.view(torch.int16))
    finally:
        torch.cuda.synchronize()
        e.free()


def test_moe_entry_points_argument_errors(gpu):
    from constellation_amd.engine import Context, Expert, Layer
    print("[abi] cx_moe_* errors", flush=True)
    E, H, I, T, K = 32, 1024, 512, 3, 8
    experts = [Expert.generate(0, 142, 0x800 + 4 * i, hidden=H, inter=I) for i in range(E)]
    sh = Expert.generate(0, 142, 0x800 + 4 * E, hidden=H, inter=I)
    layer = Layer(gpu, experts, sh)
    try:
        x = gpu.gen_normal(143, 1, (T, H), 1.0, torch.bfloat16)
        w_r = gpu.gen_normal(143, 2, (E, H), 0.02, torch.bfloat16)
        bias = gpu.gen_normal(143, 3, (E,), 0.01, torch.float32)
        ids = torch.tensor([[0, 5, 9, 13, 17, 21, 25, 29]] * T, dtype=torch.int32, device="cuda")
        wts = torch.full((T, K), 0.125, dtype=torch.float32, device="cuda")
        y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        rid = torch.empty((T, K), dtype=torch.int32, device="cuda")
        rw = torch.empty((T, K), dtype=torch.float32, device="cuda")
        s = gpu.stream()
        L = lib()
        ctx, lay = gpu.handle, layer.handle

        def dec(fn, n=T, k=K, idp=ids.data_ptr(), odt=BF16, xp=x.data_ptr()):
            return fn(ctx, lay, xp, BF16, n, idp, wts.data_ptr(), k, y.data_ptr(), odt, None, s)

        for fn in (L.cx_moe_decode, L.cx_moe_prefill):
            _expect(dec(fn, n=0), CX_EINVAL, "bad n_tokens/top_k")
            _expect(dec(fn, k=65), CX_EINVAL, "bad n_tokens/top_k")
            _expect(dec(fn, idp=None), CX_EINVAL, "NULL buffer")
            _expect(dec(fn, xp=None), CX_EINVAL, "NULL buffer")
            _expect(dec(fn, odt=F32), CX_EINVAL, "dtypes must be fp16/bf16")
        _expect(L.cx_moe_decode(None, lay, x.data_ptr(), BF16, T, ids.data_ptr(), wts.data_ptr(), K,
                                y.data_ptr(), BF16, None, s), CX_EINVAL, "NULL context or layer")

        def lay_call(in_dt=BF16, n_group=8, topk_group=4, top_k=K, bp=bias.data_ptr()):
            return L.cx_moe_layer(ctx, lay, x.data_ptr(), in_dt, T, w_r.data_ptr(), BF16, bp, None,
                                  n_group, topk_group, top_k, 1, 2.5, y.data_ptr(), BF16, None,
                                  rid.data_ptr(), rw.data_ptr(), s)

        _expect(lay_call(in_dt=FP16), CX_EINVAL, "in_dtype must be bf16")
        _expect(lay_call(n_group=7), CX_EINVAL, "num_experts=32 not divisible by n_group=7")
        _expect(lay_call(topk_group=9), CX_EINVAL, "invalid topk_group=9 for n_group=8")
        _expect(lay_call(top_k=0), CX_EINVAL, "invalid top_k=0 for num_experts=32")
        _expect(lay_call(top_k=33), CX_EINVAL, "invalid top_k=33 for num_experts=32")
        _expect(lay_call(bp=None), CX_EINVAL, "NULL buffer")
        # valid calls on the same context equal a fresh context's
        assert lay_call() == CX_OK
        yl = y.clone()
        assert dec(L.cx_moe_decode) == CX_OK
        yd = y.clone()
        with Context(0) as fresh:
            y0, _, ids0, w0 = fresh.moe_layer(layer, x, w_r, bias, n_group=8, topk_group=4, top_k=K)
            yd0 = fresh.moe(layer, x, ids, wts)
        torch.cuda.synchronize()
        assert torch.equal(rid, ids0) and torch.equal(rw.view(torch.int32), w0.view(torch.int32))
        assert torch.equal(yl.view(torch.int16), y0.view(torch.int16))
        assert torch.equal(yd.view(torch.int16), yd0.view(torch.int16))
    finally:
        torch.cuda.synchronize()
        layer.close()
        for e in experts:
            e.free()
        sh.free()
