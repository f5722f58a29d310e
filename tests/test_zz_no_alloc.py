"""The allocation-free single-expert entry point (cx_expert_run_static) against
cx_expert_run, through the C ABI.

cx_expert_run_static runs the same kernels with the library's static device
scratch instead of the context's grown buffers, so its outputs must equal
cx_expert_run's bit for bit (cx_expert_run is itself held to the oracle by
tests/test_gpu_expert.py; one case here is also checked against the oracle).
Two calls in a row, the second smaller, cover reuse of the shared array.
The file is named to be collected last: it also has to pass after every
other GPU test has run in the same process.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from oracle.oracle import BF16, FP16, rel_l2

pytestmark = pytest.mark.gpu
TDT = {FP16: torch.float16, BF16: torch.bfloat16}


def _run_static(e, x: torch.Tensor, out_dt: int):
    from constellation_amd._lib import lib
    from constellation_amd.engine import cx_dtype
    T = x.shape[0]
    y = torch.empty((T, e.hidden), dtype=TDT[out_dt], device=x.device)
    yf = torch.empty((T, e.hidden), dtype=torch.float32, device=x.device)
    rc = lib().cx_expert_run_static(0, C.byref(e.desc), x.data_ptr(), cx_dtype(x.dtype), T,
                                    y.data_ptr(), out_dt, yf.data_ptr(),
                                    torch.cuda.current_stream(0).cuda_stream)
    return rc, y, yf


def _run_ctx(gpu, e, x, out_dt):
    return gpu.expert_run(e, x, out_dtype=TDT[out_dt], want_f32=True)


@pytest.mark.parametrize("in_dt,out_dt", [(BF16, BF16), (FP16, FP16)])
def test_static_matches_context_path_full_size(gpu, in_dt, out_dt):
    """DeepSeek-V3 expert (7168 x 2048): the tile path (8 tokens) and then the
    small k-part path (3 tokens), back to back on the shared array."""
    from constellation_amd._lib import CX_OK
    from constellation_amd.engine import Expert
    print(f"[no_alloc] full size in={in_dt} out={out_dt}", flush=True)
    e = Expert.generate(0, 77, 0x500)
    try:
        x = gpu.gen_normal(77, 0x5F0, (8, 7168), 1.0, TDT[in_dt])
        for T in (8, 3):
            xt = x[:T].contiguous()
            y0, yf0 = _run_ctx(gpu, e, xt, out_dt)
            rc, y1, yf1 = _run_static(e, xt, out_dt)
            assert rc == CX_OK
            torch.cuda.synchronize()
            assert torch.equal(yf0, yf1), T
            assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), T
    finally:
        e.free()


def test_static_against_oracle_and_repeat(gpu, oracle):
    """Reduced dims, checked against the CPU oracle; then a second, smaller
    call and a repeat of the first, each equal to the context path."""
    from constellation_amd._lib import CX_OK
    from constellation_amd.engine import Expert
    print("[no_alloc] oracle 1024x512", flush=True)
    H, I = 1024, 512
    e = Expert.generate(0, 78, 0x540, hidden=H, inter=I)
    try:
        x = gpu.gen_normal(78, 0x5F1, (20, H), 1.0, torch.bfloat16)
        cpu = oracle.gen_expert(78, 0x540, H, I)
        for T in (20, 2, 20):
            xt = x[:T].contiguous()
            rc, y1, yf1 = _run_static(e, xt, BF16)
            assert rc == CX_OK
            y0, yf0 = _run_ctx(gpu, e, xt, BF16)
            torch.cuda.synchronize()
            assert torch.equal(yf0, yf1) and torch.equal(y0.view(torch.int16), y1.view(torch.int16))
            _, ref = oracle.expert_ref(cpu, xt.float().cpu().numpy())
            assert rel_l2(yf1.cpu().numpy(), ref) < 1e-5
    finally:
        e.free()


def test_static_generic_block_path(gpu, oracle):
    """1x1 blocks (the reference's control-test geometry) take the generic
    kernels, whose fp32 h also lives in the static array."""
    from constellation_amd._lib import CX_OK
    from constellation_amd.engine import Expert
    print("[no_alloc] generic 1x1 blocks", flush=True)
    rng = np.random.default_rng(5)
    H, I = 64, 32
    ex = {
        "w_up": rng.integers(0, 0x7E, (I, H), dtype=np.uint8),
        "w_gate": rng.integers(0, 0x7E, (I, H), dtype=np.uint8),
        "w_down": rng.integers(0, 0x7E, (H, I), dtype=np.uint8),
        "s_up": rng.uniform(1e-3, 2e-3, (I, H)).astype(np.float32),
        "s_gate": rng.uniform(1e-3, 2e-3, (I, H)).astype(np.float32),
        "s_down": rng.uniform(1e-3, 2e-3, (H, I)).astype(np.float32),
    }
    e = Expert.upload(0, ex["w_up"], ex["s_up"], ex["w_gate"], ex["s_gate"], ex["w_down"],
                      ex["s_down"], row_block=1, col_block=1)
    try:
        x = gpu.gen_normal(79, 1, (3, H), 1.0, torch.float16)
        rc, y1, yf1 = _run_static(e, x, FP16)
        assert rc == CX_OK
        y0, yf0 = _run_ctx(gpu, e, x, FP16)
        torch.cuda.synchronize()
        assert torch.equal(yf0, yf1) and torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    finally:
        e.free()


def test_static_rejects_oversize(gpu):
    """Beyond the static array: a clear CX_EINVAL, nothing launched."""
    from constellation_amd._lib import CX_EINVAL, CX_OK, lib
    from constellation_amd.engine import Expert
    print("[no_alloc] size limit", flush=True)
    e = Expert.generate(0, 80, 0x580)
    try:
        x = gpu.gen_normal(80, 1, (33, 7168), 1.0, torch.bfloat16)
        # exactly at the limit: 32 tokens x inter 2048 fill the array (h_lo
        # ends on its last byte); the output must still equal the context path
        x32 = x[:32].contiguous()
        rc, y1, yf1 = _run_static(e, x32, BF16)
        assert rc == CX_OK
        y0, yf0 = _run_ctx(gpu, e, x32, BF16)
        torch.cuda.synchronize()
        assert torch.equal(yf0, yf1) and torch.equal(y0.view(torch.int16), y1.view(torch.int16))
        rc, _, _ = _run_static(e, x, BF16)
        assert rc == CX_EINVAL
        assert b"static" in lib().cx_last_error()
        torch.cuda.synchronize()
    finally:
        e.free()


@pytest.mark.parametrize("T", [1, 8])
def test_static_under_graph_capture(gpu, T):
    """One cx_expert_run_static call captured into a HIP graph (kernel
    launches only: the first, eager call has looked up the static array),
    replayed three times on new inputs with eager work and syncs between the
    replays; every replay equals cx_expert_run bit for bit.  T = 1 takes the
    k-part path, T = 8 the tile path."""
    from constellation_amd._lib import CX_OK
    from constellation_amd.engine import Expert
    print(f"[no_alloc] graph capture T={T}", flush=True)
    e = Expert.generate(0, 81, 0x5C0)
    try:
        xs = [gpu.gen_normal(81, 0x600 + i, (T, 7168), 1.0, torch.bfloat16) for i in range(4)]
        x = xs[0].clone()
        rc, y, yf = _run_static(e, x, BF16)  # eager warm-up on the same buffers
        assert rc == CX_OK
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side, capture_error_mode="thread_local"):
                from constellation_amd._lib import lib
                from constellation_amd.engine import cx_dtype
                rc = lib().cx_expert_run_static(0, C.byref(e.desc), x.data_ptr(), cx_dtype(x.dtype),
                                                T, y.data_ptr(), BF16, yf.data_ptr(),
                                                side.cuda_stream)
        assert rc == CX_OK
        for i in range(1, 4):
            x.copy_(xs[i])
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            y0, yf0 = _run_ctx(gpu, e, xs[i], BF16)
            torch.cuda.synchronize()
            assert torch.equal(yf0, yf), i
            assert torch.equal(y0.view(torch.int16), y.view(torch.int16)), i
        del g
    finally:
        torch.cuda.synchronize()
        e.free()
