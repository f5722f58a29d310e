"""Python-side handles over the C ABI, for torch (ROCm) device tensors.

PyTorch is used only for device memory and streams: every computation runs in
libcx_moe.so.  Calls are enqueued on torch's current stream of the tensors'
device.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np
import torch

from ._lib import (BF16, F32, FP16, CxError, DeviceInfo, ExpertDesc, MoeLayerRequestInfo, check,
                   lib)

_TORCH_TO_CX = {torch.float16: FP16, torch.bfloat16: BF16, torch.float32: F32}
_CX_TO_TORCH = {FP16: torch.float16, BF16: torch.bfloat16, F32: torch.float32}


def cx_dtype(t: torch.dtype) -> int:
    try:
        return _TORCH_TO_CX[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}") from None


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: int) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def device_count() -> int:
    n = C.c_int(0)
    check(lib().cx_device_count(C.byref(n)))
    return n.value


def device_info(device: int = 0) -> dict:
    info = DeviceInfo()
    check(lib().cx_device_query(device, C.byref(info)))
    return {
        "name": info.name.decode(), "arch": info.arch.decode(),
        "total_mem_bytes": info.total_mem_bytes, "free_mem_bytes": info.free_mem_bytes,
        "capability_flags": info.capability_flags, "compute_units": info.compute_units,
        "num_xcds": info.num_xcds,
    }


def arena_stats(device: int = 0) -> tuple[int, int]:
    u, r = C.c_uint64(0), C.c_uint64(0)
    check(lib().cx_arena_stats(device, C.byref(u), C.byref(r)))
    return u.value, r.value


LAYOUT_ROWS, LAYOUT_TILE16 = 0, 1  # cx_expert_desc::gu_layout


def untile16(a: np.ndarray) -> np.ndarray:
    """CX_LAYOUT_TILE16 bytes of a [rows, cols] matrix (as read back from the
    device, in a [rows, cols] array) in row-major order: tiles of 16 rows x
    128 columns in row-group, then column order; inside a tile, the 32 bytes
    of row r, columns 32q .. 32q + 31 at (16q + r) * 32."""
    rows, cols = a.shape
    t = a.reshape(rows // 16, cols // 128, 4, 16, 32)   # [row group][k-block][quarter][row][32 B]
    return np.ascontiguousarray(t.transpose(0, 3, 1, 2, 4)).reshape(rows, cols)


def tile16(a: np.ndarray) -> np.ndarray:
    """Row-major [rows, cols] bytes in CX_LAYOUT_TILE16 order (untile16's inverse)."""
    rows, cols = a.shape
    t = np.ascontiguousarray(a).reshape(rows // 16, 16, cols // 128, 4, 32)
    return np.ascontiguousarray(t.transpose(0, 2, 3, 1, 4)).reshape(rows, cols)


class Expert:
    """A device-resident fp8 expert living in the library's HBM arena."""

    def __init__(self, device: int, desc: ExpertDesc):
        self.device = device
        self.desc = desc
        self._live = True

    @classmethod
    def upload(cls, device: int, w_up, s_up, w_gate, s_gate, w_down, s_down, *,
               row_block: int = 128, col_block: int = 128, tiled: Optional[bool] = None) -> "Expert":
        """Upload host fp8 bytes + fp32 scale_inv (the UploadExpertAmdV2 path).
        Up and gate are re-tiled on the device (CX_LAYOUT_TILE16) when the
        shape allows, as the node's upload does; tiled=False keeps them
        row-major."""
        w_up, w_gate, w_down = (np.ascontiguousarray(a, np.uint8) for a in (w_up, w_gate, w_down))
        s_up, s_gate, s_down = (np.ascontiguousarray(a, np.float32) for a in (s_up, s_gate, s_down))
        inter, hidden = w_up.shape
        if w_gate.shape != (inter, hidden) or w_down.shape != (hidden, inter):
            raise ValueError("expert shapes must be up/gate [I,H] and down [H,I]")
        ok = inter % 16 == 0 and hidden % 128 == 0
        if tiled is None:
            tiled = ok
        elif tiled and not ok:
            raise ValueError("tiled gate/up needs inter % 16 == 0 and hidden % 128 == 0")
        ptrs = []
        try:
            for w, s, t in ((w_up, s_up, tiled), (w_gate, s_gate, tiled), (w_down, s_down, False)):
                dw, ds = C.c_void_p(), C.c_void_p()
                up = lib().cx_upload_matrix_tiled if t else lib().cx_upload_matrix
                check(up(device, w.ctypes.data, w.shape[0], w.shape[1], s.ctypes.data, s.size,
                         C.byref(dw), C.byref(ds)))
                ptrs += [dw.value, ds.value]
        except Exception:
            for p in ptrs:
                lib().cx_free_device(device, p)
            raise
        d = ExpertDesc(*ptrs, hidden, inter, row_block, col_block, row_block, col_block,
                       row_block, col_block, LAYOUT_TILE16 if tiled else LAYOUT_ROWS)
        return cls(device, d)

    @classmethod
    def generate(cls, device: int, seed: int, stream_base: int, hidden: int = 7168,
                 inter: int = 2048, block: int = 128, std: float = 0.02) -> "Expert":
        d = ExpertDesc()
        check(lib().cx_gen_expert(device, seed, stream_base, hidden, inter, block, std, C.byref(d)))
        return cls(device, d)

    @property
    def hidden(self) -> int:
        return self.desc.hidden

    @property
    def inter(self) -> int:
        return self.desc.inter

    def download(self) -> dict:
        """Copy the resident bytes back to host numpy arrays (for checks)."""
        H, I = self.hidden, self.inter
        out = {}
        specs = (("w_up", self.desc.w_up, (I, H), np.uint8, self.desc.up_rb, self.desc.up_cb),
                 ("s_up", self.desc.s_up, None, np.float32, self.desc.up_rb, self.desc.up_cb),
                 ("w_gate", self.desc.w_gate, (I, H), np.uint8, self.desc.gate_rb, self.desc.gate_cb),
                 ("s_gate", self.desc.s_gate, None, np.float32, self.desc.gate_rb, self.desc.gate_cb),
                 ("w_down", self.desc.w_down, (H, I), np.uint8, self.desc.down_rb, self.desc.down_cb),
                 ("s_down", self.desc.s_down, None, np.float32, self.desc.down_rb, self.desc.down_cb))
        for name, ptr, shape, dt, rb, cb in specs:
            if shape is None:
                rows, cols = (I, H) if name != "s_down" else (H, I)
                shape = ((rows + rb - 1) // rb, (cols + cb - 1) // cb)
            a = np.empty(shape, dt)
            _hip_d2h(a, ptr)
            if name in ("w_up", "w_gate") and self.desc.gu_layout == LAYOUT_TILE16:
                a = untile16(a)
            out[name] = a
        out.update(hidden=H, inter=I, rb=self.desc.up_rb, cb=self.desc.up_cb)
        return out

    def free(self) -> None:
        if self._live:
            check(lib().cx_free_expert(self.device, C.byref(self.desc)))
            self._live = False


def _hip_d2h(dst: np.ndarray, src_ptr: int) -> None:
    """hipMemcpy device->host through the HIP runtime already loaded by torch."""
    torch.cuda.synchronize()
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.restype = C.c_int
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    rc = hip.hipMemcpy(dst.ctypes.data, src_ptr, dst.nbytes, 2)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy D2H failed: {rc}")


class Layer:
    """Device table of resident experts (local ids 0..E-1) + optional shared expert."""

    def __init__(self, ctx: "Context", experts: Sequence[Optional[Expert]],
                 shared: Optional[Expert] = None):
        self.ctx = ctx
        self.n_experts = len(experts)
        self.experts = list(experts)
        self.shared = shared
        arr = (C.POINTER(ExpertDesc) * self.n_experts)()
        for i, e in enumerate(experts):
            arr[i] = C.pointer(e.desc) if e is not None else C.POINTER(ExpertDesc)()
        h = C.c_void_p()
        check(lib().cx_layer_create(ctx.handle, self.n_experts, arr,
                                    C.byref(shared.desc) if shared is not None else None,
                                    C.byref(h)))
        self.handle = h.value
        first = next(e for e in list(experts) + [shared] if e is not None)
        self.hidden, self.inter = first.hidden, first.inter

    def close(self) -> None:
        if self.handle:
            lib().cx_layer_destroy(self.ctx.handle, self.handle)
            self.handle = None


class Context:
    """One per device and worker thread (cx_ctx)."""

    def __init__(self, device: int = 0):
        self.device = device
        h = C.c_void_p()
        check(lib().cx_ctx_create(device, C.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            lib().cx_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def stream(self) -> int:
        return _stream(self.device)

    def sync(self) -> None:
        check(lib().cx_ctx_sync(self.handle, self.stream()))

    def profile(self, enable: bool) -> None:
        """Start (clearing totals) / stop per-kernel HIP-event timing."""
        check(lib().cx_ctx_profile(self.handle, int(enable)))

    def profile_read(self, kernel: str) -> tuple[int, float]:
        """(launches, summed ms) of one kernel since profiling started."""
        n, ms = C.c_int(0), C.c_double(0.0)
        check(lib().cx_ctx_profile_read(self.handle, kernel.encode(), C.byref(n), C.byref(ms)))
        return n.value, ms.value

    # -- single expert -----------------------------------------------------
    def expert_run(self, expert: Expert, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
                   want_f32: bool = False):
        x = x.contiguous()
        T = x.shape[0] if x.dim() == 2 else 1
        out_dtype = out_dtype or x.dtype
        y = torch.empty((T, expert.hidden), dtype=out_dtype, device=x.device)
        yf = torch.empty((T, expert.hidden), dtype=torch.float32, device=x.device) if want_f32 else None
        check(lib().cx_expert_run(self.handle, C.byref(expert.desc), x.data_ptr(), cx_dtype(x.dtype),
                                  T, y.data_ptr(), cx_dtype(out_dtype), _ptr(yf), self.stream()))
        return (y, yf) if want_f32 else y

    def expert_run_host(self, expert: Expert, x_bytes: bytes, in_dtype: int, n_tokens: int,
                        out_dtype: int) -> bytes:
        xb = np.frombuffer(x_bytes, np.uint8)
        out = np.empty(n_tokens * expert.hidden * 2, np.uint8)
        check(lib().cx_expert_run_host(self.handle, C.byref(expert.desc), xb.ctypes.data, xb.size,
                                       in_dtype, n_tokens, out.ctypes.data, out.size, out_dtype))
        return out.tobytes()

    # -- router --------------------------------------------------------------
    def route(self, x: torch.Tensor, w_router: torch.Tensor, bias: torch.Tensor, *,
              resident: Optional[torch.Tensor] = None, n_group: int = 8, topk_group: int = 4,
              top_k: int = 8, norm_topk_prob: bool = True, routed_scaling_factor: float = 2.5):
        x = x.contiguous()
        if x.dim() == 1:
            x = x.unsqueeze(0)
        T, H = x.shape
        E = w_router.shape[0]
        ids = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
        check(lib().cx_route(self.handle, x.data_ptr(), cx_dtype(x.dtype),
                             w_router.contiguous().data_ptr(), cx_dtype(w_router.dtype),
                             bias.contiguous().data_ptr(), _ptr(resident), T, H, E, n_group,
                             topk_group, top_k, int(norm_topk_prob), routed_scaling_factor,
                             ids.data_ptr(), w.data_ptr(), self.stream()))
        return ids, w

    def route_logits(self, n_tokens: int, n_experts: int, device) -> torch.Tensor:
        """fp64 router logits [n_tokens, n_experts] of the last route call."""
        out = torch.empty((n_tokens, n_experts), dtype=torch.float64, device=device)
        check(lib().cx_route_logits(self.handle, out.data_ptr(), n_tokens, n_experts,
                                    self.stream()))
        return out

    # -- grouped MoE -----------------------------------------------------------
    def moe(self, layer: Layer, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, *,
            out_dtype: Optional[torch.dtype] = None, want_f32: bool = False,
            prefill: Optional[bool] = None):
        x = x.contiguous()
        T = x.shape[0]
        K = topk_ids.shape[1] if topk_ids.dim() == 2 else 0
        out_dtype = out_dtype or x.dtype
        y = torch.empty((T, layer.hidden), dtype=out_dtype, device=x.device)
        yf = torch.empty((T, layer.hidden), dtype=torch.float32, device=x.device) if want_f32 else None
        if prefill is None:
            prefill = T > 16
        fn = lib().cx_moe_prefill if prefill else lib().cx_moe_decode
        ids = topk_ids.to(torch.int32).contiguous()
        w = topk_w.to(torch.float32).contiguous()
        check(fn(self.handle, layer.handle, x.data_ptr(), cx_dtype(x.dtype), T, ids.data_ptr(),
                 w.data_ptr(), K, y.data_ptr(), cx_dtype(out_dtype), _ptr(yf), self.stream()))
        return (y, yf) if want_f32 else y

    # -- whole-layer wire message (MoeLayerRequest / MoeLayerResponse) -------------
    def moe_layer_request(self, layer: Layer, body: bytes) -> bytes:
        """Runs one MoeLayerRequest body (host bytes, moe_layer_protocol) on
        `layer` and returns the MoeLayerResponse body (host bytes)."""
        info = MoeLayerRequestInfo()
        b = np.frombuffer(body, np.uint8)
        check(lib().cx_moe_layer_request_peek(b.ctypes.data, b.size, C.byref(info)))
        cap = lib().cx_moe_layer_response_size(info.batch_size, info.hidden_dim)
        out = np.empty(cap, np.uint8)
        n = C.c_size_t(0)
        check(lib().cx_moe_layer_request_run(self.handle, layer.handle, b.ctypes.data, b.size,
                                             out.ctypes.data, out.size, C.byref(n)))
        return out[:n.value].tobytes()

    def moe_layer(self, layer: Layer, x: torch.Tensor, w_router: torch.Tensor, bias: torch.Tensor, *,
                  resident: Optional[torch.Tensor] = None, n_group: int = 8, topk_group: int = 4,
                  top_k: int = 8, norm_topk_prob: bool = True, routed_scaling_factor: float = 2.5,
                  out_dtype: Optional[torch.dtype] = None, want_f32: bool = False, out=None):
        x = x.contiguous()
        T = x.shape[0]
        out_dtype = out_dtype or x.dtype
        if out is None:
            y = torch.empty((T, layer.hidden), dtype=out_dtype, device=x.device)
            yf = torch.empty((T, layer.hidden), dtype=torch.float32, device=x.device) if want_f32 else None
            ids = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
            w = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
        else:
            y, yf, ids, w = out
        check(lib().cx_moe_layer(self.handle, layer.handle, x.data_ptr(), cx_dtype(x.dtype), T,
                                 w_router.data_ptr(), cx_dtype(w_router.dtype), bias.data_ptr(),
                                 _ptr(resident), n_group, topk_group, top_k, int(norm_topk_prob),
                                 routed_scaling_factor, y.data_ptr(), cx_dtype(out_dtype), _ptr(yf),
                                 ids.data_ptr(), w.data_ptr(), self.stream()))
        return y, yf, ids, w

    # -- synthetic data ------------------------------------------------------
    def gen_normal(self, seed: int, stream_id: int, shape, std: float, dtype: torch.dtype):
        t = torch.empty(shape, dtype=dtype, device=f"cuda:{self.device}")
        check(lib().cx_gen_normal(self.handle, seed, stream_id, t.numel(), std, cx_dtype(dtype),
                                  t.data_ptr(), self.stream()))
        return t
