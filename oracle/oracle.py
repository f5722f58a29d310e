"""CPU oracle for the MoE expert path — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import this module, and only as the checker or the CPU baseline.
The product (constellation_amd/) never imports it.

Two layers:
  * ``Oracle`` wraps ``liboracle.so`` (cx_oracle.c, the C restatement of the
    reference's expert path, router and codecs; each C function cites the
    reference file:line it follows);
  * ``RefCpu`` wraps ``_ref/libcx_ref.so``: the reference's own C++ CPU expert
    sources compiled from /root/reference plus ref_shim.cc (present only where
    it was built).
plus float64 numpy restatements used to pin the C oracle independently.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libcx_ref.so"

_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")

FP16, BF16 = 1, 2


def build() -> None:
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def _load(path: Path) -> C.CDLL:
    if not path.exists():
        build()
    return C.CDLL(str(path))


class Oracle:
    """ctypes view of cx_oracle.c."""

    def __init__(self) -> None:
        L = _load(LIB_PATH)
        self.L = L
        L.cxo_fp8_decode.restype = C.c_float
        L.cxo_fp8_decode.argtypes = [C.c_uint8]
        L.cxo_fp8_encode.restype = C.c_uint8
        L.cxo_fp8_encode.argtypes = [C.c_float]
        for n in ("cxo_bf16_decode", "cxo_fp16_decode"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [C.c_uint16]
        for n in ("cxo_bf16_encode_ref", "cxo_bf16_encode_rne",
                  "cxo_fp16_encode_ref", "cxo_fp16_encode_rne"):
            getattr(L, n).restype = C.c_uint16
            getattr(L, n).argtypes = [C.c_float]
        L.cxo_rand64.restype = C.c_uint64
        L.cxo_rand64.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.cxo_normal.restype = C.c_float
        L.cxo_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.cxo_gen_normal_f32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, _f32p]
        L.cxo_gen_normal_bf16.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, _u16p]
        L.cxo_gen_normal_fp16.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, _u16p]
        L.cxo_gen_fp8_matrix.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_int, C.c_int,
                                         C.c_int, C.c_float, _u8p, _f32p]
        L.cxo_expert_ref.argtypes = [_u8p, _f32p, _u8p, _f32p, _u8p, _f32p, C.c_int, C.c_int,
                                     C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                     _f32p, C.c_int, _f32p, _f32p]
        L.cxo_expert_cpu_baseline.restype = C.c_int
        L.cxo_expert_cpu_baseline.argtypes = [_u8p, _f32p, _u8p, _f32p, _u8p, _f32p, C.c_int,
                                              C.c_int, C.c_int, C.c_int, _u16p, C.c_int, _u16p,
                                              C.c_int, _f32p, _f32p, C.c_int]
        L.cxo_route.restype = C.c_int
        L.cxo_route.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_int, C.c_double, _i32p, _f64p, _f64p,
                                C.c_void_p]
        # vectorised views of the scalar codecs
        self.fp8_lut = np.array([L.cxo_fp8_decode(i) for i in range(256)], dtype=np.float32)

    # -- codecs ------------------------------------------------------------
    def fp8_encode(self, v: np.ndarray) -> np.ndarray:
        f = self.L.cxo_fp8_encode
        return np.array([f(float(a)) for a in np.asarray(v, np.float32).ravel()],
                        dtype=np.uint8).reshape(np.shape(v))

    def decode_act(self, bits: np.ndarray, dtype: int) -> np.ndarray:
        bits = np.asarray(bits, np.uint16)
        if dtype == BF16:
            return (bits.astype(np.uint32) << 16).view(np.float32)
        return bits.view(np.float16).astype(np.float32)

    def encode_act(self, v: np.ndarray, dtype: int, mode: str = "rne") -> np.ndarray:
        """Encode fp32 -> fp16/bf16 bits; mode 'rne' or 'ref' (half-up)."""
        name = {(FP16, "rne"): "cxo_fp16_encode_rne", (FP16, "ref"): "cxo_fp16_encode_ref",
                (BF16, "rne"): "cxo_bf16_encode_rne", (BF16, "ref"): "cxo_bf16_encode_ref"}
        f = getattr(self.L, name[(dtype, mode)])
        v = np.asarray(v, np.float32)
        return np.array([f(float(a)) for a in v.ravel()], dtype=np.uint16).reshape(v.shape)

    # -- generator -----------------------------------------------------------
    def gen_normal(self, seed: int, stream: int, n: int, std: float, dtype: str = "f32"):
        if dtype == "f32":
            out = np.empty(n, np.float32)
            self.L.cxo_gen_normal_f32(seed, stream, n, std, out)
        else:
            out = np.empty(n, np.uint16)
            fn = self.L.cxo_gen_normal_bf16 if dtype == "bf16" else self.L.cxo_gen_normal_fp16
            fn(seed, stream, n, std, out)
        return out

    def gen_fp8_matrix(self, seed, stream, rows, cols, rb=128, cb=128, std=0.02):
        q = np.empty(rows * cols, np.uint8)
        s = np.empty(((rows + rb - 1) // rb) * ((cols + cb - 1) // cb), np.float32)
        self.L.cxo_gen_fp8_matrix(seed, stream, rows, cols, rb, cb, std, q, s)
        return q.reshape(rows, cols), s.reshape((rows + rb - 1) // rb, (cols + cb - 1) // cb)

    def gen_expert(self, seed, stream_base, hidden=7168, inter=2048, block=128, std=0.02):
        """Expert of the benchmark generator: streams base+0 up, +1 gate, +2 down."""
        wu, su = self.gen_fp8_matrix(seed, stream_base + 0, inter, hidden, block, block, std)
        wg, sg = self.gen_fp8_matrix(seed, stream_base + 1, inter, hidden, block, block, std)
        wd, sd = self.gen_fp8_matrix(seed, stream_base + 2, hidden, inter, block, block, std)
        return dict(w_up=wu, s_up=su, w_gate=wg, s_gate=sg, w_down=wd, s_down=sd,
                    hidden=hidden, inter=inter, rb=block, cb=block)

    # -- expert MLP ----------------------------------------------------------
    def expert_ref(self, ex: dict, x_f32: np.ndarray):
        """fp32 expert MLP in the reference order; returns (h [T,I], y [T,H])."""
        x = np.ascontiguousarray(np.atleast_2d(x_f32), np.float32)
        T = x.shape[0]
        H, I = ex["hidden"], ex["inter"]
        rb, cb = ex["rb"], ex["cb"]
        h = np.empty((T, I), np.float32)
        y = np.empty((T, H), np.float32)
        self.L.cxo_expert_ref(_c8(ex["w_up"]), _cf(ex["s_up"]), _c8(ex["w_gate"]), _cf(ex["s_gate"]),
                              _c8(ex["w_down"]), _cf(ex["s_down"]), H, I, rb, cb, rb, cb, rb, cb,
                              x, T, h, y)
        return h, y

    def expert_cpu_baseline(self, ex: dict, x_bits: np.ndarray, in_dtype: int, out_dtype: int,
                            threads: int = 12) -> np.ndarray:
        H, I = ex["hidden"], ex["inter"]
        y = np.empty(H, np.uint16)
        hs = np.empty(I, np.float32)
        xs = np.empty(H, np.float32)
        rc = self.L.cxo_expert_cpu_baseline(
            _c8(ex["w_up"]), _cf(ex["s_up"]), _c8(ex["w_gate"]), _cf(ex["s_gate"]),
            _c8(ex["w_down"]), _cf(ex["s_down"]), H, I, ex["rb"], ex["cb"],
            np.ascontiguousarray(x_bits, np.uint16), in_dtype, y, out_dtype, hs, xs, threads)
        assert rc == 0
        return y

    # -- router --------------------------------------------------------------
    def route(self, x: np.ndarray, w: np.ndarray, bias: np.ndarray, *, n_group=8, topk_group=4,
              top_k=8, norm=True, scale=2.5, resident=None):
        """fp64 router for one token; returns (ids, weights, margins, logits)."""
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        E, H = w.shape
        ids = np.full(top_k, -1, np.int32)
        wo = np.zeros(top_k, np.float64)
        margins = np.zeros(2, np.float64)
        logits = np.zeros(E, np.float64)
        res = None
        if resident is not None:
            res = np.ascontiguousarray(resident, np.uint8)
        k = self.L.cxo_route(x, w, np.ascontiguousarray(bias, np.float32),
                             None if res is None else res.ctypes.data, H, E, n_group, topk_group,
                             top_k, int(norm), scale, ids, wo, margins, logits.ctypes.data)
        if k < 0:
            raise RuntimeError(f"cxo_route failed: {k}")
        return ids[:k], wo[:k], margins, logits


def _c8(a):
    return np.ascontiguousarray(a, np.uint8).ravel()


def _cf(a):
    return np.ascontiguousarray(a, np.float32).ravel()


class RefCpu:
    """The reference's own CPU expert code (oracle/_ref), when built."""

    def __init__(self) -> None:
        if not REF_PATH.exists():
            build()
        if not REF_PATH.exists():
            raise FileNotFoundError(str(REF_PATH))
        L = C.CDLL(str(REF_PATH))
        self.L = L
        L.ref_fp8_decode.restype = C.c_float
        L.ref_fp8_decode.argtypes = [C.c_int, C.c_uint8]
        L.ref_encode.restype = C.c_uint16
        L.ref_encode.argtypes = [C.c_int, C.c_float]
        L.ref_decode.restype = C.c_float
        L.ref_decode.argtypes = [C.c_int, C.c_uint16]
        L.ref_fill_dummy.argtypes = [C.c_int] * 4 + [_u8p, _f32p, _u8p, _f32p, _u8p, _f32p]
        L.ref_fill_dummy_input.argtypes = [C.c_int, C.c_int, _f32p, _u16p]
        L.ref_expert_reference.restype = C.c_int
        L.ref_expert_reference.argtypes = [_u8p, _f32p, _u8p, _f32p, _u8p, _f32p, C.c_int, C.c_int,
                                           C.c_int, C.c_int, _u16p, C.c_int, C.c_int, _u16p, _f32p]
        L.ref_cpu_expert_create.restype = C.c_void_p
        L.ref_cpu_expert_create.argtypes = [_u8p, _f32p, _u8p, _f32p, _u8p, _f32p, C.c_int,
                                            C.c_int, C.c_int, C.c_int]
        L.ref_cpu_expert_run.restype = C.c_int
        L.ref_cpu_expert_run.argtypes = [C.c_void_p, _u16p, C.c_int, _u16p, C.c_int, C.c_int]
        L.ref_cpu_expert_destroy.argtypes = [C.c_void_p]

    @staticmethod
    def available() -> bool:
        return REF_PATH.exists()

    def dummy_expert(self, hidden=7168, inter=2048, rb=128, cb=128) -> dict:
        nub = ((inter + rb - 1) // rb) * ((hidden + cb - 1) // cb)
        ndb = ((hidden + rb - 1) // rb) * ((inter + cb - 1) // cb)
        wu = np.empty(inter * hidden, np.uint8)
        wg = np.empty(inter * hidden, np.uint8)
        wd = np.empty(hidden * inter, np.uint8)
        su = np.empty(nub, np.float32)
        sg = np.empty(nub, np.float32)
        sd = np.empty(ndb, np.float32)
        self.L.ref_fill_dummy(hidden, inter, rb, cb, wu, su, wg, sg, wd, sd)
        return dict(w_up=wu.reshape(inter, hidden), s_up=su, w_gate=wg.reshape(inter, hidden),
                    s_gate=sg, w_down=wd.reshape(hidden, inter), s_down=sd, hidden=hidden,
                    inter=inter, rb=rb, cb=cb)

    def dummy_input(self, hidden: int, dtype: int):
        xf = np.empty(hidden, np.float32)
        xe = np.empty(hidden, np.uint16)
        self.L.ref_fill_dummy_input(hidden, dtype, xf, xe)
        return xf, xe

    def expert_reference(self, ex: dict, x_bits, in_dtype: int, out_dtype: int):
        y = np.empty(ex["hidden"], np.uint16)
        h = np.empty(ex["inter"], np.float32)
        rc = self.L.ref_expert_reference(
            _c8(ex["w_up"]), _cf(ex["s_up"]), _c8(ex["w_gate"]), _cf(ex["s_gate"]),
            _c8(ex["w_down"]), _cf(ex["s_down"]), ex["hidden"], ex["inter"], ex["rb"], ex["cb"],
            np.ascontiguousarray(x_bits, np.uint16), in_dtype, out_dtype, y, h)
        if rc != 0:
            raise RuntimeError(f"ref_expert_reference rc={rc}")
        return y, h

    def cpu_expert(self, ex: dict):
        return _RefCpuExpert(self, ex)


class _RefCpuExpert:
    def __init__(self, ref: RefCpu, ex: dict) -> None:
        self.ref = ref
        self.hidden = ex["hidden"]
        self.h = ref.L.ref_cpu_expert_create(
            _c8(ex["w_up"]), _cf(ex["s_up"]), _c8(ex["w_gate"]), _cf(ex["s_gate"]),
            _c8(ex["w_down"]), _cf(ex["s_down"]), ex["hidden"], ex["inter"], ex["rb"], ex["cb"])
        if not self.h:
            raise RuntimeError("ref_cpu_expert_create failed")

    def run(self, x_bits, in_dtype: int, out_dtype: int, threads: int = 0) -> np.ndarray:
        y = np.empty(self.hidden, np.uint16)
        rc = self.ref.L.ref_cpu_expert_run(self.h, np.ascontiguousarray(x_bits, np.uint16),
                                           in_dtype, y, out_dtype, threads)
        if rc != 0:
            raise RuntimeError(f"ref_cpu_expert_run rc={rc}")
        return y

    def close(self) -> None:
        if self.h:
            self.ref.L.ref_cpu_expert_destroy(self.h)
            self.h = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# float64 numpy restatements (independent of the C code; used to pin it)
# ---------------------------------------------------------------------------

def fp8_decode_closed_form(code: int) -> float:
    """OCP e4m3fn from its definition (bias 7, subnormal m/8*2^-6), with the
    reference's 0x7F/0xFF -> +-448 rule (backend/fp8_lut_v2.cc:61)."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    if e == 15 and m == 7:
        return s * 448.0
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def dequant_f64(w: np.ndarray, s: np.ndarray, rb: int, cb: int, lut: np.ndarray) -> np.ndarray:
    """Blockwise dequant, server/fp8_utils.py:4-39 semantics, in float64."""
    w = np.asarray(w)
    rows, cols = w.shape
    s = np.asarray(s, np.float64).reshape((rows + rb - 1) // rb, (cols + cb - 1) // cb)
    full = np.repeat(np.repeat(s, rb, axis=0), cb, axis=1)[:rows, :cols]
    return lut.astype(np.float64)[w] * full


def expert_f64(ex: dict, x: np.ndarray, lut: np.ndarray):
    """Dequantise-then-MLP in float64 (the math the fp32 paths approximate)."""
    wu = dequant_f64(ex["w_up"], ex["s_up"], ex["rb"], ex["cb"], lut)
    wg = dequant_f64(ex["w_gate"], ex["s_gate"], ex["rb"], ex["cb"], lut)
    wd = dequant_f64(ex["w_down"], ex["s_down"], ex["rb"], ex["cb"], lut)
    x = np.atleast_2d(np.asarray(x, np.float64))
    g = x @ wg.T
    u = x @ wu.T
    h = g / (1.0 + np.exp(-g)) * u
    return h, h @ wd.T


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def dummy_expert_np(hidden: int = 7168, inter: int = 2048, rb: int = 128, cb: int = 128) -> dict:
    """FillDummyExpertBundleV2 (backend/dummy_expert_data_v2.cc:9-132) restated:
    bytes (i*7+3), (i*11+5), (i*13+17) mod 256 over the flat row-major index;
    scales 0.010+0.0005*rb+0.00005*cb (up), 0.020+0.0003*rb+0.00007*cb (gate),
    0.005+0.001*rb+0.0001*cb (down), evaluated in fp32 left to right."""
    f = np.float32

    def pattern(n, a, b):
        i = np.arange(n, dtype=np.uint64)
        return ((i * np.uint64(a) + np.uint64(b)) & np.uint64(0xFF)).astype(np.uint8)

    def scales(nr, nc, a, b, c):
        r = np.arange(nr, dtype=np.float32)[:, None]
        k = np.arange(nc, dtype=np.float32)[None, :]
        return ((f(a) + f(b) * r) + f(c) * k).astype(np.float32)

    nur, nuc = (inter + rb - 1) // rb, (hidden + cb - 1) // cb
    ndr, ndc = (hidden + rb - 1) // rb, (inter + cb - 1) // cb
    return dict(
        w_up=pattern(inter * hidden, 7, 3).reshape(inter, hidden),
        s_up=scales(nur, nuc, 0.010, 0.0005, 0.00005),
        w_gate=pattern(inter * hidden, 11, 5).reshape(inter, hidden),
        s_gate=scales(nur, nuc, 0.020, 0.0003, 0.00007),
        w_down=pattern(hidden * inter, 13, 17).reshape(hidden, inter),
        s_down=scales(ndr, ndc, 0.005, 0.001, 0.0001),
        hidden=hidden, inter=inter, rb=rb, cb=cb)
