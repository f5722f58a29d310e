"""ctypes binding of libcx_moe.so (the C ABI declared in include/cx_moe.h).

The library is loaded from the package directory only.  There is no fallback:
if it is missing, importing the engine raises, so a GPU run can never pass on
a silent CPU or PyTorch path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libcx_moe.so"

CX_OK = 0
CX_EINVAL = -1
CX_ENOMEM = -2
CX_EHIP = -3
CX_EUNSUPPORTED = -4
CX_EDEVICE = -5

CX_STATIC_SCRATCH_BYTES = 256 * 1024  # include/cx_moe.h

FP16, BF16, F32 = 1, 2, 3


class CxError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"cx error {code}: {msg}")
        self.code = code


class ExpertDesc(C.Structure):
    """cx_expert_desc: device-resident expert (plain device pointers)."""
    _fields_ = [
        ("w_up", C.c_void_p), ("s_up", C.c_void_p),
        ("w_gate", C.c_void_p), ("s_gate", C.c_void_p),
        ("w_down", C.c_void_p), ("s_down", C.c_void_p),
        ("hidden", C.c_int32), ("inter", C.c_int32),
        ("up_rb", C.c_int32), ("up_cb", C.c_int32),
        ("gate_rb", C.c_int32), ("gate_cb", C.c_int32),
        ("down_rb", C.c_int32), ("down_cb", C.c_int32),
        ("gu_layout", C.c_int32), ("reserved", C.c_int32 * 3),
    ]


class MoeLayerRequestInfo(C.Structure):
    """cx_moe_layer_request_info: header fields of a MoeLayerRequest body."""
    _fields_ = [
        ("layer_id", C.c_int32), ("batch_size", C.c_int32), ("hidden_dim", C.c_int32),
        ("top_k", C.c_int32), ("input_dtype", C.c_uint32), ("output_dtype", C.c_uint32),
        ("flags", C.c_uint32),
    ]


class DeviceInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char * 128), ("arch", C.c_char * 64),
        ("total_mem_bytes", C.c_uint64), ("free_mem_bytes", C.c_uint64),
        ("capability_flags", C.c_uint32), ("compute_units", C.c_int32),
        ("num_xcds", C.c_int32),
    ]


# name -> (restype, argtypes)
_P = C.c_void_p
_I = C.c_int
_SIGS = {
    "cx_last_error": (C.c_char_p, []),
    "cx_version": (C.c_char_p, []),
    "cx_device_count": (_I, [C.POINTER(_I)]),
    "cx_device_query": (_I, [_I, C.POINTER(DeviceInfo)]),
    "cx_upload_matrix": (_I, [_I, _P, C.c_uint64, C.c_uint64, _P, C.c_uint64,
                              C.POINTER(_P), C.POINTER(_P)]),
    "cx_upload_matrix_tiled": (_I, [_I, _P, C.c_uint64, C.c_uint64, _P, C.c_uint64,
                                    C.POINTER(_P), C.POINTER(_P)]),
    "cx_free_device": (_I, [_I, _P]),
    "cx_arena_stats": (_I, [_I, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "cx_ctx_create": (_I, [_I, C.POINTER(_P)]),
    "cx_ctx_destroy": (_I, [_P]),
    "cx_ctx_sync": (_I, [_P, _P]),
    "cx_ctx_profile": (_I, [_P, _I]),
    "cx_ctx_profile_read": (_I, [_P, C.c_char_p, C.POINTER(_I), C.POINTER(C.c_double)]),
    "cx_expert_run": (_I, [_P, C.POINTER(ExpertDesc), _P, _I, _I, _P, _I, _P, _P]),
    "cx_expert_run_static": (_I, [_I, C.POINTER(ExpertDesc), _P, _I, _I, _P, _I, _P, _P]),
    "cx_expert_run_host": (_I, [_P, C.POINTER(ExpertDesc), _P, C.c_size_t, _I, _I, _P,
                                C.c_size_t, _I]),
    "cx_layer_create": (_I, [_P, _I, C.POINTER(C.POINTER(ExpertDesc)), C.POINTER(ExpertDesc),
                             C.POINTER(_P)]),
    "cx_layer_destroy": (_I, [_P, _P]),
    "cx_route": (_I, [_P, _P, _I, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.c_float,
                      _P, _P, _P]),
    "cx_route_logits": (_I, [_P, _P, _I, _I, _P]),
    "cx_moe_decode": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _P, _I, _P, _P]),
    "cx_moe_prefill": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _P, _I, _P, _P]),
    "cx_moe_layer": (_I, [_P, _P, _P, _I, _I, _P, _I, _P, _P, _I, _I, _I, _I, C.c_float,
                          _P, _I, _P, _P, _P, _P]),
    "cx_moe_layer_request_peek": (_I, [_P, C.c_size_t, C.POINTER(MoeLayerRequestInfo)]),
    "cx_moe_layer_response_size": (C.c_size_t, [_I, _I]),
    "cx_moe_layer_request_run": (_I, [_P, _P, _P, C.c_size_t, _P, C.c_size_t,
                                      C.POINTER(C.c_size_t)]),
    "cx_gen_fp8_matrix": (_I, [_P, C.c_uint64, C.c_uint64, _I, _I, _I, _I, C.c_float, _P, _P,
                               _P]),
    "cx_gen_normal": (_I, [_P, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, _I, _P, _P]),
    "cx_gen_expert": (_I, [_I, C.c_uint64, C.c_uint64, _I, _I, _I, C.c_float,
                           C.POINTER(ExpertDesc)]),
    "cx_free_expert": (_I, [_I, C.POINTER(ExpertDesc)]),
}

EXPORTED = tuple(_SIGS)

_lib = None


def lib() -> C.CDLL:
    """Load libcx_moe.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m constellation_amd.build` "
                "(the engine has no CPU fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != CX_OK:
        msg = lib().cx_last_error()
        raise CxError(rc, msg.decode() if msg else "")
