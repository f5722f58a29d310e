"""constellation_amd — MI355X (gfx950) engine for Constellation's routed-expert
MoE hot path: DeepSeek-V3 router, fp8 128x128 block-scaled expert MLPs
(grouped decode and prefill) and the weighted combine, behind the C ABI of
include/cx_moe.h (libcx_moe.so).

Python modules:
  _lib               ctypes binding of the C ABI (no fallback)
  engine             torch-tensor handles: Context, Expert, Layer
  moe_layer_runtime  route_token_real / route_tokens: the server's router API
                     (server/moe_layer_runtime.py:232-408) on the HIP router

C++ (backend_amd/): the expert_node_v2 AMD backend plugin (upload/free,
GPU info, BackendWorkspaceAmdV2) over the same C ABI.
  build              hipcc build of libcx_moe.so
"""
from ._lib import BF16, F32, FP16, CxError, EXPORTED, LIB_PATH  # noqa: F401

__all__ = ["BF16", "F32", "FP16", "CxError", "EXPORTED", "LIB_PATH"]
