"""libcx_moe.so loads and exports every entry point declared in
include/cx_moe.h; the ctypes binding covers the same set.  No GPU calls."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "cx_moe.h"


def header_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*CX_API\s+(?:const\s+)?\w+\s*\*?\s*(cx_\w+)\s*\(", text, flags=re.M))


def test_header_declares_expected_surface():
    fns = header_functions()
    for f in ("cx_route", "cx_moe_decode", "cx_moe_prefill", "cx_expert_run",
              "cx_expert_run_host", "cx_upload_matrix", "cx_free_device", "cx_ctx_create"):
        assert f in fns, f


def test_library_exports_every_declared_symbol():
    from constellation_amd._lib import LIB_PATH
    assert LIB_PATH.exists(), "libcx_moe.so not built (python -m constellation_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    missing = header_functions() - exported
    assert not missing, missing
    # nothing but the C ABI is exported
    extra = {s for s in exported if s.startswith("cx_")} - header_functions()
    assert not extra, extra


def test_ctypes_binding_matches_header():
    from constellation_amd._lib import EXPORTED
    assert set(EXPORTED) == header_functions()


def test_library_loads_without_gpu():
    import ctypes
    from constellation_amd._lib import lib
    L = lib()
    assert isinstance(L, ctypes.CDLL)
    assert b"gfx950" in L.cx_version()
