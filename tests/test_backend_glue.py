"""The expert-node backend glue (constellation_amd/backend_amd/) compiles as a
drop-in for the reference's AMD stubs.

The glue files replace expert_node_v2/backend/amd/* of the reference tree.
This test puts them in front of the reference's own headers on the include
path (an overlay directory of symlinks; nothing is copied) and compiles every
translation unit with the reference's flags (expert_node_v2/build.py:
-std=c++20, CUDA off).  Skipped when the reference tree is not mounted.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
REF = Path(os.environ.get("CX_REFERENCE_ROOT", "/root/reference"))
GLUE = REPO / "constellation_amd" / "backend_amd"

pytestmark = pytest.mark.skipif(
    not (REF / "expert_node_v2" / "expert_format_v2.h").exists() or shutil.which("g++") is None,
    reason="reference tree or g++ not available")


def _overlay(tmp_path: Path) -> Path:
    amd = tmp_path / "overlay" / "expert_node_v2" / "backend" / "amd"
    amd.mkdir(parents=True)
    for h in GLUE.glob("*.h"):
        (amd / h.name).symlink_to(h)
    return tmp_path / "overlay"


@pytest.mark.parametrize("src", sorted(p.name for p in GLUE.glob("*.cc")))
def test_glue_compiles_against_reference_headers(tmp_path, src):
    ov = _overlay(tmp_path)
    cmd = ["g++", "-std=c++20", "-O1", "-c", "-Wall", "-Werror=return-type",
           "-DEXPERT_NODE_V2_ENABLE_CUDA=0", "-DEXPERT_NODE_V2_ENABLE_AMD=1",
           f"-I{ov}", f"-I{REF}", f"-I{REPO / 'include'}",
           str(GLUE / src), "-o", str(tmp_path / (src + ".o"))]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]


def test_glue_covers_every_amd_stub():
    """Each stub source of the reference's AMD backend has a replacement, and
    the workspace the factory needs exists."""
    stubs = {p.name for p in (REF / "expert_node_v2" / "backend" / "amd").glob("*.cc")}
    ours = {p.name for p in GLUE.glob("*.cc")}
    assert stubs <= ours, stubs - ours
    assert "backend_workspace_amd_v2.cc" in ours
