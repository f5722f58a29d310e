"""The node harness (the reference's expert node built with the AMD plugin,
oracle/_ref/node_harness) on the CPU: with no GPU the AMD probe reports no
worker (BuildLocalAmdGpuInfosV2 returns false, as the CUDA twin does), and
the reference's control loop still answers inventory, heartbeat, resident
inventory and placement through the test client's codecs.  Skipped where the
harness is not built (it needs /root/reference at build time)."""
from __future__ import annotations

import pytest

from node_client import HARNESS, ControlClient, Harness

pytestmark = pytest.mark.skipif(not HARNESS.exists(), reason="oracle/_ref/node_harness not built")


def test_control_plane_without_gpu(tmp_path):
    h = Harness(tmp_path / "node.log")
    try:
        c = ControlClient(h.ctrl)
        inv = c.inventory()
        assert inv["node_id"] == "amd_node0" and inv["gpus"] == []
        assert c.heartbeat()
        assert c.resident() == {}
        ack = c.placement([(5, 0)])  # worker 0 does not exist on this node
        assert ack["status_code"] != 0 and not ack["all_ready"]
        c.close()
        assert h.quit() == 0
        log = (tmp_path / "node.log").read_text()
        assert "arena used 0 -> 0 bytes" in log, log[-2000:]
    finally:
        h.kill()
