"""constellation_amd.moe_dispatch on the CPU: route validation with the
reference's messages (server/moe_layer_runtime.py:84-98), and the framing,
per-node route masking, shared-expert assignment and partial sums of
RemoteNode calls, through fake transports (host tensors, no GPU)."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from constellation_amd import moe_layer_protocol as P
from constellation_amd.moe_dispatch import RemoteNode, run_topk_moe_layer, validate_routes


@pytest.mark.parametrize("ids,w,msg", [
    ([[-1, -1]], [[0.5, 0.5]], "routes is empty"),
    ([[3, 3]], [[0.5, 0.5]], "duplicate expert_id in routes: 3"),
    ([[1, 2], [4, 5]], [[0.5, 0.5], [0.5, -0.25]], "negative route weight for expert 5: -0.25"),
])
def test_validate_routes_messages(ids, w, msg):
    with pytest.raises(RuntimeError, match=msg):
        validate_routes(np.asarray(ids), np.asarray(w, np.float32))


def test_validate_routes_accepts_distinct_per_token():
    validate_routes(np.asarray([[1, 2], [2, 1], [-1, 7]]), np.full((3, 2), 0.5, np.float32))


class FakeNode:
    """Decodes each framed request, records it, and answers with a constant
    partial (value) in the requested output dtype."""

    def __init__(self, value: float, status: int = 0, bad_rid: bool = False):
        self.value, self.status, self.bad_rid = value, status, bad_rid
        self.frames = []

    def __call__(self, frame: bytes) -> bytes:
        self.frames.append(frame)
        hdr = P.decode_header(frame[:16])
        assert hdr["msg_type"] == P.MOE_LAYER_REQUEST and hdr["body_len"] == len(frame) - 16
        req = P.decode_moe_layer_request(frame[16:])
        T, H = req["batch_size"], req["hidden_dim"]
        dt = torch.bfloat16 if req["output_dtype"] == 2 else torch.float16
        out = b"" if self.status else \
            torch.full((T, H), self.value, dtype=dt).view(torch.int16).numpy().tobytes()
        body = P.encode_moe_layer_response({"status_code": self.status, "batch_size": T,
                                            "hidden_dim": H, "output_dtype": req["output_dtype"],
                                            "output": out})
        rid = hdr["request_id"] + (1 if self.bad_rid else 0)
        return P.frame(P.MOE_LAYER_RESPONSE, rid, body)


def test_two_remote_nodes_mask_routes_and_sum():
    H = 16
    x = torch.randn(2, H).to(torch.bfloat16)
    ids = np.asarray([[0, 1, -1], [3, 2, 1]], np.int32)
    w = np.asarray([[0.5, 0.25, 0.0], [0.1, 0.2, 0.3]], np.float32)
    a, b = FakeNode(1.0), FakeNode(2.0)
    nodes = [RemoteNode(a, {4: [0, 2]}, shared_layers=[4]), RemoteNode(b, {4: [1, 3, 2]})]
    y = run_topk_moe_layer(nodes, x, 4, ids, w, n_experts=8)
    assert y.dtype == torch.bfloat16 and torch.equal(y.float(), torch.full((2, H), 3.0))
    for node, want_ids, shared in ((a, [[0, -1, -1], [-1, 2, -1]], True),
                                   (b, [[-1, 1, -1], [3, -1, 1]], False)):
        assert len(node.frames) == 1
        f = node.frames[0]
        magic, ver, mt, rid, n = struct.unpack("<IHHII", f[:16])
        assert (magic, ver, mt, n) == (0x45585054, 1, 42, len(f) - 16)
        req = P.decode_moe_layer_request(f[16:])
        assert (req["layer_id"], req["batch_size"], req["hidden_dim"], req["top_k"]) == (4, 2, H, 3)
        assert req["input_dtype"] == 2 and req["output_dtype"] == 2
        assert req["flags"] == (P.FLAG_SHARED if shared else 0)
        assert req["expert_ids"].tolist() == want_ids
        assert np.array_equal(req["expert_weights"], w)     # weights travel unmasked
        assert req["activation"] == x.view(torch.int16).numpy().tobytes()


def test_single_token_and_out_dtype():
    x = torch.randn(32).to(torch.float16)
    node = FakeNode(0.5)
    y = run_topk_moe_layer([RemoteNode(node, {0: range(8)}, [0])], x, 0,
                           np.asarray([[1, 5]]), np.asarray([[0.5, 0.5]]), n_experts=8,
                           out_dtype=torch.bfloat16)
    assert y.shape == (32,) and y.dtype == torch.bfloat16 and torch.all(y == 0.5)
    req = P.decode_moe_layer_request(node.frames[0][16:])
    assert req["input_dtype"] == 1 and req["output_dtype"] == 2


def test_dispatch_errors():
    x = torch.zeros(1, 16, dtype=torch.bfloat16)
    ids, w = np.asarray([[1, 2]]), np.asarray([[0.5, 0.5]], np.float32)
    with pytest.raises(RuntimeError, match="no node holds expert 2 of layer 0"):
        run_topk_moe_layer([RemoteNode(FakeNode(1.0), {0: [1]}, [0])], x, 0, ids, w, n_experts=8)
    with pytest.raises(RuntimeError, match="no node holds the shared expert of layer 0"):
        run_topk_moe_layer([RemoteNode(FakeNode(1.0), {0: [1, 2]})], x, 0, ids, w, n_experts=8)
    with pytest.raises(RuntimeError, match="status=2"):
        run_topk_moe_layer([RemoteNode(FakeNode(1.0, status=2), {0: [1, 2]}, [0])], x, 0, ids, w,
                           n_experts=8)
    with pytest.raises(P.ProtocolError, match="unexpected reply"):
        run_topk_moe_layer([RemoteNode(FakeNode(1.0, bad_rid=True), {0: [1, 2]}, [0])], x, 0, ids, w,
                           n_experts=8)
    # shared=False: a node that holds only the shared expert is not called
    extra = FakeNode(9.0)
    y = run_topk_moe_layer([RemoteNode(FakeNode(1.0), {0: [1, 2]}), RemoteNode(extra, {}, [0])], x, 0,
                           ids, w, n_experts=8, shared=False)
    assert torch.all(y == 1.0) and extra.frames == []
