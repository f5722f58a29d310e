"""The session-level drop-ins of constellation_amd.moe_layer_runtime on the
CPU: run_topk_moe_layer(session, hidden, routes) (server/moe_layer_runtime.py:
170-229) and run_moe_layer(session, hidden, layer_id) (:411-578) against a
fake InferenceSession (server/inference_session.py:22-60) whose client pool
hands out fake NodeClients (server/client.py: send_message / recv_message).

Checked: one MoeLayerRequest per (node, layer) with the node's local ids and
weights and exact v1 framing; per-expert requests of weight 1.0 under
return_aux, in route order, with the reference's aux structures; the
combine; the reference's route-validation messages; a missing placement; a
transport error invalidating the pooled connection; a failed node status;
run_moe_layer's argument checks in the reference's order, and that without
a HIP device the router refuses to run (no CPU fallback)."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from constellation_amd import moe_layer_protocol as P
from constellation_amd.moe_layer_runtime import run_moe_layer, run_topk_moe_layer

EPL = 8  # experts per layer of the fake session
H = 32


class LinearNode:
    """A fake expert node: expert e of layer l answers y = (l*EPL + e + 1) * ones,
    so a request's output is sum_k w_k * (gid_k + 1), exact in fp16 for the
    weights used here."""

    def __init__(self):
        self.requests = []

    def handle(self, msg_type: int, rid: int, body: bytes):
        frame = P.encode_header(msg_type, rid, len(body)) + body
        self.requests.append(frame)
        req = P.decode_moe_layer_request(body)
        T, Hd, layer = req["batch_size"], req["hidden_dim"], req["layer_id"]
        acc = np.zeros((T, Hd), np.float32)
        for t in range(T):
            for e, w in zip(req["expert_ids"][t], req["expert_weights"][t]):
                if e >= 0:
                    acc[t] += np.float32(w) * np.float32(layer * EPL + int(e) + 1)
        dt = torch.bfloat16 if req["output_dtype"] == 2 else torch.float16
        out = torch.from_numpy(acc).to(dt).view(torch.int16).numpy().tobytes()
        resp = P.encode_moe_layer_response({"status_code": 0, "batch_size": T, "hidden_dim": Hd,
                                            "output_dtype": req["output_dtype"], "output": out})
        return {"header": P.decode_header(P.encode_header(P.MOE_LAYER_RESPONSE, rid, len(resp))),
                "body": resp}


class FakeClient:
    def __init__(self, node, fail=False, status=None):
        self.node, self.fail, self.status = node, fail, status
        self._reply = None

    def send_message(self, msg_type, request_id, body=b""):
        if self.fail:
            raise ConnectionError("link down")
        self._reply = self.node.handle(int(msg_type), int(request_id), body)
        if self.status is not None:
            b = P.encode_moe_layer_response({"status_code": self.status, "batch_size": 1,
                                             "hidden_dim": H, "output_dtype": 1, "output": b""})
            self._reply = {"header": self._reply["header"] | {"body_len": len(b)}, "body": b}

    def recv_message(self):
        r, self._reply = self._reply, None
        return r


class FakePool:
    def __init__(self, clients):
        self.clients = clients
        self.invalidated = []

    def get(self, host, port):
        return self.clients[(host, int(port))]

    def invalidate(self, host, port):
        self.invalidated.append((host, int(port)))


class FakeSession:
    def __init__(self, placements, clients, **extra):
        self.coord = type("Coord", (), {"placements": placements})()
        self.client_pool = FakePool(clients)
        self.cfg = {"log_level": 0, "run": {"experts_per_layer": EPL}}
        self.backbone_store = None
        for k, v in extra.items():
            setattr(self, k, v)


def _session():
    """Layer 2 (global ids 16..23): 16-18 on node a:1, 19-23 on node b:2."""
    a, b = LinearNode(), LinearNode()
    placements = [{"expert_id": 2 * EPL + e, "host": "a" if e < 3 else "b",
                   "worker_port": 1 if e < 3 else 2} for e in range(EPL)]
    return FakeSession(placements, {("a", 1): FakeClient(a), ("b", 2): FakeClient(b)}), a, b


def test_one_request_per_node_with_local_ids_and_weights():
    s, a, b = _session()
    x = torch.linspace(-1, 1, H, dtype=torch.float32)
    routes = [(17, 0.5), (20, 0.25), (16, 0.125)]
    combined, weighted = run_topk_moe_layer(s, x, routes)
    want = 0.5 * 18 + 0.25 * 21 + 0.125 * 17
    assert combined.dtype == torch.float32 and torch.all(combined == want)
    assert len(a.requests) == 1 and len(b.requests) == 1
    for node, ids, ws in ((a, [1, 0], [0.5, 0.125]), (b, [4], [0.25])):
        f = node.requests[0]
        magic, ver, mt, rid, n = struct.unpack("<IHHII", f[:16])
        assert (magic, ver, mt, n) == (0x45585054, 1, 42, len(f) - 16)
        req = P.decode_moe_layer_request(f[16:])
        assert (req["layer_id"], req["batch_size"], req["hidden_dim"], req["top_k"]) == (2, 1, H, len(ids))
        # fp32 hidden travels as fp16, as the reference's wire does
        assert req["input_dtype"] == 1 and req["output_dtype"] == 1 and req["flags"] == 0
        assert req["expert_ids"].tolist() == [ids]
        assert req["expert_weights"].tolist() == [ws]
        assert req["activation"] == x.to(torch.float16).view(torch.int16).numpy().tobytes()
    # outputs are per node, not per expert
    assert [(e, w) for e, w, _ in weighted] == [(-1, 1.0), (-1, 1.0)]
    assert sum(float(p[0]) for _, _, p in weighted) == want


def test_return_aux_asks_each_expert_alone():
    s, a, b = _session()
    x = torch.linspace(-1, 1, H, dtype=torch.bfloat16)
    routes = [(17, 0.5), (20, 0.25), (16, 0.125)]
    combined, weighted, experts = run_topk_moe_layer(s, x, routes, return_aux=True)
    assert combined.dtype == torch.bfloat16
    assert float(combined[0]) == 0.5 * 18 + 0.25 * 21 + 0.125 * 17
    assert len(a.requests) == 2 and len(b.requests) == 1
    for f in a.requests + b.requests:
        req = P.decode_moe_layer_request(f[16:])
        assert req["top_k"] == 1 and req["expert_weights"].tolist() == [[1.0]]
        assert req["input_dtype"] == 2   # bf16 hidden travels as bf16
    assert [(e, w) for e, w, _ in weighted] == routes
    for (gid, w, y), d in zip(weighted, experts):
        assert y.dtype == np.float32 and np.all(y == gid + 1)
        assert d["expert_id"] == gid and d["weight"] == w and np.all(d["output"] == y)
        assert np.all(d["weighted_output"] == np.float32(w) * y) and d["output_dtype"] == 2


@pytest.mark.parametrize("routes,err,msg", [
    ([], RuntimeError, "routes is empty"),
    ([(17, 0.5), (17, 0.5)], RuntimeError, "duplicate expert_id in routes: 17"),
    ([(17, 0.5), (18, -0.25)], RuntimeError, "negative route weight for expert 18: -0.25"),
    ([(99, 0.5)], RuntimeError, "expert 99 not found in placements"),
])
def test_route_errors(routes, err, msg):
    s, _, _ = _session()
    with pytest.raises(err, match=msg):
        run_topk_moe_layer(s, torch.zeros(H), routes)


def test_hidden_checks():
    s, _, _ = _session()
    with pytest.raises(TypeError, match="hidden must be torch.Tensor, got ndarray"):
        run_topk_moe_layer(s, np.zeros(H, np.float32), [(17, 1.0)])
    with pytest.raises(RuntimeError, match=r"hidden must be 1D, got shape=\(2, 32\)"):
        run_topk_moe_layer(s, torch.zeros(2, H), [(17, 1.0)])


def test_transport_error_invalidates_connection_and_bad_status_raises():
    s, _, _ = _session()
    s.client_pool.clients[("b", 2)].fail = True
    with pytest.raises(ConnectionError, match="link down"):
        run_topk_moe_layer(s, torch.zeros(H), [(16, 0.5), (21, 0.5)])
    assert s.client_pool.invalidated == [("b", 2)]
    s, _, _ = _session()
    s.client_pool.clients[("a", 1)].status = 2
    with pytest.raises(RuntimeError, match="failed on node a:1: status=2"):
        run_topk_moe_layer(s, torch.zeros(H), [(16, 0.5)])


class Store:
    def __init__(self, entry, dtype=torch.bfloat16):
        self.entry, self.dtype = entry, dtype

    def layer(self, layer_id):
        return self.entry


def _router_session(entry, dtype=torch.bfloat16):
    s, _, _ = _session()
    s.backbone_store = Store(entry, dtype)
    s.get_router_config = lambda: {"hidden_size": H, "n_group": 2, "topk_group": 1, "top_k": 2,
                                   "norm_topk_prob": True, "routed_scaling_factor": 2.5,
                                   "scoring_func": "sigmoid", "topk_method": "noaux_tc",
                                   "n_routed_experts": EPL}
    return s


def test_run_moe_layer_checks_in_reference_order():
    s, _, _ = _session()
    with pytest.raises(RuntimeError, match="session.backbone_store is not initialized"):
        run_moe_layer(s, torch.zeros(H), 2)
    router = {"gate_weight": torch.zeros(EPL, H), "e_score_correction_bias": torch.zeros(EPL)}
    s = _router_session({"device": "cpu", "router": router})
    with pytest.raises(TypeError, match="expected dtype=torch.bfloat16, got dtype=torch.float32"):
        run_moe_layer(s, torch.zeros(H), 2)
    with pytest.raises(ValueError, match="contains non-finite values"):
        run_moe_layer(s, torch.full((H,), float("nan"), dtype=torch.bfloat16), 2)
    with pytest.raises(RuntimeError, match="hidden size mismatch: got=16 expected=32"):
        run_moe_layer(s, torch.zeros(16, dtype=torch.bfloat16), 2)
    s = _router_session({"device": "cpu"})
    with pytest.raises(RuntimeError, match="router weights are not loaded for layer 2"):
        run_moe_layer(s, torch.zeros(H, dtype=torch.bfloat16), 2)
    bad = dict(router, e_score_correction_bias=torch.zeros(EPL, dtype=torch.float64))
    s = _router_session({"device": "cpu", "router": bad})
    with pytest.raises(TypeError, match="e_score_correction_bias must be float32"):
        run_moe_layer(s, torch.zeros(H, dtype=torch.bfloat16), 2)
    s = _router_session({"device": "cpu", "router": router})
    s.cfg["run"]["restricted_expert_ids"] = [3, 9]
    with pytest.raises(RuntimeError, match=r"restricted expert id out of range for layer 2: 9 not in \[0, 8\)"):
        run_moe_layer(s, torch.zeros(H, dtype=torch.bfloat16), 2)
    s = _router_session({"device": "cpu", "router": router})
    with pytest.raises(RuntimeError, match="no resident experts found for layer 5"):
        run_moe_layer(s, torch.zeros(H, dtype=torch.bfloat16), 5)


def test_run_moe_layer_refuses_a_non_hip_device():
    router = {"gate_weight": torch.zeros(EPL, H), "e_score_correction_bias": torch.zeros(EPL)}
    s = _router_session({"device": "cpu", "router": router})
    with pytest.raises(RuntimeError, match="the router runs on a HIP device"):
        run_moe_layer(s, torch.zeros(H, dtype=torch.bfloat16), 2)
