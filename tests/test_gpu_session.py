"""Session-level drop-ins on the GPU, against the CPU oracle.

run_moe_layer(session, hidden, layer_id) (server/moe_layer_runtime.py:
411-578) with a fake InferenceSession whose placements put the even experts
of the layer on an endpoint served in this process (cx_local_nodes: a
LocalNode, the device path) and the odd ones on a "remote" endpoint whose
NodeClient hands each MoeLayerRequest body to a second layer table here
(cx_moe_layer_request_run, as the node's worker would).  The routes equal
the oracle's; the output equals the oracle's weighted sum of the routed
experts (no shared expert: the reference runs it apart); with return_aux
every expert's own output is checked, and the aux routes are the global ids.
Also: a bad route weight on the single-local-node device path is skipped
and reported by the context's next sync (no host copy of the routes)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.oracle import rel_l2
from test_gpu_moe import _free, _make_layer, _oracle_moe, _oracle_route, _router_inputs
from test_session_dropin import FakeClient, FakeSession

pytestmark = pytest.mark.gpu

E, H, I, LAYER = 32, 1024, 512, 3
CFG = dict(n_group=8, topk_group=4, top_k=8)


class WorkerNode:
    """The remote endpoint's worker: runs each request body on `layer`."""

    def __init__(self, gpu, layer):
        self.gpu, self.layer, self.requests = gpu, layer, []

    def handle(self, msg_type, rid, body):
        from constellation_amd import moe_layer_protocol as P
        self.requests.append(body)
        resp = self.gpu.moe_layer_request(self.layer, body)
        return {"header": P.decode_header(P.encode_header(P.MOE_LAYER_RESPONSE, rid, len(resp))),
                "body": resp}


class Store:
    def __init__(self, entry):
        self.entry, self.dtype = entry, torch.bfloat16

    def layer(self, layer_id):
        return self.entry


@pytest.mark.parametrize("return_aux", [False, True])
def test_run_moe_layer_session_local_and_remote(gpu, oracle, return_aux):
    from constellation_amd.engine import Layer
    from constellation_amd.moe_dispatch import LocalNode
    from constellation_amd.moe_layer_runtime import run_moe_layer
    print(f"[session] run_moe_layer return_aux={return_aux}", flush=True)
    layer, experts, sh, cpu, _ = _make_layer(gpu, oracle, E, H, I, seed=91, shared=False)
    evens = Layer(gpu, [e if i % 2 == 0 else None for i, e in enumerate(experts)], None)
    odds = Layer(gpu, [e if i % 2 == 1 else None for i, e in enumerate(experts)], None)
    worker = WorkerNode(gpu, odds)
    try:
        x, w, bias = _router_inputs(gpu, 92, 1, E, H)
        placements = [{"expert_id": LAYER * E + e, "host": "gpu" if e % 2 == 0 else "peer",
                       "worker_port": 7 if e % 2 == 0 else 8} for e in range(E)]
        s = FakeSession(placements, {("peer", 8): FakeClient(worker)},
                        cx_local_nodes={("gpu", 7): LocalNode({LAYER: evens})})
        s.cfg["run"]["experts_per_layer"] = E
        s.backbone_store = Store({"device": "cuda:0",
                                  "router": {"gate_weight": w.float(), "e_score_correction_bias": bias}})
        s.get_router_config = lambda: {"hidden_size": H, **CFG, "norm_topk_prob": True,
                                       "routed_scaling_factor": 2.5, "scoring_func": "sigmoid",
                                       "topk_method": "noaux_tc", "n_routed_experts": E}
        res = run_moe_layer(s, x[0], LAYER, return_aux=return_aux)
        torch.cuda.synchronize()
        y = res["output"]
        assert y.shape == (H,) and y.dtype == torch.bfloat16 and y.device == x.device
        oi, ow, margins, _ = _oracle_route(oracle, x, w, bias, **CFG)[0]
        assert min(margins) > 1e-12
        # the router input is fp32; the wire (and the device path) carry it as fp16
        x16 = x.float().to(torch.float16).float().cpu().numpy()
        ref = _oracle_moe(oracle, cpu, None, x16, oi[None, :], ow[None, :].astype(np.float32))[0]
        got = y.float().cpu().numpy()
        assert rel_l2(got, ref) < 1e-2
        assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 2e-3)
        n_odd = int(np.sum(oi % 2 == 1))
        assert len(worker.requests) == (n_odd if return_aux else int(n_odd > 0))
        if return_aux:
            aux = res["aux"]
            assert [e for e, _ in aux["local_routes"]] == oi.tolist()
            assert np.allclose([v for _, v in aux["local_routes"]], ow, rtol=1e-6, atol=0)
            assert aux["selected_global_expert_ids"] == [LAYER * E + int(e) for e in oi]
            for d in aux["expert_outputs"]:
                e = d["expert_id"] - LAYER * E
                want = oracle.expert_ref(cpu[e], x16)[1][0]
                assert rel_l2(d["output"], want) < 2e-3, e
    finally:
        torch.cuda.synchronize()
        evens.close()
        odds.close()
        _free(layer, experts, sh)


def test_bad_route_weight_is_flagged_on_the_device(gpu, oracle):
    """The default validate=True path of moe_dispatch.run_topk_moe_layer on one
    local node: nothing is copied to the host; the planner skips the route
    with a negative weight and the next sync raises."""
    from constellation_amd._lib import CxError
    from constellation_amd.moe_dispatch import LocalNode, check_routes, run_topk_moe_layer
    print("[session] device-side route weight check", flush=True)
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=93)
    try:
        x, _, _ = _router_inputs(gpu, 94, 2, E, H)
        ids = torch.tensor([[3, 5, 7], [1, 2, 4]], dtype=torch.int32, device=x.device)
        wts = torch.tensor([[0.5, -0.25, 0.25], [0.5, 0.25, float("nan")]], device=x.device)
        y = run_topk_moe_layer([LocalNode({0: layer})], x, 0, ids, wts, n_experts=E)
        with pytest.raises(CxError, match="negative or non-finite route weight"):
            check_routes(0)
        check_routes(0)  # the flag is cleared once reported
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(),
                          np.asarray([[3, -1, 7], [1, 2, -1]]),
                          np.asarray([[0.5, 0, 0.25], [0.5, 0.25, 0]], np.float32))
        assert rel_l2(y.float().cpu().numpy(), ref) < 1e-2
    finally:
        _free(layer, experts, sh)
