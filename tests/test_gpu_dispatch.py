"""constellation_amd.moe_dispatch on the GPU, against the CPU oracle.

  * run_moe_layer_batched with one local node holding the layer: router and
    experts in one call, every route and the combined output against the
    oracle, for decode (T <= 16) and prefill-sized batches;
  * the same layer split over two nodes (a LocalNode and a RemoteNode whose
    transport runs MoeLayerRequest bodies on a second layer table in this
    process): partial sums added in fp32, against the oracle;
  * the batched call equals the reference's per-token loop
    (full_model_runtime.py:317-331) run token by token through
    route_token_real + run_topk_moe_layer.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.oracle import rel_l2
from test_gpu_moe import _free, _make_layer, _oracle_moe, _oracle_route, _router_inputs

pytestmark = pytest.mark.gpu

E, H, I = 32, 1024, 512
CFG = dict(n_group=8, topk_group=4, top_k=8, norm_topk_prob=True, routed_scaling_factor=2.5)


def _check_routes(oracle, x, w, bias, ids):
    ids = ids.cpu().numpy()
    for t, (oi, _, margins, _) in enumerate(_oracle_route(oracle, x, w, bias)):
        if min(margins) > 1e-12:
            assert ids[t].tolist() == oi.tolist(), t


@pytest.mark.parametrize("T", [1, 5, 40])
def test_batched_layer_on_one_local_node(gpu, oracle, T):
    from constellation_amd.moe_dispatch import LocalNode, run_moe_layer_batched
    print(f"[dispatch] local node T={T}", flush=True)
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=61)
    try:
        x, w, bias = _router_inputs(gpu, 62 + T, T, E, H)
        y, ids, wts = run_moe_layer_batched([LocalNode({3: layer})], x, 3, w, bias, **CFG)
        torch.cuda.synchronize()
        assert y.shape == (T, H) and y.dtype == torch.bfloat16 and y.device == x.device
        _check_routes(oracle, x, w, bias, ids)
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids.cpu().numpy(),
                          wts.cpu().numpy())
        got = y.float().cpu().numpy()
        assert rel_l2(got, ref) < 1e-2
        assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-3)
    finally:
        _free(layer, experts, sh)


def test_layer_split_over_local_and_remote_node(gpu, oracle):
    from constellation_amd.engine import Layer
    from constellation_amd.moe_dispatch import LocalNode, RemoteNode, run_topk_moe_layer
    from constellation_amd import moe_layer_protocol as P
    print("[dispatch] local + remote node", flush=True)
    T = 6
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=71)
    evens = Layer(gpu, [e if i % 2 == 0 else None for i, e in enumerate(experts)], sh)
    odds = Layer(gpu, [e if i % 2 == 1 else None for i, e in enumerate(experts)], None)
    frames = []

    def transport(frame: bytes) -> bytes:   # the remote node's worker, in this process
        frames.append(frame)
        hdr = P.decode_header(frame[:16])
        resp = gpu.moe_layer_request(odds, frame[16:])
        return P.frame(P.MOE_LAYER_RESPONSE, hdr["request_id"], resp)
    try:
        x, w, bias = _router_inputs(gpu, 72, T, E, H)
        ids, wts = gpu.route(x, w, bias, n_group=8, topk_group=4, top_k=8)
        nodes = [LocalNode({5: evens}), RemoteNode(transport, {5: range(1, E, 2)})]
        y = run_topk_moe_layer(nodes, x, 5, ids, wts, n_experts=E)
        torch.cuda.synchronize()
        assert len(frames) == 1
        xf, ih, wh = x.float().cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
        ref = _oracle_moe(oracle, cpu, cpu_sh, xf, ih, wh)
        ref_even = _oracle_moe(oracle, cpu, cpu_sh, xf, np.where(ih % 2 == 0, ih, -1), wh)
        ref_odd = _oracle_moe(oracle, cpu, None, xf, np.where(ih % 2 == 1, ih, -1), wh)
        got = y.float().cpu().numpy()
        # two bf16 partials, each rounded once, then added in fp32 and rounded
        assert rel_l2(got, ref) < 1e-2
        bound = (np.abs(ref_even) + np.abs(ref_odd) + np.abs(ref)) * 2.0 ** -8 + 1e-3
        assert np.all(np.abs(got - ref) <= bound)
    finally:
        torch.cuda.synchronize()
        evens.close()
        odds.close()
        _free(layer, experts, sh)


def test_batched_equals_per_token_loop(gpu, oracle):
    """One batched call for T tokens against the reference's loop of one
    run_moe_layer per token: identical routes and outputs within one bf16 ulp."""
    from constellation_amd.moe_dispatch import LocalNode, run_moe_layer_batched, run_topk_moe_layer
    from constellation_amd.moe_layer_runtime import route_token_real
    print("[dispatch] batched vs per-token", flush=True)
    T = 7
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=81)
    try:
        x, w, bias = _router_inputs(gpu, 82, T, E, H)
        node = LocalNode({0: layer})
        y, ids, _ = run_moe_layer_batched([node], x, 0, w, bias, **CFG)
        rows = []
        for t in range(T):
            routes = route_token_real(x[t], w, bias, **CFG, scoring_func="sigmoid",
                                      topk_method="noaux_tc", n_routed_experts=E, hidden_size=H)
            assert [e for e, _ in routes] == ids[t].tolist()
            rows.append(run_topk_moe_layer([node], x[t], 0, np.asarray([[e for e, _ in routes]]),
                                           np.asarray([[v for _, v in routes]], np.float32),
                                           n_experts=E))
        loop = torch.stack(rows)
        torch.cuda.synchronize()
        a = y.cpu().view(torch.int16).numpy().astype(np.int32)
        b = loop.cpu().view(torch.int16).numpy().astype(np.int32)
        line = lambda v: np.where(v & 0x8000, -(v & 0x7FFF), v)  # noqa: E731
        assert np.abs(line(a & 0xFFFF) - line(b & 0xFFFF)).max() <= 1
    finally:
        _free(layer, experts, sh)
