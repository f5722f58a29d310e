"""constellation_amd.moe_layer_runtime.route_token_real: the reference's
router API (server/moe_layer_runtime.py:232-408) on the HIP router.

CPU tests: argument checks raise the reference's exception types and
messages before anything touches a device, and a CPU tensor is refused
(there is no CPU path).  GPU tests: the returned routes equal the fp64
oracle's (ids bit-exact and in descending-score order, weights rel 1e-6) for
fp32 inputs, the dtype the reference requires, with and without a resident
set, including effective_top_k < top_k.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from constellation_amd.moe_layer_runtime import route_token_real, route_tokens

KW = dict(n_group=8, topk_group=4, top_k=8, norm_topk_prob=True, routed_scaling_factor=2.5,
          scoring_func="sigmoid", topk_method="noaux_tc", n_routed_experts=256, hidden_size=7168)


def _cpu_inputs(E=256, H=7168):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(H, generator=g), torch.randn(E, H, generator=g) * 0.02,
            torch.randn(E, generator=g) * 0.01)


@pytest.mark.parametrize("change,exc,msg", [
    (dict(scoring_func="softmax"), RuntimeError, "unsupported scoring_func=softmax"),
    (dict(topk_method="greedy"), RuntimeError, "unsupported topk_method=greedy"),
    (dict(topk_group=9), RuntimeError, "invalid topk_group=9 for n_group=8"),
    (dict(topk_group=0), RuntimeError, "invalid topk_group=0 for n_group=8"),
    (dict(top_k=257), RuntimeError, "invalid top_k=257 for num_experts=256"),
    (dict(n_routed_experts=128), RuntimeError, "inconsistent with n_routed_experts=128"),
    (dict(hidden_size=4096), RuntimeError, "inconsistent with hidden_size=4096"),
    (dict(n_group=7, topk_group=4), RuntimeError, "not divisible by n_group=7"),
])
def test_argument_errors_match_reference(change, exc, msg):
    x, w, b = _cpu_inputs()
    with pytest.raises(exc, match=msg):
        route_token_real(x, w, b, **{**KW, **change})


def test_tensor_errors_match_reference():
    x, w, b = _cpu_inputs()
    with pytest.raises(TypeError, match="hidden must be torch.Tensor, got list"):
        route_token_real([0.0] * 7168, w, b, **KW)
    with pytest.raises(RuntimeError, match=r"hidden must be 1D, got shape=\(1, 7168\)"):
        route_token_real(x.view(1, -1), w, b, **KW)
    with pytest.raises(TypeError, match="e_score_correction_bias must be float32"):
        route_token_real(x, w, b.double(), **KW)
    with pytest.raises(TypeError, match="hidden must be float32 for router scoring"):
        route_token_real(x.double(), w, b, **KW)
    with pytest.raises(RuntimeError, match=r"bias shape \(255,\) incompatible with num_experts=256"):
        route_token_real(x, w, b[:255], **KW)
    with pytest.raises(RuntimeError, match="hidden dim 7167 inconsistent with hidden_size=7168"):
        route_token_real(x[:7167], w, b, **KW)


def test_cpu_tensors_are_refused():
    """No CPU path: valid arguments on a CPU device raise instead of computing."""
    x, w, b = _cpu_inputs()
    with pytest.raises(RuntimeError, match="runs on a HIP device"):
        route_token_real(x, w, b, **KW)
    with pytest.raises(RuntimeError, match="runs on a HIP device"):
        route_tokens(x.view(1, -1), w, b, **KW)


@pytest.mark.gpu
@pytest.mark.parametrize("resident", [None, "every3", "five"])
def test_route_token_real_matches_oracle(gpu, oracle, resident):
    print(f"[route_token_real] resident={resident}", flush=True)
    E, H = 256, 7168
    w = gpu.gen_normal(31, 1, (E, H), 0.02, torch.bfloat16).float()   # fp32, as the reference loads it
    b = gpu.gen_normal(31, 2, (E,), 0.01, torch.float32)
    xs = gpu.gen_normal(31, 3, (6, H), 1.0, torch.bfloat16).float()
    res_ids = None
    if resident == "every3":
        res_ids = list(range(0, E, 3)) + [E + 5, -1]   # out-of-range ids are ignored
    elif resident == "five":
        res_ids = [3, 40, 77, 200, 255]                  # effective_top_k = 5 < top_k
    mask = None
    if res_ids is not None:
        mask = np.zeros(E, np.uint8)
        mask[[e for e in res_ids if 0 <= e < E]] = 1
    wn, bn = w.cpu().numpy(), b.cpu().numpy()
    for t in range(xs.shape[0]):
        routes, aux = route_token_real(xs[t], w, b, **KW, resident_expert_ids=res_ids,
                                       return_aux=True)
        oi, ow, margins, _ = oracle.route(xs[t].cpu().numpy(), wn, bn, resident=mask)
        assert aux["effective_top_k"] == len(oi) == len(routes)
        if min(margins) <= 1e-12:
            continue
        assert [e for e, _ in routes] == oi.tolist(), t
        assert np.allclose([x for _, x in routes], ow, rtol=1e-6, atol=0), t


@pytest.mark.gpu
def test_route_tokens_batched_equals_single(gpu):
    print("[route_tokens] batched vs single", flush=True)
    E, H = 256, 7168
    w = gpu.gen_normal(32, 1, (E, H), 0.02, torch.bfloat16).float()
    b = gpu.gen_normal(32, 2, (E,), 0.01, torch.float32)
    xs = gpu.gen_normal(32, 3, (20, H), 1.0, torch.bfloat16).float()
    ids, wts = route_tokens(xs, w, b, **KW)
    torch.cuda.synchronize()
    for t in range(xs.shape[0]):
        routes = route_token_real(xs[t], w, b, **KW)
        assert [e for e, _ in routes] == ids[t].tolist()
        assert [x for _, x in routes] == wts[t].tolist()


@pytest.mark.gpu
def test_route_token_real_run_to_run_exact():
    """The reference's stability check (server/test/1_smoke_moe_router_validation.py:
    16-17, 96-162): hidden = linspace(-1e-2, 1e-2, hidden_size), routed 10 times;
    the routes (ids and weights) must be identical run to run."""
    print("[route_token_real] run to run", flush=True)
    _, w, b = _cpu_inputs()
    hidden = torch.linspace(-1e-2, 1e-2, 7168, dtype=torch.float32).cuda()
    w, b = w.cuda(), b.cuda()
    runs = [route_token_real(hidden, w, b, **KW) for _ in range(10)]
    assert len(runs[0]) == 8
    assert all(r == runs[0] for r in runs[1:])
