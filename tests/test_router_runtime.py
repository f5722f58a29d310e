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


AUX_KEYS = ("logits", "scores_raw", "scores", "scores_for_choice_raw", "scores_for_choice",
            "group_scores", "selected_group_idx", "group_mask", "score_mask", "resident_mask",
            "topk_idx", "topk_choice_vals", "topk_weight_pre_norm", "topk_weight_post_norm",
            "topk_weight", "effective_top_k", "routes")


def _reference_steps_torch(logits, bias, resident, n_group, topk_group, top_k, norm, scale):
    """The reference's router steps after the matvec (server/moe_layer_runtime.py:
    321-381), retyped with torch ops on the CPU in float64, as an independent
    check of the host-side aux builder."""
    E = logits.shape[0]
    s_raw = torch.sigmoid(logits)
    c_raw = s_raw + bias
    c = c_raw.masked_fill(~resident, float("-inf"))
    s = s_raw.masked_fill(~resident, 0.0)
    gs = torch.topk(c.view(n_group, E // n_group), k=2, dim=-1).values.sum(-1)
    sel = torch.topk(gs, k=topk_group).indices
    gm = torch.zeros(n_group, dtype=torch.bool)
    gm[sel] = True
    sm = gm.unsqueeze(-1).expand(n_group, E // n_group).reshape(E)
    k = min(top_k, int(resident.sum()))
    vals, idx = torch.topk(c.masked_fill(~sm, float("-inf")), k=k)
    w = s.gather(0, idx)
    pre = w.clone()
    if norm and k > 1:
        w = w / (w.sum() + 1e-20)
    return dict(scores_raw=s_raw, scores=s, scores_for_choice=c, group_scores=gs,
                selected_group_idx=torch.sort(sel).values, group_mask=gm, score_mask=sm,
                topk_idx=idx, topk_choice_vals=vals, topk_weight_pre_norm=pre,
                topk_weight_post_norm=w, topk_weight=w * scale)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("n_res", [256, 40, 5])
def test_route_aux_matches_reference_steps(seed, n_res):
    """_route_aux (host side of return_aux=True) against the reference's steps
    retyped in torch, for routes chosen by those same steps."""
    from constellation_amd.moe_layer_runtime import _route_aux
    g = torch.Generator().manual_seed(seed)
    E = 256
    logits = torch.randn(E, generator=g, dtype=torch.float64) * 0.7
    bias = torch.randn(E, generator=g, dtype=torch.float64) * 0.01
    resident = torch.zeros(E, dtype=torch.bool)
    resident[torch.randperm(E, generator=g)[:n_res]] = True
    ref = _reference_steps_torch(logits, bias, resident, 8, 4, 8, True, 2.5)
    routes = [(int(e), float(w)) for e, w in zip(ref["topk_idx"], ref["topk_weight"])]
    aux = _route_aux(logits.numpy(), bias.numpy(), resident.numpy(), n_group=8, topk_group=4,
                     norm_topk_prob=True, routes=routes)
    assert set(AUX_KEYS) <= set(aux)
    assert aux["effective_top_k"] == min(8, n_res)
    gs = np.sort(ref["group_scores"].numpy())[::-1]
    if gs[3] != gs[4]:
        for key in ("selected_group_idx", "group_mask", "score_mask"):
            assert np.array_equal(aux[key], ref[key].numpy()), key
    else:
        # an exact tie at the group boundary (e.g. groups with < 2 resident
        # experts score -inf): torch.topk breaks it arbitrarily, the kernel
        # and the aux toward the lower group index; the selected scores agree
        sel_ref = ref["selected_group_idx"].numpy()
        assert np.array_equal(np.sort(aux["group_scores"][aux["selected_group_idx"]]),
                              np.sort(ref["group_scores"].numpy()[sel_ref].astype(np.float32)))
    assert np.array_equal(aux["topk_idx"], ref["topk_idx"].numpy())
    for key in ("scores_raw", "scores", "scores_for_choice", "group_scores", "topk_choice_vals",
                "topk_weight_pre_norm", "topk_weight_post_norm", "topk_weight"):
        assert aux[key].dtype == np.float32, key
        assert np.allclose(aux[key], ref[key].numpy().astype(np.float32), rtol=1e-6, atol=0), key
    assert aux["logits"].dtype == np.float32 and aux["resident_mask"].dtype == bool


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
        oi, ow, margins, lg = oracle.route(xs[t].cpu().numpy(), wn, bn, resident=mask)
        assert aux["effective_top_k"] == len(oi) == len(routes)
        assert set(AUX_KEYS) <= set(aux)
        # the kernel's fp64 logits equal the oracle's exact-product sums
        assert np.allclose(aux["logits"], lg.astype(np.float32), rtol=1e-6, atol=1e-9), t
        if min(margins) <= 1e-12:
            continue
        assert [e for e, _ in routes] == oi.tolist(), t
        assert np.allclose([x for _, x in routes], ow, rtol=1e-6, atol=0), t
        assert aux["topk_idx"].tolist() == oi.tolist()
        assert np.array_equal(aux["topk_weight"], np.asarray([x for _, x in routes], np.float32))
        # every chosen expert sits in a selected group
        sel = set(aux["selected_group_idx"].tolist())
        assert len(sel) == 4 and {e // 32 for e in oi.tolist()} <= sel
        assert np.allclose(aux["topk_weight_post_norm"] * 2.5, ow, rtol=1e-6)


@pytest.mark.gpu
def test_route_token_real_fp16_hidden(gpu, oracle):
    """fp16 hidden is widened exactly, so the routes equal the oracle's on the
    fp16 values (the reference itself only takes fp32)."""
    print("[route_token_real] fp16 hidden", flush=True)
    E, H = 256, 7168
    w = gpu.gen_normal(33, 1, (E, H), 0.02, torch.bfloat16).float()
    b = gpu.gen_normal(33, 2, (E,), 0.01, torch.float32)
    xs = gpu.gen_normal(33, 3, (4, H), 1.0, torch.float16)
    wn, bn = w.cpu().numpy(), b.cpu().numpy()
    for t in range(xs.shape[0]):
        routes = route_token_real(xs[t], w, b, **KW)
        oi, ow, margins, _ = oracle.route(xs[t].float().cpu().numpy(), wn, bn)
        if min(margins) <= 1e-12:
            continue
        assert [e for e, _ in routes] == oi.tolist(), t
        assert np.allclose([x for _, x in routes], ow, rtol=1e-6, atol=0), t
    ids, _ = route_tokens(xs, w, b, **KW)
    torch.cuda.synchronize()
    assert ids.shape == (4, 8)


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
