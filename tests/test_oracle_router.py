"""Pins the fp64 router oracle (cx_oracle.c:cxo_route).  CPU only.

The reference router is torch code (server/moe_layer_runtime.py:232-408) in a
module that does not import here (it needs ml_dtypes and a checkpoint), so the
oracle is pinned by
  * a torch fp32 restatement of the same steps (the reference's arithmetic),
    compared as index sets wherever every decision margin exceeds 1e-5;
  * brute force on tiny expert counts (enumerate all group choices);
  * invariants: masked experts never chosen, k = min(top_k, #resident),
    normalised weights sum to the scaling factor.
Selection order / tie order of torch.topk(sorted=False) is unspecified, so
sets (not order) are compared.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch


def torch_route_fp32(x, w, bias, n_group, topk_group, top_k, norm, scale, resident=None):
    """Steps of route_token_real (moe_layer_runtime.py:321-381) in torch fp32."""
    x = torch.from_numpy(x).float()
    w = torch.from_numpy(w).float()
    b = torch.from_numpy(bias).float()
    E = w.shape[0]
    logits = w @ x
    s = torch.sigmoid(logits)
    c = s + b
    if resident is None:
        mask = torch.ones(E, dtype=torch.bool)
    else:
        mask = torch.from_numpy(resident.astype(bool))
    c = c.masked_fill(~mask, float("-inf"))
    s = s.masked_fill(~mask, 0.0)
    g = c.view(n_group, -1)
    gs = torch.topk(g, k=2, dim=-1, sorted=False).values.sum(-1)
    gi = torch.topk(gs, k=topk_group, sorted=False).indices
    gm = torch.zeros(n_group, dtype=torch.bool)
    gm[gi] = True
    sm = gm.unsqueeze(-1).expand(n_group, E // n_group).reshape(E)
    cc = c.masked_fill(~sm, float("-inf"))
    k = min(top_k, int(mask.sum()))
    idx = torch.topk(cc, k=k, sorted=False).indices
    wt = s.gather(0, idx)
    if norm and k > 1:
        wt = wt / (wt.sum() + 1e-20)
    return idx.numpy(), (wt * scale).numpy()


def _case(seed, E=256, H=7168):
    rng = np.random.default_rng(seed)
    # bf16-representable values, as the checkpoint's bf16 router weight and hidden
    w = torch.from_numpy(rng.normal(0, 0.02, (E, H)).astype(np.float32)).bfloat16().float().numpy()
    x = torch.from_numpy(rng.normal(0, 1, H).astype(np.float32)).bfloat16().float().numpy()
    bias = rng.normal(0, 0.01, E).astype(np.float32)
    return x, w, bias


def test_router_matches_torch_fp32_restatement(oracle):
    near, checked = 0, 0
    for seed in range(40):
        x, w, bias = _case(seed)
        ids, wts, margins, _ = oracle.route(x, w, bias)
        tid, tw = torch_route_fp32(x, w, bias, 8, 4, 8, True, 2.5)
        if min(margins) <= 1e-5:
            near += 1
            continue
        checked += 1
        assert sorted(ids.tolist()) == sorted(tid.tolist()), seed
        ours = dict(zip(ids.tolist(), wts.tolist()))
        theirs = dict(zip(tid.tolist(), tw.tolist()))
        for e in ours:
            assert abs(ours[e] - theirs[e]) <= 1e-5 * abs(theirs[e]), (seed, e)
    assert checked >= 30, (checked, near)


def _brute(x, w, bias, n_group, topk_group, top_k, norm, scale, resident=None):
    """Definition-level restatement in float64 by enumeration."""
    E = w.shape[0]
    logits = w.astype(np.float64) @ x.astype(np.float64)
    s = 1 / (1 + np.exp(-logits))
    res = np.ones(E, bool) if resident is None else resident.astype(bool)
    c = np.where(res, s + bias.astype(np.float64), -np.inf)
    s = np.where(res, s, 0.0)
    epg = E // n_group
    gs = np.array([np.sort(c[g * epg:(g + 1) * epg])[::-1][:2].sum() for g in range(n_group)])
    best = None
    for groups in itertools.combinations(range(n_group), topk_group):
        val = gs[list(groups)].sum()
        if best is None or val > best[0]:
            best = (val, groups)
    allowed = np.zeros(E, bool)
    for g in best[1]:
        allowed[g * epg:(g + 1) * epg] = True
    cand = np.where(allowed, c, -np.inf)
    k = min(top_k, int(res.sum()))
    idx = np.argsort(-cand, kind="stable")[:k]
    wt = s[idx]
    if norm and k > 1:
        wt = wt / (wt.sum() + 1e-20)
    return idx, wt * scale


@pytest.mark.parametrize("E,G,TG,K", [(8, 4, 2, 3), (16, 4, 2, 4), (32, 8, 4, 8), (12, 3, 1, 2)])
def test_router_brute_force_small(oracle, E, G, TG, K):
    rng = np.random.default_rng(E * 100 + K)
    for _ in range(30):
        w = rng.normal(0, 0.5, (E, 16)).astype(np.float32)
        x = rng.normal(0, 1, 16).astype(np.float32)
        bias = rng.normal(0, 0.05, E).astype(np.float32)
        ids, wts, _, _ = oracle.route(x, w, bias, n_group=G, topk_group=TG, top_k=K, scale=1.5)
        bi, bw = _brute(x, w, bias, G, TG, K, True, 1.5)
        assert sorted(ids.tolist()) == sorted(bi.tolist())
        assert np.allclose(np.sort(wts), np.sort(bw), rtol=1e-12)


def test_router_resident_mask_and_effective_k(oracle):
    x, w, bias = _case(7, E=64, H=256)
    resident = np.zeros(64, np.uint8)
    resident[[1, 5, 9, 40, 41]] = 1
    ids, wts, _, _ = oracle.route(x, w, bias, resident=resident)
    assert len(ids) == 5 or set(ids.tolist()) <= {1, 5, 9, 40, 41}
    assert set(ids.tolist()) <= {1, 5, 9, 40, 41}
    assert abs(wts.sum() - 2.5) < 1e-9


def test_router_weights_normalised(oracle):
    x, w, bias = _case(11)
    ids, wts, _, _ = oracle.route(x, w, bias)
    assert len(set(ids.tolist())) == 8
    assert abs(wts.sum() - 2.5) < 1e-9
    _, wts2, _, _ = oracle.route(x, w, bias, norm=False, scale=1.0)
    assert np.all(wts2 > 0) and np.all(wts2 < 1)


def test_router_logits_exact_products(oracle):
    # bf16 x bf16 products are exact in fp64; the fp64 sum matches math.fsum closely
    import math
    x, w, bias = _case(3, E=4, H=512)
    _, _, _, logits = oracle.route(x, w, bias, n_group=1, topk_group=1, top_k=2)
    for e in range(4):
        exact = math.fsum(float(a) * float(b) for a, b in zip(w[e], x))
        assert abs(logits[e] - exact) <= 1e-12 * max(1.0, abs(exact))
