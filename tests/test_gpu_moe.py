"""GPU parity of the router (cx_route) and the grouped MoE paths
(cx_moe_decode / cx_moe_prefill / cx_moe_layer) against the CPU oracle.

Router: expert index sets bit-exact against the fp64 oracle (both sides work
on exact products in fp64); weights within rel 1e-6.
MoE output: fp32 pre-cast output within rel-L2 1e-5 of the oracle's
dequantise-then-fp32 combine (bound in the spec: rel-L2 <= 1e-2, max-abs
<= 2e-2); 16-bit output equals the RNE cast of the fp32 output.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.oracle import BF16, FP16, rel_l2

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _router_inputs(gpu, seed, T, E, H, bias_skew=0.0):
    w = gpu.gen_normal(seed, 1, (E, H), 0.02, torch.bfloat16)
    bias = gpu.gen_normal(seed, 2, (E,), 0.01, torch.float32)
    if bias_skew:
        perm = np.random.default_rng(seed).permutation(E)
        rank = np.empty(E)
        rank[perm] = np.arange(1, E + 1)
        bias = bias + torch.from_numpy((bias_skew * rank ** -1.1).astype(np.float32)).cuda()
    x = gpu.gen_normal(seed, 3, (T, H), 1.0, torch.bfloat16)
    return x, w, bias


def _oracle_route(oracle, x, w, bias, **kw):
    xs = x.float().cpu().numpy()
    ws = w.float().cpu().numpy()
    bs = bias.cpu().numpy()
    res = [oracle.route(xs[t], ws, bs, **kw) for t in range(xs.shape[0])]
    return res


@pytest.mark.parametrize("T,E,H,G,TG,K", [(1, 256, 7168, 8, 4, 8), (16, 256, 7168, 8, 4, 8),
                                          (37, 64, 512, 8, 4, 6), (5, 32, 256, 4, 2, 3),
                                          (96, 256, 7168, 8, 4, 8), (45, 72, 1024, 8, 4, 6)])
def test_router_vs_oracle(gpu, oracle, T, E, H, G, TG, K):
    print(f"[route] T={T} E={E} H={H}", flush=True)
    x, w, bias = _router_inputs(gpu, 100 + T, T, E, H)
    ids, wts = gpu.route(x, w, bias, n_group=G, topk_group=TG, top_k=K)
    torch.cuda.synchronize()
    ids, wts = ids.cpu().numpy(), wts.cpu().numpy()
    for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias, n_group=G,
                                                             topk_group=TG, top_k=K)):
        if min(margins) <= 1e-12:
            continue  # exact-math tie: order undefined
        assert ids[t].tolist() == oi.tolist(), t  # same set and same (descending) order
        assert np.allclose(wts[t], ow, rtol=1e-6, atol=0), t


@pytest.mark.parametrize("xdt,wdt", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.float32)])
def test_router_many_tokens_fp32_operands(gpu, oracle, xdt, wdt):
    """The fp64-MFMA logits path (T >= 32) with fp32 activations or weights:
    products of fp32 values are exact in fp64 too."""
    print(f"[route] T=72 x={xdt} w={wdt}", flush=True)
    T, E, H = 72, 64, 2048
    x, w, bias = _router_inputs(gpu, 300, T, E, H)
    x = (x.float() * 1.37).to(xdt)   # fp32 values with more than 8 significant bits
    w = (w.float() * 0.73).to(wdt)
    ids, wts = gpu.route(x, w, bias, n_group=8, topk_group=4, top_k=8)
    torch.cuda.synchronize()
    ids, wts = ids.cpu().numpy(), wts.cpu().numpy()
    for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias)):
        if min(margins) <= 1e-12:
            continue
        assert ids[t].tolist() == oi.tolist(), t
        assert np.allclose(wts[t], ow, rtol=1e-6, atol=0), t


def test_router_resident_mask(gpu, oracle):
    print("[route] resident mask", flush=True)
    E, H = 64, 512
    x, w, bias = _router_inputs(gpu, 5, 8, E, H)
    res = np.zeros(E, np.uint8)
    res[::5] = 1  # 13 resident experts
    rdev = torch.from_numpy(res).cuda()
    ids, wts = gpu.route(x, w, bias, resident=rdev, n_group=8, topk_group=4, top_k=8)
    torch.cuda.synchronize()
    ids = ids.cpu().numpy()
    for t, (oi, ow, _, _) in enumerate(_oracle_route(oracle, x, w, bias, resident=res)):
        k = len(oi)
        assert ids[t][:k].tolist() == oi.tolist()
        assert np.all(ids[t][k:] == -1)
        assert all(res[i] for i in ids[t][:k])


def _make_layer(gpu, oracle, E, H, I, seed, shared=True):
    from constellation_amd.engine import Expert, Layer
    experts = [Expert.generate(0, seed, 0x1000 + 4 * e, hidden=H, inter=I) for e in range(E)]
    sh = Expert.generate(0, seed, 0x1000 + 4 * E, hidden=H, inter=I) if shared else None
    layer = Layer(gpu, experts, sh)
    cpu = [oracle.gen_expert(seed, 0x1000 + 4 * e, hidden=H, inter=I) for e in range(E)]
    cpu_sh = oracle.gen_expert(seed, 0x1000 + 4 * E, hidden=H, inter=I) if shared else None
    return layer, experts, sh, cpu, cpu_sh


def _free(layer, experts, sh):
    torch.cuda.synchronize()
    layer.close()
    for e in experts:
        e.free()
    if sh is not None:
        sh.free()


def _oracle_moe(oracle, cpu, cpu_sh, x_f32, ids, wts):
    """combine_outputs_torch order: y = sum_k w_k * y_k (fp32), then + shared."""
    T = x_f32.shape[0]
    out = np.zeros((T, x_f32.shape[1]), np.float32)
    cache = {}
    for t in range(T):
        acc = np.zeros(x_f32.shape[1], np.float32)
        for e, w in zip(ids[t], wts[t]):
            if e < 0:
                continue
            key = (int(e), t)
            if key not in cache:
                cache[key] = oracle.expert_ref(cpu[int(e)], x_f32[t:t + 1])[1][0]
            acc = acc + np.float32(w) * cache[key]
        if cpu_sh is not None:
            acc = acc + oracle.expert_ref(cpu_sh, x_f32[t:t + 1])[1][0]
        out[t] = acc
    return out


@pytest.mark.parametrize("T,prefill,I", [(1, False, 512), (3, False, 512), (4, False, 512),
                                         (16, False, 512), (23, True, 512), (70, True, 512),
                                         (2, False, 256), (40, True, 256)])
def test_moe_grouped_vs_oracle(gpu, oracle, T, prefill, I):
    """T <= 16: the decode pipeline (I=512, a shape it compiles) or the general
    per-item path (I=256); T > 16: the prefill grouped GEMM."""
    print(f"[moe] T={T} prefill={prefill} I={I}", flush=True)
    E, H = 32, 1024
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=11)
    try:
        x, w, bias = _router_inputs(gpu, 12, T, E, H, bias_skew=0.3 if T > 16 else 0.0)
        ids, wts = gpu.route(x, w, bias, n_group=8, topk_group=4, top_k=8)
        y, yf = gpu.moe(layer, x, ids, wts, want_f32=True, prefill=prefill)
        gpu.sync()
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids.cpu().numpy(),
                          wts.cpu().numpy())
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.abs(yf - ref).max() < 2e-2
        assert np.array_equal(_bits(y), oracle.encode_act(yf, BF16, "rne"))
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("H,I,E,T,K,dtype,shared", [
    (1024, 512, 5, 160, 4, torch.bfloat16, True),
    (2048, 1024, 4, 136, 4, torch.float16, False),
    (1024, 2048, 6, 200, 4, torch.bfloat16, True)])
def test_moe_many_tokens_per_expert(gpu, oracle, H, I, E, T, K, dtype, shared):
    """Calls with >= 128 pairs per routed expert on average take 128-pair
    items through the LDS-ring GEMM: experts cut into a full item plus a
    partial one, or a single partial item; hidden of 8 and 16 k-blocks,
    inter of 4, 8 and 16; bf16 and fp16 activations.  Every token against
    the oracle."""
    print(f"[moe] many tokens per expert H={H} I={I} E={E} T={T}", flush=True)
    assert T * K >= 128 * E
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=61 + E, shared=shared)
    try:
        x = gpu.gen_normal(62 + E, 1, (T, H), 1.0, dtype)
        rng = np.random.default_rng(E)
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        want_f32=True, prefill=True)
        gpu.sync()
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids, wts)
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.abs(yf - ref).max() < 2e-2
        code = BF16 if dtype == torch.bfloat16 else FP16
        assert np.array_equal(_bits(y), oracle.encode_act(yf, code, "rne"))
    finally:
        _free(layer, experts, sh)


def test_many_tokens_per_resident_expert(gpu, oracle):
    """A node's share: 4 of 16 experts resident, 160 tokens x 4 routes over
    them (160 pairs per resident expert), so the LDS-ring GEMM serves the call
    although 640 routes are few for all 16 slots.  Every token against the
    oracle; the layer table's empty slots are never read."""
    print("[moe] many tokens per resident expert", flush=True)
    from constellation_amd.engine import Expert, Layer
    E, H, I, T, K = 16, 1024, 512, 160, 4
    res = [1, 5, 9, 13]
    experts = [Expert.generate(0, 75, 0x1000 + 4 * e, hidden=H, inter=I) if e in res else None for e in range(E)]
    layer = Layer(gpu, experts, None)
    try:
        cpu = [oracle.gen_expert(75, 0x1000 + 4 * e, hidden=H, inter=I) if e in res else None for e in range(E)]
        x = gpu.gen_normal(76, 1, (T, H), 1.0, torch.bfloat16)
        rng = np.random.default_rng(77)
        ids = np.stack([rng.permutation(res) for _ in range(T)]).astype(np.int32)
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        want_f32=True, prefill=True)
        gpu.sync()
        ref = _oracle_moe(oracle, cpu, None, x.float().cpu().numpy(), ids, wts)
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.abs(yf - ref).max() < 2e-2
        assert np.array_equal(_bits(y), oracle.encode_act(yf, BF16, "rne"))
    finally:
        torch.cuda.synchronize()
        layer.close()
        for e in experts:
            if e is not None:
                e.free()


def test_planner_many_routes_vs_oracle(gpu, oracle):
    """4800 routes (1200 tokens x 4): more than the planner held in LDS as
    32-bit ids; staged as 16-bit ids with the validity bits in registers.
    Every token against the oracle (shared expert on, the LDS-ring GEMM)."""
    print("[moe] planner 4800 routes", flush=True)
    E, H, I, T, K = 8, 1024, 512, 1200, 4
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=64, shared=True)
    try:
        x = gpu.gen_normal(65, 1, (T, H), 1.0, torch.bfloat16)
        rng = np.random.default_rng(66)
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        want_f32=True, prefill=True)
        gpu.sync()
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids, wts)
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.abs(yf - ref).max() < 2e-2
        assert np.array_equal(_bits(y), oracle.encode_act(yf, BF16, "rne"))
    finally:
        _free(layer, experts, sh)


def test_planner_beyond_staging_matches_chunks(gpu, oracle):
    """68,000 routes (17,000 tokens x 4) exceed what the staged planner holds
    (64 per thread) and take the general planner; the same routes in four
    chunks take the staged one.  A pair's value does not depend on its item's
    other pairs, so the outputs are bit-identical."""
    print("[moe] planner beyond staging", flush=True)
    E, H, I, T, K = 4, 1024, 512, 17000, 4
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=67, shared=False)
    try:
        x = gpu.gen_normal(68, 1, (T, H), 1.0, torch.bfloat16)
        rng = np.random.default_rng(69)
        ids = torch.from_numpy(np.stack([rng.permutation(E) for _ in range(T)]).astype(np.int32)).cuda()
        wts = torch.from_numpy(rng.uniform(0.05, 1.0, (T, K)).astype(np.float32)).cuda()
        y_all, yf_all = gpu.moe(layer, x, ids, wts, want_f32=True, prefill=True)
        parts = [gpu.moe(layer, x[c:c + 4250], ids[c:c + 4250], wts[c:c + 4250], want_f32=True, prefill=True)[1]
                 for c in range(0, T, 4250)]
        gpu.sync()
        assert torch.equal(yf_all, torch.cat(parts))
        sel = np.array([0, 4249, 4250, 9000, 16999])
        ref = _oracle_moe(oracle, cpu, None, x.float().cpu().numpy()[sel], ids.cpu().numpy()[sel],
                          wts.cpu().numpy()[sel])
        got = yf_all.cpu().numpy()[sel]
        assert rel_l2(got, ref) < 1e-5 and np.abs(got - ref).max() < 2e-2
    finally:
        _free(layer, experts, sh)


def test_full_size_many_tokens_per_expert(gpu, oracle):
    """DeepSeek-V3 shapes (H=7168, I=2048) through the LDS-ring GEMM: 8
    routed experts + shared, 256 tokens x 4 routes (128 pairs per expert on
    average).  Every token against the oracle fed the device-resident
    weights, and against the decode pipeline."""
    print("[moe] full-size many tokens per expert", flush=True)
    E, H, T, K = 8, 7168, 256, 4
    from constellation_amd.engine import Expert, Layer
    experts = [Expert.generate(0, 71, 0x5000 + 4 * e) for e in range(E)]
    sh = Expert.generate(0, 71, 0x5000 + 4 * E)
    layer = Layer(gpu, experts, sh)
    try:
        x = gpu.gen_normal(72, 1, (T, H), 1.0, torch.bfloat16)
        rng = np.random.default_rng(73)
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        ids_d, wts_d = torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda()
        y, yf = gpu.moe(layer, x, ids_d, wts_d, want_f32=True, prefill=True)
        gpu.sync()
        ref = _oracle_moe_all_tokens(oracle, experts, sh, x.float().cpu().numpy(), ids, wts)
        got = yf.cpu().numpy()
        assert rel_l2(got, ref) < 1e-5, rel_l2(got, ref)  # all 256 tokens
        assert np.abs(got - ref).max() < 2e-2
        assert np.array_equal(_bits(y), oracle.encode_act(got, BF16, "rne"))
        _decode_paths_agree(gpu, layer, x, ids_d, wts_d, yf)
    finally:
        _free(layer, experts, sh)


def test_moe_prefill_hot_expert_splits_items(gpu, oracle):
    """One expert routed by every token (> 64 pairs -> several work items)."""
    print("[moe] hot expert", flush=True)
    E, H, I, T = 16, 1024, 512, 150
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=21, shared=False)
    try:
        x = gpu.gen_normal(22, 1, (T, H), 1.0, torch.float16)
        rng = np.random.default_rng(0)
        ids = np.stack([np.concatenate([[3], rng.choice([e for e in range(E) if e != 3], 3, replace=False)])
                        for _ in range(T)]).astype(np.int32)
        wts = rng.uniform(0.1, 1.0, ids.shape).astype(np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        want_f32=True, prefill=True)
        gpu.sync()
        ref = _oracle_moe(oracle, cpu, None, x.float().cpu().numpy(), ids, wts)
        assert rel_l2(yf.cpu().numpy(), ref) < 1e-5
    finally:
        _free(layer, experts, sh)


def test_moe_layer_fused_router(gpu, oracle):
    print("[moe] fused layer", flush=True)
    E, H, I, T = 32, 1024, 512, 3
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=31)
    try:
        x, w, bias = _router_inputs(gpu, 32, T, E, H)
        y, yf, ids, wts = gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=4, top_k=8,
                                        want_f32=True)
        gpu.sync()
        for t, (oi, ow, _, _) in enumerate(_oracle_route(oracle, x, w, bias)):
            assert ids[t].cpu().tolist() == oi.tolist()
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids.cpu().numpy(),
                          wts.cpu().numpy())
        assert rel_l2(yf.cpu().numpy(), ref) < 1e-5
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("T,norm,scale,K", [(1, False, 1.0, 8), (1, True, 1.7, 1), (1, False, 2.5, 4),
                                             (3, False, 2.5, 6), (40, False, 0.5, 8)])
def test_moe_layer_router_options(gpu, oracle, T, norm, scale, K):
    """Router options beyond DeepSeek-V3's defaults through cx_moe_layer:
    weights left unnormalised, other routed scaling factors and a single
    pick (no normalisation at k = 1, server/moe_layer_runtime.py:376-379).  T = 1
    takes the one-token pipeline (selection inside the routed gate/up), T = 3
    the staged decode pipeline, T = 40 the grouped prefill path; routes and
    weights against the oracle's, output within the parity bound."""
    print(f"[moe] router options T={T} norm={norm} scale={scale} K={K}", flush=True)
    E, H, I = 256, 1024, 512
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=130 + T)
    try:
        x, w, bias = _router_inputs(gpu, 131 + T + K, T, E, H)
        y, yf, ids, wts = gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=4, top_k=K,
                                        norm_topk_prob=norm, routed_scaling_factor=scale,
                                        want_f32=True)
        gpu.sync()
        checked = 0
        for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias, top_k=K,
                                                               norm=norm, scale=scale)):
            if min(margins) <= 1e-12:
                continue
            assert ids[t].cpu().tolist() == oi.tolist(), t
            assert np.allclose(wts[t].cpu().numpy(), ow, rtol=1e-6, atol=0), t
            checked += 1
        assert checked >= T - 1
        if not norm and K > 1:
            # unnormalised: each weight is scale * sigmoid(logit), never a share of 1
            assert not np.allclose(wts.sum(dim=1).cpu().numpy(), scale, rtol=1e-3)
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids.cpu().numpy(),
                          wts.cpu().numpy())
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.array_equal(_bits(y), oracle.encode_act(yf, BF16, "rne"))
    finally:
        _free(layer, experts, sh)


def test_moe_layer_decode_back_to_back(gpu, oracle):
    """The decode pipeline (T <= 16) reuses its plan, h, k-part and y_part
    buffers on every call.  Twelve calls back to back with new tokens (and
    T = 1, 2, 3 in turn), one sync at the end: each output must match the
    oracle, which stale data from an earlier call would not."""
    print("[moe] decode back to back", flush=True)
    E, H, I = 32, 1024, 512
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=41)
    try:
        _, w, bias = _router_inputs(gpu, 42, 1, E, H)
        outs = []
        for i in range(12):
            x = gpu.gen_normal(43 + i, 3, (1 + i % 3, H), 1.0, torch.bfloat16)
            _, yf, ids, wts = gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=4, top_k=8,
                                            want_f32=True)
            outs.append((x, yf, ids, wts))
        gpu.sync()
        for x, yf, ids, wts in outs:
            ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids.cpu().numpy(),
                              wts.cpu().numpy())
            assert rel_l2(yf.cpu().numpy(), ref) < 1e-5
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("prefill", [False, True])
def test_moe_bad_and_missing_experts_reported(gpu, prefill):
    print(f"[moe] error flags prefill={prefill}", flush=True)
    from constellation_amd import CxError
    from constellation_amd.engine import Expert, Layer
    H, I = 1024, 512
    e0 = Expert.generate(0, 1, 0x10, hidden=H, inter=I)
    layer = Layer(gpu, [e0, None, None, None])
    try:
        x = gpu.gen_normal(1, 1, (2, H), 1.0, torch.bfloat16)
        ids = torch.tensor([[0, 7], [0, 2]], dtype=torch.int32, device="cuda")
        w = torch.ones((2, 2), dtype=torch.float32, device="cuda")
        gpu.moe(layer, x, ids, w, prefill=prefill)
        with pytest.raises(CxError):
            gpu.sync()
        gpu.sync()  # flag cleared
    finally:
        torch.cuda.synchronize()
        layer.close()
        e0.free()


@pytest.mark.parametrize("T", [1, 16])
def test_full_size_decode_layer(gpu, oracle, T):
    """DeepSeek-V3 shapes: 8 routed of 64 resident + shared, H=7168, I=2048."""
    print(f"[moe] full size T={T}", flush=True)
    E, H, I = 64, 7168, 2048
    from constellation_amd.engine import Expert, Layer
    experts = [Expert.generate(0, 41, 0x2000 + 4 * e) for e in range(E)]
    sh = Expert.generate(0, 41, 0x2000 + 4 * E)
    layer = Layer(gpu, experts, sh)
    try:
        x, w, bias = _router_inputs(gpu, 42, T, E, H)
        ids, wts = gpu.route(x, w, bias, n_group=8, topk_group=4, top_k=8)
        y, yf = gpu.moe(layer, x, ids, wts, want_f32=True)
        gpu.sync()
        idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
        used = sorted(set(idn.ravel().tolist()))
        cpu = {e: oracle.gen_expert(41, 0x2000 + 4 * e) for e in used}
        cpu_sh = oracle.gen_expert(41, 0x2000 + 4 * E)
        ref = _oracle_moe(oracle, [cpu.get(e) for e in range(E)], cpu_sh,
                          x.float().cpu().numpy(), idn, wn)
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5 and np.abs(yf - ref).max() < 2e-2
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("T,prefill", [(1, False), (2, False), (20, True)])
def test_moe_duplicate_route_is_dropped_and_reported(gpu, oracle, T, prefill):
    """validate_routes (server/moe_layer_runtime.py:84-98) rejects a token that
    lists the same expert twice; the engine drops the repeat and reports it."""
    print(f"[moe] duplicate routes T={T}", flush=True)
    from constellation_amd import CxError
    E, H, I = 8, 1024, 512
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=51, shared=False)
    try:
        x = gpu.gen_normal(52, 1, (T, H), 1.0, torch.bfloat16)
        ids = np.tile(np.array([[1, 3]], np.int32), (T, 1))
        ids[0] = [2, 2]
        wts = np.full(ids.shape, 0.5, np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        want_f32=True, prefill=prefill)
        with pytest.raises(CxError):
            gpu.sync()
        kept = ids.copy()
        kept[0] = [2, -1]
        ref = _oracle_moe(oracle, cpu, None, x.float().cpu().numpy(), kept, wts)
        assert rel_l2(yf.cpu().numpy(), ref) < 1e-5
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("H,I,shared,K,dtype,odtype", [
    (1024, 512, True, 8, torch.bfloat16, torch.bfloat16),
    (1024, 1024, False, 4, torch.float16, torch.float16),
    (2048, 2048, True, 6, torch.bfloat16, torch.float16),
    (1024, 512, True, 1, torch.float16, torch.bfloat16),
    (1024, 2048, False, 8, torch.bfloat16, torch.bfloat16),
    (1792, 2048, True, 8, torch.bfloat16, torch.bfloat16),
    (1792, 1024, False, 7, torch.float16, torch.bfloat16)])
def test_one_token_down_combine(gpu, oracle, H, I, shared, K, dtype, odtype):
    """One token (cx_moe_decode, routes given): the down projection of every
    item and the weighted combine run as one launch (k_down_comb1) for top_k
    <= 8 — inter of 4, 8 and 16 k-blocks, with and without a shared expert,
    fewer routes than waves, mixed in/out dtypes.  Hidden 1792 on a 256-CU
    device runs 14-row tiles (128 workgroups), some of which straddle two
    128-row scale blocks; the 16-row cases keep whole tiles."""
    print(f"[moe] one-token down+combine H={H} I={I} shared={shared} K={K}", flush=True)
    E = 16
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=81 + K, shared=shared)
    try:
        x = gpu.gen_normal(82 + K, 1, (1, H), 1.0, dtype)
        rng = np.random.default_rng(K)
        ids = rng.choice(E, size=(1, K), replace=False).astype(np.int32)
        wts = rng.uniform(0.1, 1.0, size=(1, K)).astype(np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        out_dtype=odtype, want_f32=True)
        gpu.sync()
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids, wts)
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.abs(yf - ref).max() < 2e-2
        code = BF16 if odtype == torch.bfloat16 else FP16
        assert np.array_equal(_bits(y), oracle.encode_act(yf, code, "rne"))
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("T,E,shared,wdtype,mask", [
    (1, 64, True, torch.bfloat16, False), (1, 128, True, torch.float32, False),
    (1, 256, False, torch.bfloat16, False), (2, 64, True, torch.bfloat16, False),
    (5, 128, True, torch.float32, False), (16, 64, True, torch.bfloat16, False),
    (3, 256, False, torch.bfloat16, False), (4, 64, True, torch.bfloat16, True),
    (16, 256, True, torch.bfloat16, True)])
def test_moe_layer_decode_pipeline(gpu, oracle, T, E, shared, wdtype, mask):
    """cx_moe_layer for T <= 16 and register-selectable expert counts: router
    logits beside the shared expert's gate/up, selection + planner beside the
    shared expert's down, routed gate/up, routed down + combine + shared."""
    print(f"[moe] decode pipeline T={T} E={E} shared={shared} w={wdtype} mask={mask}", flush=True)
    H, I = 1024, 512
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=61 + T, shared=shared)
    try:
        x, w, bias = _router_inputs(gpu, 62 + T, T, E, H)
        w = w.to(wdtype)
        res = None
        rdev = None
        if mask:
            res = np.zeros(E, np.uint8)
            res[::3] = 1
            rdev = torch.from_numpy(res).cuda()
        y, yf, ids, wts = gpu.moe_layer(layer, x, w, bias, resident=rdev, n_group=8, topk_group=4,
                                        top_k=8, want_f32=True)
        gpu.sync()
        for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias, resident=res)):
            if min(margins) <= 1e-12:
                continue
            k = len(oi)
            assert ids[t].cpu().tolist()[:k] == oi.tolist(), t
            assert np.allclose(wts[t].cpu().numpy()[:k], ow, rtol=1e-6, atol=0), t
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids.cpu().numpy(),
                          wts.cpu().numpy())
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.abs(yf - ref).max() < 2e-2
        assert np.array_equal(_bits(y), oracle.encode_act(yf, BF16, "rne"))
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("E,H,I,shared,TG,K", [(256, 1024, 512, True, 4, 8),
                                               (256, 1024, 512, False, 3, 6),
                                               (256, 7168, 2048, True, 4, 8)])
def test_one_token_fused_selection_equals_staged(gpu, oracle, E, H, I, shared, TG, K):
    """At one token without a resident mask, cx_moe_layer selects inside the
    routed gate/up launch (every workgroup selects for itself).  A resident
    mask of all ones selects the same experts through the staged pipeline
    (selection + planner launch).  Both sum each router row's exact fp64
    products, over 512 and 256 threads, so a logit can differ in its last
    fp64 bit and a weight, rarely, by one fp32 ulp: routes must be equal,
    weights within one ulp, and where the weights are equal (all but a
    ~1e-9 chance) both outputs bit-identical.  Several tokens in turn (no
    state carried between calls); the routes equal the oracle's."""
    print(f"[moe] fused selection E={E} H={H} shared={shared} TG={TG} K={K}", flush=True)
    if H == 7168:
        from constellation_amd.engine import Expert, Layer
        experts = [Expert.generate(0, 95, 0x5800 + 4 * e) for e in range(E)]
        sh = Expert.generate(0, 95, 0x5800 + 4 * E) if shared else None
        layer = Layer(gpu, experts, sh)
    else:
        layer, experts, sh, _, _ = _make_layer(gpu, oracle, E, H, I, seed=95, shared=shared)
    try:
        _, w, bias = _router_inputs(gpu, 96, 1, E, H)
        ones = torch.ones(E, dtype=torch.uint8, device="cuda")
        for i in range(4):
            x = gpu.gen_normal(97 + i, 3, (1, H), 1.0, torch.bfloat16)
            a = gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=TG, top_k=K, want_f32=True)
            b = gpu.moe_layer(layer, x, w, bias, resident=ones, n_group=8, topk_group=TG, top_k=K,
                              want_f32=True)
            gpu.sync()
            ya, yfa, ida, wa = (t.cpu() for t in a)
            yb, yfb, idb, wb = (t.cpu() for t in b)
            assert torch.equal(ida, idb), i
            ulps = (wa.view(torch.int32).long() - wb.view(torch.int32).long()).abs()
            assert int(ulps.max()) <= 1, i
            if int(ulps.max()) == 0:
                assert torch.equal(yfa.view(torch.int32), yfb.view(torch.int32)), i
                assert torch.equal(ya.view(torch.int16), yb.view(torch.int16)), i
            else:
                assert rel_l2(yfa.numpy(), yfb.numpy()) < 1e-6, i
            oi, ow, margins, _ = _oracle_route(oracle, x, w, bias, n_group=8, topk_group=TG,
                                               top_k=K)[0]
            if min(margins) > 1e-12:
                assert ida[0].tolist() == oi.tolist(), i
                assert np.allclose(wa[0].numpy(), ow, rtol=1e-6, atol=0), i
    finally:
        _free(layer, experts, sh)


def test_one_token_fused_selection_ties(gpu, oracle):
    """The fused one-token selection decides most picks on float keys and
    falls back to exact fp64 when the largest key is shared.  Router rows
    that saturate the sigmoid (s = 1 exactly) and chosen biases make the
    choice scores c = 1 + bias: an exact 3-way tie (experts 100-102), a
    pair 2^-41 apart (41 above 40: one float key, two fp64 values), an
    exact 2-way tie (3, 7) and a distinct pair (200 above 201), in four
    groups.  The picks must come in c order, ties to the lower index, and
    equal the staged pipeline's; all eight weights equal."""
    print("[moe] fused selection ties", flush=True)
    E, H, I = 256, 1024, 512
    layer, experts, sh, _, _ = _make_layer(gpu, oracle, E, H, I, seed=98, shared=True)
    try:
        x, w, bias = _router_inputs(gpu, 99, 1, E, H)
        boost = torch.where(x[0] >= 0, 0.05, -0.05).to(torch.bfloat16)
        u = 2.0 ** -20
        plan = {100: 5 * u, 101: 5 * u, 102: 5 * u, 40: 4 * u, 41: 4 * u + 2.0 ** -41,
                3: 3 * u, 7: 3 * u, 200: 2 * u, 201: u}
        for e, b in plan.items():
            w[e] = boost
            bias[e] = b
        assert float(bias[41]) != float(bias[40])  # representable apart in fp32
        ones = torch.ones(E, dtype=torch.uint8, device="cuda")
        a = gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=4, top_k=8, want_f32=True)
        b = gpu.moe_layer(layer, x, w, bias, resident=ones, n_group=8, topk_group=4, top_k=8,
                          want_f32=True)
        gpu.sync()
        ya, yfa, ida, wa = (t.cpu() for t in a)
        yb, yfb, idb, wb = (t.cpu() for t in b)
        assert ida[0].tolist() == [100, 101, 102, 41, 40, 3, 7, 200], ida
        assert torch.equal(ida, idb)
        assert torch.equal(wa, wb) and torch.all(wa == wa[0, 0])
        assert torch.equal(yfa.view(torch.int32), yfb.view(torch.int32))
        assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("T,dtype", [(1, torch.float16), (7, torch.bfloat16), (16, torch.float16)])
def test_moe_decode_given_routes_with_shared(gpu, oracle, T, dtype):
    """cx_moe_decode (routes given): planner beside the shared expert's gate/up,
    then routed gate/up and the down + combine over every slot."""
    print(f"[moe] decode given routes T={T} {dtype}", flush=True)
    E, H, I = 48, 1024, 512
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=71 + T)
    try:
        x = gpu.gen_normal(72 + T, 1, (T, H), 1.0, dtype)
        rng = np.random.default_rng(T)
        ids = np.stack([rng.choice(E, 6, replace=False) for _ in range(T)]).astype(np.int32)
        ids[0, 5] = -1  # an empty slot
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        want_f32=True)
        gpu.sync()
        ref = _oracle_moe(oracle, cpu, cpu_sh, x.float().cpu().numpy(), ids, wts)
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        enc = FP16 if dtype == torch.float16 else BF16
        assert np.array_equal(_bits(y), oracle.encode_act(yf, enc, "rne"))
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("T", [1, 3, 8, 9, 16])
def test_full_size_moe_layer(gpu, oracle, T):
    """The benchmark path at DeepSeek-V3 shapes: cx_moe_layer with 256 resident
    experts + shared, H=7168, I=2048, bf16 router (config 1 / config 2).  T
    spans the decode regimes: activation rows staged in LDS (T <= 3), the
    shared expert's two-k-part stage 2 (T <= 8) and its full-K form (T > 8)."""
    print(f"[moe] full-size layer T={T}", flush=True)
    E, H = 256, 7168
    from constellation_amd.engine import Expert, Layer
    experts = [Expert.generate(0, 81, 0x3000 + 4 * e) for e in range(E)]
    sh = Expert.generate(0, 81, 0x3000 + 4 * E)
    layer = Layer(gpu, experts, sh)
    try:
        x, w, bias = _router_inputs(gpu, 82 + T, T, E, H)
        y, yf, ids, wts = gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=4, top_k=8,
                                        routed_scaling_factor=2.5, want_f32=True)
        gpu.sync()
        idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
        for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias)):
            if min(margins) <= 1e-12:
                continue
            assert idn[t].tolist() == oi.tolist(), t
        used = sorted(set(idn.ravel().tolist()) - {-1})
        cpu = {e: oracle.gen_expert(81, 0x3000 + 4 * e) for e in used}
        cpu_sh = oracle.gen_expert(81, 0x3000 + 4 * E)
        ref = _oracle_moe(oracle, [cpu.get(e) for e in range(E)], cpu_sh,
                          x.float().cpu().numpy(), idn, wn)
        yf = yf.cpu().numpy()
        assert rel_l2(yf, ref) < 1e-5 and np.abs(yf - ref).max() < 2e-2
        assert np.array_equal(_bits(y), oracle.encode_act(yf, BF16, "rne"))
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("T", [1, 16])
def test_full_size_moe_layer_run_to_run_exact(gpu, oracle, T):
    """The reference's router stability check (server/test/
    1_smoke_moe_router_validation.py:16-17, 96-172): hidden = linspace(-1e-2,
    1e-2, hidden_size) in the runtime dtype, the MoE layer run 10 times; the
    top-k indices and weights must not change and the output must be finite.
    Here the whole output is also bit-identical run to run (every reduction
    has a fixed order), at DeepSeek-V3 shapes; T = 16 scales the row per token."""
    print(f"[moe] run to run T={T}", flush=True)
    E, H = 256, 7168
    from constellation_amd.engine import Expert, Layer
    experts = [Expert.generate(0, 83, 0x5000 + 4 * e) for e in range(E)]
    sh = Expert.generate(0, 83, 0x5000 + 4 * E)
    layer = Layer(gpu, experts, sh)
    try:
        _, w, bias = _router_inputs(gpu, 84, 1, E, H)
        row = torch.linspace(-1e-2, 1e-2, H, dtype=torch.float32)
        x = torch.stack([row * (1.0 + 0.25 * t) for t in range(T)]).to(torch.bfloat16).cuda()
        runs = [gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=4, top_k=8,
                              routed_scaling_factor=2.5, want_f32=True) for _ in range(10)]
        gpu.sync()
        y0, yf0, ids0, w0 = (t.cpu() for t in runs[0])
        assert torch.isfinite(yf0).all()
        for y, yf, ids, wts in runs[1:]:
            assert torch.equal(ids.cpu(), ids0)
            assert torch.equal(wts.cpu().view(torch.int32), w0.view(torch.int32))
            assert torch.equal(y.cpu().view(torch.int16), y0.view(torch.int16))
            assert torch.equal(yf.cpu().view(torch.int32), yf0.view(torch.int32))
        for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias)):
            if min(margins) > 1e-12:
                assert ids0[t].tolist() == oi.tolist(), t
    finally:
        _free(layer, experts, sh)


def _oracle_moe_all_tokens(oracle, experts, shared, x_f32, ids, wts):
    """Every token against the oracle (cxo_expert_ref), fed the weights the
    device holds (Expert.download(); the generator tests hold them
    bit-identical to the oracle's own generator), one expert at a time: each
    (token, route) output y_k, then the combine_outputs_torch order
    (moe_layer_runtime.py:148-167), sum_k w_k * y_k in fp32 in route order,
    and the shared expert added last (full_model_runtime.py:348)."""
    T, H = x_f32.shape
    K = ids.shape[1]
    yk = np.zeros((T, K, H), np.float32)
    for e in sorted(set(ids[ids >= 0].tolist())):
        tk = np.argwhere(ids == e)
        _, y = oracle.expert_ref(experts[e].download(), x_f32[tk[:, 0]])
        yk[tk[:, 0], tk[:, 1]] = y
    out = np.zeros((T, H), np.float32)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for k in range(K):
            if ids[t, k] >= 0:
                acc = acc + np.float32(wts[t, k]) * yk[t, k]
        out[t] = acc
    if shared is not None:
        out = out + oracle.expert_ref(shared.download(), x_f32)[1]
    return out


def _downloaded_equals_generated(oracle, expert, seed, stream_base):
    """The device bytes of one expert equal the oracle generator's."""
    got, want = expert.download(), oracle.gen_expert(seed, stream_base)
    for k in ("w_up", "s_up", "w_gate", "s_gate", "w_down", "s_down"):
        assert np.array_equal(got[k], want[k]), k


def _decode_paths_agree(gpu, layer, x, ids, wts, yf_grouped):
    """Every token of a grouped (prefill) call again through the decode
    pipeline, which shares no GEMM kernel with it: alternate 16-token blocks
    one token per call (routed gate/up + the one-launch down/combine) and 16
    tokens per call (the B=16 kernels).  Both sum exact fp8 x activation
    products in fp32, in different k orders, so they agree to rounding."""
    T = x.shape[0]
    outs = []
    for t0 in range(0, T, 16):
        t1 = min(T, t0 + 16)
        if (t0 // 16) % 2 == 0:
            for t in range(t0, t1):
                outs.append(gpu.moe(layer, x[t:t + 1], ids[t:t + 1], wts[t:t + 1], want_f32=True)[1])
        else:
            outs.append(gpu.moe(layer, x[t0:t1], ids[t0:t1], wts[t0:t1], want_f32=True)[1])
    gpu.sync()
    dec = torch.cat(outs).cpu().numpy()
    grp = yf_grouped.cpu().numpy()
    assert rel_l2(dec, grp) < 1e-5, rel_l2(dec, grp)
    assert np.abs(dec - grp).max() < 1e-2


def test_config3_prefill_chunk_matches_oracle(gpu, oracle):
    """The config-3 benchmark call: 512 tokens through cx_moe_layer with a
    Zipf-skewed correction bias, 256 experts + shared at DeepSeek-V3 shapes
    (hot experts split into several 64-pair items).  Every token's routes
    against the oracle; every token's output against the dequantise-then-fp32
    oracle fed the device-resident weights, and against the decode pipeline;
    the 16-bit output equals RNE of the fp32 output."""
    print("[moe] config-3 prefill chunk", flush=True)
    E, H, T = 256, 7168, 512
    from constellation_amd.engine import Expert, Layer
    experts = [Expert.generate(0, 85, 0x6000 + 4 * e) for e in range(E)]
    sh = Expert.generate(0, 85, 0x6000 + 4 * E)
    layer = Layer(gpu, experts, sh)
    try:
        x, w, bias = _router_inputs(gpu, 86, T, E, H, bias_skew=0.25)
        y, yf, ids, wts = gpu.moe_layer(layer, x, w, bias, n_group=8, topk_group=4, top_k=8,
                                        routed_scaling_factor=2.5, want_f32=True)
        gpu.sync()
        idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
        assert np.bincount(idn[idn >= 0]).max() > 64  # a hot expert spans several items
        for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias)):
            if min(margins) > 1e-12:
                assert idn[t].tolist() == oi.tolist(), t
                assert np.allclose(wn[t], ow, rtol=1e-6, atol=0), t
        hot = int(np.bincount(idn[idn >= 0]).argmax())
        _downloaded_equals_generated(oracle, experts[hot], 85, 0x6000 + 4 * hot)
        ref = _oracle_moe_all_tokens(oracle, experts, sh, x.float().cpu().numpy(), idn, wn)
        got = yf.cpu().numpy()
        assert rel_l2(got, ref) < 1e-5 and np.abs(got - ref).max() < 2e-2  # all 512 tokens
        for t in range(T):
            assert rel_l2(got[t], ref[t]) < 1e-5, t
        assert np.array_equal(_bits(y), oracle.encode_act(got, BF16, "rne"))
        _decode_paths_agree(gpu, layer, x, ids, wts, yf)
    finally:
        _free(layer, experts, sh)


def test_config4_node_share_layer_matches_oracle(gpu, oracle):
    """One layer of the config-4 node share: 64 resident experts of 256 (e = 0
    mod 4), no shared expert, 32 tokens routed under the resident mask with a
    Zipf-skewed bias (the grouped path).  Routes against the oracle's masked
    router; every token's output against the oracle fed the device-resident
    weights, and against the decode pipeline."""
    print("[moe] config-4 node-share layer", flush=True)
    E, H, T = 256, 7168, 32
    from constellation_amd.engine import Expert, Layer
    res = np.zeros(E, np.uint8)
    res[::4] = 1
    experts = [Expert.generate(0, 87, 0x7000 + 4 * e) if res[e] else None for e in range(E)]
    layer = Layer(gpu, experts, None)
    try:
        x, w, bias = _router_inputs(gpu, 88, T, E, H, bias_skew=0.25)
        y, yf, ids, wts = gpu.moe_layer(layer, x, w, bias, resident=torch.from_numpy(res).cuda(),
                                        n_group=8, topk_group=4, top_k=8, routed_scaling_factor=2.5,
                                        want_f32=True)
        gpu.sync()
        idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
        assert all(res[e] for e in idn[idn >= 0])
        for t, (oi, ow, margins, _) in enumerate(_oracle_route(oracle, x, w, bias, resident=res)):
            if min(margins) > 1e-12:
                assert idn[t][:len(oi)].tolist() == oi.tolist(), t
        hot = int(np.bincount(idn[idn >= 0]).argmax())
        _downloaded_equals_generated(oracle, experts[hot], 87, 0x7000 + 4 * hot)
        ref = _oracle_moe_all_tokens(oracle, experts, None, x.float().cpu().numpy(), idn, wn)
        got = yf.cpu().numpy()
        assert rel_l2(got, ref) < 1e-5 and np.abs(got - ref).max() < 2e-2  # all 32 tokens
        for t in range(T):
            assert rel_l2(got[t], ref[t]) < 1e-5, t
        assert np.array_equal(_bits(y), oracle.encode_act(got, BF16, "rne"))
        _decode_paths_agree(gpu, layer, x, ids, wts, yf)
    finally:
        torch.cuda.synchronize()
        layer.close()
        for e in experts:
            if e is not None:
                e.free()


def test_device_probe_invariants(gpu):
    """The reference's device-probe invariants (cpu/tests/test_gpu_info_cpu_v2.cc:
    40-100): a non-empty name, total and free memory above zero; plus the
    gfx950 architecture and its fp16/bf16/fp8 capability bits."""
    from constellation_amd.engine import device_count, device_info
    assert device_count() >= 1
    info = device_info(0)
    assert info["name"] and info["arch"].startswith("gfx950")
    assert info["total_mem_bytes"] > 0 and 0 < info["free_mem_bytes"] <= info["total_mem_bytes"]
    assert info["compute_units"] > 0
    assert info["capability_flags"] & 0x7 == 0x7


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_full_size_prefill_grouped_items(gpu, oracle, dtype):
    """The grouped GEMM at DeepSeek-V3 shapes (H=7168, I=2048) with items of
    every width: expert 0 takes all 72 tokens (items of 64 + 8 pairs), expert 1
    40 (3 column tiles), expert 2 20 (2 tiles), the rest a few each (one-tile
    items, which stage x in LDS chunks); shared expert on.  bf16 and fp16
    activations; the oracle checks a sample of tokens spread over the items."""
    print(f"[moe] full-size prefill items {dtype}", flush=True)
    E, H, I, T, K = 16, 7168, 2048, 72, 4
    from constellation_amd.engine import Expert, Layer
    experts = [Expert.generate(0, 91, 0x4000 + 4 * e) for e in range(E)]
    sh = Expert.generate(0, 91, 0x4000 + 4 * E)
    layer = Layer(gpu, experts, sh)
    try:
        x = gpu.gen_normal(92, 1, (T, H), 1.0, dtype)
        rng = np.random.default_rng(93)
        ids = np.full((T, K), -1, np.int32)
        for t in range(T):
            row = [0]
            if t < 40:
                row.append(1)
            if t % 3 == 0 and len(row) < K:
                row.append(2)
            rest = rng.choice(np.arange(3, E), K - len(row), replace=False)
            ids[t] = row + rest.tolist()
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        y, yf = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        want_f32=True, prefill=True)
        gpu.sync()
        sel = np.array([0, 17, 39, 45, 63, 64, 71])
        used = sorted(set(ids[sel].ravel().tolist()))
        cpu = {e: oracle.gen_expert(91, 0x4000 + 4 * e) for e in used}
        cpu_sh = oracle.gen_expert(91, 0x4000 + 4 * E)
        ref = _oracle_moe(oracle, [cpu.get(e) for e in range(E)], cpu_sh,
                          x.float().cpu().numpy()[sel], ids[sel], wts[sel])
        yf = yf.cpu().numpy()[sel]
        assert rel_l2(yf, ref) < 1e-5, rel_l2(yf, ref)
        assert np.abs(yf - ref).max() < 2e-2
        assert np.array_equal(_bits(y)[sel], oracle.encode_act(yf, BF16 if dtype == torch.bfloat16 else FP16, "rne"))
    finally:
        _free(layer, experts, sh)


@pytest.mark.parametrize("T,dtype,shared", [(1, torch.bfloat16, True), (5, torch.float16, True),
                                             (20, torch.bfloat16, True), (3, torch.bfloat16, False)])
def test_moe_layer_request_end_to_end(gpu, oracle, T, dtype, shared):
    """One MoeLayerRequest body in, one MoeLayerResponse body out (host bytes,
    pinned staging): equal bit for bit to the device-pointer path on the same
    routes, and within the parity bound of the oracle's combine."""
    from constellation_amd import moe_layer_protocol as P
    print(f"[moe] layer request T={T} {dtype} shared={shared}", flush=True)
    E, H, I, K = 16, 1024, 512, 4
    layer, experts, sh, cpu, cpu_sh = _make_layer(gpu, oracle, E, H, I, seed=101 + T)
    try:
        x = gpu.gen_normal(102 + T, 1, (T, H), 1.0, dtype)
        rng = np.random.default_rng(T)
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        ids[0, K - 1] = -1  # a route served by another node
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        enc = FP16 if dtype == torch.float16 else BF16
        body = P.encode_moe_layer_request({
            "layer_id": 3, "batch_size": T, "hidden_dim": H, "top_k": K, "input_dtype": enc,
            "output_dtype": enc, "flags": P.FLAG_SHARED if shared else 0, "expert_ids": ids,
            "expert_weights": wts, "activation": x.cpu().view(torch.int16).numpy().tobytes()})
        resp = P.decode_moe_layer_response(gpu.moe_layer_request(layer, body))
        assert resp["status_code"] == 0 and resp["batch_size"] == T and resp["hidden_dim"] == H
        got = np.frombuffer(resp["output"], np.uint16).reshape(T, H)
        if shared:  # the device-pointer path adds the layer's shared expert too
            y = gpu.moe(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(),
                        prefill=T > 16)
            gpu.sync()
            assert np.array_equal(got, _bits(y))
        ref = _oracle_moe(oracle, cpu, cpu_sh if shared else None, x.float().cpu().numpy(), ids, wts)
        yv = oracle.decode_act(got.reshape(-1), enc).reshape(T, H)
        assert rel_l2(yv, ref) < 1e-2 and np.abs(yv - ref).max() < 2e-2
    finally:
        _free(layer, experts, sh)


def test_moe_layer_request_status_codes(gpu, oracle):
    """worker.cc:113-132 codes: 1 unknown expert, 2 not resident (also the
    shared expert asked of a layer without one), 4 execution failure (a
    route listed twice); failures carry no output."""
    from constellation_amd import moe_layer_protocol as P
    from constellation_amd.engine import Expert, Layer
    print("[moe] layer request status codes", flush=True)
    H, I = 1024, 512
    e0 = Expert.generate(0, 1, 0x10, hidden=H, inter=I)
    layer = Layer(gpu, [e0, None, None, None])
    try:
        x = gpu.gen_normal(1, 1, (2, H), 1.0, torch.bfloat16)
        act = x.cpu().view(torch.int16).numpy().tobytes()

        def run(ids, flags=0, wts=None):
            ids = np.asarray(ids, np.int32)
            if wts is None:
                wts = np.full(ids.shape, 0.5, np.float32)
            body = P.encode_moe_layer_request({
                "layer_id": 0, "batch_size": 2, "hidden_dim": H, "top_k": ids.shape[1],
                "input_dtype": BF16, "output_dtype": BF16, "flags": flags, "expert_ids": ids,
                "expert_weights": np.asarray(wts, np.float32), "activation": act})
            return P.decode_moe_layer_response(gpu.moe_layer_request(layer, body))

        ok = run([[0, -1], [0, -1]])
        assert ok["status_code"] == 0 and len(ok["output"]) == 2 * H * 2
        for ids, flags, code in (([[0, 7], [0, -1]], 0, 1), ([[0, 2], [0, -1]], 0, 2),
                                 ([[0, -1], [0, -1]], P.FLAG_SHARED, 2), ([[0, 0], [0, -1]], 0, 4)):
            r = run(ids, flags)
            assert r["status_code"] == code and r["output"] == b"", (ids, flags, r["status_code"])
        # validate_routes (server/moe_layer_runtime.py:96-97): a negative weight is
        # refused; so is a non-finite one.  The weight of an absent route (-1) is unused.
        for bad in (-0.25, float("nan"), float("inf")):
            r = run([[0, -1], [0, -1]], wts=[[bad, 0.5], [0.5, 0.5]])
            assert r["status_code"] == 4 and r["output"] == b"", bad
        assert run([[0, -1], [0, -1]], wts=[[0.5, -1.0], [0.5, float("nan")]]) == ok
        again = run([[0, -1], [0, -1]])  # a failure leaves the context usable
        assert again == ok
    finally:
        torch.cuda.synchronize()
        layer.close()
        e0.free()
