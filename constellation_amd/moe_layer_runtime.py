"""Server-side router on the MI355X: the drop-in for `route_token_real`
(server/moe_layer_runtime.py:232-408).

`route_token_real` keeps the reference's signature, argument checks, error
types and messages, and its return value (a list of (expert_id, weight)
pairs, `effective_top_k = min(top_k, #resident)` long).  The computation is
the gfx950 router of libcx_moe.so (cx_route): W_r·x accumulated exactly in
fp64, sigmoid, correction bias, resident mask, per-group sum of the top-2,
top `topk_group` groups, top `top_k` experts inside them, weights
normalised (+1e-20) and scaled.  Ties go to the lower index.  PyTorch only
supplies the device tensors and the stream; there is no CPU path — a
non-HIP device raises.

Differences from the reference, by design:
  * `hidden` may also be fp16/bf16 and `gate_weight` bf16 (the checkpoint's
    own dtype): the products are exact in fp64 either way, so the decision
    is the same as for their fp32 casts.  fp32 inputs, as the reference
    requires, are accepted unchanged; fp16 `hidden` is widened to fp32
    (exactly) before the router, which reads bf16 or fp32.
  * the returned order is descending score (the reference's
    `topk(sorted=False)` order is unspecified).
  * `return_aux=True` returns the reference's aux keys
    (moe_layer_runtime.py:386-407).  They are derived on the host from the
    router kernel's own fp64 logits (cx_route_logits) in float64 and
    returned as float32 / int64 / bool numpy arrays like the reference's,
    so `selected_group_idx`, `group_mask`, `score_mask` and
    `topk_choice_vals` describe the decision the kernel made; `topk_idx`
    and `topk_weight` are the kernel's outputs themselves.

`route_tokens` is the batched form ([T, hidden] in, device tensors out) for
prefill chunks and batched decode.
"""
from __future__ import annotations

import threading

import torch

from . import engine

_CTX_LOCK = threading.Lock()
_CTX: dict[tuple[int, int], engine.Context] = {}

_ROUTER_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _context(device: int) -> engine.Context:
    """One cx_ctx per (thread, device): a context is not shared across threads."""
    key = (threading.get_ident(), device)
    with _CTX_LOCK:
        ctx = _CTX.get(key)
        if ctx is None:
            ctx = engine.Context(device)
            _CTX[key] = ctx
        return ctx


def _hip_device(t: torch.Tensor) -> int:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"route_token_real: the router runs on a HIP device (libcx_moe.so); got device={t.device}")
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def _check_common(hidden, gate_weight, e_score_correction_bias, *, n_group, topk_group, top_k,
                  scoring_func, topk_method, n_routed_experts, hidden_size, token_ndim):
    """Argument checks in the reference's order (moe_layer_runtime.py:250-319)."""
    if scoring_func != "sigmoid":
        raise RuntimeError(f"unsupported scoring_func={scoring_func}")
    if topk_method != "noaux_tc":
        raise RuntimeError(f"unsupported topk_method={topk_method}")
    if not isinstance(hidden, torch.Tensor):
        raise TypeError(f"hidden must be torch.Tensor, got {type(hidden).__name__}")
    if not isinstance(gate_weight, torch.Tensor):
        raise TypeError(f"gate_weight must be torch.Tensor, got {type(gate_weight).__name__}")
    if not isinstance(e_score_correction_bias, torch.Tensor):
        raise TypeError(
            "e_score_correction_bias must be torch.Tensor, got "
            f"{type(e_score_correction_bias).__name__}")
    if hidden.ndim != token_ndim:
        raise RuntimeError(f"hidden must be {token_ndim}D, got shape={tuple(hidden.shape)}")
    if gate_weight.ndim != 2:
        raise RuntimeError(f"gate_weight must be 2D, got shape={tuple(gate_weight.shape)}")
    if e_score_correction_bias.ndim != 1:
        raise RuntimeError(
            f"e_score_correction_bias must be 1D, got shape={tuple(e_score_correction_bias.shape)}")
    dev = str(gate_weight.device)
    if str(hidden.device) != dev:
        raise RuntimeError(
            f"hidden device mismatch: hidden={hidden.device} gate_weight={gate_weight.device}")
    if str(e_score_correction_bias.device) != dev:
        raise RuntimeError(
            f"bias device mismatch: bias={e_score_correction_bias.device} "
            f"gate_weight={gate_weight.device}")
    if gate_weight.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"gate_weight must be float32, got {gate_weight.dtype}")
    if e_score_correction_bias.dtype != torch.float32:
        raise TypeError(
            f"e_score_correction_bias must be float32, got {e_score_correction_bias.dtype}")
    if hidden.dtype not in _ROUTER_DTYPES:
        raise TypeError(
            f"hidden must be float32 for router scoring, got {hidden.dtype}. "
            f"Cast it explicitly in the caller.")
    num_experts, gate_hidden = gate_weight.shape
    if topk_group <= 0 or topk_group > n_group:
        raise RuntimeError(f"invalid topk_group={topk_group} for n_group={n_group}")
    if top_k <= 0 or top_k > num_experts:
        raise RuntimeError(f"invalid top_k={top_k} for num_experts={num_experts}")
    if num_experts != n_routed_experts:
        raise RuntimeError(
            f"gate_weight shape {tuple(gate_weight.shape)} inconsistent with "
            f"n_routed_experts={n_routed_experts}")
    if gate_hidden != hidden_size:
        raise RuntimeError(
            f"gate_weight shape {tuple(gate_weight.shape)} inconsistent with "
            f"hidden_size={hidden_size}")
    if int(hidden.shape[-1]) != hidden_size:
        raise RuntimeError(
            f"hidden dim {int(hidden.shape[-1])} inconsistent with hidden_size={hidden_size}")
    if int(e_score_correction_bias.shape[0]) != num_experts:
        raise RuntimeError(
            f"bias shape {tuple(e_score_correction_bias.shape)} incompatible with "
            f"num_experts={num_experts}")
    if num_experts % n_group != 0:
        raise RuntimeError(f"num_experts={num_experts} not divisible by n_group={n_group}")
    return num_experts


def _resident_mask(resident_expert_ids, num_experts: int, device) -> torch.Tensor | None:
    """uint8 [E] mask (moe_layer_runtime.py:327-341); ids outside [0, E) are ignored."""
    if resident_expert_ids is None:
        return None
    keep = sorted({int(e) for e in resident_expert_ids if 0 <= int(e) < num_experts})
    if not keep:
        raise RuntimeError("resident_expert_ids produced an empty resident mask")
    mask = torch.zeros(num_experts, dtype=torch.uint8)
    mask[keep] = 1
    return mask.to(device)


def route_tokens(hidden, gate_weight, e_score_correction_bias, *, n_group: int, topk_group: int,
                 top_k: int, norm_topk_prob: bool, routed_scaling_factor: float,
                 scoring_func: str = "sigmoid", topk_method: str = "noaux_tc",
                 n_routed_experts: int | None = None, hidden_size: int | None = None,
                 resident_expert_ids=None):
    """Batched router: hidden [T, H] -> (topk_ids int32 [T, top_k], topk_w fp32 [T, top_k])
    on the device; entries past min(top_k, #resident) are id -1, weight 0."""
    E = gate_weight.shape[0] if isinstance(gate_weight, torch.Tensor) and gate_weight.ndim == 2 else 0
    num_experts = _check_common(
        hidden, gate_weight, e_score_correction_bias, n_group=n_group, topk_group=topk_group,
        top_k=top_k, scoring_func=scoring_func, topk_method=topk_method,
        n_routed_experts=E if n_routed_experts is None else n_routed_experts,
        hidden_size=int(hidden.shape[-1]) if hidden_size is None else hidden_size, token_ndim=2)
    dev = _hip_device(gate_weight)
    mask = _resident_mask(resident_expert_ids, num_experts, gate_weight.device)
    ctx = _context(dev)
    with torch.cuda.device(dev):
        ids, w = ctx.route(_router_input(hidden), gate_weight, e_score_correction_bias, resident=mask,
                           n_group=n_group, topk_group=topk_group, top_k=top_k,
                           norm_topk_prob=bool(norm_topk_prob),
                           routed_scaling_factor=float(routed_scaling_factor))
    return ids, w


def route_token_real(hidden, gate_weight: torch.Tensor, e_score_correction_bias: torch.Tensor, *,
                     n_group: int, topk_group: int, top_k: int, norm_topk_prob: bool,
                     routed_scaling_factor: float, scoring_func: str, topk_method: str,
                     n_routed_experts: int, hidden_size: int, resident_expert_ids=None,
                     return_aux: bool = False):
    """One token: returns [(expert_id, weight)] (and an aux dict when asked),
    as server/moe_layer_runtime.py:232-408 does."""
    num_experts = _check_common(
        hidden, gate_weight, e_score_correction_bias, n_group=n_group, topk_group=topk_group,
        top_k=top_k, scoring_func=scoring_func, topk_method=topk_method,
        n_routed_experts=n_routed_experts, hidden_size=hidden_size, token_ndim=1)
    dev = _hip_device(gate_weight)
    mask = _resident_mask(resident_expert_ids, num_experts, gate_weight.device)
    ctx = _context(dev)
    with torch.cuda.device(dev):
        ids, w = ctx.route(_router_input(hidden).view(1, -1), gate_weight, e_score_correction_bias,
                           resident=mask, n_group=n_group, topk_group=topk_group, top_k=top_k,
                           norm_topk_prob=bool(norm_topk_prob),
                           routed_scaling_factor=float(routed_scaling_factor))
        logits = ctx.route_logits(1, num_experts, gate_weight.device) if return_aux else None
        ctx.sync()
    ids_l = ids[0].tolist()
    w_l = w[0].tolist()
    routes = [(int(e), float(x)) for e, x in zip(ids_l, w_l) if e >= 0]
    if not return_aux:
        return routes
    aux = _route_aux(logits[0].cpu().numpy(), e_score_correction_bias.detach().cpu().numpy(),
                     None if mask is None else mask.cpu().numpy().astype(bool),
                     n_group=n_group, topk_group=topk_group, norm_topk_prob=bool(norm_topk_prob),
                     routes=routes)
    return routes, aux


def _router_input(hidden: torch.Tensor) -> torch.Tensor:
    """The router kernel reads bf16 or fp32 activations; fp16 widens exactly."""
    return hidden.float() if hidden.dtype == torch.float16 else hidden


def _route_aux(logits64, bias, resident, *, n_group: int, topk_group: int,
               norm_topk_prob: bool, routes):
    """The reference's aux dict (server/moe_layer_runtime.py:321-407), from
    the kernel's fp64 logits of one token, in the reference's step order,
    evaluated in float64 on the host (diagnostics only: the routes come from
    the kernel).  Ranking ties go to the lower index, as in the kernel."""
    import numpy as np

    E = logits64.shape[0]
    epg = E // n_group
    lg = np.asarray(logits64, np.float64)
    s_raw = 1.0 / (1.0 + np.exp(-lg))
    c_raw = s_raw + np.asarray(bias, np.float64)
    res = np.ones(E, bool) if resident is None else np.asarray(resident, bool)
    c = np.where(res, c_raw, -np.inf)
    s = np.where(res, s_raw, 0.0)
    grouped = c.reshape(n_group, epg)
    top2 = -np.sort(-grouped, axis=1, kind="stable")[:, :2]
    group_scores = top2.sum(axis=1)
    order = np.lexsort((np.arange(n_group), -group_scores))  # descending, lower index first
    sel = np.sort(order[:topk_group]).astype(np.int64)
    group_mask = np.zeros(n_group, bool)
    group_mask[sel] = True
    score_mask = np.repeat(group_mask, epg)
    idx = np.asarray([e for e, _ in routes], np.int64)
    k = int(idx.size)
    pre = s[idx]
    post = pre / (pre.sum() + 1e-20) if (norm_topk_prob and k > 1) else pre.copy()
    f32 = np.float32
    return {
        "logits": lg.astype(f32),
        "scores_raw": s_raw.astype(f32),
        "scores": s.astype(f32),
        "scores_for_choice_raw": c_raw.astype(f32),
        "scores_for_choice": c.astype(f32),
        "group_scores": group_scores.astype(f32),
        "selected_group_idx": sel,
        "group_mask": group_mask,
        "score_mask": score_mask,
        "resident_mask": res,
        "topk_idx": idx,
        "topk_choice_vals": c[idx].astype(f32),
        "topk_weight_pre_norm": pre.astype(f32),
        "topk_weight_post_norm": post.astype(f32),
        "topk_weight": np.asarray([x for _, x in routes], f32),
        "effective_top_k": k,
        "routes": routes,
    }


# ---------------------------------------------------------------------------
# Session-level drop-ins for the reference's expert dispatch
# (server/moe_layer_runtime.py:84-98, 170-229, 411-578).
#
# The session is the reference's InferenceSession (server/inference_session.py:
# 22-60): `coord.placements` (dicts with "expert_id" (global), "host",
# "worker_port"), `client_pool.get(host, port)` / `.invalidate(host, port)`
# returning a connected NodeClient (server/client.py: send_message /
# recv_message), `cfg["run"]["experts_per_layer"]`, and for run_moe_layer
# `backbone_store` and `get_router_config()`.  One optional attribute is
# read: `cx_local_nodes`, a dict (host, worker_port) -> moe_dispatch.LocalNode
# for the placement endpoints whose experts live on this process's GPU; their
# routes run on the device with no host copy.  Every other endpoint gets one
# MoeLayerRequest (msg 42) per layer through the session's client pool,
# instead of one InferRequest per expert.

def validate_routes(routes):
    """validate_routes (server/moe_layer_runtime.py:84-98): the same checks
    and messages over a list of (expert_id, weight)."""
    if not routes:
        raise RuntimeError("routes is empty")
    seen = set()
    for expert_id, weight in routes:
        expert_id = int(expert_id)
        weight = float(weight)
        if expert_id in seen:
            raise RuntimeError(f"duplicate expert_id in routes: {expert_id}")
        seen.add(expert_id)
        if weight < 0:
            raise RuntimeError(f"negative route weight for expert {expert_id}: {weight}")


def _experts_per_layer(session) -> int:
    cfg = getattr(session, "cfg", None) or {}
    run = cfg.get("run") or {}
    return int(run.get("experts_per_layer", 256))


def _placement(placements, expert_id: int):
    """find_expert_placement (server/expert_placement.py:53-58)."""
    for p in placements:
        if int(p["expert_id"]) == expert_id:
            return p
    raise RuntimeError(f"expert {expert_id} not found in placements")


def _wire_dtype(dtype: torch.dtype) -> torch.dtype:
    """16-bit activation dtype of a request: hidden's own when it is 16-bit,
    else fp16, the dtype the reference's wire carries (moe_layer_runtime.py:
    36, 41-48)."""
    return dtype if dtype in (torch.float16, torch.bfloat16) else torch.float16


def _remote_layer_call(session, host: str, port: int, layer_id: int, x16: torch.Tensor,
                       local_ids, weights, out16: torch.dtype) -> torch.Tensor:
    """One MoeLayerRequest through the session's NodeClient for (host, port);
    returns the node's weighted partial [1, H] (out16) on the host.  On a
    transport error the connection is invalidated and the error re-raised,
    as infer_one_expert does (moe_layer_runtime.py:37-53)."""
    import numpy as np

    from . import moe_layer_protocol as P
    from .moe_dispatch import _RID

    H = int(x16.shape[-1])
    K = len(local_ids)
    body = P.encode_moe_layer_request({
        "layer_id": layer_id, "batch_size": 1, "hidden_dim": H, "top_k": K,
        "input_dtype": engine.cx_dtype(x16.dtype), "output_dtype": engine.cx_dtype(out16),
        "flags": 0, "expert_ids": np.asarray([local_ids], np.int32),
        "expert_weights": np.asarray([weights], np.float32),
        "activation": x16.contiguous().cpu().view(torch.int16).numpy().tobytes()})
    pool = session.client_pool
    rid = next(_RID) & 0xFFFFFFFF
    try:
        client = pool.get(host, port)
        client.send_message(P.MOE_LAYER_REQUEST, rid, body)
        msg = client.recv_message()
    except Exception:
        pool.invalidate(host, port)
        raise
    hdr = msg["header"]
    if int(hdr["msg_type"]) != P.MOE_LAYER_RESPONSE or int(hdr["request_id"]) != rid:
        raise P.ProtocolError(
            f"unexpected reply type={int(hdr['msg_type'])} rid={int(hdr['request_id'])}")
    resp = P.decode_moe_layer_response(msg["body"])
    if resp["status_code"] != 0:
        raise RuntimeError(
            f"moe layer {layer_id} failed on node {host}:{port}: status={resp['status_code']}")
    if resp["batch_size"] != 1 or resp["hidden_dim"] != H or len(resp["output"]) != H * 2:
        raise RuntimeError(
            f"unexpected moe layer output size from node {host}:{port}: "
            f"got={len(resp['output'])} bytes expected={H * 2}")
    return torch.frombuffer(bytearray(resp["output"]), dtype=torch.int16).view(out16).view(1, H)


def run_topk_moe_layer(session, hidden, routes, *, return_aux: bool = False,
                       accum_dtype: torch.dtype = torch.float32):
    """Drop-in for run_topk_moe_layer (server/moe_layer_runtime.py:170-229):
    same signature, checks and return shape.

    hidden: 1-D tensor (the reference passes the fp32 router input);
    routes: [(global_expert_id, weight)] as run_moe_layer builds them.
    Returns (combined, weighted_outputs), or (combined, weighted_outputs,
    expert_outputs) with return_aux.  combined = sum_k w_k y_k accumulated in
    `accum_dtype` and cast to hidden's dtype, on hidden's device (the
    reference's is on the CPU).

    Routes are grouped by the placement endpoint that serves them and by
    layer.  Without return_aux each group is ONE request carrying all its
    routes and weights (MoeLayerRequest to a remote node, the device path for
    a `cx_local_nodes` endpoint): the node returns its weighted partial sum,
    so `weighted_outputs` holds one entry per node request,
    (-1, 1.0, partial) with partial an fp32 tensor on hidden's device —
    outputs are per node, not per expert.  With return_aux, every route is
    its own request of weight 1.0 (as the reference's diagnostics need each
    expert's output): `weighted_outputs` is [(expert_id, weight, y)] and
    `expert_outputs` the reference's per-expert dicts, with y the expert's
    16-bit output widened to fp32 numpy, as infer_one_expert returns it."""
    import numpy as np

    from .moe_dispatch import LocalNode

    if not isinstance(hidden, torch.Tensor):
        raise TypeError(f"hidden must be torch.Tensor, got {type(hidden).__name__}")
    if hidden.ndim != 1:
        raise RuntimeError(f"hidden must be 1D, got shape={tuple(hidden.shape)}")
    validate_routes(routes)
    routes = [(int(e), float(w)) for e, w in routes]
    hidden = hidden.detach()
    out_dtype = hidden.dtype
    x16 = hidden.to(_wire_dtype(hidden.dtype)).contiguous().view(1, -1)
    epl = _experts_per_layer(session)
    local_nodes = getattr(session, "cx_local_nodes", None) or {}
    # group by (endpoint, layer) in first-appearance order
    groups: dict = {}
    for gid, w in routes:
        p = _placement(session.coord.placements, gid)
        key = (str(p["host"]), int(p["worker_port"]), gid // epl)
        groups.setdefault(key, []).append((gid, w))

    def run_group(host, port, layer_id, members, unit_weights):
        ids = [gid % epl for gid, _ in members]
        wts = [1.0 if unit_weights else w for _, w in members]
        node = local_nodes.get((host, port))
        if node is not None:
            if not isinstance(node, LocalNode) or layer_id not in node.layers:
                raise RuntimeError(f"no local layer {layer_id} for endpoint {host}:{port}")
            dev = _hip_device(x16)
            ctx = _context(dev)
            with torch.cuda.device(dev):
                ids_d = torch.tensor([ids], dtype=torch.int32, device=x16.device)
                w_d = torch.tensor([wts], dtype=torch.float32, device=x16.device)
                y16, yf = ctx.moe(node.layers[layer_id], x16, ids_d, w_d,
                                  out_dtype=x16.dtype, want_f32=True)
            return y16, yf
        y16 = _remote_layer_call(session, host, port, layer_id, x16, ids, wts, x16.dtype)
        return y16, None

    if not return_aux:
        weighted_outputs = []
        combined = None
        for (host, port, layer_id), members in groups.items():
            y16, yf = run_group(host, port, layer_id, members, unit_weights=False)
            part = (yf if yf is not None else y16.float()).view(-1).to(hidden.device)
            weighted_outputs.append((-1, 1.0, part))
            combined = part.to(accum_dtype).clone() if combined is None else combined + part.to(accum_dtype)
        return combined.to(out_dtype), weighted_outputs

    weighted_outputs, expert_outputs = [], []
    combined = None
    for (host, port, layer_id), members in groups.items():
        for gid, w in members:
            y16, _ = run_group(host, port, layer_id, [(gid, w)], unit_weights=True)
            y = y16.view(-1).float().cpu().numpy()
            weighted_outputs.append((gid, w, y))
            expert_outputs.append({
                "expert_id": gid,
                "weight": w,
                "output": y.copy(),
                "weighted_output": (w * y).astype(np.float32, copy=False),
                "output_dtype": engine.cx_dtype(x16.dtype),
            })
    # combine_outputs_torch (moe_layer_runtime.py:148-167): in route order
    order = {gid: i for i, (gid, _) in enumerate(routes)}
    for gid, w, y in sorted(weighted_outputs, key=lambda r: order[r[0]]):
        term = torch.as_tensor(w, dtype=accum_dtype) * torch.as_tensor(y, dtype=accum_dtype)
        combined = term if combined is None else combined + term
    weighted_outputs.sort(key=lambda r: order[r[0]])
    expert_outputs.sort(key=lambda r: order[r["expert_id"]])
    return combined.to(out_dtype).to(hidden.device), weighted_outputs, expert_outputs


def _as_vector(x, name: str, dtype: torch.dtype, device: str) -> torch.Tensor:
    """as_array(x, name, ARRCFG_VECTOR_TORCH(dtype, device))
    (server/array_utils.py:61-73, 154-213): a 1-D, finite, contiguous torch
    tensor of exactly `dtype` on `device`; no cast or move."""
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} expected torch backend, got type={type(x).__name__}")
    if x.ndim != 1:
        raise ValueError(f"{name} must have ndim in [1], got shape {tuple(int(v) for v in x.shape)}")
    if x.shape[-1] == 0:
        raise ValueError(
            f"{name} must not have empty hidden dimension, got shape {tuple(int(v) for v in x.shape)}")
    if x.dtype != dtype:
        raise TypeError(f"{name} expected dtype={dtype}, got dtype={x.dtype}")
    if str(x.device) != str(device):
        raise RuntimeError(f"{name} expected device={device}, got device={x.device}")
    if not torch.all(torch.isfinite(x)).item():
        raise ValueError(f"{name} contains non-finite values")
    return x.contiguous()


def run_moe_layer(session, hidden, layer_id: int, *, return_aux: bool = False):
    """Drop-in for run_moe_layer (server/moe_layer_runtime.py:411-578): the
    same checks, resident-expert selection, router call, global ids and
    result dict ({"output": ...} plus "aux" with return_aux), with the HIP
    router (route_token_real above) and run_topk_moe_layer above (one
    request per node instead of one per expert).  gate_weight may be fp32,
    as the reference requires, or the checkpoint's bf16."""
    layer_id = int(layer_id)
    if session.backbone_store is None:
        raise RuntimeError("session.backbone_store is not initialized")
    layer_entry = session.backbone_store.layer(layer_id)
    dev = str(layer_entry["device"])
    runtime_dtype = session.backbone_store.dtype
    hidden = _as_vector(hidden, f"moe.layer{layer_id}.hidden", runtime_dtype, dev)
    router_cfg = session.get_router_config()
    hidden_size = int(router_cfg["hidden_size"])
    if int(hidden.shape[0]) != hidden_size:
        raise RuntimeError(
            f"hidden size mismatch: got={int(hidden.shape[0])} expected={hidden_size}")
    if "router" not in layer_entry:
        raise RuntimeError(f"router weights are not loaded for layer {layer_id}")
    router_entry = layer_entry["router"]
    gate_weight = router_entry["gate_weight"]
    e_score_correction_bias = router_entry["e_score_correction_bias"]
    if not isinstance(gate_weight, torch.Tensor):
        raise TypeError(f"gate_weight must be torch.Tensor, got {type(gate_weight).__name__}")
    if not isinstance(e_score_correction_bias, torch.Tensor):
        raise TypeError(
            "e_score_correction_bias must be torch.Tensor, got "
            f"{type(e_score_correction_bias).__name__}")
    if str(gate_weight.device) != dev:
        raise RuntimeError(
            f"router gate_weight expected device={dev}, got device={gate_weight.device}")
    if str(e_score_correction_bias.device) != dev:
        raise RuntimeError(
            f"router bias expected device={dev}, got device={e_score_correction_bias.device}")
    if gate_weight.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"router gate_weight must be float32, got {gate_weight.dtype}")
    if e_score_correction_bias.dtype != torch.float32:
        raise TypeError(
            f"router e_score_correction_bias must be float32, got {e_score_correction_bias.dtype}")
    router_hidden = hidden.to(dtype=torch.float32)
    experts_per_layer = int(session.cfg["run"]["experts_per_layer"])
    restricted = session.cfg["run"].get("restricted_expert_ids")
    if restricted is not None:
        resident = sorted({int(e) for e in restricted})
        max_local = int(router_cfg["n_routed_experts"])
        for eid in resident:
            if eid < 0 or eid >= max_local:
                raise RuntimeError(
                    f"restricted expert id out of range for layer {layer_id}: "
                    f"{eid} not in [0, {max_local})")
    else:
        # allowed_local_expert_ids_for_layer (server/expert_placement.py:27-43)
        resident = sorted({int(p["expert_id"]) % experts_per_layer
                           for p in session.coord.placements
                           if int(p["expert_id"]) // experts_per_layer == layer_id})
    if not resident:
        raise RuntimeError(f"no resident experts found for layer {layer_id}")
    kw = dict(n_group=int(router_cfg["n_group"]), topk_group=int(router_cfg["topk_group"]),
              top_k=min(int(router_cfg["top_k"]), len(resident)),
              norm_topk_prob=bool(router_cfg["norm_topk_prob"]),
              routed_scaling_factor=float(router_cfg["routed_scaling_factor"]),
              scoring_func=str(router_cfg["scoring_func"]),
              topk_method=str(router_cfg["topk_method"]),
              n_routed_experts=int(router_cfg["n_routed_experts"]),
              hidden_size=int(router_cfg["hidden_size"]), resident_expert_ids=resident)
    if return_aux:
        routes, aux = route_token_real(router_hidden, gate_weight, e_score_correction_bias,
                                       return_aux=True, **kw)
    else:
        routes = route_token_real(router_hidden, gate_weight, e_score_correction_bias, **kw)
        aux = None
    # make_global_expert_id (server/expert_placement.py:4-25)
    global_routes = [(layer_id * experts_per_layer + int(e), w) for e, w in routes]
    if return_aux:
        combined, weighted_outputs, expert_outputs = run_topk_moe_layer(
            session, router_hidden, global_routes, return_aux=True)
    else:
        combined, weighted_outputs = run_topk_moe_layer(
            session, router_hidden, global_routes, return_aux=False)
        expert_outputs = None
    combined_t = torch.as_tensor(combined, dtype=runtime_dtype, device=dev)
    combined_t = _as_vector(combined_t, f"moe.layer{layer_id}.output", runtime_dtype, dev)
    if not return_aux:
        return {"output": combined_t}
    return {
        "output": combined_t,
        "aux": {
            "layer_id": layer_id,
            "router_hidden": router_hidden.detach().float().cpu().numpy(),
            **aux,
            "resident_local_expert_ids": resident,
            "routes": global_routes,
            "local_routes": routes,
            "selected_global_expert_ids": [int(e) for e, _ in global_routes],
            "selected_weights": [float(w) for _, w in global_routes],
            "weighted_outputs": weighted_outputs,
            "combined_pre_cast": torch.as_tensor(combined).detach().float().cpu().numpy(),
            "expert_outputs": expert_outputs,
        },
    }
