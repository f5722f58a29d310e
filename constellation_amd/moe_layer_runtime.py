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
