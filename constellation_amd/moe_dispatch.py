"""Server side of a MoE layer on the HIP engine, batched over tokens.

Takes the role of the reference's expert dispatch and the loops around it:
  * run_topk_moe_layer / dispatch_topk_experts / combine_outputs_torch
    (server/moe_layer_runtime.py:111-229): one InferRequest per selected
    expert, sent one after another, after a device -> CPU -> numpy copy of
    the hidden state (:186-200), combined on the CPU;
  * the per-token loop of run_sparse_layer (server/full_model_runtime.py:
    317-331), which calls run_moe_layer once per token of a prefill chunk;
  * the shared expert, run apart on the attention GPU
    (deepseek_full_model_executor.py:264-316, full_model_runtime.py:348).

Here a layer call takes the whole token batch as device tensors and visits
each node once:
  * LocalNode — experts resident on this process's GPU (engine.Layer per
    layer id): cx_moe_decode / cx_moe_prefill on the device tensors, with no
    host copy.  When one local node holds every expert of the layer,
    run_moe_layer_batched routes and computes in one cx_moe_layer call.
  * RemoteNode — an expert node reached through a caller-supplied transport
    (a function from one framed request to one framed reply, or a socket to
    a worker port): one MoeLayerRequest (msg 42, v1 framing
    common/protocol.h:10-62) per layer, answered with the node's partial sum.
The shared expert is folded into the first node that holds it (FLAG_SHARED).
Partials of several nodes are added in fp32 in node order, then rounded to
the output dtype: a local node's partial enters the sum in fp32 (one
rounding in all), a remote node's arrives already rounded to 16 bits by its
node (the wire carries 16-bit activations), so a layer split across a
remote node is rounded twice.  A single node's answer is returned as it is.

Routes are checked as validate_routes does (server/moe_layer_runtime.py:
84-98): an expert listed twice for one token and a negative (or
non-finite) weight are errors.
  * validate=True (default): the planner checks every route on the device
    and skips a bad one; the error is raised (CxError, a RuntimeError) by
    the context's next synchronisation — check_routes(device) or
    engine.Context.sync() — so the call itself copies and waits for nothing.
    When the layer is split across nodes the routes are on the host anyway
    (each node's request is built there) and are checked there at once.
  * validate="host": the routes are copied to the host and checked before
    any compute, raising RuntimeError with the reference's messages ("routes
    is empty" included).
  * validate=False: no host-side check (the device still skips bad routes).
"""
from __future__ import annotations

import itertools
import socket
from typing import Callable, Optional, Sequence, Union

import numpy as np
import torch

from . import engine
from . import moe_layer_protocol as P
from .moe_layer_runtime import _context, _hip_device, route_tokens

_RID = itertools.count(1)


class LocalNode:
    """Experts resident on this process's GPU.

    layers: layer id -> engine.Layer whose entry i is the layer's local
    expert i (None where not resident here) and whose shared expert, when
    present, is the layer's shared expert."""

    def __init__(self, layers: dict[int, engine.Layer], device: int = 0):
        self.layers = dict(layers)
        self.device = device

    def resident(self, layer_id: int, n_experts: int) -> np.ndarray:
        lay = self.layers.get(layer_id)
        out = np.zeros(n_experts, bool)
        if lay is not None:
            for i, e in enumerate(lay.experts[:n_experts]):
                out[i] = e is not None
        return out

    def has_shared(self, layer_id: int) -> bool:
        lay = self.layers.get(layer_id)
        return lay is not None and lay.shared is not None


Transport = Callable[[bytes], bytes]


class RemoteNode:
    """An expert node reached through `transport`, which sends one framed
    request (header + body bytes) and returns the framed reply.

    resident: layer id -> local expert ids this node serves for that layer;
    shared_layers: layer ids whose shared expert it holds."""

    def __init__(self, transport: Transport, resident: dict[int, Sequence[int]],
                 shared_layers: Sequence[int] = ()):
        self.transport = transport
        self._resident = {int(k): sorted({int(e) for e in v}) for k, v in resident.items()}
        self._shared = {int(l) for l in shared_layers}

    @classmethod
    def over_socket(cls, sock: socket.socket, resident, shared_layers=()) -> "RemoteNode":
        """A node behind a connected worker socket (one request at a time)."""
        def transport(frame: bytes) -> bytes:
            sock.sendall(frame)
            hdr, body = P.recv_frame(sock)
            return P.encode_header(hdr["msg_type"], hdr["request_id"], hdr["body_len"]) + body
        return cls(transport, resident, shared_layers)

    def resident(self, layer_id: int, n_experts: int) -> np.ndarray:
        out = np.zeros(n_experts, bool)
        for e in self._resident.get(layer_id, ()):
            if 0 <= e < n_experts:
                out[e] = True
        return out

    def has_shared(self, layer_id: int) -> bool:
        return layer_id in self._shared

    def call(self, layer_id: int, x: torch.Tensor, ids: np.ndarray, w: np.ndarray, shared: bool,
             out_dtype: torch.dtype) -> torch.Tensor:
        """One MoeLayerRequest; returns the node's partial sum [T, H] on x's device."""
        T, H = x.shape
        K = ids.shape[1]
        dt = engine.cx_dtype(x.dtype)
        body = P.encode_moe_layer_request({
            "layer_id": layer_id, "batch_size": T, "hidden_dim": H, "top_k": K,
            "input_dtype": dt, "output_dtype": engine.cx_dtype(out_dtype),
            "flags": P.FLAG_SHARED if shared else 0, "expert_ids": ids, "expert_weights": w,
            "activation": x.contiguous().cpu().view(torch.int16).numpy().tobytes()})
        rid = next(_RID) & 0xFFFFFFFF
        reply = self.transport(P.frame(P.MOE_LAYER_REQUEST, rid, body))
        hdr = P.decode_header(reply[:P.HEADER_BYTES])
        if hdr["msg_type"] != P.MOE_LAYER_RESPONSE or hdr["request_id"] != rid or \
                hdr["body_len"] != len(reply) - P.HEADER_BYTES:
            raise P.ProtocolError(f"unexpected reply type={hdr['msg_type']} rid={hdr['request_id']}")
        resp = P.decode_moe_layer_response(reply[P.HEADER_BYTES:])
        if resp["status_code"] != 0:
            raise RuntimeError(f"moe layer {layer_id} failed on a remote node: "
                               f"status={resp['status_code']}")
        if resp["batch_size"] != T or resp["hidden_dim"] != H or len(resp["output"]) != T * H * 2:
            raise RuntimeError(f"unexpected moe layer response size for layer {layer_id}")
        out = torch.frombuffer(bytearray(resp["output"]), dtype=torch.int16).view(out_dtype)
        return out.view(T, H).to(x.device)


Node = Union[LocalNode, RemoteNode]


def validate_routes(ids: np.ndarray, w: np.ndarray) -> None:
    """validate_routes (server/moe_layer_runtime.py:84-98) for every token of
    a [T, K] route table (-1 = no route in that slot)."""
    if ids.size == 0 or not (ids >= 0).any():
        raise RuntimeError("routes is empty")
    for t in range(ids.shape[0]):
        seen = set()
        for e, x in zip(ids[t].tolist(), w[t].tolist()):
            if e < 0:
                continue
            if e in seen:
                raise RuntimeError(f"duplicate expert_id in routes: {e}")
            seen.add(e)
            if x < 0:
                raise RuntimeError(f"negative route weight for expert {e}: {x}")
            if not np.isfinite(x):
                raise RuntimeError(f"non-finite route weight for expert {e}: {x}")


def _as_2d(hidden: torch.Tensor) -> tuple[torch.Tensor, bool]:
    if hidden.ndim == 1:
        return hidden.view(1, -1), True
    if hidden.ndim != 2:
        raise RuntimeError(f"hidden must be 1D or 2D, got shape={tuple(hidden.shape)}")
    return hidden, False


def check_routes(device: int = 0) -> None:
    """Raises (CxError) if a route of an earlier call on this thread's context
    of `device` failed the device-side checks (validate=True); waits for the
    context's work on the device's current stream."""
    _context(device).sync()


def run_topk_moe_layer(nodes: Sequence[Node], hidden: torch.Tensor, layer_id: int,
                       topk_ids, topk_w, *, n_experts: int = 256, shared: bool = True,
                       out_dtype: Optional[torch.dtype] = None,
                       validate: Union[bool, str] = True) -> torch.Tensor:
    """Routed (and shared) expert compute of one layer for a token batch.

    hidden: [T, H] (or [H]) fp16/bf16 on the HIP device.  topk_ids / topk_w:
    [T, K] local expert ids (-1 = none) and weights, as device tensors or
    host arrays.  Returns [T, H] (or [H]) in out_dtype (default hidden's) on
    hidden's device: y[t] = sum_k w[t,k] expert_k(x[t]) (+ shared(x[t])).
    Each route goes to the first node in `nodes` that holds its expert; a
    route no node holds raises.  `validate`: see the module docstring."""
    if validate not in (True, False, "host"):
        raise ValueError(f"validate must be True, False or 'host', got {validate!r}")
    x, was_1d = _as_2d(hidden)
    local = any(isinstance(n, LocalNode) for n in nodes)
    dev = _hip_device(x) if local else None
    out_dtype = out_dtype or x.dtype
    ids_d = torch.as_tensor(topk_ids, device=x.device).to(torch.int32).reshape(x.shape[0], -1)
    w_d = torch.as_tensor(topk_w, device=x.device).to(torch.float32).reshape(x.shape[0], -1)
    if (validate != "host" and len(nodes) == 1 and local and layer_id in nodes[0].layers
            and (nodes[0].layers[layer_id].shared is not None) == shared):
        # one local node: routes stay on the device; the planner skips and
        # flags a route to an expert that is not resident, a repeated expert
        # and a bad weight (raised by the context's next sync)
        ctx = _context(dev)
        with torch.cuda.device(dev):
            y = ctx.moe(nodes[0].layers[layer_id], x, ids_d, w_d, out_dtype=out_dtype)
        return y.view(-1) if was_1d else y
    ids_h = ids_d.cpu().numpy()
    if validate:
        validate_routes(ids_h, w_d.cpu().numpy())
    owner = np.full(ids_h.shape, -1, np.int64)
    for n_i, node in enumerate(nodes):
        res = node.resident(layer_id, n_experts)
        take = (owner < 0) & (ids_h >= 0) & (ids_h < n_experts)
        take[take] = res[ids_h[take]]
        owner[take] = n_i
    lost = (ids_h >= 0) & (owner < 0)
    if lost.any():
        t, k = np.argwhere(lost)[0]
        raise RuntimeError(f"no node holds expert {int(ids_h[t, k])} of layer {layer_id}")
    shared_node = next((i for i, n in enumerate(nodes) if n.has_shared(layer_id)), -1) if shared else -1
    if shared and shared_node < 0:
        raise RuntimeError(f"no node holds the shared expert of layer {layer_id}")
    partials = []
    for n_i, node in enumerate(nodes):
        mine = owner == n_i
        if not mine.any() and n_i != shared_node:
            continue
        sel = np.where(mine, ids_h, -1).astype(np.int32)
        if isinstance(node, LocalNode):
            lay = node.layers[layer_id]
            ctx = _context(dev)
            sel_d = torch.from_numpy(sel).to(x.device) if not mine.all() else ids_d
            if n_i != shared_node and lay.shared is not None:
                raise RuntimeError("a local layer with a shared expert must serve the shared expert "
                                   "(list its node first)")
            with torch.cuda.device(dev):
                # a partial that is summed with others stays fp32 until the end
                y, yf = ctx.moe(lay, x, sel_d, w_d, out_dtype=out_dtype, want_f32=True)
            partials.append((y, yf))
        else:
            y = node.call(layer_id, x, sel, w_d.cpu().numpy(), n_i == shared_node, out_dtype)
            partials.append((y, None))
    if len(partials) == 1:
        y = partials[0][0]
    else:
        acc = None
        for y16, y32 in partials:
            part = y32 if y32 is not None else y16.float()
            acc = part.clone() if acc is None else acc + part
        y = acc.to(out_dtype)
    return y.view(-1) if was_1d else y


def run_moe_layer_batched(nodes: Sequence[Node], hidden: torch.Tensor, layer_id: int,
                          gate_weight: torch.Tensor, e_score_correction_bias: torch.Tensor, *,
                          n_group: int, topk_group: int, top_k: int, norm_topk_prob: bool,
                          routed_scaling_factor: float, resident_expert_ids=None,
                          shared: bool = True, out_dtype: Optional[torch.dtype] = None):
    """A MoE layer for a whole token batch: router (route_tokens, the HIP
    router) then run_topk_moe_layer — the per-token loop of
    full_model_runtime.py:317-331 as one call.  Returns (y, topk_ids, topk_w)
    on the device.  When a single local node holds the layer and the router
    reads bf16 activations, the router and experts run as one cx_moe_layer
    call (decode pipeline for up to 16 tokens)."""
    x, was_1d = _as_2d(hidden)
    E = int(gate_weight.shape[0])
    one_local = (len(nodes) == 1 and isinstance(nodes[0], LocalNode)
                 and layer_id in nodes[0].layers and resident_expert_ids is None
                 and x.dtype == torch.bfloat16)
    if one_local:
        lay = nodes[0].layers[layer_id]
        if lay.n_experts == E and (not shared or lay.shared is not None):
            dev = _hip_device(x)
            ctx = _context(dev)
            with torch.cuda.device(dev):
                if not shared and lay.shared is not None:
                    raise RuntimeError("shared=False needs a layer without a shared expert")
                y, _, ids, w = ctx.moe_layer(lay, x, gate_weight, e_score_correction_bias,
                                             n_group=n_group, topk_group=topk_group, top_k=top_k,
                                             norm_topk_prob=bool(norm_topk_prob),
                                             routed_scaling_factor=float(routed_scaling_factor),
                                             out_dtype=out_dtype or x.dtype)
            return (y.view(-1) if was_1d else y), ids, w
    ids, w = route_tokens(x, gate_weight, e_score_correction_bias, n_group=n_group,
                          topk_group=topk_group, top_k=top_k, norm_topk_prob=norm_topk_prob,
                          routed_scaling_factor=routed_scaling_factor,
                          resident_expert_ids=resident_expert_ids)
    y = run_topk_moe_layer(nodes, x, layer_id, ids, w, n_experts=E, shared=shared,
                           out_dtype=out_dtype)
    return (y.view(-1) if was_1d else y), ids, w
