"""Drop-in check of the expert-node plugin on the GPU: the reference's own node
code (control loop, resident_bg upload thread, registry, worker loop, codecs;
oracle/_ref/node_harness) with constellation_amd/backend_amd/ in the AMD slot,
driven over TCP with the reference's wire formats, every result checked
against the CPU oracle.

Covers, in order (one node process for the module):
  * BuildLocalAmd{,Dynamic}GpuInfosV2 through InventoryReply;
  * UploadExpertAmdV2 of full-size seeded experts and of the reference's
    4x8 1x1-block control expert, through LoadWeights* and the resident_bg
    thread (control.cc:130-276 -> expert_registry_v2.cc Update);
  * v1 InferRequest -> HandleInferRequest -> BackendWorkspaceAmdV2::
    RunExpertRequest at fp16->fp16 B=1 (the server's wire,
    moe_layer_runtime.py:36-48) and bf16 B=4, the echo fields, and the
    status codes 1 / 2 / 4 of worker.cc:113-132;
  * MoeLayerRequest on the reference's worker loop with the integration's
    one branch (worker.cc streamed through oracle/integrate_worker.awk;
    HandleMoeLayerRequestAmdV2 -> RunMoeLayerRequest) bit-identical to
    cx_moe_layer_request_run in this process on the same experts, and within
    the parity bound of the oracle; both message types on one connection;
  * uploads on the control thread while a worker connection infers;
  * replacement of a resident expert and a placement that drops residents
    (FreeExpertWeightsAmdV2);
  * "quit": ExpertRegistryV2::Reset frees everything through the plugin, the
    DeviceBufferV2 destructors do not abort (expert_format_v2.h:141-157) and
    the arena ends empty.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

from node_client import (HARNESS, W_UP, ControlClient, Harness, WorkerClient)
from oracle.oracle import BF16, FP16, rel_l2

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not HARNESS.exists(), reason="oracle/_ref/node_harness not built")]

H, I = 7168, 2048
LAYER, EPL = 1, 256                 # layer id, experts per layer (server/config.json)
LOCAL = [3, 17, 40, 200]            # resident local expert ids of the layer
SHARED_ID = (1 << 30) + LAYER       # SharedExpertIdV2(LAYER)
AMD = 3                             # common::GpuVendor::AMD


def gid(local: int) -> int:
    return LAYER * EPL + local        # make_global_expert_id (server/expert_placement.py:4-25)


class Node:
    def __init__(self, tmp, oracle):
        self.o = oracle
        self.h = Harness(tmp / "node.log")
        self.log_path = tmp / "node.log"
        self.ctrl = ControlClient(self.h.ctrl)
        self.experts = {gid(l): oracle.gen_expert(500 + l, 0x40) for l in LOCAL}
        self.experts[SHARED_ID] = oracle.gen_expert(500 + EPL, 0x40)

    def worker(self) -> WorkerClient:
        # the reference's RunGpuWorkerLoopV2 with the integration's
        # MoeLayerRequest branch: InferRequest and MoeLayerRequest on one port
        return WorkerClient(self.h.wbase)

    def log(self) -> str:
        return self.log_path.read_text()


@pytest.fixture(scope="module")
def node(tmp_path_factory, oracle):
    n = Node(tmp_path_factory.mktemp("node"), oracle)
    yield n
    n.ctrl.close()
    n.h.kill()


def _act(x: np.ndarray, dt: int) -> bytes:
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32))
    return t.to(torch.float16 if dt == FP16 else torch.bfloat16).view(torch.int16).numpy().tobytes()


def _act_f32(b: bytes, dt: int) -> np.ndarray:
    t = torch.from_numpy(np.frombuffer(b, np.int16).copy())
    return t.view(torch.float16 if dt == FP16 else torch.bfloat16).float().numpy()


def _assert_wire_parity(got, ref, dt):
    """A 16-bit wire output against the fp32 oracle: rel-L2 within the bar,
    and each element within half an ulp of the 16-bit format (<= 2^-8 |ref|
    for bf16, 2^-11 |ref| for fp16) plus the fp32 pipeline's own error.  The
    max-abs bar applies to fp32 outputs: bf16 rounding alone exceeds 2e-2
    where |y| > 4."""
    rel = 2.0 ** -8 if dt == BF16 else 2.0 ** -11
    assert rel_l2(got, ref) < 1e-2, rel_l2(got, ref)
    err = np.abs(got - ref) - (rel * np.abs(ref) + 1e-3)
    assert err.max() <= 0, (float(err.max()), float(np.abs(got - ref).max()))


def test_inventory_reports_the_amd_worker(node):
    print("[node] inventory", flush=True)
    inv = node.ctrl.inventory()
    assert inv["node_id"] == "amd_node0" and len(inv["gpus"]) == 1
    g = inv["gpus"][0]
    assert g["worker_id"] == 0 and g["gpu_vendor"] == AMD and g["worker_port"] == node.h.wbase
    assert g["arch_name"].startswith("gfx950") and g["gpu_name"]
    assert g["capability_flags"] == 1 | 2 | 4                      # fp16 | bf16 | fp8
    assert 0 < g["free_mem_bytes"] <= g["total_mem_bytes"] and g["total_mem_bytes"] > 200e9
    assert g["gpu_status"] == 1                                      # Idle
    assert node.ctrl.heartbeat()


def test_upload_through_the_control_plane(node):
    print("[node] load 5 full-size experts", flush=True)
    ids = sorted(node.experts)
    ack = node.ctrl.placement([(e, 0) for e in ids])
    assert ack["status_code"] == 0 and ack["needs_load"] and ack["num_target_experts"] == len(ids)
    for e in ids:
        node.ctrl.load_expert(e, 0, node.experts[e])
    assert node.ctrl.wait_resident(0, ids) == ids
    ack = node.ctrl.placement([(e, 0) for e in ids])
    assert ack["all_ready"] and ack["num_ready_experts"] == len(ids)


@pytest.mark.parametrize("dt,T", [(FP16, 1), (BF16, 4)])
def test_infer_request_matches_oracle(node, dt, T):
    print(f"[node] InferRequest dt={dt} T={T}", flush=True)
    x = np.random.default_rng(T).standard_normal((T, H)).astype(np.float32)
    act = _act(x, dt)
    w = node.worker()
    try:
        for e in (gid(3), gid(200), SHARED_ID):
            r = w.infer(e, T, H, dt, dt, act)
            assert r["status_code"] == 0 and r["batch_size"] == T and r["hidden_dim"] == H
            assert r["output_dtype"] == dt and len(r["output"]) == T * H * 2
            _, ref = node.o.expert_ref(node.experts[e], _act_f32(act, dt).reshape(T, H))
            got = _act_f32(r["output"], dt).reshape(T, H)
            _assert_wire_parity(got, ref, dt)
    finally:
        w.close()


def test_infer_status_codes(node):
    """worker.cc:113-132: 1 unknown expert, 2 not resident on this worker,
    4 execution failure (bad dtype, hidden != 7168 as the CUDA workspace
    requires, activation size mismatch); failures echo batch, hidden and
    output dtype with an empty output."""
    print("[node] status codes", flush=True)
    act = _act(np.ones((1, H), np.float32), FP16)
    e_partial = gid(99)
    node.ctrl.load_expert(e_partial, 0, node.experts[gid(3)], kinds=[W_UP])  # incoming only
    w = node.worker()
    try:
        assert w.infer(12345, 1, H, FP16, FP16, act)["status_code"] == 1
        assert w.infer(e_partial, 1, H, FP16, FP16, act)["status_code"] == 2
        for args in ((gid(3), 1, H, 3, FP16, act),            # fp32 is not a wire dtype
                     (gid(3), 1, H, FP16, 7, act),
                     (gid(3), 2, H, FP16, FP16, act),         # 2 tokens, 1 token of bytes
                     (gid(3), 1, 8, FP16, FP16, act[:16])):   # hidden 8
            r = w.infer(*args)
            assert r["status_code"] == 4 and r["output"] == b"", args
            assert (r["batch_size"], r["hidden_dim"], r["output_dtype"]) == (args[1], args[2], args[4])
        assert w.infer(gid(3), 1, H, FP16, FP16, act)["status_code"] == 0  # the connection still serves
    finally:
        w.close()


@pytest.mark.parametrize("T,shared", [(1, True), (3, True), (20, False)])
def test_moe_layer_request_equals_in_process(node, gpu, T, shared):
    """The node's MoeLayerRequest answer is bit-identical to
    cx_moe_layer_request_run in this process on the same experts, and the
    combine is within the parity bound of the oracle's."""
    from constellation_amd import moe_layer_protocol as P
    from constellation_amd.engine import Expert, Layer
    print(f"[node] MoeLayerRequest T={T} shared={shared}", flush=True)
    rng = np.random.default_rng(40 + T)
    K = 4
    ids = np.stack([rng.choice(LOCAL, K, replace=False) for _ in range(T)]).astype(np.int32)
    ids[0, K - 1] = -1                       # a route another node serves
    wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    body = P.encode_moe_layer_request({
        "layer_id": LAYER, "batch_size": T, "hidden_dim": H, "top_k": K, "input_dtype": BF16,
        "output_dtype": BF16, "flags": P.FLAG_SHARED if shared else 0, "expert_ids": ids,
        "expert_weights": wts, "activation": _act(x, BF16)})
    w = node.worker()
    try:
        r = w.moe_layer(body)
    finally:
        w.close()
    assert r["status_code"] == 0 and r["batch_size"] == T and len(r["output"]) == T * H * 2
    local = {}
    try:
        for l in LOCAL + [EPL]:
            ex = node.experts[SHARED_ID if l == EPL else gid(l)]
            local[l] = Expert.upload(0, ex["w_up"], ex["s_up"], ex["w_gate"], ex["s_gate"],
                                     ex["w_down"], ex["s_down"])
        table = [local.get(i) for i in range(EPL)]
        layer = Layer(gpu, table, local[EPL])
        mine = P.decode_moe_layer_response(gpu.moe_layer_request(layer, body))
        layer.close()
    finally:
        torch.cuda.synchronize()
        for e in local.values():
            e.free()
    assert mine == r
    xs = _act_f32(_act(x, BF16), BF16).reshape(T, H)
    ref = np.zeros((T, H), np.float32)
    for t in range(T):
        for k in range(K):
            if ids[t, k] >= 0:
                ref[t] += wts[t, k] * node.o.expert_ref(node.experts[gid(int(ids[t, k]))], xs[t:t + 1])[1][0]
        if shared:
            ref[t] += node.o.expert_ref(node.experts[SHARED_ID], xs[t:t + 1])[1][0]
    _assert_wire_parity(_act_f32(r["output"], BF16).reshape(T, H), ref, BF16)


def test_moe_layer_request_status(node):
    from constellation_amd import moe_layer_protocol as P
    print("[node] MoeLayerRequest status", flush=True)
    act = _act(np.ones((1, H), np.float32), BF16)

    def req(ids, layer_id=LAYER, flags=0):
        return P.encode_moe_layer_request({
            "layer_id": layer_id, "batch_size": 1, "hidden_dim": H, "top_k": len(ids),
            "input_dtype": BF16, "output_dtype": BF16, "flags": flags,
            "expert_ids": np.asarray(ids, np.int32), "expert_weights": np.full(len(ids), 0.5, np.float32),
            "activation": act})
    w = node.worker()
    try:
        assert w.moe_layer(req([3, 300]))["status_code"] == 1       # local id beyond the layer
        assert w.moe_layer(req([3, 5]))["status_code"] == 2         # not resident here
        assert w.moe_layer(req([3], layer_id=7))["status_code"] == 2  # a layer with nothing here
        assert w.moe_layer(req([3], flags=P.FLAG_SHARED))["status_code"] == 0
        # the same connection still serves the v1 message after the new one
        r = w.infer(gid(3), 1, H, BF16, BF16, act)
        assert r["status_code"] == 0 and len(r["output"]) == H * 2
        assert w.moe_layer(req([3, 17]))["status_code"] == 0
    finally:
        w.close()


def test_remote_node_over_socket_equals_local_node(node, gpu):
    """moe_dispatch.RemoteNode over a real worker socket (the integrated loop)
    gives the same bf16 partial as a LocalNode on the same experts in this
    process: the server-side dispatch without a host round trip per expert."""
    from constellation_amd.engine import Expert, Layer
    from constellation_amd.moe_dispatch import LocalNode, RemoteNode, run_topk_moe_layer
    print("[node] RemoteNode over a socket", flush=True)
    T, K = 4, 3
    rng = np.random.default_rng(3)
    ids = np.stack([rng.choice(LOCAL, K, replace=False) for _ in range(T)]).astype(np.int32)
    wts = rng.uniform(0.1, 1.0, ids.shape).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).cuda()
    w = node.worker()
    local = {}
    try:
        remote = RemoteNode.over_socket(w.sock, {LAYER: LOCAL}, shared_layers=[LAYER])
        y_remote = run_topk_moe_layer([remote], x, LAYER, ids, wts)
        for l in LOCAL + [EPL]:
            ex = node.experts[SHARED_ID if l == EPL else gid(l)]
            local[l] = Expert.upload(0, ex["w_up"], ex["s_up"], ex["w_gate"], ex["s_gate"],
                                     ex["w_down"], ex["s_down"])
        layer = Layer(gpu, [local.get(i) for i in range(EPL)], local[EPL])
        y_local = run_topk_moe_layer([LocalNode({LAYER: layer})], x, LAYER, ids, wts)
        torch.cuda.synchronize()
        layer.close()
        assert torch.equal(y_remote.view(torch.int16), y_local.view(torch.int16))
    finally:
        w.close()
        torch.cuda.synchronize()
        for e in local.values():
            e.free()


def test_upload_while_a_worker_infers(node):
    """resident_bg uploads (UploadExpertAmdV2 on the control side) while the
    worker thread serves requests: every answer stays identical."""
    print("[node] upload during inference", flush=True)
    act = _act(np.random.default_rng(5).standard_normal((1, H)), FP16)
    w = node.worker()
    first = w.infer(gid(17), 1, H, FP16, FP16, act)
    assert first["status_code"] == 0
    answers, stop = [], threading.Event()

    def serve():
        while not stop.is_set():
            answers.append(w.infer(gid(17), 1, H, FP16, FP16, act))
    t = threading.Thread(target=serve)
    t.start()
    try:
        extra = {gid(l): node.o.gen_expert(700 + l, 0x40) for l in (77, 78)}
        node.ctrl.placement([(e, 0) for e in sorted(node.experts) + sorted(extra)])
        for e, ex in extra.items():
            node.ctrl.load_expert(e, 0, ex)
        node.ctrl.wait_resident(0, list(extra))
    finally:
        stop.set()
        t.join(timeout=60)
        w.close()
    assert len(answers) > 0 and all(a == first for a in answers), len(answers)
    node.experts.update(extra)


def test_replace_then_drop(node):
    """Reloading a resident expert replaces it (the old one is freed first,
    expert_registry_v2.cc:267-281); a placement with
    drop_non_target_residents frees every other expert."""
    print("[node] replace and drop", flush=True)
    e = gid(40)
    new = node.o.gen_expert(900, 0x40)
    x = np.random.default_rng(9).standard_normal((1, H)).astype(np.float32)
    act = _act(x, FP16)
    _, ref_new = node.o.expert_ref(new, _act_f32(act, FP16).reshape(1, H))
    node.ctrl.load_expert(e, 0, new)
    w = node.worker()
    try:
        import time
        t0 = time.time()
        while True:   # the rebuild is asynchronous (resident_bg)
            got = _act_f32(w.infer(e, 1, H, FP16, FP16, act)["output"], FP16)
            if rel_l2(got, ref_new[0]) < 2e-3:
                break
            assert time.time() - t0 < 60, "replacement never became visible"
            time.sleep(0.05)
        ack = node.ctrl.placement([(e, 0)], drop_non_target=True)
        assert ack["status_code"] == 0 and ack["all_ready"]
        assert node.ctrl.resident() == {0: [e]}
        assert w.infer(gid(3), 1, H, FP16, FP16, act)["status_code"] == 2
        assert w.infer(e, 1, H, FP16, FP16, act)["status_code"] == 0
    finally:
        w.close()


def test_tiny_control_expert_and_quit(node):
    """The reference's control-test geometry (4x8 matrices, 1x1 blocks) uploads
    and becomes resident; inference on it answers status 4 (the workspace
    serves hidden 7168, as the CUDA one does).  Then quit: Reset frees every
    expert through FreeExpertWeightsAmdV2 and the arena ends empty."""
    print("[node] tiny expert, then quit", flush=True)
    rng = np.random.default_rng(11)
    tiny = {"w_up": rng.integers(0, 0x7E, (4, 8), dtype=np.uint8),
            "w_gate": rng.integers(0, 0x7E, (4, 8), dtype=np.uint8),
            "w_down": rng.integers(0, 0x7E, (8, 4), dtype=np.uint8),
            "s_up": np.full((4, 8), 0.5, np.float32), "s_gate": np.full((4, 8), 0.25, np.float32),
            "s_down": np.full((8, 4), 0.125, np.float32)}
    node.ctrl.placement([(7, 0), (gid(40), 0)])
    node.ctrl.load_expert(7, 0, tiny, rb=1, cb=1)
    node.ctrl.wait_resident(0, [7])
    w = node.worker()
    try:
        r = w.infer(7, 1, 8, FP16, FP16, _act(np.ones((1, 8)), FP16))
        assert r["status_code"] == 4 and r["output"] == b""
    finally:
        w.close()
    node.ctrl.close()
    rc = node.h.quit()
    log = node.log()
    assert rc == 0, log[-3000:]
    assert "-> 0 bytes" in log and "leaked device buffer" not in log
