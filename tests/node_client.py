"""A test-side client of the expert node's control and worker ports, for
driving oracle/_ref/node_harness (the reference's node with the AMD plugin).

The control-plane bodies follow the reference's codecs byte for byte
(little-endian; strings are u32 length + bytes):
  PlacementPlan 10        common/placement_codec.cc:8-20
  PlacementAck 11         common/placement_codec.cc:47-57 (16 bytes)
  InventoryReply 2        common/inventory_codec.h:10-31
  ResidentInventoryReply 4  common/resident_inventory_codec.h:9-18
  LoadWeightsBegin/Chunk/End 20/21/22  common/weight_codec.cc:9-120
  LoadWeightsAck 24 (empty), HeartbeatReply 51 (empty)
The worker messages (InferRequest 40, MoeLayerRequest 42) and the header
framing come from constellation_amd.moe_layer_protocol.
"""
from __future__ import annotations

import itertools
import socket
import struct
import time

import numpy as np

from constellation_amd import moe_layer_protocol as P

INVENTORY_REQUEST, INVENTORY_REPLY = 1, 2
RESIDENT_REQUEST, RESIDENT_REPLY = 3, 4
PLACEMENT_PLAN, PLACEMENT_ACK = 10, 11
LOAD_BEGIN, LOAD_CHUNK, LOAD_END, LOAD_ACK = 20, 21, 22, 24
HEARTBEAT_REQUEST, HEARTBEAT_REPLY = 50, 51

# TensorKind (common/protocol.h:39-46)
W_UP, W_GATE, W_DOWN, W_UP_SCALE, W_GATE_SCALE, W_DOWN_SCALE = range(6)

_rid = itertools.count(1)


class Reader:
    def __init__(self, b: bytes):
        self.b, self.o = b, 0

    def take(self, fmt: str):
        s = struct.Struct("<" + fmt)
        if self.o + s.size > len(self.b):
            raise P.ProtocolError("body too short")
        v = s.unpack_from(self.b, self.o)
        self.o += s.size
        return v[0] if len(v) == 1 else v

    def string(self) -> str:
        n = self.take("I")
        if self.o + n > len(self.b):
            raise P.ProtocolError("string runs past the body")
        s = self.b[self.o:self.o + n].decode()
        self.o += n
        return s

    def done(self) -> bool:
        return self.o == len(self.b)


def decode_inventory(body: bytes) -> dict:
    r = Reader(body)
    node = {"node_id": r.string(), "node_status": r.take("I"), "gpus": []}
    for _ in range(r.take("I")):
        g = {"worker_id": r.take("i"), "gpu_name": r.string(), "total_mem_bytes": r.take("Q"),
             "free_mem_bytes": r.take("Q"), "worker_port": r.take("I"), "gpu_status": r.take("I"),
             "gpu_vendor": r.take("I"), "capability_flags": r.take("I"), "arch_name": r.string()}
        node["gpus"].append(g)
    if not r.done():
        raise P.ProtocolError("trailing bytes in InventoryReply")
    return node


def decode_resident(body: bytes) -> dict[int, list[int]]:
    r = Reader(body)
    out = {}
    for _ in range(r.take("I")):
        w = r.take("i")
        out[w] = [r.take("i") for _ in range(r.take("I"))]
    if not r.done():
        raise P.ProtocolError("trailing bytes in ResidentInventoryReply")
    return out


def encode_placement(assignments, drop_non_target: bool) -> bytes:
    b = struct.pack("<II", 1 if drop_non_target else 0, len(assignments))
    for e, w in assignments:
        b += struct.pack("<ii", int(e), int(w))
    return b


def decode_placement_ack(body: bytes) -> dict:
    if len(body) != 16:
        raise P.ProtocolError(f"PlacementAck must be 16 bytes, got {len(body)}")
    st, nl, ar, nt, nr = struct.unpack("<IHHII", body)
    return {"status_code": st, "needs_load": bool(nl), "all_ready": bool(ar),
            "num_target_experts": nt, "num_ready_experts": nr}


def encode_load_begin(expert_id, worker_id, kind, total, shape, dtype, rb, cb) -> bytes:
    b = struct.pack("<iiiQI", expert_id, worker_id, kind, total, len(shape))
    b += b"".join(struct.pack("<Q", int(d)) for d in shape)
    d = dtype.encode()
    return b + struct.pack("<I", len(d)) + d + struct.pack("<II", rb, cb)


def encode_load_chunk(expert_id, worker_id, kind, offset, chunk: bytes) -> bytes:
    return struct.pack("<iiiQI", expert_id, worker_id, kind, offset, len(chunk)) + chunk


def encode_load_end(expert_id, worker_id, kind) -> bytes:
    return struct.pack("<iii", expert_id, worker_id, kind)


def connect(port: int, timeout_s: float = 60.0) -> socket.socket:
    t0 = time.time()
    while True:
        try:
            s = socket.create_connection(("127.0.0.1", port), timeout=timeout_s)
            s.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)
            return s
        except OSError:
            if time.time() - t0 > timeout_s:
                raise
            time.sleep(0.2)


class ControlClient:
    def __init__(self, port: int):
        self.sock = connect(port)

    def close(self):
        self.sock.close()

    def _req(self, t, body, expect):
        return P.request(self.sock, t, next(_rid), body, expect)

    def inventory(self) -> dict:
        return decode_inventory(self._req(INVENTORY_REQUEST, b"", INVENTORY_REPLY))

    def heartbeat(self) -> bool:
        return self._req(HEARTBEAT_REQUEST, b"", HEARTBEAT_REPLY) == b""

    def resident(self) -> dict[int, list[int]]:
        return decode_resident(self._req(RESIDENT_REQUEST, b"", RESIDENT_REPLY))

    def placement(self, assignments, drop_non_target=False) -> dict:
        return decode_placement_ack(self._req(PLACEMENT_PLAN, encode_placement(assignments, drop_non_target),
                                              PLACEMENT_ACK))

    def load_tensor(self, expert_id, worker_id, kind, data: np.ndarray, dtype: str, rb=128, cb=128,
                    chunk=4 << 20):
        raw = np.ascontiguousarray(data).tobytes()
        ack = self._req(LOAD_BEGIN, encode_load_begin(expert_id, worker_id, kind, len(raw), data.shape,
                                                      dtype, rb, cb), LOAD_ACK)
        assert ack == b""
        for off in range(0, len(raw), chunk):  # one-way: no ack per chunk (control.cc:660)
            self.sock.sendall(P.frame(LOAD_CHUNK, next(_rid),
                                      encode_load_chunk(expert_id, worker_id, kind, off,
                                                        raw[off:off + chunk])))
        assert self._req(LOAD_END, encode_load_end(expert_id, worker_id, kind), LOAD_ACK) == b""

    def load_expert(self, expert_id, worker_id, ex: dict, rb=128, cb=128, kinds=None):
        """ex: w_up/w_gate/w_down (uint8 fp8 bytes) and s_up/s_gate/s_down (fp32)."""
        order = [(W_UP, "w_up", "float8_e4m3fn"), (W_GATE, "w_gate", "float8_e4m3fn"),
                 (W_DOWN, "w_down", "float8_e4m3fn"), (W_UP_SCALE, "s_up", "float32"),
                 (W_GATE_SCALE, "s_gate", "float32"), (W_DOWN_SCALE, "s_down", "float32")]
        for kind, key, dt in order:
            if kinds is None or kind in kinds:
                self.load_tensor(expert_id, worker_id, kind, ex[key], dt, rb, cb)

    def wait_resident(self, worker_id, ids, timeout_s=120.0) -> list[int]:
        want = set(ids)
        t0 = time.time()
        while True:
            have = set(self.resident().get(worker_id, []))
            if want <= have:
                return sorted(have)
            if time.time() - t0 > timeout_s:
                raise TimeoutError(f"experts {sorted(want - have)} not resident after {timeout_s}s")
            time.sleep(0.05)


class WorkerClient:
    def __init__(self, port: int):
        self.sock = connect(port)

    def close(self):
        self.sock.close()

    def infer(self, expert_id, batch, hidden, in_dt, out_dt, activation: bytes) -> dict:
        body = P.encode_infer_request({"expert_id": expert_id, "batch_size": batch,
                                       "hidden_dim": hidden, "input_dtype": in_dt,
                                       "output_dtype": out_dt, "activation": activation})
        return P.decode_infer_response(P.request(self.sock, P.INFER_REQUEST, next(_rid), body,
                                                 P.INFER_RESPONSE))

    def moe_layer(self, body: bytes) -> dict:
        return P.decode_moe_layer_response(P.request(self.sock, P.MOE_LAYER_REQUEST, next(_rid), body,
                                                     P.MOE_LAYER_RESPONSE))


HARNESS = __import__("pathlib").Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "node_harness"


def free_port_pair() -> tuple[int, int]:
    """Two free local ports: control, worker base (one GPU: one worker port)."""
    socks = [socket.socket() for _ in range(2)]
    try:
        for s in socks:
            s.bind(("127.0.0.1", 0))
        return tuple(s.getsockname()[1] for s in socks)
    finally:
        for s in socks:
            s.close()


class Harness:
    """oracle/_ref/node_harness as a child process (its output goes to a log file)."""

    def __init__(self, log_path):
        import subprocess
        self.ctrl, self.wbase = free_port_pair()
        self.log = open(log_path, "w")
        self.proc = subprocess.Popen([str(HARNESS), "--control-port", str(self.ctrl),
                                      "--worker-base-port", str(self.wbase)],
                                     stdin=subprocess.PIPE, stdout=self.log, stderr=subprocess.STDOUT)

    def quit(self, timeout_s: float = 60.0) -> int:
        self.proc.stdin.write(b"quit\n")
        self.proc.stdin.flush()
        rc = self.proc.wait(timeout=timeout_s)
        self.log.close()
        return rc

    def kill(self):
        if self.proc.poll() is None:
            self.proc.kill()
            self.proc.wait(timeout=30)
        if not self.log.closed:
            self.log.close()
