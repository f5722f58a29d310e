"""Server-side codec of the whole-layer wire message.

MoeLayerRequest (msg_type 42) carries every route of a token batch that a
node's experts serve, so the server sends one request per node per layer
instead of one InferRequest per selected expert
(server/moe_layer_runtime.py:111-145, infer_one_expert :27-81).  The node
answers with MoeLayerResponse (43): the partial weighted sum of its experts
(+ the shared expert when asked), combined in route order in fp32 and rounded
once.  The header framing, little-endian packing and exact-length decoding
follow common/protocol.py:495-586; v1 InferRequest/InferResponse are left
untouched.  The byte layout is declared in include/cx_moe.h and decoded on
the node by cx_moe_layer_request_run.
"""
from __future__ import annotations

import socket
import struct

import numpy as np

# v1 framing (common/protocol.h:10-62): every message is a 16-byte little-endian
# header (magic "EXPT", version 1, msg_type, request_id, body_len) + body.
MAGIC = 0x45585054
VERSION = 1
INFER_REQUEST = 40
INFER_RESPONSE = 41
MOE_LAYER_REQUEST = 42
MOE_LAYER_RESPONSE = 43
FLAG_SHARED = 1
HEADER_BYTES = 16

_HDR = struct.Struct("<IHHII")
_I32 = struct.Struct("<i")
_U32 = struct.Struct("<I")


class ProtocolError(ValueError):
    pass


def encode_header(msg_type: int, request_id: int, body_len: int) -> bytes:
    return _HDR.pack(MAGIC, VERSION, int(msg_type), int(request_id) & 0xFFFFFFFF, int(body_len))


def decode_header(b: bytes) -> dict:
    """Header fields; a wrong magic or version is a ProtocolError, as the worker
    loop closes the connection on them (expert_node_v2/worker.cc:219-235)."""
    if len(b) != HEADER_BYTES:
        raise ProtocolError(f"header must be {HEADER_BYTES} bytes, got {len(b)}")
    magic, version, msg_type, rid, n = _HDR.unpack(b)
    if magic != MAGIC:
        raise ProtocolError(f"bad magic 0x{magic:x}")
    if version != VERSION:
        raise ProtocolError(f"bad version {version}")
    return {"magic": magic, "version": version, "msg_type": msg_type, "request_id": rid,
            "body_len": n}


def frame(msg_type: int, request_id: int, body: bytes) -> bytes:
    """Header + body, ready for one sendall."""
    return encode_header(msg_type, request_id, len(body)) + bytes(body)


def _recv_exact(sock: socket.socket, n: int) -> bytes:
    buf = bytearray()
    while len(buf) < n:
        chunk = sock.recv(n - len(buf))
        if not chunk:
            raise ConnectionError(f"connection closed after {len(buf)} of {n} bytes")
        buf += chunk
    return bytes(buf)


def recv_frame(sock: socket.socket) -> tuple[dict, bytes]:
    """Reads one framed message: (header fields, body)."""
    hdr = decode_header(_recv_exact(sock, HEADER_BYTES))
    return hdr, _recv_exact(sock, hdr["body_len"])


def request(sock: socket.socket, msg_type: int, request_id: int, body: bytes,
            expect_type: int) -> bytes:
    """Sends one framed request on a connected socket and returns the reply body
    (checking its type and request_id)."""
    sock.sendall(frame(msg_type, request_id, body))
    hdr, reply = recv_frame(sock)
    if hdr["msg_type"] != expect_type or hdr["request_id"] != (int(request_id) & 0xFFFFFFFF):
        raise ProtocolError(f"unexpected reply type={hdr['msg_type']} rid={hdr['request_id']}")
    return reply


# -- v1 InferRequest / InferResponse (common/infer_codec.cc:7-76; byte-identical) --

def encode_infer_request(msg) -> bytes:
    act = msg["activation"]
    if not isinstance(act, (bytes, bytearray)):
        raise ValueError("activation must be bytes-like")
    return (_I32.pack(int(msg["expert_id"])) + _I32.pack(int(msg["batch_size"])) +
            _I32.pack(int(msg["hidden_dim"])) + _U32.pack(int(msg["input_dtype"])) +
            _U32.pack(int(msg["output_dtype"])) + _U32.pack(len(act)) + bytes(act))


def decode_infer_response(body: bytes):
    off = 0
    vals = []
    for what in ("status_code", "batch_size", "hidden_dim"):
        b, off = _take(body, off, 4, what)
        vals.append(_I32.unpack(b)[0])
    b, off = _take(body, off, 4, "output_dtype")
    out_dt = _U32.unpack(b)[0]
    b, off = _take(body, off, 4, "output_nbytes")
    nb = _U32.unpack(b)[0]
    out, off = _take(body, off, nb, "output")
    if off != len(body):
        raise ProtocolError(f"infer_response has trailing bytes: parsed {off}, total {len(body)}")
    return {"status_code": vals[0], "batch_size": vals[1], "hidden_dim": vals[2],
            "output_dtype": out_dt, "output": out}


def _take(body: bytes, off: int, n: int, what: str):
    if off + n > len(body):
        raise ProtocolError(f"buffer too short while reading {what}")
    return body[off:off + n], off + n


def encode_moe_layer_request(msg) -> bytes:
    """msg: layer_id, batch_size, hidden_dim, top_k, input_dtype, output_dtype,
    flags, expert_ids [T*K] (int, -1 = none), expert_weights [T*K] (float),
    activation (bytes, T*H*2)."""
    T, H, K = int(msg["batch_size"]), int(msg["hidden_dim"]), int(msg["top_k"])
    ids = np.ascontiguousarray(np.asarray(msg["expert_ids"], dtype="<i4").reshape(-1))
    wts = np.ascontiguousarray(np.asarray(msg["expert_weights"], dtype="<f4").reshape(-1))
    act = msg["activation"]
    if not isinstance(act, (bytes, bytearray)):
        raise ValueError("activation must be bytes-like")
    if ids.size != T * K or wts.size != T * K:
        raise ValueError(f"expected {T * K} routes, got {ids.size} ids / {wts.size} weights")
    if len(act) != T * H * 2:
        raise ValueError(f"activation has {len(act)} bytes, expected {T * H * 2}")
    body = bytearray()
    for v in (msg["layer_id"], T, H, K):
        body += _I32.pack(int(v))
    for v in (msg["input_dtype"], msg["output_dtype"], msg.get("flags", 0), T * K):
        body += _U32.pack(int(v))
    body += ids.tobytes()
    body += wts.tobytes()
    body += _U32.pack(len(act))
    body += act
    return bytes(body)


def decode_moe_layer_request(body: bytes):
    off = 0
    vals = []
    for what in ("layer_id", "batch_size", "hidden_dim", "top_k"):
        b, off = _take(body, off, 4, what)
        vals.append(_I32.unpack(b)[0])
    for what in ("input_dtype", "output_dtype", "flags", "n_routes"):
        b, off = _take(body, off, 4, what)
        vals.append(_U32.unpack(b)[0])
    layer_id, T, H, K, in_dt, out_dt, flags, n = vals
    if n != T * K:
        raise ProtocolError(f"n_routes {n} != batch_size * top_k")
    b, off = _take(body, off, 4 * n, "expert_ids")
    ids = np.frombuffer(b, dtype="<i4").copy()
    b, off = _take(body, off, 4 * n, "expert_weights")
    wts = np.frombuffer(b, dtype="<f4").copy()
    b, off = _take(body, off, 4, "activation_nbytes")
    nb = _U32.unpack(b)[0]
    if nb != T * H * 2:
        raise ProtocolError(f"activation_nbytes {nb} != batch_size * hidden_dim * 2")
    act, off = _take(body, off, nb, "activation")
    if off != len(body):
        raise ProtocolError(f"moe_layer_request has trailing bytes: parsed {off}, total {len(body)}")
    return {"layer_id": layer_id, "batch_size": T, "hidden_dim": H, "top_k": K,
            "input_dtype": in_dt, "output_dtype": out_dt, "flags": flags,
            "expert_ids": ids.reshape(T, K), "expert_weights": wts.reshape(T, K),
            "activation": act}


def encode_moe_layer_response(msg) -> bytes:
    out = msg["output"]
    if not isinstance(out, (bytes, bytearray)):
        raise ValueError("output must be bytes-like")
    return (_I32.pack(int(msg["status_code"])) + _I32.pack(int(msg["batch_size"])) +
            _I32.pack(int(msg["hidden_dim"])) + _U32.pack(int(msg["output_dtype"])) +
            _U32.pack(len(out)) + bytes(out))


def decode_moe_layer_response(body: bytes):
    off = 0
    b, off = _take(body, off, 4, "status_code")
    status = _I32.unpack(b)[0]
    b, off = _take(body, off, 4, "batch_size")
    T = _I32.unpack(b)[0]
    b, off = _take(body, off, 4, "hidden_dim")
    H = _I32.unpack(b)[0]
    b, off = _take(body, off, 4, "output_dtype")
    out_dt = _U32.unpack(b)[0]
    b, off = _take(body, off, 4, "output_nbytes")
    nb = _U32.unpack(b)[0]
    out, off = _take(body, off, nb, "output")
    if off != len(body):
        raise ProtocolError(f"moe_layer_response has trailing bytes: parsed {off}, total {len(body)}")
    return {"status_code": status, "batch_size": T, "hidden_dim": H, "output_dtype": out_dt,
            "output": out}
