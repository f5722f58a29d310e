"""Whole-layer wire message (MoeLayerRequest 42 / MoeLayerResponse 43): the
Python server-side codec and the node-side C decoder agree on every field,
and both reject truncated, padded or inconsistent bodies (the exact-length
rule of common/infer_codec.cc:22-43).  Host-only: no GPU calls."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from constellation_amd import moe_layer_protocol as P


def _msg(T=3, H=64, K=4, seed=0, flags=P.FLAG_SHARED, in_dt=2, out_dt=1):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-1, 32, (T, K)).astype(np.int32)
    wts = rng.uniform(0, 1, (T, K)).astype(np.float32)
    act = rng.integers(0, 256, T * H * 2, dtype=np.uint8).tobytes()
    return {"layer_id": 7, "batch_size": T, "hidden_dim": H, "top_k": K, "input_dtype": in_dt,
            "output_dtype": out_dt, "flags": flags, "expert_ids": ids, "expert_weights": wts,
            "activation": act}


def _peek(body: bytes):
    from constellation_amd._lib import MoeLayerRequestInfo, check, lib
    info = MoeLayerRequestInfo()
    b = np.frombuffer(body, np.uint8) if body else np.zeros(1, np.uint8)
    check(lib().cx_moe_layer_request_peek(b.ctypes.data, len(body), C.byref(info)))
    return info


@pytest.mark.parametrize("T,H,K", [(1, 64, 8), (3, 64, 4), (20, 128, 6), (2, 64, 0)])
def test_request_round_trip_python(T, H, K):
    m = _msg(T, H, K, seed=T)
    body = P.encode_moe_layer_request(m)
    assert len(body) == 32 + 8 * T * K + 4 + T * H * 2
    d = P.decode_moe_layer_request(body)
    for k in ("layer_id", "batch_size", "hidden_dim", "top_k", "input_dtype", "output_dtype",
              "flags", "activation"):
        assert d[k] == m[k], k
    assert np.array_equal(d["expert_ids"], m["expert_ids"])
    assert np.array_equal(d["expert_weights"], m["expert_weights"])


def test_request_header_known_bytes():
    """Field order and little-endian packing, pinned on a hand-written body."""
    m = {"layer_id": 3, "batch_size": 1, "hidden_dim": 2, "top_k": 1, "input_dtype": 1,
         "output_dtype": 2, "flags": 1, "expert_ids": [5], "expert_weights": [0.5],
         "activation": b"\x01\x02\x03\x04"}
    want = bytes.fromhex("03000000" "01000000" "02000000" "01000000" "01000000" "02000000"
                         "01000000" "01000000" "05000000" "0000003f" "04000000" "01020304")
    assert P.encode_moe_layer_request(m) == want


@pytest.mark.parametrize("T,H,K,flags", [(1, 64, 8, 1), (5, 128, 3, 0), (17, 64, 6, 1)])
def test_node_decoder_agrees_with_python_encoder(T, H, K, flags):
    m = _msg(T, H, K, seed=11 * T, flags=flags)
    info = _peek(P.encode_moe_layer_request(m))
    assert (info.layer_id, info.batch_size, info.hidden_dim, info.top_k) == (7, T, H, K)
    assert (info.input_dtype, info.output_dtype, info.flags) == (2, 1, flags)


def test_response_round_trip_and_size():
    from constellation_amd._lib import lib
    out = bytes(range(256)) * 2
    body = P.encode_moe_layer_response({"status_code": 0, "batch_size": 2, "hidden_dim": 128,
                                        "output_dtype": 2, "output": out})
    assert len(body) == lib().cx_moe_layer_response_size(2, 128)
    d = P.decode_moe_layer_response(body)
    assert d == {"status_code": 0, "batch_size": 2, "hidden_dim": 128, "output_dtype": 2,
                 "output": out}
    with pytest.raises(P.ProtocolError):
        P.decode_moe_layer_response(body + b"\x00")
    with pytest.raises(P.ProtocolError):
        P.decode_moe_layer_response(body[:-1])


def _corrupt(body: bytes, field: int, value: int) -> bytes:
    b = bytearray(body)
    b[4 * field:4 * field + 4] = value.to_bytes(4, "little", signed=value < 0)
    return bytes(b)


@pytest.mark.parametrize("case", ["truncated", "trailing", "n_routes", "act_nbytes", "dtype",
                                  "flags", "top_k", "batch", "empty"])
def test_malformed_bodies_rejected_by_both_sides(case):
    from constellation_amd import CxError
    m = _msg(3, 64, 4, seed=5)
    body = P.encode_moe_layer_request(m)
    n = 3 * 4
    bad = {
        "truncated": body[:-1],
        "trailing": body + b"\x00",
        "n_routes": _corrupt(body, 7, n + 1),
        "act_nbytes": body[:32 + 8 * n] + (3 * 64 * 2 - 2).to_bytes(4, "little") + body[36 + 8 * n:-2],
        "dtype": _corrupt(body, 4, 3),
        "flags": _corrupt(body, 6, 2),
        "top_k": _corrupt(body, 3, 65),
        "batch": _corrupt(body, 1, 0),
        "empty": b"",
    }[case]
    with pytest.raises(CxError):
        _peek(bad)
    if case in ("truncated", "trailing", "n_routes", "act_nbytes", "empty"):
        with pytest.raises(P.ProtocolError):
            P.decode_moe_layer_request(bad)


def test_random_and_mutated_bodies_never_crash_and_agree():
    """Fuzz of the node-side decoder, which reads bytes off the network: random
    bodies and single-field mutations of valid ones either decode to exactly
    what the Python codec reads, or are rejected by both sides; nothing reads
    out of bounds (the decoder gets the exact buffer length)."""
    from constellation_amd import CxError
    rng = np.random.default_rng(1234)
    bodies = []
    for i in range(300):  # random lengths and bytes, header-sized and up
        bodies.append(rng.integers(0, 256, int(rng.integers(0, 96)), dtype=np.uint8).tobytes())
    for i in range(300):  # valid bodies with one header word replaced, or cut / padded
        T, H, K = int(rng.integers(1, 5)), int(rng.choice([32, 64])), int(rng.integers(0, 9))
        body = bytearray(P.encode_moe_layer_request(_msg(T, H, K, seed=i)))
        kind = i % 3
        if kind == 0:
            w = int(rng.integers(0, 9))
            v = int(rng.choice([0, 1, 2, 3, 64, 65, 0x7FFFFFFF, 0xFFFFFFFF, int(rng.integers(0, 1 << 32))]))
            at = 4 * w if w < 8 else 32 + 8 * T * K
            body[at:at + 4] = v.to_bytes(4, "little")
        elif kind == 1:
            body = body[:int(rng.integers(0, len(body)))]
        else:
            body = body + bytes(int(rng.integers(1, 9)))
        bodies.append(bytes(body))
    accepted = 0
    for body in bodies:
        try:
            py = P.decode_moe_layer_request(body)
        except P.ProtocolError:
            py = None
        try:
            info = _peek(body)
        except CxError:
            info = None
        if info is None:
            continue
        accepted += 1
        assert py is not None
        assert (info.layer_id, info.batch_size, info.hidden_dim, info.top_k) == \
            (py["layer_id"], py["batch_size"], py["hidden_dim"], py["top_k"])
        assert len(body) == 32 + 8 * py["batch_size"] * py["top_k"] + 4 + \
            py["batch_size"] * py["hidden_dim"] * 2
    assert accepted > 0
