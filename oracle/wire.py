"""Byte-level restatement of the reference's TCP wire frames.

TEST INFRASTRUCTURE: only tests/ may import this module.

Follows rust/src/model/transport/tcp.rs:
* :func:`kv_block_frame`      serialize_block_to_buffer :161-207 (+ tensor_to_bytes :90-110)
* :func:`ring_packet_frame`   serialize_packet_to_buffer :209-243
* :func:`parse_kv_block_frame` the KV branch of decode_frame_from_reader :604-787
* :func:`agent_metadata_bincode` the AgentMetadata blob of the block transport
  (block_transport.rs:36-86, serialized_block.rs:125-141)

serde_json 1.0.149 (rust/Cargo.lock), without its "preserve_order" feature, keeps a
``json!`` object in a BTreeMap, so ``to_string()`` writes the keys sorted, with no
spaces; floats go through ryu (shortest round-trip digits, plain notation for
decimal exponents -5 < kk <= 16 with ".0" on integral values, else ``d.ddde<exp>``).
"""
from __future__ import annotations

import json
import struct

import numpy as np

_DTYPE = {"float32": "float32", "bfloat16": "bfloat16", "float16": "float16"}


def ryu_f64(x: float) -> str:
    """serde_json's text for a finite f64 (ryu's pretty format, from the shortest
    round-trip digits, which Python's repr also yields)."""
    from decimal import Decimal
    if x == 0:
        return "-0.0" if str(x).startswith("-") else "0.0"
    t = Decimal(repr(abs(x))).normalize().as_tuple()
    digits = "".join(map(str, t.digits))
    n = len(digits)
    kk = n + t.exponent  # 10^(kk-1) <= |x| < 10^kk
    if n <= kk <= 16:
        body = digits + "0" * (kk - n) + ".0"
    elif 0 < kk <= 16:
        body = digits[:kk] + "." + digits[kk:]
    elif -5 < kk <= 0:
        body = "0." + "0" * (-kk) + digits
    elif n == 1:
        body = digits + "e" + str(kk - 1)
    else:
        body = digits[0] + "." + digits[1:] + "e" + str(kk - 1)
    return ("-" if x < 0 else "") + body


def _dumps(obj) -> str:
    if obj is None:
        return "null"
    if isinstance(obj, bool):
        return "true" if obj else "false"
    if isinstance(obj, int):
        return str(obj)
    if isinstance(obj, float):
        return ryu_f64(obj)
    if isinstance(obj, str):
        return json.dumps(obj)
    if isinstance(obj, (list, tuple)):
        return "[" + ",".join(_dumps(x) for x in obj) + "]"
    return "{" + ",".join(json.dumps(k) + ":" + _dumps(obj[k]) for k in sorted(obj)) + "}"


def _f32_bytes(x) -> bytes:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32)).astype("<f4").tobytes()


def kv_block_frame(layer_idx, start, end, k, v, dtype="float32", positions=None) -> bytes:
    """k / v: float arrays of the block's shape ([1, H, L, D]); dtype = the name the
    tensor kind maps to (tcp.rs:102-108); positions: int64 [L] or None."""
    meta = {"layer_idx": layer_idx, "global_seq_start": start, "global_seq_end": end,
            "k_shape": list(k.shape), "v_shape": list(v.shape), "k_bytes": k.size * 4, "v_bytes": v.size * 4,
            "k_dtype": _DTYPE[dtype], "v_dtype": _DTYPE[dtype], "position_ids": None}
    tail = b""
    if positions is not None:
        p = np.asarray(positions, dtype="<i8")
        meta["position_ids"] = {"shape": [p.size], "bytes": p.size * 8, "dtype": "int64"}
        tail = p.tobytes()
    m = _dumps(meta).encode()
    return struct.pack(">I", len(m)) + m + _f32_bytes(k) + _f32_bytes(v) + tail


def ring_packet_frame(layer_idx, q, o, lse, scale, q_dtype="float32", o_dtype="float32") -> bytes:
    meta = {"type": "ring_packet", "layer_idx": layer_idx, "scale": float(scale),
            "q_shape": list(q.shape), "o_shape": list(o.shape), "lse_shape": list(lse.shape),
            "q_bytes": q.size * 4, "o_bytes": o.size * 4, "lse_bytes": lse.size * 4,
            "q_dtype": q_dtype, "o_dtype": o_dtype, "lse_dtype": "float32"}
    m = _dumps(meta).encode()
    return struct.pack(">I", len(m)) + m + _f32_bytes(q) + _f32_bytes(o) + _f32_bytes(lse)


def parse_kv_block_frame(frame: bytes):
    """(meta dict, k f32 array, v f32 array, positions or None) of a KV block frame."""
    (n,) = struct.unpack(">I", frame[:4])
    meta = json.loads(frame[4:4 + n])
    off = 4 + n
    k = np.frombuffer(frame[off:off + meta["k_bytes"]], dtype="<f4").reshape(meta["k_shape"])
    off += meta["k_bytes"]
    v = np.frombuffer(frame[off:off + meta["v_bytes"]], dtype="<f4").reshape(meta["v_shape"])
    off += meta["v_bytes"]
    pos = None
    if meta.get("position_ids") is not None:
        pm = meta["position_ids"]
        pos = np.frombuffer(frame[off:off + pm["bytes"]], dtype="<i8").reshape(pm["shape"])
    return meta, k, v, pos


def agent_metadata_bincode(agent: str, blocks) -> bytes:
    """bincode 1.3.3 ``serialize(&AgentMetadata { agent, blocks })`` (rust/Cargo.lock;
    serialized_block.rs:125-141), its default configuration: little-endian, fixed-width
    integers, u64 lengths before strings and sequences, u32 variant index for a unit
    enum, struct fields in declaration order (block_transport.rs:36-86).  ``blocks`` is a
    list of (owner agent, block_id, addr, len, dev_id, mem_type (0 Dram, 1 Vram), meta
    bytes)."""
    def s_(b: bytes) -> bytes:
        return struct.pack("<Q", len(b)) + b
    out = s_(agent.encode()) + struct.pack("<Q", len(blocks))
    for owner, bid, addr, ln, dev, mem, meta in blocks:
        out += s_(owner.encode()) + struct.pack("<QQQQI", bid, addr, ln, dev, mem) + s_(meta)
    return out


def shape_meta(shape) -> bytes:
    """serde_json::to_vec of a Vec<i64> shape: compact, e.g. b"[1,2,3,4]"
    (serialized_block.rs:103-115)."""
    return ("[" + ",".join(str(int(x)) for x in shape) + "]").encode()
