"""Writes the small golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference holds no tensor goldens for this path (its ring tests draw inputs and
compare against a dense closed form at run time, ring.rs:2381-2521 and
rust/src/smoke/reference_algo.rs:134-167), so the fixtures are made the same way:
inputs from the reference's seeded LCG + Box-Muller generator (restated in
oracle/hcp_oracle.c), expected outputs from the f64 closed form
(oracle/closed_form.py) or, for paged staging, from the index map of
python/hcp_vllm_block_ring_plugin.py:304-337 evaluated by the C oracle.

Each fixture is an ``.npz`` of inputs (bf16 as uint16 bit patterns) and expected
outputs, plus the scalar parameters.  Sizes are kept small (a few hundred KiB in all).
"""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import clib, closed_form as C, inputs as I  # noqa: E402


def block_case(name, seed, lq, lk, hq, hkv, d, q_off, k_off, causal):
    qb, kb, vb = clib.draw_normals(seed, [(lq, hq, d), (lk, hkv, d), (lk, hkv, d)], "bf16")
    q, k, v = (I.bf16_bits_to_f32(b) for b in (qb, kb, vb))
    scale = 1 / math.sqrt(d)
    o, lse = C.attention_f64(q, k, v, np.arange(q_off, q_off + lq), np.arange(k_off, k_off + lk), scale,
                             causal=causal)
    np.savez_compressed(os.path.join(HERE, name), seed=seed, q_bits=qb, k_bits=kb, v_bits=vb,
                        q_offset=q_off, kv_offset=k_off, causal=int(causal), scale=scale,
                        o=o.astype(np.float32), lse=lse.astype(np.float32))


def ring_case(name, seed, chunks, hq, hkv, d):
    s = sum(chunks)
    q, k, v = clib.draw_normals(seed, [(s, hq, d), (s, hkv, d), (s, hkv, d)], "fp32")
    pos = np.arange(s)
    o, lse = C.attention_f64(q, k, v, pos, pos, 1 / math.sqrt(d))
    np.savez_compressed(os.path.join(HERE, name), seed=seed, chunks=np.array(chunks), q=q, k=k, v=v,
                        o=o.astype(np.float32), lse=lse.astype(np.float32))


def merge_case(name, seed):
    h, l, d, n = 2, 6, 128, 3
    parts = clib.draw_normals(seed, [(h, l, d)] * n + [(h, l)] * n, "fp32")
    os_, lses = parts[:n], [x * 3.0 for x in parts[n:]]
    lses[0][0, 1] = -np.inf                 # one empty partial in a row
    lses[1][1, 2] = lses[2][1, 2] = -np.inf
    for p in range(n):                      # an empty row in every partial
        lses[p][1, 4] = -np.inf
    for p in range(n):                      # an empty partial carries o = 0 (ring.rs:553-569)
        os_[p][np.isneginf(lses[p])] = 0.0
    o, lse = C.merge_partials_f64(os_, lses)
    np.savez_compressed(os.path.join(HERE, name), seed=seed, o_parts=np.stack(os_), lse_parts=np.stack(lses),
                        o=o.astype(np.float32), lse=lse.astype(np.float32))


def paged_case(name, seed):
    nb, bs, hkv, d = 6, 16, 2, 64
    pool = clib.draw_normals(seed, [(2, nb, bs, hkv, d)], "bf16")[0]
    table = np.array([4, 1, 5, 2], dtype=np.int32)
    t0, t1 = 5, 57                                  # ragged at both ends
    k, v = clib.paged_gather(pool, table, 0, t0, t1)
    # scatter of a fresh buffer over tokens [0, 40) of a zeroed pool with table [3, 0, 5]
    src_k, src_v = clib.draw_normals(seed + 1, [(hkv, 40, d), (hkv, 40, d)], "bf16")
    scat = np.full_like(pool, 0x7fc1)              # poison: untouched slots keep it
    stable = np.array([3, 0, 5], dtype=np.int32)
    clib.paged_scatter(scat, stable, 0, 0, 40, src_k, src_v, zero_tail=True)
    np.savez_compressed(os.path.join(HERE, name), seed=seed, pool_bits=pool, table=table, t0=t0, t1=t1,
                        k_bits=k, v_bits=v, scatter_table=stable, scatter_k_bits=src_k, scatter_v_bits=src_v,
                        scatter_pool_bits=scat)


def decode_case(name, seed):
    b, hq, hkv, d, bs, nb = 2, 8, 2, 64, 16, 12
    qb, poolb = clib.draw_normals(seed, [(b, hq, d), (2, nb, bs, hkv, d)], "bf16")
    tables = I.permuted_block_table(seed, nb).astype(np.int32).reshape(b, nb // b)
    t0, t1 = 16, 88                                 # 72 tokens, a partial last block
    q, pool = I.bf16_bits_to_f32(qb), I.bf16_bits_to_f32(poolb)
    o = np.zeros((b, hq, d))
    lse = np.zeros((b, hq))
    for i in range(b):
        k, v = clib.paged_gather(pool, tables[i], 0, t0, t1)
        oi, li = C.attention_f64(q[i][None], k.transpose(1, 0, 2), v.transpose(1, 0, 2), np.zeros(1),
                                 np.zeros(t1 - t0), 1 / math.sqrt(d), causal=False)
        o[i], lse[i] = oi[0], li[0]
    np.savez_compressed(os.path.join(HERE, name), seed=seed, q_bits=qb, pool_bits=poolb, tables=tables,
                        t0=t0, t1=t1, o=o.astype(np.float32), lse=lse.astype(np.float32))


def kats(name):
    """Known answers asserted by the reference's own tests for this path."""
    data = {
        "vanilla_assignment": {"source": "rust/src/model/attention/strategy.rs:157-163",
                               "chunks": [3, 1], "expected": [0, 0, 0, 1]},
        "vanilla_offsets_c3": {"source": "rust/src/smoke/reference_algo.rs:92-116 (prefix sums)",
                               "chunks": [12288, 8192, 8192, 4096], "expected": [0, 12288, 20480, 28672]},
        "ring_sources": {"source": "rust/src/model/transport/mock.rs:143-149 (round r from (d-1-r) mod N)",
                         "num_domains": 4,
                         "expected": {"0": [0, 3, 2, 1], "1": [1, 0, 3, 2], "2": [2, 1, 0, 3], "3": [3, 2, 1, 0]}},
        "strategies": [
            {"source": "rust/src/model/attention/strategy.rs:165-170", "strategy": "striped",
             "chunks": [3, 1], "assignment": [0, 1, 0, 0]},
            {"source": "rust/src/model/attention/strategy.rs:172-181", "strategy": "zigzag",
             "chunks": [3, 1], "assignment": [0, 0, 1, 0], "positions": [[0, 1, 3], [2]]},
            {"source": "rust/src/model/attention/strategy.rs:183-192", "strategy": "zigzag",
             "chunks": [4, 4], "assignment": [0, 0, 1, 1, 1, 1, 0, 0], "positions": [[0, 1, 6, 7], [2, 3, 4, 5]]},
            {"source": "rust/src/model/attention/strategy.rs:194-201", "strategy": "striped",
             "chunks": [3, 1], "inverse_perm": [0, 3, 1, 2]},
        ],
    }
    with open(os.path.join(HERE, name), "w") as f:
        json.dump(data, f, indent=1)


def wire_frames(name):
    """Frames of the reference's own TCP transport tests, restated byte for byte."""
    from oracle import wire as W
    ar = lambda n, s, shape: (np.arange(n, dtype=np.float32) * s).reshape(shape)
    cases = [
        ("positioned_partial_frame", "rust/src/model/transport/tcp.rs:816-864",
         dict(layer_idx=7, start=2, end=10, k=ar(4, 1.0, (1, 1, 2, 2)), v=ar(4, 0.25, (1, 1, 2, 2)),
              positions=[2, 9])),
        ("positioned_roundtrip", "rust/src/model/transport/tcp.rs:898-935",
         dict(layer_idx=5, start=0, end=3, k=ar(6, 1.0, (1, 1, 3, 2)), v=ar(6, 0.5, (1, 1, 3, 2)),
              positions=[0, 9, 16777217])),
        ("unpositioned", "rust/src/model/transport/tcp.rs:867-896 (KvBlock::single)",
         dict(layer_idx=3, start=4, end=6, k=ar(4, 1.0, (1, 1, 2, 2)), v=ar(4, 1.0, (1, 1, 2, 2)), positions=None)),
    ]
    out = []
    for cname, src, c in cases:
        frame = W.kv_block_frame(c["layer_idx"], c["start"], c["end"], c["k"], c["v"], "float32", c["positions"])
        out.append({"name": cname, "source": src, "kind": "kv_block", "layer_idx": c["layer_idx"],
                    "start": c["start"], "end": c["end"], "k": c["k"].tolist(), "v": c["v"].tolist(),
                    "positions": c["positions"], "frame_hex": frame.hex()})
    # the legacy frame of tcp.rs:937-963: position_ids removed from the meta
    legacy = W.kv_block_frame(2, 4, 6, ar(4, 1.0, (1, 1, 2, 2)), ar(4, 1.0, (1, 1, 2, 2)), "float32", None)
    n = int.from_bytes(legacy[:4], "big")
    meta = json.loads(legacy[4:4 + n])
    del meta["position_ids"]
    m = W._dumps(meta).encode()
    out.append({"name": "legacy_without_position_metadata", "source": "rust/src/model/transport/tcp.rs:802-813,937-963",
                "kind": "kv_block", "layer_idx": 2, "start": 4, "end": 6, "positions": None,
                "frame_hex": (len(m).to_bytes(4, "big") + m + legacy[4 + n:]).hex()})
    q = ar(16, 0.5, (1, 2, 1, 8))
    o = ar(16, -0.25, (1, 2, 1, 8))
    lse = ar(2, 1.5, (1, 2, 1))
    pk = W.ring_packet_frame(4, q, o, lse, 1 / math.sqrt(8), "bfloat16", "bfloat16")
    out.append({"name": "ring_packet", "source": "rust/src/model/transport/tcp.rs:209-243", "kind": "ring_packet",
                "layer_idx": 4, "scale": 1 / math.sqrt(8), "q": q.tolist(), "o": o.tolist(), "lse": lse.tolist(),
                "frame_hex": pk.hex()})
    with open(os.path.join(HERE, name), "w") as f:
        json.dump(out, f, indent=1)


def main():
    block_case("block_bf16_gqa4.npz", 101, 72, 136, 4, 1, 128, 100, 0, True)
    block_case("block_bf16_future_d64.npz", 102, 64, 64, 2, 2, 64, 0, 50, True)
    ring_case("ring_fp32_two_domains.npz", 42, [40, 24], 2, 2, 64)
    merge_case("merge_three_parts.npz", 103)
    paged_case("paged_bf16_ragged.npz", 104)
    decode_case("decode_bf16_small.npz", 105)
    kats("reference_kats.json")
    wire_frames("wire_frames.json")


if __name__ == "__main__":
    main()
