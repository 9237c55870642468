"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU tests pin the fixtures to the oracle by independent routes: the seeded generator
reproduces the stored inputs bit for bit, the f64 closed form reproduces the stored
outputs, the op-for-op libtorch restatement of ring.rs lands within the reference's
Relaxed tier (1e-4, rust/src/error.rs:56-76) of them, the paged fixture matches a
pure-Python evaluation of the index map, and the reference's own known answers hold for
the host helpers.  GPU tests run the HIP library through the C ABI on the stored
inputs and compare with the stored outputs (bf16: out <= 2e-2, LSE <= 1e-3; fp32:
1e-4; paged staging bit-exact).
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import hcp_ring_amd as H
from oracle import clib, closed_form as C, inputs as I, tch_ring as T

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BLOCK_FIXTURES = ["block_bf16_gqa4.npz", "block_bf16_future_d64.npz"]


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def f32(bits):
    return I.bf16_bits_to_f32(bits)


def bhsd(x):
    return torch.from_numpy(np.ascontiguousarray(x)).permute(1, 0, 2).unsqueeze(0)


# ------------------------------------------------------------------------ CPU ----
@pytest.mark.parametrize("name", BLOCK_FIXTURES)
def test_block_fixture_inputs_regenerate(name):
    g = load(name)
    fresh = clib.draw_normals(int(g["seed"]), [g["q_bits"].shape, g["k_bits"].shape, g["v_bits"].shape], "bf16")
    for a, b in zip(fresh, (g["q_bits"], g["k_bits"], g["v_bits"])):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("name", BLOCK_FIXTURES)
def test_block_fixture_matches_closed_form_and_restatement(name):
    g = load(name)
    q, k, v = f32(g["q_bits"]), f32(g["k_bits"]), f32(g["v_bits"])
    lq, lk = q.shape[0], k.shape[0]
    qo, ko, sc = int(g["q_offset"]), int(g["kv_offset"]), float(g["scale"])
    qp, kp = np.arange(qo, qo + lq), np.arange(ko, ko + lk)
    o, lse = C.attention_f64(q, k, v, qp, kp, sc, causal=bool(g["causal"]))
    assert np.abs(o - g["o"]).max() <= 1e-6
    assert np.array_equal(np.isneginf(lse), np.isneginf(g["lse"]))
    fin = np.isfinite(lse)
    assert np.abs(lse[fin] - g["lse"][fin]).max() <= 1e-5
    # ring.rs:538-571 restated op for op in fp32 on the same upcasts
    rep = q.shape[1] // k.shape[1]
    to, tl = T.positioned_local_compact_partial(sc, bhsd(q), torch.from_numpy(qp),
                                                T.repeat_kv_heads(bhsd(k), rep),
                                                T.repeat_kv_heads(bhsd(v), rep), torch.from_numpy(kp))
    to = to[0].permute(1, 0, 2).numpy()
    tl = tl[0].T.numpy()
    assert np.abs(to - g["o"]).max() <= 1e-4
    assert np.abs(tl[fin] - g["lse"][fin]).max() <= 1e-4


def test_block_future_fixture_has_empty_rows():
    g = load("block_bf16_future_d64.npz")
    # q positions 0..63 against keys 50..113: rows 0..49 see nothing -> (0, -inf)
    assert np.isneginf(g["lse"][:50]).all() and np.isfinite(g["lse"][50:]).all()
    assert (g["o"][:50] == 0).all()


def test_ring_fixture_relaxed_tier():
    g = load("ring_fp32_two_domains.npz")
    chunks = [int(c) for c in g["chunks"]]
    fresh = clib.draw_normals(int(g["seed"]), [g["q"].shape, g["k"].shape, g["v"].shape], "fp32")
    assert all(np.array_equal(a, b) for a, b in zip(fresh, (g["q"], g["k"], g["v"])))
    out = T.ring_attention_replay(1 / math.sqrt(g["q"].shape[2]), bhsd(g["q"]), bhsd(g["k"]), bhsd(g["v"]),
                                  chunks)
    assert np.abs(out[0].permute(1, 0, 2).numpy() - g["o"]).max() <= 1e-4


def test_merge_fixture_by_logaddexp():
    g = load("merge_three_parts.npz")
    lses, os_ = g["lse_parts"].astype(np.float64), g["o_parts"].astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        lse = np.logaddexp.reduce(lses, axis=0)
        w = np.where(np.isfinite(lse)[None], np.exp(lses - lse[None]), 0.0)
    o = (w[..., None] * os_).sum(axis=0)
    assert np.array_equal(np.isneginf(lse), np.isneginf(g["lse"]))
    fin = np.isfinite(lse)
    assert np.abs(lse[fin] - g["lse"][fin]).max() <= 1e-5
    assert np.abs(o - g["o"]).max() <= 1e-5
    assert (g["o"][~fin] == 0).all()


def test_paged_fixture_by_python_index_map():
    g = load("paged_bf16_ragged.npz")
    pool, table, t0, t1 = g["pool_bits"], g["table"], int(g["t0"]), int(g["t1"])
    bs = pool.shape[2]
    for plane, out in ((0, g["k_bits"]), (1, g["v_bits"])):
        for t in range(t0, t1):
            blk, slot = table[t // bs], t % bs
            assert np.array_equal(out[:, t - t0], pool[plane, blk, slot])
    # scatter: written slots hold the source, the tail of the last block is zero,
    # every other block keeps the poison pattern
    scat, st = g["scatter_pool_bits"], g["scatter_table"]
    for t in range(40):
        assert np.array_equal(scat[0, st[t // bs], t % bs], g["scatter_k_bits"][:, t])
        assert np.array_equal(scat[1, st[t // bs], t % bs], g["scatter_v_bits"][:, t])
    assert (scat[:, st[2], 40 % bs:] == 0).all()
    untouched = [b for b in range(pool.shape[1]) if b not in set(st.tolist())]
    assert (scat[:, untouched] == 0x7fc1).all()


def test_decode_fixture_matches_restatement():
    g = load("decode_bf16_small.npz")
    q, pool = f32(g["q_bits"]), f32(g["pool_bits"])
    t0, t1 = int(g["t0"]), int(g["t1"])
    hq, hkv, d = q.shape[1], pool.shape[3], q.shape[2]
    for b in range(q.shape[0]):
        k, v = clib.paged_gather(pool, g["tables"][b], 0, t0, t1)
        kx = T.repeat_kv_heads(torch.from_numpy(k).unsqueeze(0), hq // hkv)
        vx = T.repeat_kv_heads(torch.from_numpy(v).unsqueeze(0), hq // hkv)
        o, lse = T.decode_local_compact_partial(1 / math.sqrt(d), torch.from_numpy(q[b]).view(1, hq, 1, d), kx, vx)
        assert np.abs(o.view(hq, d).numpy() - g["o"][b]).max() <= 1e-4
        assert np.abs(lse.view(hq).numpy() - g["lse"][b]).max() <= 1e-4


def test_reference_known_answers():
    with open(os.path.join(GOLD, "reference_kats.json")) as f:
        kat = json.load(f)
    a = kat["vanilla_assignment"]
    assert H.vanilla_assignment(a["chunks"]) == a["expected"]
    o = kat["vanilla_offsets_c3"]
    assert H.vanilla_offsets(o["chunks"], sum(o["chunks"])) == o["expected"]
    r = kat["ring_sources"]
    for tgt, srcs in r["expected"].items():
        assert H.ring_sources(int(tgt), r["num_domains"]) == srcs


def test_strategy_known_answers_oracle_and_library():
    # strategy.rs:157-201 asserted by the reference; the oracle's procedure and the
    # library's closed forms (host helpers, no GPU) must both reproduce them.
    from oracle import strategy as SP
    with open(os.path.join(GOLD, "reference_kats.json")) as f:
        kat = json.load(f)
    for case in kat["strategies"]:
        chunks, strat = case["chunks"], case["strategy"]
        a = SP.build_assignment(chunks, strat)
        if "assignment" in case:
            assert a == case["assignment"] and H.build_assignment(chunks, strat) == case["assignment"]
        if "positions" in case:
            assert SP.build_domain_positions(a) == case["positions"]
            assert H.domain_positions(chunks, strat) == sum(case["positions"], [])
        if "inverse_perm" in case:
            assert SP.build_inverse_perm(a) == case["inverse_perm"]
            assert H.inverse_perm(chunks, strat) == case["inverse_perm"]


# ------------------------------------------------------------------------ GPU ----
def dev(bits, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("name", BLOCK_FIXTURES)
def test_gpu_block_partial_on_fixture(gpu, name):
    g = load(name)
    q, k, v = (dev(g[n]).permute(1, 0, 2) for n in ("q_bits", "k_bits", "v_bits"))
    o, lse = H.block_partial(q, k, v, int(g["q_offset"]), int(g["kv_offset"]), causal=bool(g["causal"]),
                             scale=float(g["scale"]))
    torch.cuda.synchronize()
    o, lse = o.cpu().numpy().transpose(1, 0, 2), lse.cpu().numpy().T
    assert np.array_equal(np.isneginf(lse), np.isneginf(g["lse"]))
    fin = np.isfinite(g["lse"])
    assert np.abs(o - g["o"]).max() <= 2e-2
    assert np.abs(lse[fin] - g["lse"][fin]).max() <= 1e-3
    assert (o[~fin] == 0).all()


@pytest.mark.gpu
def test_gpu_ring_replay_fp32_on_fixture(gpu):
    g = load("ring_fp32_two_domains.npz")
    q, k, v = (torch.from_numpy(g[n]).cuda().permute(1, 0, 2) for n in ("q", "k", "v"))
    out, lse = H.ring_attention_replay(q, k, v, [int(c) for c in g["chunks"]])
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy().transpose(1, 0, 2) - g["o"]).max() <= 1e-4
    assert np.abs(lse.cpu().numpy().T - g["lse"]).max() <= 1e-4


@pytest.mark.gpu
def test_gpu_lse_merge_on_fixture(gpu):
    g = load("merge_three_parts.npz")
    parts = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in g["o_parts"]]
    lses = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in g["lse_parts"]]
    out, lse = H.lse_merge(parts, lses, out_dtype=torch.float32)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    assert np.array_equal(np.isneginf(lse), np.isneginf(g["lse"]))
    fin = np.isfinite(g["lse"])
    assert np.abs(lse[fin] - g["lse"][fin]).max() <= 1e-5
    assert np.abs(out - g["o"]).max() <= 1e-5
    assert (out[~fin] == 0).all()


@pytest.mark.gpu
def test_gpu_paged_gather_scatter_on_fixture(gpu):
    g = load("paged_bf16_ragged.npz")
    pool = dev(g["pool_bits"])
    table = torch.from_numpy(g["table"]).cuda()
    k, v = H.paged_kv_gather(pool, table, 0, int(g["t0"]), int(g["t1"]))
    torch.cuda.synchronize()
    assert np.array_equal(k.cpu().view(torch.int16).numpy().view(np.uint16), g["k_bits"])
    assert np.array_equal(v.cpu().view(torch.int16).numpy().view(np.uint16), g["v_bits"])
    scat = torch.full(pool.shape, 0x7fc1, dtype=torch.int16).view(torch.bfloat16).cuda()
    H.paged_kv_scatter(scat, torch.from_numpy(g["scatter_table"]).cuda(), 0, 0, 40,
                       dev(g["scatter_k_bits"]), dev(g["scatter_v_bits"]), zero_tail=True)
    torch.cuda.synchronize()
    assert np.array_equal(scat.cpu().view(torch.int16).numpy().view(np.uint16), g["scatter_pool_bits"])


@pytest.mark.gpu
def test_gpu_paged_decode_on_fixture(gpu):
    g = load("decode_bf16_small.npz")
    q, pool = dev(g["q_bits"]), dev(g["pool_bits"])
    tables = torch.from_numpy(g["tables"]).cuda()
    o, lse = H.decode_local_compact_partial(q, pool, tables, int(g["t0"]), int(g["t1"]))
    torch.cuda.synchronize()
    assert np.abs(o.cpu().numpy() - g["o"]).max() <= 2e-2
    assert np.abs(lse.cpu().numpy() - g["lse"]).max() <= 1e-3


def _wire_cases():
    with open(os.path.join(GOLD, "wire_frames.json")) as f:
        return json.load(f)


def test_wire_frame_oracle_round_trip():
    # The oracle's parser recovers what the reference's tests assert after a TCP
    # round trip (layer, range, positions, tensors), from the stored frames.
    from oracle import wire as W
    for c in _wire_cases():
        if c["kind"] != "kv_block":
            continue
        meta, k, v, pos = W.parse_kv_block_frame(bytes.fromhex(c["frame_hex"]))
        assert (meta["layer_idx"], meta["global_seq_start"], meta["global_seq_end"]) == (c["layer_idx"], c["start"],
                                                                                         c["end"])
        assert (pos is None and c["positions"] is None) or pos.tolist() == c["positions"]
        if "k" in c:
            assert k.tolist() == c["k"] and v.tolist() == c["v"]


def test_wire_headers_match_reference_frames():
    # The library's host-side header writer is byte-identical to the restated
    # serde_json output of serialize_block_to_buffer / serialize_packet_to_buffer.
    for c in _wire_cases():
        frame = bytes.fromhex(c["frame_hex"])
        n = 4 + int.from_bytes(frame[:4], "big")
        if c["kind"] == "ring_packet":
            q = np.array(c["q"])
            desc = H.PacketFrameDesc(c["layer_idx"], H.DTYPE_BF16, H.DTYPE_BF16, q.shape[0], q.shape[1], q.shape[3], 0,
                                     c["scale"])
            assert H._header("hcp_packet_frame_header", desc) == frame[:n]
            d, hb = H.packet_frame_parse(frame)
            assert hb == n and (d.batch, d.num_heads, d.head_dim, d.layer_idx) == (1, 2, 8, 4)
            assert d.scale == c["scale"] and d.q_dtype == H.DTYPE_BF16
            continue
        d, hb = H.kv_frame_parse(frame)
        assert hb == n
        assert (d.layer_idx, d.global_seq_start, d.global_seq_end) == (c["layer_idx"], c["start"], c["end"])
        assert d.has_positions == (c["positions"] is not None)
        if c["name"].startswith("legacy"):
            continue  # written by the reference's old serializer only
        assert H.kv_frame_header(d) == frame[:n]


def test_wire_parse_rejects_inconsistent_headers():
    c = _wire_cases()[0]
    frame = bytearray(bytes.fromhex(c["frame_hex"]))
    bad = bytes(frame).replace(b'"k_bytes":16', b'"k_bytes":17')
    with pytest.raises(H.HcpRingError):
        H.kv_frame_parse(bad)
    with pytest.raises(H.HcpRingError):
        H.kv_frame_parse(bytes(frame[:10]))


@pytest.mark.parametrize("scale", [0.125, 1.0, 100.0, 1e-5, 1.5e-7, 1e16, 1e17, 123456.789, 0.08838834764831845,
                                   2.0 ** -20, 0.0001, 3.0e-5])
def test_packet_header_float_format(scale):
    # serde_json writes f64 through ryu: the library's writer (std::to_chars digits) and
    # the oracle's (Python repr digits) must agree on every notation branch.
    from oracle import wire as W
    q = np.zeros((1, 2, 1, 4), dtype=np.float32)
    ref = W.ring_packet_frame(0, q, q, np.zeros((1, 2, 1), np.float32), scale, "float32", "float32")
    desc = H.PacketFrameDesc(0, H.DTYPE_F32, H.DTYPE_F32, 1, 2, 4, 0, scale)
    hdr = H._header("hcp_packet_frame_header", desc)
    assert hdr == ref[:len(hdr)]


def test_ryu_notation_examples():
    from oracle import wire as W
    cases = {1.0: "1.0", 100.0: "100.0", 1e16: "1e16", 1.5e-7: "1.5e-7", 1e-5: "0.00001", 0.1: "0.1",
             123456.0: "123456.0", 1e15: "1000000000000000.0", 1.2345e30: "1.2345e30", -2.5: "-2.5"}
    for x, s in cases.items():
        assert W.ryu_f64(x) == s, x
