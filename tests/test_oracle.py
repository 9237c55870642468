"""CPU tests that pin the oracle before it is trusted (no GPU).

Each check ties an oracle function to something it does not restate: the reference's
own test assertions (ring.rs / strategy.rs / cache.rs), closed forms, invariants, or
brute force on tiny inputs.  Planted-mistake tests show the checks would catch a
dropped term, an off-by-one mask or a wrong head map.
"""
import math

import numpy as np
import pytest
import torch

from oracle import clib, closed_form as C, inputs as I, tch_ring as T


def _bhsd(x):
    """[S, H, D] numpy -> [1, H, S, D] torch (the reference's layout)."""
    return torch.from_numpy(np.ascontiguousarray(x)).permute(1, 0, 2).unsqueeze(0)


# ------------------------------------------------------------------ generator ----
def test_lcg_jump_ahead_matches_recurrence():
    for seed in (0, 42, 46, 2**63 + 5):
        vec = [int(x) for x in I.lcg_states(seed, 70_000)]
        assert vec == I.lcg_scalar_states(seed, 70_000)


def test_lcg_known_answer():
    # reference_algo.rs:66-74, first draw of seed 42, computed with exact integers.
    s1 = (42 * 6364136223846793005 + 1442695040888963407) % 2**64
    u1 = ((s1 >> 11) + 0.5) / 2**53
    assert int(I.lcg_states(42, 1)[0]) == s1
    assert clib.draw_uniforms(42, 1)[0] == u1


def test_c_generator_matches_numpy_stream_with_spare():
    # Odd counts cross the Box-Muller spare (reference_algo.rs:79-89).
    ns = I.NormalStream(44)
    parts = [ns.draw(n) for n in (7, 1, 1000, 3)]
    a = np.concatenate(parts)
    b, = clib.draw_normals(44, [(a.size,)], "f64")
    np.testing.assert_allclose(a, b, rtol=1e-13, atol=1e-13)
    # same stream split across tensors
    x, y = clib.draw_normals(44, [(7,), (1004,)], "f64")
    np.testing.assert_array_equal(np.concatenate([x, y]), b)


def test_normals_are_standard():
    x, = clib.draw_normals(7, [(1_000_000,)], "f64")
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1.0) < 5e-3


def test_bf16_rounding_is_nearest_even():
    vals = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.5, 3.0e38, 1e-40], dtype=np.float32)
    bits = I.f32_to_bf16_bits(vals)
    assert bits[0] == 0x3F80 and bits[1] == 0x3F80 and bits[2] == 0x3F82
    r = np.random.default_rng(0).standard_normal(200_000).astype(np.float32) * 10
    ref = torch.from_numpy(r).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(I.f32_to_bf16_bits(r), ref)
    c_bits, = clib.draw_normals(43, [(4096,)], "bf16")
    f32, = clib.draw_normals(43, [(4096,)], "fp32")
    np.testing.assert_array_equal(c_bits, I.f32_to_bf16_bits(f32))


def test_c5_chunk_draw():
    ch = I.c5_chunks()
    assert ch == [21504, 13312, 18432, 23552, 24576, 9216, 8192, 12288]
    assert sum(ch) == 131072 and all(c % 1024 == 0 and c >= 8192 for c in ch)


def test_block_table_is_seeded_permutation():
    p = I.permuted_block_table(45, 4096)
    assert sorted(p.tolist()) == list(range(4096))
    np.testing.assert_array_equal(p, I.permuted_block_table(45, 4096))
    assert not np.array_equal(p, np.arange(4096))


def test_config_flop_counts_match_baseline():
    cases = {c.name: c for c in I.config_cases()}
    assert math.isclose(cases["c1_cpu_smoke"].causal_flops(), 1.0748e9, rel_tol=1e-4)
    assert math.isclose(cases["c2_qwen25_3b"].causal_flops(), 2.7491e11, rel_tol=1e-4)
    assert math.isclose(cases["c3_llama3_8b"].causal_flops(), 8.7964e12, rel_tol=1e-4)
    assert math.isclose(cases["c5_staged_128k"].causal_flops(), 1.4074e14, rel_tol=1e-4)
    assert C.ring_pairs([12288, 8192, 8192, 4096]) == [
        (0, 0), (1, 1), (1, 0), (2, 2), (2, 1), (2, 0), (3, 3), (3, 2), (3, 1), (3, 0)]


# ------------------------------------------------------------------ closed form ----
def _rand(seed, shape):
    return np.random.default_rng(seed).standard_normal(shape)


def test_closed_form_brute_force_tiny():
    q, k, v = _rand(1, (5, 2, 3)), _rand(2, (5, 1, 3)), _rand(3, (5, 1, 3))
    pos = np.arange(5)
    o, lse = C.attention_f64(q, k, v, pos, pos, 0.7)
    for i in range(5):
        for h in range(2):
            s = [0.7 * float(np.dot(q[i, h], k[j, 0])) for j in range(i + 1)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            assert abs(lse[i, h] - (m + math.log(sum(w)))) < 1e-12
            ref = sum(w[j] * v[j, 0] for j in range(i + 1)) / sum(w)
            np.testing.assert_allclose(o[i, h], ref, atol=1e-12)


def test_closed_form_no_visible_key_is_zero_and_neg_inf():
    q, k, v = _rand(1, (3, 1, 4)), _rand(2, (4, 1, 4)), _rand(3, (4, 1, 4))
    o, lse = C.attention_f64(q, k, v, np.arange(3), np.arange(10, 14), 0.5)
    assert np.all(lse == -np.inf) and np.all(o == 0)


def test_merge_of_partition_equals_full_attention():
    q, k, v = _rand(4, (6, 4, 8)), _rand(5, (20, 2, 8)), _rand(6, (20, 2, 8))
    qp, kp = np.arange(14, 20), np.arange(20)
    full_o, full_l = C.attention_f64(q, k, v, qp, kp, 0.3)
    cuts = [0, 3, 9, 17, 20]
    parts = [C.attention_f64(q, k[a:b], v[a:b], qp, kp[a:b], 0.3) for a, b in zip(cuts, cuts[1:])]
    for order in ([0, 1, 2, 3], [3, 1, 0, 2]):
        o, l = C.merge_partials_f64([parts[i][0] for i in order], [parts[i][1] for i in order])
        np.testing.assert_allclose(o, full_o, atol=1e-12)
        np.testing.assert_allclose(l, full_l, atol=1e-12)
    # a fully-future partial is neutral
    o, l = C.merge_partials_f64([parts[0][0], np.zeros_like(parts[0][0])],
                                [parts[0][1], np.full_like(parts[0][1], -np.inf)])
    np.testing.assert_allclose(o, parts[0][0], atol=1e-15)


@pytest.mark.parametrize("mistake", ["swapped_weights", "lse_without_max", "unnormalised"])
def test_planted_merge_mistakes_are_caught(mistake):
    """A merge with a planted mistake no longer reproduces full attention from a partition."""
    q, k, v = _rand(7, (6, 2, 8)), _rand(8, (20, 2, 8)), _rand(9, (20, 2, 8))
    qp, kp = np.arange(14, 20), np.arange(20)
    full_o, full_l = C.attention_f64(q, k, v, qp, kp, 0.3)
    (o1, l1), (o2, l2) = (C.attention_f64(q, k[a:b], v[a:b], qp, kp[a:b], 0.3) for a, b in ((0, 7), (7, 20)))
    m = np.maximum(l1, l2)
    w1, w2 = np.exp(l1 - m), np.exp(l2 - m)
    if mistake == "swapped_weights":
        w1, w2 = w2, w1
    o = (w1[..., None] * o1 + w2[..., None] * o2)
    if mistake != "unnormalised":
        o = o / (w1 + w2)[..., None]
    lse = np.log(w1 + w2) + (0.0 if mistake == "lse_without_max" else m)
    err = max(np.abs(o - full_o).max(), np.abs(lse - full_l).max())
    assert err > 1e-3, f"planted {mistake} not detected (err={err})"


# ------------------------------------------------------------------ tch restatement ----
def test_single_block_fold_equals_softmax():
    # ring.rs:2150-2226: one non-causal fold from rm=-inf equals softmax(QK^T)V.
    torch.manual_seed(42)
    q, k, v = torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8)
    scale = 1 / math.sqrt(8)
    rm = torch.full((1, 2, 4), float("-inf"))
    rs = torch.zeros(1, 2, 4)
    obh = torch.zeros(1, 2, 4, 8)
    pos = torch.arange(4)
    _, _, out = T.process_kv_block(scale, q, pos, k, v, pos, rm, rs, obh, False)
    ref = torch.softmax(q @ k.transpose(2, 3) * scale, -1) @ v
    assert (ref - out).abs().mean() < 1e-4


def test_ring_causal_matches_closed_form_small():
    # ring.rs:2591-2652 (4 domains, S=16, causal) against f64 closed form.
    q, k, v = _rand(7, (16, 4, 8)), _rand(8, (16, 4, 8)), _rand(9, (16, 4, 8))
    f = lambda x: _bhsd(x.astype(np.float32))
    out = T.ring_attention_replay(1 / math.sqrt(8), f(q), f(k), f(v), [4, 4, 4, 4])
    ref, _ = C.attention_f64(q, k, v, np.arange(16), np.arange(16), 1 / math.sqrt(8))
    assert np.abs(out[0].permute(1, 0, 2).numpy() - ref).max() < 1e-5


def test_c1_ring_replay_strict_tier():
    # The CPU smoke config c1 against the closed form at the Strict tier (error.rs:56-76).
    case = I.config_cases()[0]
    q, k, v = I.make_qkv(case)
    out, lse = T.ring_attention_replay(case.scale, _bhsd(q), _bhsd(k), _bhsd(v), case.chunks,
                                       return_lse=True)
    pos = np.arange(case.seq_len)
    ref_o, ref_l = C.attention_f64(q, k, v, pos, pos, case.scale)
    err = np.abs(out[0].permute(1, 0, 2).numpy() - ref_o)
    assert err.max() <= 1e-5 and err.mean() <= 1e-6
    assert np.abs(lse[0].permute(1, 0).numpy() - ref_l).max() <= 1e-5


def test_positioned_accumulator_strided_shards_any_starter():
    # ring.rs:2381-2521: 3 domains holding strided KV shards; (o, lse) equal the
    # closed form for every starter, to 1e-5.
    hq, d, total, ql = 2, 4, 24, 3
    q, k, v = _rand(10, (ql, hq, d)), _rand(11, (total, hq, d)), _rand(12, (total, hq, d))
    qp = np.arange(total - ql, total)
    ref_o, ref_l = C.attention_f64(q, k, v, qp, np.arange(total), 0.5)
    f = lambda x: _bhsd(x.astype(np.float32))
    shards = [np.arange(dom, total, 3) for dom in range(3)]
    for starter in range(3):
        sh = shards[starter]
        o, l = T.positioned_local_compact_partial(0.5, f(q), torch.from_numpy(qp), f(k[sh]), f(v[sh]),
                                                  torch.from_numpy(sh))
        for hop in range(1, 3):
            sh = shards[(starter + hop) % 3]
            o, l = T.positioned_merge_compact_partial(0.5, f(q), torch.from_numpy(qp), o, l, f(k[sh]),
                                                      f(v[sh]), torch.from_numpy(sh))
        assert np.abs(o[0].permute(1, 0, 2).numpy() - ref_o).max() < 1e-5
        assert np.abs(l[0].permute(1, 0).numpy() - ref_l).max() < 1e-5


def test_decode_partial_merge_matches_closed_form():
    # ring.rs:625-663: decode partial over one segment, merge with the others.
    q, k, v = _rand(13, (1, 8, 16)), _rand(14, (40, 2, 16)), _rand(15, (40, 2, 16))
    ref_o, ref_l = C.attention_f64(q, k, v, np.array([0]), np.arange(40), 0.25, causal=False)
    f = lambda x: _bhsd(x.astype(np.float32))
    o, l = T.decode_local_compact_partial(0.25, f(q), f(k[:17]), f(v[:17]))
    o, l = T.decode_merge_compact_partial(0.25, f(q), o, l, f(k[17:31]), f(v[17:31]))
    o, l = T.decode_merge_compact_partial(0.25, f(q), o, l, f(k[31:]), f(v[31:]))
    assert np.abs(o[0, :, 0].numpy() - ref_o[0]).max() < 1e-5
    assert np.abs(l[0, :, 0].numpy() - ref_l[0]).max() < 1e-5


def _growth_shards(k, v, chunks, upto, n):
    """Durable segments after growth sharding: prefill chunk of each domain plus the
    decode tokens it owns (position p kept by domain p mod N, ring.rs:1930-1936)."""
    f = lambda x: _bhsd(x.astype(np.float32))
    prefill = chunks[-1][1]
    out = []
    for d, (a, b) in enumerate(chunks):
        idx = list(range(a, b)) + [p for p in range(prefill, upto) if p % n == d]
        out.append((f(k[idx]), f(v[idx])))
    return out


@pytest.mark.parametrize("double_count", [False, True])
def test_decode_q_ring_growth_sharding_matches_closed_form(double_count):
    # The reference's own decode Q-ring check (ring.rs:3400-3560): three domains with
    # uneven prefill chunks [0,3) [3,5) [5,7), growth-sharded decode steps, every node's
    # final packet equals full-KV attention.  The planted mistake merges the current
    # token again in Phase 2 (k instead of k_peer) and must be rejected.
    n, chunks, steps = 3, [(0, 3), (3, 5), (5, 7)], 4
    total = chunks[-1][1] + steps
    k, v = _rand(30, (total, 2, 16)), _rand(31, (total, 2, 16))
    qs = _rand(32, (steps, 1, 4, 16))
    f = lambda x: _bhsd(x.astype(np.float32))
    for t in range(steps):
        pos = chunks[-1][1] + t
        ref_o, ref_l = C.attention_f64(qs[t], k[:pos + 1], v[:pos + 1], np.array([0]), np.arange(pos + 1), 0.25,
                                       causal=False)
        durable = _growth_shards(k, v, chunks, pos, n)
        if double_count:
            durable = [(torch.cat([a, f(k[pos:pos + 1])], 2), torch.cat([b, f(v[pos:pos + 1])], 2))
                       for a, b in durable]
        for seed in range(n):
            o, l = T.ring_decode_attention(0.25, f(qs[t]), durable, f(k[pos:pos + 1]), f(v[pos:pos + 1]), seed)
            err = np.abs(o[0, :, 0].numpy() - ref_o[0]).max()
            if double_count:
                assert err > 1e-3, f"double-counted current token not detected (err={err})"
            else:
                assert err < 1e-5
                assert np.abs(l[0, :, 0].numpy() - ref_l[0]).max() < 1e-5


def test_decode_q_ring_empty_durable_segment_passes_packet():
    # A domain that owns nothing yet (N > prefill chunks' owners) leaves the packet as is.
    k, v, q = _rand(33, (5, 1, 8)), _rand(34, (5, 1, 8)), _rand(35, (1, 2, 8))
    f = lambda x: _bhsd(x.astype(np.float32))
    durable = [(f(k[:4]), f(v[:4])), (f(k[:0]), f(v[:0]))]
    ref_o, _ = C.attention_f64(q, k, v, np.array([0]), np.arange(5), 0.3, causal=False)
    for seed in (0, 1):
        o, _ = T.ring_decode_attention(0.3, f(q), durable, f(k[4:]), f(v[4:]), seed)
        assert np.abs(o[0, :, 0].numpy() - ref_o[0]).max() < 1e-5


def test_fully_future_source_gives_zero_and_neg_inf():
    q, k, v = (torch.randn(1, 2, 3, 4) for _ in range(3))
    o, l = T.positioned_local_compact_partial(0.5, q, torch.arange(3), k, v, torch.arange(5, 8))
    assert torch.all(o == 0) and torch.all(l == float("-inf"))


def test_single_local_token_stays_causal_with_future_peer_kv():
    # worker_sdk/tch_backend.rs:1809-1905: one local query must ignore later peer keys.
    q, k, v = _rand(16, (1, 2, 8)), _rand(17, (6, 2, 8)), _rand(18, (6, 2, 8))
    f = lambda x: _bhsd(x.astype(np.float32))
    o, l = T.positioned_local_compact_partial(0.35, f(q), torch.tensor([2]), f(k), f(v), torch.arange(6))
    ref_o, ref_l = C.attention_f64(q, k[:3], v[:3], np.array([2]), np.arange(3), 0.35)
    assert np.abs(o[0, :, 0].numpy() - ref_o[0]).max() < 1e-5


def test_bf16_state_lse_is_coarser_than_fp32_upcast():
    # The reference keeps rm/rs in the query dtype (ring.rs:553-555): its bf16 LSE is
    # quantised; the 1e-3 LSE criterion is therefore judged on fp32 upcasts.
    case = I.RingCase("tiny_bf16", [96, 64], 4, 2, 64, "bf16", 99)
    q, k, v = I.make_qkv(case)
    qb, kb, vb = (_bhsd(I.to_f32(x)).to(torch.bfloat16) for x in (q, k, v))
    q32, k32, v32 = (_bhsd(I.to_f32(x)) for x in (q, k, v))
    ob, lb = T.ring_attention_replay(case.scale, qb, kb, vb, case.chunks, return_lse=True)
    o32, l32 = T.ring_attention_replay(case.scale, q32, k32, v32, case.chunks, return_lse=True)
    pos = np.arange(case.seq_len)
    ref_o, ref_l = C.attention_f64(I.to_f32(q), I.to_f32(k), I.to_f32(v), pos, pos, case.scale)
    assert np.abs(l32[0].permute(1, 0).numpy() - ref_l).max() < 1e-5
    assert np.abs(lb[0].permute(1, 0).numpy() - ref_l).max() > 1e-3
    assert np.abs(ob[0].float().permute(1, 0, 2).numpy() - ref_o).max() < 2e-2


@pytest.mark.parametrize("mistake", ["off_by_one_mask", "dropped_rescale", "wrong_head_map"])
def test_planted_mistakes_are_caught(mistake):
    """Plant a mistake in a copy of the oracle's fold; the closed form must reject it."""
    q, k, v = _rand(20, (12, 4, 8)), _rand(21, (12, 2, 8)), _rand(22, (12, 2, 8))
    pos = np.arange(12)
    ref_o, _ = C.attention_f64(q, k, v, pos, pos, 0.4)
    f = lambda x: _bhsd(x.astype(np.float32))
    kx, vx = T.repeat_kv_heads(f(k), 2), T.repeat_kv_heads(f(v), 2)
    if mistake == "wrong_head_map":  # kv head = h % Hkv instead of h // rep
        kx, vx = f(k).repeat(1, 2, 1, 1), f(v).repeat(1, 2, 1, 1)
    qp = torch.arange(12)
    kp = qp + 1 if mistake == "off_by_one_mask" else qp
    rm, rs, obh = torch.full((1, 4, 12), -1e4), torch.zeros(1, 4, 12), torch.zeros(1, 4, 12, 8)
    for a, b in [(0, 5), (5, 12)]:
        if mistake == "dropped_rescale" and a == 5:
            rm = torch.full_like(rm, -1e4)  # forget the running max between blocks
            rs = torch.zeros_like(rs)
        rm, rs, obh = T.process_kv_block(0.4, f(q), qp, kx[:, :, a:b], vx[:, :, a:b], kp[a:b], rm, rs, obh, True)
    err = np.abs(obh[0].permute(1, 0, 2).numpy() - ref_o).max()
    assert err > 1e-2, f"planted {mistake} not detected (err={err})"


# ------------------------------------------------------------------ strategies ----
STRATEGY_CHUNKS = [[3, 1], [4, 4], [5, 3, 2], [7, 1, 4, 2], [1, 9], [2, 2, 2, 2, 3], [6, 0, 3]]


@pytest.mark.parametrize("chunks", STRATEGY_CHUNKS)
@pytest.mark.parametrize("strategy", ["vanilla", "striped", "zigzag"])
def test_strategy_assignment_invariants(chunks, strategy):
    # build_assignment's contract (strategy.rs:49-52): domain i owns exactly chunks[i]
    # positions; the positions partition [0, S); the inverse permutation inverts the
    # domain-major concatenation.
    from oracle import strategy as SP
    a = SP.build_assignment(chunks, strategy)
    assert len(a) == sum(chunks)
    assert [a.count(d) for d in range(len(chunks))] == chunks
    pos = SP.build_domain_positions(a)
    flat = sum(pos, [])
    assert sorted(flat) == list(range(sum(chunks)))
    assert all(p == sorted(p) for p in pos)
    inv = SP.build_inverse_perm(a)
    assert [flat[inv[p]] for p in range(len(a))] == list(range(len(a)))


def test_zigzag_classic_and_striped_round_robin():
    # Equal chunks: ZigZag is the classic 2N-segment layout, Striped is p mod N.
    from oracle import strategy as SP
    n, c = 4, 6
    a = SP.build_assignment([c] * n, "zigzag")
    seg = c // 2
    assert a == sum([[d] * seg for d in range(n)] + [[d] * seg for d in reversed(range(n))], [])
    assert SP.build_assignment([c] * n, "striped") == [p % n for p in range(n * c)]


@pytest.mark.parametrize("strategy", ["striped", "zigzag"])
@pytest.mark.parametrize("chunks", [[48, 16], [30, 20, 14]])
def test_strategy_ring_matches_closed_form(strategy, chunks):
    # run_uneven_ring_attention (ring.rs:3226-3364) at a small size: every strategy's
    # ring, put back in global order, is full causal attention.
    s = sum(chunks)
    q, k, v = _rand(40, (s, 4, 16)), _rand(41, (s, 2, 16)), _rand(42, (s, 2, 16))
    pos = np.arange(s)
    ref_o, ref_l = C.attention_f64(q, k, v, pos, pos, 0.25)
    f = lambda x: _bhsd(x.astype(np.float32))
    o, l = T.ring_attention_replay_strategy(0.25, f(q), f(k), f(v), chunks, strategy, return_lse=True)
    assert np.abs(o[0].permute(1, 0, 2).numpy() - ref_o).max() < 1e-5
    assert np.abs(l[0].permute(1, 0).numpy() - ref_l).max() < 1e-5


def test_strategy_ring_with_contiguous_positions_is_caught():
    # Planted mistake: feed the striped layout but let every block claim contiguous
    # positions (drop the position_ids) -- the closed form must reject it.
    from oracle import strategy as SP
    chunks = [48, 16]
    s = sum(chunks)
    q, k, v = _rand(43, (s, 2, 16)), _rand(44, (s, 2, 16)), _rand(45, (s, 2, 16))
    pos = np.arange(s)
    ref_o, _ = C.attention_f64(q, k, v, pos, pos, 0.25)
    f = lambda x: _bhsd(x.astype(np.float32))
    a = SP.build_assignment(chunks, "striped")
    perm = torch.tensor(sum(SP.build_domain_positions(a), []))
    inv = torch.tensor(SP.build_inverse_perm(a))
    # the vanilla driver on permuted inputs = contiguous positions on striped data
    o = T.ring_attention_replay(0.25, f(q).index_select(2, perm), f(k).index_select(2, perm),
                                f(v).index_select(2, perm), chunks).index_select(2, inv)
    err = np.abs(o[0].permute(1, 0, 2).numpy() - ref_o).max()
    assert err > 1e-2, f"contiguous positions on a striped layout not detected (err={err})"


# ------------------------------------------------------------------ paged KV ----
def test_paged_gather_index_math_known_answer():
    # python/hcp_vllm_block_ring_plugin.py:322-327: block (t - off)//bs, slot (t - off)%bs.
    nb, bs, hkv, d = 6, 4, 2, 3
    pool = np.arange(2 * nb * bs * hkv * d, dtype=np.float32).reshape(2, nb, bs, hkv, d)
    table = np.array([3, 0, 5, 1], dtype=np.int32)
    k, v = clib.paged_gather(pool, table, 8, 9, 15)
    for t in range(9, 15):
        rel = t - 8
        blk, slot = table[rel // bs], rel % bs
        for h in range(hkv):
            np.testing.assert_array_equal(k[h, t - 9], pool[0, blk, slot, h])
            np.testing.assert_array_equal(v[h, t - 9], pool[1, blk, slot, h])


def test_paged_scatter_gather_round_trip_and_tail_zero():
    rng = np.random.default_rng(3)
    nb, bs, hkv, d = 32, 16, 8, 128
    pool = rng.integers(1, 2**16, size=(2, nb, bs, hkv, d), dtype=np.uint16)
    table = I.permuted_block_table(5, nb)[:10]
    k = rng.integers(0, 2**16, size=(hkv, 150, d), dtype=np.uint16)
    v = rng.integers(0, 2**16, size=(hkv, 150, d), dtype=np.uint16)
    before = pool.copy()
    clib.paged_scatter(pool, table, 0, 0, 150, k, v, zero_tail=True)
    k2, v2 = clib.paged_gather(pool, table, 0, 0, 150)
    np.testing.assert_array_equal(k2, k)
    np.testing.assert_array_equal(v2, v)
    last = table[149 // bs]
    assert np.all(pool[:, last, 150 % bs:] == 0)
    untouched = np.setdiff1d(np.arange(nb), table)
    np.testing.assert_array_equal(pool[:, untouched], before[:, untouched])


def test_paged_oracle_rejects_bad_block_ids():
    pool = np.zeros((2, 4, 16, 1, 8), dtype=np.uint16)
    with pytest.raises(ValueError):
        clib.paged_gather(pool, np.array([0, 9], dtype=np.int32), 0, 0, 32)


def test_block_table_matches_contiguous():
    # cache.rs:447-503: a block table over logical 16-token blocks returns the same K/V
    # as the contiguous cache.
    rng = np.random.default_rng(8)
    kv = rng.standard_normal((2, 77, 2, 16)).astype(np.float32)  # [K/V, S, H, D]
    nb, bs = 12, 16
    table = I.permuted_block_table(9, nb)[:5]
    pool = np.zeros((2, nb, bs, 2, 16), dtype=np.float32)
    clib.paged_scatter(pool, table, 0, 0, 77, kv[0].transpose(1, 0, 2), kv[1].transpose(1, 0, 2))
    k, v = clib.paged_gather(pool, table, 0, 0, 77)
    np.testing.assert_array_equal(k, kv[0].transpose(1, 0, 2))
    np.testing.assert_array_equal(v, kv[1].transpose(1, 0, 2))


# ------------------------------------------------------------------ QKV + RoPE ----
def _rope_f64(x, pos, dim, base):
    """Closed form: pair (d, d + D/2) rotated by pos * base^(-2d/D), all in f64."""
    half = dim // 2
    inv = 1.0 / base ** (2.0 * np.arange(half) / dim)
    ang = pos[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def test_rope_oracle_matches_closed_form_and_invariants():
    dim, base = 64, 10000.0
    cos, sin = T.rope_caches(dim, 256, base)
    pos = np.array([0, 1, 7, 100, 255])
    q = _rand(50, (1, 2, 5, dim)).astype(np.float32)
    k = _rand(51, (1, 1, 5, dim)).astype(np.float32)
    rq, rk = T.rope_apply(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(pos)[None], cos, sin)
    assert np.abs(rq.numpy() - _rope_f64(q.astype(np.float64), pos.astype(np.float64), dim, base)).max() < 1e-4
    # position 0 is the identity; every (d, d + D/2) pair keeps its norm
    assert np.array_equal(rq.numpy()[:, :, 0], q[:, :, 0])
    h = dim // 2
    n0 = q[..., :h] ** 2 + q[..., h:] ** 2
    n1 = rq.numpy()[..., :h] ** 2 + rq.numpy()[..., h:] ** 2
    assert np.abs(n0 - n1).max() < 1e-4


def test_rope_scores_depend_on_relative_position_only():
    dim = 128
    cos, sin = T.rope_caches(dim, 512, 10000.0)
    q = torch.from_numpy(_rand(52, (1, 1, 1, dim)).astype(np.float32))
    k = torch.from_numpy(_rand(53, (1, 1, 1, dim)).astype(np.float32))
    def score(m, n):
        rq, _ = T.rope_apply(q, q, torch.tensor([[m]]), cos, sin)
        rk, _ = T.rope_apply(k, k, torch.tensor([[n]]), cos, sin)
        return float((rq * rk).sum())
    assert abs(score(40, 10) - score(130, 100)) < 1e-3
    assert abs(score(40, 10) - score(40, 11)) > 1e-3


def test_rope_interleaved_pairing_is_caught():
    # Planted mistake: rotate adjacent pairs (2i, 2i+1) instead of the halves.
    dim = 32
    x = _rand(54, (1, 1, 3, dim))
    pos = np.array([3.0, 9.0, 20.0])
    good = _rope_f64(x, pos, dim, 10000.0)
    inv = 1.0 / 10000.0 ** (2.0 * np.arange(dim // 2) / dim)
    ang = pos[:, None] * inv[None]
    xe, xo = x[..., 0::2], x[..., 1::2]
    bad = np.empty_like(x)
    bad[..., 0::2] = xe * np.cos(ang) - xo * np.sin(ang)
    bad[..., 1::2] = xe * np.sin(ang) + xo * np.cos(ang)
    assert np.abs(good - bad).max() > 1e-2


def test_qkv_forward_oracle_matches_closed_form():
    l, hidden, hq, hkv, d = 5, 48, 4, 2, 16
    x = _rand(55, (1, l, hidden))
    wq, wk, wv = _rand(56, (hq * d, hidden)), _rand(57, (hkv * d, hidden)), _rand(58, (hkv * d, hidden))
    bq, bk, bv = _rand(59, (hq * d,)), _rand(60, (hkv * d,)), _rand(61, (hkv * d,))
    pos = np.array([4, 9, 10, 33, 60])
    cos, sin = T.rope_caches(d, 64, 10000.0)
    f = lambda a: torch.from_numpy(a.astype(np.float32))
    q, k, v = T.qkv_rope_forward(f(x), f(wq), f(wk), f(wv), f(bq), f(bk), f(bv), hq, hkv, d,
                                 torch.from_numpy(pos)[None], cos, sin)
    rq = (x[0] @ wq.T + bq).reshape(l, hq, d).transpose(1, 0, 2)
    rk = (x[0] @ wk.T + bk).reshape(l, hkv, d).transpose(1, 0, 2)
    rv = (x[0] @ wv.T + bv).reshape(l, hkv, d).transpose(1, 0, 2)
    assert np.abs(q[0].numpy() - _rope_f64(rq, pos.astype(np.float64), d, 10000.0)).max() < 1e-3
    assert np.abs(k[0].numpy() - _rope_f64(rk, pos.astype(np.float64), d, 10000.0)).max() < 1e-3
    assert np.abs(v[0].numpy() - rv).max() < 1e-4


def test_agent_metadata_bincode_known_answers():
    # Byte strings written from bincode 1.3's published default encoding (little-endian,
    # u64 length prefixes, u32 variant index), independent of the oracle's code.
    from oracle import wire as W
    assert W.agent_metadata_bincode("a", []) == bytes.fromhex("0100000000000000" "61" "0000000000000000")
    one = W.agent_metadata_bincode("ab", [("ab", 3, 0x1122334455667788, 96, 1, 1, b"[2]")])
    assert one == bytes.fromhex(
        "0200000000000000" "6162"            # agent "ab"
        "0100000000000000"                   # one block
        "0200000000000000" "6162"            # owner agent
        "0300000000000000"                   # block_id 3
        "8877665544332211"                   # addr
        "6000000000000000"                   # len 96
        "0100000000000000"                   # dev_id 1
        "01000000"                           # BlockMemType::Vram
        "0300000000000000" "5b325d")         # meta "[2]"
    assert W.shape_meta([1, 2, 3, 4]) == b"[1,2,3,4]" and W.shape_meta([]) == b"[]"
    # a planted mistake (u32 length prefixes, as bincode's varint or a 32-bit config would
    # not give) changes the bytes
    assert W.agent_metadata_bincode("a", []) != bytes.fromhex("01000000" "61" "00000000")
