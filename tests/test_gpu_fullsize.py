"""Parity at the full benchmark sizes (c2 8k and c3 32k ring prefill, c4 paged decode and
the growth-sharded decode Q-ring at its shape, c5 128k staging and prefill), through properties that do not need the whole closed form: sampled query rows
against the f64 closed form, order invariance between strategies, bit-exactness against
an independent GPU gather (torch advanced indexing) and scatter/gather round trips.
Inputs come from the device LCG generator with the bench's seeds."""
import math

import numpy as np
import pytest
import torch

import hcp_ring_amd as H
from oracle import inputs as I, tch_ring as T

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2
LSE_TOL = 1e-3


def synth(seed, shapes):
    out, off = [], 0
    for shp in shapes:
        t = torch.empty(*shp, dtype=torch.bfloat16, device="cuda")
        H.synth_normals(seed, off, t.numel(), t)
        off += t.numel()
        out.append(t)
    return out


def rows_closed_form(q32, k32, v32, rows, scale, key_end):
    """f64 attention of query rows `rows` (q32 [S, Hq, D]) over keys [0, key_end(r))."""
    hq, hkv = q32.shape[1], k32.shape[1]
    rep = hq // hkv
    o = np.zeros((len(rows), hq, q32.shape[2]))
    lse = np.zeros((len(rows), hq))
    for i, r in enumerate(rows):
        e = key_end(r)
        for g in range(hkv):
            qg = q32[r, g * rep:(g + 1) * rep].astype(np.float64)          # [rep, D]
            kg = k32[:e, g].astype(np.float64)                              # [e, D]
            s = qg @ kg.T * scale
            m = s.max(axis=1, keepdims=True)
            w = np.exp(s - m)
            den = w.sum(axis=1, keepdims=True)
            o[i, g * rep:(g + 1) * rep] = (w @ v32[:e, g].astype(np.float64)) / den
            lse[i, g * rep:(g + 1) * rep] = (m + np.log(den))[:, 0]
    return o, lse


def test_c3_full_ring_prefill_sampled_rows_and_strategy_invariance(gpu):
    chunks, hq, hkv, d = [12288, 8192, 8192, 4096], 32, 8, 128
    s = sum(chunks)
    q, k, v = synth(44, [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    out, lse = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    rows = [0, 1, 777, 12287, 12288, 20479, 20480, 28671, 28672, 31000, 32767]
    q32, k32, v32 = (x.float().cpu().numpy() for x in (q, k, v))
    ref_o, ref_l = rows_closed_form(q32, k32, v32, rows, 1 / math.sqrt(d), lambda r: r + 1)
    got_o = out.float().cpu().numpy()[:, rows].transpose(1, 0, 2)
    got_l = lse.cpu().numpy()[:, rows].T
    assert np.abs(got_o - ref_o).max() <= OUT_TOL
    assert np.abs(got_l - ref_l).max() <= LSE_TOL
    # the same sequence under ZigZag and Striped positions (rows in domain-major order)
    # agrees: the one-launch schedule AUTO takes, and ZigZag ring step by ring step
    from oracle import strategy as SP
    for strategy, schedule in (("zigzag", "auto"), ("striped", "auto"), ("zigzag", "per_step")):
        a = SP.build_assignment(chunks, strategy)
        order = torch.tensor(sum(SP.build_domain_positions(a), []), device="cuda")
        inv = torch.tensor(SP.build_inverse_perm(a), device="cuda")
        qz, kz, vz = (x.index_select(0, order).permute(1, 0, 2) for x in (q, k, v))
        oz, lz = H.ring_attention_replay(qz, kz, vz, chunks, strategy=strategy, schedule=schedule)
        oz, lz = oz.index_select(1, inv), lz.index_select(1, inv)
        torch.cuda.synchronize()
        assert (oz.float() - out.float()).abs().max().item() <= 2 * OUT_TOL, (strategy, schedule)
        assert (lz - lse).abs().max().item() <= 2 * LSE_TOL, (strategy, schedule)
        del qz, kz, vz, oz, lz


def test_c3_last_domain_whole_against_ring_attention(gpu):
    # Domain 3 of c3 whole (rows 28672..32767, 32 heads) against the op-for-op
    # restatement of ring_attention (ring.rs:861-1398) on the fp32 upcasts: its local
    # chunk, then domains 2, 1 and 0 in ring order -- every ring step of the target
    # whose rows see all four sources.
    chunks, hq, hkv, d = [12288, 8192, 8192, 4096], 32, 8, 128
    s = sum(chunks)
    q, k, v = synth(44, [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    out, lse = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks)
    assert H.last_path() == "ring_fused"
    torch.cuda.synchronize()
    offs = [0, 12288, 20480, 28672]
    off = offs[3]
    q32, k32, v32 = (x.float().cpu().numpy() for x in (q, k, v))
    f = lambda x: torch.from_numpy(x).permute(1, 0, 2).unsqueeze(0)
    kx, vx = T.repeat_kv_heads(f(k32), hq // hkv), T.repeat_kv_heads(f(v32), hq // hkv)
    sent = [T.local_micro_blocks(kx[:, :, o:o + L], vx[:, :, o:o + L], o, 4) for o, L in zip(offs, chunks)]
    ro, rl = T.ring_attention(1 / math.sqrt(d), f(q32)[:, :, off:], kx[:, :, off:], vx[:, :, off:],
                              torch.arange(off, s), off, 4, [sent[2], sent[1], sent[0]], return_lse=True)
    assert np.abs(out[:, off:].float().cpu().numpy() - ro[0].numpy()).max() <= OUT_TOL
    assert np.abs(lse[:, off:].cpu().numpy() - rl[0].numpy()).max() <= LSE_TOL


def test_c2_full_ring_prefill_both_schedules(gpu):
    # Qwen2.5-3B shape at its stated size: S=8192 in [4096, 2560, 1536], 16 q / 2 kv heads
    # (eight query heads per KV head), D=128, bf16, seed 43.
    chunks, hq, hkv, d = [4096, 2560, 1536], 16, 2, 128
    s = sum(chunks)
    q, k, v = synth(43, [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    out, lse = H.ring_attention_replay(qh, kh, vh, chunks)
    assert H.last_path() == "ring_fused"
    out_s, lse_s = H.ring_attention_replay(qh, kh, vh, chunks, schedule="per_step")
    assert H.last_path() == "mfma"
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    # every domain's first and last row, and a few inside, against the f64 closed form
    rows = [0, 1, 2047, 4095, 4096, 5000, 6655, 6656, 7000, 8191]
    q32, k32, v32 = (x.float().cpu().numpy() for x in (q, k, v))
    ref_o, ref_l = rows_closed_form(q32, k32, v32, rows, 1 / math.sqrt(d), lambda r: r + 1)
    for o, l in ((out, lse), (out_s, lse_s)):
        got_o = o.float().cpu().numpy()[:, rows].transpose(1, 0, 2)
        got_l = l.cpu().numpy()[:, rows].T
        assert np.abs(got_o - ref_o).max() <= OUT_TOL
        assert np.abs(got_l - ref_l).max() <= LSE_TOL
    # the last domain whole against the op-for-op restatement of ring_attention
    # (ring.rs:861-1398) on the fp32 upcasts: its local chunk, then domains 1 and 0
    off = 6656
    f = lambda x: torch.from_numpy(x).permute(1, 0, 2).unsqueeze(0)
    kx, vx = T.repeat_kv_heads(f(k32), hq // hkv), T.repeat_kv_heads(f(v32), hq // hkv)
    offs = [0, 4096, 6656]
    sent = [T.local_micro_blocks(kx[:, :, o:o + L], vx[:, :, o:o + L], o, 3) for o, L in zip(offs, chunks)]
    ro, rl = T.ring_attention(1 / math.sqrt(d), f(q32)[:, :, off:], kx[:, :, off:], vx[:, :, off:],
                              torch.arange(off, s), off, 3, [sent[1], sent[0]], return_lse=True)
    for o, l in ((out, lse), (out_s, lse_s)):
        assert np.abs(o[:, off:].float().cpu().numpy() - ro[0].numpy()).max() <= OUT_TOL
        assert np.abs(l[:, off:].cpu().numpy() - rl[0].numpy()).max() <= LSE_TOL


def test_qwen2_0p5b_d64_ring_prefill_q_ending_at_a_segment(gpu):
    # The reference's own model heads (Qwen2-0.5B: 14 q / 2 kv heads, D=64) on c2's chunks,
    # token-major Q/K/V as the projection writes them, both schedules.  Q is 7 x 2 MiB,
    # so it ends where the allocator's segment ends: the block kernel's Q loads must stop
    # at the view's last element (a range of whole 128-dim rows once read 128 bytes past
    # the end of Q for the last row of the last head).  Rows against the f64 closed form,
    # the last row included.
    chunks, hq, hkv, d = [4096, 2560, 1536], 14, 2, 64
    s = sum(chunks)
    q, k, v = synth(47, [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    assert (q.numel() * q.element_size()) % (2 << 20) == 0
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    out, lse = H.ring_attention_replay(qh, kh, vh, chunks)
    assert H.last_path() == "ring_fused"
    out_s, lse_s = H.ring_attention_replay(qh, kh, vh, chunks, schedule="per_step")
    assert H.last_path() == "mfma"
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    rows = [0, 1, 127, 4095, 4096, 5000, 6655, 6656, 7000, 8190, 8191]
    q32, k32, v32 = (x.float().cpu().numpy() for x in (q, k, v))
    ref_o, ref_l = rows_closed_form(q32, k32, v32, rows, 1 / math.sqrt(d), lambda r: r + 1)
    for o, l in ((out, lse), (out_s, lse_s)):
        got_o = o.float().cpu().numpy()[:, rows].transpose(1, 0, 2)
        got_l = l.cpu().numpy()[:, rows].T
        assert np.abs(got_o - ref_o).max() <= OUT_TOL
        assert np.abs(got_l - ref_l).max() <= LSE_TOL


def test_c4_full_paged_decode_every_sequence(gpu):
    batch, hq, hkv, d, bs, ctx, nb = 64, 32, 8, 128, 16, 16384, 65536
    chunks = [8192, 5120, 3072]
    q = torch.empty(batch, hq, d, dtype=torch.bfloat16, device="cuda")
    pool = torch.empty(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.synth_normals(45, 0, q.numel(), q)
    H.synth_normals(45, q.numel(), pool.numel(), pool)
    # the config's block tables: the seeded LCG Fisher-Yates permutation of the pool (as the bench draws them)
    tables_np = I.permuted_block_table(45, nb)[: batch * (ctx // bs)].reshape(batch, ctx // bs)
    tables = torch.from_numpy(tables_np).cuda()
    parts, t0 = [], 0
    for L in chunks:
        parts.append(H.decode_local_compact_partial(q, pool, tables, t0, t0 + L))
        t0 += L
    out, lse = H.lse_merge([o.view(-1, 1, d) for o, _ in parts], [l.view(-1, 1) for _, l in parts],
                           out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    out = out.view(batch, hq, d).float().cpu()
    lse = lse.view(batch, hq).cpu()
    # every sequence against the f64 closed form over its whole context, K/V read
    # through its block table from a host copy of the pool
    pool_h, q_h = pool.cpu(), q.cpu().double()
    tabs = torch.from_numpy(tables_np.astype(np.int64))
    rep, scale = hq // hkv, 1 / math.sqrt(d)
    err_o = err_l = 0.0
    for b in range(batch):
        k = pool_h[0].index_select(0, tabs[b]).reshape(ctx, hkv, d).double().permute(1, 2, 0)  # [hkv, d, ctx]
        v = pool_h[1].index_select(0, tabs[b]).reshape(ctx, hkv, d).double().permute(1, 0, 2)  # [hkv, ctx, d]
        sc = torch.matmul(q_h[b].view(hkv, rep, d), k) * scale                                 # [hkv, rep, ctx]
        rl = torch.logsumexp(sc, dim=2)
        ro = torch.matmul(torch.exp(sc - rl.unsqueeze(2)), v)                                  # [hkv, rep, d]
        err_o = max(err_o, (out[b] - ro.reshape(hq, d)).abs().max().item())
        err_l = max(err_l, (lse[b] - rl.reshape(hq)).abs().max().item())
    assert err_o <= OUT_TOL and err_l <= LSE_TOL, (err_o, err_l)


def test_decode_ring_growth_sharded_at_c4_shape(gpu):
    # The decode Q-ring (ring.rs:665-818) at c4's shape with growth sharding
    # (ring.rs:1930-1936): 64 sequences of 16384 tokens, the last 96 decode tokens each
    # in its owner's shard (p mod 3), every domain shard with its own permuted block
    # table.  From two seeds, every sequence's output equals the f64 closed form over the
    # union of its shards (the whole context).
    batch, hq, hkv, d, bs, ctx, dec, n = 64, 32, 8, 128, 16, 16384, 96, 3
    chunks = [8192, 5120, 3072 - dec]
    prefill = ctx - dec
    lens = [chunks[dom] + sum(1 for p in range(prefill, ctx) if p % n == dom) for dom in range(n)]
    nblk = [-(-L // bs) for L in lens]
    nb = batch * sum(nblk) + 1
    q = torch.empty(batch, hq, d, dtype=torch.bfloat16, device="cuda")
    pool = torch.empty(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.synth_normals(48, 0, q.numel(), q)
    H.synth_normals(48, q.numel(), pool.numel(), pool)
    perm = I.permuted_block_table(48, nb)
    shards, tabs, cur = [], [], 0
    for dom in range(n):
        tab = perm[cur:cur + batch * nblk[dom]].reshape(batch, nblk[dom])
        cur += batch * nblk[dom]
        tabs.append(torch.from_numpy(tab.astype(np.int64)))
        shards.append((torch.from_numpy(np.ascontiguousarray(tab)).cuda(),
                       torch.full((batch,), lens[dom], dtype=torch.int32, device="cuda"), lens[dom]))
    results = []
    for seed in (0, 2):
        out, lse = H.decode_ring_replay(q, pool, shards, seed)
        torch.cuda.synchronize()
        assert H.fetch_device_errors() == 0
        results.append((out.float().cpu(), lse.cpu()))
    pool_h, q_h = pool.cpu(), q.cpu().double()
    rep, scale = hq // hkv, 1 / math.sqrt(d)
    err_o = err_l = 0.0
    for b in range(batch):
        ks, vs = [], []
        for dom in range(n):
            ks.append(pool_h[0].index_select(0, tabs[dom][b]).reshape(-1, hkv, d)[:lens[dom]])
            vs.append(pool_h[1].index_select(0, tabs[dom][b]).reshape(-1, hkv, d)[:lens[dom]])
        k = torch.cat(ks).double().permute(1, 2, 0)                                            # [hkv, d, ctx]
        v = torch.cat(vs).double().permute(1, 0, 2)                                            # [hkv, ctx, d]
        sc = torch.matmul(q_h[b].view(hkv, rep, d), k) * scale                                 # [hkv, rep, ctx]
        rl = torch.logsumexp(sc, dim=2)
        ro = torch.matmul(torch.exp(sc - rl.unsqueeze(2)), v).reshape(hq, d)
        for out, lse in results:
            err_o = max(err_o, (out[b] - ro).abs().max().item())
            err_l = max(err_l, (lse[b] - rl.reshape(hq)).abs().max().item())
    assert err_o <= OUT_TOL and err_l <= LSE_TOL, (err_o, err_l)


def test_c5_full_staging_bit_exact_against_torch_indexing(gpu):
    chunks = [21504, 13312, 18432, 23552, 24576, 9216, 8192, 12288]
    hkv, d, bs = 8, 128, 16
    s = sum(chunks)
    k, v = synth(46, [(s, hkv, d), (s, hkv, d)])
    nb = s // bs
    perm = torch.from_numpy(np.random.default_rng(46).permutation(nb).astype(np.int32)).cuda()
    pool = torch.zeros(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.paged_kv_scatter(pool, perm, 0, 0, s, k.permute(1, 0, 2), v.permute(1, 0, 2))
    # independent placement check: pool[plane, perm[t // bs], t % bs] == source token t
    t = torch.arange(s, device="cuda")
    blk, slot = perm.long()[t // bs], t % bs
    assert torch.equal(pool[0][blk, slot].view(torch.int16), k.view(torch.int16))
    assert torch.equal(pool[1][blk, slot].view(torch.int16), v.view(torch.int16))
    ranges, off = [], 0
    for L in chunks:
        ko = torch.empty(hkv, L, d, dtype=torch.bfloat16, device="cuda")
        ranges.append((perm, 0, off, off + L, ko, torch.empty_like(ko)))
        off += L
    H.paged_kv_gather_batch(pool, ranges)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    for (_, _, a, b, ko, vo) in ranges:
        assert torch.equal(ko.view(torch.int16), k[a:b].permute(1, 0, 2).view(torch.int16))
        assert torch.equal(vo.view(torch.int16), v[a:b].permute(1, 0, 2).view(torch.int16))


def test_c5_full_staged_prefill_output(gpu):
    # The 128k staged replay at its config: 8 seeded chunks, Llama-3-8B heads, the K/V of
    # the whole sequence in a bs=16 pool under the LCG-permuted block table (seed 42, as
    # the bench).  Staging is bit-exact, so the paged replays equal the unpaged ones bit
    # for bit; sampled rows at every domain boundary match the f64 closed form.
    chunks = I.c5_chunks()
    assert chunks == [21504, 13312, 18432, 23552, 24576, 9216, 8192, 12288]
    hq, hkv, d, bs = 32, 8, 128, 16
    s = sum(chunks)
    q, k, v = synth(46, [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    nb = s // bs
    table = torch.from_numpy(I.permuted_block_table(42, nb)).cuda()
    pool = torch.zeros(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    H.paged_kv_scatter(pool, table, 0, 0, s, kh, vh)
    out_p, lse_p = H.ring_attention_replay_paged(qh, pool, table, chunks)
    assert H.last_path() == "ring_fused"
    out_u, lse_u = H.ring_attention_replay(qh, kh, vh, chunks)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert torch.equal(out_p, out_u) and torch.equal(lse_p, lse_u)
    assert torch.isfinite(out_p.float()).all() and torch.isfinite(lse_p).all()
    offs = [sum(chunks[:i]) for i in range(len(chunks))]
    rows = sorted({0, s - 1} | {o for o in offs} | {o - 1 for o in offs if o > 0} | {offs[3] + 777})
    q32 = q[torch.tensor(rows, device="cuda")].float().cpu().numpy()
    k32, v32 = k.float().cpu().numpy(), v.float().cpu().numpy()
    ref_o, ref_l = rows_closed_form(q32, k32, v32, list(range(len(rows))), 1 / math.sqrt(d),
                                    lambda i: rows[i] + 1)
    got_o = out_p.float().cpu().numpy()[:, rows].transpose(1, 0, 2)
    got_l = lse_p.cpu().numpy()[:, rows].T
    assert np.abs(got_o - ref_o).max() <= OUT_TOL
    assert np.abs(got_l - ref_l).max() <= LSE_TOL
    # the per-step paged schedule (a gather per ring step into per-domain ring buffers,
    # eight-pair grouped launches) agrees with the fused one within the tolerances
    out_s, lse_s = H.ring_attention_replay_paged(qh, pool, table, chunks, schedule="per_step")
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert (out_s.float() - out_p.float()).abs().max().item() <= OUT_TOL
    assert (lse_s - lse_p).abs().max().item() <= LSE_TOL


def test_c5_full_paged_zigzag_one_launch(gpu):
    # c5 (131072 tokens in 8 domains, Llama-3-8B heads) under ZigZag positions, K/V in a
    # permuted bs=16 pool in domain-major order: the one-launch schedule (chunks staged,
    # K/V gathered into position order, one positions-mode block) equals the unpaged
    # replay bit for bit; sampled rows (the first and last rows of every domain, i.e.
    # both ends of its two zigzag runs) match the f64 closed form over the keys at
    # positions up to their own.
    from oracle import strategy as SP
    chunks = I.c5_chunks()
    hq, hkv, d, bs = 32, 8, 128, 16
    s = sum(chunks)
    q, k, v = synth(48, [(s, hq, d), (s, hkv, d), (s, hkv, d)])  # position order
    a = SP.build_assignment(chunks, "zigzag")
    pos = sum(SP.build_domain_positions(a), [])                     # row r holds position pos[r]
    order = torch.tensor(pos, device="cuda")
    qd, kd, vd = (x.index_select(0, order).permute(1, 0, 2).contiguous() for x in (q, k, v))
    nb = s // bs
    table = torch.from_numpy(I.permuted_block_table(42, nb)).cuda()
    pool = torch.zeros(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.paged_kv_scatter(pool, table, 0, 0, s, kd, vd)
    out_p, lse_p = H.ring_attention_replay_paged(qd, pool, table, chunks, strategy="zigzag")
    out_u, lse_u = H.ring_attention_replay(qd, kd, vd, chunks, strategy="zigzag")
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert torch.equal(out_p, out_u) and torch.equal(lse_p, lse_u)
    offs = [sum(chunks[:i]) for i in range(len(chunks))]
    rows = sorted({o for o in offs} | {o + L - 1 for o, L in zip(offs, chunks)} |
                  {o + (L + 1) // 2 - 1 for o, L in zip(offs, chunks)} | {o + (L + 1) // 2 for o, L in zip(offs, chunks)})
    p = [pos[r] for r in rows]
    q32 = q[torch.tensor(p, device="cuda")].float().cpu().numpy()
    k32, v32 = k.float().cpu().numpy(), v.float().cpu().numpy()
    ref_o, ref_l = rows_closed_form(q32, k32, v32, list(range(len(rows))), 1 / math.sqrt(d), lambda i: p[i] + 1)
    got_o = out_p.float().cpu().numpy()[:, rows].transpose(1, 0, 2)
    got_l = lse_p.cpu().numpy()[:, rows].T
    assert np.abs(got_o - ref_o).max() <= OUT_TOL
    assert np.abs(got_l - ref_l).max() <= LSE_TOL


@pytest.mark.parametrize("tokens", [4096, 2048, 12288, 12200])
def test_llama3_8b_qkv_rope_sampled_tokens(gpu, tokens):
    # The Llama-3-8B projection (hidden 4096 -> 32 q / 8 kv heads of 128, RoPE theta 5e5)
    # at token counts whose launches take 128-, 256- and 384-token tiles (12200: 384 with
    # a partial last tile); sampled tokens of q, k and v against the f64 closed form
    # rotated with the library's own table, and for 12200 the paged append against the
    # plain views, bit for bit.
    hidden, hq, hkv, d = 4096, 32, 8, 128
    x, wq, wk, wv = synth(47, [(tokens, hidden), (hq * d, hidden), (hkv * d, hidden), (hkv * d, hidden)])
    for w in (wq, wk, wv):
        w.mul_(1.0 / math.sqrt(hidden))
    table = H.rope_table(d, tokens + 64, 500000.0)
    pos = torch.arange(64, 64 + tokens, dtype=torch.int64, device="cuda")
    q, k, v = H.qkv_rope_project(x, wq, wk, wv, hq, hkv, d, positions=pos, table=table)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    rows = np.unique(np.array([0, 1, 127, 128, 255, 383, 384, tokens // 2, tokens - 2, tokens - 1]))
    xs = x[torch.from_numpy(rows).cuda()].double().cpu().numpy()
    tab = table.cpu().double().numpy()
    c, s = tab[0][rows + 64], tab[1][rows + 64]
    for got, w, heads, rot in ((q, wq, hq, True), (k, wk, hkv, True), (v, wv, hkv, False)):
        y = (xs @ w.double().cpu().numpy().T).reshape(len(rows), heads, d)
        if rot:
            y1, y2 = y[..., : d // 2], y[..., d // 2:]
            y = np.concatenate([y1 * c[:, None] - y2 * s[:, None], y1 * s[:, None] + y2 * c[:, None]], axis=-1)
        g = got[:, torch.from_numpy(rows).cuda()].transpose(0, 1).double().cpu().numpy()
        bound = np.abs(y) / 128 + 1e-3 * np.abs(y).max()
        assert np.all(np.abs(g - y) <= bound), (tokens, float(np.abs(g - y).max()))
    if tokens == 12200:
        bs_, off = 16, 5
        nb = (tokens + off + bs_ - 1) // bs_ + 3
        pool = torch.zeros(2, nb, bs_, hkv, d, dtype=torch.bfloat16, device="cuda")
        blocks = torch.from_numpy(np.random.default_rng(48).permutation(nb).astype(np.int32)).cuda()
        q2 = H.qkv_rope_project_paged(x, wq, wk, wv, hq, hkv, d, pool, blocks, 0, off, positions=pos, table=table)
        k2, v2 = H.paged_kv_gather(pool, blocks, 0, off, off + tokens)
        torch.cuda.synchronize()
        assert H.fetch_device_errors() == 0
        assert torch.equal(q.view(torch.int16), q2.view(torch.int16))
        assert torch.equal(k.view(torch.int16), k2.view(torch.int16))
        assert torch.equal(v.view(torch.int16), v2.view(torch.int16))


def test_block_partial_key_range_beyond_4gib(gpu):
    """K/V views spanning more than 4 GiB (2.2M keys stored token-major, [L, Hkv, D]):
    every DMA descriptor covers one tile's rows, so no byte count wraps at 2^32.  The
    whole range in one block partial equals the LSE merge of its two halves."""
    lk, hkv, d, hq, lq = 2_200_000, 8, 128, 32, 128
    q = torch.empty(lq, hq, d, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(lk, hkv, d, dtype=torch.bfloat16, device="cuda")
    v = torch.empty_like(k)
    off = 0
    for t in (q, k, v):
        H.synth_normals(47, off, t.numel(), t)
        off += t.numel()
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    assert kh.stride(1) * 2 * lk > 2 ** 32
    o, l = H.block_partial(qh, kh, vh, lk, 0)          # queries after every key
    half = lk // 2
    o1, l1 = H.block_partial(qh, kh[:, :half], vh[:, :half], lk, 0)
    o2, l2 = H.block_partial(qh, kh[:, half:], vh[:, half:], lk, half)
    om, lm = H.lse_merge([o1, o2], [l1, l2], out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert H.last_path() in ("mfma", "general")
    o, l, om, lm = (x.cpu().numpy() for x in (o, l, om, lm))
    assert np.abs(l - lm).max() <= 1e-4
    # both sides round P to bf16 against different reference maxima: up to 2 x 2^-9
    assert np.abs(o - om).max() <= 4e-3 * np.abs(om).max()
    del k, v
