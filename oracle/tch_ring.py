"""Op-for-op libtorch (CPU) restatement of the reference's blockwise ring attention.

TEST INFRASTRUCTURE: only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module.  It is the checker and the timed CPU
baseline, never the product path.

The reference is Rust calling libtorch through ``tch`` 0.24.0
(``rust/src/model/attention/ring.rs``); it cannot be built here (no cargo/rustc), so
this module replays the same ATen op sequence through PyTorch's CPU backend:

* :func:`process_kv_block`            ring.rs:201-370
* :func:`repeat_kv_heads`             ring.rs:496-512 (and the forward-path expand :1962-1984)
* :func:`positioned_local_compact_partial`  ring.rs:538-571
* :func:`positioned_merge_compact_partial`  ring.rs:574-603
* :func:`decode_local_partial`        ring.rs:625-639 (+ compact variant :515-523)
* :func:`decode_merge_packet`         ring.rs:647-663 (+ compact variant :525-536)
* :func:`ring_decode_attention`       ring.rs:665-818 (the decode Q-ring, one packet's journey)
* :func:`ring_attention`              ring.rs:861-1398 (tiling, order, early exit, output)
* :func:`rope_caches`, :func:`rope_apply`  rust/src/model/layers/rotary.rs:56-158
* :func:`qkv_rope_forward`            ring.rs:1865-1908 (projection, bias, head split, RoPE)
* :func:`ring_attention_replay`       CS2 of the reference tests (ring.rs:3014-3165,
                                      3230-3364): every domain driven in one process,
                                      peers delivered by a mock transport
                                      (rust/src/model/transport/mock.rs:99-159).
* :func:`ring_attention_replay_strategy`  run_uneven_ring_attention (ring.rs:3226-3364)
                                      with Striped / ZigZag positions.

Tensor layout follows the reference: ``[batch, heads, seq, head_dim]``; positions are
int64 CPU tensors.  The running state (rm, rs, obh) is kept in the query dtype, as the
reference does (ring.rs:553-555, 967-976); call with fp32 tensors to get "the same
algorithm on exact fp32 upcasts".
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

NEG_INIT = -1e4  # ring.rs:553, 967-972: finite running-max init


def process_kv_block(scale: float, q_chunk, q_pos, k_chunk, v_chunk, k_pos, rm, rs, obh,
                     apply_causal_mask: bool):
    """Fold one K/V block into the running (rm, rs, obh); returns the new triple.

    ring.rs:201-370.  ``q_chunk`` [B,H,qc,D], ``k_chunk``/``v_chunk`` [B,H,kc,D] (already
    GQA-expanded), ``q_pos`` [qc] and ``k_pos`` [kc] int64 global positions.
    """
    kv_chunk_len = k_pos.shape[0]
    if kv_chunk_len <= 0:  # :215-217
        return rm, rs, obh
    if apply_causal_mask:  # :222-228 early exit when every key is in the future
        if int(k_pos.min()) > int(q_pos.max()):
            return rm, rs, obh
    scores = torch.matmul(q_chunk, k_chunk.transpose(2, 3)) * scale  # :238
    q_kind = q_chunk.dtype
    if apply_causal_mask:  # :249-273
        q_pos_t = q_pos.unsqueeze(1).unsqueeze(0).unsqueeze(0)
        k_pos_t = k_pos.unsqueeze(0).unsqueeze(0).unsqueeze(0)
        causal = q_pos_t.ge(k_pos_t)
        neg_inf = torch.tensor(float("-inf")).to(q_kind)
        zero = torch.zeros(1, dtype=q_kind)
        neg_inf_mask = torch.where(causal.logical_not(), neg_inf, zero)
        scores = scores + neg_inf_mask
    local_max = scores.amax(dim=3, keepdim=False)  # :313
    neg_inf_t = torch.tensor(float("-inf")).to(q_kind)
    all_masked = local_max.eq(neg_inf_t)  # :322
    local_max_safe = local_max.masked_fill(all_masked, 0.0)  # :323
    weights = (scores - local_max_safe.unsqueeze(3)).exp()  # :328
    local_sum = weights.sum(dim=3, keepdim=False, dtype=q_kind)  # :333
    local_pv = torch.matmul(weights, v_chunk)  # :338
    new_max = torch.maximum(rm, local_max)  # :341
    exp_prev = (rm - new_max).exp()  # :345
    exp_local = (local_max - new_max).exp()  # :348
    new_sum = exp_prev * rs + exp_local * local_sum  # :352
    new_sum_safe = torch.where(new_sum.ne(0.0), new_sum, torch.ones_like(new_sum))  # :355
    obh = (exp_prev.unsqueeze(3) * rs.unsqueeze(3) * obh
           + exp_local.unsqueeze(3) * local_pv) / new_sum_safe.unsqueeze(3)  # :361-363
    return new_max, new_sum, obh  # :366-367


def repeat_kv_heads(k, num_rep: int):
    """GQA expand [B,Hkv,L,D] -> [B,Hkv*rep,L,D]; kv head of q head h is h // rep (ring.rs:496-512)."""
    if num_rep == 1:
        return k
    b, h, s, d = k.shape
    return k.unsqueeze(2).expand(b, h, num_rep, s, d).reshape(b, h * num_rep, s, d)


def _init_state(q):
    b, h, lq, d = q.shape
    rm = torch.full((b, h, lq), NEG_INIT, dtype=q.dtype)
    rs = torch.zeros((b, h, lq), dtype=q.dtype)
    obh = torch.zeros((b, h, lq, d), dtype=q.dtype)
    return rm, rs, obh


def positioned_local_compact_partial(scale, q, q_positions, k, v, k_positions):
    """Per-ring-step partial (o, lse fp32) over one causal source (ring.rs:538-571)."""
    num_rep = q.shape[1] // k.shape[1]
    k, v = repeat_kv_heads(k, num_rep), repeat_kv_heads(v, num_rep)
    rm, rs, obh = _init_state(q)
    rm, rs, obh = process_kv_block(scale, q, q_positions.reshape(-1), k, v,
                                   k_positions.reshape(-1), rm, rs, obh, True)
    lse = (rm + rs.log()).to(torch.float32)  # :569
    return obh, lse


def positioned_merge_compact_partial(scale, q, q_positions, o, lse, k, v, k_positions):
    """Merge a running (o, lse) with one more causal source (ring.rs:574-603)."""
    num_rep = q.shape[1] // k.shape[1]
    k, v = repeat_kv_heads(k, num_rep), repeat_kv_heads(v, num_rep)
    rm = lse.to(q.dtype)  # :585
    rs = torch.ones_like(rm)
    obh = o
    rm, rs, obh = process_kv_block(scale, q, q_positions.reshape(-1), k, v,
                                   k_positions.reshape(-1), rm, rs, obh, True)
    return obh, (rm + rs.log()).to(torch.float32)


def decode_local_partial(scale, q, k, v):
    """Single query, non-causal partial (ring.rs:625-639); k/v already expanded."""
    b, h, _, d = q.shape
    rm = torch.full((b, h, 1), NEG_INIT, dtype=q.dtype)
    rs = torch.zeros((b, h, 1), dtype=q.dtype)
    obh = torch.zeros((b, h, 1, d), dtype=q.dtype)
    q_pos = torch.zeros(1, dtype=torch.int64)
    k_pos = torch.zeros(k.shape[2], dtype=torch.int64)
    rm, rs, obh = process_kv_block(scale, q, q_pos, k, v, k_pos, rm, rs, obh, False)
    return obh, (rm + rs.log()).to(torch.float32)


def decode_local_compact_partial(scale, q, k, v):
    num_rep = q.shape[1] // k.shape[1]
    return decode_local_partial(scale, q, repeat_kv_heads(k, num_rep), repeat_kv_heads(v, num_rep))


def decode_merge_packet(scale, q, o, lse, k, v):
    """Merge a ring packet's (o, lse) with a local segment (ring.rs:647-663)."""
    rm = lse.to(q.dtype)
    rs = torch.ones_like(rm)
    obh = o
    q_pos = torch.zeros(1, dtype=torch.int64)
    k_pos = torch.zeros(k.shape[2], dtype=torch.int64)
    rm, rs, obh = process_kv_block(scale, q, q_pos, k, v, k_pos, rm, rs, obh, False)
    return obh, (rm + rs.log()).to(torch.float32)


def ring_decode_attention(scale, q, durable, cur_k, cur_v, seed: int):
    """One packet's journey of ring_decode_attention (ring.rs:665-818).

    durable[d] = (k, v) of domain d before this step, compact heads [B, Hkv, L_d, D]
    (growth sharding, ring.rs:1930-1936); cur_k / cur_v = the new token [B, Hkv, 1, D].
    Phase 0 seeds the packet at domain `seed` with the partial over its local segment
    [durable; current token] (decode_local_partial); each of the N-1 rounds merges the
    next domain's durable segment without the current token (k_peer = narrow(0,
    local_len - 1), decode_merge_packet), visiting seed+1, ..., seed-1 (mod N).  An
    empty durable segment passes the packet through unchanged (lse + log 1)."""
    n = len(durable)
    k, v = durable[seed]
    o, lse = decode_local_compact_partial(scale, q, torch.cat([k, cur_k], 2), torch.cat([v, cur_v], 2))
    for j in range(1, n):
        k, v = durable[(seed + j) % n]
        if k.shape[2] == 0:
            continue
        o, lse = decode_merge_compact_partial(scale, q, o, lse, k, v)
    return o, lse


def decode_merge_compact_partial(scale, q, o, lse, k, v):
    num_rep = q.shape[1] // k.shape[1]
    return decode_merge_packet(scale, q, o, lse, repeat_kv_heads(k, num_rep),
                               repeat_kv_heads(v, num_rep))


def rope_caches(dim: int, max_seq_len: int, base: float):
    """RotaryEmbedding::new (rotary.rs:56-97): inv_freq[i] = 1 / base^(2i/dim) in f64
    cast to f32; angles = positions (f32) x inv_freq (f32); cos / sin in f32."""
    half = dim // 2
    inv = torch.tensor([1.0 / base ** ((2.0 * i) / dim) for i in range(half)], dtype=torch.float32)
    ang = torch.arange(max_seq_len, dtype=torch.float32).unsqueeze(1) * inv.unsqueeze(0)
    return ang.cos(), ang.sin()


def rope_apply(q, k, position_ids, cos_cache, sin_cache):
    """RotaryEmbedding::apply + rotate_pairs (rotary.rs:103-158): halves (d, d + D/2)
    rotated by the cached angle of each token's position, cos / sin cast to q's dtype."""
    b, s = position_ids.shape
    half = cos_cache.shape[1]
    flat = position_ids.reshape(-1)
    cos = cos_cache.index_select(0, flat).view(b, s, half).unsqueeze(1).to(q.dtype)
    sin = sin_cache.index_select(0, flat).view(b, s, half).unsqueeze(1).to(q.dtype)

    def rot(x):
        x1, x2 = x[..., :half], x[..., half:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=3)

    return rot(q), rot(k)


def qkv_rope_forward(x, wq, wk, wv, bq, bk, bv, num_heads: int, num_kv_heads: int, head_dim: int,
                     position_ids, cos_cache, sin_cache, rope: bool = True):
    """The head of forward (ring.rs:1865-1908): x [B, L, hidden] -> q [B, Hq, L, D],
    k / v [B, Hkv, L, D] (projection, bias, head split, RoPE)."""
    b, l, _ = x.shape
    q = x.matmul(wq.transpose(0, 1))
    if bq is not None:
        q = q + bq
    k = x.matmul(wk.transpose(0, 1))
    if bk is not None:
        k = k + bk
    v = x.matmul(wv.transpose(0, 1))
    if bv is not None:
        v = v + bv
    q = q.view(b, l, num_heads, head_dim).transpose(1, 2)
    k = k.view(b, l, num_kv_heads, head_dim).transpose(1, 2)
    v = v.view(b, l, num_kv_heads, head_dim).transpose(1, 2)
    if rope:
        q, k = rope_apply(q, k, position_ids, cos_cache, sin_cache)
    return q, k, v


def chunk_sizes(seq_len: int, num_domains: int, micro_override: int = 0):
    """(q_chunk, kv_chunk, micro_block) sizes of one domain (ring.rs:925-935)."""
    q_chunk = min(max(-(-seq_len // num_domains), 1), 2048)
    kv_chunk = 2048 if seq_len == 1 else q_chunk
    micro = micro_override if micro_override > 0 else max(kv_chunk, 1024)
    return q_chunk, kv_chunk, micro


@dataclass
class KvMicroBlock:
    """The ring payload (rust/src/model/transport/block.rs:19-35)."""

    global_seq_start: int
    global_seq_end: int
    k: torch.Tensor
    v: torch.Tensor
    micro_block_idx: int
    total_micro_blocks: int
    position_ids: torch.Tensor | None = None  # block.rs:32-34 (Striped / ZigZag)


@dataclass
class RingStats:
    blocks_folded: int = 0
    blocks_skipped: int = 0
    visits: list = field(default_factory=list)


def ring_attention(scale, q, k, v, query_positions, global_seq_start: int, num_domains: int,
                   peer_rounds, apply_causal: bool = True, return_lse: bool = False,
                   stats: RingStats | None = None, local_kv_positions=None):
    """Per-domain driver (ring.rs:861-1398) with an in-memory transport.

    ``q`` [1,H,S_d,D], ``k``/``v`` [1,H,S_d,D] (post-expand, ring.rs:1962-1984),
    ``query_positions`` [S_d] int64.  ``peer_rounds[r]`` is the list of micro blocks the
    predecessor delivers in round r (source domain (d-1-r) mod N, ``mock.rs:143-149``).
    Phase 1 folds local KV tiles of ``kv_chunk`` per q-chunk state (:1208-1229); Phase 2
    folds every received micro block into every q-chunk state, in arrival order
    (:1239-1311).  Returns ``cat(obh)`` along seq (:1397); with ``return_lse`` also
    ``rm + log(rs)`` in fp32 (the reference driver itself returns no LSE).  Key
    positions: ``local_kv_positions`` narrowed per tile, else contiguous from
    ``global_seq_start`` (build_k_pos, :1024-1034); a peer block's ``position_ids``,
    else its [start, end) range (peer_k_pos, :1037-1046).
    """
    seq_len = q.shape[2]
    local_kv_len = k.shape[2]
    q_chunk, kv_chunk, _ = chunk_sizes(seq_len, num_domains)
    states = []
    for qs in range(0, seq_len, q_chunk):
        qe = min(qs + q_chunk, seq_len)
        qc = q[:, :, qs:qe]
        rm = torch.full(qc.shape[:3], NEG_INIT, dtype=q.dtype)
        rs = torch.zeros(qc.shape[:3], dtype=q.dtype)
        obh = torch.zeros(qc.shape, dtype=q.dtype)
        states.append([qc, query_positions[qs:qe], rm, rs, obh])

    def fold(st, kb, vb, kp, tag):
        before = st[2]
        st[2], st[3], st[4] = process_kv_block(scale, st[0], st[1], kb, vb, kp, st[2], st[3],
                                               st[4], apply_causal)
        if stats is not None:
            if st[2] is before:
                stats.blocks_skipped += 1
            else:
                stats.blocks_folded += 1
            stats.visits.append(tag)

    for st in states:  # Phase 1
        for ks in range(0, local_kv_len, kv_chunk):
            ke = min(ks + kv_chunk, local_kv_len)
            if local_kv_positions is not None:
                kp = local_kv_positions[ks:ke]
            else:
                kp = torch.arange(global_seq_start + ks, global_seq_start + ke, dtype=torch.int64)
            fold(st, k[:, :, ks:ke], v[:, :, ks:ke], kp, ("local", global_seq_start + ks))
    for r, blocks in enumerate(peer_rounds):  # Phase 2
        for blk in blocks:
            if blk.position_ids is not None:
                kp = blk.position_ids
            else:
                kp = torch.arange(blk.global_seq_start, blk.global_seq_end, dtype=torch.int64)
            for st in states:
                fold(st, blk.k, blk.v, kp, ("peer", r, blk.global_seq_start))
    out = torch.cat([st[4] for st in states], dim=2)
    if not return_lse:
        return out
    lse = torch.cat([(st[2] + st[3].log()).to(torch.float32) for st in states], dim=2)
    return out, lse


def local_micro_blocks(k, v, global_seq_start: int, num_domains: int, micro_override: int = 0,
                       positions=None):
    """Split a domain's (expanded) K/V into its sent micro blocks (ring.rs:980-1020);
    each block carries the matching slice of ``positions`` when given."""
    seq_len = k.shape[2]
    _, _, micro = chunk_sizes(seq_len, num_domains, micro_override)
    n = -(-seq_len // micro)
    out = []
    for i in range(n):
        s, e = i * micro, min((i + 1) * micro, seq_len)
        out.append(KvMicroBlock(global_seq_start + s, global_seq_start + e, k[:, :, s:e],
                                v[:, :, s:e], i, n, None if positions is None else positions[s:e]))
    return out


def ring_attention_replay_strategy(scale, q_all, k_all, v_all, chunks, strategy: str,
                                   causal: bool = True, return_lse: bool = False):
    """run_uneven_ring_attention (ring.rs:3226-3364) for any strategy: gather every
    domain's Q/K/V at its positions (build_domain_positions), run each domain's ring with
    those positions for its queries, local KV and the peer blocks it receives, then put
    the outputs back in global order with build_inverse_perm.  Inputs and outputs are
    in global order, ``[1, H, S, D]``."""
    from oracle import strategy as SP
    n = len(chunks)
    seq = q_all.shape[2]
    if sum(chunks) != seq:
        raise ValueError(f"chunk sum {sum(chunks)} != seq_len {seq}")
    assign = SP.build_assignment(list(chunks), strategy)
    positions = SP.build_domain_positions(assign)
    inverse = torch.tensor(SP.build_inverse_perm(assign), dtype=torch.int64)
    num_rep = q_all.shape[1] // k_all.shape[1]
    kx = repeat_kv_heads(k_all, num_rep)
    vx = repeat_kv_heads(v_all, num_rep)
    pos_t = [torch.tensor(p, dtype=torch.int64) for p in positions]
    sent = [local_micro_blocks(kx.index_select(2, pos_t[d]), vx.index_select(2, pos_t[d]), positions[d][0], n,
                               positions=pos_t[d]) for d in range(n)]
    outs, lses = [], []
    for d in range(n):
        rounds = [sent[(d - 1 - r) % n] for r in range(n - 1)]
        res = ring_attention(scale, q_all.index_select(2, pos_t[d]), kx.index_select(2, pos_t[d]),
                             vx.index_select(2, pos_t[d]), pos_t[d], positions[d][0], n, rounds,
                             apply_causal=causal, return_lse=return_lse, local_kv_positions=pos_t[d])
        if return_lse:
            outs.append(res[0])
            lses.append(res[1])
        else:
            outs.append(res)
    out = torch.cat(outs, dim=2).index_select(2, inverse)
    if not return_lse:
        return out
    return out, torch.cat(lses, dim=2).index_select(2, inverse)


def ring_attention_replay(scale, q_all, k_all, v_all, chunks, causal: bool = True,
                          return_lse: bool = False, stats: list | None = None):
    """Drive every domain of a vanilla (contiguous) split in one process.

    ``q_all`` [1,Hq,S,D], ``k_all``/``v_all`` [1,Hkv,S,D]; ``chunks`` are the per-domain
    lengths (must sum to S, ``reference_algo.rs:92-116``).  Domain d owns global
    positions ``[off_d, off_d + chunks[d])`` (strategy.rs:53-63).  Returns the
    concatenation of every domain's output along seq (and LSE when asked).
    """
    n = len(chunks)
    seq = q_all.shape[2]
    if sum(chunks) != seq:
        raise ValueError(f"chunk sum {sum(chunks)} != seq_len {seq}")
    num_rep = q_all.shape[1] // k_all.shape[1]
    offs = [sum(chunks[:i]) for i in range(n)]
    kx = repeat_kv_heads(k_all, num_rep)
    vx = repeat_kv_heads(v_all, num_rep)
    sent = []
    for d in range(n):
        s, e = offs[d], offs[d] + chunks[d]
        sent.append(local_micro_blocks(kx[:, :, s:e], vx[:, :, s:e], s, n))
    outs, lses = [], []
    for d in range(n):
        s, e = offs[d], offs[d] + chunks[d]
        rounds = [sent[(d - 1 - r) % n] for r in range(n - 1)]
        st = RingStats() if stats is not None else None
        res = ring_attention(scale, q_all[:, :, s:e], kx[:, :, s:e], vx[:, :, s:e],
                             torch.arange(s, e, dtype=torch.int64), s, n, rounds,
                             apply_causal=causal, return_lse=return_lse, stats=st)
        if stats is not None:
            stats.append(st)
        if return_lse:
            outs.append(res[0])
            lses.append(res[1])
        else:
            outs.append(res)
    out = torch.cat(outs, dim=2)
    return (out, torch.cat(lses, dim=2)) if return_lse else out


def causal_flops_executed(chunks, num_q_heads: int, head_dim: int) -> float:
    """FLOPs the blockwise path actually executes (full tiles, early exit only)."""
    n = len(chunks)
    offs = [sum(chunks[:i]) for i in range(n)]
    total = 0.0
    for d in range(n):
        qc, kc, _ = chunk_sizes(chunks[d], n)
        for src in range(n):
            _, skc, micro = chunk_sizes(chunks[src], n)
            blk = skc if src == d else micro
            for qs in range(0, chunks[d], qc):
                qe = min(qs + qc, chunks[d])
                qmax = offs[d] + qe - 1
                for ks in range(0, chunks[src], blk):
                    ke = min(ks + blk, chunks[src])
                    if offs[src] + ks > qmax:
                        continue
                    total += 4.0 * (qe - qs) * (ke - ks) * head_dim * num_q_heads
    return total


def mean_abs(x) -> float:
    return float(x.abs().mean())


def attention_scale(head_dim: int) -> float:
    """1/sqrt(D) (ring.rs:152, reference_algo.rs:130-132)."""
    return 1.0 / math.sqrt(head_dim)
