"""GPU parity tests: every kernel through the C ABI against the oracle on identical
seeded inputs.

Tolerances: attention outputs max-abs <= 2e-2, LSE (fp32)
max-abs <= 1e-3 against the same algorithm on exact fp32 upcasts of the bf16 inputs;
paged gather/scatter bit-exact.  The fp32 path is held to the reference's Relaxed tier
(1e-4, rust/src/error.rs:56-76).
"""
import math

import numpy as np
import pytest
import torch

import hcp_ring_amd as H
from oracle import clib, closed_form as C, inputs as I, tch_ring as T

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2
LSE_TOL = 1e-3


def dev_bits(bits: np.ndarray, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype).cuda()


def draw(seed, shapes, dtype):
    """Seeded inputs: (device tensors, fp32 upcasts as numpy)."""
    if dtype == torch.float32:
        arrs = clib.draw_normals(seed, shapes, "fp32")
        return [torch.from_numpy(a).cuda() for a in arrs], arrs
    if dtype == torch.float16:
        arrs = clib.draw_normals(seed, shapes, "fp32")
        t = [torch.from_numpy(a).to(torch.float16) for a in arrs]
        return [x.cuda() for x in t], [x.float().numpy() for x in t]
    bits = clib.draw_normals(seed, shapes, "bf16")
    return [dev_bits(b) for b in bits], [I.bf16_bits_to_f32(b) for b in bits]


def bhsd(x32):
    return torch.from_numpy(np.ascontiguousarray(x32)).permute(1, 0, 2).unsqueeze(0)


BLOCK_CASES = [
    # name, Lq, Lk, Hq, Hkv, D, q_off, k_off, causal, dtype
    ("diag_gqa4", 200, 200, 8, 2, 128, 0, 0, True, torch.bfloat16),
    ("full_past", 130, 250, 8, 2, 128, 300, 0, True, torch.bfloat16),
    ("partly_future", 200, 100, 8, 2, 128, 0, 50, True, torch.bfloat16),
    ("wholly_future", 64, 64, 4, 1, 128, 0, 1000, True, torch.bfloat16),
    ("noncausal", 100, 333, 4, 4, 128, 0, 0, False, torch.bfloat16),
    ("gqa8_qwen", 96, 517, 16, 2, 128, 600, 100, True, torch.bfloat16),
    ("mha_d64_f16", 300, 300, 4, 4, 64, 77, 77, True, torch.float16),
    ("diag_unaligned_offsets", 257, 260, 8, 8, 128, 1003, 1000, True, torch.bfloat16),
    # fp32: the fp32 matrix-core kernel (head dims multiples of 4 up to 128), else the
    # scalar general kernel (head dim 136)
    ("fp32_d64", 150, 150, 8, 8, 64, 0, 0, True, torch.float32),
    ("fp32_gqa4_d128_past", 200, 300, 8, 2, 128, 100, 0, True, torch.float32),
    ("fp32_d96_noncausal", 150, 260, 4, 4, 96, 0, 0, False, torch.float32),
    ("fp32_d36_partly_future", 200, 100, 6, 2, 36, 0, 50, True, torch.float32),
    ("fp32_d4_diag", 70, 90, 2, 1, 4, 20, 0, True, torch.float32),
    ("fp32_wholly_future", 64, 64, 4, 1, 128, 0, 1000, True, torch.float32),
    ("fp32_general_d136", 90, 120, 4, 2, 136, 30, 0, True, torch.float32),
    ("gqa2_long_noncausal", 160, 1000, 8, 4, 128, 0, 0, False, torch.bfloat16),
    ("gqa2_causal_long_past", 300, 1500, 4, 2, 128, 1200, 0, True, torch.bfloat16),
    # head dims below 128 run in the head-dim-128 kernel, zero-padded
    ("d96_padded_gqa4", 200, 300, 8, 2, 96, 0, 0, True, torch.bfloat16),
    ("d112_f16_noncausal", 150, 260, 4, 4, 112, 0, 0, False, torch.float16),
    ("d48_full_past", 130, 250, 4, 2, 48, 300, 0, True, torch.bfloat16),
    ("d8_diag", 70, 90, 2, 1, 8, 20, 0, True, torch.bfloat16),
    # GQA ratios that are not powers of two: Qwen2-0.5B (14 q / 2 kv heads, D=64: one
    # head per workgroup) and 6 at D=128 (two per workgroup)
    ("qwen2_0p5b_rep7_d64", 150, 300, 14, 2, 64, 150, 0, True, torch.bfloat16),
    ("gqa6_d128", 120, 260, 12, 2, 128, 140, 0, True, torch.bfloat16),
    # head dim 64 (the half-width instantiation: MFMAs on the first 64 dims of the
    # zero-padded 128-dim rows) across GQA ratios, causal offsets, fp16 without masking
    # and an odd KV head count
    ("d64_gqa4_causal_past", 300, 700, 16, 4, 64, 650, 0, True, torch.bfloat16),
    ("d64_rep8_two_groups", 96, 517, 16, 2, 64, 600, 100, True, torch.bfloat16),
    ("d64_rep2_noncausal_f16", 160, 1000, 8, 4, 64, 0, 0, False, torch.float16),
    ("d64_odd_kv_heads", 150, 260, 6, 3, 64, 140, 0, True, torch.bfloat16),
]


@pytest.mark.parametrize("case", BLOCK_CASES, ids=[c[0] for c in BLOCK_CASES])
def test_block_partial_matches_oracle(gpu, case):
    name, lq, lk, hq, hkv, d, qo, ko, causal, dt = case
    (q, k, v), (q32, k32, v32) = draw(len(name) * 7 + lq, [(lq, hq, d), (lk, hkv, d), (lk, hkv, d)], dt)
    scale = 1 / math.sqrt(d)
    o, lse = H.block_partial(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), qo, ko,
                             causal=causal, scale=scale)
    torch.cuda.synchronize()
    if dt == torch.float32:
        assert H.last_path() == ("mfma_f32" if d % 4 == 0 and d <= 128 else "general"), name
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    ref_o, ref_l = C.attention_f64(q32, k32, v32, np.arange(qo, qo + lq), np.arange(ko, ko + lk), scale,
                                   causal=causal)
    ref_o, ref_l = ref_o.transpose(1, 0, 2), ref_l.T
    assert np.array_equal(np.isneginf(lse), np.isneginf(ref_l))
    fin = np.isfinite(ref_l)
    tol = 1e-4 if dt == torch.float32 else OUT_TOL
    assert np.abs(o - ref_o).max() <= tol
    if fin.any():
        assert np.abs(lse[fin] - ref_l[fin]).max() <= (1e-4 if dt == torch.float32 else LSE_TOL)
    assert np.all(o[~fin] == 0)
    # the op-for-op restatement on fp32 upcasts agrees as well
    if causal:
        to, tl = T.positioned_local_compact_partial(scale, bhsd(q32), torch.arange(qo, qo + lq),
                                                    bhsd(k32), bhsd(v32), torch.arange(ko, ko + lk))
        tl = tl[0].numpy()
        assert np.abs(o - to[0].numpy()).max() <= tol
        if fin.any():
            assert np.abs(lse[fin] - tl[fin]).max() <= LSE_TOL


@pytest.mark.parametrize("d,causal,accumulate", [(128, True, False), (64, False, False), (96, True, True),
                                                (36, True, True)])
def test_fp32_matrix_core_kernel_matches_scalar_kernel(gpu, d, causal, accumulate):
    # The fp32 matrix-core kernel against the scalar general kernel on the same inputs:
    # an output that is not 16-byte aligned sends a block to the scalar one.  Accumulate:
    # both merge the same running state (a first source folded by the scalar kernel).
    lq, lk, hq, hkv = 170, 290, 8, 2
    (q, k, v), (q32, k32, v32) = draw(90 + d, [(lq, hq, d), (lk, hkv, d), (lk, hkv, d)], torch.float32)
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    outs = []
    for aligned in (True, False):
        buf = torch.empty(hq * lq * d + 4, dtype=torch.float32, device="cuda")
        o = (buf[:hq * lq * d] if aligned else buf[1:1 + hq * lq * d]).view(hq, lq, d)
        lse = torch.empty(hq, lq, dtype=torch.float32, device="cuda")
        if accumulate:
            H.block_partial(qh, kh[:, :100], vh[:, :100], 150, 0, causal=causal, o=o, lse=lse)
            assert H.last_path() == ("mfma_f32" if aligned else "general")
            H.block_partial(qh, kh[:, 100:], vh[:, 100:], 150, 100, causal=causal, o=o, lse=lse, accumulate=True)
        else:
            H.block_partial(qh, kh, vh, 150, 0, causal=causal, o=o, lse=lse)
        assert H.last_path() == ("mfma_f32" if aligned else "general")
        torch.cuda.synchronize()
        outs.append((o.cpu().numpy(), lse.cpu().numpy()))
    (o1, l1), (o2, l2) = outs
    assert np.abs(o1 - o2).max() <= 1e-5 and np.abs(l1 - l2).max() <= 1e-5
    ref_o, ref_l = C.attention_f64(q32, k32, v32, np.arange(150, 150 + lq), np.arange(lk), 1 / math.sqrt(d),
                                   causal=causal)
    assert np.abs(o1 - ref_o.transpose(1, 0, 2)).max() <= 1e-4
    assert np.abs(l1 - ref_l.T).max() <= 1e-4


def test_block_partial_head_major_and_unaligned_views(gpu):
    (q, k, v), (q32, k32, v32) = draw(5, [(96, 4, 130), (96, 4, 130), (96, 4, 130)], torch.bfloat16)
    # [L, H, 130] sliced to D=128: seq stride 520 is not a multiple of 8 -> general kernel.
    qs, ks, vs = (x[:, :, :128].permute(1, 0, 2) for x in (q, k, v))
    o1, l1 = H.block_partial(qs, ks, vs, 0, 0)
    # the same data head-major contiguous -> matrix-core kernel
    o2, l2 = H.block_partial(qs.contiguous(), ks.contiguous(), vs.contiguous(), 0, 0)
    torch.cuda.synchronize()
    ref_o, ref_l = C.attention_f64(q32[:, :, :128], k32[:, :, :128], v32[:, :, :128], np.arange(96),
                                   np.arange(96), 1 / math.sqrt(128))
    for o, l in ((o1, l1), (o2, l2)):
        assert np.abs(o.cpu().numpy() - ref_o.transpose(1, 0, 2)).max() <= OUT_TOL
        assert np.abs(l.cpu().numpy() - ref_l.T).max() <= LSE_TOL


@pytest.mark.parametrize("d", [128, 96], ids=["d128", "d96_padded"])
def test_block_partial_accumulate_is_positioned_merge(gpu, d):
    # ring.rs:574-603: (o, lse) of source A merged in place with source B; the running
    # fp32 state keeps the caller's head dim (96: rows of 96 floats) on the padded path.
    (q, k, v), (q32, k32, v32) = draw(11, [(150, 8, d), (400, 2, d), (400, 2, d)], torch.bfloat16)
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    o, l = H.positioned_local_compact_partial(qh, 300, kh[:, 250:], vh[:, 250:], 250)
    o2, l2 = H.positioned_merge_compact_partial(qh, 300, o, l, kh[:, :250], vh[:, :250], 0)
    torch.cuda.synchronize()
    ref_o, ref_l = C.attention_f64(q32, k32, v32, np.arange(300, 450), np.arange(400), 1 / math.sqrt(d))
    assert H.last_path() == "mfma"
    assert np.abs(o2.cpu().numpy() - ref_o.transpose(1, 0, 2)).max() <= OUT_TOL
    assert np.abs(l2.cpu().numpy() - ref_l.T).max() <= LSE_TOL


@pytest.mark.parametrize("h,l,n", [(8, 333, 5), (3, 37, 1), (1, 45, 2), (5, 21, 9)],
                         ids=["five_parts", "one_part_odd_rows", "two_parts_odd_rows", "nine_parts_two_groups"])
def test_lse_merge_matches_closed_form(gpu, h, l, n):
    # row counts h * l both even and odd (each thread merges two consecutive rows), and
    # part counts for every group size of the kernel (1, 2, 4, 8 and a second group)
    rng = np.random.default_rng(4 + n)
    d = 128
    os_ = [rng.standard_normal((h, l, d)).astype(np.float32) for _ in range(n)]
    ls = [rng.normal(3.0, 2.0, (h, l)).astype(np.float32) for _ in range(n)]
    e = n - 1                     # an empty partial on some rows
    ls[e][:, : l // 3] = -np.inf
    os_[e][:, : l // 3] = 0
    dead = l // 2                 # a row with no keys at all
    for x in ls:
        x[0, dead] = -np.inf
    for x in os_:
        x[0, dead] = 0
    out, lse = H.lse_merge([torch.from_numpy(x).cuda() for x in os_], [torch.from_numpy(x).cuda() for x in ls],
                           out_dtype=torch.bfloat16)
    out32, lse32 = H.lse_merge([torch.from_numpy(x).cuda() for x in os_], [torch.from_numpy(x).cuda() for x in ls],
                               out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref_o, ref_l = C.merge_partials_f64(os_, ls)
    assert np.abs(out32.cpu().numpy() - ref_o).max() < 1e-5
    # bf16 output: within one bf16 rounding (relative 2^-8) of the f64 merge
    assert np.all(np.abs(out.float().cpu().numpy() - ref_o) <= np.abs(ref_o) * 2.0**-8 + 1e-6)
    lse = lse.cpu().numpy()
    assert lse[0, dead] == -np.inf and np.all(out.float().cpu().numpy()[0, dead] == 0)
    fin = np.isfinite(ref_l)
    assert np.abs(lse[fin] - ref_l[fin]).max() < 1e-5


def test_bf16_output_rounding_is_round_to_nearest_even(gpu):
    # A one-part merge is the identity (weight exp(0) / 1 = 1 exactly), so its bf16 output
    # is the kernels' shared fp32 -> bf16 rounding of the input, checked bit for bit
    # against round-to-nearest-even on the bits: ties (low half 0x8000) with even and odd
    # kept mantissas, carries into the next binade, the largest finite values (to inf) and
    # infinities.  Inputs are normal or infinite, so the result does not depend on the
    # kernel's denormal mode; -0 is left out (0 + 1 * -0 is +0).
    rng = np.random.default_rng(6)
    h, l, d = 2, 256, 128
    bits = rng.integers(0, 2**32, h * l * d, dtype=np.uint64).astype(np.uint32)
    bits[1::3] = (bits[1::3] & 0xFFFF0000) | 0x8000
    special = np.array([0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F808001, 0x3FFF8000, 0x3FFFFFFF, 0x7F7FFFFF,
                        0x7F7F8000, 0x7F7F7FFF, 0xFF7FFFFF, 0xFF7F8000, 0x7F800000, 0xFF800000, 0x00800000,
                        0x80808000, 0x477FE000, 0x3F800000], dtype=np.uint32)
    bits[: special.size] = special
    expo = bits & 0x7F800000
    bits[expo == 0] |= 0x00800000                                   # no zeros or denormals
    bits[(expo == 0x7F800000) & ((bits & 0x007FFFFF) != 0)] &= 0xFF800000   # NaN -> inf
    o = bits.view(np.float32).reshape(h, l, d)
    lse = rng.standard_normal((h, l)).astype(np.float32)
    out, _ = H.lse_merge([torch.from_numpy(o).cuda()], [torch.from_numpy(lse).cuda()], out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    u = bits.astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(int(bits[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:5]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_gather_scatter_bit_exact(gpu, dtype):
    nb, bs, hkv, d = 96, 16, 8, 128
    rng = np.random.default_rng(6)
    if dtype == torch.bfloat16:
        pool_np = rng.integers(0, 2**16, size=(2, nb, bs, hkv, d), dtype=np.uint16)
        pool = torch.from_numpy(pool_np.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        pool_np = rng.standard_normal((2, nb, bs, hkv, d)).astype(np.float32)
        pool = torch.from_numpy(pool_np).cuda()
    table_np = I.permuted_block_table(7, nb)[:40]
    table = torch.from_numpy(table_np).cuda()
    off, t0, t1 = 32, 45, 590  # unaligned range, table starting at global position 32
    k, v = H.paged_kv_gather(pool, table, off, t0, t1)
    torch.cuda.synchronize()
    rk, rv = clib.paged_gather(pool_np, table_np, off, t0, t1)
    view_np = lambda x: x.cpu().view(torch.int16 if dtype == torch.bfloat16 else torch.int32).numpy()
    assert np.array_equal(view_np(k), rk.view(np.int16 if dtype == torch.bfloat16 else np.int32))
    assert np.array_equal(view_np(v), rv.view(np.int16 if dtype == torch.bfloat16 else np.int32))
    # scatter new data back (zero tail) and compare the whole pool with the oracle's scatter
    k2 = torch.flip(k, dims=[1]).contiguous()
    v2 = torch.flip(v, dims=[1]).contiguous()
    H.paged_kv_scatter(pool, table, off, t0, t1, k2, v2, zero_tail=True)
    torch.cuda.synchronize()
    clib.paged_scatter(pool_np, table_np, off, t0, t1, _np_bits(k2), _np_bits(v2), zero_tail=True)
    assert np.array_equal(_np_bits(pool), pool_np)
    # gather(scatter(x)) == x
    k3, v3 = H.paged_kv_gather(pool, table, off, t0, t1)
    assert np.array_equal(_np_bits(k3), _np_bits(k2)) and np.array_equal(_np_bits(v3), _np_bits(v2))
    # a sub-range in the middle without the zero tail leaves every other slot alone
    k4 = torch.roll(k2, 3, dims=1)[:, :100].contiguous()
    v4 = torch.roll(v2, 5, dims=1)[:, :100].contiguous()
    H.paged_kv_scatter(pool, table, off, t0 + 7, t0 + 107, k4, v4, zero_tail=False)
    torch.cuda.synchronize()
    clib.paged_scatter(pool_np, table_np, off, t0 + 7, t0 + 107, _np_bits(k4), _np_bits(v4), zero_tail=False)
    assert np.array_equal(_np_bits(pool), pool_np)
    assert H.fetch_device_errors() == 0


def _np_bits(t):
    if t.dtype == torch.bfloat16:
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


def test_paged_gather_strided_ring_buffer(gpu):
    # gather straight into a token-major [L, Hkv, D] buffer (a strided [Hkv, L, D] view)
    nb, bs, hkv, d = 16, 16, 4, 64
    rng = np.random.default_rng(9)
    pool_np = rng.integers(0, 2**16, size=(2, nb, bs, hkv, d), dtype=np.uint16)
    pool = torch.from_numpy(pool_np.view(np.int16)).view(torch.bfloat16).cuda()
    table_np = I.permuted_block_table(3, nb)
    table = torch.from_numpy(table_np).cuda()
    buf_k = torch.zeros(200, hkv, d, dtype=torch.bfloat16, device="cuda")
    buf_v = torch.zeros(200, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.paged_kv_gather(pool, table, 0, 10, 210, buf_k.permute(1, 0, 2), buf_v.permute(1, 0, 2))
    torch.cuda.synchronize()
    rk, rv = clib.paged_gather(pool_np, table_np, 0, 10, 210)
    assert np.array_equal(_np_bits(buf_k.permute(1, 0, 2).contiguous()), rk)
    assert np.array_equal(_np_bits(buf_v.permute(1, 0, 2).contiguous()), rv)


def test_paged_bad_block_id_sets_device_flag(gpu):
    pool = torch.zeros(2, 8, 16, 2, 64, dtype=torch.bfloat16, device="cuda")
    table = torch.tensor([0, 99, 1], dtype=torch.int32, device="cuda")
    H.fetch_device_errors()
    k, v = H.paged_kv_gather(pool, table, 0, 0, 48)
    assert H.fetch_device_errors() & 1
    assert H.fetch_device_errors() == 0


DECODE_CASES = [
    # name, B, Hq, Hkv, D, bs, ctx, t0, t1, ragged
    ("c4_shape_small", 4, 32, 8, 128, 16, 1024, 0, 1024, False),
    ("middle_chunk", 3, 32, 8, 128, 16, 900, 320, 700, False),
    ("ragged_lens", 5, 16, 4, 128, 32, 600, 100, 600, True),
    ("d64_bs16", 2, 8, 2, 64, 16, 300, 7, 290, False),
    # the reference's own models: Qwen2-0.5B (14 q / 2 kv, D=64: seven query heads per
    # KV head, two waves per workgroup) and Qwen2.5-3B (16 q / 2 kv, D=128: eight)
    ("qwen2_0p5b_rep7_d64", 3, 14, 2, 64, 16, 700, 0, 700, False),
    ("qwen25_3b_rep8_d128", 4, 16, 2, 128, 16, 1000, 64, 1000, True),
    ("rep16_one_kv_head", 2, 16, 1, 128, 32, 500, 0, 500, False),
    ("rep12_three_kv_heads", 2, 36, 3, 64, 16, 333, 5, 333, False),
    # head dims other than 64 and 128: the D=128 kernel with zero-padded columns
    ("d96_padded", 3, 32, 8, 96, 16, 700, 30, 700, True),
    ("d80_rep5", 2, 10, 2, 80, 32, 450, 0, 450, False),
    ("d32_rep4", 2, 8, 2, 32, 16, 260, 0, 260, False),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_paged_decode_matches_oracle(gpu, case):
    name, b, hq, hkv, d, bs, ctx, t0, t1, ragged = case
    nblk_seq = (ctx + bs - 1) // bs
    nb = b * nblk_seq + 3
    (q, kv), (q32, kv32) = draw(31 + b, [(b, hq, d), (2, nb, bs, hkv, d)], torch.bfloat16)
    perm = I.permuted_block_table(40 + b, nb)
    tables_np = perm[: b * nblk_seq].reshape(b, nblk_seq)
    tables = torch.from_numpy(np.ascontiguousarray(tables_np)).cuda()
    lens_np = np.array([ctx - 37 * i for i in range(b)], dtype=np.int32) if ragged else None
    lens = torch.from_numpy(lens_np).cuda() if ragged else None
    o, lse = H.decode_local_compact_partial(q, kv, tables, t0, t1, seq_lens=lens)
    torch.cuda.synchronize()
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    scale = 1 / math.sqrt(d)
    for i in range(b):
        end = min(t1, int(lens_np[i])) if ragged else t1
        kk, vv = clib.paged_gather(kv32, tables_np[i], 0, t0, end)
        ref_o, ref_l = C.attention_f64(q32[i:i + 1], kk.transpose(1, 0, 2), vv.transpose(1, 0, 2),
                                       np.zeros(1), np.zeros(end - t0), scale, causal=False)
        assert np.abs(o[i] - ref_o[0]).max() <= OUT_TOL, name
        assert np.abs(lse[i] - ref_l[0]).max() <= LSE_TOL, name
        # op-for-op decode restatement (ring.rs:625-639) on fp32 upcasts
        to, tl = T.decode_local_compact_partial(scale, bhsd(q32[i:i + 1]), bhsd(kk.transpose(1, 0, 2)),
                                                bhsd(vv.transpose(1, 0, 2)))
        assert np.abs(lse[i] - tl[0, :, 0].numpy()).max() <= LSE_TOL


def test_synth_normals_match_oracle_generator(gpu):
    for dtype, kind in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        n = 100_003
        out = torch.empty(n, dtype=dtype, device="cuda")
        H.synth_normals(44, 0, n, out)
        part = torch.empty(1001, dtype=dtype, device="cuda")
        H.synth_normals(44, 5001, 1001, part)  # odd offset: starts on a spare
        torch.cuda.synchronize()
        ref, = clib.draw_normals(44, [(n,)], kind)
        got = _np_bits(out) if dtype == torch.bfloat16 else out.cpu().numpy()
        mism = np.count_nonzero(got != ref)
        assert mism <= n * 1e-4, mism  # device libm may differ from glibc in the last f64 ulp
        assert torch.equal(part, out[5001:6002])


RING_CASES = [
    ("c1_fp32", [640, 384], 8, 8, 64, torch.float32, 42),
    ("c2_small", [512, 320, 192], 16, 2, 128, torch.bfloat16, 43),
    ("uneven4", [300, 77, 500, 123], 8, 2, 128, torch.bfloat16, 50),
    # 10 domains: the first ring steps hold 10 blocks, launched as groups of 8 + 2
    ("ten_domains", [200, 64, 130, 96, 300, 50, 128, 77, 256, 99], 8, 2, 128, torch.bfloat16, 51),
    # head ratios 1, 3 (one head per workgroup), 6 (two) and 8, chunks off the 128-key
    # tile grid so past sources straddle tiles and end in partial ones
    ("mha_unaligned", [190, 333, 61], 4, 4, 128, torch.bfloat16, 52),
    ("gqa3_fp16", [257, 129, 400], 6, 2, 128, torch.float16, 53),
    ("gqa6", [96, 450, 200], 12, 2, 128, torch.bfloat16, 54),
    ("gqa8_two_domains", [1000, 536], 16, 2, 128, torch.bfloat16, 55),
    ("single_domain", [700], 8, 2, 128, torch.bfloat16, 56),
    # zero-padded head dims in the fused ring and the per-step kernel
    ("d96_padded", [300, 200, 133], 8, 2, 96, torch.bfloat16, 58),
    ("d80_f16", [150, 260], 4, 4, 80, torch.float16, 59),
    ("d32_gqa4", [200, 100, 64], 8, 2, 32, torch.bfloat16, 60),
    # the reference's own model shape (Qwen2-0.5B: 14 q / 2 kv heads, D=64, GQA 7) and a
    # D=64 fp16 multi-head case
    ("qwen2_0p5b_d64", [320, 200, 136], 14, 2, 64, torch.bfloat16, 61),
    ("mha_d64_f16", [257, 190], 6, 6, 64, torch.float16, 62),
    ("d64_gqa4_uneven4", [300, 77, 500, 123], 16, 4, 64, torch.bfloat16, 63),
    ("d64_odd_kv_padded", [200, 150], 3, 3, 64, torch.bfloat16, 64),
]


@pytest.mark.parametrize("schedule", ["auto", "per_step"])
@pytest.mark.parametrize("case", RING_CASES, ids=[c[0] for c in RING_CASES])
def test_ring_replay_matches_tch_blockwise(gpu, case, schedule):
    name, chunks, hq, hkv, d, dt, seed = case
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(seed, [(s, hq, d), (s, hkv, d), (s, hkv, d)], dt)
    scale = 1 / math.sqrt(d)
    out, lse = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks,
                                       schedule=schedule)
    torch.cuda.synchronize()
    # BF16/F16 at head dims that are multiples of 8 up to 128 take the fused ring kernel
    # unless a per-step schedule is asked for
    fused = dt != torch.float32 and d % 8 == 0 and d <= 128 and schedule == "auto"
    assert H.last_path() == ("ring_fused" if fused else "mfma_f32" if dt == torch.float32 else "mfma")
    if dt == torch.float32 and schedule == "auto":
        # fp32 (c1): the whole replay as one block on the fp32 matrix-core kernel
        H.replay_timing(True)
        H.replay_timing_read()
        H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks)
        assert H.replay_timing_read()["block"][1] == 1
        H.replay_timing(False)
    out = out.float().cpu().numpy()
    lse = lse.cpu().numpy()
    # the reference driver on fp32 upcasts (ring.rs:861-1398 restated op for op)
    ro, rl = T.ring_attention_replay(scale, bhsd(q32), bhsd(k32), bhsd(v32), chunks, return_lse=True)
    ro, rl = ro[0].numpy(), rl[0].numpy()
    if dt == torch.float32:
        assert np.abs(out - ro).max() <= 1e-4 and np.abs(out - ro).mean() <= 1e-5
        assert np.abs(lse - rl).max() <= 1e-4
    else:
        assert np.abs(out - ro).max() <= OUT_TOL
        assert np.abs(lse - rl).max() <= LSE_TOL
        # and the reference's own dtype (bf16 state): at least as close to the fp32
        # restatement as that path is, and within the bf16 output tolerance of it whenever
        # it is itself within that tolerance of the fp32 result (its bf16 state drifts by
        # 0.013-0.022 on these cases: 0.022 at d96_padded, where ours is 0.007 off)
        rb = T.ring_attention_replay(scale, bhsd(q32).to(torch.bfloat16), bhsd(k32).to(torch.bfloat16),
                                     bhsd(v32).to(torch.bfloat16), chunks)[0].float().numpy()
        err_rb = np.abs(rb - ro).max()
        assert np.abs(out - ro).max() <= err_rb
        if err_rb <= OUT_TOL:
            assert np.abs(out - rb).max() <= OUT_TOL


@pytest.mark.parametrize("schedule,d", [("auto", 128), ("per_step", 128), ("fused", 128), ("fused", 96)])
def test_ring_replay_paged_matches_unpaged(gpu, schedule, d):
    chunks = [256, 96, 160]
    s, hq, hkv, bs = sum(chunks), 8, 2, 16
    (q, k, v), _ = draw(77, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.bfloat16)
    nb = s // bs + 5
    table_np = I.permuted_block_table(78, nb)[: s // bs]
    table = torch.from_numpy(table_np).cuda()
    pool = torch.zeros(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.paged_kv_scatter(pool, table, 0, 0, s, k.permute(1, 0, 2), v.permute(1, 0, 2))
    o1, l1 = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks,
                                     schedule=schedule)
    # the fused schedule needs no workspace unpaged, and only the two staging buffers paged
    if schedule == "fused":
        assert H.replay_workspace_size(torch.bfloat16, hq, hkv, d, chunks, schedule="fused") == 0
        assert H.replay_workspace_size(torch.bfloat16, hq, hkv, d, chunks, paged=True, schedule="fused") == \
            2 * ((s * hkv * d * 2 + 255) // 256 * 256)
    o2, l2 = H.ring_attention_replay_paged(q.permute(1, 0, 2), pool, table, chunks, schedule=schedule)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 96)])
def test_ring_replay_8_byte_aligned_output_takes_the_per_step_schedule(gpu, dtype, d):
    # The fused schedule stores final rows 16 bytes at a time and so takes only 16-byte
    # aligned outputs: an output whose rows are 8- but not 16-byte aligned (row stride
    # D + 4 elements, base offset 4) is refused there, and "auto" replays it per step.
    chunks = [256, 96, 160]
    s, hq, hkv = sum(chunks), 8, 2
    (q, k, v), _ = draw(79, [(s, hq, d), (s, hkv, d), (s, hkv, d)], dtype)
    args = (q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks)
    o1, l1 = H.ring_attention_replay(*args, schedule="fused")
    buf = torch.zeros(hq, s, d + 4, dtype=dtype, device="cuda")
    out = buf[:, :, 4:]
    assert out.data_ptr() % 16 == 8
    with pytest.raises(H.HcpRingError, match="16-byte"):
        H.ring_attention_replay(*args, schedule="fused", out=out)
    o2, l2 = H.ring_attention_replay(*args, schedule="auto", out=out)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert (o1.float() - o2.float()).abs().max().item() <= OUT_TOL
    assert (l1 - l2).abs().max().item() <= LSE_TOL
    assert not buf[:, :, :4].any()


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 128), (6, 2, 128), (16, 2, 128), (8, 2, 80)])
def test_ring_replay_fused_noncausal_wraps_round_the_ring(gpu, hq, hkv, d):
    # Without causal masking every domain folds every source; after source 0 the ring
    # wraps to N-1, ..., t+1 (rows [off_t + len_t, S) read from the top down).
    chunks = [200, 333, 150, 90]
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(57, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.bfloat16)
    scale = 1 / math.sqrt(d)
    outs = {}
    for sched in ("fused", "per_step"):
        outs[sched] = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks,
                                              causal=False, schedule=sched)
    torch.cuda.synchronize()
    pos = np.arange(s)
    ro, rl = C.attention_f64(q32, k32, v32, pos, pos, scale, causal=False)
    for sched, (o, l) in outs.items():
        assert np.abs(o.float().cpu().numpy() - ro.transpose(1, 0, 2)).max() <= OUT_TOL, sched
        assert np.abs(l.cpu().numpy() - rl.T).max() <= LSE_TOL, sched


def test_ring_replay_fused_rejects_what_it_cannot_run(gpu):
    chunks, d = [64, 64], 128
    s = sum(chunks)
    q = torch.zeros(8, s, d, dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros(2, s, d, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(H.HcpRingError) as e:   # fp32 beyond the fp32 matrix-core kernel's head dims
        q132 = torch.zeros(8, s, 132, device="cuda")
        kv132 = torch.zeros(2, s, 132, device="cuda")
        H.ring_attention_replay(q132, kv132, kv132, chunks, schedule="fused")
    assert e.value.code == -6
    with pytest.raises(H.HcpRingError) as e:   # rows not on 16-byte boundaries
        qq = torch.zeros(8, s, d + 4, dtype=torch.bfloat16, device="cuda")[:, :, 4:]
        H.ring_attention_replay(qq, kv, kv, chunks, schedule="fused")
    assert e.value.code == -6
    # AUTO falls back to the per-step kernels for such views, and says so
    H.ring_attention_replay(qq, kv, kv, chunks)
    assert H.last_path() == "general"


def test_paged_gather_batch_bit_exact(gpu):
    # several ranges (different tables, offsets and unaligned bounds) in one launch
    nb, bs, hkv, d = 128, 16, 8, 128
    rng = np.random.default_rng(12)
    pool_np = rng.integers(0, 2**16, size=(2, nb, bs, hkv, d), dtype=np.uint16)
    pool = torch.from_numpy(pool_np.view(np.int16)).view(torch.bfloat16).cuda()
    perm = I.permuted_block_table(13, nb)
    specs = [(perm[:30], 0, 0, 480), (perm[30:70], 64, 70, 600), (perm[70:90], 0, 5, 5), (perm[90:128], 16, 17, 610)]
    ranges, refs = [], []
    for tab, off, t0, t1 in specs:
        ko = torch.zeros(hkv, t1 - t0, d, dtype=torch.bfloat16, device="cuda")
        vo = torch.zeros_like(ko)
        ranges.append((torch.from_numpy(np.ascontiguousarray(tab)).cuda(), off, t0, t1, ko, vo))
        refs.append(clib.paged_gather(pool_np, tab, off, t0, t1) if t1 > t0 else None)
    H.paged_kv_gather_batch(pool, ranges)
    torch.cuda.synchronize()
    for (tab, off, t0, t1, ko, vo), ref in zip(ranges, refs):
        if ref is None:
            continue
        assert np.array_equal(_np_bits(ko), ref[0]) and np.array_equal(_np_bits(vo), ref[1])
    assert H.fetch_device_errors() == 0


DECODE_RING_CASES = [
    # name, prefill chunk per domain, decode steps per sequence, Hq, Hkv, D, block_size
    ("three_domains_uneven", [300, 200, 200], [5, 9, 2], 16, 4, 128, 16),
    ("four_domains_one_empty", [160, 96, 64, 0], [0, 1, 2], 8, 2, 64, 32),
    ("four_domains_ragged_zero", [160, 96, 64, 0], [1, 2, 3], 32, 8, 128, 16),
    ("qwen2_0p5b_rep7", [200, 120, 90], [3, 4], 14, 2, 64, 16),
    ("qwen25_3b_rep8", [256, 100], [2, 5, 1], 16, 2, 128, 16),
    ("d96_padded", [200, 150], [3, 2], 16, 4, 96, 16),
]


@pytest.mark.parametrize("case", DECODE_RING_CASES, ids=[c[0] for c in DECODE_RING_CASES])
def test_decode_ring_growth_sharding(gpu, case):
    """ring_decode_attention (ring.rs:665-818) over growth-sharded paged shards: every
    seed gives full-KV attention of the new token, and matches the oracle's journey."""
    name, chunks, steps, hq, hkv, d, bs = case
    n, b = len(chunks), len(steps)
    prefill = sum(chunks)
    starts = np.concatenate([[0], np.cumsum(chunks)])
    pos = [prefill + s for s in steps]            # the new token's global position
    total = max(pos) + 1
    (q, k_all, v_all), (q32, k32, v32) = draw(70 + n, [(b, hq, d), (b, total, hkv, d), (b, total, hkv, d)],
                                               torch.bfloat16)
    # shard[dom][i] = global positions domain dom holds for sequence i, the new token
    # included at its owner (update_sharded keep = true appends before attention)
    shard = [[list(range(starts[dom], starts[dom + 1])) +
              [p for p in range(prefill, pos[i] + 1) if H.decode_ring_owner(p, n) == dom] for i in range(b)]
             for dom in range(n)]
    nblk = [[-(-len(shard[dom][i]) // bs) for i in range(b)] for dom in range(n)]
    nb = sum(map(sum, nblk)) + 3
    perm = I.permuted_block_table(80 + n, nb)
    pool = torch.zeros((2, nb, bs, hkv, d), dtype=torch.bfloat16)
    kc, vc = k_all.cpu(), v_all.cpu()
    shards, cursor = [], 0
    for dom in range(n):
        width = max(max(nblk[dom]), 1)
        tab = np.full((b, width), -1, dtype=np.int32)   # ragged padding is never read
        for i in range(b):
            tab[i, :nblk[dom][i]] = perm[cursor:cursor + nblk[dom][i]]
            cursor += nblk[dom][i]
            for j, p in enumerate(shard[dom][i]):
                pool[0, tab[i, j // bs], j % bs] = kc[i, p]
                pool[1, tab[i, j // bs], j % bs] = vc[i, p]
        lens = [len(shard[dom][i]) for i in range(b)]
        max_len = max(lens)
        shards.append((torch.from_numpy(tab).cuda() if max_len else None,
                       torch.tensor(lens, dtype=torch.int32).cuda(), max_len))
    pool = pool.cuda()
    scale = 1 / math.sqrt(d)
    for seed in range(n):
        out, lse = H.decode_ring_replay(q, pool, shards, seed)
        torch.cuda.synchronize()
        out, lse = out.float().cpu().numpy(), lse.cpu().numpy()
        assert H.fetch_device_errors() == 0
        for i in range(b):
            kp, vp = k32[i, :pos[i] + 1], v32[i, :pos[i] + 1]
            ref_o, ref_l = C.attention_f64(q32[i:i + 1], kp, vp, np.zeros(1), np.zeros(pos[i] + 1), scale,
                                           causal=False)
            assert np.abs(out[i] - ref_o[0]).max() <= OUT_TOL, (name, seed, i)
            assert np.abs(lse[i] - ref_l[0]).max() <= LSE_TOL, (name, seed, i)
            # the oracle's journey on fp32 upcasts: durable shards without the new token
            durable = []
            for dom in range(n):
                idx = [p for p in shard[dom][i] if p != pos[i]]
                durable.append((bhsd(k32[i, idx]), bhsd(v32[i, idx])))
            cur = pos[i]
            to, tl = T.ring_decode_attention(scale, bhsd(q32[i:i + 1]), durable, bhsd(k32[i, cur:cur + 1]),
                                             bhsd(v32[i, cur:cur + 1]), seed)
            assert np.abs(out[i] - to[0, :, 0].numpy()).max() <= OUT_TOL, (name, seed, i)
            assert np.abs(lse[i] - tl[0, :, 0].numpy()).max() <= LSE_TOL, (name, seed, i)


def test_decode_ring_rejects_bad_seed_and_owner(gpu):
    q = torch.zeros(1, 4, 64, dtype=torch.bfloat16, device="cuda")
    pool = torch.zeros(2, 2, 16, 1, 64, dtype=torch.bfloat16, device="cuda")
    tab = torch.zeros(1, 1, dtype=torch.int32, device="cuda")
    with pytest.raises(H.HcpRingError):
        H.decode_ring_replay(q, pool, [(tab, None, 4), (tab, None, 4)], 2)
    with pytest.raises(H.HcpRingError):
        H.decode_ring_owner(5, 0)


def _strategy_rows(chunks, strategy):
    from oracle import strategy as SP
    a = SP.build_assignment(chunks, strategy)
    pos = SP.build_domain_positions(a)
    return pos, np.array(SP.build_inverse_perm(a))


POSITIONED_CASES = [
    # name, Lq, Lk, Hq, Hkv, D, dtype, position pattern
    ("striped_peer_d128", 300, 200, 8, 2, 128, torch.bfloat16, "striped"),
    ("zigzag_local_d128", 320, 320, 8, 2, 128, torch.bfloat16, "zigzag_local"),
    ("gaps_unsorted_q_d128", 257, 333, 16, 2, 128, torch.bfloat16, "gaps"),
    ("striped_d64_f16", 200, 300, 4, 4, 64, torch.float16, "striped_rev"),
    ("gaps_fp32", 150, 190, 4, 2, 64, torch.float32, "gaps"),
    # keys in any order (ring.rs:249-273 masks key by key; the committed-KV slab appends
    # positions in arrival order, self_driving.rs:180-224): sorted on the device first
    ("shuffled_gqa4_d128", 300, 1500, 16, 4, 128, torch.bfloat16, "shuffled"),        # one sort tile
    ("shuffled_5k_merge_passes", 200, 5000, 8, 2, 128, torch.bfloat16, "shuffled"),  # 3 tiles, 2 merge passes
    ("arrival_runs_9k", 256, 9000, 8, 1, 128, torch.bfloat16, "runs"),               # 5 tiles, 3 passes
    ("shuffled_ties_d64_f16", 180, 1200, 4, 2, 64, torch.float16, "ties"),
    ("shuffled_fp32", 150, 1100, 4, 2, 64, torch.float32, "shuffled"),
]


def _positions(pattern, lq, lk, seed):
    rng = np.random.default_rng(seed)
    if pattern == "striped":        # target domain 0, source domain 1 of a striped split
        pos, _ = _strategy_rows([lq, lk], "striped")
        return np.array(pos[0]), np.array(pos[1])
    if pattern == "striped_rev":    # target domain 1, source domain 0
        pos, _ = _strategy_rows([lk, lq], "striped")
        return np.array(pos[1]), np.array(pos[0])
    if pattern == "zigzag_local":   # a zigzag domain against its own keys
        pos, _ = _strategy_rows([lq, 2 * lq, lq], "zigzag")
        return np.array(pos[0]), np.array(pos[0])
    qp = rng.choice(4 * (lq + lk), size=lq, replace=False)          # any order
    if pattern == "shuffled":       # keys in any order
        return qp, rng.choice(4 * (lq + lk), size=lk, replace=False)
    if pattern == "ties":           # any order, many equal key positions
        return qp, rng.integers(0, 2 * (lq + lk), size=lk)
    if pattern == "runs":           # sorted runs concatenated in arrival order, overlapping ranges
        cuts = np.sort(rng.choice(np.arange(1, lk), size=6, replace=False))
        return qp, np.concatenate([np.sort(r) for r in np.split(rng.choice(4 * (lq + lk), size=lk,
                                                                           replace=False), cuts)])
    kp = np.sort(rng.choice(4 * (lq + lk), size=lk, replace=False))  # non-decreasing
    return qp, kp


@pytest.mark.parametrize("case", POSITIONED_CASES, ids=[c[0] for c in POSITIONED_CASES])
def test_block_partial_positioned_matches_closed_form(gpu, case):
    name, lq, lk, hq, hkv, d, dt, pattern = case
    qp, kp = _positions(pattern, lq, lk, lq + lk)
    (q, k, v), (q32, k32, v32) = draw(lq * 3 + lk, [(lq, hq, d), (lk, hkv, d), (lk, hkv, d)], dt)
    scale = 1 / math.sqrt(d)
    qpt, kpt = torch.from_numpy(qp.astype(np.int64)).cuda(), torch.from_numpy(kp.astype(np.int64)).cuda()
    o, lse = H.positioned_local_compact_partial(q.permute(1, 0, 2), qpt, k.permute(1, 0, 2), v.permute(1, 0, 2),
                                                kpt)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    ref_o, ref_l = C.attention_f64(q32, k32, v32, qp, kp, scale)
    ref_o, ref_l = ref_o.transpose(1, 0, 2), ref_l.T
    assert np.array_equal(np.isneginf(lse), np.isneginf(ref_l)), name
    fin = np.isfinite(ref_l)
    tol = 1e-4 if dt == torch.float32 else OUT_TOL
    assert np.abs(o - ref_o).max() <= tol, name
    assert np.abs(lse[fin] - ref_l[fin]).max() <= (1e-4 if dt == torch.float32 else LSE_TOL), name
    assert np.all(o[~fin] == 0)
    # op-for-op restatement with the same position tensors (ring.rs:538-571)
    to, tl = T.positioned_local_compact_partial(scale, bhsd(q32), torch.from_numpy(qp.astype(np.int64)),
                                                T.repeat_kv_heads(bhsd(k32), hq // hkv),
                                                T.repeat_kv_heads(bhsd(v32), hq // hkv),
                                                torch.from_numpy(kp.astype(np.int64)))
    assert np.abs(o - to[0].numpy()).max() <= tol, name


@pytest.mark.parametrize("dt,d", [(torch.float32, 4), (torch.bfloat16, 128)])
def test_positioned_partial_committed_kv_positions(gpu, dt, d):
    # The reference's own case (ring.rs:2247-2370, ring_forward_uses_independent_query_and_
    # committed_kv_positions): queries at positions [3, 5] against committed keys at
    # [0, 4, 3, 5] -- key 4 lies in query 3's future although it precedes key 3 in the
    # list.  fp32 head dim 4 (the test's shape, fp32 matrix-core kernel) and bf16 head dim 128.
    qp, kp = np.array([3, 5]), np.array([0, 4, 3, 5])
    (q, k, v), (q32, k32, v32) = draw(2343 + d, [(2, 1, d), (4, 1, d), (4, 1, d)], dt)
    scale = 1 / math.sqrt(d)
    t = lambda a: torch.tensor(a, dtype=torch.int64, device="cuda")
    o, lse = H.positioned_local_compact_partial(q.permute(1, 0, 2), t(qp), k.permute(1, 0, 2), v.permute(1, 0, 2),
                                                t(kp))
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    ref_o, ref_l = C.attention_f64(q32, k32, v32, qp, kp, scale)
    tol_o, tol_l = (1e-5, 1e-5) if dt == torch.float32 else (OUT_TOL, LSE_TOL)
    assert np.abs(o.cpu().numpy() - ref_o.transpose(1, 0, 2)).max() <= tol_o
    assert np.abs(lse.cpu().numpy() - ref_l.T).max() <= tol_l
    # a prefix reading of the list (keys [0, 4, 3] for query 3) differs from the answer
    wrong_o, _ = C.attention_f64(q32[:1], k32[:3], v32[:3], qp[:1], np.array([0, 3, 3]), scale)
    assert np.abs(wrong_o[0] - ref_o[0]).max() > 10 * tol_o
    to, tl = T.positioned_local_compact_partial(scale, bhsd(q32), torch.from_numpy(qp), bhsd(k32), bhsd(v32),
                                                torch.from_numpy(kp))
    assert np.abs(o.cpu().numpy() - to[0].numpy()).max() <= tol_o
    assert np.abs(lse.cpu().numpy() - tl[0].numpy()).max() <= tol_l


def test_positioned_merge_keys_in_any_order(gpu):
    # positioned_merge_compact_partial (ring.rs:574-603) with shuffled keys on both
    # sides: local partial over one half of a shuffled 2000-key list, merged with the
    # other half, equals attention over the whole list (GQA 4, D=128, bf16).
    lq, lk, hq, hkv, d = 260, 2000, 16, 4, 128
    rng = np.random.default_rng(7)
    qp = rng.choice(3 * lk, size=lq, replace=False)
    kp = rng.choice(3 * lk, size=lk, replace=False)
    (q, k, v), (q32, k32, v32) = draw(2024, [(lq, hq, d), (lk, hkv, d), (lk, hkv, d)], torch.bfloat16)
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    t = lambda a: torch.tensor(a, dtype=torch.int64, device="cuda")
    h = 1100
    o, l = H.positioned_local_compact_partial(qh, t(qp), kh[:, :h], vh[:, :h], t(kp[:h]))
    o, l = H.positioned_merge_compact_partial(qh, t(qp), o, l, kh[:, h:], vh[:, h:], t(kp[h:]))
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    scale = 1 / math.sqrt(d)
    ref_o, ref_l = C.attention_f64(q32, k32, v32, qp, kp, scale)
    fin = np.isfinite(ref_l.T)
    o, l = o.cpu().numpy(), l.cpu().numpy()
    assert np.array_equal(np.isneginf(l), ~fin)
    assert np.abs(o - ref_o.transpose(1, 0, 2)).max() <= OUT_TOL
    assert np.abs(l[fin] - ref_l.T[fin]).max() <= LSE_TOL
    # the restatement's merge re-entry on the same halves (state in fp32 upcasts)
    ex = lambda a: T.repeat_kv_heads(bhsd(a), hq // hkv)
    tq, tqp = bhsd(q32), torch.from_numpy(qp)
    to, tl = T.positioned_local_compact_partial(scale, tq, tqp, ex(k32[:h]), ex(v32[:h]), torch.from_numpy(kp[:h]))
    to, tl = T.positioned_merge_compact_partial(scale, tq, tqp, to, tl, ex(k32[h:]), ex(v32[h:]),
                                                torch.from_numpy(kp[h:]))
    assert np.abs(o - to[0].numpy()).max() <= OUT_TOL


def test_block_partial_positioned_merge_and_flag(gpu):
    # positioned_merge_compact_partial with positions (ring.rs:574-603): a striped
    # target merged with two sources; then the same source with its key list reversed
    # gives the same partial and raises no flag (keys in any order are sorted first).
    pos, _ = _strategy_rows([160, 96, 64], "striped")
    (q, k, v), (q32, k32, v32) = draw(91, [(320, 8, 128), (320, 2, 128), (320, 2, 128)], torch.bfloat16)
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    t = lambda a: torch.tensor(a, dtype=torch.int64, device="cuda")
    o, l = H.positioned_local_compact_partial(qh[:, :160], t(pos[0]), kh[:, :160], vh[:, :160], t(pos[0]))
    o, l = H.positioned_merge_compact_partial(qh[:, :160], t(pos[0]), o, l, kh[:, 256:], vh[:, 256:], t(pos[2]))
    o, l = H.positioned_merge_compact_partial(qh[:, :160], t(pos[0]), o, l, kh[:, 160:256], vh[:, 160:256],
                                              t(pos[1]))
    torch.cuda.synchronize()
    flat = np.array(sum(pos, []))
    ref_o, ref_l = C.attention_f64(q32[:160], k32, v32, flat[:160], flat, 1 / math.sqrt(128))
    assert np.abs(o.cpu().numpy() - ref_o.transpose(1, 0, 2)).max() <= OUT_TOL
    assert np.abs(l.cpu().numpy() - ref_l.T).max() <= LSE_TOL
    assert H.fetch_device_errors() == 0
    o1, l1 = H.positioned_local_compact_partial(qh[:, :160], t(pos[0]), kh[:, 160:256], vh[:, 160:256], t(pos[1]))
    rev = t(pos[1][::-1].copy())
    o2, l2 = H.positioned_local_compact_partial(qh[:, :160], t(pos[0]), kh[:, 160:256].flip(1),
                                                vh[:, 160:256].flip(1).contiguous(), rev)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert torch.equal(torch.isneginf(l1), torch.isneginf(l2))
    fin = torch.isfinite(l1)
    assert (o1 - o2).abs().max().item() <= 1e-5 and (l1[fin] - l2[fin]).abs().max().item() <= 1e-5


STRATEGY_RING_CASES = [
    # name, chunks, Hq, Hkv, D, dtype, seed   (ring.rs:3168-3224 is 3:1 fp32)
    ("fp32_3to1", [768, 256], 4, 4, 64, torch.float32, 60),
    ("bf16_uneven4", [900, 300, 500, 348], 8, 2, 128, torch.bfloat16, 61),
    ("f16_d64_three", [400, 250, 150], 4, 2, 64, torch.float16, 62),
    ("bf16_d96_padded", [500, 300, 212], 8, 2, 96, torch.bfloat16, 63),
]


@pytest.mark.parametrize("schedule", ["auto", "per_step"])
@pytest.mark.parametrize("strategy", ["striped", "zigzag"])
@pytest.mark.parametrize("case", STRATEGY_RING_CASES, ids=[c[0] for c in STRATEGY_RING_CASES])
def test_ring_replay_strategy_matches_full_attention(gpu, case, strategy, schedule):
    name, chunks, hq, hkv, d, dt, seed = case
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(seed, [(s, hq, d), (s, hkv, d), (s, hkv, d)], dt)
    pos, inv = _strategy_rows(chunks, strategy)
    rows = torch.tensor(sum(pos, []), device="cuda")
    # domain-major inputs: row r holds global position rows[r]
    qd, kd, vd = (x.index_select(0, rows).permute(1, 0, 2) for x in (q, k, v))
    H.replay_timing(True)
    H.replay_timing_read()
    out, lse = H.ring_attention_replay(qd, kd, vd, chunks, strategy=strategy, schedule=schedule)
    launches = H.replay_timing_read()["block"][1]
    H.replay_timing(False)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    # AUTO: one positions-mode launch over the whole sequence against K / V in position
    # order (fp32 on the fp32 matrix-core kernel); per step: launches per ring step
    if schedule == "auto":
        assert launches == 1, (name, launches)
    else:
        assert launches >= len(chunks), (name, launches)
    out = out.float().cpu().numpy()[:, inv]
    lse = lse.cpu().numpy()[:, inv]
    p = np.arange(s)
    ref_o, ref_l = C.attention_f64(q32, k32, v32, p, p, 1 / math.sqrt(d))
    tol_o = 1e-4 if dt == torch.float32 else OUT_TOL
    tol_l = 1e-4 if dt == torch.float32 else LSE_TOL
    assert np.abs(out - ref_o.transpose(1, 0, 2)).max() <= tol_o, (name, strategy)
    assert np.abs(lse - ref_l.T).max() <= tol_l, (name, strategy)
    if dt == torch.float32:
        # the reference's own driver with these positions, on the same fp32 inputs
        ro = T.ring_attention_replay_strategy(1 / math.sqrt(d), bhsd(q32), bhsd(k32), bhsd(v32), chunks, strategy)
        assert np.abs(out - ro[0].numpy()).max() <= 1e-4


def test_reference_uneven_3to1_every_strategy(gpu):
    # The reference's own strategy check at its own size (ring.rs:3168-3224 through
    # run_uneven_ring_attention, ring.rs:3226-3364): S=4096 split 3:1, 8 heads, head dim
    # 128, fp32, vanilla / striped / zigzag, each against full attention after the
    # inverse permutation -- mean |delta| < 1e-4 there, and no NaN; here also the max.
    chunks, hq, hkv, d = [3072, 1024], 8, 8, 128
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(66, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.float32)
    p = np.arange(s)
    ref_o, ref_l = C.attention_f64(q32, k32, v32, p, p, 1 / math.sqrt(d))
    ref_o = ref_o.transpose(1, 0, 2)
    for strategy in ("vanilla", "striped", "zigzag"):
        pos, inv = _strategy_rows(chunks, strategy)
        rows = torch.tensor(sum(pos, []), device="cuda")
        qd, kd, vd = (x.index_select(0, rows).permute(1, 0, 2) for x in (q, k, v))
        out, lse = H.ring_attention_replay(qd, kd, vd, chunks, strategy=strategy)
        torch.cuda.synchronize()
        assert H.fetch_device_errors() == 0
        out = out.cpu().numpy()[:, inv]
        lse = lse.cpu().numpy()[:, inv]
        assert np.isfinite(out).all() and np.isfinite(lse).all(), strategy
        err = np.abs(out - ref_o)
        assert err.mean() < 1e-4 and err.max() <= 1e-4, (strategy, err.mean(), err.max())
        assert np.abs(lse - ref_l.T).max() <= 1e-4, strategy


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "noncausal"])
def test_fp32_replay_one_launch(gpu, causal):
    # fp32 (the reference's CPU dtype): AUTO runs the whole replay as one block on the
    # fp32 matrix-core kernel, causal or not; it agrees with the per-step schedule and
    # with the f64 closed form at the fp32 tier (1e-4).
    chunks, hq, hkv, d = [300, 170, 250], 8, 2, 64
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(97, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.float32)
    args = (q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks)
    H.replay_timing(True)
    H.replay_timing_read()
    o1, l1 = H.ring_attention_replay(*args, causal=causal)
    launches = H.replay_timing_read()["block"][1]
    H.replay_timing(False)
    assert H.last_path() == "mfma_f32" and launches == 1
    o2, l2 = H.ring_attention_replay(*args, causal=causal, schedule="per_step")
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    pos = np.arange(s)
    ro, rl = C.attention_f64(q32, k32, v32, pos, pos, 1 / math.sqrt(d), causal=causal)
    for o, l in ((o1, l1), (o2, l2)):
        assert np.abs(o.cpu().numpy() - ro.transpose(1, 0, 2)).max() <= 1e-4
        assert np.abs(l.cpu().numpy() - rl.T).max() <= 1e-4


@pytest.mark.parametrize("strategy", ["vanilla", "zigzag"])
def test_fp32_paged_replay_one_launch_matches_unpaged(gpu, strategy):
    # fp32 K/V in a permuted paged pool: the one-launch schedule stages every chunk once
    # (and, for ZigZag, copies K/V in position order), then runs the same block as the
    # unpaged replay: bit for bit equal.
    chunks = [256, 96, 160]
    s, hq, hkv, d, bs = sum(chunks), 8, 2, 64, 16
    (q, k, v), _ = draw(98, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.float32)
    nb = s // bs + 3
    table = torch.from_numpy(I.permuted_block_table(99, nb)[: s // bs]).cuda()
    pool = torch.zeros(2, nb, bs, hkv, d, dtype=torch.float32, device="cuda")
    H.paged_kv_scatter(pool, table, 0, 0, s, k.permute(1, 0, 2), v.permute(1, 0, 2))
    o1, l1 = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks,
                                     strategy=strategy)
    o2, l2 = H.ring_attention_replay_paged(q.permute(1, 0, 2), pool, table, chunks, strategy=strategy)
    assert H.last_path() == "mfma_f32"
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_ring_replay_paged_strategy_matches_unpaged(gpu):
    chunks = [256, 96, 160]
    s, hq, hkv, d, bs = sum(chunks), 8, 2, 128, 16
    (q, k, v), _ = draw(79, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.bfloat16)
    nb = s // bs + 5
    table = torch.from_numpy(I.permuted_block_table(80, nb)[: s // bs]).cuda()
    pool = torch.zeros(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.paged_kv_scatter(pool, table, 0, 0, s, k.permute(1, 0, 2), v.permute(1, 0, 2))
    o1, l1 = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks,
                                     strategy="zigzag")
    o2, l2 = H.ring_attention_replay_paged(q.permute(1, 0, 2), pool, table, chunks, strategy="zigzag")
    # the fused schedule is what AUTO ran: the same single launch, bit for bit
    o3, l3 = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks,
                                     strategy="zigzag", schedule="fused")
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    assert torch.equal(o1, o3) and torch.equal(l1, l3)


def _wire_cases():
    import json
    import os
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "wire_frames.json")) as f:
        return json.load(f)


def test_kv_frame_pack_reproduces_reference_frames(gpu):
    # header + device-packed payload == the stored frames of the reference's TCP tests
    for c in _wire_cases():
        if c["kind"] != "kv_block" or "k" not in c:
            continue
        k = torch.tensor(c["k"], dtype=torch.float32).cuda()[0]
        v = torch.tensor(c["v"], dtype=torch.float32).cuda()[0]
        pos = torch.tensor(c["positions"], dtype=torch.int64).cuda() if c["positions"] is not None else None
        hdr, payload = H.kv_frame_pack(k, v, c["layer_idx"], c["start"], c["end"], positions=pos)
        torch.cuda.synchronize()
        assert hdr + payload.cpu().numpy().tobytes() == bytes.fromhex(c["frame_hex"]), c["name"]


@pytest.mark.parametrize("dtype,hkv,rep,length,d", [(torch.bfloat16, 2, 4, 300, 128), (torch.float16, 4, 1, 77, 64),
                                                    (torch.float32, 1, 8, 33, 128)])
def test_kv_frame_expand_and_round_trip(gpu, dtype, hkv, rep, length, d):
    from oracle import wire as W
    (kb, vb), _ = draw(150 + length, [(length, hkv, d + 8), (length, hkv, d + 8)], dtype)
    k, v = kb[:, :, :d].permute(1, 0, 2), vb[:, :, :d].permute(1, 0, 2)   # strided [Hkv, L, D] views
    pos = torch.arange(5, 5 + 3 * length, 3, dtype=torch.int64, device="cuda")
    hdr, payload = H.kv_frame_pack(k, v, 9, 5, 5 + 3 * length, positions=pos, num_heads=hkv * rep)
    torch.cuda.synchronize()
    # the oracle frame of the GQA-expanded fp32 block (ring.rs:999-1019, tcp.rs:161-207)
    kx = k.float().cpu().repeat_interleave(rep, 0).unsqueeze(0).numpy()
    vx = v.float().cpu().repeat_interleave(rep, 0).unsqueeze(0).numpy()
    name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[dtype]
    ref = W.kv_block_frame(9, 5, 5 + 3 * length, kx, vx, name, pos.cpu().numpy())
    frame = hdr + payload.cpu().numpy().tobytes()
    assert frame == ref
    # receive: parse the header, keep one head per group, unpack bit-exactly
    desc, hb = H.kv_frame_parse(frame)
    assert hb == len(hdr) and desc.num_heads == hkv * rep and desc.dtype == H.dtype_code(dtype)
    desc.num_kv_heads = hkv
    ko = torch.zeros(hkv, length, d, dtype=dtype, device="cuda")
    vo = torch.zeros_like(ko)
    po = torch.zeros(length, dtype=torch.int64, device="cuda")
    H.kv_frame_unpack(desc, payload, ko, vo, po)
    torch.cuda.synchronize()
    assert torch.equal(ko.view(torch.uint8 if dtype != torch.float32 else torch.int32),
                       k.contiguous().view(torch.uint8 if dtype != torch.float32 else torch.int32))
    assert torch.equal(vo, v) and torch.equal(po, pos)


def test_packet_frame_matches_oracle_and_round_trips(gpu):
    from oracle import wire as W
    b, h, d = 3, 32, 128
    (qb,), _ = draw(160, [(b, h, d + 16)], torch.bfloat16)
    q = qb[:, :, :d]                                   # strided [B, H, D] view
    o = torch.randn(b, h, d, device="cuda")
    lse = torch.randn(b, h, device="cuda")
    scale = 1 / math.sqrt(d)
    hdr, payload = H.packet_frame_pack(q, o, lse, 12, scale)
    torch.cuda.synchronize()
    ref = W.ring_packet_frame(12, q.float().cpu().unsqueeze(2).numpy(), o.cpu().unsqueeze(2).numpy(),
                              lse.cpu().unsqueeze(2).numpy(), scale, "bfloat16", "float32")
    frame = hdr + payload.cpu().numpy().tobytes()
    assert frame == ref
    desc, hb = H.packet_frame_parse(frame)
    assert hb == len(hdr) and desc.scale == scale and (desc.batch, desc.num_heads, desc.head_dim) == (b, h, d)
    qo = torch.zeros(b, h, d, dtype=torch.bfloat16, device="cuda")
    oo, lo = torch.zeros_like(o), torch.zeros_like(lse)
    H.packet_frame_unpack(desc, payload, qo, oo, lo)
    torch.cuda.synchronize()
    assert torch.equal(qo, q) and torch.equal(oo, o) and torch.equal(lo, lse)


def test_rope_table_matches_oracle(gpu):
    for d, rows, base in ((128, 4096, 500000.0), (64, 131072, 10000.0)):
        t = H.rope_table(d, rows, base)
        torch.cuda.synchronize()
        cos, sin = T.rope_caches(d, rows, base)
        assert np.abs(t[0].cpu().numpy() - cos.numpy()).max() <= 2e-6, (d, rows)
        assert np.abs(t[1].cpu().numpy() - sin.numpy()).max() <= 2e-6, (d, rows)


QKV_CASES = [
    # name, tokens, hidden, Hq, Hkv, D, dtype, bias, rope, positions
    ("llama_like_bf16", 300, 512, 8, 2, 128, torch.bfloat16, False, True, "contiguous"),
    ("qwen_like_bias_f16_d64", 200, 256, 14, 2, 64, torch.float16, True, True, "striped"),
    ("no_rope_bf16", 64, 128, 4, 4, 128, torch.bfloat16, False, False, None),
    ("many_stages_bias_bf16", 513, 1024, 8, 2, 128, torch.bfloat16, True, True, "offset"),
]


def _qkv_inputs(tokens, hidden, hq, hkv, d, dtype, bias, seed):
    rng_parts = clib.draw_normals(seed, [(tokens, hidden), (hq * d, hidden), (hkv * d, hidden), (hkv * d, hidden),
                                         ((hq + 2 * hkv) * d,)], "fp32")
    x = torch.from_numpy(rng_parts[0]).to(dtype)
    ws = [torch.from_numpy(w / math.sqrt(hidden)).to(dtype) for w in rng_parts[1:4]]
    b = torch.from_numpy(rng_parts[4] * 0.5).to(dtype)
    bs = [b[: hq * d], b[hq * d: (hq + hkv) * d], b[(hq + hkv) * d:]] if bias else [None] * 3
    return x, ws, bs


@pytest.mark.parametrize("case", QKV_CASES, ids=[c[0] for c in QKV_CASES])
def test_qkv_rope_project_matches_closed_form(gpu, case):
    name, tokens, hidden, hq, hkv, d, dtype, bias, rope, pat = case
    x, ws, bs = _qkv_inputs(tokens, hidden, hq, hkv, d, dtype, bias, 200 + tokens)
    if pat == "striped":
        pos_np = np.array(_strategy_rows([tokens, tokens + 17], "striped")[0][0])
    elif pat == "offset":
        pos_np = np.arange(1000, 1000 + tokens)
    else:
        pos_np = np.arange(tokens)
    rows = 4096
    table = H.rope_table(d, rows, 10000.0)
    pos = torch.from_numpy(pos_np.astype(np.int64)).cuda()
    dev = lambda t: t.cuda() if t is not None else None
    q, k, v = H.qkv_rope_project(dev(x), *(dev(w) for w in ws), hq, hkv, d, positions=pos, table=table,
                                 bq=dev(bs[0]), bk=dev(bs[1]), bv=dev(bs[2]), rope=rope)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    # closed form in f64 on the stored inputs, rotated with the library's own table
    x64 = x.double().numpy()
    tab = table.cpu().double().numpy()
    outs = []
    for i, (w, b, heads) in enumerate(zip(ws, bs, (hq, hkv, hkv))):
        y = x64 @ w.double().numpy().T + (b.double().numpy() if b is not None else 0.0)
        y = y.reshape(tokens, heads, d).transpose(1, 0, 2)
        if rope and i < 2:
            c, s = tab[0][pos_np][None], tab[1][pos_np][None]
            y1, y2 = y[..., : d // 2], y[..., d // 2:]
            y = np.concatenate([y1 * c - y2 * s, y1 * s + y2 * c], axis=-1)
        outs.append(y)
    for got, ref in zip((q, k, v), outs):
        g = got.double().cpu().numpy()
        bound = np.abs(ref) / 128 + 1e-3 * np.abs(ref).max()
        assert np.all(np.abs(g - ref) <= bound), (name, float(np.abs(g - ref).max()))
    # the reference's own op sequence in fp32 (ring.rs:1865-1908, rotary.rs:103-158)
    cos, sin = T.rope_caches(d, rows, 10000.0)
    f32 = lambda t: t.float() if t is not None else None
    tq, tk, tv = T.qkv_rope_forward(f32(x)[None], *(f32(w) for w in ws), *(f32(b) for b in bs), hq, hkv, d,
                                    torch.from_numpy(pos_np.astype(np.int64))[None], cos, sin, rope=rope)
    for got, ref in zip((q, k, v), (tq[0], tk[0], tv[0])):
        assert (got.float().cpu() - ref).abs().max() <= 1e-2 * ref.abs().max() + 1e-3, name


def test_qkv_rope_project_paged_append_matches_views(gpu):
    tokens, hidden, hq, hkv, d, bs_ = 150, 256, 8, 2, 128, 16
    x, ws, _ = _qkv_inputs(tokens, hidden, hq, hkv, d, torch.bfloat16, False, 310)
    x, ws = x.cuda(), [w.cuda() for w in ws]
    table = H.rope_table(d, 1024, 10000.0)
    pos = torch.arange(37, 37 + tokens, dtype=torch.int64, device="cuda")
    q1, k1, v1 = H.qkv_rope_project(x, *ws, hq, hkv, d, positions=pos, table=table)
    nb = 24
    pool = torch.zeros(2, nb, bs_, hkv, d, dtype=torch.bfloat16, device="cuda")
    blocks = torch.from_numpy(I.permuted_block_table(311, nb)[:14].astype(np.int32)).cuda()
    q2 = H.qkv_rope_project_paged(x, *ws, hq, hkv, d, pool, blocks, 16, 16 + 37, positions=pos, table=table)
    k2, v2 = H.paged_kv_gather(pool, blocks, 16, 16 + 37, 16 + 37 + tokens)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)


def test_qkv_rope_8_byte_aligned_views_match_contiguous(gpu):
    # Row starts that are 8- but not 16-byte aligned (row stride D + 4 elements, base offset
    # 4 elements) take the 8-byte store path; the values are those of contiguous outputs.
    tokens, hidden, hq, hkv, d = 200, 256, 8, 2, 128
    x, ws, bs = _qkv_inputs(tokens, hidden, hq, hkv, d, torch.bfloat16, True, 330)
    x, ws, bs = x.cuda(), [w.cuda() for w in ws], [b.cuda() for b in bs]
    table = H.rope_table(d, 512, 10000.0)
    pos = torch.arange(7, 7 + tokens, dtype=torch.int64, device="cuda")
    q1, k1, v1 = H.qkv_rope_project(x, *ws, hq, hkv, d, positions=pos, table=table, bq=bs[0], bk=bs[1], bv=bs[2])
    views = [torch.zeros(h, tokens, d + 4, dtype=torch.bfloat16, device="cuda")[:, :, 4:] for h in (hq, hkv, hkv)]
    q2, k2, v2 = H.qkv_rope_project(x, *ws, hq, hkv, d, positions=pos, table=table, bq=bs[0], bk=bs[1], bv=bs[2],
                                    q_out=views[0], k_out=views[1], v_out=views[2])
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    assert views[0].data_ptr() % 16 == 8
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)


def test_qkv_rope_bad_positions_and_block_ids_flag_and_skip(gpu):
    # A position outside the table leaves that token's q / k unrotated and raises flag 4;
    # a block id outside the pool leaves that block's tokens unwritten and raises flag 1.
    # Every other row is bit-identical to a clean launch.  Hq*D = 896 puts the q / k
    # boundary inside a 256-feature tile.
    tokens, hidden, hq, hkv, d, bs_, rows = 100, 256, 14, 2, 64, 16, 512
    x, ws, _ = _qkv_inputs(tokens, hidden, hq, hkv, d, torch.bfloat16, False, 320)
    x, ws = x.cuda(), [w.cuda() for w in ws]
    table = H.rope_table(d, rows, 10000.0)
    pos = torch.arange(3, 3 + tokens, dtype=torch.int64, device="cuda")
    H.fetch_device_errors()
    q1, k1, v1 = H.qkv_rope_project(x, *ws, hq, hkv, d, positions=pos, table=table)
    qn, kn, _ = H.qkv_rope_project(x, *ws, hq, hkv, d, positions=pos, table=table, rope=False)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 0
    bad_tok = [5, 70]
    bad = pos.clone()
    bad[5], bad[70] = rows, -1
    q2, k2, v2 = H.qkv_rope_project(x, *ws, hq, hkv, d, positions=bad, table=table)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 4
    keep = [t for t in range(tokens) if t not in bad_tok]
    assert torch.equal(q2[:, keep], q1[:, keep]) and torch.equal(k2[:, keep], k1[:, keep])
    assert torch.equal(q2[:, bad_tok], qn[:, bad_tok]) and torch.equal(k2[:, bad_tok], kn[:, bad_tok])
    assert torch.equal(v2, v1)

    nb = 12
    blocks = torch.from_numpy(I.permuted_block_table(321, nb)[:7].astype(np.int32)).cuda()
    pool1 = torch.zeros(2, nb, bs_, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.qkv_rope_project_paged(x, *ws, hq, hkv, d, pool1, blocks, 0, 0, positions=pos, table=table)
    bad_blocks = blocks.clone()
    bad_blocks[2] = nb
    pool2 = torch.zeros_like(pool1)
    q3 = H.qkv_rope_project_paged(x, *ws, hq, hkv, d, pool2, bad_blocks, 0, 0, positions=pos, table=table)
    torch.cuda.synchronize()
    assert H.fetch_device_errors() == 1
    assert torch.equal(q3, q1)
    lost = int(blocks[2])
    assert not pool2[:, lost].any()
    others = [b for b in range(nb) if b != lost]
    assert torch.equal(pool2[:, others], pool1[:, others])


@pytest.mark.parametrize("dtype,chunks,hq,hkv,d", [(torch.float32, [40, 24, 36], 4, 2, 64),
                                                   (torch.bfloat16, [128, 96, 200], 8, 2, 128)])
def test_ring_runtime_domains_match_full_attention(gpu, dtype, chunks, hq, hkv, d):
    # One HipRingAttnRuntime per domain (the reference's RingAttnRuntime contract):
    # each binds its chunk, runs its ring, and returns its rows of causal attention.
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(170 + d, [(s, hq, d), (s, hkv, d), (s, hkv, d)], dtype)
    ids = [f"domain-{i}" for i in range(len(chunks))]
    offs = np.concatenate([[0], np.cumsum(chunks)])
    rts = []
    for i in range(len(chunks)):
        rt = H.RingAttnRuntime("hip")
        rt.init(i, ids, chunks, hq, d, dtype)
        a, b = offs[i], offs[i + 1]
        rt.bind_layer(3, q[a:b].permute(1, 0, 2), k[a:b].permute(1, 0, 2), v[a:b].permute(1, 0, 2))
        rts.append(rt)
    p = np.arange(s)
    ref_o, ref_l = C.attention_f64(q32, k32, v32, p, p, 1 / math.sqrt(d))
    tol_o = 1e-4 if dtype == torch.float32 else OUT_TOL
    tol_l = 1e-4 if dtype == torch.float32 else LSE_TOL
    for i, rt in enumerate(rts):
        mx, sm, out = rt.run_ring_attention_layer(3)
        a, b = offs[i], offs[i + 1]
        assert np.all(sm == 1.0)
        assert np.abs(out - ref_o[a:b].transpose(1, 0, 2)).max() <= tol_o, i
        assert np.abs(mx - ref_l[a:b].T).max() <= tol_l, i
    # an initial state is merged in first: extra keys at positions before the sequence
    e = 8
    (ek, ev), (ek32, ev32) = draw(180 + d, [(e, hkv, d), (e, hkv, d)], dtype)
    i = 1
    a, b = offs[i], offs[i + 1]
    eo, el = C.attention_f64(q32[a:b], ek32, ev32, np.arange(a, b), np.arange(-e, 0), 1 / math.sqrt(d))
    init = (el.T.astype(np.float32) - 1.0, np.full(el.T.shape, math.e, np.float32),
            eo.transpose(1, 0, 2).astype(np.float32))             # m + ln(l) = lse
    mx, sm, out = rts[i].run_ring_attention_layer(3, init)
    kk, vv = np.concatenate([ek32, k32]), np.concatenate([ev32, v32])
    ro, rl = C.attention_f64(q32[a:b], kk, vv, np.arange(a, b), np.concatenate([np.arange(-e, 0), p]), 1 / math.sqrt(d))
    assert np.abs(out - ro.transpose(1, 0, 2)).max() <= tol_o
    assert np.abs(mx - rl.T).max() <= tol_l
    for rt in rts:
        rt.shutdown()


def _poll_all(agent, want, tries=1000):
    """Poll until `want` completions have arrived (each poll returns at once)."""
    got = []
    for _ in range(tries):
        got += agent.poll_transfers()
        if len(got) >= want:
            break
        torch.cuda.synchronize()
    return got


def test_block_transport_round_trips_a_registered_block(gpu):
    # The reference's own check (serialized_block.rs:205-254) on device memory: the
    # receiver registers an empty destination, the sender its data; metadata goes both
    # ways; the transfer lands in the receiver's block bit for bit, with the completion
    # naming that block and both wire counters at the block's bytes.
    from oracle import wire as W
    sender, receiver = H.BlockAgent.pair("agent-a", "agent-b")
    try:
        dest = torch.zeros(1, 2, 3, 4, dtype=torch.float32, device="cuda")
        dest_id, dest_desc = receiver.register_block(dest)
        src = torch.arange(24, dtype=torch.float32, device="cuda").reshape(1, 2, 3, 4)
        src_id, src_desc = sender.register_block(src)
        assert dest_desc["mem_type"] == src_desc["mem_type"] == 1            # Vram
        assert dest_desc["dev_id"] == torch.cuda.current_device() and dest_desc["meta"] == b"[1,2,3,4]"
        s_md, r_md = sender.local_metadata(), receiver.local_metadata()
        # stable bytes: the bincode AgentMetadata of the descriptors (oracle restatement)
        assert r_md == W.agent_metadata_bincode("agent-b", [("agent-b", dest_id, dest_desc["addr"], 96,
                                                             dest_desc["dev_id"], 1, b"[1,2,3,4]")])
        assert receiver.load_remote_metadata(s_md) == "agent-a"
        assert sender.load_remote_metadata(r_md) == "agent-b"
        sender.submit_transfer(src_id, sender.remote_desc("agent-b", dest_id))
        done = _poll_all(receiver, 1)
        assert done == [(dest_id, 96)]
        assert torch.equal(dest.view(torch.int32), src.view(torch.int32))
        assert sender.wire_bytes() == (96, 0) and receiver.wire_bytes() == (0, 96)
        assert receiver.poll_transfers() == [] and sender.poll_transfers() == []
    finally:
        sender.destroy()
        receiver.destroy()


def test_block_transport_deregister_waits_for_pending_copies(gpu):
    # A 256 MiB transfer posted on a side stream, then the source deregistered at once
    # and overwritten on the default stream: deregister returns only after the copy
    # has read the block, so the destination holds the original bytes; the receiver
    # still polls the completion, and destroy after a fresh post leaves the copy whole.
    sender, receiver = H.BlockAgent.pair("src-side", "dst-side")
    side = torch.cuda.Stream()
    try:
        n = 64 << 20
        src = torch.arange(n, dtype=torch.int32, device="cuda")
        dst = torch.zeros(n, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        sid, _ = sender.register_block(src)
        did, _ = receiver.register_block(dst)
        sender.load_remote_metadata(receiver.local_metadata())
        sender.submit_transfer(sid, sender.remote_desc("dst-side", did), stream=side)
        sender.deregister_block(sid)
        src.fill_(-1)
        torch.cuda.synchronize()
        assert _poll_all(receiver, 1) == [(did, 4 * n)]
        assert torch.equal(dst, torch.arange(n, dtype=torch.int32, device="cuda"))
        src2 = torch.full((n,), 7, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        sid2, _ = sender.register_block(src2)
        sender.submit_transfer(sid2, sender.remote_desc("dst-side", did), stream=side)
        sender.destroy()
        src2.fill_(-1)
        torch.cuda.synchronize()
        assert bool((dst == 7).all())
        assert _poll_all(receiver, 1) == [(did, 4 * n)]
    finally:
        sender.destroy()
        receiver.destroy()


def test_block_transport_carries_a_kv_wire_frame(gpu):
    # The KV frame payload of a c3-shaped chunk (GQA-expanded fp32 K/V + positions,
    # tcp.rs:161-207) moved between registered device blocks, then unpacked at the
    # receiver: the K/V and positions arrive bit-exact.
    hkv, rep, length, d = 8, 4, 1024, 128
    (kb, vb), _ = draw(160, [(length, hkv, d), (length, hkv, d)], torch.bfloat16)
    k, v = kb.permute(1, 0, 2), vb.permute(1, 0, 2)
    pos = torch.arange(12288, 12288 + length, dtype=torch.int64, device="cuda")
    hdr, payload = H.kv_frame_pack(k, v, 3, 12288, 12288 + length, positions=pos, num_heads=hkv * rep)
    a, b = H.BlockAgent.pair("domain-0", "domain-1")
    try:
        inbox = torch.empty_like(payload)
        in_id, _ = b.register_block(inbox)
        out_id, _ = a.register_block(payload)
        a.load_remote_metadata(b.local_metadata())
        b.load_remote_metadata(a.local_metadata())
        a.submit_transfer(out_id, a.remote_desc("domain-1", in_id))
        assert _poll_all(b, 1) == [(in_id, payload.numel() * payload.element_size())]
        desc, _ = H.kv_frame_parse(hdr + b"")
        desc.num_kv_heads = hkv
        ko, vo = torch.zeros_like(k.contiguous()), torch.zeros_like(v.contiguous())
        po = torch.zeros_like(pos)
        H.kv_frame_unpack(desc, inbox, ko, vo, po)
        torch.cuda.synchronize()
        assert torch.equal(ko.view(torch.int16), k.contiguous().view(torch.int16))
        assert torch.equal(vo.view(torch.int16), v.contiguous().view(torch.int16)) and torch.equal(po, pos)
    finally:
        a.destroy()
        b.destroy()


@pytest.mark.parametrize("causal", [True, False])
def test_traced_fused_replay_statistics_and_perf_log(gpu, causal, tmp_path):
    # The traced fused ring (per-ring-call timing, ring.rs:820-844,1376-1395) computes
    # the same bits as the untraced one, and its per-domain statistics follow the ring's
    # geometry: workgroups per domain, 128-key tiles folded, peer chunks and their K/V
    # bytes; the JSONL events carry the reference's ring_attention fields.
    import json
    chunks, hq, hkv, d = [900, 300, 500, 348], 8, 2, 128
    s = sum(chunks)
    (q, k, v), _ = draw(71, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.bfloat16)
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    ref_o, ref_l = H.ring_attention_replay(qh, kh, vh, chunks, causal=causal)
    need = H.trace_record_bytes(torch.bfloat16, hq, hkv, d, chunks, causal)
    small = torch.zeros(need // 2, dtype=torch.uint8, device="cuda")
    H.trace_attach(small)
    with pytest.raises(H.HcpRingError, match="trace buffer too small"):
        H.ring_attention_replay(qh, kh, vh, chunks, causal=causal)
    buf = torch.zeros(need, dtype=torch.uint8, device="cuda")
    H.trace_attach(buf)
    try:
        o, l = H.ring_attention_replay(qh, kh, vh, chunks, causal=causal)
        assert H.last_path() == "ring_fused"
        doms, launch = H.trace_read()
        log = tmp_path / "perf.jsonl"
        H.trace_perf_log(3, str(log))
    finally:
        H.trace_attach(None)
    torch.cuda.synchronize()
    assert torch.equal(o, ref_o) and torch.equal(l, ref_l)
    n = len(chunks)
    offs = [sum(chunks[:i]) for i in range(n)]
    tq, groups = 32 * 8 // 4, hq // 4           # G = 4 query heads per workgroup
    row_bytes = hkv * d * 2 * 2
    assert [x["domain"] for x in doms] == list(range(n))
    total_tiles = 0
    for t, x in enumerate(doms):
        assert x["workgroups"] == -(-chunks[t] // tq) * groups
        tiles = 0
        for qt in range(-(-chunks[t] // tq)):
            q_end = min(chunks[t], (qt + 1) * tq)
            local = -(-(q_end if causal else chunks[t]) // 128)
            below = -(-offs[t] // 128)
            above = 0 if causal else -(-(s - offs[t] - chunks[t]) // 128)
            tiles += local + below + above
        assert x["key_tiles"] == tiles * groups
        total_tiles += tiles * groups
        srcs = list(range(t)) if causal else [j for j in range(n) if j != t]
        assert x["peer_chunks"] == len(srcs)
        assert x["kv_recv_bytes"] == sum(chunks[j] for j in srcs) * row_bytes
        users = (n - 1 - t) if causal else (n - 1)
        assert x["kv_sent_bytes"] == chunks[t] * row_bytes * users
        assert x["local_cu_ms"] > 0 and x["span_ms"] > 0
        assert (x["peer_cu_ms"] > 0) == (len(srcs) > 0)
        assert 300 < x["clock_mhz"] < 3000
    assert launch["workgroups"] == sum(x["workgroups"] for x in doms)
    assert 1 <= launch["cus"] <= 256 and launch["span_ms"] > 0
    assert launch["wg_ms_min"] <= launch["wg_ms_mean"] <= launch["wg_ms_max"]
    cu_ms = sum(x["local_cu_ms"] + x["peer_cu_ms"] for x in doms)
    assert cu_ms <= launch["busy_cu_ms"] * 1.0001
    lines = [json.loads(x) for x in log.read_text().splitlines()]
    assert [e["domain"] for e in lines] == list(range(n))
    for e, x in zip(lines, doms):
        assert e["event"] == "ring_attention" and e["layer"] == 3 and e["num_domains"] == n
        assert e["seq_len"] == chunks[e["domain"]] and e["overlap"] == 1
        assert e["kv_recv_bytes"] == x["kv_recv_bytes"] and e["micro_blocks"] == x["peer_chunks"]
        assert abs(e["local_compute_ms"] - round(x["local_compute_ms"], 3)) < 2e-3
        for key in ("total_ms", "peer_compute_ms", "recv_ms", "send_ms", "forward_ms", "flush_ms",
                    "kv_sent_bytes", "wire_sent_bytes", "wire_recv_bytes", "ts"):
            assert key in e


@pytest.mark.parametrize("schedule", ["auto", "per_step"])
@pytest.mark.parametrize("d", [8, 16, 24, 40, 56, 64, 72])
def test_ring_replay_head_dims_around_the_half_width_kernel(gpu, d, schedule):
    # Head dims up to 64 take the half-width instantiation (the MFMAs of the first 64 dims
    # of the zero-padded 128-dim rows), 72 the full one: every multiple of 8 below 64 and
    # the boundary, token-major Q/K/V, uneven causal chunks, GQA 2, fused and per step,
    # against the f64 closed form.
    chunks, hq, hkv = [150, 97, 70], 4, 2
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(70 + d, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.bfloat16)
    out, lse = H.ring_attention_replay(q.permute(1, 0, 2), k.permute(1, 0, 2), v.permute(1, 0, 2), chunks,
                                       schedule=schedule)
    assert H.last_path() == ("ring_fused" if schedule == "auto" else "mfma")
    torch.cuda.synchronize()
    pos = np.arange(s)
    ref_o, ref_l = C.attention_f64(q32, k32, v32, pos, pos, 1 / math.sqrt(d))
    assert np.abs(out.float().cpu().numpy() - ref_o.transpose(1, 0, 2)).max() <= OUT_TOL
    assert np.abs(lse.cpu().numpy() - ref_l.T).max() <= LSE_TOL


@pytest.mark.parametrize("schedule", ["auto", "per_step"])
def test_d64_token_major_and_head_major_layouts_agree(gpu, schedule):
    # The same Qwen2-0.5B-shaped ring (14 q / 2 kv heads, D=64) with token-major K/V
    # (both KV heads in one row of the view) and with head-major K/V: both within
    # tolerance of the restatement of ring_attention and of each other, the token-major
    # one traced (its workgroup count is the decomposition's: one query head per group,
    # 256 rows per workgroup).
    chunks, hq, hkv, d = [700, 300, 500], 14, 2, 64
    s = sum(chunks)
    (q, k, v), (q32, k32, v32) = draw(65, [(s, hq, d), (s, hkv, d), (s, hkv, d)], torch.bfloat16)
    qh = q.permute(1, 0, 2)
    o1, l1 = H.ring_attention_replay(qh, k.permute(1, 0, 2), v.permute(1, 0, 2), chunks, schedule=schedule)
    o2, l2 = H.ring_attention_replay(qh, k.permute(1, 0, 2).contiguous(), v.permute(1, 0, 2).contiguous(), chunks,
                                     schedule=schedule)
    torch.cuda.synchronize()
    ro, rl = T.ring_attention_replay(1 / math.sqrt(d), bhsd(q32), bhsd(k32), bhsd(v32), chunks, return_lse=True)
    for o, l in ((o1, l1), (o2, l2)):
        assert np.abs(o.float().cpu().numpy() - ro[0].numpy()).max() <= OUT_TOL
        assert np.abs(l.cpu().numpy() - rl[0].numpy()).max() <= LSE_TOL
    assert (o1.float() - o2.float()).abs().max().item() <= OUT_TOL
    if schedule == "auto":
        buf = torch.zeros(H.trace_record_bytes(torch.bfloat16, hq, hkv, d, chunks), dtype=torch.uint8, device="cuda")
        H.trace_attach(buf)
        try:
            o3, _ = H.ring_attention_replay(qh, k.permute(1, 0, 2), v.permute(1, 0, 2), chunks)
            doms, launch = H.trace_read()
        finally:
            H.trace_attach(None)
        assert torch.equal(o3, o1)
        # 14 head groups of one query head, 256 rows per workgroup
        assert launch["workgroups"] == sum(-(-c // 256) for c in chunks) * 14
