"""hcp_paged_decode_partial_static (the decode entry point that allocates nothing) against
hcp_paged_decode_partial with a caller workspace: two calls in a row through the C ABI,
the second on a smaller input, each bit-identical to the workspace entry point's result
(same kernels, same split plan), and the rejection of a call whose split partials
exceed the static array."""
import ctypes
import math

import numpy as np
import pytest
import torch

import hcp_ring_amd as H
from oracle import inputs as I

pytestmark = pytest.mark.gpu


def _inputs(seed, b, hq, hkv, d, bs, ctx):
    nblk = (ctx + bs - 1) // bs
    nb = b * nblk + 2
    q = torch.empty(b, hq, d, dtype=torch.bfloat16, device="cuda")
    pool = torch.empty(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.synth_normals(seed, 0, q.numel(), q)
    H.synth_normals(seed, q.numel(), pool.numel(), pool)
    tables = torch.from_numpy(np.ascontiguousarray(I.permuted_block_table(seed, nb)[: b * nblk].reshape(b, nblk)))
    return q, pool, tables.cuda()


def _static_call(q, pool, tables, t0, t1, seq_lens=None):
    b, hq, d = q.shape
    desc = H.decode_desc(q, pool, tables, t0, t1, 1 / math.sqrt(d))
    pp = H.paged_pool(pool)
    o = torch.full((b, hq, d), float("nan"), dtype=torch.float32, device="cuda")
    lse = torch.full((b, hq), float("nan"), dtype=torch.float32, device="cuda")
    qv = H.View(q.data_ptr(), q.stride(1), q.stride(0))
    rc = H.lib().hcp_paged_decode_partial_static(ctypes.byref(desc), ctypes.byref(pp), qv, H._ptr(tables),
                                                 H._ptr(seq_lens), H._ptr(o), H._ptr(lse), None)
    return rc, o, lse


@pytest.mark.parametrize("case", [
    # seed, batch, Hq, Hkv, D, bs, ctx, t0, t1, ragged -- the second call is the smaller one
    ((90, 16, 32, 8, 128, 16, 4096, 0, 4096, False), (91, 3, 14, 2, 64, 16, 700, 100, 650, True)),
])
def test_static_decode_matches_workspace_decode_twice(gpu, case):
    for seed, b, hq, hkv, d, bs, ctx, t0, t1, ragged in case:
        q, pool, tables = _inputs(seed, b, hq, hkv, d, bs, ctx)
        lens = torch.tensor([ctx - 41 * i for i in range(b)], dtype=torch.int32, device="cuda") if ragged else None
        ref_o, ref_l = H.decode_local_compact_partial(q, pool, tables, t0, t1, seq_lens=lens)
        rc, o, lse = _static_call(q, pool, tables, t0, t1, lens)
        assert rc == 0, H.last_error()
        torch.cuda.synchronize()
        assert H.fetch_device_errors() == 0
        assert torch.equal(o, ref_o) and torch.equal(lse, ref_l), (seed, b)


def test_static_decode_rejects_calls_beyond_the_array(gpu):
    # 512 sequences x 64 query heads x (128 + 1) fp32 per split: more than 16 MiB
    q, pool, tables = _inputs(92, 512, 64, 8, 128, 16, 64)
    desc = H.decode_desc(q, pool, tables, 0, 64, 1 / math.sqrt(128))
    need = H.lib().hcp_paged_decode_workspace_size(ctypes.byref(desc), ctypes.byref(H.paged_pool(pool)))
    assert need > (16 << 20)
    rc, o, _ = _static_call(q, pool, tables, 0, 64)
    assert rc == -6 and "static scratch" in H.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(o).all()  # nothing ran


def test_static_decode_allocates_nothing(gpu):
    # The advertised contract: after a warm-up call (code objects loaded, occupancy and
    # the static array's address cached), another call changes neither torch's pools
    # nor the device's free memory.
    q, pool, tables = _inputs(93, 8, 32, 8, 128, 16, 2048)
    rc, _, _ = _static_call(q, pool, tables, 0, 2048)
    assert rc == 0, H.last_error()
    o = torch.empty(8, 32, 128, dtype=torch.float32, device="cuda")
    lse = torch.empty(8, 32, dtype=torch.float32, device="cuda")
    desc = H.decode_desc(q, pool, tables, 0, 2048, 1 / math.sqrt(128))
    pp = H.paged_pool(pool)
    qv = H.View(q.data_ptr(), q.stride(1), q.stride(0))
    import gc
    gc.collect()  # tensors of earlier tests released now, not during the measured calls
    torch.cuda.synchronize()
    before = (torch.cuda.memory_allocated(), torch.cuda.memory_reserved(), torch.cuda.mem_get_info()[0])
    for _ in range(3):
        rc = H.lib().hcp_paged_decode_partial_static(ctypes.byref(desc), ctypes.byref(pp), qv, H._ptr(tables), None,
                                                     H._ptr(o), H._ptr(lse), None)
        assert rc == 0, H.last_error()
    torch.cuda.synchronize()
    after = (torch.cuda.memory_allocated(), torch.cuda.memory_reserved(), torch.cuda.mem_get_info()[0])
    # nothing grew: torch's pools (allocated, reserved) and the device's free bytes
    assert after[0] <= before[0] and after[1] == before[1] and after[2] == before[2], (before, after)


def test_static_decode_replays_in_a_graph(gpu):
    # Captured in a HIP graph (it records no memset nodes) and replayed three times with
    # eager work and synchronisations in between, each replay on new query values:
    # every replay equals the eager workspace entry point on the same inputs.
    q, pool, tables = _inputs(94, 4, 16, 4, 128, 16, 1024)
    o = torch.empty(4, 16, 128, dtype=torch.float32, device="cuda")
    lse = torch.empty(4, 16, dtype=torch.float32, device="cuda")
    desc = H.decode_desc(q, pool, tables, 0, 1024, 1 / math.sqrt(128))
    pp = H.paged_pool(pool)
    qv = H.View(q.data_ptr(), q.stride(1), q.stride(0))
    call = lambda: H.lib().hcp_paged_decode_partial_static(ctypes.byref(desc), ctypes.byref(pp), qv, H._ptr(tables),
                                                           None, H._ptr(o), H._ptr(lse), H._stream())
    assert call() == 0, H.last_error()  # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = call()
    assert rc == 0, H.last_error()
    for seed in (95, 96, 97):
        H.synth_normals(seed, 0, q.numel(), q)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref_o, ref_l = H.decode_local_compact_partial(q, pool, tables, 0, 1024)
        torch.cuda.synchronize()
        assert torch.equal(o, ref_o) and torch.equal(lse, ref_l), seed
