"""C-ABI checks that need no GPU: the library loads, exports what the header declares,
and validates arguments before touching a device."""
import ctypes
import math

import numpy as np

import pytest
import torch

import hcp_ring_amd as H


def test_library_exports_every_header_function(hcp):
    names = hcp.header_functions()
    assert len(names) >= 14
    lib = ctypes.CDLL(hcp.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version(hcp):
    import re
    header = open(hcp.HEADER).read()
    want = int(re.search(r"#define HCP_RING_ABI_VERSION (\d+)", header).group(1))
    assert hcp.lib().hcp_ring_abi_version() == want == hcp.ABI_VERSION == 3


def test_positioned_workspace_size_covers_the_key_sort(hcp):
    # lim int32 per query row; with causal=1 the flag, two (int64 key, int32 row) sort
    # buffers and the sorted K / V copies [Hkv, Lk, D] -- each region 256-byte aligned.
    a = lambda x: (x + 255) // 256 * 256
    d = hcp.BlockDesc(2, 16, 4, 128, 300, 1500, 0, 0, 1, 0, 0.1)
    want = a(300 * 4) + 256 + 2 * a(1500 * 8) + 2 * a(1500 * 4) + 2 * a(4 * 1500 * 128 * 2)
    assert hcp.lib().hcp_ring_block_partial_positioned_workspace_size(ctypes.byref(d)) == want
    d.causal = 0
    assert hcp.lib().hcp_ring_block_partial_positioned_workspace_size(ctypes.byref(d)) == a(300 * 4)
    d.causal, d.dtype = 1, 99
    assert hcp.lib().hcp_ring_block_partial_positioned_workspace_size(ctypes.byref(d)) == 0


def test_null_descriptor_is_invalid(hcp):
    v = hcp.View(0, 0, 1)
    rc = hcp.lib().hcp_ring_block_partial(None, v, v, v, None, None, None)
    assert rc == -6
    assert "null descriptor" in hcp.last_error()


def test_bad_head_ratio_is_invalid(hcp):
    d = hcp.BlockDesc(2, 6, 4, 128, 8, 8, 0, 0, 1, 0, 0.1)
    v = hcp.View(16, 0, 128)
    rc = hcp.lib().hcp_ring_block_partial(ctypes.byref(d), v, v, v, ctypes.c_void_p(16),
                                          ctypes.c_void_p(16), None)
    assert rc == -6 and "multiple of num_kv_heads" in hcp.last_error()


def test_merge_rejects_too_many_parts(hcp):
    v = hcp.View(16, 0, 128)
    rc = hcp.lib().hcp_ring_lse_merge(65, None, None, 1, 1, 128, 2, v, None, None)
    assert rc == -6


def test_paged_rejects_short_table(hcp):
    pool = hcp.PagedPool(16, 8, 16, 8, 128, 2)
    v = hcp.View(16, 128, 128 * 8)
    rc = hcp.lib().hcp_paged_kv_gather(ctypes.byref(pool), ctypes.c_void_p(16), 2, 0, 0, 40, v, v, None)
    assert rc == -6 and "too short" in hcp.last_error()


def test_replay_workspace_size_matches_plan(hcp):
    chunks = [12288, 8192, 8192, 4096]
    n = hcp.replay_workspace_size(torch.bfloat16, 32, 8, 128, chunks)
    # One running fp32 state o [32, L, 128] + lse [32, L] per domain with more than one
    # source: domain 0 only sees itself and writes its rows directly.
    rows = 32 * (8192 + 8192 + 4096)
    assert n == rows * 128 * 4 + rows * 4
    assert hcp.replay_workspace_size(torch.bfloat16, 32, 8, 128, [5, 0]) == 0


@pytest.mark.parametrize("strategy", ["striped", "zigzag"])
def test_positioned_replay_workspace_fused_and_auto(hcp, strategy):
    # Fused with explicit positions: positions int64 [S], a 256-byte flag, the row of
    # each position int32 [S], K and V in position order [Hkv, S, D] and the key limits
    # int32 [S]; paged, the two staging buffers come first.  AUTO covers both the fused
    # and the per-step layouts.
    chunks, hq, hkv, d = [1000, 600, 424], 8, 2, 128
    s = sum(chunks)
    a = lambda n: (n + 255) // 256 * 256
    stage = a(s * hkv * d * 2)
    fused = a(8 * s) + 256 + a(4 * s) + 2 * stage + a(4 * s)
    size = lambda **kw: hcp.replay_workspace_size(torch.bfloat16, hq, hkv, d, chunks, strategy=strategy, **kw)
    assert size(schedule="fused") == fused
    assert size(schedule="fused", paged=True) == fused + 2 * stage
    per = size(schedule="per_step")
    assert per > 0 and size() == max(per, fused)
    assert size(paged=True) == max(size(schedule="per_step", paged=True), fused + 2 * stage)


def test_vanilla_helpers_known_answers(hcp):
    # strategy.rs:157-163 (vanilla [3,1] -> [0,0,0,1]); reference_algo.rs:92-116 chunk sum.
    assert hcp.vanilla_assignment([3, 1]) == [0, 0, 0, 1]
    assert hcp.vanilla_offsets([640, 384], 1024) == [0, 640]
    with pytest.raises(ValueError):
        hcp.vanilla_offsets([640, 383], 1024)
    assert hcp.ring_sources(1, 4) == [1, 0, 3, 2]


def test_device_count_without_gpu(hcp):
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    c = ctypes.c_int(-1)
    assert hcp.lib().hcp_ring_device_count(ctypes.byref(c)) == -5
    assert c.value == 0


@pytest.mark.parametrize("strategy", ["vanilla", "striped", "zigzag"])
def test_strategy_helpers_match_oracle_procedure(strategy):
    # The library's closed-form positions (host helpers, no GPU) against the oracle's
    # step-by-step restatement of strategy.rs:53-143, zero-length chunks included.
    from oracle import strategy as SP
    rng = np.random.default_rng(5)
    cases = [[3, 1], [4, 4], [6, 0, 3], [1], [0, 5], [2, 7, 1, 9]]
    cases += [list(rng.integers(0, 40, size=rng.integers(2, 9))) for _ in range(30)]
    for chunks in cases:
        chunks = [int(c) for c in chunks]
        if sum(chunks) == 0:
            continue
        a = SP.build_assignment(chunks, strategy)
        assert H.build_assignment(chunks, strategy) == a, chunks
        assert H.domain_positions(chunks, strategy) == sum(SP.build_domain_positions(a), []), chunks
        assert H.inverse_perm(chunks, strategy) == SP.build_inverse_perm(a), chunks


def test_strategy_helpers_reject_bad_arguments():
    with pytest.raises(H.HcpRingError):
        H.build_assignment([3, 1], 7)
    with pytest.raises(H.HcpRingError):
        H.build_assignment([3, -1], "striped")


def test_runtime_smoke_and_init_validation():
    # The reference's Init checks (src/ringattn_runtime.cc:17-37) and its three-domain
    # Init / Run / Shutdown smoke (rust_bridge.cc:646-681); no GPU work is involved.
    assert H.cxx_smoke_domain_count() == 3
    ids, lens = ["d0", "d1"], [6, 4]
    rt = H.RingAttnRuntime("hip")
    with pytest.raises(H.HcpRingError):          # chunk lengths must sum to the sequence
        rt.init(0, ids, lens, 2, 8, torch.float32, global_seq_len=11)
    with pytest.raises(H.HcpRingError):
        rt.init(0, ["", "d1"], lens, 2, 8, torch.float32)
    with pytest.raises(H.HcpRingError):
        rt.init(0, ids, lens, 2, 8, torch.float32, block_sizes=[0, 16])
    with pytest.raises(H.HcpRingError):
        rt.init(0, ids, lens, 0, 8, torch.float32)
    with pytest.raises(H.HcpRingError):          # no CPU path in this library
        rt.init(0, ids, lens, 2, 8, torch.float32, device="cpu")
    with pytest.raises(H.HcpRingError):          # run before a successful Init
        H.RingAttnRuntime("hip").run_ring_attention_layer(0)
    rt.init(1, ids, lens, 2, 8, torch.float32)
    mx, sm, out = rt.run_ring_attention_layer(0)  # nothing bound: the empty state passes through
    assert np.isneginf(mx).all() and (sm == 0).all() and (out == 0).all()
    state = (np.full((2, 4), 0.5, np.float32), np.full((2, 4), 2.0, np.float32), np.ones((2, 4, 8), np.float32))
    mx, sm, out = rt.run_ring_attention_layer(0, state)
    assert np.array_equal(mx, state[0]) and np.array_equal(sm, state[1]) and np.array_equal(out, state[2])
    rt.shutdown()
    bad = H.RingAttnRuntime("cpu")
    with pytest.raises(H.HcpRingError):
        bad.init(0, ids, lens, 2, 8, torch.float32)


# Every entry point that takes a descriptor, pool, count or handle rejects a null or
# zero one with status -6 (invalid arguments, the rust_bridge.cc:109-128 meaning) and
# a message naming itself, before any device work.
NULL_CHECKED = [
    "hcp_ring_block_partial", "hcp_ring_block_partial_positioned", "hcp_ring_lse_merge",
    "hcp_paged_kv_gather", "hcp_paged_kv_scatter", "hcp_paged_kv_gather_batch",
    "hcp_paged_decode_partial", "hcp_paged_decode_partial_static", "hcp_decode_ring_replay",
    "hcp_ring_prefill_replay",
    "hcp_ring_prefill_replay_paged", "hcp_kv_frame_header", "hcp_kv_frame_parse",
    "hcp_kv_frame_pack", "hcp_kv_frame_unpack", "hcp_packet_frame_header",
    "hcp_packet_frame_parse", "hcp_packet_frame_pack", "hcp_packet_frame_unpack",
    "hcp_qkv_rope_project", "hcp_qkv_rope_project_paged", "hcp_ring_build_assignment",
    "hcp_ring_domain_positions", "hcp_ring_inverse_perm", "hcp_rope_table",
    "hcp_ringattn_runtime_init", "hcp_ringattn_runtime_bind_layer",
    "hcp_ringattn_runtime_run_layer", "hcp_ringattn_runtime_shutdown", "hcp_block_agent_pair_create",
    "hcp_block_agent_destroy", "hcp_block_register", "hcp_block_deregister", "hcp_block_local_metadata",
    "hcp_block_load_remote_metadata", "hcp_block_remote_desc", "hcp_block_submit_transfer",
    "hcp_block_poll_transfers", "hcp_block_wire_bytes",
]


def _null_args(fn, view_type):
    args = []
    for t in fn.argtypes:
        if t is view_type:
            args.append(view_type(None, 0, 1))
        elif t in (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_double,
                   ctypes.c_float, ctypes.c_int):
            args.append(0)
        else:
            args.append(None)
    return args


@pytest.mark.parametrize("name", NULL_CHECKED)
def test_null_or_zero_arguments_are_invalid(hcp, name):
    fn = getattr(hcp.lib(), name)
    rc = fn(*_null_args(fn, hcp.View))
    assert rc == -6, (name, rc, hcp.last_error())
    assert hcp.last_error().startswith(name + ":"), hcp.last_error()


def test_m0_scan_accepts_the_dma_sequence_and_rejects_anything_else():
    # build.py's check that the LDS DMA helper owns M0 (csrc/lds_dma.hpp): planted
    # violations in a synthetic instruction stream must raise.
    import importlib.util
    import os
    spec = importlib.util.spec_from_file_location(
        "hcp_build_m0", os.path.join(os.path.dirname(H.LIB_PATH), "..", "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    seq = ["s_mov_b32 m0, s12", "s_nop 0", "buffer_load_dwordx4 v3, s[8:11], 0 offen lds"]
    ok = ["v_mov_b32_e32 v1, 0"] + seq + ["s_waitcnt vmcnt(0)"] + seq
    assert b.scan_m0(ok) == 2
    planted = [
        ["s_mov_b32 m0, -1"] + seq,                                     # compiler M0 value
        seq[:1] + ["v_mov_b32_e32 v1, 0"] + seq[2:],                    # something between def and DMA
        ["buffer_load_dwordx4 v3, s[8:11], 0 offen lds"],                # DMA without its M0 def
        seq + ["s_mov_b32 s4, m0"],                                     # M0 read elsewhere
        seq + ["v_movrels_b32_e32 v0, v1"],                             # implicit M0 (indexing)
        seq + ["s_sendmsg sendmsg(MSG_GS_DONE)"],                       # implicit M0 (messages)
    ]
    for ins in planted:
        with pytest.raises(RuntimeError):
            b.scan_m0(ins)


def test_block_transport_metadata_without_a_gpu(hcp):
    # register -> local_metadata -> load_remote_metadata on host blocks (Dram): the blob
    # is the bincode AgentMetadata of the oracle (field order of block_transport.rs:36-86)
    from oracle import wire as W
    a, b = hcp.BlockAgent.pair("agent-a", "agent-b")
    try:
        x = np.arange(24, dtype=np.float32).reshape(1, 2, 3, 4)
        y = np.zeros((5, 7), dtype=np.int16)
        ix, dx = a.register_block(x)
        iy, dy = a.register_block(y)
        assert (ix, iy) == (0, 1)
        assert dx["mem_type"] == 0 and dx["meta"] == b"[1,2,3,4]" and dx["len"] == 96 and dx["addr"] == x.ctypes.data
        blob = a.local_metadata()
        want = W.agent_metadata_bincode("agent-a", [("agent-a", i, d["addr"], d["len"], d["dev_id"], d["mem_type"],
                                                     d["meta"]) for i, d in ((ix, dx), (iy, dy))])
        assert blob == want
        assert b.load_remote_metadata(blob) == "agent-a"
        r = b.remote_desc("agent-a", iy)
        assert r.agent == b"agent-a" and r.block_id == iy and hcp.block_desc_dict(r.desc) == dy
        a.deregister_block(ix)
        assert a.local_metadata() == W.agent_metadata_bincode("agent-a", [("agent-a", iy, dy["addr"], dy["len"], 0, 0,
                                                                           dy["meta"])])
        # malformed blobs: short, trailing byte, unknown BlockMemType variant
        for bad in (blob[:-1], blob + b"\0", blob[:blob.index(b"[1,2") - 12] + b"\2" + blob[blob.index(b"[1,2") - 11:]):
            with pytest.raises(hcp.HcpRingError) as e:
                b.load_remote_metadata(bad)
            assert e.value.code == -6
        # transfers are checked before any device work: unknown local block, length mismatch
        z = np.zeros(3, dtype=np.float32)
        iz, _ = b.register_block(z)
        b2 = a.load_remote_metadata(b.local_metadata())
        with pytest.raises(hcp.HcpRingError):
            a.submit_transfer(ix, a.remote_desc(b2, iz), stream=0)          # deregistered
        with pytest.raises(hcp.HcpRingError):
            a.submit_transfer(iy, a.remote_desc(b2, iz), stream=0)          # 70 bytes into 12
        assert b.poll_transfers() == [] and a.wire_bytes() == (0, 0)
    finally:
        a.destroy()
        b.destroy()


def test_trace_entry_points_validate_without_gpu(hcp):
    # Reading with nothing attached, or with nothing traced yet, is refused before any
    # device work; the record size follows the fused launch geometry.
    assert hcp.lib().hcp_ring_trace_attach(None, 0) == 0
    n = ctypes.c_int32(0)
    doms = (hcp.TraceDomain * 4)()
    assert hcp.lib().hcp_ring_trace_read(None, doms, 4, ctypes.byref(n), None) == -6
    assert "no trace buffer attached" in hcp.last_error()
    assert hcp.lib().hcp_ring_trace_attach(ctypes.c_void_p(4), 64) == -6  # misaligned
    assert hcp.lib().hcp_ring_trace_attach(ctypes.c_void_p(256), 64) == 0
    assert hcp.lib().hcp_ring_trace_read(None, doms, 4, ctypes.byref(n), None) == -6
    assert "no traced replay" in hcp.last_error()
    assert hcp.lib().hcp_ring_trace_attach(None, 0) == 0
    # c3: 4 domains, G = 4 (64 query rows per workgroup), 8 head groups
    chunks = [12288, 8192, 8192, 4096]
    wgs = sum((c + 63) // 64 for c in chunks) * 8
    assert hcp.trace_record_bytes(torch.bfloat16, 32, 8, 128, chunks) == wgs * (16 + 2 * 4) * 4
    # c2: G = 8 (32 rows), 2 head groups
    assert hcp.trace_record_bytes(torch.bfloat16, 16, 2, 128, [4096, 2560, 1536]) == 512 * (16 + 6) * 4
    # perf log with no path and no HCP_PERF_LOG is a no-op, even without a trace
    import os
    old = os.environ.pop("HCP_PERF_LOG", None)
    try:
        assert hcp.lib().hcp_ring_trace_perf_log(None, 0, None) == 0
    finally:
        if old is not None:
            os.environ["HCP_PERF_LOG"] = old
