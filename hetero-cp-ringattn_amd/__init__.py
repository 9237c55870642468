"""Python bindings of ``libhcp_ring_amd.so`` (the C ABI in ``include/hcp_ring.h``).

The operator names mirror the reference's ring-attention backend
(``HcpRingAttentionBackend`` in rust/src/model/attention/ring.rs):

* :func:`positioned_local_compact_partial`  ring.rs:538-571 -> ``hcp_ring_block_partial``
* :func:`positioned_merge_compact_partial`  ring.rs:574-603 -> ``hcp_ring_block_partial``
  (accumulate=1)
* :func:`lse_merge`                         merge of ring-step partials -> ``hcp_ring_lse_merge``
* :func:`decode_local_compact_partial`      ring.rs:515-523 over a paged pool ->
  ``hcp_paged_decode_partial``
* :func:`paged_kv_gather` / :func:`paged_kv_scatter`  the vLLM block extract / insert of
  python/hcp_vllm_block_ring_plugin.py:143-174, 304-337 -> ``hcp_paged_kv_*``
* :func:`ring_attention_replay`             ring.rs:861-1398 for every domain on one GPU ->
  ``hcp_ring_prefill_replay`` (``_paged`` variant stages K/V from a block pool)

Tensors are torch CUDA tensors (device memory and streams only; every computation
runs in the HIP library).  A ``[heads, tokens, head_dim]`` argument may be any strided
view whose last dimension is contiguous, e.g. ``x.permute(1, 0, 2)`` of a token-major
``[tokens, heads, head_dim]`` tensor.  Errors raise :class:`HcpRingError` carrying the
ABI status code and the library's message.
"""
from __future__ import annotations

import ctypes
import math
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# HCP_RING_AMD_LIB selects another build of the library (e.g. one built with other
# compile-time options); the default is the in-tree build.
LIB_PATH = os.environ.get("HCP_RING_AMD_LIB") or os.path.join(HERE, "lib", "libhcp_ring_amd.so")
HEADER = os.path.join(HERE, "..", "include", "hcp_ring.h")
# HCP_RING_ABI_VERSION these bindings are written against; lib() refuses any other.
ABI_VERSION = 3

DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 1, 2, 3

STATUS_NAMES = {
    0: "OK", -1: "MISMATCH", -2: "EXCEPTION", -3: "UNKNOWN", -4: "DEVICE", -5: "BACKEND",
    -6: "INVALID",
}


class HcpRingError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{STATUS_NAMES.get(code, code)}] {message}")
        self.code = code
        self.message = message


class View(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("head_stride", ctypes.c_int64),
                ("seq_stride", ctypes.c_int64)]


class BlockDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("num_q_heads", ctypes.c_int32),
                ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("q_len", ctypes.c_int64), ("kv_len", ctypes.c_int64),
                ("q_offset", ctypes.c_int64), ("kv_offset", ctypes.c_int64),
                ("causal", ctypes.c_int32), ("accumulate", ctypes.c_int32),
                ("scale", ctypes.c_float)]


class PagedPool(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("num_blocks", ctypes.c_int64),
                ("block_size", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("elem_bytes", ctypes.c_int32)]


class PagedRange(ctypes.Structure):
    _fields_ = [("block_table", ctypes.c_void_p), ("table_len", ctypes.c_int64),
                ("table_seq_offset", ctypes.c_int64), ("t0", ctypes.c_int64), ("t1", ctypes.c_int64),
                ("k_out", View), ("v_out", View)]


class DecodeShard(ctypes.Structure):
    _fields_ = [("block_tables", ctypes.c_void_p), ("table_stride", ctypes.c_int64),
                ("table_len", ctypes.c_int64), ("seq_lens", ctypes.c_void_p),
                ("max_len", ctypes.c_int64)]


class DecodeDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("batch", ctypes.c_int32),
                ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("reserved0", ctypes.c_int32),
                ("t0", ctypes.c_int64), ("t1", ctypes.c_int64),
                ("table_stride", ctypes.c_int64), ("table_len", ctypes.c_int64),
                ("scale", ctypes.c_float)]


class ReplayDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("num_q_heads", ctypes.c_int32),
                ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("num_domains", ctypes.c_int32), ("causal", ctypes.c_int32),
                ("chunk_lens", ctypes.POINTER(ctypes.c_int64)), ("scale", ctypes.c_float),
                ("strategy", ctypes.c_int32), ("schedule", ctypes.c_int32)]


class TraceDomain(ctypes.Structure):
    _fields_ = [("domain", ctypes.c_int32), ("workgroups", ctypes.c_int32), ("key_tiles", ctypes.c_int64),
                ("peer_chunks", ctypes.c_int64), ("kv_recv_bytes", ctypes.c_int64), ("kv_sent_bytes", ctypes.c_int64),
                ("span_ms", ctypes.c_double), ("local_cu_ms", ctypes.c_double), ("peer_cu_ms", ctypes.c_double),
                ("local_compute_ms", ctypes.c_double), ("peer_compute_ms", ctypes.c_double),
                ("clock_mhz", ctypes.c_double)]


class TraceLaunch(ctypes.Structure):
    _fields_ = [("workgroups", ctypes.c_int64), ("cus", ctypes.c_int32), ("reserved0", ctypes.c_int32),
                ("span_ms", ctypes.c_double), ("busy_cu_ms", ctypes.c_double), ("idle_gap_cu_ms", ctypes.c_double),
                ("tail_cu_ms", ctypes.c_double), ("head_cu_ms", ctypes.c_double), ("clock_mhz", ctypes.c_double),
                ("wg_ms_min", ctypes.c_double), ("wg_ms_mean", ctypes.c_double), ("wg_ms_max", ctypes.c_double)]


BLOCK_AGENT_MAX = 64
BLOCK_META_MAX = 256


class BlockDescC(ctypes.Structure):
    _fields_ = [("addr", ctypes.c_uint64), ("len", ctypes.c_uint64), ("dev_id", ctypes.c_uint64),
                ("mem_type", ctypes.c_int32), ("meta_len", ctypes.c_uint32),
                ("meta", ctypes.c_uint8 * BLOCK_META_MAX)]


class RemoteBlockDescC(ctypes.Structure):
    _fields_ = [("agent", ctypes.c_char * BLOCK_AGENT_MAX), ("block_id", ctypes.c_uint64), ("desc", BlockDescC)]


class BlockCompletionC(ctypes.Structure):
    _fields_ = [("block_id", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]


class KvFrameDesc(ctypes.Structure):
    _fields_ = [("layer_idx", ctypes.c_int64), ("global_seq_start", ctypes.c_int64),
                ("global_seq_end", ctypes.c_int64), ("dtype", ctypes.c_int32), ("num_heads", ctypes.c_int32),
                ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("len", ctypes.c_int64),
                ("has_positions", ctypes.c_int32), ("reserved0", ctypes.c_int32)]


class PacketFrameDesc(ctypes.Structure):
    _fields_ = [("layer_idx", ctypes.c_int64), ("q_dtype", ctypes.c_int32), ("o_dtype", ctypes.c_int32),
                ("batch", ctypes.c_int32), ("num_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("reserved0", ctypes.c_int32), ("scale", ctypes.c_double)]


class QkvDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("hidden", ctypes.c_int32), ("num_q_heads", ctypes.c_int32),
                ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("rope", ctypes.c_int32),
                ("tokens", ctypes.c_int64), ("rope_rows", ctypes.c_int64)]


# RingSchedulingStrategy (strategy.rs:14-24) -> HCP_STRATEGY_*
STRATEGIES = {"vanilla": 0, "striped": 1, "zigzag": 2}


SCHEDULES = {"auto": 0, "per_step": 1, "fused": 2}
PATHS = {0: "none", 1: "mfma", 2: "ring_fused", 3: "general", 4: "mfma_f32"}


def schedule_code(schedule) -> int:
    """HCP_SCHEDULE_* of a name ("auto", "per_step", "fused") or an int."""
    if isinstance(schedule, int):
        return schedule
    return SCHEDULES[schedule]


def last_path() -> str:
    """Kernel path of this thread's last attention call ("mfma", "ring_fused",
    "general" -- the scalar fp32 kernel -- or "none"), hcp_ring_last_path."""
    return PATHS[lib().hcp_ring_last_path()]


def strategy_code(strategy) -> int:
    if isinstance(strategy, int):
        return strategy
    key = str(strategy).lower()
    if key not in STRATEGIES:
        raise ValueError(f"unknown strategy {strategy!r} (vanilla, striped or zigzag)")
    return STRATEGIES[key]


_lib = None


def lib() -> ctypes.CDLL:
    """Load the HIP library; raises if it was not built (there is no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HcpRingError(-5, f"{LIB_PATH} is missing; run hetero-cp-ringattn_amd/build.py")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    sig = {
        "hcp_ring_last_error": ([], ctypes.c_char_p),
        "hcp_ring_abi_version": ([], ctypes.c_int),
        "hcp_ring_last_path": ([], ctypes.c_int),
        "hcp_ring_device_count": ([ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
        "hcp_ring_fetch_device_errors": ([vp, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
        "hcp_ring_block_partial": ([ctypes.POINTER(BlockDesc), View, View, View, vp, vp, vp],
                                   ctypes.c_int),
        "hcp_ring_block_partial_positioned_workspace_size": ([ctypes.POINTER(BlockDesc)], ctypes.c_size_t),
        "hcp_ring_block_partial_positioned": ([ctypes.POINTER(BlockDesc), View, vp, View, View, vp, vp, vp, vp,
                                               ctypes.c_size_t, vp], ctypes.c_int),
        "hcp_ring_build_assignment": ([i32, i32, ctypes.POINTER(i64), ctypes.POINTER(i32)], ctypes.c_int),
        "hcp_ring_domain_positions": ([i32, i32, ctypes.POINTER(i64), ctypes.POINTER(i64)], ctypes.c_int),
        "hcp_ring_inverse_perm": ([i32, i32, ctypes.POINTER(i64), ctypes.POINTER(i64)], ctypes.c_int),
        "hcp_ring_lse_merge": ([i32, ctypes.POINTER(vp), ctypes.POINTER(vp), i32, i64, i32, i32,
                                View, vp, vp], ctypes.c_int),
        "hcp_paged_kv_gather": ([ctypes.POINTER(PagedPool), vp, i64, i64, i64, i64, View, View,
                                 vp], ctypes.c_int),
        "hcp_paged_kv_scatter": ([ctypes.POINTER(PagedPool), vp, i64, i64, i64, i64, View, View,
                                  i32, vp], ctypes.c_int),
        "hcp_paged_kv_gather_batch": ([ctypes.POINTER(PagedPool), i32, ctypes.POINTER(PagedRange),
                                       vp], ctypes.c_int),
        "hcp_paged_decode_workspace_size": ([ctypes.POINTER(DecodeDesc),
                                             ctypes.POINTER(PagedPool)], ctypes.c_size_t),
        "hcp_paged_decode_partial": ([ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedPool), View,
                                      vp, vp, vp, vp, vp, ctypes.c_size_t, vp], ctypes.c_int),
        "hcp_paged_decode_partial_static": ([ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedPool), View,
                                             vp, vp, vp, vp, vp], ctypes.c_int),
        "hcp_decode_ring_owner": ([i64, i32], ctypes.c_int),
        "hcp_decode_ring_workspace_size": ([ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedPool), i32,
                                            ctypes.POINTER(DecodeShard)], ctypes.c_size_t),
        "hcp_decode_ring_replay": ([ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedPool), View, i32,
                                    ctypes.POINTER(DecodeShard), i32, View, vp, vp, ctypes.c_size_t, vp],
                                   ctypes.c_int),
        "hcp_ring_replay_workspace_size": ([ctypes.POINTER(ReplayDesc), i32], ctypes.c_size_t),
        "hcp_ring_prefill_replay": ([ctypes.POINTER(ReplayDesc), View, View, View, View, vp, vp,
                                     ctypes.c_size_t, vp], ctypes.c_int),
        "hcp_ring_prefill_replay_paged": ([ctypes.POINTER(ReplayDesc), View,
                                           ctypes.POINTER(PagedPool), vp, i64, View, vp, vp,
                                           ctypes.c_size_t, vp], ctypes.c_int),
        "hcp_kv_frame_payload_bytes": ([ctypes.POINTER(KvFrameDesc)], ctypes.c_size_t),
        "hcp_kv_frame_header": ([ctypes.POINTER(KvFrameDesc), vp, ctypes.c_size_t,
                                 ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
        "hcp_kv_frame_parse": ([ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(KvFrameDesc),
                                ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
        "hcp_kv_frame_pack": ([ctypes.POINTER(KvFrameDesc), View, View, vp, vp, vp], ctypes.c_int),
        "hcp_kv_frame_unpack": ([ctypes.POINTER(KvFrameDesc), vp, View, View, vp, vp], ctypes.c_int),
        "hcp_packet_frame_payload_bytes": ([ctypes.POINTER(PacketFrameDesc)], ctypes.c_size_t),
        "hcp_packet_frame_header": ([ctypes.POINTER(PacketFrameDesc), vp, ctypes.c_size_t,
                                     ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
        "hcp_packet_frame_parse": ([ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(PacketFrameDesc),
                                    ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
        "hcp_packet_frame_pack": ([ctypes.POINTER(PacketFrameDesc), View, vp, vp, vp, vp], ctypes.c_int),
        "hcp_packet_frame_unpack": ([ctypes.POINTER(PacketFrameDesc), vp, View, vp, vp, vp], ctypes.c_int),
        "hcp_rope_table": ([i32, i64, ctypes.c_double, vp, vp], ctypes.c_int),
        "hcp_qkv_rope_project": ([ctypes.POINTER(QkvDesc), vp, i64, vp, vp, vp, vp, vp, vp, vp, vp, View, View,
                                  View, vp], ctypes.c_int),
        "hcp_qkv_rope_project_paged": ([ctypes.POINTER(QkvDesc), vp, i64, vp, vp, vp, vp, vp, vp, vp, vp, View,
                                        ctypes.POINTER(PagedPool), vp, i64, i64, i64, vp], ctypes.c_int),
        "hcp_ringattn_runtime_create": ([ctypes.c_char_p, ctypes.POINTER(vp)], ctypes.c_int),
        "hcp_ringattn_runtime_destroy": ([vp], None),
        "hcp_ringattn_runtime_init": ([vp, i32, i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(i64),
                                       ctypes.POINTER(i64), ctypes.c_char_p, i64, i64, i64, i32], ctypes.c_int),
        "hcp_ringattn_runtime_bind_layer": ([vp, i32, i32, View, View, View, f32, vp], ctypes.c_int),
        "hcp_ringattn_runtime_run_layer": ([vp, i32, i64, vp, vp, vp, vp, vp, vp], ctypes.c_int),
        "hcp_ringattn_runtime_shutdown": ([vp], ctypes.c_int),
        "hcp_ringattn_cxx_smoke_domain_count": ([], ctypes.c_int),
        "hcp_synth_normals": ([ctypes.c_uint64, i64, i64, i32, vp, vp], ctypes.c_int),
        "hcp_block_agent_pair_create": ([ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(vp), ctypes.POINTER(vp)],
                                        ctypes.c_int),
        "hcp_block_agent_destroy": ([vp], ctypes.c_int),
        "hcp_block_register": ([vp, vp, ctypes.c_uint64, ctypes.POINTER(i64), i32, ctypes.POINTER(ctypes.c_uint64),
                                ctypes.POINTER(BlockDescC)], ctypes.c_int),
        "hcp_block_deregister": ([vp, ctypes.c_uint64], ctypes.c_int),
        "hcp_block_local_metadata": ([vp, vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
        "hcp_block_load_remote_metadata": ([vp, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p], ctypes.c_int),
        "hcp_block_remote_desc": ([vp, ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(RemoteBlockDescC)],
                                  ctypes.c_int),
        "hcp_block_submit_transfer": ([vp, ctypes.c_uint64, ctypes.POINTER(RemoteBlockDescC), vp], ctypes.c_int),
        "hcp_block_poll_transfers": ([vp, ctypes.POINTER(BlockCompletionC), ctypes.c_size_t,
                                      ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
        "hcp_block_wire_bytes": ([vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
        "hcp_ring_trace_attach": ([vp, ctypes.c_size_t], ctypes.c_int),
        "hcp_ring_trace_record_bytes": ([ctypes.POINTER(ReplayDesc)], ctypes.c_size_t),
        "hcp_ring_trace_read": ([vp, ctypes.POINTER(TraceDomain), i32, ctypes.POINTER(i32),
                                 ctypes.POINTER(TraceLaunch)], ctypes.c_int),
        "hcp_ring_trace_perf_log": ([vp, i32, ctypes.c_char_p], ctypes.c_int),
        "hcp_ring_replay_timing": ([i32], ctypes.c_int),
        "hcp_ring_replay_timing_read": ([ctypes.POINTER(ctypes.c_double), ctypes.POINTER(i64)],
                                        ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    got = L.hcp_ring_abi_version()
    if got != ABI_VERSION:
        raise HcpRingError(-5, f"{LIB_PATH} has ABI version {got}; these bindings need {ABI_VERSION}")
    _lib = L
    return L


def header_functions() -> list[str]:
    """Names of the functions declared in include/hcp_ring.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+\**(hcp_[a-z_0-9]+)\s*\(",
                                 text, flags=re.M)))


def _check(rc: int) -> None:
    if rc != 0:
        msg = lib().hcp_ring_last_error()
        raise HcpRingError(rc, msg.decode() if msg else "")


def last_error() -> str:
    m = lib().hcp_ring_last_error()
    return m.decode() if m else ""


# ---------------------------------------------------------------------------------
# torch plumbing
# ---------------------------------------------------------------------------------
def _torch():
    import torch
    return torch


def dtype_code(t) -> int:
    torch = _torch()
    return {torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16, torch.float32: DTYPE_F32}[t]


def _stream(stream=None):
    """hipStream_t of a torch stream (default: the current one); an int is taken as the
    raw handle (0: the default stream)."""
    if isinstance(stream, int):
        return ctypes.c_void_p(stream)
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def view(t) -> View:
    """[heads, tokens, head_dim] tensor (last dim contiguous) -> hcp_ring_view."""
    if t.dim() != 3:
        raise ValueError("expected a [heads, tokens, head_dim] tensor")
    if t.stride(2) != 1 and t.shape[2] > 1:
        raise ValueError("head_dim must be the contiguous dimension")
    return View(t.data_ptr(), t.stride(0), t.stride(1))


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


# ---------------------------------------------------------------------------------
# (1) block partial
# ---------------------------------------------------------------------------------
def block_partial(q, k, v, q_offset: int, kv_offset: int, causal: bool = True,
                  scale: float | None = None, o=None, lse=None, accumulate: bool = False,
                  stream=None):
    """One ring step: q [Hq, Lq, D], k/v [Hkv, Lk, D] -> (o [Hq,Lq,D] fp32, lse [Hq,Lq] fp32)."""
    torch = _torch()
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    if o is None:
        o = torch.empty((hq, lq, d), dtype=torch.float32, device=q.device)
    if lse is None:
        lse = torch.empty((hq, lq), dtype=torch.float32, device=q.device)
    desc = BlockDesc(dtype_code(q.dtype), hq, hkv, d, lq, lk, q_offset, kv_offset,
                     1 if causal else 0, 1 if accumulate else 0,
                     scale if scale is not None else 1.0 / math.sqrt(d))
    _check(lib().hcp_ring_block_partial(ctypes.byref(desc), view(q), view(k), view(v), _ptr(o),
                                        _ptr(lse), _stream(stream)))
    return o, lse


def block_partial_positioned(q, q_positions, k, v, kv_positions, causal: bool = True,
                             scale: float | None = None, o=None, lse=None, accumulate: bool = False,
                             workspace=None, stream=None):
    """As :func:`block_partial` with explicit global positions: q_positions [Lq] and
    kv_positions [Lk] (device int64 tensors, each in any order); key j is visible to
    query i iff kv_positions[j] <= q_positions[i] (ring.rs:249-273).  A key list that
    is not non-decreasing is sorted on the device with its K / V rows (workspace)."""
    torch = _torch()
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    if o is None:
        o = torch.empty((hq, lq, d), dtype=torch.float32, device=q.device)
    if lse is None:
        lse = torch.empty((hq, lq), dtype=torch.float32, device=q.device)
    desc = BlockDesc(dtype_code(q.dtype), hq, hkv, d, lq, lk, 0, 0, 1 if causal else 0, 1 if accumulate else 0,
                     scale if scale is not None else 1.0 / math.sqrt(d))
    for name, t, n in (("q_positions", q_positions, lq), ("kv_positions", kv_positions, lk)):
        if t.dtype != torch.int64 or t.numel() != n or not t.is_contiguous() or t.device != q.device:
            raise ValueError(f"{name} must be a contiguous int64 tensor of {n} elements on {q.device}")
    need = lib().hcp_ring_block_partial_positioned_workspace_size(ctypes.byref(desc))
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    _check(lib().hcp_ring_block_partial_positioned(ctypes.byref(desc), view(q), _ptr(q_positions), view(k),
                                                   view(v), _ptr(kv_positions), _ptr(o), _ptr(lse),
                                                   _ptr(workspace), workspace.numel(), _stream(stream)))
    return o, lse


def positioned_local_compact_partial(q, q_offset, k, v, kv_offset, scale=None, stream=None):
    """ring.rs:538-571 on the GPU: causal partial over one source -> (o fp32, lse fp32).

    q_offset / kv_offset are either the global start of contiguous positions (ints) or
    position tensors (device int64, as the reference's q_pos / k_pos)."""
    if isinstance(q_offset, int) and isinstance(kv_offset, int):
        return block_partial(q, k, v, q_offset, kv_offset, True, scale, stream=stream)
    return block_partial_positioned(q, q_offset, k, v, kv_offset, True, scale, stream=stream)


def positioned_merge_compact_partial(q, q_offset, o, lse, k, v, kv_offset, scale=None,
                                     stream=None):
    """ring.rs:574-603 on the GPU: merge (o, lse) with one more causal source (new tensors)."""
    o2, l2 = o.clone(), lse.clone()
    if isinstance(q_offset, int) and isinstance(kv_offset, int):
        return block_partial(q, k, v, q_offset, kv_offset, True, scale, o=o2, lse=l2,
                             accumulate=True, stream=stream)
    return block_partial_positioned(q, q_offset, k, v, kv_offset, True, scale, o=o2, lse=l2,
                                    accumulate=True, stream=stream)


# ---------------------------------------------------------------------------------
# (2) LSE merge
# ---------------------------------------------------------------------------------
def lse_merge(o_parts, lse_parts, out_dtype=None, out=None, lse_out=None, stream=None):
    """Merge partials (each o [H,L,D] fp32 contiguous, lse [H,L] fp32)."""
    torch = _torch()
    h, l, d = o_parts[0].shape
    if out is None:
        out = torch.empty((h, l, d), dtype=out_dtype or torch.bfloat16, device=o_parts[0].device)
    if lse_out is None:
        lse_out = torch.empty((h, l), dtype=torch.float32, device=o_parts[0].device)
    n = len(o_parts)
    op = (ctypes.c_void_p * n)(*[p.data_ptr() for p in o_parts])
    lp = (ctypes.c_void_p * n)(*[p.data_ptr() for p in lse_parts])
    _check(lib().hcp_ring_lse_merge(n, op, lp, h, l, d, dtype_code(out.dtype), view(out),
                                    _ptr(lse_out), _stream(stream)))
    return out, lse_out


# ---------------------------------------------------------------------------------
# (3) paged KV staging
# ---------------------------------------------------------------------------------
def paged_pool(pool) -> PagedPool:
    """pool tensor [2, num_blocks, block_size, Hkv, D] -> hcp_paged_pool."""
    if pool.dim() != 5 or pool.shape[0] != 2 or not pool.is_contiguous():
        raise ValueError("pool must be a contiguous [2, num_blocks, block_size, Hkv, D] tensor")
    return PagedPool(pool.data_ptr(), pool.shape[1], pool.shape[2], pool.shape[3], pool.shape[4],
                     pool.element_size())


def paged_kv_gather(pool, block_table, table_seq_offset, t0, t1, k_out=None, v_out=None,
                    stream=None):
    torch = _torch()
    _, nb, bs, hkv, d = pool.shape
    if k_out is None:
        k_out = torch.empty((hkv, t1 - t0, d), dtype=pool.dtype, device=pool.device)
        v_out = torch.empty((hkv, t1 - t0, d), dtype=pool.dtype, device=pool.device)
    pp = paged_pool(pool)
    _check(lib().hcp_paged_kv_gather(ctypes.byref(pp), _ptr(block_table), block_table.numel(),
                                     table_seq_offset, t0, t1, view(k_out), view(v_out),
                                     _stream(stream)))
    return k_out, v_out


def paged_kv_scatter(pool, block_table, table_seq_offset, t0, t1, k_in, v_in, zero_tail=True,
                     stream=None):
    pp = paged_pool(pool)
    _check(lib().hcp_paged_kv_scatter(ctypes.byref(pp), _ptr(block_table), block_table.numel(),
                                      table_seq_offset, t0, t1, view(k_in), view(v_in),
                                      1 if zero_tail else 0, _stream(stream)))


def paged_kv_gather_batch(pool, ranges, stream=None):
    """ranges: list of (block_table, table_seq_offset, t0, t1, k_out, v_out); one launch."""
    paged_gather_plan(pool, ranges, stream)()


def paged_gather_plan(pool, ranges, stream=None):
    """Builds the descriptors of a batched gather once and returns a callable that
    launches it (for repeated staging of the same ranges without per-call host work).
    The tensors must stay alive while the callable is used."""
    n = len(ranges)
    arr = (PagedRange * max(n, 1))()
    for i, (tab, off, t0, t1, ko, vo) in enumerate(ranges):
        arr[i] = PagedRange(tab.data_ptr(), tab.numel(), off, t0, t1, view(ko), view(vo))
    pp = paged_pool(pool)
    st = _stream(stream)
    fn = lib().hcp_paged_kv_gather_batch

    def run():
        _check(fn(ctypes.byref(pp), n, arr, st))

    return run


def fetch_device_errors(stream=None) -> int:
    flags = ctypes.c_int(0)
    _check(lib().hcp_ring_fetch_device_errors(_stream(stream), ctypes.byref(flags)))
    return flags.value


# ---------------------------------------------------------------------------------
# (4) paged decode
# ---------------------------------------------------------------------------------
def decode_desc(q, pool, block_tables, t0, t1, scale=None) -> DecodeDesc:
    b, hq, d = q.shape
    return DecodeDesc(dtype_code(q.dtype), b, hq, pool.shape[3], d, 0, t0, t1,
                      block_tables.stride(0), block_tables.shape[1],
                      scale if scale is not None else 1.0 / math.sqrt(d))


def decode_workspace_size(q, pool, block_tables, t0, t1) -> int:
    desc = decode_desc(q, pool, block_tables, t0, t1)
    pp = paged_pool(pool)
    return lib().hcp_paged_decode_workspace_size(ctypes.byref(desc), ctypes.byref(pp))


def decode_local_compact_partial(q, pool, block_tables, t0, t1, seq_lens=None, scale=None,
                                 workspace=None, o=None, lse=None, stream=None):
    """ring.rs:515-523 / 625-639 for a batch: q [B, Hq, D] over tokens [t0, t1) of each
    sequence's paged KV -> (o [B,Hq,D] fp32, lse [B,Hq] fp32)."""
    torch = _torch()
    b, hq, d = q.shape
    desc = decode_desc(q, pool, block_tables, t0, t1, scale)
    pp = paged_pool(pool)
    need = lib().hcp_paged_decode_workspace_size(ctypes.byref(desc), ctypes.byref(pp))
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    if o is None:
        o = torch.empty((b, hq, d), dtype=torch.float32, device=q.device)
        lse = torch.empty((b, hq), dtype=torch.float32, device=q.device)
    qv = View(q.data_ptr(), q.stride(1), q.stride(0))
    _check(lib().hcp_paged_decode_partial(ctypes.byref(desc), ctypes.byref(pp), qv,
                                          _ptr(block_tables), _ptr(seq_lens), _ptr(o), _ptr(lse),
                                          _ptr(workspace), workspace.numel(), _stream(stream)))
    return o, lse


# ---------------------------------------------------------------------------------
# (4b) decode Q-ring with growth sharding
# ---------------------------------------------------------------------------------
def decode_ring_owner(global_pos: int, num_domains: int) -> int:
    """Domain that persists the decode token at global_pos (ring.rs:1921-1942)."""
    r = lib().hcp_decode_ring_owner(global_pos, num_domains)
    if r < 0:
        raise HcpRingError(r, "bad position or domain count")
    return r


def _shards(shards):
    arr = (DecodeShard * len(shards))()
    for i, (tables, seq_lens, max_len) in enumerate(shards):
        arr[i] = DecodeShard(tables.data_ptr() if tables is not None else None,
                             tables.stride(0) if tables is not None else 0,
                             tables.shape[1] if tables is not None else 0,
                             seq_lens.data_ptr() if seq_lens is not None else None, max_len)
    return arr


def _ring_desc(q, pool, scale=None):
    b, hq, d = q.shape
    return DecodeDesc(dtype_code(q.dtype), b, hq, pool.shape[3], d, 0, 0, 0, 0, 0,
                      scale if scale is not None else 1.0 / math.sqrt(d))


def decode_ring_workspace_size(q, pool, shards) -> int:
    """Workspace bytes hcp_decode_ring_replay needs for these shards."""
    desc, pp, arr = _ring_desc(q, pool), paged_pool(pool), _shards(shards)
    return lib().hcp_decode_ring_workspace_size(ctypes.byref(desc), ctypes.byref(pp), len(shards), arr)


def decode_ring_replay(q, pool, shards, seed_domain, scale=None, out=None, lse_out=None, workspace=None,
                       stream=None):
    """ring_decode_attention (ring.rs:665-818) for a batch on one GPU.

    q [B, Hq, D]; shards: per domain (block_tables [B, n] int32, seq_lens [B] int32 or
    None, max_len); the packet starts at seed_domain and visits its successors.
    Returns (out [B, Hq, D] in q's dtype, lse [B, Hq] fp32)."""
    torch = _torch()
    b, hq, d = q.shape
    desc = _ring_desc(q, pool, scale)
    pp = paged_pool(pool)
    arr = _shards(shards)
    n = len(shards)
    need = lib().hcp_decode_ring_workspace_size(ctypes.byref(desc), ctypes.byref(pp), n, arr)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=q.device)
    if lse_out is None:
        lse_out = torch.empty((b, hq), dtype=torch.float32, device=q.device)
    qv = View(q.data_ptr(), q.stride(1), q.stride(0))
    ov = View(out.data_ptr(), out.stride(1), out.stride(0))
    _check(lib().hcp_decode_ring_replay(ctypes.byref(desc), ctypes.byref(pp), qv, n, arr, seed_domain, ov,
                                        _ptr(lse_out), _ptr(workspace), workspace.numel(), _stream(stream)))
    return out, lse_out


# ---------------------------------------------------------------------------------
# (5) ring replay
# ---------------------------------------------------------------------------------
def replay_desc(dtype, hq, hkv, d, chunks, causal=True, scale=None, strategy="vanilla", schedule="auto"):
    arr = (ctypes.c_int64 * len(chunks))(*chunks)
    desc = ReplayDesc(dtype_code(dtype), hq, hkv, d, len(chunks), 1 if causal else 0, arr,
                      scale if scale is not None else 1.0 / math.sqrt(d), strategy_code(strategy),
                      schedule_code(schedule))
    return desc, arr


def replay_workspace_size(dtype, hq, hkv, d, chunks, causal=True, paged=False, strategy="vanilla",
                          schedule="auto") -> int:
    desc, _arr = replay_desc(dtype, hq, hkv, d, chunks, causal, strategy=strategy, schedule=schedule)
    return lib().hcp_ring_replay_workspace_size(ctypes.byref(desc), 1 if paged else 0)


def ring_attention_replay(q, k, v, chunks, causal=True, scale=None, out=None, lse_out=None,
                          workspace=None, stream=None, strategy="vanilla", schedule="auto"):
    """Every domain's ring on one GPU.  q [Hq, S, D], k/v [Hkv, S, D] (strided views ok)
    -> (out [Hq, S, D] in q's dtype, lse [Hq, S] fp32).

    Rows are in domain-major order (row r = position ``domain_positions(chunks,
    strategy)[r]``; the global order for "vanilla"); ``inverse_perm`` maps back.
    ``schedule``: "auto" (one fused launch where it applies), "per_step" (one grouped
    launch per ring step) or "fused".  Fused with "striped" / "zigzag" positions: K/V
    copied in position order, then one positions-mode block over the whole sequence;
    fused fp32: one block over the sequence on the fp32 matrix-core kernel."""
    torch = _torch()
    hq, s, d = q.shape
    hkv = k.shape[0]
    desc, arr = replay_desc(q.dtype, hq, hkv, d, chunks, causal, scale, strategy, schedule)
    need = lib().hcp_ring_replay_workspace_size(ctypes.byref(desc), 0)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    if out is None:
        out = torch.empty((hq, s, d), dtype=q.dtype, device=q.device)
    if lse_out is None:
        lse_out = torch.empty((hq, s), dtype=torch.float32, device=q.device)
    _check(lib().hcp_ring_prefill_replay(ctypes.byref(desc), view(q), view(k), view(v), view(out),
                                         _ptr(lse_out), _ptr(workspace), workspace.numel(),
                                         _stream(stream)))
    del arr
    return out, lse_out


def ring_attention_replay_paged(q, pool, block_table, chunks, causal=True, scale=None, out=None,
                                lse_out=None, workspace=None, stream=None, strategy="vanilla", schedule="auto"):
    """As :func:`ring_attention_replay`, K/V gathered from a paged pool (the pool holds
    the sequence in the same domain-major order): per ring step with "per_step", every
    chunk once before the fused launch otherwise."""
    torch = _torch()
    hq, s, d = q.shape
    hkv = pool.shape[3]
    desc, arr = replay_desc(q.dtype, hq, hkv, d, chunks, causal, scale, strategy, schedule)
    need = lib().hcp_ring_replay_workspace_size(ctypes.byref(desc), 1)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    if out is None:
        out = torch.empty((hq, s, d), dtype=q.dtype, device=q.device)
    if lse_out is None:
        lse_out = torch.empty((hq, s), dtype=torch.float32, device=q.device)
    pp = paged_pool(pool)
    _check(lib().hcp_ring_prefill_replay_paged(ctypes.byref(desc), view(q), ctypes.byref(pp),
                                               _ptr(block_table), block_table.numel(), view(out),
                                               _ptr(lse_out), _ptr(workspace), workspace.numel(),
                                               _stream(stream)))
    del arr
    return out, lse_out


# ---------------------------------------------------------------------------------
# (6b) block-direct transport (block_transport.rs KvBlockTransport)
# ---------------------------------------------------------------------------------
class BlockAgent:
    """One side of a linked pair of block transports (the KvBlockTransport methods of
    block_transport.rs:97-126 over hcp_block_*).  Blocks are device or host memory given
    as torch tensors / numpy arrays (kept referenced while registered)."""

    def __init__(self, handle, name: str):
        self._h = ctypes.c_void_p(handle)
        self.name = name
        self._keep = {}

    @staticmethod
    def pair(name_a: str = "agent-a", name_b: str = "agent-b"):
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        _check(lib().hcp_block_agent_pair_create(name_a.encode(), name_b.encode(), ctypes.byref(a), ctypes.byref(b)))
        return BlockAgent(a.value, name_a), BlockAgent(b.value, name_b)

    def register_block(self, tensor):
        """(block id, descriptor dict) of the tensor's memory, its shape in the metadata."""
        if hasattr(tensor, "data_ptr"):
            ptr, nbytes, shape = tensor.data_ptr(), tensor.numel() * tensor.element_size(), list(tensor.shape)
        else:
            ptr, nbytes, shape = tensor.ctypes.data, tensor.nbytes, list(tensor.shape)
        dims = (ctypes.c_int64 * max(len(shape), 1))(*shape)
        bid, desc = ctypes.c_uint64(), BlockDescC()
        _check(lib().hcp_block_register(self._h, ptr, nbytes, dims, len(shape), ctypes.byref(bid), ctypes.byref(desc)))
        self._keep[bid.value] = tensor
        return bid.value, block_desc_dict(desc)

    def deregister_block(self, block_id: int):
        _check(lib().hcp_block_deregister(self._h, block_id))
        self._keep.pop(block_id, None)

    def local_metadata(self) -> bytes:
        n = ctypes.c_size_t()
        _check(lib().hcp_block_local_metadata(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        _check(lib().hcp_block_local_metadata(self._h, buf, n.value, ctypes.byref(n)))
        return buf.raw[: n.value]

    def load_remote_metadata(self, blob: bytes) -> str:
        name = ctypes.create_string_buffer(BLOCK_AGENT_MAX)
        _check(lib().hcp_block_load_remote_metadata(self._h, blob, len(blob), name))
        return name.value.decode()

    def remote_desc(self, peer: str, block_id: int) -> RemoteBlockDescC:
        out = RemoteBlockDescC()
        _check(lib().hcp_block_remote_desc(self._h, peer.encode(), block_id, ctypes.byref(out)))
        return out

    def submit_transfer(self, local_block_id: int, remote: RemoteBlockDescC, stream=None):
        _check(lib().hcp_block_submit_transfer(self._h, local_block_id, ctypes.byref(remote), _stream(stream)))

    def poll_transfers(self, capacity: int = 64):
        out = (BlockCompletionC * capacity)()
        n = ctypes.c_size_t()
        _check(lib().hcp_block_poll_transfers(self._h, out, capacity, ctypes.byref(n)))
        return [(out[i].block_id, out[i].bytes) for i in range(n.value)]

    def wire_bytes(self):
        sent, recv = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().hcp_block_wire_bytes(self._h, ctypes.byref(sent), ctypes.byref(recv)))
        return sent.value, recv.value

    def destroy(self):
        if self._h:
            _check(lib().hcp_block_agent_destroy(self._h))
            self._h = None
            self._keep.clear()


def block_desc_dict(d: BlockDescC) -> dict:
    return {"addr": d.addr, "len": d.len, "dev_id": d.dev_id, "mem_type": d.mem_type,
            "meta": bytes(d.meta[: d.meta_len])}


# ---------------------------------------------------------------------------------
# (6) wire frames (tcp.rs)
# ---------------------------------------------------------------------------------
def _header(fn, desc) -> bytes:
    n = ctypes.c_size_t(0)
    getattr(lib(), fn)(ctypes.byref(desc), None, 0, ctypes.byref(n))
    buf = ctypes.create_string_buffer(n.value)
    _check(getattr(lib(), fn)(ctypes.byref(desc), buf, n.value, ctypes.byref(n)))
    return buf.raw[:n.value]


def kv_frame_desc(layer_idx, start, end, dtype, num_heads, num_kv_heads, head_dim, length,
                  has_positions) -> KvFrameDesc:
    return KvFrameDesc(layer_idx, start, end, dtype_code(dtype) if not isinstance(dtype, int) else dtype,
                       num_heads, num_kv_heads, head_dim, length, 1 if has_positions else 0, 0)


def kv_frame_header(desc: KvFrameDesc) -> bytes:
    """[meta_len u32 BE][meta_json] of a KV block frame (tcp.rs:161-207)."""
    return _header("hcp_kv_frame_header", desc)


def kv_frame_pack(k, v, layer_idx, start, end, positions=None, num_heads=None, stream=None):
    """KvBlock -> (header bytes, payload uint8 device tensor).  k / v [Hkv, L, D] views;
    the wire carries num_heads (default Hkv) heads, head h from view head h / rep."""
    torch = _torch()
    hkv, length, d = k.shape
    desc = kv_frame_desc(layer_idx, start, end, k.dtype, num_heads or hkv, hkv, d, length, positions is not None)
    n = lib().hcp_kv_frame_payload_bytes(ctypes.byref(desc))
    if n == 0:
        raise HcpRingError(-6, "invalid KV frame descriptor")
    payload = torch.empty(n, dtype=torch.uint8, device=k.device)
    _check(lib().hcp_kv_frame_pack(ctypes.byref(desc), view(k), view(v), _ptr(positions), _ptr(payload),
                                   _stream(stream)))
    return kv_frame_header(desc), payload


def kv_frame_parse(frame: bytes):
    """(KvFrameDesc, header bytes) of a received frame."""
    desc = KvFrameDesc()
    hb = ctypes.c_size_t(0)
    _check(lib().hcp_kv_frame_parse(frame, len(frame), ctypes.byref(desc), ctypes.byref(hb)))
    return desc, hb.value


def kv_frame_unpack(desc: KvFrameDesc, payload, k_out, v_out, positions_out=None, stream=None):
    _check(lib().hcp_kv_frame_unpack(ctypes.byref(desc), _ptr(payload), view(k_out), view(v_out),
                                     _ptr(positions_out), _stream(stream)))
    return k_out, v_out, positions_out


def packet_frame_pack(q, o, lse, layer_idx, scale, o_dtype=None, stream=None):
    """RingPacket -> (header bytes, payload).  q [B, H, D] view, o fp32 [B, H, D], lse fp32 [B, H]."""
    torch = _torch()
    b, h, d = q.shape
    desc = PacketFrameDesc(layer_idx, dtype_code(q.dtype), dtype_code(o_dtype or torch.float32), b, h, d, 0,
                           float(scale))
    n = lib().hcp_packet_frame_payload_bytes(ctypes.byref(desc))
    if n == 0:
        raise HcpRingError(-6, "invalid packet frame descriptor")
    payload = torch.empty(n, dtype=torch.uint8, device=q.device)
    qv = View(q.data_ptr(), q.stride(1), q.stride(0))
    _check(lib().hcp_packet_frame_pack(ctypes.byref(desc), qv, _ptr(o), _ptr(lse), _ptr(payload), _stream(stream)))
    return _header("hcp_packet_frame_header", desc), payload


def packet_frame_parse(frame: bytes):
    desc = PacketFrameDesc()
    hb = ctypes.c_size_t(0)
    _check(lib().hcp_packet_frame_parse(frame, len(frame), ctypes.byref(desc), ctypes.byref(hb)))
    return desc, hb.value


def packet_frame_unpack(desc: PacketFrameDesc, payload, q_out, o_out, lse_out, stream=None):
    qv = View(q_out.data_ptr(), q_out.stride(1), q_out.stride(0))
    _check(lib().hcp_packet_frame_unpack(ctypes.byref(desc), _ptr(payload), qv, _ptr(o_out), _ptr(lse_out),
                                         _stream(stream)))
    return q_out, o_out, lse_out


# ---------------------------------------------------------------------------------
# (7) fused QKV projection + RoPE + KV append
# ---------------------------------------------------------------------------------
def rope_table(head_dim: int, rows: int, base: float = 10000.0, device="cuda", stream=None):
    """cos / sin caches of RotaryEmbedding::new (rotary.rs:64-97) -> fp32 [2, rows, D/2]."""
    torch = _torch()
    t = torch.empty((2, rows, head_dim // 2), dtype=torch.float32, device=device)
    _check(lib().hcp_rope_table(head_dim, rows, float(base), _ptr(t), _stream(stream)))
    return t


def _qkv_args(x, wq, num_q_heads, num_kv_heads, head_dim, positions, table, rope):
    torch = _torch()
    tokens, hidden = x.shape
    if x.stride(1) != 1:
        raise ValueError("x rows must be contiguous")
    desc = QkvDesc(dtype_code(x.dtype), hidden, num_q_heads, num_kv_heads, head_dim, 1 if rope else 0, tokens,
                   table.shape[1] if table is not None else 0)
    if rope and (positions is None or positions.dtype != torch.int64 or positions.numel() != tokens):
        raise ValueError("rope needs int64 positions of one entry per token")
    return desc


def qkv_rope_project(x, wq, wk, wv, num_q_heads, num_kv_heads, head_dim, positions=None, table=None,
                     bq=None, bk=None, bv=None, rope=True, q_out=None, k_out=None, v_out=None, stream=None):
    """ring.rs:1865-1908 on the GPU: x [L, hidden] -> q [Hq, L, D], k / v [Hkv, L, D]
    (q, k rotated at ``positions`` with the ``table`` of :func:`rope_table`)."""
    torch = _torch()
    tokens = x.shape[0]
    desc = _qkv_args(x, wq, num_q_heads, num_kv_heads, head_dim, positions, table, rope)
    if q_out is None:
        q_out = torch.empty((num_q_heads, tokens, head_dim), dtype=x.dtype, device=x.device)
    if k_out is None:
        k_out = torch.empty((num_kv_heads, tokens, head_dim), dtype=x.dtype, device=x.device)
    if v_out is None:
        v_out = torch.empty((num_kv_heads, tokens, head_dim), dtype=x.dtype, device=x.device)
    _check(lib().hcp_qkv_rope_project(ctypes.byref(desc), _ptr(x), x.stride(0), _ptr(wq), _ptr(wk), _ptr(wv),
                                      _ptr(bq), _ptr(bk), _ptr(bv), _ptr(positions), _ptr(table), view(q_out),
                                      view(k_out), view(v_out), _stream(stream)))
    return q_out, k_out, v_out


def qkv_rope_project_paged(x, wq, wk, wv, num_q_heads, num_kv_heads, head_dim, pool, block_table,
                           table_seq_offset: int, t0: int, positions=None, table=None, bq=None, bk=None, bv=None,
                           rope=True, q_out=None, stream=None):
    """As :func:`qkv_rope_project`, k / v appended to the paged pool at sequence
    positions t0 .. t0 + L (KvCache::update, cache.rs:191-251)."""
    torch = _torch()
    tokens = x.shape[0]
    desc = _qkv_args(x, wq, num_q_heads, num_kv_heads, head_dim, positions, table, rope)
    if q_out is None:
        q_out = torch.empty((num_q_heads, tokens, head_dim), dtype=x.dtype, device=x.device)
    pp = paged_pool(pool)
    _check(lib().hcp_qkv_rope_project_paged(ctypes.byref(desc), _ptr(x), x.stride(0), _ptr(wq), _ptr(wk),
                                            _ptr(wv), _ptr(bq), _ptr(bk), _ptr(bv), _ptr(positions), _ptr(table),
                                            view(q_out), ctypes.byref(pp), _ptr(block_table), block_table.numel(),
                                            table_seq_offset, t0, _stream(stream)))
    return q_out


# ---------------------------------------------------------------------------------
# (8) domain runtime (RingAttnRuntime)
# ---------------------------------------------------------------------------------
class RingAttnRuntime:
    """The reference's per-domain runtime (include/hcp_ringattn/core/ringattn_runtime.h)
    on the GPU: Init / BindLayer / RunRingAttentionLayer / Shutdown."""

    def __init__(self, device_type: str = "hip"):
        h = ctypes.c_void_p()
        _check(lib().hcp_ringattn_runtime_create(device_type.encode(), ctypes.byref(h)))
        self._h = h
        self._shape = None

    def init(self, domain_index: int, domain_ids, seq_chunk_lens, num_heads: int, head_dim: int, dtype,
             block_sizes=None, device: str = "hip", global_seq_len: int | None = None):
        n = len(domain_ids)
        ids = (ctypes.c_char_p * n)(*[d.encode() for d in domain_ids])
        lens = (ctypes.c_int64 * n)(*seq_chunk_lens)
        bss = (ctypes.c_int64 * n)(*(block_sizes or [16] * n))
        total = sum(seq_chunk_lens) if global_seq_len is None else global_seq_len
        code = dtype if isinstance(dtype, int) else dtype_code(dtype)
        _check(lib().hcp_ringattn_runtime_init(self._h, domain_index, n, ids, lens, bss, device.encode(), total,
                                               num_heads, head_dim, code))
        self._shape = (num_heads, seq_chunk_lens[domain_index], head_dim)

    def bind_layer(self, layer: int, q, k, v, scale: float | None = None, stream=None):
        """q [Hq, L, D], k / v [Hkv, L, D] device views of this domain's chunk."""
        sc = scale if scale is not None else 1.0 / math.sqrt(q.shape[2])
        _check(lib().hcp_ringattn_runtime_bind_layer(self._h, layer, k.shape[0], view(q), view(k), view(v), sc,
                                                     _stream(stream)))

    def run_ring_attention_layer(self, layer: int, initial_state=None):
        """-> (running_max [H, L], running_sum [H, L], output [H, L, D]) numpy fp32."""
        import numpy as np
        h, l, d = self._shape or (0, 0, 0)  # before Init the library reports the error
        mx, sm, out = (np.empty((max(h, 1), max(l, 1)), np.float32), np.empty((max(h, 1), max(l, 1)), np.float32),
                       np.empty((max(h, 1), max(l, 1), max(d, 1)), np.float32))
        mx, sm, out = mx[:h, :l], sm[:h, :l], out[:h, :l, :d]
        ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        if initial_state is None:
            args = (0, None, None, None)
        else:
            im, isum, io = (np.ascontiguousarray(a, dtype=np.float32) for a in initial_state)
            args = (l, ptr(im), ptr(isum), ptr(io))
        _check(lib().hcp_ringattn_runtime_run_layer(self._h, layer, *args, ptr(mx), ptr(sm), ptr(out)))
        return mx, sm, out

    def shutdown(self):
        _check(lib().hcp_ringattn_runtime_shutdown(self._h))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.hcp_ringattn_runtime_destroy(h)
            self._h = None


def cxx_smoke_domain_count() -> int:
    """The reference's three-domain runtime smoke (rust_bridge.cc:646-681) on "hip" runtimes."""
    return lib().hcp_ringattn_cxx_smoke_domain_count()


# ---------------------------------------------------------------------------------
# synthetic inputs and host helpers
# ---------------------------------------------------------------------------------
def synth_normals(seed: int, offset: int, count: int, out, stream=None):
    """Fill ``out`` (contiguous, F32/BF16/F16) with normals offset..offset+count-1."""
    _check(lib().hcp_synth_normals(ctypes.c_uint64(seed), offset, count, dtype_code(out.dtype),
                                   _ptr(out), _stream(stream)))
    return out


def trace_record_bytes(dtype, hq, hkv, d, chunks, causal=True) -> int:
    """Bytes of trace records one fused replay of this shape writes."""
    desc, _arr = replay_desc(dtype, hq, hkv, d, chunks, causal)
    return lib().hcp_ring_trace_record_bytes(ctypes.byref(desc))


def trace_attach(buffer) -> None:
    """Trace every later fused replay with vanilla positions on this thread into
    ``buffer`` (a device tensor, kept referenced by the caller); ``None`` detaches."""
    if buffer is None:
        _check(lib().hcp_ring_trace_attach(None, 0))
    else:
        _check(lib().hcp_ring_trace_attach(_ptr(buffer), buffer.numel() * buffer.element_size()))


def _struct_dict(x) -> dict:
    return {name: getattr(x, name) for name, _ in x._fields_ if not name.startswith("reserved")}


def trace_read(stream=None):
    """(per-domain statistics, launch statistics) of the last traced replay."""
    doms = (TraceDomain * 64)()
    n = ctypes.c_int32(0)
    launch = TraceLaunch()
    _check(lib().hcp_ring_trace_read(_stream(stream), doms, 64, ctypes.byref(n), ctypes.byref(launch)))
    return [_struct_dict(doms[i]) for i in range(n.value)], _struct_dict(launch)


def trace_perf_log(layer_idx: int, path: str | None = None, stream=None) -> None:
    """Append the last traced replay's ring_attention events (JSONL) to ``path`` or
    to $HCP_PERF_LOG (ring.rs:820-844)."""
    _check(lib().hcp_ring_trace_perf_log(_stream(stream), layer_idx, path.encode() if path else None))


def replay_timing(enable: bool) -> None:
    """Turn per-launch HIP-event timing of the replay driver on or off."""
    _check(lib().hcp_ring_replay_timing(1 if enable else 0))


def replay_timing_read() -> dict:
    """Summed kernel ms and launch counts since the last read: block, merge, gather."""
    ms = (ctypes.c_double * 3)()
    n = (ctypes.c_int64 * 3)()
    _check(lib().hcp_ring_replay_timing_read(ms, n))
    return {k: (ms[i], n[i]) for i, k in enumerate(("block", "merge", "gather"))}


def vanilla_offsets(chunks, seq_len: int | None = None) -> list[int]:
    """Global start of each domain's contiguous chunk (strategy.rs:53-63).

    Raises ValueError when the chunks do not sum to ``seq_len`` (the InvalidChunkSum of
    rust/src/error.rs:15-16, rust/src/smoke/reference_algo.rs:92-116) or a chunk is empty.
    """
    if any(c <= 0 for c in chunks):
        raise ValueError("every chunk must be non-empty")
    if seq_len is not None and sum(chunks) != seq_len:
        raise ValueError(f"invalid chunk sum: actual {sum(chunks)}, expected {seq_len}")
    out, acc = [], 0
    for c in chunks:
        out.append(acc)
        acc += c
    return out


def vanilla_assignment(chunks) -> list[int]:
    """Owner domain of every global position for contiguous chunks (strategy.rs:53-63)."""
    out = []
    for d, c in enumerate(chunks):
        out.extend([d] * c)
    return out


def _strategy_call(fn, ctype, chunks, strategy):
    n = len(chunks)
    arr = (ctypes.c_int64 * n)(*chunks)
    out = (ctype * max(sum(chunks), 1))()
    _check(getattr(lib(), fn)(strategy_code(strategy), n, arr, out))
    return list(out[:sum(chunks)])


def build_assignment(chunks, strategy="vanilla") -> list[int]:
    """Domain owning each global position (build_assignment, strategy.rs:53-110)."""
    return _strategy_call("hcp_ring_build_assignment", ctypes.c_int32, chunks, strategy)


def domain_positions(chunks, strategy="vanilla") -> list[int]:
    """Every domain's ascending positions, concatenated in domain order
    (build_domain_positions, strategy.rs:114-121)."""
    return _strategy_call("hcp_ring_domain_positions", ctypes.c_int64, chunks, strategy)


def inverse_perm(chunks, strategy="vanilla") -> list[int]:
    """Row of each global position in the domain-major concatenation
    (build_inverse_perm, strategy.rs:129-143)."""
    return _strategy_call("hcp_ring_inverse_perm", ctypes.c_int64, chunks, strategy)


def ring_sources(target: int, num_domains: int) -> list[int]:
    """Sources visited by ``target`` in ring order: local, then the predecessor chain
    (ring.rs:1208-1311 with the mock ring of rust/src/model/transport/mock.rs:143-149)."""
    return [(target - s) % num_domains for s in range(num_domains)]
