// extern "C" boundary of the ring-attention path (declared in include/hcp_ring.h).
//
// Conventions follow the reference's FFI bridge (src/rust_bridge.cc): int status,
// caller-owned buffers, every exception caught at the boundary, and a message getter
// -- here thread-local instead of the bridge's process-global std::string
// (rust_bridge.cc:19-27,614-644).  The C++ ring-replay driver (the single-GPU
// counterpart of HcpRingAttentionBackend::ring_attention, ring.rs:861-1398) lives here
// too; it only enqueues kernels.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <functional>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "../../include/hcp_ring.h"
#include "../../include/hcp_ringattn/core/ringattn_runtime.h"

namespace hcp {


// Sticky device-side error flags, one copy per device (static device variable).
__device__ int g_hcp_device_errors;

// Scratch of hcp_paged_decode_partial_static (the per-split decode partials of one
// call), one copy per device for the life of the process.  Host code never uses this
// name as an address: static_scratch() resolves the device's copy.
constexpr size_t kStaticScratchBytes = HCP_DECODE_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// Device address of `scratch` on the current device, looked up once per device (with
// that device current) by hipGetSymbolAddress.
void* static_scratch() {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  HCP_HIP(hipGetDevice(&dev));
  require(dev >= 0 && dev < 64, "device index out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* ptr = nullptr;
    HCP_HIP(hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch)));
    require(ptr != nullptr, "no device address for the static scratch");
    ptrs[dev] = ptr;
  }
  return ptrs[dev];
}

int* device_error_flags() {
  static std::mutex mu;
  static int* ptrs[64] = {};
  int dev = 0;
  HCP_HIP(hipGetDevice(&dev));
  require(dev >= 0 && dev < 64, "device index out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    HCP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(g_hcp_device_errors)));
    ptrs[dev] = static_cast<int*>(p);
  }
  return ptrs[dev];
}

namespace {

thread_local std::string g_last_error;
thread_local int g_last_path = HCP_PATH_NONE;

// The kernel a block launch takes (see launch_block_partial / launch_block_group).
int block_path(const BlockLaunch& L) {
  if (!L.force_general && block_uses_mfma(L.dtype, L.d)) return HCP_PATH_MFMA;
  return block_uses_mfma_f32(L) ? HCP_PATH_MFMA_F32 : HCP_PATH_GENERAL;
}

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

template <typename F>
int guarded(const char* fn, F&& body) {
  try {
    g_last_error.clear();
    body();
    return HCP_RING_OK;
  } catch (const Error& e) {
    return fail(e.code, std::string(fn) + ": " + e.what());
  } catch (const std::exception& e) {
    return fail(HCP_RING_E_EXCEPTION, std::string(fn) + ": " + e.what());
  } catch (...) {
    return fail(HCP_RING_E_UNKNOWN, std::string(fn) + ": unknown exception");
  }
}

int elem_size(int dtype) {
  switch (dtype) {
    case kF16:
    case kBF16: return 2;
    case kF32: return 4;
    default: throw Error(-6, "unsupported dtype " + std::to_string(dtype));
  }
}

void check_view(const hcp_ring_view& v, const char* name, int64_t len) {
  if (len == 0) return;
  require(v.data != nullptr, std::string(name) + ": null data pointer");
  require(v.head_stride >= 0 && v.seq_stride > 0, std::string(name) + ": strides must be positive");
}

void check_block_desc(const hcp_ring_block_desc* d) {
  require(d != nullptr, "null descriptor");
  elem_size(d->dtype);
  require(d->num_q_heads > 0 && d->num_kv_heads > 0, "head counts must be positive");
  require(d->num_q_heads % d->num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  require(d->head_dim > 0 && d->head_dim <= 256, "head_dim must be in [1, 256]");
  require(d->q_len >= 0 && d->kv_len >= 0, "lengths must be >= 0");
  require(d->q_len <= INT32_MAX && d->kv_len <= INT32_MAX, "lengths must fit in int32");
  require(d->causal == 0 || d->causal == 1, "causal must be 0 or 1");
  require(d->accumulate == 0 || d->accumulate == 1, "accumulate must be 0 or 1");
  require(d->scale > 0.f, "scale must be positive");
}

bool mfma_layout_ok(const hcp_ring_view& v) {
  return reinterpret_cast<uintptr_t>(v.data) % 16 == 0 && v.head_stride % 8 == 0 && v.seq_stride % 8 == 0;
}

// The merge writes 4 elements per lane: rows must start on 4-element boundaries.
void check_out_view(const hcp_ring_view& out, int dtype) {
  const int es = elem_size(dtype);
  require(reinterpret_cast<uintptr_t>(out.data) % (4 * es) == 0 && out.head_stride % 4 == 0 &&
              out.seq_stride % 4 == 0,
          "out must be aligned to 4 elements with strides multiple of 4");
}

BlockLaunch make_launch(const hcp_ring_block_desc* d, hcp_ring_view q, hcp_ring_view k, hcp_ring_view v,
                        float* o, float* lse) {
  BlockLaunch L;
  L.dtype = d->dtype;
  L.q = q.data; L.k = k.data; L.v = v.data;
  L.q_hs = q.head_stride; L.q_ss = q.seq_stride;
  L.k_hs = k.head_stride; L.k_ss = k.seq_stride;
  L.v_hs = v.head_stride; L.v_ss = v.seq_stride;
  L.o = o; L.lse = lse;
  L.hq = d->num_q_heads; L.hkv = d->num_kv_heads; L.d = d->head_dim;
  L.lq = d->q_len; L.lk = d->kv_len;
  L.q_off = d->q_offset; L.k_off = d->kv_offset;
  L.causal = d->causal; L.accumulate = d->accumulate;
  L.scale = d->scale;
  // The matrix-core kernel reads 16-byte rows; other layouts take the general kernel.
  L.force_general = !(mfma_layout_ok(q) && mfma_layout_ok(k) && mfma_layout_ok(v));
  return L;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

StrategySpec make_spec(int32_t strategy, int32_t n, const int64_t* chunks, bool allow_empty) {
  require(strategy == kStrategyVanilla || strategy == kStrategyStriped || strategy == kStrategyZigZag,
          "strategy must be 0 (vanilla), 1 (striped) or 2 (zigzag)");
  require(n >= 1 && n <= kMaxDomains, "num_domains must be in [1, 64]");
  require(chunks != nullptr, "null chunk_lens");
  StrategySpec sp{};
  sp.strategy = strategy;
  sp.n = n;
  int64_t total = 0;
  for (int d = 0; d < n; ++d) {
    require(chunks[d] >= (allow_empty ? 0 : 1), allow_empty ? "chunk lengths must be >= 0" : "every chunk length must be >= 1");
    sp.chunks[d] = chunks[d];
    total += chunks[d];
    require(total <= INT32_MAX, "total sequence length must fit in int32");
  }
  return sp;
}

// ---- ring replay planning ----
struct ReplayPlan {
  int n;
  StrategySpec spec;
  int schedule = HCP_SCHEDULE_AUTO;
  size_t fused_stage_bytes = 0;           // fused paged replay: each of the K and V staging buffers [Hkv, S, D]
  // Fused replay with explicit positions (after the paged staging): positions int64 [S],
  // the copy flag, the row of each position int32 [S], K / V in position order
  // [Hkv, S, D] and the per-row key limits int32 [S].
  size_t fp_pos = 0, fp_flag = 0, fp_rows = 0, fp_kc = 0, fp_vc = 0, fp_lim = 0;
  size_t fp_total = 0;
  bool positioned = false;                // causal with explicit positions (Striped / ZigZag)
  size_t pos_off = 0, lim_off = 0;        // workspace: positions int64 [S], key limits int32 [N, S]
  std::vector<int64_t> len, off, first, last;
  std::vector<std::vector<int>> sources;  // per target, in ring order, non-empty only
  std::vector<size_t> state_off;          // byte offset of each target's running fp32 (o, lse)
  size_t partial_bytes = 0;
  size_t staging_off = 0;
  size_t staging_bytes_per_domain = 0;
  size_t total = 0;
  int64_t seq = 0;
};

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Optional per-launch timing of the replay driver: HIP events recorded on the launch
// stream around every block-kernel, merge and gather launch (benchmark instrumentation).
enum TimedKind { kTimedBlock = 0, kTimedMerge = 1, kTimedGather = 2, kTimedKinds = 3 };
struct ReplayTiming {
  std::mutex mu;
  bool enabled = false;
  std::vector<hipEvent_t> pool;
  std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
};
ReplayTiming& timing() {
  static ReplayTiming t;
  return t;
}
hipEvent_t take_event(ReplayTiming& t) {
  if (!t.pool.empty()) {
    hipEvent_t e = t.pool.back();
    t.pool.pop_back();
    return e;
  }
  hipEvent_t e;
  HCP_HIP(hipEventCreate(&e));
  return e;
}
// Runs `launch` bracketed by events when timing is on.
template <typename F>
void timed(int kind, hipStream_t stream, F&& launch) {
  ReplayTiming& t = timing();
  std::unique_lock<std::mutex> lock(t.mu);
  if (!t.enabled) {
    lock.unlock();
    launch();
    return;
  }
  hipEvent_t a = take_event(t), b = take_event(t);
  HCP_HIP(hipEventRecord(a, stream));
  launch();
  HCP_HIP(hipEventRecord(b, stream));
  t.pending.push_back({kind, {a, b}});
}

ReplayPlan plan_replay(const hcp_ring_replay_desc* d, bool paged) {
  require(d != nullptr, "null descriptor");
  require(d->num_domains >= 1 && d->num_domains <= 64, "num_domains must be in [1, 64]");
  require(d->chunk_lens != nullptr, "null chunk_lens");
  const StrategySpec spec = make_spec(d->strategy, d->num_domains, d->chunk_lens, false);
  require(d->schedule == HCP_SCHEDULE_AUTO || d->schedule == HCP_SCHEDULE_PER_STEP ||
              d->schedule == HCP_SCHEDULE_FUSED,
          "schedule must be 0 (auto), 1 (per ring step) or 2 (fused)");
  require(d->num_q_heads > 0 && d->num_kv_heads > 0 && d->num_q_heads % d->num_kv_heads == 0,
          "bad head counts");
  require(d->head_dim > 0 && d->head_dim <= 256, "head_dim must be in [1, 256]");
  require(d->causal == 0 || d->causal == 1, "causal must be 0 or 1");
  require(d->scale > 0.f, "scale must be positive");
  const int es = elem_size(d->dtype);
  ReplayPlan p;
  p.n = d->num_domains;
  p.spec = spec;
  p.positioned = d->causal && d->strategy != kStrategyVanilla;
  int64_t acc = 0;
  int64_t max_len = 0;
  for (int i = 0; i < p.n; ++i) {
    const int64_t l = d->chunk_lens[i];
    p.len.push_back(l);
    p.off.push_back(acc);
    // Domain-major storage: rows [off, off + len) hold domain i's tokens in ascending
    // position order, first and last of which bound its positions.
    p.first.push_back(strategy_position(spec, i, 0));
    p.last.push_back(strategy_position(spec, i, l - 1));
    acc += l;
    max_len = std::max(max_len, l);
  }
  p.seq = acc;
  p.sources.resize(p.n);
  p.state_off.resize(p.n);
  size_t cur = 0;
  for (int t = 0; t < p.n; ++t) {
    for (int s = 0; s < p.n; ++s) {
      const int src = ((t - s) % p.n + p.n) % p.n;
      // A source wholly in the target's future contributes nothing (ring.rs:222-228).
      if (d->causal && p.first[src] > p.last[t]) continue;
      p.sources[t].push_back(src);
    }
    // A target with one source writes its output rows directly and needs no state.
    p.state_off[t] = cur;
    if (p.sources[t].size() > 1) {
      const size_t rows = static_cast<size_t>(d->num_q_heads) * p.len[t];
      cur += align256(rows * d->head_dim * sizeof(float)) + align256(rows * sizeof(float));
    }
  }
  p.partial_bytes = cur;
  if (p.positioned) {
    p.pos_off = cur;
    cur += align256(static_cast<size_t>(p.seq) * sizeof(int64_t));
    p.lim_off = cur;
    cur += align256(static_cast<size_t>(p.n) * p.seq * sizeof(int32_t));
  }
  p.staging_off = cur;
  if (paged) {
    p.staging_bytes_per_domain =
        align256(static_cast<size_t>(max_len) * d->num_kv_heads * d->head_dim * es) * 2;
    cur += p.staging_bytes_per_domain * p.n;
  }
  p.total = cur;
  p.schedule = d->schedule;
  // The fused schedule keeps no state in HBM; paged, it stages the whole sequence once
  // at the start of the workspace (the per-step layout's need covers it: its staging
  // alone holds N chunks of the longest length).
  p.fused_stage_bytes = align256(static_cast<size_t>(p.seq) * d->num_kv_heads * d->head_dim * es);
  if (p.positioned) {
    size_t c = paged ? 2 * p.fused_stage_bytes : 0;
    const size_t n8 = align256(static_cast<size_t>(p.seq) * sizeof(int64_t));
    const size_t n4 = align256(static_cast<size_t>(p.seq) * sizeof(int32_t));
    p.fp_pos = c;
    c += n8;
    p.fp_flag = c;
    c += 256;
    p.fp_rows = c;
    c += n4;
    p.fp_kc = c;
    c += p.fused_stage_bytes;
    p.fp_vc = c;
    c += p.fused_stage_bytes;
    p.fp_lim = c;
    c += n4;
    p.fp_total = c;
  }
  if (d->schedule == HCP_SCHEDULE_FUSED) {
    p.total = p.positioned ? p.fp_total : paged ? 2 * p.fused_stage_bytes : 0;
  } else if (d->schedule == HCP_SCHEDULE_AUTO && p.positioned) {
    // AUTO runs the fused layout where the views allow it, else the per-step one
    p.total = std::max(p.total, p.fp_total);
  }
  return p;
}

// Trace of fused replays (hcp_ring_trace_attach): the caller's device buffer and the
// geometry of the last traced replay, per thread like the rest of the call state.
struct TraceState {
  void* buf = nullptr;
  size_t bytes = 0;
  bool have = false;  // a traced replay ran since the buffer was attached
  int n = 0, hkv = 0, d = 0, es = 0;
  std::vector<int64_t> len;
  std::vector<std::vector<int>> sources;  // per target, ring order
  int64_t blocks = 0;
  int stride = 0;
};
thread_local TraceState g_trace;

// Whole replay as one fused-ring launch (HCP_SCHEDULE_FUSED): q / k / v / out are the
// whole-sequence views.
void run_replay_fused(const hcp_ring_replay_desc* d, const ReplayPlan& p, hcp_ring_view q, hcp_ring_view k,
                      hcp_ring_view v, hcp_ring_view out, float* lse_out, hipStream_t stream) {
  RingLaunch L{};
  L.dtype = d->dtype;
  L.d = d->head_dim;
  L.hq = d->num_q_heads;
  L.hkv = d->num_kv_heads;
  L.n = p.n;
  L.causal = d->causal;
  L.scale = d->scale;
  L.q = q.data; L.k = k.data; L.v = v.data;
  L.q_hs = q.head_stride; L.q_ss = q.seq_stride;
  L.k_hs = k.head_stride; L.k_ss = k.seq_stride;
  L.v_hs = v.head_stride; L.v_ss = v.seq_stride;
  L.out = out.data;
  L.out_hs = out.head_stride;
  L.out_ss = out.seq_stride;
  L.lse = lse_out;
  L.lse_hs = p.seq;
  L.len = p.len.data();
  if (g_trace.buf != nullptr) {
    const int64_t blocks = ring_fused_workgroups(L.hq, L.hkv, p.n, p.len.data());
    const int stride = ring_trace_words(p.n);
    const size_t need = static_cast<size_t>(blocks) * stride * sizeof(uint32_t);
    require(g_trace.bytes >= need, "trace buffer too small: need " + std::to_string(need) + " bytes");
    L.trace = static_cast<uint32_t*>(g_trace.buf);
    L.trace_stride = stride;
    g_trace.have = true;
    g_trace.n = p.n;
    g_trace.hkv = d->num_kv_heads;
    g_trace.d = d->head_dim;
    g_trace.es = elem_size(d->dtype);
    g_trace.len = p.len;
    g_trace.sources = p.sources;
    g_trace.blocks = blocks;
    g_trace.stride = stride;
  }
  timed(kTimedBlock, stream, [&] { launch_ring_fused(L, stream); });
  g_last_path = HCP_PATH_RING_FUSED;
}

// One block over the whole sequence: S query rows against S keys (the domains' chunks
// in domain-major order), the output rows and LSE written directly.  With vanilla
// positions it is the whole causal (or full) attention of the replay; with explicit
// positions the caller adds the row limits and the position-ordered K / V.
BlockLaunch whole_sequence_launch(const hcp_ring_replay_desc* d, const ReplayPlan& p, hcp_ring_view q,
                                  hcp_ring_view k, hcp_ring_view v, hcp_ring_view out, float* lse_out) {
  hcp_ring_block_desc bd;
  bd.dtype = d->dtype;
  bd.num_q_heads = d->num_q_heads;
  bd.num_kv_heads = d->num_kv_heads;
  bd.head_dim = d->head_dim;
  bd.q_len = p.seq;
  bd.kv_len = p.seq;
  bd.q_offset = 0;
  bd.kv_offset = 0;
  bd.causal = d->causal;
  bd.accumulate = 0;
  bd.scale = d->scale;
  BlockLaunch L = make_launch(&bd, q, k, v, nullptr, nullptr);
  L.fin_out = out.data;
  L.fin_dtype = d->dtype;
  L.fin_hs = out.head_stride;
  L.fin_ss = out.seq_stride;
  L.fin_lse = lse_out;
  L.fin_lse_hs = p.seq;
  return L;
}

// Whole replay with explicit positions (Striped / ZigZag) as one positions-mode launch
// of the block kernel: attention over a set of keys does not depend on their order, so
// with K / V put in position order every query row sees a prefix of the keys -- those
// at positions up to its own (ring.rs:249-273 masks key by key) -- and the whole
// sequence is one block of S query rows against S keys, its output rows and LSE written
// directly, with no running state in HBM between ring steps.  A strategy's positions
// are a permutation of [0, S): the row of each position and each row's key limit
// (position + 1) follow in one pass, with no sort.  q / k / v / out are the whole-
// sequence views in domain-major order (rows [off_t, off_t + len_t) hold domain t's
// tokens in ascending position order); k / v paged: the staged copies.
void run_replay_fused_positioned(const hcp_ring_replay_desc* d, const ReplayPlan& p, hcp_ring_view q,
                                 hcp_ring_view k, hcp_ring_view v, hcp_ring_view out, float* lse_out, char* base,
                                 hipStream_t stream) {
  const int es = elem_size(d->dtype);
  int64_t* pos = reinterpret_cast<int64_t*>(base + p.fp_pos);
  int* flag = reinterpret_cast<int*>(base + p.fp_flag);
  int32_t* rows = reinterpret_cast<int32_t*>(base + p.fp_rows);
  int32_t* lim = reinterpret_cast<int32_t*>(base + p.fp_lim);
  launch_domain_positions(p.spec, p.seq, pos, stream);
  launch_position_inverse(pos, p.seq, rows, lim, flag, device_error_flags(), stream);
  KvSortedGather g{};
  g.flag = flag;
  g.rows = rows;
  g.n = p.seq;
  g.hkv = d->num_kv_heads;
  g.row_bytes = static_cast<int64_t>(d->head_dim) * es;
  g.k = static_cast<const char*>(k.data);
  g.v = static_cast<const char*>(v.data);
  g.k_hs_bytes = k.head_stride * es;
  g.k_ss_bytes = k.seq_stride * es;
  g.v_hs_bytes = v.head_stride * es;
  g.v_ss_bytes = v.seq_stride * es;
  g.kc = base + p.fp_kc;
  g.vc = base + p.fp_vc;
  timed(kTimedGather, stream, [&] { launch_kv_sorted_gather(g, stream); });
  BlockLaunch L = whole_sequence_launch(d, p, q, k, v, out, lse_out);
  L.q_lim = lim;
  L.kv_sel = flag;
  L.k_alt = g.kc;
  L.v_alt = g.vc;
  L.alt_hs = p.seq * d->head_dim;
  L.alt_ss = d->head_dim;
  timed(kTimedBlock, stream, [&] { launch_block_partial(L, stream); });
  g_last_path = block_path(L);
}

// Per-domain and per-launch statistics of the last traced replay (layout of the
// records: include/hcp_ring.h, hcp_ring_trace_attach).
void trace_stats(hipStream_t stream, std::vector<hcp_ring_trace_domain>& doms, hcp_ring_trace_launch& L) {
  const TraceState& t = g_trace;
  require(t.buf != nullptr, "no trace buffer attached");
  require(t.have, "no traced replay since the trace buffer was attached");
  HCP_HIP(hipStreamSynchronize(stream));
  std::vector<uint32_t> w(static_cast<size_t>(t.blocks) * t.stride);
  HCP_HIP(hipMemcpy(w.data(), t.buf, w.size() * sizeof(uint32_t), hipMemcpyDeviceToHost));
  auto u64 = [&](int64_t rec, int word) {
    const uint32_t* r = w.data() + rec * t.stride + word;
    return static_cast<uint64_t>(r[0]) | (static_cast<uint64_t>(r[1]) << 32);
  };
  constexpr double kTicksPerMs = 1e5;  // s_memrealtime runs at 100 MHz
  doms.assign(t.n, hcp_ring_trace_domain{});
  std::vector<uint64_t> d_first(t.n, UINT64_MAX), d_last(t.n, 0), d_ticks(t.n, 0), d_clk(t.n, 0);
  std::map<uint32_t, std::vector<std::pair<uint64_t, uint64_t>>> per_cu;
  L = hcp_ring_trace_launch{};
  uint64_t first = UINT64_MAX, last = 0, busy = 0, clk = 0, wmin = UINT64_MAX, wmax = 0;
  for (int64_t r = 0; r < t.blocks; ++r) {
    const uint64_t t0 = u64(r, 0), t1 = u64(r, 2), c0 = u64(r, 4), c1 = u64(r, 6);
    const uint32_t* hdr = w.data() + r * t.stride;
    const int dom = static_cast<int>(hdr[10] & 0xffffu);
    require(t1 > t0 && dom < t.n, "incomplete trace record " + std::to_string(r));
    hcp_ring_trace_domain& D = doms[dom];
    D.workgroups += 1;
    D.key_tiles += hdr[12];
    uint64_t prev = t0, local = 0, peer = 0;
    for (int s = 0; s < t.n; ++s) {
      const uint64_t st = u64(r, 16 + 2 * s);
      if (st == 0) continue;
      const uint64_t seg = st > prev ? st - prev : 0;
      (s == 0 ? local : peer) += seg;
      prev = std::max(prev, st);
    }
    D.local_cu_ms += local / kTicksPerMs;
    D.peer_cu_ms += peer / kTicksPerMs;
    d_first[dom] = std::min(d_first[dom], t0);
    d_last[dom] = std::max(d_last[dom], t1);
    d_ticks[dom] += t1 - t0;
    d_clk[dom] += c1 - c0;
    per_cu[(hdr[9] << 16) | ((hdr[8] >> 8) & 0xffu)].push_back({t0, t1});
    first = std::min(first, t0);
    last = std::max(last, t1);
    busy += t1 - t0;
    clk += c1 - c0;
    wmin = std::min(wmin, t1 - t0);
    wmax = std::max(wmax, t1 - t0);
  }
  L.workgroups = t.blocks;
  L.cus = static_cast<int32_t>(per_cu.size());
  L.span_ms = (last - first) / kTicksPerMs;
  L.busy_cu_ms = busy / kTicksPerMs;
  L.clock_mhz = busy > 0 ? 100.0 * clk / busy : 0.0;
  L.wg_ms_min = wmin / kTicksPerMs;
  L.wg_ms_max = wmax / kTicksPerMs;
  L.wg_ms_mean = t.blocks > 0 ? L.busy_cu_ms / t.blocks : 0.0;
  for (auto& kv : per_cu) {
    auto& v = kv.second;
    std::sort(v.begin(), v.end());
    L.head_cu_ms += (v.front().first - first) / kTicksPerMs;
    L.tail_cu_ms += (last - v.back().second) / kTicksPerMs;
    uint64_t end = v.front().second;
    for (size_t i = 1; i < v.size(); ++i) {
      if (v[i].first > end) L.idle_gap_cu_ms += (v[i].first - end) / kTicksPerMs;
      end = std::max(end, v[i].second);
    }
  }
  const double cus = std::max(1, L.cus);
  const int64_t row_bytes = static_cast<int64_t>(t.hkv) * t.d * t.es * 2;  // K and V of one token
  for (int dom = 0; dom < t.n; ++dom) {
    hcp_ring_trace_domain& D = doms[dom];
    D.domain = dom;
    D.span_ms = d_last[dom] > d_first[dom] ? (d_last[dom] - d_first[dom]) / kTicksPerMs : 0.0;
    D.local_compute_ms = D.local_cu_ms / cus;
    D.peer_compute_ms = D.peer_cu_ms / cus;
    D.clock_mhz = d_ticks[dom] > 0 ? 100.0 * d_clk[dom] / d_ticks[dom] : 0.0;
    for (int src : t.sources[dom])
      if (src != dom) {
        D.peer_chunks += 1;
        D.kv_recv_bytes += t.len[src] * row_bytes;
      }
    for (int tgt = 0; tgt < t.n; ++tgt)
      if (tgt != dom)
        for (int src : t.sources[tgt])
          if (src == dom) D.kv_sent_bytes += t.len[dom] * row_bytes;
  }
}

void run_replay(const hcp_ring_replay_desc* d, hcp_ring_view q, hcp_ring_view k, hcp_ring_view v,
                const hcp_paged_pool* pool, const int32_t* table, int64_t table_len,
                hcp_ring_view out, float* lse_out, void* ws, size_t ws_bytes, hipStream_t stream) {
  const bool paged = pool != nullptr;
  ReplayPlan p = plan_replay(d, paged);
  g_last_path = HCP_PATH_NONE;
  require(ws != nullptr || p.total == 0, "null workspace");
  require(ws_bytes >= p.total, "workspace too small: need " + std::to_string(p.total) + " bytes");
  check_view(q, "q", p.seq);
  check_view(out, "out", p.seq);
  check_out_view(out, d->dtype);
  require(d->head_dim % 4 == 0, "head_dim must be a multiple of 4");
  const int es = elem_size(d->dtype);
  char* base = static_cast<char*>(ws);
  int* err = paged ? device_error_flags() : nullptr;
  if (paged) {
    require(pool->data != nullptr && table != nullptr, "null pool or block table");
    require(pool->num_kv_heads == d->num_kv_heads && pool->head_dim == d->head_dim,
            "pool shape does not match the descriptor");
    require(pool->elem_bytes == es, "pool element size does not match dtype");
    require(pool->block_size >= 1, "block_size must be >= 1");
    require((p.seq - 1) / pool->block_size < table_len, "block table shorter than the sequence");
  } else {
    check_view(k, "k", p.seq);
    check_view(v, "v", p.seq);
  }
  // Fused schedule: one matrix-core launch for the whole replay -- BF16/F16 (head_dim a
  // multiple of 8 up to 128, 16-byte rows): the fused ring for vanilla positions, one
  // positions-mode block over the sequence otherwise; FP32 (head_dim a multiple of 4 up
  // to 128, an output aligned for 16-byte stores): one block over the sequence on the
  // fp32 matrix-core kernel.  AUTO takes it wherever it applies.
  const bool f32 = d->dtype == kF32;
  const bool fused_ok =
      f32 ? block_uses_mfma_f32(whole_sequence_launch(d, p, q, k, v, out, lse_out))
          : ring_fused_applies(d->dtype, d->head_dim) && mfma_layout_ok(q) && mfma_layout_ok(out) &&
                (paged || (mfma_layout_ok(k) && mfma_layout_ok(v)));
  if (p.schedule == HCP_SCHEDULE_FUSED)
    require(fused_ok,
            "the fused schedule needs BF16/F16 with head_dim a multiple of 8 up to 128 and 16-byte "
            "aligned rows and strides, or FP32 with head_dim a multiple of 4 up to 128 and an output "
            "aligned for 16-byte stores");
  if (fused_ok && p.schedule != HCP_SCHEDULE_PER_STEP) {
    hcp_ring_view kk = k, vv = v;
    if (paged) {
      // every chunk staged once, in one batched bit-exact gather, as [Hkv, S, D]
      const int64_t hs = p.seq * d->head_dim;
      kk = hcp_ring_view{base, hs, d->head_dim};
      vv = hcp_ring_view{base + p.fused_stage_bytes, hs, d->head_dim};
      std::vector<PagedRangeDesc> rs;
      for (int s = 0; s < p.n; ++s) {
        const int64_t o = p.off[s] * d->head_dim;
        rs.push_back(PagedRangeDesc{table, 0, p.off[s], p.off[s] + p.len[s], static_cast<char*>(kk.data) + o * es,
                                    static_cast<char*>(vv.data) + o * es, hs, d->head_dim});
      }
      timed(kTimedGather, stream, [&] {
        launch_paged_copy_batch(true, pool->data, pool->num_blocks, pool->block_size, pool->num_kv_heads,
                                pool->head_dim, pool->elem_bytes, static_cast<int>(rs.size()), rs.data(), 0, err,
                                stream);
      });
    }
    if (p.positioned) {
      run_replay_fused_positioned(d, p, q, kk, vv, out, lse_out, base, stream);
    } else if (f32) {
      const BlockLaunch L = whole_sequence_launch(d, p, q, kk, vv, out, lse_out);
      timed(kTimedBlock, stream, [&] { launch_block_partial(L, stream); });
      g_last_path = block_path(L);
    } else {
      run_replay_fused(d, p, q, kk, vv, out, lse_out, stream);
    }
    return;
  }
  // Explicit positions: generate every domain's positions in HBM, then the key limits
  // of every (target row, source) pair, once per replay.
  int32_t* lims = nullptr;
  if (p.positioned) {
    int64_t* pos = reinterpret_cast<int64_t*>(base + p.pos_off);
    lims = reinterpret_cast<int32_t*>(base + p.lim_off);
    launch_domain_positions(p.spec, p.seq, pos, stream);
    KeyLimitArgs la{};
    la.q_pos = pos;
    la.n_q = p.seq;
    la.k_pos = pos;
    int64_t max_len = 0;
    for (int i = 0; i < p.n; ++i) {
      la.k_off[i] = p.off[i];
      la.k_len[i] = p.len[i];
      max_len = std::max(max_len, p.len[i]);
    }
    la.lim = lims;
    la.lim_stride = p.seq;
    la.err = device_error_flags();
    launch_key_limits(la, p.n, max_len, stream);
  }
  // Ring step s: domain t consumes source (t - s) mod N (local first, then the
  // predecessor chain, as the mock ring delivers it: mock.rs:143-149).
  for (int s = 0; s < p.n; ++s) {
    std::vector<hcp_ring_view> ks(p.n, k), vs(p.n, v);
    if (paged) {
      // Stage every domain's source chunk of this step into its ring buffer: one
      // batched, bit-exact gather for the whole step.
      std::vector<PagedRangeDesc> rs;
      for (int t = 0; t < p.n; ++t) {
        const int src = ((t - s) % p.n + p.n) % p.n;
        bool used = false;
        for (int x : p.sources[t]) used = used || x == src;
        if (!used) continue;
        char* stg = base + p.staging_off + static_cast<size_t>(t) * p.staging_bytes_per_domain;
        const int64_t hs = p.len[src] * d->head_dim;  // [Hkv, L, D] packed per source length
        ks[t] = hcp_ring_view{stg, hs, d->head_dim};
        vs[t] = hcp_ring_view{stg + p.staging_bytes_per_domain / 2, hs, d->head_dim};
        rs.push_back(PagedRangeDesc{table, 0, p.off[src], p.off[src] + p.len[src], ks[t].data, vs[t].data, hs,
                                    d->head_dim});
      }
      timed(kTimedGather, stream, [&] {
        launch_paged_copy_batch(true, pool->data, pool->num_blocks, pool->block_size, pool->num_kv_heads,
                                pool->head_dim, pool->elem_bytes, static_cast<int>(rs.size()), rs.data(), 0, err,
                                stream);
      });
    }
    // The step's blocks write distinct targets' state: one grouped launch.
    std::vector<BlockLaunch> step_launches;
    for (int t = 0; t < p.n; ++t) {
      const int src = ((t - s) % p.n + p.n) % p.n;
      int idx = -1;
      for (size_t i = 0; i < p.sources[t].size(); ++i)
        if (p.sources[t][i] == src) idx = static_cast<int>(i);
      if (idx < 0) continue;  // fully-future source
      hcp_ring_view kv_k = ks[t], kv_v = vs[t];
      if (!paged) {
        kv_k.data = static_cast<char*>(k.data) + p.off[src] * k.seq_stride * es;
        kv_v.data = static_cast<char*>(v.data) + p.off[src] * v.seq_stride * es;
      }
      hcp_ring_view qv = q;
      qv.data = static_cast<char*>(q.data) + p.off[t] * q.seq_stride * es;
      hcp_ring_block_desc bd;
      bd.dtype = d->dtype;
      bd.num_q_heads = d->num_q_heads;
      bd.num_kv_heads = d->num_kv_heads;
      bd.head_dim = d->head_dim;
      bd.q_len = p.len[t];
      bd.kv_len = p.len[src];
      bd.q_offset = p.off[t];
      bd.kv_offset = p.off[src];
      bd.causal = d->causal;
      // Sources arrive in ring order and are folded into the target's running fp32
      // state as they come (positioned_merge_compact_partial, ring.rs:574-603); the
      // last one also normalises into the output rows [off_t, off_t + len_t) and the
      // LSE, so no separate merge pass is needed.
      bd.accumulate = idx > 0 ? 1 : 0;
      bd.scale = d->scale;
      char* state = base + p.state_off[t];
      const size_t rows = static_cast<size_t>(d->num_q_heads) * p.len[t];
      float* po = reinterpret_cast<float*>(state);
      float* pl = reinterpret_cast<float*>(state + align256(rows * d->head_dim * sizeof(float)));
      BlockLaunch L = make_launch(&bd, qv, kv_k, kv_v, po, pl);
      if (lims != nullptr) L.q_lim = lims + static_cast<int64_t>(src) * p.seq + p.off[t];
      if (idx + 1 == static_cast<int>(p.sources[t].size())) {
        L.fin_out = static_cast<char*>(out.data) + p.off[t] * out.seq_stride * es;
        L.fin_dtype = d->dtype;
        L.fin_hs = out.head_stride;
        L.fin_ss = out.seq_stride;
        L.fin_lse = lse_out ? lse_out + p.off[t] : nullptr;
        L.fin_lse_hs = p.seq;
      }
      step_launches.push_back(L);
    }
    timed(kTimedBlock, stream, [&] {
      launch_block_group(step_launches.data(), static_cast<int>(step_launches.size()), stream);
    });
    for (const BlockLaunch& L : step_launches)
      if (g_last_path != HCP_PATH_GENERAL) g_last_path = block_path(L);
  }
}

// Workspace of the positioned block entry: the per-row key limits, then (causal) the
// key-order flag, the two (key, row) sort buffers and the sorted-row K / V copies.
struct PositionedWorkspace {
  size_t lim = 0, flag = 0, key[2] = {0, 0}, row[2] = {0, 0}, kc = 0, vc = 0, total = 0;
};

PositionedWorkspace positioned_workspace(const hcp_ring_block_desc* d) {
  PositionedWorkspace w;
  size_t cur = 0;
  w.lim = cur;
  cur += align256(static_cast<size_t>(d->q_len) * sizeof(int32_t));
  if (d->causal == 1 && d->kv_len > 0) {
    const size_t n = static_cast<size_t>(d->kv_len);
    w.flag = cur;
    cur += 256;
    for (int i = 0; i < 2; ++i) {
      w.key[i] = cur;
      cur += align256(n * sizeof(int64_t));
    }
    for (int i = 0; i < 2; ++i) {
      w.row[i] = cur;
      cur += align256(n * sizeof(int32_t));
    }
    const size_t copy = align256(static_cast<size_t>(d->num_kv_heads) * n * d->head_dim * elem_size(d->dtype));
    w.kc = cur;
    cur += copy;
    w.vc = cur;
    cur += copy;
  }
  w.total = cur;
  return w;
}

}  // namespace

int block_transport_guard(const char* fn, const std::function<void()>& body) { return guarded(fn, body); }

}  // namespace hcp

using namespace hcp;

extern "C" {

const char* hcp_ring_last_error(void) { return g_last_error.c_str(); }

int hcp_ring_last_path(void) { return g_last_path; }

int hcp_ring_abi_version(void) { return HCP_RING_ABI_VERSION; }

int hcp_ring_device_count(int* count) {
  return guarded(__func__, [&] {
    require(count != nullptr, "null count");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
      *count = 0;
      throw Error(HCP_RING_E_BACKEND, "no usable HIP device");
    }
    *count = n;
  });
}

int hcp_ring_fetch_device_errors(void* stream, int* flags) {
  return guarded(__func__, [&] {
    require(flags != nullptr, "null flags");
    int* dev = device_error_flags();
    HCP_HIP(hipStreamSynchronize(as_stream(stream)));
    int host = 0;
    HCP_HIP(hipMemcpy(&host, dev, sizeof(int), hipMemcpyDeviceToHost));
    const int zero = 0;
    HCP_HIP(hipMemcpy(dev, &zero, sizeof(int), hipMemcpyHostToDevice));
    *flags = host;
  });
}

int hcp_ring_block_partial(const hcp_ring_block_desc* desc, hcp_ring_view q, hcp_ring_view k,
                           hcp_ring_view v, float* o, float* lse, void* stream) {
  return guarded(__func__, [&] {
    check_block_desc(desc);
    check_view(q, "q", desc->q_len);
    check_view(k, "k", desc->kv_len);
    check_view(v, "v", desc->kv_len);
    if (desc->q_len > 0) require(o != nullptr && lse != nullptr, "null o or lse");
    const BlockLaunch L = make_launch(desc, q, k, v, o, lse);
    launch_block_partial(L, as_stream(stream));
    g_last_path = desc->q_len > 0 ? block_path(L) : HCP_PATH_NONE;
  });
}

size_t hcp_ring_block_partial_positioned_workspace_size(const hcp_ring_block_desc* desc) {
  if (desc == nullptr || desc->q_len < 0 || desc->kv_len < 0 || desc->num_kv_heads <= 0 || desc->head_dim <= 0)
    return 0;
  try {
    return positioned_workspace(desc).total;
  } catch (...) {
    return 0;  // unsupported dtype: the entry point itself reports it
  }
}

int hcp_ring_block_partial_positioned(const hcp_ring_block_desc* desc, hcp_ring_view q, const int64_t* q_positions,
                                      hcp_ring_view k, hcp_ring_view v, const int64_t* kv_positions, float* o,
                                      float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return guarded(__func__, [&] {
    check_block_desc(desc);
    check_view(q, "q", desc->q_len);
    check_view(k, "k", desc->kv_len);
    check_view(v, "v", desc->kv_len);
    if (desc->q_len == 0) return;
    require(o != nullptr && lse != nullptr, "null o or lse");
    BlockLaunch L = make_launch(desc, q, k, v, o, lse);
    if (desc->causal) {
      const PositionedWorkspace w = positioned_workspace(desc);
      require(q_positions != nullptr, "null q_positions");
      require(kv_positions != nullptr || desc->kv_len == 0, "null kv_positions");
      require(workspace != nullptr && workspace_bytes >= w.total,
              "workspace too small: need " + std::to_string(w.total) + " bytes");
      char* base = static_cast<char*>(workspace);
      const hipStream_t st = as_stream(stream);
      KeyLimitArgs la{};
      la.q_pos = q_positions;
      la.n_q = desc->q_len;
      la.k_pos = kv_positions;
      la.k_off[0] = 0;
      la.k_len[0] = desc->kv_len;
      la.lim = reinterpret_cast<int32_t*>(base + w.lim);
      la.lim_stride = 0;
      la.err = nullptr;  // keys in any order are handled below
      if (desc->kv_len > 0) {
        // A key list that is not non-decreasing is sorted with its rows, and K / V are
        // read through the sorted order (device-side decision: nothing happens for a
        // list already in order).  Attention over a set of keys does not depend on
        // their order (ring.rs:249-273 masks key by key).
        int* flag = reinterpret_cast<int*>(base + w.flag);
        int64_t* const keys[2] = {reinterpret_cast<int64_t*>(base + w.key[0]),
                                  reinterpret_cast<int64_t*>(base + w.key[1])};
        int32_t* const rows[2] = {reinterpret_cast<int32_t*>(base + w.row[0]),
                                  reinterpret_cast<int32_t*>(base + w.row[1])};
        launch_key_sort(kv_positions, desc->kv_len, flag, keys, rows, st);
        const int f = key_sort_passes(desc->kv_len) % 2;
        const int es = elem_size(desc->dtype);
        KvSortedGather g{};
        g.flag = flag;
        g.rows = rows[f];
        g.n = desc->kv_len;
        g.hkv = desc->num_kv_heads;
        g.row_bytes = static_cast<int64_t>(desc->head_dim) * es;
        g.k = static_cast<const char*>(k.data);
        g.v = static_cast<const char*>(v.data);
        g.k_hs_bytes = k.head_stride * es;
        g.k_ss_bytes = k.seq_stride * es;
        g.v_hs_bytes = v.head_stride * es;
        g.v_ss_bytes = v.seq_stride * es;
        g.kc = base + w.kc;
        g.vc = base + w.vc;
        launch_kv_sorted_gather(g, st);
        la.sel = flag;
        la.k_pos_sorted = keys[f];
        L.kv_sel = flag;
        L.k_alt = g.kc;
        L.v_alt = g.vc;
        L.alt_hs = desc->kv_len * desc->head_dim;
        L.alt_ss = desc->head_dim;
      }
      launch_key_limits(la, 1, desc->kv_len, st);
      L.q_lim = la.lim;
    }
    launch_block_partial(L, as_stream(stream));
    g_last_path = block_path(L);
  });
}

int hcp_ring_build_assignment(int32_t strategy, int32_t num_domains, const int64_t* chunk_lens,
                              int32_t* assignment) {
  return guarded(__func__, [&] {
    const StrategySpec sp = make_spec(strategy, num_domains, chunk_lens, true);
    require(assignment != nullptr, "null assignment");
    for (int d = 0; d < sp.n; ++d)
      for (int64_t i = 0; i < sp.chunks[d]; ++i) assignment[strategy_position(sp, d, i)] = d;
  });
}

int hcp_ring_domain_positions(int32_t strategy, int32_t num_domains, const int64_t* chunk_lens,
                              int64_t* positions) {
  return guarded(__func__, [&] {
    const StrategySpec sp = make_spec(strategy, num_domains, chunk_lens, true);
    require(positions != nullptr, "null positions");
    int64_t r = 0;
    for (int d = 0; d < sp.n; ++d)
      for (int64_t i = 0; i < sp.chunks[d]; ++i) positions[r++] = strategy_position(sp, d, i);
  });
}

int hcp_ring_inverse_perm(int32_t strategy, int32_t num_domains, const int64_t* chunk_lens, int64_t* inverse) {
  return guarded(__func__, [&] {
    const StrategySpec sp = make_spec(strategy, num_domains, chunk_lens, true);
    require(inverse != nullptr, "null inverse");
    int64_t r = 0;
    for (int d = 0; d < sp.n; ++d)
      for (int64_t i = 0; i < sp.chunks[d]; ++i) inverse[strategy_position(sp, d, i)] = r++;
  });
}

int hcp_ring_lse_merge(int32_t num_parts, const float* const* o_parts, const float* const* lse_parts,
                       int32_t num_heads, int64_t q_len, int32_t head_dim, int32_t out_dtype,
                       hcp_ring_view out, float* lse_out, void* stream) {
  return guarded(__func__, [&] {
    require(num_parts >= 1 && num_parts <= 64, "num_parts must be in [1, 64]");
    require(o_parts != nullptr && lse_parts != nullptr, "null partial arrays");
    for (int i = 0; i < num_parts; ++i)
      require(o_parts[i] != nullptr && lse_parts[i] != nullptr, "null partial pointer");
    require(num_heads > 0 && q_len >= 0, "bad shape");
    require(head_dim > 0 && head_dim <= 256 && head_dim % 4 == 0, "head_dim must be a multiple of 4 in [4, 256]");
    elem_size(out_dtype);
    check_view(out, "out", q_len);
    check_out_view(out, out_dtype);
    launch_lse_merge(num_parts, o_parts, lse_parts, num_heads, q_len, head_dim, out_dtype, out.data,
                     out.head_stride, out.seq_stride, lse_out, q_len, as_stream(stream));
  });
}

static void check_pool(const hcp_paged_pool* pool) {
  require(pool != nullptr && pool->data != nullptr, "null pool");
  require(pool->num_blocks > 0 && pool->block_size > 0 && pool->num_kv_heads > 0 && pool->head_dim > 0,
          "pool dimensions must be positive");
  require(pool->elem_bytes == 2 || pool->elem_bytes == 4, "elem_bytes must be 2 or 4");
}

static void check_paged_range(const hcp_paged_pool* pool, const int32_t* table, int64_t table_len,
                              int64_t off, int64_t t0, int64_t t1) {
  require(table != nullptr, "null block table");
  require(t0 >= off && t1 >= t0, "need table_seq_offset <= t0 <= t1");
  if (t1 > t0) require((t1 - 1 - off) / pool->block_size < table_len, "block table too short for [t0, t1)");
}

int hcp_paged_kv_gather(const hcp_paged_pool* pool, const int32_t* block_table, int64_t table_len,
                        int64_t table_seq_offset, int64_t t0, int64_t t1, hcp_ring_view k_out,
                        hcp_ring_view v_out, void* stream) {
  return guarded(__func__, [&] {
    check_pool(pool);
    check_paged_range(pool, block_table, table_len, table_seq_offset, t0, t1);
    check_view(k_out, "k_out", t1 - t0);
    check_view(v_out, "v_out", t1 - t0);
    require(k_out.head_stride == v_out.head_stride && k_out.seq_stride == v_out.seq_stride,
            "k_out and v_out must share strides");
    launch_paged_copy(true, pool->data, pool->num_blocks, pool->block_size, pool->num_kv_heads, pool->head_dim,
                      pool->elem_bytes, block_table, table_seq_offset, t0, t1, k_out.data, v_out.data,
                      k_out.head_stride, k_out.seq_stride, 0, device_error_flags(), as_stream(stream));
  });
}

int hcp_paged_kv_scatter(const hcp_paged_pool* pool, const int32_t* block_table, int64_t table_len,
                         int64_t table_seq_offset, int64_t t0, int64_t t1, hcp_ring_view k_in,
                         hcp_ring_view v_in, int32_t zero_tail, void* stream) {
  return guarded(__func__, [&] {
    check_pool(pool);
    check_paged_range(pool, block_table, table_len, table_seq_offset, t0, t1);
    check_view(k_in, "k_in", t1 - t0);
    check_view(v_in, "v_in", t1 - t0);
    require(k_in.head_stride == v_in.head_stride && k_in.seq_stride == v_in.seq_stride,
            "k_in and v_in must share strides");
    launch_paged_copy(false, pool->data, pool->num_blocks, pool->block_size, pool->num_kv_heads, pool->head_dim,
                      pool->elem_bytes, block_table, table_seq_offset, t0, t1, k_in.data, v_in.data,
                      k_in.head_stride, k_in.seq_stride, zero_tail ? 1 : 0, device_error_flags(),
                      as_stream(stream));
  });
}

int hcp_paged_kv_gather_batch(const hcp_paged_pool* pool, int32_t num_ranges, const hcp_paged_range* ranges,
                              void* stream) {
  return guarded(__func__, [&] {
    check_pool(pool);
    require(num_ranges >= 0 && (num_ranges == 0 || ranges != nullptr), "bad range array");
    std::vector<PagedRangeDesc> rs;
    rs.reserve(num_ranges);
    for (int i = 0; i < num_ranges; ++i) {
      const hcp_paged_range& r = ranges[i];
      check_paged_range(pool, r.block_table, r.table_len, r.table_seq_offset, r.t0, r.t1);
      check_view(r.k_out, "k_out", r.t1 - r.t0);
      check_view(r.v_out, "v_out", r.t1 - r.t0);
      require(r.k_out.head_stride == r.v_out.head_stride && r.k_out.seq_stride == r.v_out.seq_stride,
              "k_out and v_out must share strides");
      rs.push_back(PagedRangeDesc{r.block_table, r.table_seq_offset, r.t0, r.t1, r.k_out.data, r.v_out.data,
                                  r.k_out.head_stride, r.k_out.seq_stride});
    }
    launch_paged_copy_batch(true, pool->data, pool->num_blocks, pool->block_size, pool->num_kv_heads,
                            pool->head_dim, pool->elem_bytes, num_ranges, rs.data(), 0, device_error_flags(),
                            as_stream(stream));
  });
}

size_t hcp_paged_decode_workspace_size(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool) {
  if (desc == nullptr || pool == nullptr || desc->batch <= 0) return 0;
  (void)pool;
  return decode_workspace_bytes(desc->dtype, desc->batch, desc->num_q_heads, desc->num_kv_heads, desc->head_dim, desc->t0, desc->t1);
}

int hcp_paged_decode_partial(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool, hcp_ring_view q,
                             const int32_t* block_tables, const int32_t* seq_lens, float* o, float* lse,
                             void* workspace, size_t workspace_bytes, void* stream) {
  return guarded(__func__, [&] {
    require(desc != nullptr, "null descriptor");
    check_pool(pool);
    require(desc->batch > 0, "batch must be positive");
    require(desc->num_q_heads > 0 && desc->num_kv_heads == pool->num_kv_heads, "kv heads must match the pool");
    require(desc->head_dim == pool->head_dim, "head_dim must match the pool");
    require(pool->elem_bytes == 2, "paged decode needs a 16-bit pool");
    require(desc->t0 >= 0 && desc->t1 >= desc->t0, "need 0 <= t0 <= t1");
    require(block_tables != nullptr && o != nullptr && lse != nullptr, "null pointer");
    require(desc->table_len >= 1 && desc->table_stride >= desc->table_len, "bad table shape");
    if (desc->t1 > desc->t0) require((desc->t1 - 1) / pool->block_size < desc->table_len, "block table too short");
    require(desc->scale > 0.f, "scale must be positive");
    check_view(q, "q", 1);
    require(mfma_layout_ok(q), "q must be 16-byte aligned with strides multiple of 8");
    launch_paged_decode(desc->dtype, desc->batch, desc->num_q_heads, desc->num_kv_heads, desc->head_dim, q.data,
                        q.seq_stride, q.head_stride, pool->data, pool->num_blocks, pool->block_size, block_tables,
                        desc->table_stride, desc->table_len, seq_lens, desc->t0, desc->t1, desc->scale, o, lse,
                        workspace, workspace_bytes, device_error_flags(), as_stream(stream));
  });
}

int hcp_paged_decode_partial_static(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool,
                                    hcp_ring_view q, const int32_t* block_tables, const int32_t* seq_lens, float* o,
                                    float* lse, void* stream) {
  return guarded(__func__, [&] {
    require(desc != nullptr && pool != nullptr, "null descriptor or pool");
    require(desc->batch > 0, "batch must be positive");
    const size_t need = decode_workspace_bytes(desc->dtype, desc->batch, desc->num_q_heads, desc->num_kv_heads,
                                               desc->head_dim, desc->t0, desc->t1);
    require(need <= kStaticScratchBytes, "the split partials need " + std::to_string(need) +
                                             " bytes, more than the static scratch's " +
                                             std::to_string(kStaticScratchBytes) +
                                             "; use hcp_paged_decode_partial with a workspace");
    void* ws = static_scratch();
    const int rc = hcp_paged_decode_partial(desc, pool, q, block_tables, seq_lens, o, lse, ws, kStaticScratchBytes,
                                            stream);
    if (rc != 0) throw Error(rc, g_last_error);
  });
}

// ---- decode Q-ring replay ----
}  // extern "C": internal helpers below have C++ linkage
namespace {
struct DecodeRingPlan {
  size_t part_o = 0, part_lse = 0, part_bytes = 0, dec_off = 0, total = 0;
};
DecodeRingPlan plan_decode_ring(const hcp_paged_decode_desc* desc, int n, const hcp_decode_shard* shards) {
  require(desc != nullptr && shards != nullptr, "null descriptor or shards");
  require(n >= 1 && n <= 64, "num_domains must be in [1, 64]");
  require(desc->batch > 0 && desc->num_q_heads > 0 && desc->head_dim > 0, "bad decode shape");
  DecodeRingPlan p;
  const size_t rows = static_cast<size_t>(desc->batch) * desc->num_q_heads;
  p.part_o = align256(rows * desc->head_dim * sizeof(float));
  p.part_lse = align256(rows * sizeof(float));
  p.part_bytes = p.part_o + p.part_lse;
  p.dec_off = p.part_bytes * n;
  size_t dec = 0;
  for (int i = 0; i < n; ++i) {
    require(shards[i].max_len >= 0, "shard max_len must be >= 0");
    dec = std::max(dec, decode_workspace_bytes(desc->dtype, desc->batch, desc->num_q_heads, desc->num_kv_heads,
                                               desc->head_dim, 0, shards[i].max_len));
  }
  p.total = p.dec_off + align256(dec);
  return p;
}
}  // namespace
extern "C" {

int hcp_decode_ring_owner(int64_t global_pos, int32_t num_domains) {
  if (num_domains <= 0 || global_pos < 0) return HCP_RING_E_INVALID;
  return static_cast<int>(global_pos % num_domains);
}

size_t hcp_decode_ring_workspace_size(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool,
                                      int32_t num_domains, const hcp_decode_shard* shards) {
  (void)pool;
  try {
    return plan_decode_ring(desc, num_domains, shards).total;
  } catch (...) {
    return 0;
  }
}

int hcp_decode_ring_replay(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool, hcp_ring_view q,
                           int32_t num_domains, const hcp_decode_shard* shards, int32_t seed_domain,
                           hcp_ring_view out, float* lse_out, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return guarded(__func__, [&] {
    const DecodeRingPlan plan = plan_decode_ring(desc, num_domains, shards);
    check_pool(pool);
    require(seed_domain >= 0 && seed_domain < num_domains, "seed_domain out of range");
    require(desc->num_kv_heads == pool->num_kv_heads && desc->head_dim == pool->head_dim,
            "descriptor does not match the pool");
    require(pool->elem_bytes == 2, "paged decode needs a 16-bit pool");
    require(desc->scale > 0.f, "scale must be positive");
    require(workspace != nullptr && workspace_bytes >= plan.total,
            "workspace too small: need " + std::to_string(plan.total) + " bytes");
    check_view(q, "q", 1);
    require(mfma_layout_ok(q), "q must be 16-byte aligned with strides multiple of 8");
    check_view(out, "out", 1);
    check_out_view(out, desc->dtype);
    require(out.seq_stride == static_cast<int64_t>(desc->num_q_heads) * out.head_stride,
            "out must hold the [batch, Hq] rows at one stride (seq_stride == Hq * head_stride)");
    char* base = static_cast<char*>(workspace);
    std::vector<const float*> os, ls;
    for (int j = 0; j < num_domains; ++j) {
      // Journey order: the seed domain's partial first, then its successors.
      const int dom = (seed_domain + j) % num_domains;
      const hcp_decode_shard& sh = shards[dom];
      float* po = reinterpret_cast<float*>(base + static_cast<size_t>(j) * plan.part_bytes);
      float* pl = reinterpret_cast<float*>(base + static_cast<size_t>(j) * plan.part_bytes + plan.part_o);
      if (sh.max_len > 0) {
        require(sh.block_tables != nullptr, "null block table of a non-empty shard");
        require(sh.table_len >= 1 && sh.table_stride >= sh.table_len, "bad shard table shape");
        require((sh.max_len - 1) / pool->block_size < sh.table_len, "shard block table too short");
      }
      launch_paged_decode(desc->dtype, desc->batch, desc->num_q_heads, desc->num_kv_heads, desc->head_dim, q.data,
                          q.seq_stride, q.head_stride, pool->data, pool->num_blocks, pool->block_size,
                          sh.block_tables, sh.table_stride, std::max<int64_t>(sh.table_len, 1), sh.seq_lens, 0,
                          sh.max_len, desc->scale, po, pl, base + plan.dec_off, workspace_bytes - plan.dec_off,
                          device_error_flags(), as_stream(stream));
      os.push_back(po);
      ls.push_back(pl);
    }
    launch_lse_merge(num_domains, os.data(), ls.data(), desc->batch * desc->num_q_heads, 1, desc->head_dim,
                     desc->dtype, out.data, out.head_stride, out.head_stride, lse_out, 1, as_stream(stream));
  });
}

}  // extern "C": internal helpers below have C++ linkage
namespace {

void check_kv_frame(const hcp_kv_frame_desc* d) {
  require(d != nullptr, "null descriptor");
  elem_size(d->dtype);
  require(d->num_heads > 0 && d->num_kv_heads > 0 && d->num_heads % d->num_kv_heads == 0,
          "num_heads must be a positive multiple of num_kv_heads");
  require(d->head_dim > 0, "head_dim must be positive");
  require(d->len >= 0 && d->layer_idx >= 0 && d->global_seq_start >= 0 && d->global_seq_end >= 0,
          "negative layer index, range or length");
  require(d->has_positions == 0 || d->has_positions == 1, "has_positions must be 0 or 1");
}

size_t kv_plane_bytes(const hcp_kv_frame_desc* d) {
  return static_cast<size_t>(d->num_heads) * d->len * d->head_dim * 4;
}

void check_packet_frame(const hcp_packet_frame_desc* d) {
  require(d != nullptr, "null descriptor");
  elem_size(d->q_dtype);
  elem_size(d->o_dtype);
  require(d->batch > 0 && d->num_heads > 0 && d->head_dim > 0, "bad packet shape");
  require(d->layer_idx >= 0, "negative layer index");
}

void write_header(const std::string& meta, void* out, size_t cap, size_t* written) {
  require(written != nullptr, "null written");
  const size_t n = 4 + meta.size();
  *written = n;
  require(out != nullptr && cap >= n, "header buffer too small: need " + std::to_string(n) + " bytes");
  unsigned char* o = static_cast<unsigned char*>(out);
  const uint32_t m = static_cast<uint32_t>(meta.size());
  o[0] = static_cast<unsigned char>(m >> 24);
  o[1] = static_cast<unsigned char>(m >> 16);
  o[2] = static_cast<unsigned char>(m >> 8);
  o[3] = static_cast<unsigned char>(m);
  std::memcpy(o + 4, meta.data(), meta.size());
}

const JVal& field(const JVal& o, const char* key) {
  auto it = o.obj.find(key);
  require(it != o.obj.end(), std::string("header: missing ") + key);
  return it->second;
}

int64_t field_int(const JVal& o, const char* key) {
  const JVal& v = field(o, key);
  require(v.kind == JVal::kNum && v.integral, std::string("header: ") + key + " is not an integer");
  return v.inum;
}

std::vector<int64_t> field_shape(const JVal& o, const char* key) {
  const JVal& v = field(o, key);
  require(v.kind == JVal::kArr, std::string("header: ") + key + " is not an array");
  std::vector<int64_t> s;
  for (const JVal& x : v.arr) {
    require(x.kind == JVal::kNum && x.integral, std::string("header: bad ") + key);
    s.push_back(x.inum);
  }
  return s;
}

int field_dtype(const JVal& o, const char* key) {
  auto it = o.obj.find(key);
  if (it == o.obj.end() || it->second.kind != JVal::kStr) return kF32;  // tcp.rs:701-704
  return dtype_from_wire_name(it->second.str);
}

}  // namespace
extern "C" {

size_t hcp_kv_frame_payload_bytes(const hcp_kv_frame_desc* desc) {
  try {
    check_kv_frame(desc);
    return 2 * kv_plane_bytes(desc) + (desc->has_positions ? static_cast<size_t>(desc->len) * 8 : 0);
  } catch (...) {
    return 0;
  }
}

int hcp_kv_frame_header(const hcp_kv_frame_desc* desc, void* out, size_t capacity, size_t* written) {
  return guarded(__func__, [&] {
    check_kv_frame(desc);
    write_header(kv_frame_meta(desc->layer_idx, desc->global_seq_start, desc->global_seq_end, desc->dtype,
                               desc->num_heads, desc->len, desc->head_dim, desc->has_positions != 0),
                 out, capacity, written);
  });
}

int hcp_kv_frame_parse(const void* frame, size_t frame_bytes, hcp_kv_frame_desc* desc, size_t* header_bytes) {
  return guarded(__func__, [&] {
    require(desc != nullptr && header_bytes != nullptr, "null output");
    const JVal m = parse_frame_meta(static_cast<const unsigned char*>(frame), frame_bytes, header_bytes);
    auto t = m.obj.find("type");
    require(t == m.obj.end() || t->second.kind != JVal::kStr, "header: not a KV block frame");
    const std::vector<int64_t> ks = field_shape(m, "k_shape"), vs = field_shape(m, "v_shape");
    require(ks.size() == 4 && ks[0] == 1 && ks == vs, "header: k/v shapes must be equal [1, H, L, D]");
    hcp_kv_frame_desc d{};
    d.layer_idx = field_int(m, "layer_idx");
    d.global_seq_start = field_int(m, "global_seq_start");
    d.global_seq_end = field_int(m, "global_seq_end");
    d.dtype = field_dtype(m, "k_dtype");
    require(field_dtype(m, "v_dtype") == d.dtype, "header: k and v dtypes differ");
    require(ks[1] > 0 && ks[1] <= INT32_MAX && ks[3] > 0 && ks[3] <= INT32_MAX && ks[2] >= 0, "header: bad shape");
    d.num_heads = d.num_kv_heads = static_cast<int32_t>(ks[1]);
    d.len = ks[2];
    d.head_dim = static_cast<int32_t>(ks[3]);
    require(field_int(m, "k_bytes") == static_cast<int64_t>(kv_plane_bytes(&d)) &&
                field_int(m, "v_bytes") == static_cast<int64_t>(kv_plane_bytes(&d)),
            "header: k_bytes / v_bytes do not match the fp32 shape");
    auto p = m.obj.find("position_ids");
    if (p != m.obj.end() && p->second.kind != JVal::kNull) {
      require(p->second.kind == JVal::kObj, "header: bad position_ids");
      require(field(p->second, "dtype").str == "int64", "header: position_ids must be int64");
      const std::vector<int64_t> ps = field_shape(p->second, "shape");
      require(ps.size() == 1 && ps[0] == d.len && field_int(p->second, "bytes") == d.len * 8,
              "header: position_ids shape does not match the block");
      d.has_positions = 1;
    }
    check_kv_frame(&d);
    *desc = d;
  });
}

int hcp_kv_frame_pack(const hcp_kv_frame_desc* desc, hcp_ring_view k, hcp_ring_view v, const int64_t* positions,
                      void* payload, void* stream) {
  return guarded(__func__, [&] {
    check_kv_frame(desc);
    check_view(k, "k", desc->len);
    check_view(v, "v", desc->len);
    require(payload != nullptr, "null payload");
    require(!desc->has_positions || positions != nullptr || desc->len == 0, "null positions");
    const int64_t rep = desc->num_heads / desc->num_kv_heads;
    float* wire = static_cast<float*>(payload);
    const size_t plane = kv_plane_bytes(desc);
    launch_wire_segment(true, desc->dtype, k.data, wire, desc->num_heads, rep, desc->len, desc->head_dim,
                        k.head_stride, k.seq_stride, as_stream(stream));
    launch_wire_segment(true, desc->dtype, v.data, wire + plane / 4, desc->num_heads, rep, desc->len,
                        desc->head_dim, v.head_stride, v.seq_stride, as_stream(stream));
    if (desc->has_positions && desc->len > 0)
      HCP_HIP(hipMemcpyAsync(static_cast<char*>(payload) + 2 * plane, positions, desc->len * 8,
                             hipMemcpyDeviceToDevice, as_stream(stream)));
  });
}

int hcp_kv_frame_unpack(const hcp_kv_frame_desc* desc, const void* payload, hcp_ring_view k, hcp_ring_view v,
                        int64_t* positions, void* stream) {
  return guarded(__func__, [&] {
    check_kv_frame(desc);
    check_view(k, "k", desc->len);
    check_view(v, "v", desc->len);
    require(payload != nullptr, "null payload");
    const int64_t rep = desc->num_heads / desc->num_kv_heads;
    float* wire = const_cast<float*>(static_cast<const float*>(payload));
    const size_t plane = kv_plane_bytes(desc);
    launch_wire_segment(false, desc->dtype, k.data, wire, desc->num_heads, rep, desc->len, desc->head_dim,
                        k.head_stride, k.seq_stride, as_stream(stream));
    launch_wire_segment(false, desc->dtype, v.data, wire + plane / 4, desc->num_heads, rep, desc->len,
                        desc->head_dim, v.head_stride, v.seq_stride, as_stream(stream));
    if (desc->has_positions && positions != nullptr && desc->len > 0)
      HCP_HIP(hipMemcpyAsync(positions, static_cast<const char*>(payload) + 2 * plane, desc->len * 8,
                             hipMemcpyDeviceToDevice, as_stream(stream)));
  });
}

size_t hcp_packet_frame_payload_bytes(const hcp_packet_frame_desc* desc) {
  try {
    check_packet_frame(desc);
    const size_t rows = static_cast<size_t>(desc->batch) * desc->num_heads;
    return rows * desc->head_dim * 4 * 2 + rows * 4;
  } catch (...) {
    return 0;
  }
}

int hcp_packet_frame_header(const hcp_packet_frame_desc* desc, void* out, size_t capacity, size_t* written) {
  return guarded(__func__, [&] {
    check_packet_frame(desc);
    write_header(packet_frame_meta(desc->layer_idx, desc->q_dtype, desc->o_dtype, desc->batch, desc->num_heads,
                                   desc->head_dim, desc->scale),
                 out, capacity, written);
  });
}

int hcp_packet_frame_parse(const void* frame, size_t frame_bytes, hcp_packet_frame_desc* desc,
                           size_t* header_bytes) {
  return guarded(__func__, [&] {
    require(desc != nullptr && header_bytes != nullptr, "null output");
    const JVal m = parse_frame_meta(static_cast<const unsigned char*>(frame), frame_bytes, header_bytes);
    const JVal& t = field(m, "type");
    require(t.kind == JVal::kStr && t.str == "ring_packet", "header: not a ring_packet frame");
    const std::vector<int64_t> qs = field_shape(m, "q_shape"), os = field_shape(m, "o_shape"),
                               ls = field_shape(m, "lse_shape");
    require(qs.size() == 4 && qs[2] == 1 && qs == os, "header: q/o shapes must be equal [B, H, 1, D]");
    require(ls.size() == 3 && ls[0] == qs[0] && ls[1] == qs[1] && ls[2] == 1, "header: lse shape must be [B, H, 1]");
    require(qs[0] > 0 && qs[0] <= INT32_MAX && qs[1] > 0 && qs[1] <= INT32_MAX && qs[3] > 0 && qs[3] <= INT32_MAX,
            "header: bad shape");
    hcp_packet_frame_desc d{};
    d.layer_idx = field_int(m, "layer_idx");
    d.q_dtype = field_dtype(m, "q_dtype");
    d.o_dtype = field_dtype(m, "o_dtype");
    d.batch = static_cast<int32_t>(qs[0]);
    d.num_heads = static_cast<int32_t>(qs[1]);
    d.head_dim = static_cast<int32_t>(qs[3]);
    const JVal& sc = field(m, "scale");
    require(sc.kind == JVal::kNum, "header: scale is not a number");
    d.scale = sc.num;
    const int64_t qb = static_cast<int64_t>(d.batch) * d.num_heads * d.head_dim * 4;
    require(field_int(m, "q_bytes") == qb && field_int(m, "o_bytes") == qb &&
                field_int(m, "lse_bytes") == static_cast<int64_t>(d.batch) * d.num_heads * 4,
            "header: byte counts do not match the fp32 shapes");
    check_packet_frame(&d);
    *desc = d;
  });
}

int hcp_packet_frame_pack(const hcp_packet_frame_desc* desc, hcp_ring_view q, const float* o, const float* lse,
                          void* payload, void* stream) {
  return guarded(__func__, [&] {
    check_packet_frame(desc);
    check_view(q, "q", 1);
    require(o != nullptr && lse != nullptr && payload != nullptr, "null o, lse or payload");
    const int64_t rows = static_cast<int64_t>(desc->batch) * desc->num_heads;
    float* wire = static_cast<float*>(payload);
    // q: wire row b = batch b, its [num_heads, head_dim] at (seq_stride, head_stride).
    launch_wire_segment(true, desc->q_dtype, q.data, wire, desc->batch, 1, desc->num_heads, desc->head_dim,
                        q.seq_stride, q.head_stride, as_stream(stream));
    launch_wire_segment(true, kF32, const_cast<float*>(o), wire + rows * desc->head_dim, rows, 1, 1,
                        desc->head_dim, desc->head_dim, desc->head_dim, as_stream(stream));
    launch_wire_segment(true, kF32, const_cast<float*>(lse), wire + 2 * rows * desc->head_dim, rows, 1, 1, 1, 1, 1,
                        as_stream(stream));
  });
}

int hcp_packet_frame_unpack(const hcp_packet_frame_desc* desc, const void* payload, hcp_ring_view q, float* o,
                            float* lse, void* stream) {
  return guarded(__func__, [&] {
    check_packet_frame(desc);
    check_view(q, "q", 1);
    require(o != nullptr && lse != nullptr && payload != nullptr, "null o, lse or payload");
    const int64_t rows = static_cast<int64_t>(desc->batch) * desc->num_heads;
    float* wire = const_cast<float*>(static_cast<const float*>(payload));
    launch_wire_segment(false, desc->q_dtype, q.data, wire, desc->batch, 1, desc->num_heads, desc->head_dim,
                        q.seq_stride, q.head_stride, as_stream(stream));
    launch_wire_segment(false, kF32, o, wire + rows * desc->head_dim, rows, 1, 1, desc->head_dim, desc->head_dim,
                        desc->head_dim, as_stream(stream));
    launch_wire_segment(false, kF32, lse, wire + 2 * rows * desc->head_dim, rows, 1, 1, 1, 1, 1,
                        as_stream(stream));
  });
}

}  // extern "C": internal helpers below have C++ linkage
namespace {

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

QkvArgs make_qkv(const hcp_qkv_desc* d, const void* x, int64_t x_ss, const void* wq, const void* wk, const void* wv,
                 const void* bq, const void* bk, const void* bv, const int64_t* positions, const float* table,
                 hcp_ring_view q_out) {
  require(d != nullptr, "null descriptor");
  require(d->dtype == kBF16 || d->dtype == kF16, "dtype must be BF16 or F16");
  require(d->head_dim == 64 || d->head_dim == 128, "head_dim must be 64 or 128");
  require(d->hidden > 0 && d->hidden % 32 == 0, "hidden must be a positive multiple of 32");
  require(d->num_q_heads > 0 && d->num_kv_heads > 0, "head counts must be positive");
  require((static_cast<int64_t>(d->num_q_heads) * d->head_dim) % 128 == 0 &&
              (static_cast<int64_t>(d->num_kv_heads) * d->head_dim) % 128 == 0,
          "Hq*D and Hkv*D must be multiples of 128");
  require(static_cast<int64_t>(d->num_q_heads + 2 * d->num_kv_heads) * d->head_dim <= INT32_MAX,
          "too many output features");
  require(d->tokens >= 0 && d->tokens <= INT32_MAX, "tokens must be in [0, 2^31)");
  require(d->rope == 0 || d->rope == 1, "rope must be 0 or 1");
  require(x != nullptr || d->tokens == 0, "null x");
  require(aligned(x, 16) && x_ss % 8 == 0 && x_ss >= d->hidden, "x must be 16-byte aligned, row stride a multiple of 8 >= hidden");
  require(wq && wk && wv && aligned(wq, 16) && aligned(wk, 16) && aligned(wv, 16), "weights must be non-null and 16-byte aligned");
  if (d->rope) require(positions != nullptr && table != nullptr && d->rope_rows > 0, "rope needs positions and a table");
  require(q_out.data != nullptr && aligned(q_out.data, 8) && q_out.head_stride % 4 == 0 && q_out.seq_stride % 4 == 0,
          "q_out must be 8-byte aligned with strides multiple of 4");
  QkvArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_ss = x_ss;
  a.w[0] = static_cast<const uint16_t*>(wq);
  a.w[1] = static_cast<const uint16_t*>(wk);
  a.w[2] = static_cast<const uint16_t*>(wv);
  a.bias[0] = static_cast<const uint16_t*>(bq);
  a.bias[1] = static_cast<const uint16_t*>(bk);
  a.bias[2] = static_cast<const uint16_t*>(bv);
  a.nq = d->num_q_heads * d->head_dim;
  a.nkv = d->num_kv_heads * d->head_dim;
  a.hidden = d->hidden;
  a.tokens = static_cast<int32_t>(d->tokens);
  a.rope = d->rope;
  a.pos = positions;
  a.rope_cos = table;
  a.rope_sin = table ? table + d->rope_rows * (d->head_dim / 2) : nullptr;
  a.rope_rows = d->rope_rows;
  a.out[0] = static_cast<uint16_t*>(q_out.data);
  a.out_hs[0] = q_out.head_stride;
  a.out_ss[0] = q_out.seq_stride;
  a.err = device_error_flags();
  return a;
}

void check_qkv_out(const hcp_ring_view& v, const char* name) {
  require(v.data != nullptr && aligned(v.data, 8) && v.head_stride % 4 == 0 && v.seq_stride % 4 == 0,
          std::string(name) + " must be 8-byte aligned with strides multiple of 4");
}

}  // namespace
extern "C" {

int hcp_rope_table(int32_t head_dim, int64_t rows, double base, float* table, void* stream) {
  return guarded(__func__, [&] {
    require(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 256, "head_dim must be even and <= 256");
    require(rows >= 0 && rows <= (int64_t(1) << 24), "rows must be in [0, 2^24] (fp32-exact positions)");
    require(base > 0, "base must be positive");
    require(table != nullptr || rows == 0, "null table");
    launch_rope_table(head_dim, rows, base, table, table + rows * (head_dim / 2), as_stream(stream));
  });
}

int hcp_qkv_rope_project(const hcp_qkv_desc* desc, const void* x, int64_t x_row_stride, const void* wq,
                         const void* wk, const void* wv, const void* bq, const void* bk, const void* bv,
                         const int64_t* positions, const float* rope_table, hcp_ring_view q_out, hcp_ring_view k_out,
                         hcp_ring_view v_out, void* stream) {
  return guarded(__func__, [&] {
    QkvArgs a = make_qkv(desc, x, x_row_stride, wq, wk, wv, bq, bk, bv, positions, rope_table, q_out);
    check_qkv_out(k_out, "k_out");
    check_qkv_out(v_out, "v_out");
    a.out[1] = static_cast<uint16_t*>(k_out.data);
    a.out_hs[1] = k_out.head_stride;
    a.out_ss[1] = k_out.seq_stride;
    a.out[2] = static_cast<uint16_t*>(v_out.data);
    a.out_hs[2] = v_out.head_stride;
    a.out_ss[2] = v_out.seq_stride;
    launch_qkv_rope(desc->dtype, desc->head_dim, a, as_stream(stream));
  });
}

int hcp_qkv_rope_project_paged(const hcp_qkv_desc* desc, const void* x, int64_t x_row_stride, const void* wq,
                               const void* wk, const void* wv, const void* bq, const void* bk, const void* bv,
                               const int64_t* positions, const float* rope_table, hcp_ring_view q_out,
                               const hcp_paged_pool* pool, const int32_t* block_table, int64_t table_len,
                               int64_t table_seq_offset, int64_t t0, void* stream) {
  return guarded(__func__, [&] {
    QkvArgs a = make_qkv(desc, x, x_row_stride, wq, wk, wv, bq, bk, bv, positions, rope_table, q_out);
    check_pool(pool);
    require(pool->elem_bytes == 2 && pool->num_kv_heads == desc->num_kv_heads && pool->head_dim == desc->head_dim,
            "pool does not match the descriptor");
    require(aligned(pool->data, 8), "pool must be 8-byte aligned");
    require(block_table != nullptr && table_len >= 1, "null or empty block table");
    require(t0 >= table_seq_offset, "t0 must be >= table_seq_offset");
    a.pool = static_cast<uint16_t*>(pool->data);
    a.plane_elems = pool->num_blocks * pool->block_size * static_cast<int64_t>(pool->num_kv_heads) * pool->head_dim;
    a.num_blocks = pool->num_blocks;
    a.bs = pool->block_size;
    a.hkv = pool->num_kv_heads;
    a.table = block_table;
    a.table_len = table_len;
    a.table_off = table_seq_offset;
    a.t0 = t0;
    launch_qkv_rope(desc->dtype, desc->head_dim, a, as_stream(stream));
  });
}

}  // extern "C": internal helpers below have C++ linkage
namespace {

int status_code(const hcp_ringattn::Status& st, const char* fn) {
  using C = hcp_ringattn::Status::Code;
  if (st.ok()) return HCP_RING_OK;
  const int code = st.code() == C::kInvalidArgument ? -6 : (st.code() == C::kUnimplemented ? -5 : -2);
  return fail(code, std::string(fn) + ": " + st.message());
}

hcp_ringattn::TensorDType runtime_dtype(int32_t d) {
  switch (d) {
    case kF16: return hcp_ringattn::TensorDType::kFloat16;
    case kBF16: return hcp_ringattn::TensorDType::kBFloat16;
    case kF32: return hcp_ringattn::TensorDType::kFloat32;
    default: return hcp_ringattn::TensorDType::kUnknown;
  }
}

hcp_ringattn::BoundaryTensor host_f32(const char* name, std::vector<int64_t> shape, const float* data, size_t n) {
  hcp_ringattn::BoundaryTensor t;
  t.name = name;
  t.dtype = hcp_ringattn::TensorDType::kFloat32;
  t.shape = std::move(shape);
  t.payload.resize(n * 4);
  std::memcpy(t.payload.data(), data, n * 4);
  return t;
}

}  // namespace
extern "C" {

struct hcp_ringattn_runtime {
  std::unique_ptr<hcp_ringattn::RingAttnRuntime> impl;
  int64_t num_heads = 0, head_dim = 0, len = 0;
};

int hcp_ringattn_runtime_create(const char* device_type, hcp_ringattn_runtime** out) {
  return guarded(__func__, [&] {
    require(device_type != nullptr && out != nullptr, "null argument");
    auto* rt = new hcp_ringattn_runtime;
    rt->impl = hcp_ringattn::CreateRingAttnRuntime(device_type);
    *out = rt;
  });
}

void hcp_ringattn_runtime_destroy(hcp_ringattn_runtime* rt) { delete rt; }

int hcp_ringattn_runtime_init(hcp_ringattn_runtime* rt, int32_t domain_index, int32_t num_domains,
                              const char* const* domain_ids, const int64_t* seq_chunk_lens,
                              const int64_t* block_sizes, const char* device, int64_t global_seq_len,
                              int64_t num_heads, int64_t head_dim, int32_t dtype) {
  g_last_error.clear();
  if (rt == nullptr || domain_ids == nullptr || seq_chunk_lens == nullptr || block_sizes == nullptr ||
      device == nullptr || num_domains <= 0 || domain_index < 0 || domain_index >= num_domains)
    return fail(-6, std::string(__func__) + ": null argument or domain_index out of range");
  hcp_ringattn::RingAttnConfig g;
  g.global_seq_len = global_seq_len;
  g.num_heads = num_heads;
  g.head_dim = head_dim;
  g.dtype = runtime_dtype(dtype);
  for (int i = 0; i < num_domains; ++i) {
    if (domain_ids[i] == nullptr) return fail(-6, std::string(__func__) + ": null domain id");
    g.domains.push_back({domain_ids[i], "", 0, seq_chunk_lens[i], block_sizes[i], device});
  }
  const int rc = status_code(rt->impl->Init(g.domains[domain_index], g), __func__);
  if (rc == 0) {
    rt->num_heads = num_heads;
    rt->head_dim = head_dim;
    rt->len = seq_chunk_lens[domain_index];
  }
  return rc;
}

int hcp_ringattn_runtime_bind_layer(hcp_ringattn_runtime* rt, int32_t layer_index, int32_t num_kv_heads,
                                    hcp_ring_view q, hcp_ring_view k, hcp_ring_view v, float scale, void* stream) {
  g_last_error.clear();
  if (rt == nullptr) return fail(-6, std::string(__func__) + ": null runtime");
  auto* hip = dynamic_cast<hcp_ringattn::HipRingAttnRuntime*>(rt->impl.get());
  if (hip == nullptr) return fail(-5, std::string(__func__) + ": runtime cannot bind device inputs");
  return status_code(hip->BindLayer(layer_index, num_kv_heads, q, k, v, scale, stream), __func__);
}

int hcp_ringattn_runtime_run_layer(hcp_ringattn_runtime* rt, int32_t layer_index, int64_t in_seq_len,
                                   const float* in_max, const float* in_sum, const float* in_output,
                                   float* out_max, float* out_sum, float* out_output) {
  g_last_error.clear();
  if (rt == nullptr || out_max == nullptr || out_sum == nullptr || out_output == nullptr)
    return fail(-6, std::string(__func__) + ": null runtime or output array");
  const int64_t h = rt->num_heads, d = rt->head_dim, l = rt->len;
  const size_t rows = static_cast<size_t>(h) * l;
  hcp_ringattn::RingAttnSoftmaxState in, out;
  if (in_seq_len > 0) {
    if (in_seq_len != l || in_max == nullptr || in_sum == nullptr || in_output == nullptr)
      return fail(-6, std::string(__func__) + ": initial state must cover the domain's chunk");
    in.seq_len = l;
    in.num_heads = h;
    in.head_dim = d;
    in.running_max = host_f32("running_max", {h, l}, in_max, rows);
    in.running_sum = host_f32("running_sum", {h, l}, in_sum, rows);
    in.output = host_f32("output", {h, l, d}, in_output, rows * d);
  }
  const int rc = status_code(rt->impl->RunRingAttentionLayer(layer_index, in, &out), __func__);
  if (rc != 0) return rc;
  if (out.seq_len == 0) {  // nothing bound and no initial state: an empty state
    for (size_t i = 0; i < rows; ++i) out_max[i] = -INFINITY, out_sum[i] = 0.f;
    std::memset(out_output, 0, rows * d * 4);
    return 0;
  }
  std::memcpy(out_max, out.running_max.payload.data(), rows * 4);
  std::memcpy(out_sum, out.running_sum.payload.data(), rows * 4);
  std::memcpy(out_output, out.output.payload.data(), rows * d * 4);
  return 0;
}

int hcp_ringattn_runtime_shutdown(hcp_ringattn_runtime* rt) {
  g_last_error.clear();
  if (rt == nullptr) return fail(-6, std::string(__func__) + ": null runtime");
  return status_code(rt->impl->Shutdown(), __func__);
}

int hcp_ringattn_cxx_smoke_domain_count(void) {
  try {
    hcp_ringattn::RingAttnConfig g;
    g.global_seq_len = 1024;
    g.num_heads = 8;
    g.head_dim = 64;
    g.domains = {{"domain-0", "127.0.0.1", 26001, 512, 128, "hip"},
                 {"domain-1", "127.0.0.1", 26002, 256, 64, "hip"},
                 {"domain-2", "127.0.0.1", 26003, 256, 64, "hip"}};
    int ok = 0;
    for (const auto& dom : g.domains) {
      auto rt = hcp_ringattn::CreateRingAttnRuntime(dom.device);
      hcp_ringattn::RingAttnSoftmaxState init_state, out_state;
      if (!rt->Init(dom, g).ok()) return -1;
      if (!rt->RunRingAttentionLayer(0, init_state, &out_state).ok()) return -2;
      if (!rt->Shutdown().ok()) return -3;
      ++ok;
    }
    return ok;
  } catch (const std::exception&) {
    return -10;
  } catch (...) {
    return -11;
  }
}

size_t hcp_ring_replay_workspace_size(const hcp_ring_replay_desc* desc, int32_t paged) {
  try {
    return plan_replay(desc, paged != 0).total;
  } catch (...) {
    return 0;
  }
}

int hcp_ring_prefill_replay(const hcp_ring_replay_desc* desc, hcp_ring_view q, hcp_ring_view k, hcp_ring_view v,
                            hcp_ring_view out, float* lse_out, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return guarded(__func__, [&] {
    run_replay(desc, q, k, v, nullptr, nullptr, 0, out, lse_out, workspace, workspace_bytes, as_stream(stream));
  });
}

int hcp_ring_prefill_replay_paged(const hcp_ring_replay_desc* desc, hcp_ring_view q, const hcp_paged_pool* pool,
                                  const int32_t* block_table, int64_t table_len, hcp_ring_view out, float* lse_out,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  return guarded(__func__, [&] {
    check_pool(pool);
    hcp_ring_view none{nullptr, 0, 1};
    run_replay(desc, q, none, none, pool, block_table, table_len, out, lse_out, workspace, workspace_bytes,
               as_stream(stream));
  });
}

int hcp_ring_trace_attach(void* buffer, size_t bytes) {
  return guarded(__func__, [&] {
    require(buffer == nullptr || bytes > 0, "empty trace buffer");
    require(reinterpret_cast<uintptr_t>(buffer) % 8 == 0, "trace buffer must be 8-byte aligned");
    g_trace = TraceState{};
    g_trace.buf = buffer;
    g_trace.bytes = buffer != nullptr ? bytes : 0;
  });
}

size_t hcp_ring_trace_record_bytes(const hcp_ring_replay_desc* desc) {
  try {
    const ReplayPlan p = plan_replay(desc, false);
    const int64_t wg = ring_fused_workgroups(desc->num_q_heads, desc->num_kv_heads, p.n, p.len.data());
    return static_cast<size_t>(wg) * ring_trace_words(p.n) * sizeof(uint32_t);
  } catch (...) {
    return 0;
  }
}

int hcp_ring_trace_read(void* stream, hcp_ring_trace_domain* out, int32_t capacity, int32_t* num_domains,
                        hcp_ring_trace_launch* launch) {
  return guarded(__func__, [&] {
    require(out != nullptr && num_domains != nullptr, "null output");
    std::vector<hcp_ring_trace_domain> doms;
    hcp_ring_trace_launch L;
    trace_stats(as_stream(stream), doms, L);
    require(capacity >= static_cast<int32_t>(doms.size()), "capacity below the number of domains");
    std::copy(doms.begin(), doms.end(), out);
    *num_domains = static_cast<int32_t>(doms.size());
    if (launch != nullptr) *launch = L;
  });
}

int hcp_ring_trace_perf_log(void* stream, int32_t layer_idx, const char* path) {
  return guarded(__func__, [&] {
    const char* target = path != nullptr ? path : std::getenv("HCP_PERF_LOG");
    if (target == nullptr || *target == 0) return;
    std::vector<hcp_ring_trace_domain> doms;
    hcp_ring_trace_launch L;
    trace_stats(as_stream(stream), doms, L);
    const auto now = std::chrono::system_clock::now().time_since_epoch();
    const long long ms_total = std::chrono::duration_cast<std::chrono::milliseconds>(now).count();
    char ts[48];
    std::snprintf(ts, sizeof ts, "%lld.%03lldZ", ms_total / 1000, ms_total % 1000);
    std::string lines;
    for (const auto& D : doms) {
      char buf[1024];
      std::snprintf(buf, sizeof buf,
                    "{\"ts\":\"%s\",\"event\":\"ring_attention\",\"domain\":%d,\"layer\":%d,\"total_ms\":%.3f,"
                    "\"local_compute_ms\":%.3f,\"peer_compute_ms\":%.3f,\"recv_ms\":0.000,\"send_ms\":0.000,"
                    "\"forward_ms\":0.000,\"flush_ms\":0.000,\"kv_sent_bytes\":%lld,\"kv_recv_bytes\":%lld,"
                    "\"wire_sent_bytes\":0,\"wire_recv_bytes\":0,\"micro_blocks\":%lld,\"num_domains\":%d,"
                    "\"seq_len\":%lld,\"overlap\":1,\"workgroups\":%d,\"key_tiles\":%lld,\"local_cu_ms\":%.3f,"
                    "\"peer_cu_ms\":%.3f,\"clock_mhz\":%.1f,\"schedule\":\"fused\"}\n",
                    ts, D.domain, layer_idx, D.span_ms, D.local_compute_ms, D.peer_compute_ms,
                    static_cast<long long>(D.kv_sent_bytes), static_cast<long long>(D.kv_recv_bytes),
                    static_cast<long long>(D.peer_chunks), g_trace.n,
                    static_cast<long long>(g_trace.len[D.domain]), D.workgroups,
                    static_cast<long long>(D.key_tiles), D.local_cu_ms, D.peer_cu_ms, D.clock_mhz);
      lines += buf;
    }
    FILE* f = std::fopen(target, "a");
    require(f != nullptr, std::string("cannot open perf log ") + target);
    const size_t wrote = std::fwrite(lines.data(), 1, lines.size(), f);
    std::fclose(f);
    require(wrote == lines.size(), std::string("short write to perf log ") + target);
  });
}

int hcp_ring_replay_timing(int32_t enable) {
  return guarded(__func__, [&] {
    ReplayTiming& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    t.enabled = enable != 0;
  });
}

int hcp_ring_replay_timing_read(double* ms, int64_t* launches) {
  return guarded(__func__, [&] {
    require(ms != nullptr && launches != nullptr, "null output arrays");
    ReplayTiming& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    for (int k = 0; k < kTimedKinds; ++k) {
      ms[k] = 0.0;
      launches[k] = 0;
    }
    for (auto& e : t.pending) {
      HCP_HIP(hipEventSynchronize(e.second.second));
      float el = 0.f;
      HCP_HIP(hipEventElapsedTime(&el, e.second.first, e.second.second));
      ms[e.first] += el;
      launches[e.first] += 1;
      t.pool.push_back(e.second.first);
      t.pool.push_back(e.second.second);
    }
    t.pending.clear();
  });
}

int hcp_synth_normals(uint64_t seed, int64_t offset, int64_t count, int32_t dtype, void* out, void* stream) {
  return guarded(__func__, [&] {
    require(offset >= 0 && count >= 0, "offset and count must be >= 0");
    if (count > 0) require(out != nullptr, "null out");
    launch_synth_normals(seed, offset, count, dtype, out, as_stream(stream));
  });
}

}  // extern "C"
