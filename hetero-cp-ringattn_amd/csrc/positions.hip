// Global positions of non-contiguous scheduling strategies and per-row key limits.
//
// strategy.rs:53-143 assigns every global position of a prompt to a domain (Vanilla:
// contiguous chunks; Striped: weighted round-robin; ZigZag: a prefix run plus a suffix
// run per domain) and lists each domain's positions in ascending order (local storage
// order).  The reference builds these lists by scanning the whole sequence; here the
// i-th local position of domain d has a closed form (O(N) per element), evaluated on the
// host (assignment helpers, first/last positions for the future-source skip) and on the
// device (the replay's position arrays, generated in HBM without a host copy).
//
// Key limits: the causal mask of process_kv_block (ring.rs:201-370) keeps key j for
// query i iff k_pos[j] <= q_pos[i].  With key positions non-decreasing (every list the
// strategies produce, and any contiguous slice of one) the visible keys of a query row
// are a prefix of the key chunk, of length lim[i] = #{j : k_pos[j] <= q_pos[i]}.  The
// block kernels take lim[] instead of (q_offset, kv_offset) and keep their tile
// skipping: a tile is skipped when it starts at or past every row's limit of a wave and
// unmasked when it ends before every row's limit.  key_limits_kernel computes lim[] by
// binary search and flags key lists that are not non-decreasing (error bit 1).
#include "kernels.hpp"

namespace hcp {

__host__ __device__ int64_t strategy_position(const StrategySpec& s, int d, int64_t i) {
  const int n = s.n;
  if (s.strategy == kStrategyStriped) {
    // Round r hands one slot to every domain whose quota exceeds r, in domain order, so
    // the i-th slot of domain d is in round i after sum_e min(c_e, i) earlier slots and
    // after the domains e < d still active in round i.
    int64_t pos = 0;
    for (int e = 0; e < n; ++e) {
      const int64_t c = s.chunks[e];
      pos += c < i ? c : i;
      if (e < d && c > i) ++pos;
    }
    return pos;
  }
  if (s.strategy == kStrategyZigZag) {
    // Prefix run of ceil(c/2) in domain order, then suffix runs of floor(c/2) in
    // reverse domain order.
    int64_t before = 0, all_prefix = 0, later_suffix = 0;
    for (int e = 0; e < n; ++e) {
      const int64_t p = s.chunks[e] - s.chunks[e] / 2;
      all_prefix += p;
      if (e < d) before += p;
      if (e > d) later_suffix += s.chunks[e] / 2;
    }
    const int64_t pd = s.chunks[d] - s.chunks[d] / 2;
    return i < pd ? before + i : all_prefix + later_suffix + (i - pd);
  }
  int64_t off = 0;
  for (int e = 0; e < d; ++e) off += s.chunks[e];
  return off + i;
}

namespace {

constexpr int kPosThreads = 256;

__global__ __launch_bounds__(kPosThreads) void domain_positions_kernel(StrategySpec s, int64_t seq, int64_t* out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kPosThreads + threadIdx.x;
  if (r >= seq) return;
  int d = 0;
  int64_t i = r;
  while (d + 1 < s.n && i >= s.chunks[d]) {
    i -= s.chunks[d];
    ++d;
  }
  out[r] = strategy_position(s, d, i);
}

__global__ __launch_bounds__(kPosThreads) void key_limits_kernel(KeyLimitArgs a) {
  const int src = blockIdx.y;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kPosThreads + threadIdx.x;
  const int64_t* kp = a.k_pos + a.k_off[src];
  const int64_t len = a.k_len[src];
  if (r + 1 < len && kp[r] > kp[r + 1]) atomicOr(a.err, 2);
  if (r >= a.n_q) return;
  const int64_t qp = a.q_pos[r];
  int64_t lo = 0, hi = len;  // count of keys with position <= qp
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (kp[mid] <= qp) lo = mid + 1;
    else hi = mid;
  }
  a.lim[static_cast<int64_t>(src) * a.lim_stride + r] = static_cast<int32_t>(lo);
}

}  // namespace

void launch_domain_positions(const StrategySpec& s, int64_t seq, int64_t* out, hipStream_t stream) {
  if (seq <= 0) return;
  domain_positions_kernel<<<static_cast<unsigned>(ceil_div(seq, kPosThreads)), kPosThreads, 0, stream>>>(s, seq,
                                                                                                          out);
  HCP_HIP(hipGetLastError());
}

void launch_key_limits(const KeyLimitArgs& a, int n_src, int64_t max_k_len, hipStream_t stream) {
  const int64_t rows = a.n_q > max_k_len ? a.n_q : max_k_len;
  if (rows <= 0 || n_src <= 0) return;
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, kPosThreads)), static_cast<unsigned>(n_src));
  key_limits_kernel<<<grid, kPosThreads, 0, stream>>>(a);
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
