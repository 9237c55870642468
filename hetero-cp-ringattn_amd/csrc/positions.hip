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
// binary search.  A key list in any other order is sorted first, with its K / V rows
// (launch_key_sort, launch_kv_sorted_gather below).
#include <algorithm>

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
  // the sorted copy when the key list was found out of order (positioned block entry)
  const bool sorted_copy = a.sel != nullptr && *a.sel != 0;
  const int64_t* kp = (sorted_copy ? a.k_pos_sorted : a.k_pos) + a.k_off[src];
  const int64_t len = a.k_len[src];
  if (a.err != nullptr && r + 1 < len && kp[r] > kp[r + 1]) atomicOr(a.err, 2);
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

// ---- keys in any order ----
// The visible keys of a query row are a prefix of the key list only when the list is
// non-decreasing.  Attention does not depend on the order of its keys, so a list that
// is not (the reference's committed-KV slab appends positions in arrival order,
// self_driving.rs:180-224, and its own test passes [0, 4, 3, 5], ring.rs:2343) is
// sorted on the device, with its rows, and the block kernels read K / V through the
// sorted row order from copies in the workspace.  key_order_kernel decides; every
// later kernel of the sequence does nothing when the list was already in order, so a
// sorted list costs a few empty launches and no copy.

constexpr int kOrderThreads = 1024;
constexpr int kSortTile = 2048;      // (key, row) pairs sorted per workgroup in LDS
constexpr int kSortThreads = 1024;

// (key, row) pairs compare by key, then row: all pairs are distinct, so every pass is
// a permutation and equal keys keep their list order.
__device__ __forceinline__ bool pair_less(int64_t ka, int32_t ia, int64_t kb, int32_t ib) {
  return ka < kb || (ka == kb && ia < ib);
}

// *flag = 1 iff k[j] > k[j + 1] for some j (one workgroup, so no flag clearing is needed).
__global__ __launch_bounds__(kOrderThreads) void key_order_kernel(const int64_t* k, int64_t n, int* flag) {
  int bad = 0;
  for (int64_t j = threadIdx.x; j + 1 < n; j += kOrderThreads) bad |= k[j] > k[j + 1] ? 1 : 0;
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) *flag = bad;
}

// Bitonic sort of one tile of kSortTile pairs in LDS; the tile past n is padded with
// pairs larger than any real one, which end up at its end and are not written.
__global__ __launch_bounds__(kSortThreads) void key_tile_sort_kernel(const int64_t* k, int64_t n, const int* flag,
                                                                     int64_t* okey, int32_t* orow) {
  if (*flag == 0) return;
  __shared__ int64_t sk[kSortTile];
  __shared__ int32_t sr[kSortTile];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
  for (int e = threadIdx.x; e < kSortTile; e += kSortThreads) {
    const int64_t g = base + e;
    sk[e] = g < n ? k[g] : INT64_MAX;
    sr[e] = g < n ? static_cast<int32_t>(g) : INT32_MAX;
  }
  __syncthreads();
  for (int size = 2; size <= kSortTile; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int e = threadIdx.x; e < kSortTile; e += kSortThreads) {
        const int p = e ^ stride;
        if (p > e) {
          const bool ascending = (e & size) == 0;
          const bool e_greater = pair_less(sk[p], sr[p], sk[e], sr[e]);
          if (e_greater == ascending) {
            const int64_t tk = sk[e];
            sk[e] = sk[p];
            sk[p] = tk;
            const int32_t tr = sr[e];
            sr[e] = sr[p];
            sr[p] = tr;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int e = threadIdx.x; e < kSortTile; e += kSortThreads) {
    const int64_t g = base + e;
    if (g < n) {
      okey[g] = sk[e];
      orow[g] = sr[e];
    }
  }
}

// One merge pass: sorted runs of `width` pairs are merged two by two.  Each pair goes
// to its rank in the merged run: its index in its own run plus the number of pairs of
// the partner run that are smaller (binary search; distinct pairs make the ranks a
// permutation of the two runs' slots).  A run without a partner is copied through.
__global__ __launch_bounds__(kPosThreads) void key_merge_kernel(const int64_t* ikey, const int32_t* irow, int64_t n,
                                                                int64_t width, const int* flag, int64_t* okey,
                                                                int32_t* orow) {
  if (*flag == 0) return;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kPosThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t run = i / width;
  const int64_t o0 = (run ^ 1) * width;
  const int64_t o1 = o0 + width < n ? o0 + width : n;
  const int64_t x = ikey[i];
  const int32_t xr = irow[i];
  int64_t lo = o0, hi = o0 < n ? o1 : o0;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (pair_less(ikey[mid], irow[mid], x, xr)) lo = mid + 1;
    else hi = mid;
  }
  const int64_t out = (run & ~int64_t(1)) * width + (i - run * width) + (lo - o0);
  okey[out] = x;
  orow[out] = xr;
}

// Row r of every head of the sorted copies is row rows[r] of the K / V views, moved in
// units of U bytes (U divides the row bytes and both views' byte strides and bases).
template <typename U>
__global__ __launch_bounds__(kPosThreads) void kv_sorted_gather_kernel(KvSortedGather g) {
  if (*g.flag == 0) return;
  const int64_t units_per_row = g.row_bytes / static_cast<int64_t>(sizeof(U));
  const int64_t total = static_cast<int64_t>(g.hkv) * g.n * units_per_row;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * kPosThreads + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * kPosThreads) {
    const int64_t c = u % units_per_row;
    const int64_t hr = u / units_per_row;  // head * n + sorted row
    const int64_t h = hr / g.n, r = hr - h * g.n;
    const int64_t src = g.rows[r];
    const int64_t ko = h * g.k_hs_bytes + src * g.k_ss_bytes;
    const int64_t vo = h * g.v_hs_bytes + src * g.v_ss_bytes;
    reinterpret_cast<U*>(g.kc)[u] = reinterpret_cast<const U*>(g.k + ko)[c];
    reinterpret_cast<U*>(g.vc)[u] = reinterpret_cast<const U*>(g.v + vo)[c];
  }
}

}  // namespace

int key_sort_passes(int64_t n) {
  int passes = 0;
  for (int64_t w = kSortTile; w < n; w <<= 1) ++passes;
  return passes;
}

void launch_key_sort(const int64_t* k, int64_t n, int* flag, int64_t* const key[2], int32_t* const row[2],
                     hipStream_t stream) {
  if (n <= 0) return;
  key_order_kernel<<<1, kOrderThreads, 0, stream>>>(k, n, flag);
  HCP_HIP(hipGetLastError());
  key_tile_sort_kernel<<<static_cast<unsigned>(ceil_div(n, kSortTile)), kSortThreads, 0, stream>>>(k, n, flag, key[0],
                                                                                                    row[0]);
  HCP_HIP(hipGetLastError());
  int cur = 0;
  for (int64_t w = kSortTile; w < n; w <<= 1, cur ^= 1) {
    key_merge_kernel<<<static_cast<unsigned>(ceil_div(n, kPosThreads)), kPosThreads, 0, stream>>>(
        key[cur], row[cur], n, w, flag, key[cur ^ 1], row[cur ^ 1]);
    HCP_HIP(hipGetLastError());
  }
}

void launch_kv_sorted_gather(const KvSortedGather& g, hipStream_t stream) {
  if (g.n <= 0 || g.hkv <= 0) return;
  const uint64_t bits = static_cast<uint64_t>(g.row_bytes) | static_cast<uint64_t>(g.k_hs_bytes) |
                        static_cast<uint64_t>(g.k_ss_bytes) | static_cast<uint64_t>(g.v_hs_bytes) |
                        static_cast<uint64_t>(g.v_ss_bytes) | reinterpret_cast<uintptr_t>(g.k) |
                        reinterpret_cast<uintptr_t>(g.v) | reinterpret_cast<uintptr_t>(g.kc) |
                        reinterpret_cast<uintptr_t>(g.vc);
  const int unit = (bits & 15) == 0 ? 16 : (bits & 7) == 0 ? 8 : (bits & 3) == 0 ? 4 : (bits & 1) == 0 ? 2 : 1;
  const int64_t total = static_cast<int64_t>(g.hkv) * g.n * (g.row_bytes / unit);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, kPosThreads), 65536));
  switch (unit) {
    case 16: kv_sorted_gather_kernel<uint4><<<blocks, kPosThreads, 0, stream>>>(g); break;
    case 8: kv_sorted_gather_kernel<uint2><<<blocks, kPosThreads, 0, stream>>>(g); break;
    case 4: kv_sorted_gather_kernel<uint32_t><<<blocks, kPosThreads, 0, stream>>>(g); break;
    case 2: kv_sorted_gather_kernel<uint16_t><<<blocks, kPosThreads, 0, stream>>>(g); break;
    default: kv_sorted_gather_kernel<uint8_t><<<blocks, kPosThreads, 0, stream>>>(g); break;
  }
  HCP_HIP(hipGetLastError());
}

void launch_domain_positions(const StrategySpec& s, int64_t seq, int64_t* out, hipStream_t stream) {
  if (seq <= 0) return;
  domain_positions_kernel<<<static_cast<unsigned>(ceil_div(seq, kPosThreads)), kPosThreads, 0, stream>>>(s, seq,
                                                                                                          out);
  HCP_HIP(hipGetLastError());
}

namespace {
// Positions that are a permutation of [0, n) (a replay's strategy positions): row
// rows[p] holds position p, and row r sees the keys [0, pos[r] + 1) of the position-
// ordered list.  *flag = 1 selects the position-ordered K / V copies.  A position out
// of range (not produced by the strategy kernel) is skipped and flagged (error bit 1).
__global__ __launch_bounds__(kPosThreads) void position_inverse_kernel(const int64_t* pos, int64_t n, int32_t* rows,
                                                                       int32_t* lim, int* flag, int* err) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kPosThreads + threadIdx.x;
  if (r == 0) *flag = 1;
  if (r >= n) return;
  const int64_t p = pos[r];
  if (p < 0 || p >= n) {
    atomicOr(err, 2);
    lim[r] = 0;
    return;
  }
  rows[p] = static_cast<int32_t>(r);
  lim[r] = static_cast<int32_t>(p + 1);
}
}  // namespace

void launch_position_inverse(const int64_t* pos, int64_t n, int32_t* rows, int32_t* lim, int* flag, int* err,
                             hipStream_t stream) {
  if (n <= 0) return;
  position_inverse_kernel<<<static_cast<unsigned>(ceil_div(n, kPosThreads)), kPosThreads, 0, stream>>>(pos, n, rows,
                                                                                                       lim, flag, err);
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
