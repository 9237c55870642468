// Single-query paged decode partial over one domain chunk.
//
// Replaces decode_local_partial / decode_local_compact_partial (ring.rs:625-639,
// :515-523): one query token per sequence, no causal mask (ring.rs:631-637), output
// normalised o and natural-log lse in fp32.  KV is read in place from the vLLM pool
// [2, num_blocks, bs, Hkv, D] (python/hcp_vllm_block_ring_plugin.py:8-14) through the
// sequence's block table -- no gather, no GQA expand copy.
//
// Work split (HBM-bound: every K/V byte is read exactly once):
//   * grid = (splits, batch, ceil(Hkv / W)) with W = min(8, Hkv) waves per workgroup, so one
//     workgroup reads whole pool token rows (4 waves: 0.7% slower on c4).
//     A workgroup owns one sequence, a contiguous run of 16-token groups of the chunk
//     and W kv heads: wave w handles kv head W*blockIdx.z + w, so per 16 tokens a wave
//     reads 16 K rows and 16 V rows of its head (4 KiB each for D=128, bf16) straight
//     from the pool.
//   * Scores: S^T = K Q^T on MFMA 16x16x32 (A = 16 key rows loaded from the pool, 16
//     bytes per lane; B = the rep <= 16 query heads of the kv head -- the GQA group of
//     repeat_decode_kv_heads, ring.rs:496-512 -- zero-padded to 16 columns, held in
//     registers for the whole kernel).
//   * Online softmax per query head in the log2 domain; P goes through a small LDS
//     slot (broadcast reads) and PV runs on VALU with each lane owning 8 head-dim
//     values of 4 of the 16 keys for R query heads (R = 4, 8 or 16, the smallest that
//     holds rep; fp32 accumulators), reduced across lanes once at the end.
//   * Each split writes (o, lse) to the workspace; the LSE merge kernel combines the
//     splits of a sequence (heads = batch*Hq, q_len = 1).
#include <map>
#include <mutex>
#include <tuple>

#include "kernels.hpp"

namespace hcp {

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_bs, q_hs;  // element strides: batch, head
  const uint16_t* pool;
  int64_t plane_elems;
  int64_t num_blocks;
  int32_t bs, hkv, hq, rep;
  const int32_t* tables;
  int64_t table_stride, table_len;
  const int32_t* seq_lens;
  int64_t t0, t1;
  int64_t g_begin;      // first 16-token group index (t0 / 16)
  int32_t groups_per_split;
  int32_t n_groups;     // total groups in [g_begin*16, t1)
  float scale_log2;
  float* ws_o;          // [splits][batch*hq][D]
  float* ws_lse;        // [splits][batch*hq]
  int32_t batch;
  int* err;
  int32_t dn;           // head dim of the pool rows, q and the partials (the D=128 kernel:
                        // any multiple of 8 up to 128, columns past it read as zeros)
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ f32x4 mma16(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mma16<kBF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mma16<kF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ float lo_half(uint32_t w) {
  return DT == kBF16 ? __uint_as_float(w << 16) : f16_bits_to_f32(static_cast<uint16_t>(w & 0xffffu));
}
template <int DT>
__device__ __forceinline__ float hi_half(uint32_t w) {
  return DT == kBF16 ? __uint_as_float(w & 0xffff0000u) : f16_bits_to_f32(static_cast<uint16_t>(w >> 16));
}

constexpr int kDecWaves = 8;  // most kv heads per workgroup (one per wave)

// One wave per kv head.  Per 16-key group the wave needs the head's 16 K rows and 16 V
// rows (4 KiB each for D=128); the next group's loads are issued before a group is
// computed, and the block ids come from one table load per 64 groups.
template <int D, int DT, int R, bool PAD>
__global__ __launch_bounds__(512) void paged_decode_kernel(DecodeArgs a) {
  // PAD: head dim a.dn < D; the 16-byte columns past it are not loaded (zeros) nor stored
  const int dn = PAD ? a.dn : D;
  constexpr int KS = D / 32;        // k-steps of 32 for the QK^T product
  constexpr int DCH = D / 8;        // 8-wide d chunks per row (16 for D=128)
  constexpr int TPL = 16 * DCH / 64;  // keys per lane in PV (4 for D=128)

  __shared__ __attribute__((aligned(16))) float p_lds[kDecWaves][16][R];  // [wave][key][query col]

  const int b = blockIdx.y;
  const int split = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kvh = blockIdx.z * (blockDim.x >> 6) + wave;
  if (kvh >= a.hkv) return;  // no workgroup barriers below
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;   // MFMA column = query head within the kv group
  const int grp = lane >> 4;   // MFMA k-group / key group
  // PV role: lane owns d chunk pv_dc (8 values) of keys pv_tg*TPL .. +TPL.
  const int pv_dc = lane % DCH;
  const int pv_tg = lane / DCH;

  int64_t t_end = a.t1;
  if (a.seq_lens != nullptr) t_end = min(t_end, static_cast<int64_t>(a.seq_lens[b]));
  const int g0 = split * a.groups_per_split;
  // Stop at this sequence's own last group: table entries past its length may be
  // padding (ragged batches) and are neither read nor validated.
  const int64_t g_seq = t_end > a.t0 ? (t_end + 15) / 16 - a.g_begin : 0;
  const int g1 = static_cast<int>(min(static_cast<int64_t>(min(a.n_groups, g0 + a.groups_per_split)), g_seq));
  const int32_t* table = a.tables + static_cast<int64_t>(b) * a.table_stride;

  // Q^T fragments: lane (col, grp) holds Q[head kvh*rep + col][grp*8 + 32*s .. +8].
  u32x4 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    u32x4 v = {0, 0, 0, 0};
    if (col < a.rep && (!PAD || grp * 8 + 32 * s < dn))
      v = *reinterpret_cast<const u32x4*>(a.q + b * a.q_bs + (kvh * a.rep + col) * a.q_hs + grp * 8 + 32 * s);
    qf[s] = v;
  }

  // PV accumulators cover rep <= R query heads per kv head (checked by the launcher).
  float acc[R][8];
#pragma unroll
  for (int c = 0; c < R; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[c][e] = 0.f;
  float m_run = -1.0e30f, l_run = 0.f;

  const int64_t row_elems = static_cast<int64_t>(a.hkv) * dn;  // one slot, all heads

  struct Group {
    u32x4 k[KS];
    u32x4 v[TPL];
    int64_t tok0;
    bool ok;
  };
  // Block ids of the split's groups, 64 at a time: lane i holds the table entry of
  // group ids_base + i, read back with readlane, so no group waits on a table load.
  // Keys tok0 .. tok0+15 of group g lie in table entry tok0 / bs (bs is a multiple of 16).
  int ids = -1, ids_base = g0 - 64;
  auto block_of = [&](int g, int64_t entry) __attribute__((always_inline)) {
    if (g - ids_base >= 64) {
      ids_base = g;
      const int64_t e = (a.g_begin + g + lane) * 16 / a.bs;
      ids = g + lane < g1 && e < a.table_len ? table[e] : -1;
    }
    const int32_t blk = __builtin_amdgcn_readlane(ids, g - ids_base);
    return entry < a.table_len ? blk : -1;
  };
  auto load_group = [&](int g, Group& G) {
    G.tok0 = (a.g_begin + g) * 16;
    const int64_t entry = G.tok0 / a.bs;
    const int32_t blk = block_of(g, entry);
    G.ok = blk >= 0 && blk < a.num_blocks;
    if (!G.ok) {
      if (lane == 0 && entry < a.table_len) atomicOr(a.err, 1);
#pragma unroll
      for (int s = 0; s < KS; ++s) G.k[s] = u32x4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < TPL; ++j) G.v[j] = u32x4{0, 0, 0, 0};
      return;
    }
    const int slot0 = static_cast<int>(G.tok0 - entry * a.bs);
    const uint16_t* kslot = a.pool + (static_cast<int64_t>(blk) * a.bs + slot0) * row_elems + kvh * dn;
    const uint16_t* krow = kslot + col * row_elems + grp * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      G.k[s] = !PAD || grp * 8 + 32 * s < dn ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(krow + 32 * s))
                                             : u32x4{0, 0, 0, 0};
    const uint16_t* vrow = kslot + a.plane_elems + pv_dc * 8;
    const bool v_in = !PAD || pv_dc * 8 < dn;
#pragma unroll
    for (int j = 0; j < TPL; ++j)
      G.v[j] = v_in ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vrow + (pv_tg * TPL + j) * row_elems))
                    : u32x4{0, 0, 0, 0};
  };
  auto compute_group = [&](const Group& G) {
    if (!G.ok) return;
    // ---- S^T = K Q^T: lane (col = query, grp) holds keys grp*4 + i ----
    f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) s4 = mma16<DT>(G.k[s], qf[s], s4);
    float tmax = -INFINITY;
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t t = G.tok0 + grp * 4 + i;
      const bool ok = t >= a.t0 && t < t_end;
      sv[i] = ok ? s4[i] * a.scale_log2 : -INFINITY;
      tmax = fmaxf(tmax, sv[i]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = __builtin_amdgcn_exp2f(sv[i] - m_new);
      psum += p;
      if (col < R) p_lds[wave][grp * 4 + i][col] = p;
    }
    l_run = l_run * alpha + psum;  // per-lane partial over its keys (rescaled)
    // alpha of query column c lives in lane c.
    float al[R];
#pragma unroll
    for (int c = 0; c < R; ++c) al[c] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), c));
#pragma unroll
    for (int c = 0; c < R; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[c][e] *= al[c];
    __builtin_amdgcn_wave_barrier();
    // ---- O += P V (VALU): lane owns 8 head-dim values of keys pv_tg*TPL .. +TPL ----
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
      const int key = pv_tg * TPL + j;
      const int64_t t = G.tok0 + key;
      const bool ok = t >= a.t0 && t < t_end;
      const u32x4 vv = ok ? G.v[j] : u32x4{0, 0, 0, 0};
      float vf[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        vf[2 * w] = lo_half<DT>(vv[w]);
        vf[2 * w + 1] = hi_half<DT>(vv[w]);
      }
#pragma unroll
      for (int c4 = 0; c4 < R; c4 += 4) {
        const float4 p4 = *reinterpret_cast<const float4*>(&p_lds[wave][key][c4]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[c4][e] += p4.x * vf[e];
          acc[c4 + 1][e] += p4.y * vf[e];
          acc[c4 + 2][e] += p4.z * vf[e];
          acc[c4 + 3][e] += p4.w * vf[e];
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // Rolling double buffer: group g + 1 is loading while group g is computed.
  Group ga, gb;
  if (g0 < g1) load_group(g0, ga);
  for (int g = g0; g < g1; g += 2) {
    if (g + 1 < g1) load_group(g + 1, gb);
    compute_group(ga);
    if (g + 2 < g1) load_group(g + 2, ga);
    if (g + 1 < g1) compute_group(gb);
  }

  // ---- epilogue: reduce over key subgroups, normalise, write split partial ----
  const int64_t ws_row_base = static_cast<int64_t>(split) * a.batch * a.hq + static_cast<int64_t>(b) * a.hq;
  float l = l_run;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);  // lanes with the same col now hold the total over keys
#pragma unroll
  for (int c = 0; c < R; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[c][e];
      // Lanes with equal pv_dc hold the same d for different key subgroups.
      for (int off = DCH; off < 64; off *= 2) v += __shfl_xor(v, off);
      acc[c][e] = v;
    }
  float lc[R];
#pragma unroll
  for (int c = 0; c < R; ++c) lc[c] = __shfl(l, c);
  if (pv_tg == 0 && (!PAD || pv_dc * 8 < dn)) {
#pragma unroll
    for (int c = 0; c < R; ++c) {
      if (c >= a.rep) break;
      const float inv = lc[c] > 0.f ? 1.f / lc[c] : 0.f;
      float* orow = a.ws_o + (ws_row_base + kvh * a.rep + c) * dn + pv_dc * 8;
      reinterpret_cast<float4*>(orow)[0] =
          make_float4(acc[c][0] * inv, acc[c][1] * inv, acc[c][2] * inv, acc[c][3] * inv);
      reinterpret_cast<float4*>(orow)[1] =
          make_float4(acc[c][4] * inv, acc[c][5] * inv, acc[c][6] * inv, acc[c][7] * inv);
    }
  }
  if (lane < a.rep && lane < R) {
    const float lt = l;  // lane c holds column c's total
    a.ws_lse[ws_row_base + kvh * a.rep + lane] = lt > 0.f ? (m_run + __log2f(lt)) * kLn2 : -INFINITY;
  }
}

struct DecodePlan {
  int splits;
  int groups_per_split;
  int n_groups;
  int64_t g_begin;
};

// Query heads per kv head the PV accumulators hold: the smallest of 4, 8, 16 >= rep.
int decode_width(int rep) { return rep <= 4 ? 4 : rep <= 8 ? 8 : 16; }
// Waves (kv heads) per workgroup.
int decode_waves(int hkv) { return std::min(hkv, kDecWaves); }

template <int D, int DT, bool PAD = false>
const void* decode_fn(int r) {
  switch (r) {
    case 4: return reinterpret_cast<const void*>(&paged_decode_kernel<D, DT, 4, PAD>);
    case 8: return reinterpret_cast<const void*>(&paged_decode_kernel<D, DT, 8, PAD>);
    default: return reinterpret_cast<const void*>(&paged_decode_kernel<D, DT, 16, PAD>);
  }
}

// Workgroups of the decode kernel resident at once on the current device (CUs x
// occupancy); 256 CUs x 3 when no device can be queried.
int decode_slots(int d, int dtype, int r, int waves) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, int, int, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 768;
  }
  std::lock_guard<std::mutex> lock(mu);
  // the instantiation the launch takes: head dims other than 64 and 128 run the
  // zero-padding (PAD) build of the 128 kernel, whose register use may differ
  const bool pad = d != 64 && d != 128;
  const int dk = d == 64 ? 64 : pad ? -1 : 128;
  const auto key = std::make_tuple(dev, dk, dtype, r, waves);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int cus = 0, per_cu = 0;
  const void* fn = dtype == kBF16
                       ? (d == 64 ? decode_fn<64, kBF16>(r) : pad ? decode_fn<128, kBF16, true>(r) : decode_fn<128, kBF16>(r))
                       : (d == 64 ? decode_fn<64, kF16>(r) : pad ? decode_fn<128, kF16, true>(r) : decode_fn<128, kF16>(r));
  int slots = 768;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 64 * waves, 0) == hipSuccess && cus > 0 &&
      per_cu > 0)
    slots = cus * per_cu;
  else
    (void)hipGetLastError();
  cache[key] = slots;
  return slots;
}

DecodePlan plan_decode(int batch, int hq, int hkv, int d, int dtype, int64_t t0, int64_t t1) {
  DecodePlan p;
  p.g_begin = t0 / 16;
  const int64_t g_end = t1 > t0 ? (t1 + 15) / 16 : p.g_begin;
  p.n_groups = static_cast<int>(g_end - p.g_begin);
  // grid = splits x batch x kv-head groups.  One round of resident workgroups: a
  // partial second round leaves most CUs idle for its whole length (a measured 13-25%
  // loss at c4), and fewer splits also mean fewer partials to merge.  At least 4 groups
  // (64 keys) per split.
  const int waves = decode_waves(hkv);
  const int rows = std::max(batch, 1) * ((hkv + waves - 1) / waves);
  int splits = std::max(1, decode_slots(d, dtype, decode_width(hq / hkv), waves) / rows);
  splits = std::min(splits, 64);
  int gps = static_cast<int>(ceil_div(std::max(p.n_groups, 1), splits));
  gps = std::max(gps, 4);
  p.groups_per_split = gps;
  p.splits = static_cast<int>(ceil_div(std::max(p.n_groups, 1), gps));
  return p;
}

size_t decode_workspace_bytes(int dtype, int batch, int hq, int hkv, int d, int64_t t0, int64_t t1) {
  const DecodePlan p = plan_decode(batch, hq, hkv, d, dtype, t0, t1);
  const size_t rows = static_cast<size_t>(p.splits) * batch * hq;
  auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
  return al(rows * d * sizeof(float)) + al(rows * sizeof(float));
}

template <int D, int DT, bool PAD = false>
static void launch_decode_kernel(int r, dim3 grid, int waves, const DecodeArgs& a, hipStream_t stream) {
  switch (r) {
    case 4: paged_decode_kernel<D, DT, 4, PAD><<<grid, 64 * waves, 0, stream>>>(a); break;
    case 8: paged_decode_kernel<D, DT, 8, PAD><<<grid, 64 * waves, 0, stream>>>(a); break;
    default: paged_decode_kernel<D, DT, 16, PAD><<<grid, 64 * waves, 0, stream>>>(a); break;
  }
}

void launch_paged_decode(int dtype, int batch, int hq, int hkv, int d, const void* q, int64_t q_bs,
                         int64_t q_hs, const void* pool, int64_t num_blocks, int bs,
                         const int32_t* tables, int64_t table_stride, int64_t table_len,
                         const int32_t* seq_lens, int64_t t0, int64_t t1, float scale, float* o,
                         float* lse, void* ws, size_t ws_bytes, int* err, hipStream_t stream) {
  require(hq % hkv == 0 && hq / hkv <= 16, "paged_decode: num_q_heads/num_kv_heads must be <= 16");
  require(bs % 16 == 0, "paged_decode: block_size must be a multiple of 16");
  require(d > 0 && d <= 128 && d % 8 == 0, "paged_decode: head_dim must be a multiple of 8 up to 128");
  require(dtype == kBF16 || dtype == kF16, "paged_decode: dtype must be BF16 or F16");
  const DecodePlan p = plan_decode(batch, hq, hkv, d, dtype, t0, t1);
  require(ws_bytes >= decode_workspace_bytes(dtype, batch, hq, hkv, d, t0, t1), "paged_decode: workspace too small");
  auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
  const size_t rows = static_cast<size_t>(p.splits) * batch * hq;
  float* ws_o = static_cast<float*>(ws);
  float* ws_lse = reinterpret_cast<float*>(static_cast<char*>(ws) + al(rows * d * sizeof(float)));

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_bs = q_bs;
  a.q_hs = q_hs;
  a.pool = static_cast<const uint16_t*>(pool);
  a.plane_elems = num_blocks * bs * hkv * static_cast<int64_t>(d);
  a.num_blocks = num_blocks;
  a.bs = bs;
  a.hkv = hkv;
  a.hq = hq;
  a.rep = hq / hkv;
  a.tables = tables;
  a.table_stride = table_stride;
  a.table_len = table_len;
  a.seq_lens = seq_lens;
  a.t0 = t0;
  a.t1 = t1;
  a.g_begin = p.g_begin;
  a.groups_per_split = p.groups_per_split;
  a.n_groups = p.n_groups;
  a.scale_log2 = scale * kLog2e;
  a.ws_o = ws_o;
  a.ws_lse = ws_lse;
  a.batch = batch;
  a.err = err;
  a.dn = d;
  const int waves = decode_waves(hkv);
  const int r = decode_width(a.rep);
  const dim3 grid(static_cast<unsigned>(p.splits), static_cast<unsigned>(batch),
                  static_cast<unsigned>((hkv + waves - 1) / waves));
  // head dim 64: its own kernel; other multiples of 8 up to 128: the D=128 kernel with
  // the columns past d zero-padded
  if (dtype == kBF16) {
    if (d == 128) launch_decode_kernel<128, kBF16>(r, grid, waves, a, stream);
    else if (d == 64) launch_decode_kernel<64, kBF16>(r, grid, waves, a, stream);
    else launch_decode_kernel<128, kBF16, true>(r, grid, waves, a, stream);
  } else {
    if (d == 128) launch_decode_kernel<128, kF16>(r, grid, waves, a, stream);
    else if (d == 64) launch_decode_kernel<64, kF16>(r, grid, waves, a, stream);
    else launch_decode_kernel<128, kF16, true>(r, grid, waves, a, stream);
  }
  HCP_HIP(hipGetLastError());
  // Merge the splits of every (sequence, head): rows = batch*hq, one token each.
  const float* o_parts[64];
  const float* l_parts[64];
  for (int s = 0; s < p.splits; ++s) {
    o_parts[s] = ws_o + static_cast<size_t>(s) * batch * hq * d;
    l_parts[s] = ws_lse + static_cast<size_t>(s) * batch * hq;
  }
  launch_lse_merge(p.splits, o_parts, l_parts, batch * hq, 1, d, kF32, o, d, d, lse, 1, stream);
}

}  // namespace hcp
