// Flash-style block kernel for one ring step: (query chunk, KV chunk) -> (o, lse) fp32.
//
// Replaces process_kv_block's op sequence (ring.rs:201-370: QK^T*scale, causal
// -inf mask on global positions, amax / exp / sum, PV, rescale-merge) and the
// positioned partial / merge wrappers (ring.rs:538-603).  The online softmax is the
// same recurrence; scores never leave registers.
//
// Matrix-core path (bf16 / fp16, head_dim 64 or 128), gfx950 MFMA 32x32x16:
//   * A workgroup is 8 waves.  Each wave owns 32 query tokens of ONE query head.
//     The 8 waves cover G query heads that share a KV head (GQA, G in {1,2,4,8}) times
//     8/G blocks of 32 tokens, so one K/V tile in LDS feeds 256 query rows and the
//     GQA expand of ring.rs:496-512 never materialises.
//   * Scores are computed transposed, S^T = K Q^T (A = K rows from LDS, B = Q held in
//     registers), so each lane owns one query column: the row max needs one cross-lane
//     exchange (lane ^ 32) and the row sum is reduced once at the end.
//   * The K rows of each 32-row MFMA block are read in a fixed permuted order (kperm)
//     chosen so that the fp32 S^T accumulator, converted to bf16, IS the B operand of
//     O^T = V^T P^T for k-steps of 16 keys.  V^T comes from LDS, where the loader
//     stores V transposed ([d][kv]) with a 4x8 register transpose.
//   * Online softmax in the log2 domain with the scale folded in; the running max is
//     only moved (and O rescaled) when a row's max grows by more than 8 (2^8 bound on
//     P), which keeps the result exact and skips most rescales.
//   * K/V tiles of 64 keys are double-buffered in LDS; global loads of tile t+1 are in
//     flight while tile t is computed.  One barrier per tile.
//   * Causal: tiles wholly in a wave's future are skipped, tiles wholly visible are
//     unmasked, only tiles straddling the diagonal (or the kv tail) are masked.
//
// General path (fp32, or any head_dim <= 256): one thread per (query row, head), K/V
// tiles staged in LDS as fp32.  Used for the fp32 CPU-smoke config.
#include "kernels.hpp"

namespace hcp {

struct BlockArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_hs, q_ss, k_hs, k_ss, v_hs, v_ss;  // element strides
  float* o;
  float* lse;
  int32_t hq, hkv, rep;   // rep = hq / hkv
  int32_t lq, lk;
  int64_t q_off, k_off;
  int32_t causal, accumulate;
  float scale_log2;        // softmax scale * log2(e)
  int32_t n_qtiles, n_groups;
};

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kBK = 64;           // keys per tile
constexpr int kKPad = 8;          // bf16 pad per K row in LDS
constexpr int kVtStride = kBK + 8;  // bf16 per V^T row in LDS (144 B)
constexpr float kRescaleThreshold = 8.0f;
constexpr float kInitMax = -1.0e30f;

// C-row r of a 32x32 S^T block holds key kperm(r) of that block:
// r = j*8 + h*4 + i  ->  16*(j/2) + 8*h + 4*(j%2) + i.
__device__ __forceinline__ int kperm(int r) {
  const int j = r >> 3, h = (r >> 2) & 1, i = r & 3;
  return 16 * (j >> 1) + 8 * h + 4 * (j & 1) + i;
}

template <int DT>
struct MfmaOps;

template <>
struct MfmaOps<kBF16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag pack(const float* p) {
    frag r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<__bf16>(p[i]);
    return r;
  }
};

template <>
struct MfmaOps<kF16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag pack(const float* p) {
    frag r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(p[i]);
    return r;
  }
};

template <typename F>
__device__ __forceinline__ F as_frag(u32x4 v) {
  return __builtin_bit_cast(F, v);
}

// Map blockIdx.x so that each XCD (blocks are dealt round-robin over 8 XCDs) gets a
// contiguous range of logical tiles: neighbouring tiles share K/V in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int kXcd = 8;
  const int per = nblocks / kXcd;
  const int rem = nblocks % kXcd;
  const int xcd = bid % kXcd;
  const int idx = bid / kXcd;
  // XCDs [0, rem) own per+1 tiles, the rest own per.
  const int start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
  return start + idx;
}

}  // namespace

// Raw buffer resource over [base, base + bytes): loads past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int32_t n = bytes <= 0 ? 0 : (bytes > 0x7ffffff0LL ? 0x7ffffff0 : static_cast<int32_t>(bytes));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// {x[lane], x[lane ^ 32]} in some order, on the VALU (no LDS round trip).
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int D, int DT, int G>
__global__ __launch_bounds__(kThreads, 1) void flash_block_kernel(BlockArgs a) {
  using Ops = MfmaOps<DT>;
  using frag = typename Ops::frag;
  constexpr int TB = kWaves / G;  // 32-token blocks per workgroup
  constexpr int TQ = 32 * TB;     // query tokens per workgroup
  constexpr int KS = D / 16;      // k-steps of the QK^T product
  constexpr int DB = D / 32;      // 32-row blocks of O^T
  constexpr int KROW = D + kKPad; // bf16 per K row in LDS
  constexpr int KCH = D / 8;      // 16-byte chunks per K/V row
  constexpr int K_LOADS = kBK * KCH / 256;    // per K-loader thread
  constexpr int V_ITEMS = (kBK / 4) * KCH;    // (4-row group, chunk) items

  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[2][kBK * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][D * kVtStride];

  const int nblk = gridDim.x;
  const int logical = xcd_remap(blockIdx.x, nblk);
  // Head-group-major: each XCD's contiguous share of logical tiles covers the query
  // tiles of as few KV heads as possible, so its CUs stream the same K/V through that
  // XCD's L2.  Within a head group, heavier (later, causal) query tiles come first.
  const int hg = logical / a.n_qtiles;
  const int qt = a.n_qtiles - 1 - logical % a.n_qtiles;

  const int tid = threadIdx.x;
  // Wave index as a scalar: everything derived from it stays in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lcol = lane & 31;   // query column owned by this lane
  const int lhalf = lane >> 5;  // 0/1: which 8-wide k slice this lane feeds

  const int head = hg * G + (wave % G);
  const int kvh = (hg * G) / a.rep;
  const int tq0 = qt * TQ;                       // first query token of the workgroup
  const int wq0 = tq0 + (wave / G) * 32;         // first query token of this wave
  const int my_q = wq0 + lcol;                   // this lane's query token
  const int q_end = min(a.lq, tq0 + TQ);

  // Keys visible to some row of this workgroup.
  int n_kv = a.lk;
  if (a.causal) {
    const int64_t lim = a.q_off + q_end - a.k_off;  // keys j < lim are visible to the last row
    n_kv = static_cast<int>(lim <= 0 ? 0 : (lim < a.lk ? lim : a.lk));
  }
  const int n_tiles = (n_kv + kBK - 1) / kBK;

  // Q^T fragments (B operand): Q[my_q][lhalf*8 + 16*s .. +8]; rows past lq read zeros.
  frag qf[KS];
  {
    const uint16_t* qbase = a.q + head * a.q_hs + static_cast<int64_t>(wq0) * a.q_ss;
    const auto qr = make_rsrc(qbase, static_cast<int64_t>(a.lq - wq0) * a.q_ss * 2);
    const int32_t qoff = (lcol * static_cast<int32_t>(a.q_ss) + lhalf * 8) * 2;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = as_frag<frag>(buf_load16(qr, qoff + 32 * s));
  }

  f32x16 oacc[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[b][r] = 0.f;
  float m_run = kInitMax;  // reference max, log2 domain (scaled)
  float l_run = 0.f;       // this lane's partial row sum

  // ---- loader roles: waves 0-3 stage K, waves 4-7 stage V (transposed) ----
  const bool k_loader = wave < 4;
  const int lt = tid & 255;
  const uint16_t* kbase = a.k + kvh * a.k_hs;
  const uint16_t* vbase = a.v + kvh * a.v_hs;
  // V item of this thread: 4 consecutive keys x one 8-wide d chunk.
  const int v_rg = lt % (kBK / 4);
  const int v_dc = lt / (kBK / 4);
  const bool v_active = !k_loader && lt < V_ITEMS;
  // Byte offsets within a tile (tile base = row kv0).
  int32_t ld_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (k_loader) {
      const int c = lt + 256 * (i < K_LOADS ? i : 0);
      ld_off[i] = ((c / KCH) * static_cast<int32_t>(a.k_ss) + (c % KCH) * 8) * 2;
    } else {
      ld_off[i] = ((v_rg * 4 + i) * static_cast<int32_t>(a.v_ss) + v_dc * 8) * 2;
    }
  }
  const uint16_t* ld_base = k_loader ? kbase : vbase;
  const int64_t ld_ss = k_loader ? a.k_ss : a.v_ss;

  u32x4 stage[4];
  auto load_tile = [&](int t) {
    const int kv0 = t * kBK;
    const auto r = make_rsrc(ld_base + kv0 * ld_ss, static_cast<int64_t>(a.lk - kv0) * ld_ss * 2);
    if (k_loader) {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) stage[i] = buf_load16(r, ld_off[i]);
    } else if (v_active) {
#pragma unroll
      for (int i = 0; i < 4; ++i) stage[i] = buf_load16(r, ld_off[i]);
    }
  };
  auto store_tile = [&](int buf) {
    if (k_loader) {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int c = lt + 256 * i;
        const int row = c / KCH, ch = c % KCH;
        *reinterpret_cast<u32x4*>(&ks_lds[buf][row * KROW + ch * 8]) = stage[i];
      }
    } else if (v_active) {
      // stage[i] holds d = v_dc*8 .. +8 of key v_rg*4+i; write V^T rows d, keys v_rg*4..+4.
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        const int w = dd >> 1;
        u32x2 pk;
        if (dd & 1) {
          pk[0] = __builtin_amdgcn_perm(stage[1][w], stage[0][w], 0x07060302u);
          pk[1] = __builtin_amdgcn_perm(stage[3][w], stage[2][w], 0x07060302u);
        } else {
          pk[0] = __builtin_amdgcn_perm(stage[1][w], stage[0][w], 0x05040100u);
          pk[1] = __builtin_amdgcn_perm(stage[3][w], stage[2][w], 0x05040100u);
        }
        *reinterpret_cast<u32x2*>(&vt_lds[buf][(v_dc * 8 + dd) * kVtStride + v_rg * 4]) = pk;
      }
    }
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  // Q fragments and tile 0 are resident before the loop: the prefetch issued inside
  // the loop is then the only outstanding memory traffic during the MFMA section.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int krow0 = kperm(lcol);  // permuted K row fed by this lane (within a 32-block)
  const float c = a.scale_log2;
  // Causal limit of this lane relative to key 0 of the chunk: key j visible iff j <= qlim.
  const int64_t qlim64 = a.q_off + my_q - a.k_off;
  const int64_t wave_lim_first = a.q_off + wq0 - a.k_off;                  // first row of the wave
  const int64_t wave_lim_last = a.q_off + min(wq0 + 31, a.lq - 1) - a.k_off;  // last row

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);

    const int kv0 = t * kBK;
    // Skip tiles wholly in this wave's future (causal) -- other waves may need them.
    const bool wave_live = !a.causal || kv0 <= wave_lim_last;
    if (wave_live && wq0 < a.lq) {
      const bool need_mask = (kv0 + kBK > a.lk) || (a.causal && kv0 + kBK - 1 > wave_lim_first);

      // ---- S^T = K Q^T for two 32-key blocks ----
      f32x16 sacc[2];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[b][r] = 0.f;
      const uint16_t* kl = &ks_lds[buf][0];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(kl + (32 * b + krow0) * KROW + lhalf * 8 + 16 * s);
          sacc[b] = Ops::mma(as_frag<frag>(raw), qf[s], sacc[b]);
        }
      }

      // ---- mask (boundary tiles only), tile row max on raw scores ----
      if (need_mask) {
        // key kv0 + kl visible iff kl <= lim (kl = tile-local key index).
        int64_t lim64 = a.lk - 1 - kv0;
        if (a.causal) lim64 = min(lim64, qlim64 - kv0);
        const int lim = static_cast<int>(max(min(lim64, static_cast<int64_t>(kBK)), static_cast<int64_t>(-1))) - 8 * lhalf;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int j = r >> 2, i = r & 3;
            const int kl0 = 32 * b + 16 * (j >> 1) + 4 * (j & 1) + i;  // kl minus 8*lhalf
            sacc[b][r] = kl0 <= lim ? sacc[b][r] : -INFINITY;
          }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sacc[b][r]);
      tmax = max_xor32(tmax) * c;

      // ---- lazy rescale: move the reference max only when it grows by > 8 ----
      const bool grow = tmax > m_run + kRescaleThreshold;
      if (__any(grow)) {
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int b = 0; b < DB; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[b][r] *= alpha;
        m_run = m_new;
      }

      // ---- P = 2^(s*c - m) as 16-bit B operands, row-sum partial ----
      frag pf[4];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][r], c, -m_run));
          l_run += p[r];
        }
        pf[2 * b] = Ops::pack(p);
        pf[2 * b + 1] = Ops::pack(p + 8);
      }

      // ---- O^T += V^T P^T ----
      const uint16_t* vl = &vt_lds[buf][0];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int b = 0; b < DB; ++b) {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(vl + (32 * b + lcol) * kVtStride + 16 * s + 8 * lhalf);
          oacc[b] = Ops::mma(as_frag<frag>(raw), pf[s], oacc[b]);
        }
      }
    }

    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: normalise, LSE (natural log), optional merge with running partial ----
  if (my_q >= a.lq) return;
  const float l_tot = sum_xor32(l_run);
  const bool any = l_tot > 0.f;
  const float inv = any ? 1.f / l_tot : 0.f;
  const float lse_new = any ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  const int64_t row = static_cast<int64_t>(head) * a.lq + my_q;
  float* orow = a.o + row * D;
  if (!a.accumulate) {
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4 v = make_float4(oacc[b][4 * j] * inv, oacc[b][4 * j + 1] * inv, oacc[b][4 * j + 2] * inv,
                               oacc[b][4 * j + 3] * inv);
        *reinterpret_cast<float4*>(orow + 32 * b + 8 * j + 4 * lhalf) = v;
      }
    if (lhalf == 0) a.lse[row] = lse_new;
  } else {
    const float lse_old = a.lse[row];
    const float m = fmaxf(lse_old, lse_new);
    const bool m_ok = m != -INFINITY;
    const float w_old = m_ok ? __expf(lse_old - m) : 0.f;
    const float w_new = m_ok ? __expf(lse_new - m) : 0.f;
    const float den = w_old + w_new;
    const float rden = den > 0.f ? 1.f / den : 0.f;
    const float c_old = w_old * rden;
    const float c_new = w_new * rden * inv;
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4* p = reinterpret_cast<float4*>(orow + 32 * b + 8 * j + 4 * lhalf);
        const float4 old = *p;
        *p = make_float4(c_old * old.x + c_new * oacc[b][4 * j], c_old * old.y + c_new * oacc[b][4 * j + 1],
                         c_old * old.z + c_new * oacc[b][4 * j + 2], c_old * old.w + c_new * oacc[b][4 * j + 3]);
      }
    if (lhalf == 0) a.lse[row] = m_ok ? m + __logf(den) : -INFINITY;
  }
}

// ----------------------------------------------------------------------------------
// General kernel: one thread per (query row, head); fp32 math, K/V tiles in LDS.
// ----------------------------------------------------------------------------------
struct GenArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t q_hs, q_ss, k_hs, k_ss, v_hs, v_ss;
  float* o;
  float* lse;
  int32_t hq, rep, lq, lk, d;
  int64_t q_off, k_off;
  int32_t causal, accumulate;
  float scale;
};

constexpr int kGenRows = 64;
constexpr int kGenBK = 32;

template <int DT, int DMAX>
__global__ __launch_bounds__(kGenRows) void general_block_kernel(GenArgs a) {
  __shared__ float ks[kGenBK][DMAX];
  __shared__ float vs[kGenBK][DMAX];
  const int head = blockIdx.y;
  const int kvh = head / a.rep;
  const int row = blockIdx.x * kGenRows + threadIdx.x;
  const bool live = row < a.lq;
  const int d = a.d;
  float qv[DMAX], acc[DMAX];
  for (int i = 0; i < DMAX; ++i) {
    qv[i] = (live && i < d) ? load_elem<DT>(a.q, head * a.q_hs + static_cast<int64_t>(row) * a.q_ss + i) : 0.f;
    acc[i] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int64_t qpos = a.q_off + row;
  int n_kv = a.lk;
  if (a.causal) {
    const int last = min(a.lq, static_cast<int>(blockIdx.x + 1) * kGenRows) - 1;
    const int64_t lim = a.q_off + last + 1 - a.k_off;
    n_kv = static_cast<int>(lim <= 0 ? 0 : (lim < a.lk ? lim : a.lk));
  }
  for (int kv0 = 0; kv0 < n_kv; kv0 += kGenBK) {
    __syncthreads();
    for (int e = threadIdx.x; e < kGenBK * d; e += kGenRows) {
      const int r = e / d, c = e % d;
      const int kv = kv0 + r;
      ks[r][c] = kv < a.lk ? load_elem<DT>(a.k, kvh * a.k_hs + static_cast<int64_t>(kv) * a.k_ss + c) : 0.f;
      vs[r][c] = kv < a.lk ? load_elem<DT>(a.v, kvh * a.v_hs + static_cast<int64_t>(kv) * a.v_ss + c) : 0.f;
    }
    __syncthreads();
    if (!live) continue;
    const int nk = min(kGenBK, n_kv - kv0);
    for (int r = 0; r < nk; ++r) {
      const int64_t kpos = a.k_off + kv0 + r;
      if (a.causal && kpos > qpos) continue;
      float s = 0.f;
      for (int i = 0; i < DMAX; ++i)
        if (i < d) s += qv[i] * ks[r][i];
      s *= a.scale;
      const float m_new = fmaxf(m, s);
      const float alpha = __expf(m - m_new);  // m = -inf first time -> 0
      const float p = __expf(s - m_new);
      l = l * alpha + p;
      for (int i = 0; i < DMAX; ++i)
        if (i < d) acc[i] = acc[i] * alpha + p * vs[r][i];
      m = m_new;
    }
  }
  if (!live) return;
  const bool any = l > 0.f;
  const float inv = any ? 1.f / l : 0.f;
  const float lse_new = any ? m + __logf(l) : -INFINITY;
  const int64_t orow = static_cast<int64_t>(head) * a.lq + row;
  if (!a.accumulate) {
    for (int i = 0; i < d && i < DMAX; ++i) a.o[orow * d + i] = acc[i] * inv;
    a.lse[orow] = lse_new;
  } else {
    const float lse_old = a.lse[orow];
    const float mm = fmaxf(lse_old, lse_new);
    const bool ok = mm != -INFINITY;
    const float w_old = ok ? __expf(lse_old - mm) : 0.f;
    const float w_new = ok ? __expf(lse_new - mm) : 0.f;
    const float den = w_old + w_new;
    const float rden = den > 0.f ? 1.f / den : 0.f;
    for (int i = 0; i < d && i < DMAX; ++i)
      a.o[orow * d + i] = (w_old * a.o[orow * d + i] + w_new * acc[i] * inv) * rden;
    a.lse[orow] = ok ? mm + __logf(den) : -INFINITY;
  }
}

// ----------------------------------------------------------------------------------
// Host launcher
// ----------------------------------------------------------------------------------

template <int D, int DT>
static void launch_mfma(const BlockLaunch& L, hipStream_t stream) {
  BlockArgs a;
  a.q = static_cast<const uint16_t*>(L.q);
  a.k = static_cast<const uint16_t*>(L.k);
  a.v = static_cast<const uint16_t*>(L.v);
  a.q_hs = L.q_hs; a.q_ss = L.q_ss; a.k_hs = L.k_hs; a.k_ss = L.k_ss; a.v_hs = L.v_hs; a.v_ss = L.v_ss;
  a.o = L.o;
  a.lse = L.lse;
  a.hq = L.hq;
  a.hkv = L.hkv;
  a.rep = L.hq / L.hkv;
  a.lq = static_cast<int32_t>(L.lq);
  a.lk = static_cast<int32_t>(L.lk);
  a.q_off = L.q_off;
  a.k_off = L.k_off;
  a.causal = L.causal;
  a.accumulate = L.accumulate;
  a.scale_log2 = L.scale * kLog2e;
  int g = 1;
  for (int cand : {8, 4, 2}) {
    if (a.rep % cand == 0) { g = cand; break; }
  }
  const int tq = 32 * (kWaves / g);
  a.n_qtiles = static_cast<int32_t>(ceil_div(L.lq, tq));
  a.n_groups = L.hq / g;
  const dim3 grid(static_cast<unsigned>(a.n_qtiles * a.n_groups));
  switch (g) {
    case 8: flash_block_kernel<D, DT, 8><<<grid, kThreads, 0, stream>>>(a); break;
    case 4: flash_block_kernel<D, DT, 4><<<grid, kThreads, 0, stream>>>(a); break;
    case 2: flash_block_kernel<D, DT, 2><<<grid, kThreads, 0, stream>>>(a); break;
    default: flash_block_kernel<D, DT, 1><<<grid, kThreads, 0, stream>>>(a); break;
  }
}

template <int DT>
static void launch_general(const BlockLaunch& L, hipStream_t stream) {
  GenArgs a;
  a.q = L.q; a.k = L.k; a.v = L.v;
  a.q_hs = L.q_hs; a.q_ss = L.q_ss; a.k_hs = L.k_hs; a.k_ss = L.k_ss; a.v_hs = L.v_hs; a.v_ss = L.v_ss;
  a.o = L.o; a.lse = L.lse;
  a.hq = L.hq; a.rep = L.hq / L.hkv;
  a.lq = static_cast<int32_t>(L.lq); a.lk = static_cast<int32_t>(L.lk); a.d = L.d;
  a.q_off = L.q_off; a.k_off = L.k_off;
  a.causal = L.causal; a.accumulate = L.accumulate;
  a.scale = L.scale;
  const dim3 grid(static_cast<unsigned>(ceil_div(L.lq, kGenRows)), static_cast<unsigned>(L.hq));
  if (L.d <= 64) general_block_kernel<DT, 64><<<grid, kGenRows, 0, stream>>>(a);
  else if (L.d <= 128) general_block_kernel<DT, 128><<<grid, kGenRows, 0, stream>>>(a);
  else general_block_kernel<DT, 256><<<grid, kGenRows, 0, stream>>>(a);
}

// True when the matrix-core kernel handles this shape.
bool block_uses_mfma(int dtype, int d) {
  return (dtype == kBF16 || dtype == kF16) && (d == 64 || d == 128);
}

void launch_block_partial(const BlockLaunch& L, hipStream_t stream) {
  if (L.lq == 0) return;
  if (!L.force_general && block_uses_mfma(L.dtype, L.d)) {
    if (L.dtype == kBF16) {
      if (L.d == 128) launch_mfma<128, kBF16>(L, stream);
      else launch_mfma<64, kBF16>(L, stream);
    } else {
      if (L.d == 128) launch_mfma<128, kF16>(L, stream);
      else launch_mfma<64, kF16>(L, stream);
    }
  } else {
    switch (L.dtype) {
      case kF32: launch_general<kF32>(L, stream); break;
      case kBF16: launch_general<kBF16>(L, stream); break;
      case kF16: launch_general<kF16>(L, stream); break;
      default: throw Error(-6, "block_partial: dtype must be BF16, F16 or F32");
    }
  }
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
