// Flash-style block kernel for one ring step: (query chunk, KV chunk) -> (o, lse) fp32.
//
// Replaces process_kv_block's op sequence (ring.rs:201-370: QK^T*scale, causal
// -inf mask on global positions, amax / exp / sum, PV, rescale-merge) and the
// positioned partial / merge wrappers (ring.rs:538-603).  The online softmax is the
// same recurrence; scores never leave registers.
//
// Matrix-core path (bf16 / fp16, head_dim 128 and every other multiple of 8 below it
// zero-padded to 128), gfx950 MFMA 32x32x16:
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
//   * flash_block_pingpong_kernel / flash_ring_kernel: tiles of 128 keys, asynchronous
//     global->LDS loads and two wave groups that alternate MFMA and softmax phases.
//   * Causal: tiles wholly in a wave's future are skipped, tiles wholly visible are
//     unmasked, only tiles straddling the diagonal (or the kv tail) are masked.  The
//     visible keys of a row are a prefix of the chunk: j <= q_off + i - k_off for
//     contiguous positions, j < q_lim[i] for explicit positions (Striped / ZigZag,
//     ring.rs:1024-1046, with non-decreasing key positions; a key list in any other
//     order is read through sorted-row copies, see positions.hip).
//
// fp32 matrix-core path (mfma_f32_block_kernel, head_dim a multiple of 4 up to 128):
// v_mfma_f32_32x32x2f32 for both products, 4 waves over 128 query rows of one head.
//
// General path (any other shape, head_dim <= 256): one thread per (query row, head),
// K/V tiles staged in LDS as fp32.
#include <algorithm>
#include <cstdlib>
#include <vector>

#include "kernels.hpp"
#include "lds_dma.hpp"

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
  void* fin_out;           // final mode when non-null (see BlockLaunch)
  int32_t fin_dtype;
  int64_t fin_hs, fin_ss;
  float* fin_lse;
  int64_t fin_lse_hs;
  const int32_t* q_lim;    // positions mode when non-null (causal): row i sees keys [0, q_lim[i])
  int32_t d;               // head dim of the views and the state (the head-dim-128 kernel: <= 128,
                           // a multiple of 8; columns d .. 127 are zero padding in LDS and registers)
  // positions mode, keys in any order: K / V come from the sorted-row copies when *kv_sel
  const int32_t* kv_sel;
  const uint16_t* k_alt;
  const uint16_t* v_alt;
  int64_t alt_hs, alt_ss;
};

// Up to kMaxGroup independent (query chunk, KV chunk) pairs with the same head layout in
// one launch of the head-dim-128 kernel (one ring step of a replay).  Workgroups are
// numbered head group first, then pair, then query tile (heaviest first): logical id
// hg * qt_begin[n] + qt_begin[p] + j is query tile n_qtiles_p - 1 - j of pair p.
constexpr int kMaxGroup = 8;
struct BlockGroup {
  BlockArgs a[kMaxGroup];
  int32_t n;
  int32_t qt_begin[kMaxGroup + 1];
};
static_assert(sizeof(BlockGroup) <= 4096, "kernel arguments are limited to 4 KiB");

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr float kInitMax = -1.0e30f;
constexpr float kGrowSum = 256.0f;  // 2^8: largest partial row sum kept without a max pass

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

// Causal visibility of a workgroup of the matrix-core kernels: key j of the chunk is
// visible to a query row iff j <= that row's limit.  n_kv = keys visible to some row of
// the workgroup; lane = this lane's row limit; wave_first / wave_last = the smallest /
// largest limit over the wave's rows inside the chunk.  Contiguous positions give
// limit = q_off + row - k_off (monotone in the row); explicit positions give
// limit = q_lim[row] - 1, reduced over the wave and, through `red` (one barrier that
// every thread of the workgroup reaches), over the workgroup.
struct RowLimits {
  int n_kv;
  int64_t lane, wave_first, wave_last;
};
template <bool POS>
__device__ __forceinline__ RowLimits row_limits(const BlockArgs& a, int q_end, int wq0, int my_q, int wave,
                                                int lane, int* red) {
  RowLimits r;
  r.n_kv = a.lk;
  if constexpr (!POS) {
    r.lane = a.q_off + my_q - a.k_off;
    r.wave_first = a.q_off + wq0 - a.k_off;
    r.wave_last = a.q_off + min(wq0 + 31, a.lq - 1) - a.k_off;
    if (a.causal) {
      const int64_t lim = a.q_off + q_end - a.k_off;  // keys j < lim are visible to the last row
      r.n_kv = static_cast<int>(lim <= 0 ? 0 : (lim < a.lk ? lim : a.lk));
    }
    return r;
  }
  const bool valid = my_q < a.lq;
  const int mine = valid ? min(max(a.q_lim[my_q], 0), a.lk) : 0;
  int lo = valid ? mine : a.lk, hi = mine;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    lo = min(lo, __shfl_xor(lo, off));
    hi = max(hi, __shfl_xor(hi, off));
  }
  if (lane == 0) red[wave] = hi;
  __syncthreads();
  int wg = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) wg = max(wg, red[w]);
  r.lane = mine - 1;
  r.wave_first = lo - 1;
  r.wave_last = hi - 1;
  if (a.causal) r.n_kv = wg;
  return r;
}

// 4 fp32 values as 16-bit `dtype` (bf16 or f16), packed in element order.
__device__ __forceinline__ u32x2 pack4(int dtype, float x0, float x1, float x2, float x3) {
  u32x2 w;
  if (dtype == kBF16) {
    w[0] = f32x2_to_bf16x2_bits(x0, x1);
    w[1] = f32x2_to_bf16x2_bits(x2, x3);
  } else {
    w[0] = static_cast<uint32_t>(f32_to_f16_bits(x0)) | (static_cast<uint32_t>(f32_to_f16_bits(x1)) << 16);
    w[1] = static_cast<uint32_t>(f32_to_f16_bits(x2)) | (static_cast<uint32_t>(f32_to_f16_bits(x3)) << 16);
  }
  return w;
}

// Stores 4 consecutive fp32 values as `dtype` at element offset `off` of `base`.
__device__ __forceinline__ void store4(void* base, int dtype, int64_t off, float x0, float x1, float x2, float x3) {
  if (dtype == kF32) {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + off) = make_float4(x0, x1, x2, x3);
  } else {
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(base) + off) = pack4(dtype, x0, x1, x2, x3);
  }
}

// Epilogue of one (head, query row): normalise O, LSE in natural log; in accumulate
// mode merge with the running fp32 partial in (o, lse) (the rm = lse, rs = 1 re-entry
// of ring.rs:585-587 in closed form); write either the fp32 state or, in final mode,
// the output rows in the query dtype.  Lanes l and l + 32 hold the two interleaved
// 4-wide d slices of each 8-wide group.
template <int D>
__device__ __forceinline__ void write_row(const BlockArgs& a, int head, int my_q, int lhalf,
                                          const f32x16 (&oacc)[D / 32], float m_run, float l_tot, int dn = D) {
  constexpr int DB = D / 32;
  const bool any = l_tot > 0.f;
  const float inv = any ? 1.f / l_tot : 0.f;
  const float lse_new = any ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  const int64_t row = static_cast<int64_t>(head) * a.lq + my_q;
  // the running fp32 state (null in a fused ring, which writes final rows only)
  float* orow = a.o != nullptr ? a.o + row * dn : nullptr;
  float c_old = 0.f, c_new = inv, lse_out = lse_new;
  if (a.accumulate) {
    const float lse_old = a.lse[row];
    const float m = fmaxf(lse_old, lse_new);
    const bool m_ok = m != -INFINITY;
    const float w_old = m_ok ? __expf(lse_old - m) : 0.f;
    const float w_new = m_ok ? __expf(lse_new - m) : 0.f;
    const float den = w_old + w_new;
    const float rden = den > 0.f ? 1.f / den : 0.f;
    c_old = w_old * rden;
    c_new = w_new * rden * inv;
    lse_out = m_ok ? m + __logf(den) : -INFINITY;
  }
  const int64_t fin_row = head * a.fin_hs + static_cast<int64_t>(my_q) * a.fin_ss;
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int dcol = 32 * b + 8 * j + 4 * lhalf;
      if (dcol >= dn) continue;  // zero-padded columns
      float x0 = c_new * oacc[b][4 * j], x1 = c_new * oacc[b][4 * j + 1];
      float x2 = c_new * oacc[b][4 * j + 2], x3 = c_new * oacc[b][4 * j + 3];
      if (a.accumulate) {
        const float4 old = *reinterpret_cast<const float4*>(orow + dcol);
        x0 += c_old * old.x; x1 += c_old * old.y; x2 += c_old * old.z; x3 += c_old * old.w;
      }
      if (a.fin_out) store4(a.fin_out, a.fin_dtype, fin_row + dcol, x0, x1, x2, x3);
      else *reinterpret_cast<float4*>(orow + dcol) = make_float4(x0, x1, x2, x3);
    }
  if (lhalf == 0) {
    if (a.fin_out) {
      if (a.fin_lse) a.fin_lse[head * a.fin_lse_hs + my_q] = lse_out;
    } else {
      a.lse[row] = lse_out;
    }
  }
}

// Final-mode epilogue of one (head, query row) of a fused ring: normalised output row
// in `dtype` at element offset `off` of `out`, natural-log LSE to *lse (if non-null);
// lanes l and l + 32 hold the two interleaved 4-wide d slices of each 8-wide group.
template <int D>
__device__ __forceinline__ void write_final_row(void* out, int dtype, int64_t off, float* lse, int lhalf,
                                                const f32x16 (&oacc)[D / 32], float m_run, float l_tot, int dn) {
  constexpr int DB = D / 32;
  const bool any = l_tot > 0.f;
  const float inv = any ? 1.f / l_tot : 0.f;
  // 16-bit rows whose starts are 16-byte aligned across the wave: lanes l and l + 32 hold
  // the two 4-wide halves of each 8-wide group, so swapping groups (j, j + 1) with
  // v_permlane32_swap hands each lane one whole group, stored as 16 bytes (half the store
  // instructions of 8-byte stores).  Lanes l and l + 32 share their row, so both are
  // active or neither.  The fused schedule's launcher admits only 16-byte aligned
  // outputs; the 8-byte path below is the fallback for any other caller.
  const bool st16 = dtype != kF32 && __all(((reinterpret_cast<uintptr_t>(out) + static_cast<uintptr_t>(off) * 2) & 15) == 0);
  if (st16) {
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        if (32 * b + 8 * j >= dn) continue;  // zero-padded columns
        const u32x2 lo = pack4(dtype, inv * oacc[b][4 * j], inv * oacc[b][4 * j + 1], inv * oacc[b][4 * j + 2],
                               inv * oacc[b][4 * j + 3]);
        const u32x2 hi = pack4(dtype, inv * oacc[b][4 * j + 4], inv * oacc[b][4 * j + 5], inv * oacc[b][4 * j + 6],
                               inv * oacc[b][4 * j + 7]);
        u32x4 w;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto r = __builtin_amdgcn_permlane32_swap(hi[k], lo[k], false, false);
          w[k] = r[0];
          w[2 + k] = r[1];
        }
        const int dcol = 32 * b + 8 * (j + 1 - lhalf);
        if (dcol < dn) *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + off + dcol) = w;
      }
  } else {
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int dcol = 32 * b + 8 * j + 4 * lhalf;
        if (dcol >= dn) continue;  // zero-padded columns
        store4(out, dtype, off + dcol, inv * oacc[b][4 * j], inv * oacc[b][4 * j + 1], inv * oacc[b][4 * j + 2],
               inv * oacc[b][4 * j + 3]);
      }
  }
  if (lhalf == 0 && lse != nullptr) *lse = any ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
}

// ----------------------------------------------------------------------------------
// Head-dim-128 kernel: asynchronous global->LDS tiles, two wave groups in ping-pong.
//
// 8 waves, one query head and 32 query tokens per wave, S^T = K Q^T with K rows in
// kperm order, P^T straight from the S^T accumulators.
//
// Tiles.  The K and V tiles of 128 keys reach LDS without passing through registers:
// buffer_load_dwordx4 ... lds writes 1 KiB per wave instruction (4 rows of 128
// dims).  For LDS chunk p of row r the DMA fetches global chunk p ^ swz(r): K rows
// use swz = r & 15, V rows 4 * (r & 3), which makes the fragment reads bank-conflict
// free.  K fragments (A of S^T) are ds_read_b128; V^T fragments (A of O^T = V^T P^T)
// come from row-major V through ds_read_b64_tr_b16, two reads giving one lane the 8
// keys of its head-dim column.  K has a ring of two 32 KiB buffers and V a ring of
// three (160 KiB of LDS, all of it; V's third buffer gives its loads a super-step more
// slack).  The kernel also compiles for 64-key tiles with rings of three; 128 keys
// halve the per-tile barriers, DMA issue and softmax bookkeeping and measured 5% faster.
// The half-width instantiation (head dims up to 64) keeps 64 dims per LDS row: 8 rows
// per DMA instruction, swizzles K (r >> 1) & 7 and V 4 ((r >> 1) & 1), 16 KiB tiles
// (80 KiB of LDS; against 128-dim rows with a zero half, +2.6% on a 32k Qwen2-0.5B
// ring and +4-6% at 8k; a third K buffer measured 2% slower).
//
// Ping-pong.  The work of a tile is split in two phases per wave -- M: the MFMA phase
// (O^T += V^T P^T of the previous tile, then S^T = K Q^T of this tile: 64 MFMAs fed by
// 96 LDS reads) and X: the softmax phase of that tile on the VALU -- and the two waves
// that share a SIMD (waves w and w + 4; the pairing is read from HW_ID) run them out of
// phase: in super-step u the lead group runs M(u) then X(u), the other group X(u-1)
// then M(u), so while one issues its MFMAs the other's exponentials run beside them.
// The only barrier of a super-step is the one that publishes its K/V tiles; the two
// orders keep the phases apart between barriers (a barrier between the phases as well
// measured 1.5% slower: it drains the matrix core at every phase change).  The M phase
// runs at wave priority 1, so its MFMAs issue first and the VALU stream fills the gaps.
//
// Tile t's K is read in super-step t, its V in super-step t + 1 (by the PV product of
// M(t + 1)).  With NBK and NBV buffers per ring, in super-step u each wave issues its
// DMA share of K_{u+NBK-1} and V_{u+NBV-2} (into buffers freed by the previous
// super-step's closing barrier; the lead group issues after its first barrier, so its
// MFMA phase starts at once), and at its end waits for K_{u+1} and V_u.
// ----------------------------------------------------------------------------------
constexpr int kBK3 = 128;  // keys per K/V tile of the head-dim-128 kernel
constexpr int kD3 = 128;

// Empty asm that uses x: keeps the code producing x on this side of the next barrier
// (the compiler may otherwise move register-only work across s_barrier).
template <typename T>
__device__ __forceinline__ void pin(const T& x) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only parses device code; its asm has no "v" registers
  asm volatile("" : : "v"(x));
#else
  (void)x;
#endif
}

__device__ __forceinline__ int simd_id() {
  int r;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID, 4, 2)" : "=s"(r));
  return r;
}

// Fused single-GPU ring replay (vanilla positions): every target domain's ring in one
// launch.  A workgroup owns one query tile of one target domain t and folds that
// target's sources in ring order -- t, t-1, ..., t-N+1 (mod N), the order in which
// ring_attention receives them (ring.rs:1208-1311, mock.rs:143-149) -- skipping keys
// wholly in its future (ring.rs:222-228); the running (m, l, O) stays in registers
// across sources and the last tile writes the output rows and the LSE.  With the
// domains' chunks stored in order, the keys of sources t-1, t-2, ..., 0 are the rows
// [0, off_t) of the K/V views read backwards, and (without causal masking) those of
// t-1 wrapping round to t+1 are then [off_t + len_t, S) read backwards: the 128-key
// tiles after the local source are taken from the top of that range down, so each
// source is folded whole, after its successor in the ring, and a tile's rows follow
// from its index alone.  Workgroups are numbered tile-rank-major over head groups, so
// blockIdx b goes to XCD b mod 8 with the heavier (later) query tiles first on every XCD.
struct RingPlan {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_hs, q_ss, k_hs, k_ss, v_hs, v_ss;  // element strides (whole-sequence views)
  void* out;
  int64_t out_hs, out_ss;
  float* lse;                                   // [Hq, S] rows, or null
  int64_t lse_hs;
  int32_t dtype;                                // query / output dtype
  int32_t d;                                    // head dim (<= 128, multiple of 8; zero-padded to 128)
  int32_t hq, hkv, rep, n_groups, n, causal;
  float scale_log2;
  int32_t off[kMaxDomains], len[kMaxDomains];   // rows (= global positions) of each domain
  int32_t qt_begin[kMaxDomains + 1];            // query tiles of slot s (domain n-1-s)
  uint32_t* trace;                              // trace records (the TRACE kernels only)
  int32_t trace_stride;                         // 32-bit words per record
};
static_assert(sizeof(RingPlan) <= 4096, "kernel arguments are limited to 4 KiB");

// Trace record of one workgroup of a traced fused ring (hcp_ring_trace_attach), 32-bit
// words: [0, 2) s_memrealtime at entry (100 MHz), [2, 4) at the end, [4, 6) / [6, 8)
// s_memtime (shader clock) at entry / end, 8 HW_ID, 9 XCC_ID, 10 target domain |
// head group << 16, 11 query tile, 12 key tiles folded, [13, 16) zero, then for ring
// position s (0 = the local chunk, s = source (t - s) mod N) the s_memrealtime at which
// the workgroup moved past that source, two words each (0: never visited).
constexpr int kTraceHeaderWords = 16;

template <int DT, int G, bool POS, int BK, bool RING, class P, bool TRACE = false, int DWN = kD3>
__device__ __forceinline__ void pingpong_body(const P& plan) {
  using Ops = MfmaOps<DT>;
  using frag = typename Ops::frag;
  // DW = DWN: the head dims a wave folds and the width of a K / V row in LDS (head dims
  // below it zero-padded by the DMA).  DWN = 64 (head dims up to 64) runs the same loop
  // on 128-byte LDS rows: half the LDS, half the DMA instructions, its own swizzles.
  static_assert(DWN == kD3 || DWN == kD3 / 2, "dims folded: 128 or 64");
  constexpr int DW = DWN;
  static_assert(kWaves % G == 0, "heads per group must divide the waves");
  constexpr int TB = kWaves / G;
  constexpr int TQ = 32 * TB;
  constexpr int KS = DW / 16;
  constexpr int DB = DW / 32;
  // PW: bytes of a K / V row in LDS, the dims a wave folds (256 for 128 dims, 128 for
  // the half-width kernel); CPR 16-byte chunks per row, RPI rows per 1 KiB DMA.
  constexpr int PW = DW * 2;
  constexpr int CPR = PW / 16;
  constexpr int RPI = 1024 / PW;
  constexpr int kDmaPerWave = BK / RPI / kWaves;  // 1 KiB DMA instructions per wave per tile (K or V)
  constexpr int kTile = BK * PW;                 // bytes of one K or V tile
  constexpr int NKB = BK / 32;                   // 32-key blocks of S^T per tile
  constexpr int NPS = BK / 16;                   // 16-key steps of the PV product per tile
  // LDS buffers per ring: 3 + 3 tiles of 64 keys (96 KiB); 2 K + 3 V tiles of 128 keys
  // (160 KiB at 128 dims, 80 KiB at 64; two V buffers measured 0.4% slower).
  constexpr int NBK = BK == 64 ? 3 : 2;
  constexpr int NBV = 3;
  __shared__ __attribute__((aligned(1024))) uint16_t k_lds[NBK * BK * PW / 2];
  __shared__ __attribute__((aligned(1024))) uint16_t v_lds[NBV * BK * PW / 2];
  // Two small reduction arrays live at the start of the last V buffer, which the DMA
  // first writes in super-step 1, after every read of them.
  int* const lim_red = reinterpret_cast<int*>(v_lds + (NBV - 1) * BK * PW / 2);
  int* const simd_of = lim_red + kWaves;

  [[maybe_unused]] uint64_t trace_t0 = 0, trace_c0 = 0;
  if constexpr (TRACE) {
    trace_t0 = __builtin_amdgcn_s_memrealtime();
    trace_c0 = __builtin_amdgcn_s_memtime();
  }
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lcol = lane & 31;
  const int lhalf = lane >> 5;

  // ---- work item: head group, query tile, and the views it reads ----
  int hg, qt, t_dom = 0;
  const BlockArgs* ap = nullptr;  // block mode: the block of this workgroup
  const uint16_t *qv, *kv, *vv;
  int64_t q_hs, q_ss, k_hs, k_ss, v_hs, v_ss;
  int lq, rep, causal, dn;
  float c;
  if constexpr (RING) {
    const int logical = blockIdx.x;
    hg = logical % plan.n_groups;
    const int rank = logical / plan.n_groups;
    int slot = 0;
    while (slot + 1 < plan.n && rank >= plan.qt_begin[slot + 1]) ++slot;
    t_dom = plan.n - 1 - slot;
    qt = plan.qt_begin[slot + 1] - 1 - rank;  // a domain's last (heaviest) tile first
    qv = plan.q + static_cast<int64_t>(plan.off[t_dom]) * plan.q_ss;
    kv = plan.k; vv = plan.v;
    q_hs = plan.q_hs; q_ss = plan.q_ss; k_hs = plan.k_hs; k_ss = plan.k_ss; v_hs = plan.v_hs; v_ss = plan.v_ss;
    lq = plan.len[t_dom];
    rep = plan.rep;
    causal = plan.causal;
    c = plan.scale_log2;
    dn = plan.d;
  } else {
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int per_hg = plan.qt_begin[plan.n];
    hg = logical / per_hg;
    const int rem = logical - hg * per_hg;
    int pi = 0;
    while (pi + 1 < plan.n && rem >= plan.qt_begin[pi + 1]) ++pi;
    ap = &plan.a[pi];
    qt = ap->n_qtiles - 1 - (rem - plan.qt_begin[pi]);
    qv = ap->q; kv = ap->k; vv = ap->v;
    q_hs = ap->q_hs; q_ss = ap->q_ss; k_hs = ap->k_hs; k_ss = ap->k_ss; v_hs = ap->v_hs; v_ss = ap->v_ss;
    if constexpr (POS) {
      // a key list found out of order: its sorted-row copies (one scalar load per workgroup)
      if (ap->kv_sel != nullptr && __builtin_amdgcn_readfirstlane(*ap->kv_sel) != 0) {
        kv = ap->k_alt; vv = ap->v_alt;
        k_hs = v_hs = ap->alt_hs;
        k_ss = v_ss = ap->alt_ss;
      }
    }
    lq = ap->lq;
    rep = ap->rep;
    causal = ap->causal;
    c = ap->scale_log2;
    dn = ap->d;
  }

  const int head = hg * G + (wave % G);  // this wave's query head
  const int kvh = (hg * G) / rep;          // the KV head whose rows the tiles hold
  const int tq0 = qt * TQ;
  const int wq0 = tq0 + (wave / G) * 32;
  const int my_q = wq0 + lcol;
  const int q_end = min(lq, tq0 + TQ);

  if (lane == 0) simd_of[wave] = simd_id();
  RowLimits rl;
  if constexpr (RING) {
    rl.n_kv = 0;
    rl.lane = rl.wave_first = rl.wave_last = 0;
  } else {
    rl = row_limits<POS>(*ap, q_end, wq0, my_q, wave, lane, lim_red);
  }

  // ---- key tiles ----
  // Tiles 0 .. nt0-1 cover the rows [b0, e0) of the local source (the block's chunk), in
  // order; in a fused ring, tiles nt0 .. nt0+na-1 then walk [0, off_t) from the top
  // down and, without causal masking, the rest walk [off_t + len_t, S) the same way (the
  // lowest tile of each range may be partial).  Key row r of the K/V views lies
  // r + kdelta positions after query row 0 of the workgroup's block.
  int b0, e0, na = 0, nb = 0, top_b = 0, low_b = 0;
  int64_t kdelta;
  if constexpr (RING) {
    const int off_t = plan.off[t_dom];
    b0 = off_t;
    e0 = off_t + (causal ? q_end : lq);
    na = (off_t + BK - 1) / BK;
    if (!causal) {
      low_b = off_t + lq;
      top_b = plan.off[plan.n - 1] + plan.len[plan.n - 1];
      nb = (top_b - low_b + BK - 1) / BK;
    }
    kdelta = -static_cast<int64_t>(off_t);
  } else {
    b0 = 0;
    e0 = rl.n_kv;
    kdelta = ap->k_off - ap->q_off;
  }
  const int nt0 = (e0 - b0 + BK - 1) / BK;
  const int n_tiles = nt0 + na + nb;
  // rows [kr, ke) of tile t (the keys visible to some row of the workgroup)
  auto tile_rows = [&](int t, int& kr, int& ke) __attribute__((always_inline)) {
    if (!RING || t < nt0) {
      kr = b0 + t * BK;
      ke = e0;
    } else if (t < nt0 + na) {
      ke = b0 - (t - nt0) * BK;
      kr = max(ke - BK, 0);
    } else {
      ke = top_b - (t - nt0 - na) * BK;
      kr = max(ke - BK, low_b);
    }
  };

  // Swizzles (16-byte chunk index XOR, per row) that make the fragment reads bank-
  // conflict free: 256-byte rows K r & 15, V 4 (r & 3); 128-byte rows K (r >> 1) & 7,
  // V 4 ((r >> 1) & 1) (the row's parity already spreads rows over the two bank halves).
  auto swz_k = [](int r) __attribute__((always_inline)) { return PW == 256 ? (r & 15) : ((r >> 1) & 7); };
  auto swz_v = [](int r) __attribute__((always_inline)) { return PW == 256 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); };
  // ---- DMA set-up: wave w fills rows BK/8 w .. BK/8 w + BK/8 - 1 of every K and V tile ----
  const uint16_t* kbase = kv + kvh * k_hs;
  const uint16_t* vbase = vv + kvh * v_hs;
  const uint32_t k_lds0 = lds_offset(k_lds) + wave * (kDmaPerWave * 1024);
  const uint32_t v_lds0 = lds_offset(v_lds) + wave * (kDmaPerWave * 1024);
  uint32_t k_voff[kDmaPerWave], v_voff[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int r = (wave * kDmaPerWave + j) * RPI + lane / CPR;
    const int p = lane % CPR;
    // global chunk p ^ swz(r) of row r; chunks past the head dim get an offset beyond any
    // tile's records (tiles stay below 2^31 bytes), so the DMA writes zeros there
    const int kc = p ^ swz_k(r), vc = p ^ swz_v(r);
    k_voff[j] = kc * 8 < dn ? static_cast<uint32_t>(r * k_ss * 2 + (kc << 4)) : 0x80000000u;
    v_voff[j] = vc * 8 < dn ? static_cast<uint32_t>(r * v_ss * 2 + (vc << 4)) : 0x80000000u;
  }
  // Buffer descriptors of a tile's rows [kr, ke): a few scalar instructions per tile
  // (every wave of the CU shares one scalar unit, and the DMA issue sits on the
  // critical path of both wave groups).  The launcher keeps a tile's bytes (BK rows)
  // below 2^31, so row offsets and sizes are 32-bit products.
  const uint64_t k_addr = reinterpret_cast<uint64_t>(kbase), v_addr = reinterpret_cast<uint64_t>(vbase);
  const uint32_t k_rb = static_cast<uint32_t>(k_ss) * 2u, v_rb = static_cast<uint32_t>(v_ss) * 2u;
  auto tile_srd = [](uint64_t base, uint32_t rb, int kr, int ke) __attribute__((always_inline)) {
    const uint64_t at = base + static_cast<uint64_t>(static_cast<uint32_t>(kr)) * rb;
    u32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(at));
    r[1] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(at >> 32) & 0xffffu);
    // the tile's own rows only: at most BK of them (below 2^31 bytes), however long the
    // rest of the range, so the records never wrap and 0x80000000 stays out of range
    r[2] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(min(ke - kr, BK)) * rb);
    r[3] = 0x00020000u;
    return r;
  };
  auto dma_k = [&](int kr, int ke, int buf) __attribute__((always_inline)) {
    const u32x4 sr = tile_srd(k_addr, k_rb, kr, ke);
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) dma16(sr, k_voff[j], k_lds0 + buf * kTile + j * 1024);
  };
  auto dma_v = [&](int kr, int ke, int buf) __attribute__((always_inline)) {
    const u32x4 sr = tile_srd(v_addr, v_rb, kr, ke);
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) dma16(sr, v_voff[j], v_lds0 + buf * kTile + j * 1024);
  };
  auto issue_k = [&](int t, int buf) __attribute__((always_inline)) {
    int kr, ke;
    tile_rows(t, kr, ke);
    dma_k(kr, ke, buf);
  };
  auto issue_v = [&](int t, int buf) __attribute__((always_inline)) {
    int kr, ke;
    tile_rows(t, kr, ke);
    dma_v(kr, ke, buf);
  };

  // prologue: K_0 .. K_{NBK-2}, V_0 .. V_{NBV-3}
#pragma unroll
  for (int t = 0; t < NBK - 1; ++t)
    if (t < n_tiles) issue_k(t, t);
#pragma unroll
  for (int t = 0; t < NBV - 2; ++t)
    if (t < n_tiles) issue_v(t, t);

  frag qf[KS];
  {
    const uint16_t* qbase = qv + head * q_hs + static_cast<int64_t>(wq0) * q_ss;
    // The range covers the wave's own rows (at most 32) and ends at the last one's
    // element dn - 1: the fragment loads cover DW dims of every row, so with dn < DW a
    // range of whole rows would let the last row of the last head read up to
    // 2 (DW - dn) bytes past the end of Q; and a range from here to the chunk's end
    // could pass the descriptor's 2 GiB limit on long chunks.
    const int q_rows = min(lq - wq0, 32);
    const auto qr = make_rsrc(qbase, q_rows > 0 ? (static_cast<int64_t>(q_rows - 1) * q_ss + dn) * 2 : 0);
    const int32_t qoff = (lcol * static_cast<int32_t>(q_ss) + lhalf * 8) * 2;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 x = buf_load16(qr, qoff + 32 * s);
      // head-dim columns 16s + 8*lhalf .. +7; past the head dim: zero padding
      qf[s] = as_frag<frag>(16 * s + 8 * lhalf < dn ? x : u32x4{0u, 0u, 0u, 0u});
    }
  }

  const int krow = kperm(lcol);
  // K fragment s of a lane sits at k_rd0 ^ (s << 5) in a tile: (lhalf + 2s) ^ (krow & 15)
  // changes only bits 1-3 of the 16-byte column index with s, and tile bases are
  // 1 KiB-aligned, so the XOR commutes with adding the base.
  const uint32_t k_rd0 = krow * PW + ((lhalf ^ swz_k(krow)) << 4);
  const int g16 = lane >> 4, sl = lane & 15;
  uint32_t v_rd[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) {  // 32-dim block of the LDS row
    // row 8 (g16 >> 1) + (sl >> 2) of a 16-key step (and 4 rows on), so swz_v of that
    // row is 4 (sl >> 2) for 256-byte rows and 4 ((sl >> 3) & 1) for 128-byte ones
    const int vs = PW == 256 ? (sl >> 2) : ((sl >> 3) & 1);
    v_rd[b] = (8 * (g16 >> 1) + (sl >> 2)) * PW + ((4 * (b ^ vs) + 2 * (g16 & 1) + ((sl & 3) >> 1)) << 4) + 8 * (sl & 1);
  }
  const uint32_t k_lds_off = lds_offset(k_lds);
  const char* v_lds_c = reinterpret_cast<const char*>(v_lds);

  f32x16 oacc[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[b][r] = 0.f;
  f32x16 sacc[NKB];
  frag pf[NPS];
  float m_run = kInitMax;
  float l_run = 0.f;

  const int64_t qlim64 = rl.lane;
  const int64_t wave_lim_first = rl.wave_first;
  const int64_t wave_lim_last = rl.wave_last;

  __builtin_amdgcn_s_waitcnt(0);  // Q fragments and the first tiles resident
  __syncthreads();
  bool lead = true;
  {
    const int mine = simd_of[wave];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) lead = lead && !(w < wave && simd_of[w] == mine);
  }
  lead = __builtin_amdgcn_readfirstlane(static_cast<int>(lead)) != 0;

  // Last tile with a key visible to some row of this wave (-1: none); the tiles a wave
  // computes are 0 .. last_live, so both phases of the steady-state loop below run
  // unconditionally.  In a fused ring every tile up to the last is computed: tiles
  // past a wave's rows occur only on the local source's diagonal and are masked.
  int last_live = n_tiles - 1;
  if (wq0 >= lq) last_live = -1;
  else if (!RING && causal) last_live = wave_lim_last < 0 ? -1 : static_cast<int>(min(static_cast<int64_t>(last_live), wave_lim_last / BK));
  auto live = [&](int t) __attribute__((always_inline)) { return t >= 0 && t <= last_live; };

  // ---- M phase pieces: O^T += V^T P^T of the previous tile (V buffer vb), S^T = K Q^T of this tile (K buffer kb) ----
  auto pv_part = [&](int vb) __attribute__((always_inline)) {
    const char* vl = v_lds_c + vb * kTile;
#pragma unroll
    for (int s = 0; s < NPS; ++s) {
#pragma unroll
      for (int b = 0; b < DB; ++b) {
        const char* p0 = vl + v_rd[b] + s * 16 * PW;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p0));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p0 + 4 * PW));
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        oacc[b] = Ops::mma(as_frag<frag>(u32x4{lo2[0], lo2[1], hi2[0], hi2[1]}), pf[s], oacc[b]);
      }
    }
  };
  auto s_part = [&](int kb) __attribute__((always_inline)) {
    const uint32_t kl = k_lds_off + kb * kTile + k_rd0;
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[b][r] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t ks = kl ^ static_cast<uint32_t>(s << 5);
#pragma unroll
      for (int b = 0; b < NKB; ++b) {
        const frag kf = as_frag<frag>(*reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
            static_cast<uintptr_t>(ks + b * 32 * PW)));
        sacc[b] = Ops::mma(kf, qf[s], sacc[b]);
      }
    }
  };
  // Steady state: both products in one block, LDS reads running ahead of the MFMAs that
  // consume them (8 Vt reads, then 2 per PV MFMA, then the K reads one per MFMA).
  auto m_full = [&](int kb, int vb) __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(1);  // the MFMA stream first; the other wave's VALU fills in
    pv_part(vb);
    s_part(kb);
    constexpr int A = 8;            // Vt reads issued before the first MFMA (4 KiB per wave in flight)
    constexpr int NPV = NPS * DB;   // PV MFMAs (2 Vt reads each)
    constexpr int NS = NKB * KS;    // S MFMAs (1 K read each)
    __builtin_amdgcn_sched_group_barrier(0x100, A, 0);
#pragma unroll
    for (int i = 0; i < NPV - A / 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, A / 2, 0);
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int b = 0; b < DB; ++b) pin(oacc[b]);
#pragma unroll
    for (int b = 0; b < NKB; ++b) pin(sacc[b]);
  };

  // ---- X phase: mask, P = 2^(s*c - m) against the running reference max m, lazy
  // rescale.  The tile max (32 v_max3 and a cross-lane step per tile) is an eighth of
  // the phase's VALU instructions, and VALU issue (about one instruction per 7 cycles
  // per SIMD while the other wave's MFMAs run) bounds these kernels as much as the
  // MFMA rate does, so the max is computed only when needed:
  // on the first tile, and when some lane's partial row sum leaves [0, 2^T] (every p
  // is at most that sum, so a sum within bounds means no p exceeded 2^T and the tile
  // stands; otherwise the tile is redone against the new max, as the eager scheme
  // would have done). ----
  auto xphase = [&](int t) __attribute__((always_inline)) {
    int kv0, ke;
    tile_rows(t, kv0, ke);
    const int rows_left = ke - kv0;                     // visible rows from the tile's first key on
    const int64_t krel = kv0 + kdelta;                  // position of that key relative to query row 0
    bool need_mask = rows_left < BK;
    if (causal) need_mask = need_mask || (POS ? kv0 + BK - 1 > wave_lim_first : krel + BK - 1 > wq0);
    if (need_mask) {
      // key kv0 + j of the segment is visible to this lane iff j <= lim
      int64_t lim64 = rows_left - 1;
      if (causal) lim64 = min(lim64, POS ? qlim64 - kv0 : static_cast<int64_t>(my_q) - krel);
      const int lim = static_cast<int>(max(min(lim64, static_cast<int64_t>(BK)), static_cast<int64_t>(-1))) - 8 * lhalf;
#pragma unroll
      for (int b = 0; b < NKB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = r >> 2, i = r & 3;
          const int kl0 = 32 * b + 16 * (j >> 1) + 4 * (j & 1) + i;
          sacc[b][r] = kl0 <= lim ? sacc[b][r] : -INFINITY;
        }
    }
    auto exp_pack = [&](float& lsum) __attribute__((always_inline)) {
      float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int b = 0; b < NKB; ++b) {
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][r], c, -m_run));
          ls[r & 3] += p[r];
        }
        pf[2 * b] = Ops::pack(p);
        pf[2 * b + 1] = Ops::pack(p + 8);
      }
      lsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };
    float lsum = 0.f;
    bool redo = t == 0;
    if (!redo) {
      exp_pack(lsum);
      redo = __any(!(lsum <= kGrowSum));
    }
    if (redo) {
      float tmax = -INFINITY;
#pragma unroll
      for (int b = 0; b < NKB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sacc[b][r]);
      tmax = max_xor32(tmax) * c;
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int b = 0; b < DB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[b][r] *= alpha;
      m_run = m_new;
      exp_pack(lsum);
    }
    l_run += lsum;
#pragma unroll
    for (int s = 0; s < NPS; ++s) pin(pf[s]);
    pin(l_run);
  };

  // Super-step u (u = 0 .. n_tiles): issue K_{u+NBK-1} and V_{u+NBV-2} (K first); the
  // two phases; wait for this wave's share of K_{u+1} and V_u; barrier.  K_t sits in K
  // buffer t mod NBK, V_t in V buffer t mod NBV; a K buffer is free after the super-step
  // that reads it, a V buffer after the one that follows.  Every wave passes the same
  // barriers.
  auto k_count = [&](int w) __attribute__((always_inline)) {
    return w >= 0 && w + NBK - 1 < n_tiles ? kDmaPerWave : 0;
  };
  auto v_count = [&](int w) __attribute__((always_inline)) {
    return w >= 0 && w + NBV - 2 < n_tiles ? kDmaPerWave : 0;
  };
  auto issue = [&](int u) __attribute__((always_inline)) {
    if constexpr (NBK - 1 == NBV - 2) {
      // K and V of the same tile: one row range for both
      const int t = u + NBK - 1;
      if (t < n_tiles) {
        int kr, ke;
        tile_rows(t, kr, ke);
        dma_k(kr, ke, t % NBK);
        dma_v(kr, ke, t % NBV);
      }
    } else {
      if (u + NBK - 1 < n_tiles) issue_k(u + NBK - 1, (u + NBK - 1) % NBK);
      if (u + NBV - 2 < n_tiles) issue_v(u + NBV - 2, (u + NBV - 2) % NBV);
    }
  };
  auto settle = [&](int u) __attribute__((always_inline)) {
    if (u < n_tiles) {
      // Loads issued after the later of K_{u+1} (issued in super-step u + 2 - NBK) and
      // V_u (in u + 2 - NBV; V after K within a super-step) may stay in flight.
      const int sk = u + 2 - NBK, sv = u + 2 - NBV;
      int allow = sk > sv ? v_count(sk) : 0;
      for (int w = max(sk, sv) + 1; w <= u; ++w) allow += k_count(w) + v_count(w);
      if (allow >= 8) wait_vmcnt<8>();
      else if (allow >= 6) wait_vmcnt<6>();
      else if (allow >= 4) wait_vmcnt<4>();
      else if (allow >= 2) wait_vmcnt<2>();
      else wait_vmcnt<0>();
      __syncthreads();
    }
  };
  const int hot = max(last_live, 0);  // super-steps 1 .. hot have both products live
  // Ring positions of super-step u: rk = u mod NBK (K_u), rv = (u - 1) mod NBV (V_{u-1}).
  auto next = [](int r, int nb) __attribute__((always_inline)) { return r + 1 == nb ? 0 : r + 1; };
  // The lead group issues its DMA share between its two phases, so its MFMA phase
  // starts right after the barrier that opens the super-step; the lag group passes the
  // barrier right after its MFMA phase and issues the next super-step's share before
  // its X phase.  Both groups run one loop body (M, then X, of tile u): a single copy
  // of the phases in the kernel, which also keeps the register allocation to one
  // assignment of the accumulators.
  if (lead) {
    if (live(0)) s_part(0);
    issue(0);
    if (live(0)) xphase(0);
    settle(0);
  } else {
    issue(0);
    if (live(0)) s_part(0);
    settle(0);
    issue(1);
    if (live(0)) xphase(0);
  }
  // Trace: wave 0 stamps the time at which its tiles move from one source to the next
  // (a tile belongs to the source of its top row; ring position (t - d) mod N).
  [[maybe_unused]] int trace_slot = 0;
  [[maybe_unused]] uint32_t* trace_rec = nullptr;
  auto trace_tile = [&](int t) __attribute__((always_inline)) {
    if constexpr (TRACE && RING) {
      if (wave != 0 || t < nt0) return;
      int kr, ke;
      tile_rows(t, kr, ke);
      int dom = 0;
      while (dom + 1 < plan.n && ke - 1 >= plan.off[dom + 1]) ++dom;
      const int slot = (t_dom - dom + plan.n) % plan.n;
      if (slot != trace_slot) {
        const uint64_t now = __builtin_amdgcn_s_memrealtime();
        if (lane == 0) *reinterpret_cast<uint64_t*>(trace_rec + kTraceHeaderWords + 2 * trace_slot) = now;
        trace_slot = slot;
      }
    }
  };
  if constexpr (TRACE && RING) trace_rec = plan.trace + static_cast<int64_t>(blockIdx.x) * plan.trace_stride;
  const int lag = lead ? 0 : 1;
  int u = 1, rk = 1 % NBK, rv = 0;
  for (; u <= hot; ++u, rk = next(rk, NBK), rv = next(rv, NBV)) {
    if constexpr (TRACE) trace_tile(u);
    m_full(rk, rv);
    if (!lead) settle(u);
    issue(u + lag);
    xphase(u);
    if (lead) settle(u);
  }
  for (; u <= n_tiles; ++u, rv = next(rv, NBV)) {
    if (live(u - 1)) pv_part(rv);
    if (lead) issue(u);
    settle(u);
    if (!lead) issue(u + 1);
  }

  if (my_q >= lq) return;
  if constexpr (RING) {
    const int64_t row = static_cast<int64_t>(plan.off[t_dom]) + my_q;
    write_final_row<DW>(plan.out, plan.dtype, head * plan.out_hs + row * plan.out_ss,
                       plan.lse != nullptr ? plan.lse + head * plan.lse_hs + row : nullptr, lhalf, oacc, m_run,
                       sum_xor32(l_run), dn);
    if constexpr (TRACE) {
      if (wave == 0) {  // wave 0 always holds rows (a query tile's first 32 rows exist)
        const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
        const uint64_t c1 = __builtin_amdgcn_s_memtime();
        uint32_t hw, xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        if (lane == 0) {
          uint64_t* r64 = reinterpret_cast<uint64_t*>(trace_rec);
          r64[0] = trace_t0;
          r64[1] = t1;
          r64[2] = trace_c0;
          r64[3] = c1;
          *reinterpret_cast<u32x4*>(trace_rec + 8) =
              u32x4{hw, xcc, static_cast<uint32_t>(t_dom) | (static_cast<uint32_t>(hg) << 16), static_cast<uint32_t>(qt)};
          *reinterpret_cast<u32x4*>(trace_rec + 12) = u32x4{static_cast<uint32_t>(n_tiles), 0u, 0u, 0u};
          r64[kTraceHeaderWords / 2 + trace_slot] = t1;
        }
      }
    }
  } else {
    write_row<DW>(*ap, head, my_q, lhalf, oacc, m_run, sum_xor32(l_run), dn);
  }
}

template <int DT, int G, bool POS, int BK, int DWN>
__global__ __launch_bounds__(kThreads, 1) void flash_block_pingpong_kernel(BlockGroup grp) {
  pingpong_body<DT, G, POS, BK, false, BlockGroup, false, DWN>(grp);
}

template <int DT, int G, int BK, bool TRACE, int DWN>
__global__ __launch_bounds__(kThreads, 1) void flash_ring_kernel(RingPlan plan) {
  pingpong_body<DT, G, false, BK, true, RingPlan, TRACE, DWN>(plan);
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
  void* fin_out;
  int32_t fin_dtype;
  int64_t fin_hs, fin_ss;
  float* fin_lse;
  int64_t fin_lse_hs;
  const int32_t* q_lim;
  const int32_t* kv_sel;   // as BlockArgs
  const void* k_alt;
  const void* v_alt;
  int64_t alt_hs, alt_ss;
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
  if (a.q_lim != nullptr && a.kv_sel != nullptr && *a.kv_sel != 0) {
    a.k = a.k_alt; a.v = a.v_alt;
    a.k_hs = a.v_hs = a.alt_hs;
    a.k_ss = a.v_ss = a.alt_ss;
  }
  const bool live = row < a.lq;
  const int d = a.d;
  float qv[DMAX], acc[DMAX];
  for (int i = 0; i < DMAX; ++i) {
    qv[i] = (live && i < d) ? load_elem<DT>(a.q, head * a.q_hs + static_cast<int64_t>(row) * a.q_ss + i) : 0.f;
    acc[i] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  // Causal: this row sees keys [0, row_lim) of the chunk (a prefix, see row_limits).
  int64_t row_lim = a.lk;
  int n_kv = a.lk;
  if (a.causal) {
    if (a.q_lim != nullptr) {
      row_lim = live ? min(max(a.q_lim[row], 0), a.lk) : 0;
      int hi = static_cast<int>(row_lim);  // one wave per workgroup
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) hi = max(hi, __shfl_xor(hi, off));
      n_kv = hi;
    } else {
      row_lim = a.q_off + row + 1 - a.k_off;
      const int last = min(a.lq, static_cast<int>(blockIdx.x + 1) * kGenRows) - 1;
      const int64_t lim = a.q_off + last + 1 - a.k_off;
      n_kv = static_cast<int>(lim <= 0 ? 0 : (lim < a.lk ? lim : a.lk));
    }
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
      if (kv0 + r >= row_lim) continue;
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
  float c_old = 0.f, c_new = inv, lse_out = lse_new;
  if (a.accumulate) {
    const float lse_old = a.lse[orow];
    const float mm = fmaxf(lse_old, lse_new);
    const bool ok = mm != -INFINITY;
    const float w_old = ok ? __expf(lse_old - mm) : 0.f;
    const float w_new = ok ? __expf(lse_new - mm) : 0.f;
    const float den = w_old + w_new;
    const float rden = den > 0.f ? 1.f / den : 0.f;
    c_old = w_old * rden;
    c_new = w_new * rden * inv;
    lse_out = ok ? mm + __logf(den) : -INFINITY;
  }
  for (int i = 0; i < d && i < DMAX; ++i) {
    float x = c_new * acc[i];
    if (a.accumulate) x += c_old * a.o[orow * d + i];
    if (a.fin_out) store_elem_rt(a.fin_out, a.fin_dtype, head * a.fin_hs + static_cast<int64_t>(row) * a.fin_ss + i, x);
    else a.o[orow * d + i] = x;
  }
  if (a.fin_out) {
    if (a.fin_lse) a.fin_lse[head * a.fin_lse_hs + row] = lse_out;
  } else {
    a.lse[orow] = lse_out;
  }
}

// ----------------------------------------------------------------------------------
// fp32 matrix-core kernel (v_mfma_f32_32x32x2f32): the reference's fp32 fold
// (ring.rs:201-370, its CPU default and c1's dtype) with fp32 products on the matrix
// cores.  A workgroup is 4 waves over 128 query rows of one head (32 rows a wave); K / V
// tiles of 32 keys are staged in LDS as fp32, the next tile's loads in flight (in
// registers) while the current one is folded.  Per tile a wave computes
//   S^T (32 keys x 32 rows) = K Q^T  in DP/2 MFMAs, k-step s taking dim
//                                    8 (s / 4) + 4 half + (s mod 4) in lane half `half`;
//   O^T (DP dims x 32 rows) += V^T P^T  in 16 MFMAs per 32 dims, k-step s pairing the
//                                    keys a lane already holds as element s of S^T
//                                    (8 (s / 4) + 4 half + s mod 4), so P needs no shuffle.
// LDS layouts make each 16-byte read feed four k-steps: K rows in dim order ([key][dim],
// a loaded 16-byte group stored as is), whose dims 8u + 4 half .. +3 are k-steps
// 4u .. 4u+3 of a lane half; V stored transposed ([dim][key]), where the four keys of
// k-steps 4t .. 4t+3 of a lane half are adjacent.  Element i of a 32x32
// accumulator holds row 8 (i / 4) + 4 half + (i mod 4), column lane mod 32 -- the
// layout of the head-dim-128 kernel's O^T, whose epilogue indexing this one shares.
// Masking, the online softmax (base 2, scale folded into the exponent), the running-
// state merge (accumulate) and the final-row mode are those of general_block_kernel.
// ----------------------------------------------------------------------------------
constexpr int kF32Waves = 4;
constexpr int kF32Threads = 64 * kF32Waves;
constexpr int kF32Rows = 32 * kF32Waves;
constexpr int kF32BK = 32;

template <int DP>
__global__ __launch_bounds__(kF32Threads) void mfma_f32_block_kernel(GenArgs a) {
  static_assert(DP % 32 == 0 && DP <= 128, "padded head dim");
  constexpr int DB = DP / 32;
  constexpr int KS = DP / 2;
  constexpr int KLS = DP + 4;          // K row stride (floats), 16-byte aligned
  constexpr int VLS = kF32BK + 4;      // V^T row stride (floats), 16-byte aligned
  constexpr int NV4 = kF32BK * DP / 4 / kF32Threads;  // float4 of K (and of V) per thread per tile
  static_assert(NV4 >= 1 && kF32BK * DP % (4 * kF32Threads) == 0, "tile split");
  __shared__ __attribute__((aligned(16))) float ks[kF32BK * KLS];
  __shared__ __attribute__((aligned(16))) float vt[DP * VLS];
  __shared__ int red[kF32Waves];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lcol = lane & 31, half = lane >> 5;
  // work item: heads innermost, query tiles from the last (the most keys under causal
  // masking) to the first, so every head's heaviest tiles start first
  const int n_qt = (a.lq + kF32Rows - 1) / kF32Rows;
  const int head = blockIdx.x % a.hq;
  const int qt = n_qt - 1 - static_cast<int>(blockIdx.x / a.hq);
  const int kvh = head / a.rep;
  const int d = a.d;
  if (a.q_lim != nullptr && a.kv_sel != nullptr && __builtin_amdgcn_readfirstlane(*a.kv_sel) != 0) {
    a.k = a.k_alt; a.v = a.v_alt;
    a.k_hs = a.v_hs = a.alt_hs;
    a.k_ss = a.v_ss = a.alt_ss;
  }
  const float* kf = static_cast<const float*>(a.k) + kvh * a.k_hs;
  const float* vf = static_cast<const float*>(a.v) + kvh * a.v_hs;
  const int tq0 = qt * kF32Rows;
  const int row = tq0 + 32 * wave + lcol;
  const bool live = row < a.lq;

  // Q^T fragments: k-step s, this lane's row, dim 8 (s / 4) + 4 half + (s mod 4) (zero
  // past the head dim)
  float qf[KS];
  {
    const float* qr = static_cast<const float*>(a.q) + head * a.q_hs + static_cast<int64_t>(row) * a.q_ss;
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2) {
      const int dim = 8 * (s2 >> 2) + 4 * half + (s2 & 3);
      qf[s2] = (live && dim < d) ? qr[dim] : 0.f;
    }
  }
  // Keys [0, row_lim) of the chunk are visible to this lane's row; n_kv bounds the tiles.
  int64_t row_lim = a.lk;
  int n_kv = a.lk;
  if (a.causal) {
    if (a.q_lim != nullptr) {
      row_lim = live ? min(max(a.q_lim[row], 0), a.lk) : 0;
      int hi = static_cast<int>(row_lim);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) hi = max(hi, __shfl_xor(hi, off));
      if (lane == 0) red[wave] = hi;
      __syncthreads();
      hi = 0;
#pragma unroll
      for (int w = 0; w < kF32Waves; ++w) hi = max(hi, red[w]);
      n_kv = hi;
    } else {
      row_lim = a.q_off + row + 1 - a.k_off;
      const int last = min(a.lq, tq0 + kF32Rows) - 1;
      const int64_t lim = a.q_off + last + 1 - a.k_off;
      n_kv = static_cast<int>(lim <= 0 ? 0 : (lim < a.lk ? lim : a.lk));
    }
  }
  row_lim = live ? min(row_lim, static_cast<int64_t>(a.lk)) : 0;
  // the wave's last visible key + 1: tiles from there on are skipped by this wave
  int wave_hi = static_cast<int>(max(row_lim, int64_t(0)));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) wave_hi = max(wave_hi, __shfl_xor(wave_hi, off));
  wave_hi = __builtin_amdgcn_readfirstlane(wave_hi);

  // Tile loads: float4 j of this thread is row e / (DP/4), dims 4 (e mod DP/4) .. +3 of
  // the tile (e = tid + j * threads); zero past the chunk or the head dim.
  float4 kr[NV4], vr[NV4];
  auto load_tile = [&](int kv0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
      const int e = tid + j * kF32Threads;
      const int r = e / (DP / 4), c4 = 4 * (e % (DP / 4));
      const int kv = kv0 + r;
      const bool in = kv < a.lk && c4 < d;
      const float* kp = kf + static_cast<int64_t>(kv) * a.k_ss + c4;
      const float* vp = vf + static_cast<int64_t>(kv) * a.v_ss + c4;
      kr[j] = in ? make_float4(kp[0], kp[1], kp[2], kp[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
      vr[j] = in ? make_float4(vp[0], vp[1], vp[2], vp[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store_tile = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
      const int e = tid + j * kF32Threads;
      const int r = e / (DP / 4), c4 = 4 * (e % (DP / 4));
      *reinterpret_cast<float4*>(&ks[r * KLS + c4]) = kr[j];
      vt[(c4 + 0) * VLS + r] = vr[j].x;
      vt[(c4 + 1) * VLS + r] = vr[j].y;
      vt[(c4 + 2) * VLS + r] = vr[j].z;
      vt[(c4 + 3) * VLS + r] = vr[j].w;
    }
  };

  const float c = a.scale * kLog2e;
  f32x16 oacc[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[b][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  if (n_kv > 0) load_tile(0);
  for (int kv0 = 0; kv0 < n_kv; kv0 += kF32BK) {
    __syncthreads();  // the previous tile's reads are done
    store_tile();
    __syncthreads();
    if (kv0 + kF32BK < n_kv) load_tile(kv0 + kF32BK);  // in flight while this tile is folded
    if (kv0 >= wave_hi) continue;  // no key of this tile is visible to the wave's rows
    // S^T in two accumulators (even / odd groups of four k-steps), summed after
    f32x16 sa, sb;
#pragma unroll
    for (int r = 0; r < 16; ++r) sa[r] = sb[r] = 0.f;
    const float* kl = &ks[lcol * KLS + 4 * half];
#pragma unroll
    for (int u = 0; u < KS / 4; ++u) {
      const float4 k4 = *reinterpret_cast<const float4*>(kl + 8 * u);
      f32x16& acc = (u & 1) ? sb : sa;
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.x, qf[4 * u + 0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.y, qf[4 * u + 1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.z, qf[4 * u + 2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.w, qf[4 * u + 3], acc, 0, 0, 0);
    }
    // K reads two ahead of the MFMAs that use them (all 16 at once take 64 registers)
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int i = 0; i < KS / 4 - 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    // element i: key kv0 + 8 (i / 4) + 4 half + (i mod 4) of this lane's row
    const int64_t vis = row_lim - kv0;  // keys of the tile visible to the row: [0, vis)
    float p[16];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = 8 * (i >> 2) + 4 * half + (i & 3);
      p[i] = j < vis ? (sa[i] + sb[i]) * c : -INFINITY;
      mx = fmaxf(mx, p[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    // a row with no visible key so far keeps m = -inf, p = 0 and its (zero) state
    const bool none = m_new == -INFINITY;
    const float alpha = none ? 1.f : exp2f(m_run - m_new);
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      p[i] = none ? 0.f : exp2f(p[i] - m_new);
      ls += p[i];
    }
    l_run = l_run * alpha + ls;
    // alpha is exactly 1 where the running max did not grow: the accumulators are
    // rescaled only when it grew in some lane of the wave (mostly the first tiles)
    if (__any(m_new != m_run)) {
      asm volatile("");  // a real branch: not turned into unconditional multiplies
#pragma unroll
      for (int b = 0; b < DB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[b][r] *= alpha;
    }
    m_run = m_new;
    // O^T += V^T P^T: k-steps 4t .. 4t+3 take keys 8t + 4 half + 0..3, adjacent in V^T
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float4 v4[DB];
#pragma unroll
      for (int b = 0; b < DB; ++b)
        v4[b] = *reinterpret_cast<const float4*>(&vt[(32 * b + lcol) * VLS + 8 * t + 4 * half]);
#pragma unroll
      for (int b = 0; b < DB; ++b) oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4[b].x, p[4 * t + 0], oacc[b], 0, 0, 0);
#pragma unroll
      for (int b = 0; b < DB; ++b) oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4[b].y, p[4 * t + 1], oacc[b], 0, 0, 0);
#pragma unroll
      for (int b = 0; b < DB; ++b) oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4[b].z, p[4 * t + 2], oacc[b], 0, 0, 0);
#pragma unroll
      for (int b = 0; b < DB; ++b) oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4[b].w, p[4 * t + 3], oacc[b], 0, 0, 0);
    }
    // V^T reads one group (DB reads) ahead, then one per DB MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, DB, 1);
#pragma unroll
    for (int i = 0; i < 3 * DB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * DB, 1);
  }
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!live) return;
  const bool any = l_tot > 0.f;
  const float inv = any ? 1.f / l_tot : 0.f;
  const float lse_new = any ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  const int64_t orow = static_cast<int64_t>(head) * a.lq + row;
  float c_old = 0.f, c_new = inv, lse_out = lse_new;
  if (a.accumulate) {
    const float lse_old = a.lse[orow];
    const float mm = fmaxf(lse_old, lse_new);
    const bool ok = mm != -INFINITY;
    const float w_old = ok ? __expf(lse_old - mm) : 0.f;
    const float w_new = ok ? __expf(lse_new - mm) : 0.f;
    const float den = w_old + w_new;
    const float rden = den > 0.f ? 1.f / den : 0.f;
    c_old = w_old * rden;
    c_new = w_new * rden * inv;
    lse_out = ok ? mm + __logf(den) : -INFINITY;
  }
  const int64_t fin_row = head * a.fin_hs + static_cast<int64_t>(row) * a.fin_ss;
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int dcol = 32 * b + 8 * j + 4 * half;
      if (dcol >= d) continue;  // head dims are multiples of 4: whole groups only
      float x0 = c_new * oacc[b][4 * j], x1 = c_new * oacc[b][4 * j + 1];
      float x2 = c_new * oacc[b][4 * j + 2], x3 = c_new * oacc[b][4 * j + 3];
      if (a.accumulate) {
        const float4 old = *reinterpret_cast<const float4*>(a.o + orow * d + dcol);
        x0 += c_old * old.x; x1 += c_old * old.y; x2 += c_old * old.z; x3 += c_old * old.w;
      }
      if (a.fin_out) store4(a.fin_out, a.fin_dtype, fin_row + dcol, x0, x1, x2, x3);
      else *reinterpret_cast<float4*>(a.o + orow * d + dcol) = make_float4(x0, x1, x2, x3);
    }
  if (half == 0) {
    if (a.fin_out) {
      if (a.fin_lse) a.fin_lse[head * a.fin_lse_hs + row] = lse_out;
    } else {
      a.lse[orow] = lse_out;
    }
  }
}

// ----------------------------------------------------------------------------------
// Host launcher
// ----------------------------------------------------------------------------------

// Heads per workgroup of the matrix-core kernels: the largest of 8, 4, 2 dividing
// Hq / Hkv (query heads that share a KV head), else 1.
static int heads_per_group(int rep) {
  for (int cand : {8, 4, 2})
    if (rep % cand == 0) return cand;
  return 1;
}

// Work decomposition of the matrix-core kernels: query heads per group (sharing a K/V
// tile), query rows per workgroup and head groups per query tile.
struct Geometry {
  int g, tq, n_groups;
};
static Geometry geometry(int hq, int hkv) {
  Geometry r;
  r.g = heads_per_group(hq / hkv);
  r.tq = 32 * (kWaves / r.g);
  r.n_groups = hq / r.g;
  return r;
}

// The head-dim-128 kernels form buffer descriptors with 32-bit row arithmetic: a tile of
// kBK3 rows of either view must stay below 2^31 bytes.
static void check_tile_bytes(int64_t k_ss, int64_t v_ss) {
  require(k_ss > 0 && v_ss > 0 && k_ss * 2 * kBK3 < (int64_t(1) << 31) && v_ss * 2 * kBK3 < (int64_t(1) << 31),
          "k/v sequence strides too large for the matrix-core kernel");
}

static BlockArgs make_args(const BlockLaunch& L) {
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
  a.fin_out = L.fin_out; a.fin_dtype = L.fin_dtype; a.fin_hs = L.fin_hs; a.fin_ss = L.fin_ss;
  a.fin_lse = L.fin_lse; a.fin_lse_hs = L.fin_lse_hs;
  a.q_lim = L.causal ? L.q_lim : nullptr;
  a.kv_sel = L.kv_sel;
  a.k_alt = static_cast<const uint16_t*>(L.k_alt);
  a.v_alt = static_cast<const uint16_t*>(L.v_alt);
  a.alt_hs = L.alt_hs;
  a.alt_ss = L.alt_ss;
  a.d = static_cast<int32_t>(L.d);
  const Geometry geo = geometry(L.hq, L.hkv);
  a.n_qtiles = static_cast<int32_t>(ceil_div(L.lq, geo.tq));
  a.n_groups = geo.n_groups;
  return a;
}

// Head dims up to 64 take the half-width instantiation (DWN = 64): same tiles and
// zero padding, half the MFMA work of the 128-dim fold.
static bool half_width_d(int d) { return d <= kD3 / 2; }

// One launch of the head-dim-128 kernel over grp.a[0 .. grp.n) (same dtype, heads, and
// positions mode; every pair has at least one query tile).
template <int DT, int G, int DWN>
static void launch_pingpong_g(const BlockGroup& grp, bool pos, dim3 grid, hipStream_t stream) {
  if (pos) flash_block_pingpong_kernel<DT, G, true, kBK3, DWN><<<grid, kThreads, 0, stream>>>(grp);
  else flash_block_pingpong_kernel<DT, G, false, kBK3, DWN><<<grid, kThreads, 0, stream>>>(grp);
}

template <int DT, int DWN>
static void launch_pingpong_w(const BlockGroup& grp, int g, bool pos, dim3 grid, hipStream_t stream) {
  switch (g) {
    case 8: launch_pingpong_g<DT, 8, DWN>(grp, pos, grid, stream); break;
    case 4: launch_pingpong_g<DT, 4, DWN>(grp, pos, grid, stream); break;
    case 2: launch_pingpong_g<DT, 2, DWN>(grp, pos, grid, stream); break;
    default: launch_pingpong_g<DT, 1, DWN>(grp, pos, grid, stream); break;
  }
}

template <int DT>
static void launch_pingpong(BlockGroup& grp, hipStream_t stream) {
  const BlockArgs& a0 = grp.a[0];
  for (int i = 0; i < grp.n; ++i) {
    check_tile_bytes(grp.a[i].k_ss, grp.a[i].v_ss);
    if (grp.a[i].kv_sel != nullptr) check_tile_bytes(grp.a[i].alt_ss, grp.a[i].alt_ss);
  }
  grp.qt_begin[0] = 0;
  for (int i = 0; i < grp.n; ++i) grp.qt_begin[i + 1] = grp.qt_begin[i] + grp.a[i].n_qtiles;
  const dim3 grid(static_cast<unsigned>(grp.qt_begin[grp.n] * a0.n_groups));
  const bool pos = a0.q_lim != nullptr;
  const int g = geometry(a0.hq, a0.hkv).g;
  if (half_width_d(a0.d)) launch_pingpong_w<DT, kD3 / 2>(grp, g, pos, grid, stream);
  else launch_pingpong_w<DT, kD3>(grp, g, pos, grid, stream);
}

template <int DT>
static void launch_mfma(const BlockLaunch& L, hipStream_t stream) {
  BlockGroup grp;
  grp.n = 1;
  grp.a[0] = make_args(L);
  launch_pingpong<DT>(grp, stream);
}

static GenArgs make_gen_args(const BlockLaunch& L) {
  GenArgs a;
  a.q = L.q; a.k = L.k; a.v = L.v;
  a.q_hs = L.q_hs; a.q_ss = L.q_ss; a.k_hs = L.k_hs; a.k_ss = L.k_ss; a.v_hs = L.v_hs; a.v_ss = L.v_ss;
  a.o = L.o; a.lse = L.lse;
  a.hq = L.hq; a.rep = L.hq / L.hkv;
  a.lq = static_cast<int32_t>(L.lq); a.lk = static_cast<int32_t>(L.lk); a.d = L.d;
  a.q_off = L.q_off; a.k_off = L.k_off;
  a.causal = L.causal; a.accumulate = L.accumulate;
  a.scale = L.scale;
  a.fin_out = L.fin_out; a.fin_dtype = L.fin_dtype; a.fin_hs = L.fin_hs; a.fin_ss = L.fin_ss;
  a.fin_lse = L.fin_lse; a.fin_lse_hs = L.fin_lse_hs;
  a.q_lim = L.causal ? L.q_lim : nullptr;
  a.kv_sel = L.kv_sel;
  a.k_alt = L.k_alt;
  a.v_alt = L.v_alt;
  a.alt_hs = L.alt_hs;
  a.alt_ss = L.alt_ss;
  return a;
}

template <int DT>
static void launch_general(const BlockLaunch& L, hipStream_t stream) {
  const GenArgs a = make_gen_args(L);
  const dim3 grid(static_cast<unsigned>(ceil_div(L.lq, kGenRows)), static_cast<unsigned>(L.hq));
  if (L.d <= 64) general_block_kernel<DT, 64><<<grid, kGenRows, 0, stream>>>(a);
  else if (L.d <= 128) general_block_kernel<DT, 128><<<grid, kGenRows, 0, stream>>>(a);
  else general_block_kernel<DT, 256><<<grid, kGenRows, 0, stream>>>(a);
}

// Head dims the head-dim-128 kernel takes: up to 128 in 16-byte columns, zero-padded in
// LDS.  Head dims up to 64 run its half-width instantiation (the MFMAs and fragment reads
// of dims 64-127 not issued); a dedicated head-dim-64 kernel with register-staged 64-key
// tiles measured 7-29% slower than even the zero-padded full-width form.
static bool padded_d_ok(int d) { return d > 0 && d <= kD3 && d % 8 == 0; }

// True when the matrix-core kernels handle this shape.
bool block_uses_mfma(int dtype, int d) { return (dtype == kBF16 || dtype == kF16) && padded_d_ok(d); }

// The fp32 matrix-core kernel: head dims that are multiples of 4 up to 128 (any view
// layout: Q / K / V are read one element per lane), with the state and final rows it
// writes four values at a time aligned for that (16-byte fp32, 8-byte 16-bit stores).
bool block_uses_mfma_f32(const BlockLaunch& L) {
  if (L.dtype != kF32 || L.d % 4 != 0 || L.d > kD3) return false;
  auto aligned = [](const void* p, uintptr_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  if (L.fin_out != nullptr &&
      (!aligned(L.fin_out, L.fin_dtype == kF32 ? 16 : 8) || L.fin_hs % 4 != 0 || L.fin_ss % 4 != 0))
    return false;
  if ((L.fin_out == nullptr || L.accumulate) && !aligned(L.o, 16)) return false;
  return true;
}

static void launch_mfma_f32(const BlockLaunch& L, hipStream_t stream) {
  const GenArgs a = make_gen_args(L);
  const int64_t items = ceil_div(L.lq, kF32Rows) * static_cast<int64_t>(L.hq);
  require(items <= INT32_MAX, "fp32 block: too many work items");
  const dim3 grid(static_cast<unsigned>(items));
  const dim3 block(kF32Threads);
  switch ((L.d + 31) / 32) {
    case 1: mfma_f32_block_kernel<32><<<grid, block, 0, stream>>>(a); break;
    case 2: mfma_f32_block_kernel<64><<<grid, block, 0, stream>>>(a); break;
    case 3: mfma_f32_block_kernel<96><<<grid, block, 0, stream>>>(a); break;
    default: mfma_f32_block_kernel<128><<<grid, block, 0, stream>>>(a); break;
  }
}

void launch_block_partial(const BlockLaunch& L, hipStream_t stream) {
  if (L.lq == 0) return;
  if (!L.force_general && block_uses_mfma(L.dtype, L.d)) {
    if (L.dtype == kBF16) launch_mfma<kBF16>(L, stream);
    else launch_mfma<kF16>(L, stream);
  } else if (block_uses_mfma_f32(L)) {
    launch_mfma_f32(L, stream);
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

// Visible (query, key) pairs of one block, for ordering the pairs of a group: exact for
// contiguous positions, lq * lk / 2 for explicit ones.
static double block_work(const BlockLaunch& L) {
  const double lq = static_cast<double>(L.lq), lk = static_cast<double>(L.lk);
  if (!L.causal) return lq * lk;
  if (L.q_lim != nullptr) return lq * lk / 2;
  // row i sees min(max(c + i, 0), lk) keys, c = q_off - k_off + 1
  const int64_t c = L.q_off - L.k_off + 1;
  const int64_t i0 = std::min<int64_t>(std::max<int64_t>(0, 1 - c), L.lq);
  const int64_t i1 = std::min<int64_t>(std::max<int64_t>(0, L.lk - c), L.lq);
  double w = static_cast<double>(L.lq - std::max(i0, i1)) * lk;
  if (i1 > i0) w += static_cast<double>(i1 - i0) * static_cast<double>(c) + 0.5 * static_cast<double>(i0 + i1 - 1) * static_cast<double>(i1 - i0);
  return w;
}

void launch_block_group(const BlockLaunch* Ls, int n, hipStream_t stream) {
  std::vector<const BlockLaunch*> live;
  for (int i = 0; i < n; ++i)
    if (Ls[i].lq > 0) live.push_back(&Ls[i]);
  if (live.empty()) return;
  const BlockLaunch& f = *live[0];
  bool grouped = !f.force_general && block_uses_mfma(f.dtype, f.d) && padded_d_ok(f.d);
  for (const BlockLaunch* L : live)
    grouped = grouped && !L->force_general && L->dtype == f.dtype && L->d == f.d && L->hq == f.hq &&
              L->hkv == f.hkv && (L->causal && L->q_lim != nullptr) == (f.causal && f.q_lim != nullptr);
  if (!grouped) {
    for (const BlockLaunch* L : live) launch_block_partial(*L, stream);
    return;
  }
  // heaviest pairs first: their workgroups are dispatched first on every XCD
  std::stable_sort(live.begin(), live.end(),
                   [](const BlockLaunch* x, const BlockLaunch* y) { return block_work(*x) > block_work(*y); });
  for (size_t base = 0; base < live.size(); base += kMaxGroup) {
    BlockGroup grp;
    grp.n = static_cast<int32_t>(std::min<size_t>(kMaxGroup, live.size() - base));
    for (int i = 0; i < grp.n; ++i) grp.a[i] = make_args(*live[base + i]);
    if (f.dtype == kBF16) launch_pingpong<kBF16>(grp, stream);
    else launch_pingpong<kF16>(grp, stream);
  }
  HCP_HIP(hipGetLastError());
}

template <int DT, bool TRACE, int DWN>
static void launch_ring_kernel_w(int g, dim3 grid, const RingPlan& p, hipStream_t stream) {
  switch (g) {
    case 8: flash_ring_kernel<DT, 8, kBK3, TRACE, DWN><<<grid, kThreads, 0, stream>>>(p); break;
    case 4: flash_ring_kernel<DT, 4, kBK3, TRACE, DWN><<<grid, kThreads, 0, stream>>>(p); break;
    case 2: flash_ring_kernel<DT, 2, kBK3, TRACE, DWN><<<grid, kThreads, 0, stream>>>(p); break;
    default: flash_ring_kernel<DT, 1, kBK3, TRACE, DWN><<<grid, kThreads, 0, stream>>>(p); break;
  }
}

template <int DT, bool TRACE>
static void launch_ring_kernel(int g, dim3 grid, const RingPlan& p, hipStream_t stream) {
  if (half_width_d(p.d)) launch_ring_kernel_w<DT, TRACE, kD3 / 2>(g, grid, p, stream);
  else launch_ring_kernel_w<DT, TRACE, kD3>(g, grid, p, stream);
}

bool ring_fused_applies(int dtype, int d) { return (dtype == kBF16 || dtype == kF16) && padded_d_ok(d); }

void launch_ring_fused(const RingLaunch& L, hipStream_t stream) {
  require(ring_fused_applies(L.dtype, L.d),
          "fused ring: dtype must be BF16 or F16 with head_dim a multiple of 8 up to 128");
  check_tile_bytes(L.k_ss, L.v_ss);
  require(L.n >= 1 && L.n <= kMaxDomains, "fused ring: 1 to 64 domains");
  RingPlan p{};
  p.q = static_cast<const uint16_t*>(L.q);
  p.k = static_cast<const uint16_t*>(L.k);
  p.v = static_cast<const uint16_t*>(L.v);
  p.q_hs = L.q_hs; p.q_ss = L.q_ss; p.k_hs = L.k_hs; p.k_ss = L.k_ss; p.v_hs = L.v_hs; p.v_ss = L.v_ss;
  p.out = L.out; p.out_hs = L.out_hs; p.out_ss = L.out_ss;
  p.lse = L.lse; p.lse_hs = L.lse_hs;
  p.dtype = L.dtype;
  p.d = L.d;
  p.hq = L.hq; p.hkv = L.hkv; p.rep = L.hq / L.hkv;
  const Geometry geo = geometry(L.hq, L.hkv);
  const int g = geo.g, tq = geo.tq;
  p.n_groups = geo.n_groups;
  p.n = L.n;
  p.causal = L.causal;
  p.scale_log2 = L.scale * kLog2e;
  int64_t acc = 0;
  for (int i = 0; i < L.n; ++i) {
    require(L.len[i] >= 1, "fused ring: every chunk length must be >= 1");
    p.off[i] = static_cast<int32_t>(acc);
    p.len[i] = static_cast<int32_t>(L.len[i]);
    acc += L.len[i];
    require(acc <= INT32_MAX, "fused ring: total length must fit in int32");
  }
  // slot s holds domain n-1-s: later domains (more visible keys under causal masking) first
  p.qt_begin[0] = 0;
  for (int s = 0; s < L.n; ++s) p.qt_begin[s + 1] = p.qt_begin[s] + static_cast<int32_t>(ceil_div(p.len[L.n - 1 - s], tq));
  const int64_t blocks = static_cast<int64_t>(p.qt_begin[L.n]) * p.n_groups;
  require(blocks <= INT32_MAX, "fused ring: too many workgroups");
  require(blocks == ring_fused_workgroups(L.hq, L.hkv, L.n, L.len), "fused ring: workgroup count");
  p.trace = L.trace;
  p.trace_stride = L.trace_stride;
  if (L.trace != nullptr) require(L.trace_stride >= kTraceHeaderWords + 2 * L.n, "fused ring: trace stride");
  const dim3 grid(static_cast<unsigned>(blocks));
  if (L.dtype == kBF16) {
    if (L.trace != nullptr) launch_ring_kernel<kBF16, true>(g, grid, p, stream);
    else launch_ring_kernel<kBF16, false>(g, grid, p, stream);
  } else {
    if (L.trace != nullptr) launch_ring_kernel<kF16, true>(g, grid, p, stream);
    else launch_ring_kernel<kF16, false>(g, grid, p, stream);
  }
  HCP_HIP(hipGetLastError());
}

int64_t ring_fused_workgroups(int hq, int hkv, int n, const int64_t* len) {
  const Geometry geo = geometry(hq, hkv);
  int64_t tiles = 0;
  for (int i = 0; i < n; ++i) tiles += ceil_div(len[i], geo.tq);
  return tiles * geo.n_groups;
}

int ring_trace_words(int n) { return kTraceHeaderWords + 2 * n; }

}  // namespace hcp
