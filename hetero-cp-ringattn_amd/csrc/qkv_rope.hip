// Fused QKV projection + RoPE + KV append: the producer of the ring operator's inputs.
//
// Replaces the head of HcpRingAttentionBackend::forward (ring.rs:1865-1936): three
// projections x W^T (+ bias), the head split, the rotary embedding of q and k
// (RotaryEmbedding::apply / rotate_pairs, rust/src/model/layers/rotary.rs:103-158) at
// each token's global position, and the KV-cache append (KvCache::update,
// cache.rs:191-251; the positioned slab append of self_driving.rs:180-228), as one
// matrix-core GEMM whose epilogue does everything after the accumulation:
//
//   * C^T = W X^T on v_mfma_f32_32x32x16 (A = weight rows, B = token rows, both
//     hidden-contiguous), so a lane owns one token and 16 features of each 32-feature
//     block.  A workgroup computes 256 features x TN tokens (TN = 128, 256 or 384,
//     chosen per launch) with 8 waves of 64 features x TN/2 tokens: a wave's 64
//     features are the 32-feature blocks at d and d + D/2 of one head, so each RoPE
//     partner pair sits in the same lane and register slot of the wave's two blocks --
//     the rotation needs no data exchange.
//   * Weight and token tiles of 32 hidden values reach LDS through buffer_load ... lds
//     (four buffers, three stages in flight, one barrier per stage); chunk p of tile row
//     r holds global chunk p ^ ((r >> 2) & 3), which keeps the fragment reads free of
//     bank conflicts.  The loop is software-pipelined: a stage's DMA instructions are
//     spread through the MFMAs of the stage three before it, the second K half's
//     fragments are read while the first half's MFMAs run, and the next stage's barrier
//     sits inside this stage's second half, so its first fragments arrive while the
//     matrix core still has this stage's MFMAs queued (measured on the Llama-3-8B layer:
//     +7.6% over one barrier and one DMA burst at each stage start).
//   * Epilogue, in fp32: + bias, rotate (x1 cos - x2 sin, x1 sin + x2 cos) with cos/sin
//     from the table row of the token's position, round once to the storage dtype and
//     store 8 consecutive head dims (16 bytes) per lane -- the two lanes holding halves
//     of an 8-dim group swap them with v_permlane32_swap, half the store instructions of
//     8-byte stores (+2.3% on the Llama-3-8B layer); 8-byte stores when a row start is
//     not 16-byte aligned: q into [Hq, L, D], k / v into [Hkv, L, D] views or appended to
//     the paged pool through the block table.
#include <cmath>

#include "kernels.hpp"
#include "lds_dma.hpp"

namespace hcp {


namespace {

constexpr int kQWaves = 8;
constexpr int kQThreads = kQWaves * 64;
constexpr int kQTileF = 256;                 // features per workgroup
constexpr int kQK = 32;                      // hidden values per stage
constexpr int kQRow = kQK * 2;               // bytes per tile row in LDS
constexpr int kQOperandW = kQTileF * kQRow;  // 16 KiB
constexpr int kQBufs = 4;
constexpr int kQGroupM = 4;                  // token tiles per placement group

template <int DT>
struct QkvMfma;
template <>
struct QkvMfma<kBF16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct QkvMfma<kF16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ uint32_t qswz(int r) { return static_cast<uint32_t>((r >> 2) & 3); }

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == kBF16) return f32x2_to_bf16x2_bits(a, b);
  else return static_cast<uint32_t>(f32_to_f16_bits(a)) | (static_cast<uint32_t>(f32_to_f16_bits(b)) << 16);
}

template <int DT>
__device__ __forceinline__ float ld16(const uint16_t* p) {
  return DT == kBF16 ? bf16_bits_to_f32(*p) : f16_bits_to_f32(*p);
}

// TN = tokens per workgroup (256 or 128).  Wave w owns feature group wf = w & 3 and
// token half wt = w >> 2: 64 features -- the 32-feature blocks at fbase and
// fbase + D/2 of one head, i.e. RoPE partners -- times TN/2 tokens.
template <int DT, int D, int TN>
__global__ __launch_bounds__(kQThreads, 1) void qkv_rope_kernel(QkvArgs a) {
  using Ops = QkvMfma<DT>;
  using frag = typename Ops::frag;
  constexpr int TB = TN / 64;                   // 32-token blocks per wave
  constexpr int XJ = TN / 128;                  // token-row DMA instructions per wave per stage
  constexpr int kOperandX = TN * kQRow;
  constexpr int kStage = kQOperandW + kOperandX;
  constexpr int kPerStage = 2 + XJ;             // DMA instructions per wave per stage
  constexpr int kPair = D / 64;                 // waves per head
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kQBufs * kStage];

  // ---- placement: groups of kQGroupM token tiles x every feature tile ----
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int per_group = kQGroupM * a.n_tiles_n;
  const int first_m = (logical / per_group) * kQGroupM;
  const int gsize = min(a.n_tiles_m - first_m, kQGroupM);
  const int in_group = logical % per_group;
  const int tok0 = (first_m + in_group % gsize) * TN;
  const int feat0 = (in_group / gsize) * kQTileF;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lcol = lane & 31, lhalf = lane >> 5;
  const int wf = wave & 3;   // feature group
  const int wt = wave >> 2;  // token half
  const int fbase = D * (wf / kPair) + 32 * (wf % kPair);  // first feature of the group in the tile
  const int n_feat = a.nq + 2 * a.nkv;

  // ---- DMA roles: wave w copies weight rows 32w .. 32w + 31 and token rows
  // (TN / 8) w .. (TN / 8) (w + 1) - 1 ----
  const int frow = feat0 + 32 * wave;  // never straddles q/k/v (boundaries are multiples of 128)
  int which = 0, local = frow;
  if (frow >= a.nq + a.nkv) {
    which = 2;
    local = frow - a.nq - a.nkv;
  } else if (frow >= a.nq) {
    which = 1;
    local = frow - a.nq;
  }
  const int64_t rows_left = frow >= n_feat ? 0 : (which == 0 ? a.nq : a.nkv) - local;
  const u32x4 srd_w = make_srd(a.w[which] + static_cast<int64_t>(local) * a.hidden,
                               rows_left * a.hidden * 2);
  const int trow = tok0 + (TN / 8) * wave;
  const u32x4 srd_x = make_srd(a.x + static_cast<int64_t>(trow) * a.x_ss,
                               trow >= a.tokens ? 0 : (static_cast<int64_t>(a.tokens - trow) * a.x_ss * 2));
  uint32_t w_voff[2], x_voff[XJ];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * j + (lane >> 2);        // row within the wave's 32 weight rows
    const int tr = 32 * wave + r;              // row within the tile (swizzle key)
    w_voff[j] = static_cast<uint32_t>(r * a.hidden * 2) + (((lane & 3) ^ qswz(tr)) << 4);
  }
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int r = 16 * j + (lane >> 2);        // row within the wave's token rows
    const int tr = (TN / 8) * wave + r;
    x_voff[j] = static_cast<uint32_t>(r * a.x_ss * 2) + (((lane & 3) ^ qswz(tr)) << 4);
  }
  const uint32_t lds0 = lds_offset(lds);
  // DMA instruction j (< kPerStage) of stage st into buffer buf: weight rows first.
  auto issue_one = [&](int st, int buf, int j) __attribute__((always_inline)) {
    const uint32_t kb = static_cast<uint32_t>(st) * kQRow;
    if (j < 2) {
      dma16(srd_w, w_voff[j] + kb, lds0 + buf * kStage + wave * (32 * kQRow) + j * 1024);
    } else {
      dma16(srd_x, x_voff[j - 2] + kb, lds0 + buf * kStage + kQOperandW + wave * ((TN / 8) * kQRow) + (j - 2) * 1024);
    }
  };
  auto issue = [&](int st, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kPerStage; ++j) issue_one(st, buf, j);
  };

  // ---- fragment read offsets (bytes within a stage buffer) ----
  // Rows 32 tb and D/2 i apart share the swizzle key ((r >> 2) & 3 is unchanged by a
  // multiple of 16), so one offset per sub-step and operand serves every block.
  uint32_t w_rd[2], x_rd[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int c = 2 * s + lhalf;
    const int rw = fbase + lcol;
    w_rd[s] = rw * kQRow + ((c ^ qswz(rw)) << 4);
    const int rx = (TN / 2) * wt + lcol;
    x_rd[s] = kQOperandW + rx * kQRow + ((c ^ qswz(rx)) << 4);
  }
  constexpr uint32_t kWStep = (D / 2) * kQRow, kXStep = 32 * kQRow;
  static_assert((D / 2) % 16 == 0, "swizzle key shared across the weight blocks");

  f32x16 acc[2][TB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][tb][r] = 0.f;

  const int n_st = a.hidden / kQK;
  if (n_st > 0) issue(0, 0);
  if (n_st > 1) issue(1, 1);
  if (n_st > 2) issue(2, 2);

  // Stage st resident for every wave: this wave's DMA of it done (at most the stages
  // issued after it still in flight), this wave's reads of older stages done, then the
  // barrier.
  auto sync_stage = [&](int st) __attribute__((always_inline)) {
    const int after = min(2, max(0, n_st - 1 - st));
    if (after >= 2) wait_vmcnt<2 * kPerStage>();
    else if (after == 1) wait_vmcnt<kPerStage>();
    else wait_vmcnt<0>();
    wait_lgkmcnt0();
    __syncthreads();
  };
  auto rd = [&](int bf, uint32_t off) __attribute__((always_inline)) {
    return __builtin_bit_cast(frag, *reinterpret_cast<const u32x4*>(lds + bf * kStage + off));
  };
  // MFMA (flat index over the stage) after which the next stage's barrier sits: after the
  // last DMA instruction and at least two token blocks into the second K half.
  constexpr int kMidA = 3 * (kPerStage - 1) + 1 > 2 * TB + 3 ? 3 * (kPerStage - 1) + 1 : 2 * TB + 3;
  constexpr int kMid = kMidA % 2 ? kMidA : kMidA + 1;
  constexpr int kMidTb = (kMid - 2 * TB) / 2;  // last second-half token block before it
  static_assert(kMid < 4 * TB, "barrier inside the stage");
  static_assert(3 * (kPerStage - 1) + 1 < 4 * TB, "every DMA instruction issued inside the stage");

  frag w0[2], x0[TB];  // first-half fragments of the current stage, read ahead
  if (n_st > 0) {
    sync_stage(0);
#pragma unroll
    for (int i = 0; i < 2; ++i) w0[i] = rd(0, w_rd[0] + i * kWStep);
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) x0[tb] = rd(0, x_rd[0] + tb * kXStep);
  }
  // compute(st, bufc): the MFMAs of stage st (buffer bufc).  The DMA of stage st + 3 (into
  // buffer (bufc + 3) & 3, last read in stage st - 1, before this stage's barrier) is
  // spread through them, one instruction after every third MFMA from the second, so the
  // waves' address traffic does not queue at the stage start.
  auto compute = [&](int st, auto bufc) __attribute__((always_inline)) {
    constexpr int bf = decltype(bufc)::value;
    constexpr int nb = (bf + 1) & 3;
    const int pf = st + 3 < n_st ? st + 3 : -1;
    auto dma_after = [&](int m) __attribute__((always_inline)) {
      if (m % 3 == 1 && m / 3 < kPerStage && pf >= 0) {
        __builtin_amdgcn_sched_barrier(0);
        issue_one(pf, (bf + 3) & 3, m / 3);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    frag w1[2], x1[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      if (tb == TB - 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i) w1[i] = rd(bf, w_rd[1] + i * kWStep);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        acc[i][tb] = Ops::mma(w0[i], x0[tb], acc[i][tb]);
        dma_after(2 * tb + i);
      }
      x1[tb] = rd(bf, x_rd[1] + tb * kXStep);
    }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int m = 2 * TB + 2 * tb + i;
        acc[i][tb] = Ops::mma(w1[i], x1[tb], acc[i][tb]);
        dma_after(m);
        if (m == kMid) {  // after the last stage: an extra barrier and unused reads
          sync_stage(st + 1);
#pragma unroll
          for (int j = 0; j < 2; ++j) w0[j] = rd(nb, w_rd[0] + j * kWStep);
#pragma unroll
          for (int t = 0; t <= kMidTb; ++t) x0[t] = rd(nb, x_rd[0] + t * kXStep);
        }
      }
      if (tb > kMidTb) x0[tb] = rd(nb, x_rd[0] + tb * kXStep);
    }
  };
  for (int st = 0; st < n_st; st += kQBufs) {
    compute(st, IntC<0>{});
    if (st + 1 < n_st) compute(st + 1, IntC<1>{});
    if (st + 2 < n_st) compute(st + 2, IntC<2>{});
    if (st + 3 < n_st) compute(st + 3, IntC<3>{});
  }

  // ---- epilogue ----
  const int fw0 = feat0 + fbase;     // first feature of this wave
  if (fw0 >= n_feat) return;
  int ow = 0, of = fw0;              // output tensor and its feature offset
  if (fw0 >= a.nq + a.nkv) {
    ow = 2;
    of = fw0 - a.nq - a.nkv;
  } else if (fw0 >= a.nq) {
    ow = 1;
    of = fw0 - a.nq;
  }
  const uint16_t* bias = a.bias[ow];
  const bool rot = a.rope && ow < 2;
  const int head = of / D;
  const int dh = of % D;             // head dim of block 0 (block 1 is dh + D/2)
  // 16-byte stores need every row start 16-byte aligned
  const bool st16 = (ow == 0 || a.pool == nullptr)
                        ? ((reinterpret_cast<uintptr_t>(a.out[ow]) | static_cast<uintptr_t>(a.out_hs[ow]) * 2 |
                            static_cast<uintptr_t>(a.out_ss[ow]) * 2) % 16) == 0
                        : reinterpret_cast<uintptr_t>(a.pool) % 16 == 0;
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int t = tok0 + (TN / 2) * wt + 32 * tb + lcol;
    if (t >= a.tokens) continue;
    float v[2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lf = (D / 2) * i + 8 * (r >> 2) + 4 * lhalf + (r & 3);
        v[i][r] = acc[i][tb][r] + (bias ? ld16<DT>(bias + of + lf) : 0.f);
      }
    if (rot) {
      const int64_t p = a.pos[t];
      if (p < 0 || p >= a.rope_rows) {
        if (lhalf == 0) atomicOr(a.err, 4);
      } else {
        const float* crow = a.rope_cos + p * (D / 2);
        const float* srow = a.rope_sin + p * (D / 2);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = dh + 8 * g + 4 * lhalf;
          const float4 cs = *reinterpret_cast<const float4*>(crow + d0);
          const float4 sn = *reinterpret_cast<const float4*>(srow + d0);
          const float cc[4] = {cs.x, cs.y, cs.z, cs.w}, ss[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x1 = v[0][4 * g + i], x2 = v[1][4 * g + i];
            v[0][4 * g + i] = x1 * cc[i] - x2 * ss[i];
            v[1][4 * g + i] = x1 * ss[i] + x2 * cc[i];
          }
        }
      }
    }
    // store 4 consecutive head dims per (block, group)
    int32_t blk = 0;
    int64_t slot = 0;
    if (ow != 0 && a.pool != nullptr) {
      const int64_t sp = a.t0 + t - a.table_off;  // position of this token in the table
      const int64_t entry = sp / a.bs;
      blk = (sp >= 0 && entry < a.table_len) ? a.table[entry] : -1;
      if (blk < 0 || blk >= a.num_blocks) {
        if (lhalf == 0) atomicOr(a.err, 1);
        continue;
      }
      slot = sp - entry * a.bs;
    }
    uint16_t* row;
    if (ow == 0 || a.pool == nullptr) {
      row = a.out[ow] + head * a.out_hs[ow] + static_cast<int64_t>(t) * a.out_ss[ow];
    } else {
      row = a.pool + (ow == 2 ? a.plane_elems : 0) + ((static_cast<int64_t>(blk) * a.bs + slot) * a.hkv + head) * D;
    }
    u32x2 pk[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        pk[i][g][0] = pack2<DT>(v[i][4 * g], v[i][4 * g + 1]);
        pk[i][g][1] = pack2<DT>(v[i][4 * g + 2], v[i][4 * g + 3]);
      }
    if (st16) {
      // lanes 0-31 hold dims +0..3 of each 8-dim group, lanes 32-63 dims +4..7: after the
      // swap of groups (g, g + 1) lane lhalf = 0 holds all 8 dims of group g + 1 and
      // lhalf = 1 those of group g
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int g = 0; g < 4; g += 2) {
          u32x4 w;
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const auto r = __builtin_amdgcn_permlane32_swap(pk[i][g + 1][k], pk[i][g][k], false, false);
            w[k] = r[0];
            w[2 + k] = r[1];
          }
          const int gs = g + 1 - lhalf;
          *reinterpret_cast<u32x4*>(row + dh + (D / 2) * i + 8 * gs) = w;
        }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<u32x2*>(row + dh + (D / 2) * i + 8 * g + 4 * lhalf) = pk[i][g];
    }
  }
}

constexpr int kRopeThreads = 256;
struct RopeArgs {
  float inv_freq[128];
  int32_t half;
  int64_t rows;
  float* cos;
  float* sin;
};

__global__ __launch_bounds__(kRopeThreads) void rope_table_kernel(RopeArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  if (i >= a.rows * a.half) return;
  const int64_t m = i / a.half;
  const int j = static_cast<int>(i - m * a.half);
  // positions are exact in fp32 below 2^24; angle = m * inv_freq[j] in fp32
  const float ang = static_cast<float>(m) * a.inv_freq[j];
  a.cos[i] = cosf(ang);
  a.sin[i] = sinf(ang);
}

}  // namespace

void launch_rope_table(int d, int64_t rows, double base, float* cos, float* sin, hipStream_t stream) {
  require(d % 2 == 0 && d / 2 <= 128, "rope: head_dim must be even and <= 256");
  RopeArgs a{};
  a.half = d / 2;
  for (int j = 0; j < a.half; ++j)  // rotary.rs:72-78: 1 / base^(2j / dim) in f64, then f32
    a.inv_freq[j] = static_cast<float>(1.0 / std::pow(base, (2.0 * j) / d));
  a.rows = rows;
  a.cos = cos;
  a.sin = sin;
  const int64_t n = rows * a.half;
  if (n == 0) return;
  rope_table_kernel<<<static_cast<unsigned>(ceil_div(n, kRopeThreads)), kRopeThreads, 0, stream>>>(a);
  HCP_HIP(hipGetLastError());
}

// Token tile TN in {128, 256, 384}: the one with the least modelled time, i.e. rounds
// of workgroups over the device's compute units times the time one tile of that size
// takes relative to TN = 256 (0.62 and 1.41: bigger tiles reuse each LDS fragment more),
// a partly filled last round counted as 0.5 + 0.5 x its fill (it runs at a higher clock
// with part of the chip idle).  Fitted to a sweep of the Llama-3-8B projection over
// 1024-24576 tokens on MI355X, where it picks the fastest tile at every count (the
// earlier model, 1.57 and whole rounds, missed 4096, 6144 and 24576 tokens by 7-12%).
// Llama-3-8B at 12288 tokens: 768 tiles of 384 are 3 full rounds of 256 CUs.
static int qkv_token_tile(int64_t tiles_f, int64_t tokens) {
  int dev = 0, cus = 0;
  HCP_HIP(hipGetDevice(&dev));
  HCP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (cus <= 0) return 256;
  const int tn[3] = {128, 256, 384};
  const double cost[3] = {0.62, 1.0, 1.41};
  int best = 1;
  double best_t = 0.0;
  for (int i = 0; i < 3; ++i) {
    const int64_t tiles = tiles_f * ceil_div(tokens, tn[i]);
    const int64_t full = tiles / cus;
    const double fill = static_cast<double>(tiles - full * cus) / cus;
    const double t = (static_cast<double>(full) + (fill > 0.0 ? 0.5 + 0.5 * fill : 0.0)) * cost[i];
    if (i == 0 || t < best_t - 1e-9 || (i == 1 && t <= best_t + 1e-9)) {
      best = i;
      best_t = t;
    }
  }
  return tn[best];
}

void launch_qkv_rope(int dtype, int d, QkvArgs& a, hipStream_t stream) {
  const int n_feat = a.nq + 2 * a.nkv;
  a.n_tiles_n = static_cast<int32_t>(ceil_div(n_feat, kQTileF));
  const int tn = qkv_token_tile(a.n_tiles_n, a.tokens);
  a.n_tiles_m = static_cast<int32_t>(ceil_div(a.tokens, tn));
  const unsigned grid = static_cast<unsigned>(a.n_tiles_n * a.n_tiles_m);
  if (grid == 0) return;
  auto go = [&](auto tnc) {
    constexpr int TN = decltype(tnc)::value;
    if (dtype == kBF16) {
      if (d == 128) qkv_rope_kernel<kBF16, 128, TN><<<grid, kQThreads, 0, stream>>>(a);
      else qkv_rope_kernel<kBF16, 64, TN><<<grid, kQThreads, 0, stream>>>(a);
    } else {
      if (d == 128) qkv_rope_kernel<kF16, 128, TN><<<grid, kQThreads, 0, stream>>>(a);
      else qkv_rope_kernel<kF16, 64, TN><<<grid, kQThreads, 0, stream>>>(a);
    }
  };
  if (tn == 128) go(IntC<128>{});
  else if (tn == 384) go(IntC<384>{});
  else go(IntC<256>{});
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
