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
//     block.  A workgroup computes 256 features x 256 tokens with 8 waves of
//     128 features x 64 tokens: a wave's 128 features are one head (D = 128) or two
//     (D = 64), so the RoPE partners d and d + D/2 sit in the same lane and register
//     slot of blocks b and b + D/64 -- the rotation needs no data exchange.
//   * Weight and token tiles of 32 hidden values reach LDS through buffer_load ... lds
//     (four buffers, three stages in flight, one barrier per stage); chunk p of tile row
//     r holds global chunk p ^ ((r >> 2) & 3), which keeps the fragment reads free of
//     bank conflicts.
//   * Epilogue, in fp32: + bias, rotate (x1 cos - x2 sin, x1 sin + x2 cos) with cos/sin
//     from the table row of the token's position, round once to the storage dtype and
//     store 4 consecutive head dims (8 bytes) per lane: q into [Hq, L, D], k / v into
//     [Hkv, L, D] views or appended to the paged pool through the block table.
#include <cmath>

#include "kernels.hpp"
#include "lds_dma.hpp"

namespace hcp {


namespace {

constexpr int kQWaves = 8;
constexpr int kQThreads = kQWaves * 64;
constexpr int kQTile = 256;                  // features and tokens per workgroup
constexpr int kQK = 32;                      // hidden values per stage
constexpr int kQRow = kQK * 2;               // bytes per tile row in LDS
constexpr int kQOperand = kQTile * kQRow;    // 16 KiB
constexpr int kQStage = 2 * kQOperand;       // weights then tokens
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
  if constexpr (DT == kBF16) return static_cast<uint32_t>(f32_to_bf16_bits(a)) | (static_cast<uint32_t>(f32_to_bf16_bits(b)) << 16);
  else return static_cast<uint32_t>(f32_to_f16_bits(a)) | (static_cast<uint32_t>(f32_to_f16_bits(b)) << 16);
}

template <int DT>
__device__ __forceinline__ float ld16(const uint16_t* p) {
  return DT == kBF16 ? bf16_bits_to_f32(*p) : f16_bits_to_f32(*p);
}

template <int DT, int D>
__global__ __launch_bounds__(kQThreads, 1) void qkv_rope_kernel(QkvArgs a) {
  using Ops = QkvMfma<DT>;
  using frag = typename Ops::frag;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kQBufs * kQStage];

  // ---- placement: groups of kQGroupM token tiles x every feature tile ----
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int per_group = kQGroupM * a.n_tiles_n;
  const int first_m = (logical / per_group) * kQGroupM;
  const int gsize = min(a.n_tiles_m - first_m, kQGroupM);
  const int in_group = logical % per_group;
  const int tok0 = (first_m + in_group % gsize) * kQTile;
  const int feat0 = (in_group / gsize) * kQTile;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lcol = lane & 31, lhalf = lane >> 5;
  const int wf = wave & 1;   // 128-feature half of the tile
  const int wt = wave >> 1;  // 64-token quarter of the tile
  const int n_feat = a.nq + 2 * a.nkv;

  // ---- DMA roles: wave w copies weight rows and token rows 32w .. 32w + 31 ----
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
  const int trow = tok0 + 32 * wave;
  const u32x4 srd_x = make_srd(a.x + static_cast<int64_t>(trow) * a.x_ss,
                               trow >= a.tokens ? 0 : (static_cast<int64_t>(a.tokens - trow) * a.x_ss * 2));
  uint32_t w_voff[2], x_voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * j + (lane >> 2);        // row within the wave's 32
    const int tr = 32 * wave + r;              // row within the tile (swizzle key)
    const uint32_t ch = ((lane & 3) ^ qswz(tr)) << 4;
    w_voff[j] = static_cast<uint32_t>(r * a.hidden * 2) + ch;
    x_voff[j] = static_cast<uint32_t>(r * a.x_ss * 2) + ch;
  }
  const uint32_t lds0 = lds_offset(lds);
  auto issue = [&](int st, int buf) __attribute__((always_inline)) {
    const uint32_t kb = static_cast<uint32_t>(st) * kQRow;
    const uint32_t base = lds0 + buf * kQStage + wave * (32 * kQRow);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(srd_w, w_voff[j] + kb, base + j * 1024);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(srd_x, x_voff[j] + kb, base + kQOperand + j * 1024);
  };

  // ---- fragment read offsets (bytes within a stage buffer) ----
  uint32_t w_rd[4][2], x_rd[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int c = 2 * s + lhalf;
#pragma unroll
    for (int fb = 0; fb < 4; ++fb) {
      const int r = 128 * wf + 32 * fb + lcol;
      w_rd[fb][s] = r * kQRow + ((c ^ qswz(r)) << 4);
    }
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const int r = 64 * wt + 32 * tb + lcol;
      x_rd[tb][s] = kQOperand + r * kQRow + ((c ^ qswz(r)) << 4);
    }
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int fb = 0; fb < 4; ++fb)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[fb][tb][r] = 0.f;

  const int n_st = a.hidden / kQK;
  if (n_st > 0) issue(0, 0);
  if (n_st > 1) issue(1, 1);
  if (n_st > 2) issue(2, 2);

  auto compute = [&](auto bufc) __attribute__((always_inline)) {
    constexpr int bf = decltype(bufc)::value;
    const uint8_t* L = lds + bf * kQStage;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      frag wfr[4], xfr[2];
#pragma unroll
      for (int fb = 0; fb < 4; ++fb) wfr[fb] = __builtin_bit_cast(frag, *reinterpret_cast<const u32x4*>(L + w_rd[fb][s]));
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) xfr[tb] = __builtin_bit_cast(frag, *reinterpret_cast<const u32x4*>(L + x_rd[tb][s]));
#pragma unroll
      for (int fb = 0; fb < 4; ++fb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) acc[fb][tb] = Ops::mma(wfr[fb], xfr[tb], acc[fb][tb]);
    }
  };
  auto step = [&](int st, auto bufc) __attribute__((always_inline)) {
    constexpr int bf = decltype(bufc)::value;
    // Stage st is resident once at most the stages issued after it are in flight.
    const int after = min(2, n_st - 1 - st);
    if (after >= 2) wait_vmcnt<8>();
    else if (after == 1) wait_vmcnt<4>();
    else wait_vmcnt<0>();
    __syncthreads();  // stage st visible; every wave is done with stage st - 1's buffer
    if (st + 3 < n_st) issue(st + 3, (bf + 3) & 3);
    compute(bufc);
  };
  for (int st = 0; st < n_st; st += kQBufs) {
    step(st, IntC<0>{});
    if (st + 1 < n_st) step(st + 1, IntC<1>{});
    if (st + 2 < n_st) step(st + 2, IntC<2>{});
    if (st + 3 < n_st) step(st + 3, IntC<3>{});
  }

  // ---- epilogue ----
  const int fw0 = feat0 + 128 * wf;  // first feature of this wave
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
  constexpr int kPair = D / 64;  // block distance of the RoPE partner
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const int t = tok0 + 64 * wt + 32 * tb + lcol;
    if (t >= a.tokens) continue;
    float v[4][16];
#pragma unroll
    for (int fb = 0; fb < 4; ++fb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lf = 32 * fb + 8 * (r >> 2) + 4 * lhalf + (r & 3);
        v[fb][r] = acc[fb][tb][r] + (bias ? ld16<DT>(bias + of + lf) : 0.f);
      }
    if (rot) {
      const int64_t p = a.pos[t];
      if (p < 0 || p >= a.rope_rows) {
        if (lhalf == 0) atomicOr(a.err, 4);
      } else {
        const float* crow = a.rope_cos + p * (D / 2);
        const float* srow = a.rope_sin + p * (D / 2);
#pragma unroll
        for (int fb = 0; fb < 4; ++fb) {
          if ((fb / kPair) % 2 != 0) continue;  // first half of a head
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d0 = (32 * fb + 8 * g + 4 * lhalf) % D;
            const float4 cs = *reinterpret_cast<const float4*>(crow + d0);
            const float4 sn = *reinterpret_cast<const float4*>(srow + d0);
            const float cc[4] = {cs.x, cs.y, cs.z, cs.w}, ss[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float x1 = v[fb][4 * g + i], x2 = v[fb + kPair][4 * g + i];
              v[fb][4 * g + i] = x1 * cc[i] - x2 * ss[i];
              v[fb + kPair][4 * g + i] = x1 * ss[i] + x2 * cc[i];
            }
          }
        }
      }
    }
    // store 4 consecutive head dims per (block, group)
#pragma unroll
    for (int fb = 0; fb < 4; ++fb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int f = of + 32 * fb + 8 * g + 4 * lhalf;
        const int head = f / D, d0 = f % D;
        u32x2 pk;
        pk[0] = pack2<DT>(v[fb][4 * g], v[fb][4 * g + 1]);
        pk[1] = pack2<DT>(v[fb][4 * g + 2], v[fb][4 * g + 3]);
        uint16_t* dst;
        if (ow == 0 || a.pool == nullptr) {
          dst = a.out[ow] + head * a.out_hs[ow] + static_cast<int64_t>(t) * a.out_ss[ow] + d0;
        } else {
          const int64_t sp = a.t0 + t - a.table_off;  // position of this token in the table
          const int64_t entry = sp / a.bs;
          const int32_t blk = (sp >= 0 && entry < a.table_len) ? a.table[entry] : -1;
          if (blk < 0 || blk >= a.num_blocks) {
            if (lhalf == 0 && g == 0 && fb == 0) atomicOr(a.err, 1);
            continue;
          }
          dst = a.pool + (ow == 2 ? a.plane_elems : 0) +
                ((static_cast<int64_t>(blk) * a.bs + (sp - entry * a.bs)) * a.hkv + head) * D + d0;
        }
        *reinterpret_cast<u32x2*>(dst) = pk;
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

void launch_qkv_rope(int dtype, int d, QkvArgs& a, hipStream_t stream) {
  const int n_feat = a.nq + 2 * a.nkv;
  a.n_tiles_n = static_cast<int32_t>(ceil_div(n_feat, kQTile));
  a.n_tiles_m = static_cast<int32_t>(ceil_div(a.tokens, kQTile));
  const unsigned grid = static_cast<unsigned>(a.n_tiles_n * a.n_tiles_m);
  if (grid == 0) return;
  if (dtype == kBF16) {
    if (d == 128) qkv_rope_kernel<kBF16, 128><<<grid, kQThreads, 0, stream>>>(a);
    else qkv_rope_kernel<kBF16, 64><<<grid, kQThreads, 0, stream>>>(a);
  } else {
    if (d == 128) qkv_rope_kernel<kF16, 128><<<grid, kQThreads, 0, stream>>>(a);
    else qkv_rope_kernel<kF16, 64><<<grid, kQThreads, 0, stream>>>(a);
  }
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
