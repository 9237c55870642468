// LSE merge of ring-step partials (closed form of the re-entry merge in
// positioned_merge_compact_partial / decode_merge_packet, ring.rs:574-603, :647-663):
//   m = max_i lse_i,  w_i = e^(lse_i - m),
//   o = sum_i w_i o_i / sum_i w_i,  lse = m + ln sum_i w_i,  all -inf -> (0, -inf).
//
// Layout: each partial is o [H, L, D] fp32 and lse [H, L] fp32 (as the block kernel
// writes them).  One row (h, t) = D fp32 is handled by D/4 lanes with 16-byte loads,
// so a wavefront covers 64*4/D rows per instruction, and each thread takes two
// consecutive rows (measured +2-4% over one on the c3 partials; four: +2-3%).  The partials are folded in one
// pass, in groups of up to 8 whose loads are all in flight together, with the running
// max, sum and accumulator rescaled when a group raises the max (the same closed form,
// grouped).  HBM-bound: algorithmic bytes per row = n*(4D + 4) read + (D*out_bytes + 4)
// written.
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace hcp {

constexpr int kMaxMergeParts = 64;

struct MergeArgs {
  const float* o[kMaxMergeParts];
  const float* lse[kMaxMergeParts];
  int32_t n;
  int32_t heads;
  int64_t q_len;
  int32_t d;
  int32_t lanes_per_row;  // D/4 rounded up to a power of two
  void* out;
  int64_t out_hs, out_ss;  // elements
  float* lse_out;
  int64_t lse_out_hs;      // elements between heads of lse_out
};

// 16-byte streaming load: each partial is read once.
__device__ __forceinline__ float4 nt_load4(const float* p) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 x = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
  return make_float4(x[0], x[1], x[2], x[3]);
}

template <int OUT_DT, int NP, int R>
__global__ __launch_bounds__(256) void lse_merge_kernel(MergeArgs a) {
  const int lpr = a.lanes_per_row;
  // R consecutive rows per thread (same 16-byte column of each): R * NP loads in flight.
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / lpr * R;
  const int lane_in_row = threadIdx.x % lpr;
  const int64_t rows = static_cast<int64_t>(a.heads) * a.q_len;
  if (row0 >= rows) return;
  const int n = a.n;
  const int c = lane_in_row * 4;
  const bool active = c < a.d;

  // One pass over the partials in groups of NP: every load of a group (NP lse values
  // and NP 16-byte slices of o, for each of the R rows) is issued before any is used,
  // and the running (max, sum, acc) is rescaled when a group raises the max.
  float m[R], den[R];
  float4 acc[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    m[k] = -INFINITY;
    den[k] = 0.f;
    acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int base = 0; base < n; base += NP) {
    float l[R][NP];
    float4 v[R][NP];
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
      for (int u = 0; u < NP; ++u) {
        const bool in = base + u < n && row0 + k < rows;
        l[k][u] = in ? a.lse[base + u][row0 + k] : -INFINITY;
        v[k][u] = (in && active) ? nt_load4(a.o[base + u] + (row0 + k) * a.d + c)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      float mg = l[k][0];
#pragma unroll
      for (int u = 1; u < NP; ++u) mg = fmaxf(mg, l[k][u]);
      const float mn = fmaxf(m[k], mg);
      if (mn == -INFINITY) continue;  // every partial so far is empty
      const float sc = __expf(m[k] - mn);  // 0 while m = -inf
      den[k] *= sc;
      acc[k].x *= sc;
      acc[k].y *= sc;
      acc[k].z *= sc;
      acc[k].w *= sc;
#pragma unroll
      for (int u = 0; u < NP; ++u) {
        const float w = __expf(l[k][u] - mn);  // exp(-inf) = 0 for empty partials
        den[k] += w;
        acc[k].x += w * v[k][u].x;
        acc[k].y += w * v[k][u].y;
        acc[k].z += w * v[k][u].z;
        acc[k].w += w * v[k][u].w;
      }
      m[k] = mn;
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t row = row0 + k;
    if (row >= rows) break;
    const int64_t h = row / a.q_len;
    const int64_t t = row - h * a.q_len;
    const bool any = m[k] != -INFINITY;
    const float inv = (any && den[k] > 0.f) ? 1.f / den[k] : 0.f;
    if (active) {
      const int64_t base = h * a.out_hs + t * a.out_ss + c;
      if constexpr (OUT_DT == kF32) {
        store16_nt_sc1(static_cast<float*>(a.out) + base,
                       __builtin_bit_cast(u32x4, make_float4(acc[k].x * inv, acc[k].y * inv, acc[k].z * inv, acc[k].w * inv)));
      } else {
        uint16_t b0, b1, b2, b3;
        if constexpr (OUT_DT == kBF16) {
          b0 = f32_to_bf16_bits(acc[k].x * inv);
          b1 = f32_to_bf16_bits(acc[k].y * inv);
          b2 = f32_to_bf16_bits(acc[k].z * inv);
          b3 = f32_to_bf16_bits(acc[k].w * inv);
        } else {
          b0 = f32_to_f16_bits(acc[k].x * inv);
          b1 = f32_to_f16_bits(acc[k].y * inv);
          b2 = f32_to_f16_bits(acc[k].z * inv);
          b3 = f32_to_f16_bits(acc[k].w * inv);
        }
        uint2 packed;
        packed.x = static_cast<uint32_t>(b0) | (static_cast<uint32_t>(b1) << 16);
        packed.y = static_cast<uint32_t>(b2) | (static_cast<uint32_t>(b3) << 16);
        store8_nt_sc1(static_cast<uint16_t*>(a.out) + base, u32x2{packed.x, packed.y});
      }
    }
    if (a.lse_out != nullptr && lane_in_row == 0) {
      a.lse_out[h * a.lse_out_hs + t] = (any && den[k] > 0.f) ? m[k] + __logf(den[k]) : -INFINITY;
    }
  }
}

void launch_lse_merge(int n, const float* const* o_parts, const float* const* lse_parts,
                      int heads, int64_t q_len, int d, int out_dtype, void* out, int64_t out_hs,
                      int64_t out_ss, float* lse_out, int64_t lse_out_hs, hipStream_t stream) {
  require(n >= 1 && n <= kMaxMergeParts, "lse_merge: num_parts must be in [1, 64]");
  require(d % 4 == 0 && d <= 256, "lse_merge: head_dim must be a multiple of 4, <= 256");
  if (q_len == 0 || heads == 0) return;
  MergeArgs a;
  for (int i = 0; i < n; ++i) {
    a.o[i] = o_parts[i];
    a.lse[i] = lse_parts[i];
  }
  a.n = n;
  a.heads = heads;
  a.q_len = q_len;
  a.d = d;
  int lpr = 1;
  while (lpr < d / 4) lpr *= 2;
  a.lanes_per_row = lpr;
  a.out = out;
  a.out_hs = out_hs;
  a.out_ss = out_ss;
  a.lse_out = lse_out;
  a.lse_out_hs = lse_out_hs;
#ifndef HCP_MERGE_R
#define HCP_MERGE_R 2
#endif
  constexpr int R = HCP_MERGE_R;
  const int64_t threads = ceil_div(static_cast<int64_t>(heads) * q_len, R) * lpr;
  const dim3 grid(static_cast<unsigned>(ceil_div(threads, 256)));
  // Group size: all partials in one group up to 4, else groups of 8.
  auto go = [&](auto np) {
    constexpr int NP = decltype(np)::value;
    switch (out_dtype) {
      case kBF16: lse_merge_kernel<kBF16, NP, R><<<grid, 256, 0, stream>>>(a); break;
      case kF16: lse_merge_kernel<kF16, NP, R><<<grid, 256, 0, stream>>>(a); break;
      case kF32: lse_merge_kernel<kF32, NP, R><<<grid, 256, 0, stream>>>(a); break;
      default: throw Error(-6, "lse_merge: out_dtype must be BF16, F16 or F32");
    }
  };
  if (n == 1) go(IntC<1>{});
  else if (n == 2) go(IntC<2>{});
  else if (n <= 4) go(IntC<4>{});
  else go(IntC<8>{});
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
