// LSE merge of ring-step partials (closed form of the re-entry merge in
// positioned_merge_compact_partial / decode_merge_packet, ring.rs:574-603, :647-663):
//   m = max_i lse_i,  w_i = e^(lse_i - m),
//   o = sum_i w_i o_i / sum_i w_i,  lse = m + ln sum_i w_i,  all -inf -> (0, -inf).
//
// Layout: each partial is o [H, L, D] fp32 and lse [H, L] fp32 (as the block kernel
// writes them).  One row (h, t) = D fp32 is handled by D/4 lanes with 16-byte loads,
// so a wavefront covers 64*4/D rows per instruction; the per-row max/sum over the n
// partials runs in every lane of the row (n is small), the row's lse is loaded once
// per lane group.  HBM-bound: algorithmic bytes per row = n*(4D + 4) read +
// (D*out_bytes + 4) written.
#include "kernels.hpp"

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

template <int OUT_DT>
__global__ __launch_bounds__(256) void lse_merge_kernel(MergeArgs a) {
  const int lpr = a.lanes_per_row;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / lpr;
  const int lane_in_row = threadIdx.x % lpr;
  const int64_t rows = static_cast<int64_t>(a.heads) * a.q_len;
  if (row >= rows) return;
  const int64_t h = row / a.q_len;
  const int64_t t = row - h * a.q_len;
  const int n = a.n;

  float m = -INFINITY;
  for (int i = 0; i < n; ++i) m = fmaxf(m, a.lse[i][row]);
  const bool any = m != -INFINITY;
  const float m_safe = any ? m : 0.f;

  const int c = lane_in_row * 4;
  const bool active = c < a.d;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float den = 0.f;
  int i = 0;
  // Four partials in flight per step.
  for (; i + 4 <= n; i += 4) {
    float l4[4];
    float4 v4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      l4[u] = a.lse[i + u][row];
      v4[u] = active ? *reinterpret_cast<const float4*>(a.o[i + u] + row * a.d + c)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float w = __expf(l4[u] - m_safe);  // exp(-inf) = 0 for empty partials
      den += w;
      acc.x += w * v4[u].x;
      acc.y += w * v4[u].y;
      acc.z += w * v4[u].z;
      acc.w += w * v4[u].w;
    }
  }
  for (; i < n; ++i) {
    const float l = a.lse[i][row];
    const float4 v = active ? *reinterpret_cast<const float4*>(a.o[i] + row * a.d + c)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    const float w = __expf(l - m_safe);
    den += w;
    acc.x += w * v.x;
    acc.y += w * v.y;
    acc.z += w * v.z;
    acc.w += w * v.w;
  }
  const float inv = (any && den > 0.f) ? 1.f / den : 0.f;
  if (active) {
    const int64_t base = h * a.out_hs + t * a.out_ss + c;
    if constexpr (OUT_DT == kF32) {
      *reinterpret_cast<float4*>(static_cast<float*>(a.out) + base) =
          make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    } else {
      uint16_t b0, b1, b2, b3;
      if constexpr (OUT_DT == kBF16) {
        b0 = f32_to_bf16_bits(acc.x * inv);
        b1 = f32_to_bf16_bits(acc.y * inv);
        b2 = f32_to_bf16_bits(acc.z * inv);
        b3 = f32_to_bf16_bits(acc.w * inv);
      } else {
        b0 = f32_to_f16_bits(acc.x * inv);
        b1 = f32_to_f16_bits(acc.y * inv);
        b2 = f32_to_f16_bits(acc.z * inv);
        b3 = f32_to_f16_bits(acc.w * inv);
      }
      uint2 packed;
      packed.x = static_cast<uint32_t>(b0) | (static_cast<uint32_t>(b1) << 16);
      packed.y = static_cast<uint32_t>(b2) | (static_cast<uint32_t>(b3) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + base) = packed;
    }
  }
  if (a.lse_out != nullptr && lane_in_row == 0) {
    a.lse_out[h * a.lse_out_hs + t] = (any && den > 0.f) ? m + __logf(den) : -INFINITY;
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
  const int64_t threads = static_cast<int64_t>(heads) * q_len * lpr;
  const dim3 grid(static_cast<unsigned>(ceil_div(threads, 256)));
  switch (out_dtype) {
    case kBF16: lse_merge_kernel<kBF16><<<grid, 256, 0, stream>>>(a); break;
    case kF16: lse_merge_kernel<kF16><<<grid, 256, 0, stream>>>(a); break;
    case kF32: lse_merge_kernel<kF32><<<grid, 256, 0, stream>>>(a); break;
    default: throw Error(-6, "lse_merge: out_dtype must be BF16, F16 or F32");
  }
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
