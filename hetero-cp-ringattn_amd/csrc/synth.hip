// Synthetic normal inputs on the device (benchmark data; no reference counterpart).
//
// Same stream as the reference's correctness model (rust/src/smoke/reference_algo.rs:56-90):
// state_{n+1} = a*state_n + c (mod 2^64), u = ((state >> 11) + 0.5) / 2^53, Box-Muller
// pairs (r cos, r sin).  Normal 2j and 2j+1 come from LCG draws 2j+1 and 2j+2 after the
// seed.  Each thread jumps straight to its first pair (A^k, C_k by square-and-multiply)
// and then steps the LCG for a run of consecutive pairs.
#include "kernels.hpp"

namespace hcp {

constexpr uint64_t kLcgA = 6364136223846793005ULL;
constexpr uint64_t kLcgC = 1442695040888963407ULL;
constexpr int kPairsPerThread = 64;

// State after k steps from s: A^k s + c (A^{k-1} + ... + 1).
__device__ uint64_t lcg_jump(uint64_t s, uint64_t k) {
  uint64_t acc_mul = 1, acc_add = 0;
  uint64_t cur_mul = kLcgA, cur_add = kLcgC;
  while (k) {
    if (k & 1) {
      acc_mul *= cur_mul;
      acc_add = acc_add * cur_mul + cur_add;
    }
    cur_add = cur_add * (cur_mul + 1);
    cur_mul *= cur_mul;
    k >>= 1;
  }
  return acc_mul * s + acc_add;
}

__device__ __forceinline__ double open01(uint64_t st) {
  return (static_cast<double>(st >> 11) + 0.5) / 9007199254740992.0;
}

template <int DT>
__global__ __launch_bounds__(256) void synth_normals_kernel(uint64_t seed, int64_t offset, int64_t count,
                                                            void* out) {
  const int64_t first_pair = offset / 2;
  const int64_t last_pair = (offset + count - 1) / 2;
  const int64_t run = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t p0 = first_pair + run * kPairsPerThread;
  if (p0 > last_pair) return;
  uint64_t st = lcg_jump(seed, static_cast<uint64_t>(2 * p0));
  for (int i = 0; i < kPairsPerThread; ++i) {
    const int64_t pair = p0 + i;
    if (pair > last_pair) break;
    st = st * kLcgA + kLcgC;
    const double u1 = open01(st);
    st = st * kLcgA + kLcgC;
    const double u2 = open01(st);
    const double r = sqrt(-2.0 * log(u1));
    const double th = 2.0 * 3.14159265358979323846 * u2;
    const double z[2] = {r * cos(th), r * sin(th)};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t n = 2 * pair + h;
      if (n < offset || n >= offset + count) continue;
      const float f = static_cast<float>(z[h]);
      store_elem<DT>(out, n - offset, f);
    }
  }
}

void launch_synth_normals(uint64_t seed, int64_t offset, int64_t count, int dtype, void* out,
                          hipStream_t stream) {
  if (count <= 0) return;
  const int64_t pairs = (offset + count - 1) / 2 - offset / 2 + 1;
  const int64_t threads = ceil_div(pairs, kPairsPerThread);
  const dim3 grid(static_cast<unsigned>(ceil_div(threads, 256)));
  switch (dtype) {
    case kF32: synth_normals_kernel<kF32><<<grid, 256, 0, stream>>>(seed, offset, count, out); break;
    case kBF16: synth_normals_kernel<kBF16><<<grid, 256, 0, stream>>>(seed, offset, count, out); break;
    case kF16: synth_normals_kernel<kF16><<<grid, 256, 0, stream>>>(seed, offset, count, out); break;
    default: throw Error(-6, "synth_normals: dtype must be F32, BF16 or F16");
  }
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
