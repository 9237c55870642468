// Asynchronous global -> LDS loads and workgroup placement helpers shared by the
// matrix-core kernels (gfx950).
#pragma once

#include "hcp_common.hpp"

namespace hcp {

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// Buffer descriptor as four SGPRs (base, stride 0, num_records, flags): reads past the
// end return zeros.
__device__ __forceinline__ u32x4 make_srd(const void* base, int64_t bytes) {
  const uint32_t n = bytes <= 0 ? 0u : (bytes > 0x7ffffff0LL ? 0x7ffffff0u : static_cast<uint32_t>(bytes));
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane(n);
  r[3] = 0x00020000u;
  return r;
}

// One wave-wide 16-byte-per-lane load straight into LDS at lds_addr + 16 * lane.  The
// compiler does not track it: callers wait with s_waitcnt vmcnt themselves (the
// compiler's own LDS-DMA builtin makes it wait for every DMA before any read of the same
// LDS array, which would serialise the kernels' multi-buffer pipelines).  M0 is set and
// consumed inside the statement; clang warns that a clobber of the reserved M0 is not
// preserved around it.  That is harmless only while the compiler keeps no value of its
// own in M0, so the build (build.py, check_m0) disassembles every object that includes
// this header and fails if any instruction other than this statement's three touches M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(u32x4 srd, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(srd), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
// The same load with the nt (streaming) cache-policy bit, for data each workgroup reads
// once and no other workgroup reads again (the KV staging gather: +2.2% on c5).
__device__ __forceinline__ void dma16_nt(u32x4 srd, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :
               : "v"(voff), "s"(srd), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N) for N < 64 (vmcnt bits [3:0] and [15:14]); expcnt and lgkmcnt
// left unconstrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0): this wave's LDS reads have returned; vmcnt and expcnt left
// unconstrained.
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

template <int V>
struct IntC {
  static constexpr int value = V;
};

// Map blockIdx.x so that each XCD (blocks are dealt round-robin over 8 XCDs) gets a
// contiguous range of logical tiles: neighbouring tiles share data in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int kXcd = 8;
  const int per = nblocks / kXcd;
  const int rem = nblocks % kXcd;
  const int xcd = bid % kXcd;
  const int idx = bid / kXcd;
  const int start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
  return start + idx;
}

}  // namespace hcp
