// Shared definitions for the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace hcp {

// bf16 / fp16 vectors as the gfx950 MFMA builtins take them.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

enum DType : int32_t { kF16 = 1, kBF16 = 2, kF32 = 3, kI32 = 4, kI64 = 5 };

// Error raised inside the library; the C-ABI layer turns it into a status code.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    throw Error(-5, std::string(what) + ": " + hipGetErrorString(e));
  }
}

#define HCP_HIP(expr) ::hcp::hip_check((expr), #expr)

inline void require(bool ok, const std::string& msg) {
  if (!ok) throw Error(-6, msg);
}

// Sticky device-side error flags (bit 0: paged block id out of range; bit 1: key
// positions not non-decreasing).
// Defined in capi.hip; kernels set bits with atomicOr through this pointer
// argument resolved once per device by the host (hipGetSymbolAddress).
int* device_error_flags();

// ---- scalar conversions (device) ----
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits through gfx950's v_cvt_pk_bf16_f32: the same
// bits as (u + 0x7fff + ((u >> 16) & 1)) >> 16 for every non-NaN input and the quieted
// (u >> 16) | 0x40 for NaNs (all 2^32 inputs compared on the device).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two values in one instruction: lo in bits 0-15, hi in bits 16-31.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// Global stores with the nt and sc1 cache-policy bits (streamed, written back at system
// scope), for write streams nothing reads again in the same kernel.  Measured in
// same-run A/Bs: KV staging scatter +3.5% and gather +2.7% over nt alone (c5; sc1 alone
// +3%, sc0 alone +0.7%), wire-frame pack +13.5% and unpack +6.3% over plain stores, LSE
// merge +3.2%.
// On gfx940+ a VALU write to the data VGPRs of a VMEM store wider than 64 bits needs
// two wait states after the store; the compiler's hazard recognizer does not see
// stores inside inline asm, so the 16-byte form provides them itself (s_nop 1).
__device__ __forceinline__ void store16_nt_sc1(void* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off nt sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store8_nt_sc1(void* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off nt sc1" : : "v"(p), "v"(v) : "memory");
}

// Element load/store by dtype (used by the general kernels).
template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i);
template <>
__device__ __forceinline__ float load_elem<kF32>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <>
__device__ __forceinline__ float load_elem<kBF16>(const void* p, int64_t i) {
  return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <>
__device__ __forceinline__ float load_elem<kF16>(const void* p, int64_t i) {
  return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v);
template <>
__device__ __forceinline__ void store_elem<kF32>(void* p, int64_t i, float v) {
  static_cast<float*>(p)[i] = v;
}
template <>
__device__ __forceinline__ void store_elem<kBF16>(void* p, int64_t i, float v) {
  static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
}
template <>
__device__ __forceinline__ void store_elem<kF16>(void* p, int64_t i, float v) {
  static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
}
// Store with the dtype chosen at run time.
__device__ __forceinline__ void store_elem_rt(void* p, int dtype, int64_t i, float v) {
  if (dtype == kF32) store_elem<kF32>(p, i, v);
  else if (dtype == kBF16) store_elem<kBF16>(p, i, v);
  else store_elem<kF16>(p, i, v);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace hcp
