// Wire frames of the ring transport: device-side pack / unpack of the tensor payload
// and the host-side frame header.
//
// The reference's TCP transport (rust/src/model/transport/tcp.rs:20-40,161-243,604-787)
// sends a KvBlock as
//     [meta_len: u32 BE][meta_json][k f32 LE][v f32 LE][position_ids i64 LE, optional]
// and a decode RingPacket as
//     [meta_len: u32 BE][meta_json][q f32 LE][o f32 LE][lse f32 LE]
// where every float tensor travels as the fp32 upcast of its contiguous [1, H, L, D]
// (resp. [B, H, 1, D], [B, H, 1]) view, the original dtype named in meta_json, and the
// JSON is serde_json's compact output of a map without key-order preservation, i.e.
// keys in sorted order (serde_json 1.0.149, rust/Cargo.lock; no "preserve_order").
//
// Here the payload (the bulk) is produced and consumed on the GPU straight from / into
// the ring buffers: the pack kernel reads K/V with the compact Hkv heads and writes the
// wire's expanded heads (the reference sends post-GQA-expand blocks, ring.rs:999-1019)
// as fp32; unpack converts back to the storage dtype (exact for values that were bf16
// or fp16) and keeps one copy of each expanded head group.  The header is built and
// parsed on the host.
#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "kernels.hpp"

namespace hcp {
namespace {

constexpr int kWireThreads = 256;

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == kF32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == kBF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, float x) {
  if constexpr (DT == kF32) static_cast<float*>(p)[i] = x;
  else if constexpr (DT == kBF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(x);
  else static_cast<_Float16*>(p)[i] = static_cast<_Float16>(x);
}

// Wire element (hw, t, d) of a [rows_wire, L, D] tensor <-> storage element
// (hw / rep, t, d) at base + (hw / rep) * hs + t * ss + d.  VEC consecutive d per thread.
struct WireSeg {
  void* tensor;       // storage view base
  float* wire;        // fp32 wire payload segment (16-byte aligned when VEC == 4)
  int64_t rows;       // wire rows (expanded heads or batch)
  int64_t rep;        // wire rows per storage row (GQA expand; 1 otherwise)
  int64_t len, dim;   // L, D
  int64_t hs, ss;     // storage strides (elements)
};

template <int DT, int VEC>
__global__ __launch_bounds__(kWireThreads) void wire_pack_kernel(WireSeg s) {
  const int64_t per_row = s.len * s.dim / VEC;
  const int64_t n = s.rows * per_row;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kWireThreads + threadIdx.x; g < n;
       g += static_cast<int64_t>(gridDim.x) * kWireThreads) {
    const int64_t hw = g / per_row;
    const int64_t e = (g - hw * per_row) * VEC;
    const int64_t t = e / s.dim, d = e - t * s.dim;
    const int64_t src = (hw / s.rep) * s.hs + t * s.ss + d;
    if constexpr (VEC == 4) {
      float4 v = make_float4(load_as_f32<DT>(s.tensor, src), load_as_f32<DT>(s.tensor, src + 1),
                             load_as_f32<DT>(s.tensor, src + 2), load_as_f32<DT>(s.tensor, src + 3));
      reinterpret_cast<float4*>(s.wire)[g] = v;
    } else {
      s.wire[g] = load_as_f32<DT>(s.tensor, src);
    }
  }
}

// Storage rows = rows / rep; storage row h reads wire row h * rep.
template <int DT, int VEC>
__global__ __launch_bounds__(kWireThreads) void wire_unpack_kernel(WireSeg s) {
  const int64_t per_row = s.len * s.dim / VEC;
  const int64_t n = (s.rows / s.rep) * per_row;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kWireThreads + threadIdx.x; g < n;
       g += static_cast<int64_t>(gridDim.x) * kWireThreads) {
    const int64_t h = g / per_row;
    const int64_t e = (g - h * per_row) * VEC;
    const int64_t t = e / s.dim, d = e - t * s.dim;
    const int64_t dst = h * s.hs + t * s.ss + d;
    const int64_t w = (h * s.rep * per_row) + (g - h * per_row);
    if constexpr (VEC == 4) {
      const float4 v = reinterpret_cast<const float4*>(s.wire)[w];
      store_from_f32<DT>(s.tensor, dst, v.x);
      store_from_f32<DT>(s.tensor, dst + 1, v.y);
      store_from_f32<DT>(s.tensor, dst + 2, v.z);
      store_from_f32<DT>(s.tensor, dst + 3, v.w);
    } else {
      store_from_f32<DT>(s.tensor, dst, s.wire[w]);
    }
  }
}

// Vectorised forms for 16-byte aligned rows (checked by the launcher), index arithmetic
// in 32 bits when it fits.  Pack: four consecutive d of one storage row per thread (one
// 8-byte load for 2-byte dtypes), stored to each of the row's rep expanded wire rows, so
// every store instruction of a wave writes one contiguous 1 KiB run (eight d per thread,
// two 16-byte stores 32 bytes apart per lane, measured 18% slower), with the nt + sc1
// cache policy (+13.5% over plain stores; nt alone was slower).  Unpack: eight d per
// thread from the first wire row of each group, one 16-byte store (four d per thread
// measured 7% slower).
template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float (&f)[8]) {
  if constexpr (DT == kF32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == kBF16) {
        f[2 * j] = __uint_as_float(w[j] << 16);
        f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      } else {
        f[2 * j] = f16_bits_to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
        f[2 * j + 1] = f16_bits_to_f32(static_cast<uint16_t>(w[j] >> 16));
      }
    }
  }
}
template <int DT>
__device__ __forceinline__ void store8(void* p, int64_t i, const float4& a, const float4& b) {
  if constexpr (DT == kF32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = a;
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i + 4) = b;
  } else {
    const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == kBF16)
        w[j] = f32x2_to_bf16x2_bits(f[2 * j], f[2 * j + 1]);
      else
        w[j] = static_cast<uint32_t>(f32_to_f16_bits(f[2 * j])) | (static_cast<uint32_t>(f32_to_f16_bits(f[2 * j + 1])) << 16);
    }
    store16_nt_sc1(static_cast<uint16_t*>(p) + i, u32x4{w[0], w[1], w[2], w[3]});
  }
}

template <int DT, typename I>
__global__ __launch_bounds__(kWireThreads) void wire_pack8_kernel(WireSeg s) {
  const I per_row = static_cast<I>(s.len * s.dim / 4);
  const I dim = static_cast<I>(s.dim);
  const I n = static_cast<I>(s.rows / s.rep) * per_row;
  for (I g = static_cast<I>(blockIdx.x) * kWireThreads + threadIdx.x; g < n;
       g += static_cast<I>(gridDim.x) * kWireThreads) {
    const I h = g / per_row;
    const I c = g - h * per_row;
    const I e = c * 4;
    const I t = e / dim, d = e - t * dim;
    const int64_t src = static_cast<int64_t>(h) * s.hs + static_cast<int64_t>(t) * s.ss + d;
    float4 a;
    if constexpr (DT == kF32) {
      a = *reinterpret_cast<const float4*>(static_cast<const float*>(s.tensor) + src);
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(s.tensor) + src);
      if constexpr (DT == kBF16) {
        a = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                        __uint_as_float(u.y & 0xffff0000u));
      } else {
        a = make_float4(f16_bits_to_f32(static_cast<uint16_t>(u.x & 0xffffu)), f16_bits_to_f32(static_cast<uint16_t>(u.x >> 16)),
                        f16_bits_to_f32(static_cast<uint16_t>(u.y & 0xffffu)), f16_bits_to_f32(static_cast<uint16_t>(u.y >> 16)));
      }
    }
    float4* w = reinterpret_cast<float4*>(s.wire) + static_cast<int64_t>(h) * s.rep * per_row + c;
    for (int64_t r = 0; r < s.rep; ++r) store16_nt_sc1(w + r * per_row, __builtin_bit_cast(u32x4, a));
  }
}

template <int DT, typename I>
__global__ __launch_bounds__(kWireThreads) void wire_unpack8_kernel(WireSeg s) {
  const I per_row = static_cast<I>(s.len * s.dim / 8);
  const I dim = static_cast<I>(s.dim);
  const I n = static_cast<I>(s.rows / s.rep) * per_row;
  for (I g = static_cast<I>(blockIdx.x) * kWireThreads + threadIdx.x; g < n;
       g += static_cast<I>(gridDim.x) * kWireThreads) {
    const I h = g / per_row;
    const I c = g - h * per_row;
    const I e = c * 8;
    const I t = e / dim, d = e - t * dim;
    const float4* w = reinterpret_cast<const float4*>(s.wire) + (static_cast<int64_t>(h) * s.rep * per_row + c) * 2;
    store8<DT>(s.tensor, static_cast<int64_t>(h) * s.hs + static_cast<int64_t>(t) * s.ss + d, w[0], w[1]);
  }
}

template <typename I>
void launch_seg8(bool pack, int dtype, const WireSeg& s, hipStream_t stream) {
  const int64_t n = (s.rows / s.rep) * (s.len * s.dim / (pack ? 4 : 8));
  if (n <= 0) return;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(n, kWireThreads), 8192));
#define HCP_WIRE8_LAUNCH(DTV)                                                                     \
  if (pack) wire_pack8_kernel<DTV, I><<<grid, kWireThreads, 0, stream>>>(s);                     \
  else wire_unpack8_kernel<DTV, I><<<grid, kWireThreads, 0, stream>>>(s);
  switch (dtype) {
    case kF32: HCP_WIRE8_LAUNCH(kF32) break;
    case kBF16: HCP_WIRE8_LAUNCH(kBF16) break;
    case kF16: HCP_WIRE8_LAUNCH(kF16) break;
    default: throw Error(-6, "wire: dtype must be F16, BF16 or F32");
  }
#undef HCP_WIRE8_LAUNCH
  HCP_HIP(hipGetLastError());
}

template <int VEC>
void launch_seg(bool pack, int dtype, const WireSeg& s, hipStream_t stream) {
  const int64_t rows = pack ? s.rows : s.rows / s.rep;
  const int64_t n = rows * (s.len * s.dim / VEC);
  if (n <= 0) return;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(n, kWireThreads), 8192));
#define HCP_WIRE_LAUNCH(DTV)                                                                      \
  if (pack) wire_pack_kernel<DTV, VEC><<<grid, kWireThreads, 0, stream>>>(s);                    \
  else wire_unpack_kernel<DTV, VEC><<<grid, kWireThreads, 0, stream>>>(s);
  switch (dtype) {
    case kF32: HCP_WIRE_LAUNCH(kF32) break;
    case kBF16: HCP_WIRE_LAUNCH(kBF16) break;
    case kF16: HCP_WIRE_LAUNCH(kF16) break;
    default: throw Error(-6, "wire: dtype must be F16, BF16 or F32");
  }
#undef HCP_WIRE_LAUNCH
  HCP_HIP(hipGetLastError());
}

}  // namespace

void launch_wire_segment(bool pack, int dtype, void* tensor, float* wire, int64_t rows, int64_t rep, int64_t len,
                         int64_t dim, int64_t hs, int64_t ss, hipStream_t stream) {
  WireSeg s{tensor, wire, rows, rep, len, dim, hs, ss};
  require(rep >= 1 && rows % rep == 0, "wire: rows must be a multiple of the expand factor");
  const int64_t es = dtype == kF32 ? 4 : 2;
  const bool rows16 = dim % 8 == 0 && reinterpret_cast<uintptr_t>(tensor) % 16 == 0 && (hs * es) % 16 == 0 &&
                      (ss * es) % 16 == 0 && reinterpret_cast<uintptr_t>(wire) % 16 == 0;
  if (rows16) {
    if (rows / rep * len * dim < (int64_t(1) << 31)) launch_seg8<uint32_t>(pack, dtype, s, stream);
    else launch_seg8<int64_t>(pack, dtype, s, stream);
  } else if (dim % 4 == 0) {
    require(reinterpret_cast<uintptr_t>(wire) % 16 == 0, "wire: payload must be 16-byte aligned");
    launch_seg<4>(pack, dtype, s, stream);
  } else {
    require(reinterpret_cast<uintptr_t>(wire) % 4 == 0, "wire: payload must be 4-byte aligned");
    launch_seg<1>(pack, dtype, s, stream);
  }
}

// ---------------------------------------------------------------------------------
// Host side: serde_json-compatible header text and a small JSON reader.
// ---------------------------------------------------------------------------------
const char* dtype_wire_name(int dtype) {
  switch (dtype) {
    case kF32: return "float32";
    case kF16: return "float16";
    case kBF16: return "bfloat16";
    default: throw Error(-6, "wire: dtype must be F16, BF16 or F32");
  }
}

int dtype_from_wire_name(const std::string& s) {
  // tcp.rs:149-154: unknown names decode as float32.
  if (s == "float16") return kF16;
  if (s == "bfloat16") return kBF16;
  return kF32;
}

// f64 as serde_json writes it (ryu's shortest round-trip digits; plain notation with
// ".0" for integers up to 16 digits, "0.000ddd" down to 1e-5, else d.ddde<exp>).
std::string json_f64(double x) {
  require(std::isfinite(x), "wire: non-finite float in header");
  if (x == 0) return std::signbit(x) ? "-0.0" : "0.0";
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof(buf), x, std::chars_format::scientific);
  std::string sci(buf, r.ptr);
  std::string out;
  if (sci[0] == '-') {
    out = "-";
    sci = sci.substr(1);
  }
  const size_t epos = sci.find('e');
  std::string digits = sci.substr(0, 1) + (epos > 2 ? sci.substr(2, epos - 2) : "");
  const int e10 = std::stoi(sci.substr(epos + 1));
  const int len = static_cast<int>(digits.size());
  const int kk = e10 + 1;  // position of the decimal point relative to the digits
  if (len <= kk && kk <= 16) {
    out += digits + std::string(kk - len, '0') + ".0";
  } else if (0 < kk && kk <= 16) {
    out += digits.substr(0, kk) + "." + digits.substr(kk);
  } else if (-5 < kk && kk <= 0) {
    out += "0." + std::string(-kk, '0') + digits;
  } else {
    out += digits.substr(0, 1);
    if (len > 1) out += "." + digits.substr(1);
    out += "e" + std::to_string(kk - 1);
  }
  return out;
}

namespace {

std::string shape_json(const std::vector<int64_t>& s) {
  std::string o = "[";
  for (size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
  return o + "]";
}

}  // namespace

std::string kv_frame_meta(int64_t layer_idx, int64_t start, int64_t end, int dtype, int64_t heads, int64_t len,
                          int64_t dim, bool positions) {
  const std::vector<int64_t> shape{1, heads, len, dim};
  const std::string bytes = std::to_string(heads * len * dim * 4);
  const std::string dt = std::string("\"") + dtype_wire_name(dtype) + "\"";
  std::string pos = "null";
  if (positions)
    pos = "{\"bytes\":" + std::to_string(len * 8) + ",\"dtype\":\"int64\",\"shape\":[" + std::to_string(len) + "]}";
  return "{\"global_seq_end\":" + std::to_string(end) + ",\"global_seq_start\":" + std::to_string(start) +
         ",\"k_bytes\":" + bytes + ",\"k_dtype\":" + dt + ",\"k_shape\":" + shape_json(shape) +
         ",\"layer_idx\":" + std::to_string(layer_idx) + ",\"position_ids\":" + pos + ",\"v_bytes\":" + bytes +
         ",\"v_dtype\":" + dt + ",\"v_shape\":" + shape_json(shape) + "}";
}

std::string packet_frame_meta(int64_t layer_idx, int q_dtype, int o_dtype, int64_t batch, int64_t heads,
                              int64_t dim, double scale) {
  const std::vector<int64_t> qs{batch, heads, 1, dim}, ls{batch, heads, 1};
  const std::string qb = std::to_string(batch * heads * dim * 4), lb = std::to_string(batch * heads * 4);
  return "{\"layer_idx\":" + std::to_string(layer_idx) + ",\"lse_bytes\":" + lb +
         ",\"lse_dtype\":\"float32\",\"lse_shape\":" + shape_json(ls) + ",\"o_bytes\":" + qb + ",\"o_dtype\":\"" +
         dtype_wire_name(o_dtype) + "\",\"o_shape\":" + shape_json(qs) + ",\"q_bytes\":" + qb +
         ",\"q_dtype\":\"" + dtype_wire_name(q_dtype) + "\",\"q_shape\":" + shape_json(qs) +
         ",\"scale\":" + json_f64(scale) + ",\"type\":\"ring_packet\"}";
}

namespace {

struct JReader {
  const char* p;
  const char* end;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < end && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  std::string str() {
    require(eat('"'), "header: expected a string");
    std::string s;
    while (p < end && *p != '"') {
      require(*p != '\\', "header: escapes are not used in frame headers");
      s += *p++;
    }
    require(p < end, "header: unterminated string");
    ++p;
    return s;
  }
  JVal value(int depth) {
    require(depth < 8, "header: nesting too deep");
    ws();
    require(p < end, "header: truncated");
    JVal v;
    if (*p == '{') {
      ++p;
      v.kind = JVal::kObj;
      if (eat('}')) return v;
      do {
        std::string k = str();
        require(eat(':'), "header: expected ':'");
        v.obj[k] = value(depth + 1);
      } while (eat(','));
      require(eat('}'), "header: expected '}'");
    } else if (*p == '[') {
      ++p;
      v.kind = JVal::kArr;
      if (eat(']')) return v;
      do v.arr.push_back(value(depth + 1));
      while (eat(','));
      require(eat(']'), "header: expected ']'");
    } else if (*p == '"') {
      v.kind = JVal::kStr;
      v.str = str();
    } else if (end - p >= 4 && std::strncmp(p, "null", 4) == 0) {
      p += 4;
    } else {
      const char* b = p;
      while (p < end && (std::isdigit(static_cast<unsigned char>(*p)) || *p == '-' || *p == '+' || *p == '.' ||
                         *p == 'e' || *p == 'E'))
        ++p;
      require(p > b, "header: unexpected character");
      const std::string t(b, p);
      v.kind = JVal::kNum;
      v.num = std::stod(t);
      v.integral = t.find_first_of(".eE") == std::string::npos;
      if (v.integral) v.inum = std::stoll(t);
    }
    return v;
  }
};

}  // namespace

JVal parse_frame_meta(const unsigned char* frame, size_t n, size_t* header_bytes) {
  require(frame != nullptr && n >= 4, "header: frame shorter than the length prefix");
  const uint32_t meta_len = (static_cast<uint32_t>(frame[0]) << 24) | (static_cast<uint32_t>(frame[1]) << 16) |
                            (static_cast<uint32_t>(frame[2]) << 8) | static_cast<uint32_t>(frame[3]);
  require(4 + static_cast<size_t>(meta_len) <= n, "header: frame shorter than meta_len");
  JReader r{reinterpret_cast<const char*>(frame) + 4, reinterpret_cast<const char*>(frame) + 4 + meta_len};
  JVal v = r.value(0);
  r.ws();
  require(r.p == r.end && v.kind == JVal::kObj, "header: meta is not one JSON object");
  *header_bytes = 4 + meta_len;
  return v;
}

}  // namespace hcp
