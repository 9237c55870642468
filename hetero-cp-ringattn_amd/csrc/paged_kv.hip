// Paged-KV staging: vLLM block pool <-> contiguous head-major ring buffer.
//
// Pool layout [2, num_blocks, block_size, num_kv_heads, head_dim]
// (python/hcp_vllm_block_ring_plugin.py:8-14); token t of a sequence lives in
// block_table[(t - table_seq_offset) / block_size] at slot (t - table_seq_offset) % bs
// (:304-337).  The ring buffer is the KvBlock layout [H, L, D]
// (rust/src/model/transport/block.rs:11-35), here any strided [H, L, D] view.
//
// One workgroup moves one table entry (a physical block: block_size x Hkv rows of
// head_dim elements, both planes).  The pool side of a block is one contiguous span
// per plane (32 KiB for bs=16, Hkv=8, D=128, bf16), read or written with 16-byte
// accesses in address order; the ring-buffer side is Hkv runs of block_size rows.
// HBM-bound byte copy: algorithmic traffic = 2 planes x rows x row_bytes x (read+write).
#include "kernels.hpp"

namespace hcp {

struct PagedCopyArgs {
  uint8_t* pool;            // plane 0 (K); plane 1 at + plane_bytes
  int64_t plane_bytes;
  int64_t num_blocks;
  const int32_t* table;
  int64_t table_seq_offset;
  int64_t t0, t1;
  int64_t first_entry;      // table index of the first block touched
  uint8_t* k_buf;           // ring-buffer side (gather: dst, scatter: src)
  uint8_t* v_buf;
  int64_t head_stride_b;    // bytes between heads
  int64_t seq_stride_b;     // bytes between tokens
  int32_t bs, hkv, row_bytes;
  int32_t zero_tail;
  int* err;
};

template <typename V, bool kGather>
__global__ __launch_bounds__(256) void paged_copy_kernel(PagedCopyArgs a) {
  const int64_t entry = a.first_entry + blockIdx.x;
  const int32_t blk = a.table[entry];
  if (blk < 0 || blk >= a.num_blocks) {
    if (threadIdx.x == 0) atomicOr(a.err, 1);
    return;
  }
  constexpr int kVec = sizeof(V);
  const int vec_per_row = a.row_bytes / kVec;
  const int vec_per_slot = vec_per_row * a.hkv;
  const int total = vec_per_slot * a.bs;
  const int64_t block_tok0 = a.table_seq_offset + entry * a.bs;  // global token of slot 0
  const int64_t block_bytes = static_cast<int64_t>(a.bs) * a.hkv * a.row_bytes;
  uint8_t* pk = a.pool + static_cast<int64_t>(blk) * block_bytes;
  uint8_t* pv = pk + a.plane_bytes;

  constexpr int kUnroll = 4;
  for (int base = threadIdx.x; base < total; base += 256 * kUnroll) {
    V rk[kUnroll], rv[kUnroll];
    int64_t boff[kUnroll];
    bool ok[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = base + u * 256;
      const int slot = c / vec_per_slot;
      const int rem = c - slot * vec_per_slot;
      const int h = rem / vec_per_row;
      const int cv = rem - h * vec_per_row;
      const int64_t tok = block_tok0 + slot;
      ok[u] = (c < total) && tok >= a.t0 && tok < a.t1;
      boff[u] = h * a.head_stride_b + (tok - a.t0) * a.seq_stride_b + static_cast<int64_t>(cv) * kVec;
      if (ok[u]) {
        if constexpr (kGather) {
          rk[u] = *reinterpret_cast<const V*>(pk + static_cast<int64_t>(c) * kVec);
          rv[u] = *reinterpret_cast<const V*>(pv + static_cast<int64_t>(c) * kVec);
        } else {
          rk[u] = *reinterpret_cast<const V*>(a.k_buf + boff[u]);
          rv[u] = *reinterpret_cast<const V*>(a.v_buf + boff[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = base + u * 256;
      if (ok[u]) {
        if constexpr (kGather) {
          *reinterpret_cast<V*>(a.k_buf + boff[u]) = rk[u];
          *reinterpret_cast<V*>(a.v_buf + boff[u]) = rv[u];
        } else {
          *reinterpret_cast<V*>(pk + static_cast<int64_t>(c) * kVec) = rk[u];
          *reinterpret_cast<V*>(pv + static_cast<int64_t>(c) * kVec) = rv[u];
        }
      } else if (!kGather && a.zero_tail && c < total) {
        // Slots after the last written token of the sequence's last block.
        const int slot = c / vec_per_slot;
        const int64_t tok = block_tok0 + slot;
        if (tok >= a.t1) {
          V z;
          __builtin_memset(&z, 0, sizeof(V));
          *reinterpret_cast<V*>(pk + static_cast<int64_t>(c) * kVec) = z;
          *reinterpret_cast<V*>(pv + static_cast<int64_t>(c) * kVec) = z;
        }
      }
    }
  }
}

// Host launcher shared by gather and scatter.  Shapes were validated by the caller.
void launch_paged_copy(bool gather, void* pool, int64_t num_blocks, int bs, int hkv, int d,
                       int elem_bytes, const int32_t* table, int64_t table_seq_offset,
                       int64_t t0, int64_t t1, void* k_buf, void* v_buf, int64_t head_stride,
                       int64_t seq_stride, int zero_tail, int* err, hipStream_t stream) {
  if (t1 <= t0) return;
  PagedCopyArgs a;
  a.row_bytes = d * elem_bytes;
  a.pool = static_cast<uint8_t*>(pool);
  a.plane_bytes = num_blocks * bs * hkv * static_cast<int64_t>(a.row_bytes);
  a.num_blocks = num_blocks;
  a.table = table;
  a.table_seq_offset = table_seq_offset;
  a.t0 = t0;
  a.t1 = t1;
  a.first_entry = (t0 - table_seq_offset) / bs;
  const int64_t last_entry = (t1 - 1 - table_seq_offset) / bs;
  a.k_buf = static_cast<uint8_t*>(k_buf);
  a.v_buf = static_cast<uint8_t*>(v_buf);
  a.head_stride_b = head_stride * elem_bytes;
  a.seq_stride_b = seq_stride * elem_bytes;
  a.bs = bs;
  a.hkv = hkv;
  a.zero_tail = zero_tail;
  a.err = err;
  const dim3 grid(static_cast<unsigned>(last_entry - a.first_entry + 1));
  // Widest access that every row start and stride allows.
  auto aligned = [&](int v) {
    return a.row_bytes % v == 0 && a.head_stride_b % v == 0 && a.seq_stride_b % v == 0 &&
           reinterpret_cast<uintptr_t>(pool) % v == 0 && reinterpret_cast<uintptr_t>(k_buf) % v == 0 &&
           reinterpret_cast<uintptr_t>(v_buf) % v == 0;
  };
  if (aligned(16)) {
    if (gather) paged_copy_kernel<uint4, true><<<grid, 256, 0, stream>>>(a);
    else paged_copy_kernel<uint4, false><<<grid, 256, 0, stream>>>(a);
  } else if (aligned(4)) {
    if (gather) paged_copy_kernel<uint32_t, true><<<grid, 256, 0, stream>>>(a);
    else paged_copy_kernel<uint32_t, false><<<grid, 256, 0, stream>>>(a);
  } else {
    if (gather) paged_copy_kernel<uint16_t, true><<<grid, 256, 0, stream>>>(a);
    else paged_copy_kernel<uint16_t, false><<<grid, 256, 0, stream>>>(a);
  }
  HCP_HIP(hipGetLastError());
}

}  // namespace hcp
