// Paged-KV staging: vLLM block pool <-> contiguous head-major ring buffer.
//
// Pool layout [2, num_blocks, block_size, num_kv_heads, head_dim]
// (python/hcp_vllm_block_ring_plugin.py:8-14); token t of a sequence lives in
// block_table[(t - table_seq_offset) / block_size] at slot (t - table_seq_offset) % bs
// (:304-337).  The ring buffer is the KvBlock layout [H, L, D]
// (rust/src/model/transport/block.rs:11-35), here any strided [H, L, D] view.
//
// The pool side of a table entry (a physical block: block_size x Hkv rows of head_dim
// elements) is one contiguous span per plane (32 KiB for bs=16, Hkv=8, D=128, bf16);
// the ring-buffer side is Hkv runs of block_size rows.  Lanes walk an entry in
// ring-buffer order (head, token, chunk), so the head-major side is written in 1 KiB
// runs per wave instruction (writing it in the pool's 256-byte pieces measured 17%
// slower).  The gather of 16-byte-aligned shapes goes through LDS (paged_gather_lds_kernel:
// both sides contiguous, quarter planes per workgroup), and so does the scatter
// (paged_scatter_lds_kernel); other shapes copy through registers (paged_copy_kernel,
// whole entries per workgroup).
// HBM-bound byte copy: algorithmic traffic = 2 planes x rows x row_bytes x (read+write).
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace hcp {

// Up to kMaxRanges ranges (each: a sequence's block table and a token range) are
// copied by one launch; blockIdx.x walks the concatenation of their table entries.
constexpr int kMaxRanges = 16;

struct PagedRange {
  const int32_t* table;
  int64_t table_seq_offset;
  int64_t t0, t1;
  int64_t first_entry;      // table index of the first block touched
  uint8_t* k_buf;           // ring-buffer side (gather: dst, scatter: src)
  uint8_t* v_buf;
  int64_t head_stride_b;    // bytes between heads
  int64_t seq_stride_b;     // bytes between tokens
};

struct PagedCopyArgs {
  uint8_t* pool;            // plane 0 (K); plane 1 at + plane_bytes
  int64_t plane_bytes;
  int64_t num_blocks;
  int32_t bs, hkv, row_bytes;
  int32_t zero_tail;
  int32_t n_ranges;
  int32_t block_begin[kMaxRanges + 1];  // prefix sums of blocks per range
  PagedRange r[kMaxRanges];
  int* err;
};

// Each thread moves kU vectors of each plane per pass: all 2*kU loads are issued before
// any store, so a 256-thread workgroup keeps 2*kU*256*sizeof(V) bytes in flight.
// Range of entry bid of the concatenated ranges.
__device__ __forceinline__ int range_of(const PagedCopyArgs& a, int bid) {
  int ri = 0;
  while (ri + 1 < a.n_ranges && bid >= a.block_begin[ri + 1]) ++ri;
  return ri;
}

template <typename V, bool kGather, int kU>
__device__ __forceinline__ void paged_copy_entry(const PagedCopyArgs& a, int bid, int32_t blk) {
  const int ri = range_of(a, bid);
  const PagedRange& R = a.r[ri];
  const int64_t entry = R.first_entry + (bid - a.block_begin[ri]);
  if (blk < 0 || blk >= a.num_blocks) {
    if (threadIdx.x == 0) atomicOr(a.err, 1);
    return;
  }
  constexpr int kVec = sizeof(V);
  const int vec_per_row = a.row_bytes / kVec;
  const int vec_per_head = vec_per_row * a.bs;  // one head's rows of the block
  const int total = vec_per_head * a.hkv;
  const int64_t block_tok0 = R.table_seq_offset + entry * a.bs;  // token of slot 0
  const int64_t block_bytes = static_cast<int64_t>(a.bs) * a.hkv * a.row_bytes;
  uint8_t* pk = a.pool + static_cast<int64_t>(blk) * block_bytes;
  uint8_t* pv = pk + a.plane_bytes;

  for (int base = threadIdx.x; base < total; base += 256 * kU) {
    V rk[kU], rv[kU];
    int64_t boff[kU];
    int pc[kU], slot_of[kU];
    bool ok[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      // Vector c of this entry in ring-buffer order (head, slot, chunk): the 64 lanes of
      // a wave cover 4 consecutive tokens of one head, 1 KiB contiguous in the
      // head-major buffer; in the pool they are 4 rows of 256 B (chunk pc).
      const int c = base + u * 256;
      const int h = c / vec_per_head;
      const int rem = c - h * vec_per_head;
      const int slot = rem / vec_per_row;
      const int cv = rem - slot * vec_per_row;
      const int64_t tok = block_tok0 + slot;
      slot_of[u] = slot;
      pc[u] = (slot * a.hkv + h) * vec_per_row + cv;
      ok[u] = (c < total) && tok >= R.t0 && tok < R.t1;
      boff[u] = h * R.head_stride_b + (tok - R.t0) * R.seq_stride_b + static_cast<int64_t>(cv) * kVec;
      if (ok[u]) {
        if constexpr (kGather) {
          rk[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(pk + static_cast<int64_t>(pc[u]) * kVec));
          rv[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(pv + static_cast<int64_t>(pc[u]) * kVec));
        } else {
          rk[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(R.k_buf + boff[u]));
          rv[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(R.v_buf + boff[u]));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = base + u * 256;
      if (ok[u]) {
        if constexpr (kGather) {
          __builtin_nontemporal_store(rk[u], reinterpret_cast<V*>(R.k_buf + boff[u]));
          __builtin_nontemporal_store(rv[u], reinterpret_cast<V*>(R.v_buf + boff[u]));
        } else {
          __builtin_nontemporal_store(rk[u], reinterpret_cast<V*>(pk + static_cast<int64_t>(pc[u]) * kVec));
          __builtin_nontemporal_store(rv[u], reinterpret_cast<V*>(pv + static_cast<int64_t>(pc[u]) * kVec));
        }
      } else if (!kGather && a.zero_tail && c < total) {
        // Slots after the last written token of the sequence's last block.
        if (block_tok0 + slot_of[u] >= R.t1) {
          V z;
          __builtin_memset(&z, 0, sizeof(V));
          *reinterpret_cast<V*>(pk + static_cast<int64_t>(pc[u]) * kVec) = z;
          *reinterpret_cast<V*>(pv + static_cast<int64_t>(pc[u]) * kVec) = z;
        }
      }
    }
  }
}

template <typename V, bool kGather, int kU>
__global__ __launch_bounds__(256) void paged_copy_kernel(PagedCopyArgs a) {
  // Workgroup i copies table entries i, i + grid, ... of the concatenated ranges.  The
  // block ids of its next kPre entries are read in parallel (one lane each) before any
  // of them is copied, so the table reads do not wait in line with the data.
  constexpr int kPre = 8;
  __shared__ int32_t blk_s[kPre];
  const int n_all = a.block_begin[a.n_ranges];
  for (int first = blockIdx.x; first < n_all; first += kPre * gridDim.x) {
    if (threadIdx.x < kPre) {
      const int bid = first + threadIdx.x * gridDim.x;
      int32_t b = -1;
      if (bid < n_all) {
        const int ri = range_of(a, bid);
        b = a.r[ri].table[a.r[ri].first_entry + (bid - a.block_begin[ri])];
      }
      blk_s[threadIdx.x] = b;
    }
    __syncthreads();
    for (int j = 0; j < kPre; ++j) {
      const int bid = first + j * gridDim.x;
      if (bid >= n_all) break;
      paged_copy_entry<V, kGather, kU>(a, bid, blk_s[j]);
    }
    __syncthreads();  // blk_s is rewritten by the next round
  }
}

// Gather through LDS (16-byte aligned): a work item is 1/P of one plane of one table
// entry (bs/P consecutive slots, every kv head).  It reaches LDS by buffer_load ... lds
// in address order (1 KiB per wave instruction, contiguous on both sides); the lanes
// then read LDS in head-major order and write the ring buffer in runs of bs/P rows per
// head.  Small items keep many workgroups resident per CU, so loads of some overlap the
// stores of others.
template <int P>
__global__ __launch_bounds__(256) void paged_gather_lds_kernel(PagedCopyArgs a, int item_bytes) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t stage[];
  const int n_items = P * 2 * a.block_begin[a.n_ranges];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int blk_bytes = a.bs * a.hkv * a.row_bytes;  // one plane of one block
  const int n_dma = item_bytes >> 10;                 // 1 KiB DMA instructions per item
  const int vec_per_row = a.row_bytes >> 4;
  const int slots = a.bs / P;
  const int vec_per_head = vec_per_row * slots;
  const int total = vec_per_head * a.hkv;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int bid = item / (2 * P), plane = (item / P) & 1, part = item % P;
    const int ri = range_of(a, bid);
    const PagedRange& R = a.r[ri];
    const int64_t entry = R.first_entry + (bid - a.block_begin[ri]);
    const int32_t blk = __builtin_amdgcn_readfirstlane(R.table[entry]);
    if (blk < 0 || blk >= a.num_blocks) {
      if (threadIdx.x == 0 && plane == 0 && part == 0) atomicOr(a.err, 1);
      continue;
    }
    const u32x4 srd = make_srd(a.pool + plane * a.plane_bytes + static_cast<int64_t>(blk) * blk_bytes +
                                   static_cast<int64_t>(part) * item_bytes, item_bytes);
    for (int i = wave; i < n_dma; i += 4)
      dma16_nt(srd, static_cast<uint32_t>((i << 10) + lane * 16), lds_offset(stage) + (i << 10));
    wait_vmcnt<0>();
    __syncthreads();
    uint8_t* dst = plane ? R.v_buf : R.k_buf;
    const int64_t tok0 = R.table_seq_offset + entry * a.bs + static_cast<int64_t>(part) * slots;
    for (int c = threadIdx.x; c < total; c += 256) {
      const int h = c / vec_per_head;
      const int rem = c - h * vec_per_head;
      const int slot = rem / vec_per_row;
      const int cv = rem - slot * vec_per_row;
      const int64_t tok = tok0 + slot;
      if (tok < R.t0 || tok >= R.t1) continue;
      const int pc = ((slot * a.hkv + h) * vec_per_row + cv) << 4;
      const int64_t boff = h * R.head_stride_b + (tok - R.t0) * R.seq_stride_b + static_cast<int64_t>(cv) * 16;
      store16_nt_sc1(dst + boff, *reinterpret_cast<const u32x4*>(&stage[pc]));
    }
    __syncthreads();  // the stage is refilled by the next item
  }
}

// Scatter through LDS, the mirror of the gather above: the lanes read an item's rows
// from the head-major buffer in 1 KiB runs (head, token, chunk order) into LDS at
// their pool positions, then write the pool block span in address order.  Slots before
// t0 are left alone; slots from t1 on are zero-filled when zero_tail is set.  The reads
// do not depend on the block id, so they are issued before it is checked: the block-
// table read overlaps them instead of preceding them.
template <int P>
__global__ __launch_bounds__(256) void paged_scatter_lds_kernel(PagedCopyArgs a, int item_bytes) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t stage[];
  const int n_items = P * 2 * a.block_begin[a.n_ranges];
  const int blk_bytes = a.bs * a.hkv * a.row_bytes;
  const int vec_per_row = a.row_bytes >> 4;
  const int slots = a.bs / P;
  const int vec_per_head = vec_per_row * slots;
  const int vec_per_slot = vec_per_row * a.hkv;
  const int total = vec_per_head * a.hkv;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int bid = item / (2 * P), plane = (item / P) & 1, part = item % P;
    const int ri = range_of(a, bid);
    const PagedRange& R = a.r[ri];
    const int64_t entry = R.first_entry + (bid - a.block_begin[ri]);
    const int32_t blk_raw = R.table[entry];
    const uint8_t* src = plane ? R.v_buf : R.k_buf;
    const int64_t tok0 = R.table_seq_offset + entry * a.bs + static_cast<int64_t>(part) * slots;
    for (int c = threadIdx.x; c < total; c += 256) {
      const int h = c / vec_per_head;
      const int rem = c - h * vec_per_head;
      const int slot = rem / vec_per_row;
      const int cv = rem - slot * vec_per_row;
      const int64_t tok = tok0 + slot;
      if (tok < R.t0 || tok >= R.t1) continue;
      const int pc = ((slot * a.hkv + h) * vec_per_row + cv) << 4;
      const int64_t boff = h * R.head_stride_b + (tok - R.t0) * R.seq_stride_b + static_cast<int64_t>(cv) * 16;
      *reinterpret_cast<u32x4*>(&stage[pc]) = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + boff));
    }
    const int32_t blk = __builtin_amdgcn_readfirstlane(blk_raw);
    __syncthreads();
    if (blk < 0 || blk >= a.num_blocks) {  // uniform: every thread skips the stores
      if (threadIdx.x == 0 && plane == 0 && part == 0) atomicOr(a.err, 1);
      continue;  // the next item's LDS writes come after this item's barrier above
    }
    uint8_t* dst = a.pool + plane * a.plane_bytes + static_cast<int64_t>(blk) * blk_bytes +
                   static_cast<int64_t>(part) * item_bytes;
    for (int c = threadIdx.x; c < total; c += 256) {
      const int64_t tok = tok0 + c / vec_per_slot;
      if (tok >= R.t0 && tok < R.t1) {
        store16_nt_sc1(dst + (c << 4), *reinterpret_cast<const u32x4*>(&stage[c << 4]));
      } else if (tok >= R.t1 && a.zero_tail) {
        *reinterpret_cast<u32x4*>(dst + (c << 4)) = u32x4{0u, 0u, 0u, 0u};
      }
    }
    __syncthreads();  // the stage is refilled by the next item
  }
}

// Host launcher shared by gather and scatter.  Shapes were validated by the caller.
void launch_paged_copy_batch(bool gather, void* pool, int64_t num_blocks, int bs, int hkv, int d,
                             int elem_bytes, int n, const PagedRangeDesc* ranges, int zero_tail,
                             int* err, hipStream_t stream) {
  int next = 0;
  while (next < n) {
    PagedCopyArgs a;
    a.row_bytes = d * elem_bytes;
    a.pool = static_cast<uint8_t*>(pool);
    a.plane_bytes = num_blocks * bs * hkv * static_cast<int64_t>(a.row_bytes);
    a.num_blocks = num_blocks;
    a.bs = bs;
    a.hkv = hkv;
    a.zero_tail = zero_tail;
    a.err = err;
    int m = 0;
    int blocks = 0;
    bool al16 = a.row_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(pool) % 16 == 0;
    bool al4 = a.row_bytes % 4 == 0 && reinterpret_cast<uintptr_t>(pool) % 4 == 0;
    for (; next < n && m < kMaxRanges; ++next) {
      const PagedRangeDesc& d_ = ranges[next];
      if (d_.t1 <= d_.t0) continue;
      PagedRange& R = a.r[m];
      R.table = d_.table;
      R.table_seq_offset = d_.table_seq_offset;
      R.t0 = d_.t0;
      R.t1 = d_.t1;
      R.first_entry = (d_.t0 - d_.table_seq_offset) / bs;
      const int64_t last_entry = (d_.t1 - 1 - d_.table_seq_offset) / bs;
      R.k_buf = static_cast<uint8_t*>(d_.k_buf);
      R.v_buf = static_cast<uint8_t*>(d_.v_buf);
      R.head_stride_b = d_.head_stride * elem_bytes;
      R.seq_stride_b = d_.seq_stride * elem_bytes;
      a.block_begin[m] = blocks;
      blocks += static_cast<int>(last_entry - R.first_entry + 1);
      auto ok = [&](int v) {
        return R.head_stride_b % v == 0 && R.seq_stride_b % v == 0 &&
               reinterpret_cast<uintptr_t>(R.k_buf) % v == 0 && reinterpret_cast<uintptr_t>(R.v_buf) % v == 0;
      };
      al16 = al16 && ok(16);
      al4 = al4 && ok(4);
      ++m;
    }
    if (m == 0) continue;
    a.n_ranges = m;
    a.block_begin[m] = blocks;
    // About two table entries per workgroup (128 KiB for bs=16, Hkv=8, D=128 bf16).
    const dim3 grid(static_cast<unsigned>(blocks > 2048 ? (blocks + 1) / 2 : blocks));
    // Widest access that every row start and stride allows.
    const int64_t blk_bytes = static_cast<int64_t>(bs) * hkv * a.row_bytes;
    // LDS path: 1/P of a plane per item, P the largest of 4, 2, 1 leaving whole-KiB items
    // of at most 32 KiB (measured on c5 against P = 8, 2, 1 and the register path: 4 is
    // fastest).
    int parts = 0;
    for (int pp : {4, 2, 1})
      if (parts == 0 && bs % pp == 0 && (blk_bytes / pp) % 1024 == 0 && blk_bytes / pp <= 32768) parts = pp;
    if (al16 && parts > 0) {
      const int item_bytes = static_cast<int>(blk_bytes / parts);
      const int64_t items = 2LL * parts * blocks;
      // one item per workgroup (measured on c5: 5758-5777 GB/s against 5495-5537 with two)
      const dim3 lgrid(static_cast<unsigned>(items < (1LL << 24) ? items : (1LL << 24)));
      if (gather) {
        if (parts == 4) paged_gather_lds_kernel<4><<<lgrid, 256, item_bytes, stream>>>(a, item_bytes);
        else if (parts == 2) paged_gather_lds_kernel<2><<<lgrid, 256, item_bytes, stream>>>(a, item_bytes);
        else paged_gather_lds_kernel<1><<<lgrid, 256, item_bytes, stream>>>(a, item_bytes);
      } else {
        if (parts == 4) paged_scatter_lds_kernel<4><<<lgrid, 256, item_bytes, stream>>>(a, item_bytes);
        else if (parts == 2) paged_scatter_lds_kernel<2><<<lgrid, 256, item_bytes, stream>>>(a, item_bytes);
        else paged_scatter_lds_kernel<1><<<lgrid, 256, item_bytes, stream>>>(a, item_bytes);
      }
    } else if (al16) {
      if (gather) paged_copy_kernel<u32x4, true, 8><<<grid, 256, 0, stream>>>(a);
      else paged_copy_kernel<u32x4, false, 8><<<grid, 256, 0, stream>>>(a);
    } else if (al4) {
      if (gather) paged_copy_kernel<uint32_t, true, 8><<<grid, 256, 0, stream>>>(a);
      else paged_copy_kernel<uint32_t, false, 8><<<grid, 256, 0, stream>>>(a);
    } else {
      if (gather) paged_copy_kernel<uint16_t, true, 8><<<grid, 256, 0, stream>>>(a);
      else paged_copy_kernel<uint16_t, false, 8><<<grid, 256, 0, stream>>>(a);
    }
    HCP_HIP(hipGetLastError());
  }
}

void launch_paged_copy(bool gather, void* pool, int64_t num_blocks, int bs, int hkv, int d,
                       int elem_bytes, const int32_t* table, int64_t table_seq_offset,
                       int64_t t0, int64_t t1, void* k_buf, void* v_buf, int64_t head_stride,
                       int64_t seq_stride, int zero_tail, int* err, hipStream_t stream) {
  PagedRangeDesc r{table, table_seq_offset, t0, t1, k_buf, v_buf, head_stride, seq_stride};
  launch_paged_copy_batch(gather, pool, num_blocks, bs, hkv, d, elem_bytes, 1, &r, zero_tail, err, stream);
}

}  // namespace hcp
