/*
 * CPU oracle for the ring-attention path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker.  The shipped HIP library never links it.
 *
 * Contents
 *   1. The reference's synthetic-input generator (LCG + Box-Muller), restated from
 *      rust/src/smoke/reference_algo.rs:56-90, with the fp32 / bf16 rounding used by
 *      the configs (f64 -> fp32 round-to-nearest-even -> bf16 round-to-nearest-even).
 *   2. Paged-KV gather / scatter over the vLLM cache layout
 *      [2, num_blocks, block_size, num_kv_heads, head_dim]
 *      (python/hcp_vllm_block_ring_plugin.py:8-14 layout, :143-174 extract/insert,
 *      :304-337 get_kv_block_from_table index math, :520-530 tail-slot zero fill),
 *      into / out of a contiguous head-major ring buffer [num_kv_heads, L, head_dim]
 *      (the KvBlock [B, H, S, D] layout, rust/src/model/transport/block.rs:11-35).
 *
 * Build: see oracle/Makefile (plain gcc, no dependencies beyond libm).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define LCG_A 6364136223846793005ULL
#define LCG_C 1442695040888963407ULL

typedef struct {
  uint64_t state;
  int has_spare;
  double spare;
} oracle_rng;

/* reference_algo.rs:66-74 */
static double next_open01(oracle_rng* r) {
  r->state = r->state * LCG_A + LCG_C;
  uint64_t value = r->state >> 11;
  return ((double)value + 0.5) / (double)(1ULL << 53);
}

/* reference_algo.rs:79-89: first call returns r*cos and keeps r*sin as the spare. */
static double standard_normal(oracle_rng* r) {
  if (r->has_spare) {
    r->has_spare = 0;
    return r->spare;
  }
  double u1 = next_open01(r);
  double u2 = next_open01(r);
  double radius = sqrt(-2.0 * log(u1));
  double angle = 2.0 * M_PI * u2;
  r->spare = radius * sin(angle);
  r->has_spare = 1;
  return radius * cos(angle);
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

/*
 * Draw `count` standard normals for each of `num_tensors` tensors, one stream, in
 * order (Q, then K, then V: rust/src/smoke/correctness.rs:11-29).
 * out_kind: 0 -> f64, 1 -> fp32, 2 -> bf16 bits (via fp32).
 * outs[i] must hold counts[i] elements of the requested kind.
 */
void oracle_draw_normals(uint64_t seed, int num_tensors, const int64_t* counts,
                         void* const* outs, int out_kind) {
  oracle_rng r = {seed, 0, 0.0};
  for (int t = 0; t < num_tensors; ++t) {
    int64_t n = counts[t];
    if (out_kind == 0) {
      double* o = (double*)outs[t];
      for (int64_t i = 0; i < n; ++i) o[i] = standard_normal(&r);
    } else if (out_kind == 1) {
      float* o = (float*)outs[t];
      for (int64_t i = 0; i < n; ++i) o[i] = (float)standard_normal(&r);
    } else {
      uint16_t* o = (uint16_t*)outs[t];
      for (int64_t i = 0; i < n; ++i) o[i] = f32_to_bf16_rne((float)standard_normal(&r));
    }
  }
}

/* Uniform open-interval draws (the same LCG) for block-table permutations etc. */
void oracle_draw_uniforms(uint64_t seed, int64_t n, double* out) {
  oracle_rng r = {seed, 0, 0.0};
  for (int64_t i = 0; i < n; ++i) out[i] = next_open01(&r);
}

/*
 * Paged gather of tokens [t0, t1) of one sequence.
 * Token t lives in physical block table[(t - table_seq_offset) / bs] at slot
 * (t - table_seq_offset) % bs (hcp_vllm_block_ring_plugin.py:324-327).
 * pool: [2][num_blocks][bs][hkv][d] elements of elem_bytes each; K is plane 0, V plane 1.
 * out_k / out_v: element (h, j, :) at ((h * out_head_stride) + j * out_seq_stride) elems.
 * Returns 0, or -6 if a table entry or index is out of range (nothing written then).
 */
int oracle_paged_gather(const void* pool, int64_t num_blocks, int64_t bs, int64_t hkv,
                        int64_t d, int64_t elem_bytes, const int32_t* table,
                        int64_t table_len, int64_t table_seq_offset, int64_t t0, int64_t t1,
                        void* out_k, void* out_v, int64_t out_head_stride,
                        int64_t out_seq_stride) {
  if (t1 < t0 || t0 < table_seq_offset) return -6;
  if (t1 > t0 && (t1 - 1 - table_seq_offset) / bs >= table_len) return -6;
  for (int64_t t = t0; t < t1; ++t) {
    int64_t rel = t - table_seq_offset;
    int32_t blk = table[rel / bs];
    if (blk < 0 || blk >= num_blocks) return -6;
  }
  const uint8_t* p = (const uint8_t*)pool;
  const int64_t row = d * elem_bytes;
  const int64_t plane = num_blocks * bs * hkv * row;
  for (int64_t t = t0; t < t1; ++t) {
    int64_t rel = t - table_seq_offset;
    int64_t blk = table[rel / bs];
    int64_t slot = rel % bs;
    for (int64_t h = 0; h < hkv; ++h) {
      int64_t src = ((blk * bs + slot) * hkv + h) * row;
      int64_t dst = (h * out_head_stride + (t - t0) * out_seq_stride) * elem_bytes;
      memcpy((uint8_t*)out_k + dst, p + src, (size_t)row);
      memcpy((uint8_t*)out_v + dst, p + plane + src, (size_t)row);
    }
  }
  return 0;
}

/*
 * Paged scatter (inverse of the gather).  With zero_tail != 0 the slots after the last
 * written token in its physical block are zero-filled, as the plugin does for a partial
 * last block (hcp_vllm_block_ring_plugin.py:520-530).
 */
int oracle_paged_scatter(void* pool, int64_t num_blocks, int64_t bs, int64_t hkv, int64_t d,
                         int64_t elem_bytes, const int32_t* table, int64_t table_len,
                         int64_t table_seq_offset, int64_t t0, int64_t t1, const void* in_k,
                         const void* in_v, int64_t in_head_stride, int64_t in_seq_stride,
                         int zero_tail) {
  if (t1 < t0 || t0 < table_seq_offset) return -6;
  if (t1 > t0 && (t1 - 1 - table_seq_offset) / bs >= table_len) return -6;
  for (int64_t t = t0; t < t1; ++t) {
    int32_t blk = table[(t - table_seq_offset) / bs];
    if (blk < 0 || blk >= num_blocks) return -6;
  }
  uint8_t* p = (uint8_t*)pool;
  const int64_t row = d * elem_bytes;
  const int64_t plane = num_blocks * bs * hkv * row;
  for (int64_t t = t0; t < t1; ++t) {
    int64_t rel = t - table_seq_offset;
    int64_t blk = table[rel / bs];
    int64_t slot = rel % bs;
    for (int64_t h = 0; h < hkv; ++h) {
      int64_t dst = ((blk * bs + slot) * hkv + h) * row;
      int64_t src = (h * in_head_stride + (t - t0) * in_seq_stride) * elem_bytes;
      memcpy(p + dst, (const uint8_t*)in_k + src, (size_t)row);
      memcpy(p + plane + dst, (const uint8_t*)in_v + src, (size_t)row);
    }
  }
  if (zero_tail && t1 > t0) {
    int64_t rel = t1 - table_seq_offset;
    int64_t slot = rel % bs;
    if (slot != 0) {
      int64_t blk = table[(rel - 1) / bs];
      for (int64_t s = slot; s < bs; ++s) {
        int64_t dst = ((blk * bs + s) * hkv) * row;
        memset(p + dst, 0, (size_t)(hkv * row));
        memset(p + plane + dst, 0, (size_t)(hkv * row));
      }
    }
  }
  return 0;
}
