/*
 * hcp_ring.h -- C ABI of the MI355X-native ring-attention compute path.
 *
 * Drop-in boundary for the blockwise ring-attention operator of hetero-cp-ringattn
 * (HcpRingAttentionBackend in rust/src/model/attention/ring.rs).  Every entry point is
 * `extern "C"`, takes plain pointers and sizes, and returns an int status in the style
 * of the reference's FFI bridge (src/rust_bridge.cc:109-128,180-199,715-721):
 *
 *     0  success
 *    -1  numeric mismatch            (reserved; rust_bridge.cc -1)
 *    -2  C++ exception caught at the boundary (rust_bridge.cc -2)
 *    -3  unknown exception           (rust_bridge.cc -3)
 *    -4  bad device index            (rust_bridge.cc -4, bad device name)
 *    -5  GPU backend unavailable or a HIP call failed (rust_bridge.cc -5)
 *    -6  invalid arguments, null pointer or size mismatch (rust_bridge.cc -6)
 *
 * The human-readable message of the last failing call on the calling thread is
 * returned by hcp_ring_last_error() (thread-local; the reference keeps one
 * process-global std::string per smoke, rust_bridge.cc:19-27,614-644).
 *
 * Memory: every tensor pointer is a DEVICE pointer owned by the caller.  Entry points
 * never allocate device memory; scratch comes in through a caller-provided workspace
 * whose size the matching *_workspace_size() query reports.  Work is enqueued on the
 * given stream (hipStream_t passed as void*; NULL = the default stream) and returns
 * without synchronising.
 *
 * Layout convention (hcp_ring_view): a [heads, tokens, head_dim] tensor whose last
 * dimension is contiguous; element (h, t, d) lives at data + h*head_stride +
 * t*seq_stride + d (strides in ELEMENTS).  Both the reference's head-major [B,H,S,D]
 * tensors and the projection's token-major [S,H,D] view (ring.rs:1884-1903,
 * view+transpose) are expressible without a copy.
 */
#ifndef HCP_RING_H_
#define HCP_RING_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HCP_RING_ABI_VERSION 3

enum hcp_ring_status {
  HCP_RING_OK = 0,
  HCP_RING_E_MISMATCH = -1,
  HCP_RING_E_EXCEPTION = -2,
  HCP_RING_E_UNKNOWN = -3,
  HCP_RING_E_DEVICE = -4,
  HCP_RING_E_BACKEND = -5,
  HCP_RING_E_INVALID = -6
};

/* Element types; numbering of TensorDType (include/hcp_ringattn/core/tensor_types.h:9-16). */
enum hcp_ring_dtype {
  HCP_DTYPE_F16 = 1,
  HCP_DTYPE_BF16 = 2,
  HCP_DTYPE_F32 = 3,
  HCP_DTYPE_I32 = 4,
  HCP_DTYPE_I64 = 5
};

typedef struct hcp_ring_view {
  void* data;          /* device pointer of element (0, 0, 0)            */
  int64_t head_stride; /* elements between consecutive heads              */
  int64_t seq_stride;  /* elements between consecutive tokens             */
} hcp_ring_view;

/* ---------------------------------------------------------------------------------
 * Library state
 * ------------------------------------------------------------------------------- */

/* Message of the last failing call on this thread ("" if none). */
const char* hcp_ring_last_error(void);

/* HCP_RING_ABI_VERSION of the loaded library. */
int hcp_ring_abi_version(void);

/* Number of visible GPUs in *count; -5 when no HIP device is usable. */
int hcp_ring_device_count(int* count);

/*
 * Kernel path taken by the last successful attention call on this thread (block
 * partials, positioned partials, ring replays): lets a caller see which kernel ran --
 * a 16-bit view whose rows or strides are not 16-byte multiples, or a head_dim that is
 * not a multiple of 8 up to 128, goes to the scalar general kernel instead of the
 * matrix cores; fp32 runs on the fp32 matrix-core kernel where its head_dim is a
 * multiple of 4 up to 128 (and its outputs are aligned for 4-wide stores), else on the
 * general kernel.  No reference counterpart (the reference has one ATen path).
 */
enum hcp_ring_path {
  HCP_PATH_NONE = 0,        /* no attention call yet, or it launched nothing */
  HCP_PATH_MFMA = 1,        /* matrix-core block kernels (one launch per block or ring step) */
  HCP_PATH_RING_FUSED = 2,  /* the fused ring kernel (one launch per replay) */
  HCP_PATH_GENERAL = 3,     /* the scalar fp32 general kernel for at least one block */
  HCP_PATH_MFMA_F32 = 4     /* the fp32 matrix-core block kernel (fp32 views, head_dim a
                               multiple of 4 up to 128) */
};
int hcp_ring_last_path(void);

/*
 * Reads and clears the sticky device-side error flags of the current device
 * (bit 0: a paged block id outside [0, num_blocks) was met and that row skipped;
 * bit 1: a replay's generated key positions were not non-decreasing (an internal
 *        consistency check; hcp_ring_block_partial_positioned takes keys in any order
 *        and never sets it);
 * bit 2: a RoPE position outside the cos / sin table).
 * Synchronises `stream`.
 */
int hcp_ring_fetch_device_errors(void* stream, int* flags);

/* ---------------------------------------------------------------------------------
 * (1) Block partial: one ring step = one (query chunk, KV chunk) pair.
 *
 * Replaces process_kv_block + positioned_local_compact_partial
 * (ring.rs:201-370, :538-571) and, with accumulate=1,
 * positioned_merge_compact_partial (ring.rs:574-603).
 *
 * Query token i has global position q_offset+i, key token j has kv_offset+j;
 * with causal=1 a key is visible iff q_pos >= k_pos (ring.rs:249-273).  Query head h
 * reads KV head h / (num_q_heads/num_kv_heads) (the GQA expand of ring.rs:496-512,
 * done by index, no copy).  Outputs, fp32:
 *     o   [num_q_heads, q_len, head_dim] contiguous, normalised (softmax-weighted V);
 *     lse [num_q_heads, q_len]           contiguous, natural-log log-sum-exp of the
 *                                        scaled scores; -inf (and o = 0) for a row
 *                                        that sees no key.
 * With accumulate=1, o/lse hold a running partial on entry and are replaced by the
 * merge of it with this block (the rm=lse, rs=1, obh=o re-entry of ring.rs:585-587).
 * dtype: BF16 or F16 (matrix-core path: head_dim any multiple of 8 up to 128, run by
 * the head-dim-128 kernel with the columns past head_dim zero-padded, up to 64 by its
 * half-width form, 64 dims per LDS row) or
 * F32 (any head_dim <= 256; F16/BF16 with other head dims take the same general
 * kernel).
 * ------------------------------------------------------------------------------- */
typedef struct hcp_ring_block_desc {
  int32_t dtype;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int64_t q_len;
  int64_t kv_len;
  int64_t q_offset;
  int64_t kv_offset;
  int32_t causal;
  int32_t accumulate;
  float scale; /* softmax scale, 1/sqrt(head_dim) in the reference (ring.rs:152) */
} hcp_ring_block_desc;

int hcp_ring_block_partial(const hcp_ring_block_desc* desc, hcp_ring_view q, hcp_ring_view k,
                           hcp_ring_view v, float* o, float* lse, void* stream);

/* ---------------------------------------------------------------------------------
 * (1b) Block partial with explicit positions (Striped / ZigZag and any other
 * non-contiguous split): positioned_local_compact_partial /
 * positioned_merge_compact_partial with position tensors (ring.rs:538-603; the
 * KvBlock position_ids of block.rs:32-34, used by ring.rs:1024-1046).
 *
 * As (1), with desc->q_offset / kv_offset ignored: query i has global position
 * q_positions[i], key j has kv_positions[j] (DEVICE int64 arrays, the reference's
 * Int64 position tensors), and with causal=1 a key is visible iff
 * kv_positions[j] <= q_positions[i] (ring.rs:249-273, key by key).  Both lists may be
 * in any order.  A key list that is not non-decreasing (the committed-KV slab appends
 * positions in arrival order, self_driving.rs:180-224; the reference's own test passes
 * [0, 4, 3, 5], ring.rs:2343) is sorted on the device together with its K / V rows
 * into the workspace, and the fold reads them in that order; the decision is taken on
 * the device, so a list already in order costs a few empty launches and no copy.  The
 * workspace (hcp_ring_block_partial_positioned_workspace_size bytes) holds one int32 per
 * query row and, with causal=1, the sort buffers (12 bytes per key, twice) and the
 * sorted K / V copies (2 * num_kv_heads * kv_len * head_dim elements).  With causal=0
 * positions are not read.
 * ------------------------------------------------------------------------------- */
size_t hcp_ring_block_partial_positioned_workspace_size(const hcp_ring_block_desc* desc);

int hcp_ring_block_partial_positioned(const hcp_ring_block_desc* desc, hcp_ring_view q,
                                      const int64_t* q_positions, hcp_ring_view k, hcp_ring_view v,
                                      const int64_t* kv_positions, float* o, float* lse,
                                      void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * (1c) Scheduling strategies (RingSchedulingStrategy, strategy.rs:14-24) -- host only.
 *
 * hcp_ring_build_assignment: assignment[p] = domain owning global position p
 *     (build_assignment, strategy.rs:53-110); chunk_lens[d] >= 0 positions each.
 * hcp_ring_domain_positions: every domain's positions in ascending (local storage)
 *     order, concatenated in domain order (build_domain_positions, :114-121).
 * hcp_ring_inverse_perm: inverse[p] = row of position p in that concatenation
 *     (build_inverse_perm, :129-143).
 * Output arrays are HOST arrays of sum(chunk_lens) elements.  No GPU is used.
 * ------------------------------------------------------------------------------- */
enum {
  HCP_STRATEGY_VANILLA = 0,
  HCP_STRATEGY_STRIPED = 1,
  HCP_STRATEGY_ZIGZAG = 2
};

int hcp_ring_build_assignment(int32_t strategy, int32_t num_domains, const int64_t* chunk_lens,
                              int32_t* assignment);
int hcp_ring_domain_positions(int32_t strategy, int32_t num_domains, const int64_t* chunk_lens,
                              int64_t* positions);
int hcp_ring_inverse_perm(int32_t strategy, int32_t num_domains, const int64_t* chunk_lens,
                          int64_t* inverse);

/* ---------------------------------------------------------------------------------
 * (2) LSE merge of ring-step partials.
 *
 * Replaces the re-entry merge of positioned_merge_compact_partial / decode_merge_packet
 * (ring.rs:574-603, :647-663) applied across all steps, in closed form:
 *   m = max_i lse_i;  o = sum_i e^(lse_i-m) o_i / sum_i e^(lse_i-m);
 *   lse = m + ln sum_i e^(lse_i-m);  all -inf -> (o = 0, lse = -inf).
 * o_parts / lse_parts are HOST arrays of num_parts DEVICE pointers, each partial laid
 * out as hcp_ring_block_partial writes it ([H, q_len, D] and [H, q_len] fp32).
 * The merged output goes to `out` (out_dtype BF16, F16 or F32, strided view) and, if
 * lse_out is not NULL, to lse_out [H, q_len] fp32.  1 <= num_parts <= 64.
 * ------------------------------------------------------------------------------- */
int hcp_ring_lse_merge(int32_t num_parts, const float* const* o_parts,
                       const float* const* lse_parts, int32_t num_heads, int64_t q_len,
                       int32_t head_dim, int32_t out_dtype, hcp_ring_view out, float* lse_out,
                       void* stream);

/* ---------------------------------------------------------------------------------
 * (3) Paged-KV staging: vLLM block layout <-> contiguous ring buffer.
 *
 * Pool layout [2, num_blocks, block_size, num_kv_heads, head_dim] (plane 0 = K,
 * plane 1 = V), python/hcp_vllm_block_ring_plugin.py:8-14.  Token t of the sequence
 * lives in physical block block_table[(t - table_seq_offset) / block_size], slot
 * (t - table_seq_offset) % block_size (:304-337).  Gather copies tokens [t0, t1) to
 * k_out/v_out (row t - t0); scatter is its inverse and, with zero_tail=1, zero-fills
 * the slots after t1 in t1's block (the partial-last-block rule of :520-530).
 * Copies are bit-exact.  block_table is a DEVICE int32 array of table_len entries.
 * Block ids outside [0, num_blocks) are skipped and raise device error flag bit 0.
 * elem_bytes: 2 (bf16/fp16) or 4 (fp32).
 * ------------------------------------------------------------------------------- */
typedef struct hcp_paged_pool {
  void* data;
  int64_t num_blocks;
  int32_t block_size;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t elem_bytes;
} hcp_paged_pool;

int hcp_paged_kv_gather(const hcp_paged_pool* pool, const int32_t* block_table, int64_t table_len,
                        int64_t table_seq_offset, int64_t t0, int64_t t1, hcp_ring_view k_out,
                        hcp_ring_view v_out, void* stream);

int hcp_paged_kv_scatter(const hcp_paged_pool* pool, const int32_t* block_table,
                         int64_t table_len, int64_t table_seq_offset, int64_t t0, int64_t t1,
                         hcp_ring_view k_in, hcp_ring_view v_in, int32_t zero_tail,
                         void* stream);

/* Many gathers from one pool in one launch (e.g. every domain's chunk of a ring step);
 * each range has the meaning of one hcp_paged_kv_gather call.  ranges is a HOST array. */
typedef struct hcp_paged_range {
  const int32_t* block_table; /* DEVICE int32 array of table_len entries */
  int64_t table_len;
  int64_t table_seq_offset;
  int64_t t0;
  int64_t t1;
  hcp_ring_view k_out;
  hcp_ring_view v_out;        /* same strides as k_out */
} hcp_paged_range;

int hcp_paged_kv_gather_batch(const hcp_paged_pool* pool, int32_t num_ranges,
                              const hcp_paged_range* ranges, void* stream);

/* ---------------------------------------------------------------------------------
 * (4) Paged single-query decode partial over one domain chunk.
 *
 * Replaces decode_local_partial / decode_local_compact_partial (ring.rs:625-639,
 * :515-523) for a batch of independent sequences: each sequence b has one query
 * token q[b] ([num_q_heads, head_dim] at q.data + b*q.seq_stride + h*q.head_stride)
 * and attends, without a causal mask (ring.rs:631-637), to its tokens
 * [t0, min(t1, seq_lens[b])) read straight from the paged pool through row b of
 * block_tables (token t in block block_tables[b*table_stride + t/block_size]).
 * seq_lens may be NULL (every sequence covers [t0, t1)); table entries past a
 * sequence's own range are neither read nor validated (ragged padding).  Outputs fp32:
 *     o [batch, num_q_heads, head_dim], lse [batch, num_q_heads] (-inf, o = 0 when the
 *     range is empty).
 * The chunk is split across workgroups; workspace holds the split partials
 * (hcp_paged_decode_workspace_size bytes, 256-byte aligned).
 * dtype BF16 or F16, head_dim a multiple of 8 up to 128 (64: its own kernel; others run
 * the head-dim-128 kernel with the columns past head_dim zero-padded), block_size a
 * multiple of 16, and at most 16
 * query heads per KV head (num_q_heads / num_kv_heads <= 16: the GQA groups of
 * repeat_decode_kv_heads, ring.rs:496-512, of the reference's models -- 7 for
 * Qwen2-0.5B, 8 for Qwen2.5-3B, 4 for Llama-3-8B).
 * ------------------------------------------------------------------------------- */
typedef struct hcp_paged_decode_desc {
  int32_t dtype;
  int32_t batch;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t reserved0;
  int64_t t0;
  int64_t t1;
  int64_t table_stride;
  int64_t table_len;
  float scale;
} hcp_paged_decode_desc;

size_t hcp_paged_decode_workspace_size(const hcp_paged_decode_desc* desc,
                                       const hcp_paged_pool* pool);

int hcp_paged_decode_partial(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool,
                             hcp_ring_view q, const int32_t* block_tables,
                             const int32_t* seq_lens, float* o, float* lse, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * (4a) hcp_paged_decode_partial without a workspace argument: it allocates nothing,
 * taking its split partials from a static device array of 16 MiB (HCP_DECODE_STATIC_
 * SCRATCH_BYTES) that each GPU the library runs on holds until the process ends.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Returns -6 when the call needs more than the array
 * (hcp_paged_decode_workspace_size(desc, pool) > HCP_DECODE_STATIC_SCRATCH_BYTES);
 * otherwise the same results as hcp_paged_decode_partial.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (concurrent streams, other threads)
 * race, so serialise them.  Every byte a call reads from the array it has written first.
 */
#define HCP_DECODE_STATIC_SCRATCH_BYTES (16u << 20)
int hcp_paged_decode_partial_static(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool,
                                    hcp_ring_view q, const int32_t* block_tables,
                                    const int32_t* seq_lens, float* o, float* lse, void* stream);

/* ---------------------------------------------------------------------------------
 * (4b) Decode Q-ring with growth sharding (ring_decode_attention, ring.rs:665-818;
 * ownership rule ring.rs:1921-1942; KvCache::update_sharded, cache.rs:40-48,104-121).
 *
 * Each of num_domains domains holds its own shard of every sequence's KV in the paged
 * pool: its prefill chunk plus the decode tokens it owns (the token at global
 * position p is persisted only by domain hcp_decode_ring_owner(p, N) = p mod N; the
 * other domains drop it).  Together the shards hold every token once, the new token
 * included: its owner appends it (hcp_paged_kv_scatter) before the call, as
 * update_sharded(keep = true) does.  The ring starts a packet (q, o, lse) at
 * seed_domain with the partial over that domain's shard, and the packet visits
 * seed+1, seed+2, ... (mod N), each domain merging its shard into the accumulator
 * (decode_merge_packet, ring.rs:647-663).  After N-1 hops the accumulator is the
 * layer's attention output; the seed only fixes the merge order.
 * This entry replays the whole journey on one GPU: one hcp_paged_decode_partial-style
 * pass per shard, then the closed-form merge in journey order into out (q dtype,
 * [batch, Hq, D] as a view with head_stride / seq_stride = batch stride) and lse_out
 * ([batch, Hq] fp32, may be NULL).  An empty shard passes the packet through
 * unchanged (lse + log 1).  desc->t0/t1 are ignored: shard s covers tokens
 * [0, shards[s].max_len) of its table, clipped per sequence by shards[s].seq_lens.
 * ------------------------------------------------------------------------------- */
typedef struct hcp_decode_shard {
  const int32_t* block_tables; /* DEVICE int32 [batch, table_stride], this domain's tables */
  int64_t table_stride;
  int64_t table_len;           /* entries used per sequence (>= ceil(max_len / block_size)) */
  const int32_t* seq_lens;     /* DEVICE int32 [batch] tokens held per sequence, or NULL */
  int64_t max_len;             /* upper bound of seq_lens (tokens) */
} hcp_decode_shard;

int hcp_decode_ring_owner(int64_t global_pos, int32_t num_domains);

size_t hcp_decode_ring_workspace_size(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool,
                                      int32_t num_domains, const hcp_decode_shard* shards);

int hcp_decode_ring_replay(const hcp_paged_decode_desc* desc, const hcp_paged_pool* pool,
                           hcp_ring_view q, int32_t num_domains, const hcp_decode_shard* shards,
                           int32_t seed_domain, hcp_ring_view out, float* lse_out, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * (5) Single-GPU ring replay of a whole prefill (the ring_attention driver).
 *
 * Replays ring_attention (ring.rs:861-1398) for every domain of an uneven split.
 * desc->strategy picks the assignment (strategy.rs:53-110, see (1c)): with
 * HCP_STRATEGY_VANILLA domain d owns global positions [off_d, off_d + chunk_lens[d]);
 * with STRIPED or ZIGZAG it owns the positions hcp_ring_domain_positions lists, and
 * the causal masks follow them (the position_ids path of ring.rs:1024-1046, as in
 * the reference's run_uneven_ring_attention, ring.rs:3226-3360).  Domain d visits sources
 * (d - s) mod N for s = 0..N-1 (local first, then the predecessor chain), skips
 * sources entirely in its future (ring.rs:222-228), and folds each source into the
 * domain's running fp32 (o, lse) state as it arrives with (1) in accumulate mode (the
 * positioned_merge_compact_partial re-entry, ring.rs:574-603); the last source of a
 * domain writes the normalised rows straight into out.  q/k/v/out cover the whole
 * sequence in domain-major order: rows [off_d, off_d + chunk_lens[d]) hold domain d's
 * tokens in its local order (for VANILLA this is the global order; otherwise row r
 * holds position hcp_ring_domain_positions[r], and hcp_ring_inverse_perm maps the
 * output back to global order).  out receives the merged
 * attention (dtype = desc->dtype), lse_out (may be NULL) the merged LSE [Hq, S] fp32.
 * Workspace: hcp_ring_replay_workspace_size bytes (one fp32 state per domain with
 * more than one source, the positions and per-row key limits of a causal STRIPED /
 * ZIGZAG replay, plus the paged staging area).
 *
 * With a paged pool (hcp_ring_prefill_replay_paged), K/V are not given as views: each
 * source domain's chunk is first gathered with (3) from the pool through block_table
 * (table_seq_offset 0) into a staging area inside the workspace, then consumed.
 *
 * desc->schedule picks how the ring steps reach the GPU (the result is the same up to
 * fp32 rounding; no reference counterpart, the reference runs one domain per process):
 *   HCP_SCHEDULE_PER_STEP  one grouped block-kernel launch per ring step, the state
 *                          of every domain with more than one source kept in fp32 in
 *                          the workspace between steps (the schedule a multi-GPU ring
 *                          would run, one step per exchange);
 *   HCP_SCHEDULE_FUSED     one matrix-core launch for the whole replay, with the
 *                          running state in registers and the output rows written
 *                          directly (no fp32 state in HBM).  VANILLA positions (or
 *                          causal = 0): each workgroup folds all sources of its
 *                          domain's query tile in ring order.  Causal STRIPED /
 *                          ZIGZAG: K/V are first copied in position order (the
 *                          positions are a permutation of [0, S): one pass gives each
 *                          position's row, then one gather), so every query row sees
 *                          a prefix of the keys, and the whole sequence runs as one
 *                          positions-mode block (1) of S rows against S keys.
 *                          Applies to BF16/F16, head_dim a multiple of 8 up to 128,
 *                          and q/k/v/out views with 16-byte aligned rows, and to FP32
 *                          with head_dim a multiple of 4 up to 128 and an output
 *                          aligned for 16-byte stores (one block over the sequence on
 *                          the fp32 matrix-core kernel, vanilla or explicit
 *                          positions); -6 otherwise.  The paged form gathers every
 *                          chunk once, in one batched launch, then runs it;
 *   HCP_SCHEDULE_AUTO (0)  FUSED where it applies, else PER_STEP.
 * Workspace: hcp_ring_replay_workspace_size reports the need of the requested schedule
 * (AUTO: the larger of the two).  FUSED needs none unpaged with VANILLA positions; with
 * STRIPED / ZIGZAG it holds the positions, the row of each position, K/V in position
 * order (2 * Hkv * S * head_dim elements) and the per-row key limits.
 * ------------------------------------------------------------------------------- */
enum hcp_ring_schedule {
  HCP_SCHEDULE_AUTO = 0,
  HCP_SCHEDULE_PER_STEP = 1,
  HCP_SCHEDULE_FUSED = 2
};

typedef struct hcp_ring_replay_desc {
  int32_t dtype;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t num_domains;
  int32_t causal;
  const int64_t* chunk_lens; /* HOST array of num_domains lengths (each >= 1) */
  float scale;
  int32_t strategy;          /* HCP_STRATEGY_* (0 = vanilla) */
  int32_t schedule;          /* HCP_SCHEDULE_* (0 = auto) */
} hcp_ring_replay_desc;

size_t hcp_ring_replay_workspace_size(const hcp_ring_replay_desc* desc, int32_t paged);

int hcp_ring_prefill_replay(const hcp_ring_replay_desc* desc, hcp_ring_view q, hcp_ring_view k,
                            hcp_ring_view v, hcp_ring_view out, float* lse_out, void* workspace,
                            size_t workspace_bytes, void* stream);

int hcp_ring_prefill_replay_paged(const hcp_ring_replay_desc* desc, hcp_ring_view q,
                                  const hcp_paged_pool* pool, const int32_t* block_table,
                                  int64_t table_len, hcp_ring_view out, float* lse_out,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * (6) Wire frames of the ring transport (TcpKvTransport, rust/src/model/transport/
 * tcp.rs:20-40; serialize_block_to_buffer :161-207; serialize_packet_to_buffer
 * :209-243; decode_frame_from_reader :604-787).
 *
 * A KvBlock frame is [meta_len u32 BE][meta_json][k f32 LE][v f32 LE][positions i64 LE]
 * and a RingPacket frame [meta_len u32 BE][meta_json][q f32 LE][o f32 LE][lse f32 LE].
 * The header (length prefix + JSON, byte-identical to the reference's serde_json
 * output: compact, keys sorted) is built and parsed on the HOST; the payload (the
 * fp32 tensor bytes, plus the int64 positions) is packed and unpacked on the DEVICE
 * straight from / into strided views.  A frame on the wire is header then payload.
 *
 * KV frames: k / v views hold num_kv_heads heads of [len, head_dim] in `dtype`; the
 * wire carries num_heads = rep * num_kv_heads heads (the reference sends blocks after
 * the GQA expand, ring.rs:999-1019: pass num_heads = Hq to interoperate with it, or
 * num_heads = num_kv_heads for the compact form).  Pack writes wire head h from view
 * head h / rep; unpack writes view head h from wire head h * rep.  The k/v shape in
 * the header is [1, num_heads, len, head_dim]; position_ids, when present, is int64 [len].
 * hcp_kv_frame_parse fills a descriptor from a received header (num_kv_heads =
 * num_heads; lower it before unpacking to keep one head per group); a header whose
 * position_ids is null or absent (the legacy frame, tcp.rs:802-813,937-963) gives
 * has_positions = 0.  The payload pointer must be 16-byte aligned (4-byte when
 * head_dim is not a multiple of 4); header buffers are HOST memory.
 * ------------------------------------------------------------------------------- */
typedef struct hcp_kv_frame_desc {
  int64_t layer_idx;
  int64_t global_seq_start;
  int64_t global_seq_end;
  int32_t dtype;         /* storage dtype, named in k_dtype / v_dtype */
  int32_t num_heads;     /* heads on the wire */
  int32_t num_kv_heads;  /* heads of the k / v views (divides num_heads) */
  int32_t head_dim;
  int64_t len;           /* tokens in the block */
  int32_t has_positions;
  int32_t reserved0;
} hcp_kv_frame_desc;

size_t hcp_kv_frame_payload_bytes(const hcp_kv_frame_desc* desc);
int hcp_kv_frame_header(const hcp_kv_frame_desc* desc, void* out, size_t capacity, size_t* written);
int hcp_kv_frame_parse(const void* frame, size_t frame_bytes, hcp_kv_frame_desc* desc,
                       size_t* header_bytes);
int hcp_kv_frame_pack(const hcp_kv_frame_desc* desc, hcp_ring_view k, hcp_ring_view v,
                      const int64_t* positions, void* payload, void* stream);
int hcp_kv_frame_unpack(const hcp_kv_frame_desc* desc, const void* payload, hcp_ring_view k,
                        hcp_ring_view v, int64_t* positions, void* stream);

/* Decode Q-ring packets (RingPacket, block.rs:74-93): q [batch, num_heads, 1, head_dim]
 * in q_dtype (a view: seq_stride = batch stride, head_stride = head stride), o the fp32
 * accumulator [batch, num_heads, head_dim] (o_dtype is the name written for it, the
 * reference keeps o in the query dtype), lse fp32 [batch, num_heads]. */
typedef struct hcp_packet_frame_desc {
  int64_t layer_idx;
  int32_t q_dtype;
  int32_t o_dtype;
  int32_t batch;
  int32_t num_heads;
  int32_t head_dim;
  int32_t reserved0;
  double scale;
} hcp_packet_frame_desc;

size_t hcp_packet_frame_payload_bytes(const hcp_packet_frame_desc* desc);
int hcp_packet_frame_header(const hcp_packet_frame_desc* desc, void* out, size_t capacity,
                            size_t* written);
int hcp_packet_frame_parse(const void* frame, size_t frame_bytes, hcp_packet_frame_desc* desc,
                           size_t* header_bytes);
int hcp_packet_frame_pack(const hcp_packet_frame_desc* desc, hcp_ring_view q, const float* o,
                          const float* lse, void* payload, void* stream);
int hcp_packet_frame_unpack(const hcp_packet_frame_desc* desc, const void* payload, hcp_ring_view q,
                            float* o, float* lse, void* stream);

/* ---------------------------------------------------------------------------------
 * (7) Fused QKV projection + RoPE + KV append (the head of HcpRingAttentionBackend::
 * forward, ring.rs:1865-1936: q/k/v = x W^T + b, head split, RotaryEmbedding::apply at
 * the tokens' global positions (rust/src/model/layers/rotary.rs:64-158), and the
 * KV-cache append (KvCache::update, cache.rs:191-251; the positioned slab of
 * self_driving.rs:180-228)).
 *
 * hcp_rope_table writes the reference's cos / sin caches for positions [0, rows):
 * table[0 : rows*D/2] = cos(m * inv_freq[j]), table[rows*D/2 : rows*D] = sin(...),
 * row-major [rows, D/2], with inv_freq[j] = (float)(1 / base^(2j/D)) and the angle
 * formed in fp32 (rotary.rs:72-97).  DEVICE memory of rows*D floats.
 *
 * hcp_qkv_rope_project: x [tokens, hidden] (row stride x_row_stride elements), weights
 * in the HF layout [out_features, hidden] (rows contiguous: wq [Hq*D, hidden], wk / wv
 * [Hkv*D, hidden]), optional biases (NULL = none).  Outputs in the input dtype:
 * q_out [Hq, tokens, D] and k_out / v_out [Hkv, tokens, D] as views, q and k rotated
 * with positions[t] (DEVICE int64 [tokens]) when desc->rope is set (rotate_pairs:
 * halves d and d + D/2).  Accumulation and the epilogue run in fp32 and round once.
 * The _paged form appends k / v to the paged pool instead: token t goes to sequence
 * position t0 + t through block_table (as hcp_paged_kv_scatter, without the tail
 * fill); bad block ids set device error bit 0, positions outside the RoPE table bit 2.
 * dtype BF16 or F16; head_dim 64 or 128; hidden a multiple of 32; Hq*D and Hkv*D
 * multiples of 128; x, weights 16-byte aligned, x_row_stride a multiple of 8 and
 * >= hidden; output views 8-byte aligned with strides multiple of 4.
 * ------------------------------------------------------------------------------- */
typedef struct hcp_qkv_desc {
  int32_t dtype;
  int32_t hidden;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t rope;          /* 1: rotate q and k */
  int64_t tokens;
  int64_t rope_rows;     /* rows of the cos / sin tables */
} hcp_qkv_desc;

int hcp_rope_table(int32_t head_dim, int64_t rows, double base, float* table, void* stream);

int hcp_qkv_rope_project(const hcp_qkv_desc* desc, const void* x, int64_t x_row_stride,
                         const void* wq, const void* wk, const void* wv, const void* bq,
                         const void* bk, const void* bv, const int64_t* positions,
                         const float* rope_table, hcp_ring_view q_out, hcp_ring_view k_out,
                         hcp_ring_view v_out, void* stream);

int hcp_qkv_rope_project_paged(const hcp_qkv_desc* desc, const void* x, int64_t x_row_stride,
                               const void* wq, const void* wk, const void* wv, const void* bq,
                               const void* bk, const void* bv, const int64_t* positions,
                               const float* rope_table, hcp_ring_view q_out,
                               const hcp_paged_pool* pool, const int32_t* block_table,
                               int64_t table_len, int64_t table_seq_offset, int64_t t0,
                               void* stream);

/* ---------------------------------------------------------------------------------
 * (8) Domain runtime (RingAttnRuntime, the reference's include/hcp_ringattn/core/
 * ringattn_runtime.h:10-29 and its smoke, src/rust_bridge.cc:646-681) through plain C.
 *
 * The C++ interface is include/hcp_ringattn/core/ringattn_runtime.h
 * (hcp_ringattn::CreateRingAttnRuntime); these entries wrap it for FFI callers.
 * init: this runtime is domain `domain_index` of num_domains domains, with their ids
 * and seq_chunk_lens / block_sizes in ring order, global_seq_len = the sum of the
 * chunk lengths, num_heads / head_dim / dtype (HCP_DTYPE_*) of the layer, device
 * "hip".  bind_layer: the domain's q [Hq, L, D], k / v [Hkv, L, D] device views for a
 * layer.  run_layer: HOST fp32 arrays, initial state (in_seq_len = 0 for none) and the
 * resulting state: max [Hq, L] (= LSE), sum [Hq, L] (= 1), output [Hq, L, D].
 * Status: 0 ok, -6 invalid argument, -5 unimplemented, -2 internal.
 * hcp_ringattn_cxx_smoke_domain_count runs the reference's three-domain
 * Init / Run / Shutdown smoke on "hip" runtimes: returns 3, or -1 / -2 / -3 when Init /
 * Run / Shutdown fails and -10 / -11 on an exception (the reference's codes).
 * ------------------------------------------------------------------------------- */
typedef struct hcp_ringattn_runtime hcp_ringattn_runtime;

int hcp_ringattn_runtime_create(const char* device_type, hcp_ringattn_runtime** out);
void hcp_ringattn_runtime_destroy(hcp_ringattn_runtime* rt);
int hcp_ringattn_runtime_init(hcp_ringattn_runtime* rt, int32_t domain_index, int32_t num_domains,
                              const char* const* domain_ids, const int64_t* seq_chunk_lens,
                              const int64_t* block_sizes, const char* device, int64_t global_seq_len,
                              int64_t num_heads, int64_t head_dim, int32_t dtype);
int hcp_ringattn_runtime_bind_layer(hcp_ringattn_runtime* rt, int32_t layer_index, int32_t num_kv_heads,
                                    hcp_ring_view q, hcp_ring_view k, hcp_ring_view v, float scale,
                                    void* stream);
int hcp_ringattn_runtime_run_layer(hcp_ringattn_runtime* rt, int32_t layer_index, int64_t in_seq_len,
                                   const float* in_max, const float* in_sum, const float* in_output,
                                   float* out_max, float* out_sum, float* out_output);
int hcp_ringattn_runtime_shutdown(hcp_ringattn_runtime* rt);
int hcp_ringattn_cxx_smoke_domain_count(void);

/* ---------------------------------------------------------------------------------
 * (6b) Block-direct transport (KvBlockTransport, rust/src/model/transport/
 * block_transport.rs:36-126; in-memory reference implementation serialized_block.rs).
 *
 * The NIXL-style lifecycle on one GPU: two agents are created as a linked pair
 * (SerializedBlockTransport::create_pair, serialized_block.rs:69-77); each registers
 * memory blocks (register_block), advertises them as a metadata blob
 * (local_metadata), ingests the peer's blob (load_remote_metadata), posts transfers
 * from a local block into a peer block (submit_transfer: an asynchronous copy of the
 * raw bytes on `stream`, device or host memory) and collects the completions posted to
 * it without blocking (poll_transfers: an event query per transfer).  Descriptors are
 * BlockDesc / RemoteBlockDesc in the reference's field order; mem_type follows
 * BlockMemType (0 = Dram, 1 = Vram: device memory registers as Vram with dev_id = its
 * device); meta is serde_json's compact text of the registered shape (e.g. "[1,2,3,4]",
 * serialized_block.rs:103-115).  Metadata blobs are byte-compatible with the
 * reference's bincode 1.3.3 serialisation of AgentMetadata (little-endian, u64
 * lengths, u32 enum variants, blocks in ascending id).  A transfer needs equal block
 * lengths and the peer's current registration (-6 otherwise); the wire counters count
 * the bytes of posted transfers (sent) and polled completions (recv).  deregister
 * waits for every posted copy that still reads or writes the block, and destroy for
 * every copy reading the agent's blocks or queued to it, so the caller may release a
 * block's memory as soon as either returns.  All calls on one pair are serialised by
 * a mutex; strings are NUL-terminated host memory.
 * ------------------------------------------------------------------------------- */
#define HCP_BLOCK_AGENT_MAX 64
#define HCP_BLOCK_META_MAX 256

enum hcp_block_mem_type { HCP_BLOCK_DRAM = 0, HCP_BLOCK_VRAM = 1 };

typedef struct hcp_block_desc {
  uint64_t addr;
  uint64_t len;
  uint64_t dev_id;
  int32_t mem_type;                 /* hcp_block_mem_type */
  uint32_t meta_len;
  uint8_t meta[HCP_BLOCK_META_MAX];
} hcp_block_desc;

typedef struct hcp_remote_block_desc {
  char agent[HCP_BLOCK_AGENT_MAX];  /* owner agent name */
  uint64_t block_id;                /* owner-local block id */
  hcp_block_desc desc;
} hcp_remote_block_desc;

typedef struct hcp_block_completion {
  uint64_t block_id;                /* receiver-local block that was written */
  uint64_t bytes;
} hcp_block_completion;

typedef struct hcp_block_agent hcp_block_agent;

int hcp_block_agent_pair_create(const char* name_a, const char* name_b, hcp_block_agent** a,
                                hcp_block_agent** b);
int hcp_block_agent_destroy(hcp_block_agent* agent);
int hcp_block_register(hcp_block_agent* agent, void* data, uint64_t bytes, const int64_t* shape,
                       int32_t ndim, uint64_t* block_id, hcp_block_desc* desc_out);
int hcp_block_deregister(hcp_block_agent* agent, uint64_t block_id);
/* out may be NULL to query the size into *written. */
int hcp_block_local_metadata(const hcp_block_agent* agent, void* out, size_t capacity, size_t* written);
/* agent_out (HCP_BLOCK_AGENT_MAX bytes, may be NULL) receives the peer's agent name. */
int hcp_block_load_remote_metadata(hcp_block_agent* agent, const void* blob, size_t len, char* agent_out);
/* The descriptor `peer` advertised for block_id in its last loaded metadata. */
int hcp_block_remote_desc(const hcp_block_agent* agent, const char* peer, uint64_t block_id,
                          hcp_remote_block_desc* out);
int hcp_block_submit_transfer(hcp_block_agent* agent, uint64_t local_block_id,
                              const hcp_remote_block_desc* remote, void* stream);
int hcp_block_poll_transfers(hcp_block_agent* agent, hcp_block_completion* out, size_t capacity,
                             size_t* n);
int hcp_block_wire_bytes(const hcp_block_agent* agent, uint64_t* sent, uint64_t* recv);

/* ---------------------------------------------------------------------------------
 * Replay kernel timing (no reference counterpart; benchmark instrumentation; the
 * reference logs wall-clock compute per phase to HCP_PERF_LOG, ring.rs:820-844).
 *
 * With timing enabled, the replay driver brackets every block-kernel (kind 0), merge
 * (kind 1) and paged-gather (kind 2) launch with HIP events on the launch stream.
 * hcp_ring_replay_timing_read waits for the recorded events, writes the summed kernel
 * milliseconds and launch counts per kind into ms[3] / launches[3], and clears them.
 * ------------------------------------------------------------------------------- */
int hcp_ring_replay_timing(int32_t enable);

int hcp_ring_replay_timing_read(double* ms, int64_t* launches);

/* ---------------------------------------------------------------------------------
 * Per-ring-call trace and perf events (the JSONL perf log of ring.rs:820-844 and the
 * ring_attention event of ring.rs:1376-1395, HCP_PERF_LOG).
 *
 * hcp_ring_trace_attach: every later BF16/F16 fused-schedule replay with VANILLA
 * positions (or causal = 0) on the calling thread (hcp_ring_prefill_replay / _paged
 * taking the fused ring; the one-block fused forms run untraced) runs the traced build
 * of the fused ring kernel, which writes one record per workgroup into `buffer` (caller-
 * owned DEVICE memory of `bytes`; null detaches).  A replay needs
 * hcp_ring_trace_record_bytes(desc) bytes (-6 if the buffer is smaller).  Records are
 * 16 + 2 * num_domains 32-bit words: [0,2) s_memrealtime (100 MHz) at workgroup entry,
 * [2,4) at its end, [4,6) / [6,8) s_memtime (shader clock) at entry / end, 8 HW_ID,
 * 9 XCC_ID, 10 target domain | head group << 16, 11 query tile, 12 128-key tiles
 * folded, 13-15 zero, then per ring position s (0 = own chunk, s = source (t - s) mod N)
 * the s_memrealtime at which the workgroup moved past that source (0: not visited).
 * Each traced replay overwrites the records of the previous one.
 *
 * hcp_ring_trace_read: waits for `stream`, reads the last traced replay's records and
 * aggregates them per target domain (out[0 .. num_domains), capacity >= num_domains)
 * and for the whole launch (*launch, may be null).  compute_ms fields are CU-time
 * divided by the CUs the launch used (the time the domain's share would take with
 * the GPU to itself); span_ms is wall time from the first workgroup's start to the
 * last one's end.
 *
 * hcp_ring_trace_perf_log: the same statistics appended as one JSON line per domain
 * to `path` (null: the HCP_PERF_LOG environment variable; neither set: nothing is
 * written and 0 is returned), in the reference's ring_attention event shape:
 * {"ts","event":"ring_attention","domain","layer","total_ms","local_compute_ms",
 * "peer_compute_ms","recv_ms","send_ms","forward_ms","flush_ms","kv_sent_bytes",
 * "kv_recv_bytes","wire_sent_bytes","wire_recv_bytes","micro_blocks","num_domains",
 * "seq_len","overlap"} plus "workgroups","key_tiles","local_cu_ms","peer_cu_ms",
 * "clock_mhz","schedule".  Transfer times and wire bytes are 0 (the ring is replayed in
 * HBM); kv_recv_bytes are the peer chunks' K/V bytes the domain folded and
 * kv_sent_bytes its own chunk's bytes times the domains that folded it (Hkv layout, as
 * a multi-GPU ring would move them); micro_blocks counts the peer chunks folded.
 * ------------------------------------------------------------------------------- */
typedef struct hcp_ring_trace_domain {
  int32_t domain;
  int32_t workgroups;
  int64_t key_tiles;         /* 128-key tiles folded by the domain's workgroups */
  int64_t peer_chunks;       /* peer sources folded */
  int64_t kv_recv_bytes;
  int64_t kv_sent_bytes;
  double span_ms;
  double local_cu_ms;        /* CU-milliseconds on the domain's own chunk */
  double peer_cu_ms;         /* CU-milliseconds on peer chunks */
  double local_compute_ms;   /* local_cu_ms / cus */
  double peer_compute_ms;    /* peer_cu_ms / cus */
  double clock_mhz;          /* mean shader clock over the domain's workgroups */
} hcp_ring_trace_domain;

typedef struct hcp_ring_trace_launch {
  int64_t workgroups;
  int32_t cus;               /* distinct CUs that ran a workgroup */
  int32_t reserved0;
  double span_ms;            /* first workgroup start to last workgroup end */
  double busy_cu_ms;         /* sum of workgroup durations */
  double idle_gap_cu_ms;     /* sum over CUs of the gaps between consecutive workgroups */
  double tail_cu_ms;         /* sum over CUs of (launch end - the CU's last workgroup end) */
  double head_cu_ms;         /* sum over CUs of (the CU's first start - launch start) */
  double clock_mhz;          /* busy-time-weighted mean shader clock */
  double wg_ms_min;          /* shortest, mean and longest workgroup */
  double wg_ms_mean;
  double wg_ms_max;
} hcp_ring_trace_launch;

int hcp_ring_trace_attach(void* buffer, size_t bytes);

size_t hcp_ring_trace_record_bytes(const hcp_ring_replay_desc* desc);

int hcp_ring_trace_read(void* stream, hcp_ring_trace_domain* out, int32_t capacity, int32_t* num_domains,
                        hcp_ring_trace_launch* launch);

int hcp_ring_trace_perf_log(void* stream, int32_t layer_idx, const char* path);

/* ---------------------------------------------------------------------------------
 * Synthetic inputs (no reference counterpart; used by the benchmark).
 *
 * Writes normals n = offset .. offset+count-1 of the LCG + Box-Muller stream of
 * rust/src/smoke/reference_algo.rs:56-90 started at `seed` (normal 2j is r*cos,
 * 2j+1 is r*sin of pair j), rounded f64 -> fp32 (-> bf16/fp16), to out (dtype F32,
 * BF16 or F16), computed on the device with LCG jump-ahead.
 * ------------------------------------------------------------------------------- */
int hcp_synth_normals(uint64_t seed, int64_t offset, int64_t count, int32_t dtype, void* out,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HCP_RING_H_ */
