// Host-side launchers of the gfx950 kernels (internal to the library).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "hcp_common.hpp"

namespace hcp {

// One (query chunk, KV chunk) block partial; see block_attn.hip.
struct BlockLaunch {
  int dtype;
  const void *q, *k, *v;
  int64_t q_hs, q_ss, k_hs, k_ss, v_hs, v_ss;  // element strides
  float* o;
  float* lse;
  int hq, hkv, d;
  int64_t lq, lk, q_off, k_off;
  int causal, accumulate;
  float scale;
  bool force_general;  // take the general kernel even where the matrix-core one applies
  // Final mode (fin_out != nullptr): instead of the fp32 state (o, lse), write the
  // normalised rows in fin_dtype to fin_out[head * fin_hs + row * fin_ss + d] and the
  // LSE to fin_lse[head * fin_lse_hs + row] (after merging the running state first
  // when accumulate is set).
  void* fin_out = nullptr;
  int fin_dtype = 0;
  int64_t fin_hs = 0, fin_ss = 0;
  float* fin_lse = nullptr;
  int64_t fin_lse_hs = 0;
  // Positions mode (causal only, q_lim != nullptr): row i of the query chunk sees keys
  // [0, q_lim[i]) of the KV chunk instead of those with k_off + j <= q_off + i.
  const int32_t* q_lim = nullptr;
  // Positions mode with keys in any order: when kv_sel is non-null and *kv_sel != 0 (a
  // device flag), the kernels read K / V from the sorted-row copies k_alt / v_alt
  // ([hkv, lk, d] contiguous, strides alt_hs / alt_ss) instead of k / v.
  const int* kv_sel = nullptr;
  const void* k_alt = nullptr;
  const void* v_alt = nullptr;
  int64_t alt_hs = 0, alt_ss = 0;
};

bool block_uses_mfma(int dtype, int d);
// Whether an fp32 block runs on the fp32 matrix-core kernel (else the scalar one).
bool block_uses_mfma_f32(const BlockLaunch& L);
void launch_block_partial(const BlockLaunch& L, hipStream_t stream);
// Independent blocks (distinct outputs) in as few launches as the kernels allow: one
// launch per up to 8 head-dim-128 MFMA blocks of the same head layout, else one each.
void launch_block_group(const BlockLaunch* Ls, int n, hipStream_t stream);

// A whole single-GPU ring replay with vanilla positions in one launch (fused ring, see
// block_attn.hip): q / k / v / out are whole-sequence [heads, S, D] views whose rows
// are the domains' chunks in order; lse [hq, lse_hs >= S] or null.
struct RingLaunch {
  int dtype, d, hq, hkv, n, causal;
  float scale;
  const void *q, *k, *v;
  int64_t q_hs, q_ss, k_hs, k_ss, v_hs, v_ss;
  void* out;
  int64_t out_hs, out_ss;
  float* lse;
  int64_t lse_hs;
  const int64_t* len;  // HOST array of n chunk lengths
  // Traced launch (non-null): one record of trace_stride >= ring_trace_words(n) 32-bit
  // words per workgroup (layout in block_attn.hip, kTraceHeaderWords).
  uint32_t* trace = nullptr;
  int trace_stride = 0;
};
bool ring_fused_applies(int dtype, int d);
void launch_ring_fused(const RingLaunch& L, hipStream_t stream);
// Workgroups of the fused ring launch for this head layout and chunk list.
int64_t ring_fused_workgroups(int hq, int hkv, int n, const int64_t* len);
// 32-bit words of one trace record of an n-domain fused ring.
int ring_trace_words(int n);

void launch_lse_merge(int n, const float* const* o_parts, const float* const* lse_parts, int heads,
                      int64_t q_len, int d, int out_dtype, void* out, int64_t out_hs, int64_t out_ss,
                      float* lse_out, int64_t lse_out_hs, hipStream_t stream);

// One token range of one sequence for the batched paged copy.
struct PagedRangeDesc {
  const int32_t* table;
  int64_t table_seq_offset;
  int64_t t0, t1;
  void* k_buf;
  void* v_buf;
  int64_t head_stride, seq_stride;  // elements
};
void launch_paged_copy_batch(bool gather, void* pool, int64_t num_blocks, int bs, int hkv, int d,
                             int elem_bytes, int n, const PagedRangeDesc* ranges, int zero_tail,
                             int* err, hipStream_t stream);

void launch_paged_copy(bool gather, void* pool, int64_t num_blocks, int bs, int hkv, int d,
                       int elem_bytes, const int32_t* table, int64_t table_seq_offset, int64_t t0,
                       int64_t t1, void* k_buf, void* v_buf, int64_t head_stride, int64_t seq_stride,
                       int zero_tail, int* err, hipStream_t stream);

size_t decode_workspace_bytes(int dtype, int batch, int hq, int hkv, int d, int64_t t0, int64_t t1);
void launch_paged_decode(int dtype, int batch, int hq, int hkv, int d, const void* q, int64_t q_bs,
                         int64_t q_hs, const void* pool, int64_t num_blocks, int bs,
                         const int32_t* tables, int64_t table_stride, int64_t table_len,
                         const int32_t* seq_lens, int64_t t0, int64_t t1, float scale, float* o,
                         float* lse, void* ws, size_t ws_bytes, int* err, hipStream_t stream);

// Scheduling strategies (strategy.rs:14-24) and their closed-form positions; see
// positions.hip.
constexpr int kMaxDomains = 64;
enum Strategy : int32_t { kStrategyVanilla = 0, kStrategyStriped = 1, kStrategyZigZag = 2 };
struct StrategySpec {
  int32_t strategy;
  int32_t n;
  int64_t chunks[kMaxDomains];
};
// Global position of the i-th token (local storage order) of domain d.
__host__ __device__ int64_t strategy_position(const StrategySpec& s, int d, int64_t i);
void launch_domain_positions(const StrategySpec& s, int64_t seq, int64_t* out, hipStream_t stream);
// pos: a permutation of [0, n).  rows[pos[r]] = r, lim[r] = pos[r] + 1 (the keys of the
// position-ordered list row r sees), *flag = 1; a position out of range sets bit 1 of
// *err.
void launch_position_inverse(const int64_t* pos, int64_t n, int32_t* rows, int32_t* lim, int* flag, int* err,
                             hipStream_t stream);

// lim[src * lim_stride + r] = #{j < k_len[src] : k_pos[k_off[src] + j] <= q_pos[r]} for
// r < n_q, by binary search over a non-decreasing key list: k_pos, or k_pos_sorted when
// sel is non-null and *sel != 0 (a list launch_key_sort found out of order).  With err
// non-null, sets error bit 1 when the searched list is not non-decreasing.
struct KeyLimitArgs {
  const int64_t* q_pos;
  int64_t n_q;
  const int64_t* k_pos;
  int64_t k_off[kMaxDomains];
  int64_t k_len[kMaxDomains];
  int32_t* lim;
  int64_t lim_stride;
  int* err;
  const int* sel;
  const int64_t* k_pos_sorted;
};
void launch_key_limits(const KeyLimitArgs& a, int n_src, int64_t max_k_len, hipStream_t stream);

// Keys in any order (positions.hip): *flag = 1 iff k[0 .. n) is not non-decreasing;
// then (and only then) the (key, row) pairs are sorted into key[f] / row[f] with
// f = key_sort_passes(n) % 2 (key[1 - f] / row[1 - f] are scratch).  Stream-ordered,
// no host synchronisation.
int key_sort_passes(int64_t n);
void launch_key_sort(const int64_t* k, int64_t n, int* flag, int64_t* const key[2], int32_t* const row[2],
                     hipStream_t stream);
// When *flag != 0: kc / vc [hkv, n, row_bytes] (contiguous) get row rows[r] of the K / V
// views for every head (byte strides); nothing otherwise.
struct KvSortedGather {
  const int* flag;
  const int32_t* rows;
  int64_t n;
  int32_t hkv;
  int64_t row_bytes;
  const char* k;
  const char* v;
  int64_t k_hs_bytes, k_ss_bytes, v_hs_bytes, v_ss_bytes;
  char* kc;
  char* vc;
};
void launch_kv_sorted_gather(const KvSortedGather& g, hipStream_t stream);

// Wire frames (wire.hip): fp32 payload segments <-> strided storage views, the
// serde_json-compatible headers and a reader for them.
void launch_wire_segment(bool pack, int dtype, void* tensor, float* wire, int64_t rows, int64_t rep, int64_t len,
                         int64_t dim, int64_t hs, int64_t ss, hipStream_t stream);
const char* dtype_wire_name(int dtype);
int dtype_from_wire_name(const std::string& s);
std::string json_f64(double x);
std::string kv_frame_meta(int64_t layer_idx, int64_t start, int64_t end, int dtype, int64_t heads, int64_t len,
                          int64_t dim, bool positions);
std::string packet_frame_meta(int64_t layer_idx, int q_dtype, int o_dtype, int64_t batch, int64_t heads,
                              int64_t dim, double scale);
// A JSON value restricted to what the frame headers hold.
struct JVal {
  enum Kind { kNull, kNum, kStr, kArr, kObj } kind = kNull;
  double num = 0;
  bool integral = false;
  int64_t inum = 0;
  std::string str;
  std::vector<JVal> arr;
  std::map<std::string, JVal> obj;
};
JVal parse_frame_meta(const unsigned char* frame, size_t n, size_t* header_bytes);

// Fused QKV projection + RoPE + KV append (qkv_rope.hip).
struct QkvArgs {
  const uint16_t* x;
  int64_t x_ss;                 // elements between token rows
  const uint16_t* w[3];         // q, k, v weights [out, hidden], rows contiguous
  const uint16_t* bias[3];      // or null
  int32_t nq, nkv;              // Hq * D, Hkv * D
  int32_t hidden;
  int32_t tokens;
  int32_t rope;
  const int64_t* pos;           // [tokens] global positions (RoPE rows)
  const float* rope_cos;        // [rope_rows, D/2]
  const float* rope_sin;
  int64_t rope_rows;
  uint16_t* out[3];             // views (k / v null when paged)
  int64_t out_hs[3], out_ss[3];
  uint16_t* pool;               // paged append of k / v
  int64_t plane_elems, num_blocks;
  int32_t bs, hkv;
  const int32_t* table;
  int64_t table_len, table_off, t0;
  int* err;
  int32_t n_tiles_n, n_tiles_m;
};
void launch_qkv_rope(int dtype, int d, QkvArgs& a, hipStream_t stream);
// cos / sin tables [rows, d/2] of RotaryEmbedding (rotary.rs:64-97).
void launch_rope_table(int d, int64_t rows, double base, float* cos, float* sin, hipStream_t stream);

void launch_synth_normals(uint64_t seed, int64_t offset, int64_t count, int dtype, void* out,
                          hipStream_t stream);

}  // namespace hcp
