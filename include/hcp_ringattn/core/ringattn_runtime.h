// Domain runtime interface (the reference's include/hcp_ringattn/core/
// ringattn_runtime.h:10-29, same virtual methods and factory) and its MI355X
// implementation, HipRingAttnRuntime.
//
// The reference ships only a no-op implementation (src/ringattn_runtime.cc:12-67).
// Here CreateRingAttnRuntime("hip") returns a runtime that runs the domain's ring on
// the GPU: every runtime created in the process joins one ring registry keyed by
// domain_id; BindLayer registers a domain's local Q / K / V (device views) for a
// layer, and RunRingAttentionLayer folds the domain's own K/V and then its
// predecessors' (source (d - s) mod N, the order of mock.rs:143-149) into the state,
// with the contiguous positions of the configured chunk lengths (strategy.rs:53-63),
// through hcp_ring_block_partial.  A domain with no binding for the layer passes the
// state through unchanged, as the no-op runtime does.
#pragma once

#include <memory>
#include <string>

#include "hcp_ring.h"
#include "hcp_ringattn/core/ringattn_protocol.h"
#include "hcp_ringattn/core/status.h"

namespace hcp_ringattn {

class RingAttnRuntime {
 public:
  virtual ~RingAttnRuntime() = default;
  virtual Status Init(const RingAttnDomainConfig& config, const RingAttnConfig& global_config) = 0;
  virtual Status RunRingAttentionLayer(int layer_index, const RingAttnSoftmaxState& initial_state,
                                       RingAttnSoftmaxState* out_state) = 0;
  virtual Status Shutdown() = 0;
};

// device_type "hip" / "rocm" / "gpu" (any other name: Init fails with
// kInvalidArgument, there is no CPU path in this library).
std::unique_ptr<RingAttnRuntime> CreateRingAttnRuntime(const std::string& device_type);

class HipRingAttnRuntime : public RingAttnRuntime {
 public:
  // Registers this domain's query chunk and local K/V for `layer_index`: q [Hq, L, D],
  // k / v [Hkv, L, D] views (dtype = the global config's dtype), L = seq_chunk_len,
  // Hq = global num_heads, D = head_dim; work is enqueued on `stream`.
  virtual Status BindLayer(int layer_index, int num_kv_heads, hcp_ring_view q, hcp_ring_view k,
                           hcp_ring_view v, float scale, void* stream) = 0;
};

}  // namespace hcp_ringattn
