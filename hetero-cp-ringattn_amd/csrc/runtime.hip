// HipRingAttnRuntime: the domain runtime interface of the reference
// (include/hcp_ringattn/core/ringattn_runtime.h:10-29; only a no-op implementation
// exists there, src/ringattn_runtime.cc:12-67) backed by the ring kernels.
//
// All runtimes of a process share one ring registry keyed by (domain_id, layer).  A
// domain's RunRingAttentionLayer folds its own K/V and then its predecessors' in ring
// order into its query chunk's state, each source one hcp_ring_block_partial launch
// (accumulate mode after the first), with the causal masks of the contiguous chunk
// positions.  The state leaves the runtime in the re-entry form of ring.rs:585-587
// (running_max = LSE, running_sum = 1, output = normalised O); a state given on entry is
// merged in first (its LSE = running_max + ln running_sum).
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "hcp_ringattn/core/ringattn_runtime.h"
#include "kernels.hpp"

namespace hcp_ringattn {
namespace {

using Code = Status::Code;

struct Binding {
  int num_kv_heads = 0;
  hcp_ring_view q{}, k{}, v{};
  float scale = 0.f;
  hipStream_t stream = nullptr;
};

struct Registry {
  std::mutex mu;
  std::map<std::pair<std::string, int>, Binding> layers;
};
Registry& registry() {
  static Registry r;
  return r;
}

int abi_dtype(TensorDType t) {
  switch (t) {
    case TensorDType::kFloat16: return HCP_DTYPE_F16;
    case TensorDType::kBFloat16: return HCP_DTYPE_BF16;
    case TensorDType::kFloat32: return HCP_DTYPE_F32;
    default: return -1;
  }
}

BoundaryTensor f32_tensor(const char* name, const char* layout, std::vector<int64_t> shape, const float* data,
                          size_t n) {
  BoundaryTensor t;
  t.name = name;
  t.dtype = TensorDType::kFloat32;
  t.layout = layout;
  t.shape = std::move(shape);
  t.payload.resize(n * sizeof(float));
  std::memcpy(t.payload.data(), data, n * sizeof(float));
  return t;
}

class Runtime final : public HipRingAttnRuntime {
 public:
  explicit Runtime(std::string device_type) : device_type_(std::move(device_type)) {}
  ~Runtime() override { Shutdown(); }

  Status Init(const RingAttnDomainConfig& config, const RingAttnConfig& global) override {
    // The reference's checks (src/ringattn_runtime.cc:17-37), then what the GPU path needs.
    if (config.domain_id.empty()) return Status::Error(Code::kInvalidArgument, "domain_id must not be empty");
    if (config.seq_chunk_len <= 0)
      return Status::Error(Code::kInvalidArgument, "seq_chunk_len must be positive for domain=", config.domain_id);
    if (config.block_size <= 0)
      return Status::Error(Code::kInvalidArgument, "block_size must be positive for domain=", config.domain_id);
    if (global.global_seq_len <= 0 || global.num_heads <= 0 || global.head_dim <= 0)
      return Status::Error(Code::kInvalidArgument, "global config is incomplete");
    for (const std::string& dev : {device_type_, config.device}) {
      if (dev != "hip" && dev != "rocm" && dev != "gpu")
        return Status::Error(Code::kInvalidArgument, "device '", dev,
                             "' is not served by this library (use \"hip\"; there is no CPU path)");
    }
    if (abi_dtype(global.dtype) < 0) return Status::Error(Code::kInvalidArgument, "dtype must be F16, BF16 or F32");
    int me = -1;
    int64_t acc = 0;
    offsets_.clear();
    lens_.clear();
    ids_.clear();
    for (size_t i = 0; i < global.domains.size(); ++i) {
      const RingAttnDomainConfig& dc = global.domains[i];
      if (dc.seq_chunk_len <= 0)
        return Status::Error(Code::kInvalidArgument, "seq_chunk_len must be positive for domain=", dc.domain_id);
      if (dc.domain_id == config.domain_id) me = static_cast<int>(i);
      offsets_.push_back(acc);
      lens_.push_back(dc.seq_chunk_len);
      ids_.push_back(dc.domain_id);
      acc += dc.seq_chunk_len;
    }
    if (me < 0) return Status::Error(Code::kInvalidArgument, "domain ", config.domain_id, " is not in the global config");
    if (global.domains[me].seq_chunk_len != config.seq_chunk_len)
      return Status::Error(Code::kInvalidArgument, "seq_chunk_len differs from the global config for ", config.domain_id);
    if (acc != global.global_seq_len)  // InvalidChunkSum, rust/src/error.rs:15-16
      return Status::Error(Code::kInvalidArgument, "invalid chunk sum: actual ", acc, ", expected ",
                           global.global_seq_len);
    config_ = config;
    global_ = global;
    index_ = me;
    ready_ = true;
    return Status::Ok();
  }

  Status BindLayer(int layer, int num_kv_heads, hcp_ring_view q, hcp_ring_view k, hcp_ring_view v, float scale,
                   void* stream) override {
    if (!ready_) return Status::Error(Code::kInvalidArgument, "BindLayer before Init");
    if (num_kv_heads <= 0 || global_.num_heads % num_kv_heads != 0)
      return Status::Error(Code::kInvalidArgument, "num_heads must be a multiple of num_kv_heads");
    if (q.data == nullptr || k.data == nullptr || v.data == nullptr || !(scale > 0.f))
      return Status::Error(Code::kInvalidArgument, "null q / k / v or non-positive scale");
    Binding b;
    b.num_kv_heads = num_kv_heads;
    b.q = q;
    b.k = k;
    b.v = v;
    b.scale = scale;
    b.stream = static_cast<hipStream_t>(stream);
    Registry& r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    r.layers[{config_.domain_id, layer}] = b;
    return Status::Ok();
  }

  Status RunRingAttentionLayer(int layer, const RingAttnSoftmaxState& in, RingAttnSoftmaxState* out) override {
    if (out == nullptr) return Status::Error(Code::kInvalidArgument, "out_state must not be null");
    if (!ready_) return Status::Error(Code::kInvalidArgument, "RunRingAttentionLayer before Init");
    std::vector<Binding> src(ids_.size());
    std::vector<bool> have(ids_.size(), false);
    {
      Registry& r = registry();
      std::lock_guard<std::mutex> lock(r.mu);
      for (size_t i = 0; i < ids_.size(); ++i) {
        auto it = r.layers.find({ids_[i], layer});
        if (it != r.layers.end()) {
          src[i] = it->second;
          have[i] = true;
        }
      }
    }
    if (!have[index_]) {  // nothing bound here: the state passes through
      *out = in;
      return Status::Ok();
    }
    try {
      run(layer, src, have, in, out);
    } catch (const hcp::Error& e) {
      return Status::Error(e.code == -6 ? Code::kInvalidArgument : Code::kInternal, e.what());
    } catch (const std::exception& e) {
      return Status::Error(Code::kInternal, e.what());
    }
    return Status::Ok();
  }

  Status Shutdown() override {
    if (o_) (void)hipFree(o_);
    if (lse_) (void)hipFree(lse_);
    o_ = lse_ = nullptr;
    state_elems_ = 0;
    if (ready_) {
      Registry& r = registry();
      std::lock_guard<std::mutex> lock(r.mu);
      for (auto it = r.layers.begin(); it != r.layers.end();) {
        if (it->first.first == config_.domain_id) it = r.layers.erase(it);
        else ++it;
      }
    }
    ready_ = false;
    return Status::Ok();
  }

 private:
  void run(int layer, const std::vector<Binding>& src, const std::vector<bool>& have, const RingAttnSoftmaxState& in,
           RingAttnSoftmaxState* out) {
    const Binding& me = src[index_];
    const int64_t hq = global_.num_heads, d = global_.head_dim, lq = lens_[index_];
    const size_t rows = static_cast<size_t>(hq) * lq;
    if (state_elems_ < rows) {
      if (o_) HCP_HIP(hipFree(o_));
      if (lse_) HCP_HIP(hipFree(lse_));
      o_ = lse_ = nullptr;
      HCP_HIP(hipMalloc(&o_, rows * d * sizeof(float)));
      HCP_HIP(hipMalloc(&lse_, rows * sizeof(float)));
      state_elems_ = rows;
    }
    bool seeded = false;
    if (in.seq_len > 0) {  // merge the caller's state first: LSE = m + ln l
      hcp::require(in.seq_len == lq && in.num_heads == hq && in.head_dim == d,
                   "initial state shape does not match the domain's query chunk");
      hcp::require(in.running_max.payload.size() == rows * 4 && in.running_sum.payload.size() == rows * 4 &&
                       in.output.payload.size() == rows * d * 4,
                   "initial state tensors must be fp32 [H, L], [H, L], [H, L, D]");
      std::vector<float> lse(rows);
      const float* m = reinterpret_cast<const float*>(in.running_max.payload.data());
      const float* l = reinterpret_cast<const float*>(in.running_sum.payload.data());
      for (size_t i = 0; i < rows; ++i) lse[i] = l[i] > 0.f ? m[i] + std::log(l[i]) : -INFINITY;
      HCP_HIP(hipMemcpyAsync(lse_, lse.data(), rows * 4, hipMemcpyHostToDevice, me.stream));
      HCP_HIP(hipMemcpyAsync(o_, in.output.payload.data(), rows * d * 4, hipMemcpyHostToDevice, me.stream));
      HCP_HIP(hipStreamSynchronize(me.stream));
      seeded = true;
    }
    const int n = static_cast<int>(ids_.size());
    for (int s = 0; s < n; ++s) {
      const int j = ((index_ - s) % n + n) % n;  // local first, then the predecessor chain
      if (offsets_[j] > offsets_[index_] + lq - 1) continue;  // wholly in the future (ring.rs:222-228)
      hcp::require(have[j], "domain " + ids_[j] + " has no inputs for layer " + std::to_string(layer));
      hcp::require(src[j].num_kv_heads == me.num_kv_heads, "domains disagree on num_kv_heads");
      hcp_ring_block_desc bd{};
      bd.dtype = abi_dtype(global_.dtype);
      bd.num_q_heads = static_cast<int32_t>(hq);
      bd.num_kv_heads = me.num_kv_heads;
      bd.head_dim = static_cast<int32_t>(d);
      bd.q_len = lq;
      bd.kv_len = lens_[j];
      bd.q_offset = offsets_[index_];
      bd.kv_offset = offsets_[j];
      bd.causal = 1;
      bd.accumulate = seeded ? 1 : 0;
      bd.scale = me.scale;
      if (hcp_ring_block_partial(&bd, me.q, src[j].k, src[j].v, o_, lse_, me.stream) != 0)
        throw hcp::Error(-2, std::string("block partial failed: ") + hcp_ring_last_error());
      seeded = true;
    }
    std::vector<float> lse(rows), o(rows * d), ones(rows, 1.f);
    HCP_HIP(hipMemcpyAsync(lse.data(), lse_, rows * 4, hipMemcpyDeviceToHost, me.stream));
    HCP_HIP(hipMemcpyAsync(o.data(), o_, rows * d * 4, hipMemcpyDeviceToHost, me.stream));
    HCP_HIP(hipStreamSynchronize(me.stream));
    out->seq_len = lq;
    out->num_heads = hq;
    out->head_dim = d;
    out->running_max = f32_tensor("running_max", "hl", {hq, lq}, lse.data(), rows);
    out->running_sum = f32_tensor("running_sum", "hl", {hq, lq}, ones.data(), rows);
    out->output = f32_tensor("output", "hld", {hq, lq, d}, o.data(), rows * d);
  }

  std::string device_type_;
  RingAttnDomainConfig config_;
  RingAttnConfig global_;
  std::vector<int64_t> offsets_, lens_;
  std::vector<std::string> ids_;
  int index_ = -1;
  bool ready_ = false;
  float* o_ = nullptr;
  float* lse_ = nullptr;
  size_t state_elems_ = 0;
};

}  // namespace

std::unique_ptr<RingAttnRuntime> CreateRingAttnRuntime(const std::string& device_type) {
  return std::make_unique<Runtime>(device_type);
}

}  // namespace hcp_ringattn
