// Block-direct transport on one GPU: the KvBlockTransport lifecycle of
// rust/src/model/transport/block_transport.rs:36-126 (register -> local metadata ->
// load remote metadata -> submit transfer -> poll completions) with the semantics of its
// in-memory reference implementation (serialized_block.rs:53-190): agents come in
// linked pairs, a transfer posted on one lands in the peer's registered block, and
// the peer observes it by polling.  Here the blocks are device (or host) memory, the
// transfer is an asynchronous copy on the caller's stream -- the raw bytes, as NIXL
// moves registered memory -- and its completion is an event query, so polling never
// blocks.
//
// Metadata blobs are bincode 1.3.3 (rust/Cargo.lock) in its default configuration:
// little-endian, u64 lengths for strings and sequences, u32 enum variant indices,
// fields in declaration order -- AgentMetadata { agent, blocks: [RemoteBlockDesc
// { agent, block_id, desc: BlockDesc { addr, len, dev_id, mem_type, meta } }] }.
// A registered block's meta is serde_json's compact text of its shape ("[1,2,3,4]"),
// as register_block writes it (serialized_block.rs:103-115).
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "../../include/hcp_ring.h"

namespace hcp {
namespace {

struct Pending {
  uint64_t block_id;   // destination block (the receiving agent's)
  uint64_t bytes;
  hipEvent_t done;
  int src_side;        // the posting agent's side within the pair
  uint64_t src_block;  // its local source block
};

// State shared by the two agents of a pair: each agent's inbox of posted transfers.
struct PairState {
  std::mutex mu;
  std::deque<Pending> inbox[2];
  std::vector<hipEvent_t> events;  // recycled completion events
};

struct Block {
  hcp_block_desc desc;
};

}  // namespace
}  // namespace hcp

struct hcp_block_agent {
  std::string name;
  int side;  // 0 or 1 within its pair
  std::shared_ptr<hcp::PairState> pair;
  hcp_block_agent* peer = nullptr;
  uint64_t next_id = 0;
  std::map<uint64_t, hcp::Block> blocks;
  // descriptors advertised by peers, by agent name then block id
  std::map<std::string, std::map<uint64_t, hcp_remote_block_desc>> remote;
  uint64_t sent = 0, recv = 0;
};

namespace hcp {
namespace {

void put_u64(std::string& b, uint64_t v) {
  for (int i = 0; i < 8; ++i) b.push_back(static_cast<char>((v >> (8 * i)) & 0xff));
}
void put_u32(std::string& b, uint32_t v) {
  for (int i = 0; i < 4; ++i) b.push_back(static_cast<char>((v >> (8 * i)) & 0xff));
}
void put_bytes(std::string& b, const void* p, size_t n) {
  put_u64(b, n);
  b.append(static_cast<const char*>(p), n);
}

struct Reader {
  const unsigned char* p;
  size_t n, at = 0;
  void need(size_t k) {
    require(at + k <= n, "agent metadata: blob ends early at byte " + std::to_string(at));
  }
  uint64_t u64() {
    need(8);
    uint64_t v = 0;
    for (int i = 0; i < 8; ++i) v |= static_cast<uint64_t>(p[at + i]) << (8 * i);
    at += 8;
    return v;
  }
  uint32_t u32() {
    need(4);
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) v |= static_cast<uint32_t>(p[at + i]) << (8 * i);
    at += 4;
    return v;
  }
  std::string bytes(size_t max) {
    const uint64_t k = u64();
    require(k <= max, "agent metadata: field of " + std::to_string(k) + " bytes exceeds " + std::to_string(max));
    need(k);
    std::string s(reinterpret_cast<const char*>(p + at), k);
    at += k;
    return s;
  }
};

void serialize_desc(std::string& b, const hcp_block_desc& d) {
  put_u64(b, d.addr);
  put_u64(b, d.len);
  put_u64(b, d.dev_id);
  put_u32(b, static_cast<uint32_t>(d.mem_type));
  put_bytes(b, d.meta, d.meta_len);
}

std::string agent_metadata(const hcp_block_agent& a) {
  std::string b;
  put_bytes(b, a.name.data(), a.name.size());
  put_u64(b, a.blocks.size());
  for (const auto& kv : a.blocks) {  // ascending block id
    put_bytes(b, a.name.data(), a.name.size());
    put_u64(b, kv.first);
    serialize_desc(b, kv.second.desc);
  }
  return b;
}

void check_name(const char* name) {
  require(name != nullptr && name[0] != '\0', "agent name must be non-empty");
  require(std::strlen(name) < HCP_BLOCK_AGENT_MAX, "agent name too long");
}

void copy_name(char* dst, const std::string& s) {
  std::memset(dst, 0, HCP_BLOCK_AGENT_MAX);
  std::memcpy(dst, s.data(), s.size());
}

bool same_desc(const hcp_block_desc& x, const hcp_block_desc& y) {
  return x.addr == y.addr && x.len == y.len && x.dev_id == y.dev_id && x.mem_type == y.mem_type &&
         x.meta_len == y.meta_len && std::memcmp(x.meta, y.meta, x.meta_len) == 0;
}

// Waits for every queued copy that reads from or writes into block `block_id` of the
// agent on `side` (all blocks when block_id is UINT64_MAX).  The copies stay queued,
// so the receiver still observes them through poll_transfers.  Called with the pair's
// mutex held.
void wait_block_copies(PairState& st, int side, uint64_t block_id) {
  for (int q = 0; q < 2; ++q)
    for (const Pending& p : st.inbox[q]) {
      const bool writes = q == side && (block_id == UINT64_MAX || p.block_id == block_id);
      const bool reads = p.src_side == side && (block_id == UINT64_MAX || p.src_block == block_id);
      if (writes || reads) HCP_HIP(hipEventSynchronize(p.done));
    }
}

}  // namespace

// Shared with capi.hip's boundary helpers.
int block_transport_guard(const char* fn, const std::function<void()>& body);

}  // namespace hcp

using namespace hcp;

extern "C" {

int hcp_block_agent_pair_create(const char* name_a, const char* name_b, hcp_block_agent** a, hcp_block_agent** b) {
  return block_transport_guard(__func__, [&] {
    require(a != nullptr && b != nullptr, "null agent out-pointer");
    check_name(name_a);
    check_name(name_b);
    require(std::strcmp(name_a, name_b) != 0, "the two agents of a pair need different names");
    auto st = std::make_shared<PairState>();
    std::unique_ptr<hcp_block_agent> x(new hcp_block_agent), y(new hcp_block_agent);
    x->name = name_a;
    y->name = name_b;
    x->side = 0;
    y->side = 1;
    x->pair = st;
    y->pair = st;
    x->peer = y.get();
    y->peer = x.get();
    *a = x.release();
    *b = y.release();
  });
}

int hcp_block_agent_destroy(hcp_block_agent* agent) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr, "null agent");
    {
      std::lock_guard<std::mutex> lock(agent->pair->mu);
      if (agent->peer != nullptr) agent->peer->peer = nullptr;
      // Copies this agent posted that read its blocks: wait for them (the peer still
      // polls their completions).  Transfers queued for this agent: wait, then drop.
      wait_block_copies(*agent->pair, agent->side, UINT64_MAX);
      for (Pending& p : agent->pair->inbox[agent->side]) agent->pair->events.push_back(p.done);
      agent->pair->inbox[agent->side].clear();
      if (agent->peer == nullptr && agent->pair.use_count() == 1) {
        for (hipEvent_t e : agent->pair->events) (void)hipEventDestroy(e);
        agent->pair->events.clear();
      }
    }
    delete agent;
  });
}

int hcp_block_register(hcp_block_agent* agent, void* data, uint64_t bytes, const int64_t* shape, int32_t ndim,
                       uint64_t* block_id, hcp_block_desc* desc_out) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr && data != nullptr && block_id != nullptr, "null agent, data or block_id");
    require(bytes > 0, "bytes must be positive");
    require(ndim >= 0 && ndim <= 16 && (ndim == 0 || shape != nullptr), "ndim must be in [0, 16]");
    hcp_block_desc d{};
    d.addr = reinterpret_cast<uint64_t>(data);
    d.len = bytes;
    // device memory registers as VRAM on its device, anything else as DRAM
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, data) == hipSuccess && attr.type == hipMemoryTypeDevice) {
      d.mem_type = HCP_BLOCK_VRAM;
      d.dev_id = static_cast<uint64_t>(attr.device);
    } else {
      (void)hipGetLastError();
      d.mem_type = HCP_BLOCK_DRAM;
      d.dev_id = 0;
    }
    std::string meta = "[";
    for (int i = 0; i < ndim; ++i) meta += (i ? "," : "") + std::to_string(shape[i]);
    meta += "]";
    require(meta.size() <= HCP_BLOCK_META_MAX, "shape text exceeds the descriptor's meta field");
    d.meta_len = static_cast<uint32_t>(meta.size());
    std::memcpy(d.meta, meta.data(), meta.size());
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    const uint64_t id = agent->next_id++;
    agent->blocks[id] = Block{d};
    *block_id = id;
    if (desc_out != nullptr) *desc_out = d;
  });
}

int hcp_block_deregister(hcp_block_agent* agent, uint64_t block_id) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr, "null agent");
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    require(agent->blocks.count(block_id) == 1, "block " + std::to_string(block_id) + " is not registered");
    // The caller may free the block's memory once this returns: finish every copy
    // that still reads or writes it (the reference's in-memory transport copies
    // synchronously, so it has no such window).
    wait_block_copies(*agent->pair, agent->side, block_id);
    agent->blocks.erase(block_id);
  });
}

int hcp_block_local_metadata(const hcp_block_agent* agent, void* out, size_t capacity, size_t* written) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr && written != nullptr, "null agent or written");
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    const std::string blob = agent_metadata(*agent);
    *written = blob.size();
    if (out != nullptr) {
      require(capacity >= blob.size(), "metadata needs " + std::to_string(blob.size()) + " bytes");
      std::memcpy(out, blob.data(), blob.size());
    }
  });
}

int hcp_block_load_remote_metadata(hcp_block_agent* agent, const void* blob, size_t len, char* agent_out) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr && blob != nullptr, "null agent or blob");
    Reader r{static_cast<const unsigned char*>(blob), len};
    const std::string name = r.bytes(HCP_BLOCK_AGENT_MAX - 1);
    const uint64_t n = r.u64();
    require(n <= (len - r.at) / 45, "agent metadata: block count exceeds the blob");  // 45 = smallest entry
    std::map<uint64_t, hcp_remote_block_desc> got;
    for (uint64_t i = 0; i < n; ++i) {
      hcp_remote_block_desc rd{};
      copy_name(rd.agent, r.bytes(HCP_BLOCK_AGENT_MAX - 1));
      rd.block_id = r.u64();
      rd.desc.addr = r.u64();
      rd.desc.len = r.u64();
      rd.desc.dev_id = r.u64();
      const uint32_t mt = r.u32();
      require(mt <= 1, "agent metadata: mem_type variant " + std::to_string(mt));
      rd.desc.mem_type = static_cast<int32_t>(mt);
      const std::string meta = r.bytes(HCP_BLOCK_META_MAX);
      rd.desc.meta_len = static_cast<uint32_t>(meta.size());
      std::memcpy(rd.desc.meta, meta.data(), meta.size());
      got[rd.block_id] = rd;
    }
    require(r.at == len, "agent metadata: " + std::to_string(len - r.at) + " trailing bytes");
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    agent->remote[name] = std::move(got);
    if (agent_out != nullptr) copy_name(agent_out, name);
  });
}

int hcp_block_remote_desc(const hcp_block_agent* agent, const char* peer, uint64_t block_id,
                          hcp_remote_block_desc* out) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr && peer != nullptr && out != nullptr, "null agent, peer or out");
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    auto it = agent->remote.find(peer);
    require(it != agent->remote.end(), std::string("no metadata loaded for agent ") + peer);
    auto jt = it->second.find(block_id);
    require(jt != it->second.end(), "agent " + std::string(peer) + " advertised no block " + std::to_string(block_id));
    *out = jt->second;
  });
}

int hcp_block_submit_transfer(hcp_block_agent* agent, uint64_t local_block_id, const hcp_remote_block_desc* remote,
                              void* stream) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr && remote != nullptr, "null agent or remote descriptor");
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    auto lt = agent->blocks.find(local_block_id);
    require(lt != agent->blocks.end(), "local block " + std::to_string(local_block_id) + " not registered");
    hcp_block_agent* peer = agent->peer;
    require(peer != nullptr, "the peer agent was destroyed");
    require(std::strncmp(remote->agent, peer->name.c_str(), HCP_BLOCK_AGENT_MAX) == 0,
            "remote block belongs to agent " + std::string(remote->agent, strnlen(remote->agent, HCP_BLOCK_AGENT_MAX)) +
                ", not to the peer " + peer->name);
    auto rt = peer->blocks.find(remote->block_id);
    require(rt != peer->blocks.end(), "the peer has no registered block " + std::to_string(remote->block_id));
    require(same_desc(rt->second.desc, remote->desc), "remote descriptor does not match the peer's registration");
    const hcp_block_desc& src = lt->second.desc;
    const hcp_block_desc& dst = rt->second.desc;
    require(src.len == dst.len, "local block has " + std::to_string(src.len) + " bytes, remote " +
                                    std::to_string(dst.len));
    hipStream_t s = static_cast<hipStream_t>(stream);
    HCP_HIP(hipMemcpyAsync(reinterpret_cast<void*>(dst.addr), reinterpret_cast<const void*>(src.addr), src.len,
                           hipMemcpyDefault, s));
    hipEvent_t e;
    if (!agent->pair->events.empty()) {
      e = agent->pair->events.back();
      agent->pair->events.pop_back();
    } else {
      HCP_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    HCP_HIP(hipEventRecord(e, s));
    agent->pair->inbox[peer->side].push_back(Pending{remote->block_id, src.len, e, agent->side, local_block_id});
    agent->sent += src.len;
  });
}

int hcp_block_poll_transfers(hcp_block_agent* agent, hcp_block_completion* out, size_t capacity, size_t* n) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr && n != nullptr, "null agent or n");
    require(out != nullptr || capacity == 0, "null completions array");
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    auto& q = agent->pair->inbox[agent->side];
    size_t k = 0;
    for (auto it = q.begin(); it != q.end() && k < capacity;) {
      const hipError_t st = hipEventQuery(it->done);
      if (st == hipErrorNotReady) {
        (void)hipGetLastError();
        ++it;
        continue;
      }
      HCP_HIP(st);
      out[k++] = hcp_block_completion{it->block_id, it->bytes};
      agent->recv += it->bytes;
      agent->pair->events.push_back(it->done);
      it = q.erase(it);
    }
    *n = k;
  });
}

int hcp_block_wire_bytes(const hcp_block_agent* agent, uint64_t* sent, uint64_t* recv) {
  return block_transport_guard(__func__, [&] {
    require(agent != nullptr && sent != nullptr && recv != nullptr, "null agent, sent or recv");
    std::lock_guard<std::mutex> lock(agent->pair->mu);
    *sent = agent->sent;
    *recv = agent->recv;
  });
}

}  // extern "C"
