// The reference's GPU session lifecycle around the paged cache, for the ops
// of this library: the executor loop of the safetensors session
// (execute_graph_gpu_with_weights_and_cache, onnx-rt/src/cuda/gpu_executor.rs:
// 290-433) and the session that owns the cache (Session::run_safetensors and
// reset_kv_cache, onnx-rt/src/session.rs:969-1049; the cache allocation and
// Gemma layer kinds, session.rs:579-593 and :1221-1233).
//
//   reference                                        here (namespace sai::rocm)
//   graph::ExecutionNode (the fields the loop reads) ExecutionNode
//   SessionError (session.rs:27-76)                  SessionError
//   dispatch_gpu_node (gpu_executor.rs:490-514)      dispatch_gpu_node
//   execute_graph_gpu_with_weights_and_cache         execute_graph_gpu_with_cache
//   layer_kinds_for_gemma (session.rs:579-593)       layer_kinds_for_gemma
//   Session (safetensors + cuda fields)              GpuSession
//
// Differences by design: the node set is this library's (GroupQueryAttention,
// RotaryEmbedding; any other op is the executor's "no GPU implementation"
// error, for the caller to route elsewhere); inputs are device tensors moved
// into the value map (no host bridge, no initializers: the weights belong to
// the ops this library does not implement); the cache is the quantised paged
// one, and rank-3 GQA nodes use it (the reference bypasses it for rank-3).
#ifndef SAI_GQA_SESSION_HPP
#define SAI_GQA_SESSION_HPP

#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "gqa_host.hpp"

namespace sai::rocm {

// graph::ExecutionNode, the fields the executor reads. Empty input names are
// absent optional inputs.
struct ExecutionNode {
  std::string name;
  std::string op_type;
  std::vector<std::string> inputs;
  std::vector<std::string> outputs;
  std::vector<AttributeProto> attributes;
};

// session.rs:27-76, the variants this path raises; to_string() is its Display.
struct SessionError {
  enum class Kind { ExecutionFailed, InvalidInput, InvalidConfig };
  Kind kind = Kind::ExecutionFailed;
  std::string message;
  static SessionError execution(std::string m) { return {Kind::ExecutionFailed, std::move(m)}; }
  static SessionError input(std::string m) { return {Kind::InvalidInput, std::move(m)}; }
  static SessionError config(std::string m) { return {Kind::InvalidConfig, std::move(m)}; }
  std::string to_string() const;
};

// gpu_executor.rs:490-514 for this library's ops: RotaryEmbedding and
// GroupQueryAttention go to dispatch_rotary_embedding / dispatch_gqa; any
// other op_type is InternalError "GPU executor: no GPU implementation for
// {op}".
Result<std::vector<DeviceTensor>, OpError> dispatch_gpu_node(
    RocmRuntime& runtime, const std::string& op_type,
    const std::vector<const DeviceTensor*>& inputs, const std::vector<AttributeProto>& attrs,
    KvCacheDispatchCtx* kv_cache_ctx);

// gpu_executor.rs:290-433. `inputs` seed the value map by name; `nodes` run in
// the given (topological) order, each node's outputs stored under their names
// (empty names skipped); with a cache, GQA nodes take layers 0, 1, ... and
// one advance_position commits the pass when any did. Returns the
// `output_names` tensors in order. Errors: ExecutionFailed "{node}: {OpError}",
// "kv_cache advance_position: ...", "GPU executor: output tensor '{name}' not
// produced".
Result<std::vector<DeviceTensor>, SessionError> execute_graph_gpu_with_cache(
    RocmRuntime& runtime, const std::vector<ExecutionNode>& nodes,
    std::vector<std::pair<std::string, DeviceTensor>> inputs,
    const std::vector<std::string>& output_names, GpuKvCache* kv_cache);

// session.rs:579-593: the last layer and every pattern-th layer (counting
// from 1) are global, the others sliding windows of max(1, sliding_window).
std::vector<LayerKind> layer_kinds_for_gemma(size_t num_hidden_layers, size_t sliding_window,
                                             size_t sliding_window_pattern);

// The cache geometry a session allocates (session.rs:1221-1233: one layer per
// hidden layer, the model's kv heads and head_dim, max_seq_len capped by the
// caller). sliding_window 0 makes every layer global.
struct SessionConfig {
  size_t num_hidden_layers = 0;
  size_t num_key_value_heads = 0;
  size_t head_dim = 0;
  size_t max_seq_len = 0;
  size_t max_batch = 1;
  KvQuant quant = KvQuant::Int8;
  size_t sliding_window = 0;
  size_t sliding_window_pattern = 6;
};

// A session over one device: the graph of attention nodes, the paged cache
// behind a mutex (the reference's Arc<Mutex<GpuKvCache>>), run() once per
// forward pass. Not movable (the cache keeps a pointer to the runtime).
class GpuSession {
 public:
  static Result<std::unique_ptr<GpuSession>, SessionError> create(
      int device, const SessionConfig& config, std::vector<ExecutionNode> graph,
      std::vector<std::string> output_names);
  GpuSession(const GpuSession&) = delete;
  GpuSession& operator=(const GpuSession&) = delete;

  // session.rs:969-1033: lock the cache, run the graph with it, return the
  // declared outputs. Synchronises the device before returning.
  Result<std::vector<DeviceTensor>, SessionError> run(
      std::vector<std::pair<std::string, DeviceTensor>> inputs);
  // session.rs:1041-1049: the next run() starts at position 0.
  Result<Unit, SessionError> reset_kv_cache();
  // Committed tokens of every sequence.
  size_t position() const;
  const std::vector<LayerKind>& layer_kinds() const { return kinds_; }
  RocmRuntime& runtime() { return rt_; }

 private:
  explicit GpuSession(RocmRuntime rt) : rt_(std::move(rt)) {}
  RocmRuntime rt_;
  std::vector<LayerKind> kinds_;
  std::unique_ptr<GpuKvCache> cache_;
  mutable std::mutex mu_;
  std::vector<ExecutionNode> graph_;
  std::vector<std::string> output_names_;
};

}  // namespace sai::rocm

#endif  // SAI_GQA_SESSION_HPP
