// Implementation of the session lifecycle mirror (gqa_session.hpp). Host code
// only, over the host mirror of gqa_host.hpp.
#include "gqa_session.hpp"

#include <algorithm>
#include <map>

namespace sai::rocm {

std::string SessionError::to_string() const {
  switch (kind) {
    case Kind::InvalidInput: return "invalid input: " + message;
    case Kind::InvalidConfig: return "invalid config: " + message;
    case Kind::ExecutionFailed: break;
  }
  return "execution failed: " + message;
}

Result<std::vector<DeviceTensor>, OpError> dispatch_gpu_node(
    RocmRuntime& runtime, const std::string& op_type,
    const std::vector<const DeviceTensor*>& inputs, const std::vector<AttributeProto>& attrs,
    KvCacheDispatchCtx* kv_cache_ctx) {
  if (op_type == "RotaryEmbedding")
    return dispatch_rotary_embedding(runtime, inputs, attrs, kv_cache_ctx);
  if (op_type == "GroupQueryAttention") return dispatch_gqa(runtime, inputs, attrs, kv_cache_ctx);
  return OpError::internal("GPU executor: no GPU implementation for " + op_type);
}

Result<std::vector<DeviceTensor>, SessionError> execute_graph_gpu_with_cache(
    RocmRuntime& runtime, const std::vector<ExecutionNode>& nodes,
    std::vector<std::pair<std::string, DeviceTensor>> inputs,
    const std::vector<std::string>& output_names, GpuKvCache* kv_cache) {
  // seed_inputs_into_value_map (gpu_executor.rs:325-335): the caller's
  // tensors move in
  std::map<std::string, DeviceTensor> value_map;
  for (auto& [name, t] : inputs) value_map[name] = std::move(t);
  KvCacheDispatchCtx ctx{kv_cache, 0};
  KvCacheDispatchCtx* ctx_ptr = kv_cache ? &ctx : nullptr;
  // run_one_node (gpu_executor.rs:381-419) over the nodes in order
  for (const ExecutionNode& node : nodes) {
    std::vector<const DeviceTensor*> in;
    in.reserve(node.inputs.size());
    for (const std::string& n : node.inputs) {
      auto it = n.empty() ? value_map.end() : value_map.find(n);
      in.push_back(it == value_map.end() ? nullptr : &it->second);
    }
    auto outs = dispatch_gpu_node(runtime, node.op_type, in, node.attributes, ctx_ptr);
    if (!outs) return SessionError::execution(node.name + ": " + outs.error().to_string());
    auto& produced = outs.value();
    for (size_t i = 0; i < produced.size() && i < node.outputs.size(); ++i) {
      if (node.outputs[i].empty()) continue;
      produced[i].name = node.outputs[i];
      value_map[node.outputs[i]] = std::move(produced[i]);
    }
  }
  // finalize_kv_cache (gpu_executor.rs:421-433): one advance per pass, when
  // an attention node used the cache
  if (ctx_ptr && ctx.next_layer_idx > 0) {
    auto adv = kv_cache->advance_position(nullptr);
    if (!adv)
      return SessionError::execution("kv_cache advance_position: " + adv.error().to_string());
  }
  // collect_graph_outputs (gpu_executor.rs:435-450)
  std::vector<DeviceTensor> results;
  for (const std::string& name : output_names) {
    auto it = value_map.find(name);
    if (it == value_map.end())
      return SessionError::execution("GPU executor: output tensor '" + name + "' not produced");
    results.push_back(std::move(it->second));
    value_map.erase(it);
  }
  return results;
}

std::vector<LayerKind> layer_kinds_for_gemma(size_t num_hidden_layers, size_t sliding_window,
                                             size_t sliding_window_pattern) {
  const size_t pattern = std::max<size_t>(1, sliding_window_pattern);
  std::vector<LayerKind> kinds;
  kinds.reserve(num_hidden_layers);
  for (size_t i = 0; i < num_hidden_layers; ++i) {
    const bool global = i + 1 == num_hidden_layers || (i + 1) % pattern == 0;
    kinds.push_back(global ? LayerKind::global()
                           : LayerKind::sliding_window(std::max<size_t>(1, sliding_window)));
  }
  return kinds;
}

Result<std::unique_ptr<GpuSession>, SessionError> GpuSession::create(
    int device, const SessionConfig& config, std::vector<ExecutionNode> graph,
    std::vector<std::string> output_names) {
  auto rt = RocmRuntime::init(device);
  if (!rt) return SessionError::execution("rocm runtime: " + rt.error().to_string());
  std::unique_ptr<GpuSession> s(new GpuSession(std::move(rt).value()));
  // a model without windowing has only global layers (gemma.rs:285-289)
  s->kinds_ = config.sliding_window == 0
                  ? std::vector<LayerKind>(config.num_hidden_layers, LayerKind::global())
                  : layer_kinds_for_gemma(config.num_hidden_layers, config.sliding_window,
                                          config.sliding_window_pattern);
  auto cache = GpuKvCache::allocate(s->rt_, config.num_hidden_layers, config.num_key_value_heads,
                                    config.head_dim, config.max_seq_len, config.quant, s->kinds_,
                                    config.max_batch);
  if (!cache) return SessionError::execution("kv_cache alloc: " + cache.error().to_string());
  s->cache_ = std::make_unique<GpuKvCache>(std::move(cache).value());
  s->graph_ = std::move(graph);
  s->output_names_ = std::move(output_names);
  return s;
}

Result<std::vector<DeviceTensor>, SessionError> GpuSession::run(
    std::vector<std::pair<std::string, DeviceTensor>> inputs) {
  std::lock_guard<std::mutex> lock(mu_);
  auto outs = execute_graph_gpu_with_cache(rt_, graph_, std::move(inputs), output_names_,
                                           cache_.get());
  if (!outs) return outs.error();
  auto sync = rt_.synchronize();
  if (!sync) return SessionError::execution("synchronize: " + sync.error().to_string());
  return outs;
}

Result<Unit, SessionError> GpuSession::reset_kv_cache() {
  std::lock_guard<std::mutex> lock(mu_);
  cache_->reset();
  return Unit{};
}

size_t GpuSession::position() const {
  std::lock_guard<std::mutex> lock(mu_);
  return cache_->current_position();
}

}  // namespace sai::rocm
