// splash_q4.hpp — header-only C++ face of the C ABI in splash_q4.h with the reference's splash::ops signatures
// (runtime/ops/Linear.hpp:247-300, runtime/ops/MoE.hpp:387-423): plans are values, add calls launch on a HIP
// stream (the reference's CommandGraph), and a failed validation throws std::invalid_argument with the reference's
// message before anything is launched (Linear.cpp:19-32,203-221; MoE.cpp:27-62). The library itself never lets an
// exception cross the C boundary; this header turns its status codes back into exceptions.
#ifndef SPLASH_Q4_HPP
#define SPLASH_Q4_HPP

#include <stdexcept>
#include <string>

#include "splash_q4.h"

namespace splash_q4::ops {

using Buffer = sq_buffer;
using Projection = sq_projection;
using LinearWorkload = sq_linear_workload;
using LinearConfig = sq_linear_config;
using LinearPlan = sq_linear_plan;
using LinearScratch = sq_linear_scratch;
using LinearScratchSize = sq_linear_scratch_size;
using LinearBuffers = sq_linear_buffers;
using MoeShape = sq_moe_shape;
using MoePlan = sq_moe_plan;
using MoeConfig = sq_moe_config;
using MoeWeights = sq_moe_weights;
using MoeBuffers = sq_moe_buffers;
using PreparedInput = sq_prepared_input;
using NormWeights = sq_norm_weights;
using QuantizedSegment = sq_segment;
using Graph = void *;   // a hipStream_t; nullptr is the default stream

enum class LinearEpilogue : uint32_t {
  None = SQ_EPILOGUE_NONE,
  Residual = SQ_EPILOGUE_RESIDUAL,
  GateUp = SQ_EPILOGUE_GATE_UP,
  UpWithGate = SQ_EPILOGUE_UP_WITH_GATE,
};

// Throws what the reference throws for a status the library returned.
inline void check(int status) {
  if (status == SQ_OK) return;
  const char *message = sq_last_error();
  if (status == SQ_INVALID_ARGUMENT) throw std::invalid_argument(message ? message : "invalid argument");
  throw std::runtime_error(message ? message : "splash_q4 runtime error");
}

// ProjectionShape (Weights.hpp:16-25): output and input sizes.
struct ProjectionShape {
  uint32_t outputSize, inputSize;
};

// The gate, up and down projections of one SwiGLU block and a prefill chunk's buffers for it (Linear.hpp:139-149).
struct SwiGluProjections {
  const Projection *gate = nullptr;
  const Projection *up = nullptr;
  const Projection *down = nullptr;
};
struct PrefillFfnBuffers {
  Buffer normalized, gateScratch, intermediate;
  LinearScratch scratch;
};

class Linear final {
 public:
  explicit Linear(sq_device device = {0}) noexcept : device_(device) {}

  [[nodiscard]] LinearPlan plan(LinearWorkload workload) const {
    LinearPlan out{};
    check(sq_linear_plan_for(&device_, &workload, nullptr, nullptr, &out));
    return out;
  }
  [[nodiscard]] LinearPlan plan(LinearWorkload workload, const Projection &projection,
                                const Projection *gate = nullptr) const {
    LinearPlan out{};
    check(sq_linear_plan_for(&device_, &workload, &projection, gate, &out));
    return out;
  }
  [[nodiscard]] static LinearPlan plan(LinearWorkload workload, LinearConfig config, uint32_t destination) {
    LinearPlan out{};
    check(sq_linear_plan_config(&workload, &config, destination, &out));
    return out;
  }
  [[nodiscard]] LinearPlan prefillPlan(const Projection &projection, uint32_t rows, LinearEpilogue epilogue) const {
    LinearPlan out{};
    check(sq_linear_prefill_plan(&device_, &projection, rows, static_cast<uint32_t>(epilogue), &out));
    return out;
  }
  [[nodiscard]] LinearPlan decodePlan(const Projection &projection, uint32_t lanes,
                                      LinearEpilogue epilogue = LinearEpilogue::None,
                                      const Projection *gate = nullptr) const {
    LinearPlan out{};
    check(sq_linear_decode_plan(&device_, &projection, lanes, static_cast<uint32_t>(epilogue), gate, &out));
    return out;
  }
  [[nodiscard]] LinearScratchSize decodeScratchSize(ProjectionShape shape) const {
    LinearScratchSize out{};
    check(sq_linear_decode_scratch_size(&device_, shape.outputSize, shape.inputSize, &out));
    return out;
  }
  [[nodiscard]] LinearScratchSize prefillScratchSize(ProjectionShape shape) const {
    LinearScratchSize out{};
    check(sq_linear_prefill_scratch_size(&device_, shape.outputSize, shape.inputSize, &out));
    return out;
  }
  // Linear::decodeStorageRows (Linear.hpp:254-257).
  [[nodiscard]] uint32_t decodeStorageRows(uint32_t rows, ProjectionShape shape) const {
    uint32_t out = 0;
    check(sq_linear_decode_storage_rows(&device_, rows, shape.outputSize, shape.inputSize, &out));
    return out;
  }
  // Linear::ggufFloatTile (Linear.hpp:273-276): an SQ_FLOAT_TILE_* value.
  [[nodiscard]] uint32_t ggufFloatTile(uint32_t rows, uint32_t outputSize, uint32_t formatId) const {
    uint32_t out = 0;
    check(sq_linear_float_tile(&device_, rows, outputSize, formatId, &out));
    return out;
  }
  // LinearPlan::scratchSize and gateScratchBytes of one plan.
  [[nodiscard]] static LinearScratchSize scratchSize(const LinearPlan &plan, uint64_t *gateScratchBytes = nullptr) {
    LinearScratchSize out{};
    uint64_t gate = 0;
    check(sq_linear_plan_scratch(&plan, &out, &gate));
    if (gateScratchBytes) *gateScratchBytes = gate;
    return out;
  }

  // Returns what the scratch table describes after the dispatch (Linear.cpp:222-231).
  PreparedInput add(Graph graph, LinearBuffers buffers, const Projection &projection, const LinearPlan &plan,
                    const Projection *gate = nullptr) const {
    PreparedInput out{};
    check(sq_linear_add_prepared(graph, &buffers, &projection, &plan, gate, &out));
    return out;
  }
  // LinearPlan::input (Linear.hpp:199-202).
  [[nodiscard]] static uint32_t input(const LinearPlan &plan) {
    uint32_t layout = 0;
    check(sq_linear_plan_input(&plan, &layout));
    return layout;
  }
  void addPrefill(Graph graph, Buffer input, const Projection &projection, Buffer output, uint32_t rows,
                  LinearScratch scratch = {}) const {
    check(sq_linear_add_prefill(&device_, graph, input, &projection, output, rows, &scratch));
  }
  void addPrefillUpWithGate(Graph graph, Buffer input, const Projection &up, Buffer gateScratch, Buffer output,
                            uint32_t rows, LinearScratch scratch) const {
    check(sq_linear_add_prefill_up_with_gate(&device_, graph, input, &up, gateScratch, output, rows, &scratch));
  }
  void addPrefillResidual(Graph graph, Buffer input, const Projection &projection, Buffer residual, Buffer output,
                          uint32_t rows, LinearScratch scratch) const {
    check(sq_linear_add_prefill_residual(&device_, graph, input, &projection, residual, output, rows, &scratch));
  }
  void addPrefillSwiGlu(Graph graph, const SwiGluProjections &ffn, const PrefillFfnBuffers &buffers, Buffer residual,
                        Buffer output, uint32_t rows) const {
    check(sq_linear_add_prefill_swiglu(&device_, graph, ffn.gate, ffn.up, ffn.down, buffers.normalized,
                                       buffers.gateScratch, buffers.intermediate, &buffers.scratch, residual, output,
                                       rows));
  }

 private:
  sq_device device_;
};

// Normalization (Normalization.hpp:29-40).
class Normalization final {
 public:
  static PreparedInput addRms(Graph graph, Buffer input, const NormWeights &weight, Buffer output, uint32_t width,
                              uint32_t rows, LinearScratch scratch = {}, uint32_t layout = SQ_LINEAR_INPUT_PLAIN) {
    PreparedInput out{};
    check(sq_norm_add_rms(graph, input, &weight, output, width, rows, &scratch, layout, &out));
    return out;
  }
};

// addGgufFloat (Linear.hpp:34-40) for F32 or BF16 rows, on `tile` (SQ_FLOAT_TILE_*).
inline void addGgufFloat(Graph graph, Buffer input, const QuantizedSegment &weights, Buffer output, uint32_t rows,
                         uint32_t outStride, uint32_t outOffset, uint32_t destination, uint32_t tile) {
  check(sq_float_add(graph, input, &weights, output, rows, outStride, outOffset, destination, tile));
}

// MoE (MoE.hpp:387-423). The config the reference's execution plans derive (ExecutionPlans::moeConfig) is
// MoE::config's here.
class MoE final {
 public:
  [[nodiscard]] static MoeConfig config(const MoeShape &shape, uint32_t rows, uint32_t phase) {
    MoeConfig out{};
    check(sq_moe_config_for(&shape, rows, phase, &out));
    return out;
  }
  [[nodiscard]] static MoePlan prefillPlan(const MoeShape &shape, uint32_t rows, const MoeConfig &config) {
    MoePlan out{};
    check(sq_moe_prefill_plan(&shape, rows, &config, &out));
    return out;
  }
  [[nodiscard]] static MoePlan decodePlan(const MoeShape &shape, uint32_t lanes, const MoeConfig &config) {
    MoePlan out{};
    check(sq_moe_decode_plan(&shape, lanes, &config, &out));
    return out;
  }
  void add(Graph graph, const MoeBuffers &buffers, const MoeWeights &weights, const MoePlan &plan) const {
    check(sq_moe_add(graph, &buffers, &weights, &plan));
  }
  void addRouting(Graph graph, const MoeBuffers &buffers, const MoeWeights &weights, const MoePlan &plan) const {
    check(sq_moe_add_routing(graph, &buffers, &weights, &plan));
  }
  void addRouted(Graph graph, const MoeBuffers &buffers, const MoeWeights &weights, const MoePlan &plan) const {
    check(sq_moe_add_routed(graph, &buffers, &weights, &plan));
  }
  // MoE::addRoutes (MoE.hpp:403-411): router may be null (the scores are the caller's).
  static void addRoutes(Graph graph, Buffer input, const QuantizedSegment *router, Buffer sharedScalarGate,
                        Buffer scores, Buffer selected, Buffer routingWeights, uint32_t rows, const MoeShape &shape,
                        uint32_t routerTile) {
    check(sq_moe_add_routes(graph, input, router, sharedScalarGate, scores, selected, routingWeights, rows, &shape,
                            routerTile));
  }
  // MoE::addExpertLoad (MoE.hpp:411-420) and MoE::expertLoadGroups (MoE.cpp:545-551).
  static void addExpertLoad(Graph graph, Buffer staging, Buffer arena, Buffer slots, Buffer sources,
                            const sq_moe_expert_load_params &params, uint32_t jobs, Buffer grid) {
    check(sq_moe_expert_load(graph, staging, arena, slots, sources, &params, jobs, grid));
  }
  [[nodiscard]] static uint32_t expertLoadGroups(const sq_moe_expert_load_params &params) {
    return sq_moe_expert_load_groups(&params);
  }
};

// Load-time weight preparation (gguf_repack.metal:232-238; GgufPreparation.cpp:141-193).
inline void repack(Graph graph, Buffer src, Buffer dst, const void *params) {
  check(sq_gguf_repack(graph, src, dst, params));
}
inline void mlxRepack(Graph graph, uint32_t formatId, uint32_t rows, uint32_t inputSize, Buffer weight,
                      Buffer scales, Buffer biases, Buffer plane0, Buffer meta) {
  check(sq_mlx_repack(graph, formatId, rows, inputSize, weight, scales, biases, plane0, meta));
}

}  // namespace splash_q4::ops

#endif
