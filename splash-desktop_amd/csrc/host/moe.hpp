// ops::MoE over HIP: the routed and shared experts' grouped gather-GEMM (reference: runtime/ops/MoE.hpp:19-423 and
// runtime/ops/MoE.cpp:27-543). A step starts from fp32 router scores in the grouped-input scratch: the block's router
// rows projected by the routing itself (MoeWeights::router), or the caller's.
#pragma once
#include "ops.hpp"

namespace sq::ops {

// MoeRouter (MoE.hpp:22-28).
enum class MoeRouter : uint32_t { Softmax = SQ_MOE_ROUTER_SOFTMAX, SigmoidNormalized = SQ_MOE_ROUTER_SIGMOID_NORMALIZED };

// MoeShape (MoE.hpp:54-102). The shared expert is sharedSlices experts (ids experts on) every row visits after its
// routed ones, each of the routed experts' intermediate width; with sharedGate each slice's weight is the sigmoid
// of the row's product with the block's fp32 scalar gate, else 1. The routings kernels run are the reference's
// compiled ones (kCompiledMoeRoutings, MoE.hpp:34-46) and, here, routed experts alone (Softmax, no slices).
struct MoeShape {
  uint32_t hiddenSize = 0, experts = 0, expertsPerToken = 0, expertIntermediateSize = 0;
  uint32_t expertFormat = SQ_FMT_AF4G64;
  MoeRouter router = MoeRouter::Softmax;
  uint32_t sharedSlices = 0;
  bool sharedGate = false;
  [[nodiscard]] bool compiledRouting() const noexcept {
    return (router == MoeRouter::Softmax && sharedSlices == 1 && sharedGate) ||
           (router == MoeRouter::SigmoidNormalized && sharedSlices == 2 && !sharedGate) ||
           (router == MoeRouter::Softmax && sharedSlices == 0 && !sharedGate);
  }
  [[nodiscard]] bool valid() const noexcept {
    return hiddenSize && hiddenSize % 256 == 0 && experts && experts <= SQ_MOE_WIDE_EXPERT_SLOTS && expertsPerToken &&
           expertsPerToken <= experts && expertsPerToken <= 64 && expertIntermediateSize &&
           expertIntermediateSize % 64 == 0 && sq_format_supported(expertFormat) && compiledRouting();
  }
  [[nodiscard]] uint32_t routesPerToken() const noexcept { return expertsPerToken + sharedSlices; }
  // routerWidth (MoE.hpp:94-96): the fp32 scores of a row of the router's output.
  [[nodiscard]] uint32_t routerWidth() const noexcept {
    return experts > SQ_MOE_EXPERT_SLOTS ? SQ_MOE_WIDE_EXPERT_SLOTS : SQ_MOE_EXPERT_SLOTS;
  }
};

enum class MoePhase : uint8_t { Prefill, Decode };

// MoeExpertTile, MoeGgufTile (MoE.hpp:284,297) and MoeConfig (MoE.hpp:333-346); FloatTile is the float
// projection's (ops.hpp).
enum class MoeExpertTile : uint8_t { M8 = 8, M32 = 32 };
enum class MoeGgufTile : uint8_t { Staged, Register };
struct MoeConfig {
  MoeExpertTile expertTile = MoeExpertTile::M8;
  MoeGgufTile ggufTile = MoeGgufTile::Staged;
  FloatTile ggufRouterTile = FloatTile::Simdgroup;
  bool cpuBf16Experts = false;
};

// moeMaximumTiles (MoE.hpp:200-205): every routed expert may leave one partial tile and no tile is empty; each shared
// slice fills one tile per tileRows rows.
[[nodiscard]] constexpr uint32_t moeMaximumTiles(uint32_t rows, const MoeShape &shape, uint32_t tileRows) noexcept {
  const uint32_t routed = rows * shape.expertsPerToken;
  return std::min(routed / tileRows + shape.experts, routed) + shape.sharedSlices * ((rows + tileRows - 1) / tileRows);
}

struct MoeWorkspace {
  uint64_t selectedExperts = 0, routingWeights = 0, tileDescriptors = 0, tileCount = 0, groupedRoutes = 0,
           routeRows = 0, groupedInput = 0, expertIntermediate = 0, expertOutput = 0;
};
struct MoeScratch {
  Buffer selectedExperts, routingWeights, tileDescriptors, tileCount, groupedRoutes, routeRows, groupedInput,
      expertIntermediate, expertOutput;
};
// BlockExpertProjection (MoE.hpp:111-148): the routed experts' planes, `slots` experts per projection, expert e's
// rows from slotTable[e] * N on; the shared slices' planes, slice s's rows s * N on, in a format of their own (the
// shared down's slices are the column windows of a shared_slices * I wide down); the block's fp32 scalar gate.
struct MoeWeights {
  QuantizedSegment gate, up, down;
  Buffer slotTable;
  uint32_t slots = 0;
  QuantizedSegment sharedGate, sharedUp, sharedDown;
  Buffer sharedScalarGate;
  // The router (BlockMoeWeights::router, MoE.hpp:133): F32 or BF16 rows [experts][hidden]. With it the routing
  // projects the input onto it into the scores first (MoE::addRoutes, MoE.cpp:527-543); without it the scores are
  // the caller's.
  QuantizedSegment router;
};
// MoeBuffers (MoE.hpp:375-385). The router's fp32 scores live in scratch.groupedInput, rows of routerWidth() (the
// caller's when the block has no router rows). verifyRows: a verify step's live rows per lane of
// SQ_TARGET_VERIFY_ROWS rows; routed routes of the rows past them go to no tile and add nothing.
struct MoeBuffers {
  Buffer input, residual, output;
  MoeScratch scratch;
  Buffer verifyRows;
};

class MoePlan {
public:
  [[nodiscard]] MoeShape shape() const noexcept { return shape_; }
  [[nodiscard]] uint32_t rows() const noexcept { return rows_; }
  [[nodiscard]] MoePhase phase() const noexcept { return phase_; }
  [[nodiscard]] MoeConfig configuration() const noexcept { return config_; }
  [[nodiscard]] uint32_t tileRows() const noexcept { return uint32_t(config_.expertTile); }
  [[nodiscard]] uint32_t maximumTiles() const noexcept { return maximumTiles_; }
  [[nodiscard]] const MoeWorkspace &workspace() const noexcept { return workspace_; }
  // MoePlan::MoePlan (MoE.cpp:196-206): decode plans take 8-row tiles, and the register tile is refused.
  MoePlan(MoeShape shape, uint32_t rows, MoeConfig config, MoePhase phase);

private:
  MoeShape shape_;
  uint32_t rows_;
  MoeConfig config_;
  MoePhase phase_;
  uint32_t maximumTiles_;
  MoeWorkspace workspace_;
};

struct MoE {
  // The device's policy (ExecutionPlans::moeConfig, ExecutionPlans.cpp:56-65): Staged tiles; in prefill 8-row tiles
  // while a chunk's routes average at most one row per expert, else 32 (moeGgufPrefillTile, MoE.hpp:321-330); in
  // decode 8-row tiles.
  [[nodiscard]] static MoeConfig config(MoeShape shape, uint32_t rows, MoePhase phase);
  [[nodiscard]] static MoePlan prefillPlan(MoeShape shape, uint32_t rows, MoeConfig config);
  // Decode steps of `lanes` lanes of 8 rows (MoE.cpp:567-571) and, here, of any rows up to 32 on 8-row tiles.
  [[nodiscard]] static MoePlan decodePlan(MoeShape shape, uint32_t lanes, MoeConfig config);
  [[nodiscard]] static MoePlan decodeRows(MoeShape shape, uint32_t rows);
  static void add(hipStream_t graph, const MoeBuffers &buffers, const MoeWeights &weights, const MoePlan &plan);
  // rowsTable (MoE::add's fusion): the route select also writes the block's input rows in the tiles' read order
  // there, and addRouted with rowsReady reads them from the expert-output scratch instead of writing them itself.
  static void addRouting(hipStream_t graph, const MoeBuffers &buffers, const MoeWeights &weights, const MoePlan &plan,
                         Buffer rowsTable = {});
  static void addRouted(hipStream_t graph, const MoeBuffers &buffers, const MoeWeights &weights, const MoePlan &plan,
                        bool rowsReady = false);
  // MoE::addRoutes (MoE.hpp:403-411; MoE.cpp:527-543): the routing of `rows` rows of `input` with no plan and no
  // grouping. With router rows (F32 or BF16, [experts][hidden]) it projects the input onto them into `scores` (rows of
  // shape.routerWidth() fp32 slots) on `routerTile`; with a null router it reads the scores already there. Then each
  // row's top-k experts and shared slices, and their routing weights, into `selected` and `routingWeights`
  // (shape.routesPerToken() per row). `sharedScalarGate` (fp32 [hidden]) is read only for a gated shared expert.
  static void addRoutes(hipStream_t graph, Buffer input, const QuantizedSegment &router, Buffer sharedScalarGate,
                        Buffer scores, Buffer selected, Buffer routingWeights, uint32_t rows, MoeShape shape,
                        FloatTile routerTile, Buffer rowsTable = {});
  // MoE::addExpertLoad (MoE.hpp:411-420): up to `jobs` streamed experts' gate, up and down native rows from
  // `staging` repacked into their slots of `arena` (moe_expert_load); `slots`, `sources` and `grid` are device
  // buffers an earlier dispatch may write. Validates the projections and the buffers' sizes before the launch.
  static void addExpertLoad(hipStream_t graph, Buffer staging, Buffer arena, Buffer slots, Buffer sources,
                            const SqMoeExpertLoadParams &params, uint32_t jobs, Buffer grid);
  // MoE::expertLoadGroups (MoE.cpp:545-551): the workgroups that repack one job's largest projection.
  static uint32_t expertLoadGroups(const SqMoeExpertLoadParams &params) noexcept;
};

}  // namespace sq::ops
