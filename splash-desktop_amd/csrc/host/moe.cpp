// ops::MoE dispatch: routing (top-k select, grouping into expert tiles), then the routed work (gate/up pass with the
// gather folded in, down pass, combine). Reference: runtime/ops/MoE.cpp:27-84,116-192,445-543.
#include "moe.hpp"

#include "../kernels/kernels.hpp"

namespace sq::ops {
namespace {

void launched(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// MoE.cpp:64-84: the grouped rows' intermediates and outputs. The grouped input holds the router's fp32 scores, a
// row of routerWidth() per row, until the routed work overwrites them, as the reference's gather does, with the
// block's input rows in the expert tiles' read order (the gate/up pass gathers through the routes as it reads, so
// the rows are the block's, not the routes').
MoeWorkspace workspaceFor(const MoeShape &shape, uint32_t rows, uint32_t tileRows) {
  if (!shape.valid()) throw std::invalid_argument("invalid MoE workspace shape");
  const uint64_t routes = uint64_t{rows} * shape.routesPerToken();
  const uint32_t tiles = moeMaximumTiles(rows, shape, tileRows);
  const uint64_t groupedRows = uint64_t{tiles} * tileRows;
  const uint32_t widest = std::max(shape.hiddenSize, shape.expertIntermediateSize);
  const uint64_t scoreBytes = uint64_t{rows} * shape.routerWidth() * 4;
  const uint64_t inputBytes = uint64_t{rows} * shape.hiddenSize * 2;
  return {routes * 4, routes * 4, uint64_t{tiles} * sizeof(SqMoeTileDescriptor), sizeof(SqMoeTileCount),
          groupedRows * 4, routes * 4, std::max(scoreBytes, inputBytes),
          groupedRows * shape.expertIntermediateSize * 2, groupedRows * widest * 2};
}

// A routed or shared projection: `slots` experts (slices) of n rows of k inputs, each projection in a format of its
// own (MoE.cpp:27-62).
void requireExperts(const QuantizedSegment &s, uint32_t slots, uint32_t n, uint32_t k, const char *name) {
  if (s.outputSize != uint64_t{slots} * n || s.inputSize != k)
    throw std::invalid_argument(std::string("MoE expert ") + name + " does not match the plan");
  if (!kern::row_tile_format(s.formatId))
    throw std::invalid_argument(std::string("the MoE expert passes do not run ") + s.name() + " weights");
  requireSegmentPlanes(s, std::string("MoE expert ") + name);
}

void validate(const MoeBuffers &b, const MoeWeights &w, const MoePlan &plan) {
  const MoeShape s = plan.shape();
  const uint32_t h = s.hiddenSize, in = s.expertIntermediateSize;
  if (!w.slots) throw std::invalid_argument("MoE routed experts have no slots");
  requireBytes(w.slotTable, uint64_t{s.experts} * 4, "MoE slot table");
  requireExperts(w.gate, w.slots, in, h, "gate");
  requireExperts(w.up, w.slots, in, h, "up");
  requireExperts(w.down, w.slots, h, in, "down");
  if (s.sharedSlices) {
    // The shared slices (MoE.cpp:40-60).
    requireExperts(w.sharedGate, s.sharedSlices, in, h, "shared gate");
    requireExperts(w.sharedUp, s.sharedSlices, in, h, "shared up");
    requireExperts(w.sharedDown, s.sharedSlices, h, in, "shared down");
    if (s.sharedGate) requireBytes(w.sharedScalarGate, uint64_t{h} * 4, "MoE shared scalar gate weight");
  }
  if (w.router.plane0 && (!w.router.isFloat() || w.router.outputSize != s.experts || w.router.inputSize != h))
    throw std::invalid_argument("MoE router does not match the plan");
  const uint64_t hiddenRows = uint64_t{plan.rows()} * h * 2;
  requireBytes(b.input, hiddenRows, "MoE input");
  if (b.residual) requireBytes(b.residual, hiddenRows, "MoE residual");
  requireBytes(b.output, hiddenRows, "MoE output");
  const MoeWorkspace &need = plan.workspace();
  const MoeScratch &sc = b.scratch;
  requireBytes(sc.selectedExperts, need.selectedExperts, "MoE selected experts");
  requireBytes(sc.routingWeights, need.routingWeights, "MoE routing weights");
  requireBytes(sc.tileDescriptors, need.tileDescriptors, "MoE tile descriptors");
  requireBytes(sc.tileCount, need.tileCount, "MoE tile count");
  requireBytes(sc.groupedRoutes, need.groupedRoutes, "MoE grouped routes");
  requireBytes(sc.routeRows, need.routeRows, "MoE route rows");
  requireBytes(sc.groupedInput, need.groupedInput, "MoE grouped input");
  requireBytes(sc.expertIntermediate, need.expertIntermediate, "MoE expert intermediate");
  requireBytes(sc.expertOutput, need.expertOutput, "MoE expert output");
  // The combine and the input rows' reordering move eight bf16 a lane, the expert passes read 16-byte chunks of
  // their input rows.
  const auto aligned = [](const Buffer &buffer) { return (reinterpret_cast<uintptr_t>(buffer.ptr) & 15u) == 0; };
  if (!aligned(b.input) || !aligned(b.residual) || !aligned(b.output) || !aligned(sc.groupedInput) ||
      !aligned(sc.expertIntermediate) || !aligned(sc.expertOutput))
    throw std::invalid_argument(
        "MoE input, output, residual, grouped input, expert intermediate and expert output buffers are 16-byte aligned");
  if (b.verifyRows) {
    // A verify step's rows are its lanes' blocks (MoE.cpp:467-475).
    if (plan.phase() != MoePhase::Decode) throw std::invalid_argument("only a verify step's MoE routes its verify rows");
    const uint32_t lanes = (plan.rows() + SQ_TARGET_VERIFY_ROWS - 1) / SQ_TARGET_VERIFY_ROWS;
    requireBytes(b.verifyRows, uint64_t{lanes} * 4, "MoE verify rows");
  }
}

}  // namespace

MoePlan::MoePlan(MoeShape shape, uint32_t rows, MoeConfig config, MoePhase phase)
    : shape_(shape), rows_(rows), config_(config), phase_(phase) {
  if (!rows || rows > SQ_PREFILL_TOKEN_BUDGET || (phase == MoePhase::Decode && rows > SQ_MAXIMUM_DECODE_ROWS))
    throw std::invalid_argument("invalid MoE rows");
  if (config.expertTile != MoeExpertTile::M8 && config.expertTile != MoeExpertTile::M32)
    throw std::invalid_argument("invalid MoE expert tile configuration");
  if (phase == MoePhase::Decode && config.expertTile != MoeExpertTile::M8)
    throw std::invalid_argument("invalid MoE expert tile configuration");
  if (config.ggufTile == MoeGgufTile::Register)
    throw std::invalid_argument(
        "the register expert tile is the reference's Apple9 tile; MI355X plans run the staged expert tiles");
  if (config.ggufTile != MoeGgufTile::Staged) throw std::invalid_argument("invalid MoE GGUF tile");
  if (config.ggufRouterTile != FloatTile::Simdgroup && config.ggufRouterTile != FloatTile::NeuralAccelerator)
    throw std::invalid_argument("invalid MoE router tile");
  workspace_ = workspaceFor(shape, rows, tileRows());
  maximumTiles_ = moeMaximumTiles(rows, shape, tileRows());
}

MoeConfig MoE::config(MoeShape shape, uint32_t rows, MoePhase phase) {
  MoeConfig c;
  // ExecutionPlans.cpp:62: the router's tile by Linear's float-tile policy.
  c.ggufRouterTile = Linear(DeviceCapabilities{}).floatTile(rows, shape.experts, SQ_FLOAT32_ROWS);
  if (phase == MoePhase::Prefill)
    c.expertTile = uint64_t{rows} * shape.expertsPerToken <= shape.experts ? MoeExpertTile::M8 : MoeExpertTile::M32;
  return c;
}
MoePlan MoE::prefillPlan(MoeShape shape, uint32_t rows, MoeConfig config) {
  if (!rows || rows > SQ_PREFILL_TOKEN_BUDGET) throw std::invalid_argument("invalid MoE prefill rows");
  return MoePlan(shape, rows, config, MoePhase::Prefill);
}
MoePlan MoE::decodePlan(MoeShape shape, uint32_t lanes, MoeConfig config) {
  if (!lanes || lanes > SQ_MAXIMUM_BATCH_WIDTH) throw std::invalid_argument("invalid MoE decode batch width");
  return MoePlan(shape, lanes * SQ_TARGET_VERIFY_ROWS, config, MoePhase::Decode);
}
MoePlan MoE::decodeRows(MoeShape shape, uint32_t rows) {
  return MoePlan(shape, rows, config(shape, rows, MoePhase::Decode), MoePhase::Decode);
}

void MoE::add(hipStream_t graph, const MoeBuffers &b, const MoeWeights &w, const MoePlan &plan) {
  validate(b, w, plan);
  // Where gate and up share a format (routed, and shared if any), the gate/up pass is one gathering pass and the
  // expert-output scratch is free until the down pass writes it: the route select then writes the input rows in the
  // tiles' read order there, and the routed work skips its own input-rows dispatch. (Gate and up of different
  // formats park the gate's output in that scratch, so they keep the separate dispatch.)
  const MoeShape s = plan.shape();
  const bool onePass = w.gate.formatId == w.up.formatId &&
                       (!s.sharedSlices || w.sharedGate.formatId == w.sharedUp.formatId);
  if (onePass) {
    addRouting(graph, b, w, plan, b.scratch.expertOutput);
    addRouted(graph, b, w, plan, true);
    return;
  }
  addRouting(graph, b, w, plan);
  addRouted(graph, b, w, plan);
}

void MoE::addRoutes(hipStream_t graph, Buffer input, const QuantizedSegment &router, Buffer sharedScalarGate,
                    Buffer scores, Buffer selected, Buffer routingWeights, uint32_t rows, MoeShape s,
                    FloatTile routerTile, Buffer rowsTable) {
  if (!s.valid()) throw std::invalid_argument("invalid MoE routing shape");
  if (!rows || rows > SQ_PREFILL_TOKEN_BUDGET) throw std::invalid_argument("invalid MoE routing rows");
  if (router.plane0 && (!router.isFloat() || router.outputSize != s.experts || router.inputSize != s.hiddenSize))
    throw std::invalid_argument("MoE router does not match the plan");
  const uint32_t stride = s.routerWidth();
  const uint64_t routes = uint64_t{rows} * s.routesPerToken();
  requireBytes(input, uint64_t{rows} * s.hiddenSize * 2, "MoE input");
  requireBytes(scores, uint64_t{rows} * stride * 4, "MoE router scores");
  requireBytes(selected, routes * 4, "MoE selected experts");
  requireBytes(routingWeights, routes * 4, "MoE routing weights");
  if (s.sharedGate) requireBytes(sharedScalarGate, uint64_t{s.hiddenSize} * 4, "MoE shared scalar gate weight");
  // The select kernel reads the scores and the shared gate's input rows in 16-byte vectors.
  const auto aligned = [](const Buffer &buffer) { return (reinterpret_cast<uintptr_t>(buffer.ptr) & 15u) == 0; };
  if (!aligned(input) || !aligned(scores) || !aligned(sharedScalarGate) || !aligned(rowsTable))
    throw std::invalid_argument("MoE routing input, scores and shared scalar gate are 16-byte aligned");
  if (rowsTable) requireBytes(rowsTable, uint64_t{rows} * s.hiddenSize * 2, "MoE input rows table");
  // The router's fp32 scores, rows of routerWidth() (MoE.cpp:527-543), when the block carries its rows; else the
  // caller wrote them there.
  if (router.plane0) addGgufFloat(graph, input, router, scores, rows, stride, 0, FloatOutput::Float32, routerTile);
  const SqMoeRouteParams route{rows, s.hiddenSize, s.experts, s.expertsPerToken};
  launched(kern::launch_moe_route_select(scores.as<const float>(), stride, selected.as<uint32_t>(),
                                         routingWeights.as<float>(), route, input.as<const uint16_t>(),
                                         s.sharedGate ? sharedScalarGate.as<const float>() : nullptr,
                                         uint32_t(s.router), s.sharedSlices, rowsTable.as<uint16_t>(), graph),
           "MoE route select");
}

uint32_t MoE::expertLoadGroups(const SqMoeExpertLoadParams &params) noexcept {
  uint64_t groups = 0;
  for (const SqMoeExpertLoadProjection &q : params.projections)
    groups = std::max(groups, (uint64_t{q.rows} * (q.columns / 32) + SQ_MOE_EXPERT_LOAD_THREADS - 1) /
                                  SQ_MOE_EXPERT_LOAD_THREADS);
  return groups > UINT32_MAX ? 0u : static_cast<uint32_t>(groups);
}

void MoE::addExpertLoad(hipStream_t graph, Buffer staging, Buffer arena, Buffer slots, Buffer sources,
                        const SqMoeExpertLoadParams &params, uint32_t jobs, Buffer grid) {
  const char *names[3] = {"gate", "up", "down"};
  bool any = false;
  for (int z = 0; z < 3; ++z) {
    const SqMoeExpertLoadProjection &q = params.projections[z];
    if (!q.rows) continue;
    any = true;
    const std::string what = std::string("MoE expert load ") + names[z];
    if (!sq_format_supported(q.format)) throw std::invalid_argument(what + " takes a format this build runs");
    const SqQuantFormat f = sq_format(q.format);
    if (q.rows % SQ_TILE_ROWS || !q.columns || q.columns % f.block_elements)
      throw std::invalid_argument(what + " takes whole plane tiles of rows and whole native blocks");
    if (q.row_bytes < uint64_t{q.columns} / f.block_elements * f.block_bytes)
      throw std::invalid_argument(what + " rows are shorter than their blocks");
    const uint64_t groups = q.columns / 32;
    const uint64_t need[3] = {q.rows * groups * f.plane0_bytes, q.rows * groups * f.plane1_bytes,
                              q.rows * (groups / f.meta_groups) * f.meta_bytes};
    for (int i = 0; i < 3; ++i)
      if (q.slot_bytes[i] < need[i]) throw std::invalid_argument(what + " slots are smaller than their planes");
  }
  const uint32_t groups = expertLoadGroups(params);
  if (!jobs || !any) return;
  if (jobs > 65535 || !groups) throw std::invalid_argument("invalid MoE expert load grid");
  requireBytes(slots, uint64_t{jobs} * 4, "MoE expert load slots");
  requireBytes(sources, uint64_t{jobs} * 3 * 8, "MoE expert load sources");
  requireBytes(grid, 12, "MoE expert load grid");
  if (!staging || !arena) throw std::invalid_argument("MoE expert load needs its staging and arena buffers");
  if ((reinterpret_cast<uintptr_t>(sources.ptr) & 7u) || (reinterpret_cast<uintptr_t>(slots.ptr) & 3u) ||
      (reinterpret_cast<uintptr_t>(grid.ptr) & 3u))
    throw std::invalid_argument("MoE expert load sources are 8-byte and slots and grid 4-byte aligned");
  launched(kern::launch_expert_load(staging.as<const uint8_t>(), staging.bytes, arena.as<uint8_t>(), arena.bytes,
                                    slots.as<const uint32_t>(), sources.as<const uint64_t>(), params, groups, jobs,
                                    grid.as<const uint32_t>(), graph),
           "MoE expert load");
}

void MoE::addRouting(hipStream_t graph, const MoeBuffers &b, const MoeWeights &w, const MoePlan &plan,
                     Buffer rowsTable) {
  validate(b, w, plan);
  const MoeShape s = plan.shape();
  const MoeScratch &sc = b.scratch;
  // The scores live in the grouped input (MoE.cpp:445-459).
  addRoutes(graph, b.input, w.router, s.sharedGate ? w.sharedScalarGate : Buffer{}, sc.groupedInput,
            sc.selectedExperts, sc.routingWeights, plan.rows(), s, plan.configuration().ggufRouterTile, rowsTable);
  const SqMoeGroupParams group{plan.rows(), s.expertsPerToken, plan.tileRows(), s.experts,
                               s.expertIntermediateSize / SQ_TILE_COLUMNS, s.hiddenSize / SQ_TILE_COLUMNS,
                               SQ_TARGET_VERIFY_ROWS, 0};
  launched(kern::launch_moe_group(sc.selectedExperts.as<const uint32_t>(), sc.tileDescriptors.as<SqMoeTileDescriptor>(),
                                  sc.tileCount.as<SqMoeTileCount>(), sc.groupedRoutes.as<uint32_t>(),
                                  sc.routeRows.as<uint32_t>(), b.verifyRows.as<const uint32_t>(), group,
                                  s.sharedSlices, graph),
           "MoE grouping");
}

void MoE::addRouted(hipStream_t graph, const MoeBuffers &b, const MoeWeights &w, const MoePlan &plan,
                    bool rowsReady) {
  validate(b, w, plan);
  const MoeShape s = plan.shape();
  const MoeScratch &sc = b.scratch;
  kern::MoeExpertArgs a{};
  a.tiles = sc.tileDescriptors.as<const SqMoeTileDescriptor>();
  a.tile_count = sc.tileCount.as<const SqMoeTileCount>();
  a.slots = w.slotTable.as<const uint32_t>();
  a.tile_rows = plan.tileRows();
  a.max_tiles = plan.maximumTiles();
  a.routes = sc.groupedRoutes.as<const uint32_t>();
  a.routes_per_row = s.routesPerToken();
  a.experts = s.experts;
  // Plane views of tensor slot n: the routed projection's and the shared one's.
  const auto bind = [&](int n, const QuantizedSegment &routed, const QuantizedSegment &shared) {
    a.plane0[n] = routed.plane0.as<const uint8_t>();
    a.meta[n] = routed.meta.as<const uint8_t>();
    a.plane1[n] = routed.plane1.as<const uint8_t>();
    a.shared_plane0[n] = shared.plane0.as<const uint8_t>();
    a.shared_meta[n] = shared.meta.as<const uint8_t>();
    a.shared_plane1[n] = shared.plane1.as<const uint8_t>();
  };
  const QuantizedSegment none{};
  // The tiles of one format run in one launch: the routed and shared tiles together when their formats agree
  // (mode 2), else each on its own (modes 0 and 1). `formats(mode)` gives a launch's (first, second) formats.
  const auto launches = [&](auto &&formats, auto &&launch) {
    const auto [r0, r1] = formats(0);
    if (!s.sharedSlices) return launch(0, r0, r1);
    const auto [s0, s1] = formats(1);
    if (r0 == s0 && r1 == s1) return launch(2, r0, r1);
    launch(0, r0, r1);
    launch(1, s0, s1);
  };
  // Gate and up over the input rows of the routes: intermediate = bf16(bf16(up) silu(bf16(gate))), in one pass when
  // the two share a format, else the gate into the output scratch and up with the gate epilogue (MoE.cpp:154-173).
  const auto gateUpFormats = [&](uint32_t mode) {
    return mode == 0 ? std::pair{w.gate.formatId, w.up.formatId} : std::pair{w.sharedGate.formatId, w.sharedUp.formatId};
  };
  // The block's input rows in the tiles' read order, over the router's scores (MoE.cpp:480-517 opens the same way
  // with its gather).
  if (rowsReady) {
    a.input = sc.expertOutput.as<const uint16_t>();
  } else {
    launched(kern::launch_moe_input_rows(b.input.as<const uint16_t>(), plan.rows(), s.hiddenSize,
                                         sc.groupedInput.as<uint16_t>(), graph),
             "MoE input rows");
    a.input = sc.groupedInput.as<const uint16_t>();
  }
  a.K = s.hiddenSize;
  a.output_size = s.expertIntermediateSize;
  a.gather = 1;
  // A launch of the shared slices alone with few tiles (every tile full: the rows of a block of a few thousand rows)
  // runs each tile's rows as two 16-row halves, a workgroup each, so that it fills twice the SIMDs; each row
  // computes what it does in the whole tile (35B layer, Q8_0 shared gate/up over 2048 rows: 512 -> 1024 waves).
  const auto halves = [&](uint32_t mode, uint32_t outputSize) -> uint32_t {
    const uint64_t tiles = uint64_t{s.sharedSlices} * ((plan.rows() + plan.tileRows() - 1) / plan.tileRows());
    return mode == 1 && plan.tileRows() > 16 && tiles * (outputSize / 64) <= 2 * kern::kPrefillUnits ? 1 : 0;
  };
  launches(gateUpFormats, [&](uint32_t mode, uint32_t gateFormat, uint32_t upFormat) {
    a.mode = mode;
    a.row_halves = halves(mode, s.expertIntermediateSize);
    if (gateFormat == upFormat) {
      bind(0, w.gate, w.sharedGate);
      bind(1, w.up, w.sharedUp);
      a.fmt = gateFormat;
      a.gate_up = 1;
      a.gate = nullptr;
      a.output = sc.expertIntermediate.as<uint16_t>();
      launched(kern::launch_moe_expert(a, graph), "MoE gate/up pass");
      return;
    }
    a.gate_up = 0;
    bind(0, w.gate, w.sharedGate);
    bind(1, none, none);
    a.fmt = gateFormat;
    a.gate = nullptr;
    a.output = sc.expertOutput.as<uint16_t>();
    launched(kern::launch_moe_expert(a, graph), "MoE gate pass");
    bind(0, w.up, w.sharedUp);
    a.fmt = upFormat;
    a.gate = sc.expertOutput.as<const uint16_t>();
    a.output = sc.expertIntermediate.as<uint16_t>();
    launched(kern::launch_moe_expert(a, graph), "MoE up pass");
  });
  // Down over the grouped intermediate rows.
  a.input = sc.expertIntermediate.as<const uint16_t>();
  a.routes = nullptr;
  a.gather = 0;
  a.gate_up = 0;
  a.gate = nullptr;
  bind(0, w.down, w.sharedDown);
  bind(1, none, none);
  a.output = sc.expertOutput.as<uint16_t>();
  a.K = s.expertIntermediateSize;
  a.output_size = s.hiddenSize;
  const auto downFormats = [&](uint32_t mode) {
    return std::pair{mode == 0 ? w.down.formatId : w.sharedDown.formatId, 0u};
  };
  launches(downFormats, [&](uint32_t mode, uint32_t format, uint32_t) {
    a.mode = mode;
    a.row_halves = halves(mode, s.hiddenSize);
    a.fmt = format;
    launched(kern::launch_moe_expert(a, graph), "MoE down pass");
  });
  const SqMoeCombineParams combine{plan.rows(), s.hiddenSize, s.routesPerToken()};
  launched(kern::launch_moe_combine(sc.expertOutput.as<const uint16_t>(), sc.routeRows.as<const uint32_t>(),
                                    sc.routingWeights.as<const float>(), b.residual.as<const uint16_t>(),
                                    b.output.as<uint16_t>(), combine, graph),
           "MoE combine");
}

}  // namespace sq::ops
