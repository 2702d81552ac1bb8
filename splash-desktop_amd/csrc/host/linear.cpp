// ops::Linear over HIP: plan policy, validation and dispatch of the decode and prefill tiles.
// Reference: runtime/ops/Linear.cpp:19-258 and runtime/ops/LinearGguf.cpp:396-923.
#include <algorithm>
#include <cmath>

#include "../kernels/kernels.hpp"
#include "ops.hpp"

namespace sq::ops {

void requireBytes(const Buffer &buffer, uint64_t bytes, std::string_view what) {
  if (buffer.sizeBytes() < bytes)
    throw std::invalid_argument(std::string(what) + " buffer holds " + std::to_string(buffer.sizeBytes()) +
                                " bytes, needs " + std::to_string(bytes));
}

namespace {

void requireLaunch(hipError_t e, std::string_view what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Linear.cpp:19-32, with decode workloads of any 1..32 rows: the decode tile runs genuine small-M steps, so a
// workload of one lane's eight rows (the reference's unit) is one case of it.
void validate(LinearWorkload w) {
  if (!w.matrix.outputSize || w.matrix.outputSize % 64 || !w.matrix.inputSize || w.matrix.inputSize % 64)
    throw std::invalid_argument("invalid linear matrix");
  if (w.phase == LinearPhase::Prefill) {
    if (!w.rows || w.rows > SQ_PREFILL_TOKEN_BUDGET || w.epilogue == LinearEpilogue::GateUp)
      throw std::invalid_argument("invalid linear prefill workload");
  } else {
    if (!w.rows || w.rows > SQ_MAXIMUM_DECODE_ROWS || w.epilogue == LinearEpilogue::UpWithGate)
      throw std::invalid_argument("invalid linear decode workload");
  }
}

LinearWorkload decodeWorkload(LinearMatrix matrix, uint32_t lanes, LinearEpilogue epilogue) {
  if (!lanes || lanes > SQ_MAXIMUM_BATCH_WIDTH) throw std::invalid_argument("invalid linear decode batch width");
  return {matrix, lanes * SQ_TARGET_VERIFY_ROWS, LinearPhase::Decode, epilogue};
}

constexpr uint32_t kPrefillTileRows = 128;
// The decode tile holds at most four lanes of rows; prefill chunks of up to that many rows run it too.
constexpr uint32_t kMaximumStagedRows = SQ_MAXIMUM_DECODE_ROWS;

// Groups of 32 inputs per meta unit, whose multiples a K partition of the decode tile takes: Q4_K's eight (a
// super-block) when the formats are unknown.
uint32_t planScaleGroups(const Projection *p, const Projection *gate) {
  uint32_t unit = 1;
  bool any = false;
  for (const Projection *q : {p, gate})
    if (q)
      for (const QuantizedSegment &s : q->blocks().segments) unit = std::max(unit, s.format().meta_groups), any = true;
  return any ? unit : 8;
}

// The projection is the plan's matrix and each segment fills whole 64-column tiles of it (LinearGguf.cpp:324-332).
void requireSegments(const Projection &p, LinearMatrix matrix) {
  if (p.outputSize != matrix.outputSize || p.inputSize != matrix.inputSize)
    throw std::invalid_argument("block projection does not match plan");
  for (const QuantizedSegment &s : p.blocks().segments) {
    if (s.outputSize % SQ_TILE_COLUMNS) throw std::invalid_argument("block segments do not fill whole column tiles");
    requireSegmentPlanes(s, "projection");
  }
}

char epilogueOf(LinearEpilogue e) { return e == LinearEpilogue::Residual ? 1 : e == LinearEpilogue::UpWithGate ? 2 : 0; }

kern::Segment kernelSegment(const QuantizedSegment &s) {
  return {s.plane0.as<const uint8_t>(), s.meta.as<const uint8_t>(), s.outputSize / SQ_TILE_COLUMNS, s.columnOffset,
          s.plane1.as<const uint8_t>(), s.formatId};
}

}  // namespace

QuantizedSegment QuantizedSegment::planes(uint32_t formatId, uint32_t outputSize, uint32_t inputSize, Buffer plane0,
                                          Buffer plane1, Buffer meta) {
  if (formatId >= SQ_FMT_COUNT) throw std::invalid_argument("unknown GGUF segment format");
  if (!sq_format_supported(formatId))
    throw std::invalid_argument("format " + std::to_string(formatId) +
                                " is not one this build runs (Q4_K, Q5_K, Q6_K, Q8_0, af4g32, af4g64, af4g128, af8g64)");
  QuantizedSegment s;
  s.plane0 = plane0;
  s.plane1 = plane1;
  s.meta = meta;
  s.outputSize = outputSize;
  s.inputSize = inputSize;
  s.formatId = formatId;
  return s;
}

// QuantizedSegment::rows (Weights.hpp:88-99): F32 or BF16 rows, `outputSize` rows of `inputSize` values in plane0.
QuantizedSegment QuantizedSegment::rows(uint32_t formatId, uint32_t outputSize, uint32_t inputSize, Buffer values) {
  if (formatId != kFloat32 && formatId != SQ_FMT_BF16)
    throw std::invalid_argument("float rows are F32 or BF16 (other formats' native rows are not taken here)");
  QuantizedSegment s;
  s.plane0 = values;
  s.outputSize = outputSize;
  s.inputSize = inputSize;
  s.formatId = formatId;
  return s;
}

void requireTableScratch(const LinearScratch &scratch, LinearInput layout, uint32_t width, uint32_t rows) {
  if (layout == LinearInput::Table16)
    throw std::invalid_argument("the Table16 layout is the Apple9 register tile's, which this device does not run");
  if (layout != LinearInput::HalfRows) throw std::invalid_argument("a table producer takes a table layout");
  if (!rows || width % 64) throw std::invalid_argument("a prefill table takes whole 64-input spans");
  requireBytes(scratch.input, tableBytes(width, rows), "norm table scratch");
  requireBytes(scratch.sums, tableSumsBytes(rows), "norm table sums");
  if (reinterpret_cast<uintptr_t>(scratch.input.ptr) & 15u)
    throw std::invalid_argument("the prefill table is 16-byte aligned");
}

// Weights.hpp:134-143.
Projection::Projection(uint32_t output, uint32_t input, BlockWeights weights)
    : outputSize(output), inputSize(input), weights_(std::move(weights)) {
  if (weights_.segments.empty()) throw std::invalid_argument("block projection has no segments");
  uint32_t covered = 0;
  for (const QuantizedSegment &s : weights_.segments) {
    if (s.inputSize != input || s.columnOffset != covered || !s.outputSize || s.outputSize > output - covered)
      throw std::invalid_argument("block segments do not tile the projection");
    covered += s.outputSize;
  }
}

// Each plane must reach the unit of the segment's last row and last group (LinearGguf.cpp:905-923).
void requireSegmentPlanes(const QuantizedSegment &segment, std::string_view what, uint32_t planeInputs) {
  if (!sq_format_supported(segment.formatId))
    throw std::invalid_argument(std::string(what) + " takes planes of a format this build runs");
  const SqQuantFormat f = segment.format();
  if (!segment.outputSize || !segment.inputSize || segment.inputSize % f.block_elements ||
      segment.outputSize % SQ_TILE_ROWS)
    throw std::invalid_argument(std::string(what) + " planes take whole native blocks and plane tiles");
  const uint32_t groups = segment.inputSize / 32, units = groups / f.meta_groups;
  const uint32_t rowGroups = (planeInputs ? planeInputs : segment.inputSize) / 32, rowUnits = rowGroups / f.meta_groups;
  const auto planeBytes = [&](uint32_t blocks, uint32_t rowBlocks, uint32_t unitBytes) {
    return (sq_tile_index(segment.outputSize - 1, blocks - 1, rowBlocks) + 1) * unitBytes;
  };
  const std::string name(what);
  requireBytes(segment.plane0, planeBytes(groups, rowGroups, f.plane0_bytes), name + " plane0");
  requireBytes(segment.meta, planeBytes(units, rowUnits, f.meta_bytes), name + " meta");
  if (f.plane1_bytes) requireBytes(segment.plane1, planeBytes(groups, rowGroups, f.plane1_bytes), name + " plane1");
}

// ---------------------------------------------------------------- plans

LinearPlan::LinearPlan(LinearWorkload w, LinearConfig config, FloatOutput destination)
    : workload_(w), config_(config), destination_(destination) {
  validate(w);
  if (destination == FloatOutput::Float32 && (w.phase != LinearPhase::Decode || w.epilogue != LinearEpilogue::None))
    throw std::invalid_argument("an fp32 destination takes a plain decode projection");
  requireConfiguration();
}

// LinearGguf.cpp:396-423 for the tiles this build runs.
void LinearPlan::requireConfiguration() const {
  const uint32_t k = workload_.matrix.inputSize;
  const LinearConfig &c = config_;
  const bool decode = workload_.phase == LinearPhase::Decode;
  if (c.tile == LinearTile::GgufRegister)
    throw std::invalid_argument("the register tile is the reference's Apple9 tile; MI355X plans run the decode and prefill tiles");
  if (c.spread && c.tile != LinearTile::GgufStaged) throw std::invalid_argument("only the staged block tile spreads its walks");
  if (c.oneGateUpPass && (c.tile != LinearTile::GgufStaged || !decode || workload_.epilogue != LinearEpilogue::GateUp))
    throw std::invalid_argument("only a staged block gate/up decode runs gate and up in one pass");
  if (c.sixteenRows && (c.tile != LinearTile::GgufStaged || !decode || workload_.rows != SQ_TARGET_VERIFY_ROWS))
    throw std::invalid_argument("only a staged one-lane block decode runs the 16-row tile");
  if (c.tile == LinearTile::GgufPrefill) {
    if (decode || c.splits != 1) throw std::invalid_argument("invalid block prefill configuration");
    return;
  }
  if (!c.validSplits() || (k / 32) % c.splits) throw std::invalid_argument("staged block splits take whole 32-input groups");
  if (workload_.rows > kMaximumStagedRows)
    throw std::invalid_argument("the staged block tile runs prefill chunks of up to 32 rows");
}

uint32_t LinearPlan::storageRows() const noexcept {
  if (config_.tile == LinearTile::GgufPrefill)
    return (workload_.rows + kPrefillTileRows - 1) / kPrefillTileRows * kPrefillTileRows;
  return config_.sixteenRows ? 16 : workload_.rows;
}

// Decode tile: [split][row][column] fp32 partials and a counter per 64 destination columns (LinearGguf.cpp:432-453).
// Prefill tile: the activations in fp16 and one fp32 scale per row, which its prepare dispatch writes, and where the
// projection halves its tiles' K the fp32 sums of both halves (kern::prefill_split), or where its tiles may run past
// a round as stream pieces the pieces' fp32 sums and a counter a stream tile (kern::prefill_stream).
LinearScratchSize LinearPlan::scratchSize() const noexcept {
  const auto [n, k] = workload_.matrix;
  if (config_.tile == LinearTile::GgufPrefill) {
    const uint64_t rows = storageRows();
    const kern::PrefillScratch halves = kern::prefill_scratch_bytes(workload_.rows, n / SQ_TILE_COLUMNS, k);
    return {uint64_t{workload_.rows} * k * 2, rows * 4, halves.partials, halves.counters, 0};
  }
  // Counters: one per workgroup column of the decode tile, at most one per 16 destination columns.
  const uint64_t columns = config_.oneGateUpPass ? 2 * uint64_t{n} : n;
  return config_.splits > 1 ? LinearScratchSize{0, 0, uint64_t{config_.splits} * storageRows() * columns * 4,
                                                uint64_t{n / 16} * 4, 0}
                            : LinearScratchSize{};
}

LinearInput LinearPlan::input() const noexcept {
  return config_.tile == LinearTile::GgufPrefill ? LinearInput::HalfRows : LinearInput::Plain;
}

uint64_t LinearPlan::gateScratchBytes() const noexcept {
  const bool needed = workload_.epilogue == LinearEpilogue::UpWithGate ||
                      (workload_.epilogue == LinearEpilogue::GateUp && !config_.oneGateUpPass);
  return needed ? uint64_t{storageRows()} * workload_.matrix.outputSize * 2 : 0;
}

// MI355X's split law. Both decode tiles stream a 64-column tile's K slices through one workgroup; a split adds a
// reduction tail (partials stored, a counter, partials read back: device-scope round trips after the workgroup's
// last load) and spreads the tile over more compute units. Measured on MI355X, a workgroup streams its bytes fastest
// up to about kColumnBytes (column tile) or kRowBytes (row tile, whose MFMA and close work per byte grows with the
// rows) per dispatch, and a grid larger than the device queues workgroups. The split is the fewest K partitions
// whose workgroups stream at most that many bytes, without growing the grid past the compute units, among those
// whose slices fit one workgroup of the tile the rows run (a partition takes whole meta units). It depends on the
// shape and the tile kind, never on the rows themselves, so a row's result is the same in any batch of its kind.
namespace {
constexpr double kColumnBytes = 160e3, kRowBytes = 80e3;
// The row tile's 16-column workgroups (one MFMA column block a wave: a quarter of the MFMAs and operands, the same
// activation loads and input sums) pay while four a tile times the splits fit one a compute unit: K 4096 x N 1024
// at M = 8 / 16 8.6 / 9.5 -> 7.8 / 9.1 us; allowed two a unit, N 4096 went 8.8 / 9.7 -> 11.0 / 13.5 us.
constexpr uint64_t kRowSliceUnits = 1;
// A tile whose split (above) would leave the row tile in 64-column workgroups runs unsplit in 16-column ones while
// four a tile fit one a compute unit and each streams at most kRowNarrowBytes: K 4096 x N 4096 (36.9 KB each) at
// M = 8 / 16 8.4 / 8.8 -> 7.1 / 8.4 us (two splits before); K 14336 x N 4096 (129 KB each) lost, 12.6 -> 18.8 us
// at M = 8, and so did a tile already in 16-column workgroups made unsplit (N 1024 at M = 16, 7.5 -> 7.9 us).
constexpr double kRowNarrowBytes = 40e3;
// A row tile already split whose split, doubled, would still fit 16-column workgroups on the compute units takes
// the doubled split while each K partition still streams at least kRowFillBytes: the few tiles then spread over
// the whole device, and the split tail, paid once, costs little more. Measured (graph-replayed, one box, M = 8 /
// 16 / 32): K 4096 x N 1024 6.81 / 7.44 / 9.32 -> 6.70 / 6.99 / 8.10 us (four splits, not two), N 512 6.58 / 7.24
// / 9.13 -> 6.24 / 6.60 / 7.71; an unsplit tile stays unsplit (K 2048 x N 1024 at two splits: 4.6 -> 5.7 us at
// M = 8), and a split whose 64-column workgroups already fill a quarter of the device stays (K 4096 x N 2048 at
// four splits: 6.88 -> 7.68 us at M = 8).
constexpr double kRowFillBytes = 32e3;
// A split of more than two that leaves the row tile in 64-column workgroups gives way to the largest smaller split
// (of at least two) whose 16-column workgroups fit the compute units, while each of those streams at most
// kRowNarrowSplitBytes. Measured (M = 8 / 16 / 32): K 5120 x N 2048 af4g64 8.32 / 8.52 / 11.98 -> 7.48 / 8.31 /
// 11.41 us, Q4_K 8.99 / 9.16 / 12.70 -> 7.55 / 8.30 / 11.50 (two splits, 23 and 21 KB a workgroup, not four);
// K 8192 x N 2048 (37 KB a workgroup in two splits) stays at four: 8.50 / 8.98 / 11.50 against 9.03 / 10.33 /
// 14.30.
constexpr double kRowNarrowSplitBytes = 30e3;
}  // namespace

uint32_t Linear::decodeSplits(uint32_t n, uint32_t k, uint32_t rows, uint32_t groupUnit, bool pair) const noexcept {
  const uint32_t G = k / 32, blocks = n / 16, tiles = n / 64;
  const uint32_t format = groupUnit == 8 ? SQ_FMT_Q4K : groupUnit == 4 ? SQ_FMT_AF4G128
                        : groupUnit == 2 ? SQ_FMT_AF4G64 : SQ_FMT_AF4G32;
  // The split law sees the tile kind only: one row stands for the column tile, sixteen or thirty-two for the row
  // tile's register budgets.
  const bool column = rows <= kern::kColumnTileRows;
  const uint32_t kind = column ? 1 : rows <= 16 ? 16 : SQ_MAXIMUM_DECODE_ROWS;
  const double tileBytes = (pair ? 2.0 : 1.0) * 64 * (k * 0.5 + G * 4.0 / groupUnit);
  const double budget = column ? kColumnBytes : kRowBytes;
  // A column-tile pair whose tiles already outnumber the compute units takes the byte budget's split past them: its
  // registers leave one workgroup a unit, so unsplit the tiles past a round trail in a short second one. Measured
  // (graph-replayed, 17408 x 5120 at 1 / 2 / 4 rows, one pass unsplit against four splits): Q4_K 26.9 / 29.3 / 29.9
  // -> 22.4 / 25.6 / 26.1 us, Q5_K 44.8 / 47.5 / 48.0 -> 36.3 / 39.5 / 40.2, Q6_K 46.7 / 49.5 / 50.5 -> 38.2 / 41.9
  // / 42.9, Q8_0 54.2 / 56.3 / 57.3 -> 44.0 / 47.8 / 49.1, af4g64 25.5 / 27.2 / 28.4 -> 24.7 / 28.0 / 28.5; at
  // 14336 x 4096 (224 tiles) the unsplit pair stays the faster in every format.
  const bool pastUnits = column && pair && tiles > computeUnits_;
  uint32_t best = 0;
  for (uint32_t s = 1; s <= LinearConfig::kMaximumSplits && G % (s * groupUnit) == 0; s *= 2) {
    if (!kern::decode_layout(format, blocks, k, s, pair, kind).nb) continue;
    if (best && uint64_t{tiles} * s > computeUnits_ && !pastUnits) break;
    best = s;
    if (tileBytes / s <= budget) break;
  }
  const uint64_t narrowUnits = kRowSliceUnits * computeUnits_;
  // The unsplit 16-column rule holds for the tile of up to 16 rows; with 32 rows the split measured faster (K 4096
  // x N 4096 at M = 32: 12.48 us unsplit, 10.88 in two splits).
  if (!column && kind <= 16 && best > 1 && uint64_t{tiles} * best * 4 > narrowUnits &&
      uint64_t{tiles} * 4 <= narrowUnits && tileBytes / 4 <= kRowNarrowBytes &&
      kern::decode_layout(format, blocks, k, 1, pair, kind).nb)
    return 1;
  if (!column && best > 2 && uint64_t{tiles} * best * 4 > narrowUnits)
    for (uint32_t s = best / 2; s >= 2; s /= 2)
      if (uint64_t{tiles} * s * 4 <= narrowUnits) {
        if (tileBytes / (4.0 * s) <= kRowNarrowSplitBytes && kern::decode_layout(format, blocks, k, s, pair, kind).nb)
          best = s;
        break;
      }
  while (!column && best > 1 && best * 2 <= LinearConfig::kMaximumSplits && G % (best * 2 * groupUnit) == 0 &&
         uint64_t{tiles} * best * 2 * 4 <= narrowUnits && tileBytes / (best * 2) >= kRowFillBytes &&
         kern::decode_layout(format, blocks, k, best * 2, pair, kind).nb)
    best *= 2;
  return best ? best : 1;
}

LinearConfig Linear::baseline(LinearWorkload w, const Projection *p, const Projection *gate) const {
  if (w.phase == LinearPhase::Prefill && w.rows > kMaximumStagedRows) return {.tile = LinearTile::GgufPrefill};
  // A gate/up pair of single tensors of one format runs in one dispatch: both walks share the activations' loads.
  const bool pair = w.phase == LinearPhase::Decode && w.epilogue == LinearEpilogue::GateUp && p && gate &&
                    p->blocks().segments.size() == 1 && gate->blocks().segments.size() == 1 &&
                    p->blocks().segments.front().formatId == gate->blocks().segments.front().formatId;
  return decodeConfig(w, planScaleGroups(p, gate), pair);
}

LinearConfig Linear::decodeConfig(LinearWorkload w, uint32_t unit, bool pair) const noexcept {
  const auto [n, k] = w.matrix;
  LinearConfig c{.tile = LinearTile::GgufStaged, .splits = decodeSplits(n, k, w.rows, unit, pair)};
  c.oneGateUpPass = pair;
  // On the row tile a pair whose one pass would take K splits runs as two passes, each under the single tensor's
  // split law (the split tail and the pair's shorter slices cost more than the second pass's activation loads).
  // Measured (af4g64, graph-replayed): 17408 x 5120 at 5 / 8 / 16 / 32 rows 46.9 / 47.8 / 49.0 / 113.6 us in one
  // pass (2, 2, 2, 4 splits) against 38.8 / 40.1 / 47.1 / 81.6 in two unsplit; 14336 x 4096 at 32 rows 40.1
  // against 31.0. Unsplit pairs keep the one pass (14336 x 4096 at 5 to 16 rows: 15.3-17.0 us against 18.2-21.5).
  if (pair && w.rows > kern::kColumnTileRows && c.splits > 1) {
    c.oneGateUpPass = false;
    c.splits = decodeSplits(n, k, w.rows, unit, false);
  }
  return c;
}

LinearPlan Linear::plan(LinearWorkload workload) const {
  validate(workload);
  return LinearPlan(workload, baseline(workload, nullptr, nullptr));
}
LinearPlan Linear::plan(LinearWorkload workload, LinearConfig config, FloatOutput destination) {
  return LinearPlan(workload, config, destination);
}
LinearPlan Linear::plan(LinearWorkload w, const Projection &p, const Projection *gate) const {
  validate(w);
  return LinearPlan(w, baseline(w, &p, gate), p.destination);
}
LinearPlan Linear::decodePlan(const Projection &p, uint32_t lanes, LinearEpilogue epilogue, const Projection *gate) const {
  return plan(decodeWorkload({p.outputSize, p.inputSize}, lanes, epilogue), p, gate);
}
LinearPlan Linear::prefillPlan(const Projection &p, uint32_t rows, LinearEpilogue epilogue) const {
  return plan({{p.outputSize, p.inputSize}, rows, LinearPhase::Prefill, epilogue}, p);
}
uint32_t Linear::decodeStorageRows(uint32_t rows, ProjectionShape shape) const {
  const LinearWorkload w{{shape.outputSize, shape.inputSize}, rows, LinearPhase::Decode, LinearEpilogue::None};
  validate(w);
  return LinearPlan(w, baseline(w, nullptr, nullptr)).storageRows();
}
// Every decode plan a projection of this shape can take: the split law sees the format's scale-group unit (a
// partition takes whole units: 1, 2, 4 or 8 groups of 32 inputs), and a gate/up plan may be a one-pass pair, whose
// partials hold both tensors' columns.
LinearScratchSize Linear::decodeScratchSize(ProjectionShape shape) const {
  LinearScratchSize bound;
  for (uint32_t rows = 1; rows <= SQ_MAXIMUM_DECODE_ROWS; ++rows)
    for (const auto e : {LinearEpilogue::None, LinearEpilogue::Residual, LinearEpilogue::GateUp})
      for (const uint32_t unit : {1u, 2u, 4u, 8u})
        for (const bool pair : {false, true}) {
          if (pair && e != LinearEpilogue::GateUp) continue;
          const LinearWorkload w{{shape.outputSize, shape.inputSize}, rows, LinearPhase::Decode, e};
          bound.include(LinearPlan(w, decodeConfig(w, unit, pair)).scratchSize());
        }
  return bound;
}
// MI355X's float-tile policy: the matrix-core tile from kern::kFloatMfmaRows rows on, the lane chains below (a
// decode step's handful of rows). Measured on the reference's 35B router (2048 rows x 256 experts x 2048 inputs):
// 76 us on the lane chains, 41 us on the matrix cores. The reference's rule (LinearGguf.cpp:837-844) weighs tiles
// per core of an Apple10 device; the row threshold here depends on neither the columns nor the format.
FloatTile Linear::floatTile(uint32_t rows, uint32_t outputSize, uint32_t formatId) const noexcept {
  (void)outputSize;
  (void)formatId;
  return rows >= kern::kFloatMfmaRows ? FloatTile::NeuralAccelerator : FloatTile::Simdgroup;
}

// Every chunk of 1..SQ_PREFILL_TOKEN_BUDGET rows: the prefill tile's halved-K partials (2 rows N fp32) exist only in
// a band of row counts (for 4096 inputs x 14336 outputs, 257..512 rows), so no short list of row counts bounds them.
// A plan's scratch does not depend on its epilogue; the three epilogues are taken all the same.
LinearScratchSize Linear::prefillScratchSize(ProjectionShape shape) const {
  LinearScratchSize bound;
  for (uint32_t rows = 1; rows <= SQ_PREFILL_TOKEN_BUDGET; ++rows)
    for (const auto e : {LinearEpilogue::None, LinearEpilogue::Residual, LinearEpilogue::UpWithGate})
      bound.include(plan({{shape.outputSize, shape.inputSize}, rows, LinearPhase::Prefill, e}).scratchSize());
  return bound;
}

// ---------------------------------------------------------------- dispatch

PreparedInput Linear::add(hipStream_t graph, LinearBuffers b, const Projection &p, const LinearPlan &selected,
                          const Projection *gate) const {
  const LinearWorkload w = selected.workload();
  const auto [n, k] = w.matrix;
  if ((w.epilogue == LinearEpilogue::GateUp) != (gate != nullptr))
    throw std::invalid_argument("a gate/up plan takes a gate projection and no other plan does");
  const uint64_t rows = selected.storageRows();
  requireBytes(b.input, rows * k * 2, "projection input");
  requireBytes(b.output, rows * n * elementBytes(selected.destination()), "projection output");
  if (w.epilogue == LinearEpilogue::Residual) requireBytes(b.residual, rows * n * 2, "projection residual");
  requireBytes(b.gateScratch, selected.gateScratchBytes(), "projection gate scratch");
  const LinearScratchSize scratch = selected.scratchSize();
  requireBytes(b.scratch.input, scratch.input, "projection scratch table");
  requireBytes(b.scratch.sums, scratch.sums, "projection scratch sums");
  requireBytes(b.scratch.partials, scratch.partials, "projection partials");
  requireBytes(b.scratch.counters, scratch.counters, "projection counters");
  requireSegments(p, w.matrix);
  if (gate) requireSegments(*gate, w.matrix);
  if (selected.configuration().tile == LinearTile::GgufPrefill) {
    // The prefill tile moves activations, outputs, epilogue operands, the table and a halved tile's fp32 partials in
    // 16-byte vectors (the row scales and a stream dispatch's counters in 4-byte words).
    const auto aligned = [](const Buffer &buffer) { return (reinterpret_cast<uintptr_t>(buffer.ptr) & 15u) == 0; };
    if (!aligned(b.input) || !aligned(b.output) || !aligned(b.residual) || !aligned(b.gateScratch) ||
        !aligned(b.scratch.input) || !aligned(b.scratch.partials) ||
        (reinterpret_cast<uintptr_t>(b.scratch.sums.ptr) & 3u) ||
        (reinterpret_cast<uintptr_t>(b.scratch.counters.ptr) & 3u))
      throw std::invalid_argument("prefill projection buffers are 16-byte aligned");
  }
  const std::vector<QuantizedSegment> &segments = p.blocks().segments;
  if (selected.destination() == FloatOutput::Float32 && segments.size() > 1)
    throw std::invalid_argument("an fp32 destination takes a single-tensor block projection");
  const LinearConfig config = selected.configuration();
  // Each tile states the formats it runs (the decode column tile to four rows, the row tile past it, the prefill
  // tile).
  const bool staged = config.tile == LinearTile::GgufStaged;
  const bool column = staged && w.rows <= kern::kColumnTileRows;
  for (const Projection *q : {&p, gate})
    if (q)
      for (const QuantizedSegment &s : q->blocks().segments)
        if (!(column ? kern::column_tile_format(s.formatId)
                     : staged ? kern::row_tile_format(s.formatId) : kern::prefill_tile_format(s.formatId)))
          throw std::invalid_argument(std::string(staged ? "the decode tile" : "the prefill tile") + " does not run " +
                                      s.name() + " weights");
  const uint32_t groupUnit = planScaleGroups(&p, gate);
  if (config.tile == LinearTile::GgufStaged) {
    if ((k / 32) % (config.splits * groupUnit))
      throw std::invalid_argument("a K partition of the staged tile takes whole scale groups of the projection's format");
    for (const QuantizedSegment &s : segments)
      if (!kern::decode_layout(s.formatId, n / 16, k, config.splits, config.oneGateUpPass, w.rows).nb)
        throw std::invalid_argument("the staged tile holds at most 256 groups of 32 inputs per K partition (64 for a "
                                    "one-pass gate/up): take more splits");
  }
  if (w.epilogue == LinearEpilogue::GateUp) {
    if (segments.size() != 1 || gate->blocks().segments.size() != 1)
      throw std::invalid_argument("block gate/up takes single tensors");
  }
  // Segments run one dispatch per format, at most three each (fused projections: q|k|v).
  std::vector<std::vector<const QuantizedSegment *>> byFormat;
  for (const QuantizedSegment &s : segments) {
    auto it = std::find_if(byFormat.begin(), byFormat.end(),
                           [&](const auto &g) { return g.front()->formatId == s.formatId; });
    if (it == byFormat.end()) byFormat.push_back({&s});
    else it->push_back(&s);
  }
  for (const auto &group : byFormat)
    if (group.size() > 3) throw std::invalid_argument("a block projection takes at most three segments per format");
  if (segments.size() > 1 && w.epilogue != LinearEpilogue::None)
    throw std::invalid_argument("a fused block projection takes at most three segments and no epilogue");

  if (config.tile == LinearTile::GgufPrefill) {
    // The table is prepared unless the scratch already holds this input's (a fused RMS norm, or a projection of the
    // same input before).
    if (!b.prepared.describes(b.input, LinearInput::HalfRows))
      requireLaunch(kern::launch_prefill_prepare(b.input.as<const uint16_t>(), w.rows, k,
                                                 b.scratch.input.as<uint16_t>(), b.scratch.sums.as<float>(), graph),
                    "prefill prepare");
    for (const auto &group : byFormat) {
      kern::PrefillArgs a{};
      a.half_input = b.scratch.input.as<const uint16_t>();
      a.row_scale = b.scratch.sums.as<const float>();
      a.segments = (uint32_t)group.size();
      for (size_t i = 0; i < group.size(); ++i) a.seg[i] = kernelSegment(*group[i]);
      a.output = b.output.as<uint16_t>();
      a.aux = w.epilogue == LinearEpilogue::Residual ? b.residual.as<const uint16_t>()
                                                     : b.gateScratch.as<const uint16_t>();
      a.K = k;
      a.rows = w.rows;
      a.out_stride = n;
      a.partials = b.scratch.partials.as<float>();
      a.counters = b.scratch.counters.as<uint32_t>();
      requireLaunch(kern::launch_prefill(group.front()->formatId, epilogueOf(w.epilogue), a, graph), "prefill tile");
    }
    return {b.input, LinearInput::HalfRows};
  }
  // The decode tiles' 64-column workgroups (a tile's K slices in one workgroup) leave most compute units idle when
  // a dispatch has few tiles times splits; while four times as many still fit one a compute unit it takes 16-column
  // workgroups, four for each, which compute the same bits (measured on MI355X, column tile, K 4096: N 4096 at M = 1
  // 5.8 -> 4.5 us, N 1024 5.5 -> 3.9 us; N 14336, 224 tiles, was slower: 7.8 -> 9.1 us).
  const auto columnSlices = [&](uint32_t tiles) -> uint32_t {
    const uint64_t units = w.rows <= kern::kColumnTileRows ? computeUnits_ : kRowSliceUnits * computeUnits_;
    return uint64_t{tiles} * config.splits * 4 <= units ? 4 : 1;
  };
  const auto decode = [&](const std::vector<const QuantizedSegment *> &group, uint32_t epilogue, Buffer output,
                          Buffer aux, bool f32) {
    kern::DecodeArgs a{};
    a.input = b.input.as<const uint16_t>();
    a.segments = (uint32_t)group.size();
    for (size_t i = 0; i < group.size(); ++i) a.seg[i] = kernelSegment(*group[i]);
    a.output = output.ptr;
    a.aux = aux.as<const uint16_t>();
    a.partials = b.scratch.partials.as<float>();
    a.counters = b.scratch.counters.as<uint32_t>();
    a.K = k;
    a.rows = w.rows;
    a.splits = config.splits;
    a.out_stride = n;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < a.segments; ++i) tiles += a.seg[i].tiles;
    a.column_slices = columnSlices(tiles);
    // Segments of different formats run in one dispatch, each workgroup in its own segment's format.
    uint32_t fmt = group.front()->formatId;
    for (const QuantizedSegment *s : group)
      if (s->formatId != fmt) fmt = kern::kSegmentFormats;
    requireLaunch(kern::launch_decode(fmt, epilogue, f32, a, graph), "decode tile");
  };
  if (w.epilogue == LinearEpilogue::GateUp && config.oneGateUpPass) {
    const QuantizedSegment &g = gate->blocks().segments.front(), &u = segments.front();
    if (g.formatId != u.formatId || g.columnOffset != u.columnOffset)
      throw std::invalid_argument("a one-pass block gate/up takes single tensors of one format");
    kern::DecodeArgs a{};
    a.input = b.input.as<const uint16_t>();
    a.seg[0] = kernelSegment(u);
    a.segments = 1;
    a.gate = kernelSegment(g);
    a.output = b.output.ptr;
    a.partials = b.scratch.partials.as<float>();
    a.counters = b.scratch.counters.as<uint32_t>();
    a.K = k;
    a.rows = w.rows;
    a.splits = config.splits;
    a.out_stride = n;
    a.column_slices = columnSlices(a.seg[0].tiles);
    requireLaunch(kern::launch_decode(u.formatId, kern::EpNone, false, a, graph), "gate/up decode tile");
    return b.prepared;
  }
  // The decode tiles read the plain rows and leave the scratch table as it was.
  if (w.epilogue == LinearEpilogue::GateUp) {
    // A gate pass into the gate scratch, then the up pass whose epilogue multiplies silu(gate) into bf16(up).
    decode({&gate->blocks().segments.front()}, kern::EpNone, b.gateScratch, {}, false);
    decode({&segments.front()}, kern::EpUpWithGate, b.output, b.gateScratch, false);
    return b.prepared;
  }
  const Buffer aux = w.epilogue == LinearEpilogue::Residual ? b.residual : b.gateScratch;
  if (segments.size() > 1 && segments.size() <= 3) {
    // A fused projection's segments in one dispatch whatever their formats (LinearGguf.cpp:655-667), those with the
    // most bytes per weight first so that their workgroups do not form the tail. Each tile computes what it does
    // alone: the split and slices take whole meta units of every segment's format.
    std::vector<const QuantizedSegment *> order;
    for (const QuantizedSegment &s : segments) order.push_back(&s);
    const auto bitsPerWeight = [](const QuantizedSegment *s) {
      const SqQuantFormat f = s->format();
      return (f.plane0_bytes + f.plane1_bytes) * 8.0 / 32.0 + f.meta_bytes * 8.0 / (32.0 * f.meta_groups);
    };
    std::stable_sort(order.begin(), order.end(),
                     [&](const QuantizedSegment *x, const QuantizedSegment *y) { return bitsPerWeight(x) > bitsPerWeight(y); });
    decode(order, kern::EpNone, b.output, {}, false);
    return b.prepared;
  }
  for (const auto &group : byFormat)
    decode(group, epilogueOf(w.epilogue), b.output, aux, selected.destination() == FloatOutput::Float32);
  return b.prepared;
}

void Linear::addPrefill(hipStream_t graph, Buffer input, const Projection &p, Buffer output, uint32_t rows,
                        LinearScratch scratch) const {
  add(graph, {.input = input, .output = output, .scratch = scratch}, p, prefillPlan(p, rows, LinearEpilogue::None));
}
void Linear::addPrefillResidual(hipStream_t graph, Buffer input, const Projection &p, Buffer residual, Buffer output,
                                uint32_t rows, LinearScratch scratch) const {
  add(graph, {.input = input, .output = output, .residual = residual, .scratch = scratch}, p,
      prefillPlan(p, rows, LinearEpilogue::Residual));
}
void Linear::addPrefillUpWithGate(hipStream_t graph, Buffer input, const Projection &up, Buffer gateScratch,
                                  Buffer output, uint32_t rows, LinearScratch scratch) const {
  add(graph, {.input = input, .output = output, .gateScratch = gateScratch, .scratch = scratch}, up,
      prefillPlan(up, rows, LinearEpilogue::UpWithGate));
}
// Linear.cpp:244-250.
void Linear::addPrefillSwiGlu(hipStream_t graph, const SwiGluProjections &ffn, const PrefillFfnBuffers &b,
                              Buffer residual, Buffer output, uint32_t rows) const {
  // Gate and up read the same rows: up takes the table gate's dispatch prepared.
  const PreparedInput normalized =
      add(graph, {.input = b.normalized, .output = b.gateScratch, .scratch = b.scratch}, *ffn.gate,
          prefillPlan(*ffn.gate, rows, LinearEpilogue::None));
  add(graph, {.input = b.normalized, .output = b.intermediate, .gateScratch = b.gateScratch, .scratch = b.scratch,
              .prepared = normalized},
      *ffn.up, prefillPlan(*ffn.up, rows, LinearEpilogue::UpWithGate));
  addPrefillResidual(graph, b.intermediate, *ffn.down, residual, output, rows, b.scratch);
}

}  // namespace sq::ops
