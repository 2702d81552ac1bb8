// The operator layer of the quantized matmul path: the reference's splash::ops::Linear and splash::ops::MoE
// surface (runtime/ops/Linear.hpp:16-337, runtime/ops/Weights.hpp:16-188, runtime/ops/MoE.hpp:19-423) restated over
// HIP. A "graph" is a HIP stream: add() validates everything first and throws std::invalid_argument before anything
// is launched, then launches in order on the stream. Policy constants are MI355X's.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

#include "../abi.h"

namespace sq::ops {

// A device buffer view (the reference's MetalBuffer view): base pointer and the bytes the view spans.
struct Buffer {
  void *ptr = nullptr;
  uint64_t bytes = 0;
  [[nodiscard]] uint64_t sizeBytes() const noexcept { return ptr ? bytes : 0; }
  explicit operator bool() const noexcept { return ptr != nullptr; }
  template <class T> [[nodiscard]] T *as() const noexcept { return static_cast<T *>(ptr); }
};

// BufferExtent.hpp:243-255.
[[nodiscard]] constexpr uint64_t rowBytes(uint64_t rows, uint64_t stride, uint64_t width, uint64_t elementBytes) noexcept {
  return rows && width ? ((rows - 1) * stride + width) * elementBytes : 0;
}
void requireBytes(const Buffer &buffer, uint64_t bytes, std::string_view what);

enum class FloatOutput : uint8_t { BFloat16, Float32 };
// FloatTile (Linear.hpp:29-33): the tile of a float projection. On MI355X Simdgroup is the lane-chain kernel (a wave
// of four rows by four columns, K split over the lanes) and NeuralAccelerator the matrix-core tile (the fp32
// 16x16x4 MFMA, 32 rows by 32 columns a workgroup, K a multiple of 256); both round only in fp32 accumulation, within
// one bound (K / 64 + 8 roundings of sum |x w|). Linear::floatTile picks one.
enum class FloatTile : uint8_t { Simdgroup, NeuralAccelerator };
[[nodiscard]] constexpr uint64_t elementBytes(FloatOutput type) noexcept {
  return type == FloatOutput::Float32 ? 4 : 2;
}

// Weights.hpp:79-121. Planes: repacked planes in format formatId, which the block tiles read. Rows: the tensor's
// rows as stored, inputSize values per output column in plane0, F32 (formatId kFloat32) or BF16 (SQ_FMT_BF16),
// which the float projection multiplies unrounded in fp32 (the MoE router is one).
struct QuantizedSegment {
  static constexpr uint32_t kFloat32 = SQ_FLOAT32_ROWS;
  Buffer plane0, plane1, meta;
  uint32_t outputSize = 0, inputSize = 0, columnOffset = 0, formatId = SQ_FMT_COUNT;
  [[nodiscard]] static QuantizedSegment planes(uint32_t formatId, uint32_t outputSize, uint32_t inputSize,
                                               Buffer plane0, Buffer plane1, Buffer meta);
  [[nodiscard]] static QuantizedSegment rows(uint32_t formatId, uint32_t outputSize, uint32_t inputSize, Buffer values);
  [[nodiscard]] bool isFloat() const noexcept { return formatId == kFloat32 || formatId == SQ_FMT_BF16; }
  [[nodiscard]] SqQuantFormat format() const noexcept { return sq_format(formatId); }
  [[nodiscard]] const char *name() const noexcept { return sq_format_name(formatId); }
};
struct BlockWeights {
  std::vector<QuantizedSegment> segments;
};

struct ProjectionShape {
  uint32_t outputSize = 0, inputSize = 0;
};

// Weights.hpp:131-188: segments tile the projection's leading output columns in order.
class Projection {
public:
  Projection() = default;
  Projection(uint32_t output, uint32_t input, BlockWeights weights);
  [[nodiscard]] const BlockWeights &blocks() const noexcept { return weights_; }
  [[nodiscard]] ProjectionShape shape() const noexcept { return {outputSize, inputSize}; }
  uint32_t outputSize = 0, inputSize = 0;
  FloatOutput destination = FloatOutput::BFloat16;

private:
  BlockWeights weights_;
};

// Throws unless the segment's planes hold every tile of its weights (LinearGguf.cpp:905-923).
void requireSegmentPlanes(const QuantizedSegment &segment, std::string_view what, uint32_t planeInputs = 0);

enum class LinearPhase : uint8_t { Prefill, Decode };
enum class LinearEpilogue : uint8_t { None, Residual, GateUp, UpWithGate };
// GgufStaged: the decode tile (decode, and prefill chunks of up to 32 rows), split over K. GgufPrefill: the prefill
// tile. GgufRegister names the reference's Apple9 register tile, which MI355X has no use for: plans never pick it
// and an explicit plan of it is refused.
enum class LinearTile : uint8_t { GgufStaged, GgufPrefill, GgufRegister };

struct LinearMatrix {
  uint32_t outputSize = 0, inputSize = 0;
};
struct LinearWorkload {
  LinearMatrix matrix;
  uint32_t rows = 0;
  LinearPhase phase = LinearPhase::Decode;
  LinearEpilogue epilogue = LinearEpilogue::None;
};
struct LinearConfig {
  LinearTile tile = LinearTile::GgufStaged;
  uint32_t splits = 1;
  static constexpr uint32_t kMaximumSplits = SQ_MAXIMUM_SPLITS;
  bool spread = false;
  bool oneGateUpPass = false;
  bool sixteenRows = false;
  [[nodiscard]] constexpr bool validSplits() const noexcept {
    return splits && splits <= kMaximumSplits && !(splits & (splits - 1));
  }
};

struct LinearScratch {
  Buffer input, sums, partials, counters, rotated;
};
struct LinearScratchSize {
  uint64_t input = 0, sums = 0, partials = 0, counters = 0, rotated = 0;
  [[nodiscard]] uint64_t bytes() const noexcept { return input + sums + partials + counters + rotated; }
  LinearScratchSize &include(const LinearScratchSize &o) noexcept {
    input = std::max(input, o.input);
    sums = std::max(sums, o.sums);
    partials = std::max(partials, o.partials);
    counters = std::max(counters, o.counters);
    rotated = std::max(rotated, o.rotated);
    return *this;
  }
};
struct SwiGluProjections {
  const Projection *gate = nullptr, *up = nullptr, *down = nullptr;
};
struct PrefillFfnBuffers {
  Buffer normalized, gateScratch, intermediate;
  LinearScratch scratch;
};

// LinearInput (Linear.hpp:166-169): the activation layout a plan reads. Table16 is the reference's Apple9 register
// tile table, which no MI355X plan reads; HalfRows is the prefill tile's prepared input (the rows in fp16 scaled by
// a power of two per row, in the tile's group order, in scratch.input, and the powers in scratch.sums), which the
// prefill's own prepare dispatch or a fused RMS norm writes.
enum class LinearInput : uint8_t { Plain = SQ_LINEAR_INPUT_PLAIN, Table16 = SQ_LINEAR_INPUT_TABLE16,
                                   HalfRows = SQ_LINEAR_INPUT_HALF_ROWS };
// PreparedInput (Linear.hpp:184-190): the scratch table currently holds `source` in `layout`. Producers return it,
// consumers accept it and return what the scratch describes after their dispatch.
struct PreparedInput {
  Buffer source;
  LinearInput layout = LinearInput::Plain;
  [[nodiscard]] bool describes(const Buffer &input, LinearInput want) const noexcept {
    return layout == want && source.ptr == input.ptr && source.bytes == input.bytes;
  }
};
// The table bytes a producer writes for `rows` rows of `width` inputs (Linear.hpp:172-174), and its row scales.
[[nodiscard]] constexpr uint64_t tableBytes(uint32_t width, uint64_t rows) noexcept { return uint64_t{width} * rows * 2; }
[[nodiscard]] constexpr uint64_t tableSumsBytes(uint64_t rows) noexcept { return rows * 4; }
// Throws unless `scratch` holds the `layout` table of `rows` rows of `width` inputs (Linear.hpp:175-179).
void requireTableScratch(const LinearScratch &scratch, LinearInput layout, uint32_t width, uint32_t rows);

class LinearPlan {
public:
  [[nodiscard]] LinearWorkload workload() const noexcept { return workload_; }
  [[nodiscard]] LinearConfig configuration() const noexcept { return config_; }
  [[nodiscard]] FloatOutput destination() const noexcept { return destination_; }
  [[nodiscard]] uint32_t storageRows() const noexcept;
  [[nodiscard]] LinearScratchSize scratchSize() const noexcept;
  [[nodiscard]] uint64_t gateScratchBytes() const noexcept;
  // The layout the producer of this plan's input may write: HalfRows for the prefill tile, Plain otherwise.
  [[nodiscard]] LinearInput input() const noexcept;
  LinearPlan(LinearWorkload workload, LinearConfig config, FloatOutput destination = FloatOutput::BFloat16);

private:
  void requireConfiguration() const;
  LinearWorkload workload_;
  LinearConfig config_;
  FloatOutput destination_;
};

struct LinearBuffers {
  Buffer input, output, residual, gateScratch;
  LinearScratch scratch{};
  // What the scratch table holds (after a fused RMS norm, say). A plan that reads a table prepares one unless this
  // describes its input.
  PreparedInput prepared{};
};

// The device the policy plans for (the reference's DeviceCapabilities, reduced to what the MI355X policy reads).
struct DeviceCapabilities {
  uint32_t computeUnits = 256;
};

class Linear {
public:
  explicit Linear(const DeviceCapabilities &device) noexcept : computeUnits_(device.computeUnits ? device.computeUnits : 256) {}
  [[nodiscard]] LinearPlan plan(LinearWorkload workload) const;
  [[nodiscard]] LinearPlan plan(LinearWorkload workload, const Projection &projection,
                                const Projection *gate = nullptr) const;
  [[nodiscard]] uint32_t decodeStorageRows(uint32_t rows, ProjectionShape shape) const;
  [[nodiscard]] LinearPlan prefillPlan(const Projection &projection, uint32_t rows, LinearEpilogue epilogue) const;
  [[nodiscard]] LinearPlan decodePlan(const Projection &projection, uint32_t lanes,
                                      LinearEpilogue epilogue = LinearEpilogue::None,
                                      const Projection *gate = nullptr) const;
  [[nodiscard]] LinearScratchSize decodeScratchSize(ProjectionShape shape) const;
  [[nodiscard]] LinearScratchSize prefillScratchSize(ProjectionShape shape) const;
  // ggufFloatTile (Linear.hpp:273-276; LinearGguf.cpp:837-844): the tile of a float projection of `rows` rows into
  // `outputSize` columns of rows in `formatId` on this device.
  [[nodiscard]] FloatTile floatTile(uint32_t rows, uint32_t outputSize, uint32_t formatId) const noexcept;
  [[nodiscard]] static LinearPlan plan(LinearWorkload workload, LinearConfig config, FloatOutput destination);
  // Returns what the scratch table describes after the dispatch (Linear.cpp:203-231).
  PreparedInput add(hipStream_t graph, LinearBuffers buffers, const Projection &projection, const LinearPlan &plan,
                    const Projection *gate = nullptr) const;
  void addPrefill(hipStream_t graph, Buffer input, const Projection &projection, Buffer output, uint32_t rows,
                  LinearScratch scratch = {}) const;
  void addPrefillUpWithGate(hipStream_t graph, Buffer input, const Projection &up, Buffer gateScratch, Buffer output,
                            uint32_t rows, LinearScratch scratch) const;
  void addPrefillResidual(hipStream_t graph, Buffer input, const Projection &projection, Buffer residual,
                          Buffer output, uint32_t rows, LinearScratch scratch) const;
  void addPrefillSwiGlu(hipStream_t graph, const SwiGluProjections &ffn, const PrefillFfnBuffers &buffers,
                        Buffer residual, Buffer output, uint32_t rows) const;
  // The K partitions the decode tile splits an n x k projection of `rows` rows into on this device.
  [[nodiscard]] uint32_t decodeSplits(uint32_t n, uint32_t k, uint32_t rows, uint32_t groupUnit,
                                      bool pair = false) const noexcept;

private:
  [[nodiscard]] LinearConfig baseline(LinearWorkload workload, const Projection *projection,
                                      const Projection *gate) const;
  // The decode plan of a projection whose formats take `unit` scale groups a meta unit; `pair` runs a gate/up pair
  // of one format as one pass where the policy keeps it.
  [[nodiscard]] LinearConfig decodeConfig(LinearWorkload workload, uint32_t unit, bool pair) const noexcept;
  uint32_t computeUnits_;
};

// NormWeights (Normalization.hpp:14-23): the per-channel multipliers of an RMS norm, bf16 or F32 as stored.
struct NormWeights {
  Buffer buffer;
  bool float32 = false;
  [[nodiscard]] constexpr uint64_t bytes(uint32_t width) const noexcept { return uint64_t{width} * (float32 ? 4 : 2); }
};

// Normalization (Normalization.hpp:29-40).
struct Normalization {
  // out = bf16((x * rsqrt(sum x^2 / width + 1e-6)) * w) per row; also writes the consumer's `layout` table into
  // `scratch` when it is not Plain, and throws when `scratch` cannot hold it; returns what the scratch describes.
  static PreparedInput addRms(hipStream_t graph, Buffer input, const NormWeights &weight, Buffer output,
                              uint32_t width, uint32_t rows, LinearScratch scratch = {},
                              LinearInput layout = LinearInput::Plain);
};

// addGgufFloat (Linear.hpp:34-40) for a float segment: out[r][outOffset + n] = sum_k input[r][k] W[n][k] for rows
// r < `rows`, in fp32, into a `type` destination of `outStride` columns, on `tile` (the matrix-core tile takes K a
// multiple of 256, as the reference's neural accelerator tile takes K a multiple of 32).
void addGgufFloat(hipStream_t graph, Buffer input, const QuantizedSegment &weights, Buffer output, uint32_t rows,
                  uint32_t outStride, uint32_t outOffset, FloatOutput type, FloatTile tile);

}  // namespace sq::ops
