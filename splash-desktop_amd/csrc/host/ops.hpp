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
[[nodiscard]] constexpr uint64_t elementBytes(FloatOutput type) noexcept {
  return type == FloatOutput::Float32 ? 4 : 2;
}

// Weights.hpp:79-121, planes layout (the float-rows layout is the router's, outside this path).
struct QuantizedSegment {
  Buffer plane0, plane1, meta;
  uint32_t outputSize = 0, inputSize = 0, columnOffset = 0, formatId = SQ_FMT_COUNT;
  [[nodiscard]] static QuantizedSegment planes(uint32_t formatId, uint32_t outputSize, uint32_t inputSize,
                                               Buffer plane0, Buffer plane1, Buffer meta);
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

class LinearPlan {
public:
  [[nodiscard]] LinearWorkload workload() const noexcept { return workload_; }
  [[nodiscard]] LinearConfig configuration() const noexcept { return config_; }
  [[nodiscard]] FloatOutput destination() const noexcept { return destination_; }
  [[nodiscard]] uint32_t storageRows() const noexcept;
  [[nodiscard]] LinearScratchSize scratchSize() const noexcept;
  [[nodiscard]] uint64_t gateScratchBytes() const noexcept;
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
  [[nodiscard]] static LinearPlan plan(LinearWorkload workload, LinearConfig config, FloatOutput destination);
  void add(hipStream_t graph, LinearBuffers buffers, const Projection &projection, const LinearPlan &plan,
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
  uint32_t computeUnits_;
};

}  // namespace sq::ops
