// The producers either side of the projections: Normalization::addRms (reference: runtime/ops/Normalization.cpp:16-38)
// and the float projection of F32 or BF16 rows, addGgufFloat (runtime/ops/LinearGguf.cpp:806-818), which the MoE
// router runs through.
#include "ops.hpp"

#include "../kernels/kernels.hpp"

namespace sq::ops {
namespace {

void launched(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

bool aligned16(const Buffer &b) { return (reinterpret_cast<uintptr_t>(b.ptr) & 15u) == 0; }

}  // namespace

PreparedInput Normalization::addRms(hipStream_t graph, Buffer input, const NormWeights &weight, Buffer output,
                                    uint32_t width, uint32_t rows, LinearScratch scratch, LinearInput layout) {
  const uint64_t bytes = uint64_t{rows} * width * 2;
  if (!rows || !width) throw std::invalid_argument("a norm takes rows of inputs");
  requireBytes(input, bytes, "norm input");
  requireBytes(output, bytes, "norm output");
  requireBytes(weight.buffer, weight.bytes(width), "norm weights");
  if (width % 64) throw std::invalid_argument("the norm takes rows of whole 64-input spans");
  if (!aligned16(input) || !aligned16(output) || !aligned16(weight.buffer))
    throw std::invalid_argument("norm input, output and weights are 16-byte aligned");
  const bool table = layout != LinearInput::Plain;
  if (table) requireTableScratch(scratch, layout, width, rows);
  launched(kern::launch_rms_norm(input.as<const uint16_t>(), weight.buffer.ptr, weight.float32, output.as<uint16_t>(),
                                 width, rows, table ? scratch.input.as<uint16_t>() : nullptr,
                                 table ? scratch.sums.as<float>() : nullptr, graph),
           "rms norm");
  return table ? PreparedInput{output, layout} : PreparedInput{};
}

void addGgufFloat(hipStream_t graph, Buffer input, const QuantizedSegment &w, Buffer output, uint32_t rows,
                  uint32_t outStride, uint32_t outOffset, FloatOutput type, FloatTile tile) {
  if (!w.isFloat()) throw std::invalid_argument("the float projection takes F32 or BF16 rows");
  if (tile != FloatTile::Simdgroup && tile != FloatTile::NeuralAccelerator)
    throw std::invalid_argument("unknown float tile");
  const bool matrix = tile == FloatTile::NeuralAccelerator;
  if (matrix && w.inputSize % kern::kFloatMfmaInputs)
    throw std::invalid_argument("the matrix-core float tile takes inputs in multiples of 256");
  if (!rows || !w.outputSize || !w.inputSize || w.inputSize % 4)
    throw std::invalid_argument("the float projection takes rows of a multiple of 4 inputs");
  if (uint64_t{outOffset} + w.outputSize > outStride)
    throw std::invalid_argument("the float projection's columns fall outside its destination");
  const bool f32 = w.formatId == QuantizedSegment::kFloat32;
  requireBytes(w.plane0, uint64_t{w.outputSize} * w.inputSize * (f32 ? 4 : 2), "float rows");
  requireBytes(input, uint64_t{rows} * w.inputSize * 2, "float projection input");
  requireBytes(output, rowBytes(rows, outStride, uint64_t{outOffset} + w.outputSize, elementBytes(type)),
               "float projection output");
  if (!aligned16(w.plane0) || (reinterpret_cast<uintptr_t>(input.ptr) & 7u))
    throw std::invalid_argument("float rows are 16-byte aligned and the input 8-byte aligned");
  launched(kern::launch_float_rows(input.as<const uint16_t>(), w.plane0.ptr, f32, output.ptr,
                                   type == FloatOutput::Float32, rows, w.outputSize, w.inputSize, outStride, outOffset,
                                   matrix, graph),
           "float projection");
}

}  // namespace sq::ops
