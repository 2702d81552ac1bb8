// The C ABI (include/splash_q4.h) over the operator layer: translates the POD structs, catches every exception at
// the boundary into a status code and a thread-local message, and launches on the caller's stream.
#include "../../../include/splash_q4.h"

#include <cstddef>
#include <cstring>
#include <mutex>
#include <string>

#include "../kernels/kernels.hpp"
#include "moe.hpp"
#include "ops.hpp"

namespace {

thread_local std::string lastError;

template <class F> int guarded(F &&f) {
  try {
    f();
    lastError.clear();
    return SQ_OK;
  } catch (const std::invalid_argument &e) {
    lastError = e.what();
    return SQ_INVALID_ARGUMENT;
  } catch (const std::exception &e) {
    lastError = e.what();
    return SQ_RUNTIME_ERROR;
  } catch (...) {
    lastError = "unknown error";
    return SQ_RUNTIME_ERROR;
  }
}

using namespace sq::ops;

Buffer buf(const sq_buffer &b) { return {b.ptr, b.bytes}; }
sq_buffer cbuf(const Buffer &b) { return {b.ptr, b.bytes}; }

template <class T> const T &need(const T *p, const char *what) {
  if (!p) throw std::invalid_argument(std::string(what) + " is null");
  return *p;
}
template <class T> T *need(T *p, const char *what) {
  if (!p) throw std::invalid_argument(std::string(what) + " is null");
  return p;
}

QuantizedSegment segment(const sq_segment &s) {
  QuantizedSegment q = QuantizedSegment::planes(s.format_id, s.output_size, s.input_size, buf(s.plane0), buf(s.plane1),
                                                buf(s.meta));
  q.columnOffset = s.column_offset;
  return q;
}

Projection projection(const sq_projection &p) {
  if (p.segment_count == 0 || p.segment_count > SQ_MAX_SEGMENTS)
    throw std::invalid_argument("block projection has no segments");
  BlockWeights blocks;
  for (uint32_t i = 0; i < p.segment_count; ++i) blocks.segments.push_back(segment(p.segments[i]));
  Projection out(p.output_size, p.input_size, std::move(blocks));
  if (p.destination > SQ_OUTPUT_F32) throw std::invalid_argument("invalid projection destination");
  out.destination = p.destination == SQ_OUTPUT_F32 ? FloatOutput::Float32 : FloatOutput::BFloat16;
  return out;
}

LinearWorkload workload(const sq_linear_workload &w) {
  if (w.phase > SQ_PHASE_DECODE || w.epilogue > SQ_EPILOGUE_UP_WITH_GATE)
    throw std::invalid_argument("invalid linear workload");
  return {{w.output_size, w.input_size}, w.rows, LinearPhase(w.phase), LinearEpilogue(w.epilogue)};
}
LinearConfig config(const sq_linear_config &c) {
  if (c.tile > SQ_TILE_REGISTER) throw std::invalid_argument("invalid linear tile");
  LinearConfig out;
  out.tile = LinearTile(c.tile);
  out.splits = c.splits;
  out.spread = c.spread != 0;
  out.oneGateUpPass = c.one_gate_up_pass != 0;
  out.sixteenRows = c.sixteen_rows != 0;
  return out;
}
sq_linear_plan cplan(const LinearPlan &p) {
  const LinearWorkload w = p.workload();
  const LinearConfig c = p.configuration();
  sq_linear_plan out{};
  out.workload = {w.matrix.outputSize, w.matrix.inputSize, w.rows, uint32_t(w.phase), uint32_t(w.epilogue)};
  out.config = {uint32_t(c.tile), c.splits, c.spread, c.oneGateUpPass, c.sixteenRows};
  out.destination = uint32_t(p.destination());
  out.storage_rows = p.storageRows();
  return out;
}
LinearPlan plan(const sq_linear_plan &p) {
  if (p.destination > SQ_OUTPUT_F32) throw std::invalid_argument("invalid plan destination");
  return Linear::plan(workload(p.workload), config(p.config), FloatOutput(p.destination));
}
Linear linear(const sq_device *d) { return Linear(DeviceCapabilities{d ? d->compute_units : 0}); }
LinearScratch linearScratch(const sq_linear_scratch *s) {
  if (!s) return {};
  return {buf(s->input), buf(s->sums), buf(s->partials), buf(s->counters), buf(s->rotated)};
}
sq_linear_scratch_size csize(const LinearScratchSize &s) { return {s.input, s.sums, s.partials, s.counters, s.rotated}; }
PreparedInput prepared(const sq_prepared_input &p) {
  if (p.layout > SQ_LINEAR_INPUT_HALF_ROWS) throw std::invalid_argument("unknown linear input layout");
  return {buf(p.source), LinearInput(p.layout)};
}
sq_prepared_input cprepared(const PreparedInput &p) { return {cbuf(p.source), uint32_t(p.layout)}; }
hipStream_t stream(void *graph) { return static_cast<hipStream_t>(graph); }
void launched(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

extern "C" {

const char *sq_last_error(void) { return lastError.c_str(); }
const char *sq_version(void) { return "splash_q4 0.1 gfx950"; }

int sq_linear_plan_for(const sq_device *device, const sq_linear_workload *w, const sq_projection *p,
                       const sq_projection *gate, sq_linear_plan *out) {
  return guarded([&] {
    const Linear l = linear(device);
    if (!p) {
      *out = cplan(l.plan(workload(need(w, "workload"))));
      return;
    }
    const Projection proj = projection(*p);
    if (gate) {
      const Projection g = projection(*gate);
      *out = cplan(l.plan(workload(need(w, "workload")), proj, &g));
    } else {
      *out = cplan(l.plan(workload(need(w, "workload")), proj));
    }
  });
}

int sq_linear_plan_config(const sq_linear_workload *w, const sq_linear_config *c, uint32_t destination,
                          sq_linear_plan *out) {
  return guarded([&] {
    if (destination > SQ_OUTPUT_F32) throw std::invalid_argument("invalid plan destination");
    *out = cplan(Linear::plan(workload(need(w, "workload")), config(need(c, "config")), FloatOutput(destination)));
  });
}

int sq_linear_decode_plan(const sq_device *device, const sq_projection *p, uint32_t lanes, uint32_t epilogue,
                          const sq_projection *gate, sq_linear_plan *out) {
  return guarded([&] {
    if (epilogue > SQ_EPILOGUE_UP_WITH_GATE) throw std::invalid_argument("invalid epilogue");
    const Projection proj = projection(need(p, "projection"));
    if (gate) {
      const Projection g = projection(*gate);
      *out = cplan(linear(device).decodePlan(proj, lanes, LinearEpilogue(epilogue), &g));
    } else {
      *out = cplan(linear(device).decodePlan(proj, lanes, LinearEpilogue(epilogue)));
    }
  });
}

int sq_linear_prefill_plan(const sq_device *device, const sq_projection *p, uint32_t rows, uint32_t epilogue,
                           sq_linear_plan *out) {
  return guarded([&] {
    if (epilogue > SQ_EPILOGUE_UP_WITH_GATE) throw std::invalid_argument("invalid epilogue");
    *out = cplan(linear(device).prefillPlan(projection(need(p, "projection")), rows, LinearEpilogue(epilogue)));
  });
}

int sq_linear_plan_scratch(const sq_linear_plan *p, sq_linear_scratch_size *out, uint64_t *gate_scratch_bytes) {
  return guarded([&] {
    const LinearPlan lp = plan(need(p, "plan"));
    if (out) *out = csize(lp.scratchSize());
    if (gate_scratch_bytes) *gate_scratch_bytes = lp.gateScratchBytes();
  });
}

int sq_linear_decode_scratch_size(const sq_device *device, uint32_t n, uint32_t k, sq_linear_scratch_size *out) {
  return guarded([&] { *out = csize(linear(device).decodeScratchSize({n, k})); });
}
int sq_linear_prefill_scratch_size(const sq_device *device, uint32_t n, uint32_t k, sq_linear_scratch_size *out) {
  return guarded([&] { *out = csize(linear(device).prefillScratchSize({n, k})); });
}

int sq_require_segment_planes(const sq_segment *s, const char *what, uint32_t plane_inputs) {
  return guarded([&] { requireSegmentPlanes(segment(need(s, "segment")), what ? what : "segment", plane_inputs); });
}

int sq_linear_add_prepared(void *graph, const sq_linear_buffers *b, const sq_projection *p, const sq_linear_plan *lp,
                           const sq_projection *gate, sq_prepared_input *result) {
  return guarded([&] {
    const sq_linear_buffers &bb = need(b, "buffers");
    LinearBuffers buffers{buf(bb.input), buf(bb.output), buf(bb.residual), buf(bb.gate_scratch), linearScratch(&bb.scratch),
                          prepared(bb.prepared)};
    const Projection proj = projection(need(p, "projection"));
    const LinearPlan selected = plan(need(lp, "plan"));
    const Linear l(DeviceCapabilities{});
    PreparedInput after;
    if (gate) {
      const Projection g = projection(*gate);
      after = l.add(stream(graph), buffers, proj, selected, &g);
    } else {
      after = l.add(stream(graph), buffers, proj, selected);
    }
    if (result) *result = cprepared(after);
  });
}
int sq_linear_add(void *graph, const sq_linear_buffers *b, const sq_projection *p, const sq_linear_plan *lp,
                  const sq_projection *gate) {
  return sq_linear_add_prepared(graph, b, p, lp, gate, nullptr);
}
}  // extern "C"

// ---- The entry point that allocates nothing (sq_linear_add_static)

namespace {

// The scratch of sq_linear_add_static: one array per GPU, held from the library's first use on that GPU to the end
// of the process. In host code `scratch` names a host-side stand-in; kernels get the device address that
// hipGetSymbolAddress gives, once per device (staticScratch).
constexpr uint64_t kStaticScratchBytes = SQ_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
constexpr int kMaximumDevices = 64;
std::mutex staticScratchMutex;
void *staticScratchBase[kMaximumDevices] = {};

void *staticScratch() {
  int device = 0;
  launched(hipGetDevice(&device), "static scratch device");
  if (device < 0 || device >= kMaximumDevices) throw std::runtime_error("static scratch: device index out of range");
  const std::lock_guard<std::mutex> lock(staticScratchMutex);
  if (!staticScratchBase[device]) {
    void *ptr = nullptr;
    launched(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "static scratch address");
    if (!ptr) throw std::runtime_error("static scratch address: null");
    staticScratchBase[device] = ptr;
  }
  return staticScratchBase[device];
}

// Clears `words` counters before a dispatch: a fill kernel rather than a memset, so that a captured graph replays it
// as a kernel node.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *words, uint32_t count) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) words[i] = 0;
}

// The plan's scratch regions (counters, partials, the prefill table and its row scales, the gate scratch) at
// 256-byte aligned offsets of the static array.
struct StaticLayout {
  uint64_t counters = 0, partials = 0, input = 0, sums = 0, gate = 0, end = 0;
};
StaticLayout staticLayout(const LinearScratchSize &s, uint64_t gateBytes) {
  const auto round = [](uint64_t v) { return (v + 255) & ~uint64_t{255}; };
  StaticLayout l;
  l.partials = round(l.counters + s.counters);
  l.input = round(l.partials + s.partials);
  l.sums = round(l.input + s.input);
  l.gate = round(l.sums + s.sums);
  l.end = l.gate + gateBytes;
  return l;
}

}  // namespace

extern "C" {

int sq_linear_add_static(void *graph, const sq_linear_buffers *b, const sq_projection *p, const sq_linear_plan *lp,
                         const sq_projection *gate) {
  return guarded([&] {
    const sq_linear_buffers &bb = need(b, "buffers");
    const Projection proj = projection(need(p, "projection"));
    const LinearPlan selected = plan(need(lp, "plan"));
    if (bb.prepared.source.ptr || bb.prepared.source.bytes || bb.prepared.layout)
      throw std::invalid_argument("the static-scratch entry point prepares its own table: buffers->prepared must be empty");
    const LinearScratchSize sizes = selected.scratchSize();
    // An up-with-gate plan's gate "scratch" is the caller's gate projection output, the operand its epilogue reads
    // (Linear::addPrefillUpWithGate): it stays the caller's buffer. Only a two-pass gate/up pair's gate, which the
    // plan writes and reads itself, comes from the static array.
    const bool callerGate = selected.workload().epilogue == LinearEpilogue::UpWithGate;
    const uint64_t gateBytes = callerGate ? 0 : selected.gateScratchBytes();
    const StaticLayout l = staticLayout(sizes, gateBytes);
    if (l.end > kStaticScratchBytes)
      throw std::invalid_argument("the plan needs " + std::to_string(l.end) + " bytes of scratch; the static scratch holds " +
                                  std::to_string(kStaticScratchBytes));
    uint8_t *base = static_cast<uint8_t *>(staticScratch());
    const auto region = [&](uint64_t offset, uint64_t bytes) { return bytes ? Buffer{base + offset, bytes} : Buffer{}; };
    if (sizes.counters) {
      const uint32_t words = uint32_t(sizes.counters / 4);
      hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, stream(graph),
                         reinterpret_cast<uint32_t *>(base + l.counters), words);
      launched(hipGetLastError(), "static scratch counters");
    }
    const LinearScratch sc{region(l.input, sizes.input), region(l.sums, sizes.sums),
                           region(l.partials, sizes.partials), region(l.counters, sizes.counters), {}};
    const LinearBuffers buffers{buf(bb.input), buf(bb.output), buf(bb.residual),
                                callerGate ? buf(bb.gate_scratch) : region(l.gate, gateBytes), sc, {}};
    const Linear linearOp(DeviceCapabilities{});
    if (gate) {
      const Projection g = projection(*gate);
      linearOp.add(stream(graph), buffers, proj, selected, &g);
    } else {
      linearOp.add(stream(graph), buffers, proj, selected);
    }
  });
}

int sq_linear_plan_input(const sq_linear_plan *lp, uint32_t *layout) {
  return guarded([&] {
    if (!layout) throw std::invalid_argument("layout is null");
    *layout = uint32_t(plan(need(lp, "plan")).input());
  });
}

int sq_norm_add_rms(void *graph, sq_buffer input, const sq_norm_weights *weight, sq_buffer output, uint32_t width,
                    uint32_t rows, const sq_linear_scratch *s, uint32_t layout, sq_prepared_input *result) {
  return guarded([&] {
    if (layout > SQ_LINEAR_INPUT_HALF_ROWS) throw std::invalid_argument("unknown linear input layout");
    const sq_norm_weights &w = need(weight, "norm weights");
    const PreparedInput after = Normalization::addRms(stream(graph), buf(input), NormWeights{buf(w.buffer), w.float32 != 0},
                                                      buf(output), width, rows, linearScratch(s), LinearInput(layout));
    if (result) *result = cprepared(after);
  });
}

int sq_float_add(void *graph, sq_buffer input, const sq_segment *weights, sq_buffer output, uint32_t rows,
                 uint32_t out_stride, uint32_t out_offset, uint32_t destination, uint32_t tile) {
  return guarded([&] {
    if (destination > SQ_OUTPUT_F32) throw std::invalid_argument("unknown float destination");
    if (tile > SQ_FLOAT_TILE_NEURAL_ACCELERATOR) throw std::invalid_argument("unknown float tile");
    const sq_segment &w = need(weights, "float rows");
    addGgufFloat(stream(graph), buf(input), QuantizedSegment::rows(w.format_id, w.output_size, w.input_size, buf(w.plane0)),
                 buf(output), rows, out_stride, out_offset, FloatOutput(destination), FloatTile(tile));
  });
}

int sq_linear_float_tile(const sq_device *device, uint32_t rows, uint32_t output_size, uint32_t format_id,
                         uint32_t *tile) {
  return guarded([&] { *need(tile, "tile") = uint32_t(linear(device).floatTile(rows, output_size, format_id)); });
}

int sq_linear_decode_storage_rows(const sq_device *device, uint32_t rows, uint32_t output_size, uint32_t input_size,
                                  uint32_t *storage_rows) {
  return guarded([&] {
    *need(storage_rows, "storage rows") = linear(device).decodeStorageRows(rows, {output_size, input_size});
  });
}

int sq_linear_add_prefill(const sq_device *device, void *graph, sq_buffer input, const sq_projection *p,
                          sq_buffer output, uint32_t rows, const sq_linear_scratch *s) {
  return guarded([&] {
    linear(device).addPrefill(stream(graph), buf(input), projection(need(p, "projection")), buf(output), rows, linearScratch(s));
  });
}
int sq_linear_add_prefill_residual(const sq_device *device, void *graph, sq_buffer input, const sq_projection *p,
                                   sq_buffer residual, sq_buffer output, uint32_t rows, const sq_linear_scratch *s) {
  return guarded([&] {
    linear(device).addPrefillResidual(stream(graph), buf(input), projection(need(p, "projection")), buf(residual),
                                      buf(output), rows, linearScratch(s));
  });
}
int sq_linear_add_prefill_up_with_gate(const sq_device *device, void *graph, sq_buffer input, const sq_projection *up,
                                       sq_buffer gate_scratch, sq_buffer output, uint32_t rows,
                                       const sq_linear_scratch *s) {
  return guarded([&] {
    linear(device).addPrefillUpWithGate(stream(graph), buf(input), projection(need(up, "projection")),
                                        buf(gate_scratch), buf(output), rows, linearScratch(s));
  });
}
int sq_linear_add_prefill_swiglu(const sq_device *device, void *graph, const sq_projection *gate,
                                 const sq_projection *up, const sq_projection *down, sq_buffer normalized,
                                 sq_buffer gate_scratch, sq_buffer intermediate, const sq_linear_scratch *s,
                                 sq_buffer residual, sq_buffer output, uint32_t rows) {
  return guarded([&] {
    const Projection g = projection(need(gate, "gate")), u = projection(need(up, "up")), d = projection(need(down, "down"));
    const PrefillFfnBuffers b{buf(normalized), buf(gate_scratch), buf(intermediate), linearScratch(s)};
    linear(device).addPrefillSwiGlu(stream(graph), {&g, &u, &d}, b, buf(residual), buf(output), rows);
  });
}

int sq_gguf_repack(void *graph, sq_buffer src, sq_buffer dst, const void *params) {
  return guarded([&] {
    SqGgufRepackParams p;
    std::memcpy(&p, &need(static_cast<const char *>(params), "params"), sizeof p);
    if (!sq_format_supported(p.fmt)) throw std::invalid_argument("repack takes a format this build runs");
    const SqQuantFormat f = sq_format(p.fmt);
    if (!p.rows || p.rows % SQ_TILE_ROWS || !p.input_size || p.input_size % f.block_elements)
      throw std::invalid_argument("a repack chunk takes whole plane tiles of rows and whole native blocks");
    const uint64_t rowBytes = uint64_t(p.input_size) / f.block_elements * f.block_bytes;
    if (p.src_row_bytes < rowBytes) throw std::invalid_argument("repack source rows are shorter than their blocks");
    const uint64_t groups = p.input_size / 32, units = groups / f.meta_groups;
    const uint64_t plane0 = uint64_t(p.rows) * groups * f.plane0_bytes, meta = uint64_t(p.rows) * units * f.meta_bytes;
    const uint64_t plane1 = uint64_t(p.rows) * groups * f.plane1_bytes;
    if (p.dst_meta < plane0) throw std::invalid_argument("repack meta offset overlaps plane0");
    if (plane1 && (p.dst_plane1 < plane0 || (p.dst_plane1 < p.dst_meta + meta && p.dst_meta < p.dst_plane1 + plane1)))
      throw std::invalid_argument("repack plane1 overlaps plane0 or meta");
    if (plane1) requireBytes(buf(dst), uint64_t(p.dst_plane1) + plane1, "repack destination");
    requireBytes(buf(src), (uint64_t(p.rows) - 1) * p.src_row_bytes + rowBytes, "repack source");
    requireBytes(buf(dst), uint64_t(p.dst_meta) + meta, "repack destination");
    launched(sq::kern::launch_repack(static_cast<const uint8_t *>(src.ptr), static_cast<uint8_t *>(dst.ptr), p,
                                     stream(graph)),
             "repack");
  });
}

int sq_mlx_repack(void *graph, uint32_t fmt, uint32_t rows, uint32_t k, sq_buffer weight, sq_buffer scales,
                  sq_buffer biases, sq_buffer plane0, sq_buffer meta) {
  return guarded([&] {
    if (!sq_affine_format(fmt)) throw std::invalid_argument("the MLX repack takes a 4-bit or 8-bit MLX affine format");
    const SqQuantFormat f = sq_format(fmt);
    if (!rows || rows % SQ_TILE_ROWS || !k || k % f.block_elements)
      throw std::invalid_argument("an MLX repack takes whole plane tiles of rows and whole groups");
    const uint64_t groups = k / f.block_elements, bits = fmt == SQ_FMT_AF8G64 ? 8 : 4;
    requireBytes(buf(weight), uint64_t(rows) * k * bits / 8, "MLX weight");
    requireBytes(buf(scales), uint64_t(rows) * groups * 2, "MLX scales");
    requireBytes(buf(biases), uint64_t(rows) * groups * 2, "MLX biases");
    requireBytes(buf(plane0), uint64_t(rows) * (k / 32) * f.plane0_bytes, "plane0");
    requireBytes(buf(meta), uint64_t(rows) * groups * 4, "meta");
    launched(sq::kern::launch_mlx_repack(fmt, static_cast<const uint32_t *>(weight.ptr),
                                         static_cast<const uint16_t *>(scales.ptr),
                                         static_cast<const uint16_t *>(biases.ptr), rows, k,
                                         static_cast<uint8_t *>(plane0.ptr), static_cast<uint8_t *>(meta.ptr),
                                         stream(graph)),
             "MLX repack");
  });
}

int sq_diag_stream_read(void *graph, sq_buffer src, sq_buffer sink, uint32_t workgroups, uint32_t threads) {
  return guarded([&] {
    if (!src.ptr || !src.bytes || src.bytes % 16) throw std::invalid_argument("stream source is whole 16-byte vectors");
    if (!workgroups || !threads || threads > 1024 || threads % 64)
      throw std::invalid_argument("stream launch takes workgroups of 64..1024 threads, whole waves");
    requireBytes(buf(sink), uint64_t{workgroups} * 4, "stream sink");
    launched(sq::kern::launch_stream_read(src.ptr, src.bytes, static_cast<uint32_t *>(sink.ptr), workgroups, threads,
                                          stream(graph)),
             "stream read");
  });
}

int sq_diag_mfma_peak(void *graph, sq_buffer sink, uint32_t workgroups, uint32_t waves_per_simd,
                      uint32_t iterations) {
  return guarded([&] {
    if (!workgroups || !iterations) throw std::invalid_argument("MFMA loop takes workgroups and iterations");
    if (waves_per_simd != 1 && waves_per_simd != 2) throw std::invalid_argument("MFMA loop runs 1 or 2 waves a SIMD");
    requireBytes(buf(sink), uint64_t{workgroups} * 4, "MFMA loop sink");
    launched(sq::kern::launch_mfma_peak(workgroups, waves_per_simd, iterations, static_cast<float *>(sink.ptr),
                                        stream(graph)),
             "MFMA loop");
  });
}

int sq_dequant(void *graph, const sq_segment *s, sq_buffer values, sq_buffer halves) {
  return guarded([&] {
    const QuantizedSegment q = segment(need(s, "segment"));
    requireSegmentPlanes(q, "dequant");
    const uint64_t n = uint64_t(q.outputSize) * q.inputSize;
    if (values.ptr) requireBytes(buf(values), n * 4, "dequant values");
    if (halves.ptr) requireBytes(buf(halves), n * 2, "dequant halves");
    launched(sq::kern::launch_dequant(q.formatId, q.plane0.as<const uint8_t>(), q.plane1.as<const uint8_t>(),
                                      q.meta.as<const uint8_t>(),
                                      q.outputSize, q.inputSize, static_cast<float *>(values.ptr),
                                      static_cast<uint16_t *>(halves.ptr), stream(graph)),
             "dequant");
  });
}

}  // extern "C"

// ---- MoE

namespace {
MoeShape moeShape(const sq_moe_shape &s) {
  if (s.router > SQ_MOE_ROUTER_SIGMOID_NORMALIZED) throw std::invalid_argument("unknown MoE router");
  return {s.hidden_size, s.experts, s.experts_per_token, s.expert_intermediate_size, s.expert_format,
          MoeRouter(s.router), s.shared_slices, s.shared_gated != 0};
}
sq_moe_config cconfig(const MoeConfig &c) {
  return {uint32_t(c.expertTile), uint32_t(c.ggufTile), uint32_t(c.ggufRouterTile), uint32_t(c.cpuBf16Experts)};
}
MoeConfig moeConfig(const sq_moe_config &c) {
  if (c.expert_tile != SQ_MOE_EXPERT_TILE_M8 && c.expert_tile != SQ_MOE_EXPERT_TILE_M32)
    throw std::invalid_argument("invalid MoE expert tile configuration");
  if (c.gguf_tile > SQ_MOE_GGUF_TILE_REGISTER) throw std::invalid_argument("invalid MoE GGUF tile");
  if (c.router_tile > SQ_FLOAT_TILE_NEURAL_ACCELERATOR) throw std::invalid_argument("invalid MoE router tile");
  return {MoeExpertTile(c.expert_tile), MoeGgufTile(c.gguf_tile), FloatTile(c.router_tile), c.cpu_bf16_experts != 0};
}
sq_moe_plan cmoe(const MoePlan &p) {
  sq_moe_plan out{};
  const MoeShape s = p.shape();
  out.shape = {s.hiddenSize, s.experts, s.expertsPerToken, s.expertIntermediateSize, s.expertFormat,
               uint32_t(s.router), s.sharedSlices, uint32_t(s.sharedGate)};
  out.rows = p.rows();
  out.phase = uint32_t(p.phase());
  out.tile_rows = p.tileRows();
  out.maximum_tiles = p.maximumTiles();
  out.config = cconfig(p.configuration());
  const MoeWorkspace &w = p.workspace();
  out.workspace = {w.selectedExperts, w.routingWeights, w.tileDescriptors, w.tileCount, w.groupedRoutes,
                   w.routeRows, w.groupedInput, w.expertIntermediate, w.expertOutput};
  return out;
}
// The plan a caller holds, rebuilt and checked: the same shape, rows, phase and config give the same plan.
MoePlan moePlan(const sq_moe_plan &p) {
  if (p.phase > SQ_PHASE_DECODE) throw std::invalid_argument("invalid MoE phase");
  const MoePlan plan(moeShape(p.shape), p.rows, moeConfig(p.config),
                     p.phase == SQ_PHASE_DECODE ? MoePhase::Decode : MoePhase::Prefill);
  if (plan.tileRows() != p.tile_rows || plan.maximumTiles() != p.maximum_tiles)
    throw std::invalid_argument("MoE plan fields do not match its shape, rows and config");
  return plan;
}
// The shared views are read only when the plan has shared slices.
MoeWeights moeWeights(const sq_moe_weights &w, const sq_moe_plan &p) {
  MoeWeights out{segment(w.gate), segment(w.up), segment(w.down), buf(w.slot_table), w.slots, {}, {}, {}, {}, {}};
  if (w.router.plane0.ptr)
    out.router = QuantizedSegment::rows(w.router.format_id, w.router.output_size, w.router.input_size,
                                        buf(w.router.plane0));
  if (p.shape.shared_slices) {
    out.sharedGate = segment(w.shared_gate);
    out.sharedUp = segment(w.shared_up);
    out.sharedDown = segment(w.shared_down);
    if (p.shape.shared_gated) out.sharedScalarGate = buf(w.shared_scalar_gate);
  }
  return out;
}
MoeBuffers moeBuffers(const sq_moe_buffers &b) {
  const sq_moe_scratch &s = b.scratch;
  return {buf(b.input), buf(b.residual), buf(b.output),
          MoeScratch{buf(s.selected_experts), buf(s.routing_weights), buf(s.tile_descriptors), buf(s.tile_count),
                     buf(s.grouped_routes), buf(s.route_rows), buf(s.grouped_input), buf(s.expert_intermediate),
                     buf(s.expert_output)},
          buf(b.verify_rows)};
}
}  // namespace

extern "C" {

int sq_moe_config_for(const sq_moe_shape *shape, uint32_t rows, uint32_t phase, sq_moe_config *out) {
  return guarded([&] {
    if (phase > SQ_PHASE_DECODE) throw std::invalid_argument("invalid MoE phase");
    *need(out, "config") = cconfig(MoE::config(moeShape(need(shape, "shape")), rows,
                                               phase == SQ_PHASE_DECODE ? MoePhase::Decode : MoePhase::Prefill));
  });
}
int sq_moe_prefill_plan(const sq_moe_shape *shape, uint32_t rows, const sq_moe_config *config, sq_moe_plan *out) {
  return guarded([&] {
    const MoeShape s = moeShape(need(shape, "shape"));
    *need(out, "plan") =
        cmoe(MoE::prefillPlan(s, rows, config ? moeConfig(*config) : MoE::config(s, rows, MoePhase::Prefill)));
  });
}
int sq_moe_decode_plan(const sq_moe_shape *shape, uint32_t lanes, const sq_moe_config *config, sq_moe_plan *out) {
  return guarded([&] {
    const MoeShape s = moeShape(need(shape, "shape"));
    const MoeConfig c = config ? moeConfig(*config) : MoE::config(s, lanes * SQ_TARGET_VERIFY_ROWS, MoePhase::Decode);
    *need(out, "plan") = cmoe(MoE::decodePlan(s, lanes, c));
  });
}
int sq_moe_decode_rows_plan(const sq_moe_shape *shape, uint32_t rows, sq_moe_plan *out) {
  return guarded([&] { *need(out, "plan") = cmoe(MoE::decodeRows(moeShape(need(shape, "shape")), rows)); });
}
uint32_t sq_moe_router_width(const sq_moe_shape *shape) {
  if (!shape) return 0;
  MoeShape s;
  s.experts = shape->experts;
  return s.routerWidth();
}
// Each MoE call rebuilds and checks the plan before it reads the buffers or weights.
int sq_moe_add(void *graph, const sq_moe_buffers *b, const sq_moe_weights *w, const sq_moe_plan *p) {
  return guarded([&] {
    const MoePlan plan = moePlan(need(p, "plan"));
    MoE::add(stream(graph), moeBuffers(need(b, "buffers")), moeWeights(need(w, "weights"), *p), plan);
  });
}
int sq_moe_add_routing(void *graph, const sq_moe_buffers *b, const sq_moe_weights *w, const sq_moe_plan *p) {
  return guarded([&] {
    const MoePlan plan = moePlan(need(p, "plan"));
    MoE::addRouting(stream(graph), moeBuffers(need(b, "buffers")), moeWeights(need(w, "weights"), *p), plan);
  });
}
int sq_moe_add_routed(void *graph, const sq_moe_buffers *b, const sq_moe_weights *w, const sq_moe_plan *p) {
  return guarded([&] {
    const MoePlan plan = moePlan(need(p, "plan"));
    MoE::addRouted(stream(graph), moeBuffers(need(b, "buffers")), moeWeights(need(w, "weights"), *p), plan);
  });
}
int sq_moe_add_routes(void *graph, sq_buffer input, const sq_segment *router, sq_buffer shared_scalar_gate,
                      sq_buffer scores, sq_buffer selected, sq_buffer routing_weights, uint32_t rows,
                      const sq_moe_shape *shape, uint32_t router_tile) {
  return guarded([&] {
    if (router_tile > SQ_FLOAT_TILE_NEURAL_ACCELERATOR) throw std::invalid_argument("invalid MoE router tile");
    const MoeShape s = moeShape(need(shape, "shape"));
    QuantizedSegment r;
    if (router && router->plane0.ptr)
      r = QuantizedSegment::rows(router->format_id, router->output_size, router->input_size, buf(router->plane0));
    MoE::addRoutes(stream(graph), buf(input), r, buf(shared_scalar_gate), buf(scores), buf(selected),
                   buf(routing_weights), rows, s, FloatTile(router_tile));
  });
}

static_assert(sizeof(sq_moe_expert_load_params) == sizeof(SqMoeExpertLoadParams) &&
                  offsetof(sq_moe_expert_load_projection, planes) == offsetof(SqMoeExpertLoadProjection, planes) &&
                  offsetof(sq_moe_expert_load_projection, slot_bytes) ==
                      offsetof(SqMoeExpertLoadProjection, slot_bytes),
              "sq_moe_expert_load_params is the reference's MoeExpertLoadParams");
uint32_t sq_moe_expert_load_groups(const sq_moe_expert_load_params *params) {
  if (!params) return 0;
  SqMoeExpertLoadParams p;
  std::memcpy(&p, params, sizeof p);
  return MoE::expertLoadGroups(p);
}

int sq_moe_expert_load(void *graph, sq_buffer staging, sq_buffer arena, sq_buffer slots, sq_buffer sources,
                       const sq_moe_expert_load_params *params, uint32_t jobs, sq_buffer grid) {
  return guarded([&] {
    SqMoeExpertLoadParams p;
    std::memcpy(&p, &need(params, "params"), sizeof p);
    MoE::addExpertLoad(stream(graph), buf(staging), buf(arena), buf(slots), buf(sources), p, jobs, buf(grid));
  });
}

}  // extern "C"
