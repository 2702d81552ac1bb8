// Launch interface between the host operators (csrc/host) and the HIP kernels (csrc/kernels/*.hip). Everything
// here takes device pointers and plain sizes; the host validates shapes and buffer extents before it calls in.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../abi.h"

namespace sq::kern {

enum Epilogue : uint32_t { EpNone = 0, EpResidual = 1, EpUpWithGate = 2 };

// One weight tensor's planes in a dispatch: its 64-column tiles write destination columns
// [out_offset, out_offset + 64 * tiles).
struct Segment {
  const uint8_t *plane0;
  const uint8_t *meta;
  uint32_t tiles;
  uint32_t out_offset;
  const uint8_t *plane1;   // the high bits of Q5_K and Q6_K (null for the other formats)
  uint32_t fmt;            // SQ_FMT_*: read by a decode dispatch of kSegmentFormats
};

// The decode tiles: y[r][c] = sum_k x[r][k] w[c][k] over up to three segments of one format, or of any formats when
// launch_decode is given kSegmentFormats (each workgroup then runs its own segment's format; no epilogue, bf16
// output, the layout of the segments' longest meta unit, so each tile computes what it does alone). With
// gate.plane0 set, gate (gate) and up (seg[0]) run in one pass and the output is bf16(bf16(up) silu(bf16(gate))).
// Split partials are fp32 [split][rows][out_stride] (a gate/up pair's [split][rows][2 out_stride], gate's columns
// then up's); counters one per workgroup column (grid.x, at most one per 16 destination columns), zero before and
// after each dispatch.
//  - The column tile (rows <= kColumnTileRows): grid (64-column tiles, splits) of up to kColumnMaxWaves waves, each
//    lane one destination column.
//  - The row tile (more rows): grid (64-column tiles, splits) of up to 16 waves (fewer for more than 16 rows or a
//    gate/up pair), rows on the MFMA's 16-row side.
constexpr uint32_t kColumnTileRows = 4;
constexpr uint32_t kSegmentFormats = 0xFFFFFFFFu;
// The formats each tile runs: the decode column and row tiles, the prefill tile and the MoE expert passes, every
// format this build takes.
SQ_HD inline bool column_tile_format(uint32_t f) { return sq_format_supported(f); }
SQ_HD inline bool row_tile_format(uint32_t f) { return sq_format_supported(f); }
SQ_HD inline bool prefill_tile_format(uint32_t f) { return sq_format_supported(f); }
// The column tile's most waves (K slices) per workgroup, and the most groups of 32 inputs one wave streams.
constexpr uint32_t kColumnMaxWaves = 16, kColumnMaxGroups = 32;
// An MI355X's compute units, past which a row tile's 64-column workgroups take the longest slices (decode_layout).
constexpr uint32_t kDecodeUnits = 256;
struct DecodeArgs {
  const uint16_t *input;   // bf16 [rows][K]
  Segment seg[3];
  uint32_t segments;
  Segment gate;            // a one-pass gate/up pair's gate (plane0 null otherwise)
  void *output;            // bf16 or fp32 [rows][out_stride]
  const uint16_t *aux;     // bf16 [rows][out_stride]: the residual, or the gate of an up-with-gate pass
  float *partials;
  uint32_t *counters;
  uint32_t K, rows, splits, out_stride;
  // Column tile: 4 asks for 16-column workgroups (each wave four K slices; the same bits as 64-column ones), which
  // spread a projection of few tiles over more compute units; 0 or 1 for 64-column workgroups.
  uint32_t column_slices;
};
// A decode dispatch's layout: nb waves per workgroup, each a K slice of ks groups of 32 inputs (8, 16 or 32) of the
// split. {0, 0} when the split is not one the tile runs (a K partition takes whole meta units, and the split's
// slices must fit one workgroup).
struct DecodeLayout {
  uint32_t nb, ks;
};
DecodeLayout decode_layout(uint32_t fmt, uint32_t blocks, uint32_t K, uint32_t splits, bool pair, uint32_t rows);
// The format whose layout a dispatch takes: fmt, or for kSegmentFormats the segment format of the longest meta unit.
uint32_t layout_format(uint32_t fmt, const DecodeArgs &args);
hipError_t launch_decode(uint32_t fmt, uint32_t epilogue, bool f32_output, const DecodeArgs &args,
                         hipStream_t stream);
hipError_t launch_decode_column(uint32_t fmt, uint32_t epilogue, bool f32_output, const DecodeArgs &args,
                                hipStream_t stream);

// The prefill tile (rows > 32): activations converted once to fp16 with a power-of-two scale per row
// (launch_prefill_prepare, [rows][K] fp16 in the order the tile reads), then dequantised fp16 weights on MFMA.
hipError_t launch_prefill_prepare(const uint16_t *input, uint32_t rows, uint32_t K, uint16_t *half_input,
                                  float *row_scale, hipStream_t stream);
struct PrefillArgs {
  const uint16_t *half_input;  // fp16 [rows][K], rows scaled by 2^-e
  const float *row_scale;      // 2^e per row
  Segment seg[3];
  uint32_t segments;
  uint16_t *output;            // bf16 [rows][out_stride]
  const uint16_t *aux;
  uint32_t K, rows, out_stride;
  float *partials;             // a split or stream dispatch's fp32 pieces (prefill_scratch_bytes)
  uint32_t *counters;          // a stream dispatch's counter a stream tile, zero between dispatches
  uint32_t column_group0;      // set by launch_prefill: the dispatch's first column group,
  uint32_t split_at, split_columns;   // the step its pieces are cut at, the partial planes' row length
  // Set by launch_prefill for a stream dispatch (prefill_stream): its whole tiles, its stream tiles, the steps of a
  // range and the row blocks.
  uint32_t stream_dp, stream_tiles, stream_range, stream_row_blocks;
};
hipError_t launch_prefill(uint32_t fmt, uint32_t epilogue, const PrefillArgs &args, hipStream_t stream);
// The prefill dispatch's shape: tiles of bm rows (128 or 256) by four plane tiles, row_blocks x column_groups of
// them, 64 inputs a step, one workgroup each. With `split` (prefill_split of the projection's rows, whole width and
// K), the tiles from column group whole_groups on are cut at step split_at between two workgroups, which store their
// fp32 sums [2][rows][split columns] to the partials for a close dispatch that adds the pieces in K order and
// applies the epilogue (the schedule cuts every tile in halves: whole_groups 0, split_at half the steps).
constexpr uint32_t kPrefillUnits = 256, kPrefillSplitTiles = 64;   // an MI355X's compute units
struct PrefillSchedule {
  uint32_t bm, split, row_blocks, column_groups, whole_groups, split_at;
};
bool prefill_split(uint32_t rows, uint32_t plane_tiles, uint32_t K);
// A whole-K dispatch's stream schedule: its first dp_tiles tiles whole, the next stream_tiles as pieces of `range`
// steps, `workgroups` workgroups in all (none: stream_tiles 0).
struct PrefillStream {
  uint32_t dp_tiles, stream_tiles, range, workgroups;
};
PrefillStream prefill_stream(uint32_t row_blocks, uint32_t column_groups, uint32_t K);
PrefillSchedule prefill_schedule(uint32_t rows, uint32_t plane_tiles, uint32_t K, bool split);
// The partials and counters a prefill of `rows` over a projection of `plane_tiles` plane tiles uses (halved K:
// partials only; a stream dispatch: both).
struct PrefillScratch {
  uint64_t partials, counters;
};
PrefillScratch prefill_scratch_bytes(uint32_t rows, uint32_t plane_tiles, uint32_t K);

// Dequantisation of every weight of a segment's planes: fp32 fma(q, s, z) and the staged tile's fp16 rounding of
// it, [N][K] each (either may be null).
hipError_t launch_dequant(uint32_t fmt, const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, uint32_t N,
                          uint32_t K, float *values, uint16_t *halves, hipStream_t stream);
// Load-time repacks: native rows (GgufRepackParams layout) into plane0 / meta, and MLX tensors (uint32 codes,
// bf16 scales and biases) straight into plane0 / meta.
hipError_t launch_repack(const uint8_t *src, uint8_t *dst, const SqGgufRepackParams &params, hipStream_t stream);
// moe_expert_load: grid (groups, jobs, 3) of SQ_MOE_EXPERT_LOAD_THREADS threads, the device's grid[0..2] the live
// part of it.
hipError_t launch_expert_load(const uint8_t *staging, uint64_t staging_bytes, uint8_t *arena, uint64_t arena_bytes,
                              const uint32_t *slots, const uint64_t *sources, const SqMoeExpertLoadParams &params,
                              uint32_t groups, uint32_t jobs, const uint32_t *grid, hipStream_t stream);
// Measurement aid (diag.hip): a read-only stream of `bytes` (a multiple of 16) over `workgroups` workgroups.
// The RMS norm producer: out = bf16((x * rsqrt(sum x^2 / width + 1e-6)) * w) per row, w bf16 or fp32; with
// half_input set it also writes the prefill tile's prepared input of `out` (half_input [rows][width], row_scale
// [rows]), the bits launch_prefill_prepare would write from it. width % 64 == 0; buffers 16-byte aligned.
hipError_t launch_rms_norm(const uint16_t *input, const void *weight, bool f32_weights, uint16_t *output,
                           uint32_t width, uint32_t rows, uint16_t *half_input, float *row_scale, hipStream_t stream);
// A float projection: out[r][out_offset + n] = sum_k x[r][k] W[n][k] for W's N rows of K values stored fp32 or bf16,
// fp32 products and sums, into fp32 or bf16 [rows][out_stride]. K % 4 == 0. `mfma` runs the fp32 MFMA tile (K a
// multiple of kFloatMfmaInputs, any rows), else the lane chains; either way an output takes at most K / 64 + 8
// roundings. kFloatMfmaRows: the rows from which the policy takes the MFMA tile.
constexpr uint32_t kFloatMfmaRows = 64, kFloatMfmaInputs = 256;
hipError_t launch_float_rows(const uint16_t *input, const void *weights, bool f32_weights, void *output,
                             bool f32_output, uint32_t rows, uint32_t N, uint32_t K, uint32_t out_stride,
                             uint32_t out_offset, bool mfma, hipStream_t stream);
hipError_t launch_stream_read(const void *src, uint64_t bytes, uint32_t *sink, uint32_t workgroups, uint32_t threads,
                              hipStream_t stream);
hipError_t launch_mfma_peak(uint32_t workgroups, uint32_t waves_per_simd, uint32_t iterations, float *sink,
                            hipStream_t stream);
hipError_t launch_mlx_repack(uint32_t fmt, const uint32_t *weight, const uint16_t *scales, const uint16_t *biases,
                             uint32_t rows, uint32_t K, uint8_t *plane0, uint8_t *meta, hipStream_t stream);

// MoE.
// With rows_table set, each row's wave also writes its input row in the expert tiles' read order there (what
// launch_moe_input_rows writes), so MoE::add needs no separate dispatch for it.
hipError_t launch_moe_route_select(const float *scores, uint32_t score_stride, uint32_t *selected,
                                   float *routing_weights, const SqMoeRouteParams &params, const uint16_t *input,
                                   const float *shared_gate, uint32_t router, uint32_t shared, uint16_t *rows_table,
                                   hipStream_t stream);
hipError_t launch_moe_group(const uint32_t *selected, SqMoeTileDescriptor *tiles, SqMoeTileCount *tile_count,
                            uint32_t *grouped_routes, uint32_t *route_rows, const uint32_t *verify_rows,
                            const SqMoeGroupParams &params, uint32_t shared, hipStream_t stream);
// The block's input rows [rows][K] in the expert tiles' read order (the table the expert passes read): 16-byte
// chunk 4 g + c of a row holds inputs 32 g + 4 c .. +3 then 32 g + 16 + 4 c .. +3.
hipError_t launch_moe_input_rows(const uint16_t *input, uint32_t rows, uint32_t K, uint16_t *table,
                                 hipStream_t stream);
// An expert pass over the grouped rows, tile by tile: gate_up: gate and up of each tile's expert in one pass over
// input rows routes[row] / routes_per_row, out = bf16(bf16(up) silu(bf16(gate))); else one tensor, over those input
// rows when `gather` (a gate or up of its own format) and over the grouped input rows otherwise, out = bf16(y), or
// with `gate` set (the gate pass's bf16 output, [tiles * tile_rows][output_size]) bf16(bf16(y) silu(gate)), the
// one-pass result bit for bit. Every pass reads its input rows in the read order of launch_moe_input_rows, and the
// gathering passes (gate/up) write their rows in that order too, for the down pass; the down pass writes in column
// order. Routed tiles (expert < experts) read the routed planes, expert e's rows from slots[e] * output_size on;
// shared tiles (expert experts + s) the shared planes, slice s's rows s * output_size on. `mode` picks the tiles a
// launch runs: 0 routed, 1 shared, 2 both (one format).
struct MoeExpertArgs {
  const uint16_t *input;        // gate/up: the step's rows [rows][K]; down: grouped rows [tiles * tile_rows][K]
  const uint32_t *routes;       // gate/up: the route of each grouped row (~0u padding)
  const SqMoeTileDescriptor *tiles;
  const SqMoeTileCount *tile_count;
  const uint8_t *plane0[2];     // gate (or the single pass's weights), up
  const uint8_t *meta[2];
  const uint8_t *plane1[2];     // Q5_K and Q6_K high bits (null otherwise)
  const uint8_t *shared_plane0[2];
  const uint8_t *shared_meta[2];
  const uint8_t *shared_plane1[2];
  const uint32_t *slots;
  uint16_t *output;             // [tiles * tile_rows][output_size]
  const uint16_t *gate;         // a single tensor's up-with-gate operand (null otherwise)
  uint32_t K, output_size, tile_rows, max_tiles, fmt, gate_up, routes_per_row, experts, mode, gather;
  uint32_t row_halves;          // 1: each tile's rows in 16-row halves, a workgroup each (tile_rows <= 32)
};
hipError_t launch_moe_expert(const MoeExpertArgs &args, hipStream_t stream);
hipError_t launch_moe_combine(const uint16_t *expert_output, const uint32_t *route_rows,
                              const float *routing_weights, const uint16_t *residual, uint16_t *output,
                              const SqMoeCombineParams &params, hipStream_t stream);

}  // namespace sq::kern
