/*
 * splash_q4 — MI355X (gfx950) quantized matmul path: bf16 activations x 4-bit group-quantized weights (and the
 * adjacent 5-, 6- and 8-bit formats), fp32 accumulation. C ABI over the reference's splash::ops::Linear /
 * splash::ops::MoE call surface.
 *
 * Conventions
 *  - Buffers are device-pointer views {ptr, bytes} (the reference's MetalBuffer views). The caller owns every
 *    buffer; nothing here allocates device memory.
 *  - A "graph" is a hipStream_t passed as void*: an add call validates everything, then launches in order on it.
 *    NULL is the default stream.
 *  - Every function returns SQ_OK or an error code; nothing is launched when it fails. sq_last_error() holds the
 *    thread's message for the last failure (the text of the reference's std::invalid_argument where it has one).
 *  - Format ids, plane layouts and parameter blocks are the reference's (runtime/metal/abi/QuantFormat.h, Gguf.h,
 *    MoE.h): Q4_K (0), Q5_K (3), Q6_K (4), Q8_0 (6), MLX affine 4-bit in groups of 32, 64 and 128 (25, 26, 27)
 *    and MLX affine 8-bit in groups of 64 (35), in every entry point.
 *  - Split scratch (partials, counters) is reused serially on one stream: counters are zero at allocation and every
 *    split or stream dispatch returns them to zero; two streams never share one scratch.
 * Reference interfaces each entry point replaces are named in its comment (paths under the reference checkout).
 */
#ifndef SPLASH_Q4_H
#define SPLASH_Q4_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SQ_OK 0
#define SQ_INVALID_ARGUMENT 1 /* the reference throws std::invalid_argument */
#define SQ_RUNTIME_ERROR 2    /* a HIP launch or runtime failure */

#define SQ_FMT_Q4K 0u
#define SQ_FMT_Q5K 3u
#define SQ_FMT_Q6K 4u
#define SQ_FMT_Q80 6u
#define SQ_FMT_AF4G32 25u
#define SQ_FMT_AF4G64 26u
#define SQ_FMT_AF4G128 27u
#define SQ_FMT_AF8G64 35u
/* Float rows (QuantizedSegment::rows, Weights.hpp:67-81): F32 rows carry the format id kFloat32, BF16 rows
 * GGUF_FMT_BF16; the float projection multiplies them unrounded in fp32. */
#define SQ_FMT_BF16 41u
#define SQ_FLOAT32_ROWS 0xFFFFFFFFu

/* enum values match the reference's enum class order (Linear.hpp:67-80, Weights.hpp:62) */
#define SQ_PHASE_PREFILL 0u
#define SQ_PHASE_DECODE 1u
#define SQ_EPILOGUE_NONE 0u
#define SQ_EPILOGUE_RESIDUAL 1u
#define SQ_EPILOGUE_GATE_UP 2u
#define SQ_EPILOGUE_UP_WITH_GATE 3u
#define SQ_TILE_STAGED 0u   /* LinearTile::GgufStaged: the decode tile */
#define SQ_TILE_PREFILL 1u  /* LinearTile::GgufPrefill */
#define SQ_TILE_REGISTER 2u /* LinearTile::GgufRegister: refused (Apple9 only) */
#define SQ_OUTPUT_BF16 0u
#define SQ_OUTPUT_F32 1u
#define SQ_MAX_SEGMENTS 3u

typedef struct sq_buffer {
  void *ptr;
  uint64_t bytes;
} sq_buffer;

/* QuantizedSegment, planes layout (runtime/ops/Weights.hpp:79-121). */
typedef struct sq_segment {
  sq_buffer plane0, plane1, meta;
  uint32_t output_size, input_size, column_offset, format_id;
} sq_segment;

/* Projection (runtime/ops/Weights.hpp:131-188): segments tile the leading output columns in order. */
typedef struct sq_projection {
  uint32_t output_size, input_size;
  uint32_t segment_count;
  uint32_t destination; /* SQ_OUTPUT_* */
  sq_segment segments[SQ_MAX_SEGMENTS];
} sq_projection;

/* LinearWorkload / LinearConfig / LinearPlan (runtime/ops/Linear.hpp:93-214). */
typedef struct sq_linear_workload {
  uint32_t output_size, input_size, rows, phase, epilogue;
} sq_linear_workload;
typedef struct sq_linear_config {
  uint32_t tile, splits, spread, one_gate_up_pass, sixteen_rows;
} sq_linear_config;
typedef struct sq_linear_plan {
  sq_linear_workload workload;
  sq_linear_config config;
  uint32_t destination;
  uint32_t storage_rows;
} sq_linear_plan;

/* LinearScratch / LinearScratchSize / LinearBuffers (runtime/ops/Linear.hpp:125-162,216-226). A decode plan's
 * partials hold its K splits' fp32 sums; a prefill plan's, where its tiles' K is halved (projections of 64 to 128
 * tiles of 256 rows by 256 columns, K a multiple of 512), the two halves' fp32 sums [2][rows][N], and where its
 * tiles number more than one round over the 256 compute units (K a multiple of 256), the fp32 sums of the last
 * round's stream pieces (128 MiB: two 256 x 256 tiles of sums for each of 256 workgroups) with a 4-byte counter
 * a stream tile. */
typedef struct sq_linear_scratch_size {
  uint64_t input, sums, partials, counters, rotated;
} sq_linear_scratch_size;
typedef struct sq_linear_scratch {
  sq_buffer input, sums, partials, counters, rotated;
} sq_linear_scratch;
/* LinearInput (Linear.hpp:166-169): the activation layout a plan reads. TABLE16 is the reference's Apple9 register
 * tile table, which no plan here reads (a producer asked for it is refused); HALF_ROWS is this build's prefill
 * table: the rows in fp16, scaled by a power of two per row and stored group by group in the prefill tile's read
 * order, in scratch.input, with the powers (fp32) in scratch.sums. */
#define SQ_LINEAR_INPUT_PLAIN 0u
#define SQ_LINEAR_INPUT_TABLE16 1u
#define SQ_LINEAR_INPUT_HALF_ROWS 2u
/* PreparedInput (Linear.hpp:184-190): the scratch table currently holds `source` in `layout`. */
typedef struct sq_prepared_input {
  sq_buffer source;
  uint32_t layout;
} sq_prepared_input;
typedef struct sq_linear_buffers {
  sq_buffer input, output, residual, gate_scratch;
  sq_linear_scratch scratch;
  /* What the scratch table holds (LinearBuffers::prepared, Linear.hpp:216-226): a plan that reads a table prepares
   * one unless this describes its input (same pointer and bytes). All zero: nothing. */
  sq_prepared_input prepared;
} sq_linear_buffers;

/* DeviceCapabilities, as far as the MI355X policy reads it (the decode split law, and the column tile's 16-column
 * workgroups for dispatches of few tiles, which compute the same bits as 64-column ones); compute_units 0 takes 256.
 * The prefill tile's schedule is a function of the shape alone, for the MI355X's 256 compute units. */
typedef struct sq_device {
  uint32_t compute_units;
} sq_device;

const char *sq_last_error(void);
/* Library version string. */
const char *sq_version(void);

/* ---- planning (host only; no GPU needed) ---- */

/* Linear::plan(LinearWorkload) and Linear::plan(workload, projection, gate) (Linear.cpp:151-164).
 * projection and gate may be NULL. */
int sq_linear_plan_for(const sq_device *device, const sq_linear_workload *workload, const sq_projection *projection,
                       const sq_projection *gate, sq_linear_plan *out);
/* static Linear::plan(workload, config, destination) (Linear.cpp:155-157). */
int sq_linear_plan_config(const sq_linear_workload *workload, const sq_linear_config *config, uint32_t destination,
                          sq_linear_plan *out);
/* Linear::decodePlan (Linear.cpp:166-169): rows = lanes * 8. */
int sq_linear_decode_plan(const sq_device *device, const sq_projection *projection, uint32_t lanes, uint32_t epilogue,
                          const sq_projection *gate, sq_linear_plan *out);
/* Linear::prefillPlan (Linear.cpp:170-172). */
int sq_linear_prefill_plan(const sq_device *device, const sq_projection *projection, uint32_t rows, uint32_t epilogue,
                           sq_linear_plan *out);
/* LinearPlan::scratchSize and gateScratchBytes (LinearGguf.cpp:432-453, Linear.cpp:123-129). */
int sq_linear_plan_scratch(const sq_linear_plan *plan, sq_linear_scratch_size *out, uint64_t *gate_scratch_bytes);
/* Linear::decodeScratchSize / prefillScratchSize (Linear.cpp:174-196). */
int sq_linear_decode_scratch_size(const sq_device *device, uint32_t output_size, uint32_t input_size,
                                  sq_linear_scratch_size *out);
int sq_linear_prefill_scratch_size(const sq_device *device, uint32_t output_size, uint32_t input_size,
                                   sq_linear_scratch_size *out);
/* Linear::decodeStorageRows (Linear.hpp:254-257; Linear.cpp:145-149): the rows of storage a decode step of `rows`
 * rows (1..32) binds for a projection of output_size x input_size, the storage_rows of its decode plans, which every
 * epilogue shares. The engine sizes its decode activation and output buffers with it (QwenTarget.cpp:125,
 * DFlashDraft.cpp:239). */
int sq_linear_decode_storage_rows(const sq_device *device, uint32_t rows, uint32_t output_size, uint32_t input_size,
                                  uint32_t *storage_rows);
/* Linear::ggufFloatTile (Linear.hpp:273-276; LinearGguf.cpp:837-844): the SQ_FLOAT_TILE_* a float projection of `rows`
 * rows into output_size columns of rows in format_id takes on this device. MI355X's policy: the matrix-core tile
 * from 64 rows on, the lane chains below. ExecutionPlans picks the MoE router's tile with it (ExecutionPlans.cpp:62),
 * as sq_moe_config_for does. */
int sq_linear_float_tile(const sq_device *device, uint32_t rows, uint32_t output_size, uint32_t format_id,
                         uint32_t *tile);
/* requireSegmentPlanes (LinearGguf.cpp:905-923): SQ_OK when the planes hold every tile of the segment. */
int sq_require_segment_planes(const sq_segment *segment, const char *what, uint32_t plane_inputs);

/* ---- dispatch ---- */

/* Linear::add (Linear.cpp:203-232; LinearGguf.cpp:579-802): the plan's projection of buffers->input. A decode of a
 * projection of up to SQ_MAX_SEGMENTS segments runs them in one dispatch whatever their formats (gguf_decode_fused);
 * a prefill runs one dispatch per format. A prefill plan's input, output, residual, gate scratch, scratch table and
 * partials are 16-byte aligned and its row scales (scratch sums) 4-byte aligned. Whether a prefill halves its tiles'
 * K depends on the chunk's rows as well as the shape (a 4096-input, 14336-output projection halves from 257 to 512
 * rows), so a row's output bits may differ between chunks of different row counts; each lies within the row's fp64
 * interval. The same holds for the tiles past a prefill's whole rounds over the compute units, whose K runs in
 * pieces on several workgroups (their sums add in K order whatever order the pieces finish in, so a chunk's bits
 * repeat from run to run). A decode row's bits depend only on the shape and the tile kind its rows run (1..4 rows,
 * 5..16, 17..32). */
int sq_linear_add(void *graph, const sq_linear_buffers *buffers, const sq_projection *projection,
                  const sq_linear_plan *plan, const sq_projection *gate);
/* Linear::add with its result: *prepared (may be NULL) receives what the scratch table describes after the
 * dispatch (the PreparedInput Linear::add returns, Linear.cpp:222-231). */
int sq_linear_add_prepared(void *graph, const sq_linear_buffers *buffers, const sq_projection *projection,
                           const sq_linear_plan *plan, const sq_projection *gate, sq_prepared_input *prepared);
/* No counterpart in the reference: Linear::add for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). The same plans and kernels as sq_linear_add, but
 * the split partials and counters, the prefill table and its row scales and a two-pass gate/up pair's gate scratch
 * come from a static array of SQ_STATIC_SCRATCH_BYTES per GPU inside the library (held from its first use on that GPU
 * to the end of the process); buffers->scratch is ignored and buffers->prepared must be empty. buffers->gate_scratch
 * is read only by an UP_WITH_GATE plan, as the gate operand its epilogue multiplies in (the caller's gate projection
 * output, checked to hold the plan's rows as sq_linear_add checks it), and ignored by every other plan. A plan whose
 * scratch exceeds the array is refused (SQ_INVALID_ARGUMENT). Nothing is allocated: it launches a counter-clearing
 * kernel, then the plan's dispatches. Every call on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (two streams, two threads) race; calls in one stream's order do not. */
#define SQ_STATIC_SCRATCH_BYTES (16u << 20)
int sq_linear_add_static(void *graph, const sq_linear_buffers *buffers, const sq_projection *projection,
                         const sq_linear_plan *plan, const sq_projection *gate);
/* LinearPlan::input (Linear.hpp:199-202): the layout the producer of the plan's input may write (SQ_LINEAR_INPUT_*):
 * HALF_ROWS for a prefill plan, PLAIN otherwise. */
int sq_linear_plan_input(const sq_linear_plan *plan, uint32_t *layout);

/* ---- producers either side of the path ---- */

/* NormWeights (Normalization.hpp:14-23): the per-channel multipliers of an RMS norm, bf16 (float32 0) or F32. */
typedef struct sq_norm_weights {
  sq_buffer buffer;
  uint32_t float32;
} sq_norm_weights;
/* Normalization::addRms (Normalization.hpp:35-39; Normalization.cpp:16-38): output = bf16((x rsqrt(sum x^2 / width +
 * 1e-6)) w) for `rows` rows of `width` bf16 inputs. With layout SQ_LINEAR_INPUT_HALF_ROWS it also writes the prefill
 * table of `output` into *scratch (input: rows * width * 2 bytes, sums: rows * 4), the bits the prefill's own
 * preparation would write; *prepared (may be NULL) receives what the scratch then describes. scratch may be NULL
 * for PLAIN. width % 64 == 0; input, output, weights and the table 16-byte aligned. */
int sq_norm_add_rms(void *graph, sq_buffer input, const sq_norm_weights *weight, sq_buffer output, uint32_t width,
                    uint32_t rows, const sq_linear_scratch *scratch, uint32_t layout, sq_prepared_input *prepared);
/* addGgufFloat (Linear.hpp:34-40; LinearGguf.cpp:847-853) for a float segment (format SQ_FLOAT32_ROWS or
 * SQ_FMT_BF16, its rows in plane0): output[r][out_offset + n] = sum_k input[r][k] W[n][k] for r < rows, products and
 * sums in fp32, into an fp32 or bf16 (destination SQ_OUTPUT_*) destination of out_stride columns, on `tile`
 * (SQ_FLOAT_TILE_*, sq_linear_float_tile's choice or the caller's). input_size % 4 == 0; the matrix-core tile takes
 * input_size a multiple of 256 (the reference's neural accelerator tile: 32), else SQ_INVALID_ARGUMENT. Both tiles lie
 * within (input_size / 64 + 8) 2^-24 sum |x w| of the exact sum. */
int sq_float_add(void *graph, sq_buffer input, const sq_segment *weights, sq_buffer output, uint32_t rows,
                 uint32_t out_stride, uint32_t out_offset, uint32_t destination, uint32_t tile);
/* Linear::addPrefill / addPrefillResidual / addPrefillUpWithGate (Linear.cpp:234-256). */
int sq_linear_add_prefill(const sq_device *device, void *graph, sq_buffer input, const sq_projection *projection,
                          sq_buffer output, uint32_t rows, const sq_linear_scratch *scratch);
int sq_linear_add_prefill_residual(const sq_device *device, void *graph, sq_buffer input,
                                   const sq_projection *projection, sq_buffer residual, sq_buffer output,
                                   uint32_t rows, const sq_linear_scratch *scratch);
int sq_linear_add_prefill_up_with_gate(const sq_device *device, void *graph, sq_buffer input, const sq_projection *up,
                                       sq_buffer gate_scratch, sq_buffer output, uint32_t rows,
                                       const sq_linear_scratch *scratch);
/* Linear::addPrefillSwiGlu (Linear.cpp:244-250): output = residual + down(silu(gate x) * up x). */
int sq_linear_add_prefill_swiglu(const sq_device *device, void *graph, const sq_projection *gate,
                                 const sq_projection *up, const sq_projection *down, sq_buffer normalized,
                                 sq_buffer gate_scratch, sq_buffer intermediate, const sq_linear_scratch *scratch,
                                 sq_buffer residual, sq_buffer output, uint32_t rows);

/* ---- weight preparation (load time) ---- */

/* The gguf_repack dispatch (kernels/shared/gguf_repack.metal:232-238; GgufRepack.h:10-18): native rows in src
 * (src_row_bytes apart) into dst: plane0 at 0, meta at dst_meta, and Q5_K's and Q6_K's high bits at dst_plane1
 * (unused by the other formats).
 * params points at the reference's 24-byte GgufRepackParams {rows, input_size, fmt, src_row_bytes, dst_plane1,
 * dst_meta}. */
int sq_gguf_repack(void *graph, sq_buffer src, sq_buffer dst, const void *params);
/* MLX tensors (mlx.core.quantize affine, bits 4 or 8: uint32 codes [rows][K * bits / 32], bf16 scales and biases
 * [rows][K/group]) straight into planes: the loader's native-block build (model/GgufPreparation.cpp:141-193) and
 * the repack in one dispatch. */
int sq_mlx_repack(void *graph, uint32_t format_id, uint32_t rows, uint32_t input_size, sq_buffer weight,
                  sq_buffer scales, sq_buffer biases, sq_buffer plane0, sq_buffer meta);
/* Every weight of a segment dequantised: fp32 fma(q, s, z) (Q6_K s (q - 32), Q8_0 d v) and its fp16 rounding (the
 * staged tiles' weight), [N][K] each; either output may have a NULL ptr (reference test kernel
 * gguf_test_dequant_<fmt>, dev/tests/engine/gguf_dequant_test.metal:5-21). */
int sq_dequant(void *graph, const sq_segment *segment, sq_buffer values_f32, sq_buffer values_f16);

/* ---- measurement ---- */

/* No counterpart in the reference: a read-only stream of src (whole 16-byte vectors) by `workgroups` workgroups of
 * `threads` threads, thread g folding vectors g, g + S, g + 2S, ... (S = workgroups * threads). A workgroup's word of
 * sink is written only when one of its threads' folds equals the marker word 0x9E3779B9 (the thread's index + 1), so
 * no store is timed. The HBM floor the GEMV is measured against (bench.py). */
int sq_diag_stream_read(void *graph, sq_buffer src, sq_buffer sink, uint32_t workgroups, uint32_t threads);

/* No counterpart in the reference: `workgroups` workgroups of four waves (at most waves_per_simd, 1 or 2, resident a
 * SIMD), each wave running `iterations` x 8 independent 16x16x32 f16 MFMAs (16384 flops each) on operands held in
 * registers. The sustained MFMA ceiling the prefill GEMM is measured against (bench.py). */
int sq_diag_mfma_peak(void *graph, sq_buffer sink, uint32_t workgroups, uint32_t waves_per_simd, uint32_t iterations);

/* ---- MoE (runtime/ops/MoE.hpp:387-423) ---- */

/* MoeRouter (MoE.hpp:22-28): Softmax weights the top_k routes by the softmax of their scores, SigmoidNormalized by
 * each one's sigmoid over the sum of theirs. */
#define SQ_MOE_ROUTER_SOFTMAX 0u
#define SQ_MOE_ROUTER_SIGMOID_NORMALIZED 1u

/* MoeShape (MoE.hpp:54-102). The reference compiles two routings, (Softmax, 1 shared slice, gated) and
 * (SigmoidNormalized, 2 shared slices, ungated) (kCompiledMoeRoutings, MoE.hpp:34-46); this build also takes
 * (Softmax, no shared expert). The shared expert is shared_slices experts every row visits after its routed ones,
 * each of the routed experts' intermediate width; gated, slice weights are sigmoid(x . g) of the block's fp32
 * scalar gate g, else 1. */
typedef struct sq_moe_shape {
  uint32_t hidden_size, experts, experts_per_token, expert_intermediate_size;
  uint32_t expert_format; /* the format of most routed expert weights (each projection runs in its own) */
  uint32_t router;        /* SQ_MOE_ROUTER_* */
  uint32_t shared_slices; /* 0, 1 or 2 */
  uint32_t shared_gated;  /* 1: slice weights sigmoid(x . g); 0: 1 */
} sq_moe_shape;
typedef struct sq_moe_workspace {
  uint64_t selected_experts, routing_weights, tile_descriptors, tile_count, grouped_routes, route_rows,
      grouped_input, expert_intermediate, expert_output;
} sq_moe_workspace;
/* MoeExpertTile (MoE.hpp:284): the rows of an expert tile. */
#define SQ_MOE_EXPERT_TILE_M8 8u
#define SQ_MOE_EXPERT_TILE_M32 32u
/* MoeGgufTile (MoE.hpp:297): Staged runs here; Register is the reference's Apple9 tile, which a plan refuses. */
#define SQ_MOE_GGUF_TILE_STAGED 0u
#define SQ_MOE_GGUF_TILE_REGISTER 1u
/* FloatTile (Linear.hpp:29-33): a float projection's tile (the MoE router's among them). On MI355X SIMDGROUP runs
 * the lane chains (a wave of four rows by four columns, K over the lanes) and NEURAL_ACCELERATOR the matrix-core tile
 * (fp32 16x16x4 MFMA, 32 rows by 32 columns a workgroup, K a multiple of 256); their results lie within one fp32
 * bound. */
#define SQ_FLOAT_TILE_SIMDGROUP 0u
#define SQ_FLOAT_TILE_NEURAL_ACCELERATOR 1u
/* MoeConfig (MoE.hpp:333-346): the device's policy for a MoE plan. cpu_bf16_experts opts the reference's streamed
 * CPU experts in; its experts here are never streamed, so the flag selects nothing, as the reference's MoE::add
 * takes the GPU route for weights that are not streamed (MoE.cpp:225-245). */
typedef struct sq_moe_config {
  uint32_t expert_tile; /* SQ_MOE_EXPERT_TILE_* */
  uint32_t gguf_tile;   /* SQ_MOE_GGUF_TILE_* */
  uint32_t router_tile; /* SQ_FLOAT_TILE_* */
  uint32_t cpu_bf16_experts;
} sq_moe_config;
typedef struct sq_moe_plan {
  sq_moe_shape shape;
  uint32_t rows, phase, tile_rows, maximum_tiles;
  sq_moe_config config;
  sq_moe_workspace workspace;
} sq_moe_plan;
/* BlockExpertProjection (MoE.hpp:111-148). routed: `slots` experts' planes in one segment of slots * N rows.
 * shared: the shared slices' planes in their order, slice s's rows s * N on (a shared down of shared_slices * I
 * inputs laid out as shared_slices column windows of I inputs, window s rows s * H on). Each of the six segments
 * has a format of its own (MoE.cpp:27-62): a gate and up of different formats run as a gate pass and an up pass
 * whose epilogue reads the gate's bf16 output from expert_output (MoE.cpp:154-173), the same bits as one pass.
 * shared_scalar_gate: the block's fp32 gate [hidden] for a gated shared expert. The shared views are ignored
 * without shared slices. */
typedef struct sq_moe_weights {
  sq_segment gate, up, down;
  sq_buffer slot_table; /* uint32 per expert: its slot */
  uint32_t slots;
  sq_segment shared_gate, shared_up, shared_down;
  sq_buffer shared_scalar_gate;
  /* BlockMoeWeights::router (MoE.hpp:133): F32 (SQ_FLOAT32_ROWS) or BF16 rows [experts][hidden] in plane0. The
   * routing projects the input onto it into the router scores (MoE::addRoutes, MoE.cpp:527-543). With plane0 NULL
   * the routing reads scores the caller wrote (below). */
  sq_segment router;
} sq_moe_weights;
/* MoeScratch (MoE.hpp:225-245), sized by the plan's workspace. As in the reference, the router's fp32 scores live in
 * grouped_input, a row of the shape's router width (256 expert slots, or 512 past 256 experts:
 * sq_moe_router_width) per row; a block without router rows takes the caller's scores from there. As the reference's
 * gather does, the routed work (sq_moe_add_routed) then overwrites them, with the block's input rows in the expert
 * tiles' read order; the gate/up pass reads those through the grouped routes. Every buffer here, and the block's
 * input, output and residual, is 16-byte aligned. */
typedef struct sq_moe_scratch {
  sq_buffer selected_experts, routing_weights, tile_descriptors, tile_count, grouped_routes, route_rows,
      grouped_input, expert_intermediate, expert_output;
} sq_moe_scratch;
/* MoeBuffers (MoE.hpp:375-385). residual may be a NULL view (zeros). verify_rows: a verify step's live rows per lane
 * of 8 rows, a uint32 per lane (ceil(rows / 8) of them); routed routes of rows past their lane's count are grouped
 * into no tile, their route_rows are ~0u and the combine adds nothing for them, so such a row's output is its
 * residual plus its shared slices' routes (moe_group_routes_verified, moe.metal:164-173,196-236, 496). A NULL view:
 * every row routes. Decode plans only. */
typedef struct sq_moe_buffers {
  sq_buffer input, residual, output;
  sq_moe_scratch scratch;
  sq_buffer verify_rows;
} sq_moe_buffers;

/* The policy a plan takes when its config is NULL (ExecutionPlans::moeConfig, ExecutionPlans.cpp:56-65): Staged tiles,
 * 8-row tiles in decode and, in prefill, 8-row tiles while rows * top_k <= experts, else 32 (moeGgufPrefillTile,
 * MoE.hpp:321-330). phase is SQ_PHASE_*. */
int sq_moe_config_for(const sq_moe_shape *shape, uint32_t rows, uint32_t phase, sq_moe_config *out);
/* MoE::prefillPlan(shape, rows, config) (MoE.cpp:561-565): rows 1..2048. config NULL takes sq_moe_config_for's. */
int sq_moe_prefill_plan(const sq_moe_shape *shape, uint32_t rows, const sq_moe_config *config, sq_moe_plan *out);
/* MoE::decodePlan(shape, lanes, config) (MoE.cpp:567-571): lanes 1..4 of 8 rows each, 8-row tiles. */
int sq_moe_decode_plan(const sq_moe_shape *shape, uint32_t lanes, const sq_moe_config *config, sq_moe_plan *out);
/* No counterpart in the reference: a decode plan of any 1..32 rows (the reference's decode rows are lanes * 8). */
int sq_moe_decode_rows_plan(const sq_moe_shape *shape, uint32_t rows, sq_moe_plan *out);
/* MoeShape::routerWidth (MoE.hpp:94-96): the fp32 scores a row of the router scores holds. */
uint32_t sq_moe_router_width(const sq_moe_shape *shape);
/* MoE::add = addRouting then addRouted (MoE.cpp:225-525). */
int sq_moe_add(void *graph, const sq_moe_buffers *buffers, const sq_moe_weights *weights, const sq_moe_plan *plan);
int sq_moe_add_routing(void *graph, const sq_moe_buffers *buffers, const sq_moe_weights *weights,
                       const sq_moe_plan *plan);
int sq_moe_add_routed(void *graph, const sq_moe_buffers *buffers, const sq_moe_weights *weights,
                      const sq_moe_plan *plan);
/* MoE::addRoutes (MoE.hpp:403-411; MoE.cpp:527-543): the routing of `rows` rows (1..2048) of `input` (bf16
 * [rows][hidden]) with no plan and no grouping, into caller buffers. With router rows (router non-NULL, plane0 set:
 * F32 or BF16 [experts][hidden]) it first projects the input onto them into `scores` on router_tile (SQ_FLOAT_TILE_*);
 * otherwise it reads the fp32 scores the caller wrote there. scores: rows of sq_moe_router_width(shape) fp32 slots;
 * selected (uint32) and routing_weights (fp32): experts_per_token + shared_slices per row, the top-k experts then
 * the shared slices, as sq_moe_add_routing writes them. shared_scalar_gate (fp32 [hidden]) is read only for a gated
 * shared expert. input, scores and shared_scalar_gate are 16-byte aligned. */
int sq_moe_add_routes(void *graph, sq_buffer input, const sq_segment *router, sq_buffer shared_scalar_gate,
                      sq_buffer scores, sq_buffer selected, sq_buffer routing_weights, uint32_t rows,
                      const sq_moe_shape *shape, uint32_t router_tile);
/* MoE::addExpertLoad (MoE.hpp:411-420, MoE.cpp:553-558; kernel moe_expert_load, gguf_repack.metal:239-257): the
 * gate, up and down projections of up to `jobs` streamed experts repacked into their slots of `arena`. Job j's
 * projection z takes its native rows (row_bytes apart) from staging + sources[3 j + z] (bytes) on, and writes them
 * as sq_gguf_repack does into plane i of slot slots[j]: arena + planes[i] + slots[j] * slot_bytes[i] (plane0, plane1,
 * meta). params is the reference's 192-byte MoeExpertLoadParams: three 64-byte MoeExpertLoadProjection
 * {format, rows, columns, row_bytes, planes[3], slot_bytes[3]} (rows 0: no projection). slots: jobs uint32; sources:
 * 3 jobs uint64 (8-byte aligned); grid: three uint32 workgroup counts (x, y, z) that an earlier dispatch may write,
 * the reference's indirect grid. The launch covers (sq_moe_expert_load_groups(params), jobs, 3) workgroups of 256
 * threads, and those past grid's counts do nothing. A job whose rows or slot planes would lie outside staging or
 * arena writes nothing. */
typedef struct sq_moe_expert_load_projection {
  uint32_t format_id, rows, columns, row_bytes;
  uint64_t planes[3];     /* plane0, plane1, meta: byte offsets in the arena */
  uint64_t slot_bytes[3]; /* bytes a slot in each */
} sq_moe_expert_load_projection;
typedef struct sq_moe_expert_load_params {
  sq_moe_expert_load_projection projections[3]; /* gate, up, down */
} sq_moe_expert_load_params;
int sq_moe_expert_load(void *graph, sq_buffer staging, sq_buffer arena, sq_buffer slots, sq_buffer sources,
                       const sq_moe_expert_load_params *params, uint32_t jobs, sq_buffer grid);
/* MoE::expertLoadGroups (MoE.cpp:545-551): the workgroups that repack one job's largest projection (0 without
 * params). */
uint32_t sq_moe_expert_load_groups(const sq_moe_expert_load_params *params);

#ifdef __cplusplus
}
#endif
#endif
