/*
 * CPU oracle for the 4-bit quantized matmul path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's semantics for the formats, the load-time repack, the dequantised
 * values, the fp64 projection and its error bound, and the MoE routing/grouping/combine. Only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it, and only as the checker or the
 * reported CPU baseline: the product path never calls it.
 *
 * Reference files followed (paths under the reference checkout):
 *   runtime/metal/abi/QuantFormat.h:147-294          format rows, quant_slot, quant_tile_index
 *   runtime/metal/kernels/shared/gguf_repack.metal:24-74   repack of af4 and Q4_K groups
 *   dev/tests/engine/GgufFormatReference.hpp:217-380  mlxNative, groupPack (values), metaPack, repack
 *   dev/tests/engine/GgufFormatReference.hpp:758-797  Dot and projectionBound
 *   runtime/metal/kernels/common/gguf_staged.h:11-16  staged fp16 value = fp16(fma(q, s, z))
 *   runtime/metal/kernels/common/quant_formats.h:105-118,591-617  Q4_K and affine coefficients
 *   runtime/metal/kernels/shared/moe.metal:23-112,175-278,480-505  route select, grouping, combine
 *   dev/tests/engine/GgufFixtures.hpp:148-165        the Q4_K golden fixture (mt19937 draws)
 */
#ifndef SQ_ORACLE_H
#define SQ_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Format ids of the reference's kQuantFormats table (QuantFormat.h:83-133). */
#define SQO_FMT_Q4K 0u
#define SQO_FMT_Q5K 3u
#define SQO_FMT_Q6K 4u
#define SQO_FMT_Q80 6u
#define SQO_FMT_AF4G32 25u
#define SQO_FMT_AF4G64 26u
#define SQO_FMT_AF4G128 27u
#define SQO_FMT_AF8G64 35u

typedef struct {
  uint32_t ggml_type, block_elements, block_bytes, plane0_bytes, plane1_bytes, meta_bytes, meta_groups;
} sqo_format;

/* 0 on success, -1 for a format the oracle does not restate. */
int sqo_format_info(uint32_t fmt, sqo_format *out);
uint32_t sqo_quant_slot(uint32_t e);
uint64_t sqo_tile_index(uint32_t row, uint32_t block, uint32_t blocks);

/* IEEE conversions (round to nearest even). */
uint16_t sqo_f32_to_f16(float f);
float sqo_f16_to_f32(uint16_t h);
uint16_t sqo_f32_to_bf16(float f);
float sqo_bf16_to_f32(uint16_t b);

/* MLX tensors of an affine format -> the loader's native rows {bf16 s, bf16 z, codes} per group. */
int sqo_mlx_native(uint32_t fmt, uint32_t rows, uint32_t K, const uint8_t *weight, const uint16_t *scales,
                   const uint16_t *biases, uint8_t *native);
/* Native rows -> plane0, plane1 (NULL for a format without one) and meta (layout of QuantFormat.h:3-9); values
 * (fp32, [N][K]) may be NULL. */
int sqo_repack(uint32_t fmt, const uint8_t *native, uint32_t N, uint32_t K, uint8_t *plane0, uint8_t *plane1,
               uint8_t *meta, float *values);
/* Inverse of sqo_repack (for the round-trip invariant). */
int sqo_unpack(uint32_t fmt, const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, uint32_t N,
               uint32_t K, uint8_t *native);
/* The fp32 values and the staged tile's fp16 bits of every weight of the planes ([N][K] each, either may be NULL). */
int sqo_plane_values(uint32_t fmt, const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, uint32_t N,
                     uint32_t K, float *values, uint16_t *halves);
/* The reference test fixture: native rows of random bytes, mt19937(seed), finite random half scales. */
int sqo_fixture(uint32_t fmt, uint32_t rows, uint32_t K, uint32_t seed, uint8_t *native);

/* fp64 projection y[m][n] = sum_k x[m][k] w[n][k] over bf16 x and fp32 weights, with the magnitudes of the
 * reference's Dot (value, sum |x w|, sum |x|, max |w|). Any output pointer but value may be NULL. */
void sqo_project_f64(uint32_t M, uint32_t N, uint32_t K, const uint16_t *x, const float *w, double *value,
                     double *magnitude, double *inputs, double *largest, int threads);
/* projectionBound (GgufFormatReference.hpp:794-797). */
double sqo_projection_bound(double magnitude, double inputs, double largest, int staged);
/* The reference's staged numerics on the CPU: fp16-rounded weights, exact products, sequential fp32 sums in K order.
 * out is fp32 [M][N]. */
void sqo_project_staged_f32(uint32_t M, uint32_t N, uint32_t K, const uint16_t *x, const uint16_t *halves,
                            float *out, int threads);

/* CPU baseline: the same quantized matmul as the GPU path (planes in, fma(q, s, z) in fp32, fp32 accumulation,
 * bf16 out), threaded over output columns. Returns seconds taken. */
double sqo_cpu_matmul(uint32_t fmt, uint32_t M, uint32_t N, uint32_t K, const uint16_t *x, const uint8_t *plane0,
                      const uint8_t *meta, uint16_t *out, int threads);

/* MoE (moe.metal): top-k of fp32 scores [rows][experts] (descending, ties to the lower id) with their weights
 * (router 0: renormalised softmax; 1: sigmoids over their sum), fp64 here, into rows of per_row routes. */
void sqo_route_select(uint32_t rows, uint32_t experts, uint32_t top_k, uint32_t router, uint32_t per_row,
                      const float *scores, uint32_t *selected, double *weights);
/* Grouping into tiles of tile_rows rows: routed routes by expert (stable in route order), then `shared` slices'
 * tiles of every row; returns the tile count. tiles: 2 uint32 per tile (expert, live rows); grouped_routes
 * [tiles * tile_rows] (~0u padding); route_rows [rows * (top_k + shared)]. */
uint32_t sqo_group_routes(uint32_t rows, uint32_t top_k, uint32_t shared, uint32_t experts, uint32_t tile_rows,
                          const uint32_t *selected, const uint32_t *verify_rows, uint32_t lane_rows, uint32_t *tiles,
                          uint32_t *grouped_routes, uint32_t *route_rows);

#ifdef __cplusplus
}
#endif
#endif
