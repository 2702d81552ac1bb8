// Byte-level contract shared by the host planner, the C-ABI and the HIP kernels: the quantized-plane geometry and
// the kernel parameter blocks, with the field layouts and sizes the reference's engine uses, so that a caller built
// against the reference's structs hands the same bytes over.
//
// Reference interfaces restated here (paths under the reference checkout):
//   runtime/metal/abi/QuantFormat.h:83-133,147-156,185-187,254-294   format ids, format rows, slots, tile index
//   runtime/metal/abi/Gguf.h:13-106                                   tile geometry and parameter structs
//   runtime/metal/abi/GgufRepack.h:10-18                              repack parameters
//   runtime/metal/abi/MoE.h:19-181                                    MoE parameter structs
//   runtime/metal/abi/ExecutionGeometry.h:7-17                        batch and prefill geometry
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP_DEVICE_COMPILE__)
#define SQ_HD __host__ __device__
#else
#define SQ_HD
#endif

// ---------------------------------------------------------------- format ids (QuantFormat.h:83-133)
// The ids keep the reference's numbering, so a caller's format ids mean the same formats here.
#define SQ_FMT_Q4K 0u
#define SQ_FMT_Q5K 3u
#define SQ_FMT_Q6K 4u
#define SQ_FMT_Q80 6u
#define SQ_FMT_AF4G32 25u
#define SQ_FMT_AF4G64 26u
#define SQ_FMT_AF4G128 27u
#define SQ_FMT_AF8G64 35u
#define SQ_FMT_BF16 41u   // as float rows only (QuantizedSegment::rows)
#define SQ_FMT_COUNT 48u
// QuantizedSegment::kFloat32 (Weights.hpp:81): the format id of F32 rows, which no format row names.
#define SQ_FLOAT32_ROWS 0xFFFFFFFFu
// LinearInput (Linear.hpp:166-169) and this build's prefill table (the prefill tile's prepared input).
#define SQ_LINEAR_INPUT_PLAIN 0u
#define SQ_LINEAR_INPUT_TABLE16 1u
#define SQ_LINEAR_INPUT_HALF_ROWS 2u

// A format row (QuantFormat.h:147-156): the bytes of a native block and of the planes' units.
struct SqQuantFormat {
  uint32_t ggml_type;      // GGUF tensor type, or the MLX affine tag 0x4D4C0000 | bits << 8 | group
  uint32_t block_elements; // elements per native block
  uint32_t block_bytes;    // bytes per native block
  uint32_t plane0_bytes;   // per row and group of 32
  uint32_t plane1_bytes;   // per row and group of 32
  uint32_t meta_bytes;     // per row and meta unit
  uint32_t meta_groups;    // groups of 32 per meta unit
};

// The formats this build runs: Q4_K, Q5_K, Q6_K and Q8_0 (QuantFormat.h:159,162,163,165), the 4-bit MLX affine
// ones (QuantFormat.h:185-187) and af8g64 (QuantFormat.h:192). Every other id is a format of the reference this
// build does not take; the host rejects it before any launch.
SQ_HD inline bool sq_format_supported(uint32_t f) {
  return f == SQ_FMT_Q4K || f == SQ_FMT_Q5K || f == SQ_FMT_Q6K || f == SQ_FMT_Q80 || f == SQ_FMT_AF4G32 ||
         f == SQ_FMT_AF4G64 || f == SQ_FMT_AF4G128 || f == SQ_FMT_AF8G64;
}
SQ_HD inline SqQuantFormat sq_format(uint32_t f) {
  switch (f) {
    case SQ_FMT_Q4K: return {12u, 256u, 144u, 16u, 0u, 16u, 8u};
    case SQ_FMT_Q5K: return {13u, 256u, 176u, 16u, 4u, 16u, 8u};
    case SQ_FMT_Q6K: return {14u, 256u, 210u, 16u, 8u, 20u, 8u};
    case SQ_FMT_Q80: return {8u, 32u, 34u, 32u, 0u, 2u, 1u};
    case SQ_FMT_AF4G32: return {0x4D4C0000u | (4u << 8) | 32u, 32u, 20u, 16u, 0u, 4u, 1u};
    case SQ_FMT_AF4G64: return {0x4D4C0000u | (4u << 8) | 64u, 64u, 36u, 16u, 0u, 4u, 2u};
    case SQ_FMT_AF4G128: return {0x4D4C0000u | (4u << 8) | 128u, 128u, 68u, 16u, 0u, 4u, 4u};
    case SQ_FMT_AF8G64: return {0x4D4C0000u | (8u << 8) | 64u, 64u, 68u, 32u, 0u, 4u, 2u};
    default: return {0u, 0u, 0u, 0u, 0u, 0u, 0u};
  }
}
SQ_HD inline const char *sq_format_name(uint32_t f) {
  switch (f) {
    case SQ_FMT_Q4K: return "q4k";
    case SQ_FMT_Q5K: return "q5k";
    case SQ_FMT_Q6K: return "q6k";
    case SQ_FMT_Q80: return "q80";
    case SQ_FMT_AF4G32: return "af4g32";
    case SQ_FMT_AF4G64: return "af4g64";
    case SQ_FMT_AF4G128: return "af4g128";
    case SQ_FMT_AF8G64: return "af8g64";
    default: return "unsupported";
  }
}
SQ_HD inline bool sq_affine_format(uint32_t f) { return (f >= SQ_FMT_AF4G32 && f <= SQ_FMT_AF4G128) || f == SQ_FMT_AF8G64; }
// Byte offsets in block_q6_K (llama.cpp: ql[128], qh[64], int8 scales[16], half d).
#define SQ_Q6K_SCALES 192u
#define SQ_Q6K_D 208u

// Element e (0..31) of a group sits at slot 8c + 2p + (e & 1): chunk c = (e >> 2) & 3, pair p = 2 (e >> 4) +
// ((e >> 1) & 1) (QuantFormat.h:18-26,254). Word c of a 4-bit plane unit holds slots 8c..8c+7, pair p's first
// element at bits 4p and its second at bits 16 + 4p.
SQ_HD inline uint32_t sq_quant_slot(uint32_t e) { return 8u * ((e >> 2) & 3u) + 4u * (e >> 4) + (e & 3u); }

// Planes hold rows in tiles of 64 (QuantFormat.h:258); (row, block) of a [rows/64][blocks][64] plane
// (QuantFormat.h:292-294).
#define SQ_TILE_ROWS 64u
SQ_HD inline uint64_t sq_tile_index(uint32_t row, uint32_t block, uint32_t blocks) {
  return ((uint64_t)(row / SQ_TILE_ROWS) * blocks + block) * SQ_TILE_ROWS + row % SQ_TILE_ROWS;
}

// ---------------------------------------------------------------- geometry (ExecutionGeometry.h, Gguf.h)
#define SQ_TARGET_VERIFY_ROWS 8u        // rows of one decode lane
#define SQ_MAXIMUM_BATCH_WIDTH 4u       // decode lanes
#define SQ_PREFILL_TOKEN_BUDGET 2048u   // rows of a prefill chunk
#define SQ_TILE_COLUMNS 64u             // output columns of a column tile (Gguf.h:13)
#define SQ_MAXIMUM_DECODE_ROWS (SQ_TARGET_VERIFY_ROWS * SQ_MAXIMUM_BATCH_WIDTH)
#define SQ_MAXIMUM_SPLITS 16u           // LinearConfig::kMaximumSplits (Linear.hpp:106)

// ---------------------------------------------------------------- kernel parameter blocks (Gguf.h:55-106)
struct SqGgufPrefillParams {
  uint32_t input_size;  // K
  uint32_t rows;        // rows of the chunk
  uint32_t out_stride;  // columns of a destination row
  uint32_t out_offset;  // first destination column of this segment
};
static_assert(sizeof(SqGgufPrefillParams) == 16, "GgufPrefillParams is 16 bytes");

struct SqGgufPrefillSegmentsParams {
  uint32_t input_size;
  uint32_t rows;
  uint32_t out_stride;
  uint32_t cols[3];     // columns per segment; 0 past the last
  uint32_t offset[3];   // first destination column per segment
};
static_assert(sizeof(SqGgufPrefillSegmentsParams) == 36, "GgufPrefillSegmentsParams is 36 bytes");

struct SqGgufDecodeParams {
  uint32_t input_size;  // K
  uint32_t splits;      // K partitions; 1 = no cross-workgroup reduction
  uint32_t out_stride;  // columns of a destination row
  uint32_t out_offset;  // first destination column of the tensor
  uint32_t spread;      // accepted for the reference's layout; the kernels here walk K in order
};
static_assert(sizeof(SqGgufDecodeParams) == 20, "GgufDecodeParams is 20 bytes");

struct SqGgufDecodeFusedParams {
  uint32_t input_size;
  uint32_t splits;
  uint32_t out_stride;
  uint32_t cols[3];
  uint32_t fmt[3];
  uint32_t offset[3];
  uint32_t spread;
};
static_assert(sizeof(SqGgufDecodeFusedParams) == 52, "GgufDecodeFusedParams is 52 bytes");

// GgufRepack.h:10-18: a chunk of native rows into one buffer, plane0 at 0, then plane1 and meta.
struct SqGgufRepackParams {
  uint32_t rows;          // rows of the chunk (a multiple of 64)
  uint32_t input_size;    // K of the chunk
  uint32_t fmt;           // format id
  uint32_t src_row_bytes; // bytes per staged row
  uint32_t dst_plane1;    // byte offsets in the output buffer
  uint32_t dst_meta;
};
static_assert(sizeof(SqGgufRepackParams) == 24, "GgufRepackParams is 24 bytes");

// ---------------------------------------------------------------- MoE (MoE.h:19-181)
// ops::MoeRouter (MoE.hpp:22-28): how the top_k routes are weighted.
#define SQ_MOE_ROUTER_SOFTMAX 0u
#define SQ_MOE_ROUTER_SIGMOID_NORMALIZED 1u
#define SQ_MOE_EXPERT_SLOTS 256u
#define SQ_MOE_WIDE_EXPERT_SLOTS 512u
struct SqMoeRouteParams {
  uint32_t rows, input_size, experts, top_k;
};
static_assert(sizeof(SqMoeRouteParams) == 16, "MoeRouteParams is 16 bytes");
struct SqMoeTileDescriptor {
  uint32_t expert, rows;
};
static_assert(sizeof(SqMoeTileDescriptor) == 8, "MoeTileDescriptor is 8 bytes");
struct SqMoeGroupParams {
  uint32_t rows, top_k, tile_rows, experts, gate_up_columns, down_columns, lane_rows, rotation_columns;
};
static_assert(sizeof(SqMoeGroupParams) == 32, "MoeGroupParams is 32 bytes");
struct SqMoeTileCount {
  uint32_t tiles;
  uint32_t gate_up_grid[3];
  uint32_t down_grid[3];
  uint32_t routed_grid[3];
};
static_assert(sizeof(SqMoeTileCount) == 40, "MoeTileCount is 40 bytes");
struct SqMoeGatherParams {
  uint32_t tile_rows, input_size, routes_per_row;
};
static_assert(sizeof(SqMoeGatherParams) == 12, "MoeGatherParams is 12 bytes");
struct SqMoeGgufExpertParams {
  uint32_t input_size, output_size, experts, routed_format, shared_format;
};
static_assert(sizeof(SqMoeGgufExpertParams) == 20, "MoeGgufExpertParams is 20 bytes");
struct SqMoeGgufGateUpParams {
  uint32_t input_size, output_size, experts, gate_routed_format, gate_shared_format, up_routed_format,
      up_shared_format;
};
static_assert(sizeof(SqMoeGgufGateUpParams) == 28, "MoeGgufGateUpParams is 28 bytes");
struct SqMoeCombineParams {
  uint32_t rows, hidden_size, routes_per_row;
};
static_assert(sizeof(SqMoeCombineParams) == 12, "MoeCombineParams is 12 bytes");
// One projection (gate, up or down) of the experts a load writes into their slots (MoE.h:146-168): rows x columns
// in `format`, job j's native rows of row_bytes each staged from its source on, and its plane0, plane1 and meta
// planes in the arena from planes[i] on, slot_bytes[i] bytes a slot.
struct SqMoeExpertLoadProjection {
  uint32_t format, rows, columns, row_bytes;
  uint64_t planes[3];
  uint64_t slot_bytes[3];
};
static_assert(sizeof(SqMoeExpertLoadProjection) == 64, "MoeExpertLoadProjection is 64 bytes");
struct SqMoeExpertLoadParams {
  struct SqMoeExpertLoadProjection projections[3];
};
static_assert(sizeof(SqMoeExpertLoadParams) == 192, "MoeExpertLoadParams is 192 bytes");
// The threads of a moe_expert_load workgroup, each of which repacks one (row, 32-wide K group) pair (MoE.h:170-172).
#define SQ_MOE_EXPERT_LOAD_THREADS 256u
