// Host-only use of the C++ face (include/splash_q4.hpp): plans, scratch sizes and the reference's exceptions.
// Nothing here touches a GPU. Built and run by tests/test_capi.py.
#include <cstdio>
#include <stdexcept>

#include "splash_q4.hpp"

using namespace splash_q4::ops;

int main() {
  const Linear linear({256});
  Projection p{};
  p.output_size = 14336;
  p.input_size = 4096;
  p.segment_count = 1;
  p.destination = SQ_OUTPUT_BF16;
  p.segments[0].output_size = 14336;
  p.segments[0].input_size = 4096;
  p.segments[0].format_id = SQ_FMT_AF4G64;
  p.segments[0].plane0.bytes = 14336ull * 4096 / 2;
  p.segments[0].meta.bytes = 14336ull * 4096 / 64 * 4;
  const LinearPlan decode = linear.decodePlan(p, 1);
  const LinearPlan prefill = linear.prefillPlan(p, 2048, LinearEpilogue::None);
  const LinearScratchSize s = linear.decodeScratchSize({14336, 4096});
  std::printf("decode rows %u tile %u splits %u; prefill tile %u; decode partials %llu\n", decode.storage_rows,
              decode.config.tile, decode.config.splits, prefill.config.tile, (unsigned long long)s.partials);
  std::printf("storage rows %u; float tile %u at 2048 rows, %u at 8\n", linear.decodeStorageRows(8, {14336, 4096}),
              linear.ggufFloatTile(2048, 256, SQ_FLOAT32_ROWS), linear.ggufFloatTile(8, 256, SQ_FLOAT32_ROWS));
  const MoeShape shape{2048, 128, 8, 768, SQ_FMT_AF4G64, SQ_MOE_ROUTER_SOFTMAX, 0, 0};
  const MoePlan moe = MoE::decodePlan(shape, 2, MoE::config(shape, 16, SQ_PHASE_DECODE));
  const MoePlan moePrefill = MoE::prefillPlan(shape, 512, MoE::config(shape, 512, SQ_PHASE_PREFILL));
  std::printf("moe decode rows %u tile %u; moe prefill tile %u\n", moe.rows, moe.tile_rows, moePrefill.tile_rows);
  sq_moe_expert_load_params load{};
  load.projections[0] = {SQ_FMT_Q4K, 128, 512, 288, {0, 0, 0}, {1u << 20, 0, 1u << 20}};
  load.projections[2] = {SQ_FMT_Q6K, 256, 256, 210, {0, 0, 0}, {1u << 20, 1u << 20, 1u << 20}};
  std::printf("expert load groups %u\n", MoE::expertLoadGroups(load));
  try {
    (void)linear.decodePlan(p, 0);
    std::printf("no exception\n");
    return 1;
  } catch (const std::invalid_argument &e) {
    std::printf("invalid_argument: %s\n", e.what());
  }
  return 0;
}
