/* CPU baseline of the quantized matmul (measurement and test infrastructure; not the product): a persistent thread
 * pool running y = x W^T over plane weights with the reference's dequantisation, fp32 sums and a bf16 output. */
#ifndef SQ_CPU_H
#define SQ_CPU_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sqo_pool sqo_pool;
/* The instruction set the kernels run: "avx512bf16", "avx512f", "avx2+fma" or "scalar" (the best the CPU has). */
const char *sqo_cpu_isa(void);
/* A pool of `threads` threads (the caller's thread is one of them), started once. */
sqo_pool *sqo_pool_create(int threads);
void sqo_pool_destroy(sqo_pool *pool);
int sqo_pool_threads(const sqo_pool *pool);
const char *sqo_pool_isa(const sqo_pool *pool);
/* Runs the pool's later calls on the kernel named isa (one of sqo_cpu_isa's names); -1 when the CPU lacks it. */
int sqo_pool_set_isa(sqo_pool *pool, const char *isa);
/* Holds the permuted-input buffer for M x K (allocation outside any timed call); 0 on success. */
int sqo_pool_reserve(sqo_pool *pool, uint32_t M, uint32_t K);
/* y = x W^T for x bf16 [M][K] and W in format fmt (MLX affine 4-bit groups 32/64/128, or Q4_K) as planes
 * (plane0, meta), out bf16 [M][N]. Returns the call's wall seconds, or a negative value for a format or shape it
 * does not take (N % 64, K % 256) or an M x K past the reserved buffer. */
double sqo_pool_matmul(sqo_pool *pool, uint32_t fmt, uint32_t M, uint32_t N, uint32_t K, const uint16_t *x,
                       const uint8_t *plane0, const uint8_t *meta, uint16_t *out);

#ifdef __cplusplus
}
#endif
#endif
