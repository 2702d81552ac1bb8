/* CPU baseline of the quantized matmul (test and measurement infrastructure, not the product): y = x W^T for bf16
 * activations x [M][K] and plane weights W [N][K] in MLX affine 4-bit (groups of 32, 64, 128) or GGUF Q4_K, with the
 * reference's semantics: every weight dequantised in fp32 as fma(q, s, z) (GgufFormatReference.hpp:369-380,
 * quant_formats.h:591-617), products and sums in fp32, the output rounded once to bf16. Only bench.py's cpu_baseline
 * and tests/ load it.
 *
 * Layout of the work. A persistent pool of threads (created once, outside any timed call) splits the 64-column plane
 * tiles of W among its threads. A thread walks its tiles column by column; for each group of 32 inputs it loads the
 * column's 16 code bytes, widens them to 32 fp32 codes (low and high nibbles), dequantises them with two vector FMAs
 * and multiply-adds them into one vector accumulator per row, against the rows' inputs permuted once per call into
 * the codes' byte order. Rows go in blocks of eight, so each dequantised group serves eight rows. AVX-512F, AVX2+FMA
 * or scalar code is chosen at run time from what the CPU reports.
 *
 * Where the CPU reports AVX512_BF16 the pool runs the bf16 dot-product kernel instead (columns_bf16): the group's 32
 * codes become bf16 q (exact) and VDPBF16PS multiplies them with the rows' bf16 inputs (exact products, fp32 sums),
 * one scale group at a time; the close is acc += s * sum(q x) per scale group on the vector and z * sum(x) per row in
 * scalar. These are the exact-operand numerics of the GPU's decode tiles, within the same accumulation bound. The
 * instruction treats bf16 subnormal inputs as zero. sqo_pool_set_isa picks another kernel the CPU has. */
#define _GNU_SOURCE
#include "sq_cpu.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "sq_oracle.h"

enum { kRowBlock = 8, kMaxThreads = 256 };

/* The input index of the low (h = 0) and high (h = 1) nibble of code byte b of a group (quant_slot,
 * QuantFormat.h:254: slot pair p of word w at bits 4p and 16 + 4p). */
static uint8_t g_element[16][2];
static void init_elements(void) {
  for (uint32_t e = 0; e < 32; ++e) {
    const uint32_t s = sqo_quant_slot(e), word = s / 8, j = s % 8, p = j / 2;
    const uint32_t bit = (j & 1) ? 16 + 4 * p : 4 * p;
    g_element[4 * word + bit / 8][(bit % 8) / 4] = (uint8_t)e;
  }
}

typedef struct {
  uint32_t fmt, M, N, K, G, units, meta_groups, meta_bytes;
  const float *xp; /* [M][G][2][16]: row m's inputs of group g, low-nibble order then high-nibble order */
  const uint16_t *xb; /* the same inputs as bf16 (the bf16 kernel) */
  const float *sx;    /* [M][G / sg]: the sum of row m's inputs over scale group u (the bf16 kernel) */
  const uint8_t *plane0, *meta;
  uint16_t *out;
} job_t;

struct sqo_pool {
  int threads;
  pthread_t tid[kMaxThreads];
  pthread_mutex_t mu;
  pthread_cond_t go, done;
  uint64_t generation;
  int remaining, quit;
  job_t job;
  float *xp, *sx;
  uint16_t *xb;
  size_t xp_floats;
  int kind; /* 3 AVX512_BF16, 2 AVX-512F, 1 AVX2+FMA, 0 scalar */
};

static inline float bf16f(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE half to float, exact (subnormals scaled in, infinities and NaNs kept). */
static inline float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t u;
  if (e == 31) u = sign | 0x7F800000u | (m << 13);
  else if (e) u = sign | ((e + 112u) << 23) | (m << 13);
  else {
    float f = (float)m * 0x1p-24f;
    memcpy(&u, &f, 4);
    u |= sign;
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Column n's code bytes and meta, group by group: plane0 [N/64][G][64][16 B] (group g of column n at plane + 1024 g),
 * meta [N/64][units][64][meta_bytes] (unit u at meta + 64 meta_bytes u). */
typedef struct {
  const uint8_t *plane, *meta;
} column_t;
static inline column_t column_at(const job_t *j, uint32_t n) {
  const size_t tile = n / 64, lane = n % 64;
  return (column_t){j->plane0 + (tile * j->G * 64 + lane) * 16, j->meta + (tile * j->units * 64 + lane) * j->meta_bytes};
}

/* fp32 (s, z) of group g of a column. */
static inline void group_coef(const job_t *j, column_t c, uint32_t g, float *s, float *z) {
  const uint8_t *m = c.meta + (size_t)(g / j->meta_groups) * 64 * j->meta_bytes;
  if (j->fmt != SQO_FMT_Q4K) {
    uint16_t sb, zb;
    memcpy(&sb, m, 2);
    memcpy(&zb, m + 2, 2);
    *s = bf16f(sb);
    *z = bf16f(zb);
    return;
  }
  /* Q4_K: s = d sc, m = -dmin mn from the 6-bit fields of sub-block g % 8 (get_scale_min_k4). */
  uint16_t d16, m16;
  memcpy(&d16, m, 2);
  memcpy(&m16, m + 2, 2);
  const uint8_t *q = m + 4;
  const uint32_t b = g % 8;
  uint32_t sc, mn;
  if (b < 4) {
    sc = q[b] & 63u;
    mn = q[b + 4] & 63u;
  } else {
    sc = (q[b + 4] & 15u) | ((q[b - 4] >> 6) << 4);
    mn = (q[b + 4] >> 4) | ((q[b] >> 6) << 4);
  }
  *s = h2f(d16) * (float)sc;
  *z = -(h2f(m16) * (float)mn);
}

/* Round to nearest even (the inputs are finite sums). */
static inline uint16_t to_bf16(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__attribute__((target("avx512f"))) static float hsum512(__m512 v) { return _mm512_reduce_add_ps(v); }

__attribute__((target("avx512f"))) static void columns_avx512(const job_t *j, uint32_t n0, uint32_t n1) {
  const __m512i nib = _mm512_set1_epi32(15);
  for (uint32_t n = n0; n < n1; ++n)
    for (uint32_t r0 = 0; r0 < j->M; r0 += kRowBlock) {
      const column_t col = column_at(j, n);
      const uint32_t rows = j->M - r0 < kRowBlock ? j->M - r0 : kRowBlock;
      __m512 acc[kRowBlock];
      for (uint32_t r = 0; r < kRowBlock; ++r) acc[r] = _mm512_setzero_ps();
      for (uint32_t g = 0; g < j->G; ++g) {
        float s, z;
        group_coef(j, col, g, &s, &z);
        const __m128i c = _mm_loadu_si128((const __m128i *)(col.plane + (size_t)g * 1024));
        const __m512i b = _mm512_cvtepu8_epi32(c);
        const __m512 vs = _mm512_set1_ps(s), vz = _mm512_set1_ps(z);
        const __m512 wl = _mm512_fmadd_ps(_mm512_cvtepi32_ps(_mm512_and_si512(b, nib)), vs, vz);
        const __m512 wh = _mm512_fmadd_ps(_mm512_cvtepi32_ps(_mm512_srli_epi32(b, 4)), vs, vz);
        const float *x = j->xp + ((size_t)r0 * j->G + g) * 32;
        for (uint32_t r = 0; r < rows; ++r) {
          const float *xr = x + (size_t)r * j->G * 32;
          acc[r] = _mm512_fmadd_ps(wl, _mm512_loadu_ps(xr), acc[r]);
          acc[r] = _mm512_fmadd_ps(wh, _mm512_loadu_ps(xr + 16), acc[r]);
        }
      }
      for (uint32_t r = 0; r < rows; ++r) j->out[(size_t)(r0 + r) * j->N + n] = to_bf16(hsum512(acc[r]));
    }
}

/* The scale group's span in groups of 32: the affine formats' meta unit, Q4_K's 32-input sub-block. */
static inline uint32_t scale_groups(const job_t *j) { return j->fmt == SQO_FMT_Q4K ? 1u : j->meta_groups; }

/* Rows r0..r0 + R - 1 of column n (R a constant at each call, so the accumulators stay in registers). */
__attribute__((target("avx512f,avx512bw,avx512bf16"), always_inline)) static inline void column_bf16_rows(
    const job_t *j, __m512i table, uint32_t n, uint32_t r0, const int R) {
  const __m256i nib = _mm256_set1_epi16(15);
  const uint32_t sg = scale_groups(j);
  const column_t col = column_at(j, n);
  __m512 acc[kRowBlock];
  float zacc[kRowBlock];
  for (int r = 0; r < R; ++r) {
    acc[r] = _mm512_setzero_ps();
    zacc[r] = 0.0f;
  }
  for (uint32_t g0 = 0; g0 < j->G; g0 += sg) {
    float s, z;
    group_coef(j, col, g0, &s, &z);
    __m512 c[kRowBlock];
    for (int r = 0; r < R; ++r) c[r] = _mm512_setzero_ps();
    for (uint32_t g = g0; g < g0 + sg; ++g) {
      /* Words 0..15: the low nibbles of code bytes 0..15, words 16..31 the high ones (the inputs' order). */
      const __m256i b = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i *)(col.plane + (size_t)g * 1024)));
      const __m512i q =
          _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_and_si256(b, nib)), _mm256_srli_epi16(b, 4), 1);
      const __m512bh w = (__m512bh)_mm512_permutexvar_epi16(q, table);
      const uint16_t *x = j->xb + ((size_t)r0 * j->G + g) * 32;
      for (int r = 0; r < R; ++r)
        c[r] = _mm512_dpbf16_ps(c[r], w, (__m512bh)_mm512_loadu_si512(x + (size_t)r * j->G * 32));
    }
    const __m512 vs = _mm512_set1_ps(s);
    const uint32_t units = j->G / sg;
    const float *sx = j->sx + (size_t)r0 * units + g0 / sg;
    for (int r = 0; r < R; ++r) {
      acc[r] = _mm512_fmadd_ps(vs, c[r], acc[r]);
      zacc[r] = fmaf(z, sx[(size_t)r * units], zacc[r]);
    }
  }
  for (int r = 0; r < R; ++r) j->out[(size_t)(r0 + r) * j->N + n] = to_bf16(hsum512(acc[r]) + zacc[r]);
}

__attribute__((target("avx512f,avx512bw,avx512bf16"))) static void columns_bf16(const job_t *j, uint32_t n0,
                                                                                 uint32_t n1) {
  /* bf16 of q for q = 0..15 (twice: vpermw indexes 32 words). */
  uint16_t lut[32];
  for (int q = 0; q < 32; ++q) {
    const float f = (float)(q & 15);
    uint32_t u;
    memcpy(&u, &f, 4);
    lut[q] = (uint16_t)(u >> 16);
  }
  const __m512i table = _mm512_loadu_si512(lut);
  for (uint32_t n = n0; n < n1; ++n)
    for (uint32_t r0 = 0; r0 < j->M; r0 += kRowBlock) {
      switch (j->M - r0 < kRowBlock ? j->M - r0 : kRowBlock) {
        case 1: column_bf16_rows(j, table, n, r0, 1); break;
        case 2: column_bf16_rows(j, table, n, r0, 2); break;
        case 3: column_bf16_rows(j, table, n, r0, 3); break;
        case 4: column_bf16_rows(j, table, n, r0, 4); break;
        case 5: column_bf16_rows(j, table, n, r0, 5); break;
        case 6: column_bf16_rows(j, table, n, r0, 6); break;
        case 7: column_bf16_rows(j, table, n, r0, 7); break;
        default: column_bf16_rows(j, table, n, r0, 8); break;
      }
    }
}

__attribute__((target("avx2,fma"))) static float hsum256(__m256 v) {
  const __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  const __m128 t = _mm_add_ps(s, _mm_movehl_ps(s, s));
  return _mm_cvtss_f32(_mm_add_ss(t, _mm_shuffle_ps(t, t, 1)));
}

__attribute__((target("avx2,fma"))) static void columns_avx2(const job_t *j, uint32_t n0, uint32_t n1) {
  const __m256i nib = _mm256_set1_epi32(15);
  for (uint32_t n = n0; n < n1; ++n)
    for (uint32_t r0 = 0; r0 < j->M; r0 += kRowBlock) {
      const column_t col = column_at(j, n);
      const uint32_t rows = j->M - r0 < kRowBlock ? j->M - r0 : kRowBlock;
      __m256 acc[kRowBlock];
      for (uint32_t r = 0; r < kRowBlock; ++r) acc[r] = _mm256_setzero_ps();
      for (uint32_t g = 0; g < j->G; ++g) {
        float s, z;
        group_coef(j, col, g, &s, &z);
        const __m128i c = _mm_loadu_si128((const __m128i *)(col.plane + (size_t)g * 1024));
        const __m256 vs = _mm256_set1_ps(s), vz = _mm256_set1_ps(z);
        const float *x = j->xp + ((size_t)r0 * j->G + g) * 32;
        for (int half = 0; half < 2; ++half) {
          const __m256i b = _mm256_cvtepu8_epi32(half ? _mm_srli_si128(c, 8) : c);
          const __m256 wl = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_and_si256(b, nib)), vs, vz);
          const __m256 wh = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_srli_epi32(b, 4)), vs, vz);
          for (uint32_t r = 0; r < rows; ++r) {
            const float *xr = x + (size_t)r * j->G * 32 + 8 * half;
            acc[r] = _mm256_fmadd_ps(wl, _mm256_loadu_ps(xr), acc[r]);
            acc[r] = _mm256_fmadd_ps(wh, _mm256_loadu_ps(xr + 16), acc[r]);
          }
        }
      }
      for (uint32_t r = 0; r < rows; ++r) j->out[(size_t)(r0 + r) * j->N + n] = to_bf16(hsum256(acc[r]));
    }
}

static void columns_scalar(const job_t *j, uint32_t n0, uint32_t n1) {
  for (uint32_t n = n0; n < n1; ++n)
    for (uint32_t r = 0; r < j->M; ++r) {
      const column_t col = column_at(j, n);
      float acc = 0.0f;
      for (uint32_t g = 0; g < j->G; ++g) {
        float s, z;
        group_coef(j, col, g, &s, &z);
        const uint8_t *c = col.plane + (size_t)g * 1024;
        const float *x = j->xp + ((size_t)r * j->G + g) * 32;
        for (int b = 0; b < 16; ++b) {
          acc = fmaf(fmaf((float)(c[b] & 15u), s, z), x[b], acc);
          acc = fmaf(fmaf((float)(c[b] >> 4), s, z), x[16 + b], acc);
        }
      }
      j->out[(size_t)r * j->N + n] = to_bf16(acc);
    }
}

/* Thread t's share: tiles [t T / threads, (t + 1) T / threads) of the T plane tiles. */
static void run_share(sqo_pool *p, int t) {
  const job_t *j = &p->job;
  const uint32_t tiles = j->N / 64, t0 = (uint32_t)((uint64_t)tiles * t / p->threads),
                 t1 = (uint32_t)((uint64_t)tiles * (t + 1) / p->threads);
  if (t0 == t1) return;
  if (p->kind == 3) columns_bf16(j, 64 * t0, 64 * t1);
  else if (p->kind == 2) columns_avx512(j, 64 * t0, 64 * t1);
  else if (p->kind == 1) columns_avx2(j, 64 * t0, 64 * t1);
  else columns_scalar(j, 64 * t0, 64 * t1);
}

typedef struct {
  sqo_pool *pool;
  int index;
} worker_arg;
static worker_arg g_args[kMaxThreads];

static void *worker(void *arg) {
  const worker_arg *a = (const worker_arg *)arg;
  sqo_pool *p = a->pool;
  uint64_t seen = 0;
  for (;;) {
    pthread_mutex_lock(&p->mu);
    while (p->generation == seen && !p->quit) pthread_cond_wait(&p->go, &p->mu);
    if (p->quit) {
      pthread_mutex_unlock(&p->mu);
      return NULL;
    }
    seen = p->generation;
    pthread_mutex_unlock(&p->mu);
    run_share(p, a->index);
    pthread_mutex_lock(&p->mu);
    if (--p->remaining == 0) pthread_cond_signal(&p->done);
    pthread_mutex_unlock(&p->mu);
  }
}

static const char *const kNames[] = {"scalar", "avx2+fma", "avx512f", "avx512bf16"};
/* Whether the CPU runs kernel kind k. */
static int cpu_has(int k) {
  __builtin_cpu_init();
  switch (k) {
    case 3: return __builtin_cpu_supports("avx512bf16") && __builtin_cpu_supports("avx512bw");
    case 2: return __builtin_cpu_supports("avx512f");
    case 1: return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    default: return k == 0;
  }
}
static int cpu_kind(void) {
  for (int k = 3; k > 0; --k)
    if (cpu_has(k)) return k;
  return 0;
}
const char *sqo_cpu_isa(void) { return kNames[cpu_kind()]; }

sqo_pool *sqo_pool_create(int threads) {
  if (threads < 1) threads = 1;
  if (threads > kMaxThreads) threads = kMaxThreads;
  init_elements();
  sqo_pool *p = (sqo_pool *)calloc(1, sizeof(sqo_pool));
  p->threads = threads;
  p->kind = cpu_kind();
  pthread_mutex_init(&p->mu, NULL);
  pthread_cond_init(&p->go, NULL);
  pthread_cond_init(&p->done, NULL);
  /* Thread 0 is the caller's; workers take shares 1..threads-1. Only one pool runs at a time (g_args). */
  for (int t = 1; t < threads; ++t) {
    g_args[t].pool = p;
    g_args[t].index = t;
    pthread_create(&p->tid[t], NULL, worker, &g_args[t]);
  }
  return p;
}

void sqo_pool_destroy(sqo_pool *p) {
  if (!p) return;
  pthread_mutex_lock(&p->mu);
  p->quit = 1;
  pthread_cond_broadcast(&p->go);
  pthread_mutex_unlock(&p->mu);
  for (int t = 1; t < p->threads; ++t) pthread_join(p->tid[t], NULL);
  free(p->xp);
  free(p->xb);
  free(p->sx);
  free(p);
}

int sqo_pool_threads(const sqo_pool *p) { return p->threads; }
const char *sqo_pool_isa(const sqo_pool *p) { return kNames[p->kind]; }

int sqo_pool_set_isa(sqo_pool *p, const char *isa) {
  for (int k = 0; k < 4; ++k)
    if (!strcmp(isa, kNames[k])) {
      if (!cpu_has(k)) return -1;
      p->kind = k;
      return 0;
    }
  return -1;
}

int sqo_pool_reserve(sqo_pool *p, uint32_t M, uint32_t K) {
  const size_t need = (size_t)M * K;
  if (need <= p->xp_floats) return 0;
  free(p->xp);
  free(p->xb);
  free(p->sx);
  p->xp = (float *)aligned_alloc(64, (need * sizeof(float) + 63) / 64 * 64);
  p->xb = (uint16_t *)aligned_alloc(64, (need * sizeof(uint16_t) + 63) / 64 * 64);
  p->sx = (float *)aligned_alloc(64, (need / 32 * sizeof(float) + 63) / 64 * 64);
  const int ok = p->xp && p->xb && p->sx;
  p->xp_floats = ok ? need : 0;
  return ok ? 0 : -1;
}

double sqo_pool_matmul(sqo_pool *p, uint32_t fmt, uint32_t M, uint32_t N, uint32_t K, const uint16_t *x,
                       const uint8_t *plane0, const uint8_t *meta, uint16_t *out) {
  if (fmt != SQO_FMT_Q4K && fmt != SQO_FMT_AF4G32 && fmt != SQO_FMT_AF4G64 && fmt != SQO_FMT_AF4G128) return -1.0;
  if (!M || N % 64 || K % 256 || (size_t)M * K > p->xp_floats) return -1.0;
  sqo_format f;
  sqo_format_info(fmt, &f);
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  const uint32_t G = K / 32;
  /* The rows' inputs in the codes' byte order, once per call, and their sums per scale group. */
  const uint32_t sg = fmt == SQO_FMT_Q4K ? 1u : f.meta_groups;
  for (uint32_t r = 0; r < M; ++r)
    for (uint32_t g = 0; g < G; ++g) {
      float *d = p->xp + ((size_t)r * G + g) * 32;
      uint16_t *e = p->xb + ((size_t)r * G + g) * 32;
      const uint16_t *s = x + (size_t)r * K + (size_t)g * 32;
      float sum = 0.0f;
      for (int b = 0; b < 16; ++b) {
        e[b] = s[g_element[b][0]];
        e[16 + b] = s[g_element[b][1]];
        d[b] = sqo_bf16_to_f32(e[b]);
        d[16 + b] = sqo_bf16_to_f32(e[16 + b]);
        sum += d[b] + d[16 + b];
      }
      float *unit = p->sx + (size_t)r * (G / sg) + g / sg;
      *unit = g % sg ? *unit + sum : sum;
    }
  p->job = (job_t){fmt, M, N, K, G, G / f.meta_groups, f.meta_groups, f.meta_bytes, p->xp, p->xb, p->sx,
                   plane0, meta, out};
  pthread_mutex_lock(&p->mu);
  p->remaining = p->threads - 1;
  ++p->generation;
  pthread_cond_broadcast(&p->go);
  pthread_mutex_unlock(&p->mu);
  run_share(p, 0);
  pthread_mutex_lock(&p->mu);
  while (p->remaining > 0) pthread_cond_wait(&p->done, &p->mu);
  pthread_mutex_unlock(&p->mu);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}
