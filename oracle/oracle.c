/*
 * oracle.c - C restatement of the reference's CPU arithmetic for the quantized-weight path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker and the CPU baseline of bench.py. The product
 * (libtmhip.so) never links or calls this file.
 *
 * What it restates (paths into georgeguimaraes/transmuter):
 *  - oracle_dequantize_nbits: Quantized.dequantize_weight/4 (lib/transmuter/ops/quantized.ex:
 *    234-240) with Packed.unpack/2 and dequantize/3 (lib/transmuter/ops/packed.ex:9-36) and
 *    block_zero_points/5 (quantized.ex:306-325): the load-time dequantization of move/2
 *    (lib/transmuter.ex:1230-1240), in f32 or f16 (each operation rounded to the type).
 *  - oracle_gemm_f32 / oracle_gemm_f16w: the matmul that runs after move/2 on the EXLA CPU
 *    backend, Nx.dot(a, [-1], w, [1]) (quantized.ex:44) over the dequantized {N, K} weights,
 *    f32 accumulation (AVX2 FMA, f16 weights widened with F16C), on `threads` OpenMP threads
 *    (XLA runs Eigen on a persistent thread pool).
 *  - oracle_matmul_nbits_in_graph: the same call without move/2, which dequantizes the weights
 *    in the graph on every call (quantized.ex:39-44), then the dot.
 *  - oracle_matmul_integer: MatMulInteger's exact s32 sums (quantized.ex:105-110,
 *    lib/transmuter/ops/nn.ex:537-555), wrapping like s32.
 * Pinned by tests/test_oracle_c.py against oracle/oracle.py and the reference's fixtures.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: renormalise */
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while (!(man & 0x400u));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Round to nearest even, with subnormals, overflow to infinity and NaN kept. */
static uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t absx = x & 0x7FFFFFFFu;
  if (absx > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520: inf */
  if (absx < 0x38800000u) {                                   /* below 2^-14: subnormal or 0 */
    if (absx < 0x33000000u) return sign;                      /* below 2^-25 rounds to 0 */
    const uint32_t e = absx >> 23;                            /* 102 .. 112 */
    const uint32_t man = (absx & 0x7FFFFFu) | 0x800000u;
    /* value = man * 2^(e-150) = (man >> (126-e)) units of 2^-24, the f16 subnormal step */
    const uint32_t sh = 126u - e;
    uint32_t r = man >> sh;
    const uint32_t rem = man & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = absx - 0x38000000u; /* rebias the exponent: 127 - 15 = 112 << 23 */
  const uint32_t rem = r & 0x1FFFu;
  r >>= 13;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

static float round_f16(float f) { return f16_to_f32(f32_to_f16(f)); }

/* out_f16: 0 writes f32 values to w_out, 1 writes f16 bit patterns (uint16_t). */
int oracle_dequantize_nbits(const uint8_t* b, const float* scales, const uint8_t* zp_packed,
                            const float* zp_float, int64_t K, int64_t N, int bits, int block_size,
                            int out_f16, void* w_out) {
  if (bits != 2 && bits != 4 && bits != 8) return 1;
  const int64_t blocks = (K + block_size - 1) / block_size;
  const int64_t row_bytes = blocks * block_size * bits / 8;
  const int64_t zrow = (blocks * bits + 7) / 8;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t k = 0; k < K; ++k) {
      const int64_t bit = k * bits;
      const uint32_t q = (b[n * row_bytes + bit / 8] >> (bit % 8)) & mask;
      const int64_t blk = k / block_size;
      float z;
      if (zp_packed) {
        const int64_t zb = blk * bits;
        z = (float)((zp_packed[n * zrow + zb / 8] >> (zb % 8)) & mask);
      } else if (zp_float) {
        z = zp_float[n * blocks + blk];
      } else {
        z = (float)(1u << (bits - 1));
      }
      float s = scales[n * blocks + blk];
      if (out_f16) {
        s = round_f16(s);
        z = round_f16(z);
        const float d = round_f16((float)q - z);
        ((uint16_t*)w_out)[n * K + k] = f32_to_f16(d * s);
      } else {
        const float d = (float)q - z;
        ((float*)w_out)[n * K + k] = d * s;
      }
    }
  }
  return 0;
}

/* One output row n of Y = A . W^T: f32 products accumulated in f32 (8 lanes of AVX2 FMA, then
 * the lanes added), W read as f32 or widened from f16 with F16C as it is read. */
static void gemm_row(const float* a, const void* w, int w_f16, int64_t M, int64_t N, int64_t K, float* y, int64_t n) {
  for (int64_t m = 0; m < M; ++m) {
    const float* am = a + m * K;
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    int64_t k = 0;
    if (w_f16) {
      const uint16_t* wn = (const uint16_t*)w + n * K;
      for (; k + 16 <= K; k += 16) {
        const __m256 w0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(wn + k)));
        const __m256 w1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(wn + k + 8)));
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(am + k), w0, acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(am + k + 8), w1, acc1);
      }
      float tail = 0.f;
      for (; k < K; ++k) tail += am[k] * f16_to_f32(wn[k]);
      float lanes[8];
      _mm256_storeu_ps(lanes, _mm256_add_ps(acc0, acc1));
      y[m * N + n] = ((lanes[0] + lanes[1]) + (lanes[2] + lanes[3])) + ((lanes[4] + lanes[5]) + (lanes[6] + lanes[7])) + tail;
    } else {
      const float* wn = (const float*)w + n * K;
      for (; k + 16 <= K; k += 16) {
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(am + k), _mm256_loadu_ps(wn + k), acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(am + k + 8), _mm256_loadu_ps(wn + k + 8), acc1);
      }
      float tail = 0.f;
      for (; k < K; ++k) tail += am[k] * wn[k];
      float lanes[8];
      _mm256_storeu_ps(lanes, _mm256_add_ps(acc0, acc1));
      y[m * N + n] = ((lanes[0] + lanes[1]) + (lanes[2] + lanes[3])) + ((lanes[4] + lanes[5]) + (lanes[6] + lanes[7])) + tail;
    }
  }
}

/* Rows split over `threads` OpenMP threads (a persistent team, as XLA's CPU backend runs its dot
 * on a persistent Eigen thread pool). */
static int gemm(const float* a, const void* w, int w_f16, int64_t M, int64_t N, int64_t K, float* y,
                int threads) {
  if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t n = 0; n < N; ++n) gemm_row(a, w, w_f16, M, N, K, y, n);
  return 0;
}

/* Y[M, N] = A[M, K] . W[N, K]^T, f32 weights. */
int oracle_gemm_f32(const float* a, const float* w, int64_t M, int64_t N, int64_t K, float* y, int threads) {
  return gemm(a, w, 0, M, N, K, y, threads);
}

/* The same with f16 weights (bit patterns), each widened to f32 as it is read. */
int oracle_gemm_f16w(const float* a, const uint16_t* w, int64_t M, int64_t N, int64_t K, float* y,
                     int threads) {
  return gemm(a, w, 1, M, N, K, y, threads);
}

/* MatMulNBits without a moved weight (quantized.ex:39-44): every call dequantizes W in the
 * activations' type (f16 or f32, out_f16) into `scratch` (N*K values), then runs the dot. The
 * dequantization splits over the same threads by rows. */
int oracle_matmul_nbits_in_graph(const float* a, const uint8_t* b, const float* scales, const uint8_t* zp_packed,
                                 int64_t M, int64_t K, int64_t N, int bits, int block_size, int out_f16,
                                 void* scratch, float* y, int threads) {
  if (threads < 1) threads = 1;
  if (bits != 2 && bits != 4 && bits != 8) return 1;
  const int64_t blocks = (K + block_size - 1) / block_size;
  const int64_t row_bytes = blocks * block_size * bits / 8;
  const int64_t zrow = (blocks * bits + 7) / 8;
  int bad = 0;
#pragma omp parallel for num_threads(threads) schedule(static) reduction(| : bad)
  for (int64_t n = 0; n < N; ++n) {
    void* out = out_f16 ? (void*)((uint16_t*)scratch + n * K) : (void*)((float*)scratch + n * K);
    bad |= oracle_dequantize_nbits(b + n * row_bytes, scales + n * blocks, zp_packed ? zp_packed + n * zrow : NULL,
                                   NULL, K, 1, bits, block_size, out_f16, out);
  }
  if (bad) return 1;
  return gemm(a, scratch, out_f16, M, N, K, y, threads);
}
/* y[b, m, n] = sum_k (a - az[m]) (b - bz[n]) mod 2^32; a_signed / b_signed select s8 data. */
int oracle_matmul_integer(const uint8_t* a, int a_signed, const uint8_t* bm, int b_signed,
                          const uint8_t* az, int64_t az_count, const uint8_t* bz, int64_t bz_count,
                          int64_t batch, int64_t M, int64_t K, int64_t N, int b_batched, int32_t* y) {
  for (int64_t t = 0; t < batch; ++t) {
    const uint8_t* at = a + t * M * K;
    const uint8_t* bt = bm + (b_batched ? t * K * N : 0);
    for (int64_t m = 0; m < M; ++m) {
      const int64_t zm = az ? (a_signed ? (int8_t)az[az_count == 1 ? 0 : m] : az[az_count == 1 ? 0 : m]) : 0;
      for (int64_t n = 0; n < N; ++n) {
        const int64_t zn = bz ? (b_signed ? (int8_t)bz[bz_count == 1 ? 0 : n] : bz[bz_count == 1 ? 0 : n]) : 0;
        int64_t acc = 0;
        for (int64_t k = 0; k < K; ++k) {
          const int64_t av = (a_signed ? (int8_t)at[m * K + k] : at[m * K + k]) - zm;
          const int64_t bv = (b_signed ? (int8_t)bt[k * N + n] : bt[k * N + n]) - zn;
          acc += av * bv;
        }
        y[(t * M + m) * N + n] = (int32_t)(uint32_t)(uint64_t)acc;
      }
    }
  }
  return 0;
}

/* Helpers the tests use to pin the f16 conversions against numpy. */
void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}
