// MatMulNBits on gfx950: the packed-weight store, its dequantization, and Y = A . W^T.
//
// Reference arithmetic (georgeguimaraes/transmuter):
//   lib/transmuter/ops/quantized.ex:30-46    MatMulNBits handler
//   lib/transmuter/ops/quantized.ex:226-240  nbits_sizes/1, dequantize_weight/4
//   lib/transmuter/ops/quantized.ex:294-325  unpack/2 (sign), block_zero_points/5
//   lib/transmuter/ops/packed.ex:9-36        unpack/2 (lowest bits first), dequantize/3
//   lib/transmuter.ex:1104-1240              move/2: packs each weight once at load
//
// Kernels
//   k_dequant         the {N, K} weights, bit-exact, in any float type
//   k_gemv_dec        (tmh_gemv.h) decode GEMV for M <= 16, f16 Y (an f16 bias or none)
//   k_gemv_f16        f16 A and f16 weights, M <= 16*MT per block row: every lane unpacks its
//                     16 bytes in registers into exact f16 weights (q - zero) * scale and feeds
//                     v_mfma_f32_16x16x32_f16; four wavefronts split K and add through LDS
//   k_gemm_f16        the same fragments for larger M, 128x128 tiles per workgroup
//   k_matmul_general  any float types and float zero points, f32 FMA on the vector ALUs
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <type_traits>
#include <cstdlib>
#include <vector>

#include "tmh_device.h"
#include "tmh_internal.h"

using namespace tmh;

// Scratch memory of tmh_matmul_nbits_noalloc: the split-K partial sums of its prefill GEMMs,
// for callers that cannot allocate (graph capture, serving loops). Each device the library
// runs on holds its own copy until the process ends. In host code `scratch` names a host-side
// stand-in, not device memory: kernels get the address that hipGetSymbolAddress gives for
// each device (noalloc_scratch_init).
constexpr size_t kNoallocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) float scratch[kNoallocScratchBytes / sizeof(float)];

namespace {

constexpr int kWaves = 4;
constexpr int kMaxConcat = 8;
constexpr int kThreads = 64 * kWaves;

int ilog2(int v) {
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

// ------------------------------------------------------------------ host repack

// Position of value i of a 32-bit word in the tiled layout (see tmh_weight).
inline int value_pos(int bits, int i) { return bits == 8 ? 8 * i : (i & 1) * 16 + (i >> 1) * bits; }

uint32_t reorder_word(uint32_t natural, int bits) {
  if (bits == 8) return natural;
  const int count = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t out = 0;
  for (int i = 0; i < count; ++i) out |= ((natural >> (i * bits)) & mask) << value_pos(bits, i);
  return out;
}

// Zero point of block b of row n from packed rows of ceil(blocks*bits/8) bytes, lowest bits
// first (quantized.ex:316-323).
uint8_t packed_zero(const uint8_t* zp, int64_t zrow, int bits, int64_t n, int64_t b) {
  const int64_t bit = b * bits;
  const uint8_t byte = zp[n * zrow + bit / 8];
  return static_cast<uint8_t>((byte >> (bit % 8)) & ((1 << bits) - 1));
}

float round_host(float x, int dt) {
  if (dt == TMH_F16) return f16_to_f32(f32_to_f16(x));
  if (dt == TMH_BF16) return bf16_to_f32(f32_to_bf16(x));
  return x;
}

void store_host(void* p, int dt, size_t i, float v) {
  if (dt == TMH_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
  } else if (dt == TMH_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

int merge_float(int a, int b) {
  if (a == b) return a;
  return TMH_F32;
}

// ------------------------------------------------------------------ kernels

// The {N, K} weights in OUT, computed in OUT from the stored scales (type WDT) and zero points.
template <int BITS, int WDT, int OUT, int ZK>
__global__ __launch_bounds__(256) void k_dequant(const uint4_t* __restrict__ qt,
                                                 const void* __restrict__ sc,
                                                 const void* __restrict__ zp, void* __restrict__ out,
                                                 int64_t N, int64_t K, int64_t nchunks, int nbc,
                                                 int bsc_shift, int64_t total_lanes) {
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int PER_WORD = 32 / BITS;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= total_lanes) return;
  const int lane = static_cast<int>(id & 63);
  const int64_t tc = id >> 6;
  const int64_t t = tc / nchunks;
  const int64_t c = tc - t * nchunks;
  const int r = lane & 15, g = lane >> 4;
  const int64_t n = t * 16 + r;
  if (n >= N) return;
  const uint4_t w = qt[id];
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
    for (int v = 0; v < PER_WORD; ++v) {
      const int woff = g * GW + wi * PER_WORD + v;
      const int64_t k = c * CW + woff;
      if (k >= K) continue;
      const int64_t p = (tc * nbc + (woff >> bsc_shift)) * 16 + r;
      const float s = round_to<OUT>(load_as_f32<WDT>(sc, p));
      float z;
      if constexpr (ZK == TMH_ZP_PACKED) {
        const uint8_t byte = static_cast<const uint8_t*>(zp)[zp_byte<BITS>(p)];
        z = static_cast<float>(zp_field<BITS>(byte, zp_shift<BITS>(static_cast<uint32_t>(p))));
      } else if constexpr (ZK == TMH_ZP_FLOAT) {
        z = round_to<OUT>(static_cast<const float*>(zp)[p]);
      } else {
        z = static_cast<float>(1 << (BITS - 1));
      }
      const float q = static_cast<float>(word_value<BITS>(w[wi], v));
      store_as<OUT>(out, n * K + k, dequant_value<OUT>(q, z, s));
    }
  }
}

// Eight f16 values of A row m at columns k..k+7 (zeros outside the matrix).
__device__ __forceinline__ half8_t load_a8(const _Float16* __restrict__ A, int64_t m, int64_t M,
                                           int64_t k, int64_t K, int64_t lda, bool vec) {
  half8_t a = {};
  if (m >= M || k >= K) return a;
  const _Float16* p = A + m * lda + k;
  if (vec && k + 8 <= K) {
    a = *reinterpret_cast<const half8_t*>(p);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = (k + e < K) ? p[e] : static_cast<_Float16>(0.0f);
  }
  return a;
}

// Scale and 1024 + zero of parameter entry p, as f16 pairs.
template <bool HAS_ZP, int BITS>
__device__ __forceinline__ void load_params(const uint16_t* __restrict__ sc,
                                            const uint8_t* __restrict__ zp, int64_t p, half2_t& ss,
                                            half2_t& zz) {
  const uint32_t s = sc[p];
  ss = __builtin_bit_cast(half2_t, s | (s << 16));
  uint32_t z;
  if constexpr (HAS_ZP) {
    z = 0x6400u + zp_field<BITS>(zp[zp_byte<BITS>(p)], zp_shift<BITS>(static_cast<uint32_t>(p)));
  } else {
    z = 0x6400u + (1u << (BITS - 1));
  }
  zz = __builtin_bit_cast(half2_t, z | (z << 16));
}

// Adds the partial sums of the block's wavefronts and writes rows m0.. of one 16-column tile.
template <int MT>
__device__ __forceinline__ void gemv_epilogue(float4_t (&acc)[MT], float4_t* red, int nwaves, int64_t t,
                                              int64_t m0, int64_t M, int64_t N,
                                              const void* __restrict__ bias, int bias_dt,
                                              void* __restrict__ Y, int y_dt, int dot_dt,
                                              int64_t ldy) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[(wave * MT + mt) * 64 + lane] = acc[mt];
  __syncthreads();
  // Wave w finishes m-tiles w, w + nwaves, ...
  for (int mt = wave; mt < MT; mt += nwaves) {
    float4_t s = red[mt * 64 + lane];
    for (int w = 1; w < nwaves; ++w) s += red[(w * MT + mt) * 64 + lane];
    const int64_t n = t * 16 + (lane & 15);
    if (n >= N) continue;
    const float b = bias ? load_float_rt(bias, bias_dt, n) : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t m = m0 + mt * 16 + 4 * (lane >> 4) + e;
      if (m >= M) continue;
      float v = s[e];
      if (dot_dt == DT_F16) v = round_to<DT_F16>(v);
      if (bias) v += b;
      store_float_rt(Y, y_dt, m * ldy + n, v);
    }
  }
}

// Eight f16 values of A row m at columns k..k+7 when A rows are 16-byte aligned and K is a
// multiple of 8: one unconditional 16-byte load (of row 0 when out of range, then zeroed), so
// the loads of a round can all issue before the first one is used.
__device__ __forceinline__ half8_t load_a8_fast(const _Float16* __restrict__ A, int64_t m, int64_t M,
                                                int64_t k, int64_t K, int64_t lda) {
  const bool ok = m < M && k < K;
  const half8_t v = *reinterpret_cast<const half8_t*>(A + (ok ? m * lda + k : 0));
  return ok ? v : half8_t{};
}

// One workgroup per 16-column tile (and per 16*MT rows of A). Its nwaves = blockDim.x / 64
// wavefronts split K: wave w takes chunks w*U .. w*U+U-1, then w*U + nwaves*U.., and issues
// the U weight loads of a round, their parameters and (a_fast) their A fragments together,
// so a small GEMV has its whole weight in flight at once instead of one chunk per latency.
template <int BITS, int MT, bool HAS_ZP, bool SPLIT, int U>
__global__ __launch_bounds__(1024) void k_gemv_f16(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, int64_t M, int64_t K, int64_t lda, bool a_fast,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ Y, int y_dt, int dot_dt,
    int64_t ldy, int64_t N, int64_t nchunks, int nbc, int bsc_shift) {
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int STEPS = GW / 8;
  constexpr bool HOIST = MT * U * STEPS <= 16;
  extern __shared__ float4_t red[];
  const int nwaves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t t = blockIdx.x;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 16 * MT;
  float4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int64_t base = static_cast<int64_t>(wave) * U; base < nchunks; base += static_cast<int64_t>(nwaves) * U) {
    uint4_t w[U];
    half2_t ss[U], zz[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = base + u < nchunks ? base + u : nchunks - 1;
      w[u] = qt[(t * nchunks + c) * 64 + lane];
      if constexpr (!SPLIT)
        load_params<HAS_ZP, BITS>(sc, zp, ((t * nchunks + c) * nbc + ((g * GW) >> bsc_shift)) * 16 + r, ss[u], zz[u]);
    }
    half8_t af[HOIST ? U : 1][HOIST ? STEPS : 1][HOIST ? MT : 1];
    if constexpr (HOIST) {
      if (a_fast) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int i = 0; i < STEPS; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              af[u][i][mt] = load_a8_fast(A, m0 + mt * 16 + r, M, (base + u) * CW + g * GW + 8 * i,
                                          base + u < nchunks ? K : 0, lda);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = base + u;
      if (c >= nchunks) break;
      const int64_t kbase = c * CW + g * GW;
#pragma unroll
      for (int i = 0; i < STEPS; ++i) {
        if constexpr (SPLIT)
          load_params<HAS_ZP, BITS>(sc, zp, ((t * nchunks + c) * nbc + ((g * GW + 8 * i) >> bsc_shift)) * 16 + r,
                                    ss[u], zz[u]);
        const half8_t b = unpack_step<BITS>(w[u], i, zz[u], ss[u]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          half8_t a;
          if constexpr (HOIST) {
            a = a_fast ? af[u][i][mt] : load_a8(A, m0 + mt * 16 + r, M, kbase + 8 * i, K, lda, false);
          } else {
            a = a_fast ? load_a8_fast(A, m0 + mt * 16 + r, M, kbase + 8 * i, K, lda)
                       : load_a8(A, m0 + mt * 16 + r, M, kbase + 8 * i, K, lda, false);
          }
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[mt], 0, 0, 0);
        }
      }
    }
  }
  gemv_epilogue<MT>(acc, red, nwaves, t, m0, M, N, bias, bias_dt, Y, y_dt, dot_dt, ldy);
}


// 128 x 128 output tile per workgroup: wave (wm, wn) computes rows 64*wm.. and columns
// 64*wn.. (four 16-row tiles by four 16-column tiles) over all of K.
template <int BITS, bool HAS_ZP, bool SPLIT>
__global__ __launch_bounds__(256) void k_gemm_f16(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, int64_t M, int64_t K, int64_t lda, bool a_vec,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ Y, int y_dt, int dot_dt,
    int64_t ldy, int64_t N, int64_t ntiles, int64_t nchunks, int nbc, int bsc_shift) {
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int STEPS = GW / 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 8 + wn * 4;  // first 16-column tile
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 128 + wm * 64;
  float4_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int64_t c = 0; c < nchunks; ++c) {
    uint4_t w[4];
    int64_t tcs[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int64_t t = t0 + nt < ntiles ? t0 + nt : ntiles - 1;
      tcs[nt] = t * nchunks + c;
      w[nt] = qt[tcs[nt] * 64 + lane];
    }
    const int64_t kbase = c * CW + g * GW;
    half2_t ss[4], zz[4];
    if constexpr (!SPLIT) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        load_params<HAS_ZP, BITS>(sc, zp, (tcs[nt] * nbc + ((g * GW) >> bsc_shift)) * 16 + r, ss[nt], zz[nt]);
    }
#pragma unroll
    for (int i = 0; i < STEPS; ++i) {
      half8_t bf[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        if constexpr (SPLIT)
          load_params<HAS_ZP, BITS>(sc, zp, (tcs[nt] * nbc + ((g * GW + 8 * i) >> bsc_shift)) * 16 + r, ss[nt], zz[nt]);
        bf[nt] = unpack_step<BITS>(w[nt], i, zz[nt], ss[nt]);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const half8_t a = load_a8(A, m0 + mt * 16 + r, M, kbase + 8 * i, K, lda, a_vec);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bf[nt], acc[mt][nt], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int64_t n = (t0 + nt) * 16 + r;
    if (t0 + nt >= ntiles || n >= N) continue;
    const float b = bias ? load_float_rt(bias, bias_dt, n) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + mt * 16 + 4 * g + e;
        if (m >= M) continue;
        float v = acc[mt][nt][e];
        if (dot_dt == DT_F16) v = round_to<DT_F16>(v);
        if (bias) v += b;
        store_float_rt(Y, y_dt, m * ldy + n, v);
      }
    }
  }
}

// Prefill GEMM: BM x 64*WN output tile per workgroup of 2*WN wavefronts (BM = 256 or 128; WN = 2:
// one wavefront per SIMD, WN = 4: two per SIMD), k-blocks of one chunk (CW weights).
//  - A: the k-block's BM rows x CW f16 go global -> LDS by buffer_load ... lds (no VGPRs),
//    double buffered, rows of CW*2 bytes whose 16-byte pieces are XOR-swizzled by row so the
//    MFMA fragment reads of 16 rows hit distinct banks. Rows past M lie outside the buffer
//    range and read zeros (their outputs are never stored). A partial last k-block goes through
//    registers and is zeroed past K.
//  - B: with BM = 256 and WN = 2, wavefront (wm, wn) computes rows 128*wm.. and columns 64*wn..
//    (four 16-column weight tiles, each dequantized fragment feeding eight MFMAs); otherwise
//    ("tall"), each wavefront computes all BM rows of two tiles (each fragment feeding BM/16).
//    The tiles' weights, scales and zero points are loaded one k-block ahead and dequantized in
//    registers (exact f16) for v_mfma_f32_16x16x32_f16.
// BM = 128 gives shapes with few 256-row blocks (M = 2048, N = 2048) enough workgroups without
// splitting K, and its 64 KiB of LDS lets two workgroups share a CU.
constexpr int kGemmBM = 256;  // largest tile height: bounds the A rows a launch may touch

// How the prefill GEMM's operands reach the MFMAs (the template argument MODE):
//  GM_F16   f16 A and f16 weights (q - zero) * scale made exact in f16 registers from the packed
//           bits (unpack_step), v_mfma_f32_16x16x32_f16;
//  GM_BF16  bf16 A and bf16 weights: (q - zero) * scale formed exactly in f32 and rounded once to
//           bf16, as the reference's bf16 dequantization rounds it (packed or no zero points),
//           v_mfma_f32_16x16x32_bf16;
//  GM_SPLIT any other float types (f32 A, f32 weights, float zero points, mixed types): A is split
//           by k_split_a into bf16 hi + lo (hi = bf16(a), lo = bf16(a - hi): 16 significant bits,
//           f32's exponent range), the weights are dequantized in f32 and rounded to their own type
//           WT as the reference does, then split the same way, and each product takes three bf16
//           MFMAs (hi*hi + lo*hi + hi*lo; the dropped lo*lo term is below 2^-16 of each product).
enum : int { GM_F16 = 0, GM_BF16 = 1, GM_SPLIT = 2 };

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// LDS of one workgroup: the double-buffered A tile (two tiles, hi and lo, for GM_SPLIT), or
// (KS = 2) the partial sums of half the wavefronts after the k-loop, whichever is larger.
template <int BITS, int BM, int KS = 1, int MODE = GM_F16>
constexpr size_t gemm_lds_bytes() {
  constexpr size_t a_tiles = 2 * static_cast<size_t>(BM) * (512 / BITS) * 2 * (MODE == GM_SPLIT ? 2 : 1);
  constexpr size_t partial = KS > 1 ? static_cast<size_t>(BM) * 128 * sizeof(float) : 0;
  return a_tiles > partial ? a_tiles : partial;
}

// One MFMA step of a 16x16 output tile: weights (first operand) times A.
template <int MODE>
__device__ __forceinline__ float4_t gm_mma(const uint4_t& b, const uint4_t& a, float4_t c) {
  if constexpr (MODE == GM_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, b), __builtin_bit_cast(half8_t, a), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, b), __builtin_bit_cast(bf16x8_t, a), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ float byte_f32(uint32_t x, int b) { return static_cast<float>((x >> (8 * b)) & 0xFFu); }

// The eight values q of MFMA step i of a lane's 16 weight bytes, in k order, as f32 (in the
// tiled layout's word order: value 2j at bits j*BITS, value 2j+1 at bits 16 + j*BITS).
template <int BITS>
__device__ __forceinline__ void step_values(const uint4_t& w, int i, float (&q)[8]) {
  if constexpr (BITS == 4) {
    // Bytes of x & 0x0F0F0F0F hold values 0, 4, 1, 5; of (x >> 4) & 0x0F0F0F0F values 2, 6, 3, 7.
    const uint32_t x = w[i];
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    q[0] = byte_f32(lo, 0);
    q[1] = byte_f32(lo, 2);
    q[2] = byte_f32(hi, 0);
    q[3] = byte_f32(hi, 2);
    q[4] = byte_f32(lo, 1);
    q[5] = byte_f32(lo, 3);
    q[6] = byte_f32(hi, 1);
    q[7] = byte_f32(hi, 3);
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int b = 0; b < 4; ++b) q[4 * h + b] = byte_f32(w[2 * i + h], b);
  } else {  // 2 bits: step i uses half of word i/2, pair j at bits 2j and 16 + 2j
    const uint32_t x = w[i >> 1] >> (8 * (i & 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t p = (x >> (2 * j)) & 0x00030003u;
      q[2 * j] = byte_f32(p, 0);
      q[2 * j + 1] = byte_f32(p, 2);
    }
  }
}

// bf16 bits of two f32 values (round to nearest even) as one word, the first in the low half.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t p = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, p);
}

// GM_BF16 weights of step i: (q - zero) * scale = fma(q, scale, -zero * scale), exact in f32 (q and
// zero are integers below 256 and the scale a bf16 value), rounded once to bf16.
template <int BITS>
__device__ __forceinline__ uint4_t dequant_bf16(const uint4_t& w, int i, float s, float nzs) {
  float q[8];
  step_values<BITS>(w, i, q);
  uint4_t out;
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = pack_bf16(fmaf(q[2 * j], s, nzs), fmaf(q[2 * j + 1], s, nzs));
  return out;
}

// f32 value x rounded to type WT and back (f32: unchanged).
template <int WT>
__device__ __forceinline__ float round_wt(float x) {
  if constexpr (WT == DT_F32) return x;
  else return round_to<WT>(x);
}

// GM_SPLIT weights of step i: (q - zero) rounded to the weight type WT, times the scale, rounded
// to WT (the reference's dequantization in WT), then split into bf16 hi and lo.
template <int BITS, int WT>
__device__ __forceinline__ void dequant_split(const uint4_t& w, int i, float s, float z, uint4_t& hi, uint4_t& lo) {
  float q[8];
  step_values<BITS>(w, i, q);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float w0 = round_wt<WT>(round_wt<WT>(q[2 * j] - z) * s);
    const float w1 = round_wt<WT>(round_wt<WT>(q[2 * j + 1] - z) * s);
    const uint32_t h = pack_bf16(w0, w1);
    hi[j] = h;
    lo[j] = pack_bf16(w0 - __builtin_bit_cast(float, h << 16), w1 - __builtin_bit_cast(float, h & 0xFFFF0000u));
  }
}

// Slot of 16-byte piece `piece` in LDS row `row` (q4 rows hold 16 pieces, q8 rows 8); its own
// inverse, and a function of row % 16 only.
template <int BITS>
__device__ __forceinline__ int a_slot(int row, int piece) {
  return piece ^ frag_swizzle<BITS == 8 ? 8 : 16>(row);
}

// An f32 sum rounded to the dot's type (Nx.dot of two f16 or two bf16 operands gives that type).
__device__ __forceinline__ float round_dot(float x, int dot_dt) {
  return dot_dt == DT_F16 ? round_to<DT_F16>(x) : (dot_dt == DT_BF16 ? round_to<DT_BF16>(x) : x);
}

// Four consecutive outputs of row offset `row` (columns n.., those below N) in any float type: the
// dot type's rounding, then the bias. Kept out of line so that the GEMM epilogue's loops over its
// accumulator tiles stay small enough to unroll (the tiles then stay in registers).
__device__ __noinline__ void store_quad_any(float4_t v, void* Y, int y_dt, int dot_dt, const void* bias, int bias_dt,
                                            int64_t row, int64_t n, int64_t N) {
  for (int e = 0; e < 4 && n + e < N; ++e) {
    float x = v[e];
    x = round_dot(x, dot_dt);
    if (bias) x += load_float_rt(bias, bias_dt, n + e);
    store_float_rt(Y, y_dt, row + n + e, x);
  }
}

// (The body; k_gemm_lds and its stamping build k_gemm_lds_tl below are the kernels.)
// MODE (GM_*) and WT (GM_SPLIT: the weights' type) select the operand path; zk is the zero
// point kind (TMH_ZP_*) read by GM_SPLIT, whose zero points are packed (BITS bits per parameter
// entry) or f32 (float) per entry. For GM_SPLIT, A is the bf16 hi rows [M][lda] followed by the lo rows.
template <int BITS, bool HAS_ZP, bool SPLIT, int WN, int BM, int KS, bool TL, int MODE, int WT>
__device__ __forceinline__ void gemm_lds(
    const uint4_t* __restrict__ qt, const void* __restrict__ sc, const void* __restrict__ zp,
    const void* __restrict__ A, int64_t M, int64_t K, int64_t lda, const void* __restrict__ bias,
    int bias_dt, void* __restrict__ Y, int y_dt, int dot_dt, int64_t ldy, int64_t N, int64_t ntiles,
    int64_t nchunks, int nbc, int bsc_shift, int mblocks, int nblocks, int chunks_per_split,
    float* __restrict__ ws, int zk, uint32_t* __restrict__ tl) {
  const TlStart tl0 = TL ? tl_clock() : TlStart{0u, 0u};
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int STEPS = GW / 8;
  constexpr int ROWB = CW * 2;           // bytes per LDS row
  constexpr int PPR = CW / 8;            // 16-byte pieces per row
  constexpr int RPI = 64 / PPR;          // rows per wavefront load instruction
  constexpr int NWAVE = 2 * WN * KS;
  constexpr int RW = BM / NWAVE;         // A rows each wavefront brings into LDS
  // KS == 2 (BM = 64 or 128, WN = 2 only): eight wavefronts, two per SIMD; wavefronts w and w + 4 share
  // an output sub-tile and take the first and second half of each k-block's MFMA steps, and the
  // second half's partial sums add to the first's through LDS after the k-loop.
  static_assert(KS == 1 || (KS == 2 && BM <= 128 && WN == 2), "K split inside the workgroup");
  constexpr int LSTEPS = STEPS / KS;     // MFMA steps per k-block of one wavefront
  constexpr int LOADS = RW / RPI;        // load instructions per wavefront per k-block
  constexpr int NJ = SPLIT ? STEPS : 1;  // parameter entries per tile per k-block
  // Tall (WN == 4, eight wavefronts, two per SIMD; or BM <= 128): each wavefront takes all BM
  // rows and two weight tiles, so every dequantized fragment feeds BM/16 MFMAs. BM == 256 with
  // WN == 2 (four wavefronts): 128 rows and four tiles per wavefront.
  // Measured alternatives, none faster on the SmolLM3-3B shapes: four wavefronts each taking all
  // 256 rows of four tiles (one per SIMD; half the LDS reads per MFMA) were 4-15% slower; eight-
  // wavefront 128-row tiles held to 128 VGPRs (four per SIMD) spilled and were slower; reading A
  // fragments two or three ahead instead of one changed nothing.
  static_assert(BM == 64 || BM == 128 || BM == 256, "tile height");
  constexpr bool TALL = WN == 4 || BM <= 128;
  constexpr int MTW = TALL ? BM / 16 : 8;
  constexpr int NTW = TALL ? 2 : 4;
  static_assert(MODE == GM_F16 || (TALL && !SPLIT), "the bf16 paths use the tall layout, one parameter per lane");
  constexpr int ABUF = BM * ROWB * (MODE == GM_SPLIT ? 2 : 1);  // LDS bytes of one A buffer (hi, then lo)
  constexpr int SES = MODE == GM_SPLIT && WT == DT_F32 ? 4 : 2;  // bytes per stored scale
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int wl = wave % (2 * WN);        // the wavefront's output sub-tile
  const int kh = wave / (2 * WN);        // its half of the k-block's steps (KS == 2)
  const int wm = TALL ? 0 : wl / WN, wn = TALL ? wl : wl % WN;
  // Consecutive workgroups take the m-blocks of one n-block, so each XCD keeps one m-block's
  // A rows in its L2 while the weights stream past.
  // With split K (ws != nullptr), workgroup blocks of mblocks*nblocks take consecutive ranges of
  // chunks_per_split chunks and write f32 partial sums to ws[split][M][N].
  const unsigned tiles = static_cast<unsigned>(mblocks) * static_cast<unsigned>(nblocks);
  const int split = static_cast<int>(blockIdx.x / tiles);
  const unsigned tile = blockIdx.x % tiles;
  const int mb = static_cast<int>(tile % static_cast<unsigned>(mblocks));
  const int nb = static_cast<int>(tile / static_cast<unsigned>(mblocks));
  const int m0 = mb * BM;
  const int t0 = TALL ? nb * 4 * WN + wl * NTW : (nb * WN + wn) * 4;
  const uint32_t nch = static_cast<uint32_t>(nchunks);
  const uint32_t kb0 = static_cast<uint32_t>(split) * static_cast<uint32_t>(chunks_per_split);
  const uint32_t kb1 = kb0 + chunks_per_split < nch ? kb0 + chunks_per_split : nch;

  const auto a_rsrc = buffer_rsrc(A, static_cast<uint32_t>(M * lda * 2));
  const auto alo_rsrc = buffer_rsrc(static_cast<const uint8_t*>(A) + (MODE == GM_SPLIT ? M * lda * 2 : 0),
                                    MODE == GM_SPLIT ? static_cast<uint32_t>(M * lda * 2) : 0u);
  const auto q_rsrc = buffer_rsrc(qt, static_cast<uint32_t>(ntiles * nchunks * 1024));
  const uint32_t n_params = static_cast<uint32_t>(ntiles * nchunks * nbc * 16);
  const auto s_rsrc = buffer_rsrc(sc, n_params * SES);
  const uint32_t z_bytes = MODE == GM_SPLIT ? (zk == TMH_ZP_FLOAT ? n_params * 4 : zk == TMH_ZP_PACKED ? zp_byte<BITS>(n_params) : 0u)
                                            : (HAS_ZP ? zp_byte<BITS>(n_params) : 0u);
  const auto z_rsrc = buffer_rsrc(zp, z_bytes);
  const uint32_t zsh = zp_shift<BITS>(r);  // every entry this lane reads is one of row r

  // A loads of this wavefront: rows wave*RW + s*RPI + lane/PPR, LDS slot lane%PPR. Offsets are
  // formed per load (few live registers); rows at or past M lie outside the buffer range and
  // read zeros (their outputs are never stored).
  const int a_lrow = lane / PPR, a_lslot = lane % PPR;
  const uint32_t a_row0 = static_cast<uint32_t>(m0 + wave * RW + a_lrow) * static_cast<uint32_t>(lda) * 2;
  const uint32_t a_rstep = static_cast<uint32_t>(RPI) * static_cast<uint32_t>(lda) * 2;
  auto a_off = [&](int s2) -> uint32_t {
    const int piece = a_slot<BITS>(wave * RW + s2 * RPI + a_lrow, a_lslot);  // the swizzle is its own inverse
    return a_row0 + static_cast<uint32_t>(s2) * a_rstep + piece * 16;
  };
  auto load_a = [&](uint32_t kb, int buf, int s_lo = 0, int s_hi = 1 << 30) {
    uint8_t* base = lds + buf * ABUF + wave * RW * ROWB;
    if (static_cast<int64_t>(kb + 1) * CW <= K) {
#pragma unroll
      for (int s2 = 0; s2 < LOADS; ++s2)
        if (s2 >= s_lo && s2 < s_hi) {
          lds_dma16(a_rsrc, base + s2 * RPI * ROWB, a_off(s2), kb * (CW * 2));
          if constexpr (MODE == GM_SPLIT) lds_dma16(alo_rsrc, base + BM * ROWB + s2 * RPI * ROWB, a_off(s2), kb * (CW * 2));
        }
    } else {
      // (GM_SPLIT's A is zero-padded to whole chunks by k_split_a, so it never comes here.)
      // A k-block that reaches past K: through registers, zero past K. The whole offset is in
      // the VGPR operand so the buffer range check covers it.
#pragma unroll
      for (int s2 = 0; s2 < LOADS; ++s2) {
        if (s2 < s_lo || s2 >= s_hi) continue;
        const int row = wave * RW + s2 * RPI + a_lrow;
        const int piece = a_slot<BITS>(row, a_lslot);
        uint4_t v = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_off(s2) + kb * (CW * 2), 0, 0);
        if (static_cast<int64_t>(kb) * CW + piece * 8 >= K) v = uint4_t{0u, 0u, 0u, 0u};
        *reinterpret_cast<uint4_t*>(base + (s2 * RPI + a_lrow) * ROWB + a_lslot * 16) = v;
      }
    }
  };
  // This wavefront's four weight tiles and their parameters; tiles past N read zeros.
  const uint32_t b_base = (static_cast<uint32_t>(t0) * nch * 64 + lane) * 16, b_tstep = nch * 1024;
  const uint32_t p_base = (static_cast<uint32_t>(t0) * nch * nbc + ((g * GW) >> bsc_shift)) * 16 + r;
  const uint32_t p_tstep = nch * static_cast<uint32_t>(nbc) * 16;
  struct BStage {
    uint4_t w[NTW];
    uint32_t s[NJ][NTW];
    uint32_t z[NJ][NTW];
  };
  auto load_b = [&](uint32_t kb, BStage& st, int t_lo = 0, int t_hi = 1 << 30) {
    const uint32_t kofs = kb * static_cast<uint32_t>(nbc) * 16;
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      if (nt < t_lo || nt >= t_hi) continue;
      st.w[nt] = __builtin_amdgcn_raw_buffer_load_b128(q_rsrc, b_base + nt * b_tstep, kb * 1024, 0);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        uint32_t e = p_base + nt * p_tstep;
        if constexpr (SPLIT) e += static_cast<uint32_t>(((g * GW + 8 * j) >> bsc_shift) - ((g * GW) >> bsc_shift)) * 16;
        if constexpr (SES == 4) st.s[j][nt] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, e * 4, kofs * 4, 0);
        else st.s[j][nt] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, e * 2, kofs * 2, 0);
        if constexpr (MODE == GM_SPLIT) {
          // Float zero points are f32 per entry, packed ones BITS bits (a wavefront-uniform choice).
          if (zk == TMH_ZP_FLOAT) st.z[j][nt] = __builtin_amdgcn_raw_buffer_load_b32(z_rsrc, e * 4, kofs * 4, 0);
          else if (zk == TMH_ZP_PACKED) st.z[j][nt] = __builtin_amdgcn_raw_buffer_load_b8(z_rsrc, zp_byte<BITS>(e), zp_byte<BITS>(kofs), 0);
        } else if constexpr (HAS_ZP) {
          st.z[j][nt] = __builtin_amdgcn_raw_buffer_load_b8(z_rsrc, zp_byte<BITS>(e), zp_byte<BITS>(kofs), 0);
        }
      }
    }
  };

  float4_t acc[MTW][NTW];
#pragma unroll
  for (int a = 0; a < MTW; ++a)
#pragma unroll
    for (int b = 0; b < NTW; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto dequant = [&](const BStage& st, int i, half8_t (&bf)[NTW]) {
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int j = SPLIT ? i : 0;
      const uint32_t sv = st.s[j][nt];
      const uint32_t zv = HAS_ZP ? 0x6400u + zp_field<BITS>(st.z[j][nt], zsh) : 0x6400u + (1u << (BITS - 1));
      bf[nt] = unpack_step<BITS>(st.w[nt], i, __builtin_bit_cast(half2_t, zv | (zv << 16)),
                                 __builtin_bit_cast(half2_t, sv | (sv << 16)));
    }
  };
  // The next k-block's loads: the weights, scales and zero points (from HBM, the longest
  // latency) at the first step, the A tile (L2) spread over the steps so that the eight
  // wavefronts do not queue all of it on the CU's memory path at once after each barrier. The
  // barrier at the end of the k-block waits for all of them. (Weights issued after the A tile,
  // in the second half of the steps: 357 against 371 TFLOP/s over the SmolLM3-3B projections at
  // M = 256, the same at M = 2048.)
  auto issue = [&](int i, uint32_t kb, int buf, BStage& st) {
    if (i == 0) load_b(kb, st);
    load_a(kb, buf, i * LOADS / LSTEPS, (i + 1) * LOADS / LSTEPS);
  };
  // Software pipeline over the k-block's steps: once fragment mt of step i has fed its four
  // MFMAs, the same registers take fragment mt of step i+1 from LDS; step i+1's weights are
  // dequantized (into the other of two register sets) while step i's MFMAs run.
  // The scale and zero point of a parameter entry as f32 (the bf16 paths).
  auto scale_of = [&](uint32_t bits) -> float {
    if constexpr (MODE == GM_SPLIT && WT == DT_F32) return __builtin_bit_cast(float, bits);
    else if constexpr (MODE == GM_SPLIT && WT == DT_F16) return f16_bits_to_f32(static_cast<uint16_t>(bits));
    else return __builtin_bit_cast(float, bits << 16);  // bf16
  };
  auto zero_of = [&](uint32_t bits) -> float {
    constexpr float kDefault = static_cast<float>(1 << (BITS - 1));
    if constexpr (MODE == GM_SPLIT)
      return zk == TMH_ZP_FLOAT ? __builtin_bit_cast(float, bits)
                                : (zk == TMH_ZP_PACKED ? static_cast<float>(zp_field<BITS>(bits, zsh)) : kDefault);
    else return HAS_ZP ? static_cast<float>(zp_field<BITS>(bits, zsh)) : kDefault;
  };
  auto compute = [&](int buf, const BStage& st, bool more, uint32_t kbn, BStage& nst) {
    const uint8_t* abase = lds + buf * ABUF + (wm * 128 + r) * ROWB;
    if constexpr (MODE != GM_F16) {
      // The bf16 paths (tall layout): the step pipeline of the f16 path, with the weights
      // dequantized through f32 and, for GM_SPLIT, the hi and lo parts of A and of the weights
      // (three MFMAs per product).
      auto steps = [&](auto khc) {
        constexpr int KH = decltype(khc)::value;
#pragma unroll
        for (int li = 0; li < LSTEPS; ++li) {
          const int i = KH * LSTEPS + li;
          if (more) issue(li, kbn, buf ^ 1, nst);
          uint4_t bh[NTW], bl[NTW];
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) {
            const float s = scale_of(st.s[0][nt]), z = zero_of(st.z[0][nt]);
            if constexpr (MODE == GM_BF16) bh[nt] = dequant_bf16<BITS>(st.w[nt], i, s, -z * s);
            else dequant_split<BITS, WT>(st.w[nt], i, s, z, bh[nt], bl[nt]);
          }
          const int slot = a_slot<BITS>(r, g * (GW / 8) + i) * 16;
          uint4_t a = *reinterpret_cast<const uint4_t*>(abase + slot), al{};
          if constexpr (MODE == GM_SPLIT) al = *reinterpret_cast<const uint4_t*>(abase + BM * ROWB + slot);
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt) {
            uint4_t an{}, aln{};
            if (mt + 1 < MTW) {
              an = *reinterpret_cast<const uint4_t*>(abase + (mt + 1) * 16 * ROWB + slot);
              if constexpr (MODE == GM_SPLIT)
                aln = *reinterpret_cast<const uint4_t*>(abase + BM * ROWB + (mt + 1) * 16 * ROWB + slot);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
              acc[mt][nt] = gm_mma<MODE>(bh[nt], a, acc[mt][nt]);
              if constexpr (MODE == GM_SPLIT) {
                acc[mt][nt] = gm_mma<MODE>(bl[nt], a, acc[mt][nt]);
                acc[mt][nt] = gm_mma<MODE>(bh[nt], al, acc[mt][nt]);
              }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (mt + 1 < MTW) {
              a = an;
              if constexpr (MODE == GM_SPLIT) al = aln;
            }
          }
        }
      };
      if constexpr (KS == 1) {
        steps(std::integral_constant<int, 0>{});
      } else if (kh == 0) {
        steps(std::integral_constant<int, 0>{});
      } else {
        steps(std::integral_constant<int, 1>{});
      }
      return;
    } else if constexpr (TALL) {
      // Two wavefronts per SIMD: each keeps few registers live and relies on the other to fill
      // its waits; one set of weight fragments per step, A fragments read one ahead of use.
      // Step i = KH * LSTEPS + li stays a compile-time index (KH is the wavefront's half).
      auto steps = [&](auto khc) {
        constexpr int KH = decltype(khc)::value;
#pragma unroll
        for (int li = 0; li < LSTEPS; ++li) {
          const int i = KH * LSTEPS + li;
          if (more) issue(li, kbn, buf ^ 1, nst);
          half8_t bc[NTW];
          dequant(st, i, bc);
          // A fragment mt + 1 is read while fragment mt feeds its MFMAs; the scheduling
          // barriers keep the compiler from sinking each read next to its first use.
          const int slot = a_slot<BITS>(r, g * (GW / 8) + i) * 16;
          half8_t a = *reinterpret_cast<const half8_t*>(abase + slot);
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt) {
            half8_t an;
            if (mt + 1 < MTW) an = *reinterpret_cast<const half8_t*>(abase + (mt + 1) * 16 * ROWB + slot);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
              acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bc[nt], a, acc[mt][nt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (mt + 1 < MTW) a = an;
          }
        }
      };
      if constexpr (KS == 1) {
        steps(std::integral_constant<int, 0>{});
      } else if (kh == 0) {
        steps(std::integral_constant<int, 0>{});
      } else {
        steps(std::integral_constant<int, 1>{});
      }
      return;
    }
    half8_t af[8], b0[NTW], b1[NTW];
    {
      const int slot = a_slot<BITS>(r, g * (GW / 8)) * 16;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) af[mt] = *reinterpret_cast<const half8_t*>(abase + mt * 16 * ROWB + slot);
    }
    dequant(st, 0, b0);
#pragma unroll
    for (int i = 0; i < STEPS; ++i) {
      if (more) issue(i, kbn, buf ^ 1, nst);
      half8_t(&bc)[NTW] = (i & 1) ? b1 : b0;
      half8_t(&bn)[NTW] = (i & 1) ? b0 : b1;
      if (i + 1 < STEPS) dequant(st, i + 1, bn);
      const int slot = a_slot<BITS>(r, g * (GW / 8) + i + 1) * 16;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)  // weights as the first operand: lane holds 4 columns of one row
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bc[nt], af[mt], acc[mt][nt], 0, 0, 0);
        if (i + 1 < STEPS) af[mt] = *reinterpret_cast<const half8_t*>(abase + mt * 16 * ROWB + slot);
      }
    }
  };
  BStage cur, next;
  load_a(kb0, 0);
  load_b(kb0, cur);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // (A bare s_barrier after explicit waits, which keeps the next k-block's weight loads in flight
  // across the barrier where __syncthreads' fences make the compiler wait for them, with the loop
  // unrolled twice to avoid the stage copy, measured 3x slower on 11008 -> 2048: 228 VGPRs
  // instead of 142 at 128 rows, and worse at 256.)
  for (uint32_t kb = kb0; kb < kb1; ++kb) {
    const int buf = static_cast<int>((kb - kb0) & 1);
    const bool more = kb + 1 < kb1;
    compute(buf, cur, more, kb + 1, next);
    if (more) {
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    if (more) cur = next;
  }
  if constexpr (KS == 2) {
    // The second half's partial sums through LDS (free after the k-loop's last barrier: no
    // load into it is in flight) into the first half's; the first half stores.
    auto* part = reinterpret_cast<float4_t*>(lds);
    if (kh == 1) {
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) part[((wl * MTW + mt) * NTW + nt) * 64 + lane] = acc[mt][nt];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] += part[((wl * MTW + mt) * NTW + nt) * 64 + lane];
    }
  }
  // Lane (16g + r) holds, for each (mt, nt), row mt*16 + r and the 4 columns nt*16 + 4g ...
  // Two-byte outputs without a bias: f16 (the f16 and split paths) or bf16 (the bf16 path).
  constexpr int HDT = MODE == GM_BF16 ? DT_BF16 : DT_F16;
  const bool f16_out = y_dt == HDT && dot_dt == HDT && !bias;
  const bool vec_out = (ldy % 4) == 0;
  auto pack4 = [](float4_t v) -> uint2 {
    if constexpr (HDT == DT_BF16) return make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
    const half2_t lo = {static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1])};
    const half2_t hi = {static_cast<_Float16>(v[2]), static_cast<_Float16>(v[3])};
    return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
  };
  // Whole tiles of f32 partial sums, or of f16 outputs with 16-byte aligned rows, go out through
  // LDS: each wavefront writes its accumulators there in the MFMA layout, then every thread
  // stores 16 contiguous bytes of a row, so a store instruction writes whole cache lines (from
  // the MFMA layout a lane holds 4 columns: 16 rows x 8 or 16 bytes per instruction). The tile
  // goes in passes of as many rows as the LDS holds; 16-byte units are XOR-swizzled by row.
  // (Stores measured 4-9% of the SmolLM3-3B projections at M = 2048, 25% at M = 256; f32
  // partial sums that need two passes were slower staged than stored directly, 16 bytes a lane.
  // The f16 rows store non-temporally: 2048 -> 11008 at M = 2048, 45 MB out, 109.8 -> 107.9 us;
  // the partial sums, read back by the reduction, gain nothing from it.)
  constexpr bool kPartialsFit = static_cast<int>(gemm_lds_bytes<BITS, BM, KS, MODE>()) >= BM * 64 * WN * 4;
  // The partial sums go out written through the L2 (kWriteThrough) where one split's M x N fits
  // a buffer's 32-bit offsets: otherwise they sit dirty in the L2 until the kernel's end, whose
  // write-back the reduction's launch waits for (2048 -> 2048 at M = 256, 8 MB of partial sums:
  // 63.4 -> 61.2 us per four calls; 11008 -> 2048, M = 256: 109.7 -> 104.5 us).
  const bool wt_ok = ws && M * N * 4 < (int64_t(1) << 31);
  const auto wt_rsrc = buffer_rsrc(ws ? ws + static_cast<int64_t>(split) * M * N : ws,
                                   wt_ok ? static_cast<uint32_t>(M * N * 4) : 0u);
  const bool staged = ws ? kPartialsFit && (N % 4) == 0
                         : f16_out && (ldy % 8) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
  if (staged) {
    auto out_tile = [&](auto esz_c) {
      constexpr int ESZ = decltype(esz_c)::value;  // bytes per output: 4 (partial sums) or 2 (f16)
      constexpr int BN = 64 * WN;
      constexpr int RS = BN * ESZ;  // bytes per staged row
      constexpr int UPR = RS / 16;  // 16-byte units per row
      constexpr int CAP = static_cast<int>(gemm_lds_bytes<BITS, BM, KS, MODE>());
      constexpr int RPP = CAP / RS >= BM ? BM : CAP / RS;  // rows per pass
      static_assert(RPP >= 16 && BM % RPP == 0 && UPR >= 8, "staging shape");
      constexpr int NTHR = 128 * WN * KS;
      const int col0 = nb * BN;
      for (int pass = 0; pass < BM / RPP; ++pass) {
        __syncthreads();  // the LDS is free: A tiles, partial sums or the previous pass are read
        if (KS == 1 || kh == 0) {
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt) {
            const int row = wm * 128 + mt * 16;  // the 16 rows of fragment mt lie in one pass
            if (row / RPP != pass) continue;
            const int prow = row % RPP + r;
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
              const int byte = ((t0 + nt) * 16 + 4 * g - col0) * ESZ;
              uint8_t* p = lds + prow * RS + (((byte >> 4) ^ (prow & 7)) << 4) + (byte & 15);
              const float4_t v = acc[mt][nt];
              if constexpr (ESZ == 4) {
                *reinterpret_cast<float4_t*>(p) = v;
              } else {
                *reinterpret_cast<uint2*>(p) = pack4(v);
              }
            }
          }
        }
        __syncthreads();
        for (int idx = tid; idx < RPP * UPR; idx += NTHR) {
          const int prow = idx / UPR, unit = idx % UPR;
          const int64_t m = m0 + pass * RPP + prow;
          const int64_t n = col0 + unit * (16 / ESZ);
          if (m >= M || n >= N) continue;
          const uint4_t v = *reinterpret_cast<const uint4_t*>(lds + prow * RS + ((unit ^ (prow & 7)) << 4));
          if constexpr (ESZ == 4) {
            float* dst = ws + (static_cast<int64_t>(split) * M + m) * N + n;
            if (n + 4 <= N && wt_ok) {
              __builtin_amdgcn_raw_buffer_store_b128(v, wt_rsrc, static_cast<uint32_t>((m * N + n) * 4), 0, kWriteThrough);
            } else if (n + 4 <= N) {
              *reinterpret_cast<uint4_t*>(dst) = v;
            } else {
              const float4_t f = __builtin_bit_cast(float4_t, v);  // whole vector: hipcc 7.2 miscompiled element casts
              for (int e = 0; e < 4 && n + e < N; ++e) dst[e] = f[e];
            }
          } else {
            uint16_t* dst = static_cast<uint16_t*>(Y) + m * ldy + n;
            if (n + 8 <= N) {
              __builtin_nontemporal_store(v, reinterpret_cast<uint4_t*>(dst));
            } else {
              const uint32_t words[4] = {v[0], v[1], v[2], v[3]};
              for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = static_cast<uint16_t>(words[e >> 1] >> ((e & 1) * 16));
            }
          }
        }
      }
    };
    if (ws)
      out_tile(std::integral_constant<int, 4>{});
    else
      out_tile(std::integral_constant<int, 2>{});
    if constexpr (TL) tl_stamp(tl, tl0);
    return;
  }
  if (KS == 2 && kh == 1) {
    if constexpr (TL) tl_stamp(tl, tl0);
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) {
    const int64_t m = m0 + wm * 128 + mt * 16 + r;
    if (m >= M) continue;
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int64_t n = static_cast<int64_t>(t0 + nt) * 16 + 4 * g;
      if (n >= N) continue;
      const float4_t v = acc[mt][nt];
      if (ws) {
        float* dst = ws + (static_cast<int64_t>(split) * M + m) * N + n;
        if (n + 4 <= N && (N % 4) == 0 && wt_ok) {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uint4_t, v), wt_rsrc,
                                                 static_cast<uint32_t>((m * N + n) * 4), 0, kWriteThrough);
        } else if (n + 4 <= N && (N % 4) == 0) {
          *reinterpret_cast<float4_t*>(dst) = v;
        } else {
          for (int e = 0; e < 4 && n + e < N; ++e) dst[e] = v[e];
        }
        continue;
      }
      if (f16_out && vec_out && n + 4 <= N) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(Y) + m * ldy + n) = pack4(v);
        continue;
      }
      if (MODE == GM_SPLIT && y_dt == DT_F32 && dot_dt == DT_F32 && !bias && vec_out && n + 4 <= N &&
          (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {
        *reinterpret_cast<float4_t*>(static_cast<float*>(Y) + m * ldy + n) = v;
        continue;
      }
      store_quad_any(v, Y, y_dt, dot_dt, bias, bias_dt, m * ldy, n, N);
    }
  }
  if constexpr (TL) tl_stamp(tl, tl0);
}

template <int BITS, bool HAS_ZP, bool SPLIT, int WN, int BM, int KS, int MODE = GM_F16, int WT = DT_F16>
__global__ __launch_bounds__(128 * WN * KS) void k_gemm_lds(
    const uint4_t* __restrict__ qt, const void* __restrict__ sc, const void* __restrict__ zp,
    const void* __restrict__ A, int64_t M, int64_t K, int64_t lda, const void* __restrict__ bias,
    int bias_dt, void* __restrict__ Y, int y_dt, int dot_dt, int64_t ldy, int64_t N, int64_t ntiles,
    int64_t nchunks, int nbc, int bsc_shift, int mblocks, int nblocks, int chunks_per_split,
    float* __restrict__ ws, int zk) {
  gemm_lds<BITS, HAS_ZP, SPLIT, WN, BM, KS, false, MODE, WT>(qt, sc, zp, A, M, K, lda, bias, bias_dt, Y, y_dt, dot_dt,
                                                             ldy, N, ntiles, nchunks, nbc, bsc_shift, mblocks, nblocks,
                                                             chunks_per_split, ws, zk, nullptr);
}

template <int BITS, bool HAS_ZP, bool SPLIT, int WN, int BM, int KS, int MODE = GM_F16, int WT = DT_F16>
__global__ __launch_bounds__(128 * WN * KS) void k_gemm_lds_tl(
    const uint4_t* __restrict__ qt, const void* __restrict__ sc, const void* __restrict__ zp,
    const void* __restrict__ A, int64_t M, int64_t K, int64_t lda, const void* __restrict__ bias,
    int bias_dt, void* __restrict__ Y, int y_dt, int dot_dt, int64_t ldy, int64_t N, int64_t ntiles,
    int64_t nchunks, int nbc, int bsc_shift, int mblocks, int nblocks, int chunks_per_split,
    float* __restrict__ ws, int zk, uint32_t* __restrict__ tl) {
  gemm_lds<BITS, HAS_ZP, SPLIT, WN, BM, KS, true, MODE, WT>(qt, sc, zp, A, M, K, lda, bias, bias_dt, Y, y_dt, dot_dt,
                                                            ldy, N, ntiles, nchunks, nbc, bsc_shift, mblocks, nblocks,
                                                            chunks_per_split, ws, zk, tl);
}

// GM_SPLIT's A operand: A [M, K] of type ADT (rows lda apart) as bf16 hi = bf16(a) and lo =
// bf16(a - hi) (a - hi is exact in f32), each [M, Kp] with the rows zero-padded from K to Kp
// (whole chunks), the lo rows after all the hi rows. One thread per 8 consecutive values of a row.
template <int ADT>
__global__ __launch_bounds__(256) void k_split_a(const void* __restrict__ A, int64_t M, int64_t K, int64_t lda,
                                                 int64_t Kp, uint16_t* __restrict__ out) {
  const int64_t per_row = Kp / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= M * per_row) return;
  const int64_t m = idx / per_row, k0 = (idx - m * per_row) * 8;
  uint4_t hi, lo;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t k = k0 + 2 * j;
    const float x0 = k < K ? load_as_f32<ADT>(A, m * lda + k) : 0.f;
    const float x1 = k + 1 < K ? load_as_f32<ADT>(A, m * lda + k + 1) : 0.f;
    const uint32_t h = pack_bf16(x0, x1);
    hi[j] = h;
    lo[j] = pack_bf16(x0 - __builtin_bit_cast(float, h << 16), x1 - __builtin_bit_cast(float, h & 0xFFFF0000u));
  }
  *reinterpret_cast<uint4_t*>(out + m * Kp + k0) = hi;
  *reinterpret_cast<uint4_t*>(out + (M + m) * Kp + k0) = lo;
}

// Split-K epilogue: Y = sum over the splits of ws[split][M][N] (in split order), rounded to the
// dot type, plus the bias, in Y's type. Four consecutive outputs per thread.
__device__ __forceinline__ void splitk_reduce_quads(const float* __restrict__ ws, int splits, int64_t M, int64_t N,
                                                    const void* __restrict__ bias, int bias_dt, void* __restrict__ Y,
                                                    int y_dt, int dot_dt, int64_t ldy);

template <bool TL>
__device__ __forceinline__ void splitk_reduce(const float* __restrict__ ws, int splits, int64_t M, int64_t N,
                                              const void* __restrict__ bias, int bias_dt, void* __restrict__ Y,
                                              int y_dt, int dot_dt, int64_t ldy, uint32_t* __restrict__ tl) {
  const TlStart tl0 = TL ? tl_clock() : TlStart{0u, 0u};
  splitk_reduce_quads(ws, splits, M, N, bias, bias_dt, Y, y_dt, dot_dt, ldy);
  if constexpr (TL) tl_stamp(tl, tl0);
}

__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ ws, int splits, int64_t M, int64_t N,
                                                       const void* __restrict__ bias, int bias_dt, void* __restrict__ Y,
                                                       int y_dt, int dot_dt, int64_t ldy) {
  splitk_reduce<false>(ws, splits, M, N, bias, bias_dt, Y, y_dt, dot_dt, ldy, nullptr);
}

__global__ __launch_bounds__(256) void k_splitk_reduce_tl(const float* __restrict__ ws, int splits, int64_t M, int64_t N,
                                                          const void* __restrict__ bias, int bias_dt,
                                                          void* __restrict__ Y, int y_dt, int dot_dt, int64_t ldy,
                                                          uint32_t* __restrict__ tl) {
  splitk_reduce<true>(ws, splits, M, N, bias, bias_dt, Y, y_dt, dot_dt, ldy, tl);
}

// One thread's four consecutive outputs (the body of k_splitk_reduce).
__device__ __forceinline__ void splitk_reduce_quads(const float* __restrict__ ws, int splits, int64_t M, int64_t N,
                                                    const void* __restrict__ bias, int bias_dt, void* __restrict__ Y,
                                                    int y_dt, int dot_dt, int64_t ldy) {
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const int64_t total = M * N;
  if (i4 >= total) return;
  const bool vec = (N % 4) == 0;
  if (vec) {
    float4_t v = *reinterpret_cast<const float4_t*>(ws + i4);
    for (int sp = 1; sp < splits; ++sp) v += *reinterpret_cast<const float4_t*>(ws + sp * total + i4);
    const int64_t m = i4 / N, n = i4 - m * N;
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = round_dot(v[e], dot_dt);
      if (bias) x[e] += load_float_rt(bias, bias_dt, n + e);
    }
    if (y_dt == DT_F16 && ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(Y) & 7) == 0) {
      // Four f16 outputs in one 8-byte store.
      const uint32_t lo = f32_to_f16_bits(x[0]) | (static_cast<uint32_t>(f32_to_f16_bits(x[1])) << 16);
      const uint32_t hi = f32_to_f16_bits(x[2]) | (static_cast<uint32_t>(f32_to_f16_bits(x[3])) << 16);
      *reinterpret_cast<uint64_t*>(static_cast<uint16_t*>(Y) + m * ldy + n) =
          static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
      return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) store_float_rt(Y, y_dt, m * ldy + n + e, x[e]);
    return;
  }
  for (int64_t i = i4; i < i4 + 4 && i < total; ++i) {
    float x = ws[i];
    for (int sp = 1; sp < splits; ++sp) x += ws[sp * total + i];
    const int64_t m = i / N, n = i - m * N;
    x = round_dot(x, dot_dt);
    if (bias) x += load_float_rt(bias, bias_dt, n);
    store_float_rt(Y, y_dt, m * ldy + n, x);
  }
}

// Any float types: the weights dequantize bit-exactly in WDT, then f32 FMA with A.
// Block (t, y): rows 4*y .. 4*y+3 of A against the 16 columns of tile t.
constexpr int kGeneralRows = 4;

template <int BITS, int WDT, int ZK>
__global__ __launch_bounds__(256) void k_matmul_general(
    const uint4_t* __restrict__ qt, const void* __restrict__ sc, const void* __restrict__ zp,
    const void* __restrict__ A, int a_dt, int64_t M, int64_t K, int64_t lda,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ Y, int y_dt, int dot_dt,
    int64_t ldy, int64_t N, int64_t nchunks, int nbc, int bsc_shift) {
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int PER_WORD = 32 / BITS;
  __shared__ float red[kWaves][kGeneralRows][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t t = blockIdx.x;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kGeneralRows;
  const int64_t mcount = M - m0 < kGeneralRows ? M - m0 : kGeneralRows;
  float acc[kGeneralRows] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t c = wave; c < nchunks; c += kWaves) {
    const int64_t tc = t * nchunks + c;
    const uint4_t w = qt[tc * 64 + lane];
    for (int e = 0; e < GW; ++e) {
      const int64_t k = c * CW + g * GW + e;
      if (k >= K) break;
      const int woff = g * GW + e;
      const int64_t p = (tc * nbc + (woff >> bsc_shift)) * 16 + r;
      const float s = load_as_f32<WDT>(sc, p);
      float z;
      if constexpr (ZK == TMH_ZP_PACKED) {
        const uint8_t byte = static_cast<const uint8_t*>(zp)[zp_byte<BITS>(p)];
        z = static_cast<float>(zp_field<BITS>(byte, zp_shift<BITS>(static_cast<uint32_t>(p))));
      } else if constexpr (ZK == TMH_ZP_FLOAT) {
        z = static_cast<const float*>(zp)[p];
      } else {
        z = static_cast<float>(1 << (BITS - 1));
      }
      const uint32_t word = w[e / PER_WORD];
      const float wv = dequant_value<WDT>(static_cast<float>(word_value<BITS>(word, e % PER_WORD)), z, s);
#pragma unroll
      for (int mm = 0; mm < kGeneralRows; ++mm)
        if (mm < mcount) acc[mm] = fmaf(load_float_rt(A, a_dt, (m0 + mm) * lda + k), wv, acc[mm]);
    }
  }
#pragma unroll
  for (int mm = 0; mm < kGeneralRows; ++mm) {
    float v = acc[mm];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (g == 0) red[wave][mm][r] = v;
  }
  __syncthreads();
  if (wave == 0 && g == 0) {
    const int64_t n = t * 16 + r;
    if (n < N) {
      const float b = bias ? load_float_rt(bias, bias_dt, n) : 0.0f;
      for (int mm = 0; mm < mcount; ++mm) {
        float v = red[0][mm][r] + red[1][mm][r] + red[2][mm][r] + red[3][mm][r];
        if (dot_dt == DT_F16) v = round_to<DT_F16>(v);
        else if (dot_dt == DT_BF16) v = round_to<DT_BF16>(v);
        if (bias) v += b;
        store_float_rt(Y, y_dt, (m0 + mm) * ldy + n, v);
      }
    }
  }
}

// ------------------------------------------------------------------ launch helpers

template <int BITS, int WDT, int OUT>
void launch_dequant_zk(const tmh_weight* w, void* out, hipStream_t s, int bsc_shift) {
  const int64_t lanes = w->ntiles * w->nchunks * 64;
  const dim3 grid(static_cast<unsigned>((lanes + 255) / 256));
  const auto* qt = reinterpret_cast<const uint4_t*>(w->d_q);
  switch (w->zp_kind) {
    case TMH_ZP_PACKED:
      k_dequant<BITS, WDT, OUT, TMH_ZP_PACKED><<<grid, 256, 0, s>>>(qt, w->d_scale, w->d_zero, out, w->N, w->K, w->nchunks, w->nbc, bsc_shift, lanes);
      break;
    case TMH_ZP_FLOAT:
      k_dequant<BITS, WDT, OUT, TMH_ZP_FLOAT><<<grid, 256, 0, s>>>(qt, w->d_scale, w->d_zero, out, w->N, w->K, w->nchunks, w->nbc, bsc_shift, lanes);
      break;
    default:
      k_dequant<BITS, WDT, OUT, TMH_ZP_NONE><<<grid, 256, 0, s>>>(qt, w->d_scale, w->d_zero, out, w->N, w->K, w->nchunks, w->nbc, bsc_shift, lanes);
  }
}

template <int BITS, int WDT>
void launch_dequant_out(const tmh_weight* w, void* out, int out_dt, hipStream_t s, int bsc_shift) {
  switch (out_dt) {
    case TMH_F16: launch_dequant_zk<BITS, WDT, DT_F16>(w, out, s, bsc_shift); break;
    case TMH_BF16: launch_dequant_zk<BITS, WDT, DT_BF16>(w, out, s, bsc_shift); break;
    default: launch_dequant_zk<BITS, WDT, DT_F32>(w, out, s, bsc_shift);
  }
}

template <int BITS>
void launch_dequant_bits(const tmh_weight* w, void* out, int out_dt, hipStream_t s, int bsc_shift) {
  switch (w->wdtype) {
    case TMH_F16: launch_dequant_out<BITS, DT_F16>(w, out, out_dt, s, bsc_shift); break;
    case TMH_BF16: launch_dequant_out<BITS, DT_BF16>(w, out, out_dt, s, bsc_shift); break;
    default: launch_dequant_out<BITS, DT_F32>(w, out, out_dt, s, bsc_shift);
  }
}

struct MatArgs {
  const void* a;
  int a_dt;
  int64_t M, lda;
  bool a_vec;
  const void* bias;
  int bias_dt;
  void* y;
  int y_dt, dot_dt;
  int64_t ldy;
  float* ws = nullptr;       // split-K partial sums (gemm_scratch), resolved by the entry point
  void* a_split = nullptr;   // GM_SPLIT's hi and lo rows of A (gemm_scratch)
  size_t split_cap = SIZE_MAX;  // most bytes of partial sums the plan may use
  bool no_split_a = false;   // no scratch memory for GM_SPLIT's rows of A: the general kernel runs
};

int bsc_shift_of(const tmh_weight* w) {
  const int cw = chunk_weights(w->bits);
  return ilog2(std::min(w->block_size, cw));
}

// True when a lane's k-group of one chunk spans more than one block (parameters per step).
bool split_params(const tmh_weight* w) { return w->block_size < chunk_weights(w->bits) / 4; }

template <int BITS, int MT, bool HAS_ZP, bool SPLIT, int U>
void launch_gemv_u(const tmh_weight* w, const MatArgs& a, hipStream_t s, int waves) {
  const int64_t mblocks = (a.M + 16 * MT - 1) / (16 * MT);
  const dim3 grid(static_cast<unsigned>(w->ntiles), static_cast<unsigned>(mblocks));
  const size_t lds = static_cast<size_t>(waves) * MT * 64 * sizeof(float4_t);
  k_gemv_f16<BITS, MT, HAS_ZP, SPLIT, U><<<grid, 64 * waves, lds, s>>>(
      reinterpret_cast<const uint4_t*>(w->d_q), static_cast<const uint16_t*>(w->d_scale),
      static_cast<const uint8_t*>(w->d_zero), static_cast<const _Float16*>(a.a), a.M, w->K, a.lda,
      a.a_vec, a.bias, a.bias_dt, a.y, a.y_dt, a.dot_dt, a.ldy, w->N, w->nchunks, w->nbc,
      bsc_shift_of(w));
}

// Chunks per wavefront round (U) and wavefronts per block: up to 16 wavefronts, each with
// 1, 2 or 4 chunk loads in flight, so that K of up to 64 chunks needs one round.
template <int BITS, int MT, bool HAS_ZP, bool SPLIT>
void launch_gemv(const tmh_weight* w, const MatArgs& a, hipStream_t s, int num_cus) {
  const int64_t c = w->nchunks;
  // The decode GEMV (tmh_gemv.hip): f16 Y without bias or with an f16 one, aligned A, 32-bit
  // offsets.
  if (MT == 1 && a.y_dt == TMH_F16 && a.dot_dt == TMH_F16 && (!a.bias || a.bias_dt == TMH_F16) &&
      decode_gemv_ok(w, a.M, a.lda, a.ldy, a.a, a.y)) {
    launch_decode_gemv(w, a.a, a.M, a.lda, a.y, a.ldy, s, num_cus, a.bias);
    return;
  }
  if (c <= 16) {
    launch_gemv_u<BITS, MT, HAS_ZP, SPLIT, 1>(w, a, s, static_cast<int>(c));
  } else if (c <= 32) {
    launch_gemv_u<BITS, MT, HAS_ZP, SPLIT, 2>(w, a, s, static_cast<int>((c + 1) / 2));
  } else {
    launch_gemv_u<BITS, MT, HAS_ZP, SPLIT, 4>(w, a, s, static_cast<int>(std::min<int64_t>(16, (c + 3) / 4)));
  }
}

template <int BITS, bool HAS_ZP, bool SPLIT>
void launch_gemm(const tmh_weight* w, const MatArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((w->ntiles + 7) / 8), static_cast<unsigned>((a.M + 127) / 128));
  k_gemm_f16<BITS, HAS_ZP, SPLIT><<<grid, kThreads, 0, s>>>(
      reinterpret_cast<const uint4_t*>(w->d_q), static_cast<const uint16_t*>(w->d_scale),
      static_cast<const uint8_t*>(w->d_zero), static_cast<const _Float16*>(a.a), a.M, w->K, a.lda,
      a.a_vec, a.bias, a.bias_dt, a.y, a.y_dt, a.dot_dt, a.ldy, w->N, w->ntiles, w->nchunks, w->nbc,
      bsc_shift_of(w));
}

// Split K when the output tiles cannot fill the GPU: partial sums go to the context's
// workspace (tmh_matmul_nbits) or the fixed per-device scratch (tmh_matmul_nbits_noalloc) and
// k_splitk_reduce adds them. During stream capture the workspace cannot grow, so a captured
// tmh_matmul_nbits that finds it too small fails rather than running a different plan.
// Tile shape and K split of one prefill GEMM. Each candidate (BM x 64*WN tiles; KS = 2 for the
// 128x128 tile on eight wavefronts that split each k-block's steps; 1-16 splits of K) is priced
// as rounds of workgroups over the CUs times the work of one, at the per-CU rate the tile shape
// sustains on MI355X with every CU busy (dense f16 TFLOP/s per CU, measured on the SmolLM3-3B
// and 2048x4096x8192 shapes; with these rates the plan chosen for each SmolLM3-3B projection at
// M = 256 and 2048 was the fastest of the candidates timed, or within 6% of it), plus the f32
// partial sums a split writes and the reduction reads back.
// TMH_GEMM_PLAN="bm,wn,splits[,ks]" in the environment forces a plan (tests use it to reach every
// tile shape; an invalid value is ignored).
struct GemmShape {
  int bm, wn, ks;
  double rate;  // dense f16 FLOP/s per CU
};
constexpr GemmShape kGemmShapes[] = {
    {256, 2, 1, 2.8e12}, {256, 4, 1, 3.9e12}, {128, 2, 1, 2.4e12}, {128, 4, 1, 3.3e12}, {128, 2, 2, 2.9e12},
    {64, 2, 1, 1.6e12},  {64, 4, 1, 2.0e12},  {64, 2, 2, 2.0e12}};

struct GemmPlan {
  int bm, wn, splits, cps, ks = 1;
};

int cus_of(const tmh_ctx* ctx) { return ctx->num_cus > 0 ? ctx->num_cus : 256; }

// gemm_lds_bytes at run time.
size_t gemm_lds_bytes_rt(int bits, int bm, int ks, int mode) {
  const size_t a_tiles = 2 * static_cast<size_t>(bm) * (512 / bits) * 2 * (mode == GM_SPLIT ? 2 : 1);
  const size_t partial = ks > 1 ? static_cast<size_t>(bm) * 128 * sizeof(float) : 0;
  return std::max(a_tiles, partial);
}

// The tile shapes each operand path is built for: every shape for f16 operands; the tall shapes
// 128x128 and 64x128 on eight wavefronts for the bf16 paths (their 256x256 tile spills registers);
// none whose A buffers exceed 128 KiB of LDS (2-bit rows are 512 bytes, and GM_SPLIT keeps two tiles).
bool shape_built(int bits, int bm, int wn, int ks, int mode) {
  if (gemm_lds_bytes_rt(bits, bm, ks, mode) > 128 * 1024) return false;
  const bool eight = (bm == 128 || bm == 64) && ((wn == 2 && ks == 2) || (wn == 4 && ks == 1));
  if (mode == GM_BF16) return eight;
  if (mode == GM_SPLIT) return eight && wn == 2;
  return true;
}

// split_cap bounds the f32 partial sums a split plan keeps (splits * M * N * 4 bytes): plans
// beyond it are not considered, a forced one included. The bf16 path is priced at the f16 rates
// and GM_SPLIT at a third of them (three MFMAs per product).
GemmPlan plan_gemm(int64_t M, int64_t N, int64_t ntiles, int64_t nchunks, int bits, int cus,
                   size_t split_cap = SIZE_MAX, int mode = GM_F16) {
  auto fits = [&](int64_t splits) {
    return splits == 1 ||
           static_cast<double>(splits) * static_cast<double>(M) * static_cast<double>(N) * 4.0 <= static_cast<double>(split_cap);
  };
  const double cw = 512.0 / bits;
  const double slow = mode == GM_SPLIT ? 3.0 : 1.0;
  GemmPlan best{128, 2, 1, static_cast<int>(nchunks), 2};
  double best_t = 1e30;
  for (const GemmShape& sh : kGemmShapes) {
    if (!shape_built(bits, sh.bm, sh.wn, sh.ks, mode)) continue;
    const int64_t mblocks = (M + sh.bm - 1) / sh.bm;
    const int64_t tiles = mblocks * ((ntiles + 4 * sh.wn - 1) / (4 * sh.wn));
    const double chunk_s = slow * 2.0 * sh.bm * 64.0 * sh.wn * cw / sh.rate;
    for (int64_t splits = 1; splits <= 16; ++splits) {
      if (splits > 1 && 2 * splits > nchunks) break;
      const int64_t cps = (nchunks + splits - 1) / splits;
      const int64_t used = (nchunks + cps - 1) / cps;
      if (used != splits || !fits(splits)) continue;
      // A last round that occupies a fraction f of the CUs runs each workgroup faster (less
      // memory contention, a higher clock): priced at 0.6 + 0.4 f of a full round.
      const int64_t wgs = tiles * splits, full = wgs / cus, rem = wgs % cus;
      const double rounds = static_cast<double>(full) + (rem ? 0.6 + 0.4 * static_cast<double>(rem) / cus : 0.0);
      double t = rounds * cps * chunk_s;
      if (splits > 1) t += 2.0 * splits * M * N * 4 / 5e12;
      if (t < best_t) {
        best_t = t;
        best = GemmPlan{sh.bm, sh.wn, static_cast<int>(splits), static_cast<int>(cps), sh.ks};
      }
    }
  }
  if (const char* f = getenv("TMH_GEMM_PLAN")) {
    int bm = 0, wn = 0, sp = 0, ks = 1;
    const int got = sscanf(f, "%d,%d,%d,%d", &bm, &wn, &sp, &ks);
    if ((got == 3 || got == 4) && (bm == 64 || bm == 128 || bm == 256) && (wn == 2 || wn == 4) && sp >= 1 &&
        sp <= nchunks && (ks == 1 || (ks == 2 && bm <= 128 && wn == 2)) && shape_built(bits, bm, wn, ks, mode)) {
      const int cps = static_cast<int>((nchunks + sp - 1) / sp);
      const int used = static_cast<int>((nchunks + cps - 1) / cps);
      if (fits(used)) best = GemmPlan{bm, wn, used, cps, ks};
    }
  }
  return best;
}

// A operand of one GEMM launch: the caller's A, or GM_SPLIT's hi/lo rows (K padded to whole chunks).
struct GemmA {
  const void* a;
  int64_t K, lda;
};

template <int BITS, bool HAS_ZP, bool SPLIT, int WN, int BM, int KS = 1, int MODE = GM_F16, int WT = DT_F16>
void launch_gemm_lds_wn(const tmh_weight* w, const MatArgs& a, const GemmA& ga, hipStream_t s, int splits, int cps) {
  const int mblocks = static_cast<int>((a.M + BM - 1) / BM);
  const int nblocks = static_cast<int>((w->ntiles + 4 * WN - 1) / (4 * WN));
  const int64_t tiles = static_cast<int64_t>(mblocks) * nblocks;
  // The entry point provides the partial sums (gemm_scratch) whenever the plan splits K.
  float* ws = splits > 1 ? a.ws : nullptr;
  const dim3 grid(static_cast<unsigned>(tiles * splits));
  constexpr int kLds = static_cast<int>(gemm_lds_bytes<BITS, BM, KS, MODE>());
  static_assert(kLds <= 128 * 1024, "the A buffers must fit 128 KiB of LDS");
  static const hipError_t attr[2] = {
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_lds<BITS, HAS_ZP, SPLIT, WN, BM, KS, MODE, WT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kLds),
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_lds_tl<BITS, HAS_ZP, SPLIT, WN, BM, KS, MODE, WT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kLds)};
  (void)attr;
#define TMH_GEMM_ARGS                                                                                               \
  reinterpret_cast<const uint4_t*>(w->d_q), w->d_scale, w->d_zero, ga.a, a.M, ga.K, ga.lda, a.bias, a.bias_dt, a.y, \
      a.y_dt, a.dot_dt, a.ldy, w->N, w->ntiles, w->nchunks, w->nbc, bsc_shift_of(w), mblocks, nblocks, cps, ws,    \
      w->zp_kind
  if (uint32_t* tl = timeline_slots(TMH_TL_GEMM_LDS, static_cast<int64_t>(grid.x) * 2 * WN * KS))
    k_gemm_lds_tl<BITS, HAS_ZP, SPLIT, WN, BM, KS, MODE, WT><<<grid, 128 * WN * KS, kLds, s>>>(TMH_GEMM_ARGS, tl);
  else
    k_gemm_lds<BITS, HAS_ZP, SPLIT, WN, BM, KS, MODE, WT><<<grid, 128 * WN * KS, kLds, s>>>(TMH_GEMM_ARGS);
#undef TMH_GEMM_ARGS
  if (ws) {
    const int64_t quads = (a.M * w->N + 3) / 4;
    const unsigned rgrid = static_cast<unsigned>((quads + 255) / 256);
    if (uint32_t* tl = timeline_slots(TMH_TL_SPLITK_REDUCE, static_cast<int64_t>(rgrid) * 4))
      k_splitk_reduce_tl<<<rgrid, 256, 0, s>>>(ws, splits, a.M, w->N, a.bias, a.bias_dt, a.y, a.y_dt, a.dot_dt, a.ldy,
                                              tl);
    else
      k_splitk_reduce<<<rgrid, 256, 0, s>>>(ws, splits, a.M, w->N, a.bias, a.bias_dt, a.y, a.y_dt, a.dot_dt, a.ldy);
  }
}

// Launches the plan's tile shape (only shapes shape_built() allows reach here).
template <int BITS, bool HAS_ZP, bool SPLIT, int MODE = GM_F16, int WT = DT_F16>
void launch_gemm_plan(const tmh_weight* w, const MatArgs& a, const GemmA& ga, hipStream_t s, const GemmPlan& p) {
  if (p.bm == 64 && p.ks == 2) {
    launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 2, 64, 2, MODE, WT>(w, a, ga, s, p.splits, p.cps);
  } else if (p.bm == 128 && p.ks == 2) {
    if constexpr (gemm_lds_bytes<BITS, 128, 2, MODE>() <= 128 * 1024)
      launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 2, 128, 2, MODE, WT>(w, a, ga, s, p.splits, p.cps);
  } else if constexpr (MODE == GM_BF16) {
    if (p.bm == 128) {
      if constexpr (gemm_lds_bytes<BITS, 128, 1, MODE>() <= 128 * 1024)
        launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 4, 128, 1, MODE, WT>(w, a, ga, s, p.splits, p.cps);
    } else {
      launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 4, 64, 1, MODE, WT>(w, a, ga, s, p.splits, p.cps);
    }
  } else if constexpr (MODE == GM_F16) {
    if (p.bm == 64) {
      if (p.wn == 4)
        launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 4, 64>(w, a, ga, s, p.splits, p.cps);
      else
        launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 2, 64>(w, a, ga, s, p.splits, p.cps);
    } else if (p.bm == 128) {
      if (p.wn == 4)
        launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 4, 128>(w, a, ga, s, p.splits, p.cps);
      else
        launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 2, 128>(w, a, ga, s, p.splits, p.cps);
    } else if constexpr (BITS != 2) {
      if (p.wn == 4)
        launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 4, 256>(w, a, ga, s, p.splits, p.cps);
      else
        launch_gemm_lds_wn<BITS, HAS_ZP, SPLIT, 2, 256>(w, a, ga, s, p.splits, p.cps);
    }
  }
}

// f16 A, f16 weights, no float zero points: the MFMA kernels (GEMV, LDS-tiled GEMM).
bool fast_path(const tmh_weight* w, const MatArgs& a) {
  return a.a_dt == TMH_F16 && w->wdtype == TMH_F16 && w->zp_kind != TMH_ZP_FLOAT;
}

// The operand path of the LDS-tiled prefill GEMM for a call, or -1 where it does not apply: M > 64
// and 32-bit buffer offsets over the weights; f16 A with f16 weights (GM_F16) and bf16 A with bf16
// weights (GM_BF16, one parameter entry per lane) without float zero points read A as given and
// need it aligned, with 32-bit offsets over it (and a tile of rows past M); every other float
// combination goes through GM_SPLIT (one parameter entry per lane, 32-bit offsets over its hi and
// lo rows) unless the call cannot give it scratch memory for them (no_split_a).
int gemm_mode(const tmh_weight* w, const MatArgs& a) {
  if (a.M <= 64 || w->ntiles * w->nchunks * 1024 + 16 * w->nchunks * 1024 >= (int64_t(1) << 31)) return -1;
  const bool direct_f16 = a.a_dt == TMH_F16 && w->wdtype == TMH_F16 && w->zp_kind != TMH_ZP_FLOAT;
  const bool direct_bf16 = a.a_dt == TMH_BF16 && w->wdtype == TMH_BF16 && w->zp_kind != TMH_ZP_FLOAT;
  if (direct_f16 || direct_bf16) {
    if (!a.a_vec || (a.M + kGemmBM) * a.lda * 2 >= (int64_t(1) << 31)) return -1;
    if (direct_bf16 && split_params(w)) return -1;
    return direct_f16 ? GM_F16 : GM_BF16;
  }
  if (split_params(w) || a.no_split_a) return -1;
  const int64_t kp = w->nchunks * chunk_weights(w->bits);
  if ((a.M + kGemmBM) * kp * 2 >= (int64_t(1) << 31)) return -1;
  return GM_SPLIT;
}

// Scratch memory of one call: GM_SPLIT's hi and lo rows of A, then the f32 partial sums of a plan
// that splits K (splits * M * N), each 256-byte aligned; zeros where the call needs none.
struct GemmScratch {
  size_t a_split = 0, partials = 0;
  size_t total() const { return a_split + partials; }
};

size_t split_a_bytes(const tmh_weight* w, int64_t M) {
  const size_t kp = static_cast<size_t>(w->nchunks) * chunk_weights(w->bits);
  return (2 * static_cast<size_t>(M) * kp * 2 + 255) / 256 * 256;
}

GemmScratch gemm_scratch(const tmh_ctx* ctx, const tmh_weight* w, const MatArgs& a) {
  GemmScratch g;
  const int mode = gemm_mode(w, a);
  if (mode < 0) return g;
  if (mode == GM_SPLIT) g.a_split = split_a_bytes(w, a.M);
  const GemmPlan p = plan_gemm(a.M, w->N, w->ntiles, w->nchunks, w->bits, cus_of(ctx), a.split_cap, mode);
  if (p.splits > 1) g.partials = static_cast<size_t>(p.splits) * static_cast<size_t>(a.M) * static_cast<size_t>(w->N) * sizeof(float);
  return g;
}

template <int BITS, bool HAS_ZP, bool SPLIT>
void launch_fast_variant(tmh_ctx* ctx, const tmh_weight* w, const MatArgs& a, hipStream_t s) {
  if (a.M <= 16) {
    launch_gemv<BITS, 1, HAS_ZP, SPLIT>(w, a, s, ctx->num_cus);
  } else if (a.M <= 32) {
    launch_gemv<BITS, 2, HAS_ZP, SPLIT>(w, a, s, ctx->num_cus);
  } else if (a.M <= 64 || BITS == 2) {
    launch_gemv<BITS, 4, HAS_ZP, SPLIT>(w, a, s, ctx->num_cus);
  } else if constexpr (BITS != 2) {
    launch_gemm<BITS, HAS_ZP, SPLIT>(w, a, s);
  }
}

template <int BITS>
void launch_fast_bits(tmh_ctx* ctx, const tmh_weight* w, const MatArgs& a, hipStream_t s) {
  const bool zp = w->zp_kind == TMH_ZP_PACKED;
  const bool split = split_params(w);
  if (zp && split) launch_fast_variant<BITS, true, true>(ctx, w, a, s);
  else if (zp) launch_fast_variant<BITS, true, false>(ctx, w, a, s);
  else if (split) launch_fast_variant<BITS, false, true>(ctx, w, a, s);
  else launch_fast_variant<BITS, false, false>(ctx, w, a, s);
}

// The prefill GEMM on operand path `mode` (gemm_mode), with GM_SPLIT's hi/lo rows of A made first.
template <int BITS>
void launch_gemm_bits(tmh_ctx* ctx, const tmh_weight* w, const MatArgs& a, hipStream_t s, int mode) {
  const GemmPlan p = plan_gemm(a.M, w->N, w->ntiles, w->nchunks, BITS, cus_of(ctx), a.split_cap, mode);
  const bool zp = w->zp_kind == TMH_ZP_PACKED;
  if (mode == GM_F16) {
    const GemmA ga{a.a, w->K, a.lda};
    const bool split = split_params(w);
    if (zp && split) launch_gemm_plan<BITS, true, true>(w, a, ga, s, p);
    else if (zp) launch_gemm_plan<BITS, true, false>(w, a, ga, s, p);
    else if (split) launch_gemm_plan<BITS, false, true>(w, a, ga, s, p);
    else launch_gemm_plan<BITS, false, false>(w, a, ga, s, p);
    return;
  }
  if (mode == GM_BF16) {
    const GemmA ga{a.a, w->K, a.lda};
    if (zp) launch_gemm_plan<BITS, true, false, GM_BF16, DT_BF16>(w, a, ga, s, p);
    else launch_gemm_plan<BITS, false, false, GM_BF16, DT_BF16>(w, a, ga, s, p);
    return;
  }
  const int64_t kp = w->nchunks * chunk_weights(BITS);
  const int64_t quads = a.M * (kp / 8);
  auto* split_rows = static_cast<uint16_t*>(a.a_split);
  const unsigned sgrid = static_cast<unsigned>((quads + 255) / 256);
  switch (a.a_dt) {
    case TMH_F16: k_split_a<DT_F16><<<sgrid, 256, 0, s>>>(a.a, a.M, w->K, a.lda, kp, split_rows); break;
    case TMH_BF16: k_split_a<DT_BF16><<<sgrid, 256, 0, s>>>(a.a, a.M, w->K, a.lda, kp, split_rows); break;
    default: k_split_a<DT_F32><<<sgrid, 256, 0, s>>>(a.a, a.M, w->K, a.lda, kp, split_rows);
  }
  const GemmA ga{split_rows, kp, kp};
  switch (w->wdtype) {
    case TMH_F16: launch_gemm_plan<BITS, false, false, GM_SPLIT, DT_F16>(w, a, ga, s, p); break;
    case TMH_BF16: launch_gemm_plan<BITS, false, false, GM_SPLIT, DT_BF16>(w, a, ga, s, p); break;
    default: launch_gemm_plan<BITS, false, false, GM_SPLIT, DT_F32>(w, a, ga, s, p);
  }
}

template <int BITS, int WDT>
void launch_general_wd(const tmh_weight* w, const MatArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(w->ntiles), static_cast<unsigned>((a.M + kGeneralRows - 1) / kGeneralRows));
  const auto* qt = reinterpret_cast<const uint4_t*>(w->d_q);
  const int shift = bsc_shift_of(w);
#define TMH_GENERAL(ZK)                                                                        \
  k_matmul_general<BITS, WDT, ZK><<<grid, kThreads, 0, s>>>(                                   \
      qt, w->d_scale, w->d_zero, a.a, a.a_dt, a.M, w->K, a.lda, a.bias, a.bias_dt, a.y, a.y_dt, \
      a.dot_dt, a.ldy, w->N, w->nchunks, w->nbc, shift)
  switch (w->zp_kind) {
    case TMH_ZP_PACKED: TMH_GENERAL(TMH_ZP_PACKED); break;
    case TMH_ZP_FLOAT: TMH_GENERAL(TMH_ZP_FLOAT); break;
    default: TMH_GENERAL(TMH_ZP_NONE);
  }
#undef TMH_GENERAL
}

template <int BITS>
void launch_general_bits(const tmh_weight* w, const MatArgs& a, hipStream_t s) {
  switch (w->wdtype) {
    case TMH_F16: launch_general_wd<BITS, DT_F16>(w, a, s); break;
    case TMH_BF16: launch_general_wd<BITS, DT_BF16>(w, a, s); break;
    default: launch_general_wd<BITS, DT_F32>(w, a, s);
  }
}

// Validated sizes of one weight's tiled layout.
struct PackPlan {
  int64_t K, N, blocks, row_bytes, nchunks, ntiles, zrow;
  int bits, block_size, cw, bsc, nbc, wdtype, zp_kind, zp_dtype, scales_dtype;
  size_t q_bytes, scale_bytes, zero_bytes;
};

int plan_nbits(tmh_ctx* ctx, const uint8_t* h_b, size_t b_bytes, const void* h_scales, int scales_dtype,
               size_t scales_count, const void* h_zero_points, int zp_kind, int zp_dtype, size_t zp_count,
               int64_t K, int64_t N, int bits, int block_size, int weight_dtype, PackPlan* p) {
  if (bits != 2 && bits != 4 && bits != 8)
    return fail(ctx, TMH_ERR_INVALID, "MatMulNBits bits must be 2, 4 or 8, got %d", bits);
  if (block_size < 16 || (block_size & (block_size - 1)) != 0)
    return fail(ctx, TMH_ERR_INVALID, "MatMulNBits block_size must be a power of two >= 16, got %d", block_size);
  if (K <= 0 || N <= 0)
    return fail(ctx, TMH_ERR_INVALID, "MatMulNBits K and N must be positive, got K=%lld N=%lld", (long long)K, (long long)N);
  if (K > (int64_t(1) << 31) || N > (int64_t(1) << 31))
    return fail(ctx, TMH_ERR_INVALID, "MatMulNBits K and N must be at most 2^31");
  if (!is_float_dtype(scales_dtype))
    return fail(ctx, TMH_ERR_INVALID, "scales must be f32, f16 or bf16, got %s", dtype_name(scales_dtype));
  if (!is_float_dtype(weight_dtype))
    return fail(ctx, TMH_ERR_INVALID, "the weight type must be f32, f16 or bf16, got %s", dtype_name(weight_dtype));
  if (!h_b || !h_scales) return fail(ctx, TMH_ERR_INVALID, "B and scales must not be NULL");
  const int64_t blocks = (K + block_size - 1) / block_size;
  const int64_t row_bytes = blocks * block_size * bits / 8;
  if (static_cast<int64_t>(b_bytes) != N * row_bytes)
    return fail(ctx, TMH_ERR_INVALID,
                "B holds %zu bytes; N=%lld rows of %lld blocks of %d %d-bit weights need %lld", b_bytes,
                (long long)N, (long long)blocks, block_size, bits, (long long)(N * row_bytes));
  if (static_cast<int64_t>(scales_count) != N * blocks)
    return fail(ctx, TMH_ERR_INVALID, "scales hold %zu values; N*blocks is %lld", scales_count, (long long)(N * blocks));
  const int64_t zrow = (blocks * bits + 7) / 8;
  if (zp_kind == TMH_ZP_PACKED) {
    if (zp_dtype != TMH_U8) return fail(ctx, TMH_ERR_INVALID, "packed zero points must be u8, got %s", dtype_name(zp_dtype));
    if (!h_zero_points) return fail(ctx, TMH_ERR_INVALID, "zero points are NULL");
    if (static_cast<int64_t>(zp_count) != N * zrow)
      return fail(ctx, TMH_ERR_INVALID, "packed zero points hold %zu bytes; N rows of %lld bytes need %lld", zp_count,
                  (long long)zrow, (long long)(N * zrow));
  } else if (zp_kind == TMH_ZP_FLOAT) {
    if (!is_float_dtype(zp_dtype))
      return fail(ctx, TMH_ERR_INVALID, "float zero points must be f32, f16 or bf16, got %s", dtype_name(zp_dtype));
    if (!h_zero_points) return fail(ctx, TMH_ERR_INVALID, "zero points are NULL");
    if (static_cast<int64_t>(zp_count) != N * blocks)
      return fail(ctx, TMH_ERR_INVALID, "float zero points hold %zu values; N*blocks is %lld", zp_count, (long long)(N * blocks));
  } else if (zp_kind != TMH_ZP_NONE) {
    return fail(ctx, TMH_ERR_INVALID, "unknown zero point kind %d", zp_kind);
  }
  p->K = K;
  p->N = N;
  p->bits = bits;
  p->block_size = block_size;
  p->blocks = blocks;
  p->row_bytes = row_bytes;
  p->zrow = zrow;
  p->nchunks = (row_bytes + kChunkBytes - 1) / kChunkBytes;
  p->ntiles = (N + kTileRows - 1) / kTileRows;
  p->cw = chunk_weights(bits);
  p->bsc = std::min(block_size, p->cw);
  p->nbc = p->cw / p->bsc;
  p->wdtype = weight_dtype;
  p->zp_kind = zp_kind;
  p->zp_dtype = zp_dtype;
  p->scales_dtype = scales_dtype;
  const int64_t n_params = p->ntiles * p->nchunks * p->nbc * 16;
  p->q_bytes = static_cast<size_t>(p->ntiles * p->nchunks * 1024);
  p->scale_bytes = static_cast<size_t>(n_params * dtype_size(weight_dtype));
  p->zero_bytes = zp_kind == TMH_ZP_PACKED ? static_cast<size_t>(n_params * bits / 8)
                  : zp_kind == TMH_ZP_FLOAT ? static_cast<size_t>(n_params) * sizeof(float) : 0;
  return TMH_OK;
}

// Fills the tiled weights, scales and zero points of a validated plan.
void fill_nbits(const PackPlan& p, const uint8_t* h_b, const void* h_scales, const void* h_zero_points,
                uint8_t* q, void* scale, void* zero) {
  std::memset(q, 0, p.q_bytes);
  for (int64_t t = 0; t < p.ntiles; ++t) {
    for (int64_t c = 0; c < p.nchunks; ++c) {
      uint8_t* dst = q + (t * p.nchunks + c) * 1024;
      for (int l = 0; l < 64; ++l) {
        const int r = l & 15, g = l >> 4;
        const int64_t n = t * 16 + r;
        const int64_t off = c * kChunkBytes + g * 16;
        uint8_t bytes[16] = {0};
        if (n < p.N)
          for (int i = 0; i < 16; ++i)
            if (off + i < p.row_bytes) bytes[i] = h_b[n * p.row_bytes + off + i];
        for (int wd = 0; wd < 4; ++wd) {
          uint32_t x;
          std::memcpy(&x, bytes + 4 * wd, 4);
          x = reorder_word(x, p.bits);
          std::memcpy(dst + l * 16 + 4 * wd, &x, 4);
        }
      }
    }
  }
  const auto* zp8 = static_cast<const uint8_t*>(h_zero_points);
  auto* zero8 = static_cast<uint8_t*>(zero);
  auto* zerof = static_cast<float*>(zero);
  const int zper = 8 / p.bits;  // packed zero points per byte
  if (p.zp_kind == TMH_ZP_PACKED) std::memset(zero8, 0, p.zero_bytes);
  for (int64_t t = 0; t < p.ntiles; ++t) {
    for (int64_t c = 0; c < p.nchunks; ++c) {
      for (int j = 0; j < p.nbc; ++j) {
        const int64_t b = (c * p.cw + static_cast<int64_t>(j) * p.bsc) / p.block_size;
        for (int r = 0; r < 16; ++r) {
          const int64_t n = t * 16 + r;
          const size_t e = static_cast<size_t>(((t * p.nchunks + c) * p.nbc + j) * 16 + r);
          const bool valid = n < p.N && b < p.blocks;
          // The scales in the weight type (the Nx.as_type/2 of dequantize_weight/4).
          const float s = valid ? round_host(load_float(h_scales, p.scales_dtype, static_cast<size_t>(n * p.blocks + b)), p.wdtype) : 0.0f;
          store_host(scale, p.wdtype, e, s);
          if (p.zp_kind == TMH_ZP_PACKED) {
            const uint8_t z = !valid ? static_cast<uint8_t>(1 << (p.bits - 1))
                              : p.bits == 8 ? zp8[n * p.zrow + b] : packed_zero(zp8, p.zrow, p.bits, n, b);
            zero8[e / zper] |= static_cast<uint8_t>(z << ((e % zper) * p.bits));
          } else if (p.zp_kind == TMH_ZP_FLOAT) {
            zerof[e] = valid ? round_host(load_float(h_zero_points, p.zp_dtype, static_cast<size_t>(n * p.blocks + b)), p.wdtype) : 0.0f;
          }
        }
      }
    }
  }
}


// Concatenation of packed weights along N: output lane-slot (t, c, l) holds row n = 16t + l%16,
// taken from the part that owns n (its local row n - first[p]), same chunk and k-group.
struct ConcatParts {
  const uint8_t* q[kMaxConcat];
  const uint8_t* scale[kMaxConcat];
  const uint8_t* zero[kMaxConcat];
  int64_t first[kMaxConcat + 1];  // first row of each part; first[count] = total N
  int count;
};

// Packed zero points (zero_bits 2, 4 or 8) move entry by entry: rows r.. of a byte can come from
// different parts, so lanes r of one (t, c, j) gather their byte by shuffles; float zero points
// (zero_bits 0, zero_bytes 4) are copied byte for byte with the scales.
__global__ __launch_bounds__(256) void k_concat_tiles(ConcatParts parts, uint8_t* __restrict__ q,
                                                      uint8_t* __restrict__ scale, uint8_t* __restrict__ zero,
                                                      int64_t nchunks, int nbc, int scale_bytes, int zero_bytes,
                                                      int zero_bits, int64_t lanes_total) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= lanes_total) return;
  const int lane = static_cast<int>(id & 63);
  const int64_t tc = id >> 6;
  const int64_t t = tc / nchunks;
  const int64_t c = tc - t * nchunks;
  const int r = lane & 15, g = lane >> 4;
  const int64_t n = t * 16 + r;
  int p = 0;
  while (p + 1 < parts.count && n >= parts.first[p + 1]) ++p;
  const bool valid = n < parts.first[parts.count];
  const int64_t ln = n - parts.first[p];
  const int64_t st = ln >> 4;
  const int sr = static_cast<int>(ln & 15);
  const int64_t src_tc = st * nchunks + c;
  uint4_t v = {0u, 0u, 0u, 0u};
  if (valid) v = reinterpret_cast<const uint4_t*>(parts.q[p])[src_tc * 64 + 16 * g + sr];
  reinterpret_cast<uint4_t*>(q)[id] = v;
  // Parameters: slot (t, c, j, r) for j < nbc, written by the lanes with g == 0 (lanes 0-15 of
  // the wavefront; lanes_total is a multiple of 64, so all sixteen are here).
  if (g != 0) return;
  for (int j = 0; j < nbc; ++j) {
    const int64_t dst = (tc * nbc + j) * 16 + r;
    const int64_t src = (src_tc * nbc + j) * 16 + sr;
    for (int b = 0; b < scale_bytes; ++b)
      scale[dst * scale_bytes + b] = valid ? parts.scale[p][src * scale_bytes + b] : 0;
    if (zero_bits) {
      const int per = 8 / zero_bits;
      uint32_t z = 0u;
      if (valid) z = (parts.zero[p][src / per] >> ((src % per) * zero_bits)) & ((1u << zero_bits) - 1u);
      z <<= (r % per) * zero_bits;
      if (per >= 2) z |= __shfl_xor(z, 1);
      if (per >= 4) z |= __shfl_xor(z, 2);
      if (r % per == 0) zero[dst / per] = static_cast<uint8_t>(z);
    } else {
      for (int b = 0; b < zero_bytes; ++b)
        zero[dst * zero_bytes + b] = valid ? parts.zero[p][src * zero_bytes + b] : 0;
    }
  }
}

// The tiled layout of a weight from its ONNX layout on the device (the same bytes fill_nbits
// writes on the host). k_pack_tiles: lane-slot (t, c, l) takes row 16t + l%16, bytes
// 64c + 16(l/16) .. +15 of B (zeros past the row or past N), each 32-bit word reordered so that
// value 2j sits at bits j*bits and value 2j+1 at 16 + j*bits.
__global__ __launch_bounds__(256) void k_pack_tiles(const uint8_t* __restrict__ b, int64_t N, int64_t row_bytes,
                                                    int64_t nchunks, int bits, uint4_t* __restrict__ q,
                                                    int64_t lanes_total) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= lanes_total) return;
  const int l = static_cast<int>(id & 63);
  const int64_t tc = id >> 6;
  const int64_t t = tc / nchunks, c = tc - t * nchunks;
  const int64_t n = t * 16 + (l & 15);
  const int64_t off = c * kChunkBytes + (l >> 4) * 16;
  uint4_t v = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int wd = 0; wd < 4; ++wd) {
    uint32_t x = 0;
    if (n < N && off + 4 * wd < row_bytes)  // rows are whole words: block bytes are multiples of 4
      x = *reinterpret_cast<const uint32_t*>(b + n * row_bytes + off + 4 * wd);
    if (bits != 8) {
      const int count = 32 / bits;
      const uint32_t mask = (1u << bits) - 1u;
      uint32_t out = 0;
      for (int i = 0; i < count; ++i) out |= ((x >> (i * bits)) & mask) << ((i & 1) * 16 + (i >> 1) * bits);
      x = out;
    }
    v[wd] = x;
  }
  q[id] = v;
}

// k_pack_params: entry (t, c, j, r) holds block (c*CW + j*bsc) / block_size of row 16t + r: the
// scale rounded to the weight type, the packed zero point in `bits` bits (the thread of the
// byte's first entry writes the byte: the entries of a byte are rows r.. of one (t, c, j)), or a
// float zero point rounded to the weight type (kept as f32); entries past N or past the blocks
// hold scale 0 and zero point 2^(bits-1) (0 for float zero points).
template <int WDT>
__global__ __launch_bounds__(256) void k_pack_params(const void* __restrict__ scales, int scales_dt,
                                                     const void* __restrict__ zp, int zp_kind, int zp_dt, int64_t N,
                                                     int64_t blocks, int64_t zrow, int bits, int block_size,
                                                     int64_t nchunks, int nbc, int cw, int bsc, void* __restrict__ scale,
                                                     void* __restrict__ zero, int64_t entries) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= entries) return;
  const int r = static_cast<int>(e & 15);
  const int64_t tcj = e >> 4;
  const int j = static_cast<int>(tcj % nbc);
  const int64_t tc = tcj / nbc;
  const int64_t t = tc / nchunks, c = tc - t * nchunks;
  const int64_t n = t * 16 + r;
  const int64_t blk = (c * cw + static_cast<int64_t>(j) * bsc) / block_size;
  const bool valid = n < N && blk < blocks;
  const float sv = valid ? round_to<WDT>(load_float_rt(scales, scales_dt, n * blocks + blk)) : 0.0f;
  store_as<WDT>(scale, e, sv);
  if (zp_kind == TMH_ZP_PACKED) {
    const int per = 8 / bits;
    if (r % per != 0) return;
    uint32_t packed = 0u;
    for (int i = 0; i < per; ++i) {
      const int64_t ni = n + i;
      uint32_t z = 1u << (bits - 1);
      if (ni < N && blk < blocks) {
        const int64_t bit = blk * bits;
        const uint8_t byte = static_cast<const uint8_t*>(zp)[ni * zrow + bit / 8];
        z = bits == 8 ? byte : (byte >> (bit % 8)) & ((1u << bits) - 1u);
      }
      packed |= z << (i * bits);
    }
    static_cast<uint8_t*>(zero)[e / per] = static_cast<uint8_t>(packed);
  } else if (zp_kind == TMH_ZP_FLOAT) {
    static_cast<float*>(zero)[e] = valid ? round_to<WDT>(load_float_rt(zp, zp_dt, n * blocks + blk)) : 0.0f;
  }
}

}  // namespace

extern "C" {

int tmh_pack_nbits_host(const uint8_t* h_b, size_t b_bytes, const void* h_scales, int scales_dtype,
                        size_t scales_count, const void* h_zero_points, int zp_kind, int zp_dtype,
                        size_t zp_count, int64_t K, int64_t N, int bits, int block_size, int weight_dtype,
                        void* h_q, size_t* q_bytes, void* h_scale, size_t* scale_bytes, void* h_zero,
                        size_t* zero_bytes) {
  PackPlan p;
  TMH_TRY(plan_nbits(nullptr, h_b, b_bytes, h_scales, scales_dtype, scales_count, h_zero_points, zp_kind, zp_dtype,
                     zp_count, K, N, bits, block_size, weight_dtype, &p));
  if (!q_bytes || !scale_bytes || !zero_bytes) return fail(nullptr, TMH_ERR_INVALID, "the size outputs must not be NULL");
  const bool query = !h_q && !h_scale && !h_zero;
  if (!query) {
    if (!h_q || !h_scale || (p.zero_bytes && !h_zero))
      return fail(nullptr, TMH_ERR_INVALID, "pass every output buffer, or none to query the sizes");
    if (*q_bytes < p.q_bytes || *scale_bytes < p.scale_bytes || *zero_bytes < p.zero_bytes)
      return fail(nullptr, TMH_ERR_INVALID, "an output buffer is too small: need %zu, %zu and %zu bytes", p.q_bytes,
                  p.scale_bytes, p.zero_bytes);
    fill_nbits(p, h_b, h_scales, h_zero_points, static_cast<uint8_t*>(h_q), h_scale, h_zero);
  }
  *q_bytes = p.q_bytes;
  *scale_bytes = p.scale_bytes;
  *zero_bytes = p.zero_bytes;
  return TMH_OK;
}

int tmh_weight_upload_nbits(tmh_ctx* ctx, const uint8_t* h_b, size_t b_bytes, const void* h_scales,
                            int scales_dtype, size_t scales_count, const void* h_zero_points,
                            int zp_kind, int zp_dtype, size_t zp_count, int64_t K, int64_t N,
                            int bits, int block_size, int weight_dtype, tmh_weight** out) {
  if (!ctx) return fail(nullptr, TMH_ERR_INVALID, "the context is NULL");
  if (!out) return fail(ctx, TMH_ERR_INVALID, "out is NULL");
  *out = nullptr;
  PackPlan p;
  TMH_TRY(plan_nbits(ctx, h_b, b_bytes, h_scales, scales_dtype, scales_count, h_zero_points, zp_kind, zp_dtype,
                     zp_count, K, N, bits, block_size, weight_dtype, &p));
  TMH_TRY(use_device(ctx));
  std::vector<uint8_t> q(p.q_bytes), scale(p.scale_bytes), zero(p.zero_bytes);
  fill_nbits(p, h_b, h_scales, h_zero_points, q.data(), scale.data(), zero.data());

  tmh_weight* w = new tmh_weight();
  w->device = ctx->device;
  w->K = p.K;
  w->N = p.N;
  w->bits = p.bits;
  w->block_size = p.block_size;
  w->blocks = p.blocks;
  w->row_bytes = p.row_bytes;
  w->nchunks = p.nchunks;
  w->ntiles = p.ntiles;
  w->nbc = p.nbc;
  w->wdtype = p.wdtype;
  w->zp_kind = p.zp_kind;
  int st = TMH_OK;
  auto copy = [&](void** dst, const std::vector<uint8_t>& src) {
    if (st != TMH_OK || src.empty()) return;
    st = check_hip(ctx, hipMalloc(dst, src.size()), "hipMalloc (weight)");
    if (st == TMH_OK)
      st = check_hip(ctx, hipMemcpy(*dst, src.data(), src.size(), hipMemcpyHostToDevice), "hipMemcpy (weight)");
  };
  copy(reinterpret_cast<void**>(&w->d_q), q);
  copy(&w->d_scale, scale);
  copy(&w->d_zero, zero);
  if (st != TMH_OK) {
    tmh_weight_free(w);
    return st;
  }
  w->device_bytes = q.size() + scale.size() + zero.size();
  *out = w;
  return TMH_OK;
}

int tmh_weight_pack_nbits(tmh_ctx* ctx, const void* d_b, size_t b_bytes, const void* d_scales, int scales_dtype,
                          size_t scales_count, const void* d_zero_points, int zp_kind, int zp_dtype, size_t zp_count,
                          int64_t K, int64_t N, int bits, int block_size, int weight_dtype, void* stream,
                          tmh_weight** out) {
  if (!ctx) return fail(nullptr, TMH_ERR_INVALID, "the context is NULL");
  if (!out) return fail(ctx, TMH_ERR_INVALID, "out is NULL");
  *out = nullptr;
  PackPlan p;
  TMH_TRY(plan_nbits(ctx, static_cast<const uint8_t*>(d_b), b_bytes, d_scales, scales_dtype, scales_count,
                     d_zero_points, zp_kind, zp_dtype, zp_count, K, N, bits, block_size, weight_dtype, &p));
  TMH_TRY(use_device(ctx));
  hipStream_t s = pick_stream(ctx, stream);
  tmh_weight* w = new tmh_weight();
  w->device = ctx->device;
  w->K = p.K;
  w->N = p.N;
  w->bits = p.bits;
  w->block_size = p.block_size;
  w->blocks = p.blocks;
  w->row_bytes = p.row_bytes;
  w->nchunks = p.nchunks;
  w->ntiles = p.ntiles;
  w->nbc = p.nbc;
  w->wdtype = p.wdtype;
  w->zp_kind = p.zp_kind;
  int st = check_hip(ctx, hipMalloc(reinterpret_cast<void**>(&w->d_q), p.q_bytes), "hipMalloc (weight)");
  if (st == TMH_OK) st = check_hip(ctx, hipMalloc(&w->d_scale, p.scale_bytes), "hipMalloc (weight)");
  if (st == TMH_OK && p.zero_bytes) st = check_hip(ctx, hipMalloc(&w->d_zero, p.zero_bytes), "hipMalloc (weight)");
  if (st != TMH_OK) {
    tmh_weight_free(w);
    return st;
  }
  const int64_t lanes = p.ntiles * p.nchunks * 64;
  k_pack_tiles<<<static_cast<unsigned>((lanes + 255) / 256), 256, 0, s>>>(
      static_cast<const uint8_t*>(d_b), p.N, p.row_bytes, p.nchunks, p.bits, reinterpret_cast<uint4_t*>(w->d_q), lanes);
  const int64_t entries = p.ntiles * p.nchunks * p.nbc * 16;
  const unsigned pgrid = static_cast<unsigned>((entries + 255) / 256);
#define TMH_PACK_PARAMS(WDT)                                                                                        \
  k_pack_params<WDT><<<pgrid, 256, 0, s>>>(d_scales, scales_dtype, d_zero_points, p.zp_kind, zp_dtype, p.N, p.blocks, \
                                           p.zrow, p.bits, p.block_size, p.nchunks, p.nbc, p.cw, p.bsc, w->d_scale,  \
                                           w->d_zero, entries)
  switch (p.wdtype) {
    case TMH_F16: TMH_PACK_PARAMS(DT_F16); break;
    case TMH_BF16: TMH_PACK_PARAMS(DT_BF16); break;
    default: TMH_PACK_PARAMS(DT_F32);
  }
#undef TMH_PACK_PARAMS
  st = check_launch(ctx, "k_pack_tiles/k_pack_params");
  if (st != TMH_OK) {
    tmh_weight_free(w);
    return st;
  }
  w->device_bytes = p.q_bytes + p.scale_bytes + p.zero_bytes;
  *out = w;
  return TMH_OK;
}

void tmh_weight_free(tmh_weight* w) {
  if (!w) return;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(w->device);
  if (w->d_q) (void)hipFree(w->d_q);
  if (w->d_scale) (void)hipFree(w->d_scale);
  if (w->d_zero) (void)hipFree(w->d_zero);
  (void)hipSetDevice(prev);
  delete w;
}

int tmh_weight_concat_nbits(tmh_ctx* ctx, const tmh_weight* const* parts, int count, tmh_weight** out) {
  TMH_TRY(use_device(ctx));
  if (!out) return fail(ctx, TMH_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (!parts || count < 1 || count > kMaxConcat)
    return fail(ctx, TMH_ERR_INVALID, "concatenation takes 1 to %d weights, got %d", kMaxConcat, count);
  const tmh_weight* w0 = parts[0];
  if (!w0) return fail(ctx, TMH_ERR_INVALID, "weight 0 is NULL");
  ConcatParts cp{};
  cp.count = count;
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    const tmh_weight* w = parts[i];
    if (!w) return fail(ctx, TMH_ERR_INVALID, "weight %d is NULL", i);
    if (w->device != ctx->device) return fail(ctx, TMH_ERR_INVALID, "weight %d lives on device %d", i, w->device);
    if (w->K != w0->K || w->bits != w0->bits || w->block_size != w0->block_size || w->wdtype != w0->wdtype ||
        w->zp_kind != w0->zp_kind)
      return fail(ctx, TMH_ERR_INVALID,
                  "weight %d differs from weight 0 in K, bits, block_size, weight type or zero point kind", i);
    cp.q[i] = w->d_q;
    cp.scale[i] = static_cast<const uint8_t*>(w->d_scale);
    cp.zero[i] = static_cast<const uint8_t*>(w->d_zero);
    cp.first[i] = total;
    total += w->N;
  }
  cp.first[count] = total;
  if (total > (int64_t(1) << 31)) return fail(ctx, TMH_ERR_INVALID, "the concatenated N is too large");
  tmh_weight* w = new tmh_weight(*w0);
  w->d_q = nullptr;
  w->d_scale = nullptr;
  w->d_zero = nullptr;
  w->N = total;
  w->ntiles = (total + kTileRows - 1) / kTileRows;
  const int64_t n_params = w->ntiles * w->nchunks * w->nbc * 16;
  const int scale_bytes = dtype_size(w->wdtype);
  const int zero_bytes = w->zp_kind == TMH_ZP_FLOAT ? 4 : 0;
  const int zero_bits = w->zp_kind == TMH_ZP_PACKED ? w->bits : 0;
  const size_t qb = static_cast<size_t>(w->ntiles * w->nchunks * 1024);
  const size_t sb = static_cast<size_t>(n_params * scale_bytes);
  const size_t zb = static_cast<size_t>(zero_bits ? n_params * zero_bits / 8 : n_params * zero_bytes);
  int st = check_hip(ctx, hipMalloc(reinterpret_cast<void**>(&w->d_q), qb), "hipMalloc (weight)");
  if (st == TMH_OK) st = check_hip(ctx, hipMalloc(&w->d_scale, sb), "hipMalloc (weight)");
  if (st == TMH_OK && zb) st = check_hip(ctx, hipMalloc(&w->d_zero, zb), "hipMalloc (weight)");
  if (st != TMH_OK) {
    tmh_weight_free(w);
    return st;
  }
  const int64_t lanes = w->ntiles * w->nchunks * 64;
  k_concat_tiles<<<static_cast<unsigned>((lanes + 255) / 256), 256, 0, ctx->stream>>>(
      cp, w->d_q, static_cast<uint8_t*>(w->d_scale), static_cast<uint8_t*>(w->d_zero), w->nchunks, w->nbc,
      scale_bytes, zero_bytes, zero_bits, lanes);
  st = check_launch(ctx, "k_concat_tiles");
  if (st == TMH_OK) st = check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (st != TMH_OK) {
    tmh_weight_free(w);
    return st;
  }
  w->device_bytes = qb + sb + zb;
  *out = w;
  return TMH_OK;
}

int tmh_weight_info(const tmh_weight* w, int64_t* K, int64_t* N, int* bits, int* block_size,
                    int* weight_dtype, size_t* device_bytes) {
  if (!w) return fail(nullptr, TMH_ERR_INVALID, "the weight is NULL");
  if (K) *K = w->K;
  if (N) *N = w->N;
  if (bits) *bits = w->bits;
  if (block_size) *block_size = w->block_size;
  if (weight_dtype) *weight_dtype = w->wdtype;
  if (device_bytes) *device_bytes = w->device_bytes;
  return TMH_OK;
}

int tmh_dequantize_nbits(tmh_ctx* ctx, const tmh_weight* w, void* d_out, int out_dtype, void* stream) {
  TMH_TRY(use_device(ctx));
  if (!w) return fail(ctx, TMH_ERR_INVALID, "the weight is NULL");
  if (w->device != ctx->device) return fail(ctx, TMH_ERR_INVALID, "the weight lives on device %d, the context on %d", w->device, ctx->device);
  if (!d_out) return fail(ctx, TMH_ERR_INVALID, "the output is NULL");
  if (!is_float_dtype(out_dtype)) return fail(ctx, TMH_ERR_INVALID, "the output type must be f32, f16 or bf16, got %s", dtype_name(out_dtype));
  hipStream_t s = pick_stream(ctx, stream);
  const int shift = bsc_shift_of(w);
  switch (w->bits) {
    case 2: launch_dequant_bits<2>(w, d_out, out_dtype, s, shift); break;
    case 4: launch_dequant_bits<4>(w, d_out, out_dtype, s, shift); break;
    default: launch_dequant_bits<8>(w, d_out, out_dtype, s, shift);
  }
  return check_launch(ctx, "k_dequant");
}

}  // extern "C"

namespace {

// The device address of `scratch` per device, looked up once per device with that device
// current (tmh_ctx_create calls noalloc_scratch_init), or the error of the lookup.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};

// Validates a MatMulNBits call and fills its arguments; *run is false when there is nothing to do.
int prepare_matmul(tmh_ctx* ctx, const tmh_weight* w, const void* d_a, int a_dtype, int64_t M, int64_t lda,
                   const void* d_bias, int bias_dtype, void* d_y, int y_dtype, int64_t ldy, MatArgs* out,
                   bool* run) {
  *run = false;
  TMH_TRY(use_device(ctx));
  if (!w) return fail(ctx, TMH_ERR_INVALID, "the weight is NULL");
  if (w->device != ctx->device) return fail(ctx, TMH_ERR_INVALID, "the weight lives on device %d, the context on %d", w->device, ctx->device);
  if (M < 0) return fail(ctx, TMH_ERR_INVALID, "M must not be negative, got %lld", (long long)M);
  if (!is_float_dtype(a_dtype)) return fail(ctx, TMH_ERR_INVALID, "A must be f32, f16 or bf16, got %s", dtype_name(a_dtype));
  if (!is_float_dtype(y_dtype)) return fail(ctx, TMH_ERR_INVALID, "Y must be f32, f16 or bf16, got %s", dtype_name(y_dtype));
  if (d_bias && !is_float_dtype(bias_dtype)) return fail(ctx, TMH_ERR_INVALID, "the bias must be f32, f16 or bf16, got %s", dtype_name(bias_dtype));
  if (lda < w->K) return fail(ctx, TMH_ERR_INVALID, "lda %lld is below K %lld", (long long)lda, (long long)w->K);
  if (ldy < w->N) return fail(ctx, TMH_ERR_INVALID, "ldy %lld is below N %lld", (long long)ldy, (long long)w->N);
  // Nx.dot/4 gives the merged type of A and W; the bias then merges again (quantized.ex:44-45).
  const int dot_dt = merge_float(a_dtype, w->wdtype);
  const int expect = d_bias ? merge_float(dot_dt, bias_dtype) : dot_dt;
  if (y_dtype != expect)
    return fail(ctx, TMH_ERR_INVALID, "Y must be %s for A %s, weights %s%s%s", dtype_name(expect), dtype_name(a_dtype),
                dtype_name(w->wdtype), d_bias ? " and bias " : "", d_bias ? dtype_name(bias_dtype) : "");
  if (M == 0) return TMH_OK;
  if (!d_a || !d_y) return fail(ctx, TMH_ERR_INVALID, "A and Y must not be NULL");
  if (M > (int64_t(1) << 31) / 2) return fail(ctx, TMH_ERR_INVALID, "M is too large");
  *out = MatArgs{d_a, a_dtype, M, lda,
                 (reinterpret_cast<uintptr_t>(d_a) % 16 == 0) && (lda % 8 == 0) && (w->K % 8 == 0),
                 d_bias, bias_dtype, d_y, y_dtype, dot_dt, ldy};
  *run = true;
  return TMH_OK;
}

// Launches a prepared MatMulNBits call (its scratch memory, if any, in a.ws and a.a_split).
int launch_matmul(tmh_ctx* ctx, const tmh_weight* w, const MatArgs& a, hipStream_t s) {
  if (const int mode = gemm_mode(w, a); mode >= 0) {
    switch (w->bits) {
      case 2: launch_gemm_bits<2>(ctx, w, a, s, mode); break;
      case 4: launch_gemm_bits<4>(ctx, w, a, s, mode); break;
      default: launch_gemm_bits<8>(ctx, w, a, s, mode);
    }
    return check_launch(ctx, "k_gemm_lds");
  }
  if (fast_path(w, a)) {
    switch (w->bits) {
      case 2: launch_fast_bits<2>(ctx, w, a, s); break;
      case 4: launch_fast_bits<4>(ctx, w, a, s); break;
      default: launch_fast_bits<8>(ctx, w, a, s);
    }
    return check_launch(ctx, "k_gemv_f16/k_gemm_f16");
  }
  if (a.a_dt == TMH_F32 && a.y_dt == TMH_F32 && !a.bias && decode_gemv_f32_ok(w, a.M, a.lda, a.ldy, a.a)) {
    launch_decode_gemv_f32(w, a.a, a.M, a.lda, a.y, a.ldy, s);
    return check_launch(ctx, "k_gemv_f32");
  }
  switch (w->bits) {
    case 2: launch_general_bits<2>(w, a, s); break;
    case 4: launch_general_bits<4>(w, a, s); break;
    default: launch_general_bits<8>(w, a, s);
  }
  return check_launch(ctx, "k_matmul_general");
}

}  // namespace

namespace tmh {

void noalloc_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device]) return;
  void* p = nullptr;
  const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (err != hipSuccess) {
    (void)hipGetLastError();
    g_scratch_err[device] = err;
    return;
  }
  g_scratch[device] = static_cast<float*>(p);
  g_scratch_err[device] = hipSuccess;
}

}  // namespace tmh

extern "C" {

int tmh_matmul_nbits(tmh_ctx* ctx, const tmh_weight* w, const void* d_a, int a_dtype, int64_t M,
                     int64_t lda, const void* d_bias, int bias_dtype, void* d_y, int y_dtype,
                     int64_t ldy, void* stream) {
  TimelineScope timeline(ctx);
  MatArgs a{};
  bool run = false;
  TMH_TRY(prepare_matmul(ctx, w, d_a, a_dtype, M, lda, d_bias, bias_dtype, d_y, y_dtype, ldy, &a, &run));
  if (!run) return TMH_OK;
  hipStream_t s = pick_stream(ctx, stream);
  const GemmScratch g = gemm_scratch(ctx, w, a);
  if (const size_t need = g.total()) {
    // A graph must replay what an eager call computes, so a call that needs scratch memory never
    // runs another plan instead: without the workspace (it cannot grow while the stream is
    // captured) the call fails.
    auto* ws = static_cast<uint8_t*>(workspace(ctx, need, s));
    if (!ws)
      return fail(ctx, TMH_ERR_UNSUPPORTED,
                  "MatMulNBits with M=%lld, N=%lld, K=%lld needs a %zu-byte workspace (split K or the split rows "
                  "of A), which cannot be allocated now (not while the stream is being captured into a graph): "
                  "run the call once before capture",
                  (long long)M, (long long)w->N, (long long)w->K, need);
    a.a_split = g.a_split ? ws : nullptr;
    a.ws = g.partials ? reinterpret_cast<float*>(ws + g.a_split) : nullptr;
  }
  return launch_matmul(ctx, w, a, s);
}

int tmh_matmul_nbits_noalloc(tmh_ctx* ctx, const tmh_weight* w, const void* d_a, int a_dtype, int64_t M,
                             int64_t lda, const void* d_bias, int bias_dtype, void* d_y, int y_dtype, int64_t ldy,
                             void* stream) {
  TimelineScope timeline(ctx);
  MatArgs a{};
  bool run = false;
  TMH_TRY(prepare_matmul(ctx, w, d_a, a_dtype, M, lda, d_bias, bias_dtype, d_y, y_dtype, ldy, &a, &run));
  if (!run) return TMH_OK;
  // The call keeps its scratch memory within the scratch area: GM_SPLIT's rows of A when they fit
  // (else the general kernel runs), then the partial sums of the best plan that fits in the rest
  // (where tmh_matmul_nbits's plan would need more: fewer splits of K, or none).
  if (gemm_mode(w, a) == GM_SPLIT && split_a_bytes(w, a.M) > kNoallocScratchBytes) a.no_split_a = true;
  const size_t rows_a = gemm_mode(w, a) == GM_SPLIT ? split_a_bytes(w, a.M) : 0;
  a.split_cap = kNoallocScratchBytes - rows_a;
  const GemmScratch g = gemm_scratch(ctx, w, a);
  if (const size_t need = g.total()) {
    if (need > kNoallocScratchBytes)  // the plan honours the cap; kept as a guard on the scratch's bounds
      return fail(ctx, TMH_ERR_INVALID, "MatMulNBits scratch of %zu bytes exceeds the %zu-byte area", need,
                  kNoallocScratchBytes);
    float* p = nullptr;
    hipError_t err = hipErrorInvalidDevice;
    if (ctx->device >= 0 && ctx->device < kMaxDevices) {
      std::lock_guard<std::mutex> lock(g_scratch_mu);
      p = g_scratch[ctx->device];
      err = g_scratch_err[ctx->device];
    }
    if (!p) return check_hip(ctx, err == hipSuccess ? hipErrorInvalidDevice : err, "the scratch memory of tmh_matmul_nbits_noalloc");
    auto* base = reinterpret_cast<uint8_t*>(p);
    a.a_split = g.a_split ? base : nullptr;
    a.ws = g.partials ? reinterpret_cast<float*>(base + g.a_split) : nullptr;
  }
  return launch_matmul(ctx, w, a, pick_stream(ctx, stream));
}

}  // extern "C"
