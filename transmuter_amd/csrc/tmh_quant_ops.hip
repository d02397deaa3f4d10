// GatherBlockQuantized, DequantizeLinear and MatMulInteger on gfx950.
//
// Reference arithmetic (georgeguimaraes/transmuter):
//   lib/transmuter/ops/quantized.ex:49-66    GatherBlockQuantized
//   lib/transmuter/ops/quantized.ex:70-84    DequantizeLinear, expand_quant_param/3 at :328-353
//   lib/transmuter/ops/quantized.ex:105-110  MatMulInteger, per_axis/3 at :288-291
//   lib/transmuter/ops/nn.ex:537-555         integer_product/5: exact s32 sums
//   lib/transmuter/ops/quantized.ex:94-103   DynamicQuantizeLinear
#include <algorithm>
#include <cmath>
#include <cstdio>

#include "tmh_device.h"
#include "tmh_internal.h"

using namespace tmh;

namespace {

// ------------------------------------------------------------------ GatherBlockQuantized

// Bytes [u*UB, u*UB + UB) of a gathered row, each value dequantized in DT:
// (q - zero) * scale, q and zero exact small integers, one rounding (packed.ex:28-36).
// ONE_BLOCK: the thread's values share one quantization block (one scale and zero point).
// VEC_OUT: the values leave as 8- or 16-byte stores.
template <int DT, int BITS, int UB, bool ONE_BLOCK, bool VEC_OUT>
__global__ __launch_bounds__(256) void k_gather_bq(
    const uint8_t* __restrict__ data, bool data_signed, int64_t rows, int64_t row_bytes,
    const void* __restrict__ ids, bool ids64, uint32_t n_ids, const void* __restrict__ scales,
    int64_t blocks, int64_t bs, const void* __restrict__ zp, int zp_dt, int64_t zrow,
    void* __restrict__ out, uint32_t units) {
  constexpr int PER = 8 / BITS;
  constexpr int V = UB * PER;
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  if (idx >= n_ids * units) return;
  const uint32_t i = idx / units;
  const uint32_t u = idx - i * units;
  int64_t id = ids64 ? static_cast<const int64_t*>(ids)[i] : static_cast<const int32_t*>(ids)[i];
  if (id < 0) id += rows;  // ONNX: a negative index counts from the end
  id = id < 0 ? 0 : (id >= rows ? rows - 1 : id);
  const int64_t D = row_bytes * PER;
  uint8_t bytes[UB];
  if constexpr (UB == 4) {
    const uint32_t x = reinterpret_cast<const uint32_t*>(data + id * row_bytes)[u];
#pragma unroll
    for (int b = 0; b < 4; ++b) bytes[b] = static_cast<uint8_t>(x >> (8 * b));
  } else {
    bytes[0] = data[id * row_bytes + u];
  }
  const float zdefault = data_signed ? 0.0f : static_cast<float>(1 << (BITS - 1));
  auto zero_of = [&](int64_t blk) -> float {
    if (!zp) return zdefault;
    if (zp_dt == TMH_U8 || zp_dt == TMH_S8) {
      const int64_t bit = blk * BITS;
      const uint8_t zb = static_cast<const uint8_t*>(zp)[id * zrow + bit / 8];
      int zq;
      if constexpr (BITS == 8) {
        zq = zp_dt == TMH_S8 ? static_cast<int>(static_cast<int8_t>(zb)) : static_cast<int>(zb);
      } else {
        zq = (zb >> (bit % 8)) & ((1 << BITS) - 1);
        if (zp_dt == TMH_S8 && zq >= (1 << (BITS - 1))) zq -= (1 << BITS);
      }
      return static_cast<float>(zq);
    }
    return round_to<DT>(load_float_rt(zp, zp_dt, id * blocks + blk));
  };
  const int64_t col0 = static_cast<int64_t>(u) * V;
  float s = 0.f, z = 0.f;
  if constexpr (ONE_BLOCK) {
    const int64_t blk = col0 / bs;
    s = load_as_f32<DT>(scales, id * blocks + blk);
    z = zero_of(blk);
  }
  float vals[V];
#pragma unroll
  for (int b = 0; b < UB; ++b) {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      int q;
      if constexpr (BITS == 8) {
        q = data_signed ? static_cast<int>(static_cast<int8_t>(bytes[b])) : static_cast<int>(bytes[b]);
      } else {
        q = (bytes[b] >> (v * BITS)) & ((1 << BITS) - 1);
        if (data_signed && q >= (1 << (BITS - 1))) q -= (1 << BITS);
      }
      if constexpr (!ONE_BLOCK) {
        const int64_t blk = (col0 + b * PER + v) / bs;
        s = load_as_f32<DT>(scales, id * blocks + blk);
        z = zero_of(blk);
      }
      vals[b * PER + v] = dequant_value<DT>(static_cast<float>(q), z, s);
    }
  }
  const int64_t o = static_cast<int64_t>(i) * D + col0;
  if constexpr (VEC_OUT) {
    constexpr int ES = DT == DT_F32 ? 4 : 2;
    uint32_t words[V * ES / 4];
#pragma unroll
    for (int k = 0; k < V * ES / 4; ++k) {
      if constexpr (DT == DT_F32) {
        words[k] = __builtin_bit_cast(uint32_t, vals[k]);
      } else if constexpr (DT == DT_F16) {
        words[k] = f32_to_f16_bits(vals[2 * k]) | (static_cast<uint32_t>(f32_to_f16_bits(vals[2 * k + 1])) << 16);
      } else {
        words[k] = f32_to_bf16_bits(vals[2 * k]) | (static_cast<uint32_t>(f32_to_bf16_bits(vals[2 * k + 1])) << 16);
      }
    }
    auto* dst = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(out) + o * ES);
    if constexpr (V * ES == 8) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(words[0], words[1]);
    } else {
#pragma unroll
      for (int k = 0; k < V * ES / 16; ++k)
        reinterpret_cast<uint4*>(dst)[k] = make_uint4(words[4 * k], words[4 * k + 1], words[4 * k + 2], words[4 * k + 3]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < V; ++k) store_as<DT>(out, o + k, vals[k]);
  }
}

template <int DT, int BITS, int UB, bool ONE_BLOCK>
void launch_gather_ub(const uint8_t* data, bool sgn, int64_t rows, int64_t row_bytes, const void* ids,
                      bool ids64, int64_t n_ids, const void* scales, int64_t blocks, int64_t bs,
                      const void* zp, int zp_dt, int64_t zrow, void* out, int64_t units, bool vec_out, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n_ids * units + 255) / 256));
  const auto n = static_cast<uint32_t>(n_ids);
  const auto un = static_cast<uint32_t>(units);
  if constexpr (UB == 4) {
    if (vec_out) {
      k_gather_bq<DT, BITS, UB, ONE_BLOCK, true><<<grid, 256, 0, s>>>(data, sgn, rows, row_bytes, ids, ids64, n, scales,
                                                                      blocks, bs, zp, zp_dt, zrow, out, un);
      return;
    }
  }
  k_gather_bq<DT, BITS, UB, ONE_BLOCK, false><<<grid, 256, 0, s>>>(data, sgn, rows, row_bytes, ids, ids64, n, scales,
                                                                   blocks, bs, zp, zp_dt, zrow, out, un);
}

template <int DT, int BITS>
void launch_gather(const uint8_t* data, bool sgn, int64_t rows, int64_t row_bytes, const void* ids,
                   bool ids64, int64_t n_ids, const void* scales, int64_t blocks, int64_t bs,
                   const void* zp, int zp_dt, int64_t zrow, void* out, hipStream_t s) {
  constexpr int PER = 8 / BITS;
  constexpr int ES = DT == DT_F32 ? 4 : 2;
  const bool vec = row_bytes % 4 == 0 && reinterpret_cast<uintptr_t>(data) % 4 == 0;
  const int64_t units = vec ? row_bytes / 4 : row_bytes;
  const int64_t D = row_bytes * PER;
  if (vec) {
    const bool one = bs % (4 * PER) == 0;
    const bool vec_out = reinterpret_cast<uintptr_t>(out) % 16 == 0 && (D * ES) % 16 == 0;
    if (one)
      launch_gather_ub<DT, BITS, 4, true>(data, sgn, rows, row_bytes, ids, ids64, n_ids, scales, blocks, bs, zp, zp_dt,
                                          zrow, out, units, vec_out, s);
    else
      launch_gather_ub<DT, BITS, 4, false>(data, sgn, rows, row_bytes, ids, ids64, n_ids, scales, blocks, bs, zp, zp_dt,
                                           zrow, out, units, vec_out, s);
  } else {
    launch_gather_ub<DT, BITS, 1, false>(data, sgn, rows, row_bytes, ids, ids64, n_ids, scales, blocks, bs, zp, zp_dt,
                                         zrow, out, units, false, s);
  }
}

template <int DT>
void launch_gather_bits(int bits, const uint8_t* data, bool sgn, int64_t rows, int64_t row_bytes,
                        const void* ids, bool ids64, int64_t n_ids, const void* scales,
                        int64_t blocks, int64_t bs, const void* zp, int zp_dt, int64_t zrow,
                        void* out, hipStream_t s) {
  switch (bits) {
    case 2: launch_gather<DT, 2>(data, sgn, rows, row_bytes, ids, ids64, n_ids, scales, blocks, bs, zp, zp_dt, zrow, out, s); break;
    case 4: launch_gather<DT, 4>(data, sgn, rows, row_bytes, ids, ids64, n_ids, scales, blocks, bs, zp, zp_dt, zrow, out, s); break;
    default: launch_gather<DT, 8>(data, sgn, rows, row_bytes, ids, ids64, n_ids, scales, blocks, bs, zp, zp_dt, zrow, out, s);
  }
}

// ------------------------------------------------------------------ DequantizeLinear

__device__ __forceinline__ int32_t load_int_rt(const void* p, int dt, int64_t i) {
  switch (dt) {
    case TMH_U8: return static_cast<const uint8_t*>(p)[i];
    case TMH_S8: return static_cast<const int8_t*>(p)[i];
    case TMH_U16: return static_cast<const uint16_t*>(p)[i];
    case TMH_S16: return static_cast<const int16_t*>(p)[i];
    default: return static_cast<const int32_t*>(p)[i];
  }
}

template <int OUT>
__global__ __launch_bounds__(256) void k_dequantize_linear(
    const void* __restrict__ x, int x_dt, bool x_int, int64_t dim, int64_t inner,
    const void* __restrict__ scale, int scale_dt, const void* __restrict__ zero, int zero_dt,
    int mode, int64_t bs, int64_t nb, void* __restrict__ y, int64_t total) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int64_t per_outer = dim * inner;
  const int64_t o = e / per_outer;
  const int64_t rem = e - o * per_outer;
  const int64_t d = rem / inner;
  const int64_t in = rem - d * inner;
  int64_t p = 0;
  if (mode == TMH_QPARAM_AXIS) p = d;
  else if (mode == TMH_QPARAM_BLOCKED) p = (o * nb + d / bs) * inner + in;
  float v;
  if (x_int) {
    // s32 subtraction, wrapping as the reference's s32 arithmetic does.
    uint32_t shifted = static_cast<uint32_t>(load_int_rt(x, x_dt, e));
    if (zero) shifted -= static_cast<uint32_t>(load_int_rt(zero, zero_dt, p));
    v = static_cast<float>(static_cast<int32_t>(shifted));
  } else {
    v = load_float_rt(x, x_dt, e);
    if (zero) v = v - load_float_rt(zero, zero_dt, p);
  }
  const float s = load_float_rt(scale, scale_dt, p);
  const float prod = v * s;
  store_as<OUT>(y, e, prod);
}

// ------------------------------------------------------------------ MatMulInteger

constexpr int kMiTile = 16;
constexpr int kMiK = 64;

// y[bt, m, n] = sum_k (a - a_zero[m]) (b - b_zero[n]), wrapping mod 2^32. Each f32 chunk sum of
// the reference is exact, so the exact integer sum is its value.
__global__ __launch_bounds__(256) void k_matmul_integer(
    const void* __restrict__ a, bool a_signed, const void* __restrict__ b, bool b_signed,
    const void* __restrict__ a_zero, int64_t a_zero_count, const void* __restrict__ b_zero,
    int64_t b_zero_count, int64_t M, int64_t K, int64_t N, bool b_batched, int32_t* __restrict__ y) {
  __shared__ int32_t sa[kMiTile][kMiK + 1];
  __shared__ int32_t sb[kMiK][kMiTile + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t bt = blockIdx.z;
  const int64_t m = static_cast<int64_t>(blockIdx.y) * kMiTile + ty;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kMiTile + tx;
  const auto* a8 = static_cast<const uint8_t*>(a) + bt * M * K;
  const auto* b8 = static_cast<const uint8_t*>(b) + (b_batched ? bt * K * N : 0);
  auto av = [&](int64_t mm, int64_t kk) -> int32_t {
    const uint8_t raw = a8[mm * K + kk];
    int32_t v = a_signed ? static_cast<int8_t>(raw) : raw;
    if (a_zero) {
      const uint8_t z = static_cast<const uint8_t*>(a_zero)[a_zero_count == 1 ? 0 : mm];
      v -= a_signed ? static_cast<int8_t>(z) : z;
    }
    return v;
  };
  auto bv = [&](int64_t kk, int64_t nn) -> int32_t {
    const uint8_t raw = b8[kk * N + nn];
    int32_t v = b_signed ? static_cast<int8_t>(raw) : raw;
    if (b_zero) {
      const uint8_t z = static_cast<const uint8_t*>(b_zero)[b_zero_count == 1 ? 0 : nn];
      v -= b_signed ? static_cast<int8_t>(z) : z;
    }
    return v;
  };
  uint32_t acc = 0;
  for (int64_t k0 = 0; k0 < K; k0 += kMiK) {
    for (int idx = threadIdx.x; idx < kMiTile * kMiK; idx += 256) {
      const int rr = idx / kMiK, kk = idx % kMiK;
      const int64_t gm = static_cast<int64_t>(blockIdx.y) * kMiTile + rr;
      sa[rr][kk] = (gm < M && k0 + kk < K) ? av(gm, k0 + kk) : 0;
      const int kb = idx / kMiTile, cc = idx % kMiTile;
      const int64_t gn = static_cast<int64_t>(blockIdx.x) * kMiTile + cc;
      sb[kb][cc] = (gn < N && k0 + kb < K) ? bv(k0 + kb, gn) : 0;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < kMiK; ++kk) acc += static_cast<uint32_t>(sa[ty][kk] * sb[kk][tx]);
    __syncthreads();
  }
  if (m < M && n < N) y[(bt * M + m) * N + n] = static_cast<int32_t>(acc);
}


// ------------------------------------------------------------------ MatMulInteger on int8 MFMA

// With a = sa + oa (sa the s8 form of a: the byte itself for s8 data, a ^ 0x80 = a - 128 for
// u8 data, so oa is 0 or 128) and likewise b:
//   sum_k (a - az_m)(b - bz_n) = sum_k sa sb + cb_n * rs_m + ca_m * cs_n + K * ca_m * cb_n
// with ca_m = oa - az_m, cb_n = ob - bz_n, rs_m = sum_k sa[m][k], cs_n = sum_k sb[k][n], all
// modulo 2^32 (the s32 wrap of the exact sum). The sa sb sums run on v_mfma_i32_16x16x64_i8.

// rs for every row of every A batch, cs for every column of every B batch.
__global__ __launch_bounds__(256) void k_int8_sums(const uint8_t* __restrict__ a, bool a_signed,
                                                    const uint8_t* __restrict__ b, bool b_signed, int64_t a_rows,
                                                    int64_t K, int64_t N, int64_t b_batches, int32_t* __restrict__ rs,
                                                    int32_t* __restrict__ cs) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < a_rows) {
    const uint8_t* row = a + i * K;
    uint32_t sum = 0;
    for (int64_t k = 0; k < K; ++k) sum += static_cast<uint32_t>(static_cast<int8_t>(a_signed ? row[k] : row[k] ^ 0x80));
    rs[i] = static_cast<int32_t>(sum);
  }
  const int64_t j = i - a_rows;
  if (j >= 0 && j < b_batches * N) {
    const int64_t bt = j / N, n = j - bt * N;
    const uint8_t* col = b + bt * K * N + n;
    uint32_t sum = 0;
    for (int64_t k = 0; k < K; ++k)
      sum += static_cast<uint32_t>(static_cast<int8_t>(b_signed ? col[k * N] : col[k * N] ^ 0x80));
    cs[j] = static_cast<int32_t>(sum);
  }
}

constexpr int kI8Tile = 128;  // output rows and columns per workgroup
constexpr int kI8K = 64;      // k per step (one MFMA deep)
constexpr int kI8Row = 80;    // LDS bytes per row of 64: 16-byte pieces of 8 consecutive rows on distinct banks

// 128 x 128 outputs per workgroup of four wavefronts (64 x 64 each, 4 x 4 MFMA tiles). Per
// k-step A's rows and B's columns go to LDS as s8 bytes, B transposed through 4 x 4 byte
// blocks, zeros outside the matrices.
__global__ __launch_bounds__(256) void k_matmul_integer_mfma(
    const uint8_t* __restrict__ a, bool a_signed, const uint8_t* __restrict__ b, bool b_signed,
    const void* __restrict__ a_zero, int64_t a_zero_count, const void* __restrict__ b_zero,
    int64_t b_zero_count, int64_t M, int64_t K, int64_t N, bool b_batched, const int32_t* __restrict__ rs,
    const int32_t* __restrict__ cs, int32_t* __restrict__ y) {
  __shared__ __align__(16) uint8_t sA[kI8Tile * kI8Row];
  __shared__ __align__(16) uint8_t sB[kI8Tile * kI8Row];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 15, g = lane >> 4;
  const int64_t bt = blockIdx.z;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kI8Tile, n0 = static_cast<int64_t>(blockIdx.x) * kI8Tile;
  const uint8_t* a8 = a + bt * M * K;
  const uint8_t* b8 = b + (b_batched ? bt * K * N : 0);
  const uint32_t aflip = a_signed ? 0u : 0x80808080u, bflip = b_signed ? 0u : 0x80808080u;
  const bool a_vec = (K % 16) == 0 && (reinterpret_cast<uintptr_t>(a) % 16) == 0;
  const bool b_vec = (N % 4) == 0 && (reinterpret_cast<uintptr_t>(b) % 4) == 0;
  int4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = int4_t{0, 0, 0, 0};
  for (int64_t k0 = 0; k0 < K; k0 += kI8K) {
    // A: 128 rows x 64 bytes, 16 bytes per thread and load.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + 256 * h;
      const int row = c >> 2, kc = (c & 3) * 16;
      const int64_t gm = m0 + row, gk = k0 + kc;
      uint4_t v = {0u, 0u, 0u, 0u};
      if (gm < M) {
        if (a_vec && gk + 16 <= K) {
          v = *reinterpret_cast<const uint4_t*>(a8 + gm * K + gk) ^ aflip;
        } else {
          for (int e = 0; e < 16; ++e)
            if (gk + e < K) v[e >> 2] |= static_cast<uint32_t>(a8[gm * K + gk + e] ^ (aflip & 0xFFu)) << (8 * (e & 3));
        }
      }
      *reinterpret_cast<uint4_t*>(sA + row * kI8Row + kc) = v;
    }
    // B: 64 k x 128 columns as 4 x 4 byte blocks, stored column-major (sB[n][k]).
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int u = tid + 256 * h;
      const int kq = u >> 5, nq = u & 31;
      const int64_t gk = k0 + 4 * kq, gn = n0 + 4 * nq;
      uint32_t rw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw[i] = 0;
        if (gk + i < K) {
          if (b_vec && gn + 4 <= N) {
            rw[i] = *reinterpret_cast<const uint32_t*>(b8 + (gk + i) * N + gn) ^ bflip;
          } else {
            for (int e = 0; e < 4; ++e)
              if (gn + e < N) rw[i] |= static_cast<uint32_t>(b8[(gk + i) * N + gn + e] ^ (bflip & 0xFFu)) << (8 * e);
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t col = ((rw[0] >> (8 * e)) & 0xFFu) | (((rw[1] >> (8 * e)) & 0xFFu) << 8) |
                             (((rw[2] >> (8 * e)) & 0xFFu) << 16) | (((rw[3] >> (8 * e)) & 0xFFu) << 24);
        *reinterpret_cast<uint32_t*>(sB + (4 * nq + e) * kI8Row + 4 * kq) = col;
      }
    }
    __syncthreads();
    int4_t af[4], bf[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      af[mt] = *reinterpret_cast<const int4_t*>(sA + (wm * 64 + mt * 16 + r) * kI8Row + g * 16);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
      bf[nt] = *reinterpret_cast<const int4_t*>(sB + (wn * 64 + nt * 16 + r) * kI8Row + g * 16);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)  // B first: a lane ends with 4 consecutive columns of one row
        acc[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[nt], af[mt], acc[mt][nt], 0, 0, 0);
    __syncthreads();
  }
  const uint32_t oa = a_signed ? 0u : 128u, ob = b_signed ? 0u : 128u;
  auto zero_of = [](const void* z, int64_t count, int64_t i, bool sgn) -> uint32_t {
    if (!z) return 0u;
    const uint8_t raw = static_cast<const uint8_t*>(z)[count == 1 ? 0 : i];
    return sgn ? static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(raw))) : raw;
  };
  const uint32_t kk = static_cast<uint32_t>(K);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int64_t m = m0 + wm * 64 + mt * 16 + r;
    if (m >= M) continue;
    const uint32_t ca = oa - zero_of(a_zero, a_zero_count, m, a_signed);
    const uint32_t rsm = static_cast<uint32_t>(rs[bt * M + m]);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int64_t n = n0 + wn * 64 + nt * 16 + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (n + e >= N) break;
        const uint32_t cb = ob - zero_of(b_zero, b_zero_count, n + e, b_signed);
        const uint32_t csn = static_cast<uint32_t>(cs[(b_batched ? bt * N : 0) + n + e]);
        const uint32_t v = static_cast<uint32_t>(acc[mt][nt][e]) + cb * rsm + ca * csn + kk * ca * cb;
        y[(bt * M + m) * N + n + e] = static_cast<int32_t>(v);
      }
    }
  }
}

// ------------------------------------------------------------------ DynamicQuantizeLinear

// scale = (max(x, 0) - min(x, 0)) / 255 (1 when that is 0), zero = saturate(round(-low / scale)),
// in f32 with round-half-even, as quantized.ex:94-103.
__device__ __forceinline__ void dql_params(float low, float high, float* scale, uint8_t* zero) {
  low = fminf(low, 0.f);
  high = fmaxf(high, 0.f);
  float sc = (high - low) / 255.f;
  if (sc == 0.f) sc = 1.f;
  const float z = rintf(-low / sc);
  *scale = sc;
  *zero = static_cast<uint8_t>(fminf(fmaxf(z, 0.f), 255.f));
}

// Minimum and maximum of the block's share of x; with one block, the scale and zero point.
__global__ __launch_bounds__(256) void k_dql_minmax(const float* __restrict__ x, int64_t n, float* __restrict__ part,
                                                     float* __restrict__ scale, uint8_t* __restrict__ zero) {
  __shared__ float lo_s[256], hi_s[256];
  float lo = INFINITY, hi = -INFINITY;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    lo = fminf(lo, x[i]);
    hi = fmaxf(hi, x[i]);
  }
  lo_s[threadIdx.x] = lo;
  hi_s[threadIdx.x] = hi;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      lo_s[threadIdx.x] = fminf(lo_s[threadIdx.x], lo_s[threadIdx.x + w]);
      hi_s[threadIdx.x] = fmaxf(hi_s[threadIdx.x], hi_s[threadIdx.x + w]);
    }
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  if (gridDim.x == 1) {
    dql_params(lo_s[0], hi_s[0], scale, zero);
  } else {
    part[2 * blockIdx.x] = lo_s[0];
    part[2 * blockIdx.x + 1] = hi_s[0];
  }
}

__global__ __launch_bounds__(64) void k_dql_finalize(const float* __restrict__ part, int parts, float* __restrict__ scale,
                                                      uint8_t* __restrict__ zero) {
  if (threadIdx.x != 0) return;
  float lo = INFINITY, hi = -INFINITY;
  for (int i = 0; i < parts; ++i) {
    lo = fminf(lo, part[2 * i]);
    hi = fmaxf(hi, part[2 * i + 1]);
  }
  dql_params(lo, hi, scale, zero);
}

// y = saturate(round(x / scale) + zero), four values per thread.
__global__ __launch_bounds__(256) void k_dql_quantize(const float* __restrict__ x, int64_t n,
                                                       const float* __restrict__ scale, const uint8_t* __restrict__ zero,
                                                       uint8_t* __restrict__ y) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  const float sc = *scale, z = static_cast<float>(*zero);
  auto q = [&](float v) -> uint32_t { return static_cast<uint32_t>(fminf(fmaxf(rintf(v / sc) + z, 0.f), 255.f)); };
  if (i + 4 <= n && (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (reinterpret_cast<uintptr_t>(y) % 4) == 0) {
    const float4_t v = *reinterpret_cast<const float4_t*>(x + i);
    *reinterpret_cast<uint32_t*>(y + i) = q(v[0]) | (q(v[1]) << 8) | (q(v[2]) << 16) | (q(v[3]) << 24);
  } else {
    for (int e = 0; e < 4 && i + e < n; ++e) y[i + e] = static_cast<uint8_t>(q(x[i + e]));
  }
}

}  // namespace

extern "C" {

int tmh_gather_block_quantized(tmh_ctx* ctx, const void* d_data, int data_dtype, int64_t rows,
                               int64_t row_bytes, const void* d_ids, int ids_dtype, int64_t n_ids,
                               const void* d_scales, int scales_dtype, int64_t blocks,
                               const void* d_zero_points, int zp_dtype, int bits, void* d_out,
                               void* stream) {
  TMH_TRY(use_device(ctx));
  if (bits != 2 && bits != 4 && bits != 8)
    return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized bits must be 2, 4 or 8, got %d", bits);
  if (data_dtype != TMH_U8 && data_dtype != TMH_S8)
    return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized data must be u8 or s8, got %s", dtype_name(data_dtype));
  if (ids_dtype != TMH_S32 && ids_dtype != TMH_S64)
    return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized indices must be s32 or s64, got %s", dtype_name(ids_dtype));
  if (!is_float_dtype(scales_dtype))
    return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized scales must be f32, f16 or bf16, got %s", dtype_name(scales_dtype));
  if (rows <= 0 || row_bytes <= 0 || blocks <= 0 || n_ids < 0)
    return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized sizes must be positive");
  const int64_t D = row_bytes * (8 / bits);
  if (D % blocks != 0)
    return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized rows of %lld values do not split into %lld blocks", (long long)D, (long long)blocks);
  if (d_zero_points && !(zp_dtype == TMH_U8 || zp_dtype == TMH_S8 || is_float_dtype(zp_dtype)))
    return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized zero points must be u8, s8 or float, got %s", dtype_name(zp_dtype));
  if (n_ids == 0) return TMH_OK;
  if (!d_data || !d_ids || !d_scales || !d_out) return fail(ctx, TMH_ERR_INVALID, "GatherBlockQuantized: NULL pointer");
  if (n_ids * row_bytes >= (int64_t(1) << 32) - 256)
    return fail(ctx, TMH_ERR_UNSUPPORTED, "GatherBlockQuantized: %lld ids of %lld bytes exceed 2^32 packed bytes per call",
                (long long)n_ids, (long long)row_bytes);
  hipStream_t s = pick_stream(ctx, stream);
  const int64_t bs = D / blocks;
  const int64_t zrow = (blocks * bits + 7) / 8;
  const bool sgn = data_dtype == TMH_S8;
  const bool ids64 = ids_dtype == TMH_S64;
  const auto* data = static_cast<const uint8_t*>(d_data);
  switch (scales_dtype) {
    case TMH_F16: launch_gather_bits<DT_F16>(bits, data, sgn, rows, row_bytes, d_ids, ids64, n_ids, d_scales, blocks, bs, d_zero_points, zp_dtype, zrow, d_out, s); break;
    case TMH_BF16: launch_gather_bits<DT_BF16>(bits, data, sgn, rows, row_bytes, d_ids, ids64, n_ids, d_scales, blocks, bs, d_zero_points, zp_dtype, zrow, d_out, s); break;
    default: launch_gather_bits<DT_F32>(bits, data, sgn, rows, row_bytes, d_ids, ids64, n_ids, d_scales, blocks, bs, d_zero_points, zp_dtype, zrow, d_out, s);
  }
  return check_launch(ctx, "k_gather_bq");
}

int tmh_dequantize_linear(tmh_ctx* ctx, const void* d_x, int x_dtype, int64_t outer, int64_t dim,
                          int64_t inner, const void* d_scale, int scale_dtype, const void* d_zero,
                          int zero_dtype, int mode, int64_t block_size, void* d_y, void* stream) {
  TMH_TRY(use_device(ctx));
  const bool x_int = x_dtype == TMH_U8 || x_dtype == TMH_S8 || x_dtype == TMH_U16 ||
                     x_dtype == TMH_S16 || x_dtype == TMH_S32;
  if (!x_int && !is_float_dtype(x_dtype))
    return fail(ctx, TMH_ERR_INVALID, "DequantizeLinear x must be an 8/16/32-bit integer or float, got %s", dtype_name(x_dtype));
  if (!is_float_dtype(scale_dtype))
    return fail(ctx, TMH_ERR_INVALID, "DequantizeLinear scale must be f32, f16 or bf16, got %s", dtype_name(scale_dtype));
  if (d_zero) {
    const bool z_int = zero_dtype == TMH_U8 || zero_dtype == TMH_S8 || zero_dtype == TMH_U16 ||
                       zero_dtype == TMH_S16 || zero_dtype == TMH_S32;
    if (x_int != z_int || (!z_int && !is_float_dtype(zero_dtype)))
      return fail(ctx, TMH_ERR_INVALID, "DequantizeLinear zero point %s does not fit x %s", dtype_name(zero_dtype), dtype_name(x_dtype));
  }
  if (outer < 0 || dim < 0 || inner < 0) return fail(ctx, TMH_ERR_INVALID, "DequantizeLinear sizes must not be negative");
  if (mode != TMH_QPARAM_TENSOR && mode != TMH_QPARAM_AXIS && mode != TMH_QPARAM_BLOCKED)
    return fail(ctx, TMH_ERR_INVALID, "unknown DequantizeLinear parameter layout %d", mode);
  if (mode == TMH_QPARAM_BLOCKED && block_size <= 0)
    return fail(ctx, TMH_ERR_INVALID, "blocked DequantizeLinear needs a positive block_size");
  const int64_t total = outer * dim * inner;
  if (total == 0) return TMH_OK;
  if (!d_x || !d_scale || !d_y) return fail(ctx, TMH_ERR_INVALID, "DequantizeLinear: NULL pointer");
  hipStream_t s = pick_stream(ctx, stream);
  const int64_t nb = mode == TMH_QPARAM_BLOCKED ? (dim + block_size - 1) / block_size : 1;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  switch (scale_dtype) {
    case TMH_F16: k_dequantize_linear<DT_F16><<<grid, 256, 0, s>>>(d_x, x_dtype, x_int, dim, inner, d_scale, scale_dtype, d_zero, zero_dtype, mode, block_size, nb, d_y, total); break;
    case TMH_BF16: k_dequantize_linear<DT_BF16><<<grid, 256, 0, s>>>(d_x, x_dtype, x_int, dim, inner, d_scale, scale_dtype, d_zero, zero_dtype, mode, block_size, nb, d_y, total); break;
    default: k_dequantize_linear<DT_F32><<<grid, 256, 0, s>>>(d_x, x_dtype, x_int, dim, inner, d_scale, scale_dtype, d_zero, zero_dtype, mode, block_size, nb, d_y, total);
  }
  return check_launch(ctx, "k_dequantize_linear");
}

int tmh_matmul_integer(tmh_ctx* ctx, const void* d_a, int a_dtype, const void* d_b, int b_dtype,
                       const void* d_a_zero, int64_t a_zero_count, const void* d_b_zero,
                       int64_t b_zero_count, int64_t batch, int64_t M, int64_t K, int64_t N,
                       int b_batched, void* d_y, void* stream) {
  TMH_TRY(use_device(ctx));
  if ((a_dtype != TMH_U8 && a_dtype != TMH_S8) || (b_dtype != TMH_U8 && b_dtype != TMH_S8))
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger takes u8 or s8 values, got %s and %s", dtype_name(a_dtype), dtype_name(b_dtype));
  if (batch < 0 || M < 0 || K < 0 || N < 0) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger sizes must not be negative");
  if (d_a_zero && a_zero_count != 1 && a_zero_count != M)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger a_zero_point holds %lld values; 1 or M=%lld expected", (long long)a_zero_count, (long long)M);
  if (d_b_zero && b_zero_count != 1 && b_zero_count != N)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger b_zero_point holds %lld values; 1 or N=%lld expected", (long long)b_zero_count, (long long)N);
  if (batch == 0 || M == 0 || N == 0) return TMH_OK;
  if (!d_a || !d_b || !d_y) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger: NULL pointer");
  if (batch > 65535) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger batch must be below 65536");
  hipStream_t s = pick_stream(ctx, stream);
  const bool a_sgn = a_dtype == TMH_S8, b_sgn = b_dtype == TMH_S8;
  const int64_t b_batches = b_batched ? batch : 1;
  const size_t sums_bytes = static_cast<size_t>(batch * M + b_batches * N) * sizeof(int32_t);
  auto* sums = K > 0 ? static_cast<int32_t*>(workspace(ctx, sums_bytes, s)) : nullptr;
  if (!sums) {
    // K = 0, or no workspace inside a graph capture: the LDS-tiled kernel needs none.
    const dim3 grid(static_cast<unsigned>((N + kMiTile - 1) / kMiTile), static_cast<unsigned>((M + kMiTile - 1) / kMiTile),
                    static_cast<unsigned>(batch));
    k_matmul_integer<<<grid, 256, 0, s>>>(d_a, a_sgn, d_b, b_sgn, d_a_zero, a_zero_count, d_b_zero, b_zero_count, M, K, N,
                                          b_batched != 0, static_cast<int32_t*>(d_y));
    return check_launch(ctx, "k_matmul_integer");
  }
  const auto* a8 = static_cast<const uint8_t*>(d_a);
  const auto* b8 = static_cast<const uint8_t*>(d_b);
  int32_t* rs = sums;
  int32_t* cs = sums + batch * M;
  const int64_t lines = batch * M + b_batches * N;
  k_int8_sums<<<static_cast<unsigned>((lines + 255) / 256), 256, 0, s>>>(a8, a_sgn, b8, b_sgn, batch * M, K, N,
                                                                        b_batches, rs, cs);
  TMH_TRY(check_launch(ctx, "k_int8_sums"));
  const dim3 grid(static_cast<unsigned>((N + kI8Tile - 1) / kI8Tile), static_cast<unsigned>((M + kI8Tile - 1) / kI8Tile),
                  static_cast<unsigned>(batch));
  k_matmul_integer_mfma<<<grid, 256, 0, s>>>(a8, a_sgn, b8, b_sgn, d_a_zero, a_zero_count, d_b_zero, b_zero_count, M,
                                             K, N, b_batched != 0, rs, cs, static_cast<int32_t*>(d_y));
  return check_launch(ctx, "k_matmul_integer_mfma");
}

int tmh_dynamic_quantize_linear(tmh_ctx* ctx, const void* d_x, int x_dtype, int64_t n, void* d_y, void* d_scale,
                                void* d_zero, void* stream) {
  TMH_TRY(use_device(ctx));
  if (x_dtype != TMH_F32)
    return fail(ctx, TMH_ERR_UNSUPPORTED, "DynamicQuantizeLinear takes f32 values, got %s", dtype_name(x_dtype));
  if (n < 0) return fail(ctx, TMH_ERR_INVALID, "DynamicQuantizeLinear size must not be negative");
  if (!d_scale || !d_zero || (n > 0 && (!d_x || !d_y)))
    return fail(ctx, TMH_ERR_INVALID, "DynamicQuantizeLinear: NULL pointer");
  hipStream_t s = pick_stream(ctx, stream);
  const auto* x = static_cast<const float*>(d_x);
  auto* scale = static_cast<float*>(d_scale);
  auto* zero = static_cast<uint8_t*>(d_zero);
  // One workgroup per 64 Ki values, at most 256; their partial ranges go through the workspace
  // (one workgroup does it all when there is none, inside a graph capture).
  int parts = static_cast<int>(std::min<int64_t>(256, (n + 65535) / 65536));
  float* part = nullptr;
  if (parts > 1) {
    part = static_cast<float*>(workspace(ctx, static_cast<size_t>(parts) * 2 * sizeof(float), s));
    if (!part) parts = 1;
  }
  k_dql_minmax<<<static_cast<unsigned>(std::max(parts, 1)), 256, 0, s>>>(x, n, part, scale, zero);
  TMH_TRY(check_launch(ctx, "k_dql_minmax"));
  if (parts > 1) {
    k_dql_finalize<<<1, 64, 0, s>>>(part, parts, scale, zero);
    TMH_TRY(check_launch(ctx, "k_dql_finalize"));
  }
  if (n == 0) return TMH_OK;
  k_dql_quantize<<<static_cast<unsigned>((n + 1023) / 1024), 256, 0, s>>>(x, n, scale, zero, static_cast<uint8_t*>(d_y));
  return check_launch(ctx, "k_dql_quantize");
}

}  // extern "C"
