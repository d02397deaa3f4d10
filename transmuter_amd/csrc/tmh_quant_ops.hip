// GatherBlockQuantized, DequantizeLinear and MatMulInteger on gfx950.
//
// Reference arithmetic (georgeguimaraes/transmuter):
//   lib/transmuter/ops/quantized.ex:49-66    GatherBlockQuantized
//   lib/transmuter/ops/quantized.ex:70-84    DequantizeLinear, expand_quant_param/3 at :328-353
//   lib/transmuter/ops/quantized.ex:105-110  MatMulInteger, per_axis/3 at :288-291
//   lib/transmuter/ops/nn.ex:537-555         integer_product/5: exact s32 sums
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
  const dim3 grid(static_cast<unsigned>((N + kMiTile - 1) / kMiTile), static_cast<unsigned>((M + kMiTile - 1) / kMiTile),
                  static_cast<unsigned>(batch));
  k_matmul_integer<<<grid, 256, 0, s>>>(d_a, a_dtype == TMH_S8, d_b, b_dtype == TMH_S8, d_a_zero, a_zero_count,
                                        d_b_zero, b_zero_count, M, K, N, b_batched != 0, static_cast<int32_t*>(d_y));
  return check_launch(ctx, "k_matmul_integer");
}

}  // extern "C"
