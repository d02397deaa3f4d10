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

// Rows of whole 256-byte slices (row_bytes % 256 == 0), 4 bytes per lane in one quantization
// block, 16-byte-aligned output: each wavefront takes S consecutive (id, slice) pairs. Lane j
// loads slice j's id (one vector load for the wavefront) and each row is broadcast from its lane;
// the data, scale and zero point loads of all S slices then issue before the first value is
// computed, so a wavefront pays the id latency and the row latency once for S slices instead of
// once per half row. Each slice's values leave as one 16-byte store per lane (1 KiB contiguous
// per instruction), written through the L2 (kWriteThrough): at the [8, 512] x 1024 f16 lookup the
// 8 MiB of output cost 1.4 us over an empty launch with ordinary stores and 0.9 us with
// non-temporal ones, and written through 3.6 against 3.7 us per lookup in graph replays (the next
// launch then waits on no write-back of dirty lines; non-temporal and written through, 3.6 us at
// 3.0 against 3.05 TB/s). A slice past the
// end (the last wavefront's) stores to an offset beyond the output buffer's range, which the
// hardware drops: no branch, so no slice's loads wait behind another's stores. `spr_magic` is
// floor(2^32 / slices_per_row) + 1 (slices_per_row > 1): umulhi(sl, spr_magic) equals
// sl / slices_per_row for every sl < 2^32 / slices_per_row, which the launcher checks.
// (The body; k_gather_bq_rows and its stamping build k_gather_bq_rows_tl below are the kernels.)
template <int DT, int BITS, int S, bool IDS64, bool HAS_ZP, bool TL>
__device__ __forceinline__ void gather_bq_rows(
    const uint8_t* __restrict__ data, bool data_signed, uint32_t rows, uint32_t row_bytes,
    const void* __restrict__ ids, uint32_t n_slices, uint32_t slices_per_row, uint32_t spr_magic,
    const void* __restrict__ scales, uint32_t blocks, uint32_t bs_shift, const uint8_t* __restrict__ zp,
    bool zp_signed, uint32_t zrow, void* __restrict__ out, uint32_t* __restrict__ tl) {
  const TlStart tl0 = TL ? tl_clock() : TlStart{0u, 0u};
  constexpr int PER = 8 / BITS;
  constexpr int V = 4 * PER;  // values per lane and slice
  constexpr int ES = DT == DT_F32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  const uint32_t s0 = wave * S;
  if (s0 >= n_slices) {
    if constexpr (TL) tl_stamp(tl, tl0);
    return;
  }
  const uint32_t D = row_bytes * PER;
  const auto d_rsrc = buffer_rsrc(data, rows * row_bytes);
  const auto s_rsrc = buffer_rsrc(scales, rows * blocks * ES);
  const auto z_rsrc = buffer_rsrc(zp, HAS_ZP ? rows * zrow : 0u);
  const auto o_rsrc = buffer_rsrc(out, (n_slices / slices_per_row) * D * ES);
  // The rows of the S slices first (lane j loads slice j's id, one vector load, then each row
  // is broadcast from its lane), then every data, scale and zero point load, then the values.
  const uint32_t my_sl = s0 + (lane < S ? lane : S - 1) < n_slices ? s0 + (lane < S ? lane : S - 1) : n_slices - 1;
  int64_t my_id;
  const uint32_t my_i = slices_per_row == 1 ? my_sl : __umulhi(my_sl, spr_magic);
  if constexpr (IDS64) my_id = static_cast<const int64_t*>(ids)[my_i];
  else my_id = static_cast<const int32_t*>(ids)[my_i];
  my_id = my_id < 0 ? my_id + rows : my_id;  // ONNX: a negative index counts from the end
  const uint32_t my_row = static_cast<uint32_t>(my_id < 0 ? 0 : (my_id >= rows ? rows - 1 : my_id));
  uint32_t row[S];
#pragma unroll
  for (int j = 0; j < S; ++j) row[j] = __builtin_amdgcn_readlane(my_row, j);
  uint32_t x[S], sv[S], zv[S];
  uint32_t bit[S];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const uint32_t sl = s0 + j < n_slices ? s0 + j : n_slices - 1;
    const uint32_t i = slices_per_row == 1 ? sl : __umulhi(sl, spr_magic);
    const uint32_t r = row[j];
    const uint32_t byte = (sl - i * slices_per_row) * 256 + lane * 4;
    const uint32_t blk = (byte * PER) >> bs_shift;
    x[j] = __builtin_amdgcn_raw_buffer_load_b32(d_rsrc, r * row_bytes + byte, 0, 0);
    if constexpr (ES == 4) sv[j] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, (r * blocks + blk) * 4, 0, 0);
    else sv[j] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, (r * blocks + blk) * 2, 0, 0);
    bit[j] = blk * BITS;
    if constexpr (HAS_ZP) zv[j] = __builtin_amdgcn_raw_buffer_load_b8(z_rsrc, r * zrow + bit[j] / 8, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const uint32_t sl = s0 + j;
    const uint32_t i = slices_per_row == 1 ? sl : __umulhi(sl, spr_magic);
    uint32_t words[V * ES / 4];
    if constexpr (DT == DT_F16) {
      // Packed f16: each 32-bit word holds the values 2k, 2k+1 as 1024 + q (0x6400 | q), the
      // nibbles' high one at bits 20-23 (1024 + 16 q), so one fma per pair gives q - zero
      // exactly and one multiply by the scale rounds once, as the f32 product rounded to f16
      // does (the product of two f16 values is exact in f32). Signed values are offset by
      // 2^(BITS-1) (their top bit flipped), and the zero point with them.
      constexpr int HALF = 1 << (BITS - 1);
      int zq;
      if constexpr (HAS_ZP) {
        if constexpr (BITS == 8) {
          zq = zp_signed ? static_cast<int>(static_cast<int8_t>(zv[j])) : static_cast<int>(zv[j] & 0xFFu);
        } else {
          zq = (zv[j] >> (bit[j] % 8)) & ((1 << BITS) - 1);
          if (zp_signed && zq >= HALF) zq -= (1 << BITS);
        }
      } else {
        zq = data_signed ? 0 : HALF;
      }
      const int zz = zq + (data_signed ? HALF : 0);
      const uint32_t xs = data_signed ? x[j] ^ (BITS == 4 ? 0x88888888u : 0x80808080u) : x[j];
      const _Float16 s16 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(sv[j]));
      const half2_t s2 = {s16, s16};
      if constexpr (BITS == 4) {
        const half2_t mul = {static_cast<_Float16>(1.0f), static_cast<_Float16>(0.0625f)};
        const half2_t add = {static_cast<_Float16>(-(1024 + zz)), static_cast<_Float16>(-(64 + zz))};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t p = (__builtin_amdgcn_perm(xs, xs, 0x01010101u * k) & 0x00F0000Fu) | 0x64006400u;
          const half2_t d = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, p), mul, add);
          words[k] = __builtin_bit_cast(uint32_t, d * s2);
        }
      } else {
        const _Float16 a = static_cast<_Float16>(-(1024 + zz));
        const half2_t add = {a, a};
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const uint32_t sel = (2 * k) * 0x00000101u + (2 * k + 1) * 0x01010000u;  // bytes 2k, 2k+1 to 0, 2
          const uint32_t p = (__builtin_amdgcn_perm(xs, xs, sel) & 0x00FF00FFu) | 0x64006400u;
          const half2_t d = __builtin_bit_cast(half2_t, p) + add;
          words[k] = __builtin_bit_cast(uint32_t, d * s2);
        }
      }
    } else {
      float z;
      if constexpr (HAS_ZP) {
        int zq;
        if constexpr (BITS == 8) {
          zq = zp_signed ? static_cast<int>(static_cast<int8_t>(zv[j])) : static_cast<int>(zv[j] & 0xFFu);
        } else {
          zq = (zv[j] >> (bit[j] % 8)) & ((1 << BITS) - 1);
          if (zp_signed && zq >= (1 << (BITS - 1))) zq -= (1 << BITS);
        }
        z = static_cast<float>(zq);
      } else {
        z = data_signed ? 0.f : static_cast<float>(1 << (BITS - 1));
      }
      float sc;
      if constexpr (DT == DT_F32) sc = __builtin_bit_cast(float, sv[j]);
      else if constexpr (DT == DT_F16) sc = f16_bits_to_f32(static_cast<uint16_t>(sv[j]));
      else sc = bf16_bits_to_f32(static_cast<uint16_t>(sv[j]));
      float vals[V];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (x[j] >> (8 * b)) & 0xFFu;
#pragma unroll
        for (int v = 0; v < PER; ++v) {
          int q;
          if constexpr (BITS == 8) {
            q = data_signed ? static_cast<int>(static_cast<int8_t>(byte)) : static_cast<int>(byte);
          } else {
            q = (byte >> (v * BITS)) & ((1 << BITS) - 1);
            if (data_signed && q >= (1 << (BITS - 1))) q -= (1 << BITS);
          }
          vals[b * PER + v] = dequant_value<DT>(static_cast<float>(q), z, sc);
        }
      }
#pragma unroll
      for (int k = 0; k < V * ES / 4; ++k) {
        if constexpr (DT == DT_F32) words[k] = __builtin_bit_cast(uint32_t, vals[k]);
        else words[k] = f32_to_bf16_bits(vals[2 * k]) | (static_cast<uint32_t>(f32_to_bf16_bits(vals[2 * k + 1])) << 16);
      }
    }
    const uint32_t o = (i * D + ((sl - i * slices_per_row) * 256 + lane * 4) * PER) * ES;
    const uint32_t off = sl < n_slices ? o : 0xFFFFFF00u;  // past the range: dropped
    if constexpr (V * ES == 8) {  // 8-bit values in a 2-byte type: 8 bytes per lane
      typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
      __builtin_amdgcn_raw_buffer_store_b64(uint2_t{words[0], words[1]}, o_rsrc, off, 0, kWriteThrough);
    } else {
#pragma unroll
      for (int k = 0; k < V * ES / 16; ++k)
        __builtin_amdgcn_raw_buffer_store_b128(uint4_t{words[4 * k], words[4 * k + 1], words[4 * k + 2], words[4 * k + 3]},
                                               o_rsrc, off + 16 * k, 0, kWriteThrough);
    }
  }
  if constexpr (TL) tl_stamp(tl, tl0);
}

template <int DT, int BITS, int S, bool IDS64, bool HAS_ZP>
__global__ __launch_bounds__(256) void k_gather_bq_rows(
    const uint8_t* __restrict__ data, bool data_signed, uint32_t rows, uint32_t row_bytes,
    const void* __restrict__ ids, uint32_t n_slices, uint32_t slices_per_row, uint32_t spr_magic,
    const void* __restrict__ scales, uint32_t blocks, uint32_t bs_shift, const uint8_t* __restrict__ zp,
    bool zp_signed, uint32_t zrow, void* __restrict__ out) {
  gather_bq_rows<DT, BITS, S, IDS64, HAS_ZP, false>(data, data_signed, rows, row_bytes, ids, n_slices, slices_per_row,
                                                    spr_magic, scales, blocks, bs_shift, zp, zp_signed, zrow, out,
                                                    nullptr);
}

template <int DT, int BITS, int S, bool IDS64, bool HAS_ZP>
__global__ __launch_bounds__(256) void k_gather_bq_rows_tl(
    const uint8_t* __restrict__ data, bool data_signed, uint32_t rows, uint32_t row_bytes,
    const void* __restrict__ ids, uint32_t n_slices, uint32_t slices_per_row, uint32_t spr_magic,
    const void* __restrict__ scales, uint32_t blocks, uint32_t bs_shift, const uint8_t* __restrict__ zp,
    bool zp_signed, uint32_t zrow, void* __restrict__ out, uint32_t* __restrict__ tl) {
  gather_bq_rows<DT, BITS, S, IDS64, HAS_ZP, true>(data, data_signed, rows, row_bytes, ids, n_slices, slices_per_row,
                                                   spr_magic, scales, blocks, bs_shift, zp, zp_signed, zrow, out, tl);
}

template <int DT, int BITS, bool IDS64, bool HAS_ZP>
void launch_gather_rows(const uint8_t* data, bool sgn, int64_t rows, int64_t row_bytes, const void* ids,
                        int64_t n_ids, const void* scales, int64_t blocks, int64_t bs, const void* zp,
                        bool zp_signed, int64_t zrow, void* out, hipStream_t s) {
  constexpr int S = 4;
  const int64_t spr = row_bytes / 256, n_slices = n_ids * spr;
  int shift = 0;
  while ((int64_t(1) << shift) < bs) ++shift;
  const int64_t waves = (n_slices + S - 1) / S;
  const auto magic = static_cast<uint32_t>((uint64_t(1) << 32) / static_cast<uint64_t>(spr) + 1);
  const unsigned grid = static_cast<unsigned>((waves + 3) / 4);
#define TMH_GATHER_ARGS                                                                                               \
  data, sgn, static_cast<uint32_t>(rows), static_cast<uint32_t>(row_bytes), ids, static_cast<uint32_t>(n_slices),    \
      static_cast<uint32_t>(spr), magic, scales, static_cast<uint32_t>(blocks), static_cast<uint32_t>(shift),         \
      static_cast<const uint8_t*>(zp), zp_signed, static_cast<uint32_t>(zrow), out
  if (uint32_t* tl = timeline_slots(TMH_TL_GATHER_ROWS, static_cast<int64_t>(grid) * 4))
    k_gather_bq_rows_tl<DT, BITS, S, IDS64, HAS_ZP><<<grid, 256, 0, s>>>(TMH_GATHER_ARGS, tl);
  else
    k_gather_bq_rows<DT, BITS, S, IDS64, HAS_ZP><<<grid, 256, 0, s>>>(TMH_GATHER_ARGS);
#undef TMH_GATHER_ARGS
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
    // Whole 256-byte slices, power-of-two blocks, no or packed zero points and 32-bit offsets:
    // several slices per wavefront.
    const bool packed_zp = zp && (zp_dt == TMH_U8 || zp_dt == TMH_S8);
    if constexpr (BITS != 2) {
      if (one && vec_out && row_bytes % 256 == 0 && (bs & (bs - 1)) == 0 && (!zp || packed_zp) &&
          rows * row_bytes < (int64_t(1) << 32) && rows * blocks * ES < (int64_t(1) << 32) &&
          rows * zrow < (int64_t(1) << 32) && n_ids * D * ES < (int64_t(1) << 32) - 256 &&
          n_ids * (row_bytes / 256) * (row_bytes / 256) < (int64_t(1) << 32)) {
        const bool zs = zp_dt == TMH_S8;
        if (ids64 && zp) launch_gather_rows<DT, BITS, true, true>(data, sgn, rows, row_bytes, ids, n_ids, scales, blocks, bs, zp, zs, zrow, out, s);
        else if (ids64) launch_gather_rows<DT, BITS, true, false>(data, sgn, rows, row_bytes, ids, n_ids, scales, blocks, bs, zp, zs, zrow, out, s);
        else if (zp) launch_gather_rows<DT, BITS, false, true>(data, sgn, rows, row_bytes, ids, n_ids, scales, blocks, bs, zp, zs, zrow, out, s);
        else launch_gather_rows<DT, BITS, false, false>(data, sgn, rows, row_bytes, ids, n_ids, scales, blocks, bs, zp, zs, zrow, out, s);
        return;
      }
    }
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

// The same values for tensors of fewer than 2^31 elements: four consecutive elements per thread,
// one 32-bit split of the first index into (outer, axis, inner) and a step for the rest, and an
// 8- or 16-byte store when y is aligned for it.
template <int OUT>
__global__ __launch_bounds__(256) void k_dequantize_linear4(
    const void* __restrict__ x, int x_dt, bool x_int, uint32_t dim, uint32_t inner,
    const void* __restrict__ scale, int scale_dt, const void* __restrict__ zero, int zero_dt,
    int mode, uint32_t bs, uint32_t nb, void* __restrict__ y, uint32_t total, bool y_vec) {
  const uint32_t e0 = (blockIdx.x * blockDim.x + threadIdx.x) * 4u;
  if (e0 >= total) return;
  const uint32_t per_outer = dim * inner;
  uint32_t o = e0 / per_outer;
  const uint32_t rem = e0 - o * per_outer;
  uint32_t d = rem / inner;
  uint32_t in = rem - d * inner;
  float out[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t e = e0 + j;
    if (e < total) {
      uint32_t p = 0;
      if (mode == TMH_QPARAM_AXIS) p = d;
      else if (mode == TMH_QPARAM_BLOCKED) p = (o * nb + d / bs) * inner + in;
      float v;
      if (x_int) {
        uint32_t shifted = static_cast<uint32_t>(load_int_rt(x, x_dt, e));
        if (zero) shifted -= static_cast<uint32_t>(load_int_rt(zero, zero_dt, p));
        v = static_cast<float>(static_cast<int32_t>(shifted));
      } else {
        v = load_float_rt(x, x_dt, e);
        if (zero) v = v - load_float_rt(zero, zero_dt, p);
      }
      out[j] = v * load_float_rt(scale, scale_dt, p);
    }
    if (++in == inner) {
      in = 0;
      if (++d == dim) {
        d = 0;
        ++o;
      }
    }
  }
  if (y_vec && e0 + 4 <= total) {
    if constexpr (OUT == DT_F32) {
      *reinterpret_cast<float4_t*>(static_cast<float*>(y) + e0) = float4_t{out[0], out[1], out[2], out[3]};
    } else {
      uint16_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = OUT == DT_F16 ? f32_to_f16_bits(out[j]) : f32_to_bf16_bits(out[j]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + e0) =
          make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (e0 + j < total) store_as<OUT>(y, e0 + j, out[j]);
  }
}

// DequantizeLinear of 1-byte integers (SIGNED: s8) with per-tensor parameters or parameters
// along the last axis (AXIS, dim % 4 == 0): four elements per thread from one 4-byte load, their
// four scales and zero points (1-byte, x's type) from one 8/16-byte and one 4-byte load. Same
// arithmetic as k_dequantize_linear4: the exact integer x - zero in f32, times the scale read as
// f32, rounded once to the scale's type OUT.
template <int OUT, bool SIGNED, bool HAS_ZERO, bool AXIS>
__global__ __launch_bounds__(256) void k_dequantize_linear_b4(const uint32_t* __restrict__ x,
                                                              const void* __restrict__ scale,
                                                              const uint32_t* __restrict__ zero, uint32_t dim,
                                                              void* __restrict__ y, uint32_t quads) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= quads) return;
  const uint32_t xv = x[t];
  float sc[4];
  uint32_t zv = 0;
  if constexpr (AXIS) {
    const uint32_t d4 = (t * 4u) % dim / 4u;  // the four elements share a row: parameters d .. d+3
    if constexpr (OUT == DT_F32) {
      const float4_t v = reinterpret_cast<const float4_t*>(scale)[d4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = v[j];
    } else {
      const uint2 v = reinterpret_cast<const uint2*>(scale)[d4];
      const uint32_t w[2] = {v.x, v.y};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const auto h = static_cast<uint16_t>(w[j / 2] >> (16 * (j % 2)));
        sc[j] = OUT == DT_F16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
      }
    }
    if constexpr (HAS_ZERO) zv = zero[d4];
  } else {
    const float s0 = load_as_f32<OUT>(scale, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = s0;
    if constexpr (HAS_ZERO) zv = (reinterpret_cast<const uint8_t*>(zero)[0]) * 0x01010101u;
  }
  float out[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t xb = (xv >> (8 * j)) & 0xFFu, zb = (zv >> (8 * j)) & 0xFFu;
    const int q = SIGNED ? static_cast<int>(static_cast<int8_t>(xb)) : static_cast<int>(xb);
    const int z = SIGNED ? static_cast<int>(static_cast<int8_t>(zb)) : static_cast<int>(zb);
    out[j] = static_cast<float>(q - z) * sc[j];
  }
  // Non-temporal stores: the output (four times the input's bytes in f32) is not read again here.
  if constexpr (OUT == DT_F32) {
    __builtin_nontemporal_store(float4_t{out[0], out[1], out[2], out[3]}, reinterpret_cast<float4_t*>(y) + t);
  } else {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    uint16_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = OUT == DT_F16 ? f32_to_f16_bits(out[j]) : f32_to_bf16_bits(out[j]);
    __builtin_nontemporal_store(u32x2_t{h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16)},
                                reinterpret_cast<u32x2_t*>(y) + t);
  }
}

template <int OUT, bool SIGNED>
void launch_dql_b4(const void* x, const void* scale, const void* zero, bool axis, uint32_t dim, void* y,
                   uint32_t quads, hipStream_t s) {
  const dim3 grid((quads + 255) / 256);
  const auto* xq = static_cast<const uint32_t*>(x);
  const auto* zq = static_cast<const uint32_t*>(zero);
  if (axis) {
    if (zero)
      k_dequantize_linear_b4<OUT, SIGNED, true, true><<<grid, 256, 0, s>>>(xq, scale, zq, dim, y, quads);
    else
      k_dequantize_linear_b4<OUT, SIGNED, false, true><<<grid, 256, 0, s>>>(xq, scale, zq, dim, y, quads);
  } else if (zero) {
    k_dequantize_linear_b4<OUT, SIGNED, true, false><<<grid, 256, 0, s>>>(xq, scale, zq, dim, y, quads);
  } else {
    k_dequantize_linear_b4<OUT, SIGNED, false, false><<<grid, 256, 0, s>>>(xq, scale, zq, dim, y, quads);
  }
}

// ------------------------------------------------------------------ MatMulInteger on int8 MFMA

// y[bt, m, n] = sum_k (a - a_zero[m]) (b - b_zero[n]), wrapping mod 2^32. Each f32 chunk sum of
// the reference is exact, so the exact integer sum is its value. With a = sa + oa (sa the s8
// form of a: the byte itself for s8 data, a ^ 0x80 = a - 128 for u8 data, so oa is 0 or 128)
// and likewise b:
//   sum_k (a - az_m)(b - bz_n) = sum_k sa sb + cb_n * rs_m + ca_m * cs_n + K * ca_m * cb_n
// with ca_m = oa - az_m, cb_n = ob - bz_n, rs_m = sum_k sa[m][k], cs_n = sum_k sb[k][n], all
// modulo 2^32. The sa sb sums run on v_mfma_i32_16x16x64_i8; rs and cs are summed (v_dot4
// against ones) from the same bytes as they are staged into LDS.

constexpr int kI8Tile = 128;  // output rows and columns per workgroup
constexpr int kI8K = 128;     // k per step: two MFMAs deep

// LDS tiles hold 128 rows (A rows, or B columns) of 128 k-bytes, no padding; the 16-byte chunk
// c of row x sits at chunk c ^ ((x & 7) ^ ((x >> 3) & 7)). Eight consecutive rows reading one
// chunk (an MFMA fragment read) then hit eight different chunks, and the B columns one
// wavefront's 4-byte writes cover (8 apart) spread over them too.
__device__ __forceinline__ int i8_lds_offset(int x, int chunk) {
  return x * kI8K + ((chunk ^ ((x & 7) ^ ((x >> 3) & 7))) << 4);
}

__device__ __forceinline__ uint32_t dot4_ones(uint32_t w, uint32_t acc) {
  return static_cast<uint32_t>(__builtin_amdgcn_sdot4(static_cast<int>(w), 0x01010101, static_cast<int>(acc), false));
}

typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

// 128 x 128 outputs per workgroup of eight wavefronts, two per SIMD (64 x 32 each, 4 x 2 MFMA
// tiles), so one wavefront's stalls are covered by the other's work. Each k-step's A rows
// (16 bytes per load) and B rows (4 k-rows x 8 columns per thread) are read into registers while
// the previous step's MFMAs run, then stored to LDS as s8: A as is, B transposed to k-contiguous
// columns through 4 x 4 byte blocks (v_perm). Zeros outside the matrices.
// VEC: K and N are multiples of 16, both matrices 16-byte aligned, (M + 128) K and (K + 128) N
// below 2^31; every load is then one unconditional buffer load at a 32-bit offset formed once
// and advanced per step (a branch per load makes the compiler wait for each load in turn).
template <bool VEC>
__global__ __launch_bounds__(512) void k_matmul_integer_mfma(
    const uint8_t* __restrict__ a, bool a_signed, const uint8_t* __restrict__ b, bool b_signed,
    const uint8_t* __restrict__ a_zero, int64_t a_zero_count, const uint8_t* __restrict__ b_zero,
    int64_t b_zero_count, int64_t M, int64_t K, int64_t N, bool b_batched, int32_t* __restrict__ y) {
  __shared__ __align__(16) uint8_t sA[kI8Tile * kI8K];
  __shared__ __align__(16) uint8_t sB[kI8Tile * kI8K];
  __shared__ uint32_t sRs[kI8Tile];
  __shared__ uint32_t sCs[8][kI8Tile];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int r = lane & 15, g = lane >> 4;
  const int64_t bt = blockIdx.z;
  // Workgroups go to the eight XCDs round-robin by linear id. When the tile count is a multiple
  // of 8, XCD x takes tiles [x T/8, (x+1) T/8) of an order that walks groups of four m-tiles
  // m-fastest, so one XCD's tiles share few A rows and B columns (its own L2).
  uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
  const uint32_t tiles = gridDim.x * gridDim.y;
  if (tiles % 8 == 0) tile = (tile % 8) * (tiles / 8) + tile / 8;
  const uint32_t group = tile / (4 * gridDim.x), first_m = 4 * group;
  const uint32_t group_m = min(4u, gridDim.y - first_m), in_group = tile - group * 4 * gridDim.x;
  const int64_t m0 = static_cast<int64_t>(first_m + in_group % group_m) * kI8Tile;
  const int64_t n0 = static_cast<int64_t>(in_group / group_m) * kI8Tile;
  const uint8_t* a8 = a + bt * M * K;
  const uint8_t* b8 = b + (b_batched ? bt * K * N : 0);
  const uint32_t aflip = a_signed ? 0u : 0x80808080u, bflip = b_signed ? 0u : 0x80808080u;
  // This thread's share of a k-step: A rows (tid >> 3) + 64h, chunk tid & 7 (h = 0, 1); B k-rows
  // 4 * (tid >> 4) + i (i = 0..3), columns 8 * (tid & 15) + j (j = 0..7).
  const int a_row = tid >> 3, a_chunk = tid & 7;
  const int b_kq = tid >> 4, b_nq = tid & 15;
  // va/vb hold the loaded bytes. For VEC the loads are unconditional, and amask (bytes to keep)
  // and bmask (flip to apply) are applied when the bytes go to LDS, so the loads of the next
  // step are not waited for before this step's MFMAs. Rows of A past M and k-rows of B past K
  // lie outside the buffer ranges and read zeros; A bytes past K belong to the next row and are
  // masked; B columns past N reach only outputs that are never stored.
  uint4_t va[2];
  uint2_t vb[4];
  uint32_t amask[2] = {0u, 0u}, bmask[4] = {0u, 0u, 0u, 0u};
  const auto a_rsrc = buffer_rsrc(a8, VEC ? static_cast<uint32_t>(M * K) : 0u);
  const auto b_rsrc = buffer_rsrc(b8, VEC ? static_cast<uint32_t>(K * N) : 0u);
  uint32_t a_off[2] = {0u, 0u}, b_off[4] = {0u, 0u, 0u, 0u};
  if constexpr (VEC) {
#pragma unroll
    for (int h = 0; h < 2; ++h) a_off[h] = static_cast<uint32_t>((m0 + a_row + 64 * h) * K + 16 * a_chunk);
#pragma unroll
    for (int i = 0; i < 4; ++i) b_off[i] = static_cast<uint32_t>((4 * b_kq + i) * N + n0 + 8 * b_nq);
  }
  const uint32_t b_step = static_cast<uint32_t>(kI8K * N);
  auto load = [&](int64_t k0, uint32_t step) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t gk = k0 + 16 * a_chunk;
      if constexpr (VEC) {
        va[h] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_off[h] + step * kI8K, 0, 0);
        amask[h] = gk < K ? 0xFFFFFFFFu : 0u;
      } else {
        const int64_t gm = m0 + a_row + 64 * h;
        uint4_t v = {0u, 0u, 0u, 0u};
        if (gm < M && gk < K)
          for (int e = 0; e < 16; ++e)
            if (gk + e < K) v[e >> 2] |= static_cast<uint32_t>(a8[gm * K + gk + e] ^ (aflip & 0xFFu)) << (8 * (e & 3));
        va[h] = v;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t gk = k0 + 4 * b_kq + i;
      if constexpr (VEC) {
        vb[i] = __builtin_amdgcn_raw_buffer_load_b64(b_rsrc, b_off[i] + step * b_step, 0, 0);
        bmask[i] = gk < K ? bflip : 0u;
      } else {
        const int64_t gn = n0 + 8 * b_nq;
        uint2_t v = {0u, 0u};
        if (gk < K && gn < N)
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) v[e >> 2] |= static_cast<uint32_t>(b8[gk * N + gn + e] ^ (bflip & 0xFFu)) << (8 * (e & 3));
        vb[i] = v;
      }
    }
  };
  uint32_t rsum[2] = {0u, 0u};
  uint32_t csum[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) csum[j] = 0u;
  int4_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = int4_t{0, 0, 0, 0};
  if (K > 0) load(0, 0u);
  uint32_t step = 0;
  for (int64_t k0 = 0; k0 < K; k0 += kI8K, ++step) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint4_t v = va[h];
      if constexpr (VEC) v = (v ^ aflip) & amask[h];
      *reinterpret_cast<uint4_t*>(sA + i8_lds_offset(a_row + 64 * h, a_chunk)) = v;
#pragma unroll
      for (int q = 0; q < 4; ++q) rsum[h] = dot4_ones(v[q], rsum[h]);
    }
    // Column c of the 4 x 8 block is bytes c of vb[0..3]: word c >> 2 of each, byte c & 3.
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t x0 = vb[0][q] ^ bmask[0], x1 = vb[1][q] ^ bmask[1];
      const uint32_t x2 = vb[2][q] ^ bmask[2], x3 = vb[3][q] ^ bmask[3];
      const uint32_t lo01 = __builtin_amdgcn_perm(x1, x0, 0x05010400u), hi01 = __builtin_amdgcn_perm(x1, x0, 0x07030602u);
      const uint32_t lo23 = __builtin_amdgcn_perm(x3, x2, 0x05010400u), hi23 = __builtin_amdgcn_perm(x3, x2, 0x07030602u);
      const uint32_t col[4] = {__builtin_amdgcn_perm(lo23, lo01, 0x05040100u), __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                               __builtin_amdgcn_perm(hi23, hi01, 0x05040100u), __builtin_amdgcn_perm(hi23, hi01, 0x07060302u)};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = 8 * b_nq + 4 * q + e;
        *reinterpret_cast<uint32_t*>(sB + i8_lds_offset(n, b_kq >> 2) + 4 * (b_kq & 3)) = col[e];
        csum[4 * q + e] = dot4_ones(col[e], csum[4 * q + e]);
      }
    }
    __syncthreads();
    if (k0 + kI8K < K) load(k0 + kI8K, step + 1);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      int4_t af[4], bf[2];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        af[mt] = *reinterpret_cast<const int4_t*>(sA + i8_lds_offset(wm * 64 + mt * 16 + r, 4 * half + g));
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        bf[nt] = *reinterpret_cast<const int4_t*>(sB + i8_lds_offset(wn * 32 + nt * 16 + r, 4 * half + g));
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)  // B first: a lane ends with 4 consecutive columns of one row
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[nt], af[mt], acc[mt][nt], 0, 0, 0);
    }
    __syncthreads();
  }
  // rs: the 8 lanes of a row (consecutive) hold its 8 chunks' sums. cs: the 4 lanes of a
  // wavefront with one tid & 15 hold 4 of the 32 k-quads' sums, the eight wavefronts the rest.
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t v = rsum[h];
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    if (a_chunk == 0) sRs[a_row + 64 * h] = v;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t v = csum[j];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (lane < 16) sCs[wave][8 * b_nq + j] = v;
  }
  __syncthreads();
  if (tid < kI8Tile) {
    uint32_t v = sCs[0][tid];
#pragma unroll
    for (int w = 1; w < 8; ++w) v += sCs[w][tid];
    sCs[0][tid] = v;
  }
  __syncthreads();
  const uint32_t oa = a_signed ? 0u : 128u, ob = b_signed ? 0u : 128u;
  auto zero_of = [](const uint8_t* z, int64_t count, int64_t i, bool sgn) -> uint32_t {
    if (!z) return 0u;
    const uint8_t raw = z[count == 1 ? 0 : i];
    return sgn ? static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(raw))) : raw;
  };
  const uint32_t kk = static_cast<uint32_t>(K);
  const bool y_vec = (N % 4) == 0 && (reinterpret_cast<uintptr_t>(y) % 16) == 0;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int ml = wm * 64 + mt * 16 + r;
    const int64_t m = m0 + ml;
    if (m >= M) continue;
    const uint32_t ca = oa - zero_of(a_zero, a_zero_count, m, a_signed);
    const uint32_t rsm = sRs[ml];
    int32_t* yrow = y + (bt * M + m) * N;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int nl = wn * 32 + nt * 16 + 4 * g;
      const int64_t n = n0 + nl;
      if (n >= N) continue;
      int4_t out;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t cb = ob - zero_of(b_zero, b_zero_count, n + e < N ? n + e : n, b_signed);
        out[e] = static_cast<int32_t>(static_cast<uint32_t>(acc[mt][nt][e]) + cb * rsm + ca * sCs[0][nl + e] + kk * ca * cb);
      }
      if (y_vec) {
        // Non-temporal: the s32 output (four bytes per product) is not read again here (2048^3: 29.3 -> 27.1 us under the tracer).
        __builtin_nontemporal_store(out, reinterpret_cast<int4_t*>(yrow + n));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) yrow[n + e] = out[e];
      }
    }
  }
}

// ------------------------------------------------------------------ DynamicQuantizeLinear

// scale = (max(x, 0) - min(x, 0)) / 255 (1 when that is 0), zero = saturate(round(-low / scale)),
// in f32 with round-half-even, as quantized.ex:94-103.
__device__ __forceinline__ void dql_param_values(float low, float high, float& sc, uint8_t& zq) {
  low = fminf(low, 0.f);
  high = fmaxf(high, 0.f);
  sc = (high - low) / 255.f;
  if (sc == 0.f) sc = 1.f;
  const float z = rintf(-low / sc);
  zq = static_cast<uint8_t>(fminf(fmaxf(z, 0.f), 255.f));
}

__device__ __forceinline__ void dql_params(float low, float high, float* scale, uint8_t* zero) {
  float sc;
  uint8_t zq;
  dql_param_values(low, high, sc, zq);
  *scale = sc;
  *zero = zq;
}

// Minimum and maximum over the workgroup (up to 16 wavefronts, one value pair per lane): a
// shuffle reduction inside each wavefront, then one exchange through LDS; every thread ends with
// both. min and max do not depend on the order of their operands' combination.
__device__ __forceinline__ void dql_block_range(float& lo, float& hi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  __shared__ float lo_s[16], hi_s[16];
  const int waves = static_cast<int>(blockDim.x >> 6);
  if ((threadIdx.x & 63) == 0) {
    lo_s[threadIdx.x >> 6] = lo;
    hi_s[threadIdx.x >> 6] = hi;
  }
  __syncthreads();
  lo = lo_s[0];
  hi = hi_s[0];
  for (int w = 1; w < waves; ++w) {
    lo = fminf(lo, lo_s[w]);
    hi = fmaxf(hi, hi_s[w]);
  }
}

// Minimum and maximum of the workgroup's share of x (16-byte loads, four in flight per thread
// when x is 16-byte aligned); with one workgroup, the scale and zero point.
__global__ __launch_bounds__(256) void k_dql_minmax(const float* __restrict__ x, int64_t n, float* __restrict__ part,
                                                     float* __restrict__ scale, uint8_t* __restrict__ zero) {
  float lo = INFINITY, hi = -INFINITY;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t tail = 0;
  if ((reinterpret_cast<uintptr_t>(x) % 16) == 0) {
    const int64_t n4 = n / 4;
    const auto* x4 = reinterpret_cast<const float4_t*>(x);
    int64_t i = t;
    for (; i + 3 * stride < n4; i += 4 * stride) {
      float4_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = x4[i + u * stride];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo = fminf(lo, v[u][e]);
          hi = fmaxf(hi, v[u][e]);
        }
    }
    for (; i < n4; i += stride)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo = fminf(lo, x4[i][e]);
        hi = fmaxf(hi, x4[i][e]);
      }
    tail = n4 * 4;
  }
  for (int64_t i = tail + t; i < n; i += stride) {
    lo = fminf(lo, x[i]);
    hi = fmaxf(hi, x[i]);
  }
  dql_block_range(lo, hi);
  if (threadIdx.x != 0) return;
  if (gridDim.x == 1) {
    dql_params(lo, hi, scale, zero);
  } else {
    part[2 * blockIdx.x] = lo;
    part[2 * blockIdx.x + 1] = hi;
  }
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

// The quantize pass with the range reduction folded in: every workgroup issues its loads of x,
// then reduces the `parts` partial ranges (through LDS) to the scale and zero point (all
// workgroups compute the same values); workgroup 0 stores them. Grid-stride over groups of 1024 values,
// four per thread, so that few workgroups repeat the reduction.
__global__ __launch_bounds__(256) void k_dql_quantize_reduce(const float* __restrict__ x, int64_t n,
                                                              const float* __restrict__ part, int parts,
                                                              float* __restrict__ scale, uint8_t* __restrict__ zero,
                                                              uint8_t* __restrict__ y) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 1024;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 1024 + threadIdx.x * 4;
  const bool vec = (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (reinterpret_cast<uintptr_t>(y) % 4) == 0;
  float4_t v = float4_t{0.f, 0.f, 0.f, 0.f};
  if (vec && i + 4 <= n) v = *reinterpret_cast<const float4_t*>(x + i);
  float lo = INFINITY, hi = -INFINITY;
  for (int p = threadIdx.x; p < parts; p += blockDim.x) {
    lo = fminf(lo, part[2 * p]);
    hi = fmaxf(hi, part[2 * p + 1]);
  }
  dql_block_range(lo, hi);
  float sc;
  uint8_t zq;
  dql_param_values(lo, hi, sc, zq);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *scale = sc;
    *zero = zq;
  }
  const float z = static_cast<float>(zq);
  auto q = [&](float f) -> uint32_t { return static_cast<uint32_t>(fminf(fmaxf(rintf(f / sc) + z, 0.f), 255.f)); };
  // rint(x / sc) without the division, bit for bit: rcp = 1 / sc and q0 = x * rcp are each
  // rounded once, so q0 lies within |x / sc| 2^-22 of the rounded quotient; where q0 is further
  // than that from every half-integer (the only points where rint's result changes) both round to
  // the same integer. Otherwise (or where q0 is not finite) the wavefront takes the division for
  // its four values, a uniform branch so that the common case skips it (9.6 -> 9.0 us at 2048 x
  // 2048; computing both and selecting took 10.5).
  const float rcp = 1.f / sc;
  for (; i < n; i += stride) {
    if (vec && i + 4 <= n) {
      const float4_t w = v;
      if (i + stride + 4 <= n) v = *reinterpret_cast<const float4_t*>(x + i + stride);
      uint32_t packed = 0u;
      bool near_half = false;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float q0 = w[e] * rcp;
        const float frac = q0 - floorf(q0);
        near_half = near_half || !(fabsf(frac - 0.5f) > fabsf(q0) * 0x1p-21f);
        packed |= static_cast<uint32_t>(fminf(fmaxf(rintf(q0) + z, 0.f), 255.f)) << (8 * e);
      }
      if (__any(near_half)) packed = q(w[0]) | (q(w[1]) << 8) | (q(w[2]) << 16) | (q(w[3]) << 24);
      *reinterpret_cast<uint32_t*>(y + i) = packed;
    } else {
      for (int e = 0; e < 4 && i + e < n; ++e) y[i + e] = static_cast<uint8_t>(q(x[i + e]));
    }
  }
}

// The sums of an empty contraction (K = 0): every output is 0. A kernel rather than a memset, so
// a graph capture records a kernel node.
__global__ __launch_bounds__(256) void k_zero_s32(int32_t* __restrict__ y, int64_t n) {
  for (int64_t i = blockIdx.x * int64_t{256} + threadIdx.x; i < n; i += int64_t{gridDim.x} * 256) y[i] = 0;
}

}  // namespace

extern "C" {

int tmh_gather_block_quantized(tmh_ctx* ctx, const void* d_data, int data_dtype, int64_t rows,
                               int64_t row_bytes, const void* d_ids, int ids_dtype, int64_t n_ids,
                               const void* d_scales, int scales_dtype, int64_t blocks,
                               const void* d_zero_points, int zp_dtype, int bits, void* d_out,
                               void* stream) {
  TimelineScope timeline(ctx);
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
  {
    // 1-byte x with per-tensor or last-axis parameters: the vectorized kernel.
    const int out_bytes = scale_dtype == TMH_F16 || scale_dtype == TMH_BF16 ? 2 : 4;
    const auto aligned = [](const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
    const bool axis = mode == TMH_QPARAM_AXIS && inner == 1 && dim % 4 == 0;
    if ((x_dtype == TMH_U8 || x_dtype == TMH_S8) && (!d_zero || zero_dtype == x_dtype) &&
        (mode == TMH_QPARAM_TENSOR || axis) && total % 4 == 0 && total / 4 < (int64_t{1} << 31) &&
        aligned(d_x, 4) && aligned(d_y, 4 * out_bytes) && (!axis || aligned(d_scale, 4 * out_bytes)) &&
        (!axis || !d_zero || aligned(d_zero, 4))) {
      const auto quads = static_cast<uint32_t>(total / 4), d32 = static_cast<uint32_t>(dim);
      const bool sgn = x_dtype == TMH_S8;
      switch (scale_dtype) {
        case TMH_F16:
          sgn ? launch_dql_b4<DT_F16, true>(d_x, d_scale, d_zero, axis, d32, d_y, quads, s)
              : launch_dql_b4<DT_F16, false>(d_x, d_scale, d_zero, axis, d32, d_y, quads, s);
          break;
        case TMH_BF16:
          sgn ? launch_dql_b4<DT_BF16, true>(d_x, d_scale, d_zero, axis, d32, d_y, quads, s)
              : launch_dql_b4<DT_BF16, false>(d_x, d_scale, d_zero, axis, d32, d_y, quads, s);
          break;
        default:
          sgn ? launch_dql_b4<DT_F32, true>(d_x, d_scale, d_zero, axis, d32, d_y, quads, s)
              : launch_dql_b4<DT_F32, false>(d_x, d_scale, d_zero, axis, d32, d_y, quads, s);
      }
      return check_launch(ctx, "k_dequantize_linear_b4");
    }
  }
  if (total < (int64_t{1} << 31) - 4) {
    const int out_bytes = scale_dtype == TMH_F16 || scale_dtype == TMH_BF16 ? 2 : 4;
    const bool y_vec = reinterpret_cast<uintptr_t>(d_y) % (4 * out_bytes) == 0;
    const dim3 grid(static_cast<unsigned>((total + 1023) / 1024));
    const auto d32 = static_cast<uint32_t>(dim), i32 = static_cast<uint32_t>(inner), t32 = static_cast<uint32_t>(total);
    const auto bs32 = static_cast<uint32_t>(mode == TMH_QPARAM_BLOCKED ? block_size : 1), nb32 = static_cast<uint32_t>(nb);
    switch (scale_dtype) {
      case TMH_F16: k_dequantize_linear4<DT_F16><<<grid, 256, 0, s>>>(d_x, x_dtype, x_int, d32, i32, d_scale, scale_dtype, d_zero, zero_dtype, mode, bs32, nb32, d_y, t32, y_vec); break;
      case TMH_BF16: k_dequantize_linear4<DT_BF16><<<grid, 256, 0, s>>>(d_x, x_dtype, x_int, d32, i32, d_scale, scale_dtype, d_zero, zero_dtype, mode, bs32, nb32, d_y, t32, y_vec); break;
      default: k_dequantize_linear4<DT_F32><<<grid, 256, 0, s>>>(d_x, x_dtype, x_int, d32, i32, d_scale, scale_dtype, d_zero, zero_dtype, mode, bs32, nb32, d_y, t32, y_vec);
    }
    return check_launch(ctx, "k_dequantize_linear4");
  }
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
  if (K == 0) {
    // Nothing to contract: the sums are zeros (A and B hold no bytes, and may be NULL).
    if (!d_y) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger: NULL pointer");
    const int64_t n = batch * M * N;
    k_zero_s32<<<static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 4096)), 256, 0, pick_stream(ctx, stream)>>>(
        static_cast<int32_t*>(d_y), n);
    return check_launch(ctx, "k_zero_s32");
  }
  if (!d_a || !d_b || !d_y) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger: NULL pointer");
  if (batch > 65535) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger batch must be below 65536");
  if ((M + kI8Tile - 1) / kI8Tile > 65535)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger M=%lld exceeds %lld rows", (long long)M, 65535LL * kI8Tile);
  hipStream_t s = pick_stream(ctx, stream);
  const dim3 grid(static_cast<unsigned>((N + kI8Tile - 1) / kI8Tile), static_cast<unsigned>((M + kI8Tile - 1) / kI8Tile),
                  static_cast<unsigned>(batch));
  const bool vec = K % 16 == 0 && N % 16 == 0 && reinterpret_cast<uintptr_t>(d_a) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(d_b) % 16 == 0 && (M + kI8Tile) * K + kI8K < (int64_t{1} << 31) &&
                   (K + kI8K) * N + kI8Tile < (int64_t{1} << 31);
  auto* kernel = vec ? k_matmul_integer_mfma<true> : k_matmul_integer_mfma<false>;
  kernel<<<grid, 512, 0, s>>>(static_cast<const uint8_t*>(d_a), a_dtype == TMH_S8, static_cast<const uint8_t*>(d_b),
                              b_dtype == TMH_S8, static_cast<const uint8_t*>(d_a_zero), a_zero_count,
                              static_cast<const uint8_t*>(d_b_zero), b_zero_count, M, K, N, b_batched != 0,
                              static_cast<int32_t*>(d_y));
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
  // One workgroup per 16 Ki values, at most 2048; their partial ranges go through the workspace
  // (one workgroup does it all when there is none, inside a graph capture).
  int parts = static_cast<int>(std::min<int64_t>(2048, (n + 16383) / 16384));
  float* part = nullptr;
  if (parts > 1) {
    part = static_cast<float*>(workspace(ctx, static_cast<size_t>(parts) * 2 * sizeof(float), s));
    if (!part) parts = 1;
  }
  k_dql_minmax<<<static_cast<unsigned>(std::max(parts, 1)), 256, 0, s>>>(x, n, part, scale, zero);
  TMH_TRY(check_launch(ctx, "k_dql_minmax"));
  if (parts > 1) {
    const int64_t groups = (n + 1023) / 1024;
    k_dql_quantize_reduce<<<static_cast<unsigned>(std::min<int64_t>(groups, 1024)), 256, 0, s>>>(
        x, n, part, parts, scale, zero, static_cast<uint8_t*>(d_y));
    return check_launch(ctx, "k_dql_quantize_reduce");
  }
  if (n == 0) return TMH_OK;
  k_dql_quantize<<<static_cast<unsigned>((n + 1023) / 1024), 256, 0, s>>>(x, n, scale, zero, static_cast<uint8_t*>(d_y));
  return check_launch(ctx, "k_dql_quantize");
}

}  // extern "C"
