// Device-side helpers shared by the kernels: number formats, rounding, vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tmh {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

// Dequantization / storage types, as the ONNX codes of the C ABI.
enum : int { DT_F32 = 1, DT_F16 = 10, DT_BF16 = 16 };

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// The f32 value of an f32 result rounded to type DT (the reference computes each operation of
// a narrow type in f32 and rounds once).
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == DT_F16) {
    return static_cast<float>(static_cast<_Float16>(x));
  } else if constexpr (DT == DT_BF16) {
    return bf16_bits_to_f32(f32_to_bf16_bits(x));
  } else {
    return x;
  }
}

// (q - zero) * scale in type DT, each operation rounded (Packed.dequantize/3); zero and
// scale already hold DT values.
template <int DT>
__device__ __forceinline__ float dequant_value(float q, float zero, float scale) {
  float d = round_to<DT>(q - zero);
  return round_to<DT>(d * scale);
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == DT_F16) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else if constexpr (DT == DT_BF16) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return static_cast<const float*>(p)[i];
  }
}

// A float element of runtime type dt (1 = f32, 10 = f16, 16 = bf16).
__device__ __forceinline__ float load_float_rt(const void* p, int dt, int64_t i) {
  if (dt == DT_F16) return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dt == DT_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_float_rt(void* p, int dt, int64_t i, float v) {
  if (dt == DT_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  } else if (dt == DT_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

template <int DT>
__device__ __forceinline__ void store_as(void* p, int64_t i, float v) {
  if constexpr (DT == DT_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  } else if constexpr (DT == DT_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

// Value i (0 <= i < 32/BITS) of a 32-bit word of the tiled weight layout: value 2j at bits
// j*BITS, value 2j+1 at bits 16 + j*BITS (8-bit words keep their byte order).
template <int BITS>
__device__ __forceinline__ uint32_t word_value(uint32_t x, int i) {
  if constexpr (BITS == 8) {
    return (x >> (8 * i)) & 0xFFu;
  } else {
    const int pos = (i & 1) * 16 + (i >> 1) * BITS;
    return (x >> pos) & ((1u << BITS) - 1u);
  }
}

// Packed zero points of the tiled layout take BITS bits each, as in the reference's rows of
// packed zero points (two a byte for 4-bit weights, four for 2-bit, one for 8-bit): parameter
// entry e sits at bits zp_shift(e) of byte zp_byte(e). Entries are (tile, chunk, block, row r)
// with r = e % 16, so a lane's shift is that of its row, the same for every entry it reads.
template <int BITS, typename I>
__host__ __device__ constexpr I zp_byte(I e) {
  return e / (8 / BITS);
}
template <int BITS>
__host__ __device__ constexpr uint32_t zp_shift(uint32_t e) {
  return (e % (8 / BITS)) * BITS;
}
template <int BITS>
__device__ __forceinline__ uint32_t zp_field(uint32_t byte, uint32_t shift) {
  if constexpr (BITS == 8) return byte & 0xFFu;
  else return (byte >> shift) & ((1u << BITS) - 1u);
}

// (x & mask) | orv in one v_and_or_b32: the mask comes from an SGPR and orv from a VGPR, which
// the one-scalar-operand limit of VOP3 on this target allows (two literals would not).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t orv) {
  uint32_t out;
  asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(out) : "v"(x), "s"(mask), "v"(orv));
  return out;
}

// Eight exact f16 weights (q - zero) * scale of MFMA step i of a lane, from its 16 bytes.
// zz holds 1024 + zero and ss the scale as f16 (only the low halves are read: the packed
// operations take them as splats); a 16-bit half 0x6400 | q is the f16 number 1024 + q, so
// (0x6400 | q) - (1024 + zero) is q - zero exactly.
// 4 bits: the nibbles at bits 4-7 of each half are masked in place, 0x6400 | q << 4 = 1024 + 16q,
// and (1024 + 16q) / 16 - (64 + zero) is q - zero exactly in one fused multiply-add (every
// intermediate is a small integer); four pairs then take 5 bit operations instead of 7.
template <int BITS>
__device__ __forceinline__ half8_t unpack_step(const uint4_t& w, int i, half2_t zz, half2_t ss) {
  const half2_t z2 = {zz[0], zz[0]}, s2 = {ss[0], ss[0]};
  uint32_t pr[4];
  if constexpr (BITS == 4) {
    const uint32_t x = w[i];
    const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u);
    pr[0] = and_or(x, 0x000F000Fu, magic);
    pr[1] = and_or(x, 0x00F000F0u, magic);
    pr[2] = and_or(x >> 8, 0x000F000Fu, magic);
    pr[3] = and_or(x >> 8, 0x00F000F0u, magic);
    // 64 + zero: the zero's 4 bits moved under the f16 exponent of 64 (ulp 1/16).
    const uint16_t z64 = static_cast<uint16_t>(0x5400u + ((__builtin_bit_cast(uint16_t, zz[0]) & 0xFFu) << 4));
    const _Float16 z64h = __builtin_bit_cast(_Float16, z64);
    const half2_t z16 = {z64h, z64h};
    const half2_t sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    half8_t out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half2_t q = __builtin_bit_cast(half2_t, pr[j]);
      const half2_t d = (j & 1) ? __builtin_elementwise_fma(q, sixteenth, -z16) : q - z2;
      const half2_t wv = d * s2;
      out[2 * j] = wv[0];
      out[2 * j + 1] = wv[1];
    }
    return out;
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t x = w[2 * i + h];
      pr[2 * h] = (x & 0xFFu) | ((x << 8) & 0x00FF0000u) | 0x64006400u;
      pr[2 * h + 1] = ((x >> 16) & 0xFFu) | ((x >> 8) & 0x00FF0000u) | 0x64006400u;
    }
  } else {  // 2 bits: step i uses half of word i/2
    const uint32_t x = w[i >> 1] >> (8 * (i & 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) pr[j] = ((x >> (2 * j)) & 0x00030003u) | 0x64006400u;
  }
  half8_t out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const half2_t q = __builtin_bit_cast(half2_t, pr[j]);
    const half2_t wv = (q - z2) * s2;
    out[2 * j] = wv[0];
    out[2 * j + 1] = wv[1];
  }
  return out;
}

// XOR swizzle of the 16-byte pieces of LDS rows that 16 lanes read as MFMA fragments (lane r of a
// lane group reads row r, all lanes the same piece): piece p of row r sits in slot
// p ^ frag_swizzle<PPR>(r). The values were found by timing ds_read_b128 over candidate tables on
// MI355X: with them a wavefront's read has no bank conflict, while p ^ r (the textbook choice)
// spends half the LDS's active cycles on conflicts (1.7x slower). PPR = pieces per row: 16
// (256-byte rows) or 32 use a transposed nibble of r, 8 (128-byte rows) bits 1-3 of r.
template <int PPR>
__device__ __forceinline__ int frag_swizzle(int r) {
  if constexpr (PPR == 8) return (((r >> 1) & 1) << 1) | ((r >> 2) & 1) | (((r >> 3) & 1) << 2);
  else return ((r & 3) << 2) | ((r >> 2) & 3);
}

// Raw buffer resource over `bytes` bytes: a load whose VGPR offset is at or beyond `bytes`
// returns zeros, so tiles past N need no address clamps or selects. Every in-range access of
// these kernels stays inside its buffer.
// Cache policy of a buffer store whose data no later instruction of the kernel reads: the nt
// bit (streaming), so an output written once does not displace the inputs still being read.
constexpr int kNonTemporal = 2;
// Cache policy sc1 (device scope): the store writes its line through the XCD's L2, so the line
// is not left dirty there for the write-back at the kernel's end, which the next launch on the
// stream waits for. It pays where a kernel's stores overlap its later work (split-K partial
// sums, the row gather); where the stores come last (a GEMV's output) they only finish later.
constexpr int kWriteThrough = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

// 16 bytes per lane from a buffer straight into LDS at lds + 16 * lane (buffer_load_dwordx4
// ... lds: the data never passes through VGPRs). `lds` must be wavefront-uniform. The body
// exists in the device pass only; the host pass of hipcc does not accept LDS address spaces.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, uint32_t voffset,
                                          uint32_t soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(lds), 16, voffset,
                                           soffset, 0, 0);
#endif
}

// Timeline stamps of the measurement builds of a kernel (tmh_timeline_begin): the low 32 bits of
// the GPU's constant 100 MHz real-time counter and of the shader clock's cycle counter.
struct TlStart {
  uint32_t real, cycles;
};

__device__ __forceinline__ TlStart tl_clock() {
  return TlStart{static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime()),
                 static_cast<uint32_t>(__builtin_amdgcn_s_memtime())};
}

// Writes this wavefront's stamps into its 16-byte slot (linear workgroup * wavefronts per
// workgroup + wavefront) of the launch's slots: real-time start and end, cycle counter start
// and end. The end is read once every memory access the wavefront issued has completed. Lane 0
// must call it (it stores); other lanes may.
__device__ __forceinline__ void tl_stamp(uint32_t* tl, TlStart t0) {
  __builtin_amdgcn_s_waitcnt(0);
  const TlStart t1 = tl_clock();
  const uint32_t block = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const uint32_t wave = block * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if ((threadIdx.x & 63) == 0)
    *reinterpret_cast<uint4*>(tl + 4 * static_cast<size_t>(wave)) = make_uint4(t0.real, t1.real, t0.cycles, t1.cycles);
}

}  // namespace tmh
