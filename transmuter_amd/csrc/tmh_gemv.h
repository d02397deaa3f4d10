// Decode GEMV kernel (M <= 16): f16 A, f16 weights from the tiled packed layout, f16 Y, an
// optional f16 bias.
//
// Reference: MatMulNBits (lib/transmuter/ops/quantized.ex:30-46) after move/2, the dot of
// quantized.ex:44 over dequantized {N, K} weights (Quantized.dequantize_weight/4, :234-240).
//
// A workgroup of NW wavefronts covers TN consecutive 16-column tiles. Its wavefronts split the
// chunks of K, U chunks each and round: every load of a round (the weights of U chunks x TN
// tiles, their scales and zero points, and the A fragments) issues before the first is used.
// Each lane unpacks its 16 weight bytes in registers into exact f16 (q - zero) * scale and feeds
// v_mfma_f32_16x16x32_f16 with the weights as the first operand, so a lane ends with 4
// consecutive columns of one row of Y; the wavefronts' partial sums add through LDS and the lanes
// of rows below M store 8 bytes each.
//
// A fragments: lane (g, r) needs A[r][chunk*CW + g*GW + 8i ..] for step i. With ALDS false each
// lane loads its own four 16-byte pieces (16 rows x 4 scattered pieces per instruction, cheap
// while few rows are real). With ALDS true (M > 4) a wavefront loads its chunk's rows as whole
// 256-byte rows (4 rows per instruction, contiguous) straight into its own LDS area
// (buffer_load ... lds, XOR-swizzled by row, frag_swizzle), waits for them and reads the fragments
// back (no barrier: the area is the wavefront's own). At M = 16 that takes a 1024 -> 3072 launch
// from 3.63 to 3.25 us (through registers and ds_write) and 3.10 us (by DMA); at M <= 4 it costs
// 0.03-0.16 us.
//
// A reads stop at K (a multiple of 8): values past K in a row of A (the next row, or padding
// when lda > K) read as zeros, since the weights' padding past K is not zero.
//
// The arguments the first loads need come first (12 dwords): the library compiles this kernel
// with its leading arguments preloaded into SGPRs at wave launch, so a wavefront issues its
// weight loads without first waiting for a kernel-argument load. Addressing is 32-bit through
// buffer resources: rows of A past M and tiles past the weight read zeros.
#pragma once

#include "tmh_device.h"

namespace tmh {

// shape = M | nbc << 8 | bsc_shift << 16 | pad << 24: rows of A (1..16), parameter entries per
// row and chunk, log2 of the weights one parameter entry covers, and (nch * CW - K) / 4, the
// values of the last chunks past K. K travels in shape rather than as an argument of its own:
// one more argument made a launch 0.09-0.17 us slower.
// (The body; k_gemv_dec and its stamping build k_gemv_dec_tl below are the kernels.)
template <int BITS, bool HAS_ZP, bool SPLIT, int U, int NW, int TN, bool ALDS, bool TL, bool BIAS = false>
__device__ __forceinline__ void gemv_dec(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N, uint32_t* __restrict__ tl,
    const _Float16* __restrict__ bias = nullptr) {
  const TlStart tl0 = TL ? tl_clock() : TlStart{0u, 0u};
  constexpr int CW = 512 / BITS;   // weights per chunk row
  constexpr int GW = CW / 4;       // weights per lane per chunk
  constexpr int STEPS = GW / 8;    // MFMA steps per chunk
  constexpr int NJ = SPLIT ? STEPS : 1;
  constexpr int RB = CW * 2 / 16;  // 16-byte pieces per A row of a chunk
  // With A staged through LDS, each wavefront's partial sums go to the start of its own A area
  // (it has read its last fragments by then), so both fit in 64 KiB also at 16 wavefronts.
  constexpr int A_WAVE = U * 16 * RB;  // 16-byte pieces of A per wavefront
  constexpr int RED_WAVE = ALDS ? A_WAVE : TN * 64;
  static_assert(!ALDS || TN * 64 <= A_WAVE, "the partial sums must fit a wavefront's A area");
  __shared__ uint4_t a_lds[ALDS ? NW * A_WAVE : 1];
  __shared__ float4_t red_own[NW > 1 && !ALDS ? NW * TN * 64 : 1];
  float4_t* red = ALDS ? reinterpret_cast<float4_t*>(a_lds) : red_own;
  const uint32_t M = shape & 0xFFu, nbc = (shape >> 8) & 0xFFu, bsc_shift = (shape >> 16) & 0xFFu;
  const uint32_t K = nch * CW - (shape >> 24) * 4;
  const int lane = threadIdx.x & 63;
  // Wavefront-uniform through readfirstlane, so chunk offsets go to the loads' scalar offset.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const uint32_t t0 = blockIdx.x * TN;
  const uint32_t n_params = ntiles * nch * nbc * 16;
  const auto q_rsrc = buffer_rsrc(qt, ntiles * nch * 1024);
  const auto s_rsrc = buffer_rsrc(sc, n_params * 2);
  const auto z_rsrc = buffer_rsrc(zp, HAS_ZP ? zp_byte<BITS>(n_params) : 0u);
  const uint32_t zsh = zp_shift<BITS>(r);
  const auto a_rsrc = buffer_rsrc(A, M * lda * 2);
  const uint32_t a_row = static_cast<uint32_t>(r) < M ? static_cast<uint32_t>(r) * lda * 2 : 0x80000000u;
  // The bias of the lane's four output columns (zeros where the four columns do not all lie
  // below N: that case stores one column at a time and reads the bias there), loaded right after
  // the first round's weights: its kernel argument is not preloaded, and loaded ahead of them
  // its fetch held back the weights' loads.
  typedef uint32_t u32x2b_t __attribute__((ext_vector_type(2)));
  u32x2b_t bias_v[TN];
  bool bias_loaded = false;
  auto load_bias = [&]() {
    if constexpr (BIAS) {
      const auto b_rsrc = buffer_rsrc(bias, N * 2);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint32_t n = (t0 + tn) * 16 + 4 * g;
        bias_v[tn] = __builtin_amdgcn_raw_buffer_load_b64(b_rsrc, n + 4 <= N ? n * 2 : 0x80000000u, 0, 0);
      }
      bias_loaded = true;
    }
  };
  float4_t acc[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) acc[tn] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (uint32_t base = wave * U; base < nch; base += NW * U) {
    uint4_t w[U][TN];
    uint32_t sv[U][TN][NJ], zv[U][TN][NJ];
    half8_t af[U][STEPS];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t c = base + u < nch ? base + u : nch - 1;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint32_t t = t0 + tn;  // t >= ntiles reads zeros
        w[u][tn] = __builtin_amdgcn_raw_buffer_load_b128(q_rsrc, (t * nch * 64 + lane) * 16, c * 1024, 0);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t e = ((t * nch + c) * nbc + ((g * GW + 8 * j * (SPLIT ? 1 : 0)) >> bsc_shift)) * 16 + r;
          sv[u][tn][j] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, e * 2, 0, 0);
          if constexpr (HAS_ZP) zv[u][tn][j] = __builtin_amdgcn_raw_buffer_load_b8(z_rsrc, zp_byte<BITS>(e), 0, 0);
        }
      }
      if constexpr (ALDS) {
        // The chunk's rows go global -> LDS by buffer_load ... lds, 16 bytes a lane: instruction j
        // fills rows (64/RB)*j + lane/RB, slot lane%RB, each lane loading the piece that belongs
        // in its slot of the swizzled layout (the swizzle is its own inverse).
        constexpr int RPI = 64 / RB;
        uint4_t* mine = a_lds + wave * A_WAVE + u * 16 * RB;
#pragma unroll
        for (int j = 0; j < 16 / RPI; ++j) {
          const uint32_t row = RPI * j + lane / RB, p = (lane % RB) ^ frag_swizzle<RB>(row);
          const uint32_t k = (base + u) * CW + 8 * p;  // K is a multiple of 8: a piece is in or past K
          const uint32_t off = (base + u < nch && row < M && k < K) ? row * lda * 2 + k * 2 : 0x80000000u;
          lds_dma16(a_rsrc, reinterpret_cast<uint8_t*>(mine + RPI * j * RB), off, 0);
        }
      } else {
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
          const uint32_t k = (base + u) * CW + g * GW + 8 * i;
          const uint32_t off = base + u < nch && k < K ? a_row + k * 2 : 0x80000000u;
          af[u][i] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off, 0, 0));
        }
      }
    }
    if (BIAS && !bias_loaded) load_bias();
    if constexpr (ALDS) {
      // The DMAs have written the chunks' rows once no vector-memory operation is outstanding
      // (the weights, issued first, are needed next anyway); lanes then read pieces that other
      // lanes' loads wrote.
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
      asm volatile("" ::: "memory");
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint4_t* mine = a_lds + wave * A_WAVE + u * 16 * RB;
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
          const uint32_t p = g * (GW / 8) + i;
          af[u][i] = __builtin_bit_cast(half8_t, mine[r * RB + (p ^ frag_swizzle<RB>(r))]);
        }
      }
    }
    // Every chunk of the round is computed, also one past K (its A fragments are zeros, so it
    // adds 0): a branch here would let the compiler sink that chunk's loads behind the first
    // chunk's wait and MFMAs, one memory latency per chunk.
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int i = 0; i < STEPS; ++i) {
        const int j = SPLIT ? i : 0;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const uint32_t zq = HAS_ZP ? 0x6400u + zp_field<BITS>(zv[u][tn][j], zsh) : 0x6400u + (1u << (BITS - 1));
          const half8_t b = unpack_step<BITS>(w[u][tn], i, __builtin_bit_cast(half2_t, zq | (zq << 16)),
                                              __builtin_bit_cast(half2_t, sv[u][tn][j] | (sv[u][tn][j] << 16)));
          acc[tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, af[u][i], acc[tn], 0, 0, 0);
        }
      }
    }
  }
  if (BIAS && !bias_loaded) load_bias();  // a wavefront that had no chunk
  if constexpr (NW > 1) {
    if constexpr (ALDS) {  // the partial sums overwrite A pieces that other lanes read
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) red[wave * RED_WAVE + tn * 64 + lane] = acc[tn];
    __syncthreads();
  }
  if (static_cast<uint32_t>(r) >= M) return;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    if constexpr (NW > 1) {
      if (tn % NW != static_cast<int>(wave)) continue;
      // Every partial sum is read before the first is added (one LDS latency, not NW of them:
      // left alone the compiler reads two at a time into reused registers).
      float4_t part[NW];
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) part[w2] = red[w2 * RED_WAVE + tn * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);
      acc[tn] = part[0];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) acc[tn] += part[w2];
    } else if (wave != 0) {
      continue;
    }
    const uint32_t n = (t0 + tn) * 16 + 4 * g;
    if (n >= N) continue;
    _Float16* dst = Y + r * ldy + n;
    float4_t v = acc[tn];
    if constexpr (BIAS) {
      // Y = (A . W^T rounded to f16) + bias, rounded to f16 (the reference's Nx.add of the f16 dot).
      if (n + 4 <= N) {
        // The whole vector reinterpreted at once: hipcc 7.2 read element 0 of an integer vector
        // for every index under __builtin_bit_cast of one element.
        typedef _Float16 half4b_t __attribute__((ext_vector_type(4)));
        const half4b_t b = __builtin_bit_cast(half4b_t, bias_v[tn]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<float>(static_cast<_Float16>(v[e])) + static_cast<float>(b[e]);
      } else {
        for (uint32_t e = 0; e < 4 && n + e < N; ++e)
          v[e] = static_cast<float>(static_cast<_Float16>(v[e])) + static_cast<float>(bias[n + e]);
      }
    }
    if (n + 4 <= N && (ldy % 4) == 0) {
      const half2_t lo = {static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1])};
      const half2_t hi = {static_cast<_Float16>(v[2]), static_cast<_Float16>(v[3])};
      typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
      const u32x2_t w = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
      // Streaming grids (several tiles per workgroup: outputs of megabytes, as the lm_head's
      // 151936 columns at M = 8) store non-temporally (17.3 -> 17.1 us there); one-tile grids
      // (the decode projections) keep ordinary stores, which there finish sooner (2.66 against
      // 2.79 us per launch).
      if constexpr (TN > 1) __builtin_nontemporal_store(w, reinterpret_cast<u32x2_t*>(dst));
      else *reinterpret_cast<u32x2_t*>(dst) = w;
    } else {
      for (uint32_t e = 0; e < 4 && n + e < N; ++e) dst[e] = static_cast<_Float16>(v[e]);
    }
  }
  if constexpr (TL) tl_stamp(tl, tl0);  // lane 0 (row 0) always gets here
}

template <int BITS, bool HAS_ZP, bool SPLIT, int U, int NW, int TN, bool ALDS>
__global__ __launch_bounds__(64 * NW) void k_gemv_dec(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N) {
  gemv_dec<BITS, HAS_ZP, SPLIT, U, NW, TN, ALDS, false>(qt, sc, zp, A, nch, ntiles, lda, shape, Y, ldy, N, nullptr);
}

// The same GEMV with a bias (an f16 [N] added to the f16 result); a kernel of its own, so the
// kernels without one keep their argument list (one more argument costs every launch).
template <int BITS, bool HAS_ZP, bool SPLIT, int U, int NW, int TN, bool ALDS>
__global__ __launch_bounds__(64 * NW) void k_gemv_dec_bias(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N, const _Float16* __restrict__ bias) {
  gemv_dec<BITS, HAS_ZP, SPLIT, U, NW, TN, ALDS, false, true>(qt, sc, zp, A, nch, ntiles, lda, shape, Y, ldy, N,
                                                              nullptr, bias);
}

template <int BITS, bool HAS_ZP, bool SPLIT, int U, int NW, int TN, bool ALDS>
__global__ __launch_bounds__(64 * NW) void k_gemv_dec_tl(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N, uint32_t* __restrict__ tl) {
  gemv_dec<BITS, HAS_ZP, SPLIT, U, NW, TN, ALDS, true>(qt, sc, zp, A, nch, ntiles, lda, shape, Y, ldy, N, tl);
}

// Piece P of a k-group's A values: the 16 bytes lane P of each row (16 lanes) of the wavefront
// holds, broadcast to the row (DPP row_newbcast).
template <int P>
__device__ __forceinline__ half8_t row_piece(const uint4_t& x) {
  uint4_t b;
#pragma unroll
  for (int d = 0; d < 4; ++d) b[d] = __builtin_amdgcn_update_dpp(0u, x[d], 0x150 + P, 0xF, 0xF, false);
  return __builtin_bit_cast(half8_t, b);
}

// The decode GEMV for one row of A (M = 1), 4- or 8-bit weights whose parameters are constant
// over a lane's GW values (block_size >= GW), f16 A / scales / Y, an optional f16 bias: dot products instead
// of MFMAs, which at one row leave 15 of 16 MFMA columns empty while the per-weight scaling
// costs the same VALU work.
//
// Lane (g, r) takes the GW values of row r in k-group g of each chunk. The f16 pairs 0x6400 | q
// (= 1024 + q; 4 bits: also 0x6400 | q << 4 = 1024 + 16q for the nibbles at bits 4-7 of each
// half) go straight into v_dot2_f32_f16 against the matching pairs of A, with f32 sums De (pairs
// 1024 + q) and Do (pairs 1024 + 16q). Then
//   sum (q - zero) * a = De + Do / 16 - (1024 * Se + 64 * So + zero * (Se + So)),
// Se and So being the sums of the matching A values (shared by all tiles of a chunk), and the
// lane adds scale * that to its row's sum. Every product (q + 1024) * a is exact in f32; the
// result differs from the reference's dot over f16-rounded weights (q - zero) * scale only by
// that rounding and by f32 summation order.
// The four lanes of a row and the wavefronts of the workgroup add through LDS in a fixed order.
// Chunk rounds, launch shapes and buffer addressing are those of k_gemv_dec.
// (The body; k_gemv_dot and its stamping build k_gemv_dot_tl below are the kernels.)
template <int BITS, bool HAS_ZP, int U, int NW, int TN, bool TL, bool BIAS = false>
__device__ __forceinline__ void gemv_dot(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N, uint32_t* __restrict__ tl,
    const _Float16* __restrict__ bias = nullptr) {
  const TlStart tl0 = TL ? tl_clock() : TlStart{0u, 0u};
  static_assert(BITS == 4 || BITS == 8, "4- or 8-bit weights");
  constexpr int CW = 512 / BITS;  // weights per chunk row
  constexpr int GW = CW / 4;      // weights per lane per chunk
  constexpr int NP = GW / 8;      // 16-byte pieces of A per lane per chunk
  constexpr bool DEDUP = TN == 1; // one A load per chunk and row broadcasts (resident grids)
  __shared__ __align__(16) float red[NW * TN * 64];
  (void)ldy;
  const uint32_t nbc = (shape >> 8) & 0xFFu, bsc_shift = (shape >> 16) & 0xFFu;
  const uint32_t K = nch * CW - (shape >> 24) * 4;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const uint32_t t0 = blockIdx.x * TN;
  const uint32_t n_params = ntiles * nch * nbc * 16;
  const auto q_rsrc = buffer_rsrc(qt, ntiles * nch * 1024);
  const auto s_rsrc = buffer_rsrc(sc, n_params * 2);
  const auto z_rsrc = buffer_rsrc(zp, HAS_ZP ? zp_byte<BITS>(n_params) : 0u);
  const uint32_t zsh = zp_shift<BITS>(r);
  const auto a_rsrc = buffer_rsrc(A, K * 2);
  const half2_t one2 = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
  // The bias of the lane's output column (row r of each tile), loaded right after the first
  // round's weights (as in gemv_dec).
  _Float16 bias_v[TN];
  bool bias_loaded = false;
  auto load_bias = [&]() {
    if constexpr (BIAS) {
      const auto b_rsrc = buffer_rsrc(bias, N * 2);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        bias_v[tn] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(
                                                      b_rsrc, ((t0 + tn) * 16 + r) * 2, 0, 0)));
      bias_loaded = true;
    }
  };
  float acc[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) acc[tn] = 0.f;
  for (uint32_t base = wave * U; base < nch; base += NW * U) {
    uint4_t w[U][TN];
    uint32_t sv[U][TN], zv[U][TN];
    uint4_t mine[U][DEDUP ? 1 : NP];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t c = base + u < nch ? base + u : nch - 1;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint32_t t = t0 + tn;  // t >= ntiles reads zeros
        w[u][tn] = __builtin_amdgcn_raw_buffer_load_b128(q_rsrc, (t * nch * 64 + lane) * 16, c * 1024, 0);
        const uint32_t e = ((t * nch + c) * nbc + ((g * GW) >> bsc_shift)) * 16 + r;
        sv[u][tn] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, e * 2, 0, 0);
        if constexpr (HAS_ZP) zv[u][tn] = __builtin_amdgcn_raw_buffer_load_b8(z_rsrc, zp_byte<BITS>(e), 0, 0);
      }
      if constexpr (DEDUP) {
        // The chunk's A values of k-group g are NP 16-byte pieces, the same for the group's 16
        // lanes: lanes (g, r < NP) load piece r, and row broadcasts (a row of the wavefront being
        // one k-group's 16 lanes) hand every lane the NP pieces below. One A load per wavefront
        // and chunk instead of NP: 2.88 against 3.00 us per stamped launch at the Qwen3-0.6B
        // shapes. (Streaming grids, whose A fragments serve several tiles, keep one load per
        // piece: the broadcasts cost more there, 18.6 against 17.5 us on the 151936 x 1024 lm_head.)
        const uint32_t k = (base + u) * CW + g * GW + 8 * r;  // a piece lies wholly in or past K
        mine[u][0] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, base + u < nch && r < NP && k < K ? k * 2 : 0x80000000u, 0, 0);
      } else {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const uint32_t k = (base + u) * CW + g * GW + 8 * p;  // a piece lies wholly in or past K
          mine[u][p] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, base + u < nch && k < K ? k * 2 : 0x80000000u, 0, 0);
        }
      }
    }
    if (BIAS && !bias_loaded) load_bias();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      half8_t av[1][NP];
      if constexpr (DEDUP) {
        av[0][0] = row_piece<0>(mine[u][0]);
        av[0][1] = row_piece<1>(mine[u][0]);
        if constexpr (NP > 2) {
          av[0][2] = row_piece<2>(mine[u][0]);
          av[0][3] = row_piece<3>(mine[u][0]);
        }
      } else {
#pragma unroll
        for (int p = 0; p < NP; ++p) av[0][p] = __builtin_bit_cast(half8_t, mine[u][p]);
      }
      // Sums of this lane's A values, split by the pair form their weights take. (A pieces are
      // held as f16 vectors: pairs are taken by element, since hipcc 7.2 read element 0 of an
      // integer vector for every index under __builtin_bit_cast of one element.)
      float se = 0.f, so = 0.f;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const half2_t ap = {av[0][p][2 * j], av[0][p][2 * j + 1]};
          if (BITS == 4 && (j & 1)) so = __builtin_amdgcn_fdot2(ap, one2, so, false);
          else se = __builtin_amdgcn_fdot2(ap, one2, se, false);
        }
      }
      const float base_sum = BITS == 4 ? fmaf(1024.f, se, 64.f * so) : 1024.f * se;
      const float sa = se + so;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u);
        float de = 0.f, dq = 0.f;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          half2_t ap[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) ap[j] = half2_t{av[0][p][2 * j], av[0][p][2 * j + 1]};
          if constexpr (BITS == 4) {
            // Word p holds values 8p .. 8p+7: pairs (0,1) and (4,5) in low-nibble form, (2,3) and
            // (6,7) in high-nibble form, against A pairs 0, 2 and 1, 3 of piece p.
            const uint32_t x = w[u][tn][p];
            de = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, and_or(x, 0x000F000Fu, magic)), ap[0], de, false);
            dq = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, and_or(x, 0x00F000F0u, magic)), ap[1], dq, false);
            de = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, and_or(x >> 8, 0x000F000Fu, magic)), ap[2], de, false);
            dq = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, and_or(x >> 8, 0x00F000F0u, magic)), ap[3], dq, false);
          } else {
            // Words 2p, 2p+1 hold values 8p .. 8p+7 in byte order.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const uint32_t x = w[u][tn][2 * p + h];
              const uint32_t lo = (x & 0xFFu) | ((x << 8) & 0x00FF0000u) | 0x64006400u;
              const uint32_t hi = ((x >> 16) & 0xFFu) | ((x >> 8) & 0x00FF0000u) | 0x64006400u;
              de = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, lo), ap[2 * h], de, false);
              de = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, hi), ap[2 * h + 1], de, false);
            }
          }
        }
        const float z = HAS_ZP ? static_cast<float>(zp_field<BITS>(zv[u][tn], zsh)) : static_cast<float>(1 << (BITS - 1));
        const float s = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(sv[u][tn])));
        const float dot = BITS == 4 ? fmaf(dq, 0.0625f, de) : de;
        acc[tn] = fmaf(s, dot - fmaf(z, sa, base_sum), acc[tn]);
      }
    }
  }
  if (BIAS && !bias_loaded) load_bias();  // a wavefront that had no chunk
  // Row r's four lane sums of a wavefront sit together (one 16-byte read each).
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) red[(wave * TN + tn) * 64 + r * 4 + g] = acc[tn];
  __syncthreads();
  // Tile tn's 16 sums are added by lanes 0-15 of wavefront tn % NW, each over its row's four
  // lanes in every wavefront, in a fixed order; all the partial sums are read before the first
  // is added.
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    if (tn % NW != static_cast<int>(wave) || g != 0) continue;
    float4_t part[NW];
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) part[w2] = reinterpret_cast<const float4_t*>(red)[(w2 * TN + tn) * 16 + r];
    __builtin_amdgcn_sched_barrier(0);
    float v = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2)
#pragma unroll
      for (int g2 = 0; g2 < 4; ++g2) v += part[w2][g2];
    const uint32_t n = (t0 + tn) * 16 + r;
    // With a bias: the f16 dot plus the bias, rounded to f16 (the reference's Nx.add).
    if constexpr (BIAS) v = static_cast<float>(static_cast<_Float16>(v)) + static_cast<float>(bias_v[tn]);
    if (n < N) Y[n] = static_cast<_Float16>(v);
  }
  if constexpr (TL) tl_stamp(tl, tl0);
}

template <int BITS, bool HAS_ZP, int U, int NW, int TN>
__global__ __launch_bounds__(64 * NW) void k_gemv_dot(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N) {
  gemv_dot<BITS, HAS_ZP, U, NW, TN, false>(qt, sc, zp, A, nch, ntiles, lda, shape, Y, ldy, N, nullptr);
}

// The same with a bias (f16 [N]), as k_gemv_dec_bias.
template <int BITS, bool HAS_ZP, int U, int NW, int TN>
__global__ __launch_bounds__(64 * NW) void k_gemv_dot_bias(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N, const _Float16* __restrict__ bias) {
  gemv_dot<BITS, HAS_ZP, U, NW, TN, false, true>(qt, sc, zp, A, nch, ntiles, lda, shape, Y, ldy, N, nullptr, bias);
}

template <int BITS, bool HAS_ZP, int U, int NW, int TN>
__global__ __launch_bounds__(64 * NW) void k_gemv_dot_tl(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const _Float16* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    _Float16* __restrict__ Y, uint32_t ldy, uint32_t N, uint32_t* __restrict__ tl) {
  gemv_dot<BITS, HAS_ZP, U, NW, TN, true>(qt, sc, zp, A, nch, ntiles, lda, shape, Y, ldy, N, tl);
}

// The same GEMV over f32 A and f32 weights (the reference's CPU configuration after move/2: f32
// scales, so W = (q - zero) * scale in f32, one rounding) for M <= MM rows, f32 Y, no bias.
// Lane (g, r) dequantizes its 16 bytes (row r, GW consecutive k) to f32 and accumulates
// A[m][k] * W[r][k] with f32 FMAs; the four lanes of a row add by shuffles, the wavefronts of
// the workgroup through LDS, in a fixed order.
template <int BITS, bool HAS_ZP, bool SPLIT, int NW, int MM>
__global__ __launch_bounds__(64 * NW) void k_gemv_f32(
    const uint4_t* __restrict__ qt, const float* __restrict__ sc, const uint8_t* __restrict__ zp,
    const float* __restrict__ A, uint32_t nch, uint32_t ntiles, uint32_t lda, uint32_t shape,
    float* __restrict__ Y, uint32_t ldy, uint32_t N) {
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int STEPS = GW / 8;
  constexpr int NJ = SPLIT ? STEPS : 1;
  __shared__ float red[NW][MM][16];
  const uint32_t M = shape & 0xFFu, nbc = (shape >> 8) & 0xFFu, bsc_shift = (shape >> 16) & 0xFFu;
  const uint32_t K = nch * CW - (shape >> 24) * 4;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const uint32_t t = blockIdx.x;
  const uint32_t n_params = ntiles * nch * nbc * 16;
  const auto q_rsrc = buffer_rsrc(qt, ntiles * nch * 1024);
  const auto s_rsrc = buffer_rsrc(sc, n_params * 4);
  const auto z_rsrc = buffer_rsrc(zp, HAS_ZP ? zp_byte<BITS>(n_params) : 0u);
  const uint32_t zsh = zp_shift<BITS>(r);
  const auto a_rsrc = buffer_rsrc(A, M * lda * 4);
  float acc[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.f;
  for (uint32_t c = wave; c < nch; c += NW) {
    const uint4_t w = __builtin_amdgcn_raw_buffer_load_b128(q_rsrc, (t * nch * 64 + lane) * 16, c * 1024, 0);
    float sv[NJ], zv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t e = ((t * nch + c) * nbc + ((g * GW + 8 * j * (SPLIT ? 1 : 0)) >> bsc_shift)) * 16 + r;
      sv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, e * 4, 0, 0));
      zv[j] = HAS_ZP ? static_cast<float>(zp_field<BITS>(__builtin_amdgcn_raw_buffer_load_b8(z_rsrc, zp_byte<BITS>(e), 0, 0), zsh))
                     : static_cast<float>(1 << (BITS - 1));
    }
    // A[m][k0 .. k0 + GW) as 16-byte pieces (zeros past M or K), held as floats: with hipcc 7.2
    // a __builtin_bit_cast of one element of an integer vector read element 0 for every index.
    float4_t av[MM][GW / 4];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int i = 0; i < GW / 4; ++i) {
        const uint32_t k = c * CW + g * GW + 4 * i;
        const uint32_t off = static_cast<uint32_t>(m) < M && k < K ? m * lda * 4 + k * 4 : 0x80000000u;
        av[m][i] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off, 0, 0));
      }
    constexpr int PER_WORD = 32 / BITS;
#pragma unroll
    for (int e = 0; e < GW; ++e) {
      const int j = SPLIT ? e / 8 : 0;
      const float q = static_cast<float>(word_value<BITS>(w[e / PER_WORD], e % PER_WORD));
      const float wv = (q - zv[j]) * sv[j];
#pragma unroll
      for (int m = 0; m < MM; ++m) acc[m] = fmaf(av[m][e / 4][e % 4], wv, acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    acc[m] += __shfl_xor(acc[m], 16);
    acc[m] += __shfl_xor(acc[m], 32);
    if (g == 0) red[wave][m][r] = acc[m];
  }
  __syncthreads();
  if (wave != 0 || g != 0) return;
  const uint32_t n = t * 16 + r;
  if (n >= N) return;
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    if (static_cast<uint32_t>(m) >= M) break;
    float v = red[0][m][r];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) v += red[w2][m][r];
    Y[m * ldy + n] = v;
  }
}

}  // namespace tmh
