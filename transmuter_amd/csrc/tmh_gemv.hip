// Launch plan of the decode GEMVs (k_gemv_dot for one row of A, k_gemv_dec, tmh_gemv.h):
// MatMulNBits with M <= 16 rows of f16 A, f16 weights, f16 Y, no bias or an f16 one
// (lib/transmuter/ops/quantized.ex:30-46 after move/2).
//
// This file is compiled with the kernels' leading arguments preloaded into SGPRs
// (-mllvm -amdgpu-kernarg-preload-count): at the Qwen3-0.6B projection shapes that takes a
// launch from 3.16 to 2.78 us, and a plain read of the same bytes from 1.99 to 1.82 us.
//
// Two regimes, measured on MI355X inside HIP graphs:
//  - one-shot (the whole grid resident at once: the Qwen3-0.6B projections): one chunk per
//    wavefront and round (U = 1), as many wavefronts as chunks (NW = nch, up to 16), one tile
//    per workgroup. Latency-bound: more chunks per wavefront or more tiles per workgroup were
//    0.07-0.4 us slower per launch. A is staged through LDS for M > 4. Ablations of the MFMA
//    kernel at M = 1 (2.66 us per launch): without the final store 2.40, without the
//    cross-wavefront sum 2.47, without the unpack and MFMAs 2.41; an empty kernel costs 1.57 and
//    a plain read of the weights 1.82. One row of A goes to k_gemv_dot in the same shape (2.64).
//  - the same grids over 1.1 GB of weight copies (twelve lm_head copies) read HBM at 5.5-5.8
//    TB/s in a plain read; k_gemv_dot at M = 1 takes 17.3-18.7 us there (5.0-5.2 TB/s), this
//    kernel at M = 8 19.7-20.4 us. The figures below are over three copies.
//  - streaming (lm_head-sized N): U = 2 chunks per wavefront loaded together, NW = nch / 2
//    wavefronts, four tiles per workgroup, so every A fragment serves four tiles (two tiles for
//    one row of A, through k_gemv_dot). On 151936 x 1024 with random weights rotating over three
//    copies (270 MB, more than the last-level cache): 17.0-17.4 us at M = 8 (5.3-5.4 TB/s) and
//    15.7-16.2 us at M = 1 with k_gemv_dot (5.6-5.7 TB/s); a plain read of the same bytes takes
//    14.2 us (6.5 TB/s). U = 1 with two rounds was 17.5-19.4 us. Persistent wavefronts that
//    double-buffer whole tiles, one wavefront walking all of K for a group of tiles with loads
//    three chunks ahead (19.5-23 us), A staged whole in LDS per workgroup (24-28 us), scales
//    staged through LDS with wide loads, and non-temporal weight loads were no faster.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "tmh_gemv.h"
#include "tmh_internal.h"

namespace tmh {
namespace {

constexpr size_t kStaticLds = 64 * 1024;

struct DecArgs {
  const uint4_t* qt;
  const uint16_t* sc;
  const uint8_t* zp;
  const _Float16* a;
  uint32_t nch, ntiles, lda, shape;
  _Float16* y;
  uint32_t ldy, n;
  const _Float16* bias = nullptr;  // f16 [N] added to Y, or none
};

template <int BITS, bool HAS_ZP, bool SPLIT, int NW, int TN, bool ALDS, int U = 1>
void go(const DecArgs& d, hipStream_t s) {
  // The LDS-staged A needs U * 16 rows of a chunk per wavefront (the partial sums reuse that
  // space); shapes where that exceeds the static LDS of a workgroup load A directly.
  constexpr size_t rb = (512 / BITS) * 2 / 16;
  constexpr size_t red = NW > 1 ? static_cast<size_t>(NW) * TN * 64 * 16 : 0;
  constexpr bool A_LDS = ALDS && static_cast<size_t>(NW) * U * 16 * rb * 16 <= kStaticLds;
  static_assert(red <= kStaticLds, "partial sums exceed the static LDS");
  const unsigned grid = (d.ntiles + TN - 1) / TN;
  if (d.bias) {  // (the bias build has no stamping build: its launches are not on the timeline)
    k_gemv_dec_bias<BITS, HAS_ZP, SPLIT, U, NW, TN, A_LDS><<<grid, 64 * NW, 0, s>>>(
        d.qt, d.sc, d.zp, d.a, d.nch, d.ntiles, d.lda, d.shape, d.y, d.ldy, d.n, d.bias);
    return;
  }
  if (uint32_t* tl = timeline_slots(TMH_TL_GEMV_DEC, static_cast<int64_t>(grid) * NW)) {
    k_gemv_dec_tl<BITS, HAS_ZP, SPLIT, U, NW, TN, A_LDS><<<grid, 64 * NW, 0, s>>>(
        d.qt, d.sc, d.zp, d.a, d.nch, d.ntiles, d.lda, d.shape, d.y, d.ldy, d.n, tl);
    return;
  }
  k_gemv_dec<BITS, HAS_ZP, SPLIT, U, NW, TN, A_LDS><<<grid, 64 * NW, 0, s>>>(d.qt, d.sc, d.zp, d.a, d.nch, d.ntiles,
                                                                              d.lda, d.shape, d.y, d.ldy, d.n);
}

// Wavefront counts the one-shot kernels are built for: the chunk count rounded up to one of
// them (the extra wavefronts find no chunk and add zeros).
int round_waves(int64_t w) {
  for (int c : {1, 2, 4, 8, 12}) if (w <= c) return c;
  return 16;
}

template <int BITS, bool HAS_ZP, bool SPLIT, bool ALDS>
void one_shot(const DecArgs& d, int nw, hipStream_t s) {
  switch (nw) {
    case 1: go<BITS, HAS_ZP, SPLIT, 1, 1, ALDS>(d, s); break;
    case 2: go<BITS, HAS_ZP, SPLIT, 2, 1, ALDS>(d, s); break;
    case 4: go<BITS, HAS_ZP, SPLIT, 4, 1, ALDS>(d, s); break;
    case 8: go<BITS, HAS_ZP, SPLIT, 8, 1, ALDS>(d, s); break;
    case 12: go<BITS, HAS_ZP, SPLIT, 12, 1, ALDS>(d, s); break;
    default: go<BITS, HAS_ZP, SPLIT, 16, 1, ALDS>(d, s);
  }
}

template <int BITS, bool HAS_ZP, bool SPLIT>
void streaming(const DecArgs& d, int nw, hipStream_t s) {
  switch (nw) {
    case 1: go<BITS, HAS_ZP, SPLIT, 1, 4, false, 2>(d, s); break;
    case 2: go<BITS, HAS_ZP, SPLIT, 2, 4, false, 2>(d, s); break;
    case 4: go<BITS, HAS_ZP, SPLIT, 4, 4, false, 2>(d, s); break;
    default: go<BITS, HAS_ZP, SPLIT, 8, 4, false, 2>(d, s);
  }
}

template <int BITS, bool HAS_ZP, int NW, int TN, int U>
void go_dot(const DecArgs& d, hipStream_t s) {
  const unsigned grid = (d.ntiles + TN - 1) / TN;
  if (d.bias) {
    k_gemv_dot_bias<BITS, HAS_ZP, U, NW, TN><<<grid, 64 * NW, 0, s>>>(d.qt, d.sc, d.zp, d.a, d.nch, d.ntiles, d.lda,
                                                                       d.shape, d.y, d.ldy, d.n, d.bias);
    return;
  }
  if (uint32_t* tl = timeline_slots(TMH_TL_GEMV_DOT, static_cast<int64_t>(grid) * NW)) {
    k_gemv_dot_tl<BITS, HAS_ZP, U, NW, TN><<<grid, 64 * NW, 0, s>>>(d.qt, d.sc, d.zp, d.a, d.nch, d.ntiles, d.lda,
                                                                     d.shape, d.y, d.ldy, d.n, tl);
    return;
  }
  k_gemv_dot<BITS, HAS_ZP, U, NW, TN><<<grid, 64 * NW, 0, s>>>(d.qt, d.sc, d.zp, d.a, d.nch, d.ntiles, d.lda, d.shape,
                                                                d.y, d.ldy, d.n);
}

// Which kernel serves one row of A: the dot-product kernel unless TMH_GEMV_PLAN=mfma in the
// environment forces the MFMA kernel (how the tests reach both at M = 1; read at each call).
bool dot_for_one_row() {
  const char* v = std::getenv("TMH_GEMV_PLAN");
  return !(v && std::strcmp(v, "mfma") == 0);
}

template <int BITS, bool HAS_ZP, bool SPLIT>
void launch_bits(const DecArgs& d, int64_t M, int num_cus, hipStream_t s) {
  const int64_t nch = d.nch;
  // Wavefronts of the one-shot shape per CU up to which a grid counts as resident: 24, or 16 for
  // one row of A (the merged Qwen3-0.6B gate/up projection, 384 tiles x 8 chunks, runs the
  // one-shot shape with its one A load per chunk: merged launches 2.85 against 2.87 us on average
  // with the streaming shape; at M = 8 and 16 the one-shot shape is faster there too, 3.37
  // against 3.52 us).
  const int64_t resident = static_cast<int64_t>(num_cus > 0 ? num_cus : 256) * (M == 1 ? 16 : 24);
  const bool resident_grid = static_cast<int64_t>(d.ntiles) * std::min<int64_t>(nch, 16) <= resident;
  if constexpr (BITS != 2 && !SPLIT) {
    // One row of A: the dot-product kernel. Over a streaming grid two chunks per wavefront load
    // together, and four tiles share a workgroup where the grid spans thousands of tiles (151936 x
    // 1024 q4 over 1.1 GB of rotating copies: 17.5 against 18.2-18.5 us with two tiles; one chunk
    // per wavefront 18.5-19.3, four 19.0-22.6), two below that; where the whole grid is resident,
    // one chunk per wavefront and one tile per workgroup, as the MFMA kernel's one-shot shape
    // (Qwen3-0.6B projections: 2.64 against 2.67 us per launch, merged 3.04 against 3.06; the
    // streaming shape there: 2.97).
    if (M == 1 && !resident_grid && dot_for_one_row()) {
      const bool wide = d.ntiles >= 2048;
      switch (std::min(8, round_waves((nch + 1) / 2))) {
        case 1: wide ? go_dot<BITS, HAS_ZP, 1, 4, 2>(d, s) : go_dot<BITS, HAS_ZP, 1, 2, 2>(d, s); break;
        case 2: wide ? go_dot<BITS, HAS_ZP, 2, 4, 2>(d, s) : go_dot<BITS, HAS_ZP, 2, 2, 2>(d, s); break;
        case 4: wide ? go_dot<BITS, HAS_ZP, 4, 4, 2>(d, s) : go_dot<BITS, HAS_ZP, 4, 2, 2>(d, s); break;
        default: wide ? go_dot<BITS, HAS_ZP, 8, 4, 2>(d, s) : go_dot<BITS, HAS_ZP, 8, 2, 2>(d, s);
      }
      return;
    }
    if (M == 1 && dot_for_one_row() && nch > 16) {
      // More chunks than 16 wavefronts take in one round (3072 -> 1024: 24): two chunks per
      // wavefront, loaded together, instead of a second round behind the first round's compute
      // (stamped in-kernel span 2.43 against 2.58 us per launch).
      switch (std::min(16, round_waves((nch + 1) / 2))) {
        case 12: go_dot<BITS, HAS_ZP, 12, 1, 2>(d, s); break;
        default: go_dot<BITS, HAS_ZP, 16, 1, 2>(d, s);
      }
      return;
    }
    if (M == 1 && dot_for_one_row()) {
      switch (round_waves(nch)) {
        case 1: go_dot<BITS, HAS_ZP, 1, 1, 1>(d, s); break;
        case 2: go_dot<BITS, HAS_ZP, 2, 1, 1>(d, s); break;
        case 4: go_dot<BITS, HAS_ZP, 4, 1, 1>(d, s); break;
        case 8: go_dot<BITS, HAS_ZP, 8, 1, 1>(d, s); break;
        case 12: go_dot<BITS, HAS_ZP, 12, 1, 1>(d, s); break;
        default: go_dot<BITS, HAS_ZP, 16, 1, 1>(d, s);
      }
      return;
    }
  }
  if (resident_grid) {
    const int nw = round_waves(nch);
    if (M > 4)
      one_shot<BITS, HAS_ZP, SPLIT, true>(d, nw, s);
    else
      one_shot<BITS, HAS_ZP, SPLIT, false>(d, nw, s);
    return;
  }
  // Streaming: two chunks per wavefront loaded together (at most 8 wavefronts, more rounds for
  // larger K), four tiles per workgroup.
  streaming<BITS, HAS_ZP, SPLIT>(d, std::min(8, round_waves((nch + 1) / 2)), s);
}

// One row of A (the reference's single-op case) takes the one-row build: the four-row build
// would load and multiply three rows of zeros (C1, 1024 -> 3072 f32).
template <int BITS, bool HAS_ZP, bool SPLIT, int NW>
void go_f32(const DecArgs& d, const float* a, float* y, hipStream_t s) {
  if ((d.shape & 0xFFu) == 1)
    k_gemv_f32<BITS, HAS_ZP, SPLIT, NW, 1><<<d.ntiles, 64 * NW, 0, s>>>(
        d.qt, reinterpret_cast<const float*>(d.sc), d.zp, a, d.nch, d.ntiles, d.lda, d.shape, y, d.ldy, d.n);
  else
    k_gemv_f32<BITS, HAS_ZP, SPLIT, NW, 4><<<d.ntiles, 64 * NW, 0, s>>>(
        d.qt, reinterpret_cast<const float*>(d.sc), d.zp, a, d.nch, d.ntiles, d.lda, d.shape, y, d.ldy, d.n);
}

template <int BITS, bool HAS_ZP, bool SPLIT>
void launch_f32_bits(const DecArgs& d, const float* a, float* y, hipStream_t s) {
  switch (round_waves(d.nch)) {
    case 1: go_f32<BITS, HAS_ZP, SPLIT, 1>(d, a, y, s); break;
    case 2: go_f32<BITS, HAS_ZP, SPLIT, 2>(d, a, y, s); break;
    case 4: go_f32<BITS, HAS_ZP, SPLIT, 4>(d, a, y, s); break;
    case 8: go_f32<BITS, HAS_ZP, SPLIT, 8>(d, a, y, s); break;
    case 12: go_f32<BITS, HAS_ZP, SPLIT, 12>(d, a, y, s); break;
    default: go_f32<BITS, HAS_ZP, SPLIT, 16>(d, a, y, s);
  }
}

// (nch * CW - K) / 4: the values of the last chunks past K, in fours (K is a multiple of 4).
int64_t pad_quads(const tmh_weight* w) { return (w->nchunks * chunk_weights(w->bits) - w->K) / 4; }

DecArgs dec_args(const tmh_weight* w, const void* a, int64_t M, int64_t lda, void* y, int64_t ldy) {
  const int cw = chunk_weights(w->bits);
  const int bsc = std::min(w->block_size, cw);
  int shift = 0;
  while ((1 << shift) < bsc) ++shift;
  return DecArgs{reinterpret_cast<const uint4_t*>(w->d_q), static_cast<const uint16_t*>(w->d_scale),
                 static_cast<const uint8_t*>(w->d_zero), static_cast<const _Float16*>(a),
                 static_cast<uint32_t>(w->nchunks), static_cast<uint32_t>(w->ntiles), static_cast<uint32_t>(lda),
                 static_cast<uint32_t>(M) | (static_cast<uint32_t>(w->nbc) << 8) | (static_cast<uint32_t>(shift) << 16) |
                     (static_cast<uint32_t>(pad_quads(w)) << 24),
                 static_cast<_Float16*>(y), static_cast<uint32_t>(ldy), static_cast<uint32_t>(w->N)};
}

}  // namespace

bool decode_gemv_f32_ok(const tmh_weight* w, int64_t M, int64_t lda, int64_t ldy, const void* a) {
  return M >= 1 && M <= 4 && reinterpret_cast<uintptr_t>(a) % 16 == 0 && lda % 4 == 0 && w->K % 4 == 0 &&
         M * lda * 4 < (int64_t(1) << 31) && w->ntiles * w->nchunks * 1024 < (int64_t(1) << 31) &&
         w->ntiles * w->nchunks * w->nbc * 16 * 4 < (int64_t(1) << 31) && ldy < (int64_t(1) << 30) &&
         w->wdtype == TMH_F32 && w->zp_kind != TMH_ZP_FLOAT && w->ntiles < (int64_t(1) << 31) && pad_quads(w) < 256;
}

void launch_decode_gemv_f32(const tmh_weight* w, const void* a, int64_t M, int64_t lda, void* y, int64_t ldy,
                            hipStream_t s) {
  const DecArgs d = dec_args(w, a, M, lda, y, ldy);
  const bool zp = w->zp_kind == TMH_ZP_PACKED;
  const bool split = w->block_size < chunk_weights(w->bits) / 4;
  const auto* af = static_cast<const float*>(a);
  auto* yf = static_cast<float*>(y);
#define TMH_DEC32(B)                                                    \
  if (zp && split) launch_f32_bits<B, true, true>(d, af, yf, s);        \
  else if (zp) launch_f32_bits<B, true, false>(d, af, yf, s);           \
  else if (split) launch_f32_bits<B, false, true>(d, af, yf, s);        \
  else launch_f32_bits<B, false, false>(d, af, yf, s);
  switch (w->bits) {
    case 2: { TMH_DEC32(2) } break;
    case 4: { TMH_DEC32(4) } break;
    default: { TMH_DEC32(8) }
  }
#undef TMH_DEC32
}

bool decode_gemv_ok(const tmh_weight* w, int64_t M, int64_t lda, int64_t ldy, const void* a, const void* y) {
  return M >= 1 && M <= 16 && reinterpret_cast<uintptr_t>(a) % 16 == 0 && lda % 8 == 0 && w->K % 8 == 0 &&
         M * lda * 2 < (int64_t(1) << 31) && w->ntiles * w->nchunks * 1024 < (int64_t(1) << 31) &&
         w->ntiles * w->nchunks * w->nbc * 16 * 2 < (int64_t(1) << 31) && ldy < (int64_t(1) << 30) &&
         (reinterpret_cast<uintptr_t>(y) & 7) == 0 && w->wdtype == TMH_F16 && w->zp_kind != TMH_ZP_FLOAT &&
         pad_quads(w) < 256;
}

void launch_decode_gemv(const tmh_weight* w, const void* a, int64_t M, int64_t lda, void* y, int64_t ldy,
                        hipStream_t s, int num_cus, const void* bias) {
  const int cw = chunk_weights(w->bits);
  DecArgs d = dec_args(w, a, M, lda, y, ldy);
  d.bias = static_cast<const _Float16*>(bias);
  const bool zp = w->zp_kind == TMH_ZP_PACKED;
  const bool split = w->block_size < cw / 4;  // a lane's k-group spans several blocks
#define TMH_DEC(B)                                                   \
  if (zp && split) launch_bits<B, true, true>(d, M, num_cus, s);      \
  else if (zp) launch_bits<B, true, false>(d, M, num_cus, s);         \
  else if (split) launch_bits<B, false, true>(d, M, num_cus, s);      \
  else launch_bits<B, false, false>(d, M, num_cus, s);
  switch (w->bits) {
    case 2: { TMH_DEC(2) } break;
    case 4: { TMH_DEC(4) } break;
    default: { TMH_DEC(8) }
  }
#undef TMH_DEC
}

}  // namespace tmh
