// QMoE (com.microsoft) on gfx950: routing, grouping by expert, grouped expert GEMMs over
// packed weights, activation and the weighted sum over each token's experts.
//
// Reference (georgeguimaraes/transmuter):
//   lib/transmuter/ops/moe.ex:42-61    QMoE: top-k router values, a softmax over those k values,
//                                      experts dequantized as (q - zero) * scale
//   lib/transmuter/ops/moe.ex:64-102   experts/4: fc1 (and fc3), activation, fc2, bias of the
//                                      row's expert, weighted sum over the slots (weight 0 adds 0)
//   lib/transmuter/ops/moe.ex:108-138  route/3: the routed rows; the dense variant (every expert
//                                      on every token, weight 0 for the unselected) sums the same
//   lib/transmuter/ops/moe.ex:158-165  topk/2: a stable descending sort (lower index first)
//   lib/transmuter/ops/moe.ex:176-206  activate/2 and swiglu_gate/3
//   lib/transmuter/ops/moe.ex:216-253  dequant/6: block-wise or per-row scales and zero points
//
// Layout on the device: the experts of one weight are one tmh_weight of E*N rows (expert e owns
// rows e*N.. and 16-row tiles e*N/16..). A call sorts its T*k (token, slot) rows by expert, runs
// each expert's rows against its tiles in work items of up to 32 or 64 rows, and keeps the
// intermediates in expert order; the last product writes its rows back in (token, slot) order
// (expert order on the general path), and the final sum reads them per token, slot by slot.
#include <algorithm>
#include <cmath>
#include <type_traits>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "tmh_device.h"
#include "tmh_internal.h"

using namespace tmh;

namespace {

constexpr int kMoeRows = 32;  // rows per work item of the general product

// ------------------------------------------------------------------ routing and grouping

// Order key of a router value: larger values give larger keys and equal values equal keys, with
// -0 taken as +0 and NaN as -inf, as the float comparisons of the sort see them.
__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) x = -INFINITY;
  if (x == 0.f) x = 0.f;
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t key) {
  return __builtin_bit_cast(float, (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

// The largest of the wavefront's 64 values, in every lane: a running maximum over rows of 16
// lanes (row_shr 1, 2, 4, 8), across rows (row_bcast 15 and 31), read from lane 63. A lane with no
// source lane keeps its own value.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto step = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  const int x = static_cast<int>(v);
  v = step(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(x, x, 0x111, 0xf, 0xf, false)));
  v = step(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x112, 0xf, 0xf, false)));
  v = step(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x114, 0xf, 0xf, false)));
  v = step(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x118, 0xf, 0xf, false)));
  v = step(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x142, 0xa, 0xf, false)));
  v = step(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x143, 0xc, 0xf, false)));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// One wavefront per token: the k largest router values (lower index first among equals), a
// softmax over them in f32. Lane l holds the order keys of experts l, l + 64, ... (EJ of them;
// key 0, below every expert's key, past E). Round r takes the largest key left (a wavefront
// maximum), the lowest expert index that holds it (the first 64-expert group whose ballot is not
// empty, then its lowest lane), and sets that key to 0; lane r keeps the round's value and index.
// (The body; k_moe_route and its stamping build k_moe_route_tl below are the kernels.)
template <int RDT, int EJ>
__device__ __forceinline__ void moe_route(const void* __restrict__ router, int T, int E, int k,
                                          int* __restrict__ topi, float* __restrict__ topw) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  uint32_t key[EJ];
#pragma unroll
  for (int j = 0; j < EJ; ++j) {
    const int e = lane + 64 * j;
    key[j] = e < E ? order_key(load_as_f32<RDT>(router, static_cast<int64_t>(t) * E + e)) : 0u;
  }
  float sel_v = 0.f;
  int sel_i = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t best = key[0];
#pragma unroll
    for (int j = 1; j < EJ; ++j) best = key[j] > best ? key[j] : best;
    const uint32_t m = wave_max_u32(best);
    int e = 0;
    bool found = false;
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      const uint64_t b = __ballot(key[j] == m);
      if (!found && b) {
        e = 64 * j + __builtin_ctzll(b);
        found = true;
      }
    }
    e = e < E ? e : E - 1;  // (m is a key of an expert, so e < E already)
#pragma unroll
    for (int j = 0; j < EJ; ++j)
      if (e == lane + 64 * j) key[j] = 0u;
    if (lane == r) {
      sel_v = key_value(m);
      sel_i = e;
    }
  }
  const float mx = __shfl(sel_v, 0);
  const float ex = lane < k ? expf(sel_v - mx) : 0.f;
  float sum = ex;
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (lane < k) {
    topi[t * k + lane] = sel_i;
    topw[t * k + lane] = ex / sum;
  }
}

// Inclusive prefix sum over the wavefront's 64 lanes: within rows of 16 (row_shr 1, 2, 4, 8),
// then across rows (row_bcast 15 into rows 1 and 3, row_bcast 31 into rows 2 and 3). A lane with
// no source lane adds 0.
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
  return v;
}

// One workgroup of 1024 threads (thread e for expert e): rows per expert, expert offsets (exclusive
// prefix of the counts), the list of work items (expert << 16 | item of the expert, `rows` rows
// each; the items with the most 16-row m-tiles first), and the position of every (token, slot)
// row in expert order (perm) with its inverse
// (slot_pos). Each thread loads four rows' experts per round before its LDS atomics; up to 4096
// rows the ids stay in registers from the count to the placement. The prefix sums run per
// wavefront in DPP steps, then across the 16 wavefronts.
// (The body; k_moe_plan and k_moe_plan_tl below are the kernels.)
__device__ __forceinline__ void moe_plan(int* __restrict__ counts, int E, int rows, const int* __restrict__ topi,
                                         int Tk, int* __restrict__ offsets, int* __restrict__ items,
                                         int* __restrict__ n_items, int* __restrict__ perm,
                                         int* __restrict__ slot_pos) {
  constexpr int R = 4;
  __shared__ int first_s[1024], fill[1024], wsum_r[16], wsum_i[16], cls_next[5];
  const int e = threadIdx.x, lane = e & 63, wave = e >> 6;
  fill[e] = 0;
  if (e < 5) cls_next[e] = 0;
  __syncthreads();
  int ex[R];
  for (int base = 0; base < Tk; base += 1024 * R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int idx = base + u * 1024 + e;
      ex[u] = idx < Tk ? topi[idx] : -1;
    }
#pragma unroll
    for (int u = 0; u < R; ++u)
      if (ex[u] >= 0) atomicAdd(&fill[ex[u]], 1);
  }
  __syncthreads();
  const int c = fill[e];
  const int nb = (c + rows - 1) / rows;
  if (e < E) counts[e] = c;
  // Work items in descending order of their 16-row m-tiles (the heaviest first: the products'
  // workgroups run in item order, so the last ones to start are light). An expert's items are
  // full but its last (q_last m-tiles); the order within a class is the atomics' (any order
  // computes the same outputs).
  const int q_full = rows / 16, q_last = nb > 0 ? (c - (nb - 1) * rows + 15) / 16 : 0;
  if (e < E && nb > 0) {
    if (nb > 1) atomicAdd(&cls_next[q_full], nb - 1);
    atomicAdd(&cls_next[q_last], 1);
  }
  int sr = wave_inclusive_sum(c), si = wave_inclusive_sum(nb);  // inclusive prefix sums of rows and items
  if (lane == 63) {
    wsum_r[wave] = sr;
    wsum_i[wave] = si;
  }
  __syncthreads();
  for (int w2 = 0; w2 < wave; ++w2) {
    sr += wsum_r[w2];
    si += wsum_i[w2];
  }
  const int first_row = sr - c;
  if (e < E) offsets[e] = first_row;
  if (e == 1023) *n_items = si;
  if (e == 0) {  // each class's first item position, the classes in descending order
    int run = 0;
    for (int q = 4; q >= 1; --q) {
      const int n = cls_next[q];
      cls_next[q] = run;
      run += n;
    }
  }
  first_s[e] = first_row;
  fill[e] = 0;
  __syncthreads();
  if (e < E && nb > 0) {
    for (int b = 0; b + 1 < nb; ++b) items[atomicAdd(&cls_next[q_full], 1)] = (e << 16) | b;
    items[atomicAdd(&cls_next[q_last], 1)] = (e << 16) | (nb - 1);
  }
  const bool held = Tk <= 1024 * R;
  for (int base = 0; base < Tk; base += 1024 * R) {
    if (!held) {
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const int idx = base + u * 1024 + e;
        ex[u] = idx < Tk ? topi[idx] : -1;
      }
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (ex[u] < 0) continue;
      const int idx = base + u * 1024 + e;
      const int pos = first_s[ex[u]] + atomicAdd(&fill[ex[u]], 1);
      perm[pos] = idx;
      slot_pos[idx] = pos;
    }
  }
}

// The routing and planning kernels and their stamping builds (each wavefront stamps after the body).
template <int RDT, int EJ>
__global__ __launch_bounds__(256) void k_moe_route(const void* __restrict__ router, int T, int E, int k,
                                                   int* __restrict__ topi, float* __restrict__ topw) {
  moe_route<RDT, EJ>(router, T, E, k, topi, topw);
}

template <int RDT, int EJ>
__global__ __launch_bounds__(256) void k_moe_route_tl(const void* __restrict__ router, int T, int E, int k,
                                                      int* __restrict__ topi, float* __restrict__ topw,
                                                      uint32_t* __restrict__ tl) {
  const TlStart t0 = tl_clock();
  moe_route<RDT, EJ>(router, T, E, k, topi, topw);
  tl_stamp(tl, t0);
}

__global__ __launch_bounds__(1024) void k_moe_plan(int* __restrict__ counts, int E, int rows, const int* __restrict__ topi,
                                                   int Tk, int* __restrict__ offsets, int* __restrict__ items,
                                                   int* __restrict__ n_items, int* __restrict__ perm,
                                                   int* __restrict__ slot_pos) {
  moe_plan(counts, E, rows, topi, Tk, offsets, items, n_items, perm, slot_pos);
}

__global__ __launch_bounds__(1024) void k_moe_plan_tl(int* __restrict__ counts, int E, int rows,
                                                      const int* __restrict__ topi, int Tk, int* __restrict__ offsets,
                                                      int* __restrict__ items, int* __restrict__ n_items,
                                                      int* __restrict__ perm, int* __restrict__ slot_pos,
                                                      uint32_t* __restrict__ tl) {
  const TlStart t0 = tl_clock();
  moe_plan(counts, E, rows, topi, Tk, offsets, items, n_items, perm, slot_pos);
  tl_stamp(tl, t0);
}

// ------------------------------------------------------------------ activations

enum : int { ACT_RELU = 0, ACT_GELU = 1, ACT_SILU = 2, ACT_IDENTITY = 3, ACT_SWIGLU = 4 };

template <int DT>
__device__ __forceinline__ float rt(float x) {
  return round_to<DT>(x);
}

template <int DT>
__device__ __forceinline__ float sigmoid_t(float x) {
  return rt<DT>(1.f / (1.f + expf(-x)));
}

// swiglu_gate/3 (moe.ex:199-206): g * sigmoid(alpha * g) * (l + beta), g and l limited first
// when limit is not 0; each operation rounds to the input type.
template <int DT>
__device__ __forceinline__ float swiglu(float g, float l, float alpha, float beta, float limit) {
  if (limit != 0.f) {
    g = fminf(g, limit);
    l = fminf(fmaxf(l, -limit), limit);
  }
  const float sg = sigmoid_t<DT>(rt<DT>(alpha * g));
  return rt<DT>(rt<DT>(g * sg) * rt<DT>(l + beta));
}

// The activation of one element: elementwise activations of h, or swiglu of (h, l).
template <int DT>
__device__ __forceinline__ float activate(int act, float h, float l, float alpha, float beta, float limit) {
  switch (act) {
    case ACT_RELU: return fmaxf(h, 0.f);
    case ACT_SILU: return rt<DT>(h * sigmoid_t<DT>(h));
    case ACT_GELU: return rt<DT>(h * rt<DT>(0.5f * rt<DT>(1.f + rt<DT>(erff(rt<DT>(h * 0.70710678118654752f))))));
    case ACT_SWIGLU: return swiglu<DT>(h, l, alpha, beta, limit);
    default: return h;
  }
}

// ------------------------------------------------------------------ grouped expert GEMMs

// The rows of a work item: expert, first sorted row, row count.
struct MoeItem {
  int e, row0, rows;
};

__device__ __forceinline__ MoeItem moe_item(const int* items, int item, const int* offsets, const int* counts,
                                            int rows) {
  const int it = items[item];
  const int e = it >> 16, b = it & 0xffff;
  return MoeItem{e, offsets[e] + b * rows, min(rows, counts[e] - b * rows)};
}

// LDS slot of 16-byte piece `piece` of A row `row`: the XOR swizzle (frag_swizzle) under which
// the fragment reads of 16 consecutive rows meet no bank conflict (8-bit weights: 8 pieces per row).
template <int BITS>
__device__ __forceinline__ int a_slot_moe(int row, int piece) {
  return piece ^ frag_swizzle<BITS == 8 ? 8 : 16>(row);
}

// Epilogue of the fast grouped product: none (the f16 sums), an activation of the sums plus the
// bias, or swiglu of two tiles (fc1 and fc3, or the two halves of fc1).
enum : int { EPI_STORE = 0, EPI_ACT = 1, EPI_GLU = 2 };

// out[row][n] = epilogue(sum_k A[src(row)][k] * W_e[n][k]) for the up to 16*MT sorted rows of
// one work item, f16 in and out with f32 sums (v_mfma_f32_16x16x32_f16). src(row) = perm[row] /
// perm_div when perm is given (rows gathered from the tokens), else row. Each of the eight
// wavefronts owns one 16-column output tile (and, for EPI_GLU, the matching tile of the second
// weight) over all of K; the item's A rows pass through LDS one chunk at a time, double
// buffered, with the next chunk's weights in flight.
// (The body; k_moe_gemm_f16 and its stamping build k_moe_gemm_f16_tl below are the kernels.)
template <int BITS, bool HAS_ZP, bool SPLIT, int EPI, int MT, bool TL>
__device__ __forceinline__ void moe_gemm_f16(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const uint4_t* __restrict__ qt2, const uint16_t* __restrict__ sc2, const uint8_t* __restrict__ zp2,
    int tile_off2, int ntiles, int nchunks, int nbc, int bsc_shift, int tiles_per_expert, int out_tiles, int gpw,
    const _Float16* __restrict__ A, int a_rows, int lda, const int* __restrict__ perm, int perm_div,
    const int* __restrict__ items, const int* __restrict__ n_items, const int* __restrict__ offsets,
    const int* __restrict__ counts, const void* __restrict__ bias1, const void* __restrict__ bias2, int bias_dt,
    int bias_ld, int act, float alpha, float beta, float limit, _Float16* __restrict__ out, int ldo,
    const int* __restrict__ out_perm, uint32_t* __restrict__ tl) {
  const TlStart tl0 = TL ? tl_clock() : TlStart{0u, 0u};
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int STEPS = GW / 8;
  constexpr int NJ = SPLIT ? STEPS : 1;
  constexpr int ROWB = CW * 2;                   // LDS bytes per A row
  constexpr int PPR = CW / 8;                    // 16-byte pieces per row
  constexpr int ROWS = 16 * MT;                  // rows per work item
  constexpr int PIECES = ROWS * PPR;             // per chunk
  constexpr int LOADS = (PIECES + 511) / 512;    // per thread
  constexpr int NW = EPI == EPI_GLU ? 2 : 1;
  __shared__ __align__(16) uint8_t lds[2 * ROWS * ROWB];
  if (static_cast<int>(blockIdx.y) >= *n_items) {
    if constexpr (TL) tl_stamp(tl, tl0);
    return;
  }
  const MoeItem it = moe_item(items, blockIdx.y, offsets, counts, ROWS);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches, one LDS ring base
  const int r = lane & 15, g = lane >> 4;
  // The workgroup's groups of eight output tiles: g0 .. g0 + ng - 1, one after the other through
  // one chunk pipeline (the next group's first weights in flight during the last chunk).
  const int g0 = blockIdx.x * gpw;
  const int ng = min(gpw, (out_tiles + 7) / 8 - g0);
  auto lt_of = [&](int gi) { return (g0 + gi) * 8 + wave; };  // this wavefront's output tile within the expert
  auto active_g = [&](int gi) { return lt_of(gi) < out_tiles; };
  const uint32_t nch = static_cast<uint32_t>(nchunks);
  const uint32_t n_params = static_cast<uint32_t>(ntiles) * nch * nbc * 16;
  const auto a_rsrc = buffer_rsrc(A, static_cast<uint32_t>(a_rows) * lda * 2);
  __amdgpu_buffer_rsrc_t q_rsrc[NW], s_rsrc[NW], z_rsrc[NW];
  uint32_t tile0[NW];  // the weight tiles of group 0; group gi adds 8 gi
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    q_rsrc[v] = buffer_rsrc(v ? qt2 : qt, static_cast<uint32_t>(ntiles) * nch * 1024);
    s_rsrc[v] = buffer_rsrc(v ? sc2 : sc, n_params * 2);
    z_rsrc[v] = buffer_rsrc(v ? zp2 : zp, HAS_ZP ? zp_byte<BITS>(n_params) : 0u);
    tile0[v] = static_cast<uint32_t>(it.e * tiles_per_expert + lt_of(0) + (v ? tile_off2 : 0));
  }
  // A pieces this thread brings to LDS: row p / PPR, piece p % PPR of p = (tid + 512 l) mod
  // PIECES (rows past the item, and k past K, read zeros). Where 512 * LOADS exceeds PIECES, two
  // threads store the same piece, the same bytes.
  uint32_t a_src[LOADS];
  int a_dst[LOADS], a_k[LOADS];
#pragma unroll
  for (int l = 0; l < LOADS; ++l) {
    const int p = (tid + 512 * l) % PIECES;
    const int row = p / PPR, piece = p % PPR;
    const int src = row < it.rows ? (perm ? perm[it.row0 + row] / perm_div : it.row0 + row) : -1;
    a_src[l] = src >= 0 ? static_cast<uint32_t>(src) * lda * 2 + piece * 16 : 0x80000000u;
    a_dst[l] = row * ROWB + a_slot_moe<BITS>(row, piece) * 16;
    a_k[l] = piece * 8;
  }
  auto load_a = [&](uint32_t c, uint4_t (&v)[LOADS]) {
#pragma unroll
    for (int l = 0; l < LOADS; ++l) {
      const bool in_k = static_cast<int>(c) * CW + a_k[l] < lda;  // lda = K, a multiple of 8
      v[l] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, in_k ? a_src[l] + c * CW * 2 : 0x80000000u, 0, 0);
    }
  };
  auto store_a = [&](int buf, const uint4_t (&v)[LOADS]) {
#pragma unroll
    for (int l = 0; l < LOADS; ++l) *reinterpret_cast<uint4_t*>(lds + buf * ROWS * ROWB + a_dst[l]) = v[l];
  };
  struct WStage {
    uint4_t w[NW];
    uint32_t s[NW][NJ], z[NW][NJ];
  };
  auto load_w = [&](int gi, uint32_t c, WStage& st) {
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const uint32_t tile = tile0[v] + 8u * static_cast<uint32_t>(gi);
      st.w[v] = __builtin_amdgcn_raw_buffer_load_b128(q_rsrc[v], (tile * nch * 64 + lane) * 16, c * 1024, 0);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint32_t e = ((tile * nch + c) * nbc + ((g * GW + 8 * j * (SPLIT ? 1 : 0)) >> bsc_shift)) * 16 + r;
        st.s[v][j] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc[v], e * 2, 0, 0);
        if constexpr (HAS_ZP) st.z[v][j] = __builtin_amdgcn_raw_buffer_load_b8(z_rsrc[v], zp_byte<BITS>(e), 0, 0);
      }
    }
  };
  float4_t acc[NW][MT];
#pragma unroll
  for (int v = 0; v < NW; ++v)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[v][mt] = float4_t{0.f, 0.f, 0.f, 0.f};
  // The epilogue of group gi: lane (16g + r) holds rows mt*16 + r and columns lt*16 + 4g .. +3.
  auto store_group = [&](int gi) {
    const int n = lt_of(gi) * 16 + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int i = mt * 16 + r;
      if (i >= it.rows) continue;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float h = rt<DT_F16>(acc[0][mt][e]);
        if (EPI != EPI_STORE && bias1)
          h = rt<DT_F16>(h + load_float_rt(bias1, bias_dt, static_cast<int64_t>(it.e) * bias_ld + n + e));
        float l = 0.f;
        if constexpr (EPI == EPI_GLU) {
          l = rt<DT_F16>(acc[NW - 1][mt][e]);
          if (bias2)
            l = rt<DT_F16>(l + load_float_rt(bias2, bias_dt, static_cast<int64_t>(it.e) * bias_ld + n + e + tile_off2 * 16));
        }
        y[e] = EPI == EPI_STORE ? h : activate<DT_F16>(act, h, l, alpha, beta, limit);
      }
      const half2_t lo = {static_cast<_Float16>(y[0]), static_cast<_Float16>(y[1])};
      const half2_t hi = {static_cast<_Float16>(y[2]), static_cast<_Float16>(y[3])};
      const int orow = out_perm ? out_perm[it.row0 + i] : it.row0 + i;
      _Float16* dst = out + static_cast<int64_t>(orow) * ldo + n;
      *reinterpret_cast<uint2*>(dst) = make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
    }
  };
  // The chunk loop over the workgroup's groups (steps s: group s / nch, chunk s % nch),
  // specialized for the m-tiles that hold rows of this item (MA of MT, uniform per workgroup): an
  // item of 17-32 rows runs half the MFMAs and LDS reads of a full one.
  auto run = [&](auto ma) {
    constexpr int MA = decltype(ma)::value;
    uint4_t av[LOADS];
    WStage cur, next;
    load_a(0, av);
    if (active_g(0)) load_w(0, 0, cur);
    store_a(0, av);
    __syncthreads();
    const uint32_t total = static_cast<uint32_t>(ng) * nch;
    uint32_t c = 0;
    int gi = 0;
    for (uint32_t s = 0; s < total; ++s) {
      const bool more = s + 1 < total;
      const bool last_chunk = c + 1 == nch;
      const uint32_t c1 = last_chunk ? 0u : c + 1;
      const int gi1 = last_chunk ? gi + 1 : gi;
      if (more) {
        load_a(c1, av);
        if (active_g(gi1)) load_w(gi1, c1, next);
      }
      if (active_g(gi)) {
        const uint8_t* abase = lds + (s & 1) * ROWS * ROWB;
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
          const int piece = g * (GW / 8) + i;
          half8_t af[MA];
#pragma unroll
          for (int mt = 0; mt < MA; ++mt)
            af[mt] = *reinterpret_cast<const half8_t*>(abase + (mt * 16 + r) * ROWB + a_slot_moe<BITS>(mt * 16 + r, piece) * 16);
          const int j = SPLIT ? i : 0;
#pragma unroll
          for (int v = 0; v < NW; ++v) {
            const uint32_t zq = HAS_ZP ? 0x6400u + zp_field<BITS>(cur.z[v][j], zp_shift<BITS>(r)) : 0x6400u + (1u << (BITS - 1));
            const half8_t b = unpack_step<BITS>(cur.w[v], i, __builtin_bit_cast(half2_t, zq | (zq << 16)),
                                                __builtin_bit_cast(half2_t, cur.s[v][j] | (cur.s[v][j] << 16)));
#pragma unroll
            for (int mt = 0; mt < MA; ++mt)
              acc[v][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, af[mt], acc[v][mt], 0, 0, 0);
          }
        }
        if (last_chunk) {
          store_group(gi);
#pragma unroll
          for (int v = 0; v < NW; ++v)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[v][mt] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
      if (more) store_a((s + 1) & 1, av);
      __syncthreads();
      if (more) cur = next;
      c = c1;
      gi = gi1;
    }
  };
  const int used = (it.rows + 15) / 16;
  if (MT >= 4 && used > 2) {
    if (used > 3) run(std::integral_constant<int, MT>{});
    else run(std::integral_constant<int, MT >= 4 ? 3 : MT>{});
  } else if (MT >= 2 && used > 1) {
    run(std::integral_constant<int, MT >= 2 ? 2 : MT>{});
  } else {
    run(std::integral_constant<int, 1>{});
  }
  if constexpr (TL) tl_stamp(tl, tl0);
}

template <int BITS, bool HAS_ZP, bool SPLIT, int EPI, int MT>
__global__ __launch_bounds__(512) void k_moe_gemm_f16(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const uint4_t* __restrict__ qt2, const uint16_t* __restrict__ sc2, const uint8_t* __restrict__ zp2,
    int tile_off2, int ntiles, int nchunks, int nbc, int bsc_shift, int tiles_per_expert, int out_tiles, int gpw,
    const _Float16* __restrict__ A, int a_rows, int lda, const int* __restrict__ perm, int perm_div,
    const int* __restrict__ items, const int* __restrict__ n_items, const int* __restrict__ offsets,
    const int* __restrict__ counts, const void* __restrict__ bias1, const void* __restrict__ bias2, int bias_dt,
    int bias_ld, int act, float alpha, float beta, float limit, _Float16* __restrict__ out, int ldo,
    const int* __restrict__ out_perm) {
  moe_gemm_f16<BITS, HAS_ZP, SPLIT, EPI, MT, false>(
      qt, sc, zp, qt2, sc2, zp2, tile_off2, ntiles, nchunks, nbc, bsc_shift, tiles_per_expert, out_tiles, gpw, A, a_rows,
      lda, perm,
      perm_div, items, n_items, offsets, counts, bias1, bias2, bias_dt, bias_ld, act, alpha, beta, limit, out, ldo, out_perm,
      nullptr);
}

template <int BITS, bool HAS_ZP, bool SPLIT, int EPI, int MT>
__global__ __launch_bounds__(512) void k_moe_gemm_f16_tl(
    const uint4_t* __restrict__ qt, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    const uint4_t* __restrict__ qt2, const uint16_t* __restrict__ sc2, const uint8_t* __restrict__ zp2,
    int tile_off2, int ntiles, int nchunks, int nbc, int bsc_shift, int tiles_per_expert, int out_tiles, int gpw,
    const _Float16* __restrict__ A, int a_rows, int lda, const int* __restrict__ perm, int perm_div,
    const int* __restrict__ items, const int* __restrict__ n_items, const int* __restrict__ offsets,
    const int* __restrict__ counts, const void* __restrict__ bias1, const void* __restrict__ bias2, int bias_dt,
    int bias_ld, int act, float alpha, float beta, float limit, _Float16* __restrict__ out, int ldo,
    const int* __restrict__ out_perm, uint32_t* __restrict__ tl) {
  moe_gemm_f16<BITS, HAS_ZP, SPLIT, EPI, MT, true>(
      qt, sc, zp, qt2, sc2, zp2, tile_off2, ntiles, nchunks, nbc, bsc_shift, tiles_per_expert, out_tiles, gpw, A, a_rows,
      lda, perm,
      perm_div, items, n_items, offsets, counts, bias1, bias2, bias_dt, bias_ld, act, alpha, beta, limit, out, ldo, out_perm,
      tl);
}

// The same product for any float types (A in a_dt, weights dequantized in WDT, out in out_dt):
// one 16-column tile per workgroup, the four wavefronts splitting the chunks of K.
template <int BITS, int WDT, int ZK>
__global__ __launch_bounds__(256) void k_moe_gemm_general(
    const uint4_t* __restrict__ qt, const void* __restrict__ sc, const void* __restrict__ zp, int nchunks, int nbc,
    int bsc_shift, int tiles_per_expert, int K, const void* __restrict__ A, int a_dt, int lda,
    const int* __restrict__ perm, int perm_div, const int* __restrict__ items, const int* __restrict__ n_items,
    const int* __restrict__ offsets, const int* __restrict__ counts, void* __restrict__ out, int out_dt, int ldo) {
  constexpr int CW = 512 / BITS;
  constexpr int GW = CW / 4;
  constexpr int PER_WORD = 32 / BITS;
  __shared__ float red[4][kMoeRows][16];
  if (static_cast<int>(blockIdx.y) >= *n_items) return;
  const MoeItem it = moe_item(items, blockIdx.y, offsets, counts, kMoeRows);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t t = static_cast<int64_t>(it.e) * tiles_per_expert + blockIdx.x;
  int64_t src[kMoeRows];
#pragma unroll
  for (int i = 0; i < kMoeRows; ++i)
    src[i] = i < it.rows ? (perm ? perm[it.row0 + i] / perm_div : it.row0 + i) : 0;
  float acc[kMoeRows];
#pragma unroll
  for (int i = 0; i < kMoeRows; ++i) acc[i] = 0.f;
  for (int c = wave; c < nchunks; c += 4) {
    const int64_t tc = t * nchunks + c;
    const uint4_t w = qt[tc * 64 + lane];
    for (int e = 0; e < GW; ++e) {
      const int k = c * CW + g * GW + e;
      if (k >= K) break;
      const int64_t p = (tc * nbc + ((g * GW + e) >> bsc_shift)) * 16 + r;
      const float s = load_as_f32<WDT>(sc, p);
      float z;
      if constexpr (ZK == TMH_ZP_PACKED) {
        const uint8_t byte = static_cast<const uint8_t*>(zp)[zp_byte<BITS>(p)];
        z = static_cast<float>(zp_field<BITS>(byte, zp_shift<BITS>(static_cast<uint32_t>(p))));
      } else {
        z = static_cast<float>(1 << (BITS - 1));
      }
      const float wv = dequant_value<WDT>(static_cast<float>(word_value<BITS>(w[e / PER_WORD], e % PER_WORD)), z, s);
#pragma unroll
      for (int i = 0; i < kMoeRows; ++i)
        if (i < it.rows) acc[i] = fmaf(load_float_rt(A, a_dt, src[i] * lda + k), wv, acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < kMoeRows; ++i) {
    float v = acc[i];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (g == 0) red[wave][i][r] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x >> 4; i < it.rows; i += 16) {
    const int col = threadIdx.x & 15;
    const float v = red[0][i][col] + red[1][i][col] + red[2][i][col] + red[3][i][col];
    store_float_rt(out, out_dt, static_cast<int64_t>(it.row0 + i) * ldo + blockIdx.x * 16 + col, v);
  }
}

// ------------------------------------------------------------------ activation and sum

// Activated rows: hact[row][c] from h1 (and h3), with the biases of the row's expert.
// fusion (for swiglu): 0 with h3 = gate h1, linear h3; 2 = halves of h1; otherwise interleaved.
template <int DT>
__global__ __launch_bounds__(256) void k_moe_activate(const void* __restrict__ h1, const void* __restrict__ h3, int n1,
                                                      int inter, const void* __restrict__ b1,
                                                      const void* __restrict__ b3, int bias_dt,
                                                      const int* __restrict__ perm, const int* __restrict__ topi,
                                                      int Tk, int act, int fusion, float alpha, float beta, float limit,
                                                      void* __restrict__ hact) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int width = act == ACT_SWIGLU ? inter : n1;
  if (idx >= static_cast<int64_t>(Tk) * width) return;
  const int row = static_cast<int>(idx / width), c = static_cast<int>(idx - static_cast<int64_t>(row) * width);
  const int e = topi[perm[row]];
  auto h = [&](const void* src, const void* bias, int col) -> float {
    float v = load_as_f32<DT>(src, static_cast<int64_t>(row) * n1 + col);
    if (bias) v = rt<DT>(v + load_float_rt(bias, bias_dt, static_cast<int64_t>(e) * n1 + col));
    return v;
  };
  float g, l = 0.f;
  if (act != ACT_SWIGLU) {
    g = h(h1, b1, c);
  } else if (h3) {
    g = h(h1, b1, c);
    l = h(h3, b3, c);
  } else if (fusion == 2) {
    g = h(h1, b1, c);
    l = h(h1, b1, inter + c);
  } else {
    g = h(h1, b1, 2 * c);
    l = h(h1, b1, 2 * c + 1);
  }
  const float y = activate<DT>(act, g, l, alpha, beta, limit);
  store_as<DT>(hact, idx, y);
}

// y[t][h] = sum over the token's slots j of weight_j * (o[row of (t, j)][h] + fc2 bias), in slot
// order; a slot of weight 0 adds 0. V consecutive columns per thread. The row of (t, j) is
// slot_pos[t * k + j] for o in expert order, t * k + j for o in token order (slot_pos null).
// (The body; k_moe_combine and k_moe_combine_tl below are the kernels.)
template <int DT, int V>
__device__ __forceinline__ void moe_combine(const void* __restrict__ o, int H, const void* __restrict__ b2,
                                            int bias_dt, const int* __restrict__ topi,
                                            const float* __restrict__ topw, const int* __restrict__ slot_pos,
                                            int T, int k, void* __restrict__ y, bool y_vec) {
  constexpr int JU = 8;  // slots whose loads are in flight together
  const int64_t idx = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * V;
  if (idx >= static_cast<int64_t>(T) * H) return;
  const int t = static_cast<int>(idx / H), hc = static_cast<int>(idx - static_cast<int64_t>(t) * H);
  if constexpr (DT == DT_F16 && V == 8) {
    if (!b2) {
      // f16 rows without a bias: the products and sums in packed f16. Each product of two f16
      // values is exact in f32 and each sum of two f16 values rounds the same from f32 as
      // directly, so v_pk_mul_f16 then v_pk_add_f16 give the bits of the f32 steps rounded to
      // f16 after each one, at an eighth of the instructions.
#pragma clang fp contract(off)
      half8_t acc = {};
      for (int j0 = 0; j0 < k; j0 += JU) {
        half8_t ov[JU];
        _Float16 wgt[JU];
#pragma unroll
        for (int u = 0; u < JU; ++u) {
          const int j = j0 + u < k ? j0 + u : k - 1;
          wgt[u] = static_cast<_Float16>(topw[t * k + j]);
          const int64_t row = slot_pos ? slot_pos[t * k + j] : t * k + j;
          ov[u] = *reinterpret_cast<const half8_t*>(static_cast<const _Float16*>(o) + row * H + hc);
        }
#pragma unroll
        for (int u = 0; u < JU; ++u) {
          if (j0 + u >= k || wgt[u] == static_cast<_Float16>(0.f)) continue;
          const half8_t prod = ov[u] * wgt[u];
          acc = acc + prod;
        }
      }
      if (y_vec) {
        *reinterpret_cast<half8_t*>(static_cast<_Float16*>(y) + idx) = acc;
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) store_as<DT>(y, idx + v, static_cast<float>(acc[v]));
      }
      return;
    }
  }
  float sum[V];
#pragma unroll
  for (int v = 0; v < V; ++v) sum[v] = 0.f;
  for (int j0 = 0; j0 < k; j0 += JU) {
    // Slot data and rows of up to JU slots first (slots past k repeat slot k-1 and are not
    // summed), then the sum in slot order.
    float wgt[JU];
    int ex[JU];
    float ov[JU][V];
#pragma unroll
    for (int u = 0; u < JU; ++u) {
      const int j = j0 + u < k ? j0 + u : k - 1;
      wgt[u] = rt<DT>(topw[t * k + j]);
      ex[u] = topi[t * k + j];
      const int64_t row = slot_pos ? slot_pos[t * k + j] : t * k + j;
      if constexpr (DT == DT_F16 && V == 8) {
        const half8_t h8 = *reinterpret_cast<const half8_t*>(static_cast<const _Float16*>(o) + row * H + hc);
#pragma unroll
        for (int v = 0; v < V; ++v) ov[u][v] = static_cast<float>(h8[v]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) ov[u][v] = load_as_f32<DT>(o, row * H + hc + v);
      }
    }
#pragma unroll
    for (int u = 0; u < JU; ++u) {
      if (j0 + u >= k || wgt[u] == 0.f) continue;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        float x = ov[u][v];
        if (b2) x = rt<DT>(x + load_float_rt(b2, bias_dt, static_cast<int64_t>(ex[u]) * H + hc + v));
        sum[v] = rt<DT>(sum[v] + rt<DT>(x * wgt[u]));
      }
    }
  }
  if (DT == DT_F16 && V == 8 && y_vec) {
    half8_t h8;
#pragma unroll
    for (int v = 0; v < V; ++v) h8[v] = static_cast<_Float16>(sum[v]);
    *reinterpret_cast<half8_t*>(static_cast<_Float16*>(y) + idx) = h8;
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) store_as<DT>(y, idx + v, sum[v]);
  }
}

template <int DT, int V>
__global__ __launch_bounds__(256) void k_moe_combine(const void* __restrict__ o, int H, const void* __restrict__ b2,
                                                     int bias_dt, const int* __restrict__ topi,
                                                     const float* __restrict__ topw, const int* __restrict__ slot_pos,
                                                     int T, int k, void* __restrict__ y, bool y_vec) {
  moe_combine<DT, V>(o, H, b2, bias_dt, topi, topw, slot_pos, T, k, y, y_vec);
}

template <int DT, int V>
__global__ __launch_bounds__(256) void k_moe_combine_tl(const void* __restrict__ o, int H, const void* __restrict__ b2,
                                                        int bias_dt, const int* __restrict__ topi,
                                                        const float* __restrict__ topw,
                                                        const int* __restrict__ slot_pos, int T, int k,
                                                        void* __restrict__ y, bool y_vec, uint32_t* __restrict__ tl) {
  const TlStart t0 = tl_clock();
  moe_combine<DT, V>(o, H, b2, bias_dt, topi, topw, slot_pos, T, k, y, y_vec);
  tl_stamp(tl, t0);
}

// ------------------------------------------------------------------ launchers

int bsc_shift_moe(const tmh_weight* w) {
  int cw = 512 / w->bits, bs = std::min(w->block_size, cw), s = 0;
  while ((1 << s) < bs) ++s;
  return s;
}

// The epilogue of a fast grouped product.
struct MoeEpilogue {
  int kind = EPI_STORE;
  const tmh_weight* w2 = nullptr;  // EPI_GLU: the weight of the second tile (fc3, or fc1 itself)
  int tile_off2 = 0;               // and that tile's offset within the expert
  int out_tiles = 0;               // output tiles per expert
  const void *bias1 = nullptr, *bias2 = nullptr;
  int bias_dt = TMH_F32, bias_ld = 0, act = ACT_IDENTITY;
  float alpha = 1.f, beta = 0.f, limit = 0.f;
  int rows = 32;                   // rows per work item: 32 or 64
  const int* out_perm = nullptr;   // output row of each sorted row (else the sorted row itself)
};

template <int BITS, bool HAS_ZP, bool SPLIT, int EPI, int MT>
void launch_moe_f16_e(const tmh_weight* w, int tpe, const void* A, int a_rows, int lda, const int* perm, int perm_div,
                      const int* items, const int* n_items, int max_items, const int* offsets, const int* counts,
                      void* out, int ldo, const MoeEpilogue& ep, hipStream_t s) {
  const tmh_weight* w2 = ep.w2 ? ep.w2 : w;
  // Groups of eight output tiles per workgroup, one after the other: the stored products (fc2,
  // many groups per item) run four, so the workgroups' prologues and the last partial round of
  // workgroups shrink; the others one.
  const int groups = (ep.out_tiles + 7) / 8;
  const char* gpw_env = std::getenv("TMH_MOE_GPW");
  const int gpw = gpw_env ? std::max(1, std::atoi(gpw_env)) : (EPI == EPI_STORE && groups >= 16 ? 4 : 1);
  const dim3 grid(static_cast<unsigned>((groups + gpw - 1) / gpw), static_cast<unsigned>(max_items));
#define TMH_MOE_ARGS                                                                                                   \
  reinterpret_cast<const uint4_t*>(w->d_q), static_cast<const uint16_t*>(w->d_scale),                                 \
      static_cast<const uint8_t*>(w->d_zero), reinterpret_cast<const uint4_t*>(w2->d_q),                              \
      static_cast<const uint16_t*>(w2->d_scale), static_cast<const uint8_t*>(w2->d_zero), ep.tile_off2,               \
      static_cast<int>(w->ntiles), static_cast<int>(w->nchunks), w->nbc, bsc_shift_moe(w), tpe, ep.out_tiles, gpw,    \
      static_cast<const _Float16*>(A), a_rows, lda, perm, perm_div, items, n_items, offsets, counts, ep.bias1,        \
      ep.bias2, ep.bias_dt, ep.bias_ld, ep.act, ep.alpha, ep.beta, ep.limit, static_cast<_Float16*>(out), ldo,       \
      ep.out_perm
  if (uint32_t* tl = timeline_slots(TMH_TL_MOE_GEMM, static_cast<int64_t>(grid.x) * grid.y * 8))
    k_moe_gemm_f16_tl<BITS, HAS_ZP, SPLIT, EPI, MT><<<grid, 512, 0, s>>>(TMH_MOE_ARGS, tl);
  else
    k_moe_gemm_f16<BITS, HAS_ZP, SPLIT, EPI, MT><<<grid, 512, 0, s>>>(TMH_MOE_ARGS);
#undef TMH_MOE_ARGS
}

template <int BITS, bool HAS_ZP, bool SPLIT>
void launch_moe_f16_v(const tmh_weight* w, int tpe, const void* A, int a_rows, int lda, const int* perm, int perm_div,
                      const int* items, const int* n_items, int max_items, const int* offsets, const int* counts,
                      void* out, int ldo, const MoeEpilogue& ep, hipStream_t s) {
#define TMH_MOE_EPI(E, MT) \
  launch_moe_f16_e<BITS, HAS_ZP, SPLIT, E, MT>(w, tpe, A, a_rows, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, ldo, ep, s)
  if (ep.rows == 64) {
    if (ep.kind == EPI_GLU) TMH_MOE_EPI(EPI_GLU, 4);
    else if (ep.kind == EPI_ACT) TMH_MOE_EPI(EPI_ACT, 4);
    else TMH_MOE_EPI(EPI_STORE, 4);
  } else {
    if (ep.kind == EPI_GLU) TMH_MOE_EPI(EPI_GLU, 2);
    else if (ep.kind == EPI_ACT) TMH_MOE_EPI(EPI_ACT, 2);
    else TMH_MOE_EPI(EPI_STORE, 2);
  }
#undef TMH_MOE_EPI
}

template <int BITS>
void launch_moe_f16(const tmh_weight* w, int tpe, const void* A, int a_rows, int lda, const int* perm, int perm_div,
                    const int* items, const int* n_items, int max_items, const int* offsets, const int* counts,
                    void* out, int ldo, const MoeEpilogue& ep, hipStream_t s) {
  const bool zp = w->zp_kind == TMH_ZP_PACKED;
  const bool split = w->block_size < (512 / BITS) / 4;
#define TMH_MOE_F16(Z, S) \
  launch_moe_f16_v<BITS, Z, S>(w, tpe, A, a_rows, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, ldo, ep, s)
  if (zp && split) TMH_MOE_F16(true, true);
  else if (zp) TMH_MOE_F16(true, false);
  else if (split) TMH_MOE_F16(false, true);
  else TMH_MOE_F16(false, false);
#undef TMH_MOE_F16
}

template <int BITS, int WDT>
void launch_moe_general_w(const tmh_weight* w, int tpe, const void* A, int a_dt, int lda, const int* perm, int perm_div,
                          const int* items, const int* n_items, int max_items, const int* offsets, const int* counts,
                          void* out, int out_dt, int ldo, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(tpe), static_cast<unsigned>(max_items));
  const auto* qt = reinterpret_cast<const uint4_t*>(w->d_q);
  const int sh = bsc_shift_moe(w);
  if (w->zp_kind == TMH_ZP_PACKED)
    k_moe_gemm_general<BITS, WDT, TMH_ZP_PACKED><<<grid, 256, 0, s>>>(
        qt, w->d_scale, w->d_zero, static_cast<int>(w->nchunks), w->nbc, sh, tpe, static_cast<int>(w->K), A, a_dt, lda,
        perm, perm_div, items, n_items, offsets, counts, out, out_dt, ldo);
  else
    k_moe_gemm_general<BITS, WDT, TMH_ZP_NONE><<<grid, 256, 0, s>>>(
        qt, w->d_scale, w->d_zero, static_cast<int>(w->nchunks), w->nbc, sh, tpe, static_cast<int>(w->K), A, a_dt, lda,
        perm, perm_div, items, n_items, offsets, counts, out, out_dt, ldo);
}

template <int BITS>
void launch_moe_general(const tmh_weight* w, int tpe, const void* A, int a_dt, int lda, const int* perm, int perm_div,
                        const int* items, const int* n_items, int max_items, const int* offsets, const int* counts,
                        void* out, int out_dt, int ldo, hipStream_t s) {
  switch (w->wdtype) {
    case TMH_F16:
      launch_moe_general_w<BITS, DT_F16>(w, tpe, A, a_dt, lda, perm, perm_div, items, n_items, max_items, offsets,
                                         counts, out, out_dt, ldo, s);
      break;
    case TMH_BF16:
      launch_moe_general_w<BITS, DT_BF16>(w, tpe, A, a_dt, lda, perm, perm_div, items, n_items, max_items, offsets,
                                          counts, out, out_dt, ldo, s);
      break;
    default:
      launch_moe_general_w<BITS, DT_F32>(w, tpe, A, a_dt, lda, perm, perm_div, items, n_items, max_items, offsets,
                                         counts, out, out_dt, ldo, s);
  }
}

// The fast grouped product applies: f16 rows and weights, packed or no zero points, K a multiple
// of 8, 32-bit buffer offsets.
bool moe_fast(const tmh_weight* w, int a_dt, const void* A, int a_rows, int lda) {
  return a_dt == TMH_F16 && w->wdtype == TMH_F16 && w->zp_kind != TMH_ZP_FLOAT && lda % 8 == 0 &&
         reinterpret_cast<uintptr_t>(A) % 16 == 0 && static_cast<int64_t>(a_rows) * lda * 2 < (int64_t(1) << 31) &&
         (w->ntiles + 1) * w->nchunks * 1024 < (int64_t(1) << 31);
}

// One grouped product: rows (gathered through perm when given) times each row's expert. The
// fast path applies the epilogue; the general path stores the sums (EPI_STORE only).
void moe_gemm(const tmh_weight* w, int experts, const void* A, int a_dt, int a_rows, int lda, const int* perm,
              int perm_div, const int* items, const int* n_items, int max_items, const int* offsets,
              const int* counts, void* out, int ldo, hipStream_t s, MoeEpilogue ep = MoeEpilogue()) {
  const int tpe = static_cast<int>(w->N / experts / 16);
  if (moe_fast(w, a_dt, A, a_rows, lda)) {
    if (ep.out_tiles == 0) ep.out_tiles = tpe;
    switch (w->bits) {
      case 2: launch_moe_f16<2>(w, tpe, A, a_rows, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, ldo, ep, s); break;
      case 4: launch_moe_f16<4>(w, tpe, A, a_rows, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, ldo, ep, s); break;
      default: launch_moe_f16<8>(w, tpe, A, a_rows, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, ldo, ep, s);
    }
    return;
  }
  switch (w->bits) {
    case 2: launch_moe_general<2>(w, tpe, A, a_dt, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, a_dt, ldo, s); break;
    case 4: launch_moe_general<4>(w, tpe, A, a_dt, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, a_dt, ldo, s); break;
    default: launch_moe_general<8>(w, tpe, A, a_dt, lda, perm, perm_div, items, n_items, max_items, offsets, counts, out, a_dt, ldo, s);
  }
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

}  // namespace

extern "C" {

int tmh_weight_upload_qmoe(tmh_ctx* ctx, const uint8_t* h_w, size_t w_bytes, const void* h_scales, int scales_dtype,
                           size_t scales_count, const uint8_t* h_zero_points, size_t zp_bytes, int64_t E, int64_t N,
                           int64_t K, int bits, int64_t block_size, int weight_dtype, tmh_weight** out) {
  if (!ctx) return fail(nullptr, TMH_ERR_INVALID, "the context is NULL");
  if (!out) return fail(ctx, TMH_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (bits != 2 && bits != 4 && bits != 8)
    return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE expert_weight_bits must be 2, 4 or 8, got %d", bits);
  if (E <= 0 || N <= 0 || K <= 0) return fail(ctx, TMH_ERR_INVALID, "QMoE weights must have positive sizes");
  if (N % 16 != 0) return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE expert rows (%lld) must be a multiple of 16", (long long)N);
  if ((K * bits) % 8 != 0) return fail(ctx, TMH_ERR_INVALID, "QMoE rows of %lld %d-bit values are not whole bytes", (long long)K, bits);
  const int64_t row_bytes = K * bits / 8;
  if (!h_w || w_bytes != static_cast<size_t>(E * N * row_bytes))
    return fail(ctx, TMH_ERR_INVALID, "QMoE weights hold %zu bytes; %lld expected", w_bytes, (long long)(E * N * row_bytes));
  const int64_t rows = E * N;
  const bool blockwise = block_size > 0 && h_scales;
  int64_t bs, blocks;  // block size and blocks per row as given
  if (blockwise) {
    if (block_size < 16 || (block_size & (block_size - 1)))
      return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE block_size must be a power of two of at least 16, got %lld", (long long)block_size);
    if (scales_count % rows != 0) return fail(ctx, TMH_ERR_INVALID, "QMoE scales do not split into %lld rows", (long long)rows);
    bs = block_size;
    blocks = static_cast<int64_t>(scales_count) / rows;  // K pads to whole blocks (moe.ex:225-233)
    if (blocks * bs < K) return fail(ctx, TMH_ERR_INVALID, "QMoE has %lld blocks of %lld for K=%lld", (long long)blocks, (long long)bs, (long long)K);
  } else {
    if (h_scales && scales_count != static_cast<size_t>(rows))
      return fail(ctx, TMH_ERR_INVALID, "QMoE per-row scales hold %zu values; %lld expected", scales_count, (long long)rows);
    bs = 512 / bits;  // one scale and zero point per chunk, copied from the row's
    blocks = (K + bs - 1) / bs;
  }
  const int64_t kb = (K + bs - 1) / bs;  // blocks that hold values of the row
  const int64_t bbytes = bs * bits / 8;
  // B as MatMulNBits lays it out: [rows, kb, bs*bits/8], zero past K.
  std::vector<uint8_t> b(static_cast<size_t>(rows * kb * bbytes), 0);
  for (int64_t rr = 0; rr < rows; ++rr)
    std::copy_n(h_w + rr * row_bytes, row_bytes, b.begin() + rr * kb * bbytes);
  const int sdt = h_scales ? scales_dtype : TMH_F32;
  if (!is_float_dtype(sdt)) return fail(ctx, TMH_ERR_INVALID, "QMoE scales must be float");
  const size_t ses = static_cast<size_t>(dtype_size(sdt));
  std::vector<uint8_t> scales(static_cast<size_t>(rows * kb) * ses);
  const float one = 1.f;
  for (int64_t rr = 0; rr < rows; ++rr)
    for (int64_t bl = 0; bl < kb; ++bl) {
      const uint8_t* src = !h_scales ? reinterpret_cast<const uint8_t*>(&one)
                           : blockwise ? static_cast<const uint8_t*>(h_scales) + (rr * blocks + bl) * ses
                                       : static_cast<const uint8_t*>(h_scales) + rr * ses;
      std::copy_n(src, ses, scales.begin() + (rr * kb + bl) * ses);
    }
  // Zero points of every (row, block), then packed as MatMulNBits rows of ceil(kb*bits/8) bytes.
  const int64_t per = 8 / bits, zrow = (kb * bits + 7) / 8;
  auto value = [&](const uint8_t* packed, int64_t i) -> uint8_t {
    return static_cast<uint8_t>((packed[i / per] >> ((i % per) * bits)) & ((1 << bits) - 1));
  };
  std::vector<uint8_t> zero;
  if (h_zero_points) {
    zero.assign(static_cast<size_t>(rows * zrow), 0);
    const int64_t in_row = (blocks * bits + 7) / 8, zn = (N + per - 1) / per;
    const size_t expect = static_cast<size_t>(blockwise ? rows * in_row : E * zn);
    if (zp_bytes != expect)
      return fail(ctx, TMH_ERR_INVALID, "QMoE zero points hold %zu bytes; %zu expected", zp_bytes, expect);
    for (int64_t rr = 0; rr < rows; ++rr) {
      // Block-wise: {E, N, ceil(blocks*bits/8)} packed along the blocks; per row: {E, N} packed
      // along N (moe.ex:233-244).
      const uint8_t z_row = blockwise ? 0 : value(h_zero_points + (rr / N) * zn, rr % N);
      for (int64_t bl = 0; bl < kb; ++bl) {
        const uint8_t z = blockwise ? value(h_zero_points + rr * in_row, bl) : z_row;
        zero[rr * zrow + bl / per] |= static_cast<uint8_t>(z << ((bl % per) * bits));
      }
    }
  }
  return tmh_weight_upload_nbits(ctx, b.data(), b.size(), scales.data(), sdt, static_cast<size_t>(rows * kb),
                                 h_zero_points ? zero.data() : nullptr, h_zero_points ? TMH_ZP_PACKED : TMH_ZP_NONE,
                                 TMH_U8, zero.size(), K, rows, bits, static_cast<int>(bs), weight_dtype, out);
}

int tmh_qmoe(tmh_ctx* ctx, const void* d_x, int x_dtype, int64_t T, int64_t H, const void* d_router, int router_dtype,
             int64_t E, int k, const tmh_weight* fc1, const void* d_fc1_bias, const tmh_weight* fc2,
             const void* d_fc2_bias, const tmh_weight* fc3, const void* d_fc3_bias, int bias_dtype, int activation,
             int swiglu_fusion, float alpha, float beta, float limit, void* d_y, void* stream) {
  TimelineScope timeline(ctx);
  // The sizes are checked before the device is touched (a context-free caller gets the same errors).
  if (!is_float_dtype(x_dtype) || !is_float_dtype(router_dtype))
    return fail(ctx, TMH_ERR_INVALID, "QMoE input and router must be float tensors");
  if (E <= 0 || E > 1024) return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE supports 1 to 1024 experts, got %lld", (long long)E);
  if (k <= 0 || k > 32 || k > E) return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE k must be in 1..min(32, experts), got %d", k);
  if (activation < ACT_RELU || activation > ACT_SWIGLU) return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE activation %d", activation);
  if (T < 0 || H <= 0) return fail(ctx, TMH_ERR_INVALID, "QMoE sizes must be positive");
  // Work items are numbered expert << 16 | item, with at least kMoeRows rows per item, and an
  // expert receives at most one row per token (the k experts of a token are distinct): T tokens
  // must not give an expert more than 2^16 items.
  if ((T + kMoeRows - 1) / kMoeRows > (int64_t(1) << 16))
    return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE supports at most %lld tokens per call, got %lld",
                (long long)kMoeRows << 16, (long long)T);
  if (T * k >= (int64_t(1) << 24)) return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE supports fewer than 2^24 routed rows");
  TMH_TRY(use_device(ctx));
  if (!fc1 || !fc2) return fail(ctx, TMH_ERR_INVALID, "QMoE needs fc1 and fc2 weights");
  if (fc1->N % E || fc2->N % E) return fail(ctx, TMH_ERR_INVALID, "QMoE weights do not hold %lld experts", (long long)E);
  const int64_t n1 = fc1->N / E;
  if (fc1->K != H || fc2->N / E != H)
    return fail(ctx, TMH_ERR_INVALID, "QMoE fc1 [%lld, %lld] and fc2 rows %lld do not fit hidden size %lld", (long long)n1,
                (long long)fc1->K, (long long)(fc2->N / E), (long long)H);
  // The grouped products give each expert whole 16-row weight tiles, and the final sum reads
  // eight columns per thread: rows per expert (fc1, fc3) and H must be multiples of 16, as
  // tmh_weight_upload_qmoe makes them.
  if (n1 % 16 || H % 16)
    return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE needs multiples of 16 rows per expert; fc1 has %lld and fc2 %lld",
                (long long)n1, (long long)H);
  const bool two = activation == ACT_SWIGLU && swiglu_fusion == 0 && fc3;
  if (two && (fc3->N != fc1->N || fc3->K != fc1->K)) return fail(ctx, TMH_ERR_INVALID, "QMoE fc3 must match fc1");
  const int64_t inter = activation == ACT_SWIGLU && !two ? n1 / 2 : n1;
  if (activation == ACT_SWIGLU && !two && n1 % 2) return fail(ctx, TMH_ERR_INVALID, "QMoE swiglu needs an even fc1 width");
  if (fc2->K != inter)
    return fail(ctx, TMH_ERR_INVALID, "QMoE fc2 takes %lld inputs; the activation gives %lld", (long long)fc2->K, (long long)inter);
  if (fc1->wdtype != x_dtype || fc2->wdtype != x_dtype || (two && fc3->wdtype != x_dtype))
    return fail(ctx, TMH_ERR_INVALID, "QMoE weights must dequantize in the input's type (%s)", dtype_name(x_dtype));
  if (T == 0) return TMH_OK;
  if (!d_x || !d_router || !d_y) return fail(ctx, TMH_ERR_INVALID, "QMoE: NULL pointer");
  const int64_t tk = T * k;
  hipStream_t s = pick_stream(ctx, stream);
  const size_t es = static_cast<size_t>(dtype_size(x_dtype));
  // Rows per work item: 64 when experts average more than 24 rows and every product takes the
  // fast path (each expert's weights are then mostly read once), else 32.
  const int64_t inter_i = inter;
  const bool all_fast = moe_fast(fc1, x_dtype, d_x, static_cast<int>(T), static_cast<int>(H)) &&
                        (!two || moe_fast(fc3, x_dtype, d_x, static_cast<int>(T), static_cast<int>(H))) &&
                        fc2->wdtype == TMH_F16 && fc2->zp_kind != TMH_ZP_FLOAT && inter_i % 8 == 0 &&
                        tk * inter_i * 2 < (int64_t(1) << 31) && (fc2->ntiles + 1) * fc2->nchunks * 1024 < (int64_t(1) << 31);
  const int rows = all_fast && tk > 24 * E ? 64 : kMoeRows;
  const int max_items = static_cast<int>((tk + rows - 1) / rows + E);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  };
  const size_t o_counts = take(E * 4), o_offsets = take(E * 4), o_nitems = take(4);
  const size_t o_items = take(static_cast<size_t>(max_items) * 4), o_topi = take(tk * 4), o_topw = take(tk * 4);
  const size_t o_perm = take(tk * 4), o_slot = take(tk * 4);
  const size_t o_h1 = take(tk * n1 * es), o_h3 = two ? take(tk * n1 * es) : 0;
  const size_t o_act = take(tk * inter * es), o_o = take(tk * H * es);
  auto* ws = static_cast<uint8_t*>(workspace(ctx, off, s));
  if (!ws)
    return fail(ctx, TMH_ERR_UNSUPPORTED, "QMoE needs a %zu-byte workspace; run it once outside graph capture first", off);
  auto* counts = reinterpret_cast<int*>(ws + o_counts);
  auto* offsets = reinterpret_cast<int*>(ws + o_offsets);
  auto* n_items = reinterpret_cast<int*>(ws + o_nitems);
  auto* items = reinterpret_cast<int*>(ws + o_items);
  auto* topi = reinterpret_cast<int*>(ws + o_topi);
  auto* topw = reinterpret_cast<float*>(ws + o_topw);
  auto* perm = reinterpret_cast<int*>(ws + o_perm);
  auto* slot_pos = reinterpret_cast<int*>(ws + o_slot);
  void* h1 = ws + o_h1;
  void* h3 = two ? ws + o_h3 : nullptr;
  void* hact = ws + o_act;
  void* o = ws + o_o;
  const int ti = static_cast<int>(T), ki = k, ei = static_cast<int>(E), tki = static_cast<int>(tk);
  const unsigned route_grid = static_cast<unsigned>((T + 3) / 4);
  {
    // Router keys per lane: 2 up to 128 experts, 4 up to 256, 16 up to 1024.
    uint32_t* tl = timeline_slots(TMH_TL_MOE_ROUTE, static_cast<int64_t>(route_grid) * 4);
#define TMH_MOE_ROUTE_J(RDT, EJ)                                                                              \
  if (tl) k_moe_route_tl<RDT, EJ><<<route_grid, 256, 0, s>>>(d_router, ti, ei, ki, topi, topw, tl);             \
  else k_moe_route<RDT, EJ><<<route_grid, 256, 0, s>>>(d_router, ti, ei, ki, topi, topw)
#define TMH_MOE_ROUTE(RDT)                 \
  if (ei <= 128) TMH_MOE_ROUTE_J(RDT, 2);  \
  else if (ei <= 256) TMH_MOE_ROUTE_J(RDT, 4); \
  else TMH_MOE_ROUTE_J(RDT, 16)
    switch (router_dtype) {
      case TMH_F16: TMH_MOE_ROUTE(DT_F16); break;
      case TMH_BF16: TMH_MOE_ROUTE(DT_BF16); break;
      default: TMH_MOE_ROUTE(DT_F32);
    }
#undef TMH_MOE_ROUTE
#undef TMH_MOE_ROUTE_J
  }
  if (uint32_t* tl = timeline_slots(TMH_TL_MOE_PLAN, 16))
    k_moe_plan_tl<<<1, 1024, 0, s>>>(counts, ei, rows, topi, tki, offsets, items, n_items, perm, slot_pos, tl);
  else
    k_moe_plan<<<1, 1024, 0, s>>>(counts, ei, rows, topi, tki, offsets, items, n_items, perm, slot_pos);
  TMH_TRY(check_launch(ctx, "k_moe_plan"));
  const int hi = static_cast<int>(H), n1i = static_cast<int>(n1), inti = static_cast<int>(inter);
  // fc1 (and fc3) with the activation in the product's epilogue where the fast path allows it:
  // swiglu of fc1 and fc3 tiles, of the two halves of fc1, or an elementwise activation.
  // Interleaved swiglu pairs and the general path store the sums and activate separately.
  MoeEpilogue ep;
  ep.rows = rows;
  ep.bias1 = d_fc1_bias;
  ep.bias_dt = bias_dtype;
  ep.bias_ld = n1i;
  ep.act = activation;
  ep.alpha = alpha;
  ep.beta = beta;
  ep.limit = limit;
  // The fused swiglu product reads fc3's tiles with fc1's layout parameters (bits, parameter
  // entries per chunk, zero point kind); fc3 of another layout runs as its own product.
  const bool same_layout = !two || (fc3->bits == fc1->bits && fc3->nbc == fc1->nbc &&
                                    fc3->block_size == fc1->block_size && fc3->zp_kind == fc1->zp_kind &&
                                    fc3->nchunks == fc1->nchunks && fc3->ntiles == fc1->ntiles);
  const bool fused = moe_fast(fc1, x_dtype, d_x, ti, hi) && (!two || moe_fast(fc3, x_dtype, d_x, ti, hi)) &&
                     same_layout && (activation != ACT_SWIGLU || two || (swiglu_fusion == 2 && inter % 16 == 0));
  if (fused) {
    if (activation == ACT_SWIGLU) {
      ep.kind = EPI_GLU;
      ep.w2 = two ? fc3 : fc1;
      ep.bias2 = two ? d_fc3_bias : d_fc1_bias;
      ep.tile_off2 = two ? 0 : inti / 16;
      ep.out_tiles = inti / 16;
    } else {
      ep.kind = EPI_ACT;
    }
    moe_gemm(fc1, ei, d_x, x_dtype, ti, hi, perm, ki, items, n_items, max_items, offsets, counts, hact, inti, s, ep);
    TMH_TRY(check_launch(ctx, "k_moe_gemm (fc1)"));
  } else {
    moe_gemm(fc1, ei, d_x, x_dtype, ti, hi, perm, ki, items, n_items, max_items, offsets, counts, h1, n1i, s);
    if (two) moe_gemm(fc3, ei, d_x, x_dtype, ti, hi, perm, ki, items, n_items, max_items, offsets, counts, h3, n1i, s);
    TMH_TRY(check_launch(ctx, "k_moe_gemm (fc1)"));
    const int64_t act_n = tk * (activation == ACT_SWIGLU ? inter : n1);
    const unsigned act_grid = static_cast<unsigned>((act_n + 255) / 256);
#define TMH_MOE_ACT(DT)                                                                                                  \
  k_moe_activate<DT><<<act_grid, 256, 0, s>>>(h1, h3, n1i, inti, d_fc1_bias, two ? d_fc3_bias : nullptr, bias_dtype,    \
                                              perm, topi, tki, activation, swiglu_fusion, alpha, beta, limit, hact)
    switch (x_dtype) {
      case TMH_F16: TMH_MOE_ACT(DT_F16); break;
      case TMH_BF16: TMH_MOE_ACT(DT_BF16); break;
      default: TMH_MOE_ACT(DT_F32);
    }
#undef TMH_MOE_ACT
    TMH_TRY(check_launch(ctx, "k_moe_activate"));
  }
  // fc2 on the fast path writes each row at its (token, slot) index, so the final sum reads a
  // token's rows in one run; the general path keeps expert order.
  const bool fc2_fast = moe_fast(fc2, x_dtype, hact, tki, inti);
  MoeEpilogue ep2;
  ep2.rows = rows;
  ep2.out_perm = fc2_fast ? perm : nullptr;
  const int* o_rows = fc2_fast ? nullptr : slot_pos;
  moe_gemm(fc2, ei, hact, x_dtype, tki, inti, nullptr, 1, items, n_items, max_items, offsets, counts, o, hi, s, ep2);
  TMH_TRY(check_launch(ctx, "k_moe_gemm (fc2)"));
  // H is a multiple of 16: eight columns per thread.
  const unsigned out_grid = static_cast<unsigned>((T * H / 8 + 255) / 256);
  uint32_t* tl_sum = timeline_slots(TMH_TL_MOE_COMBINE, static_cast<int64_t>(out_grid) * 4);
  const bool y_vec = reinterpret_cast<uintptr_t>(d_y) % 16 == 0;
#define TMH_MOE_SUM(DT)                                                                                            \
  if (tl_sum)                                                                                                      \
    k_moe_combine_tl<DT, 8><<<out_grid, 256, 0, s>>>(o, hi, d_fc2_bias, bias_dtype, topi, topw, o_rows, ti, ki, d_y,   \
                                                    y_vec, tl_sum);                                                \
  else                                                                                                             \
    k_moe_combine<DT, 8><<<out_grid, 256, 0, s>>>(o, hi, d_fc2_bias, bias_dtype, topi, topw, o_rows, ti, ki, d_y, y_vec)
  switch (x_dtype) {
    case TMH_F16: TMH_MOE_SUM(DT_F16); break;
    case TMH_BF16: TMH_MOE_SUM(DT_BF16); break;
    default: TMH_MOE_SUM(DT_F32);
  }
#undef TMH_MOE_SUM
  return check_launch(ctx, "k_moe_combine");
}

}  // extern "C"
