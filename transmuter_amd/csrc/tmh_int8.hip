// MatMulInteger with a prepared B: B transposed once (for an initializer, at load) into s8 rows of
// k, its column sums and zero-point terms precomputed, so the GEMM streams both operands
// global -> LDS with buffer_load ... lds, three stages deep, and spends its VALU work only on the
// A flip and A's row sums. Reference: MatMulInteger (lib/transmuter/ops/quantized.ex:105-110),
// the exact integer sums of NN.integer_product/5 (lib/transmuter/ops/nn.ex:537-555).
//
// With sa = a - oa (oa = 128 for u8 A, whose bytes are flipped by ^ 0x80; 0 for s8) and
// sb = b - ob (likewise, applied when B is prepared):
//   sum_k (a - az_m)(b - bz_n) = sum_k sa sb + cb_n * rs_m + ca_m * cs_n + K * ca_m * cb_n (mod 2^32)
// with ca_m = oa - az_m, cb_n = ob - bz_n, rs_m = sum_k sa = (sum_k a) - oa K, cs_n = sum_k sb.
#include <algorithm>

#include "tmh_device.h"
#include "tmh_internal.h"

struct tmh_int8_weight {
  int device = 0;
  int64_t K = 0, Kp = 0, N = 0;  // Kp: K rounded up to a whole GEMM k-step
  int8_t* d_bt = nullptr;        // [N][Kp] s8, zero past K
  int32_t* d_cs = nullptr;       // [N] column sums of sb over k < K
  int32_t* d_cb = nullptr;       // [N] ob - bz_n
  size_t device_bytes = 0;
};

namespace tmh {
namespace {

constexpr int kQT = 128;   // output rows and columns per workgroup
constexpr int kQPad = 256;  // a prepared B's rows of k are padded to whole GEMM steps (of 128 or 256 bytes)

// B [K][N] (u8 or s8) -> Bt [N][Kp] as s8 (u8 flipped by ^ 0x80 = b - 128), zero past K. A
// workgroup moves one 128 (k) x 128 (n) tile: 16-byte loads along n (a wavefront reads eight whole
// 128-byte rows) into LDS rows of 132 bytes (the read-back below then meets at most two-way bank
// conflicts), the flip applied and rows past K zeroed on the way in; then each thread reads the 4
// columns x 16 rows it owns as sixteen 4-byte words, transposes them in 4 x 4 byte blocks
// (v_perm_b32) and stores four 16-byte pieces along k, so the eight threads of one output row
// write its 128 bytes whole.
constexpr int kTT = 128;    // tile edge, bytes of k and of n
constexpr int kTRow = 132;  // LDS bytes per tile row

__global__ __launch_bounds__(256) void k_i8_transpose(const uint8_t* __restrict__ b, uint32_t flip, uint32_t K, uint32_t N,
                                                      uint32_t Kp, bool vec, uint8_t* __restrict__ bt) {
  __shared__ __align__(16) uint32_t t[kTT * kTRow / 4];
  const uint32_t n0 = blockIdx.x * kTT, k0 = blockIdx.y * kTT;
  const int tid = threadIdx.x;
  const uint32_t flip4 = flip * 0x01010101u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = tid + 256 * i;
    const int row = p >> 3, piece = p & 7;
    const uint32_t k = k0 + row, n = n0 + 16 * piece;
    uint4_t v = uint4_t{0u, 0u, 0u, 0u};
    if (k < K) {
      if (vec) {
        if (n < N) v = *reinterpret_cast<const uint4_t*>(b + static_cast<size_t>(k) * N + n);
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (n + e < N) v[e >> 2] |= static_cast<uint32_t>(b[static_cast<size_t>(k) * N + n + e]) << (8 * (e & 3));
      }
      v ^= flip4;  // columns past N are flipped too; no thread stores them
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) t[row * (kTRow / 4) + 4 * piece + w] = v[w];
  }
  __syncthreads();
  const int kp = tid & 7, ng = tid >> 3;  // k bytes 16 kp .. +15, columns 4 ng .. +3
  uint32_t d[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) d[i] = t[(16 * kp + i) * (kTRow / 4) + ng];
  uint4_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // Rows 4q .. 4q+3 of the thread's 16: output word q of column j holds byte j of each.
    const uint32_t lo01 = __builtin_amdgcn_perm(d[4 * q + 1], d[4 * q], 0x05010400u);
    const uint32_t hi01 = __builtin_amdgcn_perm(d[4 * q + 1], d[4 * q], 0x07030602u);
    const uint32_t lo23 = __builtin_amdgcn_perm(d[4 * q + 3], d[4 * q + 2], 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(d[4 * q + 3], d[4 * q + 2], 0x07030602u);
    o[0][q] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
    o[1][q] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
    o[2][q] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
    o[3][q] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t n = n0 + 4 * ng + j;
    if (n < N) *reinterpret_cast<uint4_t*>(bt + static_cast<size_t>(n) * Kp + k0 + 16 * kp) = o[j];
  }
}

void launch_i8_transpose(const uint8_t* b, bool b_signed, int64_t K, int64_t N, int64_t Kp, uint8_t* bt, hipStream_t s) {
  const bool vec = N % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0;
  const dim3 grid(static_cast<unsigned>((N + kTT - 1) / kTT), static_cast<unsigned>(Kp / kTT));
  k_i8_transpose<<<grid, 256, 0, s>>>(b, b_signed ? 0u : 0x80u, static_cast<uint32_t>(K), static_cast<uint32_t>(N),
                                      static_cast<uint32_t>(Kp), vec, bt);
}

// cs_n = sum_k sb (over Bt's row n: zeros past K add nothing) and cb_n = ob - bz_n; one
// wavefront per row, lanes over its 4-byte words, a shuffle reduction.
__global__ __launch_bounds__(256) void k_i8_colsum(const uint32_t* __restrict__ bt, int64_t Kp, int64_t N,
                                                   const uint8_t* __restrict__ b_zero, int64_t b_zero_count,
                                                   bool b_signed, int32_t* __restrict__ cs, int32_t* __restrict__ cb) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  int32_t s = 0;
  const uint32_t* row = bt + n * (Kp / 4);
  for (int64_t i = lane; i < Kp / 4; i += 64) s = __builtin_amdgcn_sdot4(static_cast<int>(row[i]), 0x01010101, s, false);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane != 0) return;
  cs[n] = s;
  int32_t bz = 0;
  if (b_zero) {
    const uint8_t raw = b_zero[b_zero_count == 1 ? 0 : n];
    bz = b_signed ? static_cast<int32_t>(static_cast<int8_t>(raw)) : static_cast<int32_t>(raw);
  }
  cb[n] = (b_signed ? 0 : 128) - bz;
}

// At most n vector-memory operations of this thread outstanding (n a multiple of 4, up to 12).
__device__ __forceinline__ void wait_vm(uint32_t n) {
  if (n >= 12)
    __builtin_amdgcn_s_waitcnt(12 | (7 << 4) | (15 << 8));
  else if (n >= 8)
    __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8));
  else if (n >= 4)
    __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (15 << 8));
  else
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
}

// 128 x 128 outputs per workgroup of eight wavefronts: wavefront w computes the 64 x 64 quadrant
// w & 3 over k-half w >> 2 of every step (4 x 4 tiles of v_mfma_i32_16x16x64_i8, B fragments first
// so a lane ends with 4 consecutive columns of one row); the halves add through LDS at the end.
// Each step's A rows and Bt rows (KQ bytes of k) go global -> LDS by buffer_load ... lds, 16 bytes
// per lane into rows whose 16-byte pieces are XOR-swizzled by row (frag_swizzle: conflict-free
// fragment reads; a lane loads the global piece that belongs in its slot), issued STAGES - 1 steps
// ahead into a ring of STAGES stages, so one barrier per step both publishes step s and frees the
// stage that the next issue overwrites.
// A: rows past M lie past the buffer range and read zeros (their outputs are not stored), pieces
// past K are pointed past it too (K is a multiple of 16). The raw bytes of A are summed per row
// (v_dot4_u32_u8; v_dot4_i32_i8 for s8 A) as the fragments are read, by the wavefronts of the left
// quadrants.
template <bool A_SIGNED, int KQ, int STAGES, int NW = 8>
__global__ __launch_bounds__(64 * NW) void k_mmi_bt(const uint8_t* __restrict__ a,
                                                const int8_t* __restrict__ bt, const int32_t* __restrict__ cs,
                                                const int32_t* __restrict__ cb, const uint8_t* __restrict__ a_zero,
                                                int64_t a_zero_count, uint32_t M, uint32_t K, uint32_t Kp, uint32_t N,
                                                int32_t* __restrict__ y, bool y_vec) {
  constexpr int PPR = KQ / 16;                  // 16-byte pieces per LDS row
  constexpr int RPI = 64 / PPR;                 // rows one wavefront's DMA instruction fills
  constexpr int KS = NW / 4;                    // wavefronts sharing a quadrant, each a k-part of a step
  constexpr int DMA = kQT / RPI / NW;           // DMA instructions per wavefront per operand and step
  constexpr int STAGE = 2 * kQT * KQ;           // bytes of one stage (A and B tiles)
  constexpr int SUB = KQ / KS / 64;             // MFMA k-steps of 64 in a wavefront's k-part
  static_assert(DMA >= 1 && SUB >= 1, "step shape");
  constexpr uint32_t aflip = A_SIGNED ? 0u : 0x80808080u;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int quad = wave & 3, wm = quad >> 1, wn = quad & 1, kh = wave >> 2;
  const int r = lane & 15, g = lane >> 4;
  // Workgroups go to the eight XCDs round-robin by linear id; with a tile count that is a multiple
  // of 8, XCD x takes tiles [x T/8, (x+1) T/8) of an order that walks groups of four m-tiles
  // m-fastest, so one XCD's tiles share few A rows and B columns (its own L2).
  uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
  const uint32_t tiles = gridDim.x * gridDim.y;
  if (tiles % 8 == 0) tile = (tile % 8) * (tiles / 8) + tile / 8;
  const uint32_t group = tile / (4 * gridDim.x), first_m = 4 * group;
  const uint32_t group_m = min(4u, gridDim.y - first_m), in_group = tile - group * 4 * gridDim.x;
  const uint32_t m0 = (first_m + in_group % group_m) * kQT;
  const uint32_t n0 = (in_group / group_m) * kQT;
  const uint8_t* a8 = a + static_cast<int64_t>(blockIdx.z) * M * K;
  const auto a_rsrc = buffer_rsrc(a8, M * K);
  const auto b_rsrc = buffer_rsrc(bt, N * Kp);
  // This lane's DMA rows (RPI-row groups DMA * w + j) and the global piece its slot holds.
  uint32_t a_off[DMA], b_off[DMA], gpc[DMA];
#pragma unroll
  for (int j = 0; j < DMA; ++j) {
    const int row = RPI * (DMA * wave + j) + lane / PPR;
    gpc[j] = static_cast<uint32_t>((lane % PPR) ^ frag_swizzle<PPR>(row));
    a_off[j] = (m0 + row) * K + gpc[j] * 16;
    b_off[j] = (n0 + row) * Kp + gpc[j] * 16;
  }
  const uint32_t steps = Kp / KQ;
  auto issue = [&](uint32_t s) {
    uint8_t* sa = lds + (s % STAGES) * STAGE;
    uint8_t* sb = sa + kQT * KQ;
    const uint32_t k0 = s * KQ;
#pragma unroll
    for (int j = 0; j < DMA; ++j) {
      const int row0 = RPI * (DMA * wave + j);
      lds_dma16(a_rsrc, sa + row0 * KQ, k0 + gpc[j] * 16 < K ? a_off[j] + k0 : 0x80000000u, 0);
      lds_dma16(b_rsrc, sb + row0 * KQ, b_off[j] + k0, 0);
    }
  };
  int4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = int4_t{0, 0, 0, 0};
  uint32_t raw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p)
    if (static_cast<uint32_t>(p) < steps) issue(p);
  for (uint32_t s = 0; s < steps; ++s) {
    // This thread's DMAs of step s are done when at most those of the later steps already issued
    // (2 DMA per step) are in flight.
    wait_vm(2 * DMA * min(steps - 1 - s, static_cast<uint32_t>(STAGES - 2)));
    // A bare barrier: __syncthreads' fence would also wait for the later steps' loads. The empty
    // asm statements keep the compiler from moving memory accesses across it; the waits above and
    // the LDS reads of step s - 1, complete before its MFMAs, make it a full barrier for this ring.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (s + STAGES - 1 < steps) issue(s + STAGES - 1);
    const uint8_t* sa = lds + (s % STAGES) * STAGE;
    const uint8_t* sb = sa + kQT * KQ;
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      const int c = kh * (PPR / KS) + 4 * u + g;  // this lane's 16-byte piece of the step's KQ bytes
      int4_t af[4], bf[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = 64 * wm + 16 * mt + r;
        const uint4_t v = *reinterpret_cast<const uint4_t*>(sa + row * KQ + ((c ^ frag_swizzle<PPR>(row)) << 4));
        if (wn == 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            raw[mt] = A_SIGNED ? static_cast<uint32_t>(__builtin_amdgcn_sdot4(static_cast<int>(v[e]), 0x01010101,
                                                                              static_cast<int>(raw[mt]), false))
                               : __builtin_amdgcn_udot4(v[e], 0x01010101u, raw[mt], false);
        }
        af[mt] = __builtin_bit_cast(int4_t, v ^ aflip);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int row = 64 * wn + 16 * nt + r;
        bf[nt] = *reinterpret_cast<const int4_t*>(sb + row * KQ + ((c ^ frag_swizzle<PPR>(row)) << 4));
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[nt], af[mt], acc[mt][nt], 0, 0, 0);
    }
  }
  __syncthreads();  // every stage read: the LDS takes the other k-parts' sums
  // The k-parts of a quadrant add in a tree through LDS slots of 64 KiB (parts KS/2.. into
  // 0.., then ...), and A's row sums per part go to rs_part[part][row].
  constexpr int SLOT = 4 * 16 * 64;  // int4 entries of one slot: 4 quadrants x 16 tiles x 64 lanes
  auto* part = reinterpret_cast<int4_t*>(lds);
  auto* rs_part = reinterpret_cast<uint32_t*>(lds + (KS / 2) * SLOT * 16);
  if (wn == 0) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      uint32_t v = raw[mt];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (g == 0) rs_part[kh * kQT + 64 * wm + 16 * mt + r] = v;
    }
  }
  if constexpr (KS == 1) __syncthreads();  // the row sums, read across quadrants below
#pragma unroll
  for (int half = KS / 2; half >= 1; half /= 2) {
    if (kh >= half && kh < 2 * half) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) part[(kh - half) * SLOT + ((quad * 4 + mt) * 4 + nt) * 64 + lane] = acc[mt][nt];
    }
    __syncthreads();
    if (kh < half) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] += part[kh * SLOT + ((quad * 4 + mt) * 4 + nt) * 64 + lane];
    }
    __syncthreads();
  }
  if (kh != 0) return;
  const uint32_t oa = A_SIGNED ? 0u : 128u;
  constexpr bool a_signed = A_SIGNED;
  // The column terms of this lane's 4 x 4 columns, one 16-byte load each (the arrays are padded to
  // whole groups of 4; groups past N read zeros).
  const uint32_t terms = (N + 3) / 4 * 16;
  const auto cb_rsrc = buffer_rsrc(cb, terms), cs_rsrc = buffer_rsrc(cs, terms);
  int4_t cbv[4], csv[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const uint32_t n = n0 + 64 * wn + 16 * nt + 4 * g;
    cbv[nt] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(cb_rsrc, n * 4, 0, 0));
    csv[nt] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(cs_rsrc, n * 4, 0, 0));
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int ml = 64 * wm + 16 * mt + r;
    const uint32_t m = m0 + ml;
    if (m >= M) continue;
    uint32_t az = 0u;
    if (a_zero) {
      const uint8_t zr = a_zero[a_zero_count == 1 ? 0 : m];
      az = a_signed ? static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(zr))) : zr;
    }
    const uint32_t ca = oa - az;
    uint32_t rs = 0u - oa * K;
#pragma unroll
    for (int p = 0; p < KS; ++p) rs += rs_part[p * kQT + ml];
    int32_t* yrow = y + (static_cast<int64_t>(blockIdx.z) * M + m) * N;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const uint32_t n = n0 + 64 * wn + 16 * nt + 4 * g;
      if (n >= N) continue;
      const int4_t v = acc[mt][nt];
      int4_t out;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t cbn = static_cast<uint32_t>(cbv[nt][e]), csn = static_cast<uint32_t>(csv[nt][e]);
        out[e] = static_cast<int32_t>(static_cast<uint32_t>(v[e]) + cbn * rs + ca * csn + K * ca * cbn);
      }
      if (y_vec) {
        // Non-temporal: the s32 output (four bytes per product) is not read again here (2048^3: 20.7 -> 19.1 us under the tracer).
        __builtin_nontemporal_store(out, reinterpret_cast<int4_t*>(yrow + n));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) yrow[n + e] = out[e];
      }
    }
  }
}

}  // namespace
}  // namespace tmh

using namespace tmh;

extern "C" {

int tmh_int8_weight_prepare(tmh_ctx* ctx, const void* d_b, int b_dtype, const void* d_b_zero, int64_t b_zero_count,
                            int64_t K, int64_t N, void* stream, tmh_int8_weight** out) {
  if (!out) return fail(ctx, TMH_ERR_INVALID, "tmh_int8_weight_prepare: out is NULL");
  *out = nullptr;
  TMH_TRY(use_device(ctx));
  if (b_dtype != TMH_U8 && b_dtype != TMH_S8)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger takes u8 or s8 values, got %s", dtype_name(b_dtype));
  if (K < 1 || N < 1) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger B must have K, N >= 1");
  if (!d_b) return fail(ctx, TMH_ERR_INVALID, "tmh_int8_weight_prepare: B is NULL");
  if (d_b_zero && b_zero_count != 1 && b_zero_count != N)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger b_zero_point holds %lld values; 1 or N=%lld expected",
                (long long)b_zero_count, (long long)N);
  const int64_t Kp = (K + kQPad - 1) / kQPad * kQPad;
  if ((N + kQT) * Kp >= (int64_t{1} << 31) || K % 16 != 0)
    return fail(ctx, TMH_ERR_UNSUPPORTED,
                "a prepared MatMulInteger B needs K a multiple of 16 and (N + 128) * (K padded to 256) below 2^31");
  auto* w = new tmh_int8_weight();
  w->device = ctx->device;
  w->K = K;
  w->Kp = Kp;
  w->N = N;
  // The column terms are padded to whole 16-byte groups, which the GEMM loads whole.
  const size_t terms = static_cast<size_t>((N + 3) / 4 * 4) * 4;
  int st = check_hip(ctx, hipMalloc(reinterpret_cast<void**>(&w->d_bt), static_cast<size_t>(N * Kp)), "hipMalloc");
  if (st == TMH_OK) st = check_hip(ctx, hipMalloc(reinterpret_cast<void**>(&w->d_cs), terms), "hipMalloc");
  if (st == TMH_OK) st = check_hip(ctx, hipMalloc(reinterpret_cast<void**>(&w->d_cb), terms), "hipMalloc");
  if (st != TMH_OK) {
    tmh_int8_weight_free(w);
    return st;
  }
  w->device_bytes = static_cast<size_t>(N * Kp) + 2 * terms;
  hipStream_t s = pick_stream(ctx, stream);
  launch_i8_transpose(static_cast<const uint8_t*>(d_b), b_dtype == TMH_S8, K, N, Kp, reinterpret_cast<uint8_t*>(w->d_bt), s);
  st = check_launch(ctx, "k_i8_transpose");
  if (st == TMH_OK) {
    k_i8_colsum<<<static_cast<unsigned>((N + 3) / 4), 256, 0, s>>>(
        reinterpret_cast<const uint32_t*>(w->d_bt), Kp, N, static_cast<const uint8_t*>(d_b_zero), b_zero_count,
        b_dtype == TMH_S8, w->d_cs, w->d_cb);
    st = check_launch(ctx, "k_i8_colsum");
  }
  if (st != TMH_OK) {
    tmh_int8_weight_free(w);
    return st;
  }
  *out = w;
  return TMH_OK;
}

void tmh_int8_weight_free(tmh_int8_weight* w) {
  if (!w) return;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(w->device);
  (void)hipFree(w->d_bt);
  (void)hipFree(w->d_cs);
  (void)hipFree(w->d_cb);
  (void)hipSetDevice(prev);
  delete w;
}

int tmh_int8_weight_info(const tmh_int8_weight* w, int64_t* K, int64_t* N, size_t* device_bytes) {
  if (!w) return fail(nullptr, TMH_ERR_INVALID, "tmh_int8_weight_info: the weight is NULL");
  if (K) *K = w->K;
  if (N) *N = w->N;
  if (device_bytes) *device_bytes = w->device_bytes;
  return TMH_OK;
}

int tmh_matmul_integer_prepared(tmh_ctx* ctx, const void* d_a, int a_dtype, const void* d_a_zero, int64_t a_zero_count,
                                int64_t batch, int64_t M, const tmh_int8_weight* w, void* d_y, void* stream) {
  TMH_TRY(use_device(ctx));
  if (!w) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger: the prepared B is NULL");
  if (w->device != ctx->device)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger: B was prepared on device %d, the context uses %d", w->device,
                ctx->device);
  if (a_dtype != TMH_U8 && a_dtype != TMH_S8)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger takes u8 or s8 values, got %s", dtype_name(a_dtype));
  if (batch < 0 || M < 0) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger sizes must not be negative");
  if (d_a_zero && a_zero_count != 1 && a_zero_count != M)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger a_zero_point holds %lld values; 1 or M=%lld expected",
                (long long)a_zero_count, (long long)M);
  if (batch == 0 || M == 0) return TMH_OK;
  if (!d_a || !d_y) return fail(ctx, TMH_ERR_INVALID, "MatMulInteger: NULL pointer");
  if (batch > 65535 || (M + kQT - 1) / kQT > 65535)
    return fail(ctx, TMH_ERR_INVALID, "MatMulInteger: batch %lld or M %lld too large", (long long)batch, (long long)M);
  if ((M + kQT) * w->K >= (int64_t{1} << 31) || reinterpret_cast<uintptr_t>(d_a) % 16 != 0)
    return fail(ctx, TMH_ERR_UNSUPPORTED, "MatMulInteger with a prepared B needs a 16-byte aligned A of (M + 128) * K "
                                          "below 2^31 bytes");
  hipStream_t s = pick_stream(ctx, stream);
  const dim3 grid(static_cast<unsigned>((w->N + kQT - 1) / kQT), static_cast<unsigned>((M + kQT - 1) / kQT),
                  static_cast<unsigned>(batch));
  const bool y_vec = w->N % 4 == 0 && reinterpret_cast<uintptr_t>(d_y) % 16 == 0;
  // 256-byte k-steps in two stages, eight wavefronts: 20.5 us at 2048^3 u8 x u8 (840 TOP/s)
  // against 21.0 us for 128-byte steps in three stages, 22.0 in four, and 20.7 with sixteen
  // wavefronts; the unprepared kernel takes 28.5 us.
  constexpr int kLds = 2 * 2 * kQT * 256;
  auto* kernel = a_dtype == TMH_S8 ? k_mmi_bt<true, 256, 2> : k_mmi_bt<false, 256, 2>;
  static const hipError_t attr[2] = {
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_mmi_bt<true, 256, 2>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kLds),
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_mmi_bt<false, 256, 2>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kLds)};
  (void)attr;
  kernel<<<grid, 512, kLds, s>>>(static_cast<const uint8_t*>(d_a), w->d_bt, w->d_cs, w->d_cb,
                                 static_cast<const uint8_t*>(d_a_zero), a_zero_count, static_cast<uint32_t>(M),
                                 static_cast<uint32_t>(w->K), static_cast<uint32_t>(w->Kp), static_cast<uint32_t>(w->N),
                                 static_cast<int32_t*>(d_y), y_vec);
  return check_launch(ctx, "k_mmi_bt");
}

}  // extern "C"
