// Measurement floors for the benchmark (no reference counterpart): an empty kernel, which is the
// cost of one launch in a stream or graph, and a plain read of a packed weight's bytes with the
// decode GEMV's load pattern (one 16-byte load per lane, 1 KiB per wavefront), which is what a
// kernel that only reads the weights once costs. Compiled, like the decode GEMV, with the
// leading kernel arguments preloaded into SGPRs.
#include "tmh_internal.h"
#include "tmh_device.h"

namespace {

__global__ __launch_bounds__(64) void k_floor_empty() {}

// The stamping build (timeline): the same empty launch, each wavefront writing its stamps.
__global__ __launch_bounds__(64) void k_floor_empty_tl(uint32_t* __restrict__ tl) {
  tmh::tl_stamp(tl, tmh::tl_clock());
}

// Reads `kib` KiB; stores a word only if the bytes read xor to a marker (so the loads are not
// removed), which a caller's sink absorbs.
template <bool TL>
__device__ __forceinline__ void floor_read(const tmh::uint4_t* __restrict__ p, uint32_t kib, uint32_t* __restrict__ sink,
                                           uint32_t* __restrict__ tl) {
  const tmh::TlStart tl0 = TL ? tmh::tl_clock() : tmh::TlStart{0u, 0u};
  const uint32_t wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv < kib) {
    const auto rs = tmh::buffer_rsrc(p, kib * 1024);
    const tmh::uint4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, (wv * 64 + (threadIdx.x & 63)) * 16, 0, 0);
    if ((v[0] ^ v[1] ^ v[2] ^ v[3]) == 0x9E3779B9u) sink[0] = wv;
  }
  if constexpr (TL) tmh::tl_stamp(tl, tl0);
}

__global__ __launch_bounds__(256) void k_floor_read(const tmh::uint4_t* __restrict__ p, uint32_t kib,
                                                    uint32_t* __restrict__ sink) {
  floor_read<false>(p, kib, sink, nullptr);
}

__global__ __launch_bounds__(256) void k_floor_read_tl(const tmh::uint4_t* __restrict__ p, uint32_t kib,
                                                       uint32_t* __restrict__ sink, uint32_t* __restrict__ tl) {
  floor_read<true>(p, kib, sink, tl);
}

// Reads every byte of a weight once, 16 bytes per lane: its packed weights (n0 pieces), then its
// scales (n1) and its zero points (n2), as one range of pieces; stores like k_floor_read.
template <bool TL>
__device__ __forceinline__ void floor_read_all(const tmh::uint4_t* __restrict__ q, uint32_t n0,
                                               const tmh::uint4_t* __restrict__ s, uint32_t n1,
                                               const tmh::uint4_t* __restrict__ z, uint32_t n2,
                                               uint32_t* __restrict__ sink, uint32_t* __restrict__ tl) {
  const tmh::TlStart tl0 = TL ? tmh::tl_clock() : tmh::TlStart{0u, 0u};
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  tmh::uint4_t v{0u, 0u, 0u, 0u};
  if (i < n0) {
    v = __builtin_amdgcn_raw_buffer_load_b128(tmh::buffer_rsrc(q, n0 * 16), i * 16, 0, 0);
  } else if (i < n0 + n1) {
    v = __builtin_amdgcn_raw_buffer_load_b128(tmh::buffer_rsrc(s, n1 * 16), (i - n0) * 16, 0, 0);
  } else if (i < n0 + n1 + n2) {
    v = __builtin_amdgcn_raw_buffer_load_b128(tmh::buffer_rsrc(z, n2 * 16), (i - n0 - n1) * 16, 0, 0);
  }
  if ((v[0] ^ v[1] ^ v[2] ^ v[3]) == 0x9E3779B9u) sink[0] = i;
  if constexpr (TL) tmh::tl_stamp(tl, tl0);
}

__global__ __launch_bounds__(256) void k_floor_read_all(const tmh::uint4_t* __restrict__ q, uint32_t n0,
                                                        const tmh::uint4_t* __restrict__ s, uint32_t n1,
                                                        const tmh::uint4_t* __restrict__ z, uint32_t n2,
                                                        uint32_t* __restrict__ sink) {
  floor_read_all<false>(q, n0, s, n1, z, n2, sink, nullptr);
}

__global__ __launch_bounds__(256) void k_floor_read_all_tl(const tmh::uint4_t* __restrict__ q, uint32_t n0,
                                                           const tmh::uint4_t* __restrict__ s, uint32_t n1,
                                                           const tmh::uint4_t* __restrict__ z, uint32_t n2,
                                                           uint32_t* __restrict__ sink, uint32_t* __restrict__ tl) {
  floor_read_all<true>(q, n0, s, n1, z, n2, sink, tl);
}

// Writes zeros over `pieces` 16-byte pieces of dst with non-temporal stores, four per wavefront
// and 1 KiB contiguous per instruction: the store pattern of the vocabulary gather
// (k_gather_bq_rows) without its loads.
template <bool TL>
__device__ __forceinline__ void floor_write(tmh::uint4_t* __restrict__ dst, uint32_t pieces, uint32_t* __restrict__ tl) {
  const tmh::TlStart tl0 = TL ? tmh::tl_clock() : tmh::TlStart{0u, 0u};
  const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const auto rs = tmh::buffer_rsrc(dst, pieces * 16);
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t piece = (wave * 4 + j) * 64 + lane;  // past the range: dropped
    __builtin_amdgcn_raw_buffer_store_b128(tmh::uint4_t{0u, 0u, 0u, 0u}, rs, piece * 16, 0, tmh::kNonTemporal);
  }
  if constexpr (TL) tmh::tl_stamp(tl, tl0);
}

__global__ __launch_bounds__(256) void k_floor_write(tmh::uint4_t* __restrict__ dst, uint32_t pieces) {
  floor_write<false>(dst, pieces, nullptr);
}

__global__ __launch_bounds__(256) void k_floor_write_tl(tmh::uint4_t* __restrict__ dst, uint32_t pieces,
                                                        uint32_t* __restrict__ tl) {
  floor_write<true>(dst, pieces, tl);
}

}  // namespace

using namespace tmh;

extern "C" {

int tmh_floor_empty(tmh_ctx* ctx, int workgroups, void* stream) {
  TimelineScope timeline(ctx);
  TMH_TRY(use_device(ctx));
  if (workgroups < 1) return fail(ctx, TMH_ERR_INVALID, "tmh_floor_empty: workgroups must be positive");
  if (uint32_t* tl = timeline_slots(TMH_TL_FLOOR_EMPTY, workgroups))
    k_floor_empty_tl<<<static_cast<unsigned>(workgroups), 64, 0, pick_stream(ctx, stream)>>>(tl);
  else
    k_floor_empty<<<static_cast<unsigned>(workgroups), 64, 0, pick_stream(ctx, stream)>>>();
  return check_launch(ctx, "k_floor_empty");
}

int tmh_floor_read(tmh_ctx* ctx, const tmh_weight* w, void* d_sink, void* stream) {
  TimelineScope timeline(ctx);
  TMH_TRY(use_device(ctx));
  if (!w || !d_sink) return fail(ctx, TMH_ERR_INVALID, "tmh_floor_read: NULL argument");
  const int64_t kib = w->ntiles * w->nchunks;
  if (kib * 1024 >= (int64_t(1) << 32)) return fail(ctx, TMH_ERR_INVALID, "tmh_floor_read: the weight is too large");
  const unsigned grid = static_cast<unsigned>((kib + 3) / 4);
  if (uint32_t* tl = timeline_slots(TMH_TL_FLOOR_READ, static_cast<int64_t>(grid) * 4))
    k_floor_read_tl<<<grid, 256, 0, pick_stream(ctx, stream)>>>(
        reinterpret_cast<const uint4_t*>(w->d_q), static_cast<uint32_t>(kib), static_cast<uint32_t*>(d_sink), tl);
  else
    k_floor_read<<<grid, 256, 0, pick_stream(ctx, stream)>>>(
        reinterpret_cast<const uint4_t*>(w->d_q), static_cast<uint32_t>(kib), static_cast<uint32_t*>(d_sink));
  return check_launch(ctx, "k_floor_read");
}

int tmh_floor_read_all(tmh_ctx* ctx, const tmh_weight* w, void* d_sink, void* stream) {
  TimelineScope timeline(ctx);
  TMH_TRY(use_device(ctx));
  if (!w || !d_sink) return fail(ctx, TMH_ERR_INVALID, "tmh_floor_read_all: NULL argument");
  // The stored layout: 1 KiB per (tile, chunk) of weights; nbc * 16 parameter entries per (tile,
  // chunk), each a scale of the weight type and a zero point (`bits` bits packed, or f32 for float
  // zero points).
  const int64_t entries = w->ntiles * w->nchunks * w->nbc * 16;
  const int64_t n0 = w->ntiles * w->nchunks * 64;
  const int64_t n1 = entries * dtype_size(w->wdtype) / 16;
  const int64_t n2 = w->zp_kind == TMH_ZP_PACKED ? entries * w->bits / 8 / 16 : (w->zp_kind == TMH_ZP_FLOAT ? entries * 4 / 16 : 0);
  if ((n0 + n1 + n2) * 16 >= (int64_t(1) << 32))
    return fail(ctx, TMH_ERR_INVALID, "tmh_floor_read_all: the weight is too large");
  const unsigned grid = static_cast<unsigned>((n0 + n1 + n2 + 255) / 256);
  const auto* q = reinterpret_cast<const uint4_t*>(w->d_q);
  const auto* s = static_cast<const uint4_t*>(w->d_scale);
  const auto* z = static_cast<const uint4_t*>(w->d_zero);
  if (uint32_t* tl = timeline_slots(TMH_TL_FLOOR_READ_ALL, static_cast<int64_t>(grid) * 4))
    k_floor_read_all_tl<<<grid, 256, 0, pick_stream(ctx, stream)>>>(
        q, static_cast<uint32_t>(n0), s, static_cast<uint32_t>(n1), z, static_cast<uint32_t>(n2),
        static_cast<uint32_t*>(d_sink), tl);
  else
    k_floor_read_all<<<grid, 256, 0, pick_stream(ctx, stream)>>>(q, static_cast<uint32_t>(n0), s,
                                                                   static_cast<uint32_t>(n1), z,
                                                                   static_cast<uint32_t>(n2),
                                                                   static_cast<uint32_t*>(d_sink));
  return check_launch(ctx, "k_floor_read_all");
}

int tmh_floor_write(tmh_ctx* ctx, void* d_dst, size_t bytes, void* stream) {
  TimelineScope timeline(ctx);
  TMH_TRY(use_device(ctx));
  if (!d_dst || bytes == 0 || bytes % 16 != 0 || bytes >= (size_t(1) << 32))
    return fail(ctx, TMH_ERR_INVALID, "tmh_floor_write: a buffer of whole 16-byte pieces below 4 GiB is needed");
  const uint32_t pieces = static_cast<uint32_t>(bytes / 16);
  const unsigned grid = static_cast<unsigned>((pieces + 1023) / 1024);  // 4 KiB per wavefront, four per workgroup
  if (uint32_t* tl = timeline_slots(TMH_TL_FLOOR_WRITE, static_cast<int64_t>(grid) * 4))
    k_floor_write_tl<<<grid, 256, 0, pick_stream(ctx, stream)>>>(static_cast<uint4_t*>(d_dst), pieces, tl);
  else
    k_floor_write<<<grid, 256, 0, pick_stream(ctx, stream)>>>(static_cast<uint4_t*>(d_dst), pieces);
  return check_launch(ctx, "k_floor_write");
}

}  // extern "C"
