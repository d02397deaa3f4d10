// Measurement floors for the benchmark (no reference counterpart): an empty kernel, which is the
// cost of one launch in a stream or graph, and a plain read of a packed weight's bytes with the
// decode GEMV's load pattern (one 16-byte load per lane, 1 KiB per wavefront), which is what a
// kernel that only reads the weights once costs. Compiled, like the decode GEMV, with the
// leading kernel arguments preloaded into SGPRs.
#include "tmh_internal.h"
#include "tmh_device.h"

namespace {

__global__ __launch_bounds__(64) void k_floor_empty() {}

// Reads `kib` KiB; stores a word only if the bytes read xor to a marker (so the loads are not
// removed), which a caller's sink absorbs.
__global__ __launch_bounds__(256) void k_floor_read(const tmh::uint4_t* __restrict__ p, uint32_t kib,
                                                    uint32_t* __restrict__ sink) {
  const uint32_t wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= kib) return;
  const auto rs = tmh::buffer_rsrc(p, kib * 1024);
  const tmh::uint4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, (wv * 64 + (threadIdx.x & 63)) * 16, 0, 0);
  if ((v[0] ^ v[1] ^ v[2] ^ v[3]) == 0x9E3779B9u) sink[0] = wv;
}

}  // namespace

using namespace tmh;

extern "C" {

int tmh_floor_empty(tmh_ctx* ctx, int workgroups, void* stream) {
  TMH_TRY(use_device(ctx));
  if (workgroups < 1) return fail(ctx, TMH_ERR_INVALID, "tmh_floor_empty: workgroups must be positive");
  k_floor_empty<<<static_cast<unsigned>(workgroups), 64, 0, pick_stream(ctx, stream)>>>();
  return check_launch(ctx, "k_floor_empty");
}

int tmh_floor_read(tmh_ctx* ctx, const tmh_weight* w, void* d_sink, void* stream) {
  TMH_TRY(use_device(ctx));
  if (!w || !d_sink) return fail(ctx, TMH_ERR_INVALID, "tmh_floor_read: NULL argument");
  const int64_t kib = w->ntiles * w->nchunks;
  if (kib * 1024 >= (int64_t(1) << 32)) return fail(ctx, TMH_ERR_INVALID, "tmh_floor_read: the weight is too large");
  k_floor_read<<<static_cast<unsigned>((kib + 3) / 4), 256, 0, pick_stream(ctx, stream)>>>(
      reinterpret_cast<const uint4_t*>(w->d_q), static_cast<uint32_t>(kib), static_cast<uint32_t*>(d_sink));
  return check_launch(ctx, "k_floor_read");
}

}  // extern "C"
