// Internal declarations shared by the translation units of libtmhip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/transmuter_hip.h"

// Launch timeline of a context (measurement only, tmh_timeline_begin): the instrumented kernels
// write, per wavefront, the low 32 bits of the GPU's 100 MHz real-time counter and of its shader
// cycle counter at the wavefront's start and end into consecutive four-word slots of a caller's
// device buffer, and each launch is logged with its kernel and its first slot.
struct tmh_timeline_state {
  uint32_t* d_slots = nullptr;  // 4 words per wavefront
  int64_t capacity = 0, used = 0, dropped = 0;
  std::vector<int64_t> log;  // kernel id, first slot, wavefronts: three per launch
};

struct tmh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string error;
  int num_cus = 0;
  void* ws = nullptr;  // workspace of split-K partial sums, grown on demand outside capture
  size_t ws_bytes = 0;
  // Workspaces replaced by a larger one. A graph captured earlier keeps their addresses in its
  // kernel arguments, so they stay allocated until the context is destroyed.
  std::vector<void*> ws_retired;
  tmh_timeline_state* tl = nullptr;  // while a timeline is recorded
};

// Tiled device layout of a MatMulNBits weight.
//
// Rows are grouped in tiles of 16 (one MFMA column block); each row's packed bytes are cut in
// chunks of 64 bytes (CW = 512/bits weights). One (tile, chunk) holds 16 rows x 64 bytes =
// 1 KiB, stored so that lane l = 16*g + r of a wavefront loads 16 contiguous bytes at offset
// 16*l: row r of the tile, bytes 16*g .. 16*g+15 of the chunk. A wavefront's 16-byte load
// therefore reads 1 KiB contiguously, and lane l holds the MFMA B-operand data of column r
// for k-group g.
//
// Within each 32-bit word the sub-byte values are reordered so that value 2j sits at bits
// j*bits and value 2j+1 at bits 16 + j*bits: ((x >> j*bits) & mask16) is the pair
// (value 2j, value 2j+1), one per 16-bit half. 8-bit weights keep their byte order.
//
// Per (tile, chunk) the scales and zero points of the blocks each row touches are stored as
// params[tile][chunk][j][r], j < nbc = max(1, CW / block_size): block j of the chunk's row r.
// Packed zero points take `bits` bits per entry, entry e at bits (e % (8/bits)) * bits of byte
// e / (8/bits) (two a byte for 4-bit weights: rows 2i and 2i+1 of one block share a byte); float
// zero points are f32 per entry.
struct tmh_weight {
  int device = 0;
  int64_t K = 0, N = 0;
  int bits = 4, block_size = 32;
  int64_t blocks = 0;   // ceil(K / block_size)
  int64_t row_bytes = 0;  // blocks * block_size * bits / 8
  int64_t nchunks = 0;  // ceil(row_bytes / 64)
  int64_t ntiles = 0;   // ceil(N / 16)
  int nbc = 1;          // parameter entries per row per chunk
  int wdtype = TMH_F16; // dequantization type (F32, F16, BF16)
  int zp_kind = TMH_ZP_NONE;
  uint8_t* d_q = nullptr;   // ntiles*nchunks*1024 bytes
  void* d_scale = nullptr;  // ntiles*nchunks*nbc*16 values of wdtype
  void* d_zero = nullptr;   // packed zero points (bits each) or f32 float zero points, same entries
  size_t device_bytes = 0;
};

namespace tmh {

constexpr int kTileRows = 16;
constexpr int kChunkBytes = 64;

inline int chunk_weights(int bits) { return kChunkBytes * 8 / bits; }

inline int dtype_size(int dt) {
  switch (dt) {
    case TMH_F32: case TMH_S32: return 4;
    case TMH_F16: case TMH_BF16: case TMH_U16: case TMH_S16: return 2;
    case TMH_U8: case TMH_S8: return 1;
    case TMH_S64: return 8;
    default: return 0;
  }
}

inline bool is_float_dtype(int dt) { return dt == TMH_F32 || dt == TMH_F16 || dt == TMH_BF16; }

const char* dtype_name(int dt);

// Error bookkeeping: the message goes to the context, or to a thread-local slot.
int fail(tmh_ctx* ctx, int status, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int check_hip(tmh_ctx* ctx, hipError_t err, const char* what);
hipStream_t pick_stream(tmh_ctx* ctx, void* stream);
int use_device(tmh_ctx* ctx);
int check_launch(tmh_ctx* ctx, const char* kernel);
// The context's workspace of at least `bytes` bytes for work on `stream`, or nullptr when it
// would have to grow while the stream is being captured into a graph (or cannot grow).
void* workspace(tmh_ctx* ctx, size_t bytes, hipStream_t stream);

// Host conversions (round to nearest even).
float f16_to_f32(uint16_t h);
uint16_t f32_to_f16(float f);
float bf16_to_f32(uint16_t h);
uint16_t f32_to_bf16(float f);
float load_float(const void* p, int dt, size_t i);  // host read of a float array element

// The decode GEMV of tmh_gemv.hip (k_gemv_dec, k_gemv_dot): Y [M, N] f16 = A [M, K] f16 . W^T
// (+ an f16 bias [N], or none) for M <= 16, f16 weights, packed or no zero points. decode_gemv_ok
// tells whether it applies (alignment, 32-bit offsets); launch_decode_gemv picks the launch shape
// for the size and launches.
bool decode_gemv_ok(const tmh_weight* w, int64_t M, int64_t lda, int64_t ldy, const void* a, const void* y);
void launch_decode_gemv(const tmh_weight* w, const void* a, int64_t M, int64_t lda, void* y, int64_t ldy,
                        hipStream_t s, int num_cus, const void* bias = nullptr);
// The f32 decode GEMV (k_gemv_f32): f32 A and weights, f32 Y without bias, M <= 4.
bool decode_gemv_f32_ok(const tmh_weight* w, int64_t M, int64_t lda, int64_t ldy, const void* a);
void launch_decode_gemv_f32(const tmh_weight* w, const void* a, int64_t M, int64_t lda, void* y, int64_t ldy,
                            hipStream_t s);

// Looks up, once per device and with that device current, the device address of the scratch
// memory tmh_matmul_nbits_noalloc uses (a failure is reported by that call).
void noalloc_scratch_init(int device);

// Timeline recording. An entry point that launches instrumented kernels holds a TimelineScope
// for its context; a launcher asks timeline_slots for the slots of a launch of `waves`
// wavefronts and launches the stamping build of its kernel when it gets some (nullptr: no
// timeline is on, or its slots ran out and the launch goes unrecorded).
uint32_t* timeline_slots(int kernel, int64_t waves);
class TimelineScope {
 public:
  explicit TimelineScope(tmh_ctx* ctx);
  ~TimelineScope();
  TimelineScope(const TimelineScope&) = delete;
  TimelineScope& operator=(const TimelineScope&) = delete;

 private:
  tmh_timeline_state* prev_;
};

}  // namespace tmh

#define TMH_TRY(expr)          \
  do {                         \
    int _st = (expr);          \
    if (_st != TMH_OK) return _st; \
  } while (0)
