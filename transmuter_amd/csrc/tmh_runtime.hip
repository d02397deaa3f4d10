// Context, memory, events, graphs and error reporting of the C ABI.
#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include "tmh_internal.h"

namespace tmh {

static thread_local std::string g_thread_error;

const char* dtype_name(int dt) {
  switch (dt) {
    case TMH_F32: return "f32";
    case TMH_F16: return "f16";
    case TMH_BF16: return "bf16";
    case TMH_U8: return "u8";
    case TMH_S8: return "s8";
    case TMH_U16: return "u16";
    case TMH_S16: return "s16";
    case TMH_S32: return "s32";
    case TMH_S64: return "s64";
    default: return "unknown type";
  }
}

int fail(tmh_ctx* ctx, int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->error = buf;
  g_thread_error = buf;
  return status;
}

int check_hip(tmh_ctx* ctx, hipError_t err, const char* what) {
  if (err == hipSuccess) return TMH_OK;
  const int status = err == hipErrorOutOfMemory ? TMH_ERR_OOM : TMH_ERR_DEVICE;
  return fail(ctx, status, "%s: %s", what, hipGetErrorString(err));
}

int use_device(tmh_ctx* ctx) {
  if (!ctx) return fail(nullptr, TMH_ERR_INVALID, "the context is NULL");
  return check_hip(ctx, hipSetDevice(ctx->device), "hipSetDevice");
}

hipStream_t pick_stream(tmh_ctx* ctx, void* stream) {
  return stream ? static_cast<hipStream_t>(stream) : ctx->stream;
}

int check_launch(tmh_ctx* ctx, const char* kernel) {
  return check_hip(ctx, hipGetLastError(), kernel);
}

void* workspace(tmh_ctx* ctx, size_t bytes, hipStream_t stream) {
  if (ctx->ws_bytes >= bytes) return ctx->ws;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &status) != hipSuccess || status != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;
  }
  // The old workspace is not freed: queued work and graphs captured earlier may still use it.
  // It is retired until tmh_ctx_destroy, and the new one at least doubles, so the retired
  // buffers together stay below the size of the current one.
  size_t size = std::max(bytes, 2 * ctx->ws_bytes);
  void* p = nullptr;
  if (hipMalloc(&p, size) != hipSuccess) {
    (void)hipGetLastError();
    size = bytes;
    if (hipMalloc(&p, size) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
  }
  if (ctx->ws) ctx->ws_retired.push_back(ctx->ws);
  ctx->ws = p;
  ctx->ws_bytes = size;
  return p;
}

float f16_to_f32(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

float bf16_to_f32(uint16_t h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

float load_float(const void* p, int dt, size_t i) {
  switch (dt) {
    case TMH_F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case TMH_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    default: return static_cast<const float*>(p)[i];
  }
}

namespace {
thread_local tmh_timeline_state* t_timeline = nullptr;
}  // namespace

TimelineScope::TimelineScope(tmh_ctx* ctx) : prev_(t_timeline) { t_timeline = ctx ? ctx->tl : nullptr; }

TimelineScope::~TimelineScope() { t_timeline = prev_; }

uint32_t* timeline_slots(int kernel, int64_t waves) {
  tmh_timeline_state* tl = t_timeline;
  if (!tl) return nullptr;
  if (waves <= 0 || tl->used + waves > tl->capacity) {
    ++tl->dropped;
    return nullptr;
  }
  uint32_t* slots = tl->d_slots + 4 * tl->used;
  tl->log.insert(tl->log.end(), {static_cast<int64_t>(kernel), tl->used, waves});
  tl->used += waves;
  return slots;
}

}  // namespace tmh

using namespace tmh;

extern "C" {

int tmh_abi_version(void) { return TMH_ABI_VERSION; }

int tmh_device_count(int* count) {
  if (!count) return fail(nullptr, TMH_ERR_INVALID, "count is NULL");
  *count = 0;
  int n = 0;
  hipError_t err = hipGetDeviceCount(&n);
  if (err != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return fail(nullptr, TMH_ERR_NO_DEVICE, "no HIP device: %s",
                err == hipSuccess ? "none visible" : hipGetErrorString(err));
  }
  *count = n;
  return TMH_OK;
}

int tmh_ctx_create(int device, tmh_ctx** out) {
  if (!out) return fail(nullptr, TMH_ERR_INVALID, "out is NULL");
  *out = nullptr;
  int n = 0;
  TMH_TRY(tmh_device_count(&n));
  if (device < 0 || device >= n)
    return fail(nullptr, TMH_ERR_INVALID, "device %d is out of range (%d devices)", device, n);
  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return check_hip(nullptr, err, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, TMH_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950",
                device, prop.gcnArchName);
  err = hipSetDevice(device);
  if (err != hipSuccess) return check_hip(nullptr, err, "hipSetDevice");
  noalloc_scratch_init(device);
  tmh_ctx* ctx = new tmh_ctx();
  ctx->device = device;
  ctx->num_cus = prop.multiProcessorCount;
  err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (err != hipSuccess) {
    delete ctx;
    return check_hip(nullptr, err, "hipStreamCreateWithFlags");
  }
  *out = ctx;
  return TMH_OK;
}

void tmh_ctx_destroy(tmh_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) {
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
  }
  if (ctx->ws) (void)hipFree(ctx->ws);
  for (void* p : ctx->ws_retired) (void)hipFree(p);
  delete ctx->tl;
  delete ctx;
}

const char* tmh_last_error(const tmh_ctx* ctx) {
  if (ctx) return ctx->error.c_str();
  return g_thread_error.c_str();
}

void* tmh_ctx_stream(tmh_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int tmh_alloc(tmh_ctx* ctx, size_t bytes, void** d_out) {
  TMH_TRY(use_device(ctx));
  if (!d_out) return fail(ctx, TMH_ERR_INVALID, "d_out is NULL");
  *d_out = nullptr;
  if (bytes == 0) return TMH_OK;
  return check_hip(ctx, hipMalloc(d_out, bytes), "hipMalloc");
}

int tmh_free(tmh_ctx* ctx, void* d_ptr) {
  TMH_TRY(use_device(ctx));
  if (!d_ptr) return TMH_OK;
  return check_hip(ctx, hipFree(d_ptr), "hipFree");
}

int tmh_upload(tmh_ctx* ctx, void* d_dst, const void* h_src, size_t bytes) {
  TMH_TRY(use_device(ctx));
  if (bytes == 0) return TMH_OK;
  if (!d_dst || !h_src) return fail(ctx, TMH_ERR_INVALID, "tmh_upload: NULL pointer");
  TMH_TRY(check_hip(ctx, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream),
                    "hipMemcpyAsync H2D"));
  return check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

int tmh_upload_file(tmh_ctx* ctx, void* d_dst, const char* path, int64_t offset, size_t bytes) {
  TMH_TRY(use_device(ctx));
  if (!path) return fail(ctx, TMH_ERR_INVALID, "tmh_upload_file: NULL path");
  if (offset < 0) return fail(ctx, TMH_ERR_INVALID, "tmh_upload_file: negative offset");
  if (bytes == 0) return TMH_OK;
  if (!d_dst) return fail(ctx, TMH_ERR_INVALID, "tmh_upload_file: NULL destination");
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(ctx, TMH_ERR_INVALID, "tmh_upload_file: cannot open %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0 || static_cast<uint64_t>(offset) + bytes > static_cast<uint64_t>(st.st_size)) {
    close(fd);
    return fail(ctx, TMH_ERR_INVALID, "tmh_upload_file: %s holds no %zu bytes at offset %lld", path, bytes,
                (long long)offset);
  }
  // Two pinned 16 MiB staging buffers: the file is read into one while the other copies.
  constexpr size_t kChunk = size_t(16) << 20;
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int st_code = TMH_OK;
  for (int i = 0; i < 2 && st_code == TMH_OK; ++i) {
    st_code = check_hip(ctx, hipHostMalloc(&stage[i], kChunk, hipHostMallocDefault), "hipHostMalloc");
    if (st_code == TMH_OK) st_code = check_hip(ctx, hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "hipEventCreate");
  }
  auto* dst = static_cast<uint8_t*>(d_dst);
  for (size_t pos = 0, i = 0; st_code == TMH_OK && pos < bytes; ++i) {
    const int b = static_cast<int>(i & 1);
    if (i >= 2) st_code = check_hip(ctx, hipEventSynchronize(done[b]), "hipEventSynchronize");
    const size_t n = std::min(kChunk, bytes - pos);
    for (size_t got = 0; st_code == TMH_OK && got < n;) {
      const ssize_t r = pread(fd, static_cast<uint8_t*>(stage[b]) + got, n - got, offset + static_cast<int64_t>(pos + got));
      if (r < 0 && errno == EINTR) continue;
      if (r <= 0) st_code = fail(ctx, TMH_ERR_INVALID, "tmh_upload_file: reading %s failed", path);
      else got += static_cast<size_t>(r);
    }
    if (st_code == TMH_OK)
      st_code = check_hip(ctx, hipMemcpyAsync(dst + pos, stage[b], n, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync H2D");
    if (st_code == TMH_OK) st_code = check_hip(ctx, hipEventRecord(done[b], ctx->stream), "hipEventRecord");
    pos += n;
  }
  const int sync = check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (st_code == TMH_OK) st_code = sync;
  for (int i = 0; i < 2; ++i) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  close(fd);
  return st_code;
}

int tmh_download(tmh_ctx* ctx, void* h_dst, const void* d_src, size_t bytes) {
  TMH_TRY(use_device(ctx));
  if (bytes == 0) return TMH_OK;
  if (!h_dst || !d_src) return fail(ctx, TMH_ERR_INVALID, "tmh_download: NULL pointer");
  TMH_TRY(check_hip(ctx, hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream),
                    "hipMemcpyAsync D2H"));
  return check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

int tmh_copy_2d(tmh_ctx* ctx, void* d_dst, size_t dst_pitch, const void* d_src, size_t src_pitch,
                size_t width_bytes, size_t rows, void* stream) {
  TMH_TRY(use_device(ctx));
  if (width_bytes == 0 || rows == 0) return TMH_OK;
  if (!d_dst || !d_src) return fail(ctx, TMH_ERR_INVALID, "tmh_copy_2d: NULL pointer");
  if (dst_pitch < width_bytes || src_pitch < width_bytes)
    return fail(ctx, TMH_ERR_INVALID, "tmh_copy_2d: a pitch is below the row width");
  return check_hip(ctx,
                   hipMemcpy2DAsync(d_dst, dst_pitch, d_src, src_pitch, width_bytes, rows, hipMemcpyDeviceToDevice,
                                    pick_stream(ctx, stream)),
                   "hipMemcpy2DAsync");
}

int tmh_synchronize(tmh_ctx* ctx, void* stream) {
  TMH_TRY(use_device(ctx));
  return check_hip(ctx, hipStreamSynchronize(pick_stream(ctx, stream)), "hipStreamSynchronize");
}

int tmh_event_create(tmh_ctx* ctx, void** event_out) {
  TMH_TRY(use_device(ctx));
  if (!event_out) return fail(ctx, TMH_ERR_INVALID, "event_out is NULL");
  hipEvent_t ev;
  TMH_TRY(check_hip(ctx, hipEventCreate(&ev), "hipEventCreate"));
  *event_out = ev;
  return TMH_OK;
}

int tmh_event_destroy(tmh_ctx* ctx, void* event) {
  TMH_TRY(use_device(ctx));
  if (!event) return TMH_OK;
  return check_hip(ctx, hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

int tmh_event_record(tmh_ctx* ctx, void* event, void* stream) {
  TMH_TRY(use_device(ctx));
  if (!event) return fail(ctx, TMH_ERR_INVALID, "event is NULL");
  return check_hip(ctx, hipEventRecord(static_cast<hipEvent_t>(event), pick_stream(ctx, stream)),
                   "hipEventRecord");
}

int tmh_event_query(tmh_ctx* ctx, void* event, int* done) {
  TMH_TRY(use_device(ctx));
  if (!event || !done) return fail(ctx, TMH_ERR_INVALID, "tmh_event_query: NULL argument");
  const hipError_t err = hipEventQuery(static_cast<hipEvent_t>(event));
  if (err == hipErrorNotReady) {
    (void)hipGetLastError();
    *done = 0;
    return TMH_OK;
  }
  *done = err == hipSuccess ? 1 : 0;
  return check_hip(ctx, err, "hipEventQuery");
}

int tmh_event_synchronize(tmh_ctx* ctx, void* event) {
  TMH_TRY(use_device(ctx));
  if (!event) return fail(ctx, TMH_ERR_INVALID, "tmh_event_synchronize: NULL event");
  return check_hip(ctx, hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
}

int tmh_event_elapsed(tmh_ctx* ctx, void* start, void* end, float* ms_out) {
  TMH_TRY(use_device(ctx));
  if (!start || !end || !ms_out) return fail(ctx, TMH_ERR_INVALID, "tmh_event_elapsed: NULL");
  TMH_TRY(check_hip(ctx, hipEventSynchronize(static_cast<hipEvent_t>(end)), "hipEventSynchronize"));
  return check_hip(ctx,
                   hipEventElapsedTime(ms_out, static_cast<hipEvent_t>(start),
                                       static_cast<hipEvent_t>(end)),
                   "hipEventElapsedTime");
}

int tmh_graph_begin(tmh_ctx* ctx, void* stream) {
  TMH_TRY(use_device(ctx));
  return check_hip(ctx, hipStreamBeginCapture(pick_stream(ctx, stream), hipStreamCaptureModeThreadLocal),
                   "hipStreamBeginCapture");
}

int tmh_graph_end(tmh_ctx* ctx, void* stream, void** graph_exec_out) {
  TMH_TRY(use_device(ctx));
  if (!graph_exec_out) return fail(ctx, TMH_ERR_INVALID, "graph_exec_out is NULL");
  *graph_exec_out = nullptr;
  hipGraph_t graph = nullptr;
  TMH_TRY(check_hip(ctx, hipStreamEndCapture(pick_stream(ctx, stream), &graph), "hipStreamEndCapture"));
  hipGraphExec_t exec = nullptr;
  hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  TMH_TRY(check_hip(ctx, err, "hipGraphInstantiate"));
  *graph_exec_out = exec;
  return TMH_OK;
}

int tmh_graph_launch(tmh_ctx* ctx, void* graph_exec, void* stream) {
  TMH_TRY(use_device(ctx));
  if (!graph_exec) return fail(ctx, TMH_ERR_INVALID, "graph_exec is NULL");
  return check_hip(ctx, hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), pick_stream(ctx, stream)),
                   "hipGraphLaunch");
}

int tmh_graph_destroy(tmh_ctx* ctx, void* graph_exec) {
  TMH_TRY(use_device(ctx));
  if (!graph_exec) return TMH_OK;
  return check_hip(ctx, hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
}

int tmh_timeline_begin(tmh_ctx* ctx, void* d_slots, int64_t capacity) {
  TMH_TRY(use_device(ctx));
  if (!d_slots || capacity < 1) return fail(ctx, TMH_ERR_INVALID, "tmh_timeline_begin: no slots");
  if (reinterpret_cast<uintptr_t>(d_slots) % 16 != 0)
    return fail(ctx, TMH_ERR_INVALID, "tmh_timeline_begin: the slots must be 16-byte aligned");
  if (capacity > (int64_t(1) << 31)) return fail(ctx, TMH_ERR_INVALID, "tmh_timeline_begin: too many slots");
  delete ctx->tl;
  ctx->tl = new tmh_timeline_state();
  ctx->tl->d_slots = static_cast<uint32_t*>(d_slots);
  ctx->tl->capacity = capacity;
  return TMH_OK;
}

int tmh_timeline_end(tmh_ctx* ctx, int64_t* h_log, int64_t max_launches, int64_t* launches, int64_t* dropped) {
  if (!ctx) return fail(nullptr, TMH_ERR_INVALID, "the context is NULL");
  if (!ctx->tl) return fail(ctx, TMH_ERR_INVALID, "tmh_timeline_end: no timeline is being recorded");
  const int64_t n = static_cast<int64_t>(ctx->tl->log.size() / 3);
  const int64_t copy = std::max<int64_t>(0, std::min(n, max_launches));
  if (h_log && copy) std::memcpy(h_log, ctx->tl->log.data(), static_cast<size_t>(copy) * 3 * sizeof(int64_t));
  if (launches) *launches = n;
  if (dropped) *dropped = ctx->tl->dropped;
  delete ctx->tl;
  ctx->tl = nullptr;
  return TMH_OK;
}

}  // extern "C"
