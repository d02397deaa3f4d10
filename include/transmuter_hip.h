/*
 * transmuter_hip.h - C ABI of the MI355X (gfx950) library behind Transmuter's quantized-weight
 * operators: com.microsoft MatMulNBits, GatherBlockQuantized, DequantizeLinear and
 * MatMulInteger (and the grouped-expert QMoE products).
 *
 * The reference (georgeguimaraes/transmuter) has no native code of its own: its operators are
 * Elixir functions over Nx (lib/transmuter/ops/quantized.ex). These entry points are what a
 * NIF bound by those handlers calls. Each declaration names the reference function whose
 * arithmetic it replaces.
 *
 * Conventions
 *  - Every call returns a tmh_status; 0 is success. On failure tmh_last_error() holds a
 *    message. TMH_ERR_INVALID and TMH_ERR_UNSUPPORTED are the cases the reference raises
 *    ArgumentError for (quantized.ex:33-34, :53-57); a NIF maps them to that exception.
 *  - Pointers named d_* are device pointers (from tmh_alloc or any HIP allocation on the
 *    context's device); pointers named h_* are host pointers the caller owns.
 *  - Element types use ONNX TensorProto.DataType codes (tmh_dtype).
 *  - `stream` is a hipStream_t; NULL means the context's own stream. Calls are asynchronous
 *    on that stream unless stated otherwise.
 *  - Shapes are int64_t element counts; no call reads or writes outside the extents given.
 *  - Prefill MatMulNBits (split K), DynamicQuantizeLinear and QMoE keep
 *    intermediates in one workspace per context, grown outside graph capture. Calls of one
 *    context on two streams must not run at the same time; use a context per concurrent stream.
 *    A call that would have to grow the workspace while its stream is being captured into a
 *    graph fails with TMH_ERR_UNSUPPORTED (run it once before the capture). A workspace that
 *    grows is not freed: graphs captured earlier keep its address, so it stays allocated until
 *    tmh_ctx_destroy, after which no graph that used it may be launched.
 */
#ifndef TRANSMUTER_HIP_H
#define TRANSMUTER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMH_ABI_VERSION 1

typedef enum {
  TMH_OK = 0,
  TMH_ERR_INVALID = 1,     /* bad argument: sizes, types, null pointers */
  TMH_ERR_UNSUPPORTED = 2, /* valid ONNX that this path does not run (g_idx, gather_axis != 0) */
  TMH_ERR_DEVICE = 3,      /* a HIP runtime error */
  TMH_ERR_OOM = 4,         /* device memory exhausted */
  TMH_ERR_NO_DEVICE = 5    /* no usable gfx950 device */
} tmh_status;

/* ONNX TensorProto.DataType codes (lib/transmuter/ops.ex:700-713). */
typedef enum {
  TMH_F32 = 1,
  TMH_U8 = 2,
  TMH_S8 = 3,
  TMH_U16 = 4,
  TMH_S16 = 5,
  TMH_S32 = 6,
  TMH_S64 = 7,
  TMH_F16 = 10,
  TMH_BF16 = 16
} tmh_dtype;

/* Zero points of a MatMulNBits weight (quantized.ex:306-325): none (2^(bits-1)), packed
 * integers (rows of ceil(blocks*bits/8) bytes, lowest bits first), or one float per block. */
typedef enum { TMH_ZP_NONE = 0, TMH_ZP_PACKED = 1, TMH_ZP_FLOAT = 2 } tmh_zp_kind;

/* Quantization parameter layout of DequantizeLinear (quantized.ex:328-353). */
typedef enum { TMH_QPARAM_TENSOR = 0, TMH_QPARAM_AXIS = 1, TMH_QPARAM_BLOCKED = 2 } tmh_qparam_mode;

typedef struct tmh_ctx tmh_ctx;       /* one device, one stream, the last error */
typedef struct tmh_weight tmh_weight; /* a device-resident packed MatMulNBits weight */
typedef struct tmh_int8_weight tmh_int8_weight; /* a MatMulInteger B prepared for the int8 GEMM */

/* ------------------------------------------------------------------ context and memory */

/* The ABI version this library implements (TMH_ABI_VERSION). */
int tmh_abi_version(void);

/* Number of HIP devices visible to the process. Fails with TMH_ERR_NO_DEVICE when none. */
int tmh_device_count(int* count);

/* Creates a context on `device`: sets it current for the calling thread and creates a stream.
 * Fails with TMH_ERR_NO_DEVICE when the device is not a gfx950 GPU. */
int tmh_ctx_create(int device, tmh_ctx** out);
void tmh_ctx_destroy(tmh_ctx* ctx);

/* The last error message of `ctx`, or of the calling thread when ctx is NULL. Never NULL. */
const char* tmh_last_error(const tmh_ctx* ctx);

/* The context's hipStream_t. */
void* tmh_ctx_stream(tmh_ctx* ctx);

/* Device memory of the context's device. tmh_alloc of 0 bytes gives NULL and succeeds. */
int tmh_alloc(tmh_ctx* ctx, size_t bytes, void** d_out);
int tmh_free(tmh_ctx* ctx, void* d_ptr);

/* Synchronous copies: host to device, device to host (after the context's stream drains). */
int tmh_upload(tmh_ctx* ctx, void* d_dst, const void* h_src, size_t bytes);
int tmh_download(tmh_ctx* ctx, void* h_dst, const void* d_src, size_t bytes);

/*
 * Synchronous copy of bytes [offset, offset + bytes) of a file to device memory, through two
 * pinned 16 MiB staging buffers: the device upload of an initializer kept in an ONNX external
 * data file (Ops.read_external/2, lib/transmuter/ops.ex:674-697, read by
 * DeferredTensor.value/1 at move time, lib/transmuter/deferred_tensor.ex), without a host copy
 * of the whole tensor.
 */
int tmh_upload_file(tmh_ctx* ctx, void* d_dst, const char* path, int64_t offset, size_t bytes);

/* Copies `rows` rows of width_bytes between device buffers with row pitches (bytes):
 * the Split that Fusion.matmuls/2 puts after a merged matmul (lib/transmuter/fusion.ex:
 * 495-507) takes column ranges of the merged output this way. Asynchronous. */
int tmh_copy_2d(tmh_ctx* ctx, void* d_dst, size_t dst_pitch, const void* d_src, size_t src_pitch,
                size_t width_bytes, size_t rows, void* stream);

/* Blocks until the stream (NULL: the context's) has finished its work. */
int tmh_synchronize(tmh_ctx* ctx, void* stream);

/* HIP events on a stream: completion fences of asynchronous calls and timing. tmh_event_query
 * sets *done to 1 when the work recorded before the event has finished, 0 otherwise, without
 * blocking; tmh_event_synchronize blocks until it has; tmh_event_elapsed waits for `end`. */
int tmh_event_create(tmh_ctx* ctx, void** event_out);
int tmh_event_destroy(tmh_ctx* ctx, void* event);
int tmh_event_record(tmh_ctx* ctx, void* event, void* stream);
int tmh_event_query(tmh_ctx* ctx, void* event, int* done);
int tmh_event_synchronize(tmh_ctx* ctx, void* event);
int tmh_event_elapsed(tmh_ctx* ctx, void* start, void* end, float* ms_out);

/* HIP graphs: capture the calls made on `stream` between begin and end into an executable
 * graph, then replay it. Every compute call of this library is capture-safe (no allocation,
 * no memset, no host synchronisation). */
int tmh_graph_begin(tmh_ctx* ctx, void* stream);
int tmh_graph_end(tmh_ctx* ctx, void* stream, void** graph_exec_out);
int tmh_graph_launch(tmh_ctx* ctx, void* graph_exec, void* stream);
int tmh_graph_destroy(tmh_ctx* ctx, void* graph_exec);

/* ------------------------------------------------------------------ MatMulNBits */

/*
 * Uploads one MatMulNBits weight and keeps it on the device in the library's tiled layout.
 * Replaces the load-time weight preparation of Transmuter.move/2 (lib/transmuter.ex:1104-1182,
 * dequantized_weight/6 at :1230-1240) and of Transmuter.EMLX.weight/6 (lib/transmuter/emlx.ex:
 * 104-148): the weight is packed once, not dequantized to floats.
 *
 *  h_b           B, u8 [N, blocks, block_size*bits/8], blocks = ceil(K/block_size)
 *  h_scales      [N*blocks] of scales_dtype (F32, F16 or BF16)
 *  h_zero_points none (NULL), packed u8 [N*ceil(blocks*bits/8)], or [N*blocks] floats of
 *                zp_dtype, per zp_kind
 *  weight_dtype  the type the weights dequantize in (F32, F16 or BF16): the scales' type
 *                after :compute_type on the moved path, A's type in the graph (quantized.ex:42)
 *  bits          2, 4 or 8; block_size a power of two >= 16 (nbits_sizes/1, quantized.ex:226)
 * Sizes must match exactly; counts are element counts.
 */
int tmh_weight_upload_nbits(tmh_ctx* ctx, const uint8_t* h_b, size_t b_bytes, const void* h_scales,
                            int scales_dtype, size_t scales_count, const void* h_zero_points,
                            int zp_kind, int zp_dtype, size_t zp_count, int64_t K, int64_t N,
                            int bits, int block_size, int weight_dtype, tmh_weight** out);
void tmh_weight_free(tmh_weight* w);

/*
 * The host half of tmh_weight_upload_nbits: validates the same arguments and writes the
 * tiled weights, the per-block scales (weight_dtype) and the zero points (`bits` bits each for
 * packed ones, as many a byte as the reference's rows hold; f32 for float zero points) into
 * caller buffers, without touching a device. With all three
 * buffers NULL it only stores the byte counts; otherwise *q_bytes, *scale_bytes and
 * *zero_bytes give the buffer capacities on entry and the bytes written on return. A NIF can
 * pack on a host thread and upload later. No reference counterpart beyond move/2's
 * dequantized_weight/6 (lib/transmuter.ex:1230-1240), whose device work this avoids.
 */
int tmh_pack_nbits_host(const uint8_t* h_b, size_t b_bytes, const void* h_scales, int scales_dtype,
                        size_t scales_count, const void* h_zero_points, int zp_kind, int zp_dtype,
                        size_t zp_count, int64_t K, int64_t N, int bits, int block_size,
                        int weight_dtype, void* h_q, size_t* q_bytes, void* h_scale,
                        size_t* scale_bytes, void* h_zero, size_t* zero_bytes);

/*
 * tmh_weight_upload_nbits from device buffers: B, the scales and the zero points already on the
 * device (the inputs of a MatMulNBits node that move/2 did not rewrite, whose weights the
 * reference dequantizes on the device at every call, quantized.ex:39-42 and :234-240). The same
 * arguments and checks (d_* are device pointers of the sizes given), the same device bytes as
 * the host packing; the repacking runs on `stream` (NULL: the context's) and the weight may be
 * used by later work on that stream at once. Free with tmh_weight_free after that work is done.
 */
int tmh_weight_pack_nbits(tmh_ctx* ctx, const void* d_b, size_t b_bytes, const void* d_scales, int scales_dtype,
                          size_t scales_count, const void* d_zero_points, int zp_kind, int zp_dtype, size_t zp_count,
                          int64_t K, int64_t N, int bits, int block_size, int weight_dtype, void* stream,
                          tmh_weight** out);

/*
 * One weight whose rows are the rows of parts[0], then parts[1], ...: the packed form of the
 * weight concatenation of Fusion.matmuls/2 (lib/transmuter/fusion.ex:430-539), which merges
 * the MatMulNBits that read one input (q/k/v, gate/up) into one matmul over [sum N, K]. The
 * parts must share K, bits, block_size, weight type and zero point kind; 1 <= count <= 8.
 * The parts stay valid (the caller frees them). Synchronous on the context's stream.
 */
int tmh_weight_concat_nbits(tmh_ctx* ctx, const tmh_weight* const* parts, int count,
                            tmh_weight** out);

/* K, N, bits, block_size, the weight type and the device bytes the weight holds. */
int tmh_weight_info(const tmh_weight* w, int64_t* K, int64_t* N, int* bits, int* block_size,
                    int* weight_dtype, size_t* device_bytes);

/*
 * The {N, K} float weights of `w` in out_dtype, row-major, bit-exact to
 * Quantized.dequantize_weight/4 (quantized.ex:234-240; unpack packed.ex:9-23, zero points
 * quantized.ex:306-325, (q - zero) * scale packed.ex:28-36) computed in out_dtype.
 */
int tmh_dequantize_nbits(tmh_ctx* ctx, const tmh_weight* w, void* d_out, int out_dtype, void* stream);

/*
 * Y = A . W^T (+ bias): MatMulNBits (quantized.ex:30-46) over a packed weight.
 *  d_a    [M, K] of a_dtype (F32, F16, BF16), rows lda elements apart (lda >= K)
 *  d_bias NULL or [N] of bias_dtype
 *  d_y    [M, N] of y_dtype, rows ldy elements apart (ldy >= N)
 * The sums accumulate in f32 and round once to y_dtype. M >= 0 (M == 0 does nothing).
 * For M > 64 with f16 A the library picks the GEMM's tile shape and K split itself; the
 * environment variable TMH_GEMM_PLAN="bm,wn,splits[,ks]" (bm 128 or 256, wn 2 or 4; ks 2, with
 * bm 128 and wn 2 only, splits each k-block between two wavefronts) forces them, for tests and
 * tuning (an invalid value is ignored). A call whose plan splits K keeps splits*M*N f32 partial
 * sums in the context's workspace; during graph capture it fails with TMH_ERR_UNSUPPORTED when
 * the workspace is too small, so a graph always computes what an eager call does.
 */
int tmh_matmul_nbits(tmh_ctx* ctx, const tmh_weight* w, const void* d_a, int a_dtype, int64_t M,
                     int64_t lda, const void* d_bias, int bias_dtype, void* d_y, int y_dtype,
                     int64_t ldy, void* stream);

/*
 * tmh_matmul_nbits for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Same arguments and checks, but a prefill GEMM whose plan splits K keeps its f32
 * partial sums in a fixed 64 MiB scratch area per device (set up by tmh_ctx_create) instead of
 * the context's workspace, and the call neither allocates nor frees. Where tmh_matmul_nbits's
 * plan keeps at most 64 MiB of partial sums (every plan up to M * N = 2^22 outputs at 4 splits,
 * for example), both run the same kernels and plan and give the same bits; beyond that this call
 * runs the best plan whose partial sums fit (fewer K splits, or none, also when TMH_GEMM_PLAN
 * forces more), whose sums differ from tmh_matmul_nbits's only in f32 summation order. Every call
 * on one device shares that device's scratch, which keeps
 * the last call's partial sums: calls on one device that overlap in time (other streams, other
 * contexts, other threads) race and must be serialized by the caller.
 */
int tmh_matmul_nbits_noalloc(tmh_ctx* ctx, const tmh_weight* w, const void* d_a, int a_dtype, int64_t M,
                             int64_t lda, const void* d_bias, int bias_dtype, void* d_y, int y_dtype,
                             int64_t ldy, void* stream);

/* ------------------------------------------------------------------ GatherBlockQuantized */

/*
 * GatherBlockQuantized with gather_axis 0 and the quantize axis last (quantized.ex:49-66):
 * out[i, :] = (unpack(data[ids[i], :]) - zero) * scale per block, in scales_dtype, bit-exact.
 *  d_data        [rows, row_bytes] of data_dtype: U8 (unsigned values) or S8 (int4 values,
 *                sign extended; 8-bit signed data when bits == 8)
 *  d_ids         [n_ids] of ids_dtype (S32 or S64); a negative id counts from the end
 *                (-rows..-1); ids outside [-rows, rows) clamp to [0, rows-1], as an XLA
 *                gather clamps its start indices
 *  d_scales      [rows, blocks] of scales_dtype (F32, F16, BF16)
 *  d_zero_points NULL (0 for S8 data, 2^(bits-1) for U8) or packed [rows, zp_row_bytes]
 *                (U8 or S8, zp_row_bytes = ceil(blocks*bits/8))
 *  d_out         [n_ids, row_bytes*8/bits] of scales_dtype
 * row_bytes*8/bits must be a multiple of blocks.
 */
int tmh_gather_block_quantized(tmh_ctx* ctx, const void* d_data, int data_dtype, int64_t rows,
                               int64_t row_bytes, const void* d_ids, int ids_dtype, int64_t n_ids,
                               const void* d_scales, int scales_dtype, int64_t blocks,
                               const void* d_zero_points, int zp_dtype, int bits, void* d_out,
                               void* stream);

/* ------------------------------------------------------------------ DequantizeLinear */

/*
 * DequantizeLinear (quantized.ex:70-84 with expand_quant_param/3 at :328-353), bit-exact:
 * integer x subtracts the zero point in s32, float x in f32; the value converts to f32, is
 * multiplied by the f32 scale and rounds to scale_dtype.
 * x is viewed as [outer, dim, inner], dim being the quantization axis. The scale (and zero
 * point) is one value (TMH_QPARAM_TENSOR), [dim] (TMH_QPARAM_AXIS) or
 * [outer, ceil(dim/block_size), inner] (TMH_QPARAM_BLOCKED).
 *  x_dtype     U8, S8, U16, S16, S32, F16, F32 (or BF16)
 *  scale_dtype F32, F16, BF16; zero NULL or of zero_dtype (integer types, or float for float x)
 */
int tmh_dequantize_linear(tmh_ctx* ctx, const void* d_x, int x_dtype, int64_t outer, int64_t dim,
                          int64_t inner, const void* d_scale, int scale_dtype, const void* d_zero,
                          int zero_dtype, int mode, int64_t block_size, void* d_y, void* stream);

/* ------------------------------------------------------------------ MatMulInteger */

/*
 * MatMulInteger (quantized.ex:105-110; exact sums of NN.integer_product/5, nn.ex:537-555):
 * y[b, m, n] = sum_k (a[b, m, k] - a_zero[m]) * (b[(b,) k, n] - b_zero[n]) as s32
 * (two's complement, as the reference's s32 additions).
 *  d_a [batch, M, K] U8 or S8; d_b [K, N] (b_batched 0) or [batch, K, N] (1), U8 or S8
 *  d_a_zero NULL, one value or [M] (a_zero_count 1 or M), of a's type
 *  d_b_zero NULL, one value or [N] (b_zero_count 1 or N), of b's type
 *  d_y [batch, M, N] S32
 * With K = 0, d_a and d_b may be NULL and y is all zeros; with batch, M or N = 0 nothing is read
 * or written.
 */
int tmh_matmul_integer(tmh_ctx* ctx, const void* d_a, int a_dtype, const void* d_b, int b_dtype,
                       const void* d_a_zero, int64_t a_zero_count, const void* d_b_zero,
                       int64_t b_zero_count, int64_t batch, int64_t M, int64_t K, int64_t N,
                       int b_batched, void* d_y, void* stream);

/*
 * MatMulInteger with a B prepared once (no reference counterpart: for a B that is an initializer,
 * prepared at load as move/2 prepares MatMulNBits weights, lib/transmuter.ex:1104-1240).
 * tmh_int8_weight_prepare transposes B [K, N] (U8 or S8, on the device) into s8 rows of k,
 * zero-padded to a multiple of 256, and precomputes its column sums and the zero-point terms of
 * b_zero (NULL, one value or [N] of B's type); asynchronous on `stream`, whose later work may use
 * the weight at once. K must be a multiple of 16 and (N + 128) * (K padded to 256) below 2^31
 * (TMH_ERR_UNSUPPORTED otherwise; the caller keeps B and uses tmh_matmul_integer). tmh_matmul_integer_prepared computes what tmh_matmul_integer
 * computes for the same B and zero points: y[b, m, n] = sum_k (a[b, m, k] - a_zero[m]) *
 * (B[k, n] - b_zero[n]) as s32 (mod 2^32), A [batch, M, K] U8 or S8, 16-byte aligned, with
 * (M + 128) * K below 2^31; y [batch, M, N] S32.
 */
int tmh_int8_weight_prepare(tmh_ctx* ctx, const void* d_b, int b_dtype, const void* d_b_zero,
                            int64_t b_zero_count, int64_t K, int64_t N, void* stream,
                            tmh_int8_weight** out);
void tmh_int8_weight_free(tmh_int8_weight* w);
int tmh_int8_weight_info(const tmh_int8_weight* w, int64_t* K, int64_t* N, size_t* device_bytes);
int tmh_matmul_integer_prepared(tmh_ctx* ctx, const void* d_a, int a_dtype, const void* d_a_zero,
                                int64_t a_zero_count, int64_t batch, int64_t M,
                                const tmh_int8_weight* w, void* d_y, void* stream);

/* ------------------------------------------------------------------ DynamicQuantizeLinear */

/*
 * DynamicQuantizeLinear (quantized.ex:94-103), the u8 activations MatMulInteger takes:
 * low = min(min(x), 0), high = max(max(x), 0), scale = (high - low) / 255 (1 when 0),
 * zero = saturate(round(-low / scale)), y = saturate(round(x / scale) + zero), in f32 with
 * rounding half to even. The scale and zero point are written on the device.
 *  d_x [n] F32; d_y [n] U8; d_scale one F32; d_zero one U8
 */
int tmh_dynamic_quantize_linear(tmh_ctx* ctx, const void* d_x, int x_dtype, int64_t n, void* d_y,
                                void* d_scale, void* d_zero, void* stream);

/* ------------------------------------------------------------------ QMoE */

/* activation_type of QMoE (moe.ex:176-196) */
enum { TMH_ACT_RELU = 0, TMH_ACT_GELU = 1, TMH_ACT_SILU = 2, TMH_ACT_IDENTITY = 3, TMH_ACT_SWIGLU = 4 };

/*
 * The expert weights of one QMoE input (fc1, fc2 or fc3) as one packed weight of E*N rows,
 * dequantized as MoE.dequant/6 does (moe.ex:216-253): (q - zero) * scale in weight_dtype (the
 * QMoE input's type).
 *  h_w [E, N, K*bits/8] U8, values low bits first
 *  block_size > 0 with scales: scales [E, N, blocks] (blocks * block_size >= K), zero points
 *    NULL or [E, N, ceil(blocks*bits/8)] packed along the blocks
 *  block_size 0 (or no scales): scales NULL (no scaling) or [E, N] / [E, N, 1], zero points NULL
 *    or [E, ceil(N*bits/8)] packed along N; absent zero points are 2^(bits-1)
 * N must be a multiple of 16; bits 2, 4 or 8. Free with tmh_weight_free.
 */
int tmh_weight_upload_qmoe(tmh_ctx* ctx, const uint8_t* h_w, size_t w_bytes, const void* h_scales,
                           int scales_dtype, size_t scales_count, const uint8_t* h_zero_points,
                           size_t zp_bytes, int64_t E, int64_t N, int64_t K, int bits, int64_t block_size,
                           int weight_dtype, tmh_weight** out);

/*
 * QMoE (com.microsoft; moe.ex:42-61 and experts/4 at :64-102): each token's k largest router
 * values (lower expert index first among equals) and a softmax over them weight the outputs of
 * its experts: fc2(act(fc1(x) + b1[, fc3(x) + b3]) ) + b2, summed over the token's slots.
 *  d_x [T, H] of x_dtype; d_router [T, E] float; fc1 [E*N1, H]; fc2 [E*H, inter]; fc3 NULL or
 *  as fc1 (swiglu with swiglu_fusion 0); biases NULL or [E, N1] / [E, H] of bias_dtype.
 *  activation TMH_ACT_*; swiglu: fusion 0 with fc3 (gate fc1, linear fc3), 1 (or 0 without fc3)
 *  interleaved pairs, 2 halves; g * sigmoid(alpha * g) * (l + beta), g and l limited by limit
 *  when it is not 0.
 *  d_y [T, H] of x_dtype. Uses the context's workspace, which grows outside graph capture only.
 */
int tmh_qmoe(tmh_ctx* ctx, const void* d_x, int x_dtype, int64_t T, int64_t H, const void* d_router,
             int router_dtype, int64_t E, int k, const tmh_weight* fc1, const void* d_fc1_bias,
             const tmh_weight* fc2, const void* d_fc2_bias, const tmh_weight* fc3, const void* d_fc3_bias,
             int bias_dtype, int activation, int swiglu_fusion, float alpha, float beta, float limit,
             void* d_y, void* stream);

/* ------------------------------------------------------------------ measurement floors */

/*
 * Launch and read floors for benchmarks (no reference counterpart). tmh_floor_empty launches an
 * empty kernel of `workgroups` one-wavefront workgroups: the cost of one launch. tmh_floor_read
 * reads the packed weight bytes of `w` once with the decode GEMV's load pattern (one 16-byte
 * load per lane, 1 KiB per wavefront) and writes nothing to d_sink (4 bytes) unless the bytes
 * xor to a marker: the cost of a kernel that only reads the weights. Asynchronous.
 */
int tmh_floor_empty(tmh_ctx* ctx, int workgroups, void* stream);
int tmh_floor_read(tmh_ctx* ctx, const tmh_weight* w, void* d_sink, void* stream);

/*
 * More floors (no reference counterpart). tmh_floor_read_all reads every byte the weight holds on
 * the device once (its packed weights, scales and zero points), 16 bytes per lane: the cost of a
 * kernel that only reads what a GEMV over it reads. tmh_floor_write writes `bytes` (a multiple of
 * 16, below 4 GiB) of zeros to d_dst with the vocabulary gather's store pattern (16-byte
 * non-temporal stores, 4 KiB per wavefront): the cost of a gather's output alone. Asynchronous.
 */
int tmh_floor_read_all(tmh_ctx* ctx, const tmh_weight* w, void* d_sink, void* stream);
int tmh_floor_write(tmh_ctx* ctx, void* d_dst, size_t bytes, void* stream);

/*
 * Launch timeline (measurement; no reference counterpart). Between tmh_timeline_begin and
 * tmh_timeline_end, the calls of `ctx` launch a stamping build of their main kernels (the kernel
 * ids below): every wavefront writes the low 32 bits of the GPU's 100 MHz real-time counter at its
 * start and, once its memory accesses have completed, at its end, then the low 32 bits of the
 * shader cycle counter at the same two points, as four u32 into its own 16-byte slot of d_slots
 * (16-byte aligned, `capacity` slots; wavefront w of a launch in its slot first + w, w counting
 * workgroups in linear order times their wavefronts), launch after launch in the order the calls
 * are made. The stamping builds compute what the ordinary ones do. A launch captured into a graph
 * keeps its slots, so each replay of the graph writes them again; the first wavefront's start to
 * the last one's end is the kernel's time on the GPU inside the replay. Launches beyond the
 * capacity run the ordinary build and are counted as dropped. tmh_timeline_end stops recording and
 * copies the log: for each launch its kernel id, first slot and wavefronts (three int64 each) into
 * h_log (at most max_launches launches), the launch count into *launches and the dropped count
 * into *dropped.
 */
enum {
  TMH_TL_GEMV_DOT = 1,      /* k_gemv_dot: decode GEMV for one row of A */
  TMH_TL_GEMV_DEC = 2,      /* k_gemv_dec: decode GEMV, MFMA, M <= 16 */
  TMH_TL_GEMM_LDS = 3,      /* k_gemm_lds: prefill GEMM */
  TMH_TL_SPLITK_REDUCE = 4, /* k_splitk_reduce: the prefill GEMM's split-K sum */
  TMH_TL_MOE_GEMM = 5,      /* k_moe_gemm_f16: QMoE grouped expert product */
  TMH_TL_FLOOR_EMPTY = 6,   /* k_floor_empty */
  TMH_TL_FLOOR_READ = 7,    /* k_floor_read */
  TMH_TL_GATHER_ROWS = 8,   /* k_gather_bq_rows: GatherBlockQuantized of whole rows */
  TMH_TL_FLOOR_READ_ALL = 9, /* k_floor_read_all */
  TMH_TL_FLOOR_WRITE = 10,  /* k_floor_write */
  TMH_TL_MOE_ROUTE = 11,    /* k_moe_route: QMoE top-k routing */
  TMH_TL_MOE_PLAN = 12,     /* k_moe_plan: QMoE grouping by expert */
  TMH_TL_MOE_COMBINE = 13   /* k_moe_combine: QMoE weighted sum over each token's experts */
};
int tmh_timeline_begin(tmh_ctx* ctx, void* d_slots, int64_t capacity);
int tmh_timeline_end(tmh_ctx* ctx, int64_t* h_log, int64_t max_launches, int64_t* launches, int64_t* dropped);

#ifdef __cplusplus
}
#endif

#endif /* TRANSMUTER_HIP_H */
