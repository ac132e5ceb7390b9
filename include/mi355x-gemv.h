/*
 * mi355x-gemv.h -- the thin C-ABI layer between host C++ and the gfx950 HIP
 * kernels of the decode GEMV path.
 *
 * Everything here takes plain pointers and sizes.  Device pointers are
 * addresses returned by mi355x_malloc (or any HIP device allocation on the
 * same device).  No call throws; every int-returning call returns one of the
 * MI355X_* status codes and, on failure, leaves a message retrievable with
 * mi355x_last_error() on the calling thread.
 *
 * Interfaces replaced (reference file:line):
 *   mi355x_gemv            XdnaGemvEngine::run / run_quant
 *                          (include/xdna/xdna_gemv_engine.h:141-170,
 *                           src/xdna-gemv-engine.cpp:1817-1992)
 *   mi355x_gemv_bf16       XdnaGemvEngine::run_bf16 / run_quant_bf16
 *                          (include/xdna/xdna_gemv_engine.h:148-170)
 *   mi355x_prepack_*       Q4Prepacker::pack / dequantize_packed
 *                          (include/xdna/q4_prepack.h:25-45) -- successor:
 *                          repack into the HBM-resident planar layout
 *   mi355x_ctx_*           the engine object and its XRT device/staging
 *                          (XdnaGemvEngine ctor, src/xdna-gemv-engine.cpp:1725-1750;
 *                           DmaStreamer, include/xdna/dma_streamer.h:64-111)
 *   mi355x_row_bytes       bytes_per_row_for_quant (include/xdna/kquants.h:196-200)
 *   mi355x_set_iq_grid     ggml's iq3xxs_grid / iq2s_grid tables, which the
 *                          reference reaches only through ggml-cpu via dlsym
 *                          (src/xdna-gemv-engine.cpp:1388-1396)
 */
#ifndef MI355X_GEMV_H
#define MI355X_GEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355X_API __attribute__((visibility("default")))

/* status codes */
#define MI355X_OK 0
#define MI355X_EINVAL (-1)       /* invalid argument: shape, size, type, pointer */
#define MI355X_EUNSUPPORTED (-2) /* valid ggml input this build does not compute */
#define MI355X_EHIP (-3)         /* HIP runtime error (message carries hipError) */
#define MI355X_ENOMEM (-4)       /* device or pinned-host allocation failed */

/* ggml type ids (GGUF on-disk values) of the weight formats */
#define MI355X_TYPE_F32 0
#define MI355X_TYPE_Q4_0 2
#define MI355X_TYPE_Q3_K 11
#define MI355X_TYPE_Q4_K 12
#define MI355X_TYPE_Q5_K 13
#define MI355X_TYPE_Q6_K 14
#define MI355X_TYPE_IQ3_XXS 18
#define MI355X_TYPE_IQ3_S 21
#define MI355X_TYPE_IQ2_S 22
#define MI355X_TYPE_IQ4_XS 23

typedef struct mi355x_ctx mi355x_ctx; /* one device + one HIP stream */

/* Device id of a host-only context (mi355x_ctx_create): bound to no GPU, it
 * needs no HIP device.  Options can be set on it; every entry point that
 * would reach a device fails before doing so, as a lost device would: it
 * returns MI355X_EHIP with "<entry>: hipErrorNoDevice (...) [host-only
 * context]".  For running the device-error paths of host code (the ggml
 * plugin's) on machines without a GPU.  No counterpart in the reference,
 * whose engine without hardware computes on the CPU instead
 * (src/xdna-gemv-engine.cpp:1738-1749). */
#define MI355X_DEVICE_HOST_ONLY (-1)

/* Message of the last failing call on this thread ("" if none). */
MI355X_API const char *mi355x_last_error(void);

/* Fault injection for tests: no GPU fault and no device needed.  No
 * counterpart in the reference, whose engine reports device failures by
 * throwing and whose plugin turns that into GGML_STATUS_FAILED
 * (src/ggml-xdna.cpp:299-305, 803-807).  After `skip` more calls that reach
 * it, the next call of the entry point named `entry` ("mi355x_gemv",
 * "mi355x_gemv_multi", "mi355x_memcpy_h2d", "mi355x_ctx_fence",
 * "mi355x_server_gemv", ...; "*" for any entry point that would reach a
 * device) fails before any device work, as if HIP had returned `hip_error`
 * (a hipError_t value): MI355X_EHIP (MI355X_ENOMEM for hipErrorOutOfMemory)
 * with mi355x_last_error() = "<entry>: <hipErrorName> (<hipErrorString>)
 * [injected]".  One fault at a time, process-wide, disarmed once it fired;
 * entry NULL disarms.  The environment variable
 * MI355X_INJECT_FAULT="<entry>:<hip_error>[:<skip>]" arms one at first use
 * of the library. */
MI355X_API int mi355x_inject_fault(const char *entry, int hip_error, int skip);

/* ---- devices and contexts ------------------------------------------------ */
MI355X_API int mi355x_device_count(int *count);
/* Creates a context on `device` with its own non-blocking HIP stream
 * (MI355X_DEVICE_HOST_ONLY: a host-only context, see above). */
MI355X_API int mi355x_ctx_create(int device, mi355x_ctx **out);
MI355X_API void mi355x_ctx_destroy(mi355x_ctx *ctx);
/* Waits for all work queued on the context's stream. */
MI355X_API int mi355x_ctx_sync(mi355x_ctx *ctx);
/* Lower-latency wait for a host loop that issues one GEMV group at a time
 * (no counterpart in the reference, whose engine calls block): queues a
 * one-wave kernel that stores a sequence number into pinned host memory and
 * spins until it arrives (falling back to mi355x_ctx_sync after 2 ms).  On
 * return every kernel and copy queued before the call has completed and its
 * writes to device memory and to pinned (hipHostMalloc) host memory are
 * visible to the caller.  Copies into pageable host memory queued directly
 * with HIP need mi355x_ctx_sync. */
MI355X_API int mi355x_ctx_fence(mi355x_ctx *ctx);
/* The context's hipStream_t, as an opaque pointer. */
MI355X_API void *mi355x_ctx_stream(mi355x_ctx *ctx);
MI355X_API int mi355x_ctx_device(mi355x_ctx *ctx);
/* Free and total device memory (hipMemGetInfo) of the context's device. */
MI355X_API int mi355x_mem_info(mi355x_ctx *ctx, size_t *free_bytes, size_t *total_bytes);
/* Device name and PCI bus id into caller buffers (NUL-terminated). */
MI355X_API int mi355x_device_describe(int device, char *name, size_t name_len, char *pci,
                                      size_t pci_len);

/* Per-context options.
 *   MI355X_OPT_VARIANT: which kernel family computes GEMVs --
 *     MI355X_VARIANT_AUTO (default: for Q4_0 digit planes where they apply;
 *       for the K/IQ types 16-bit activation digits (row form) for Q3_K,
 *       Q4_K, Q5_K and Q6_K, IQ4_XS rows of at most 8192 values, and
 *       IQ3_S/IQ3_XXS/IQ2_S rows of at most 8192 values with N >= 4096, one
 *       row per wavefront step; f32 activations for the rest: longer IQ rows
 *       and smaller IQ matrices),
 *     MI355X_VARIANT_EXACT_F32 (codes -> f32, fp32 FMA; activations used
 *       exactly as given), MI355X_VARIANT_DIGITS (activations as fixed point
 *       per 32-value block -- 20-bit for Q4_0 with int4 dot8 products, 16-bit
 *       for the K/IQ types with int8 dot4 products),
 *     MI355X_VARIANT_GGML_Q8 (the arithmetic of ggml's CPU backend, so that
 *       results follow ggml-cpu rather than the f32 references: Q4_0 -- the
 *       activation row quantized to Q8_0 per 32-value block, integer block
 *       dot products scaled by d_w * d_x, blocks summed in order; the eight
 *       256-value types -- the row quantized to Q8_K per superblock and
 *       ggml's generic vec_dot_<type>_q8_K sums, rows of up to 16384 values;
 *       BF16 activations for Q4_0 and longer K/IQ rows return
 *       MI355X_EUNSUPPORTED in this variant).
 *   MI355X_OPT_ROWS_PER_WAVE: 0 (auto) or 1, 2, 4 rows per wavefront step
 *     (rows and K-split forms); 4, 8 or 16 rows per step (stream form).
 *   MI355X_OPT_WAVES_PER_GROUP: 0 (auto), 8 or 16 wavefronts per workgroup
 *     (digit-plane Q4_0 kernel).
 *   MI355X_OPT_GRID: 0 (auto) or a cap on the number of workgroups.
 *   MI355X_OPT_PREFETCH: 0 (auto), 1 (each wavefront requests its next row
 *     group before reducing the current one -- for the K/IQ row form before
 *     decoding it, one row per wavefront step), 2 (off).
 *   MI355X_OPT_FORM: work split of the digit-plane kernels (Q4_0; the
 *     pipelined form also for the K/IQ types) --
 *     MI355X_FORM_AUTO (default), MI355X_FORM_ROWS (a wavefront owns whole
 *     rows), MI355X_FORM_KSPLIT (a wavefront owns one 64-block column of 2 or
 *     4 rows; needs rows of a multiple of 8 blocks), MI355X_FORM_STREAM (one
 *     workgroup per CU; a lane owns one block of every row of its team and
 *     keeps that block's activation digits in registers; K <= 16384),
 *     MI355X_FORM_PIPE (one workgroup per CU -- eight wavefronts for Q4_0,
 *     four for the K/IQ types -- each wavefront owning a run of consecutive
 *     rows whose loads are issued two (Q4_0) or three (K/IQ) rows ahead of
 *     their dot products; Q4_0: K a multiple of 2048 up to 16384, 16-byte
 *     aligned weights and activation row; K/IQ types: 16-bit digit
 *     arithmetic, any K).
 *   MI355X_OPT_OVERLAP: 0 (default: off) or S = 2, 3, 4.  With S,
 *     consecutive mi355x_gemv calls may run at the same time: the context
 *     uses S - 1 of the 3 more streams of the same kind it creates with its
 *     own (consecutive streams get distinct hardware queues), and GEMVs with f32
 *     activations on a 16-byte boundary (IQ3_XXS and IQ2_S once the context
 *     holds the current grid, after one such GEMV) take the S streams in
 *     turn, so that up to S launches are in flight and each one's start
 *     overlaps the previous ones' ends.  The caller promises
 *     that such a run of calls is independent: none reads an output that
 *     another in the run writes, and no two write the same output.  Every
 *     other call on the context (copies, fills, prepack, the other GEMV
 *     entry points, sync, fence, mi355x_ctx_stream, set_option, frees)
 *     first makes the context's stream wait for the second stream, so it
 *     is ordered after the whole run, as are later GEMVs on that stream.
 *     Not for HIP stream capture; one thread per context. */
#define MI355X_OPT_VARIANT 1
#define MI355X_OPT_ROWS_PER_WAVE 2
#define MI355X_OPT_WAVES_PER_GROUP 3
#define MI355X_OPT_GRID 4
#define MI355X_OPT_PREFETCH 5
#define MI355X_OPT_FORM 6
#define MI355X_OPT_OVERLAP 7
#define MI355X_VARIANT_AUTO 0
#define MI355X_VARIANT_EXACT_F32 1
#define MI355X_VARIANT_DIGITS 2
#define MI355X_VARIANT_GGML_Q8 3
#define MI355X_FORM_AUTO 0
#define MI355X_FORM_ROWS 1
#define MI355X_FORM_KSPLIT 2
#define MI355X_FORM_STREAM 3
#define MI355X_FORM_PIPE 4
MI355X_API int mi355x_ctx_set_option(mi355x_ctx *ctx, int option, int64_t value);

/* ---- memory ----------------------------------------------------------------
 * Copies and fills are ordered on the context's stream; the *_sync forms
 * return after completion. */
MI355X_API int mi355x_malloc(mi355x_ctx *ctx, size_t bytes, void **dptr);
MI355X_API int mi355x_free(mi355x_ctx *ctx, void *dptr);
/* Page-locked host memory (hipHostMalloc) for staging transfers. */
MI355X_API int mi355x_host_malloc(size_t bytes, void **hptr);
MI355X_API int mi355x_host_free(void *hptr);
/* The device address of page-locked host memory from mi355x_host_malloc
 * (kernels read and write it over PCIe), for any byte inside it. */
MI355X_API int mi355x_host_device_ptr(const void *hptr, void **dptr);
MI355X_API int mi355x_memcpy_h2d(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes);
MI355X_API int mi355x_memcpy_d2h(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes);
MI355X_API int mi355x_memcpy_d2d(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Enqueue-only copies on the context's stream: with host memory from
 * mi355x_host_malloc they return at once (wait with mi355x_ctx_sync or
 * mi355x_ctx_fence before touching the host side); pageable host memory
 * works but the runtime may stage it synchronously. */
MI355X_API int mi355x_memcpy_h2d_async(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes);
MI355X_API int mi355x_memcpy_d2h_async(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Fill with a byte value using a kernel (safe under graph capture). */
MI355X_API int mi355x_fill(mi355x_ctx *ctx, void *dst, uint8_t value, size_t bytes);

/* ---- formats ------------------------------------------------------------- */
/* Bytes of one ggml row of K values of `type`; -1 if K is not a multiple
 * of the type's block or the type is unknown. */
MI355X_API int64_t mi355x_row_bytes(int type, int64_t K);
/* 1 if this build computes GEMVs of `type` right now (IQ3_XXS and IQ2_S need
 * their grid installed with mi355x_set_iq_grid first), else 0. */
MI355X_API int mi355x_type_ready(int type);
/* Installs the IQ3_XXS (uint32[256]) or IQ2_S (uint64[1024]) grid for every
 * context created afterwards and every existing one.  `bytes` must equal the
 * table size and every byte a magnitude in 1..127 (as in ggml's grids),
 * else MI355X_EINVAL.  Table contents are ggml's; this library does not ship
 * them. */
MI355X_API int mi355x_set_iq_grid(int type, const void *table, size_t bytes);

/* ---- prepack: ggml raw bytes <-> resident layout ----------------------------
 * The resident layout of a tensor occupies exactly the same bytes as its
 * ggml encoding (N * row_bytes) and is a row-local byte permutation of it, so
 * any byte range [offset, offset+size) of the ggml encoding maps to the same
 * set of rows.  Q4_0 rows become [16-byte nibble groups of every block][fp16
 * scales of every block]; K-quant and IQ rows become one plane per block
 * field (codes, high bits, signs, scales, fp16 d).  The plane order of a
 * K/IQ row depends on the row's address mod 4, so resident tensors of those
 * types must start on a 4-byte boundary (mi355x_malloc gives 256).
 *
 * Scatter `size` bytes of ggml encoding (host memory), which start at byte
 * `offset` of the tensor, into the resident tensor `packed_dev`. */
MI355X_API int mi355x_prepack_from_host(mi355x_ctx *ctx, int type, int64_t N, int64_t K,
                                        void *packed_dev, const void *raw_host, size_t offset,
                                        size_t size);
/* Same, with the raw bytes already on the device (raw_dev holds `size`
 * bytes).  raw_dev and packed_dev must not overlap. */
MI355X_API int mi355x_prepack_from_device(mi355x_ctx *ctx, int type, int64_t N, int64_t K,
                                          void *packed_dev, const void *raw_dev, size_t offset,
                                          size_t size);
/* Gather ggml bytes [offset, offset+size) of a resident tensor into host
 * memory (the inverse permutation). */
MI355X_API int mi355x_unpack_to_host(mi355x_ctx *ctx, int type, int64_t N, int64_t K,
                                     const void *packed_dev, void *raw_host, size_t offset,
                                     size_t size);

/* ---- GEMV ----------------------------------------------------------------
 * y[r] = sum_c w[r][c] * x[c] for r < N, with W the resident (prepacked)
 * tensor of N rows of K values.  x and y are device pointers; the call only
 * enqueues work on the context's stream (use mi355x_ctx_sync to wait).
 * Validation mirrors XdnaGemvEngine::run (src/xdna-gemv-engine.cpp:1823-1839):
 * K must be a multiple of the block, N*row_bytes must not overflow. */
MI355X_API int mi355x_gemv(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                           const float *x, float *y);
/* Several GEMVs that share the activation row: y_j = W_j x for j < njobs
 * (1..MI355X_MULTI_MAX_JOBS), every W_j a resident tensor of `type` with
 * N_j rows of K values.  Q4_0 runs as one launch: in the AUTO and DIGITS
 * variants for rows of whole 64-block columns (K a multiple of 2048, up to
 * 16384), 16-byte aligned, with a 16-byte aligned x (the pipelined form; the
 * same per-row arithmetic as mi355x_gemv, the 64 lane partials of a row
 * added in the order of the rows-per-wavefront the combined row count
 * picks), in the GGML_Q8 variant for K up to 16384 (bit-identical to one
 * call per matrix); otherwise one launch per matrix, as mi355x_gemv.  No
 * counterpart in the reference: it serves graph_compute, which groups the
 * consecutive MUL_MAT nodes that read one activation (src/ggml-xdna.cpp:
 * 783-823 runs them one at a time). */
#define MI355X_MULTI_MAX_JOBS 8
typedef struct mi355x_gemv_job {
    const void *W; /* resident tensor of N rows */
    int64_t N;
    float *y;      /* N outputs (device memory) */
} mi355x_gemv_job;
MI355X_API int mi355x_gemv_multi(mi355x_ctx *ctx, int type, int64_t K, const float *x, int njobs,
                                 const mi355x_gemv_job *jobs);
/* Same with BF16 activations (raw bits), widened exactly to f32. */
MI355X_API int mi355x_gemv_bf16(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                                const uint16_t *x_bf16, float *y);
/* M activation rows at once (row m at x + m*x_stride floats, output at
 * y + m*y_stride floats); the M-row case the reference admits for weights in
 * its own buffer type and computes as M sequential GEMVs
 * (src/ggml-xdna.cpp:110-112, 287-296).  Q4_0 with the digit-plane
 * arithmetic (variants AUTO and DIGITS), rows a multiple of 256 values and
 * 16-byte aligned weights: up to 8 activations per pass over the weights
 * (one staging launch into a context buffer, one batched launch).  Other
 * cases:
 * M sequential GEMVs.  Calls on one context serialise on its lock while
 * they enqueue. */
MI355X_API int mi355x_gemv_batched(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                                   const float *x, int64_t x_stride, float *y, int64_t y_stride,
                                   int64_t M);

/* Allocation-free form of mi355x_gemv_batched, for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses
 * that forbid it).  No counterpart in the reference.  Same arguments and the
 * same outputs, bit for bit; the K-split batched form keeps its activation
 * tiles in the library's static device scratch of
 * MI355X_NOALLOC_SCRATCH_BYTES (336 KiB per device, held until the process
 * ends; enough for 8 activations of K = 16384 per pass, the most the form
 * stages) instead of a context buffer grown with hipMalloc.  Every call on
 * one device shares that scratch: calls that overlap on one device (two
 * streams or contexts of the same device) race.  Nothing else allocates:
 * K/IQ weights need 16-byte aligned activation rows (x and x_stride a
 * multiple of 4 floats), IQ3_XXS / IQ2_S need their grid already on the
 * context (one mi355x_gemv of the type first); otherwise MI355X_EINVAL /
 * MI355X_EUNSUPPORTED with a message. */
#define MI355X_NOALLOC_SCRATCH_BYTES 344064
MI355X_API int mi355x_gemv_batched_noalloc(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                                           const float *x, int64_t x_stride, float *y, int64_t y_stride,
                                           int64_t M);

/* ---- persistent GEMV server (decode loops) ---------------------------------
 * No counterpart in the reference (its engine calls block, one dispatch
 * each).  For a host loop that issues one Q4_0 GEMV group at a time -- batch-1
 * decode -- launch and completion cost more than the kernel.  A server keeps
 * one workgroup per CU resident (cooperative launch on its own stream) and
 * takes commands through pinned host memory: mi355x_server_gemv copies x,
 * publishes the jobs and returns once every output is written.  Jobs share x
 * and K; outputs are device-visible pointers (device memory, or pinned host
 * memory through hipHostGetDevicePointer).  The variant of the server's
 * context at the call picks the arithmetic per row: AUTO and DIGITS the digit
 * kernel's row form (bit-identical to MI355X_FORM_ROWS), GGML_Q8 ggml-cpu's
 * Q8_0 numerics (bit-identical to mi355x_gemv in that variant); EXACT_F32 is
 * MI355X_EUNSUPPORTED.  K: a multiple of
 * 256 up to max_k (<= 16384); weights 16-byte aligned.  The resident kernel
 * leaves by itself after 1 s without a command (the next call relaunches it),
 * on mi355x_server_stop / _destroy, and before any mi355x_free or
 * mi355x_ctx_destroy on its device, from any context or thread (a hipFree
 * would wait for it; such a stop waits for the command in flight).  Calls on
 * one server serialise on its lock; destroy servers before their context. */
typedef struct mi355x_server mi355x_server;
typedef struct mi355x_server_job {
    const void *W; /* resident Q4_0 tensor of N rows */
    int64_t N;
    float *y;      /* N outputs */
} mi355x_server_job;
MI355X_API int mi355x_server_create(mi355x_ctx *ctx, int64_t max_k, mi355x_server **out);
MI355X_API int mi355x_server_gemv(mi355x_server *s, const float *x, int64_t K, int njobs,
                                  const mi355x_server_job *jobs);
/* A SwiGLU feed-forward block as one server command (no counterpart in the
 * reference, where ggml-cpu runs the GLU between two MUL_MATs):
 *   g = W_gate x, u = W_up x   (F rows each, K columns),
 *   h_i = silu(g_i) * u_i      (h stays in the server's device memory),
 *   y = W_down h               (N rows, F columns),
 * with a grid barrier between the stages instead of a return to the host.
 * Each GEMV has the arithmetic mi355x_server_gemv gives it in the context's
 * variant.  silu(g) * u is computed in f32, one IEEE operation per step, with
 * no other contraction than the fmas named:
 *   t = -g; c = min(max(t, -87.3), 88);
 *   n = fma(c, 1.44269504088896341, 12582912) - 12582912;
 *   r = fma(-n, 0.693145751953125, c); r = fma(-n, 1.42860682030941723e-6, r);
 *   p = 1/5040; p = fma(p, r, k) for k = 1/720, 1/120, 1/24, 1/6, 0.5, 1, 1
 *     (each constant the f32 quotient);
 *   e = t < -87.3 ? 0 : p * 2^n;  h = g / (1 + e) * u  (division correctly
 *   rounded),
 * so a host that evaluates the same steps gets the same h, and then the same
 * y.  K and F: multiples of 256 up to max_k; weights 16-byte aligned; y
 * device-visible as for mi355x_server_gemv. */
MI355X_API int mi355x_server_swiglu(mi355x_server *s, const float *x, int64_t K, const void *W_gate,
                                    const void *W_up, int64_t F, const void *W_down, int64_t N, float *y);
/* The rest of a pre-norm transformer layer after attention as one server
 * command (no counterpart in the reference):
 *   r  = resid + W_o x           (W_o: H rows, K columns; resid: H floats),
 *   xn = rmsnorm(r) * norm_w     (norm_w: H floats in device memory),
 *   y  = r + W_down (silu(W_gate xn) * (W_up xn))   (gate/up: F rows, H
 *        columns; down: H rows, F columns; SiLU as mi355x_server_swiglu),
 * with grid barriers between the stages.  The GEMVs have mi355x_server_gemv's
 * arithmetic in the context's variant, the additions are single f32 adds,
 * and rmsnorm takes these steps: ss = the sum of r_i^2 in double as 16
 * partial sums p_k = sum over i0 = 0, 16, 32, ... of r[i0 + k]^2 in that order,
 * l_k = (p_k + p_{4+k}) + (p_{8+k} + p_{12+k}) for k < 4,
 * ss = (l_0 + l_1) + (l_2 + l_3);  s = 1 / sqrt(float(ss / H) + eps) in f32
 * (correctly rounded);  xn_i = (r_i * s) * norm_w_i.  K, H, F: multiples of
 * 256, H <= 4096, F <= max_k and K + H <= max_k; y device-visible.
 * The server keeps y in device memory until the next block command: resid
 * NULL takes the residual from there (the previous block command's y, same
 * H), and y NULL leaves it there only -- a layer loop passes the host's
 * residual once and reads y back after its last layer.
 * With W_next (else NULL, and the three after it ignored): after another
 * grid barrier, y_next = W_next (rmsnorm(y) * next_norm_w) -- the next
 * layer's q|k|v (N_next rows, H columns) -- in the same command. */
MI355X_API int mi355x_server_block(mi355x_server *s, const float *x, int64_t K, const void *W_o,
                                   const float *resid, int64_t H, const float *norm_w, float eps,
                                   const void *W_gate, const void *W_up, int64_t F, const void *W_down,
                                   float *y, const float *next_norm_w, const void *W_next, int64_t N_next,
                                   float *y_next);
MI355X_API int mi355x_server_stop(mi355x_server *s);
/* 1 while the server's resident kernel is running, 0 once it has left (after
 * its idle time, a stop, or before the first command); < 0 on error. */
MI355X_API int mi355x_server_running(mi355x_server *s);
MI355X_API void mi355x_server_destroy(mi355x_server *s);

/* ---- measurement -----------------------------------------------------------
 * Times `iters` back-to-back launches of mi355x_gemv on the context's stream
 * with HIP events, rotating through `n_weights` resident copies of W
 * (weights[i]), after `warmup` untimed launches.  *ms_total receives the
 * elapsed milliseconds of the timed launches.  With MI355X_OPT_OVERLAP = S,
 * launch i writes y + (i % S) * N (y holds S * N floats) and the timed span
 * ends after every stream's launches. */
MI355X_API int mi355x_time_gemv(mi355x_ctx *ctx, int type, const void *const *weights,
                                int n_weights, int64_t N, int64_t K, const float *x, float *y,
                                int warmup, int iters, double *ms_total);

#ifdef __cplusplus
}
#endif

#endif
