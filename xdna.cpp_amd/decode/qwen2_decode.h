/*
 * qwen2_decode.h -- batch-1 greedy decoder of a Qwen2-shaped model with Q4_0
 * weights, for end-to-end measurement of the decode GEMV path.
 *
 * Everything except the matrix-vector products runs on the host in C++
 * (RMSNorm, RoPE, grouped-query attention over a f32 KV cache, SwiGLU,
 * residuals, embedding lookup, argmax).  Every weight matrix -- per layer
 * q, k, v, o, gate, up, down, plus the tied output projection -- is a Q4_0
 * GEMV done by a backend: either the MI355X library (weights prepacked once
 * into HBM) or a caller-supplied function (a CPU reference).
 *
 * Weights are random: seeded N(0, 0.02) f32 values quantized with ggml's Q4_0
 * rule; norms are 1, q/k/v biases N(0, 0.02).
 */
#ifndef QWEN2_DECODE_H
#define QWEN2_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QD_API __attribute__((visibility("default")))

typedef struct qd_config {
    int n_layers;       /* 36 for the 3B shape */
    int hidden;         /* 2048 */
    int n_heads;        /* 16 */
    int n_kv_heads;     /* 2 */
    int head_dim;       /* 128 (a multiple of 8) */
    int ffn;            /* 11008 */
    int vocab;          /* 151936 */
    float rope_theta;   /* 1e6 */
    float norm_eps;     /* 1e-6 */
    uint64_t seed;
} qd_config;

typedef struct qd_model qd_model;

/* Matrix ids: 7 per layer (q, k, v, o, gate, up, down) in that order, then
 * the output projection (tied to the token embedding) at 7 * n_layers. */
#define QD_Q 0
#define QD_K 1
#define QD_V 2
#define QD_O 3
#define QD_GATE 4
#define QD_UP 5
#define QD_DOWN 6

/* A backend GEMV: y[0..N) = W_id (N x K, ggml Q4_0 bytes) * x[0..K). */
typedef int (*qd_gemv_fn)(void *user, int id, const uint8_t *w, int64_t N, int64_t K, const float *x,
                          float *y);

QD_API qd_model *qd_model_create(const qd_config *cfg, int threads);
QD_API void qd_model_free(qd_model *m);
QD_API int qd_n_matrices(const qd_model *m);
/* ggml Q4_0 bytes of matrix `id` and its shape. */
QD_API const uint8_t *qd_matrix(const qd_model *m, int id, int64_t *N, int64_t *K);
/* Vector `id`: 5 per layer (attn norm, ffn norm, q bias, k bias, v bias),
 * then the output norm at 5 * n_layers. */
QD_API const float *qd_vector(const qd_model *m, int id, int *n);
QD_API const char *qd_last_error(void);
/* Logits (n = vocab floats) behind the last token of the last qd_generate. */
QD_API int qd_last_logits(const qd_model *m, float *out, int n);
/* The weight quantizer (ggml's Q4_0 rule), exposed for tests. */
QD_API void qd_quantize_q4_0(const float *x, int64_t N, int64_t K, uint8_t *out);
/* The host's SwiGLU step, g[i] = silu(g[i]) * u[i], in the f32 steps that
 * mi355x_server_swiglu states (exposed for tests). */
QD_API void qd_silu_mul(float *g, const float *u, int n);
/* The host's RMSNorm, out = x * s * w with s from the double sum of squares
 * in the order mi355x_server_block states (exposed for tests). */
QD_API void qd_rmsnorm(const float *x, const float *w, float *out, int n, float eps);

/* Moves every matrix into HBM (prepacked) on `device`; later runs with
 * backend 0 use it. */
QD_API int qd_attach_gpu(qd_model *m, int device);

/* GEMV groups (q|k|v, gate|up) whose matrices lie back to back in HBM run
 * as one launch when `on` (the default); off = one launch per matrix, as a
 * ggml graph with one MUL_MAT node per weight dispatches them. */
QD_API void qd_set_fuse(qd_model *m, int on);
/* Server mode with fused groups: the layer's o projection, both residual
 * adds, the FFN norm, gate|up, SiLU and down as one mi355x_server_block
 * command when `on` (the default); off = the o command, then the FFN as one
 * mi355x_server_swiglu command. */
QD_API void qd_set_block(qd_model *m, int on);
/* Server mode with fused groups: gate|up, SiLU and down as one
 * mi355x_server_swiglu command when `on` (the default); off = gate|up and
 * down as two GEMV commands with SiLU on the host, so that only the
 * matrix-vector products run on the GPU (the split of a ggml backend that
 * claims MUL_MAT alone).  Block commands need it on. */
QD_API void qd_set_swiglu(qd_model *m, int on);
/* How activations and outputs cross PCIe on the GPU path:
 * QD_IO_STAGED: x is copied into HBM and y back from HBM around the launches
 * (the traffic pattern of a ggml backend whose buffers are device memory);
 * QD_IO_MAPPED (default): the kernels read x from and write y to pinned
 * host memory directly, saving two copy commands per GEMV group (outputs
 * longer than 65536 floats, i.e. the vocabulary projection, still use one
 * device-to-host copy). */
#define QD_IO_STAGED 0
#define QD_IO_MAPPED 1
QD_API int qd_set_io(qd_model *m, int mode);
/* How GEMV groups reach the GPU on the GPU path:
 * QD_WAIT_SERVER (default): every group is a command to a persistent GEMV
 * server (mi355x_server_*), outputs in pinned memory, no launch per group --
 * for the AUTO, DIGITS and GGML_Q8 variants with rows of multiples of 256
 * values on a device with cooperative launch, else as QD_WAIT_FENCE;
 * QD_WAIT_FENCE: one launch per group, then mi355x_ctx_fence (spin on a
 * completion word in pinned memory); QD_WAIT_STREAM: one launch per group,
 * then mi355x_ctx_sync (hipStreamSynchronize).  qd_last_wait gives the mode
 * the last GPU decode used. */
#define QD_WAIT_STREAM 0
#define QD_WAIT_FENCE 1
#define QD_WAIT_SERVER 2
/* QD_WAIT_PLUGIN: every group through the ggml plugin (the drop-in
 * boundary): weights placed as ggml tensors in the plugin's device buffer
 * (a second resident copy, made on first use), and per group the activation
 * copied in, one graph_compute over the group's MUL_MAT nodes, the outputs
 * copied out and a synchronize -- the calls ggml-backend makes for a
 * backend's split of a graph.  qd_last_launches counts MUL_MAT nodes. */
#define QD_WAIT_PLUGIN 3
QD_API int qd_set_wait(qd_model *m, int mode);
/* QD_WAIT_PLUGIN: how the plugin's graph_compute runs a group
 * (GGML_MI355X_GROUPS_LAUNCH, the default, or GGML_MI355X_GROUPS_SERVER of
 * ggml-mi355x.h). */
QD_API int qd_set_plugin_groups(qd_model *m, int mode);
QD_API int qd_last_wait(const qd_model *m);
/* Kernel variant of the GPU GEMVs (MI355X_OPT_VARIANT of mi355x-gemv.h):
 * MI355X_VARIANT_GGML_Q8 gives ggml-cpu's Q8_0-activation arithmetic. */
QD_API int qd_set_variant(qd_model *m, int variant);
/* GPU GEMV launches in the generation phase of the last qd_generate. */
QD_API int64_t qd_last_launches(const qd_model *m);

/* Greedy decode: processes `n_prompt` tokens one at a time, then generates
 * `n_gen` tokens into out_tokens.  backend 0 = MI355X, 1 = `cpu_gemv`.
 * The generation phase is the n_gen - 1 forward passes after the prompt
 * (the first generated token comes from the last prompt position).
 * timings (optional, 4 doubles): prompt seconds, generation-phase seconds,
 * seconds inside GEMV calls in the generation phase (backend 0: activation
 * upload, GEMV launches and output download), host-op seconds in the
 * generation phase. */
QD_API int qd_generate(qd_model *m, int backend, qd_gemv_fn cpu_gemv, void *user, const int32_t *prompt,
                       int n_prompt, int n_gen, int32_t *out_tokens, double *timings);

#ifdef __cplusplus
}
#endif

#endif
