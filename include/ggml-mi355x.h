/*
 * ggml-mi355x.h -- the ggml backend plugin surface of libggml-mi355x.so.
 *
 * The library is a dynamically loaded ggml backend (GGML_BACKEND_PATH) that
 * claims single-row GGML_OP_MUL_MAT on Q4_0, Q3_K..Q6_K, IQ4_XS, IQ3_S and --
 * when their grids are installed -- IQ3_XXS and IQ2_S weights, and computes
 * them with gfx950 kernels on weights resident in HBM.
 *
 * Entry points and the reference interface each one replaces:
 *   ggml_backend_init / ggml_backend_score   include/xdna/ggml-xdna.h:147-148,
 *                                            src/ggml-xdna.cpp:721-730
 *   ggml_backend_mi355x_reg                  ggml_backend_xdna_reg (ggml-xdna.h:165)
 *   ggml_backend_mi355x_init / _free / ggml_backend_is_mi355x
 *                                            ggml_backend_xdna_init / _free / ggml_backend_is_xdna
 *                                            (ggml-xdna.h:156-158, src/ggml-xdna.cpp:736-776)
 *   ggml_backend_mi355x_buffer_type / _host_buffer_type
 *                                            ggml_backend_xdna_buffer_type / _host_buffer_type
 *                                            (ggml-xdna.h:160-161)
 *   ggml_backend_mi355x_graph_compute        ggml_backend_xdna_graph_compute
 *                                            (ggml-xdna.h:151, src/ggml-xdna.cpp:783-823)
 *   ggml_backend_mi355x_supports_op / _compute_graph on struct ggml_tensor_mi355x
 *                                            the compatibility harness API on
 *                                            struct ggml_tensor_xdna
 *                                            (ggml-xdna.h:131-142, 163-164;
 *                                             src/ggml-xdna.cpp:778-781, 825-844)
 *   ggml_backend_mi355x_set_op_mul_mat       no counterpart: the reference hard-binds
 *                                            GGML_OP_MUL_MAT at compile time
 *   ggml_backend_mi355x_load_iq_grids_from_ggml
 *                                            no counterpart: the reference reaches
 *                                            IQ3_XXS / IQ2_S only through ggml-cpu
 *                                            (src/xdna-gemv-engine.cpp:1388-1396)
 *   ggml_backend_mi355x_set_kernel_variant   no counterpart: selects the arithmetic
 *                                            (MI355X_OPT_VARIANT), e.g. ggml-cpu's
 *                                            Q8 activation numerics, which the
 *                                            reference takes from ggml-cpu when it
 *                                            is loaded (src/xdna-gemv-engine.cpp:
 *                                            1382-1399)
 *   ggml_backend_mi355x_set_group_mode       no counterpart: how graph_compute runs
 *                                            a group of single-row MUL_MATs whose
 *                                            activation and outputs are host-resident
 *
 * The compatibility API takes host pointers in `data` (like the reference's
 * harness); ggml graphs handed to graph_compute hold device pointers of
 * tensors allocated in this plugin's buffer type.
 */
#ifndef GGML_MI355X_H
#define GGML_MI355X_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MI355X_API __attribute__((visibility("default")))

struct ggml_backend_reg;
struct ggml_backend;
struct ggml_backend_buffer_type;
struct ggml_cgraph;

/* Op ids of the compatibility tensor struct (the reference harness values). */
#define GGML_MI355X_OP_NONE 0
#define GGML_MI355X_OP_RMS_NORM 15
#define GGML_MI355X_OP_MUL_MAT 18

/* Compatibility tensor (field order of the reference's ggml_tensor_xdna). */
struct ggml_tensor_mi355x {
    int32_t type;   /* ggml type id */
    int64_t ne[4];  /* elements per dimension */
    size_t nb[4];   /* byte strides (0 = contiguous) */
    uint32_t op;    /* GGML_MI355X_OP_* */
    int32_t op_params[16];
    int32_t flags;
    struct ggml_tensor_mi355x *src[10];
    void *data; /* host memory */
    char name[64];
    void *extra;
};

/* ---- dynamic-loading entry points (ggml backend API) ---------------------- */
GGML_MI355X_API struct ggml_backend_reg *ggml_backend_init(void);
/* 100 when a HIP device is present, 0 otherwise. */
GGML_MI355X_API int ggml_backend_score(void);

GGML_MI355X_API struct ggml_backend_reg *ggml_backend_mi355x_reg(void);
GGML_MI355X_API struct ggml_backend *ggml_backend_mi355x_init(size_t dev_num);
GGML_MI355X_API bool ggml_backend_is_mi355x(struct ggml_backend *backend);
GGML_MI355X_API void ggml_backend_mi355x_free(struct ggml_backend *backend);
GGML_MI355X_API struct ggml_backend_buffer_type *ggml_backend_mi355x_buffer_type(size_t dev_num);
GGML_MI355X_API struct ggml_backend_buffer_type *ggml_backend_mi355x_host_buffer_type(void);
/* Returns enum ggml_status: 0 success, -1 failed. */
GGML_MI355X_API int ggml_backend_mi355x_graph_compute(struct ggml_backend *backend, struct ggml_cgraph *cgraph);

/* ---- compatibility harness API -------------------------------------------- */
GGML_MI355X_API bool ggml_backend_mi355x_supports_op(struct ggml_backend *backend,
                                                     const struct ggml_tensor_mi355x *op);
GGML_MI355X_API bool ggml_backend_mi355x_compute_graph(struct ggml_backend *backend,
                                                       struct ggml_tensor_mi355x **nodes, size_t n_nodes);

/* ---- host-application hooks ------------------------------------------------
 * The value of GGML_OP_MUL_MAT in the host's ggml.  Resolved automatically
 * through ggml_op_name() when the host exports it; a host without it (a test
 * harness) sets it here.  Returns false for a negative value. */
GGML_MI355X_API bool ggml_backend_mi355x_set_op_mul_mat(int op);
/* Rebuilds the IQ3_XXS and IQ2_S grids by dequantizing probe blocks through
 * the host's exported ggml dequantize_row_iq3_xxs / dequantize_row_iq2_s,
 * cross-checks random blocks against them, and installs the grids.  Returns
 * the number of types enabled (0, 1 or 2). */
GGML_MI355X_API int ggml_backend_mi355x_load_iq_grids_from_ggml(void);
/* The kernel variant (MI355X_VARIANT_* of mi355x-gemv.h) of this backend's
 * GEMVs; also reachable through the registry's get_proc_address.  False for a
 * backend of another type or an unknown variant. */
GGML_MI355X_API bool ggml_backend_mi355x_set_kernel_variant(struct ggml_backend *backend, int variant);
/* Small tensors of the plugin's non-weight buffers (an activation row, a
 * group's outputs) stay in a page-locked host shadow of the buffer once the
 * host writes them or a single-row MUL_MAT outputs them, so a decode step
 * moves them with memcpy instead of copy commands.  graph_compute runs a
 * group of consecutive single-row MUL_MATs that share such an activation,
 * with every output host-resident, as
 *   GGML_MI355X_GROUPS_LAUNCH (default): one launch reading and writing the
 *     shadow through its device address, then a wait on a completion word;
 *   GGML_MI355X_GROUPS_SERVER: Q4_0 rows of a multiple of 256 values (up to
 *     16384) as one command to the device's persistent GEMV server
 *     (mi355x_server_gemv: no launch; returns with the outputs in the
 *     shadow); other groups as GGML_MI355X_GROUPS_LAUNCH.
 * Either way graph_compute returns after every kernel that touches a shadow
 * has finished.  False for a backend of another type or an unknown mode. */
#define GGML_MI355X_GROUPS_SERVER 0
#define GGML_MI355X_GROUPS_LAUNCH 1
GGML_MI355X_API bool ggml_backend_mi355x_set_group_mode(struct ggml_backend *backend, int mode);

#ifdef __cplusplus
}
#endif

#endif
