// Self-declared mirror of the ggml backend ABI this plugin implements.
//
// No ggml / llama.cpp checkout exists in the build image, so the structures
// the plugin fills are declared here.  Their field order follows the
// positional initialisers of the reference plugin, which compiled against
// llama.cpp 0ec4027a2 (backend API version 3):
//   ggml_backend_buffer_i        src/ggml-xdna.cpp:361-376
//   ggml_backend_buffer fields   src/ggml-xdna.cpp:398-403
//   ggml_backend_buffer_type_i   src/ggml-xdna.cpp:461-470
//   ggml_backend_buffer_type     src/ggml-xdna.cpp:479-489
//   ggml_backend_device_i        src/ggml-xdna.cpp:599-615
//   ggml_backend_dev_props       src/ggml-xdna.cpp:516-528
//   ggml_backend_reg(_i)         src/ggml-xdna.cpp:660-671
//   ggml_backend(_i)             src/ggml-xdna.cpp:696-713, 739-743
// Slots the plugin leaves empty are declared as untyped function pointers:
// only their position matters.  ggml_tensor / ggml_cgraph follow ggml.h /
// ggml-impl.h of the same line (tensor: 336 bytes; cgraph: n_nodes at byte 4,
// nodes at byte 16).  ggml type ids are GGUF on-disk values (stable); the
// GGML_OP_MUL_MAT value is NOT stable across ggml versions and is resolved
// at run time through ggml's exported ggml_op_name() (see ggml_mi355x.cpp).
#pragma once

#include <stddef.h>
#include <stdint.h>

extern "C" {

#define GGML_MAX_DIMS 4
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_SRC 10
#define GGML_MAX_NAME 64
#define GGML_MI355X_BACKEND_API_VERSION 3

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

// GGUF type ids used by this plugin
enum {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q3_K = 11,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_IQ3_XXS = 18,
    GGML_TYPE_IQ3_S = 21,
    GGML_TYPE_IQ2_S = 22,
    GGML_TYPE_IQ4_XS = 23,
};

enum ggml_backend_buffer_usage {
    GGML_BACKEND_BUFFER_USAGE_ANY = 0,
    GGML_BACKEND_BUFFER_USAGE_WEIGHTS = 1,
    GGML_BACKEND_BUFFER_USAGE_COMPUTE = 2,
};

// Only the value the plugin reports is given; GPU is 1 in every ggml line.
enum ggml_backend_dev_type {
    GGML_BACKEND_DEVICE_TYPE_CPU = 0,
    GGML_BACKEND_DEVICE_TYPE_GPU = 1,
};

struct ggml_backend_buffer;
struct ggml_backend_buffer_type;
struct ggml_backend_device;
struct ggml_backend_reg;
struct ggml_backend;
struct ggml_cgraph;

typedef struct ggml_backend_buffer *ggml_backend_buffer_t;
typedef struct ggml_backend_buffer_type *ggml_backend_buffer_type_t;
typedef struct ggml_backend_device *ggml_backend_dev_t;
typedef struct ggml_backend_reg *ggml_backend_reg_t;
typedef struct ggml_backend *ggml_backend_t;
typedef void *ggml_backend_event_t;
typedef void *ggml_backend_graph_plan_t;
typedef void (*ggml_abi_unused_fn)(void);

struct ggml_tensor {
    int32_t type;  // enum ggml_type
    struct ggml_backend_buffer *buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t nb[GGML_MAX_DIMS];
    int32_t op;  // enum ggml_op
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor *src[GGML_MAX_SRC];
    struct ggml_tensor *view_src;
    size_t view_offs;
    void *data;
    char name[GGML_MAX_NAME];
    void *extra;
    char padding[8];
};

struct ggml_cgraph {
    int size;
    int n_nodes;
    int n_leafs;
    struct ggml_tensor **nodes;
    // further members are not read by the plugin
};

typedef uint8_t ggml_guid[16];
typedef ggml_guid *ggml_guid_t;

struct ggml_backend_buffer_i {
    void (*free_buffer)(ggml_backend_buffer_t buffer);
    void *(*get_base)(ggml_backend_buffer_t buffer);
    enum ggml_status (*init_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor);
    void (*memset_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor, uint8_t value, size_t offset,
                          size_t size);
    void (*set_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor, const void *data, size_t offset,
                       size_t size);
    void (*get_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor *tensor, void *data, size_t offset,
                       size_t size);
    ggml_abi_unused_fn set_tensor_2d;
    ggml_abi_unused_fn get_tensor_2d;
    bool (*cpy_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor *src, struct ggml_tensor *dst);
    void (*clear)(ggml_backend_buffer_t buffer, uint8_t value);
    void (*reset)(ggml_backend_buffer_t buffer);
    ggml_abi_unused_fn set_tensor_n;
    ggml_abi_unused_fn get_tensor_n;
    ggml_abi_unused_fn cpy_tensor_n;
};

struct ggml_backend_buffer {
    struct ggml_backend_buffer_i iface;
    ggml_backend_buffer_type_t buft;
    void *context;
    size_t size;
    enum ggml_backend_buffer_usage usage;
};

struct ggml_backend_buffer_type_i {
    const char *(*get_name)(ggml_backend_buffer_type_t buft);
    ggml_backend_buffer_t (*alloc_buffer)(ggml_backend_buffer_type_t buft, size_t size);
    ggml_abi_unused_fn alloc_buffer_n;
    size_t (*get_alignment)(ggml_backend_buffer_type_t buft);
    size_t (*get_max_size)(ggml_backend_buffer_type_t buft);
    size_t (*get_alloc_size)(ggml_backend_buffer_type_t buft, const struct ggml_tensor *tensor);
    ggml_abi_unused_fn get_alloc_size_n;
    bool (*is_host)(ggml_backend_buffer_type_t buft);
};

struct ggml_backend_buffer_type {
    struct ggml_backend_buffer_type_i iface;
    ggml_backend_dev_t device;
    void *context;
};

struct ggml_backend_dev_caps {
    bool async;
    bool host_buffer;
    bool buffer_from_host_ptr;
    bool events;
    bool mmap_support;
};

struct ggml_backend_dev_props {
    const char *name;
    const char *description;
    enum ggml_backend_dev_type type;
    size_t memory_free;
    size_t memory_total;
    const char *device_id;
    struct ggml_backend_dev_caps caps;
};

struct ggml_backend_device_i {
    const char *(*get_name)(ggml_backend_dev_t dev);
    const char *(*get_description)(ggml_backend_dev_t dev);
    void (*get_memory)(ggml_backend_dev_t dev, size_t *free, size_t *total);
    enum ggml_backend_dev_type (*get_type)(ggml_backend_dev_t dev);
    void (*get_props)(ggml_backend_dev_t dev, struct ggml_backend_dev_props *props);
    ggml_backend_t (*init_backend)(ggml_backend_dev_t dev, const char *params);
    ggml_backend_buffer_type_t (*get_buffer_type)(ggml_backend_dev_t dev);
    ggml_backend_buffer_type_t (*get_host_buffer_type)(ggml_backend_dev_t dev);
    ggml_backend_buffer_t (*buffer_from_host_ptr)(ggml_backend_dev_t dev, void *ptr, size_t size,
                                                  size_t max_tensor_size);
    bool (*supports_op)(ggml_backend_dev_t dev, const struct ggml_tensor *op);
    bool (*supports_buft)(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft);
    bool (*offload_op)(ggml_backend_dev_t dev, const struct ggml_tensor *op);
    ggml_abi_unused_fn event_new;
    ggml_abi_unused_fn event_free;
    ggml_abi_unused_fn event_synchronize;
};

struct ggml_backend_device {
    struct ggml_backend_device_i iface;
    ggml_backend_reg_t reg;
    void *context;
};

struct ggml_backend_reg_i {
    const char *(*get_name)(ggml_backend_reg_t reg);
    size_t (*get_device_count)(ggml_backend_reg_t reg);
    ggml_backend_dev_t (*get_device)(ggml_backend_reg_t reg, size_t index);
    void *(*get_proc_address)(ggml_backend_reg_t reg, const char *name);
};

struct ggml_backend_reg {
    int api_version;
    struct ggml_backend_reg_i iface;
    void *context;
};

struct ggml_backend_i {
    const char *(*get_name)(ggml_backend_t backend);
    void (*free)(ggml_backend_t backend);
    void (*set_tensor_async)(ggml_backend_t backend, struct ggml_tensor *tensor, const void *data, size_t offset,
                             size_t size);
    void (*get_tensor_async)(ggml_backend_t backend, const struct ggml_tensor *tensor, void *data, size_t offset,
                             size_t size);
    ggml_abi_unused_fn set_tensor_2d_async;
    ggml_abi_unused_fn get_tensor_2d_async;
    ggml_abi_unused_fn cpy_tensor_async;
    void (*synchronize)(ggml_backend_t backend);
    ggml_abi_unused_fn graph_plan_create;
    ggml_abi_unused_fn graph_plan_free;
    ggml_abi_unused_fn graph_plan_update;
    ggml_abi_unused_fn graph_plan_compute;
    enum ggml_status (*graph_compute)(ggml_backend_t backend, struct ggml_cgraph *cgraph);
    ggml_abi_unused_fn event_record;
    ggml_abi_unused_fn event_wait;
    ggml_abi_unused_fn graph_optimize;
};

struct ggml_backend {
    ggml_guid_t guid;
    struct ggml_backend_i iface;
    ggml_backend_dev_t device;
    void *context;
};

}  // extern "C"

static_assert(sizeof(ggml_tensor) == 336, "ggml_tensor layout");
static_assert(offsetof(ggml_tensor, ne) == 16, "ggml_tensor::ne");
static_assert(offsetof(ggml_tensor, op) == 80, "ggml_tensor::op");
static_assert(offsetof(ggml_tensor, src) == 152, "ggml_tensor::src");
static_assert(offsetof(ggml_tensor, data) == 248, "ggml_tensor::data");
static_assert(offsetof(ggml_tensor, name) == 256, "ggml_tensor::name");
static_assert(offsetof(ggml_cgraph, n_nodes) == 4 && offsetof(ggml_cgraph, nodes) == 16, "ggml_cgraph");
static_assert(sizeof(ggml_backend_buffer_i) == 14 * sizeof(void *), "buffer_i slots");
static_assert(sizeof(ggml_backend_buffer_type_i) == 8 * sizeof(void *), "buffer_type_i slots");
static_assert(sizeof(ggml_backend_device_i) == 15 * sizeof(void *), "device_i slots");
static_assert(sizeof(ggml_backend_i) == 16 * sizeof(void *), "backend_i slots");
