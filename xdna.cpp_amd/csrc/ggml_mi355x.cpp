// ggml backend plugin for MI355X: registry, device, device/host buffer types,
// backend and graph_compute for single-row quantized MUL_MAT.  Host C++ only;
// all device work goes through the C-ABI of mi355x-gemv.h.
//
// Reference counterparts (random-unknown-username/xdna.cpp):
//   supports_op_impl       src/ggml-xdna.cpp:95-147
//   process_mul_mat_node   src/ggml-xdna.cpp:150-308
//   buffer / buffer type   src/ggml-xdna.cpp:316-489 (host memory there; HBM here)
//   device / registry      src/ggml-xdna.cpp:495-671
//   backend, entry points  src/ggml-xdna.cpp:677-844
#include "ggml_abi.h"

#include "ggml-mi355x.h"
#include "mi355x-gemv.h"

#include <dlfcn.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

namespace {

constexpr uint32_t kBackendMagic = 0x4D333535;  // "M355"
constexpr size_t kAlignment = 256;

// ---------------------------------------------------------------------------
// op id of GGML_OP_MUL_MAT in the host's ggml
// ---------------------------------------------------------------------------
std::atomic<int> g_op_mul_mat{-1};

int op_mul_mat() {
    int v = g_op_mul_mat.load(std::memory_order_relaxed);
    if (v >= 0) return v;
    if (const char *env = std::getenv("MI355X_GGML_OP_MUL_MAT")) {
        v = std::atoi(env);
        if (v >= 0) {
            g_op_mul_mat.store(v);
            return v;
        }
    }
    // ggml exports `const char *ggml_op_name(enum ggml_op)`; MUL_MAT sits well
    // inside its table in every ggml release, so the scan stops there.
    typedef const char *(*op_name_fn)(int);
    auto fn = reinterpret_cast<op_name_fn>(dlsym(RTLD_DEFAULT, "ggml_op_name"));
    if (fn) {
        for (int i = 0; i < 128; ++i) {
            const char *n = fn(i);
            if (n && std::strcmp(n, "MUL_MAT") == 0) {
                g_op_mul_mat.store(i);
                return i;
            }
        }
    }
    return -1;
}

bool trace_supports() {
    static const bool t = std::getenv("MI355X_TRACE_SUPPORTS") != nullptr;
    return t;
}
bool trace_nodes() {
    static const bool t = std::getenv("MI355X_TRACE_NODES") != nullptr;
    return t;
}

// ---------------------------------------------------------------------------
// weight formats
// ---------------------------------------------------------------------------
// Block size of a claimable weight type (0 = not claimable), bytes per block.
// Same table as the reference's type switch (src/ggml-xdna.cpp:185-254).
int block_values(int type) {
    switch (type) {
    case GGML_TYPE_Q4_0: return 32;
    case GGML_TYPE_Q4_K: case GGML_TYPE_Q5_K: case GGML_TYPE_Q3_K: case GGML_TYPE_Q6_K:
    case GGML_TYPE_IQ4_XS: case GGML_TYPE_IQ3_S: case GGML_TYPE_IQ3_XXS: case GGML_TYPE_IQ2_S:
        return 256;
    default: return 0;
    }
}

const char *type_name(int type) {
    switch (type) {
    case GGML_TYPE_Q4_0: return "Q4_0";
    case GGML_TYPE_Q4_K: return "Q4_K";
    case GGML_TYPE_Q5_K: return "Q5_K";
    case GGML_TYPE_Q3_K: return "Q3_K";
    case GGML_TYPE_Q6_K: return "Q6_K";
    case GGML_TYPE_IQ4_XS: return "IQ4_XS";
    case GGML_TYPE_IQ3_S: return "IQ3_S";
    case GGML_TYPE_IQ3_XXS: return "IQ3_XXS";
    case GGML_TYPE_IQ2_S: return "IQ2_S";
    default: return "?";
    }
}

// (block values, bytes per block) of any type ggml may place in our buffer,
// for byte-size computations; 0/0 for types this plugin does not know.
void type_geometry(int type, int64_t *blk, int64_t *bytes) {
    *blk = 1;
    *bytes = 0;
    switch (type) {
    case GGML_TYPE_F32: *bytes = 4; return;
    case GGML_TYPE_F16: case 30 /* BF16 */: *bytes = 2; return;
    case 24 /* I8 */: *bytes = 1; return;
    case 25 /* I16 */: *bytes = 2; return;
    case 26 /* I32 */: *bytes = 4; return;
    case 27 /* I64 */: case 28 /* F64 */: *bytes = 8; return;
    case 3 /* Q4_1 */: *blk = 32; *bytes = 20; return;
    case 6 /* Q5_0 */: *blk = 32; *bytes = 22; return;
    case 7 /* Q5_1 */: *blk = 32; *bytes = 24; return;
    case 8 /* Q8_0 */: *blk = 32; *bytes = 34; return;
    default: break;
    }
    const int bv = block_values(type);
    if (bv) {
        *blk = bv;
        *bytes = mi355x_row_bytes(type, bv);
    }
}

// ggml_nbytes of a tensor (row 0 in full, then strides of the other dims).
size_t tensor_nbytes(const ggml_tensor *t) {
    int64_t blk, bytes;
    type_geometry(t->type, &blk, &bytes);
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (t->ne[i] <= 0) return 0;
    typedef size_t (*nbytes_fn)(const ggml_tensor *);
    static auto *p_nbytes = reinterpret_cast<nbytes_fn>(dlsym(RTLD_DEFAULT, "ggml_nbytes"));
    if (bytes == 0) return p_nbytes ? p_nbytes(t) : 0;
    size_t n = static_cast<size_t>(t->ne[0] / blk) * static_cast<size_t>(bytes);
    for (int i = 1; i < GGML_MAX_DIMS; ++i) n += static_cast<size_t>(t->ne[i] - 1) * t->nb[i];
    return n;
}

// ---------------------------------------------------------------------------
// batch geometry of a MUL_MAT node
// ---------------------------------------------------------------------------
// A node multiplies activation batch (i2, i3) -- ne[2] x ne[3] of them, each
// M rows -- by weight matrix (i2 / r2, i3 / r3), r = activation batches per
// weight matrix (ggml's broadcast).  Byte strides left at 0 (the
// compatibility struct) mean densely packed.
inline int64_t extent(int64_t ne) { return ne > 0 ? ne : 1; }
inline size_t stride_or(size_t nb, size_t dense) { return nb != 0 ? nb : dense; }

template <typename T>
bool broadcast_ok(const T *op) {
    const auto *w = op->src[0];
    const auto *a = op->src[1];
    const int64_t b2 = extent(a->ne[2]), b3 = extent(a->ne[3]);
    return b2 % extent(w->ne[2]) == 0 && b3 % extent(w->ne[3]) == 0 && extent(op->ne[2]) == b2 &&
           extent(op->ne[3]) == b3;
}

struct BatchGeometry {
    int64_t batches2 = 1, batches3 = 1;   // activation batches
    int64_t per_w2 = 1, per_w3 = 1;       // activation batches per weight matrix
    size_t w_b2 = 0, w_b3 = 0;            // weight matrix strides
    size_t a_row = 0, a_b2 = 0, a_b3 = 0; // activation row / batch strides
    size_t o_row = 0, o_b2 = 0, o_b3 = 0; // output row / batch strides

    size_t weight_at(int64_t i2, int64_t i3) const {
        return static_cast<size_t>(i2 / per_w2) * w_b2 + static_cast<size_t>(i3 / per_w3) * w_b3;
    }
    size_t act_at(int64_t i2, int64_t i3) const {
        return static_cast<size_t>(i2) * a_b2 + static_cast<size_t>(i3) * a_b3;
    }
    size_t out_at(int64_t i2, int64_t i3) const {
        return static_cast<size_t>(i2) * o_b2 + static_cast<size_t>(i3) * o_b3;
    }
};

template <typename T>
BatchGeometry batch_geometry(const T *node, int64_t N, int64_t K, int64_t M, size_t row_bytes) {
    const auto *w = node->src[0];
    const auto *a = node->src[1];
    BatchGeometry g;
    g.batches2 = extent(a->ne[2]);
    g.batches3 = extent(a->ne[3]);
    g.per_w2 = g.batches2 / extent(w->ne[2]);
    g.per_w3 = g.batches3 / extent(w->ne[3]);
    g.w_b2 = stride_or(w->nb[2], static_cast<size_t>(N) * row_bytes);
    g.w_b3 = stride_or(w->nb[3], g.w_b2 * static_cast<size_t>(extent(w->ne[2])));
    g.a_row = stride_or(a->nb[1], static_cast<size_t>(K) * sizeof(float));
    g.a_b2 = stride_or(a->nb[2], g.a_row * static_cast<size_t>(M));
    g.a_b3 = stride_or(a->nb[3], g.a_b2 * static_cast<size_t>(g.batches2));
    g.o_row = stride_or(node->nb[1], static_cast<size_t>(N) * sizeof(float));
    g.o_b2 = stride_or(node->nb[2], g.o_row * static_cast<size_t>(M));
    g.o_b3 = stride_or(node->nb[3], g.o_b2 * static_cast<size_t>(g.batches2));
    return g;
}

// ---------------------------------------------------------------------------
// claim rule (src/ggml-xdna.cpp:95-147) on any tensor-like struct
// ---------------------------------------------------------------------------
template <typename T>
bool claim_mul_mat(const T *op, int mul_mat_id, bool weights_resident) {
    if (!op || mul_mat_id < 0 || static_cast<int>(op->op) != mul_mat_id) return false;
    const auto *src0 = op->src[0];
    const auto *src1 = op->src[1];
    if (!src0 || !src1) return false;
    if (src1->type != GGML_TYPE_F32) return false;
    if (src1->nb[0] != 0 && src1->nb[0] != sizeof(float)) return false;
    const int64_t K = src0->ne[0];
    const int64_t N = src0->ne[1];
    const int64_t M = src1->ne[1];
    // size cutoff: N >= 32 and N % 4 == 0; M == 1 unless the weights live in
    // this plugin's buffer (src/ggml-xdna.cpp:110-112)
    if (N < 32 || N % 4 != 0) return false;
    if (!weights_resident && M != 1) return false;
    // weight batches broadcast over activation batches as in ggml (each
    // weight matrix serves a whole number of them); anything else would
    // index weights past the tensor
    if (!broadcast_ok(op)) return false;
    const int bv = block_values(src0->type);
    if (bv == 0 || K % bv != 0) return false;
    if (!mi355x_type_ready(src0->type)) return false;
    const int64_t rb = mi355x_row_bytes(src0->type, K);
    return src0->nb[1] == 0 || static_cast<int64_t>(src0->nb[1]) == rb;
}

// ---------------------------------------------------------------------------
// devices
// ---------------------------------------------------------------------------
struct DevCtx {
    int device = 0;
    std::string name, description, pci;
    ggml_backend_device dev{};
    ggml_backend_buffer_type buft{};
    ggml_backend_buffer_type host_buft{};
    std::mutex mu;
    mi355x_ctx *xfer = nullptr;  // context for buffer transfers

    mi355x_ctx *transfer_ctx() {
        std::lock_guard<std::mutex> lk(mu);
        if (!xfer && mi355x_ctx_create(device, &xfer) != MI355X_OK) xfer = nullptr;
        return xfer;
    }

    // The device's persistent GEMV server, shared by its backends (one
    // resident kernel per device: it holds every CU), on a context of its
    // own whose variant is set per command; made on first use.  While it is
    // resident a launched GEMV kernel would find no room on the CUs until
    // the server's idle exit, so the launch paths stop it first.
    std::mutex srv_mu;
    mi355x_ctx *srv_ctx = nullptr;
    mi355x_server *srv = nullptr;
    bool srv_failed = false;
    bool srv_active = false;  // a command ran since the last stop
    int backends = 0;         // live backends on the device (mu)
    static constexpr int64_t kServerMaxK = 16384;

    mi355x_server *server() {  // srv_mu held
        if (!srv && !srv_failed) {
            if (mi355x_ctx_create(device, &srv_ctx) != MI355X_OK ||
                mi355x_server_create(srv_ctx, kServerMaxK, &srv) != MI355X_OK) {
                srv = nullptr;
                srv_failed = true;
            }
        }
        return srv;
    }
    // Before a launch on this device: the server leaves the CUs.
    void yield_cus() {
        std::lock_guard<std::mutex> lk(srv_mu);
        if (srv && srv_active) {
            if (mi355x_server_stop(srv) != MI355X_OK)
                std::fprintf(stderr, "[mi355x error] server stop: %s\n", mi355x_last_error());
            srv_active = false;
        }
    }
};

ggml_backend_reg g_reg{};
std::vector<DevCtx *> g_devs;
std::once_flag g_reg_once;

void init_registry();

DevCtx *dev_ctx(ggml_backend_dev_t dev) { return dev ? static_cast<DevCtx *>(dev->context) : nullptr; }
DevCtx *buft_dev(ggml_backend_buffer_type_t buft) {
    return buft && buft->device ? static_cast<DevCtx *>(buft->device->context) : nullptr;
}

// ---------------------------------------------------------------------------
// device buffer (HBM)
// ---------------------------------------------------------------------------
// Disjoint byte ranges [start, end) of a buffer, merged where they touch.
class RangeSet {
  public:
    bool empty() const { return r_.empty(); }
    void clear() { r_.clear(); }
    // [a, b) lies inside one range
    bool covers(size_t a, size_t b) const {
        if (a >= b) return true;
        auto it = r_.upper_bound(a);
        if (it == r_.begin()) return false;
        --it;
        return it->second >= b;
    }
    // some byte of [a, b) lies in a range
    bool touches(size_t a, size_t b) const {
        if (a >= b || r_.empty()) return false;
        auto it = r_.lower_bound(b);
        if (it == r_.begin()) return false;
        --it;
        return it->second > a;
    }
    void remove(size_t a, size_t b) {
        if (a >= b) return;
        auto it = r_.upper_bound(a);
        if (it != r_.begin()) {
            auto p = std::prev(it);
            if (p->first < a && p->second > a) {
                const size_t end = p->second;
                p->second = a;
                if (end > b) {
                    r_.emplace(b, end);
                    return;
                }
            }
        }
        it = r_.lower_bound(a);
        while (it != r_.end() && it->first < b) {
            if (it->second > b) {
                const size_t end = it->second;
                r_.erase(it);
                r_.emplace(b, end);
                return;
            }
            it = r_.erase(it);
        }
    }
    void add(size_t a, size_t b) {
        if (a >= b) return;
        remove(a, b);
        auto it = r_.emplace(a, b).first;
        if (it != r_.begin()) {
            auto p = std::prev(it);
            if (p->second == a) {
                p->second = b;
                r_.erase(it);
                it = p;
            }
        }
        auto n = std::next(it);
        if (n != r_.end() && n->first == it->second) {
            it->second = n->second;
            r_.erase(n);
        }
    }
    // the parts of [a, b) that lie in ranges, in order
    std::vector<std::pair<size_t, size_t>> parts(size_t a, size_t b) const {
        std::vector<std::pair<size_t, size_t>> out;
        if (a >= b) return out;
        auto it = r_.upper_bound(a);
        if (it != r_.begin()) --it;
        for (; it != r_.end() && it->first < b; ++it) {
            const size_t lo = std::max(a, it->first), hi = std::min(b, it->second);
            if (lo < hi) out.emplace_back(lo, hi);
        }
        return out;
    }

  private:
    std::map<size_t, size_t> r_;  // start -> end
};

// Host-resident ranges of a device buffer.  A decode step hands the device
// one activation row (a few KB) per group of MUL_MATs and takes the group's
// outputs back; a copy command each way costs more than the GEMV itself.  A
// buffer that does not hold weights (ggml's compute and KV buffers) therefore
// gets a page-locked host shadow of its own size on first use, and the
// bytes of tensors of at most kMirrorMax bytes that the host writes
// (set_tensor, memset) or a single-row MUL_MAT outputs live there: their
// range of the buffer is "host-resident".  GEMV kernels read activations from
// and write outputs to the shadow through its device address (the persistent
// server takes the activation from the shadow directly), and get_tensor reads
// it with a memcpy.  The device bytes of a host-resident range are stale: any
// access that needs them (a larger or strided MUL_MAT, a device-to-device
// copy, reads of prepacked tensors) first copies the range to the device and
// drops it from the set.  Every path that reads or writes a buffer's bytes
// goes through this file, so the set is the whole truth.
constexpr size_t kMirrorMax = size_t(1) << 20;
constexpr size_t kShadowMaxBuffer = size_t(256) << 20;

struct BufCtx {
    DevCtx *dc = nullptr;
    void *base = nullptr;  // device pointer (or pinned host pointer)
    size_t size = 0;
    bool host = false;
    bool own_struct = false;  // ggml_backend_buffer allocated here (no ggml-base)
    std::mutex smu;           // shadow, shadow_dev, resident
    uint8_t *shadow = nullptr;      // page-locked host copy, made on first use
    uint8_t *shadow_dev = nullptr;  // its device address
    bool shadow_failed = false;
    RangeSet resident;  // host-resident byte ranges (offsets into the buffer)

    size_t off(const void *p) const {
        return static_cast<size_t>(static_cast<const uint8_t *>(p) - static_cast<const uint8_t *>(base));
    }
};

void log_error(const char *what) {
    std::fprintf(stderr, "[mi355x error] %s: %s\n", what, mi355x_last_error());
}

// The shadow of a buffer that may hold host-resident ranges, made on first
// use (smu held): none for host buffers, weight buffers and buffers larger
// than kShadowMaxBuffer.
bool shadow_ready(ggml_backend_buffer_t buffer, BufCtx *bc) {
    if (bc->shadow) return true;
    if (bc->host || bc->shadow_failed || bc->size > kShadowMaxBuffer ||
        buffer->usage == GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
        return false;
    void *h = nullptr, *d = nullptr;
    if (mi355x_host_malloc(bc->size, &h) != MI355X_OK || mi355x_host_device_ptr(h, &d) != MI355X_OK) {
        if (h) mi355x_host_free(h);
        bc->shadow_failed = true;
        return false;
    }
    bc->shadow = static_cast<uint8_t *>(h);
    bc->shadow_dev = static_cast<uint8_t *>(d);
    return true;
}

// Copies the host-resident parts of [a, b) to the device with `x` and drops
// them from the set (smu held).  False if a copy failed (that part stays
// host-resident).
bool materialise(BufCtx *bc, mi355x_ctx *x, size_t a, size_t b) {
    bool ok = true;
    for (const auto &p : bc->resident.parts(a, b)) {
        if (mi355x_memcpy_h2d(x, static_cast<uint8_t *>(bc->base) + p.first, bc->shadow + p.first,
                              p.second - p.first) != MI355X_OK) {
            log_error("materialise host-resident range");
            ok = false;
            continue;
        }
        bc->resident.remove(p.first, p.second);
    }
    return ok;
}

// The base tensor whose rows define the resident layout of `t`'s bytes.
const ggml_tensor *layout_base(const ggml_tensor *t) { return t->view_src ? t->view_src : t; }

// Number of K-value rows of a contiguous weight tensor.
int64_t weight_rows(const ggml_tensor *t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

// Tensors whose resident byte order differs from ggml's: every weight type
// the kernels read (Q4_0 code/scale planes, K/IQ field planes).
bool prepacked(const ggml_tensor *t) {
    const ggml_tensor *b = layout_base(t);
    const int bv = block_values(b->type);
    return bv != 0 && t->type == b->type && b->ne[0] % bv == 0;
}

void buf_free(ggml_backend_buffer_t buffer) {
    if (!buffer || !buffer->context) return;
    auto *bc = static_cast<BufCtx *>(buffer->context);
    if (bc->host) {
        mi355x_host_free(bc->base);
    } else if (mi355x_ctx *x = bc->dc->transfer_ctx()) {
        mi355x_free(x, bc->base);
    }
    if (bc->shadow) mi355x_host_free(bc->shadow);
    const bool own = bc->own_struct;
    delete bc;
    buffer->context = nullptr;
    if (own) delete buffer;
}

void *buf_get_base(ggml_backend_buffer_t buffer) {
    return buffer && buffer->context ? static_cast<BufCtx *>(buffer->context)->base : nullptr;
}

enum ggml_status buf_init_tensor(ggml_backend_buffer_t, ggml_tensor *) { return GGML_STATUS_SUCCESS; }

// Host -> tensor bytes [offset, offset+size) in ggml encoding, on the stream
// of `x` (synchronous).  Q4_0 weights are scattered into the resident layout.
void upload(mi355x_ctx *x, ggml_tensor *tensor, const void *data, size_t offset, size_t size) {
    uint8_t *dst = static_cast<uint8_t *>(tensor->data) + offset;
    if (prepacked(tensor)) {
        const ggml_tensor *b = layout_base(tensor);
        const size_t o = static_cast<size_t>(dst - static_cast<const uint8_t *>(b->data));
        if (mi355x_prepack_from_host(x, b->type, weight_rows(b), b->ne[0], b->data, data, o, size))
            log_error("set_tensor: prepack");
        return;
    }
    if (mi355x_memcpy_h2d(x, dst, data, size)) log_error("set_tensor");
}

// Tensor bytes [offset, offset+size) in ggml encoding -> host (synchronous).
void download(mi355x_ctx *x, const ggml_tensor *tensor, void *data, size_t offset, size_t size) {
    const uint8_t *src = static_cast<const uint8_t *>(tensor->data) + offset;
    if (prepacked(tensor)) {
        const ggml_tensor *b = layout_base(tensor);
        const size_t o = static_cast<size_t>(src - static_cast<const uint8_t *>(b->data));
        if (mi355x_unpack_to_host(x, b->type, weight_rows(b), b->ne[0], b->data, data, o, size))
            log_error("get_tensor: unpack");
        return;
    }
    if (mi355x_memcpy_d2h(x, data, src, size)) log_error("get_tensor");
}

// A tensor whose bytes may be host-resident: not prepacked, at most
// kMirrorMax bytes.
bool mirrorable(const ggml_tensor *t) { return !prepacked(t) && tensor_nbytes(t) <= kMirrorMax; }

// The byte range a write to `t` may change in the device bytes: exactly
// [offset, offset + size) of t, or, for prepacked tensors (a row-local
// permutation), the whole base tensor.
std::pair<size_t, size_t> device_span(const BufCtx *bc, const ggml_tensor *t, size_t offset, size_t size) {
    if (prepacked(t)) {
        const ggml_tensor *b = layout_base(t);
        const size_t a = bc->off(b->data);
        return {a, a + tensor_nbytes(b)};
    }
    const size_t a = bc->off(t->data) + offset;
    return {a, a + size};
}

// Host write of [offset, offset + size) of a mirrorable tensor into the
// shadow (the range becomes host-resident); false if the buffer has no
// shadow (the caller writes the device).
bool write_host_resident(ggml_backend_buffer_t buffer, BufCtx *bc, ggml_tensor *t, const void *data, size_t offset,
                         size_t size) {
    if (!mirrorable(t)) return false;
    std::lock_guard<std::mutex> lk(bc->smu);
    if (!shadow_ready(buffer, bc)) return false;
    const size_t a = bc->off(t->data) + offset;
    std::memcpy(bc->shadow + a, data, size);
    bc->resident.add(a, a + size);
    return true;
}

// After a device write of (part of) `t`: its device bytes are current.
void device_written(BufCtx *bc, const ggml_tensor *t, size_t offset, size_t size) {
    std::lock_guard<std::mutex> lk(bc->smu);
    if (bc->resident.empty()) return;
    const auto sp = device_span(bc, t, offset, size);
    bc->resident.remove(sp.first, sp.second);
}

// Before a device read of (part of) `t`: copies its host-resident bytes to
// the device with `x`.
bool device_current(BufCtx *bc, mi355x_ctx *x, const ggml_tensor *t, size_t offset, size_t size) {
    std::lock_guard<std::mutex> lk(bc->smu);
    if (bc->resident.empty()) return true;
    const auto sp = device_span(bc, t, offset, size);
    return materialise(bc, x, sp.first, sp.second);
}

void buf_set_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, const void *data, size_t offset,
                    size_t size) {
    if (!buffer || !tensor || !tensor->data || !data || size == 0) return;
    auto *bc = static_cast<BufCtx *>(buffer->context);
    if (bc->host) {
        std::memcpy(static_cast<uint8_t *>(tensor->data) + offset, data, size);
        return;
    }
    if (write_host_resident(buffer, bc, tensor, data, offset, size)) return;
    mi355x_ctx *x = bc->dc->transfer_ctx();
    if (!x) return log_error("set_tensor: no device context");
    if (prepacked(tensor)) bc->dc->yield_cus();  // the scatter kernel needs CUs
    upload(x, tensor, data, offset, size);
    device_written(bc, tensor, offset, size);
}

void buf_get_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *tensor, void *data, size_t offset,
                    size_t size) {
    if (!buffer || !tensor || !tensor->data || !data || size == 0) return;
    auto *bc = static_cast<BufCtx *>(buffer->context);
    if (bc->host) {
        std::memcpy(data, static_cast<const uint8_t *>(tensor->data) + offset, size);
        return;
    }
    mi355x_ctx *x = bc->dc->transfer_ctx();
    if (!prepacked(tensor)) {
        const size_t a = bc->off(tensor->data) + offset;
        {
            std::lock_guard<std::mutex> lk(bc->smu);
            if (bc->resident.covers(a, a + size)) {
                std::memcpy(data, bc->shadow + a, size);
                return;
            }
        }
        if (!x) return log_error("get_tensor: no device context");
        // device bytes, then the host-resident parts over them
        download(x, tensor, data, offset, size);
        std::lock_guard<std::mutex> lk(bc->smu);
        for (const auto &p : bc->resident.parts(a, a + size))
            std::memcpy(static_cast<uint8_t *>(data) + (p.first - a), bc->shadow + p.first, p.second - p.first);
        return;
    }
    if (!x) return log_error("get_tensor: no device context");
    device_current(bc, x, tensor, offset, size);
    bc->dc->yield_cus();  // the gather kernel needs CUs
    download(x, tensor, data, offset, size);
}

void buf_memset_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, uint8_t value, size_t offset,
                       size_t size) {
    if (!buffer || !tensor || !tensor->data || size == 0) return;
    auto *bc = static_cast<BufCtx *>(buffer->context);
    uint8_t *dst = static_cast<uint8_t *>(tensor->data) + offset;
    if (bc->host) {
        std::memset(dst, value, size);
        return;
    }
    if (mirrorable(tensor)) {
        std::lock_guard<std::mutex> lk(bc->smu);
        if (shadow_ready(buffer, bc)) {
            const size_t a = bc->off(tensor->data) + offset;
            std::memset(bc->shadow + a, value, size);
            bc->resident.add(a, a + size);
            return;
        }
    }
    if (prepacked(tensor)) {
        // fill the ggml bytes with `value` through the prepack permutation
        const size_t chunk = std::min<size_t>(size, size_t(16) << 20);
        std::vector<uint8_t> fill(chunk, value);
        for (size_t done = 0; done < size; done += chunk)
            buf_set_tensor(buffer, tensor, fill.data(), offset + done, std::min(chunk, size - done));
        return;
    }
    mi355x_ctx *x = bc->dc->transfer_ctx();
    if (!x || mi355x_fill(x, dst, value, size) || mi355x_ctx_sync(x)) return log_error("memset_tensor");
    device_written(bc, tensor, offset, size);
}

bool buf_cpy_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *src, ggml_tensor *dst) {
    // device-to-device copies between tensors of this plugin on one device;
    // both sides share the resident layout when their rows match
    if (!buffer || !src || !dst || !src->buffer || !src->data || !dst->data) return false;
    auto *bc = static_cast<BufCtx *>(buffer->context);
    if (bc->host || src->buffer->iface.get_base != buffer->iface.get_base) return false;
    auto *sbc = static_cast<BufCtx *>(src->buffer->context);
    if (!sbc || sbc->host || sbc->dc != bc->dc) return false;
    if (prepacked(src) != prepacked(dst)) return false;
    if (prepacked(src) && (src->view_src || dst->view_src || src->ne[0] != dst->ne[0])) return false;
    const size_t n = tensor_nbytes(src);
    if (n != tensor_nbytes(dst)) return false;
    mi355x_ctx *x = bc->dc->transfer_ctx();
    if (!x || !device_current(sbc, x, src, 0, n)) return false;
    if (mi355x_memcpy_d2d(x, dst->data, src->data, n) != MI355X_OK) return false;
    device_written(bc, dst, 0, n);
    return true;
}

void buf_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    if (!buffer || !buffer->context) return;
    auto *bc = static_cast<BufCtx *>(buffer->context);
    if (bc->host) {
        std::memset(bc->base, value, bc->size);
        return;
    }
    mi355x_ctx *x = bc->dc->transfer_ctx();
    if (!x || mi355x_fill(x, bc->base, value, bc->size) || mi355x_ctx_sync(x)) return log_error("clear");
    std::lock_guard<std::mutex> lk(bc->smu);
    bc->resident.clear();
}

const ggml_backend_buffer_i kBufferIface = {
    /* .free_buffer   = */ buf_free,
    /* .get_base      = */ buf_get_base,
    /* .init_tensor   = */ buf_init_tensor,
    /* .memset_tensor = */ buf_memset_tensor,
    /* .set_tensor    = */ buf_set_tensor,
    /* .get_tensor    = */ buf_get_tensor,
    /* .set_tensor_2d = */ nullptr,
    /* .get_tensor_2d = */ nullptr,
    /* .cpy_tensor    = */ buf_cpy_tensor,
    /* .clear         = */ buf_clear,
    /* .reset         = */ nullptr,
    /* .set_tensor_n  = */ nullptr,
    /* .get_tensor_n  = */ nullptr,
    /* .cpy_tensor_n  = */ nullptr,
};

// Buffers are made by ggml-base's ggml_backend_buffer_init when the host
// exports it (ggml then owns and deletes the struct); otherwise here.
ggml_backend_buffer_t make_buffer(ggml_backend_buffer_type_t buft, BufCtx *bc, size_t size) {
    typedef ggml_backend_buffer_t (*init_fn)(ggml_backend_buffer_type_t, ggml_backend_buffer_i, void *, size_t);
    static auto *p_init = reinterpret_cast<init_fn>(dlsym(RTLD_DEFAULT, "ggml_backend_buffer_init"));
    if (p_init) return p_init(buft, kBufferIface, bc, size);
    auto *buf = new (std::nothrow) ggml_backend_buffer{kBufferIface, buft, bc, size, GGML_BACKEND_BUFFER_USAGE_ANY};
    if (buf) bc->own_struct = true;
    return buf;
}

const char *buft_get_name(ggml_backend_buffer_type_t buft) {
    DevCtx *dc = buft_dev(buft);
    return buft == (dc ? &dc->host_buft : nullptr) ? "MI355X_Host" : "MI355X";
}

ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    DevCtx *dc = buft_dev(buft);
    if (!dc) return nullptr;
    const bool host = buft == &dc->host_buft;
    void *p = nullptr;
    if (host) {
        if (mi355x_host_malloc(size, &p) != MI355X_OK) return log_error("alloc_buffer (host)"), nullptr;
    } else {
        mi355x_ctx *x = dc->transfer_ctx();
        if (!x || mi355x_malloc(x, size, &p) != MI355X_OK) return log_error("alloc_buffer"), nullptr;
    }
    auto *bc = new (std::nothrow) BufCtx();
    if (bc) {
        bc->dc = dc;
        bc->base = p;
        bc->size = size;
        bc->host = host;
    }
    ggml_backend_buffer_t buf = bc ? make_buffer(buft, bc, size) : nullptr;
    if (!buf) {
        if (host) mi355x_host_free(p);
        else mi355x_free(dc->transfer_ctx(), p);
        delete bc;
    }
    return buf;
}

size_t buft_get_alignment(ggml_backend_buffer_type_t) { return kAlignment; }
size_t buft_get_max_size(ggml_backend_buffer_type_t) { return SIZE_MAX; }
size_t buft_get_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor *t) { return t ? tensor_nbytes(t) : 0; }
bool buft_is_host(ggml_backend_buffer_type_t buft) {
    DevCtx *dc = buft_dev(buft);
    return dc && buft == &dc->host_buft;
}

const ggml_backend_buffer_type_i kBufferTypeIface = {
    /* .get_name         = */ buft_get_name,
    /* .alloc_buffer     = */ buft_alloc_buffer,
    /* .alloc_buffer_n   = */ nullptr,
    /* .get_alignment    = */ buft_get_alignment,
    /* .get_max_size     = */ buft_get_max_size,
    /* .get_alloc_size   = */ buft_get_alloc_size,
    /* .get_alloc_size_n = */ nullptr,
    /* .is_host          = */ buft_is_host,
};

bool in_our_device_buffer(const ggml_tensor *t) {
    if (!t || !t->buffer || !t->buffer->buft) return false;
    DevCtx *dc = buft_dev(t->buffer->buft);
    if (!dc || t->buffer->buft != &dc->buft) return false;
    return std::find(g_devs.begin(), g_devs.end(), dc) != g_devs.end();
}

// ---------------------------------------------------------------------------
// backend
// ---------------------------------------------------------------------------
struct BackendCtx {
    uint32_t magic = kBackendMagic;
    DevCtx *dc = nullptr;
    mi355x_ctx *ctx = nullptr;
    std::mutex mu;
    // device scratch for the compatibility path (host-pointer graphs)
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    // Pinned bounce memory of the async tensor copies: set_tensor_async
    // copies the caller's bytes into it and enqueues the upload;
    // get_tensor_async enqueues the download into it and synchronize copies
    // the bytes out to the caller (ggml's contract: the destination is read
    // after synchronize).  Slices are handed out in order and released
    // together at synchronize.
    static constexpr size_t kPinBytes = size_t(32) << 20;
    uint8_t *pin = nullptr;
    size_t pin_used = 0;
    struct Pending {
        void *dst;
        const void *src;
        size_t n;
    };
    std::vector<Pending> pending;
    // something was enqueued on the stream since the last completed wait
    bool queued = false;
    // persistent GEMV server for single-row Q4_0 groups whose activation and
    // outputs are host-resident (made on first use; none where the device
    // has no cooperative launch)
    int variant = MI355X_VARIANT_AUTO;
    // launches measured ahead of server commands for the 3B decode (285-290
    // against 279-287 tok/s on the same boxes)
    int group_mode = GGML_MI355X_GROUPS_LAUNCH;

    ~BackendCtx() {
        if (ctx) {
            // queued work ends before the bounce memory goes; downloads never
            // collected by a synchronize are dropped, not copied: their
            // destinations may be gone with the caller
            if (mi355x_ctx_sync(ctx) != MI355X_OK) log_error("backend free: sync");
            if (!pending.empty())
                std::fprintf(stderr, "[mi355x error] backend freed with %zu get_tensor_async result(s) not "
                                     "synchronized; dropped\n", pending.size());
            pending.clear();
            if (scratch) mi355x_free(ctx, scratch);
            mi355x_ctx_destroy(ctx);
        }
        if (pin) mi355x_host_free(pin);
        magic = 0;
    }

    // A 256-byte aligned slice of the bounce memory, or null (too large, or
    // no pinned memory): the caller takes the synchronous path.
    uint8_t *take(size_t n) {
        if (!pin && mi355x_host_malloc(kPinBytes, reinterpret_cast<void **>(&pin)) != MI355X_OK) pin = nullptr;
        if (!pin || n > kPinBytes) return nullptr;
        if (pin_used + n > kPinBytes && flush() != 0) return nullptr;
        uint8_t *p = pin + pin_used;
        pin_used = (pin_used + n + 255) & ~size_t(255);
        return p;
    }

    // Waits for everything queued, hands the downloads to their callers and
    // frees the bounce memory.
    int flush() {
        if (!ctx) return -1;
        const int rc = mi355x_ctx_fence(ctx);
        if (rc == MI355X_OK) queued = false;
        for (const Pending &p : pending) std::memcpy(p.dst, p.src, p.n);
        pending.clear();
        pin_used = 0;
        return rc == MI355X_OK ? 0 : -1;
    }


    void *ensure_scratch(size_t bytes) {
        if (scratch_bytes >= bytes) return scratch;
        if (scratch) mi355x_free(ctx, scratch);
        scratch = nullptr;
        scratch_bytes = 0;
        if (mi355x_malloc(ctx, bytes, &scratch) != MI355X_OK) return nullptr;
        scratch_bytes = bytes;
        return scratch;
    }
};

ggml_guid_t backend_guid() {
    static ggml_guid guid = {0x4d, 0x49, 0x33, 0x35, 0x35, 0x58, 0x2d, 0x67,
                             0x65, 0x6d, 0x76, 0x2d, 0x71, 0x75, 0x61, 0x6e};
    return &guid;
}

BackendCtx *backend_ctx(ggml_backend_t backend) {
    if (!backend || !backend->guid) return nullptr;
    if (std::memcmp(backend->guid, backend_guid(), sizeof(ggml_guid)) != 0) return nullptr;
    auto *bc = static_cast<BackendCtx *>(backend->context);
    return bc && bc->magic == kBackendMagic ? bc : nullptr;
}

const char *backend_get_name(ggml_backend_t backend) {
    BackendCtx *bc = backend_ctx(backend);
    return bc ? bc->dc->name.c_str() : "MI355X";
}

void backend_free(ggml_backend_t backend) {
    BackendCtx *bc = backend_ctx(backend);
    if (!bc) return;
    DevCtx *dc = bc->dc;
    delete bc;
    delete backend;
    // the last backend of the device: its server leaves the CUs
    bool last;
    {
        std::lock_guard<std::mutex> lk(dc->mu);
        last = --dc->backends == 0;
    }
    if (last) dc->yield_cus();
}

// Copies for tensors in this backend's device memory run on the backend's own
// stream, so they are ordered after the kernels already queued there (an
// activation upload cannot overtake the GEMV still reading the previous one).
// They complete before returning.
bool on_backend_device(BackendCtx *bc, const ggml_tensor *t) {
    return in_our_device_buffer(t) && buft_dev(t->buffer->buft) == bc->dc;
}

void backend_set_tensor_async(ggml_backend_t backend, ggml_tensor *tensor, const void *data, size_t offset,
                              size_t size) {
    BackendCtx *bc = backend_ctx(backend);
    if (!bc || !tensor || !tensor->buffer || !tensor->data || !data || size == 0) return;
    if (!on_backend_device(bc, tensor)) return buf_set_tensor(tensor->buffer, tensor, data, offset, size);
    std::lock_guard<std::mutex> lk(bc->mu);
    auto *buf = static_cast<BufCtx *>(tensor->buffer->context);
    // an activation row: into the buffer's shadow, nothing enqueued (no
    // queued kernel reads the shadow: graph_compute waits for every kernel
    // that does)
    if (write_host_resident(tensor->buffer, buf, tensor, data, offset, size)) return;
    if (!prepacked(tensor)) {
        if (uint8_t *b = bc->take(size)) {
            std::memcpy(b, data, size);
            if (mi355x_memcpy_h2d_async(bc->ctx, static_cast<uint8_t *>(tensor->data) + offset, b, size))
                log_error("set_tensor_async");
            bc->queued = true;
            device_written(buf, tensor, offset, size);
            return;
        }
    }
    if (prepacked(tensor)) bc->dc->yield_cus();  // the scatter kernel needs CUs
    upload(bc->ctx, tensor, data, offset, size);
    device_written(buf, tensor, offset, size);
}

void backend_get_tensor_async(ggml_backend_t backend, const ggml_tensor *tensor, void *data, size_t offset,
                              size_t size) {
    BackendCtx *bc = backend_ctx(backend);
    if (!bc || !tensor || !tensor->buffer || !tensor->data || !data || size == 0) return;
    if (!on_backend_device(bc, tensor)) {
        if (mi355x_ctx_sync(bc->ctx)) log_error("get_tensor_async: sync");
        return buf_get_tensor(tensor->buffer, tensor, data, offset, size);
    }
    std::lock_guard<std::mutex> lk(bc->mu);
    auto *buf = static_cast<BufCtx *>(tensor->buffer->context);
    if (!prepacked(tensor)) {
        {
            // host-resident: final already (graph_compute returns after every
            // kernel that writes the shadow)
            std::lock_guard<std::mutex> sl(buf->smu);
            const size_t a = buf->off(tensor->data) + offset;
            if (buf->resident.covers(a, a + size)) {
                std::memcpy(data, buf->shadow + a, size);
                return;
            }
        }
        if (!device_current(buf, bc->ctx, tensor, offset, size)) return;
        if (uint8_t *b = bc->take(size)) {
            if (mi355x_memcpy_d2h_async(bc->ctx, b, static_cast<const uint8_t *>(tensor->data) + offset, size))
                return log_error("get_tensor_async");
            bc->queued = true;
            bc->pending.push_back({data, b, size});
            return;
        }
    }
    if (!device_current(buf, bc->ctx, tensor, offset, size)) return;
    if (prepacked(tensor)) bc->dc->yield_cus();  // the gather kernel needs CUs
    download(bc->ctx, tensor, data, offset, size);
}

void backend_synchronize(ggml_backend_t backend) {
    BackendCtx *bc = backend_ctx(backend);
    if (!bc) return;
    std::lock_guard<std::mutex> lk(bc->mu);
    if (!bc->queued && bc->pending.empty()) return;  // nothing in flight
    if (bc->flush()) log_error("synchronize");
}

// One MUL_MAT node: validation and batch/row iteration of the reference's
// process_mul_mat_node (src/ggml-xdna.cpp:150-308).  `host` selects the
// compatibility path, whose data pointers are host memory.
template <typename T>
bool process_mul_mat(BackendCtx *bc, T *node, bool host) {
    auto *src0 = node->src[0];
    auto *src1 = node->src[1];
    if (!src0 || !src1) {
        std::fprintf(stderr, "[mi355x error] node '%s' missing src0/src1\n", node->name);
        return false;
    }
    if (src1->type != GGML_TYPE_F32) {
        std::fprintf(stderr, "[mi355x error] node '%s' src1 type %d != F32\n", node->name, src1->type);
        return false;
    }
    if (!node->data || !src0->data || !src1->data) {
        std::fprintf(stderr, "[mi355x error] node '%s' null data ptrs: node->data=%p src0->data=%p src1->data=%p\n",
                     node->name, node->data, src0->data, src1->data);
        return false;
    }
    const int64_t K = src0->ne[0];
    const int64_t N = src0->ne[1];
    const int64_t M = src1->ne[1];
    if (M == 0 || N == 0) return true;
    if (M < 0 || N < 0 || K < 0) {
        std::fprintf(stderr, "[mi355x error] node '%s' negative dim: M=%ld N=%ld K=%ld\n", node->name, (long)M,
                     (long)N, (long)K);
        return false;
    }
    const int type = src0->type;
    const int bv = block_values(type);
    if (bv == 0) {
        std::fprintf(stderr, "[mi355x error] node '%s' unsupported src0 type=%d\n", node->name, type);
        return false;
    }
    if (K % bv != 0) {
        std::fprintf(stderr, "[mi355x error] node '%s' %s K=%ld not div by %d\n", node->name, type_name(type),
                     (long)K, bv);
        return false;
    }
    const size_t row_bytes = static_cast<size_t>(mi355x_row_bytes(type, K));
    if (src0->nb[1] != 0 && src0->nb[1] != row_bytes) {
        std::fprintf(stderr, "[mi355x error] node '%s' src0 nb1 mismatch: %zu != %zu\n", node->name,
                     (size_t)src0->nb[1], row_bytes);
        return false;
    }
    if (src1->nb[0] != 0 && src1->nb[0] != sizeof(float)) {
        std::fprintf(stderr, "[mi355x error] node '%s' src1 rows are not contiguous\n", node->name);
        return false;
    }
    if (!broadcast_ok(node)) {
        std::fprintf(stderr, "[mi355x error] node '%s' weight batches do not divide the activation batches\n",
                     node->name);
        return false;
    }
    const size_t total_weight_bytes = static_cast<size_t>(N) * row_bytes;
    const BatchGeometry bg = batch_geometry(node, N, K, M, row_bytes);
    const size_t src1_stride1 = bg.a_row, dst_stride1 = bg.o_row;

    const auto *w_base = static_cast<const uint8_t *>(src0->data);
    const auto *a_base = static_cast<const uint8_t *>(src1->data);
    auto *o_base = static_cast<uint8_t *>(node->data);

    if (!host) {
        for (int64_t i3 = 0; i3 < bg.batches3; ++i3) {
            for (int64_t i2 = 0; i2 < bg.batches2; ++i2) {
                const uint8_t *w = w_base + bg.weight_at(i2, i3);
                const uint8_t *a = a_base + bg.act_at(i2, i3);
                uint8_t *o = o_base + bg.out_at(i2, i3);
                // M > 1 (weights in this backend's buffer): one batched call,
                // which reads the weights once per group of activations where
                // the rows are whole floats apart, else M single GEMVs
                // (src/ggml-xdna.cpp:281-297 loops)
                const bool whole = src1_stride1 % sizeof(float) == 0 && dst_stride1 % sizeof(float) == 0;
                if (M > 1 && whole) {
                    if (mi355x_gemv_batched(bc->ctx, type, w, N, K, reinterpret_cast<const float *>(a),
                                            static_cast<int64_t>(src1_stride1 / sizeof(float)),
                                            reinterpret_cast<float *>(o),
                                            static_cast<int64_t>(dst_stride1 / sizeof(float)), M) != MI355X_OK) {
                        std::fprintf(stderr, "[mi355x error] node '%s' batched GEMV dispatch: %s\n", node->name,
                                     mi355x_last_error());
                        return false;
                    }
                    continue;
                }
                for (int64_t m = 0; m < M; ++m) {
                    if (mi355x_gemv(bc->ctx, type, w, N, K, reinterpret_cast<const float *>(a + m * src1_stride1),
                                    reinterpret_cast<float *>(o + m * dst_stride1)) != MI355X_OK) {
                        std::fprintf(stderr, "[mi355x error] node '%s' GEMV dispatch: %s\n", node->name,
                                     mi355x_last_error());
                        return false;
                    }
                }
            }
        }
        return true;
    }

    // compatibility path: weights, activation rows and outputs are host memory;
    // each weight matrix is uploaded (prepacked) into device scratch per call
    const size_t w_al = (total_weight_bytes + 255) & ~size_t(255);
    const size_t x_bytes = static_cast<size_t>(K) * sizeof(float);
    const size_t y_bytes = static_cast<size_t>(N) * sizeof(float);
    uint8_t *scratch = static_cast<uint8_t *>(bc->ensure_scratch(w_al + x_bytes + 256 + y_bytes));
    if (!scratch) {
        std::fprintf(stderr, "[mi355x error] node '%s' scratch allocation: %s\n", node->name, mi355x_last_error());
        return false;
    }
    uint8_t *dw = scratch;
    float *dx = reinterpret_cast<float *>(scratch + w_al);
    float *dy = reinterpret_cast<float *>(scratch + w_al + ((x_bytes + 255) & ~size_t(255)));
    for (int64_t i3 = 0; i3 < bg.batches3; ++i3) {
        for (int64_t i2 = 0; i2 < bg.batches2; ++i2) {
            const uint8_t *w = w_base + bg.weight_at(i2, i3);
            if (mi355x_prepack_from_host(bc->ctx, type, N, K, dw, w, 0, total_weight_bytes) != MI355X_OK) {
                std::fprintf(stderr, "[mi355x error] node '%s' weight upload: %s\n", node->name, mi355x_last_error());
                return false;
            }
            const uint8_t *a = a_base + bg.act_at(i2, i3);
            uint8_t *o = o_base + bg.out_at(i2, i3);
            for (int64_t m = 0; m < M; ++m) {
                if (mi355x_memcpy_h2d(bc->ctx, dx, a + m * src1_stride1, x_bytes) != MI355X_OK ||
                    mi355x_gemv(bc->ctx, type, dw, N, K, dx, dy) != MI355X_OK ||
                    mi355x_memcpy_d2h(bc->ctx, o + m * dst_stride1, dy, y_bytes) != MI355X_OK) {
                    std::fprintf(stderr, "[mi355x error] node '%s' GEMV: %s\n", node->name, mi355x_last_error());
                    return false;
                }
            }
        }
    }
    return true;
}

// A MUL_MAT node that is one GEMV of a single activation row (M = 1, no
// weight or activation batches, dense f32 rows, all data in place): the
// nodes graph_compute may group.  Anything else goes through
// process_mul_mat, which also reports what is wrong.
bool single_row_gemv(const ggml_tensor *node) {
    const ggml_tensor *src0 = node->src[0], *src1 = node->src[1];
    if (!src0 || !src1 || !node->data || !src0->data || !src1->data || src1->type != GGML_TYPE_F32) return false;
    const int bv = block_values(src0->type);
    const int64_t K = src0->ne[0], N = src0->ne[1];
    if (bv == 0 || K <= 0 || N <= 0 || K % bv != 0 || src1->ne[0] != K) return false;
    if (src1->ne[1] != 1 || src1->ne[2] != 1 || src1->ne[3] != 1 || src0->ne[2] != 1 || src0->ne[3] != 1)
        return false;
    if (node->ne[0] != N || node->ne[1] != 1 || node->ne[2] != 1 || node->ne[3] != 1) return false;
    const size_t row_bytes = static_cast<size_t>(mi355x_row_bytes(src0->type, K));
    if (src0->nb[1] != 0 && src0->nb[1] != row_bytes) return false;
    if ((src1->nb[0] != 0 && src1->nb[0] != sizeof(float)) || (node->nb[0] != 0 && node->nb[0] != sizeof(float)))
        return false;
    return true;
}

// Consecutive nodes i.. that read the same activation row with weights of
// one type and length: the number that can go to one mi355x_gemv_multi.
int gemv_group(ggml_cgraph *g, int i, int mm) {
    const ggml_tensor *a = g->nodes[i];
    if (!single_row_gemv(a)) return 1;
    int n = 1;
    while (i + n < g->n_nodes && n < MI355X_MULTI_MAX_JOBS) {
        const ggml_tensor *b = g->nodes[i + n];
        if (!b || b->op != mm || !single_row_gemv(b) || b->src[1]->data != a->src[1]->data ||
            b->src[0]->type != a->src[0]->type || b->src[0]->ne[0] != a->src[0]->ne[0])
            break;
        ++n;
    }
    return n;
}

// Where the bytes of a tensor in a device buffer of this plugin are for a
// kernel: host-resident (the shadow: `host` for the server, `dev` its device
// address) or on the device (`dev` = data).  Host-resident parts of a range
// that is not host-resident as a whole are copied to the device first.
struct Loc {
    const uint8_t *host = nullptr;
    uint8_t *dev = nullptr;
    bool ok = true;
};

Loc locate_input(BackendCtx *bc, const ggml_tensor *t, size_t bytes) {
    Loc l;
    l.dev = static_cast<uint8_t *>(t->data);
    if (!in_our_device_buffer(t)) return l;
    auto *buf = static_cast<BufCtx *>(t->buffer->context);
    std::lock_guard<std::mutex> lk(buf->smu);
    if (buf->resident.empty()) return l;
    const size_t a = buf->off(t->data);
    if (buf->resident.covers(a, a + bytes)) {
        l.host = buf->shadow + a;
        l.dev = buf->shadow_dev + a;
    } else {
        l.ok = materialise(buf, bc->ctx, a, a + bytes);
    }
    return l;
}

// The output of a single-row GEMV node: into the shadow of its buffer when
// the tensor may be host-resident there (`host` set), else the device.
Loc locate_output(const ggml_tensor *t) {
    Loc l;
    l.dev = static_cast<uint8_t *>(t->data);
    if (!in_our_device_buffer(t) || !mirrorable(t)) return l;
    auto *buf = static_cast<BufCtx *>(t->buffer->context);
    std::lock_guard<std::mutex> lk(buf->smu);
    if (!shadow_ready(t->buffer, buf)) return l;
    const size_t a = buf->off(t->data);
    l.host = buf->shadow + a;
    l.dev = buf->shadow_dev + a;
    return l;
}

// Marks an output's range host-resident (written into the shadow) or
// device-current.
void output_written(const ggml_tensor *t, bool host, size_t bytes) {
    if (!in_our_device_buffer(t)) return;
    auto *buf = static_cast<BufCtx *>(t->buffer->context);
    std::lock_guard<std::mutex> lk(buf->smu);
    const size_t a = buf->off(t->data);
    if (host) buf->resident.add(a, a + bytes);
    else buf->resident.remove(a, a + bytes);
}

// n >= 1 consecutive single-row GEMV nodes that share their activation row
// (gemv_group).  With the activation and every output host-resident, Q4_0
// rows of a multiple of 256 values go to the backend's persistent server:
// one command, no launch, no copy, returning when the outputs are in the
// shadow.  Otherwise one launch (mi355x_gemv_multi, or mi355x_gemv) on the
// backend's stream; *host_io is set when that launch reads or writes a shadow
// (graph_compute then waits for it before returning).
bool run_gemv_group(BackendCtx *bc, ggml_tensor *const *nodes, int n, bool *host_io) {
    const ggml_tensor *a = nodes[0];
    const ggml_tensor *w0 = a->src[0];
    const int type = w0->type;
    const int64_t K = w0->ne[0];
    const Loc x = locate_input(bc, a->src[1], static_cast<size_t>(K) * sizeof(float));
    if (!x.ok) {
        std::fprintf(stderr, "[mi355x error] node '%s' activation not on the device: %s\n", a->name,
                     mi355x_last_error());
        return false;
    }
    mi355x_gemv_job jobs[MI355X_MULTI_MAX_JOBS] = {};
    bool out_host[MI355X_MULTI_MAX_JOBS] = {};
    bool all_host = true, aligned = true;
    for (int j = 0; j < n; ++j) {
        const ggml_tensor *t = nodes[j];
        const Loc y = locate_output(t);
        out_host[j] = y.host != nullptr;
        all_host = all_host && out_host[j];
        aligned = aligned && (reinterpret_cast<uintptr_t>(t->src[0]->data) & 15) == 0;
        jobs[j] = {t->src[0]->data, t->src[0]->ne[1], reinterpret_cast<float *>(y.dev)};
    }
    if (bc->group_mode == GGML_MI355X_GROUPS_SERVER && x.host && all_host && type == GGML_TYPE_Q4_0 &&
        K % 256 == 0 && K <= DevCtx::kServerMaxK && n <= 4 && aligned &&
        bc->variant != MI355X_VARIANT_EXACT_F32) {
        DevCtx *dc = bc->dc;
        std::lock_guard<std::mutex> sl(dc->srv_mu);
        if (mi355x_server *srv = dc->server()) {
            // the server reads the shadow with the host's loads: whatever the
            // stream still runs must have written it first
            if (bc->queued && mi355x_ctx_fence(bc->ctx) == MI355X_OK) bc->queued = false;
            mi355x_server_job sj[4];
            for (int j = 0; j < n; ++j) sj[j] = {jobs[j].W, jobs[j].N, jobs[j].y};
            int rc = mi355x_ctx_set_option(dc->srv_ctx, MI355X_OPT_VARIANT, bc->variant);
            if (rc == MI355X_OK) rc = mi355x_server_gemv(srv, reinterpret_cast<const float *>(x.host), K, n, sj);
            if (rc == MI355X_OK) {
                dc->srv_active = true;
                for (int j = 0; j < n; ++j) output_written(nodes[j], true, static_cast<size_t>(jobs[j].N) * 4);
                return true;
            }
            // EUNSUPPORTED (a row count the server does not hold): the
            // launch below computes the group
            if (rc != MI355X_EUNSUPPORTED) {
                std::fprintf(stderr, "[mi355x error] node '%s' server GEMV: %s\n", a->name, mi355x_last_error());
                return false;
            }
        }
    }
    bc->dc->yield_cus();
    const float *xp = reinterpret_cast<const float *>(x.dev);
    const int rc = n > 1 ? mi355x_gemv_multi(bc->ctx, type, K, xp, n, jobs)
                         : mi355x_gemv(bc->ctx, type, jobs[0].W, jobs[0].N, K, xp, jobs[0].y);
    if (rc != MI355X_OK) {
        if (n > 1)
            std::fprintf(stderr, "[mi355x error] nodes '%s'.. (%d sharing one activation) GEMV dispatch: %s\n",
                         a->name, n, mi355x_last_error());
        else
            std::fprintf(stderr, "[mi355x error] node '%s' GEMV dispatch: %s\n", a->name, mi355x_last_error());
        return false;
    }
    bc->queued = true;
    bool any_host = x.host != nullptr;
    for (int j = 0; j < n; ++j) {
        output_written(nodes[j], out_host[j], static_cast<size_t>(jobs[j].N) * 4);
        any_host = any_host || out_host[j];
    }
    if (any_host) *host_io = true;
    return true;
}

enum ggml_status backend_graph_compute(ggml_backend_t backend, ggml_cgraph *cgraph) {
    if (!backend || !cgraph) return GGML_STATUS_FAILED;
    if (cgraph->n_nodes > 0 && !cgraph->nodes) return GGML_STATUS_FAILED;
    BackendCtx *bc = backend_ctx(backend);
    if (!bc) return GGML_STATUS_FAILED;
    std::lock_guard<std::mutex> lk(bc->mu);
    const int mm = op_mul_mat();
    const bool trace = trace_nodes();
    double total_ms = 0.0;
    int count = 0;
    bool host_io = false;
    enum ggml_status status = GGML_STATUS_SUCCESS;
    for (int i = 0; i < cgraph->n_nodes; ++i) {
        ggml_tensor *node = cgraph->nodes[i];
        if (!node || mm < 0 || node->op != mm) continue;  // other nodes carry no work here
        auto t0 = std::chrono::steady_clock::now();
        if (single_row_gemv(node)) {
            // consecutive MUL_MATs that share their activation row: one
            // command or launch (the per-node trace keeps one per node)
            const int n = trace ? 1 : gemv_group(cgraph, i, mm);
            if (!run_gemv_group(bc, cgraph->nodes + i, n, &host_io)) {
                status = GGML_STATUS_FAILED;
                break;
            }
            i += n - 1;
        } else {
            // M > 1, batches, strided rows: device memory only
            const size_t in_bytes = tensor_nbytes(node->src[1]);
            if (in_our_device_buffer(node->src[1])) {
                auto *buf = static_cast<BufCtx *>(node->src[1]->buffer->context);
                if (!device_current(buf, bc->ctx, node->src[1], 0, in_bytes)) {
                    status = GGML_STATUS_FAILED;
                    break;
                }
            }
            bc->dc->yield_cus();
            if (!process_mul_mat(bc, node, false)) {
                status = GGML_STATUS_FAILED;
                break;
            }
            bc->queued = true;
            output_written(node, false, tensor_nbytes(node));
        }
        if (trace) {
            if (mi355x_ctx_sync(bc->ctx)) {
                status = GGML_STATUS_FAILED;
                break;
            }
            const double ms =
                std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            total_ms += ms;
            ++count;
            std::fprintf(stderr, "[mi355x trace] node %3d: %-30s | type=%2d | N=%6ld K=%5ld | %6.3f ms\n", i,
                         node->name[0] ? node->name : "unnamed", node->src[0]->type, (long)node->src[0]->ne[1],
                         (long)node->src[0]->ne[0], ms);
        }
    }
    // kernels that read or write a shadow finish before the host may touch
    // it again (a failed graph waits too: its launches may still run)
    if (host_io) {
        if (mi355x_ctx_fence(bc->ctx) != MI355X_OK) {
            log_error("graph_compute: wait");
            status = GGML_STATUS_FAILED;
        } else if (bc->pending.empty()) {
            bc->queued = false;
        }
    }
    if (trace && count > 0) std::fprintf(stderr, "[mi355x trace] TOTAL: %d nodes, %6.3f ms\n", count, total_ms);
    return status;
}

const ggml_backend_i kBackendIface = {
    /* .get_name            = */ backend_get_name,
    /* .free                = */ backend_free,
    /* .set_tensor_async    = */ backend_set_tensor_async,
    /* .get_tensor_async    = */ backend_get_tensor_async,
    /* .set_tensor_2d_async = */ nullptr,
    /* .get_tensor_2d_async = */ nullptr,
    /* .cpy_tensor_async    = */ nullptr,
    /* .synchronize         = */ backend_synchronize,
    /* .graph_plan_create   = */ nullptr,
    /* .graph_plan_free     = */ nullptr,
    /* .graph_plan_update   = */ nullptr,
    /* .graph_plan_compute  = */ nullptr,
    /* .graph_compute       = */ backend_graph_compute,
    /* .event_record        = */ nullptr,
    /* .event_wait          = */ nullptr,
    /* .graph_optimize      = */ nullptr,
};

ggml_backend_t make_backend(size_t dev_num) {
    init_registry();
    if (dev_num >= g_devs.size()) return nullptr;
    auto *bc = new (std::nothrow) BackendCtx();
    if (!bc) return nullptr;
    bc->dc = g_devs[dev_num];
    if (mi355x_ctx_create(bc->dc->device, &bc->ctx) != MI355X_OK) {
        log_error("backend init");
        delete bc;
        return nullptr;
    }
    auto *backend = new (std::nothrow) ggml_backend{backend_guid(), kBackendIface, &bc->dc->dev, bc};
    if (!backend) {
        delete bc;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(bc->dc->mu);
    ++bc->dc->backends;
    return backend;
}

// ---------------------------------------------------------------------------
// device interface
// ---------------------------------------------------------------------------
const char *dev_get_name(ggml_backend_dev_t dev) { return dev_ctx(dev)->name.c_str(); }
const char *dev_get_description(ggml_backend_dev_t dev) { return dev_ctx(dev)->description.c_str(); }

void dev_get_memory(ggml_backend_dev_t dev, size_t *free, size_t *total) {
    size_t f = 0, t = 0;
    if (mi355x_ctx *x = dev_ctx(dev)->transfer_ctx()) mi355x_mem_info(x, &f, &t);
    if (free) *free = f;
    if (total) *total = t;
}

enum ggml_backend_dev_type dev_get_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_get_props(ggml_backend_dev_t dev, ggml_backend_dev_props *props) {
    if (!props) return;
    DevCtx *dc = dev_ctx(dev);
    props->name = dc->name.c_str();
    props->description = dc->description.c_str();
    props->type = GGML_BACKEND_DEVICE_TYPE_GPU;
    dev_get_memory(dev, &props->memory_free, &props->memory_total);
    props->device_id = dc->pci.c_str();
    props->caps.async = true;
    props->caps.host_buffer = true;
    props->caps.buffer_from_host_ptr = false;
    props->caps.events = false;
    props->caps.mmap_support = false;
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char *) {
    DevCtx *dc = dev_ctx(dev);
    for (size_t i = 0; i < g_devs.size(); ++i)
        if (g_devs[i] == dc) return make_backend(i);
    return nullptr;
}

ggml_backend_buffer_type_t dev_get_buffer_type(ggml_backend_dev_t dev) { return &dev_ctx(dev)->buft; }
ggml_backend_buffer_type_t dev_get_host_buffer_type(ggml_backend_dev_t dev) { return &dev_ctx(dev)->host_buft; }

bool dev_supports_op(ggml_backend_dev_t dev, const ggml_tensor *op) {
    (void)dev;
    const int mm = op_mul_mat();
    // The loader probes with weights in a zero-size buffer or in this
    // plugin's buffer type (src/ggml-xdna.cpp:81-89); both lift M == 1.
    const ggml_tensor *src0 = op && op->src[0] ? op->src[0] : nullptr;
    const bool resident = src0 && src0->buffer && (src0->buffer->size == 0 || in_our_device_buffer(src0));
    const bool res = claim_mul_mat(op, mm, resident);
    if (trace_supports() && op && op->op == mm) {
        const ggml_tensor *s1 = op->src[1];
        std::fprintf(stderr, "[supports_op] %-25s | type=%2d | N=%6ld K=%5ld M=%3ld buf_sz=%zu | -> %s\n", op->name,
                     src0 ? src0->type : -1, src0 ? (long)src0->ne[1] : 0L, src0 ? (long)src0->ne[0] : 0L,
                     s1 ? (long)s1->ne[1] : 0L, (src0 && src0->buffer) ? src0->buffer->size : size_t(0),
                     res ? "YES" : "NO");
    }
    return res;
}

bool dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft) {
    return buft && buft == &dev_ctx(dev)->buft;
}

// Weights outside this plugin's buffer would cross PCIe for every token, so
// no op is pulled onto the device from host buffers.
bool dev_offload_op(ggml_backend_dev_t, const ggml_tensor *) { return false; }

const ggml_backend_device_i kDeviceIface = {
    /* .get_name             = */ dev_get_name,
    /* .get_description      = */ dev_get_description,
    /* .get_memory           = */ dev_get_memory,
    /* .get_type             = */ dev_get_type,
    /* .get_props            = */ dev_get_props,
    /* .init_backend         = */ dev_init_backend,
    /* .get_buffer_type      = */ dev_get_buffer_type,
    /* .get_host_buffer_type = */ dev_get_host_buffer_type,
    /* .buffer_from_host_ptr = */ nullptr,
    /* .supports_op          = */ dev_supports_op,
    /* .supports_buft        = */ dev_supports_buft,
    /* .offload_op           = */ dev_offload_op,
    /* .event_new            = */ nullptr,
    /* .event_free           = */ nullptr,
    /* .event_synchronize    = */ nullptr,
};

// ---------------------------------------------------------------------------
// registry
// ---------------------------------------------------------------------------
const char *reg_get_name(ggml_backend_reg_t) { return "MI355X"; }
size_t reg_get_device_count(ggml_backend_reg_t) {
    init_registry();
    return g_devs.size();
}
ggml_backend_dev_t reg_get_device(ggml_backend_reg_t, size_t index) {
    init_registry();
    return index < g_devs.size() ? &g_devs[index]->dev : nullptr;
}

void *reg_get_proc_address(ggml_backend_reg_t, const char *name) {
    if (!name) return nullptr;
    if (!std::strcmp(name, "ggml_backend_mi355x_init")) return reinterpret_cast<void *>(ggml_backend_mi355x_init);
    if (!std::strcmp(name, "ggml_backend_is_mi355x")) return reinterpret_cast<void *>(ggml_backend_is_mi355x);
    if (!std::strcmp(name, "ggml_backend_mi355x_free")) return reinterpret_cast<void *>(ggml_backend_mi355x_free);
    if (!std::strcmp(name, "ggml_backend_mi355x_load_iq_grids_from_ggml"))
        return reinterpret_cast<void *>(ggml_backend_mi355x_load_iq_grids_from_ggml);
    if (!std::strcmp(name, "ggml_backend_mi355x_set_kernel_variant"))
        return reinterpret_cast<void *>(ggml_backend_mi355x_set_kernel_variant);
    if (!std::strcmp(name, "ggml_backend_mi355x_set_group_mode"))
        return reinterpret_cast<void *>(ggml_backend_mi355x_set_group_mode);
    return nullptr;
}

const ggml_backend_reg_i kRegIface = {
    /* .get_name         = */ reg_get_name,
    /* .get_device_count = */ reg_get_device_count,
    /* .get_device       = */ reg_get_device,
    /* .get_proc_address = */ reg_get_proc_address,
};

void init_registry() {
    std::call_once(g_reg_once, [] {
        g_reg.api_version = GGML_MI355X_BACKEND_API_VERSION;
        g_reg.iface = kRegIface;
        g_reg.context = nullptr;
        int n = 0;
        if (mi355x_device_count(&n) != MI355X_OK) n = 0;
        for (int d = 0; d < n; ++d) {
            auto *dc = new DevCtx();
            dc->device = d;
            dc->name = "MI355X" + std::to_string(d);
            char desc[256] = {0}, pci[64] = {0};
            if (mi355x_device_describe(d, desc, sizeof desc, pci, sizeof pci) == MI355X_OK) {
                dc->description = desc;
                dc->pci = pci;
            } else {
                dc->description = "AMD Instinct MI355X";
            }
            dc->dev = ggml_backend_device{kDeviceIface, &g_reg, dc};
            dc->buft = ggml_backend_buffer_type{kBufferTypeIface, &dc->dev, dc};
            dc->host_buft = ggml_backend_buffer_type{kBufferTypeIface, &dc->dev, dc};
            g_devs.push_back(dc);
        }
        // MI355X_HOST_ONLY_DEVICE=1 lists one more device, bound to no GPU
        // (a host-only context of the C-ABI): its backend and buffers fail
        // every device call the way a lost device would, so the plugin's
        // error surface (GGML_STATUS_FAILED, [mi355x error] messages) can
        // be exercised on a machine without a GPU
        const char *ho = std::getenv("MI355X_HOST_ONLY_DEVICE");
        if (ho && *ho && std::strcmp(ho, "0") != 0) {
            auto *dc = new DevCtx();
            dc->device = MI355X_DEVICE_HOST_ONLY;
            dc->name = "MI355X_HOST_ONLY";
            dc->description = "host-only device (no GPU; every device call fails)";
            dc->pci = "none";
            dc->dev = ggml_backend_device{kDeviceIface, &g_reg, dc};
            dc->buft = ggml_backend_buffer_type{kBufferTypeIface, &dc->dev, dc};
            dc->host_buft = ggml_backend_buffer_type{kBufferTypeIface, &dc->dev, dc};
            g_devs.push_back(dc);
        }
    });
}

}  // namespace

// ---------------------------------------------------------------------------
// IQ grids from the host's ggml (defined in ggml_mi355x_iq.cpp)
// ---------------------------------------------------------------------------
int mi355x_iq_grids_from_ggml_impl();

extern "C" {

ggml_backend_reg *ggml_backend_init(void) {
    init_registry();
    ggml_backend_mi355x_load_iq_grids_from_ggml();
    return &g_reg;
}

int ggml_backend_score(void) {
    int n = 0;
    return mi355x_device_count(&n) == MI355X_OK && n > 0 ? 100 : 0;
}

ggml_backend_reg *ggml_backend_mi355x_reg(void) {
    init_registry();
    return &g_reg;
}

ggml_backend *ggml_backend_mi355x_init(size_t dev_num) { return make_backend(dev_num); }

bool ggml_backend_is_mi355x(ggml_backend *backend) { return backend_ctx(backend) != nullptr; }

void ggml_backend_mi355x_free(ggml_backend *backend) { backend_free(backend); }

ggml_backend_buffer_type *ggml_backend_mi355x_buffer_type(size_t dev_num) {
    init_registry();
    return dev_num < g_devs.size() ? &g_devs[dev_num]->buft : nullptr;
}

ggml_backend_buffer_type *ggml_backend_mi355x_host_buffer_type(void) {
    init_registry();
    return g_devs.empty() ? nullptr : &g_devs[0]->host_buft;
}

int ggml_backend_mi355x_graph_compute(ggml_backend *backend, ggml_cgraph *cgraph) {
    return backend_graph_compute(backend, cgraph);
}

bool ggml_backend_mi355x_supports_op(ggml_backend *backend, const ggml_tensor_mi355x *op) {
    (void)backend;
    return claim_mul_mat(op, GGML_MI355X_OP_MUL_MAT, false);
}

bool ggml_backend_mi355x_compute_graph(ggml_backend *backend, ggml_tensor_mi355x **nodes, size_t n_nodes) {
    if (!backend || !nodes || n_nodes == 0) return false;
    BackendCtx *bc = backend_ctx(backend);
    if (!bc) return false;
    std::lock_guard<std::mutex> lk(bc->mu);
    for (size_t i = 0; i < n_nodes; ++i) {
        ggml_tensor_mi355x *node = nodes[i];
        if (!node || node->op != GGML_MI355X_OP_MUL_MAT) continue;
        bc->dc->yield_cus();
        if (!process_mul_mat(bc, node, true)) return false;
    }
    return true;
}

bool ggml_backend_mi355x_set_op_mul_mat(int op) {
    if (op < 0) return false;
    g_op_mul_mat.store(op);
    return true;
}

int ggml_backend_mi355x_load_iq_grids_from_ggml(void) { return mi355x_iq_grids_from_ggml_impl(); }

bool ggml_backend_mi355x_set_group_mode(ggml_backend *backend, int mode) {
    BackendCtx *bc = backend_ctx(backend);
    if (!bc || (mode != GGML_MI355X_GROUPS_SERVER && mode != GGML_MI355X_GROUPS_LAUNCH)) return false;
    std::lock_guard<std::mutex> lk(bc->mu);
    bc->group_mode = mode;
    return true;
}

bool ggml_backend_mi355x_set_kernel_variant(ggml_backend *backend, int variant) {
    BackendCtx *bc = backend_ctx(backend);
    if (!bc) return false;
    std::lock_guard<std::mutex> lk(bc->mu);
    if (mi355x_ctx_set_option(bc->ctx, MI355X_OPT_VARIANT, variant) != MI355X_OK) return false;
    bc->variant = variant;
    return true;
}

}  // extern "C"
