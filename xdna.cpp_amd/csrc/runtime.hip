// C-ABI of the HIP layer: contexts, memory, prepack entry points, GEMV
// dispatch with the reference's validation rules, and a timing helper.
#include "internal.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

namespace mi355x {

namespace {
thread_local std::string g_last_error;

// Process-wide IQ grid tables (host copies) installed by mi355x_set_iq_grid.
std::mutex g_grid_mu;
std::vector<uint8_t> g_iq3xxs_grid;  // 256 * 4 bytes
std::vector<uint8_t> g_iq2s_grid;    // 1024 * 8 bytes
std::atomic<uint64_t> g_grid_version{0};
constexpr size_t kIq3xxsGridBytes = 256 * 4;
constexpr size_t kIq2sGridBytes = 1024 * 8;

constexpr size_t kStagingMax = size_t(64) << 20;

int64_t block_values(int type) {
    switch (type) {
    case MI355X_TYPE_Q4_0: return 32;
    case MI355X_TYPE_Q3_K: case MI355X_TYPE_Q4_K: case MI355X_TYPE_Q5_K: case MI355X_TYPE_Q6_K:
    case MI355X_TYPE_IQ4_XS: case MI355X_TYPE_IQ3_S: case MI355X_TYPE_IQ3_XXS: case MI355X_TYPE_IQ2_S:
        return 256;
    default: return 0;
    }
}

int64_t block_bytes(int type) {
    switch (type) {
    case MI355X_TYPE_Q4_0: return 18;
    case MI355X_TYPE_Q3_K: return 110;
    case MI355X_TYPE_Q4_K: return 144;
    case MI355X_TYPE_Q5_K: return 176;
    case MI355X_TYPE_Q6_K: return 210;
    case MI355X_TYPE_IQ4_XS: return 136;
    case MI355X_TYPE_IQ3_S: return 110;
    case MI355X_TYPE_IQ3_XXS: return 98;
    case MI355X_TYPE_IQ2_S: return 82;
    default: return 0;
    }
}

const char *type_name(int type) {
    switch (type) {
    case MI355X_TYPE_Q4_0: return "Q4_0";
    case MI355X_TYPE_Q3_K: return "Q3_K";
    case MI355X_TYPE_Q4_K: return "Q4_K";
    case MI355X_TYPE_Q5_K: return "Q5_K";
    case MI355X_TYPE_Q6_K: return "Q6_K";
    case MI355X_TYPE_IQ4_XS: return "IQ4_XS";
    case MI355X_TYPE_IQ3_S: return "IQ3_S";
    case MI355X_TYPE_IQ3_XXS: return "IQ3_XXS";
    case MI355X_TYPE_IQ2_S: return "IQ2_S";
    default: return "unknown";
    }
}

// Validates a (type, N, K) weight tensor; returns its total bytes in *total.
int check_tensor(int type, int64_t N, int64_t K, uint64_t *total, const char *who) {
    const int64_t bv = block_values(type);
    if (bv == 0) return set_error(MI355X_EINVAL, std::string(who) + ": unsupported weight type id " + std::to_string(type));
    if (N < 0 || K < 0)
        return set_error(MI355X_EINVAL, std::string(who) + ": negative dimension N=" + std::to_string(N) +
                                            " K=" + std::to_string(K));
    if (K % bv != 0)
        return set_error(MI355X_EINVAL, std::string(who) + ": K must be a multiple of " + std::to_string(bv) +
                                            " for " + type_name(type) + " (got " + std::to_string(K) + ")");
    const uint64_t rb = static_cast<uint64_t>(K / bv) * static_cast<uint64_t>(block_bytes(type));
    if (N != 0 && rb > UINT64_MAX / static_cast<uint64_t>(N))
        return set_error(MI355X_EINVAL, std::string(who) + ": integer overflow computing weight bytes (N=" +
                                            std::to_string(N) + ", bytes_per_row=" + std::to_string(rb) + ")");
    *total = rb * static_cast<uint64_t>(N);
    return MI355X_OK;
}

int ensure_staging(mi355x_ctx *ctx, size_t want) {
    want = std::min(want, kStagingMax);
    if (ctx->staging_bytes >= want) return MI355X_OK;
    if (ctx->staging) {
        int rc = free_device(ctx, ctx->staging);
        if (rc) return rc;
        ctx->staging = nullptr;
        ctx->staging_bytes = 0;
    }
    hipError_t e = hipMalloc(&ctx->staging, want);
    if (e != hipSuccess) {
        ctx->staging = nullptr;
        return set_error(MI355X_ENOMEM, std::string("staging allocation failed: ") + hipGetErrorString(e));
    }
    ctx->staging_bytes = want;
    return MI355X_OK;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        // a host-only context (device < 0) touches no device
        if (dev < 0 || hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (dev >= 0 && prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// gate: false for the calls an entry point makes for itself after passing
// the device gate once
int gemv_common(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const void *x, bool xbf16,
                float *y, const char *who, bool overlap_ok = false, bool gate = true) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, std::string(who) + ": null context");
    uint64_t total = 0;
    int rc = check_tensor(type, N, K, &total, who);
    if (rc) return rc;
    if (N == 0) return MI355X_OK;
    if (!W || !x || !y) return set_error(MI355X_EINVAL, std::string(who) + ": null pointer argument provided");
    if (gate && (rc = device_gate(ctx, who))) return rc;
    if (type != MI355X_TYPE_Q4_0 && (reinterpret_cast<uintptr_t>(W) & 1) != 0)
        return set_error(MI355X_EINVAL, std::string(who) + ": W must be a row of a resident tensor (2-byte aligned)");
    if (!mi355x_type_ready(type))
        return set_error(MI355X_EUNSUPPORTED, std::string(who) + ": " + type_name(type) +
                                                  " needs its grid table (mi355x_set_iq_grid)");
    DeviceGuard dg(ctx->device);
    // Overlapped GEMVs use nothing of the context's but its streams and its
    // grid copies: f32 activations, 16-byte aligned (no conversion buffer),
    // and for IQ3_XXS / IQ2_S grids already on the context (no upload into
    // a buffer that a GEMV on the other stream may be reading).
    const bool grid_type = type == MI355X_TYPE_IQ3_XXS || type == MI355X_TYPE_IQ2_S;
    const bool ov = overlap_ok && ctx->overlap && !xbf16 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                    (!grid_type || ctx->grids_version == g_grid_version.load());
    if (!ov) {
        rc = ov_join(ctx);
        if (rc) return rc;
    }
    if (grid_type && !ov) {
        rc = sync_iq_grids(ctx);
        if (rc) return rc;
    }
    GemvArgs a{type, static_cast<const uint8_t *>(W), N, K, x, xbf16, y};
    if (!ov) return type == MI355X_TYPE_Q4_0 ? launch_gemv_q4_0(ctx, a) : launch_gemv_kquant(ctx, a);
    if (!ctx->ov_open) {
        // the other streams start after everything queued so far
        MI355X_HIP(hipEventRecord(ctx->ov_fork, ctx->stream));
        for (int i = 0; i + 1 < ctx->overlap; ++i) MI355X_HIP(hipStreamWaitEvent(ctx->ov_streams[i], ctx->ov_fork, 0));
        ctx->ov_open = true;
        ctx->ov_next = 0;
    }
    // the launchers queue on ctx->stream: point it at this call's stream
    hipStream_t primary = ctx->stream;
    if (ctx->ov_next) ctx->stream = ctx->ov_streams[ctx->ov_next - 1];
    rc = type == MI355X_TYPE_Q4_0 ? launch_gemv_q4_0(ctx, a) : launch_gemv_kquant(ctx, a);
    ctx->stream = primary;
    ctx->ov_next = (ctx->ov_next + 1) % ctx->overlap;
    return rc;
}

}  // namespace

int set_error(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

namespace {

// One armed fault at a time, process-wide (mi355x_inject_fault, or the
// environment variable MI355X_INJECT_FAULT="<entry>:<hipError_t>[:<skip>]"
// read on first use).
struct Fault {
    std::mutex mu;
    std::atomic<bool> armed{false};
    std::string entry;
    int error = 0;
    int skip = 0;
};
Fault g_fault;
std::once_flag g_fault_env_once;

void arm_fault(const char *entry, int error, int skip) {
    std::lock_guard<std::mutex> lk(g_fault.mu);
    g_fault.entry = entry ? entry : "";
    g_fault.error = error;
    g_fault.skip = skip > 0 ? skip : 0;
    g_fault.armed.store(entry != nullptr && *entry != 0 && error != 0);
}

void read_fault_env() {
    const char *v = std::getenv("MI355X_INJECT_FAULT");
    if (!v || !*v) return;
    const std::string spec(v);
    const size_t c1 = spec.find(':');
    if (c1 == std::string::npos) return;
    const size_t c2 = spec.find(':', c1 + 1);
    const int error = std::atoi(spec.substr(c1 + 1, c2 == std::string::npos ? std::string::npos : c2 - c1 - 1).c_str());
    const int skip = c2 == std::string::npos ? 0 : std::atoi(spec.substr(c2 + 1).c_str());
    arm_fault(spec.substr(0, c1).c_str(), error, skip);
}

}  // namespace

int device_gate(const mi355x_ctx *ctx, const char *entry) {
    std::call_once(g_fault_env_once, read_fault_env);
    if (g_fault.armed.load(std::memory_order_relaxed)) {
        std::lock_guard<std::mutex> lk(g_fault.mu);
        if (g_fault.armed.load() && (g_fault.entry == "*" || g_fault.entry == entry)) {
            if (g_fault.skip > 0) {
                --g_fault.skip;
            } else {
                g_fault.armed.store(false);
                const hipError_t e = static_cast<hipError_t>(g_fault.error);
                const int rc = hip_error(e, entry);
                g_last_error += " [injected]";
                return rc;
            }
        }
    }
    if (host_only(ctx)) {
        const int rc = hip_error(hipErrorNoDevice, entry);
        g_last_error += " [host-only context]";
        return rc;
    }
    return MI355X_OK;
}

int hip_error(hipError_t e, const char *what) {
    g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return e == hipErrorOutOfMemory ? MI355X_ENOMEM : MI355X_EHIP;
}

void clear_error() { g_last_error.clear(); }

int ov_join(mi355x_ctx *ctx) {
    if (!ctx || !ctx->ov_open) return MI355X_OK;
    ctx->ov_open = false;
    for (int i = 0; i + 1 < ctx->overlap; ++i) {
        MI355X_HIP(hipEventRecord(ctx->ov_join_ev[i], ctx->ov_streams[i]));
        MI355X_HIP(hipStreamWaitEvent(ctx->stream, ctx->ov_join_ev[i], 0));
    }
    return MI355X_OK;
}

int free_device(mi355x_ctx *ctx, void *p) {
    if (!p) return MI355X_OK;
    int rc = ov_join(ctx);
    if (rc) return rc;
    rc = stop_servers(ctx);
    if (rc) return rc;
    MI355X_HIP(hipStreamSynchronize(ctx->stream));
    MI355X_HIP(hipFree(p));
    return MI355X_OK;
}

// Fixed-size cache (no heap allocation: the allocation-free entry point goes
// through here); a full table just recomputes.
int occupancy(const void *kernel, int block_threads, size_t lds_bytes) {
    struct Entry {
        const void *kernel;
        int threads;
        size_t lds;
        int occ;
    };
    constexpr int kSlots = 512;
    static std::mutex mu;
    static Entry cache[kSlots];
    static int used = 0;
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < used; ++i)
        if (cache[i].kernel == kernel && cache[i].threads == block_threads && cache[i].lds == lds_bytes)
            return cache[i].occ;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, block_threads, lds_bytes) != hipSuccess ||
        occ < 1)
        occ = 1;
    if (used < kSlots) cache[used++] = {kernel, block_threads, lds_bytes, occ};
    return occ;
}

int sync_iq_grids(mi355x_ctx *ctx) {
    const uint64_t v = g_grid_version.load();
    if (ctx->grids_version == v) return MI355X_OK;
    std::lock_guard<std::mutex> lk(g_grid_mu);
    auto upload = [&](std::vector<uint8_t> &host, void **dev) -> int {
        if (host.empty()) return MI355X_OK;
        if (!*dev) MI355X_HIP(hipMalloc(dev, host.size()));
        MI355X_HIP(hipMemcpyAsync(*dev, host.data(), host.size(), hipMemcpyHostToDevice, ctx->stream));
        MI355X_HIP(hipStreamSynchronize(ctx->stream));
        return MI355X_OK;
    };
    int rc = upload(g_iq3xxs_grid, &ctx->iq3xxs_grid);
    if (!rc) rc = upload(g_iq2s_grid, &ctx->iq2s_grid);
    if (!rc) ctx->grids_version = g_grid_version.load();
    return rc;
}

}  // namespace mi355x

using namespace mi355x;

extern "C" {

const char *mi355x_last_error(void) { return g_last_error.c_str(); }

int mi355x_inject_fault(const char *entry, int hip_error, int skip) {
    clear_error();
    if (entry && *entry && (hip_error == 0 || skip < 0))
        return set_error(MI355X_EINVAL, "mi355x_inject_fault: a fault needs a nonzero hipError_t and skip >= 0");
    std::call_once(g_fault_env_once, read_fault_env);
    arm_fault(entry, hip_error, skip);
    return MI355X_OK;
}

int mi355x_device_count(int *count) {
    clear_error();
    if (!count) return set_error(MI355X_EINVAL, "mi355x_device_count: null pointer");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) n = 0;
    else if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
    *count = n;
    return MI355X_OK;
}

int mi355x_ctx_create(int device, mi355x_ctx **out) {
    clear_error();
    if (!out) return set_error(MI355X_EINVAL, "mi355x_ctx_create: null output pointer");
    *out = nullptr;
    if (device == MI355X_DEVICE_HOST_ONLY) {
        // no device, no stream: every device entry point fails at its gate
        auto *ctx = new (std::nothrow) mi355x_ctx();
        if (!ctx) return set_error(MI355X_ENOMEM, "mi355x_ctx_create: out of host memory");
        ctx->device = MI355X_DEVICE_HOST_ONLY;
        *out = ctx;
        return MI355X_OK;
    }
    int rc = device_gate(nullptr, "mi355x_ctx_create");
    if (rc) return rc;
    int n = 0;
    rc = mi355x_device_count(&n);
    if (rc) return rc;
    if (device < 0 || device >= n)
        return set_error(MI355X_EINVAL, "mi355x_ctx_create: device " + std::to_string(device) + " of " +
                                            std::to_string(n) + " HIP devices");
    DeviceGuard dg(device);
    auto *ctx = new (std::nothrow) mi355x_ctx();
    if (!ctx) return set_error(MI355X_ENOMEM, "mi355x_ctx_create: out of host memory");
    ctx->device = device;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        delete ctx;
        return hip_error(e, "hipGetDeviceProperties");
    }
    ctx->num_cus = prop.multiProcessorCount;
    ctx->max_lds_per_block = prop.sharedMemPerBlock;
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return hip_error(e, "hipStreamCreateWithFlags");
    }
    // MI355X_OPT_OVERLAP's streams, created right after the context's own:
    // HIP hands hardware queues to streams in turn (GPU_MAX_HW_QUEUES, 4 by
    // default), so four streams created together sit on four queues, which
    // overlapped launches need; created later, other streams made in between
    // could put two of them on one queue
    for (int i = 0; i < 3 && e == hipSuccess; ++i) e = hipStreamCreateWithFlags(&ctx->ov_streams[i], hipStreamNonBlocking);
    if (e != hipSuccess) {
        for (hipStream_t st : ctx->ov_streams)
            if (st) (void)hipStreamDestroy(st);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_error(e, "hipStreamCreateWithFlags");
    }
    void *word = nullptr, *word_dev = nullptr;
    e = hipHostMalloc(&word, 64, hipHostMallocMapped);
    if (e == hipSuccess) {
        std::memset(word, 0, 64);
        e = hipHostGetDevicePointer(&word_dev, word, 0);
    }
    if (e != hipSuccess) {
        if (word) (void)hipHostFree(word);
        for (hipStream_t st : ctx->ov_streams) (void)hipStreamDestroy(st);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_error(e, "completion word allocation");
    }
    ctx->fence_host = static_cast<uint32_t *>(word);
    ctx->fence_dev = static_cast<uint32_t *>(word_dev);
    // the device address of the static scratch, once per device, with the
    // device current (the allocation-free entry point uses only this address)
    rc = resolve_scratch(device, &ctx->scratch);
    if (rc) {
        const std::string msg = mi355x_last_error();
        mi355x_ctx_destroy(ctx);
        return set_error(rc, msg);
    }
    *out = ctx;
    return MI355X_OK;
}

void mi355x_ctx_destroy(mi355x_ctx *ctx) {
    if (!ctx) return;
    if (host_only(ctx)) {
        delete ctx;
        return;
    }
    DeviceGuard dg(ctx->device);
    (void)ov_join(ctx);
    for (void *p : {ctx->staging, ctx->xconv, ctx->mbtiles, ctx->iq3xxs_grid, ctx->iq2s_grid})
        (void)free_device(ctx, p);
    (void)stop_servers(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->fence_host) (void)hipHostFree(ctx->fence_host);
    for (int i = 0; i < 3; ++i) {
        if (ctx->ov_streams[i]) {
            (void)hipStreamSynchronize(ctx->ov_streams[i]);
            (void)hipStreamDestroy(ctx->ov_streams[i]);
        }
        if (ctx->ov_join_ev[i]) (void)hipEventDestroy(ctx->ov_join_ev[i]);
    }
    if (ctx->ov_fork) (void)hipEventDestroy(ctx->ov_fork);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int mi355x_ctx_sync(mi355x_ctx *ctx) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_ctx_sync: null context");
    int rc = device_gate(ctx, "mi355x_ctx_sync");
    if (rc) return rc;
    rc = ov_join(ctx);
    if (rc) return rc;
    MI355X_HIP(hipStreamSynchronize(ctx->stream));
    return MI355X_OK;
}

namespace {

// One lane stores the sequence number with release semantics at system
// scope: everything the stream ran before this kernel is visible to the host
// once the host reads the number.
__global__ void fence_signal_kernel(uint32_t *word, uint32_t value) {
    if (threadIdx.x == 0) __hip_atomic_store(word, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Host spin budget before falling back to hipStreamSynchronize.
constexpr double kFenceSpinSeconds = 2e-3;

}  // namespace

int mi355x_ctx_fence(mi355x_ctx *ctx) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_ctx_fence: null context");
    const int grc = device_gate(ctx, "mi355x_ctx_fence");
    if (grc) return grc;
    DeviceGuard dg(ctx->device);
    const int jrc = ov_join(ctx);
    if (jrc) return jrc;
    const uint32_t v = ctx->fence_seq.fetch_add(1) + 1;
    fence_signal_kernel<<<1, 64, 0, ctx->stream>>>(ctx->fence_dev, v);
    MI355X_HIP(hipGetLastError());
    // values are handed out in order; a later one also covers this call
    auto reached = [&] {
        return static_cast<int32_t>(__atomic_load_n(ctx->fence_host, __ATOMIC_ACQUIRE) - v) >= 0;
    };
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; !reached(); ++i) {
        if ((i & 255) == 255 &&
            std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kFenceSpinSeconds) {
            MI355X_HIP(hipStreamSynchronize(ctx->stream));
            return MI355X_OK;
        }
    }
    return MI355X_OK;
}

int mi355x_ctx_set_option(mi355x_ctx *ctx, int option, int64_t value) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: null context");
    if (!host_only(ctx)) {
        DeviceGuard dg(ctx->device);
        const int rc = ov_join(ctx);
        if (rc) return rc;
    }
    switch (option) {
    case MI355X_OPT_OVERLAP: {
        if (value < 0 || value > 4)
            return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: overlap must be 0 (off) or 2 to 4 streams");
        if (value == 1) return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: overlap needs 2 to 4 streams");
        if (value >= 2) {
            const int rc = device_gate(ctx, "mi355x_ctx_set_option");
            if (rc) return rc;
        }
        DeviceGuard dg(ctx->device);
        if (value >= 2 && !ctx->ov_fork) MI355X_HIP(hipEventCreateWithFlags(&ctx->ov_fork, hipEventDisableTiming));
        for (int i = 0; i + 1 < value; ++i) {
            if (!ctx->ov_streams[i]) MI355X_HIP(hipStreamCreateWithFlags(&ctx->ov_streams[i], hipStreamNonBlocking));
            if (!ctx->ov_join_ev[i])
                MI355X_HIP(hipEventCreateWithFlags(&ctx->ov_join_ev[i], hipEventDisableTiming));
        }
        ctx->overlap = static_cast<int>(value);
        return MI355X_OK;
    }
    case MI355X_OPT_VARIANT:
        if (value != MI355X_VARIANT_AUTO && value != MI355X_VARIANT_EXACT_F32 && value != MI355X_VARIANT_DIGITS &&
            value != MI355X_VARIANT_GGML_Q8)
            return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: unknown kernel variant");
        ctx->kernel_variant = static_cast<int>(value);
        return MI355X_OK;
    case MI355X_OPT_ROWS_PER_WAVE:
        if (value != 0 && value != 1 && value != 2 && value != 4 && value != 8 && value != 16)
            return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: rows per wave must be 0, 1, 2, 4, 8 or 16");
        ctx->rows_override = static_cast<int>(value);
        return MI355X_OK;
    case MI355X_OPT_WAVES_PER_GROUP:
        if (value != 0 && value != 8 && value != 16)
            return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: waves per workgroup must be 0, 8 or 16");
        ctx->waves_override = static_cast<int>(value);
        return MI355X_OK;
    case MI355X_OPT_PREFETCH:
        if (value != 0 && value != 1 && value != 2)
            return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: prefetch must be 0 (auto), 1 (on) or 2 (off)");
        ctx->prefetch_override = static_cast<int>(value);
        return MI355X_OK;
    case MI355X_OPT_FORM:
        if (value != MI355X_FORM_AUTO && value != MI355X_FORM_ROWS && value != MI355X_FORM_KSPLIT &&
            value != MI355X_FORM_STREAM && value != MI355X_FORM_PIPE)
            return set_error(MI355X_EINVAL,
                             "mi355x_ctx_set_option: form must be 0 (auto), 1 (rows), 2 (K-split), 3 (stream) or 4 (pipelined)");
        ctx->form_override = static_cast<int>(value);
        return MI355X_OK;
    case MI355X_OPT_GRID:
        if (value < 0) return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: negative grid");
        ctx->grid_override = value;
        return MI355X_OK;
    default:
        return set_error(MI355X_EINVAL, "mi355x_ctx_set_option: unknown option " + std::to_string(option));
    }
}

void *mi355x_ctx_stream(mi355x_ctx *ctx) {
    if (!ctx) return nullptr;
    // work the caller queues on the stream comes after every overlapped GEMV
    (void)ov_join(ctx);
    return static_cast<void *>(ctx->stream);
}

int mi355x_ctx_device(mi355x_ctx *ctx) { return ctx ? ctx->device : -1; }

int mi355x_mem_info(mi355x_ctx *ctx, size_t *free_bytes, size_t *total_bytes) {
    clear_error();
    if (!ctx || !free_bytes || !total_bytes) return set_error(MI355X_EINVAL, "mi355x_mem_info: null pointer");
    const int rc = device_gate(ctx, "mi355x_mem_info");
    if (rc) return rc;
    DeviceGuard dg(ctx->device);
    MI355X_HIP(hipMemGetInfo(free_bytes, total_bytes));
    return MI355X_OK;
}

int mi355x_device_describe(int device, char *name, size_t name_len, char *pci, size_t pci_len) {
    clear_error();
    hipDeviceProp_t prop;
    MI355X_HIP(hipGetDeviceProperties(&prop, device));
    if (name && name_len) {
        std::snprintf(name, name_len, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    }
    if (pci && pci_len) {
        std::snprintf(pci, pci_len, "%04x:%02x:%02x.0", prop.pciDomainID, prop.pciBusID, prop.pciDeviceID);
    }
    return MI355X_OK;
}

int mi355x_malloc(mi355x_ctx *ctx, size_t bytes, void **dptr) {
    clear_error();
    if (!ctx || !dptr) return set_error(MI355X_EINVAL, "mi355x_malloc: null pointer");
    *dptr = nullptr;
    const int rc = device_gate(ctx, "mi355x_malloc");
    if (rc) return rc;
    DeviceGuard dg(ctx->device);
    hipError_t e = hipMalloc(dptr, bytes == 0 ? 256 : bytes);
    if (e != hipSuccess) {
        *dptr = nullptr;
        return set_error(MI355X_ENOMEM, "hipMalloc(" + std::to_string(bytes) + "): " + hipGetErrorString(e));
    }
    return MI355X_OK;
}

int mi355x_free(mi355x_ctx *ctx, void *dptr) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_free: null context");
    if (!dptr) return MI355X_OK;
    const int rc = device_gate(ctx, "mi355x_free");
    if (rc) return rc;
    DeviceGuard dg(ctx->device);
    return free_device(ctx, dptr);
}

int mi355x_host_malloc(size_t bytes, void **hptr) {
    clear_error();
    if (!hptr) return set_error(MI355X_EINVAL, "mi355x_host_malloc: null pointer");
    *hptr = nullptr;
    hipError_t e = hipHostMalloc(hptr, bytes == 0 ? 64 : bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        *hptr = nullptr;
        return set_error(MI355X_ENOMEM, "hipHostMalloc(" + std::to_string(bytes) + "): " + hipGetErrorString(e));
    }
    return MI355X_OK;
}

int mi355x_host_free(void *hptr) {
    clear_error();
    if (!hptr) return MI355X_OK;
    MI355X_HIP(hipHostFree(hptr));
    return MI355X_OK;
}

int mi355x_host_device_ptr(const void *hptr, void **dptr) {
    clear_error();
    if (!hptr || !dptr) return set_error(MI355X_EINVAL, "mi355x_host_device_ptr: null pointer");
    *dptr = nullptr;
    MI355X_HIP(hipHostGetDevicePointer(dptr, const_cast<void *>(hptr), 0));
    return MI355X_OK;
}

static int copy_sync(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes, hipMemcpyKind kind,
                     const char *who) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, std::string(who) + ": null context");
    if (bytes == 0) return MI355X_OK;
    if (!dst || !src) return set_error(MI355X_EINVAL, std::string(who) + ": null pointer");
    const int grc = device_gate(ctx, who);
    if (grc) return grc;
    DeviceGuard dg(ctx->device);
    const int jrc = ov_join(ctx);
    if (jrc) return jrc;
    MI355X_HIP(hipMemcpyAsync(dst, src, bytes, kind, ctx->stream));
    MI355X_HIP(hipStreamSynchronize(ctx->stream));
    return MI355X_OK;
}

int mi355x_memcpy_h2d(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_sync(ctx, dst, src, bytes, hipMemcpyHostToDevice, "mi355x_memcpy_h2d");
}
int mi355x_memcpy_d2h(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_sync(ctx, dst, src, bytes, hipMemcpyDeviceToHost, "mi355x_memcpy_d2h");
}
int mi355x_memcpy_d2d(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_sync(ctx, dst, src, bytes, hipMemcpyDeviceToDevice, "mi355x_memcpy_d2d");
}

static int copy_async(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes, hipMemcpyKind kind,
                      const char *who) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, std::string(who) + ": null context");
    if (bytes == 0) return MI355X_OK;
    if (!dst || !src) return set_error(MI355X_EINVAL, std::string(who) + ": null pointer");
    const int grc = device_gate(ctx, who);
    if (grc) return grc;
    DeviceGuard dg(ctx->device);
    const int jrc = ov_join(ctx);
    if (jrc) return jrc;
    MI355X_HIP(hipMemcpyAsync(dst, src, bytes, kind, ctx->stream));
    return MI355X_OK;
}
int mi355x_memcpy_h2d_async(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_async(ctx, dst, src, bytes, hipMemcpyHostToDevice, "mi355x_memcpy_h2d_async");
}
int mi355x_memcpy_d2h_async(mi355x_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_async(ctx, dst, src, bytes, hipMemcpyDeviceToHost, "mi355x_memcpy_d2h_async");
}

int mi355x_fill(mi355x_ctx *ctx, void *dst, uint8_t value, size_t bytes) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_fill: null context");
    if (bytes && !dst) return set_error(MI355X_EINVAL, "mi355x_fill: null pointer");
    int rc = device_gate(ctx, "mi355x_fill");
    if (rc) return rc;
    DeviceGuard dg(ctx->device);
    rc = ov_join(ctx);
    if (rc) return rc;
    return launch_fill(ctx, dst, value, bytes);
}

int64_t mi355x_row_bytes(int type, int64_t K) {
    const int64_t bv = block_values(type);
    if (bv == 0 || K < 0 || K % bv != 0) return -1;
    return (K / bv) * block_bytes(type);
}

int mi355x_type_ready(int type) {
    switch (type) {
    case MI355X_TYPE_Q4_0: case MI355X_TYPE_Q3_K: case MI355X_TYPE_Q4_K: case MI355X_TYPE_Q5_K:
    case MI355X_TYPE_Q6_K: case MI355X_TYPE_IQ4_XS: case MI355X_TYPE_IQ3_S:
        return 1;
    case MI355X_TYPE_IQ3_XXS: {
        std::lock_guard<std::mutex> lk(g_grid_mu);
        return g_iq3xxs_grid.empty() ? 0 : 1;
    }
    case MI355X_TYPE_IQ2_S: {
        std::lock_guard<std::mutex> lk(g_grid_mu);
        return g_iq2s_grid.empty() ? 0 : 1;
    }
    default: return 0;
    }
}

int mi355x_set_iq_grid(int type, const void *table, size_t bytes) {
    clear_error();
    if (!table) return set_error(MI355X_EINVAL, "mi355x_set_iq_grid: null table");
    std::lock_guard<std::mutex> lk(g_grid_mu);
    const uint8_t *p = static_cast<const uint8_t *>(table);
    if (type == MI355X_TYPE_IQ3_XXS) {
        if (bytes != kIq3xxsGridBytes)
            return set_error(MI355X_EINVAL, "mi355x_set_iq_grid: IQ3_XXS grid is 1024 bytes");
    } else if (type == MI355X_TYPE_IQ2_S) {
        if (bytes != kIq2sGridBytes)
            return set_error(MI355X_EINVAL, "mi355x_set_iq_grid: IQ2_S grid is 8192 bytes");
    } else {
        return set_error(MI355X_EINVAL, "mi355x_set_iq_grid: only IQ3_XXS and IQ2_S take a grid");
    }
    // the kernels negate magnitudes bytewise (carry-free for 1..127)
    for (size_t i = 0; i < bytes; ++i)
        if (p[i] == 0 || p[i] > 127)
            return set_error(MI355X_EINVAL, "mi355x_set_iq_grid: grid magnitudes must be 1..127");
    (type == MI355X_TYPE_IQ3_XXS ? g_iq3xxs_grid : g_iq2s_grid).assign(p, p + bytes);
    g_grid_version.fetch_add(1);
    return MI355X_OK;
}

// K/IQ resident rows pick their plane order from the row address mod 4
// (kq_layout.h), so a resident tensor must start on a 4-byte boundary.
static int check_resident_base(int type, const void *base, const char *who) {
    if (type != MI355X_TYPE_Q4_0 && (reinterpret_cast<uintptr_t>(base) & 3) != 0)
        return set_error(MI355X_EINVAL, std::string(who) + ": resident tensor must start on a 4-byte boundary");
    return MI355X_OK;
}

static int check_range(int type, int64_t N, int64_t K, size_t offset, size_t size, const char *who) {
    uint64_t total = 0;
    int rc = check_tensor(type, N, K, &total, who);
    if (rc) return rc;
    if (offset > total || size > total - offset)
        return set_error(MI355X_EINVAL, std::string(who) + ": byte range [" + std::to_string(offset) + ", +" +
                                            std::to_string(size) + ") exceeds tensor of " + std::to_string(total) +
                                            " bytes");
    return MI355X_OK;
}

int mi355x_prepack_from_host(mi355x_ctx *ctx, int type, int64_t N, int64_t K, void *packed_dev,
                             const void *raw_host, size_t offset, size_t size) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_prepack_from_host: null context");
    int rc = check_range(type, N, K, offset, size, "mi355x_prepack_from_host");
    if (rc || size == 0) return rc;
    if (!packed_dev || !raw_host) return set_error(MI355X_EINVAL, "mi355x_prepack_from_host: null pointer");
    rc = check_resident_base(type, packed_dev, "mi355x_prepack_from_host");
    if (rc) return rc;
    rc = device_gate(ctx, "mi355x_prepack_from_host");
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    DeviceGuard dg(ctx->device);
    rc = ov_join(ctx);
    if (rc) return rc;
    rc = ensure_staging(ctx, size);
    if (rc) return rc;
    const uint8_t *src = static_cast<const uint8_t *>(raw_host);
    for (size_t done = 0; done < size;) {
        const size_t n = std::min(size - done, ctx->staging_bytes);
        MI355X_HIP(hipMemcpyAsync(ctx->staging, src + done, n, hipMemcpyHostToDevice, ctx->stream));
        rc = launch_prepack_scatter(ctx, type, N, K, static_cast<uint8_t *>(packed_dev),
                                    static_cast<const uint8_t *>(ctx->staging), offset + done, n);
        if (rc) return rc;
        MI355X_HIP(hipStreamSynchronize(ctx->stream));
        done += n;
    }
    return MI355X_OK;
}

int mi355x_prepack_from_device(mi355x_ctx *ctx, int type, int64_t N, int64_t K, void *packed_dev,
                               const void *raw_dev, size_t offset, size_t size) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_prepack_from_device: null context");
    int rc = check_range(type, N, K, offset, size, "mi355x_prepack_from_device");
    if (rc || size == 0) return rc;
    if (!packed_dev || !raw_dev) return set_error(MI355X_EINVAL, "mi355x_prepack_from_device: null pointer");
    rc = check_resident_base(type, packed_dev, "mi355x_prepack_from_device");
    if (rc) return rc;
    rc = device_gate(ctx, "mi355x_prepack_from_device");
    if (rc) return rc;
    DeviceGuard dg(ctx->device);
    rc = ov_join(ctx);
    if (rc) return rc;
    rc = launch_prepack_scatter(ctx, type, N, K, static_cast<uint8_t *>(packed_dev),
                                static_cast<const uint8_t *>(raw_dev), offset, size);
    if (rc) return rc;
    MI355X_HIP(hipStreamSynchronize(ctx->stream));
    return MI355X_OK;
}

int mi355x_unpack_to_host(mi355x_ctx *ctx, int type, int64_t N, int64_t K, const void *packed_dev,
                          void *raw_host, size_t offset, size_t size) {
    clear_error();
    if (!ctx) return set_error(MI355X_EINVAL, "mi355x_unpack_to_host: null context");
    int rc = check_range(type, N, K, offset, size, "mi355x_unpack_to_host");
    if (rc || size == 0) return rc;
    if (!packed_dev || !raw_host) return set_error(MI355X_EINVAL, "mi355x_unpack_to_host: null pointer");
    rc = check_resident_base(type, packed_dev, "mi355x_unpack_to_host");
    if (rc) return rc;
    rc = device_gate(ctx, "mi355x_unpack_to_host");
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    DeviceGuard dg(ctx->device);
    rc = ov_join(ctx);
    if (rc) return rc;
    rc = ensure_staging(ctx, size);
    if (rc) return rc;
    uint8_t *dst = static_cast<uint8_t *>(raw_host);
    for (size_t done = 0; done < size;) {
        const size_t n = std::min(size - done, ctx->staging_bytes);
        rc = launch_prepack_gather(ctx, type, N, K, static_cast<uint8_t *>(ctx->staging),
                                   static_cast<const uint8_t *>(packed_dev), offset + done, n);
        if (rc) return rc;
        MI355X_HIP(hipMemcpyAsync(dst + done, ctx->staging, n, hipMemcpyDeviceToHost, ctx->stream));
        MI355X_HIP(hipStreamSynchronize(ctx->stream));
        done += n;
    }
    return MI355X_OK;
}

int mi355x_gemv(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *x, float *y) {
    return gemv_common(ctx, type, W, N, K, x, false, y, "mi355x_gemv", true);
}

int mi355x_gemv_multi(mi355x_ctx *ctx, int type, int64_t K, const float *x, int njobs, const mi355x_gemv_job *jobs) {
    clear_error();
    static const char *who = "mi355x_gemv_multi";
    if (!ctx || !x || !jobs) return set_error(MI355X_EINVAL, std::string(who) + ": null pointer argument provided");
    if (njobs < 1 || njobs > MI355X_MULTI_MAX_JOBS)
        return set_error(MI355X_EINVAL, std::string(who) + ": 1 to " + std::to_string(MI355X_MULTI_MAX_JOBS) +
                                            " jobs per call");
    MultiJob mj[MI355X_MULTI_MAX_JOBS];
    for (int j = 0; j < njobs; ++j) {
        uint64_t total = 0;
        const int rc = check_tensor(type, jobs[j].N, K, &total, who);
        if (rc) return rc;
        if (!jobs[j].W || !jobs[j].y)
            return set_error(MI355X_EINVAL, std::string(who) + ": null pointer argument provided");
        mj[j] = {static_cast<const uint8_t *>(jobs[j].W), jobs[j].N, jobs[j].y};
    }
    {
        const int rc = device_gate(ctx, who);
        if (rc) return rc;
    }
    {
        DeviceGuard dg(ctx->device);
        const int rc = ov_join(ctx);
        if (rc) return rc;
    }
    if (type == MI355X_TYPE_Q4_0 && K > 0) {
        bool all = true;
        for (int j = 0; j < njobs; ++j) all = all && jobs[j].N > 0 && (reinterpret_cast<uintptr_t>(jobs[j].W) & 1) == 0;
        if (all) {
            DeviceGuard dg(ctx->device);
            bool launched = false;
            const int rc = launch_gemv_q4_0_multi(ctx, K, x, mj, njobs, &launched);
            if (rc || launched) return rc;
        }
    }
    // one launch per matrix where the shared form does not apply
    for (int j = 0; j < njobs; ++j) {
        const int rc = gemv_common(ctx, type, jobs[j].W, jobs[j].N, K, x, false, jobs[j].y, who, false, false);
        if (rc) return rc;
    }
    return MI355X_OK;
}

int mi355x_gemv_bf16(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const uint16_t *x_bf16,
                     float *y) {
    return gemv_common(ctx, type, W, N, K, x_bf16, true, y, "mi355x_gemv_bf16");
}

namespace {

// mi355x_gemv_batched and its allocation-free form (noalloc: activation tiles
// in the device's static scratch; no path that would allocate).
int gemv_batched(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *x, int64_t x_stride,
                 float *y, int64_t y_stride, int64_t M, bool noalloc, const char *who) {
    clear_error();
    if (M < 0) return set_error(MI355X_EINVAL, std::string(who) + ": negative M");
    if (ctx && M > 0) {
        const int rc = device_gate(ctx, who);
        if (rc) return rc;
    }
    if (ctx) {
        DeviceGuard dg(ctx->device);
        const int rc = ov_join(ctx);
        if (rc) return rc;
    }
    if (M > 1 && (x_stride < K || y_stride < N))
        return set_error(MI355X_EINVAL, std::string(who) + ": strides smaller than a row");
    if (noalloc && ctx && M > 0 && N > 0) {
        if (!ctx->scratch) return set_error(MI355X_EUNSUPPORTED, std::string(who) + ": no static scratch on the device");
        // the K/IQ kernels copy unaligned activations into a context buffer,
        // and IQ3_XXS / IQ2_S grids reach a context on its first such GEMV:
        // both would allocate
        if (type != MI355X_TYPE_Q4_0 &&
            ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (M > 1 && (x_stride & 3) != 0)))
            return set_error(MI355X_EINVAL, std::string(who) +
                                                ": K/IQ weights need 16-byte aligned activation rows here");
        if ((type == MI355X_TYPE_IQ3_XXS && !ctx->iq3xxs_grid) || (type == MI355X_TYPE_IQ2_S && !ctx->iq2s_grid))
            return set_error(MI355X_EUNSUPPORTED, std::string(who) +
                                                      ": the grid is not on this context yet (one mi355x_gemv of "
                                                      "this type on the context first)");
    }
    // Q4_0 digit-plane arithmetic: up to q4_0_mb_capacity() activations per
    // launch of the batched form (weights read once per launch)
    if (ctx && type == MI355X_TYPE_Q4_0 && M >= 2 && N > 0 && W && x && y &&
        (ctx->kernel_variant == MI355X_VARIANT_AUTO || ctx->kernel_variant == MI355X_VARIANT_DIGITS)) {
        uint64_t total = 0;
        int rc = check_tensor(type, N, K, &total, who);
        if (rc) return rc;
        GemvArgs a{type, static_cast<const uint8_t *>(W), N, K, x, false, y};
        const int cap = q4_0_mb_capacity(ctx, a);
        if (cap >= 2) {
            DeviceGuard dg(ctx->device);
            for (int64_t m0 = 0; m0 < M;) {
                const int chunk = static_cast<int>(std::min<int64_t>(cap, M - m0));
                GemvArgs c{type, static_cast<const uint8_t *>(W), N, K, x + m0 * x_stride, false, y + m0 * y_stride};
                // a one-activation remainder also runs in this form, so every
                // output of the call has the same arithmetic
                rc = launch_gemv_q4_0_mb(ctx, c, x_stride, y_stride, chunk, noalloc ? ctx->scratch : nullptr);
                if (rc) return rc;
                m0 += chunk;
            }
            return MI355X_OK;
        }
    }
    for (int64_t m = 0; m < M; ++m) {
        int rc = gemv_common(ctx, type, W, N, K, x + m * x_stride, false, y + m * y_stride, who, false, false);
        if (rc) return rc;
    }
    return MI355X_OK;
}

}  // namespace

int mi355x_gemv_batched(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *x,
                        int64_t x_stride, float *y, int64_t y_stride, int64_t M) {
    return gemv_batched(ctx, type, W, N, K, x, x_stride, y, y_stride, M, false, "mi355x_gemv_batched");
}

int mi355x_gemv_batched_noalloc(mi355x_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *x,
                                int64_t x_stride, float *y, int64_t y_stride, int64_t M) {
    return gemv_batched(ctx, type, W, N, K, x, x_stride, y, y_stride, M, true, "mi355x_gemv_batched_noalloc");
}

int mi355x_time_gemv(mi355x_ctx *ctx, int type, const void *const *weights, int n_weights, int64_t N, int64_t K,
                     const float *x, float *y, int warmup, int iters, double *ms_total) {
    clear_error();
    if (!ctx || !weights || n_weights < 1 || iters < 1 || warmup < 0 || !ms_total)
        return set_error(MI355X_EINVAL, "mi355x_time_gemv: bad arguments");
    {
        const int grc = device_gate(ctx, "mi355x_time_gemv");
        if (grc) return grc;
    }
    DeviceGuard dg(ctx->device);
    // with MI355X_OPT_OVERLAP (S streams) consecutive launches may run at
    // once: launch i writes y + (i % S) * N
    auto out = [&](int i) { return ctx->overlap ? y + (i % ctx->overlap) * N : y; };
    for (int i = 0; i < warmup; ++i) {
        int rc = mi355x_gemv(ctx, type, weights[i % n_weights], N, K, x, out(i));
        if (rc) return rc;
    }
    {
        const int rc = ov_join(ctx);
        if (rc) return rc;
    }
    hipEvent_t e0, e1;
    MI355X_HIP(hipEventCreate(&e0));
    hipError_t e = hipEventCreate(&e1);
    if (e != hipSuccess) {
        (void)hipEventDestroy(e0);
        return hip_error(e, "hipEventCreate");
    }
    int rc = MI355X_OK;
    if (hipEventRecord(e0, ctx->stream) != hipSuccess) rc = set_error(MI355X_EHIP, "hipEventRecord");
    for (int i = 0; i < iters && rc == MI355X_OK; ++i)
        rc = mi355x_gemv(ctx, type, weights[i % n_weights], N, K, x, out(i));
    if (rc == MI355X_OK) rc = ov_join(ctx);
    if (rc == MI355X_OK && hipEventRecord(e1, ctx->stream) != hipSuccess) rc = set_error(MI355X_EHIP, "hipEventRecord");
    if (rc == MI355X_OK) {
        e = hipEventSynchronize(e1);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e != hipSuccess) rc = hip_error(e, "hipEventElapsedTime");
        else *ms_total = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

}  // extern "C"
