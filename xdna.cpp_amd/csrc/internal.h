// Host-side internals of the HIP layer (not part of the public C-ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "mi355x-gemv.h"

struct mi355x_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int num_cus = 0;
    size_t max_lds_per_block = 0;
    // device staging for raw weight bytes on their way into a resident tensor
    void *staging = nullptr;
    size_t staging_bytes = 0;
    // f32 activations for the K/IQ kernels when the caller's are BF16 or not
    // 16-byte aligned (grown on demand, freed with the context)
    void *xconv = nullptr;
    size_t xconv_bytes = 0;
    // digit-plane tiles of the activations of a batched Q4_0 call (grown on
    // demand, freed with the context)
    void *mbtiles = nullptr;
    size_t mbtiles_bytes = 0;
    // device address of the library's static scratch on this device
    // (allocation-free entry point)
    void *scratch = nullptr;
    // per-context copies of the IQ grids (device), valid when non-null
    void *iq3xxs_grid = nullptr;
    void *iq2s_grid = nullptr;
    uint64_t grids_version = 0;
    // tuning / numerics options (mi355x_ctx_set_option)
    int kernel_variant = MI355X_VARIANT_AUTO;
    int rows_override = 0;
    int waves_override = 0;
    int prefetch_override = 0;
    int64_t grid_override = 0;
    int form_override = MI355X_FORM_AUTO;
    // MI355X_OPT_OVERLAP: `overlap` streams in rotation (0: off) -- the
    // context's stream and up to three more of the same flags and priority;
    // consecutive eligible mi355x_gemv calls take them in turn (ov_next: the
    // stream of the next one) after a fork event on the context's stream;
    // any other call joins the others back first.
    int overlap = 0;
    bool ov_open = false;
    int ov_next = 0;
    hipStream_t ov_streams[3] = {nullptr, nullptr, nullptr};
    hipEvent_t ov_fork = nullptr;
    hipEvent_t ov_join_ev[3] = {nullptr, nullptr, nullptr};
    std::mutex mu;  // serialises calls that share the staging buffer
    // completion word for mi355x_ctx_fence: pinned host memory the signal
    // kernel writes, and the last value handed out
    uint32_t *fence_host = nullptr;
    uint32_t *fence_dev = nullptr;
    std::atomic<uint32_t> fence_seq{0};
};

namespace mi355x {

// Ends an open run of overlapped GEMVs: the context's stream waits for the
// second stream's work (no-op when none is open).
int ov_join(mi355x_ctx *ctx);

// Thread-local error message plumbing.
int set_error(int code, const std::string &msg);
int hip_error(hipError_t e, const char *what);
void clear_error();

// Gate of every entry point that would reach the device: MI355X_OK, or the
// error of an armed injected fault for `entry` (mi355x_inject_fault), or, on
// a host-only context (device MI355X_DEVICE_HOST_ONLY), hipErrorNoDevice.
// Nothing here touches the device.
int device_gate(const mi355x_ctx *ctx, const char *entry);
inline bool host_only(const mi355x_ctx *ctx) { return ctx && ctx->device < 0; }

#define MI355X_HIP(call)                                \
    do {                                                \
        hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return ::mi355x::hip_error(e_, #call); \
    } while (0)

struct GemvArgs {
    int type;
    const uint8_t *W;
    int64_t N;
    int64_t K;
    const void *x;  // float or bf16 bits
    bool x_bf16;
    float *y;
};

// Kernel launchers, one per weight family; return MI355X_* codes.
int launch_gemv_q4_0(mi355x_ctx *ctx, const GemvArgs &a);
bool q4_0_dp_supports(const mi355x_ctx *ctx, const GemvArgs &a);
int launch_gemv_q4_0_dp(mi355x_ctx *ctx, const GemvArgs &a);
// Stops the resident kernel of every server on the context's device, whatever
// context created it (they relaunch on their next call): a hipFree on a
// device waits for every kernel still running there.
int stop_servers(mi355x_ctx *ctx);
// hipFree of a device allocation of the library: stops the device's servers,
// waits for the context's stream, then frees.  Null is a no-op.
int free_device(mi355x_ctx *ctx, void *p);
// Batched form: M activation rows (x + m*x_stride) into y + m*y_stride,
// M <= q4_0_mb_capacity() (0: form not applicable).
int q4_0_mb_capacity(const mi355x_ctx *ctx, const GemvArgs &a);
// fixed_tiles: the device's static scratch (allocation-free entry point), or
// null for the context's own tile buffer (grown with hipMalloc on demand).
int launch_gemv_q4_0_mb(mi355x_ctx *ctx, const GemvArgs &a, int64_t x_stride, int64_t y_stride, int M,
                        void *fixed_tiles);
// Device address of the static scratch on `device` (the device must be
// current); resolved once per device with hipGetSymbolAddress.
int resolve_scratch(int device, void **out);
size_t scratch_bytes();
// Several Q4_0 matrices that share the activation row x as one launch of
// the pipelined form (*launched = false where that form does not apply: the
// caller launches each matrix on its own).
struct MultiJob {
    const uint8_t *W;
    int64_t N;
    float *y;
};
int launch_gemv_q4_0_multi(mi355x_ctx *ctx, int64_t K, const float *x, const MultiJob *jobs, int n, bool *launched);
bool q4_0_st_supports(const mi355x_ctx *ctx, const GemvArgs &a);
bool q4_0_q8_supports(const mi355x_ctx *ctx, const GemvArgs &a);
int launch_gemv_q4_0_q8(mi355x_ctx *ctx, const GemvArgs &a);
int launch_gemv_q4_0_st(mi355x_ctx *ctx, const GemvArgs &a);
int launch_gemv_kquant(mi355x_ctx *ctx, const GemvArgs &a);

// Prepack kernels: byte-range scatter/gather between ggml and resident order.
int launch_prepack_scatter(mi355x_ctx *ctx, int type, int64_t N, int64_t K, uint8_t *packed,
                           const uint8_t *raw, size_t offset, size_t size);
int launch_prepack_gather(mi355x_ctx *ctx, int type, int64_t N, int64_t K, uint8_t *raw,
                          const uint8_t *packed, size_t offset, size_t size);
int launch_fill(mi355x_ctx *ctx, void *dst, uint8_t value, size_t bytes);

// Resident workgroups per CU of `kernel` at this block size and LDS (cached).
int occupancy(const void *kernel, int block_threads, size_t lds_bytes);

// Refresh the context's device copies of the IQ grids from the global table.
int sync_iq_grids(mi355x_ctx *ctx);

}  // namespace mi355x
