// K-quant and IQ decode GEMVs for gfx950 (placeholder until the kernels land).
#include "device_common.h"
#include "internal.h"

namespace mi355x {

int launch_gemv_kquant(mi355x_ctx *ctx, const GemvArgs &a) {
    (void)ctx;
    (void)a;
    return set_error(MI355X_EUNSUPPORTED, "this weight type has no GPU kernel yet");
}

}  // namespace mi355x
