// C-ABI wrapper over the reference's own CPU sources -- TEST INFRASTRUCTURE.
//
// oracle/Makefile compiles this file together with the reference's sources
// where they lie under /root/reference (src/xdna-q4-0-reference.cpp,
// src/cpu-q4-gemv-engine.cpp, src/xdna-q4-prepack.cpp and the header-only
// include/xdna/kquants.h) into oracle/_ref/libxdna_ref.so.  Tests use it to
// pin the C oracle bit-for-bit; bench.py may time Q4GemvEngine::run as the
// reference CPU baseline.  Nothing here is shipped.
#include "xdna/cpu_q4_gemv_engine.h"
#include "xdna/kquants.h"
#include "xdna/q4_0_reference.h"
#include "xdna/q4_prepack.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <new>
#include <stdexcept>
#include <memory>
#include <string>

namespace {
thread_local std::string g_err;

template <typename F>
int guarded(F &&f) {
    try {
        f();
        return 0;
    } catch (const std::exception &e) {
        g_err = e.what();
        return -1;
    } catch (...) {
        g_err = "unknown exception";
        return -1;
    }
}
}  // namespace

extern "C" {

const char *ref_last_error(void) { return g_err.c_str(); }

float ref_fp16_to_f32(uint16_t h) { return xdna::q4_0::fp16_to_float(h); }
float ref_bf16_to_f32(uint16_t b) { return xdna::q4_0::bf16_to_float(xdna::q4_0::bf16_from_bits(b)); }
uint16_t ref_f32_to_bf16(float f) { return xdna::q4_0::float_to_bf16(f).bits; }

int ref_q4_0_validate_row(uint64_t values, uint64_t bytes) {
    return guarded([&] { xdna::q4_0::validate_row(values, bytes); });
}
int ref_q4_0_validate_matrix(uint64_t rows, uint64_t values, uint64_t bytes) {
    return guarded([&] { xdna::q4_0::validate_matrix(rows, values, bytes); });
}
int ref_q4_0_dequantize_row(const uint8_t *row, uint64_t bytes, uint64_t values, float *out) {
    return guarded([&] { xdna::q4_0::dequantize_row(row, bytes, values, out); });
}
int ref_q4_0_dot_f32(const uint8_t *row, uint64_t bytes, uint64_t values, const float *x,
                     uint64_t nx, float *out) {
    return guarded([&] { *out = xdna::q4_0::dot_f32(row, bytes, values, x, nx); });
}
int ref_q4_0_gemv_f32(const uint8_t *W, uint64_t bytes, uint64_t N, uint64_t K,
                      const float *x, uint64_t nx, float *y, uint64_t ny) {
    return guarded([&] { xdna::q4_0::gemv_f32(W, bytes, N, K, x, nx, y, ny); });
}
int ref_q4_0_gemv_bf16(const uint8_t *W, uint64_t bytes, uint64_t N, uint64_t K,
                       const uint16_t *x, uint64_t nx, float *y, uint64_t ny) {
    return guarded([&] {
        xdna::q4_0::gemv_bf16(W, bytes, N, K, reinterpret_cast<const xdna::q4_0::Bf16 *>(x),
                              nx, y, ny);
    });
}

// ggml type id -> the reference's K/IQ scalar GEMV (include/xdna/kquants.h:495-577)
int ref_gemv_kq(int type, const uint8_t *W, uint64_t N, uint64_t K, const float *x, float *y) {
    return guarded([&] {
        switch (type) {
        case 12: xdna::gemv_q4_K_ref(W, N, K, x, y); break;
        case 13: xdna::gemv_q5_K_ref(W, N, K, x, y); break;
        case 11: xdna::gemv_q3_K_ref(W, N, K, x, y); break;
        case 14: xdna::gemv_q6_K_ref(W, N, K, x, y); break;
        case 23: xdna::gemv_iq4_xs_ref(W, N, K, x, y); break;
        case 21: xdna::gemv_iq3_s_ref(W, N, K, x, y); break;
        default: throw std::invalid_argument("type has no reference GEMV");
        }
    });
}

int ref_dequant_kq(int type, const uint8_t *row, uint64_t K, float *y) {
    return guarded([&] {
        const int64_t k = static_cast<int64_t>(K);
        switch (type) {
        case 12: xdna::dequantize_row_q4_K_ref(reinterpret_cast<const xdna::block_q4_K *>(row), y, k); break;
        case 13: xdna::dequantize_row_q5_K_ref(reinterpret_cast<const xdna::block_q5_K *>(row), y, k); break;
        case 11: xdna::dequantize_row_q3_K_ref(reinterpret_cast<const xdna::block_q3_K *>(row), y, k); break;
        case 14: xdna::dequantize_row_q6_K_ref(reinterpret_cast<const xdna::block_q6_K *>(row), y, k); break;
        case 23: xdna::dequantize_row_iq4_xs_ref(reinterpret_cast<const xdna::block_iq4_xs *>(row), y, k); break;
        case 21: xdna::dequantize_row_iq3_s_ref(reinterpret_cast<const xdna::block_iq3_s *>(row), y, k); break;
        default: throw std::invalid_argument("type has no reference dequantizer");
        }
    });
}

// The reference's CPU GEMV engine (src/cpu-q4-gemv-engine.cpp:142-177).
void *ref_cpu_engine_new(void) { return new (std::nothrow) xdna::Q4GemvEngine(4, 4); }
void ref_cpu_engine_free(void *e) { delete static_cast<xdna::Q4GemvEngine *>(e); }
int ref_cpu_engine_run(void *e, const uint8_t *W, uint64_t bytes, uint64_t N, uint64_t K,
                       const float *x, float *y) {
    return guarded([&] { static_cast<xdna::Q4GemvEngine *>(e)->run(W, bytes, N, K, x, y); });
}

// The reference's BF16 planar prepacker (src/xdna-q4-prepack.cpp:237-340).
int ref_prepack_layout(uint64_t M, uint64_t K, uint64_t cols, uint64_t out[6]) {
    return guarded([&] {
        auto l = xdna::Q4Prepacker::compute_layout(M, K, cols, 32);
        out[0] = l.rows_per_column;
        out[1] = l.groups_per_row;
        out[2] = l.weight_bytes_per_row;
        out[3] = l.scale_bytes_per_row;
        out[4] = l.packed_bytes_per_row;
        out[5] = l.total_packed_bytes;
    });
}
int ref_prepack_pack(const uint8_t *src, uint64_t M, uint64_t K, uint8_t *dst, uint64_t cols) {
    return guarded([&] { xdna::Q4Prepacker::pack(src, M, K, dst, cols, 32); });
}
int ref_prepack_dequant(const uint8_t *packed, uint64_t M, uint64_t K, float *out, uint64_t cols) {
    return guarded([&] { xdna::Q4Prepacker::dequantize_packed(packed, M, K, out, cols, 32); });
}

// The IQ3_S grid, so tests can checksum the transcription used elsewhere.
void ref_iq3s_grid(uint32_t out[512]) { std::memcpy(out, xdna::iq3s_grid, sizeof(xdna::iq3s_grid)); }

}  // extern "C"
