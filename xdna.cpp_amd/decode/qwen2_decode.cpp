// Batch-1 greedy decoder of a Qwen2-shaped model with Q4_0 weights; see
// qwen2_decode.h.  The model shape and the decode loop follow the BASELINE
// e2e configuration (Qwen2.5-3B: 36 layers, hidden 2048, 16 query / 2 KV
// heads of 128, SwiGLU 11008, RMSNorm, RoPE theta 1e6, vocab 151936, tied
// embeddings); only the matrix-vector products leave the host.
#include "qwen2_decode.h"

#include "ggml-mi355x.h"
#include "ggml_abi.h"
#include "mi355x-gemv.h"

#include <hip/hip_runtime_api.h>

#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(const std::string &msg) {
    g_err = msg;
    return -1;
}

// ---- seeded normal weights ----------------------------------------------------
uint64_t splitmix64(uint64_t &s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Xoshiro {
    uint64_t s[4];
    Xoshiro(uint64_t seed, uint64_t stream, uint64_t row) {
        uint64_t t = seed ^ (stream * 0xD1342543DE82EF95ull) ^ (row * 0x2545F4914F6CDD1Dull);
        for (auto &v : s) v = splitmix64(t);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    double uniform() { return (static_cast<double>(next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
};

// n values ~ N(0, sigma^2): Marsaglia's polar method on pairs of uniforms
// in (-1, 1), rejecting points outside the unit disc
void normals(Xoshiro &rng, float *out, int64_t n, float sigma) {
    for (int64_t i = 0; i < n; i += 2) {
        double u, v, s;
        do {
            u = 2.0 * rng.uniform() - 1.0;
            v = 2.0 * rng.uniform() - 1.0;
            s = u * u + v * v;
        } while (s >= 1.0 || s == 0.0);
        const double f = std::sqrt(-2.0 * std::log(s) / s);
        out[i] = static_cast<float>(u * f) * sigma;
        if (i + 1 < n) out[i + 1] = static_cast<float>(v * f) * sigma;
    }
}

// IEEE half bits of f (round to nearest even)
uint16_t to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7FFFFFFFu;
    if (x >= 0x7F800000u) return static_cast<uint16_t>(sign | 0x7C00u | (x > 0x7F800000u ? 0x200u : 0));
    if (x >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);  // rounds to inf
    if (x < 0x38800000u) {                                                // subnormal half
        if (x < 0x33000000u) return static_cast<uint16_t>(sign);
        const int e = static_cast<int>(x >> 23);
        const uint32_t m = (x & 0x7FFFFFu) | 0x800000u;
        // value m * 2^(e - 150) = r * 2^-24: r = m >> (126 - e), rounded
        const int shift = 125 - e;
        const uint32_t keep = m >> (shift + 1);
        const uint32_t rest = m & ((2u << shift) - 1);
        const uint32_t half = 1u << shift;
        uint32_t r = keep + (rest > half || (rest == half && (keep & 1)));
        return static_cast<uint16_t>(sign | r);
    }
    const uint32_t e = (x >> 23) - 112;
    const uint32_t m = x & 0x7FFFFFu;
    uint32_t r = (e << 10) | (m >> 13);
    const uint32_t rest = m & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 1))) ++r;
    return static_cast<uint16_t>(sign | r);
}

float from_half(uint16_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF, bits;
    if (e == 0) {
        float f = std::ldexp(static_cast<float>(m), -24);
        std::memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// ggml's Q4_0 rule: per 32 values, d = (value of largest |x|) / -8, codes
// min(15, trunc(x / d + 8.5)), d stored as half.
void quantize_q4_0_row(const float *x, int64_t K, uint8_t *out) {
    for (int64_t b = 0; b < K / 32; ++b) {
        const float *v = x + 32 * b;
        float amax = 0.f, mx = 0.f;
        for (int j = 0; j < 32; ++j) {
            if (std::fabs(v[j]) > amax) {
                amax = std::fabs(v[j]);
                mx = v[j];
            }
        }
        const float d = mx / -8.0f;
        const float id = d != 0.f ? 1.0f / d : 0.f;
        uint8_t *blk = out + 18 * b;
        const uint16_t hd = to_half(d);
        blk[0] = static_cast<uint8_t>(hd & 0xFF);
        blk[1] = static_cast<uint8_t>(hd >> 8);
        for (int j = 0; j < 16; ++j) {
            const int q0 = std::min(15, static_cast<int>(static_cast<int8_t>(v[j] * id + 8.5f)));
            const int q1 = std::min(15, static_cast<int>(static_cast<int8_t>(v[j + 16] * id + 8.5f)));
            blk[2 + j] = static_cast<uint8_t>(q0 | (q1 << 4));
        }
    }
}

void dequant_q4_0_row(const uint8_t *row, int64_t K, float *out) {
    for (int64_t b = 0; b < K / 32; ++b) {
        const uint8_t *blk = row + 18 * b;
        const float d = from_half(static_cast<uint16_t>(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 16; ++j) {
            out[32 * b + j] = static_cast<float>((blk[2 + j] & 15) - 8) * d;
            out[32 * b + 16 + j] = static_cast<float>((blk[2 + j] >> 4) - 8) * d;
        }
    }
}

struct Matrix {
    int64_t N = 0, K = 0;
    std::vector<uint8_t> q;  // ggml Q4_0 bytes, N * K/32 * 18
    void *dev = nullptr;     // resident copy in HBM (inside qd_model::weights)
};

// The decode's GEMVs through the ggml plugin, the drop-in boundary: the
// weights are ggml tensors in the plugin's device buffer (set_tensor
// prepacks them), and each GEMV group is a graph of MUL_MAT nodes reading one
// activation tensor, run as ggml-backend runs a backend's split of a graph:
// the activation copied in (set_tensor_async), graph_compute (which sends
// consecutive nodes that share the activation to one multi-job launch), the
// outputs copied out (get_tensor_async), synchronize.  No ggml is linked
// here, so the harness names the MUL_MAT op id itself.
constexpr int kPluginOpMulMat = 29;

struct PluginDecode {
    ggml_backend *be = nullptr;
    // as llama.cpp allocates them: the weights in one buffer (usage WEIGHTS),
    // the graph's activations and outputs in a compute buffer
    ggml_backend_buffer *buf = nullptr, *cbuf = nullptr;
    std::vector<ggml_tensor> w, out;  // per matrix id: weight, MUL_MAT node
    ggml_tensor x{};                  // the activation row (ne[0] set per group)

    ~PluginDecode() {
        if (cbuf && cbuf->iface.free_buffer) cbuf->iface.free_buffer(cbuf);
        if (buf && buf->iface.free_buffer) buf->iface.free_buffer(buf);
        if (be) ggml_backend_mi355x_free(be);
    }
};

}  // namespace

struct qd_model {
    qd_config c{};
    int threads = 1;
    std::vector<Matrix> mats;  // 7 per layer, then the tied output/embedding
    std::vector<std::vector<float>> attn_norm, ffn_norm, bq, bk, bv;
    std::vector<float> out_norm;
    std::vector<float> last_logits;  // logits of the last generated token
    // device side
    mi355x_ctx *ctx = nullptr;
    void *weights = nullptr;  // every matrix, resident, back to back in id order
    bool fuse = true;         // one launch for matrices that are adjacent in HBM
    bool block = true;        // server mode: o through down as one command
    bool swiglu = true;       // server mode: gate|up, SiLU, down as one command
    int plugin_groups = GGML_MI355X_GROUPS_LAUNCH;  // plugin mode: how graph_compute runs a group
    int64_t last_launches = 0;
    float *dx = nullptr, *dy = nullptr;  // activation in, outputs out
    float *ffn_norm_dev = nullptr;       // the FFN norm weights, n_layers * hidden
    float *attn_norm_dev = nullptr;      // the attention norm weights, n_layers * hidden
    size_t dy_floats = 0;
    float *hx = nullptr, *hy = nullptr;  // pinned staging
    // device addresses of hx / hy (pinned host memory the kernels can read
    // and write directly over PCIe)
    const float *hx_dev = nullptr;
    float *hy_dev = nullptr;
    int io_mode = QD_IO_MAPPED;
    int wait_mode = QD_WAIT_SERVER;
    int variant = MI355X_VARIANT_AUTO;
    int last_wait = QD_WAIT_FENCE;  // the mode the last GPU decode used

    mi355x_server *server = nullptr;
    std::unique_ptr<PluginDecode> plugin;

    ~qd_model() {
        plugin.reset();
        if (server) mi355x_server_destroy(server);
        if (ctx) {
            if (weights) mi355x_free(ctx, weights);
            if (dx) mi355x_free(ctx, dx);
            if (dy) mi355x_free(ctx, dy);
            if (ffn_norm_dev) mi355x_free(ctx, ffn_norm_dev);
            if (attn_norm_dev) mi355x_free(ctx, attn_norm_dev);
            mi355x_ctx_destroy(ctx);
        }
        if (hx) mi355x_host_free(hx);
        if (hy) mi355x_host_free(hy);
    }

    int q_dim() const { return c.n_heads * c.head_dim; }
    int kv_dim() const { return c.n_kv_heads * c.head_dim; }
};

namespace {

void fill_matrix(Matrix &m, int64_t N, int64_t K, uint64_t seed, uint64_t stream) {
    m.N = N;
    m.K = K;
    const int64_t rb = K / 32 * 18;
    m.q.resize(static_cast<size_t>(N * rb));
#pragma omp parallel
    {
        std::vector<float> row(static_cast<size_t>(K));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < N; ++r) {
            Xoshiro rng(seed, stream, static_cast<uint64_t>(r));
            normals(rng, row.data(), K, 0.02f);
            quantize_q4_0_row(row.data(), K, m.q.data() + r * rb);
        }
    }
}

void fill_vector(std::vector<float> &v, int64_t n, uint64_t seed, uint64_t stream, bool ones) {
    v.resize(static_cast<size_t>(n));
    if (ones) {
        std::fill(v.begin(), v.end(), 1.0f);
        return;
    }
    Xoshiro rng(seed, stream, 0);
    normals(rng, v.data(), n, 0.02f);
}

void rmsnorm(const float *x, const float *w, float *out, int n, float eps) {
    // sum of squares in double (a float's square is exact there), in 16
    // interleaved partial sums so the loop runs at vector throughput
    __m256d acc[4] = {_mm256_setzero_pd(), _mm256_setzero_pd(), _mm256_setzero_pd(), _mm256_setzero_pd()};
    int i0 = 0;
    for (; i0 + 16 <= n; i0 += 16)
        for (int j = 0; j < 4; ++j) {
            const __m256d v = _mm256_cvtps_pd(_mm_loadu_ps(x + i0 + 4 * j));
            acc[j] = _mm256_fmadd_pd(v, v, acc[j]);
        }
    alignas(32) double lanes[4];
    _mm256_store_pd(lanes, _mm256_add_pd(_mm256_add_pd(acc[0], acc[1]), _mm256_add_pd(acc[2], acc[3])));
    double ss = (lanes[0] + lanes[1]) + (lanes[2] + lanes[3]);
    for (int i = i0; i < n; ++i) ss += static_cast<double>(x[i]) * x[i];
    const float s = 1.0f / std::sqrt(static_cast<float>(ss / n) + eps);
    for (int i = 0; i < n; ++i) out[i] = x[i] * s * w[i];
}

// rotate-half RoPE of one head vector; cs holds cos then sin of
// pos * theta^(-2i/hd) for i < hd/2
void rope(float *v, int hd, const float *cs) {
    const int h = hd / 2;
    for (int i = 0; i < h; ++i) {
        const float c = cs[i], s = cs[h + i];
        const float a = v[i], b = v[i + h];
        v[i] = a * c - b * s;
        v[i + h] = b * c + a * s;
    }
}

// e^x for the host ops, written to vectorize: x = n ln2 + r with n =
// round(x / ln2) and |r| <= ln2/2 (Cody-Waite split of ln2 into a part exact
// in float and a remainder), e^r by its degree-7 Taylor polynomial (relative
// error < 5e-9 on that range), times 2^n built in the exponent bits.  Inputs
// below -87.3 give 0, above 88 are clamped to 88 (the callers never get there:
// softmax arguments are <= 0, SiLU's are -g).  Every multiply-add is an
// explicit fma, so the result does not depend on the compiler's contraction
// choices: these are the steps of mi355x_server_swiglu's SiLU, which gives the
// same bits on the GPU (the one product left, p * 2^n, is exact unless it is
// subnormal, where 1 + e^x rounds to 1 either way).
inline float fast_exp(float x) {
    const float xc = std::min(std::max(x, -87.3f), 88.0f);
    // round to nearest by adding and subtracting 1.5 * 2^23 (|x / ln2| < 2^22)
    const float n = std::fma(xc, 1.44269504088896341f, 12582912.0f) - 12582912.0f;
    const float r = std::fma(-n, 1.42860682030941723e-6f, std::fma(-n, 0.693145751953125f, xc));
    float p = 1.0f / 5040.0f;
    p = std::fma(p, r, 1.0f / 720.0f);
    p = std::fma(p, r, 1.0f / 120.0f);
    p = std::fma(p, r, 1.0f / 24.0f);
    p = std::fma(p, r, 1.0f / 6.0f);
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    const int32_t bits = (static_cast<int32_t>(n) + 127) << 23;
    float scale;
    std::memcpy(&scale, &bits, 4);
    const float e = p * scale;  // computed unconditionally so the select vectorizes
    return x < -87.3f ? 0.0f : e;
}

// g[i] = silu(g[i]) * u[i] = g / (1 + e^-g) * u
void silu_mul(float *g, const float *u, int n) {
#pragma omp simd
    for (int i = 0; i < n; ++i) g[i] = g[i] / (1.0f + fast_exp(-g[i])) * u[i];
}

// Grouped-query attention of one position over n_t cached positions:
// att[h] = softmax(q[h] . K_g^T / sqrt(hd)) V_g, g = h / (n_heads / n_kv).
// Cache layouts (tcap = capacity, a multiple of 8):
//   K: [g][t / 8][i][t % 8] -- 8 positions of one dimension side by side, so
//      a score pass covers 8 positions per AVX2 register for up to 8 heads
//      that share K_g, reading 4 KB contiguous blocks (unused slots zero);
//   V: [g][t][i].
// Passes: scores (in blocks of 32 positions), softmax per head, then P V in
// 8-wide slices of the head dimension.  sc has n_heads * tcap floats.
template <int NJ>
void scores_block(const float *q, const float *Kg, int hd, int tcap, int t0, int t1, float scale, float *sc) {
    for (int t = t0; t < t1; t += 8) {
        const float *blk = Kg + static_cast<size_t>(t) * hd;  // block t / 8 starts at (t / 8) * 8 * hd
        __m256 acc[NJ];
        for (int j = 0; j < NJ; ++j) acc[j] = _mm256_setzero_ps();
        for (int i = 0; i < hd; ++i) {
            const __m256 k = _mm256_loadu_ps(blk + 8 * i);
            for (int j = 0; j < NJ; ++j) acc[j] = _mm256_fmadd_ps(_mm256_set1_ps(q[j * hd + i]), k, acc[j]);
        }
        const __m256 sv = _mm256_set1_ps(scale);
        for (int j = 0; j < NJ; ++j) _mm256_storeu_ps(sc + static_cast<size_t>(j) * tcap + t, _mm256_mul_ps(acc[j], sv));
    }
}

template <int NJ>
void pv_slice(const float *P, const float *V, int hd, int tcap, int n_t, float *out) {
    __m256 acc[NJ];
    for (int j = 0; j < NJ; ++j) acc[j] = _mm256_setzero_ps();
    for (int t = 0; t < n_t; ++t) {
        const __m256 v = _mm256_loadu_ps(V + static_cast<size_t>(t) * hd);
        for (int j = 0; j < NJ; ++j)
            acc[j] = _mm256_fmadd_ps(_mm256_set1_ps(P[static_cast<size_t>(j) * tcap + t]), v, acc[j]);
    }
    for (int j = 0; j < NJ; ++j) _mm256_storeu_ps(out + static_cast<size_t>(j) * hd, acc[j]);
}

typedef void (*scores_fn)(const float *, const float *, int, int, int, int, float, float *);
typedef void (*pv_fn)(const float *, const float *, int, int, int, float *);
constexpr scores_fn kScores[8] = {scores_block<1>, scores_block<2>, scores_block<3>, scores_block<4>,
                                  scores_block<5>, scores_block<6>, scores_block<7>, scores_block<8>};
constexpr pv_fn kPv[8] = {pv_slice<1>, pv_slice<2>, pv_slice<3>, pv_slice<4>,
                          pv_slice<5>, pv_slice<6>, pv_slice<7>, pv_slice<8>};

constexpr int kAttThreads = 8;

void attention(const float *q, const float *K, const float *V, int n_t, int tcap, int n_heads, int n_kv, int hd,
               float *sc, float *att) {
    const int group = n_heads / n_kv;
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    const int hb_count = (group + 7) / 8;  // blocks of up to 8 heads per KV head
    const int n_chunks = (n_t + 31) / 32;  // score blocks: enough tasks for a 16-thread team
    const int n_slices = hd / 8;
    // a thread team pays off only for long contexts, and a team of more
    // than kAttThreads costs more in synchronisation than it saves
#pragma omp parallel if (n_t >= 64) num_threads(std::min(omp_get_max_threads(), kAttThreads))
    {
#pragma omp for collapse(3) schedule(static)
        for (int g = 0; g < n_kv; ++g)
            for (int hb = 0; hb < hb_count; ++hb)
                for (int ch = 0; ch < n_chunks; ++ch) {
                    const int h0 = g * group + 8 * hb, nj = std::min(8, group - 8 * hb);
                    kScores[nj - 1](q + static_cast<size_t>(h0) * hd, K + static_cast<size_t>(g) * hd * tcap, hd,
                                    tcap, 32 * ch, std::min(n_t, 32 * ch + 32), scale,
                                    sc + static_cast<size_t>(h0) * tcap);
                }
#pragma omp for schedule(static)
        for (int h = 0; h < n_heads; ++h) {
            float *p = sc + static_cast<size_t>(h) * tcap;
            float mx = -INFINITY;
#pragma omp simd reduction(max : mx)
            for (int t = 0; t < n_t; ++t) mx = std::max(mx, p[t]);
            float sum = 0.f;
#pragma omp simd reduction(+ : sum)
            for (int t = 0; t < n_t; ++t) {
                p[t] = fast_exp(p[t] - mx);
                sum += p[t];
            }
            const float inv = 1.0f / sum;
#pragma omp simd
            for (int t = 0; t < n_t; ++t) p[t] *= inv;
        }
#pragma omp for collapse(3) schedule(static)
        for (int g = 0; g < n_kv; ++g)
            for (int hb = 0; hb < hb_count; ++hb)
                for (int sl = 0; sl < n_slices; ++sl) {
                    const int h0 = g * group + 8 * hb, nj = std::min(8, group - 8 * hb);
                    kPv[nj - 1](sc + static_cast<size_t>(h0) * tcap, V + static_cast<size_t>(g) * hd * tcap + 8 * sl, hd,
                                tcap, n_t, att + static_cast<size_t>(h0) * hd + 8 * sl);
                }
    }
}

// index of the first largest element, as std::max_element: 32 lanes (four
// independent registers, so the compare-select chains overlap) each keep
// their first maximum above -inf (strict >), then ties go to the lowest
// index.  NaNs never win, except at index 0, where max_element keeps them.
int argmax(const float *x, int n) {
    if (n < 64 || std::isnan(x[0])) return static_cast<int>(std::max_element(x, x + n) - x);
    __m256 best[4];
    __m256i bi[4], idx[4];
    for (int a = 0; a < 4; ++a) {
        best[a] = _mm256_set1_ps(-INFINITY);
        bi[a] = _mm256_set1_epi32(-1);
        idx[a] = _mm256_add_epi32(_mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7), _mm256_set1_epi32(8 * a));
    }
    const __m256i step = _mm256_set1_epi32(32);
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int a = 0; a < 4; ++a) {
            const __m256 v = _mm256_loadu_ps(x + i + 8 * a);
            const __m256 gt = _mm256_cmp_ps(v, best[a], _CMP_GT_OQ);
            best[a] = _mm256_blendv_ps(best[a], v, gt);
            bi[a] = _mm256_blendv_epi8(bi[a], idx[a], _mm256_castps_si256(gt));
            idx[a] = _mm256_add_epi32(idx[a], step);
        }
    alignas(32) float bv[32];
    alignas(32) int32_t bx[32];
    for (int a = 0; a < 4; ++a) {
        _mm256_store_ps(bv + 8 * a, best[a]);
        _mm256_store_si256(reinterpret_cast<__m256i *>(bx + 8 * a), bi[a]);
    }
    int r = -1;
    float rv = -INFINITY;
    for (int l = 0; l < 32; ++l)
        if (bx[l] >= 0 && (r < 0 || bv[l] > rv || (bv[l] == rv && bx[l] < r))) {
            rv = bv[l];
            r = bx[l];
        }
    for (; i < n; ++i)
        if (x[i] > rv) {
            rv = x[i];
            r = i;
        }
    return r < 0 ? 0 : r;  // nothing above -inf: max_element keeps index 0
}

double now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

extern "C" {

const char *qd_last_error(void) { return g_err.c_str(); }

void qd_quantize_q4_0(const float *x, int64_t N, int64_t K, uint8_t *out) {
    for (int64_t r = 0; r < N; ++r) quantize_q4_0_row(x + r * K, K, out + r * (K / 32) * 18);
}

qd_model *qd_model_create(const qd_config *cfg, int threads) {
    if (!cfg || cfg->n_layers <= 0 || cfg->hidden % 32 || cfg->ffn % 32 || cfg->head_dim % 8 ||
        cfg->n_heads % cfg->n_kv_heads) {
        fail("qd_model_create: invalid configuration");
        return nullptr;
    }
    auto m = std::make_unique<qd_model>();
    m->c = *cfg;
    m->threads = std::max(1, threads);
    omp_set_num_threads(m->threads);
    const int L = cfg->n_layers, H = cfg->hidden;
    m->mats.resize(static_cast<size_t>(7 * L + 1));
    for (int l = 0; l < L; ++l) {
        const uint64_t s = static_cast<uint64_t>(l) * 16;
        fill_matrix(m->mats[7 * l + QD_Q], m->q_dim(), H, cfg->seed, s + 0);
        fill_matrix(m->mats[7 * l + QD_K], m->kv_dim(), H, cfg->seed, s + 1);
        fill_matrix(m->mats[7 * l + QD_V], m->kv_dim(), H, cfg->seed, s + 2);
        fill_matrix(m->mats[7 * l + QD_O], H, m->q_dim(), cfg->seed, s + 3);
        fill_matrix(m->mats[7 * l + QD_GATE], cfg->ffn, H, cfg->seed, s + 4);
        fill_matrix(m->mats[7 * l + QD_UP], cfg->ffn, H, cfg->seed, s + 5);
        fill_matrix(m->mats[7 * l + QD_DOWN], H, cfg->ffn, cfg->seed, s + 6);
        m->attn_norm.emplace_back();
        m->ffn_norm.emplace_back();
        m->bq.emplace_back();
        m->bk.emplace_back();
        m->bv.emplace_back();
        fill_vector(m->attn_norm.back(), H, cfg->seed, s + 7, true);
        fill_vector(m->ffn_norm.back(), H, cfg->seed, s + 8, true);
        fill_vector(m->bq.back(), m->q_dim(), cfg->seed, s + 9, false);
        fill_vector(m->bk.back(), m->kv_dim(), cfg->seed, s + 10, false);
        fill_vector(m->bv.back(), m->kv_dim(), cfg->seed, s + 11, false);
    }
    fill_matrix(m->mats[7 * L], cfg->vocab, H, cfg->seed, 1u << 20);
    fill_vector(m->out_norm, H, cfg->seed, (1u << 20) + 1, true);
    return m.release();
}

void qd_model_free(qd_model *m) { delete m; }

int qd_n_matrices(const qd_model *m) { return m ? static_cast<int>(m->mats.size()) : 0; }

const float *qd_vector(const qd_model *m, int id, int *n) {
    if (!m || id < 0 || id > 5 * m->c.n_layers) return nullptr;
    const std::vector<float> *v = &m->out_norm;
    if (id < 5 * m->c.n_layers) {
        const int l = id / 5;
        const std::vector<float> *per[5] = {&m->attn_norm[l], &m->ffn_norm[l], &m->bq[l], &m->bk[l], &m->bv[l]};
        v = per[id % 5];
    }
    if (n) *n = static_cast<int>(v->size());
    return v->data();
}

void qd_set_fuse(qd_model *m, int on) {
    if (m) m->fuse = on != 0;
}

int qd_set_variant(qd_model *m, int variant) {
    if (!m || !m->ctx) return fail("qd_set_variant: qd_attach_gpu first");
    if (mi355x_ctx_set_option(m->ctx, MI355X_OPT_VARIANT, variant) != MI355X_OK)
        return fail(std::string("qd_set_variant: ") + mi355x_last_error());
    m->variant = variant;
    return 0;
}

int qd_set_io(qd_model *m, int mode) {
    if (!m) return fail("qd_set_io: null model");
    if (mode != QD_IO_STAGED && mode != QD_IO_MAPPED) return fail("qd_set_io: unknown mode");
    m->io_mode = mode;
    return 0;
}

int qd_set_wait(qd_model *m, int mode) {
    if (!m) return fail("qd_set_wait: null model");
    if (mode != QD_WAIT_STREAM && mode != QD_WAIT_FENCE && mode != QD_WAIT_SERVER && mode != QD_WAIT_PLUGIN)
        return fail("qd_set_wait: unknown mode");
    m->wait_mode = mode;
    return 0;
}

int64_t qd_last_launches(const qd_model *m) { return m ? m->last_launches : 0; }

int qd_last_wait(const qd_model *m) { return m ? m->last_wait : -1; }

int qd_last_logits(const qd_model *m, float *out, int n) {
    if (!m || !out || n != m->c.vocab || m->last_logits.size() != static_cast<size_t>(n))
        return fail("qd_last_logits: no logits of that size");
    std::memcpy(out, m->last_logits.data(), static_cast<size_t>(n) * 4);
    return 0;
}

const uint8_t *qd_matrix(const qd_model *m, int id, int64_t *N, int64_t *K) {
    if (!m || id < 0 || id >= static_cast<int>(m->mats.size())) return nullptr;
    if (N) *N = m->mats[id].N;
    if (K) *K = m->mats[id].K;
    return m->mats[id].q.data();
}

int qd_attach_gpu(qd_model *m, int device) {
    if (!m) return fail("qd_attach_gpu: null model");
    if (m->weights) return 0;
    if (!m->ctx && mi355x_ctx_create(device, &m->ctx) != MI355X_OK)
        return fail(std::string("qd_attach_gpu: ") + mi355x_last_error());
    // One allocation, matrices in id order.  Resident Q4_0 rows are
    // contiguous, so q|k|v and gate|up form single taller matrices whenever
    // no alignment padding separates them (row bytes a multiple of 16).
    std::vector<size_t> off(m->mats.size());
    size_t total = 0;
    for (size_t i = 0; i < m->mats.size(); ++i) {
        off[i] = total;
        total = (total + m->mats[i].q.size() + 15) / 16 * 16;
    }
    if (mi355x_malloc(m->ctx, total, &m->weights) != MI355X_OK)
        return fail(std::string("qd_attach_gpu: ") + mi355x_last_error());
    for (size_t i = 0; i < m->mats.size(); ++i) {
        Matrix &mat = m->mats[i];
        mat.dev = static_cast<uint8_t *>(m->weights) + off[i];
        if (mi355x_prepack_from_host(m->ctx, MI355X_TYPE_Q4_0, mat.N, mat.K, mat.dev, mat.q.data(), 0, mat.q.size()) !=
            MI355X_OK)
            return fail(std::string("qd_attach_gpu: ") + mi355x_last_error());
    }
    const size_t xf = static_cast<size_t>(std::max(m->c.ffn, std::max(m->c.hidden, m->q_dim())));
    // outputs of a block command: y, then the next layer's q|k|v
    m->dy_floats = static_cast<size_t>(std::max<int64_t>(
        2 * m->c.ffn, std::max<int64_t>(m->c.vocab, m->c.hidden + m->q_dim() + 2 * m->kv_dim())));
    void *p = nullptr;
    if (mi355x_malloc(m->ctx, xf * 4, &p) != MI355X_OK) return fail(mi355x_last_error());
    m->dx = static_cast<float *>(p);
    if (mi355x_malloc(m->ctx, m->dy_floats * 4, &p) != MI355X_OK) return fail(mi355x_last_error());
    m->dy = static_cast<float *>(p);
    if (mi355x_host_malloc(xf * 4, &p) != MI355X_OK) return fail(mi355x_last_error());
    m->hx = static_cast<float *>(p);
    if (mi355x_host_malloc(m->dy_floats * 4, &p) != MI355X_OK) return fail(mi355x_last_error());
    m->hy = static_cast<float *>(p);
    void *dp = nullptr;
    if (hipHostGetDevicePointer(&dp, m->hx, 0) != hipSuccess) return fail("qd_attach_gpu: hipHostGetDevicePointer");
    m->hx_dev = static_cast<const float *>(dp);
    if (hipHostGetDevicePointer(&dp, m->hy, 0) != hipSuccess) return fail("qd_attach_gpu: hipHostGetDevicePointer");
    m->hy_dev = static_cast<float *>(dp);
    const size_t H = static_cast<size_t>(m->c.hidden);
    if (mi355x_malloc(m->ctx, m->c.n_layers * H * 4, &p) != MI355X_OK) return fail(mi355x_last_error());
    m->ffn_norm_dev = static_cast<float *>(p);
    if (mi355x_malloc(m->ctx, m->c.n_layers * H * 4, &p) != MI355X_OK) return fail(mi355x_last_error());
    m->attn_norm_dev = static_cast<float *>(p);
    for (int l = 0; l < m->c.n_layers; ++l)
        if (mi355x_memcpy_h2d(m->ctx, m->ffn_norm_dev + l * H, m->ffn_norm[l].data(), H * 4) != MI355X_OK ||
            mi355x_memcpy_h2d(m->ctx, m->attn_norm_dev + l * H, m->attn_norm[l].data(), H * 4) != MI355X_OK)
            return fail(mi355x_last_error());
    return 0;
}

namespace {

// Puts every matrix into the plugin's buffer on the context's device and
// builds the MUL_MAT nodes (weights, then node outputs, then the activation
// row, each at the buffer type's alignment).
int attach_plugin(qd_model *m) {
    if (m->plugin) return 0;
    if (!m->ctx) return fail("plugin decode: qd_attach_gpu first");
    const int device = mi355x_ctx_device(m->ctx);
    if (!ggml_backend_mi355x_set_op_mul_mat(kPluginOpMulMat)) return fail("plugin decode: op id");
    auto P = std::make_unique<PluginDecode>();
    P->be = ggml_backend_mi355x_init(static_cast<size_t>(device));
    if (!P->be) return fail("plugin decode: ggml_backend_mi355x_init failed");
    ggml_backend_buffer_type *buft = ggml_backend_mi355x_buffer_type(static_cast<size_t>(device));
    if (!buft) return fail("plugin decode: no buffer type");
    const size_t al = buft->iface.get_alignment(buft);
    auto up = [al](size_t v) { return (v + al - 1) / al * al; };
    const size_t n = m->mats.size();
    std::vector<size_t> woff(n), ooff(n);
    size_t total = 0, ctotal = 0;
    int64_t max_k = 0;
    for (size_t i = 0; i < n; ++i) {
        woff[i] = total;
        total = up(total + m->mats[i].q.size());
        max_k = std::max(max_k, m->mats[i].K);
    }
    for (size_t i = 0; i < n; ++i) {
        ooff[i] = ctotal;
        ctotal = up(ctotal + static_cast<size_t>(m->mats[i].N) * 4);
    }
    const size_t xoff = ctotal;
    ctotal = up(ctotal + static_cast<size_t>(max_k) * 4);
    P->buf = buft->iface.alloc_buffer(buft, total);
    if (!P->buf) return fail("plugin decode: buffer allocation failed");
    P->buf->usage = GGML_BACKEND_BUFFER_USAGE_WEIGHTS;
    P->cbuf = buft->iface.alloc_buffer(buft, ctotal);
    if (!P->cbuf) return fail("plugin decode: compute buffer allocation failed");
    P->cbuf->usage = GGML_BACKEND_BUFFER_USAGE_COMPUTE;
    auto *base = static_cast<uint8_t *>(P->buf->iface.get_base(P->buf));
    auto *cbase = static_cast<uint8_t *>(P->cbuf->iface.get_base(P->cbuf));
    P->w.resize(n);
    P->out.resize(n);
    P->x.type = GGML_TYPE_F32;
    P->x.buffer = P->cbuf;
    P->x.data = cbase + xoff;
    std::snprintf(P->x.name, sizeof(P->x.name), "x");
    for (size_t i = 0; i < n; ++i) {
        const Matrix &mat = m->mats[i];
        const size_t rb = static_cast<size_t>(mat.K / 32 * 18);
        ggml_tensor &w = P->w[i];
        w.type = GGML_TYPE_Q4_0;
        w.ne[0] = mat.K;
        w.ne[1] = mat.N;
        w.ne[2] = w.ne[3] = 1;
        w.nb[0] = 18;
        w.nb[1] = rb;
        w.nb[2] = w.nb[3] = rb * static_cast<size_t>(mat.N);
        w.buffer = P->buf;
        w.data = base + woff[i];
        std::snprintf(w.name, sizeof(w.name), "w%zu", i);
        if (P->buf->iface.init_tensor && P->buf->iface.init_tensor(P->buf, &w) != GGML_STATUS_SUCCESS)
            return fail("plugin decode: init_tensor failed");
        P->buf->iface.set_tensor(P->buf, &w, mat.q.data(), 0, mat.q.size());
        ggml_tensor &o = P->out[i];
        o.type = GGML_TYPE_F32;
        o.ne[0] = mat.N;
        o.ne[1] = o.ne[2] = o.ne[3] = 1;
        o.nb[0] = 4;
        o.nb[1] = o.nb[2] = o.nb[3] = static_cast<size_t>(mat.N) * 4;
        o.op = kPluginOpMulMat;
        o.src[0] = &P->w[i];
        o.src[1] = &P->x;
        o.buffer = P->cbuf;
        o.data = cbase + ooff[i];
        std::snprintf(o.name, sizeof(o.name), "mm%zu", i);
    }
    P->be->iface.synchronize(P->be);
    m->plugin = std::move(P);
    return 0;
}

}  // namespace

int qd_generate(qd_model *m, int backend, qd_gemv_fn cpu_gemv, void *user, const int32_t *prompt, int n_prompt,
                int n_gen, int32_t *out_tokens, double *timings) {
    if (!m || !prompt || n_prompt <= 0 || n_gen < 0 || (n_gen > 0 && !out_tokens))
        return fail("qd_generate: bad arguments");
    if (backend == 0 && !m->ctx) return fail("qd_generate: qd_attach_gpu first");
    if (backend == 1 && !cpu_gemv) return fail("qd_generate: no CPU GEMV");
    const qd_config &c = m->c;
    const int H = c.hidden, QD = m->q_dim(), KVD = m->kv_dim(), hd = c.head_dim;
    const int L = c.n_layers, T = n_prompt + std::max(n_gen, 1);
    omp_set_num_threads(m->threads);
    // the server computes the digit-plane arithmetic or ggml-cpu's Q8_0
    // numerics on rows of multiples of 256 values; the exact-f32 variant and
    // other shapes take launch + fence
    const bool use_plugin = backend == 0 && m->wait_mode == QD_WAIT_PLUGIN;
    if (use_plugin) {
        if (attach_plugin(m)) return -1;
        if (!ggml_backend_mi355x_set_kernel_variant(m->plugin->be, m->variant))
            return fail("qd_generate: plugin kernel variant");
        if (!ggml_backend_mi355x_set_group_mode(m->plugin->be, m->plugin_groups))
            return fail("qd_generate: plugin group mode");
    }
    bool use_server = backend == 0 && m->wait_mode == QD_WAIT_SERVER && m->variant != MI355X_VARIANT_EXACT_F32;
    int64_t max_k = 0;
    for (const Matrix &mat : m->mats) {
        max_k = std::max<int64_t>(max_k, mat.K);
        if (mat.K % 256 != 0) use_server = false;
    }
    // the block command's payload is the attention output and the residual
    max_k = std::max<int64_t>(max_k, (m->q_dim() + H + 255) / 256 * 256);
    if (use_server && !m->server && mi355x_server_create(m->ctx, max_k, &m->server) != MI355X_OK)
        use_server = false;  // e.g. no cooperative launch: one launch per group
    const int wait = !use_server && m->wait_mode == QD_WAIT_SERVER ? QD_WAIT_FENCE : m->wait_mode;
    // the feed-forward block as one SwiGLU server command (fused groups
    // only); with `block`, also o, both residual adds and the FFN norm
    const bool swiglu = backend == 0 && use_server && m->fuse && m->swiglu && c.ffn % 256 == 0;
    const bool block = swiglu && m->block && H % 256 == 0 && H <= 4096 && QD % 256 == 0;
    // q, k and v back to back in HBM: the block command can run them as one job
    bool qkv_adjacent = true;
    for (int l = 0; l < L; ++l) {
        const Matrix &mq = m->mats[7 * l + QD_Q], &mk = m->mats[7 * l + QD_K], &mv = m->mats[7 * l + QD_V];
        const auto *bq = static_cast<const uint8_t *>(mq.dev), *bk = static_cast<const uint8_t *>(mk.dev);
        qkv_adjacent = qkv_adjacent && mk.dev == bq + mq.N * (H / 32) * 18 && mv.dev == bk + mk.N * (H / 32) * 18;
    }

    // per layer: keys [g][t / 8][i][t % 8], values [g][t][i] (see attention())
    const int tcap = (T + 7) / 8 * 8;
    std::vector<float> kc(static_cast<size_t>(L) * KVD * tcap, 0.0f), vc(static_cast<size_t>(L) * KVD * tcap);
    std::vector<float> h(H), xn(std::max(H, c.ffn)), q(QD), k(KVD), v(KVD), att(QD), o(H), g(c.ffn), u(c.ffn),
        dn(H), logits(c.vocab);
    std::vector<float> inv_freq(hd / 2), rope_cs(hd), sc(static_cast<size_t>(c.n_heads) * tcap);
    for (int i = 0; i < hd / 2; ++i)
        inv_freq[i] = std::pow(c.rope_theta, -2.0f * static_cast<float>(i) / static_cast<float>(hd));
    double t_gemv = 0.0, t_host = 0.0;
    int64_t launches = 0;
    int rc = 0;

    // GEMVs that share one activation: y_i = W_ids[i] x; outputs land in
    // outs[i].  Staged I/O uploads x once and downloads all outputs once;
    // mapped I/O lets the kernels read x from, and write y to, pinned host
    // memory (outputs above kMappedOutMax floats still go through HBM and
    // one copy: a 600 KB vocabulary row is faster as one DMA).
    constexpr int64_t kMappedOutMax = 65536;
    auto gemvs = [&](const float *x, int64_t K, std::initializer_list<int> ids, std::initializer_list<float *> outs) {
        const double t0 = now();
        if (use_plugin) {
            PluginDecode &P = *m->plugin;
            P.x.ne[0] = K;
            P.x.ne[1] = P.x.ne[2] = P.x.ne[3] = 1;
            P.x.nb[0] = 4;
            P.x.nb[1] = P.x.nb[2] = P.x.nb[3] = static_cast<size_t>(K) * 4;
            P.be->iface.set_tensor_async(P.be, &P.x, x, 0, static_cast<size_t>(K) * 4);
            ggml_tensor *nodes[8];
            int nn = 0;
            for (int id : ids) nodes[nn++] = &P.out[id];
            ggml_cgraph g{};
            g.size = g.n_nodes = nn;
            g.nodes = nodes;
            if (P.be->iface.graph_compute(P.be, &g) != GGML_STATUS_SUCCESS) return -1;
            auto oi = outs.begin();
            for (int id : ids)
                P.be->iface.get_tensor_async(P.be, &P.out[id], *oi++, 0, static_cast<size_t>(m->mats[id].N) * 4);
            P.be->iface.synchronize(P.be);
            launches += nn;  // nodes
        } else if (backend == 0 && use_server) {
            // one server command per group: runs of matrices adjacent in HBM
            // with the same K are one job, outputs land in pinned memory
            mi355x_server_job jobs[4];
            int nj = 0;
            int64_t off = 0;
            const Matrix *run = nullptr;
            for (int id : ids) {
                const Matrix &mat = m->mats[id];
                if (run && m->fuse && mat.K == run->K &&
                    mat.dev == static_cast<const uint8_t *>(jobs[nj - 1].W) + jobs[nj - 1].N * (run->K / 32) * 18) {
                    jobs[nj - 1].N += mat.N;
                } else {
                    if (nj == 4) return -1;
                    jobs[nj++] = {mat.dev, mat.N, m->hy_dev + off};
                }
                off += mat.N;
                run = &mat;
            }
            if (mi355x_server_gemv(m->server, x, K, nj, jobs) != MI355X_OK) return -1;
            launches += nj;
            off = 0;
            auto oi = outs.begin();
            for (int id : ids) {
                std::memcpy(*oi++, m->hy + off, static_cast<size_t>(m->mats[id].N) * 4);
                off += m->mats[id].N;
            }
        } else if (backend == 0) {
            // all on the context's stream: one wait per group
            const hipStream_t st = static_cast<hipStream_t>(mi355x_ctx_stream(m->ctx));
            int64_t n_out = 0;
            for (int id : ids) n_out += m->mats[id].N;
            const bool map_x = m->io_mode == QD_IO_MAPPED;
            const bool map_y = map_x && n_out <= kMappedOutMax;
            const float *xin = map_x ? m->hx_dev : m->dx;
            float *yout = map_y ? m->hy_dev : m->dy;
            std::memcpy(m->hx, x, static_cast<size_t>(K) * 4);
            if (!map_x &&
                hipMemcpyAsync(m->dx, m->hx, static_cast<size_t>(K) * 4, hipMemcpyHostToDevice, st) != hipSuccess)
                return -1;
            // consecutive matrices adjacent in HBM with the same K run as one
            int64_t off = 0, run_n = 0;
            const Matrix *run = nullptr;
            for (int id : ids) {
                const Matrix &mat = m->mats[id];
                if (run && m->fuse && mat.K == run->K &&
                    mat.dev == static_cast<const uint8_t *>(run->dev) + run_n * (run->K / 32) * 18) {
                    run_n += mat.N;
                    continue;
                }
                if (run && mi355x_gemv(m->ctx, MI355X_TYPE_Q4_0, run->dev, run_n, run->K, xin, yout + off) != MI355X_OK)
                    return -1;
                if (run) ++launches;
                off += run_n;
                run = &mat;
                run_n = mat.N;
            }
            if (mi355x_gemv(m->ctx, MI355X_TYPE_Q4_0, run->dev, run_n, run->K, xin, yout + off) != MI355X_OK)
                return -1;
            off += run_n;
            ++launches;
            if (!map_y &&
                hipMemcpyAsync(m->hy, m->dy, static_cast<size_t>(off) * 4, hipMemcpyDeviceToHost, st) != hipSuccess)
                return -1;
            // the outputs are in pinned host memory, which the fence covers
            if ((wait == QD_WAIT_FENCE ? mi355x_ctx_fence(m->ctx) : mi355x_ctx_sync(m->ctx)) != MI355X_OK)
                return -1;
            off = 0;
            auto oi = outs.begin();
            for (int id : ids) {
                std::memcpy(*oi++, m->hy + off, static_cast<size_t>(m->mats[id].N) * 4);
                off += m->mats[id].N;
            }
        } else {
            auto oi = outs.begin();
            for (int id : ids) {
                const Matrix &mat = m->mats[id];
                if (cpu_gemv(user, id, mat.q.data(), mat.N, mat.K, x, *oi++) != 0) return -1;
            }
        }
        t_gemv += now() - t0;
        return 0;
    };

    // positions 0 .. n_prompt-1 take the prompt; the logits after the last
    // prompt token give generated token 0, and each of positions n_prompt ..
    // n_prompt + n_gen - 2 takes the previous generated token and yields the
    // next: n_gen - 1 forward passes in the generation phase
    const double t_start = now();
    double t_gen0 = t_start;
    const int n_pos = n_gen > 0 ? n_prompt + n_gen - 1 : n_prompt;
    int32_t tok = prompt[0];
    for (int pos = 0; pos < n_pos; ++pos) {
        if (pos == n_prompt) {
            t_gen0 = now();
            t_gemv = 0.0;
            launches = 0;
            t_host = 0.0;
        }
        if (pos < n_prompt) tok = prompt[pos];
        double th = now();
        for (int i = 0; i < hd / 2; ++i) {
            const float f = static_cast<float>(pos) * inv_freq[i];
            rope_cs[i] = std::cos(f);
            rope_cs[hd / 2 + i] = std::sin(f);
        }
        dequant_q4_0_row(m->mats[7 * L].q.data() + static_cast<int64_t>(tok) * (H / 32) * 18, H, h.data());
        bool have_qkv = false;    // the last block command computed this layer's q|k|v
        bool have_dev_h = false;  // the server holds the residual (a block command ran this pass)
        for (int l = 0; l < L; ++l) {
            if (have_qkv) {
                std::memcpy(q.data(), m->hy + H, static_cast<size_t>(QD) * 4);
                std::memcpy(k.data(), m->hy + H + QD, static_cast<size_t>(KVD) * 4);
                std::memcpy(v.data(), m->hy + H + QD + KVD, static_cast<size_t>(KVD) * 4);
                have_qkv = false;
            } else {
                rmsnorm(h.data(), m->attn_norm[l].data(), xn.data(), H, c.norm_eps);
                t_host += now() - th;
                if ((rc = gemvs(xn.data(), H, {7 * l + QD_Q, 7 * l + QD_K, 7 * l + QD_V},
                                {q.data(), k.data(), v.data()})))
                    break;
                th = now();
            }
            for (int i = 0; i < QD; ++i) q[i] += m->bq[l][i];
            for (int i = 0; i < KVD; ++i) {
                k[i] += m->bk[l][i];
                v[i] += m->bv[l][i];
            }
            for (int hh = 0; hh < c.n_heads; ++hh) rope(q.data() + hh * hd, hd, rope_cs.data());
            for (int hh = 0; hh < c.n_kv_heads; ++hh) rope(k.data() + hh * hd, hd, rope_cs.data());
            float *kl = kc.data() + static_cast<size_t>(l) * KVD * tcap, *vl = vc.data() + static_cast<size_t>(l) * KVD * tcap;
            for (int g = 0; g < c.n_kv_heads; ++g) {
                float *kb = kl + static_cast<size_t>(g) * hd * tcap + static_cast<size_t>(pos / 8) * 8 * hd + pos % 8;
                for (int i = 0; i < hd; ++i) kb[8 * i] = k[g * hd + i];
                std::memcpy(vl + (static_cast<size_t>(g) * tcap + pos) * hd, v.data() + g * hd, static_cast<size_t>(hd) * 4);
            }
            attention(q.data(), kl, vl, pos + 1, tcap, c.n_heads, c.n_kv_heads, hd, sc.data(), att.data());
            t_host += now() - th;
            if (block) {
                // o, residual, FFN norm, gate|up, SiLU, down, residual -- and
                // the next layer's attention norm and q|k|v -- one command
                const double t0 = now();
                const Matrix &wo = m->mats[7 * l + QD_O], &wg = m->mats[7 * l + QD_GATE],
                             &wu = m->mats[7 * l + QD_UP], &wd = m->mats[7 * l + QD_DOWN];
                const bool next = l + 1 < L && qkv_adjacent;
                const Matrix &wq = m->mats[7 * (next ? l + 1 : l) + QD_Q];
                // the residual stays in the server between layers: the host
                // sends it with layer 0 and reads it back when it needs it
                const bool need_h = !next;
                if (mi355x_server_block(m->server, att.data(), QD, wo.dev, l == 0 || !have_dev_h ? h.data() : nullptr,
                                        H, m->ffn_norm_dev + static_cast<size_t>(l) * H, c.norm_eps, wg.dev, wu.dev,
                                        c.ffn, wd.dev, need_h ? m->hy_dev : nullptr,
                                        next ? m->attn_norm_dev + static_cast<size_t>(l + 1) * H : nullptr,
                                        next ? wq.dev : nullptr, QD + 2 * KVD, m->hy_dev + H) != MI355X_OK) {
                    rc = -1;
                    break;
                }
                if (need_h) std::memcpy(h.data(), m->hy, static_cast<size_t>(H) * 4);
                have_dev_h = true;
                launches += next ? 4 : 3;
                have_qkv = next;
                t_gemv += now() - t0;
                th = now();
                continue;
            }
            if ((rc = gemvs(att.data(), QD, {7 * l + QD_O}, {o.data()}))) break;
            th = now();
            for (int i = 0; i < H; ++i) h[i] += o[i];
            rmsnorm(h.data(), m->ffn_norm[l].data(), xn.data(), H, c.norm_eps);
            t_host += now() - th;
            if (swiglu) {
                // gate|up, SiLU and down as one server command
                const double t0 = now();
                const Matrix &wg = m->mats[7 * l + QD_GATE], &wu = m->mats[7 * l + QD_UP],
                             &wd = m->mats[7 * l + QD_DOWN];
                if (mi355x_server_swiglu(m->server, xn.data(), H, wg.dev, wu.dev, c.ffn, wd.dev, H, m->hy_dev) !=
                    MI355X_OK) {
                    rc = -1;
                    break;
                }
                std::memcpy(dn.data(), m->hy, static_cast<size_t>(H) * 4);
                launches += 2;
                t_gemv += now() - t0;
                th = now();
            } else {
                if ((rc = gemvs(xn.data(), H, {7 * l + QD_GATE, 7 * l + QD_UP}, {g.data(), u.data()}))) break;
                th = now();
                silu_mul(g.data(), u.data(), c.ffn);
                t_host += now() - th;
                if ((rc = gemvs(g.data(), c.ffn, {7 * l + QD_DOWN}, {dn.data()}))) break;
                th = now();
            }
            for (int i = 0; i < H; ++i) h[i] += dn[i];
        }
        if (rc) break;
        rmsnorm(h.data(), m->out_norm.data(), xn.data(), H, c.norm_eps);
        t_host += now() - th;
        if (pos + 1 < n_prompt || n_gen == 0) continue;  // only the last prompt token needs logits
        if ((rc = gemvs(xn.data(), H, {7 * L}, {logits.data()}))) break;
        th = now();
        tok = argmax(logits.data(), c.vocab);
        t_host += now() - th;
        out_tokens[pos + 1 - n_prompt] = tok;
    }
    if (n_gen > 0 && n_pos == n_prompt) t_gen0 = now();  // n_gen == 1: no generation-phase passes
    const double t_end = now();
    // the resident server kernel leaves with the decode loop
    if (m->server && mi355x_server_stop(m->server) != MI355X_OK && !rc) rc = -1;
    if (rc) return fail(std::string("qd_generate: GEMV failed: ") + (backend == 0 ? mi355x_last_error() : "callback"));
    if (n_gen > 0) m->last_logits = logits;
    m->last_launches = backend == 0 ? launches : 0;
    if (backend == 0) m->last_wait = use_plugin ? QD_WAIT_PLUGIN : use_server ? QD_WAIT_SERVER : wait;
    if (timings) {
        timings[0] = t_gen0 - t_start;
        timings[1] = t_end - t_gen0;
        timings[2] = t_gemv;
        timings[3] = t_host;
    }
    return 0;
}

void qd_silu_mul(float *g, const float *u, int n) { silu_mul(g, u, n); }

void qd_rmsnorm(const float *x, const float *w, float *out, int n, float eps) { rmsnorm(x, w, out, n, eps); }

void qd_set_block(qd_model *m, int on) {
    if (m) m->block = on != 0;
}

void qd_set_swiglu(qd_model *m, int on) {
    if (m) m->swiglu = on != 0;
}

int qd_set_plugin_groups(qd_model *m, int mode) {
    if (!m || (mode != GGML_MI355X_GROUPS_SERVER && mode != GGML_MI355X_GROUPS_LAUNCH))
        return fail("qd_set_plugin_groups: unknown mode");
    m->plugin_groups = mode;
    return 0;
}

}  // extern "C"
