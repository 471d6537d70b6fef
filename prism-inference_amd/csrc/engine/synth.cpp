/*
 * synth.cpp - deterministic synthetic weights and activations (host only).
 *
 * The reference's hot-path bench never uploads weights or inputs
 * (prism_moe_bench.cpp:143-161), so the workloads here are defined from
 * scratch and reproducibly:
 *
 *   key(seed, stream)  = splitmix64(seed ^ splitmix64(stream + GOLDEN))
 *   bits(i)            = splitmix64(key + i * GOLDEN)
 *   u1 = (bits[63:40] + 0.5) / 2^24,  u2 = (bits[23:0] + 0.5) / 2^24
 *   z(i)               = sqrt(-2 ln u1) * cos(2 pi u2)     (Box-Muller, double)
 *   value              = fp16(std * z(i))                  (round-to-nearest-even)
 *
 * Streams: activations use stream 0; block b's tensor kind k of expert e uses
 * ((b + 1) << 24) | (k << 16) | e. Every W and b is ~N(0, 0.02), LN gamma = 1
 * and beta = 0. The router bias depends on the routing mode: random like any
 * bias, zero ("uniform"), or fitted so that the top-1 load follows a target
 * distribution (Zipf s = 1.1 over the experts, or 50% on expert 0 and the rest
 * uniform). The fit treats each expert's logit noise over tokens as
 * N(0, |W_r[e]|^2) - the LN2 output has unit variance per channel - samples
 * 8192 tokens of it from the same generator, and iterates
 * b_e += 0.3 * sigma * (ln p_e - ln q_e) on the sampled argmax frequencies q.
 * The load a real run produces is measured by the bench, not assumed.
 */
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "engine_internal.h"

namespace {

constexpr uint64_t GOLDEN = 0x9E3779B97F4A7C15ULL;

inline uint64_t splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) { return splitmix64(seed ^ splitmix64(stream + GOLDEN)); }

inline double normal_at(uint64_t key, uint64_t i) {
    const uint64_t bits = splitmix64(key + i * GOLDEN);
    const double u1 = ((double)(bits >> 40) + 0.5) * (1.0 / 16777216.0);
    const double u2 = ((double)(bits & 0xFFFFFFULL) + 0.5) * (1.0 / 16777216.0);
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

template <class F>
void parallel_for(int64_t n, F&& fn) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < (1 << 16)) nt = 1;
    if (nt == 1) { fn(int64_t(0), n); return; }
    std::vector<std::thread> th;
    const int64_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const int64_t a = t * chunk, b = std::min(n, a + chunk);
        if (a >= b) break;
        th.emplace_back([&fn, a, b] { fn(a, b); });
    }
    for (auto& x : th) x.join();
}

void fill_normal(uint16_t* dst, int64_t n, uint64_t seed, uint64_t stream, float stdv) {
    const uint64_t key = stream_key(seed, stream);
    parallel_for(n, [&](int64_t a, int64_t b) {
        for (int64_t i = a; i < b; ++i) dst[i] = prism::float_to_half((float)(stdv * normal_at(key, i)));
    });
}

void fill_const(uint16_t* dst, int64_t n, float v) {
    const uint16_t h = prism::float_to_half(v);
    for (int64_t i = 0; i < n; ++i) dst[i] = h;
}

uint64_t tensor_stream(int block, int kind, int expert) {
    return ((uint64_t)(block + 1) << 24) | ((uint64_t)kind << 16) | (uint64_t)expert;
}

enum Kind { K_QKV_W = 1, K_QKV_B, K_OUT_W, K_OUT_B, K_RTR_W, K_RTR_B, K_W1, K_B1, K_W2, K_B2, K_CAL };

/* Fit router biases so the top-1 share of expert e approaches p[e]. */
void fit_router_bias(const uint16_t* wr, int N, int D, const std::vector<double>& p, uint64_t seed, int block,
                     uint16_t* bias_out) {
    std::vector<double> sigma(N);
    double smean = 0;
    for (int e = 0; e < N; ++e) {
        double s = 0;
        for (int c = 0; c < D; ++c) { const double w = prism::half_to_float(wr[(size_t)e * D + c]); s += w * w; }
        sigma[e] = std::sqrt(s);
        smean += sigma[e] / N;
    }
    const int M = 8192;
    std::vector<float> z((size_t)M * N);
    const uint64_t key = stream_key(seed, tensor_stream(block, K_CAL, 0));
    for (int64_t i = 0; i < (int64_t)M * N; ++i) z[i] = (float)(sigma[i % N] * normal_at(key, i));
    std::vector<double> b(N), q(N);
    for (int e = 0; e < N; ++e) b[e] = smean * std::log(p[e]);
    for (int iter = 0; iter < 150; ++iter) {
        std::fill(q.begin(), q.end(), 0.5 / M); /* smoothing */
        for (int m = 0; m < M; ++m) {
            const float* zm = &z[(size_t)m * N];
            int best = 0;
            double bv = zm[0] + b[0];
            for (int e = 1; e < N; ++e) {
                const double v = zm[e] + b[e];
                if (v > bv) { bv = v; best = e; }
            }
            q[best] += 1.0 / M;
        }
        double mean_b = 0;
        for (int e = 0; e < N; ++e) {
            b[e] += 0.3 * smean * (std::log(p[e]) - std::log(q[e]));
            mean_b += b[e] / N;
        }
        for (int e = 0; e < N; ++e) b[e] -= mean_b;
    }
    for (int e = 0; e < N; ++e) bias_out[e] = prism::float_to_half((float)b[e]);
}

}  // namespace

using namespace prism;

extern "C" int prism_synth_normal_f16(uint16_t* dst, int64_t n, uint64_t seed, uint64_t stream, float stdv) {
    if (!dst || n < 0) {
        set_global_error("prism_synth_normal_f16: bad arguments");
        return PRISM_ERR_INVALID;
    }
    fill_normal(dst, n, seed, stream, stdv);
    return PRISM_OK;
}

extern "C" int prism_synth_weights(const prism_model_desc* d, uint64_t seed, int32_t routing, uint16_t* blob,
                                   int64_t blob_elems, prism_block_offsets* offs) {
    std::string why;
    if (!shape_supported(d, &why)) {
        set_global_error(why);
        return PRISM_ERR_UNSUPPORTED;
    }
    if (!blob || !offs || routing < PRISM_ROUTE_RANDOM || routing > PRISM_ROUTE_ADVERSARIAL) {
        set_global_error("prism_synth_weights: bad arguments");
        return PRISM_ERR_INVALID;
    }
    const int64_t total = layout_blocks(d, offs);
    if (blob_elems < total) {
        set_global_error("prism_synth_weights: blob too small for the layout");
        return PRISM_ERR_INVALID;
    }
    memset(blob, 0, sizeof(uint16_t) * (size_t)total);
    const int D = d->dim, N = d->n_experts;
    const float sd = 0.02f;
    std::vector<double> target;
    if (N > 1 && routing == PRISM_ROUTE_ZIPF) {
        double z = 0;
        for (int e = 0; e < N; ++e) z += std::pow(e + 1.0, -1.1);
        for (int e = 0; e < N; ++e) target.push_back(std::pow(e + 1.0, -1.1) / z);
    } else if (N > 1 && routing == PRISM_ROUTE_ADVERSARIAL) {
        target.push_back(0.5);
        for (int e = 1; e < N; ++e) target.push_back(0.5 / (N - 1));
    }
    for (int b = 0; b < d->n_blocks; ++b) {
        const prism_block_offsets& o = offs[b];
        fill_const(blob + o.ln1_g, D, 1.0f);
        fill_const(blob + o.ln1_b, D, 0.0f);
        fill_normal(blob + o.qkv_w, 3LL * D * D, seed, tensor_stream(b, K_QKV_W, 0), sd);
        fill_normal(blob + o.qkv_b, 3LL * D, seed, tensor_stream(b, K_QKV_B, 0), sd);
        fill_normal(blob + o.out_w, (int64_t)D * D, seed, tensor_stream(b, K_OUT_W, 0), sd);
        fill_normal(blob + o.out_b, D, seed, tensor_stream(b, K_OUT_B, 0), sd);
        fill_const(blob + o.ln2_g, D, 1.0f);
        fill_const(blob + o.ln2_b, D, 0.0f);
        if (N > 1) {
            fill_normal(blob + o.router_w, (int64_t)N * D, seed, tensor_stream(b, K_RTR_W, 0), sd);
            if (routing == PRISM_ROUTE_RANDOM)
                fill_normal(blob + o.router_b, N, seed, tensor_stream(b, K_RTR_B, 0), sd);
            else if (routing == PRISM_ROUTE_UNIFORM)
                fill_const(blob + o.router_b, N, 0.0f);
            else
                fit_router_bias(blob + o.router_w, N, D, target, seed, b, blob + o.router_b);
        }
        for (int e = 0; e < N; ++e) {
            const int64_t eo = (int64_t)e * o.exp_stride;
            fill_normal(blob + o.exp_w1 + eo, (int64_t)D * D, seed, tensor_stream(b, K_W1, e), sd);
            fill_normal(blob + o.exp_b1 + eo, D, seed, tensor_stream(b, K_B1, e), sd);
            fill_normal(blob + o.exp_w2 + eo, (int64_t)D * D, seed, tensor_stream(b, K_W2, e), sd);
            fill_normal(blob + o.exp_b2 + eo, D, seed, tensor_stream(b, K_B2, e), sd);
        }
    }
    return PRISM_OK;
}
