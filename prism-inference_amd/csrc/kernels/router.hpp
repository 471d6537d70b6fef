/*
 * router.hpp - router stage: LN2 + router GEMM + top-1 argmax + counting sort.
 *
 * Restates shaders/moe_router.comp.glsl:24-52 widened to N logits
 * (moe_ffn_16exp.comp.glsl:27-34 is the N-wide form the reference intended):
 * logits = r16(W_r LN2(h) + b_r), first max wins (strict >, :42-45), the
 * expert id is written per token (:48) and the per-expert count is
 * incremented (:51). The count atomics become a workgroup-local LDS
 * histogram plus one global atomic per (workgroup, expert); each token's LDS
 * rank then places it in its expert's bucket of `perm`, which is the
 * expert-contiguous segment the grouped expert GEMM consumes.
 *
 * Workgroup = 4 waves x 32 tokens. A lane owns one token of a 16-token tile
 * and the 8-channel slices 32*ks + 8*g .. +7 of it, which is exactly the
 * B-operand fragment of logits^T = W_r * hn^T, so LN2 runs in registers.
 */
#pragma once
#include "common.hpp"

#define ROUTER_TOKENS_PER_WG 128

template <int DIM>
__device__ __forceinline__ void router_body(const RouterArgs& a) {
    constexpr int KS = DIM / 32;
    constexpr int TT = 2; /* token tiles per wave */
    __shared__ int hist[64];
    __shared__ int base[64];

    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int l16 = lane & 15;
    const int g = lane >> 4;
    if (threadIdx.x < 64) hist[threadIdx.x] = 0;
    __syncthreads();

    const int tok0 = blockIdx.x * ROUTER_TOKENS_PER_WG + wave * 16 * TT;
    int my_e[TT], my_rank[TT];

#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        const int token = tok0 + 16 * tt + l16;
        const bool valid = token < a.n_tokens;
        float x[KS][8];
        const uint16_t* row = a.in + (int64_t)(valid ? token : 0) * DIM;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const h8 v = valid ? *reinterpret_cast<const h8*>(row + 32 * ks + 8 * g) : h8{};
#pragma unroll
            for (int j = 0; j < 8; ++j) x[ks][j] = (float)v[j];
        }
        float s = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j) s += x[ks][j];
        s += __shfl_xor(s, 16, 64);
        s += __shfl_xor(s, 32, 64);
        const float mean = s * (1.0f / DIM);
        float q = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j) { const float t = x[ks][j] - mean; q += t * t; }
        q += __shfl_xor(q, 16, 64);
        q += __shfl_xor(q, 32, 64);
        const float inv = 1.0f / sqrtf(q * (1.0f / DIM) + PRISM_LN_EPS);
        h8 hn[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = 32 * ks + 8 * g + j;
                hn[ks][j] = (f16)((x[ks][j] - mean) * inv * a.ln_g[c] + a.ln_b[c]);
            }

        /* logits^T: element i of row tile rt = expert 16rt+4g+i, token l16 */
        float best_v = -3.0e38f;
        int best_e = 0x7fffffff;
        for (int rt = 0; rt < a.np / 16; ++rt) {
            f4 acc = f4_zero();
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) acc = mfma_16x16x32(load_frag(a.wr, rt * KS + ks, lane), hn[ks], acc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = 16 * rt + 4 * g + i;
                const float lv = (float)(f16)(acc[i] + a.br[e]);
                if (lv > best_v) { best_v = lv; best_e = e; }
            }
        }
        /* combine the 4 lane groups: larger logit wins, ties go to the lower id */
#pragma unroll
        for (int m = 16; m <= 32; m <<= 1) {
            const float ov = __shfl_xor(best_v, m, 64);
            const int oe = __shfl_xor(best_e, m, 64);
            if (ov > best_v || (ov == best_v && oe < best_e)) { best_v = ov; best_e = oe; }
        }
        if (best_e >= a.n_experts || best_e < 0) best_e = 0; /* non-finite logits */
        my_e[tt] = best_e;
        my_rank[tt] = 0;
        if (valid && g == 0) my_rank[tt] = atomicAdd(&hist[best_e], 1);
    }
    __syncthreads();
    if (threadIdx.x < a.n_experts) {
        const int c = hist[threadIdx.x];
        base[threadIdx.x] = c ? atomicAdd(&a.counts[threadIdx.x], c) : 0;
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        const int token = tok0 + 16 * tt + l16;
        if (token < a.n_tokens && g == 0) {
            const int e = my_e[tt];
            a.assign[token] = e;
            const int slot = base[e] + my_rank[tt];
            if (slot < a.cap) a.perm[(int64_t)e * a.cap + slot] = token;
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) prism_router_d256(RouterArgs a) {
    router_body<256>(a);
}
extern "C" __global__ void __launch_bounds__(256) prism_router_d128(RouterArgs a) {
    router_body<128>(a);
}
