/*
 * attn.hpp - attention stage: one workgroup per 8x8 window, 4 waves.
 *
 * Restates shaders/split2_qkv_attn_d256.comp.glsl:24-79 (window mapping
 * :25-33, zero-vector padded slots :31-37, QKV :39-51, softmax core :53-69,
 * out-proj + fp16 residual :71-78) with the pre-LayerNorm added, as:
 *
 *  1. LN1 of the window's 64 slots -> xs (LDS, fp16). Padded slots are zero.
 *  2. Wave w owns heads w and w+4. Per head, one MFMA GEMM pass over the
 *     model dim produces Q^T and K^T (rows = channel, cols = token) and V
 *     (rows = token, cols = channel), fp32 accumulate, bias, fp16 round.
 *  3. S^T = K Q^T is one MFMA per 16x16 tile straight from those registers:
 *     an accumulator lane holds 4 consecutive channels of one token, which is
 *     exactly a k-slice of an operand under the permuted k numbering
 *     k(g, j) = 16*(j/4) + 4g + j%4. Softmax runs down the key axis: 16
 *     values in-lane plus two cross-lane xor shuffles. P = exp(...) stays in
 *     registers and O^T = V^T P^T is again register-to-register MFMA.
 *     O^T is normalised, rounded to fp16 and written to os (LDS).
 *  4. Out-proj C^T = Wo * O^T, bias, fp16 round, + x (fp16 round), store.
 *
 * Weights (packed fragments) are read straight from global memory; all
 * workgroups read the same 0.5 MiB per block, which stays L2-resident.
 */
#pragma once
#include "common.hpp"

template <int DIM, int HD>
__device__ __forceinline__ void attn_window_body(const AttnArgs& a) {
    static_assert(DIM / HD == 8, "8 heads");
    constexpr int KS = DIM / 32;        /* k-steps over the model dim      */
    constexpr int CT = HD / 16;         /* 16-channel tiles per head       */
    constexpr int LDS = DIM + 8;        /* padded LDS row, halfs           */
    constexpr int ORT = DIM / 64;       /* out-proj row tiles per wave     */
    constexpr float LOG2E = 1.4426950408889634f;
    const float scale = (HD == 32) ? 0.1767766953f : 1.0f / sqrtf((float)HD);
    const float sl2 = scale * LOG2E;

    __shared__ __attribute__((aligned(16))) f16 xs[64 * LDS];
    __shared__ __attribute__((aligned(16))) f16 os[64 * LDS];

    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int l16 = lane & 15;
    const int g = lane >> 4;

    const int wg = blockIdx.x;
    const int frame = wg / a.windows_per_frame;
    const int wi = wg - frame * a.windows_per_frame;
    const int wy = wi / a.wx;
    const int wxx = wi - wy * a.wx;
    const uint16_t* in = a.in + (int64_t)frame * a.frame_elems;
    uint16_t* out = a.out + (int64_t)frame * a.frame_elems;

    /* ---- 1. LN1 ------------------------------------------------------ */
    {
        constexpr int LPS = DIM / 16;
        constexpr int SPI = 64 / LPS; /* slots per wave iteration */
#pragma unroll
        for (int it = 0; it < 16 / SPI; ++it) {
            const int s = wave * 16 + it * SPI + lane / LPS;
            const int gy = wy * 8 + (s >> 3), gx = wxx * 8 + (s & 7);
            const bool valid = gy < a.H && gx < a.W;
            const int t = valid ? gy * a.W + gx : 0;
            ln_row_to_lds<DIM>(in + (int64_t)t * DIM, valid, a.ln_g, a.ln_b, xs + s * LDS);
        }
    }
    __syncthreads();

    /* ---- 2./3. per head ----------------------------------------------- */
#pragma unroll 1
    for (int hh = 0; hh < 2; ++hh) {
        const int h = wave + 4 * hh;
        f4 accQ[CT][4], accK[CT][4], accV[4][CT];
#pragma unroll
        for (int c = 0; c < CT; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) { accQ[c][t] = f4_zero(); accK[c][t] = f4_zero(); accV[t][c] = f4_zero(); }

        const int rtq = (h * HD) / 16;
        const int rtk = (DIM + h * HD) / 16;
        const int rtv = (2 * DIM + h * HD) / 16;
#pragma unroll 2
        for (int ks = 0; ks < KS; ++ks) {
            h8 xf[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                xf[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * ks + 8 * g);
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const h8 wq = load_frag(a.wqkv, (rtq + c) * KS + ks, lane);
                const h8 wk = load_frag(a.wqkv, (rtk + c) * KS + ks, lane);
                const h8 wv = load_frag(a.wqkv, (rtv + c) * KS + ks, lane);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    accQ[c][t] = mfma_16x16x32(wq, xf[t], accQ[c][t]);
                    accK[c][t] = mfma_16x16x32(wk, xf[t], accK[c][t]);
                    accV[t][c] = mfma_16x16x32(xf[t], wv, accV[t][c]);
                }
            }
        }

        /* bias + fp16 round. Q^T/K^T element i: channel 16c+4g+i, token 16t+l16.
         * V element i: token 16t+4g+i, channel 16c+l16. */
        h4 q4[CT][4], k4[CT][4], v4[4][CT];
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            const int chq = h * HD + 16 * c + 4 * g;
            const int chv = 2 * DIM + h * HD + 16 * c + l16;
            const float bv = a.bqkv[chv];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    q4[c][t][i] = (f16)(accQ[c][t][i] + a.bqkv[chq + i]);
                    k4[c][t][i] = (f16)(accK[c][t][i] + a.bqkv[DIM + chq + i]);
                    v4[t][c][i] = (f16)(accV[t][c][i] + bv);
                }
            }
        }

        /* S^T[key tile kt][query tile qt]: element i = key 16kt+4g+i, query 16qt+l16 */
        f4 s[4][4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) {
                if constexpr (CT == 2) {
                    const h8 ka = {k4[0][kt][0], k4[0][kt][1], k4[0][kt][2], k4[0][kt][3],
                                   k4[1][kt][0], k4[1][kt][1], k4[1][kt][2], k4[1][kt][3]};
                    const h8 qb = {q4[0][qt][0], q4[0][qt][1], q4[0][qt][2], q4[0][qt][3],
                                   q4[1][qt][0], q4[1][qt][1], q4[1][qt][2], q4[1][qt][3]};
                    s[kt][qt] = mfma_16x16x32(ka, qb, f4_zero());
                } else {
                    s[kt][qt] = mfma_16x16x16(k4[0][kt], q4[0][qt], f4_zero());
                }
            }

        /* softmax down the key axis for each query column */
        h4 p[4][4];
        float inv[4];
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
            float m = -3.0e38f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) m = fmaxf(m, s[kt][qt][i]);
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            float sum = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = exp2f((s[kt][qt][i] - m) * sl2);
                    sum += e;
                    p[kt][qt][i] = (f16)e;
                }
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            inv[qt] = 1.0f / fmaxf(sum, 1e-6f);
        }

        /* O^T[channel tile dt][query tile qt] = V^T P^T over 64 keys (2 k-steps) */
#pragma unroll
        for (int dt = 0; dt < CT; ++dt)
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) {
                f4 o = f4_zero();
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const h8 va = {v4[2 * st][dt][0], v4[2 * st][dt][1], v4[2 * st][dt][2], v4[2 * st][dt][3],
                                   v4[2 * st + 1][dt][0], v4[2 * st + 1][dt][1], v4[2 * st + 1][dt][2],
                                   v4[2 * st + 1][dt][3]};
                    const h8 pb = {p[2 * st][qt][0], p[2 * st][qt][1], p[2 * st][qt][2], p[2 * st][qt][3],
                                   p[2 * st + 1][qt][0], p[2 * st + 1][qt][1], p[2 * st + 1][qt][2],
                                   p[2 * st + 1][qt][3]};
                    o = mfma_16x16x32(va, pb, o);
                }
                h4 r;
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = (f16)(o[i] * inv[qt]);
                *reinterpret_cast<h4*>(os + (16 * qt + l16) * LDS + h * HD + 16 * dt + 4 * g) = r;
            }
    }
    __syncthreads();

    /* ---- 4. out-proj + residual --------------------------------------- */
    f4 acc[ORT][4];
#pragma unroll
    for (int r = 0; r < ORT; ++r)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[r][t] = f4_zero();
#pragma unroll 2
    for (int ks = 0; ks < KS; ++ks) {
        h8 of[4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
            of[t] = *reinterpret_cast<const h8*>(os + (16 * t + l16) * LDS + 32 * ks + 8 * g);
#pragma unroll
        for (int r = 0; r < ORT; ++r) {
            const h8 w = load_frag(a.wo, (wave * ORT + r) * KS + ks, lane);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[r][t] = mfma_16x16x32(w, of[t], acc[r][t]);
        }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int s = 16 * t + l16;
        const int gy = wy * 8 + (s >> 3), gx = wxx * 8 + (s & 7);
        if (gy < a.H && gx < a.W) {
            const int64_t base = (int64_t)(gy * a.W + gx) * DIM;
#pragma unroll
            for (int r = 0; r < ORT; ++r) {
                const int ch = (wave * ORT + r) * 16 + 4 * g;
                const h4 xin = *reinterpret_cast<const h4*>(in + base + ch);
                h4 y;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f16 po = (f16)(acc[r][t][i] + a.bo[ch + i]);
                    y[i] = (f16)((float)po + (float)xin[i]);
                }
                *reinterpret_cast<h4*>(out + base + ch) = y;
            }
        }
    }
}

extern "C" __global__ void __launch_bounds__(256, 2) prism_attn_d256(AttnArgs a) {
    attn_window_body<256, 32>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) prism_attn_d128(AttnArgs a) {
    attn_window_body<128, 16>(a);
}
