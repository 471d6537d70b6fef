/*
 * route.hpp - per-token routing math shared by the router stage and the
 * attention kernel's fused routing epilogue.
 *
 * Restates shaders/moe_router.comp.glsl:24-52 widened to N logits
 * (moe_ffn_16exp.comp.glsl:27-34): hn = LN2(h), logits = r16(W_r hn + b_r)
 * (LN2's affine folded into W_r and b_r on the host),
 * expert = first index of the maximum (strict >, moe_router.comp.glsl:42-45).
 *
 * Lane layout (one 16-token tile per wave): lane (g = lane >> 4, l16 = lane & 15)
 * holds channels 32*ks + 8*g .. +7 of token l16 in cur[ks], which is exactly
 * the B-operand fragment of logits^T = W_r * hn^T, so the LayerNorm runs in
 * registers and feeds the MFMAs directly. Element i of row tile rt of the
 * result is expert 16*rt + 4*g + i of token l16. Every split of the work
 * below (whole tokens per wave, or one row tile per wave with the partial
 * maxima merged in row-tile order) gives the same expert: the maximum fp16
 * logit, lowest id among ties.
 */
#pragma once
#include "common.hpp"

/* hn = r16((h - mean) / sqrt(var + eps)) in the same lane layout as cur (the
 * B operand of the router GEMM). */
template <int DIM>
__device__ __forceinline__ void route_ln(const h8 (&cur)[DIM / 32], h8 (&hn)[DIM / 32]) {
    constexpr int KS = DIM / 32;
    float s = 0.f, q = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) moments8(cur[ks], s, q);
    s = sum_groups(s);
    q = sum_groups(q);
    float mean;
    const float inv = ln_inv<DIM>(s, q, mean);
    const float nmi = -mean * inv;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; j += 4) {
            f4 t;
#pragma unroll
            for (int i = 0; i < 4; ++i) t[i] = ln_apply(cur[ks][j + i], inv, nmi);
            const h4 q4 = cvt_h4(t);
#pragma unroll
            for (int i = 0; i < 4; ++i) hn[ks][j + i] = q4[i];
        }
    }
}

/* Best (fp16-rounded logit, expert) of one 16-expert row tile rt for the
 * token of this lane's column: 4 values in-lane, then the 4 lane groups.
 * Larger logit wins, ties go to the lower id; a tile with no finite logit
 * returns (-3e38, INT_MAX). */
__device__ __forceinline__ void route_tile_best(const f4& acc, int rt, int g, float& best_v, int& best_e) {
    const h4 lg = cvt_h4(acc); /* logits are fp16 values */
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lv = (float)lg[i];
        if (lv > best_v) { best_v = lv; best_e = 16 * rt + 4 * g + i; }
    }
}

/* (a_v, a_e) vs (b_v, b_e): larger logit, then lower id. Symmetric, so the
 * two lanes of a pair agree. */
__device__ __forceinline__ void route_pick(float av, int ae, float bv, int be, float& v, int& e) {
    const bool b_wins = bv > av || (bv == av && be < ae);
    v = b_wins ? bv : av;
    e = b_wins ? be : ae;
}

__device__ __forceinline__ void route_combine_groups(float& best_v, int& best_e) {
    float av, bv;
    int ae, be;
    lanes_x16(best_v, av, bv);
    lanes_x16(best_e, ae, be);
    route_pick(av, ae, bv, be, best_v, best_e);
    lanes_x32(best_v, av, bv);
    lanes_x32(best_e, ae, be);
    route_pick(av, ae, bv, be, best_v, best_e);
}

/* The best (fp16 logit, expert) of row tiles rt0 .. rt0+NR-1 for the token of
 * this lane's column, the same in all 4 lane groups. frag(r, ks) returns the
 * packed W_r fragment of row tile rt0 + r, k-step ks. s_br holds 16*NPT
 * biases with -inf past the real experts. Larger logit wins, ties go to the
 * lower id, so the best of consecutive ranges merged in range order with
 * route_pick equals the best of their union. */
template <int DIM, int NR, class Frag>
__device__ __forceinline__ void route_partial(const h8 (&cur)[DIM / 32], const float* s_br, int g, int rt0,
                                              Frag&& frag, float& best_v, int& best_e) {
    constexpr int KS = DIM / 32;
    h8 hn[KS];
    route_ln<DIM>(cur, hn);
    f4 acc[NR]; /* starts at the router bias */
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int b = 16 * (rt0 + r) + 4 * g;
        acc[r] = f4{s_br[b], s_br[b + 1], s_br[b + 2], s_br[b + 3]};
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = mfma_16x16x32(frag(r, ks), hn[ks], acc[r]);
    best_v = -3.0e38f;
    best_e = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < NR; ++r) route_tile_best(acc[r], rt0 + r, g, best_v, best_e);
    route_combine_groups(best_v, best_e);
}

/* The token's expert over all NPT row tiles (frag(rt, ks) as above with
 * rt0 = 0), in all 4 lane groups of its column. */
template <int DIM, int NPT, class Frag>
__device__ __forceinline__ int route_token(const h8 (&cur)[DIM / 32], const float* s_br, int g, int n_experts,
                                           Frag&& frag) {
    float best_v;
    int best_e;
    route_partial<DIM, NPT>(cur, s_br, g, 0, frag, best_v, best_e);
    if (best_e >= n_experts || best_e < 0) best_e = 0; /* non-finite logits */
    return best_e;
}
