/*
 * router.hpp - router stage: LN2 + router GEMM + top-1 argmax + counting sort.
 *
 * Restates shaders/moe_router.comp.glsl:24-52 widened to N logits
 * (moe_ffn_16exp.comp.glsl:27-34 is the N-wide form the reference intended):
 * the per-token math (route_token, route.hpp) gives the expert, the expert id
 * is written per token (:48) and the per-expert count is incremented (:51).
 * The count atomics become a workgroup-local LDS histogram plus one global
 * atomic per (workgroup, expert), on counters count_stride ints apart (the
 * stage call uses a private row with counters 256 B apart, so the atomics of
 * different experts do not serialise on one cache line); each token's LDS
 * rank then places it in its expert's bucket of `perm`, which is the
 * expert-contiguous segment the grouped expert GEMM consumes.
 *
 * Workgroup = 4 waves, each taking `tiles_per_wave` consecutive 16-token
 * tiles (2 at small batch, up to 8 at large batch, so a big launch issues
 * 4x fewer global atomics); the next tile's rows are loaded while the current
 * one is computed. A lane owns one token of a tile and the 8-channel slices
 * 32*ks + 8*g .. +7 of it, which is exactly the B-operand fragment of
 * logits^T = W_r * hn^T, so LN2 runs in registers. Each token's expert and
 * LDS rank are parked in LDS and scattered after the workgroup's bucket bases
 * are known.
 * NPT = padded experts / 16 is a template parameter; the workgroup copies
 * the NPT*KS router fragments into LDS once and every wave reads them from
 * there, which keeps the register count low enough for several workgroups
 * per CU.
 */
#pragma once
#include "route.hpp"

template <int DIM, int KS>
__device__ __forceinline__ void router_load_tile(const RouterArgs& a, int token, int g, h8 (&xr)[KS]) {
    /* past the last token: token 0's row is read (no branch around the
       loads, so they go out together) and zeros are kept */
    const bool ok = token < a.n_tokens;
    const uint16_t* row = a.in + (int64_t)(ok ? token : 0) * DIM;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const h8 v = *reinterpret_cast<const h8*>(row + 32 * ks + 8 * g);
        xr[ks] = ok ? v : h8{};
    }
}

template <int DIM, int NPT>
__device__ __forceinline__ void router_body(const RouterArgs& a) {
    constexpr int KS = DIM / 32;
    constexpr int NF = NPT * KS;     /* router fragments */
    constexpr int MAXTOK = 4 * ROUTER_MAX_TILES_PER_WAVE * 16;
    __shared__ int hist[64];
    __shared__ int base[64];
    __shared__ float s_br[16 * NPT];
    __shared__ __attribute__((aligned(16))) h8 s_wr[NF * 64]; /* fragment-ordered W_r */
    __shared__ int s_e[MAXTOK], s_rank[MAXTOK];

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;
    const int tpw = a.tiles_per_wave;
    const int wg_tokens = 64 * tpw;
    const int tok_wg0 = blockIdx.x * wg_tokens;

    /* first tile's rows, then the cooperative W_r copy and parameters */
    h8 xr[KS];
    router_load_tile<DIM, KS>(a, tok_wg0 + wave * tpw * 16 + l16, g, xr);
    {
        /* every load of the copy is issued before its first LDS store (one
           memory round trip, not one per pass) */
        static_assert(NF * 64 % 256 == 0 && 16 * NPT <= 256, "whole passes");
        constexpr int NP = NF * 64 / 256;
        const FragSrc src_r(a.wr, 16u * NPT * DIM * 2u);
        const int tid = (int)threadIdx.x;
        h8 v[NP];
#pragma unroll
        for (int k = 0; k < NP; ++k) v[k] = src_r.load((tid + 256 * k) / 64, ((tid + 256 * k) % 64) * 16);
        const float br = a.br[min(tid, 16 * NPT - 1)];
#pragma unroll
        for (int k = 0; k < NP; ++k) s_wr[tid + 256 * k] = v[k];
        if (tid < 16 * NPT) s_br[tid] = br;
    }
    if (threadIdx.x < 64) hist[threadIdx.x] = 0;
    __syncthreads();

#pragma unroll 1
    for (int it = 0; it < tpw; ++it) {
        const int local = (wave * tpw + it) * 16 + l16;
        const int token = tok_wg0 + local;
        h8 cur[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) cur[ks] = xr[ks];
        if (it + 1 < tpw) router_load_tile<DIM, KS>(a, token + 16, g, xr); /* next tile in flight */

        const int best_e = route_token<DIM, NPT>(cur, s_br, g, a.n_experts,
                                                 [&](int rt, int ks) { return s_wr[(rt * KS + ks) * 64 + lane]; });
        if (g == 0) {
            s_e[local] = best_e;
            s_rank[local] = token < a.n_tokens ? atomicAdd(&hist[best_e], 1) : 0;
        }
    }
    __syncthreads();
    if (threadIdx.x < a.n_experts) {
        const int c = hist[threadIdx.x];
        base[threadIdx.x] = c ? atomicAdd(&a.counts[threadIdx.x * a.count_stride], c) : 0;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < wg_tokens; j += 256) {
        const int token = tok_wg0 + j;
        if (token < a.n_tokens) {
            const int e = s_e[j];
            a.assign[token] = e;
            const int slot = base[e] + s_rank[j];
            if (slot < a.cap) a.perm[(int64_t)e * a.cap + slot] = token;
        }
    }
}

#define PRISM_ROUTER_KERNEL(D, NPT)                                                                 \
    extern "C" __global__ void __launch_bounds__(256, 3) prism_router_d##D##_n##NPT(RouterArgs a) {\
        router_body<D, NPT>(a);                                                                     \
    }
PRISM_ROUTER_KERNEL(256, 1)
PRISM_ROUTER_KERNEL(256, 2)
PRISM_ROUTER_KERNEL(256, 3)
PRISM_ROUTER_KERNEL(256, 4)
PRISM_ROUTER_KERNEL(128, 1)
PRISM_ROUTER_KERNEL(128, 2)
PRISM_ROUTER_KERNEL(128, 3)
PRISM_ROUTER_KERNEL(128, 4)
#undef PRISM_ROUTER_KERNEL
