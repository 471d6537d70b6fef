/*
 * project.hpp - projection adapters either side of the block chain.
 *
 * Restates shaders/pw_project_128to256.comp.glsl:25-37 (y = r16(W x + b), then
 * ReLU) and shaders/pw_project_256to128.comp.glsl:25-32 (y = r16(W x + b)),
 * which the reference runs one thread per token, as a GEMM over 64-token
 * tiles: C^T = W * X^T with the packed weights as the A operand. A token's
 * row is contiguous (HWC), so a lane's B fragment (token 16t + l16, channels
 * 32ks + 8g .. +7) is one 16-byte global load and the tile needs no LDS.
 * Workgroup = 4 waves; wave w computes output rows [w*OUT/4, +OUT/4) of the
 * tile's 64 tokens, accumulators starting at the bias. The tile's row loads
 * and the wave's weight fragments all go out before the first MFMA.
 */
#pragma once
#include "common.hpp"

template <int IN, int OUT, bool RELU>
__device__ __forceinline__ void project_body(const ProjArgs& a) {
    constexpr int KS = IN / 32;  /* k-steps                     */
    constexpr int RT = OUT / 64; /* 16-row output tiles per wave */
    constexpr int TT = 4;        /* 16-token tiles per workgroup */
    static_assert(IN % 32 == 0 && OUT % 64 == 0, "shape");

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;
    const int64_t tok0 = (int64_t)blockIdx.x * 64;

    h8 xf[TT][KS];
    bool valid[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int64_t tk = tok0 + 16 * t + l16;
        valid[t] = tk < a.n_tokens;
        const uint16_t* row = a.in + (valid[t] ? tk : 0) * IN + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) xf[t][ks] = valid[t] ? *reinterpret_cast<const h8*>(row + 32 * ks) : h8{};
    }
    const FragSrc src(a.w, (unsigned)(OUT * IN * 2));
    h8 wf[RT][KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int r = 0; r < RT; ++r) wf[r][ks] = src.load((wave * RT + r) * KS + ks, lane * 16);
    sched_fence();

    f4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int ch = (wave * RT + r) * 16 + 4 * g;
        const f4 bb = {a.b[ch], a.b[ch + 1], a.b[ch + 2], a.b[ch + 3]};
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = bb;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[r][t] = mfma_16x16x32(wf[r][ks], xf[t][ks], acc[r][t]);

#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if (!valid[t]) continue;
        uint16_t* orow = a.out + (tok0 + 16 * t + l16) * OUT;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            f4 v = acc[r][t];
            /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
            if constexpr (RELU) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            }
            *reinterpret_cast<h4*>(orow + (wave * RT + r) * 16 + 4 * g) = cvt_h4(v);
        }
    }
}

/* up: encoder channels (128) -> model dim, ReLU; down: model dim -> 128 */
extern "C" __global__ void __launch_bounds__(256, 2) prism_project_up_d256(ProjArgs a) {
    project_body<128, 256, true>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) prism_project_down_d256(ProjArgs a) {
    project_body<256, 128, false>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) prism_project_up_d128(ProjArgs a) {
    project_body<128, 128, true>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) prism_project_down_d128(ProjArgs a) {
    project_body<128, 128, false>(a);
}
