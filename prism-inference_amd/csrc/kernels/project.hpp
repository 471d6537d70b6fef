/*
 * project.hpp - projection adapters either side of the block chain.
 *
 * Restates shaders/pw_project_128to256.comp.glsl:25-37 (y = r16(W x + b), then
 * ReLU) and shaders/pw_project_256to128.comp.glsl:25-32 (y = r16(W x + b)),
 * which the reference runs one thread per token, as a GEMM over 64-token
 * tiles: C^T = W * X^T with the packed weights as the A operand. A tile's 64
 * token rows are one contiguous block in and one out (HWC): they pass through
 * an LDS tile as whole rows, 16 bytes per lane, and the B fragments (token
 * 16t + l16, channels 32ks + 8g .. +7) are read from there. Workgroup = 4
 * waves; wave w computes output rows [w*OUT/4, +OUT/4) of a tile's 64
 * tokens, accumulators starting at the bias. Persistent: workgroup b takes
 * tiles b, b + G, b + 2G, ... (G = the grid), holds its waves' weight
 * fragments in registers across them, and requests the next tile's rows
 * before the current tile's MFMAs.
 */
#pragma once
#include "common.hpp"

template <int IN, int OUT, bool RELU>
__device__ __forceinline__ void project_body(const ProjArgs& a) {
    constexpr int KS = IN / 32;  /* k-steps                     */
    constexpr int RT = OUT / 64; /* 16-row output tiles per wave */
    constexpr int TT = 4;        /* 16-token tiles per token tile */
    constexpr int LI = IN + 8, LO = OUT + 8;  /* padded LDS rows (halfs) */
    constexpr int EI = 64 * IN / 8 / 256;     /* 16-byte input chunks per thread  */
    constexpr int EO = 64 * OUT / 8 / 256;    /* 16-byte output chunks per thread */
    static_assert(IN % 32 == 0 && OUT % 64 == 0 && EI >= 1 && EO >= 1, "shape");
    __shared__ __attribute__((aligned(16))) f16 tin[64 * LI];
    __shared__ __attribute__((aligned(16))) f16 tout[64 * LO];

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;
    const int64_t ntiles = (a.n_tokens + 63) / 64;

    /* the rows of token tile `tile` (one contiguous block): 16 bytes per
     * lane, whole cache lines per wave load; rows past the end read the
     * tile's last row (no branch around the loads, so they go out together)
     * and are kept as zero */
    auto load_rows = [&](int64_t tile, h8 (&x)[EI]) {
        const int64_t tok0 = tile * 64;
        const int rows = (int)min<int64_t>(64, a.n_tokens - tok0);
#pragma unroll
        for (int k = 0; k < EI; ++k) {
            const int q = threadIdx.x + 256 * k, r = q / (IN / 8), c8 = (q % (IN / 8)) * 8;
            const h8 v = *reinterpret_cast<const h8*>(a.in + (tok0 + min(r, rows - 1)) * IN + c8);
            x[k] = r < rows ? v : h8{};
        }
    };
    int64_t tile = blockIdx.x;
    h8 xin[EI];
    if (tile < ntiles) load_rows(tile, xin);
    /* this wave's weight fragments and its bias, held for every tile */
    const FragSrc src(a.w, (unsigned)(OUT * IN * 2));
    h8 wf[RT][KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int r = 0; r < RT; ++r) wf[r][ks] = src.load((wave * RT + r) * KS + ks, lane * 16);
    f4 bias[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int ch = (wave * RT + r) * 16 + 4 * g;
        bias[r] = f4{a.b[ch], a.b[ch + 1], a.b[ch + 2], a.b[ch + 3]};
    }

    for (; tile < ntiles; tile += gridDim.x) { /* uniform over the workgroup */
        const int64_t tok0 = tile * 64;
        const int rows = (int)min<int64_t>(64, a.n_tokens - tok0);
#pragma unroll
        for (int k = 0; k < EI; ++k) {
            const int q = threadIdx.x + 256 * k, r = q / (IN / 8), c8 = (q % (IN / 8)) * 8;
            *reinterpret_cast<h8*>(tin + r * LI + c8) = xin[k];
        }
        __syncthreads(); /* the input tile is in; the previous tile's output rows are out of tout */
        /* the next tile's rows go out now and arrive under this tile's MFMAs */
        if (tile + gridDim.x < ntiles) load_rows(tile + gridDim.x, xin);

        f4 acc[RT][TT]; /* starts at the bias */
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[r][t] = bias[r];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const h8 xf = *reinterpret_cast<const h8*>(tin + (16 * t + l16) * LI + 32 * ks + 8 * g);
#pragma unroll
                for (int r = 0; r < RT; ++r) acc[r][t] = mfma_16x16x32(wf[r][ks], xf, acc[r][t]);
            }
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                f4 v = acc[r][t];
                /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
                if constexpr (RELU) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
                }
                *reinterpret_cast<h4*>(tout + (16 * t + l16) * LO + (wave * RT + r) * 16 + 4 * g) = cvt_h4(v);
            }
        __syncthreads(); /* the output tile is complete; every wave is done reading tin */
        /* every LDS read first, then the stores (a read under a store's
           condition costs one LDS round trip per pass) */
        h8 yo[EO];
#pragma unroll
        for (int k = 0; k < EO; ++k) {
            const int q = threadIdx.x + 256 * k, r = q / (OUT / 8), c8 = (q % (OUT / 8)) * 8;
            yo[k] = *reinterpret_cast<const h8*>(tout + r * LO + c8);
        }
#pragma unroll
        for (int k = 0; k < EO; ++k) {
            const int q = threadIdx.x + 256 * k, r = q / (OUT / 8), c8 = (q % (OUT / 8)) * 8;
            if (r < rows) *reinterpret_cast<h8*>(a.out + (tok0 + r) * OUT + c8) = yo[k];
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
