/*
 * common.hpp - device helpers shared by the gfx950 kernels.
 *
 * MFMA operand layout used throughout (v_mfma_f32_16x16x32_f16, wave64):
 *   A (16 x 32): lane l holds A[l & 15][8*(l >> 4) + j], j = 0..7
 *   B (32 x 16): lane l holds B[8*(l >> 4) + j][l & 15]
 *   C (16 x 16): lane l holds C[4*(l >> 4) + i][l & 15], i = 0..3
 * The reduction index k only has to be numbered the same way in A and B, so
 * a kernel may hand the MFMA any bijection (lane group, j) -> k; the
 * attention core uses that to feed accumulators straight back in as operands.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kernel_args.h"

typedef _Float16 f16;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

#define PRISM_LN_EPS 1e-5f

__device__ __forceinline__ f4 mfma_16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_16x16x16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 f4_zero() { return f4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

/* Sum over groups of `width` consecutive lanes (width a power of two <= 64). */
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = 1; m < WIDTH; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

/* One fragment (1 KiB, 16 B per lane) of a packed weight matrix. */
__device__ __forceinline__ h8 load_frag(const uint16_t* packed, int frag, int lane) {
    return reinterpret_cast<const h8*>(packed)[frag * 64 + lane];
}

/* GELU-tanh, 0.5u(1 + tanh(0.7978846(u + 0.044715u^3))), evaluated through the
 * identity 0.5(1 + tanh(z)) = 1/(1 + exp(-2z)). */
__device__ __forceinline__ float gelu_tanh(float u) {
    const float z = 0.7978846f * (u + 0.044715f * u * u * u);
    return u / (1.0f + __expf(-2.0f * z));
}

/*
 * LayerNorm of rows into an LDS tile, LPS = DIM/16 lanes per row and 16
 * channels per lane. Rows whose `valid` flag is false are written as zeros.
 * Two-pass mean / biased variance in fp32; output rounded to fp16.
 */
template <int DIM>
__device__ __forceinline__ void ln_row_to_lds(const uint16_t* row, bool valid, const float* g,
                                              const float* b, f16* dst) {
    constexpr int LPS = DIM / 16;
    const int c0 = (lane_id() % LPS) * 16;
    float v[16];
    if (valid) {
        const h8* p = reinterpret_cast<const h8*>(row + c0);
        const h8 a0 = p[0], a1 = p[1];
#pragma unroll
        for (int j = 0; j < 8; ++j) { v[j] = (float)a0[j]; v[8 + j] = (float)a1[j]; }
    } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += v[j];
    s = group_sum<LPS>(s);
    const float mean = s * (1.0f / DIM);
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) { const float t = v[j] - mean; q += t * t; }
    q = group_sum<LPS>(q);
    const float inv = 1.0f / sqrtf(q * (1.0f / DIM) + PRISM_LN_EPS);
    h8 o0, o1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        o0[j] = valid ? (f16)((v[j] - mean) * inv * g[c0 + j] + b[c0 + j]) : (f16)0.f;
        o1[j] = valid ? (f16)((v[8 + j] - mean) * inv * g[c0 + 8 + j] + b[c0 + 8 + j]) : (f16)0.f;
    }
    h8* d = reinterpret_cast<h8*>(dst + c0);
    d[0] = o0;
    d[1] = o1;
}
