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
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

#define PRISM_LN_EPS 1e-5f

__device__ __forceinline__ f4 mfma_16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_16x16x16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 f4_zero() { return f4{0.f, 0.f, 0.f, 0.f}; }

/* Stops the machine scheduler from moving any instruction across this point.
 * Used at k-step boundaries so prefetch loads stay where they are issued
 * instead of being sunk next to their first use. */
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

/*
 * Cross-lane reductions without the LDS crossbar (ds_bpermute, ~100 cycles
 * each): gfx950's v_permlane16_swap / v_permlane32_swap with both operands x
 * return (x of lane l & ~16, x of lane l | 16) (resp. 32), so op(r0, r1) is
 * x op x[l ^ 16] in every lane, and DPP row permutations combine lanes
 * within a row of 16. Every pairing is symmetric (both lanes of a pair
 * compute the same a op b), so all lanes of a group end with identical bits.
 */
__device__ __forceinline__ void lanes_x16(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    a = __builtin_bit_cast(float, (unsigned)r[0]);
    b = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ void lanes_x32(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    a = __builtin_bit_cast(float, (unsigned)r[0]);
    b = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ void lanes_x16(int v, int& a, int& b) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    a = (int)r[0];
    b = (int)r[1];
}
__device__ __forceinline__ void lanes_x32(int v, int& a, int& b) {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    a = (int)r[0];
    b = (int)r[1];
}
/* v + v[l ^ 16] + v[l ^ 32] + v[l ^ 48]: sum over the 4 lane groups */
__device__ __forceinline__ float sum_groups(float v) {
    float a, b;
    lanes_x16(v, a, b);
    lanes_x32(a + b, a, b);
    return a + b;
}
/* NaN-propagating maximum (IEEE 754-2019 maximum, v_maximum3_f32 on gfx950).
 * Unlike fmaxf it needs no canonicalising copy of operands the compiler
 * cannot prove canonical (MFMA results, cross-lane moves): one instruction
 * per 2 or 3 inputs. A NaN among the inputs gives NaN. */
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float vmax3(float a, float b, float c) { return vmax(vmax(a, b), c); }

__device__ __forceinline__ float max_groups(float v) {
    float a, b;
    lanes_x16(v, a, b);
    lanes_x32(vmax(a, b), a, b);
    return vmax(a, b);
}

/* Largest of the 16 values of four accumulators, as a tree of 3-input
 * maxima (NaN if any is NaN). */
__device__ __forceinline__ float max16(const f4 (&s)[4]) {
    const float a0 = vmax3(s[0][0], s[0][1], s[0][2]), a1 = vmax3(s[0][3], s[1][0], s[1][1]);
    const float a2 = vmax3(s[1][2], s[1][3], s[2][0]), a3 = vmax3(s[2][1], s[2][2], s[2][3]);
    const float a4 = vmax3(s[3][0], s[3][1], s[3][2]);
    return vmax(vmax3(a0, a1, a2), vmax3(a3, a4, s[3][3]));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
/* Sum over groups of WIDTH (4, 8 or 16) consecutive lanes, on DPP:
 * quad_perm xor 1, quad_perm xor 2, then row_half_mirror (pairs the two
 * quads of each 8-lane half) and, for 16, row_mirror first (pairs quad q
 * with quad 3 - q). */
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(WIDTH == 4 || WIDTH == 8 || WIDTH == 16, "group width");
    v += dpp<0xB1>(v);  /* quad_perm [1,0,3,2] */
    v += dpp<0x4E>(v);  /* quad_perm [2,3,0,1] */
    if constexpr (WIDTH == 16) v += dpp<0x140>(v); /* row_mirror      */
    if constexpr (WIDTH >= 8) v += dpp<0x141>(v);  /* row_half_mirror */
    return v;
}

/* Inclusive prefix sum over the 64 lanes of a wave on DPP (no LDS crossbar):
 * shifted adds within each row of 16 (row_shr 1, 2, 4, 8; lanes shifted in
 * from outside the row add 0), then row 0's total into row 1 and row 2's
 * into row 3 (row_bcast:15 on rows 1 and 3), then the total of rows 0-1 into
 * rows 2 and 3 (row_bcast:31). */
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false); /* row_shr:1  */
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false); /* row_shr:2  */
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false); /* row_shr:4  */
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false); /* row_shr:8  */
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); /* row_bcast:15 */
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); /* row_bcast:31 */
    return v;
}

/* One fragment (1 KiB, 16 B per lane) of a packed weight matrix. */
__device__ __forceinline__ h8 load_frag(const uint16_t* packed, int frag, int lane) {
    return reinterpret_cast<const h8*>(packed)[frag * 64 + lane];
}

/*
 * Packed weight matrix read through a buffer resource: the base and size sit
 * in SGPRs, the fragment offset (frag * 1 KiB, wave-uniform) in an SGPR and
 * the lane offset (lane * 16 B) in one shared VGPR, so a wave can keep dozens
 * of fragment loads in flight without spending VGPRs on addresses. Offsets at
 * or past `bytes` read as zero instead of faulting.
 */
struct FragSrc {
    __amdgpu_buffer_rsrc_t r;
    __device__ __forceinline__ FragSrc(const uint16_t* base, uint32_t bytes)
        : r(__builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000)) {}
    template <int CPOL = 0>
    __device__ __forceinline__ h8 load(int frag, int lane_off) const {
        return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, frag * 1024, CPOL));
    }
};

/* 2^x on the hardware transcendental unit (v_exp_f32). */
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
/* 1/x on the hardware reciprocal unit (v_rcp_f32, 1 ulp). */
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

/* GELU-tanh, 0.5u(1 + tanh(0.7978846(u + 0.044715u^3))), evaluated through the
 * identity 0.5(1 + tanh(z)) = 1/(1 + exp(-2z)) = 1/(1 + 2^(-2z log2 e)), with
 * -2z log2 e = u (K + K c u^2) (K = -2 * 0.7978846 * log2 e, c = 0.044715).
 * The fp16 input enters the products as a mixed-precision operand
 * (v_fma_mix), so it needs no conversion: 7 instructions per value. Large
 * negative u gives 2^+inf = inf and u * 0 = -0; large positive u gives u * 1. */
__device__ __forceinline__ float gelu_tanh_h(f16 u) {
    constexpr float K = -2.0f * 0.7978846f * 1.4426950408889634f;
    const float uf = (float)u;
    /* products as fma(x, y, 0): the form v_fma_mix takes with an fp16 operand */
    const float a = __builtin_fmaf(__builtin_fmaf(__builtin_fmaf(uf, uf, 0.0f), K * 0.044715f, K), uf, 0.0f);
    return __builtin_fmaf(uf, fast_rcp(1.0f + fast_exp2(a)), 0.0f);
}

/*
 * Every fp32 -> fp16 rounding point goes through `opaque` first: the value is
 * pinned in fp32 registers, so the compiler cannot fold the producing
 * multiply/FMA and the conversion into one v_fma_mix*_f16 (a single rounding
 * straight to fp16). That fold is applied to some unrolled copies and not
 * others, which would make a token's result depend on its row in a tile.
 * The asm emits no instruction.
 */
template <class T>
__device__ __forceinline__ T opaque(T v) {
    asm("" : "+v"(v));
    return v;
}

/* fp16 a + b with one rounding: the reference's fp16 residual add. */
__device__ __forceinline__ h4 add_f16x4(h4 a, h4 b) { return opaque(a) + opaque(b); }
__device__ __forceinline__ h8 add_f16x8(h8 a, h8 b) { return opaque(a) + opaque(b); }

/* Packed conversion of 4 fp32 values to fp16 (round to nearest even). */
__device__ __forceinline__ h4 cvt_h4(f4 v) {
    v = opaque(v);
    return h4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
}

/*
 * LayerNorm of rows into an LDS tile, LPS = DIM/16 lanes per row and 16
 * channels per lane, in two steps so a kernel can put every row load in
 * flight before it does any math: ln_load fetches the lane's 16 halfs of a
 * row, ln_store normalises them into `dst` (and
 * copies the raw values to `raw_dst` if given). Lane i of a row holds
 * channels 8i..8i+7 and DIM/2+8i..+7, so each of the two 16-byte loads of a
 * wave reads contiguous half rows (whole cache lines, not every other 16
 * bytes of them). Mean / biased variance in fp32; output rounded to fp16;
 * invalid rows are written as zeros. The affine is folded into the next
 * GEMM's weights on the host, so there are no gamma/beta here.
 */
/* LayerNorm building blocks (biased variance, eps 1e-5, fp32 statistics):
 * the sum and the sum of squares of fp16 values come straight from the fp16
 * pairs on v_dot2_f32_f16 (products exact, fp32 accumulation), the variance
 * is E[x^2] - mean^2 (clamped at 0), and each value is normalised as
 * z = fma(x, inv, -mean*inv) with the fp16 x as a mixed-precision operand
 * (one instruction per value; gamma and beta live in the consuming GEMM's
 * weights and bias). */
__device__ __forceinline__ void moments8(const h8& x, float& s, float& q) {
    const h2 one = {(f16)1.0f, (f16)1.0f};
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const h2 p = {x[j], x[j + 1]};
        s = __builtin_amdgcn_fdot2(p, one, s, false);
        q = __builtin_amdgcn_fdot2(p, p, q, false);
    }
}
template <int N>
__device__ __forceinline__ float ln_inv(float s, float q, float& mean) {
    mean = s * (1.0f / N);
    const float var = fmaxf(__builtin_fmaf(-mean, mean, q * (1.0f / N)), 0.f);
    return __builtin_amdgcn_rsqf(var + PRISM_LN_EPS); /* v_rsq_f32, 1 ulp; argument >= 1e-5 */
}
__device__ __forceinline__ float ln_apply(f16 x, float inv, float nmi) {
    return __builtin_fmaf((float)x, inv, nmi);
}

struct RowChunk {
    h8 a0, a1;
};

/* 16 bytes at byte offset `off` of a row tensor. The host keeps every
 * launch's rows under 4 GiB (the reference's 32-bit byte offsets), so the
 * offset is a 32-bit unsigned VGPR and the compiler uses the SGPR-base +
 * VGPR-offset global addressing form: no 64-bit address arithmetic.
 * NT: non-temporal access (the `nt` cache policy). The 8-wave kernels of
 * small launches use it (batch 1: 441 -> 427 us per frame); the large
 * launches do not (batch 16 was 4 % slower with it). */
template <bool NT = false>
__device__ __forceinline__ h8 ld_row16(const uint16_t* base, uint32_t off) {
    const h8* p = reinterpret_cast<const h8*>(reinterpret_cast<const unsigned char*>(base) + off);
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT = false>
__device__ __forceinline__ void st_row16(uint16_t* base, uint32_t off, h8 v) {
    h8* p = reinterpret_cast<h8*>(reinterpret_cast<unsigned char*>(base) + off);
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

/* The caller passes an in-bounds row also for a padded or absent row (its
 * values are then never used: ln_store writes zeros for it and its raw copy
 * is never stored), so the load needs no zero fill and no branch. */
template <int DIM, bool NT = false>
__device__ __forceinline__ RowChunk ln_load(const uint16_t* base, uint32_t row) {
    constexpr int LPS = DIM / 16;
    const uint32_t ca = (lane_id() % LPS) * 8;
    const uint32_t off = (row * DIM + ca) * 2u;
    return RowChunk{ld_row16<NT>(base, off), ld_row16<NT>(base, off + DIM)};
}

/* ZERO: an invalid row (padded window slot) is written as zeros, through
 * inv = nmi = 0, which gives +0 for every finite stand-in value; the
 * attention kernel's stand-in is its window's slot 0, so a non-finite one
 * only reaches a window whose every output is already NaN. ZERO = false:
 * the caller never uses an invalid row's output (its GEMM column is never
 * stored), so it is left as computed from the stand-in row. */
template <int DIM, bool ZERO = true>
__device__ __forceinline__ void ln_store(const RowChunk& rc, bool valid, f16* dst, f16* raw_dst) {
    constexpr int LPS = DIM / 16;
    const int ca = (lane_id() % LPS) * 8, cb = ca + DIM / 2;
    if (raw_dst) {
        *reinterpret_cast<h8*>(raw_dst + ca) = rc.a0;
        *reinterpret_cast<h8*>(raw_dst + cb) = rc.a1;
    }
    float s = 0.f, q = 0.f;
    moments8(rc.a0, s, q);
    moments8(rc.a1, s, q);
    s = group_sum<LPS>(s);
    q = group_sum<LPS>(q);
    float mean;
    float inv = ln_inv<DIM>(s, q, mean);
    float nmi = -mean * inv;
    if constexpr (ZERO) { /* an invalid row normalises to +0 (its stand-in row is finite or its window is NaN anyway) */
        inv = valid ? inv : 0.f;
        nmi = valid ? nmi : 0.f;
    }
    h8 o0, o1;
#pragma unroll
    for (int j = 0; j < 8; j += 4) {
        const f4 n0 = {ln_apply(rc.a0[j], inv, nmi), ln_apply(rc.a0[j + 1], inv, nmi),
                       ln_apply(rc.a0[j + 2], inv, nmi), ln_apply(rc.a0[j + 3], inv, nmi)};
        const f4 n1 = {ln_apply(rc.a1[j], inv, nmi), ln_apply(rc.a1[j + 1], inv, nmi),
                       ln_apply(rc.a1[j + 2], inv, nmi), ln_apply(rc.a1[j + 3], inv, nmi)};
        const h4 p0 = cvt_h4(n0), p1 = cvt_h4(n1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o0[j + i] = p0[i];
            o1[j + i] = p1[i];
        }
    }
    *reinterpret_cast<h8*>(dst + ca) = o0;
    *reinterpret_cast<h8*>(dst + cb) = o1;
}
