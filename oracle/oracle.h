/*
 * oracle.h - CPU restatement of the Prism bottleneck block chain.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity oracle: tests/, the smoke
 * entry point and the bench's cpu_baseline leg may load it; the product
 * (libprism.so + prism_kernels.hsaco) never links, loads or calls it.
 *
 * Reference files it follows (paths relative to the reference repository):
 *   shaders/split2_qkv_attn_d256.comp.glsl:24-79  attention stage
 *   shaders/attention_windowed.comp.glsl:99-138   runtime heads/head_dim
 *   shaders/moe_router.comp.glsl:24-52            router stage (N-wide)
 *   shaders/moe_ffn_16exp.comp.glsl:27-34         intended N-wide argmax
 *   shaders/moe_expert_skip.comp.glsl:25-54       expert stage
 *   shaders/pw_project_128to256.comp.glsl:25-37   projection 128 -> 256 + ReLU
 *   shaders/pw_project_256to128.comp.glsl:25-32   projection 256 -> 128
 *   shaders/conv3x3_coopvec_9ch.comp.glsl:27-72   encoder input conv
 *   shaders/strided_conv_coopvec_32ch.comp.glsl:30-77, strided_conv_split_{64,128}ch
 *                                                 stride-2 encoder convs
 *   shaders/dec{3,2,1}_fused.comp.glsl            fused decoder stages
 *   shaders/pw_conv_coopvec_32to12.comp.glsl:28-55 output conv
 *   shaders/pixelshuffle_sigmoid.comp.glsl:28-56  PixelShuffle + sigmoid
 *   vulkan_engine/prism_moe_bench.cpp:164-172     weight offset layout
 *   vulkan_engine/prism_moe_bench.cpp:262-291     per-block host order
 *
 * All values are carried as float. In "faithful" mode every point where the
 * shaders store an fp16 value is rounded to fp16 (round-to-nearest-even),
 * including the fp16 residual adds; in "fp32" mode nothing is rounded after
 * the fp16 inputs and weights.
 */
#ifndef PRISM_ORACLE_H
#define PRISM_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int dim;        /* 128 or 256 */
    int n_heads;    /* 8 */
    int head_dim;   /* dim / n_heads */
    int n_experts;  /* 1 = dense FFN block (no router) */
    int H, W;       /* token grid */
    int window;     /* 8 */
    int batch;      /* frames, consecutive at H*W*dim stride */
    int faithful;   /* 1 = round to fp16 at the shader's points, 0 = pure fp32 */
} oracle_cfg;

/* Element offsets of one block's tensors inside the flat weight blob. */
typedef struct {
    int64_t ln1_g, ln1_b, qkv_w, qkv_b, out_w, out_b;
    int64_t ln2_g, ln2_b, router_w, router_b;
    int64_t exp_w1, exp_b1, exp_w2, exp_b2, exp_stride;
} oracle_block_offsets;

/* fp16 <-> fp32 helpers (IEEE binary16, round-to-nearest-even). */
void oracle_f16_to_f32(const uint16_t* src, float* dst, size_t n);
void oracle_f32_to_f16(const float* src, uint16_t* dst, size_t n);

/* LayerNorm over the last axis of x[n][d]: biased variance, eps = 1e-5. */
void oracle_layernorm(const float* x, const float* g, const float* b,
                      int n, int d, int round16, float* y);

/* GELU-tanh of moe_expert_skip.comp.glsl:43-46, elementwise, fp32. */
void oracle_gelu(const float* x, float* y, size_t n);

/* One attention stage: y = x + OutProj(WindowMHSA(QKV(LN1(x)))). */
int oracle_attn_stage(const oracle_cfg* c, const float* w,
                      const oracle_block_offsets* o, const float* x, float* y);

/* The window-attention core alone, on precomputed q/k/v [n_slots][dim]. */
void oracle_window_attention(const oracle_cfg* c, const float* q, const float* k,
                             const float* v, float* out);

/* Router: logits[t][e] = W_r LN2(h) + b_r, assign[t] = first argmax.
 * logits may be NULL. */
int oracle_router_stage(const oracle_cfg* c, const float* w,
                        const oracle_block_offsets* o, const float* h,
                        int32_t* assign, float* logits);

/* Expert stage: y = h + FFN_{assign[t]}(LN2(h)). assign NULL = expert 0. */
int oracle_expert_stage(const oracle_cfg* c, const float* w,
                        const oracle_block_offsets* o, const float* h,
                        const int32_t* assign, float* y);

/* n_blocks blocks: attn -> router -> experts. assign_out is
 * [n_blocks][batch*H*W] or NULL; h_out (attention outputs) likewise. */
int oracle_forward(const oracle_cfg* c, const float* w,
                   const oracle_block_offsets* offs, int n_blocks,
                   const float* x, float* y, int32_t* assign_out, float* h_out);

/* Projection adapter (pw_project_128to256 with relu = 1, pw_project_256to128
 * with relu = 0): y[t] = r16(W x[t] + b), then max(y, 0) if relu.
 * W is [out_dim][in_dim]; in_dim % 8 == 0. */
int oracle_project(const float* W, const float* b, int in_dim, int out_dim, int relu, const float* x,
                   int n, int faithful, float* y);

/* Encoder / decoder stages on CHW maps (oracle.c has the formulas). */
int oracle_conv3x3(const float* x, int cin, int h, int w, int stride, const float* W, const float* b, int cout,
                   int relu, int faithful, float* y);
/* The reference's split strided convs with their per-group fp16 rounding
 * (mode 0: two groups combined in fp32, the 64-channel shader; mode 1: a
 * running fp16 sum, the 128-channel shader); stride 2, ReLU. */
int oracle_conv3x3_split(const float* x, int cin, int h, int w, const float* W, const float* b, int cout, int groups,
                         int mode, float* y);
int oracle_dec_stage(const float* up, int cup, int uh, int uw, const float* skip, int cskip, int oh, int ow,
                     const float* W, const float* b, int cout, int faithful, float* y);
int oracle_pw_conv(const float* x, int cin, int h, int w, const float* W, const float* b, int cout, int relu,
                   int faithful, float* y);
int oracle_pixelshuffle_sigmoid(const float* x, int h, int w, int s, int faithful, float* y);

int oracle_max_threads(void);
void oracle_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
