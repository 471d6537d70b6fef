/*
 * kernel_args.h - argument blocks passed by value to the gfx950 kernels.
 *
 * Shared by the host engine (which fills them and launches through
 * hipModuleLaunchKernel) and the device code. Plain C, no HIP types.
 *
 * Packed weight format ("A-fragment order"): a row-major fp16 matrix
 * W[rows][K] is stored as fragments of the 16x16x32 fp16 MFMA. Fragment
 * (rt, ks) covers rows 16*rt .. 16*rt+15 and columns 32*ks .. 32*ks+31 and is
 * 64 lanes x 8 halfs = 1 KiB contiguous; lane l holds
 *   W[16*rt + (l & 15)][32*ks + 8*(l >> 4) + j],  j = 0..7
 * at halfs ((rt*KS + ks)*64 + l)*8 + j, KS = K/32. One wave reads one
 * fragment with one fully coalesced 16-byte load per lane.
 *
 * LayerNorms carry no parameters here: the matrices that consume an LN's
 * output (W_qkv for LN1; W_r and every expert's W1 for LN2) are stored with
 * the LN affine folded in, W' = r16(W diag(gamma)) and b' = b + W beta, so a
 * kernel only normalises, z = (x - mean) / sqrt(var + eps).
 */
#ifndef PRISM_KERNEL_ARGS_H
#define PRISM_KERNEL_ARGS_H
#include <stdint.h>

typedef struct AttnArgs {
    const uint16_t* in;   /* features + input_offset (fp16 HWC)         */
    uint16_t* out;        /* features + output_offset                   */
    const uint16_t* wqkv; /* packed [3*dim/16][dim/32] fragments         */
    const float* bqkv;    /* [3*dim]                                     */
    const float* bqkv_pad; /* [3*dim] the QKV of a padded window slot (whose
                              LN1 output is the zero vector): the blob's bias,
                              without LN1's beta term that bqkv carries;
                              NULL when that term is zero (beta = 0)     */
    const uint16_t* wo;   /* packed [dim/16][dim/32]                     */
    const float* bo;      /* [dim]                                       */
    int64_t frame_elems;  /* H*W*dim                                     */
    int32_t H, W;         /* token grid                                  */
    int32_t wx;           /* windows per row = ceil(W/8)                 */
    int32_t windows_per_frame;
    /* fused routing (routed kernels only; the block chain's MoE blocks) */
    const uint16_t* wr;   /* packed [np/16][dim/32]; rows >= n_experts 0 */
    const float* br;      /* [np]; entries >= n_experts are -inf          */
    int32_t* assign;      /* [cap] expert id per token                    */
    int32_t* counts;      /* expert e's total at counts[e * count_stride], zero on entry */
    int32_t* perm;        /* [n_experts][cap] token ids bucketed by expert */
    int32_t* zero_next;   /* if set, workgroup 0 clears zero_next[e * count_stride],
                             e < n_experts: the next block's counters            */
    int32_t n_experts;
    int32_t cap;          /* tokens in the launch = batch * H * W         */
    int32_t count_stride; /* ints between counters (a cache line apart in the chain) */
    int32_t pad_;
    /* fused up-projection (first block of the adapted chain): if set, `in`
     * holds 128-channel rows (in_frame_elems per frame) and the block's input
     * is x = r16(ReLU(W_up e + b_up)), computed in the prologue */
    const uint16_t* up_w; /* packed [dim/16][128/32]                    */
    const float* up_b;    /* [dim]                                       */
    int64_t in_frame_elems; /* H*W*dim, or H*W*128 with up_w               */
    /* fused dense FFN (prism_attn_d128[_w8]_ffn): the block's expert 0 */
    const uint16_t* ffn_w1; /* packed [dim/16][dim/32], LN2 folded in    */
    const float* ffn_b1;  /* [dim]                                       */
    const uint16_t* ffn_w2; /* packed [dim/16][dim/32]                   */
    const float* ffn_b2;  /* [dim]                                       */
} AttnArgs;

/* Router stage: at most this many 16-token tiles per wave (the LDS tables
 * are sized for it). */
#define ROUTER_MAX_TILES_PER_WAVE 8

typedef struct RouterArgs {
    const uint16_t* in;   /* features + input_offset                     */
    const uint16_t* wr;   /* packed [np/16][dim/32]; rows >= n_experts are 0 */
    const float* br;      /* [np]; entries >= n_experts are -inf          */
    int32_t* assign;      /* [n_tokens] expert id                         */
    int32_t* counts;      /* expert e's total at counts[e * count_stride] (zero on entry) */
    int32_t* perm;        /* [n_experts][cap] token ids bucketed by expert */
    int32_t n_tokens;     /* tokens in this launch (batch * per-frame)     */
    int32_t n_experts;
    int32_t np;           /* n_experts rounded up to 16                    */
    int32_t cap;          /* bucket capacity = n_tokens                    */
    int32_t tiles_per_wave; /* 16-token tiles per wave: WG = 64*tiles tokens */
    int32_t count_stride; /* ints between counters                         */
} RouterArgs;

typedef struct ExpertArgs {
    const uint16_t* in;   /* h: features + input_offset                   */
    uint16_t* out;        /* features + output_offset                     */
    const uint16_t* w1;   /* packed, expert e at + e*dim*dim halfs        */
    const float* b1;      /* [n_experts][dim]                             */
    const uint16_t* w2;
    const float* b2;
    const int32_t* counts; /* counts[e * count_stride]; NULL = dense stage (expert 0) */
    const int32_t* perm;  /* [n_experts][cap]                             */
    int32_t n_tokens;
    int32_t n_experts;
    int32_t cap;
    int32_t count_stride;
    /* fused down-projection (last block of the adapted chain): if set, the
     * block output y goes through r16(W_dn y + b_dn) and `out` holds
     * 128-channel rows */
    const uint16_t* dn_w; /* packed [128/16][dim/32]                    */
    const float* dn_b;    /* [128]                                       */
    int32_t wnt;          /* d256 8-wave 64-token kernel: expert weights
                             read non-temporally (past the memory-side
                             cache)                                       */
} ExpertArgs;

typedef struct ProjArgs {
    const uint16_t* in;   /* [n_tokens][in_dim] fp16                      */
    uint16_t* out;        /* [n_tokens][out_dim] fp16                     */
    const uint16_t* w;    /* packed [out_dim/16][in_dim/32]               */
    const float* b;       /* [out_dim]                                    */
    int64_t n_tokens;
} ProjArgs;

/* Encoder / decoder stages (codec.hpp). Grid: x = ceil(out pixels /
 * (64 * CODEC_TT_<stage>)) (enc0: blocks of CODEC_ENC0_ROWS x CODEC_ENC0_COLS), y = frames;
 * 256 threads. */
typedef struct CodecArgs {
    const uint16_t* in;   /* the CHW frame (enc0), an NHWC map, or the decoder's coarse map */
    const uint16_t* skip; /* decoder skip map (NHWC), NULL for the encoder */
    uint16_t* out;        /* NHWC output map; the CHW display image for dec1_out */
    const uint16_t* w;    /* packed [COUT/16][K/32] fragments                 */
    const float* b;       /* [COUT]                                           */
    const uint16_t* w2;   /* dec1_out: packed 32 -> 12 fragment, rows padded to 16,
                             columns permuted to the accumulator lane order    */
    const float* b2;      /* dec1_out: [16], entries 12..15 zero              */
    int64_t in_frame, skip_frame, out_frame; /* elements per frame           */
    int32_t in_w, in_h;   /* conv input map, or the decoder's coarse map      */
    int32_t out_w, out_h; /* output map (dec1_out: before the PixelShuffle)   */
} CodecArgs;

/* 16-pixel tiles per wave of each codec stage, and (RS) how many waves share a
 * pixel group, splitting its output channels: a workgroup covers
 * 16 * TT * 4 / RS pixels */
#define CODEC_TT_ENC1 4
/* enc0 output block per workgroup (rows x columns) */
#define CODEC_ENC0_ROWS 4
#define CODEC_ENC0_COLS 64
#define CODEC_TT_ENC2 2
#define CODEC_TT_ENC3 2
#define CODEC_TT_DEC3 2
#define CODEC_TT_DEC2 4
#define CODEC_TT_DEC1 2
#define CODEC_RS_ENC1 1
#define CODEC_RS_ENC2 1
#define CODEC_RS_ENC3 1
#define CODEC_RS_DEC3 1
#define CODEC_RS_DEC2 1
/* KSP: how many waves of a pixel group split the stage's reduction (its
 * k-steps) instead of its channels; a workgroup then covers
 * 16 * TT * 4 / KSP pixels (RS is 1 for such a stage) */
#define CODEC_KSP_ENC1 1
#define CODEC_KSP_ENC2 1
#define CODEC_KSP_ENC3 4
#define CODEC_KSP_DEC3 1
#define CODEC_KSP_DEC2 1
/* the fused enc0 + enc1 launch: enc1 output block per workgroup (r1 rows x
 * columns; its e0 region is (2 rows + 1) x (2 columns + 1)) */
#define CODEC_ENC01_ROWS 4
#define CODEC_ENC01_COLS 32
/* the fused enc2 + enc3 launch: enc3 output block per workgroup (r3 rows x
 * columns, 32 pixels), and whether the blocks go to the XCDs in bands */
#define CODEC_ENC23_ROWS 4
#define CODEC_ENC23_COLS 8
#define CODEC_ENC23_BAND 1
/* enc2 over an LDS window (codec_conv_window): output block rows x columns,
 * weight fragments this many k-steps ahead */
#define CODEC_WIN_ROWS_ENC2 2
#define CODEC_WIN_COLS_ENC2 16
#define CODEC_WIN_DW_ENC2 3

#endif
