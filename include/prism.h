/*
 * prism.h - C ABI of the MI355X-native Prism bottleneck transformer.
 *
 * Drop-in for the reference's hot path: the per-block sequence
 *   split2_qkv_attn_d256 -> moe_router -> moe_expert_skip
 * (reference vulkan_engine/prism_moe_bench.cpp:262-291, :414-438).
 *
 * Conventions kept from the reference's operator surface:
 *  - Activations are fp16, HWC, token-major: element (t, c) of a frame sits at
 *    t*dim + c with t = y*W + x (prism_moe_bench.cpp:137, stage shaders'
 *    coopVecLoadNV(..., (input_offset + t*dim)*2)). A batch is consecutive
 *    frames at a stride of n_tokens*dim elements.
 *  - Weights are one flat fp16 blob; every tensor is addressed by its ELEMENT
 *    offset, row-major [out][in] (prism_moe_bench.cpp:164-172,
 *    vulkan_engine/export_weights.py:96-120).
 *  - One launch per block stage; the launch parameter structs mirror the
 *    stages' push-constant blocks field for field, plus the offsets of the
 *    pre-LayerNorm tensors (LN1 before attention, LN2 before router/experts).
 *  - Feature and aux arenas are caller-owned device buffers addressed by
 *    element offsets, as the reference's bindings 1 (fp16 features) and 2
 *    (int32 aux) are.
 *
 * Every entry point returns 0 on success or a negative PRISM_ERR_* code; no
 * C++ exception crosses the ABI. prism_last_error() gives the message.
 * A context is not thread-safe; calls on one context are stream-ordered.
 * Streams are passed as void* holding a hipStream_t (NULL = default stream).
 */
#ifndef PRISM_H
#define PRISM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRISM_OK               0
#define PRISM_ERR_INVALID     -1 /* bad argument, size, offset or shape      */
#define PRISM_ERR_UNSUPPORTED -2 /* valid but not implemented (e.g. dim 192) */
#define PRISM_ERR_HIP         -3 /* a HIP runtime call failed                */
#define PRISM_ERR_STATE       -4 /* e.g. weights not loaded                  */
#define PRISM_ERR_BLOB        -5 /* weight blob or offset table inconsistent */
#define PRISM_ERR_NOMEM       -6 /* host or device allocation failed         */
#define PRISM_ERR_CODE_OBJECT -7 /* kernel code object missing or invalid    */

/* Routing modes for the synthetic weight generator. */
#define PRISM_ROUTE_RANDOM      0 /* router bias ~N(0, 0.02) like every bias  */
#define PRISM_ROUTE_UNIFORM     1 /* router bias = 0 (near-uniform load)      */
#define PRISM_ROUTE_ZIPF        2 /* bias fitted to a Zipf(1.1) expert load   */
#define PRISM_ROUTE_ADVERSARIAL 3 /* bias fitted to 50% on expert 0, rest uniform */

typedef struct prism_ctx prism_ctx;

/* Model shape. n_experts == 1 is a dense block (FFN d->d->d, no router).
 * Supported: (dim 256, 8 heads x 32) and (dim 128, 8 heads x 16); window 8;
 * 1 <= n_experts <= 64. */
typedef struct prism_model_desc {
    int32_t dim, n_blocks, n_heads, head_dim, n_experts;
    int32_t spatial_h, spatial_w, window;
} prism_model_desc;

/* Element offsets of one block's tensors in the fp16 blob. Expert e's tensors
 * are at exp_* + e*exp_stride (prism_moe_bench.cpp:168-170). For a dense
 * block router_w/router_b are unused. */
typedef struct prism_block_offsets {
    int64_t ln1_g, ln1_b, qkv_w, qkv_b, out_w, out_b;
    int64_t ln2_g, ln2_b, router_w, router_b;
    int64_t exp_w1, exp_b1, exp_w2, exp_b2, exp_stride;
} prism_block_offsets;

/* Attention stage parameters: shaders/split2_qkv_attn_d256.comp.glsl:11-16
 * {n_tokens, dim, n_heads, head_dim, spatial_w, spatial_h, window_size,
 *  qkv_w, qkv_b, out_w, out_b, input_offset, output_offset} + LN1 offsets.
 * n_tokens is the per-frame token count and must equal spatial_w*spatial_h,
 * and be at least 64: every window keys all 64 of its slots, which is the
 * reference's key set (the first min(64, n_tokens) slots) exactly when a frame
 * has 64 tokens or more; smaller frames are refused with
 * PRISM_ERR_UNSUPPORTED (attention stage calls and the block chains). */
typedef struct prism_attn_push {
    int32_t n_tokens, dim, n_heads, head_dim;
    int32_t spatial_w, spatial_h, window_size;
    int64_t qkv_w, qkv_b, out_w, out_b;
    int64_t input_offset, output_offset;
    int64_t ln1_g, ln1_b;
} prism_attn_push;

/* Router stage parameters: shaders/moe_router.comp.glsl:11-17
 * {n_tokens, dim, n_experts, router_w, router_b, input_offset,
 *  assignment_offset, count_offset} + LN2 offsets + perm_offset.
 * aux layout: assignment [batch*n_tokens] int32 (expert id per token),
 * counts [n_experts] (tokens per expert), and perm [n_experts][batch*n_tokens]
 * (token indices bucketed by expert: the counting sort's output; the order
 * inside a bucket is unspecified). The call writes the counts itself (the
 * router kernel counts into a row of the context's own, then a one-workgroup
 * launch copies the totals), so nothing is required of them on entry. */
typedef struct prism_router_push {
    int32_t n_tokens, dim, n_experts;
    int64_t router_w, router_b;
    int64_t input_offset;
    int64_t assignment_offset, count_offset;
    int64_t ln2_g, ln2_b;
    int64_t perm_offset;
} prism_router_push;

/* Expert stage parameters: shaders/moe_expert_skip.comp.glsl:13-18
 * {n_tokens, dim, expert_id, w1, b1, w2, b2, input_offset, output_offset,
 *  assignment_offset}, widened to ONE launch for all experts: expert_id is
 * replaced by n_experts + expert_stride (expert e at w1 + e*expert_stride),
 * and the router's count/perm regions are read (not modified) instead of
 * re-scanning the assignment. n_experts == 1 with count_offset < 0 is the
 * dense FFN stage (every token, expert 0). */
typedef struct prism_expert_push {
    int32_t n_tokens, dim, n_experts;
    int64_t w1, b1, w2, b2, expert_stride;
    int64_t input_offset, output_offset;
    int64_t assignment_offset, count_offset;
    int64_t ln2_g, ln2_b;
    int64_t perm_offset;
} prism_expert_push;

/* ---- host-only helpers (no GPU needed) -------------------------------- */

/* Fill offs[0..n_blocks) with the blob layout (the reference's bump
 * allocator wa(), prism_moe_bench.cpp:164-172, repeated per block with the LN
 * tensors added) and return the blob size in elements. offs may be NULL. */
int prism_layout(const prism_model_desc* desc, prism_block_offsets* offs,
                 int64_t* total_elems);

/* Check a model description and an offset table against a blob of
 * blob_elems fp16 elements: shapes supported, every tensor in bounds and
 * 8-element (16-byte) aligned. */
int prism_validate(const prism_model_desc* desc, const prism_block_offsets* offs,
                   int64_t blob_elems);

/* Synthetic weights: every W and b ~N(0, 0.02), LN gamma = 1, beta = 0, from a
 * counter-based generator (splitmix64 + Box-Muller) keyed on (seed, tensor).
 * The router bias follows `routing` (PRISM_ROUTE_*). Writes blob (blob_elems
 * fp16) and offs (n_blocks entries). */
int prism_synth_weights(const prism_model_desc* desc, uint64_t seed, int32_t routing,
                        uint16_t* blob, int64_t blob_elems, prism_block_offsets* offs);

/* n fp16 values ~N(0, std^2) from the same generator (stream selects the
 * tensor). Activations use stream 0. */
int prism_synth_normal_f16(uint16_t* dst, int64_t n, uint64_t seed, uint64_t stream,
                           float std);

/* Tokens per expert of an assignment array (host helper for load reports). */
int prism_histogram(const int32_t* assign, int64_t n, int32_t n_experts, int64_t* counts);

/* The device weight layout: repack a row-major fp16 matrix w[rows][k] into
 * 16x16x32-MFMA A-operand fragments (fragment (rt, ks) = rows 16rt..16rt+15 x
 * columns 32ks..32ks+31, 1 KiB, lane l holding w[16rt + l%16][32ks + 8(l/16)
 * + 0..7]). Rows rows..rows_padded-1 are zero. k % 32 == 0, rows_padded % 16
 * == 0. prism_load_weights applies this to every GEMM weight. No reference
 * counterpart: the reference hands row-major matrices to coopVecMatMulAddNV
 * (e.g. shaders/moe_expert_skip.comp.glsl:36-39). */
int prism_pack_weight(const uint16_t* w, int32_t rows, int32_t k, int32_t rows_padded,
                      uint16_t* dst);

/* ---- context ------------------------------------------------------------ */

/* Create a context on HIP device `device`, loading the kernel code object
 * from code_object_path (NULL = prism_kernels.hsaco next to this library).
 * On failure *out is NULL and prism_last_error(NULL) has the message. */
int prism_create(prism_ctx** out, int32_t device, const char* code_object_path);
void prism_destroy(prism_ctx* ctx);
const char* prism_last_error(const prism_ctx* ctx);

/* Upload a weight blob (host memory, fp16, `bytes` long) laid out per offs
 * (desc->n_blocks entries) and repack it into the device's MFMA fragment
 * layout. Equivalent of PrismVulkan::LoadWeights (prism_vulkan.cpp:558-611).
 * Each LayerNorm's gamma/beta is folded into the weights that consume its
 * output (W' = r16(W diag(gamma)), b' = b + W beta); a folded weight that
 * overflows fp16 fails with PRISM_ERR_BLOB, and the previous weights stay
 * loaded. */
int prism_load_weights(prism_ctx* ctx, const prism_model_desc* desc, const void* blob,
                       size_t bytes, const prism_block_offsets* offs);

/* Same, reading the blob from a file (the exporter's flat .weights format). */
int prism_load_weights_file(prism_ctx* ctx, const prism_model_desc* desc,
                            const char* path, const prism_block_offsets* offs);

/* ---- per-stage launches (one dispatch each) --------------------------- */

/* features: device fp16 arena; aux: device int32 arena. The weight offsets
 * in the push structs must name tensors of a loaded block. prism_router
 * writes the assignment, the counts (from zero) and the buckets; it counts
 * into a row of the context's own, counters 256 bytes apart, and a
 * one-workgroup launch copies the totals to `counts`, so router and
 * attention-route calls on one context must not overlap on different
 * streams. */
int prism_attn(prism_ctx* ctx, const prism_attn_push* p, void* features, int32_t batch,
               void* stream);
int prism_router(prism_ctx* ctx, const prism_router_push* p, const void* features,
                 int32_t* aux, int32_t batch, void* stream);
int prism_experts(prism_ctx* ctx, const prism_expert_push* p, void* features,
                  int32_t* aux, int32_t batch, void* stream);

/* Attention and router stages in ONE launch: the attention kernel routes its
 * output tile before storing it (LN2 + router GEMM + argmax + counting sort
 * in its epilogue), replacing the two dispatches
 * prism_moe_bench.cpp:266-275. pr must name the same block as pa and read
 * its output (pr->input_offset == pa->output_offset, same n_tokens); the
 * features at pa->output_offset, assignment, counts and perm come out as
 * prism_attn followed by prism_router would leave them (bit-identical expert
 * ids and counts; the order inside a bucket is unspecified). No reference
 * counterpart as a single call: the block chain uses it for MoE blocks. The
 * kernel counts into a row of the context's own, counters 256 bytes apart,
 * and a one-workgroup launch copies the totals to `counts`: calls on one
 * context must not overlap on different streams. */
int prism_attn_route(prism_ctx* ctx, const prism_attn_push* pa, const prism_router_push* pr,
                     void* features, int32_t* aux, int32_t batch, void* stream);

/* ---- whole block chain -------------------------------------------------- */

/* Run all loaded blocks on `batch` frames: in and out are device fp16
 * [batch][H*W][dim] (in is not modified). Eager launches. */
int prism_forward(prism_ctx* ctx, const void* in, void* out, int32_t batch, void* stream);

/* Same chain replayed from a hipGraph captured on the first call for this
 * (in, out, batch, stream); later calls with the same arguments only launch
 * the graph. */
int prism_forward_graph(prism_ctx* ctx, const void* in, void* out, int32_t batch,
                        void* stream);

/* prism_forward without any allocation: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under hipGraph stream
 * capture, tight serving loops, harnesses that forbid hipMalloc): the same
 * launches as prism_forward, bit-identical output, but the chain's workspace
 * (attention output, ping-pong rows, per-block assignments, routing
 * counters, buckets) lives in a fixed per-GPU device array of 16 MiB that the
 * library holds from prism_create until the process ends; the call itself
 * allocates and frees nothing. A forward whose workspace exceeds 16 MiB
 * (2*n*dim*2 + n_blocks*n*4 + n_experts*n*4 bytes + the counter rows, n =
 * batch*H*W; e.g. MoE-64 d256 x 16 blocks at 68x120 fits at batch 1) is
 * refused with PRISM_ERR_INVALID before any launch. The array keeps the last
 * call's contents (the call clears the counters it needs first). Calls on one
 * GPU, from any context, stream or host thread, share the array and run one
 * after another: each call's stream first waits for the previous call's
 * launches (one event per GPU, recorded after every call). Under stream
 * capture that wait is not recorded into the graph, so replays of a captured
 * call are ordered only by the stream the caller launches them on. */
int prism_forward_noalloc(prism_ctx* ctx, const void* in, void* out, int32_t batch, void* stream);

/* Measurement aid, no counterpart in the reference (the reference times its
 * recorded frame with timestamp queries around the whole chain,
 * prism_moe_bench.cpp:183-209). Runs the launches of prism_forward for
 * `batch` frames (the same kernels, grids and arguments, sub-chain by
 * sub-chain) one after another on `stream`, with an event between every two
 * launches, waits for them, and returns the mean duration in ms of the
 * chain's attention launches (attn_ms) and of its expert launches
 * (expert_ms), and the workgroup count of each (the first launch of each
 * kind). A dense block runs its FFN inside its attention launch, so a dense
 * model reports expert_ms = 0 and expert_grid = 0. `out` receives the
 * chain's output, as from prism_forward. */
int prism_chain_launch_times(prism_ctx* ctx, const void* in, void* out, int32_t batch, void* stream,
                             float* attn_ms, float* expert_ms, int32_t* attn_grid, int32_t* expert_grid);

/* Device pointer to the expert assignment of every block of the most recent
 * forward: [n_blocks][batch*H*W] int32. */
int prism_forward_assignments(prism_ctx* ctx, const int32_t** assign_dev,
                              int64_t* tokens_per_block);

/* ---- projection adapters (either side of the block chain) --------------- */

/* Element offsets of the two adapters in an fp16 blob: the reference's
 * end-to-end layout (prism_moe_bench.cpp:351-352) proj_up_w [dim][in_dim],
 * proj_up_b [dim], proj_dn_w [in_dim][dim], proj_dn_b [in_dim]. in_dim is the
 * encoder's channel count (128). */
typedef struct prism_adapter_offsets {
    int32_t in_dim, pad_;
    int64_t up_w, up_b, down_w, down_b;
} prism_adapter_offsets;

/* Projection stage parameters: shaders/pw_project_128to256.comp.glsl:11-15 and
 * shaders/pw_project_256to128.comp.glsl:9-13 {n_tokens, w_offset, b_offset,
 * input_offset, output_offset}. n_tokens is per frame; the weight offsets must
 * name the loaded adapter. */
typedef struct prism_project_push {
    int32_t n_tokens, pad_;
    int64_t w_offset, b_offset, input_offset, output_offset;
} prism_project_push;

/* Place the adapters in a blob from element `base` on (8-element aligned,
 * the reference's wa() order); *end = first element past them. Host only. */
int prism_adapter_layout(const prism_model_desc* desc, int32_t in_dim, int64_t base,
                         prism_adapter_offsets* offs, int64_t* end);

/* Upload both adapters (host fp16 blob, `bytes` long) for the loaded model's
 * dim; in_dim 128. Loading weights of another dim drops them. */
int prism_load_adapters(prism_ctx* ctx, const void* blob, size_t bytes,
                        const prism_adapter_offsets* offs);

/* pw_project_128to256 (shaders/pw_project_128to256.comp.glsl:20-40):
 * out = ReLU(r16(W_up x + b_up)), in_dim -> dim channels per token.
 * pw_project_256to128 (shaders/pw_project_256to128.comp.glsl:20-33):
 * out = r16(W_down x + b_down), dim -> in_dim. One launch each. */
int prism_project_up(prism_ctx* ctx, const prism_project_push* p, void* features,
                     int32_t batch, void* stream);
int prism_project_down(prism_ctx* ctx, const prism_project_push* p, void* features,
                       int32_t batch, void* stream);

/* The transformer section of the reference's end-to-end frame
 * (prism_moe_bench.cpp:408-444): up-projection, every block, down-projection.
 * in and out: device fp16 [batch][H*W][in_dim] (in is not modified). The
 * up-projection runs inside the first block's attention launch and the
 * down-projection inside the last block's expert launch; the result is
 * bit-identical to prism_project_up, prism_forward, prism_project_down.
 * _graph replays a captured hipGraph like prism_forward_graph. */
int prism_forward_adapted(prism_ctx* ctx, const void* in, void* out, int32_t batch,
                          void* stream);
int prism_forward_adapted_graph(prism_ctx* ctx, const void* in, void* out, int32_t batch,
                                void* stream);

/* ---- model files ------------------------------------------------------- */

/* The on-disk model is a pair: <name>.weights, flat fp16 values with no header
 * (what the reference's exporter writes, vulkan_engine/export_weights.py:
 * 96-113), and <name>.json, its sidecar ("format": "prism-transformer-v1":
 * total_fp16_values, total_bytes, the model shape, and one entry per layer with
 * its kind, block and fp16 element offsets, extending the reference's
 * per-layer weight_offset_fp16 / bias_offset_fp16 entries, :115-120). Written
 * by prism-inference_amd/export_weights.py. */

/* Host only: parse and validate a sidecar. offs receives desc->n_blocks
 * entries (offs_capacity at least that; offs may be NULL to query the shape);
 * adapters / has_adapters / total_elems may be NULL. */
int prism_read_model_json(const char* json_path, prism_model_desc* desc, prism_block_offsets* offs,
                          int32_t offs_capacity, prism_adapter_offsets* adapters, int32_t* has_adapters,
                          int64_t* total_elems);

/* Load a model pair: sidecar (json_path, or NULL = weights_path with
 * ".weights" replaced by ".json"), file size checked against it, then the
 * blocks (prism_load_weights) and, if the sidecar has them, the adapters.
 * Replaces PrismVulkan::LoadWeights (prism_vulkan.cpp:558-611). */
int prism_load_model_file(prism_ctx* ctx, const char* weights_path, const char* json_path);

/* ---- conv encoder / fused decoder (the end-to-end frame) ---------------- */

/* The end-to-end frame of prism_moe_bench.cpp:387-471 around the blocks:
 *   encoder  enc0 conv3x3 9->32 (render resolution r0), enc1 conv3x3/2 32->64
 *            (r1), enc2 conv3x3/2 64->128 (r2), enc3 conv3x3/2 128->128 (r3 =
 *            the token grid), each + ReLU;
 *   [adapters + blocks on the r3 tokens];
 *   decoder  dec3 NN-up + concat enc2 -> PW 256->128 (r2), dec2 NN-up + concat
 *            enc1 -> PW 192->64 (r1), dec1 NN-up + concat enc0 -> PW 96->32
 *            (r0), each + ReLU; output PW 32->12; PixelShuffle(2) + sigmoid
 *            -> RGB at 2 x r0.
 * r(i+1) = ceil(r(i) / 2) and r3 must be the model's spatial_h x spatial_w;
 * render_w * render_h * 64 (the 32-channel fp16 map) must stay under 2^31.
 * Weight offsets (fp16 elements, 8-aligned), row-major [out][in] with the
 * reference's column orders: conv k = ic*9 + ky*3 + kx (enc*), concat order
 * upsampled channels first (dec*). */
typedef struct prism_codec_offsets {
    int32_t render_w, render_h; /* r0, e.g. 960 x 540 */
    int32_t in_channels, scale; /* 9 and 2 (the only values supported) */
    int64_t enc0_w, enc0_b, enc1_w, enc1_b, enc2_w, enc2_b, enc3_w, enc3_b;
    int64_t dec3_w, dec3_b, dec2_w, dec2_b, dec1_w, dec1_b, out_w, out_b;
} prism_codec_offsets;

/* Place the encoder, the adapters and the decoder in a blob from element
 * `base` on, in the reference's wa() order (prism_moe_bench.cpp:347-357:
 * enc_ic, enc1, enc2, enc3, proj_up, proj_dn, d3_pw, d2_pw, d1_pw, out_pw);
 * *end = first element past them. adapters may be NULL. Host only. */
int prism_codec_layout(const prism_model_desc* desc, int32_t render_w, int32_t render_h, int64_t base,
                       prism_codec_offsets* codec, prism_adapter_offsets* adapters, int64_t* end);

/* Upload the encoder and decoder weights (host fp16 blob, `bytes` long) for
 * the loaded model; loading weights of another shape drops them. */
int prism_load_codec(prism_ctx* ctx, const void* blob, size_t bytes, const prism_codec_offsets* offs);

/* The encoder: frame fp16 CHW [batch][9][render_h][render_w] -> bottleneck
 * fp16 [batch][r3 tokens][128] (token-major, the adapted chain's input). The
 * encoder maps stay in the engine for the next prism_decode of `batch`
 * frames. Two launches: enc0 + enc1 in one (enc1 reads its input from the
 * workgroup's on-chip copy of e0), then enc2 + enc3 in one (enc3 reads its
 * input from the workgroup's on-chip copy of e2); the result equals stages
 * 0-3 of prism_codec_stage bit for bit. */
int prism_encode(prism_ctx* ctx, const void* frame, void* bottleneck, int32_t batch, void* stream);

/* The decoder: bottleneck fp16 [batch][r3 tokens][128] -> display fp16 CHW
 * [batch][3][2 render_h][2 render_w], with the skips of the last
 * prism_encode (same batch). Two launches: dec3, then dec2 + dec1 + output
 * conv + PixelShuffle + sigmoid in one (the dec2 map stays on chip); the
 * result equals stages 4, 5 and 6 of prism_codec_stage bit for bit. */
int prism_decode(prism_ctx* ctx, const void* bottleneck, void* display, int32_t batch, void* stream);

/* One codec stage on caller buffers, for stage-level checks: stage 0..3 =
 * enc0..enc3 (in: the CHW frame for stage 0, else the previous NHWC map;
 * skip unused), 4 = dec3, 5 = dec2 (in: the coarse NHWC map, skip: the
 * encoder map of the output resolution), 6 = dec1 + output conv +
 * PixelShuffle + sigmoid (out: the CHW display image). Maps between stages
 * are NHWC fp16 [batch][pixels][channels]. */
int prism_codec_stage(prism_ctx* ctx, int32_t stage, const void* in, const void* skip, void* out, int32_t batch,
                      void* stream);

/* The whole end-to-end frame: encoder, up-projection, every block,
 * down-projection, decoder (needs the codec and the adapters loaded).
 * frame: [batch][9][render_h][render_w], display: [batch][3][2 render_h]
 * [2 render_w], both fp16 CHW. _graph replays a captured hipGraph. */
int prism_forward_e2e(prism_ctx* ctx, const void* frame, void* display, int32_t batch, void* stream);
int prism_forward_e2e_graph(prism_ctx* ctx, const void* frame, void* display, int32_t batch, void* stream);

/* ---- host renderer interop ---------------------------------------------- */

/* PrismVulkan::InitWithDevice (vulkan_engine/prism_vulkan.h:81-85,
 * prism_vulkan.cpp:27-48): an engine on the renderer's device and queue.
 * Here: prism_create on `device`, bound to the renderer's stream (a
 * hipStream_t of that device; NULL = the null stream), on which
 * prism_infer_gpu runs. A stream of another device is refused. */
int prism_init_with_device(prism_ctx** out, int32_t device, void* stream, const char* code_object_path);

/* PrismVulkan::InferGPU (prism_vulkan.h:93-98, prism_vulkan.cpp:922-1005): one
 * inference from caller device memory to caller device memory at byte offsets
 * into the caller's buffers, then wait for it. *infer_ms (may be NULL)
 * receives the inference's GPU time (HIP events around the graph launch).
 * Zero-copy: the kernels read in_buf + in_offset and write out_buf +
 * out_offset themselves, where the reference copies through its own feature
 * buffer. Runs a captured hipGraph (captured on the first call for a given
 * pair of addresses) on the bound stream: the whole end-to-end frame (frame
 * in, display out, as prism_forward_e2e) when the codec and adapters are
 * loaded, else the adapted chain, in/out [batch][H*W][in_dim], when adapters
 * are loaded, else the blocks, [batch][H*W][dim]. Both addresses 16-byte
 * aligned; the two ranges must not overlap. */
int prism_infer_gpu(prism_ctx* ctx, const void* in_buf, uint64_t in_offset, void* out_buf, uint64_t out_offset,
                    int32_t batch, float* infer_ms);

/* Renderer-owned memory as engine buffers: import an allocation exported as an
 * opaque file descriptor (a VkDeviceMemory exported through
 * VK_KHR_external_memory_fd, or any dma-buf of this device) and map its first
 * `size` bytes as a device pointer for prism_infer_gpu / prism_forward. The
 * caller keeps its descriptor (the library imports a duplicate and closes
 * that at release). Release waits for the device, then unmaps. No reference
 * counterpart: the reference shares the renderer's VkDevice and VkBuffers
 * directly. */
typedef struct prism_external_buffer prism_external_buffer;
int prism_import_external_memory(prism_ctx* ctx, int32_t fd, uint64_t size, prism_external_buffer** buf,
                                 void** dev_ptr);
int prism_release_external_memory(prism_ctx* ctx, prism_external_buffer* buf);

/* aux arena size in int32 elements that a router + expert pair needs for
 * n_experts experts and batch*n_tokens tokens when laid out as
 * [assignment | counts | perm]. */
int64_t prism_aux_elems(int32_t n_experts, int64_t tokens);

#ifdef __cplusplus
}
#endif
#endif /* PRISM_H */
