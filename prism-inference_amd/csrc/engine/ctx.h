/* ctx.h - the engine context and helpers shared by the host engine's
 * translation units (engine.cpp, codec.cpp). */
#ifndef PRISM_CTX_H
#define PRISM_CTX_H

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <vector>

#include "../kernel_args.h"
#include "prism.h"

namespace prism {

struct DevBlock {
    prism_block_offsets offs;
    uint16_t* wqkv;
    float* bqkv;
    float* bqkv_pad; /* the blob's QKV bias for padded window slots; NULL if LN1 beta = 0 */
    uint16_t* wo;
    float* bo;
    uint16_t* wr;
    float* br;
    uint16_t* w1;
    float* b1;
    uint16_t* w2;
    float* b2;
};

}  // namespace prism

using prism::DevBlock;

/* The chain's per-expert counters sit 256 bytes apart: every workgroup of a
 * routed attention launch adds to them, and counters sharing a cache line
 * would serialise those atomics in one memory channel. */
static constexpr int CHAIN_COUNT_STRIDE = 64;
/* The chain runs as up to CHAIN_SPLIT independent sub-chains, one per
 * CHAIN_SPLIT_FRAMES frames, on their own streams (parallel branches of the
 * hipGraph): windows and tokens never interact across frames, and one
 * sub-chain's expert launches overlap another's attention launches and the
 * tails of both. */
static constexpr int CHAIN_SPLIT = 2;
static constexpr int CHAIN_SPLIT_FRAMES = 2;
static_assert(CHAIN_SPLIT >= 1 && CHAIN_SPLIT <= 4, "sub-chain streams");
/* d256 expert launches of at least this many 128-token tiles (two per CU)
 * use the 128-token kernel: each streamed weight fragment then feeds twice
 * the tokens. Smaller grids keep 64-token tiles (8 waves below 512 tiles).
 * A stage call of that size uses 96-token tiles of the same body instead:
 * alone on the GPU, its last round of workgroups is then less empty (batch 8
 * to 16 at 68x120: 7-13 % faster); inside the block chain the other
 * sub-chain's attention launch fills that round, and 128-token tiles stay
 * ahead there. */
static constexpr int EXPERT_WIDE_MIN_TILES = 512;
/* The share of the 256 MB memory-side cache the weights may keep across
 * small-batch frames: when a model's weights exceed it, the 8-wave 64-token
 * expert kernel (the small grids of batch 1-2) reads the expert weights of
 * the first blocks non-temporally, so the rest stays resident from one frame
 * to the next instead of the whole cyclic stream missing (prism_load_weights
 * sets wnt_blocks). */
static constexpr int64_t WEIGHT_CACHE_KEEP = 224ll << 20;
/* Workgroups of a projection stage launch (persistent, 64-token tiles in a
 * loop; the d256 kernels' 210-220 VGPRs allow two per CU). At batch 16,
 * 68x120, up 128->256: 512 workgroups 18.5 us, 384 20.6, 256 23.5, 1024
 * 21.8 (one workgroup per tile: 20.5). */
static constexpr int PROJ_GRID_MAX = 512;

/* Attention keys all 64 slots of a window. The reference keys the first
 * min(64, n_tokens) slots in slot order (split2_qkv_attn_d256.comp.glsl:33,60),
 * which differs only for frames of fewer than 64 tokens: those are refused. */
static constexpr int ATTN_MIN_TOKENS = 64;
#define ATTN_MIN_TOKENS_WHY "the reference keys only the first n_tokens window slots below 64 tokens"

/* The block chain's working buffers for one forward: the engine's workspace
 * or the allocation-free path's scratch. */
struct ChainWs {
    uint16_t* attn = nullptr;    /* [n][dim] attention output h            */
    uint16_t* scratch = nullptr; /* [n][dim] ping-pong                     */
    uint16_t* io = nullptr;      /* adapted chain: [n][dim] 256-channel rows */
    int32_t* assign = nullptr;   /* [n_blocks][n]                          */
    int32_t* counts = nullptr;   /* [CHAIN_SPLIT][n_blocks][N][CHAIN_COUNT_STRIDE] */
    int32_t* perm = nullptr;     /* per sub-chain j: [N][its tokens], back to back */
    int64_t n = 0;               /* tokens of the forward (assignment row stride) */
};

enum ChainMode { CHAIN_BLOCKS = 0, CHAIN_ADAPTED = 1, CHAIN_E2E = 2 };

struct prism_ctx {
    int device = 0;
    hipModule_t module = nullptr;
    hipFunction_t f_attn[2][2][5] = {}; /* [d128, d256][4 waves, 8 waves][routed: padded experts / 16] */
    hipFunction_t f_attn_ffn[2][2] = {}; /* dense blocks, FFN fused: [d128, d256][4 waves, 8 waves] */
    hipFunction_t f_router[2][4] = {};  /* [dim][padded experts / 16 - 1] */
    hipFunction_t f_expert[2][2] = {};  /* [dim][4 waves, 8 waves], 64-token tiles */
    hipFunction_t f_expert_wide = nullptr; /* d256, 128-token tiles */
    hipFunction_t f_expert_wide96 = nullptr; /* d256, 96-token tiles (large stage calls) */
    hipFunction_t f_zero = nullptr;
    hipFunction_t f_take = nullptr;
    hipFunction_t f_proj[2][2] = {};    /* [dim][up, down] */
    hipFunction_t f_codec[7] = {};     /* enc0..enc3, dec3, dec2, dec1_out */
    hipFunction_t f_codec21 = nullptr; /* dec2 + dec1_out in one launch (the decoder's last two stages) */
    hipFunction_t f_enc01 = nullptr;   /* enc0 + enc1 in one launch (the encoder's first two stages) */
    hipFunction_t f_enc23 = nullptr;   /* enc2 + enc3 in one launch (the encoder's last two stages) */
    std::string err;

    bool loaded = false;
    prism_model_desc desc{};
    void* warena = nullptr;
    std::vector<DevBlock> blocks;
    int wnt_blocks = 0; /* leading blocks whose expert weights stream non-temporally */

    /* projection adapters (prism_load_adapters) */
    void* aarena = nullptr;
    bool adapters = false;
    prism_adapter_offsets aoffs{};
    uint16_t *up_w = nullptr, *down_w = nullptr; /* packed */
    float *up_b = nullptr, *down_b = nullptr;

    /* forward workspace */
    void* ws = nullptr;
    int ws_batch = 0;
    ChainWs wsb;                  /* its buffers (ws_batch frames)             */
    int64_t ws_tokens = 0;
    int64_t fwd_tokens = 0;       /* tokens per block of the last forward */
    const int32_t* fwd_assign = nullptr; /* [n_blocks][fwd_tokens] of the last forward */
    void* scratch = nullptr;      /* this device's allocation-free workspace (scratch.hip) */
    bool counts_dirty = false;    /* block 0's counters may be nonzero */
    unsigned last_grid = 0;       /* workgroups of the last kernel launched (chain timing) */
    int32_t* stage_counts = nullptr; /* prism_attn_route: private counters, CHAIN_COUNT_STRIDE apart */
    bool stage_dirty = false;        /* ... possibly nonzero (a call stopped between its launches) */

    hipStream_t user_stream = nullptr;  /* prism_init_with_device: the renderer's stream */
    hipEvent_t ev_t0 = nullptr, ev_t1 = nullptr; /* prism_infer_gpu timing */

    hipStream_t cap_stream = nullptr;
    hipStream_t sub_stream[3] = {};   /* sub-chains 1.. (default priority) */
    hipEvent_t ev_fork = nullptr, ev_join[3] = {};
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    const void* g_in = nullptr;
    void* g_out = nullptr;
    int g_batch = 0;
    int g_mode = 0;               /* ChainMode of the captured graph */

    /* conv encoder / fused decoder (codec.cpp) */
    bool codec = false;
    prism_codec_offsets coffs{};
    void* carena = nullptr;       /* packed stage weights + fp32 biases */
    const uint16_t* cw[8] = {};   /* enc0..enc3, dec3, dec2, dec1, out (packed) */
    const float* cb[8] = {};
    int cr_w[4] = {}, cr_h[4] = {}; /* r0 (render) .. r3 (= the token grid) */
    void* cws = nullptr;          /* codec workspace for cws_batch frames */
    int cws_batch = 0;
    uint16_t *ce0 = nullptr, *ce1 = nullptr, *ce2 = nullptr; /* encoder maps kept for the decoder's skips */
    uint16_t *cbott = nullptr, *cchain = nullptr;             /* bottleneck in / chain out (e2e) */
    uint16_t *cd3 = nullptr;
};

/* The allocation-free forward's workspace: one device array of this many
 * bytes per GPU (scratch.hip), e.g. MoE-64 d256 x 16 blocks at 68x120 and
 * batch 1 takes 11.5 MB of it. */
static constexpr size_t PRISM_SCRATCH_BYTES = size_t(16) << 20;
static constexpr int PRISM_SCRATCH_MAX_DEVICES = 64;

/* scratch.hip: the scratch array's address on `device` (which must be the
 * current device), taken once per device and kept, together with the
 * device's completion event for the array's calls. */
hipError_t scratch_device_address(int device, void** out);
/* the event the last prism_forward_noalloc on `device` recorded after its
 * launches (created by scratch_device_address), and the host lock that
 * orders those calls */
hipEvent_t scratch_done_event(int device);
std::mutex& scratch_call_mutex(int device);

/* Record the message on the context (if any) and the thread; returns code. */
int fail(prism_ctx* c, int code, const char* fmt, ...);

#define HIP_TRY(ctx, call)                                                                   \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess)                                                                \
            return fail((ctx), PRISM_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
    } while (0)

/* engine.cpp: forget the captured chain graph */
void drop_graph(prism_ctx* c);

/* codec.cpp: the conv encoder / fused decoder stages on a stream */
void codec_release(prism_ctx* c);
int codec_ensure_workspace(prism_ctx* c, int batch);
int codec_enqueue_encode(prism_ctx* c, const uint16_t* frame, uint16_t* bottleneck, int batch, hipStream_t s);
int codec_enqueue_decode(prism_ctx* c, const uint16_t* bottleneck, uint16_t* display, int batch, hipStream_t s);
int64_t codec_frame_elems(const prism_ctx* c);   /* 9 * render_h * render_w */
int64_t codec_display_elems(const prism_ctx* c); /* 3 * (2 render_h) * (2 render_w) */

#endif
