/*
 * codec.cpp - host side of the conv encoder / fused decoder (kernels in
 * csrc/kernels/codec.hpp): weight repacking, the codec workspace and the
 * stage launches of the end-to-end frame (prism_moe_bench.cpp:387-471).
 *
 * Weights arrive in the reference's layouts (row-major [out][in]; conv
 * columns k = ic*9 + ky*3 + kx) and are repacked once into MFMA A-fragment
 * order: the stride-2 convs with columns reordered to k = tap*Cin + ic (the
 * kernels read NHWC taps), the input conv with its 81 columns as 9 taps x 16,
 * the output conv with rows padded to 16 and columns permuted to the
 * accumulator-lane order its fused kernel feeds it in. Biases become fp32.
 */
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "ctx.h"
#include "engine_internal.h"

using namespace prism;

namespace {

enum { ST_ENC0, ST_ENC1, ST_ENC2, ST_ENC3, ST_DEC3, ST_DEC2, ST_DEC1, N_STAGES };
const int kTT[N_STAGES] = {4, CODEC_TT_ENC1, CODEC_TT_ENC2, CODEC_TT_ENC3, /* enc0: own grid */
                           CODEC_TT_DEC3, CODEC_TT_DEC2, CODEC_TT_DEC1};
const int kRS[N_STAGES] = {1, CODEC_RS_ENC1, CODEC_RS_ENC2, CODEC_RS_ENC3, CODEC_RS_DEC3, CODEC_RS_DEC2, 1};
const int kKSP[N_STAGES] = {1, CODEC_KSP_ENC1, CODEC_KSP_ENC2, CODEC_KSP_ENC3, CODEC_KSP_DEC3, CODEC_KSP_DEC2, 1};
const int kInRes[N_STAGES] = {0, 0, 1, 2, 3, 2, 1};  /* resolution index of the (coarse) input map */
const int kOutRes[N_STAGES] = {0, 1, 2, 3, 2, 1, 0}; /* of the output map (dec1: before the shuffle) */
const int kInCh[N_STAGES] = {9, 32, 64, 128, 128, 128, 64};
const int kSkipCh[N_STAGES] = {0, 0, 0, 0, 128, 64, 32};
const int kOutCh[N_STAGES] = {32, 64, 128, 128, 128, 64, 12}; /* dec1: 12 channels = 3 planes x 2x2 */

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

size_t round256(size_t n) { return (n + 255) & ~size_t(255); }

/* The kernel arguments of stage st. */
CodecArgs stage_args(const prism_ctx* c, int st, const uint16_t* in, const uint16_t* skip, uint16_t* out) {
    CodecArgs a;
    memset(&a, 0, sizeof a);
    const int ir = kInRes[st], orr = kOutRes[st];
    a.in = in;
    a.skip = skip;
    a.out = out;
    a.w = c->cw[st];
    a.b = c->cb[st];
    a.w2 = st == ST_DEC1 ? c->cw[7] : nullptr;
    a.b2 = st == ST_DEC1 ? c->cb[7] : nullptr;
    a.in_w = c->cr_w[ir];
    a.in_h = c->cr_h[ir];
    a.out_w = c->cr_w[orr];
    a.out_h = c->cr_h[orr];
    const int64_t in_pix = (int64_t)a.in_w * a.in_h, out_pix = (int64_t)a.out_w * a.out_h;
    a.in_frame = in_pix * kInCh[st];
    a.skip_frame = out_pix * kSkipCh[st];
    a.out_frame = out_pix * kOutCh[st];
    return a;
}

int launch_stage(prism_ctx* c, int st, const uint16_t* in, const uint16_t* skip, uint16_t* out, int batch,
                 hipStream_t s) {
    CodecArgs a = stage_args(c, st, in, skip, out);
    const int64_t out_pix = (int64_t)a.out_w * a.out_h;
    const int64_t per_wg = 64 * kTT[st] / (kRS[st] * kKSP[st]); /* pixels per workgroup */
    const unsigned gx = st == ST_ENC0 ? (unsigned)(((a.out_w + CODEC_ENC0_COLS - 1) / CODEC_ENC0_COLS) *
                                                  ((a.out_h + CODEC_ENC0_ROWS - 1) / CODEC_ENC0_ROWS))
                        : st == ST_ENC2 ? (unsigned)(((a.out_w + CODEC_WIN_COLS_ENC2 - 1) / CODEC_WIN_COLS_ENC2) *
                                                     ((a.out_h + CODEC_WIN_ROWS_ENC2 - 1) / CODEC_WIN_ROWS_ENC2))
                                        : (unsigned)((out_pix + per_wg - 1) / per_wg);
    void* params[] = {&a};
    const hipError_t e = hipModuleLaunchKernel(c->f_codec[st], gx, (unsigned)batch, 1, 256, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipModuleLaunchKernel(codec stage %d): %s", st, hipGetErrorString(e));
    return PRISM_OK;
}

/* dec2 and dec1_out as one launch (prism_codec_dec21_out): 2 x 32 blocks of
 * the r1 map, each with the 4 x 64 r0 block above it. d2 = the dec3 map, e1
 * and e0 the skips. */
int launch_dec21(prism_ctx* c, const uint16_t* d3, const uint16_t* e1, const uint16_t* e0, uint16_t* display,
                 int batch, hipStream_t s) {
    CodecArgs a2 = stage_args(c, ST_DEC2, d3, e1, nullptr);
    CodecArgs a1 = stage_args(c, ST_DEC1, nullptr, e0, display);
    const unsigned gx = (unsigned)(((a2.out_w + 31) / 32) * ((a2.out_h + 1) / 2));
    void* params[] = {&a2, &a1};
    const hipError_t e = hipModuleLaunchKernel(c->f_codec21, gx, (unsigned)batch, 1, 256, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipModuleLaunchKernel(dec2 + dec1): %s", hipGetErrorString(e));
    return PRISM_OK;
}

/* Packed copy of W[rows][K] with column j of the packed matrix taken from
 * column colmap(j) of W (-1 = zero), rows padded to rows_p, Kp columns. */
template <class F>
void pack_mapped(const uint16_t* W, int rows, int K, int rows_p, int Kp, F colmap, std::vector<uint16_t>& dst) {
    std::vector<uint16_t> tmp((size_t)rows * Kp, 0);
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < Kp; ++j) {
            const int k = colmap(j);
            if (k >= 0 && k < K) tmp[(size_t)r * Kp + j] = W[(size_t)r * K + k];
        }
    dst.assign((size_t)rows_p * Kp, 0);
    pack_fragments(tmp.data(), rows, Kp, rows_p, dst.data());
}

int check_ctx(prism_ctx* c) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->codec) return fail(c, PRISM_ERR_STATE, "encoder / decoder weights not loaded");
    return PRISM_OK;
}

}  // namespace

void codec_release(prism_ctx* c) {
    drop_graph(c);
    if (c->carena) (void)hipFree(c->carena);
    if (c->cws) (void)hipFree(c->cws);
    c->carena = nullptr;
    c->cws = nullptr;
    c->cws_batch = 0;
    c->codec = false;
    for (int i = 0; i < 8; ++i) {
        c->cw[i] = nullptr;
        c->cb[i] = nullptr;
    }
    c->ce0 = c->ce1 = c->ce2 = c->cbott = c->cchain = c->cd3 = nullptr;
}

int64_t codec_frame_elems(const prism_ctx* c) { return 9LL * c->cr_w[0] * c->cr_h[0]; }
int64_t codec_display_elems(const prism_ctx* c) { return 12LL * c->cr_w[0] * c->cr_h[0]; }

int codec_ensure_workspace(prism_ctx* c, int batch) {
    if (c->cws && c->cws_batch >= batch) return PRISM_OK;
    drop_graph(c); /* a captured graph may point into the old workspace */
    if (c->cws) (void)hipFree(c->cws);
    c->cws = nullptr;
    c->cws_batch = 0;
    const int64_t p0 = (int64_t)c->cr_w[0] * c->cr_h[0], p1 = (int64_t)c->cr_w[1] * c->cr_h[1];
    const int64_t p2 = (int64_t)c->cr_w[2] * c->cr_h[2], p3 = (int64_t)c->cr_w[3] * c->cr_h[3];
    /* e0, e1, e2, bottleneck, chain output, d3 (the dec2 map stays in the
     * fused dec2 + dec1 launch's LDS) */
    const int64_t elems[6] = {p0 * 32, p1 * 64, p2 * 128, p3 * 128, p3 * 128, p2 * 128};
    size_t off[6], total = 0;
    for (int i = 0; i < 6; ++i) {
        off[i] = total;
        total += round256((size_t)batch * elems[i] * 2);
    }
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, total);
    if (e != hipSuccess)
        return fail(c, PRISM_ERR_NOMEM, "hipMalloc(%zu) for the encoder / decoder maps: %s", total, hipGetErrorString(e));
    uint8_t* b = static_cast<uint8_t*>(p);
    c->cws = p;
    c->cws_batch = batch;
    c->ce0 = reinterpret_cast<uint16_t*>(b + off[0]);
    c->ce1 = reinterpret_cast<uint16_t*>(b + off[1]);
    c->ce2 = reinterpret_cast<uint16_t*>(b + off[2]);
    c->cbott = reinterpret_cast<uint16_t*>(b + off[3]);
    c->cchain = reinterpret_cast<uint16_t*>(b + off[4]);
    c->cd3 = reinterpret_cast<uint16_t*>(b + off[5]);
    return PRISM_OK;
}

/* enc0 and enc1 as one launch (prism_codec_enc01): CODEC_ENC01_ROWS x
 * CODEC_ENC01_COLS blocks of the r1 map, each with the e0 region under it;
 * writes both maps. */
int launch_enc01(prism_ctx* c, const uint16_t* frame, uint16_t* e0, uint16_t* e1, int batch, hipStream_t s) {
    CodecArgs a0 = stage_args(c, ST_ENC0, frame, nullptr, e0);
    CodecArgs a1 = stage_args(c, ST_ENC1, nullptr, nullptr, e1);
    const unsigned gx = (unsigned)(((a1.out_w + CODEC_ENC01_COLS - 1) / CODEC_ENC01_COLS) *
                                   ((a1.out_h + CODEC_ENC01_ROWS - 1) / CODEC_ENC01_ROWS));
    void* params[] = {&a0, &a1};
    const hipError_t e = hipModuleLaunchKernel(c->f_enc01, gx, (unsigned)batch, 1, 256, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipModuleLaunchKernel(enc0 + enc1): %s", hipGetErrorString(e));
    return PRISM_OK;
}

/* enc2 and enc3 as one launch (prism_codec_enc23): CODEC_ENC23_ROWS x
 * CODEC_ENC23_COLS blocks of the bottleneck, each with the e2 region and the
 * e1 window under it; writes the e2 map and the bottleneck. 8 waves. */
int launch_enc23(prism_ctx* c, const uint16_t* e1, uint16_t* e2, uint16_t* bottleneck, int batch, hipStream_t s) {
    CodecArgs a2 = stage_args(c, ST_ENC2, e1, nullptr, e2);
    CodecArgs a3 = stage_args(c, ST_ENC3, nullptr, nullptr, bottleneck);
    const unsigned gx = (unsigned)(((a3.out_w + CODEC_ENC23_COLS - 1) / CODEC_ENC23_COLS) *
                                   ((a3.out_h + CODEC_ENC23_ROWS - 1) / CODEC_ENC23_ROWS));
    void* params[] = {&a2, &a3};
    const hipError_t e = hipModuleLaunchKernel(c->f_enc23, gx, (unsigned)batch, 1, 512, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipModuleLaunchKernel(enc2 + enc3): %s", hipGetErrorString(e));
    return PRISM_OK;
}

int codec_enqueue_encode(prism_ctx* c, const uint16_t* frame, uint16_t* bottleneck, int batch, hipStream_t s) {
    int rc = launch_enc01(c, frame, c->ce0, c->ce1, batch, s);
    if (!rc) rc = launch_enc23(c, c->ce1, c->ce2, bottleneck, batch, s);
    return rc;
}

int codec_enqueue_decode(prism_ctx* c, const uint16_t* bottleneck, uint16_t* display, int batch, hipStream_t s) {
    int rc = launch_stage(c, ST_DEC3, bottleneck, c->ce2, c->cd3, batch, s);
    if (!rc) rc = launch_dec21(c, c->cd3, c->ce1, c->ce0, display, batch, s);
    return rc;
}

extern "C" int prism_load_codec(prism_ctx* c, const void* blob, size_t bytes, const prism_codec_offsets* o) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->loaded) return fail(c, PRISM_ERR_STATE, "load the model weights before the encoder / decoder");
    if (!blob || !o || bytes % 2) return fail(c, PRISM_ERR_INVALID, "blob / offsets NULL or odd byte count");
    std::string why;
    const int v = validate_codec(&c->desc, o, (int64_t)(bytes / 2), &why);
    if (v) return fail(c, v, "%s", why.c_str());
    int rw[4], rh[4];
    (void)codec_resolutions(&c->desc, o->render_w, o->render_h, rw, rh, nullptr);
    const uint16_t* w = static_cast<const uint16_t*>(blob);

    std::vector<uint16_t> packed[8];
    const auto id = [](int j) { return j; };
    /* enc0: packed column tap*16 + ic (9 taps x 16, 160 columns; ic >= 9 and
     * tap 9 are zero) <- stored column ic*9 + tap */
    pack_mapped(w + o->enc0_w, 32, 81, 32, 160,
                [](int j) { const int tap = j / 16, ic = j % 16; return tap < 9 && ic < 9 ? ic * 9 + tap : -1; },
                packed[0]);
    /* enc1..3: packed column tap*Cin + ic <- stored column ic*9 + tap */
    const int cins[3] = {32, 64, 128}, couts[3] = {64, 128, 128};
    const int64_t encw[3] = {o->enc1_w, o->enc2_w, o->enc3_w};
    for (int i = 0; i < 3; ++i) {
        const int cin = cins[i];
        pack_mapped(w + encw[i], couts[i], 9 * cin, couts[i], 9 * cin,
                    [cin](int j) { return (j % cin) * 9 + j / cin; }, packed[1 + i]);
    }
    pack_mapped(w + o->dec3_w, 128, 256, 128, 256, id, packed[4]);
    pack_mapped(w + o->dec2_w, 64, 192, 64, 192, id, packed[5]);
    pack_mapped(w + o->dec1_w, 32, 96, 32, 96, id, packed[6]);
    /* output conv: lane (g, row) element j of the A fragment must hold the
     * column of dec1 channel 16*(j/4) + 4g + j%4, the channel that element j of
     * the fused kernel's B fragment (dec1's accumulator lane) carries */
    pack_mapped(w + o->out_w, 12, 32, 16, 32,
                [](int j) { const int g = j / 8, e = j % 8; return 16 * (e / 4) + 4 * g + e % 4; }, packed[7]);

    const int64_t boff[8] = {o->enc0_b, o->enc1_b, o->enc2_b, o->enc3_b, o->dec3_b, o->dec2_b, o->dec1_b, o->out_b};
    const int bn[8] = {32, 64, 128, 128, 128, 64, 32, 12};
    const int bpad[8] = {32, 64, 128, 128, 128, 64, 32, 16};
    std::vector<float> bias[8];
    for (int i = 0; i < 8; ++i) {
        bias[i].assign(bpad[i], 0.f);
        for (int k = 0; k < bn[i]; ++k) bias[i][k] = half_to_float(w[boff[i] + k]);
    }
    size_t woff[8], bo[8], total = 0;
    for (int i = 0; i < 8; ++i) {
        woff[i] = total;
        total += round256(packed[i].size() * 2);
        bo[i] = total;
        total += round256(bias[i].size() * 4);
    }
    HIP_TRY(c, hipSetDevice(c->device));
    void* arena = nullptr;
    hipError_t e = hipMalloc(&arena, total);
    if (e != hipSuccess) return fail(c, PRISM_ERR_NOMEM, "hipMalloc(%zu) for the codec weights: %s", total, hipGetErrorString(e));
    uint8_t* a = static_cast<uint8_t*>(arena);
    for (int i = 0; i < 8 && e == hipSuccess; ++i) {
        e = hipMemcpy(a + woff[i], packed[i].data(), packed[i].size() * 2, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(a + bo[i], bias[i].data(), bias[i].size() * 4, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        (void)hipFree(arena);
        return fail(c, PRISM_ERR_HIP, "hipMemcpy codec weights: %s", hipGetErrorString(e));
    }
    codec_release(c);
    c->carena = arena;
    for (int i = 0; i < 8; ++i) {
        c->cw[i] = reinterpret_cast<const uint16_t*>(a + woff[i]);
        c->cb[i] = reinterpret_cast<const float*>(a + bo[i]);
    }
    for (int i = 0; i < 4; ++i) {
        c->cr_w[i] = rw[i];
        c->cr_h[i] = rh[i];
    }
    c->coffs = *o;
    c->codec = true;
    return PRISM_OK;
}

extern "C" int prism_codec_stage(prism_ctx* c, int32_t stage, const void* in, const void* skip, void* out,
                                 int32_t batch, void* stream) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (stage < 0 || stage >= N_STAGES) return fail(c, PRISM_ERR_INVALID, "codec stage %d (0..6)", stage);
    const bool dec = stage >= ST_DEC3;
    if (!in || !out || (dec && !skip)) return fail(c, PRISM_ERR_INVALID, "codec stage %d: NULL buffer", stage);
    if (!aligned16(in) || !aligned16(out) || (dec && !aligned16(skip)))
        return fail(c, PRISM_ERR_INVALID, "codec buffers must be 16-byte aligned");
    if (batch < 1 || batch > 65535) return fail(c, PRISM_ERR_INVALID, "batch %d", batch);
    HIP_TRY(c, hipSetDevice(c->device));
    return launch_stage(c, stage, static_cast<const uint16_t*>(in), dec ? static_cast<const uint16_t*>(skip) : nullptr,
                        static_cast<uint16_t*>(out), batch, (hipStream_t)stream);
}

extern "C" int prism_encode(prism_ctx* c, const void* frame, void* bottleneck, int32_t batch, void* stream) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!frame || !bottleneck) return fail(c, PRISM_ERR_INVALID, "frame or bottleneck is NULL");
    if (!aligned16(frame) || !aligned16(bottleneck)) return fail(c, PRISM_ERR_INVALID, "buffers must be 16-byte aligned");
    if (batch < 1 || batch > 65535) return fail(c, PRISM_ERR_INVALID, "batch %d", batch);
    HIP_TRY(c, hipSetDevice(c->device));
    rc = codec_ensure_workspace(c, batch);
    if (rc) return rc;
    return codec_enqueue_encode(c, static_cast<const uint16_t*>(frame), static_cast<uint16_t*>(bottleneck), batch,
                                (hipStream_t)stream);
}

extern "C" int prism_decode(prism_ctx* c, const void* bottleneck, void* display, int32_t batch, void* stream) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!bottleneck || !display) return fail(c, PRISM_ERR_INVALID, "bottleneck or display is NULL");
    if (!aligned16(bottleneck) || !aligned16(display)) return fail(c, PRISM_ERR_INVALID, "buffers must be 16-byte aligned");
    if (batch < 1) return fail(c, PRISM_ERR_INVALID, "batch %d", batch);
    if (!c->cws || c->cws_batch < batch)
        return fail(c, PRISM_ERR_STATE, "no encoder maps for %d frames (prism_encode first)", batch);
    HIP_TRY(c, hipSetDevice(c->device));
    return codec_enqueue_decode(c, static_cast<const uint16_t*>(bottleneck), static_cast<uint16_t*>(display), batch,
                                (hipStream_t)stream);
}
