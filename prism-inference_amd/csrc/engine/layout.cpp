/*
 * layout.cpp - blob layout, validation, MFMA fragment packing (host only).
 *
 * The blob layout is the reference MoE bench's bump allocator
 * (vulkan_engine/prism_moe_bench.cpp:164-172: qkv_w, qkv_b, out_w, out_b,
 * [ffn], rtr_w, rtr_b, then experts e0..eN-1 as {w1, b1, w2, b2} at a fixed
 * stride) with three changes: the LayerNorm tensors are added (LN1 before
 * qkv_w, LN2 before the router), every block gets its own tensors instead of
 * reusing block 0's, and each tensor starts on an 8-element (16-byte)
 * boundary so the loader can use 16-byte loads.
 */
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "engine_internal.h"

namespace prism {

static int64_t bump(int64_t& cur, int64_t n) {
    const int64_t o = cur;
    cur += (n + 7) & ~int64_t(7);
    return o;
}

bool shape_supported(const prism_model_desc* d, std::string* why) {
    char buf[256];
    if (!d) { if (why) *why = "model description is NULL"; return false; }
    const bool s256 = d->dim == 256 && d->n_heads == 8 && d->head_dim == 32;
    const bool s128 = d->dim == 128 && d->n_heads == 8 && d->head_dim == 16;
    if (!s256 && !s128) {
        snprintf(buf, sizeof buf, "unsupported shape dim=%d heads=%d head_dim=%d (supported: 256/8x32, 128/8x16)",
                 d->dim, d->n_heads, d->head_dim);
        if (why) *why = buf;
        return false;
    }
    if (d->window != 8) {
        snprintf(buf, sizeof buf, "unsupported window %d (supported: 8)", d->window);
        if (why) *why = buf;
        return false;
    }
    if (d->n_experts < 1 || d->n_experts > 64) {
        snprintf(buf, sizeof buf, "n_experts %d out of range [1, 64]", d->n_experts);
        if (why) *why = buf;
        return false;
    }
    if (d->n_blocks < 1 || d->n_blocks > 4096) {
        snprintf(buf, sizeof buf, "n_blocks %d out of range [1, 4096]", d->n_blocks);
        if (why) *why = buf;
        return false;
    }
    if (d->spatial_h < 1 || d->spatial_w < 1 || (int64_t)d->spatial_h * d->spatial_w > (1 << 24) ||
        (int64_t)d->spatial_h * d->spatial_w * d->dim * 2 > 0xffffffffll) { /* a frame's rows under 4 GiB */
        snprintf(buf, sizeof buf, "token grid %dx%d out of range", d->spatial_h, d->spatial_w);
        if (why) *why = buf;
        return false;
    }
    return true;
}

int64_t layout_blocks(const prism_model_desc* d, prism_block_offsets* offs) {
    const int64_t D = d->dim, N = d->n_experts;
    int64_t cur = 0;
    for (int b = 0; b < d->n_blocks; ++b) {
        prism_block_offsets o;
        o.ln1_g = bump(cur, D);
        o.ln1_b = bump(cur, D);
        o.qkv_w = bump(cur, 3 * D * D);
        o.qkv_b = bump(cur, 3 * D);
        o.out_w = bump(cur, D * D);
        o.out_b = bump(cur, D);
        o.ln2_g = bump(cur, D);
        o.ln2_b = bump(cur, D);
        if (N > 1) {
            o.router_w = bump(cur, N * D);
            o.router_b = bump(cur, N);
        } else {
            o.router_w = o.router_b = -1;
        }
        o.exp_stride = 2 * D * D + 2 * D;
        o.exp_w1 = cur;
        o.exp_b1 = cur + D * D;
        o.exp_w2 = cur + D * D + D;
        o.exp_b2 = cur + 2 * D * D + D;
        cur += N * o.exp_stride;
        if (offs) offs[b] = o;
    }
    return cur;
}

static bool span_ok(int64_t off, int64_t n, int64_t total) {
    return off >= 0 && (off & 7) == 0 && n >= 0 && off <= total && n <= total - off;
}

int validate_blocks(const prism_model_desc* d, const prism_block_offsets* offs, int64_t total,
                    std::string* why) {
    if (!shape_supported(d, why)) return PRISM_ERR_UNSUPPORTED;
    if (!offs) { if (why) *why = "offset table is NULL"; return PRISM_ERR_INVALID; }
    if (total < 0) { if (why) *why = "negative blob size"; return PRISM_ERR_BLOB; }
    const int64_t D = d->dim, N = d->n_experts;
    char buf[256];
    for (int b = 0; b < d->n_blocks; ++b) {
        const prism_block_offsets& o = offs[b];
        struct { const char* name; int64_t off, n; } t[] = {
            {"ln1_g", o.ln1_g, D}, {"ln1_b", o.ln1_b, D}, {"qkv_w", o.qkv_w, 3 * D * D},
            {"qkv_b", o.qkv_b, 3 * D}, {"out_w", o.out_w, D * D}, {"out_b", o.out_b, D},
            {"ln2_g", o.ln2_g, D}, {"ln2_b", o.ln2_b, D},
            {"router_w", o.router_w, N > 1 ? N * D : 0}, {"router_b", o.router_b, N > 1 ? N : 0},
        };
        for (auto& x : t) {
            if (x.n == 0) continue;
            if (!span_ok(x.off, x.n, total)) {
                snprintf(buf, sizeof buf, "block %d: %s [%lld, +%lld) outside the blob (%lld elems) or not 8-aligned",
                         b, x.name, (long long)x.off, (long long)x.n, (long long)total);
                if (why) *why = buf;
                return PRISM_ERR_BLOB;
            }
        }
        if (o.exp_stride < 0 || (o.exp_stride & 7) || (N > 1 && o.exp_stride == 0)) {
            snprintf(buf, sizeof buf, "block %d: bad expert stride %lld", b, (long long)o.exp_stride);
            if (why) *why = buf;
            return PRISM_ERR_BLOB;
        }
        for (int64_t e : {int64_t(0), N - 1}) {
            const int64_t eo = e * o.exp_stride;
            struct { const char* name; int64_t off, n; } u[] = {
                {"exp_w1", o.exp_w1 + eo, D * D}, {"exp_b1", o.exp_b1 + eo, D},
                {"exp_w2", o.exp_w2 + eo, D * D}, {"exp_b2", o.exp_b2 + eo, D},
            };
            for (auto& x : u) {
                if (!span_ok(x.off, x.n, total)) {
                    snprintf(buf, sizeof buf, "block %d expert %lld: %s outside the blob or not 8-aligned", b,
                             (long long)e, x.name);
                    if (why) *why = buf;
                    return PRISM_ERR_BLOB;
                }
            }
        }
    }
    return PRISM_OK;
}

int validate_adapters(const prism_model_desc* d, const prism_adapter_offsets* a, int64_t total,
                      std::string* why) {
    if (!shape_supported(d, why)) return PRISM_ERR_UNSUPPORTED;
    if (!a) { if (why) *why = "adapter offsets are NULL"; return PRISM_ERR_INVALID; }
    if (a->in_dim != 128) {
        if (why) *why = "adapter in_dim " + std::to_string(a->in_dim) + " (supported: 128)";
        return PRISM_ERR_UNSUPPORTED;
    }
    const int64_t D = d->dim, I = a->in_dim;
    struct { const char* name; int64_t off, n; } t[] = {
        {"up_w", a->up_w, D * I}, {"up_b", a->up_b, D}, {"down_w", a->down_w, I * D}, {"down_b", a->down_b, I},
    };
    for (auto& x : t) {
        if (!span_ok(x.off, x.n, total)) {
            if (why) *why = std::string("adapter ") + x.name + " outside the blob or not 8-aligned";
            return PRISM_ERR_BLOB;
        }
    }
    return PRISM_OK;
}

void pack_fragments(const uint16_t* W, int rows, int K, int rows_padded, uint16_t* dst) {
    const int KS = K / 32;
    for (int rt = 0; rt < rows_padded / 16; ++rt)
        for (int ks = 0; ks < KS; ++ks)
            for (int l = 0; l < 64; ++l) {
                const int r = 16 * rt + (l & 15);
                const int k0 = 32 * ks + 8 * (l >> 4);
                uint16_t* d = dst + ((size_t)(rt * KS + ks) * 64 + l) * 8;
                if (r < rows)
                    memcpy(d, W + (size_t)r * K + k0, 16);
                else
                    memset(d, 0, 16);
            }
}

bool fold_layernorm(const uint16_t* W, int rows, int K, const uint16_t* gamma, const uint16_t* beta,
                    const uint16_t* bias, uint16_t* Wf, float* bias_f, std::string* why) {
    std::vector<float> g(K), be(K);
    for (int i = 0; i < K; ++i) {
        g[i] = half_to_float(gamma[i]);
        be[i] = half_to_float(beta[i]);
    }
    for (int o = 0; o < rows; ++o) {
        const uint16_t* wr = W + (size_t)o * K;
        uint16_t* fr = Wf + (size_t)o * K;
        double shift = 0.0;
        for (int i = 0; i < K; ++i) {
            const float w = half_to_float(wr[i]);
            const float p = w * g[i]; /* exact: an fp16 x fp16 product fits fp32 */
            const uint16_t h = float_to_half(p);
            if ((h & 0x7c00) == 0x7c00 && std::isfinite(p)) {
                if (why) *why = "LayerNorm gamma times weight overflows fp16 (row " + std::to_string(o) +
                                ", channel " + std::to_string(i) + ")";
                return false;
            }
            fr[i] = h;
            shift += (double)w * (double)be[i];
        }
        const float b = half_to_float(bias[o]);
        /* beta = 0 leaves the bias bit-identical (also a -0 bias) */
        bias_f[o] = shift == 0.0 ? b : (float)((double)b + shift);
    }
    return true;
}

float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { /* subnormal: renormalise */
            e = 1;
            while (!(m & 0x400)) { m <<= 1; --e; }
            m &= 0x3ff;
            bits = s | ((e + 112) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000;
    const uint32_t absx = x & 0x7fffffff;
    if (absx >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00 | (absx > 0x7f800000u ? 0x200 : 0));
    if (absx >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00);
    if (absx < 0x38800000u) { /* below the smallest normal half: subnormal / zero */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        const uint32_t e = absx >> 23;
        const uint32_t m = (absx & 0x7fffff) | 0x800000;
        const int shift = 126 - (int)e; /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((absx >> 13) - (112u << 10));
    const uint32_t rem = absx & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) ++r;
    return (uint16_t)(sign | r);
}

}  // namespace prism

using namespace prism;

extern "C" int prism_layout(const prism_model_desc* desc, prism_block_offsets* offs, int64_t* total) {
    std::string why;
    if (!shape_supported(desc, &why)) {
        set_global_error(why);
        return PRISM_ERR_UNSUPPORTED;
    }
    const int64_t n = layout_blocks(desc, offs);
    if (total) *total = n;
    return PRISM_OK;
}

extern "C" int prism_adapter_layout(const prism_model_desc* desc, int32_t in_dim, int64_t base,
                                    prism_adapter_offsets* offs, int64_t* end) {
    std::string why;
    if (!shape_supported(desc, &why)) {
        set_global_error(why);
        return PRISM_ERR_UNSUPPORTED;
    }
    if (in_dim != 128 || base < 0 || !offs) {
        set_global_error("prism_adapter_layout: in_dim must be 128, base >= 0, offs non-NULL");
        return PRISM_ERR_INVALID;
    }
    /* proj_up_w, proj_up_b, proj_dn_w, proj_dn_b (prism_moe_bench.cpp:351-352) */
    int64_t cur = (base + 7) & ~int64_t(7);
    const int64_t D = desc->dim;
    offs->in_dim = in_dim;
    offs->pad_ = 0;
    offs->up_w = bump(cur, D * in_dim);
    offs->up_b = bump(cur, D);
    offs->down_w = bump(cur, (int64_t)in_dim * D);
    offs->down_b = bump(cur, in_dim);
    if (end) *end = cur;
    return PRISM_OK;
}

/* Encoder / decoder tensor table: name, offset, element count. */
struct CodecTensor {
    const char* name;
    int64_t off, n;
};

static int codec_tensors(const prism_codec_offsets* c, CodecTensor* t) {
    const CodecTensor v[] = {
        {"enc0_w", c->enc0_w, 32 * 81},   {"enc0_b", c->enc0_b, 32},   {"enc1_w", c->enc1_w, 64 * 288},
        {"enc1_b", c->enc1_b, 64},        {"enc2_w", c->enc2_w, 128 * 576}, {"enc2_b", c->enc2_b, 128},
        {"enc3_w", c->enc3_w, 128 * 1152}, {"enc3_b", c->enc3_b, 128}, {"dec3_w", c->dec3_w, 128 * 256},
        {"dec3_b", c->dec3_b, 128},       {"dec2_w", c->dec2_w, 64 * 192}, {"dec2_b", c->dec2_b, 64},
        {"dec1_w", c->dec1_w, 32 * 96},   {"dec1_b", c->dec1_b, 32},   {"out_w", c->out_w, 12 * 32},
        {"out_b", c->out_b, 12},
    };
    const int n = (int)(sizeof v / sizeof v[0]);
    for (int i = 0; i < n; ++i) t[i] = v[i];
    return n;
}

bool prism::codec_resolutions(const prism_model_desc* d, int render_w, int render_h, int* rw, int* rh,
                              std::string* why) {
    if (render_w < 1 || render_h < 1 || render_w > 16384 || render_h > 16384) {
        if (why) *why = "render size " + std::to_string(render_w) + "x" + std::to_string(render_h) + " out of range";
        return false;
    }
    /* the conv stages address a frame's maps with 32-bit byte offsets; the
     * largest is the 32-channel fp16 map at the render size (64 B a pixel) */
    if ((int64_t)render_w * render_h * 64 > (int64_t)0x7fffffff) {
        if (why)
            *why = "render size " + std::to_string(render_w) + "x" + std::to_string(render_h) +
                   " too large: its 32-channel map exceeds 2 GiB per frame";
        return false;
    }
    rw[0] = render_w;
    rh[0] = render_h;
    for (int i = 1; i < 4; ++i) { /* a 3x3 stride-2 conv with padding 1 */
        rw[i] = (rw[i - 1] + 1) / 2;
        rh[i] = (rh[i - 1] + 1) / 2;
    }
    if (rw[3] != d->spatial_w || rh[3] != d->spatial_h) {
        if (why)
            *why = "render size " + std::to_string(render_w) + "x" + std::to_string(render_h) + " encodes to " +
                   std::to_string(rw[3]) + "x" + std::to_string(rh[3]) + ", the model's token grid is " +
                   std::to_string(d->spatial_w) + "x" + std::to_string(d->spatial_h);
        return false;
    }
    return true;
}

int prism::validate_codec(const prism_model_desc* d, const prism_codec_offsets* c, int64_t total, std::string* why) {
    if (!shape_supported(d, why)) return PRISM_ERR_UNSUPPORTED;
    if (!c) { if (why) *why = "codec offsets are NULL"; return PRISM_ERR_INVALID; }
    if (c->in_channels != 9 || c->scale != 2) {
        if (why)
            *why = "codec in_channels " + std::to_string(c->in_channels) + ", scale " + std::to_string(c->scale) +
                   " (supported: 9 and 2)";
        return PRISM_ERR_UNSUPPORTED;
    }
    int rw[4], rh[4];
    if (!codec_resolutions(d, c->render_w, c->render_h, rw, rh, why)) return PRISM_ERR_INVALID;
    CodecTensor t[16];
    const int n = codec_tensors(c, t);
    for (int i = 0; i < n; ++i)
        if (!span_ok(t[i].off, t[i].n, total)) {
            if (why) *why = std::string("codec ") + t[i].name + " outside the blob or not 8-aligned";
            return PRISM_ERR_BLOB;
        }
    return PRISM_OK;
}

extern "C" int prism_codec_layout(const prism_model_desc* desc, int32_t render_w, int32_t render_h, int64_t base,
                                  prism_codec_offsets* c, prism_adapter_offsets* ad, int64_t* end) {
    std::string why;
    if (!shape_supported(desc, &why)) {
        set_global_error(why);
        return PRISM_ERR_UNSUPPORTED;
    }
    int rw[4], rh[4];
    if (!c || base < 0) {
        set_global_error("prism_codec_layout: codec offsets NULL or base < 0");
        return PRISM_ERR_INVALID;
    }
    if (!codec_resolutions(desc, render_w, render_h, rw, rh, &why)) {
        set_global_error(why);
        return PRISM_ERR_INVALID;
    }
    /* enc_ic, enc1, enc2, enc3, proj_up, proj_dn, d3_pw, d2_pw, d1_pw, out_pw
     * (prism_moe_bench.cpp:347-357) */
    int64_t cur = (base + 7) & ~int64_t(7);
    const int64_t D = desc->dim, I = 128;
    c->render_w = render_w;
    c->render_h = render_h;
    c->in_channels = 9;
    c->scale = 2;
    c->enc0_w = bump(cur, 32 * 81);
    c->enc0_b = bump(cur, 32);
    c->enc1_w = bump(cur, 64 * 288);
    c->enc1_b = bump(cur, 64);
    c->enc2_w = bump(cur, 128 * 576);
    c->enc2_b = bump(cur, 128);
    c->enc3_w = bump(cur, 128 * 1152);
    c->enc3_b = bump(cur, 128);
    prism_adapter_offsets a{};
    a.in_dim = (int32_t)I;
    a.up_w = bump(cur, D * I);
    a.up_b = bump(cur, D);
    a.down_w = bump(cur, I * D);
    a.down_b = bump(cur, I);
    if (ad) *ad = a;
    c->dec3_w = bump(cur, 128 * 256);
    c->dec3_b = bump(cur, 128);
    c->dec2_w = bump(cur, 64 * 192);
    c->dec2_b = bump(cur, 64);
    c->dec1_w = bump(cur, 32 * 96);
    c->dec1_b = bump(cur, 32);
    c->out_w = bump(cur, 12 * 32);
    c->out_b = bump(cur, 12);
    if (end) *end = cur;
    return PRISM_OK;
}

extern "C" int prism_validate(const prism_model_desc* desc, const prism_block_offsets* offs,
                              int64_t blob_elems) {
    std::string why;
    const int rc = validate_blocks(desc, offs, blob_elems, &why);
    if (rc) set_global_error(why);
    return rc;
}

extern "C" int prism_pack_weight(const uint16_t* w, int32_t rows, int32_t k, int32_t rows_padded,
                                 uint16_t* dst) {
    if (!w || !dst || rows < 0 || k <= 0 || k % 32 || rows_padded < rows || rows_padded % 16) {
        set_global_error("prism_pack_weight: bad arguments");
        return PRISM_ERR_INVALID;
    }
    pack_fragments(w, rows, k, rows_padded, dst);
    return PRISM_OK;
}

extern "C" int64_t prism_aux_elems(int32_t n_experts, int64_t tokens) {
    if (n_experts < 1 || tokens < 0) return -1;
    return tokens + n_experts + (int64_t)n_experts * tokens;
}

extern "C" int prism_histogram(const int32_t* assign, int64_t n, int32_t n_experts, int64_t* counts) {
    if (!assign || !counts || n < 0 || n_experts < 1) return PRISM_ERR_INVALID;
    for (int e = 0; e < n_experts; ++e) counts[e] = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t e = assign[i];
        if (e < 0 || e >= n_experts) return PRISM_ERR_INVALID;
        counts[e]++;
    }
    return PRISM_OK;
}
