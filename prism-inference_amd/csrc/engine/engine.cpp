/*
 * engine.cpp - host engine: code object, weights, per-stage launches, block
 * chain and its hipGraph.
 *
 * Mirrors the reference's engine surface (vulkan_engine/prism_vulkan.h:73-117:
 * Init / LoadWeights / RecordCommandBuffer / InferGPU) and the MoE bench's
 * per-block recording (prism_moe_bench.cpp:262-291): kernels come from one
 * code object (hipModuleLoad, the analogue of loadPipeline(".spv")), each
 * stage is one hipModuleLaunchKernel, and the per-frame block chain is
 * captured once into a hipGraph (the analogue of the once-recorded command
 * buffer that is re-submitted every frame, prism_moe_bench.cpp:183-209).
 */
#include <dlfcn.h>
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "../kernel_args.h"
#include "ctx.h"
#include "engine_internal.h"

namespace prism {

static thread_local std::string g_error;
void set_global_error(const std::string& msg) { g_error = msg; }

}  // namespace prism

using namespace prism;

int fail(prism_ctx* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    g_error = buf;
    return code;
}

static int dim_index(int dim) { return dim == 256 ? 1 : 0; }

static std::string default_code_object() {
    Dl_info info;
    if (dladdr((void*)&prism_create, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        const size_t s = p.find_last_of('/');
        return (s == std::string::npos ? std::string(".") : p.substr(0, s)) + "/prism_kernels.hsaco";
    }
    return "prism_kernels.hsaco";
}

/* ------------------------------------------------------------ lifecycle */

extern "C" int prism_create(prism_ctx** out, int32_t device, const char* code_object_path) {
    if (!out) return fail(nullptr, PRISM_ERR_INVALID, "prism_create: out is NULL");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return fail(nullptr, PRISM_ERR_HIP, "no HIP device available (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n)
        return fail(nullptr, PRISM_ERR_INVALID, "device %d out of range (%d devices)", device, n);
    const std::string path = code_object_path ? std::string(code_object_path) : default_code_object();
    {
        std::ifstream f(path, std::ios::binary);
        if (!f.good()) return fail(nullptr, PRISM_ERR_CODE_OBJECT, "code object not found: %s", path.c_str());
    }
    prism_ctx* c = new prism_ctx();
    c->device = device;
    e = hipSetDevice(device);
    if (e != hipSuccess) {
        delete c;
        return fail(nullptr, PRISM_ERR_HIP, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
    }
    /* this device's allocation-free workspace (prism_forward_noalloc) */
    e = scratch_device_address(device, &c->scratch);
    if (e != hipSuccess) {
        delete c;
        return fail(nullptr, PRISM_ERR_HIP, "device address of the scratch array on device %d: %s", device,
                    hipGetErrorString(e));
    }
    e = hipModuleLoad(&c->module, path.c_str());
    if (e != hipSuccess) {
        delete c;
        return fail(nullptr, PRISM_ERR_CODE_OBJECT, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    }
    struct { hipFunction_t* f; const char* name; } fns[] = {
        {&c->f_router[0][0], "prism_router_d128_n1"}, {&c->f_router[0][1], "prism_router_d128_n2"},
        {&c->f_router[0][2], "prism_router_d128_n3"}, {&c->f_router[0][3], "prism_router_d128_n4"},
        {&c->f_router[1][0], "prism_router_d256_n1"}, {&c->f_router[1][1], "prism_router_d256_n2"},
        {&c->f_router[1][2], "prism_router_d256_n3"}, {&c->f_router[1][3], "prism_router_d256_n4"},
        {&c->f_expert[0][0], "prism_expert_d128_bm64"},  {&c->f_expert[1][0], "prism_expert_d256_bm64"},
        {&c->f_expert[0][1], "prism_expert_d128_bm64_w8"}, {&c->f_expert[1][1], "prism_expert_d256_bm64_w8"},
        {&c->f_expert_wide, "prism_expert_d256_bm128"}, {&c->f_expert_wide96, "prism_expert_d256_bm96"},
        {&c->f_zero, "prism_zero_i32"}, {&c->f_take, "prism_take_counts"},
        {&c->f_proj[0][0], "prism_project_up_d128"},   {&c->f_proj[0][1], "prism_project_down_d128"},
        {&c->f_proj[1][0], "prism_project_up_d256"},   {&c->f_proj[1][1], "prism_project_down_d256"},
        {&c->f_codec[0], "prism_codec_enc0"}, {&c->f_codec[1], "prism_codec_enc1"},
        {&c->f_codec[2], "prism_codec_enc2"}, {&c->f_codec[3], "prism_codec_enc3"},
        {&c->f_codec[4], "prism_codec_dec3"}, {&c->f_codec[5], "prism_codec_dec2"},
        {&c->f_codec[6], "prism_codec_dec1_out"}, {&c->f_codec21, "prism_codec_dec21_out"},
        {&c->f_enc01, "prism_codec_enc01"},   {&c->f_enc23, "prism_codec_enc23"},
        {&c->f_attn_ffn[0][0], "prism_attn_d128_ffn"}, {&c->f_attn_ffn[0][1], "prism_attn_d128_w8_ffn"},
        {&c->f_attn_ffn[1][0], "prism_attn_d256_ffn"}, {&c->f_attn_ffn[1][1], "prism_attn_d256_w8_ffn"},
    };
    std::vector<std::pair<hipFunction_t*, std::string>> all;
    for (auto& f : fns) all.emplace_back(f.f, f.name);
    for (int di = 0; di < 2; ++di)
        for (int w8 = 0; w8 < 2; ++w8)
            for (int r = 0; r <= 4; ++r)
                all.emplace_back(&c->f_attn[di][w8][r], std::string("prism_attn_d") + (di ? "256" : "128") +
                                                            (w8 ? "_w8" : "") + (r ? "_r" + std::to_string(r) : ""));
    for (auto& f : all) {
        e = hipModuleGetFunction(f.first, c->module, f.second.c_str());
        if (e != hipSuccess) {
            (void)hipModuleUnload(c->module);
            delete c;
            return fail(nullptr, PRISM_ERR_CODE_OBJECT, "kernel %s missing from %s: %s", f.second.c_str(), path.c_str(),
                        hipGetErrorString(e));
        }
    }
    e = hipStreamCreateWithFlags(&c->cap_stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreate(&c->ev_t0);
    if (e == hipSuccess) e = hipEventCreate(&c->ev_t1);
    for (int j = 0; j + 1 < CHAIN_SPLIT && e == hipSuccess; ++j) {
        e = hipStreamCreateWithFlags(&c->sub_stream[j], hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&c->ev_join[j], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        for (int j = 0; j + 1 < CHAIN_SPLIT; ++j) {
            if (c->ev_join[j]) (void)hipEventDestroy(c->ev_join[j]);
            if (c->sub_stream[j]) (void)hipStreamDestroy(c->sub_stream[j]);
        }
        if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
        if (c->ev_t0) (void)hipEventDestroy(c->ev_t0);
        if (c->ev_t1) (void)hipEventDestroy(c->ev_t1);
        if (c->cap_stream) (void)hipStreamDestroy(c->cap_stream);
        (void)hipModuleUnload(c->module);
        delete c;
        return fail(nullptr, PRISM_ERR_HIP, "hipStreamCreate / hipEventCreate: %s", hipGetErrorString(e));
    }
    *out = c;
    return PRISM_OK;
}

void drop_graph(prism_ctx* c) {
    if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->gexec = nullptr;
    c->graph = nullptr;
    c->g_in = nullptr;
    c->g_out = nullptr;
    c->g_batch = 0;
    c->g_mode = CHAIN_BLOCKS;
}

static void drop_adapters(prism_ctx* c) {
    if (c->aarena) (void)hipFree(c->aarena);
    c->aarena = nullptr;
    c->adapters = false;
    c->up_w = c->down_w = nullptr;
    c->up_b = c->down_b = nullptr;
}

static void drop_workspace(prism_ctx* c) {
    if (c->ws) (void)hipFree(c->ws);
    if (c->fwd_assign == c->wsb.assign) c->fwd_assign = nullptr;
    c->ws = nullptr;
    c->wsb = ChainWs{};
    c->ws_batch = 0;
    c->ws_tokens = 0;
}

extern "C" void prism_destroy(prism_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipDeviceSynchronize();
    drop_graph(c);
    drop_workspace(c);
    drop_adapters(c);
    codec_release(c);
    if (c->warena) (void)hipFree(c->warena);
    for (int j = 0; j + 1 < CHAIN_SPLIT; ++j) {
        if (c->ev_join[j]) (void)hipEventDestroy(c->ev_join[j]);
        if (c->sub_stream[j]) (void)hipStreamDestroy(c->sub_stream[j]);
    }
    if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
    if (c->ev_t0) (void)hipEventDestroy(c->ev_t0);
    if (c->ev_t1) (void)hipEventDestroy(c->ev_t1);
    if (c->stage_counts) (void)hipFree(c->stage_counts);
    if (c->cap_stream) (void)hipStreamDestroy(c->cap_stream);
    if (c->module) (void)hipModuleUnload(c->module);
    delete c;
}

extern "C" const char* prism_last_error(const prism_ctx* c) { return c ? c->err.c_str() : g_error.c_str(); }

/* ------------------------------------------------------------ weights */

namespace {

struct Arena {
    size_t off = 0;
    size_t take(size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) & ~size_t(255);
        return o;
    }
};

struct BlockPlan {
    size_t wqkv, bqkv, bqkv_pad, wo, bo, wr, br, w1, b1, w2, b2;
};

inline int round16(int n) { return (n + 15) & ~15; }

/* Tokens in one launch: the counting sort's int32 slots, and the kernels
 * address a launch's rows with 32-bit byte offsets (as the reference's
 * shaders do), so its activations stay under 4 GiB. */
inline bool tokens_fit(int64_t n, int dim) { return n <= 0x7fffffff / 64 && n * dim * 2 <= 0xffffffffll; }

}  // namespace

extern "C" int prism_load_weights(prism_ctx* c, const prism_model_desc* d, const void* blob, size_t bytes,
                                  const prism_block_offsets* offs) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!blob) return fail(c, PRISM_ERR_INVALID, "weight blob is NULL");
    if (bytes % 2) return fail(c, PRISM_ERR_BLOB, "blob size %zu is not a whole number of fp16 values", bytes);
    std::string why;
    const int rc = validate_blocks(d, offs, (int64_t)(bytes / 2), &why);
    if (rc) return fail(c, rc, "%s", why.c_str());
    HIP_TRY(c, hipSetDevice(c->device));

    const int D = d->dim, N = d->n_experts, NP = N > 1 ? round16(N) : 0;
    const uint16_t* src = static_cast<const uint16_t*>(blob);
    Arena ar;
    std::vector<BlockPlan> plan(d->n_blocks);
    for (int b = 0; b < d->n_blocks; ++b) {
        BlockPlan& p = plan[b];
        p.wqkv = ar.take(3ull * D * D * 2);
        p.bqkv = ar.take(3ull * D * 4);
        p.bqkv_pad = ar.take(3ull * D * 4);
        p.wo = ar.take(1ull * D * D * 2);
        p.bo = ar.take(D * 4);
        p.wr = ar.take((size_t)NP * D * 2);
        p.br = ar.take((size_t)NP * 4);
        p.w1 = ar.take((size_t)N * D * D * 2);
        p.b1 = ar.take((size_t)N * D * 4);
        p.w2 = ar.take((size_t)N * D * D * 2);
        p.b2 = ar.take((size_t)N * D * 4);
    }
    std::vector<uint8_t> host;
    try {
        host.assign(ar.off, 0);
    } catch (...) {
        return fail(c, PRISM_ERR_NOMEM, "cannot allocate %zu bytes of host staging", ar.off);
    }
    auto f32 = [&](size_t at, const uint16_t* s, int n) {
        float* dst = reinterpret_cast<float*>(host.data() + at);
        for (int i = 0; i < n; ++i) dst[i] = half_to_float(s[i]);
    };
    /* Each LayerNorm's affine goes into the weights that consume its output
     * (LN1 -> W_qkv, LN2 -> W_r and every expert's W1): the kernels then only
     * normalise, z = (x - mean) * inv, and W' = r16(W diag(gamma)),
     * b' = b + W beta. With gamma = 1, beta = 0 the packed weights and biases
     * are the blob's own values. */
    std::vector<uint16_t> fw((size_t)3 * D * D);
    auto fold_pack = [&](int64_t w, int rows, int rows_padded, int64_t gam, int64_t bet, int64_t bias, size_t dst_w,
                         size_t dst_b, std::string* why) {
        if (!fold_layernorm(src + w, rows, D, src + gam, src + bet, src + bias, fw.data(),
                            reinterpret_cast<float*>(host.data() + dst_b), why))
            return false;
        pack_fragments(fw.data(), rows, D, rows_padded, reinterpret_cast<uint16_t*>(host.data() + dst_w));
        return true;
    };
    for (int b = 0; b < d->n_blocks; ++b) {
        const BlockPlan& p = plan[b];
        const prism_block_offsets& o = offs[b];
        bool ok = fold_pack(o.qkv_w, 3 * D, 3 * D, o.ln1_g, o.ln1_b, o.qkv_b, p.wqkv, p.bqkv, &why);
        f32(p.bqkv_pad, src + o.qkv_b, 3 * D); /* a padded slot's zero vector meets no beta */
        pack_fragments(src + o.out_w, D, D, D, reinterpret_cast<uint16_t*>(host.data() + p.wo));
        f32(p.bo, src + o.out_b, D);
        if (ok && N > 1) {
            ok = fold_pack(o.router_w, N, NP, o.ln2_g, o.ln2_b, o.router_b, p.wr, p.br, &why);
            float* br = reinterpret_cast<float*>(host.data() + p.br);
            for (int e = N; e < NP; ++e) br[e] = -INFINITY;
        }
        for (int e = 0; ok && e < N; ++e) {
            const int64_t eo = (int64_t)e * o.exp_stride;
            ok = fold_pack(o.exp_w1 + eo, D, D, o.ln2_g, o.ln2_b, o.exp_b1 + eo, p.w1 + (size_t)e * D * D * 2,
                           p.b1 + (size_t)e * D * 4, &why);
            pack_fragments(src + o.exp_w2 + eo, D, D, D,
                           reinterpret_cast<uint16_t*>(host.data() + p.w2) + (size_t)e * D * D);
            f32(p.b2 + (size_t)e * D * 4, src + o.exp_b2 + eo, D);
        }
        if (!ok) return fail(c, PRISM_ERR_BLOB, "block %d: %s", b, why.c_str());
    }

    (void)hipDeviceSynchronize();
    drop_graph(c);
    /* the last forward's assignments belong to the weights being replaced */
    c->fwd_assign = nullptr;
    c->fwd_tokens = 0;
    if (c->warena) {
        (void)hipFree(c->warena);
        c->warena = nullptr;
    }
    c->loaded = false;
    void* arena = nullptr;
    hipError_t e = hipMalloc(&arena, ar.off);
    if (e != hipSuccess) return fail(c, PRISM_ERR_NOMEM, "hipMalloc(%zu) for weights: %s", ar.off, hipGetErrorString(e));
    e = hipMemcpy(arena, host.data(), ar.off, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(arena);
        return fail(c, PRISM_ERR_HIP, "weight upload: %s", hipGetErrorString(e));
    }
    c->warena = arena;
    c->blocks.assign(d->n_blocks, DevBlock{});
    uint8_t* base = static_cast<uint8_t*>(arena);
    for (int b = 0; b < d->n_blocks; ++b) {
        const BlockPlan& p = plan[b];
        DevBlock& k = c->blocks[b];
        k.offs = offs[b];
        k.wqkv = reinterpret_cast<uint16_t*>(base + p.wqkv);
        k.bqkv = reinterpret_cast<float*>(base + p.bqkv);
        /* with LN1 beta = 0 the folded bias is the blob's: padded slots need nothing else */
        bool beta1 = false;
        for (int i = 0; i < D && !beta1; ++i) beta1 = (src[offs[b].ln1_b + i] & 0x7fff) != 0;
        k.bqkv_pad = beta1 ? reinterpret_cast<float*>(base + p.bqkv_pad) : nullptr;
        k.wo = reinterpret_cast<uint16_t*>(base + p.wo);
        k.bo = reinterpret_cast<float*>(base + p.bo);
        k.wr = N > 1 ? reinterpret_cast<uint16_t*>(base + p.wr) : nullptr;
        k.br = N > 1 ? reinterpret_cast<float*>(base + p.br) : nullptr;
        k.w1 = reinterpret_cast<uint16_t*>(base + p.w1);
        k.b1 = reinterpret_cast<float*>(base + p.b1);
        k.w2 = reinterpret_cast<uint16_t*>(base + p.w2);
        k.b2 = reinterpret_cast<float*>(base + p.b2);
    }
    if (c->desc.n_experts != d->n_experts || c->desc.dim != d->dim || c->desc.n_blocks != d->n_blocks ||
        c->desc.spatial_h != d->spatial_h || c->desc.spatial_w != d->spatial_w)
        drop_workspace(c);
    if (c->desc.dim != d->dim) drop_adapters(c);
    if (c->desc.spatial_h != d->spatial_h || c->desc.spatial_w != d->spatial_w) codec_release(c);
    c->desc = *d;
    {
        /* leading blocks whose expert weights the 64-token kernels stream
           past the memory-side cache: enough of them that the rest of the
           arena fits the share it may keep */
        const int64_t excess = (int64_t)ar.off - WEIGHT_CACHE_KEEP;
        const int64_t per_block = (int64_t)d->n_experts * 2 * D * D * 2;
        c->wnt_blocks = excess > 0 ? (int)std::min<int64_t>(d->n_blocks, (excess + per_block - 1) / per_block) : 0;
    }
    c->loaded = true;
    return PRISM_OK;
}

extern "C" int prism_load_weights_file(prism_ctx* c, const prism_model_desc* d, const char* path,
                                       const prism_block_offsets* offs) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!path) return fail(c, PRISM_ERR_INVALID, "path is NULL");
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f.is_open()) return fail(c, PRISM_ERR_INVALID, "cannot open %s", path);
    const std::streamsize size = f.tellg();
    f.seekg(0);
    std::vector<char> data;
    try {
        data.resize((size_t)size);
    } catch (...) {
        return fail(c, PRISM_ERR_NOMEM, "cannot allocate %lld bytes for %s", (long long)size, path);
    }
    if (size > 0 && !f.read(data.data(), size)) return fail(c, PRISM_ERR_INVALID, "short read on %s", path);
    return prism_load_weights(c, d, data.data(), data.size(), offs);
}

extern "C" int prism_load_adapters(prism_ctx* c, const void* blob, size_t bytes, const prism_adapter_offsets* a) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->loaded) return fail(c, PRISM_ERR_STATE, "load the model weights before the adapters");
    if (!blob) return fail(c, PRISM_ERR_INVALID, "adapter blob is NULL");
    if (bytes % 2) return fail(c, PRISM_ERR_BLOB, "blob size %zu is not a whole number of fp16 values", bytes);
    std::string why;
    const int rc = validate_adapters(&c->desc, a, (int64_t)(bytes / 2), &why);
    if (rc) return fail(c, rc, "%s", why.c_str());
    HIP_TRY(c, hipSetDevice(c->device));
    const int D = c->desc.dim, I = a->in_dim;
    const uint16_t* src = static_cast<const uint16_t*>(blob);
    Arena ar;
    const size_t o_uw = ar.take((size_t)D * I * 2), o_ub = ar.take((size_t)D * 4);
    const size_t o_dw = ar.take((size_t)I * D * 2), o_db = ar.take((size_t)I * 4);
    std::vector<uint8_t> host(ar.off, 0);
    pack_fragments(src + a->up_w, D, I, D, reinterpret_cast<uint16_t*>(host.data() + o_uw));
    pack_fragments(src + a->down_w, I, D, I, reinterpret_cast<uint16_t*>(host.data() + o_dw));
    float* ub = reinterpret_cast<float*>(host.data() + o_ub);
    float* db = reinterpret_cast<float*>(host.data() + o_db);
    for (int i = 0; i < D; ++i) ub[i] = half_to_float(src[a->up_b + i]);
    for (int i = 0; i < I; ++i) db[i] = half_to_float(src[a->down_b + i]);

    (void)hipDeviceSynchronize();
    drop_graph(c);
    drop_adapters(c);
    void* arena = nullptr;
    hipError_t e = hipMalloc(&arena, ar.off);
    if (e != hipSuccess) return fail(c, PRISM_ERR_NOMEM, "hipMalloc(%zu) for adapters: %s", ar.off, hipGetErrorString(e));
    e = hipMemcpy(arena, host.data(), ar.off, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(arena);
        return fail(c, PRISM_ERR_HIP, "adapter upload: %s", hipGetErrorString(e));
    }
    uint8_t* b = static_cast<uint8_t*>(arena);
    c->aarena = arena;
    c->up_w = reinterpret_cast<uint16_t*>(b + o_uw);
    c->up_b = reinterpret_cast<float*>(b + o_ub);
    c->down_w = reinterpret_cast<uint16_t*>(b + o_dw);
    c->down_b = reinterpret_cast<float*>(b + o_db);
    c->aoffs = *a;
    c->adapters = true;
    return PRISM_OK;
}

extern "C" int prism_load_model_file(prism_ctx* c, const char* weights_path, const char* json_path) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!weights_path) return fail(c, PRISM_ERR_INVALID, "weights_path is NULL");
    const std::string jp = json_path ? std::string(json_path) : sidecar_path(weights_path);
    std::string text, why;
    if (!read_text_file(jp.c_str(), &text)) return fail(c, PRISM_ERR_INVALID, "cannot read %s", jp.c_str());
    prism_model_desc d{};
    std::vector<prism_block_offsets> offs;
    prism_adapter_offsets ad{};
    bool has_ad = false;
    int64_t total = 0;
    int rc = read_model_json(text, &d, &offs, &ad, &has_ad, &total, &why);
    if (rc) return fail(c, rc, "%s: %s", jp.c_str(), why.c_str());
    std::ifstream f(weights_path, std::ios::binary | std::ios::ate);
    if (!f.is_open()) return fail(c, PRISM_ERR_INVALID, "cannot open %s", weights_path);
    const std::streamsize size = f.tellg();
    if (size != (std::streamsize)(2 * total))
        return fail(c, PRISM_ERR_BLOB, "%s holds %lld bytes, its sidecar says %lld", weights_path, (long long)size,
                    (long long)(2 * total));
    f.seekg(0);
    std::vector<char> data;
    try {
        data.resize((size_t)size);
    } catch (...) {
        return fail(c, PRISM_ERR_NOMEM, "cannot allocate %lld bytes for %s", (long long)size, weights_path);
    }
    if (size > 0 && !f.read(data.data(), size)) return fail(c, PRISM_ERR_INVALID, "short read on %s", weights_path);
    rc = prism_load_weights(c, &d, data.data(), data.size(), offs.data());
    if (rc) return rc;
    return has_ad ? prism_load_adapters(c, data.data(), data.size(), &ad) : PRISM_OK;
}

/* ------------------------------------------------------------ launches */

namespace {

template <class A>
int launch(prism_ctx* c, hipFunction_t f, unsigned grid, A& args, hipStream_t s, unsigned block = 256) {
    void* params[] = {&args};
    hipError_t e = hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipModuleLaunchKernel: %s", hipGetErrorString(e));
    c->last_grid = grid;
    return PRISM_OK;
}

/* Routing outputs of a routed attention launch (block chain, MoE blocks). */
struct RouteOut {
    int32_t* assign;
    int32_t* counts; /* zero on entry; expert e at counts[e * count_stride] */
    int32_t* perm;
    int32_t count_stride;
    int32_t* zero_next; /* counters this launch clears for a later one, or NULL */
};

/* ffn: a dense block's FFN runs in the same launch (the window's rows never
 * leave the CU between the two), and `out` receives the block's output */
int enqueue_attn(prism_ctx* c, const DevBlock& k, const uint16_t* in, uint16_t* out, int H, int W, int batch,
                 hipStream_t s, const RouteOut* route = nullptr, bool up = false, bool ffn = false) {
    const int D = c->desc.dim;
    if (ffn && (route || c->desc.n_experts != 1))
        return fail(c, PRISM_ERR_INVALID, "the fused FFN is for dense blocks");
    AttnArgs a{};
    if (ffn) {
        a.ffn_w1 = k.w1;
        a.ffn_b1 = k.b1;
        a.ffn_w2 = k.w2;
        a.ffn_b2 = k.b2;
    }
    if (up) { /* the adapted chain's first block: 128-channel input rows */
        a.up_w = c->up_w;
        a.up_b = c->up_b;
    }
    a.in = in;
    a.out = out;
    a.wqkv = k.wqkv;
    a.bqkv = k.bqkv;
    a.bqkv_pad = k.bqkv_pad;
    a.wo = k.wo;
    a.bo = k.bo;
    a.frame_elems = (int64_t)H * W * D;
    a.in_frame_elems = (int64_t)H * W * (up ? c->aoffs.in_dim : D);
    a.H = H;
    a.W = W;
    a.wx = (W + 7) / 8;
    a.windows_per_frame = a.wx * ((H + 7) / 8);
    int npt = 0;
    if (route) {
        const int N = c->desc.n_experts;
        npt = round16(N) / 16;
        a.wr = k.wr;
        a.br = k.br;
        a.assign = route->assign;
        a.counts = route->counts;
        a.perm = route->perm;
        a.n_experts = N;
        a.cap = (int32_t)((int64_t)batch * H * W);
        a.count_stride = route->count_stride;
        a.zero_next = route->zero_next;
    }
    const int64_t grid = (int64_t)a.windows_per_frame * batch;
    if (grid <= 0 || grid > 0x7fffffff) return fail(c, PRISM_ERR_INVALID, "attention grid %lld out of range", (long long)grid);
    /* fewer than two windows per CU: one 8-wave workgroup per window (a head per
     * wave) shortens each window's serial path; otherwise 4 waves x 2 per CU */
    const int w8 = grid < 512 ? 1 : 0;
    const hipFunction_t f = ffn ? c->f_attn_ffn[dim_index(D)][w8] : c->f_attn[dim_index(D)][w8][npt];
    if (!f) return fail(c, PRISM_ERR_INVALID, "no fused FFN kernel for d%d at %lld windows", D, (long long)grid);
    return launch(c, f, (unsigned)grid, a, s, w8 ? 512u : 256u);
}

int enqueue_zero(prism_ctx* c, int32_t* p, int32_t n, hipStream_t s) {
    void* params[] = {&p, &n};
    const unsigned grid = (unsigned)std::max(1, std::min(64, (n + 255) / 256));
    hipError_t e = hipModuleLaunchKernel(c->f_zero, grid, 1, 1, 256, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipModuleLaunchKernel(zero): %s", hipGetErrorString(e));
    return PRISM_OK;
}

int enqueue_router(prism_ctx* c, const DevBlock& k, const uint16_t* in, int32_t* assign, int32_t* counts,
                   int32_t* perm, int64_t n, hipStream_t s, int32_t count_stride) {
    const int N = c->desc.n_experts;
    RouterArgs a{};
    a.in = in;
    a.wr = k.wr;
    a.br = k.br;
    a.assign = assign;
    a.counts = counts;
    a.perm = perm;
    a.n_tokens = (int32_t)n;
    a.n_experts = N;
    a.np = round16(N);
    a.cap = (int32_t)n;
    a.count_stride = count_stride;
    /* tiles per wave for about 512 workgroups (two per CU): one tile per wave
     * at frame scale, 4 at batch 16 (measured 8.9 / 22.2 us; more, smaller
     * workgroups each copy W_r into LDS, fewer leave CUs idle) */
    a.tiles_per_wave = (int32_t)std::min<int64_t>(ROUTER_MAX_TILES_PER_WAVE, std::max<int64_t>(1, (n + 32767) / 32768));
    const int64_t grid = (n + 64 * a.tiles_per_wave - 1) / (64 * a.tiles_per_wave);
    return launch(c, c->f_router[dim_index(c->desc.dim)][a.np / 16 - 1], (unsigned)grid, a, s);
}

int enqueue_experts(prism_ctx* c, const DevBlock& k, const uint16_t* in, uint16_t* out, const int32_t* counts,
                    const int32_t* perm, int64_t n, hipStream_t s, int32_t count_stride = 1, bool dn = false,
                    bool stage = false, bool wnt = false) {
    const int D = c->desc.dim, N = counts ? c->desc.n_experts : 1;
    ExpertArgs a{};
    if (dn) { /* the adapted chain's last block: 128-channel output rows */
        a.dn_w = c->down_w;
        a.dn_b = c->down_b;
    }
    a.in = in;
    a.out = out;
    a.w1 = k.w1;
    a.b1 = k.b1;
    a.w2 = k.w2;
    a.b2 = k.b2;
    a.counts = counts;
    a.perm = perm;
    a.n_tokens = (int32_t)n;
    a.n_experts = N;
    a.cap = (int32_t)n;
    a.count_stride = count_stride;
    a.wnt = wnt ? 1 : 0;
    /* tiles: the worst case of ceil(n / bm) + one partial tile per expert,
     * a multiple of 8 (the kernels' XCD-major tile order) */
    auto tiles_of = [&](int64_t bm) { return ((n + bm - 1) / bm + (counts ? N : 0) + 7) / 8 * 8; };
    if (D == 256 && !dn && tiles_of(128) >= EXPERT_WIDE_MIN_TILES)
        return stage ? launch(c, c->f_expert_wide96, (unsigned)tiles_of(96), a, s, 256u)
                     : launch(c, c->f_expert_wide, (unsigned)tiles_of(128), a, s, 256u);
    const int64_t tiles = tiles_of(64);
    /* fewer tiles than two per CU: 8 waves per tile halve each wave's weight stream */
    const int w8 = tiles < 512 ? 1 : 0;
    return launch(c, c->f_expert[dim_index(D)][w8], (unsigned)tiles, a, s, w8 ? 512u : 256u);
}

/* up: in_dim -> dim with ReLU; down: dim -> in_dim. n tokens. */
int enqueue_project(prism_ctx* c, bool up, const uint16_t* in, uint16_t* out, int64_t n, hipStream_t s) {
    ProjArgs a{};
    a.in = in;
    a.out = out;
    a.w = up ? c->up_w : c->down_w;
    a.b = up ? c->up_b : c->down_b;
    a.n_tokens = n;
    const int64_t tiles = (n + 63) / 64;
    if (tiles <= 0 || tiles > 0x7fffffff) return fail(c, PRISM_ERR_INVALID, "projection tiles %lld out of range", (long long)tiles);
    /* persistent workgroups, each looping over 64-token tiles */
    const int64_t grid = std::min<int64_t>(tiles, PROJ_GRID_MAX);
    return launch(c, c->f_proj[dim_index(c->desc.dim)][up ? 0 : 1], (unsigned)grid, a, s);
}

/* which: 0 = attention (qkv_w), 1 = router (router_w), 2 = experts (exp_w1) */
const DevBlock* find_block(prism_ctx* c, int64_t key, int which) {
    for (const DevBlock& k : c->blocks) {
        const int64_t v = which == 0 ? k.offs.qkv_w : which == 1 ? k.offs.router_w : k.offs.exp_w1;
        if (v == key) return &k;
    }
    return nullptr;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

static int check_attn(prism_ctx* c, const prism_attn_push* p, void* features, int32_t batch, const DevBlock** kb) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->loaded) return fail(c, PRISM_ERR_STATE, "weights not loaded");
    if (!p || !features) return fail(c, PRISM_ERR_INVALID, "push or features is NULL");
    if (batch < 1) return fail(c, PRISM_ERR_INVALID, "batch %d < 1", batch);
    if (p->dim != c->desc.dim || p->n_heads != c->desc.n_heads || p->head_dim != c->desc.head_dim)
        return fail(c, PRISM_ERR_INVALID, "push shape dim=%d heads=%d head_dim=%d does not match the loaded model", p->dim,
                    p->n_heads, p->head_dim);
    if (p->window_size != 8) return fail(c, PRISM_ERR_UNSUPPORTED, "window_size %d (supported: 8)", p->window_size);
    if (p->spatial_w < 1 || p->spatial_h < 1 || (int64_t)p->spatial_w * p->spatial_h != p->n_tokens)
        return fail(c, PRISM_ERR_INVALID, "n_tokens %d != spatial_w*spatial_h (%d*%d)", p->n_tokens, p->spatial_w,
                    p->spatial_h);
    if (p->n_tokens < ATTN_MIN_TOKENS)
        return fail(c, PRISM_ERR_UNSUPPORTED, "%d tokens per frame: attention needs at least %d (%s)", p->n_tokens,
                    ATTN_MIN_TOKENS, ATTN_MIN_TOKENS_WHY);
    if (!tokens_fit(p->n_tokens, p->dim)) /* a frame's rows, addressed with 32-bit offsets */
        return fail(c, PRISM_ERR_INVALID, "%d tokens per frame is too many", p->n_tokens);
    const DevBlock* k = find_block(c, p->qkv_w, 0);
    if (!k || k->offs.qkv_b != p->qkv_b || k->offs.out_w != p->out_w || k->offs.out_b != p->out_b ||
        k->offs.ln1_g != p->ln1_g || k->offs.ln1_b != p->ln1_b)
        return fail(c, PRISM_ERR_INVALID, "attention weight offsets do not name a loaded block");
    if (p->input_offset < 0 || p->output_offset < 0)
        return fail(c, PRISM_ERR_INVALID, "negative feature offset");
    uint16_t* f = static_cast<uint16_t*>(features);
    if (!aligned16(f + p->input_offset) || !aligned16(f + p->output_offset))
        return fail(c, PRISM_ERR_INVALID, "feature offsets must be 16-byte aligned (multiples of 8 elements)");
    *kb = k;
    return PRISM_OK;
}

static int check_router(prism_ctx* c, const prism_router_push* p, const void* features, int32_t* aux, int32_t batch,
                        const DevBlock** kb) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->loaded) return fail(c, PRISM_ERR_STATE, "weights not loaded");
    if (!p || !features || !aux) return fail(c, PRISM_ERR_INVALID, "push, features or aux is NULL");
    if (c->desc.n_experts < 2) return fail(c, PRISM_ERR_STATE, "the loaded model is dense (no router)");
    if (batch < 1 || p->n_tokens < 1) return fail(c, PRISM_ERR_INVALID, "batch %d / n_tokens %d < 1", batch, p->n_tokens);
    if (p->dim != c->desc.dim || p->n_experts != c->desc.n_experts)
        return fail(c, PRISM_ERR_INVALID, "push dim=%d n_experts=%d does not match the loaded model", p->dim, p->n_experts);
    const int64_t n = (int64_t)batch * p->n_tokens;
    if (!tokens_fit(n, c->desc.dim)) return fail(c, PRISM_ERR_INVALID, "%lld tokens is too many", (long long)n);
    const DevBlock* k = find_block(c, p->router_w, 1);
    if (!k || k->offs.router_b != p->router_b || k->offs.ln2_g != p->ln2_g || k->offs.ln2_b != p->ln2_b)
        return fail(c, PRISM_ERR_INVALID, "router weight offsets do not name a loaded block");
    if (p->input_offset < 0 || p->assignment_offset < 0 || p->count_offset < 0 || p->perm_offset < 0)
        return fail(c, PRISM_ERR_INVALID, "negative offset");
    const uint16_t* f = static_cast<const uint16_t*>(features);
    if (!aligned16(f + p->input_offset)) return fail(c, PRISM_ERR_INVALID, "input_offset must be a multiple of 8");
    *kb = k;
    return PRISM_OK;
}

extern "C" int prism_attn(prism_ctx* c, const prism_attn_push* p, void* features, int32_t batch, void* stream) {
    const DevBlock* k = nullptr;
    const int rc = check_attn(c, p, features, batch, &k);
    if (rc) return rc;
    HIP_TRY(c, hipSetDevice(c->device));
    uint16_t* f = static_cast<uint16_t*>(features);
    return enqueue_attn(c, *k, f + p->input_offset, f + p->output_offset, p->spatial_h, p->spatial_w, batch,
                        (hipStream_t)stream);
}

/* The routing stage calls count into a private row, counters 256 B apart as
 * in the chain (every workgroup adds to them; adjacent counters would
 * serialise those atomics), and prism_take_counts then moves the totals to
 * the caller's contiguous counts, clearing the row for the next call. */
static int stage_counts_begin(prism_ctx* c, hipStream_t s) {
    if (!c->stage_counts) {
        const size_t bytes = sizeof(int32_t) * 64 * CHAIN_COUNT_STRIDE;
        HIP_TRY(c, hipMalloc((void**)&c->stage_counts, bytes));
        HIP_TRY(c, hipMemset(c->stage_counts, 0, bytes));
    }
    if (c->stage_dirty) {
        const int rc = enqueue_zero(c, c->stage_counts, 64 * CHAIN_COUNT_STRIDE, s);
        if (rc) return rc;
        c->stage_dirty = false;
    }
    c->stage_dirty = true; /* until stage_counts_take has been enqueued */
    return PRISM_OK;
}

static int stage_counts_take(prism_ctx* c, int32_t* dst, int32_t n, hipStream_t s) {
    int32_t* src = c->stage_counts;
    int32_t stride = CHAIN_COUNT_STRIDE;
    void* params[] = {&src, &stride, &dst, &n};
    const hipError_t e = hipModuleLaunchKernel(c->f_take, 1, 1, 1, 64, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipModuleLaunchKernel(take counts): %s", hipGetErrorString(e));
    c->stage_dirty = false;
    return PRISM_OK;
}

extern "C" int prism_router(prism_ctx* c, const prism_router_push* p, const void* features, int32_t* aux,
                            int32_t batch, void* stream) {
    const DevBlock* k = nullptr;
    int rc = check_router(c, p, features, aux, batch, &k);
    if (rc) return rc;
    HIP_TRY(c, hipSetDevice(c->device));
    const hipStream_t s = (hipStream_t)stream;
    rc = stage_counts_begin(c, s);
    if (rc) return rc;
    const uint16_t* f = static_cast<const uint16_t*>(features);
    rc = enqueue_router(c, *k, f + p->input_offset, aux + p->assignment_offset, c->stage_counts,
                        aux + p->perm_offset, (int64_t)batch * p->n_tokens, s, CHAIN_COUNT_STRIDE);
    if (rc) return rc;
    return stage_counts_take(c, aux + p->count_offset, p->n_experts, s);
}

extern "C" int prism_attn_route(prism_ctx* c, const prism_attn_push* pa, const prism_router_push* pr, void* features,
                                int32_t* aux, int32_t batch, void* stream) {
    const DevBlock *ka = nullptr, *kr = nullptr;
    int rc = check_attn(c, pa, features, batch, &ka);
    if (rc) return rc;
    rc = check_router(c, pr, features, aux, batch, &kr);
    if (rc) return rc;
    if (ka != kr) return fail(c, PRISM_ERR_INVALID, "attention and router pushes name different blocks");
    if (pr->input_offset != pa->output_offset || pr->n_tokens != pa->n_tokens)
        return fail(c, PRISM_ERR_INVALID, "the router must read the attention output (input_offset %lld != %lld)",
                    (long long)pr->input_offset, (long long)pa->output_offset);
    HIP_TRY(c, hipSetDevice(c->device));
    const hipStream_t s = (hipStream_t)stream;
    rc = stage_counts_begin(c, s);
    if (rc) return rc;
    uint16_t* f = static_cast<uint16_t*>(features);
    const RouteOut ro{aux + pr->assignment_offset, c->stage_counts, aux + pr->perm_offset, CHAIN_COUNT_STRIDE, nullptr};
    rc = enqueue_attn(c, *ka, f + pa->input_offset, f + pa->output_offset, pa->spatial_h, pa->spatial_w, batch, s, &ro);
    if (rc) return rc;
    return stage_counts_take(c, aux + pr->count_offset, pr->n_experts, s);
}

extern "C" int prism_experts(prism_ctx* c, const prism_expert_push* p, void* features, int32_t* aux, int32_t batch,
                             void* stream) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->loaded) return fail(c, PRISM_ERR_STATE, "weights not loaded");
    if (!p || !features) return fail(c, PRISM_ERR_INVALID, "push or features is NULL");
    if (batch < 1 || p->n_tokens < 1) return fail(c, PRISM_ERR_INVALID, "batch %d / n_tokens %d < 1", batch, p->n_tokens);
    const bool dense = p->count_offset < 0;
    if (p->dim != c->desc.dim) return fail(c, PRISM_ERR_INVALID, "push dim %d does not match the model", p->dim);
    if (dense ? p->n_experts != 1 : p->n_experts != c->desc.n_experts)
        return fail(c, PRISM_ERR_INVALID, "n_experts %d does not match the model (%d) / dense mode", p->n_experts,
                    c->desc.n_experts);
    if (!dense && (!aux || p->perm_offset < 0))
        return fail(c, PRISM_ERR_INVALID, "routed expert stage needs aux with count and perm regions");
    const int64_t n = (int64_t)batch * p->n_tokens;
    if (!tokens_fit(n, c->desc.dim)) return fail(c, PRISM_ERR_INVALID, "%lld tokens is too many", (long long)n);
    const DevBlock* k = find_block(c, p->w1, 2);
    if (!k || k->offs.exp_b1 != p->b1 || k->offs.exp_w2 != p->w2 || k->offs.exp_b2 != p->b2 ||
        k->offs.exp_stride != p->expert_stride || k->offs.ln2_g != p->ln2_g || k->offs.ln2_b != p->ln2_b)
        return fail(c, PRISM_ERR_INVALID, "expert weight offsets do not name a loaded block");
    if (p->input_offset < 0 || p->output_offset < 0) return fail(c, PRISM_ERR_INVALID, "negative feature offset");
    uint16_t* f = static_cast<uint16_t*>(features);
    if (!aligned16(f + p->input_offset) || !aligned16(f + p->output_offset))
        return fail(c, PRISM_ERR_INVALID, "feature offsets must be multiples of 8 elements");
    HIP_TRY(c, hipSetDevice(c->device));
    return enqueue_experts(c, *k, f + p->input_offset, f + p->output_offset, dense ? nullptr : aux + p->count_offset,
                           dense ? nullptr : aux + p->perm_offset, n, (hipStream_t)stream, 1, false, true);
}

static int project_stage(prism_ctx* c, bool up, const prism_project_push* p, void* features, int32_t batch,
                         void* stream) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->adapters) return fail(c, PRISM_ERR_STATE, "adapters not loaded");
    if (!p || !features) return fail(c, PRISM_ERR_INVALID, "push or features is NULL");
    if (batch < 1 || p->n_tokens < 1) return fail(c, PRISM_ERR_INVALID, "batch %d / n_tokens %d < 1", batch, p->n_tokens);
    const int64_t w = up ? c->aoffs.up_w : c->aoffs.down_w, b = up ? c->aoffs.up_b : c->aoffs.down_b;
    if (p->w_offset != w || p->b_offset != b)
        return fail(c, PRISM_ERR_INVALID, "projection weight offsets do not name the loaded %s adapter", up ? "up" : "down");
    if (p->input_offset < 0 || p->output_offset < 0) return fail(c, PRISM_ERR_INVALID, "negative feature offset");
    uint16_t* f = static_cast<uint16_t*>(features);
    if (!aligned16(f + p->input_offset) || !aligned16(f + p->output_offset))
        return fail(c, PRISM_ERR_INVALID, "feature offsets must be multiples of 8 elements");
    HIP_TRY(c, hipSetDevice(c->device));
    return enqueue_project(c, up, f + p->input_offset, f + p->output_offset, (int64_t)batch * p->n_tokens,
                           (hipStream_t)stream);
}

extern "C" int prism_project_up(prism_ctx* c, const prism_project_push* p, void* features, int32_t batch,
                                void* stream) {
    return project_stage(c, true, p, features, batch, stream);
}

extern "C" int prism_project_down(prism_ctx* c, const prism_project_push* p, void* features, int32_t batch,
                                  void* stream) {
    return project_stage(c, false, p, features, batch, stream);
}

/* ------------------------------------------------------------ block chain */

/* Byte offsets of the chain's buffers for n tokens (io: also the adapted
 * chain's 256-channel buffer), from one base; returns the total size. */
struct ChainLayout {
    size_t attn, scr, asg, cnt, perm, io, bytes;
};
static ChainLayout chain_layout(const prism_model_desc& d, int64_t n, bool io) {
    const size_t D = d.dim, N = d.n_experts, NB = d.n_blocks;
    Arena ar;
    ChainLayout L;
    L.attn = ar.take((size_t)n * D * 2);
    L.scr = ar.take((size_t)n * D * 2);
    L.asg = ar.take(NB * (size_t)n * 4);
    L.cnt = ar.take((size_t)CHAIN_SPLIT * NB * N * CHAIN_COUNT_STRIDE * 4);
    L.perm = ar.take(N * (size_t)n * 4);
    L.io = ar.take(io ? (size_t)n * D * 2 : 0);
    L.bytes = ar.off;
    return L;
}

static ChainWs chain_ws_at(void* base, const ChainLayout& L, int64_t n, bool io) {
    uint8_t* b = static_cast<uint8_t*>(base);
    ChainWs w;
    w.attn = reinterpret_cast<uint16_t*>(b + L.attn);
    w.scratch = reinterpret_cast<uint16_t*>(b + L.scr);
    w.io = io ? reinterpret_cast<uint16_t*>(b + L.io) : nullptr;
    w.assign = reinterpret_cast<int32_t*>(b + L.asg);
    w.counts = reinterpret_cast<int32_t*>(b + L.cnt);
    w.perm = reinterpret_cast<int32_t*>(b + L.perm);
    w.n = n;
    return w;
}

/* io: also the adapted chain's 256-channel buffer */
static int ensure_workspace(prism_ctx* c, int batch, bool io = false) {
    if (c->ws && c->ws_batch >= batch && (!io || c->wsb.io)) return PRISM_OK;
    io = io || (c->ws && c->wsb.io); /* keep it once allocated */
    drop_graph(c);
    drop_workspace(c);
    const int64_t n = (int64_t)batch * c->desc.spatial_h * c->desc.spatial_w;
    if (!tokens_fit(n, c->desc.dim)) return fail(c, PRISM_ERR_INVALID, "%lld tokens is too many", (long long)n);
    const ChainLayout L = chain_layout(c->desc, n, io);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, L.bytes);
    if (e != hipSuccess) return fail(c, PRISM_ERR_NOMEM, "hipMalloc(%zu) for the workspace: %s", L.bytes, hipGetErrorString(e));
    e = hipMemset(p, 0, L.bytes);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return fail(c, PRISM_ERR_HIP, "hipMemset workspace: %s", hipGetErrorString(e));
    }
    c->ws = p;
    c->ws_batch = batch;
    c->ws_tokens = n;
    c->wsb = chain_ws_at(p, L, n, io);
    c->counts_dirty = false; /* zero-filled above */
    return PRISM_OK;
}

/* Block b reads the previous block's output (block 0 reads `in`) and writes
 * `out` if (n_blocks-1-b) is even, the scratch buffer otherwise, so the last
 * block always lands in `out` and `in` is only read. MoE blocks run two
 * launches: attention with fused routing, then the experts. Each block has
 * its own row of counters; block b's attention launch clears block b+1's
 * row, and the last block clears block 0's for the next chain, so a complete
 * chain leaves row 0 at zero. The workspace starts zeroed; a one-block model
 * clears its row inside the chain; after a chain that failed part-way, the
 * next prism_forward / prism_forward_graph call clears the counters first.
 * With 2 * CHAIN_SPLIT_FRAMES frames or more the batch runs as sub-chains
 * (own counter rows, own bucket region, disjoint frames of every buffer). */
/* Sub-chain j: frames [f0, f0 + nf) through every block, in -> out (this
 * sub-chain's frames). adapted: in and out hold 128-channel rows; block 0's
 * attention runs the up-projection in its prologue and the last block's
 * expert stage the down-projection in its epilogue, the blocks in between
 * ping-pong through the 256-channel buffers (ws.io, ws.scratch). */
/* Events between the launches of a timed chain (prism_chain_launch_times):
 * ev[0] before the first launch, ev[i] after launch i, whose kind (0 =
 * attention, 1 = experts) and grid are kept. */
struct ChainTimer {
    std::vector<hipEvent_t> ev;
    std::vector<int> kind;
    std::vector<unsigned> grid;
    size_t n = 0; /* events recorded */
};

static int timer_mark(prism_ctx* c, ChainTimer* tm, int kind, hipStream_t s) {
    if (!tm) return PRISM_OK;
    if (tm->n >= tm->ev.size()) return fail(c, PRISM_ERR_STATE, "chain timer: more launches than events");
    HIP_TRY(c, hipEventRecord(tm->ev[tm->n], s));
    if (tm->n > 0) {
        tm->kind.push_back(kind);
        tm->grid.push_back(c->last_grid);
    }
    ++tm->n;
    return PRISM_OK;
}

static int enqueue_subchain(prism_ctx* c, const ChainWs& ws, int j, int f0, int nf, const uint16_t* in,
                            uint16_t* out, hipStream_t s, bool adapted = false, ChainTimer* tm = nullptr) {
    const int NB = c->desc.n_blocks, H = c->desc.spatial_h, W = c->desc.spatial_w, D = c->desc.dim;
    const int N = c->desc.n_experts;
    const bool moe = N > 1;
    const int64_t T = (int64_t)H * W, n = (int64_t)nf * T, t0 = (int64_t)f0 * T, n_all = ws.n;
    const size_t row = (size_t)N * CHAIN_COUNT_STRIDE;
    int32_t* counts0 = ws.counts + (size_t)j * NB * row;
    int32_t* perm = ws.perm + (size_t)N * t0; /* this half's buckets: [N][n] */
    uint16_t* attn = ws.attn + t0 * D;
    uint16_t* scratch = ws.scratch + t0 * D;
    uint16_t* mid = adapted ? ws.io + t0 * D : out; /* 256-channel stand-in for `out` */
    if (moe && NB == 1) {
        const int rc = enqueue_zero(c, counts0, (int32_t)row, s);
        if (rc) return rc;
    }
    const uint16_t* src = in;
    for (int b = 0; b < NB; ++b) {
        const DevBlock& k = c->blocks[b];
        const bool first = adapted && b == 0, last = adapted && b == NB - 1;
        uint16_t* dst = last ? out : ((NB - 1 - b) % 2 == 0) ? mid : scratch;
        if (moe) {
            int32_t* counts = counts0 + (size_t)b * row;
            const RouteOut ro{ws.assign + (size_t)b * n_all + t0, counts, perm, CHAIN_COUNT_STRIDE,
                              NB > 1 ? counts0 + (size_t)((b + 1) % NB) * row : nullptr};
            int rc = enqueue_attn(c, k, src, attn, H, W, nf, s, &ro, first);
            if (!rc) rc = timer_mark(c, tm, 0, s);
            if (!rc)
                rc = enqueue_experts(c, k, attn, dst, counts, perm, n, s, CHAIN_COUNT_STRIDE, last, false,
                                     b < c->wnt_blocks);
            if (!rc) rc = timer_mark(c, tm, 1, s);
            if (rc) return rc;
        } else if (!last) { /* one launch: attention + the FFN */
            int rc = enqueue_attn(c, k, src, dst, H, W, nf, s, nullptr, first, true);
            if (!rc) rc = timer_mark(c, tm, 0, s);
            if (rc) return rc;
        } else {
            int rc = enqueue_attn(c, k, src, attn, H, W, nf, s, nullptr, first);
            if (!rc) rc = timer_mark(c, tm, 0, s);
            if (!rc) rc = enqueue_experts(c, k, attn, dst, nullptr, nullptr, n, s, 1, last);
            if (!rc) rc = timer_mark(c, tm, 1, s);
            if (rc) return rc;
        }
        src = dst;
    }
    return PRISM_OK;
}

static int enqueue_forward_impl(prism_ctx* c, const ChainWs& ws, const uint16_t* in, uint16_t* out, int batch,
                                hipStream_t s, bool adapted = false) {
    const int64_t T = (int64_t)c->desc.spatial_h * c->desc.spatial_w;
    const int64_t D = adapted ? c->aoffs.in_dim : c->desc.dim; /* channels of in and out */
    c->fwd_tokens = (int64_t)batch * T;
    c->fwd_assign = ws.assign;
    const int S = std::max(1, std::min(CHAIN_SPLIT, batch / CHAIN_SPLIT_FRAMES));
    if (S == 1) return enqueue_subchain(c, ws, 0, 0, batch, in, out, s, adapted);
    /* fork: sub-chain j > 0 on sub_stream[j-1], sub-chain 0 on s, then join */
    HIP_TRY(c, hipEventRecord(c->ev_fork, s));
    int rc = PRISM_OK;
    for (int j = S - 1; j >= 0; --j) {
        const int f0 = (int)((int64_t)batch * j / S), f1 = (int)((int64_t)batch * (j + 1) / S);
        hipStream_t sj = j ? c->sub_stream[j - 1] : s;
        if (j) HIP_TRY(c, hipStreamWaitEvent(sj, c->ev_fork, 0));
        const int r = enqueue_subchain(c, ws, j, f0, f1 - f0, in + f0 * T * D, out + f0 * T * D, sj, adapted);
        if (!rc) rc = r;
        if (j) HIP_TRY(c, hipEventRecord(c->ev_join[j - 1], sj));
    }
    for (int j = 1; j < S; ++j) HIP_TRY(c, hipStreamWaitEvent(s, c->ev_join[j - 1], 0));
    return rc;
}

/* Clears block 0's counters on `s` if a failed chain may have left them set. */
static int clean_counts(prism_ctx* c, hipStream_t s) {
    if (!c->counts_dirty || c->desc.n_experts < 2) return PRISM_OK;
    /* every half-chain's counter rows (small) */
    const int rc = enqueue_zero(c, c->wsb.counts, CHAIN_SPLIT * c->desc.n_blocks * c->desc.n_experts * CHAIN_COUNT_STRIDE, s);
    if (rc == PRISM_OK) c->counts_dirty = false;
    return rc;
}

static int forward_checks(prism_ctx* c, const void* in, void* out, int batch) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->loaded) return fail(c, PRISM_ERR_STATE, "weights not loaded");
    if (!in || !out) return fail(c, PRISM_ERR_INVALID, "in or out is NULL");
    if (!aligned16(in) || !aligned16(out)) return fail(c, PRISM_ERR_INVALID, "in/out must be 16-byte aligned");
    if (batch < 1) return fail(c, PRISM_ERR_INVALID, "batch %d < 1", batch);
    if ((int64_t)c->desc.spatial_h * c->desc.spatial_w < ATTN_MIN_TOKENS)
        return fail(c, PRISM_ERR_UNSUPPORTED, "%dx%d token grid: attention needs at least %d tokens per frame (%s)",
                    c->desc.spatial_h, c->desc.spatial_w, ATTN_MIN_TOKENS, ATTN_MIN_TOKENS_WHY);
    return PRISM_OK;
}

/* The chain (CHAIN_BLOCKS); wrapped in the projection adapters (CHAIN_ADAPTED:
 * the up-projection fused into the first block's attention, the
 * down-projection into the last block's expert stage, 128-channel in and
 * out); and that inside the encoder and decoder (CHAIN_E2E): encode(frame ->
 * cbott), adapted chain(cbott -> cchain), decode(cchain -> display). */
static int enqueue_chain(prism_ctx* c, const uint16_t* in, uint16_t* out, int batch, int mode, hipStream_t s) {
    ChainWs ws = c->wsb;
    ws.n = (int64_t)batch * c->desc.spatial_h * c->desc.spatial_w; /* rows of this forward */
    if (mode == CHAIN_BLOCKS) return enqueue_forward_impl(c, ws, in, out, batch, s);
    if (mode == CHAIN_E2E) {
        int rc = codec_enqueue_encode(c, in, c->cbott, batch, s);
        if (!rc) rc = enqueue_chain(c, c->cbott, c->cchain, batch, CHAIN_ADAPTED, s);
        if (!rc) rc = codec_enqueue_decode(c, c->cchain, out, batch, s);
        return rc;
    }
    return enqueue_forward_impl(c, ws, in, out, batch, s, true);
}

static int mode_ready(prism_ctx* c, int mode, int batch) {
    if (mode != CHAIN_BLOCKS && !c->adapters) return fail(c, PRISM_ERR_STATE, "adapters not loaded");
    if (mode == CHAIN_E2E && !c->codec) return fail(c, PRISM_ERR_STATE, "encoder / decoder weights not loaded");
    int rc = ensure_workspace(c, batch, mode != CHAIN_BLOCKS);
    if (!rc && mode == CHAIN_E2E) rc = codec_ensure_workspace(c, batch);
    return rc;
}

static int run_forward(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream, int mode) {
    int rc = forward_checks(c, in, out, batch);
    if (rc) return rc;
    HIP_TRY(c, hipSetDevice(c->device));
    rc = mode_ready(c, mode, batch);
    if (rc) return rc;
    rc = clean_counts(c, (hipStream_t)stream);
    if (rc) return rc;
    rc = enqueue_chain(c, static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), batch, mode,
                       (hipStream_t)stream);
    if (rc) c->counts_dirty = true; /* launched part of the chain */
    return rc;
}

/* `before`, if given, is recorded on the stream right before the graph launch
 * (after any capture and counter clear), so its distance to an event recorded
 * after the call is the chain's GPU time alone. */
static int run_forward_graph(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream, int mode,
                             hipEvent_t before = nullptr) {
    int rc = forward_checks(c, in, out, batch);
    if (rc) return rc;
    HIP_TRY(c, hipSetDevice(c->device));
    rc = mode_ready(c, mode, batch); /* may reallocate (which drops the graph) */
    if (rc) return rc;
    if (!(c->gexec && c->g_in == in && c->g_out == out && c->g_batch == batch && c->g_mode == mode)) {
        drop_graph(c);
        HIP_TRY(c, hipStreamSynchronize(c->cap_stream));
        HIP_TRY(c, hipStreamBeginCapture(c->cap_stream, hipStreamCaptureModeThreadLocal));
        /* captured, not run: a failure here leaves the counters untouched */
        rc = enqueue_chain(c, static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), batch, mode,
                           c->cap_stream);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(c->cap_stream, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
        c->graph = g;
        const hipError_t ei = hipGraphInstantiate(&c->gexec, g, nullptr, nullptr, 0);
        if (ei != hipSuccess) {
            drop_graph(c);
            return fail(c, PRISM_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(ei));
        }
        c->g_in = in;
        c->g_out = out;
        c->g_batch = batch;
        c->g_mode = mode;
    }
    rc = clean_counts(c, (hipStream_t)stream);
    if (rc) return rc;
    if (before) HIP_TRY(c, hipEventRecord(before, (hipStream_t)stream));
    HIP_TRY(c, hipGraphLaunch(c->gexec, (hipStream_t)stream));
    /* the replayed chain writes its assignment rows at this token count (a
     * capture sets it too, but a replay of a cached graph captures nothing) */
    c->fwd_tokens = (int64_t)batch * c->desc.spatial_h * c->desc.spatial_w;
    c->fwd_assign = c->wsb.assign;
    return PRISM_OK;
}

extern "C" int prism_forward(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream) {
    return run_forward(c, in, out, batch, stream, CHAIN_BLOCKS);
}

extern "C" int prism_forward_graph(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream) {
    return run_forward_graph(c, in, out, batch, stream, CHAIN_BLOCKS);
}

extern "C" int prism_forward_adapted(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream) {
    return run_forward(c, in, out, batch, stream, CHAIN_ADAPTED);
}

extern "C" int prism_forward_adapted_graph(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream) {
    return run_forward_graph(c, in, out, batch, stream, CHAIN_ADAPTED);
}

extern "C" int prism_forward_e2e(prism_ctx* c, const void* frame, void* display, int32_t batch, void* stream) {
    return run_forward(c, frame, display, batch, stream, CHAIN_E2E);
}

extern "C" int prism_forward_e2e_graph(prism_ctx* c, const void* frame, void* display, int32_t batch, void* stream) {
    return run_forward_graph(c, frame, display, batch, stream, CHAIN_E2E);
}

extern "C" int prism_chain_launch_times(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream,
                                        float* attn_ms, float* expert_ms, int32_t* attn_grid,
                                        int32_t* expert_grid) {
    int rc = forward_checks(c, in, out, batch);
    if (rc) return rc;
    if (!attn_ms || !expert_ms) return fail(c, PRISM_ERR_INVALID, "attn_ms or expert_ms is NULL");
    HIP_TRY(c, hipSetDevice(c->device));
    rc = mode_ready(c, CHAIN_BLOCKS, batch);
    if (rc) return rc;
    const hipStream_t s = (hipStream_t)stream;
    rc = clean_counts(c, s);
    if (rc) return rc;
    ChainWs ws = c->wsb;
    const int64_t T = (int64_t)c->desc.spatial_h * c->desc.spatial_w, D = c->desc.dim;
    ws.n = (int64_t)batch * T;
    c->fwd_tokens = ws.n;
    c->fwd_assign = ws.assign;
    /* the sub-chains of prism_forward, one after another on one stream */
    const int S = std::max(1, std::min(CHAIN_SPLIT, batch / CHAIN_SPLIT_FRAMES));
    ChainTimer tm;
    tm.ev.assign((size_t)2 * c->desc.n_blocks * S + 1, nullptr);
    for (auto& e : tm.ev) {
        const hipError_t he = hipEventCreate(&e);
        if (he != hipSuccess) {
            for (auto& x : tm.ev)
                if (x) (void)hipEventDestroy(x);
            return fail(c, PRISM_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(he));
        }
    }
    const uint16_t* src = static_cast<const uint16_t*>(in);
    uint16_t* dst = static_cast<uint16_t*>(out);
    rc = timer_mark(c, &tm, -1, s);
    for (int j = 0; j < S && !rc; ++j) {
        const int f0 = (int)((int64_t)batch * j / S), f1 = (int)((int64_t)batch * (j + 1) / S);
        rc = enqueue_subchain(c, ws, j, f0, f1 - f0, src + f0 * T * D, dst + f0 * T * D, s, false, &tm);
    }
    if (rc) c->counts_dirty = true; /* launched part of the chain */
    double sum[2] = {0, 0};
    int cnt[2] = {0, 0};
    unsigned grid[2] = {0, 0};
    if (!rc) {
        const hipError_t he = hipEventSynchronize(tm.ev[tm.n - 1]);
        if (he != hipSuccess) rc = fail(c, PRISM_ERR_HIP, "hipEventSynchronize: %s", hipGetErrorString(he));
        for (size_t i = 1; i < tm.n && !rc; ++i) {
            float ms = 0.f;
            const hipError_t ee = hipEventElapsedTime(&ms, tm.ev[i - 1], tm.ev[i]);
            if (ee != hipSuccess) {
                rc = fail(c, PRISM_ERR_HIP, "hipEventElapsedTime: %s", hipGetErrorString(ee));
                break;
            }
            const int k = tm.kind[i - 1];
            sum[k] += ms;
            if (!cnt[k]++) grid[k] = tm.grid[i - 1];
        }
    }
    for (auto& e : tm.ev) (void)hipEventDestroy(e);
    if (rc) return rc;
    *attn_ms = (float)(sum[0] / std::max(1, cnt[0]));
    *expert_ms = (float)(sum[1] / std::max(1, cnt[1]));
    if (attn_grid) *attn_grid = (int32_t)grid[0];
    if (expert_grid) *expert_grid = (int32_t)grid[1];
    return PRISM_OK;
}

/* The eager chain with its workspace in this device's scratch array instead
 * of the context's allocation: no hipMalloc / hipFree, ever. The counter rows
 * are cleared by a fill launch first (the array keeps the previous call's
 * contents); everything else is written before it is read. Calls on one GPU,
 * from any context and stream, run one after another: the call's stream waits
 * for the device's completion event of the previous call, and the call
 * records it after its own launches (under a host lock, so concurrent callers
 * cannot interleave those steps). Under stream capture the wait and record
 * are left out (an event recorded outside a capture cannot be waited on
 * inside it): the captured graph's launches are then ordered by the stream the
 * caller replays it on. */
extern "C" int prism_forward_noalloc(prism_ctx* c, const void* in, void* out, int32_t batch, void* stream) {
    int rc = forward_checks(c, in, out, batch);
    if (rc) return rc;
    if (!c->scratch) return fail(c, PRISM_ERR_STATE, "no scratch array on device %d", c->device);
    const int64_t n = (int64_t)batch * c->desc.spatial_h * c->desc.spatial_w;
    if (!tokens_fit(n, c->desc.dim)) return fail(c, PRISM_ERR_INVALID, "%lld tokens is too many", (long long)n);
    const ChainLayout L = chain_layout(c->desc, n, false);
    if (L.bytes > PRISM_SCRATCH_BYTES)
        return fail(c, PRISM_ERR_INVALID,
                    "prism_forward_noalloc: batch %d of %dx%d tokens needs %zu bytes of workspace, more than the "
                    "%zu-byte scratch array (prism_forward allocates instead)",
                    batch, c->desc.spatial_h, c->desc.spatial_w, L.bytes, (size_t)PRISM_SCRATCH_BYTES);
    HIP_TRY(c, hipSetDevice(c->device));
    const hipStream_t s = (hipStream_t)stream;
    const ChainWs ws = chain_ws_at(c->scratch, L, n, false);
    const int N = c->desc.n_experts, NB = c->desc.n_blocks;
    const hipEvent_t done = scratch_done_event(c->device);
    if (!done) return fail(c, PRISM_ERR_STATE, "no scratch completion event on device %d", c->device);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(c, hipStreamIsCapturing(s, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(scratch_call_mutex(c->device));
    if (!capturing) HIP_TRY(c, hipStreamWaitEvent(s, done, 0));
    if (N > 1) {
        rc = enqueue_zero(c, ws.counts, CHAIN_SPLIT * NB * N * CHAIN_COUNT_STRIDE, s);
        if (rc) return rc;
    }
    rc = enqueue_forward_impl(c, ws, static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), batch, s);
    /* recorded even after a failed enqueue: the event then covers whatever
     * part of the chain was launched */
    if (!capturing) {
        const hipError_t e = hipEventRecord(done, s);
        if (!rc && e != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipEventRecord: %s", hipGetErrorString(e));
    }
    return rc;
}

extern "C" int prism_forward_assignments(prism_ctx* c, const int32_t** assign_dev, int64_t* tokens_per_block) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!c->fwd_assign) return fail(c, PRISM_ERR_STATE, "no forward has run");
    if (assign_dev) *assign_dev = c->fwd_assign;
    if (tokens_per_block) *tokens_per_block = c->fwd_tokens;
    return PRISM_OK;
}

/* ------------------------------------------------------------ host renderer interop */

extern "C" int prism_init_with_device(prism_ctx** out, int32_t device, void* stream, const char* code_object_path) {
    const int rc = prism_create(out, device, code_object_path);
    if (rc) return rc;
    prism_ctx* c = *out;
    if (stream) {
        int sdev = -1;
        const hipError_t e = hipStreamGetDevice((hipStream_t)stream, &sdev);
        if (e != hipSuccess || sdev != device) {
            prism_destroy(c);
            *out = nullptr;
            return fail(nullptr, PRISM_ERR_INVALID, "stream is not a stream of device %d (%s, device %d)", device,
                        hipGetErrorString(e), sdev);
        }
    }
    c->user_stream = (hipStream_t)stream;
    return PRISM_OK;
}

extern "C" int prism_infer_gpu(prism_ctx* c, const void* in_buf, uint64_t in_offset, void* out_buf,
                               uint64_t out_offset, int32_t batch, float* infer_ms) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!in_buf || !out_buf) return fail(c, PRISM_ERR_INVALID, "in_buf or out_buf is NULL");
    if (!c->loaded) return fail(c, PRISM_ERR_STATE, "weights not loaded");
    if (batch < 1) return fail(c, PRISM_ERR_INVALID, "batch %d < 1", batch);
    const int mode = c->adapters ? (c->codec ? CHAIN_E2E : CHAIN_ADAPTED) : CHAIN_BLOCKS;
    const uint64_t tok = (uint64_t)batch * c->desc.spatial_h * c->desc.spatial_w;
    uint64_t in_bytes = tok * (mode == CHAIN_ADAPTED ? c->aoffs.in_dim : c->desc.dim) * 2, out_bytes = in_bytes;
    if (mode == CHAIN_E2E) {
        in_bytes = (uint64_t)batch * codec_frame_elems(c) * 2;
        out_bytes = (uint64_t)batch * codec_display_elems(c) * 2;
    }
    const char* in = static_cast<const char*>(in_buf) + in_offset;
    char* out = static_cast<char*>(out_buf) + out_offset;
    if (in < out + out_bytes && out < in + in_bytes)
        return fail(c, PRISM_ERR_INVALID, "input and output ranges overlap (%llu / %llu bytes)",
                    (unsigned long long)in_bytes, (unsigned long long)out_bytes);
    int rc = run_forward_graph(c, in, out, batch, c->user_stream, mode, c->ev_t0);
    if (rc) return rc;
    HIP_TRY(c, hipEventRecord(c->ev_t1, c->user_stream));
    HIP_TRY(c, hipEventSynchronize(c->ev_t1));
    float ms = 0.f;
    HIP_TRY(c, hipEventElapsedTime(&ms, c->ev_t0, c->ev_t1));
    if (infer_ms) *infer_ms = ms;
    return PRISM_OK;
}

struct prism_external_buffer {
    hipExternalMemory_t mem;
    void* ptr;
    int fd;     /* the library's duplicate of the caller's descriptor */
    int device;
};

extern "C" int prism_import_external_memory(prism_ctx* c, int32_t fd, uint64_t size, prism_external_buffer** buf,
                                            void** dev_ptr) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!buf || !dev_ptr) return fail(c, PRISM_ERR_INVALID, "buf or dev_ptr is NULL");
    *buf = nullptr;
    *dev_ptr = nullptr;
    if (fd < 0) return fail(c, PRISM_ERR_INVALID, "fd %d is not a descriptor", fd);
    if (size == 0) return fail(c, PRISM_ERR_INVALID, "size is 0");
    const int dfd = fcntl(fd, F_DUPFD_CLOEXEC, 0);
    if (dfd < 0) return fail(c, PRISM_ERR_INVALID, "fd %d: %s", fd, strerror(errno));
    hipError_t e = hipSetDevice(c->device);
    hipExternalMemory_t mem = nullptr;
    if (e == hipSuccess) {
        hipExternalMemoryHandleDesc d;
        memset(&d, 0, sizeof d);
        d.type = hipExternalMemoryHandleTypeOpaqueFd;
        d.handle.fd = dfd;
        d.size = size;
        e = hipImportExternalMemory(&mem, &d);
    }
    if (e != hipSuccess) {
        close(dfd);
        return fail(c, PRISM_ERR_HIP, "hipImportExternalMemory(fd %d, %llu bytes): %s", fd, (unsigned long long)size,
                    hipGetErrorString(e));
    }
    hipExternalMemoryBufferDesc bd;
    memset(&bd, 0, sizeof bd);
    bd.offset = 0;
    bd.size = size;
    void* p = nullptr;
    e = hipExternalMemoryGetMappedBuffer(&p, mem, &bd);
    if (e != hipSuccess || !p) {
        (void)hipDestroyExternalMemory(mem);
        close(dfd);
        return fail(c, PRISM_ERR_HIP, "hipExternalMemoryGetMappedBuffer: %s", hipGetErrorString(e));
    }
    *buf = new prism_external_buffer{mem, p, dfd, c->device};
    *dev_ptr = p;
    return PRISM_OK;
}

extern "C" int prism_release_external_memory(prism_ctx* c, prism_external_buffer* b) {
    if (!c) return fail(nullptr, PRISM_ERR_INVALID, "context is NULL");
    if (!b) return fail(c, PRISM_ERR_INVALID, "buffer is NULL");
    HIP_TRY(c, hipSetDevice(b->device));
    /* work still reading or writing the buffer must end before its mapping does */
    const hipError_t es = hipDeviceSynchronize();
    const hipError_t ef = hipFree(b->ptr);
    const hipError_t ed = hipDestroyExternalMemory(b->mem);
    close(b->fd);
    delete b;
    if (es != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipDeviceSynchronize: %s", hipGetErrorString(es));
    if (ef != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipFree(mapped buffer): %s", hipGetErrorString(ef));
    if (ed != hipSuccess) return fail(c, PRISM_ERR_HIP, "hipDestroyExternalMemory: %s", hipGetErrorString(ed));
    return PRISM_OK;
}
