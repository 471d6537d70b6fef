// A host program bound to the C ABI (include/prism.h, libprism.so) the way the
// reference's C++ host would call it: build a model description, lay out and
// fill the fp16 blob, then (with a GPU) run the reference's per-block stage
// sequence (attn -> router -> experts, prism_moe_bench.cpp:266-289) and the
// captured chain, and check that both give the same bits.
// Usage: abi_host_program [gpu]   prints "ABI OK ..." on success, exit code 0.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <vector>

#include "prism.h"

#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            std::fprintf(stderr, "FAIL: " __VA_ARGS__);    \
            std::fprintf(stderr, "\n");                    \
            return 1;                                      \
        }                                                  \
    } while (0)

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
    // MoE-64 blocks at a small grid (the layout does not depend on the grid)
    prism_model_desc d{256, 2, 8, 32, 64, 20, 28, 8};
    std::vector<prism_block_offsets> offs(d.n_blocks);
    int64_t elems = 0;
    CHECK(prism_layout(&d, offs.data(), &elems) == PRISM_OK, "prism_layout");
    CHECK(offs[1].ln1_g > offs[0].exp_b2 && offs[0].exp_stride == 2 * 256 * 256 + 2 * 256, "layout order");
    std::vector<uint16_t> blob(elems);
    CHECK(prism_synth_weights(&d, 7, PRISM_ROUTE_ZIPF, blob.data(), elems, offs.data()) == PRISM_OK, "synth");
    CHECK(prism_validate(&d, offs.data(), elems) == PRISM_OK, "validate");
    CHECK(prism_validate(&d, offs.data(), elems - 8) != PRISM_OK, "validate must reject a short blob");
    // fragment layout: element (row 17, col 40) of a 32x64 matrix sits in
    // fragment (rt 1, ks 1), lane 1 + 16 * 1, slot 0
    std::vector<uint16_t> w(32 * 64), packed(32 * 64);
    for (int i = 0; i < 32 * 64; ++i) w[i] = (uint16_t)i;
    CHECK(prism_pack_weight(w.data(), 32, 64, 32, packed.data()) == PRISM_OK, "pack");
    CHECK(packed[(1 * 2 + 1) * 512 + (1 + 16) * 8 + 0] == 17 * 64 + 40, "pack layout");
    const int64_t T = (int64_t)d.spatial_h * d.spatial_w;
    const int64_t aux_n = prism_aux_elems(d.n_experts, T);
    CHECK(aux_n == T + d.n_experts + d.n_experts * T, "aux size %lld", (long long)aux_n);

    prism_ctx* ctx = nullptr;
    const int rc = prism_create(&ctx, 0, nullptr);
    if (!gpu) { // without a GPU the call fails cleanly and says why
        if (rc != PRISM_OK) {
            CHECK(ctx == nullptr && std::strlen(prism_last_error(nullptr)) > 0, "error message");
            std::printf("ABI OK (host only; prism_create: %d %s)\n", rc, prism_last_error(nullptr));
        } else {
            prism_destroy(ctx);
            std::printf("ABI OK (host only; a device is present)\n");
        }
        return 0;
    }
    CHECK(rc == PRISM_OK, "prism_create: %s", prism_last_error(nullptr));
    CHECK(prism_load_weights(ctx, &d, blob.data(), blob.size() * 2, offs.data()) == PRISM_OK, "load: %s",
          prism_last_error(ctx));

    // features arena: [x | h | y] fp16 rows, aux arena: assignment, counts, perm
    const int64_t D = d.dim, n = T;
    std::vector<uint16_t> x(n * D);
    CHECK(prism_synth_normal_f16(x.data(), n * D, 1, 0, 1.0f) == PRISM_OK, "inputs");
    void *feat = nullptr, *aux = nullptr, *in = nullptr, *out = nullptr;
    CHECK(hipMalloc(&feat, 3 * n * D * 2) == hipSuccess && hipMalloc(&aux, aux_n * 4) == hipSuccess &&
              hipMalloc(&in, n * D * 2) == hipSuccess && hipMalloc(&out, n * D * 2) == hipSuccess,
          "hipMalloc");
    CHECK(hipMemcpy(feat, x.data(), n * D * 2, hipMemcpyHostToDevice) == hipSuccess, "upload");
    CHECK(hipMemcpy(in, x.data(), n * D * 2, hipMemcpyHostToDevice) == hipSuccess, "upload");
    int64_t cur = 0, nxt = 2 * n * D;
    for (int b = 0; b < d.n_blocks; ++b) {
        const prism_block_offsets& o = offs[b];
        prism_attn_push pa{(int32_t)T, d.dim, d.n_heads, d.head_dim, d.spatial_w, d.spatial_h, d.window,
                           o.qkv_w, o.qkv_b, o.out_w, o.out_b, cur, n * D, o.ln1_g, o.ln1_b};
        prism_router_push pr{(int32_t)T, d.dim, d.n_experts, o.router_w, o.router_b, n * D,
                             0, T, o.ln2_g, o.ln2_b, T + d.n_experts};
        prism_expert_push pe{(int32_t)T, d.dim, d.n_experts, o.exp_w1, o.exp_b1, o.exp_w2, o.exp_b2,
                             o.exp_stride, n * D, nxt, 0, T, o.ln2_g, o.ln2_b, T + d.n_experts};
        CHECK(prism_attn(ctx, &pa, feat, 1, nullptr) == PRISM_OK, "attn: %s", prism_last_error(ctx));
        CHECK(prism_router(ctx, &pr, feat, (int32_t*)aux, 1, nullptr) == PRISM_OK, "router: %s",
              prism_last_error(ctx));
        CHECK(prism_experts(ctx, &pe, feat, (int32_t*)aux, 1, nullptr) == PRISM_OK, "experts: %s",
              prism_last_error(ctx));
        const int64_t t = cur;
        cur = nxt;
        nxt = t;
    }
    CHECK(prism_forward_graph(ctx, in, out, 1, nullptr) == PRISM_OK, "forward: %s", prism_last_error(ctx));
    CHECK(hipDeviceSynchronize() == hipSuccess, "sync");
    std::vector<uint16_t> y_stage(n * D), y_chain(n * D);
    CHECK(hipMemcpy(y_stage.data(), (uint16_t*)feat + cur, n * D * 2, hipMemcpyDeviceToHost) == hipSuccess, "dl");
    CHECK(hipMemcpy(y_chain.data(), out, n * D * 2, hipMemcpyDeviceToHost) == hipSuccess, "dl");
    int64_t differ = 0;
    for (int64_t i = 0; i < n * D; ++i) differ += y_stage[i] != y_chain[i];
    CHECK(differ == 0, "%lld values differ between the stage calls and the chain", (long long)differ);
    prism_destroy(ctx);
    (void)hipFree(feat);
    (void)hipFree(aux);
    (void)hipFree(in);
    (void)hipFree(out);
    std::printf("ABI OK (stage calls == chain over %d blocks, %lld values)\n", d.n_blocks, (long long)(n * D));
    return 0;
}
