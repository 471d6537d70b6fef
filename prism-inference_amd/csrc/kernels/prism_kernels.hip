/*
 * prism_kernels.hip - the gfx950 code object (prism_kernels.hsaco) loaded by
 * the host engine with hipModuleLoad and launched with hipModuleLaunchKernel.
 *
 * Kernels (extern "C" names, one per stage and supported shape):
 *   prism_attn_d{256,128}[_w8]                     attention stage (4 or 8 waves)
 *   prism_attn_d{256,128}[_w8]_r{1..4}             attention + fused routing
 *   prism_router_d{256,128}_n{1..4}                router + counting sort
 *   prism_expert_d{256,128}_bm64[_w8], _d256_bm{128,96}  grouped expert FFN
 *   prism_project_{up,down}_d{256,128}             projection adapters (128 <-> dim)
 *   prism_codec_enc{0..3}, prism_codec_dec{3,2}    conv encoder / fused decoder stages
 *   prism_codec_dec1_out                           dec1 + output conv + PixelShuffle + sigmoid
 *   prism_zero_i32                                 clears routing counters
 *   prism_take_counts                              strided counters -> contiguous (stage calls)
 */
#include "attn.hpp"
#include "router.hpp"
#include "expert.hpp"
#include "project.hpp"
#include "codec.hpp"

/* Routing counters must start at zero; a kernel (not a memset node) keeps
 * the launch safe under stream capture. */
extern "C" __global__ void __launch_bounds__(256) prism_zero_i32(int32_t* p, int32_t n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}

/* Strided counters -> a contiguous array, each counter cleared behind the
 * read (the stage call's private counters start the next call at zero). */
extern "C" __global__ void __launch_bounds__(64) prism_take_counts(int32_t* src, int32_t stride, int32_t* dst,
                                                                   int32_t n) {
    const int i = threadIdx.x;
    if (i < n) {
        dst[i] = src[i * stride];
        src[i * stride] = 0;
    }
}
