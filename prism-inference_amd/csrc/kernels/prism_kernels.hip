/*
 * prism_kernels.hip - the gfx950 code object (prism_kernels.hsaco) loaded by
 * the host engine with hipModuleLoad and launched with hipModuleLaunchKernel.
 *
 * Kernels (extern "C" names, one per stage and supported shape):
 *   prism_attn_d256 / prism_attn_d128              attention stage
 *   prism_router_d256 / prism_router_d128          router + counting sort
 *   prism_expert_d{256,128}_bm64                   grouped expert FFN
 *   prism_zero_i32                                 clears the router counts
 */
#include "attn.hpp"
#include "router.hpp"
#include "expert.hpp"

/* The router stage's counts must start at zero; a kernel (not a memset node)
 * keeps the launch safe under stream capture. */
extern "C" __global__ void __launch_bounds__(256) prism_zero_i32(int32_t* p, int32_t n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}
