/*
 * prism_kernels.hip - the gfx950 code object (prism_kernels.hsaco) loaded by
 * the host engine with hipModuleLoad and launched with hipModuleLaunchKernel.
 *
 * Kernels (extern "C" names, one per stage and supported shape):
 *   prism_attn_d256 / prism_attn_d128              attention stage
 *   prism_router_d256 / prism_router_d128          router + counting sort
 *   prism_expert_d{256,128}_bm{128,64}             grouped expert FFN
 */
#include "attn.hpp"
#include "router.hpp"
#include "expert.hpp"
