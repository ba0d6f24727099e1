// z2h_tp.hip — the token-pair K-split kernels (k_gemv_split<WF_Q8_0, ..., TP = true>: Q8_0 matmuls of
// one or two tokens, the single-stream step's projections and expert matmuls) in a translation unit of
// their own. z2h.hip declares them extern; compiled here, they leave the code layout of the library's
// other kernels as it is.
#define Z2H_TEMPLATES_ONLY
#include "z2h_kernels.h"

namespace z2d {
template __global__ void k_gemv_split<WF_Q8_0, true, MT_G, false, true>(GemvArgs);
template __global__ void k_gemv_split<WF_Q8_0, false, MT_G, false, true>(GemvArgs);
template __global__ void k_gemv_split<WF_Q8_0, true, MT, false, true>(GemvArgs);
template __global__ void k_gemv_split<WF_Q8_0, false, MT, false, true>(GemvArgs);
template __global__ void k_gemv_split<WF_Q8_0, false, MT_G, true, true>(GemvArgs);
} // namespace z2d
