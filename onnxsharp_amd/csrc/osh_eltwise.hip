// osh_eltwise.hip -- elementwise passes of the C ABI.
//
// osh_activation_f32 is the standalone form of the activation epilogue that
// the GEMM/conv kernels fuse (TensorOps.ElementWiseUnary,
// src/OnnxSharp/Tensors/TensorOps.cs:267-300): Relu and the reference SiLU.
#include "osh_common.h"

using namespace osh;

namespace osh {

template <int ACT>
__global__ __launch_bounds__(256) void activation_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                          long long n) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) y[i] = activate<ACT>(x[i]);
}

}  // namespace osh

extern "C" {

OSH_API osh_status osh_activation_f32(int64_t n, const float *d_x, int act, float *d_y, osh_stream s) {
    if (n < 0) return fail(OSH_E_INVALID, "negative element count");
    if (n == 0) return OSH_OK;
    if (!d_x || !d_y) return fail(OSH_E_INVALID, "NULL pointer");
    long long blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    // the standalone pass is TensorOps.ElementWiseUnary itself: always the reference SiLU
    const int a = act == OSH_ACT_SILU ? ACT_SILU_EXACT : act;
    switch (a) {
    case OSH_ACT_NONE:
        hipLaunchKernelGGL(activation_kernel<OSH_ACT_NONE>, dim3((unsigned)blocks), dim3(256), 0, to_stream(s), d_x,
                           d_y, (long long)n);
        break;
    case OSH_ACT_RELU:
        hipLaunchKernelGGL(activation_kernel<OSH_ACT_RELU>, dim3((unsigned)blocks), dim3(256), 0, to_stream(s), d_x,
                           d_y, (long long)n);
        break;
    case ACT_SILU_EXACT:
        hipLaunchKernelGGL(activation_kernel<ACT_SILU_EXACT>, dim3((unsigned)blocks), dim3(256), 0, to_stream(s), d_x,
                           d_y, (long long)n);
        break;
    default:
        return fail(OSH_E_INVALID, "unknown activation %d", act);
    }
    OSH_LAUNCH_CHECK("activation_kernel");
    return OSH_OK;
}

}  // extern "C"
