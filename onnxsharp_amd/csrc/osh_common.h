// osh_common.h -- shared host/device helpers of libosh_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

#include "../../include/osh_hip.h"

namespace osh {

// ------------------------------------------------------------------ errors

// Records `msg` as this thread's last error and returns `code`.
osh_status fail(osh_status code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define OSH_HIP_CHECK(expr)                                                                         \
    do {                                                                                            \
        hipError_t e_ = (expr);                                                                     \
        if (e_ != hipSuccess)                                                                       \
            return ::osh::fail(OSH_E_DEVICE, "%s failed: %s", #expr, hipGetErrorString(e_));       \
    } while (0)

// Checks a kernel launch (launch configuration errors surface here).
#define OSH_LAUNCH_CHECK(name)                                                                      \
    do {                                                                                            \
        hipError_t e_ = hipGetLastError();                                                          \
        if (e_ != hipSuccess)                                                                       \
            return ::osh::fail(OSH_E_DEVICE, "%s launch failed: %s", name, hipGetErrorString(e_)); \
    } while (0)

inline hipStream_t to_stream(osh_stream s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------- MFMA types

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------ activations

// exp(x) by the reference's own polynomial (src/OnnxSharp/Tensors/VectorMath.cs:21-43):
// clamp to [-87.3, 88.7], n = rne(x*log2e), r by a two-term ln2 split, degree-6
// Horner, 2^n from the exponent bits.  Bit-identical to the AVX2 path for
// identical inputs: every step is a single IEEE op or an fma.
__device__ __forceinline__ float exp_ref(float x) {
    x = __builtin_fminf(__builtin_fmaxf(x, -87.3f), 88.7f);
    float n = __builtin_rintf(x * 1.4426950408889634f);
    float r = __builtin_fmaf(n, -0.693145751953125f, x);
    r = __builtin_fmaf(n, -1.4286067653e-6f, r);
    float p = 1.0f / 720.0f;
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int bits = ((int)n + 127) << 23;
    return p * __int_as_float(bits);
}

// SiLU of VectorMath.Silu (VectorMath.cs:70-77): x * (1 / (1 + exp(x * -1))),
// with an IEEE division (the build keeps correctly rounded f32 division).
__device__ __forceinline__ float silu_ref(float x) {
    float e = exp_ref(x * -1.0f);
    return x * (1.0f / (1.0f + e));
}

// TensorOps.Apply Relu (TensorOps.cs:951): x > 0 ? x : 0 (NaN -> 0).
__device__ __forceinline__ float relu_ref(float x) { return x > 0.0f ? x : 0.0f; }

template <int ACT>
__device__ __forceinline__ float activate(float x) {
    if constexpr (ACT == OSH_ACT_SILU) return silu_ref(x);
    else if constexpr (ACT == OSH_ACT_RELU) return relu_ref(x);
    else return x;
}

// Dispatch a runtime activation code to a template instantiation.
#define OSH_DISPATCH_ACT(act, ACT, ...)                      \
    switch (act) {                                           \
    case OSH_ACT_NONE: { constexpr int ACT = OSH_ACT_NONE; __VA_ARGS__; } break; \
    case OSH_ACT_RELU: { constexpr int ACT = OSH_ACT_RELU; __VA_ARGS__; } break; \
    case OSH_ACT_SILU: { constexpr int ACT = OSH_ACT_SILU; __VA_ARGS__; } break; \
    default: return ::osh::fail(OSH_E_INVALID, "unknown activation %d", act); \
    }

inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace osh
