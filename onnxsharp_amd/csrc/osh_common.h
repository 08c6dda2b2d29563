// osh_common.h -- shared host/device helpers of libosh_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <mutex>
#include <string>

#include "osh_hip.h"

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

// ------------------------------------------------------------- launch log

// Notes one kernel launch of the calling thread (the kernel's host-side
// handle); osh_kernel_log names them, so a caller can tell which kernel and
// tile each call ran after first-use tuning.
void note_launch(const void *kernel);

// Every kernel launch of the library goes through this macro.
#define OSH_LAUNCH(K, ...)                                                                          \
    do {                                                                                            \
        ::osh::note_launch(reinterpret_cast<const void *>(&(K)));                                   \
        hipLaunchKernelGGL(K, __VA_ARGS__);                                                         \
    } while (0)

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

// SiLU for fused GEMM/conv epilogues: x / (1 + 2^(-x log2 e)) with the hardware
// exp2 and a reciprocal refined by one Newton step (6 VALU instead of ~30 for
// silu_ref).  The exponent is clamped at 126 so the denominator stays finite;
// the relative difference to silu_ref is a few 1e-7 for |x| < 20 and ~1e-6 at
// the clamp, far inside the 1e-4 parity bar of the FP32 outputs it feeds.
__device__ __forceinline__ float silu_fast(float x) {
    float t = __builtin_fminf(x * -1.4426950408889634f, 126.0f);
    float d = 1.0f + __builtin_amdgcn_exp2f(t);
    float r = __builtin_amdgcn_rcpf(d);
    r = __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
    return x * r;
}

// Sigmoid of VectorMath.Sigmoid (VectorMath.cs:64-68): 1 / (1 + exp(x * -1)).
__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + exp_ref(x * -1.0f)); }

// TensorOps.Apply Relu (TensorOps.cs:951): x > 0 ? x : 0 (NaN -> 0).
__device__ __forceinline__ float relu_ref(float x) { return x > 0.0f ? x : 0.0f; }

// Internal activation code: the reference SiLU polynomial in a fused epilogue
// (chosen by osh_config_set("exact_silu", 1) or ONNXSHARP_HIP_EXACT_SILU=1).
constexpr int ACT_SILU_EXACT = 103;

template <int ACT>
__device__ __forceinline__ float activate(float x) {
    if constexpr (ACT == OSH_ACT_SILU) return silu_fast(x);
    else if constexpr (ACT == ACT_SILU_EXACT) return silu_ref(x);
    else if constexpr (ACT == OSH_ACT_RELU) return relu_ref(x);
    else if constexpr (ACT == OSH_ACT_SIGMOID) return sigmoid_ref(x);
    else return x;
}

bool exact_silu();

// Workgroups are dealt to the eight XCDs round-robin by linear id, and each
// XCD has its own L2.  xcd_band(L, G) renumbers workgroup L of a grid of G so
// that the workgroups of one XCD take one contiguous band of ids: XCD
// x = L % 8 takes ids [x q + min(x, r), ...) with q = G / 8, r = G % 8 -- a
// bijection on [0, G).  Neighbouring tiles, which share input lines and
// weights, then meet in the same L2.
__device__ __forceinline__ int xcd_band(int L, int G) {
    const int x = L & 7, k = L >> 3, q = G >> 3, r = G & 7;
    return x * q + (x < r ? x : r) + k;
}

// Compute units of the current device (256 on MI355X).
inline int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

// Forced gemm16 wave tile (-1 = automatic, -2 = LDS-staged tile only) and
// the number of wave tiles.
int gemm_variant();
int gemm16_variant_count();

// Forced conv16 wave tile for 3x3 convolutions (-1 = automatic, -2 = use the
// weight-stationary kernels instead) and the number of tiles.
int conv16_variant();
int conv16_variant_count();

// Forced tile for 1x1 convolutions with C % 16 == 0 (-1 = automatic, 0 = the
// GEMM tile over raw weights, 1.. = the LDS-tile kernel, -2 = the GEMM path
// only, weights packed raw) and the number of choices.
int pointwise_variant();
int pointwise_variant_count();

// Drops the record of which kernel a packed conv weight buffer at d_ptr was
// laid out for (osh_free calls it; the address may be reused).
void forget_pack(const void *d_ptr);
// Device address of the no-allocation DynamicQuantizeMatMul's static scratch
// on device dev (osh_dqmm.hip), resolved once per device.
osh_status noalloc_scratch_setup(int dev);

// Forced LDS-patch tile for the 3x3 convolutions that run in the im2col
// order (-1 = automatic) and the number of tiles.
int im2col3x3_variant();
int im2col3x3_variant_count();

// Forced tile of the grouped 3x3 launches (-1 = first-use timing) and the
// number of tiles (the LDS-patch tiles).
int group3x3_tile();
int group3x3_tile_count();
// The same for grouped pointwise launches (the pointwise LDS tiles).
int group_pointwise_tile();
int group_pointwise_tile_count();
// Forced tile of the fused 3x3 pair (-1 = first-use timing).
int pair_tile();

// Winograd F(2x2,3x3) for 3x3 stride-1 convolutions (0 = never, 1 = where
// the reference's NCHWc kernel does not apply, 2 = ahead of the NCHWc
// kernels) and the largest output map it takes (H*W; the reference's
// ONNXSHARP_WINO_MAX, default 4096).
int winograd_mode();
long long winograd_max_pixels();

// Whether the host the backend stands in for runs OnnxSharp's NCHWc 3x3
// kernel (an AVX-512 host with ONNXSHARP_NCHWC not "0", NchwcConv.cs:38-43).
// Off, the 3x3 convs the NCHWc gate would take go where the reference then
// sends them: Winograd, else the panel / im2col chain.
bool nchwc_enabled();

// DynamicQuantizeMatMul pipeline (0 = min/max launch then one fused
// quantize + GEMM launch, 1 = min/max, quantize and GEMM as three launches).
int dqmm_variant();
// Kernel launches of the calling thread's last DynamicQuantizeMatMul (2 or 3).
int dqmm_last_launches();

// Whether kernels whose tiles all give identical results may pick their tile
// by timing it on first use (osh_config "tune", ONNXSHARP_HIP_TUNE; default on).
bool tuning_enabled();

// Dispatch a runtime activation code to a template instantiation of a fused epilogue.
#define OSH_DISPATCH_ACT(act, ACT, ...)                      \
    switch (act) {                                           \
    case OSH_ACT_NONE: { constexpr int ACT = OSH_ACT_NONE; __VA_ARGS__; } break; \
    case OSH_ACT_RELU: { constexpr int ACT = OSH_ACT_RELU; __VA_ARGS__; } break; \
    case OSH_ACT_SILU:                                       \
        if (::osh::exact_silu()) { constexpr int ACT = ::osh::ACT_SILU_EXACT; __VA_ARGS__; } \
        else { constexpr int ACT = OSH_ACT_SILU; __VA_ARGS__; } \
        break;                                               \
    default: return ::osh::fail(OSH_E_INVALID, "unknown activation %d", act); \
    }

inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace osh
