// osh_eltwise.hip -- elementwise and data-movement passes of the C ABI.
//
// osh_activation_f32 is the standalone form of the activation epilogue that
// the GEMM/conv kernels fuse (TensorOps.ElementWiseUnary,
// src/OnnxSharp/Tensors/TensorOps.cs:267-300): Relu and the reference SiLU.
// The rest are the segment-continuity ops that keep a YOLO-style network on
// the device between convolutions: residual Add, MaxPool, nearest Resize,
// Transpose and the attention Softmax.  All are HBM-bound; each thread moves
// a handful of values with coalesced accesses.
#include "osh_common.h"

using namespace osh;

namespace osh {

// MathF.Max: NaN if either operand is NaN; +0 over -0.
__device__ __forceinline__ float dotnet_max(float a, float b) {
    if (a != a || b != b) return __builtin_nanf("");
    if (a > b) return a;
    if (b > a) return b;
    return __builtin_signbitf(a) ? b : a;  // equal: +0 over -0
}

template <int ACT>
__global__ __launch_bounds__(256) void activation_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                          long long n) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) y[i] = activate<ACT>(x[i]);
}

__global__ __launch_bounds__(256) void add_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                                   float *__restrict__ y, long long n) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) y[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void add4_kernel(const float4 *__restrict__ a, const float4 *__restrict__ b,
                                                    float4 *__restrict__ y, long long n4) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n4; i += stride) {
        const float4 u = a[i], v = b[i];
        y[i] = make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
    }
}

// One thread per output element.  The comparison of the reference's scalar
// path (MaxPoolLayer.Forward, src/OnnxSharp/Ops/DnnOps.cs:1564-1579): the
// maximum starts at -inf and takes an in-range element only when it is
// greater, so NaN inputs are skipped.  (The reference's 8-wide path uses
// Vector256.Max, whose NaN result depends on the operand order; for inputs
// without NaN both paths give the same bits.)
__global__ __launch_bounds__(256) void maxpool2d_kernel(osh_pool_params p, const float *__restrict__ x,
                                                         float *__restrict__ y, long long total) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int ox = (int)(idx % p.ow);
    long long t = idx / p.ow;
    const int oy = (int)(t % p.oh);
    const long long plane = t / p.oh;
    const float *xp = x + plane * p.h * p.w;
    const int iy0 = oy * p.sh - p.pt, ix0 = ox * p.sw - p.pl;
    float m = -__builtin_inff();
    for (int ky = 0; ky < p.kh; ky++) {
        const int iy = iy0 + ky;
        if ((unsigned)iy >= (unsigned)p.h) continue;
        for (int kx = 0; kx < p.kw; kx++) {
            const int ix = ix0 + kx;
            if ((unsigned)ix >= (unsigned)p.w) continue;
            const float v = xp[(long long)iy * p.w + ix];
            if (v > m) m = v;
        }
    }
    y[idx] = m;
}

// Three chained k x k, stride 1, pad k/2 max pools (SPPF: y1 = pool(x),
// y2 = pool(y1), y3 = pool(y2)) in one launch.  A workgroup owns a PT x PT
// tile of one plane: it stages x over the tile plus a 3r halo in LDS (-inf
// outside the image), then derives y1 over the tile plus 2r, y2 over the
// tile plus r and y3 over the tile, each level as a row pass then a column
// pass (outputs outside the image are set to -inf for the next level).
// Every max is the comparison of maxpool2d_kernel (start at -inf, take v only
// when v > max): with rows taken in order and each row's columns in order,
// the two passes keep the first of equal maxima in row-major order exactly as
// the k x k scan does, never take a NaN, and a -inf pad is never taken; so
// the chain is bit-identical to three separate pools.
template <int K>
__global__ __launch_bounds__(256) void maxpool_chain3_kernel(int h, int w, int c, const float *__restrict__ x,
                                                             long long x_bstride, float *__restrict__ y1,
                                                             float *__restrict__ y2, float *__restrict__ y3,
                                                             long long y_bstride, int tiles_x) {
    constexpr int PT = 16, R = K / 2;
    constexpr int S0 = PT + 6 * R, S1 = PT + 4 * R, S2 = PT + 2 * R;
    __shared__ float l0[S0 * S0], l1[S1 * S1], l2[S2 * S2], tmp[S0 * S1];
    const int plane = blockIdx.y;  // n * c + channel
    const int n = plane / c, ch = plane - n * c;
    const int ty = blockIdx.x / tiles_x, tx = blockIdx.x - ty * tiles_x;
    const int oy0 = ty * PT, ox0 = tx * PT;
    const long long xoff = (long long)n * x_bstride + (long long)ch * h * w;
    const long long yoff = (long long)n * y_bstride + (long long)ch * h * w;
    const float *xp = x + xoff;
    const float ninf = -__builtin_inff();
    for (int e = threadIdx.x; e < S0 * S0; e += 256) {
        const int i = e / S0, jx = e - i * S0;
        const int iy = oy0 - 3 * R + i, ix = ox0 - 3 * R + jx;
        l0[e] = ((unsigned)iy < (unsigned)h && (unsigned)ix < (unsigned)w) ? xp[(long long)iy * w + ix] : ninf;
    }
    __syncthreads();
    // dst (SD x SD, origin o - DR) from src ((SD + 2R) x (SD + 2R))
    auto level = [&](const float *src, float *dst, int SD, int DR) {
        const int SS = SD + 2 * R;
        for (int e = threadIdx.x; e < SS * SD; e += 256) {  // row pass: SS rows x SD columns
            const int i = e / SD, jx = e - i * SD;
            float m = ninf;
#pragma unroll
            for (int kx = 0; kx < K; kx++) {
                const float v = src[i * SS + jx + kx];
                if (v > m) m = v;
            }
            tmp[e] = m;
        }
        __syncthreads();
        for (int e = threadIdx.x; e < SD * SD; e += 256) {  // column pass
            const int i = e / SD, jx = e - i * SD;
            const int py = oy0 - DR + i, px = ox0 - DR + jx;
            float m = ninf;
#pragma unroll
            for (int ky = 0; ky < K; ky++) {
                const float v = tmp[(i + ky) * SD + jx];
                if (v > m) m = v;
            }
            dst[e] = ((unsigned)py < (unsigned)h && (unsigned)px < (unsigned)w) ? m : ninf;
        }
        __syncthreads();
    };
    level(l0, l1, S1, 2 * R);
    level(l1, l2, S2, R);
    level(l2, l0, PT, 0);  // y3 over the tile, into the (free) x buffer
    for (int e = threadIdx.x; e < PT * PT; e += 256) {
        const int i = e / PT, jx = e - i * PT;
        const int py = oy0 + i, px = ox0 + jx;
        if (py >= h || px >= w) continue;
        const long long o = yoff + (long long)py * w + px;
        y1[o] = l1[(i + 2 * R) * S1 + jx + 2 * R];
        y2[o] = l2[(i + R) * S2 + jx + R];
        y3[o] = l0[i * PT + jx];
    }
}

// DflSoftmax, one thread per (image, side, pixel): three passes over the
// pixel's bins (max; sum of exponentials; weighted sum), the exponentials
// recomputed (same bits) rather than stored.  `tail` marks the columns the
// reference handles on its scalar lines: the last (width % 8) of each block
// of 256 pixels.

__global__ __launch_bounds__(256) void dfl_kernel(int sides, int bins, int pixels, const float *__restrict__ x,
                                                  long long x_bs, float *__restrict__ y, long long y_bs,
                                                  long long total) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int n = (int)(idx % pixels);
    const long long t = idx / pixels;
    const int side = (int)(t % sides);
    const long long img = t / sides;
    const float *src = x + img * x_bs + (long long)side * bins * pixels + n;
    const int col = n % 256;
    const int width = min(256, pixels - (n - col));
    const bool tail = col >= (width & ~7);
    float m = -__builtin_inff();
    for (int b = 0; b < bins; b++) {
        const float v = src[(long long)b * pixels];
        m = tail ? dotnet_max(m, v) : (m > v ? m : v);  // Avx.Max(max, row) keeps the row value unless max > row
    }
    float sum = 0.0f;
    for (int b = 0; b < bins; b++) sum = sum + exp_ref(src[(long long)b * pixels] - m);
    const float inv = 1.0f / sum;
    float w = 0.0f;
    for (int b = 0; b < bins; b++) {
        const float p = exp_ref(src[(long long)b * pixels] - m) * inv;
        if (tail) {
            const float prod = p * (float)b;
            w = w + prod;
        } else {
            w = __builtin_fmaf(p, (float)b, w);
        }
    }
    y[img * y_bs + (long long)side * pixels + n] = w;
}

__global__ __launch_bounds__(256) void resize_nearest_kernel(int c, int h, int w, int fh, int fw,
                                                              const float *__restrict__ x, float *__restrict__ y,
                                                              long long y_batch_stride, long long total) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int ow = w * fw, oh = h * fh;
    const int ox = (int)(idx % ow);
    long long t = idx / ow;
    const int oy = (int)(t % oh);
    t /= oh;
    const int ch = (int)(t % c);
    const long long n = t / c;
    const float v = x[((n * c + ch) * h + oy / fh) * (long long)w + ox / fw];
    y[n * y_batch_stride + ((long long)ch * oh + oy) * ow + ox] = v;
}

// The 2x case with an even input width: a thread reads two neighbouring
// input pixels (8 bytes) and writes the four output pixels of each of its two
// output rows as one 16-byte store, with 32-bit indices.
__global__ __launch_bounds__(256) void resize2x_kernel(int c, int h, int w2, const float2 *__restrict__ x,
                                                       float *__restrict__ y, long long y_batch_stride, int total) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int ix = idx % w2;  // pair of input columns 2 ix, 2 ix + 1
    int t = idx / w2;
    const int iy = t % h;
    t /= h;
    const int ch = t % c, n = t / c;
    const float2 v = x[idx];
    const int ow = 4 * w2;
    float *row = y + n * y_batch_stride + ((long long)ch * 2 * h + 2 * iy) * ow + 4 * ix;
    const float4 o = make_float4(v.x, v.x, v.y, v.y);
    *reinterpret_cast<float4 *>(row) = o;
    *reinterpret_cast<float4 *>(row + ow) = o;
}

// 32 x 32 tiles through LDS so that both the read and the write are coalesced.
__global__ __launch_bounds__(256) void transpose_kernel(int rows, int cols, const float *__restrict__ x,
                                                         long long xs, float *__restrict__ y, long long ys) {
    __shared__ float tile[32][33];
    const float *xb = x + blockIdx.z * xs;
    float *yb = y + blockIdx.z * ys;
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int gr = r0 + r, gc = c0 + tx;
        if (gr < rows && gc < cols) tile[r][tx] = xb[(long long)gr * cols + gc];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int gc = c0 + r, gr = r0 + tx;  // output row gc, column gr
        if (gc < cols && gr < rows) yb[(long long)gc * rows + gr] = tile[tx][r];
    }
}

__device__ __forceinline__ float wave_max_f(float v) {
    for (int o = 32; o > 0; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}


// VectorMath.SoftmaxRow (src/OnnxSharp/Tensors/VectorMath.cs:172-204,246-287)
// on v = x * scale (the Mul node before the Softmax rounds it), summed in its
// order: the reference's eight float lanes each add the exponentials of
// v[8j + k] in order of j; the eight lane sums are added to 0 in lane order,
// then the (cols % 8) tail values; y = e * (1 / sum).
//   The max only enters through (v - max), whose exponential does not depend
// on how equal candidates (+0 / -0) were ordered, so any order gives the
// same bits for inputs without NaN (NaN inputs: not pinned).
// One wave per row: all lanes compute the exponentials into the wave's LDS row
// (SOFTMAX_LDS_COLS at most; longer rows use the row of y itself), lanes 0-7
// form the lane sums from it, lane 0 the total.
constexpr int SOFTMAX_LDS_COLS = 4096;

template <bool LDS>
__global__ __launch_bounds__(256) void softmax_kernel(long long rows, int cols, float scale,
                                                      const float *__restrict__ x, float *__restrict__ y) {
    extern __shared__ float srow[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * 4 + wave;
    const bool live = row < rows;
    const float *xr = x + (live ? row : 0) * cols;
    float *yr = y + (live ? row : 0) * cols;
    float *buf = LDS ? srow + wave * cols : yr;
    float m = -__builtin_inff();
    if (live)
        for (int c = lane; c < cols; c += 64) m = __builtin_fmaxf(m, xr[c] * scale);
    m = wave_max_f(m);
    if (live)
        for (int c = lane; c < cols; c += 64) buf[c] = exp_ref(xr[c] * scale - m);
    if (LDS) __syncthreads();
    else __threadfence();  // the lane sums read values other lanes wrote to y
    const int vec = cols & ~7;
    float part = 0.0f;
    if (live && lane < 8)
        for (int i = lane; i < vec; i += 8) part = part + buf[i];
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; q++) sum = sum + __shfl(part, q);
    if (live && lane == 0)
        for (int i = vec; i < cols; i++) sum = sum + buf[i];
    const float inv = 1.0f / __shfl(sum, 0);
    if (live)
        for (int c = lane; c < cols; c += 64) yr[c] = buf[c] * inv;
}

static unsigned grid_for(long long n, long long per_block, long long cap) {
    long long b = (n + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return (unsigned)b;
}

}  // namespace osh

extern "C" {

OSH_API osh_status osh_add_f32(int64_t n, const float *d_a, const float *d_b, float *d_y, osh_stream s) {
    if (n < 0) return fail(OSH_E_INVALID, "Add: negative element count");
    if (n == 0) return OSH_OK;
    if (!d_a || !d_b || !d_y) return fail(OSH_E_INVALID, "Add: NULL pointer");
    const bool vec = n % 4 == 0 && ((reinterpret_cast<uintptr_t>(d_a) | reinterpret_cast<uintptr_t>(d_b) |
                                     reinterpret_cast<uintptr_t>(d_y)) & 15) == 0;
    if (vec) {
        OSH_LAUNCH(add4_kernel, dim3(grid_for(n / 4, 256, 8192)), dim3(256), 0, to_stream(s),
                           reinterpret_cast<const float4 *>(d_a), reinterpret_cast<const float4 *>(d_b),
                           reinterpret_cast<float4 *>(d_y), (long long)(n / 4));
    } else {
        OSH_LAUNCH(add_kernel, dim3(grid_for(n, 256, 8192)), dim3(256), 0, to_stream(s), d_a, d_b, d_y,
                           (long long)n);
    }
    OSH_LAUNCH_CHECK("add_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_maxpool2d_f32(const osh_pool_params *p, const float *d_x, float *d_y, osh_stream s) {
    if (!p || !d_x || !d_y) return fail(OSH_E_INVALID, "MaxPool: NULL argument");
    if (p->n <= 0 || p->c <= 0 || p->h <= 0 || p->w <= 0 || p->kh <= 0 || p->kw <= 0 || p->sh <= 0 || p->sw <= 0 ||
        p->oh <= 0 || p->ow <= 0 || p->pt < 0 || p->pl < 0)
        return fail(OSH_E_INVALID, "MaxPool: bad parameters");
    // every window must hold at least one input element
    if ((long long)(p->oh - 1) * p->sh - p->pt >= p->h || (long long)(p->ow - 1) * p->sw - p->pl >= p->w ||
        p->kh <= p->pt || p->kw <= p->pl)
        return fail(OSH_E_INVALID, "MaxPool: output window outside the input");
    const long long total = (long long)p->n * p->c * p->oh * p->ow;
    OSH_LAUNCH(maxpool2d_kernel, dim3(grid_for(total, 256, 0x7fffffff)), dim3(256), 0, to_stream(s), *p,
                       d_x, d_y, total);
    OSH_LAUNCH_CHECK("maxpool2d_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_maxpool_chain3_f32(int n, int c, int h, int w, int k, const float *d_x, int64_t x_batch_stride,
                                          float *d_y1, float *d_y2, float *d_y3, int64_t y_batch_stride,
                                          osh_stream s) {
    if (n <= 0 || c <= 0 || h <= 0 || w <= 0) return fail(OSH_E_INVALID, "MaxPool chain: bad sizes");
    if (k != 3 && k != 5 && k != 7) return fail(OSH_E_UNSUPPORTED, "MaxPool chain: kernel %d (3, 5 or 7 supported)", k);
    if (!d_x || !d_y1 || !d_y2 || !d_y3) return fail(OSH_E_INVALID, "MaxPool chain: NULL pointer");
    const long long plane = (long long)c * h * w;
    if (x_batch_stride < plane || y_batch_stride < plane)
        return fail(OSH_E_INVALID, "MaxPool chain: batch stride below c*h*w");
    if ((long long)n * c > 65535) return fail(OSH_E_UNSUPPORTED, "MaxPool chain: more than 65535 planes");
    const int tiles_x = (w + 15) / 16, tiles_y = (h + 15) / 16;
    if ((long long)tiles_x * tiles_y > 0x7fffffff) return fail(OSH_E_UNSUPPORTED, "MaxPool chain: image too large");
    dim3 grid((unsigned)(tiles_x * tiles_y), (unsigned)(n * c));
    hipStream_t st = to_stream(s);
    if (k == 3)
        OSH_LAUNCH(maxpool_chain3_kernel<3>, grid, dim3(256), 0, st, h, w, c, d_x, (long long)x_batch_stride,
                           d_y1, d_y2, d_y3, (long long)y_batch_stride, tiles_x);
    else if (k == 5)
        OSH_LAUNCH(maxpool_chain3_kernel<5>, grid, dim3(256), 0, st, h, w, c, d_x, (long long)x_batch_stride,
                           d_y1, d_y2, d_y3, (long long)y_batch_stride, tiles_x);
    else
        OSH_LAUNCH(maxpool_chain3_kernel<7>, grid, dim3(256), 0, st, h, w, c, d_x, (long long)x_batch_stride,
                           d_y1, d_y2, d_y3, (long long)y_batch_stride, tiles_x);
    OSH_LAUNCH_CHECK("maxpool_chain3_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_dfl_f32(int batches, int sides, int bins, int pixels, const float *d_x,
                               int64_t x_batch_stride, float *d_y, int64_t y_batch_stride, osh_stream s) {
    if (batches <= 0 || sides <= 0 || pixels <= 0) return fail(OSH_E_INVALID, "DflSoftmax: bad sizes");
    if (bins < 2) return fail(OSH_E_INVALID, "DflSoftmax: bins=%d (need at least 2)", bins);
    if (!d_x || !d_y) return fail(OSH_E_INVALID, "DflSoftmax: NULL pointer");
    if (x_batch_stride < (long long)sides * bins * pixels || y_batch_stride < (long long)sides * pixels)
        return fail(OSH_E_INVALID, "DflSoftmax: batch stride below one image");
    const long long total = (long long)batches * sides * pixels;
    if (total > 0x7fffffffLL * 256) return fail(OSH_E_UNSUPPORTED, "DflSoftmax: too many outputs");
    OSH_LAUNCH(dfl_kernel, dim3(grid_for(total, 256, 0x7fffffff)), dim3(256), 0, to_stream(s), sides, bins,
                       pixels, d_x, (long long)x_batch_stride, d_y, (long long)y_batch_stride, total);
    OSH_LAUNCH_CHECK("dfl_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_resize_nearest_f32(int n, int c, int h, int w, int fh, int fw, const float *d_x, float *d_y,
                                          int64_t y_batch_stride, osh_stream s) {
    if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || fh <= 0 || fw <= 0) return fail(OSH_E_INVALID, "Resize: bad sizes");
    if (!d_x || !d_y) return fail(OSH_E_INVALID, "Resize: NULL pointer");
    const long long plane = (long long)c * h * fh * w * fw;
    if (y_batch_stride < plane) return fail(OSH_E_INVALID, "Resize: output batch stride below c*oh*ow");
    const long long total = (long long)n * plane;
    const long long pairs = (long long)n * c * h * w / 2;
    if (fh == 2 && fw == 2 && w % 2 == 0 && pairs < (1LL << 31) && y_batch_stride % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(d_x) & 7) == 0 && (reinterpret_cast<uintptr_t>(d_y) & 15) == 0) {
        OSH_LAUNCH(resize2x_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, to_stream(s), c, h,
                           w / 2, reinterpret_cast<const float2 *>(d_x), d_y, (long long)y_batch_stride, (int)pairs);
        OSH_LAUNCH_CHECK("resize2x_kernel");
        return OSH_OK;
    }
    OSH_LAUNCH(resize_nearest_kernel, dim3(grid_for(total, 256, 0x7fffffff)), dim3(256), 0, to_stream(s), c,
                       h, w, fh, fw, d_x, d_y, (long long)y_batch_stride, total);
    OSH_LAUNCH_CHECK("resize_nearest_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_transpose_f32(int batch, int rows, int cols, const float *d_x, int64_t x_batch_stride,
                                     float *d_y, int64_t y_batch_stride, osh_stream s) {
    if (batch < 0 || rows < 0 || cols < 0) return fail(OSH_E_INVALID, "Transpose: negative size");
    if (batch == 0 || rows == 0 || cols == 0) return OSH_OK;
    if (!d_x || !d_y) return fail(OSH_E_INVALID, "Transpose: NULL pointer");
    if (batch > 65535) return fail(OSH_E_UNSUPPORTED, "Transpose: batch %d exceeds the grid limit", batch);
    dim3 grid(ceil_div(cols, 32), ceil_div(rows, 32), batch);
    if (grid.y > 65535) return fail(OSH_E_UNSUPPORTED, "Transpose: %d rows exceed the grid limit", rows);
    OSH_LAUNCH(transpose_kernel, grid, dim3(256), 0, to_stream(s), rows, cols, d_x, (long long)x_batch_stride,
                       d_y, (long long)y_batch_stride);
    OSH_LAUNCH_CHECK("transpose_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_softmax_f32(int64_t rows, int cols, float scale, const float *d_x, float *d_y, osh_stream s) {
    if (rows < 0 || cols < 0) return fail(OSH_E_INVALID, "Softmax: negative size");
    if (rows == 0 || cols == 0) return OSH_OK;
    if (!d_x || !d_y) return fail(OSH_E_INVALID, "Softmax: NULL pointer");
    if (d_x == d_y) return fail(OSH_E_INVALID, "Softmax: in-place is not supported");
    if (cols <= SOFTMAX_LDS_COLS)
        OSH_LAUNCH(softmax_kernel<true>, dim3(grid_for(rows, 4, 0x7fffffff)), dim3(256),
                           (size_t)4 * cols * sizeof(float), to_stream(s), (long long)rows, cols, scale, d_x, d_y);
    else
        OSH_LAUNCH(softmax_kernel<false>, dim3(grid_for(rows, 4, 0x7fffffff)), dim3(256), 0, to_stream(s),
                           (long long)rows, cols, scale, d_x, d_y);
    OSH_LAUNCH_CHECK("softmax_kernel");
    return OSH_OK;
}

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
        OSH_LAUNCH(activation_kernel<OSH_ACT_NONE>, dim3((unsigned)blocks), dim3(256), 0, to_stream(s), d_x,
                           d_y, (long long)n);
        break;
    case OSH_ACT_RELU:
        OSH_LAUNCH(activation_kernel<OSH_ACT_RELU>, dim3((unsigned)blocks), dim3(256), 0, to_stream(s), d_x,
                           d_y, (long long)n);
        break;
    case ACT_SILU_EXACT:
        OSH_LAUNCH(activation_kernel<ACT_SILU_EXACT>, dim3((unsigned)blocks), dim3(256), 0, to_stream(s), d_x,
                           d_y, (long long)n);
        break;
    case OSH_ACT_SIGMOID:
        OSH_LAUNCH(activation_kernel<OSH_ACT_SIGMOID>, dim3((unsigned)blocks), dim3(256), 0, to_stream(s),
                           d_x, d_y, (long long)n);
        break;
    default:
        return fail(OSH_E_INVALID, "unknown activation %d", act);
    }
    OSH_LAUNCH_CHECK("activation_kernel");
    return OSH_OK;
}

}  // extern "C"
