// osh_runtime.hip -- device, memory, copies, streams, events and errors of
// the C ABI (include/osh_hip.h).  Replaces the Vulkan runtime layer of the
// reference backend (src/OnnxSharp.Vulkan/VkDevice.cs, VkBufferPool.cs,
// VkSegment.cs) with plain HIP calls.
#include <cxxabi.h>

#include <cstdarg>
#include <cstdlib>
#include <cstring>

#include <vector>

#include "osh_common.h"
#include "osh_conv_pair.h"

namespace osh {

static thread_local char g_err[512] = "";

osh_status fail(osh_status code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = 0; }

const char *last_error() { return g_err; }

// Kernels launched by the calling thread since its last osh_kernel_log reset
// (bounded: launches past the bound are counted, not kept).
static constexpr size_t kLaunchLogMax = 4096;
static thread_local std::vector<const void *> t_launch_log;
static thread_local long long t_launch_count = 0;

void note_launch(const void *kernel) {
    if (t_launch_log.size() < kLaunchLogMax) t_launch_log.push_back(kernel);
    ++t_launch_count;
}

// "name<args>" of a kernel's host handle: its device symbol demangled, without
// the return type and the parameter list (the form rocprofv3 prints).
static std::string kernel_name(const void *kernel) {
    const char *mangled = hipKernelNameRefByPtr(kernel, nullptr);
    if (!mangled) {
        (void)hipGetLastError();
        return "?";
    }
    int status = 0;
    char *dem = abi::__cxa_demangle(mangled, nullptr, nullptr, &status);
    std::string s = (status == 0 && dem) ? dem : mangled;
    free(dem);
    if (s.compare(0, 5, "void ") == 0) s.erase(0, 5);
    if (s.compare(0, 5, "osh::") == 0) s.erase(0, 5);
    int depth = 0;
    for (size_t i = 0; i < s.size(); ++i) {
        if (s[i] == '<') ++depth;
        else if (s[i] == '>') --depth;
        else if (s[i] == '(' && depth == 0) {
            s.resize(i);
            break;
        }
    }
    return s;
}

static int g_exact_silu = -1;  // -1: read ONNXSHARP_HIP_EXACT_SILU on first use
static int g_gemm_variant = -3;  // -3: read ONNXSHARP_HIP_GEMM_VARIANT on first use
static int g_conv16_variant = -3;  // -3: read ONNXSHARP_HIP_CONV16_VARIANT on first use
static int g_tune = -1;             // -1: read ONNXSHARP_HIP_TUNE on first use
static int g_pw_variant = -3;       // -3: read ONNXSHARP_HIP_POINTWISE_VARIANT on first use
static int g_dqmm_variant = -3;     // -3: read ONNXSHARP_HIP_DQMM_VARIANT on first use
static int g_winograd = -3;         // -3: read ONNXSHARP_HIP_WINOGRAD on first use
static int g_nchwc = -3;            // -3: read ONNXSHARP_NCHWC on first use
static int g_i2c_variant = -3;      // -3: read ONNXSHARP_HIP_IM2COL3X3_VARIANT on first use
static int g_group3x3_tile = -1;    // forced tile of grouped 3x3 launches (-1: first-use timing)
static int g_group_pw_tile = -1;    // forced tile of grouped pointwise launches (-1: first-use timing)
static int g_pair_tile = -1;        // forced tile of the fused 3x3 pair (-1: first-use timing)
static long long g_wino_max = -3;   // -3: read ONNXSHARP_WINO_MAX on first use

bool exact_silu() {
    if (g_exact_silu < 0) {
        const char *e = getenv("ONNXSHARP_HIP_EXACT_SILU");
        g_exact_silu = (e && atoi(e) != 0) ? 1 : 0;
    }
    return g_exact_silu == 1;
}

int gemm_variant() {
    if (g_gemm_variant == -3) {
        const char *e = getenv("ONNXSHARP_HIP_GEMM_VARIANT");
        g_gemm_variant = e ? atoi(e) : -1;
    }
    return g_gemm_variant;
}

bool tuning_enabled() {
    if (g_tune < 0) {
        const char *e = getenv("ONNXSHARP_HIP_TUNE");
        g_tune = (e && atoi(e) == 0) ? 0 : 1;
    }
    return g_tune == 1;
}

int conv16_variant() {
    if (g_conv16_variant == -3) {
        const char *e = getenv("ONNXSHARP_HIP_CONV16_VARIANT");
        g_conv16_variant = e ? atoi(e) : -1;
    }
    return g_conv16_variant;
}

int pointwise_variant() {
    if (g_pw_variant == -3) {
        const char *e = getenv("ONNXSHARP_HIP_POINTWISE_VARIANT");
        g_pw_variant = e ? atoi(e) : -1;
    }
    return g_pw_variant;
}

int im2col3x3_variant() {
    if (g_i2c_variant == -3) {
        const char *e = getenv("ONNXSHARP_HIP_IM2COL3X3_VARIANT");
        g_i2c_variant = e ? atoi(e) : -1;
    }
    return g_i2c_variant;
}

int group3x3_tile() { return g_group3x3_tile; }
int group_pointwise_tile() { return g_group_pw_tile; }
int pair_tile() { return g_pair_tile; }

int winograd_mode() {
    if (g_winograd == -3) {
        const char *e = getenv("ONNXSHARP_HIP_WINOGRAD");
        const int v = e ? atoi(e) : 1;
        g_winograd = (v >= 0 && v <= 2) ? v : 1;
    }
    return g_winograd;
}

bool nchwc_enabled() {
    if (g_nchwc == -3) {
        // the reference's own switch (NchwcConv.cs:38-40): anything but "0" keeps it on
        const char *e = getenv("ONNXSHARP_NCHWC");
        g_nchwc = (e && strcmp(e, "0") == 0) ? 0 : 1;
    }
    return g_nchwc == 1;
}

long long winograd_max_pixels() {
    if (g_wino_max == -3) {
        // the reference's own knob (Winograd.cs:38-40): a number, else 4096
        const char *e = getenv("ONNXSHARP_WINO_MAX");
        char *end = nullptr;
        const long long v = e ? strtoll(e, &end, 10) : 0;
        g_wino_max = (e && end != e && *end == 0) ? v : 4096;
    }
    return g_wino_max;
}

int dqmm_variant() {
    if (g_dqmm_variant == -3) {
        const char *e = getenv("ONNXSHARP_HIP_DQMM_VARIANT");
        const int v = e ? atoi(e) : 0;
        g_dqmm_variant = (v == 1 || v == 2) ? v : 0;
    }
    return g_dqmm_variant;
}

__global__ void fill_u8_kernel(uint8_t *__restrict__ p, uint8_t v, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

}  // namespace osh

using namespace osh;

extern "C" {

OSH_API const char *osh_last_error(void) { return osh::last_error(); }

OSH_API osh_status osh_config_set(const char *key, int value) {
    if (!key) return fail(OSH_E_INVALID, "key is NULL");
    if (strcmp(key, "exact_silu") == 0) {
        g_exact_silu = value != 0;
        return OSH_OK;
    }
    if (strcmp(key, "tune") == 0) {
        g_tune = value != 0;
        return OSH_OK;
    }
    if (strcmp(key, "conv16_variant") == 0) {
        if (value < -1 || value >= conv16_variant_count())
            return fail(OSH_E_INVALID, "conv16_variant %d out of range [-1, %d)", value, conv16_variant_count());
        g_conv16_variant = value;
        return OSH_OK;
    }
    if (strcmp(key, "pointwise_variant") == 0) {
        if (value < -2 || value >= pointwise_variant_count())
            return fail(OSH_E_INVALID, "pointwise_variant %d out of range [-2, %d)", value, pointwise_variant_count());
        g_pw_variant = value;
        return OSH_OK;
    }
    if (strcmp(key, "gemm_variant") == 0) {
        if (value < -2 || value >= gemm16_variant_count())
            return fail(OSH_E_INVALID, "gemm_variant %d out of range [-2, %d)", value, gemm16_variant_count());
        g_gemm_variant = value;
        return OSH_OK;
    }
    if (strcmp(key, "im2col3x3_variant") == 0) {
        if (value < -1 || value >= im2col3x3_variant_count())
            return fail(OSH_E_INVALID, "im2col3x3_variant %d out of range [-1, %d)", value,
                        im2col3x3_variant_count());
        g_i2c_variant = value;
        return OSH_OK;
    }
    if (strcmp(key, "group3x3_tile") == 0) {
        if (value < -1 || value >= group3x3_tile_count())
            return fail(OSH_E_INVALID, "group3x3_tile %d out of range [-1, %d)", value, group3x3_tile_count());
        g_group3x3_tile = value;
        return OSH_OK;
    }
    if (strcmp(key, "pair_tile") == 0) {
        if (value < -1 || value > conv_pair_tile_count())
            return fail(OSH_E_INVALID, "pair_tile %d out of range [-1, %d]", value, conv_pair_tile_count());
        g_pair_tile = value;
        return OSH_OK;
    }
    if (strcmp(key, "group_pointwise_tile") == 0) {
        if (value < -1 || value >= group_pointwise_tile_count())
            return fail(OSH_E_INVALID, "group_pointwise_tile %d out of range [-1, %d)", value,
                        group_pointwise_tile_count());
        g_group_pw_tile = value;
        return OSH_OK;
    }
    if (strcmp(key, "winograd") == 0) {
        if (value < 0 || value > 2) return fail(OSH_E_INVALID, "winograd %d out of range [0, 2]", value);
        g_winograd = value;
        return OSH_OK;
    }
    if (strcmp(key, "winograd_max_pixels") == 0) {
        g_wino_max = value;
        return OSH_OK;
    }
    if (strcmp(key, "nchwc") == 0) {
        if (value != 0 && value != 1) return fail(OSH_E_INVALID, "nchwc %d: 0 or 1", value);
        g_nchwc = value;
        return OSH_OK;
    }
    if (strcmp(key, "dqmm_variant") == 0) {
        if (value < 0 || value > 2) return fail(OSH_E_INVALID, "dqmm_variant %d out of range [0, 3)", value);
        g_dqmm_variant = value;
        return OSH_OK;
    }
    return fail(OSH_E_INVALID, "unknown option '%s'", key);
}

OSH_API osh_status osh_config_get(const char *key, int *value) {
    if (!key || !value) return fail(OSH_E_INVALID, "NULL argument");
    if (strcmp(key, "exact_silu") == 0) {
        *value = exact_silu() ? 1 : 0;
        return OSH_OK;
    }
    if (strcmp(key, "gemm_variant") == 0) {
        *value = gemm_variant();
        return OSH_OK;
    }
    if (strcmp(key, "conv16_variant") == 0) {
        *value = conv16_variant();
        return OSH_OK;
    }
    if (strcmp(key, "pointwise_variant") == 0) {
        *value = pointwise_variant();
        return OSH_OK;
    }
    if (strcmp(key, "im2col3x3_variant") == 0) {
        *value = im2col3x3_variant();
        return OSH_OK;
    }
    if (strcmp(key, "im2col3x3_variants") == 0) {
        *value = im2col3x3_variant_count();
        return OSH_OK;
    }
    if (strcmp(key, "group3x3_tile") == 0) {
        *value = group3x3_tile();
        return OSH_OK;
    }
    if (strcmp(key, "group3x3_tiles") == 0) {
        *value = group3x3_tile_count();
        return OSH_OK;
    }
    if (strcmp(key, "group_pointwise_tile") == 0) {
        *value = group_pointwise_tile();
        return OSH_OK;
    }
    if (strcmp(key, "pair_tile") == 0) {
        *value = pair_tile();
        return OSH_OK;
    }
    if (strcmp(key, "pair_tiles") == 0) {
        *value = conv_pair_tile_count() + 1;
        return OSH_OK;
    }
    if (strcmp(key, "group_pointwise_tiles") == 0) {
        *value = group_pointwise_tile_count();
        return OSH_OK;
    }
    if (strcmp(key, "winograd") == 0) {
        *value = winograd_mode();
        return OSH_OK;
    }
    if (strcmp(key, "nchwc") == 0) {
        *value = nchwc_enabled() ? 1 : 0;
        return OSH_OK;
    }
    if (strcmp(key, "winograd_max_pixels") == 0) {
        const long long v = winograd_max_pixels();
        *value = v > 2147483647LL ? 2147483647 : (v < -2147483647LL ? -2147483647 : (int)v);
        return OSH_OK;
    }
    if (strcmp(key, "dqmm_variant") == 0) {
        *value = dqmm_variant();
        return OSH_OK;
    }
    if (strcmp(key, "dqmm_launches") == 0) {
        *value = dqmm_last_launches();
        return OSH_OK;
    }
    if (strcmp(key, "pointwise_variants") == 0) {
        *value = pointwise_variant_count();
        return OSH_OK;
    }
    if (strcmp(key, "conv16_variants") == 0) {
        *value = conv16_variant_count();
        return OSH_OK;
    }
    if (strcmp(key, "tune") == 0) {
        *value = tuning_enabled() ? 1 : 0;
        return OSH_OK;
    }
    if (strcmp(key, "gemm_variants") == 0) {
        *value = gemm16_variant_count();
        return OSH_OK;
    }
    return fail(OSH_E_INVALID, "unknown option '%s'", key);
}

OSH_API osh_status osh_device_count(int *count) {
    if (!count) return fail(OSH_E_INVALID, "count is NULL");
    OSH_HIP_CHECK(hipGetDeviceCount(count));
    return OSH_OK;
}

OSH_API osh_status osh_init(int dev, osh_device_info *info) {
    int n = 0;
    OSH_HIP_CHECK(hipGetDeviceCount(&n));
    if (dev < 0 || dev >= n) return fail(OSH_E_INVALID, "device %d out of range (%d devices)", dev, n);
    hipDeviceProp_t p;
    OSH_HIP_CHECK(hipGetDeviceProperties(&p, dev));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(OSH_E_UNSUPPORTED, "device %d is %s; this library is built for gfx950 only", dev,
                    p.gcnArchName);
    OSH_HIP_CHECK(hipSetDevice(dev));
    if (info) {
        memset(info, 0, sizeof(*info));
        strncpy(info->name, p.name, sizeof(info->name) - 1);
        strncpy(info->arch, p.gcnArchName, sizeof(info->arch) - 1);
        info->compute_units = p.multiProcessorCount;
        info->clock_khz = p.clockRate;
        info->total_mem = p.totalGlobalMem;
        info->lds_per_block = p.sharedMemPerBlock;
    }
    // The no-allocation DQM's scratch address is resolved here when it can be;
    // if not, osh_dqmm_u8s8_noalloc resolves it (and reports why it cannot) on
    // its first call, and nothing else depends on it.
    if (noalloc_scratch_setup(dev) != OSH_OK) clear_error();
    return OSH_OK;
}

OSH_API osh_status osh_kernel_log(int reset, char *buf, size_t bytes, int *count) {
    if (count) *count = (int)t_launch_count;
    if (buf && bytes) {
        std::string all;
        for (const void *k : t_launch_log) {
            all += kernel_name(k);
            all += '\n';
        }
        if (all.size() + 1 > bytes)
            return fail(OSH_E_INVALID, "buffer of %zu bytes holds fewer than the %zu the log needs", bytes,
                        all.size() + 1);
        memcpy(buf, all.c_str(), all.size() + 1);
    }
    if (reset) {
        t_launch_log.clear();
        t_launch_count = 0;
    }
    return OSH_OK;
}

OSH_API osh_status osh_device_synchronize(void) {
    OSH_HIP_CHECK(hipDeviceSynchronize());
    return OSH_OK;
}

OSH_API osh_status osh_malloc(void **d_ptr, size_t bytes) {
    if (!d_ptr) return fail(OSH_E_INVALID, "d_ptr is NULL");
    *d_ptr = nullptr;
    if (bytes == 0) return OSH_OK;
    hipError_t e = hipMalloc(d_ptr, bytes);
    if (e != hipSuccess) {
        // a failed allocation is reported here and nowhere else: clear the
        // runtime's sticky last error so the caller's next HIP call does not
        // see it again
        (void)hipGetLastError();
        *d_ptr = nullptr;
        return fail(OSH_E_NOMEM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    }
    return OSH_OK;
}

OSH_API osh_status osh_free(void *d_ptr) {
    if (d_ptr) forget_pack(d_ptr);
    if (d_ptr) OSH_HIP_CHECK(hipFree(d_ptr));
    return OSH_OK;
}

OSH_API osh_status osh_host_alloc(void **h_ptr, size_t bytes) {
    if (!h_ptr) return fail(OSH_E_INVALID, "h_ptr is NULL");
    *h_ptr = nullptr;
    if (bytes == 0) return OSH_OK;
    hipError_t e = hipHostMalloc(h_ptr, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *h_ptr = nullptr;
        return fail(OSH_E_NOMEM, "hipHostMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    }
    return OSH_OK;
}

OSH_API osh_status osh_host_free(void *h_ptr) {
    if (h_ptr) OSH_HIP_CHECK(hipHostFree(h_ptr));
    return OSH_OK;
}

static osh_status copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, osh_stream s) {
    if (bytes == 0) return OSH_OK;
    if (!dst || !src) return fail(OSH_E_INVALID, "NULL pointer in copy of %zu bytes", bytes);
    OSH_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, kind, to_stream(s)));
    return OSH_OK;
}

OSH_API osh_status osh_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes, osh_stream s) {
    return copy(d_dst, h_src, bytes, hipMemcpyHostToDevice, s);
}

OSH_API osh_status osh_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes, osh_stream s) {
    return copy(h_dst, d_src, bytes, hipMemcpyDeviceToHost, s);
}

OSH_API osh_status osh_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes, osh_stream s) {
    return copy(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, s);
}

OSH_API osh_status osh_memset_d8(void *d_dst, int value, size_t bytes, osh_stream s) {
    if (bytes == 0) return OSH_OK;
    if (!d_dst) return fail(OSH_E_INVALID, "d_dst is NULL");
    size_t blocks = (bytes + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    OSH_LAUNCH(fill_u8_kernel, dim3((unsigned)blocks), dim3(256), 0, to_stream(s), (uint8_t *)d_dst,
                       (uint8_t)value, bytes);
    OSH_LAUNCH_CHECK("fill_u8_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_stream_create(osh_stream *s) {
    if (!s) return fail(OSH_E_INVALID, "s is NULL");
    hipStream_t st;
    OSH_HIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = st;
    return OSH_OK;
}

OSH_API osh_status osh_stream_destroy(osh_stream s) {
    if (s) OSH_HIP_CHECK(hipStreamDestroy(to_stream(s)));
    return OSH_OK;
}

OSH_API osh_status osh_stream_sync(osh_stream s) {
    OSH_HIP_CHECK(hipStreamSynchronize(to_stream(s)));
    return OSH_OK;
}

OSH_API osh_status osh_event_create(osh_event *e) {
    if (!e) return fail(OSH_E_INVALID, "e is NULL");
    hipEvent_t ev;
    OSH_HIP_CHECK(hipEventCreate(&ev));
    *e = ev;
    return OSH_OK;
}

OSH_API osh_status osh_event_destroy(osh_event e) {
    if (e) OSH_HIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(e)));
    return OSH_OK;
}

OSH_API osh_status osh_event_record(osh_event e, osh_stream s) {
    if (!e) return fail(OSH_E_INVALID, "e is NULL");
    OSH_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(e), to_stream(s)));
    return OSH_OK;
}

OSH_API osh_status osh_event_elapsed_ms(osh_event start, osh_event stop, float *ms) {
    if (!start || !stop || !ms) return fail(OSH_E_INVALID, "NULL argument");
    OSH_HIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
    OSH_HIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
    return OSH_OK;
}

OSH_API osh_status osh_stream_wait_event(osh_stream s, osh_event e) {
    if (!e) return fail(OSH_E_INVALID, "e is NULL");
    OSH_HIP_CHECK(hipStreamWaitEvent(to_stream(s), reinterpret_cast<hipEvent_t>(e), 0));
    return OSH_OK;
}

OSH_API osh_status osh_graph_begin(osh_stream s) {
    if (!s) return fail(OSH_E_INVALID, "graph capture needs a stream from osh_stream_create");
    OSH_HIP_CHECK(hipStreamBeginCapture(to_stream(s), hipStreamCaptureModeThreadLocal));
    return OSH_OK;
}

OSH_API osh_status osh_graph_end(osh_stream s, osh_graph *g) {
    if (!s || !g) return fail(OSH_E_INVALID, "NULL argument");
    *g = nullptr;
    hipGraph_t graph = nullptr;
    OSH_HIP_CHECK(hipStreamEndCapture(to_stream(s), &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(OSH_E_DEVICE, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
    *g = exec;
    return OSH_OK;
}

OSH_API osh_status osh_graph_launch(osh_graph g, osh_stream s) {
    if (!g) return fail(OSH_E_INVALID, "graph is NULL");
    OSH_HIP_CHECK(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(g), to_stream(s)));
    return OSH_OK;
}

OSH_API osh_status osh_graph_destroy(osh_graph g) {
    if (g) OSH_HIP_CHECK(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(g)));
    return OSH_OK;
}

OSH_API osh_status osh_graph_builder_create(osh_graph_builder *b) {
    if (!b) return fail(OSH_E_INVALID, "NULL argument");
    hipGraph_t g = nullptr;
    OSH_HIP_CHECK(hipGraphCreate(&g, 0));
    *b = g;
    return OSH_OK;
}

OSH_API osh_status osh_graph_add_captured(osh_graph_builder b, osh_stream s, const osh_graph_node *deps, int ndeps,
                                          osh_graph_node *node) {
    if (!b || !s || !node || ndeps < 0 || (ndeps > 0 && !deps)) return fail(OSH_E_INVALID, "bad argument");
    *node = nullptr;
    hipGraph_t child = nullptr;
    OSH_HIP_CHECK(hipStreamEndCapture(to_stream(s), &child));
    hipGraphNode_t n = nullptr;
    hipError_t e = hipGraphAddChildGraphNode(&n, reinterpret_cast<hipGraph_t>(b),
                                             reinterpret_cast<const hipGraphNode_t *>(deps), (size_t)ndeps, child);
    (void)hipGraphDestroy(child);  // the node holds its own copy
    if (e != hipSuccess) return fail(OSH_E_DEVICE, "hipGraphAddChildGraphNode failed: %s", hipGetErrorString(e));
    *node = n;
    return OSH_OK;
}

OSH_API osh_status osh_graph_add_captured_flat(osh_graph_builder b, osh_stream s, const osh_graph_node *deps,
                                               int ndeps, osh_graph_node *first, osh_graph_node *last) {
    if (!b || !s || !first || !last || ndeps < 0 || (ndeps > 0 && !deps)) return fail(OSH_E_INVALID, "bad argument");
    *first = *last = nullptr;
    hipGraph_t seg = nullptr;
    OSH_HIP_CHECK(hipStreamEndCapture(to_stream(s), &seg));
    // the capture of one stream is a chain: one root, at most one dependent
    // per node, every node a kernel launch
    std::vector<hipGraphNode_t> chain;
    const char *why = nullptr;
    size_t nroots = 0;
    if (hipGraphGetRootNodes(seg, nullptr, &nroots) != hipSuccess) why = "hipGraphGetRootNodes failed";
    else if (nroots > 1) why = "the capture is not one chain";
    if (!why && nroots == 1) {
        hipGraphNode_t node = nullptr;
        size_t one = 1;
        if (hipGraphGetRootNodes(seg, &node, &one) != hipSuccess) why = "hipGraphGetRootNodes failed";
        while (!why && node) {
            hipGraphNodeType t;
            if (hipGraphNodeGetType(node, &t) != hipSuccess || t != hipGraphNodeTypeKernel) {
                why = "the capture holds a node that is not a kernel launch";
                break;
            }
            chain.push_back(node);
            size_t nd = 0;
            if (hipGraphNodeGetDependentNodes(node, nullptr, &nd) != hipSuccess) why = "dependent query failed";
            else if (nd > 1) why = "the capture is not one chain";
            else if (nd == 0) node = nullptr;
            else if (hipGraphNodeGetDependentNodes(node, &node, &nd) != hipSuccess) why = "dependent query failed";
        }
    }
    if (why) {
        (void)hipGraphDestroy(seg);
        return fail(OSH_E_UNSUPPORTED, "flat graph: %s", why);
    }
    // copy the kernel nodes (their parameter values are copied at creation)
    hipGraph_t g = reinterpret_cast<hipGraph_t>(b);
    hipGraphNode_t prev = nullptr;
    for (size_t i = 0; i < chain.size(); i++) {
        hipKernelNodeParams kp{};
        hipError_t e = hipGraphKernelNodeGetParams(chain[i], &kp);
        hipGraphNode_t nn = nullptr;
        if (e == hipSuccess) {
            if (i == 0) e = hipGraphAddKernelNode(&nn, g, reinterpret_cast<const hipGraphNode_t *>(deps), (size_t)ndeps, &kp);
            else e = hipGraphAddKernelNode(&nn, g, &prev, 1, &kp);
        }
        if (e != hipSuccess) {
            (void)hipGraphDestroy(seg);
            return fail(OSH_E_DEVICE, "flat graph: kernel node copy failed: %s", hipGetErrorString(e));
        }
        if (i == 0) *first = nn;
        prev = nn;
    }
    *last = prev;
    (void)hipGraphDestroy(seg);
    return OSH_OK;
}

OSH_API osh_status osh_graph_instantiate(osh_graph_builder b, osh_graph *g) {
    if (!b || !g) return fail(OSH_E_INVALID, "NULL argument");
    *g = nullptr;
    hipGraphExec_t exec = nullptr;
    OSH_HIP_CHECK(hipGraphInstantiate(&exec, reinterpret_cast<hipGraph_t>(b), nullptr, nullptr, 0));
    *g = exec;
    return OSH_OK;
}

OSH_API osh_status osh_graph_builder_destroy(osh_graph_builder b) {
    if (b) OSH_HIP_CHECK(hipGraphDestroy(reinterpret_cast<hipGraph_t>(b)));
    return OSH_OK;
}

}  // extern "C"
