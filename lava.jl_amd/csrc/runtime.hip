// runtime.hip -- device-memory plumbing, errors and capability queries.
//
// Lava itself owns nothing at run time: buffers, queues and launches are
// Mantle's (README.md:11-13; src/compiler/cache.jl:16-17).  A C ABI called from
// Julia's `ccall` needs the minimum of that layer -- allocate, copy, synchronise,
// time -- so it is here as thin wrappers over the HIP runtime.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "lava_hip_internal.hpp"

namespace lava {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int hip_fail(hipError_t e, const char* what) {
    set_error("%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
    return e == hipErrorNoDevice ? LAVA_HIP_ERR_NO_DEVICE : LAVA_HIP_ERR_HIP;
}

// Names of the kernels this thread launched, '+'-separated, the newest last (lava_hip_kernel_log).
static thread_local char g_klog[256] = "";

static void log_kernel(const char* name) {
    const size_t m = strlen(name);
    if (m + 1 >= sizeof(g_klog)) return;
    size_t n = strlen(g_klog);
    while (n > 0 && n + 1 + m + 1 > sizeof(g_klog)) {   // drop the oldest names until this one fits
        const char* plus = strchr(g_klog, '+');
        if (plus == nullptr) {
            n = 0;
            break;
        }
        memmove(g_klog, plus + 1, strlen(plus + 1) + 1);
        n = strlen(g_klog);
    }
    if (n > 0) g_klog[n++] = '+';
    memcpy(g_klog + n, name, m + 1);
}

int check_launch(const char* kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("launch of %s failed: %s (%d)", kernel, hipGetErrorString(e), (int)e);
        return LAVA_HIP_ERR_HIP;
    }
    log_kernel(kernel);
    return LAVA_HIP_OK;
}

// Kernel choices pinned by lava_hip_set_kernel_override, per family (0 = automatic).
static std::atomic<int> g_override[3];

int kernel_override(int family) {
    return family > 0 && family < 3 ? g_override[family].load(std::memory_order_relaxed) : 0;
}

__global__ void fill_bytes_kernel(uint8_t* __restrict__ dst, uint8_t value, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const uint32_t w = 0x01010101u * value;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    // 16-byte stores over the aligned body, bytes at the ends
    const size_t head = (16 - ((uintptr_t)dst & 15)) & 15;
    if (n <= head + 16) {
        for (; i < n; i += stride) dst[i] = value;
        return;
    }
    for (size_t b = i; b < head; b += stride) dst[b] = value;
    uint4* body = reinterpret_cast<uint4*>(dst + head);
    const size_t nv = (n - head) / 16;
    for (size_t v = i; v < nv; v += stride) body[v] = make_uint4(w, w, w, w);
    for (size_t b = head + nv * 16 + i; b < n; b += stride) dst[b] = value;
}

// Device-to-device copy as a kernel (not an SDMA transfer): safe under graph
// capture and visible to the shader counters.  16-byte moves when both ends are
// 16-byte aligned, bytes otherwise.
__global__ void copy_bytes_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
        const size_t nv = n / 16;
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
        uint4* d4 = reinterpret_cast<uint4*>(dst);
        for (size_t v = i0; v < nv; v += stride) d4[v] = s4[v];
        for (size_t b = nv * 16 + i0; b < n; b += stride) dst[b] = src[b];
    } else {
        for (size_t b = i0; b < n; b += stride) dst[b] = src[b];
    }
}

// Reads [src, src + 16 n16) once -- 16-byte loads with the nontemporal hint, UNROLL of them in
// flight per thread, the threads of a workgroup on adjacent 16-byte words in each load -- and
// stores the XOR of everything a thread read to sink[thread], so that no load is dropped.  The
// read bandwidth the part sustains (lava_hip_read_stream).
typedef uint32_t rs_u32x4 __attribute__((ext_vector_type(4)));

template <int UNROLL>
__global__ void __launch_bounds__(256) read_stream_kernel(const rs_u32x4* __restrict__ src, size_t n16,
                                                          uint32_t* __restrict__ sink) {
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nth = (size_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    size_t i = tid;
    for (; i + (UNROLL - 1) * nth < n16; i += UNROLL * nth) {
        rs_u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * nth);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += nth) {
        const rs_u32x4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    sink[tid] = acc;
}

// MFMA issue loop (lava_hip_mfma_loop): each lane reads four (a, b) operand pairs of 16 bytes
// from the caller's buffers once, then issues `iters` rounds of independent MFMAs -- 16 of a 16x16
// form on 16 accumulators, or 4 of a 32x32 form on 4 -- with operand pair t % 4 for accumulator t
// and no memory access in the loop.  The matrix-core rate the part sustains on that data at the
// clock its power budget allows, the ceiling beside the published peak.
typedef float ml_f32x4 __attribute__((ext_vector_type(4)));
typedef float ml_f32x16 __attribute__((ext_vector_type(16)));
typedef int ml_i32x4 __attribute__((ext_vector_type(4)));
typedef int ml_i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 ml_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 ml_bf16x8 __attribute__((ext_vector_type(8)));

template <int OP>
__global__ void __launch_bounds__(1024, 1) mfma_loop_kernel(const rs_u32x4* __restrict__ a,
                                                           const rs_u32x4* __restrict__ b, size_t n16,
                                                           int iters, float* __restrict__ sink) {
    // 81 KB of LDS (never touched: the entry rejects iters < 1) hold the part to one workgroup
    // per CU, so that waves per SIMD is blockDim / 256 as asked
    __shared__ float one_per_cu[81 * 256];
    if (iters < 0) one_per_cu[threadIdx.x] = 0.f;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    ml_i32x4 op[8];
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        op[2 * o] = (ml_i32x4)a[(tid * 4 + o) % n16];
        op[2 * o + 1] = (ml_i32x4)b[(tid * 4 + o) % n16];
    }
    constexpr bool WIDE = (OP == LAVA_HIP_MFMA_F16_32X32X16 || OP == LAVA_HIP_MFMA_BF16_32X32X16 ||
                           OP == LAVA_HIP_MFMA_I8_32X32X32);
    ml_f32x4 c4[WIDE ? 1 : 16];
    ml_f32x16 c16[WIDE ? 4 : 1];
    for (int t = 0; t < (WIDE ? 1 : 16); ++t) c4[t] = ml_f32x4{0.f, 0.f, 0.f, 0.f};
    for (int t = 0; t < (WIDE ? 4 : 1); ++t)
        for (int r = 0; r < 16; ++r) c16[t][r] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < (WIDE ? 4 : 16); ++t) {
            const ml_i32x4 x = op[2 * (t & 3)], y = op[2 * (t & 3) + 1];
            if constexpr (OP == LAVA_HIP_MFMA_F16_16X16X32)
                c4[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16((ml_f16x8)x, (ml_f16x8)y, c4[t], 0, 0, 0);
            else if constexpr (OP == LAVA_HIP_MFMA_BF16_16X16X32)
                c4[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16((ml_bf16x8)x, (ml_bf16x8)y, c4[t], 0, 0, 0);
            else if constexpr (OP == LAVA_HIP_MFMA_I8_16X16X64)
                c4[t] = (ml_f32x4)__builtin_amdgcn_mfma_i32_16x16x64_i8(x, y, (ml_i32x4)c4[t], 0, 0, 0);
            else if constexpr (OP == LAVA_HIP_MFMA_F16_32X32X16)
                c16[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16((ml_f16x8)x, (ml_f16x8)y, c16[t], 0, 0, 0);
            else if constexpr (OP == LAVA_HIP_MFMA_BF16_32X32X16)
                c16[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16((ml_bf16x8)x, (ml_bf16x8)y, c16[t], 0, 0, 0);
            else
                c16[t] = (ml_f32x16)__builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, (ml_i32x16)c16[t], 0, 0, 0);
        }
    }
    // the accumulators' bits, folded by multiply-add (accumulators that hold equal values do not
    // cancel, as they would under XOR) so that no MFMA is dropped
    uint32_t h = 0;
    for (int t = 0; t < (WIDE ? 1 : 16); ++t)
        for (int r = 0; r < 4; ++r) h = h * 0x9E3779B1u + __float_as_uint(c4[t][r]);
    for (int t = 0; t < (WIDE ? 4 : 1); ++t)
        for (int r = 0; r < 16; ++r) h = h * 0x9E3779B1u + __float_as_uint(c16[t][r]);
    sink[tid] = __uint_as_float(h);
}

template <int OP>
static void launch_mfma_loop(int blocks, int threads, hipStream_t s, const rs_u32x4* a, const rs_u32x4* b,
                             size_t n16, int iters, float* sink) {
    hipLaunchKernelGGL(mfma_loop_kernel<OP>, dim3((unsigned)blocks), dim3((unsigned)threads), 0, s, a, b, n16, iters,
                       sink);
}

}  // namespace lava

using namespace lava;

extern "C" {

const char* lava_hip_last_error(void) { return g_err; }

const char* lava_hip_kernel_log(void) { return g_klog; }

void lava_hip_kernel_log_clear(void) { g_klog[0] = 0; }

int lava_hip_set_kernel_override(int family, int choice) {
    const bool ok = (family == LAVA_HIP_FAMILY_ATTN && (choice == 0 || choice == 3 || choice == 5)) ||
                    (family == LAVA_HIP_FAMILY_GEMM && choice >= 0 && choice <= 4);
    LAVA_ARG(ok, "set_kernel_override: unknown family %d or choice %d", family, choice);
    g_override[family].store(choice, std::memory_order_relaxed);
    return LAVA_HIP_OK;
}

int lava_hip_version(void) { return 100; }

int lava_hip_init(void) {
    static std::once_flag once;
    static int status = LAVA_HIP_OK;
    static char msg[512];
    std::call_once(once, [] {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n == 0) {
            snprintf(msg, sizeof(msg), "no HIP device available (%s)", hipGetErrorString(e));
            status = LAVA_HIP_ERR_NO_DEVICE;
            return;
        }
        hipDeviceProp_t p;
        e = hipGetDeviceProperties(&p, 0);
        if (e != hipSuccess) {
            snprintf(msg, sizeof(msg), "hipGetDeviceProperties failed: %s", hipGetErrorString(e));
            status = LAVA_HIP_ERR_HIP;
            return;
        }
        if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
            snprintf(msg, sizeof(msg), "device 0 is %s; liblava_hip.so is built for gfx950 only", p.gcnArchName);
            status = LAVA_HIP_ERR_NO_DEVICE;
            return;
        }
    });
    if (status != LAVA_HIP_OK) set_error("%s", msg);
    return status;
}

int lava_hip_device_count(int* count) {
    LAVA_ARG(count != nullptr, "device_count: null output pointer");
    *count = 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) return LAVA_HIP_OK;
    LAVA_HIP_TRY(e);
    *count = n;
    return LAVA_HIP_OK;
}

int lava_hip_malloc(void** ptr, size_t bytes) {
    LAVA_ARG(ptr != nullptr, "malloc: null output pointer");
    *ptr = nullptr;
    if (bytes == 0) return LAVA_HIP_OK;
    LAVA_HIP_TRY(hipMalloc(ptr, bytes));
    return LAVA_HIP_OK;
}

int lava_hip_free(void* ptr) {
    if (ptr == nullptr) return LAVA_HIP_OK;
    LAVA_HIP_TRY(hipFree(ptr));
    return LAVA_HIP_OK;
}

int lava_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return LAVA_HIP_OK;
    LAVA_ARG(dst != nullptr && src != nullptr, "memcpy_h2d: null pointer");
    LAVA_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return LAVA_HIP_OK;
}

int lava_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return LAVA_HIP_OK;
    LAVA_ARG(dst != nullptr && src != nullptr, "memcpy_d2h: null pointer");
    LAVA_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return LAVA_HIP_OK;
}

int lava_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return LAVA_HIP_OK;
    LAVA_ARG(dst != nullptr && src != nullptr, "memcpy_d2d: null pointer");
    size_t blocks = (bytes / 16 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       static_cast<uint8_t*>(dst), static_cast<const uint8_t*>(src), bytes);
    LAVA_LAUNCH_CHECK("copy_bytes_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_fill_bytes(void* dst, uint8_t value, size_t bytes, void* stream) {
    if (bytes == 0) return LAVA_HIP_OK;
    LAVA_ARG(dst != nullptr, "fill_bytes: null pointer");
    size_t blocks = (bytes / 16 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       static_cast<uint8_t*>(dst), value, bytes);
    LAVA_LAUNCH_CHECK("fill_bytes_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_synchronize(void) {
    LAVA_HIP_TRY(hipDeviceSynchronize());
    return LAVA_HIP_OK;
}

int lava_hip_stream_synchronize(void* stream) {
    LAVA_HIP_TRY(hipStreamSynchronize(as_stream(stream)));
    return LAVA_HIP_OK;
}

int lava_hip_stream_create(void** stream) {
    LAVA_ARG(stream != nullptr, "stream_create: null output pointer");
    hipStream_t s;
    LAVA_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return LAVA_HIP_OK;
}

int lava_hip_stream_destroy(void* stream) {
    if (stream == nullptr) return LAVA_HIP_OK;
    // the stream's W8A16 workspace may be in use by work still queued on it
    LAVA_HIP_TRY(hipStreamSynchronize(as_stream(stream)));
    lava::w8a16_release_stream(stream);
    LAVA_HIP_TRY(hipStreamDestroy(as_stream(stream)));
    return LAVA_HIP_OK;
}

int lava_hip_event_create(void** event) {
    LAVA_ARG(event != nullptr, "event_create: null output pointer");
    hipEvent_t e;
    LAVA_HIP_TRY(hipEventCreate(&e));
    *event = e;
    return LAVA_HIP_OK;
}

int lava_hip_event_destroy(void* event) {
    if (event == nullptr) return LAVA_HIP_OK;
    LAVA_HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return LAVA_HIP_OK;
}

int lava_hip_event_record(void* event, void* stream) {
    LAVA_ARG(event != nullptr, "event_record: null event");
    LAVA_HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
    return LAVA_HIP_OK;
}

int lava_hip_event_elapsed_ms(float* ms, void* start, void* stop) {
    LAVA_ARG(ms != nullptr && start != nullptr && stop != nullptr, "event_elapsed_ms: null argument");
    LAVA_HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
    LAVA_HIP_TRY(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
    return LAVA_HIP_OK;
}

int lava_hip_read_stream(const void* src, size_t bytes, uint32_t* sink, int blocks, int unroll, void* stream) {
    LAVA_ARG(src != nullptr && sink != nullptr, "read_stream: null pointer");
    LAVA_ARG(aligned(src, 16) && bytes % 16 == 0, "read_stream: src must be 16-byte aligned and bytes a multiple of 16");
    LAVA_ARG(blocks >= 1 && blocks <= 65536, "read_stream: blocks = %d outside [1, 65536]", blocks);
    LAVA_ARG(unroll == 4 || unroll == 8 || unroll == 16, "read_stream: unroll = %d is not 4, 8 or 16", unroll);
    const rs_u32x4* s4 = static_cast<const rs_u32x4*>(src);
    const size_t n16 = bytes / 16;
    hipStream_t s = as_stream(stream);
    if (unroll == 4)
        hipLaunchKernelGGL(read_stream_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, s4, n16, sink);
    else if (unroll == 8)
        hipLaunchKernelGGL(read_stream_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, s, s4, n16, sink);
    else
        hipLaunchKernelGGL(read_stream_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, s, s4, n16, sink);
    LAVA_LAUNCH_CHECK("read_stream_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_mfma_loop(int op, const void* a, const void* b, size_t bytes, int blocks, int waves_per_simd,
                       int iters, float* sink, void* stream) {
    LAVA_ARG(a != nullptr && b != nullptr && sink != nullptr, "mfma_loop: null pointer");
    LAVA_ARG(aligned(a, 16) && aligned(b, 16) && bytes >= 16 && bytes % 16 == 0,
             "mfma_loop: a and b must be 16-byte aligned and bytes a positive multiple of 16");
    LAVA_ARG(op >= LAVA_HIP_MFMA_F16_16X16X32 && op <= LAVA_HIP_MFMA_I8_32X32X32, "mfma_loop: unknown form %d", op);
    LAVA_ARG(blocks >= 1 && blocks <= 65536, "mfma_loop: blocks = %d outside [1, 65536]", blocks);
    LAVA_ARG(waves_per_simd == 1 || waves_per_simd == 2 || waves_per_simd == 4,
             "mfma_loop: waves_per_simd = %d is not 1, 2 or 4", waves_per_simd);
    LAVA_ARG(iters >= 1, "mfma_loop: iters = %d < 1", iters);
    const rs_u32x4* a4 = static_cast<const rs_u32x4*>(a);
    const rs_u32x4* b4 = static_cast<const rs_u32x4*>(b);
    const size_t n16 = bytes / 16;
    const int threads = 256 * waves_per_simd;
    hipStream_t s = as_stream(stream);
    switch (op) {
        case LAVA_HIP_MFMA_F16_16X16X32:
            launch_mfma_loop<LAVA_HIP_MFMA_F16_16X16X32>(blocks, threads, s, a4, b4, n16, iters, sink);
            break;
        case LAVA_HIP_MFMA_BF16_16X16X32:
            launch_mfma_loop<LAVA_HIP_MFMA_BF16_16X16X32>(blocks, threads, s, a4, b4, n16, iters, sink);
            break;
        case LAVA_HIP_MFMA_I8_16X16X64:
            launch_mfma_loop<LAVA_HIP_MFMA_I8_16X16X64>(blocks, threads, s, a4, b4, n16, iters, sink);
            break;
        case LAVA_HIP_MFMA_F16_32X32X16:
            launch_mfma_loop<LAVA_HIP_MFMA_F16_32X32X16>(blocks, threads, s, a4, b4, n16, iters, sink);
            break;
        case LAVA_HIP_MFMA_BF16_32X32X16:
            launch_mfma_loop<LAVA_HIP_MFMA_BF16_32X32X16>(blocks, threads, s, a4, b4, n16, iters, sink);
            break;
        default:
            launch_mfma_loop<LAVA_HIP_MFMA_I8_32X32X32>(blocks, threads, s, a4, b4, n16, iters, sink);
            break;
    }
    LAVA_LAUNCH_CHECK("mfma_loop_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_graph_capture_begin(void* stream) {
    LAVA_ARG(stream != nullptr, "graph_capture_begin: the NULL stream cannot be captured");
    LAVA_HIP_TRY(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeGlobal));
    return LAVA_HIP_OK;
}

int lava_hip_graph_capture_end(void* stream, void** exec) {
    LAVA_ARG(stream != nullptr && exec != nullptr, "graph_capture_end: null stream or output pointer");
    *exec = nullptr;
    hipGraph_t g = nullptr;
    LAVA_HIP_TRY(hipStreamEndCapture(as_stream(stream), &g));
    hipGraphExec_t e = nullptr;
    const hipError_t r = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);   // the executable graph keeps what it needs
    LAVA_HIP_TRY(r);
    *exec = e;
    return LAVA_HIP_OK;
}

int lava_hip_graph_launch(void* exec, void* stream) {
    LAVA_ARG(exec != nullptr, "graph_launch: null graph");
    LAVA_HIP_TRY(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), as_stream(stream)));
    return LAVA_HIP_OK;
}

int lava_hip_graph_destroy(void* exec) {
    if (exec == nullptr) return LAVA_HIP_OK;
    LAVA_HIP_TRY(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec)));
    return LAVA_HIP_OK;
}

// gfx950 MFMA shapes, subgroup scope, as (ab, acc, M, N, K).  Dense forms only.
static const int32_t kShapes[][5] = {
    {LAVA_HIP_F16, LAVA_HIP_F32, 16, 16, 16}, {LAVA_HIP_F16, LAVA_HIP_F32, 16, 16, 32},
    {LAVA_HIP_F16, LAVA_HIP_F32, 32, 32, 8},  {LAVA_HIP_F16, LAVA_HIP_F32, 32, 32, 16},
    {LAVA_HIP_BF16, LAVA_HIP_F32, 16, 16, 16}, {LAVA_HIP_BF16, LAVA_HIP_F32, 16, 16, 32},
    {LAVA_HIP_BF16, LAVA_HIP_F32, 32, 32, 8}, {LAVA_HIP_BF16, LAVA_HIP_F32, 32, 32, 16},
    {LAVA_HIP_I8, LAVA_HIP_I32, 16, 16, 32},  {LAVA_HIP_I8, LAVA_HIP_I32, 16, 16, 64},
    {LAVA_HIP_I8, LAVA_HIP_I32, 32, 32, 16},  {LAVA_HIP_I8, LAVA_HIP_I32, 32, 32, 32},
    {LAVA_HIP_F32, LAVA_HIP_F32, 16, 16, 4},  {LAVA_HIP_F32, LAVA_HIP_F32, 32, 32, 2},
    {LAVA_HIP_F64, LAVA_HIP_F64, 16, 16, 4},
};

int lava_hip_matrix_shapes(int32_t* out, int max_rows, int* count) {
    LAVA_ARG(count != nullptr, "matrix_shapes: null count pointer");
    const int n = (int)(sizeof(kShapes) / sizeof(kShapes[0]));
    *count = n;
    if (out == nullptr) return LAVA_HIP_OK;
    for (int i = 0; i < n && i < max_rows; ++i) {
        for (int j = 0; j < 5; ++j) out[6 * i + j] = kShapes[i][j];
        out[6 * i + 5] = 0;
    }
    return LAVA_HIP_OK;
}

int lava_hip_device_caps(int64_t* out, int n) {
    LAVA_ARG(out != nullptr || n == 0, "device_caps: null output pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    hipDeviceProp_t p;
    LAVA_HIP_TRY(hipGetDeviceProperties(&p, 0));
    int64_t v[12];
    v[0] = 1;                                   // coopmat: MFMA present
    v[1] = 16;                                  // tile: squarest fp16->fp32 shape
    v[2] = p.warpSize;                          // subgroup
    v[3] = p.warpSize;                          // coopmatsubgroup
    v[4] = (int64_t)p.sharedMemPerBlock;        // sharedbudget
    v[5] = p.maxThreadsPerBlock;                // workgrouplimit
    v[6] = p.multiProcessorCount;               // cores
    v[7] = (int64_t)(p.maxThreadsPerMultiProcessor / p.warpSize);  // warps resident per CU
    v[8] = p.clockRate;                         // kHz
    v[9] = (int64_t)p.totalGlobalMem;
    v[10] = p.l2CacheSize;
    v[11] = 950;
    for (int i = 0; i < n && i < 12; ++i) out[i] = v[i];
    return LAVA_HIP_OK;
}

}  // extern "C"
