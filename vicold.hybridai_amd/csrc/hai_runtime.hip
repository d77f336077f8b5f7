// hai_runtime.hip -- runtime wrappers of the C ABI, synthetic weight fill and
// the primitive probe used to pin device numerics.
#include "hai_common.h"
#include "hai_device.h"

#include <cstdlib>
#include <string>

namespace hai {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }

bool bounds_checking() {
    static const bool on = [] {
        const char* e = std::getenv("HAI_CHECK_BOUNDS");
        return e != nullptr && e[0] != '\0' && e[0] != '0';
    }();
    return on;
}

namespace {
int extent_in_allocation(const void* p, size_t bytes, const char* what) {
    if (bytes == 0) return HAI_OK;
    if (p == nullptr) return invalid(what);
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) != hipSuccess) {
        (void)hipGetLastError();
        set_error(std::string("bounds check: ") + what + " is not inside a device allocation");
        return HAI_ERR_INVALID_ARGUMENT;
    }
    const uintptr_t b = reinterpret_cast<uintptr_t>(base);
    const uintptr_t q = reinterpret_cast<uintptr_t>(p);
    if (q + bytes > b + size) {
        set_error(std::string("bounds check: ") + what + " needs " + std::to_string(bytes) + " bytes from offset " +
                  std::to_string(q - b) + " of a " + std::to_string(size) + "-byte allocation");
        return HAI_ERR_INVALID_ARGUMENT;
    }
    return HAI_OK;
}
}  // namespace

int check_extent(const void* p, size_t bytes, const char* what) {
    return bounds_checking() ? extent_in_allocation(p, bytes, what) : HAI_OK;
}

}  // namespace hai

extern "C" int hai_debug_check_extent(const void* p, size_t bytes) {
    return hai::extent_in_allocation(p, bytes, "range");
}

using namespace hai;

extern "C" {

const char* hai_last_error(void) { return g_last_error.c_str(); }

int hai_device_count(int* count) {
    if (count == nullptr) return invalid("count");
    return check_hip(hipGetDeviceCount(count), "hipGetDeviceCount");
}
int hai_set_device(int device) { return check_hip(hipSetDevice(device), "hipSetDevice"); }
int hai_get_device(int* device) {
    if (device == nullptr) return invalid("device");
    return check_hip(hipGetDevice(device), "hipGetDevice");
}
int hai_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return invalid("ptr");
    const hipError_t e = hipMalloc(ptr, bytes == 0 ? 256 : bytes);
    if (e == hipErrorOutOfMemory) {
        set_error("hipMalloc: out of memory");
        return HAI_ERR_OUT_OF_MEMORY;
    }
    return check_hip(e, "hipMalloc");
}
int hai_free(void* ptr) { return check_hip(hipFree(ptr), "hipFree"); }
int hai_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)),
                     "hipMemcpyAsync(H2D)");
}
int hai_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)),
                     "hipMemcpyAsync(D2H)");
}
int hai_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)),
                     "hipMemcpyAsync(D2D)");
}
int hai_memcpy_h2d_2d(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width, size_t height,
                      void* stream) {
    if (height == 0 || width == 0) return HAI_OK;
    if (dst == nullptr || src == nullptr || width > dst_pitch || width > src_pitch)
        return invalid("memcpy_h2d_2d: null pointer or width beyond a pitch");
    return check_hip(hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, width, height, hipMemcpyHostToDevice,
                                      as_stream(stream)),
                     "hipMemcpy2DAsync(H2D)");
}
int hai_memcpy(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, as_stream(stream)),
                     "hipMemcpyAsync(default)");
}
int hai_host_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return invalid("ptr");
    const hipError_t e = hipHostMalloc(ptr, bytes == 0 ? 256 : bytes, hipHostMallocDefault);
    if (e == hipErrorOutOfMemory) {
        set_error("hipHostMalloc: out of memory");
        return HAI_ERR_OUT_OF_MEMORY;
    }
    return check_hip(e, "hipHostMalloc");
}
int hai_host_free(void* ptr) { return check_hip(hipHostFree(ptr), "hipHostFree"); }
int hai_memset(void* dst, int value, size_t bytes, void* stream) {
    return check_hip(hipMemsetAsync(dst, value, bytes, as_stream(stream)), "hipMemsetAsync");
}
int hai_stream_create(void** stream) {
    if (stream == nullptr) return invalid("stream");
    hipStream_t s = nullptr;
    const int rc = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return rc;
}
int hai_stream_destroy(void* stream) {
    return check_hip(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
}
int hai_stream_synchronize(void* stream) {
    return check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}
int hai_device_synchronize(void) { return check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }
int hai_event_create(void** event) {
    if (event == nullptr) return invalid("event");
    hipEvent_t e = nullptr;
    const int rc = check_hip(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return rc;
}
int hai_event_destroy(void* event) {
    return check_hip(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "hipEventDestroy");
}
int hai_event_record(void* event, void* stream) {
    return check_hip(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)),
                     "hipEventRecord");
}
int hai_stream_wait_event(void* stream, void* event) {
    return check_hip(hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0),
                     "hipStreamWaitEvent");
}
int hai_event_synchronize(void* event) {
    return check_hip(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)), "hipEventSynchronize");
}
int hai_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (ms == nullptr) return invalid("ms");
    return check_hip(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                         reinterpret_cast<hipEvent_t>(stop)),
                     "hipEventElapsedTime");
}
int hai_graph_begin_capture(void* stream) {
    return check_hip(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal),
                     "hipStreamBeginCapture");
}
int hai_graph_end_capture(void* stream, void** graph_exec) {
    if (graph_exec == nullptr) return invalid("graph_exec");
    hipGraph_t g = nullptr;
    int rc = check_hip(hipStreamEndCapture(as_stream(stream), &g), "hipStreamEndCapture");
    if (rc != HAI_OK) return rc;
    hipGraphExec_t exec = nullptr;
    rc = check_hip(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    hipGraphDestroy(g);
    *graph_exec = exec;
    return rc;
}
int hai_graph_launch(void* graph_exec, void* stream) {
    return check_hip(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), as_stream(stream)),
                     "hipGraphLaunch");
}
int hai_graph_destroy(void* graph_exec) {
    return check_hip(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)),
                     "hipGraphExecDestroy");
}

}  // extern "C"

namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// One thread per element; grid-stride over rows*cols.
__global__ void fill_synthetic_kernel(uint16_t* __restrict__ dst, int64_t rows, int64_t cols,
                                      int64_t ld, uint64_t key, float scale) {
    const int64_t n = rows * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const uint64_t h = splitmix64(key + static_cast<uint64_t>(i));
        const int32_t s = static_cast<int32_t>((h & 0xffffu) + ((h >> 16) & 0xffffu) +
                                               ((h >> 32) & 0xffffu) + (h >> 48));
        const int64_t r = i / cols;
        const int64_t c = i - r * cols;
        dst[r * ld + c] = f2bf(static_cast<float>(s - 131070) * scale);
    }
}

// Synthetic FP8 block scales: (0.5 + 1.5 u) / 448, u the top 24 bits of the
// stream value (exact in fp32).
__global__ void fill_scales_kernel(float* __restrict__ dst, int64_t n, uint64_t key) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const uint64_t h = splitmix64(key + static_cast<uint64_t>(i));
        const float u = static_cast<float>(static_cast<uint32_t>(h >> 40)) * 0x1p-24f;
        dst[i] = (0.5f + 1.5f * u) / 448.0f;
    }
}

__global__ void debug_math_kernel(float* y, const float* x, int64_t n, int fn) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r = 0.0f;
    switch (fn) {
        case 0: r = cexp(v); break;
        case 1: r = clog1p(v); break;
        case 2: r = csigmoid(v); break;
        case 3: r = csilu(v); break;
        case 4: r = csqrt(v); break;
        case 5: r = 1.0f / v; break;
        case 6: r = bfr(v); break;
        default: r = v; break;
    }
    y[i] = r;
}

uint64_t host_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

}  // namespace

extern "C" {

int hai_fill_synthetic_bf16(void* dst, int64_t rows, int64_t cols, int64_t ld, uint64_t seed,
                            uint32_t tensor_id, float std_dev, void* stream) {
    if (dst == nullptr || rows < 0 || cols < 0 || ld < cols) return invalid("fill_synthetic");
    if (rows == 0 || cols == 0) return HAI_OK;
    const uint64_t key = host_splitmix64(seed ^ (static_cast<uint64_t>(tensor_id) << 32));
    const float scale = static_cast<float>(static_cast<double>(std_dev) * 1.7320508075688772 / 65536.0);
    const int64_t n = rows * cols;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    fill_synthetic_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint16_t*>(dst), rows, cols, ld, key, scale);
    return launched("fill_synthetic_kernel");
}

int hai_fill_synthetic_scales_f32(float* scales, int64_t n, uint64_t seed, uint32_t tensor_id, void* stream) {
    if (scales == nullptr || n < 0 || tensor_id >= 0xfff00000u) return invalid("fill_synthetic_scales");
    if (n == 0) return HAI_OK;
    const uint32_t sid = tensor_id + (1u << 20);
    const uint64_t key = host_splitmix64(seed ^ (static_cast<uint64_t>(sid) << 32));
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    fill_scales_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream)>>>(scales, n, key);
    return launched("fill_scales_kernel");
}

int hai_debug_math_f32(float* y, const float* x, int64_t n, int fn, void* stream) {
    if (y == nullptr || x == nullptr || n < 0) return invalid("debug_math");
    if (n == 0) return HAI_OK;
    debug_math_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                        as_stream(stream)>>>(y, x, n, fn);
    return launched("debug_math_kernel");
}

}  // extern "C"
