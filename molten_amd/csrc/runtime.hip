// runtime.hip -- error state, device queries and the small device runtime
// that replaces molten's MetalContext / ComputePass / Tensor host access
// (src/metal.rs:92-416, src/tensor.rs:100-192).
#include <hip/hip_runtime.h>

#include <atomic>
#include <string>

#include "mh_host.hpp"

namespace mh {

namespace {
thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

// The device status word (MH_STATUS_* bits, set by kernels whose bounded
// waits expire).  Each device holds its own copy; host code uses the address
// hipGetSymbolAddress returns for the current device, never the name.
__device__ __align__(256) uint32_t g_status[64];
std::atomic<uint32_t*> g_status_ptr[kMaxDevices];
}  // namespace

int current_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        return -1;
    }
    return dev;
}

uint32_t* status_word() {
    const int dev = current_device();
    if (dev < 0) {
        return nullptr;
    }
    uint32_t* p = g_status_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        void* q = nullptr;
        if (hipGetSymbolAddress(&q, HIP_SYMBOL(g_status)) != hipSuccess || q == nullptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        p = static_cast<uint32_t*>(q);
        g_status_ptr[dev].store(p, std::memory_order_release);
    }
    return p;
}

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_error(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return static_cast<int>(e);
}

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        return 256;
    }
    int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0) {
            n = 256;
        }
        g_cu_count[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

int check_quant(const mh_quant_weights* w, const char* op) {
    MH_ENSURE(w != nullptr, MH_ERR_INVALID, "%s: weights are NULL", op);
    MH_ENSURE(w->codes && w->scales && w->biases, MH_ERR_INVALID,
              "%s: codes/scales/biases must be non-NULL", op);
    MH_ENSURE(w->bits == 4 || w->bits == 6, MH_ERR_UNSUPPORTED, "%s: unsupported bit width %u",
              op, w->bits);
    MH_ENSURE(w->out_features > 0 && w->in_features > 0, MH_ERR_INVALID,
              "%s: empty weight matrix [%u, %u]", op, w->out_features, w->in_features);
    MH_ENSURE(w->group_size >= 32 && w->group_size % 32 == 0, MH_ERR_UNSUPPORTED,
              "%s: group size %u is not a multiple of 32", op, w->group_size);
    MH_ENSURE(w->in_features % w->group_size == 0, MH_ERR_INVALID,
              "%s: in_features %u not a multiple of the group size %u", op, w->in_features,
              w->group_size);
    MH_ENSURE(aligned(w->codes, w->bits == 4 ? 16 : 8), MH_ERR_ALIGN,
              "%s: codes pointer not %d-byte aligned; the kernels read codes as vectors", op,
              w->bits == 4 ? 16 : 8);
    MH_ENSURE(aligned(w->scales, 2) && aligned(w->biases, 2), MH_ERR_ALIGN,
              "%s: scales/biases not 2-byte aligned", op);
    return MH_OK;
}

int check_quant_dequant(const mh_quant_weights* w, const char* op) {
    MH_ENSURE(w != nullptr, MH_ERR_INVALID, "%s: weights are NULL", op);
    if (w->bits != 8u) {
        return check_quant(w, op);
    }
    MH_ENSURE(w->codes && w->scales && w->biases, MH_ERR_INVALID,
              "%s: codes/scales/biases must be non-NULL", op);
    MH_ENSURE(w->out_features > 0 && w->in_features > 0, MH_ERR_INVALID,
              "%s: empty weight matrix [%u, %u]", op, w->out_features, w->in_features);
    MH_ENSURE(w->group_size >= 32 && w->group_size % 32 == 0, MH_ERR_UNSUPPORTED,
              "%s: group size %u is not a multiple of 32", op, w->group_size);
    MH_ENSURE(w->in_features % w->group_size == 0, MH_ERR_INVALID,
              "%s: in_features %u not a multiple of the group size %u", op, w->in_features,
              w->group_size);
    MH_ENSURE(aligned(w->codes, 16), MH_ERR_ALIGN,
              "%s: codes pointer not 16-byte aligned; the kernels read codes as vectors", op);
    MH_ENSURE(aligned(w->scales, 2) && aligned(w->biases, 2), MH_ERR_ALIGN,
              "%s: scales/biases not 2-byte aligned", op);
    return MH_OK;
}

namespace {
__global__ void k_zero(uint32_t* p, size_t words, uint8_t* tail, size_t tail_bytes) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
         i += stride) {
        p[i] = 0u;
    }
    if (blockIdx.x == 0 && threadIdx.x < tail_bytes) {
        tail[threadIdx.x] = 0u;
    }
}
}  // namespace

}  // namespace mh

extern "C" {

const char* mh_last_error(void) { return mh::g_last_error.c_str(); }

const char* mh_version(void) { return "molten-hip 0.1.0 gfx950"; }

int mh_device_count(int* count) {
    MH_ENSURE(count != nullptr, MH_ERR_INVALID, "mh_device_count: count is NULL");
    const hipError_t e = hipGetDeviceCount(count);
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipGetDeviceCount");
}

int mh_set_device(int device) {
    const hipError_t e = hipSetDevice(device);
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipSetDevice");
}

int mh_stream_create(mh_stream_t* stream) {
    MH_ENSURE(stream != nullptr, MH_ERR_INVALID, "mh_stream_create: stream is NULL");
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
        return mh::hip_error(e, "hipStreamCreateWithFlags");
    }
    *stream = reinterpret_cast<mh_stream_t>(s);
    return MH_OK;
}

int mh_stream_destroy(mh_stream_t stream) {
    const hipError_t e = hipStreamDestroy(mh::as_stream(stream));
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipStreamDestroy");
}

int mh_stream_synchronize(mh_stream_t stream) {
    const hipError_t e = hipStreamSynchronize(mh::as_stream(stream));
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipStreamSynchronize");
}

int mh_event_create(mh_event_t* event) {
    MH_ENSURE(event != nullptr, MH_ERR_INVALID, "mh_event_create: event is NULL");
    hipEvent_t ev = nullptr;
    const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        return mh::hip_error(e, "hipEventCreateWithFlags");
    }
    *event = reinterpret_cast<mh_event_t>(ev);
    return MH_OK;
}

int mh_event_destroy(mh_event_t event) {
    const hipError_t e = hipEventDestroy(reinterpret_cast<hipEvent_t>(event));
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipEventDestroy");
}

int mh_event_record(mh_event_t event, mh_stream_t stream) {
    const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(event), mh::as_stream(stream));
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipEventRecord");
}

int mh_event_synchronize(mh_event_t event) {
    const hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(event));
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipEventSynchronize");
}

int mh_malloc(void** ptr, size_t bytes) {
    MH_ENSURE(ptr != nullptr, MH_ERR_INVALID, "mh_malloc: ptr is NULL");
    const hipError_t e = hipMalloc(ptr, bytes);
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipMalloc");
}

int mh_free(void* ptr) {
    const hipError_t e = hipFree(ptr);
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipFree");
}

int mh_memcpy(void* dst, const void* src, size_t bytes, int kind, mh_stream_t stream) {
    MH_ENSURE(kind >= 1 && kind <= 3, MH_ERR_INVALID, "mh_memcpy: kind %d not in 1..3", kind);
    MH_ENSURE(bytes == 0 || (dst && src), MH_ERR_INVALID, "mh_memcpy: NULL pointer");
    if (bytes == 0) {
        return MH_OK;
    }
    const hipMemcpyKind k = kind == 1   ? hipMemcpyHostToDevice
                            : kind == 2 ? hipMemcpyDeviceToHost
                                        : hipMemcpyDeviceToDevice;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, k, mh::as_stream(stream));
    if (e == hipSuccess) {
        e = hipStreamSynchronize(mh::as_stream(stream));
    }
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "hipMemcpyAsync");
}

int mh_status(uint32_t* status, int clear, mh_stream_t stream) {
    MH_ENSURE(status != nullptr, MH_ERR_INVALID, "mh_status: status is NULL");
    uint32_t* w = mh::status_word();
    MH_ENSURE(w != nullptr, MH_ERR_RUNTIME, "mh_status: no device status word on this device");
    const hipStream_t s = mh::as_stream(stream);
    hipError_t e = hipMemcpyAsync(status, w, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) {
        e = hipStreamSynchronize(s);
    }
    if (e == hipSuccess && clear && *status != 0u) {
        e = hipMemsetAsync(w, 0, sizeof(uint32_t), s);
        if (e == hipSuccess) {
            e = hipStreamSynchronize(s);
        }
    }
    return e == hipSuccess ? MH_OK : mh::hip_error(e, "mh_status");
}

int mh_zero(void* dst, size_t bytes, mh_stream_t stream) {
    MH_ENSURE(bytes == 0 || dst, MH_ERR_INVALID, "mh_zero: NULL pointer");
    MH_ENSURE(mh::aligned(dst, 4), MH_ERR_ALIGN, "mh_zero: destination not 4-byte aligned");
    if (bytes == 0) {
        return MH_OK;
    }
    const size_t words = bytes / 4;
    const size_t tail = bytes % 4;
    const unsigned blocks =
        static_cast<unsigned>(words == 0 ? 1 : (words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096);
    hipLaunchKernelGGL(mh::k_zero, dim3(blocks), dim3(256), 0, mh::as_stream(stream),
                       static_cast<uint32_t*>(dst), words,
                       static_cast<uint8_t*>(dst) + words * 4, tail);
    return mh::launch_status("mh_zero");
}

}  // extern "C"
