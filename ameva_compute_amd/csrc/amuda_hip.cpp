// libamuda_hip.so: the BitNet entry points of the reference's amuda / BitNet C ABI on MI355X, over the kernels of
// libameva_hip.so (include/amuda_hip.h). The reference's amuda runtime binds OpenCL / Vulkan on unified-memory phones
// (src/amuda/amuda_ops.c, amuda_core.c); here a context is one HIP device and one stream, a buffer a pinned host
// copy plus an HBM allocation, an event a pair of HIP events around the kernel.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/amuda_hip.h"
#include "../../include/ameva_hip.h"

// the reference's struct layouts (x86-64 / aarch64 LP64): callers read these fields directly
static_assert(sizeof(AcContext) == 296 && offsetof(AcContext, device_name) == 40 && offsetof(AcContext, vendor_id) == 232 &&
                  offsetof(AcContext, max_work_group_size) == 240 && offsetof(AcContext, global_mem_size) == 272 &&
                  offsetof(AcContext, is_uma_supported) == 292,
              "AcContext layout");
static_assert(sizeof(AcBuffer) == 32 && offsetof(AcBuffer, size_bytes) == 16 && offsetof(AcBuffer, is_user_allocated) == 29,
              "AcBuffer layout");
static_assert(sizeof(AcEvent) == 40 && offsetof(AcEvent, duration_us) == 32, "AcEvent layout");
static_assert(sizeof(GgufTensor) == 144 && offsetof(GgufTensor, ne) == 72 && offsetof(GgufTensor, type) == 104 &&
                  offsetof(GgufTensor, data_ptr) == 120 && offsetof(GgufTensor, size_bytes) == 128,
              "GgufTensor layout");

namespace {

struct EventPair {
    hipEvent_t start, end;
    bool done;
};

hipStream_t stream_of(AcContext* ctx) { return reinterpret_cast<hipStream_t>(ctx->command_queue); }

AcResult from_hip(hipError_t e) {
    if (e == hipSuccess) return AC_SUCCESS;
    if (e == hipErrorOutOfMemory) return AC_ERR_OUT_OF_DEVICE_MEMORY;
    return AC_ERR_DRIVER_CRASH_OR_LOST;
}

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

AcResult new_buffer(AcContext* ctx, size_t size, void* user_host, AcBuffer** out) {
    if (out) *out = nullptr;
    if (!ctx || !out) return AC_ERR_NULL_POINTER;
    if (size == 0) return AC_ERR_INVALID_BUFFER_SIZE;
    AcBuffer* b = static_cast<AcBuffer*>(calloc(1, sizeof(AcBuffer)));
    if (!b) return AC_ERR_OUT_OF_HOST_MEMORY;
    b->size_bytes = size;
    b->is_mapped = true;
    b->is_user_allocated = user_host != nullptr;
    if (user_host) {
        b->host_ptr = user_host;
    } else if (hipHostMalloc(&b->host_ptr, size, hipHostMallocDefault) != hipSuccess) {
        free(b);
        return AC_ERR_OUT_OF_HOST_MEMORY;
    } else {
        memset(b->host_ptr, 0, size);
    }
    hipError_t e = hipMalloc(&b->native_mem, size);
    if (e == hipSuccess) e = hipMemcpy(b->native_mem, b->host_ptr, size, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (b->native_mem) (void)hipFree(b->native_mem);
        if (!user_host) (void)hipHostFree(b->host_ptr);
        free(b);
        return from_hip(e);
    }
    *out = b;
    return AC_SUCCESS;
}

}  // namespace

extern "C" AcResult ac_init(AcContext** out_ctx) {
    if (!out_ctx) return AC_ERR_NULL_POINTER;
    *out_ctx = nullptr;
    int n = 0, dev = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return AC_ERR_DRIVER_NOT_FOUND;
    if (hipGetDevice(&dev) != hipSuccess) return AC_ERR_DRIVER_INIT_FAILED;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return AC_ERR_DRIVER_INIT_FAILED;
    AcContext* c = static_cast<AcContext*>(calloc(1, sizeof(AcContext)));
    if (!c) return AC_ERR_OUT_OF_HOST_MEMORY;
    hipStream_t st = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) {
        free(c);
        return AC_ERR_DRIVER_INIT_FAILED;
    }
    c->device_id = reinterpret_cast<void*>((intptr_t)dev);
    c->command_queue = st;
    snprintf(c->device_name, sizeof c->device_name, "%s (%s)", p.name, p.gcnArchName);
    snprintf(c->vendor_name, sizeof c->vendor_name, "AMD");
    c->vendor_id = 0x1002u;
    c->max_compute_units = (uint32_t)p.multiProcessorCount;
    c->max_work_group_size = (uint64_t)p.maxThreadsPerBlock;
    for (int i = 0; i < 3; ++i) c->max_work_item_sizes[i] = (uint64_t)p.maxThreadsDim[i];
    c->global_mem_size = (uint64_t)p.totalGlobalMem;
    c->local_mem_size = (uint64_t)p.sharedMemPerBlock;
    c->active_quirks = 0;
    c->is_uma_supported = false;
    *out_ctx = c;
    return AC_SUCCESS;
}

extern "C" AcResult ac_destroy(AcContext* ctx) {
    if (!ctx) return AC_ERR_NULL_POINTER;
    hipStream_t st = stream_of(ctx);
    AcResult r = from_hip(hipStreamSynchronize(st));
    (void)hipStreamDestroy(st);
    free(ctx);
    return r;
}

extern "C" AcResult ac_buffer_alloc(AcContext* ctx, size_t size_bytes, AcBuffer** out_buf) {
    return new_buffer(ctx, size_bytes, nullptr, out_buf);
}

extern "C" AcResult ac_buffer_from_host(AcContext* ctx, void* aligned_ptr, size_t size_bytes, AcBuffer** out_buf) {
    if (out_buf) *out_buf = nullptr;
    if (!aligned_ptr) return AC_ERR_NULL_POINTER;
    if (((uintptr_t)aligned_ptr & 63) != 0) return AC_ERR_INVALID_ARGUMENT;  // the reference asks for 64-byte alignment
    return new_buffer(ctx, size_bytes, aligned_ptr, out_buf);
}

extern "C" AcResult ac_buffer_sync_to_device(AcContext* ctx, AcBuffer* buf) {
    if (!ctx || !buf) return AC_ERR_NULL_POINTER;
    hipStream_t st = stream_of(ctx);
    hipError_t e = hipMemcpyAsync(buf->native_mem, buf->host_ptr, buf->size_bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return from_hip(e);
}

extern "C" AcResult ac_buffer_sync_to_host(AcContext* ctx, AcBuffer* buf) {
    if (!ctx || !buf) return AC_ERR_NULL_POINTER;
    hipStream_t st = stream_of(ctx);
    hipError_t e = hipMemcpyAsync(buf->host_ptr, buf->native_mem, buf->size_bytes, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return from_hip(e);
}

extern "C" AcResult ac_buffer_free(AcContext* ctx, AcBuffer* buf) {
    if (!ctx || !buf) return AC_ERR_NULL_POINTER;
    (void)hipStreamSynchronize(stream_of(ctx));
    hipError_t e = hipFree(buf->native_mem);
    if (!buf->is_user_allocated) (void)hipHostFree(buf->host_ptr);
    free(buf);
    return from_hip(e);
}

extern "C" AcResult ac_event_wait(AcContext* ctx, AcEvent* event) {
    if (!ctx || !event || !event->native_event) return AC_ERR_NULL_POINTER;
    EventPair* ev = static_cast<EventPair*>(event->native_event);
    if (!ev->done) {
        hipError_t e = hipEventSynchronize(ev->end);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev->start, ev->end);
        if (e != hipSuccess) return from_hip(e);
        const uint64_t ns = (uint64_t)((double)ms * 1e6);
        event->start_time_ns = event->submit_time_ns;
        event->end_time_ns = event->submit_time_ns + ns;
        event->duration_us = ns / 1000;
        ev->done = true;
    }
    return AC_SUCCESS;
}

extern "C" uint64_t ac_event_get_duration_us(AcEvent* event) {
    if (!event || !event->native_event) return 0;
    EventPair* ev = static_cast<EventPair*>(event->native_event);
    if (!ev->done && hipEventSynchronize(ev->end) == hipSuccess) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, ev->start, ev->end) == hipSuccess) {
            const uint64_t ns = (uint64_t)((double)ms * 1e6);
            event->start_time_ns = event->submit_time_ns;
            event->end_time_ns = event->submit_time_ns + ns;
            event->duration_us = ns / 1000;
            ev->done = true;
        }
    }
    return event->duration_us;
}

extern "C" AcResult ac_event_free(AcContext* ctx, AcEvent* event) {
    (void)ctx;
    if (!event) return AC_ERR_NULL_POINTER;
    if (EventPair* ev = static_cast<EventPair*>(event->native_event)) {
        (void)hipEventSynchronize(ev->end);
        (void)hipEventDestroy(ev->start);
        (void)hipEventDestroy(ev->end);
        delete ev;
    }
    free(event);
    return AC_SUCCESS;
}

extern "C" AcResult ac_ops_bitnet_gemv_i2_s_exact(AcContext* ctx, int M, int K, AcBuffer* x, AcBuffer* W_packed,
                                                  float tensor_scale, AcBuffer* y, AcEvent** out_event) {
    if (out_event) *out_event = nullptr;
    if (!ctx || !x || !W_packed || !y) return AC_ERR_NULL_POINTER;
    if (M <= 0 || K <= 0 || K % 128 != 0) return AC_ERR_KERNEL_ARG_INVALID;
    const uint64_t req_x = (uint64_t)K * sizeof(float), req_w = (uint64_t)M * ((uint64_t)K / 4),
                   req_y = (uint64_t)M * sizeof(float);
    if (x->size_bytes < req_x || W_packed->size_bytes < req_w || y->size_bytes < req_y)
        return AC_ERR_INVALID_BUFFER_SIZE;
    AcResult r;
    if ((r = ac_buffer_sync_to_device(ctx, x)) != AC_SUCCESS) return r;
    if ((r = ac_buffer_sync_to_device(ctx, W_packed)) != AC_SUCCESS) return r;
    if ((r = ac_buffer_sync_to_device(ctx, y)) != AC_SUCCESS) return r;
    hipStream_t st = stream_of(ctx);
    EventPair* ev = nullptr;
    AcEvent* ae = nullptr;
    if (out_event) {
        ae = static_cast<AcEvent*>(calloc(1, sizeof(AcEvent)));
        ev = new EventPair{nullptr, nullptr, false};
        if (!ae || hipEventCreate(&ev->start) != hipSuccess || hipEventCreate(&ev->end) != hipSuccess) {
            free(ae);
            delete ev;
            return AC_ERR_OUT_OF_HOST_MEMORY;
        }
        ae->native_event = ev;
        ae->submit_time_ns = now_ns();
        (void)hipEventRecord(ev->start, st);
    }
    const int rc = amv_i2s_gemv_f32(W_packed->native_mem, M, K, static_cast<const float*>(x->native_mem),
                                    tensor_scale, static_cast<float*>(y->native_mem), st);
    if (rc != AMV_OK) {
        if (ae) ac_event_free(ctx, ae);
        return rc == AMV_ERR_INVALID_ARG ? AC_ERR_KERNEL_ARG_INVALID : AC_ERR_DRIVER_CRASH_OR_LOST;
    }
    if (ae) {
        (void)hipEventRecord(ev->end, st);
        *out_event = ae;
    }
    return AC_SUCCESS;
}

extern "C" void bitnet_raw_vec_dot_i2_s(int32_t n, float* s, const void* vx, const void* vy, int32_t nrc,
                                        int32_t kernel_type) {
    if (!s || !vx || !vy || n <= 0 || nrc <= 0 || n % 128 != 0) return;
    const int64_t rows = kernel_type == 1 ? 1 : nrc, m = kernel_type == 1 ? nrc : 1;
    const size_t wbytes = (size_t)rows * (size_t)(n / 4);
    const int64_t abytes = amv_i2s_act_bytes(m, n);
    // the kernels' activation layout: int8 [m][n] | {f32 dequant, i32 sum q} [m] (the raw dot needs no scale)
    std::vector<uint8_t> act((size_t)abytes);
    memcpy(act.data(), vy, (size_t)m * n);
    for (int64_t i = 0; i < m; ++i) {
        const int8_t* q = static_cast<const int8_t*>(vy) + i * n;
        int32_t sq = 0;
        for (int32_t j = 0; j < n; ++j) sq += q[j];
        const float one = 1.0f;
        memcpy(act.data() + m * n + 8 * i, &one, 4);
        memcpy(act.data() + m * n + 8 * i + 4, &sq, 4);
    }
    void *dw = nullptr, *da = nullptr, *ds = nullptr;
    std::vector<int32_t> sums((size_t)(rows * m));
    hipError_t e = hipMalloc(&dw, wbytes);
    if (e == hipSuccess) e = hipMalloc(&da, (size_t)abytes);
    if (e == hipSuccess) e = hipMalloc(&ds, sums.size() * sizeof(int32_t));
    if (e == hipSuccess) e = hipMemcpy(dw, vx, wbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(da, act.data(), (size_t)abytes, hipMemcpyHostToDevice);
    if (e == hipSuccess && amv_i2s_gemv_sums(dw, rows, n, da, m, static_cast<int32_t*>(ds), nullptr) == AMV_OK)
        e = hipMemcpy(sums.data(), ds, sums.size() * sizeof(int32_t), hipMemcpyDeviceToHost);
    else if (e == hipSuccess)
        e = hipErrorInvalidValue;
    if (e == hipSuccess)
        for (size_t i = 0; i < sums.size(); ++i) s[i] = (float)sums[i];
    else
        fprintf(stderr, "bitnet_raw_vec_dot_i2_s: GPU call failed (%s) (FAIL-FAST)\n", hipGetErrorString(e));
    (void)hipFree(dw);
    (void)hipFree(da);
    (void)hipFree(ds);
}

extern "C" AcResult ac_gguf_get_tensor_scale(const GgufTensor* tensor, float* out_scale) {
    if (!tensor || !out_scale) return AC_ERR_NULL_POINTER;
    if (tensor->type == 36u) {  // I2_S: the f32 after the packed codes
        if (!tensor->data_ptr) return AC_ERR_BINARY_CORRUPTED;
        const uint64_t ne0 = tensor->ne[0], ne1 = tensor->n_dims > 1 ? tensor->ne[1] : 1;
        if (ne1 != 0 && ne0 > UINT64_MAX / ne1) return AC_ERR_BINARY_CORRUPTED;
        const uint64_t packed = ne0 * ne1 / 4;
        if (packed > tensor->size_bytes || sizeof(float) > tensor->size_bytes - packed) return AC_ERR_BINARY_CORRUPTED;
        memcpy(out_scale, static_cast<const uint8_t*>(tensor->data_ptr) + packed, sizeof(float));
        return AC_SUCCESS;
    }
    if (tensor->type == 0u || tensor->type == 1u) {
        *out_scale = 1.0f;
        return AC_SUCCESS;
    }
    return AC_ERR_DEVICE_NOT_SUPPORTED;
}
