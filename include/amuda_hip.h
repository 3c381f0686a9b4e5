/*
 * amuda_hip.h -- the BitNet entry points of the reference's amuda / BitNet C ABI, on MI355X (libamuda_hip.so).
 *
 * Drop-in for the subset of the reference's amuda ABI that sits on the I2_S hot path:
 *   ac_ops_bitnet_gemv_i2_s_exact  replaces include/amuda_ops.h:73 (impl src/amuda/amuda_ops.c:299-352)
 *   bitnet_raw_vec_dot_i2_s        replaces adapters/bitnet/src/cpu/c_api.cpp:26-29
 *   ac_gguf_get_tensor_scale       replaces include/amuda_gguf.h:107 (impl src/amuda/amuda_gguf.c:659-681)
 * and the legacy context / buffer / event calls they need (include/amuda.h: ac_init, ac_destroy, ac_buffer_alloc,
 * ac_buffer_from_host, ac_buffer_sync_to_device, ac_buffer_sync_to_host, ac_buffer_free, ac_event_wait,
 * ac_event_get_duration_us, ac_event_free).
 *
 * The structs below keep the reference's field order and types (include/ac_types.h:38-91, include/amuda_gguf.h:
 * 58-68) because callers read their fields directly (buf->host_ptr, ctx->device_name, tensor->ne); the result codes
 * keep their values (include/ac_base.h:92-139). On MI355X the buffer is not unified memory: host_ptr is a pinned host
 * copy and native_mem the HBM allocation; ac_buffer_sync_to_device / _to_host copy between them (the reference's
 * cache clean / invalidate), and the ops sync their inputs to the device first, as the reference's do.
 * Single-thread-owned per context, like the reference (include/ac_types.h:11-16).
 */
#ifndef AMUDA_HIP_H
#define AMUDA_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    AC_SUCCESS = 0,
    AC_ERR_INVALID_CONTEXT = -101,
    AC_ERR_DRIVER_NOT_FOUND = -102,
    AC_ERR_DRIVER_INIT_FAILED = -105,
    AC_ERR_INVALID_ARGUMENT = -106,
    AC_ERR_FEATURE_NOT_SUPPORTED = -108,
    AC_ERR_OUT_OF_HOST_MEMORY = -201,
    AC_ERR_OUT_OF_DEVICE_MEMORY = -202,
    AC_ERR_NULL_POINTER = -205,
    AC_ERR_INVALID_BUFFER_SIZE = -206,
    AC_ERR_KERNEL_ARG_INVALID = -303,
    AC_ERR_BINARY_CORRUPTED = -304,
    AC_ERR_DEVICE_NOT_SUPPORTED = -104,
    AC_ERR_DRIVER_CRASH_OR_LOST = -601
} AcResult;

/* Legacy device context. HIP: driver_handle = NULL, platform_id = NULL, device_id = (void*)(intptr_t)ordinal,
 * context = NULL, command_queue = the context's hipStream_t. */
typedef struct {
    void* driver_handle;
    void* platform_id;
    void* device_id;
    void* context;
    void* command_queue;
    char device_name[128];
    char vendor_name[64];
    uint32_t vendor_id;
    uint32_t max_compute_units;
    uint64_t max_work_group_size;
    uint64_t max_work_item_sizes[3];
    uint64_t global_mem_size;
    uint64_t local_mem_size;
    uint32_t active_quirks;
    bool is_uma_supported;
} AcContext;

/* Buffer: host_ptr (pinned, 64-byte aligned, or the caller's memory for ac_buffer_from_host) and native_mem (HBM). */
typedef struct {
    void* host_ptr;
    void* native_mem;
    size_t size_bytes;
    uint32_t flags;
    bool is_mapped;
    bool is_user_allocated;
} AcBuffer;

/* Event of one op: native_event = this library's pair of HIP events around the kernel (opaque); the times are filled
 * by ac_event_wait / ac_event_get_duration_us. */
typedef struct {
    void* native_event;
    uint64_t submit_time_ns;
    uint64_t start_time_ns;
    uint64_t end_time_ns;
    uint64_t duration_us;
} AcEvent;

/* The GGUF tensor record the scale lookup reads (include/amuda_gguf.h:58-68). */
typedef struct {
    char name[64];
    uint32_t n_dims;
    uint64_t ne[4];
    uint32_t type; /* ggml type: 0 F32, 1 F16, 36 I2_S */
    uint64_t offset;
    void* data_ptr;
    size_t size_bytes;
    void* ac_buf; /* struct AcBuffer* in the reference (same size; a tag C++ cannot name beside the typedef) */
} GgufTensor;

AcResult ac_init(AcContext** out_ctx);
AcResult ac_destroy(AcContext* ctx);
AcResult ac_buffer_alloc(AcContext* ctx, size_t size_bytes, AcBuffer** out_buf);
AcResult ac_buffer_from_host(AcContext* ctx, void* aligned_ptr, size_t size_bytes, AcBuffer** out_buf);
AcResult ac_buffer_sync_to_device(AcContext* ctx, AcBuffer* buf);
AcResult ac_buffer_sync_to_host(AcContext* ctx, AcBuffer* buf);
AcResult ac_buffer_free(AcContext* ctx, AcBuffer* buf);
AcResult ac_event_wait(AcContext* ctx, AcEvent* event);
uint64_t ac_event_get_duration_us(AcEvent* event);
AcResult ac_event_free(AcContext* ctx, AcEvent* event);

/* y[M] = tensor_scale * (W x) with W the BitNet I2_S packing of M rows of K weights (K % 128 == 0, M * K / 4 bytes),
 * x f32 [K], code map {-1, 0, +1, 0} (amuda_ops.c:91-121). out_event (may be NULL): the kernel's event, to be freed
 * with ac_event_free. Errors as the reference: AC_ERR_NULL_POINTER, AC_ERR_KERNEL_ARG_INVALID (M, K),
 * AC_ERR_INVALID_BUFFER_SIZE (a buffer smaller than the shape). */
AcResult ac_ops_bitnet_gemv_i2_s_exact(AcContext* ctx, int M, int K, AcBuffer* x, AcBuffer* W_packed,
                                       float tensor_scale, AcBuffer* y, AcEvent** out_event);

/* The reference's raw I2_S x int8 dot on host memory (c_api.cpp:26-29 -> ggml_vec_dot_i2_i8_s): s[i] =
 * float(sum_j (c_j - 1) q_j) exactly, for kernel_type 0 (Nx1) and 2 (1x1): row i of vx (n / 4 bytes per row) against
 * vy [n]; kernel_type 1 (1xN): row 0 of vx against activation row i (vy + i * n). n % 128 == 0; invalid arguments
 * return without writing, as the reference. Runs on the GPU (copies in and out). */
void bitnet_raw_vec_dot_i2_s(int32_t n, float* s, const void* vx, const void* vy, int32_t nrc, int32_t kernel_type);

/* The f32 scale trailer of an I2_S tensor (the float after its ne0 * ne1 / 4 packed bytes); 1.0 for F32 / F16. */
AcResult ac_gguf_get_tensor_scale(const GgufTensor* tensor, float* out_scale);

#ifdef __cplusplus
}
#endif

#endif /* AMUDA_HIP_H */
