/*
 * ac_runtime_hip.h -- the reference's public ac_runtime C ABI (AMUDA 2.3), served by an MI355X HIP backend
 * (libac_runtime_hip.so).
 *
 * Drop-in for include/ac_runtime.h + include/ac_base.h + include/ac_error.h of the reference: the 53 exported names of
 * docs/abi/ac_runtime_symbols.txt:1-53 with their signatures, the descriptor layouts (sizes and offsets pinned against
 * docs/abi/ac_runtime_layout.txt), the AcResult values (ac_base.h:92-139) and the abi_version / struct_size contract
 * (ac_base.h:28-46). Handles are opaque; every out-pointer is cleared on entry; a context refuses destruction while a
 * buffer, kernel, event or batch of it lives (AC_ERR_RESOURCE_IN_USE). Single-thread-owned per context, as the
 * reference (include/ac_types.h:11-16); the error-state calls are thread-safe.
 *
 * What the HIP backend is (the reference has Vulkan and OpenCL backends, src/runtime/ac_runtime.cpp):
 *   - Context: one HIP device (the current device at creation) and one in-order, non-blocking stream of default
 *     priority. AC_BACKEND_HIP and AC_BACKEND_VULKAN (the reference's default request) both create it;
 *     ac_runtime_context_get_backend_kind reports AC_BACKEND_HIP. AC_BACKEND_OPENCL: AC_ERR_DRIVER_NOT_FOUND.
 *   - Buffers live in HBM (hipMalloc). As for the reference's OpenCL SVM buffers (ac_runtime.h:541-556) the host
 *     reaches them only through ac_runtime_buffer_write / read / fill, which are ordered after every dispatch already
 *     flushed or submitted on the context; get_mapped_ptr / flush / invalidate / is_coherent return
 *     AC_ERR_BUFFER_NOT_MAPPED; get_address gives the device address (for offset arithmetic and for HIP kernels,
 *     never for host access).
 *   - Kernels are AMDGPU code objects for the device (an ELF image, or the clang offload bundle that
 *     `hipcc --genco --offload-arch=gfx950` writes; code_size_bytes a multiple of 4, zero-padded as a SPIR-V
 *     module's would be) passed in AcKernelDesc.spirv_code / code_size_bytes; metadata.entry_point names the kernel symbol
 *     (extern "C"). SPIR-V (magic 0x07230203) returns AC_ERR_FEATURE_NOT_SUPPORTED, as does
 *     ac_runtime_kernel_create_from_source (OpenCL C). expected_spirv_sha256 is checked against the image's SHA-256
 *     (AC_ERR_BINARY_CORRUPTED on a mismatch). Arguments, in order: one pointer per binding (the start of the bound
 *     range), then -- when push_constant_size > 0 -- a struct of exactly push_constant_size bytes by value (shorter
 *     push data is zero-padded), then -- when the metadata declares specialization constants -- a struct of
 *     uint32_t value_bits, one per declared constant in ascending constant_id order (the effective values: defaults
 *     overridden by AcKernelDesc.specializations). Local-size overrides set the workgroup size of every launch.
 *   - Batches record launches on the host and issue them in order on the context's stream at flush / submit; one
 *     in-order stream already orders every dispatch after the writes of the earlier ones, so barriers cost nothing
 *     on the GPU. The automatic hazard analysis of the reference (last binding written, the others read, whole
 *     buffers) still counts barriers / elided_barriers in AcBatchStats; descriptor_cache_hits / _misses are 0 (HIP
 *     passes arguments by value, there are no descriptor sets).
 *   - Events are HIP events; gpu_duration_ns is the time between the events around the work, wall latency the host
 *     time from submission to the first observed completion.
 *   - Pipeline cache: code objects are final machine code, so the cache holds only a header naming the device
 *     architecture; merge accepts data of the same architecture and refuses any other (AC_ERR_INVALID_ARGUMENT).
 */
#ifndef AC_RUNTIME_HIP_H
#define AC_RUNTIME_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- ac_base.h ---- */
#define AC_ABI_VERSION_MAJOR 2u
#define AC_ABI_VERSION_MINOR 3u
#define AC_ABI_VERSION_PATCH 0u
#define AC_ABI_VERSION 0x00020300u
#define AC_ABI_MIN_MINOR 1u
#define AC_ABI_COMPATIBLE(v)                                                                                   \
    ((((v) >> 16) == AC_ABI_VERSION_MAJOR) && ((((v) >> 8) & 0xFFu) >= AC_ABI_MIN_MINOR) &&                    \
     ((((v) >> 8) & 0xFFu) <= AC_ABI_VERSION_MINOR) && (((v) & 0xFFu) == 0u))

typedef uint32_t AcBackendKind;
#define AC_BACKEND_UNKNOWN ((AcBackendKind)0u)
#define AC_BACKEND_VULKAN ((AcBackendKind)1u)
#define AC_BACKEND_OPENCL ((AcBackendKind)2u)
#define AC_BACKEND_HIP ((AcBackendKind)3u) /* this library: MI355X (gfx950) over HIP */

typedef uint32_t AcSpecConstantType;
#define AC_SPEC_CONSTANT_U32 ((AcSpecConstantType)0u)
#define AC_SPEC_CONSTANT_I32 ((AcSpecConstantType)1u)
#define AC_SPEC_CONSTANT_F32 ((AcSpecConstantType)2u)

typedef struct {
    uint32_t constant_id;
    AcSpecConstantType type;
    uint32_t value_bits;
} AcSpecConstant;

typedef struct {
    uint32_t constant_id;
    AcSpecConstantType type;
    uint32_t default_value_bits;
    uint32_t min_value_bits;
    uint32_t max_value_bits;
    uint32_t overrides_local_size_axis; /* 0 none, 1 x, 2 y, 3 z */
} AcSpecConstantSchemaEntry;

#define AC_PIPELINE_IDENTITY_SCHEMA_VERSION 1u
#define AC_PIPELINE_IDENTITY_SHA256_HEX_SIZE 65u

typedef enum {
    AC_SUCCESS = 0,
    AC_ERR_INVALID_CONTEXT = -101,
    AC_ERR_DRIVER_NOT_FOUND = -102,
    AC_ERR_DRIVER_SYMBOL_MISSING = -103,
    AC_ERR_DEVICE_NOT_SUPPORTED = -104,
    AC_ERR_DRIVER_INIT_FAILED = -105,
    AC_ERR_INVALID_ARGUMENT = -106,
    AC_ERR_CONTEXT_MISMATCH = -107,
    AC_ERR_FEATURE_NOT_SUPPORTED = -108,
    AC_ERR_INVALID_SHAPE = -109,
    AC_ERR_ABI_MISMATCH = -110,
    AC_ERR_BACKEND_UNAVAILABLE = -111,
    AC_ERR_OUT_OF_HOST_MEMORY = -201,
    AC_ERR_OUT_OF_DEVICE_MEMORY = -202,
    AC_ERR_BUFFER_ALIGNMENT_INVALID = -203,
    AC_ERR_BUFFER_NOT_MAPPED = -204,
    AC_ERR_NULL_POINTER = -205,
    AC_ERR_INVALID_BUFFER_SIZE = -206,
    AC_ERR_KERNEL_BUILD_FAILED = -301,
    AC_ERR_KERNEL_NOT_FOUND = -302,
    AC_ERR_KERNEL_ARG_INVALID = -303,
    AC_ERR_BINARY_CORRUPTED = -304,
    AC_ERR_INVALID_WORK_GROUP_SIZE = -401,
    AC_ERR_INVALID_WORK_ITEM_DIMS = -402,
    AC_ERR_MALI_INFINITE_LOOP_DETECTED = -403,
    AC_ERR_ADRENO_UNSAFE_SUBGROUP_OP = -404,
    AC_ERR_LAUNCH_TIMEOUT = -405,
    AC_ERR_DEVICE_BUSY = -406,
    AC_ERR_RESOURCE_IN_USE = -407,
    AC_ERR_NAN_OR_INF_DETECTED = -501,
    AC_ERR_NUMERICAL_OVERFLOW = -502,
    AC_ERR_DRIVER_CRASH_OR_LOST = -601,
    AC_ERR_OS_PROCESS_KILL_SIGNAL = -602,
    AC_ERR_THERMAL_THROTTLING_TRIPPED = -603
} AcResult;

typedef struct {
    uint32_t x;
    uint32_t y;
    uint32_t z;
} AcDim3;

/* The reference's dispatch safety budget (include/ac_dispatch.h:44-55). */
#define AC_MAX_SAFE_GROUPS_PER_AXIS 1048576u
#define AC_MAX_SAFE_TOTAL_GROUPS 16777216ull

/* ---- ac_error.h ---- */
typedef enum AmevaBackendOpKind {
    AMEVA_BACKEND_OP_NONE = 0,
    AMEVA_BACKEND_OP_BUFFER_ALLOC,
    AMEVA_BACKEND_OP_BUFFER_FREE,
    AMEVA_BACKEND_OP_BUFFER_MAP,
    AMEVA_BACKEND_OP_BUFFER_UNMAP,
    AMEVA_BACKEND_OP_COPY_HTOD,
    AMEVA_BACKEND_OP_COPY_DTOH,
    AMEVA_BACKEND_OP_DISPATCH,
    AMEVA_BACKEND_OP_SYNC
} AmevaBackendOpKind;

typedef struct AmevaBackendErrorState {
    uint64_t generation;
    int32_t first_error;
    AmevaBackendOpKind operation;
    size_t offset;
    size_t requested_bytes;
    size_t capacity_bytes;
} AmevaBackendErrorState;

#define AC_GLOBAL_CONTEXT_ID 0ULL

/* ---- ac_runtime.h ---- */
typedef struct AcContext AcContext;
typedef struct AcBuffer AcBuffer;
typedef struct AcKernel AcKernel;
typedef struct AcEvent AcEvent;
typedef struct AcCommandBatch AcCommandBatch;

typedef uint32_t AcBufferUsageFlags;
#define AC_BUFFER_USAGE_STORAGE (1u << 0)
#define AC_BUFFER_USAGE_TRANSFER_SRC (1u << 1)
#define AC_BUFFER_USAGE_TRANSFER_DST (1u << 2)
#define AC_BUFFER_USAGE_UNIFORM (1u << 3)

typedef uint32_t AcShaderStage;
#define AC_STAGE_COMPUTE ((AcShaderStage)(1u << 5))

typedef uint32_t AcRuntimeBindingType;
#define AC_RUNTIME_BINDING_STORAGE_BUFFER ((AcRuntimeBindingType)0u)
#define AC_RUNTIME_BINDING_UNIFORM_BUFFER ((AcRuntimeBindingType)1u)

typedef struct {
    uint32_t binding_index;
    AcRuntimeBindingType binding_type;
    AcShaderStage stage_flags;
} AcRuntimeBindingDesc;

typedef struct {
    const char* kernel_name;
    const char* entry_point; /* HIP: the kernel symbol in the code object */
    uint32_t binding_count;
    const AcRuntimeBindingDesc* bindings;
    size_t push_constant_size;
    AcDim3 local_size;
    uint32_t required_features;
    const char* expected_spirv_sha256; /* HIP: SHA-256 (64 hex digits) of the code object image */
    uint32_t specialization_schema_count;
    const AcSpecConstantSchemaEntry* specialization_schemas;
} AcKernelRuntimeMetadata;

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    AcBackendKind backend_kind; /* AC_BACKEND_HIP or AC_BACKEND_VULKAN: the HIP context */
    uint32_t flags;             /* must be 0 */
} AcContextDesc;

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    size_t size_bytes;
    AcBufferUsageFlags usage;
    uint32_t force_non_coherent;
} AcBufferDesc;

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    const uint32_t* spirv_code; /* HIP: the AMDGPU code object (ELF or offload bundle) */
    size_t code_size_bytes;
    const AcKernelRuntimeMetadata* metadata;
    uint32_t specialization_count;
    const AcSpecConstant* specializations;
} AcKernelDesc;

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    AcKernel* kernel;
    AcBuffer** buffers;
    uint32_t buffer_count;
    const void* push_constants;
    size_t push_constants_size;
    AcDim3 grid_dim;
} AcLaunchDesc;

#define AC_BATCH_MAX_DISPATCHES 65536u
#define AC_BATCH_FLAG_EXPLICIT_BARRIERS (1u << 0)
#define AC_BATCH_FLAG_TIMESTAMPS (1u << 1)
#define AC_BATCH_FLAG_DISPATCH_TIMESTAMPS (1u << 2)

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    uint32_t max_dispatches;
    uint32_t flags;
} AcBatchDesc;

typedef struct {
    AcBuffer* buffer;
    uint64_t offset;
    uint64_t range;
} AcBufferBinding;

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    uint32_t dispatches;
    uint32_t barriers;
    uint32_t elided_barriers;
    uint32_t flushes;
    uint64_t descriptor_cache_hits;
    uint64_t descriptor_cache_misses;
} AcBatchStats;

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    uint64_t max_storage_buffer_range;
    uint64_t min_storage_buffer_offset_alignment;
    uint64_t max_memory_allocation_size;
    uint32_t max_compute_workgroup_count[3];
    uint32_t max_compute_workgroup_size[3];
    uint32_t max_compute_workgroup_invocations;
    uint32_t max_compute_shared_memory_size;
    uint32_t max_push_constants_size;
    uint32_t subgroup_size;
    uint32_t timestamps_supported;
    float timestamp_period_ns;
    uint32_t integer_dot_product;             /* appended: filled when struct_size covers it */
    uint32_t integer_dot_product_accelerated; /* appended */
} AcDeviceLimits;

#define AC_KERNEL_SOURCE_BINDING_RANGES (1u << 0)

typedef struct {
    uint32_t abi_version;
    uint32_t struct_size;
    const char* source;
    size_t source_size;
    const char* build_options;
    const AcKernelRuntimeMetadata* metadata;
    uint32_t flags;
} AcKernelSourceDesc;

uint32_t ac_runtime_abi_version(void);

AcResult ac_runtime_context_create(const AcContextDesc* desc, AcContext** out_ctx);
AcResult ac_runtime_context_destroy(AcContext* ctx);
AcResult ac_runtime_context_get_device_name(const AcContext* ctx, char* out_name, size_t max_len);
AcResult ac_runtime_context_get_backend_kind(const AcContext* ctx, AcBackendKind* out_kind);
AcResult ac_runtime_context_get_limits(const AcContext* ctx, AcDeviceLimits* out_limits);

AcResult ac_runtime_buffer_create(AcContext* ctx, const AcBufferDesc* desc, AcBuffer** out_buf);
AcResult ac_runtime_buffer_destroy(AcBuffer* buf);
AcResult ac_runtime_buffer_get_mapped_ptr(const AcBuffer* buf, void** out_ptr);
AcResult ac_runtime_buffer_get_size(const AcBuffer* buf, size_t* out_size);
AcResult ac_runtime_buffer_get_allocation_size(const AcBuffer* buf, size_t* out_alloc_size);
AcResult ac_runtime_buffer_is_coherent(const AcBuffer* buf, uint32_t* out_is_coherent);
AcResult ac_runtime_buffer_flush(AcBuffer* buf, size_t offset, size_t size_bytes);
AcResult ac_runtime_buffer_invalidate(AcBuffer* buf, size_t offset, size_t size_bytes);
AcResult ac_runtime_buffer_write(AcBuffer* buf, size_t offset, const void* src, size_t size_bytes);
AcResult ac_runtime_buffer_read(AcBuffer* buf, size_t offset, void* dst, size_t size_bytes);
AcResult ac_runtime_buffer_fill(AcBuffer* buf, size_t offset, size_t size_bytes, uint8_t value);
AcResult ac_runtime_buffer_get_address(const AcBuffer* buf, void** out_address);

AcResult ac_runtime_kernel_create(AcContext* ctx, const AcKernelDesc* desc, AcKernel** out_kernel);
AcResult ac_runtime_kernel_create_from_source(AcContext* ctx, const AcKernelSourceDesc* desc, AcKernel** out_kernel);
AcResult ac_runtime_kernel_destroy(AcKernel* kernel);
AcResult ac_runtime_kernel_get_pipeline_identity(const AcKernel* kernel, char* out_hex, size_t out_hex_size);
AcResult ac_runtime_kernel_get_effective_local_size(const AcKernel* kernel, AcDim3* out_local_size);
AcResult ac_runtime_kernel_get_push_constant_size(const AcKernel* kernel, size_t* out_size);

AcResult ac_runtime_dispatch(AcContext* ctx, const AcLaunchDesc* desc, AcEvent** out_event);
AcResult ac_runtime_event_wait(AcEvent* event, uint64_t timeout_ns);
AcResult ac_runtime_event_get_timing(AcEvent* event, uint64_t* out_wall_latency_ns, uint64_t* out_gpu_duration_ns);
AcResult ac_runtime_event_destroy(AcEvent* event);

AcResult ac_runtime_batch_begin(AcContext* context, AcCommandBatch** out_batch);
AcResult ac_runtime_batch_begin_ex(AcContext* context, const AcBatchDesc* desc, AcCommandBatch** out_batch);
AcResult ac_runtime_batch_dispatch(AcCommandBatch* batch, AcKernel* kernel, const AcLaunchDesc* launch,
                                   AcEvent** out_event);
AcResult ac_runtime_batch_dispatch_bindings(AcCommandBatch* batch, AcKernel* kernel, const AcBufferBinding* bindings,
                                            uint32_t binding_count, const void* push_constants,
                                            size_t push_constants_size, AcDim3 grid_dim);
AcResult ac_runtime_batch_barrier(AcCommandBatch* batch);
AcResult ac_runtime_batch_flush(AcCommandBatch* batch);
AcResult ac_runtime_batch_submit(AcCommandBatch* batch, AcEvent** out_completion_event);
AcResult ac_runtime_batch_abort(AcCommandBatch* batch);
void ac_runtime_batch_destroy(AcCommandBatch* batch);
AcResult ac_runtime_batch_get_dispatch_times(const AcCommandBatch* batch, uint64_t* out_ns, uint32_t capacity,
                                             uint32_t* out_count);
AcResult ac_runtime_batch_get_stats(const AcCommandBatch* batch, AcBatchStats* out_stats);

AcResult ac_runtime_pipeline_cache_merge(AcContext* ctx, const void* data, size_t size);
AcResult ac_runtime_pipeline_cache_get_data(AcContext* ctx, void* data, size_t* inout_size);

void ac_runtime_set_error(int32_t error_code, AmevaBackendOpKind op, size_t offset, size_t requested_bytes,
                          size_t capacity_bytes);
AmevaBackendErrorState ac_runtime_get_error_state(void);
int32_t ac_runtime_consume_error(void);
uint64_t ac_runtime_advance_generation(void);
uint64_t ac_runtime_get_generation(void);
void ac_runtime_reset_error_state(void);
void ac_runtime_set_error_ctx(uint64_t context_id, int32_t error_code, AmevaBackendOpKind op, size_t offset,
                              size_t requested_bytes, size_t capacity_bytes);
AmevaBackendErrorState ac_runtime_get_error_state_ctx(uint64_t context_id);
int32_t ac_runtime_consume_error_ctx(uint64_t context_id);
uint64_t ac_runtime_advance_generation_ctx(uint64_t context_id);
uint64_t ac_runtime_get_generation_ctx(uint64_t context_id);
void ac_runtime_reset_error_state_ctx(uint64_t context_id);

#ifdef __cplusplus
}
#endif

#endif /* AC_RUNTIME_HIP_H */
