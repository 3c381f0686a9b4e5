// libac_runtime_hip.so -- the reference's ac_runtime C ABI (include/ac_runtime.h, AMUDA 2.3) on an MI355X HIP
// backend. The contract (validation order, result codes, child tracking, batch states) follows the reference's
// front end src/runtime/ac_runtime.cpp and its Vulkan batch recorder src/backend/vulkan/ac_vk_dispatch.cpp:728-1420;
// the device side is HIP: HBM buffers, AMDGPU code-object kernels launched with hipModuleLaunchKernel, one in-order
// stream per context, HIP events for timing. The header states the HIP conventions (kernel arguments, host access).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/ac_runtime_hip.h"

namespace {

constexpr uint32_t MAGIC_CONTEXT = 0xAC4A0001u;
constexpr uint32_t MAGIC_BUFFER = 0xAC4A0002u;
constexpr uint32_t MAGIC_KERNEL = 0xAC4A0003u;
constexpr uint32_t MAGIC_EVENT = 0xAC4A0004u;
constexpr uint32_t MAGIC_BATCH = 0xAC4A0005u;
constexpr size_t MAX_PUSH = 128;        // AcLaunchDesc.push_constants_size <= 128 (ac_runtime.h:136)
constexpr uint32_t MAX_BINDINGS = 16;   // ac_runtime.cpp:626-628
constexpr uint32_t MAX_SPECS = 16;      // ac_runtime.cpp:608, 662
constexpr uint64_t OFFSET_ALIGN = 4;    // binding offsets: dword aligned (HIP has no descriptor alignment rule)
constexpr size_t ALLOC_GRANULE = 256;   // allocation sizes are rounded up to this
constexpr uint32_t LEGACY_BATCH_DISPATCHES = 8;  // ac_runtime_batch_begin = begin_ex with 8 dispatches, no flags

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

// ---- SHA-256 (FIPS 180-4), for the pipeline identity and the code-object check ----
struct Sha256 {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t buf[64];
    size_t n = 0;
    uint64_t bits = 0;
    static uint32_t rotr(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }
    void block(const uint8_t* p) {
        static const uint32_t k[64] = {
            0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
            0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
            0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
            0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
            0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
            0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
            0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
            0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    void update(const void* data, size_t len) {
        const uint8_t* p = (const uint8_t*)data;
        bits += (uint64_t)len * 8;
        while (len) {
            const size_t t = std::min(len, 64 - n);
            memcpy(buf + n, p, t);
            n += t; p += t; len -= t;
            if (n == 64) { block(buf); n = 0; }
        }
    }
    void final(uint8_t out[32]) {
        const uint64_t b = bits;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (n != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(b >> (56 - 8 * i));
        update(len, 8);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
    }
};

void hex32(const uint8_t d[32], char out[65]) {
    static const char* x = "0123456789abcdef";
    for (int i = 0; i < 32; ++i) { out[2 * i] = x[d[i] >> 4]; out[2 * i + 1] = x[d[i] & 15]; }
    out[64] = '\0';
}

void le32(Sha256& s, uint32_t v) {
    const uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    s.update(b, 4);
}

AcResult hip_result(hipError_t e) {
    switch (e) {
    case hipSuccess: return AC_SUCCESS;
    case hipErrorOutOfMemory: return AC_ERR_OUT_OF_DEVICE_MEMORY;
    case hipErrorInvalidConfiguration: return AC_ERR_INVALID_WORK_GROUP_SIZE;
    case hipErrorInvalidValue: return AC_ERR_KERNEL_ARG_INVALID;
    case hipErrorNoDevice:
    case hipErrorInsufficientDriver: return AC_ERR_DRIVER_NOT_FOUND;
    default: return AC_ERR_DRIVER_CRASH_OR_LOST;
    }
}

// HBM allocation shared by the buffer handle and every recorded launch that binds it: it is released after the
// handle is destroyed and the last batch that recorded it has let go (the reference's retained references,
// ac_vk_dispatch.cpp:760-805).
struct DevMem {
    void* ptr = nullptr;
    size_t size = 0, alloc = 0;
    int device = 0;
    hipStream_t stream = nullptr;
    ~DevMem() {
        if (ptr) {
            (void)hipSetDevice(device);
            (void)hipStreamSynchronize(stream);  // no launch on the context's stream may still read it
            (void)hipFree(ptr);
        }
    }
};

struct KernelImage {
    std::vector<uint8_t> image;
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
    int device = 0;
    hipStream_t stream = nullptr;
    ~KernelImage() {
        if (module) {
            (void)hipSetDevice(device);
            (void)hipStreamSynchronize(stream);
            (void)hipModuleUnload(module);
        }
    }
};

// Completion of a piece of work: the HIP events around it, the host time it was issued and first seen complete.
struct Completion {
    hipEvent_t start = nullptr, end = nullptr;
    bool issued = false, done = false;
    uint64_t submit_ns = 0, done_ns = 0;
    ~Completion() {
        if (start) (void)hipEventDestroy(start);
        if (end) (void)hipEventDestroy(end);
    }
};

struct ErrorStates {
    std::mutex mu;
    std::unordered_map<uint64_t, AmevaBackendErrorState> map;
    AmevaBackendErrorState& get(uint64_t id) {
        auto it = map.find(id);
        if (it == map.end()) it = map.emplace(id, AmevaBackendErrorState{1, 0, AMEVA_BACKEND_OP_NONE, 0, 0, 0}).first;
        return it->second;
    }
};
ErrorStates& errors() {
    static ErrorStates e;
    return e;
}

void clear_error(AmevaBackendErrorState& s) {
    s.first_error = 0;
    s.operation = AMEVA_BACKEND_OP_NONE;
    s.offset = s.requested_bytes = s.capacity_bytes = 0;
}

}  // namespace

struct AcContext {
    uint32_t magic;
    int device;
    hipStream_t stream;
    hipDeviceProp_t prop;
    uint32_t buffers, kernels, events, batches;
};

struct AcBuffer {
    uint32_t magic;
    AcContext* ctx;
    std::shared_ptr<DevMem> mem;
};

struct AcKernel {
    uint32_t magic;
    AcContext* ctx;
    std::shared_ptr<KernelImage> img;
    uint32_t binding_count;
    size_t push_size;
    AcDim3 local;                  // effective local size (after local-size overrides)
    std::vector<uint32_t> spec;    // effective specialization values, ascending constant_id
    char identity[AC_PIPELINE_IDENTITY_SHA256_HEX_SIZE];
};

struct AcEvent {
    uint32_t magic;
    AcContext* ctx;
    std::shared_ptr<Completion> c;
};

namespace {

struct Launch {
    std::shared_ptr<KernelImage> img;
    AcDim3 grid, local;
    std::vector<std::shared_ptr<DevMem>> mems;
    std::vector<void*> ptrs;
    std::vector<uint8_t> push;
    std::vector<uint32_t> spec;
    std::shared_ptr<Completion> ev;  // a logical per-dispatch event, or null
};

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

bool ctx_ok(const AcContext* c) { return c && c->magic == MAGIC_CONTEXT; }
bool buf_ok(const AcBuffer* b) { return b && b->magic == MAGIC_BUFFER && b->mem; }
bool ker_ok(const AcKernel* k) { return k && k->magic == MAGIC_KERNEL && k->img; }

AcResult launch_one(hipStream_t st, const Launch& l) {
    std::vector<void*> params;
    params.reserve(l.ptrs.size() + 2);
    for (auto& p : l.ptrs) params.push_back((void*)&p);
    if (!l.push.empty()) params.push_back((void*)l.push.data());
    if (!l.spec.empty()) params.push_back((void*)l.spec.data());
    hipError_t e = hipModuleLaunchKernel(l.img->function, l.grid.x, l.grid.y, l.grid.z, l.local.x, l.local.y,
                                         l.local.z, 0, st, params.empty() ? nullptr : params.data(), nullptr);
    return hip_result(e);
}

AcResult new_completion(std::shared_ptr<Completion>& c) {
    try {
        c = std::make_shared<Completion>();
    } catch (...) {
        return AC_ERR_OUT_OF_HOST_MEMORY;
    }
    if (hipEventCreate(&c->start) != hipSuccess || hipEventCreate(&c->end) != hipSuccess) {
        c.reset();
        return AC_ERR_DRIVER_CRASH_OR_LOST;
    }
    return AC_SUCCESS;
}

AcEvent* wrap_event(AcContext* ctx, std::shared_ptr<Completion> c) {
    AcEvent* ev = new (std::nothrow) AcEvent;
    if (!ev) return nullptr;
    ev->magic = MAGIC_EVENT;
    ev->ctx = ctx;
    ev->c = std::move(c);
    ctx->events++;
    return ev;
}

// the dispatch safety budget of the reference (ac_vk_dispatch.cpp:251-300) plus HIP's work-item limits
AcResult check_grid(const AcDim3& g, const AcDim3& local) {
    if (g.x == 0 || g.y == 0 || g.z == 0) return AC_ERR_INVALID_WORK_GROUP_SIZE;
    if (g.x > AC_MAX_SAFE_GROUPS_PER_AXIS || g.y > AC_MAX_SAFE_GROUPS_PER_AXIS || g.z > AC_MAX_SAFE_GROUPS_PER_AXIS)
        return AC_ERR_INVALID_WORK_GROUP_SIZE;
    const uint64_t total = (uint64_t)g.x * g.y * g.z;
    if (total > AC_MAX_SAFE_TOTAL_GROUPS) return AC_ERR_INVALID_WORK_GROUP_SIZE;
    if ((uint64_t)g.x * local.x > 0xFFFFFFFFull || (uint64_t)g.y * local.y > 0xFFFFFFFFull ||
        (uint64_t)g.z * local.z > 0xFFFFFFFFull)
        return AC_ERR_INVALID_WORK_GROUP_SIZE;
    return AC_SUCCESS;
}

// Arguments of one launch: bound pointers, push data zero-padded to the kernel's size, the specialization values.
AcResult make_launch(const AcKernel* k, const std::shared_ptr<DevMem>* mems, const uint64_t* offsets, uint32_t count,
                     const void* push, size_t push_size, AcDim3 grid, Launch& l) {
    if (count != k->binding_count) return AC_ERR_KERNEL_ARG_INVALID;
    if (push_size > MAX_PUSH) return AC_ERR_INVALID_ARGUMENT;
    if (push_size > 0 && !push) return AC_ERR_NULL_POINTER;
    if (push_size > k->push_size) return AC_ERR_KERNEL_ARG_INVALID;
    const AcResult r = check_grid(grid, k->local);
    if (r != AC_SUCCESS) return r;
    try {
        l.img = k->img;
        l.grid = grid;
        l.local = k->local;
        l.mems.assign(mems, mems + count);
        l.ptrs.resize(count);
        for (uint32_t i = 0; i < count; ++i) l.ptrs[i] = (uint8_t*)mems[i]->ptr + offsets[i];
        l.push.assign(k->push_size, 0);
        if (push_size) memcpy(l.push.data(), push, push_size);
        l.spec = k->spec;
    } catch (...) {
        return AC_ERR_OUT_OF_HOST_MEMORY;
    }
    return AC_SUCCESS;
}

bool spec_in_bounds(AcSpecConstantType t, uint32_t v, uint32_t lo, uint32_t hi) {
    switch (t) {
    case AC_SPEC_CONSTANT_U32: return v >= lo && v <= hi;
    case AC_SPEC_CONSTANT_I32: {
        int32_t a, b, c;
        memcpy(&a, &v, 4); memcpy(&b, &lo, 4); memcpy(&c, &hi, 4);
        return a >= b && a <= c;
    }
    case AC_SPEC_CONSTANT_F32: {
        float a, b, c;
        memcpy(&a, &v, 4); memcpy(&b, &lo, 4); memcpy(&c, &hi, 4);
        return std::isfinite(a) && std::isfinite(b) && std::isfinite(c) && a >= b && a <= c;
    }
    default: return false;
    }
}

AcResult check_metadata(const AcKernelRuntimeMetadata* m) {
    if (!m->kernel_name || !m->kernel_name[0] || !m->entry_point || !m->entry_point[0]) return AC_ERR_INVALID_ARGUMENT;
    if (!m->expected_spirv_sha256 || strlen(m->expected_spirv_sha256) != 64) return AC_ERR_INVALID_ARGUMENT;
    if (m->local_size.x == 0 || m->local_size.y == 0 || m->local_size.z == 0) return AC_ERR_INVALID_WORK_GROUP_SIZE;
    if (m->push_constant_size > MAX_PUSH) return AC_ERR_INVALID_ARGUMENT;
    if (m->binding_count > 0 && !m->bindings) return AC_ERR_NULL_POINTER;
    if (m->binding_count > MAX_BINDINGS) return AC_ERR_INVALID_ARGUMENT;
    for (uint32_t i = 0; i < m->binding_count; ++i) {
        const AcRuntimeBindingDesc& b = m->bindings[i];
        if (b.stage_flags != AC_STAGE_COMPUTE) return AC_ERR_INVALID_ARGUMENT;
        if (b.binding_type != AC_RUNTIME_BINDING_STORAGE_BUFFER && b.binding_type != AC_RUNTIME_BINDING_UNIFORM_BUFFER)
            return AC_ERR_INVALID_ARGUMENT;
        for (uint32_t j = i + 1; j < m->binding_count; ++j)
            if (b.binding_index == m->bindings[j].binding_index) return AC_ERR_INVALID_ARGUMENT;
    }
    if (m->specialization_schema_count > MAX_SPECS) return AC_ERR_INVALID_ARGUMENT;
    if (m->specialization_schema_count > 0 && !m->specialization_schemas) return AC_ERR_NULL_POINTER;
    for (uint32_t i = 0; i < m->specialization_schema_count; ++i) {
        const AcSpecConstantSchemaEntry& s = m->specialization_schemas[i];
        if (s.type > AC_SPEC_CONSTANT_F32) return AC_ERR_INVALID_ARGUMENT;
        for (uint32_t j = i + 1; j < m->specialization_schema_count; ++j) {
            const AcSpecConstantSchemaEntry& t = m->specialization_schemas[j];
            if (s.constant_id == t.constant_id) return AC_ERR_INVALID_ARGUMENT;
            if (s.overrides_local_size_axis != 0 && s.overrides_local_size_axis == t.overrides_local_size_axis)
                return AC_ERR_INVALID_ARGUMENT;
        }
        // min <= max (finite for f32) and the default inside
        if (!spec_in_bounds(s.type, s.min_value_bits, s.min_value_bits, s.max_value_bits)) return AC_ERR_INVALID_ARGUMENT;
        if (!spec_in_bounds(s.type, s.default_value_bits, s.min_value_bits, s.max_value_bits))
            return AC_ERR_INVALID_ARGUMENT;
        if (s.overrides_local_size_axis > 3) return AC_ERR_INVALID_ARGUMENT;
        if (s.overrides_local_size_axis != 0) {
            if (s.type != AC_SPEC_CONSTANT_U32) return AC_ERR_INVALID_ARGUMENT;
            if (s.default_value_bits == 0 || s.min_value_bits == 0) return AC_ERR_INVALID_ARGUMENT;
            const uint32_t axis_size = s.overrides_local_size_axis == 1   ? m->local_size.x
                                       : s.overrides_local_size_axis == 2 ? m->local_size.y
                                                                          : m->local_size.z;
            if (s.default_value_bits != axis_size) return AC_ERR_INVALID_ARGUMENT;
        }
    }
    return AC_SUCCESS;
}

}  // namespace

extern "C" {

uint32_t ac_runtime_abi_version(void) { return AC_ABI_VERSION; }

// ---------------------------------------------------------------------------------------------------------------
// Context (ac_runtime.cpp:95-232)
// ---------------------------------------------------------------------------------------------------------------
AcResult ac_runtime_context_create(const AcContextDesc* desc, AcContext** out_ctx) {
    if (out_ctx) *out_ctx = nullptr;
    if (!desc || !out_ctx) return AC_ERR_NULL_POINTER;
    if (!AC_ABI_COMPATIBLE(desc->abi_version)) return AC_ERR_INVALID_ARGUMENT;
    if (desc->struct_size != sizeof(AcContextDesc)) return AC_ERR_INVALID_ARGUMENT;
    if (desc->flags != 0) return AC_ERR_INVALID_ARGUMENT;
    if (desc->backend_kind == AC_BACKEND_OPENCL) return AC_ERR_DRIVER_NOT_FOUND;
    if (desc->backend_kind != AC_BACKEND_HIP && desc->backend_kind != AC_BACKEND_VULKAN)
        return AC_ERR_DEVICE_NOT_SUPPORTED;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return AC_ERR_DRIVER_NOT_FOUND;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return AC_ERR_DRIVER_INIT_FAILED;
    AcContext* c = new (std::nothrow) AcContext{};
    if (!c) return AC_ERR_OUT_OF_HOST_MEMORY;
    c->device = dev;
    if (hipGetDeviceProperties(&c->prop, dev) != hipSuccess ||
        hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return AC_ERR_DRIVER_INIT_FAILED;
    }
    c->magic = MAGIC_CONTEXT;
    *out_ctx = c;
    return AC_SUCCESS;
}

AcResult ac_runtime_context_destroy(AcContext* ctx) {
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (ctx->buffers || ctx->kernels || ctx->events || ctx->batches) return AC_ERR_RESOURCE_IN_USE;
    DeviceGuard g(ctx->device);
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
    ctx->magic = 0;
    delete ctx;
    return e == hipSuccess ? AC_SUCCESS : AC_ERR_DRIVER_CRASH_OR_LOST;
}

AcResult ac_runtime_context_get_backend_kind(const AcContext* ctx, AcBackendKind* out_kind) {
    if (out_kind) *out_kind = AC_BACKEND_UNKNOWN;
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!out_kind) return AC_ERR_NULL_POINTER;
    *out_kind = AC_BACKEND_HIP;
    return AC_SUCCESS;
}

AcResult ac_runtime_context_get_device_name(const AcContext* ctx, char* out_name, size_t max_len) {
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!out_name || max_len == 0) return AC_ERR_INVALID_ARGUMENT;
    snprintf(out_name, max_len, "%s (%s)", ctx->prop.name, ctx->prop.gcnArchName);
    return AC_SUCCESS;
}

AcResult ac_runtime_context_get_limits(const AcContext* ctx, AcDeviceLimits* l) {
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!l) return AC_ERR_NULL_POINTER;
    const size_t base = offsetof(AcDeviceLimits, integer_dot_product);
    if (!AC_ABI_COMPATIBLE(l->abi_version) || l->struct_size < base || l->struct_size > sizeof(AcDeviceLimits))
        return AC_ERR_INVALID_ARGUMENT;
    const hipDeviceProp_t& p = ctx->prop;
    l->max_storage_buffer_range = (uint64_t)p.totalGlobalMem;
    l->min_storage_buffer_offset_alignment = OFFSET_ALIGN;
    l->max_memory_allocation_size = (uint64_t)p.totalGlobalMem;
    l->max_compute_workgroup_count[0] = AC_MAX_SAFE_GROUPS_PER_AXIS;
    l->max_compute_workgroup_count[1] = std::min<uint32_t>(AC_MAX_SAFE_GROUPS_PER_AXIS, (uint32_t)p.maxGridSize[1]);
    l->max_compute_workgroup_count[2] = std::min<uint32_t>(AC_MAX_SAFE_GROUPS_PER_AXIS, (uint32_t)p.maxGridSize[2]);
    for (int i = 0; i < 3; ++i) l->max_compute_workgroup_size[i] = (uint32_t)p.maxThreadsDim[i];
    l->max_compute_workgroup_invocations = (uint32_t)p.maxThreadsPerBlock;
    l->max_compute_shared_memory_size = (uint32_t)p.sharedMemPerBlock;
    l->max_push_constants_size = (uint32_t)MAX_PUSH;
    l->subgroup_size = (uint32_t)p.warpSize;
    l->timestamps_supported = 1;
    l->timestamp_period_ns = 1.0f;  // durations are reported in nanoseconds
    if (l->struct_size >= offsetof(AcDeviceLimits, integer_dot_product_accelerated) + sizeof(uint32_t)) {
        l->integer_dot_product = 1;              // v_dot4_i32_iu8
        l->integer_dot_product_accelerated = 1;
    }
    return AC_SUCCESS;
}

// ---------------------------------------------------------------------------------------------------------------
// Buffers (ac_runtime.cpp:247-532): HBM, host access through write / read / fill
// ---------------------------------------------------------------------------------------------------------------
AcResult ac_runtime_buffer_create(AcContext* ctx, const AcBufferDesc* desc, AcBuffer** out_buf) {
    if (out_buf) *out_buf = nullptr;
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!desc || !out_buf) return AC_ERR_NULL_POINTER;
    if (!AC_ABI_COMPATIBLE(desc->abi_version)) return AC_ERR_INVALID_ARGUMENT;
    if (desc->struct_size != sizeof(AcBufferDesc)) return AC_ERR_INVALID_ARGUMENT;
    if (desc->size_bytes == 0) return AC_ERR_INVALID_BUFFER_SIZE;
    const AcBufferUsageFlags known =
        AC_BUFFER_USAGE_STORAGE | AC_BUFFER_USAGE_TRANSFER_SRC | AC_BUFFER_USAGE_TRANSFER_DST | AC_BUFFER_USAGE_UNIFORM;
    if (desc->usage == 0 || (desc->usage & ~known) != 0) return AC_ERR_INVALID_ARGUMENT;
    if (desc->force_non_coherent > 1u) return AC_ERR_INVALID_ARGUMENT;
    if (desc->size_bytes > SIZE_MAX - ALLOC_GRANULE) return AC_ERR_OUT_OF_DEVICE_MEMORY;
    DeviceGuard g(ctx->device);
    std::shared_ptr<DevMem> m;
    try {
        m = std::make_shared<DevMem>();
    } catch (...) {
        return AC_ERR_OUT_OF_HOST_MEMORY;
    }
    m->size = desc->size_bytes;
    m->alloc = (desc->size_bytes + ALLOC_GRANULE - 1) / ALLOC_GRANULE * ALLOC_GRANULE;
    m->device = ctx->device;
    m->stream = ctx->stream;
    if (hipMalloc(&m->ptr, m->alloc) != hipSuccess) {
        m->ptr = nullptr;
        (void)hipGetLastError();
        return AC_ERR_OUT_OF_DEVICE_MEMORY;
    }
    AcBuffer* b = new (std::nothrow) AcBuffer;
    if (!b) return AC_ERR_OUT_OF_HOST_MEMORY;
    b->magic = MAGIC_BUFFER;
    b->ctx = ctx;
    b->mem = std::move(m);
    ctx->buffers++;
    *out_buf = b;
    return AC_SUCCESS;
}

AcResult ac_runtime_buffer_destroy(AcBuffer* buf) {
    if (!buf || buf->magic != MAGIC_BUFFER) return AC_ERR_INVALID_ARGUMENT;
    DeviceGuard g(buf->ctx->device);
    if (buf->ctx->buffers > 0) buf->ctx->buffers--;
    buf->magic = 0;
    buf->mem.reset();
    delete buf;
    return AC_SUCCESS;
}

AcResult ac_runtime_buffer_get_mapped_ptr(const AcBuffer* buf, void** out_ptr) {
    if (out_ptr) *out_ptr = nullptr;
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_ptr) return AC_ERR_NULL_POINTER;
    return AC_ERR_BUFFER_NOT_MAPPED;
}

AcResult ac_runtime_buffer_get_size(const AcBuffer* buf, size_t* out_size) {
    if (out_size) *out_size = 0;
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_size) return AC_ERR_NULL_POINTER;
    *out_size = buf->mem->size;
    return AC_SUCCESS;
}

AcResult ac_runtime_buffer_get_allocation_size(const AcBuffer* buf, size_t* out_alloc_size) {
    if (out_alloc_size) *out_alloc_size = 0;
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_alloc_size) return AC_ERR_NULL_POINTER;
    *out_alloc_size = buf->mem->alloc;
    return AC_SUCCESS;
}

AcResult ac_runtime_buffer_is_coherent(const AcBuffer* buf, uint32_t* out_is_coherent) {
    if (out_is_coherent) *out_is_coherent = 0;
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_is_coherent) return AC_ERR_NULL_POINTER;
    return AC_ERR_BUFFER_NOT_MAPPED;
}

AcResult ac_runtime_buffer_flush(AcBuffer* buf, size_t, size_t) {
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    return AC_ERR_BUFFER_NOT_MAPPED;
}

AcResult ac_runtime_buffer_invalidate(AcBuffer* buf, size_t, size_t) {
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    return AC_ERR_BUFFER_NOT_MAPPED;
}

static AcResult host_copy(AcBuffer* buf, size_t offset, void* host, size_t n, bool to_device) {
    const size_t size = buf->mem->size;
    if (offset > size || n > size - offset) return AC_ERR_INVALID_BUFFER_SIZE;
    if (n == 0) return AC_SUCCESS;
    DeviceGuard g(buf->ctx->device);
    uint8_t* d = (uint8_t*)buf->mem->ptr + offset;
    hipError_t e = to_device ? hipMemcpyAsync(d, host, n, hipMemcpyHostToDevice, buf->ctx->stream)
                             : hipMemcpyAsync(host, d, n, hipMemcpyDeviceToHost, buf->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(buf->ctx->stream);
    return e == hipSuccess ? AC_SUCCESS : AC_ERR_DRIVER_CRASH_OR_LOST;
}

AcResult ac_runtime_buffer_write(AcBuffer* buf, size_t offset, const void* src, size_t size_bytes) {
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    if (!src && size_bytes) return AC_ERR_NULL_POINTER;
    return host_copy(buf, offset, const_cast<void*>(src), size_bytes, true);
}

AcResult ac_runtime_buffer_read(AcBuffer* buf, size_t offset, void* dst, size_t size_bytes) {
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    if (!dst && size_bytes) return AC_ERR_NULL_POINTER;
    return host_copy(buf, offset, dst, size_bytes, false);
}

AcResult ac_runtime_buffer_fill(AcBuffer* buf, size_t offset, size_t size_bytes, uint8_t value) {
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    const size_t size = buf->mem->size;
    if (offset > size || size_bytes > size - offset) return AC_ERR_INVALID_BUFFER_SIZE;
    if (size_bytes == 0) return AC_SUCCESS;
    DeviceGuard g(buf->ctx->device);
    hipError_t e = hipMemsetAsync((uint8_t*)buf->mem->ptr + offset, value, size_bytes, buf->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(buf->ctx->stream);
    return e == hipSuccess ? AC_SUCCESS : AC_ERR_DRIVER_CRASH_OR_LOST;
}

AcResult ac_runtime_buffer_get_address(const AcBuffer* buf, void** out_address) {
    if (out_address) *out_address = nullptr;
    if (!buf_ok(buf)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_address) return AC_ERR_NULL_POINTER;
    *out_address = buf->mem->ptr;
    return AC_SUCCESS;
}

// ---------------------------------------------------------------------------------------------------------------
// Kernels (ac_runtime.cpp:586-1076): AMDGPU code objects
// ---------------------------------------------------------------------------------------------------------------
AcResult ac_runtime_kernel_create(AcContext* ctx, const AcKernelDesc* desc, AcKernel** out_kernel) {
    if (out_kernel) *out_kernel = nullptr;
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!desc || !out_kernel) return AC_ERR_NULL_POINTER;
    if (!AC_ABI_COMPATIBLE(desc->abi_version)) return AC_ERR_INVALID_ARGUMENT;
    if (desc->struct_size != sizeof(AcKernelDesc)) return AC_ERR_INVALID_ARGUMENT;
    if (!desc->spirv_code) return AC_ERR_NULL_POINTER;
    if (desc->code_size_bytes == 0 || desc->code_size_bytes % 4 != 0) return AC_ERR_INVALID_ARGUMENT;
    if (!desc->metadata) return AC_ERR_NULL_POINTER;
    if (desc->specialization_count > MAX_SPECS) return AC_ERR_INVALID_ARGUMENT;
    if (desc->specialization_count > 0 && !desc->specializations) return AC_ERR_NULL_POINTER;
    const AcKernelRuntimeMetadata* m = desc->metadata;
    AcResult r = check_metadata(m);
    if (r != AC_SUCCESS) return r;
    for (uint32_t i = 0; i < desc->specialization_count; ++i) {
        const AcSpecConstant& s = desc->specializations[i];
        if (s.type > AC_SPEC_CONSTANT_F32) return AC_ERR_INVALID_ARGUMENT;
        for (uint32_t j = i + 1; j < desc->specialization_count; ++j)
            if (s.constant_id == desc->specializations[j].constant_id) return AC_ERR_INVALID_ARGUMENT;
        const AcSpecConstantSchemaEntry* match = nullptr;
        for (uint32_t k = 0; k < m->specialization_schema_count; ++k)
            if (m->specialization_schemas[k].constant_id == s.constant_id) match = &m->specialization_schemas[k];
        if (!match) return AC_ERR_KERNEL_ARG_INVALID;
        if (s.type != match->type) return AC_ERR_INVALID_ARGUMENT;
        if (match->overrides_local_size_axis != 0 && s.value_bits == 0) return AC_ERR_INVALID_ARGUMENT;
        if (!spec_in_bounds(match->type, s.value_bits, match->min_value_bits, match->max_value_bits))
            return AC_ERR_INVALID_ARGUMENT;
    }

    // what the image is: SPIR-V is the Vulkan backend's; this backend loads AMDGPU code objects, as an ELF or as the
    // clang offload bundle `hipcc --genco` writes
    const uint8_t* code = (const uint8_t*)desc->spirv_code;
    if (desc->spirv_code[0] == 0x07230203u) return AC_ERR_FEATURE_NOT_SUPPORTED;
    static const char bundle[] = "__CLANG_OFFLOAD_BUNDLE__";
    const bool elf = code[0] == 0x7F && code[1] == 'E' && code[2] == 'L' && code[3] == 'F';
    const bool is_bundle = desc->code_size_bytes >= sizeof(bundle) - 1 && memcmp(code, bundle, sizeof(bundle) - 1) == 0;
    if (!elf && !is_bundle) return AC_ERR_BINARY_CORRUPTED;
    uint8_t digest[32];
    char hex[65];
    {
        Sha256 s;
        s.update(code, desc->code_size_bytes);
        s.final(digest);
        hex32(digest, hex);
        for (int i = 0; i < 64; ++i) {
            const char c = m->expected_spirv_sha256[i];
            const char lc = (c >= 'A' && c <= 'F') ? (char)(c - 'A' + 'a') : c;
            if (lc != hex[i]) return AC_ERR_BINARY_CORRUPTED;
        }
    }

    // effective specialization set (defaults overridden by the caller) and local size
    std::vector<AcSpecConstant> eff;
    AcDim3 local = m->local_size;
    for (uint32_t k = 0; k < m->specialization_schema_count; ++k) {
        const AcSpecConstantSchemaEntry& s = m->specialization_schemas[k];
        uint32_t v = s.default_value_bits;
        for (uint32_t c = 0; c < desc->specialization_count; ++c)
            if (desc->specializations[c].constant_id == s.constant_id) v = desc->specializations[c].value_bits;
        eff.push_back({s.constant_id, s.type, v});
        if (s.overrides_local_size_axis == 1) local.x = v;
        if (s.overrides_local_size_axis == 2) local.y = v;
        if (s.overrides_local_size_axis == 3) local.z = v;
    }
    std::sort(eff.begin(), eff.end(), [](const AcSpecConstant& a, const AcSpecConstant& b) {
        return a.constant_id < b.constant_id;
    });
    const uint64_t threads = (uint64_t)local.x * local.y * local.z;
    if (local.x > (uint32_t)ctx->prop.maxThreadsDim[0] || local.y > (uint32_t)ctx->prop.maxThreadsDim[1] ||
        local.z > (uint32_t)ctx->prop.maxThreadsDim[2] || threads > (uint64_t)ctx->prop.maxThreadsPerBlock)
        return AC_ERR_INVALID_WORK_GROUP_SIZE;

    // the reference's canonical pipeline identity (ac_runtime.cpp:787-838): domain, schema version, image digest,
    // entry point, effective specialization entries
    char identity[AC_PIPELINE_IDENTITY_SHA256_HEX_SIZE];
    {
        static const uint8_t domain[18] = {'A', 'M', 'E', 'V', 'A', '-', 'P', 'I', 'P',
                                           'E', 'L', 'I', 'N', 'E', '-', 'I', 'D', '\0'};
        Sha256 s;
        s.update(domain, sizeof(domain));
        le32(s, AC_PIPELINE_IDENTITY_SCHEMA_VERSION);
        s.update(digest, 32);
        const size_t ep = strlen(m->entry_point);
        le32(s, (uint32_t)ep);
        s.update(m->entry_point, ep);
        le32(s, (uint32_t)eff.size());
        for (const AcSpecConstant& e : eff) {
            le32(s, e.constant_id);
            le32(s, e.type);
            le32(s, e.value_bits);
        }
        uint8_t d[32];
        s.final(d);
        hex32(d, identity);
    }

    DeviceGuard g(ctx->device);
    std::shared_ptr<KernelImage> img;
    try {
        img = std::make_shared<KernelImage>();
        img->image.assign(code, code + desc->code_size_bytes);
    } catch (...) {
        return AC_ERR_OUT_OF_HOST_MEMORY;
    }
    img->device = ctx->device;
    img->stream = ctx->stream;
    if (hipModuleLoadData(&img->module, img->image.data()) != hipSuccess) {
        img->module = nullptr;
        (void)hipGetLastError();
        return AC_ERR_BINARY_CORRUPTED;
    }
    if (hipModuleGetFunction(&img->function, img->module, m->entry_point) != hipSuccess) {
        (void)hipGetLastError();
        return AC_ERR_KERNEL_NOT_FOUND;
    }
    AcKernel* k = new (std::nothrow) AcKernel;
    if (!k) return AC_ERR_OUT_OF_HOST_MEMORY;
    k->magic = MAGIC_KERNEL;
    k->ctx = ctx;
    k->img = std::move(img);
    k->binding_count = m->binding_count;
    k->push_size = m->push_constant_size;
    k->local = local;
    for (const AcSpecConstant& e : eff) k->spec.push_back(e.value_bits);
    memcpy(k->identity, identity, sizeof(identity));
    ctx->kernels++;
    *out_kernel = k;
    return AC_SUCCESS;
}

AcResult ac_runtime_kernel_create_from_source(AcContext* ctx, const AcKernelSourceDesc* desc, AcKernel** out_kernel) {
    if (out_kernel) *out_kernel = nullptr;
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!desc || !out_kernel) return AC_ERR_NULL_POINTER;
    if (desc->abi_version < 0x00020300u || !AC_ABI_COMPATIBLE(desc->abi_version) ||
        desc->struct_size != sizeof(AcKernelSourceDesc))
        return AC_ERR_INVALID_ARGUMENT;
    return AC_ERR_FEATURE_NOT_SUPPORTED;  // OpenCL C: the reference's OpenCL backend; this one takes code objects
}

AcResult ac_runtime_kernel_destroy(AcKernel* kernel) {
    if (!kernel || kernel->magic != MAGIC_KERNEL) return AC_ERR_INVALID_ARGUMENT;
    DeviceGuard g(kernel->ctx->device);
    if (kernel->ctx->kernels > 0) kernel->ctx->kernels--;
    kernel->magic = 0;
    kernel->img.reset();
    delete kernel;
    return AC_SUCCESS;
}

AcResult ac_runtime_kernel_get_pipeline_identity(const AcKernel* kernel, char* out_hex, size_t out_hex_size) {
    if (out_hex && out_hex_size > 0) out_hex[0] = '\0';
    if (!ker_ok(kernel)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_hex) return AC_ERR_NULL_POINTER;
    if (out_hex_size < AC_PIPELINE_IDENTITY_SHA256_HEX_SIZE) return AC_ERR_INVALID_ARGUMENT;
    memcpy(out_hex, kernel->identity, AC_PIPELINE_IDENTITY_SHA256_HEX_SIZE);
    return AC_SUCCESS;
}

AcResult ac_runtime_kernel_get_effective_local_size(const AcKernel* kernel, AcDim3* out_local_size) {
    if (out_local_size) *out_local_size = AcDim3{0, 0, 0};
    if (!ker_ok(kernel)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_local_size) return AC_ERR_NULL_POINTER;
    *out_local_size = kernel->local;
    return AC_SUCCESS;
}

AcResult ac_runtime_kernel_get_push_constant_size(const AcKernel* kernel, size_t* out_size) {
    if (!out_size) return AC_ERR_NULL_POINTER;
    *out_size = 0;
    if (!ker_ok(kernel)) return AC_ERR_INVALID_ARGUMENT;
    *out_size = kernel->push_size;
    return AC_SUCCESS;
}

// ---------------------------------------------------------------------------------------------------------------
// Dispatch and events (ac_runtime.cpp:1080-1300)
// ---------------------------------------------------------------------------------------------------------------
AcResult ac_runtime_dispatch(AcContext* ctx, const AcLaunchDesc* desc, AcEvent** out_event) {
    if (out_event) *out_event = nullptr;
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!desc) return AC_ERR_NULL_POINTER;
    if (!AC_ABI_COMPATIBLE(desc->abi_version)) return AC_ERR_INVALID_ARGUMENT;
    if (desc->struct_size != sizeof(AcLaunchDesc)) return AC_ERR_INVALID_ARGUMENT;
    if (!desc->kernel || desc->kernel->magic != MAGIC_KERNEL) return AC_ERR_INVALID_ARGUMENT;
    if (desc->kernel->ctx != ctx) return AC_ERR_CONTEXT_MISMATCH;
    if (desc->grid_dim.x == 0 || desc->grid_dim.y == 0 || desc->grid_dim.z == 0) return AC_ERR_INVALID_WORK_GROUP_SIZE;
    if (desc->buffer_count > 0 && !desc->buffers) return AC_ERR_NULL_POINTER;
    if (desc->buffer_count > MAX_BINDINGS) return AC_ERR_INVALID_ARGUMENT;
    std::shared_ptr<DevMem> mems[MAX_BINDINGS];
    uint64_t offs[MAX_BINDINGS] = {};
    for (uint32_t i = 0; i < desc->buffer_count; ++i) {
        const AcBuffer* b = desc->buffers[i];
        if (!b || b->magic != MAGIC_BUFFER) return AC_ERR_NULL_POINTER;
        if (b->ctx != ctx) return AC_ERR_CONTEXT_MISMATCH;
        mems[i] = b->mem;
    }
    Launch l;
    AcResult r = make_launch(desc->kernel, mems, offs, desc->buffer_count, desc->push_constants,
                             desc->push_constants_size, desc->grid_dim, l);
    if (r != AC_SUCCESS) return r;
    std::shared_ptr<Completion> c;
    r = new_completion(c);
    if (r != AC_SUCCESS) return r;
    DeviceGuard g(ctx->device);
    c->submit_ns = now_ns();
    if (hipEventRecord(c->start, ctx->stream) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
    r = launch_one(ctx->stream, l);
    if (r != AC_SUCCESS) {
        (void)hipGetLastError();
        return r;
    }
    if (hipEventRecord(c->end, ctx->stream) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
    c->issued = true;
    if (!out_event) {  // synchronous contract: returns after the GPU finished
        const hipError_t e = hipEventSynchronize(c->end);
        return e == hipSuccess ? AC_SUCCESS : AC_ERR_DRIVER_CRASH_OR_LOST;
    }
    AcEvent* ev = wrap_event(ctx, std::move(c));
    if (!ev) return AC_ERR_OUT_OF_HOST_MEMORY;
    *out_event = ev;
    return AC_SUCCESS;
}

static AcResult completion_poll(Completion& c, bool& done) {
    done = c.done;
    if (done) return AC_SUCCESS;
    const hipError_t e = hipEventQuery(c.end);
    if (e == hipSuccess) {
        c.done = true;
        c.done_ns = now_ns();
        done = true;
        return AC_SUCCESS;
    }
    if (e == hipErrorNotReady) return AC_SUCCESS;
    return AC_ERR_DRIVER_CRASH_OR_LOST;
}

AcResult ac_runtime_event_wait(AcEvent* event, uint64_t timeout_ns) {
    if (!event || event->magic != MAGIC_EVENT || !event->c) return AC_ERR_INVALID_ARGUMENT;
    Completion& c = *event->c;
    if (!c.issued) return AC_ERR_INVALID_ARGUMENT;  // its batch was not flushed or submitted yet
    DeviceGuard g(event->ctx->device);
    const uint64_t t0 = now_ns();
    for (;;) {
        bool done = false;
        const AcResult r = completion_poll(c, done);
        if (r != AC_SUCCESS) return r;
        if (done) return AC_SUCCESS;
        if (timeout_ns == UINT64_MAX) {
            if (hipEventSynchronize(c.end) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
            continue;
        }
        if (now_ns() - t0 >= timeout_ns) return AC_ERR_LAUNCH_TIMEOUT;
        std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

AcResult ac_runtime_event_get_timing(AcEvent* event, uint64_t* out_wall_latency_ns, uint64_t* out_gpu_duration_ns) {
    if (!event || event->magic != MAGIC_EVENT || !event->c) return AC_ERR_INVALID_ARGUMENT;
    if (!out_wall_latency_ns && !out_gpu_duration_ns) return AC_ERR_NULL_POINTER;
    Completion& c = *event->c;
    if (!c.issued) return AC_ERR_INVALID_ARGUMENT;
    DeviceGuard g(event->ctx->device);
    bool done = false;
    const AcResult r = completion_poll(c, done);
    if (r != AC_SUCCESS) return r;
    if (!done) return AC_ERR_DEVICE_BUSY;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, c.start, c.end) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
    if (out_wall_latency_ns) *out_wall_latency_ns = c.done_ns - c.submit_ns;
    if (out_gpu_duration_ns) *out_gpu_duration_ns = (uint64_t)std::llround((double)ms * 1e6);
    return AC_SUCCESS;
}

AcResult ac_runtime_event_destroy(AcEvent* event) {
    if (!event || event->magic != MAGIC_EVENT) return AC_ERR_INVALID_ARGUMENT;
    DeviceGuard g(event->ctx->device);
    if (event->ctx->events > 0) event->ctx->events--;
    event->magic = 0;
    event->c.reset();
    delete event;
    return AC_SUCCESS;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------------------------
// Batches (ac_runtime.cpp:1304-1520, 1583-1765; recorder semantics ac_vk_dispatch.cpp:728-1420)
// ---------------------------------------------------------------------------------------------------------------
struct AcCommandBatch {
    enum State { RECORDING, SUBMITTED, ABORTED };
    uint32_t magic;
    AcContext* ctx;
    uint32_t max_dispatches, flags;
    State state = RECORDING;
    std::vector<Launch> recs;
    size_t issued = 0;
    uint32_t dispatches = 0, barriers = 0, elided = 0, flushes = 0;
    std::vector<const DevMem*> read, written;  // automatic hazard analysis since the last barrier
    hipEvent_t t0 = nullptr;                   // batch start, recorded before its first launch
    std::vector<hipEvent_t> ts;                // after every dispatch (AC_BATCH_FLAG_DISPATCH_TIMESTAMPS)
    std::shared_ptr<Completion> done;          // the submission's completion
    ~AcCommandBatch() {
        if (t0) (void)hipEventDestroy(t0);
        for (hipEvent_t e : ts) (void)hipEventDestroy(e);
    }
};

namespace {

bool batch_ok(const AcCommandBatch* b) { return b && b->magic == MAGIC_BATCH; }

AcResult batch_new(AcContext* ctx, uint32_t max_dispatches, uint32_t flags, AcCommandBatch** out) {
    AcCommandBatch* b = new (std::nothrow) AcCommandBatch;
    if (!b) return AC_ERR_OUT_OF_HOST_MEMORY;
    b->magic = MAGIC_BATCH;
    b->ctx = ctx;
    b->max_dispatches = max_dispatches;
    b->flags = flags;
    ctx->batches++;
    *out = b;
    return AC_SUCCESS;
}

// issue every recorded, not yet issued launch on the context's stream, in order
AcResult batch_issue(AcCommandBatch* b) {
    DeviceGuard g(b->ctx->device);
    hipStream_t st = b->ctx->stream;
    if (!b->t0) {
        if (hipEventCreate(&b->t0) != hipSuccess || hipEventRecord(b->t0, st) != hipSuccess)
            return AC_ERR_DRIVER_CRASH_OR_LOST;
    }
    for (; b->issued < b->recs.size(); ++b->issued) {
        Launch& l = b->recs[b->issued];
        if (l.ev) {
            l.ev->submit_ns = now_ns();
            if (hipEventRecord(l.ev->start, st) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
        }
        AcResult r = launch_one(st, l);
        if (r != AC_SUCCESS) {
            (void)hipGetLastError();
            return r;
        }
        if (l.ev) {
            if (hipEventRecord(l.ev->end, st) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
            l.ev->issued = true;
        }
        if (b->flags & AC_BATCH_FLAG_DISPATCH_TIMESTAMPS) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
            b->ts.push_back(e);
            if (hipEventRecord(e, st) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
        }
    }
    return AC_SUCCESS;
}

AcResult batch_record(AcCommandBatch* b, AcKernel* k, const std::shared_ptr<DevMem>* mems, const uint64_t* offsets,
                      uint32_t count, const void* push, size_t push_size, AcDim3 grid, AcEvent** out_event) {
    if (b->state != AcCommandBatch::RECORDING) return AC_ERR_INVALID_ARGUMENT;
    if (b->dispatches >= b->max_dispatches) return AC_ERR_DEVICE_BUSY;
    Launch l;
    AcResult r = make_launch(k, mems, offsets, count, push, push_size, grid, l);
    if (r != AC_SUCCESS) return r;
    if (out_event) {
        r = new_completion(l.ev);
        if (r != AC_SUCCESS) return r;
    }
    // hazard analysis of the reference's recorder (ac_vk_dispatch.cpp:771-784): the last binding is written, the
    // others read; a dispatch that writes what was read, or touches what was written, since the last barrier needs
    // one. On one in-order HIP stream the order is kept anyway; the analysis feeds AcBatchStats.
    if (!(b->flags & AC_BATCH_FLAG_EXPLICIT_BARRIERS) && count > 0) {
        auto has = [](const std::vector<const DevMem*>& v, const DevMem* x) {
            return std::find(v.begin(), v.end(), x) != v.end();
        };
        const DevMem* w = mems[count - 1].get();
        bool hazard = has(b->read, w);
        for (uint32_t i = 0; i < count && !hazard; ++i) hazard = has(b->written, mems[i].get());
        if (hazard) {
            b->barriers++;
            b->read.clear();
            b->written.clear();
        } else {
            b->elided++;
        }
        for (uint32_t i = 0; i + 1 < count; ++i)
            if (!has(b->read, mems[i].get())) b->read.push_back(mems[i].get());
        if (!has(b->written, w)) b->written.push_back(w);
    }
    AcEvent* ev = nullptr;
    if (out_event) {
        ev = wrap_event(b->ctx, l.ev);
        if (!ev) return AC_ERR_OUT_OF_HOST_MEMORY;
    }
    try {
        b->recs.push_back(std::move(l));
    } catch (...) {
        if (ev) ac_runtime_event_destroy(ev);
        return AC_ERR_OUT_OF_HOST_MEMORY;
    }
    b->dispatches++;
    if (out_event) *out_event = ev;
    return AC_SUCCESS;
}

void batch_drop_unissued(AcCommandBatch* b) {
    b->recs.erase(b->recs.begin() + (ptrdiff_t)b->issued, b->recs.end());
}

}  // namespace

extern "C" {

AcResult ac_runtime_batch_begin(AcContext* context, AcCommandBatch** out_batch) {
    if (out_batch) *out_batch = nullptr;
    if (!context || !out_batch) return AC_ERR_NULL_POINTER;
    if (context->magic != MAGIC_CONTEXT) return AC_ERR_INVALID_CONTEXT;
    return batch_new(context, LEGACY_BATCH_DISPATCHES, 0, out_batch);
}

AcResult ac_runtime_batch_begin_ex(AcContext* context, const AcBatchDesc* desc, AcCommandBatch** out_batch) {
    if (out_batch) *out_batch = nullptr;
    if (!context || !desc || !out_batch) return AC_ERR_NULL_POINTER;
    if (context->magic != MAGIC_CONTEXT) return AC_ERR_INVALID_CONTEXT;
    if (!AC_ABI_COMPATIBLE(desc->abi_version) || desc->struct_size != sizeof(AcBatchDesc))
        return AC_ERR_INVALID_ARGUMENT;
    if (desc->max_dispatches == 0 || desc->max_dispatches > AC_BATCH_MAX_DISPATCHES) return AC_ERR_INVALID_ARGUMENT;
    if (desc->flags & ~(AC_BATCH_FLAG_EXPLICIT_BARRIERS | AC_BATCH_FLAG_TIMESTAMPS | AC_BATCH_FLAG_DISPATCH_TIMESTAMPS))
        return AC_ERR_INVALID_ARGUMENT;
    return batch_new(context, desc->max_dispatches, desc->flags, out_batch);
}

AcResult ac_runtime_batch_dispatch(AcCommandBatch* batch, AcKernel* kernel, const AcLaunchDesc* launch,
                                   AcEvent** out_event) {
    if (out_event) *out_event = nullptr;
    if (!batch || !kernel || !launch) return AC_ERR_NULL_POINTER;
    if (batch->magic != MAGIC_BATCH) return AC_ERR_INVALID_ARGUMENT;
    if (kernel->magic != MAGIC_KERNEL) return AC_ERR_INVALID_ARGUMENT;
    if (!AC_ABI_COMPATIBLE(launch->abi_version) || launch->struct_size != sizeof(AcLaunchDesc))
        return AC_ERR_INVALID_ARGUMENT;
    if (launch->kernel != kernel) return AC_ERR_INVALID_ARGUMENT;
    if (kernel->ctx != batch->ctx) return AC_ERR_CONTEXT_MISMATCH;
    if (launch->buffer_count > MAX_BINDINGS) return AC_ERR_INVALID_ARGUMENT;
    if (launch->buffer_count > 0 && !launch->buffers) return AC_ERR_NULL_POINTER;
    std::shared_ptr<DevMem> mems[MAX_BINDINGS];
    uint64_t offs[MAX_BINDINGS] = {};
    for (uint32_t i = 0; i < launch->buffer_count; ++i) {
        const AcBuffer* b = launch->buffers[i];
        if (!b || b->magic != MAGIC_BUFFER) return AC_ERR_NULL_POINTER;
        if (b->ctx != batch->ctx) return AC_ERR_CONTEXT_MISMATCH;
        mems[i] = b->mem;
    }
    return batch_record(batch, kernel, mems, offs, launch->buffer_count, launch->push_constants,
                        launch->push_constants_size, launch->grid_dim, out_event);
}

AcResult ac_runtime_batch_dispatch_bindings(AcCommandBatch* batch, AcKernel* kernel, const AcBufferBinding* bindings,
                                            uint32_t binding_count, const void* push_constants,
                                            size_t push_constants_size, AcDim3 grid_dim) {
    if (!batch || !kernel || (binding_count > 0 && !bindings)) return AC_ERR_NULL_POINTER;
    if (batch->magic != MAGIC_BATCH || !ker_ok(kernel)) return AC_ERR_INVALID_ARGUMENT;
    if (kernel->ctx != batch->ctx) return AC_ERR_CONTEXT_MISMATCH;
    if (binding_count > MAX_BINDINGS) return AC_ERR_INVALID_ARGUMENT;
    if (push_constants_size > MAX_PUSH || (push_constants_size > 0 && !push_constants)) return AC_ERR_INVALID_ARGUMENT;
    std::shared_ptr<DevMem> mems[MAX_BINDINGS];
    uint64_t offs[MAX_BINDINGS];
    for (uint32_t i = 0; i < binding_count; ++i) {
        const AcBuffer* b = bindings[i].buffer;
        if (!b || b->magic != MAGIC_BUFFER || !b->mem) return AC_ERR_NULL_POINTER;
        if (b->ctx != batch->ctx) return AC_ERR_CONTEXT_MISMATCH;
        const uint64_t off = bindings[i].offset, range = bindings[i].range, size = b->mem->size;
        if (off % OFFSET_ALIGN != 0) return AC_ERR_BUFFER_ALIGNMENT_INVALID;
        if (range == 0 || off >= size || range > size - off) return AC_ERR_INVALID_BUFFER_SIZE;
        mems[i] = b->mem;
        offs[i] = off;
    }
    return batch_record(batch, kernel, mems, offs, binding_count, push_constants, push_constants_size, grid_dim,
                        nullptr);
}

AcResult ac_runtime_batch_barrier(AcCommandBatch* batch) {
    if (!batch_ok(batch)) return AC_ERR_INVALID_ARGUMENT;
    if (batch->state != AcCommandBatch::RECORDING) return AC_ERR_INVALID_ARGUMENT;
    // one in-order stream: the next launch already sees every earlier write; the barrier is bookkeeping
    batch->barriers++;
    batch->read.clear();
    batch->written.clear();
    return AC_SUCCESS;
}

AcResult ac_runtime_batch_flush(AcCommandBatch* batch) {
    if (!batch_ok(batch)) return AC_ERR_INVALID_ARGUMENT;
    if (batch->state != AcCommandBatch::RECORDING) return AC_ERR_INVALID_ARGUMENT;
    if (batch->issued == batch->recs.size()) return AC_SUCCESS;  // nothing recorded since the last flush
    const AcResult r = batch_issue(batch);
    if (r != AC_SUCCESS) {
        batch_drop_unissued(batch);
        batch->state = AcCommandBatch::ABORTED;
        return r;
    }
    batch->flushes++;
    return AC_SUCCESS;
}

AcResult ac_runtime_batch_submit(AcCommandBatch* batch, AcEvent** out_completion_event) {
    if (out_completion_event) *out_completion_event = nullptr;
    if (!batch_ok(batch)) return AC_ERR_INVALID_ARGUMENT;
    if (batch->state != AcCommandBatch::RECORDING) return AC_ERR_INVALID_ARGUMENT;
    std::shared_ptr<Completion> c;
    AcResult r = new_completion(c);
    if (r != AC_SUCCESS) return r;
    r = batch_issue(batch);
    if (r != AC_SUCCESS) {
        batch_drop_unissued(batch);
        batch->state = AcCommandBatch::ABORTED;
        return r;
    }
    DeviceGuard g(batch->ctx->device);
    c->submit_ns = now_ns();
    // the completion spans the batch from its first launch (t0 is already on the stream) to now
    if (hipEventRecord(c->start, batch->ctx->stream) != hipSuccess ||
        hipEventRecord(c->end, batch->ctx->stream) != hipSuccess)
        return AC_ERR_DRIVER_CRASH_OR_LOST;
    std::swap(c->start, batch->t0);  // the batch's start event measures the whole submission
    c->issued = true;
    batch->done = c;
    batch->state = AcCommandBatch::SUBMITTED;
    if (out_completion_event) {
        AcEvent* ev = wrap_event(batch->ctx, std::move(c));
        if (!ev) return AC_ERR_OUT_OF_HOST_MEMORY;
        *out_completion_event = ev;
    }
    return AC_SUCCESS;
}

AcResult ac_runtime_batch_abort(AcCommandBatch* batch) {
    if (!batch_ok(batch)) return AC_ERR_INVALID_ARGUMENT;
    if (batch->state == AcCommandBatch::ABORTED) return AC_SUCCESS;
    if (batch->state != AcCommandBatch::RECORDING) return AC_ERR_INVALID_ARGUMENT;
    batch_drop_unissued(batch);
    batch->state = AcCommandBatch::ABORTED;
    return AC_SUCCESS;
}

void ac_runtime_batch_destroy(AcCommandBatch* batch) {
    if (!batch_ok(batch)) return;
    if (batch->state == AcCommandBatch::RECORDING) ac_runtime_batch_abort(batch);
    DeviceGuard g(batch->ctx->device);
    if (batch->ctx->batches > 0) batch->ctx->batches--;
    batch->magic = 0;
    delete batch;  // launches already issued keep running; the events obtained from the batch stay valid
}

AcResult ac_runtime_batch_get_dispatch_times(const AcCommandBatch* batch, uint64_t* out_ns, uint32_t capacity,
                                             uint32_t* out_count) {
    if (out_count) *out_count = 0;
    if (!batch_ok(batch)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_ns || !out_count) return AC_ERR_NULL_POINTER;
    if (!(batch->flags & AC_BATCH_FLAG_DISPATCH_TIMESTAMPS)) return AC_ERR_FEATURE_NOT_SUPPORTED;
    if (batch->state != AcCommandBatch::SUBMITTED || !batch->done) return AC_ERR_DEVICE_BUSY;
    DeviceGuard g(batch->ctx->device);
    bool done = false;
    const AcResult r = completion_poll(*batch->done, done);
    if (r != AC_SUCCESS) return r;
    if (!done) return AC_ERR_DEVICE_BUSY;
    const uint32_t n = (uint32_t)batch->ts.size();
    if (capacity < n) return AC_ERR_INVALID_ARGUMENT;
    hipEvent_t prev = batch->done->start;  // the batch start
    for (uint32_t i = 0; i < n; ++i) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, prev, batch->ts[i]) != hipSuccess) return AC_ERR_DRIVER_CRASH_OR_LOST;
        out_ns[i] = (uint64_t)std::llround((double)std::max(ms, 0.0f) * 1e6);
        prev = batch->ts[i];
    }
    *out_count = n;
    return AC_SUCCESS;
}

AcResult ac_runtime_batch_get_stats(const AcCommandBatch* batch, AcBatchStats* out_stats) {
    if (!batch_ok(batch)) return AC_ERR_INVALID_ARGUMENT;
    if (!out_stats) return AC_ERR_NULL_POINTER;
    if (!AC_ABI_COMPATIBLE(out_stats->abi_version) || out_stats->struct_size != sizeof(AcBatchStats))
        return AC_ERR_INVALID_ARGUMENT;
    out_stats->dispatches = batch->dispatches;
    out_stats->barriers = batch->barriers;
    out_stats->elided_barriers = batch->elided;
    out_stats->flushes = batch->flushes;
    out_stats->descriptor_cache_hits = 0;
    out_stats->descriptor_cache_misses = 0;
    return AC_SUCCESS;
}

// ---------------------------------------------------------------------------------------------------------------
// Pipeline cache: a header naming the device architecture (code objects need no compilation to cache)
// ---------------------------------------------------------------------------------------------------------------
namespace {
struct CacheHeader {
    char magic[8];
    uint32_t version;
    uint32_t header_size;
    char arch[64];
    uint64_t entries;
};
constexpr char CACHE_MAGIC[8] = {'A', 'C', 'H', 'I', 'P', 'P', 'C', '1'};
CacheHeader cache_header(const AcContext* ctx) {
    CacheHeader h{};
    memcpy(h.magic, CACHE_MAGIC, 8);
    h.version = 1;
    h.header_size = (uint32_t)sizeof(CacheHeader);
    snprintf(h.arch, sizeof(h.arch), "%s", ctx->prop.gcnArchName);
    return h;
}
}  // namespace

AcResult ac_runtime_pipeline_cache_merge(AcContext* ctx, const void* data, size_t size) {
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!data) return AC_ERR_NULL_POINTER;
    if (size < sizeof(CacheHeader)) return AC_ERR_INVALID_ARGUMENT;
    CacheHeader h;
    memcpy(&h, data, sizeof(h));
    const CacheHeader mine = cache_header(ctx);
    if (memcmp(h.magic, mine.magic, 8) != 0 || h.version != mine.version || h.header_size != mine.header_size ||
        h.entries != 0 || size != sizeof(CacheHeader))
        return AC_ERR_INVALID_ARGUMENT;  // malformed
    if (strncmp(h.arch, mine.arch, sizeof(h.arch)) != 0) return AC_ERR_INVALID_ARGUMENT;  // another device
    return AC_SUCCESS;
}

AcResult ac_runtime_pipeline_cache_get_data(AcContext* ctx, void* data, size_t* inout_size) {
    if (!ctx_ok(ctx)) return AC_ERR_INVALID_CONTEXT;
    if (!inout_size) return AC_ERR_NULL_POINTER;
    if (!data) {
        *inout_size = sizeof(CacheHeader);
        return AC_SUCCESS;
    }
    if (*inout_size < sizeof(CacheHeader)) return AC_ERR_INVALID_BUFFER_SIZE;
    const CacheHeader h = cache_header(ctx);
    memcpy(data, &h, sizeof(h));
    *inout_size = sizeof(h);
    return AC_SUCCESS;
}

// ---------------------------------------------------------------------------------------------------------------
// Generation-based error state (the reference's src/runtime/ac_error.cpp): first error wins within a generation,
// one state per context id, generation 1 at first use
// ---------------------------------------------------------------------------------------------------------------
void ac_runtime_set_error_ctx(uint64_t context_id, int32_t error_code, AmevaBackendOpKind op, size_t offset,
                              size_t requested_bytes, size_t capacity_bytes) {
    if (error_code == 0) return;
    std::lock_guard<std::mutex> lk(errors().mu);
    AmevaBackendErrorState& s = errors().get(context_id);
    if (s.first_error == 0) {
        s.first_error = error_code;
        s.operation = op;
        s.offset = offset;
        s.requested_bytes = requested_bytes;
        s.capacity_bytes = capacity_bytes;
    }
}

AmevaBackendErrorState ac_runtime_get_error_state_ctx(uint64_t context_id) {
    std::lock_guard<std::mutex> lk(errors().mu);
    return errors().get(context_id);
}

int32_t ac_runtime_consume_error_ctx(uint64_t context_id) {
    std::lock_guard<std::mutex> lk(errors().mu);
    AmevaBackendErrorState& s = errors().get(context_id);
    const int32_t e = s.first_error;
    clear_error(s);
    return e;
}

uint64_t ac_runtime_advance_generation_ctx(uint64_t context_id) {
    std::lock_guard<std::mutex> lk(errors().mu);
    AmevaBackendErrorState& s = errors().get(context_id);
    s.generation++;
    clear_error(s);
    return s.generation;
}

uint64_t ac_runtime_get_generation_ctx(uint64_t context_id) {
    std::lock_guard<std::mutex> lk(errors().mu);
    return errors().get(context_id).generation;
}

void ac_runtime_reset_error_state_ctx(uint64_t context_id) {
    std::lock_guard<std::mutex> lk(errors().mu);
    clear_error(errors().get(context_id));
}

void ac_runtime_set_error(int32_t error_code, AmevaBackendOpKind op, size_t offset, size_t requested_bytes,
                          size_t capacity_bytes) {
    ac_runtime_set_error_ctx(AC_GLOBAL_CONTEXT_ID, error_code, op, offset, requested_bytes, capacity_bytes);
}
AmevaBackendErrorState ac_runtime_get_error_state(void) { return ac_runtime_get_error_state_ctx(AC_GLOBAL_CONTEXT_ID); }
int32_t ac_runtime_consume_error(void) { return ac_runtime_consume_error_ctx(AC_GLOBAL_CONTEXT_ID); }
uint64_t ac_runtime_advance_generation(void) { return ac_runtime_advance_generation_ctx(AC_GLOBAL_CONTEXT_ID); }
uint64_t ac_runtime_get_generation(void) { return ac_runtime_get_generation_ctx(AC_GLOBAL_CONTEXT_ID); }
void ac_runtime_reset_error_state(void) { ac_runtime_reset_error_state_ctx(AC_GLOBAL_CONTEXT_ID); }

}  // extern "C"
