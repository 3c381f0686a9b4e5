// ggml backend plugin "AMEVA" on MI355X: registry, device AMEVA0, buffer type and buffers (with the MI355X weight
// layout), and the graph engine that runs a ggml graph on one in-order HIP stream through the kernel ABI of
// include/ameva_hip.h.
//
// Behaviour follows the reference plugin (adapters/llama/ggml-ameva/):
//   * one process-wide device; graph_compute is serialised by a mutex and returns after completion (synchronize NULL);
//   * contract first: every node of the graph goes through op_unsupported_reason before anything runs, and one
//     unsupported node fails the whole graph with a "(FAIL-FAST)" line (ggml-ameva.cpp:5330-5343); supports_op uses
//     the same function, so the scheduler never hands the backend a node it would reject; no CPU fallback;
//   * quantized weights live in the MI355X layout (amv_repack), converted when a MUL_MAT first reads them (the lazy
//     repack of ggml-ameva.cpp:5352-5373) and converted back by get_tensor, so other backends see ggml bytes;
//   * MUL_MAT routes like enc_mul_mat (3607): int8-MFMA GEMM from 8 columns for Q4_0 / Q8_0, GEMV otherwise; the
//     quantized activations of one src1 are reused by every MUL_MAT that reads it (the a8_src cache, 2738-2749);
//   * RMS_NORM followed by a MUL by the norm weight runs as one kernel (ameva_find_fusion, 4345), and a one-row
//     MUL_MAT followed by ADD or GLU SWIGLU (split) by the GEMV's epilogue (the reference's MUL_MAT fusion pairs);
//     llama.cpp's q/k/v (+ ROPE, SET_ROWS) and gate/up (+ SWIGLU) node groups run as one launch each, and at K = 4096
//     the RMS_NORM + MUL before a Q4_0 group or a Q4_K q/k/v group is computed inside it (no launch of its own);
//   * counters and failure injection as ggml-ameva.h:30-98.
// On MI355X the Vulkan hazard tracking of the reference (ameva_record, 2174) is the in-order stream itself: each
// kernel starts after the previous one has finished, so no barrier bookkeeping is needed.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/ameva_hip.h"
#include "../../include/ggml-ameva.h"
#include "ggml_abi.h"

namespace {

// ------------------------------------------------------------------------------------------------ counters
struct Counters {
    std::atomic<int64_t> supports_query{0}, supported_op{0}, gpu_op{0}, mul_mat{0}, qmv{0}, mmq{0};
    std::atomic<int64_t> ctx_create{0}, ctx_destroy{0}, buf_create{0}, buf_destroy{0};
    std::atomic<int64_t> repacked_tensors{0}, repacked_bytes{0}, fused{0}, act_reuse{0};
};
Counters g_cnt;
std::atomic<int> g_fail{AMEVA_FAIL_NONE};
// bumped whenever device memory a captured graph may read changes meaning outside a graph: a weight changing layout
// (repacked at first use, or returned to ggml bytes by a write), a buffer allocated, freed or cleared
std::atomic<int64_t> g_layout_gen{0};

// AMEVA_PROFILE (ggml-ameva.cpp:104-114 of the reference): 1 = totals per graph (host encode, wait, launches),
// 2 = also the GPU time of each node kind, from a HIP event recorded after every node on the graph's stream.
// AMEVA_TRACE=1: one stderr line per graph before its launches and one after completion.
int env_level(const char* name) {
    const char* e = std::getenv(name);
    return e && (e[0] == '1' || e[0] == '2') && e[1] == 0 ? e[0] - '0' : 0;
}
int profile_level() {
    static const int level = env_level("AMEVA_PROFILE");
    return level;
}
// AMEVA_MMQ_FORM=scaled: batched MUL_MATs above 64 tokens on operands rounded to f16 once (~3e-4 relative L2 from
// the exact form); anything else (the default): exact integer block sums
bool mmq_scaled() {
    static const bool on = [] {
        const char* e = std::getenv("AMEVA_MMQ_FORM");
        return e && std::strcmp(e, "scaled") == 0;
    }();
    return on;
}
bool trace_on() {
    static const bool on = env_level("AMEVA_TRACE") == 1;
    return on;
}
struct Profile {
    std::mutex mu;
    int64_t graphs = 0, nodes = 0, launches = 0, gpu_samples = 0;
    double encode_ms = 0, wait_ms = 0, gpu_ms = 0;
    struct Kind {
        double ms = 0;
        int64_t n = 0;
    };
    std::vector<std::pair<std::string, Kind>> kinds;  // in order of first appearance
    void add_kind(const std::string& k, double ms) {
        for (auto& e : kinds)
            if (e.first == k) {
                e.second.ms += ms;
                e.second.n++;
                return;
            }
        kinds.push_back({k, Kind{ms, 1}});
    }
};
Profile g_prof;
double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}
const char* op_name(int op) {
    switch (op) {
    case GGML_OP_ADD: return "ADD";
    case GGML_OP_MUL: return "MUL";
    case GGML_OP_RMS_NORM: return "RMS_NORM";
    case GGML_OP_MUL_MAT: return "MUL_MAT";
    case GGML_OP_CPY: return "CPY";
    case GGML_OP_CONT: return "CONT";
    case GGML_OP_GET_ROWS: return "GET_ROWS";
    case GGML_OP_SET_ROWS: return "SET_ROWS";
    case GGML_OP_ROPE: return "ROPE";
    case GGML_OP_FLASH_ATTN_EXT: return "FLASH_ATTN_EXT";
    case GGML_OP_GLU: return "GLU";
    default: return "OTHER";
    }
}
const char* type_name(int t) {
    switch (t) {
    case GGML_TYPE_F32: return "f32";
    case GGML_TYPE_F16: return "f16";
    case GGML_TYPE_Q4_0: return "q4_0";
    case GGML_TYPE_Q8_0: return "q8_0";
    case GGML_TYPE_Q4_K: return "q4_K";
    case GGML_TYPE_Q6_K: return "q6_K";
    default: return "other";
    }
}

void log_line(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::fprintf(stderr, "ggml-ameva: ");
    std::vfprintf(stderr, fmt, ap);
    std::fprintf(stderr, "\n");
    va_end(ap);
}

// ------------------------------------------------------------------------------------------------ ggml sizes
int64_t blck_size(int t) {
    switch (t) {
    case GGML_TYPE_Q4_0:
    case GGML_TYPE_Q8_0: return 32;
    case GGML_TYPE_Q4_K:
    case GGML_TYPE_Q6_K:
    case GGML_TYPE_Q8_K: return 256;
    default: return 1;
    }
}
int64_t type_size(int t) {
    switch (t) {
    case GGML_TYPE_F32: return 4;
    case GGML_TYPE_F16: return 2;
    case GGML_TYPE_BF16: return 2;
    case GGML_TYPE_Q4_0: return 18;
    case GGML_TYPE_Q8_0: return 34;
    case GGML_TYPE_Q4_K: return 144;
    case GGML_TYPE_Q6_K: return 210;
    case GGML_TYPE_Q8_K: return 292;
    case GGML_TYPE_I8: return 1;
    case GGML_TYPE_I16: return 2;
    case GGML_TYPE_I32: return 4;
    case GGML_TYPE_I64: return 8;
    default: return 0;
    }
}
// ggml_nbytes
size_t nbytes(const ggml_tensor* t) {
    const int64_t bs = blck_size(t->type);
    size_t n;
    if (bs == 1) {
        n = (size_t)type_size(t->type);
        for (int i = 0; i < GGML_MAX_DIMS; ++i) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    } else {
        n = (size_t)(t->ne[0] * (int64_t)t->nb[0] / bs);
        for (int i = 1; i < GGML_MAX_DIMS; ++i) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return n;
}
int64_t nelements(const ggml_tensor* t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t nrows(const ggml_tensor* t) { return t->ne[1] * t->ne[2] * t->ne[3]; }
bool is_contiguous(const ggml_tensor* t) {
    const int64_t ts = type_size(t->type), bs = blck_size(t->type);
    if (ts == 0) return false;
    size_t next = (size_t)ts;
    if ((int64_t)t->nb[0] != ts) return false;
    next = (size_t)(ts * (t->ne[0] / bs));
    for (int i = 1; i < GGML_MAX_DIMS; ++i) {
        if (t->ne[i] != 1 && t->nb[i] != next) return false;
        next *= (size_t)t->ne[i];
    }
    return true;
}
float op_f32(const ggml_tensor* t, int i) {
    float f;
    std::memcpy(&f, &t->op_params[i], 4);
    return f;
}
bool quant_weight_type(int t) {
    return t == GGML_TYPE_Q4_0 || t == GGML_TYPE_Q8_0 || t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q6_K;
}
bool noop(int op) {
    return op == GGML_OP_NONE || op == GGML_OP_RESHAPE || op == GGML_OP_VIEW || op == GGML_OP_PERMUTE ||
           op == GGML_OP_TRANSPOSE;
}
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ------------------------------------------------------------------------------------------------ device state
struct Device;
Device* device();

// per buffer: device memory and the layout state of the quantized weights it holds
struct BufCtx {
    void* dev = nullptr;
    size_t size = 0;
    std::mutex mu;
    std::unordered_map<const void*, int> repacked;  // tensor data -> ggml type, for tensors in the MI355X layout
};

const char* buft_get_name(ggml_backend_buffer_type_t) { return GGML_AMEVA_DEVICE_NAME; }
ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size);
size_t buft_get_alignment(ggml_backend_buffer_type_t) { return 256; }
size_t buft_get_max_size(ggml_backend_buffer_type_t) { return (size_t)64 << 30; }
size_t buft_get_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor* t) { return nbytes(t); }
bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

struct ggml_backend_buffer_type g_buft = {
    {buft_get_name, buft_alloc_buffer, buft_get_alignment, buft_get_max_size, buft_get_alloc_size, buft_is_host},
    nullptr,
    nullptr};

bool is_ours(const ggml_tensor* t) { return t && t->buffer && t->buffer->buft == &g_buft; }

// device-side scratch of a graph (activation quantization, attention partials, status word); grows, never shrinks
struct Arena {
    uint8_t* base = nullptr;
    size_t cap = 0, used = 0;
    bool reserve(size_t need) {
        if (need <= cap) return true;
        if (base) (void)hipFree(base);
        base = nullptr;
        cap = 0;
        size_t c = need + need / 2 + (1 << 20);
        if (hipMalloc(&base, c) != hipSuccess) return false;
        cap = c;
        return true;
    }
    void* take(size_t n) {
        const size_t off = (used + 255) & ~(size_t)255;
        if (off + n > cap) return nullptr;
        used = off + n;
        return base + off;
    }
};

// The last graph computed, as a signature of everything its launches bake in (per node and source: op, type, shape,
// strides, data address, view offset, op parameters), and its capture as a HIP graph with the counter increments
// one run of it makes.
struct Replay {
    std::vector<int64_t> sig;
    int64_t gen = -1;                  // g_layout_gen when sig was computed
    hipGraphExec_t exec = nullptr;     // captured on the second computation of an identical graph
    const void* arena_base = nullptr;  // the scratch the capture addresses
    bool uncapturable = false;         // capture of this signature failed once: eager from now on
    int64_t d_gpu_op = 0, d_mul_mat = 0, d_qmv = 0, d_mmq = 0, d_fused = 0, d_act_reuse = 0, encoded = 0;
    void drop() {
        if (exec) (void)hipGraphExecDestroy(exec);
        exec = nullptr;
        uncapturable = false;
    }
};

// arrival counters for gate/up GEMVs of up to 2 x 65536 rows (AMV_SWIGLU_COUNTER_WORDS)
#define AMEVA_COUNTER_WORDS AMV_SWIGLU_COUNTER_WORDS(2 * 65536)

struct Device {
    std::mutex compute_mu;
    hipStream_t stream = nullptr;
    Arena arena;
    Replay replay;
    unsigned int* status = nullptr;       // bad-index counter of SET_ROWS / GET_ROWS
    unsigned int* counters = nullptr;     // arrival counters of the fused gate/up GEMV's tail (zero between calls)
    unsigned int* status_host = nullptr;  // pinned copy of it, written by the graph's last kernel
    unsigned int* status_host_dev = nullptr;  // the same pinned word as the device addresses it
    bool status_clean = false;            // status holds zeros (the last run ended with k_status_out)
    std::vector<hipEvent_t> events;  // AMEVA_PROFILE=2: one after every node of a graph (grows, reused)
    hipEvent_t done = nullptr;       // recorded after a graph's last kernel: the bounded completion wait polls it
    bool inited = false;
    hipEvent_t event(size_t i) {
        while (events.size() <= i) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) return nullptr;
            events.push_back(e);
        }
        return events[i];
    }
    bool init() {
        if (inited) return true;
        if (hipSetDevice(0) != hipSuccess) return false;
        if (hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess) return false;
        if (hipMalloc(&status, 256) != hipSuccess) return false;
        if (hipHostMalloc((void**)&status_host, 256, hipHostMallocDefault) != hipSuccess) return false;
        if (hipHostGetDevicePointer((void**)&status_host_dev, status_host, 0) != hipSuccess) return false;
        if (hipMemset(status, 0, 256) != hipSuccess) return false;
        status_clean = true;
        if (hipMalloc(&counters, AMEVA_COUNTER_WORDS * 4) != hipSuccess ||
            hipMemset(counters, 0, AMEVA_COUNTER_WORDS * 4) != hipSuccess)
            return false;
        if (hipEventCreateWithFlags(&done, hipEventDisableTiming) != hipSuccess) return false;
        inited = true;
        g_cnt.ctx_create++;
        return true;
    }
};

Device* device() {
    static Device d;
    return &d;
}

// ------------------------------------------------------------------------------------------------ buffers
void buf_free(ggml_backend_buffer_t b) {
    g_layout_gen++;
    BufCtx* c = (BufCtx*)b->context;
    if (c) {
        std::lock_guard<std::mutex> lk(c->mu);
        for (auto& kv : c->repacked) {
            (void)kv;
            g_cnt.repacked_tensors--;
        }
        (void)hipFree(c->dev);
        delete c;
    }
    g_cnt.buf_destroy++;
}
void* buf_get_base(ggml_backend_buffer_t b) { return ((BufCtx*)b->context)->dev; }
void buf_memset(ggml_backend_buffer_t b, ggml_tensor* t, uint8_t v, size_t off, size_t size);

// converts a quantized tensor between ggml blocks and the MI355X layout in place (through a temporary copy)
bool convert_in_place(ggml_tensor* t, bool to_repacked) {
    g_layout_gen++;
    const size_t n = nbytes(t);
    void* tmp = nullptr;
    if (hipMalloc(&tmp, n) != hipSuccess) return false;
    bool ok = hipMemcpy(tmp, t->data, n, hipMemcpyDeviceToDevice) == hipSuccess;
    if (ok) {
        const int rc = to_repacked ? amv_repack(t->type, tmp, t->data, t->ne[1], t->ne[0], nullptr)
                                   : amv_unrepack(t->type, tmp, t->data, t->ne[1], t->ne[0], nullptr);
        ok = rc == AMV_OK && hipDeviceSynchronize() == hipSuccess;
        if (rc != AMV_OK) log_line("repack of %s failed: %s", t->name, amv_last_error());
    }
    (void)hipFree(tmp);
    return ok;
}

bool repackable(const ggml_tensor* t) {
    return quant_weight_type(t->type) && t->ne[2] == 1 && t->ne[3] == 1 && is_contiguous(t) && t->view_src == nullptr &&
           t->ne[0] % blck_size(t->type) == 0 && aligned16(t->data);
}

// returns the tensor to ggml layout if it is held repacked (before a partial write or a raw read)
bool ensure_raw(BufCtx* c, ggml_tensor* t) {
    auto it = c->repacked.find(t->data);
    if (it == c->repacked.end()) return true;
    if (!convert_in_place(t, false)) return false;
    c->repacked.erase(it);
    g_cnt.repacked_tensors--;
    g_cnt.repacked_bytes -= (int64_t)nbytes(t);
    return true;
}

// A write of a tensor held repacked first returns it to the ggml layout (the write is in ggml bytes). When that
// fails, a partial write stops there (its bytes would land in a layout the kernels read differently); a write of
// the whole tensor replaces every byte, so the tensor is marked as held in ggml layout and written.
void forget_repacked(BufCtx* c, const ggml_tensor* t) {
    auto it = c->repacked.find(t->data);
    if (it == c->repacked.end()) return;
    c->repacked.erase(it);
    g_cnt.repacked_tensors--;
    g_cnt.repacked_bytes -= (int64_t)nbytes(t);
    g_layout_gen++;
}

void buf_memset(ggml_backend_buffer_t b, ggml_tensor* t, uint8_t v, size_t off, size_t size) {
    BufCtx* c = (BufCtx*)b->context;
    std::lock_guard<std::mutex> lk(c->mu);
    if (!ensure_raw(c, t)) {
        if (off != 0 || size != nbytes(t)) {
            log_line("memset_tensor %s: could not restore the ggml layout; nothing written (FAIL-FAST)", t->name);
            return;
        }
        forget_repacked(c, t);
    }
    if (hipMemset((uint8_t*)t->data + off, v, size) != hipSuccess) log_line("memset_tensor %s: failed", t->name);
}

void buf_set_tensor(ggml_backend_buffer_t b, ggml_tensor* t, const void* data, size_t off, size_t size) {
    BufCtx* c = (BufCtx*)b->context;
    std::lock_guard<std::mutex> lk(c->mu);
    if (!ensure_raw(c, t)) {
        if (off != 0 || size != nbytes(t)) {
            log_line("set_tensor %s: could not restore the ggml layout; nothing written (FAIL-FAST)", t->name);
            return;
        }
        forget_repacked(c, t);
    }
    if (hipMemcpy((uint8_t*)t->data + off, data, size, hipMemcpyHostToDevice) != hipSuccess)
        log_line("set_tensor %s: copy failed", t->name);
}

void buf_get_tensor(ggml_backend_buffer_t b, const ggml_tensor* t, void* data, size_t off, size_t size) {
    BufCtx* c = (BufCtx*)b->context;
    std::lock_guard<std::mutex> lk(c->mu);
    auto it = c->repacked.find(t->data);
    if (it == c->repacked.end()) {
        (void)hipMemcpy(data, (const uint8_t*)t->data + off, size, hipMemcpyDeviceToHost);
        return;
    }
    // a repacked weight is read in ggml layout: convert a copy
    const size_t n = nbytes(t);
    void* tmp = nullptr;
    if (hipMalloc(&tmp, n) != hipSuccess) {
        log_line("get_tensor %s: no memory for the layout conversion", t->name);
        return;
    }
    if (amv_unrepack(t->type, t->data, tmp, t->ne[1], t->ne[0], nullptr) == AMV_OK)
        (void)hipMemcpy(data, (const uint8_t*)tmp + off, size, hipMemcpyDeviceToHost);
    (void)hipFree(tmp);
}

bool buf_cpy_tensor(ggml_backend_buffer_t b, const ggml_tensor* src, ggml_tensor* dst) {
    if (!is_ours(src)) return false;
    BufCtx* c = (BufCtx*)b->context;
    std::lock_guard<std::mutex> lk(c->mu);
    if (!ensure_raw(c, dst)) return false;
    BufCtx* cs = (BufCtx*)src->buffer->context;
    if (cs != c) {
        std::lock_guard<std::mutex> lk2(cs->mu);
        if (!ensure_raw(cs, const_cast<ggml_tensor*>(src))) return false;
    } else if (!ensure_raw(c, const_cast<ggml_tensor*>(src))) {
        return false;
    }
    return hipMemcpy(dst->data, src->data, nbytes(src), hipMemcpyDeviceToDevice) == hipSuccess;
}

void buf_clear(ggml_backend_buffer_t b, uint8_t v) {
    g_layout_gen++;
    BufCtx* c = (BufCtx*)b->context;
    std::lock_guard<std::mutex> lk(c->mu);
    g_cnt.repacked_tensors -= (int64_t)c->repacked.size();
    c->repacked.clear();
    (void)hipMemset(c->dev, v, c->size);
}

const ggml_backend_buffer_i g_buf_iface = {
    buf_free, buf_get_base, nullptr, buf_memset, buf_set_tensor, buf_get_tensor, nullptr, nullptr, buf_cpy_tensor,
    buf_clear, nullptr};

ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    if (!device()->init()) {
        log_line("no HIP device (FAIL-FAST)");
        return nullptr;
    }
    g_layout_gen++;
    BufCtx* c = new BufCtx;
    c->size = size;
    if (hipMalloc(&c->dev, size ? size : 256) != hipSuccess) {
        log_line("alloc_buffer: hipMalloc of %zu bytes failed", size);
        delete c;
        return nullptr;
    }
    g_cnt.buf_create++;
    return ggml_backend_buffer_init(buft, g_buf_iface, c, size);
}

// ------------------------------------------------------------------------------------------------ the contract
const char* unsupported_reason(const ggml_tensor* n) {
    if (g_fail.load() == AMEVA_FAIL_TENSOR_RANGE_OOB) return "failure injection: tensor range out of bounds";
    if (noop(n->op)) return nullptr;
    if (!is_ours(n)) return "destination is not in an AMEVA buffer";
    for (int i = 0; i < GGML_MAX_SRC && n->src[i]; ++i)
        if (!is_ours(n->src[i])) return "a source is not in an AMEVA buffer";
    const ggml_tensor* s0 = n->src[0];
    const ggml_tensor* s1 = n->src[1];
    switch (n->op) {
    case GGML_OP_MUL_MAT: {
        if (!quant_weight_type(s0->type)) return "MUL_MAT src0 type is not Q4_0, Q8_0, Q4_K or Q6_K";
        if (s0->ne[2] != 1 || s0->ne[3] != 1) return "MUL_MAT src0 must be a 2-D weight";
        if (!is_contiguous(s0)) return "MUL_MAT src0 rows must be contiguous";
        if (s0->view_src) {  // a view of whole rows of a 2-D weight (ggml_view_2d at a row offset)
            const ggml_tensor* p = s0->view_src;
            if (p->type != s0->type || p->ne[0] != s0->ne[0] || p->ne[2] != 1 || p->ne[3] != 1 || p->view_src ||
                !is_contiguous(p) || s0->nb[1] != p->nb[1] || s0->view_offs % p->nb[1] != 0 ||
                s0->view_offs + nbytes(s0) > nbytes(p) || !aligned16(p->data))
                return "MUL_MAT src0 view must be whole rows of a 2-D quantized weight";
        } else if (!aligned16(s0->data)) {
            return "MUL_MAT src0 must be 16-byte aligned";
        }
        if (s1->type != GGML_TYPE_F32 || !is_contiguous(s1)) return "MUL_MAT src1 must be contiguous F32";
        if (s1->ne[0] != s0->ne[0]) return "MUL_MAT inner dimensions differ";
        if (n->type != GGML_TYPE_F32 || !is_contiguous(n)) return "MUL_MAT dst must be contiguous F32";
        if (s0->ne[0] % blck_size(s0->type) != 0) return "MUL_MAT row is not whole blocks";
        return nullptr;
    }
    case GGML_OP_RMS_NORM:
        if (s0->type != GGML_TYPE_F32 || n->type != GGML_TYPE_F32) return "RMS_NORM is F32 only";
        if (!is_contiguous(s0) || !is_contiguous(n)) return "RMS_NORM needs contiguous rows";
        if (s0->ne[0] % 4 != 0 || !aligned16(s0->data) || !aligned16(n->data)) return "RMS_NORM rows must be 16-byte units";
        return nullptr;
    case GGML_OP_ADD:
    case GGML_OP_MUL: {
        if (s0->type != GGML_TYPE_F32 || s1->type != GGML_TYPE_F32 || n->type != GGML_TYPE_F32) return "binary op is F32 only";
        if (!is_contiguous(s0) || !is_contiguous(s1) || !is_contiguous(n)) return "binary op needs contiguous tensors";
        if (s1->ne[0] != s0->ne[0]) return "binary op broadcast along dim 0 is not supported";
        const bool same = s1->ne[1] == s0->ne[1] && s1->ne[2] == s0->ne[2] && s1->ne[3] == s0->ne[3];
        const bool one_row = nrows(s1) == 1;
        const bool rows_only = s1->ne[1] == s0->ne[1] && s1->ne[2] == 1 && s1->ne[3] == 1;
        if (!same && !one_row && !rows_only) return "binary op broadcast pattern not supported";
        return nullptr;
    }
    case GGML_OP_ROPE: {
        const int mode = n->op_params[2];
        if (s0->type != GGML_TYPE_F32 || n->type != GGML_TYPE_F32) return "ROPE is F32 only";
        if (!is_contiguous(s0) || !is_contiguous(n)) return "ROPE needs contiguous tensors";
        if (mode != 0 && mode != 2) return "ROPE mode must be NORMAL or NEOX";
        if (n->src[2]) return "ROPE frequency factors not supported";
        if (op_f32(n, 7) != 0.0f) return "ROPE YaRN ext_factor != 0 not supported";
        if (s1->type != GGML_TYPE_I32 || s1->ne[0] != s0->ne[2]) return "ROPE positions must be I32 per token";
        if (s0->ne[3] != 1) return "ROPE ne[3] must be 1";
        if (n->op_params[1] <= 0 || n->op_params[1] > s0->ne[0] || n->op_params[1] % 2) return "ROPE n_dims invalid";
        return nullptr;
    }
    case GGML_OP_FLASH_ATTN_EXT: {
        const ggml_tensor *q = s0, *k = s1, *v = n->src[2], *m = n->src[3];
        if (n->src[4]) return "FLASH_ATTN_EXT sinks not supported";
        const bool kvq = k->type == GGML_TYPE_Q8_0 || k->type == GGML_TYPE_Q4_0;  // a quantized cache
        if (q->type != GGML_TYPE_F32 || (k->type != GGML_TYPE_F16 && !kvq) || v->type != k->type)
            return "FLASH_ATTN_EXT needs F32 q and an F16, Q8_0 or Q4_0 K/V cache (K and V of one type)";
        if (q->ne[0] != 128 || v->ne[0] != 128 || k->ne[0] != 128) return "FLASH_ATTN_EXT head size must be 128";
        if (q->ne[1] != 1 || q->ne[3] != 1 || k->ne[3] != 1) return "FLASH_ATTN_EXT decode (one query) only";
        if (q->nb[0] != 4 || q->nb[2] != 128 * 4 || !aligned16(q->data)) return "FLASH_ATTN_EXT q heads must be contiguous";
        if (!kvq && (k->nb[0] != 2 || v->nb[0] != 2 || k->nb[1] % 16 || k->nb[2] % 16 || v->nb[1] % 16 ||
                     v->nb[2] % 16 || !aligned16(k->data) || !aligned16(v->data)))
            return "FLASH_ATTN_EXT f16 K/V rows must be 16-byte aligned";
        if (kvq && (k->nb[0] != (size_t)type_size(k->type) || v->nb[0] != (size_t)type_size(v->type) || k->nb[1] % 2 ||
                    k->nb[2] % 2 || v->nb[1] % 2 || v->nb[2] % 2 || ((uintptr_t)k->data & 1) || ((uintptr_t)v->data & 1)))
            return "FLASH_ATTN_EXT quantized K/V rows must be dense blocks at even addresses";
        if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2]) return "FLASH_ATTN_EXT K/V shapes differ";
        const int64_t G = q->ne[2] / k->ne[2];
        if (q->ne[2] % k->ne[2] || (G != 1 && G != 2 && G != 4 && G != 8)) return "FLASH_ATTN_EXT GQA group not 1/2/4/8";
        if (op_f32(n, 1) != 0.0f || op_f32(n, 2) != 0.0f) return "FLASH_ATTN_EXT ALiBi / softcap not supported";
        if (m && (m->type != GGML_TYPE_F16 || m->ne[0] < k->ne[1] || m->nb[0] != 2 || m->ne[2] != 1))
            return "FLASH_ATTN_EXT mask must be F16 [n_kv, ...] shared by all heads";
        if (n->type != GGML_TYPE_F32 || !is_contiguous(n)) return "FLASH_ATTN_EXT dst must be contiguous F32";
        return nullptr;
    }
    case GGML_OP_GLU: {
        if (n->op_params[0] != GGML_GLU_OP_SWIGLU) return "GLU op other than SWIGLU";
        if (!s1) {
            if (nrows(s0) != 1) return "GLU single-tensor form only for one row";
        } else if (s1->type != GGML_TYPE_F32 || !is_contiguous(s1) || nelements(s1) != nelements(s0)) {
            return "GLU src1 must match src0";
        }
        if (s0->type != GGML_TYPE_F32 || !is_contiguous(s0) || n->type != GGML_TYPE_F32 || !is_contiguous(n))
            return "GLU is contiguous F32 only";
        return nullptr;
    }
    case GGML_OP_SET_ROWS: {
        const bool q = n->type == GGML_TYPE_Q8_0 || n->type == GGML_TYPE_Q4_0;  // a quantized KV cache
        if (s0->type != GGML_TYPE_F32 || (n->type != GGML_TYPE_F16 && !q)) return "SET_ROWS F32 -> F16, Q8_0 or Q4_0 only";
        if (s1->type != GGML_TYPE_I64 && s1->type != GGML_TYPE_I32) return "SET_ROWS index must be I32 or I64";
        if (s0->ne[2] != 1 || s0->ne[3] != 1 || n->ne[2] != 1 || n->ne[3] != 1) return "SET_ROWS 2-D only";
        if (s0->nb[0] != 4 || n->nb[0] != (size_t)type_size(n->type) || s1->nb[0] != (size_t)type_size(s1->type))
            return "SET_ROWS rows must be dense";
        if (q && (n->ne[0] % 32 || n->nb[1] % 2 || ((uintptr_t)n->data & 1)))
            return "SET_ROWS quantized rows must be whole blocks at even addresses";
        if (s0->ne[0] != n->ne[0] || s1->ne[0] != s0->ne[1]) return "SET_ROWS shapes differ";
        return nullptr;
    }
    case GGML_OP_CPY:
    case GGML_OP_CONT:
        if (s0->type != GGML_TYPE_F32 || (n->type != GGML_TYPE_F32 && n->type != GGML_TYPE_F16)) return "CPY F32 -> F32/F16 only";
        if (!is_contiguous(s0) || !is_contiguous(n) || nelements(s0) != nelements(n)) return "CPY needs contiguous tensors";
        return nullptr;
    case GGML_OP_GET_ROWS:
        if (s0->type != GGML_TYPE_F32 && s0->type != GGML_TYPE_F16 && s0->type != GGML_TYPE_Q4_0 &&
            s0->type != GGML_TYPE_Q8_0)
            return "GET_ROWS source type not supported";
        if (s1->type != GGML_TYPE_I32 || s0->ne[2] != 1 || s0->ne[3] != 1 || !is_contiguous(s0) || !is_contiguous(s1))
            return "GET_ROWS needs a 2-D source and I32 indices";
        if (n->type != GGML_TYPE_F32 || !is_contiguous(n)) return "GET_ROWS dst must be F32";
        return nullptr;
    default: return "op not implemented on AMEVA";
    }
}

// ------------------------------------------------------------------------------------------------ graph engine
struct ActEntry {
    const void* data;
    size_t bytes;
    int atype;
    int64_t m, k;  // the rows and row length it was quantized as (a reshaped view of the same bytes differs)
    void* act;
};

struct Engine {
    Device* dev = nullptr;
    hipStream_t st = nullptr;
    std::vector<ActEntry> acts;  // quantized activations valid at this point of the graph
    ActEntry pending_act{};      // one written by the node being encoded (registered after its own invalidation)
    bool failed = false;
    std::string why;
    std::vector<std::string> labels;  // AMEVA_PROFILE=2: the kind of each timed node (events 0 .. n)
    int64_t encoded = 0;              // nodes encoded (a fused pair counts once)

    bool fail(const ggml_tensor* n, const char* what) {
        failed = true;
        char buf[512];
        std::snprintf(buf, sizeof(buf), "node %s (op %d): %s", n ? n->name : "?", n ? (int)n->op : -1, what);
        why = buf;
        return false;
    }
    bool rc(const ggml_tensor* n, int r) { return r == AMV_OK ? true : fail(n, amv_last_error()); }

    // a node's output overwrites memory that cached activations were quantized from
    void invalidate(const ggml_tensor* n) {
        const uint8_t* lo = (const uint8_t*)n->data;
        const uint8_t* hi = lo + nbytes(n);
        for (size_t i = 0; i < acts.size();) {
            const uint8_t* a = (const uint8_t*)acts[i].data;
            if (a < hi && lo < a + acts[i].bytes) acts.erase(acts.begin() + i);
            else ++i;
        }
    }

    void* act_for(const ggml_tensor* n, const ggml_tensor* x, int atype, int64_t m, int64_t k) {
        for (auto& e : acts)
            if (e.data == x->data && e.atype == atype && e.bytes == nbytes(x) && e.m == m && e.k == k) {
                g_cnt.act_reuse++;
                return e.act;
            }
        void* act = dev->arena.take((size_t)amv_act_bytes(atype, m, k));
        if (!act) {
            fail(n, "scratch exhausted");
            return nullptr;
        }
        if (amv_quantize_act(atype, (const float*)x->data, m, k, AMV_Q8_X86, nullptr, act, st) != AMV_OK) {
            fail(n, amv_last_error());
            return nullptr;
        }
        acts.push_back({x->data, nbytes(x), atype, m, k, act});
        return act;
    }

    // ep: the fused next node (ADD, or GLU SWIGLU split) of a one-row MUL_MAT, computed in the GEMV's epilogue
    bool mul_mat(const ggml_tensor* n, const ggml_tensor* ep = nullptr) {
        const ggml_tensor *w = n->src[0], *x = n->src[1];
        const int64_t K = w->ne[0], M = nrows(x);
        // batched (M >= 8) MUL_MATs run on the matrix cores for Q4_0 / Q8_0 / Q4_K / Q6_K (the reference's switch at
        // AMEVA_QGEMM_MIN_M). Above 64 tokens the exact form (exact per-block integer sums, ggml's f32 epilogue: the
        // reference's MMQ arithmetic) reads the plain Q8_0 / Q8_K layout; Q4_K batches of 8..64 tokens read the f16
        // copies of AMV_ACT_Q8_K_MMA; AMEVA_MMQ_FORM=scaled selects the scaled layouts (f16 q * d) above 64 tokens
        const bool mmq = M >= 8 && (w->type == GGML_TYPE_Q4_0 || w->type == GGML_TYPE_Q8_0 || w->type == GGML_TYPE_Q4_K ||
                                    w->type == GGML_TYPE_Q6_K);
        const bool kq = w->type == GGML_TYPE_Q4_K || w->type == GGML_TYPE_Q6_K;
        const bool deq = mmq && M > 64 && mmq_scaled() && w->type != GGML_TYPE_Q6_K;  // Q6_K: exact form only
        const int atype = deq ? (kq ? AMV_ACT_Q8_K_DEQ : AMV_ACT_Q8_0_DEQ)
                        : (mmq && w->type == GGML_TYPE_Q4_K && M <= 64) ? AMV_ACT_Q8_K_MMA
                        : kq ? (int)GGML_TYPE_Q8_K : (int)GGML_TYPE_Q8_0;
        if (!mmq && !ep && raw_readable(w)) return mul_mat_raw(n, atype);
        const void* wp = weight_ptr(n);
        if (!wp) return false;
        if (g_fail.load() == AMEVA_FAIL_MAP_SRC1) return fail(n, "failure injection: src1");
        void* act = act_for(n, x, atype, M, K);
        if (!act) return false;
        if (g_fail.load() == AMEVA_FAIL_DISPATCH) return fail(n, "failure injection: dispatch");
        return mul_mat_run(n, ep, wp, act, atype, M, mmq);
    }

    // A Q4_0 / Q8_0 weight that stays in ggml's block layout for this read: outside a WEIGHTS buffer (or a row view of
    // a tensor) and not held repacked. The GEMV reads its blocks in place (the reference's raw-layout MUL_MAT,
    // ameva_qmm.comp:315-372) instead of repacking a copy into scratch on every use; WEIGHTS tensors are still
    // repacked in place once, which later reads amortise.
    bool raw_readable(const ggml_tensor* w) {
        if (w->type != GGML_TYPE_Q4_0 && w->type != GGML_TYPE_Q8_0) return false;
        if (w->ne[0] % 64 != 0 || ((uintptr_t)w->data & 3) != 0 || w->nb[1] % 4 != 0) return false;
        BufCtx* bc = (BufCtx*)w->buffer->context;
        const ggml_tensor* base = w->view_src ? w->view_src : w;
        std::lock_guard<std::mutex> lk(bc->mu);
        if (bc->repacked.count(base->data)) return false;
        return w->view_src || w->buffer->usage != GGML_BACKEND_BUFFER_USAGE_WEIGHTS || !repackable(w);
    }

    bool mul_mat_raw(const ggml_tensor* n, int atype) {
        const ggml_tensor *w = n->src[0], *x = n->src[1];
        const int64_t N = w->ne[1], K = w->ne[0], M = nrows(x);
        if (g_fail.load() == AMEVA_FAIL_MAP_SRC1) return fail(n, "failure injection: src1");
        void* act = act_for(n, x, atype, M, K);
        if (!act) return false;
        if (g_fail.load() == AMEVA_FAIL_DISPATCH) return fail(n, "failure injection: dispatch");
        if (!rc(n, amv_mul_mat_vec_raw(w->type, w->data, (int64_t)w->nb[1], N, K, act, M, (float*)n->data, N, nullptr,
                                       st)))
            return false;
        g_cnt.mul_mat++;
        g_cnt.qmv++;
        return true;
    }

    // src0 of a MUL_MAT in the MI355X layout: weights are repacked in place once (WEIGHTS buffers); a quantized
    // tensor of any other buffer is repacked into scratch for this use. NULL (and the engine failed) on error.
    const void* weight_ptr(const ggml_tensor* n) {
        const ggml_tensor* w = n->src[0];
        const int64_t N = w->ne[1], K = w->ne[0];
        const void* wp = w->data;
        BufCtx* bc = (BufCtx*)w->buffer->context;
        if (w->view_src) {
            // rows of another weight: their ggml bytes (from a layout copy of the parent when the parent is held
            // repacked) are repacked into scratch for this use
            const ggml_tensor* p = w->view_src;
            std::lock_guard<std::mutex> lk(bc->mu);
            const uint8_t* src = (const uint8_t*)w->data;
            if (bc->repacked.count(p->data)) {
                uint8_t* raw = (uint8_t*)dev->arena.take(nbytes(p));
                if (!raw) return fail(n, "scratch exhausted"), nullptr;
                if (!rc(n, amv_unrepack(p->type, p->data, raw, p->ne[1], p->ne[0], st))) return nullptr;
                src = raw + w->view_offs;
            }
            void* tmp = dev->arena.take(nbytes(w));
            if (!tmp) return fail(n, "scratch exhausted"), nullptr;
            if (!rc(n, amv_repack(w->type, src, tmp, N, K, st))) return nullptr;
            wp = tmp;
        } else {
            std::lock_guard<std::mutex> lk(bc->mu);
            if (!bc->repacked.count(w->data)) {
                if (w->buffer->usage == GGML_BACKEND_BUFFER_USAGE_WEIGHTS && repackable(w)) {
                    if (!convert_in_place(const_cast<ggml_tensor*>(w), true)) return fail(n, "weight repack failed"), nullptr;
                    bc->repacked[w->data] = w->type;
                    g_cnt.repacked_tensors++;
                    g_cnt.repacked_bytes += (int64_t)nbytes(w);
                } else {
                    void* tmp = dev->arena.take(nbytes(w));
                    if (!tmp) return fail(n, "scratch exhausted"), nullptr;
                    if (!rc(n, amv_repack(w->type, w->data, tmp, N, K, st))) return nullptr;
                    wp = tmp;
                }
            }
        }
        return wp;
    }

    bool mul_mat_run(const ggml_tensor* n, const ggml_tensor* ep, const void* wp, void* act, int atype, int64_t M,
                     bool mmq) {
        const ggml_tensor *w = n->src[0];
        const int64_t N = w->ne[1], K = w->ne[0];
        int r;
        if (ep) {
            const ggml_tensor* e = ep->src[0] == n ? ep->src[1] : ep->src[0];
            int mode = AMV_EP_ADD;
            if (ep->op == GGML_OP_GLU) {
                const bool swapped = ep->op_params[1] != 0;  // swapped: silu(src1) * src0
                const bool n_is_gate = (ep->src[0] == n) != swapped;
                mode = n_is_gate ? AMV_EP_SILU_MUL : AMV_EP_MUL_SILU;
            }
            r = amv_mul_mat_vec_ep(w->type, wp, N, K, act, (float*)n->data, mode, (const float*)e->data,
                                   (float*)ep->data, st);
        } else {
            r = mmq ? amv_mul_mat_q_act(w->type, wp, N, K, act, atype, M, (float*)n->data, N, st)
                    : amv_mul_mat_vec(w->type, wp, N, K, act, M, (float*)n->data, N, st);
        }
        if (!rc(n, r)) return false;
        g_cnt.mul_mat++;
        g_cnt.qmv++;
        if (mmq) g_cnt.mmq++;
        return true;
    }

    bool binary(const ggml_tensor* n, int op) {
        const ggml_tensor *a = n->src[0], *b = n->src[1];
        return rc(n, amv_binary(op, (const float*)a->data, (const float*)b->data, (float*)n->data, nrows(a), a->ne[0],
                                nrows(b), st));
    }

    // The activation type (Q8_0 or Q8_K) the first later one-row GEMV MUL_MAT reading `out` (the same bytes: out
    // itself or a view of it) quantizes it to, or 0: the producer of `out` can then write that activation row in the
    // same pass (act_for finds it in the cache); rows = k = elements of out.
    const ggml_cgraph* graph = nullptr;
    int gemv_act_type(int from, const ggml_tensor* out) const {
        for (int i = from; graph && i < graph->n_nodes; ++i) {
            const ggml_tensor* c = graph->nodes[i];
            if (c->op != GGML_OP_MUL_MAT || c->src[1]->data != out->data || nbytes(c->src[1]) != nbytes(out)) continue;
            const ggml_tensor* w = c->src[0];
            if (nrows(c->src[1]) != 1 || c->src[1]->type != GGML_TYPE_F32 || w->ne[0] != nelements(out)) return 0;
            if (w->type == GGML_TYPE_Q4_0 || w->type == GGML_TYPE_Q8_0) return w->ne[0] % 32 == 0 ? (int)GGML_TYPE_Q8_0 : 0;
            if (w->type == GGML_TYPE_Q4_K || w->type == GGML_TYPE_Q6_K) return w->ne[0] % 256 == 0 ? (int)GGML_TYPE_Q8_K : 0;
            return 0;
        }
        return 0;
    }
    void* fused_act(const ggml_tensor* n, const ggml_tensor* out, int atype) {
        void* act = dev->arena.take((size_t)amv_act_bytes(atype, 1, nelements(out)));
        if (!act) fail(n, "scratch exhausted");
        return act;
    }

    bool rms_norm(int i, const ggml_tensor* n, const ggml_tensor* mul) {
        const ggml_tensor* x = n->src[0];
        const float eps = op_f32(n, 0);
        const ggml_tensor* out = mul ? mul : n;
        const int atype = nrows(x) == 1 && aligned16(out->data) ? gemv_act_type(i + (mul ? 2 : 1), out) : 0;
        const ggml_tensor* w = mul ? (mul->src[0] == n ? mul->src[1] : mul->src[0]) : nullptr;
        if (atype) {  // the next GEMV's activation row in the same pass
            void* act = fused_act(n, out, atype);
            if (!act) return false;
            if (!rc(n, amv_rms_norm_act((const float*)x->data, 1, x->ne[0], eps, w ? (const float*)w->data : nullptr,
                                        (float*)n->data, mul ? (float*)mul->data : nullptr, act, atype, AMV_Q8_X86,
                                        st)))
                return false;
            pending_act = {out->data, nbytes(out), atype, 1, nelements(out), act};
            return true;
        }
        if (!mul) return rc(n, amv_rms_norm((const float*)x->data, nrows(x), x->ne[0], eps, nullptr, (float*)n->data,
                                            nullptr, nullptr, AMV_Q8_X86, st));
        return rc(n, amv_rms_norm((const float*)x->data, nrows(x), x->ne[0], eps, (const float*)w->data,
                                  (float*)n->data, (float*)mul->data, nullptr, AMV_Q8_X86, st));
    }

    bool rope(const ggml_tensor* n) {
        const ggml_tensor *x = n->src[0], *pos = n->src[1];
        return rc(n, amv_rope((const float*)x->data, (float*)n->data, (const int32_t*)pos->data, x->ne[2], x->ne[1],
                              x->ne[0], n->op_params[1], n->op_params[2], op_f32(n, 5), op_f32(n, 6), op_f32(n, 8), st));
    }

    bool flash_attn(int i, const ggml_tensor* n) {
        const ggml_tensor *q = n->src[0], *k = n->src[1], *v = n->src[2], *m = n->src[3];
        const int64_t n_head = q->ne[2], n_head_kv = k->ne[2], n_kv = k->ne[1], D = q->ne[0];
        const int64_t ws = amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv, D);
        void* work = dev->arena.take((size_t)ws);
        if (!work) return fail(n, "scratch exhausted");
        // the o projection's activation row written by the split merge (Q8_K needs an even GQA group)
        int atype = q->ne[1] == 1 && aligned16(n->data) ? gemv_act_type(i + 1, n) : 0;
        if (atype == (int)GGML_TYPE_Q8_K && (n_head / n_head_kv) % 2 != 0) atype = 0;
        void* act = atype ? fused_act(n, n, atype) : nullptr;
        if (atype && !act) return false;
        // K / V strides in bytes; a Q8_0 / Q4_0 cache meets q quantized to Q8_0 (x86 rule), as ggml's CPU kernel does
        if (!rc(n, amv_flash_attn_decode_kv(k->type, (const float*)q->data, k->data, v->data, m ? m->data : nullptr,
                                            (float*)n->data, n_head, n_head_kv, n_kv, nullptr, D, (int64_t)k->nb[1],
                                            (int64_t)k->nb[2], (int64_t)v->nb[1], (int64_t)v->nb[2], op_f32(n, 0),
                                            work, ws, nullptr, act, atype ? atype : (int)GGML_TYPE_Q8_0, AMV_Q8_X86,
                                            st)))
            return false;
        if (act) pending_act = {n->data, nbytes(n), atype, 1, nelements(n), act};
        return true;
    }

    bool glu(const ggml_tensor* n) {
        const ggml_tensor *a = n->src[0], *b = n->src[1];
        const bool swapped = n->op_params[1] != 0;
        if (b) {
            const ggml_tensor* g = swapped ? b : a;
            const ggml_tensor* u = swapped ? a : b;
            return rc(n, amv_swiglu((const float*)g->data, (const float*)u->data, (float*)n->data, nelements(n), st));
        }
        const int64_t h = a->ne[0] / 2;
        const float* g = (const float*)a->data + (swapped ? h : 0);
        const float* u = (const float*)a->data + (swapped ? 0 : h);
        return rc(n, amv_swiglu(g, u, (float*)n->data, h, st));
    }

    bool set_rows(const ggml_tensor* n) {
        const ggml_tensor *src = n->src[0], *idx = n->src[1];
        if (n->type != GGML_TYPE_F16)  // Q8_0 / Q4_0 cache rows: ggml's from_float of the type (Q8_0 x86 rule)
            return rc(n, amv_set_rows_q(n->type, (const float*)src->data, (int64_t)src->nb[1] / 4, n->data,
                                        (int64_t)n->nb[1], src->ne[1], src->ne[0], idx->data,
                                        idx->type == GGML_TYPE_I64 ? 64 : 32, n->ne[1], AMV_Q8_X86, dev->status, st));
        return rc(n, amv_set_rows_f16((const float*)src->data, (int64_t)src->nb[1] / 4, n->data, (int64_t)n->nb[1] / 2,
                                      src->ne[1], src->ne[0], idx->data, idx->type == GGML_TYPE_I64 ? 64 : 32, n->ne[1],
                                      dev->status, st));
    }

    bool cpy(const ggml_tensor* n) {
        const ggml_tensor* src = n->src[0];
        if (n->type == GGML_TYPE_F32)
            return hipMemcpyAsync(n->data, src->data, nbytes(src), hipMemcpyDeviceToDevice, st) == hipSuccess
                       ? true
                       : fail(n, "copy failed");
        return rc(n, amv_set_rows_f16((const float*)src->data, nelements(src), n->data, nelements(src), 1,
                                      nelements(src), nullptr, 0, 1, nullptr, st));
    }

    bool get_rows(const ggml_tensor* n) {
        const ggml_tensor *src = n->src[0], *idx = n->src[1];
        const void* sp = src->data;
        BufCtx* bc = (BufCtx*)src->buffer->context;
        {
            std::lock_guard<std::mutex> lk(bc->mu);
            if (bc->repacked.count(src->data)) {  // a weight also used by MUL_MAT: read a ggml-layout copy
                void* tmp = dev->arena.take(nbytes(src));
                if (!tmp) return fail(n, "scratch exhausted");
                if (!rc(n, amv_unrepack(src->type, src->data, tmp, src->ne[1], src->ne[0], st))) return false;
                sp = tmp;
            }
        }
        return rc(n, amv_get_rows(src->type, sp, src->ne[1], src->ne[0], (const int32_t*)idx->data, nelements(idx),
                                  (float*)n->data, dev->status, st));
    }

    // scratch a graph can need at most (activation buffers, attention partials, layout copies)
    static size_t scratch_bound(const ggml_cgraph* g) {
        size_t s = 1 << 20;
        for (int i = 0; i < g->n_nodes; ++i) {
            const ggml_tensor* n = g->nodes[i];
            if (n->op == GGML_OP_MUL_MAT) {
                s += (size_t)amv_act_bytes(AMV_ACT_Q8_0_MMA, nrows(n->src[1]), n->src[1]->ne[0]) + 4096;
                s += (size_t)amv_act_bytes(AMV_ACT_Q8_K_MMA, nrows(n->src[1]), (n->src[1]->ne[0] + 255) / 256 * 256) + 4096;
                if (n->src[0]->view_src) s += nbytes(n->src[0]->view_src) + nbytes(n->src[0]) + 512;
                else if (n->src[0]->buffer->usage != GGML_BACKEND_BUFFER_USAGE_WEIGHTS) s += nbytes(n->src[0]) + 256;
            } else if (n->op == GGML_OP_FLASH_ATTN_EXT) {
                const int64_t ws = amv_flash_attn_workspace_bytes(n->src[0]->ne[2], n->src[1]->ne[2], n->src[1]->ne[1], 128);
                s += (size_t)(ws > 0 ? ws : 0) + 256;
            } else if (n->op == GGML_OP_GET_ROWS) {
                s += nbytes(n->src[0]) + 256;
            }
        }
        return s;
    }

    // MUL by a one-row weight that consumes this RMS_NORM output and nothing else reads that output later
    static const ggml_tensor* fusable_mul(const ggml_cgraph* g, int i) {
        const ggml_tensor* n = g->nodes[i];
        if (i + 1 >= g->n_nodes) return nullptr;
        const ggml_tensor* m = g->nodes[i + 1];
        if (m->op != GGML_OP_MUL) return nullptr;
        const ggml_tensor* w = m->src[0] == n ? m->src[1] : (m->src[1] == n ? m->src[0] : nullptr);
        if (!w || w->type != GGML_TYPE_F32 || nrows(w) != 1 || w->ne[0] != n->ne[0] || !aligned16(w->data)) return nullptr;
        if (m->type != GGML_TYPE_F32 || !is_contiguous(m) || !aligned16(m->data)) return nullptr;
        return m;
    }

    // ADD or GLU SWIGLU (split form) right after a one-row GEMV MUL_MAT that consumes its result with a contiguous f32
    // vector of N elements: computed in the GEMV's epilogue (ameva_find_fusion's MUL_MAT pairs); the MUL_MAT's own
    // output is still written. The fused output must not overlap the activation row, the weight, the MUL_MAT output or
    // the other operand.
    static bool overlaps(const ggml_tensor* a, const ggml_tensor* b) {
        const uint8_t *a0 = (const uint8_t*)a->data, *b0 = (const uint8_t*)b->data;
        return a0 < b0 + nbytes(b) && b0 < a0 + nbytes(a);
    }
    static const ggml_tensor* fusable_epilogue(const ggml_cgraph* g, int i) {
        const ggml_tensor* n = g->nodes[i];
        if (i + 1 >= g->n_nodes || nrows(n->src[1]) != 1) return nullptr;
        const ggml_type wt = n->src[0]->type;
        if (wt != GGML_TYPE_Q4_0 && wt != GGML_TYPE_Q8_0 && wt != GGML_TYPE_Q4_K && wt != GGML_TYPE_Q6_K) return nullptr;
        const ggml_tensor* e = g->nodes[i + 1];
        if (e->op != GGML_OP_ADD && !(e->op == GGML_OP_GLU && e->src[1] && e->op_params[0] == GGML_GLU_OP_SWIGLU))
            return nullptr;
        const ggml_tensor* other = e->src[0] == n ? e->src[1] : (e->src[1] == n ? e->src[0] : nullptr);
        const int64_t N = n->ne[0];
        if (!other || other == n || other->type != GGML_TYPE_F32 || nelements(other) != N || !is_contiguous(other))
            return nullptr;
        if (e->type != GGML_TYPE_F32 || nelements(e) != N || !is_contiguous(e)) return nullptr;
        if (overlaps(e, n->src[1]) || overlaps(e, n) || overlaps(e, other) || overlaps(e, n->src[0])) return nullptr;
        return e;
    }

    // the kind a node's GPU time is booked under: op, and for MUL_MAT the weight type, kernel family and fusion
    static std::string kind_of(const ggml_tensor* n, const ggml_tensor* fused) {
        std::string k = op_name(n->op);
        if (n->op == GGML_OP_MUL_MAT) {
            k += std::string(" ") + type_name(n->src[0]->type) + (nrows(n->src[1]) >= 8 ? " batched" : " gemv");
        }
        if (fused) k += std::string("+") + op_name(fused->op);
        return k;
    }

    // ---- node groups of llama.cpp's decode layer that run as one launch (recognised at their first node)
    static const ggml_tensor* root(const ggml_tensor* t) { return t->view_src ? t->view_src : t; }
    // a node outside `group` (graph indices) computes from t or a view of it
    bool read_outside(const ggml_tensor* t, const std::vector<int>& group) const {
        for (int i = 0; i < graph->n_nodes; ++i) {
            const ggml_tensor* c = graph->nodes[i];
            if (noop(c->op) || std::find(group.begin(), group.end(), i) != group.end()) continue;
            for (int j = 0; j < GGML_MAX_SRC; ++j)
                if (c->src[j] && root(c->src[j]) == t) return true;
        }
        return false;
    }
    static bool gemv_q4(const ggml_tensor* c, const ggml_tensor* x) {  // one-row Q4_0 / Q4_K MUL_MAT of x
        const ggml_tensor* w = c->src[0];
        if (c->op != GGML_OP_MUL_MAT || c->src[1]->data != x->data || nbytes(c->src[1]) != nbytes(x) ||
            nrows(c->src[1]) != 1 || c->src[1]->type != GGML_TYPE_F32 || w->view_src || w->ne[1] % 2 != 0)
            return false;
        if (w->type == GGML_TYPE_Q4_0) return w->ne[0] % 4096 == 0;
        return w->type == GGML_TYPE_Q4_K && w->ne[0] % 256 == 0;
    }

    // q, k, v MUL_MATs of one activation row, ROPE NORMAL of q and k over whole heads at one position, SET_ROWS of
    // k (roped) and v into f16 caches at one row, nothing else in between: amv_gemv_rope_kv_seg
    struct QkvGroup {
        const ggml_tensor *mq, *mk, *mv, *rq, *rk, *sk, *sv;
        int last;
    };
    bool match_qkv(int i, QkvGroup& f) const {
        const ggml_tensor* n0 = graph->nodes[i];
        const ggml_tensor* x = n0->src[1];
        if (!gemv_q4(n0, x)) return false;
        const ggml_tensor *mm[3], *ro[2], *sr[2];
        int nm = 0, nr = 0, ns = 0;
        std::vector<int> group;
        for (int j = i; j < graph->n_nodes && j < i + 32 && !(nm == 3 && nr == 2 && ns == 2); ++j) {
            const ggml_tensor* c = graph->nodes[j];
            if (!noop(c->op)) {
                if (nm < 3 && gemv_q4(c, x) && c->src[0]->type == n0->src[0]->type && c->src[0]->ne[0] == n0->src[0]->ne[0])
                    mm[nm++] = c;
                else if (nr < 2 && c->op == GGML_OP_ROPE)
                    ro[nr++] = c;
                else if (ns < 2 && c->op == GGML_OP_SET_ROWS)
                    sr[ns++] = c;
                else
                    return false;
            }
            group.push_back(j);
            f.last = j;
        }
        if (!(nm == 3 && nr == 2 && ns == 2)) return false;
        f.rk = f.rq = f.sk = f.sv = nullptr;
        for (int a = 0; a < 2; ++a)
            for (int b = 0; b < 2; ++b)
                if (root(sr[b]->src[0]) == ro[a]) {
                    f.rk = ro[a], f.rq = ro[1 - a], f.sk = sr[b], f.sv = sr[1 - b];
                }
        if (!f.rk) return false;
        f.mq = f.mk = f.mv = nullptr;
        for (int a = 0; a < 3; ++a) {
            if (root(f.rq->src[0]) == mm[a]) f.mq = mm[a];
            else if (root(f.rk->src[0]) == mm[a]) f.mk = mm[a];
            else if (root(f.sv->src[0]) == mm[a]) f.mv = mm[a];
        }
        if (!f.mq || !f.mk || !f.mv) return false;
        const ggml_tensor *qi = f.rq->src[0], *ki = f.rk->src[0], *pos = f.rq->src[1], *idx = f.sk->src[1];
        const int64_t D = qi->ne[0], nh = qi->ne[1], nkv = ki->ne[1];
        if (ki->ne[0] != D || qi->ne[2] != 1 || ki->ne[2] != 1 || D % 2 != 0) return false;
        for (const ggml_tensor* r : {f.rq, f.rk})
            if (r->op_params[2] != 0 || r->op_params[1] != D || r->type != GGML_TYPE_F32 || !is_contiguous(r) ||
                !is_contiguous(r->src[0]))
                return false;
        if (f.rk->src[1] != pos || pos->type != GGML_TYPE_I32 || nelements(pos) != 1) return false;
        for (int p : {5, 6, 8})
            if (op_f32(f.rq, p) != op_f32(f.rk, p)) return false;
        if (f.mq->ne[0] != nh * D || f.mk->ne[0] != nkv * D || f.mv->ne[0] != nkv * D) return false;
        if (f.sv->src[1] != idx || idx->type != GGML_TYPE_I64 || nelements(idx) != 1) return false;
        for (const ggml_tensor* c : {f.sk, f.sv})
            if (c->type != GGML_TYPE_F16 || c->ne[0] != nkv * D || c->nb[0] != 2 || nrows(c->src[0]) != 1 ||
                c->src[0]->type != GGML_TYPE_F32 || !is_contiguous(c->src[0]))
                return false;
        if (f.sk->nb[1] != f.sv->nb[1] || f.sk->ne[1] != f.sv->ne[1] || f.sk->nb[1] % 2 != 0) return false;
        if (!is_contiguous(f.mv)) return false;
        // The launch writes q, k, v and both cache rows at once and reads the position and the row index while it
        // writes. ggml-alloc may place a node's output in the memory of a tensor that is dead by then in the graph's
        // own node order (k in q's memory after the q ROPE, say), which is safe node by node but not in one launch:
        // the group is taken only when all of these are disjoint.
        const ggml_tensor* outs[5] = {f.rq, f.rk, f.mv, f.sk, f.sv};
        for (int a = 0; a < 5; ++a) {
            if (overlaps(outs[a], pos) || overlaps(outs[a], idx)) return false;
            for (int b = a + 1; b < 5; ++b)
                if (overlaps(outs[a], outs[b])) return false;
        }
        // the un-rotated q and k exist only inside the launch
        return !read_outside(f.mq, group) && !read_outside(f.mk, group);
    }
    bool run_qkv(const QkvGroup& f) {
        const ggml_tensor* x = f.mq->src[1];
        const int wt = f.mq->src[0]->type;
        const int64_t K = f.mq->src[0]->ne[0];
        const ggml_tensor *qi = f.rq->src[0], *ki = f.rk->src[0];
        const void* wq = weight_ptr(f.mq);
        const void* wk = wq ? weight_ptr(f.mk) : nullptr;
        const void* wv = wk ? weight_ptr(f.mv) : nullptr;
        if (!wv) return false;
        const int atype = wt == GGML_TYPE_Q4_K ? (int)GGML_TYPE_Q8_K : (int)GGML_TYPE_Q8_0;
        void* act = act_for(f.mq, x, atype, 1, K);
        if (!act) return false;
        if (!rc(f.mq, amv_gemv_rope_kv_seg(wt, wq, wk, wv, K, act, (float*)f.rq->data, (float*)f.rk->data,
                                           (float*)f.mv->data, qi->ne[1], ki->ne[1], qi->ne[0],
                                           (const int32_t*)f.rq->src[1]->data, op_f32(f.rq, 5), op_f32(f.rq, 6),
                                           op_f32(f.rq, 8), f.sk->data, f.sv->data, (int64_t)f.sk->nb[1] / 2,
                                           (const int64_t*)f.sk->src[1]->data, f.sk->ne[1], dev->status, st)))
            return false;
        g_cnt.mul_mat += 3;
        g_cnt.qmv += 3;
        g_cnt.fused += 6;  // k, v, both ROPEs and both SET_ROWS ride on the q launch
        return true;
    }

    // gate and up MUL_MATs of one activation row and the GLU SWIGLU of their results, the product read by a later
    // one-row GEMV: amv_gemv_swiglu_q8_seg, which also writes that GEMV's activation row
    struct GateUp {
        const ggml_tensor *gate, *up, *glu;
        int last, atype;
    };
    bool match_gate_up(int i, GateUp& f) const {
        const ggml_tensor* n0 = graph->nodes[i];
        const ggml_tensor* x = n0->src[1];
        if (!gemv_q4(n0, x)) return false;
        std::vector<int> group{i};
        int j = i + 1;
        while (j < graph->n_nodes && noop(graph->nodes[j]->op)) group.push_back(j++);
        if (j >= graph->n_nodes) return false;
        const ggml_tensor* n1 = graph->nodes[j];
        if (!gemv_q4(n1, x) || n1->src[0]->type != n0->src[0]->type || n1->src[0]->ne[0] != n0->src[0]->ne[0] ||
            n1->src[0]->ne[1] != n0->src[0]->ne[1])
            return false;
        group.push_back(j++);
        while (j < graph->n_nodes && noop(graph->nodes[j]->op)) group.push_back(j++);
        if (j >= graph->n_nodes) return false;
        const ggml_tensor* e = graph->nodes[j];
        if (e->op != GGML_OP_GLU || !e->src[1] || e->op_params[0] != GGML_GLU_OP_SWIGLU) return false;
        if (!((e->src[0] == n0 && e->src[1] == n1) || (e->src[0] == n1 && e->src[1] == n0))) return false;
        group.push_back(j);
        const int64_t F = n0->src[0]->ne[1];
        if (F > 65536 || e->type != GGML_TYPE_F32 || nelements(e) != F || !is_contiguous(e) || !aligned16(e->data))
            return false;
        const bool swapped = e->op_params[1] != 0;  // swapped: silu(src1) * src0
        f.gate = swapped ? e->src[1] : e->src[0];
        f.up = swapped ? e->src[0] : e->src[1];
        f.glu = e;
        f.last = j;
        f.atype = gemv_act_type(j + 1, e);
        if (!f.atype || F % (f.atype == (int)GGML_TYPE_Q8_K ? 256 : 32) != 0) return false;
        return !read_outside(n0, group) && !read_outside(n1, group);
    }
    bool run_gate_up(const GateUp& f) {
        const ggml_tensor* x = f.gate->src[1];
        const int wt = f.gate->src[0]->type;
        const int64_t K = f.gate->src[0]->ne[0], F = f.gate->src[0]->ne[1];
        const void* wg = weight_ptr(f.gate);
        const void* wu = wg ? weight_ptr(f.up) : nullptr;
        if (!wu) return false;
        const int atype = wt == GGML_TYPE_Q4_K ? (int)GGML_TYPE_Q8_K : (int)GGML_TYPE_Q8_0;
        void* act = act_for(f.gate, x, atype, 1, K);
        if (!act) return false;
        void* act_out = fused_act(f.glu, f.glu, f.atype);
        if (!act_out) return false;
        if (!rc(f.gate, amv_gemv_swiglu_q8_seg(wt, wg, wu, F, K, act, (float*)f.glu->data, act_out, f.atype,
                                               AMV_Q8_X86, dev->counters, st)))
            return false;
        pending_act = {f.glu->data, nbytes(f.glu), f.atype, 1, F, act_out};
        g_cnt.mul_mat += 2;
        g_cnt.qmv += 2;
        g_cnt.fused += 2;  // up and SWIGLU ride on the gate launch
        return true;
    }

    // RMS_NORM + MUL by a one-row norm weight whose product feeds only the q/k/v group or the gate/up group right
    // after them: the norm is computed inside that group's launch (amv_rms_norm_gemv_*_seg: per workgroup, into LDS,
    // the bytes the norm launch would write) at K = 4096: q/k/v groups of Q4_0 or Q4_K weights, gate/up groups of
    // Q4_0 weights whose SWIGLU row feeds a Q8_0 GEMV. Neither the RMS_NORM nor the MUL output is
    // written, so both must be read by nothing else and not be graph outputs; the norm's input is read by every
    // workgroup during the launch, so no output of the group may overlap it.
    struct NormFold {
        const ggml_tensor *norm, *mul;
        QkvGroup qg;
        GateUp gu;
        bool qkv;
        int last;
    };
    bool match_norm_fold(int i, NormFold& f) const {
        const ggml_tensor* n = graph->nodes[i];
        const ggml_tensor* m = fusable_mul(graph, i);
        if (!m) return false;
        const ggml_tensor* x = n->src[0];
        if (x->type != GGML_TYPE_F32 || nrows(x) != 1 || x->ne[0] != 4096 || !is_contiguous(x) || !aligned16(x->data))
            return false;
        constexpr int32_t FLAG_OUTPUT = 2;  // GGML_TENSOR_FLAG_OUTPUT
        if ((n->flags | m->flags) & FLAG_OUTPUT) return false;
        int j = i + 2;
        while (j < graph->n_nodes && noop(graph->nodes[j]->op)) ++j;
        if (j >= graph->n_nodes) return false;
        const ggml_tensor* c = graph->nodes[j];
        const ggml_type wt = c->src[0]->type;
        if (c->op != GGML_OP_MUL_MAT || c->src[1]->data != m->data || (wt != GGML_TYPE_Q4_0 && wt != GGML_TYPE_Q4_K) ||
            c->src[0]->ne[0] != 4096)
            return false;
        const int out_act = wt == GGML_TYPE_Q4_K ? (int)GGML_TYPE_Q8_K : (int)GGML_TYPE_Q8_0;
        f.norm = n;
        f.mul = m;
        if (match_qkv(j, f.qg)) {
            f.qkv = true;
            f.last = f.qg.last;
            for (const ggml_tensor* o : {f.qg.rq, f.qg.rk, f.qg.mv, f.qg.sk, f.qg.sv})
                if (overlaps(o, x)) return false;
        } else if (wt == GGML_TYPE_Q4_0 && match_gate_up(j, f.gu) && f.gu.atype == out_act) {
            // (Q4_K keeps its FFN norm launch: that fold measured slower on the 32-layer model)
            f.qkv = false;
            f.last = f.gu.last;
            if (overlaps(f.gu.glu, x)) return false;
        } else {
            return false;
        }
        std::vector<int> group;
        for (int g = i; g <= f.last; ++g) group.push_back(g);
        return !read_outside(n, group) && !read_outside(m, group);
    }
    bool run_norm_fold(const NormFold& f) {
        const ggml_tensor* x = f.norm->src[0];
        const ggml_tensor* w = f.mul->src[0] == f.norm ? f.mul->src[1] : f.mul->src[0];
        const float eps = op_f32(f.norm, 0);
        if (f.qkv) {
            const QkvGroup& q = f.qg;
            const int wt = q.mq->src[0]->type;
            const int64_t K = q.mq->src[0]->ne[0];
            const ggml_tensor *qi = q.rq->src[0], *ki = q.rk->src[0];
            const void* wq = weight_ptr(q.mq);
            const void* wk = wq ? weight_ptr(q.mk) : nullptr;
            const void* wv = wk ? weight_ptr(q.mv) : nullptr;
            if (!wv) return false;
            if (!rc(q.mq, amv_rms_norm_gemv_rope_kv_seg(
                              (const float*)x->data, (const float*)w->data, eps, AMV_Q8_X86, wt, wq, wk, wv, K,
                              (float*)q.rq->data, (float*)q.rk->data, (float*)q.mv->data, qi->ne[1], ki->ne[1],
                              qi->ne[0], (const int32_t*)q.rq->src[1]->data, op_f32(q.rq, 5), op_f32(q.rq, 6),
                              op_f32(q.rq, 8), q.sk->data, q.sv->data, (int64_t)q.sk->nb[1] / 2,
                              (const int64_t*)q.sk->src[1]->data, q.sk->ne[1], dev->status, st)))
                return false;
            g_cnt.mul_mat += 3;
            g_cnt.qmv += 3;
            g_cnt.fused += 8;  // the norm, its MUL, k, v, both ROPEs and both SET_ROWS ride on the q launch
            return true;
        }
        const GateUp& u = f.gu;
        const int wt = u.gate->src[0]->type;
        const int64_t K = u.gate->src[0]->ne[0], F = u.gate->src[0]->ne[1];
        const void* wg = weight_ptr(u.gate);
        const void* wu = wg ? weight_ptr(u.up) : nullptr;
        if (!wu) return false;
        void* act_out = fused_act(u.glu, u.glu, u.atype);
        if (!act_out) return false;
        if (!rc(u.gate, amv_rms_norm_gemv_swiglu_q8_seg((const float*)x->data, (const float*)w->data, eps, AMV_Q8_X86,
                                                        wt, wg, wu, F, K, (float*)u.glu->data, act_out, dev->counters,
                                                        st)))
            return false;
        pending_act = {u.glu->data, nbytes(u.glu), u.atype, 1, F, act_out};
        g_cnt.mul_mat += 2;
        g_cnt.qmv += 2;
        g_cnt.fused += 4;  // the norm, its MUL, up and SWIGLU ride on the gate launch
        return true;
    }

    bool run(ggml_cgraph* g) {
        graph = g;
        const bool prof = profile_level() >= 2;
        if (prof) {
            hipEvent_t e0 = dev->event(0);
            if (!e0 || hipEventRecord(e0, st) != hipSuccess) return fail(nullptr, "profile event");
        }
        for (int i = 0; i < g->n_nodes; ++i) {
            const ggml_tensor* n = g->nodes[i];
            if (noop(n->op)) continue;
            const ggml_tensor* first = n;
            bool ok = true;
            if ((n->op == GGML_OP_MUL_MAT || n->op == GGML_OP_RMS_NORM) && g_fail.load() == AMEVA_FAIL_NONE) {
                QkvGroup qg;
                GateUp gu;
                NormFold nf;
                int last = -1;
                if (n->op == GGML_OP_RMS_NORM) {
                    if (match_norm_fold(i, nf)) {
                        ok = run_norm_fold(nf);
                        last = nf.last;
                    }
                } else if (match_qkv(i, qg)) {
                    ok = run_qkv(qg);
                    last = qg.last;
                } else if (match_gate_up(i, gu)) {
                    ok = run_gate_up(gu);
                    last = gu.last;
                }
                if (last >= 0) {
                    if (!ok) return false;
                    for (int j = i; j <= last; ++j) invalidate(g->nodes[j]);
                    if (pending_act.act) {
                        acts.push_back(pending_act);
                        pending_act = {};
                    }
                    g_cnt.gpu_op++;
                    encoded++;
                    if (prof) {
                        labels.push_back(kind_of(first, g->nodes[last]));
                        hipEvent_t ev = dev->event(labels.size());
                        if (!ev || hipEventRecord(ev, st) != hipSuccess) return fail(n, "profile event");
                    }
                    i = last;
                    continue;
                }
            }
            switch (n->op) {
            case GGML_OP_MUL_MAT: {
                const ggml_tensor* e = fusable_epilogue(g, i);
                ok = mul_mat(n, e);
                if (ok && e) {
                    invalidate(n);
                    g_cnt.gpu_op++;
                    g_cnt.fused++;
                    ++i;
                    n = e;
                }
                break;
            }
            case GGML_OP_RMS_NORM: {
                const ggml_tensor* m = fusable_mul(g, i);
                ok = rms_norm(i, n, m);
                if (ok && m) {
                    invalidate(n);
                    invalidate(m);
                    g_cnt.gpu_op++;
                    g_cnt.fused++;
                    ++i;
                    n = m;
                }
                break;
            }
            case GGML_OP_ADD: ok = binary(n, 0); break;
            case GGML_OP_MUL: ok = binary(n, 1); break;
            case GGML_OP_ROPE: ok = rope(n); break;
            case GGML_OP_FLASH_ATTN_EXT: ok = flash_attn(i, n); break;
            case GGML_OP_GLU: ok = glu(n); break;
            case GGML_OP_SET_ROWS: ok = set_rows(n); break;
            case GGML_OP_CPY:
            case GGML_OP_CONT: ok = cpy(n); break;
            case GGML_OP_GET_ROWS: ok = get_rows(n); break;
            default: ok = fail(n, "no encoder");
            }
            if (!ok) return false;
            invalidate(n);
            if (pending_act.act) {  // an activation row written with the node's output: valid from here on
                acts.push_back(pending_act);
                pending_act = {};
            }
            g_cnt.gpu_op++;
            encoded++;
            if (prof) {
                labels.push_back(kind_of(first, n != first ? n : nullptr));
                hipEvent_t e = dev->event(labels.size());
                if (!e || hipEventRecord(e, st) != hipSuccess) return fail(n, "profile event");
            }
        }
        return true;
    }
};

// The status words are cleared by kernels, not memset nodes: the last kernel of every run (eager or captured) copies
// the bad-index count to pinned host memory and clears the words for the next run; a run that stopped early leaves
// them for k_clear_status before the next one.
__global__ void k_clear_status(unsigned int* s) { s[threadIdx.x] = 0u; }
__global__ void k_status_out(unsigned int* s, unsigned int* host) {
    const unsigned int v = s[0];
    if (threadIdx.x == 0) host[0] = v;
    s[threadIdx.x] = 0u;
}

void sig_tensor(std::vector<int64_t>& s, const ggml_tensor* t) {
    s.push_back((int64_t)(uintptr_t)t->data);
    s.push_back((int64_t)t->type);
    s.push_back((int64_t)t->op);
    for (int i = 0; i < 4; ++i) {
        s.push_back(t->ne[i]);
        s.push_back((int64_t)t->nb[i]);
    }
    s.push_back((int64_t)t->view_offs);
    s.push_back((int64_t)(uintptr_t)t->buffer);
    for (int i = 0; i < 16; ++i) s.push_back(t->op_params[i]);
}

std::vector<int64_t> graph_signature(const ggml_cgraph* g) {
    std::vector<int64_t> s;
    s.reserve((size_t)g->n_nodes * 8 * 30);
    s.push_back(g->n_nodes);
    for (int i = 0; i < g->n_nodes; ++i) {
        const ggml_tensor* n = g->nodes[i];
        sig_tensor(s, n);
        for (int j = 0; j < GGML_MAX_SRC; ++j) {
            if (n->src[j]) sig_tensor(s, n->src[j]);
            else s.push_back(-1);
        }
    }
    return s;
}

// AMEVA_GRAPH=0: every graph runs eagerly (no capture, no replay)
bool graph_replay_on() {
    static const bool on = [] {
        const char* e = std::getenv("AMEVA_GRAPH");
        return !(e && e[0] == '0' && e[1] == 0);
    }();
    return on;
}

// Bounded completion wait (ggml-ameva.cpp:5545-5561): a graph gets 30 s plus its multiply-accumulates at 0.05e9 per
// second (at most two hours; AMEVA_WAIT_TIMEOUT_S = 1..86400 seconds replaces that, any other value aborts), then it
// fails with GGML_STATUS_FAILED instead of blocking the caller for ever. The wait polls an event recorded after the
// graph's last kernel: spinning for the first 2 ms (a decode graph completes in a fraction of that), then sleeping
// 50 us between polls. Failure injection point 7 (AMEVA_FAIL_WAIT_TIMEOUT) gives a limit of zero.
double graph_macs(const ggml_cgraph* g) {
    double macs = 0.0;
    for (int i = 0; i < g->n_nodes; ++i) {
        const ggml_tensor* n = g->nodes[i];
        if (n->op == GGML_OP_MUL_MAT) macs += (double)nelements(n) * (double)n->src[0]->ne[0];
        else if (n->op == GGML_OP_FLASH_ATTN_EXT)  // q.k and p.v over every key of every query head
            macs += 2.0 * (double)n->src[0]->ne[0] * (double)n->src[1]->ne[1] * (double)n->src[0]->ne[2] *
                    (double)n->src[0]->ne[1];
        else macs += (double)nelements(n);
    }
    return macs;
}
uint64_t wait_limit_ns(double macs) {
    static const uint64_t override_s = [] {
        const char* e = std::getenv("AMEVA_WAIT_TIMEOUT_S");
        if (!e || !*e) return (uint64_t)0;
        char* end = nullptr;
        const unsigned long long v = std::strtoull(e, &end, 10);
        if (!end || *end || v < 1 || v > 86400) {
            log_line("AMEVA_WAIT_TIMEOUT_S must be 1..86400 (got \"%s\")", e);
            std::abort();
        }
        return (uint64_t)v;
    }();
    if (g_fail.load() == AMEVA_FAIL_WAIT_TIMEOUT) return 0;
    const uint64_t work_s = (uint64_t)std::min(7170.0, macs / 0.05e9);
    return (override_s ? override_s : 30 + work_s) * 1000000000ull;
}
struct WaitResult {
    hipError_t se = hipSuccess;
    bool timed_out = false;
};
WaitResult bounded_wait(Device* d, uint64_t limit_ns) {
    WaitResult w;
    if ((w.se = hipEventRecord(d->done, d->stream)) != hipSuccess) return w;
    const auto t0 = std::chrono::steady_clock::now();
    for (uint64_t polls = 0;; ++polls) {
        const uint64_t el = (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                                std::chrono::steady_clock::now() - t0).count();
        if (el >= limit_ns) {
            w.timed_out = true;
            return w;
        }
        const hipError_t q = hipEventQuery(d->done);
        if (q == hipSuccess) return w;
        if (q != hipErrorNotReady) {
            w.se = q;
            return w;
        }
        if (el > 2000000) std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
}
enum ggml_status finish_graph(Device* d, bool ok, const std::string& why, const WaitResult& w);

enum ggml_status graph_compute(ggml_backend_t, ggml_cgraph* g) {
    Device* d = device();
    std::lock_guard<std::mutex> lk(d->compute_mu);
    if (!d->init()) {
        log_line("no HIP device (FAIL-FAST)");
        return GGML_STATUS_FAILED;
    }
    // contract pass over the whole graph before anything runs
    for (int i = 0; i < g->n_nodes; ++i) {
        const char* why = unsupported_reason(g->nodes[i]);
        if (why) {
            log_line("graph rejected at node %d %s: %s (FAIL-FAST)", i, g->nodes[i]->name, why);
            return GGML_STATUS_FAILED;
        }
    }
    if (!d->arena.reserve(Engine::scratch_bound(g))) {
        log_line("scratch allocation failed (FAIL-FAST)");
        return GGML_STATUS_FAILED;
    }
    d->arena.used = 0;
    const int prof = profile_level();
    const uint64_t limit_ns = wait_limit_ns(graph_macs(g));
    // A graph identical to the last one (same signature, no layout change since) is replayed from its HIP graph,
    // captured on its second computation; the first runs eagerly (it repacks weights on first use).
    Replay& rp = d->replay;
    const bool can_graph = graph_replay_on() && !prof && g_fail.load() == AMEVA_FAIL_NONE;
    std::vector<int64_t> sig;
    bool same = false;
    if (can_graph) {
        sig = graph_signature(g);
        same = sig == rp.sig && rp.gen == g_layout_gen.load();
        if (same && rp.exec && rp.arena_base != d->arena.base) rp.drop();  // the scratch moved: capture again
    }
    if (!d->status_clean) hipLaunchKernelGGL(k_clear_status, dim3(1), dim3(64), 0, d->stream, d->status);
    d->status_clean = false;  // until a run completes through k_status_out
    if (same && rp.exec) {
        if (trace_on()) std::fprintf(stderr, "AMEVA_TRACE graph replay nodes=%d\n", g->n_nodes);
        const bool ok = hipGraphLaunch(rp.exec, d->stream) == hipSuccess;
        if (ok) {
            g_cnt.gpu_op += rp.d_gpu_op;
            g_cnt.mul_mat += rp.d_mul_mat;
            g_cnt.qmv += rp.d_qmv;
            g_cnt.mmq += rp.d_mmq;
            g_cnt.fused += rp.d_fused;
            g_cnt.act_reuse += rp.d_act_reuse;
        }
        return finish_graph(d, ok, ok ? std::string() : std::string("graph replay failed"),
                            ok ? bounded_wait(d, limit_ns) : WaitResult{});
    }
    if (!same || !can_graph) {
        rp.drop();
        rp.sig = std::move(sig);  // empty when graphs are off: never equal to a real signature
    }
    if (same && !rp.exec && !rp.uncapturable) {
        // second computation: capture, then launch the capture (the captured work has not run yet)
        const int64_t c0[6] = {g_cnt.gpu_op, g_cnt.mul_mat, g_cnt.qmv, g_cnt.mmq, g_cnt.fused, g_cnt.act_reuse};
        Engine e;
        e.dev = d;
        e.st = d->stream;
        hipGraph_t graph = nullptr;
        bool ok = hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal) == hipSuccess;
        if (ok) {
            ok = e.run(g);
            if (ok) hipLaunchKernelGGL(k_status_out, dim3(1), dim3(64), 0, d->stream, d->status, d->status_host_dev);
            const bool ended = hipStreamEndCapture(d->stream, &graph) == hipSuccess;
            ok = ok && ended && graph &&
                 hipGraphInstantiate(&rp.exec, graph, nullptr, nullptr, 0) == hipSuccess;
            if (graph) (void)hipGraphDestroy(graph);
        }
        (void)hipGetLastError();
        if (ok) {
            rp.arena_base = d->arena.base;
            rp.d_gpu_op = g_cnt.gpu_op - c0[0];
            rp.d_mul_mat = g_cnt.mul_mat - c0[1];
            rp.d_qmv = g_cnt.qmv - c0[2];
            rp.d_mmq = g_cnt.mmq - c0[3];
            rp.d_fused = g_cnt.fused - c0[4];
            rp.d_act_reuse = g_cnt.act_reuse - c0[5];
            rp.encoded = e.encoded;
            if (trace_on()) std::fprintf(stderr, "AMEVA_TRACE graph captured nodes=%d\n", g->n_nodes);
            const bool launched = hipGraphLaunch(rp.exec, d->stream) == hipSuccess;
            return finish_graph(d, launched, launched ? std::string() : std::string("graph launch failed"),
                                launched ? bounded_wait(d, limit_ns) : WaitResult{});
        }
        // not capturable (a step needed something a capture cannot hold): undo the counts, run eagerly below
        if (rp.exec) (void)hipGraphExecDestroy(rp.exec);
        rp.exec = nullptr;
        rp.uncapturable = true;
        g_cnt.gpu_op = c0[0];
        g_cnt.mul_mat = c0[1];
        g_cnt.qmv = c0[2];
        g_cnt.mmq = c0[3];
        g_cnt.fused = c0[4];
        g_cnt.act_reuse = c0[5];
        d->arena.used = 0;
    }
    const double t0 = prof || trace_on() ? now_ms() : 0.0;
    Engine e;
    e.dev = d;
    e.st = d->stream;
    const bool ok = e.run(g);
    if (ok) hipLaunchKernelGGL(k_status_out, dim3(1), dim3(64), 0, d->stream, d->status, d->status_host_dev);
    const double t1 = prof || trace_on() ? now_ms() : 0.0;
    int64_t graph_no = 0;
    if (trace_on()) {
        std::lock_guard<std::mutex> pl(g_prof.mu);
        graph_no = g_prof.graphs;
        std::fprintf(stderr, "AMEVA_TRACE graph=%lld nodes=%d encoded=%lld encode_ms=%.3f\n", (long long)graph_no,
                     g->n_nodes, (long long)e.encoded, t1 - t0);
    }
    const WaitResult w = bounded_wait(d, limit_ns);  // also after a failed encode: what was queued completes
    const hipError_t se = w.timed_out ? hipErrorNotReady : w.se;
    if (prof) {
        const double t2 = now_ms();
        std::lock_guard<std::mutex> pl(g_prof.mu);
        g_prof.graphs++;
        g_prof.nodes += g->n_nodes;
        g_prof.launches += e.encoded;
        g_prof.encode_ms += t1 - t0;
        g_prof.wait_ms += t2 - t1;
        if (ok && se == hipSuccess && prof >= 2 && !e.labels.empty()) {
            double total = 0;
            for (size_t i = 0; i < e.labels.size(); ++i) {
                float ms = 0.0f;
                if (hipEventElapsedTime(&ms, d->events[i], d->events[i + 1]) != hipSuccess) continue;
                g_prof.add_kind(e.labels[i], ms);
                total += ms;
            }
            g_prof.gpu_ms += total;
            g_prof.gpu_samples++;
        }
    }
    if (trace_on())
        std::fprintf(stderr, "AMEVA_TRACE graph=%lld done status=%s\n", (long long)graph_no,
                     ok && se == hipSuccess ? "ok" : "failed");
    if (!ok) {
        log_line("%s (FAIL-FAST)", e.why.c_str());
        return GGML_STATUS_FAILED;
    }
    rp.gen = g_layout_gen.load();  // the layout this run left (its first use repacked the weights)
    return finish_graph(d, true, std::string(), w);
}

// after the graph's work is queued (eager) or launched (replay): wait, then the status word
enum ggml_status finish_graph(Device* d, bool ok, const std::string& why, const WaitResult& w) {
    if (!ok) {
        log_line("%s (FAIL-FAST)", why.c_str());
        return GGML_STATUS_FAILED;
    }
    if (w.timed_out) {
        // the graph may still run: the status words are cleared before the next one
        log_line("graph did not complete within the wait limit%s (FAIL-FAST)",
                 g_fail.load() == AMEVA_FAIL_WAIT_TIMEOUT ? " (failure injection: wait timeout)" : "");
        return GGML_STATUS_FAILED;
    }
    const hipError_t se = w.se;
    if (se != hipSuccess) {
        log_line("graph execution failed: %s (FAIL-FAST)", hipGetErrorString(se));
        return GGML_STATUS_FAILED;
    }
    d->status_clean = true;  // k_status_out ran last
    const unsigned int bad = *(volatile unsigned int*)d->status_host;  // copied by the graph's last kernel
    if (bad != 0 || g_fail.load() == AMEVA_FAIL_INVALIDATE_DST) {
        log_line("%u row indices out of range (FAIL-FAST)", bad);
        return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

// ------------------------------------------------------------------------------------------------ backend / device
ggml_guid g_guid = {0x61, 0x6d, 0x65, 0x76, 0x61, 0x2d, 0x6d, 0x69, 0x33, 0x35, 0x35, 0x78, 0x2d, 0x68, 0x69, 0x70};

const char* be_get_name(ggml_backend_t) { return GGML_AMEVA_NAME; }
void be_free(ggml_backend_t b) {
    g_cnt.ctx_destroy++;
    delete b;
}

const ggml_backend_i g_backend_iface = {be_get_name, be_free, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                        nullptr,     nullptr, nullptr, nullptr, graph_compute, nullptr, nullptr, nullptr};

const char* dev_get_name(ggml_backend_dev_t) { return GGML_AMEVA_DEVICE_NAME; }
const char* dev_get_description(ggml_backend_dev_t) { return GGML_AMEVA_DEVICE_DESCRIPTION; }
void dev_get_memory(ggml_backend_dev_t, size_t* fr, size_t* total) {
    *fr = 0;
    *total = 0;
    if (device()->init()) (void)hipMemGetInfo(fr, total);
}
enum ggml_backend_dev_type dev_get_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }
void dev_get_props(ggml_backend_dev_t d, ggml_backend_dev_props* p) {
    p->name = dev_get_name(d);
    p->description = dev_get_description(d);
    dev_get_memory(d, &p->memory_free, &p->memory_total);
    p->type = GGML_BACKEND_DEVICE_TYPE_GPU;
    p->device_id = nullptr;
    p->caps = {false, false, false, false};
}
ggml_backend_t dev_init_backend(ggml_backend_dev_t, const char*) { return ggml_backend_ameva_init(0); }
ggml_backend_buffer_type_t dev_get_buffer_type(ggml_backend_dev_t) { return &g_buft; }
bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor* op) {
    g_cnt.supports_query++;
    const bool ok = unsupported_reason(op) == nullptr;
    if (ok) g_cnt.supported_op++;
    return ok;
}
bool dev_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t b) { return b == &g_buft; }
bool dev_offload_op(ggml_backend_dev_t, const ggml_tensor* op) {
    // a weight held by the host is worth copying for batches of prompt size
    return op->op == GGML_OP_MUL_MAT && op->ne[1] >= 32;
}

struct ggml_backend_device g_device;
struct ggml_backend_reg g_reg;

const char* reg_get_name(ggml_backend_reg_t) { return GGML_AMEVA_NAME; }
size_t reg_get_device_count(ggml_backend_reg_t) { return 1; }
ggml_backend_dev_t reg_get_device(ggml_backend_reg_t, size_t i) { return i == 0 ? &g_device : nullptr; }
void* reg_get_proc_address(ggml_backend_reg_t, const char* name) {
    if (std::strcmp(name, "ggml_backend_ameva_profile_report") == 0) return (void*)ggml_backend_ameva_profile_report;
    if (std::strcmp(name, "ggml_backend_ameva_reset_counters") == 0) return (void*)ggml_backend_ameva_reset_counters;
    return nullptr;
}

void setup_registry() {
    static std::once_flag once;
    std::call_once(once, [] {
        g_device.iface = {dev_get_name,        dev_get_description, dev_get_memory,  dev_get_type,    dev_get_props,
                          dev_init_backend,    dev_get_buffer_type, nullptr,         nullptr,         dev_supports_op,
                          dev_supports_buft,   dev_offload_op,      nullptr,         nullptr,         nullptr};
        g_device.reg = &g_reg;
        g_device.context = nullptr;
        g_reg.api_version = GGML_BACKEND_API_VERSION;
        g_reg.iface = {reg_get_name, reg_get_device_count, reg_get_device, reg_get_proc_address};
        g_reg.context = nullptr;
        g_buft.device = &g_device;
    });
}

// ---- load-time check of the host's ggml ABI (the reference's ameva_abi_check, ggml-ameva-device.cpp:415-495)
// ggml-backend-impl.h carries no ABI version: a libggml-base built from other headers (another member count in a
// vtable, another GGML_MAX_NAME) reads this plugin's structs at shifted offsets. Before the registry reaches the
// host, objects laid out by ggml_abi.h are read back through the host's own accessors, and every op and type value
// the engine dispatches on is named by the host. The accessors are looked up in the library that provides
// ggml_backend_buffer_init (the plugin's one link-time host symbol), else in the global scope.
struct abi_init_params {  // struct ggml_init_params (ggml.h)
    size_t mem_size;
    void* mem_buffer;
    bool no_alloc;
};
struct ggml_context;

const char* abi_check() {
    static std::once_flag once;
    static char msg[448];
    static const char* result = nullptr;
    std::call_once(once, [] {
        void* lib = nullptr;
        Dl_info info{};
        if (dladdr((void*)&ggml_backend_buffer_init, &info) && info.dli_fname)
            lib = dlopen(info.dli_fname, RTLD_LAZY | RTLD_NOLOAD);
        const char* missing = nullptr;
        auto sym = [&](const char* name) -> void* {
            void* p = lib ? dlsym(lib, name) : nullptr;
            if (!p) p = dlsym(RTLD_DEFAULT, name);
            if (!p && !missing) missing = name;
            return p;
        };
        auto get_device = (ggml_backend_dev_t(*)(ggml_backend_t))sym("ggml_backend_get_device");
        auto buf_size = (size_t(*)(ggml_backend_buffer_t))sym("ggml_backend_buffer_get_size");
        auto buf_type = (ggml_backend_buffer_type_t(*)(ggml_backend_buffer_t))sym("ggml_backend_buffer_get_type");
        auto buft_device = (ggml_backend_dev_t(*)(ggml_backend_buffer_type_t))sym("ggml_backend_buft_get_device");
        auto dev_reg = (ggml_backend_reg_t(*)(ggml_backend_dev_t))sym("ggml_backend_dev_backend_reg");
        auto op_nm = (const char* (*)(int))sym("ggml_op_name");
        auto type_nm = (const char* (*)(int))sym("ggml_type_name");
        auto overhead = (size_t(*)(void))sym("ggml_tensor_overhead");
        auto init = (ggml_context * (*)(abi_init_params))sym("ggml_init");
        auto free_ctx = (void (*)(ggml_context*))sym("ggml_free");
        auto new_2d = (ggml_tensor * (*)(ggml_context*, int, int64_t, int64_t))sym("ggml_new_tensor_2d");
        auto mul_mat = (ggml_tensor * (*)(ggml_context*, ggml_tensor*, ggml_tensor*))sym("ggml_mul_mat");
        auto nbytes_fn = (size_t(*)(const ggml_tensor*))sym("ggml_nbytes");
        auto set_name = (ggml_tensor * (*)(ggml_tensor*, const char*))sym("ggml_set_name");
        auto get_name = (const char* (*)(const ggml_tensor*))sym("ggml_get_name");
        if (lib) dlclose(lib);
        if (missing) {
            std::snprintf(msg, sizeof(msg), "the host's libggml-base does not export %s: its ABI cannot be checked",
                          missing);
            result = msg;
            return;
        }
        const char* what = nullptr;
        ggml_backend pb{};
        pb.device = &g_device;
        ggml_backend_buffer_type pbt{};
        pbt.device = &g_device;
        ggml_backend_buffer pbuf{};
        pbuf.buft = &pbt;
        pbuf.size = 0x5A17;
        ggml_backend_device pd{};
        pd.reg = &g_reg;
        if (get_device(&pb) != &g_device) what = "struct ggml_backend (ggml_backend_i member count)";
        else if (buf_size(&pbuf) != 0x5A17 || buf_type(&pbuf) != &pbt)
            what = "struct ggml_backend_buffer (ggml_backend_buffer_i member count)";
        else if (buft_device(&pbt) != &g_device) what = "struct ggml_backend_buffer_type";
        else if (dev_reg(&pd) != &g_reg) what = "struct ggml_backend_device";
        // every op and type value graph_compute and supports_op switch on
        static const struct { int v; const char* name; } ops[] = {
            {GGML_OP_NONE, "NONE"},         {GGML_OP_ADD, "ADD"},         {GGML_OP_MUL, "MUL"},
            {GGML_OP_RMS_NORM, "RMS_NORM"}, {GGML_OP_MUL_MAT, "MUL_MAT"}, {GGML_OP_CPY, "CPY"},
            {GGML_OP_CONT, "CONT"},         {GGML_OP_RESHAPE, "RESHAPE"}, {GGML_OP_VIEW, "VIEW"},
            {GGML_OP_PERMUTE, "PERMUTE"},   {GGML_OP_TRANSPOSE, "TRANSPOSE"}, {GGML_OP_GET_ROWS, "GET_ROWS"},
            {GGML_OP_SET_ROWS, "SET_ROWS"}, {GGML_OP_SOFT_MAX, "SOFT_MAX"}, {GGML_OP_ROPE, "ROPE"},
            {GGML_OP_FLASH_ATTN_EXT, "FLASH_ATTN_EXT"}, {GGML_OP_UNARY, "UNARY"}, {GGML_OP_GLU, "GLU"}};
        static const struct { int v; const char* name; } types[] = {
            {GGML_TYPE_F32, "f32"},   {GGML_TYPE_F16, "f16"},   {GGML_TYPE_Q4_0, "q4_0"}, {GGML_TYPE_Q8_0, "q8_0"},
            {GGML_TYPE_Q4_K, "q4_K"}, {GGML_TYPE_Q6_K, "q6_K"}, {GGML_TYPE_I32, "i32"},   {GGML_TYPE_I64, "i64"}};
        for (const auto& o : ops) {
            const char* s = what ? nullptr : op_nm(o.v);
            if (!what && (!s || std::strcmp(s, o.name) != 0)) what = "enum ggml_op";
        }
        for (const auto& t : types) {
            const char* s = what ? nullptr : type_nm(t.v);
            if (!what && (!s || std::strcmp(s, t.name) != 0)) what = "enum ggml_type";
        }
        if (!what) {
            // struct ggml_tensor: a MUL_MAT node built by the host, read with this plugin's layout
            ggml_context* ctx = init(abi_init_params{8 * overhead(), nullptr, true});
            if (!ctx) {
                what = "ggml_init for the tensor layout probe";
            } else {
                ggml_tensor* a = new_2d(ctx, GGML_TYPE_F32, 8, 3);
                ggml_tensor* b = new_2d(ctx, GGML_TYPE_F32, 8, 2);
                ggml_tensor* c = a && b ? mul_mat(ctx, a, b) : nullptr;
                if (!c || c->op != GGML_OP_MUL_MAT || c->src[0] != a || c->src[1] != b || c->type != GGML_TYPE_F32 ||
                    c->ne[0] != 3 || c->ne[1] != 2 || a->nb[1] != 32 || nbytes_fn(c) != 24 || c->data != nullptr)
                    what = "struct ggml_tensor";
                // the host cuts a name to its own GGML_MAX_NAME - 1 characters; extra sits behind name[]
                char probe[512];
                std::memset(probe, 'n', sizeof(probe) - 1);
                probe[sizeof(probe) - 1] = 0;
                if (!what && std::strlen(get_name(set_name(c, probe))) != sizeof(c->name) - 1)
                    what = "struct ggml_tensor (GGML_MAX_NAME)";
                free_ctx(ctx);
            }
        }
        if (what) {
            std::snprintf(msg, sizeof(msg),
                          "ABI mismatch with the loaded libggml-base: %s differs from the ggml 0.9.8 layout "
                          "libggml-ameva.so was built with (offsetof(ggml_backend, device) = %zu); rebuild it against "
                          "the host's ggml headers",
                          what, offsetof(ggml_backend, device));
            result = msg;
        }
    });
    return result;
}

}  // namespace

// ------------------------------------------------------------------------------------------------ exports
extern "C" {

ggml_backend_reg_t ggml_backend_ameva_reg(void) {
    setup_registry();
    return &g_reg;
}
void ggml_backend_ameva_register(void) {
    if (const char* why = abi_check()) {
        log_line("not registering the AMEVA backend: %s", why);
        return;
    }
    setup_registry();
}
void ggml_backend_ameva_teardown(void) {
    Device* d = device();
    std::lock_guard<std::mutex> lk(d->compute_mu);
    if (d->inited) {
        (void)hipStreamSynchronize(d->stream);
        if (d->arena.base) (void)hipFree(d->arena.base);
        d->arena = Arena{};
        d->replay.drop();
        d->replay.sig.clear();
        (void)hipFree(d->status);
        (void)hipFree(d->counters);
        d->counters = nullptr;
        (void)hipHostFree(d->status_host);
        d->status_host = nullptr;
        (void)hipStreamDestroy(d->stream);
        d->inited = false;
    }
}
// the dynamic loader's entry (ggml-ameva.cpp:5693-5702): NULL when the host's ggml ABI differs, so the loader
// reports the backend as failed instead of reading this plugin's structs at the wrong offsets
ggml_backend_reg_t ggml_backend_init(void) {
    if (const char* why = abi_check()) {
        log_line("refusing to load: %s", why);
        return nullptr;
    }
    return ggml_backend_ameva_reg();
}
// the reason ggml_backend_init refuses, or NULL when the host's ABI matches
const char* ggml_backend_ameva_abi_check(void) { return abi_check(); }
int ggml_backend_score(void) { return 100; }

ggml_backend_t ggml_backend_ameva_init(size_t dev_num) {
    if (dev_num != 0) {
        log_line("device %zu does not exist (AMEVA0 only)", dev_num);
        return nullptr;
    }
    if (const char* why = abi_check()) {
        log_line("cannot create the AMEVA backend: %s", why);
        return nullptr;
    }
    setup_registry();
    if (!device()->init()) {
        log_line("no HIP device (FAIL-FAST)");
        return nullptr;
    }
    ggml_backend* b = new ggml_backend;
    b->guid = &g_guid;
    b->iface = g_backend_iface;
    b->device = &g_device;
    b->context = nullptr;
    return b;
}
bool ggml_backend_is_ameva(ggml_backend_t b) { return b && b->guid == &g_guid; }
ggml_backend_buffer_type_t ggml_backend_ameva_buffer_type(size_t dev_num) {
    setup_registry();
    return dev_num == 0 ? &g_buft : nullptr;
}

int64_t ggml_backend_ameva_get_supports_query_count(void) { return g_cnt.supports_query; }
int64_t ggml_backend_ameva_get_supported_op_count(void) { return g_cnt.supported_op; }
int64_t ggml_backend_ameva_get_gpu_op_count(void) { return g_cnt.gpu_op; }
int64_t ggml_backend_ameva_get_q5_0_cpu_dequant_count(void) { return 0; }
int64_t ggml_backend_ameva_get_f32_gpu_sgemm_dispatch_count(void) { return g_cnt.mul_mat; }
int64_t ggml_backend_ameva_get_context_create_count(void) { return g_cnt.ctx_create; }
int64_t ggml_backend_ameva_get_context_destroy_count(void) { return g_cnt.ctx_destroy; }
int64_t ggml_backend_ameva_get_kernel_create_count(void) { return 0; }
int64_t ggml_backend_ameva_get_kernel_destroy_count(void) { return 0; }
int64_t ggml_backend_ameva_get_buffer_create_count(void) { return g_cnt.buf_create; }
int64_t ggml_backend_ameva_get_buffer_destroy_count(void) { return g_cnt.buf_destroy; }
int64_t ggml_backend_ameva_get_event_create_count(void) { return 0; }
int64_t ggml_backend_ameva_get_event_destroy_count(void) { return 0; }
int64_t ggml_backend_ameva_get_q5_0_staging_alloc_count(void) { return 0; }
int64_t ggml_backend_ameva_get_q5_0_staging_free_count(void) { return 0; }
int64_t ggml_backend_ameva_get_repacked_tensor_count(void) { return g_cnt.repacked_tensors; }
int64_t ggml_backend_ameva_get_repacked_bytes(void) { return g_cnt.repacked_bytes; }
int64_t ggml_backend_ameva_get_qmv_mul_mat_count(void) { return g_cnt.qmv; }
int64_t ggml_backend_ameva_get_mmq_mul_mat_count(void) { return g_cnt.mmq; }
int64_t ggml_backend_ameva_get_mmqb_mul_mat_count(void) { return 0; }
int64_t ggml_backend_ameva_get_fused_pair_count(void) { return g_cnt.fused; }
int64_t ggml_backend_ameva_get_act_quant_reuse_count(void) { return g_cnt.act_reuse; }
// the convolution / group-norm / windowed-node counters of the reference (ggml-ameva.h:70-78): this plugin runs none
// of those ops (it declines them in supports_op), so they stay 0 and the f16 convolution decoder is "not determined"
int64_t ggml_backend_ameva_get_conv_count(void) { return 0; }
int ggml_backend_ameva_get_conv_f16_decoder(void) { return -1; }
int64_t ggml_backend_ameva_get_conv_bias_count(void) { return 0; }
int64_t ggml_backend_ameva_get_group_norm_count(void) { return 0; }
int64_t ggml_backend_ameva_get_window_node_count(void) { return 0; }
const char* ggml_backend_ameva_get_build_commit(void) {
#ifdef AMEVA_BUILD_COMMIT
    return AMEVA_BUILD_COMMIT;
#else
    return "unknown";
#endif
}
void ggml_backend_ameva_reset_counters(void) {
    // stored state (repacked tensors and bytes) is not cleared, as in the reference
    g_cnt.supports_query = 0;
    g_cnt.supported_op = 0;
    g_cnt.gpu_op = 0;
    g_cnt.mul_mat = 0;
    g_cnt.qmv = 0;
    g_cnt.mmq = 0;
    g_cnt.fused = 0;
    g_cnt.act_reuse = 0;
}
void ggml_backend_ameva_profile_report(void) {
    std::lock_guard<std::mutex> pl(g_prof.mu);
    const double gr = g_prof.graphs ? (double)g_prof.graphs : 1.0;
    if (profile_level() >= 2) {
        std::vector<size_t> order(g_prof.kinds.size());
        double total = 0;
        for (size_t i = 0; i < order.size(); ++i) {
            order[i] = i;
            total += g_prof.kinds[i].second.ms;
        }
        std::sort(order.begin(), order.end(),
                  [](size_t a, size_t b) { return g_prof.kinds[a].second.ms > g_prof.kinds[b].second.ms; });
        for (size_t i : order) {
            const auto& k = g_prof.kinds[i];
            std::fprintf(stderr, "AMEVA_PROFILE kind=\"%s\" nodes=%lld gpu_ms=%.3f share=%.1f%% per_node_us=%.2f\n",
                         k.first.c_str(), (long long)k.second.n, k.second.ms, total > 0 ? 100.0 * k.second.ms / total : 0.0,
                         k.second.n ? 1e3 * k.second.ms / (double)k.second.n : 0.0);
        }
    }
    std::fprintf(stderr, "AMEVA_PROFILE graphs=%lld nodes=%lld encoded=%lld mul_mat=%lld mmq_mul_mat=%lld fused_pairs=%lld "
                         "act_quant_reuse=%lld\n",
                 (long long)g_prof.graphs, (long long)g_prof.nodes, (long long)g_prof.launches,
                 (long long)g_cnt.mul_mat.load(), (long long)g_cnt.mmq.load(), (long long)g_cnt.fused.load(),
                 (long long)g_cnt.act_reuse.load());
    std::fprintf(stderr, "AMEVA_PROFILE per_graph_ms encode=%.3f wait=%.3f gpu=%.3f (gpu samples %lld)\n",
                 g_prof.encode_ms / gr, g_prof.wait_ms / gr,
                 g_prof.gpu_samples ? g_prof.gpu_ms / (double)g_prof.gpu_samples : 0.0, (long long)g_prof.gpu_samples);
    std::fprintf(stderr, "AMEVA_PROFILE repacked_tensors=%lld repacked_mib=%.1f\n",
                 (long long)g_cnt.repacked_tensors.load(), (double)g_cnt.repacked_bytes.load() / 1048576.0);
}
void ggml_backend_ameva_set_failure_injection(AmevaFailureInjectionPoint p) { g_fail = (int)p; }
AmevaFailureInjectionPoint ggml_backend_ameva_get_failure_injection(void) { return (AmevaFailureInjectionPoint)g_fail.load(); }
const char* ggml_backend_ameva_op_unsupported_reason(const void* node) {
    return unsupported_reason((const ggml_tensor*)node);
}

}  // extern "C"
