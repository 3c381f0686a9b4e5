// libac_bitnet_hip.so -- the BitNet b1.58 per-token engine of the reference (adapters/bitnet/src/core/
// ac_bitnet_engine.cpp) on MI355X, over the kernel ABI of libameva_hip.so. The public API and its error rules follow the
// reference engine (Configure :135-193, UploadLayer :195-228, UploadOutput :230-251, EvalToken :383-426, LMHead
// :428-444); the token step follows RecordLayer :290-341 and the CPU arithmetic it mirrors (llama_bitnet_core.cpp:
// 1186-1265). On MI355X everything lives in HBM and the whole step is one HIP graph, captured at the first call (one
// with and one without the head) and replayed: the position, the key count and the RoPE table reach it through a
// pinned staging buffer copied at the start of the step.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ac_bitnet_engine_hip.h"
#include "../../include/ameva_hip.h"

namespace ameva {
namespace core {

namespace {

std::string step_text(const std::string& step, int result) {
    return "[ac_bitnet] " + step + " failed (AcResult " + std::to_string(result) + ")";
}

void hip_check(hipError_t e, const char* step) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw AcBitNetError(std::string(step) + ": " + hipGetErrorString(e),
                            e == hipErrorOutOfMemory ? (int)AC_ERR_OUT_OF_DEVICE_MEMORY : (int)AC_ERR_DRIVER_CRASH_OR_LOST);
    }
}

void amv_check(int r, const char* step) {
    if (r != 0) throw AcBitNetError(std::string(step) + ": " + amv_last_error(), (int)AC_ERR_KERNEL_ARG_INVALID);
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

}  // namespace

AcBitNetError::AcBitNetError(const std::string& step, int result)
    : std::runtime_error(step_text(step, result)), result_(result) {}

struct AcBitNetEngine::Impl {
    struct Layer {
        uint8_t* mem = nullptr;  // norms and the seven projections, 256-byte aligned pieces
        const float *attn_norm = nullptr, *attn_sub_norm = nullptr, *ffn_norm = nullptr, *ffn_sub_norm = nullptr;
        const uint8_t *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr, *wg = nullptr, *wu = nullptr,
                      *wd = nullptr;
        size_t off_attn_sub = 0, off_ffn_sub = 0;
        float s_q = 1, s_k = 1, s_v = 1, s_o = 1, s_g = 1, s_u = 1, s_d = 1;
        bool has_attn_sub = false, has_ffn_sub = false, uploaded = false;
        float *kc = nullptr, *vc = nullptr;
    };

    bool initialized = false, configured = false, profile = false;
    int device = 0;
    hipStream_t st = nullptr;
    std::string device_name;
    BitNetGpuConfig cfg;
    std::vector<Layer> layers;
    // scratch
    float *x = nullptr, *y = nullptr, *q = nullptr, *att = nullptr, *gate = nullptr, *up = nullptr, *cs = nullptr,
          *logits = nullptr, *out_norm = nullptr;
    int32_t* pos_dev = nullptr;  // [pos, n_kv]
    void* fa_ws = nullptr;
    int64_t fa_ws_bytes = 0;
    uint16_t* lm_head = nullptr;
    uint32_t n_vocab = 0;
    // pinned staging of what one step reads from the host: x (n_embd), the RoPE table (head_dim), pos and n_kv
    float* h_stage = nullptr;
    size_t stage_floats = 0;
    // [short context][0 layers, 1 layers + head]. At a context of at most kFoldKeys keys (4 key splits) the
    // attention's split merge runs inside the output projection's prologue (amv_bitnet_gemv_fa_merge, bit-identical
    // to the merge launch it replaces): one launch fewer per layer; the environment variable
    // AMV_BITNET_FOLD_MERGE=0 keeps the merge launch at every position.
    static constexpr uint32_t kFoldKeys = 256;
    hipGraphExec_t graph[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};
    bool fold_merge = true, short_ctx = false;
    void drop_graphs() {
        for (auto& gs : graph)
            for (auto& g : gs) {
                if (g) (void)hipGraphExecDestroy(g);
                g = nullptr;
            }
    }
    uint64_t weight_bytes = 0, lm_head_bytes = 0, kv_bytes = 0;
    std::vector<void*> allocs;

    void* dev_alloc(size_t bytes, const char* what) {
        void* p = nullptr;
        const hipError_t e = hipMalloc(&p, std::max<size_t>(bytes, 16));
        if (e != hipSuccess) {
            (void)hipGetLastError();
            throw AcBitNetError(std::string("hipMalloc ") + what + " (" + std::to_string(bytes) + " bytes)",
                                (int)AC_ERR_OUT_OF_DEVICE_MEMORY);
        }
        allocs.push_back(p);
        return p;
    }
    void upload(void* dst, const void* src, size_t bytes, const char* what) {
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st), what);
        hip_check(hipStreamSynchronize(st), what);
    }

    // One token step on the stream (capturable: kernel launches only). with_head: the final norm and the LM head.
    struct Timer {
        Impl* im;
        std::vector<std::pair<const char*, hipEvent_t>> marks;
        void mark(const char* name) {
            if (!im->profile) return;
            hipEvent_t e;
            hip_check(hipEventCreate(&e), "hipEventCreate");
            hip_check(hipEventRecord(e, im->st), "hipEventRecord");
            marks.push_back({name, e});
        }
    };

    void record_step(bool with_head, Timer* t) {
        const uint32_t E = cfg.n_embd, F = cfg.n_ffn, H = cfg.n_heads, KVH = cfg.n_kv_heads, hd = cfg.head_dim;
        const uint32_t kv = KVH * hd;
        const float inv_sqrt = 1.0f / std::sqrt((float)hd);  // multi_head_attention of the CPU path
        auto mark = [&](const char* n) {
            if (t) t->mark(n);
        };
        mark("start");
        const float eps = cfg.norm_eps;
        for (const Layer& L : layers) {
            // attn_norm + int8 -> Q | K | V -> RoPE -> k, v into the cache row of the position: one launch
            const void* w_qkv[3] = {L.wq, L.wk, L.wv};
            const int64_t r_qkv[3] = {(int64_t)H * hd, kv, kv};
            const float s_qkv[3] = {L.s_q, L.s_k, L.s_v};
            float* d_qkv[3] = {q, L.kc, L.vc};
            amv_check(amv_bitnet_gemv_fused(x, nullptr, L.attn_norm, E, eps, 0, 1, 3, w_qkv, r_qkv, s_qkv, d_qkv, 0, cs,
                                            pos_dev, cfg.n_ctx, st),
                      "attn_norm + q8 + attn_q/k/v + rope");
            mark("norm_qkv_rope");
            const int64_t r_e[1] = {E};
            float* d_x[1] = {x};
            if (short_ctx) {
                // the splits only; their merge + attn_sub_norm + int8 -> output projection added to x
                const int64_t nk = std::min<int64_t>(cfg.n_ctx, kFoldKeys);
                int32_t n_split = 0, split_len = 0;
                amv_check(amv_flash_attn_split_kv(0, q, L.kc, L.vc, nullptr, H, KVH, nk, pos_dev + 1, hd,
                                                  (int64_t)kv * 4, (int64_t)hd * 4, (int64_t)kv * 4, (int64_t)hd * 4,
                                                  inv_sqrt, fa_ws, fa_ws_bytes, 0, &n_split, &split_len, st),
                          "attention splits");
                mark("attention");
                amv_check(amv_bitnet_gemv_fa_merge((const float*)fa_ws, n_split, split_len, nk, pos_dev + 1,
                                                   L.attn_sub_norm, E, eps, L.has_attn_sub ? 1 : 0, L.wo, E, L.s_o, x,
                                                   1, st),
                          "attention merge + attn_sub_norm + q8 + attn_output + residual");
                mark("norm_o");
            } else {
                amv_check(amv_flash_attn_decode_kv(0, q, L.kc, L.vc, nullptr, att, H, KVH, cfg.n_ctx, pos_dev + 1, hd,
                                                   (int64_t)kv * 4, (int64_t)hd * 4, (int64_t)kv * 4, (int64_t)hd * 4,
                                                   inv_sqrt, fa_ws, fa_ws_bytes, nullptr, nullptr, 8, 0, st),
                          "attention");
                mark("attention");
                // attn_sub_norm (when present) + int8 -> output projection added to x
                const void* w_o[1] = {L.wo};
                const float s_o[1] = {L.s_o};
                amv_check(amv_bitnet_gemv_fused(att, nullptr, L.attn_sub_norm, E, eps, 0, L.has_attn_sub ? 1 : 0, 1,
                                                w_o, r_e, s_o, d_x, 1, nullptr, nullptr, 0, st),
                          "attn_sub_norm + q8 + attn_output + residual");
                mark("norm_o");
            }
            // ffn_norm + int8 -> gate | up
            const void* w_gu[2] = {L.wg, L.wu};
            const int64_t r_gu[2] = {F, F};
            const float s_gu[2] = {L.s_g, L.s_u};
            float* d_gu[2] = {gate, up};
            amv_check(amv_bitnet_gemv_fused(x, nullptr, L.ffn_norm, E, eps, 0, 1, 2, w_gu, r_gu, s_gu, d_gu, 0, nullptr,
                                            nullptr, 0, st),
                      "ffn_norm + q8 + ffn_gate/up");
            mark("norm_gate_up");
            // relu(gate)^2 * up or silu(gate) * up -> ffn_sub_norm (when present) + int8 -> down projection added to x
            const void* w_d[1] = {L.wd};
            const float s_d[1] = {L.s_d};
            amv_check(amv_bitnet_gemv_fused(gate, up, L.ffn_sub_norm, F, eps, cfg.relu2_ffn ? 1 : 2,
                                            L.has_ffn_sub ? 1 : 0, 1, w_d, r_e, s_d, d_x, 1, nullptr, nullptr, 0, st),
                      "ffn activation + ffn_sub_norm + q8 + ffn_down + residual");
            mark("act_norm_down");
        }
        if (with_head) {
            amv_check(amv_bitnet_norm_q8(x, nullptr, out_norm, E, cfg.norm_eps, 0, 1, y, nullptr, st), "output_norm");
            mark("norm_q8");
            amv_check(amv_gemv_f16(lm_head, n_vocab, E, y, logits, st), "lm_head");
            mark("gemv_f16");
        }
    }

    void stage_inputs(uint32_t pos, const float* x_in) {
        const uint32_t E = cfg.n_embd, hd = cfg.head_dim, half = hd / 2;
        // RoPE factors of this position, computed as apply_rope of the CPU path does (llama_bitnet_core.cpp:1011-1013)
        float* tab = h_stage + E;
        for (uint32_t i = 0; i < half; ++i) {
            const float theta = (float)pos / std::pow(cfg.rope_theta, (float)(2 * i) / (float)hd);
            tab[i] = std::cos(theta);
            tab[half + i] = std::sin(theta);
        }
        if (x_in) std::memcpy(h_stage, x_in, (size_t)E * 4);
        int32_t* pp = reinterpret_cast<int32_t*>(h_stage + E + hd);
        short_ctx = fold_merge && pos + 1 <= std::min<uint32_t>(cfg.n_ctx, kFoldKeys);
        pp[0] = (int32_t)pos;
        pp[1] = (int32_t)pos + 1;
        if (x_in) hip_check(hipMemcpyAsync(x, h_stage, (size_t)E * 4, hipMemcpyHostToDevice, st), "upload x");
        hip_check(hipMemcpyAsync(cs, tab, (size_t)hd * 4, hipMemcpyHostToDevice, st), "upload rope table");
        hip_check(hipMemcpyAsync(pos_dev, pp, 8, hipMemcpyHostToDevice, st), "upload position");
    }

    void run_step(bool with_head) {
        if (profile) {  // eager, with an event after every kernel group
            Timer t{this, {}};
            record_step(with_head, &t);
            hip_check(hipStreamSynchronize(st), "token step");
            double total = 0;
            std::vector<std::pair<std::string, double>> per;
            for (size_t i = 1; i < t.marks.size(); ++i) {
                float ms = 0;
                hip_check(hipEventElapsedTime(&ms, t.marks[i - 1].second, t.marks[i].second), "hipEventElapsedTime");
                total += ms;
                auto it = std::find_if(per.begin(), per.end(), [&](auto& p) { return p.first == t.marks[i].first; });
                if (it == per.end()) per.push_back({t.marks[i].first, ms});
                else it->second += ms;
            }
            fprintf(stderr, "[ac_bitnet] profile: GPU %.3f ms", total);
            for (auto& p : per) fprintf(stderr, " | %s %.3f ms", p.first.c_str(), p.second);
            fprintf(stderr, "\n");
            for (auto& m : t.marks) (void)hipEventDestroy(m.second);
            return;
        }
        hipGraphExec_t& g = graph[short_ctx ? 1 : 0][with_head ? 1 : 0];
        if (!g) {
            hipGraph_t gr = nullptr;
            hip_check(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            try {
                record_step(with_head, nullptr);
            } catch (...) {
                hipGraph_t dropped = nullptr;
                (void)hipStreamEndCapture(st, &dropped);
                if (dropped) (void)hipGraphDestroy(dropped);
                throw;
            }
            hip_check(hipStreamEndCapture(st, &gr), "hipStreamEndCapture");
            const hipError_t e = hipGraphInstantiate(&g, gr, nullptr, nullptr, 0);
            (void)hipGraphDestroy(gr);
            hip_check(e, "hipGraphInstantiate");
        }
        hip_check(hipGraphLaunch(g, st), "hipGraphLaunch");
    }

    void release() {
        if (st) (void)hipStreamSynchronize(st);
        drop_graphs();
        for (void* p : allocs) (void)hipFree(p);
        allocs.clear();
        if (h_stage) (void)hipHostFree(h_stage);
        h_stage = nullptr;
        if (st) (void)hipStreamDestroy(st);
        st = nullptr;
        layers.clear();
        configured = initialized = false;
    }
};

AcBitNetEngine::AcBitNetEngine() : impl_(new Impl) {}
AcBitNetEngine::~AcBitNetEngine() { impl_->release(); }

void AcBitNetEngine::Initialize() {
    Impl& m = *impl_;
    if (m.initialized) return;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        throw AcBitNetError("no HIP device", (int)AC_ERR_DRIVER_NOT_FOUND);
    }
    hip_check(hipGetDevice(&m.device), "hipGetDevice");
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, m.device), "hipGetDeviceProperties");
    m.device_name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    if (const char* e = getenv("AC_BITNET_GEMV")) {
        const std::string mode = *e ? e : "auto";
        if (mode != "auto" && mode != "dot" && mode != "emu")
            throw AcBitNetError("AC_BITNET_GEMV must be auto, dot or emu, got " + mode, (int)AC_ERR_INVALID_ARGUMENT);
    }
    if (const char* e = getenv("AC_BITNET_PROFILE")) {
        if (strcmp(e, "1") == 0) m.profile = true;
        else if (*e && strcmp(e, "0") != 0)
            throw AcBitNetError(std::string("AC_BITNET_PROFILE must be 0 or 1, got ") + e, (int)AC_ERR_INVALID_ARGUMENT);
    }
    if (const char* e = getenv("AMV_BITNET_FOLD_MERGE")) {
        if (strcmp(e, "0") == 0) m.fold_merge = false;
        else if (*e && strcmp(e, "1") != 0)
            throw AcBitNetError(std::string("AMV_BITNET_FOLD_MERGE must be 0 or 1, got ") + e,
                                (int)AC_ERR_INVALID_ARGUMENT);
    }
    hip_check(hipStreamCreateWithFlags(&m.st, hipStreamNonBlocking), "hipStreamCreate");
    fprintf(stderr, "[ac_bitnet] %s: i2_s GEMV through v_dot4 (exact integers), token step in one HIP graph\n",
            m.device_name.c_str());
    m.initialized = true;
}

void AcBitNetEngine::Configure(const BitNetGpuConfig& cfg) {
    Impl& m = *impl_;
    if (!m.initialized) throw AcBitNetError("Configure before Initialize", (int)AC_ERR_INVALID_ARGUMENT);
    if (m.configured) throw AcBitNetError("Configure called twice", (int)AC_ERR_INVALID_ARGUMENT);
    const bool shapes_ok = cfg.n_embd % 128 == 0 && cfg.n_ffn % 128 == 0 && cfg.n_layers > 0 && cfg.n_ctx > 0 &&
                           cfg.n_kv_heads > 0 && cfg.n_heads % cfg.n_kv_heads == 0 && cfg.head_dim % 2 == 0 &&
                           cfg.head_dim <= 256 && cfg.n_heads * cfg.head_dim == cfg.n_embd;
    if (!shapes_ok) {
        throw AcBitNetError("unsupported model shape (n_embd " + std::to_string(cfg.n_embd) + ", n_ffn " +
                                std::to_string(cfg.n_ffn) + ", heads " + std::to_string(cfg.n_heads) + "/" +
                                std::to_string(cfg.n_kv_heads) + ", head_dim " + std::to_string(cfg.head_dim) + ")",
                            (int)AC_ERR_INVALID_ARGUMENT);
    }
    const uint32_t G = cfg.n_heads / cfg.n_kv_heads;
    if (cfg.head_dim != 128 || (G != 1 && G != 2 && G != 4 && G != 8) || cfg.n_embd > 16384 || cfg.n_ffn > 16384 ||
        cfg.n_ctx > 128u * 1024u) {
        throw AcBitNetError("shape outside the MI355X kernels (head_dim 128, n_heads / n_kv_heads in {1, 2, 4, 8}, "
                            "n_embd and n_ffn <= 16384, n_ctx <= 131072)",
                            (int)AC_ERR_FEATURE_NOT_SUPPORTED);
    }
    m.cfg = cfg;
    const uint32_t E = cfg.n_embd, F = cfg.n_ffn, hd = cfg.head_dim, kv = cfg.n_kv_heads * hd, qd = cfg.n_heads * hd;
    const size_t erow = E / 4, frow = F / 4;
    m.layers.assign(cfg.n_layers, Impl::Layer());
    for (auto& L : m.layers) {
        size_t off = 0;
        auto take = [&](size_t bytes) {
            const size_t o = off;
            off = align_up(off + bytes);
            return o;
        };
        const size_t o_an = take(4ull * E), o_asn = take(4ull * E), o_fn = take(4ull * E), o_fsn = take(4ull * F);
        const size_t o_q = take(qd * erow), o_k = take(kv * erow), o_v = take(kv * erow), o_o = take(E * erow);
        const size_t o_g = take(F * erow), o_u = take(F * erow), o_d = take(E * frow);
        L.mem = (uint8_t*)m.dev_alloc(off, "layer weights");
        L.attn_norm = (const float*)(L.mem + o_an);
        L.off_attn_sub = o_asn;
        L.ffn_norm = (const float*)(L.mem + o_fn);
        L.off_ffn_sub = o_fsn;
        L.wq = L.mem + o_q;
        L.wk = L.mem + o_k;
        L.wv = L.mem + o_v;
        L.wo = L.mem + o_o;
        L.wg = L.mem + o_g;
        L.wu = L.mem + o_u;
        L.wd = L.mem + o_d;
        m.weight_bytes += off;
        const size_t kvb = 4ull * cfg.n_ctx * kv;
        L.kc = (float*)m.dev_alloc(kvb, "K cache");
        L.vc = (float*)m.dev_alloc(kvb, "V cache");
        hip_check(hipMemsetAsync(L.kc, 0, kvb, m.st), "clear K cache");
        hip_check(hipMemsetAsync(L.vc, 0, kvb, m.st), "clear V cache");
        m.kv_bytes += 2 * kvb;
    }
    m.x = (float*)m.dev_alloc(4ull * E, "x");
    m.y = (float*)m.dev_alloc(4ull * E, "x normalized");
    m.q = (float*)m.dev_alloc(4ull * qd, "q");
    m.att = (float*)m.dev_alloc(4ull * qd, "attention");
    m.gate = (float*)m.dev_alloc(4ull * F, "gate");
    m.up = (float*)m.dev_alloc(4ull * F, "up");
    m.cs = (float*)m.dev_alloc(4ull * hd, "rope table");
    m.pos_dev = (int32_t*)m.dev_alloc(8, "position");
    m.fa_ws_bytes = amv_flash_attn_workspace_bytes(cfg.n_heads, cfg.n_kv_heads, cfg.n_ctx, hd);
    if (m.fa_ws_bytes <= 0) throw AcBitNetError("attention workspace", (int)AC_ERR_INVALID_ARGUMENT);
    m.fa_ws = m.dev_alloc((size_t)m.fa_ws_bytes, "attention workspace");
    m.stage_floats = E + hd + 2;
    hip_check(hipHostMalloc((void**)&m.h_stage, m.stage_floats * 4, hipHostMallocDefault), "hipHostMalloc staging");
    hip_check(hipStreamSynchronize(m.st), "configure");
    m.configured = true;
}

void AcBitNetEngine::UploadLayer(uint32_t l, const BitNetGpuLayerHost& lay) {
    Impl& m = *impl_;
    if (!m.configured || l >= m.cfg.n_layers)
        throw AcBitNetError("UploadLayer: layer out of range", (int)AC_ERR_INVALID_ARGUMENT);
    if (!lay.attn_norm || !lay.ffn_norm || !lay.wq || !lay.wk || !lay.wv || !lay.wo || !lay.w_gate || !lay.w_up ||
        !lay.w_down) {
        throw AcBitNetError("layer " + std::to_string(l) + " lacks a norm or projection tensor the GPU chain needs",
                            (int)AC_ERR_INVALID_ARGUMENT);
    }
    const bool has_ffn_sub = lay.ffn_sub_norm != nullptr;
    if (has_ffn_sub != m.cfg.relu2_ffn) {
        throw AcBitNetError("layer " + std::to_string(l) + ": ffn_sub_norm presence differs from the model's FFN form",
                            (int)AC_ERR_INVALID_ARGUMENT);
    }
    Impl::Layer& L = m.layers[l];
    const uint32_t E = m.cfg.n_embd, F = m.cfg.n_ffn, kv = m.cfg.n_kv_heads * m.cfg.head_dim;
    const size_t erow = E / 4, frow = F / 4;
    m.upload((void*)L.attn_norm, lay.attn_norm, 4ull * E, "attn_norm");
    m.upload((void*)L.ffn_norm, lay.ffn_norm, 4ull * E, "ffn_norm");
    L.has_attn_sub = lay.attn_sub_norm != nullptr;
    L.has_ffn_sub = has_ffn_sub;
    L.attn_sub_norm = L.has_attn_sub ? (const float*)(L.mem + L.off_attn_sub) : nullptr;
    L.ffn_sub_norm = L.has_ffn_sub ? (const float*)(L.mem + L.off_ffn_sub) : nullptr;
    if (L.has_attn_sub) m.upload((void*)L.attn_sub_norm, lay.attn_sub_norm, 4ull * E, "attn_sub_norm");
    if (L.has_ffn_sub) m.upload((void*)L.ffn_sub_norm, lay.ffn_sub_norm, 4ull * F, "ffn_sub_norm");
    m.upload((void*)L.wq, lay.wq, (size_t)m.cfg.n_heads * m.cfg.head_dim * erow, "attn_q");
    m.upload((void*)L.wk, lay.wk, (size_t)kv * erow, "attn_k");
    m.upload((void*)L.wv, lay.wv, (size_t)kv * erow, "attn_v");
    m.upload((void*)L.wo, lay.wo, (size_t)E * erow, "attn_output");
    m.upload((void*)L.wg, lay.w_gate, (size_t)F * erow, "ffn_gate");
    m.upload((void*)L.wu, lay.w_up, (size_t)F * erow, "ffn_up");
    m.upload((void*)L.wd, lay.w_down, (size_t)E * frow, "ffn_down");
    L.s_q = lay.scale_wq;
    L.s_k = lay.scale_wk;
    L.s_v = lay.scale_wv;
    L.s_o = lay.scale_wo;
    L.s_g = lay.scale_w_gate;
    L.s_u = lay.scale_w_up;
    L.s_d = lay.scale_w_down;
    L.uploaded = true;
    // the captured steps hold the norm pointers of this layer: capture again
    m.drop_graphs();
}

void AcBitNetEngine::UploadOutput(const float* output_norm, const uint16_t* lm_head_f16, uint32_t n_vocab) {
    Impl& m = *impl_;
    if (!m.configured || !output_norm || !lm_head_f16 || n_vocab == 0 || m.cfg.n_embd % 8 != 0)
        throw AcBitNetError("UploadOutput: missing output norm or LM head", (int)AC_ERR_INVALID_ARGUMENT);
    if (m.lm_head) throw AcBitNetError("UploadOutput called twice", (int)AC_ERR_INVALID_ARGUMENT);
    const size_t bytes = 2ull * n_vocab * m.cfg.n_embd;
    m.out_norm = (float*)m.dev_alloc(4ull * m.cfg.n_embd, "output_norm");
    m.upload(m.out_norm, output_norm, 4ull * m.cfg.n_embd, "output_norm");
    m.lm_head = (uint16_t*)m.dev_alloc(bytes, "LM head");
    m.upload(m.lm_head, lm_head_f16, bytes, "LM head");
    m.logits = (float*)m.dev_alloc(4ull * n_vocab, "logits");
    m.n_vocab = n_vocab;
    m.lm_head_bytes = bytes;
}

void AcBitNetEngine::EvalToken(uint32_t pos, const float* x_in, float* x_out, float* logits, uint32_t chunk_layers) {
    (void)chunk_layers;  // no submission-length limit to bound on MI355X
    Impl& m = *impl_;
    if (!m.configured) throw AcBitNetError("EvalToken before Configure", (int)AC_ERR_INVALID_ARGUMENT);
    if (pos >= m.cfg.n_ctx) {
        throw AcBitNetError("position " + std::to_string(pos) + " outside the KV cache of " + std::to_string(m.cfg.n_ctx),
                            (int)AC_ERR_INVALID_ARGUMENT);
    }
    if (logits && !m.lm_head) throw AcBitNetError("logits requested without an LM head", (int)AC_ERR_INVALID_ARGUMENT);
    if (!x_in) throw AcBitNetError("EvalToken: x_in is NULL", (int)AC_ERR_NULL_POINTER);
    for (uint32_t l = 0; l < m.cfg.n_layers; ++l)
        if (!m.layers[l].uploaded)
            throw AcBitNetError("layer " + std::to_string(l) + " not uploaded", (int)AC_ERR_INVALID_ARGUMENT);
    m.stage_inputs(pos, x_in);
    m.run_step(logits != nullptr);
    if (x_out) hip_check(hipMemcpyAsync(x_out, m.x, 4ull * m.cfg.n_embd, hipMemcpyDeviceToHost, m.st), "read x");
    if (logits) hip_check(hipMemcpyAsync(logits, m.logits, 4ull * m.n_vocab, hipMemcpyDeviceToHost, m.st), "read logits");
    hip_check(hipStreamSynchronize(m.st), "token step");
}

void AcBitNetEngine::LMHead(const float* x_norm, float* logits) {
    Impl& m = *impl_;
    if (!m.lm_head) throw AcBitNetError("LMHead without an uploaded LM head", (int)AC_ERR_INVALID_ARGUMENT);
    if (!x_norm || !logits) throw AcBitNetError("LMHead: NULL argument", (int)AC_ERR_NULL_POINTER);
    m.upload(m.y, x_norm, 4ull * m.cfg.n_embd, "x_norm");
    amv_check(amv_gemv_f16(m.lm_head, m.n_vocab, m.cfg.n_embd, m.y, m.logits, m.st), "lm_head");
    hip_check(hipMemcpyAsync(logits, m.logits, 4ull * m.n_vocab, hipMemcpyDeviceToHost, m.st), "read logits");
    hip_check(hipStreamSynchronize(m.st), "LM head");
}

bool AcBitNetEngine::HasLMHead() const { return impl_->lm_head != nullptr; }
const std::string& AcBitNetEngine::DeviceName() const { return impl_->device_name; }
uint64_t AcBitNetEngine::WeightBytes() const { return impl_->weight_bytes; }
uint64_t AcBitNetEngine::LMHeadBytes() const { return impl_->lm_head_bytes; }
uint64_t AcBitNetEngine::KVCacheBytes() const { return impl_->kv_bytes; }

}  // namespace core
}  // namespace ameva

// ---------------------------------------------------------------------------------------------------------------
// C entry points
// ---------------------------------------------------------------------------------------------------------------
namespace {
struct CEngine {
    ameva::core::AcBitNetEngine e;
    std::string err;
};
thread_local std::string g_create_error;

template <typename F>
int guarded(void* h, F f) {
    CEngine* c = (CEngine*)h;
    if (!c) return (int)AC_ERR_NULL_POINTER;
    try {
        f(c->e);
        c->err.clear();
        return (int)AC_SUCCESS;
    } catch (const ameva::core::AcBitNetError& x) {
        c->err = x.what();
        return x.result();
    } catch (const std::exception& x) {
        c->err = x.what();
        return (int)AC_ERR_OUT_OF_HOST_MEMORY;
    }
}
}  // namespace

extern "C" void* ac_bitnet_engine_create(void) {
    CEngine* c = nullptr;
    try {
        c = new CEngine;
        c->e.Initialize();
        g_create_error.clear();
        return c;
    } catch (const std::exception& x) {
        g_create_error = x.what();
        delete c;
        return nullptr;
    }
}

extern "C" int ac_bitnet_engine_configure(void* h, const AcBitNetConfigC* cfg) {
    if (!cfg) return (int)AC_ERR_NULL_POINTER;
    return guarded(h, [&](ameva::core::AcBitNetEngine& e) {
        ameva::core::BitNetGpuConfig c;
        c.n_embd = cfg->n_embd;
        c.n_ffn = cfg->n_ffn;
        c.n_heads = cfg->n_heads;
        c.n_kv_heads = cfg->n_kv_heads;
        c.head_dim = cfg->head_dim;
        c.n_ctx = cfg->n_ctx;
        c.n_layers = cfg->n_layers;
        c.norm_eps = cfg->norm_eps;
        c.rope_theta = cfg->rope_theta;
        c.relu2_ffn = cfg->relu2_ffn != 0;
        e.Configure(c);
    });
}

extern "C" int ac_bitnet_engine_upload_layer(void* h, uint32_t layer, const AcBitNetLayerC* lay) {
    if (!lay) return (int)AC_ERR_NULL_POINTER;
    return guarded(h, [&](ameva::core::AcBitNetEngine& e) {
        ameva::core::BitNetGpuLayerHost L;
        L.attn_norm = lay->attn_norm;
        L.attn_sub_norm = lay->attn_sub_norm;
        L.ffn_norm = lay->ffn_norm;
        L.ffn_sub_norm = lay->ffn_sub_norm;
        L.wq = lay->wq;
        L.wk = lay->wk;
        L.wv = lay->wv;
        L.wo = lay->wo;
        L.w_gate = lay->w_gate;
        L.w_up = lay->w_up;
        L.w_down = lay->w_down;
        L.scale_wq = lay->scale_wq;
        L.scale_wk = lay->scale_wk;
        L.scale_wv = lay->scale_wv;
        L.scale_wo = lay->scale_wo;
        L.scale_w_gate = lay->scale_w_gate;
        L.scale_w_up = lay->scale_w_up;
        L.scale_w_down = lay->scale_w_down;
        e.UploadLayer(layer, L);
    });
}

extern "C" int ac_bitnet_engine_upload_output(void* h, const float* output_norm, const uint16_t* lm_head_f16,
                                              uint32_t n_vocab) {
    return guarded(h, [&](ameva::core::AcBitNetEngine& e) { e.UploadOutput(output_norm, lm_head_f16, n_vocab); });
}

extern "C" int ac_bitnet_engine_eval_token(void* h, uint32_t pos, const float* x_in, float* x_out, float* logits,
                                           uint32_t chunk_layers) {
    return guarded(h, [&](ameva::core::AcBitNetEngine& e) { e.EvalToken(pos, x_in, x_out, logits, chunk_layers); });
}

extern "C" int ac_bitnet_engine_lm_head(void* h, const float* x_norm, float* logits) {
    return guarded(h, [&](ameva::core::AcBitNetEngine& e) { e.LMHead(x_norm, logits); });
}

extern "C" const char* ac_bitnet_engine_last_error(void* h) {
    return h ? ((CEngine*)h)->err.c_str() : g_create_error.c_str();
}

extern "C" void ac_bitnet_engine_destroy(void* h) { delete (CEngine*)h; }
