/*
 * ac_bitnet_engine_hip.h -- the BitNet b1.58 per-token GPU engine of the reference on MI355X (libac_bitnet_hip.so).
 *
 * Drop-in for adapters/bitnet/src/core/ac_bitnet_engine.h: the same C++ API (namespace ameva::core, AcBitNetError,
 * BitNetGpuConfig, BitNetGpuLayerHost, AcBitNetEngine with Initialize / Configure / UploadLayer / UploadOutput /
 * EvalToken / LMHead and the getters), so llama_bitnet_core.cpp's calls (:600-666, :1167, :1265) keep their code.
 * Every failure throws AcBitNetError naming the step and an AcResult (include/ac_runtime_hip.h); there is no CPU
 * fallback. Semantics of the token step, per layer, as the reference engine and the CPU path it follows
 * (llama_bitnet_core.cpp:1186-1265): RMS_NORM(x, attn_norm) -> int8 (quantize_activation_int8) -> the Q, K, V I2_S
 * projections -> RoPE of q and k (cos / sin of pos / theta^(2i/d) computed on the host as apply_rope does) -> k, v
 * into the f32 cache row of pos -> attention over positions 0 .. pos -> RMS_NORM(attention, attn_sub_norm) when
 * present -> int8 -> output projection added to x -> RMS_NORM(x, ffn_norm) -> int8 -> gate, up -> relu(gate)^2 * up
 * (relu2_ffn) or silu(gate) * up -> RMS_NORM(., ffn_sub_norm) when present -> int8 -> down projection added to x;
 * then, when logits are asked for, RMS_NORM(x, output_norm) and the f16 LM head.
 *
 * On MI355X: all state lives in HBM; each layer is 6 launches (each norm + int8 step runs inside the projection that
 * consumes it, Q|K|V and gate|up are one launch each, RoPE and the cache stores ride in the Q|K|V epilogue); the
 * token step (every layer, and the head) is one HIP graph captured at the first call and replayed, the position and
 * key count being read from device memory; chunk_layers is accepted and
 * has no effect (there is no submission-length limit to bound). Shapes: head_dim 128, n_heads / n_kv_heads in
 * {1, 2, 4, 8}, n_embd and n_ffn multiples of 128 up to 16384 (BitNet b1.58 2B: 2560 / 6912, 20 / 5 heads).
 * AC_BITNET_PROFILE=1 runs the step eagerly and prints the GPU time per kernel to stderr; AC_BITNET_GEMV must be
 * auto, dot or emu as in the reference (every value takes the v_dot4 integer path, which is exact).
 */
#ifndef AC_BITNET_ENGINE_HIP_H
#define AC_BITNET_ENGINE_HIP_H

#include <stdint.h>

#include "ac_runtime_hip.h"

#ifdef __cplusplus
#include <memory>
#include <stdexcept>
#include <string>

namespace ameva {
namespace core {

class AcBitNetError : public std::runtime_error {
public:
    AcBitNetError(const std::string& step, int result);
    int result() const { return result_; }

private:
    int result_;
};

struct BitNetGpuConfig {
    uint32_t n_embd = 0;
    uint32_t n_ffn = 0;
    uint32_t n_heads = 0;
    uint32_t n_kv_heads = 0;
    uint32_t head_dim = 0;
    uint32_t n_ctx = 0;
    uint32_t n_layers = 0;
    float norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
    bool relu2_ffn = false;
};

struct BitNetGpuLayerHost {
    const float* attn_norm = nullptr;
    const float* attn_sub_norm = nullptr;
    const float* ffn_norm = nullptr;
    const float* ffn_sub_norm = nullptr;
    const void* wq = nullptr;
    const void* wk = nullptr;
    const void* wv = nullptr;
    const void* wo = nullptr;
    const void* w_gate = nullptr;
    const void* w_up = nullptr;
    const void* w_down = nullptr;
    float scale_wq = 1.0f, scale_wk = 1.0f, scale_wv = 1.0f, scale_wo = 1.0f;
    float scale_w_gate = 1.0f, scale_w_up = 1.0f, scale_w_down = 1.0f;
};

class AcBitNetEngine {
public:
    AcBitNetEngine();
    ~AcBitNetEngine();
    AcBitNetEngine(const AcBitNetEngine&) = delete;
    AcBitNetEngine& operator=(const AcBitNetEngine&) = delete;

    void Initialize();
    void Configure(const BitNetGpuConfig& cfg);
    void UploadLayer(uint32_t l, const BitNetGpuLayerHost& lay);
    void UploadOutput(const float* output_norm, const uint16_t* lm_head_f16, uint32_t n_vocab);
    void EvalToken(uint32_t pos, const float* x_in, float* x_out, float* logits, uint32_t chunk_layers);
    void LMHead(const float* x_norm, float* logits);

    bool HasLMHead() const;
    const std::string& DeviceName() const;
    uint64_t WeightBytes() const;
    uint64_t LMHeadBytes() const;
    uint64_t KVCacheBytes() const;

    struct Impl;

private:
    std::unique_ptr<Impl> impl_;
};

}  // namespace core
}  // namespace ameva

extern "C" {
#endif

/* C entry points of the same engine (this library's addition, for hosts without C++: Python, tests). Each returns
 * AC_SUCCESS or the AcResult of the failure, whose text ac_bitnet_engine_last_error gives. */
typedef struct {
    uint32_t n_embd, n_ffn, n_heads, n_kv_heads, head_dim, n_ctx, n_layers;
    float norm_eps, rope_theta;
    int32_t relu2_ffn;
} AcBitNetConfigC;

typedef struct {
    const float *attn_norm, *attn_sub_norm, *ffn_norm, *ffn_sub_norm;
    const void *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    float scale_wq, scale_wk, scale_wv, scale_wo, scale_w_gate, scale_w_up, scale_w_down;
} AcBitNetLayerC;

void* ac_bitnet_engine_create(void); /* Initialize()d engine, or NULL (see ac_bitnet_engine_last_error(NULL)) */
int ac_bitnet_engine_configure(void* engine, const AcBitNetConfigC* cfg);
int ac_bitnet_engine_upload_layer(void* engine, uint32_t layer, const AcBitNetLayerC* lay);
int ac_bitnet_engine_upload_output(void* engine, const float* output_norm, const uint16_t* lm_head_f16,
                                   uint32_t n_vocab);
int ac_bitnet_engine_eval_token(void* engine, uint32_t pos, const float* x_in, float* x_out, float* logits,
                                uint32_t chunk_layers);
int ac_bitnet_engine_lm_head(void* engine, const float* x_norm, float* logits);
const char* ac_bitnet_engine_last_error(void* engine);
void ac_bitnet_engine_destroy(void* engine);

#ifdef __cplusplus
}
#endif

#endif /* AC_BITNET_ENGINE_HIP_H */
