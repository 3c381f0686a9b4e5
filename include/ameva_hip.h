/*
 * ameva MI355X (gfx950) kernel ABI: the thin C layer between C++/Python host code and the hand-written HIP kernels
 * of the quantized ggml hot path. Plain pointers and sizes only; every device pointer is a HIP device address, every
 * `stream` a hipStream_t (NULL = the default stream). All calls are asynchronous on `stream` and return AMV_OK or a
 * negative status; amv_last_error() then holds a message. Nothing here falls back to the CPU.
 *
 * Types are ggml_type values (reference include/ggml/ggml.h:394-437): 2 Q4_0, 8 Q8_0, 12 Q4_K, 14 Q6_K, 15 Q8_K,
 * 36 I2_S. "ggml blocks" means ggml's own byte layout (reference shaders/ameva_qmm.comp:22-36). Each entry point
 * names the reference interface it replaces.
 */
#ifndef AMEVA_HIP_H
#define AMEVA_HIP_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AMV_OK 0
#define AMV_ERR_INVALID_ARG (-1)
#define AMV_ERR_UNSUPPORTED (-2)
#define AMV_ERR_HIP (-3)

/* Q8_0 activation rounding rules (the reference documents three; ameva_act_fq.comp:5 names the x86 one):
 *   AMV_Q8_X86: d = amax/127, q = round-half-even(x * (127/amax))   -- ggml-cpu x86 quantize_row_q8_0 (default)
 *   AMV_Q8_ARM: d = amax/127, q = round-half-even(x * (1/d))        -- ggml-cpu ARM (ameva_quant_a8.comp:5)
 *   AMV_Q8_REF: d = amax/127, q = roundf(x * (1/d))                  -- quantize_row_q8_0_ref (weights, KV cache) */
#define AMV_Q8_X86 0
#define AMV_Q8_ARM 1
#define AMV_Q8_REF 2

/* Message of the last failing call on this thread ("" when none). */
const char* amv_last_error(void);
/* ABI version, major * 100 + minor. */
int amv_version(void);

/* ------------------------------------------------------------------------------------------------------------
 * Weight layout. Replaces the reference's repacked WEIGHTS-buffer format and its conversions
 * (adapters/llama/ggml-ameva/ggml-ameva-repack.h:1-69, ggml-ameva-repack.cpp:21-351, set_tensor/get_tensor at
 * ggml-ameva-buffer.cpp:509-561). The MI355X layout is structure-of-arrays per tensor of n_rows x k weights, row
 * major within each region, every region but the last starting 16-byte aligned:
 *   Q4_0: qs[n_rows][k/32][16] | d f16[n_rows][k/32]
 *   Q8_0: qs[n_rows][k/32][32] | d f16[n_rows][k/32]
 *   Q4_K: qs[n_rows][k/256][128] | head[n_rows][k/256][16] (d, dmin, scales[12])
 *   Q6_K: ql[n_rows][k/256][128] | qh[..][64] | scales[..][16] | d f16[..]
 * The size equals ggml_nbytes of the tensor and amv_unrepack(amv_repack(x)) == x byte for byte.
 * ---------------------------------------------------------------------------------------------------------- */
int64_t amv_weight_bytes(int type, int64_t n_rows, int64_t k);
int amv_repack(int type, const void* src_ggml, void* dst, int64_t n_rows, int64_t k, void* stream);
int amv_unrepack(int type, const void* src, void* dst_ggml, int64_t n_rows, int64_t k, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * Activation quantization. Replaces ameva_quant_a8.comp:32-78 / ameva_quant_a8b.comp (the dispatch recorded by
 * enc_mul_mat_mmvq, ggml-ameva.cpp:2738-2749) and ggml's quantize_row_q8_0 / quantize_row_q8_K_ref (vec_dot_type).
 * x f32 [m][k] (row stride k). Outputs (either may be NULL):
 *   y_ggml: ggml blocks, block_q8_0 (34 B: fp16 d, int8 qs[32]) or block_q8_K (292 B: f32 d, qs[256], i16 bsums[16])
 *   y_act:  the kernels' activation layout, amv_act_bytes(type, m, k) bytes:
 *           Q8_0: qs int8[m][k] | {f32 d (fp16-rounded, as ggml uses it), i32 sum(qs)}[m][k/32]
 *           Q8_K: qs int8[m][k] | f32 d[m][k/256] | i32 sum(qs)[m][k/16]
 * type AMV_T Q8_0 (8) or Q8_K (15); rule applies to Q8_0 only.
 * ---------------------------------------------------------------------------------------------------------- */
int64_t amv_act_bytes(int type, int64_t m, int64_t k);
int amv_quantize_act(int type, const float* x, int64_t m, int64_t k, int rule, void* y_ggml, void* y_act,
                     void* stream);

/* Row quantization to ggml blocks on the GPU (the quantizing row store of ameva_set_rows_q.comp:95-115, ggml
 * quantize_row_q4_0_ref; used for the KV cache and to quantize synthetic weights). x f32 [n_rows][k]. */
int amv_quantize_q4_0(const float* x, int64_t n_rows, int64_t k, void* y_ggml, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * MUL_MAT, quantized weights x quantized activations (ggml: dst = src0^T x src1).
 * Replaces enc_mul_mat / enc_mul_mat_mmvq (ggml-ameva.cpp:3607-3804, 2704-2785) with ameva_mmvq.comp /
 * ameva_qmv.comp (bs1 decode GEMV) and the CPU's ggml_vec_dot_<wtype>_q8_<x>.
 *   w:   repacked weight (amv_repack layout) of n_rows x k
 *   act: amv_quantize_act y_act of m rows x k (Q8_0 for Q4_0/Q8_0 weights, Q8_K for Q4_K/Q6_K)
 *   dst: f32, element (row n, column c) at dst[c * ldd + n]; ldd >= n_rows
 * ---------------------------------------------------------------------------------------------------------- */
int amv_mul_mat_vec(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
                    int64_t ldd, void* stream);

/* Parity instrumentation of the same kernels: the exact integer sums per weight block, int32
 * [m][n_rows][nblk * per] with nblk = k / block size, per = 2 for Q4_K (sum sc*dot, sum m*bsum) and 1 otherwise.
 * These are the per-block int32 sums of ggml's vec_dot (bit-exact contract). */
int amv_mul_mat_block_sums(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                           int32_t* sums, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AMEVA_HIP_H */
