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
#define AMV_ACT_Q8_K_MMA 1015 /* Q8_K activations with the f16 copies the batched K-quant MUL_MAT reads */
#define AMV_ACT_Q8_0_MMA 1008 /* Q8_0 activations with the f16 copies the batched Q4_0 / Q8_0 MUL_MAT reads */
#define AMV_ACT_Q8_K_DEQ 1115 /* AMV_ACT_Q8_K_MMA's layout with f16 q * d in place of f16 q (the scaled batched form) */
#define AMV_ACT_Q8_0_DEQ 1108 /* AMV_ACT_Q8_0_MMA's layout with f16 q * d in place of f16 q (the scaled batched form) */
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
 *   Q4_0: qs[n_rows][k/32][16] | d f16[n_rows/2][k/32][2] (the scales of rows 2p and 2p + 1 side by side, one dword
 *         per block pair; an odd last row follows as d f16[k/32])
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
 *           AMV_ACT_Q8_K_MMA: the Q8_K layout, then (16-byte aligned) the same values as f16 [m][k] (exact), the
 *           sums per 16 as f16 [m][k/16] and (16-byte aligned) the super-block scales transposed, f32 [k/256][m]:
 *           the batched Q4_K MUL_MAT of 8..64 tokens reads the f16 copies; its Q8_K prefix is a plain Q8_K
 *           activation of the m rows (amv_mul_mat_vec and the larger batches read it as such).
 *           AMV_ACT_Q8_0_MMA: the Q8_0 layout, then (16-byte aligned) the same values as f16 [m][k] and the block
 *           scales transposed, f32 [k/32][m]; its prefix is a plain Q8_0 activation of the m rows, which is what
 *           the batched Q4_0 / Q8_0 MUL_MAT reads.
 *           AMV_ACT_Q8_0_DEQ / AMV_ACT_Q8_K_DEQ: the same layouts (and sizes) with f16 of q * d (one rounding) in
 *           place of the f16 copies of q: the input of the scaled batched MUL_MAT.
 * type AMV_T Q8_0 (8), Q8_K (15), AMV_ACT_Q8_K_MMA, AMV_ACT_Q8_0_MMA, AMV_ACT_Q8_K_DEQ or AMV_ACT_Q8_0_DEQ; rule
 * applies to the Q8_0 forms only.
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
/* MUL_MAT of m (1..8) activation columns on Q4_0 / Q8_0 weights still in ggml's block layout, read in place: the
 * reference's raw-layout path (ameva_qmm.comp:315-372, reached from enc_mul_mat for a quantized src0 outside a WEIGHTS
 * buffer, ggml-ameva.cpp:3607-3804). Row r of the weight starts at w + r * row_bytes (a row view keeps its parent's
 * stride); k % 64 == 0, w and row_bytes dword-aligned. act: the plain Q8_0 activation of amv_quantize_act (m rows of
 * k). dst[c * ldd + r] as amv_mul_mat_vec; with sums != NULL the exact block integers sums[(c * n_rows + r) * k/32 + b]
 * are written instead (dst may then be NULL). */
int amv_mul_mat_vec_raw(int wtype, const void* w, int64_t row_bytes, int64_t n_rows, int64_t k, const void* act,
                        int64_t m, float* dst, int64_t ldd, int32_t* sums, void* stream);
/* Parity instrumentation (no counterpart in the reference; for tests): while on != 0, the Q4_0 GEMV launches of this
 * process skip the dedicated K = 4096 kernels and run the generic one-column kernel of the same rows per wave, split
 * and epilogue, whose block-sum instantiation is the one amv_mul_mat_block_sums reads; the dedicated kernels keep
 * that kernel's arithmetic and summation order, so a test compares their f32 results bit for bit. Returns the
 * previous setting. Not for production calls: the generic kernels are slower. */
int amv_debug_gemv_generic(int on);
/* Measurement instrumentation (no counterpart in the reference; for bench.py and profiles): the headline kernel's grid,
 * row mapping and weight / scale loads for a Q4_0 weight of n_rows x 4096 (n_rows even), without the activation and
 * the arithmetic; dst gets one XOR fold of the weight words per row. Its time is the read ceiling of that mapping.
 * loads = 0 launches the same grid without the loads (dst[r] = r): the fixed cost of launching and draining it. w
 * needs n_rows x 2304 readable bytes; its contents do not matter. */
int amv_debug_gemv_read_probe(const void* w, int64_t n_rows, int64_t k, uint32_t* dst, int loads, void* stream);

/* One-column GEMV with the fused epilogue of the next graph node: the reference's ameva_qmv / ameva_mmvq ep_mode
 * (ameva_qmv.comp:233-246) chosen by ameva_find_fusion (ggml-ameva.cpp:4280-4285, 4355-4375). v[n] is the dot
 * product of row n, e the epilogue operand (f32 [n_rows]), eout the epilogue output; dst[n] = v[n] is written as
 * well when dst is not NULL (the MUL_MAT node's own value, the reference's write-through).
 *   AMV_EP_NONE:     dst[n] = v[n]                                     (dst required)
 *   AMV_EP_ADD:      eout[n] = v[n] + e[n]                             (MUL_MAT -> ADD: bias, residual)
 *   AMV_EP_SILU_MUL: eout[n] = v[n] / (1 + exp(-v[n])) * e[n]          (MUL_MAT -> SWIGLU, as its gate operand)
 *   AMV_EP_MUL_SILU: eout[n] = e[n] / (1 + exp(-e[n])) * v[n]          (MUL_MAT -> SWIGLU, as its up operand)
 *   AMV_EP_SWIGLU_STACKED (no counterpart in the reference): w holds the F gate rows then the F up rows
 *     (n_rows = 2 F) and eout[i] = silu(v[i]) * v[F + i] for i < F, e unused; dst, when given, gets all 2 F values.
 * eout must not overlap act, w or e. */
#define AMV_EP_NONE 0
#define AMV_EP_ADD 1
#define AMV_EP_SILU_MUL 2
#define AMV_EP_MUL_SILU 3
#define AMV_EP_SWIGLU_STACKED 4
int amv_mul_mat_vec_ep(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* dst, int ep_mode,
                       const float* e, float* eout, void* stream);

/* Decode GEMVs that carry the next small op of a Llama layer in the same launch (no counterpart kernel in the
 * reference, whose graph runs these ops as separate nodes; each saves one ~4 us launch at bs1). One activation
 * column (Q8_0 / Q8_K layout of amv_quantize_act), results identical to the unfused sequence.
 * counters: device uint32 array, zero before the first call, left at zero by every call (self-resetting arrival
 * counters, one per 128-byte line; calls that share one array must not run concurrently). Sizes in words:
 * amv_gemv_add_rms_norm AMV_ADD_NORM_COUNTER_WORDS(n_rows), amv_gemv_swiglu_q8 AMV_SWIGLU_COUNTER_WORDS(n_rows). */
#define AMV_ADD_NORM_COUNTER_WORDS(n_rows) (32 * ((n_rows) / 32 + 2))
#define AMV_SWIGLU_COUNTER_WORDS(n_rows) (32 * ((n_rows) / 64 + 1))
/*
 *
 * amv_gemv_rope_kv: w stacks n_head * D q rows, n_head_kv * D k rows, n_head_kv * D v rows (n_rows = their sum);
 * qkv f32 [n_rows] gets q and k rotated by ROPE NORMAL (n_dims = D; amv_rope's arithmetic, positions from pos[0])
 * and v as computed; k and v also go as f16 to row kv_idx[0] of the caches (amv_rope_kv_store's layout and skip
 * rule: a row outside [0, cache_rows) is not stored and each skipped head adds 1 to *bad when bad is not NULL).
 * = MUL_MAT + ROPE + ROPE + SET_ROWS + SET_ROWS. */
int amv_gemv_rope_kv(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* qkv,
                     int64_t n_head, int64_t n_head_kv, int64_t D, const int32_t* pos, float freq_base,
                     float freq_scale, float attn_factor, void* k_cache, void* v_cache, int64_t cache_row,
                     const int64_t* kv_idx, int64_t cache_rows, unsigned int* bad, void* stream);
/* amv_gemv_add_rms_norm: eout = W act + e (dst = W act too when not NULL), then amv_rms_norm of eout (one row of
 * n_rows) into norm_y / norm_o / act_out (any may be NULL; act_out is the activation row of act_type 8 = Q8_0, with
 * `rule`, or 15 = Q8_K), done by the last workgroup of the launch.
 * = MUL_MAT + ADD + RMS_NORM + MUL (+ the next activation quantization). */
int amv_gemv_add_rms_norm(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* dst,
                          const float* e, float* eout, float eps, const float* norm_w, float* norm_y, float* norm_o,
                          void* act_out, int act_type, int rule, unsigned int* counters, void* stream);
/* amv_gemv_swiglu_q8: AMV_EP_SWIGLU_STACKED (w = F gate rows then F up rows; eout [F]) and the activation row of
 * eout into act_out (act_type 8 = Q8_0 with `rule`, F % 32 == 0; 15 = Q8_K, F % 256 == 0), each block quantized by
 * the last workgroup producing it. = MUL_MAT x 2 + SWIGLU + the next quantization. */
int amv_gemv_swiglu_q8(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* dst, float* eout,
                       void* act_out, int act_type, int rule, unsigned int* counters, void* stream);
/* The same two fused GEMVs over separate weights (no counterpart in the reference; for the ggml plugin, whose q, k,
 * v and gate, up weights are separate ggml tensors, each in its own repacked layout): Q4_0 (k % 4096 == 0) or Q4_K,
 * every matrix with an even row count. amv_gemv_rope_kv_seg: wq / wk / wv with n_head * D, n_head_kv * D and
 * n_head_kv * D rows; the rotated q and k and the v values go to q_out / k_out / v_out (the cache rows as in
 * amv_gemv_rope_kv). amv_gemv_swiglu_q8_seg: w_gate and w_up of F rows each (counters as amv_gemv_swiglu_q8 with
 * n_rows = 2 F); no dst. Results are those of the stacked calls over the concatenated rows, bit for bit. */
int amv_gemv_rope_kv_seg(int wtype, const void* wq, const void* wk, const void* wv, int64_t k, const void* act,
                         float* q_out, float* k_out, float* v_out, int64_t n_head, int64_t n_head_kv, int64_t D,
                         const int32_t* pos, float freq_base, float freq_scale, float attn_factor, void* k_cache,
                         void* v_cache, int64_t cache_row, const int64_t* kv_idx, int64_t cache_rows,
                         unsigned int* bad, void* stream);
int amv_gemv_swiglu_q8_seg(int wtype, const void* w_gate, const void* w_up, int64_t F, int64_t k, const void* act,
                           float* eout, void* act_out, int act_type, int rule, unsigned int* counters, void* stream);

/* The RMS_NORM node before a decode GEMV folded into it (the reference runs RMS_NORM + MUL and the MUL_MAT as graph
 * nodes, ggml-ameva.cpp:3607-3804 / ameva_rms_norm.comp:39-91; no single counterpart): the GEMV takes the f32 row x
 * (4096 values), RMS_NORM(x, eps) * norm_w and its Q8_0 quantization with `rule` are computed inside (amv_rms_norm_act's
 * arithmetic, the same bytes), and the rest is amv_gemv_rope_kv / amv_gemv_swiglu_q8 over that activation, bit for
 * bit. Q4_0 weights (Q8_0 activations with `rule`; act_out Q8_0) or Q4_K weights (Q8_K; act_out Q8_K) of k = 4096,
 * even row counts; x and norm_w 16-byte aligned. No activation buffer is written for the norm. */
int amv_rms_norm_gemv_rope_kv(const float* x, const float* norm_w, float eps, int rule, int wtype, const void* w,
                              int64_t n_rows, int64_t k, float* qkv, int64_t n_head, int64_t n_head_kv, int64_t D,
                              const int32_t* pos, float freq_base, float freq_scale, float attn_factor, void* k_cache,
                              void* v_cache, int64_t cache_row, const int64_t* kv_idx, int64_t cache_rows,
                              unsigned int* bad, void* stream);
int amv_rms_norm_gemv_swiglu_q8(const float* x, const float* norm_w, float eps, int rule, int wtype, const void* w,
                                int64_t n_rows, int64_t k, float* dst, float* eout, void* act_out,
                                unsigned int* counters, void* stream);
/* The same over separate matrices (llama.cpp's q, k, v and gate, up tensors; the segment rules of
 * amv_gemv_rope_kv_seg / amv_gemv_swiglu_q8_seg), bit for bit the stacked calls. */
int amv_rms_norm_gemv_rope_kv_seg(const float* x, const float* norm_w, float eps, int rule, int wtype, const void* wq,
                                  const void* wk, const void* wv, int64_t k, float* q_out, float* k_out, float* v_out,
                                  int64_t n_head, int64_t n_head_kv, int64_t D, const int32_t* pos, float freq_base,
                                  float freq_scale, float attn_factor, void* k_cache, void* v_cache, int64_t cache_row,
                                  const int64_t* kv_idx, int64_t cache_rows, unsigned int* bad, void* stream);
int amv_rms_norm_gemv_swiglu_q8_seg(const float* x, const float* norm_w, float eps, int rule, int wtype,
                                    const void* w_gate, const void* w_up, int64_t F, int64_t k, float* eout,
                                    void* act_out, unsigned int* counters, void* stream);
/* Measurement instrumentation (no counterpart in the reference): threads per workgroup of the folded-norm GEMVs
 * (256, 512 or 1024; a negative value -NT: the gate/up launches with four outputs per wave; 0 = the default). */
void amv_debug_norm_gemv_threads(int nt);

/* Parity instrumentation of the same kernels: the exact integer sums per weight block, int32
 * [m][n_rows][nblk * per] with nblk = k / block size, per = 2 for Q4_K (sum sc*dot, sum m*bsum) and 1 otherwise.
 * These are the per-block int32 sums of ggml's vec_dot (bit-exact contract). */
int amv_mul_mat_block_sums(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                           int32_t* sums, void* stream);

/* Prefill MUL_MAT with int8 MFMA (enc_mul_mat_mmq ggml-ameva.cpp:2540-2647, ameva_mmq.comp): same operands and
 * result as amv_mul_mat_vec (plain Q8_0 activations for Q4_0 / Q8_0, plain Q8_K for Q4_K / Q6_K) and many activation
 * columns (the reference switches at M >= AMEVA_QGEMM_MIN_M = 8, ggml-ameva.cpp:2486-2505). The _block_sums form
 * writes the MFMA's exact per-block integers, int32 [m][n_rows][k/32] (Q4_K: [..][k/256][2]), for the bit-exact
 * check. */
int amv_mul_mat_q(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
                  int64_t ldd, void* stream);
int amv_mul_mat_q_block_sums(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                             int32_t* sums, void* stream);
/* amv_mul_mat_q with the activation layout named: act_type AMV_T_Q8_0, AMV_ACT_Q8_0_MMA or AMV_ACT_Q8_0_DEQ for
 * Q4_0 / Q8_0 weights, AMV_T_Q8_K, AMV_ACT_Q8_K_MMA or AMV_ACT_Q8_K_DEQ for Q4_K (Q6_K: AMV_T_Q8_K or
 * AMV_ACT_Q8_K_MMA). With the plain or MMA layouts and m > 64 the product is the exact form on the int8 matrix cores
 * (one v_mfma_i32_32x32x32_i8 per 32-block: each block's ggml integer comes out exact, then ggml's f32 epilogue);
 * with the DEQ layouts and m > 64 the weights are staged as f16 (q - 8) d_w (Q4_K: (d sc) q - dmin m) against the
 * activations' f16 q_a d_a and the matrix cores accumulate across all of k (no per-block epilogue; within ~3e-4
 * relative L2 of the exact form). 8..64 tokens run the small-batch kernels (Q4_K on the MMA layout's f16 copies).
 * Block sums need a plain or MMA layout. */
int amv_mul_mat_q_act(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int act_type, int64_t m,
                      float* dst, int64_t ldd, void* stream);
int amv_mul_mat_q_act_block_sums(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int act_type,
                                 int64_t m, int32_t* sums, void* stream);
/* amv_mul_mat_q_act followed by ADD (the residual after a projection: ggml's ADD of a MUL_MAT's output,
 * enc_binary ggml-ameva.cpp:3806; no fused counterpart in the reference): dst[t][n] = (W act)[t][n] + add[t][n],
 * add f32 with row stride ldd, not overlapping dst. The exact tiled kernels add it in their epilogue (after the
 * k-split partials), the other paths in a second launch; the values equal the two ops' bit for bit. */
int amv_mul_mat_q_act_add(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int act_type,
                          int64_t m, float* dst, int64_t ldd, const float* add, void* stream);

/* Q4_K / Q6_K weights from f32 rows (ggml blocks), with this library's own deterministic rule: ggml's
 * make_qkx2_quants search (quantize_row_q4_K_ref / q6_K_ref) is not reproduced, so these weight bytes are not a
 * parity target (parity is on the dot products of given bytes). Used for synthetic K-quant weights. */
int amv_quantize_k(int type, const float* x, int64_t n_rows, int64_t k, void* y_ggml, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * BitNet I2_S. Replaces quantize_activation_int8 + bitnet_gemv / ggml_vec_dot_i2_i8_s
 * (adapters/bitnet/src/cpu/llama_bitnet_core.cpp:914-941, ggml_bitnet_mad.cpp:191-231) and the GPU engine's
 * bitnet_norm_q8.comp / bitnet_gemv_i2_s.comp (ac_bitnet_engine.cpp RecordNormQ8 268, RecordGemv 280).
 * Activations: per row absmax int8, layout q int8 [m][k] | {f32 dequant, i32 sum q}[m] (amv_i2s_act_bytes).
 * Weights: the BitNet I2_S tensor as stored (row r at r * k/4 bytes, 128-weight blocks of 32 bytes), k % 128 == 0;
 * the per-tensor scale is the f32 that follows the n_rows * k/4 payload (amuda_gguf.c:659-681) and is passed in.
 * dst[c * ldd + r] = float(sum_j (code_rj - 1) q_cj) * (dequant_c * weight_scale).
 * ---------------------------------------------------------------------------------------------------------- */
int64_t amv_i2s_act_bytes(int64_t m, int64_t k);
int amv_i2s_quantize_act(const float* x, int64_t m, int64_t k, void* act, void* stream);
int amv_i2s_gemv(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float weight_scale, float* dst,
                 int64_t ldd, void* stream);
/* the exact integers sum_j (code_rj - 1) q_cj, int32 [m][n_rows] (bit-exact contract) */
int amv_i2s_gemv_sums(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, int32_t* sums,
                      void* stream);
/* Ternary GEMV on f32 activations with the amuda code map {-1, 0, +1, 0} (bitnet_gemv_i2_s_exact, amuda_ops.c:91-121):
 * y f32 [n_rows] = scale * sum_j map(c_rj) x_j; w the BitNet packing above (k % 128 == 0), x f32 [k]. Backs
 * ac_ops_bitnet_gemv_i2_s_exact of libamuda_hip.so. */
/* dst[r] += float(isum_r) * (act_dequant * weight_scale) for one activation row (I2_S GEMV with the residual add of
 * the BitNet layer fused: llama_bitnet_core.cpp:1244, 1264). */
int amv_i2s_gemv_acc(const void* w, int64_t n_rows, int64_t k, const void* act, float weight_scale, float* dst,
                     void* stream);

/* The BitNet token step's other kernels (the reference engine ac_bitnet_engine.cpp:246-351 over the CPU arithmetic of
 * llama_bitnet_core.cpp:886-1117):
 *   amv_bitnet_norm_q8: x = a (mode 0), relu(a)^2 * b (1) or silu(a) * b (2); when do_norm, x = x / sqrt(mean x^2 + eps)
 *     times w (w may be NULL); y (may be NULL) receives x, act (may be NULL) its int8 activation in the
 *     amv_i2s_quantize_act layout (quantize_activation_int8). One row of n <= 16384 (n % 16 == 0 with act).
 *   amv_bitnet_rope_kv: RoPE (pairs i, i + hd/2) of q [n_head][hd] in place and of k [n_head_kv][hd] into row pos[0] of
 *     k_cache, v into row pos[0] of v_cache (rows of n_head_kv * hd floats), from cs = [cos 0..hd/2-1, sin 0..hd/2-1].
 *   amv_gemv_f16: y[r] = sum_c f16(w[r][c]) * x[c] (the f16 LM head), k % 8 == 0, 16-byte aligned w and x. */
int amv_bitnet_norm_q8(const float* a, const float* b, const float* w, int64_t n, float eps, int mode, int do_norm,
                       float* y, void* act, void* stream);
int amv_bitnet_rope_kv(float* q, const float* k, const float* v, const float* cs, float* k_cache, float* v_cache,
                       const int32_t* pos, int64_t n_head, int64_t n_head_kv, int64_t hd, int64_t n_ctx, void* stream);
int amv_gemv_f16(const void* w, int64_t n_rows, int64_t k, const float* x, float* y, void* stream);
/* One launch per projection group of the BitNet token step (the reference engine's RecordNormQ8 + RecordGemv pairs,
 * ac_bitnet_engine.cpp:268-341): the input's activation as amv_bitnet_norm_q8 (mode, do_norm, norm_w) computed by
 * every workgroup into LDS, then n_seg (1..3) stacked I2_S matrices: matrix s has rows[s] rows of k / 4 bytes at w[s],
 * its outputs dst[s][r] = float(isum_r) * (dequant * wscale[s]) (added to dst[s][r] when accumulate). With rope_cs
 * (= [cos 0..63, sin 0..63] of the position, head_dim 128): matrices Q | K | V, q written rotated to dst[0], k rotated
 * and v as is into row pos[0] (clamped to n_ctx - 1) of the f32 caches dst[1], dst[2] (rows of rows[1] floats): the
 * values amv_i2s_gemv + amv_bitnet_rope_kv produce. k % 128 == 0, k <= 16384, 16-byte aligned pointers. */
int amv_bitnet_gemv_fused(const float* a, const float* b, const float* norm_w, int64_t k, float eps, int mode,
                          int do_norm, int n_seg, const void* const* w, const int64_t* rows, const float* wscale,
                          float* const* dst, int accumulate, const float* rope_cs, const int32_t* pos, int64_t n_ctx,
                          void* stream);
/* The output projection group of the BitNet token step with the attention's split merge in its prologue (no
 * counterpart in the reference, whose engine runs attention as one dispatch; for the HIP engine at short contexts,
 * where the merge launch is a memory round trip the projection's prologue already pays): every workgroup merges the
 * partials of amv_flash_attn_split_kv (part, n_split splits of split_len keys, the key count n_kv_dev[0] capped at
 * n_kv_max; k / 128 heads of 128) exactly as amv_flash_attn_decode_kv's merge does, then runs
 * amv_bitnet_gemv_fused(att, NULL, norm_w, k, eps, 0, do_norm, 1, {w}, {rows}, {wscale}, {dst}, accumulate):
 * bit-identical to the split + merge + projection launches. n_kv_max may span at most min(n_split, 4) splits. */
int amv_bitnet_gemv_fa_merge(const float* part, int n_split, int split_len, int64_t n_kv_max, const int32_t* n_kv_dev,
                             const float* norm_w, int64_t k, float eps, int do_norm, const void* w, int64_t rows,
                             float wscale, float* dst, int accumulate, void* stream);

int amv_i2s_gemv_f32(const void* w, int64_t n_rows, int64_t k, const float* x, float scale, float* y, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * RMS_NORM (ggml_compute_forward_rms_norm_f32; enc_rms_norm ggml-ameva.cpp:3941 with the fused MUL of
 * ameva_find_fusion 4348-4357, ameva_rms_norm.comp): x f32 [n_rows][n]; y = x / sqrt(mean(x^2) + eps) (may be NULL),
 * o = y * w (w f32 [n]; NULL for none), act (may be NULL): the Q8_0 activation layout of amv_quantize_act, of y * w
 * when w is given (o may then be NULL) and of y otherwise, quantized with `rule` -- the input of the next MUL_MAT in
 * one pass.
 * ---------------------------------------------------------------------------------------------------------- */
int amv_rms_norm(const float* x, int64_t n_rows, int64_t n, float eps, const float* w, float* y, float* o, void* act,
                 int rule, void* stream);
/* amv_rms_norm with the fused quantization into the activation type of the next GEMV: act_type 8 = Q8_0 (`rule`,
 * n % 32 == 0) or 15 = Q8_K (n % 256 == 0); act has n_rows rows in the amv_quantize_act layout. */
int amv_rms_norm_act(const float* x, int64_t n_rows, int64_t n, float eps, const float* w, float* y, float* o,
                     void* act, int act_type, int rule, void* stream);

/* ROPE (ggml_rope_ext f32, enc_rope ggml-ameva.cpp:3965, ameva_rope.comp): x, y [n_tok][n_head][ne0] contiguous
 * (in place allowed), pos int32 [n_tok]; mode 0 NORMAL or 2 NEOX; ext_factor 0, no frequency factors. */
int amv_rope(const float* x, float* y, const int32_t* pos, int64_t n_tok, int64_t n_head, int64_t ne0, int n_dims,
             int mode, float freq_base, float freq_scale, float attn_factor, void* stream);

/* ROPE of q and k followed by the two SET_ROWS of the KV cache, in one launch (no counterpart in the reference, which
 * records ROPE enc_rope ggml-ameva.cpp:3965 and SET_ROWS ameva_set_rows.comp as separate nodes; values are those of
 * amv_rope then amv_set_rows_f16). qkv f32 [n_tok][n_head + 2 n_head_kv][D]: q heads, k heads, v heads of each token.
 * q and k heads are rotated in place (pos int32 [n_tok]); the rotated k heads and the v heads are stored as f16 at row
 * kv_idx[t] (int64) of k_cache / v_cache (row stride cache_row elements, head h at h * D, cache_rows rows). Rows
 * outside the cache are skipped and counted in *bad (device, may be NULL). */
int amv_rope_kv_store(float* qkv, const int32_t* pos, int64_t n_tok, int64_t n_head, int64_t n_head_kv, int64_t D,
                      int n_dims, int mode, float freq_base, float freq_scale, float attn_factor, void* k_cache,
                      void* v_cache, int64_t cache_row, const int64_t* kv_idx, int64_t cache_rows, unsigned int* bad,
                      void* stream);

/* GLU SWIGLU (ggml_vec_swiglu_f32; enc_glu, ameva_glu.comp:45-46): y = silu(g) * u. */
int amv_swiglu(const float* g, const float* u, float* y, int64_t n, void* stream);
/* SWIGLU of n_rows rows (g, u, y row strides in floats; ggml's split GLU over views of one gate/up row) with the
 * Q8_0 quantization of every output row fused (act: amv_quantize_act's Q8_0 layout of n_rows x n, or NULL; y may be
 * NULL when act is given). The act bytes equal amv_quantize_act of y. */
int amv_swiglu_rows(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* y, int64_t y_stride,
                    int64_t n_rows, int64_t n, void* act, int rule, void* stream);
/* amv_swiglu_rows with the fused quantization into the activation type of the next MUL_MAT: act_type 8 = Q8_0
 * (`rule`, n % 32 == 0) or 15 = Q8_K (n % 256 == 0; g, u, y 16-byte aligned with strides and n multiples of 4). */
int amv_swiglu_rows_act(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* y,
                        int64_t y_stride, int64_t n_rows, int64_t n, void* act, int act_type, int rule, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * FLASH_ATTN_EXT, decode (one query position), f16 K/V cache (enc_flash_attn ggml-ameva.cpp:4204-4284 with the key
 * splits of ameva_fa_split_keys 4170-4195, ameva_flash_attn.comp + ameva_fa_combine.comp).
 *   q f32 [n_head][D] contiguous; out f32 [n_head][D]; D = 128; n_head / n_head_kv in {1, 2, 4, 8}.
 *   k, v f16: element d of key j of KV head h at k[j * k_row + h * k_head + d] (strides in elements, ggml's nb[1] / 2
 *   and nb[2] / 2: llama.cpp's cache view has k_row = n_head_kv * D, k_head = D); the first n_kv keys are used.
 *   mask f16 [n_kv] or NULL (added to the scaled scores; -inf masks a key).
 *   workspace: amv_flash_attn_workspace_bytes() bytes of device memory for the split partials.
 *   act (may be NULL): the output also quantized to the Q8_0 activation layout of amv_quantize_act (one row of
 *   n_head * D) with `rule` -- the input of the attention output projection, without a separate pass.
 * ---------------------------------------------------------------------------------------------------------- */
int64_t amv_flash_attn_workspace_bytes(int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D);
int amv_flash_attn_decode(const float* q, const void* k, const void* v, const void* mask, float* out, int64_t n_head,
                          int64_t n_head_kv, int64_t n_kv, int64_t D, int64_t k_row, int64_t k_head, int64_t v_row,
                          int64_t v_head, float scale, void* workspace, int64_t workspace_bytes, void* act, int rule,
                          void* stream);

/* amv_flash_attn_decode with the key count in device memory and a choice of output quantization (no counterpart in
 * the reference; for decode steps captured once in a HIP graph and replayed at growing positions). The key count is
 * n_kv_dev[0] when n_kv_dev is not NULL, capped at n_kv_max, which sizes the launch and the workspace
 * (amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv_max, D)). act (may be NULL): the output's activation row,
 * act_type 8 = Q8_0 (`rule`) or 15 = Q8_K (even n_head / n_head_kv). counters == NULL: the split merge runs as a
 * second launch; otherwise in the last workgroup of each KV head (one launch; counters: >= 32 * n_head_kv words,
 * zero before the first call, left at zero). Results identical to amv_flash_attn_decode at the same key count
 * whenever both pick the same key split (always when n_kv_max * n_head_kv <= 65536). */
int amv_flash_attn_decode_ex(const float* q, const void* k, const void* v, const void* mask, float* out,
                             int64_t n_head, int64_t n_head_kv, int64_t n_kv_max, const int32_t* n_kv_dev, int64_t D,
                             int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head, float scale,
                             void* workspace, int64_t workspace_bytes, unsigned int* counters, void* act, int act_type,
                             int rule, void* stream);

/* FLASH_ATTN_EXT decode over an f32, f16, Q8_0 or Q4_0 KV cache (the reference's quantized-cache attention,
 * ameva_flash_attn.comp:4-8 and 104-136; ggml_compute_forward_flash_attn_ext for the CPU semantics; the f32 cache is
 * the BitNet engine's, llama_bitnet_core.cpp:1033-1082, with q . k in f32). kv_type: 0 = F32, 1 = F16, 8 = Q8_0,
 * 2 = Q4_0 (K and V both); strides in BYTES (ggml's nb[1], nb[2]); a quantized row of D = 128 elements is 4
 * ggml blocks (136 bytes Q8_0, 72 bytes Q4_0) at a 2-byte-aligned address. For a quantized K, q is quantized to Q8_0
 * with `rule` (K's vec_dot_type, as ggml's CPU kernel does) and each score is sum_b float(isum_b) * (d_k * d_q) over
 * the exact integer block sums; V rows are dequantized exactly (q * d, (nibble - 8) * d); f16 caches behave as in
 * amv_flash_attn_decode_ex. Other arguments as amv_flash_attn_decode_ex. */
int amv_flash_attn_decode_kv(int kv_type, const float* q, const void* k, const void* v, const void* mask, float* out,
                             int64_t n_head, int64_t n_head_kv, int64_t n_kv_max, const int32_t* n_kv_dev, int64_t D,
                             int64_t k_row_bytes, int64_t k_head_bytes, int64_t v_row_bytes, int64_t v_head_bytes,
                             float scale, void* workspace, int64_t workspace_bytes, unsigned int* counters, void* act,
                             int act_type, int rule, void* stream);

/* The split pass of amv_flash_attn_decode_kv alone, for a consumer that merges the partials itself
 * (amv_bitnet_gemv_fa_merge; no counterpart in the reference). Same launch, arguments and workspace as
 * amv_flash_attn_decode_kv with counters == NULL and no output; writes the launch's split count and keys per split to
 * *n_split and *split_len. Head h, split z: (m, l, pad, pad, acc[D]) at workspace + (h * n_split + z) * (D + 4) floats
 * for the splits that hold keys. */
int amv_flash_attn_split_kv(int kv_type, const float* q, const void* k, const void* v, const void* mask, int64_t n_head,
                            int64_t n_head_kv, int64_t n_kv_max, const int32_t* n_kv_dev, int64_t D,
                            int64_t k_row_bytes, int64_t k_head_bytes, int64_t v_row_bytes, int64_t v_head_bytes,
                            float scale, void* workspace, int64_t workspace_bytes, int rule, int32_t* n_split,
                            int32_t* split_len, void* stream);

/* amv_flash_attn_decode_kv without a workspace or counters argument and without any allocation. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The split partials live in a library-owned device array of
 * amv_flash_attn_noalloc_max_bytes() bytes (8 MiB) that each GPU the library runs on holds until the process ends;
 * shapes whose partials need more (amv_flash_attn_workspace_bytes) are rejected with AMV_ERR_INVALID_ARG. The first
 * call on a device looks the array's address up (no allocation; make that call outside graph capture). Calls that
 * overlap in time on one device share the array and race; the merge always runs as a second launch. Results are
 * identical to amv_flash_attn_decode_kv with counters == NULL. */
int64_t amv_flash_attn_noalloc_max_bytes(void);
int amv_flash_attn_decode_noalloc(int kv_type, const float* q, const void* k, const void* v, const void* mask,
                                  float* out, int64_t n_head, int64_t n_head_kv, int64_t n_kv_max,
                                  const int32_t* n_kv_dev, int64_t D, int64_t k_row_bytes, int64_t k_head_bytes,
                                  int64_t v_row_bytes, int64_t v_head_bytes, float scale, void* act, int act_type,
                                  int rule, void* stream);

/* FLASH_ATTN_EXT over n_tok query positions (prompt prefill; enc_flash_attn ggml-ameva.cpp:4204-4284 with
 * q->ne[1] > 1, ameva_flash_attn.comp), on the f16 matrix cores. D = 128, n_head / n_head_kv integral.
 *   q f32: element d of head h of token t at q[t * q_tok_stride + h * q_head_stride + d] (strides in floats, multiples
 *   of 4: the q heads of a fused q/k/v row can be passed in place); out f32 [n_tok][n_head][D] contiguous.
 *   k, v f16 as in amv_flash_attn_decode (strides in elements, multiples of 8); keys 0 .. n_kv - 1.
 *   mask f16 [n_tok][mask_stride] or NULL, added to the scaled scores (ggml's KQ mask; -inf hides a key).
 *   causal_pos0 >= 0: token t is at position causal_pos0 + t and sees keys 0 .. causal_pos0 + t only (the causal
 *   mask built in); < 0: no position limit.
 * Queries that see no key get a zero row. */
int amv_flash_attn_prefill(const float* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k, const void* v,
                           const void* mask, int64_t mask_stride, float* out, int64_t n_tok, int64_t n_head,
                           int64_t n_head_kv, int64_t n_kv, int64_t D, int64_t k_row, int64_t k_head, int64_t v_row,
                           int64_t v_head, float scale, int64_t causal_pos0, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * Glue ops of the decoder graph (ameva_binary.comp, ameva_cpy.comp, ameva_set_rows.comp, ameva_get_rows(_q).comp).
 * ---------------------------------------------------------------------------------------------------------- */
/* ADD (op 0) / MUL (op 1), f32: dst[r][i] = a[r][i] op b[r % b_rows][i] for n_rows rows of n elements. */
int amv_binary(int op, const float* a, const float* b, float* dst, int64_t n_rows, int64_t n, int64_t b_rows,
               void* stream);
/* SET_ROWS / CPY f32 -> f16: row r of src (stride src_stride elements) to row idx[r] of dst (stride dst_stride), or row
 * r when idx is NULL; idx_bits 32 or 64. Out-of-range indices are skipped and counted in *bad (device, may be NULL). */
int amv_set_rows_f16(const float* src, int64_t src_stride, void* dst, int64_t dst_stride, int64_t n_rows, int64_t n,
                     const void* idx, int idx_bits, int64_t dst_rows, unsigned int* bad, void* stream);
/* SET_ROWS / CPY f32 -> Q8_0 or Q4_0 (a quantized KV cache; ameva_set_rows_q.comp:82-115): row r of src (stride
 * src_stride elements, n % 32 == 0) quantized with ggml's from_float of `type` (8 = Q8_0 with `rule`, 2 = Q4_0:
 * quantize_row_q4_0_ref) into row idx[r] (or r) of dst, dst_stride in BYTES (even, >= n / 32 blocks); out-of-range
 * indices are skipped and counted once per row in *bad. */
int amv_set_rows_q(int type, const float* src, int64_t src_stride, void* dst, int64_t dst_stride, int64_t n_rows,
                   int64_t n, const void* idx, int idx_bits, int64_t dst_rows, int rule, unsigned int* bad,
                   void* stream);
/* GET_ROWS (enc_get_rows, ameva_get_rows_q.comp): dst f32 [n_idx][n] = row idx[i] of src (type F32, F16, Q4_0,
 * Q8_0, Q4_K or Q6_K in ggml layout, src_rows rows), dequantized with ggml's dequantize_row_* expressions; rows
 * outside [0, src_rows) give zeros and add 1 to *bad when bad is not NULL. */
int amv_get_rows(int type, const void* src, int64_t src_rows, int64_t n, const int32_t* idx, int64_t n_idx, float* dst,
                 unsigned int* bad, void* stream);
/* Greedy sampling of a decode step (the argmax of llama.cpp's greedy sampler; no GPU kernel in the reference, whose
 * logits go back to the host): token[0] = index of the largest of x[0 .. n) (the first on ties; NaN never wins).
 * history (may be NULL): history[step[0]] = token when step[0] < history_len, then step[0] += 1 -- a decode loop
 * replayed as a HIP graph keeps its tokens on the device. x 16-byte aligned. */
int amv_argmax(const float* x, int64_t n, int32_t* token, int32_t* history, int32_t* step, int64_t history_len,
               void* stream);
/* amv_argmax over the whole GPU (workgroups of 2048 float4 of x; an atomic maximum of (value, index) keys and the last
 * workgroup to arrive writes the result), and, when pos / kv_idx / n_kv are not NULL, the decode position advanced:
 * pos[0] += 1, kv_idx[0] += 1, n_kv[0] += 1 -- the end of a decode step in one launch (no counterpart in the
 * reference, whose sampler runs on the host). ws: 16 bytes, 16-byte aligned, zero before the first call; every call
 * leaves them zero. Calls that overlap on one ws race. Same token as amv_argmax. */
int amv_argmax_ex(const float* x, int64_t n, int32_t* token, int32_t* history, int32_t* step, int64_t history_len,
                  int32_t* pos, int64_t* kv_idx, int32_t* n_kv, void* ws, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AMEVA_HIP_H */
