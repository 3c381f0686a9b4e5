/*
 * CPU restatement of the ggml CPU arithmetic that the ameva quantized backend must reproduce.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it. The product path (ameva_compute_amd) never links, imports or calls it.
 *
 * The reference's parity oracle is ggml's CPU backend (llama.cpp tag b8471, ggml 0.9.8; empty submodule at
 * third_party/llama.cpp, .gitmodules:4-6). It is not in this image, so every rule below is restated from the
 * behaviour documented in the reference's own sources, which cite it:
 *   block layouts        adapters/llama/ggml-ameva/shaders/ameva_qmm.comp:22-36
 *   fp16 <-> fp32        include/ggml/ggml-impl.h:388-441 (IEEE binary16, round to nearest even; restated from the
 *                        IEEE-754 definition, not from that header's bit trick)
 *   Q4_0 quantizer       adapters/llama/ggml-ameva/shaders/ameva_set_rows_q.comp:10,95-115
 *   Q8_0 quantizer       ameva_set_rows_q.comp:9,82-94 (ARM rule), ameva_act_fq.comp:5,38-41 (x86 rule)
 *   dequantization       ameva_qdecode.glsl:129-136 (Q4_0), 163-170 (Q8_0), 221-245 (Q4_K), 246-258 (Q6_K)
 *   K-quant dot formula  ameva_mmqb.comp:11-16
 *   RMSNorm              ameva_rms_norm.comp:3-7 (ggml sums the squares in double)
 *   RoPE                 ggml-ameva.cpp:3982-3984 + ameva_rope.comp:64-92 (angle by repeated f32 multiply)
 *   flash attention      ameva_flash_attn.comp:4-23, ameva_fa_combine.comp:1-9
 *   SwiGLU               ameva_glu.comp:45-46
 *   I2_S                 adapters/bitnet/src/cpu/ggml_bitnet_mad.cpp:191-231 (scalar branch),
 *                        adapters/bitnet/src/cpu/llama_bitnet_core.cpp:914-941, amuda_gguf.c:659-681 (trailer)
 * Each function below names the file:line it follows.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK4_0 32
#define QK8_0 32
#define QK_K 256
#define QK_I2S 128

/* ggml block sizes in bytes (ameva_qmm.comp:22-36) */
#define BS_Q4_0 18
#define BS_Q8_0 34
#define BS_Q4_K 144
#define BS_Q6_K 210
#define BS_Q8_K 292 /* f32 d, int8 qs[256], int16 bsums[16] */

/* ------------------------------------------------------------------------------------------------------------------
 * fp16 (IEEE binary16), round to nearest even. Behaviour of ggml_compute_fp32_to_fp16 (ggml-impl.h:414-437):
 * NaN -> 0x7E00 | sign, overflow -> inf, subnormals kept.
 * ---------------------------------------------------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t orc_fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u); /* NaN */
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf (and inf itself) */
    const int e = (int)(ax >> 23) - 127;                       /* unbiased exponent */
    if (e >= -14) {
        /* normal half: keep 10 mantissa bits, round the 13 dropped bits to nearest even */
        uint32_t m = ax & 0x7FFFFFu;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        const uint32_t rest = m & 0x1FFFu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u; /* a carry into the exponent is correct */
        return (uint16_t)(sign | h);
    }
    if (e < -25) return (uint16_t)sign; /* below half of the smallest subnormal: zero */
    /* subnormal half: value = mf * 2^(e-23) with mf the full 24-bit significand; in units of 2^-24 that is
     * mf * 2^(e+1), a right shift by d = -(e+1) bits (14..24), rounded to nearest even */
    const uint32_t mf = (ax & 0x7FFFFFu) | 0x800000u;
    const int d = -(e + 1);
    uint32_t h = mf >> d;
    const uint32_t rest = mf & ((1u << d) - 1u);
    const uint32_t half = 1u << (d - 1);
    if (rest > half || (rest == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_fp32_to_fp16_n(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp32_to_fp16(x[i]);
}
void orc_fp16_to_fp32_n(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp16_to_fp32(x[i]);
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)(v & 0xFF); p[1] = (uint8_t)(v >> 8); }

/* ------------------------------------------------------------------------------------------------------------------
 * Quantizers
 * ---------------------------------------------------------------------------------------------------------------- */

/* ggml quantize_row_q4_0_ref (ameva_set_rows_q.comp:10,95-115): max = the element of largest magnitude (first on
 * ties), d = max / -8, id = 1/d, nibble = min(15, trunc(x * id + 8.5)); element j in the low nibble of qs[j],
 * element j + 16 in the high nibble; d stored fp16. */
void orc_quantize_q4_0(const float *x, uint8_t *y, int64_t nrows, int64_t k) {
    const int64_t nb = k / QK4_0;
    for (int64_t r = 0; r < nrows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            const float *xb = x + r * k + b * QK4_0;
            uint8_t *yb = y + (r * nb + b) * BS_Q4_0;
            float amax = 0.0f, max = 0.0f;
            for (int j = 0; j < QK4_0; ++j) {
                if (amax < fabsf(xb[j])) { amax = fabsf(xb[j]); max = xb[j]; }
            }
            const float d = max / -8.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            wr16(yb, orc_fp32_to_fp16(d));
            for (int j = 0; j < 16; ++j) {
                const float x0 = xb[j] * id, x1 = xb[16 + j] * id;
                int q0 = (int)(int8_t)(x0 + 8.5f), q1 = (int)(int8_t)(x1 + 8.5f);
                if (q0 > 15) q0 = 15;
                if (q1 > 15) q1 = 15;
                yb[2 + j] = (uint8_t)(q0 | (q1 << 4));
            }
        }
    }
}

/* Q8_0 quantization rules. All store d = amax/127 as fp16 and |q| <= 127.
 *   ORC_Q8_X86 (0): ggml-cpu x86 quantize_row_q8_0 (activations on x86): id = 127/amax, round half to even
 *                   (the rule ameva_act_fq.comp:5,38-41 states).
 *   ORC_Q8_ARM (1): ggml-cpu ARM quantize_row_q8_0: id = 1/d, round half to even (ameva_set_rows_q.comp:9,82-94).
 *   ORC_Q8_REF (2): quantize_row_q8_0_ref (ggml_quantize_chunk, weights): id = 1/d, roundf (half away from zero). */
void orc_quantize_q8_0(const float *x, uint8_t *y, int64_t nrows, int64_t k, int rule) {
    const int64_t nb = k / QK8_0;
    for (int64_t r = 0; r < nrows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            const float *xb = x + r * k + b * QK8_0;
            uint8_t *yb = y + (r * nb + b) * BS_Q8_0;
            float amax = 0.0f;
            for (int j = 0; j < QK8_0; ++j) amax = fmaxf(amax, fabsf(xb[j]));
            const float d = amax / 127.0f;
            float id;
            if (rule == 0) id = amax != 0.0f ? 127.0f / amax : 0.0f;
            else id = d != 0.0f ? 1.0f / d : 0.0f;
            wr16(yb, orc_fp32_to_fp16(d));
            for (int j = 0; j < QK8_0; ++j) {
                const float v = xb[j] * id;
                float q = (rule == 2) ? roundf(v) : rintf(v);
                if (q > 127.0f) q = 127.0f;
                if (q < -127.0f) q = -127.0f;
                yb[2 + j] = (uint8_t)(int8_t)q;
            }
        }
    }
}

/* ggml quantize_row_q8_K_ref: max = the element of largest magnitude (first on ties), iscale = -127/max,
 * q = min(127, nearest-even(iscale * x)), d = 1/iscale (f32), bsums = sums of q per 16 elements. */
void orc_quantize_q8_K(const float *x, uint8_t *y, int64_t nrows, int64_t k) {
    const int64_t nb = k / QK_K;
    for (int64_t r = 0; r < nrows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            const float *xb = x + r * k + b * QK_K;
            uint8_t *yb = y + (r * nb + b) * BS_Q8_K;
            int8_t *qs = (int8_t *)(yb + 4);
            float amax = 0.0f, max = 0.0f;
            for (int j = 0; j < QK_K; ++j) {
                const float ax = fabsf(xb[j]);
                if (ax > amax) { amax = ax; max = xb[j]; }
            }
            if (amax == 0.0f) {
                memset(yb, 0, BS_Q8_K);
                continue;
            }
            const float iscale = -127.0f / max;
            for (int j = 0; j < QK_K; ++j) {
                int v = (int)rintf(iscale * xb[j]);
                qs[j] = (int8_t)(v < 127 ? v : 127);
            }
            for (int g = 0; g < 16; ++g) {
                int s = 0;
                for (int j = 0; j < 16; ++j) s += qs[16 * g + j];
                wr16(yb + 4 + QK_K + 2 * g, (uint16_t)(int16_t)s);
            }
            const float d = 1.0f / iscale;
            memcpy(yb, &d, 4);
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * Dequantization (ameva_qdecode.glsl decode(); ggml dequantize_row_*)
 * ---------------------------------------------------------------------------------------------------------------- */
static void k4_scale_min(int j, const uint8_t *q, int *sc, int *m) {
    /* get_scale_min_k4 (ameva_qdecode.glsl:229-236) */
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* type: ggml_type (2 Q4_0, 8 Q8_0, 12 Q4_K, 14 Q6_K). n elements (a multiple of the block size). */
int orc_dequantize(int type, const uint8_t *x, float *y, int64_t n) {
    if (type == 2) {
        for (int64_t b = 0; b < n / 32; ++b) {
            const uint8_t *xb = x + b * BS_Q4_0;
            const float d = orc_fp16_to_fp32(rd16(xb));
            for (int j = 0; j < 16; ++j) {
                y[32 * b + j] = (float)((xb[2 + j] & 0xF) - 8) * d;
                y[32 * b + 16 + j] = (float)((xb[2 + j] >> 4) - 8) * d;
            }
        }
        return 0;
    }
    if (type == 8) {
        for (int64_t b = 0; b < n / 32; ++b) {
            const uint8_t *xb = x + b * BS_Q8_0;
            const float d = orc_fp16_to_fp32(rd16(xb));
            for (int j = 0; j < 32; ++j) y[32 * b + j] = (float)(int8_t)xb[2 + j] * d;
        }
        return 0;
    }
    if (type == 12) {
        for (int64_t b = 0; b < n / QK_K; ++b) {
            const uint8_t *xb = x + b * BS_Q4_K;
            const float d = orc_fp16_to_fp32(rd16(xb)), dmin = orc_fp16_to_fp32(rd16(xb + 2));
            const uint8_t *sc = xb + 4, *qs = xb + 16;
            float *yb = y + b * QK_K;
            for (int c = 0; c < 4; ++c) { /* 64 weights per chunk: low nibbles, then high nibbles */
                int s1, m1, s2, m2;
                k4_scale_min(2 * c, sc, &s1, &m1);
                k4_scale_min(2 * c + 1, sc, &s2, &m2);
                const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
                const float d2 = d * (float)s2, mm2 = dmin * (float)m2;
                for (int l = 0; l < 32; ++l) yb[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0xF) - mm1;
                for (int l = 0; l < 32; ++l) yb[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - mm2;
            }
        }
        return 0;
    }
    if (type == 14) {
        for (int64_t b = 0; b < n / QK_K; ++b) {
            const uint8_t *xb = x + b * BS_Q6_K;
            const uint8_t *ql = xb, *qh = xb + 128;
            const int8_t *sc = (const int8_t *)(xb + 192);
            const float d = orc_fp16_to_fp32(rd16(xb + 208));
            float *yb = y + b * QK_K;
            for (int h = 0; h < 2; ++h) { /* two halves of 128 weights */
                const uint8_t *l4 = ql + 64 * h, *hh = qh + 32 * h;
                const int8_t *s = sc + 8 * h;
                float *yh = yb + 128 * h;
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q1 = ((l4[l] & 0xF) | (((hh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((l4[l + 32] & 0xF) | (((hh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((l4[l] >> 4) | (((hh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((l4[l + 32] >> 4) | (((hh[l] >> 6) & 3) << 4)) - 32;
                    yh[l] = d * (float)s[is + 0] * (float)q1;
                    yh[l + 32] = d * (float)s[is + 2] * (float)q2;
                    yh[l + 64] = d * (float)s[is + 4] * (float)q3;
                    yh[l + 96] = d * (float)s[is + 6] * (float)q4;
                }
            }
        }
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------------------------------------------------------
 * Dot products of one weight row with one quantized activation row, with the exact integer sums exposed.
 * fp32 combination follows ggml's generic vec_dot: sumf += (float)sumi * d_w * d_a per block.
 * ---------------------------------------------------------------------------------------------------------------- */

/* vec_dot_q4_0_q8_0: per block sumi = sum_j (nib_j - 8) * qa_j (int32, exact). blk may be NULL. */
float orc_vec_dot_q4_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *a, int32_t *blk) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / 32; ++b) {
        const uint8_t *wb = w + b * BS_Q4_0, *ab = a + b * BS_Q8_0;
        const int8_t *qa = (const int8_t *)(ab + 2);
        int32_t s = 0;
        for (int j = 0; j < 16; ++j) {
            s += ((wb[2 + j] & 0xF) - 8) * qa[j];
            s += ((wb[2 + j] >> 4) - 8) * qa[16 + j];
        }
        if (blk) blk[b] = s;
        sumf += (float)s * orc_fp16_to_fp32(rd16(wb)) * orc_fp16_to_fp32(rd16(ab));
    }
    return sumf;
}

/* vec_dot_q8_0_q8_0: per block sumi = sum_j qw_j * qa_j. */
float orc_vec_dot_q8_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *a, int32_t *blk) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / 32; ++b) {
        const uint8_t *wb = w + b * BS_Q8_0, *ab = a + b * BS_Q8_0;
        const int8_t *qw = (const int8_t *)(wb + 2), *qa = (const int8_t *)(ab + 2);
        int32_t s = 0;
        for (int j = 0; j < 32; ++j) s += qw[j] * qa[j];
        if (blk) blk[b] = s;
        sumf += (float)s * (orc_fp16_to_fp32(rd16(wb)) * orc_fp16_to_fp32(rd16(ab)));
    }
    return sumf;
}

/* vec_dot_q4_K_q8_K (formula of ameva_mmqb.comp:11-13): per super-block the integers
 *   isum = sum_u sc_u * dot(v_u, q_a,u)   (v the 4-bit values, 8 units of 32)
 *   msum = sum_u m_u * (sum of q_a over unit u)  (= sum over the 16 bsums pairs)
 * result += d_w * d_a * isum - dmin_w * d_a * msum. blk (may be NULL) receives isum, msum per super-block. */
float orc_vec_dot_q4_K_q8_K(int64_t k, const uint8_t *w, const uint8_t *a, int32_t *blk) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / QK_K; ++b) {
        const uint8_t *wb = w + b * BS_Q4_K, *ab = a + b * BS_Q8_K;
        const uint8_t *sc = wb + 4, *qs = wb + 16;
        const int8_t *qa = (const int8_t *)(ab + 4);
        float da;
        memcpy(&da, ab, 4);
        int32_t isum = 0, msum = 0;
        for (int u = 0; u < 8; ++u) {
            int s, m;
            k4_scale_min(u, sc, &s, &m);
            const int c = u / 2, hi = u & 1;
            int32_t dot = 0, asum = 0;
            for (int l = 0; l < 32; ++l) {
                const int v = hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 0xF);
                dot += v * qa[32 * u + l];
                asum += qa[32 * u + l];
            }
            isum += s * dot;
            msum += m * asum;
        }
        if (blk) { blk[2 * b] = isum; blk[2 * b + 1] = msum; }
        const float d = orc_fp16_to_fp32(rd16(wb)) * da;
        const float dmin = orc_fp16_to_fp32(rd16(wb + 2)) * da;
        sumf += d * (float)isum - dmin * (float)msum;
    }
    return sumf;
}

/* vec_dot_q6_K_q8_K: per super-block isum = sum_h sc_h * dot(q6_h - 32, q_a,h) over 16 groups of 16 weights. */
float orc_vec_dot_q6_K_q8_K(int64_t k, const uint8_t *w, const uint8_t *a, int32_t *blk) {
    float sumf = 0.0f;
    int8_t v[QK_K];
    for (int64_t b = 0; b < k / QK_K; ++b) {
        const uint8_t *wb = w + b * BS_Q6_K, *ab = a + b * BS_Q8_K;
        const int8_t *sc = (const int8_t *)(wb + 192);
        const int8_t *qa = (const int8_t *)(ab + 4);
        float da;
        memcpy(&da, ab, 4);
        for (int h = 0; h < 2; ++h) {
            const uint8_t *l4 = wb + 64 * h, *hh = wb + 128 + 32 * h;
            for (int l = 0; l < 32; ++l) {
                v[128 * h + l] = (int8_t)(((l4[l] & 0xF) | (((hh[l] >> 0) & 3) << 4)) - 32);
                v[128 * h + l + 32] = (int8_t)(((l4[l + 32] & 0xF) | (((hh[l] >> 2) & 3) << 4)) - 32);
                v[128 * h + l + 64] = (int8_t)(((l4[l] >> 4) | (((hh[l] >> 4) & 3) << 4)) - 32);
                v[128 * h + l + 96] = (int8_t)(((l4[l + 32] >> 4) | (((hh[l] >> 6) & 3) << 4)) - 32);
            }
        }
        int32_t isum = 0;
        for (int g = 0; g < 16; ++g) {
            int32_t dot = 0;
            for (int l = 0; l < 16; ++l) dot += v[16 * g + l] * qa[16 * g + l];
            isum += sc[g] * dot;
        }
        if (blk) blk[b] = isum;
        sumf += orc_fp16_to_fp32(rd16(wb + 208)) * da * (float)isum;
    }
    return sumf;
}

/* MUL_MAT on quantized weights: dst[m][n] = dot(W row n, activation row m), W [n_rows, k] in ggml layout, activations
 * already quantized to the vec_dot type (Q8_0 for Q4_0/Q8_0, Q8_K for Q4_K/Q6_K). OpenMP over rows (the CPU
 * baseline). blk (may be NULL): per-row block integers, [m][n][nblk * per] with per = 2 for Q4_K, else 1. */
int orc_mul_mat(int wtype, const uint8_t *w, int64_t n_rows, int64_t k, const uint8_t *a, int64_t m, float *dst,
                int32_t *blk) {
    int64_t wrow, arow, nblk, per = 1;
    float (*dot)(int64_t, const uint8_t *, const uint8_t *, int32_t *);
    switch (wtype) {
    case 2: wrow = k / 32 * BS_Q4_0; arow = k / 32 * BS_Q8_0; nblk = k / 32; dot = orc_vec_dot_q4_0_q8_0; break;
    case 8: wrow = k / 32 * BS_Q8_0; arow = k / 32 * BS_Q8_0; nblk = k / 32; dot = orc_vec_dot_q8_0_q8_0; break;
    case 12: wrow = k / QK_K * BS_Q4_K; arow = k / QK_K * BS_Q8_K; nblk = k / QK_K; per = 2;
        dot = orc_vec_dot_q4_K_q8_K; break;
    case 14: wrow = k / QK_K * BS_Q6_K; arow = k / QK_K * BS_Q8_K; nblk = k / QK_K; dot = orc_vec_dot_q6_K_q8_K; break;
    default: return -1;
    }
    for (int64_t c = 0; c < m; ++c) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < n_rows; ++r) {
            int32_t *bp = blk ? blk + (c * n_rows + r) * nblk * per : NULL;
            dst[c * n_rows + r] = dot(k, w + r * wrow, a + c * arow, bp);
        }
    }
    return 0;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------------------------------------------------
 * RMSNorm, RoPE, SwiGLU
 * ---------------------------------------------------------------------------------------------------------------- */

/* ggml_compute_forward_rms_norm_f32 (ameva_rms_norm.comp:3-7): sum of x*x (f32 products) in double, mean as f32,
 * scale = 1/sqrtf(mean + eps), y = x * scale; then (the following MUL) o = y * w when w != NULL. */
void orc_rms_norm(const float *x, float *y, const float *w, float *o, int64_t nrows, int64_t n, float eps) {
    for (int64_t r = 0; r < nrows; ++r) {
        const float *xr = x + r * n;
        double sum = 0.0;
        for (int64_t i = 0; i < n; ++i) sum += (double)(xr[i] * xr[i]);
        const float mean = (float)(sum / (double)n);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < n; ++i) {
            y[r * n + i] = xr[i] * scale;
            if (w && o) o[r * n + i] = y[r * n + i] * w[i];
        }
    }
}

/* ggml rope f32, modes NORMAL (0: pairs 2j, 2j+1) and NEOX (2: pairs j, j + n_dims/2), ext_factor 0, no frequency
 * factors (ggml-ameva.cpp:3982-3984, ameva_rope.comp:64-92): theta_scale = powf(base, -2/n_dims); the angle of pair
 * j is p * theta_scale^j built by repeated f32 multiplication; cos/sin by libm cosf/sinf times attn_factor.
 * x [n_tok][n_head][ne0] contiguous; pos[n_tok]; dims past n_dims copied. */
void orc_rope(const float *x, float *y, const int32_t *pos, int64_t n_tok, int64_t n_head, int64_t ne0, int n_dims,
              int mode, float freq_base, float freq_scale, float attn_factor) {
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    float *cosv = (float *)malloc(sizeof(float) * (size_t)(ne0 / 2 + 1));
    float *sinv = (float *)malloc(sizeof(float) * (size_t)(ne0 / 2 + 1));
    for (int64_t t = 0; t < n_tok; ++t) {
        float theta = (float)pos[t];
        for (int64_t j = 0; 2 * j < ne0; ++j) {
            const float th = freq_scale * theta;
            cosv[j] = cosf(th) * attn_factor;
            sinv[j] = sinf(th) * attn_factor;
            theta *= theta_scale;
        }
        for (int64_t h = 0; h < n_head; ++h) {
            const float *xr = x + (t * n_head + h) * ne0;
            float *yr = y + (t * n_head + h) * ne0;
            for (int64_t i = n_dims; i < ne0; ++i) yr[i] = xr[i];
            for (int64_t j = 0; 2 * j < n_dims; ++j) {
                const int64_t e0 = mode == 2 ? j : 2 * j;
                const int64_t e1 = mode == 2 ? j + n_dims / 2 : 2 * j + 1;
                const float x0 = xr[e0], x1 = xr[e1];
                yr[e0] = x0 * cosv[j] - x1 * sinv[j];
                yr[e1] = x0 * sinv[j] + x1 * cosv[j];
            }
        }
    }
    free(cosv);
    free(sinv);
}

/* ggml_vec_swiglu_f32 (ameva_glu.comp:45-46): y = silu(g) * u, silu(x) = x / (1 + expf(-x)). */
void orc_swiglu(const float *g, const float *u, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* ------------------------------------------------------------------------------------------------------------------
 * Flash attention, decode (one query position per head), f16 K/V cache (ameva_flash_attn.comp:4-23).
 * ggml rounds Q to f16 before the K dot product; the rest is evaluated exactly here (double), which is the value
 * ggml's f32/f16 arithmetic approximates.
 *   q f32 [n_head][D]; k, v f16 [n_head_kv][n_kv][D]; mask f16 [n_kv] or NULL; out f32 [n_head][D].
 *   Head h reads KV head h / (n_head / n_head_kv).
 * ---------------------------------------------------------------------------------------------------------------- */
void orc_flash_attn_decode(const float *q, const uint16_t *k, const uint16_t *v, const uint16_t *mask, float *out,
                           int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D, float scale) {
    const int64_t G = n_head / n_head_kv;
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < n_head; ++h) {
        const int64_t hk = h / G;
        double *s = (double *)malloc(sizeof(double) * (size_t)n_kv);
        double *acc = (double *)calloc((size_t)D, sizeof(double));
        float *qh = (float *)malloc(sizeof(float) * (size_t)D);
        for (int64_t d = 0; d < D; ++d) qh[d] = orc_fp16_to_fp32(orc_fp32_to_fp16(q[h * D + d]));
        double mx = -INFINITY;
        for (int64_t j = 0; j < n_kv; ++j) {
            const uint16_t *kr = k + (hk * n_kv + j) * D;
            double dot = 0.0;
            for (int64_t d = 0; d < D; ++d) dot += (double)qh[d] * (double)orc_fp16_to_fp32(kr[d]);
            double x = dot * (double)scale;
            if (mask) x += (double)orc_fp16_to_fp32(mask[j]);
            s[j] = x;
            if (x > mx) mx = x;
        }
        double l = 0.0;
        for (int64_t j = 0; j < n_kv; ++j) {
            if (s[j] == -INFINITY) continue;
            const double p = exp(s[j] - mx);
            l += p;
            const uint16_t *vr = v + (hk * n_kv + j) * D;
            for (int64_t d = 0; d < D; ++d) acc[d] += p * (double)orc_fp16_to_fp32(vr[d]);
        }
        for (int64_t d = 0; d < D; ++d) out[h * D + d] = l > 0.0 ? (float)(acc[d] / l) : 0.0f;
        free(s);
        free(acc);
        free(qh);
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * Flash attention, decode, over a Q8_0 or Q4_0 K/V cache (the reference's quantized-cache attention,
 * ameva_flash_attn.comp:4-8, 104-136; ggml's CPU kernel ggml_compute_forward_flash_attn_ext for what the build
 * matches): q is converted with from_float of K's vec_dot_type (quantize_row_q8_0 with `rule`), each score is
 * vec_dot_q8_0_q8_0 / vec_dot_q4_0_q8_0 of the K row and q in f32, then s * scale + mask in f32; V rows are
 * dequantized (q * d, (nibble - 8) * d); the softmax and P V are evaluated exactly here (double), the value ggml's f32
 * arithmetic approximates.
 *   kv_type 8 (Q8_0) or 2 (Q4_0) for K and V; k, v [n_head_kv][n_kv] rows of D / 32 ggml blocks; q f32 [n_head][D];
 *   mask f16 [n_kv] or NULL; out f32 [n_head][D]. Returns -1 for an unsupported type.
 * ---------------------------------------------------------------------------------------------------------------- */
int orc_flash_attn_decode_q(int kv_type, const float *q, const uint8_t *k, const uint8_t *v, const uint16_t *mask,
                            float *out, int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D, float scale,
                            int rule) {
    if (kv_type != 8 && kv_type != 2) return -1;
    const int64_t bs = kv_type == 8 ? BS_Q8_0 : BS_Q4_0, rb = D / 32 * bs, G = n_head / n_head_kv;
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < n_head; ++h) {
        const int64_t hk = h / G;
        uint8_t *qq = (uint8_t *)malloc((size_t)(D / 32 * BS_Q8_0));
        double *s = (double *)malloc(sizeof(double) * (size_t)n_kv);
        double *acc = (double *)calloc((size_t)D, sizeof(double));
        float *vr = (float *)malloc(sizeof(float) * (size_t)D);
        orc_quantize_q8_0(q + h * D, qq, 1, D, rule);
        double mx = -INFINITY;
        for (int64_t j = 0; j < n_kv; ++j) {
            const uint8_t *kr = k + (hk * n_kv + j) * rb;
            float x = kv_type == 8 ? orc_vec_dot_q8_0_q8_0(D, kr, qq, NULL) : orc_vec_dot_q4_0_q8_0(D, kr, qq, NULL);
            x = x * scale;
            if (mask) x += orc_fp16_to_fp32(mask[j]);
            s[j] = (double)x;
            if (s[j] > mx) mx = s[j];
        }
        double l = 0.0;
        for (int64_t j = 0; j < n_kv; ++j) {
            if (s[j] == -INFINITY) continue;
            const double p = exp(s[j] - mx);
            l += p;
            orc_dequantize(kv_type, v + (hk * n_kv + j) * rb, vr, D);
            for (int64_t d = 0; d < D; ++d) acc[d] += p * (double)vr[d];
        }
        for (int64_t d = 0; d < D; ++d) out[h * D + d] = l > 0.0 ? (float)(acc[d] / l) : 0.0f;
        free(qq);
        free(s);
        free(acc);
        free(vr);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------------
 * BitNet I2_S
 * ---------------------------------------------------------------------------------------------------------------- */

/* quantize_activation_int8 (llama_bitnet_core.cpp:914-926): max_abs starts at 1e-7, scale = 127/max_abs,
 * q = clamp(round-half-away(x * scale), -127, 127); returns 1/scale (the dequantization factor). One row. */
float orc_i2s_quantize_act(const float *x, int8_t *q, int64_t n) {
    float max_abs = 1e-7f;
    for (int64_t i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > max_abs) max_abs = a;
    }
    const float scale = 127.0f / max_abs;
    for (int64_t i = 0; i < n; ++i) {
        int v = (int)roundf(x[i] * scale);
        if (v > 127) v = 127;
        if (v < -127) v = -127;
        q[i] = (int8_t)v;
    }
    return 1.0f / scale;
}

/* ggml_vec_dot_i2_i8_s scalar branch (ggml_bitnet_mad.cpp:191-231) for one row: 128-weight blocks of 32 bytes, byte
 * k of a block holds weights k, 32+k, 64+k, 96+k in bits 7-6, 5-4, 3-2, 1-0; weight value = code - 1. Returns the
 * exact integer sum; blk (may be NULL) receives the int32 sum of each 128-weight block. */
int64_t orc_i2s_dot_row(int64_t k, const uint8_t *w, const int8_t *q, int32_t *blk) {
    int64_t total = 0;
    for (int64_t b = 0; b < k / QK_I2S; ++b) {
        const uint8_t *pw = w + b * 32;
        const int8_t *pq = q + b * QK_I2S;
        int32_t s = 0;
        for (int j = 0; j < 32; ++j) {
            const int c0 = (pw[j] >> 6) & 3, c1 = (pw[j] >> 4) & 3, c2 = (pw[j] >> 2) & 3, c3 = pw[j] & 3;
            s += (c0 - 1) * pq[j] + (c1 - 1) * pq[32 + j] + (c2 - 1) * pq[64 + j] + (c3 - 1) * pq[96 + j];
        }
        if (blk) blk[b] = s;
        total += s;
    }
    return total;
}

/* bitnet_gemv for I2_S (llama_bitnet_core.cpp:928-941): out[r] = (float)sumi_r * (act_dequant * weight_scale).
 * W [n_rows][k/4 bytes]; q int8 [m][k] with one dequantization factor per activation row (batch m).
 * out [m][n_rows]; sums (may be NULL) int64 [m][n_rows]. OpenMP over rows. */
void orc_i2s_gemv(const uint8_t *w, int64_t n_rows, int64_t k, const int8_t *q, const float *act_dequant, int64_t m,
                  float weight_scale, float *out, int64_t *sums) {
    for (int64_t c = 0; c < m; ++c) {
        const float total_scale = act_dequant[c] * weight_scale;
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < n_rows; ++r) {
            const int64_t s = orc_i2s_dot_row(k, w + r * (k / 4), q + c * k, NULL);
            if (sums) sums[c * n_rows + r] = s;
            out[c * n_rows + r] = (float)s * total_scale;
        }
    }
}

/* I2_S dequantization as the BitNet reference decoder (test_phase0_i2s_proof.c:150-190): code 0 -> -1, 1 -> 0,
 * 2 -> +1, 3 -> 0, times scale; n need not be a multiple of 128 (last block partial). */
void orc_i2s_dequantize(const uint8_t *w, float scale, int64_t n, float *y) {
    static const float map[4] = {-1.0f, 0.0f, 1.0f, 0.0f};
    for (int64_t i = 0; i < n; ++i) {
        const int64_t b = i / QK_I2S, r = i % QK_I2S, g = r / 32, lane = r % 32;
        const int c = (w[b * 32 + lane] >> (6 - 2 * g)) & 3;
        y[i] = scale * map[c];
    }
}

/* tensor scale of an I2_S tensor: the f32 at byte offset n_rows * k / 4 (amuda_gguf.c:659-681). */
float orc_i2s_trailer_scale(const uint8_t *tensor, int64_t n_rows, int64_t k) {
    float s;
    memcpy(&s, tensor + n_rows * (k / 4), 4);
    return s;
}

/* ------------------------------------------------------------------------------------------------------------------
 * BitNet b1.58 token step of the CPU path (llama_bitnet_core.cpp:1186-1300), the arithmetic the reference's GPU
 * engine (ac_bitnet_engine.cpp) and this build's engine follow. Non-NEON branches: sums are sequential f32.
 * ---------------------------------------------------------------------------------------------------------------- */

/* rms_norm (:886-912), F32 weight or none: scale = 1 / sqrt(sum x^2 / dim + eps), out = x * scale * w. */
void orc_bitnet_rms_norm(float *out, const float *x, const float *w, int64_t dim, float eps) {
    float sum_sq = 0.0f;
    for (int64_t i = 0; i < dim; ++i) sum_sq += x[i] * x[i];
    const float scale = 1.0f / sqrtf(sum_sq / (float)dim + eps);
    for (int64_t i = 0; i < dim; ++i) out[i] = w ? x[i] * scale * w[i] : x[i] * scale;
}

/* bitnet_gemv for an I2_S weight (:928-940): out[r] = float(isum_r) * (dequant * weight_scale). */
static void bitnet_i2s_gemv(float *out, const uint8_t *w, const int8_t *q, float dequant, int64_t in_dim,
                            int64_t out_dim, float weight_scale) {
    const float total = dequant * weight_scale;
    for (int64_t r = 0; r < out_dim; ++r) out[r] = (float)orc_i2s_dot_row(in_dim, w + r * (in_dim / 4), q, NULL) * total;
}

/* bitnet_gemv for an F16 weight, scalar branch (:992-995): out[r] = sum_c f16(w[r][c]) * x[c], sequential f32. */
void orc_bitnet_gemv_f16(float *out, const uint16_t *w, const float *x, int64_t in_dim, int64_t out_dim) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < out_dim; ++r) {
        float sum = 0.0f;
        const uint16_t *row = w + r * in_dim;
        for (int64_t c = 0; c < in_dim; ++c) sum += orc_fp16_to_fp32(row[c]) * x[c];
        out[r] = sum;
    }
}

/* apply_rope (:1006-1020): pairs (i, i + head_dim / 2), theta = pos / theta_base^(2i / head_dim). */
static void bitnet_rope(float *vec, int64_t pos, int64_t n_heads, int64_t head_dim, float theta_base) {
    const int64_t half = head_dim / 2;
    for (int64_t h = 0; h < n_heads; ++h) {
        float *hp = vec + h * head_dim;
        for (int64_t i = 0; i < half; ++i) {
            const float theta = (float)pos / powf(theta_base, (float)(2 * i) / (float)head_dim);
            const float c = cosf(theta), s = sinf(theta);
            const float v0 = hp[i], v1 = hp[i + half];
            hp[i] = v0 * c - v1 * s;
            hp[i + half] = v1 * c + v0 * s;
        }
    }
}

/* multi_head_attention (:1033-1082) over cache rows [n_ctx][n_kv_heads * head_dim] of one layer, keys 0 .. pos. */
void orc_bitnet_attention(float *out, const float *q, const float *kc, const float *vc, int64_t pos, int64_t n_heads,
                          int64_t n_kv_heads, int64_t head_dim) {
    const float inv_sqrt = 1.0f / sqrtf((float)head_dim);
    const int64_t G = n_heads / n_kv_heads, kv = n_kv_heads * head_dim;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(pos + 1));
    for (int64_t h = 0; h < n_heads; ++h) {
        const int64_t kh = h / G;
        const float *qh = q + h * head_dim;
        float max_score = -1e9f;
        for (int64_t p = 0; p <= pos; ++p) {
            const float *k = kc + p * kv + kh * head_dim;
            float dot = 0.0f;
            for (int64_t d = 0; d < head_dim; ++d) dot += qh[d] * k[d];
            scores[p] = dot * inv_sqrt;
            if (scores[p] > max_score) max_score = scores[p];
        }
        float sum_exp = 0.0f;
        for (int64_t p = 0; p <= pos; ++p) {
            scores[p] = expf(scores[p] - max_score);
            sum_exp += scores[p];
        }
        const float inv_sum = 1.0f / (sum_exp + 1e-9f);
        float *oh = out + h * head_dim;
        for (int64_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
        for (int64_t p = 0; p <= pos; ++p) {
            const float wgt = scores[p] * inv_sum;
            const float *v = vc + p * kv + kh * head_dim;
            for (int64_t d = 0; d < head_dim; ++d) oh[d] += wgt * v[d];
        }
    }
    free(scores);
}

/* One layer's tensors on the host (BitNetLayerWeights of the CPU path): F32 norms (sub norms may be NULL), I2_S
 * projections (out_rows * in_dim / 4 bytes) and their scales. */
typedef struct {
    const float *attn_norm, *attn_sub_norm, *ffn_norm, *ffn_sub_norm;
    const uint8_t *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    float scale_wq, scale_wk, scale_wv, scale_wo, scale_w_gate, scale_w_up, scale_w_down;
} OrcBitnetLayer;

/* bitnet_eval for one token at pos (:1186-1300): x [n_embd] in and out (the residual stream after the last layer);
 * caches [n_layers][n_ctx][n_kv_heads * head_dim] (row pos written here); logits (may be NULL): the final norm and
 * the F16 LM head [n_vocab][n_embd]. relu2: relu(g)^2 * u with ffn_sub_norm, else silu(g) * u. */
void orc_bitnet_token(const OrcBitnetLayer *layers, int64_t n_layers, int64_t n_embd, int64_t n_ffn, int64_t n_heads,
                      int64_t n_kv_heads, int64_t head_dim, int64_t n_ctx, float norm_eps, float rope_theta, int relu2,
                      float *k_cache, float *v_cache, int64_t pos, float *x, const float *out_norm,
                      const uint16_t *lm_head, int64_t n_vocab, float *logits) {
    const int64_t E = n_embd, F = n_ffn, kv = n_kv_heads * head_dim;
    const int64_t vmax = E > F ? E : F;
    float *xn = (float *)malloc(sizeof(float) * (size_t)vmax), *q = (float *)malloc(sizeof(float) * (size_t)E);
    float *k = (float *)malloc(sizeof(float) * (size_t)kv), *v = (float *)malloc(sizeof(float) * (size_t)kv);
    float *att = (float *)malloc(sizeof(float) * (size_t)E), *o = (float *)malloc(sizeof(float) * (size_t)E);
    float *g = (float *)malloc(sizeof(float) * (size_t)F), *u = (float *)malloc(sizeof(float) * (size_t)F);
    int8_t *q8 = (int8_t *)malloc((size_t)vmax);
    for (int64_t l = 0; l < n_layers; ++l) {
        const OrcBitnetLayer *L = layers + l;
        float *kc = k_cache + l * n_ctx * kv, *vc = v_cache + l * n_ctx * kv;
        orc_bitnet_rms_norm(xn, x, L->attn_norm, E, norm_eps);
        float dq = orc_i2s_quantize_act(xn, q8, E);
        bitnet_i2s_gemv(q, L->wq, q8, dq, E, E, L->scale_wq);
        bitnet_i2s_gemv(k, L->wk, q8, dq, E, kv, L->scale_wk);
        bitnet_i2s_gemv(v, L->wv, q8, dq, E, kv, L->scale_wv);
        bitnet_rope(q, pos, n_heads, head_dim, rope_theta);
        bitnet_rope(k, pos, n_kv_heads, head_dim, rope_theta);
        memcpy(kc + pos * kv, k, sizeof(float) * (size_t)kv);
        memcpy(vc + pos * kv, v, sizeof(float) * (size_t)kv);
        orc_bitnet_attention(att, q, kc, vc, pos, n_heads, n_kv_heads, head_dim);
        if (L->attn_sub_norm) orc_bitnet_rms_norm(att, att, L->attn_sub_norm, E, norm_eps);
        dq = orc_i2s_quantize_act(att, q8, E);
        bitnet_i2s_gemv(o, L->wo, q8, dq, E, E, L->scale_wo);
        for (int64_t i = 0; i < E; ++i) x[i] += o[i];
        orc_bitnet_rms_norm(xn, x, L->ffn_norm, E, norm_eps);
        dq = orc_i2s_quantize_act(xn, q8, E);
        bitnet_i2s_gemv(g, L->w_gate, q8, dq, E, F, L->scale_w_gate);
        bitnet_i2s_gemv(u, L->w_up, q8, dq, E, F, L->scale_w_up);
        for (int64_t i = 0; i < F; ++i) {
            if (relu2) {
                const float r = g[i] > 0.0f ? g[i] : 0.0f;
                g[i] = (r * r) * u[i];
            } else {
                g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
            }
        }
        if (L->ffn_sub_norm) orc_bitnet_rms_norm(g, g, L->ffn_sub_norm, F, norm_eps);
        dq = orc_i2s_quantize_act(g, q8, F);
        bitnet_i2s_gemv(o, L->w_down, q8, dq, F, E, L->scale_w_down);
        for (int64_t i = 0; i < E; ++i) x[i] += o[i];
    }
    if (logits) {
        orc_bitnet_rms_norm(xn, x, out_norm, E, norm_eps);
        orc_bitnet_gemv_f16(logits, lm_head, xn, E, n_vocab);
    }
    free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u); free(q8);
}
