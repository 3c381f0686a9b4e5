/* CPU baseline kernels for bench.py (test infrastructure: timed beside the GPU figures, never part of the product
 * path and not the parity checker -- ameva_oracle.c is). They restate, for x86-64 with AVX2/FMA/F16C, what ggml's
 * CPU backend does on the same hot path (ggml b8471, external to the reference tree):
 *   - vec_dot_q4_0_q8_0, AVX2 branch (ggml-cpu/arch/x86/quants.c): per 32-block, the 16 nibble bytes widened to 32
 *     bytes, minus 8, multiplied with the Q8_0 bytes by _mm256_maddubs_epi16 on |w| and sign(a, w), pairs summed by
 *     _mm256_madd_epi16, the 8 int32 converted to float and multiplied-added by d_w * d_a into 8 float lanes summed
 *     at the end;
 *   - flash attention decode over an f16 KV cache (ggml_compute_forward_flash_attn_ext_f16): per head q . k in f32
 *     from f16 rows, online softmax, V accumulated in f32.
 * Work split over threads with OpenMP. Values agree with the oracle to float rounding (the per-block sums are exact;
 * their float accumulation order differs; V accumulates in f32 where the oracle follows ggml's f16). */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QB_Q4_0 18 /* f16 d + 16 nibble bytes */
#define QB_Q8_0 34 /* f16 d + 32 int8 */

static inline float h2f(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return _cvtsh_ss(h);
}

static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

static float dot_q4_0_q8_0(int64_t nb, const uint8_t *w, const uint8_t *a) {
    const __m256i lo4 = _mm256_set1_epi8(0x0F), off8 = _mm256_set1_epi8(8), ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t *wb = w + b * QB_Q4_0, *ab = a + b * QB_Q8_0;
        const __m128i q = _mm_loadu_si128((const __m128i *)(wb + 2));
        /* bytes 0..15: low nibbles (elements 0..15), 16..31: high nibbles (elements 16..31) */
        __m256i x = _mm256_set_m128i(_mm_srli_epi16(q, 4), q);
        x = _mm256_sub_epi8(_mm256_and_si256(x, lo4), off8);
        const __m256i y = _mm256_loadu_si256((const __m256i *)(ab + 2));
        const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(x, x), _mm256_sign_epi8(y, x));
        const __m256i p32 = _mm256_madd_epi16(p16, ones);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(h2f(wb) * h2f(ab)), _mm256_cvtepi32_ps(p32), acc);
    }
    return hsum8(acc);
}

/* dst[c][r] = dot(W row r, activation row c): W Q4_0 [n_rows][k/32], activations Q8_0 [m][k/32]. Work items are
 * (16-row block, 32-token block) pairs split over threads: a weight block (37 KB at k = 4096) and an activation block
 * (139 KB) stay in the core's caches while the 512 dots between them run. */
void cpu_mul_mat_q4_0(const uint8_t *w, int64_t n_rows, int64_t k, const uint8_t *a, int64_t m, float *dst) {
    const int64_t nb = k / 32, RB = 16, CB = 32;
    const int64_t nrb = (n_rows + RB - 1) / RB, ncb = (m + CB - 1) / CB;
#pragma omp parallel for schedule(static)
    for (int64_t it = 0; it < nrb * ncb; ++it) {
        const int64_t r0 = (it / ncb) * RB, c0 = (it % ncb) * CB;
        const int64_t r1 = r0 + RB < n_rows ? r0 + RB : n_rows, c1 = c0 + CB < m ? c0 + CB : m;
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t c = c0; c < c1; ++c)
                dst[c * n_rows + r] = dot_q4_0_q8_0(nb, w + r * nb * QB_Q4_0, a + c * nb * QB_Q8_0);
    }
}

/* out[h][D] = softmax(scale * q_h . K^T) V for one query position over n_kv keys: q f32 [n_head][D], K/V f16 rows
 * [n_kv][n_head_kv][D] (head h reads KV head h / (n_head / n_head_kv)). Heads split over threads. */
void cpu_flash_attn_decode_f16(const float *q, const uint16_t *k, const uint16_t *v, float *out, int64_t n_head,
                               int64_t n_head_kv, int64_t n_kv, int64_t D, float scale) {
    const int64_t G = n_head / n_head_kv;
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < n_head; ++h) {
        const int64_t hk = h / G;
        const float *qh = q + h * D;
        float acc[256];
        float m = -INFINITY, l = 0.0f;
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int64_t t = 0; t < n_kv; ++t) {
            const uint16_t *kr = k + (t * n_head_kv + hk) * D, *vr = v + (t * n_head_kv + hk) * D;
            __m256 s8 = _mm256_setzero_ps();
            for (int64_t d = 0; d < D; d += 8)
                s8 = _mm256_fmadd_ps(_mm256_loadu_ps(qh + d), _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(kr + d))), s8);
            const float s = hsum8(s8) * scale;
            const float mn = s > m ? s : m;
            const float f = expf(m - mn), p = expf(s - mn);
            l = l * f + p;
            m = mn;
            const __m256 fv = _mm256_set1_ps(f), pv = _mm256_set1_ps(p);
            for (int64_t d = 0; d < D; d += 8) {
                const __m256 vv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(vr + d)));
                _mm256_storeu_ps(acc + d, _mm256_fmadd_ps(pv, vv, _mm256_mul_ps(_mm256_loadu_ps(acc + d), fv)));
            }
        }
        for (int64_t d = 0; d < D; ++d) out[h * D + d] = acc[d] / l;
    }
}

int cpu_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
