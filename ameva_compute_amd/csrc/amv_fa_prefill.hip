// FLASH_ATTN_EXT over many query positions (prefill) on the f16 matrix cores of MI355X.
//
// Role of ameva_flash_attn.comp for a prompt (reference: enc_flash_attn ggml-ameva.cpp:4204-4284 with ne[1] > 1):
// out[t][h] = softmax(scale * q_t k^T + mask_t) v over the keys query t may see. ggml's CPU kernel rounds q to f16
// before the dot with the f16 K; so does this one. Scores, softmax and accumulators are f32; the probabilities enter
// the P V product as f16 (the CPU accumulates V in f16 instead).
//
// One workgroup of 4 waves per (head, 64 consecutive queries); wave w owns queries 16 w .. 16 w + 15 of the tile and
// runs flash attention over blocks of 64 keys with v_mfma_f32_16x16x16f16:
//   S^T (16 keys x 16 queries) = K (16 keys x 128) . Q^T, accumulated over 8 steps of 16 dims. The reduction order
//   of the dims is free, so lane group g takes dims 32 j + 8 g .. + 7 of both K and Q for steps 2 j, 2 j + 1: every
//   lane reads 16 contiguous bytes of its K row. In the result lane (g, c) holds S[query c][keys 4 g .. 4 g + 3].
//   O^T (16 dims x 16 queries) += V^T (16 dims x 16 keys) . P^T: the P^T operand is exactly the S^T result layout,
//   so the probabilities never move between lanes; V^T comes from LDS, where the workgroup stages the key block's
//   V rows transposed ([dim][key]).
// Online softmax per query: the block maximum over the lane's 16 scores and the 4 lanes of the query (xor 16, 32),
// rescale of l and O by exp(m_old - m_new). Causal tiles stop at the last key their last query may see.
#include "amv_common.h"

#define FP_D 128
#define FP_KB 64                 // keys per block
#define FP_VT (FP_KB + 8)        // LDS row of V^T in halves (padded against bank conflicts)

typedef _Float16 fp_h4 __attribute__((ext_vector_type(4)));
typedef float fp_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ fp_h4 fp_h4_of(uint32_t lo, uint32_t hi) {
    const uint2 u = make_uint2(lo, hi);
    return __builtin_bit_cast(fp_h4, u);
}

__global__ __launch_bounds__(256) void k_fa_prefill(const float* __restrict__ q, int64_t q_ts, int64_t q_hs,
                                                   const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                   const uint16_t* __restrict__ mask, int64_t mask_stride,
                                                   float* __restrict__ out, int n_tok, int n_head, int G, int n_kv,
                                                   int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head,
                                                   float scale, int64_t pos0) {
    __shared__ uint16_t vt[FP_D * FP_VT];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
    const int h = blockIdx.y, hk = h / G;
    const int qi = blockIdx.x * 64 + 16 * w + c;  // this lane's query (column of S^T and O^T)
    const int qc = min(qi, n_tok - 1);

    // Q^T operand, f16: qb[2 j + e] = q[qi][32 j + 8 g + 4 e .. + 3]
    fp_h4 qb[8];
    {
        const float* qr = q + (int64_t)qc * q_ts + (int64_t)h * q_hs;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float4 a = *reinterpret_cast<const float4*>(qr + 32 * j + 8 * g + 4 * e);
                fp_h4 t;
                t.x = (_Float16)a.x;
                t.y = (_Float16)a.y;
                t.z = (_Float16)a.z;
                t.w = (_Float16)a.w;
                qb[2 * j + e] = t;
            }
        }
    }
    // keys this tile needs: up to the last key its last query may see
    int kend = n_kv;
    if (pos0 >= 0) kend = (int)min((int64_t)kend, pos0 + min(blockIdx.x * 64 + 63, n_tok - 1) + 1);
    const int nblk = (kend + FP_KB - 1) / FP_KB;
    const int64_t qlim = pos0 >= 0 ? pos0 + qi : (int64_t)n_kv;  // last key this query may see (causal)

    const uint16_t* kh = k + (int64_t)hk * k_head;
    const uint16_t* vh = v + (int64_t)hk * v_head;
    float m = -INFINITY, l = 0.0f;
    fp_f4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = fp_f4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int b = 0; b < nblk; ++b) {
        const int kb0 = b * FP_KB;
        // K rows of the block for the S^T operand (issued before the V staging)
        uint4 kr[4][4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint16_t* row = kh + (int64_t)min(kb0 + 16 * t + c, n_kv - 1) * k_row;
#pragma unroll
            for (int j = 0; j < 4; ++j) kr[t][j] = *reinterpret_cast<const uint4*>(row + 32 * j + 8 * g);
        }
        // stage V^T of the block: thread (key kk = tid % 64, dims 8 s .. 8 s + 7), s = 4 it + tid / 64
        __syncthreads();  // the previous block's readers are done
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int kk = tid & 63, s8 = 8 * (4 * it + (tid >> 6));
            const int key = kb0 + kk;
            uint4 val = make_uint4(0u, 0u, 0u, 0u);
            if (key < n_kv) val = *reinterpret_cast<const uint4*>(vh + (int64_t)key * v_row + s8);
            const uint32_t wv[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vt[(s8 + 2 * e) * FP_VT + kk] = (uint16_t)(wv[e] & 0xFFFFu);
                vt[(s8 + 2 * e + 1) * FP_VT + kk] = (uint16_t)(wv[e] >> 16);
            }
        }
        // S^T = K Q^T for the 4 tiles of 16 keys
        fp_f4 s[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            fp_f4 acc = fp_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(fp_h4_of(kr[t][j].x, kr[t][j].y), qb[2 * j], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(fp_h4_of(kr[t][j].z, kr[t][j].w), qb[2 * j + 1], acc, 0,
                                                            0, 0);
            }
            s[t] = acc;  // s[t][i] = S[query qi][key kb0 + 16 t + 4 g + i]
        }
        // scale, mask, causal limit; block maximum per query
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kb0 + 16 * t + 4 * g + i;
                float x = s[t][i] * scale;
                if (mask) x += amv_h2f(mask[(int64_t)qc * mask_stride + min(key, n_kv - 1)]);
                if (key >= n_kv || key > qlim) x = -INFINITY;
                s[t][i] = x;
                mx = fmaxf(mx, x);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, AMV_WAVE));
        mx = fmaxf(mx, __shfl_xor(mx, 32, AMV_WAVE));
        const float m_new = fmaxf(m, mx);
        const bool none = m_new == -INFINITY;  // nothing visible yet for this query
        const float alpha = none ? 1.0f : expf(m - m_new);
        float rs = 0.0f;
        fp_h4 p[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            fp_h4 pt;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = none ? 0.0f : expf(s[t][i] - m_new);
                rs += e;
                pt[i] = (_Float16)e;
            }
            p[t] = pt;
        }
        rs += __shfl_xor(rs, 16, AMV_WAVE);
        rs += __shfl_xor(rs, 32, AMV_WAVE);
        l = l * alpha + rs;
        m = m_new;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
        __syncthreads();  // V^T staged
        // O^T += V^T P^T
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const fp_h4 a = *reinterpret_cast<const fp_h4*>(vt + (16 * dt + c) * FP_VT + 16 * t + 4 * g);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, p[t], o[dt], 0, 0, 0);
            }
        }
    }
    if (qi < n_tok) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float* orow = out + ((int64_t)qi * n_head + h) * FP_D;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
            *reinterpret_cast<float4*>(orow + 16 * dt + 4 * g) =
                make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
    }
}

extern "C" int amv_flash_attn_prefill(const float* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k,
                                      const void* v, const void* mask, int64_t mask_stride, float* out, int64_t n_tok,
                                      int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D, int64_t k_row,
                                      int64_t k_head, int64_t v_row, int64_t v_head, float scale, int64_t causal_pos0,
                                      void* stream) {
    AMV_REQUIRE(q && k && v && out, "amv_flash_attn_prefill: null pointer");
    AMV_REQUIRE(D == FP_D, "amv_flash_attn_prefill: head size %lld not supported (128 is)", (long long)D);
    AMV_REQUIRE(n_tok > 0 && n_kv > 0 && n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0,
                "amv_flash_attn_prefill: bad shape");
    AMV_REQUIRE(n_tok <= (int64_t)1 << 24 && n_kv <= (int64_t)1 << 24 && n_head <= 65535,
                "amv_flash_attn_prefill: shape too large");
    AMV_REQUIRE(((uintptr_t)q & 15) == 0 && q_tok_stride % 4 == 0 && q_head_stride % 4 == 0,
                "amv_flash_attn_prefill: q rows must be 16-byte aligned");
    AMV_REQUIRE(((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 && k_row % 8 == 0 && k_head % 8 == 0 &&
                    v_row % 8 == 0 && v_head % 8 == 0,
                "amv_flash_attn_prefill: K/V rows must be 16-byte aligned");
    AMV_REQUIRE(((uintptr_t)out & 15) == 0, "amv_flash_attn_prefill: out must be 16-byte aligned");
    AMV_REQUIRE(mask == nullptr || mask_stride >= n_kv, "amv_flash_attn_prefill: mask stride %lld < n_kv",
                (long long)mask_stride);
    const dim3 grid((unsigned)((n_tok + 63) / 64), (unsigned)n_head);
    hipLaunchKernelGGL(k_fa_prefill, grid, dim3(256), 0, amv_stream(stream), q, q_tok_stride, q_head_stride,
                       (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)mask, mask_stride, out, (int)n_tok,
                       (int)n_head, (int)(n_head / n_head_kv), (int)n_kv, k_row, k_head, v_row, v_head, scale,
                       causal_pos0);
    return amv_check_launch("amv_flash_attn_prefill");
}
