// FLASH_ATTN_EXT for decode (one query position) over an f16 KV cache, split along the sequence (flash decoding).
//
// Role of ameva_flash_attn.comp (split_keys > 0) + ameva_fa_combine.comp (reference): softmax(scale * q k^T + mask) v
// per head; head h reads KV head h / G (G = n_head / n_head_kv), and the G query heads of a KV head share every K and
// V load. ggml's CPU kernel rounds q to f16 before the dot with f16 K; so does this one. Scores, probabilities and
// accumulators are f32.
//
// Pass 1 (k_fa_split): one workgroup of 256 per (key split, KV head). 16 lanes read one 256-byte K row (8 halves
// each) and form the G partial dots, reduced over the 16 lanes; the split's scores go to LDS; per head the split
// maximum m and l = sum exp(s - m); then each wave accumulates V rows (a lane owns 2 of the 128 dims) for its keys,
// and the 4 waves' accumulators are summed in LDS. The partial (m, l, acc[D]) of every (head, split) goes to the
// workspace. Pass 2 (k_fa_combine): per head M = max m_z, L = sum l_z e^(m_z - M), out = sum acc_z e^(m_z - M) / L.
#include "amv_common.h"

#define FA_D 128
#define FA_MAX_SPLIT 256  // keys per split at most

template <int G>
__global__ __launch_bounds__(256) void k_fa_split(const float* __restrict__ q, const uint16_t* __restrict__ k,
                                                 const uint16_t* __restrict__ v, const uint16_t* __restrict__ mask,
                                                 float* __restrict__ part, int n_kv, int64_t k_row, int64_t k_head,
                                                 int64_t v_row, int64_t v_head, int split_len, int n_split,
                                                 float scale) {
    __shared__ float sS[G][FA_MAX_SPLIT];
    __shared__ float sRed[4][G][FA_D];
    __shared__ float sM[G], sL[G];
    const int split = blockIdx.x, hk = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int kb = split * split_len;
    const int ke = min(n_kv, kb + split_len);
    const int nk = ke - kb;  // >= 1
    const uint16_t* kh = k + (size_t)hk * k_head;
    const uint16_t* vh = v + (size_t)hk * v_head;

    // q of the G heads, 8 dims per lane (dims 8 * (lane & 15) + e), rounded to f16 as ggml does
    const int d8 = 8 * (lane & 15);
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float4* qp = reinterpret_cast<const float4*>(q + (size_t)(hk * G + g) * FA_D + d8);
        const float4 a = qp[0], b = qp[1];
        const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[g][e] = amv_h2f(amv_f2h(t[e]));
    }
    // scores: key kb + 16 it + 4 wv + (lane >> 4)
    for (int base = 0; base < nk; base += 16) {
        const int kk = base + 4 * wv + (lane >> 4);
        const int kc = min(kk, nk - 1);
        const uint4 kr = *reinterpret_cast<const uint4*>(kh + (size_t)(kb + kc) * k_row + d8);
        const uint32_t kw[4] = {kr.x, kr.y, kr.z, kr.w};
        float kf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kf[2 * e] = amv_h2f(kw[e] & 0xFFFFu);
            kf[2 * e + 1] = amv_h2f(kw[e] >> 16);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s = fmaf(qv[g][e], kf[e], s);
            s += __shfl_xor(s, 1, AMV_WAVE);
            s += __shfl_xor(s, 2, AMV_WAVE);
            s += __shfl_xor(s, 4, AMV_WAVE);
            s += __shfl_xor(s, 8, AMV_WAVE);
            if ((lane & 15) == 0 && kk < nk) {
                float x = s * scale;
                if (mask) x += amv_h2f(mask[kb + kk]);
                sS[g][kk] = x;
            }
        }
    }
    __syncthreads();
    // per head: split maximum and sum of exp (wave g handles head g, g < G <= 8: waves loop over heads)
    for (int g = wv; g < G; g += 4) {
        float m = -INFINITY;
        for (int i = lane; i < nk; i += 64) m = fmaxf(m, sS[g][i]);
        m = amv_wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < nk; i += 64) {
            const float p = (m == -INFINITY) ? 0.0f : expf(sS[g][i] - m);
            sS[g][i] = p;
            l += p;
        }
        l = amv_wave_sum(l);
        if (lane == 0) {
            sM[g] = m;
            sL[g] = l;
        }
    }
    __syncthreads();
    // V accumulation: wave wv takes keys wv, wv + 4, ...; lane owns dims 2 lane, 2 lane + 1
    float acc[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.0f;
    for (int i = wv; i < nk; i += 4) {
        const uint32_t vv = *reinterpret_cast<const uint32_t*>(vh + (size_t)(kb + i) * v_row + 2 * lane);
        const float v0 = amv_h2f(vv & 0xFFFFu), v1 = amv_h2f(vv >> 16);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float p = sS[g][i];
            acc[g][0] = fmaf(p, v0, acc[g][0]);
            acc[g][1] = fmaf(p, v1, acc[g][1]);
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        sRed[wv][g][2 * lane] = acc[g][0];
        sRed[wv][g][2 * lane + 1] = acc[g][1];
    }
    __syncthreads();
    for (int e = tid; e < G * FA_D; e += 256) {
        const int g = e / FA_D, d = e % FA_D;
        const float a = (sRed[0][g][d] + sRed[1][g][d]) + (sRed[2][g][d] + sRed[3][g][d]);
        float* pp = part + ((size_t)(hk * G + g) * n_split + split) * (FA_D + 2);
        pp[2 + d] = a;
        if (d == 0) {
            pp[0] = sM[g];
            pp[1] = sL[g];
        }
    }
}

__global__ __launch_bounds__(128) void k_fa_combine(const float* __restrict__ part, float* __restrict__ out,
                                                   int n_split) {
    const int h = blockIdx.x, d = threadIdx.x;
    const float* ph = part + (size_t)h * n_split * (FA_D + 2);
    float M = -INFINITY;
    for (int z = 0; z < n_split; ++z) M = fmaxf(M, ph[(size_t)z * (FA_D + 2)]);
    float L = 0.0f, a = 0.0f;
    for (int z = 0; z < n_split; ++z) {
        const float m = ph[(size_t)z * (FA_D + 2)];
        if (m == -INFINITY) continue;
        const float f = expf(m - M);
        L = fmaf(ph[(size_t)z * (FA_D + 2) + 1], f, L);
        a = fmaf(ph[(size_t)z * (FA_D + 2) + 2 + d], f, a);
    }
    out[(size_t)h * FA_D + d] = L == 0.0f ? 0.0f : a / L;
}

static int fa_split_len(int64_t n_kv, int64_t n_head_kv) {
    // enough (split, KV head) workgroups to cover the 256 CUs twice, 16..256 keys per split
    int64_t s = (n_kv * n_head_kv + 511) / 512;
    s = ((s + 15) / 16) * 16;
    if (s < 16) s = 16;
    if (s > FA_MAX_SPLIT) s = FA_MAX_SPLIT;
    return (int)s;
}

extern "C" int64_t amv_flash_attn_workspace_bytes(int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D) {
    if (n_head <= 0 || n_head_kv <= 0 || n_kv <= 0 || D != FA_D) return -1;
    const int64_t sl = fa_split_len(n_kv, n_head_kv);
    const int64_t n_split = (n_kv + sl - 1) / sl;
    return n_head * n_split * (D + 2) * 4;
}

extern "C" int amv_flash_attn_decode(const float* q, const void* k, const void* v, const void* mask, float* out,
                                     int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D, int64_t k_row,
                                     int64_t k_head, int64_t v_row, int64_t v_head, float scale, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    AMV_REQUIRE(q && k && v && out && workspace, "amv_flash_attn_decode: null pointer");
    AMV_REQUIRE(D == FA_D, "amv_flash_attn_decode: head size %lld not supported (128 is)", (long long)D);
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0, "amv_flash_attn_decode: bad head counts");
    const int64_t G = n_head / n_head_kv;
    AMV_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "amv_flash_attn_decode: GQA group %lld not supported", (long long)G);
    AMV_REQUIRE(n_kv > 0 && n_kv <= INT32_MAX, "amv_flash_attn_decode: bad n_kv");
    AMV_REQUIRE(n_head_kv <= 65535, "amv_flash_attn_decode: too many KV heads");
    AMV_REQUIRE(k_row >= D && v_row >= D && k_row % 8 == 0 && v_row % 8 == 0 && k_head % 8 == 0 && v_head % 8 == 0 &&
                    k_head >= 0 && v_head >= 0,
                "amv_flash_attn_decode: K/V strides must be >= D and multiples of 8 elements");
    AMV_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 &&
                    ((uintptr_t)workspace & 15) == 0,
                "amv_flash_attn_decode: buffers must be 16-byte aligned");
    const int64_t need = amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv, D);
    AMV_REQUIRE(workspace_bytes >= need, "amv_flash_attn_decode: workspace %lld < %lld bytes", (long long)workspace_bytes,
                (long long)need);
    const int sl = fa_split_len(n_kv, n_head_kv);
    const int n_split = (int)((n_kv + sl - 1) / sl);
    hipStream_t st = amv_stream(stream);
    const dim3 grid(n_split, (unsigned)n_head_kv);
    float* part = (float*)workspace;
    const uint16_t* kk = (const uint16_t*)k;
    const uint16_t* vv = (const uint16_t*)v;
    const uint16_t* mm = (const uint16_t*)mask;
#define FA_LAUNCH(GG)                                                                                                   \
    hipLaunchKernelGGL(k_fa_split<GG>, grid, dim3(256), 0, st, q, kk, vv, mm, part, (int)n_kv, k_row, k_head, v_row,  \
                       v_head, sl, n_split, scale)
    switch (G) {
    case 1: FA_LAUNCH(1); break;
    case 2: FA_LAUNCH(2); break;
    case 4: FA_LAUNCH(4); break;
    default: FA_LAUNCH(8); break;
    }
#undef FA_LAUNCH
    hipLaunchKernelGGL(k_fa_combine, dim3((unsigned)n_head), dim3(FA_D), 0, st, part, out, n_split);
    return amv_check_launch("amv_flash_attn_decode");
}
