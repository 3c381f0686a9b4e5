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

// One workgroup per (split of 4 * KPW keys, KV head); each of its 4 waves owns KPW consecutive keys and works alone:
// a 16-lane group owns keys 4 u + grp (u < KPW / 4) and reads 16 B of every K and V row of them (all K and V loads of
// the wave are issued before the first is used); the G scores of a key are reduced over its 16 lanes; the wave's
// maximum, probabilities, l and P V stay in registers. The 4 wave partials are merged once through LDS.
template <int G, int KPW>
__global__ __launch_bounds__(256) void k_fa_split(const float* __restrict__ q, const uint16_t* __restrict__ k,
                                                 const uint16_t* __restrict__ v, const uint16_t* __restrict__ mask,
                                                 float* __restrict__ part, int n_kv, int64_t k_row, int64_t k_head,
                                                 int64_t v_row, int64_t v_head, int n_split, float scale) {
    constexpr int U = KPW / 4;
    __shared__ float sAcc[4][4][G][FA_D];  // [wave][lane group][head][dim]: partial P V of 4 keys per step
    __shared__ float sM[4][G], sL[4][G];
    const int split = blockIdx.x, hk = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int grp = lane >> 4, d8 = 8 * (lane & 15);
    const int kw0 = split * 4 * KPW + wv * KPW;  // first key of this wave
    const uint16_t* kh = k + (size_t)hk * k_head;
    const uint16_t* vh = v + (size_t)hk * v_head;

    uint4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = min(kw0 + 4 * u + grp, n_kv - 1);
        kr[u] = *reinterpret_cast<const uint4*>(kh + (size_t)i * k_row + d8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = min(kw0 + 4 * u + grp, n_kv - 1);
        vr[u] = *reinterpret_cast<const uint4*>(vh + (size_t)i * v_row + d8);
    }
    // q of the G heads, 8 dims per lane, rounded to f16 as ggml does
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float4* qp = reinterpret_cast<const float4*>(q + (size_t)(hk * G + g) * FA_D + d8);
        const float4 a = qp[0], b = qp[1];
        const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[g][e] = amv_round_f16(t[e]);
    }
    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t kw[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
        float kf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kf[2 * e] = amv_h2f(kw[e] & 0xFFFFu);
            kf[2 * e + 1] = amv_h2f(kw[e] >> 16);
        }
        const int i = kw0 + 4 * u + grp;
        const float mk = (i < n_kv) ? (mask ? amv_h2f(mask[i]) : 0.0f) : -INFINITY;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d = fmaf(qv[g][e], kf[e], d);
            d = amv_row16_sum(d);
            s[u][g] = (mk == -INFINITY) ? -INFINITY : d * scale + mk;
        }
    }
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mm = s[0][g];
#pragma unroll
        for (int u = 1; u < U; ++u) mm = fmaxf(mm, s[u][g]);
        mm = fmaxf(mm, __shfl_xor(mm, 16, AMV_WAVE));
        mm = fmaxf(mm, __shfl_xor(mm, 32, AMV_WAVE));
        m[g] = mm;
        float ll = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float p = (mm == -INFINITY) ? 0.0f : expf(s[u][g] - mm);
            s[u][g] = p;
            ll += p;
        }
        ll += __shfl_xor(ll, 16, AMV_WAVE);
        ll += __shfl_xor(ll, 32, AMV_WAVE);
        l[g] = ll;  // the 16 lanes of a group each counted their group's keys once: same total in every lane
    }
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t vw[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
        float vf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vf[2 * e] = amv_h2f(vw[e] & 0xFFFFu);
            vf[2 * e + 1] = amv_h2f(vw[e] >> 16);
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(s[u][g], vf[e], acc[g][e]);
    }
    // the 4 lane groups of a wave share the wave's maximum, so their accumulators add; the sum is taken in the merge
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float4* dst = reinterpret_cast<float4*>(&sAcc[wv][grp][g][d8]);
        dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
        dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            sM[wv][g] = m[g];
            sL[wv][g] = l[g];
        }
    }
    __syncthreads();
    // merge the 4 wave partials of this workgroup
    for (int e = tid; e < G * FA_D; e += 256) {
        const int g = e / FA_D, d = e % FA_D;
        const float M = fmaxf(fmaxf(sM[0][g], sM[1][g]), fmaxf(sM[2][g], sM[3][g]));
        float a = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = (sM[w][g] == -INFINITY) ? 0.0f : expf(sM[w][g] - M);
            const float aw = (sAcc[w][0][g][d] + sAcc[w][1][g][d]) + (sAcc[w][2][g][d] + sAcc[w][3][g][d]);
            a = fmaf(aw, f, a);
            L = fmaf(sL[w][g], f, L);
        }
        float* pp = part + ((size_t)(hk * G + g) * n_split + split) * (FA_D + 2);
        pp[2 + d] = a;
        if (d == 0) {
            pp[0] = M;
            pp[1] = L;
        }
    }
}

// Merge of the splits: workgroup (head h, 32-dim chunk c); thread (dim dl, split group zg of 8). With aq != NULL the
// chunk (one 32-element block of the n_head x 128 output vector) is also quantized to Q8_0 for the next MUL_MAT.
#define FA_MAX_NSPLIT 1024
__global__ __launch_bounds__(256) void k_fa_combine(const float* __restrict__ part, float* __restrict__ out,
                                                   int n_split, int8_t* __restrict__ aq, int2* __restrict__ ameta,
                                                   int rule) {
    __shared__ float sw[FA_MAX_NSPLIT];
    __shared__ float sRedM[4], sRedL[4];
    __shared__ float sAcc[8][32];
    const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float* ph = part + (size_t)h * n_split * (FA_D + 2);
    float m = -INFINITY;
    for (int z = tid; z < n_split; z += 256) m = fmaxf(m, ph[(size_t)z * (FA_D + 2)]);
    m = amv_wave_max(m);
    if (lane == 0) sRedM[wv] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(sRedM[0], sRedM[1]), fmaxf(sRedM[2], sRedM[3]));
    float l = 0.0f;
    for (int z = tid; z < n_split; z += 256) {
        const float mz = ph[(size_t)z * (FA_D + 2)];
        const float wz = (mz == -INFINITY) ? 0.0f : expf(mz - M);
        sw[z] = wz;
        l = fmaf(ph[(size_t)z * (FA_D + 2) + 1], wz, l);
    }
    l = amv_wave_sum(l);
    if (lane == 0) sRedL[wv] = l;
    __syncthreads();
    const float L = (sRedL[0] + sRedL[1]) + (sRedL[2] + sRedL[3]);
    const int dl = tid & 31, zg = tid >> 5;
    const float* pa = ph + 2 + 32 * c + dl;
    float a0 = 0.0f, a1 = 0.0f;
    int z = zg;
    for (; z + 8 < n_split; z += 16) {
        a0 = fmaf(sw[z], pa[(size_t)z * (FA_D + 2)], a0);
        a1 = fmaf(sw[z + 8], pa[(size_t)(z + 8) * (FA_D + 2)], a1);
    }
    if (z < n_split) a0 = fmaf(sw[z], pa[(size_t)z * (FA_D + 2)], a0);
    sAcc[zg][dl] = a0 + a1;
    __syncthreads();
    if (tid < 32) {
        float o = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) o += sAcc[g][tid];
        o = L == 0.0f ? 0.0f : o / L;
        const size_t idx = (size_t)h * FA_D + 32 * c + tid;
        out[idx] = o;
        if (aq) amv_q8_0_lanes32(o, rule, tid, aq + (size_t)h * FA_D + 32 * c, ameta + (size_t)h * 4 + c);
    }
}

// keys per wave: 16, or 32 when 16 would leave more than 4 workgroups per CU (long contexts)
static int fa_kpw(int64_t n_kv, int64_t n_head_kv) { return (n_kv * n_head_kv) / (4 * 16) > 1024 ? 32 : 16; }

extern "C" int64_t amv_flash_attn_workspace_bytes(int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D) {
    if (n_head <= 0 || n_head_kv <= 0 || n_kv <= 0 || D != FA_D) return -1;
    const int64_t sl = 4 * fa_kpw(n_kv, n_head_kv);
    const int64_t n_split = (n_kv + sl - 1) / sl;
    return n_head * n_split * (D + 2) * 4;
}

extern "C" int amv_flash_attn_decode(const float* q, const void* k, const void* v, const void* mask, float* out,
                                     int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D, int64_t k_row,
                                     int64_t k_head, int64_t v_row, int64_t v_head, float scale, void* workspace,
                                     int64_t workspace_bytes, void* act, int rule, void* stream) {
    AMV_REQUIRE(q && k && v && out && workspace, "amv_flash_attn_decode: null pointer");
    AMV_REQUIRE(!act || ((uintptr_t)act & 15) == 0, "amv_flash_attn_decode: act must be 16-byte aligned");
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_flash_attn_decode: bad rule");
    AMV_REQUIRE(D == FA_D, "amv_flash_attn_decode: head size %lld not supported (128 is)", (long long)D);
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0, "amv_flash_attn_decode: bad head counts");
    const int64_t G = n_head / n_head_kv;
    AMV_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "amv_flash_attn_decode: GQA group %lld not supported", (long long)G);
    AMV_REQUIRE(n_kv > 0 && n_kv <= 128LL * FA_MAX_NSPLIT, "amv_flash_attn_decode: n_kv %lld out of range",
                (long long)n_kv);
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
    const int kpw = fa_kpw(n_kv, n_head_kv);
    const int n_split = (int)((n_kv + 4 * kpw - 1) / (4 * kpw));
    hipStream_t st = amv_stream(stream);
    const dim3 grid(n_split, (unsigned)n_head_kv);
    float* part = (float*)workspace;
    const uint16_t* kk = (const uint16_t*)k;
    const uint16_t* vv = (const uint16_t*)v;
    const uint16_t* mm = (const uint16_t*)mask;
#define FA_LAUNCH(GG, KK)                                                                                              \
    hipLaunchKernelGGL((k_fa_split<GG, KK>), grid, dim3(256), 0, st, q, kk, vv, mm, part, (int)n_kv, k_row, k_head,   \
                       v_row, v_head, n_split, scale)
#define FA_G(GG)                     \
    if (kpw == 16) FA_LAUNCH(GG, 16); \
    else FA_LAUNCH(GG, 32)
    switch (G) {
    case 1: FA_G(1); break;
    case 2: FA_G(2); break;
    case 4: FA_G(4); break;
    default: FA_G(8); break;
    }
#undef FA_G
#undef FA_LAUNCH
    int8_t* aq = act ? (int8_t*)act : nullptr;
    int2* ameta = act ? (int2*)((uint8_t*)act + n_head * D) : nullptr;
    hipLaunchKernelGGL(k_fa_combine, dim3((unsigned)n_head, FA_D / 32), dim3(256), 0, st, part, out, n_split, aq,
                       ameta, rule);
    return amv_check_launch("amv_flash_attn_decode");
}
