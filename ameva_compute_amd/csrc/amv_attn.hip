// FLASH_ATTN_EXT for decode (one query position) over an f16, Q8_0 or Q4_0 KV cache, split along the sequence
// (flash decoding).
//
// Role of ameva_flash_attn.comp (split_keys > 0) + ameva_fa_combine.comp (reference): softmax(scale * q k^T + mask) v
// per head; head h reads KV head h / G (G = n_head / n_head_kv), and the G query heads of a KV head share every K and
// V load. q meets K the way ggml's CPU kernel makes it: rounded to f16 for an f16 cache; for a Q8_0 / Q4_0 cache
// quantized to Q8_0 (K's vec_dot_type, with the chosen rounding rule) and dotted in exact integers per 32-block,
// score = sum_b float(isum_b) * (d_k * d_q) (vec_dot_q8_0_q8_0 / vec_dot_q4_0_q8_0). A quantized V row is dequantized
// exactly (q * d). Scores, probabilities and accumulators are f32.
//
// Pass 1 (k_fa_split): one workgroup of 4 waves per (key split, KV head); each wave owns KPW consecutive keys and
// works alone (16 lanes per 256-byte K/V row, G partial dots reduced over the 16 lanes, wave maximum, probabilities
// and P V in registers); the 4 wave partials meet once in LDS and the workgroup's (m, l, acc[D]) per head goes to
// the workspace. Pass 2 (fa_merge): per head M = max m_z, w_z = e^(m_z - M), L = sum l_z w_z,
// out = sum w_z acc_z / L, with the quantization of the output for the next MUL_MAT fused. The merge runs either
// as its own launch (k_fa_combine, one workgroup per head) or in the last workgroup of each KV head to finish its
// split (one launch per decode step); both use the same code, so their outputs are identical. On MI355X the second
// launch is the faster of the two at Llama shapes (a single merging workgroup per KV head sits on the critical path
// after the arrival).
#include "amv_common.h"

#include <map>
#include <mutex>

#define FA_D 128
#define FA_PS (FA_D + 4)        // floats per partial: m, l, 2 pad, acc[D] (16-byte aligned rows)
#define FA_MAX_NSPLIT 1024      // splits per head (n_kv <= 128 K keys)

// Merge of the split partials of the G heads of KV head hk by the 256 threads of a workgroup; sbuf holds at least
// G * (8 * FA_D + FA_MAX_NSPLIT) + G floats of LDS.
//   per head (one wave per head): M = max m_z, w_z = e^(m_z - M) (0 for an empty split), L = wave sum of l_z w_z;
//   acc: thread (float4 column c4 = t % 32, split group zg = t / 32) sums w_z acc_z over z = zg, zg + 8, ... in
//   order, the 8 groups are added in order through LDS; out = acc / L (0 when L = 0) and its activation blocks.
// The loads of both phases for the first 64 splits of up to 4 heads are issued together (one memory round trip for
// a context of up to 64 splits: 4096 keys).
template <int G>
__device__ __forceinline__ void fa_merge(const float* part, int n_split, int ns, int hk, float* __restrict__ out,
                                         const AmvActOut& act, float* sbuf, const int* n_kv_dev = nullptr,
                                         int n_kv_max = 0, int split_len = 1) {
    constexpr int GB = G < 4 ? G : 4;  // heads per batch of acc loads
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c4 = tid & 31, zg = tid >> 5;
    float* sAcc = sbuf;                    // [G][8][FA_D]
    float* sw = sbuf + G * 8 * FA_D;       // [G][FA_MAX_NSPLIT]
    float* sL = sw + G * FA_MAX_NSPLIT;    // [G]
    const float* ph0 = part + (size_t)hk * G * n_split * FA_PS;
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // The first loads do not depend on ns (which a caller may take from a key count in device memory): they read
    // the launch's splits up to n_split - 1, and a split past ns (whose partial this launch did not write) is
    // selected away, never multiplied. Unconditional loads of valid addresses: a conditional load would be turned
    // into a select of addresses with a stack zero, i.e. slow flat loads.
    // (m, l) first: loads complete in order, so the weights and L are computed while the acc rows still arrive
    float2 ml0[(G + 3) / 4];  // (m, l) of split lane of head wv + 4 j
#pragma unroll
    for (int j = 0; j < (G + 3) / 4; ++j) {
        const int g = min(wv + 4 * j, G - 1);
        ml0[j] = *reinterpret_cast<const float2*>(ph0 + ((size_t)g * n_split + min(lane, n_split - 1)) * FA_PS);
    }
    float4 va[GB][8];  // acc rows of splits zg + 8 i of heads 0 .. GB - 1
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int z = min(zg + 8 * i, n_split - 1);
            va[g][i] = *reinterpret_cast<const float4*>(ph0 + ((size_t)g * n_split + z) * FA_PS + 4 + 4 * c4);
        }
    // with n_kv_dev, ns comes from the key count in device memory, read only now that the loads above are issued
    asm volatile("" ::: "memory");
    if (n_kv_dev) ns = (max(0, min(*n_kv_dev, n_kv_max)) + split_len - 1) / split_len;
    if (ns == 0) {  // no keys: zero outputs
        for (int c = tid; c < G * (FA_D / 4); c += 256) {
            const float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            *reinterpret_cast<float4*>(out + (size_t)hk * G * FA_D + 4 * c) = zero4;
            if (act.type) amv_act_store4(act, hk * G * (FA_D / 4) + c, v);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < (G + 3) / 4; ++j) {
        const int g = wv + 4 * j;
        if (g >= G) break;  // uniform per wave
        const float* ph = ph0 + (size_t)g * n_split * FA_PS;
        const float m0r = ml0[j].x, l0 = ml0[j].y;
        const float m0 = lane < ns ? m0r : -INFINITY;
        float m = m0;
        for (int z = lane + 64; z < ns; z += 64) m = fmaxf(m, ph[(size_t)z * FA_PS]);
        const float M = amv_wave_max_u(m);
        float l = 0.0f;
        if (lane < ns) {
            const float w = (m0 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m0 - M);
            sw[g * FA_MAX_NSPLIT + lane] = w;
            l = fmaf(l0, w, l);
        }
        for (int z = lane + 64; z < ns; z += 64) {
            const float mz = ph[(size_t)z * FA_PS];
            const float w = (mz == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mz - M);
            sw[g * FA_MAX_NSPLIT + z] = w;
            l = fmaf(ph[(size_t)z * FA_PS + 1], w, l);
        }
        l = amv_wave_sum(l);
        if (lane == 0) sL[g] = l;
    }
    __syncthreads();
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += GB) {
#pragma unroll
        for (int gb = 0; gb < GB; ++gb) {
            const int g = g0 + gb;
            const float* pa = ph0 + (size_t)g * n_split * FA_PS + 4 + 4 * c4;
            if (g0 > 0) {  // the second batch of heads (G = 8)
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    va[gb][i] = *reinterpret_cast<const float4*>(pa + (size_t)min(zg + 8 * i, ns - 1) * FA_PS);
            }
            float4 a = zero4;
            for (int z0 = zg; z0 < ns; z0 += 64) {
                float4 v[8];
                float w[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int z = z0 + 8 * i;
                    v[i] = z0 == zg ? va[gb][i] : *reinterpret_cast<const float4*>(pa + (size_t)min(z, ns - 1) * FA_PS);
                    // a split this launch did not write: its bits masked to zero (an integer mask, not a select of
                    // values, which the compiler would turn into a select of addresses with a stack zero)
                    const uint32_t km = z < ns ? 0xFFFFFFFFu : 0u;
                    v[i] = make_float4(__uint_as_float(__float_as_uint(v[i].x) & km),
                                       __uint_as_float(__float_as_uint(v[i].y) & km),
                                       __uint_as_float(__float_as_uint(v[i].z) & km),
                                       __uint_as_float(__float_as_uint(v[i].w) & km));
                    w[i] = z < ns ? sw[g * FA_MAX_NSPLIT + z] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    a.x = fmaf(w[i], v[i].x, a.x);
                    a.y = fmaf(w[i], v[i].y, a.y);
                    a.z = fmaf(w[i], v[i].z, a.z);
                    a.w = fmaf(w[i], v[i].w, a.w);
                }
            }
            *reinterpret_cast<float4*>(sAcc + (g * 8 + zg) * FA_D + 4 * c4) = a;
        }
    }
    __syncthreads();
    // thread c < G * 32 owns float4 chunk c of the G heads' outputs (the chunks of a Q8_0 or, with G even, a Q8_K
    // block sit in consecutive lanes of one wave)
    for (int c = tid; c < G * (FA_D / 4); c += 256) {
        const int g = c / (FA_D / 4), d = 4 * (c % (FA_D / 4));
        const float L = sL[g];
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float t = 0.0f;
#pragma unroll
            for (int z = 0; z < 8; ++z) t += sAcc[(g * 8 + z) * FA_D + d + e];
            v[e] = L == 0.0f ? 0.0f : t / L;
        }
        *reinterpret_cast<float4*>(out + (size_t)(hk * G + g) * FA_D + d) = make_float4(v[0], v[1], v[2], v[3]);
        if (act.type) amv_act_store4(act, hk * G * (FA_D / 4) + c, v);
    }
}

// One workgroup per (split of 4 * KPW keys, KV head); each of its 4 waves owns KPW consecutive keys and works alone:
// a 16-lane group owns keys 4 u + grp (u < KPW / 4) and reads 16 B of every K and V row of them (all K and V loads of
// the wave are issued before the first is used); the G scores of a key are reduced over its 16 lanes; the wave's
// maximum, probabilities, l and P V stay in registers. The 4 wave partials are merged once through LDS.
// The key count is read from n_kv_dev when given (capped at the launch's n_kv); splits past it do nothing. FUSED: the
// last workgroup of each KV head to arrive merges the head's splits (fa_merge).
// cache element types of the split kernel
#define FA_F16 0
#define FA_Q8_0 1
#define FA_Q4_0 2
#define FA_F32 3  // the BitNet engine's cache (llama_bitnet_core.cpp:1022-1082): f32 q . k, no rounding of q

// A lane's slice of a K / V row: .a (and .b for an f32 row, whose 8 elements are 32 bytes).
struct FaRow {
    uint4 a, b;
};

// The slice of one K / V row a lane works on: lane l16 (0..15 of its 16-lane group) owns elements 8 l16 .. 8 l16 + 7.
// f32: those 32 bytes (.a, .b). f16: those 16 bytes. Q8_0 / Q4_0 (ggml blocks of 34 / 18 bytes): element offset o = 8 (l16 & 3) in block l16 / 4;
// .x, .y = the 8 int8 (Q8_0) or the 8 qs bytes whose low (o < 16) or high (o >= 16) nibbles are the elements (Q4_0),
// .z = the block's fp16 d. Quantized rows need only 2-byte alignment (halfword loads).
template <int KT>
__device__ __forceinline__ FaRow fa_row(const uint8_t* __restrict__ row, int l16) {
    if constexpr (KT == FA_F32) {
        const uint4* p = reinterpret_cast<const uint4*>(row + 32 * l16);
        return FaRow{amv_ld_stream(p), amv_ld_stream(p + 1)};
    } else if constexpr (KT == FA_F16) {
        return FaRow{amv_ld_stream(reinterpret_cast<const uint4*>(row + 16 * l16)), make_uint4(0u, 0u, 0u, 0u)};
    } else {
        constexpr int BB = KT == FA_Q8_0 ? 34 : 18;
        const int o = 8 * (l16 & 3);
        const uint16_t* bp = reinterpret_cast<const uint16_t*>(row + BB * (l16 >> 2));
        const int h = KT == FA_Q8_0 ? 1 + (o >> 1) : 1 + ((o & 15) >> 1);
        // halfword pieces of lines the 16 lanes share: ordinary (cached) loads
        const uint32_t b0 = bp[h], b1 = bp[h + 1], b2 = bp[h + 2], b3 = bp[h + 3];
        return FaRow{make_uint4(b0 | (b1 << 16), b2 | (b3 << 16), bp[0], 0u), make_uint4(0u, 0u, 0u, 0u)};
    }
}

// The 8 elements of a quantized slice as signed bytes (Q4_0: the nibbles, not yet offset by -8).
template <int KT>
__device__ __forceinline__ uint2 fa_bytes(const uint4& r, int lane) {
    if constexpr (KT == FA_Q4_0) {
        const int sh = (lane & 3) >= 2 ? 4 : 0;
        return make_uint2((r.x >> sh) & 0x0F0F0F0Fu, (r.y >> sh) & 0x0F0F0F0Fu);
    } else {
        return make_uint2(r.x, r.y);
    }
}

// Q8_0 of q for a quantized K: the 32-block of a lane's 8 elements spans the 4 lanes l16 = 4 b .. 4 b + 3; rules of
// amv_quantize_act (ggml quantize_row_q8_0). qq: the lane's 8 int8, dq: the block's fp16-rounded d, qs: the sum of
// the lane's 8 q.
__device__ __forceinline__ void fa_quant_q(const float (&x)[8], int rule, uint32_t (&qq)[2], float& dq, int& qs) {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[e]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, AMV_WAVE));
    amax = fmaxf(amax, __shfl_xor(amax, 2, AMV_WAVE));
    const float d = amax / 127.0f;
    float id;
    if (rule == AMV_Q8_X86) id = amax != 0.0f ? 127.0f / amax : 0.0f;
    else id = d != 0.0f ? 1.0f / d : 0.0f;
    qq[0] = qq[1] = 0u;
    qs = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float t = x[e] * id;
        float qf = rule == AMV_Q8_REF ? roundf(t) : rintf(t);
        qf = fminf(127.0f, fmaxf(-127.0f, qf));
        const int qi = (int)qf;
        qs += qi;
        qq[e >> 2] |= (uint32_t)(qi & 0xFF) << (8 * (e & 3));
    }
    dq = amv_h2f(amv_f2h(d));
}

template <int G, int KPW, bool FUSED, int KT>
__global__ __launch_bounds__(256) void k_fa_split(const float* __restrict__ q, const uint8_t* __restrict__ k,
                                                 const uint8_t* __restrict__ v, const uint16_t* __restrict__ mask,
                                                 float* part, int n_kv_max, const int* __restrict__ n_kv_dev,
                                                 int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head,
                                                 int n_split, float scale, int qrule, unsigned int* counters,
                                                 float* __restrict__ out, const AmvActOut act) {
    constexpr int U = KPW / 4;
    constexpr int SBUF = 4 * 4 * G * FA_D > G * (8 * FA_D + FA_MAX_NSPLIT + 1) ? 4 * 4 * G * FA_D
                                                                              : G * (8 * FA_D + FA_MAX_NSPLIT + 1);
    __shared__ __align__(16) float sbuf[SBUF];  // [wave][lane group][head][dim] partial P V; then the merge
    __shared__ float sM[4][G], sL[4][G];
    const int split = blockIdx.x, hk = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int grp = lane >> 4, d8 = 8 * (lane & 15);
    int n_kv = n_kv_max;
    if (n_kv_dev) n_kv = max(0, min(*n_kv_dev, n_kv_max));
    const int ns = (n_kv + 4 * KPW - 1) / (4 * KPW);  // splits holding keys

    if (split < ns) {
        const int kw0 = split * 4 * KPW + wv * KPW;  // first key of this wave
        const uint8_t* kh = k + (size_t)hk * k_head;
        const uint8_t* vh = v + (size_t)hk * v_head;
        FaRow kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = min(kw0 + 4 * u + grp, n_kv - 1);
            kr[u] = fa_row<KT>(kh + (size_t)i * k_row, lane & 15);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = min(kw0 + 4 * u + grp, n_kv - 1);
            vr[u] = fa_row<KT>(vh + (size_t)i * v_row, lane & 15);
        }
        // the mask values of the lane's keys, loaded with the rest and converted where they are used (a load behind
        // a branch, or converted here, makes the compiler wait for every load issued so far); without a mask the
        // lanes read element 0 of q and ignore it
        uint16_t mraw[U];
        {
            const uint16_t* mp = mask ? mask : reinterpret_cast<const uint16_t*>(q);
#pragma unroll
            for (int u = 0; u < U; ++u) mraw[u] = mp[mask ? min(kw0 + 4 * u + grp, n_kv - 1) : 0];
        }
        // q of the G heads, 8 dims per lane: rounded to f16 for an f16 cache, else quantized to Q8_0 blocks
        float qv[G][8];
        uint32_t qq[G][2];
        float qd[G];
        int qsum[G];
        amv_h2 qh[G][4];  // f16 cache: q as f16 pairs
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float4* qp = reinterpret_cast<const float4*>(q + (size_t)(hk * G + g) * FA_D + d8);
            const float4 a = qp[0], b = qp[1];
            const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[g][e] = KT == FA_F16 ? amv_round_f16(t[e]) : t[e];
            if constexpr (KT == FA_Q8_0 || KT == FA_Q4_0) fa_quant_q(qv[g], qrule, qq[g], qd[g], qsum[g]);
            if constexpr (KT == FA_F16)
#pragma unroll
                for (int e = 0; e < 4; ++e) qh[g][e] = amv_h2{(_Float16)qv[g][2 * e], (_Float16)qv[g][2 * e + 1]};
        }
        float s[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = kw0 + 4 * u + grp;
            const float mk = (i < n_kv) ? (mask ? amv_h2f(mraw[u]) : 0.0f) : -INFINITY;
            if constexpr (KT == FA_F16) {
                // q (rounded to f16) . k as 4 v_dot2_f32_f16 per head: the f16 products are exact in f32
                const uint32_t kw[4] = {kr[u].a.x, kr[u].a.y, kr[u].a.z, kr[u].a.w};
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) d = __builtin_amdgcn_fdot2(__builtin_bit_cast(amv_h2, kw[e]), qh[g][e], d, false);
                    d = amv_row16_sum(d);
                    s[u][g] = (mk == -INFINITY) ? -INFINITY : (d * scale + mk) * AMV_LOG2E;
                }
            } else if constexpr (KT == FA_F32) {
                float kf[8];
                const uint4 x0 = kr[u].a, x1 = kr[u].b;
                const uint32_t kw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) kf[e] = __uint_as_float(kw[e]);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d = fmaf(qv[g][e], kf[e], d);
                    d = amv_row16_sum(d);
                    s[u][g] = (mk == -INFINITY) ? -INFINITY : (d * scale + mk) * AMV_LOG2E;
                }
            } else {
                const uint2 kb = fa_bytes<KT>(kr[u].a, lane);
                const float dk = amv_h2f((uint16_t)kr[u].a.z);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    int is = amv_dot4((int)kb.x, (int)qq[g][0], amv_dot4((int)kb.y, (int)qq[g][1], 0));
                    if constexpr (KT == FA_Q4_0) is -= 8 * qsum[g];
                    is += __shfl_xor(is, 1, AMV_WAVE);  // the block's exact integer sum in its 4 lanes
                    is += __shfl_xor(is, 2, AMV_WAVE);
                    // vec_dot_q8_0_q8_0: isum * (d_k * d_q); vec_dot_q4_0_q8_0: (isum * d_k) * d_q
                    const float t = (lane & 3) != 0         ? 0.0f
                                    : KT == FA_Q8_0 ? (float)is * (dk * qd[g])
                                                    : ((float)is * dk) * qd[g];
                    const float d = amv_row16_sum(t);
                    s[u][g] = (mk == -INFINITY) ? -INFINITY : (d * scale + mk) * AMV_LOG2E;
                }
            }
        }
        float m[G], l[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mm = s[0][g];
#pragma unroll
            for (int u = 1; u < U; ++u) mm = fmaxf(mm, s[u][g]);
            mm = amv_max_x32(amv_max_x16(mm));
            m[g] = mm;
            float ll = 0.0f;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float p = __builtin_amdgcn_exp2f(s[u][g] - (mm == -INFINITY ? 0.0f : mm));
                s[u][g] = p;
                ll += p;
            }
            ll = amv_sum_x32(amv_sum_x16(ll));
            l[g] = ll;  // the 16 lanes of a group each counted their group's keys once: same total in every lane
        }
        float acc[G][8];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float vf[8];
            if constexpr (KT == FA_F32) {
                const uint4 x0 = vr[u].a, x1 = vr[u].b;
                const uint32_t vw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) vf[e] = __uint_as_float(vw[e]);
            } else if constexpr (KT == FA_F16) {
                const uint32_t vw[4] = {vr[u].a.x, vr[u].a.y, vr[u].a.z, vr[u].a.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    vf[2 * e] = amv_h2f(vw[e] & 0xFFFFu);
                    vf[2 * e + 1] = amv_h2f(vw[e] >> 16);
                }
            } else {  // ggml dequantize_row_q8_0 / q4_0: q * d, (nibble - 8) * d
                const uint2 vb = fa_bytes<KT>(vr[u].a, lane);
                const float dv = amv_h2f((uint16_t)vr[u].a.z);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int lo = KT == FA_Q8_0 ? (int)(int8_t)(vb.x >> (8 * e)) : (int)((vb.x >> (8 * e)) & 0xFF) - 8;
                    const int hi = KT == FA_Q8_0 ? (int)(int8_t)(vb.y >> (8 * e)) : (int)((vb.y >> (8 * e)) & 0xFF) - 8;
                    vf[e] = (float)lo * dv;
                    vf[4 + e] = (float)hi * dv;
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(s[u][g], vf[e], acc[g][e]);
        }
        // the 4 lane groups of a wave share the wave's maximum, so their accumulators add; the sum is taken below
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float4* dst = reinterpret_cast<float4*>(sbuf + ((wv * 4 + grp) * G + g) * FA_D + d8);
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
                const float f = (sM[w][g] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sM[w][g] - M);
                const float* sa = sbuf + ((w * 4) * G + g) * FA_D + d;
                const float aw = (sa[0] + sa[G * FA_D]) + (sa[2 * G * FA_D] + sa[3 * G * FA_D]);
                a = fmaf(aw, f, a);
                L = fmaf(sL[w][g], f, L);
            }
            float* pp = part + ((size_t)(hk * G + g) * n_split + split) * FA_PS;
            if constexpr (FUSED) {  // handed over to the merging workgroup within the launch
                amv_store_coh(pp + 4 + d, a);
                if (d == 0) {
                    amv_store_coh(pp, M);
                    amv_store_coh(pp + 1, L);
                }
            } else {
                pp[4 + d] = a;
                if (d == 0) {
                    pp[0] = M;
                    pp[1] = L;
                }
            }
        }
    }
    if constexpr (FUSED) {
        if (!amv_arrive_last(counters + AMV_CNT_STRIDE * hk, gridDim.x)) return;
        amv_acquire();
        fa_merge<G>(part, n_split, ns, hk, out, act, sbuf);
    }
}

// Pass 1 for an f16 cache with q . k on the matrix cores (KPW = 16 or 32 keys per wave, as k_fa_split<G, KPW, FUSED,
// FA_F16>, same splits and partials; 32 at long contexts: 16384 / 32768 keys 18.7 / 30.5 us against 20.0 / 32.4 us
// for the VALU form): per 16-key chunk, S = K q^T of its 16 keys and the G heads is four v_mfma_f32_16x16x32_f16
// over the 128 dims (A: key l % 16, dims 32 kk + 8 (l / 16) .. + 7 of its row, loaded as 16 bytes; B: q of head
// l % 16 rounded to f16, zero columns from G on), so the f16 products are exact and summed in f32 as the dot2 form
// sums them (in another order). The result gives lane l the scores of keys 4 (l / 16) + e of head l % 16 in each
// chunk: the maximum and the sum over a head's keys are over the lane's values and the lane pairs l ^ 16, l ^ 32.
// The probabilities reach the P V layout of k_fa_split (lane group g: keys 16 c + 4 u + g, 8 dims per lane) through
// KPW x G floats of LDS per wave; P V, the merge of the 4 wave partials and the split merge are k_fa_split's.
typedef _Float16 fa_h8 __attribute__((ext_vector_type(8)));
typedef float fa_f4 __attribute__((ext_vector_type(4)));

template <int G, bool FUSED, int KPW>
__global__ __launch_bounds__(256) void k_fa_split_mf(const float* __restrict__ q, const uint8_t* __restrict__ k,
                                                    const uint8_t* __restrict__ v, const uint16_t* __restrict__ mask,
                                                    float* part, int n_kv_max, const int* __restrict__ n_kv_dev,
                                                    int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head,
                                                    int n_split, float scale, unsigned int* counters,
                                                    float* __restrict__ out, const AmvActOut act) {
    constexpr int NC = KPW / 16, U = 4;  // 16-key chunks per wave
    static_assert(KPW == 16 || KPW == 32, "16 or 32 keys per wave");
    constexpr int SBUF = 4 * 4 * G * FA_D > G * (8 * FA_D + FA_MAX_NSPLIT + 1) ? 4 * 4 * G * FA_D
                                                                              : G * (8 * FA_D + FA_MAX_NSPLIT + 1);
    __shared__ __align__(16) float sbuf[SBUF];  // [wave][lane group][head][dim] partial P V; then the merge
    __shared__ float sM[4][G], sL[4][G];
    __shared__ float sP[4][KPW][G];  // per wave: probability of key, head
    // grid (KV heads, splits): the workgroups reading the KV heads' slices of the same token rows are dispatched
    // together
    const int split = blockIdx.y, hk = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int grp = lane >> 4, c16 = lane & 15, d8 = 8 * c16;
    // Every load below is addressed within the launch's n_kv_max keys and issued before the key count in device
    // memory is read; keys from n_kv on are selected away (score -inf, V values 0), and a workgroup past the last
    // split holding keys drops its loads.
    int n_kv = n_kv_max, ns = 0;                 // ns: splits holding keys
    const int kw0 = split * 4 * KPW + wv * KPW;  // first key of this wave
    const int klast = n_kv_max - 1;
    {
        const uint8_t* kh = k + (size_t)hk * k_head;
        const uint8_t* vh = v + (size_t)hk * v_head;
        // per 16-key chunk c (keys kw0 + 16 c ..): K as the A operand: lane (grp, c16) takes key kw0 + 16 c + c16,
        // bytes 64 kk + 16 grp (an instruction covers half of each of 16 rows' lines: ordinary loads, so the second
        // half meets the line in L2)
        uint4 kr[NC][4];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int ik = min(kw0 + 16 * c + c16, klast);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                kr[c][kk] = *reinterpret_cast<const uint4*>(kh + (size_t)ik * k_row + 64 * kk + 16 * grp);
        }
        // V in k_fa_split's layout: lane (grp, c16) takes key kw0 + 16 c + 4 u + grp, dims 8 c16 .. + 7 (whole
        // 256-byte rows per 16 lanes: streamed)
        uint4 vr[NC][U];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = min(kw0 + 16 * c + 4 * u + grp, klast);
                vr[c][u] = amv_ld_stream(reinterpret_cast<const uint4*>(vh + (size_t)i * v_row + 16 * c16));
            }
        // the mask values of the lane's score keys kw0 + 16 c + 4 grp + e, loaded with the rest and converted where
        // they are used (a load behind a branch, or converted here, makes the compiler wait for every load issued so
        // far); without a mask the lanes read element 0 of q and ignore it
        uint16_t mraw[NC][4];
        {
            const uint16_t* mp = mask ? mask : reinterpret_cast<const uint16_t*>(q);
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) mraw[c][e] = mp[mask ? min(kw0 + 16 * c + 4 * grp + e, klast) : 0];
        }
        // q as the B operand: head c16 (columns from G on are zero), dims 32 kk + 8 grp .. + 7, rounded to f16
        fa_h8 qb[4];
        {
            const float* qp = q + (size_t)(hk * G + min(c16, G - 1)) * FA_D + 8 * grp;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const float4 a = *reinterpret_cast<const float4*>(qp + 32 * kk);
                const float4 b = *reinterpret_cast<const float4*>(qp + 32 * kk + 4);
                const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) qb[kk][e] = c16 < G ? (_Float16)t[e] : (_Float16)0.0f;
            }
        }
        asm volatile("" ::: "memory");  // the key count is read after the loads above are issued
        if (n_kv_dev) n_kv = max(0, min(*n_kv_dev, n_kv_max));
        ns = (n_kv + 4 * KPW - 1) / (4 * KPW);
        if (split < ns) {  // uniform per workgroup
        // lane (grp, c16): keys kw0 + 16 c + 4 grp + e of head c16, in log2 units
        float sc[NC][4];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            fa_f4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(fa_h8, kr[c][kk]), qb[kk], S, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = kw0 + 16 * c + 4 * grp + e;
                const float mk = (i < n_kv) ? (mask ? amv_h2f(mraw[c][e]) : 0.0f) : -INFINITY;
                sc[c][e] = (mk == -INFINITY) ? -INFINITY : (S[e] * scale + mk) * AMV_LOG2E;
            }
        }
        float mm = -INFINITY;
#pragma unroll
        for (int c = 0; c < NC; ++c) mm = fmaxf(mm, fmaxf(fmaxf(sc[c][0], sc[c][1]), fmaxf(sc[c][2], sc[c][3])));
        mm = amv_max_x32(amv_max_x16(mm));
        float ll = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc[c][e] = __builtin_amdgcn_exp2f(sc[c][e] - (mm == -INFINITY ? 0.0f : mm));
                ll += sc[c][e];
            }
        ll = amv_sum_x32(amv_sum_x16(ll));
        if (c16 < G) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) sP[wv][16 * c + 4 * grp + e][c16] = sc[c][e];
            if (grp == 0) {
                sM[wv][c16] = mm;
                sL[wv][c16] = ll;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float acc[G][8];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float vf[8];
                const uint32_t vw[4] = {vr[c][u].x, vr[c][u].y, vr[c][u].z, vr[c][u].w};
                const bool live = kw0 + 16 * c + 4 * u + grp < n_kv;  // a row past the keys may hold anything
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    vf[2 * e] = live ? amv_h2f(vw[e] & 0xFFFFu) : 0.0f;
                    vf[2 * e + 1] = live ? amv_h2f(vw[e] >> 16) : 0.0f;
                }
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = sP[wv][16 * c + 4 * u + grp][g];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
                }
            }
        // the 4 lane groups of a wave share the wave's maximum, so their accumulators add; the sum is taken below
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float4* dst = reinterpret_cast<float4*>(sbuf + ((wv * 4 + grp) * G + g) * FA_D + d8);
            dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
            dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
        }
        __syncthreads();
        // merge the 4 wave partials of this workgroup
        for (int e = tid; e < G * FA_D; e += 256) {
            const int g = e / FA_D, d = e % FA_D;
            const float M = fmaxf(fmaxf(sM[0][g], sM[1][g]), fmaxf(sM[2][g], sM[3][g]));
            float a = 0.0f, L = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float f = (sM[w][g] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sM[w][g] - M);
                const float* sa = sbuf + ((w * 4) * G + g) * FA_D + d;
                const float aw = (sa[0] + sa[G * FA_D]) + (sa[2 * G * FA_D] + sa[3 * G * FA_D]);
                a = fmaf(aw, f, a);
                L = fmaf(sL[w][g], f, L);
            }
            float* pp = part + ((size_t)(hk * G + g) * n_split + split) * FA_PS;
            if constexpr (FUSED) {  // handed over to the merging workgroup within the launch
                amv_store_coh(pp + 4 + d, a);
                if (d == 0) {
                    amv_store_coh(pp, M);
                    amv_store_coh(pp + 1, L);
                }
            } else {
                pp[4 + d] = a;
                if (d == 0) {
                    pp[0] = M;
                    pp[1] = L;
                }
            }
        }
        }
    }
    if constexpr (FUSED) {
        if (!amv_arrive_last(counters + AMV_CNT_STRIDE * hk, gridDim.y)) return;
        amv_acquire();
        fa_merge<G>(part, n_split, ns, hk, out, act, sbuf);
    }
}

// The merge as its own launch: one workgroup per GH heads (GH = 1, or 2 for Q8_K output blocks of 256), the key
// count from n_kv_dev when given, as in k_fa_split.
template <int GH>
__global__ __launch_bounds__(256) void k_fa_combine(const float* __restrict__ part, float* __restrict__ out,
                                                   int n_split, int n_kv_max, const int* __restrict__ n_kv_dev,
                                                   int split_len, const AmvActOut act) {
    __shared__ __align__(16) float sbuf[GH * (8 * FA_D + FA_MAX_NSPLIT + 1)];
    fa_merge<GH>(part, n_split, n_split, blockIdx.x, out, act, sbuf, n_kv_dev, n_kv_max, split_len);
}

// keys per wave: 16, or 32 when 16 would leave more than 4 workgroups per CU (long contexts)
// (measured on MI355X, f16 cache, 8 KV heads: 32 keys per wave at 4096 keys 9.97 against 9.85 us for 16)
static int fa_kpw(int64_t n_kv, int64_t n_head_kv) { return (n_kv * n_head_kv) / (4 * 16) > 1024 ? 32 : 16; }

extern "C" int64_t amv_flash_attn_workspace_bytes(int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D) {
    if (n_head <= 0 || n_head_kv <= 0 || n_kv <= 0 || D != FA_D) return -1;
    const int64_t sl = 4 * fa_kpw(n_kv, n_head_kv);
    const int64_t n_split = (n_kv + sl - 1) / sl;
    return n_head * n_split * FA_PS * 4;
}

// K / V strides in bytes; kv: AMV_T_F16, AMV_T_Q8_0 or AMV_T_Q4_0 (both caches)
static int fa_check(const char* fn, int kv, const float* q, const void* k, const void* v, const float* out,
                    const void* ws, const void* act, int rule, int64_t n_head, int64_t n_head_kv, int64_t n_kv,
                    int64_t D, int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head, int64_t workspace_bytes) {
    AMV_REQUIRE(q && k && v && out && ws, "%s: null pointer", fn);
    AMV_REQUIRE(kv == AMV_T_F32 || kv == AMV_T_F16 || kv == AMV_T_Q8_0 || kv == AMV_T_Q4_0,
                "%s: KV type %d (F32, F16, Q8_0 or Q4_0)", fn, kv);
    AMV_REQUIRE(!act || ((uintptr_t)act & 15) == 0, "%s: act must be 16-byte aligned", fn);
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "%s: bad rule", fn);
    AMV_REQUIRE(D == FA_D, "%s: head size %lld not supported (128 is)", fn, (long long)D);
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0, "%s: bad head counts", fn);
    const int64_t G = n_head / n_head_kv;
    AMV_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "%s: GQA group %lld not supported", fn, (long long)G);
    AMV_REQUIRE(n_kv > 0 && n_kv <= 128LL * FA_MAX_NSPLIT, "%s: n_kv %lld out of range", fn, (long long)n_kv);
    AMV_REQUIRE(n_head_kv <= 65535, "%s: too many KV heads", fn);
    AMV_REQUIRE(k_head >= 0 && v_head >= 0, "%s: negative head stride", fn);
    if (kv == AMV_T_F32) {
        AMV_REQUIRE(k_row >= 4 * D && v_row >= 4 * D && k_row % 16 == 0 && v_row % 16 == 0 && k_head % 16 == 0 &&
                        v_head % 16 == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0,
                    "%s: f32 K/V rows must be 16-byte aligned", fn);
    } else if (kv == AMV_T_F16) {
        AMV_REQUIRE(k_row >= 2 * D && v_row >= 2 * D && k_row % 16 == 0 && v_row % 16 == 0 && k_head % 16 == 0 &&
                        v_head % 16 == 0,
                    "%s: f16 K/V strides must be >= D and multiples of 8 elements", fn);
        AMV_REQUIRE(((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0, "%s: f16 K/V must be 16-byte aligned", fn);
    } else {
        const int64_t rb = D / 32 * (kv == AMV_T_Q8_0 ? 34 : 18);
        AMV_REQUIRE(k_row >= rb && v_row >= rb && k_row % 2 == 0 && v_row % 2 == 0 && k_head % 2 == 0 &&
                        v_head % 2 == 0,
                    "%s: quantized K/V rows must hold %lld bytes, even strides", fn, (long long)rb);
        AMV_REQUIRE(((uintptr_t)k & 1) == 0 && ((uintptr_t)v & 1) == 0, "%s: quantized K/V must be 2-byte aligned",
                    fn);
    }
    AMV_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)ws & 15) == 0, "%s: q and workspace must be 16-byte aligned",
                fn);
    const int64_t need = amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv, D);
    AMV_REQUIRE(workspace_bytes >= need, "%s: workspace %lld < %lld bytes", fn, (long long)workspace_bytes,
                (long long)need);
    return AMV_OK;
}

template <bool FUSED, int KT>
static void fa_launch_split(int G, int kpw, dim3 grid, hipStream_t st, const float* q, const uint8_t* kk,
                            const uint8_t* vv, const uint16_t* mm, float* part, int n_kv, const int* n_kv_dev,
                            int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head, int n_split, float scale,
                            int rule, unsigned int* counters, float* out, const AmvActOut& act) {
#define FA_LAUNCH(GG, KK)                                                                                              \
    hipLaunchKernelGGL((k_fa_split<GG, KK, FUSED, KT>), grid, dim3(256), 0, st, q, kk, vv, mm, part, n_kv, n_kv_dev, \
                       k_row, k_head, v_row, v_head, n_split, scale, rule, counters, out, act)
#define FA_MF(GG, KK)                                                                                            \
    hipLaunchKernelGGL((k_fa_split_mf<GG, FUSED, KK>), dim3(grid.y, grid.x), dim3(256), 0, st, q, kk, vv, mm, part, \
                       n_kv, n_kv_dev, k_row, k_head, v_row, v_head, n_split, scale, counters, out, act)
#define FA_G(GG)                                  \
    if (KT == FA_F16 && kpw == 16) FA_MF(GG, 16);  \
    else if (KT == FA_F16) FA_MF(GG, 32);          \
    else if (kpw == 16) FA_LAUNCH(GG, 16);         \
    else FA_LAUNCH(GG, 32)
    switch (G) {
    case 1: FA_G(1); break;
    case 2: FA_G(2); break;
    case 4: FA_G(4); break;
    default: FA_G(8); break;
    }
#undef FA_G
#undef FA_MF
#undef FA_LAUNCH
}

template <bool FUSED>
static void fa_launch_kv(int kv, int G, int kpw, dim3 grid, hipStream_t st, const float* q, const uint8_t* kk,
                         const uint8_t* vv, const uint16_t* mm, float* part, int n_kv, const int* n_kv_dev,
                         int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head, int n_split, float scale,
                         int rule, unsigned int* counters, float* out, const AmvActOut& act) {
    if (kv == AMV_T_F32)
        fa_launch_split<FUSED, FA_F32>(G, kpw, grid, st, q, kk, vv, mm, part, n_kv, n_kv_dev, k_row, k_head, v_row,
                                       v_head, n_split, scale, rule, counters, out, act);
    else if (kv == AMV_T_Q8_0)
        fa_launch_split<FUSED, FA_Q8_0>(G, kpw, grid, st, q, kk, vv, mm, part, n_kv, n_kv_dev, k_row, k_head, v_row,
                                        v_head, n_split, scale, rule, counters, out, act);
    else if (kv == AMV_T_Q4_0)
        fa_launch_split<FUSED, FA_Q4_0>(G, kpw, grid, st, q, kk, vv, mm, part, n_kv, n_kv_dev, k_row, k_head, v_row,
                                        v_head, n_split, scale, rule, counters, out, act);
    else
        fa_launch_split<FUSED, FA_F16>(G, kpw, grid, st, q, kk, vv, mm, part, n_kv, n_kv_dev, k_row, k_head, v_row,
                                       v_head, n_split, scale, rule, counters, out, act);
}

// split + merge; counters == NULL: the merge as a second launch, else in the split launch's last workgroups.
// K / V strides in bytes.
static int fa_run(const char* fn, int kv, const float* q, const void* k, const void* v, const void* mask, float* out,
                  int64_t n_head, int64_t n_head_kv, int64_t n_kv_max, const int32_t* n_kv_dev, int64_t D,
                  int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head, float scale, void* workspace,
                  int64_t workspace_bytes, unsigned int* counters, void* act, int act_type, int rule, void* stream) {
    int rc = fa_check(fn, kv, q, k, v, out, workspace, act, rule, n_head, n_head_kv, n_kv_max, D, k_row, k_head,
                      v_row, v_head, workspace_bytes);
    if (rc) return rc;
    const int G = (int)(n_head / n_head_kv);
    AMV_REQUIRE(!act || act_type == AMV_T_Q8_0 || (act_type == AMV_T_Q8_K && G % 2 == 0),
                "%s: act_type %d (Q8_0, or Q8_K with an even GQA group)", fn, act_type);
    const int kpw = fa_kpw(n_kv_max, n_head_kv);
    const int n_split = (int)((n_kv_max + 4 * kpw - 1) / (4 * kpw));
    hipStream_t st = amv_stream(stream);
    float* part = (float*)workspace;
    const AmvActOut ao = amv_act_out(act, n_head * D, act ? act_type : 0, rule);
    const dim3 grid(n_split, (unsigned)n_head_kv);
    const uint8_t* kk = (const uint8_t*)k;
    const uint8_t* vv = (const uint8_t*)v;
    if (counters) {
        fa_launch_kv<true>(kv, G, kpw, grid, st, q, kk, vv, (const uint16_t*)mask, part, (int)n_kv_max, n_kv_dev,
                           k_row, k_head, v_row, v_head, n_split, scale, rule, counters, out, ao);
    } else {
        fa_launch_kv<false>(kv, G, kpw, grid, st, q, kk, vv, (const uint16_t*)mask, part, (int)n_kv_max, n_kv_dev,
                            k_row, k_head, v_row, v_head, n_split, scale, rule, nullptr, nullptr, AmvActOut{});
        if (ao.type == AMV_T_Q8_K)
            hipLaunchKernelGGL(k_fa_combine<2>, dim3((unsigned)(n_head / 2)), dim3(256), 0, st, part, out, n_split,
                               (int)n_kv_max, n_kv_dev, 4 * kpw, ao);
        else
            hipLaunchKernelGGL(k_fa_combine<1>, dim3((unsigned)n_head), dim3(256), 0, st, part, out, n_split,
                               (int)n_kv_max, n_kv_dev, 4 * kpw, ao);
    }
    return amv_check_launch(fn);
}

// The split pass alone: the partials for a consumer that merges them itself (the BitNet engine's output projection,
// amv_bitnet_gemv_fa_merge). The launch, its split count and its keys per split are those of amv_flash_attn_decode_kv
// at the same n_kv_max; head h, split z at workspace + (h * n_split + z) * FA_PS floats: m, l, two pad, acc[D].
extern "C" int amv_flash_attn_split_kv(int kv_type, const float* q, const void* k, const void* v, const void* mask,
                                       int64_t n_head, int64_t n_head_kv, int64_t n_kv_max, const int32_t* n_kv_dev,
                                       int64_t D, int64_t k_row_bytes, int64_t k_head_bytes, int64_t v_row_bytes,
                                       int64_t v_head_bytes, float scale, void* workspace, int64_t workspace_bytes,
                                       int rule, int32_t* n_split_out, int32_t* split_len_out, void* stream) {
    const char* fn = "amv_flash_attn_split_kv";
    // the split pass writes no output row: the workspace stands in for `out` in the argument check
    int rc = fa_check(fn, kv_type, q, k, v, (const float*)workspace, workspace, nullptr, rule, n_head, n_head_kv,
                      n_kv_max, D, k_row_bytes, k_head_bytes, v_row_bytes, v_head_bytes, workspace_bytes);
    if (rc) return rc;
    AMV_REQUIRE(n_split_out && split_len_out, "%s: null pointer", fn);
    const int G = (int)(n_head / n_head_kv);
    const int kpw = fa_kpw(n_kv_max, n_head_kv);
    const int n_split = (int)((n_kv_max + 4 * kpw - 1) / (4 * kpw));
    fa_launch_kv<false>(kv_type, G, kpw, dim3(n_split, (unsigned)n_head_kv), amv_stream(stream), q,
                        (const uint8_t*)k, (const uint8_t*)v, (const uint16_t*)mask, (float*)workspace, (int)n_kv_max,
                        n_kv_dev, k_row_bytes, k_head_bytes, v_row_bytes, v_head_bytes, n_split, scale, rule, nullptr,
                        nullptr, AmvActOut{});
    *n_split_out = n_split;
    *split_len_out = 4 * kpw;
    return amv_check_launch(fn);
}

extern "C" int amv_flash_attn_decode(const float* q, const void* k, const void* v, const void* mask, float* out,
                                     int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D, int64_t k_row,
                                     int64_t k_head, int64_t v_row, int64_t v_head, float scale, void* workspace,
                                     int64_t workspace_bytes, void* act, int rule, void* stream) {
    return fa_run("amv_flash_attn_decode", AMV_T_F16, q, k, v, mask, out, n_head, n_head_kv, n_kv, nullptr, D,
                  2 * k_row, 2 * k_head, 2 * v_row, 2 * v_head, scale, workspace, workspace_bytes, nullptr, act,
                  AMV_T_Q8_0, rule, stream);
}

extern "C" int amv_flash_attn_decode_ex(const float* q, const void* k, const void* v, const void* mask, float* out,
                                        int64_t n_head, int64_t n_head_kv, int64_t n_kv_max, const int32_t* n_kv_dev,
                                        int64_t D, int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head,
                                        float scale, void* workspace, int64_t workspace_bytes, unsigned int* counters,
                                        void* act, int act_type, int rule, void* stream) {
    return fa_run("amv_flash_attn_decode_ex", AMV_T_F16, q, k, v, mask, out, n_head, n_head_kv, n_kv_max, n_kv_dev,
                  D, 2 * k_row, 2 * k_head, 2 * v_row, 2 * v_head, scale, workspace, workspace_bytes, counters, act,
                  act_type, rule, stream);
}

extern "C" int amv_flash_attn_decode_kv(int kv_type, const float* q, const void* k, const void* v, const void* mask,
                                        float* out, int64_t n_head, int64_t n_head_kv, int64_t n_kv_max,
                                        const int32_t* n_kv_dev, int64_t D, int64_t k_row_bytes, int64_t k_head_bytes,
                                        int64_t v_row_bytes, int64_t v_head_bytes, float scale, void* workspace,
                                        int64_t workspace_bytes, unsigned int* counters, void* act, int act_type,
                                        int rule, void* stream) {
    return fa_run("amv_flash_attn_decode_kv", kv_type, q, k, v, mask, out, n_head, n_head_kv, n_kv_max, n_kv_dev, D,
                  k_row_bytes, k_head_bytes, v_row_bytes, v_head_bytes, scale, workspace, workspace_bytes, counters,
                  act, act_type, rule, stream);
}

// ---------------------------------------------------------------------------------------------------------------
// The decode attention without a workspace argument and without any allocation (for callers that cannot allocate:
// code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). The split partials live in
// `scratch`, a file-scope device array of AMV_FA_SCRATCH_BYTES that every GPU the library runs on holds until the
// process ends. Host code never uses the array's name as a device address: its address on each device is looked up
// once with hipGetSymbolAddress (with that device current, at the first call on it) and kept per device. The
// partials are written before they are read within one call (pass 1 writes every split that holds keys, the merge
// reads only those), so nothing needs clearing; calls that overlap in time on one device race on the array.
// ---------------------------------------------------------------------------------------------------------------
#define AMV_FA_SCRATCH_BYTES (8u << 20)
static __device__ __align__(256) uint8_t scratch[AMV_FA_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
std::map<int, void*> g_scratch_ptr;  // device -> address of `scratch` on that device
}  // namespace

static void* fa_scratch(const char* fn) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        amv_set_error("%s: hipGetDevice failed", fn);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_ptr.find(dev);
    if (it != g_scratch_ptr.end()) return it->second;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        amv_set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev, hipGetErrorString(e));
        return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
    return ptr;
}

extern "C" int64_t amv_flash_attn_noalloc_max_bytes(void) { return AMV_FA_SCRATCH_BYTES; }

extern "C" int amv_flash_attn_decode_noalloc(int kv_type, const float* q, const void* k, const void* v,
                                             const void* mask, float* out, int64_t n_head, int64_t n_head_kv,
                                             int64_t n_kv_max, const int32_t* n_kv_dev, int64_t D,
                                             int64_t k_row_bytes, int64_t k_head_bytes, int64_t v_row_bytes,
                                             int64_t v_head_bytes, float scale, void* act, int act_type, int rule,
                                             void* stream) {
    const char* fn = "amv_flash_attn_decode_noalloc";
    const int64_t need = amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv_max, D);
    AMV_REQUIRE(need > 0, "%s: unsupported shape (n_head %lld, n_head_kv %lld, n_kv_max %lld, D %lld)", fn,
                (long long)n_head, (long long)n_head_kv, (long long)n_kv_max, (long long)D);
    AMV_REQUIRE(need <= (int64_t)AMV_FA_SCRATCH_BYTES,
                "%s: the split partials need %lld bytes, above the %u-byte scratch of this entry point (use "
                "amv_flash_attn_decode_kv with a workspace)", fn, (long long)need, AMV_FA_SCRATCH_BYTES);
    void* ws = fa_scratch(fn);
    if (!ws) return AMV_ERR_HIP;
    return fa_run(fn, kv_type, q, k, v, mask, out, n_head, n_head_kv, n_kv_max, n_kv_dev, D, k_row_bytes,
                  k_head_bytes, v_row_bytes, v_head_bytes, scale, ws, (int64_t)AMV_FA_SCRATCH_BYTES, nullptr, act,
                  act_type, rule, stream);
}
