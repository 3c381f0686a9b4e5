// Quantizers (activations to Q8_0 / Q8_K, rows to Q4_0) and the weight repack between ggml blocks and the MI355X
// structure-of-arrays layout. Quantization reproduces the CPU's f32 arithmetic exactly: this file is built with
// -ffp-contract=off and correctly rounded division, so x * id, 1 / d and 127 / amax round as on the CPU.
#include "amv_common.h"

// ---------------------------------------------------------------------------------------------------------------
// Q8_0 activations: one lane per element, 32 lanes per block (a wave holds two blocks).
// ggml quantize_row_q8_0 (x86: id = 127/amax, round half even; ARM: id = 1/d, round half even; ref: id = 1/d,
// roundf) -- the rules of ameva_act_fq.comp:5,38-41 and ameva_quant_a8.comp:46-54; d = amax/127 stored fp16.
// ---------------------------------------------------------------------------------------------------------------
// With a16 (AMV_ACT_Q8_0_MMA) the values also go out as f16 and the block scale transposed (row t = b / nbr, block
// j = b % nbr at dt[j * m + t]); with deq (AMV_ACT_Q8_0_DEQ) the f16 copies are q * d (one rounding) instead of q.
__global__ __launch_bounds__(256) void k_quant_q8_0(const float* __restrict__ x, int64_t n_elem, int rule,
                                                   uint8_t* __restrict__ y_ggml, int8_t* __restrict__ aq,
                                                   int2* __restrict__ ads, uint16_t* __restrict__ a16,
                                                   float* __restrict__ dt, int nbr, int m, int deq) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = i < n_elem;
    const float v = live ? x[i] : 0.0f;
    // max |x| over the 32 lanes of the block (xor offsets < 32 stay inside the half-wave)
    float amax = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, AMV_WAVE));
    const float d = amax / 127.0f;
    float id;
    if (rule == AMV_Q8_X86) id = amax != 0.0f ? 127.0f / amax : 0.0f;
    else id = d != 0.0f ? 1.0f / d : 0.0f;
    const float t = v * id;
    float qf = rule == AMV_Q8_REF ? roundf(t) : rintf(t);
    qf = fminf(127.0f, fmaxf(-127.0f, qf));
    const int q = (int)qf;
    int s = q;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, AMV_WAVE);
    if (!live) return;
    const int64_t b = i >> 5;
    const int j = (int)(i & 31);
    const uint16_t d16 = amv_f2h(d);
    if (y_ggml) {
        uint8_t* yb = y_ggml + b * 34;
        yb[2 + j] = (uint8_t)(int8_t)q;
        if (j == 0) *(uint16_t*)yb = d16;
    }
    if (aq) {
        aq[i] = (int8_t)q;
        if (j == 0) ads[b] = make_int2(__float_as_int(amv_h2f(d16)), s);
    }
    if (a16) {
        a16[i] = __builtin_bit_cast(uint16_t, deq ? (_Float16)((float)q * amv_h2f(d16)) : (_Float16)q);
        if (j == 0) dt[(b % nbr) * m + b / nbr] = amv_h2f(d16);
    }
}

// The plain layout alone (no ggml blocks, no f16 copies), four elements per lane and a block per 8 lanes
// (q8_block_lanes8: the same rules, the same bytes).
__global__ __launch_bounds__(256) void k_quant_q8_0_x4(const float4* __restrict__ x, int n4, int rule,
                                                      int8_t* __restrict__ aq, int2* __restrict__ ads) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;  // n4 % 8 == 0: the 8 lanes of a block leave together
    const float4 v4 = x[i];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    q8_block_lanes8(v, rule, i & 7, aq + 32 * (int64_t)(i >> 3), ads + (i >> 3));
}

// ---------------------------------------------------------------------------------------------------------------
// Q8_K activations (ggml quantize_row_q8_K_ref): one wave per 256-element block, 4 elements per lane.
// max = the element of largest magnitude (the first on ties), iscale = -127/max, q = min(127, round-half-even(
// iscale * x)), d = 1/iscale, bsums = sums of q over 16 elements.
// ---------------------------------------------------------------------------------------------------------------
// With a16 (AMV_ACT_Q8_K_MMA) the block's values also go out as f16, its sums per 16 as f16 and its scale transposed
// (token t = b / nsb, super-block j = b % nsb at dt[j * m + t]); with deq (AMV_ACT_Q8_K_DEQ) the f16 copies are q * d.
__global__ __launch_bounds__(256) void k_quant_q8_K(const float* __restrict__ x, int64_t n_blk,
                                                   uint8_t* __restrict__ y_ggml, int8_t* __restrict__ aq,
                                                   float* __restrict__ ad, int32_t* __restrict__ abs16,
                                                   uint16_t* __restrict__ a16, uint16_t* __restrict__ bs16,
                                                   float* __restrict__ dt, int nsb, int m, int deq) {
    const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= n_blk) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const float4 v4 = reinterpret_cast<const float4*>(x + b * 256)[lane];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    const AmvQ8K r = amv_q8_K_lanes64(v, lane);
    const int* q = r.q;
    const int s = r.s16;
    const float d = r.d;
    const int packed = amv_pack4(r.q);
    uint8_t* yb = y_ggml ? y_ggml + b * 292 : nullptr;
    if (yb) {
        reinterpret_cast<int*>(yb + 4)[lane] = packed;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(yb + 260)[lane >> 2] = (int16_t)s;
        if (lane == 0) *reinterpret_cast<float*>(yb) = d;
    }
    if (aq) {
        reinterpret_cast<int*>(aq + b * 256)[lane] = packed;
        if ((lane & 3) == 0) abs16[b * 16 + (lane >> 2)] = s;
        if (lane == 0) ad[b] = d;
    }
    if (a16) {
        const float sc = deq ? d : 1.0f;  // q * 1 = q exactly
        const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)((float)q[0] * sc));
        const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)((float)q[1] * sc));
        const uint32_t h2 = __builtin_bit_cast(uint16_t, (_Float16)((float)q[2] * sc));
        const uint32_t h3 = __builtin_bit_cast(uint16_t, (_Float16)((float)q[3] * sc));
        reinterpret_cast<uint2*>(a16 + b * 256)[lane] = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
        if ((lane & 3) == 0) bs16[b * 16 + (lane >> 2)] = __builtin_bit_cast(uint16_t, (_Float16)s);
        if (lane == 0) dt[(b % nsb) * m + b / nsb] = d;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Q4_0 rows (ggml quantize_row_q4_0_ref; ameva_set_rows_q.comp:95-115): one lane per 32-element block.
// ---------------------------------------------------------------------------------------------------------------
// One block as 9 halfwords: d (fp16), then byte j of qs = q[j] | q[j + 16] << 4. max = the first element of largest
// magnitude, d = max / -8, id = 1/d, q = min(15, (int)(x * id + 8.5)).
__device__ __forceinline__ void q4_0_block(const float (&v)[32], uint16_t (&h)[9]) {
    float amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        if (amax < fabsf(v[j])) { amax = fabsf(v[j]); mx = v[j]; }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    h[0] = amv_f2h(d);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t pair = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = 2 * k + e;
            const float x0 = v[j] * id, x1 = v[j + 16] * id;
            int q0 = (int)(x0 + 8.5f), q1 = (int)(x1 + 8.5f);
            q0 = q0 < 15 ? q0 : 15;
            q1 = q1 < 15 ? q1 : 15;
            pair |= (uint32_t)(q0 | (q1 << 4)) << (8 * e);
        }
        h[1 + k] = (uint16_t)pair;
    }
}

// One Q8_0 block as 17 halfwords (d fp16, then the 32 int8), with the rules of amv_quantize_act.
__device__ __forceinline__ void q8_0_block(const float (&v)[32], int rule, uint16_t (&h)[17]) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    float id;
    if (rule == AMV_Q8_X86) id = amax != 0.0f ? 127.0f / amax : 0.0f;
    else id = d != 0.0f ? 1.0f / d : 0.0f;
    h[0] = amv_f2h(d);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        uint32_t pair = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float t = v[2 * k + e] * id;
            float qf = rule == AMV_Q8_REF ? roundf(t) : rintf(t);
            qf = fminf(127.0f, fmaxf(-127.0f, qf));
            pair |= (uint32_t)((int)qf & 0xFF) << (8 * e);
        }
        h[1 + k] = (uint16_t)pair;
    }
}

__global__ __launch_bounds__(256) void k_quant_q4_0(const float* __restrict__ x, int64_t n_blk,
                                                   uint8_t* __restrict__ y) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blk) return;
    const float4* xp = reinterpret_cast<const float4*>(x + b * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = xp[i];
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
    uint16_t h[9];
    q4_0_block(v, h);
    uint16_t* yb = reinterpret_cast<uint16_t*>(y + b * 18);
#pragma unroll
    for (int k = 0; k < 9; ++k) yb[k] = h[k];
}

// ---------------------------------------------------------------------------------------------------------------
// SET_ROWS / CPY f32 -> Q8_0 or Q4_0 rows: ggml's from_float of the destination type (quantize_row_q8_0 with the
// chosen rule, quantize_row_q4_0_ref; the reference's ameva_set_rows_q.comp:82-115). One lane per 32-element block of
// a source row; row r goes to dst row idx[r] (or r), an index outside [0, dst_rows) is skipped and counted once.
// ---------------------------------------------------------------------------------------------------------------
template <int T>
__global__ __launch_bounds__(256) void k_set_rows_q(const float* __restrict__ src, int64_t src_stride,
                                                   uint8_t* __restrict__ dst, int64_t dst_stride, int64_t n_rows,
                                                   int nb, const int64_t* __restrict__ idx64,
                                                   const int32_t* __restrict__ idx32, int64_t dst_rows, int rule,
                                                   unsigned int* __restrict__ bad) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_rows * nb) return;
    const int64_t r = t / nb;
    const int j = (int)(t - r * nb);
    int64_t dr = r;
    if (idx64) dr = idx64[r];
    else if (idx32) dr = idx32[r];
    if (dr < 0 || dr >= dst_rows) {
        if (j == 0 && bad) atomicAdd(bad, 1u);
        return;
    }
    const float* x = src + r * src_stride + 32 * j;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = x[i];
    constexpr int BB = T == AMV_T_Q8_0 ? 34 : 18;
    uint16_t* yb = reinterpret_cast<uint16_t*>(dst + dr * dst_stride + (int64_t)BB * j);
    if constexpr (T == AMV_T_Q8_0) {
        uint16_t h[17];
        q8_0_block(v, rule, h);
#pragma unroll
        for (int k = 0; k < 17; ++k) yb[k] = h[k];
    } else {
        uint16_t h[9];
        q4_0_block(v, h);
#pragma unroll
        for (int k = 0; k < 9; ++k) yb[k] = h[k];
    }
}

extern "C" int amv_set_rows_q(int type, const float* src, int64_t src_stride, void* dst, int64_t dst_stride,
                              int64_t n_rows, int64_t n, const void* idx, int idx_bits, int64_t dst_rows, int rule,
                              unsigned int* bad, void* stream) {
    AMV_REQUIRE(src && dst, "amv_set_rows_q: null pointer");
    AMV_REQUIRE(type == AMV_T_Q8_0 || type == AMV_T_Q4_0, "amv_set_rows_q: type %d (Q8_0 or Q4_0)", type);
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_set_rows_q: bad rule");
    AMV_REQUIRE(n_rows > 0 && n > 0 && n % 32 == 0 && src_stride >= n, "amv_set_rows_q: bad shape");
    const int64_t nb = n / 32, bb = type == AMV_T_Q8_0 ? 34 : 18;
    AMV_REQUIRE(dst_stride >= nb * bb && dst_stride % 2 == 0 && ((uintptr_t)dst & 1) == 0,
                "amv_set_rows_q: dst rows must hold %lld bytes at even addresses", (long long)(nb * bb));
    AMV_REQUIRE(nb <= INT32_MAX, "amv_set_rows_q: rows too long");
    AMV_REQUIRE(idx == nullptr || idx_bits == 32 || idx_bits == 64, "amv_set_rows_q: index type must be i32 or i64");
    AMV_REQUIRE(idx != nullptr || dst_rows >= n_rows, "amv_set_rows_q: dst too small");
    const int64_t total = n_rows * nb;
    const dim3 grid((unsigned)((total + 255) / 256));
    const int64_t* i64 = idx_bits == 64 ? (const int64_t*)idx : nullptr;
    const int32_t* i32 = idx_bits == 32 ? (const int32_t*)idx : nullptr;
    if (type == AMV_T_Q8_0)
        hipLaunchKernelGGL(k_set_rows_q<AMV_T_Q8_0>, grid, dim3(256), 0, amv_stream(stream), src, src_stride,
                           (uint8_t*)dst, dst_stride, n_rows, (int)nb, i64, i32, dst_rows, rule, bad);
    else
        hipLaunchKernelGGL(k_set_rows_q<AMV_T_Q4_0>, grid, dim3(256), 0, amv_stream(stream), src, src_stride,
                           (uint8_t*)dst, dst_stride, n_rows, (int)nb, i64, i32, dst_rows, rule, bad);
    return amv_check_launch("amv_set_rows_q");
}

// ---------------------------------------------------------------------------------------------------------------
// Repack ggml blocks <-> structure of arrays. One lane per block; block b = row * nb + j in both layouts.
// ---------------------------------------------------------------------------------------------------------------
template <bool FWD>
__global__ __launch_bounds__(256) void k_repack_q4_0(uint8_t* __restrict__ g, uint4* __restrict__ qs,
                                                    uint16_t* __restrict__ dd, int64_t n_blk, int nb, int n_rows) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blk) return;
    uint16_t* gb = reinterpret_cast<uint16_t*>(g + b * 18);
    const size_t di = amv_q4_0_didx((int)(b / nb), (int)(b % nb), nb, n_rows);
    if (FWD) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (uint32_t)gb[1 + 2 * i] | ((uint32_t)gb[2 + 2 * i] << 16);
        qs[b] = make_uint4(w[0], w[1], w[2], w[3]);
        dd[di] = gb[0];
    } else {
        const uint4 q = qs[b];
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        gb[0] = dd[di];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            gb[1 + 2 * i] = (uint16_t)(w[i] & 0xFFFFu);
            gb[2 + 2 * i] = (uint16_t)(w[i] >> 16);
        }
    }
}

template <bool FWD>
__global__ __launch_bounds__(256) void k_repack_q8_0(uint8_t* __restrict__ g, uint4* __restrict__ qs,
                                                    uint16_t* __restrict__ dd, int64_t n_blk) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blk) return;
    uint16_t* gb = reinterpret_cast<uint16_t*>(g + b * 34);
    if (FWD) {
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = (uint32_t)gb[1 + 2 * i] | ((uint32_t)gb[2 + 2 * i] << 16);
        qs[2 * b] = make_uint4(w[0], w[1], w[2], w[3]);
        qs[2 * b + 1] = make_uint4(w[4], w[5], w[6], w[7]);
        dd[b] = gb[0];
    } else {
        const uint4 q0 = qs[2 * b], q1 = qs[2 * b + 1];
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        gb[0] = dd[b];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            gb[1 + 2 * i] = (uint16_t)(w[i] & 0xFFFFu);
            gb[2 + 2 * i] = (uint16_t)(w[i] >> 16);
        }
    }
}

// Q4_K: 144-byte blocks (16-byte aligned when the tensor is): head 16 B | qs 128 B
template <bool FWD>
__global__ __launch_bounds__(256) void k_repack_q4_K(uint8_t* __restrict__ g, uint4* __restrict__ qs,
                                                    uint4* __restrict__ head, int64_t n_blk) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blk) return;
    uint4* gb = reinterpret_cast<uint4*>(g + b * 144);
    if (FWD) {
        head[b] = gb[0];
#pragma unroll
        for (int i = 0; i < 8; ++i) qs[8 * b + i] = gb[1 + i];
    } else {
        gb[0] = head[b];
#pragma unroll
        for (int i = 0; i < 8; ++i) gb[1 + i] = qs[8 * b + i];
    }
}

// Q6_K: 210-byte blocks (2-byte aligned): ql 128 | qh 64 | scales 16 | d 2
template <bool FWD>
__global__ __launch_bounds__(256) void k_repack_q6_K(uint8_t* __restrict__ g, uint32_t* __restrict__ ql,
                                                    uint32_t* __restrict__ qh, uint32_t* __restrict__ sc,
                                                    uint16_t* __restrict__ dd, int64_t n_blk) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blk) return;
    uint16_t* gb = reinterpret_cast<uint16_t*>(g + b * 210);
    if (FWD) {
        for (int i = 0; i < 32; ++i) ql[32 * b + i] = (uint32_t)gb[2 * i] | ((uint32_t)gb[2 * i + 1] << 16);
        for (int i = 0; i < 16; ++i) qh[16 * b + i] = (uint32_t)gb[64 + 2 * i] | ((uint32_t)gb[65 + 2 * i] << 16);
        for (int i = 0; i < 4; ++i) sc[4 * b + i] = (uint32_t)gb[96 + 2 * i] | ((uint32_t)gb[97 + 2 * i] << 16);
        dd[b] = gb[104];
    } else {
        for (int i = 0; i < 32; ++i) {
            gb[2 * i] = (uint16_t)(ql[32 * b + i] & 0xFFFFu);
            gb[2 * i + 1] = (uint16_t)(ql[32 * b + i] >> 16);
        }
        for (int i = 0; i < 16; ++i) {
            gb[64 + 2 * i] = (uint16_t)(qh[16 * b + i] & 0xFFFFu);
            gb[65 + 2 * i] = (uint16_t)(qh[16 * b + i] >> 16);
        }
        for (int i = 0; i < 4; ++i) {
            gb[96 + 2 * i] = (uint16_t)(sc[4 * b + i] & 0xFFFFu);
            gb[97 + 2 * i] = (uint16_t)(sc[4 * b + i] >> 16);
        }
        gb[104] = dd[b];
    }
}

static inline unsigned grid_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

static int repack_impl(int type, uint8_t* g, uint8_t* r, int64_t n_rows, int64_t k, bool fwd, hipStream_t st) {
    AMV_REQUIRE(g && r, "amv_repack: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0, "amv_repack: empty tensor (%lld x %lld)", (long long)n_rows, (long long)k);
    AMV_REQUIRE(((uintptr_t)r & 15) == 0, "amv_repack: repacked buffer must be 16-byte aligned");
    switch (type) {
    case AMV_T_Q4_0: {
        AMV_REQUIRE(k % 32 == 0, "amv_repack: Q4_0 k %% 32 != 0");
        AMV_REQUIRE(((uintptr_t)g & 1) == 0, "amv_repack: ggml buffer must be 2-byte aligned");
        const int64_t nb = n_rows * (k / 32);
        uint4* qs = reinterpret_cast<uint4*>(r);
        uint16_t* dd = reinterpret_cast<uint16_t*>(r + nb * 16);
        const int nbr = (int)(k / 32);
        if (fwd) hipLaunchKernelGGL(k_repack_q4_0<true>, grid_for(nb, 256), 256, 0, st, g, qs, dd, nb, nbr, (int)n_rows);
        else hipLaunchKernelGGL(k_repack_q4_0<false>, grid_for(nb, 256), 256, 0, st, g, qs, dd, nb, nbr, (int)n_rows);
        break;
    }
    case AMV_T_Q8_0: {
        AMV_REQUIRE(k % 32 == 0, "amv_repack: Q8_0 k %% 32 != 0");
        AMV_REQUIRE(((uintptr_t)g & 1) == 0, "amv_repack: ggml buffer must be 2-byte aligned");
        const int64_t nb = n_rows * (k / 32);
        uint4* qs = reinterpret_cast<uint4*>(r);
        uint16_t* dd = reinterpret_cast<uint16_t*>(r + nb * 32);
        if (fwd) hipLaunchKernelGGL(k_repack_q8_0<true>, grid_for(nb, 256), 256, 0, st, g, qs, dd, nb);
        else hipLaunchKernelGGL(k_repack_q8_0<false>, grid_for(nb, 256), 256, 0, st, g, qs, dd, nb);
        break;
    }
    case AMV_T_Q4_K: {
        AMV_REQUIRE(k % 256 == 0, "amv_repack: Q4_K k %% 256 != 0");
        AMV_REQUIRE(((uintptr_t)g & 15) == 0, "amv_repack: Q4_K ggml buffer must be 16-byte aligned");
        const int64_t nb = n_rows * (k / 256);
        uint4* qs = reinterpret_cast<uint4*>(r);
        uint4* head = reinterpret_cast<uint4*>(r + nb * 128);
        if (fwd) hipLaunchKernelGGL(k_repack_q4_K<true>, grid_for(nb, 256), 256, 0, st, g, qs, head, nb);
        else hipLaunchKernelGGL(k_repack_q4_K<false>, grid_for(nb, 256), 256, 0, st, g, qs, head, nb);
        break;
    }
    case AMV_T_Q6_K: {
        AMV_REQUIRE(k % 256 == 0, "amv_repack: Q6_K k %% 256 != 0");
        AMV_REQUIRE(((uintptr_t)g & 1) == 0, "amv_repack: ggml buffer must be 2-byte aligned");
        const int64_t nb = n_rows * (k / 256);
        uint32_t* ql = reinterpret_cast<uint32_t*>(r);
        uint32_t* qh = reinterpret_cast<uint32_t*>(r + nb * 128);
        uint32_t* sc = reinterpret_cast<uint32_t*>(r + nb * 192);
        uint16_t* dd = reinterpret_cast<uint16_t*>(r + nb * 208);
        if (fwd) hipLaunchKernelGGL(k_repack_q6_K<true>, grid_for(nb, 256), 256, 0, st, g, ql, qh, sc, dd, nb);
        else hipLaunchKernelGGL(k_repack_q6_K<false>, grid_for(nb, 256), 256, 0, st, g, ql, qh, sc, dd, nb);
        break;
    }
    default: amv_set_error("amv_repack: unsupported type %d", type); return AMV_ERR_UNSUPPORTED;
    }
    return amv_check_launch("amv_repack");
}

extern "C" int amv_repack(int type, const void* src_ggml, void* dst, int64_t n_rows, int64_t k, void* stream) {
    return repack_impl(type, (uint8_t*)src_ggml, (uint8_t*)dst, n_rows, k, true, amv_stream(stream));
}

extern "C" int amv_unrepack(int type, const void* src, void* dst_ggml, int64_t n_rows, int64_t k, void* stream) {
    return repack_impl(type, (uint8_t*)dst_ggml, (uint8_t*)src, n_rows, k, false, amv_stream(stream));
}

extern "C" int amv_quantize_act(int type, const float* x, int64_t m, int64_t k, int rule, void* y_ggml, void* y_act,
                                void* stream) {
    AMV_REQUIRE(x, "amv_quantize_act: null input");
    AMV_REQUIRE(m > 0 && k > 0, "amv_quantize_act: empty input (%lld x %lld)", (long long)m, (long long)k);
    AMV_REQUIRE(((uintptr_t)x & 15) == 0, "amv_quantize_act: input must be 16-byte aligned");
    AMV_REQUIRE(y_act == nullptr || ((uintptr_t)y_act & 15) == 0, "amv_quantize_act: y_act must be 16-byte aligned");
    hipStream_t st = amv_stream(stream);
    const int deq = type == AMV_ACT_Q8_0_DEQ || type == AMV_ACT_Q8_K_DEQ;
    if (type == AMV_ACT_Q8_0_DEQ) type = AMV_ACT_Q8_0_MMA;  // same layout, scaled f16 copies
    if (type == AMV_ACT_Q8_K_DEQ) type = AMV_ACT_Q8_K_MMA;
    if (type == AMV_T_Q8_0 || type == AMV_ACT_Q8_0_MMA) {
        AMV_REQUIRE(k % 32 == 0, "amv_quantize_act: Q8_0 needs k %% 32 == 0 (k = %lld)", (long long)k);
        AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_quantize_act: bad rule %d", rule);
        AMV_REQUIRE(y_ggml == nullptr || ((uintptr_t)y_ggml & 1) == 0, "amv_quantize_act: y_ggml misaligned");
        AMV_REQUIRE(type == AMV_T_Q8_0 || y_act, "amv_quantize_act: AMV_ACT_Q8_0_MMA needs y_act");
        AMV_REQUIRE(m <= INT32_MAX && k / 32 <= INT32_MAX, "amv_quantize_act: shape too large");
        const int64_t n = m * k;
        int8_t* aq = y_act ? (int8_t*)y_act : nullptr;
        int2* ads = y_act ? (int2*)((uint8_t*)y_act + n) : nullptr;
        uint16_t* a16 = nullptr;
        float* dt = nullptr;
        if (type == AMV_ACT_Q8_0_MMA) {
            const AmvQ80Mma L = amv_q8_0_mma_layout(m, k);
            a16 = (uint16_t*)((uint8_t*)y_act + L.a16);
            dt = (float*)((uint8_t*)y_act + L.dt);
        }
        if (!y_ggml && !a16 && n / 4 <= INT32_MAX)
            hipLaunchKernelGGL(k_quant_q8_0_x4, grid_for(n / 4, 256), 256, 0, st, reinterpret_cast<const float4*>(x),
                               (int)(n / 4), rule, aq, ads);
        else
            hipLaunchKernelGGL(k_quant_q8_0, grid_for(n, 256), 256, 0, st, x, n, rule, (uint8_t*)y_ggml, aq, ads, a16,
                               dt, (int)(k / 32), (int)m, deq);
    } else if (type == AMV_T_Q8_K || type == AMV_ACT_Q8_K_MMA) {
        AMV_REQUIRE(k % 256 == 0, "amv_quantize_act: Q8_K needs k %% 256 == 0 (k = %lld)", (long long)k);
        AMV_REQUIRE(y_ggml == nullptr || ((uintptr_t)y_ggml & 3) == 0, "amv_quantize_act: y_ggml misaligned");
        AMV_REQUIRE(type == AMV_T_Q8_K || y_act, "amv_quantize_act: AMV_ACT_Q8_K_MMA needs y_act");
        AMV_REQUIRE(m * (k / 256) <= INT32_MAX, "amv_quantize_act: too many blocks");
        const int64_t n = m * k, nb = n / 256;
        int8_t* aq = y_act ? (int8_t*)y_act : nullptr;
        float* ad = y_act ? (float*)((uint8_t*)y_act + n) : nullptr;
        int32_t* abs16 = y_act ? (int32_t*)((uint8_t*)y_act + n + nb * 4) : nullptr;
        uint16_t *a16 = nullptr, *bs16 = nullptr;
        float* dt = nullptr;
        if (type == AMV_ACT_Q8_K_MMA) {
            const AmvQ8kMma L = amv_q8k_mma_layout(m, k);
            a16 = (uint16_t*)((uint8_t*)y_act + L.a16);
            bs16 = (uint16_t*)((uint8_t*)y_act + L.bs16);
            dt = (float*)((uint8_t*)y_act + L.dt);
        }
        hipLaunchKernelGGL(k_quant_q8_K, grid_for(nb, 4), 256, 0, st, x, nb, (uint8_t*)y_ggml, aq, ad, abs16, a16,
                           bs16, dt, (int)(k / 256), (int)m, deq);
    } else {
        amv_set_error("amv_quantize_act: unsupported activation type %d", type);
        return AMV_ERR_UNSUPPORTED;
    }
    return amv_check_launch("amv_quantize_act");
}

extern "C" int amv_quantize_q4_0(const float* x, int64_t n_rows, int64_t k, void* y_ggml, void* stream) {
    AMV_REQUIRE(x && y_ggml, "amv_quantize_q4_0: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0 && k % 32 == 0, "amv_quantize_q4_0: bad shape %lld x %lld", (long long)n_rows,
                (long long)k);
    AMV_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)y_ggml & 1) == 0, "amv_quantize_q4_0: misaligned buffer");
    const int64_t nb = n_rows * (k / 32);
    hipLaunchKernelGGL(k_quant_q4_0, grid_for(nb, 256), 256, 0, amv_stream(stream), x, nb, (uint8_t*)y_ggml);
    return amv_check_launch("amv_quantize_q4_0");
}

// ---------------------------------------------------------------------------------------------------------------
// Q4_K / Q6_K weight quantization with this library's own deterministic rule (ggml's make_qkx2_quants search is not
// reproduced: the weight bytes of these types are not a parity target, the dot products on given bytes are).
// One lane per 256-weight super-block; output in ggml's block layout.
//   Q4_K: per 32-weight unit u: lo = min(0, min x), hi = max(lo, max x), scale_u = (hi - lo) / 15, min_u = -lo;
//         d = max scale_u / 63, dmin = max min_u / 63 (fp16); sc_u = rint(scale_u / d), m_u = rint(min_u / dmin)
//         (<= 63); q = clamp(rint((x + dmin m_u) / (d sc_u)), 0, 15).
//   Q6_K: per 16-weight group g: scale_g = max|x| / 31; d = max scale_g / 127 (fp16); sc_g = rint(scale_g / d)
//         (<= 127); q = clamp(rint(x / (d sc_g)), -32, 31).
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(128) void k_quant_q4_K(const float* __restrict__ x, int64_t n_sb, uint8_t* __restrict__ y) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_sb) return;
    const float* xb = x + b * 256;
    float scl[8], mns[8];
    float maxs = 0.0f, maxm = 0.0f;
    for (int u = 0; u < 8; ++u) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; ++i) {
            lo = fminf(lo, xb[32 * u + i]);
            hi = fmaxf(hi, xb[32 * u + i]);
        }
        hi = fmaxf(hi, lo);
        scl[u] = (hi - lo) / 15.0f;
        mns[u] = -lo;
        maxs = fmaxf(maxs, scl[u]);
        maxm = fmaxf(maxm, mns[u]);
    }
    const uint16_t d16 = amv_f2h(maxs / 63.0f), m16 = amv_f2h(maxm / 63.0f);
    const float df = amv_h2f(d16), mf = amv_h2f(m16);
    int sc[8], mq[8];
    for (int u = 0; u < 8; ++u) {
        sc[u] = df > 0.0f ? min(63, (int)rintf(scl[u] / df)) : 0;
        mq[u] = mf > 0.0f ? min(63, (int)rintf(mns[u] / mf)) : 0;
    }
    uint8_t blk[144];
    blk[0] = (uint8_t)(d16 & 0xFF);
    blk[1] = (uint8_t)(d16 >> 8);
    blk[2] = (uint8_t)(m16 & 0xFF);
    blk[3] = (uint8_t)(m16 >> 8);
    for (int j = 0; j < 4; ++j) {
        blk[4 + j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        blk[8 + j] = (uint8_t)((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
        blk[12 + j] = (uint8_t)((sc[j + 4] & 15) | ((mq[j + 4] & 15) << 4));
    }
    for (int c = 0; c < 4; ++c) {
        for (int l = 0; l < 32; ++l) {
            int qq[2];
            for (int h = 0; h < 2; ++h) {
                const int u = 2 * c + h;
                const float dl = df * (float)sc[u], ml = mf * (float)mq[u];
                int q = 0;
                if (dl > 0.0f) q = (int)rintf((xb[64 * c + 32 * h + l] + ml) / dl);
                qq[h] = min(15, max(0, q));
            }
            blk[16 + 32 * c + l] = (uint8_t)(qq[0] | (qq[1] << 4));
        }
    }
    uint4* yb = reinterpret_cast<uint4*>(y + b * 144);
    const uint4* src = reinterpret_cast<const uint4*>(blk);
    for (int i = 0; i < 9; ++i) yb[i] = src[i];
}

__global__ __launch_bounds__(128) void k_quant_q6_K(const float* __restrict__ x, int64_t n_sb, uint8_t* __restrict__ y) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_sb) return;
    const float* xb = x + b * 256;
    float scl[16], maxs = 0.0f;
    for (int g = 0; g < 16; ++g) {
        float a = 0.0f;
        for (int i = 0; i < 16; ++i) a = fmaxf(a, fabsf(xb[16 * g + i]));
        scl[g] = a / 31.0f;
        maxs = fmaxf(maxs, scl[g]);
    }
    const uint16_t d16 = amv_f2h(maxs / 127.0f);
    const float df = amv_h2f(d16);
    int sc[16];
    for (int g = 0; g < 16; ++g) sc[g] = df > 0.0f ? min(127, (int)rintf(scl[g] / df)) : 0;
    uint8_t blk[210];
    for (int i = 0; i < 192; ++i) blk[i] = 0;
    for (int h = 0; h < 2; ++h) {
        for (int l = 0; l < 32; ++l) {
            int q[4];
            for (int s = 0; s < 4; ++s) {
                const int e = 128 * h + 32 * s + l;
                const float dl = df * (float)sc[e >> 4];
                int t = 0;
                if (dl > 0.0f) t = (int)rintf(xb[e] / dl);
                q[s] = min(31, max(-32, t)) + 32;
            }
            blk[64 * h + l] = (uint8_t)((q[0] & 15) | ((q[2] & 15) << 4));
            blk[64 * h + 32 + l] = (uint8_t)((q[1] & 15) | ((q[3] & 15) << 4));
            blk[128 + 32 * h + l] = (uint8_t)((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6));
        }
    }
    for (int g = 0; g < 16; ++g) blk[192 + g] = (uint8_t)(int8_t)sc[g];
    blk[208] = (uint8_t)(d16 & 0xFF);
    blk[209] = (uint8_t)(d16 >> 8);
    uint16_t* yb = reinterpret_cast<uint16_t*>(y + b * 210);
    for (int i = 0; i < 105; ++i) yb[i] = (uint16_t)(blk[2 * i] | (blk[2 * i + 1] << 8));
}

extern "C" int amv_quantize_k(int type, const float* x, int64_t n_rows, int64_t k, void* y_ggml, void* stream) {
    AMV_REQUIRE(x && y_ggml, "amv_quantize_k: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0 && k % 256 == 0, "amv_quantize_k: bad shape %lld x %lld", (long long)n_rows,
                (long long)k);
    const int64_t nsb = n_rows * (k / 256);
    if (type == AMV_T_Q4_K) {
        AMV_REQUIRE(((uintptr_t)y_ggml & 15) == 0, "amv_quantize_k: Q4_K output must be 16-byte aligned");
        hipLaunchKernelGGL(k_quant_q4_K, grid_for(nsb, 128), 128, 0, amv_stream(stream), x, nsb, (uint8_t*)y_ggml);
    } else if (type == AMV_T_Q6_K) {
        AMV_REQUIRE(((uintptr_t)y_ggml & 1) == 0, "amv_quantize_k: Q6_K output must be 2-byte aligned");
        hipLaunchKernelGGL(k_quant_q6_K, grid_for(nsb, 128), 128, 0, amv_stream(stream), x, nsb, (uint8_t*)y_ggml);
    } else {
        amv_set_error("amv_quantize_k: type %d is not a K-quant this library quantizes (12 Q4_K, 14 Q6_K)", type);
        return AMV_ERR_UNSUPPORTED;
    }
    return amv_check_launch("amv_quantize_k");
}
