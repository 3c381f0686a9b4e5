// Shared device helpers and host-side error plumbing of the ameva MI355X (gfx950) library.
// Every translation unit is compiled with -ffp-contract=off and correctly rounded f32 division/sqrt, so that the
// quantizers reproduce the CPU's f32 rounding bit for bit; kernels that want fused multiply-adds call fmaf.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/ameva_hip.h"

// ggml_type values (include/ggml/ggml.h:394-437 of the reference)
enum {
    AMV_T_F32 = 0, AMV_T_F16 = 1, AMV_T_Q4_0 = 2, AMV_T_Q8_0 = 8, AMV_T_Q4_K = 12, AMV_T_Q6_K = 14,
    AMV_T_Q8_K = 15, AMV_T_I2_S = 36
};

#define AMV_WAVE 64

// Offsets (bytes) of the matrix-core extension of the AMV_ACT_Q8_K_MMA activation layout: after the Q8_K layout
// (rounded up to 16 bytes) come the int8 values as f16 [m][k], the sums per 16 as f16 [m][k/16] and the super-block
// scales transposed, f32 [k/256][m]; all exact copies (|sum of 16 int8| <= 2032 is exact in f16).
struct AmvQ8kMma {
    int64_t a16, bs16, dt, total;
};
static inline AmvQ8kMma amv_q8k_mma_layout(int64_t m, int64_t k) {
    AmvQ8kMma L;
    const int64_t q8k = m * k + m * (k / 256) * 4 + m * (k / 16) * 4;
    L.a16 = (q8k + 15) & ~(int64_t)15;
    L.bs16 = L.a16 + 2 * m * k;
    L.dt = (L.bs16 + 2 * m * (k / 16) + 15) & ~(int64_t)15;
    L.total = L.dt + 4 * m * (k / 256);
    return L;
}

// Offsets (bytes) of the AMV_ACT_Q8_0_MMA activation layout: after the Q8_0 layout (int8 [m][k], {f32 d, i32 sum}
// [m][k/32]; rounded up to 16 bytes) come the int8 values as f16 [m][k] (exact) and the block scales transposed, f32
// [k/32][m].
struct AmvQ80Mma {
    int64_t a16, dt, total;
};
static inline AmvQ80Mma amv_q8_0_mma_layout(int64_t m, int64_t k) {
    AmvQ80Mma L;
    const int64_t q80 = m * k + m * (k / 32) * 8;
    L.a16 = (q80 + 15) & ~(int64_t)15;
    L.dt = L.a16 + 2 * m * k;  // 2 m k is a multiple of 64 (k % 32 == 0)
    L.total = L.dt + 4 * m * (k / 32);
    return L;
}

// ---------------------------------------------------------------------------------------------------------------
// host: error state (first message of the failing call, per thread)
void amv_set_error(const char* fmt, ...);
int amv_check_launch(const char* what);

#define AMV_REQUIRE(cond, ...)                  \
    do {                                        \
        if (!(cond)) {                          \
            amv_set_error(__VA_ARGS__);         \
            return AMV_ERR_INVALID_ARG;         \
        }                                       \
    } while (0)

static inline hipStream_t amv_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// the per-device split-k workspace of the batched kernels (amv_splitk_workspace): fixed, never grown
#define AMV_SPLITK_WS_BYTES ((size_t)128 << 20)

// ---------------------------------------------------------------------------------------------------------------
// device: fp16 <-> f32
// f32 -> fp16 for stored quantization scales: IEEE round to nearest even done in integers, with ggml's NaN (0x7E00)
// and the sign of zero kept. The hardware conversion is not used here because the compiler folds a preceding
// multiplication into v_fma_mix (an fma with a +0 addend), which turns ggml's d = 0 / -8 = -0.0 into +0.0.
__device__ __forceinline__ uint16_t amv_f2h(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to infinity
    const int e = (int)(ax >> 23) - 127;
    uint32_t h, rest, half;
    if (e >= -14) {  // normal half: drop 13 mantissa bits
        h = ((uint32_t)(e + 15) << 10) | ((ax & 0x7FFFFFu) >> 13);
        rest = ax & 0x1FFFu;
        half = 0x1000u;
    } else if (e >= -25) {  // subnormal half: the 24-bit significand shifted right by -(e + 1) = 14..24 bits
        const uint32_t mf = (ax & 0x7FFFFFu) | 0x800000u;
        const int d = -(e + 1);
        h = mf >> d;
        rest = mf & ((1u << d) - 1u);
        half = 1u << (d - 1);
    } else {
        return (uint16_t)sign;
    }
    if (rest > half || (rest == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}
// f32 -> fp16 -> f32 rounding of a value loaded from memory (v_cvt_f16_f32, round to nearest even): one instruction,
// for rounding points of a computation (ggml's f16 q in flash attention); the stored scales above use amv_f2h.
__device__ __forceinline__ float amv_round_f16(float x) { return (float)(_Float16)x; }
// Streaming loads for data read once per launch (GEMV weights, KV rows): non-temporal, so the lines do not displace
// what is reused (activations) in L2 and the Infinity Cache. Measured on MI355X: a cold 33 MB read runs ~7 % faster.
// Only for loads whose wave instruction covers whole lines: a line that a later instruction reads again is fetched
// twice when the first read was non-temporal.
typedef unsigned int amv_v4u __attribute__((ext_vector_type(4)));
// Workgroup index -> tile index for a one-dimensional grid: MI355X hands workgroup i to XCD i % 8 and each XCD has its
// own L2, so consecutive tile indices (tiles that share an operand, ordered by the caller) go to one XCD: XCD x runs
// tiles x * g8 .. x * g8 + g8 - 1 (g8 = total / 8); the last total % 8 workgroups keep their index.
__device__ __forceinline__ int amv_xcd_tile(int id, int total) {
    const int g8 = total >> 3;
    return id < 8 * g8 ? (id & 7) * g8 + (id >> 3) : id;
}

__device__ __forceinline__ uint4 amv_ld_stream(const uint4* p) {
    const amv_v4u v = __builtin_nontemporal_load(reinterpret_cast<const amv_v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t amv_ld_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint16_t amv_ld_stream(const uint16_t* p) { return __builtin_nontemporal_load(p); }

__device__ __forceinline__ float amv_h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// Index (in fp16 units) of the scale of Q4_0 block j of row `row` in the repacked scale array: rows are paired,
// d[p][j][0..1] holding rows 2p and 2p + 1, so a wave owning both rows fetches the two scales with one dword; an
// odd last row follows as a plain run of nb scales. Same size as the ggml tensor.
__device__ __forceinline__ size_t amv_q4_0_didx(int row, int j, int nb, int n_rows) {
    const int ne = n_rows & ~1;
    return row < ne ? ((size_t)(row >> 1) * nb + j) * 2 + (row & 1) : (size_t)ne * nb + j;
}

// byte i (0..11) of the packed 6-bit scales held in three words
__device__ __forceinline__ uint32_t k4_byte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xFFu;
}
// get_scale_min_k4 of a Q4_K super-block (reference ameva_qdecode.glsl:229-236)
__device__ __forceinline__ void k4_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, int& sc, int& m) {
    if (j < 4) {
        sc = (int)(k4_byte(s0, s1, s2, j) & 63u);
        m = (int)(k4_byte(s0, s1, s2, j + 4) & 63u);
    } else {
        sc = (int)((k4_byte(s0, s1, s2, j + 4) & 0xFu) | ((k4_byte(s0, s1, s2, j - 4) >> 6) << 4));
        m = (int)((k4_byte(s0, s1, s2, j + 4) >> 4) | ((k4_byte(s0, s1, s2, j) >> 6) << 4));
    }
}

// Scales and mins of the unit pair 2c, 2c + 1 (c = 0..3, may vary per lane) without branches: byte pair c & 1 of each
// scale dword; for c >= 2 the 6-bit values are the low (scale) / high (min) nibbles of bytes 8..11 with the top two
// bits from bytes 0..3 (scales) / 4..7 (mins), as get_scale_min_k4.
__device__ __forceinline__ void k4_scale_min_pair(int c, uint32_t s0, uint32_t s1, uint32_t s2, int& sl, int& ml,
                                                  int& sh, int& mh) {
    const int sh16 = 16 * (c & 1);
    const uint32_t A = s0 >> sh16, B = s1 >> sh16, C = s2 >> sh16;
    const uint32_t scp = c < 2 ? (A & 0x3F3Fu) : ((C & 0x0F0Fu) | ((A >> 2) & 0x3030u));
    const uint32_t mp = c < 2 ? (B & 0x3F3Fu) : (((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u));
    sl = (int)(scp & 0xFFu);
    sh = (int)((scp >> 8) & 0xFFu);
    ml = (int)(mp & 0xFFu);
    mh = (int)((mp >> 8) & 0xFFu);
}

// signed 4x8-bit dot product with 32-bit accumulate (v_dot4_i32_i8)
__device__ __forceinline__ int amv_dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Sum over the 16 lanes of each DPP row (lanes 16 r .. 16 r + 15), result in every lane of the row, with DPP row
// permutations (VALU only, no LDS round trip): quad_perm [1,0,3,2] and [2,3,0,1] sum each quad, row_half_mirror
// (lane i <-> 7 - i) pairs the two quads of each 8, row_mirror (i <-> 15 - i) the two halves of the row.
#define AMV_DPP_ADD(v, ctrl) \
    ((v) + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), 0xF, 0xF, false)))
__device__ __forceinline__ float amv_row16_sum(float v) {
    v = AMV_DPP_ADD(v, 0xB1);   // quad_perm [1,0,3,2]
    v = AMV_DPP_ADD(v, 0x4E);   // quad_perm [2,3,0,1]
    v = AMV_DPP_ADD(v, 0x141);  // row_half_mirror
    v = AMV_DPP_ADD(v, 0x140);  // row_mirror
    return v;
}

// wave64 sum: every lane ends with the total, (row 0 + row 1) + (row 2 + row 3) of the DPP row sums, the four row
// totals read with v_readlane (no LDS round trip)
__device__ __forceinline__ float amv_wave_sum(float v) {
    const int i = __float_as_int(amv_row16_sum(v));
    return (__int_as_float(__builtin_amdgcn_readlane(i, 0)) + __int_as_float(__builtin_amdgcn_readlane(i, 16))) +
           (__int_as_float(__builtin_amdgcn_readlane(i, 32)) + __int_as_float(__builtin_amdgcn_readlane(i, 48)));
}
#define AMV_LOG2E 1.4426950408889634f
typedef _Float16 amv_h2 __attribute__((ext_vector_type(2)));  // scores kept in log2 units meet v_exp_f32 (2^x) directly

// Reductions over the lane pairs l, l ^ 16 and l, l ^ 32 without LDS (v_permlane16_swap / v_permlane32_swap trade
// the odd 16-lane rows / the upper half of the wave with the other copy): the same result in both lanes.
__device__ __forceinline__ float amv_max_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float amv_sum_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float amv_max_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float amv_sum_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wave-uniform reductions without LDS round trips: DPP within each 16-lane row, then the four row results read into
// scalar registers (rows summed in the order 0, 1, 2, 3). The result is the same in every lane.
template <int CTRL>
__device__ __forceinline__ int amv_dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ double amv_dpp_d(double v) {
    const int lo = amv_dpp_i<CTRL>(__double2loint(v)), hi = amv_dpp_i<CTRL>(__double2hiint(v));
    return __hiloint2double(hi, lo);
}
__device__ __forceinline__ int amv_wave_sum_i_u(int v) {
    v += amv_dpp_i<0xB1>(v);
    v += amv_dpp_i<0x4E>(v);
    v += amv_dpp_i<0x141>(v);
    v += amv_dpp_i<0x140>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}
__device__ __forceinline__ float amv_wave_max_u(float v) {
    v = fmaxf(v, __int_as_float(amv_dpp_i<0xB1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(amv_dpp_i<0x4E>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(amv_dpp_i<0x141>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(amv_dpp_i<0x140>(__float_as_int(v))));
    const int i = __float_as_int(v);
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(i, 0)), __int_as_float(__builtin_amdgcn_readlane(i, 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(i, 32)), __int_as_float(__builtin_amdgcn_readlane(i, 48))));
}
__device__ __forceinline__ double amv_wave_sum_d_u(double v) {
    v += amv_dpp_d<0xB1>(v);
    v += amv_dpp_d<0x4E>(v);
    v += amv_dpp_d<0x141>(v);
    v += amv_dpp_d<0x140>(v);
    const int lo = __double2loint(v), hi = __double2hiint(v);
    double t = __hiloint2double(__builtin_amdgcn_readlane(hi, 0), __builtin_amdgcn_readlane(lo, 0));
#pragma unroll
    for (int r = 16; r < 64; r += 16)
        t += __hiloint2double(__builtin_amdgcn_readlane(hi, r), __builtin_amdgcn_readlane(lo, r));
    return t;
}

// Q8_0 quantization of one 32-element block held one element per lane by 32 consecutive lanes of a wave (lane j of
// the block holds element j): the rules of amv_quantize_act (ggml quantize_row_q8_0 x86 / ARM / ref). Every lane of
// the 32 must call it. Writes the int8 of its element to qs[j]; lane j == 0 writes {fp16-rounded d, sum q} to *meta.
__device__ __forceinline__ void amv_q8_0_lanes32(float v, int rule, int j, int8_t* __restrict__ qs,
                                                 int2* __restrict__ meta) {
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
    qs[j] = (int8_t)q;
    if (j == 0) *meta = make_int2(__float_as_int(amv_h2f(amv_f2h(d))), s);
}
// Q8_0 quantization of one 32-element block spread over 8 consecutive lanes (4 elements each, lane j of the 8 holds
// elements 4j .. 4j + 3): the rules of amv_quantize_act. All 8 lanes must call it; stores 4 int8 per lane. The rule
// is uniform, so it is a branch to one of three instantiations rather than both roundings and both reciprocals in
// every lane.
template <int RULE>
__device__ __forceinline__ void q8_block_lanes8_r(const float (&v)[4], int j, int8_t* __restrict__ qs,
                                                  int2* __restrict__ meta) {
    // the 8 lanes' max and sum by DPP within the lane octet (xor 1, xor 2, mirror of the half row): exact, so the
    // order does not matter
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, __int_as_float(amv_dpp_i<0xB1>(__float_as_int(amax))));
    amax = fmaxf(amax, __int_as_float(amv_dpp_i<0x4E>(__float_as_int(amax))));
    amax = fmaxf(amax, __int_as_float(amv_dpp_i<0x141>(__float_as_int(amax))));
    const float d = amax / 127.0f;
    float id;
    if constexpr (RULE == AMV_Q8_X86) id = amax != 0.0f ? 127.0f / amax : 0.0f;
    else id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t packed = 0;
    int s = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float t = v[e] * id;
        float qf = RULE == AMV_Q8_REF ? roundf(t) : rintf(t);
        qf = fminf(127.0f, fmaxf(-127.0f, qf));
        const int q = (int)qf;
        s += q;
        packed |= (uint32_t)(q & 0xFF) << (8 * e);
    }
    s += amv_dpp_i<0xB1>(s);
    s += amv_dpp_i<0x4E>(s);
    s += amv_dpp_i<0x141>(s);
    reinterpret_cast<uint32_t*>(qs)[j] = packed;
    if (j == 0) *meta = make_int2(__float_as_int(amv_h2f(amv_f2h(d))), s);
}
__device__ __forceinline__ void q8_block_lanes8(const float (&v)[4], int rule, int j, int8_t* __restrict__ qs,
                                                int2* __restrict__ meta) {
    if (rule == AMV_Q8_X86) q8_block_lanes8_r<AMV_Q8_X86>(v, j, qs, meta);
    else if (rule == AMV_Q8_ARM) q8_block_lanes8_r<AMV_Q8_ARM>(v, j, qs, meta);
    else q8_block_lanes8_r<AMV_Q8_REF>(v, j, qs, meta);
}

// ---------------------------------------------------------------------------------------------------------------
// Q8_K quantization (ggml quantize_row_q8_K) of one 256-element block held by a whole wave, 4 consecutive elements
// per lane: max = the element of largest magnitude (the first on ties), iscale = -127/max, q = min(127,
// round-half-even(iscale * x)), d = 1/iscale; s16 = sum of q over the lane's group of 16 (lanes 4 i .. 4 i + 3), in
// every lane of the group. An all-zero block gives q = 0, d = 0.
struct AmvQ8K {
    int q[4];
    int s16;
    float d;
};
__device__ __forceinline__ AmvQ8K amv_q8_K_lanes64(const float (&v)[4], int lane) {
    AmvQ8K r;
    float am = 0.0f;
    int ai = 0x7FFFFFFF;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float a = fabsf(v[e]);
        if (a > am) { am = a; ai = 4 * lane + e; }
    }
    // (largest magnitude, then smallest index) is an exact, order-free choice: DPP within each row of 16 lanes (xor
    // 1, xor 2, half-row mirror, row mirror), then the four rows' picks through scalar registers
    const auto pick = [&](float om, int oi) {
        if (om > am || (om == am && oi < ai)) { am = om; ai = oi; }
    };
    pick(__int_as_float(amv_dpp_i<0xB1>(__float_as_int(am))), amv_dpp_i<0xB1>(ai));
    pick(__int_as_float(amv_dpp_i<0x4E>(__float_as_int(am))), amv_dpp_i<0x4E>(ai));
    pick(__int_as_float(amv_dpp_i<0x141>(__float_as_int(am))), amv_dpp_i<0x141>(ai));
    pick(__int_as_float(amv_dpp_i<0x140>(__float_as_int(am))), amv_dpp_i<0x140>(ai));
    {
        const int ab = __float_as_int(am);
        float bm = __int_as_float(__builtin_amdgcn_readlane(ab, 0));
        int bi = __builtin_amdgcn_readlane(ai, 0);
#pragma unroll
        for (int row = 16; row < 64; row += 16) {
            const float om = __int_as_float(__builtin_amdgcn_readlane(ab, row));
            const int oi = __builtin_amdgcn_readlane(ai, row);
            if (om > bm || (om == bm && oi < bi)) { bm = om; bi = oi; }
        }
        am = bm;
        ai = bi;
    }
    if (am == 0.0f) {
        r.q[0] = r.q[1] = r.q[2] = r.q[3] = 0;
        r.s16 = 0;
        r.d = 0.0f;
        return r;
    }
    const float vsel = (ai & 3) == 0 ? v[0] : ((ai & 3) == 1 ? v[1] : ((ai & 3) == 2 ? v[2] : v[3]));
    const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vsel), ai >> 2));
    const float iscale = -127.0f / mx;
    int s = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = (int)rintf(iscale * v[e]);
        r.q[e] = t < 127 ? t : 127;
        s += r.q[e];
    }
    s += amv_dpp_i<0xB1>(s);
    s += amv_dpp_i<0x4E>(s);
    r.s16 = s;
    r.d = 1.0f / iscale;
    return r;
}
__device__ __forceinline__ int amv_pack4(const int (&q)[4]) {
    return (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | ((q[3] & 0xFF) << 24);
}

// Activation output of a fused quantization: one row in the amv_quantize_act layout of its type. Q8_0: qs [n], then
// {f32 d, i32 sum q} per 32 at meta; Q8_K: qs [n], f32 d per 256 at meta, i32 sums per 16 at sums16.
struct AmvActOut {
    int8_t* qs;
    void* meta;
    int32_t* sums16;
    int type;  // AMV_T_Q8_0 or AMV_T_Q8_K; 0: no output
    int rule;  // Q8_0 rounding rule
};
// host: the descriptor of an activation of m rows of n values at act (amv_quantize_act layout); type 0 = none
static inline AmvActOut amv_act_out(void* act, int64_t n, int type, int rule, int64_t m = 1) {
    AmvActOut o{nullptr, nullptr, nullptr, 0, rule};
    if (!act || !type) return o;
    o.qs = (int8_t*)act;
    o.meta = (uint8_t*)act + m * n;
    o.sums16 = type == AMV_T_Q8_K ? (int32_t*)((uint8_t*)act + m * n + m * (n / 256) * 4) : nullptr;
    o.type = type;
    return o;
}
// the descriptor of row r of an m-row activation (amv_quantize_act layout: all rows' qs, then all rows' metadata)
__host__ __device__ inline AmvActOut amv_act_row(const AmvActOut& a, int64_t r, int64_t n) {
    AmvActOut o = a;
    if (!a.type) return o;
    o.qs = a.qs + r * n;
    if (a.type == AMV_T_Q8_0) {
        o.meta = reinterpret_cast<int2*>(a.meta) + r * (n / 32);
    } else {
        o.meta = reinterpret_cast<float*>(a.meta) + r * (n / 256);
        o.sums16 = a.sums16 + r * (n / 16);
    }
    return o;
}
// Quantizes the 4 consecutive values of float4 chunk c of the row. Q8_0: the 8 chunks of a 32-block must be in 8
// consecutive lanes; Q8_K: the 64 chunks of a 256-block must be the 64 lanes of one wave, in order.
__device__ __forceinline__ void amv_act_store4(const AmvActOut& o, int c, const float (&v)[4]) {
    if (o.type == AMV_T_Q8_0) {
        q8_block_lanes8(v, o.rule, c & 7, o.qs + 32 * (c >> 3), reinterpret_cast<int2*>(o.meta) + (c >> 3));
    } else if (o.type == AMV_T_Q8_K) {
        const AmvQ8K r = amv_q8_K_lanes64(v, c & 63);
        reinterpret_cast<int*>(o.qs)[c] = amv_pack4(r.q);
        if ((c & 3) == 0) o.sums16[c >> 2] = r.s16;
        if ((c & 63) == 0) reinterpret_cast<float*>(o.meta)[c >> 6] = r.d;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Data one workgroup hands to another inside a launch. The 8 XCDs of MI355X have private L2s; agent-scope fences
// make ordinary stores visible by writing back and invalidating the whole L2 (tens of us when every wave does it),
// so the handed-over values are instead stored and loaded with agent-scope relaxed atomics (sc1: coherent across
// the XCDs without touching the rest of the cache), and amv_arrive_last orders them with a wait on the wave's own
// memory counter.
__device__ __forceinline__ void amv_store_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float amv_load_coh(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 amv_load4_coh(const float* p) {
    return make_float4(amv_load_coh(p), amv_load_coh(p + 1), amv_load_coh(p + 2), amv_load_coh(p + 3));
}

// ---------------------------------------------------------------------------------------------------------------
// RMS_NORM of one row, shared by the norm kernel and the fused GEMV tail so that both produce the same bits. The
// sum of squares is defined for 1024 virtual lanes: lane t sums the float4 chunks t, t + 1024, ... as f32 squares in
// double, amv_wave_sum_d_u per virtual wave (DPP within each row of 16 lanes, then the four row sums in order), then
// the 16 wave sums by amv_rms_total. A workgroup of NT threads (NT
// divides 1024) plays V = 1024 / NT virtual lanes per thread (t = tid + NT v) and loads all V chunks of a round
// before summing, so a row of up to 1024 chunks costs one memory round trip (its w chunks load in the same one) and
// its values stay in registers for the second pass: y = x * scale, o = y * w, act = the quantized o (y without w). Any output may be NULL; the chunks
// of a quantization block sit in consecutive lanes as amv_act_store4 needs (n % 32 == 0 with Q8_0, % 256 with
// Q8_K).
#define AMV_RMS_VLANES 1024
// the 16 virtual-wave sums in a fixed order: lanes 0..15 of each row hold sred[0..15], DPP within the row (xor 1,
// xor 2, half-row mirror, row mirror), then lane 0's value, uniform over the wave. Every lane of the wave must call it.
__device__ __forceinline__ double amv_rms_total(const double* sred) {
    static_assert(AMV_RMS_VLANES / 64 == 16, "one row of 16 lanes holds the virtual-wave sums");
    double v = sred[threadIdx.x & 15];
    v += amv_dpp_d<0xB1>(v);
    v += amv_dpp_d<0x4E>(v);
    v += amv_dpp_d<0x141>(v);
    v += amv_dpp_d<0x140>(v);
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), 0),
                            __builtin_amdgcn_readlane(__double2loint(v), 0));
}
__device__ __forceinline__ float amv_rms_scale(double tot, int n, float eps) {
    const float mean = (float)(tot / (double)n);
    return 1.0f / sqrtf(mean + eps);
}
// chunk c of the second pass; wv = chunk c of w when has_w
__device__ __forceinline__ void amv_rms_chunk(int c, float4 v, float scale, bool has_w, float4 wv,
                                              float* __restrict__ y, float* __restrict__ o, const AmvActOut& act) {
    const float4 yv = make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
    if (y) reinterpret_cast<float4*>(y)[c] = yv;
    float4 qv = yv;
    if (has_w) {
        qv = make_float4(yv.x * wv.x, yv.y * wv.y, yv.z * wv.z, yv.w * wv.w);
        if (o) reinterpret_cast<float4*>(o)[c] = qv;
    }
    if (act.type) {
        const float vals[4] = {qv.x, qv.y, qv.z, qv.w};
        amv_act_store4(act, c, vals);
    }
}
template <int NT>
__device__ __forceinline__ void amv_rms_row(const float4* __restrict__ x4, int n4, float eps,
                                            const float* __restrict__ w, float* __restrict__ y,
                                            float* __restrict__ o, const AmvActOut& act, double* sred) {
    static_assert(AMV_RMS_VLANES % NT == 0 && NT % 64 == 0, "NT must divide 1024 in whole waves");
    constexpr int V = AMV_RMS_VLANES / NT;
    const int tid = threadIdx.x;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 xr[V], wr[V];
    double s[V];
#pragma unroll
    for (int v = 0; v < V; ++v) s[v] = 0.0;
    for (int k0 = 0; k0 < n4; k0 += AMV_RMS_VLANES) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int c = k0 + tid + NT * v;
            xr[v] = c < n4 ? x4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            // a row of one round: its w chunks load with x (one memory round trip for both)
            wr[v] = c < n4 && w && n4 <= AMV_RMS_VLANES ? w4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {  // absent chunks add exact zeros
            s[v] += (double)(xr[v].x * xr[v].x);
            s[v] += (double)(xr[v].y * xr[v].y);
            s[v] += (double)(xr[v].z * xr[v].z);
            s[v] += (double)(xr[v].w * xr[v].w);
        }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const double t = amv_wave_sum_d_u(s[v]);
        if ((tid & 63) == 0) sred[(tid + NT * v) >> 6] = t;
    }
    __syncthreads();
    const float scale = amv_rms_scale(amv_rms_total(sred), 4 * n4, eps);
    if (n4 <= AMV_RMS_VLANES) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int c = tid + NT * v;
            if (c < n4) amv_rms_chunk(c, xr[v], scale, w != nullptr, wr[v], y, o, act);
        }
    } else {
        for (int c = tid; c < n4; c += NT)
            amv_rms_chunk(c, x4[c], scale, w != nullptr, w ? w4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f), y, o, act);
    }
}

// amv_rms_row for a row of exactly 1024 float4 chunks (4096 values) with the MUL weight, in two parts so that a
// kernel can issue other loads between them: amv_rms1024_load issues the row's x and w loads (before anything else,
// so that waiting for them never waits for later loads), amv_rms1024_quant sums, meets in sred and writes the
// quantized row to act (any AmvActOut, one pointing to LDS included). Same arithmetic and order as amv_rms_row, so
// the same bytes.
template <int NT>
struct AmvRms1024 {
    static constexpr int V = AMV_RMS_VLANES / NT;
    float4 x[V], w[V];
};
template <int NT>
__device__ __forceinline__ void amv_rms1024_load(const float4* __restrict__ x4, const float4* __restrict__ w4,
                                                 AmvRms1024<NT>& r) {
#pragma unroll
    for (int v = 0; v < AmvRms1024<NT>::V; ++v) {
        r.x[v] = x4[threadIdx.x + NT * v];
        r.w[v] = w4[threadIdx.x + NT * v];
    }
}
template <int NT>
__device__ __forceinline__ void amv_rms1024_quant(const AmvRms1024<NT>& r, float eps, const AmvActOut& act,
                                                  double* sred) {
    constexpr int V = AmvRms1024<NT>::V;
    const int tid = threadIdx.x;
#pragma unroll
    for (int v = 0; v < V; ++v) {
        double t = 0.0;
        t += (double)(r.x[v].x * r.x[v].x);
        t += (double)(r.x[v].y * r.x[v].y);
        t += (double)(r.x[v].z * r.x[v].z);
        t += (double)(r.x[v].w * r.x[v].w);
        t = amv_wave_sum_d_u(t);
        if ((tid & 63) == 0) sred[(tid + NT * v) >> 6] = t;
    }
    __syncthreads();
    const float scale = amv_rms_scale(amv_rms_total(sred), 4096, eps);
#pragma unroll
    for (int v = 0; v < V; ++v) amv_rms_chunk(tid + NT * v, r.x[v], scale, true, r.w[v], nullptr, nullptr, act);
}

// amv_rms1024_quant with the activation type and the Q8_0 rule fixed at compile time (AT = AMV_T_Q8_0 with RULE, or
// AMV_T_Q8_K): the same arithmetic and bytes, without the code of the other types and rules in the kernel.
template <int NT, int AT, int RULE>
__device__ __forceinline__ void amv_rms1024_quant_t(const AmvRms1024<NT>& r, float eps, int8_t* __restrict__ qs,
                                                    void* __restrict__ meta, int32_t* __restrict__ sums16,
                                                    double* sred) {
    constexpr int V = AmvRms1024<NT>::V;
    const int tid = threadIdx.x;
#pragma unroll
    for (int v = 0; v < V; ++v) {
        double t = 0.0;
        t += (double)(r.x[v].x * r.x[v].x);
        t += (double)(r.x[v].y * r.x[v].y);
        t += (double)(r.x[v].z * r.x[v].z);
        t += (double)(r.x[v].w * r.x[v].w);
        t = amv_wave_sum_d_u(t);
        if ((tid & 63) == 0) sred[(tid + NT * v) >> 6] = t;
    }
    __syncthreads();
    const float scale = amv_rms_scale(amv_rms_total(sred), 4096, eps);
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int c = tid + NT * v;
        const float4 x = r.x[v], w = r.w[v];
        const float4 yv = make_float4(x.x * scale, x.y * scale, x.z * scale, x.w * scale);
        const float vals[4] = {yv.x * w.x, yv.y * w.y, yv.z * w.z, yv.w * w.w};
        if constexpr (AT == AMV_T_Q8_0) {
            q8_block_lanes8_r<RULE>(vals, c & 7, qs + 32 * (c >> 3), reinterpret_cast<int2*>(meta) + (c >> 3));
        } else {
            const AmvQ8K q = amv_q8_K_lanes64(vals, c & 63);
            reinterpret_cast<int*>(qs)[c] = amv_pack4(q.q);
            if ((c & 3) == 0) sums16[c >> 2] = q.s16;
            if ((c & 63) == 0) reinterpret_cast<float*>(meta)[c >> 6] = q.d;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// ROPE of one pair (x0, x1) with pair index j at position p: the angle freq_scale * (p * theta_scale^j) built by
// repeated f32 multiplication (ggml's rope f32, reference ameva_rope.comp:64-92). Shared by every ROPE kernel.
__device__ __forceinline__ void amv_rope_cs(float p, int j, float theta_scale, float freq_scale, float attn_factor,
                                            float& c, float& s) {
    float theta = p;
    for (int k = 0; k < j; ++k) theta *= theta_scale;
    const float ang = freq_scale * theta;
    c = cosf(ang) * attn_factor;
    s = sinf(ang) * attn_factor;
}
__device__ __forceinline__ void amv_rope_apply(float c, float s, float x0, float x1, float& y0, float& y1) {
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}
__device__ __forceinline__ void amv_rope_pair(float p, int j, float theta_scale, float freq_scale, float attn_factor,
                                              float x0, float x1, float& y0, float& y1) {
    float c, s;
    amv_rope_cs(p, j, theta_scale, freq_scale, attn_factor, c, s);
    amv_rope_apply(c, s, x0, x1, y0, y1);
}

// ---------------------------------------------------------------------------------------------------------------
// Last-arrival test of a launch-wide (or group-wide) tail: each of `target` workgroups calls it once, with every
// thread of the workgroup, after storing its handed-over values with amv_store_coh; it returns true in exactly one
// of them, the last to arrive, which may then read all of them with amv_load_coh (or after amv_acquire). Each wave first waits until its
// own stores have completed (s_waitcnt vmcnt(0)), so they are performed before the workgroup's arrival; the counter
// is an atomicInc that wraps at target, so it is back to zero for the next launch without a reset.
__device__ __forceinline__ bool amv_arrive_last(unsigned int* counter, unsigned int target) {
    __shared__ unsigned int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicInc(counter, target - 1u) == target - 1u ? 1u : 0u;
    __syncthreads();
    return s_last != 0u;
}
// Arrivals on one counter serialize at the memory side (~12 ns each on MI355X: 512 workgroups add ~6 us), so each
// counter sits in its own 128-byte line (AMV_CNT_STRIDE words) and a launch-wide tail meets in two levels: groups of
// AMV_ARRIVE_GROUP workgroups on counters[(1 + group) * stride], the last of each group on counters[0]. Returns true
// in the last workgroup of the launch.
#define AMV_CNT_STRIDE 32
#define AMV_ARRIVE_GROUP 16
__device__ __forceinline__ bool amv_arrive_last_tree(unsigned int* counters) {
    const unsigned int n = gridDim.x, gi = blockIdx.x / AMV_ARRIVE_GROUP;
    const unsigned int n_groups = (n + AMV_ARRIVE_GROUP - 1) / AMV_ARRIVE_GROUP;
    const unsigned int gsize = min((unsigned int)AMV_ARRIVE_GROUP, n - gi * AMV_ARRIVE_GROUP);
    if (!amv_arrive_last(counters + AMV_CNT_STRIDE * (1 + gi), gsize)) return false;
    return amv_arrive_last(counters, n_groups);
}
// Instead of amv_load_coh for a larger read: one agent-scope acquire (invalidates this XCD's L2 once), after which
// ordinary (float4) loads see the handed-over values. For a workgroup that runs once per launch.
__device__ __forceinline__ void amv_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
