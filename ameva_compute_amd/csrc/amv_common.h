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

// wave64 sum: every lane ends with the total (DPP within rows, then two cross-row exchanges)
__device__ __forceinline__ float amv_wave_sum(float v) {
    v = amv_row16_sum(v);
    v += __shfl_xor(v, 16, AMV_WAVE);
    v += __shfl_xor(v, 32, AMV_WAVE);
    return v;
}
__device__ __forceinline__ int amv_wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, AMV_WAVE);
    return v;
}
__device__ __forceinline__ float amv_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, AMV_WAVE));
    return v;
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
