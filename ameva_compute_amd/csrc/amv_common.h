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
__device__ __forceinline__ float amv_h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// signed 4x8-bit dot product with 32-bit accumulate (v_dot4_i32_i8)
__device__ __forceinline__ int amv_dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// wave64 butterfly sum: every lane ends with the total
__device__ __forceinline__ float amv_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, AMV_WAVE);
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
