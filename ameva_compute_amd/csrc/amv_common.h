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
// device: fp16 <-> f32 (v_cvt_f16_f32 rounds to nearest even; the conversion back is exact)
__device__ __forceinline__ uint16_t amv_f2h(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
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
