// BitNet b1.58 I2_S: per-token absmax int8 activation quantization and the ternary GEMV.
//
// Role of bitnet_norm_q8.comp / bitnet_gemv_i2_s.comp (reference, src/shaders) and of the CPU path
// quantize_activation_int8 + ggml_vec_dot_i2_i8_s + bitnet_gemv (adapters/bitnet/src/cpu/llama_bitnet_core.cpp:914-941,
// ggml_bitnet_mad.cpp:191-231 scalar branch). Weight layout is the BitNet one, used in place (it is already
// row-major and 16-byte aligned per row when k % 64 == 0): row r is k/4 bytes; 128-weight blocks of 32 bytes; byte i of
// a block holds the 2-bit codes of weights i, 32 + i, 64 + i, 96 + i in bits 7-6, 5-4, 3-2, 1-0; weight = code - 1.
// y[r] = float(sum_j (c_rj - 1) q_j) * (act_dequant * weight_scale); the integer is formed exactly as
// sum_j c_rj q_j - sum_j q_j with v_dot4_i32_i8 (codes 0..3 are valid signed bytes).
#include "amv_common.h"

// ---------------------------------------------------------------------------------------------------------------
// quantize_activation_int8: one workgroup of 256 per row. max_abs starts at 1e-7, scale = 127 / max_abs,
// q = clamp(roundf(x * scale), -127, 127) (round half away from zero), dequant = 1 / scale, plus sum(q).
// Output layout: q int8 [m][k] | {f32 dequant, i32 sum q} [m].
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_i2s_quant(const float* __restrict__ x, int k, int8_t* __restrict__ q,
                                                  int2* __restrict__ meta) {
    __shared__ float smax[4];
    __shared__ int ssum[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* xr = x + (size_t)row * k;
    float amax = 1e-7f;
    for (int i = tid; i < k; i += 256) amax = fmaxf(amax, fabsf(xr[i]));
    amax = amv_wave_max(amax);
    if (lane == 0) smax[w] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    const float scale = 127.0f / amax;
    int s = 0;
    for (int i = tid; i < k; i += 256) {
        float v = roundf(xr[i] * scale);
        v = fminf(127.0f, fmaxf(-127.0f, v));
        q[(size_t)row * k + i] = (int8_t)(int)v;
        s += (int)v;
    }
    s = amv_wave_sum_i(s);
    if (lane == 0) ssum[w] = s;
    __syncthreads();
    if (tid == 0) meta[row] = make_int2(__float_as_int(1.0f / scale), ssum[0] + ssum[1] + ssum[2] + ssum[3]);
}

// ---------------------------------------------------------------------------------------------------------------
// GEMV: a wave owns R rows; the k/64 16-byte slices of a row go to the lanes (slice j: block j/2, bytes
// 16 (j%2) .. +15, i.e. weights 16 (j%2) + i + 32 g of the block). OUT_SUMS writes the exact integer per row.
// ---------------------------------------------------------------------------------------------------------------
template <int R, bool OUT_SUMS>
__global__ __launch_bounds__(256) void k_i2s_gemv(const uint4* __restrict__ w, int n_rows, int nsl,
                                                 const int8_t* __restrict__ q, const int2* __restrict__ meta,
                                                 float wscale, float* __restrict__ dst, int32_t* __restrict__ isums) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (row0 >= n_rows) return;
    const int4* a4 = reinterpret_cast<const int4*>(q);
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0;
    for (int j0 = 0; j0 < nsl; j0 += 64) {
        const int j = j0 + lane;
        const int jj = min(j, nsl - 1);
        uint4 c[R];
#pragma unroll
        for (int r = 0; r < R; ++r) c[r] = w[(size_t)min(row0 + r, n_rows - 1) * nsl + jj];
        if (j < nsl) {
            const int b = jj >> 1, p = jj & 1;
            int4 a[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) a[g] = a4[b * 8 + 2 * g + p];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int s = acc[r];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int sh = 6 - 2 * g;
                    s = amv_dot4((int)((c[r].x >> sh) & 0x03030303u), a[g].x, s);
                    s = amv_dot4((int)((c[r].y >> sh) & 0x03030303u), a[g].y, s);
                    s = amv_dot4((int)((c[r].z >> sh) & 0x03030303u), a[g].z, s);
                    s = amv_dot4((int)((c[r].w >> sh) & 0x03030303u), a[g].w, s);
                }
                acc[r] = s;
            }
        }
    }
    const int2 m = meta[0];
    const float total_scale = __int_as_float(m.x) * wscale;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int t = amv_wave_sum_i(acc[r]) - m.y;
        if (lane == 0 && row0 + r < n_rows) {
            if (OUT_SUMS) isums[row0 + r] = t;
            else dst[row0 + r] = (float)t * total_scale;
        }
    }
}

extern "C" int64_t amv_i2s_act_bytes(int64_t m, int64_t k) { return (m < 0 || k < 0) ? -1 : m * k + m * 8; }

extern "C" int amv_i2s_quantize_act(const float* x, int64_t m, int64_t k, void* act, void* stream) {
    AMV_REQUIRE(x && act, "amv_i2s_quantize_act: null pointer");
    AMV_REQUIRE(m > 0 && k > 0 && k <= INT32_MAX && m <= 65535 * 1024, "amv_i2s_quantize_act: bad shape");
    AMV_REQUIRE(((uintptr_t)act & 15) == 0, "amv_i2s_quantize_act: act must be 16-byte aligned");
    AMV_REQUIRE(k % 128 == 0, "amv_i2s_quantize_act: k %% 128 != 0");
    int8_t* q = (int8_t*)act;
    int2* meta = (int2*)((uint8_t*)act + m * k);
    hipLaunchKernelGGL(k_i2s_quant, dim3((unsigned)m), dim3(256), 0, amv_stream(stream), x, (int)k, q, meta);
    return amv_check_launch("amv_i2s_quantize_act");
}

static int i2s_gemv_impl(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float wscale,
                         float* dst, int64_t ldd, int32_t* sums, void* stream) {
    AMV_REQUIRE(w && act && (dst || sums), "amv_i2s_gemv: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0 && m > 0 && n_rows <= INT32_MAX, "amv_i2s_gemv: bad shape");
    AMV_REQUIRE(k % 128 == 0, "amv_i2s_gemv: k %% 128 != 0 (k = %lld)", (long long)k);
    AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0, "amv_i2s_gemv: buffers must be 16-byte aligned");
    AMV_REQUIRE(!dst || ldd >= n_rows, "amv_i2s_gemv: ldd < n_rows");
    hipStream_t st = amv_stream(stream);
    const int nsl = (int)(k / 64);
    const int R = 2;
    const int waves = (int)((n_rows + R - 1) / R);
    for (int64_t c = 0; c < m; ++c) {
        const int8_t* q = (const int8_t*)act + c * k;
        const int2* meta = (const int2*)((const uint8_t*)act + m * k) + c;
        if (sums) {
            hipLaunchKernelGGL((k_i2s_gemv<R, true>), dim3((waves + 3) / 4), dim3(256), 0, st, (const uint4*)w,
                               (int)n_rows, nsl, q, meta, wscale, nullptr, sums + c * n_rows);
        } else {
            hipLaunchKernelGGL((k_i2s_gemv<R, false>), dim3((waves + 3) / 4), dim3(256), 0, st, (const uint4*)w,
                               (int)n_rows, nsl, q, meta, wscale, dst + c * ldd, nullptr);
        }
    }
    return amv_check_launch("amv_i2s_gemv");
}

extern "C" int amv_i2s_gemv(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float weight_scale,
                            float* dst, int64_t ldd, void* stream) {
    AMV_REQUIRE(dst, "amv_i2s_gemv: null dst");
    return i2s_gemv_impl(w, n_rows, k, act, m, weight_scale, dst, ldd, nullptr, stream);
}

extern "C" int amv_i2s_gemv_sums(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                                 int32_t* sums, void* stream) {
    AMV_REQUIRE(sums, "amv_i2s_gemv_sums: null output");
    return i2s_gemv_impl(w, n_rows, k, act, m, 0.0f, nullptr, 0, sums, stream);
}
