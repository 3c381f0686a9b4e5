// The kernels of the BitNet b1.58 token step that the ternary GEMV does not cover (the per-token engine of the
// reference, adapters/bitnet/src/core/ac_bitnet_engine.cpp:246-351, whose arithmetic follows the CPU path
// adapters/bitnet/src/cpu/llama_bitnet_core.cpp:886-1117):
//   k_bitnet_norm_q8   the FFN activation (relu(gate)^2 * up or silu(gate) * up) when asked, RMS_NORM with an optional
//                      weight when asked, and quantize_activation_int8 of the result, one row per workgroup;
//   k_bitnet_rope_kv   RoPE of q and k (apply_rope: pairs i, i + head_dim / 2) from a cos / sin table, k and v into
//                      the f32 cache row of the position held in device memory;
//   k_gemv_f16         y = W x with f16 weight rows and f32 x (the f16 LM head).
// The attention over the f32 cache is the split kernel of amv_attn.hip (cache type F32).
#include "amv_common.h"

#define BN_THREADS 1024
#define BN_MAX_PER_THREAD 16  // rows up to 16384 elements

// mode 0: x = a; 1: x = relu(a)^2 * b; 2: x = silu(a) * b (forward_swiglu, llama_bitnet_core.cpp:1093-1105).
// do_norm: x = x * (1 / sqrt(sum x^2 / n + eps)) * w (w NULL: no weight; rms_norm :886-912). The sum of squares is
// taken in double (the exact value the CPU's f32 loop approximates). y (may be NULL) receives x; act (may be NULL) the
// int8 activation of x in the layout of amv_i2s_quantize_act (q [n] | {f32 dequant, i32 sum q}), by
// quantize_activation_int8 (:914-926).
__global__ __launch_bounds__(BN_THREADS) void k_bitnet_norm_q8(const float* __restrict__ a, const float* __restrict__ b,
                                                              const float* __restrict__ w, int n, float eps, int mode,
                                                              int do_norm, float* __restrict__ y,
                                                              int8_t* __restrict__ q, int2* __restrict__ meta) {
    __shared__ double sd[BN_THREADS / 64];
    __shared__ float sf[BN_THREADS / 64];
    __shared__ int si[BN_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float v[BN_MAX_PER_THREAD];
#pragma unroll
    for (int e = 0; e < BN_MAX_PER_THREAD; ++e) {
        const int i = tid + e * BN_THREADS;
        float x = 0.0f;
        if (i < n) {
            x = a[i];
            if (mode == 1) {
                const float r = x > 0.0f ? x : 0.0f;
                x = (r * r) * b[i];
            } else if (mode == 2) {
                x = (x / (1.0f + expf(-x))) * b[i];
            }
        }
        v[e] = x;
    }
    if (do_norm) {
        double s = 0.0;
#pragma unroll
        for (int e = 0; e < BN_MAX_PER_THREAD; ++e) s += (double)v[e] * (double)v[e];
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, AMV_WAVE);
        if (lane == 0) sd[wv] = s;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int i = 0; i < BN_THREADS / 64; ++i) tot += sd[i];
        const float scale = 1.0f / sqrtf((float)tot / (float)n + eps);
#pragma unroll
        for (int e = 0; e < BN_MAX_PER_THREAD; ++e) {
            const int i = tid + e * BN_THREADS;
            if (i < n) v[e] = w ? (v[e] * scale) * w[i] : v[e] * scale;
        }
    }
    if (y) {
#pragma unroll
        for (int e = 0; e < BN_MAX_PER_THREAD; ++e) {
            const int i = tid + e * BN_THREADS;
            if (i < n) y[i] = v[e];
        }
    }
    if (!q) return;
    float amax = 1e-7f;
#pragma unroll
    for (int e = 0; e < BN_MAX_PER_THREAD; ++e)
        if (tid + e * BN_THREADS < n) amax = fmaxf(amax, fabsf(v[e]));
    amax = amv_wave_max(amax);
    if (lane == 0) sf[wv] = amax;
    __syncthreads();
    amax = sf[0];
#pragma unroll
    for (int i = 1; i < BN_THREADS / 64; ++i) amax = fmaxf(amax, sf[i]);
    const float scale = 127.0f / amax;
    int s = 0;
#pragma unroll
    for (int e = 0; e < BN_MAX_PER_THREAD; ++e) {
        const int i = tid + e * BN_THREADS;
        if (i < n) {
            float t = roundf(v[e] * scale);
            t = fminf(127.0f, fmaxf(-127.0f, t));
            q[i] = (int8_t)(int)t;
            s += (int)t;
        }
    }
    s = amv_wave_sum_i(s);
    if (lane == 0) si[wv] = s;
    __syncthreads();
    if (tid == 0) {
        int tot = 0;
        for (int i = 0; i < BN_THREADS / 64; ++i) tot += si[i];
        *meta = make_int2(__float_as_int(1.0f / scale), tot);
    }
}

extern "C" int amv_bitnet_norm_q8(const float* a, const float* b, const float* w, int64_t n, float eps, int mode,
                                  int do_norm, float* y, void* act, void* stream) {
    AMV_REQUIRE(a && (y || act), "amv_bitnet_norm_q8: null pointer");
    AMV_REQUIRE(mode >= 0 && mode <= 2 && (mode == 0 || b), "amv_bitnet_norm_q8: mode %d (0 plain, 1 relu2, 2 silu) "
                "needs the second operand for 1 and 2", mode);
    AMV_REQUIRE(n > 0 && n <= (int64_t)BN_THREADS * BN_MAX_PER_THREAD, "amv_bitnet_norm_q8: n %lld out of range",
                (long long)n);
    AMV_REQUIRE(!act || (((uintptr_t)act & 15) == 0 && n % 16 == 0), "amv_bitnet_norm_q8: act must be 16-byte aligned");
    int8_t* q = (int8_t*)act;
    int2* meta = act ? (int2*)((uint8_t*)act + n) : nullptr;
    hipLaunchKernelGGL(k_bitnet_norm_q8, dim3(1), dim3(BN_THREADS), 0, amv_stream(stream), a, b, w, (int)n, eps, mode,
                       do_norm, y, q, meta);
    return amv_check_launch("amv_bitnet_norm_q8");
}

// apply_rope (llama_bitnet_core.cpp:1006-1020) with the factors of the position precomputed in cs ([cos 0..h-1,
// sin 0..h-1], h = head_dim / 2): x_i' = x_i cos - x_{i+h} sin, x_{i+h}' = x_{i+h} cos + x_i sin. q (n_head heads)
// rotates in place; k (n_head_kv heads) rotates into row pos[0] of k_cache, v is copied into row pos[0] of v_cache
// (rows of n_head_kv * head_dim floats, store_kv_cache :1022-1031). One thread per rotated pair or copied value.
__global__ __launch_bounds__(256) void k_bitnet_rope_kv(float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, const float* __restrict__ cs,
                                                       float* __restrict__ k_cache, float* __restrict__ v_cache,
                                                       const int* __restrict__ pos, int n_head, int n_head_kv, int hd,
                                                       int n_ctx) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int h2 = hd / 2, kv = n_head_kv * hd;
    const int p = min(max(*pos, 0), n_ctx - 1);  // the host checks the position; clamped for memory safety
    float* krow = k_cache + (size_t)p * kv;
    float* vrow = v_cache + (size_t)p * kv;
    const int nq = n_head * h2, nk = n_head_kv * h2;
    if (t < nq + nk) {
        const int hp = t < nq ? t : t - nq;
        const int head = hp / h2, i = hp % h2;
        const float c = cs[i], s = cs[h2 + i];
        if (t < nq) {
            float* hq = q + (size_t)head * hd;
            const float v0 = hq[i], v1 = hq[i + h2];
            hq[i] = v0 * c - v1 * s;
            hq[i + h2] = v1 * c + v0 * s;
        } else {
            const float* hk = k + (size_t)head * hd;
            const float v0 = hk[i], v1 = hk[i + h2];
            krow[head * hd + i] = v0 * c - v1 * s;
            krow[head * hd + i + h2] = v1 * c + v0 * s;
        }
    } else if (t < nq + nk + kv) {
        const int i = t - nq - nk;
        vrow[i] = v[i];
    }
}

extern "C" int amv_bitnet_rope_kv(float* q, const float* k, const float* v, const float* cs, float* k_cache,
                                  float* v_cache, const int32_t* pos, int64_t n_head, int64_t n_head_kv, int64_t hd,
                                  int64_t n_ctx, void* stream) {
    AMV_REQUIRE(q && k && v && cs && k_cache && v_cache && pos, "amv_bitnet_rope_kv: null pointer");
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && hd > 0 && hd % 2 == 0 && n_ctx > 0 && n_head * hd <= (1 << 24),
                "amv_bitnet_rope_kv: bad shape");
    const int64_t total = (n_head + n_head_kv) * (hd / 2) + n_head_kv * hd;
    hipLaunchKernelGGL(k_bitnet_rope_kv, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream), q, k,
                       v, cs, k_cache, v_cache, pos, (int)n_head, (int)n_head_kv, (int)hd, (int)n_ctx);
    return amv_check_launch("amv_bitnet_rope_kv");
}

// y[r] = sum_c f16(W[r][c]) x[c] (bitnet_gemv for an F16 weight, llama_bitnet_core.cpp:964-996): R = 2 rows per wave,
// 8 weights (16 bytes, a streaming load) per lane and step, f32 sums reduced over the wave. k % 8 == 0.
__global__ __launch_bounds__(256) void k_gemv_f16(const uint4* __restrict__ w, int n_rows, int k8,
                                                 const float4* __restrict__ x, float* __restrict__ y) {
    constexpr int R = 2;
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= n_rows) return;
    float acc[R] = {0.0f, 0.0f};
    for (int j = lane; j < k8; j += 64) {
        const float4 xa = x[2 * j], xb = x[2 * j + 1];
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint4 u = amv_ld_stream(w + (size_t)min(row0 + r, n_rows - 1) * k8 + j);
            const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
            float s = acc[r];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s = fmaf(amv_h2f(uw[e] & 0xFFFFu), xv[2 * e], s);
                s = fmaf(amv_h2f(uw[e] >> 16), xv[2 * e + 1], s);
            }
            acc[r] = s;
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float t = amv_wave_sum(acc[r]);
        if (lane == 0 && row0 + r < n_rows) y[row0 + r] = t;
    }
}

extern "C" int amv_gemv_f16(const void* w, int64_t n_rows, int64_t k, const float* x, float* y, void* stream) {
    AMV_REQUIRE(w && x && y, "amv_gemv_f16: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0 && k % 8 == 0 && n_rows <= INT32_MAX && k / 8 <= INT32_MAX,
                "amv_gemv_f16: bad shape (k %% 8 == 0)");
    AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0, "amv_gemv_f16: w and x must be 16-byte aligned");
    const int64_t waves = (n_rows + 1) / 2;
    hipLaunchKernelGGL(k_gemv_f16, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, amv_stream(stream),
                       (const uint4*)w, (int)n_rows, (int)(k / 8), (const float4*)x, y);
    return amv_check_launch("amv_gemv_f16");
}
