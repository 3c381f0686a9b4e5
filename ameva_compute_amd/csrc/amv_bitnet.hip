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

#include <algorithm>

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
        s = amv_wave_sum_d_u(s);  // DPP within rows, readlane across them: no LDS round trip per step
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
    amax = amv_wave_max_u(amax);
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
    s = amv_wave_sum_i_u(s);
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

// ---------------------------------------------------------------------------------------------------------------
// One launch per projection group of the BitNet token step: the activation of the group's input vector (FFN
// activation, RMS_NORM, quantize_activation_int8 exactly as k_bitnet_norm_q8) is computed by EVERY workgroup into its
// own LDS, then the workgroup's rows of up to three stacked I2_S matrices (Q | K | V, or gate | up) are dotted against
// it from LDS. The input vector is a few KB and sits in L2, so recomputing it per workgroup costs less than the
// launch and the global round trip it replaces; the weight rows of the wave are requested right after the prologue's
// own loads and arrive while it runs. Epilogue per row: float(isum - sum q) * (dequant * scale_of_its_matrix), written
// or added (the residual add). ROPE: the wave's rows are pairs (i, i + 64) of one 128-row head (rows of every matrix
// are a multiple of 128), so the rotation of apply_rope is done in registers with the position's cos / sin table, q is
// written rotated, k rotated and v as is into the f32 cache rows of the position read from device memory (the
// separate k_bitnet_rope_kv path computes the same values).
// NT threads (NT / 64 waves, R rows per wave), V4 float4 of the input per thread: k <= 4 * NT * V4. Reductions are
// DPP within rows plus readlanes (no LDS round trips), and every load before the first barrier is unconditional.
// ---------------------------------------------------------------------------------------------------------------

struct BnSegs {
    const uint4* w[3];  // rows of matrix s: [end[s - 1], end[s]), each k / 4 bytes
    float* dst[3];
    float wscale[3];
    int end[3];
};

__device__ __forceinline__ int bn_seg(const BnSegs& sg, int r) { return r < sg.end[0] ? 0 : (r < sg.end[1] ? 1 : 2); }
// field s of the segment table by selects over constant indices: an indexed read of the kernel-argument struct
// becomes a vector load from memory with a full wait in front of the weight loads
template <typename T>
__device__ __forceinline__ T bn_pick(int s, T v0, T v1, T v2) { return s == 0 ? v0 : (s == 1 ? v1 : v2); }
__device__ __forceinline__ int bn_beg(const BnSegs& sg, int s) { return bn_pick(s, 0, sg.end[0], sg.end[1]); }

// MODE 3 input: the flash-attention split partials of amv_flash_attn_split_kv (per head h and split z, BN_FA_PS
// floats at part + (h * n_split + z) * BN_FA_PS: m, l, two pad, acc[128]), merged per element in the prologue; the
// key count from n_kv[0] (capped at n_kv_max) gives the splits holding keys, at most BN_FA_ZM
#define BN_FA_PS 132
#define BN_FA_ZM 4
struct BnFa {
    const float* part;
    const int* n_kv;
    int n_split, split_len, n_kv_max;
};

template <int MODE>
__device__ __forceinline__ float bn_act_t(float x, float y) {
    if constexpr (MODE == 1) {
        const float r = x > 0.0f ? x : 0.0f;
        return (r * r) * y;
    } else if constexpr (MODE == 2) {
        return (x / (1.0f + expf(-x))) * y;
    } else {
        return x;
    }
}

template <int NT, int V4, bool ROPE, int MODE, int R>
__global__ __launch_bounds__(NT) void k_bitnet_qgemv(const float4* __restrict__ a, const float4* __restrict__ b,
                                                    const float4* __restrict__ nw, int k, float eps, int do_norm, const BnSegs sg, int n_seg, int accumulate,
                                                    const float* __restrict__ cs, const int* __restrict__ pos,
                                                    int n_ctx, const BnFa fa) {
    constexpr int NW = NT / 64, NIT = (NT * V4 + 1023) / 1024;  // k <= 4 NT V4: 16-byte weight slices <= 64 NIT
    __shared__ __align__(16) int sq[NT * V4];  // the int8 activation, 4 per int
    __shared__ double sd[NW];
    __shared__ float sf[NW];
    __shared__ int si[NW];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n_rows = sg.end[n_seg - 1];
    const int wave = blockIdx.x * NW + wv;
    // rows of the wave: R consecutive rows, or with ROPE R / 2 pairs (i, i + 64) of one 128-row head
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (ROPE) {
            constexpr int PW = 64 / (R / 2);  // waves per head
            const int i = (wave % PW) + PW * (r >> 1);
            rows[r] = (wave / PW) * 128 + i + 64 * (r & 1);
        } else {
            rows[r] = R * wave + r;
        }
    }
    const bool active = rows[0] < n_rows;  // uniform per wave; every wave takes part in the prologue
    const int nsl = k >> 6;                // 16-byte slices per weight row
    // prologue: x = act(a, b); v = RMS_NORM(x) (* w); q = int8(v). Its loads are issued first and the weight rows
    // of the wave right after them: loads complete in order, so the prologue waits only for its own data while the
    // weights stream in.
    const int n4 = k >> 2;
    // every load is unconditional (an absent norm_w reads a instead; rows past the end read the last row): a load
    // under a branch makes the wait at the join conservative, i.e. a wait for the weights before the prologue
    const float4* wp = nw ? nw : a;
    float4 xv[V4], bv[V4], wn[V4];
    constexpr int VP = MODE == 3 ? V4 : 1;
    float4 pv[VP][BN_FA_ZM];  // MODE 3: acc of splits 0 .. BN_FA_ZM - 1 of the thread's float4s (head i4 / 32)
    float2 pml[VP][BN_FA_ZM];  // and their (m, l)
    // MODE 3: the key count first, a scalar load whose wait does not cover the vector loads below
    const int fa_nkv = MODE == 3 ? *fa.n_kv : 0;
    if constexpr (MODE == 3) {
#pragma unroll
        for (int u = 0; u < V4; ++u) {
            const int i4 = min(tid + NT * u, n4 - 1);
            const float* ph = fa.part + (size_t)(i4 >> 5) * fa.n_split * BN_FA_PS;
#pragma unroll
            for (int z = 0; z < BN_FA_ZM; ++z) {
                const float* pz = ph + (size_t)min(z, fa.n_split - 1) * BN_FA_PS;
                pv[u][z] = *reinterpret_cast<const float4*>(pz + 4 + 4 * (i4 & 31));
                pml[u][z] = *reinterpret_cast<const float2*>(pz);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < V4; ++u) xv[u] = a[min(tid + NT * u, n4 - 1)];
    }
    if constexpr (MODE == 1 || MODE == 2) {
#pragma unroll
        for (int u = 0; u < V4; ++u) bv[u] = b[min(tid + NT * u, n4 - 1)];
    }
#pragma unroll
    for (int u = 0; u < V4; ++u) wn[u] = wp[min(tid + NT * u, n4 - 1)];
    __builtin_amdgcn_sched_barrier(0);  // keep the weight loads behind the prologue's
    uint4 c[R][NIT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(rows[r], n_rows - 1);
        const int s = bn_seg(sg, row);
        const uint4* wr = bn_pick(s, sg.w[0], sg.w[1], sg.w[2]) + (size_t)(row - bn_beg(sg, s)) * nsl;
#pragma unroll
        for (int it = 0; it < NIT; ++it) c[r][it] = amv_ld_stream(wr + min(it * 64 + lane, nsl - 1));
    }
    if constexpr (MODE == 3) {
        // the split merge of k_fa_combine, per element and in its order, so the result is bit-identical to the
        // merged attention row: M = max m_z, w_z = 2^(m_z - M) (0 for an empty split), L = (l_0 w_0 + l_1 w_1) +
        // (l_2 w_2 + l_3 w_3) (the wave sum's DPP order over splits in lanes 0..3), t = sum over the 8 split groups
        // in order of fma(w_z, acc_z, 0), x = t / L (0 when L = 0). Splits past the count are masked with integer
        // masks, never selected as loaded values.
        const int nkv = max(0, min(fa_nkv, fa.n_kv_max));
        const int ns = (nkv + fa.split_len - 1) / fa.split_len;
#pragma unroll
        for (int u = 0; u < V4; ++u) {
            float mz[BN_FA_ZM], w[BN_FA_ZM], lw[BN_FA_ZM];
            uint32_t km[BN_FA_ZM];
            float M = -INFINITY;
#pragma unroll
            for (int z = 0; z < BN_FA_ZM; ++z) {
                km[z] = z < ns ? 0xFFFFFFFFu : 0u;
                mz[z] = __uint_as_float((__float_as_uint(pml[u][z].x) & km[z]) | (0xFF800000u & ~km[z]));
                M = fmaxf(M, mz[z]);
            }
#pragma unroll
            for (int z = 0; z < BN_FA_ZM; ++z) {
                w[z] = mz[z] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mz[z] - M);
                lw[z] = fmaf(__uint_as_float(__float_as_uint(pml[u][z].y) & km[z]), w[z], 0.0f);
            }
            const float L = (lw[0] + lw[1]) + (lw[2] + lw[3]);
            float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int z = 0; z < BN_FA_ZM; ++z) {
                const float4 v = pv[u][z];
                t[0] += fmaf(w[z], __uint_as_float(__float_as_uint(v.x) & km[z]), 0.0f);
                t[1] += fmaf(w[z], __uint_as_float(__float_as_uint(v.y) & km[z]), 0.0f);
                t[2] += fmaf(w[z], __uint_as_float(__float_as_uint(v.z) & km[z]), 0.0f);
                t[3] += fmaf(w[z], __uint_as_float(__float_as_uint(v.w) & km[z]), 0.0f);
            }
#pragma unroll
            for (int z = BN_FA_ZM; z < 8; ++z)  // the empty split groups add +0 (turning a -0 sum into +0)
#pragma unroll
                for (int e = 0; e < 4; ++e) t[e] += 0.0f;
            xv[u] = L == 0.0f ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                              : make_float4(t[0] / L, t[1] / L, t[2] / L, t[3] / L);
        }
    }
    // branch-free from here to the first barrier (a branch would let the compiler sink the prologue loads behind
    // the weight loads): scale 1 without the norm and weight 1 without norm_w (x * 1 = x)
#pragma unroll
    for (int u = 0; u < V4; ++u) {
        const bool in = tid + NT * u < n4;
        if constexpr (MODE == 1 || MODE == 2) {
            xv[u].x = bn_act_t<MODE>(xv[u].x, bv[u].x);
            xv[u].y = bn_act_t<MODE>(xv[u].y, bv[u].y);
            xv[u].z = bn_act_t<MODE>(xv[u].z, bv[u].z);
            xv[u].w = bn_act_t<MODE>(xv[u].w, bv[u].w);
        }
        if (!in) xv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    double ss = 0.0;
#pragma unroll
    for (int u = 0; u < V4; ++u)
        ss += (double)xv[u].x * xv[u].x + (double)xv[u].y * xv[u].y + (double)xv[u].z * xv[u].z +
              (double)xv[u].w * xv[u].w;
    ss = amv_wave_sum_d_u(ss);  // DPP within rows, readlane across them: no LDS round trip per step
    if (lane == 0) sd[wv] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < NW; ++i) tot += sd[i];
    const float scale = do_norm ? 1.0f / sqrtf((float)tot / (float)k + eps) : 1.0f;
    const bool use_w = do_norm && nw;
#pragma unroll
    for (int u = 0; u < V4; ++u) {
        xv[u].x = (xv[u].x * scale) * (use_w ? wn[u].x : 1.0f);
        xv[u].y = (xv[u].y * scale) * (use_w ? wn[u].y : 1.0f);
        xv[u].z = (xv[u].z * scale) * (use_w ? wn[u].z : 1.0f);
        xv[u].w = (xv[u].w * scale) * (use_w ? wn[u].w : 1.0f);
    }
    float amax = 1e-7f;
#pragma unroll
    for (int u = 0; u < V4; ++u)
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xv[u].x), fabsf(xv[u].y)), fmaxf(fabsf(xv[u].z), fabsf(xv[u].w))));
    amax = amv_wave_max_u(amax);
    if (lane == 0) sf[wv] = amax;
    __syncthreads();
    amax = sf[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) amax = fmaxf(amax, sf[i]);
    const float qs = 127.0f / amax;
    int isum = 0;
#pragma unroll
    for (int u = 0; u < V4; ++u) {
        const int i = tid + NT * u;
        if (i < n4) {
            const float t[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
            uint32_t packed = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int qi = (int)fminf(127.0f, fmaxf(-127.0f, roundf(t[e] * qs)));
                isum += qi;
                packed |= (uint32_t)(qi & 0xFF) << (8 * e);
            }
            sq[i] = (int)packed;
        }
    }
    isum = amv_wave_sum_i_u(isum);
    if (lane == 0) si[wv] = isum;
    __syncthreads();
    int qsum = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) qsum += si[i];
    if (!active) return;
    // the ternary dots from LDS (lane j: 16 weight bytes = 64 weights of 128-block j / 2, half j % 2)
    const int4* aq = reinterpret_cast<const int4*>(sq);
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int j = it * 64 + lane;
        if (j < nsl) {
            const int bb = j >> 1, p = j & 1;
            int4 av[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) av[g] = aq[bb * 8 + 2 * g + p];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int s = acc[r];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int sh = 6 - 2 * g;
                    s = amv_dot4((int)((c[r][it].x >> sh) & 0x03030303u), av[g].x, s);
                    s = amv_dot4((int)((c[r][it].y >> sh) & 0x03030303u), av[g].y, s);
                    s = amv_dot4((int)((c[r][it].z >> sh) & 0x03030303u), av[g].z, s);
                    s = amv_dot4((int)((c[r][it].w >> sh) & 0x03030303u), av[g].w, s);
                }
                acc[r] = s;
            }
        }
    }
    const float dq = 1.0f / qs;
    int t[R];
#pragma unroll
    for (int r = 0; r < R; ++r) t[r] = amv_wave_sum_i_u(acc[r]) - qsum;
    if (lane != 0) return;
    if (ROPE) {
        const int s = bn_seg(sg, rows[0]);  // every row of the wave is in one matrix (128-row heads)
        const int beg = bn_beg(sg, s);
        const float ts = dq * bn_pick(s, sg.wscale[0], sg.wscale[1], sg.wscale[2]);
        const int width = sg.end[1] - sg.end[0];     // K and V rows are equal (checked on the host)
        const int p = min(max(*pos, 0), n_ctx - 1);  // the host checks the position; clamped for memory safety
#pragma unroll
        for (int h = 0; h < R / 2; ++h) {
            const int r0 = rows[2 * h], r1 = rows[2 * h + 1];
            const float v0 = (float)t[2 * h] * ts, v1 = (float)t[2 * h + 1] * ts;
            const int i = r0 & 127, local = r0 - beg;
            if (s == 0) {
                const float cc = cs[i], sn = cs[64 + i];
                sg.dst[0][r0] = v0 * cc - v1 * sn;
                sg.dst[0][r1] = v1 * cc + v0 * sn;
            } else {
                float* row = (s == 1 ? sg.dst[1] : sg.dst[2]) + (size_t)p * width + local;
                if (s == 1) {
                    const float cc = cs[i], sn = cs[64 + i];
                    row[0] = v0 * cc - v1 * sn;
                    row[64] = v1 * cc + v0 * sn;
                } else {
                    row[0] = v0;
                    row[64] = v1;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = rows[r];
        if (row >= n_rows) break;
        const int s = bn_seg(sg, row);
        const float out = (float)t[r] * (dq * bn_pick(s, sg.wscale[0], sg.wscale[1], sg.wscale[2]));
        float* d = bn_pick(s, sg.dst[0], sg.dst[1], sg.dst[2]) + (row - bn_beg(sg, s));
        if (accumulate) *d = *d + out;
        else *d = out;
    }
}

extern "C" int amv_bitnet_gemv_fused(const float* a, const float* b, const float* norm_w, int64_t k, float eps,
                                     int mode, int do_norm, int n_seg, const void* const* w, const int64_t* rows,
                                     const float* wscale, float* const* dst, int accumulate, const float* rope_cs,
                                     const int32_t* pos, int64_t n_ctx, void* stream) {
    AMV_REQUIRE(a && w && rows && wscale && dst, "amv_bitnet_gemv_fused: null pointer");
    AMV_REQUIRE(mode >= 0 && mode <= 2 && (mode == 0 || b), "amv_bitnet_gemv_fused: mode %d (0 plain, 1 relu2, 2 silu) "
                "needs the second operand for 1 and 2", mode);
    AMV_REQUIRE(k > 0 && k % 128 == 0 && k <= 16384, "amv_bitnet_gemv_fused: k %lld (a multiple of 128, <= 16384)",
                (long long)k);
    AMV_REQUIRE(n_seg >= 1 && n_seg <= 3, "amv_bitnet_gemv_fused: n_seg %d (1..3)", n_seg);
    AMV_REQUIRE((((uintptr_t)a | (uintptr_t)b | (uintptr_t)norm_w) & 15) == 0,
                "amv_bitnet_gemv_fused: a, b and norm_w must be 16-byte aligned");
    BnSegs sg{};
    int64_t total = 0;
    for (int s = 0; s < 3; ++s) {
        if (s < n_seg) {
            AMV_REQUIRE(w[s] && dst[s] && rows[s] > 0, "amv_bitnet_gemv_fused: matrix %d: null pointer or no rows", s);
            AMV_REQUIRE(((uintptr_t)w[s] & 15) == 0, "amv_bitnet_gemv_fused: weights must be 16-byte aligned");
            total += rows[s];
            AMV_REQUIRE(total <= (1 << 24), "amv_bitnet_gemv_fused: too many rows");
            sg.w[s] = (const uint4*)w[s];
            sg.dst[s] = dst[s];
            sg.wscale[s] = wscale[s];
        }
        sg.end[s] = (int)total;
    }
    const bool rope = rope_cs != nullptr;
    if (rope) {
        AMV_REQUIRE(mode == 0 && n_seg == 3 && rows[0] % 128 == 0 && rows[1] % 128 == 0 && rows[2] == rows[1] &&
                        !accumulate && pos && n_ctx > 0,
                    "amv_bitnet_gemv_fused: RoPE needs Q | K | V (head_dim 128, K and V of equal rows, mode 0), the "
                    "position and the context length, and no accumulation");
    }
    // Launch shape (measured on MI355X, cold weights): 2 rows per wave, 4 from 8192 rows on (the per-wave fixed
    // work of the prologue then counts half as often: gate | up 13824 x 2560 8.3 -> 7.4 us, while 2560- and 3840-row
    // launches lose ~1 us with 4); 512 threads per workgroup (against 256 / 1024: 4.1 / 4.5-5.9 us for Q | K | V),
    // 1024 when k > 8192 so the input fits 4 float4 per thread.
    const int R = total >= 8192 ? 4 : 2;
    const int64_t waves = (total + R - 1) / R;
    hipStream_t st = amv_stream(stream);
    const float4 *a4 = (const float4*)a, *b4 = (const float4*)b, *w4 = (const float4*)norm_w;
#define BN_QG_LAUNCH(NT, V4, ROPE, MODE, RR, CS, POS, CTX)                                                       \
    hipLaunchKernelGGL((k_bitnet_qgemv<NT, V4, ROPE, MODE, RR>),                                                   \
                       dim3((unsigned)((waves + NT / 64 - 1) / (NT / 64))), dim3(NT), 0, st, a4, b4, w4, (int)k, eps,  \
                       do_norm, sg, n_seg, accumulate, CS, POS, CTX, BnFa{})
#define BN_QG_R(NT, V4, RR)                                                                                        \
    do {                                                                                                           \
        if (rope) BN_QG_LAUNCH(NT, V4, true, 0, RR, rope_cs, pos, (int)n_ctx);                                     \
        else if (mode == 1) BN_QG_LAUNCH(NT, V4, false, 1, RR, nullptr, nullptr, 0);                               \
        else if (mode == 2) BN_QG_LAUNCH(NT, V4, false, 2, RR, nullptr, nullptr, 0);                               \
        else BN_QG_LAUNCH(NT, V4, false, 0, RR, nullptr, nullptr, 0);                                              \
    } while (0)
#define BN_QG(NT, V4)                                                                                              \
    do {                                                                                                           \
        if (R == 4) BN_QG_R(NT, V4, 4);                                                                            \
        else BN_QG_R(NT, V4, 2);                                                                                   \
    } while (0)
    if (k > 8192) BN_QG(1024, 4);
    else if (k > 4096) BN_QG(512, 4);
    else if (k > 2048) BN_QG(512, 2);
    else BN_QG(512, 1);
#undef BN_QG
#undef BN_QG_R
#undef BN_QG_LAUNCH
    return amv_check_launch("amv_bitnet_gemv_fused");
}

extern "C" int amv_bitnet_gemv_fa_merge(const float* part, int n_split, int split_len, int64_t n_kv_max,
                                        const int32_t* n_kv_dev, const float* norm_w, int64_t k, float eps,
                                        int do_norm, const void* w, int64_t rows, float wscale, float* dst,
                                        int accumulate, void* stream) {
    AMV_REQUIRE(part && n_kv_dev && w && dst, "amv_bitnet_gemv_fa_merge: null pointer");
    AMV_REQUIRE(k > 0 && k % 128 == 0 && k <= 16384, "amv_bitnet_gemv_fa_merge: k %lld (heads of 128, <= 16384)",
                (long long)k);
    AMV_REQUIRE(n_split >= 1 && split_len >= 1 && n_kv_max >= 1 &&
                    (n_kv_max + split_len - 1) / split_len <= std::min(n_split, BN_FA_ZM),
                "amv_bitnet_gemv_fa_merge: %lld keys in splits of %d need more than min(%d, %d) splits",
                (long long)n_kv_max, split_len, n_split, BN_FA_ZM);
    AMV_REQUIRE(rows > 0 && rows <= (1 << 24), "amv_bitnet_gemv_fa_merge: rows %lld", (long long)rows);
    AMV_REQUIRE((((uintptr_t)part | (uintptr_t)norm_w | (uintptr_t)w) & 15) == 0,
                "amv_bitnet_gemv_fa_merge: part, norm_w and the weights must be 16-byte aligned");
    BnSegs sg{};
    sg.w[0] = (const uint4*)w;
    sg.dst[0] = dst;
    sg.wscale[0] = wscale;
    sg.end[0] = sg.end[1] = sg.end[2] = (int)rows;
    const BnFa fa{part, n_kv_dev, n_split, split_len, (int)n_kv_max};
    const int R = rows >= 8192 ? 4 : 2;  // the launch shape of amv_bitnet_gemv_fused
    const int64_t waves = (rows + R - 1) / R;
    hipStream_t st = amv_stream(stream);
    const float4 *a4 = (const float4*)part, *w4 = (const float4*)norm_w;
#define BN_FM_LAUNCH(NT, V4, RR)                                                                                  \
    hipLaunchKernelGGL((k_bitnet_qgemv<NT, V4, false, 3, RR>), dim3((unsigned)((waves + NT / 64 - 1) / (NT / 64))), \
                       dim3(NT), 0, st, a4, nullptr, w4, (int)k, eps, do_norm, sg, 1, accumulate, nullptr, nullptr,  \
                       0, fa)
#define BN_FM(NT, V4)                          \
    do {                                       \
        if (R == 4) BN_FM_LAUNCH(NT, V4, 4);   \
        else BN_FM_LAUNCH(NT, V4, 2);          \
    } while (0)
    if (k > 8192) BN_FM(1024, 4);
    else if (k > 4096) BN_FM(512, 4);
    else if (k > 2048) BN_FM(512, 2);
    else BN_FM(512, 1);
#undef BN_FM
#undef BN_FM_LAUNCH
    return amv_check_launch("amv_bitnet_gemv_fa_merge");
}
