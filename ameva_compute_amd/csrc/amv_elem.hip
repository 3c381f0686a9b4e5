// Glue ops of the decoder graph: ADD / MUL with row broadcast (residuals, norm weights), f32 -> f16 copies and
// SET_ROWS into an f16 KV cache, GET_ROWS (embedding lookup) from f32 / f16 / Q4_0 / Q8_0 / Q4_K / Q6_K rows.
// Roles of ameva_binary.comp, ameva_cpy.comp, ameva_set_rows.comp and ameva_get_rows(_q).comp of the reference.
#include "amv_common.h"

#include <algorithm>

// dst[r][i] = a[r][i] op b[r % b_rows][i]   (op 0 add, 1 mul); n = elements per row
__global__ __launch_bounds__(256) void k_binary(const float* __restrict__ a, const float* __restrict__ b,
                                               float* __restrict__ dst, int64_t n_rows, int64_t n, int64_t b_rows,
                                               int op) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_rows * n) return;
    const int64_t r = i / n, c = i - r * n;
    const float x = a[i], y = b[(r % b_rows) * n + c];
    dst[i] = op == 0 ? x + y : x * y;
}

extern "C" int amv_binary(int op, const float* a, const float* b, float* dst, int64_t n_rows, int64_t n, int64_t b_rows,
                          void* stream) {
    AMV_REQUIRE(a && b && dst, "amv_binary: null pointer");
    AMV_REQUIRE(op == 0 || op == 1, "amv_binary: op %d (0 add, 1 mul)", op);
    AMV_REQUIRE(n_rows > 0 && n > 0 && b_rows > 0 && b_rows <= n_rows, "amv_binary: bad shape");
    const int64_t total = n_rows * n;
    hipLaunchKernelGGL(k_binary, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream), a, b, dst,
                       n_rows, n, b_rows, op);
    return amv_check_launch("amv_binary");
}

// f32 rows -> f16 rows at dst row idx[r] (SET_ROWS) or row r (idx NULL, CPY); row strides in elements.
// An index outside [0, dst_rows) is not written and is counted in *bad (the reference's status buffer).
__global__ __launch_bounds__(256) void k_rows_f16(const float* __restrict__ src, int64_t src_stride,
                                                 uint16_t* __restrict__ dst, int64_t dst_stride, int64_t n_rows,
                                                 int64_t n, const int64_t* __restrict__ idx64,
                                                 const int32_t* __restrict__ idx32, int64_t dst_rows,
                                                 unsigned int* __restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_rows * n) return;
    const int64_t r = i / n, c = i - r * n;
    int64_t dr = r;
    if (idx64) dr = idx64[r];
    else if (idx32) dr = idx32[r];
    if (dr < 0 || dr >= dst_rows) {
        if (c == 0 && bad) atomicAdd(bad, 1u);
        return;
    }
    dst[dr * dst_stride + c] = amv_f2h(src[r * src_stride + c]);
}

extern "C" int amv_set_rows_f16(const float* src, int64_t src_stride, void* dst, int64_t dst_stride, int64_t n_rows,
                                int64_t n, const void* idx, int idx_bits, int64_t dst_rows, unsigned int* bad,
                                void* stream) {
    AMV_REQUIRE(src && dst, "amv_set_rows_f16: null pointer");
    AMV_REQUIRE(n_rows > 0 && n > 0 && src_stride >= n && dst_stride >= n, "amv_set_rows_f16: bad shape");
    AMV_REQUIRE(idx == nullptr || idx_bits == 32 || idx_bits == 64, "amv_set_rows_f16: index type must be i32 or i64");
    AMV_REQUIRE(idx != nullptr || dst_rows >= n_rows, "amv_set_rows_f16: dst too small");
    const int64_t total = n_rows * n;
    hipLaunchKernelGGL(k_rows_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream), src,
                       src_stride, (uint16_t*)dst, dst_stride, n_rows, n,
                       idx_bits == 64 ? (const int64_t*)idx : nullptr, idx_bits == 32 ? (const int32_t*)idx : nullptr,
                       dst_rows, bad);
    return amv_check_launch("amv_set_rows_f16");
}

// GET_ROWS: dst f32 [n_idx][n] = dequantized row idx[i] of src (type F32, F16, Q4_0, Q8_0, Q4_K, Q6_K: ggml blocks,
// row stride in bytes). Dequantization as ggml's dequantize_row_* (ameva_get_rows_q.comp), the same f32 expressions.
__global__ __launch_bounds__(256) void k_get_rows(const uint8_t* __restrict__ src, int64_t row_bytes, int type,
                                                 const int32_t* __restrict__ idx, int64_t n_idx, int64_t n,
                                                 int64_t src_rows, float* __restrict__ dst,
                                                 unsigned int* __restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_idx * n) return;
    const int64_t r = i / n, c = i - r * n;
    const int64_t sr = idx[r];
    if (sr < 0 || sr >= src_rows) {
        if (c == 0 && bad) atomicAdd(bad, 1u);
        dst[i] = 0.0f;
        return;
    }
    const uint8_t* row = src + sr * row_bytes;
    float v;
    if (type == AMV_T_F32) {
        v = reinterpret_cast<const float*>(row)[c];
    } else if (type == AMV_T_F16) {
        v = amv_h2f(reinterpret_cast<const uint16_t*>(row)[c]);
    } else if (type == AMV_T_Q4_0) {
        const uint8_t* blk = row + (c / 32) * 18;
        const int j = (int)(c % 32);
        const float d = amv_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const int nib = j < 16 ? (blk[2 + j] & 0xF) : (blk[2 + j - 16] >> 4);
        v = (float)(nib - 8) * d;
    } else if (type == AMV_T_Q8_0) {
        const uint8_t* blk = row + (c / 32) * 34;
        const float d = amv_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        v = (float)(int8_t)blk[2 + c % 32] * d;
    } else if (type == AMV_T_Q4_K) {
        // dequantize_row_q4_K: chunk of 64 = 32 low nibbles (sub-block 2 ch) then 32 high nibbles (2 ch + 1)
        const uint8_t* blk = row + (c / 256) * 144;
        const int e = (int)(c % 256), ch = e / 64, l = e % 64;
        const int sub = 2 * ch + (l >= 32);
        const uint8_t qb = blk[16 + 32 * ch + (l & 31)];
        const int q = l < 32 ? (qb & 0xF) : (qb >> 4);
        const uint8_t* sc = blk + 4;
        int scl, mn;
        if (sub < 4) {
            scl = sc[sub] & 63;
            mn = sc[sub + 4] & 63;
        } else {
            scl = (sc[sub + 4] & 0xF) | ((sc[sub - 4] >> 6) << 4);
            mn = (sc[sub + 4] >> 4) | ((sc[sub] >> 6) << 4);
        }
        const float d = amv_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const float dmin = amv_h2f((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
        v = (d * (float)scl) * (float)q - dmin * (float)mn;
    } else {  // Q6_K (dequantize_row_q6_K): halves of 128, quarters of 32 take ql low/high nibbles and 2 qh bits
        const uint8_t* blk = row + (c / 256) * 210;
        const int e = (int)(c % 256), h = e / 128, r = e % 128, qt = r / 32, l = r % 32;
        const uint8_t lb = blk[64 * h + l + 32 * (qt & 1)];
        const int lo = qt < 2 ? (lb & 0xF) : (lb >> 4);
        const int hi = (blk[128 + 32 * h + l] >> (2 * qt)) & 3;
        const int q = (lo | (hi << 4)) - 32;
        const float d = amv_h2f((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
        v = d * (float)(int8_t)blk[192 + 8 * h + l / 16 + 2 * qt] * (float)q;
    }
    dst[i] = v;
}

extern "C" int amv_get_rows(int type, const void* src, int64_t src_rows, int64_t n, const int32_t* idx, int64_t n_idx,
                            float* dst, unsigned int* bad, void* stream) {
    AMV_REQUIRE(src && idx && dst, "amv_get_rows: null pointer");
    AMV_REQUIRE(n_idx > 0 && n > 0 && src_rows > 0, "amv_get_rows: bad shape");
    int64_t rb;
    switch (type) {
    case AMV_T_F32: rb = n * 4; break;
    case AMV_T_F16: rb = n * 2; break;
    case AMV_T_Q4_0: AMV_REQUIRE(n % 32 == 0, "amv_get_rows: n %% 32"); rb = n / 32 * 18; break;
    case AMV_T_Q8_0: AMV_REQUIRE(n % 32 == 0, "amv_get_rows: n %% 32"); rb = n / 32 * 34; break;
    case AMV_T_Q4_K: AMV_REQUIRE(n % 256 == 0, "amv_get_rows: n %% 256"); rb = n / 256 * 144; break;
    case AMV_T_Q6_K: AMV_REQUIRE(n % 256 == 0, "amv_get_rows: n %% 256"); rb = n / 256 * 210; break;
    default: amv_set_error("amv_get_rows: type %d not supported", type); return AMV_ERR_UNSUPPORTED;
    }
    const int64_t total = n_idx * n;
    hipLaunchKernelGGL(k_get_rows, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream),
                       (const uint8_t*)src, rb, type, idx, n_idx, n, src_rows, dst, bad);
    return amv_check_launch("amv_get_rows");
}

// ---------------------------------------------------------------------------------------------------------------
// Greedy sampling: the index of the largest of x[0 .. n) (the first on ties; NaN never wins), written to token[0];
// with history, also to history[step[0]] (when below history_len) and step[0] incremented, so a decode loop replayed
// as a HIP graph keeps its token and its output on the device. One workgroup of 1024: float4 loads, then wave and
// workgroup reductions with the same (value, index) order.
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ void argmax_take(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int n, int32_t* __restrict__ token,
                                                int32_t* __restrict__ history, int32_t* __restrict__ step,
                                                int history_len) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    const int n4 = n / 4;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    // eight float4 loads of a thread in flight per round (a 128256-entry row: 4 rounds instead of 32 dependent
    // ones); the selection is order-free (larger value, then smaller index), so the rounds may take any order
    for (int i0 = tid; i0 < n4; i0 += 8 * 1024) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = x4[min(i0 + 1024 * u, n4 - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + 1024 * u;
            if (i < n4) {
                argmax_take(bv, bi, v[u].x, 4 * i);
                argmax_take(bv, bi, v[u].y, 4 * i + 1);
                argmax_take(bv, bi, v[u].z, 4 * i + 2);
                argmax_take(bv, bi, v[u].w, 4 * i + 3);
            }
        }
    }
    for (int i = 4 * n4 + tid; i < n; i += 1024) argmax_take(bv, bi, x[i], i);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_take(bv, bi, __shfl_xor(bv, o, AMV_WAVE), __shfl_xor(bi, o, AMV_WAVE));
    if (lane == 0) {
        sv[wv] = bv;
        si[wv] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w) argmax_take(bv, bi, sv[w], si[w]);
        const int t = bi == 0x7FFFFFFF ? 0 : bi;  // all NaN: token 0
        token[0] = t;
        if (history) {
            const int s = step[0];
            if (s >= 0 && s < history_len) history[s] = t;
            step[0] = s + 1;
        }
    }
}

// The argmax spread over the GPU: workgroup b of 256 threads takes float4 chunks [2048 b, 2048 b + 2048) of x (eight
// loads per thread in flight, one round), reduces them with argmax_take's order, and offers its best as one 64-bit
// key to an atomic maximum: the high word is the value mapped to an unsigned order (x >= 0: bits | 2^31, x < 0: ~bits;
// -0 as +0, so equal values meet on equal keys), the low word 2^32 - 1 - index (the smaller index wins a tie); a
// workgroup with no candidate (NaN only) offers 0. Each workgroup then arrives on a counter (atomicInc wrapping at
// the grid size, after its maximum has completed); the last to arrive takes the key with an exchange that leaves 0,
// so ws holds zeros again for the next call, and writes the token (0 when no value was a candidate), the history
// and, when given, the decode position advanced by one (pos, kv_idx and n_kv each + 1).
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
    if (i == 0x7FFFFFFF) return 0ull;
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
}
__global__ __launch_bounds__(256) void k_argmax_mw(const float* __restrict__ x, int n, int32_t* __restrict__ token,
                                                  int32_t* __restrict__ history, int32_t* __restrict__ step,
                                                  int history_len, int32_t* pos, int64_t* kv_idx, int32_t* n_kv,
                                                  unsigned long long* ws) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n4 = n / 4, c0 = blockIdx.x * 2048;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = x4[min(c0 + 256 * u + tid, n4 - 1)];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int i = c0 + 256 * u + tid;
        if (i < n4) {
            argmax_take(bv, bi, v[u].x, 4 * i);
            argmax_take(bv, bi, v[u].y, 4 * i + 1);
            argmax_take(bv, bi, v[u].z, 4 * i + 2);
            argmax_take(bv, bi, v[u].w, 4 * i + 3);
        }
    }
    if (blockIdx.x == gridDim.x - 1)
        for (int i = 4 * n4 + tid; i < n; i += 256) argmax_take(bv, bi, x[i], i);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_take(bv, bi, __shfl_xor(bv, o, AMV_WAVE), __shfl_xor(bi, o, AMV_WAVE));
    if (lane == 0) {
        sv[wv] = bv;
        si[wv] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w) argmax_take(bv, bi, sv[w], si[w]);
        atomicMax(ws, argmax_key(bv, bi));
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned int* cnt = reinterpret_cast<unsigned int*>(ws + 1);
        if (atomicInc(cnt, gridDim.x - 1u) == gridDim.x - 1u) {
            const unsigned long long k = atomicExch(ws, 0ull);
            const int t = k == 0ull ? 0 : (int)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
            token[0] = t;
            if (history) {
                const int s = step[0];
                if (s >= 0 && s < history_len) history[s] = t;
                step[0] = s + 1;
            }
            if (pos) pos[0] += 1;
            if (kv_idx) kv_idx[0] += 1;
            if (n_kv) n_kv[0] += 1;
        }
    }
}

extern "C" int amv_argmax_ex(const float* x, int64_t n, int32_t* token, int32_t* history, int32_t* step,
                             int64_t history_len, int32_t* pos, int64_t* kv_idx, int32_t* n_kv, void* ws,
                             void* stream) {
    AMV_REQUIRE(x && token && ws, "amv_argmax_ex: null pointer");
    AMV_REQUIRE(n > 0 && n <= INT32_MAX - 8192, "amv_argmax_ex: bad length %lld", (long long)n);
    AMV_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)ws & 15) == 0, "amv_argmax_ex: x and ws must be 16-byte aligned");
    AMV_REQUIRE(!history || (step && history_len > 0 && history_len <= INT32_MAX),
                "amv_argmax_ex: history needs step and history_len");
    const int64_t blocks = std::max<int64_t>(1, (n / 4 + 2047) / 2048);
    hipLaunchKernelGGL(k_argmax_mw, dim3((unsigned)blocks), dim3(256), 0, amv_stream(stream), x, (int)n, token, history,
                       step, (int)history_len, pos, kv_idx, n_kv, reinterpret_cast<unsigned long long*>(ws));
    return amv_check_launch("amv_argmax_ex");
}

extern "C" int amv_argmax(const float* x, int64_t n, int32_t* token, int32_t* history, int32_t* step,
                          int64_t history_len, void* stream) {
    AMV_REQUIRE(x && token, "amv_argmax: null pointer");
    AMV_REQUIRE(n > 0 && n <= INT32_MAX, "amv_argmax: bad length %lld", (long long)n);
    AMV_REQUIRE(((uintptr_t)x & 15) == 0, "amv_argmax: x must be 16-byte aligned");
    AMV_REQUIRE(!history || (step && history_len > 0 && history_len <= INT32_MAX),
                "amv_argmax: history needs step and history_len");
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, amv_stream(stream), x, (int)n, token, history, step,
                       (int)history_len);
    return amv_check_launch("amv_argmax");
}
