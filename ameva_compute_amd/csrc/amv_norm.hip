// RMS_NORM (with the fused MUL by the norm weight and the fused Q8_0 quantization of the next GEMV's input), ROPE
// and SWIGLU for the decode/prefill path.
//
// RMS_NORM follows ggml_compute_forward_rms_norm_f32 (reference ameva_rms_norm.comp:3-7): squares as f32 products
// summed in double, mean = (float)(sum / n), scale = 1 / sqrtf(mean + eps), y = x * scale, o = y * w. Division and
// sqrt are correctly rounded (build flags), so y and o match the CPU bit for bit whenever the two double sums round
// to the same f32 mean. ROPE follows ggml's rope f32 (ggml-ameva.cpp:3982-3984, ameva_rope.comp:64-92): the angle of
// pair j is freq_scale * (p * theta_scale^j) built by the same repeated f32 multiplication as the CPU.
#include "amv_common.h"

#include <algorithm>

// One workgroup of 1024 per row (amv_rms_row with one virtual lane per thread).
#define RMS_THREADS 1024
__global__ __launch_bounds__(RMS_THREADS) void k_rms_norm(const float* __restrict__ x, int n, float eps,
                                                         const float* __restrict__ w, float* __restrict__ y,
                                                         float* __restrict__ o, const AmvActOut act) {
    __shared__ double sred[AMV_RMS_VLANES / 64];
    const size_t row = blockIdx.x;
    amv_rms_row<RMS_THREADS>(reinterpret_cast<const float4*>(x + row * n), n / 4, eps, w, y ? y + row * n : nullptr,
                             o ? o + row * n : nullptr, amv_act_row(act, row, n), sred);
}

extern "C" int amv_rms_norm_act(const float* x, int64_t n_rows, int64_t n, float eps, const float* w, float* y,
                                float* o, void* act, int act_type, int rule, void* stream) {
    AMV_REQUIRE(x, "amv_rms_norm: null input");
    AMV_REQUIRE(n_rows > 0 && n > 0 && n_rows <= INT32_MAX && n <= INT32_MAX, "amv_rms_norm: bad shape");
    AMV_REQUIRE(n % 4 == 0, "amv_rms_norm: n %% 4 != 0");
    AMV_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)o & 15) == 0 &&
                    ((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0,
                "amv_rms_norm: buffers must be 16-byte aligned");
    AMV_REQUIRE(!o || w, "amv_rms_norm: o needs the weight w");
    AMV_REQUIRE(y || o || act, "amv_rms_norm: no output requested");
    AMV_REQUIRE(!act || act_type == AMV_T_Q8_0 || act_type == AMV_T_Q8_K, "amv_rms_norm: act_type %d (Q8_0 or Q8_K)",
                act_type);
    AMV_REQUIRE(!act || n % (act_type == AMV_T_Q8_K ? 256 : 32) == 0,
                "amv_rms_norm: the fused quantization needs n %% block size == 0");
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_rms_norm: bad rule");
    // the quantized output is of y * w when the weight is given (o may then be NULL), of y otherwise
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)n_rows), dim3(RMS_THREADS), 0, amv_stream(stream), x, (int)n, eps, w,
                       y, o, amv_act_out(act, n, act ? act_type : 0, rule, n_rows));
    return amv_check_launch("amv_rms_norm");
}

extern "C" int amv_rms_norm(const float* x, int64_t n_rows, int64_t n, float eps, const float* w, float* y, float* o,
                            void* act, int rule, void* stream) {
    return amv_rms_norm_act(x, n_rows, n, eps, w, y, o, act, AMV_T_Q8_0, rule, stream);
}

// ---------------------------------------------------------------------------------------------------------------
// ROPE: x, y [n_tok][n_head][ne0] contiguous f32 (in place allowed), pos int32 [n_tok]; mode 0 NORMAL (pairs 2j, 2j+1)
// or 2 NEOX (pairs j, j + n_dims/2); elements past n_dims copied. One lane per pair.
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rope(const float* x, float* y,  // may alias (in place)
                                             const int32_t* __restrict__ pos, int64_t n_pairs, int n_head, int ne0,
                                             int n_dims, int neox, float theta_scale, float freq_scale,
                                             float attn_factor) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_pairs) return;
    const int half = ne0 / 2;
    const int j = (int)(i % half);
    const int64_t th = i / half;  // token * n_head + head
    const int t = (int)(th / n_head);
    const float* xr = x + th * ne0;
    float* yr = y + th * ne0;
    if (2 * j >= n_dims) {
        const float a = xr[2 * j], b = xr[2 * j + 1];
        yr[2 * j] = a;
        yr[2 * j + 1] = b;
        return;
    }
    const int e0 = neox ? j : 2 * j;
    const int e1 = neox ? j + n_dims / 2 : 2 * j + 1;
    float y0, y1;
    amv_rope_pair((float)pos[t], j, theta_scale, freq_scale, attn_factor, xr[e0], xr[e1], y0, y1);
    yr[e0] = y0;
    yr[e1] = y1;
}

extern "C" int amv_rope(const float* x, float* y, const int32_t* pos, int64_t n_tok, int64_t n_head, int64_t ne0,
                        int n_dims, int mode, float freq_base, float freq_scale, float attn_factor, void* stream) {
    AMV_REQUIRE(x && y && pos, "amv_rope: null pointer");
    AMV_REQUIRE(n_tok > 0 && n_head > 0 && ne0 > 0 && ne0 % 2 == 0, "amv_rope: bad shape");
    AMV_REQUIRE(n_dims > 0 && n_dims <= ne0 && n_dims % 2 == 0, "amv_rope: bad n_dims %d", n_dims);
    AMV_REQUIRE(mode == 0 || mode == 2, "amv_rope: mode %d not supported (NORMAL 0 and NEOX 2 are)", mode);
    // the same expression as the CPU (ggml-ameva.cpp:3984)
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    const int64_t n_pairs = n_tok * n_head * (ne0 / 2);
    hipLaunchKernelGGL(k_rope, dim3((unsigned)((n_pairs + 255) / 256)), dim3(256), 0, amv_stream(stream), x, y, pos,
                       n_pairs, (int)n_head, (int)ne0, n_dims, mode == 2 ? 1 : 0, theta_scale, freq_scale, attn_factor);
    return amv_check_launch("amv_rope");
}

// ---------------------------------------------------------------------------------------------------------------
// ROPE of q and k + SET_ROWS of k and v into the f16 cache. Token t's row of qkv holds n_head q heads, n_head_kv k
// heads and n_head_kv v heads of D floats. q and k heads are rotated in place (k_rope's arithmetic, so the values equal
// ROPE's), k and v heads are also stored as f16 (amv_f2h, round to nearest even as the CPU's fp32 -> fp16) at row
// kv_idx[t] of the caches; rows outside [0, cache_rows) are skipped and counted in *bad (once per k / v head).
// Workgroup (token t, group of HPW heads): the cos / sin of the token's pairs are computed once into LDS (the angle
// loop and sincos are the costly part of a pair), then thread i handles pair i % (D / 2) of head i / (D / 2), so a
// wave's loads and stores cover consecutive pairs (NORMAL: one 8-byte load, one 8-byte store and one 4-byte f16 pair
// store per pair).
// ---------------------------------------------------------------------------------------------------------------
#define ROPE_MAX_PAIRS 256  // D <= 512
#define ROPE_RB 12          // pairs per thread and round (a 48-head token of D = 128: one round)
template <bool NEOX, int HALF>  // HALF: D / 2 known at compile time (0: read from D)
__global__ __launch_bounds__(256) void k_rope_kv(float* __restrict__ qkv, const int32_t* __restrict__ pos, int n_head,
                                                int n_head_kv, int D, int n_dims, int hpw, float theta_scale,
                                                float freq_scale, float attn_factor, uint16_t* __restrict__ kc,
                                                uint16_t* __restrict__ vc, int64_t cache_row,
                                                const int64_t* __restrict__ kv_idx, int64_t cache_rows,
                                                unsigned int* __restrict__ bad, bool pair_stores) {
    __shared__ float s_c[ROPE_MAX_PAIRS], s_s[ROPE_MAX_PAIRS];
    const int t = blockIdx.x, tid = threadIdx.x;
    const int half = HALF ? HALF : D / 2, n_all = n_head + 2 * n_head_kv;
    const int h0 = blockIdx.y * hpw, h1 = min(n_all, h0 + hpw);
    float* xt = qkv + (int64_t)t * n_all * D;
    // rounds of ROPE_RB pairs per thread: every load of a round is issued before its stores (the stores go to the
    // same rows, so the compiler would otherwise keep each pair's load behind the previous pair's store); the first
    // round's loads are in flight while the cos / sin are computed
    float2 x[ROPE_RB];
    const auto load_round = [&](int i0) {
#pragma unroll
        for (int u = 0; u < ROPE_RB; ++u) {
            const int i = min(i0 + 256 * u, h1 * half - 1);  // past the end: re-read the last pair, not stored
            const int h = i / half, j = i - h * half;
            const float* xr = xt + (int64_t)h * D;
            if (NEOX && h < n_head + n_head_kv && 2 * j < n_dims) x[u] = make_float2(xr[j], xr[j + n_dims / 2]);
            else x[u] = *reinterpret_cast<const float2*>(xr + 2 * j);
        }
    };
    const int first = h0 * half + tid;
    load_round(first);
    const float p = (float)pos[t];
    for (int j = tid; 2 * j < n_dims; j += 256) {
        float c, sn;
        amv_rope_cs(p, j, theta_scale, freq_scale, attn_factor, c, sn);
        s_c[j] = c;
        s_s[j] = sn;
    }
    const int64_t dr = kv_idx[t];
    const bool store = dr >= 0 && dr < cache_rows;
    if (!store && bad) {  // one count per k / v head of this group
        const int nkv = max(0, h1 - max(h0, n_head));
        if (tid == 0 && nkv > 0) atomicAdd(bad, (unsigned)nkv);
    }
    __syncthreads();
    for (int i0 = first; i0 < h1 * half; i0 += 256 * ROPE_RB) {
        if (i0 != first) load_round(i0);
#pragma unroll
        for (int u = 0; u < ROPE_RB; ++u) {
            const int i = i0 + 256 * u;
            if (i >= h1 * half) break;
            const int h = i / half, j = i - h * half;
            float* xr = xt + (int64_t)h * D;
            const bool is_q = h < n_head, is_v = h >= n_head + n_head_kv;
            const bool rot = !is_v && 2 * j < n_dims;
            uint16_t* cr = nullptr;
            if (!is_q && store)
                cr = (is_v ? vc + (int64_t)(h - n_head - n_head_kv) * D : kc + (int64_t)(h - n_head) * D) +
                     dr * cache_row;
            float2 y = x[u];
            if (rot) amv_rope_apply(s_c[j], s_s[j], x[u].x, x[u].y, y.x, y.y);
            // element indices of the pair: NEOX rotates j with j + n_dims / 2, else 2 j with 2 j + 1
            const int e0 = NEOX && rot ? j : 2 * j, e1 = NEOX && rot ? j + n_dims / 2 : 2 * j + 1;
            if (!is_v) {
                if (NEOX && rot) {
                    xr[e0] = y.x;
                    xr[e1] = y.y;
                } else {
                    *reinterpret_cast<float2*>(xr + 2 * j) = y;
                }
            }
            if (cr) {
                if (!(NEOX && rot) && pair_stores) {
                    *reinterpret_cast<uint32_t*>(cr + 2 * j) = (uint32_t)amv_f2h(y.x) | ((uint32_t)amv_f2h(y.y) << 16);
                } else {
                    cr[e0] = amv_f2h(y.x);
                    cr[e1] = amv_f2h(y.y);
                }
            }
        }
    }
}

extern "C" int amv_rope_kv_store(float* qkv, const int32_t* pos, int64_t n_tok, int64_t n_head, int64_t n_head_kv,
                                 int64_t D, int n_dims, int mode, float freq_base, float freq_scale, float attn_factor,
                                 void* k_cache, void* v_cache, int64_t cache_row, const int64_t* kv_idx,
                                 int64_t cache_rows, unsigned int* bad, void* stream) {
    AMV_REQUIRE(qkv && pos && k_cache && v_cache && kv_idx, "amv_rope_kv_store: null pointer");
    AMV_REQUIRE(n_tok > 0 && n_tok <= INT32_MAX && n_head > 0 && n_head_kv > 0 && D > 0 && D % 2 == 0 &&
                    D <= 2 * ROPE_MAX_PAIRS && n_head + 2 * n_head_kv <= 65535,
                "amv_rope_kv_store: bad shape");
    AMV_REQUIRE(((uintptr_t)qkv & 7) == 0, "amv_rope_kv_store: qkv must be 8-byte aligned");
    AMV_REQUIRE(n_dims > 0 && n_dims <= D && n_dims % 2 == 0, "amv_rope_kv_store: bad n_dims %d", n_dims);
    AMV_REQUIRE(mode == 0 || mode == 2, "amv_rope_kv_store: mode %d not supported (NORMAL 0 and NEOX 2 are)", mode);
    AMV_REQUIRE(cache_row >= n_head_kv * D && cache_rows > 0, "amv_rope_kv_store: cache row %lld < %lld",
                (long long)cache_row, (long long)(n_head_kv * D));
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    // heads per workgroup: all of a token's heads when there are enough tokens to fill the GPU, else fewer
    const int n_all = (int)(n_head + 2 * n_head_kv);
    const int hpw = (int)std::max<int64_t>(1, std::min<int64_t>(n_all, (int64_t)n_all * n_tok / 512));
    const dim3 grid((unsigned)n_tok, (unsigned)((n_all + hpw - 1) / hpw));
    // f16 pairs as one 4-byte store when every pair starts 4-byte aligned
    const bool pairs = cache_row % 2 == 0 && ((uintptr_t)k_cache & 3) == 0 && ((uintptr_t)v_cache & 3) == 0;
    // D = 128 (every Llama head): the (head, pair) of an item by shifts instead of a division by a run-time D / 2
#define ROPE_LAUNCH(NX, HF)                                                                                         \
    hipLaunchKernelGGL((k_rope_kv<NX, HF>), grid, dim3(256), 0, amv_stream(stream), qkv, pos, (int)n_head,          \
                       (int)n_head_kv, (int)D, n_dims, hpw, theta_scale, freq_scale, attn_factor, (uint16_t*)k_cache, \
                       (uint16_t*)v_cache, cache_row, kv_idx, cache_rows, bad, pairs)
    if (mode == 2) {
        if (D == 128) ROPE_LAUNCH(true, 64);
        else ROPE_LAUNCH(true, 0);
    } else {
        if (D == 128) ROPE_LAUNCH(false, 64);
        else ROPE_LAUNCH(false, 0);
    }
#undef ROPE_LAUNCH
    return amv_check_launch("amv_rope_kv_store");
}

// ---------------------------------------------------------------------------------------------------------------
// SWIGLU (ggml_vec_swiglu_f32; ameva_glu.comp:45-46): y = g / (1 + expf(-g)) * u
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ g, const float* __restrict__ u,
                                               float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float a = g[i];
    y[i] = (a / (1.0f + expf(-a))) * u[i];
}

extern "C" int amv_swiglu(const float* g, const float* u, float* y, int64_t n, void* stream) {
    AMV_REQUIRE(g && u && y && n > 0, "amv_swiglu: bad arguments");
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, amv_stream(stream), g, u, y, n);
    return amv_check_launch("amv_swiglu");
}

// SWIGLU of n_rows rows (row strides in floats) with the Q8_0 quantization of each output row fused: thread i is
// element i % n of row i / n, a 32-lane half-wave one Q8_0 block (n % 32 == 0).
__global__ __launch_bounds__(256) void k_swiglu_q8(const float* __restrict__ g, int64_t gs, const float* __restrict__ u,
                                                  int64_t us, float* __restrict__ y, int64_t ys, int64_t n_rows,
                                                  int64_t n, int rule, int8_t* __restrict__ aq, int2* __restrict__ am) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // n_rows * n is a multiple of 32
    if (i >= n_rows * n) return;                                       // whole 32-lane blocks leave together
    const int64_t r = i / n, c = i - r * n;
    const float a = g[r * gs + c];
    const float h = (a / (1.0f + expf(-a))) * u[r * us + c];
    if (y) y[r * ys + c] = h;
    if (aq) amv_q8_0_lanes32(h, rule, (int)(c & 31), aq + r * n + (c & ~(int64_t)31), am + r * (n / 32) + c / 32);
}

// The same SWIGLU four elements per thread (float4 chunk i of the concatenated rows), with the quantization of each
// output row to Q8_0 or Q8_K fused (amv_act_store4: a Q8_0 block is 8 consecutive lanes, a Q8_K block one wave); the
// values and bytes equal k_swiglu_q8's and amv_quantize_act's.
__device__ __forceinline__ float amv_swiglu1(float a, float b) { return (a / (1.0f + expf(-a))) * b; }
__global__ __launch_bounds__(256) void k_swiglu_act(const float* __restrict__ g, int64_t gs,
                                                   const float* __restrict__ u, int64_t us, float* __restrict__ y,
                                                   int64_t ys, int total4, int n4, const AmvActOut act) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total4) return;  // rows hold whole quantization blocks, so blocks leave together
    const int r = i / n4, c = i - r * n4;
    const float4 a = *reinterpret_cast<const float4*>(g + r * gs + 4 * c);
    const float4 b = *reinterpret_cast<const float4*>(u + r * us + 4 * c);
    const float h[4] = {amv_swiglu1(a.x, b.x), amv_swiglu1(a.y, b.y), amv_swiglu1(a.z, b.z), amv_swiglu1(a.w, b.w)};
    if (y) *reinterpret_cast<float4*>(y + r * ys + 4 * c) = make_float4(h[0], h[1], h[2], h[3]);
    if (act.type) amv_act_store4(amv_act_row(act, r, 4 * (int64_t)n4), c, h);
}

extern "C" int amv_swiglu_rows_act(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* y,
                                   int64_t y_stride, int64_t n_rows, int64_t n, void* act, int act_type, int rule,
                                   void* stream) {
    AMV_REQUIRE(g && u && (y || act) && n_rows > 0 && n > 0, "amv_swiglu_rows: bad arguments");
    AMV_REQUIRE(g_stride >= n && u_stride >= n && (!y || y_stride >= n), "amv_swiglu_rows: row stride < n");
    AMV_REQUIRE(!act || act_type == AMV_T_Q8_0 || act_type == AMV_T_Q8_K,
                "amv_swiglu_rows: act_type %d (Q8_0 or Q8_K)", act_type);
    const int bs = act_type == AMV_T_Q8_K ? 256 : 32;
    AMV_REQUIRE(!act || n % bs == 0, "amv_swiglu_rows: the quantized output needs n %% %d == 0", bs);
    AMV_REQUIRE(!act || ((uintptr_t)act & 7) == 0, "amv_swiglu_rows: act must be 8-byte aligned");
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_swiglu_rows: unknown rule %d", rule);
    const bool vec = n % 4 == 0 && g_stride % 4 == 0 && u_stride % 4 == 0 && (!y || y_stride % 4 == 0) &&
                     ((uintptr_t)g & 15) == 0 && ((uintptr_t)u & 15) == 0 && ((uintptr_t)y & 15) == 0 &&
                     n_rows * std::max(std::max(g_stride, u_stride), y ? y_stride : 0) <= INT32_MAX;
    hipStream_t st = amv_stream(stream);
    if (vec) {
        const int64_t total4 = n_rows * (n / 4);
        hipLaunchKernelGGL(k_swiglu_act, dim3((unsigned)((total4 + 255) / 256)), dim3(256), 0, st, g, g_stride, u,
                           u_stride, y, y_stride, (int)total4, (int)(n / 4),
                           amv_act_out(act, n, act ? act_type : 0, rule, n_rows));
    } else {
        AMV_REQUIRE(!act || act_type == AMV_T_Q8_0,
                    "amv_swiglu_rows: the Q8_K output needs 16-byte aligned rows of whole float4s");
        int8_t* aq = (int8_t*)act;
        int2* am = act ? reinterpret_cast<int2*>(aq + n_rows * n) : nullptr;
        const int64_t total = n_rows * n;
        hipLaunchKernelGGL(k_swiglu_q8, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, g, g_stride, u,
                           u_stride, y, y_stride, n_rows, n, rule, aq, am);
    }
    return amv_check_launch("amv_swiglu_rows");
}

extern "C" int amv_swiglu_rows(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* y,
                               int64_t y_stride, int64_t n_rows, int64_t n, void* act, int rule, void* stream) {
    return amv_swiglu_rows_act(g, g_stride, u, u_stride, y, y_stride, n_rows, n, act, AMV_T_Q8_0, rule, stream);
}
