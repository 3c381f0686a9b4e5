// Decode GEMV (MUL_MAT with few activation columns) on quantized weights, MI355X wave64.
//
// Role of ameva_mmvq.comp / ameva_qmv.comp (reference, bs1 decode). The design is the MI355X one:
//  * weights in the structure-of-arrays layout of amv_repack, so a wave's weight load is one contiguous 1 KiB
//    (64 lanes x 16 B, global_load_dwordx4) per row and unit;
//  * a wave owns R weight rows; lane l takes the 32-weight blocks l, l + 64, ... of each row, and all R x U loads of
//    one step are issued before any is consumed (R x U x 16 B in flight per lane);
//  * the dequantization stays in integers: 4-bit / 8-bit weights against int8 activations with v_dot4_i32_i8, giving
//    per block exactly ggml's int32 sum (the Q4_0 offset -8 enters as -8 * sum(q_a), from the quantizer's block sums);
//  * f32 per block: acc += sumi * (d_w * d_a), then one butterfly reduction per row at the end.
// The BLOCK_SUMS instantiation stores the int32 block sums instead (parity instrumentation of the same code).
#include "amv_common.h"

#define M4 0x0F0F0F0Fu

// ------------------------------------------------------------------------------------------------ Q4_0 x Q8_0
template <int R, int U, bool BLOCK_SUMS>
__global__ __launch_bounds__(256) void k_mmv_q4_0(const uint4* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                 int n_rows, int nb, const int8_t* __restrict__ aq,
                                                 const int2* __restrict__ ads, float* __restrict__ dst,
                                                 int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (row0 >= n_rows) return;  // uniform per wave
    const int4* a4 = reinterpret_cast<const int4*>(aq);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int j0 = 0; j0 < nb; j0 += 64 * U) {
        uint4 w[U][R];
        uint16_t dw[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(j0 + 64 * u + lane, nb - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const size_t bi = (size_t)min(row0 + r, n_rows - 1) * nb + j;
                w[u][r] = wq[bi];
                dw[u][r] = wd[bi];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + 64 * u + lane;
            if (j < nb) {
                const int4 a0 = a4[2 * j], a1 = a4[2 * j + 1];
                const int2 ds = ads[j];
                const float da = __int_as_float(ds.x);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint4 q = w[u][r];
                    int s = amv_dot4((int)(q.x & M4), a0.x, 0);
                    s = amv_dot4((int)(q.y & M4), a0.y, s);
                    s = amv_dot4((int)(q.z & M4), a0.z, s);
                    s = amv_dot4((int)(q.w & M4), a0.w, s);
                    s = amv_dot4((int)((q.x >> 4) & M4), a1.x, s);
                    s = amv_dot4((int)((q.y >> 4) & M4), a1.y, s);
                    s = amv_dot4((int)((q.z >> 4) & M4), a1.z, s);
                    s = amv_dot4((int)((q.w >> 4) & M4), a1.w, s);
                    s -= 8 * ds.y;
                    if (BLOCK_SUMS) {
                        if (row0 + r < n_rows) sums[(size_t)(row0 + r) * nb + j] = s;
                    } else {
                        acc[r] = fmaf((float)s, amv_h2f(dw[u][r]) * da, acc[r]);
                    }
                }
            }
        }
    }
    if (!BLOCK_SUMS) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float t = amv_wave_sum(acc[r]);
            if (lane == 0 && row0 + r < n_rows) dst[row0 + r] = t;
        }
    }
}

// ------------------------------------------------------------------------------------------------ Q8_0 x Q8_0
template <int R, int U, bool BLOCK_SUMS>
__global__ __launch_bounds__(256) void k_mmv_q8_0(const uint4* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                 int n_rows, int nb, const int8_t* __restrict__ aq,
                                                 const int2* __restrict__ ads, float* __restrict__ dst,
                                                 int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (row0 >= n_rows) return;
    const int4* a4 = reinterpret_cast<const int4*>(aq);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int j0 = 0; j0 < nb; j0 += 64 * U) {
        uint4 w0[U][R], w1[U][R];
        uint16_t dw[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(j0 + 64 * u + lane, nb - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const size_t bi = (size_t)min(row0 + r, n_rows - 1) * nb + j;
                w0[u][r] = wq[2 * bi];
                w1[u][r] = wq[2 * bi + 1];
                dw[u][r] = wd[bi];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + 64 * u + lane;
            if (j < nb) {
                const int4 a0 = a4[2 * j], a1 = a4[2 * j + 1];
                const float da = __int_as_float(ads[j].x);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint4 p = w0[u][r], q = w1[u][r];
                    int s = amv_dot4((int)p.x, a0.x, 0);
                    s = amv_dot4((int)p.y, a0.y, s);
                    s = amv_dot4((int)p.z, a0.z, s);
                    s = amv_dot4((int)p.w, a0.w, s);
                    s = amv_dot4((int)q.x, a1.x, s);
                    s = amv_dot4((int)q.y, a1.y, s);
                    s = amv_dot4((int)q.z, a1.z, s);
                    s = amv_dot4((int)q.w, a1.w, s);
                    if (BLOCK_SUMS) {
                        if (row0 + r < n_rows) sums[(size_t)(row0 + r) * nb + j] = s;
                    } else {
                        acc[r] = fmaf((float)s, amv_h2f(dw[u][r]) * da, acc[r]);
                    }
                }
            }
        }
    }
    if (!BLOCK_SUMS) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float t = amv_wave_sum(acc[r]);
            if (lane == 0 && row0 + r < n_rows) dst[row0 + r] = t;
        }
    }
}

// ------------------------------------------------------------------------------------------------ dispatch
struct MmvArgs {
    int wtype;
    const uint8_t* w;
    int n_rows, k;
    const int8_t* aq;      // this column's int8 activations
    const void* ameta0;    // Q8_0: {d, sum} per block; Q8_K: d per block
    const void* ameta1;    // Q8_K: sums per 16
    float* dst;
    int32_t* sums;
};

template <int R, int U, bool S>
static void launch_q4_0(const MmvArgs& a, hipStream_t st) {
    const int nb = a.k / 32;
    const int64_t nblk = (int64_t)a.n_rows * nb;
    const uint4* wq = reinterpret_cast<const uint4*>(a.w);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(a.w + nblk * 16);
    const int2* ads = reinterpret_cast<const int2*>(a.ameta0);
    const int8_t* aq = a.aq;
    const int waves = (a.n_rows + R - 1) / R;
    hipLaunchKernelGGL((k_mmv_q4_0<R, U, S>), dim3((waves + 3) / 4), dim3(256), 0, st, wq, wd, a.n_rows, nb, aq, ads,
                       a.dst, a.sums);
}

template <int R, int U, bool S>
static void launch_q8_0(const MmvArgs& a, hipStream_t st) {
    const int nb = a.k / 32;
    const int64_t nblk = (int64_t)a.n_rows * nb;
    const uint4* wq = reinterpret_cast<const uint4*>(a.w);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(a.w + nblk * 32);
    const int2* ads = reinterpret_cast<const int2*>(a.ameta0);
    const int8_t* aq = a.aq;
    const int waves = (a.n_rows + R - 1) / R;
    hipLaunchKernelGGL((k_mmv_q8_0<R, U, S>), dim3((waves + 3) / 4), dim3(256), 0, st, wq, wd, a.n_rows, nb, aq, ads,
                       a.dst, a.sums);
}

// Kernel variant (rows per wave R, blocks-per-lane unroll U) chosen from the block count of a row; the table is the
// result of the launch-shape sweep on MI355X (see the bench and profiles of this repository).
template <bool S>
static int mmv_one_column(const MmvArgs& a, hipStream_t st) {
    const int nb = a.k / 32;
    switch (a.wtype) {
    case AMV_T_Q4_0:
        if (nb <= 64) launch_q4_0<4, 1, S>(a, st);
        else if (nb <= 128) launch_q4_0<4, 2, S>(a, st);
        else launch_q4_0<2, 4, S>(a, st);
        return AMV_OK;
    case AMV_T_Q8_0:
        if (nb <= 64) launch_q8_0<4, 1, S>(a, st);
        else if (nb <= 128) launch_q8_0<2, 2, S>(a, st);
        else launch_q8_0<2, 2, S>(a, st);
        return AMV_OK;
    default: amv_set_error("amv_mul_mat_vec: weight type %d not supported", a.wtype); return AMV_ERR_UNSUPPORTED;
    }
}

static int check_common(const char* fn, int wtype, const void* w, int64_t n_rows, int64_t k, const void* act,
                        int64_t m) {
    AMV_REQUIRE(w && act, "%s: null pointer", fn);
    AMV_REQUIRE(n_rows > 0 && k > 0 && m > 0, "%s: empty shape", fn);
    AMV_REQUIRE(n_rows <= INT32_MAX && k <= INT32_MAX, "%s: shape too large", fn);
    AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0, "%s: w and act must be 16-byte aligned", fn);
    if (wtype == AMV_T_Q4_0 || wtype == AMV_T_Q8_0) {
        AMV_REQUIRE(k % 32 == 0, "%s: k %% 32 != 0", fn);
        AMV_REQUIRE(n_rows * (k / 32) <= INT32_MAX, "%s: too many blocks", fn);
    } else if (wtype == AMV_T_Q4_K || wtype == AMV_T_Q6_K) {
        AMV_REQUIRE(k % 256 == 0, "%s: k %% 256 != 0", fn);
    } else {
        amv_set_error("%s: weight type %d not supported", fn, wtype);
        return AMV_ERR_UNSUPPORTED;
    }
    return AMV_OK;
}

static int act_type_of(int wtype) { return (wtype == AMV_T_Q4_K || wtype == AMV_T_Q6_K) ? AMV_T_Q8_K : AMV_T_Q8_0; }

// Column c of an activation buffer of m columns (amv_quantize_act y_act layout).
static void column_view(MmvArgs& a, const uint8_t* act, int64_t m, int64_t c) {
    const int64_t k = a.k;
    a.aq = reinterpret_cast<const int8_t*>(act + c * k);
    if (act_type_of(a.wtype) == AMV_T_Q8_0) {
        a.ameta0 = act + m * k + c * (k / 32) * 8;
        a.ameta1 = nullptr;
    } else {
        a.ameta0 = act + m * k + c * (k / 256) * 4;
        a.ameta1 = act + m * k + m * (k / 256) * 4 + c * (k / 16) * 4;
    }
}

extern "C" int amv_mul_mat_vec(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                               float* dst, int64_t ldd, void* stream) {
    int rc = check_common("amv_mul_mat_vec", wtype, w, n_rows, k, act, m);
    if (rc) return rc;
    AMV_REQUIRE(dst, "amv_mul_mat_vec: null dst");
    AMV_REQUIRE(ldd >= n_rows, "amv_mul_mat_vec: ldd %lld < n_rows %lld", (long long)ldd, (long long)n_rows);
    hipStream_t st = amv_stream(stream);
    for (int64_t c = 0; c < m; ++c) {
        MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, dst + c * ldd, nullptr};
        column_view(a, (const uint8_t*)act, m, c);
        rc = mmv_one_column<false>(a, st);
        if (rc) return rc;
    }
    return amv_check_launch("amv_mul_mat_vec");
}

extern "C" int amv_mul_mat_block_sums(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act,
                                      int64_t m, int32_t* sums, void* stream) {
    int rc = check_common("amv_mul_mat_block_sums", wtype, w, n_rows, k, act, m);
    if (rc) return rc;
    AMV_REQUIRE(sums, "amv_mul_mat_block_sums: null output");
    hipStream_t st = amv_stream(stream);
    const int64_t per = (wtype == AMV_T_Q4_K) ? 2 : 1;
    const int64_t nblk = (act_type_of(wtype) == AMV_T_Q8_0 ? k / 32 : k / 256) * per;
    for (int64_t c = 0; c < m; ++c) {
        MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, nullptr,
                  sums + c * n_rows * nblk};
        column_view(a, (const uint8_t*)act, m, c);
        rc = mmv_one_column<true>(a, st);
        if (rc) return rc;
    }
    return amv_check_launch("amv_mul_mat_block_sums");
}
