// Prefill MUL_MAT (many activation columns) on quantized weights with CDNA4 int8 MFMA.
//
// Role of ameva_mmq.comp / ameva_mmqb.comp (reference, enc_mul_mat_mmq ggml-ameva.cpp:2540-2647). For every 32-weight
// block b the exact integer block sums S[n][m][b] = sum_k w_int[n][k] q_a[m][k] (the ints of ggml's
// vec_dot_q4_0_q8_0 / q8_0_q8_0) come out of one v_mfma_i32_16x16x32_i8 per 16 x 16 tile (K = 32 = one block, so a
// block's sums are never mixed with another block's scale); the f32 epilogue adds S * (d_w[n][b] * d_a[m][b]).
// That per-block f32 epilogue (3 VALU ops per output per block) is the bound of this kernel, not the MFMA.
//
// MFMA operand layout (16x16x32 i8): lane l supplies row i = l % 16 of A and column j = l % 16 of B, 8 int8 of
// k = 8 (l / 16) .. 8 (l / 16) + 7 each; it receives D[4 (l / 16) + r][l % 16], r = 0..3. Here A = weight rows
// (i <-> n) and B = activation rows (j <-> token m), so a lane's 4 outputs share one token and span 4 weight rows.
// Q4_0 block bytes: element k < 16 is the low nibble of byte k, element 16 + k the high nibble, so lane group g
// takes bytes 8 (g & 1) .. + 7 and nibble half g >> 1; (nib - 8) as a signed byte is ((nib + 0x78) ^ 0x80).
#include "amv_common.h"

typedef int v4i __attribute__((ext_vector_type(4)));

// TI 16-row weight tiles and TJ 16-token tiles per wave; a workgroup is 2 x 2 waves: 32 TI rows x 32 TJ tokens.
// U blocks per pipeline step: the loads of step s + 1 are in flight while step s computes.

// Operands of U consecutive blocks for one wave: A (8 weight bytes per 16-row tile), the weight scales of the 4
// rows whose outputs the lane holds (rows 4 g .. 4 g + 3 of each tile, as fp16 pairs), B (8 activation bytes per
// 16-token tile) and the activation scale of the lane's token.
template <int TI, int TJ, int U>
struct MmqFrag {
    uint2 a[U][TI];
    uint32_t d[U][TI][2];
    uint2 bq[U][TJ];
    float da[U][TJ];
};

// FULL: the launch's row tiles are whole and n_rows even (Q4_0: the scales of rows 4 g .. 4 g + 3 are two dwords of
// the paired layout); otherwise rows are clamped and each scale is read alone.
template <int WT, int TI, int TJ, int U, bool FULL, bool FULLK>
__device__ __forceinline__ void mmq_load(MmqFrag<TI, TJ, U>& f, int b0, const uint8_t* __restrict__ wq,
                                         const uint16_t* __restrict__ wd, int N, int nb, const int8_t* __restrict__ aq,
                                         const int2* __restrict__ ameta, int K, const int (&nrow)[TI],
                                         const int (&mrow)[TJ], int n_wave, int g) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int b = FULLK ? b0 + u : min(b0 + u, nb - 1);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const size_t bi = (size_t)nrow[i] * nb + b;
            if (WT == AMV_T_Q4_0) f.a[u][i] = *reinterpret_cast<const uint2*>(wq + bi * 16 + 8 * (g & 1));
            else f.a[u][i] = *reinterpret_cast<const uint2*>(wq + bi * 32 + 8 * g);
            const int r4 = n_wave + 16 * i + 4 * g;
            if (WT == AMV_T_Q4_0 && FULL) {
                const uint32_t* wd2 = reinterpret_cast<const uint32_t*>(wd);
                f.d[u][i][0] = wd2[(size_t)(r4 >> 1) * nb + b];
                f.d[u][i][1] = wd2[(size_t)((r4 >> 1) + 1) * nb + b];
            } else {
                uint32_t h[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = min(r4 + r, N - 1);
                    h[r] = wd[WT == AMV_T_Q4_0 ? amv_q4_0_didx(row, b, nb, N) : (size_t)row * nb + b];
                }
                f.d[u][i][0] = h[0] | (h[1] << 16);
                f.d[u][i][1] = h[2] | (h[3] << 16);
            }
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            f.bq[u][j] = *reinterpret_cast<const uint2*>(aq + (size_t)mrow[j] * K + 32 * b + 8 * g);
            f.da[u][j] = __int_as_float(ameta[(size_t)mrow[j] * nb + b].x);
        }
    }
}

// One pipeline step: the U blocks of f through the MFMAs and the f32 epilogue (or the exact sums when SUMS).
template <int WT, bool SUMS, int TI, int TJ, int U, bool FULLK>
__device__ __forceinline__ void mmq_compute(const MmqFrag<TI, TJ, U>& f, int b0, int nb, int sh, float (&acc)[TI][TJ][4],
                                            int N, int M, int n_wave, int m_wave, int g, int r16,
                                            int32_t* __restrict__ sums) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int b = b0 + u;
        if (!FULLK && b >= nb) break;
        long A[TI];
        float dw[TI][4];
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            uint2 q = f.a[u][i];
            if (WT == AMV_T_Q4_0) {
                // (nibble - 8) as a signed byte: ((nibble + 0x78) ^ 0x80)
                q.x = (((q.x >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
                q.y = (((q.y >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
            }
            A[i] = (long)(((uint64_t)q.y << 32) | q.x);
            dw[i][0] = amv_h2f(f.d[u][i][0]);
            dw[i][1] = amv_h2f(f.d[u][i][0] >> 16);
            dw[i][2] = amv_h2f(f.d[u][i][1]);
            dw[i][3] = amv_h2f(f.d[u][i][1] >> 16);
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const long B = (long)(((uint64_t)f.bq[u][j].y << 32) | f.bq[u][j].x);
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const v4i zero = {0, 0, 0, 0};
                const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[i], B, zero, 0, 0, 0);
                if (SUMS) {
                    const int m = m_wave + 16 * j + r16;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = n_wave + 16 * i + 4 * g + r;
                        if (m < M && n < N) sums[((size_t)m * N + n) * nb + b] = C[r];
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf((float)C[r], dw[i][r] * f.da[u][j], acc[i][j][r]);
                }
            }
        }
    }
}

// FULLK: nb % U == 0 (every step is whole: block indices need no clamp and fold into load offsets).
template <int WT, bool SUMS, int TI, int TJ, int U, bool FULL, bool FULLK>
__global__ __launch_bounds__(256) void k_mmq(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N,
                                            int nb, const int8_t* __restrict__ aq, const int2* __restrict__ ameta,
                                            int M, float* __restrict__ dst, int64_t ldd, int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int n_wave = blockIdx.x * (2 * 16 * TI) + (w & 1) * (16 * TI);
    const int m_wave = blockIdx.y * (2 * 16 * TJ) + (w >> 1) * (16 * TJ);
    const int K = nb * 32;
    float acc[TI][TJ][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
    int nrow[TI], mrow[TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i) nrow[i] = min(n_wave + 16 * i + r16, N - 1);
#pragma unroll
    for (int j = 0; j < TJ; ++j) mrow[j] = min(m_wave + 16 * j + r16, M - 1);
    const int sh = (g >> 1) * 4;  // Q4_0: nibble half of this lane group

    // two operand sets in ping-pong: the loads of one step are in flight while the other computes
    // (steps of U blocks; the last step may be partial when nb % U != 0)
    const int steps = (nb + U - 1) / U;
    MmqFrag<TI, TJ, U> f0, f1;
    mmq_load<WT, TI, TJ, U, FULL, FULLK>(f0, 0, wq, wd, N, nb, aq, ameta, K, nrow, mrow, n_wave, g);
    int s = 0;
    for (; s + 2 <= steps; s += 2) {
        mmq_load<WT, TI, TJ, U, FULL, FULLK>(f1, (s + 1) * U, wq, wd, N, nb, aq, ameta, K, nrow, mrow, n_wave, g);
        mmq_compute<WT, SUMS, TI, TJ, U, FULLK>(f0, s * U, nb, sh, acc, N, M, n_wave, m_wave, g, r16, sums);
        if (s + 2 < steps)
            mmq_load<WT, TI, TJ, U, FULL, FULLK>(f0, (s + 2) * U, wq, wd, N, nb, aq, ameta, K, nrow, mrow, n_wave, g);
        mmq_compute<WT, SUMS, TI, TJ, U, FULLK>(f1, (s + 1) * U, nb, sh, acc, N, M, n_wave, m_wave, g, r16, sums);
    }
    if (s < steps) mmq_compute<WT, SUMS, TI, TJ, U, FULLK>(f0, s * U, nb, sh, acc, N, M, n_wave, m_wave, g, r16, sums);
    if (!SUMS) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int m = m_wave + 16 * j + r16;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int n = n_wave + 16 * i + 4 * g;
                float* o = dst + (size_t)m * ldd + n;
                if (FULL && ldd % 4 == 0) {
                    *reinterpret_cast<float4*>(o) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < N) o[r] = acc[i][j][r];
                }
            }
        }
    }
}

template <int WT, bool SUMS, int TI, int TJ, int U>
static void mmq_launch(const uint8_t* wq, const uint16_t* wd, int N, int nb, const int8_t* aq, const int2* ameta,
                       int M, float* dst, int64_t ldd, int32_t* sums, hipStream_t st) {
    const dim3 grid((unsigned)((N + 32 * TI - 1) / (32 * TI)), (unsigned)((M + 32 * TJ - 1) / (32 * TJ)));
    const bool full = N % (32 * TI) == 0 && (!dst || ((uintptr_t)dst & 15) == 0);
    if (full && nb % U == 0)
        hipLaunchKernelGGL((k_mmq<WT, SUMS, TI, TJ, U, true, true>), grid, dim3(256), 0, st, wq, wd, N, nb, aq, ameta, M,
                           dst, ldd, sums);
    else
        hipLaunchKernelGGL((k_mmq<WT, SUMS, TI, TJ, U, false, false>), grid, dim3(256), 0, st, wq, wd, N, nb, aq, ameta,
                           M, dst, ldd, sums);
}

// Token tile by batch and grid fill (MI355X sweep, 512 tokens): 128-token workgroups (TJ = 4, one block per step)
// while that still gives >= 192 workgroups (gate/up 28672 rows: 169 TOPS, q/k/v 6144: 136), otherwise 64 tokens
// (TJ = 2, two blocks per step; the 4096-row projections: 130-134 TOPS against 93-98 with TJ = 4).
template <int WT, bool SUMS>
static void mmq_dispatch(const uint8_t* wq, const uint16_t* wd, int N, int nb, const int8_t* aq, const int2* ameta,
                         int M, float* dst, int64_t ldd, int32_t* sums, hipStream_t st) {
    const int64_t row_tiles = (N + 127) / 128;
    if (M <= 32) mmq_launch<WT, SUMS, 4, 1, 2>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
    else if (M <= 64 || row_tiles * ((M + 127) / 128) < 192)
        mmq_launch<WT, SUMS, 4, 2, 2>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
    else mmq_launch<WT, SUMS, 4, 4, 1>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
}

static int mmq_impl(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
                    int64_t ldd, int32_t* sums, void* stream) {
    AMV_REQUIRE(w && act && (dst || sums), "amv_mul_mat_q: null pointer");
    AMV_REQUIRE(wtype == AMV_T_Q4_0 || wtype == AMV_T_Q8_0, "amv_mul_mat_q: weight type %d not supported (Q4_0, Q8_0)",
                wtype);
    AMV_REQUIRE(n_rows > 0 && m > 0 && k > 0 && k % 32 == 0, "amv_mul_mat_q: bad shape");
    AMV_REQUIRE(n_rows <= INT32_MAX && m <= 65535LL * 32 && n_rows * (k / 32) <= INT32_MAX, "amv_mul_mat_q: too large");
    AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0, "amv_mul_mat_q: buffers must be 16-byte aligned");
    AMV_REQUIRE(!dst || ldd >= n_rows, "amv_mul_mat_q: ldd < n_rows");
    const int nb = (int)(k / 32);
    const int64_t nblk = n_rows * nb;
    const uint8_t* wq = (const uint8_t*)w;
    const uint16_t* wd = (const uint16_t*)(wq + nblk * (wtype == AMV_T_Q4_0 ? 16 : 32));
    const int8_t* aq = (const int8_t*)act;
    const int2* ameta = (const int2*)((const uint8_t*)act + m * k);
    hipStream_t st = amv_stream(stream);
    if (wtype == AMV_T_Q4_0) {
        if (sums) mmq_dispatch<AMV_T_Q4_0, true>(wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums, st);
        else mmq_dispatch<AMV_T_Q4_0, false>(wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums, st);
    } else {
        if (sums) mmq_dispatch<AMV_T_Q8_0, true>(wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums, st);
        else mmq_dispatch<AMV_T_Q8_0, false>(wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums, st);
    }
    return amv_check_launch("amv_mul_mat_q");
}

extern "C" int amv_mul_mat_q(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                             float* dst, int64_t ldd, void* stream) {
    AMV_REQUIRE(dst, "amv_mul_mat_q: null dst");
    return mmq_impl(wtype, w, n_rows, k, act, m, dst, ldd, nullptr, stream);
}

extern "C" int amv_mul_mat_q_block_sums(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act,
                                        int64_t m, int32_t* sums, void* stream) {
    AMV_REQUIRE(sums, "amv_mul_mat_q_block_sums: null output");
    return mmq_impl(wtype, w, n_rows, k, act, m, nullptr, 0, sums, stream);
}
