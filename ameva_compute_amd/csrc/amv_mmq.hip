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
// KS = 4: the 4 waves share one tile (16 TI rows x 16 TJ tokens per workgroup) and split its pipeline steps
// (wave w takes steps w, w + 4, ...); their f32 partials are added in LDS in wave order (small batches: many
// workgroups instead of few long ones).
template <int WT, bool SUMS, int TI, int TJ, int U, bool FULL, bool FULLK, int WR, int KS>
__global__ __launch_bounds__(256) void k_mmq(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N,
                                            int nb, const int8_t* __restrict__ aq, const int2* __restrict__ ameta,
                                            int M, float* __restrict__ dst, int64_t ldd, int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    // WR waves along the weight rows, 4 / WR along the tokens (KS = 1); with KS = 4 one tile per workgroup
    const int n_wave = KS == 4 ? blockIdx.x * (16 * TI) : blockIdx.x * (WR * 16 * TI) + (w % WR) * (16 * TI);
    const int m_wave = KS == 4 ? blockIdx.y * (16 * TJ) : blockIdx.y * ((4 / WR) * 16 * TJ) + (w / WR) * (16 * TJ);
    const int ks = KS == 4 ? w : 0;
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
    int s = ks;
    if (s < steps) mmq_load<WT, TI, TJ, U, FULL, FULLK>(f0, s * U, wq, wd, N, nb, aq, ameta, K, nrow, mrow, n_wave, g);
    for (; s + KS < steps; s += 2 * KS) {
        mmq_load<WT, TI, TJ, U, FULL, FULLK>(f1, (s + KS) * U, wq, wd, N, nb, aq, ameta, K, nrow, mrow, n_wave, g);
        mmq_compute<WT, SUMS, TI, TJ, U, FULLK>(f0, s * U, nb, sh, acc, N, M, n_wave, m_wave, g, r16, sums);
        if (s + 2 * KS < steps)
            mmq_load<WT, TI, TJ, U, FULL, FULLK>(f0, (s + 2 * KS) * U, wq, wd, N, nb, aq, ameta, K, nrow, mrow, n_wave,
                                                 g);
        mmq_compute<WT, SUMS, TI, TJ, U, FULLK>(f1, (s + KS) * U, nb, sh, acc, N, M, n_wave, m_wave, g, r16, sums);
    }
    if (s < steps) mmq_compute<WT, SUMS, TI, TJ, U, FULLK>(f0, s * U, nb, sh, acc, N, M, n_wave, m_wave, g, r16, sums);
    if constexpr (KS == 4 && !SUMS) {
        __shared__ float red[3][TI * TJ * 4][64];
        if (w > 0) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) red[w - 1][(i * TJ + j) * 4 + r][lane] = acc[i][j][r];
        }
        __syncthreads();
        if (w > 0) return;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int q = (i * TJ + j) * 4 + r;
                    acc[i][j][r] = ((acc[i][j][r] + red[0][q][lane]) + red[1][q][lane]) + red[2][q][lane];
                }
    }
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

// ---------------------------------------------------------------------------------------------------------------
// Small batches (m <= 32) of Q4_0 / Q8_0, streamed like the GEMV (k_mmq_sb). A wave owns 16 weight rows and all the
// tokens (one or two 16-token tiles); the 4 waves of a workgroup take every fourth group of 4 blocks of those rows
// and add their f32 partials in LDS in wave order. Per group each lane issues whole 16-byte loads: block 4 q + g of
// its row (lane group g = l / 16), of its token's activation row and of the scale runs of 4 blocks; a 4 x 4 transpose
// of dwords across the lane groups (v_permlane32_swap, then v_permlane16_swap) hands lane group g dword g of every
// block, i.e. the MFMA operands of one v_mfma_i32_16x16x32_i8 per block: lane group g supplies the k slots 8 g .. 8 g
// + 7 as weights 4 g .. 4 g + 3 (Q4_0: the low nibbles of bytes 4 g .. 4 g + 3; Q8_0: those bytes) and weights
// 16 + 4 g .. 16 + 4 g + 3 (high nibbles; bytes 16 + 4 g ..), the activations in the same slots. Each block's exact
// integer comes out of its MFMA, then the f32 epilogue acc += S * (d_w * d_a). The loads of the next group are in
// flight while a group computes. Needs nb % 4 == 0 (16-byte scale runs) and, for Q4_0, an even row count (paired
// scales).
// ---------------------------------------------------------------------------------------------------------------
typedef unsigned int sb_v4u __attribute__((ext_vector_type(4)));
typedef unsigned int sb_v2u __attribute__((ext_vector_type(2)));

// lane group g of (x0, x1, x2, x3) ends up with dword g of the values lane groups 0..3 held: x_j <- x_g of group j
__device__ __forceinline__ void sb_transpose4(uint32_t& x0, uint32_t& x1, uint32_t& x2, uint32_t& x3) {
    const auto a = __builtin_amdgcn_permlane32_swap(x0, x2, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(x1, x3, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    x0 = c[0];
    x1 = c[1];
    x2 = d[0];
    x3 = d[1];
}
__device__ __forceinline__ void sb_transpose4(sb_v4u& v) {
    uint32_t x0 = v.x, x1 = v.y, x2 = v.z, x3 = v.w;
    sb_transpose4(x0, x1, x2, x3);
    v = sb_v4u{x0, x1, x2, x3};
}

template <int WT, int TI, int TJ, int NW, bool SUMS>
__global__ __launch_bounds__(64 * NW) void k_mmq_sb(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N,
                                               int nb, const int8_t* __restrict__ aq, const int2* __restrict__ ameta,
                                               int M, float* __restrict__ dst, int64_t ldd,
                                               int32_t* __restrict__ sums) {
    constexpr int QW = WT == AMV_T_Q4_0 ? 1 : 2;  // 16-byte chunks per weight block
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16 * TI;
    const size_t K = (size_t)nb * 32;
    const int ngrp = nb >> 2;
    const sb_v4u* wr[TI];
#pragma unroll
    for (int i = 0; i < TI; ++i)
        wr[i] = reinterpret_cast<const sb_v4u*>(wq) + (size_t)min(n0 + 16 * i + r16, N - 1) * nb * QW;
    const sb_v4u* ar[TJ];
    const int2* mr[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int t = min(16 * j + r16, M - 1);
        ar[j] = reinterpret_cast<const sb_v4u*>(aq + t * K);
        mr[j] = ameta + (size_t)t * nb;
    }
    // scale runs of the lane's 4 output rows 16 i + 4 g .. + 3 of each tile: Q4_0 two row pairs, Q8_0 four rows
    const sb_v4u* sp[TI][2];
    const sb_v2u* sq[TI][4];
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        if constexpr (WT == AMV_T_Q4_0) {
            const int pmax = N / 2 - 1, pb = ((n0 + 16 * i) >> 1) + 2 * g;
            sp[i][0] = reinterpret_cast<const sb_v4u*>(wd) + (size_t)min(pb, pmax) * (nb >> 2);
            sp[i][1] = reinterpret_cast<const sb_v4u*>(wd) + (size_t)min(pb + 1, pmax) * (nb >> 2);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                sq[i][e] = reinterpret_cast<const sb_v2u*>(wd) + (size_t)min(n0 + 16 * i + 4 * g + e, N - 1) * (nb >> 2);
        }
    }
    float acc[TI][TJ][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;

    // one group's loads: lane group g takes block 4 q + g of its rows and tokens (with that block's activation scale)
    // and the scale runs of blocks 4 q .. 4 q + 3 of its output rows
    sb_v4u lw[2][TI][QW], la[2][TJ][2], ls[2][TI][2];
    sb_v2u lq[2][TI][4];
    float lm[2][TJ];
    const auto load = [&](int s, int q) {
        const size_t b = (size_t)4 * q + g;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int c = 0; c < QW; ++c) lw[s][i][c] = __builtin_nontemporal_load(wr[i] + b * QW + c);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            la[s][j][0] = ar[j][2 * b];
            la[s][j][1] = ar[j][2 * b + 1];
            lm[s][j] = __int_as_float(mr[j][b].x);
        }
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            if constexpr (WT == AMV_T_Q4_0) {
                ls[s][i][0] = sp[i][0][q];
                ls[s][i][1] = sp[i][1][q];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) lq[s][i][e] = sq[i][e][q];
            }
        }
    };
    const auto compute = [&](int s, int q) {
        // operands: dword g of each block of the group; the activation scales of all 4 blocks
        sb_v4u wv[TI][QW], av[TJ][2];
        uint32_t da[TJ][4];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int c = 0; c < QW; ++c) {
                wv[i][c] = lw[s][i][c];
                sb_transpose4(wv[i][c]);
            }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            av[j][0] = la[s][j][0];
            av[j][1] = la[s][j][1];
            sb_transpose4(av[j][0]);
            sb_transpose4(av[j][1]);
            const uint32_t d = __float_as_uint(lm[s][j]);
            da[j][0] = da[j][1] = da[j][2] = da[j][3] = d;
            sb_transpose4(da[j][0], da[j][1], da[j][2], da[j][3]);  // da[j][jb]: the scale of block 4 q + jb
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            long A[TI];
            float dw[TI][4];
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                uint32_t lo, hi;
                if constexpr (WT == AMV_T_Q4_0) {
                    const uint32_t x = wv[i][0][jb];
                    lo = ((x & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;  // (nibble - 8) as a signed byte
                    hi = (((x >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
                    dw[i][0] = amv_h2f(ls[s][i][0][jb]);
                    dw[i][1] = amv_h2f(ls[s][i][0][jb] >> 16);
                    dw[i][2] = amv_h2f(ls[s][i][1][jb]);
                    dw[i][3] = amv_h2f(ls[s][i][1][jb] >> 16);
                } else {
                    lo = wv[i][0][jb];
                    hi = wv[i][1][jb];
#pragma unroll
                    for (int e = 0; e < 4; ++e) dw[i][e] = amv_h2f(lq[s][i][e][jb >> 1] >> (16 * (jb & 1)));
                }
                A[i] = (long)(((uint64_t)hi << 32) | lo);
            }
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const long B = (long)(((uint64_t)av[j][1][jb] << 32) | av[j][0][jb]);
                const float dav = __uint_as_float(da[j][jb]);
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const v4i zero = {0, 0, 0, 0};
                    const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[i], B, zero, 0, 0, 0);
                    if constexpr (SUMS) {
                        const int m = 16 * j + r16;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int n = n0 + 16 * i + 4 * g + e;
                            if (m < M && n < N) sums[((size_t)m * N + n) * nb + 4 * q + jb] = C[e];
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf((float)C[e], dw[i][e] * dav, acc[i][j][e]);
                    }
                }
            }
        }
    };
    // the wave's groups w, w + NW, ..., two buffers; no load sits behind a branch inside an iteration, so the
    // wait before each compute covers exactly the loads it reads (a conditional load made the compiler wait for the
    // prefetch as well)
    const int nit = (ngrp - w + NW - 1) / NW;
    if (nit > 0) {
        load(0, w);
        int k = 0;
        for (; k + 2 < nit; k += 2) {
            load(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);  // each prefetch goes out before the compute that follows it
            compute(0, w + k * NW);
            __builtin_amdgcn_sched_barrier(0);
            load(0, w + (k + 2) * NW);
            __builtin_amdgcn_sched_barrier(0);
            compute(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (nit - k == 2) {
            load(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);
            compute(0, w + k * NW);
            compute(1, w + (k + 1) * NW);
        } else {
            compute(0, w + k * NW);
        }
    }
    if constexpr (!SUMS) {
        __shared__ float red[NW - 1][TI * TJ * 4][64];
        if (w > 0) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) red[w - 1][(i * TJ + j) * 4 + e][lane] = acc[i][j][e];
        }
        __syncthreads();
        if (w > 0) return;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int m = 16 * j + r16;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int x = (i * TJ + j) * 4 + e;
                    float v = acc[i][j][e];
#pragma unroll
                    for (int o = 0; o < NW - 1; ++o) v += red[o][x][lane];  // wave order
                    const int n = n0 + 16 * i + 4 * g + e;
                    if (m < M && n < N) dst[(size_t)m * ldd + n] = v;
                }
            }
    }
}

// the streamed small-batch kernel where it applies: two 16-row tiles per wave (sharing the activation operands) and
// 4 waves per workgroup while that leaves >= 256 workgroups, else one tile per wave and 8 waves splitting k
template <int WT, bool SUMS>
static bool mmq_sb_launch(const uint8_t* wq, const uint16_t* wd, int N, int nb, const int8_t* aq, const int2* ameta,
                          int M, float* dst, int64_t ldd, int32_t* sums, hipStream_t st) {
    if (M > 32 || nb % 4 != 0 || (WT == AMV_T_Q4_0 && N % 2 != 0)) return false;
    const bool two = (N + 31) / 32 >= 256;
    const dim3 grid((unsigned)(two ? (N + 31) / 32 : (N + 15) / 16));
#define SB(TI, TJ, NW) hipLaunchKernelGGL((k_mmq_sb<WT, TI, TJ, NW, SUMS>), grid, dim3(64 * NW), 0, st, wq, wd, N, nb, \
                                          aq, ameta, M, dst, ldd, sums)
    if (M <= 16) {
        if (two) SB(2, 1, 4);
        else SB(1, 1, 8);
    } else {
        if (two) SB(2, 2, 4);
        else SB(1, 2, 8);
    }
#undef SB
    return true;
}

template <int WT, bool SUMS, int TI, int TJ, int U, int WR = 2, int KS = 1>
static void mmq_launch(const uint8_t* wq, const uint16_t* wd, int N, int nb, const int8_t* aq, const int2* ameta,
                       int M, float* dst, int64_t ldd, int32_t* sums, hipStream_t st) {
    constexpr int RT = KS == 4 ? 16 * TI : WR * 16 * TI, MT = KS == 4 ? 16 * TJ : (4 / WR) * 16 * TJ;
    const dim3 grid((unsigned)((N + RT - 1) / RT), (unsigned)((M + MT - 1) / MT));
    const bool full = N % RT == 0 && (!dst || ((uintptr_t)dst & 15) == 0);
    if (full && nb % U == 0)
        hipLaunchKernelGGL((k_mmq<WT, SUMS, TI, TJ, U, true, true, WR, KS>), grid, dim3(256), 0, st, wq, wd, N, nb, aq,
                           ameta, M, dst, ldd, sums);
    else
        hipLaunchKernelGGL((k_mmq<WT, SUMS, TI, TJ, U, false, false, WR, KS>), grid, dim3(256), 0, st, wq, wd, N, nb,
                           aq, ameta, M, dst, ldd, sums);
}

// Token tile by batch and grid fill (MI355X sweep, 512 tokens): 128-token workgroups (TJ = 4, one block per step)
// while that still gives >= 192 workgroups (gate/up 28672 rows: 169 TOPS, q/k/v 6144: 136), otherwise 64 tokens
// (TJ = 2, two blocks per step; the 4096-row projections: 130-134 TOPS against 93-98 with TJ = 4).
template <int WT, bool SUMS>
static void mmq_dispatch(const uint8_t* wq, const uint16_t* wd, int N, int nb, const int8_t* aq, const int2* ameta,
                         int M, float* dst, int64_t ldd, int32_t* sums, hipStream_t st) {
    const int64_t row_tiles = (N + 127) / 128;
    if (mmq_sb_launch<WT, SUMS>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st)) return;
    if (M <= 32) {
        // small batches: one 16 TI x 16 TJ tile per workgroup, its 4 waves splitting k; the largest row tile that
        // still gives >= 224 workgroups (M = 16: 14336 x 4096 28 us with TI = 4, 4096 x 14336 41 us with TI = 1)
        const int ti = N / 64 >= 224 ? 4 : (N / 32 >= 224 ? 2 : 1);
        if (M <= 16) {
            if (ti == 4) mmq_launch<WT, SUMS, 4, 1, 2, 1, 4>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
            else if (ti == 2) mmq_launch<WT, SUMS, 2, 1, 4, 1, 4>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
            else mmq_launch<WT, SUMS, 1, 1, 4, 1, 4>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
        } else {
            if (ti == 4) mmq_launch<WT, SUMS, 4, 2, 2, 1, 4>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
            else if (ti == 2) mmq_launch<WT, SUMS, 2, 2, 2, 1, 4>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
            else mmq_launch<WT, SUMS, 1, 2, 4, 1, 4>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
        }
    } else if (M <= 64 || row_tiles * ((M + 127) / 128) < 192)
        mmq_launch<WT, SUMS, 4, 2, 2>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
    else mmq_launch<WT, SUMS, 4, 4, 1>(wq, wd, N, nb, aq, ameta, M, dst, ldd, sums, st);
}

// ---------------------------------------------------------------------------------------------------------------
// Q4_K x Q8_K for many tokens on the f16 matrix cores (v_mfma_f32_32x32x16_f16), with ggml's integer structure kept
// exactly: per 256-weight super-block ggml forms I1 = sum_u sc_u * dot_u (dot_u the int dot of 32-weight unit u) and
// I2 = sum_u m_u * bsum_u, then adds d_a * (d * I1 - dmin * I2). Here the weight operand carries sc_u * q (<= 945)
// and the activation operand q_a (<= 127), both exact in f16, so the MFMA's f32 sums are exact integers while they
// stay below 2^24: each super-block is summed in two accumulators of 128 products (<= 15.4 M each), whose f32 sum
// rounds exactly as ggml's conversion of the int32 I1. I2 is one more exact MFMA per super-block (m_u against the
// f16 sums per 16 of the activations). The f32 epilogue thus runs once per 256 weights instead of per 32.
// Roles: A = activations (32 tokens x 16 k), B = weights (16 k x 32 rows), so lane l's output column is weight row
// l % 32 (its own scales) and its 16 outputs are tokens 8 (r / 4) + 4 (l / 32) + r % 4. k slots: lane half h owns
// the weights 128 h .. 128 h + 127 of a super-block (bytes 64 h .. 64 h + 63 of its 128 qs bytes); step s (0..15)
// takes weights 128 h + 8 s .. + 7 (chunk 2 h + s / 8, nibble (s / 4) % 2, bytes 32 (s / 8) + 8 (s % 4) .. + 7).
// ---------------------------------------------------------------------------------------------------------------
typedef _Float16 k4_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 k4_h2 __attribute__((ext_vector_type(2)));
typedef float k4_f16v __attribute__((ext_vector_type(16)));
typedef _Float16 k4_h4 __attribute__((ext_vector_type(4)));
typedef float k4_f16v4 __attribute__((ext_vector_type(4)));

// 8 nibbles (bytes of x0, x1 after the nibble select) -> 8 f16 values nib * sc (exact)
__device__ __forceinline__ k4_h8 k4_nib_f16(uint32_t x0, uint32_t x1, k4_h2 sc2) {
    const k4_h2 off = {(_Float16)1024.0f, (_Float16)1024.0f};
    const uint32_t m64 = 0x64646464u;
    const k4_h2 p0 = __builtin_bit_cast(k4_h2, __builtin_amdgcn_perm(x0, m64, 0x00050004u));  // 1024 + n0, 1024 + n1
    const k4_h2 p1 = __builtin_bit_cast(k4_h2, __builtin_amdgcn_perm(x0, m64, 0x00070006u));
    const k4_h2 p2 = __builtin_bit_cast(k4_h2, __builtin_amdgcn_perm(x1, m64, 0x00050004u));
    const k4_h2 p3 = __builtin_bit_cast(k4_h2, __builtin_amdgcn_perm(x1, m64, 0x00070006u));
    const k4_h2 v0 = (p0 - off) * sc2, v1 = (p1 - off) * sc2, v2 = (p2 - off) * sc2, v3 = (p3 - off) * sc2;
    return k4_h8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
}

// 33..64 tokens: a workgroup of 2 x 2 waves on 64 rows x 64 TT tokens, each wave one 32 x 32 TT tile over all the
// super-blocks (smaller batches run k_mmq_q4k_sb).
template <bool SUMS, int TT>
__global__ __launch_bounds__(256) void k_mmq_q4k(const uint4* __restrict__ wq, const uint4* __restrict__ wh, int N,
                                                int nsb, const uint16_t* __restrict__ a16,
                                                const uint16_t* __restrict__ bs16, const float* __restrict__ dt, int M,
                                                float* __restrict__ dst, int64_t ldd, int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, c = lane & 31, h = lane >> 5;
    const int row0 = blockIdx.x * 64 + 32 * (w & 1);
    const int tok0 = blockIdx.y * (64 * TT) + 32 * TT * (w >> 1);
    const int K = nsb * 256;
    const int row = min(row0 + c, N - 1);
    const uint4* qrow = wq + (size_t)row * nsb * 8 + 4 * h;  // 8 uint4 of qs per super-block; this half's 4
    const uint4* hrow = wh + (size_t)row * nsb;
    const uint16_t* arow[TT];
    const uint16_t* brow[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int tok = min(tok0 + 32 * t + c, M - 1);
        arow[t] = a16 + (size_t)tok * K + 128 * h;
        brow[t] = bs16 + (size_t)tok * (K / 16) + 8 * h;
    }
    k4_f16v acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

    // the weights of the next super-block are loaded while this one computes
    uint4 nq4[4], nhd;
#pragma unroll
    for (int i = 0; i < 4; ++i) nq4[i] = qrow[i];
    nhd = hrow[0];
    for (int j = 0; j < nsb; ++j) {
        uint4 q4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q4[i] = nq4[i];
        const uint4 hd = nhd;
        const int jn = min(j + 1, nsb - 1);  // the last super-block reloads itself (unused)
#pragma unroll
        for (int i = 0; i < 4; ++i) nq4[i] = qrow[(size_t)jn * 8 + i];
        nhd = hrow[jn];
        // scales and mins of units 4 h .. 4 h + 3 (get_scale_min_k4 on the 12 packed bytes)
        int scv[4], mv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) k4_scale_min(4 * h + e, hd.y, hd.z, hd.w, scv[e], mv[e]);
        k4_f16v C0[TT], C1[TT], I2[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) C0[t][r] = C1[t][r] = 0.0f;
#pragma unroll
        for (int st = 0; st < 16; ++st) {
            const int jj = st >> 3, nib = (st >> 2) & 1, seg = st & 3;
            const uint4 v = q4[2 * jj + (seg >> 1)];
            uint32_t x0 = (seg & 1) ? v.z : v.x, x1 = (seg & 1) ? v.w : v.y;
            x0 = (x0 >> (4 * nib)) & 0x0F0F0F0Fu;
            x1 = (x1 >> (4 * nib)) & 0x0F0F0F0Fu;
            const _Float16 scf = (_Float16)(float)scv[2 * jj + nib];
            const k4_h8 B = k4_nib_f16(x0, x1, k4_h2{scf, scf});
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const k4_h8 A = *reinterpret_cast<const k4_h8*>(arow[t] + (size_t)j * 256 + 8 * st);
                if (st < 8) C0[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, B, C0[t], 0, 0, 0);
                else C1[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, B, C1[t], 0, 0, 0);
            }
        }
        // I2: m of the lane's units against the activation sums per 16 (slot e <-> sum 8 h + e <-> unit 4 h + e / 2)
        {
            k4_h8 Bm;
#pragma unroll
            for (int e = 0; e < 8; ++e) Bm[e] = (_Float16)(float)mv[e >> 1];
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const k4_h8 A = *reinterpret_cast<const k4_h8*>(brow[t] + (size_t)j * 16);
                k4_f16v z;
#pragma unroll
                for (int r = 0; r < 16; ++r) z[r] = 0.0f;
                I2[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, Bm, z, 0, 0, 0);
            }
        }
        const float d = amv_h2f(hd.x), dmin = amv_h2f(hd.x >> 16);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int tk = tok0 + 32 * t + 8 * r4 + 4 * h;  // tokens tk .. tk + 3 of outputs 4 r4 .. 4 r4 + 3
                float da[4];
                if (!SUMS) {
                    if (tk + 3 < M && (M & 3) == 0) {
                        const float4 d4 = *reinterpret_cast<const float4*>(dt + (size_t)j * M + tk);
                        da[0] = d4.x; da[1] = d4.y; da[2] = d4.z; da[3] = d4.w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) da[e] = dt[(size_t)j * M + min(tk + e, M - 1)];
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * r4 + e;
                    if (SUMS) {
                        const int tok = tk + e, n = row0 + c;
                        if (tok < M && n < N) {
                            int32_t* o = sums + (((size_t)tok * N + n) * nsb + j) * 2;
                            o[0] = (int)C0[t][r] + (int)C1[t][r];
                            o[1] = (int)I2[t][r];
                        }
                    } else {
                        const float i1 = C0[t][r] + C1[t][r];
                        acc[t][r] = fmaf(da[e], fmaf(d, i1, -dmin * I2[t][r]), acc[t][r]);
                    }
                }
            }
        }
    }
    if (!SUMS) {
        const int n = row0 + c;
        if (n < N) {
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int tok = tok0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (tok < M) dst[(size_t)tok * ldd + n] = acc[t][r];
                }
        }
    }
}

// Small batches (m <= 32) of Q4_K, streamed like k_mmq_sb (k_mmq_q4k_sb). A wave owns TI 16-row weight tiles and
// every token (TJ 16-token tiles); the waves of a workgroup take every NW-th super-block. Roles: A = activations (the
// f16 copies of AMV_ACT_Q8_K_MMA, token l % 16), B = weights (row l % 16), so a lane's 4 outputs are one weight row
// (its own d, dmin and scales) and tokens 4 g .. 4 g + 3. k slots of unit u (one v_mfma_f32_16x16x32_f16 per unit):
// lane group g supplies weights 8 g .. 8 g + 7 of the unit, i.e. the nibbles (low for even u, high for odd u) of bytes
// 8 g .. 8 g + 7 of chunk u / 2; each lane loads chunk g of its row's super-block (32 bytes) and a 4 x 4 transpose of
// the even and of the odd dwords across the lane groups hands it bytes 8 g .. 8 g + 7 of every chunk. The weight
// operand is sc_u * q (<= 945, exact in f16), so each half super-block's f32 sum (<= 15.4 M) is ggml's integer exactly;
// I2 = sum_u m_u bsum_u is one v_mfma_f32_16x16x16_f16 of the activation 16-sums against the mins; then
// acc += d_a (d I1 - dmin I2). The loads of the next super-block are in flight while one computes.
template <int TI, int TJ, int NW, bool SUMS>
__global__ __launch_bounds__(64 * NW) void k_mmq_q4k_sb(const uint4* __restrict__ wq, const uint4* __restrict__ wh,
                                                       int N, int nsb, const uint16_t* __restrict__ a16,
                                                       const uint16_t* __restrict__ bs16, const float* __restrict__ dt,
                                                       int M, float* __restrict__ dst, int64_t ldd,
                                                       int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16 * TI;
    const size_t K = (size_t)nsb * 256;
    const sb_v4u* qr[TI];
    const sb_v4u* hr[TI];
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const size_t row = (size_t)min(n0 + 16 * i + r16, N - 1);
        qr[i] = reinterpret_cast<const sb_v4u*>(wq) + row * nsb * 8 + 2 * g;  // chunk g: 2 x 16 bytes of 8 per super-block
        hr[i] = reinterpret_cast<const sb_v4u*>(wh) + row * nsb;
    }
    const uint16_t* ar[TJ];
    const uint16_t* br[TJ];
    int tk[TJ][4];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const size_t t = (size_t)min(16 * j + r16, M - 1);
        ar[j] = a16 + t * K + 8 * g;
        br[j] = bs16 + t * (K / 16) + 4 * g;
#pragma unroll
        for (int e = 0; e < 4; ++e) tk[j][e] = min(16 * j + 4 * g + e, M - 1);
    }
    float acc[TI][TJ][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;

    sb_v4u lq[2][TI][2], lh[2][TI], la[2][TJ][8];
    sb_v2u lb[2][TJ];
    float ld[2][TJ][4];
    const auto load = [&](int s, int sb) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            lq[s][i][0] = __builtin_nontemporal_load(qr[i] + (size_t)sb * 8);
            lq[s][i][1] = __builtin_nontemporal_load(qr[i] + (size_t)sb * 8 + 1);
            lh[s][i] = __builtin_nontemporal_load(hr[i] + sb);
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
#pragma unroll
            for (int u = 0; u < 8; ++u) la[s][j][u] = *reinterpret_cast<const sb_v4u*>(ar[j] + (size_t)sb * 256 + 32 * u);
            lb[s][j] = *reinterpret_cast<const sb_v2u*>(br[j] + (size_t)sb * 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) ld[s][j][e] = dt[(size_t)sb * M + tk[j][e]];
        }
    };
    const auto compute = [&](int s, int sb) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            // bytes 8 g .. 8 g + 7 of chunk c: dwords 2 g, 2 g + 1 -> ev[c], od[c]
            uint32_t ev[4] = {lq[s][i][0].x, lq[s][i][0].z, lq[s][i][1].x, lq[s][i][1].z};
            uint32_t od[4] = {lq[s][i][0].y, lq[s][i][0].w, lq[s][i][1].y, lq[s][i][1].w};
            sb_transpose4(ev[0], ev[1], ev[2], ev[3]);
            sb_transpose4(od[0], od[1], od[2], od[3]);
            const sb_v4u hd = lh[s][i];
            int scv[8], mlo, mhi, dummy;
#pragma unroll
            for (int u = 0; u < 8; ++u) k4_scale_min(u, hd.y, hd.z, hd.w, scv[u], dummy);
            k4_scale_min(2 * g, hd.y, hd.z, hd.w, dummy, mlo);  // the mins of units 2 g, 2 g + 1 (the I2 k slots)
            k4_scale_min(2 * g + 1, hd.y, hd.z, hd.w, dummy, mhi);
            k4_f16v4 C0[TJ], C1[TJ], I2[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) C0[j][e] = C1[j][e] = I2[j][e] = 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = u >> 1, sh = 4 * (u & 1);
                const _Float16 scf = (_Float16)(float)scv[u];
                const k4_h8 B = k4_nib_f16((ev[c] >> sh) & 0x0F0F0F0Fu, (od[c] >> sh) & 0x0F0F0F0Fu, k4_h2{scf, scf});
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const k4_h8 A = __builtin_bit_cast(k4_h8, la[s][j][u]);
                    if (u < 4) C0[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, C0[j], 0, 0, 0);
                    else C1[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, C1[j], 0, 0, 0);
                }
            }
            // I2: k slot 4 g + e <-> 16-sum 4 g + e of the super-block <-> unit 2 g + e / 2
            const k4_h4 Bm = {(_Float16)(float)mlo, (_Float16)(float)mlo, (_Float16)(float)mhi, (_Float16)(float)mhi};
            const float d = amv_h2f(hd.x), dmin = amv_h2f(hd.x >> 16);
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const k4_h4 Am = __builtin_bit_cast(k4_h4, lb[s][j]);
                I2[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(Am, Bm, I2[j], 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (SUMS) {
                        const int tok = 16 * j + 4 * g + e, n = n0 + 16 * i + r16;
                        if (tok < M && n < N) {
                            int32_t* o = sums + (((size_t)tok * N + n) * nsb + sb) * 2;
                            o[0] = (int)C0[j][e] + (int)C1[j][e];
                            o[1] = (int)I2[j][e];
                        }
                    } else {
                        acc[i][j][e] = fmaf(ld[s][j][e], fmaf(d, C0[j][e] + C1[j][e], -dmin * I2[j][e]), acc[i][j][e]);
                    }
                }
            }
        }
    };
    // the wave's super-blocks w, w + NW, ..., two buffers; no load sits behind a branch inside an iteration, so the
    // wait before each compute covers exactly the loads it reads (a conditional load made the compiler wait for the
    // prefetch as well)
    const int nit = (nsb - w + NW - 1) / NW;
    if (nit > 0) {
        load(0, w);
        int k = 0;
        for (; k + 2 < nit; k += 2) {
            load(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);  // each prefetch goes out before the compute that follows it
            compute(0, w + k * NW);
            __builtin_amdgcn_sched_barrier(0);
            load(0, w + (k + 2) * NW);
            __builtin_amdgcn_sched_barrier(0);
            compute(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (nit - k == 2) {
            load(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);
            compute(0, w + k * NW);
            compute(1, w + (k + 1) * NW);
        } else {
            compute(0, w + k * NW);
        }
    }
    if constexpr (!SUMS) {
        __shared__ float red[NW - 1][TI * TJ * 4][64];
        if (w > 0) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) red[w - 1][(i * TJ + j) * 4 + e][lane] = acc[i][j][e];
        }
        __syncthreads();
        if (w > 0) return;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int x = (i * TJ + j) * 4 + e;
                    float v = acc[i][j][e];
#pragma unroll
                    for (int o = 0; o < NW - 1; ++o) v += red[o][x][lane];  // wave order
                    const int tok = 16 * j + 4 * g + e, n = n0 + 16 * i + r16;
                    if (tok < M && n < N) dst[(size_t)tok * ldd + n] = v;
                }
    }
}

// Small batches (m <= 32) of Q6_K, streamed like k_mmq_sb (k_mmq_q6k_sb): the exact integers of ggml's
// vec_dot_q6_K_q8_K, I = sum over the 16 sub-blocks s of a super-block of sc_s sum_k q_k a_k (q = 6-bit code - 32,
// sc_s int8), then dst += (d * d_a) I. A wave owns TI 16-row weight tiles and every token (TJ 16-token tiles); the NW
// waves of a workgroup take every NW-th super-block and add their f32 partials in LDS in wave order. Roles: A =
// activations (token l % 16), B = weights (row l % 16), so a lane's 4 outputs are its own weight row (its own scales
// and d) and tokens 4 g .. 4 g + 3 (lane group g = l / 16).
// Loads: 16 bytes per lane with consecutive lanes on consecutive bytes (lane 4 r + c: row or token r, 16-byte chunk
// c), so each quad of lanes reads 64 contiguous bytes of a row; ds_bpermute then moves chunk g of row r to lane
// 16 g + r, the MFMA operand layout. Chunks: ql bytes 64 h + 16 c (half h = 0, 1), qh bytes 16 c, the activation
// bytes 64 q + 16 c (q = 0..3), the scale dword c. In ggml's Q6_K layout ql byte 64 h + 16 g + i holds in its low
// nibble element 128 h + 16 g + i (sub-block 8 h + g) and in its high nibble element 128 h + 64 + 16 g + i (sub-block
// 8 h + 4 + g), with bits 2 t, 2 t + 1 of qh byte 32 h + 16 (g & 1) + i above them (quarter t = g >> 1, + 2 for the
// high nibble); the qh chunk of half h sits in lane group 2 h + (g & 1) and v_permlane32_swap hands it over. So for
// q = 2 h + hi lane group g holds sub-block 4 q + g whole (16 signed bytes q - 32), and so does the activation lane
// of the same group. A dot product does not depend on the order of k, so each operand is rearranged the same way
// across lane groups: v_permlane16_swap of (bytes 0..7, bytes 8..15) gives X = sub-block 4 q in groups 0 and 1,
// 4 q + 2 in groups 2 and 3, and Y = 4 q + 1 | 4 q + 3. Two v_mfma_i32_16x16x32_i8 per operand, each with the other
// sub-block's activation slots set to zero, give the two sub-block sums apart. The loads of the next super-block are
// in flight while one computes. Reads the plain Q8_K layout (the prefix of AMV_ACT_Q8_K_MMA too).
template <int TI, int TJ, int NW, bool SUMS>
__global__ __launch_bounds__(64 * NW) void k_mmq_q6k_sb(const uint8_t* __restrict__ wl, const uint8_t* __restrict__ wqh,
                                                       const uint32_t* __restrict__ wsc,
                                                       const uint16_t* __restrict__ wd,
                                                       int N, int nsb, const int8_t* __restrict__ aq,
                                                       const float* __restrict__ ad, int M, float* __restrict__ dst,
                                                       int64_t ldd, int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r16 = lane & 15, g = lane >> 4;
    const int lr4 = lane >> 2, lc = lane & 3;  // load layout: row / token lr4, chunk lc
    const int perm = 4 * (4 * r16 + g);        // ds_bpermute address: the load lane holding chunk g of row r16
    const int n0 = blockIdx.x * 16 * TI;
    const size_t K = (size_t)nsb * 256;
    const uint8_t* lr[TI];
    const uint8_t* hr[TI];
    size_t rb[TI];  // row * nsb
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const size_t row = (size_t)min(n0 + 16 * i + lr4, N - 1);
        rb[i] = row * nsb;
        lr[i] = wl + rb[i] * 128 + 16 * lc;
        hr[i] = wqh + rb[i] * 64 + 16 * lc;
    }
    const int8_t* ar[TJ];
    const float* dr[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const size_t t = (size_t)min(16 * j + lr4, M - 1);
        ar[j] = aq + t * K + 16 * lc;
        dr[j] = ad + t * nsb;
    }
    float acc[TI][TJ][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;

    sb_v4u lq[2][TI][2], lh[2][TI], la[2][TJ][4];
    uint32_t ls[2][TI], ldw[2][TI];
    float lda[2][TJ];
    const auto load = [&](int s, int sb) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
                lq[s][i][h] =
                    __builtin_nontemporal_load(reinterpret_cast<const sb_v4u*>(lr[i] + (size_t)sb * 128 + 64 * h));
            lh[s][i] = __builtin_nontemporal_load(reinterpret_cast<const sb_v4u*>(hr[i] + (size_t)sb * 64));
            ls[s][i] = wsc[(rb[i] + sb) * 4 + lc];
            ldw[s][i] = wd[rb[i] + sb];
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                la[s][j][c] = *reinterpret_cast<const sb_v4u*>(ar[j] + (size_t)sb * 256 + 64 * c);
            lda[s][j] = dr[j][sb];
        }
    };
    const auto bperm = [&](uint32_t v) { return (uint32_t)__builtin_amdgcn_ds_bpermute(perm, (int)v); };
    const auto bperm4 = [&](const sb_v4u& v, uint32_t (&o)[4]) {
        o[0] = bperm(v.x);
        o[1] = bperm(v.y);
        o[2] = bperm(v.z);
        o[3] = bperm(v.w);
    };
    // (bytes 0..7, bytes 8..15) of the 4 lane groups' sub-blocks -> X = groups (0: 0..7 of group 0's, 1: 8..15 of
    // group 0's, 2: 0..7 of group 2's, 3: 8..15 of group 2's), Y the same of groups 1 and 3
    const auto pair = [](const uint32_t (&v)[4], long& X, long& Y) {
        const auto p0 = __builtin_amdgcn_permlane16_swap(v[0], v[2], false, false);
        const auto p1 = __builtin_amdgcn_permlane16_swap(v[1], v[3], false, false);
        X = (long)(((uint64_t)p1[0] << 32) | p0[0]);
        Y = (long)(((uint64_t)p1[1] << 32) | p0[1]);
    };
    const auto compute = [&](int s, int sb) {
        // the activation scales of the lane's output tokens 16 j + 4 g + e, loaded by lanes 4 (4 g + e) + c
        float da[TJ][4];
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) da[j][e] = __shfl(lda[s][j], 16 * g + 4 * e, AMV_WAVE);
        // activation operands of the 4 quarters c (sub-blocks 4 c .. 4 c + 3)
        long AX[TJ][4], AY[TJ][4];
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint32_t v[4];
                bperm4(la[s][j][c], v);
                pair(v, AX[j][c], AY[j][c]);
            }
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            int I[TJ][4];
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) I[j][e] = 0;
            // the 4 scale dwords and d of row r16: loaded by lanes 4 r16 + c
            uint32_t scw[4];
#pragma unroll
            for (int c = 0; c < 4; ++c)
                scw[c] = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * r16 + c), (int)ls[s][i]);
            const uint32_t dw = (uint32_t)__builtin_amdgcn_ds_bpermute(16 * r16, (int)ldw[s][i]);
            // the qh run of half h for this lane group: lane group 2 h + (g & 1) holds it
            uint32_t qh[2][4];
            {
                uint32_t hv[4];
                bperm4(lh[s][i], hv);
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const auto r = __builtin_amdgcn_permlane32_swap(hv[d], hv[d], false, false);
                    qh[0][d] = r[0];
                    qh[1][d] = r[1];
                }
            }
            uint32_t qlw[2][4];  // ql chunk g of each half
            bperm4(lq[s][i][0], qlw[0]);
            bperm4(lq[s][i][1], qlw[1]);
            const int sh = 2 * (g >> 1);  // qh bit pair of the low nibble's quarter (+ 4 for the high nibble)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int h = c >> 1, hi = c & 1;
                uint32_t x[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t lo = ((hi ? qlw[h][d] >> 4 : qlw[h][d]) & 0x0F0F0F0Fu) |
                                        (((qh[h][d] >> (sh + 4 * hi)) & 0x03030303u) << 4);
                    const uint32_t f = lo ^ 0x20202020u;  // 6-bit code - 32: bit 5 flipped, then copied up
                    const uint32_t m5 = f & 0x20202020u;
                    x[d] = f | (m5 << 2) | (m5 << 1);
                }
                long BX, BY;
                pair(x, BX, BY);
                // sc bytes 4 c .. 4 c + 3: X holds sub-blocks 4 c | 4 c + 2, Y 4 c + 1 | 4 c + 3
                const int s0 = (int)(int8_t)scw[c], s1 = (int)(int8_t)(scw[c] >> 8);
                const int s2 = (int)(int8_t)(scw[c] >> 16), s3 = (int)(int8_t)(scw[c] >> 24);
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const v4i zero = {0, 0, 0, 0};
                    const long AXa = g < 2 ? AX[j][c] : 0L, AXb = g < 2 ? 0L : AX[j][c];
                    const long AYa = g < 2 ? AY[j][c] : 0L, AYb = g < 2 ? 0L : AY[j][c];
                    const v4i C0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(AXa, BX, zero, 0, 0, 0);
                    const v4i C2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(AXb, BX, zero, 0, 0, 0);
                    const v4i C1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(AYa, BY, zero, 0, 0, 0);
                    const v4i C3 = __builtin_amdgcn_mfma_i32_16x16x32_i8(AYb, BY, zero, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) I[j][e] += s0 * C0[e] + s2 * C2[e] + s1 * C1[e] + s3 * C3[e];
                }
            }
            const float d = amv_h2f((uint16_t)dw);
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (SUMS) {
                        const int tok = 16 * j + 4 * g + e, n = n0 + 16 * i + r16;
                        if (tok < M && n < N) sums[((size_t)tok * N + n) * nsb + sb] = I[j][e];
                    } else {
                        acc[i][j][e] = fmaf(d * da[j][e], (float)I[j][e], acc[i][j][e]);
                    }
                }
        }
    };
    // the wave's super-blocks w, w + NW, ..., two buffers; no load sits behind a branch inside an iteration, so the
    // wait before each compute covers exactly the loads it reads (a conditional load made the compiler wait for the
    // prefetch as well)
    const int nit = (nsb - w + NW - 1) / NW;
    if (nit > 0) {
        load(0, w);
        int k = 0;
        for (; k + 2 < nit; k += 2) {
            load(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);  // each prefetch goes out before the compute that follows it
            compute(0, w + k * NW);
            __builtin_amdgcn_sched_barrier(0);
            load(0, w + (k + 2) * NW);
            __builtin_amdgcn_sched_barrier(0);
            compute(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (nit - k == 2) {
            load(1, w + (k + 1) * NW);
            __builtin_amdgcn_sched_barrier(0);
            compute(0, w + k * NW);
            compute(1, w + (k + 1) * NW);
        } else {
            compute(0, w + k * NW);
        }
    }
    if constexpr (!SUMS) {
        __shared__ float red[NW - 1][TI * TJ * 4][64];
        if (w > 0) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) red[w - 1][(i * TJ + j) * 4 + e][lane] = acc[i][j][e];
        }
        __syncthreads();
        if (w > 0) return;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int x = (i * TJ + j) * 4 + e;
                    float v = acc[i][j][e];
#pragma unroll
                    for (int o = 0; o < NW - 1; ++o) v += red[o][x][lane];  // wave order
                    const int tok = 16 * j + 4 * g + e, n = n0 + 16 * i + r16;
                    if (tok < M && n < N) dst[(size_t)tok * ldd + n] = v;
                }
    }
}

// Q6_K batches of m <= 32 tokens (plain Q8_K activations or the Q8_K prefix of AMV_ACT_Q8_K_MMA)
static int mmq_q6k_sb(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst, int64_t ldd,
                      int32_t* sums, hipStream_t st) {
    AMV_REQUIRE(k % 256 == 0, "amv_mul_mat_q: Q6_K needs k %% 256 == 0");
    AMV_REQUIRE(m >= 1 && m <= 32, "amv_mul_mat_q: the small-batch Q6_K kernel takes 1..32 tokens");
    const int nsb = (int)(k / 256);
    const int64_t nblk = n_rows * nsb;
    const uint8_t* base = (const uint8_t*)w;
    const uint8_t* wl = base;
    const uint8_t* wqh = base + nblk * 128;
    const uint32_t* wsc = (const uint32_t*)(base + nblk * 192);
    const uint16_t* wd = (const uint16_t*)(base + nblk * 208);
    const int8_t* aq = (const int8_t*)act;
    const float* ad = (const float*)((const uint8_t*)act + m * k);
#define Q6K_SB(TI, TJ, NW)                                                                                          \
    do {                                                                                                             \
        const dim3 G((unsigned)((n_rows + 16 * TI - 1) / (16 * TI)));                                              \
        if (sums) hipLaunchKernelGGL((k_mmq_q6k_sb<TI, TJ, NW, true>), G, dim3(64 * NW), 0, st, wl, wqh, wsc, wd,   \
                                     (int)n_rows, nsb, aq, ad, (int)m, dst, ldd, sums);                              \
        else hipLaunchKernelGGL((k_mmq_q6k_sb<TI, TJ, NW, false>), G, dim3(64 * NW), 0, st, wl, wqh, wsc, wd,       \
                                (int)n_rows, nsb, aq, ad, (int)m, dst, ldd, sums);                                   \
    } while (0)
    // one 16-row tile per wave; 2 waves per workgroup when there are >= 512 tiles (14336 rows), else 4. Measured on
    // MI355X at 14336 x 4096 / 4096 x 14336 (us, hot weights): M = 16 17.6 / 17.2 against 18.5 / 18.4 for two tiles
    // per wave and 4 / 8 waves, and 19-58 for 8 or 16 waves or two tiles with 2 waves; M = 32 28.5 / 26.0 against
    // 33.9 / 26.0 (two tiles per wave with 2 waves 28.4 / 74.8)
    const bool wide = (n_rows + 15) / 16 >= 512;
    if (m <= 16) {
        if (wide) Q6K_SB(1, 1, 2);
        else Q6K_SB(1, 1, 4);
    } else {
        if (wide) Q6K_SB(1, 2, 2);
        else Q6K_SB(1, 2, 4);
    }
#undef Q6K_SB
    return amv_check_launch("amv_mul_mat_q");
}

static int mmq_q4k(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst, int64_t ldd,
                   int32_t* sums, hipStream_t st) {
    AMV_REQUIRE(k % 256 == 0, "amv_mul_mat_q: Q4_K needs k %% 256 == 0");
    const int nsb = (int)(k / 256);
    const int64_t nblk = n_rows * nsb;
    const uint4* wq = (const uint4*)w;
    const uint4* wh = (const uint4*)((const uint8_t*)w + nblk * 128);
    const AmvQ8kMma L = amv_q8k_mma_layout(m, k);
    const uint16_t* a16 = (const uint16_t*)((const uint8_t*)act + L.a16);
    const uint16_t* bs16 = (const uint16_t*)((const uint8_t*)act + L.bs16);
    const float* dt = (const float*)((const uint8_t*)act + L.dt);
    const unsigned gx = (unsigned)((n_rows + 63) / 64);
    if (m <= 32) {
        // small batches, streamed: two 16-row tiles per wave and 4 waves while that leaves >= 256 workgroups, else one
        // tile and 8 waves splitting the super-blocks (4 for two token tiles)
        const bool two = (n_rows + 31) / 32 >= 256;
        const dim3 G((unsigned)(two ? (n_rows + 31) / 32 : (n_rows + 15) / 16));
#define Q4K_SB(TI, TJ, NW)                                                                                           \
    do {                                                                                                              \
        if (sums) hipLaunchKernelGGL((k_mmq_q4k_sb<TI, TJ, NW, true>), G, dim3(64 * NW), 0, st, wq, wh, (int)n_rows, \
                                     nsb, a16, bs16, dt, (int)m, dst, ldd, sums);                                     \
        else hipLaunchKernelGGL((k_mmq_q4k_sb<TI, TJ, NW, false>), G, dim3(64 * NW), 0, st, wq, wh, (int)n_rows, nsb, \
                                a16, bs16, dt, (int)m, dst, ldd, sums);                                               \
    } while (0)
        if (m <= 16) {
            if (two) Q4K_SB(2, 1, 4);
            else Q4K_SB(1, 1, 8);
        } else {
            if (two) Q4K_SB(2, 2, 4);
            else Q4K_SB(1, 2, 4);  // 8 waves of this tile would spill registers
        }
#undef Q4K_SB
    } else {  // 33..64 tokens: 64-row x 64-token tiles of 2 x 2 waves
        const dim3 G(gx, (unsigned)((m + 63) / 64));
        if (sums) hipLaunchKernelGGL((k_mmq_q4k<true, 1>), G, dim3(256), 0, st, wq, wh, (int)n_rows, nsb, a16, bs16, dt,
                                     (int)m, dst, ldd, sums);
        else hipLaunchKernelGGL((k_mmq_q4k<false, 1>), G, dim3(256), 0, st, wq, wh, (int)n_rows, nsb, a16, bs16, dt,
                                (int)m, dst, ldd, sums);
    }
    return amv_check_launch("amv_mul_mat_q");
}

// amv_qgemm.hip: Q4_0 / Q8_0 / Q4_K / Q6_K on the int8 matrix cores with exact block integers, plain activation
// layouts
int amv_qgemm(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
              int64_t ldd, int32_t* sums, hipStream_t st, const float* add = nullptr);

// Batches above this many tokens go to the tiled kernels (amv_qgemm for the exact layouts and the plain ones, the f16
// kernels for the scaled DEQ layouts); smaller ones to the k_mmq kernels of this file, which read the plain Q8_0
// prefix (Q4_0 / Q8_0) or the f16 copies of AMV_ACT_Q8_K_MMA (Q4_K).
#define MMQ16_MIN_M 64

// q4k_mma: act is AMV_ACT_Q8_K_MMA (the small-batch Q4_K kernels read its f16 copies); with a plain Q8_K act every
// Q4_K batch runs the tiled int8 kernel
static int mmq_impl(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
                    int64_t ldd, int32_t* sums, void* stream, bool q4k_mma = false) {
    AMV_REQUIRE(w && act && (dst || sums), "amv_mul_mat_q: null pointer");
    AMV_REQUIRE(wtype == AMV_T_Q4_0 || wtype == AMV_T_Q8_0 || wtype == AMV_T_Q4_K || wtype == AMV_T_Q6_K,
                "amv_mul_mat_q: weight type %d not supported (Q4_0, Q8_0, Q4_K, Q6_K)", wtype);
    AMV_REQUIRE(n_rows > 0 && m > 0 && k > 0 && k % 32 == 0, "amv_mul_mat_q: bad shape");
    AMV_REQUIRE(n_rows <= INT32_MAX && m <= 65535LL * 32 && n_rows * (k / 32) <= INT32_MAX, "amv_mul_mat_q: too large");
    AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0, "amv_mul_mat_q: buffers must be 16-byte aligned");
    AMV_REQUIRE(!dst || ldd >= n_rows, "amv_mul_mat_q: ldd < n_rows");
    // Q6_K up to 32 tokens: the streamed small-batch kernel (the plain Q8_K prefix of either layout)
    if (wtype == AMV_T_Q6_K && m <= 32) return mmq_q6k_sb(w, n_rows, k, act, m, dst, ldd, sums, amv_stream(stream));
    // the tiled int8 kernel reads the plain prefix of any layout
    if (m > MMQ16_MIN_M || wtype == AMV_T_Q6_K || (wtype == AMV_T_Q4_K && !q4k_mma)) {
        AMV_REQUIRE((wtype != AMV_T_Q4_K && wtype != AMV_T_Q6_K) || k % 256 == 0,
                    "amv_mul_mat_q: K-quants need k %% 256 == 0");
        AMV_REQUIRE(m * k <= INT32_MAX && m <= 65535LL * 128, "amv_mul_mat_q: too large");
        return amv_qgemm(wtype, w, n_rows, k, act, m, dst, ldd, sums, amv_stream(stream));
    }
    if (wtype == AMV_T_Q4_K) return mmq_q4k(w, n_rows, k, act, m, dst, ldd, sums, amv_stream(stream));
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

// amv_mmq16.hip: the scaled form of Q4_0 / Q8_0 (AMV_ACT_Q8_0_DEQ activations) and Q4_K (AMV_ACT_Q8_K_DEQ) on the f16
// matrix cores with LDS-staged tiles
int amv_mmq16(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
              int64_t ldd, hipStream_t st);
int amv_mmq16_q4k(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst, int64_t ldd,
                  hipStream_t st);


// dst[t][n] += add[t][n] (row stride ldd): the residual of a fused ADD for the kernels that do not take it
__global__ __launch_bounds__(256) void k_add_rows(float* __restrict__ dst, const float* __restrict__ add, int64_t ldd,
                                                 int m, int n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)m * n) return;
    const int64_t o = (i / n) * ldd + i % n;
    dst[o] = dst[o] + add[o];
}

static int mmq_act_impl(const char* fn, int wtype, const void* w, int64_t n_rows, int64_t k, const void* act,
                        int act_type, int64_t m, float* dst, int64_t ldd, int32_t* sums, void* stream,
                        const float* add = nullptr) {
    const bool deq = act_type == AMV_ACT_Q8_0_DEQ || act_type == AMV_ACT_Q8_K_DEQ;
    const bool q80x = act_type == AMV_ACT_Q8_0_MMA || act_type == AMV_ACT_Q8_0_DEQ;
    const bool q8kx = act_type == AMV_ACT_Q8_K_MMA || act_type == AMV_ACT_Q8_K_DEQ;
    // Q6_K batches above 32 tokens run the tiled int8 kernel (up to 32 the streamed k_mmq_q6k_sb)
    const bool tiled = (m > MMQ16_MIN_M && (((q80x || act_type == AMV_T_Q8_0) && (wtype == AMV_T_Q4_0 || wtype == AMV_T_Q8_0)) ||
                                            ((q8kx || act_type == AMV_T_Q8_K) && wtype == AMV_T_Q4_K))) ||
                       ((q8kx || act_type == AMV_T_Q8_K) && wtype == AMV_T_Q6_K && m > 32);
    if (add && !(tiled && !deq)) {  // only the exact tiled kernels add the residual in their epilogue
        int rc = mmq_act_impl(fn, wtype, w, n_rows, k, act, act_type, m, dst, ldd, nullptr, stream);
        if (rc) return rc;
        const int64_t total = m * n_rows;
        hipLaunchKernelGGL(k_add_rows, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream), dst,
                           add, ldd, (int)m, (int)n_rows);
        return amv_check_launch(fn);
    }
    if (tiled) {
        AMV_REQUIRE(w && act && (dst || sums), "%s: null pointer", fn);
        AMV_REQUIRE(!(deq && sums), "%s: block sums need the exact layout (AMV_ACT_Q8_0_MMA / AMV_ACT_Q8_K_MMA), not "
                    "the scaled one", fn);
        AMV_REQUIRE(n_rows > 0 && k > 0 && k % 32 == 0, "%s: bad shape", fn);
        AMV_REQUIRE(n_rows <= INT32_MAX && m <= 65535LL * 128 && m * k <= INT32_MAX && n_rows * (k / 32) <= INT32_MAX,
                    "%s: too large", fn);
        AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0, "%s: buffers must be 16-byte aligned", fn);
        AMV_REQUIRE(!dst || ldd >= n_rows, "%s: ldd < n_rows", fn);
        if (wtype == AMV_T_Q4_K || wtype == AMV_T_Q6_K) AMV_REQUIRE(k % 256 == 0, "%s: K-quants need k %% 256 == 0", fn);
        AMV_REQUIRE(!(deq && wtype == AMV_T_Q6_K), "%s: Q6_K has no scaled form (use Q8_K or AMV_ACT_Q8_K_MMA)", fn);
        if (!deq) return amv_qgemm(wtype, w, n_rows, k, act, m, dst, ldd, sums, amv_stream(stream), add);
        if (wtype == AMV_T_Q4_K) return amv_mmq16_q4k(w, n_rows, k, act, m, dst, ldd, amv_stream(stream));
        return amv_mmq16(wtype, w, n_rows, k, act, m, dst, ldd, amv_stream(stream));
    }
    // a plain Q8_K activation of a Q4_K batch this small goes to the tiled int8 kernel (mmq_impl with q4k_mma false):
    // the small-batch Q4_K kernels read the f16 copies that only AMV_ACT_Q8_K_MMA holds
    const bool ok = (act_type == AMV_T_Q8_0 || q80x) ? (wtype == AMV_T_Q4_0 || wtype == AMV_T_Q8_0)
                                                     : ((q8kx || act_type == AMV_T_Q8_K) &&
                                                        (wtype == AMV_T_Q4_K || wtype == AMV_T_Q6_K));
    AMV_REQUIRE(ok, "%s: activation type %d does not feed weight type %d", fn, act_type, wtype);
    AMV_REQUIRE(!(deq && wtype == AMV_T_Q6_K), "%s: Q6_K has no scaled form (use Q8_K or AMV_ACT_Q8_K_MMA)", fn);
    // the small-batch Q4_K kernel reads the f16 copies as exact integers
    AMV_REQUIRE(!(deq && wtype == AMV_T_Q4_K), "%s: Q4_K batches of m <= %d need the exact layout AMV_ACT_Q8_K_MMA",
                fn, MMQ16_MIN_M);
    return mmq_impl(wtype, w, n_rows, k, act, m, dst, ldd, sums, stream, q8kx);
}

extern "C" int amv_mul_mat_q_act(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int act_type,
                                 int64_t m, float* dst, int64_t ldd, void* stream) {
    AMV_REQUIRE(dst, "amv_mul_mat_q_act: null dst");
    return mmq_act_impl("amv_mul_mat_q_act", wtype, w, n_rows, k, act, act_type, m, dst, ldd, nullptr, stream);
}

extern "C" int amv_mul_mat_q_act_add(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act,
                                     int act_type, int64_t m, float* dst, int64_t ldd, const float* add, void* stream) {
    AMV_REQUIRE(dst && add, "amv_mul_mat_q_act_add: null dst or add");
    AMV_REQUIRE(add + (m - 1) * ldd + n_rows <= dst || dst + (m - 1) * ldd + n_rows <= add,
                "amv_mul_mat_q_act_add: add overlaps dst");
    return mmq_act_impl("amv_mul_mat_q_act_add", wtype, w, n_rows, k, act, act_type, m, dst, ldd, nullptr, stream,
                        add);
}

extern "C" int amv_mul_mat_q_act_block_sums(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act,
                                            int act_type, int64_t m, int32_t* sums, void* stream) {
    AMV_REQUIRE(sums, "amv_mul_mat_q_act_block_sums: null output");
    return mmq_act_impl("amv_mul_mat_q_act_block_sums", wtype, w, n_rows, k, act, act_type, m, nullptr, 0, sums,
                        stream);
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
