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

#define MMQ_TI 4  // 16-row weight tiles per wave
#define MMQ_TJ 2  // 16-token tiles per wave

template <int WT, bool SUMS>
__global__ __launch_bounds__(256) void k_mmq(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N,
                                            int nb, const int8_t* __restrict__ aq, const int2* __restrict__ ameta,
                                            int M, float* __restrict__ dst, int64_t ldd, int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int n_wave = blockIdx.x * (2 * 16 * MMQ_TI) + (w & 1) * (16 * MMQ_TI);
    const int m_wave = blockIdx.y * (2 * 16 * MMQ_TJ) + (w >> 1) * (16 * MMQ_TJ);
    const int K = nb * 32;
    float acc[MMQ_TI][MMQ_TJ][4];
#pragma unroll
    for (int i = 0; i < MMQ_TI; ++i)
#pragma unroll
        for (int j = 0; j < MMQ_TJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
    int nrow[MMQ_TI], mrow[MMQ_TJ];
#pragma unroll
    for (int i = 0; i < MMQ_TI; ++i) nrow[i] = min(n_wave + 16 * i + r16, N - 1);
#pragma unroll
    for (int j = 0; j < MMQ_TJ; ++j) mrow[j] = min(m_wave + 16 * j + r16, M - 1);

    for (int b = 0; b < nb; ++b) {
        long A[MMQ_TI];
        float dwl[MMQ_TI];
#pragma unroll
        for (int i = 0; i < MMQ_TI; ++i) {
            const size_t bi = (size_t)nrow[i] * nb + b;
            uint2 q;
            if (WT == AMV_T_Q4_0) {
                q = *reinterpret_cast<const uint2*>(wq + bi * 16 + 8 * (g & 1));
                const int sh = (g >> 1) * 4;
                q.x = (((q.x >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
                q.y = (((q.y >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
            } else {
                q = *reinterpret_cast<const uint2*>(wq + bi * 32 + 8 * g);
            }
            A[i] = (long)(((uint64_t)q.y << 32) | q.x);
            dwl[i] = amv_h2f(wd[WT == AMV_T_Q4_0 ? amv_q4_0_didx(nrow[i], b, nb, N) : bi]);
        }
        long B[MMQ_TJ];
        float da[MMQ_TJ];
#pragma unroll
        for (int j = 0; j < MMQ_TJ; ++j) {
            const uint2 q = *reinterpret_cast<const uint2*>(aq + (size_t)mrow[j] * K + 32 * b + 8 * g);
            B[j] = (long)(((uint64_t)q.y << 32) | q.x);
            da[j] = __int_as_float(ameta[(size_t)mrow[j] * nb + b].x);
        }
#pragma unroll
        for (int i = 0; i < MMQ_TI; ++i) {
            // d_w of the 4 weight rows this lane's outputs belong to: rows 4 g + r of the tile, held by lanes 4 g + r
            float dw[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) dw[r] = __shfl(dwl[i], 4 * g + r, AMV_WAVE);
#pragma unroll
            for (int j = 0; j < MMQ_TJ; ++j) {
                const v4i zero = {0, 0, 0, 0};
                const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[i], B[j], zero, 0, 0, 0);
                if (SUMS) {
                    const int m = m_wave + 16 * j + r16;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = n_wave + 16 * i + 4 * g + r;
                        if (m < M && n < N) sums[((size_t)m * N + n) * nb + b] = C[r];
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf((float)C[r], dw[r] * da[j], acc[i][j][r]);
                }
            }
        }
    }
    if (!SUMS) {
#pragma unroll
        for (int j = 0; j < MMQ_TJ; ++j) {
            const int m = m_wave + 16 * j + r16;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < MMQ_TI; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = n_wave + 16 * i + 4 * g + r;
                    if (n < N) dst[(size_t)m * ldd + n] = acc[i][j][r];
                }
        }
    }
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
    const dim3 grid((unsigned)((n_rows + 32 * MMQ_TI - 1) / (32 * MMQ_TI)), (unsigned)((m + 32 * MMQ_TJ - 1) / (32 * MMQ_TJ)));
    hipStream_t st = amv_stream(stream);
    if (wtype == AMV_T_Q4_0) {
        if (sums) hipLaunchKernelGGL((k_mmq<AMV_T_Q4_0, true>), grid, dim3(256), 0, st, wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums);
        else hipLaunchKernelGGL((k_mmq<AMV_T_Q4_0, false>), grid, dim3(256), 0, st, wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums);
    } else {
        if (sums) hipLaunchKernelGGL((k_mmq<AMV_T_Q8_0, true>), grid, dim3(256), 0, st, wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums);
        else hipLaunchKernelGGL((k_mmq<AMV_T_Q8_0, false>), grid, dim3(256), 0, st, wq, wd, (int)n_rows, nb, aq, ameta, (int)m, dst, ldd, sums);
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
