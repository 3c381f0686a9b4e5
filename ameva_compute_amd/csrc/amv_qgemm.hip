// Prefill MUL_MAT (many tokens) on the int8 matrix cores of MI355X with ggml's exact block integers.
//
// Role of ameva_mmq.comp:55-163 / ameva_mmqb.comp:11-16, 54-157 (reference, enc_mul_mat_mmq ggml-ameva.cpp:2540-2647):
// dst[m][n] = sum over the blocks of row n of the f32 epilogue of one exact integer per block, as ggml's
// vec_dot_q4_0_q8_0 / q8_0_q8_0 / q4_K_q8_K compute it on the CPU:
//   Q4_0 / Q8_0 (32-blocks):  S = sum_k w_k q_k (w = q - 8 or q),           dst += S * d_a * d_w
//   Q4_K (256-blocks of 8 units of 32, 6-bit scales sc_u and mins m_u):
//                             I1 = sum_u sc_u sum_k q_k a_k, I2 = sum_u m_u sum_k a_k,
//                             dst += d_a * (d * I1 - dmin * I2)
// One v_mfma_i32_32x32x32_i8 is one 32-block (or one Q4_K unit) of a 32 x 32 tile, so S comes out of the matrix core
// as an int32, exact. The per-block epilogue is VALU work beside the matrix core: Q4_0 / Q8_0 take three operations
// per output and block (convert, scale by d_a, fma by d_w), Q4_K one integer multiply-add per unit (I1 += sc_u S_u)
// and four per super-block (I2 is one f16 MFMA of the units' mins against the activation sums per 16, exact in f32).
// The inputs are the plain activation layouts (int8 q with {f32 d, i32 sum} per 32, or Q8_K's f32 d per 256 and i32
// sums per 16): no f16 copies are read.
//
// Tiling: workgroup of 4 waves (2 x 2) on BM = 64 TT tokens x BN = 64 TW weight rows; wave (wt, ww) owns tokens
// 32 TT wt .. and rows 32 TW ww .. as TT x TW tiles of 32 x 32. MFMA operands: A = tokens, B = weight rows; lane l
// supplies token (row of A) / weight row (column of B) l % 32 and the 16 bytes 16 (l / 32) .. + 15 of the 32-block
// (any assignment of k to byte slots works as long as A and B share it); the result D of lane l holds weight row
// l % 32 and tokens 8 (r / 4) + 4 (l / 32) + r % 4, r = 0..15, so the weight scale of an output is one value per lane
// and the token scales are four float4 reads.
// Pipeline steps of 64 k (two 32-blocks, or one 32-byte Q4_K chunk = units 2c, 2c + 1): the global loads of step
// s + 1 are issued before step s computes from LDS; at staging the weights are expanded to int8 once per workgroup
// (Q4_0: n - 8 per byte with integer tricks, Q4_K: the unsigned nibbles) and the activations copied. LDS rows are
// 80 bytes (64 + 16 of padding): the 16-byte fragment reads of 32 consecutive rows hit distinct banks.
// The grid is one dimension, mapped so that the workgroups sharing a weight tile (its token tiles) are dispatched to
// the same XCD, one after another, and with a split of k each k range goes to its own group of XCDs (range z to
// XCDs 8 z / n_z ..): MI355X hands workgroup i to XCD i % 8, and each XCD has its own L2, so an XCD reads the weight
// rows of its tiles once and only its k range of the activation (on the 4096 x 14336 down shape at M = 512 with k
// split in two this cut the L2 -> memory reads from 118 to 70 MB per launch, at the same time).
#include "amv_common.h"

#include <algorithm>

typedef int qg_v4i __attribute__((ext_vector_type(4)));
typedef int qg_v16i __attribute__((ext_vector_type(16)));
typedef _Float16 qg_h8 __attribute__((ext_vector_type(8)));
typedef float qg_f16v __attribute__((ext_vector_type(16)));

#define QG_KS 64            // k per pipeline step
#define QG_LD (QG_KS + 16)  // LDS row stride in bytes

// byte-wise n - 8 of nibbles n in 0..15 (no carry crosses a byte: n + 0x78 <= 0x87)
__device__ __forceinline__ uint32_t qg_m8(uint32_t v) { return (v + 0x78787878u) ^ 0x80808080u; }


// ---------------------------------------------------------------------------------------------------------------
// Q4_0 / Q8_0
// ---------------------------------------------------------------------------------------------------------------
template <int WT>
struct QgRegs {  // one thread's share of a step: weight block (row t / 2, block t % 2), activation block (token t / 2)
    uint4 w0, w1;  // Q4_0: w0 = the 16 nibble bytes; Q8_0: the 32 bytes
    uint4 a0, a1;  // 32 int8 of the token's block
    uint32_t dw;   // the weight block's f16 scale bits
    float da;
    bool past;     // a block past the split's end: weight scale 0
};

template <int WT, int TT, int TW>
__device__ __forceinline__ QgRegs<WT> qg_load(int step, const uint8_t* __restrict__ wq,
                                        const uint16_t* __restrict__ wd, int N, int nb, int n0,
                                        const int8_t* __restrict__ aq, const int2* __restrict__ am, int M, int m0,
                                        int K, int b0, int b_end) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    const int t = threadIdx.x, blk = t & 1;
    const int b = b0 + 2 * step + blk, bc = min(b, b_end - 1);  // a block past the split's end: weight scale 0
    // the loaded values stay untouched until qg_store (any arithmetic on them here makes the compiler wait for the
    // whole prefetch at the load); the fields of a role the thread does not have are not read
    QgRegs<WT> s;
    s.past = b >= b_end;
    if (2 * BN >= 256 || t < 2 * BN) {  // (every thread of the 256 when BN = 128)
        const int row = min(n0 + (t >> 1), N - 1);
        const size_t bi = (size_t)row * nb + bc;
        if constexpr (WT == AMV_T_Q4_0) {
            s.w0 = *reinterpret_cast<const uint4*>(wq + bi * 16);
            s.dw = wd[amv_q4_0_didx(row, bc, nb, N)];
        } else {
            const uint4* p = reinterpret_cast<const uint4*>(wq + bi * 32);
            s.w0 = p[0];
            s.w1 = p[1];
            s.dw = wd[bi];
        }
    }
    if (2 * BM >= 256 || t < 2 * BM) {
        const int tok = min(m0 + (t >> 1), M - 1);
        const uint4* p = reinterpret_cast<const uint4*>(aq + (size_t)tok * K + 32 * bc);
        s.a0 = p[0];
        s.a1 = p[1];
        s.da = __int_as_float(am[(size_t)tok * nb + bc].x);
    }
    return s;
}

template <int WT, int TT, int TW>
__device__ __forceinline__ void qg_store(const QgRegs<WT>& s, int8_t* __restrict__ sW, int8_t* __restrict__ sA,
                                         float* __restrict__ sDw, float* __restrict__ sDa) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    const int t = threadIdx.x, blk = t & 1;
    if (t < 2 * BN) {
        uint4* d = reinterpret_cast<uint4*>(sW + (t >> 1) * QG_LD + 32 * blk);
        if constexpr (WT == AMV_T_Q4_0) {  // element e < 16: low nibble of byte e; 16 + e: its high nibble
            const uint4 x = s.w0;
            d[0] = make_uint4(qg_m8(x.x & 0x0F0F0F0Fu), qg_m8(x.y & 0x0F0F0F0Fu), qg_m8(x.z & 0x0F0F0F0Fu),
                              qg_m8(x.w & 0x0F0F0F0Fu));
            d[1] = make_uint4(qg_m8((x.x >> 4) & 0x0F0F0F0Fu), qg_m8((x.y >> 4) & 0x0F0F0F0Fu),
                              qg_m8((x.z >> 4) & 0x0F0F0F0Fu), qg_m8((x.w >> 4) & 0x0F0F0F0Fu));
        } else {
            d[0] = s.w0;
            d[1] = s.w1;
        }
        sDw[blk * BN + (t >> 1)] = s.past ? 0.0f : amv_h2f((uint16_t)s.dw);
    }
    if (t < 2 * BM) {
        uint4* d = reinterpret_cast<uint4*>(sA + (t >> 1) * QG_LD + 32 * blk);
        d[0] = s.a0;
        d[1] = s.a1;
        sDa[blk * BM + (t >> 1)] = s.da;
    }
}

template <int WT, bool SUMS, int TT, int TW, bool ADD = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_qgemm(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                              int N, int nb, const int8_t* __restrict__ aq,
                                              const int2* __restrict__ am, int M, float* __restrict__ dst,
                                              int64_t ldd, const float* add, int32_t* __restrict__ sums, int kb_per,
                                              int64_t zstride, int n_tw, int n_tt, int n_z) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    __shared__ __align__(16) int8_t sW[2][BN * QG_LD];
    __shared__ __align__(16) int8_t sA[2][BM * QG_LD];
    __shared__ __align__(16) float sDw[2][2 * BN];
    __shared__ __align__(16) float sDa[2][2 * BM];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wt = w & 1, ww = w >> 1, c = lane & 31, h = lane >> 5;
    // tile index: token tile fastest, then the split of k, then the weight tile
    const int T = amv_xcd_tile(blockIdx.x, n_tw * n_z * n_tt);  // token tiles, weight tiles, k ranges
    const int tt = T % n_tt, tw = (T / n_tt) % n_tw, z = T / (n_tt * n_tw);
    const int n0 = tw * BN, m0 = tt * BM;
    const int K = nb * 32;
    const int b0 = z * kb_per, b_end = min(nb, b0 + kb_per);
    const int nsteps = (b_end - b0 + 1) / 2;
    dst += (size_t)z * zstride;

    qg_f16v acc[TT][TW];
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // global loads run two steps ahead of the compute: the registers of step s + 2 are loaded while step s computes
    // and step s + 1's (loaded during step s - 1) go to LDS at its end
    QgRegs<WT> st0, st1;
    st0 = qg_load<WT, TT, TW>(0, wq, wd, N, nb, n0, aq, am, M, m0, K, b0, b_end);
    qg_store<WT, TT, TW>(st0, sW[0], sA[0], sDw[0], sDa[0]);
    st1 = qg_load<WT, TT, TW>(min(1, nsteps - 1), wq, wd, N, nb, n0, aq, am, M, m0, K, b0, b_end);
    __syncthreads();
    const auto compute = [&](int step) {
        const int buf = step & 1;
#pragma unroll 1
        for (int bl = 0; bl < 2; ++bl) {  // one block's MFMA results live at a time
            qg_v4i A[TT], B[TW];
#pragma unroll
            for (int i = 0; i < TT; ++i)
                A[i] = *reinterpret_cast<const qg_v4i*>(sA[buf] + (32 * (TT * wt + i) + c) * QG_LD + 32 * bl + 16 * h);
#pragma unroll
            for (int j = 0; j < TW; ++j)
                B[j] = *reinterpret_cast<const qg_v4i*>(sW[buf] + (32 * (TW * ww + j) + c) * QG_LD + 32 * bl + 16 * h);
            const int b = b0 + 2 * step + bl;
#pragma unroll
            for (int i = 0; i < TT; ++i) {
                const int tl = 32 * (TT * wt + i) + 4 * h;  // first token of the lane in this token tile
                float da[16];
                if constexpr (!SUMS) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v = *reinterpret_cast<const float4*>(&sDa[buf][bl * BM + tl + 8 * q]);
                        da[4 * q] = v.x;
                        da[4 * q + 1] = v.y;
                        da[4 * q + 2] = v.z;
                        da[4 * q + 3] = v.w;
                    }
                }
#pragma unroll
                for (int j = 0; j < TW; ++j) {
                    const qg_v16i zero = {};
                    const qg_v16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], B[j], zero, 0, 0, 0);
                    const int rl = 32 * (TW * ww + j) + c;  // the lane's weight row in the tile
                    if constexpr (SUMS) {
                        const int n = n0 + rl;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int m = m0 + tl + 8 * (r >> 2) + (r & 3);
                            if (b < b_end && m < M && n < N) sums[((size_t)m * N + n) * nb + b] = C[r];
                        }
                    } else {
                        const float dw = sDw[buf][bl * BN + rl];
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf((float)C[r], dw * da[r], acc[i][j][r]);
                    }
                }
            }
        }
    };
    // the prefetches are unconditional (past the last step they read the last step again) so that the wait before
    // each store covers only the registers it stores, not the prefetch issued after them
    for (int step = 0; step < nsteps; step += 2) {
        st0 = qg_load<WT, TT, TW>(min(step + 2, nsteps - 1), wq, wd, N, nb, n0, aq, am, M, m0, K, b0, b_end);
        compute(step);
        if (step + 1 >= nsteps) break;
        qg_store<WT, TT, TW>(st1, sW[1], sA[1], sDw[1], sDa[1]);
        __syncthreads();
        st1 = qg_load<WT, TT, TW>(min(step + 3, nsteps - 1), wq, wd, N, nb, n0, aq, am, M, m0, K, b0, b_end);
        compute(step + 1);
        if (step + 2 >= nsteps) break;
        qg_store<WT, TT, TW>(st0, sW[0], sA[0], sDw[0], sDa[0]);
        __syncthreads();
    }
    if constexpr (!SUMS) {
        // lane: weight row n, tokens 8 (r / 4) + 4 h + r % 4: for each r the 32 lanes of a half store 32 consecutive
        // floats of one token row
#pragma unroll
        for (int j = 0; j < TW; ++j) {
            const int n = n0 + 32 * (TW * ww + j) + c;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < TT; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + 32 * (TT * wt + i) + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (m < M) {
                        const size_t o = (size_t)m * ldd + n;
                        if constexpr (ADD) dst[o] = acc[i][j][r] + add[o];
                        else dst[o] = acc[i][j][r];
                    }
                }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Q4_K x Q8_K. Step = chunk c (0..3) of super-block j: the 32 qs bytes whose low nibbles are unit 2c and high nibbles
// unit 2c + 1. Per super-block values (unit scales and mins, d, dmin, the activation sums per 16 and d_a) are staged
// at its chunk 0 into a slot of their own, double-buffered by super-block parity.
// ---------------------------------------------------------------------------------------------------------------
struct QgKRegs {
    uint4 q;       // weight bytes 16 hf .. + 15 of the chunk (row t / 2, hf = t % 2)
    uint4 hd;      // the row's 16-byte head (d, dmin, 12 scale bytes), at chunk 0
    uint4 a0, a1;  // 32 activation int8 (token t / 2, k 64 c + 32 hf ..)
    int s[8];      // at chunk 0: the token's sums per 16, 8 hf .. 8 hf + 7
    float da;      // at chunk 0: the token's super-block scale
};

template <int TT, int TW>
__device__ __forceinline__ void qgk_load(QgKRegs& s, int step, const uint4* __restrict__ wq,
                                         const uint4* __restrict__ wh, int N, int nsb, int n0,
                                         const int8_t* __restrict__ aq, const float* __restrict__ ad,
                                         const int32_t* __restrict__ as16, int M, int m0, int K, int sb0) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    const int t = threadIdx.x, hf = t & 1;
    const int j = sb0 + (step >> 2), c = step & 3;
    if (t < 2 * BN) {
        const int row = min(n0 + (t >> 1), N - 1);
        const size_t sb = (size_t)row * nsb + j;
        s.q = wq[sb * 8 + 2 * c + hf];
        if (c == 0) s.hd = wh[sb];
    }
    if (t < 2 * BM) {
        const int tok = min(m0 + (t >> 1), M - 1);
        const uint4* p = reinterpret_cast<const uint4*>(aq + (size_t)tok * K + 256 * j + 64 * c + 32 * hf);
        s.a0 = p[0];
        s.a1 = p[1];
        if (c == 0) {
            const int32_t* q = as16 + (size_t)tok * (K / 16) + 16 * j + 8 * hf;  // 4-byte aligned only
#pragma unroll
            for (int e = 0; e < 8; ++e) s.s[e] = q[e];
            s.da = ad[(size_t)tok * nsb + j];
        }
    }
}

__device__ __forceinline__ uint32_t qg_h2(int a, int b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)b) << 16);
}

template <int TT, int TW>
__device__ __forceinline__ void qgk_store(const QgKRegs& s, int step, int8_t* __restrict__ sW,
                                          int8_t* __restrict__ sA, uint8_t* __restrict__ sSc,
                                          float* __restrict__ sD, float* __restrict__ sDm, uint16_t* __restrict__ sMn,
                                          uint16_t* __restrict__ sBs, float* __restrict__ sDa) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    const int t = threadIdx.x, hf = t & 1, c = step & 3;
    if (t < 2 * BN) {
        const int rl = t >> 1;
        uint4* d = reinterpret_cast<uint4*>(sW + rl * QG_LD);
        const uint4 x = s.q;  // unit 2c: low nibbles (elements 16 hf ..), unit 2c + 1: high nibbles
        d[hf] = make_uint4(x.x & 0x0F0F0F0Fu, x.y & 0x0F0F0F0Fu, x.z & 0x0F0F0F0Fu, x.w & 0x0F0F0F0Fu);
        d[2 + hf] = make_uint4((x.x >> 4) & 0x0F0F0F0Fu, (x.y >> 4) & 0x0F0F0F0Fu, (x.z >> 4) & 0x0F0F0F0Fu,
                               (x.w >> 4) & 0x0F0F0F0Fu);
        if (c == 0) {  // units 4 hf .. 4 hf + 3: scales (bytes) and mins (f16, on the two 16-sum slots of each unit)
            uint32_t mm[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                int sc, mn;
                k4_scale_min(4 * hf + e, s.hd.y, s.hd.z, s.hd.w, sc, mn);
                sSc[(4 * hf + e) * BN + rl] = (uint8_t)sc;
                mm[e] = qg_h2(mn, mn);
            }
            *reinterpret_cast<uint4*>(sMn + rl * 16 + 8 * hf) = make_uint4(mm[0], mm[1], mm[2], mm[3]);
            if (hf == 0) {
                sD[rl] = amv_h2f(s.hd.x);
                sDm[rl] = amv_h2f(s.hd.x >> 16);
            }
        }
    }
    if (t < 2 * BM) {
        const int tl = t >> 1;
        uint4* d = reinterpret_cast<uint4*>(sA + tl * QG_LD + 32 * hf);
        d[0] = s.a0;
        d[1] = s.a1;
        if (c == 0) {  // the 16-sums as f16 (|sum| <= 2032: exact)
            *reinterpret_cast<uint4*>(sBs + tl * 16 + 8 * hf) =
                make_uint4(qg_h2(s.s[0], s.s[1]), qg_h2(s.s[2], s.s[3]), qg_h2(s.s[4], s.s[5]), qg_h2(s.s[6], s.s[7]));
            if (hf == 0) sDa[tl] = s.da;
        }
    }
}

template <bool SUMS, int TT, int TW, bool ADD = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_qgemm_q4k(const uint4* __restrict__ wq, const uint4* __restrict__ wh, int N,
                                                  int nsb, const int8_t* __restrict__ aq, const float* __restrict__ ad,
                                                  const int32_t* __restrict__ as16, int M, float* __restrict__ dst,
                                                  int64_t ldd, const float* add, int32_t* __restrict__ sums, int sb_per,
                                                  int64_t zstride, int n_tw, int n_tt, int n_z) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    __shared__ __align__(16) int8_t sW[2][BN * QG_LD];
    __shared__ __align__(16) int8_t sA[2][BM * QG_LD];
    __shared__ __align__(16) uint8_t sSc[2][8 * BN];
    __shared__ __align__(16) float sD[2][BN], sDm[2][BN], sDa[2][BM];
    __shared__ __align__(16) uint16_t sMn[2][BN * 16], sBs[2][BM * 16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wt = w & 1, ww = w >> 1, c32 = lane & 31, h = lane >> 5;
    const int T = amv_xcd_tile(blockIdx.x, n_tw * n_z * n_tt);  // token tiles, weight tiles, k ranges
    const int tt = T % n_tt, tw = (T / n_tt) % n_tw, z = T / (n_tt * n_tw);
    const int n0 = tw * BN, m0 = tt * BM;
    const int K = nsb * 256;
    const int sb0 = z * sb_per, sb_end = min(nsb, sb0 + sb_per);
    const int nsteps = (sb_end - sb0) * 4;
    dst += (size_t)z * zstride;

    qg_f16v acc[TT][TW];
    qg_v16i I1[TT][TW];
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = 0.0f;
                I1[i][j][r] = 0;
            }

    QgKRegs st;
    qgk_load<TT, TW>(st, 0, wq, wh, N, nsb, n0, aq, ad, as16, M, m0, K, sb0);
    qgk_store<TT, TW>(st, 0, sW[0], sA[0], sSc[0], sD[0], sDm[0], sMn[0], sBs[0], sDa[0]);
    __syncthreads();
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1, j = sb0 + (step >> 2), c = step & 3, jp = (step >> 2) & 1;
        if (step + 1 < nsteps) qgk_load<TT, TW>(st, step + 1, wq, wh, N, nsb, n0, aq, ad, as16, M, m0, K, sb0);
#pragma unroll
        for (int u = 0; u < 2; ++u) {  // unit 2c + u
            qg_v4i A[TT], B[TW];
            int sc[TW];
#pragma unroll
            for (int i = 0; i < TT; ++i)
                A[i] = *reinterpret_cast<const qg_v4i*>(sA[buf] + (32 * (TT * wt + i) + c32) * QG_LD + 32 * u + 16 * h);
#pragma unroll
            for (int jj = 0; jj < TW; ++jj) {
                const int rl = 32 * (TW * ww + jj) + c32;
                B[jj] = *reinterpret_cast<const qg_v4i*>(sW[buf] + rl * QG_LD + 32 * u + 16 * h);
                sc[jj] = sSc[jp][(2 * c + u) * BN + rl];
            }
#pragma unroll
            for (int i = 0; i < TT; ++i)
#pragma unroll
                for (int jj = 0; jj < TW; ++jj) {
                    const qg_v16i zero = {};
                    const qg_v16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], B[jj], zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) I1[i][jj][r] += __mul24(C[r], sc[jj]);
                }
        }
        if (c == 3) {  // end of super-block j: I2 (mins against the 16-sums) and the f32 epilogue
#pragma unroll
            for (int i = 0; i < TT; ++i) {
                const int tl = 32 * (TT * wt + i) + 4 * h;
                const qg_h8 Abs = *reinterpret_cast<const qg_h8*>(sBs[jp] + (32 * (TT * wt + i) + c32) * 16 + 8 * h);
                float da[16];
                if constexpr (!SUMS) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v = *reinterpret_cast<const float4*>(&sDa[jp][tl + 8 * q]);
                        da[4 * q] = v.x;
                        da[4 * q + 1] = v.y;
                        da[4 * q + 2] = v.z;
                        da[4 * q + 3] = v.w;
                    }
                }
#pragma unroll
                for (int jj = 0; jj < TW; ++jj) {
                    const int rl = 32 * (TW * ww + jj) + c32;
                    const qg_h8 Bmn = *reinterpret_cast<const qg_h8*>(sMn[jp] + rl * 16 + 8 * h);
                    const qg_f16v zf = {};
                    const qg_f16v I2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(Abs, Bmn, zf, 0, 0, 0);
                    if constexpr (SUMS) {
                        const int n = n0 + rl;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int m = m0 + tl + 8 * (r >> 2) + (r & 3);
                            if (m < M && n < N) {
                                int32_t* o = sums + (((size_t)m * N + n) * nsb + j) * 2;
                                o[0] = I1[i][jj][r];
                                o[1] = (int)I2[r];
                            }
                        }
                    } else {
                        const float d = sD[jp][rl], dm = sDm[jp][rl];
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[i][jj][r] = fmaf(fmaf(d, (float)I1[i][jj][r], -(dm * I2[r])), da[r], acc[i][jj][r]);
                    }
#pragma unroll
                    for (int r = 0; r < 16; ++r) I1[i][jj][r] = 0;
                }
            }
        }
        if (step + 1 < nsteps) {
            const int sp = ((step + 1) >> 2) & 1;
            qgk_store<TT, TW>(st, step + 1, sW[buf ^ 1], sA[buf ^ 1], sSc[sp], sD[sp], sDm[sp], sMn[sp], sBs[sp],
                              sDa[sp]);
            __syncthreads();
        }
    }
    if constexpr (!SUMS) {
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const int n = n0 + 32 * (TW * ww + jj) + c32;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < TT; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + 32 * (TT * wt + i) + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (m < M) {
                        const size_t o = (size_t)m * ldd + n;
                        if constexpr (ADD) dst[o] = acc[i][jj][r] + add[o];
                        else dst[o] = acc[i][jj][r];
                    }
                }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Q6_K x Q8_K (reference vec_dot_q6_K_q8_K; ameva_qdecode.glsl:246-258 for the element layout). A super-block of 256
// is 16 sub-blocks of 16 consecutive elements with int8 scales sc_s and one f16 d: I = sum_s sc_s sum_k q_k a_k with
// q = (4 low bits from ql | 2 high bits from qh) - 32, dst += d_a d I. The sub-blocks are 16 long, so the matrix core
// runs v_mfma_i32_32x32x16_i8 (lane half h supplies 8 of the 16 bytes) and I accumulates sc_s C_s in integers. Step =
// one 128-element half n of the super-block: ql bytes 64 n .. + 63 and qh bytes 32 n .. + 31 give elements
// 128 n + {l, 32 + l, 64 + l, 96 + l} (l < 32) from ql[l] low / ql[32 + l] low / ql[l] high / ql[32 + l] high nibbles
// and qh[l] bits 0-1 / 2-3 / 4-5 / 6-7.
// ---------------------------------------------------------------------------------------------------------------
typedef long qg_i64;

#define QG6_LD (128 + 16)  // LDS row stride (bytes) of the 128-element steps

struct QgQ6Regs {
    uint4 l0, l1, qh;  // ql[16 hf ..], ql[32 + 16 hf ..], qh[16 hf ..] of the half (row t / 2, hf = t % 2)
    uint4 a0, a1, a2, a3;  // 64 activation int8 (token t / 2, elements 128 c + 64 hf ..)
    uint4 sc;          // at half 0: the row's 16 scales
    uint32_t d;        // at half 0: f16 d
    float da;          // at half 0: the token's d
};

template <int TT, int TW>
__device__ __forceinline__ void qg6_load(QgQ6Regs& s, int step, const uint4* __restrict__ wl,
                                         const uint4* __restrict__ wqh, const uint4* __restrict__ wsc,
                                         const uint16_t* __restrict__ wd, int N, int nsb, int n0,
                                         const int8_t* __restrict__ aq, const float* __restrict__ ad, int M, int m0,
                                         int K, int sb0) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    const int t = threadIdx.x, hf = t & 1;
    const int j = sb0 + (step >> 1), c = step & 1;
    if (t < 2 * BN) {
        const int row = min(n0 + (t >> 1), N - 1);
        const size_t sb = (size_t)row * nsb + j;
        s.l0 = wl[sb * 8 + 4 * c + hf];      // ql bytes 64 c + 16 hf
        s.l1 = wl[sb * 8 + 4 * c + 2 + hf];  // ql bytes 64 c + 32 + 16 hf
        s.qh = wqh[sb * 4 + 2 * c + hf];     // qh bytes 32 c + 16 hf
        if (c == 0) {
            s.sc = wsc[sb];
            s.d = wd[sb];
        }
    }
    if (t < 2 * BM) {
        const int tok = min(m0 + (t >> 1), M - 1);
        const uint4* p = reinterpret_cast<const uint4*>(aq + (size_t)tok * K + 256 * j + 128 * c + 64 * hf);
        s.a0 = p[0];
        s.a1 = p[1];
        s.a2 = p[2];
        s.a3 = p[3];
        if (c == 0) s.da = ad[(size_t)tok * nsb + j];
    }
}

// 4 bytes of ql nibbles n (already selected) and their 2 high bits hb (already at bit 4..5): n | hb - 32 per byte
__device__ __forceinline__ uint32_t qg6_q(uint32_t n, uint32_t hb) { return ((n | hb) + 0x60606060u) ^ 0x80808080u; }

template <int TT, int TW>
__device__ __forceinline__ void qg6_store(const QgQ6Regs& s, int step, int8_t* __restrict__ sW,
                                          int8_t* __restrict__ sA, int8_t* __restrict__ sSc, float* __restrict__ sD,
                                          float* __restrict__ sDa) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    const int t = threadIdx.x, hf = t & 1, c = step & 1;
    if (t < 2 * BN) {
        const int rl = t >> 1;
        uint4* d = reinterpret_cast<uint4*>(sW + rl * QG6_LD);
        const uint32_t L0[4] = {s.l0.x, s.l0.y, s.l0.z, s.l0.w}, L1[4] = {s.l1.x, s.l1.y, s.l1.z, s.l1.w};
        const uint32_t H[4] = {s.qh.x, s.qh.y, s.qh.z, s.qh.w};
        uint32_t q1[4], q2[4], q3[4], q4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q1[i] = qg6_q(L0[i] & 0x0F0F0F0Fu, (H[i] & 0x03030303u) << 4);
            q2[i] = qg6_q(L1[i] & 0x0F0F0F0Fu, (H[i] & 0x0C0C0C0Cu) << 2);
            q3[i] = qg6_q((L0[i] >> 4) & 0x0F0F0F0Fu, H[i] & 0x30303030u);
            q4[i] = qg6_q((L1[i] >> 4) & 0x0F0F0F0Fu, (H[i] >> 2) & 0x30303030u);
        }
        d[hf] = make_uint4(q1[0], q1[1], q1[2], q1[3]);      // elements 16 hf ..
        d[2 + hf] = make_uint4(q2[0], q2[1], q2[2], q2[3]);  // 32 + 16 hf ..
        d[4 + hf] = make_uint4(q3[0], q3[1], q3[2], q3[3]);  // 64 + 16 hf ..
        d[6 + hf] = make_uint4(q4[0], q4[1], q4[2], q4[3]);  // 96 + 16 hf ..
        if (c == 0) {  // scales of sub-blocks 8 hf .. 8 hf + 7 (bytes), d
            const uint32_t sw[2] = {hf ? s.sc.z : s.sc.x, hf ? s.sc.w : s.sc.y};
#pragma unroll
            for (int e = 0; e < 8; ++e) sSc[(8 * hf + e) * BN + rl] = (int8_t)((sw[e >> 2] >> (8 * (e & 3))) & 0xFFu);
            if (hf == 0) sD[rl] = amv_h2f(s.d);
        }
    }
    if (t < 2 * BM) {
        const int tl = t >> 1;
        uint4* d = reinterpret_cast<uint4*>(sA + tl * QG6_LD + 64 * hf);
        d[0] = s.a0;
        d[1] = s.a1;
        d[2] = s.a2;
        d[3] = s.a3;
        if (c == 0 && hf == 0) sDa[tl] = s.da;
    }
}

template <bool SUMS, int TT, int TW, bool ADD = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_qgemm_q6k(
    const uint4* __restrict__ wl, const uint4* __restrict__ wqh, const uint4* __restrict__ wsc,
    const uint16_t* __restrict__ wd, int N, int nsb, const int8_t* __restrict__ aq, const float* __restrict__ ad, int M,
    float* __restrict__ dst, int64_t ldd, const float* add, int32_t* __restrict__ sums, int sb_per, int64_t zstride, int n_tw, int n_tt,
    int n_z) {
    constexpr int BN = 64 * TW, BM = 64 * TT;
    __shared__ __align__(16) int8_t sW[2][BN * QG6_LD];
    __shared__ __align__(16) int8_t sA[2][BM * QG6_LD];
    __shared__ __align__(16) int8_t sSc[2][16 * BN];
    __shared__ __align__(16) float sD[2][BN], sDa[2][BM];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wt = w & 1, ww = w >> 1, c32 = lane & 31, h = lane >> 5;
    const int T = amv_xcd_tile(blockIdx.x, n_tw * n_z * n_tt);  // token tiles, weight tiles, k ranges
    const int tt = T % n_tt, tw = (T / n_tt) % n_tw, z = T / (n_tt * n_tw);
    const int n0 = tw * BN, m0 = tt * BM;
    const int K = nsb * 256;
    const int sb0 = z * sb_per, sb_end = min(nsb, sb0 + sb_per);
    const int nsteps = (sb_end - sb0) * 2;
    dst += (size_t)z * zstride;

    qg_f16v acc[TT][TW];
    qg_v16i I[TT][TW];
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = 0.0f;
                I[i][j][r] = 0;
            }

    QgQ6Regs st;
    qg6_load<TT, TW>(st, 0, wl, wqh, wsc, wd, N, nsb, n0, aq, ad, M, m0, K, sb0);
    qg6_store<TT, TW>(st, 0, sW[0], sA[0], sSc[0], sD[0], sDa[0]);
    __syncthreads();
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1, j = sb0 + (step >> 1), c = step & 1, jp = (step >> 1) & 1;
        if (step + 1 < nsteps) qg6_load<TT, TW>(st, step + 1, wl, wqh, wsc, wd, N, nsb, n0, aq, ad, M, m0, K, sb0);
#pragma unroll 2
        for (int u = 0; u < 8; ++u) {  // sub-block 8 c + u
            qg_i64 A[TT], B[TW];
            int sc[TW];
#pragma unroll
            for (int i = 0; i < TT; ++i)
                A[i] = *reinterpret_cast<const qg_i64*>(sA[buf] + (32 * (TT * wt + i) + c32) * QG6_LD + 16 * u + 8 * h);
#pragma unroll
            for (int jj = 0; jj < TW; ++jj) {
                const int rl = 32 * (TW * ww + jj) + c32;
                B[jj] = *reinterpret_cast<const qg_i64*>(sW[buf] + rl * QG6_LD + 16 * u + 8 * h);
                sc[jj] = sSc[jp][(8 * c + u) * BN + rl];
            }
#pragma unroll
            for (int i = 0; i < TT; ++i)
#pragma unroll
                for (int jj = 0; jj < TW; ++jj) {
                    const qg_v16i zero = {};
                    const qg_v16i C = __builtin_amdgcn_mfma_i32_32x32x16_i8(A[i], B[jj], zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) I[i][jj][r] += __mul24(C[r], sc[jj]);
                }
        }
        if (c == 1) {  // end of super-block j
#pragma unroll
            for (int i = 0; i < TT; ++i) {
                const int tl = 32 * (TT * wt + i) + 4 * h;
                float da[16];
                if constexpr (!SUMS) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v = *reinterpret_cast<const float4*>(&sDa[jp][tl + 8 * q]);
                        da[4 * q] = v.x;
                        da[4 * q + 1] = v.y;
                        da[4 * q + 2] = v.z;
                        da[4 * q + 3] = v.w;
                    }
                }
#pragma unroll
                for (int jj = 0; jj < TW; ++jj) {
                    const int rl = 32 * (TW * ww + jj) + c32;
                    if constexpr (SUMS) {
                        const int n = n0 + rl;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int m = m0 + tl + 8 * (r >> 2) + (r & 3);
                            if (m < M && n < N) sums[((size_t)m * N + n) * nsb + j] = I[i][jj][r];
                        }
                    } else {
                        const float d = sD[jp][rl];
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][jj][r] = fmaf(d * da[r], (float)I[i][jj][r], acc[i][jj][r]);
                    }
#pragma unroll
                    for (int r = 0; r < 16; ++r) I[i][jj][r] = 0;
                }
            }
        }
        if (step + 1 < nsteps) {
            const int sp = ((step + 1) >> 1) & 1;
            qg6_store<TT, TW>(st, step + 1, sW[buf ^ 1], sA[buf ^ 1], sSc[sp], sD[sp], sDa[sp]);
            __syncthreads();
        }
    }
    if constexpr (!SUMS) {
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const int n = n0 + 32 * (TW * ww + jj) + c32;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < TT; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + 32 * (TT * wt + i) + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (m < M) {
                        const size_t o = (size_t)m * ldd + n;
                        if constexpr (ADD) dst[o] = acc[i][jj][r] + add[o];
                        else dst[o] = acc[i][jj][r];
                    }
                }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------------------------------------------
// split of k shared with the f16 kernels (amv_mmq16.hip): workspace per device and the in-order partial sum
float* amv_splitk_workspace(size_t bytes, hipStream_t st);
int amv_splitk_count(int64_t tiles, int steps);
void amv_splitk_reduce(const float* part, int S, int64_t zstride, int64_t m, int64_t n, float* dst, int64_t ldd,
                       hipStream_t st, const float* add = nullptr);

template <int TT, int TW>
static int qgemm_launch(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
                         int64_t ldd, int32_t* sums, hipStream_t st, const float* add) {
    constexpr int BM = 64 * TT, BN = 64 * TW;
    const int8_t* aq = (const int8_t*)act;
    const int n_tw = (int)((n_rows + BN - 1) / BN), n_tt = (int)((m + BM - 1) / BM);
    const int64_t tiles = (int64_t)n_tw * n_tt;
    const bool q4k = wtype == AMV_T_Q4_K, q6k = wtype == AMV_T_Q6_K, kq = q4k || q6k;
    const int nb = (int)(k / 32), nsb = (int)(k / 256);
    const int steps = q4k ? 4 * nsb : q6k ? 4 * nsb : (nb + 1) / 2;  // in units of 64 k
    // split of k when the tiles leave CUs idle (partials in the library's workspace, summed in order of k)
    int S = sums ? 1 : amv_splitk_count(tiles, steps);
    int per = kq ? nsb : nb;
    float* out = dst;
    int64_t ldo = ldd, zstride = 0;
    if (S > 1) {
        per = kq ? (nsb + S - 1) / S : (((nb + S - 1) / S + 1) & ~1);
        S = kq ? (nsb + per - 1) / per : (nb + per - 1) / per;
        float* ws = S > 1 ? amv_splitk_workspace((size_t)S * m * n_rows * 4, st) : nullptr;
        if (S > 1 && !ws) return AMV_ERR_HIP;  // never unsplit: the summation order would change
        if (ws) {
            out = ws;
            ldo = n_rows;
            zstride = m * n_rows;
        } else {
            S = 1;
            per = kq ? nsb : nb;
        }
    }
    const dim3 grid((unsigned)(tiles * S));
    const float* kadd = S > 1 ? nullptr : add;  // with a split of k the residual joins in the sum of the partials
    if (q6k) {  // ql [n][nsb][128] | qh [n][nsb][64] | scales [n][nsb][16] | d [n][nsb]
        const int64_t nblk = n_rows * nsb;
        const uint8_t* base = (const uint8_t*)w;
        const uint4* wl = (const uint4*)base;
        const uint4* wqh = (const uint4*)(base + nblk * 128);
        const uint4* wsc = (const uint4*)(base + nblk * 192);
        const uint16_t* wd = (const uint16_t*)(base + nblk * 208);
        const float* ad = (const float*)(aq + m * k);
        if (sums)
            hipLaunchKernelGGL((k_qgemm_q6k<true, TT, TW>), grid, dim3(256), 0, st, wl, wqh, wsc, wd, (int)n_rows, nsb,
                               aq, ad, (int)m, out, ldo, kadd, sums, per, zstride, n_tw, n_tt, S);
        else if (kadd)
            hipLaunchKernelGGL((k_qgemm_q6k<false, TT, TW, true>), grid, dim3(256), 0, st, wl, wqh, wsc, wd,
                               (int)n_rows, nsb, aq, ad, (int)m, out, ldo, kadd, sums, per, zstride, n_tw, n_tt, S);
        else
            hipLaunchKernelGGL((k_qgemm_q6k<false, TT, TW>), grid, dim3(256), 0, st, wl, wqh, wsc, wd, (int)n_rows,
                               nsb, aq, ad, (int)m, out, ldo, kadd, sums, per, zstride, n_tw, n_tt, S);
    } else if (q4k) {
        const int64_t nblk = n_rows * nsb;
        const uint4* wq = (const uint4*)w;
        const uint4* wh = (const uint4*)((const uint8_t*)w + nblk * 128);
        const float* ad = (const float*)(aq + m * k);
        const int32_t* as16 = (const int32_t*)(aq + m * k + m * nsb * 4);
        if (sums)
            hipLaunchKernelGGL((k_qgemm_q4k<true, TT, TW>), grid, dim3(256), 0, st, wq, wh, (int)n_rows, nsb, aq, ad,
                               as16, (int)m, out, ldo, kadd, sums, per, zstride, n_tw, n_tt, S);
        else if (kadd)
            hipLaunchKernelGGL((k_qgemm_q4k<false, TT, TW, true>), grid, dim3(256), 0, st, wq, wh, (int)n_rows, nsb,
                               aq, ad, as16, (int)m, out, ldo, kadd, sums, per, zstride, n_tw, n_tt, S);
        else
            hipLaunchKernelGGL((k_qgemm_q4k<false, TT, TW>), grid, dim3(256), 0, st, wq, wh, (int)n_rows, nsb, aq, ad,
                               as16, (int)m, out, ldo, kadd, sums, per, zstride, n_tw, n_tt, S);
    } else {
        const int64_t nblk = n_rows * nb;
        const uint8_t* wq = (const uint8_t*)w;
        const uint16_t* wd = (const uint16_t*)(wq + nblk * (wtype == AMV_T_Q4_0 ? 16 : 32));
        const int2* am = (const int2*)(aq + m * k);
#define QG_LAUNCH(WT, SU, AD)                                                                                     \
    hipLaunchKernelGGL((k_qgemm<WT, SU, TT, TW, AD>), grid, dim3(256), 0, st, wq, wd, (int)n_rows, nb, aq, am, (int)m, \
                       out, ldo, kadd, sums, per, zstride, n_tw, n_tt, S)
        if (wtype == AMV_T_Q4_0) {
            if (sums) QG_LAUNCH(AMV_T_Q4_0, true, false);
            else if (kadd) QG_LAUNCH(AMV_T_Q4_0, false, true);
            else QG_LAUNCH(AMV_T_Q4_0, false, false);
        } else {
            if (sums) QG_LAUNCH(AMV_T_Q8_0, true, false);
            else if (kadd) QG_LAUNCH(AMV_T_Q8_0, false, true);
            else QG_LAUNCH(AMV_T_Q8_0, false, false);
        }
#undef QG_LAUNCH
    }
    if (S > 1) amv_splitk_reduce(out, S, zstride, m, n_rows, dst, ldd, st, add);
    return AMV_OK;
}

// Q4_0 / Q8_0 weights with plain Q8_0 activations (int8 [m][k], {f32 d, i32 sum} [m][k/32]); Q4_K weights with plain
// Q8_K activations (int8 [m][k], f32 d [m][k/256], i32 sums per 16 [m][k/16]). The prefixes of the MMA / DEQ layouts
// are these layouts. Tile: 128 x 128 while that gives at least 384 workgroups (1.5 per CU), else 64 x 64 (a split
// of k then fills the GPU where the tiles alone cannot). Measured on MI355X (Q4_K, exact): 14336 x 4096 at 512
// tokens 104 us with 128 x 128 against 115 us with 64 x 64; 6144 x 4096 at 512 tokens 55 us with 64 x 64 against
// 65 us (64 x 128) and 76 us (128 x 128); 14336 x 4096 at 128 tokens 47 us with 64 x 64 against 52 and 75 us.
int amv_qgemm(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
              int64_t ldd, int32_t* sums, hipStream_t st, const float* add) {
    const auto tiles = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n_rows + bn - 1) / bn); };
    const int rc = tiles(128, 128) >= 384 ? qgemm_launch<2, 2>(wtype, w, n_rows, k, act, m, dst, ldd, sums, st, add)
                                          : qgemm_launch<1, 1>(wtype, w, n_rows, k, act, m, dst, ldd, sums, st, add);
    if (rc) return rc;
    return amv_check_launch("amv_mul_mat_q_act");
}
