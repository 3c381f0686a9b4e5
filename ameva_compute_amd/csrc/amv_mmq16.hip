// Prefill MUL_MAT for Q4_0 / Q8_0 weights on the f16 matrix cores of MI355X, with exact integer block sums.
//
// Role of ameva_mmq.comp / ameva_mmqb.comp (reference, enc_mul_mat_mmq ggml-ameva.cpp:2540-2647): dst[m][n] =
// sum_b d_w[n][b] d_a[m][b] S[m][n][b], S the int32 dot of block b (ggml's vec_dot_q4_0_q8_0 / q8_0_q8_0 sumi).
// The operands of S are small integers, exact in f16: the weight (q - 8 for Q4_0, q for Q8_0) and the activation
// q_a (|q_a| <= 127); a block's 32 products sum to |S| <= 32 * 128 * 127 < 2^24, so v_mfma_f32_32x32x16_f16 (two per
// block) returns S exactly in f32. The f32 epilogue per output and block is then two VALU operations,
// t = S * d_w, acc = fma(t, d_a, acc), against three for int8 MFMA (convert, scale product, fma) -- on MI355X the
// epilogue, not the matrix core, bounds a kernel with a scale per 32 products, and the f16 rate keeps pace with it.
//
// DEQ variant (activations AMV_ACT_Q8_0_DEQ): the weights are staged as f16 (q - 8) d_w (Q4_0) or q d_w (Q8_0) and the
// activations arrive as f16 q_a d_a, so the matrix core accumulates across all of k with no per-block epilogue. Each
// operand is rounded to f16 once (relative 2^-11), so the f32 result is within ~3e-4 relative L2 of the exact-sum
// form instead of bit-identical to it; the block sums (SUMS) always use the exact form.
// Workgroup of 4 waves (2 x 2) on a tile of 64 TN weight rows x 64 TM tokens; wave (wr, wc) owns rows
// 32 TN wr .. + 32 TN and tokens 32 TM wc .. + 32 TM as TN x TM tiles of 32 x 32. Pipeline steps of 2 blocks (64 k): the
// global loads of step s + 1 are issued before step s computes from LDS; at staging the weights are converted to f16
// once per workgroup (shared by its 64 TM tokens) and the activations (already f16 copies, AMV_ACT_Q8_0_MMA) and both
// scale vectors are copied. MFMA operand layout (32x32x16 f16): lane l supplies A row l % 32 and B column l % 32 with
// 8 halves k = 8 (l / 32) .. + 7 of the 16-k step; it receives D column l % 32 (a token), rows
// 8 (r / 4) + 4 (l / 32) + r % 4, r = 0..15.
#include "amv_common.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

typedef _Float16 g16_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 g16_h2 __attribute__((ext_vector_type(2)));
typedef float g16_f16v __attribute__((ext_vector_type(16)));

#define G16_KS 64                // k per pipeline step (2 blocks)
#define G16_LDK (G16_KS + 8)     // LDS row in halves, padded by 16 B against bank conflicts

// 4 bytes of nibbles (low or high half already selected and masked) -> 4 halves (n - off) as two f16 pairs
__device__ __forceinline__ uint2 g16_nib4(uint32_t x, g16_h2 off) {
    const uint32_t m64 = 0x64646464u;
    const g16_h2 p0 = __builtin_bit_cast(g16_h2, __builtin_amdgcn_perm(x, m64, 0x00050004u)) - off;
    const g16_h2 p1 = __builtin_bit_cast(g16_h2, __builtin_amdgcn_perm(x, m64, 0x00070006u)) - off;
    return make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
}

// the two f16 pairs of v scaled by s (one rounding each)
__device__ __forceinline__ uint2 g16_scale2(uint2 v, g16_h2 sc) {
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_bit_cast(g16_h2, v.x) * sc),
                      __builtin_bit_cast(uint32_t, __builtin_bit_cast(g16_h2, v.y) * sc));
}

// Registers of one staging step: thread t < 2 BN stages (row t / 2, block t % 2) of the weights (sw) and its scale
// (sdw); every thread stages 64 bytes of one token's activations (token t / 2, block t % 2, sa) and one activation
// scale (sda). Plain arrays (a struct of them was placed in scratch by the compiler).
#define G16_NW(WT) ((WT) == AMV_T_Q4_0 ? 1 : 2)

template <int WT, int TN, int TM>
__device__ __forceinline__ void g16_load(uint4 (&sw)[G16_NW(WT)], float& sdw, uint4& sa0, uint4& sa1, uint4& sa2,
                                         uint4& sa3, float& sda, int step, const uint8_t* __restrict__ wq,
                                         const uint16_t* __restrict__ wd, int N, int nb, int n0,
                                         const uint16_t* __restrict__ a16, const float* __restrict__ dT, int M, int m0,
                                         int K, int b0, int b_end) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    const int t = threadIdx.x;
    const int blk = t & 1;
    // blocks b0 .. b_end - 1 of the row (a split of k); a block past the end reads the last one, scale 0
    const int b = b0 + 2 * step + blk, bc = min(b, b_end - 1);
    if (t < 2 * BN) {
        const int row = min(n0 + (t >> 1), N - 1);
        const size_t bi = (size_t)row * nb + bc;
        if constexpr (WT == AMV_T_Q4_0) {
            sw[0] = *reinterpret_cast<const uint4*>(wq + bi * 16);
            sdw = b < b_end ? amv_h2f(wd[amv_q4_0_didx(row, bc, nb, N)]) : 0.0f;
        } else {
            sw[0] = *reinterpret_cast<const uint4*>(wq + bi * 32);
            sw[G16_NW(WT) - 1] = *reinterpret_cast<const uint4*>(wq + bi * 32 + 16);
            sdw = b < b_end ? amv_h2f(wd[bi]) : 0.0f;
        }
    }
    if (t < 2 * BM) {
        const int tok = min(m0 + (t >> 1), M - 1);
        const uint4* ap = reinterpret_cast<const uint4*>(a16 + (size_t)tok * K + 32 * bc);
        sa0 = ap[0];
        sa1 = ap[1];
        sa2 = ap[2];
        sa3 = ap[3];
        const int tb = t / BM;  // scale of (block 2 step + tb, token t % BM)
        sda = dT[(size_t)min(b0 + 2 * step + tb, b_end - 1) * M + min(m0 + t % BM, M - 1)];
    }
}

template <int WT, int TN, int TM, bool DEQ>
__device__ __forceinline__ void g16_store(const uint4 (&sw)[G16_NW(WT)], float sdw, uint4 sa0, uint4 sa1, uint4 sa2,
                                          uint4 sa3, float sda, uint16_t* __restrict__ sA,
                                          uint16_t* __restrict__ sB, float* __restrict__ sDw,
                                          float* __restrict__ sDa) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    const int t = threadIdx.x;
    const int blk = t & 1;
    if (t < 2 * BN) {
        uint4* dst = reinterpret_cast<uint4*>(sA + (t >> 1) * G16_LDK + 32 * blk);
        const g16_h2 dw2 = {(_Float16)sdw, (_Float16)sdw};  // DEQ: the block scale (an f16 value, exact)
        if constexpr (WT == AMV_T_Q4_0) {
            // element e < 16: low nibble of byte e; element 16 + e: high nibble of byte e; value q - 8
            const g16_h2 off = {(_Float16)1032.0f, (_Float16)1032.0f};
            const uint32_t wv[4] = {sw[0].x, sw[0].y, sw[0].z, sw[0].w};
            uint2 lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[i] = g16_nib4(wv[i] & 0x0F0F0F0Fu, off);
                hi[i] = g16_nib4((wv[i] >> 4) & 0x0F0F0F0Fu, off);
                if constexpr (DEQ) {
                    lo[i] = g16_scale2(lo[i], dw2);
                    hi[i] = g16_scale2(hi[i], dw2);
                }
            }
            dst[0] = make_uint4(lo[0].x, lo[0].y, lo[1].x, lo[1].y);
            dst[1] = make_uint4(lo[2].x, lo[2].y, lo[3].x, lo[3].y);
            dst[2] = make_uint4(hi[0].x, hi[0].y, hi[1].x, hi[1].y);
            dst[3] = make_uint4(hi[2].x, hi[2].y, hi[3].x, hi[3].y);
        } else {
            // int8 q -> f16: byte (q + 128) under the exponent of 1024, minus 1152
            const g16_h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
            const uint4 w1 = sw[G16_NW(WT) - 1];
            const uint32_t wv[8] = {sw[0].x, sw[0].y, sw[0].z, sw[0].w, w1.x, w1.y, w1.z, w1.w};
            uint2 h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                h[i] = g16_nib4(wv[i] ^ 0x80808080u, off);
                if constexpr (DEQ) h[i] = g16_scale2(h[i], dw2);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = make_uint4(h[2 * i].x, h[2 * i].y, h[2 * i + 1].x, h[2 * i + 1].y);
        }
        if constexpr (!DEQ) sDw[blk * BN + (t >> 1)] = sdw;
    }
    if (t < 2 * BM) {
        uint4* bd = reinterpret_cast<uint4*>(sB + (t >> 1) * G16_LDK + 32 * blk);
        bd[0] = sa0;
        bd[1] = sa1;
        bd[2] = sa2;
        bd[3] = sa3;
        if constexpr (!DEQ) sDa[t] = sda;  // [block t / BM][token t % BM]
    }
}

template <int WT, bool SUMS, int TN, int TM, bool DEQ>
__global__ __launch_bounds__(256) void k_mmq16(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N,
                                              int nb, const uint16_t* __restrict__ a16, const float* __restrict__ dT,
                                              int M, float* __restrict__ dst, int64_t ldd,
                                              int32_t* __restrict__ sums, int vec_out, int kb_per, int64_t zstride) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    __shared__ __align__(16) uint16_t sA[2][BN * G16_LDK];
    __shared__ __align__(16) uint16_t sB[2][BM * G16_LDK];
    __shared__ __align__(16) float sDw[2][2 * BN];
    __shared__ __align__(16) float sDa[2][2 * BM];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wr = w & 1, wc = w >> 1, c = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int K = nb * 32;
    // split of k (grid z): blocks b0 .. b_end - 1, output at dst + z * zstride (a partial when split)
    const int b0 = blockIdx.z * kb_per, b_end = min(nb, b0 + kb_per);
    const int nsteps = (b_end - b0 + 1) / 2;
    dst += (size_t)blockIdx.z * zstride;

    g16_f16v acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    uint4 sw[G16_NW(WT)], sa0, sa1, sa2, sa3;
    float sdw = 0.0f, sda = 0.0f;
    g16_load<WT, TN, TM>(sw, sdw, sa0, sa1, sa2, sa3, sda, 0, wq, wd, N, nb, n0, a16, dT, M, m0, K, b0, b_end);
    g16_store<WT, TN, TM, DEQ>(sw, sdw, sa0, sa1, sa2, sa3, sda, sA[0], sB[0], sDw[0], sDa[0]);
    __syncthreads();
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1;
        if (step + 1 < nsteps)
            g16_load<WT, TN, TM>(sw, sdw, sa0, sa1, sa2, sa3, sda, step + 1, wq, wd, N, nb, n0, a16, dT, M, m0, K, b0,
                                 b_end);
        if constexpr (DEQ) {  // scaled operands: accumulate across the whole step
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int kk = 16 * ks + 8 * h;
                g16_h8 A[TN], B[TM];
#pragma unroll
                for (int i = 0; i < TN; ++i)
                    A[i] = *reinterpret_cast<const g16_h8*>(sA[buf] + (32 * (TN * wr + i) + c) * G16_LDK + kk);
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    B[j] = *reinterpret_cast<const g16_h8*>(sB[buf] + (32 * (TM * wc + j) + c) * G16_LDK + kk);
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[j], acc[i][j], 0, 0, 0);
            }
        }
#pragma unroll 1
        for (int bl = 0; bl < (DEQ ? 0 : 2); ++bl) {  // one block's accumulators live at a time
            g16_f16v C[TN][TM];
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) C[i][j][r] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int kk = 32 * bl + 16 * ks + 8 * h;
                g16_h8 A[TN], B[TM];
#pragma unroll
                for (int i = 0; i < TN; ++i)
                    A[i] = *reinterpret_cast<const g16_h8*>(sA[buf] + (32 * (TN * wr + i) + c) * G16_LDK + kk);
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    B[j] = *reinterpret_cast<const g16_h8*>(sB[buf] + (32 * (TM * wc + j) + c) * G16_LDK + kk);
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) C[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[j], C[i][j], 0, 0, 0);
            }
            const int b = b0 + 2 * step + bl;
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int tl = 32 * (TM * wc + j) + c;  // token of this lane in the tile
                if (SUMS) {
                    const int m = m0 + tl;
#pragma unroll
                    for (int i = 0; i < TN; ++i)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int n = n0 + 32 * (TN * wr + i) + 8 * (r >> 2) + 4 * h + (r & 3);
                            if (b < b_end && m < M && n < N) sums[((size_t)m * N + n) * nb + b] = (int32_t)C[i][j][r];
                        }
                } else {
                    const float da = sDa[buf][bl * BM + tl];
#pragma unroll
                    for (int i = 0; i < TN; ++i) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float4 dw4 = *reinterpret_cast<const float4*>(
                                &sDw[buf][bl * BN + 32 * (TN * wr + i) + 8 * q + 4 * h]);
                            const float dwv[4] = {dw4.x, dw4.y, dw4.z, dw4.w};
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int r = 4 * q + e;
                                acc[i][j][r] = fmaf(C[i][j][r] * dwv[e], da, acc[i][j][r]);
                            }
                        }
                    }
                }
            }
        }
        if (step + 1 < nsteps) {
            g16_store<WT, TN, TM, DEQ>(sw, sdw, sa0, sa1, sa2, sa3, sda, sA[buf ^ 1], sB[buf ^ 1], sDw[buf ^ 1],
                                       sDa[buf ^ 1]);
            __syncthreads();
        }
    }
    if constexpr (!SUMS) {
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int m = m0 + 32 * (TM * wc + j) + c;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int n = n0 + 32 * (TN * wr + i) + 8 * q + 4 * h;
                    float* o = dst + (size_t)m * ldd + n;
                    if (vec_out && n + 3 < N) {
                        *reinterpret_cast<float4*>(o) =
                            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < N) o[e] = acc[i][j][4 * q + e];
                    }
                }
        }
    }
}

// Q4_0 / Q8_0 weights (MI355X layout), activations AMV_ACT_Q8_0_MMA of m rows. Tile: 128 x 128, or 64 x 64 when
// the big tiles would leave CUs idle.
// ---------------------------------------------------------------------------------------------------------------
// Split of k for the scaled (DEQ) form when the output tiles alone leave the CUs idle (the 4096-row, k = 14336 down
// projection): split z writes its partial tile to a workspace and k_splitk_sum adds the S partials in order z = 0 ..
// S - 1 (deterministic) into dst. The workspace is this library's, one per device, grown outside graph capture and
// never freed (a captured graph keeps the address it recorded); a call under capture that would need more than the
// device's workspace runs unsplit. Calls that split k share it: two on different streams must not overlap in time
// (calls on one stream are ordered).
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_splitk_sum(const float* __restrict__ part, int S, int64_t zstride, int m,
                                                   int n, float* __restrict__ dst, int64_t ldd, int vec) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (vec) {  // 4 consecutive outputs (n % 4 == 0, 16-byte aligned rows)
        const int n4 = n >> 2;
        if (i >= (int64_t)m * n4) return;
        const int r = (int)(i / n4), c = (int)(i % n4) * 4;
        float4 a = *reinterpret_cast<const float4*>(part + (size_t)r * n + c);
        for (int z = 1; z < S; ++z) {
            const float4 b = *reinterpret_cast<const float4*>(part + z * zstride + (size_t)r * n + c);
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        *reinterpret_cast<float4*>(dst + (size_t)r * ldd + c) = a;
    } else {
        if (i >= (int64_t)m * n) return;
        const int r = (int)(i / n), c = (int)(i % n);
        float a = part[(size_t)r * n + c];
        for (int z = 1; z < S; ++z) a += part[z * zstride + (size_t)r * n + c];
        dst[(size_t)r * ldd + c] = a;
    }
}

namespace {
std::mutex g_splitk_mu;
std::map<int, std::pair<float*, size_t>> g_splitk_ws;  // device -> (buffer, bytes)
}  // namespace

float* amv_splitk_workspace(size_t bytes, hipStream_t st) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g_splitk_mu);
    auto& w = g_splitk_ws[dev];
    if (w.second >= bytes) return w.first;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return nullptr;
    }
    const size_t want = std::max(bytes, 2 * w.second);
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    w = {(float*)p, want};  // the previous buffer stays allocated: a captured graph may still write it
    return w.first;
}

// splits of k for `tiles` output tiles over `steps` pipeline steps (64 of k each): only for k >= 64 SPLITK_MIN_TOTAL
// (the partials' extra traffic, (S + 1) m n 4 bytes, must stay small beside the product), doubled while the launch has
// fewer than SPLITK_TARGET workgroups and each split keeps >= SPLITK_MIN_STEPS steps (up to 8)
#ifndef SPLITK_TARGET
#define SPLITK_TARGET 1024
#endif
#ifndef SPLITK_MIN_STEPS
#define SPLITK_MIN_STEPS 24
#endif
#ifndef SPLITK_MIN_TOTAL
#define SPLITK_MIN_TOTAL 96
#endif
int amv_splitk_count(int64_t tiles, int steps) {
    int S = 1;
    if (steps < SPLITK_MIN_TOTAL) return 1;
    while (S < 8 && tiles * S < SPLITK_TARGET && steps / (2 * S) >= SPLITK_MIN_STEPS) S *= 2;
    return S;
}

void amv_splitk_reduce(const float* part, int S, int64_t zstride, int64_t m, int64_t n, float* dst, int64_t ldd,
                       hipStream_t st) {
    const int vec = n % 4 == 0 && ldd % 4 == 0 && ((uintptr_t)dst & 15) == 0;
    const int64_t items = vec ? m * (n / 4) : m * n;
    hipLaunchKernelGGL(k_splitk_sum, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, part, S, zstride, (int)m,
                       (int)n, dst, ldd, vec);
}

int amv_mmq16(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
              int64_t ldd, int32_t* sums, int deq, hipStream_t st) {
    const int nb = (int)(k / 32);
    const int64_t nblk = n_rows * nb;
    const uint8_t* wq = (const uint8_t*)w;
    const uint16_t* wd = (const uint16_t*)(wq + nblk * (wtype == AMV_T_Q4_0 ? 16 : 32));
    const AmvQ80Mma L = amv_q8_0_mma_layout(m, k);
    const uint16_t* a16 = (const uint16_t*)((const uint8_t*)act + L.a16);
    const float* dT = (const float*)((const uint8_t*)act + L.dt);
    const int vec_out = ((uintptr_t)dst & 15) == 0 && (ldd & 3) == 0;  // float4 stores of 4 consecutive rows
    const auto grid = [&](int tn, int tm) {
        return dim3((unsigned)((n_rows + 64 * tn - 1) / (64 * tn)), (unsigned)((m + 64 * tm - 1) / (64 * tm)));
    };
    const auto wgs = [&](int tn, int tm) { const dim3 g = grid(tn, tm); return (int64_t)g.x * g.y; };
    // exact form, measured on MI355X: 128 x 128 tiles win from ~1.5 workgroups per CU (14336 x 4096 at 512 tokens: 448
    // of them, 177 us against 207 us for 896 tiles of 64 x 128); below that 64 x 64 tiles (4096 x 14336: 241 us
    // against 311)
    // scaled form (DEQ), swept over 4096 / 6144 / 14336 / 28672 x 4096 and 4096 x 14336 at m = 128, 512 for Q4_0,
    // Q8_0, Q4_K: 128 x 128 from 224 workgroups (14336 x 4096 at 512: 83 us against 131 for 64 x 64), else 64 x 64
    const int cfg = deq ? (wgs(2, 2) >= 224 ? 22 : 11) : (wgs(2, 2) >= 384 ? 22 : 11);
    // DEQ: split of k when the tiles leave CUs idle
    int nz = 1, kb_per = nb;
    float* out = dst;
    int64_t ldo = ldd, zstride = 0;
    int vo = vec_out;
    if (deq && !sums) {
        const int S = amv_splitk_count(cfg == 22 ? wgs(2, 2) : wgs(1, 1), (nb + 1) / 2);
        if (S > 1) {
            kb_per = ((nb + S - 1) / S + 1) & ~1;  // whole pipeline steps
            nz = (nb + kb_per - 1) / kb_per;
            float* ws = nz > 1 ? amv_splitk_workspace((size_t)nz * m * n_rows * 4, st) : nullptr;
            if (ws) {
                out = ws;
                ldo = n_rows;
                zstride = m * n_rows;
                vo = n_rows % 4 == 0;
            } else {
                nz = 1;
                kb_per = nb;
            }
        }
    }
    const auto gridz = [&](int tn, int tm) { dim3 g = grid(tn, tm); g.z = (unsigned)nz; return g; };
#define G16_LAUNCH(WT, S, TN, TM, D)                                                                                 \
    hipLaunchKernelGGL((k_mmq16<WT, S, TN, TM, D>), gridz(TN, TM), dim3(256), 0, st, wq, wd, (int)n_rows, nb, a16, \
                       dT, (int)m, out, ldo, sums, vo, kb_per, zstride)
#define G16_CFG(WT, S, D)                          \
    if (cfg == 22) G16_LAUNCH(WT, S, 2, 2, D);     \
    else if (cfg == 12) G16_LAUNCH(WT, S, 1, 2, D); \
    else if (cfg == 21) G16_LAUNCH(WT, S, 2, 1, D); \
    else G16_LAUNCH(WT, S, 1, 1, D)
    if (wtype == AMV_T_Q4_0) {
        if (sums) { G16_CFG(AMV_T_Q4_0, true, false); }
        else if (deq) { G16_CFG(AMV_T_Q4_0, false, true); }
        else { G16_CFG(AMV_T_Q4_0, false, false); }
    } else {
        if (sums) { G16_CFG(AMV_T_Q8_0, true, false); }
        else if (deq) { G16_CFG(AMV_T_Q8_0, false, true); }
        else { G16_CFG(AMV_T_Q8_0, false, false); }
    }
#undef G16_CFG
#undef G16_LAUNCH
    if (nz > 1) amv_splitk_reduce(out, nz, zstride, m, n_rows, dst, ldd, st);
    return amv_check_launch("amv_mul_mat_q_act");
}

// ---------------------------------------------------------------------------------------------------------------
// Q4_K on the same tiling (reference ameva_mmqb.comp:11-16 for the integer form): per super-block j of 256 weights
// I1 = sum_u sc_u dot(q_u, q_a) and I2 = sum_u m_u bsum_u (exact integers), dst += d_a (d I1 - dmin I2). The weight
// operand is sc_u * q (<= 945, exact in f16) and the activation q_a (exact); a half super-block's 128 products stay
// below 2^24, so the accumulator is folded into the f32 sum after each half (d_a d C), and I2 is one more MFMA of the
// units' mins against the activation sums per 16 (AMV_ACT_Q8_K_MMA's f16 copies). Pipeline steps of one 64-weight
// chunk (units 2c, 2c + 1: the low and high nibbles of 32 bytes); the per-super-block values (d, dmin, the mins,
// the activation 16-sums and d_a) are staged at its first chunk into a slot of their own, double-buffered by
// super-block parity.
// DEQ variant (activations AMV_ACT_Q8_K_DEQ, f16 q_a d_a): each weight is staged as f16 of (d sc) q - dmin m (the
// two products rounded to f16, then one f16 fma), so the matrix core accumulates across all of k; no mins MFMA, no
// fold (the same ~3e-4 relative L2 as the Q4_0 / Q8_0 DEQ form).
struct G16K {
    uint4 q, hd, a0, a1, a2, a3, bs;
    float da;
};

template <int TN, int TM>
__device__ __forceinline__ void g16k_load(G16K& s, int step, const uint4* __restrict__ wq, const uint4* __restrict__ wh,
                                          int N, int nsb, int n0, const uint16_t* __restrict__ a16,
                                          const uint16_t* __restrict__ bs16, const float* __restrict__ dT, int M, int m0,
                                          int K, int sb0) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    const int t = threadIdx.x, hf = t & 1;
    const int j = sb0 + (step >> 2), c = step & 3;  // super-block j (of a split starting at sb0), chunk c
    if (t < 2 * BN) {
        const int row = min(n0 + (t >> 1), N - 1);
        const size_t sb = (size_t)row * nsb + j;
        s.q = wq[sb * 8 + 2 * c + hf];  // bytes 16 hf .. + 15 of chunk c
        s.hd = wh[sb];
    }
    if (t < 2 * BM) {
        const int tok = min(m0 + (t >> 1), M - 1);
        const uint4* ap = reinterpret_cast<const uint4*>(a16 + (size_t)tok * K + 256 * j + 64 * c + 32 * hf);
        s.a0 = ap[0];
        s.a1 = ap[1];
        s.a2 = ap[2];
        s.a3 = ap[3];
        if (c == 0) {
            s.bs = *reinterpret_cast<const uint4*>(bs16 + (size_t)tok * (K / 16) + 16 * j + 8 * hf);
            s.da = dT[(size_t)j * M + tok];
        }
    }
}

template <int TN, int TM, bool DEQ>
__device__ __forceinline__ void g16k_store(const G16K& s, int step, uint16_t* __restrict__ sA, uint16_t* __restrict__ sB,
                                           float* __restrict__ sD, float* __restrict__ sDm, uint16_t* __restrict__ sMn,
                                           uint16_t* __restrict__ sBs, float* __restrict__ sDa) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    const int t = threadIdx.x, hf = t & 1, c = step & 3;
    if (t < 2 * BN) {
        const int rl = t >> 1;
        int sc0, m0u, sc1, m1u;
        k4_scale_min(2 * c, s.hd.y, s.hd.z, s.hd.w, sc0, m0u);
        k4_scale_min(2 * c + 1, s.hd.y, s.hd.z, s.hd.w, sc1, m1u);
        const g16_h2 off = {(_Float16)1024.0f, (_Float16)1024.0f};
        g16_h2 f0, f1, n0v = {(_Float16)0.0f, (_Float16)0.0f}, n1v = n0v;
        if constexpr (DEQ) {  // (d sc) and -(dmin m) of the two units, rounded to f16
            const float d = amv_h2f(s.hd.x), dmin = amv_h2f(s.hd.x >> 16);
            const _Float16 a0 = (_Float16)(d * (float)sc0), a1 = (_Float16)(d * (float)sc1);
            const _Float16 b0 = (_Float16)(-(dmin * (float)m0u)), b1 = (_Float16)(-(dmin * (float)m1u));
            f0 = {a0, a0};
            f1 = {a1, a1};
            n0v = {b0, b0};
            n1v = {b1, b1};
        } else {
            f0 = {(_Float16)(float)sc0, (_Float16)(float)sc0};
            f1 = {(_Float16)(float)sc1, (_Float16)(float)sc1};
        }
        const uint32_t wv[4] = {s.q.x, s.q.y, s.q.z, s.q.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // element 16 hf + 4 i + e of unit 2c (low nibble) and 2c + 1 (high nibble)
            const uint2 l = g16_nib4(wv[i] & 0x0F0F0F0Fu, off), h = g16_nib4((wv[i] >> 4) & 0x0F0F0F0Fu, off);
            if constexpr (DEQ) {
                lo[2 * i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, l.x), f0, n0v));
                lo[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, l.y), f0, n0v));
                hi[2 * i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, h.x), f1, n1v));
                hi[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, h.y), f1, n1v));
            } else {
                lo[2 * i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(g16_h2, l.x) * f0);
                lo[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(g16_h2, l.y) * f0);
                hi[2 * i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(g16_h2, h.x) * f1);
                hi[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(g16_h2, h.y) * f1);
            }
        }
        uint4* dl = reinterpret_cast<uint4*>(sA + rl * G16_LDK + 16 * hf);
        uint4* dh = reinterpret_cast<uint4*>(sA + rl * G16_LDK + 32 + 16 * hf);
        dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
        if (!DEQ && c == 0) {  // per super-block: d, dmin, and the mins of units 4 hf .. 4 hf + 3 on their 16-sum slots
            if (hf == 0) {
                sD[rl] = amv_h2f(s.hd.x);
                sDm[rl] = amv_h2f(s.hd.x >> 16);
            }
            uint32_t mm[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                int scx, mx;
                k4_scale_min(4 * hf + e, s.hd.y, s.hd.z, s.hd.w, scx, mx);
                const uint32_t hb = __builtin_bit_cast(uint16_t, (_Float16)(float)mx);
                mm[e] = hb | (hb << 16);  // slots 2 u, 2 u + 1 (the unit's two 16-sums)
            }
            *reinterpret_cast<uint4*>(sMn + rl * 16 + 8 * hf) = make_uint4(mm[0], mm[1], mm[2], mm[3]);
        }
    }
    if (t < 2 * BM) {
        const int tl = t >> 1;
        uint4* bd = reinterpret_cast<uint4*>(sB + tl * G16_LDK + 32 * hf);
        bd[0] = s.a0;
        bd[1] = s.a1;
        bd[2] = s.a2;
        bd[3] = s.a3;
        if (!DEQ && c == 0) {
            *reinterpret_cast<uint4*>(sBs + tl * 16 + 8 * hf) = s.bs;
            if (hf == 0) sDa[tl] = s.da;
        }
    }
}

template <bool SUMS, int TN, int TM, bool DEQ>
__global__ __launch_bounds__(256) void k_mmq16_q4k(const uint4* __restrict__ wq, const uint4* __restrict__ wh, int N,
                                                  int nsb, const uint16_t* __restrict__ a16,
                                                  const uint16_t* __restrict__ bs16, const float* __restrict__ dT,
                                                  int M, float* __restrict__ dst, int64_t ldd,
                                                  int32_t* __restrict__ sums, int vec_out, int sb_per,
                                                  int64_t zstride) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    __shared__ __align__(16) uint16_t sA[2][BN * G16_LDK];
    __shared__ __align__(16) uint16_t sB[2][BM * G16_LDK];
    __shared__ __align__(16) float sD[2][BN], sDm[2][BN], sDa[2][BM];
    __shared__ __align__(16) uint16_t sMn[2][BN * 16], sBs[2][BM * 16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wr = w & 1, wc = w >> 1, c32 = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int K = nsb * 256;
    // split of k (grid z): super-blocks sb0 .. sb_end - 1, output at dst + z * zstride (a partial when split)
    const int sb0 = blockIdx.z * sb_per, sb_end = min(nsb, sb0 + sb_per);
    const int nsteps = (sb_end - sb0) * 4;
    dst += (size_t)blockIdx.z * zstride;

    g16_f16v acc[TN][TM], C[TN][TM];
    g16_f16v C0[TN][TM];  // SUMS: the first half's exact integers
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int jj = 0; jj < TM; ++jj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][jj][r] = C[i][jj][r] = C0[i][jj][r] = 0.0f;

    G16K st;
    g16k_load<TN, TM>(st, 0, wq, wh, N, nsb, n0, a16, bs16, dT, M, m0, K, sb0);
    g16k_store<TN, TM, DEQ>(st, 0, sA[0], sB[0], sD[0], sDm[0], sMn[0], sBs[0], sDa[0]);
    __syncthreads();
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1, j = sb0 + (step >> 2), c = step & 3, jp = (step >> 2) & 1;
        if (step + 1 < nsteps) g16k_load<TN, TM>(st, step + 1, wq, wh, N, nsb, n0, a16, bs16, dT, M, m0, K, sb0);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int kk = 16 * ks + 8 * h;
            g16_h8 A[TN], B[TM];
#pragma unroll
            for (int i = 0; i < TN; ++i)
                A[i] = *reinterpret_cast<const g16_h8*>(sA[buf] + (32 * (TN * wr + i) + c32) * G16_LDK + kk);
#pragma unroll
            for (int jj = 0; jj < TM; ++jj)
                B[jj] = *reinterpret_cast<const g16_h8*>(sB[buf] + (32 * (TM * wc + jj) + c32) * G16_LDK + kk);
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int jj = 0; jj < TM; ++jj) {
                    if constexpr (DEQ) acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[jj], acc[i][jj], 0, 0, 0);
                    else C[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[jj], C[i][jj], 0, 0, 0);
                }
        }
        if (!DEQ && (c == 1 || c == 3)) {
            // fold the half super-block (and at its end I2, the mins against the activation 16-sums), tile by tile
#pragma unroll
            for (int jj = 0; jj < TM; ++jj) {
                const int tl = 32 * (TM * wc + jj) + c32;
                const float da = sDa[jp][tl];
                const g16_h8 Bs = *reinterpret_cast<const g16_h8*>(sBs[jp] + tl * 16 + 8 * h);
#pragma unroll
                for (int i = 0; i < TN; ++i) {
                    g16_f16v I2;
#pragma unroll
                    for (int r = 0; r < 16; ++r) I2[r] = 0.0f;
                    if (c == 3) {
                        const g16_h8 Am =
                            *reinterpret_cast<const g16_h8*>(sMn[jp] + (32 * (TN * wr + i) + c32) * 16 + 8 * h);
                        I2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(Am, Bs, I2, 0, 0, 0);
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int rl = 32 * (TN * wr + i) + 8 * q + 4 * h;
                        const float4 d4 = *reinterpret_cast<const float4*>(&sD[jp][rl]);
                        const float4 dm4 = *reinterpret_cast<const float4*>(&sDm[jp][rl]);
                        const float dv[4] = {d4.x, d4.y, d4.z, d4.w}, dmv[4] = {dm4.x, dm4.y, dm4.z, dm4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * q + e;
                            if constexpr (SUMS) {
                                if (c == 1) {
                                    C0[i][jj][r] = C[i][jj][r];
                                } else {
                                    const int m = m0 + tl, n = n0 + rl + e;
                                    if (m < M && n < N) {
                                        int32_t* o = sums + (((size_t)m * N + n) * nsb + j) * 2;
                                        o[0] = (int)C0[i][jj][r] + (int)C[i][jj][r];
                                        o[1] = (int)I2[r];
                                    }
                                }
                            } else if (c == 1) {
                                acc[i][jj][r] = fmaf(C[i][jj][r] * dv[e], da, acc[i][jj][r]);
                            } else {
                                acc[i][jj][r] = fmaf(fmaf(dv[e], C[i][jj][r], -dmv[e] * I2[r]), da, acc[i][jj][r]);
                            }
                            C[i][jj][r] = 0.0f;
                        }
                    }
                }
            }
        }
        if (step + 1 < nsteps) {
            const int sp = ((step + 1) >> 2) & 1;  // per-super-block slot of the next step
            g16k_store<TN, TM, DEQ>(st, step + 1, sA[buf ^ 1], sB[buf ^ 1], sD[sp], sDm[sp], sMn[sp], sBs[sp], sDa[sp]);
            __syncthreads();
        }
    }
    if constexpr (!SUMS) {
#pragma unroll
        for (int jj = 0; jj < TM; ++jj) {
            const int m = m0 + 32 * (TM * wc + jj) + c32;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int n = n0 + 32 * (TN * wr + i) + 8 * q + 4 * h;
                    float* o = dst + (size_t)m * ldd + n;
                    if (vec_out && n + 3 < N) {
                        *reinterpret_cast<float4*>(o) = make_float4(acc[i][jj][4 * q], acc[i][jj][4 * q + 1],
                                                                    acc[i][jj][4 * q + 2], acc[i][jj][4 * q + 3]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < N) o[e] = acc[i][jj][4 * q + e];
                    }
                }
        }
    }
}

// Q4_K weights (MI355X layout: qs [N][K/256][128] | head [N][K/256][16]), activations AMV_ACT_Q8_K_MMA of m rows
int amv_mmq16_q4k(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst, int64_t ldd,
                  int32_t* sums, int deq, hipStream_t st) {
    const int nsb = (int)(k / 256);
    const int64_t nblk = n_rows * nsb;
    const uint4* wq = (const uint4*)w;
    const uint4* wh = (const uint4*)((const uint8_t*)w + nblk * 128);
    const AmvQ8kMma L = amv_q8k_mma_layout(m, k);
    const uint16_t* a16 = (const uint16_t*)((const uint8_t*)act + L.a16);
    const uint16_t* bs16 = (const uint16_t*)((const uint8_t*)act + L.bs16);
    const float* dT = (const float*)((const uint8_t*)act + L.dt);
    const int vec_out = ((uintptr_t)dst & 15) == 0 && (ldd & 3) == 0;
    const auto grid = [&](int tn, int tm) {
        return dim3((unsigned)((n_rows + 64 * tn - 1) / (64 * tn)), (unsigned)((m + 64 * tm - 1) / (64 * tm)));
    };
    const auto wgs = [&](int tn, int tm) { const dim3 g = grid(tn, tm); return (int64_t)g.x * g.y; };
    // Exact form, tile by measurement on 28672/14336/6144/4096 x 4096 and 4096 x 14336 at m = 128, 512: the 64 x 128
    // tile (occupancy 2) wins once it fills 448 workgroups, else 64 x 64 (occupancy 3); the 128 x 128 tile holds 256
    // VGPRs + 123 AGPRs at occupancy 1 and lost to both everywhere.
    const int cfg = deq ? (wgs(2, 2) >= 224 ? 22 : 11) : (wgs(1, 2) >= 448 ? 12 : 11);  // DEQ: the Q4_0 sweep's rule
    int nz = 1, sb_per = nsb;
    float* out = dst;
    int64_t ldo = ldd, zstride = 0;
    int vo = vec_out;
    if (deq && !sums) {  // split of k when the tiles leave CUs idle (4 pipeline steps per super-block)
        const int S = amv_splitk_count(cfg == 22 ? wgs(2, 2) : wgs(1, 1), 4 * nsb);
        if (S > 1) {
            sb_per = (nsb + S - 1) / S;
            nz = (nsb + sb_per - 1) / sb_per;
            float* ws = nz > 1 ? amv_splitk_workspace((size_t)nz * m * n_rows * 4, st) : nullptr;
            if (ws) {
                out = ws;
                ldo = n_rows;
                zstride = m * n_rows;
                vo = n_rows % 4 == 0;
            } else {
                nz = 1;
                sb_per = nsb;
            }
        }
    }
    const auto gridz = [&](int tn, int tm) { dim3 g = grid(tn, tm); g.z = (unsigned)nz; return g; };
#define G16K_LAUNCH(S, TN, TM, D)                                                                                    \
    hipLaunchKernelGGL((k_mmq16_q4k<S, TN, TM, D>), gridz(TN, TM), dim3(256), 0, st, wq, wh, (int)n_rows, nsb, a16,  \
                       bs16, dT, (int)m, out, ldo, sums, vo, sb_per, zstride)
    if (sums) {  // instrumentation: the small tile (two accumulator sets fit its registers)
        G16K_LAUNCH(true, 1, 1, false);
    } else if (deq) {
        if (cfg == 22) G16K_LAUNCH(false, 2, 2, true);
        else if (cfg == 12) G16K_LAUNCH(false, 1, 2, true);
        else if (cfg == 21) G16K_LAUNCH(false, 2, 1, true);
        else G16K_LAUNCH(false, 1, 1, true);
    } else {
        if (cfg == 12) G16K_LAUNCH(false, 1, 2, false);
        else G16K_LAUNCH(false, 1, 1, false);
    }
#undef G16K_LAUNCH
    if (nz > 1) amv_splitk_reduce(out, nz, zstride, m, n_rows, dst, ldd, st);
    return amv_check_launch("amv_mul_mat_q_act");
}
