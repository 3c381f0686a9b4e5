// Prefill MUL_MAT in the scaled form (AMEVA_MMQ_FORM=scaled, activation layouts AMV_ACT_Q8_0_DEQ / AMV_ACT_Q8_K_DEQ)
// on the f16 matrix cores of MI355X. The exact form (ggml's block integers, the default) runs on the int8 matrix
// cores in amv_qgemm.hip; this file also holds the split-of-k workspace and partial sum both forms share.
//
// Role of ameva_mmq.comp / ameva_mmqb.comp (reference, enc_mul_mat_mmq ggml-ameva.cpp:2540-2647), with the operands
// rounded once: the weights are staged as f16 (q - 8) d_w (Q4_0), q d_w (Q8_0) or (d sc) q - dmin m (Q4_K) and the
// activations arrive as f16 q_a d_a, so the matrix core accumulates across all of k with no per-block epilogue. Each
// operand is rounded to f16 once (relative 2^-11), so the f32 result is within ~3e-4 relative L2 of the exact value.
// Workgroup of 4 waves (2 x 2) on a tile of 64 TN weight rows x 64 TM tokens; wave (wr, wc) owns rows
// 32 TN wr .. + 32 TN and tokens 32 TM wc .. + 32 TM as TN x TM tiles of 32 x 32. Pipeline steps of 64 k: the
// global loads of step s + 1 are issued before step s computes from LDS; at staging the weights are converted to
// scaled f16 once per workgroup (shared by its 64 TM tokens) and the activations copied. MFMA operand layout
// (32x32x16 f16): lane l supplies A row l % 32 and B column l % 32 with 8 halves k = 8 (l / 32) .. + 7 of the 16-k
// step; it receives D column l % 32 (a token), rows 8 (r / 4) + 4 (l / 32) + r % 4, r = 0..15.
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

// The wave's TN x TM tiles of 32 x 32 outputs to dst[token][row] (float4 stores of 4 consecutive rows when allowed)
template <int TN, int TM>
__device__ __forceinline__ void g16_write_tile(const g16_f16v (&acc)[TN][TM], float* __restrict__ dst, int64_t ldd,
                                               int N, int M, int n0, int m0, int wr, int wc, int c, int h,
                                               int vec_out) {
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

// Registers of one staging step: thread t < 2 BN stages (row t / 2, block t % 2) of the weights (sw) and its scale
// (sdw); every thread t < 2 BM stages 64 bytes of one token's f16 activations (token t / 2, block t % 2, sa). Plain
// arrays (a struct of them was placed in scratch by the compiler).
#define G16_NW(WT) ((WT) == AMV_T_Q4_0 ? 1 : 2)

template <int WT, int TN, int TM>
__device__ __forceinline__ void g16_load(uint4 (&sw)[G16_NW(WT)], float& sdw, uint4& sa0, uint4& sa1, uint4& sa2,
                                         uint4& sa3, int step, const uint8_t* __restrict__ wq,
                                         const uint16_t* __restrict__ wd, int N, int nb, int n0,
                                         const uint16_t* __restrict__ a16, int M, int m0, int K, int b0, int b_end) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    const int t = threadIdx.x;
    const int blk = t & 1;
    // blocks b0 .. b_end - 1 of the row (a split of k); a block past the end reads the last one with scale 0
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
    }
}

template <int WT, int TN, int TM>
__device__ __forceinline__ void g16_store(const uint4 (&sw)[G16_NW(WT)], float sdw, uint4 sa0, uint4 sa1, uint4 sa2,
                                          uint4 sa3, uint16_t* __restrict__ sA, uint16_t* __restrict__ sB) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    const int t = threadIdx.x;
    const int blk = t & 1;
    if (t < 2 * BN) {
        uint4* dst = reinterpret_cast<uint4*>(sA + (t >> 1) * G16_LDK + 32 * blk);
        const g16_h2 dw2 = {(_Float16)sdw, (_Float16)sdw};  // the block scale (an f16 value, exact)
        if constexpr (WT == AMV_T_Q4_0) {
            // element e < 16: low nibble of byte e; element 16 + e: high nibble of byte e; value (q - 8) d
            const g16_h2 off = {(_Float16)1032.0f, (_Float16)1032.0f};
            const uint32_t wv[4] = {sw[0].x, sw[0].y, sw[0].z, sw[0].w};
            uint2 lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[i] = g16_scale2(g16_nib4(wv[i] & 0x0F0F0F0Fu, off), dw2);
                hi[i] = g16_scale2(g16_nib4((wv[i] >> 4) & 0x0F0F0F0Fu, off), dw2);
            }
            dst[0] = make_uint4(lo[0].x, lo[0].y, lo[1].x, lo[1].y);
            dst[1] = make_uint4(lo[2].x, lo[2].y, lo[3].x, lo[3].y);
            dst[2] = make_uint4(hi[0].x, hi[0].y, hi[1].x, hi[1].y);
            dst[3] = make_uint4(hi[2].x, hi[2].y, hi[3].x, hi[3].y);
        } else {
            // int8 q -> f16: byte (q + 128) under the exponent of 1024, minus 1152; then q d
            const g16_h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
            const uint4 w1 = sw[G16_NW(WT) - 1];
            const uint32_t wv[8] = {sw[0].x, sw[0].y, sw[0].z, sw[0].w, w1.x, w1.y, w1.z, w1.w};
            uint2 h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) h[i] = g16_scale2(g16_nib4(wv[i] ^ 0x80808080u, off), dw2);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = make_uint4(h[2 * i].x, h[2 * i].y, h[2 * i + 1].x, h[2 * i + 1].y);
        }
    }
    if (t < 2 * BM) {
        uint4* bd = reinterpret_cast<uint4*>(sB + (t >> 1) * G16_LDK + 32 * blk);
        bd[0] = sa0;
        bd[1] = sa1;
        bd[2] = sa2;
        bd[3] = sa3;
    }
}

template <int WT, int TN, int TM>
__global__ __launch_bounds__(256) void k_mmq16(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N,
                                              int nb, const uint16_t* __restrict__ a16, int M,
                                              float* __restrict__ dst, int64_t ldd, int vec_out, int kb_per,
                                              int64_t zstride) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    __shared__ __align__(16) uint16_t sA[2][BN * G16_LDK];
    __shared__ __align__(16) uint16_t sB[2][BM * G16_LDK];
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
    float sdw = 0.0f;
    g16_load<WT, TN, TM>(sw, sdw, sa0, sa1, sa2, sa3, 0, wq, wd, N, nb, n0, a16, M, m0, K, b0, b_end);
    g16_store<WT, TN, TM>(sw, sdw, sa0, sa1, sa2, sa3, sA[0], sB[0]);
    __syncthreads();
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1;
        if (step + 1 < nsteps)
            g16_load<WT, TN, TM>(sw, sdw, sa0, sa1, sa2, sa3, step + 1, wq, wd, N, nb, n0, a16, M, m0, K, b0, b_end);
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
        if (step + 1 < nsteps) {
            g16_store<WT, TN, TM>(sw, sdw, sa0, sa1, sa2, sa3, sA[buf ^ 1], sB[buf ^ 1]);
            __syncthreads();
        }
    }
    g16_write_tile<TN, TM>(acc, dst, ldd, N, M, n0, m0, wr, wc, c, h, vec_out);
}

// ---------------------------------------------------------------------------------------------------------------
// Split of k when the output tiles alone leave the CUs idle (the 4096-row, k = 14336 down
// projection): split z writes its partial tile to a workspace and k_splitk_sum adds the S partials in order z = 0 ..
// S - 1 (deterministic) into dst. The workspace is this library's, one per device, grown outside graph capture and
// never freed (a captured graph keeps the address it recorded); a call under capture that would need more than the
// device's workspace runs unsplit. Calls that split k share it: two on different streams must not overlap in time
// (calls on one stream are ordered).
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_splitk_sum(const float* __restrict__ part, int S, int64_t zstride, int m,
                                                   int n, float* dst, int64_t ldd, const float* add, int vec) {
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
        if (add) {  // the residual of a fused ADD, after the partials (add may be dst)
            const float4 b = *reinterpret_cast<const float4*>(add + (size_t)r * ldd + c);
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
        if (add) a += add[(size_t)r * ldd + c];
        dst[(size_t)r * ldd + c] = a;
    }
}

namespace {
std::mutex g_splitk_mu;
std::map<int, float*> g_splitk_ws;  // device -> the workspace (AMV_SPLITK_WS_BYTES)
}  // namespace

// The split-k partials of every batched kernel live in one per-device workspace of a fixed size, allocated by the
// first call that splits k and held until the process ends: a split count S is only chosen while the launch has
// fewer than SPLITK_TARGET (1024) workgroups, so S x tiles < 2 x 1024 and S x m x n x 4 bytes stay below
// 2048 x (128 x 128) x 4 = 128 MiB. The workspace never grows, so a captured graph's pointer stays valid. Under
// stream capture no allocation is possible: a call that splits k before any uncaptured call did fails (it never
// falls back to an unsplit launch, whose f32 summation order would differ from the same call outside capture).
float* amv_splitk_workspace(size_t bytes, hipStream_t st) {
    if (bytes > AMV_SPLITK_WS_BYTES) {
        amv_set_error("split-k workspace: %zu bytes asked, %zu available", bytes, (size_t)AMV_SPLITK_WS_BYTES);
        return nullptr;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        amv_set_error("split-k workspace: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_splitk_mu);
    float*& w = g_splitk_ws[dev];
    if (w) return w;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        amv_set_error("split-k workspace: first needed under stream capture; run a batched MUL_MAT that splits k "
                      "(k >= 6144 with fewer than 1024 tiles) once before capturing");
        return nullptr;
    }
    void* p = nullptr;
    if (hipMalloc(&p, AMV_SPLITK_WS_BYTES) != hipSuccess) {
        (void)hipGetLastError();
        amv_set_error("split-k workspace: hipMalloc of %zu bytes failed", (size_t)AMV_SPLITK_WS_BYTES);
        return nullptr;
    }
    w = (float*)p;
    return w;
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
                       hipStream_t st, const float* add = nullptr) {
    const int vec = n % 4 == 0 && ldd % 4 == 0 && ((uintptr_t)dst & 15) == 0 && ((uintptr_t)add & 15) == 0;
    const int64_t items = vec ? m * (n / 4) : m * n;
    hipLaunchKernelGGL(k_splitk_sum, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, part, S, zstride, (int)m,
                       (int)n, dst, ldd, add, vec);
}

// Q4_0 / Q8_0 weights (MI355X layout), activations AMV_ACT_Q8_0_DEQ of m rows, the scaled form
int amv_mmq16(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst,
              int64_t ldd, hipStream_t st) {
    const int nb = (int)(k / 32);
    const int64_t nblk = n_rows * nb;
    const uint8_t* wq = (const uint8_t*)w;
    const uint16_t* wd = (const uint16_t*)(wq + nblk * (wtype == AMV_T_Q4_0 ? 16 : 32));
    const AmvQ80Mma L = amv_q8_0_mma_layout(m, k);
    const uint16_t* a16 = (const uint16_t*)((const uint8_t*)act + L.a16);
    const int vec_out = ((uintptr_t)dst & 15) == 0 && (ldd & 3) == 0;  // float4 stores of 4 consecutive rows
    const auto grid = [&](int tn, int tm) {
        return dim3((unsigned)((n_rows + 64 * tn - 1) / (64 * tn)), (unsigned)((m + 64 * tm - 1) / (64 * tm)));
    };
    const auto wgs = [&](int tn, int tm) { const dim3 g = grid(tn, tm); return (int64_t)g.x * g.y; };
    // swept over 4096 / 6144 / 14336 / 28672 x 4096 and 4096 x 14336 at m = 128, 512 for Q4_0, Q8_0, Q4_K: 128 x 128
    // from 224 workgroups (14336 x 4096 at 512: 83 us against 131 for 64 x 64), else 64 x 64
    const int cfg = wgs(2, 2) >= 224 ? 22 : 11;
    // split of k when the tiles leave CUs idle
    int nz = 1, kb_per = nb;
    float* out = dst;
    int64_t ldo = ldd, zstride = 0;
    int vo = vec_out;
    const int S = amv_splitk_count(cfg == 22 ? wgs(2, 2) : wgs(1, 1), (nb + 1) / 2);
    if (S > 1) {
        kb_per = ((nb + S - 1) / S + 1) & ~1;  // whole pipeline steps
        nz = (nb + kb_per - 1) / kb_per;
        float* ws = nz > 1 ? amv_splitk_workspace((size_t)nz * m * n_rows * 4, st) : nullptr;
        if (nz > 1 && !ws) return AMV_ERR_HIP;  // never unsplit: the summation order would change
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
    const auto gridz = [&](int tn, int tm) { dim3 g = grid(tn, tm); g.z = (unsigned)nz; return g; };
#define G16_LAUNCH(WT, TN, TM)                                                                                   \
    hipLaunchKernelGGL((k_mmq16<WT, TN, TM>), gridz(TN, TM), dim3(256), 0, st, wq, wd, (int)n_rows, nb, a16, \
                       (int)m, out, ldo, vo, kb_per, zstride)
    if (wtype == AMV_T_Q4_0) {
        if (cfg == 22) G16_LAUNCH(AMV_T_Q4_0, 2, 2);
        else G16_LAUNCH(AMV_T_Q4_0, 1, 1);
    } else {
        if (cfg == 22) G16_LAUNCH(AMV_T_Q8_0, 2, 2);
        else G16_LAUNCH(AMV_T_Q8_0, 1, 1);
    }
#undef G16_LAUNCH
    if (nz > 1) amv_splitk_reduce(out, nz, zstride, m, n_rows, dst, ldd, st);
    return amv_check_launch("amv_mul_mat_q_act");
}

// ---------------------------------------------------------------------------------------------------------------
// Q4_K on the same tiling (activations AMV_ACT_Q8_K_DEQ, f16 q_a d_a): each weight is staged as f16 of
// (d sc) q - dmin m (the two products rounded to f16, then one f16 fma), so the matrix core accumulates across all of
// k. Pipeline steps of one 64-weight chunk (units 2c, 2c + 1: the low and high nibbles of 32 bytes).
struct G16K {
    uint4 q, hd, a0, a1, a2, a3;
};

template <int TN, int TM>
__device__ __forceinline__ void g16k_load(G16K& s, int step, const uint4* __restrict__ wq, const uint4* __restrict__ wh,
                                          int N, int nsb, int n0, const uint16_t* __restrict__ a16, int M, int m0,
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
    }
}

template <int TN, int TM>
__device__ __forceinline__ void g16k_store(const G16K& s, int step, uint16_t* __restrict__ sA,
                                           uint16_t* __restrict__ sB) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    const int t = threadIdx.x, hf = t & 1, c = step & 3;
    if (t < 2 * BN) {
        const int rl = t >> 1;
        int sc0, m0u, sc1, m1u;
        k4_scale_min(2 * c, s.hd.y, s.hd.z, s.hd.w, sc0, m0u);
        k4_scale_min(2 * c + 1, s.hd.y, s.hd.z, s.hd.w, sc1, m1u);
        const g16_h2 off = {(_Float16)1024.0f, (_Float16)1024.0f};
        // (d sc) and -(dmin m) of the two units, rounded to f16
        const float d = amv_h2f(s.hd.x), dmin = amv_h2f(s.hd.x >> 16);
        const _Float16 a0 = (_Float16)(d * (float)sc0), a1 = (_Float16)(d * (float)sc1);
        const _Float16 b0 = (_Float16)(-(dmin * (float)m0u)), b1 = (_Float16)(-(dmin * (float)m1u));
        const g16_h2 f0 = {a0, a0}, f1 = {a1, a1}, n0v = {b0, b0}, n1v = {b1, b1};
        const uint32_t wv[4] = {s.q.x, s.q.y, s.q.z, s.q.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // element 16 hf + 4 i + e of unit 2c (low nibble) and 2c + 1 (high nibble)
            const uint2 l = g16_nib4(wv[i] & 0x0F0F0F0Fu, off), h = g16_nib4((wv[i] >> 4) & 0x0F0F0F0Fu, off);
            lo[2 * i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, l.x), f0, n0v));
            lo[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, l.y), f0, n0v));
            hi[2 * i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, h.x), f1, n1v));
            hi[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(g16_h2, h.y), f1, n1v));
        }
        uint4* dl = reinterpret_cast<uint4*>(sA + rl * G16_LDK + 16 * hf);
        uint4* dh = reinterpret_cast<uint4*>(sA + rl * G16_LDK + 32 + 16 * hf);
        dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    }
    if (t < 2 * BM) {
        const int tl = t >> 1;
        uint4* bd = reinterpret_cast<uint4*>(sB + tl * G16_LDK + 32 * hf);
        bd[0] = s.a0;
        bd[1] = s.a1;
        bd[2] = s.a2;
        bd[3] = s.a3;
    }
}

template <int TN, int TM>
__global__ __launch_bounds__(256) void k_mmq16_q4k(const uint4* __restrict__ wq, const uint4* __restrict__ wh, int N,
                                                  int nsb, const uint16_t* __restrict__ a16, int M,
                                                  float* __restrict__ dst, int64_t ldd, int vec_out, int sb_per,
                                                  int64_t zstride) {
    constexpr int BN = 64 * TN, BM = 64 * TM;
    __shared__ __align__(16) uint16_t sA[2][BN * G16_LDK];
    __shared__ __align__(16) uint16_t sB[2][BM * G16_LDK];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wr = w & 1, wc = w >> 1, c32 = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int K = nsb * 256;
    // split of k (grid z): super-blocks sb0 .. sb_end - 1, output at dst + z * zstride (a partial when split)
    const int sb0 = blockIdx.z * sb_per, sb_end = min(nsb, sb0 + sb_per);
    const int nsteps = (sb_end - sb0) * 4;
    dst += (size_t)blockIdx.z * zstride;

    g16_f16v acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int jj = 0; jj < TM; ++jj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0.0f;

    G16K st;
    g16k_load<TN, TM>(st, 0, wq, wh, N, nsb, n0, a16, M, m0, K, sb0);
    g16k_store<TN, TM>(st, 0, sA[0], sB[0]);
    __syncthreads();
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1;
        if (step + 1 < nsteps) g16k_load<TN, TM>(st, step + 1, wq, wh, N, nsb, n0, a16, M, m0, K, sb0);
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
                for (int jj = 0; jj < TM; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[jj], acc[i][jj], 0, 0, 0);
        }
        if (step + 1 < nsteps) {
            g16k_store<TN, TM>(st, step + 1, sA[buf ^ 1], sB[buf ^ 1]);
            __syncthreads();
        }
    }
    g16_write_tile<TN, TM>(acc, dst, ldd, N, M, n0, m0, wr, wc, c32, h, vec_out);
}

// Q4_K weights (MI355X layout: qs [N][K/256][128] | head [N][K/256][16]), activations AMV_ACT_Q8_K_DEQ of m rows
int amv_mmq16_q4k(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float* dst, int64_t ldd,
                  hipStream_t st) {
    const int nsb = (int)(k / 256);
    const int64_t nblk = n_rows * nsb;
    const uint4* wq = (const uint4*)w;
    const uint4* wh = (const uint4*)((const uint8_t*)w + nblk * 128);
    const AmvQ8kMma L = amv_q8k_mma_layout(m, k);
    const uint16_t* a16 = (const uint16_t*)((const uint8_t*)act + L.a16);
    const int vec_out = ((uintptr_t)dst & 15) == 0 && (ldd & 3) == 0;
    const auto grid = [&](int tn, int tm) {
        return dim3((unsigned)((n_rows + 64 * tn - 1) / (64 * tn)), (unsigned)((m + 64 * tm - 1) / (64 * tm)));
    };
    const auto wgs = [&](int tn, int tm) { const dim3 g = grid(tn, tm); return (int64_t)g.x * g.y; };
    const int cfg = wgs(2, 2) >= 224 ? 22 : 11;  // the Q4_0 sweep's rule
    int nz = 1, sb_per = nsb;
    float* out = dst;
    int64_t ldo = ldd, zstride = 0;
    int vo = vec_out;
    const int S = amv_splitk_count(cfg == 22 ? wgs(2, 2) : wgs(1, 1), 4 * nsb);  // 4 pipeline steps per super-block
    if (S > 1) {  // split of k when the tiles leave CUs idle
        sb_per = (nsb + S - 1) / S;
        nz = (nsb + sb_per - 1) / sb_per;
        float* ws = nz > 1 ? amv_splitk_workspace((size_t)nz * m * n_rows * 4, st) : nullptr;
        if (nz > 1 && !ws) return AMV_ERR_HIP;  // never unsplit: the summation order would change
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
    const auto gridz = [&](int tn, int tm) { dim3 g = grid(tn, tm); g.z = (unsigned)nz; return g; };
#define G16K_LAUNCH(TN, TM)                                                                                        \
    hipLaunchKernelGGL((k_mmq16_q4k<TN, TM>), gridz(TN, TM), dim3(256), 0, st, wq, wh, (int)n_rows, nsb, a16, (int)m, \
                       out, ldo, vo, sb_per, zstride)
    if (cfg == 22) G16K_LAUNCH(2, 2);
    else G16K_LAUNCH(1, 1);
#undef G16K_LAUNCH
    if (nz > 1) amv_splitk_reduce(out, nz, zstride, m, n_rows, dst, ldd, st);
    return amv_check_launch("amv_mul_mat_q_act");
}
