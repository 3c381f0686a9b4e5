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

#include <atomic>

#define M4 0x0F0F0F0Fu

// Epilogues of the one-column GEMV, the reference's ameva_qmv / ameva_mmvq ep_mode (ameva_qmv.comp:233-246,
// fusion pairs ggml-ameva.cpp:4280-4285). v_n is the row's dot product, e the epilogue operand, eout its output;
// dst[n] = v_n is written too when dst is not NULL (the reference's write-through of the MUL_MAT node):
//   EP 1 (MUL_MAT -> ADD):                   eout[n] = v_n + e[n]
//   EP 2 (MUL_MAT -> SWIGLU, gate operand):  eout[n] = v_n / (1 + exp(-v_n)) * e[n]
//   EP 3 (MUL_MAT -> SWIGLU, up operand):    eout[n] = e[n] / (1 + exp(-e[n])) * v_n
//   EP 4 (MI355X, one weight of stacked gate rows 0..F-1 and up rows F..2F-1): wave w computes rows w and F + w and
//        eout[w] = v_w / (1 + exp(-v_w)) * v_{F+w}; the gate and up MUL_MATs read the same activations, so one
//        launch streams both weights.
// Launches that do more than their epilogue (MI355X decode fusions; each replaces one or two launches of small
// kernels, which cost ~4 us apiece at bs1 whatever their size):
//   EP 5 ROPE_KV:     q/k/v rows stacked (n_q q rows, n_k k rows, then v rows, heads of head_dim rows); ROPE NORMAL
//                     on q and k (pair j = rows 2j, 2j + 1 of a head: exactly the two rows of a wave), dst gets the
//                     rotated q/k and the v values, and the k and v rows are also stored as f16 at cache row
//                     kv_idx[0] (k_rope_kv's arithmetic and skip/count rule)
//   EP 6 ADD_NORM:    EP 1, then the last workgroup to finish applies RMS_NORM (+MUL by norm_w, +Q8_0) to the whole
//                     eout vector (k_rms_norm's arithmetic, same bits)
//   EP 7 SWIGLU_Q8:   EP 4, then the last workgroup of each 32 outputs quantizes them to Q8_0 (amv_quantize_act's
//                     rules)
#define MMV_EP_ROPE_KV 5
#define MMV_EP_ADD_NORM 6
#define MMV_EP_SWIGLU_Q8 7
#define MMV_STACKED(EP) ((EP) == AMV_EP_SWIGLU_STACKED || (EP) == MMV_EP_SWIGLU_Q8)
#define MMV_TAIL(EP) ((EP) == MMV_EP_ADD_NORM || (EP) == MMV_EP_SWIGLU_Q8)

struct MmvPost {
    const int32_t* pos;  // ROPE_KV: position of the token
    float theta_scale, freq_scale, attn_factor;
    int n_q, n_k, head_dim;
    uint16_t* k_cache;
    uint16_t* v_cache;
    int64_t cache_row;      // elements per cache row
    const int64_t* kv_idx;  // cache row of the token
    int64_t cache_rows;
    unsigned int* bad;       // count of skipped k/v head stores (rows outside [0, cache_rows))
    unsigned int* counters;  // tails: zero before the first launch, left at zero by every launch
    const float* norm_w;     // ADD_NORM: MUL operand (NULL: none)
    float eps;
    float* norm_y;  // ADD_NORM outputs, each may be NULL: x * scale, then * norm_w
    float* norm_o;
    AmvActOut act;  // quantized output of the tail (Q8_0 or Q8_K activation row)
    // Segmented weights (EP 5 and 7 over separate matrices, SEG kernels): rows seg_row[s] .. seg_row[s + 1] - 1 of
    // the stacked row space are the rows of matrix s, held at w_seg[s] in its own layout; EP 5 writes them to
    // dst_seg[s]. n_seg = 0: one matrix; else seg_row[n_seg .. 3] are INT32_MAX.
    int n_seg;
    int seg_row[4];
    const uint8_t* w_seg[3];
    float* dst_seg[3];
};

// the segment of stacked row `row` and its row within that matrix
// The fields of segment s are read by constant index and selected: a run-time index into the by-value kernel argument
// makes the compiler read it with vector loads from the argument segment, and every weight address then waits for
// them (a memory round trip before the weight stream).
__device__ __forceinline__ int mmv_seg_first(const MmvPost& p, int s) {
    const int r0 = p.seg_row[0], r1 = p.seg_row[1], r2 = p.seg_row[2], r3 = p.seg_row[3];
    return s == 0 ? r0 : s == 1 ? r1 : s == 2 ? r2 : r3;
}
__device__ __forceinline__ const uint8_t* mmv_seg_w(const MmvPost& p, int s) {
    const uint8_t* w0 = p.w_seg[0];
    const uint8_t* w1 = p.w_seg[1];
    const uint8_t* w2 = p.w_seg[2];
    return s == 0 ? w0 : s == 1 ? w1 : w2;
}
__device__ __forceinline__ float* mmv_seg_dst(const MmvPost& p, int s) {
    float* d0 = p.dst_seg[0];
    float* d1 = p.dst_seg[1];
    float* d2 = p.dst_seg[2];
    return s == 0 ? d0 : s == 1 ? d1 : d2;
}
__device__ __forceinline__ int mmv_seg(const MmvPost& p, int row, int& local) {
    const int s = (row >= p.seg_row[1]) + (row >= p.seg_row[2]);
    local = row - mmv_seg_first(p, s);
    return s;
}

// Stacked SWIGLU: a wave owns the R / 2 consecutive outputs o = (R / 2) wave + i, i.e. gate rows o (r = i) and up
// rows F + o (r = R / 2 + i), F = n_rows / 2.
template <int EP>
__device__ __forceinline__ int mmv_row(int wave, int r, int R, int n_rows) {
    const int P = R >> 1;
    return MMV_STACKED(EP) ? P * wave + r % P + (r / P) * (n_rows >> 1) : wave * R + r;
}
template <int EP>
__device__ __forceinline__ bool mmv_wave_live(int wave, int R, int n_rows) {
    return MMV_STACKED(EP) ? (R >> 1) * wave < (n_rows >> 1) : wave * R < n_rows;
}
__device__ __forceinline__ float mmv_silu(float x) { return x / (1.0f + expf(-x)); }

// ROPE_KV: the token's cache row and the rotation of the wave's pair (a function of the position and the pair
// index only), computed at the start of the kernel where they overlap the weight stream
struct MmvRopeAt {
    float c, s;
    int64_t row;
};
template <int EP>
__device__ __forceinline__ MmvRopeAt mmv_rope_at(const MmvPost& post, int wave) {
    MmvRopeAt r{1.0f, 0.0f, 0};
    if constexpr (EP == MMV_EP_ROPE_KV) {
        r.row = post.kv_idx[0];
        const int r0 = wave * 2;
        if (r0 < post.n_q + post.n_k)
            amv_rope_cs((float)post.pos[0], (r0 % post.head_dim) >> 1, post.theta_scale, post.freq_scale,
                        post.attn_factor, r.c, r.s);
    }
    return r;
}

// End of a row group: wave sums of the R accumulators; with a split of K (S > 1 waves per row group) the S partial
// sums meet in LDS and are added in the fixed order ks = 0 .. S-1 by the group's first wave; then the epilogue.
template <int R, int EP, int S, bool SEG = false>
__device__ __forceinline__ void mmv_finish(const float (&acc)[R], int lane, int wi, int ks, bool live, int wave,
                                           int n_rows, float* __restrict__ dst, const float* __restrict__ epi,
                                           float* __restrict__ eout, const MmvPost& post, const MmvRopeAt& ra) {
    static_assert(EP != MMV_EP_ROPE_KV || R == 2, "ROPE pairs the two rows of a wave");
    static_assert(!MMV_STACKED(EP) || R == 2 || R == 4 || R == 8, "stacked SWIGLU takes 1, 2 or 4 outputs per wave");
    float t[R];
#pragma unroll
    for (int r = 0; r < R; ++r) t[r] = amv_wave_sum(acc[r]);
    if constexpr (S > 1) {
        __shared__ float part[4][R];
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) part[wi][r] = t[r];
        }
        __syncthreads();
        if (ks != 0 || !live) return;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = part[wi][r];
#pragma unroll
            for (int k = 1; k < S; ++k) v += part[wi + k][r];
            t[r] = v;
        }
    }
    if (lane != 0) return;
    if constexpr (EP == MMV_EP_ROPE_KV) {
        const int r0 = wave * 2;
        if (r0 >= n_rows) return;
        const int nqk = post.n_q + post.n_k;
        float y0 = t[0], y1 = t[1];
        if (r0 < nqk) amv_rope_apply(ra.c, ra.s, t[0], t[1], y0, y1);
        if constexpr (SEG) {
            int lr;
            const int sg = mmv_seg(post, r0, lr);
            mmv_seg_dst(post, sg)[lr] = y0;
            mmv_seg_dst(post, sg)[lr + 1] = y1;
        } else {
            dst[r0] = y0;
            dst[r0 + 1] = y1;
        }
        if (r0 >= post.n_q) {
            const int64_t dr = ra.row;
            const bool store = dr >= 0 && dr < post.cache_rows;
            const int rr = r0 < nqk ? r0 - post.n_q : r0 - nqk;  // row within the k or v block
            if (store) {
                uint16_t* c = (r0 < nqk ? post.k_cache : post.v_cache) + dr * post.cache_row + rr;
                c[0] = amv_f2h(y0);
                c[1] = amv_f2h(y1);
            } else if (rr % post.head_dim == 0 && post.bad) {
                atomicAdd(post.bad, 1u);  // once per skipped head, as k_rope_kv counts
            }
        }
        return;
    }
    if constexpr (MMV_STACKED(EP)) {
        constexpr int P = R / 2;
        const int F = n_rows >> 1;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int o = P * wave + i;
            if (o >= F) break;
            if (dst) {
                dst[o] = t[i];
                dst[o + F] = t[P + i];
            }
            if constexpr (EP == MMV_EP_SWIGLU_Q8) amv_store_coh(eout + o, mmv_silu(t[i]) * t[P + i]);
            else eout[o] = mmv_silu(t[i]) * t[P + i];
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = wave * R + r;
        if (row >= n_rows) continue;
        if (EP == AMV_EP_NONE || dst) dst[row] = t[r];
        if (EP == AMV_EP_ADD) eout[row] = t[r] + epi[row];
        if (EP == MMV_EP_ADD_NORM) amv_store_coh(eout + row, t[r] + epi[row]);
        if (EP == AMV_EP_SILU_MUL) eout[row] = mmv_silu(t[r]) * epi[row];
        if (EP == AMV_EP_MUL_SILU) eout[row] = mmv_silu(epi[row]) * t[r];
    }
}

// Tails of EP 6 and EP 7, run by every thread of the workgroup (NW waves) after the epilogue stores.
template <int EP, int S, int R, int NW = 4>
__device__ __forceinline__ void mmv_tail(const MmvPost& post, const float* eout, int n_rows) {
    if constexpr (EP == MMV_EP_ADD_NORM) {
        if (!amv_arrive_last_tree(post.counters)) return;
        amv_acquire();
        __shared__ double sred[AMV_RMS_VLANES / 64];
        amv_rms_row<256>(reinterpret_cast<const float4*>(eout), n_rows / 4, post.eps, post.norm_w, post.norm_y,
                         post.norm_o, post.act, sred);
    } else {
        // a workgroup's (NW / S) (R / 2) outputs lie in one block of BS (the launcher checks that BS divides
        // n_rows / 2); the first wave of the last workgroup quantizes it, 4 values per lane
        constexpr int per_wg = NW / S * (R / 2);
        const int BS = post.act.type == AMV_T_Q8_K ? 256 : 32;
        const int blk = (int)blockIdx.x * per_wg / BS;
        if (!amv_arrive_last(post.counters + AMV_CNT_STRIDE * blk, BS / per_wg)) return;
        const int lane = threadIdx.x;
        if (lane < BS / 4) {
            const float4 t = amv_load4_coh(eout + BS * blk + 4 * lane);
            const float v[4] = {t.x, t.y, t.z, t.w};
            amv_act_store4(post.act, BS / 4 * blk + lane, v);
        }
    }
}

// FULL: every 64 U-block step is whole (nb % (64 U) == 0) and every row of a live wave exists, so the loads need no
// clamps and the blocks no guard (all Llama shapes); otherwise indices are clamped and tail blocks skipped. Block
// indices are 32-bit (the launcher checks n_rows * nb < 2^31). PAIRS: n_rows is even, every scale sits in a pair.
// NBT: the block count of a row as a compile-time constant (128: K = 4096, the hidden size of most Llama GEMVs) or 0
// (the nb argument): with a constant the row offsets are shifts and the one-step loop has no test.
template <int R, int U, bool BLOCK_SUMS, int EP, int S, bool PAIRS, bool FULL, int NBT = 0, bool SEG = false>
__global__ __launch_bounds__(256) void k_mmv_q4_0(const uint4* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                 int n_rows, int nb_arg, const int8_t* __restrict__ aq,
                                                 const int2* __restrict__ ads, float* __restrict__ dst,
                                                 int32_t* __restrict__ sums, const float* __restrict__ epi,
                                                 float* __restrict__ eout, const MmvPost post) {
    static_assert(!BLOCK_SUMS || S == 1, "block sums are written per block, without a split of K");
    const int nb = NBT ? NBT : nb_arg;
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6, ks = wi % S;
    const int wave = blockIdx.x * (4 / S) + wi / S;  // row group; the S waves of a group split K
    const bool live = mmv_wave_live<EP>(wave, R, n_rows);
    const MmvRopeAt ra = mmv_rope_at<EP>(post, wave);  // ROPE_KV
    // No early exit for the waves past the last row (they stream clamped rows and store nothing) and, for whole steps
    // without a split, no test before the first step: all kernel arguments are then fetched in one scalar round trip
    // ahead of the first load (a branch there costs a second one at the start of every wave).
    const int4* a4 = reinterpret_cast<const int4*>(aq);
    const uint32_t* wd2 = reinterpret_cast<const uint32_t*>(wd);
    uint32_t rb[R], db[R];  // block index of (row, 0); scale index of (row, 0) minus the block offset factor
    const uint4* wqr[R];    // SEG: the row's matrix (its rows are indexed within it)
    const uint16_t* wdr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int row = min(mmv_row<EP>(wave, r, R, n_rows), n_rows - 1);
        wqr[r] = wq;
        wdr[r] = wd;
        if constexpr (SEG) {
            int lr;
            const int sg = mmv_seg(post, row, lr);
            const uint32_t rows_s = (uint32_t)(mmv_seg_first(post, sg + 1) - mmv_seg_first(post, sg));
            wqr[r] = reinterpret_cast<const uint4*>(mmv_seg_w(post, sg));
            wdr[r] = reinterpret_cast<const uint16_t*>(mmv_seg_w(post, sg) + (size_t)rows_s * nb * 16);
            row = lr;
        }
        rb[r] = (uint32_t)row * (uint32_t)nb;
        db[r] = (uint32_t)(row >> 1) * (uint32_t)nb * 2u + (uint32_t)(row & 1);  // PAIRS: + 2 j
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    constexpr bool FIRST = FULL && S == 1;  // nb >= 64 U: the first step always runs
    int j0 = (FIRST || live) ? 64 * U * ks : nb;
    if (FIRST || j0 < nb) do {
        // all loads of the step before any arithmetic: the weight stream first, then the activation blocks (L2 hits)
        int4 a0[U], a1[U];
        int2 ads_u[U];
        uint4 w[U][R];
        uint32_t dw[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = FULL ? j0 + 64 * u + lane : min(j0 + 64 * u + lane, nb - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) w[u][r] = amv_ld_stream((SEG ? wqr[r] : wq) + rb[r] + j);
            if (BLOCK_SUMS) continue;
            if constexpr (SEG && PAIRS && R % 2 == 0 && (!MMV_STACKED(EP) || R == 4)) {
                // rows 2p, 2p + 1 of one matrix (each matrix holds an even row count): both scales in one dword
#pragma unroll
                for (int r = 0; r < R; r += 2) {
                    const uint32_t d2 = amv_ld_stream(reinterpret_cast<const uint32_t*>(wdr[r]) + (db[r] >> 1) + j);
                    dw[u][r] = d2 & 0xFFFFu;
                    dw[u][r + 1] = d2 >> 16;
                }
            } else if constexpr (SEG) {
#pragma unroll
                for (int r = 0; r < R; ++r) dw[u][r] = amv_ld_stream(wdr[r] + db[r] + 2 * j);
            } else if constexpr (PAIRS && R % 2 == 0 && (!MMV_STACKED(EP) || (EP == MMV_EP_SWIGLU_Q8 && R == 4))) {
                // the wave's rows 2p, 2p + 1 read both scales with one dword (stacked gate/up with two outputs per
                // wave: rows o, o + 1 and F + o, F + o + 1, pairs since o and F = n_rows / 2 are even: the launcher
                // makes the quantization block size divide F)
#pragma unroll
                for (int r = 0; r < R; r += 2) {
                    const uint32_t d2 = amv_ld_stream(wd2 + (db[r] >> 1) + j);
                    dw[u][r] = d2 & 0xFFFFu;
                    dw[u][r + 1] = d2 >> 16;
                }
            } else if constexpr (PAIRS) {
#pragma unroll
                for (int r = 0; r < R; ++r) dw[u][r] = amv_ld_stream(wd + db[r] + 2 * j);
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    dw[u][r] = amv_ld_stream(wd + amv_q4_0_didx(min(mmv_row<EP>(wave, r, R, n_rows), n_rows - 1), j, nb, n_rows));
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = FULL ? j0 + 64 * u + lane : min(j0 + 64 * u + lane, nb - 1);
            a0[u] = a4[2 * j];
            a1[u] = a4[2 * j + 1];
            ads_u[u] = ads[j];
        }
        // every load of the step is in flight before the first dot product (the scheduler would otherwise sink some
        // of them below the arithmetic of the first rows)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + 64 * u + lane;
            if (FULL || j < nb) {
                const int2 ds = ads_u[u];
                const float da = __int_as_float(ds.x);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint4 q = w[u][r];
                    int s = amv_dot4((int)(q.x & M4), a0[u].x, 0);
                    s = amv_dot4((int)(q.y & M4), a0[u].y, s);
                    s = amv_dot4((int)(q.z & M4), a0[u].z, s);
                    s = amv_dot4((int)(q.w & M4), a0[u].w, s);
                    s = amv_dot4((int)((q.x >> 4) & M4), a1[u].x, s);
                    s = amv_dot4((int)((q.y >> 4) & M4), a1[u].y, s);
                    s = amv_dot4((int)((q.z >> 4) & M4), a1[u].z, s);
                    s = amv_dot4((int)((q.w >> 4) & M4), a1[u].w, s);
                    s -= 8 * ds.y;
                    if (BLOCK_SUMS) {
                        if (mmv_row<EP>(wave, r, R, n_rows) < n_rows) sums[(size_t)mmv_row<EP>(wave, r, R, n_rows) * nb + j] = s;
                    } else {
                        acc[r] = fmaf((float)s, amv_h2f(dw[u][r]) * da, acc[r]);
                    }
                }
            }
        }
    } while ((j0 += 64 * U * S) < nb);
    if constexpr (!BLOCK_SUMS) {
        mmv_finish<R, EP, S, SEG>(acc, lane, wi, ks, live, wave, n_rows, dst, epi, eout, post, ra);
        if constexpr (MMV_TAIL(EP)) mmv_tail<EP, S, R>(post, eout, n_rows);
    }
}

// The plain Q4_0 GEMV at K = 4096 (128 blocks per row; every q/k/v/o and gate/up GEMV of Llama-3-8B), one column, no
// epilogue, even row count: two rows per wave, each lane's two blocks of both rows and their scales issued first, then
// its activation blocks, then the arithmetic; one wave-uniform sum per row. Same arithmetic and summation order as
// k_mmv_q4_0<2, 2, ...> (bit-identical results); measured on MI355X as the faster build of the same work (14336 x
// 4096 cold: 6.72 against 6.95 us).
__global__ __launch_bounds__(256) void k_mmv_q4_0_k4096(const uint4* __restrict__ wq, const uint32_t* __restrict__ wd2,
                                                       int n_rows, const int4* __restrict__ a4,
                                                       const int2* __restrict__ ads, float* __restrict__ dst) {
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6;
    const int row0 = min((int)(blockIdx.x * 4 + wi) * 2, n_rows - 2);  // a wave past the end re-reads the last pair
    const bool live = (int)(blockIdx.x * 4 + wi) * 2 < n_rows;
    uint4 w[2][2];
    uint32_t dw[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
#pragma unroll
        for (int r = 0; r < 2; ++r) w[u][r] = amv_ld_stream(wq + (size_t)(row0 + r) * 128 + j);
        dw[u] = amv_ld_stream(wd2 + (size_t)(row0 >> 1) * 128 + j);
    }
    int4 a0[2], a1[2];
    int2 ds[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
        a0[u] = a4[2 * j];
        a1[u] = a4[2 * j + 1];
        ds[u] = ads[j];
    }
    float acc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float da = __int_as_float(ds[u].x);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint4 q = w[u][r];
            int s = amv_dot4((int)(q.x & M4), a0[u].x, 0);
            s = amv_dot4((int)(q.y & M4), a0[u].y, s);
            s = amv_dot4((int)(q.z & M4), a0[u].z, s);
            s = amv_dot4((int)(q.w & M4), a0[u].w, s);
            s = amv_dot4((int)((q.x >> 4) & M4), a1[u].x, s);
            s = amv_dot4((int)((q.y >> 4) & M4), a1[u].y, s);
            s = amv_dot4((int)((q.z >> 4) & M4), a1[u].z, s);
            s = amv_dot4((int)((q.w >> 4) & M4), a1[u].w, s);
            s -= 8 * ds[u].y;
            acc[r] = fmaf((float)s, amv_h2f(r ? dw[u] >> 16 : dw[u]) * da, acc[r]);
        }
    }
    const float t0 = amv_wave_sum(acc[0]), t1 = amv_wave_sum(acc[1]);
    if (live && lane < 2) dst[row0 + lane] = lane ? t1 : t0;
}

// Measurement instrumentation (amv_debug_gemv_read_probe): k_mmv_q4_0_k4096's grid, wave-to-row mapping and weight /
// scale loads (non-temporal, all issued first), without the activation loads and the dot products: each wave folds
// its weight bits with XOR and writes one word per row, so no load is dropped. The time of this kernel is the read
// ceiling of the mapping the headline GEMV streams with. LOAD = false keeps the grid and the stores and drops the
// loads: the fixed cost of launching and draining that grid.
template <bool LOAD>
__global__ __launch_bounds__(256) void k_gemv_read_probe(const uint4* __restrict__ wq, const uint32_t* __restrict__ wd2,
                                                        int n_rows, uint32_t* __restrict__ dst) {
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6;
    const int row0 = min((int)(blockIdx.x * 4 + wi) * 2, n_rows - 2);
    const bool live = (int)(blockIdx.x * 4 + wi) * 2 < n_rows;
    if constexpr (!LOAD) {
        if (live && lane < 2) dst[row0 + lane] = (uint32_t)(row0 + lane);
        return;
    }
    uint4 w[2][2];
    uint32_t dw[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
#pragma unroll
        for (int r = 0; r < 2; ++r) w[u][r] = amv_ld_stream(wq + (size_t)(row0 + r) * 128 + j);
        dw[u] = amv_ld_stream(wd2 + (size_t)(row0 >> 1) * 128 + j);
    }
    uint32_t x[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        x[r] = dw[0] ^ dw[1];
#pragma unroll
        for (int u = 0; u < 2; ++u) x[r] ^= w[u][r].x ^ w[u][r].y ^ w[u][r].z ^ w[u][r].w;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) x[r] ^= (uint32_t)__shfl_xor((int)x[r], o, AMV_WAVE);
    }
    if (live && lane < 2) dst[row0 + lane] = lane ? x[1] : x[0];
}

extern "C" int amv_debug_gemv_read_probe(const void* w, int64_t n_rows, int64_t k, uint32_t* dst, int loads,
                                         void* stream) {
    AMV_REQUIRE(w && dst, "amv_debug_gemv_read_probe: null pointer");
    AMV_REQUIRE(loads == 0 || loads == 1, "amv_debug_gemv_read_probe: loads must be 0 or 1");
    AMV_REQUIRE(k == 4096 && n_rows >= 2 && n_rows % 2 == 0 && n_rows <= (1 << 24),
                "amv_debug_gemv_read_probe: the headline kernel's shapes (k = 4096, even n_rows)");
    AMV_REQUIRE(((uintptr_t)w & 15) == 0, "amv_debug_gemv_read_probe: w must be 16-byte aligned");
    const uint4* wq = reinterpret_cast<const uint4*>(w);
    const uint32_t* wd2 = reinterpret_cast<const uint32_t*>((const uint8_t*)w + (size_t)n_rows * 128 * 16);
    const int waves = (int)(n_rows / 2);
    if (loads)
        hipLaunchKernelGGL(k_gemv_read_probe<true>, dim3((waves + 3) / 4), dim3(256), 0, amv_stream(stream), wq, wd2,
                           (int)n_rows, dst);
    else
        hipLaunchKernelGGL(k_gemv_read_probe<false>, dim3((waves + 3) / 4), dim3(256), 0, amv_stream(stream), wq, wd2,
                           (int)n_rows, dst);
    return amv_check_launch("amv_debug_gemv_read_probe");
}

// The stacked gate|up GEMV at K = 4096 with SWIGLU and the Q8 tail (EP 7) in the same lean form: two outputs per
// wave, rows o, o + 1 (gate) and F + o, F + o + 1 (up) with o = 2 wave, the scales of each row pair in one dword, every
// load of the wave issued before its arithmetic; the per-lane sums in the order of k_mmv_q4_0 (same bits). Measured on
// MI355X at 28672 x 4096 against the generic stacked kernel: see the launcher.
// SEG: gate and up are two matrices of F rows each (w_seg[0], w_seg[1] in their own layouts: llama.cpp's separate
// ffn_gate / ffn_up), the wave's rows o, o + 1 of both.
template <bool SEG>
__global__ __launch_bounds__(256) void k_mmv_q4_0_k4096_swiglu(const uint4* __restrict__ wq,
                                                               const uint32_t* __restrict__ wd2, int n_rows,
                                                               const int4* __restrict__ a4,
                                                               const int2* __restrict__ ads, float* __restrict__ dst,
                                                               float* __restrict__ eout, const MmvPost post) {
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6;
    const int wave = blockIdx.x * 4 + wi;
    const int F = n_rows >> 1;
    const bool live = 2 * wave < F;
    const int o = min(2 * wave, F - 2);  // a wave past the end re-reads the last pair and stores nothing
    // gate rows o, o + 1 at wg / dg, up rows at wu / du (row ou, ou + 1 of that matrix)
    const uint4* wg = wq;
    const uint4* wu = wq;
    const uint32_t* dg = wd2;
    const uint32_t* du = wd2;
    int ou = F + o;
    if constexpr (SEG) {
        wg = reinterpret_cast<const uint4*>(post.w_seg[0]);
        wu = reinterpret_cast<const uint4*>(post.w_seg[1]);
        dg = reinterpret_cast<const uint32_t*>(post.w_seg[0] + (size_t)F * 128 * 16);
        du = reinterpret_cast<const uint32_t*>(post.w_seg[1] + (size_t)F * 128 * 16);
        ou = o;
    }
    uint4 w[2][4];
    uint32_t dw[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
        w[u][0] = amv_ld_stream(wg + (size_t)o * 128 + j);
        w[u][1] = amv_ld_stream(wg + (size_t)(o + 1) * 128 + j);
        w[u][2] = amv_ld_stream(wu + (size_t)ou * 128 + j);
        w[u][3] = amv_ld_stream(wu + (size_t)(ou + 1) * 128 + j);
        dw[u][0] = amv_ld_stream(dg + (size_t)(o >> 1) * 128 + j);
        dw[u][1] = amv_ld_stream(du + (size_t)(ou >> 1) * 128 + j);
    }
    int4 a0[2], a1[2];
    int2 ds[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
        a0[u] = a4[2 * j];
        a1[u] = a4[2 * j + 1];
        ds[u] = ads[j];
    }
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float da = __int_as_float(ds[u].x);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint4 q = w[u][r];
            int s = amv_dot4((int)(q.x & M4), a0[u].x, 0);
            s = amv_dot4((int)(q.y & M4), a0[u].y, s);
            s = amv_dot4((int)(q.z & M4), a0[u].z, s);
            s = amv_dot4((int)(q.w & M4), a0[u].w, s);
            s = amv_dot4((int)((q.x >> 4) & M4), a1[u].x, s);
            s = amv_dot4((int)((q.y >> 4) & M4), a1[u].y, s);
            s = amv_dot4((int)((q.z >> 4) & M4), a1[u].z, s);
            s = amv_dot4((int)((q.w >> 4) & M4), a1[u].w, s);
            s -= 8 * ds[u].y;
            const uint32_t d2 = dw[u][r >> 1];
            acc[r] = fmaf((float)s, amv_h2f((r & 1) ? d2 >> 16 : d2) * da, acc[r]);
        }
    }
    mmv_finish<4, MMV_EP_SWIGLU_Q8, 1>(acc, lane, wi, 0, live, wave, n_rows, dst, nullptr, eout, post, MmvRopeAt{});
    mmv_tail<MMV_EP_SWIGLU_Q8, 1, 4>(post, eout, n_rows);
}

// The K = 4096 GEMV with the ADD (o projection + residual) or ROPE_KV (q/k/v + RoPE + cache rows) epilogue in the same
// lean form, two rows per wave; SEG: the rows' matrix from the segment table (each holds an even row count, so a
// wave's pair lies in one). Same sums as k_mmv_q4_0<2, 2, ...>.
template <int EP, bool SEG>
__global__ __launch_bounds__(256) void k_mmv_q4_0_k4096_ep(const uint4* __restrict__ wq,
                                                           const uint32_t* __restrict__ wd2, int n_rows,
                                                           const int4* __restrict__ a4, const int2* __restrict__ ads,
                                                           float* __restrict__ dst, const float* __restrict__ epi,
                                                           float* __restrict__ eout, const MmvPost post) {
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6;
    const int wave = blockIdx.x * 4 + wi;
    const bool live = 2 * wave < n_rows;
    const MmvRopeAt ra = mmv_rope_at<EP>(post, wave);
    int row0 = min(2 * wave, n_rows - 2);  // a wave past the end re-reads the last pair and stores nothing
    const uint4* wqs = wq;
    const uint32_t* wds = wd2;
    if constexpr (SEG) {
        int lr;
        const int sg = mmv_seg(post, row0, lr);
        const size_t rows_s = (size_t)(mmv_seg_first(post, sg + 1) - mmv_seg_first(post, sg));
        wqs = reinterpret_cast<const uint4*>(mmv_seg_w(post, sg));
        wds = reinterpret_cast<const uint32_t*>(mmv_seg_w(post, sg) + rows_s * 128 * 16);
        row0 = lr;
    }
    uint4 w[2][2];
    uint32_t dw[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
#pragma unroll
        for (int r = 0; r < 2; ++r) w[u][r] = amv_ld_stream(wqs + (size_t)(row0 + r) * 128 + j);
        dw[u] = amv_ld_stream(wds + (size_t)(row0 >> 1) * 128 + j);
    }
    int4 a0[2], a1[2];
    int2 ds[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
        a0[u] = a4[2 * j];
        a1[u] = a4[2 * j + 1];
        ds[u] = ads[j];
    }
    float acc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float da = __int_as_float(ds[u].x);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint4 q = w[u][r];
            int s = amv_dot4((int)(q.x & M4), a0[u].x, 0);
            s = amv_dot4((int)(q.y & M4), a0[u].y, s);
            s = amv_dot4((int)(q.z & M4), a0[u].z, s);
            s = amv_dot4((int)(q.w & M4), a0[u].w, s);
            s = amv_dot4((int)((q.x >> 4) & M4), a1[u].x, s);
            s = amv_dot4((int)((q.y >> 4) & M4), a1[u].y, s);
            s = amv_dot4((int)((q.z >> 4) & M4), a1[u].z, s);
            s = amv_dot4((int)((q.w >> 4) & M4), a1[u].w, s);
            s -= 8 * ds[u].y;
            acc[r] = fmaf((float)s, amv_h2f(r ? dw[u] >> 16 : dw[u]) * da, acc[r]);
        }
    }
    mmv_finish<2, EP, 1, SEG>(acc, lane, wi, 0, live, wave, n_rows, dst, epi, eout, post, ra);
}

// The lean K = 4096 GEMVs with the RMS_NORM before them folded in: every workgroup of NT threads computes
// RMS_NORM(x) * norm_w and its Q8_0 quantization into LDS (amv_rms1024_*: k_rms_norm's arithmetic, the same bytes
// as the activation that launch writes) instead of reading an activation written by a launch of its own, while its
// weight rows stream in; then the dot products of k_mmv_q4_0_k4096_swiglu (EP 7: stacked gate|up + SWIGLU + Q8_0 of
// the result, P outputs per wave) or k_mmv_q4_0_k4096_ep (EP 5: q/k/v + ROPE + cache rows, two rows per wave) with the
// activation read from LDS: the same sums in the same order, so the same bits as the norm launch followed by the
// plain lean kernel. Every wave issues its share of the row before any wave of the workgroup issues a weight load
// (a barrier between them): a CU's vector memory returns its loads in order, so a row load queued behind weight
// loads would wait for the weights (measured with per-wave timestamps: ~2 us at p90) and the norm would run after
// them instead of under them. Sized for one workgroup per CU (NT = 1024; 192 and 224 workgroups for the Llama-3-8B
// q/k/v and gate/up). EP 7 with NW P a multiple of 32: each workgroup owns whole Q8_0 blocks of the SWIGLU output and
// quantizes them from LDS after a barrier, no arrival counters (k_mmv_q4_0_k4096_swiglu's values and rules).
template <int NT, int EP, bool SEG, int P, int RULE>
__global__ __launch_bounds__(NT) void k_mmv_q4_0_k4096_norm(const float4* __restrict__ x4,
                                                            const float4* __restrict__ nw4, float eps,
                                                            const uint4* __restrict__ wq,
                                                            const uint32_t* __restrict__ wd2, int n_rows,
                                                            float* __restrict__ dst, float* __restrict__ eout,
                                                            const MmvPost post) {
    constexpr int NW = NT / 64;
    constexpr bool SW = EP == MMV_EP_SWIGLU_Q8;
    constexpr int R = SW ? 2 * P : 2;
    constexpr bool WG_TAIL = SW && (NW * P) % 32 == 0;
    static_assert(SW || EP == MMV_EP_ROPE_KV, "EP 5 or EP 7");
    static_assert(!SW || ((P == 2 || P == 4) && (WG_TAIL || 32 % (NW * P) == 0)),
                  "a workgroup's outputs are whole Q8_0 blocks or lie in one");
    __shared__ __align__(16) int8_t s_q[4096];
    __shared__ __align__(16) int2 s_m[128];
    __shared__ double sred[AMV_RMS_VLANES / 64];
    __shared__ __align__(16) float s_h[WG_TAIL ? NW * P : 4];
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6;
    const int wave = blockIdx.x * NW + wi;
    // the weight rows' addresses first (no memory access): the segment selects branch, and control flow between the
    // row loads and the barrier below lets the compiler move the barrier above the row loads
    bool live;
    const uint4* wg = wq;  // SW: gate rows o .. o + P - 1 and the same up rows; their scales in P / 2 row-pair dwords
    const uint4* wu = wq;
    const uint32_t* dg = wd2;
    const uint32_t* du = wd2;
    int o = 0, ou = 0;
    const uint4* wqs = wq;  // EP 5: rows row0, row0 + 1
    const uint32_t* wds = wd2;
    int row0 = 0;
    if constexpr (SW) {
        const int F = n_rows >> 1;
        live = P * wave < F;
        o = min(P * wave, F - P);  // a wave past the end re-reads the last rows and stores nothing
        ou = F + o;
        if constexpr (SEG) {
            wg = reinterpret_cast<const uint4*>(post.w_seg[0]);
            wu = reinterpret_cast<const uint4*>(post.w_seg[1]);
            dg = reinterpret_cast<const uint32_t*>(post.w_seg[0] + (size_t)F * 128 * 16);
            du = reinterpret_cast<const uint32_t*>(post.w_seg[1] + (size_t)F * 128 * 16);
            ou = o;
        }
    } else {
        live = 2 * wave < n_rows;
        row0 = min(2 * wave, n_rows - 2);
        if constexpr (SEG) {
            int lr;
            const int sg = mmv_seg(post, row0, lr);
            const size_t rows_s = (size_t)(mmv_seg_first(post, sg + 1) - mmv_seg_first(post, sg));
            wqs = reinterpret_cast<const uint4*>(mmv_seg_w(post, sg));
            wds = reinterpret_cast<const uint32_t*>(mmv_seg_w(post, sg) + rows_s * 128 * 16);
            row0 = lr;
        }
    }
    AmvRms1024<NT> nr;
    amv_rms1024_load<NT>(x4, nw4, nr);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();  // issue order only: no wait for the loads
    __builtin_amdgcn_sched_barrier(0);
    uint4 w[2][R];
    uint32_t dw[2][R / 2];
    if constexpr (SW) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int j = 64 * u + lane;
#pragma unroll
            for (int i = 0; i < P; ++i) {
                w[u][i] = amv_ld_stream(wg + (size_t)(o + i) * 128 + j);
                w[u][P + i] = amv_ld_stream(wu + (size_t)(ou + i) * 128 + j);
            }
#pragma unroll
            for (int q = 0; q < P / 2; ++q) {
                dw[u][q] = amv_ld_stream(dg + (size_t)((o >> 1) + q) * 128 + j);
                dw[u][P / 2 + q] = amv_ld_stream(du + (size_t)((ou >> 1) + q) * 128 + j);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int j = 64 * u + lane;
#pragma unroll
            for (int r = 0; r < 2; ++r) w[u][r] = amv_ld_stream(wqs + (size_t)(row0 + r) * 128 + j);
            dw[u][0] = amv_ld_stream(wds + (size_t)(row0 >> 1) * 128 + j);
        }
    }
    // the norm's arithmetic waits for the row only; everything after it for the weights too
    __builtin_amdgcn_sched_barrier(0);
    const MmvRopeAt ra = mmv_rope_at<EP>(post, wave);
    amv_rms1024_quant_t<NT, AMV_T_Q8_0, RULE>(nr, eps, s_q, s_m, nullptr, sred);
    __syncthreads();
    int4 a0[2], a1[2];
    int2 ds[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
        a0[u] = reinterpret_cast<const int4*>(s_q)[2 * j];
        a1[u] = reinterpret_cast<const int4*>(s_q)[2 * j + 1];
        ds[u] = s_m[j];
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float da = __int_as_float(ds[u].x);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint4 q = w[u][r];
            int s = amv_dot4((int)(q.x & M4), a0[u].x, 0);
            s = amv_dot4((int)(q.y & M4), a0[u].y, s);
            s = amv_dot4((int)(q.z & M4), a0[u].z, s);
            s = amv_dot4((int)(q.w & M4), a0[u].w, s);
            s = amv_dot4((int)((q.x >> 4) & M4), a1[u].x, s);
            s = amv_dot4((int)((q.y >> 4) & M4), a1[u].y, s);
            s = amv_dot4((int)((q.z >> 4) & M4), a1[u].z, s);
            s = amv_dot4((int)((q.w >> 4) & M4), a1[u].w, s);
            s -= 8 * ds[u].y;
            const uint32_t d2 = dw[u][r >> 1];
            acc[r] = fmaf((float)s, amv_h2f((r & 1) ? d2 >> 16 : d2) * da, acc[r]);
        }
    }
    if constexpr (WG_TAIL) {
        const int F = n_rows >> 1;
        float t[R];
#pragma unroll
        for (int r = 0; r < R; ++r) t[r] = amv_wave_sum(acc[r]);
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int o = P * wave + i;
                if (o >= F) break;
                if (dst) {
                    dst[o] = t[i];
                    dst[o + F] = t[P + i];
                }
                const float h = mmv_silu(t[i]) * t[P + i];
                eout[o] = h;
                s_h[P * wi + i] = h;
            }
        }
        __syncthreads();
        constexpr int NQ = NW * P / 4;  // chunks of 4 outputs in the workgroup: whole 8-lane Q8_0 blocks
        const int c = (int)blockIdx.x * NQ + (int)threadIdx.x;
        if (threadIdx.x < NQ && 4 * c < F) {  // whole blocks only (F % 32 == 0)
            const float4 v4 = reinterpret_cast<const float4*>(s_h)[threadIdx.x];
            const float v[4] = {v4.x, v4.y, v4.z, v4.w};
            q8_block_lanes8_r<RULE>(v, c & 7, post.act.qs + 32 * (c >> 3),
                                    reinterpret_cast<int2*>(post.act.meta) + (c >> 3));
        }
    } else {
        mmv_finish<R, EP, 1, SEG>(acc, lane, wi, 0, live, wave, n_rows, dst, nullptr, eout, post, ra);
        if constexpr (SW) mmv_tail<EP, 1, R, NW>(post, eout, n_rows);
    }
}

// ------------------------------------------------------------------------------------------------ Q8_0 x Q8_0
template <int R, int U, bool BLOCK_SUMS, int EP, int S>
__global__ __launch_bounds__(256) void k_mmv_q8_0(const uint4* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                 int n_rows, int nb, const int8_t* __restrict__ aq,
                                                 const int2* __restrict__ ads, float* __restrict__ dst,
                                                 int32_t* __restrict__ sums, const float* __restrict__ epi,
                                                 float* __restrict__ eout, const MmvPost post) {
    static_assert(!BLOCK_SUMS || S == 1, "block sums are written per block, without a split of K");
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6, ks = wi % S;
    const int wave = blockIdx.x * (4 / S) + wi / S;  // row group; the S waves of a group split K
    const bool live = mmv_wave_live<EP>(wave, R, n_rows);
    const MmvRopeAt ra = mmv_rope_at<EP>(post, wave);  // ROPE_KV
    if (S == 1 && !live && !MMV_TAIL(EP)) return;  // uniform per wave (tails need every wave)
    const int4* a4 = reinterpret_cast<const int4*>(aq);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int j0 = live ? 64 * U * ks : nb; j0 < nb; j0 += 64 * U * S) {
        uint4 w0[U][R], w1[U][R];
        uint16_t dw[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(j0 + 64 * u + lane, nb - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const size_t bi = (size_t)min(mmv_row<EP>(wave, r, R, n_rows), n_rows - 1) * nb + j;
                // each lane reads its block's 32 bytes in two halves: a line a wave touches twice must stay in L2,
                // so these loads are not streaming (measured: 14.2 us against 12.1 us at 14336 x 4096)
                w0[u][r] = wq[2 * bi];
                w1[u][r] = wq[2 * bi + 1];
                dw[u][r] = amv_ld_stream(wd + bi);
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
                        if (mmv_row<EP>(wave, r, R, n_rows) < n_rows) sums[(size_t)mmv_row<EP>(wave, r, R, n_rows) * nb + j] = s;
                    } else {
                        acc[r] = fmaf((float)s, amv_h2f(dw[u][r]) * da, acc[r]);
                    }
                }
            }
        }
    }
    if constexpr (!BLOCK_SUMS) {
        mmv_finish<R, EP, S>(acc, lane, wi, ks, live, wave, n_rows, dst, epi, eout, post, ra);
        if constexpr (MMV_TAIL(EP)) mmv_tail<EP, S, R>(post, eout, n_rows);
    }
}

// ------------------------------------------------------------------------------------------------ K-quants
// Q4_K and Q6_K rows are cut into 16-byte slices of their 4-bit data (k / 32 slices per row, 8 per 256-weight
// super-block), lane l taking slice l + 64 i. A Q4_K slice t of a super-block holds the low nibbles of weights
// 64c + 16h + (0..15) and the high nibbles of 64c + 32 + 16h + (0..15) (c = t / 2, h = t % 2), i.e. halves of
// units 2c and 2c + 1. A Q6_K slice holds ql bytes 16t .. 16t + 15 (weights 128hh + 32s + lq + (0..15) for
// s = s_lo and s_lo + 2), its two high bits come from 16 bytes of qh. Activations are Q8_K (one f32 scale per 256,
// int32 sums per 16, which also supply the constant offsets -32 (Q6_K) and the minima (Q4_K)).
// Per super-block ggml's vec_dot_q4_K_q8_K computes d*da*sum_u sc_u dot_u - dmin*da*sum_u m_u bsum_u and
// vec_dot_q6_K_q8_K d*da*sum_g sc_g dot(q6 - 32, qa)_g; the lanes form the same integers per slice.

__device__ __forceinline__ int dot16(uint4 w, int4 a, int acc) {
    acc = amv_dot4((int)w.x, a.x, acc);
    acc = amv_dot4((int)w.y, a.y, acc);
    acc = amv_dot4((int)w.z, a.z, acc);
    return amv_dot4((int)w.w, a.w, acc);
}

template <int R, bool BLOCK_SUMS, int EP, int S, bool SEG = false>
__global__ __launch_bounds__(256) void k_mmv_q4_K(const uint4* __restrict__ wq, const uint4* __restrict__ wh,
                                                 int n_rows, int nsl, const int8_t* __restrict__ aq,
                                                 const float* __restrict__ ad, const int* __restrict__ abs16,
                                                 float* __restrict__ dst, int32_t* __restrict__ sums, const float* __restrict__ epi,
                                                 float* __restrict__ eout, const MmvPost post) {
    static_assert(!BLOCK_SUMS || S == 1, "block sums are written per block, without a split of K");
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6, ks = wi % S;
    const int wave = blockIdx.x * (4 / S) + wi / S;  // row group; the S waves of a group split K
    const bool live = mmv_wave_live<EP>(wave, R, n_rows);
    const MmvRopeAt ra = mmv_rope_at<EP>(post, wave);  // ROPE_KV
    if (S == 1 && !live && !MMV_TAIL(EP)) return;  // uniform per wave (tails need every wave)
    const int nsb = nsl >> 3;
    const int4* a4 = reinterpret_cast<const int4*>(aq);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    // two 64-slice steps per pass, both steps' loads issued before either step's arithmetic (a wave's step-2 loads
    // would otherwise wait for its step-1 compute: two memory round trips in a row). A lane past the row's end
    // loads slice nsl - 1 and adds nothing; the steps add into acc in order, as one step per pass would.
    struct Step {
        uint4 q[R];
        uint32_t hv[R];  // dword lane & 3 of the super-block's 16-byte head (spread over the quad in compute)
        int4 alo, ahi;
        float da;
        int bslo, bshi;
        int j, sb, c, t;
        bool valid;
    };
    const auto load = [&](int j0, Step& st) {
        st.valid = j0 + lane < nsl;
        const int j = min(j0 + lane, nsl - 1);  // nsl is a multiple of 8: clamped lanes fill whole groups of 8
        const int sb = j >> 3, t = j & 7, c = t >> 1, h = t & 1;
        st.j = j;
        st.sb = sb;
        st.c = c;
        st.t = t;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int row = min(mmv_row<EP>(wave, r, R, n_rows), n_rows - 1);
            const uint4* wqs = wq;
            const uint4* whs = wh;
            if constexpr (SEG) {  // the row's matrix: qs of its rows, then their 16-byte heads
                int lr;
                const int sg = mmv_seg(post, row, lr);
                wqs = reinterpret_cast<const uint4*>(mmv_seg_w(post, sg));
                whs = wqs + (size_t)(mmv_seg_first(post, sg + 1) - mmv_seg_first(post, sg)) * nsl;
                row = lr;
            }
            st.q[r] = amv_ld_stream(wqs + (size_t)row * nsl + j);
            // the super-block's 16-byte head: each lane of a quad loads one dword (the quad shares the super-block:
            // groups of 8 lanes do, clamped lanes included); compute hands every lane all four by DPP (no arithmetic
            // on a loaded value here, or the compiler waits for the loads at this point)
            st.hv[r] = amv_ld_stream(reinterpret_cast<const uint32_t*>(whs + (size_t)row * nsb + sb) + (lane & 3));
        }
        st.alo = a4[sb * 16 + 4 * c + h];
        st.ahi = a4[sb * 16 + 4 * c + 2 + h];
        st.da = ad[sb];
        st.bslo = abs16[sb * 16 + 4 * c + h];
        st.bshi = abs16[sb * 16 + 4 * c + 2 + h];
    };
    const auto compute = [&](const Step& st) {
        const int sb = st.sb, c = st.c, t = st.t;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t hv = st.hv[r];
            const uint4 hd = make_uint4(__builtin_amdgcn_mov_dpp(hv, 0x00, 0xF, 0xF, false),   // quad_perm [0,0,0,0]
                                        __builtin_amdgcn_mov_dpp(hv, 0x55, 0xF, 0xF, false),   // [1,1,1,1]
                                        __builtin_amdgcn_mov_dpp(hv, 0xAA, 0xF, 0xF, false),   // [2,2,2,2]
                                        __builtin_amdgcn_mov_dpp(hv, 0xFF, 0xF, 0xF, false));  // [3,3,3,3]
            int sl, ml, sh, mh;
            k4_scale_min_pair(c, hd.y, hd.z, hd.w, sl, ml, sh, mh);
            const uint4 q = st.q[r];
            const uint4 lo = make_uint4(q.x & M4, q.y & M4, q.z & M4, q.w & M4);
            const uint4 hi = make_uint4((q.x >> 4) & M4, (q.y >> 4) & M4, (q.z >> 4) & M4, (q.w >> 4) & M4);
            int isum = sl * dot16(lo, st.alo, 0) + sh * dot16(hi, st.ahi, 0);
            int msum = ml * st.bslo + mh * st.bshi;
            if (BLOCK_SUMS) {
#pragma unroll
                for (int o = 1; o < 8; o <<= 1) {
                    isum += __shfl_xor(isum, o, AMV_WAVE);
                    msum += __shfl_xor(msum, o, AMV_WAVE);
                }
                const int rr = mmv_row<EP>(wave, r, R, n_rows);
                if (t == 0 && st.valid && rr < n_rows) {
                    sums[((size_t)rr * nsb + sb) * 2] = isum;
                    sums[((size_t)rr * nsb + sb) * 2 + 1] = msum;
                }
            } else if (st.valid) {
                const float d = amv_h2f(hd.x) * st.da, dmin = amv_h2f(hd.x >> 16) * st.da;
                acc[r] = fmaf(d, (float)isum, acc[r]);
                acc[r] = fmaf(-dmin, (float)msum, acc[r]);
            }
        }
    };
    for (int j0 = live ? 64 * ks : nsl; j0 < nsl; j0 += 128 * S) {
        Step s0, s1;
        load(j0, s0);
        load(j0 + 64 * S, s1);
        compute(s0);
        compute(s1);
    }
    if constexpr (!BLOCK_SUMS) {
        mmv_finish<R, EP, S, SEG>(acc, lane, wi, ks, live, wave, n_rows, dst, epi, eout, post, ra);
        if constexpr (MMV_TAIL(EP)) mmv_tail<EP, S, R>(post, eout, n_rows);
    }
}

// k_mmv_q4_K at K = 4096 (S = 1) with the RMS_NORM before it folded in, as k_mmv_q4_0_k4096_norm: every workgroup
// of NT threads issues its share of the row x and the norm weight, then (after a barrier, so that no row load waits
// behind a weight load of the CU) every weight slice and super-block head of its waves (both 64-slice steps), then
// computes RMS_NORM(x) * norm_w and its Q8_K quantization into LDS (amv_rms1024_*: k_rms_norm's bytes) while the
// weights stream in, and dots them in k_mmv_q4_K's order: the same bits as the norm launch followed by that kernel.
// EP 5 (q/k/v + ROPE + cache rows) or EP 7 (stacked gate|up + SWIGLU + Q8_K tail, one output per wave with R = 2).
template <int NT, int EP, bool SEG, int R = 2>
__global__ __launch_bounds__(NT) void k_mmv_q4_K_norm(const float4* __restrict__ x4, const float4* __restrict__ nw4,
                                                      float eps, const uint4* __restrict__ wq,
                                                      const uint4* __restrict__ wh, int n_rows,
                                                      float* __restrict__ dst, float* __restrict__ eout,
                                                      const MmvPost post) {
    constexpr int NW = NT / 64, NSL = 128, NSB = 16;  // K = 4096: 16-byte weight slices and super-blocks per row
    static_assert(EP == MMV_EP_ROPE_KV || EP == MMV_EP_SWIGLU_Q8, "EP 5 or EP 7");
    __shared__ __align__(16) int8_t s_q[4096];
    __shared__ __align__(16) float s_d[NSB];
    __shared__ __align__(16) int32_t s_s16[256];
    __shared__ double sred[AMV_RMS_VLANES / 64];
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6;
    const int wave = blockIdx.x * NW + wi;
    const bool live = mmv_wave_live<EP>(wave, R, n_rows);
    // the weight rows' addresses first (no memory access): the segment selects branch, and control flow between the
    // row loads and the barrier below lets the compiler move the barrier above the row loads
    int rows[R];
    const uint4* wqs[R];
    const uint4* whs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rows[r] = min(mmv_row<EP>(wave, r, R, n_rows), n_rows - 1);
        wqs[r] = wq;
        whs[r] = wh;
        if constexpr (SEG) {  // the row's matrix: qs of its rows, then their 16-byte heads
            int lr;
            const int sg = mmv_seg(post, rows[r], lr);
            wqs[r] = reinterpret_cast<const uint4*>(mmv_seg_w(post, sg));
            whs[r] = wqs[r] + (size_t)(mmv_seg_first(post, sg + 1) - mmv_seg_first(post, sg)) * NSL;
            rows[r] = lr;
        }
    }
    AmvRms1024<NT> nr;
    amv_rms1024_load<NT>(x4, nw4, nr);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();  // issue order only: no wait for the loads
    __builtin_amdgcn_sched_barrier(0);
    uint4 q[2][R];
    uint32_t hv[2][R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int j = 64 * u + lane, sb = j >> 3;
            q[u][r] = amv_ld_stream(wqs[r] + (size_t)rows[r] * NSL + j);
            hv[u][r] =
                amv_ld_stream(reinterpret_cast<const uint32_t*>(whs[r] + (size_t)rows[r] * NSB + sb) + (lane & 3));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const MmvRopeAt ra = mmv_rope_at<EP>(post, wave);
    amv_rms1024_quant_t<NT, AMV_T_Q8_K, 0>(nr, eps, s_q, s_d, s_s16, sred);
    __syncthreads();
    const int4* a4 = reinterpret_cast<const int4*>(s_q);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = 64 * u + lane;
        const int sb = j >> 3, t = j & 7, c = t >> 1, h = t & 1;
        const int4 alo = a4[sb * 16 + 4 * c + h], ahi = a4[sb * 16 + 4 * c + 2 + h];
        const float da = s_d[sb];
        const int bslo = s_s16[sb * 16 + 4 * c + h], bshi = s_s16[sb * 16 + 4 * c + 2 + h];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // the super-block head: lane l of each quad loaded dword l, DPP hands every lane all four
            const uint32_t h0 = hv[u][r];
            const uint4 hd = make_uint4(__builtin_amdgcn_mov_dpp(h0, 0x00, 0xF, 0xF, false),
                                        __builtin_amdgcn_mov_dpp(h0, 0x55, 0xF, 0xF, false),
                                        __builtin_amdgcn_mov_dpp(h0, 0xAA, 0xF, 0xF, false),
                                        __builtin_amdgcn_mov_dpp(h0, 0xFF, 0xF, 0xF, false));
            int sl, ml, sh, mh;
            k4_scale_min_pair(c, hd.y, hd.z, hd.w, sl, ml, sh, mh);
            const uint4 w = q[u][r];
            const uint4 lo = make_uint4(w.x & M4, w.y & M4, w.z & M4, w.w & M4);
            const uint4 hi = make_uint4((w.x >> 4) & M4, (w.y >> 4) & M4, (w.z >> 4) & M4, (w.w >> 4) & M4);
            const int isum = sl * dot16(lo, alo, 0) + sh * dot16(hi, ahi, 0);
            const int msum = ml * bslo + mh * bshi;
            const float d = amv_h2f(hd.x) * da, dmin = amv_h2f(hd.x >> 16) * da;
            acc[r] = fmaf(d, (float)isum, acc[r]);
            acc[r] = fmaf(-dmin, (float)msum, acc[r]);
        }
    }
    mmv_finish<R, EP, 1, SEG>(acc, lane, wi, 0, live, wave, n_rows, dst, nullptr, eout, post, ra);
    if constexpr (EP == MMV_EP_SWIGLU_Q8) mmv_tail<EP, 1, R, NW>(post, eout, n_rows);
}

template <int R, bool BLOCK_SUMS, int EP, int S>
__global__ __launch_bounds__(256) void k_mmv_q6_K(const uint4* __restrict__ wl, const uint4* __restrict__ wqh,
                                                 const uint4* __restrict__ wsc, const uint16_t* __restrict__ wd,
                                                 int n_rows, int nsl, const int8_t* __restrict__ aq,
                                                 const float* __restrict__ ad, const int* __restrict__ abs16,
                                                 float* __restrict__ dst, int32_t* __restrict__ sums, const float* __restrict__ epi,
                                                 float* __restrict__ eout, const MmvPost post) {
    static_assert(!BLOCK_SUMS || S == 1, "block sums are written per block, without a split of K");
    const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6, ks = wi % S;
    const int wave = blockIdx.x * (4 / S) + wi / S;  // row group; the S waves of a group split K
    const bool live = mmv_wave_live<EP>(wave, R, n_rows);
    const MmvRopeAt ra = mmv_rope_at<EP>(post, wave);  // ROPE_KV
    if (S == 1 && !live && !MMV_TAIL(EP)) return;  // uniform per wave (tails need every wave)
    const int nsb = nsl >> 3;
    const int4* a4 = reinterpret_cast<const int4*>(aq);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    // two 64-slice steps per pass, both steps' loads issued before either step's arithmetic (as k_mmv_q4_K)
    struct Step {
        uint4 ql[R], qh[R], sc[R];
        uint16_t dd[R];
        int4 alo, ahi;
        float da;
        int blo, bhi;
        int sb, t, slo, glo;
        bool valid;
    };
    const auto load = [&](int j0, Step& st) {
        st.valid = j0 + lane < nsl;
        const int j = min(j0 + lane, nsl - 1);
        const int sb = j >> 3, t = j & 7;
        const int hh = t >> 2, l0 = 16 * (t & 3);  // ql byte offset 64 hh + l0
        const int slo = l0 >> 5, lq = l0 & 31;      // weights 128 hh + 32 s + lq + i, s in {slo, slo + 2}
        st.sb = sb;
        st.t = t;
        st.slo = slo;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t rw = (size_t)min(mmv_row<EP>(wave, r, R, n_rows), n_rows - 1);
            const size_t rb = rw * nsb + sb;
            st.ql[r] = amv_ld_stream(wl + rw * nsl + j);
            st.qh[r] = amv_ld_stream(wqh + rb * 4 + 2 * hh + (lq >> 4));
            st.sc[r] = amv_ld_stream(wsc + rb);
            st.dd[r] = amv_ld_stream(wd + rb);
        }
        const int elo = 128 * hh + 32 * slo + lq;  // element offset in the super-block
        st.alo = a4[(sb * 256 + elo) >> 4];
        st.ahi = a4[(sb * 256 + elo + 64) >> 4];
        st.da = ad[sb];
        const int glo = elo >> 4, ghi = glo + 4;
        st.glo = glo;
        st.blo = abs16[sb * 16 + glo];
        st.bhi = abs16[sb * 16 + ghi];
    };
    const auto compute = [&](const Step& st) {
        const int sb = st.sb, t = st.t, glo = st.glo, ghi = glo + 4;
        const int shlo = 2 * st.slo, shhi = 2 * st.slo + 4;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint4 L = st.ql[r], H = st.qh[r];
            const uint4 vlo = make_uint4((L.x & M4) | (((H.x >> shlo) & 0x03030303u) << 4),
                                         (L.y & M4) | (((H.y >> shlo) & 0x03030303u) << 4),
                                         (L.z & M4) | (((H.z >> shlo) & 0x03030303u) << 4),
                                         (L.w & M4) | (((H.w >> shlo) & 0x03030303u) << 4));
            const uint4 vhi = make_uint4(((L.x >> 4) & M4) | (((H.x >> shhi) & 0x03030303u) << 4),
                                         ((L.y >> 4) & M4) | (((H.y >> shhi) & 0x03030303u) << 4),
                                         ((L.z >> 4) & M4) | (((H.z >> shhi) & 0x03030303u) << 4),
                                         ((L.w >> 4) & M4) | (((H.w >> shhi) & 0x03030303u) << 4));
            const uint32_t scw[4] = {st.sc[r].x, st.sc[r].y, st.sc[r].z, st.sc[r].w};
            const int sclo = (int)(int8_t)((scw[glo >> 2] >> (8 * (glo & 3))) & 0xFFu);
            const int schi = (int)(int8_t)((scw[ghi >> 2] >> (8 * (ghi & 3))) & 0xFFu);
            int isum = sclo * (dot16(vlo, st.alo, 0) - 32 * st.blo) + schi * (dot16(vhi, st.ahi, 0) - 32 * st.bhi);
            if (BLOCK_SUMS) {
#pragma unroll
                for (int o = 1; o < 8; o <<= 1) isum += __shfl_xor(isum, o, AMV_WAVE);
                const int rr = mmv_row<EP>(wave, r, R, n_rows);
                if (t == 0 && st.valid && rr < n_rows) sums[(size_t)rr * nsb + sb] = isum;
            } else if (st.valid) {
                acc[r] = fmaf(amv_h2f(st.dd[r]) * st.da, (float)isum, acc[r]);
            }
        }
    };
    for (int j0 = live ? 64 * ks : nsl; j0 < nsl; j0 += 128 * S) {
        Step s0, s1;
        load(j0, s0);
        load(j0 + 64 * S, s1);
        compute(s0);
        compute(s1);
    }
    if constexpr (!BLOCK_SUMS) {
        mmv_finish<R, EP, S>(acc, lane, wi, ks, live, wave, n_rows, dst, epi, eout, post, ra);
        if constexpr (MMV_TAIL(EP)) mmv_tail<EP, S, R>(post, eout, n_rows);
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
    const float* epi;      // epilogue operand
    float* eout;           // epilogue output
    MmvPost post;          // EP 5..7
};

// Parity instrumentation (amv_debug_gemv_generic): while set, the Q4_0 launches skip the lean K = 4096 kernels and run
// the generic k_mmv_q4_0 of the same rows per wave, split and epilogue, whose BLOCK_SUMS instantiation gives the
// block integers the tests compare with the oracle; the lean kernels keep that kernel's arithmetic and summation
// order, so the two f32 results must be equal bit for bit.
static std::atomic<int> g_mmv_generic{0};
extern "C" int amv_debug_gemv_generic(int on) { return g_mmv_generic.exchange(on ? 1 : 0); }

template <int R, int U, bool BS, int EP, int S>
static void launch_q4_0(const MmvArgs& a, hipStream_t st) {
    const bool lean = g_mmv_generic.load(std::memory_order_relaxed) == 0;
    const int nb = a.k / 32;
    const int64_t nblk = (int64_t)a.n_rows * nb;
    const uint4* wq = reinterpret_cast<const uint4*>(a.w);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(a.w + nblk * 16);
    const int2* ads = reinterpret_cast<const int2*>(a.ameta0);
    const int8_t* aq = a.aq;
    const int waves = MMV_STACKED(EP) ? a.n_rows / R : (a.n_rows + R - 1) / R;
    const bool full = nb % (64 * U) == 0 && (MMV_STACKED(EP) || a.n_rows % R == 0);
    const dim3 grid((waves * S + 3) / 4);
    if constexpr (!BS && EP == MMV_EP_SWIGLU_Q8 && R == 4 && S == 1 && U == 2) {
        // K = 4096: the lean kernel, stacked or over the two matrices (each of n_rows / 2 rows)
        if (nb == 128 && lean) {
            if (a.post.n_seg == 2)
                hipLaunchKernelGGL(k_mmv_q4_0_k4096_swiglu<true>, grid, dim3(256), 0, st, nullptr, nullptr, a.n_rows,
                                   reinterpret_cast<const int4*>(aq), ads, a.dst, a.eout, a.post);
            else if (a.post.n_seg == 0)
                hipLaunchKernelGGL(k_mmv_q4_0_k4096_swiglu<false>, grid, dim3(256), 0, st, wq,
                                   reinterpret_cast<const uint32_t*>(wd), a.n_rows, reinterpret_cast<const int4*>(aq),
                                   ads, a.dst, a.eout, a.post);
            if (a.post.n_seg == 2 || a.post.n_seg == 0) return;
        }
    }
    if constexpr (!BS && (EP == MMV_EP_ROPE_KV || EP == AMV_EP_ADD) && R == 2 && S == 1 && U == 2) {
        // K = 4096: the lean kernel (stacked or segmented q/k/v; o projection + residual)
        if (nb == 128 && a.n_rows % 2 == 0 && lean) {
            if (a.post.n_seg > 0)
                hipLaunchKernelGGL((k_mmv_q4_0_k4096_ep<EP, true>), grid, dim3(256), 0, st, nullptr, nullptr, a.n_rows,
                                   reinterpret_cast<const int4*>(aq), ads, a.dst, a.epi, a.eout, a.post);
            else
                hipLaunchKernelGGL((k_mmv_q4_0_k4096_ep<EP, false>), grid, dim3(256), 0, st, wq,
                                   reinterpret_cast<const uint32_t*>(wd), a.n_rows, reinterpret_cast<const int4*>(aq),
                                   ads, a.dst, a.epi, a.eout, a.post);
            return;
        }
    }
    if constexpr (!BS && (EP == MMV_EP_ROPE_KV || EP == MMV_EP_SWIGLU_Q8)) {
        if (a.post.n_seg > 0) {  // separate matrices (the launcher checked whole steps and even rows per matrix)
            const uint4* w0 = reinterpret_cast<const uint4*>(a.post.w_seg[0]);
            if (nb == 128 && U == 2)
                hipLaunchKernelGGL((k_mmv_q4_0<R, U, BS, EP, S, true, true, 128, true>), grid, dim3(256), 0, st, w0,
                                   nullptr, a.n_rows, nb, aq, ads, a.dst, a.sums, a.epi, a.eout, a.post);
            else
                hipLaunchKernelGGL((k_mmv_q4_0<R, U, BS, EP, S, true, true, 0, true>), grid, dim3(256), 0, st, w0,
                                   nullptr, a.n_rows, nb, aq, ads, a.dst, a.sums, a.epi, a.eout, a.post);
            return;
        }
    }
    if (!BS && EP == AMV_EP_NONE && S == 1 && R == 2 && a.n_rows % 2 == 0 && nb == 128 && lean)
        hipLaunchKernelGGL(k_mmv_q4_0_k4096, grid, dim3(256), 0, st, wq, reinterpret_cast<const uint32_t*>(wd),
                           a.n_rows, reinterpret_cast<const int4*>(aq), ads, a.dst);
    else if (a.n_rows % 2 == 0 && full && nb == 128 && U == 2)
        hipLaunchKernelGGL((k_mmv_q4_0<R, U, BS, EP, S, true, true, 128>), grid, dim3(256), 0, st, wq, wd, a.n_rows, nb,
                           aq, ads, a.dst, a.sums, a.epi, a.eout, a.post);
    else if (a.n_rows % 2 == 0 && full)
        hipLaunchKernelGGL((k_mmv_q4_0<R, U, BS, EP, S, true, true>), grid, dim3(256), 0, st, wq, wd, a.n_rows, nb, aq,
                           ads, a.dst, a.sums, a.epi, a.eout, a.post);
    else if (a.n_rows % 2 == 0)
        hipLaunchKernelGGL((k_mmv_q4_0<R, U, BS, EP, S, true, false>), grid, dim3(256), 0, st, wq, wd, a.n_rows, nb,
                           aq, ads, a.dst, a.sums, a.epi, a.eout, a.post);
    else
        hipLaunchKernelGGL((k_mmv_q4_0<R, U, BS, EP, S, false, false>), grid, dim3(256), 0, st, wq, wd, a.n_rows, nb,
                           aq, ads, a.dst, a.sums, a.epi, a.eout, a.post);
}

template <int R, int U, bool BS, int EP, int S>
static void launch_q8_0(const MmvArgs& a, hipStream_t st) {
    const int nb = a.k / 32;
    const int64_t nblk = (int64_t)a.n_rows * nb;
    const uint4* wq = reinterpret_cast<const uint4*>(a.w);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(a.w + nblk * 32);
    const int2* ads = reinterpret_cast<const int2*>(a.ameta0);
    const int8_t* aq = a.aq;
    const int waves = MMV_STACKED(EP) ? a.n_rows / R : (a.n_rows + R - 1) / R;
    hipLaunchKernelGGL((k_mmv_q8_0<R, U, BS, EP, S>), dim3((waves * S + 3) / 4), dim3(256), 0, st, wq, wd, a.n_rows, nb, aq, ads,
                       a.dst, a.sums, a.epi, a.eout, a.post);
}

template <int R, bool BS, int EP, int S>
static void launch_q4_K(const MmvArgs& a, hipStream_t st) {
    const int nsl = a.k / 32, nsb = a.k / 256;
    const int64_t nblk = (int64_t)a.n_rows * nsb;
    const uint4* wq = reinterpret_cast<const uint4*>(a.w);
    const uint4* wh = reinterpret_cast<const uint4*>(a.w + nblk * 128);
    const int waves = MMV_STACKED(EP) ? a.n_rows / R : (a.n_rows + R - 1) / R;
    if constexpr (!BS && (EP == MMV_EP_ROPE_KV || EP == MMV_EP_SWIGLU_Q8)) {
        if (a.post.n_seg > 0) {  // separate matrices
            hipLaunchKernelGGL((k_mmv_q4_K<R, BS, EP, S, true>), dim3((waves * S + 3) / 4), dim3(256), 0, st,
                               reinterpret_cast<const uint4*>(a.post.w_seg[0]), nullptr, a.n_rows, nsl, a.aq,
                               (const float*)a.ameta0, (const int*)a.ameta1, a.dst, a.sums, a.epi, a.eout, a.post);
            return;
        }
    }
    hipLaunchKernelGGL((k_mmv_q4_K<R, BS, EP, S>), dim3((waves * S + 3) / 4), dim3(256), 0, st, wq, wh, a.n_rows, nsl, a.aq,
                       (const float*)a.ameta0, (const int*)a.ameta1, a.dst, a.sums, a.epi, a.eout, a.post);
}

template <int R, bool BS, int EP, int S>
static void launch_q6_K(const MmvArgs& a, hipStream_t st) {
    const int nsl = a.k / 32, nsb = a.k / 256;
    const int64_t nblk = (int64_t)a.n_rows * nsb;
    const uint4* wl = reinterpret_cast<const uint4*>(a.w);
    const uint4* wqh = reinterpret_cast<const uint4*>(a.w + nblk * 128);
    const uint4* wsc = reinterpret_cast<const uint4*>(a.w + nblk * 192);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(a.w + nblk * 208);
    const int waves = MMV_STACKED(EP) ? a.n_rows / R : (a.n_rows + R - 1) / R;
    hipLaunchKernelGGL((k_mmv_q6_K<R, BS, EP, S>), dim3((waves * S + 3) / 4), dim3(256), 0, st, wl, wqh, wsc, wd, a.n_rows, nsl,
                       a.aq, (const float*)a.ameta0, (const int*)a.ameta1, a.dst, a.sums, a.epi, a.eout, a.post);
}

// Split of K over the S waves of a row group (S = 1, 2, 4). Measured on MI355X (cold, one launch, streaming
// weight loads): matrices of at most 1024 row groups are split, S doubling while the launch stays within 2048 waves
// and each wave keeps a whole 64-unit step; a long K (>= 4 steps per row group, the 4096 x 14336 down projection:
// 7.25 us with S = 2 against 7.68 us) takes S = 2 at any row count; 4096 x 4096 and 14336 x 4096 run best unsplit.
static int mmv_split(int64_t groups, int64_t steps) {
    int S = 1;
    while (S < 4 && groups * S * 2 <= 2048 && S * 2 <= steps) S *= 2;
    if (S == 1 && steps >= 4) S = 2;
    return S;
}

template <int R, int U, bool BS, int EP>
static void launch_q4_0_s(const MmvArgs& a, hipStream_t st, int S) {
    if constexpr (!BS) {
        if (S == 4) return launch_q4_0<R, U, BS, EP, 4>(a, st);
        if (S == 2) return launch_q4_0<R, U, BS, EP, 2>(a, st);
    }
    launch_q4_0<R, U, BS, EP, 1>(a, st);
}
template <int R, int U, bool BS, int EP>
static void launch_q8_0_s(const MmvArgs& a, hipStream_t st, int S) {
    if constexpr (!BS) {
        if (S == 4) return launch_q8_0<R, U, BS, EP, 4>(a, st);
        if (S == 2) return launch_q8_0<R, U, BS, EP, 2>(a, st);
    }
    launch_q8_0<R, U, BS, EP, 1>(a, st);
}
template <int R, bool BS, int EP>
static void launch_q4_K_s(const MmvArgs& a, hipStream_t st, int S) {
    if constexpr (!BS) {
        if (S == 4) return launch_q4_K<R, BS, EP, 4>(a, st);
        if (S == 2) return launch_q4_K<R, BS, EP, 2>(a, st);
    }
    launch_q4_K<R, BS, EP, 1>(a, st);
}
template <int R, bool BS, int EP>
static void launch_q6_K_s(const MmvArgs& a, hipStream_t st, int S) {
    if constexpr (!BS) {
        if (S == 4) return launch_q6_K<R, BS, EP, 4>(a, st);
        if (S == 2) return launch_q6_K<R, BS, EP, 2>(a, st);
    }
    launch_q6_K<R, BS, EP, 1>(a, st);
}

// Kernel variant (rows per wave R, blocks-per-lane unroll U) chosen from the block count of a row; the table is the
// result of the launch-shape sweep on MI355X. The stacked SWIGLU epilogue pairs gate row o with up row F + o: R = 2
// (one output per wave), or for an unsplit Q4_0 / Q4_K gate/up of 16384+ rows R = 4 (two outputs per wave: Q4_0
// layer 54.5 -> 53.2 us, Q4_K 32-layer model token 1904 -> 1877 us).
// The block-sum instrumentation runs without a split (S = 1).
template <bool BS, int EP>
static int mmv_one_column(const MmvArgs& a, hipStream_t st) {
    const int nb = a.k / 32;
    const int64_t groups2 = MMV_STACKED(EP) ? a.n_rows / 2 : (a.n_rows + 1) / 2;  // R = 2 row groups
    const auto split = [&](int64_t groups, int64_t steps) { return BS ? 1 : mmv_split(groups, steps); };
    switch (a.wtype) {
    case AMV_T_Q4_0:
        // R = 2 rows per wave (7.44 us cold for 14336 x 4096 against 8.5 us for R = 4, 11.2 us for R = 8); two 64-block
        // steps per loop iteration, so that at K = 4096 every load of a wave is issued before the first dot product
        // (14336 x 4096: 6.98 -> 6.7 us with the activations loaded first and the readlane wave sum)
        if constexpr (!BS && MMV_STACKED(EP)) {
            if (a.n_rows >= 16384 && a.n_rows % 4 == 0 && split(groups2, (nb + 127) / 128) == 1) {
                launch_q4_0_s<4, 2, BS, EP>(a, st, 1);
                return AMV_OK;
            }
        }
        launch_q4_0_s<2, 2, BS, EP>(a, st, split(groups2, (nb + 127) / 128));
        return AMV_OK;
    case AMV_T_Q8_0:
        if constexpr (!MMV_STACKED(EP) && EP != MMV_EP_ROPE_KV) {
            if (nb <= 64) {
                launch_q8_0_s<4, 1, BS, EP>(a, st, 1);
                return AMV_OK;
            }
        }
        launch_q8_0_s<2, 2, BS, EP>(a, st, split(groups2, (nb + 127) / 128));
        return AMV_OK;
    case AMV_T_Q4_K: {
        // from the MI355X sweep (cold, streaming loads): long rows split K in four (4096 x 14336: 8.5 us against 9.1 us
        // with S = 2); K = 4096 unsplit with 2 rows per wave (14336 x 4096 7.6 us, the stacked 28672 x 4096 12.6 us,
        // against 8.1 / 12.7 us for 4 rows per wave split in two, since the head arrives as one dword per lane and
        // the unit scales decode without branches). S depends on the launch shape only, so a fused epilogue sums
        // each row in the order of the plain GEMV of the same weight (bit-identical results).
        const int64_t steps = (nb + 63) / 64;
        const int S = BS ? 1 : steps >= 4 ? 4 : split(groups2, steps);
        launch_q4_K_s<2, BS, EP>(a, st, S);
        return AMV_OK;
    }
    case AMV_T_Q6_K: launch_q6_K_s<2, BS, EP>(a, st, split(groups2, (nb + 63) / 64)); return AMV_OK;
    default: amv_set_error("amv_mul_mat_vec: weight type %d not supported", a.wtype); return AMV_ERR_UNSUPPORTED;
    }
}

static int check_common(const char* fn, int wtype, const void* w, int64_t n_rows, int64_t k, const void* act,
                        int64_t m) {
    AMV_REQUIRE(w && act, "%s: null pointer", fn);
    AMV_REQUIRE(n_rows > 0 && k > 0 && m > 0, "%s: empty shape", fn);
    AMV_REQUIRE(n_rows <= INT32_MAX && k <= INT32_MAX && n_rows * (k / 32) < ((int64_t)1 << 31),
                "%s: shape too large (n_rows * k / 32 must stay below 2^31)", fn);
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

extern "C" int amv_mul_mat_vec_ep(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* dst,
                                  int ep_mode, const float* e, float* eout, void* stream) {
    int rc = check_common("amv_mul_mat_vec_ep", wtype, w, n_rows, k, act, 1);
    if (rc) return rc;
    AMV_REQUIRE(ep_mode >= AMV_EP_NONE && ep_mode <= AMV_EP_SWIGLU_STACKED, "amv_mul_mat_vec_ep: ep_mode %d unknown",
                ep_mode);
    AMV_REQUIRE(ep_mode != AMV_EP_NONE || dst, "amv_mul_mat_vec_ep: null dst");
    AMV_REQUIRE(ep_mode == AMV_EP_NONE || eout, "amv_mul_mat_vec_ep: null eout");
    AMV_REQUIRE(ep_mode == AMV_EP_NONE || ep_mode == AMV_EP_SWIGLU_STACKED || e,
                "amv_mul_mat_vec_ep: ep_mode %d needs its operand e", ep_mode);
    AMV_REQUIRE(ep_mode != AMV_EP_SWIGLU_STACKED || n_rows % 2 == 0,
                "amv_mul_mat_vec_ep: the stacked SWIGLU needs an even number of rows (gate rows, then up rows)");
    MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, dst, nullptr, e, eout};
    column_view(a, (const uint8_t*)act, 1, 0);
    hipStream_t st = amv_stream(stream);
    switch (ep_mode) {
    case AMV_EP_ADD: rc = mmv_one_column<false, AMV_EP_ADD>(a, st); break;
    case AMV_EP_SILU_MUL: rc = mmv_one_column<false, AMV_EP_SILU_MUL>(a, st); break;
    case AMV_EP_MUL_SILU: rc = mmv_one_column<false, AMV_EP_MUL_SILU>(a, st); break;
    case AMV_EP_SWIGLU_STACKED: rc = mmv_one_column<false, AMV_EP_SWIGLU_STACKED>(a, st); break;
    default: rc = mmv_one_column<false, AMV_EP_NONE>(a, st); break;
    }
    if (rc) return rc;
    return amv_check_launch("amv_mul_mat_vec_ep");
}

extern "C" int amv_mul_mat_vec(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                               float* dst, int64_t ldd, void* stream) {
    int rc = check_common("amv_mul_mat_vec", wtype, w, n_rows, k, act, m);
    if (rc) return rc;
    AMV_REQUIRE(dst, "amv_mul_mat_vec: null dst");
    AMV_REQUIRE(ldd >= n_rows, "amv_mul_mat_vec: ldd %lld < n_rows %lld", (long long)ldd, (long long)n_rows);
    hipStream_t st = amv_stream(stream);
    for (int64_t c = 0; c < m; ++c) {
        MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, dst + c * ldd, nullptr,
                  nullptr, nullptr};
        column_view(a, (const uint8_t*)act, m, c);
        rc = mmv_one_column<false, AMV_EP_NONE>(a, st);
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
                  sums + c * n_rows * nblk, nullptr, nullptr};
        column_view(a, (const uint8_t*)act, m, c);
        rc = mmv_one_column<true, AMV_EP_NONE>(a, st);
        if (rc) return rc;
    }
    return amv_check_launch("amv_mul_mat_block_sums");
}

// ------------------------------------------------------------------------------------------------ raw ggml blocks
// MUL_MAT of one to eight activation columns on Q4_0 / Q8_0 weights still in ggml's block layout: the reference's
// raw-layout path (ameva_qmm.comp:315-372) for a quantized tensor outside a WEIGHTS buffer or a row view of one, read
// in place instead of repacked per use. A block is 18 / 34 bytes, so a pair of blocks is 36 / 68 bytes and dword
// aligned whenever a row starts on a dword (k % 64 == 0, a dword-aligned row stride). A wave owns two rows; lane l takes
// block pairs l, l + 64, ... of both: each pair loads whole (two / four dword-aligned 16-byte loads and one dword, the
// 64 lanes covering 2.3 / 4.4 KB of the row contiguously), the first block's quants are realigned by two bytes
// (v_alignbyte_b32), and ggml's exact block integers come from v_dot4 as in the repacked GEMV (Q4_0: low nibbles
// against elements 0..15, high against 16..31, minus 8 sum(q_a)). f32 = sum over the lane's blocks in order of
// d_w d_a s, then the wave sum. SUMS writes the block integers [m][n_rows][k / 32] instead.
#define RAW_MAXM 8
template <int WT, bool SUMS, int MAXM>
__global__ __launch_bounds__(256) void k_mmv_raw(const uint8_t* __restrict__ w, int64_t row_bytes, int n_rows, int k,
                                                 const int8_t* __restrict__ aq, const int2* __restrict__ ameta, int m,
                                                 float* __restrict__ dst, int64_t ldd, int32_t* __restrict__ sums) {
    constexpr int PW = WT == AMV_T_Q4_0 ? 9 : 17;  // dwords of a block pair
    constexpr int NQ = WT == AMV_T_Q4_0 ? 4 : 8;   // quant dwords of a block
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
    if (row0 >= n_rows) return;  // whole waves; the kernel has no barrier
    const int nr = min(2, n_rows - row0);
    const int npair = k / 64, nblk = k / 32;
    float acc[MAXM][2];
#pragma unroll
    for (int c = 0; c < MAXM; ++c) acc[c][0] = acc[c][1] = 0.0f;
    for (int p = lane; p < npair; p += 64) {
        uint32_t D[2][PW];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(
                __builtin_assume_aligned(w + (size_t)(row0 + min(r, nr - 1)) * row_bytes + (size_t)p * 4 * PW, 4));
#pragma unroll
            for (int i = 0; i < PW; ++i) D[r][i] = src[i];
        }
#pragma unroll
        for (int c = 0; c < MAXM; ++c) {
            if (c >= m) break;  // uniform
#pragma unroll
            for (int b = 0; b < 2; ++b) {  // block 2 p + b
                const int j = 2 * p + b;
                const int4* a4 = reinterpret_cast<const int4*>(aq + (size_t)c * k + 32 * j);
                const int4 a0 = a4[0], a1 = a4[1];
                const int2 ds = ameta[(size_t)c * nblk + j];
                const float da = __int_as_float(ds.x);
                const int av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    // block b of the pair: f16 d at byte 0 (b = 0) or at dword NQ + 0's high half (b = 1), quants after
                    uint32_t q[NQ];
                    uint16_t dh;
                    if (b == 0) {
                        dh = (uint16_t)(D[r][0] & 0xFFFFu);
#pragma unroll
                        for (int i = 0; i < NQ; ++i) q[i] = __builtin_amdgcn_alignbyte(D[r][i + 1], D[r][i], 2);
                    } else {
                        dh = (uint16_t)(D[r][NQ] >> 16);
#pragma unroll
                        for (int i = 0; i < NQ; ++i) q[i] = D[r][NQ + 1 + i];
                    }
                    int sacc = 0;
                    if constexpr (WT == AMV_T_Q4_0) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) sacc = amv_dot4((int)(q[i] & M4), av[i], sacc);
#pragma unroll
                        for (int i = 0; i < 4; ++i) sacc = amv_dot4((int)((q[i] >> 4) & M4), av[4 + i], sacc);
                        sacc -= 8 * ds.y;
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) sacc = amv_dot4((int)q[i], av[i], sacc);
                    }
                    if constexpr (SUMS) {
                        if (r < nr) sums[((size_t)c * n_rows + row0 + r) * nblk + j] = sacc;
                    } else {
                        acc[c][r] = fmaf((float)sacc, amv_h2f(dh) * da, acc[c][r]);
                    }
                }
            }
        }
    }
    if constexpr (!SUMS) {
#pragma unroll
        for (int c = 0; c < MAXM; ++c) {
            if (c >= m) break;
            const float t0 = amv_wave_sum(acc[c][0]), t1 = amv_wave_sum(acc[c][1]);
            if (lane < nr) dst[(size_t)c * ldd + row0 + lane] = lane ? t1 : t0;
        }
    }
}

extern "C" int amv_mul_mat_vec_raw(int wtype, const void* w, int64_t row_bytes, int64_t n_rows, int64_t k,
                                   const void* act, int64_t m, float* dst, int64_t ldd, int32_t* sums, void* stream) {
    AMV_REQUIRE(wtype == AMV_T_Q4_0 || wtype == AMV_T_Q8_0, "amv_mul_mat_vec_raw: type %d (Q4_0 or Q8_0)", wtype);
    AMV_REQUIRE(w && act && (dst || sums), "amv_mul_mat_vec_raw: null pointer");
    AMV_REQUIRE(n_rows > 0 && n_rows <= INT32_MAX && k > 0 && k % 64 == 0 && k <= INT32_MAX,
                "amv_mul_mat_vec_raw: k %lld (a positive multiple of 64)", (long long)k);
    AMV_REQUIRE(m >= 1 && m <= RAW_MAXM, "amv_mul_mat_vec_raw: m %lld (1..%d columns)", (long long)m, RAW_MAXM);
    const int64_t blk = wtype == AMV_T_Q4_0 ? 18 : 34;
    AMV_REQUIRE(row_bytes >= k / 32 * blk && row_bytes % 4 == 0 && ((uintptr_t)w & 3) == 0,
                "amv_mul_mat_vec_raw: rows of %lld bytes (>= %lld, dword-aligned rows needed)", (long long)row_bytes,
                (long long)(k / 32 * blk));
    AMV_REQUIRE(((uintptr_t)act & 15) == 0, "amv_mul_mat_vec_raw: act must be 16-byte aligned");
    AMV_REQUIRE(!dst || ldd >= n_rows, "amv_mul_mat_vec_raw: ldd < n_rows");
    const int8_t* aq = (const int8_t*)act;
    const int2* meta = (const int2*)((const uint8_t*)act + m * k);
    const int waves = (int)((n_rows + 1) / 2);
    const dim3 grid((unsigned)((waves + 3) / 4));
    hipStream_t st = amv_stream(stream);
#define RAW_L(WTT, SU, MM) hipLaunchKernelGGL((k_mmv_raw<WTT, SU, MM>), grid, dim3(256), 0, st, (const uint8_t*)w, \
                                              row_bytes, (int)n_rows, (int)k, aq, meta, (int)m, dst, ldd, sums)
    // one column (decode) in its own instantiation: the eight-column one holds eight accumulator pairs
    if (wtype == AMV_T_Q4_0) {
        if (sums) RAW_L(AMV_T_Q4_0, true, RAW_MAXM);
        else if (m == 1) RAW_L(AMV_T_Q4_0, false, 1);
        else RAW_L(AMV_T_Q4_0, false, RAW_MAXM);
    } else {
        if (sums) RAW_L(AMV_T_Q8_0, true, RAW_MAXM);
        else if (m == 1) RAW_L(AMV_T_Q8_0, false, 1);
        else RAW_L(AMV_T_Q8_0, false, RAW_MAXM);
    }
#undef RAW_L
    return amv_check_launch("amv_mul_mat_vec_raw");
}

// ------------------------------------------------------------------------------------------------ fused decode GEMVs
static int mmv_dispatch_fused(int ep, MmvArgs& a, const void* act, hipStream_t st) {
    column_view(a, (const uint8_t*)act, 1, 0);
    int rc;
    switch (ep) {
    case MMV_EP_ROPE_KV: rc = mmv_one_column<false, MMV_EP_ROPE_KV>(a, st); break;
    case MMV_EP_ADD_NORM: rc = mmv_one_column<false, MMV_EP_ADD_NORM>(a, st); break;
    default: rc = mmv_one_column<false, MMV_EP_SWIGLU_Q8>(a, st); break;
    }
    return rc;
}

extern "C" int amv_gemv_rope_kv(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* qkv,
                                int64_t n_head, int64_t n_head_kv, int64_t D, const int32_t* pos, float freq_base,
                                float freq_scale, float attn_factor, void* k_cache, void* v_cache, int64_t cache_row,
                                const int64_t* kv_idx, int64_t cache_rows, unsigned int* bad, void* stream) {
    int rc = check_common("amv_gemv_rope_kv", wtype, w, n_rows, k, act, 1);
    if (rc) return rc;
    AMV_REQUIRE(qkv && pos && k_cache && v_cache && kv_idx, "amv_gemv_rope_kv: null pointer");
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && D > 0 && D % 2 == 0 && n_rows == (n_head + 2 * n_head_kv) * D,
                "amv_gemv_rope_kv: n_rows %lld != (n_head + 2 n_head_kv) * D", (long long)n_rows);
    AMV_REQUIRE(cache_row >= n_head_kv * D && cache_rows > 0, "amv_gemv_rope_kv: cache row %lld < %lld",
                (long long)cache_row, (long long)(n_head_kv * D));
    MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, qkv, nullptr, nullptr, nullptr};
    MmvPost& p = a.post;
    p.pos = pos;
    p.theta_scale = powf(freq_base, -2.0f / (float)D);  // amv_rope's expression with n_dims = D
    p.freq_scale = freq_scale;
    p.attn_factor = attn_factor;
    p.n_q = (int)(n_head * D);
    p.n_k = (int)(n_head_kv * D);
    p.head_dim = (int)D;
    p.k_cache = (uint16_t*)k_cache;
    p.v_cache = (uint16_t*)v_cache;
    p.cache_row = cache_row;
    p.kv_idx = kv_idx;
    p.cache_rows = cache_rows;
    p.bad = bad;
    rc = mmv_dispatch_fused(MMV_EP_ROPE_KV, a, act, amv_stream(stream));
    if (rc) return rc;
    return amv_check_launch("amv_gemv_rope_kv");
}

// Segment table of separate matrices stacked by rows (their repacked layouts stay their own).
static int mmv_segments(const char* fn, MmvPost& p, int n, const void* const* w, const int64_t* rows, int wtype,
                        int64_t k) {
    p.n_seg = n;
    int64_t r0 = 0;
    for (int s = 0; s < 4; ++s) p.seg_row[s] = INT32_MAX;
    for (int s = 0; s < n; ++s) {
        AMV_REQUIRE(w[s] && ((uintptr_t)w[s] & 15) == 0, "%s: matrix %d null or not 16-byte aligned", fn, s);
        AMV_REQUIRE(rows[s] > 0 && rows[s] % 2 == 0, "%s: matrix %d rows %lld (even, > 0)", fn, s, (long long)rows[s]);
        p.seg_row[s] = (int)r0;
        p.w_seg[s] = (const uint8_t*)w[s];
        r0 += rows[s];
    }
    p.seg_row[n] = (int)r0;
    AMV_REQUIRE(wtype == AMV_T_Q4_0 || wtype == AMV_T_Q4_K, "%s: weight type %d (Q4_0 or Q4_K)", fn, wtype);
    AMV_REQUIRE(wtype != AMV_T_Q4_0 || k % (64 * 2 * 32) == 0, "%s: Q4_0 k %% 4096 != 0", fn);
    return AMV_OK;
}

extern "C" int amv_gemv_rope_kv_seg(int wtype, const void* wq, const void* wk, const void* wv, int64_t k,
                                    const void* act, float* q_out, float* k_out, float* v_out, int64_t n_head,
                                    int64_t n_head_kv, int64_t D, const int32_t* pos, float freq_base, float freq_scale,
                                    float attn_factor, void* k_cache, void* v_cache, int64_t cache_row,
                                    const int64_t* kv_idx, int64_t cache_rows, unsigned int* bad, void* stream) {
    const int64_t n_rows = (n_head + 2 * n_head_kv) * D;
    int rc = check_common("amv_gemv_rope_kv_seg", wtype, wq, n_rows, k, act, 1);
    if (rc) return rc;
    AMV_REQUIRE(q_out && k_out && v_out && pos && k_cache && v_cache && kv_idx, "amv_gemv_rope_kv_seg: null pointer");
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && D > 0 && D % 2 == 0, "amv_gemv_rope_kv_seg: bad heads");
    AMV_REQUIRE(cache_row >= n_head_kv * D && cache_rows > 0, "amv_gemv_rope_kv_seg: cache row %lld < %lld",
                (long long)cache_row, (long long)(n_head_kv * D));
    MmvArgs a{wtype, (const uint8_t*)wq, (int)n_rows, (int)k, nullptr, nullptr, nullptr, q_out, nullptr, nullptr,
              nullptr};
    MmvPost& p = a.post;
    const void* ws[3] = {wq, wk, wv};
    const int64_t rows[3] = {n_head * D, n_head_kv * D, n_head_kv * D};
    rc = mmv_segments("amv_gemv_rope_kv_seg", p, 3, ws, rows, wtype, k);
    if (rc) return rc;
    p.dst_seg[0] = q_out;
    p.dst_seg[1] = k_out;
    p.dst_seg[2] = v_out;
    p.pos = pos;
    p.theta_scale = powf(freq_base, -2.0f / (float)D);  // amv_rope's expression with n_dims = D
    p.freq_scale = freq_scale;
    p.attn_factor = attn_factor;
    p.n_q = (int)(n_head * D);
    p.n_k = (int)(n_head_kv * D);
    p.head_dim = (int)D;
    p.k_cache = (uint16_t*)k_cache;
    p.v_cache = (uint16_t*)v_cache;
    p.cache_row = cache_row;
    p.kv_idx = kv_idx;
    p.cache_rows = cache_rows;
    p.bad = bad;
    rc = mmv_dispatch_fused(MMV_EP_ROPE_KV, a, act, amv_stream(stream));
    if (rc) return rc;
    return amv_check_launch("amv_gemv_rope_kv_seg");
}

extern "C" int amv_gemv_swiglu_q8_seg(int wtype, const void* w_gate, const void* w_up, int64_t F, int64_t k,
                                      const void* act, float* eout, void* act_out, int act_type, int rule,
                                      unsigned int* counters, void* stream) {
    int rc = check_common("amv_gemv_swiglu_q8_seg", wtype, w_gate, 2 * F, k, act, 1);
    if (rc) return rc;
    AMV_REQUIRE(eout && act_out && counters, "amv_gemv_swiglu_q8_seg: null pointer");
    AMV_REQUIRE(act_type == AMV_T_Q8_0 || act_type == AMV_T_Q8_K,
                "amv_gemv_swiglu_q8_seg: act_type %d (Q8_0 or Q8_K)", act_type);
    AMV_REQUIRE(F > 0 && F % (act_type == AMV_T_Q8_K ? 256 : 32) == 0,
                "amv_gemv_swiglu_q8_seg: F must be a multiple of the block size");
    AMV_REQUIRE(((uintptr_t)act_out & 15) == 0 && ((uintptr_t)eout & 15) == 0,
                "amv_gemv_swiglu_q8_seg: act_out and eout must be 16-byte aligned");
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_gemv_swiglu_q8_seg: bad rule");
    MmvArgs a{wtype, (const uint8_t*)w_gate, (int)(2 * F), (int)k, nullptr, nullptr, nullptr, nullptr, nullptr,
              nullptr, eout};
    MmvPost& p = a.post;
    const void* ws[2] = {w_gate, w_up};
    const int64_t rows[2] = {F, F};
    rc = mmv_segments("amv_gemv_swiglu_q8_seg", p, 2, ws, rows, wtype, k);
    if (rc) return rc;
    p.counters = counters;
    p.act = amv_act_out(act_out, F, act_type, rule);
    rc = mmv_dispatch_fused(MMV_EP_SWIGLU_Q8, a, act, amv_stream(stream));
    if (rc) return rc;
    return amv_check_launch("amv_gemv_swiglu_q8_seg");
}

extern "C" int amv_gemv_add_rms_norm(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* dst,
                                     const float* e, float* eout, float eps, const float* norm_w, float* norm_y,
                                     float* norm_o, void* act_out, int act_type, int rule, unsigned int* counters,
                                     void* stream) {
    int rc = check_common("amv_gemv_add_rms_norm", wtype, w, n_rows, k, act, 1);
    if (rc) return rc;
    AMV_REQUIRE(e && eout && counters, "amv_gemv_add_rms_norm: null pointer");
    AMV_REQUIRE(norm_y || norm_o || act_out, "amv_gemv_add_rms_norm: no norm output requested");
    AMV_REQUIRE(!norm_o || norm_w, "amv_gemv_add_rms_norm: norm_o needs norm_w");
    AMV_REQUIRE(!act_out || act_type == AMV_T_Q8_0 || act_type == AMV_T_Q8_K,
                "amv_gemv_add_rms_norm: act_type %d (Q8_0 or Q8_K)", act_type);
    AMV_REQUIRE(n_rows % 4 == 0 && (!act_out || n_rows % (act_type == AMV_T_Q8_K ? 256 : 32) == 0),
                "amv_gemv_add_rms_norm: n_rows must be a multiple of 4 (of the block size with the act output)");
    AMV_REQUIRE(((uintptr_t)eout & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && ((uintptr_t)norm_y & 15) == 0 &&
                    ((uintptr_t)norm_o & 15) == 0 && ((uintptr_t)act_out & 15) == 0,
                "amv_gemv_add_rms_norm: eout, norm buffers and act_out must be 16-byte aligned");
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_gemv_add_rms_norm: bad rule");
    MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, dst, nullptr, e, eout};
    MmvPost& p = a.post;
    p.counters = counters;
    p.norm_w = norm_w;
    p.eps = eps;
    p.norm_y = norm_y;
    p.norm_o = norm_o;
    p.act = amv_act_out(act_out, n_rows, act_out ? act_type : 0, rule);
    rc = mmv_dispatch_fused(MMV_EP_ADD_NORM, a, act, amv_stream(stream));
    if (rc) return rc;
    return amv_check_launch("amv_gemv_add_rms_norm");
}

extern "C" int amv_gemv_swiglu_q8(int wtype, const void* w, int64_t n_rows, int64_t k, const void* act, float* dst,
                                  float* eout, void* act_out, int act_type, int rule, unsigned int* counters,
                                  void* stream) {
    int rc = check_common("amv_gemv_swiglu_q8", wtype, w, n_rows, k, act, 1);
    if (rc) return rc;
    AMV_REQUIRE(eout && act_out && counters, "amv_gemv_swiglu_q8: null pointer");
    AMV_REQUIRE(act_type == AMV_T_Q8_0 || act_type == AMV_T_Q8_K, "amv_gemv_swiglu_q8: act_type %d (Q8_0 or Q8_K)",
                act_type);
    AMV_REQUIRE(n_rows % (2 * (act_type == AMV_T_Q8_K ? 256 : 32)) == 0,
                "amv_gemv_swiglu_q8: n_rows must be 2 x a multiple of the block size (gate rows, then up rows)");
    AMV_REQUIRE(((uintptr_t)act_out & 15) == 0 && ((uintptr_t)eout & 15) == 0,
                "amv_gemv_swiglu_q8: act_out and eout must be 16-byte aligned");
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "amv_gemv_swiglu_q8: bad rule");
    MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, dst, nullptr, nullptr, eout};
    MmvPost& p = a.post;
    p.counters = counters;
    p.act = amv_act_out(act_out, n_rows / 2, act_type, rule);
    rc = mmv_dispatch_fused(MMV_EP_SWIGLU_Q8, a, act, amv_stream(stream));
    if (rc) return rc;
    return amv_check_launch("amv_gemv_swiglu_q8");
}

// ---------------------------------------------------------------------------------------------------------------
// RMS_NORM (* norm_w, Q8_0) folded into the Q4_0 K = 4096 decode GEMV after it (k_mmv_q4_0_k4096_norm).
static std::atomic<int> g_norm_nt{0};
extern "C" void amv_debug_norm_gemv_threads(int nt) { g_norm_nt.store(nt, std::memory_order_relaxed); }

template <int EP, bool SEG, int P, int RULE>
static void launch_norm_gemv_r(int nt, int waves, const float* x, const float* nw, float eps, const MmvArgs& a,
                               hipStream_t st) {
    const int64_t nblk = (int64_t)a.n_rows * 128;
    const uint4* wq = SEG ? nullptr : reinterpret_cast<const uint4*>(a.w);
    const uint32_t* wd = SEG ? nullptr : reinterpret_cast<const uint32_t*>(a.w + nblk * 16);
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* w4 = reinterpret_cast<const float4*>(nw);
#define AMV_NORM_LAUNCH(NT)                                                                                        \
    hipLaunchKernelGGL((k_mmv_q4_0_k4096_norm<NT, EP, SEG, P, RULE>),                                           \
                       dim3((unsigned)((waves + NT / 64 - 1) / (NT / 64))), dim3(NT), 0, st, x4, w4, eps, wq, wd,       \
                       a.n_rows, a.dst, a.eout, a.post)
    if (nt == 256) AMV_NORM_LAUNCH(256);
    else if (nt == 512) AMV_NORM_LAUNCH(512);
    else AMV_NORM_LAUNCH(1024);
#undef AMV_NORM_LAUNCH
}
// the Q8_0 rule as a template argument: each kernel holds the code of one rule only
template <int EP, bool SEG, int P = 2>
static void launch_norm_gemv(int nt, int waves, const float* x, const float* nw, float eps, int rule, const MmvArgs& a,
                             hipStream_t st) {
    if (rule == AMV_Q8_X86) launch_norm_gemv_r<EP, SEG, P, AMV_Q8_X86>(nt, waves, x, nw, eps, a, st);
    else if (rule == AMV_Q8_ARM) launch_norm_gemv_r<EP, SEG, P, AMV_Q8_ARM>(nt, waves, x, nw, eps, a, st);
    else launch_norm_gemv_r<EP, SEG, P, AMV_Q8_REF>(nt, waves, x, nw, eps, a, st);
}

template <int EP, bool SEG>
static void launch_norm_gemv_q4k(int nt, int waves, const float* x, const float* nw, float eps, const MmvArgs& a,
                                 hipStream_t st) {
    const uint4* wq = SEG ? nullptr : reinterpret_cast<const uint4*>(a.w);
    const uint4* wh = SEG ? nullptr : reinterpret_cast<const uint4*>(a.w + (size_t)a.n_rows * 16 * 128);
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* w4 = reinterpret_cast<const float4*>(nw);
#define AMV_NORM_K_LAUNCH(NT)                                                                                      \
    hipLaunchKernelGGL((k_mmv_q4_K_norm<NT, EP, SEG>), dim3((unsigned)((waves + NT / 64 - 1) / (NT / 64))),       \
                       dim3(NT), 0, st, x4, w4, eps, wq, wh, a.n_rows, a.dst, a.eout, a.post)
    if (nt == 256) AMV_NORM_K_LAUNCH(256);
    else if (nt == 512) AMV_NORM_K_LAUNCH(512);
    else AMV_NORM_K_LAUNCH(1024);
#undef AMV_NORM_K_LAUNCH
}

static int norm_gemv_checks(const char* fn, const float* x, const float* nw, int rule, int wtype, const void* w,
                            int64_t n_rows, int64_t k) {
    AMV_REQUIRE(x && nw && w, "%s: null pointer", fn);
    AMV_REQUIRE(wtype == AMV_T_Q4_0 || wtype == AMV_T_Q4_K, "%s: weight type %d (Q4_0 or Q4_K)", fn, wtype);
    AMV_REQUIRE(k == 4096, "%s: k %lld (the folded norm takes rows of 4096)", fn, (long long)k);
    AMV_REQUIRE(n_rows > 0 && n_rows % 2 == 0 && n_rows <= (1 << 24), "%s: n_rows %lld (even)", fn,
                (long long)n_rows);
    AMV_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)nw & 15) == 0 && ((uintptr_t)w & 15) == 0,
                "%s: x, norm_w and w must be 16-byte aligned", fn);
    AMV_REQUIRE(rule >= AMV_Q8_X86 && rule <= AMV_Q8_REF, "%s: bad rule", fn);
    return AMV_OK;
}

extern "C" int amv_rms_norm_gemv_rope_kv(const float* x, const float* norm_w, float eps, int rule, int wtype,
                                         const void* w, int64_t n_rows, int64_t k, float* qkv, int64_t n_head,
                                         int64_t n_head_kv, int64_t D, const int32_t* pos, float freq_base,
                                         float freq_scale, float attn_factor, void* k_cache, void* v_cache,
                                         int64_t cache_row, const int64_t* kv_idx, int64_t cache_rows,
                                         unsigned int* bad, void* stream) {
    const char* fn = "amv_rms_norm_gemv_rope_kv";
    int rc = norm_gemv_checks(fn, x, norm_w, rule, wtype, w, n_rows, k);
    if (rc) return rc;
    AMV_REQUIRE(qkv && pos && k_cache && v_cache && kv_idx, "%s: null pointer", fn);
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && D > 0 && D % 2 == 0 && n_rows == (n_head + 2 * n_head_kv) * D,
                "%s: n_rows %lld != (n_head + 2 n_head_kv) * D", fn, (long long)n_rows);
    AMV_REQUIRE(cache_row >= n_head_kv * D && cache_rows > 0, "%s: cache row %lld < %lld", fn, (long long)cache_row,
                (long long)(n_head_kv * D));
    MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, qkv, nullptr, nullptr, nullptr};
    MmvPost& p = a.post;
    p.pos = pos;
    p.theta_scale = powf(freq_base, -2.0f / (float)D);  // amv_rope's expression with n_dims = D
    p.freq_scale = freq_scale;
    p.attn_factor = attn_factor;
    p.n_q = (int)(n_head * D);
    p.n_k = (int)(n_head_kv * D);
    p.head_dim = (int)D;
    p.k_cache = (uint16_t*)k_cache;
    p.v_cache = (uint16_t*)v_cache;
    p.cache_row = cache_row;
    p.kv_idx = kv_idx;
    p.cache_rows = cache_rows;
    p.bad = bad;
    const int nt = g_norm_nt.load(std::memory_order_relaxed);
    if (wtype == AMV_T_Q4_K)
        launch_norm_gemv_q4k<MMV_EP_ROPE_KV, false>(nt > 0 ? nt : 1024, (int)(n_rows / 2), x, norm_w, eps, a,
                                                    amv_stream(stream));
    else
        launch_norm_gemv<MMV_EP_ROPE_KV, false>(nt > 0 ? nt : 1024, (int)(n_rows / 2), x, norm_w, eps, rule, a,
                                                amv_stream(stream));
    return amv_check_launch(fn);
}

extern "C" int amv_rms_norm_gemv_swiglu_q8(const float* x, const float* norm_w, float eps, int rule, int wtype,
                                           const void* w, int64_t n_rows, int64_t k, float* dst, float* eout,
                                           void* act_out, unsigned int* counters, void* stream) {
    const char* fn = "amv_rms_norm_gemv_swiglu_q8";
    int rc = norm_gemv_checks(fn, x, norm_w, rule, wtype, w, n_rows, k);
    if (rc) return rc;
    AMV_REQUIRE(eout && act_out && counters, "%s: null pointer", fn);
    const int bs = wtype == AMV_T_Q4_K ? 256 : 32;  // the output activation: Q8_K for Q4_K, Q8_0 for Q4_0
    AMV_REQUIRE(n_rows % (2 * bs) == 0, "%s: n_rows must be 2 x a multiple of %d (gate rows, then up rows)", fn, bs);
    AMV_REQUIRE(((uintptr_t)act_out & 15) == 0 && ((uintptr_t)eout & 15) == 0,
                "%s: act_out and eout must be 16-byte aligned", fn);
    MmvArgs a{wtype, (const uint8_t*)w, (int)n_rows, (int)k, nullptr, nullptr, nullptr, dst, nullptr, nullptr, eout};
    MmvPost& p = a.post;
    p.counters = counters;
    p.act = amv_act_out(act_out, n_rows / 2, wtype == AMV_T_Q4_K ? AMV_T_Q8_K : AMV_T_Q8_0, rule);
    const int nt = g_norm_nt.load(std::memory_order_relaxed);
    if (wtype == AMV_T_Q4_K)
        launch_norm_gemv_q4k<MMV_EP_SWIGLU_Q8, false>(nt > 0 ? nt : 1024, (int)(n_rows / 2), x, norm_w, eps, a,
                                                      amv_stream(stream));
    else if (nt < 0)  // instrumentation: -NT threads, four outputs per wave
        launch_norm_gemv<MMV_EP_SWIGLU_Q8, false, 4>(-nt, (int)(n_rows / 8), x, norm_w, eps, rule, a,
                                                     amv_stream(stream));
    else  // two outputs per wave, 1024 threads by default
        launch_norm_gemv<MMV_EP_SWIGLU_Q8, false>(nt ? nt : 1024, (int)(n_rows / 4), x, norm_w, eps, rule, a,
                                                  amv_stream(stream));
    return amv_check_launch(fn);
}

extern "C" int amv_rms_norm_gemv_rope_kv_seg(const float* x, const float* norm_w, float eps, int rule, int wtype,
                                             const void* wq, const void* wk, const void* wv, int64_t k, float* q_out,
                                             float* k_out, float* v_out, int64_t n_head, int64_t n_head_kv, int64_t D,
                                             const int32_t* pos, float freq_base, float freq_scale,
                                             float attn_factor, void* k_cache, void* v_cache, int64_t cache_row,
                                             const int64_t* kv_idx, int64_t cache_rows, unsigned int* bad,
                                             void* stream) {
    const char* fn = "amv_rms_norm_gemv_rope_kv_seg";
    AMV_REQUIRE(n_head > 0 && n_head_kv > 0 && D > 0 && D % 2 == 0, "%s: bad heads", fn);
    const int64_t n_rows = (n_head + 2 * n_head_kv) * D;
    int rc = norm_gemv_checks(fn, x, norm_w, rule, wtype, wq, n_rows, k);
    if (rc) return rc;
    AMV_REQUIRE(q_out && k_out && v_out && pos && k_cache && v_cache && kv_idx, "%s: null pointer", fn);
    AMV_REQUIRE(cache_row >= n_head_kv * D && cache_rows > 0, "%s: cache row %lld < %lld", fn, (long long)cache_row,
                (long long)(n_head_kv * D));
    MmvArgs a{wtype, (const uint8_t*)wq, (int)n_rows, (int)k, nullptr, nullptr, nullptr, q_out, nullptr, nullptr,
              nullptr};
    MmvPost& p = a.post;
    const void* ws[3] = {wq, wk, wv};
    const int64_t rows[3] = {n_head * D, n_head_kv * D, n_head_kv * D};
    rc = mmv_segments(fn, p, 3, ws, rows, wtype, k);
    if (rc) return rc;
    p.dst_seg[0] = q_out;
    p.dst_seg[1] = k_out;
    p.dst_seg[2] = v_out;
    p.pos = pos;
    p.theta_scale = powf(freq_base, -2.0f / (float)D);  // amv_rope's expression with n_dims = D
    p.freq_scale = freq_scale;
    p.attn_factor = attn_factor;
    p.n_q = (int)(n_head * D);
    p.n_k = (int)(n_head_kv * D);
    p.head_dim = (int)D;
    p.k_cache = (uint16_t*)k_cache;
    p.v_cache = (uint16_t*)v_cache;
    p.cache_row = cache_row;
    p.kv_idx = kv_idx;
    p.cache_rows = cache_rows;
    p.bad = bad;
    const int nt = g_norm_nt.load(std::memory_order_relaxed);
    if (wtype == AMV_T_Q4_K)
        launch_norm_gemv_q4k<MMV_EP_ROPE_KV, true>(nt > 0 ? nt : 1024, (int)(n_rows / 2), x, norm_w, eps, a,
                                                   amv_stream(stream));
    else
        launch_norm_gemv<MMV_EP_ROPE_KV, true>(nt > 0 ? nt : 1024, (int)(n_rows / 2), x, norm_w, eps, rule, a,
                                               amv_stream(stream));
    return amv_check_launch(fn);
}

extern "C" int amv_rms_norm_gemv_swiglu_q8_seg(const float* x, const float* norm_w, float eps, int rule, int wtype,
                                               const void* w_gate, const void* w_up, int64_t F, int64_t k,
                                               float* eout, void* act_out, unsigned int* counters, void* stream) {
    const char* fn = "amv_rms_norm_gemv_swiglu_q8_seg";
    int rc = norm_gemv_checks(fn, x, norm_w, rule, wtype, w_gate, 2 * F, k);
    if (rc) return rc;
    AMV_REQUIRE(eout && act_out && counters, "%s: null pointer", fn);
    const int bs = wtype == AMV_T_Q4_K ? 256 : 32;  // the output activation: Q8_K for Q4_K, Q8_0 for Q4_0
    AMV_REQUIRE(F > 0 && F % bs == 0, "%s: F must be a multiple of %d", fn, bs);
    AMV_REQUIRE(((uintptr_t)act_out & 15) == 0 && ((uintptr_t)eout & 15) == 0,
                "%s: act_out and eout must be 16-byte aligned", fn);
    MmvArgs a{wtype, (const uint8_t*)w_gate, (int)(2 * F), (int)k, nullptr, nullptr, nullptr, nullptr, nullptr,
              nullptr, eout};
    MmvPost& p = a.post;
    const void* ws[2] = {w_gate, w_up};
    const int64_t rows[2] = {F, F};
    rc = mmv_segments(fn, p, 2, ws, rows, wtype, k);
    if (rc) return rc;
    p.counters = counters;
    p.act = amv_act_out(act_out, F, wtype == AMV_T_Q4_K ? AMV_T_Q8_K : AMV_T_Q8_0, rule);
    const int nt = g_norm_nt.load(std::memory_order_relaxed);
    if (wtype == AMV_T_Q4_K)
        launch_norm_gemv_q4k<MMV_EP_SWIGLU_Q8, true>(nt > 0 ? nt : 1024, (int)F, x, norm_w, eps, a,
                                                     amv_stream(stream));
    else if (nt < 0)
        launch_norm_gemv<MMV_EP_SWIGLU_Q8, true, 4>(-nt, (int)(F / 4), x, norm_w, eps, rule, a, amv_stream(stream));
    else
        launch_norm_gemv<MMV_EP_SWIGLU_Q8, true>(nt ? nt : 1024, (int)(F / 2), x, norm_w, eps, rule, a,
                                                 amv_stream(stream));
    return amv_check_launch(fn);
}
