// BitNet b1.58 I2_S: per-token absmax int8 activation quantization and the ternary GEMV.
//
// Role of bitnet_norm_q8.comp / bitnet_gemv_i2_s.comp (reference, src/shaders) and of the CPU path
// quantize_activation_int8 + ggml_vec_dot_i2_i8_s + bitnet_gemv (adapters/bitnet/src/cpu/llama_bitnet_core.cpp:914-941,
// ggml_bitnet_mad.cpp:191-231 scalar branch). Weight layout is the BitNet one, used in place (it is already
// row-major and 16-byte aligned per row when k % 64 == 0): row r is k/4 bytes; 128-weight blocks of 32 bytes; byte i of
// a block holds the 2-bit codes of weights i, 32 + i, 64 + i, 96 + i in bits 7-6, 5-4, 3-2, 1-0; weight = code - 1.
// y[r] = float(sum_j (c_rj - 1) q_j) * (act_dequant * weight_scale); the integer is formed exactly as
// sum_j c_rj q_j - sum_j q_j with v_dot4_i32_i8 (codes 0..3 are valid signed bytes).
#include "amv_common.h"

#include <algorithm>

// ---------------------------------------------------------------------------------------------------------------
// quantize_activation_int8: one workgroup of 256 per row. max_abs starts at 1e-7, scale = 127 / max_abs,
// q = clamp(roundf(x * scale), -127, 127) (round half away from zero), dequant = 1 / scale, plus sum(q).
// Output layout: q int8 [m][k] | {f32 dequant, i32 sum q} [m].
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_i2s_quant(const float* __restrict__ x, int k, int8_t* __restrict__ q,
                                                  int2* __restrict__ meta) {
    __shared__ float smax[4];
    __shared__ int ssum[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* xr = x + (size_t)row * k;
    float amax = 1e-7f;
    for (int i = tid; i < k; i += 256) amax = fmaxf(amax, fabsf(xr[i]));
    amax = amv_wave_max_u(amax);
    if (lane == 0) smax[w] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    const float scale = 127.0f / amax;
    int s = 0;
    for (int i = tid; i < k; i += 256) {
        float v = roundf(xr[i] * scale);
        v = fminf(127.0f, fmaxf(-127.0f, v));
        q[(size_t)row * k + i] = (int8_t)(int)v;
        s += (int)v;
    }
    s = amv_wave_sum_i_u(s);
    if (lane == 0) ssum[w] = s;
    __syncthreads();
    if (tid == 0) meta[row] = make_int2(__float_as_int(1.0f / scale), ssum[0] + ssum[1] + ssum[2] + ssum[3]);
}

// ---------------------------------------------------------------------------------------------------------------
// GEMV: a wave owns R rows; the k/64 16-byte slices of a row go to the lanes (slice j: block j/2, bytes
// 16 (j%2) .. +15, i.e. weights 16 (j%2) + i + 32 g of the block). OUT_SUMS writes the exact integer per row; ACC adds
// the result to dst (the residual add of the BitNet layer, x += W q: llama_bitnet_core.cpp:1244, 1264).
// ---------------------------------------------------------------------------------------------------------------
template <int R, bool OUT_SUMS, bool ACC = false>
__global__ __launch_bounds__(256) void k_i2s_gemv(const uint4* __restrict__ w, int n_rows, int nsl,
                                                 const int8_t* __restrict__ q, const int2* __restrict__ meta,
                                                 float wscale, float* __restrict__ dst, int32_t* __restrict__ isums) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (row0 >= n_rows) return;
    const int4* a4 = reinterpret_cast<const int4*>(q);
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0;
    // two 64-slice steps per pass, every load of both issued before either step's arithmetic and none behind a
    // lane branch (a lane past the row's end reads slice nsl - 1 and adds nothing): one memory round trip per pass
    struct Step {
        uint4 c[R];
        int4 a[4];
        bool valid;
    };
    const auto load = [&](int j0, Step& st) {
        const int j = j0 + lane;
        const int jj = min(j, nsl - 1);
        st.valid = j < nsl;
#pragma unroll
        for (int r = 0; r < R; ++r) st.c[r] = amv_ld_stream(w + (size_t)min(row0 + r, n_rows - 1) * nsl + jj);
        const int b = jj >> 1, p = jj & 1;
#pragma unroll
        for (int g = 0; g < 4; ++g) st.a[g] = a4[b * 8 + 2 * g + p];
    };
    const auto compute = [&](const Step& st) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int s = acc[r];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int sh = 6 - 2 * g;
                s = amv_dot4((int)((st.c[r].x >> sh) & 0x03030303u), st.a[g].x, s);
                s = amv_dot4((int)((st.c[r].y >> sh) & 0x03030303u), st.a[g].y, s);
                s = amv_dot4((int)((st.c[r].z >> sh) & 0x03030303u), st.a[g].z, s);
                s = amv_dot4((int)((st.c[r].w >> sh) & 0x03030303u), st.a[g].w, s);
            }
            acc[r] = st.valid ? s : acc[r];
        }
    };
    // a row of at most 64 slices (K <= 4096) takes the single step after the loop, no pass of clamped reads
    int j0 = 0;
    for (; j0 + 64 < nsl; j0 += 128) {
        Step s0, s1;
        load(j0, s0);
        load(j0 + 64, s1);
        __builtin_amdgcn_sched_barrier(0);
        compute(s0);
        compute(s1);
    }
    if (j0 < nsl) {
        Step s0;
        load(j0, s0);
        compute(s0);
    }
    const int2 m = meta[0];
    const float total_scale = __int_as_float(m.x) * wscale;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int t = amv_wave_sum_i_u(acc[r]) - m.y;
        if (lane == 0 && row0 + r < n_rows) {
            if (OUT_SUMS) isums[row0 + r] = t;
            else if (ACC) dst[row0 + r] = dst[row0 + r] + (float)t * total_scale;
            else dst[row0 + r] = (float)t * total_scale;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Batched (m >= 8 tokens) I2_S MUL_MAT on int8 MFMA. The activation scale is per token over the whole row, so the
// ternary dot stays integer across all of k: v_mfma_i32_32x32x32_i8 (the full-rate int8 shape of gfx950) accumulates
// sum_k code * q in its int32 accumulator from the first block to the last (codes 0..3 are valid signed bytes), and
// sum q is subtracted once.
// MFMA k slots may be assigned to weights in any order A and B share: in block b, step t (0..3), lane half h
// (lanes 32 h .. 32 h + 31) supplies the 16 weights 32 t + 16 h + s (s = 0..15), i.e. the 2-bit field t (shift
// 6 - 2 t) of block bytes 16 h .. 16 h + 15, and the activations q[128 b + 32 t + 16 h + s]: one 16-byte load each.
// Lane l of a 32 x 32 tile holds token column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4, r = 0..15.
// ---------------------------------------------------------------------------------------------------------------
typedef int i2s_v4i __attribute__((ext_vector_type(4)));
typedef int i2s_v16i __attribute__((ext_vector_type(16)));

#define I2S_OUT_F32 0
#define I2S_OUT_SUMS 1

// Sum of the S split partials (integers: exact in any order), minus sum q, scaled. Thread (x, y): rows 4 x .. 4 x + 3
// of token y; VEC: n_rows % 4 == 0 (16-byte partial rows), the S loads of a thread issued before its first add.
template <bool OUT_SUMS, bool VEC>
__global__ __launch_bounds__(256) void k_i2s_split_sum(const int32_t* __restrict__ part, int S, int n_rows, int m,
                                                      const int2* __restrict__ meta, float wscale,
                                                      float* __restrict__ dst, int64_t ldd,
                                                      int32_t* __restrict__ isums) {
    const int tok = blockIdx.y, r0 = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (r0 >= n_rows) return;
    const size_t plane = (size_t)m * n_rows, base = (size_t)tok * n_rows + r0;
    const int nr = min(4, n_rows - r0);
    int t[4] = {0, 0, 0, 0};
    if constexpr (VEC) {
        for (int s0 = 0; s0 < S; s0 += 8) {
            int4 v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (s0 + e < S) v[e] = *reinterpret_cast<const int4*>(part + (s0 + e) * plane + base);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (s0 + e < S) {
                    t[0] += v[e].x;
                    t[1] += v[e].y;
                    t[2] += v[e].z;
                    t[3] += v[e].w;
                }
            }
        }
    } else {
        for (int s2 = 0; s2 < S; ++s2)
            for (int e = 0; e < nr; ++e) t[e] += part[s2 * plane + base + e];
    }
    const int2 mt = meta[tok];
    const float sc = __int_as_float(mt.x) * wscale;
    for (int e = 0; e < nr; ++e) {
        if (OUT_SUMS) isums[base + e] = t[e] - mt.y;
        else dst[(size_t)tok * ldd + r0 + e] = (float)(t[e] - mt.y) * sc;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Batched I2_S (k_i2s_mmq_p): a workgroup computes a 64-row x 64-token tile over the k blocks of its split; wave w takes
// the split's blocks w, w + 4, ... in chunks of PB blocks whose global loads (the two row tiles' weight halves
// straight into the A operands, the two token tiles' activations into the B operands: one 16-byte load each, the
// k-slot assignment above) are all issued before the chunk's first MFMA, so a wave waits for memory once per chunk
// rather than once per block. The four waves' integer tiles are added in LDS in a fixed order (exact), then
// stored row-contiguous: the final values (one split) or this split's partial plane [S][m][n_rows] for
// k_i2s_split_sum. One-dimensional grid: the token tiles of a row tile, then the row tiles, then the splits, dealt
// to the XCDs in consecutive runs (amv_xcd_tile), so the workgroups sharing a weight tile share an L2.
// LDS: the four waves' tiles [wave][tile][r][lane] with the lane index XOR-swizzled by r + 16 (row tile) so that both
// the wave-wide stores (one r) and the row-wise sums (64 rows of one token) meet distinct banks: 64 KB.
// ---------------------------------------------------------------------------------------------------------------
template <int OUT, bool SPLIT, int PB>
__global__ __launch_bounds__(256) void k_i2s_mmq_p(const uint8_t* __restrict__ w, int n_rows, int kb,
                                                  const int8_t* __restrict__ q, const int2* __restrict__ meta, int m,
                                                  int kb_per, int n_rt, int n_tt, int n_sp, float wscale,
                                                  float* __restrict__ dst, int64_t ldd, int32_t* __restrict__ iout,
                                                  int32_t* __restrict__ part) {
    __shared__ int32_t red[4][4][16][64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 31, h = lane >> 5;
    const int T = amv_xcd_tile(blockIdx.x, n_tt * n_rt * n_sp);
    const int tt = T % n_tt, rt = (T / n_tt) % n_rt, sp = T / (n_tt * n_rt);
    const int row0 = rt * 64, tok0 = tt * 64;
    const int b0 = sp * kb_per, nblk = min(kb_per, kb - b0);  // >= 1 (the launcher's split)
    const size_t k = (size_t)kb * 128;
    const uint4* wr[2];
    const int4* qa[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
        wr[i] = reinterpret_cast<const uint4*>(w + (size_t)min(row0 + 32 * i + c, n_rows - 1) * kb * 32) + h;
#pragma unroll
    for (int j = 0; j < 2; ++j)
        qa[j] = reinterpret_cast<const int4*>(q + (size_t)min(tok0 + 32 * j + c, m - 1) * k + 16 * h);
    i2s_v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    const int nbw = nblk > wv ? (nblk - wv + 3) / 4 : 0;  // this wave's blocks: b0 + wv + 4 i, i < nbw
    for (int c0 = 0; c0 < nbw; c0 += PB) {
        uint4 wb[PB][2];
        int4 ab[PB][2][4];
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            if (c0 + i < nbw) {  // uniform
                const int b = b0 + wv + 4 * (c0 + i);
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) wb[i][ii] = wr[ii][2 * b];
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int t = 0; t < 4; ++t) ab[i][j][t] = qa[j][8 * b + 2 * t];
            }
        }
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            if (c0 + i >= nbw) break;  // uniform
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int sh = 6 - 2 * t;
                i2s_v4i A[2];
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
                    A[ii] = i2s_v4i{(int)((wb[i][ii].x >> sh) & 0x03030303u), (int)((wb[i][ii].y >> sh) & 0x03030303u),
                                    (int)((wb[i][ii].z >> sh) & 0x03030303u), (int)((wb[i][ii].w >> sh) & 0x03030303u)};
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int4 v = ab[i][j][t];
                        acc[ii][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[ii], i2s_v4i{v.x, v.y, v.z, v.w},
                                                                           acc[ii][j], 0, 0, 0);
                    }
            }
        }
    }
    // lane l of tile (i, j) holds token 32 j + l % 32 and rows 32 i + 8 (r / 4) + 4 (l / 32) + r % 4
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[wv][2 * i + j][r][lane ^ (r + 16 * i)] = acc[i][j][r];
    __syncthreads();
    // thread: tile row rr (64 consecutive threads = 64 consecutive rows), tokens 16 (tid / 64) .. + 15
    const int rr = tid & 63, i = rr >> 5, r32 = rr & 31;
    const int r = 4 * (r32 >> 3) + (r32 & 3), hh = (r32 >> 2) & 1;
    const int row = row0 + rr;
    if (row >= n_rows) return;  // after the only barrier
#pragma unroll 4
    for (int e = 0; e < 16; ++e) {
        const int tk = 16 * (tid >> 6) + e, j = tk >> 5;
        const int tok = tok0 + tk;
        if (tok >= m) break;
        const int ln = ((tk & 31) + 32 * hh) ^ (r + 16 * i);
        const int32_t v = ((red[0][2 * i + j][r][ln] + red[1][2 * i + j][r][ln]) + red[2][2 * i + j][r][ln]) +
                          red[3][2 * i + j][r][ln];
        if constexpr (SPLIT) {
            part[((size_t)sp * m + tok) * n_rows + row] = v;
        } else {
            const int2 mt = meta[tok];
            const int32_t t = v - mt.y;
            if constexpr (OUT == I2S_OUT_SUMS) iout[(size_t)tok * n_rows + row] = t;
            else dst[(size_t)tok * ldd + row] = (float)t * (__int_as_float(mt.x) * wscale);
        }
    }
}

float* amv_splitk_workspace(size_t bytes, hipStream_t st);

extern "C" int64_t amv_i2s_act_bytes(int64_t m, int64_t k) { return (m < 0 || k < 0) ? -1 : m * k + m * 8; }

extern "C" int amv_i2s_quantize_act(const float* x, int64_t m, int64_t k, void* act, void* stream) {
    AMV_REQUIRE(x && act, "amv_i2s_quantize_act: null pointer");
    AMV_REQUIRE(m > 0 && k > 0 && k <= INT32_MAX && m <= 65535 * 1024, "amv_i2s_quantize_act: bad shape");
    AMV_REQUIRE(((uintptr_t)act & 15) == 0, "amv_i2s_quantize_act: act must be 16-byte aligned");
    AMV_REQUIRE(k % 128 == 0, "amv_i2s_quantize_act: k %% 128 != 0");
    int8_t* q = (int8_t*)act;
    int2* meta = (int2*)((uint8_t*)act + m * k);
    hipLaunchKernelGGL(k_i2s_quant, dim3((unsigned)m), dim3(256), 0, amv_stream(stream), x, (int)k, q, meta);
    return amv_check_launch("amv_i2s_quantize_act");
}

// batch from which the MFMA kernel runs (as the Q4_0 / Q8_0 MUL_MAT, AMEVA_QGEMM_MIN_M = 8)
#define I2S_MMQ_MIN_M 8
// The batched launch (k_i2s_mmq_p): 64 x 64 tiles, k split over S workgroups when the tiles alone leave CUs idle (about
// one workgroup per CU: the four-block prefetch keeps a wave's 250 VGPRs, one wave per SIMD), the partials added by
// k_i2s_split_sum. The integers do not depend on S (exact in any order): without the workspace (first needed under
// capture) the launch runs unsplit. Measured on MI355X at batch 128, cold weights, graph replays (bench.py
// --only-i2s): 2560 x 6912 (80 tiles, 3 splits) 15.1 us (2, 4, 6 splits: 17.2, 18.4, 17.7; the former 128 x 64-tile
// split kernel 17.3); 6912 x 2560 (216 tiles, unsplit) 12.6 us (2 splits 18.0; the former 64 x 64 kernel with
// one block of lookahead 13.4). Prefetching all of a wave's blocks (up to 8) measured the same as 4. Staging the
// activations through LDS with whole-line loads (8 lanes per 128-byte token row, XOR-swizzled slots, conflict-free
// operand reads) measured 1.7-1.8x slower (23.0 / 25.8 us): the scattered direct operand loads are not what bounds
// these launches.
static void i2s_mmq_p(const void* w, int64_t n_rows, int kb, const void* act, int64_t m, float wscale, float* dst,
                      int64_t ldd, int32_t* sums, hipStream_t st) {
    const int64_t n_rt = (n_rows + 63) / 64, n_tt = (m + 63) / 64, tiles = n_rt * n_tt;
    int S = (int)std::min<int64_t>({(int64_t)kb, (int64_t)16, std::max<int64_t>(1, 256 / tiles)});
    int kb_per = (kb + S - 1) / S;
    S = (kb + kb_per - 1) / kb_per;
    int32_t* part = nullptr;
    if (S > 1) {
        const size_t bytes = (size_t)S * m * n_rows * 4;
        part = bytes <= AMV_SPLITK_WS_BYTES ? reinterpret_cast<int32_t*>(amv_splitk_workspace(bytes, st)) : nullptr;
        if (!part) {
            S = 1;
            kb_per = kb;
        }
    }
    const int8_t* q = (const int8_t*)act;
    const int2* meta = (const int2*)((const uint8_t*)act + m * (int64_t)kb * 128);
    const uint8_t* wp = (const uint8_t*)w;
    const int nbw = (kb_per + 3) / 4;  // blocks of the busiest wave
    const unsigned n_wg = (unsigned)(tiles * S);
#define I2S_P(OUT, SPLIT, PB, D, L, IO)                                                                               \
    hipLaunchKernelGGL((k_i2s_mmq_p<OUT, SPLIT, PB>), dim3(n_wg), dim3(256), 0, st, wp, (int)n_rows, kb, q, meta,     \
                       (int)m, kb_per, (int)n_rt, (int)n_tt, S, wscale, D, L, IO, part)
#define I2S_PB(OUT, SPLIT, D, L, IO)          \
    if (nbw <= 2) I2S_P(OUT, SPLIT, 2, D, L, IO); \
    else I2S_P(OUT, SPLIT, 4, D, L, IO)
    if (S == 1) {
        if (sums) {
            I2S_PB(I2S_OUT_SUMS, false, nullptr, (int64_t)0, sums);
        } else {
            I2S_PB(I2S_OUT_F32, false, dst, ldd, nullptr);
        }
        return;
    }
    I2S_PB(I2S_OUT_F32, true, nullptr, (int64_t)0, nullptr);
#undef I2S_PB
#undef I2S_P
    const dim3 g2((unsigned)((n_rows + 1023) / 1024), (unsigned)m);
    const bool vec = n_rows % 4 == 0;
#define I2S_SUM(SU, V) hipLaunchKernelGGL((k_i2s_split_sum<SU, V>), g2, dim3(256), 0, st, part, S, (int)n_rows, (int)m, \
                                          meta, wscale, dst, ldd, sums)
    if (sums) {
        if (vec) I2S_SUM(true, true);
        else I2S_SUM(true, false);
    } else {
        if (vec) I2S_SUM(false, true);
        else I2S_SUM(false, false);
    }
#undef I2S_SUM
}

static int i2s_gemv_impl(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float wscale,
                         float* dst, int64_t ldd, int32_t* sums, void* stream) {
    AMV_REQUIRE(w && act && (dst || sums), "amv_i2s_gemv: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0 && m > 0 && n_rows <= INT32_MAX && m <= 65535LL * 64 && n_rows * k / 4 < (1LL << 40),
                "amv_i2s_gemv: bad shape");
    AMV_REQUIRE(k % 128 == 0, "amv_i2s_gemv: k %% 128 != 0 (k = %lld)", (long long)k);
    AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0, "amv_i2s_gemv: buffers must be 16-byte aligned");
    AMV_REQUIRE(!dst || ldd >= n_rows, "amv_i2s_gemv: ldd < n_rows");
    hipStream_t st = amv_stream(stream);
    if (m >= I2S_MMQ_MIN_M) {
        i2s_mmq_p(w, n_rows, (int)(k / 128), act, m, wscale, dst, ldd, sums, st);
        return amv_check_launch("amv_i2s_gemv");
    }
    const int nsl = (int)(k / 64);
    const int R = 2;
    const int waves = (int)((n_rows + R - 1) / R);
    for (int64_t c = 0; c < m; ++c) {
        const int8_t* q = (const int8_t*)act + c * k;
        const int2* meta = (const int2*)((const uint8_t*)act + m * k) + c;
        if (sums) {
            hipLaunchKernelGGL((k_i2s_gemv<R, true>), dim3((waves + 3) / 4), dim3(256), 0, st, (const uint4*)w,
                               (int)n_rows, nsl, q, meta, wscale, nullptr, sums + c * n_rows);
        } else {
            hipLaunchKernelGGL((k_i2s_gemv<R, false>), dim3((waves + 3) / 4), dim3(256), 0, st, (const uint4*)w,
                               (int)n_rows, nsl, q, meta, wscale, dst + c * ldd, nullptr);
        }
    }
    return amv_check_launch("amv_i2s_gemv");
}

extern "C" int amv_i2s_gemv(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m, float weight_scale,
                            float* dst, int64_t ldd, void* stream) {
    AMV_REQUIRE(dst, "amv_i2s_gemv: null dst");
    return i2s_gemv_impl(w, n_rows, k, act, m, weight_scale, dst, ldd, nullptr, stream);
}

// dst[r] += float(isum_r) * (act_dequant * weight_scale) for one activation row (the residual add fused)
extern "C" int amv_i2s_gemv_acc(const void* w, int64_t n_rows, int64_t k, const void* act, float weight_scale,
                                float* dst, void* stream) {
    AMV_REQUIRE(w && act && dst, "amv_i2s_gemv_acc: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0 && n_rows <= INT32_MAX && k % 128 == 0, "amv_i2s_gemv_acc: bad shape");
    AMV_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)act & 15) == 0, "amv_i2s_gemv_acc: buffers must be 16-byte aligned");
    const int waves = (int)((n_rows + 1) / 2);
    const int8_t* q = (const int8_t*)act;
    const int2* meta = (const int2*)((const uint8_t*)act + k);
    hipLaunchKernelGGL((k_i2s_gemv<2, false, true>), dim3((waves + 3) / 4), dim3(256), 0, amv_stream(stream),
                       (const uint4*)w, (int)n_rows, (int)(k / 64), q, meta, weight_scale, dst, nullptr);
    return amv_check_launch("amv_i2s_gemv_acc");
}

extern "C" int amv_i2s_gemv_sums(const void* w, int64_t n_rows, int64_t k, const void* act, int64_t m,
                                 int32_t* sums, void* stream) {
    AMV_REQUIRE(sums, "amv_i2s_gemv_sums: null output");
    return i2s_gemv_impl(w, n_rows, k, act, m, 0.0f, nullptr, 0, sums, stream);
}

// ---------------------------------------------------------------------------------------------------------------
// Ternary GEMV on f32 activations, the amuda entry's arithmetic (bitnet_gemv_i2_s_exact, reference
// src/amuda/amuda_ops.c:91-121 and :299-352): y[r] = scale * sum_j map(c_rj) x_j with map = {-1, 0, +1, 0} for codes
// 0..3 (code 3 contributes nothing, unlike the integer path's c - 1). One wave per row; lane l takes bytes
// 16 l .. 16 l + 15 of each 1 KiB step of the row (one 16-byte load), i.e. half of a 32-byte block: weights
// 128 b + 16 (l % 2) + i + 32 g for byte i and code group g. f32 products summed per lane, then a wave sum; the order
// differs from the reference's sequential loop (the bar is f32 tolerance, as in its own test).
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_i2s_gemv_f32(const uint8_t* __restrict__ w, int n_rows, int k,
                                                     const float* __restrict__ x, float scale,
                                                     float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;  // uniform per wave
    const int rb = k / 4;       // bytes per row
    const uint8_t* wr = w + (size_t)row * rb;
    float acc = 0.0f;
    for (int b0 = 16 * lane; b0 < rb; b0 += 1024) {
        const uint4 v = amv_ld_stream(reinterpret_cast<const uint4*>(wr + b0));
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
        const int blk = b0 >> 5, half = (b0 >> 4) & 1;
        const float* xb = x + 128 * blk + 16 * half;
#pragma unroll
        for (int g = 0; g < 4; ++g) {  // code group g: bits 7-6, 5-4, 3-2, 1-0 of each byte
            const float4* xg = reinterpret_cast<const float4*>(xb + 32 * g);
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 xv = xg[q4];
                const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t c = (wd[q4] >> (8 * e + 6 - 2 * g)) & 3u;
                    const float m = c == 0u ? -1.0f : (c == 2u ? 1.0f : 0.0f);
                    acc = fmaf(m, xs[e], acc);
                }
            }
        }
    }
    acc = amv_wave_sum(acc);
    if (lane == 0) y[row] = acc * scale;
}

extern "C" int amv_i2s_gemv_f32(const void* w, int64_t n_rows, int64_t k, const float* x, float scale, float* y,
                                void* stream) {
    AMV_REQUIRE(w && x && y, "amv_i2s_gemv_f32: null pointer");
    AMV_REQUIRE(n_rows > 0 && k > 0 && n_rows <= INT32_MAX && k <= INT32_MAX, "amv_i2s_gemv_f32: bad shape");
    AMV_REQUIRE(k % 128 == 0, "amv_i2s_gemv_f32: k %% 128 != 0");
    AMV_REQUIRE(k % 64 == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0,
                "amv_i2s_gemv_f32: w and x must be 16-byte aligned");
    hipLaunchKernelGGL(k_i2s_gemv_f32, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0, amv_stream(stream),
                       (const uint8_t*)w, (int)n_rows, (int)k, x, scale, y);
    return amv_check_launch("amv_i2s_gemv_f32");
}
