// FLASH_ATTN_EXT over many query positions (prefill) on the f16 matrix cores of MI355X.
//
// Role of ameva_flash_attn.comp for a prompt (reference: enc_flash_attn ggml-ameva.cpp:4204-4284 with ne[1] > 1):
// out[t][h] = softmax(scale * q_t k^T + mask_t) v over the keys query t may see. ggml's CPU kernel rounds q to f16
// before the dot with the f16 K; so does this one. Scores, softmax and accumulators are f32; the probabilities enter
// the P V product as f16 (the CPU accumulates V in f16 instead).
//
// One workgroup of 4 waves per (head, 32 consecutive queries); the waves split the tile's blocks of 32 keys (wave w
// takes blocks w, w + 4, ...: the last tile of a 512-token causal prompt runs 4 blocks per wave, not 16 in a row)
// and merge their (m, l, O) through LDS at the end. Per block, each wave with v_mfma_f32_32x32x16_f16 (the full-rate
// f16 shape of gfx950):
//   S^T (32 keys x 32 queries) = K (32 keys x 128) . Q^T, 8 steps of 16 dims: lane l reads 16 contiguous bytes of
//   key l % 32 from the wave's K rows in LDS, Q^T is held in registers as f16 for the whole kernel. In the result lane
//   (c, h = l / 32) holds query c and keys 8 (r / 4) + 4 h + r % 4, r = 0..15.
//   O^T (128 dims x 32 queries) += V^T . P^T, per 32-dim tile 2 steps of 16 keys. The k slots of a step are assigned
//   so that P^T is exactly the lane's own S values (slots 0..3 = keys 16 s + 4 h + 0..3, slots 4..7 = keys
//   16 s + 8 + 4 h + 0..3: r = 8 s .. 8 s + 7), and the V^T operand comes from the row-major V block in LDS through
//   ds_read_b64_tr_b16: in each group of 16 lanes lane i receives element (4 e + i / 4, i % 4) of the 16 x 4 block the
//   group addressed, so lanes pointing at (key k0 + j / 4, dims d0 + 4 (j % 4) .. + 3) give lane i dim d0 + i of keys
//   k0 .. k0 + 3: two such reads are one operand, no transposed staging.
// Each wave stages its own K and V rows: 16 lanes per 256-byte row, 4 rows per load instruction (the loads that
// gather 16 or 32 bytes from 32 rows per instruction took half as long again), one block ahead of the one in use.
// Online softmax per query over the 16 scores of the lane and of its partner lane l ^ 32; causal tiles stop at the
// last key their last query may see, and the tiles with the most keys are launched first.
#include "amv_common.h"

#define FQ_D 128
#define FQ_KB 32            // keys per block
#define FQ_LOG2E 1.4426950408889634f
#define FQ_KLD (FQ_D + 8)   // K row stride in halves (272 bytes: the 16-byte fragment reads of 16 rows hit distinct banks)
#define FQ_VLD (FQ_D + 16)  // V row stride in halves (288 bytes: the transposing reads of 4 rows hit distinct banks)

typedef _Float16 fq_h8 __attribute__((ext_vector_type(8)));
typedef short fq_s4 __attribute__((ext_vector_type(4)));
typedef float fq_f16v __attribute__((ext_vector_type(16)));
typedef float fq_f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) fq_s4 fq_lds_s4;

// 8 halves for the V^T operand: dims d0 + i of keys k0 .. k0 + 3 and k0 + 8 .. k0 + 11 (lane i of its 16-lane group)
__device__ __forceinline__ fq_h8 fq_vt(const uint16_t* vb, int k0, int d0, int j) {
    const uint16_t* p = vb + (k0 + (j >> 2)) * FQ_VLD + d0 + 4 * (j & 3);
    const fq_s4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fq_lds_s4*)(__attribute__((address_space(3))) uint16_t*)p);
    const fq_s4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (fq_lds_s4*)(__attribute__((address_space(3))) uint16_t*)(p + 8 * FQ_VLD));
    typedef short fq_s8 __attribute__((ext_vector_type(8)));
    const fq_s8 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(fq_h8, ab);
}

// orders one wave's LDS accesses at this point (no instruction: a wave's LDS operations already run in order)
__device__ __forceinline__ void fq_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// rows key0 + 4 i (i = 0..7, clamped to the last key), 16 bytes from half col of each
typedef unsigned int fq_u4 __attribute__((ext_vector_type(4)));
struct FqRows {
    fq_u4 r[8];
};
__device__ __forceinline__ FqRows fq_load_rows(const uint16_t* __restrict__ base, int64_t row, int key0, int col,
                                               int n_kv) {
    FqRows t;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        t.r[i] = *reinterpret_cast<const fq_u4*>(base + (int64_t)min(key0 + 4 * i, n_kv - 1) * row + col);
    return t;
}

template <bool MASK>
__global__ __launch_bounds__(256) void k_fa_prefill(const float* __restrict__ q, int64_t q_ts, int64_t q_hs,
                                                   const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                   const uint16_t* __restrict__ mask, int64_t mask_stride,
                                                   float* __restrict__ out, int n_tok, int n_head, int G, int n_kv,
                                                   int64_t k_row, int64_t k_head, int64_t v_row, int64_t v_head,
                                                   float scale, int64_t pos0) {
    // per wave the K and V rows of the block it works on; after the key loop the partials of the merge
    __shared__ __align__(16) uint16_t lds[4 * FQ_KB * (FQ_KLD + FQ_VLD)];
    const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // the wave (uniform: block loop and tests run scalar)
    const int n_tiles = (int)gridDim.x;
    const int q0 = (n_tiles - 1 - (int)blockIdx.x) * 32;  // the tiles with the most keys first
    const int hq = (int)blockIdx.y, hk = hq / G;
    const int qi = q0 + c, qc = min(qi, n_tok - 1);

    // the query rows: loads first, converted to the f16 Q^T operand once the first K / V block is in flight
    fq_f4 qa[16];  // q[qi][16 s + 8 h .. + 7] = qa[2 s], qa[2 s + 1]
    {
        const float* qr = q + (int64_t)qc * q_ts + (int64_t)hq * q_hs + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            qa[2 * s] = *reinterpret_cast<const fq_f4*>(qr + 16 * s);
            qa[2 * s + 1] = *reinterpret_cast<const fq_f4*>(qr + 16 * s + 4);
        }
    }
    // keys this tile needs: up to the last key its last query may see; wave w takes blocks w, w + 4, ...
    int kend = n_kv;
    if (pos0 >= 0) kend = (int)min((int64_t)kend, pos0 + min(q0 + 31, n_tok - 1) + 1);
    const int nblk = (kend + FQ_KB - 1) / FQ_KB;
    // last key this query may see (causal limit and n_kv); keys below klim0 are visible to every query of the tile
    const int qlim = (int)min(pos0 >= 0 ? pos0 + qi : (int64_t)n_kv, (int64_t)n_kv - 1);
    const int klim0 = (int)min(pos0 >= 0 ? pos0 + q0 + 1 : (int64_t)n_kv, (int64_t)n_kv);
    const float sl2 = scale * FQ_LOG2E;

    const uint16_t* kh = k + (int64_t)hk * k_head;
    const uint16_t* vh = v + (int64_t)hk * v_head;
    uint16_t* kb = lds + w * FQ_KB * (FQ_KLD + FQ_VLD);
    uint16_t* vb = kb + FQ_KB * FQ_KLD;
    // K / V staging of a block by the wave alone: lane l moves rows l / 16 + 4 i (i = 0..7), dims 8 (l % 16) ..
    const int srow = lane >> 4, scol = 8 * (lane & 15);
    FqRows rk, rv;

    float m = -INFINITY, l = 0.0f;
    fq_f16v o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;

    const int j16 = lane & 15, g16 = lane >> 4;  // the transposing reads: lane index in its 16-lane group, the group
    // The wave's next block is in flight while it works on the current one, loaded unconditionally (the last block
    // again at the end: the addresses stay in bounds, the values go unused), so the loads of one iteration retire in
    // issue order and no wait covers a prefetch.
    const int kmax = n_kv - 1;
    if (w < nblk) {
        rk = fq_load_rows(kh, k_row, FQ_KB * w + srow, scol, n_kv);
        rv = fq_load_rows(vh, v_row, FQ_KB * w + srow, scol, n_kv);
    }
    fq_h8 qb[8];  // Q^T operand: qb[s] = q[qi][16 s + 8 h .. + 7] as f16
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const fq_f4 a = qa[2 * s], b = qa[2 * s + 1];
        qb[s] = fq_h8{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                      (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
    }
    for (int b = w; b < nblk; b += 4) {
        const int kb0 = FQ_KB * b, bn = min(b + 4, nblk - 1);
        // this block's K and V rows into the wave's LDS, the K fragments back out (lane: key c, dims 16 st + 8 h ..)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            *reinterpret_cast<fq_u4*>(&kb[(srow + 4 * i) * FQ_KLD + scol]) = rk.r[i];
            *reinterpret_cast<fq_u4*>(&vb[(srow + 4 * i) * FQ_VLD + scol]) = rv.r[i];
        }
        fq_wave_sync();
        fq_h8 kf[8];
#pragma unroll
        for (int st = 0; st < 8; ++st) kf[st] = *reinterpret_cast<const fq_h8*>(&kb[c * FQ_KLD + 16 * st + 8 * h]);
        float mk[16];
        if (MASK) {
            const uint16_t* mr = mask + (int64_t)qc * mask_stride;
#pragma unroll
            for (int r = 0; r < 16; ++r) mk[r] = amv_h2f(mr[min(kb0 + 8 * (r >> 2) + 4 * h + (r & 3), kmax)]);
        }
        rk = fq_load_rows(kh, k_row, FQ_KB * bn + srow, scol, n_kv);
        rv = fq_load_rows(vh, v_row, FQ_KB * bn + srow, scol, n_kv);
        // S^T = K Q^T
        fq_f16v s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < 8; ++st) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[st], qb[st], s, 0, 0, 0);
        // scores in log2 units (scale * log2 e folded in), the mask added, keys past the causal limit or n_kv at
        // -inf; blocks wholly inside every query's limit (most blocks of a causal prompt) skip the key tests
        const bool full = kb0 + FQ_KB <= klim0;
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float x = MASK ? (s[r] * scale + mk[r]) * FQ_LOG2E : s[r] * sl2;
            if (!full) {
                const int key = kb0 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (key > qlim) x = -INFINITY;
            }
            s[r] = x;
            mx = fmaxf(mx, x);
        }
        mx = amv_max_x32(mx);  // the query's maximum over the block's 32 keys
        // The running maximum moves only when a block exceeds it by more than 8 (a factor 256): until then the
        // exponentials stay below 256 (exact enough in f16 for P, the sums are f32) and the accumulators need no
        // rescaling, which most blocks then skip as a whole wave.
        const bool grow = mx > m + 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float alpha = grow ? (m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mx)) : 1.0f;
            if (grow) m = mx;
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        }
        const float mref = m == -INFINITY ? 0.0f : m;  // nothing visible yet: every score is -inf, every weight 0
        float rs = 0.0f;
        fq_h8 p0, p1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float e = __builtin_amdgcn_exp2f(s[r] - mref);
            rs += e;
            if (r < 8) p0[r] = (_Float16)e;
            else p1[r - 8] = (_Float16)e;
        }
        l += amv_sum_x32(rs);
        // O^T += V^T P^T (the V rows were written by this wave before the fence: LDS operations of one wave complete in
        // order)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const fq_h8 a = fq_vt(vb, 16 * ks + 4 * (g16 >> 1), 32 * dt + 16 * (g16 & 1), j16);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ks ? p1 : p0, o[dt], 0, 0, 0);
            }
        }
        fq_wave_sync();  // the K / V reads stay before the next block's writes
    }
    // merge: every wave leaves its (m, l, O^T) in LDS, then wave w combines dims 32 w .. 32 w + 31 of the tile's
    // queries over the four waves (lane for lane the same query and dims) and writes them
    __syncthreads();  // every wave is done with its K / V rows
    fq_f4* mo = reinterpret_cast<fq_f4*>(lds);          // [wave][dt][q4][lane]: o[dt][4 q4 .. 4 q4 + 3]
    float* mml = reinterpret_cast<float*>(lds) + 16384;  // [wave][m, l][lane]
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
            mo[((w * 4 + dt) * 4 + q4) * 64 + lane] =
                fq_f4{o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]};
    mml[2 * w * 64 + lane] = m;
    mml[(2 * w + 1) * 64 + lane] = l;
    __syncthreads();
    float mj[4], M = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mj[j] = mml[2 * j * 64 + lane];
        M = fmaxf(M, mj[j]);
    }
    float L = 0.0f;
    fq_f4 acc[4] = {};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float f = mj[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mj[j] - M);
        L += mml[(2 * j + 1) * 64 + lane] * f;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) acc[q4] += mo[((j * 4 + w) * 4 + q4) * 64 + lane] * f;
    }
    if (qi < n_tok) {
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        float* orow = out + ((int64_t)qi * n_head + hq) * FQ_D + 32 * w + 4 * h;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) *reinterpret_cast<fq_f4*>(orow + 8 * q4) = acc[q4] * inv;
    }
}

extern "C" int amv_flash_attn_prefill(const float* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k,
                                      const void* v, const void* mask, int64_t mask_stride, float* out, int64_t n_tok,
                                      int64_t n_head, int64_t n_head_kv, int64_t n_kv, int64_t D, int64_t k_row,
                                      int64_t k_head, int64_t v_row, int64_t v_head, float scale, int64_t causal_pos0,
                                      void* stream) {
    AMV_REQUIRE(q && k && v && out, "amv_flash_attn_prefill: null pointer");
    AMV_REQUIRE(D == FQ_D, "amv_flash_attn_prefill: head size %lld not supported (128 is)", (long long)D);
    AMV_REQUIRE(n_tok > 0 && n_kv > 0 && n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0,
                "amv_flash_attn_prefill: bad shape");
    AMV_REQUIRE(n_tok <= (int64_t)1 << 24 && n_kv <= (int64_t)1 << 24 && n_head <= 65535,
                "amv_flash_attn_prefill: shape too large");
    AMV_REQUIRE(((uintptr_t)q & 15) == 0 && q_tok_stride % 4 == 0 && q_head_stride % 4 == 0,
                "amv_flash_attn_prefill: q rows must be 16-byte aligned");
    AMV_REQUIRE(((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 && k_row % 8 == 0 && k_head % 8 == 0 &&
                    v_row % 8 == 0 && v_head % 8 == 0,
                "amv_flash_attn_prefill: K/V rows must be 16-byte aligned");
    AMV_REQUIRE(((uintptr_t)out & 15) == 0, "amv_flash_attn_prefill: out must be 16-byte aligned");
    AMV_REQUIRE(mask == nullptr || mask_stride >= n_kv, "amv_flash_attn_prefill: mask stride %lld < n_kv",
                (long long)mask_stride);
    const dim3 grid((unsigned)((n_tok + 31) / 32), (unsigned)n_head);
    hipLaunchKernelGGL(mask ? k_fa_prefill<true> : k_fa_prefill<false>, grid, dim3(256), 0, amv_stream(stream), q, q_tok_stride, q_head_stride,
                       (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)mask, mask_stride, out, (int)n_tok,
                       (int)n_head, (int)(n_head / n_head_kv), (int)n_kv, k_row, k_head, v_row, v_head, scale,
                       causal_pos0);
    return amv_check_launch("amv_flash_attn_prefill");
}
