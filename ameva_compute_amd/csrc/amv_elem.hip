// Glue ops of the decoder graph: ADD / MUL with row broadcast (residuals, norm weights), f32 -> f16 copies and
// SET_ROWS into an f16 KV cache, GET_ROWS (embedding lookup) from f32 / f16 / Q4_0 / Q8_0 / Q6_K rows.
// Roles of ameva_binary.comp, ameva_cpy.comp, ameva_set_rows.comp and ameva_get_rows(_q).comp of the reference.
#include "amv_common.h"

// dst[r][i] = a[r][i] op b[r % b_rows][i]   (op 0 add, 1 mul); n = elements per row
__global__ __launch_bounds__(256) void k_binary(const float* __restrict__ a, const float* __restrict__ b,
                                               float* __restrict__ dst, int64_t n_rows, int64_t n, int64_t b_rows,
                                               int op) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_rows * n) return;
    const int64_t r = i / n, c = i - r * n;
    const float x = a[i], y = b[(r % b_rows) * n + c];
    dst[i] = op == 0 ? x + y : x * y;
}

extern "C" int amv_binary(int op, const float* a, const float* b, float* dst, int64_t n_rows, int64_t n, int64_t b_rows,
                          void* stream) {
    AMV_REQUIRE(a && b && dst, "amv_binary: null pointer");
    AMV_REQUIRE(op == 0 || op == 1, "amv_binary: op %d (0 add, 1 mul)", op);
    AMV_REQUIRE(n_rows > 0 && n > 0 && b_rows > 0 && b_rows <= n_rows, "amv_binary: bad shape");
    const int64_t total = n_rows * n;
    hipLaunchKernelGGL(k_binary, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream), a, b, dst,
                       n_rows, n, b_rows, op);
    return amv_check_launch("amv_binary");
}

// f32 rows -> f16 rows at dst row idx[r] (SET_ROWS) or row r (idx NULL, CPY); row strides in elements.
// An index outside [0, dst_rows) is not written and is counted in *bad (the reference's status buffer).
__global__ __launch_bounds__(256) void k_rows_f16(const float* __restrict__ src, int64_t src_stride,
                                                 uint16_t* __restrict__ dst, int64_t dst_stride, int64_t n_rows,
                                                 int64_t n, const int64_t* __restrict__ idx64,
                                                 const int32_t* __restrict__ idx32, int64_t dst_rows,
                                                 unsigned int* __restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_rows * n) return;
    const int64_t r = i / n, c = i - r * n;
    int64_t dr = r;
    if (idx64) dr = idx64[r];
    else if (idx32) dr = idx32[r];
    if (dr < 0 || dr >= dst_rows) {
        if (c == 0 && bad) atomicAdd(bad, 1u);
        return;
    }
    dst[dr * dst_stride + c] = amv_f2h(src[r * src_stride + c]);
}

extern "C" int amv_set_rows_f16(const float* src, int64_t src_stride, void* dst, int64_t dst_stride, int64_t n_rows,
                                int64_t n, const void* idx, int idx_bits, int64_t dst_rows, unsigned int* bad,
                                void* stream) {
    AMV_REQUIRE(src && dst, "amv_set_rows_f16: null pointer");
    AMV_REQUIRE(n_rows > 0 && n > 0 && src_stride >= n && dst_stride >= n, "amv_set_rows_f16: bad shape");
    AMV_REQUIRE(idx == nullptr || idx_bits == 32 || idx_bits == 64, "amv_set_rows_f16: index type must be i32 or i64");
    AMV_REQUIRE(idx != nullptr || dst_rows >= n_rows, "amv_set_rows_f16: dst too small");
    const int64_t total = n_rows * n;
    hipLaunchKernelGGL(k_rows_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream), src,
                       src_stride, (uint16_t*)dst, dst_stride, n_rows, n,
                       idx_bits == 64 ? (const int64_t*)idx : nullptr, idx_bits == 32 ? (const int32_t*)idx : nullptr,
                       dst_rows, bad);
    return amv_check_launch("amv_set_rows_f16");
}

// GET_ROWS: dst f32 [n_idx][n] = dequantized row idx[i] of src (type F32, F16, Q4_0, Q8_0: ggml blocks, row stride
// in bytes). Dequantization as ggml's dequantize_row_* (ameva_get_rows_q.comp).
__global__ __launch_bounds__(256) void k_get_rows(const uint8_t* __restrict__ src, int64_t row_bytes, int type,
                                                 const int32_t* __restrict__ idx, int64_t n_idx, int64_t n,
                                                 int64_t src_rows, float* __restrict__ dst,
                                                 unsigned int* __restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_idx * n) return;
    const int64_t r = i / n, c = i - r * n;
    const int64_t sr = idx[r];
    if (sr < 0 || sr >= src_rows) {
        if (c == 0 && bad) atomicAdd(bad, 1u);
        dst[i] = 0.0f;
        return;
    }
    const uint8_t* row = src + sr * row_bytes;
    float v;
    if (type == AMV_T_F32) {
        v = reinterpret_cast<const float*>(row)[c];
    } else if (type == AMV_T_F16) {
        v = amv_h2f(reinterpret_cast<const uint16_t*>(row)[c]);
    } else if (type == AMV_T_Q4_0) {
        const uint8_t* blk = row + (c / 32) * 18;
        const int j = (int)(c % 32);
        const float d = amv_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const int nib = j < 16 ? (blk[2 + j] & 0xF) : (blk[2 + j - 16] >> 4);
        v = (float)(nib - 8) * d;
    } else {  // Q8_0
        const uint8_t* blk = row + (c / 32) * 34;
        const float d = amv_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        v = (float)(int8_t)blk[2 + c % 32] * d;
    }
    dst[i] = v;
}

extern "C" int amv_get_rows(int type, const void* src, int64_t src_rows, int64_t n, const int32_t* idx, int64_t n_idx,
                            float* dst, unsigned int* bad, void* stream) {
    AMV_REQUIRE(src && idx && dst, "amv_get_rows: null pointer");
    AMV_REQUIRE(n_idx > 0 && n > 0 && src_rows > 0, "amv_get_rows: bad shape");
    int64_t rb;
    switch (type) {
    case AMV_T_F32: rb = n * 4; break;
    case AMV_T_F16: rb = n * 2; break;
    case AMV_T_Q4_0: AMV_REQUIRE(n % 32 == 0, "amv_get_rows: n %% 32"); rb = n / 32 * 18; break;
    case AMV_T_Q8_0: AMV_REQUIRE(n % 32 == 0, "amv_get_rows: n %% 32"); rb = n / 32 * 34; break;
    default: amv_set_error("amv_get_rows: type %d not supported", type); return AMV_ERR_UNSUPPORTED;
    }
    const int64_t total = n_idx * n;
    hipLaunchKernelGGL(k_get_rows, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, amv_stream(stream),
                       (const uint8_t*)src, rb, type, idx, n_idx, n, src_rows, dst, bad);
    return amv_check_launch("amv_get_rows");
}
