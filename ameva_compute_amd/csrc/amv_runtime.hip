// Host-side plumbing of the kernel ABI: per-thread error message, launch checks, sizes of the layouts.
#include <stdarg.h>
#include <stdio.h>

#include "amv_common.h"

static thread_local char g_err[512] = {0};

void amv_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int amv_check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        amv_set_error("%s: %s", what, hipGetErrorString(e));
        return AMV_ERR_HIP;
    }
    return AMV_OK;
}

extern "C" const char* amv_last_error(void) { return g_err; }

extern "C" int amv_version(void) { return 100; }

static int64_t block_elems(int type) {
    switch (type) {
    case AMV_T_Q4_0:
    case AMV_T_Q8_0: return 32;
    case AMV_T_Q4_K:
    case AMV_T_Q6_K:
    case AMV_T_Q8_K: return 256;
    default: return 0;
    }
}

static int64_t block_bytes(int type) {
    switch (type) {
    case AMV_T_Q4_0: return 18;
    case AMV_T_Q8_0: return 34;
    case AMV_T_Q4_K: return 144;
    case AMV_T_Q6_K: return 210;
    case AMV_T_Q8_K: return 292;
    default: return 0;
    }
}

extern "C" int64_t amv_weight_bytes(int type, int64_t n_rows, int64_t k) {
    const int64_t be = block_elems(type);
    if (be == 0 || k % be != 0 || n_rows < 0) return -1;
    return n_rows * (k / be) * block_bytes(type);
}

extern "C" int64_t amv_act_bytes(int type, int64_t m, int64_t k) {
    if (m < 0) return -1;
    if (type == AMV_T_Q8_0 && k % 32 == 0) return m * k + m * (k / 32) * 8;
    if (type == AMV_T_Q8_K && k % 256 == 0) return m * k + m * (k / 256) * 4 + m * (k / 16) * 4;
    if ((type == AMV_ACT_Q8_K_MMA || type == AMV_ACT_Q8_K_DEQ) && k % 256 == 0) return amv_q8k_mma_layout(m, k).total;
    if ((type == AMV_ACT_Q8_0_MMA || type == AMV_ACT_Q8_0_DEQ) && k % 32 == 0) return amv_q8_0_mma_layout(m, k).total;
    return -1;
}
