// Kernels the ac_runtime tests load as an AMDGPU code object (hipcc --genco): they follow the runtime's argument
// convention -- one pointer per binding, then the push-constant struct by value, then the specialization values.
#include <hip/hip_runtime.h>
#include <stdint.h>

struct AxpyPush {
    uint32_t n;
    float alpha;
};

// out = alpha * x + y (bindings x, y, out)
extern "C" __global__ void ac_axpy(const float* x, const float* y, float* out, AxpyPush p) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.n) out[i] = p.alpha * x[i] + y[i];
}

struct CountPush {
    uint32_t n;
};

// out = in + 1 (bindings in, out)
extern "C" __global__ void ac_add_one(const float* in, float* out, CountPush p) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.n) out[i] = in[i] + 1.0f;
}

struct ScaleSpec {
    uint32_t scale_bits;  // constant 3 (f32)
    uint32_t local_x;     // constant 7 (u32, overrides the local size x)
};

// out = x * scale + blockDim.x (bindings x, out); records the launch's workgroup size and the spec value
extern "C" __global__ void ac_scale_spec(const float* x, float* out, CountPush p, ScaleSpec s) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.n) out[i] = x[i] * __uint_as_float(s.scale_bits) + (float)(blockDim.x == s.local_x ? blockDim.x : 0u);
}
