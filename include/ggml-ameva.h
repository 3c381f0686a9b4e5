/*
 * ggml backend plugin "AMEVA" for MI355X: the drop-in boundary of the quantized hot path. A llama.cpp (b8471) host
 * loads libggml-ameva.so with ggml_backend_load() and gets one device, AMEVA0, whose graph_compute runs the HIP
 * kernels of libameva_hip.so (include/ameva_hip.h).
 *
 * Same entry points and meaning as the reference plugin's public header (adapters/llama/ggml-ameva/ggml-ameva.h:19-98);
 * the device description and the counters that only applied to the Vulkan/Mali kernels differ as noted. The ggml
 * types are those of ggml-backend.h; when this header is used without ggml's own headers, the opaque handles below
 * are the same typedefs.
 */
#ifndef GGML_AMEVA_H
#define GGML_AMEVA_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_AMEVA_NAME "AMEVA"
#define GGML_AMEVA_DEVICE_NAME "AMEVA0"
#define GGML_AMEVA_DEVICE_DESCRIPTION "AMEVA MI355X (gfx950) HIP quantized backend"

typedef struct ggml_backend* ggml_backend_t;
typedef struct ggml_backend_buffer_type* ggml_backend_buffer_type_t;
typedef struct ggml_backend_reg* ggml_backend_reg_t;

/* Backend and device lifecycle (ggml-ameva.h:19-24). Only device 0 exists (ggml-ameva.cpp:5684-5690). */
ggml_backend_t ggml_backend_ameva_init(size_t dev_num);
bool ggml_backend_is_ameva(ggml_backend_t backend);
ggml_backend_buffer_type_t ggml_backend_ameva_buffer_type(size_t dev_num);
ggml_backend_reg_t ggml_backend_ameva_reg(void);
void ggml_backend_ameva_register(void);
void ggml_backend_ameva_teardown(void);

/* Dynamic loader entry points (ggml-ameva.cpp:5693-5707): ggml_backend_load() resolves these two. */
ggml_backend_reg_t ggml_backend_init(void);
int ggml_backend_score(void);

/* Diagnostic counters (ggml-ameva.h:30-80), the ground truth tests use that a GPU kernel ran:
 *   gpu_op_count              graph nodes completed on the GPU (views and reshapes excluded)
 *   f32_gpu_sgemm_dispatch    MUL_MAT nodes completed on the GPU, any weight type (name kept for ABI)
 *   qmv_mul_mat_count         MUL_MAT nodes on repacked weights (every quantized MUL_MAT here)
 *   mmq_mul_mat_count         of those, the nodes that ran the int8-MFMA GEMM
 *   mmqb_mul_mat_count        stays 0 (the per-256 activation GEMM of the reference is not a separate kernel here)
 *   repacked_tensor_count / repacked_bytes  weights held in the MI355X layout (stored state)
 *   fused_pair_count          nodes computed by an earlier node's kernel (RMS_NORM + MUL)
 *   q5_0_* counters           stay 0 (names kept for ABI)
 *   act_quant_reuse_count     MUL_MATs that reused another node's quantized activations (no reference counterpart) */
int64_t ggml_backend_ameva_get_supports_query_count(void);
int64_t ggml_backend_ameva_get_supported_op_count(void);
int64_t ggml_backend_ameva_get_gpu_op_count(void);
int64_t ggml_backend_ameva_get_q5_0_cpu_dequant_count(void);
int64_t ggml_backend_ameva_get_f32_gpu_sgemm_dispatch_count(void);
int64_t ggml_backend_ameva_get_context_create_count(void);
int64_t ggml_backend_ameva_get_context_destroy_count(void);
int64_t ggml_backend_ameva_get_kernel_create_count(void);
int64_t ggml_backend_ameva_get_kernel_destroy_count(void);
int64_t ggml_backend_ameva_get_buffer_create_count(void);
int64_t ggml_backend_ameva_get_buffer_destroy_count(void);
int64_t ggml_backend_ameva_get_event_create_count(void);
int64_t ggml_backend_ameva_get_event_destroy_count(void);
int64_t ggml_backend_ameva_get_q5_0_staging_alloc_count(void);
int64_t ggml_backend_ameva_get_q5_0_staging_free_count(void);
int64_t ggml_backend_ameva_get_repacked_tensor_count(void);
int64_t ggml_backend_ameva_get_repacked_bytes(void);
int64_t ggml_backend_ameva_get_qmv_mul_mat_count(void);
int64_t ggml_backend_ameva_get_mmq_mul_mat_count(void);
int64_t ggml_backend_ameva_get_mmqb_mul_mat_count(void);
int64_t ggml_backend_ameva_get_fused_pair_count(void);
int64_t ggml_backend_ameva_get_act_quant_reuse_count(void);
/* Convolution, group-norm and windowed-node counters (ggml-ameva.h:70-78). This plugin declines CONV_2D and
 * GROUP_NORM in supports_op, so the counts stay 0 and conv_f16_decoder stays -1 ("not determined"). */
int64_t ggml_backend_ameva_get_conv_count(void);
int ggml_backend_ameva_get_conv_f16_decoder(void);
int64_t ggml_backend_ameva_get_conv_bias_count(void);
int64_t ggml_backend_ameva_get_group_norm_count(void);
int64_t ggml_backend_ameva_get_window_node_count(void);
const char* ggml_backend_ameva_get_build_commit(void);
/* The host ABI check that ggml_backend_init, ggml_backend_ameva_register and ggml_backend_ameva_init run before
 * anything of the plugin reaches libggml-base (the reference's internal ameva_abi_check, ggml-ameva-device.cpp:415-495;
 * exported here, with no counterpart in the reference's header, so a host or test can read the reason): NULL when the
 * loaded libggml-base reads the plugin's ggml_backend, buffer, buffer type, device and tensor structs at the offsets
 * this build uses and names every op and type value it dispatches on the same; else the mismatch. */
const char* ggml_backend_ameva_abi_check(void);
void ggml_backend_ameva_reset_counters(void);
/* Prints the AMEVA_PROFILE report now (ggml-ameva.h profile_report; ggml-ameva.cpp:208-277): with AMEVA_PROFILE=1
 * the per-graph totals (graphs, nodes, encoded launches, host encode and wait ms), with AMEVA_PROFILE=2 also the GPU
 * time per node kind (op, weight type, GEMV or batched kernel, fused partner) from a HIP event after every node.
 * AMEVA_TRACE=1 prints one line per graph before its launches and one after completion (ggml-ameva.cpp:5526). */
void ggml_backend_ameva_profile_report(void);

/* Failure injection (ggml-ameva.h:83-98): forces a failure from the host at the named point so the FAIL-FAST paths
 * can be tested without a faulty GPU. Every injected failure makes graph_compute return GGML_STATUS_FAILED (or the
 * buffer call report an error) without launching the affected kernel. */
typedef enum {
    AMEVA_FAIL_NONE = 0,
    AMEVA_FAIL_MAP_SRC0 = 1,
    AMEVA_FAIL_MAP_SRC1 = 2,
    AMEVA_FAIL_MAP_DST = 3,
    AMEVA_FAIL_FLUSH_SRC0 = 4,
    AMEVA_FAIL_FLUSH_SRC1 = 5,
    AMEVA_FAIL_DISPATCH = 6,
    AMEVA_FAIL_WAIT_TIMEOUT = 7,
    AMEVA_FAIL_INVALIDATE_DST = 8,
    AMEVA_FAIL_OFFSET_OVERFLOW = 9,
    AMEVA_FAIL_TENSOR_RANGE_OOB = 10,
} AmevaFailureInjectionPoint;

void ggml_backend_ameva_set_failure_injection(AmevaFailureInjectionPoint point);
AmevaFailureInjectionPoint ggml_backend_ameva_get_failure_injection(void);

/* The contract of supports_op / graph_compute for one node: NULL when the node is supported, else the reason
 * (ameva_op_unsupported_reason, ggml-ameva.cpp:1671). Exposed for tests and diagnostics (no reference export). */
const char* ggml_backend_ameva_op_unsupported_reason(const void* node);

#ifdef __cplusplus
}
#endif

#endif /* GGML_AMEVA_H */
