/* Test double of the ggml host (libggml-base) for the plugin tests: ggml_backend_buffer_init (the one function a
 * backend plugin links against), the libggml-base accessors the plugin's load-time ABI check reads its structs back
 * through (ggml_backend_get_device, ggml_backend_buffer_get_size/_type, ggml_backend_buft_get_device,
 * ggml_backend_dev_backend_reg, ggml_op_name, ggml_type_name, and a minimal context that builds one MUL_MAT node), plus
 * the host-side buffer calls a test needs (set usage, free). Loaded with RTLD_GLOBAL before libggml-ameva.so so that
 * the plugin's symbols bind here, as they bind to libggml-base under llama.cpp. Test infrastructure only.
 *
 * Built with -DGGML_TESTHOST_SKEW=1 it reads struct ggml_backend as a host whose ggml_backend_i has one member fewer
 * (device one slot earlier); with -DGGML_TESTHOST_SKEW=2 it cuts tensor names as a host built with GGML_MAX_NAME 128:
 * hosts the plugin must refuse. */
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#include "../../ameva_compute_amd/csrc/ggml_abi.h"

#ifndef GGML_TESTHOST_SKEW
#define GGML_TESTHOST_SKEW 0
#endif

ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void* context, size_t size) {
    struct ggml_backend_buffer* b = (struct ggml_backend_buffer*)calloc(1, sizeof(*b));
    b->iface = iface;
    b->buft = buft;
    b->context = context;
    b->size = size;
    b->usage = GGML_BACKEND_BUFFER_USAGE_ANY;
    return b;
}

void ggml_testhost_buffer_set_usage(ggml_backend_buffer_t b, int usage) { b->usage = (enum ggml_backend_buffer_usage)usage; }

void ggml_testhost_buffer_free(ggml_backend_buffer_t b) {
    if (b->iface.free_buffer) b->iface.free_buffer(b);
    free(b);
}

size_t ggml_testhost_tensor_size(void) { return sizeof(struct ggml_tensor); }
size_t ggml_testhost_cgraph_size(void) { return sizeof(struct ggml_cgraph); }

/* ---- accessors (ggml-backend.h) */
ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend) {
#if GGML_TESTHOST_SKEW == 1
    return ((ggml_backend_dev_t*)&backend->device)[-1];
#else
    return backend->device;
#endif
}
size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) { return buffer->size; }
ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer) { return buffer->buft; }
ggml_backend_dev_t ggml_backend_buft_get_device(ggml_backend_buffer_type_t buft) { return buft->device; }
ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t device) { return device->reg; }

/* ---- names of the enum values ggml_abi.h declares (the host names ops and types by value) */
const char* ggml_op_name(enum ggml_op op) {
    switch (op) {
    case GGML_OP_NONE: return "NONE";
    case GGML_OP_DUP: return "DUP";
    case GGML_OP_ADD: return "ADD";
    case GGML_OP_SUB: return "SUB";
    case GGML_OP_MUL: return "MUL";
    case GGML_OP_DIV: return "DIV";
    case GGML_OP_RMS_NORM: return "RMS_NORM";
    case GGML_OP_MUL_MAT: return "MUL_MAT";
    case GGML_OP_SCALE: return "SCALE";
    case GGML_OP_CPY: return "CPY";
    case GGML_OP_CONT: return "CONT";
    case GGML_OP_RESHAPE: return "RESHAPE";
    case GGML_OP_VIEW: return "VIEW";
    case GGML_OP_PERMUTE: return "PERMUTE";
    case GGML_OP_TRANSPOSE: return "TRANSPOSE";
    case GGML_OP_GET_ROWS: return "GET_ROWS";
    case GGML_OP_SET_ROWS: return "SET_ROWS";
    case GGML_OP_SOFT_MAX: return "SOFT_MAX";
    case GGML_OP_ROPE: return "ROPE";
    case GGML_OP_FLASH_ATTN_EXT: return "FLASH_ATTN_EXT";
    case GGML_OP_UNARY: return "UNARY";
    case GGML_OP_GLU: return "GLU";
    default: return "?";
    }
}
const char* ggml_type_name(enum ggml_type type) {
    switch (type) {
    case GGML_TYPE_F32: return "f32";
    case GGML_TYPE_F16: return "f16";
    case GGML_TYPE_Q4_0: return "q4_0";
    case GGML_TYPE_Q8_0: return "q8_0";
    case GGML_TYPE_Q4_K: return "q4_K";
    case GGML_TYPE_Q6_K: return "q6_K";
    case GGML_TYPE_Q8_K: return "q8_K";
    case GGML_TYPE_I32: return "i32";
    case GGML_TYPE_I64: return "i64";
    default: return "?";
    }
}

/* ---- a context of F32 tensors, enough for the plugin's MUL_MAT layout probe */
struct ggml_init_params {
    size_t mem_size;
    void* mem_buffer;
    bool no_alloc;
};
#define TESTHOST_MAX_TENSORS 16
struct ggml_context {
    struct ggml_tensor* t[TESTHOST_MAX_TENSORS];
    int n;
};

size_t ggml_tensor_overhead(void) { return sizeof(struct ggml_tensor) + 16; }

struct ggml_context* ggml_init(struct ggml_init_params params) {
    (void)params;
    return (struct ggml_context*)calloc(1, sizeof(struct ggml_context));
}

void ggml_free(struct ggml_context* ctx) {
    if (!ctx) return;
    for (int i = 0; i < ctx->n; ++i) free(ctx->t[i]);
    free(ctx);
}

static struct ggml_tensor* new_tensor(struct ggml_context* ctx, int64_t ne0, int64_t ne1) {
    if (ctx->n >= TESTHOST_MAX_TENSORS) return NULL;
    /* room behind the struct: the GGML_MAX_NAME 128 variant writes names past name[64] */
    struct ggml_tensor* t = (struct ggml_tensor*)calloc(1, sizeof(struct ggml_tensor) + 256);
    t->type = GGML_TYPE_F32;
    t->ne[0] = ne0;
    t->ne[1] = ne1;
    t->ne[2] = t->ne[3] = 1;
    t->nb[0] = 4;
    t->nb[1] = 4 * (size_t)ne0;
    t->nb[2] = t->nb[3] = t->nb[1] * (size_t)ne1;
    ctx->t[ctx->n++] = t;
    return t;
}

struct ggml_tensor* ggml_new_tensor_2d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0, int64_t ne1) {
    if (type != GGML_TYPE_F32) return NULL;
    return new_tensor(ctx, ne0, ne1);
}

struct ggml_tensor* ggml_mul_mat(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b) {
    if (a->ne[0] != b->ne[0]) return NULL;
    struct ggml_tensor* c = new_tensor(ctx, a->ne[1], b->ne[1]);
    if (!c) return NULL;
    c->op = GGML_OP_MUL_MAT;
    c->src[0] = a;
    c->src[1] = b;
    return c;
}

size_t ggml_nbytes(const struct ggml_tensor* t) {
    size_t n = (size_t)t->ne[0] * t->nb[0];
    for (int i = 1; i < GGML_MAX_DIMS; ++i) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    return n;
}

struct ggml_tensor* ggml_set_name(struct ggml_tensor* t, const char* name) {
#if GGML_TESTHOST_SKEW == 2
    const size_t cap = 128;
#else
    const size_t cap = sizeof(t->name);
#endif
    /* through a pointer into the whole allocation (new_tensor leaves 256 bytes behind the struct), not through the
     * name[] array: indexing name[] past its 64 bytes would be undefined, and the optimiser exploits it */
    char* dst = (char*)t + offsetof(struct ggml_tensor, name);
    size_t i = 0;
    for (; i + 1 < cap && name[i]; ++i) dst[i] = name[i];
    dst[i] = 0;
    return t;
}

const char* ggml_get_name(const struct ggml_tensor* t) { return t->name; }
