// The part of ggml's binary interface (ggml 0.9.8 / llama.cpp b8471, GGML_BACKEND_API_VERSION 2) that a dynamically
// loaded backend plugin touches: the tensor and graph structs it reads and the five vtables it fills.
//
// libggml-base is not part of this repository, so these are this project's own declarations of that interface. A
// plugin is bound by the host's struct layouts, so field order and types follow ggml exactly (reference copy of the
// interface: include/ggml/ggml.h:394-437 (types), 673-705 (ggml_tensor), ggml-impl.h:333-351 (ggml_cgraph),
// ggml-backend.h:53-57, 138-181, ggml-backend-impl.h (vtables)); static_asserts pin the sizes a mismatch would change.
// The only function the plugin needs from libggml-base is ggml_backend_buffer_init (the host owns buffer structs).
#pragma once
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MAX_DIMS 4
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_SRC 10
#define GGML_MAX_NAME 64
#define GGML_BACKEND_API_VERSION 2

enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q4_1 = 3,
    GGML_TYPE_Q5_0 = 6,
    GGML_TYPE_Q5_1 = 7,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_Q2_K = 10,
    GGML_TYPE_Q3_K = 11,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_Q8_K = 15,
    GGML_TYPE_I8 = 24,
    GGML_TYPE_I16 = 25,
    GGML_TYPE_I32 = 26,
    GGML_TYPE_I64 = 27,
    GGML_TYPE_BF16 = 30,
    GGML_TYPE_I2_S = 36,
    GGML_TYPE_COUNT = 43,
};

// enum ggml_op: the positions this plugin dispatches on (ggml.h:485-593 of the b8471 interface; GGML_OP_COUNT = 97)
enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_DUP = 1,
    GGML_OP_ADD = 2,
    GGML_OP_ADD_ID = 3,
    GGML_OP_ADD1 = 4,
    GGML_OP_ACC = 5,
    GGML_OP_SUB = 6,
    GGML_OP_MUL = 7,
    GGML_OP_DIV = 8,
    GGML_OP_SQR = 9,
    GGML_OP_SQRT = 10,
    GGML_OP_LOG = 11,
    GGML_OP_SIN = 12,
    GGML_OP_COS = 13,
    GGML_OP_SUM = 14,
    GGML_OP_SUM_ROWS = 15,
    GGML_OP_CUMSUM = 16,
    GGML_OP_MEAN = 17,
    GGML_OP_ARGMAX = 18,
    GGML_OP_COUNT_EQUAL = 19,
    GGML_OP_REPEAT = 20,
    GGML_OP_REPEAT_BACK = 21,
    GGML_OP_CONCAT = 22,
    GGML_OP_SILU_BACK = 23,
    GGML_OP_NORM = 24,
    GGML_OP_RMS_NORM = 25,
    GGML_OP_RMS_NORM_BACK = 26,
    GGML_OP_GROUP_NORM = 27,
    GGML_OP_L2_NORM = 28,
    GGML_OP_MUL_MAT = 29,
    GGML_OP_MUL_MAT_ID = 30,
    GGML_OP_OUT_PROD = 31,
    GGML_OP_SCALE = 32,
    GGML_OP_SET = 33,
    GGML_OP_CPY = 34,
    GGML_OP_CONT = 35,
    GGML_OP_RESHAPE = 36,
    GGML_OP_VIEW = 37,
    GGML_OP_PERMUTE = 38,
    GGML_OP_TRANSPOSE = 39,
    GGML_OP_GET_ROWS = 40,
    GGML_OP_GET_ROWS_BACK = 41,
    GGML_OP_SET_ROWS = 42,
    GGML_OP_SOFT_MAX = 46,
    GGML_OP_ROPE = 48,
    GGML_OP_FLASH_ATTN_EXT = 74,
    GGML_OP_UNARY = 87,
    GGML_OP_GLU = 96,
    GGML_OP_COUNT = 97,
};

enum ggml_glu_op { GGML_GLU_OP_REGLU = 0, GGML_GLU_OP_GEGLU = 1, GGML_GLU_OP_SWIGLU = 2 };

enum ggml_status { GGML_STATUS_ALLOC_FAILED = -2, GGML_STATUS_FAILED = -1, GGML_STATUS_SUCCESS = 0, GGML_STATUS_ABORTED = 1 };

struct ggml_backend_buffer;

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer* buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor* src[GGML_MAX_SRC];
    struct ggml_tensor* view_src;
    size_t view_offs;
    void* data;
    char name[GGML_MAX_NAME];
    void* extra;
    char padding[8];
};

struct ggml_hash_set {
    size_t size;
    uint32_t* used;
    struct ggml_tensor** keys;
};

struct ggml_cgraph {
    int size;
    int n_nodes;
    int n_leafs;
    struct ggml_tensor** nodes;
    struct ggml_tensor** grads;
    struct ggml_tensor** grad_accs;
    struct ggml_tensor** leafs;
    int32_t* use_counts;
    struct ggml_hash_set visited_hash_set;
    int order;  // enum ggml_cgraph_eval_order
    uint64_t uid;
};

typedef uint8_t ggml_guid[16];
typedef ggml_guid* ggml_guid_t;

typedef struct ggml_backend_buffer_type* ggml_backend_buffer_type_t;
typedef struct ggml_backend_buffer* ggml_backend_buffer_t;
typedef struct ggml_backend_event* ggml_backend_event_t;
typedef struct ggml_backend* ggml_backend_t;
typedef void* ggml_backend_graph_plan_t;
typedef struct ggml_backend_reg* ggml_backend_reg_t;
typedef struct ggml_backend_device* ggml_backend_dev_t;

enum ggml_backend_buffer_usage {
    GGML_BACKEND_BUFFER_USAGE_ANY = 0,
    GGML_BACKEND_BUFFER_USAGE_WEIGHTS = 1,
    GGML_BACKEND_BUFFER_USAGE_COMPUTE = 2,
};

enum ggml_backend_dev_type {
    GGML_BACKEND_DEVICE_TYPE_CPU,
    GGML_BACKEND_DEVICE_TYPE_GPU,
    GGML_BACKEND_DEVICE_TYPE_IGPU,
    GGML_BACKEND_DEVICE_TYPE_ACCEL,
    GGML_BACKEND_DEVICE_TYPE_META,
};

struct ggml_backend_dev_caps {
    bool async;
    bool host_buffer;
    bool buffer_from_host_ptr;
    bool events;
};

struct ggml_backend_dev_props {
    const char* name;
    const char* description;
    size_t memory_free;
    size_t memory_total;
    enum ggml_backend_dev_type type;
    const char* device_id;
    struct ggml_backend_dev_caps caps;
};

struct ggml_backend_buffer_type_i {
    const char* (*get_name)(ggml_backend_buffer_type_t buft);
    ggml_backend_buffer_t (*alloc_buffer)(ggml_backend_buffer_type_t buft, size_t size);
    size_t (*get_alignment)(ggml_backend_buffer_type_t buft);
    size_t (*get_max_size)(ggml_backend_buffer_type_t buft);
    size_t (*get_alloc_size)(ggml_backend_buffer_type_t buft, const struct ggml_tensor* tensor);
    bool (*is_host)(ggml_backend_buffer_type_t buft);
};

struct ggml_backend_buffer_type {
    struct ggml_backend_buffer_type_i iface;
    ggml_backend_dev_t device;
    void* context;
};

struct ggml_backend_buffer_i {
    void (*free_buffer)(ggml_backend_buffer_t buffer);
    void* (*get_base)(ggml_backend_buffer_t buffer);
    enum ggml_status (*init_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor* tensor);
    void (*memset_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor* tensor, uint8_t value, size_t offset,
                          size_t size);
    void (*set_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor* tensor, const void* data, size_t offset,
                       size_t size);
    void (*get_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor* tensor, void* data, size_t offset,
                       size_t size);
    void (*set_tensor_2d)(ggml_backend_buffer_t buffer, struct ggml_tensor* tensor, const void* data, size_t offset,
                          size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    void (*get_tensor_2d)(ggml_backend_buffer_t buffer, const struct ggml_tensor* tensor, void* data, size_t offset,
                          size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    bool (*cpy_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor* src, struct ggml_tensor* dst);
    void (*clear)(ggml_backend_buffer_t buffer, uint8_t value);
    void (*reset)(ggml_backend_buffer_t buffer);
};

struct ggml_backend_buffer {
    struct ggml_backend_buffer_i iface;
    ggml_backend_buffer_type_t buft;
    void* context;
    size_t size;
    enum ggml_backend_buffer_usage usage;
};

struct ggml_backend_i {
    const char* (*get_name)(ggml_backend_t backend);
    void (*free)(ggml_backend_t backend);
    void (*set_tensor_async)(ggml_backend_t backend, struct ggml_tensor* tensor, const void* data, size_t offset,
                             size_t size);
    void (*get_tensor_async)(ggml_backend_t backend, const struct ggml_tensor* tensor, void* data, size_t offset,
                             size_t size);
    void (*set_tensor_2d_async)(ggml_backend_t backend, struct ggml_tensor* tensor, const void* data, size_t offset,
                                size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    void (*get_tensor_2d_async)(ggml_backend_t backend, const struct ggml_tensor* tensor, void* data, size_t offset,
                                size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    bool (*cpy_tensor_async)(ggml_backend_t backend_src, ggml_backend_t backend_dst, const struct ggml_tensor* src,
                             struct ggml_tensor* dst);
    void (*synchronize)(ggml_backend_t backend);
    ggml_backend_graph_plan_t (*graph_plan_create)(ggml_backend_t backend, const struct ggml_cgraph* cgraph);
    void (*graph_plan_free)(ggml_backend_t backend, ggml_backend_graph_plan_t plan);
    void (*graph_plan_update)(ggml_backend_t backend, ggml_backend_graph_plan_t plan, const struct ggml_cgraph* cgraph);
    enum ggml_status (*graph_plan_compute)(ggml_backend_t backend, ggml_backend_graph_plan_t plan);
    enum ggml_status (*graph_compute)(ggml_backend_t backend, struct ggml_cgraph* cgraph);
    void (*event_record)(ggml_backend_t backend, ggml_backend_event_t event);
    void (*event_wait)(ggml_backend_t backend, ggml_backend_event_t event);
    void (*graph_optimize)(ggml_backend_t backend, struct ggml_cgraph* cgraph);
};

struct ggml_backend {
    ggml_guid_t guid;
    struct ggml_backend_i iface;
    ggml_backend_dev_t device;
    void* context;
};

struct ggml_backend_device_i {
    const char* (*get_name)(ggml_backend_dev_t dev);
    const char* (*get_description)(ggml_backend_dev_t dev);
    void (*get_memory)(ggml_backend_dev_t dev, size_t* free, size_t* total);
    enum ggml_backend_dev_type (*get_type)(ggml_backend_dev_t dev);
    void (*get_props)(ggml_backend_dev_t dev, struct ggml_backend_dev_props* props);
    ggml_backend_t (*init_backend)(ggml_backend_dev_t dev, const char* params);
    ggml_backend_buffer_type_t (*get_buffer_type)(ggml_backend_dev_t dev);
    ggml_backend_buffer_type_t (*get_host_buffer_type)(ggml_backend_dev_t dev);
    ggml_backend_buffer_t (*buffer_from_host_ptr)(ggml_backend_dev_t dev, void* ptr, size_t size,
                                                  size_t max_tensor_size);
    bool (*supports_op)(ggml_backend_dev_t dev, const struct ggml_tensor* op);
    bool (*supports_buft)(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft);
    bool (*offload_op)(ggml_backend_dev_t dev, const struct ggml_tensor* op);
    ggml_backend_event_t (*event_new)(ggml_backend_dev_t dev);
    void (*event_free)(ggml_backend_dev_t dev, ggml_backend_event_t event);
    void (*event_synchronize)(ggml_backend_dev_t dev, ggml_backend_event_t event);
};

struct ggml_backend_device {
    struct ggml_backend_device_i iface;
    ggml_backend_reg_t reg;
    void* context;
};

struct ggml_backend_reg_i {
    const char* (*get_name)(ggml_backend_reg_t reg);
    size_t (*get_device_count)(ggml_backend_reg_t reg);
    ggml_backend_dev_t (*get_device)(ggml_backend_reg_t reg, size_t index);
    void* (*get_proc_address)(ggml_backend_reg_t reg, const char* name);
};

struct ggml_backend_reg {
    int api_version;
    struct ggml_backend_reg_i iface;
    void* context;
};

// provided by the host's libggml-base
ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void* context, size_t size);

#ifdef __cplusplus
}
static_assert(sizeof(struct ggml_tensor) == 336, "ggml_tensor layout (GGML_TENSOR_SIZE of ggml 0.9.8)");
static_assert(offsetof(struct ggml_tensor, op_params) == 84, "ggml_tensor.op_params offset");
static_assert(offsetof(struct ggml_tensor, src) == 152, "ggml_tensor.src offset");
static_assert(offsetof(struct ggml_tensor, data) == 248, "ggml_tensor.data offset");
static_assert(sizeof(struct ggml_backend_buffer_i) == 11 * sizeof(void*), "ggml_backend_buffer_i");
static_assert(sizeof(struct ggml_backend_i) == 16 * sizeof(void*), "ggml_backend_i");
static_assert(sizeof(struct ggml_backend_device_i) == 15 * sizeof(void*), "ggml_backend_device_i");
#endif
