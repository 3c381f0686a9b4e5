/* Test double of the ggml host (libggml-base) for the plugin tests: the one function a backend plugin calls into its
 * host, ggml_backend_buffer_init, plus the host-side buffer calls a test needs (set usage, free). Loaded with
 * RTLD_GLOBAL before libggml-ameva.so so that the plugin's undefined ggml_backend_buffer_init binds here, as it binds
 * to libggml-base under llama.cpp. Test infrastructure only. */
#include <stdlib.h>

#include "../../ameva_compute_amd/csrc/ggml_abi.h"

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
