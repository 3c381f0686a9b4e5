"""ctypes binding of libac_runtime_hip.so (include/ac_runtime_hip.h) for the tests: the descriptor structs, the
result codes and the signatures of the 53 exported functions (the reference's include/ac_runtime.h)."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(ROOT, "ameva_compute_amd", "libac_runtime_hip.so")
KERNELS = os.path.join(HERE, "ac_kernels", "ac_test_kernels.hsaco")

ABI = 0x00020300
BACKEND_VULKAN, BACKEND_OPENCL, BACKEND_HIP = 1, 2, 3
USAGE_STORAGE, USAGE_SRC, USAGE_DST, USAGE_UNIFORM = 1, 2, 4, 8
STAGE_COMPUTE = 1 << 5
SPEC_U32, SPEC_I32, SPEC_F32 = 0, 1, 2
FLAG_EXPLICIT, FLAG_TIMESTAMPS, FLAG_DISPATCH_TIMESTAMPS = 1, 2, 4

SUCCESS = 0
E = dict(INVALID_CONTEXT=-101, DRIVER_NOT_FOUND=-102, DEVICE_NOT_SUPPORTED=-104, INVALID_ARGUMENT=-106,
         CONTEXT_MISMATCH=-107, FEATURE_NOT_SUPPORTED=-108, OUT_OF_DEVICE_MEMORY=-202,
         BUFFER_ALIGNMENT_INVALID=-203, BUFFER_NOT_MAPPED=-204, NULL_POINTER=-205, INVALID_BUFFER_SIZE=-206,
         KERNEL_NOT_FOUND=-302, KERNEL_ARG_INVALID=-303, BINARY_CORRUPTED=-304, INVALID_WORK_GROUP_SIZE=-401,
         LAUNCH_TIMEOUT=-405, DEVICE_BUSY=-406, RESOURCE_IN_USE=-407)


class Dim3(ctypes.Structure):
    _fields_ = [("x", ctypes.c_uint32), ("y", ctypes.c_uint32), ("z", ctypes.c_uint32)]


class SpecConstant(ctypes.Structure):
    _fields_ = [("constant_id", ctypes.c_uint32), ("type", ctypes.c_uint32), ("value_bits", ctypes.c_uint32)]


class SpecSchema(ctypes.Structure):
    _fields_ = [("constant_id", ctypes.c_uint32), ("type", ctypes.c_uint32), ("default_value_bits", ctypes.c_uint32),
                ("min_value_bits", ctypes.c_uint32), ("max_value_bits", ctypes.c_uint32),
                ("overrides_local_size_axis", ctypes.c_uint32)]


class BindingDesc(ctypes.Structure):
    _fields_ = [("binding_index", ctypes.c_uint32), ("binding_type", ctypes.c_uint32),
                ("stage_flags", ctypes.c_uint32)]


class Metadata(ctypes.Structure):
    _fields_ = [("kernel_name", ctypes.c_char_p), ("entry_point", ctypes.c_char_p),
                ("binding_count", ctypes.c_uint32), ("bindings", ctypes.POINTER(BindingDesc)),
                ("push_constant_size", ctypes.c_size_t), ("local_size", Dim3),
                ("required_features", ctypes.c_uint32), ("expected_spirv_sha256", ctypes.c_char_p),
                ("specialization_schema_count", ctypes.c_uint32),
                ("specialization_schemas", ctypes.POINTER(SpecSchema))]


class ContextDesc(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32),
                ("backend_kind", ctypes.c_uint32), ("flags", ctypes.c_uint32)]


class BufferDesc(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32), ("size_bytes", ctypes.c_size_t),
                ("usage", ctypes.c_uint32), ("force_non_coherent", ctypes.c_uint32)]


class KernelDesc(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32),
                ("spirv_code", ctypes.c_void_p), ("code_size_bytes", ctypes.c_size_t),
                ("metadata", ctypes.POINTER(Metadata)), ("specialization_count", ctypes.c_uint32),
                ("specializations", ctypes.POINTER(SpecConstant))]


class LaunchDesc(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32), ("kernel", ctypes.c_void_p),
                ("buffers", ctypes.POINTER(ctypes.c_void_p)), ("buffer_count", ctypes.c_uint32),
                ("push_constants", ctypes.c_void_p), ("push_constants_size", ctypes.c_size_t), ("grid_dim", Dim3)]


class BatchDesc(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32),
                ("max_dispatches", ctypes.c_uint32), ("flags", ctypes.c_uint32)]


class BufferBinding(ctypes.Structure):
    _fields_ = [("buffer", ctypes.c_void_p), ("offset", ctypes.c_uint64), ("range", ctypes.c_uint64)]


class BatchStats(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32), ("dispatches", ctypes.c_uint32),
                ("barriers", ctypes.c_uint32), ("elided_barriers", ctypes.c_uint32), ("flushes", ctypes.c_uint32),
                ("descriptor_cache_hits", ctypes.c_uint64), ("descriptor_cache_misses", ctypes.c_uint64)]


class DeviceLimits(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32),
                ("max_storage_buffer_range", ctypes.c_uint64), ("min_storage_buffer_offset_alignment", ctypes.c_uint64),
                ("max_memory_allocation_size", ctypes.c_uint64), ("max_compute_workgroup_count", ctypes.c_uint32 * 3),
                ("max_compute_workgroup_size", ctypes.c_uint32 * 3),
                ("max_compute_workgroup_invocations", ctypes.c_uint32),
                ("max_compute_shared_memory_size", ctypes.c_uint32), ("max_push_constants_size", ctypes.c_uint32),
                ("subgroup_size", ctypes.c_uint32), ("timestamps_supported", ctypes.c_uint32),
                ("timestamp_period_ns", ctypes.c_float), ("integer_dot_product", ctypes.c_uint32),
                ("integer_dot_product_accelerated", ctypes.c_uint32)]


class KernelSourceDesc(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32), ("source", ctypes.c_char_p),
                ("source_size", ctypes.c_size_t), ("build_options", ctypes.c_char_p),
                ("metadata", ctypes.POINTER(Metadata)), ("flags", ctypes.c_uint32)]


class ErrorState(ctypes.Structure):
    _fields_ = [("generation", ctypes.c_uint64), ("first_error", ctypes.c_int32), ("operation", ctypes.c_int),
                ("offset", ctypes.c_size_t), ("requested_bytes", ctypes.c_size_t),
                ("capacity_bytes", ctypes.c_size_t)]


def desc(cls, **kw):
    d = cls(abi_version=ABI, struct_size=ctypes.sizeof(cls))
    for k, v in kw.items():
        setattr(d, k, v)
    return d


P = ctypes.c_void_p
PP = ctypes.POINTER(ctypes.c_void_p)
R = ctypes.c_int
_SIG = {
    "ac_runtime_abi_version": (ctypes.c_uint32, []),
    "ac_runtime_context_create": (R, [ctypes.POINTER(ContextDesc), PP]),
    "ac_runtime_context_destroy": (R, [P]),
    "ac_runtime_context_get_device_name": (R, [P, ctypes.c_char_p, ctypes.c_size_t]),
    "ac_runtime_context_get_backend_kind": (R, [P, ctypes.POINTER(ctypes.c_uint32)]),
    "ac_runtime_context_get_limits": (R, [P, ctypes.POINTER(DeviceLimits)]),
    "ac_runtime_buffer_create": (R, [P, ctypes.POINTER(BufferDesc), PP]),
    "ac_runtime_buffer_destroy": (R, [P]),
    "ac_runtime_buffer_get_mapped_ptr": (R, [P, PP]),
    "ac_runtime_buffer_get_size": (R, [P, ctypes.POINTER(ctypes.c_size_t)]),
    "ac_runtime_buffer_get_allocation_size": (R, [P, ctypes.POINTER(ctypes.c_size_t)]),
    "ac_runtime_buffer_is_coherent": (R, [P, ctypes.POINTER(ctypes.c_uint32)]),
    "ac_runtime_buffer_flush": (R, [P, ctypes.c_size_t, ctypes.c_size_t]),
    "ac_runtime_buffer_invalidate": (R, [P, ctypes.c_size_t, ctypes.c_size_t]),
    "ac_runtime_buffer_write": (R, [P, ctypes.c_size_t, P, ctypes.c_size_t]),
    "ac_runtime_buffer_read": (R, [P, ctypes.c_size_t, P, ctypes.c_size_t]),
    "ac_runtime_buffer_fill": (R, [P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_uint8]),
    "ac_runtime_buffer_get_address": (R, [P, PP]),
    "ac_runtime_kernel_create": (R, [P, ctypes.POINTER(KernelDesc), PP]),
    "ac_runtime_kernel_create_from_source": (R, [P, ctypes.POINTER(KernelSourceDesc), PP]),
    "ac_runtime_kernel_destroy": (R, [P]),
    "ac_runtime_kernel_get_pipeline_identity": (R, [P, ctypes.c_char_p, ctypes.c_size_t]),
    "ac_runtime_kernel_get_effective_local_size": (R, [P, ctypes.POINTER(Dim3)]),
    "ac_runtime_kernel_get_push_constant_size": (R, [P, ctypes.POINTER(ctypes.c_size_t)]),
    "ac_runtime_dispatch": (R, [P, ctypes.POINTER(LaunchDesc), PP]),
    "ac_runtime_event_wait": (R, [P, ctypes.c_uint64]),
    "ac_runtime_event_get_timing": (R, [P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "ac_runtime_event_destroy": (R, [P]),
    "ac_runtime_batch_begin": (R, [P, PP]),
    "ac_runtime_batch_begin_ex": (R, [P, ctypes.POINTER(BatchDesc), PP]),
    "ac_runtime_batch_dispatch": (R, [P, P, ctypes.POINTER(LaunchDesc), PP]),
    "ac_runtime_batch_dispatch_bindings": (R, [P, P, ctypes.POINTER(BufferBinding), ctypes.c_uint32, P,
                                               ctypes.c_size_t, Dim3]),
    "ac_runtime_batch_barrier": (R, [P]),
    "ac_runtime_batch_flush": (R, [P]),
    "ac_runtime_batch_submit": (R, [P, PP]),
    "ac_runtime_batch_abort": (R, [P]),
    "ac_runtime_batch_destroy": (None, [P]),
    "ac_runtime_batch_get_dispatch_times": (R, [P, ctypes.POINTER(ctypes.c_uint64), ctypes.c_uint32,
                                                ctypes.POINTER(ctypes.c_uint32)]),
    "ac_runtime_batch_get_stats": (R, [P, ctypes.POINTER(BatchStats)]),
    "ac_runtime_pipeline_cache_merge": (R, [P, P, ctypes.c_size_t]),
    "ac_runtime_pipeline_cache_get_data": (R, [P, P, ctypes.POINTER(ctypes.c_size_t)]),
    "ac_runtime_set_error": (None, [ctypes.c_int32, ctypes.c_int, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t]),
    "ac_runtime_get_error_state": (ErrorState, []),
    "ac_runtime_consume_error": (ctypes.c_int32, []),
    "ac_runtime_advance_generation": (ctypes.c_uint64, []),
    "ac_runtime_get_generation": (ctypes.c_uint64, []),
    "ac_runtime_reset_error_state": (None, []),
    "ac_runtime_set_error_ctx": (None, [ctypes.c_uint64, ctypes.c_int32, ctypes.c_int, ctypes.c_size_t,
                                        ctypes.c_size_t, ctypes.c_size_t]),
    "ac_runtime_get_error_state_ctx": (ErrorState, [ctypes.c_uint64]),
    "ac_runtime_consume_error_ctx": (ctypes.c_int32, [ctypes.c_uint64]),
    "ac_runtime_advance_generation_ctx": (ctypes.c_uint64, [ctypes.c_uint64]),
    "ac_runtime_get_generation_ctx": (ctypes.c_uint64, [ctypes.c_uint64]),
    "ac_runtime_reset_error_state_ctx": (None, [ctypes.c_uint64]),
}


def load():
    lib = ctypes.CDLL(LIB)
    for name, (res, args) in _SIG.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def names():
    return sorted(_SIG)
