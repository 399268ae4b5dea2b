"""ctypes binding of libnve_amd.so (include/nve_c_api.h + include/nve_amd_ext.h)."""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# NVE_AMD_LIB: another build of the library (e.g. the Makefile's `asan` target)
LIB_PATH = os.environ.get("NVE_AMD_LIB") or os.path.join(os.path.dirname(_HERE), "libnve_amd.so")

# nve_status_t
SUCCESS, INVALID_ARGUMENT, HIP_ERROR, RUNTIME, NOT_IMPLEMENTED, OUT_OF_MEMORY = range(6)
# nve_data_type_t
(DT_UNKNOWN, DT_F32, DT_BF16, DT_F16, DT_E4M3, DT_E5M2, DT_F64, DT_QI8_F32, DT_QI8_F16,
 DT_QU8_F32, DT_QU8_F16) = range(11)
DT_XI8A_F32, DT_XE4M3_F32 = 32, 33
# enums
SPARSE_FIXED, SPARSE_CSR = 0, 1
POOL_CONCAT, POOL_SUM, POOL_MEAN, POOL_WSUM, POOL_WMEAN = range(5)
KEY_INT32, KEY_INT64 = 0, 1


class NVEError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"[nve status {status}] {msg}")
        self.status = status


class InvalidArgument(NVEError, ValueError):
    pass


class NotImplementedInBuild(NVEError, NotImplementedError):
    pass


P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
U64 = ctypes.c_uint64
PI64 = ctypes.POINTER(ctypes.c_int64)
PI32 = ctypes.POINTER(ctypes.c_int32)
PP = ctypes.POINTER(ctypes.c_void_p)


class GpuTableConfig(ctypes.Structure):
    _fields_ = [("device_id", I32), ("cache_size", U64), ("row_size_in_bytes", I64),
                ("uvm_table", P), ("count_misses", ctypes.c_int), ("max_modify_size", I64),
                ("value_dtype", I32), ("private_stream", P), ("disable_uvm_update", ctypes.c_int),
                ("uvm_cpu_accumulate", ctypes.c_int), ("data_storage_on_host", ctypes.c_int),
                ("modify_on_gpu", ctypes.c_int), ("kernel_mode_type", U64),
                ("kernel_mode_value", U64), ("invalid_key", I64), ("uvm_num_rows", I64)]


class GpuLayerConfig(ctypes.Structure):
    _fields_ = [("layer_name", ctypes.c_char_p), ("device_id", I32), ("embedding_table", P),
                ("num_embeddings", I64), ("embedding_width_in_bytes", I64), ("value_dtype", I32),
                ("default_row_index", I64)]


class UvmLayerConfig(ctypes.Structure):
    _fields_ = [("layer_name", ctypes.c_char_p), ("insert_heuristic", P),
                ("min_insert_freq_gpu", I64), ("min_insert_size_gpu", I64),
                ("default_row_index", I64)]


class HierLayerConfig(ctypes.Structure):
    _fields_ = [("layer_name", ctypes.c_char_p), ("insert_heuristic", P),
                ("min_insert_freq_gpu", I64), ("min_insert_freq_host", I64),
                ("min_insert_size_gpu", I64), ("min_insert_size_host", I64),
                ("default_embedding", P), ("default_embedding_size", I64)]


class HostLayerConfig(ctypes.Structure):
    _fields_ = [("layer_name", ctypes.c_char_p), ("default_embedding", P),
                ("default_embedding_size", I64)]


class OverflowPolicyConfig(ctypes.Structure):
    _fields_ = [("overflow_margin", I64), ("handler", ctypes.c_int),
                ("resolution_margin", ctypes.c_double)]


class HostTableConfig(ctypes.Structure):
    _fields_ = [("key_size", I64), ("max_value_size", I64), ("value_dtype", I32),
                ("invalid_key", I64)]


# name -> (restype, argtypes); status-returning calls use I32
SIGNATURES = {
    "nve_get_last_error": (I32, [ctypes.POINTER(ctypes.c_char_p)]),
    "nve_gpu_table_config_default": (GpuTableConfig, []),
    "nve_gpu_embedding_layer_config_default": (GpuLayerConfig, []),
    "nve_linear_uvm_layer_config_default": (UvmLayerConfig, []),
    "nve_hierarchical_layer_config_default": (HierLayerConfig, []),
    "nve_host_embedding_layer_config_default": (HostLayerConfig, []),
    "nve_overflow_policy_config_default": (OverflowPolicyConfig, []),
    "nve_host_table_config_default": (HostTableConfig, []),
    "nve_version": (I32, [PI32, PI32, PI32]),
    "nve_abi_version": (I32, [PI32, PI32]),
    "nve_thread_pool_create": (I32, [PP, ctypes.c_char_p]),
    "nve_thread_pool_destroy": (I32, [P]),
    "nve_thread_pool_num_workers": (I32, [P, PI64]),
    "nve_configure_default_thread_pool": (I32, [ctypes.c_char_p]),
    "nve_heuristic_create_default": (I32, [PP, ctypes.POINTER(ctypes.c_float), I64]),
    "nve_heuristic_create_never": (I32, [PP]),
    "nve_heuristic_destroy": (I32, [P]),
    "nve_context_destroy": (I32, [P]),
    "nve_context_wait": (I32, [P]),
    "nve_context_get_lookup_stream": (I32, [P, PP]),
    "nve_context_get_modify_stream": (I32, [P, PP]),
    "nve_gpu_table_create": (I32, [PP, ctypes.c_int, ctypes.POINTER(GpuTableConfig), P]),
    "nve_table_destroy": (I32, [P]),
    "nve_table_find": (I32, [P, P, I64, P, P, I64, P, P]),
    "nve_table_insert": (I32, [P, P, I64, P, I64, I64, P]),
    "nve_table_update": (I32, [P, P, I64, P, I64, I64, P]),
    "nve_table_update_accumulate": (I32, [P, P, I64, P, I64, I64, P, I32]),
    "nve_table_clear": (I32, [P, P]),
    "nve_table_erase": (I32, [P, P, I64, P]),
    "nve_table_create_execution_context": (I32, [P, PP, P, P, P, P]),
    "nve_table_get_device_id": (I32, [P, PI32]),
    "nve_table_get_max_row_size": (I32, [P, PI64]),
    "nve_table_get_key_size": (I32, [P, PI64]),
    "nve_table_reset_lookup_counter": (I32, [P, P]),
    "nve_table_get_lookup_counter": (I32, [P, P, PI64]),
    "nve_create_table_factory": (I32, [PP, ctypes.c_char_p, ctypes.c_char_p]),
    "nve_table_factory_destroy": (I32, [P]),
    "nve_table_factory_produce": (I32, [P, I64, ctypes.c_char_p, PP]),
    "nve_gpu_embedding_layer_create": (I32, [PP, ctypes.c_int, ctypes.POINTER(GpuLayerConfig), P]),
    "nve_linear_uvm_layer_create": (I32, [PP, ctypes.c_int, ctypes.POINTER(UvmLayerConfig), P, P]),
    "nve_hierarchical_layer_create": (I32, [PP, ctypes.c_int, ctypes.POINTER(HierLayerConfig), P, I64, P]),
    "nve_host_embedding_layer_create": (I32, [PP, ctypes.c_int, ctypes.POINTER(HostLayerConfig), P, P]),
    "nve_layer_destroy": (I32, [P]),
    "nve_layer_lookup": (I32, [P, P, I64, P, P, I64, P, P]),
    "nve_layer_lookup_pooled": (I32, [P, P, I64, P, P, I64, P, ctypes.c_int, ctypes.c_int, P, I64,
                                      I64, P, I32, I32, P]),
    "nve_layer_insert": (I32, [P, P, I64, P, I64, I64, P, I64]),
    "nve_layer_update": (I32, [P, P, I64, P, I64, I64, P, I64]),
    "nve_layer_accumulate": (I32, [P, P, I64, P, I64, I64, P, I32, I64]),
    "nve_layer_clear": (I32, [P, P]),
    "nve_layer_erase": (I32, [P, P, I64, P, I64]),
    "nve_layer_create_execution_context": (I32, [P, PP, P, P, P, P]),
    "nve_layer_get_num_tables": (I32, [P, PI64]),
    # extensions
    "nve_amd_find_and_pool": (I32, [ctypes.c_int, I64, P, P, I64, I64, I32, ctypes.c_int,
                                    ctypes.c_int, P, I64, I64, P, I32, I32, P, I64, I32, I32, P]),
    "nve_amd_read_ceiling": (I32, [P, I64, P, I64, P, P]),
    "nve_amd_set_log_level": (I32, [I32]),
    "nve_amd_get_log_level": (I32, [P]),
    "nve_amd_log_message": (I32, [I32, ctypes.c_char_p]),
    "nve_amd_find_and_pool_multi": (I32, [ctypes.c_int, I64, ctypes.POINTER(P), P, I64, I32, I64, I64, P, P,
                                          P, I32, ctypes.c_int, I32, P, P]),
    "nve_amd_dedup_workspace_size": (I32, [I64, ctypes.POINTER(U64)]),
    "nve_amd_dedup": (I32, [ctypes.c_int, I64, P, P, P, P, P, PI64, P, U64, P]),
    "nve_amd_dedup_gather": (I32, [ctypes.c_int, I64, P, P, I64, I64, P, I64, P, U64, P]),
    "nve_amd_dedup_gather_noalloc": (I32, [ctypes.c_int, I64, P, P, I64, I64, P, I64, P]),
    "nve_amd_gpu_table_num_sets": (I32, [P, PI64]),
    "nve_amd_gpu_table_export_state": (I32, [P, P, P, P, PI64]),
    "nve_amd_gpu_table_import_state": (I32, [P, P, P, P, I64]),
    "nve_amd_gpu_table_data": (I32, [P, PP]),
    "nve_amd_table_insert_from_uvm": (I32, [P, P, I64, P]),
    "nve_amd_linear_host_table_create": (I32, [PP, ctypes.c_int, ctypes.POINTER(HostTableConfig), P, I64, I64]),
    "nve_amd_backprop_workspace_size": (I32, [I64, I64, I64, ctypes.POINTER(U64)]),
    "nve_amd_pooling_backprop": (I32, [ctypes.c_int, I64, P, ctypes.c_int, ctypes.c_int, P, I64, I64, P, I32,
                                       P, I32, I64, P, P, PI64, P, U64, P]),
}

_lib = None


def load():
    """Load libnve_amd.so (built by __graft_entry__.build / the package Makefile)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                              "(make -C nv-embedding-cache_amd)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error():
    msg = ctypes.c_char_p()
    load().nve_get_last_error(ctypes.byref(msg))
    return (msg.value or b"").decode()


def check(status):
    """Raise the Python exception matching a non-zero nve_status_t."""
    if status == SUCCESS:
        return
    msg = last_error()
    if status == INVALID_ARGUMENT:
        raise InvalidArgument(status, msg)
    if status == NOT_IMPLEMENTED:
        raise NotImplementedInBuild(status, msg)
    raise NVEError(status, msg)


def call(name, *args):
    check(getattr(load(), name)(*args))
