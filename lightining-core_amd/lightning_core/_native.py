"""ctypes binding of liblightning_core_hip.so (the C ABI in include/lightning_core_hip.h).

The shared library is built in-tree by lightining-core_amd/build.py.  Loading
fails loudly when it is missing: there is no Python or CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "liblightning_core_hip.so")

c_size = ctypes.c_size_t
c_int = ctypes.c_int
c_float = ctypes.c_float
c_char_p = ctypes.c_char_p
c_void_p = ctypes.c_void_p
FP = ctypes.POINTER(ctypes.c_float)
# Buffer parameters are declared void*: they take the plain addresses the
# binding passes (see _core._fp) as well as ctypes pointers such as FP.
BUF = ctypes.c_void_p

# lcError_t
LC_SUCCESS, LC_NOT_INITIALIZED, LC_INVALID_VALUE, LC_OUT_OF_MEMORY, LC_NOT_SUPPORTED, LC_DRIVER_ERROR, LC_UNKNOWN = range(7)
# lcDeviceKind
LC_DEVICE_CPU, LC_DEVICE_CUDA, LC_DEVICE_METAL, LC_DEVICE_HIP = range(4)
# lcDataType
LC_DTYPE_F32, LC_DTYPE_BF16, LC_DTYPE_F16 = range(3)
# lcMemcpyKind
LC_MEMCPY_HOST_TO_HOST, LC_MEMCPY_HOST_TO_DEVICE, LC_MEMCPY_DEVICE_TO_HOST, LC_MEMCPY_DEVICE_TO_DEVICE = range(4)
# lcStructId
(LC_STRUCT_BACKEND_CAPABILITIES, LC_STRUCT_COMPUTE_INTERFACE_CONTRACT, LC_STRUCT_MEMORY_INTERFACE_CONTRACT,
 LC_STRUCT_SYNC_INTERFACE_CONTRACT, LC_STRUCT_PROFILER_INTERFACE_CONTRACT,
 LC_STRUCT_BACKEND_INTERFACE_CONTRACT) = range(1, 7)


class SyncPolicy(ctypes.Structure):
    _fields_ = [("mode", c_int), ("trace_sync_boundary", c_int)]


class BackendCapabilities(ctypes.Structure):
    _fields_ = [("device", c_int), ("built", c_int), ("available", c_int), ("compute_surface", c_int),
                ("memory_surface", c_int), ("sync_surface", c_int), ("profiling_surface", c_int),
                ("runtime_trace_surface", c_int), ("sync_policy_surface", c_int), ("memory_model", c_int)]


class ComputeInterfaceContract(ctypes.Structure):
    _fields_ = [("available", c_int), ("op_dispatch_trace_surface", c_int), ("driver_tag", c_char_p)]


class MemoryInterfaceContract(ctypes.Structure):
    _fields_ = [("available", c_int), ("allocator_surface", c_int), ("memcpy_surface", c_int),
                ("memory_model", c_int), ("driver_tag", c_char_p)]


class SyncInterfaceContract(ctypes.Structure):
    _fields_ = [("available", c_int), ("sync_policy_surface", c_int), ("trace_sync_boundary_surface", c_int),
                ("driver_tag", c_char_p)]


class ProfilerInterfaceContract(ctypes.Structure):
    _fields_ = [("available", c_int), ("runtime_trace_surface", c_int), ("op_dispatch_trace_surface", c_int),
                ("trace_capacity", c_size), ("driver_tag", c_char_p)]


class BackendInterfaceContract(ctypes.Structure):
    _fields_ = [("device", c_int), ("capabilities", BackendCapabilities), ("compute", ComputeInterfaceContract),
                ("memory", MemoryInterfaceContract), ("sync", SyncInterfaceContract),
                ("profiler", ProfilerInterfaceContract)]


class RuntimeTraceEvent(ctypes.Structure):
    _fields_ = [("type", c_int), ("status", c_int), ("timestamp_ns", ctypes.c_uint64), ("size_bytes", c_size),
                ("detail0", c_int), ("detail1", c_int)]


class AttentionConfig(ctypes.Structure):
    _fields_ = [("seq_len", c_size), ("head_dim", c_size), ("causal", c_int)]


class AttentionIoPolicyC(ctypes.Structure):
    _fields_ = [("upload_q", c_int), ("upload_k", c_int), ("upload_v", c_int), ("upload_target", c_int),
                ("download_out", c_int), ("download_v", c_int), ("synchronize", c_int), ("loss_every", c_int),
                ("output_scale", c_float), ("output_bias", c_float), ("output_relu", c_int)]


class AttentionBatchedConfig(ctypes.Structure):
    _fields_ = [("batch", c_size), ("heads", c_size), ("seq_len", c_size), ("head_dim", c_size), ("causal", c_int),
                ("compute_dtype", c_int)]


class MatMulIoPolicyC(ctypes.Structure):
    _fields_ = [("upload_a", c_int), ("upload_b", c_int), ("download_out", c_int), ("synchronize", c_int)]


class VitBlockConfig(ctypes.Structure):
    _fields_ = [("batch", c_size), ("in_channels", c_size), ("image_h", c_size), ("image_w", c_size),
                ("patch", c_size), ("embed", c_size), ("heads", c_size), ("compute_dtype", c_int)]


class GraphPlannerOptions(ctypes.Structure):
    """lcGraphPlannerOptions."""
    _fields_ = [("preferred_device", c_int), ("sync_mode", c_int), ("trace_sync_boundary", c_int),
                ("group_by_backend_capability", c_int), ("separate_fallback_segments", c_int),
                ("insert_sync_on_device_change", c_int), ("enable_fusion_v1", c_int),
                ("enable_fusion_pass_conv", c_int), ("enable_fusion_pass_matmul", c_int),
                ("enable_fusion_pass_attention", c_int), ("enable_fusion_pass_attention_qkv", c_int),
                ("fusion_pass_order", c_char_p), ("enable_fusion_cost_model_v1", c_int),
                ("enable_fusion_cost_model_v2", c_int), ("enable_plan_cache", c_int),
                ("cost_profile_signature", c_char_p), ("fusion_cost_min_speedup", ctypes.c_double),
                ("cost_launch_overhead_ns", ctypes.c_double), ("cost_transfer_overhead_ns", ctypes.c_double),
                ("cost_sync_boundary_ns", ctypes.c_double), ("cost_elementwise_per_element_ns", ctypes.c_double),
                ("cost_matmul_per_mac_ns", ctypes.c_double), ("cost_conv_per_mac_ns", ctypes.c_double),
                ("planner_cost_weight_compute", ctypes.c_double), ("planner_cost_weight_boundary", ctypes.c_double),
                ("planner_cost_weight_preference", ctypes.c_double)]


class HipDeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("gcn_arch", ctypes.c_char * 64), ("compute_units", c_int),
                ("max_clock_khz", c_int), ("total_memory_bytes", c_size), ("l2_cache_bytes", c_size)]


P = ctypes.POINTER
_E = c_int  # lcError_t

# name -> (restype, argtypes); every symbol declared in include/lightning_core_hip.h
SIGNATURES = {
    # reference C ABI (lightning_core.h:113-137)
    "lcMalloc": (_E, [P(c_void_p), c_size]),
    "lcFree": (_E, [c_void_p]),
    "lcMemcpy": (_E, [c_void_p, c_void_p, c_size, c_int]),
    "lcDeviceSynchronize": (_E, []),
    "lcGetDeviceCount": (_E, [P(c_int)]),
    "lcGetPreferredDeviceForInference": (_E, [P(c_int)]),
    "lcGetPreferredDeviceForTraining": (_E, [P(c_int)]),
    "lcIsCudaAvailable": (c_int, []),
    "lcIsMetalAvailable": (c_int, []),
    "lcGetMemoryModel": (c_int, []),
    "lcGetMemoryModelName": (c_char_p, [c_int]),
    "lcSetDefaultSyncPolicy": (_E, [SyncPolicy]),
    "lcGetDefaultSyncPolicy": (SyncPolicy, []),
    "lcApplySyncPolicy": (_E, [SyncPolicy]),
    "lcApplyDefaultSyncPolicy": (_E, []),
    "lcGetBackendCapabilities": (_E, [c_int, P(BackendCapabilities)]),
    "lcGetActiveBackendCapabilities": (_E, [P(BackendCapabilities)]),
    "lcGetBackendInterfaceContract": (_E, [c_int, P(BackendInterfaceContract)]),
    "lcGetActiveBackendInterfaceContract": (_E, [P(BackendInterfaceContract)]),
    "lcGetApiVersion": (_E, [P(c_int), P(c_int), P(c_int)]),
    "lcGetApiVersionString": (c_char_p, []),
    "lcGetStructSize": (c_size, [c_int]),
    "lcCheckStructSize": (c_int, [c_int, c_size]),
    "lcBackendName": (c_char_p, []),
    "lcGetErrorString": (c_char_p, [c_int]),
    # HIP backend additions
    "lcIsHipAvailable": (c_int, []),
    "lcGetLastErrorMessage": (c_char_p, []),
    "lcSetRuntimeTraceEnabled": (None, [c_int]),
    "lcIsRuntimeTraceEnabled": (c_int, []),
    "lcClearRuntimeTraceEvents": (None, []),
    "lcGetRuntimeTraceEvents": (c_size, [P(RuntimeTraceEvent), c_size]),
    "lcGetRuntimeTraceEventCapacity": (c_size, []),
    "lcRuntimeTraceEventTypeName": (c_char_p, [c_int]),
    "lcRuntimeTraceOpKindName": (c_char_p, [c_int]),
    "lcEncodeRuntimeTraceDispatchDetail": (c_int, [c_int, c_int, c_int]),
    "lcDecodeRuntimeTraceDispatchDetail": (c_int, [c_int, P(c_int), P(c_int), P(c_int)]),
    "lcAttentionIoPolicyDefault": (AttentionIoPolicyC, []),
    "lcAttentionImplementationName": (c_char_p, [c_int]),
    "lcAttentionForward": (_E, [BUF, BUF, BUF, BUF, P(AttentionConfig), c_int]),
    "lcAttentionForwardWithPolicy": (_E, [BUF, BUF, BUF, BUF, P(AttentionConfig), c_int, P(AttentionIoPolicyC)]),
    "lcAttentionForwardBatched": (_E, [BUF, BUF, BUF, BUF, P(AttentionBatchedConfig), c_int, P(AttentionIoPolicyC)]),
    "lcAttentionSessionCreate": (_E, [P(AttentionConfig), c_int, P(c_void_p)]),
    "lcAttentionSessionCreateBatched": (_E, [P(AttentionBatchedConfig), c_int, P(c_void_p)]),
    "lcAttentionSessionDestroy": (_E, [c_void_p]),
    "lcAttentionSessionSetDefaultPolicy": (_E, [c_void_p, P(AttentionIoPolicyC)]),
    "lcAttentionSessionGetDefaultPolicy": (_E, [c_void_p, P(AttentionIoPolicyC)]),
    "lcAttentionSessionForward": (_E, [c_void_p, BUF, BUF, BUF, BUF]),
    "lcAttentionSessionForwardWithPolicy": (_E, [c_void_p, BUF, BUF, BUF, BUF, P(AttentionIoPolicyC)]),
    "lcAttentionSessionRunCached": (_E, [c_void_p, c_size]),
    "lcAttentionSessionTrainRunCached": (_E, [c_void_p, c_float, c_size]),
    "lcAttentionTrainStep": (_E, [BUF, BUF, BUF, BUF, BUF, c_float, P(AttentionConfig), c_int, BUF]),
    "lcAttentionTrainStepWithPolicy": (_E, [BUF, BUF, BUF, BUF, BUF, c_float, P(AttentionConfig), c_int, BUF,
                                            P(AttentionIoPolicyC)]),
    "lcAttentionSessionTrainStep": (_E, [c_void_p, BUF, BUF, BUF, BUF, BUF, c_float, BUF]),
    "lcAttentionSessionTrainStepWithPolicy": (_E, [c_void_p, BUF, BUF, BUF, BUF, BUF, c_float, BUF, P(AttentionIoPolicyC)]),
    "lcMatMulIoPolicyDefault": (MatMulIoPolicyC, []),
    "lcMatMul": (_E, [BUF, BUF, BUF, c_size, c_size, c_size, c_int]),
    "lcMatMulWithPolicy": (_E, [BUF, BUF, BUF, c_size, c_size, c_size, c_int, P(MatMulIoPolicyC)]),
    "lcMatMulWithPolicyBatched": (_E, [BUF, BUF, BUF, c_size, c_size, c_size, c_int, P(MatMulIoPolicyC), c_size]),
    "lcMatMulResetTuning": (_E, []),
    "lcMatMulDeviceNoAlloc": (_E, [c_void_p, c_void_p, c_void_p, c_size, c_size, c_size]),
    "lcMatMulResidentSessionCreate": (_E, [c_size, c_size, c_size, c_int, P(c_void_p)]),
    "lcMatMulResidentSessionDestroy": (_E, [c_void_p]),
    "lcMatMulResidentSessionStart": (_E, [c_void_p, BUF, BUF, BUF]),
    "lcMatMulResidentSessionRun": (_E, [c_void_p, BUF, BUF, BUF]),
    "lcMatMulResidentSessionFinish": (_E, [c_void_p, BUF, BUF, BUF]),
    "lcMatMulResidentSessionSync": (_E, [c_void_p, BUF, BUF, BUF]),
    "lcMatMulResidentSessionRunBatchSync": (_E, [c_void_p, BUF, BUF, BUF, c_size]),
    "lcMatMulResidentSessionRunBatchSyncNoDownload": (_E, [c_void_p, BUF, BUF, BUF, c_size]),
    "lcMatMulResidentSessionRunBatchSyncCachedNoDownload": (_E, [c_void_p, c_size]),
    "lcMatMulResidentSessionTimeLaunches": (_E, [c_void_p, c_size, c_void_p]),
    "lcMatMulResidentSessionKernelName": (_E, [c_void_p, ctypes.c_char_p, c_size]),
    "lcConv2dNchw": (_E, [BUF, BUF, BUF, BUF] + [c_size] * 11 + [c_int, c_int]),
    "lcConvAttentionTorchstrongNchw": (_E, [BUF, BUF, BUF, BUF] + [c_size] * 13 + [c_int]),
    "lcConvAttentionTorchstrongNchwGraph": (_E, [BUF, BUF, BUF, BUF] + [c_size] * 13 + [c_int]),
    "lcConvAttentionGraphCacheClear": (_E, []),
    "lcConvAttentionGraphCacheSize": (c_size, []),
    "lcVitBlockSessionCreate": (_E, [P(VitBlockConfig), c_int, P(c_void_p)]),
    "lcVitBlockSessionDestroy": (_E, [c_void_p]),
    "lcVitBlockSessionSetWeights": (_E, [c_void_p, BUF, BUF, BUF]),
    "lcVitBlockSessionForward": (_E, [c_void_p, BUF, BUF]),
    "lcVitBlockSessionRunCached": (_E, [c_void_p, c_size]),
    "lcVitBlockForward": (_E, [BUF, BUF, BUF, BUF, BUF, P(VitBlockConfig), c_int]),
    "lcHipGetDeviceInfo": (_E, [P(HipDeviceInfo)]),
    "lcHipTimerCreate": (_E, [P(c_void_p)]),
    "lcHipTimerDestroy": (_E, [c_void_p]),
    "lcHipTimerStart": (_E, [c_void_p]),
    "lcHipTimerStop": (_E, [c_void_p, P(c_float)]),
    "lcHipTuneCacheSave": (_E, [c_char_p]),
    "lcHipTuneCacheLoad": (_E, [c_char_p]),
    "lcHipTuneCacheSize": (c_size, []),
    "lcHipAttentionTuneCacheSave": (_E, [c_char_p]),
    "lcHipAttentionTuneCacheLoad": (_E, [c_char_p]),
    "lcHipAttentionResetTuning": (_E, []),
    "lcHipAttentionTuneCacheSize": (c_size, []),
    "lcPreloadRuntimeProfileEnv": (None, []),
    # graph IR on hip
    "lcGraphPlannerOptionsDefault": (GraphPlannerOptions, []),
    "lcGraphCreate": (_E, [P(c_void_p)]),
    "lcGraphDestroy": (_E, [c_void_p]),
    "lcGraphAddTensor": (_E, [c_void_p, P(ctypes.c_int64), c_size, c_int, c_int, c_char_p, c_int, P(c_size)]),
    "lcGraphAddNode": (_E, [c_void_p, c_char_p, P(c_size), c_size, P(c_size), c_size, P(c_size), c_size, c_char_p,
                            P(c_char_p), P(ctypes.c_int64), c_size]),
    "lcGraphCounts": (_E, [c_void_p, P(c_size), P(c_size)]),
    "lcGraphPlanCacheStats": (_E, [c_void_p, P(c_size), P(c_size)]),
    "lcGraphClearPlanCache": (_E, [c_void_p]),
    "lcGraphReport": (_E, [c_void_p, ctypes.c_char_p, c_size, P(c_size)]),
    "lcGraphDescribe": (_E, [c_void_p]),
    "lcGraphRegistry": (_E, [ctypes.c_char_p, c_size, P(c_size)]),
    "lcGraphValidate": (_E, [c_void_p]),
    "lcGraphPlanForDevice": (_E, [c_void_p, c_int]),
    "lcGraphPlanGroups": (_E, [c_void_p, P(GraphPlannerOptions)]),
    "lcGraphPlanSummary": (_E, [c_void_p, P(GraphPlannerOptions)]),
    "lcGraphFusionReport": (_E, [c_void_p, P(GraphPlannerOptions)]),
    "lcGraphExecuteF32": (_E, [c_void_p, P(GraphPlannerOptions), P(c_size), P(c_void_p), P(c_size), c_size,
                               P(c_size), P(c_void_p), c_size]),
}

_lib = None


def load():
    """Loads the library once; raises ImportError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python lightining-core_amd/build.py` "
                          "(there is no fallback implementation)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
