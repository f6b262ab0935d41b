"""ctypes binding of the C ABI in include/sandyrt_hip.h.

The library is the in-tree build sandyrt_amd/libsandyrt_hip.so.  There is no
fallback: if it is missing or fails to load, every op raises BackendMissing.
"""
from __future__ import annotations

import ctypes as C
import os

import torch

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libsandyrt_hip.so")

MAX_RANK = 8

F32, F16, BF16, I32, I64, U8 = 0, 1, 2, 3, 4, 5

_TORCH_TO_CODE = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.int32: I32,
    torch.int64: I64,
    torch.uint8: U8,
}


class BackendMissing(RuntimeError):
    pass


class SandyError(RuntimeError):
    """A call into the backend failed; the message follows the reference's wording."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class SandyTensor(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("dtype", C.c_int32),
        ("rank", C.c_int32),
        ("dims", C.c_int64 * MAX_RANK),
        ("strides", C.c_int64 * MAX_RANK),
        ("storage_offset", C.c_int64),
    ]


class SandyPagedCache(C.Structure):
    _fields_ = [
        ("pool", C.c_void_p),
        ("dtype", C.c_int32),
        ("reserved", C.c_int32),
        ("page_size", C.c_int64),
        ("prefix", C.c_int64),
        ("inner", C.c_int64),
        ("num_pages", C.c_int64),
        ("page_stride", C.c_int64),
    ]


class SandyPagedTensor(C.Structure):
    _fields_ = [
        ("pages", C.c_void_p),
        ("dtype", C.c_int32),
        ("rank", C.c_int32),
        ("dims", C.c_int64 * MAX_RANK),
        ("grow_dim", C.c_int64),
        ("page_size", C.c_int64),
        ("page_count", C.c_int64),
    ]


class SandyPagedView(C.Structure):
    _fields_ = [
        ("pages", C.c_void_p),
        ("dtype", C.c_int32),
        ("rank", C.c_int32),
        ("dims", C.c_int64 * 4),
        ("page_size", C.c_int64),
        ("page_count", C.c_int64),
    ]


class SandyRowStats(C.Structure):
    _fields_ = [
        ("sumsq", C.c_void_p),
        ("rows", C.c_int64),
        ("parts", C.c_int64),
    ]


class SandyScalarNode(C.Structure):
    _fields_ = [
        ("id", C.c_uint32),
        ("op", C.c_int32),
        ("dtype", C.c_int32),
        ("input_index", C.c_uint32),
        ("constant", C.c_double),
        ("operand_count", C.c_int32),
        ("operands", C.c_uint32 * 2),
    ]


class SandyPagedPoolDesc(C.Structure):
    _fields_ = [
        ("dtype", C.c_int32),
        ("rank", C.c_int32),
        ("dims", C.c_int64 * MAX_RANK),
        ("grow_dim", C.c_int64),
        ("page_size", C.c_int64),
        ("initial_pages", C.c_int64),
        ("max_pages", C.c_int64),
        ("max_tensors", C.c_int64),
        ("max_blocks", C.c_int64),
    ]


class SandySafetensorInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256),
        ("dtype", C.c_int32),
        ("rank", C.c_int32),
        ("dims", C.c_int64 * MAX_RANK),
        ("file_offset", C.c_uint64),
        ("nbytes", C.c_uint64),
        ("arena_offset", C.c_uint64),
    ]


class SandyPagedMeta(C.Structure):
    _fields_ = [
        ("pool", C.c_uint32),
        ("dtype", C.c_int32),
        ("rank", C.c_int32),
        ("slot", C.c_int32),
        ("dims", C.c_int64 * MAX_RANK),
        ("grow_dim", C.c_int64),
        ("page_size", C.c_int64),
        ("grow_length", C.c_int64),
        ("page_count", C.c_int64),
        ("page_element_count", C.c_int64),
    ]


T = C.POINTER(SandyTensor)
P = C.POINTER(SandyPagedCache)
PV = C.POINTER(SandyPagedView)
RS = C.POINTER(SandyRowStats)
ERR = C.c_char_p

# name -> argtypes (every function returns int; the last three args are
# stream, err buffer, err capacity unless noted)
SIGNATURES = {
    "sandy_hip_take_device_errors": [C.c_void_p, C.POINTER(C.c_uint32), ERR, C.c_size_t],
    "sandy_hip_elementwise": [C.POINTER(SandyScalarNode), C.c_int32, C.c_uint32, T, C.POINTER(C.c_int32),
                              C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_norm": [C.c_int32, T, T, T, C.c_double, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_add_rms_norm": [T, T, T, C.c_double, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_rope": [T, T, C.c_double, C.c_int64, C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_rope_pair": [T, T, T, C.c_double, C.c_int64, C.c_int32, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_softmax": [T, C.c_int64, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_decode_linear": [T, T, T, C.c_double, T, T, C.c_int32, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_paged_to_dense": [C.POINTER(SandyPagedTensor), T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_paged_stage": [C.POINTER(SandyPagedTensor), C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_reduce_sum": [T, C.c_int64, C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_gather": [T, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_attention": [T, T, T, T, C.c_int64, C.c_double, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_paged_attention": [T, P, P, T, T, C.c_int64, C.c_double, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_rope_cache": [T, C.c_int64, C.c_double, C.c_int64, C.c_int64, C.c_int32, T, C.c_void_p, ERR,
                             C.c_size_t],
    "sandy_hip_rope_pair_cached": [T, T, T, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_layout_transform": [T, T, C.c_int32, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_attention_paged_view": [T, PV, PV, T, C.c_int64, C.c_double, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_paged_attention_noalloc": [T, P, P, T, T, C.c_int64, C.c_double, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_topk": [T, C.c_int64, C.c_int64, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_moe_gather": [T, T, T, C.c_int64, C.c_int64, T, T, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_moe_matmul": [T, T, T, C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_matmul": [T, T, C.c_int32, C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_linear": [T, T, T, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_matmul_glu": [T, T, C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_matmul_residual": [T, T, T, T, RS, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_matmul_rms": [T, RS, T, C.c_double, T, C.c_int32, T, C.c_void_p, ERR, C.c_size_t],
    "sandy_hip_moe_scatter_sum": [T, T, T, T, C.c_void_p, ERR, C.c_size_t],
}

# device runtime entry points: name -> (argtypes without the trailing err/cap, restype)
DEV = C.c_void_p
U32P = C.POINTER(C.c_uint32)
DEVICE_SIGNATURES = {
    "sandy_hip_device_create": ([C.c_int32, C.POINTER(C.c_void_p)], C.c_int),
    "sandy_hip_device_destroy": ([DEV], None),
    "sandy_hip_device_stream": ([DEV], C.c_void_p),
    "sandy_hip_device_synchronize": ([DEV], C.c_int),
    "sandy_hip_device_alloc": ([DEV, C.c_uint64, U32P], C.c_int),
    "sandy_hip_device_dealloc": ([DEV, C.c_uint32], C.c_int),
    "sandy_hip_device_buffer": ([DEV, C.c_uint32], C.c_void_p),
    "sandy_hip_device_load": ([DEV, C.c_void_p, C.c_uint64, U32P], C.c_int),
    "sandy_hip_device_read": ([DEV, C.c_uint32, C.c_uint64, C.c_uint64, C.c_void_p], C.c_int),
    "sandy_hip_device_paged_pool_create": ([DEV, C.POINTER(SandyPagedPoolDesc), U32P], C.c_int),
    "sandy_hip_device_paged_pool_destroy": ([DEV, C.c_uint32], C.c_int),
    "sandy_hip_device_paged_alloc": ([DEV, C.c_uint32, U32P], C.c_int),
    "sandy_hip_device_paged_dealloc": ([DEV, C.c_uint32], C.c_int),
    "sandy_hip_device_paged_reserve": ([DEV, C.c_uint32, C.c_int64], C.c_int),
    "sandy_hip_device_paged_append": ([DEV, C.c_uint32, T], C.c_int),
    "sandy_hip_device_paged_append_step": ([DEV, C.c_uint32, U32P, C.c_int32, T], C.c_int),
    "sandy_hip_device_paged_append_step_kv": ([DEV, C.c_uint32, U32P, C.c_uint32, U32P, C.c_int32, T, T], C.c_int),
    "sandy_hip_device_paged_positions": ([DEV, C.c_uint32, U32P, C.c_int32, T], C.c_int),
    "sandy_hip_device_paged_lengths": ([DEV, C.c_uint32, U32P, C.c_int32, T], C.c_int),
    "sandy_hip_device_decode_qkv": ([DEV, C.c_uint32, U32P, C.c_uint32, U32P, C.c_int32, T, C.c_int32, T, C.c_double,
                                     C.c_int32, T], C.c_int),
    "sandy_hip_device_matmul_qkv": ([DEV, T, C.POINTER(SandyRowStats), T, C.c_double, T, C.c_uint32, U32P, C.c_uint32,
                                     U32P, C.c_int32, C.c_int32, T, C.c_double, C.c_int32, T], C.c_int),
    "sandy_hip_device_paged_meta": ([DEV, C.c_uint32, C.POINTER(SandyPagedMeta)], C.c_int),
    "sandy_hip_device_paged_read": ([DEV, C.c_uint32, C.c_void_p, C.c_uint64], C.c_int),
    "sandy_hip_device_paged_views": ([DEV, C.c_uint32, P, T, T], C.c_int),
    "sandy_hip_device_paged_sync": ([DEV, C.c_uint32], C.c_int),
    "sandy_hip_device_graph_begin": ([DEV], C.c_int),
    "sandy_hip_device_graph_end": ([DEV, U32P], C.c_int),
    "sandy_hip_device_graph_launch": ([DEV, C.c_uint32], C.c_int),
    "sandy_hip_device_graph_destroy": ([DEV, C.c_uint32], C.c_int),
}
ST = C.c_void_p
DEVICE_SIGNATURES.update({
    "sandy_hip_safetensors_open": ([C.c_char_p, C.POINTER(C.c_void_p)], C.c_int),
    "sandy_hip_safetensors_close": ([ST], None),
    "sandy_hip_safetensors_count": ([ST], C.c_int64),
    "sandy_hip_safetensors_arena_bytes": ([ST], C.c_uint64),
    "sandy_hip_safetensors_info": ([ST, C.c_int64, C.POINTER(SandySafetensorInfo)], C.c_int),
    "sandy_hip_safetensors_find": ([ST, C.c_char_p], C.c_int64),
    "sandy_hip_safetensors_upload": ([ST, C.c_void_p, C.c_uint64, C.c_void_p], C.c_int),
})
NO_ERR_ARGS = {"sandy_hip_device_destroy", "sandy_hip_device_stream", "sandy_hip_device_buffer",
               "sandy_hip_safetensors_close", "sandy_hip_safetensors_count", "sandy_hip_safetensors_arena_bytes",
               "sandy_hip_safetensors_find"}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise BackendMissing(f"{LIB_PATH} is not built (run sandyrt_amd.build.build())")
        try:
            handle = C.CDLL(LIB_PATH)
        except OSError as exc:  # pragma: no cover - depends on the box
            raise BackendMissing(f"cannot load {LIB_PATH}: {exc}") from exc
        handle.sandy_hip_version.restype = C.c_char_p
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = C.c_int
        for name, (argtypes, restype) in DEVICE_SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes + ([] if name in NO_ERR_ARGS else [ERR, C.c_size_t])
            fn.restype = restype
        _lib = handle
    return _lib


def exported_symbols():
    return ["sandy_hip_version", *SIGNATURES.keys(), *DEVICE_SIGNATURES.keys()]


def dcall(name: str, *args):
    """Invoke a device-runtime entry point (error buffer appended)."""
    buf = C.create_string_buffer(512)
    rc = getattr(lib(), name)(*args, buf, C.c_size_t(512))
    if rc != 0:
        raise SandyError(rc, buf.value.decode(errors="replace"))


def desc(t: torch.Tensor | None):
    """SandyTensor describing a torch tensor's storage view (or NULL)."""
    if t is None:
        return None
    if t.dim() > MAX_RANK:
        raise SandyError(1, f"tensor rank {t.dim()} exceeds {MAX_RANK}")
    d = SandyTensor()
    d.data = t.untyped_storage().data_ptr() if t.numel() else t.data_ptr()
    d.dtype = _TORCH_TO_CODE[t.dtype]
    d.rank = t.dim()
    for i in range(t.dim()):
        d.dims[i] = t.shape[i]
        d.strides[i] = t.stride(i)
    d.storage_offset = t.storage_offset() if t.numel() else 0
    return C.pointer(d)


def call(name: str, *args, stream=None):
    """Invoke an entry point on `stream` (default: torch's current stream)."""
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    buf = C.create_string_buffer(512)
    rc = getattr(lib(), name)(*args, C.c_void_p(stream), buf, C.c_size_t(512))
    if rc != 0:
        raise SandyError(rc, buf.value.decode(errors="replace"))


def take_device_errors(stream=None) -> int:
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    flags = C.c_uint32(0)
    buf = C.create_string_buffer(512)
    rc = lib().sandy_hip_take_device_errors(C.c_void_p(stream), C.byref(flags), buf, C.c_size_t(512))
    if rc != 0:
        raise SandyError(rc, buf.value.decode(errors="replace"))
    return flags.value
