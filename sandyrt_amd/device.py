"""Python view of the device runtime (sandy_hip_device_* in include/sandyrt_hip.h).

Method names follow sandy::device::Device (src/device/Device.h:27-66):
alloc/dealloc/load/read, createPagedPool/allocPaged/reservePaged/appendPaged/
pagedMeta/read(paged), plus the decode-step helpers (append_step, positions)
and HIP graph capture.  Tensors passed in are torch GPU tensors (device
memory only); nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from ._lib import SandyPagedMeta, SandyPagedPoolDesc, dcall, desc


class HipDevice:
    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        dcall("sandy_hip_device_create", C.c_int32(ordinal), C.byref(h))
        self.handle = h
        self._torch_stream = torch.cuda.ExternalStream(self.stream, device=torch.device("cuda", ordinal))

    # ------------------------------------------------------------ lifetime
    def close(self):
        if self.handle:
            _lib.lib().sandy_hip_device_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return _lib.lib().sandy_hip_device_stream(self.handle)

    def torch_stream(self):
        """torch view of the device stream, for ops issued on it."""
        return self._torch_stream

    def synchronize(self):
        dcall("sandy_hip_device_synchronize", self.handle)

    # ------------------------------------------------------------ buffers
    def alloc(self, nbytes: int) -> int:
        bid = C.c_uint32()
        dcall("sandy_hip_device_alloc", self.handle, C.c_uint64(nbytes), C.byref(bid))
        return bid.value

    def dealloc(self, buffer: int):
        dcall("sandy_hip_device_dealloc", self.handle, C.c_uint32(buffer))

    def load(self, host: np.ndarray) -> int:
        host = np.ascontiguousarray(host)
        bid = C.c_uint32()
        dcall("sandy_hip_device_load", self.handle, host.ctypes.data_as(C.c_void_p), C.c_uint64(host.nbytes),
              C.byref(bid))
        return bid.value

    def read(self, buffer: int, nbytes: int, offset: int = 0) -> bytes:
        out = (C.c_char * nbytes)()
        dcall("sandy_hip_device_read", self.handle, C.c_uint32(buffer), C.c_uint64(offset), C.c_uint64(nbytes), out)
        return bytes(out)

    # ------------------------------------------------------------ paged tensors
    def create_paged_pool(self, template_shape, dtype: int, grow_dim: int, page_size: int, initial_pages: int = 0,
                          max_pages: int = -1, max_tensors: int = 64, max_blocks: int = 512) -> int:
        d = SandyPagedPoolDesc()
        d.dtype = dtype
        d.rank = len(template_shape)
        for i, v in enumerate(template_shape):
            d.dims[i] = v
        d.grow_dim = grow_dim
        d.page_size = page_size
        d.initial_pages = initial_pages
        d.max_pages = max_pages
        d.max_tensors = max_tensors
        d.max_blocks = max_blocks
        pid = C.c_uint32()
        dcall("sandy_hip_device_paged_pool_create", self.handle, C.byref(d), C.byref(pid))
        return pid.value

    def destroy_paged_pool(self, pool: int):
        dcall("sandy_hip_device_paged_pool_destroy", self.handle, C.c_uint32(pool))

    def alloc_paged(self, pool: int) -> int:
        tid = C.c_uint32()
        dcall("sandy_hip_device_paged_alloc", self.handle, C.c_uint32(pool), C.byref(tid))
        return tid.value

    def dealloc_paged(self, tensor: int):
        dcall("sandy_hip_device_paged_dealloc", self.handle, C.c_uint32(tensor))

    def reserve_paged(self, tensor: int, page_count: int):
        dcall("sandy_hip_device_paged_reserve", self.handle, C.c_uint32(tensor), C.c_int64(page_count))

    def append_paged(self, tensor: int, chunk: torch.Tensor):
        dcall("sandy_hip_device_paged_append", self.handle, C.c_uint32(tensor), desc(chunk))

    def append_step(self, pool: int, tensors, rows: torch.Tensor):
        ids = (C.c_uint32 * len(tensors))(*tensors)
        dcall("sandy_hip_device_paged_append_step", self.handle, C.c_uint32(pool), ids, C.c_int32(len(tensors)),
              desc(rows))

    def append_step_kv(self, k_pool: int, k_tensors, v_pool: int, v_tensors, k_rows: torch.Tensor,
                       v_rows: torch.Tensor):
        """append_step of the K rows and of the V rows, one launch."""
        kids = (C.c_uint32 * len(k_tensors))(*k_tensors)
        vids = (C.c_uint32 * len(v_tensors))(*v_tensors)
        if len(k_tensors) != len(v_tensors):
            raise ValueError("append_step_kv takes as many K as V tensors")
        dcall("sandy_hip_device_paged_append_step_kv", self.handle, C.c_uint32(k_pool), kids, C.c_uint32(v_pool), vids,
              C.c_int32(len(k_tensors)), desc(k_rows), desc(v_rows))

    def decode_qkv(self, k_pool: int, k_tensors, v_pool: int, v_tensors, qkv: torch.Tensor, q_heads: int,
                   positions: torch.Tensor, theta: float, q_out: torch.Tensor, split_half: bool = True):
        """RoPE q into q_out, RoPE k and append it, append v -- one launch for
        a decode step's [count, (q_heads + 2 kv_heads) head_dim] q/k/v rows."""
        kids = (C.c_uint32 * len(k_tensors))(*k_tensors)
        vids = (C.c_uint32 * len(v_tensors))(*v_tensors)
        dcall("sandy_hip_device_decode_qkv", self.handle, C.c_uint32(k_pool), kids, C.c_uint32(v_pool), vids,
              C.c_int32(len(k_tensors)), desc(qkv), C.c_int32(q_heads), desc(positions), C.c_double(theta),
              C.c_int32(1 if split_half else 0), desc(q_out))
        return q_out

    def matmul_qkv(self, x: torch.Tensor, w_paired: torch.Tensor, k_pool: int, k_tensors, v_pool: int, v_tensors,
                   q_heads: int, positions: torch.Tensor, theta: float, q_out: torch.Tensor, split_half: bool = True,
                   stats=None, norm_weight: torch.Tensor = None, eps: float = 0.0):
        """The q/k/v projection with decode_qkv in its epilogue (one launch):
        x [count, k] (RMS-normalised first with the row statistics `stats` of
        ops.row_stats and `norm_weight`), w_paired from ops.pair_rope_weight,
        rows appended at positions[i], which must equal the tensors' lengths."""
        if (stats is None) != (norm_weight is None):
            raise ValueError("matmul_qkv takes both stats and norm_weight or neither")
        kids = (C.c_uint32 * len(k_tensors))(*k_tensors)
        vids = (C.c_uint32 * len(v_tensors))(*v_tensors)
        st = C.byref(_lib.SandyRowStats(stats.data_ptr(), stats.shape[0], stats.shape[1])) if stats is not None else None
        dcall("sandy_hip_device_matmul_qkv", self.handle, desc(x), st, desc(norm_weight), C.c_double(eps), desc(w_paired), C.c_uint32(k_pool), kids, C.c_uint32(v_pool), vids,
              C.c_int32(len(k_tensors)), C.c_int32(q_heads), desc(positions), C.c_double(theta),
              C.c_int32(1 if split_half else 0), desc(q_out))
        return q_out

    def positions(self, pool: int, tensors, out: torch.Tensor):
        ids = (C.c_uint32 * len(tensors))(*tensors)
        dcall("sandy_hip_device_paged_positions", self.handle, C.c_uint32(pool), ids, C.c_int32(len(tensors)),
              desc(out))
        return out

    def lengths(self, pool: int, tensors, out: torch.Tensor):
        """out[i] = device length of tensors[i] (the next row's position)."""
        ids = (C.c_uint32 * len(tensors))(*tensors)
        dcall("sandy_hip_device_paged_lengths", self.handle, C.c_uint32(pool), ids, C.c_int32(len(tensors)),
              desc(out))
        return out

    def paged_meta(self, tensor: int) -> SandyPagedMeta:
        m = SandyPagedMeta()
        dcall("sandy_hip_device_paged_meta", self.handle, C.c_uint32(tensor), C.byref(m))
        return m

    def read_paged(self, tensor: int, np_dtype) -> np.ndarray:
        m = self.paged_meta(tensor)
        shape = [m.dims[i] for i in range(m.rank)]
        out = np.empty(shape, dtype=np_dtype)
        dcall("sandy_hip_device_paged_read", self.handle, C.c_uint32(tensor), out.ctypes.data_as(C.c_void_p),
              C.c_uint64(out.nbytes))
        return out

    def paged_views(self, pool: int):
        """(SandyPagedCache pointer, block table SandyTensor pointer, lengths SandyTensor pointer)"""
        cache = _lib.SandyPagedCache()
        table = _lib.SandyTensor()
        lengths = _lib.SandyTensor()
        dcall("sandy_hip_device_paged_views", self.handle, C.c_uint32(pool), C.byref(cache), C.byref(table),
              C.byref(lengths))
        return C.pointer(cache), C.pointer(table), C.pointer(lengths)

    def paged_sync(self, pool: int):
        dcall("sandy_hip_device_paged_sync", self.handle, C.c_uint32(pool))

    # ------------------------------------------------------------ graphs
    def graph_begin(self):
        dcall("sandy_hip_device_graph_begin", self.handle)

    def graph_end(self) -> int:
        gid = C.c_uint32()
        dcall("sandy_hip_device_graph_end", self.handle, C.byref(gid))
        return gid.value

    def graph_launch(self, graph: int):
        dcall("sandy_hip_device_graph_launch", self.handle, C.c_uint32(graph))

    def graph_destroy(self, graph: int):
        dcall("sandy_hip_device_graph_destroy", self.handle, C.c_uint32(graph))
