"""Safetensors weights on the device (sandy_hip_safetensors_* in
include/sandyrt_hip.h), mirroring the reference's EagerSafeTensorWeights
(src/weight/SafeTensorWeights.h:29-48): `descriptors()` in name order and
`get_tensor(name)` -- here a torch view into one device arena that
`upload()` fills by streaming the file through pinned staging buffers."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import SandySafetensorInfo, dcall

_CODE_TO_TORCH = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16, 3: torch.int32, 4: torch.int64,
                  5: torch.uint8}


@dataclass
class TensorDesc:
    name: str
    shape: tuple
    dtype: torch.dtype
    nbytes: int
    arena_offset: int


class SafeTensors:
    def __init__(self, path: str):
        h = C.c_void_p()
        dcall("sandy_hip_safetensors_open", str(path).encode(), C.byref(h))
        self.handle = h
        self.arena = None
        self._descs = []
        for i in range(_lib.lib().sandy_hip_safetensors_count(h)):
            info = SandySafetensorInfo()
            dcall("sandy_hip_safetensors_info", h, C.c_int64(i), C.byref(info))
            self._descs.append(TensorDesc(info.name.decode(), tuple(info.dims[j] for j in range(info.rank)),
                                          _CODE_TO_TORCH[info.dtype], info.nbytes, info.arena_offset))
        self._by_name = {d.name: d for d in self._descs}

    def descriptors(self):
        return list(self._descs)

    @property
    def arena_bytes(self) -> int:
        return int(_lib.lib().sandy_hip_safetensors_arena_bytes(self.handle))

    def upload(self, device="cuda", stream=None) -> torch.Tensor:
        """Copy every tensor into one device arena (allocated here) and return it."""
        arena = torch.empty(max(256, self.arena_bytes), dtype=torch.uint8, device=device)
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        dcall("sandy_hip_safetensors_upload", self.handle, C.c_void_p(arena.data_ptr()), C.c_uint64(arena.numel()),
              C.c_void_p(s))
        self.arena = arena
        return arena

    def get_tensor(self, name: str):
        """Device view of one tensor (None when absent); upload() first."""
        d = self._by_name.get(name)
        if d is None:
            return None
        if self.arena is None:
            raise _lib.SandyError(1, "safetensors tensors are on the device only after upload()")
        flat = self.arena[d.arena_offset:d.arena_offset + d.nbytes]
        return flat.view(d.dtype).view(d.shape) if d.nbytes else torch.empty(d.shape, dtype=d.dtype,
                                                                                device=self.arena.device)

    def close(self):
        if self.handle:
            _lib.lib().sandy_hip_safetensors_close(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass
