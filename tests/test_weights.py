"""Safetensors header parsing on the CPU (sandy_hip_safetensors_open / info /
find, host code only): the reference loader's dtype table, name order and
error wording (src/weight/SafeTensorWeights.cpp:14-23, 44-117), on files
written by the safetensors package."""
import json
import os
import struct

import numpy as np
import pytest
import torch

from sandyrt_amd._lib import SandyError
from sandyrt_amd.weights import SafeTensors


def write_raw(path, header: dict, data: bytes):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


def test_descriptors_in_name_order_with_every_dtype(tmp_path):
    from safetensors.torch import save_file
    tensors = {
        "model.layers.1.w": torch.randn(3, 5, dtype=torch.bfloat16),
        "model.layers.0.w": torch.randn(7, dtype=torch.float32),
        "a.half": torch.randn(2, 2, dtype=torch.float16),
        "ids32": torch.arange(4, dtype=torch.int32),
        "ids64": torch.arange(3, dtype=torch.int64),
        "bytes": torch.arange(9, dtype=torch.uint8).view(3, 3),
        "mask": torch.tensor([True, False]),
        "empty": torch.zeros(0, 4),
    }
    p = str(tmp_path / "w.safetensors")
    save_file(tensors, p, metadata={"format": "pt"})
    st = SafeTensors(p)
    ds = st.descriptors()
    assert [d.name for d in ds] == sorted(tensors)
    by = {d.name: d for d in ds}
    want_dtype = {"model.layers.1.w": torch.bfloat16, "model.layers.0.w": torch.float32, "a.half": torch.float16,
                  "ids32": torch.int32, "ids64": torch.int64, "bytes": torch.uint8, "mask": torch.uint8,
                  "empty": torch.float32}
    for name, t in tensors.items():
        assert by[name].shape == tuple(t.shape)
        assert by[name].dtype == want_dtype[name]
        assert by[name].nbytes == t.numel() * t.element_size()
    offs = sorted((d.arena_offset, d.nbytes) for d in ds)
    for (a, n), (b, _) in zip(offs, offs[1:]):
        assert a % 256 == 0 and a + n <= b
    assert st.arena_bytes >= offs[-1][0] + offs[-1][1]
    from sandyrt_amd import _lib
    assert _lib.lib().sandy_hip_safetensors_find(st.handle, b"ids64") == [d.name for d in ds].index("ids64")
    assert _lib.lib().sandy_hip_safetensors_find(st.handle, b"absent") == -1
    st.close()


def test_metadata_and_escaped_names(tmp_path):
    p = str(tmp_path / "m.safetensors")
    header = {"__metadata__": {"k": "v"}, "café.\"q\"": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    write_raw(p, header, np.ones(2, np.float32).tobytes())
    st = SafeTensors(p)
    assert [d.name for d in st.descriptors()] == ["café.\"q\""]


@pytest.mark.parametrize("case,msg", [
    ("missing", "cannot open"),
    ("tiny", "safetensors file too small"),
    ("header", "safetensors header size exceeds file"),
    ("dtype", "unsupported safetensors dtype: F64"),
    ("json", "not valid JSON"),
    ("range", "outside the data section"),
    ("size", "does not match its shape"),
])
def test_errors_use_the_reference_wording(tmp_path, case, msg):
    p = str(tmp_path / "bad.safetensors")
    if case == "tiny":
        open(p, "wb").write(b"\x01\x02")
    elif case == "header":
        open(p, "wb").write(struct.pack("<Q", 1000) + b"{}")
    elif case == "dtype":
        write_raw(p, {"x": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "json":
        open(p, "wb").write(struct.pack("<Q", 5) + b"{\"a\":")
    elif case == "range":
        write_raw(p, {"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, b"\0" * 8)
    elif case == "size":
        write_raw(p, {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8)
    with pytest.raises(SandyError, match=msg):
        SafeTensors(p)
