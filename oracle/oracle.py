"""numpy front-end for the CPU parity checker (TEST INFRASTRUCTURE ONLY).

Two back-ends share one call surface:

* ``Oracle()`` wraps ``oracle/liboracle.so`` -- the C restatement of the
  reference CPU math (``sandy_oracle.c``), which travels with the repository;
* ``Oracle(reference=True)`` wraps ``oracle/_ref/libsandyref.so`` -- the
  reference's own ``src/core`` built from its sources by ``oracle/Makefile``,
  present only where that build could run.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may
use this module, and only as the checker.  Tensors are numpy arrays: float32
for F32, uint16 bit patterns for BF16, int32/int64 for index tensors.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libsandyref.so")

F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4

# scalar ops (src/ir/KernelIR.h:317-337 order)
(LOAD, CONST, ADD, SUB, MUL, DIV, MAX, MIN, NEG, SQRT, RSQRT, EXP, LOG, TANH,
 RELU, CAST) = range(16)


class ScalarNode(C.Structure):
    _fields_ = [
        ("id", C.c_uint32),
        ("op", C.c_int32),
        ("dtype", C.c_int32),
        ("input_index", C.c_uint32),
        ("constant", C.c_double),
        ("operand_count", C.c_int32),
        ("operands", C.c_uint32 * 2),
    ]


def make_nodes(spec):
    """spec: list of (id, op, input_index, constant, operands)"""
    arr = (ScalarNode * len(spec))()
    for i, (nid, op, inp, const, operands) in enumerate(spec):
        arr[i].id = nid
        arr[i].op = op
        arr[i].dtype = F32
        arr[i].input_index = inp
        arr[i].constant = const
        arr[i].operand_count = len(operands)
        for j, o in enumerate(operands):
            arr[i].operands[j] = o
    return arr


class OracleError(RuntimeError):
    pass


def build(reference: bool = False) -> None:
    """Compile the checker (``make -C oracle``); the reference build only when
    its source tree is present."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if reference and os.path.isdir("/root/reference/src/core"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)
        if os.path.exists(os.path.join(os.path.dirname(HERE), "sandyrt_amd", "libsandyrt_hip.so")):
            subprocess.run(["make", "-s", "-C", HERE, "binding"], check=True)


def dtype_code(a: np.ndarray, bf16: bool = False) -> int:
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.uint16:
        return BF16
    if a.dtype == np.int32:
        return I32
    if a.dtype == np.int64:
        return I64
    raise TypeError(f"unsupported array dtype {a.dtype}")


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (src/core/Tensor.h:43-49)."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    lsb = (b >> 16) & 1
    return ((b + 0x7FFF + lsb) >> 16).astype(np.uint16)


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f32(a: np.ndarray) -> np.ndarray:
    return bf16_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)


class Oracle:
    def __init__(self, reference: bool = False):
        path = REF_PATH if reference else LIB_PATH
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = C.CDLL(path)
        self.prefix = "ref_" if reference else "oracle_"
        self.reference = reference
        err = getattr(self.lib, self.prefix + "last_error")
        err.restype = C.c_char_p
        self._err = err

    def _call(self, name, *args):
        fn = getattr(self.lib, self.prefix + name)
        fn.restype = C.c_int
        conv = []
        for a in args:
            if isinstance(a, float):
                conv.append(C.c_float(a))
            elif isinstance(a, bool):
                conv.append(C.c_int(int(a)))
            elif isinstance(a, int):
                conv.append(C.c_int64(a))
            else:
                conv.append(a)
        rc = fn(*conv)
        if rc != 0:
            raise OracleError(self._err().decode())

    # ------------------------------------------------------------------ norms
    def rms_norm(self, x, weight, eps):
        cols = x.shape[-1]
        rows = x.size // cols if cols else 0
        out = np.empty_like(x)
        self._call("rms_norm", _p(x), _p(weight), _p(out), C.c_int(dtype_code(x)), rows, cols, float(eps))
        return out

    def layer_norm(self, x, weight, bias, eps):
        cols = x.shape[-1]
        rows = x.size // cols
        out = np.empty_like(x)
        self._call("layer_norm", _p(x), _p(weight), _p(bias), _p(out), C.c_int(dtype_code(x)),
                   rows, cols, float(eps))
        return out

    def softmax(self, x, axis=-1):
        axis = axis % x.ndim
        outer = int(np.prod(x.shape[:axis], dtype=np.int64))
        inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
        out = np.empty_like(x)
        if x.size == 0:
            return out
        self._call("softmax", _p(x), _p(out), C.c_int(dtype_code(x)), outer, x.shape[axis], inner)
        return out

    def sum(self, x, axis=-1, keepdims=True):
        axis = axis % x.ndim
        outer = int(np.prod(x.shape[:axis], dtype=np.int64))
        inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
        shape = list(x.shape)
        shape[axis] = 1
        out = np.empty(shape, dtype=x.dtype)
        self._call("sum", _p(x), _p(out), C.c_int(dtype_code(x)), outer, x.shape[axis], inner)
        return out if keepdims else out.reshape([d for i, d in enumerate(x.shape) if i != axis])

    def rope(self, x, theta, rotary_dim=-1, split_half=False, position_ids=None):
        dim = x.shape[-1]
        seq = x.shape[-2]
        vectors = x.size // dim
        out = np.empty_like(x)
        pos_dtype = dtype_code(position_ids) if position_ids is not None else I64
        pos_count = position_ids.size if position_ids is not None else 0
        self._call("rope", _p(x), _p(position_ids), C.c_int(pos_dtype), pos_count, _p(out),
                   C.c_int(dtype_code(x)), vectors, seq, dim, float(theta), int(rotary_dim),
                   C.c_int(int(split_half)))
        return out

    def attention(self, q, k, v, position_offsets=None, window=0, scale=-1.0):
        """q [B, H, Tq, D], k/v [B, Hkv, Tk, D] (rank 3 accepted as batch 1)."""
        squeeze = q.ndim == 3
        if squeeze:
            q, k, v = q[None], k[None], v[None]
        b, h, tq, d = q.shape
        hkv, tk = k.shape[1], k.shape[2]
        out = np.empty_like(q)
        pos_dtype = dtype_code(position_offsets) if position_offsets is not None else I64
        self._call("attention", _p(q), _p(k), _p(v), _p(position_offsets), C.c_int(pos_dtype), _p(out),
                   C.c_int(dtype_code(q)), b, h, hkv, tq, tk, d, int(window), float(scale))
        return out[0] if squeeze else out

    def topk(self, x, k, axis=-1, index_dtype=np.int64):
        axis = axis % x.ndim
        outer = int(np.prod(x.shape[:axis], dtype=np.int64))
        inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
        shape = list(x.shape)
        shape[axis] = k
        values = np.empty(shape, dtype=x.dtype)
        indices = np.empty(shape, dtype=index_dtype)
        self._call("topk", _p(x), _p(values), _p(indices), C.c_int(dtype_code(indices)),
                   C.c_int(dtype_code(x)), outer, x.shape[axis], inner, int(k))
        return values, indices

    def embedding(self, ids, weight):
        vocab = weight.shape[0]
        hidden = weight.shape[1] if weight.ndim == 2 else 1
        out = np.empty(ids.shape + weight.shape[1:], dtype=weight.dtype)
        self._call("embedding", _p(ids), C.c_int(dtype_code(ids)), ids.size, _p(weight),
                   C.c_int(dtype_code(weight)), vocab, hidden, _p(out))
        return out

    def moe_gather(self, x, topk_ids, topk_weights, num_experts, index_dtype=np.int64):
        squeeze = x.ndim == 2
        if squeeze:
            x, topk_ids, topk_weights = x[None], topk_ids[None], topk_weights[None]
        b, seq, hidden = x.shape
        top_k = topk_ids.shape[-1]
        rows = seq * top_k
        packed_x = np.empty((b, rows, hidden), dtype=x.dtype)
        packed_w = np.empty((b, rows), dtype=topk_weights.dtype)
        token_ids = np.empty((b, rows), dtype=index_dtype)
        offsets = np.empty((b, num_experts + 1), dtype=index_dtype)
        self._call("moe_gather", _p(x), C.c_int(dtype_code(x)), _p(topk_ids), C.c_int(dtype_code(topk_ids)),
                   _p(topk_weights), C.c_int(dtype_code(topk_weights)), b, seq, hidden, int(num_experts),
                   top_k, _p(packed_x), _p(packed_w), _p(token_ids), C.c_int(dtype_code(token_ids)),
                   _p(offsets), C.c_int(dtype_code(offsets)))
        if squeeze:
            return packed_x[0], packed_w[0], token_ids[0], offsets[0]
        return packed_x, packed_w, token_ids, offsets

    def moe_matmul(self, x, expert_offsets, weight, transpose_rhs=True):
        squeeze = x.ndim == 2
        if squeeze:
            x, expert_offsets = x[None], expert_offsets[None]
        b, rows, kin = x.shape
        experts = weight.shape[0]
        m = weight.shape[1] if transpose_rhs else weight.shape[2]
        out = np.empty((b, rows, m), dtype=x.dtype)
        self._call("moe_matmul", _p(x), _p(expert_offsets), C.c_int(dtype_code(expert_offsets)), _p(weight),
                   C.c_int(dtype_code(x)), b, rows, kin, experts, m, C.c_int(int(transpose_rhs)), _p(out))
        return out[0] if squeeze else out

    def moe_scatter_sum(self, packed_out, packed_weights, token_ids, seq):
        squeeze = packed_out.ndim == 2
        if squeeze:
            packed_out, packed_weights, token_ids = packed_out[None], packed_weights[None], token_ids[None]
        b, rows, hidden = packed_out.shape
        out = np.empty((b, seq, hidden), dtype=packed_out.dtype)
        self._call("moe_scatter_sum", _p(packed_out), _p(packed_weights), _p(token_ids),
                   C.c_int(dtype_code(token_ids)), C.c_int(dtype_code(packed_out)), b, rows, hidden, seq, _p(out))
        return out[0] if squeeze else out

    @staticmethod
    def matmul_shape(lshape, rshape, transpose_lhs=False, transpose_rhs=False):
        """output shape of matmul (ShapeUtil.cpp:39-71 batch broadcast)"""
        lb, rb = list(lshape[:-2]), list(rshape[:-2])
        rank = max(len(lb), len(rb))
        lb = [1] * (rank - len(lb)) + lb
        rb = [1] * (rank - len(rb)) + rb
        batch = [a if a == b or b == 1 or (a > b and a % b == 0) else b for a, b in zip(lb, rb)]
        m = lshape[-1] if transpose_lhs else lshape[-2]
        n = rshape[-2] if transpose_rhs else rshape[-1]
        return tuple(batch) + (m, n)

    def matmul(self, lhs, rhs, transpose_lhs=False, transpose_rhs=False):
        lhs, rhs = np.ascontiguousarray(lhs), np.ascontiguousarray(rhs)
        out = np.empty(self.matmul_shape(lhs.shape, rhs.shape, transpose_lhs, transpose_rhs), dtype=lhs.dtype)
        ld = (C.c_int64 * lhs.ndim)(*lhs.shape)
        rd = (C.c_int64 * rhs.ndim)(*rhs.shape)
        self._call("matmul", _p(lhs), ld, C.c_int(lhs.ndim), _p(rhs), rd, C.c_int(rhs.ndim),
                   C.c_int(int(transpose_lhs)), C.c_int(int(transpose_rhs)), _p(out), C.c_int(dtype_code(lhs)))
        return out

    def linear(self, x, weight, bias):
        rows = x.size // x.shape[-1]
        out = np.empty(x.shape[:-1] + (weight.shape[0],), dtype=x.dtype)
        self._call("linear", _p(x), _p(weight), _p(bias), _p(out), C.c_int(dtype_code(x)), rows,
                   x.shape[-1], weight.shape[0])
        return out

    # ------------------------------------------------------ element-wise ops
    def binary(self, op, lhs, rhs):
        """op: 'add' | 'mul' | 'div' with right-aligned broadcasting"""
        code = {"add": 0, "mul": 1, "div": 2}[op]
        oshape = np.broadcast_shapes(lhs.shape, rhs.shape)
        out = np.empty(oshape, dtype=lhs.dtype if lhs.ndim else rhs.dtype)
        ls = (C.c_int64 * max(1, lhs.ndim))(*lhs.shape)
        rs = (C.c_int64 * max(1, rhs.ndim))(*rhs.shape)
        os_ = (C.c_int64 * max(1, len(oshape)))(*oshape)
        self._call("binary", C.c_int(code), _p(lhs), ls, C.c_int(lhs.ndim), _p(rhs), rs, C.c_int(rhs.ndim),
                   _p(out), os_, C.c_int(len(oshape)), C.c_int(dtype_code(out)))
        return out

    def unary(self, op, x):
        code = {"relu": 10, "sqrt": 11, "tanh": 12}[op]
        out = np.empty_like(x)
        self._call("unary", C.c_int(code), _p(x), _p(out), C.c_int(dtype_code(x)), x.size)
        return out

    def elementwise_dag(self, nodes, result, inputs, broadcast, out_shape, out_dtype):
        """Fused group in fp32 registers (restatement only; the reference CPU
        device cannot execute fused groups, CpuDevice.cpp:138-190)."""
        if self.reference:
            raise OracleError("reference CPU math has no fused element-wise entry")
        n = len(inputs)
        ptrs = (C.c_void_p * max(1, n))(*[a.ctypes.data for a in inputs])
        dts = (C.c_int32 * max(1, n))(*[dtype_code(a) for a in inputs])
        numels = (C.c_int64 * max(1, n))(*[a.size for a in inputs])
        bc = (C.c_int32 * max(1, n))(*[int(b) for b in broadcast])
        out = np.empty(out_shape, dtype=out_dtype)
        self._call("elementwise_dag", nodes, C.c_int32(len(nodes)), C.c_uint32(result), ptrs, dts, numels, bc,
                   C.c_int32(n), _p(out), C.c_int(dtype_code(out)), out.size)
        return out

    def paged_to_dense(self, pool, page_ids, prefix, grow_length, page_size, inner):
        """pool: [num_pages, prefix, page_size, inner]; returns [prefix, grow, inner]."""
        out = np.empty((prefix, grow_length, inner), dtype=pool.dtype)
        ids = np.ascontiguousarray(page_ids, dtype=np.int32)
        self._call("paged_to_dense", _p(pool), prefix * page_size * inner, ids.ctypes.data_as(C.c_void_p),
                   ids.size, prefix, grow_length, page_size, inner, pool.itemsize, _p(out))
        return out
