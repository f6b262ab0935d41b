"""Host-side operator API of the gfx950 backend.

One function per KernelIR kernel family of the reference
(src/ir/KernelIR.h:65-85), with the reference's argument meaning and error
wording.  Tensors are torch tensors on the GPU (torch is the allocator and
stream provider only); every call goes through the C ABI of
include/sandyrt_hip.h into the hand-written HIP kernels.  There is no CPU
path: without the built library every call raises BackendMissing.

Outputs are allocated when `out` is not given.  Calls are stream-ordered on
torch's current stream and do not synchronise, except `check_device_errors`.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import SandyError, call, desc

# ScalarOp codes (src/ir/KernelIR.h:317-337)
LOAD, CONST, ADD, SUB, MUL, DIV, MAX, MIN, NEG, SQRT, RSQRT, EXP, LOG, TANH, RELU, CAST = range(16)


def _require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise SandyError(1, "sandyrt_amd tensors must live on the GPU")


class PagedTensor:
    """The reference's paged tensor as a kernel input (CudaDeviceBufferView
    with paged = true, src/device/cuda/CudaDevice.cpp:468-493): `pages` is a
    device uint64 tensor of page start addresses, `dims` the logical shape,
    and a page holds `page_size` rows of dimension `grow_dim` for every
    leading element ([prefix, page_size, inner],
    src/device/cuda/CudaKernelUtils.cuh:82-108).  The families that read
    paged inputs in the reference (element-wise, norm, RoPE, softmax, sum,
    embedding, attention q and positions) accept one wherever they take an
    input tensor."""

    def __init__(self, pages: torch.Tensor, dims, grow_dim: int, page_size: int, dtype: torch.dtype):
        assert pages.is_cuda and pages.dtype in (torch.int64, torch.uint64) and pages.dim() == 1
        self.pages, self.dims, self.grow_dim = pages, list(dims), grow_dim
        self.page_size, self.dtype = page_size, dtype
        self.is_cuda = True
        self.device = pages.device
        self.shape = torch.Size(self.dims)

    def struct(self):
        s = _lib.SandyPagedTensor()
        s.pages = self.pages.data_ptr() if self.pages.numel() else None
        s.dtype = _lib._TORCH_TO_CODE[self.dtype]
        s.rank = len(self.dims)
        for i, d in enumerate(self.dims):
            s.dims[i] = d
        s.grow_dim = self.grow_dim
        s.page_size = self.page_size
        s.page_count = self.pages.numel()
        return C.pointer(s)


def paged_to_dense(x: PagedTensor, out=None):
    """The logical elements of a paged tensor as a contiguous tensor (the
    gather every family runs on a paged input before its dense kernel)."""
    out = torch.empty(x.dims, dtype=x.dtype, device=x.device) if out is None else out
    call("sandy_hip_paged_to_dense", x.struct(), desc(out))
    return out


def _reads_paged(fn):
    """Inputs given as PagedTensor (also inside a list of inputs) are gathered
    to dense copies before the family's dense entry point runs."""
    import functools

    def dense(v):
        if isinstance(v, PagedTensor):
            return paged_to_dense(v)
        if isinstance(v, (list, tuple)) and any(isinstance(u, PagedTensor) for u in v):
            return type(v)(dense(u) for u in v)
        return v

    @functools.wraps(fn)
    def run(*args, **kw):
        return fn(*[dense(a) for a in args], **{k: (v if k == "out" else dense(v)) for k, v in kw.items()})

    return run


def check_device_errors() -> None:
    """Synchronise and raise the first recorded device-side value error
    (bad expert/token/position ids), worded like the reference."""
    _lib.take_device_errors()


# ------------------------------------------------------------------ norms
@_reads_paged
def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, epsilon: float, out=None):
    """NormKernelOp RMSNorm (src/core/TensorCalc.cpp:1953-2000)."""
    _require_gpu(x, weight)
    out = torch.empty_like(x) if out is None else out
    call("sandy_hip_norm", 0, desc(x), desc(weight), None, float(epsilon), desc(out))
    return out


@_reads_paged
def layer_norm(x, weight, bias, epsilon: float, out=None):
    """NormKernelOp LayerNorm (src/core/TensorCalc.cpp:2010-2077)."""
    _require_gpu(x, weight, bias)
    out = torch.empty_like(x) if out is None else out
    call("sandy_hip_norm", 1, desc(x), desc(weight), desc(bias), float(epsilon), desc(out))
    return out


def add_rms_norm(x, residual, weight, epsilon: float, sum_out=None, out=None):
    """`s = x + residual; y = rms_norm(s, weight)` in one pass; returns (s, y)."""
    _require_gpu(x, residual, weight)
    sum_out = torch.empty_like(x) if sum_out is None else sum_out
    out = torch.empty_like(x) if out is None else out
    call("sandy_hip_add_rms_norm", desc(x), desc(residual), desc(weight), float(epsilon), desc(sum_out), desc(out))
    return sum_out, out


# ------------------------------------------------------------------ rope / softmax / reductions
@_reads_paged
def rope(x, theta: float, rotary_dim: int = -1, split_half: bool = False, position_ids=None, out=None):
    """RoPEKernelOp (src/core/TensorCalc.cpp:1823-1951)."""
    _require_gpu(x, position_ids)
    out = torch.empty_like(x) if out is None else out
    call("sandy_hip_rope", desc(x), desc(position_ids), float(theta), int(rotary_dim), int(bool(split_half)),
         desc(out))
    return out


def rope_pair(q, k, theta: float, rotary_dim: int = -1, split_half: bool = False, position_ids=None, q_out=None,
              k_out=None):
    """RoPE of q and k (same positions, sequence length and head dim) in one
    launch; identical to rope(q) and rope(k)."""
    _require_gpu(q, k, position_ids)
    q_out = torch.empty_like(q) if q_out is None else q_out
    k_out = torch.empty_like(k) if k_out is None else k_out
    call("sandy_hip_rope_pair", desc(q), desc(k), desc(position_ids), float(theta), int(rotary_dim),
         int(bool(split_half)), desc(q_out), desc(k_out))
    return q_out, k_out


def rope_cache(seq: int, dim: int, theta: float, rotary_dim: int = -1, split_half: bool = True, position_ids=None,
               out=None, device="cuda"):
    """The cos/sin of a forward pass's positions, [seq, rotary_dim / 2, 2] f32,
    built once and shared by q, k and every layer (rope_pair_cached)."""
    _require_gpu(position_ids)
    rd = dim if rotary_dim < 0 else rotary_dim
    out = torch.empty(seq, rd // 2, 2, dtype=torch.float32, device=device) if out is None else out
    call("sandy_hip_rope_cache", desc(position_ids), int(seq), float(theta), int(rotary_dim), int(dim),
         int(bool(split_half)), desc(out))
    return out


def rope_pair_cached(q, k, cache, q_out=None, k_out=None):
    """Split-half RoPE of q and k (or q alone, k None) from a rope_cache."""
    _require_gpu(q, k, cache)
    q_out = torch.empty_like(q) if q_out is None else q_out
    k_out = (torch.empty_like(k) if k_out is None else k_out) if k is not None else None
    call("sandy_hip_rope_pair_cached", desc(q), desc(k), desc(cache), desc(q_out), desc(k_out))
    return q_out, k_out


@_reads_paged
def softmax(x, axis: int = -1, out=None):
    """SoftmaxKernelOp (src/core/TensorCalc.cpp:1337-1399)."""
    _require_gpu(x)
    out = torch.empty_like(x) if out is None else out
    call("sandy_hip_softmax", desc(x), int(axis), desc(out))
    return out


@_reads_paged
def sum(x, axis: int = -1, keep_dims: bool = True, out=None):  # noqa: A001 - reference op name
    """ReductionKernelOp Sum over one axis (src/core/TensorCalc.cpp:1401-1445)."""
    _require_gpu(x)
    ax = axis % x.dim()
    shape = list(x.shape)
    if keep_dims:
        shape[ax] = 1
    else:
        del shape[ax]
    out = torch.empty(shape, dtype=x.dtype, device=x.device) if out is None else out
    call("sandy_hip_reduce_sum", desc(x), int(axis), int(bool(keep_dims)), desc(out))
    return out


@_reads_paged
def embedding(ids, weight, out=None):
    """GatherKernelOp / embedding (src/core/TensorCalc.cpp:1520-1563)."""
    _require_gpu(ids, weight)
    shape = list(ids.shape) + list(weight.shape[1:])
    out = torch.empty(shape, dtype=weight.dtype, device=weight.device) if out is None else out
    call("sandy_hip_gather", desc(ids), desc(weight), desc(out))
    return out


# ------------------------------------------------------------------ fused element-wise groups
@dataclass
class ScalarNode:
    """One node of an ElementwiseKernelOp scalar DAG (src/ir/KernelIR.h:346-355)."""

    id: int
    op: int
    input_index: int = 0
    constant: float = 0.0
    operands: tuple = ()


def _nodes(nodes):
    arr = (_lib.SandyScalarNode * len(nodes))()
    for i, n in enumerate(nodes):
        arr[i].id = n.id
        arr[i].op = n.op
        arr[i].dtype = _lib.F32
        arr[i].input_index = n.input_index
        arr[i].constant = float(n.constant)
        arr[i].operand_count = len(n.operands)
        for j, o in enumerate(n.operands):
            arr[i].operands[j] = o
    return arr


@_reads_paged
def elementwise(nodes, result: int, inputs, broadcast=None, out_shape=None, out_dtype=None, out=None):
    """Run one fused ElementwiseKernelOp.  `nodes` in dependency order;
    broadcast[i] True marks a right-aligned broadcast input."""
    _require_gpu(*inputs)
    broadcast = broadcast or [False] * len(inputs)
    if out is None:
        shape = out_shape if out_shape is not None else inputs[0].shape
        dtype = out_dtype if out_dtype is not None else inputs[0].dtype
        out = torch.empty(shape, dtype=dtype, device=inputs[0].device)
    n = len(inputs)
    arr = (_lib.SandyTensor * max(1, n))()
    for i, t in enumerate(inputs):
        arr[i] = desc(t).contents
    bc = (C.c_int32 * max(1, n))(*[int(bool(b)) for b in broadcast])
    call("sandy_hip_elementwise", _nodes(nodes), len(nodes), int(result), arr, bc, n, desc(out))
    return out


# Scalar DAGs of the model-level builtins, as src/ir/BuiltinLowering.cpp
# lowers them (gelu 116-140, silu 142-158, softcap 160-185).
def silu_mul_nodes():
    """silu(gate) * up with silu(x) = (0.5 x)(1 + tanh(0.5 x)); inputs (gate, up)."""
    return [
        ScalarNode(0, LOAD, 0), ScalarNode(1, CONST, constant=0.5), ScalarNode(2, MUL, operands=(1, 0)),
        ScalarNode(3, TANH, operands=(2,)), ScalarNode(4, CONST, constant=1.0), ScalarNode(5, ADD, operands=(4, 3)),
        ScalarNode(6, MUL, operands=(2, 5)), ScalarNode(7, LOAD, 1), ScalarNode(8, MUL, operands=(6, 7)),
    ], 8


def gelu_mul_nodes():
    """gelu(gate) * up, gelu(x) = (0.5 x)(1 + tanh(0.7978845608028654 (x + 0.044715 x^3)))."""
    return [
        ScalarNode(0, LOAD, 0), ScalarNode(1, CONST, constant=0.5), ScalarNode(2, MUL, operands=(1, 0)),
        ScalarNode(3, MUL, operands=(0, 0)), ScalarNode(4, MUL, operands=(3, 0)),
        ScalarNode(5, CONST, constant=0.044715), ScalarNode(6, MUL, operands=(5, 4)),
        ScalarNode(7, ADD, operands=(0, 6)), ScalarNode(8, CONST, constant=0.7978845608028654),
        ScalarNode(9, MUL, operands=(8, 7)), ScalarNode(10, TANH, operands=(9,)),
        ScalarNode(11, CONST, constant=1.0), ScalarNode(12, ADD, operands=(11, 10)),
        ScalarNode(13, MUL, operands=(2, 12)), ScalarNode(14, LOAD, 1), ScalarNode(15, MUL, operands=(13, 14)),
    ], 15


def gelu_nodes():
    """gelu(x) = (0.5 x)(1 + tanh(0.7978845608028654 (x + 0.044715 x^3))); one input."""
    nodes, _ = gelu_mul_nodes()
    return nodes[:14], 13


def softcap_nodes(cap: float):
    """softcap(x, c) = tanh(x * (1 / c)) * c; one input."""
    return [
        ScalarNode(0, LOAD, 0), ScalarNode(1, CONST, constant=1.0 / cap), ScalarNode(2, MUL, operands=(0, 1)),
        ScalarNode(3, TANH, operands=(2,)), ScalarNode(4, CONST, constant=cap), ScalarNode(5, MUL, operands=(3, 4)),
    ], 5


def residual_add_nodes():
    return [ScalarNode(0, LOAD, 0), ScalarNode(1, LOAD, 1), ScalarNode(2, ADD, operands=(0, 1))], 2


# ------------------------------------------------------------------ attention
@_reads_paged
def attention(q, k, v, position_offsets=None, window: int = 0, scale: float = -1.0, out=None):
    """AttentionKernelOp over dense K/V (src/core/TensorCalc.cpp:1167-1314)."""
    _require_gpu(q, k, v, position_offsets)
    out = torch.empty_like(q) if out is None else out
    call("sandy_hip_attention", desc(q), desc(k), desc(v), desc(position_offsets), int(window), float(scale),
         desc(out))
    return out


@dataclass
class PagedCache:
    """A KV page pool: pool tensor [num_pages, prefix, page_size, inner], or
    one half of a K/V pool [num_pages, 2, prefix, page_size, inner] (`half`
    0 = K, 1 = V: block b's K and V pages side by side, see interleaved)."""

    pool: torch.Tensor
    half: int = -1

    @staticmethod
    def interleaved(kv_pool: torch.Tensor):
        """(K cache, V cache) over one [num_pages, 2, prefix, page_size, inner] pool."""
        return PagedCache(kv_pool, 0), PagedCache(kv_pool, 1)

    def struct(self):
        p = self.pool
        s = _lib.SandyPagedCache()
        s.dtype = _lib._TORCH_TO_CODE[p.dtype]
        if self.half < 0:
            if p.dim() != 4 or not p.is_contiguous():
                raise SandyError(1, "paged pool must be a contiguous [pages, prefix, page_size, inner] tensor")
            s.pool = p.data_ptr()
            dims = p.shape
        else:
            if p.dim() != 5 or p.shape[1] != 2 or not p.is_contiguous():
                raise SandyError(1, "interleaved paged pool must be a contiguous [pages, 2, prefix, page_size, inner] tensor")
            s.pool = p[:, self.half].data_ptr()
            dims = [p.shape[0]] + list(p.shape[2:])
            s.page_stride = 2 * p.shape[2] * p.shape[3] * p.shape[4]
        s.page_size = dims[2]
        s.prefix = dims[1]
        s.inner = dims[3]
        s.num_pages = dims[0]
        return C.pointer(s)


def paged_attention(q, k_cache: PagedCache, v_cache: PagedCache, block_table, position_offsets,
                    window: int = 0, scale: float = -1.0, out=None):
    """Decode attention (Tq = 1) over paged K/V; block_table [B, max_blocks] int32."""
    _require_gpu(q, block_table, position_offsets, k_cache.pool, v_cache.pool)
    out = torch.empty_like(q) if out is None else out
    call("sandy_hip_paged_attention", desc(q), k_cache.struct(), v_cache.struct(), desc(block_table),
         desc(position_offsets), int(window), float(scale), desc(out))
    return out


# LayoutTransformKind (src/ir/KernelIR.h:268-274)
RESHAPE, TRANSPOSE, PERMUTE, SLICE, CONTIGUOUS = range(5)


def layout_transform(x: torch.Tensor, out: torch.Tensor | None = None, kind: int = CONTIGUOUS):
    """LayoutTransformKernelOp: the logical elements of the (strided) view x,
    in row-major order, into out (default: a contiguous tensor of x's shape)."""
    _require_gpu(x, out)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device) if out is None else out
    call("sandy_hip_layout_transform", desc(x), desc(out), int(kind))
    return out


class PagedView:
    """The reference's own paged tensor (CudaPagedTensor): a logical shape
    [B, Hkv, T, D] (or [Hkv, T, D]) whose grow dimension T lives in pages of
    [prefix, page_size, D] (prefix = B * Hkv or Hkv), one page list for the
    batch.  `pages` is a device uint64 tensor of page start addresses."""

    def __init__(self, pages: torch.Tensor, dims, page_size: int, dtype: torch.dtype):
        assert pages.is_cuda and pages.dtype in (torch.int64, torch.uint64) and pages.dim() == 1
        self.pages, self.dims, self.page_size, self.dtype = pages, list(dims), page_size, dtype

    def struct(self):
        s = _lib.SandyPagedView()
        s.pages = self.pages.data_ptr()
        s.dtype = _lib._TORCH_TO_CODE[self.dtype]
        s.rank = len(self.dims)
        for i, d in enumerate(self.dims):
            s.dims[i] = d
        s.page_size = self.page_size
        s.page_count = self.pages.numel()
        return C.pointer(s)


def attention_paged_view(q, k: PagedView, v: PagedView, position_offsets=None, window: int = 0,
                         scale: float = -1.0, out=None):
    """AttentionKernelOp over the reference's paged K/V (batched decode: rank 4,
    padded T, position_offsets [B])."""
    _require_gpu(q, k.pages, v.pages)
    out = torch.empty_like(q) if out is None else out
    call("sandy_hip_attention_paged_view", desc(q), k.struct(), v.struct(), desc(position_offsets), int(window),
         float(scale), desc(out))
    return out


def paged_attention_noalloc(q, k_cache: PagedCache, v_cache: PagedCache, block_table, position_offsets,
                            window: int = 0, scale: float = -1.0, out=None):
    """paged_attention through the entry point that allocates nothing (its
    split partials sit in the library's fixed per-GPU scratch); `out` must be
    given by callers that cannot allocate."""
    _require_gpu(q, block_table, position_offsets, k_cache.pool, v_cache.pool)
    out = torch.empty_like(q) if out is None else out
    call("sandy_hip_paged_attention_noalloc", desc(q), k_cache.struct(), v_cache.struct(), desc(block_table),
         desc(position_offsets), int(window), float(scale), desc(out))
    return out


# ------------------------------------------------------------------ MoE
def topk(x, k: int, axis: int = -1, index_dtype=torch.int64, values=None, indices=None):
    """TopKKernelOp: value descending, index ascending on ties (TensorCalc.cpp:1447-1518)."""
    _require_gpu(x)
    ax = axis % x.dim()
    shape = list(x.shape)
    shape[ax] = k
    values = torch.empty(shape, dtype=x.dtype, device=x.device) if values is None else values
    indices = torch.empty(shape, dtype=index_dtype, device=x.device) if indices is None else indices
    call("sandy_hip_topk", desc(x), int(k), int(axis), desc(values), desc(indices))
    return values, indices


def moe_gather(x, topk_ids, topk_weights, num_experts: int, index_dtype=torch.int64):
    """MoeGatherKernelOp (TensorCalc.cpp:1565-1667) -> packed_x, packed_weights, token_ids, expert_offsets."""
    _require_gpu(x, topk_ids, topk_weights)
    top_k = topk_ids.shape[-1]
    lead = list(x.shape[:-2])
    seq, hidden = x.shape[-2], x.shape[-1]
    rows = seq * top_k
    dev = x.device
    packed_x = torch.empty(lead + [rows, hidden], dtype=x.dtype, device=dev)
    packed_w = torch.empty(lead + [rows], dtype=topk_weights.dtype, device=dev)
    token_ids = torch.empty(lead + [rows], dtype=index_dtype, device=dev)
    offsets = torch.empty(lead + [num_experts + 1], dtype=index_dtype, device=dev)
    call("sandy_hip_moe_gather", desc(x), desc(topk_ids), desc(topk_weights), int(num_experts), int(top_k),
         desc(packed_x), desc(packed_w), desc(token_ids), desc(offsets))
    return packed_x, packed_w, token_ids, offsets


def moe_matmul(x, expert_offsets, weight, transpose_rhs: bool = True, out=None):
    """MoeMatMulKernelOp (TensorCalc.cpp:1669-1743)."""
    _require_gpu(x, expert_offsets, weight)
    m = weight.shape[1] if transpose_rhs else weight.shape[2]
    out = torch.empty(list(x.shape[:-1]) + [m], dtype=x.dtype, device=x.device) if out is None else out
    call("sandy_hip_moe_matmul", desc(x), desc(expert_offsets), desc(weight), int(bool(transpose_rhs)), desc(out))
    return out


def moe_scatter_sum(packed_out, packed_weights, token_ids, seq: int, out=None):
    """MoeScatterSumKernelOp (TensorCalc.cpp:1745-1811)."""
    _require_gpu(packed_out, packed_weights, token_ids)
    shape = list(packed_out.shape[:-2]) + [seq, packed_out.shape[-1]]
    out = torch.empty(shape, dtype=packed_out.dtype, device=packed_out.device) if out is None else out
    call("sandy_hip_moe_scatter_sum", desc(packed_out), desc(packed_weights), desc(token_ids), desc(out))
    return out


def _matmul_shape(lshape, rshape, transpose_lhs, transpose_rhs):
    """Output shape of matmul: batch dims broadcast right-aligned (equal, 1,
    or one a multiple of the other -- ShapeUtil.cpp:39-71)."""
    if len(lshape) < 2 or len(rshape) < 2:
        raise SandyError("matmul operands must have rank >= 2")
    lb, rb = list(lshape[:-2]), list(rshape[:-2])
    rank = max(len(lb), len(rb))
    lb = [1] * (rank - len(lb)) + lb
    rb = [1] * (rank - len(rb)) + rb
    batch = []
    for a, b in zip(lb, rb):
        if a == b or b == 1 or (a > b and a % b == 0):
            batch.append(a)
        elif a == 1 or (b > a and b % a == 0):
            batch.append(b)
        else:
            raise SandyError(f"cannot broadcast matmul batch shapes {list(lshape[:-2])} and {list(rshape[:-2])}")
    m = lshape[-1] if transpose_lhs else lshape[-2]
    n = rshape[-2] if transpose_rhs else rshape[-1]
    return batch + [m, n]


def matmul(lhs, rhs, transpose_lhs: bool = False, transpose_rhs: bool = False, out=None):
    """MatMulKernelOp (TensorCalc.cpp:804-919; CudaMatMulKernels.cu:221-292)."""
    _require_gpu(lhs, rhs)
    if out is None:
        shape = _matmul_shape(list(lhs.shape), list(rhs.shape), transpose_lhs, transpose_rhs)
        out = torch.empty(shape, dtype=lhs.dtype, device=lhs.device)
    call("sandy_hip_matmul", desc(lhs), desc(rhs), int(bool(transpose_lhs)), int(bool(transpose_rhs)), desc(out))
    return out


def interleave_glu_weight(gate_w, up_w):
    """[ffn, k] gate and up weights -> the [2 ffn, k] row-interleaved weight
    of matmul_glu (row 2i = gate_i, row 2i + 1 = up_i)."""
    return torch.stack([gate_w, up_w], dim=1).reshape(2 * gate_w.shape[0], gate_w.shape[1]).contiguous()


def pair_rope_weight(w_qkv, q_heads: int, kv_heads: int, head_dim: int, split_half: bool = True):
    """[(q_heads + 2 kv_heads) head_dim, k] fused q/k/v weight -> the row order
    of sandy_hip_device_matmul_qkv: within each q and k head, row i then row
    i + head_dim / 2 for i < head_dim / 2 (split-half RoPE pairs adjacent);
    v rows and interleaved-RoPE weights unchanged."""
    if not split_half:
        return w_qkv.contiguous()
    qk = (q_heads + kv_heads) * head_dim
    half = head_dim // 2
    heads = w_qkv[:qk].reshape(q_heads + kv_heads, 2, half, w_qkv.shape[1])
    paired = heads.permute(0, 2, 1, 3).reshape(qk, w_qkv.shape[1])
    return torch.cat([paired, w_qkv[qk:]], dim=0).contiguous()


def matmul_glu(x, w_interleaved, activation: str = "silu", out=None):
    """act(x @ gate^T) * (x @ up^T) in one launch; bit-identical to matmul then
    the silu_mul / gelu_mul group."""
    _require_gpu(x, w_interleaved)
    code = {"silu": 1, "gelu": 2}[activation]
    shape = list(x.shape[:-1]) + [w_interleaved.shape[0] // 2]
    out = torch.empty(shape, dtype=x.dtype, device=x.device) if out is None else out
    call("sandy_hip_matmul_glu", desc(x), desc(w_interleaved), code, desc(out))
    return out


def row_stats_buffer(rows: int, cols: int, device="cuda"):
    """Float64 [rows, ceil(cols / 16)] buffer for the row statistics the fused
    decode GEMMs pass along (sums of squares per 16-column group)."""
    return torch.empty(rows, (cols + 15) // 16, dtype=torch.float64, device=device)


def row_stats(buf):
    """SandyRowStats describing a row_stats_buffer (keep `buf` alive)."""
    return _lib.SandyRowStats(buf.data_ptr(), buf.shape[0], buf.shape[1])


def matmul_residual(x, weight, residual, stats=None, out=None):
    """bf16(residual + bf16(x @ weight^T)) in one launch (the residual add in
    the decode GEMM's epilogue); fills `stats` (row_stats_buffer of out's
    shape) with out's row sums of squares when given."""
    _require_gpu(x, weight, residual)
    out = torch.empty(list(x.shape[:-1]) + [weight.shape[0]], dtype=x.dtype, device=x.device) if out is None else out
    st = C.byref(row_stats(stats)) if stats is not None else None
    call("sandy_hip_matmul_residual", desc(x), desc(weight), desc(residual), desc(out), st)
    return out


def matmul_rms(x, stats, norm_weight, epsilon: float, weight, activation: str | None = None, out=None):
    """rms_norm(x, norm_weight) @ weight^T with the normalisation in the GEMM's
    operand registers, from x's row statistics; activation "silu"/"gelu"
    takes the row-interleaved gate/up weight as matmul_glu does."""
    _require_gpu(x, norm_weight, weight)
    code = {None: 0, "silu": 1, "gelu": 2}[activation]
    n = weight.shape[0] // (2 if code else 1)
    out = torch.empty(list(x.shape[:-1]) + [n], dtype=x.dtype, device=x.device) if out is None else out
    call("sandy_hip_matmul_rms", desc(x), C.byref(row_stats(stats)), desc(norm_weight), float(epsilon), desc(weight),
         code, desc(out))
    return out


def decode_linear(x, weight, bias=None, ln_weight=None, ln_bias=None, epsilon: float = 1e-5, activation: str | None = None,
                  residual=None, out=None):
    """[residual +] act(linear([layer_norm](x), weight, bias)) for 1-4 fp32
    rows in one launch (the GPT-2 decode chain); activation None or "gelu"."""
    _require_gpu(x, weight, bias, ln_weight, ln_bias, residual)
    shape = list(x.shape[:-1]) + [weight.shape[0]]
    out = torch.empty(shape, dtype=x.dtype, device=x.device) if out is None else out
    act = {None: 0, "gelu": 2}[activation]
    call("sandy_hip_decode_linear", desc(x), desc(ln_weight), desc(ln_bias), C.c_double(epsilon), desc(weight),
         desc(bias), C.c_int32(act), desc(residual), desc(out))
    return out


def linear(x, weight, bias, out=None):
    """LinearKernelOp (TensorCalc.cpp:722-773): bias + x @ weight^T."""
    _require_gpu(x, weight, bias)
    out = torch.empty(list(x.shape[:-1]) + [weight.shape[0]], dtype=x.dtype, device=x.device) if out is None else out
    call("sandy_hip_linear", desc(x), desc(weight), desc(bias), desc(out))
    return out
