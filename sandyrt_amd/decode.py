"""Greedy decode step of the TinyLlama model program for a batch of
sequences, built from the C-ABI entry points and run eagerly or as one
captured HIP graph.

The step is the reference's `eval_token` program (src/models/tinyllama/
eval_token.sandy.go and common.sandy.go:1-62): embedding, 22 blocks of
RMSNorm -> q/k/v projections -> RoPE (split-half, theta 1e4) -> paged
append -> paged decode attention -> o projection -> residual add ->
RMSNorm -> SiLU-gated MLP -> residual add, then the final RMSNorm, the
lm-head and greedy token selection (src/server/Sampler.cpp:69-79).

Everything stays on the device between steps: the position of the new token
is the device-side length of the layer-0 K cache (read inside the step),
the appends advance the lengths, and the greedy token id is written where the
next step's embedding reads it -- so a captured step replays with no host
work and no host synchronisation (the reference syncs and copies per row,
src/device/cuda/CudaPagedTensor.cpp:649-740, Engine.cpp:548-596).

Layout choices (same arithmetic as the reference program):
  * RoPE of q and k and the two paged appends of each block run as one
    launch (sandy_hip_device_decode_qkv); fused_qkv=False issues the
    reference program's separate rope / append ops instead.
  * the gate/up GEMM applies the SiLU gate in its epilogue
    (sandy_hip_matmul_glu, gate/up weight rows interleaved once at
    construction); fused_glu=False runs the GEMM and the SiLU group.
  * q/k/v weights are concatenated into one [q + k + v, hidden] matrix and
    gate/up into one [2 * ffn, hidden] matrix, so each is one GEMM; the
    q/k/v and gate/up outputs are contiguous views of those GEMM outputs.
  * fused_norm (default): the residual adds run in the o and down GEMMs'
    epilogues (sandy_hip_matmul_residual), which also leave the new residual
    stream's row sums of squares, and the RMSNorms run in the q/k/v, gate/up
    and lm-head GEMMs' prologues from those sums (sandy_hip_matmul_rms): no
    norm launch after block 0's input norm, bit-identical to the unfused
    program.  With it, fused_rope_gemm (default, up to 64 sequences) also
    moves the RoPE of q and k and both paged appends into the q/k/v GEMM's
    epilogue (sandy_hip_device_matmul_qkv, q/k weight rows pair-ordered once
    at construction).  fused_norm=False runs each residual add with the next RMSNorm
    (sandy_hip_add_rms_norm) between plain GEMMs.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib, ops
from ._lib import BF16, desc
from .device import HipDevice


@dataclass
class DecodeConfig:
    layers: int = 22
    hidden: int = 2048
    heads: int = 32
    kv_heads: int = 4
    head_dim: int = 64
    ffn: int = 5632
    vocab: int = 32000
    page_size: int = 32
    eps: float = 1e-5
    theta: float = 10000.0
    max_context: int = 4096


def random_weights(cfg: DecodeConfig, seed: int = 0, std: float = 0.02, device="cuda") -> dict:
    """Random-init bf16 weights of the TinyLlama architecture (no checkpoint
    is available offline).  Norm weights are 1 + N(0, std)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def n(*shape, mean=0.0):
        return (torch.randn(*shape, generator=g, device=device) * std + mean).to(torch.bfloat16)

    qkv = (cfg.heads + 2 * cfg.kv_heads) * cfg.head_dim
    w = {"embed": n(cfg.vocab, cfg.hidden, mean=0.0) * 50, "norm": n(cfg.hidden, mean=1.0),
         "lm_head": n(cfg.vocab, cfg.hidden)}
    for layer in range(cfg.layers):
        w[f"{layer}.in_norm"] = n(cfg.hidden, mean=1.0)
        w[f"{layer}.qkv"] = n(qkv, cfg.hidden)
        w[f"{layer}.o"] = n(cfg.hidden, cfg.heads * cfg.head_dim)
        w[f"{layer}.post_norm"] = n(cfg.hidden, mean=1.0)
        w[f"{layer}.gate_up"] = n(2 * cfg.ffn, cfg.hidden)
        w[f"{layer}.down"] = n(cfg.hidden, cfg.ffn)
    return w


def weights_from_safetensors(st, cfg: DecodeConfig) -> dict:
    """Decoder weights from an uploaded checkpoint (sandyrt_amd.weights.
    SafeTensors) under the program's scoped names, weight_scope "model" ->
    "layers.{i}" -> "self_attn" / "mlp" (src/models/tinyllama/
    eval_token.sandy.go:4-13, common.sandy.go:1-62); the lm-head is also
    found at the top level, as Hugging Face checkpoints store it.  q/k/v and
    gate/up are concatenated on the device once, here."""
    def get(*names):
        for n in names:
            t = st.get_tensor(n)
            if t is not None:
                return t
        raise KeyError(f"checkpoint has none of {names}")

    w = {"embed": get("model.embed_tokens.weight"), "norm": get("model.norm.weight"),
         "lm_head": get("model.lm_head.weight", "lm_head.weight")}
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        w[f"{i}.in_norm"] = get(p + "input_layernorm.weight")
        w[f"{i}.post_norm"] = get(p + "post_attention_layernorm.weight")
        w[f"{i}.qkv"] = torch.cat([get(p + f"self_attn.{n}_proj.weight") for n in "qkv"], 0).contiguous()
        w[f"{i}.o"] = get(p + "self_attn.o_proj.weight")
        w[f"{i}.gate_up"] = torch.cat([get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight")], 0).contiguous()
        w[f"{i}.down"] = get(p + "mlp.down_proj.weight")
    return w


class _Call:
    """One C-ABI kernel entry point with its arguments bound once."""

    def __init__(self, name, *args, stream):
        self.fn = getattr(_lib.lib(), name)
        self.args = args + (C.c_void_p(stream),)
        self.buf = C.create_string_buffer(256)
        self.name = name

    def __call__(self):
        if self.fn(*self.args, self.buf, C.c_size_t(256)):
            raise _lib.SandyError(1, f"{self.name}: {self.buf.value.decode()}")


class _DevCall:
    """One device-runtime entry point (runs on the device's stream)."""

    def __init__(self, name, *args):
        self.fn = getattr(_lib.lib(), name)
        self.args = args
        self.buf = C.create_string_buffer(256)
        self.name = name

    def __call__(self):
        if self.fn(*self.args, self.buf, C.c_size_t(256)):
            raise _lib.SandyError(1, f"{self.name}: {self.buf.value.decode()}")


class TinyLlamaDecoder:
    """Owns the paged K/V caches of `batch` sequences and the step's buffers;
    the step program is a fixed list of bound calls on the device's stream.
    Sequence b owns row b of every layer's block table (its pool slot), so
    the attention reads the pools' tables directly."""

    def __init__(self, dev: HipDevice, cfg: DecodeConfig, weights: dict, batch: int = 1, fused_qkv: bool = True,
                 fused_glu: bool = True, fused_norm: bool = True, fused_rope_gemm: bool = True):
        self.dev, self.cfg, self.w, self.batch = dev, cfg, weights, batch
        self.fused_qkv, self.fused_glu, self.fused_norm = fused_qkv, fused_glu, fused_norm
        # the RoPE and paged appends in the q/k/v GEMM's epilogue (fused_norm
        # programs of at most 64 sequences): q/k rows pair-ordered once here
        self.fused_rope_gemm = fused_rope_gemm and fused_norm and fused_qkv and batch <= 64
        self.w_qkv = {}
        if self.fused_rope_gemm:
            for layer in range(cfg.layers):
                self.w_qkv[layer] = ops.pair_rope_weight(weights[f"{layer}.qkv"], cfg.heads, cfg.kv_heads,
                                                         cfg.head_dim)
        # row-interleaved gate/up weights for the gated GEMM epilogue (the
        # caller's weight dict is left as it is)
        self.w_glu = {}
        if fused_glu:
            for layer in range(cfg.layers):
                gu = weights[f"{layer}.gate_up"]
                self.w_glu[layer] = ops.interleave_glu_weight(gu[:cfg.ffn], gu[cfg.ffn:])
        c, B = cfg, batch
        bf = torch.bfloat16
        pages = (c.max_context + c.page_size - 1) // c.page_size
        self.k_pools, self.v_pools, self.k_seq, self.v_seq = [], [], [], []
        for _ in range(c.layers):
            for pools, seqs in ((self.k_pools, self.k_seq), (self.v_pools, self.v_seq)):
                p = dev.create_paged_pool([1, c.kv_heads, -1, c.head_dim], BF16, 2, c.page_size,
                                          initial_pages=B * pages, max_pages=B * pages, max_tensors=B,
                                          max_blocks=pages)
                ids = []
                for b in range(B):
                    t = dev.alloc_paged(p)
                    dev.reserve_paged(t, pages)
                    if dev.paged_meta(t).slot != b:
                        raise RuntimeError("paged pool slots are not allocated in order")
                    ids.append(t)
                pools.append(p)
                seqs.append(ids)
        dv = "cuda"
        qkv = (c.heads + 2 * c.kv_heads) * c.head_dim
        self.token = torch.zeros(B, 1, dtype=torch.int64, device=dv)  # greedy output -> next input
        self.pos = torch.zeros(B, dtype=torch.int64, device=dv)
        self.x0 = torch.empty(B, 1, c.hidden, dtype=bf, device=dv)
        self.res = [torch.empty(B, c.hidden, dtype=bf, device=dv) for _ in range(2)]
        self.h = torch.empty(B, c.hidden, dtype=bf, device=dv)
        self.qkv = torch.empty(B, qkv, dtype=bf, device=dv)
        self.qr = torch.empty(B, c.heads, 1, c.head_dim, dtype=bf, device=dv)
        self.kr = torch.empty(B, c.kv_heads, 1, c.head_dim, dtype=bf, device=dv)
        self.vr = torch.empty(B, c.kv_heads, 1, c.head_dim, dtype=bf, device=dv)
        self.ctx = torch.empty(B, c.heads, 1, c.head_dim, dtype=bf, device=dv)
        self.o = torch.empty(B, c.hidden, dtype=bf, device=dv)
        self.gu = torch.empty(B, 2 * c.ffn, dtype=bf, device=dv)
        self.act = torch.empty(B, c.ffn, dtype=bf, device=dv)
        self.d = torch.empty(B, c.hidden, dtype=bf, device=dv)
        self.logits = torch.empty(B, c.vocab, dtype=bf, device=dv)
        self.top_v = torch.empty(B, 1, dtype=bf, device=dv)
        # row statistics of the two residual-stream buffers (fused_norm)
        self.stats = [ops.row_stats_buffer(B, c.hidden) for _ in range(2)]
        self._keep = []
        self.program = self._build()
        self.graph = None

    # ------------------------------------------------------------------ program
    def _d(self, t):
        p = desc(t)
        self._keep.append(p)
        return p

    def _build(self):
        c, w, dev, s, B = self.cfg, self.w, self.dev, self.dev.stream, self.batch
        d = self._d
        prog = []
        hq, hk, D = c.heads * c.head_dim, c.kv_heads * c.head_dim, c.head_dim

        def per_position(t, heads):
            # [B, heads, D] rows of the qkv output (or of a [B, heads, 1, D]
            # buffer) seen as [1, heads, B, D]: the sequence axis is the RoPE
            # sequence, so position_ids[b] rotates every head of sequence b
            return t.reshape(B, heads, D).permute(1, 0, 2).unsqueeze(0)

        q_in = per_position(self.qkv[:, :hq], c.heads)
        k_in = per_position(self.qkv[:, hq:hq + hk], c.kv_heads)
        v_view = self.qkv[:, hq + hk:].view(B, c.kv_heads, 1, D)
        q_out, k_out = per_position(self.qr, c.heads), per_position(self.kr, c.kv_heads)
        gate, up = self.gu[:, :c.ffn], self.gu[:, c.ffn:]
        h2d, ctx2d = self.h, self.ctx.view(B, hq)
        ids0 = (C.c_uint32 * B)(*self.k_seq[0])
        self._keep.append(ids0)
        prog.append(_DevCall("sandy_hip_device_paged_lengths", dev.handle, C.c_uint32(self.k_pools[0]), ids0,
                             C.c_int32(B), d(self.pos)))
        prog.append(_Call("sandy_hip_gather", d(self.token), d(w["embed"]), d(self.x0), stream=s))
        silu, sres = ops.silu_mul_nodes()
        nodes = ops._nodes(silu)
        arr = (_lib.SandyTensor * 2)(d(gate).contents, d(up).contents)
        bc = (C.c_int32 * 2)(0, 0)
        copy_nodes = ops._nodes([ops.ScalarNode(0, ops.LOAD, 0)])
        v_arr = (_lib.SandyTensor * 1)(d(v_view).contents)
        self._keep += [nodes, arr, bc, copy_nodes, v_arr]
        x0 = self.x0.view(B, c.hidden)
        # residual stream: block input x_l in buffer A (x0 for block 0), the
        # residual after attention in buffer B
        res_a, res_b = self.res
        st_a, st_b = (ops.row_stats(t) for t in self.stats)
        self._keep += [st_a, st_b]
        if self.fused_norm:
            self._build_fused_blocks(prog, x0, nodes, sres, silu, arr, bc, st_a, st_b)
            return prog
        for layer in range(c.layers):
            if layer == 0:
                prog.append(_Call("sandy_hip_norm", C.c_int32(0), d(x0), d(w["0.in_norm"]), None, C.c_double(c.eps),
                                  d(h2d), stream=s))
                x_in = x0
            else:
                # x_l = previous residual + previous MLP output, then this block's input norm
                prog.append(_Call("sandy_hip_add_rms_norm", d(self.d), d(res_b), d(w[f"{layer}.in_norm"]),
                                  C.c_double(c.eps), d(res_a), d(h2d), stream=s))
                x_in = res_a
            prog.append(_Call("sandy_hip_matmul", d(h2d), d(w[f"{layer}.qkv"]), C.c_int32(0), C.c_int32(1),
                              d(self.qkv), stream=s))
            kid = (C.c_uint32 * B)(*self.k_seq[layer])
            vid = (C.c_uint32 * B)(*self.v_seq[layer])
            self._keep += [kid, vid]
            if self.fused_qkv:
                # RoPE q and k, append k and v: one launch
                prog.append(_DevCall("sandy_hip_device_decode_qkv", dev.handle, C.c_uint32(self.k_pools[layer]), kid,
                                     C.c_uint32(self.v_pools[layer]), vid, C.c_int32(B), d(self.qkv),
                                     C.c_int32(c.heads), d(self.pos), C.c_double(c.theta), C.c_int32(1),
                                     d(self.qr)))
            else:  # the reference program's separate ops
                prog.append(_Call("sandy_hip_rope", d(q_in), d(self.pos), C.c_double(c.theta), C.c_int64(-1),
                                  C.c_int32(1), d(q_out), stream=s))
                prog.append(_Call("sandy_hip_rope", d(k_in), d(self.pos), C.c_double(c.theta), C.c_int64(-1),
                                  C.c_int32(1), d(k_out), stream=s))
                if B == 1:
                    v_rows = v_view  # one sequence: the v slice is already contiguous
                else:  # contiguous [B, kv_heads, 1, D] rows for the batched append
                    prog.append(_Call("sandy_hip_elementwise", copy_nodes, C.c_int32(1), C.c_uint32(0), v_arr, None,
                                      C.c_int32(1), d(self.vr), stream=s))
                    v_rows = self.vr
                prog.append(_DevCall("sandy_hip_device_paged_append_step", dev.handle,
                                     C.c_uint32(self.k_pools[layer]), kid, C.c_int32(B), d(self.kr)))
                prog.append(_DevCall("sandy_hip_device_paged_append_step", dev.handle,
                                     C.c_uint32(self.v_pools[layer]), vid, C.c_int32(B), d(v_rows)))
            kc, table, _ = dev.paged_views(self.k_pools[layer])
            vc, _, _ = dev.paged_views(self.v_pools[layer])
            table.contents.dims[0] = B  # rows 0..B-1: the sequences' slots
            self._keep += [kc, vc, table]
            prog.append(_Call("sandy_hip_paged_attention", d(self.qr), kc, vc, table, d(self.pos), C.c_int64(0),
                              C.c_double(1.0 / (D ** 0.5)), d(self.ctx), stream=s))
            prog.append(_Call("sandy_hip_matmul", d(ctx2d), d(w[f"{layer}.o"]), C.c_int32(0), C.c_int32(1),
                              d(self.o), stream=s))
            prog.append(_Call("sandy_hip_add_rms_norm", d(self.o), d(x_in), d(w[f"{layer}.post_norm"]),
                              C.c_double(c.eps), d(res_b), d(h2d), stream=s))
            if self.fused_glu:  # gate/up GEMM with the SiLU gate in its epilogue: one launch
                prog.append(_Call("sandy_hip_matmul_glu", d(h2d), d(self.w_glu[layer]), C.c_int32(1), d(self.act),
                                  stream=s))
            else:
                prog.append(_Call("sandy_hip_matmul", d(h2d), d(w[f"{layer}.gate_up"]), C.c_int32(0), C.c_int32(1),
                                  d(self.gu), stream=s))
                prog.append(_Call("sandy_hip_elementwise", nodes, C.c_int32(len(silu)), C.c_uint32(sres), arr, bc,
                                  C.c_int32(2), d(self.act), stream=s))
            prog.append(_Call("sandy_hip_matmul", d(self.act), d(w[f"{layer}.down"]), C.c_int32(0), C.c_int32(1),
                              d(self.d), stream=s))
        prog.append(_Call("sandy_hip_add_rms_norm", d(self.d), d(res_b), d(w["norm"]), C.c_double(c.eps), d(res_a),
                          d(h2d), stream=s))
        prog.append(_Call("sandy_hip_matmul", d(h2d), d(w["lm_head"]), C.c_int32(0), C.c_int32(1), d(self.logits),
                          stream=s))
        prog.append(_Call("sandy_hip_topk", d(self.logits), C.c_int64(1), C.c_int64(-1), d(self.top_v),
                          d(self.token), stream=s))
        return prog

    def _attention_calls(self, prog, layer):
        """q/k/v RoPE, the paged appends and the paged decode attention of one
        block, from self.qkv to self.ctx (the fused q/k/v launch)."""
        c, dev, s, B, d = self.cfg, self.dev, self.dev.stream, self.batch, self._d
        kid = (C.c_uint32 * B)(*self.k_seq[layer])
        vid = (C.c_uint32 * B)(*self.v_seq[layer])
        self._keep += [kid, vid]
        prog.append(_DevCall("sandy_hip_device_decode_qkv", dev.handle, C.c_uint32(self.k_pools[layer]), kid,
                             C.c_uint32(self.v_pools[layer]), vid, C.c_int32(B), d(self.qkv), C.c_int32(c.heads),
                             d(self.pos), C.c_double(c.theta), C.c_int32(1), d(self.qr)))
        self._paged_attention_call(prog, layer)

    def _paged_attention_call(self, prog, layer):
        """Paged decode attention of one block, self.qr -> self.ctx."""
        c, dev, s, B, d = self.cfg, self.dev, self.dev.stream, self.batch, self._d
        kc, table, _ = dev.paged_views(self.k_pools[layer])
        vc, _, _ = dev.paged_views(self.v_pools[layer])
        table.contents.dims[0] = B  # rows 0..B-1: the sequences' slots
        self._keep += [kc, vc, table]
        prog.append(_Call("sandy_hip_paged_attention", d(self.qr), kc, vc, table, d(self.pos), C.c_int64(0),
                          C.c_double(1.0 / (c.head_dim ** 0.5)), d(self.ctx), stream=s))

    def _build_fused_blocks(self, prog, x0, nodes, sres, silu, arr, bc, st_a, st_b):
        """The blocks with the residual adds in the o / down GEMM epilogues and
        the RMSNorms in the q/k/v, gate/up and lm-head GEMM prologues."""
        c, w, s, B, d = self.cfg, self.w, self.dev.stream, self.batch, self._d
        res_a, res_b = self.res
        ctx2d = self.ctx.view(B, c.heads * c.head_dim)
        for layer in range(c.layers):
            if layer == 0:  # the embedding has no statistics: one norm launch
                prog.append(_Call("sandy_hip_norm", C.c_int32(0), d(x0), d(w["0.in_norm"]), None, C.c_double(c.eps),
                                  d(self.h), stream=s))
                x_in = x0
            else:
                x_in = res_a  # x_l with its statistics
            if not self.fused_qkv:
                raise ValueError("fused_norm takes the fused q/k/v launch")
            if self.fused_rope_gemm:
                # q/k/v GEMM (RMSNorm prologue past block 0) with RoPE and both appends in its epilogue
                kid = (C.c_uint32 * B)(*self.k_seq[layer])
                vid = (C.c_uint32 * B)(*self.v_seq[layer])
                self._keep += [kid, vid]
                lhs, st, nw = (d(self.h), None, None) if layer == 0 else (d(res_a), C.byref(st_a),
                                                                           d(w[f"{layer}.in_norm"]))
                prog.append(_DevCall("sandy_hip_device_matmul_qkv", self.dev.handle, lhs, st, nw, C.c_double(c.eps),
                                     d(self.w_qkv[layer]), C.c_uint32(self.k_pools[layer]), kid,
                                     C.c_uint32(self.v_pools[layer]), vid, C.c_int32(B), C.c_int32(c.heads),
                                     d(self.pos), C.c_double(c.theta), C.c_int32(1), d(self.qr)))
                self._paged_attention_call(prog, layer)
            else:
                if layer == 0:
                    prog.append(_Call("sandy_hip_matmul", d(self.h), d(w["0.qkv"]), C.c_int32(0), C.c_int32(1),
                                      d(self.qkv), stream=s))
                else:
                    prog.append(_Call("sandy_hip_matmul_rms", d(res_a), C.byref(st_a), d(w[f"{layer}.in_norm"]),
                                      C.c_double(c.eps), d(w[f"{layer}.qkv"]), C.c_int32(0), d(self.qkv), stream=s))
                self._attention_calls(prog, layer)
            # residual after attention: res_b = x_l + o-projection, with statistics
            prog.append(_Call("sandy_hip_matmul_residual", d(ctx2d), d(w[f"{layer}.o"]), d(x_in), d(res_b),
                              C.byref(st_b), stream=s))
            if self.fused_glu:
                prog.append(_Call("sandy_hip_matmul_rms", d(res_b), C.byref(st_b), d(w[f"{layer}.post_norm"]),
                                  C.c_double(c.eps), d(self.w_glu[layer]), C.c_int32(1), d(self.act), stream=s))
            else:
                prog.append(_Call("sandy_hip_matmul_rms", d(res_b), C.byref(st_b), d(w[f"{layer}.post_norm"]),
                                  C.c_double(c.eps), d(w[f"{layer}.gate_up"]), C.c_int32(0), d(self.gu), stream=s))
                prog.append(_Call("sandy_hip_elementwise", nodes, C.c_int32(len(silu)), C.c_uint32(sres), arr, bc,
                                  C.c_int32(2), d(self.act), stream=s))
            # x_{l+1} = res_b + down-projection, into res_a with statistics
            prog.append(_Call("sandy_hip_matmul_residual", d(self.act), d(w[f"{layer}.down"]), d(res_b), d(res_a),
                              C.byref(st_a), stream=s))
        prog.append(_Call("sandy_hip_matmul_rms", d(res_a), C.byref(st_a), d(w["norm"]), C.c_double(c.eps),
                          d(w["lm_head"]), C.c_int32(0), d(self.logits), stream=s))
        prog.append(_Call("sandy_hip_topk", d(self.logits), C.c_int64(1), C.c_int64(-1), d(self.top_v),
                          d(self.token), stream=s))

    # ------------------------------------------------------------------ running
    def prefill_cache(self, k_rows: list, v_rows: list, seq: int = 0):
        """Append context K/V ([1, kv_heads, n, head_dim] per layer) of
        sequence `seq` as if earlier tokens had been decoded."""
        torch.cuda.synchronize()
        for layer in range(self.cfg.layers):
            self.dev.append_paged(self.k_seq[layer][seq], k_rows[layer])
            self.dev.append_paged(self.v_seq[layer][seq], v_rows[layer])
        self.dev.synchronize()

    def set_token(self, token):
        """Next input token: one id for every sequence, or one per sequence."""
        if isinstance(token, int):
            self.token.fill_(token)
        else:
            self.token.copy_(torch.as_tensor(token, dtype=torch.int64).view(self.batch, 1))
        torch.cuda.synchronize()

    def step(self):
        """One decode step, launched eagerly."""
        for call in self.program:
            call()

    def capture(self):
        """Capture one step as a HIP graph (run a warm step first: workspaces
        and generated kernels must exist before capture)."""
        self.dev.graph_begin()
        try:
            self.step()
        finally:
            self.graph = self.dev.graph_end()
        return self.graph

    def replay(self):
        self.dev.graph_launch(self.graph)

    def length(self, seq: int = 0) -> int:
        self.dev.paged_sync(self.k_pools[0])
        return self.dev.paged_meta(self.k_seq[0][seq]).grow_length

    def close(self):
        if self.graph is not None:
            self.dev.graph_destroy(self.graph)
            self.graph = None
