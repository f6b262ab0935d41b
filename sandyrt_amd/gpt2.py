"""Greedy decoding of the reference's GPT-2 small program on the C-ABI ops.

The program is src/models/gpt2_small.sandy.go: token + learned position
embedding, 12 blocks of LayerNorm -> q/k/v linear -> causal attention ->
c_proj linear -> residual add -> LayerNorm -> c_fc linear -> GELU -> c_proj
linear -> residual add, final LayerNorm and logits = x wte^T.  The reference
fixes it to 16 tokens and recomputes the whole window per token
(scripts/run_gpt2.py:333-335); here the same ops run with a dense fp32 K/V
cache: the prompt is one forward pass over all its tokens, then each greedy
step runs one token whose keys and values are appended to the cache.  Every
op before the attention is row-independent and the attention of the last
row sees the same keys, so the last row's logits are those of the full
recompute.

fp32 throughout, like the reference CPU path (linear, LayerNorm, embedding,
attention, the GELU group and the lm-head matmul).  The single-token steps
read their K/V through the device runtime's paged pools (fp32 rows) with the
general attention kernel, the same arithmetic as the prompt's dense
attention.  Greedy selection is
sandy_hip_topk with k = 1 (ties -> lowest id, src/server/Sampler.cpp:69-79).
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import ctypes as C

import numpy as np
import torch

from . import _lib, ops
from ._lib import F32, desc
from .decode import _Call, _DevCall
from .device import HipDevice


@dataclass
class GPT2Config:
    layers: int = 12
    hidden: int = 768
    heads: int = 12
    head_dim: int = 64
    ffn: int = 3072
    vocab: int = 50257
    positions: int = 1024
    eps: float = 1e-5


def weight_names(cfg: GPT2Config):
    """(name, shape) in generation order; names follow the program's weight
    scopes (h.{i}.attn.q_proj.weight, ...), linear weights are [out, in]."""
    out = [("wte.weight", (cfg.vocab, cfg.hidden)), ("wpe.weight", (cfg.positions, cfg.hidden))]
    H, F = cfg.hidden, cfg.ffn
    for i in range(cfg.layers):
        p = f"h.{i}."
        out += [(p + "ln_1.weight", (H,)), (p + "ln_1.bias", (H,))]
        for n in ("q_proj", "k_proj", "v_proj", "c_proj"):
            out += [(p + f"attn.{n}.weight", (H, H)), (p + f"attn.{n}.bias", (H,))]
        out += [(p + "ln_2.weight", (H,)), (p + "ln_2.bias", (H,)),
                (p + "mlp.c_fc.weight", (F, H)), (p + "mlp.c_fc.bias", (F,)),
                (p + "mlp.c_proj.weight", (H, F)), (p + "mlp.c_proj.bias", (H,))]
    out += [("ln_f.weight", (cfg.hidden,)), ("ln_f.bias", (cfg.hidden,))]
    return out


def random_weights(cfg: GPT2Config, seed: int = 0) -> dict:
    """Host fp32 weights: every matrix, embedding and bias N(0, 0.02) from
    numpy's default_rng(seed) in weight_names order; LayerNorm gains 1 and
    shifts 0 (GPT-2's initialisation)."""
    rng = np.random.default_rng(seed)
    w = {}
    for name, shape in weight_names(cfg):
        if ".ln_" in name or name.startswith("ln_f"):
            w[name] = (np.ones if name.endswith("weight") else np.zeros)(shape, np.float32)
        else:
            w[name] = (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    return w


def prompt_ids(cfg: GPT2Config, length: int = 64, seed: int = 0) -> list:
    """The config-1 prompt: `length` ids uniform over the vocabulary."""
    return [int(t) for t in np.random.default_rng([seed, 1]).integers(0, cfg.vocab, length)]


class GPT2Runner:
    """Weights resident on the GPU; per layer one paged K and one paged V
    pool (fp32 rows, block 16) of one sequence in the device runtime.  The
    prompt is one eager pass over all its tokens; each later token runs a
    fixed program of bound C-ABI calls (position from the device-side cache
    length, appends on the device, greedy token written where the next step's
    embedding reads it), eagerly or as one captured HIP graph."""

    def __init__(self, cfg: GPT2Config, host_weights: dict, max_seq: int = 128, dev: HipDevice | None = None,
                 page_size: int = 16):
        self.cfg, self.max_seq = cfg, max_seq
        self.dev = dev if dev is not None else HipDevice(0)
        self._own_dev = dev is None
        self.w = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in host_weights.items()}
        # the decode step's q/k/v projection as one [3 hidden, hidden] linear
        for i in range(cfg.layers):
            p = f"h.{i}.attn."
            for part in ("weight", "bias"):
                self.w[p + "qkv." + part] = torch.cat([self.w[p + n + "_proj." + part] for n in ("q", "k", "v")]).contiguous()
        pages = (max_seq + page_size - 1) // page_size
        self.k_pools, self.v_pools, self.k_seq, self.v_seq = [], [], [], []
        for _ in range(cfg.layers):
            for pools, seqs in ((self.k_pools, self.k_seq), (self.v_pools, self.v_seq)):
                pool = self.dev.create_paged_pool([1, cfg.heads, -1, cfg.head_dim], F32, 2, page_size,
                                                  initial_pages=pages, max_pages=pages, max_tensors=1,
                                                  max_blocks=pages)
                t = self.dev.alloc_paged(pool)
                self.dev.reserve_paged(t, pages)
                pools.append(pool)
                seqs.append(t)
        self.length = 0
        self.gelu, self.gelu_res = ops.gelu_nodes()
        self.add, self.add_res = ops.residual_add_nodes()
        self.copy = [ops.ScalarNode(0, ops.LOAD, 0)]
        # single-token step buffers
        dv, H, f32 = "cuda", cfg.hidden, torch.float32
        self.token = torch.zeros(1, 1, dtype=torch.int64, device=dv)
        self.pos = torch.zeros(1, dtype=torch.int64, device=dv)
        self.bufs = {n: torch.empty(1, H, dtype=f32, device=dv) for n in ("te", "pe", "x", "x2", "h", "ctx", "o", "m")}
        self.bufs["qkv"] = torch.empty(1, 3 * H, dtype=f32, device=dv)
        self.bufs["f"] = torch.empty(1, cfg.ffn, dtype=f32, device=dv)
        self.bufs["g"] = torch.empty(1, cfg.ffn, dtype=f32, device=dv)
        self.logits = torch.empty(1, cfg.vocab, dtype=f32, device=dv)
        self.top_v = torch.empty(1, 1, dtype=f32, device=dv)
        self._keep = []
        self.program = self._build_step()
        self.graph = None
        torch.cuda.synchronize()  # weights and buffers ready before the device stream uses them

    def _heads(self, t, T):
        """[T, hidden] rows as [1, heads, T, D] (a strided view)."""
        return t.view(T, self.cfg.heads, self.cfg.head_dim).permute(1, 0, 2).unsqueeze(0)

    # ------------------------------------------------------------------ prompt
    def _prompt(self, ids) -> torch.Tensor:
        """All prompt tokens in one pass (positions 0 .. T-1), ordered on the
        device stream with the appends and the later steps."""
        with torch.cuda.stream(self.dev.torch_stream()):
            logits = self._prompt_ops(ids)
        self.dev.synchronize()  # callers read the logits on other streams
        return logits

    def _prompt_ops(self, ids) -> torch.Tensor:
        """Causal dense attention over the prompt's own K/V, which are then
        appended to the pools as one chunk per layer."""
        c, w = self.cfg, self.w
        T = len(ids)
        if T > self.max_seq:
            raise ValueError("GPT-2 cache is full")
        dev = w["wte.weight"].device
        ids_t = torch.tensor([ids], dtype=torch.int64, device=dev)
        pos_t = torch.arange(0, T, dtype=torch.int64, device=dev).view(1, T)
        x = ops.elementwise(self.add, self.add_res, [ops.embedding(ids_t, w["wte.weight"]),
                                                     ops.embedding(pos_t, w["wpe.weight"])]).view(T, c.hidden)
        offsets = torch.zeros(1, dtype=torch.int64, device=dev)
        for i in range(c.layers):
            p = f"h.{i}."
            h = ops.layer_norm(x, w[p + "ln_1.weight"], w[p + "ln_1.bias"], c.eps)
            q = ops.linear(h, w[p + "attn.q_proj.weight"], w[p + "attn.q_proj.bias"])
            k = ops.linear(h, w[p + "attn.k_proj.weight"], w[p + "attn.k_proj.bias"])
            v = ops.linear(h, w[p + "attn.v_proj.weight"], w[p + "attn.v_proj.bias"])
            kh = ops.elementwise(self.copy, 0, [self._heads(k, T)])  # contiguous [1, heads, T, D]
            vh = ops.elementwise(self.copy, 0, [self._heads(v, T)])
            ctx = torch.empty(T, c.hidden, dtype=torch.float32, device=dev)
            ops.attention(self._heads(q, T), kh, vh, offsets, 0, -1.0, out=self._heads(ctx, T))
            self.dev.append_paged(self.k_seq[i], kh)
            self.dev.append_paged(self.v_seq[i], vh)
            o = ops.linear(ctx, w[p + "attn.c_proj.weight"], w[p + "attn.c_proj.bias"])
            x = ops.elementwise(self.add, self.add_res, [x, o])
            h = ops.layer_norm(x, w[p + "ln_2.weight"], w[p + "ln_2.bias"], c.eps)
            f = ops.linear(h, w[p + "mlp.c_fc.weight"], w[p + "mlp.c_fc.bias"])
            f = ops.elementwise(self.gelu, self.gelu_res, [f])
            m = ops.linear(f, w[p + "mlp.c_proj.weight"], w[p + "mlp.c_proj.bias"])
            x = ops.elementwise(self.add, self.add_res, [x, m])
        h = ops.layer_norm(x[T - 1:T], w["ln_f.weight"], w["ln_f.bias"], c.eps)
        self.length = T
        return ops.matmul(h, w["wte.weight"], transpose_rhs=True)

    # ------------------------------------------------------------------ one token
    def _d(self, t):
        p = desc(t)
        self._keep.append(p)
        return p

    def _build_step(self):
        c, w, dev, s, b = self.cfg, self.w, self.dev, self.dev.stream, self.bufs
        d = self._d
        prog = []

        def ew(nodes, res, ins, out):
            arr = (_lib.SandyTensor * len(ins))(*[d(t).contents for t in ins])
            bc = (C.c_int32 * len(ins))(*([0] * len(ins)))
            cn = ops._nodes(nodes)
            self._keep += [arr, bc, cn]
            return _Call("sandy_hip_elementwise", cn, C.c_int32(len(nodes)), C.c_uint32(res), arr, bc,
                         C.c_int32(len(ins)), d(out), stream=s)

        def linear(x, name, out, ln=None, gelu=False, residual=None):
            """[residual +] gelu?(linear(layer_norm?(x))) in one launch"""
            lw, lb = (d(w[ln + ".weight"]), d(w[ln + ".bias"])) if ln else (None, None)
            bias = d(w[name + ".bias"]) if name + ".bias" in w else None
            return _Call("sandy_hip_decode_linear", d(x), lw, lb, C.c_double(c.eps), d(w[name + ".weight"]), bias,
                         C.c_int32(2 if gelu else 0), d(residual) if residual is not None else None, d(out),
                         stream=s)

        head4 = lambda t: t.view(1, c.heads, 1, c.head_dim)  # noqa: E731
        ids0 = (C.c_uint32 * 1)(self.k_seq[0])
        self._keep.append(ids0)
        prog.append(_DevCall("sandy_hip_device_paged_lengths", dev.handle, C.c_uint32(self.k_pools[0]), ids0,
                             C.c_int32(1), d(self.pos)))
        prog.append(_Call("sandy_hip_gather", d(self.token), d(w["wte.weight"]), d(b["te"].view(1, 1, -1)), stream=s))
        prog.append(_Call("sandy_hip_gather", d(self.pos.view(1, 1)), d(w["wpe.weight"]), d(b["pe"].view(1, 1, -1)),
                          stream=s))
        prog.append(ew(self.add, self.add_res, [b["te"], b["pe"]], b["x"]))
        x, x2 = b["x"], b["x2"]
        H = c.hidden
        q, k, v = b["qkv"][:, :H], b["qkv"][:, H:2 * H], b["qkv"][:, 2 * H:]
        for i in range(c.layers):
            p = f"h.{i}."
            prog.append(linear(x, p + "attn.qkv", b["qkv"], ln=p + "ln_1"))
            kid, vid = (C.c_uint32 * 1)(self.k_seq[i]), (C.c_uint32 * 1)(self.v_seq[i])
            self._keep += [kid, vid]
            # this token's K and V rows appended together (one launch)
            prog.append(_DevCall("sandy_hip_device_paged_append_step_kv", dev.handle, C.c_uint32(self.k_pools[i]), kid,
                                 C.c_uint32(self.v_pools[i]), vid, C.c_int32(1), d(head4(k)), d(head4(v))))
            kc, table, _ = dev.paged_views(self.k_pools[i])
            vc, _, _ = dev.paged_views(self.v_pools[i])
            table.contents.dims[0] = 1
            self._keep += [kc, vc, table]
            prog.append(_Call("sandy_hip_paged_attention", d(head4(q)), kc, vc, table, d(self.pos),
                              C.c_int64(0), C.c_double(-1.0), d(head4(b["ctx"])), stream=s))
            prog.append(linear(b["ctx"], p + "attn.c_proj", x2, residual=x))
            prog.append(linear(x2, p + "mlp.c_fc", b["g"], ln=p + "ln_2", gelu=True))
            prog.append(linear(b["g"], p + "mlp.c_proj", x, residual=x2))
        # logits = layer_norm(x) wte^T (no bias)
        prog.append(linear(x, "wte", self.logits, ln="ln_f"))
        prog.append(_Call("sandy_hip_topk", d(self.logits), C.c_int64(1), C.c_int64(-1), d(self.top_v),
                          d(self.token), stream=s))
        return prog

    def step(self):
        """One token through the bound program, eagerly (device stream)."""
        if self.length + 1 > self.max_seq:
            raise ValueError("GPT-2 cache is full")
        for call in self.program:
            call()
        self.length += 1

    def capture(self):
        """Capture one step as a HIP graph (run a warm step first)."""
        self.dev.graph_begin()
        try:
            for call in self.program:
                call()
        finally:
            self.graph = self.dev.graph_end()

    def replay(self):
        if self.length + 1 > self.max_seq:
            raise ValueError("GPT-2 cache is full")
        self.dev.graph_launch(self.graph)
        self.length += 1

    def forward(self, ids) -> torch.Tensor:
        """Prompt tokens (cache empty) or one token; returns that pass's last
        logits [1, vocab]."""
        if self.length == 0:
            return self._prompt(list(ids))
        if len(ids) != 1:
            raise ValueError("after the prompt, tokens are decoded one at a time")
        torch.cuda.synchronize()
        self.token.fill_(int(ids[0]))
        torch.cuda.synchronize()
        self.step()
        self.dev.synchronize()
        return self.logits

    def greedy(self, prompt, steps: int, graph: bool = True):
        """Prompt pass, then `steps` - 1 single-token steps (one captured graph
        replayed, or eager); returns (tokens, prompt seconds, decode seconds)."""
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = self._prompt(list(prompt))
        with torch.cuda.stream(self.dev.torch_stream()):
            ops.topk(logits, 1, indices=self.token)
        self.dev.synchronize()
        t1 = time.perf_counter()
        tokens = [int(self.token.item())]
        for s in range(steps - 1):
            if graph and s > 0 and self.graph is None:
                self.dev.synchronize()
                self.capture()  # the eager first step sized every workspace
            if graph and self.graph is not None:
                self.replay()
            else:
                self.step()
            self.dev.synchronize()
            tokens.append(int(self.token.item()))
        return tokens, t1 - t0, time.perf_counter() - t1

    def close(self):
        if self.graph is not None:
            self.dev.graph_destroy(self.graph)
            self.graph = None
        if self._own_dev:
            self.dev.close()
