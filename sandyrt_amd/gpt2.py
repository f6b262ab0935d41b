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
attention, the GELU group and the lm-head matmul).  Greedy selection is
sandy_hip_topk with k = 1 (ties -> lowest id, src/server/Sampler.cpp:69-79).
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np
import torch

from . import ops


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
    """Weights resident on the GPU, dense K/V caches [1, heads, max_seq, D]
    per layer, one forward pass per call."""

    def __init__(self, cfg: GPT2Config, host_weights: dict, max_seq: int = 128, device="cuda"):
        self.cfg, self.max_seq = cfg, max_seq
        self.w = {k: torch.from_numpy(np.ascontiguousarray(v)).to(device) for k, v in host_weights.items()}
        shape = (1, cfg.heads, max_seq, cfg.head_dim)
        self.k = [torch.zeros(shape, dtype=torch.float32, device=device) for _ in range(cfg.layers)]
        self.v = [torch.zeros(shape, dtype=torch.float32, device=device) for _ in range(cfg.layers)]
        self.length = 0
        self.gelu, self.gelu_res = ops.gelu_nodes()
        self.add, self.add_res = ops.residual_add_nodes()
        self.copy = [ops.ScalarNode(0, ops.LOAD, 0)]

    def _heads(self, t, T):
        """[T, hidden] rows as [1, heads, T, D] (a strided view)."""
        return t.view(T, self.cfg.heads, self.cfg.head_dim).permute(1, 0, 2).unsqueeze(0)

    def forward(self, ids) -> torch.Tensor:
        """Runs tokens `ids` at positions length .. length + T - 1, appends
        their K/V, returns the logits of the last token [1, vocab]."""
        c, w = self.cfg, self.w
        T = len(ids)
        p0 = self.length
        if p0 + T > self.max_seq:
            raise ValueError("GPT-2 cache is full")
        dev = w["wte.weight"].device
        ids_t = torch.tensor([ids], dtype=torch.int64, device=dev)
        pos_t = torch.arange(p0, p0 + T, dtype=torch.int64, device=dev).view(1, T)
        x = ops.elementwise(self.add, self.add_res, [ops.embedding(ids_t, w["wte.weight"]),
                                                     ops.embedding(pos_t, w["wpe.weight"])]).view(T, c.hidden)
        offsets = torch.tensor([p0], dtype=torch.int64, device=dev)
        for i in range(c.layers):
            p = f"h.{i}."
            h = ops.layer_norm(x, w[p + "ln_1.weight"], w[p + "ln_1.bias"], c.eps)
            q = ops.linear(h, w[p + "attn.q_proj.weight"], w[p + "attn.q_proj.bias"])
            k = ops.linear(h, w[p + "attn.k_proj.weight"], w[p + "attn.k_proj.bias"])
            v = ops.linear(h, w[p + "attn.v_proj.weight"], w[p + "attn.v_proj.bias"])
            ops.elementwise(self.copy, 0, [self._heads(k, T)], out=self.k[i][:, :, p0:p0 + T])
            ops.elementwise(self.copy, 0, [self._heads(v, T)], out=self.v[i][:, :, p0:p0 + T])
            ctx = torch.empty(T, c.hidden, dtype=torch.float32, device=dev)
            ops.attention(self._heads(q, T), self.k[i][:, :, :p0 + T], self.v[i][:, :, :p0 + T], offsets, 0, -1.0,
                          out=self._heads(ctx, T))
            o = ops.linear(ctx, w[p + "attn.c_proj.weight"], w[p + "attn.c_proj.bias"])
            x = ops.elementwise(self.add, self.add_res, [x, o])
            h = ops.layer_norm(x, w[p + "ln_2.weight"], w[p + "ln_2.bias"], c.eps)
            f = ops.linear(h, w[p + "mlp.c_fc.weight"], w[p + "mlp.c_fc.bias"])
            f = ops.elementwise(self.gelu, self.gelu_res, [f])
            m = ops.linear(f, w[p + "mlp.c_proj.weight"], w[p + "mlp.c_proj.bias"])
            x = ops.elementwise(self.add, self.add_res, [x, m])
        last = x[T - 1:T]
        h = ops.layer_norm(last, w["ln_f.weight"], w["ln_f.bias"], c.eps)
        self.length = p0 + T
        return ops.matmul(h, w["wte.weight"], transpose_rhs=True)

    def greedy(self, prompt, steps: int):
        """Prompt pass, then `steps` greedy tokens; returns (tokens, prompt
        seconds, decode seconds) with the device synchronised at both ends."""
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = self.forward(list(prompt))
        _, idx = ops.topk(logits, 1)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        tokens = [int(idx.item())]
        for _ in range(steps - 1):
            logits = self.forward([tokens[-1]])
            _, idx = ops.topk(logits, 1)
            tokens.append(int(idx.item()))
        torch.cuda.synchronize()
        return tokens, t1 - t0, time.perf_counter() - t1
