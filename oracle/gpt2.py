"""GPT-2 small greedy decoding as the reference CPU path computes it -- test
infrastructure only (the parity checker and bench.py's CPU baseline).

The op chain of src/models/gpt2_small.sandy.go on the oracle restatement of
src/core/TensorCalc.cpp (embedding 1520-1563, add/mul 562-663, tanh 775-799,
layer_norm 2010-2077, linear 722-773, attention 1167-1314, the GELU of
src/ir/BuiltinLowering.cpp:116-140 as the unfused fp32 op chain, matmul
804-919 with the transposed wte), with a K/V cache: row-independent ops give
each row the values the reference's full recompute gives it, and the last
row attends over the same keys.  Greedy selection is the first maximum
(src/server/Sampler.cpp:69-79: stable sort, ties -> lowest id)."""
from __future__ import annotations

import numpy as np

from . import oracle as O


def gelu_chain(o: O.Oracle, x):
    """gelu as the reference CPU path runs it with element-wise fusion off
    (src/ir/MidIRToKernelIR.h:12-17): one op per node of
    src/ir/BuiltinLowering.cpp:125-139, fp32 tensors, constants as scalars."""
    c = lambda v: np.array([v], np.float32)  # noqa: E731
    x3 = o.binary("mul", o.binary("mul", x, x), x)
    inner = o.binary("add", x, o.binary("mul", c(0.044715), x3))
    t = o.unary("tanh", o.binary("mul", c(0.7978845608028654), inner))
    return o.binary("mul", o.binary("mul", c(0.5), x), o.binary("add", c(1.0), t))


class GPT2Oracle:
    def __init__(self, orc: O.Oracle, cfg, weights: dict):
        self.o, self.cfg, self.w = orc, cfg, weights
        self.k = [np.zeros((1, cfg.heads, 0, cfg.head_dim), np.float32) for _ in range(cfg.layers)]
        self.v = [np.zeros((1, cfg.heads, 0, cfg.head_dim), np.float32) for _ in range(cfg.layers)]

    def forward(self, ids):
        """Tokens `ids` at positions length .. length + T - 1; returns the last
        row's logits [vocab] (fp32)."""
        o, c, w = self.o, self.cfg, self.w
        T = len(ids)
        p0 = self.k[0].shape[2]
        x = o.binary("add", o.embedding(np.array([ids], np.int64), w["wte.weight"]),
                     o.embedding(np.arange(p0, p0 + T, dtype=np.int64).reshape(1, T), w["wpe.weight"]))
        x = x.reshape(T, c.hidden)
        heads = lambda t: np.ascontiguousarray(t.reshape(1, T, c.heads, c.head_dim).transpose(0, 2, 1, 3))  # noqa: E731
        offsets = np.array([p0], np.int64)
        for i in range(c.layers):
            p = f"h.{i}."
            h = o.layer_norm(x, w[p + "ln_1.weight"], w[p + "ln_1.bias"], c.eps)
            q = o.linear(h, w[p + "attn.q_proj.weight"], w[p + "attn.q_proj.bias"])
            k = o.linear(h, w[p + "attn.k_proj.weight"], w[p + "attn.k_proj.bias"])
            v = o.linear(h, w[p + "attn.v_proj.weight"], w[p + "attn.v_proj.bias"])
            self.k[i] = np.concatenate([self.k[i], heads(k)], axis=2)
            self.v[i] = np.concatenate([self.v[i], heads(v)], axis=2)
            ctx = o.attention(heads(q), self.k[i], self.v[i], offsets, 0, -1.0)
            ctx = np.ascontiguousarray(ctx.transpose(0, 2, 1, 3)).reshape(T, c.hidden)
            x = o.binary("add", x, o.linear(ctx, w[p + "attn.c_proj.weight"], w[p + "attn.c_proj.bias"]))
            h = o.layer_norm(x, w[p + "ln_2.weight"], w[p + "ln_2.bias"], c.eps)
            f = o.linear(h, w[p + "mlp.c_fc.weight"], w[p + "mlp.c_fc.bias"])
            f = gelu_chain(o, f)
            x = o.binary("add", x, o.linear(f, w[p + "mlp.c_proj.weight"], w[p + "mlp.c_proj.bias"]))
        h = o.layer_norm(np.ascontiguousarray(x[T - 1:T]), w["ln_f.weight"], w["ln_f.bias"], c.eps)
        return o.matmul(h, w["wte.weight"], transpose_rhs=True).reshape(-1)

    def greedy(self, prompt, steps: int):
        """Returns (tokens, margins): margins[i] = top-1 minus top-2 logit at step i."""
        tokens, margins = [], []
        logits = self.forward(list(prompt))
        for s in range(steps):
            top2 = np.partition(logits, -2)[-2:]
            margins.append(float(top2[1] - top2[0]))
            tokens.append(int(np.argmax(logits)))
            if s + 1 < steps:
                logits = self.forward([tokens[-1]])
        return tokens, margins
