"""Write the golden vectors under tests/golden/*.npz.

Each fixture holds seeded inputs and the outputs of the REFERENCE's own CPU
math (sandy::core, src/core/TensorCalc.cpp) for them, computed through
oracle/_ref/libsandyref.so -- the reference's src/core compiled from its
sources by oracle/Makefile (`make -C oracle ref`).  The fixtures are data
only; the reference itself never travels with the repository.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def bf(a):
    return O.f32_to_bf16(np.asarray(a, dtype=np.float32))


def cases(rng):
    """(name, fn, kwargs) -- kwargs are numpy inputs plus scalar params"""
    n = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    out = []
    out.append(("rms_norm_f32", "rms_norm", dict(x=n(4, 64), weight=n(64), eps=1e-5)))
    out.append(("rms_norm_bf16", "rms_norm", dict(x=bf(n(5, 128)), weight=bf(n(128)), eps=1e-5)))
    out.append(("rms_norm_bf16_noweight", "rms_norm", dict(x=bf(n(3, 96)), weight=None, eps=1e-6)))
    out.append(("layer_norm_f32", "layer_norm", dict(x=n(3, 96) + 2.0, weight=n(96), bias=n(96), eps=1e-5)))
    out.append(("layer_norm_bf16", "layer_norm", dict(x=bf(n(2, 64)), weight=bf(n(64)), bias=bf(n(64)), eps=1e-5)))
    sm = n(5, 128) * 4.0
    sm[2, :] = -np.inf
    sm[3, 5] = np.inf * -1
    out.append(("softmax_f32", "softmax", dict(x=sm, axis=-1)))
    out.append(("softmax_bf16_mid", "softmax", dict(x=bf(n(2, 7, 3)), axis=1)))
    out.append(("sum_f32", "sum", dict(x=n(6, 8), axis=-1)))
    out.append(("rope_f32_split", "rope", dict(x=n(2, 3, 16, 64), theta=10000.0, rotary_dim=-1, split_half=True)))
    out.append(("rope_bf16_interleaved_partial", "rope",
                dict(x=bf(n(1, 4, 8, 64)), theta=10000.0, rotary_dim=32, split_half=False)))
    out.append(("rope_f32_ids_offset", "rope", dict(x=n(2, 5, 32), theta=10000.0, rotary_dim=-1, split_half=True,
                                                    position_ids=np.array([4000], dtype=np.int64))))
    out.append(("rope_f32_ids_seq", "rope", dict(x=n(3, 4, 64), theta=1e6, rotary_dim=16, split_half=True,
                                                 position_ids=np.array([7, 3000, 4095, 1], dtype=np.int32))))
    out.append(("rope_bf16_ids_vectors", "rope", dict(x=bf(n(2, 3, 64)), theta=10000.0, rotary_dim=-1,
                                                      split_half=True,
                                                      position_ids=rng.integers(0, 8192, 6).astype(np.int64))))
    out.append(("attention_f32_decode_gqa", "attention",
                dict(q=n(2, 8, 1, 64) * 0.3, k=n(2, 2, 40, 64) * 0.3, v=n(2, 2, 40, 64),
                     position_offsets=np.array([39, 17], dtype=np.int64), window=0, scale=-1.0)))
    out.append(("attention_bf16_decode_g8", "attention",
                dict(q=bf(n(1, 8, 1, 64)), k=bf(n(1, 1, 48, 64)), v=bf(n(1, 1, 48, 64)),
                     position_offsets=np.array([47], dtype=np.int32), window=0, scale=0.125)))
    out.append(("attention_f32_window", "attention",
                dict(q=n(1, 4, 1, 32), k=n(1, 2, 30, 32), v=n(1, 2, 30, 32),
                     position_offsets=np.array([25], dtype=np.int64), window=7, scale=-1.0)))
    out.append(("attention_f32_prefill", "attention",
                dict(q=n(1, 4, 3, 16), k=n(1, 4, 5, 16), v=n(1, 4, 5, 16), position_offsets=None,
                     window=0, scale=-1.0)))
    out.append(("attention_f32_masked_all", "attention",
                dict(q=n(1, 2, 1, 16), k=n(1, 1, 4, 16), v=n(1, 1, 4, 16),
                     position_offsets=np.array([20], dtype=np.int64), window=3, scale=-1.0)))
    tk = np.round(n(6, 128) * 2) / 2  # many ties
    out.append(("topk_f32_ties", "topk", dict(x=tk, k=8, axis=-1)))
    out.append(("topk_bf16", "topk", dict(x=bf(n(4, 128)), k=8, axis=-1)))
    out.append(("embedding_bf16", "embedding", dict(ids=np.array([3, 0, 9, 3], dtype=np.int64),
                                                   weight=bf(n(10, 16)))))
    # MoE chain
    T, H, E, K = 6, 16, 4, 2
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    w = np.abs(n(T, K))
    out.append(("moe_gather_f32", "moe_gather", dict(x=n(T, H), topk_ids=ids, topk_weights=w, num_experts=E)))
    out.append(("moe_gather_bf16_batched", "moe_gather",
                dict(x=bf(n(2, T, H)), topk_ids=np.stack([ids, ids[::-1]]), topk_weights=bf(np.stack([w, w])),
                     num_experts=E)))
    offs = np.array([0, 3, 3, 9, 12], dtype=np.int64)
    out.append(("moe_matmul_f32_t", "moe_matmul", dict(x=n(12, H), expert_offsets=offs, weight=n(E, 8, H) * 0.2,
                                                       transpose_rhs=True)))
    out.append(("moe_matmul_bf16_n", "moe_matmul", dict(x=bf(n(12, H)), expert_offsets=offs,
                                                        weight=bf(n(E, H, 8) * 0.2), transpose_rhs=False)))
    tok = rng.integers(0, T, 12).astype(np.int64)
    out.append(("moe_scatter_sum_bf16", "moe_scatter_sum",
                dict(packed_out=bf(n(12, H)), packed_weights=bf(np.abs(n(12))), token_ids=tok, seq=T)))
    out.append(("moe_scatter_sum_f32", "moe_scatter_sum",
                dict(packed_out=n(12, H), packed_weights=np.abs(n(12)), token_ids=tok, seq=T)))
    out.append(("binary_add_bcast_bf16", "binary", dict(op="add", lhs=bf(n(3, 4, 8)), rhs=bf(n(4, 1)))))
    out.append(("binary_mul_f32", "binary", dict(op="mul", lhs=n(5, 8), rhs=n(8))))
    out.append(("binary_div_f32", "binary", dict(op="div", lhs=n(5, 8), rhs=n(5, 8) + 3.0)))
    out.append(("unary_tanh_bf16", "unary", dict(op="tanh", x=bf(n(40) * 3))))
    out.append(("unary_sqrt_f32", "unary", dict(op="sqrt", x=np.abs(n(40)))))
    out.append(("unary_relu_f32", "unary", dict(op="relu", x=n(40))))
    out.append(("matmul_f32", "matmul", dict(lhs=n(2, 3, 16), rhs=n(16, 5), transpose_rhs=False)))
    out.append(("matmul_bf16_t", "matmul", dict(lhs=bf(n(5, 64)), rhs=bf(n(24, 64) * 0.2), transpose_rhs=True)))
    out.append(("matmul_f32_tlhs", "matmul", dict(lhs=n(16, 6), rhs=n(3, 16, 7), transpose_lhs=True)))
    out.append(("matmul_f32_grouped_heads", "matmul", dict(lhs=n(2, 8, 3, 16), rhs=n(2, 2, 16, 5))))
    out.append(("matmul_bf16_bcast", "matmul", dict(lhs=bf(n(4, 1, 3, 32)), rhs=bf(n(3, 5, 32)), transpose_rhs=True)))
    out.append(("linear_bf16", "linear", dict(x=bf(n(4, 48)), weight=bf(n(9, 48) * 0.2), bias=bf(n(9)))))
    out.append(("linear_f32", "linear", dict(x=n(3, 16), weight=n(8, 16), bias=n(8))))
    return out


def run(o: O.Oracle, fn: str, kw: dict):
    res = getattr(o, fn)(**kw)
    return res if isinstance(res, tuple) else (res,)


def main():
    ref = O.Oracle(reference=True)
    rng = np.random.default_rng(20251201)
    for name, fn, kw in cases(rng):
        outs = run(ref, fn, kw)
        payload = {"fn": np.array(fn)}
        for k, v in kw.items():
            if v is None:
                payload["none_" + k] = np.array(0)
            elif isinstance(v, np.ndarray):
                payload["in_" + k] = v
            else:
                payload["param_" + k] = np.array(v)
        for i, v in enumerate(outs):
            payload[f"out_{i}"] = v
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **payload)
        print("wrote", name)


def load(path):
    """-> (fn, kwargs, outputs)"""
    z = np.load(path, allow_pickle=False)
    fn = str(z["fn"])
    kw, outs = {}, []
    for k in z.files:
        if k.startswith("in_"):
            kw[k[3:]] = z[k]
        elif k.startswith("none_"):
            kw[k[5:]] = None
        elif k.startswith("param_"):
            v = z[k]
            kw[k[6:]] = v.item() if v.dtype.kind != "U" else str(v)
    i = 0
    while f"out_{i}" in z.files:
        outs.append(z[f"out_{i}"])
        i += 1
    return fn, kw, outs


if __name__ == "__main__":
    main()
