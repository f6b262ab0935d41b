#!/usr/bin/env python3
"""Benchmark of the SandyRT hot path on one MI355X.

One step = one pass of the hot path over one batch of synthetic input:

  BASELINE config 2 (TinyLlama-1.1B shape, 4096 tokens x 2048 hidden, bf16,
  inputs N(0,1), seed 1):
    1. residual add + RMSNorm        x, h [4096, 2048] -> x + h, rmsnorm(x + h) * w
    2. RoPE (theta 1e4, split-half)  q [1, 32, 4096, 64] and k [1, 4, 4096, 64]
                                     in one launch (sandy_hip_rope_pair)
    3. SiLU-gate group               silu(gate) * up, [4096, 2048] (hipRTC-generated)
  BASELINE config 3 (paged decode, bf16 KV, block 16, seed 2):
    4. decode attention, 32 sequences, ctx U[512, 4096], 32 q / 4 kv heads,
       D 64, block table = random permutation of a 32768-block pool.

Inputs are resident in HBM before timing.  Each kernel rotates over
independent replicas of its inputs, at least 1 GiB per rotation (4x the
256 MB MALL; at most 256 replicas, so only the few-MB launch-bound kernels
stay below that) so repeated launches cannot hit in the Infinity Cache.  `value` is the whole step's
algorithmic bytes / measured step time.  Per-kernel durations come from HIP
events around the replay of a captured graph of back-to-back launches; the dominant kernel
gives the `roofline` object.  `cpu_baseline` times the reference's own CPU
math (oracle/_ref, built from the reference sources) or, where that build is
absent, the oracle restatement -- on one host core, on a bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
T, HID, HQ, HKV, HD = 4096, 2048, 32, 4, 64
DEC_B, DEC_POOL, DEC_PAGE = 32, 32768, 16


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--replicas", type=int, default=4)
    p.add_argument("--kernel-iters", type=int, default=64)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--graph", action="store_true",
                   help="replay the step as a captured HIP graph (measured slower than eager launches here)")
    p.add_argument("--cpu-tokens", type=int, default=4096, help="C2 rows timed on the CPU")
    p.add_argument("--cpu-seqs", type=int, default=8, help="decode sequences timed on the CPU")
    p.add_argument("--only", default="", help="comma list of kernels to run (profiling)")
    p.add_argument("--kv-layout", choices=["split", "interleaved"], default="split",
                   help="config-3 KV pool: separate K and V pools, or one pool with each block's K and V pages "
                        "side by side")
    p.add_argument("--no-extras", action="store_true", help="skip the per-kernel table of the other configs")
    p.add_argument("--no-decode-step", action="store_true", help="skip the whole-model decode tok/s measurement")
    p.add_argument("--gpt2-only", action="store_true",
                   help="only config 1 (GPT-2 greedy decode on the GPU, tokens checked against the CPU chain)")
    p.add_argument("--decode-step-only", action="store_true",
                   help="only the whole-model decode step at config 3's batch and contexts (profiling)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run a plain 256 MiB device copy (counter calibration for rocprofv3 --pmc)")
    return p.parse_args()


MIN_ROTATION_BYTES = 1 << 30  # per kernel: 4x the 256 MB MALL


def replicas_for(nbytes, at_least, cap=256):
    """Input replicas a kernel rotates over so that one rotation moves at
    least MIN_ROTATION_BYTES (no MALL hits between repeated launches); capped
    for the few-MB kernels, which are launch-bound and reported in us."""
    return max(at_least, min(cap, -(-MIN_ROTATION_BYTES // max(1, nbytes))))


class Prepared:
    """A C-ABI call with its ctypes arguments built once (no per-call Python
    tensor inspection), so back-to-back launches keep the GPU queue full."""

    def __init__(self, name, *args):
        from sandyrt_amd import _lib
        self.fn = getattr(_lib.lib(), name)
        self.args = args
        self.buf = C.create_string_buffer(256)

    def __call__(self, stream):
        rc = self.fn(*self.args, C.c_void_p(stream), self.buf, C.c_size_t(256))
        if rc:
            raise RuntimeError(self.buf.value.decode())


def build_workload(replicas, kv_layout="split"):
    import numpy as np
    import torch
    from sandyrt_amd import _lib, ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    desc = _lib.desc
    kernels = {k: [] for k in ("add_rms_norm", "rope_qk", "silu_gate", "paged_decode")}
    keep = []
    nodes, result = ops.silu_mul_nodes()
    cnodes = ops._nodes(nodes)
    r = np.random.default_rng(2)
    ctx = r.integers(512, 4097, DEC_B).astype(np.int64)
    nblk = (ctx + DEC_PAGE - 1) // DEC_PAGE
    max_blocks = int(nblk.max())
    host = {}
    bytes_per = {
        "add_rms_norm": 4 * T * HID * 2 + HID * 2,
        "rope_qk": 2 * (HQ + HKV) * T * HD * 2,
        "silu_gate": 3 * T * HID * 2,
        "paged_decode": int(ctx.sum()) * HKV * HD * 2 * 2 + 2 * DEC_B * HQ * HD * 2 + int(nblk.sum()) * 4,
    }
    reps = {n: replicas_for(b, replicas) for n, b in bytes_per.items()}
    for rep in range(max(reps.values())):
        g.manual_seed(1 + 1000 * rep)
        bf = torch.bfloat16
        d = {}
        if rep < reps["add_rms_norm"]:
            x = torch.randn(T, HID, generator=g, device=dev).to(bf)
            h = torch.randn(T, HID, generator=g, device=dev).to(bf)
            w = torch.randn(HID, generator=g, device=dev).to(bf)
            s_out, y = torch.empty_like(x), torch.empty_like(x)
            keep += [x, h, w, s_out, y]
            d.update({n: desc(t) for n, t in dict(x=x, h=h, w=w, s=s_out, y=y).items()})
            kernels["add_rms_norm"].append(Prepared("sandy_hip_add_rms_norm", d["x"], d["h"], d["w"],
                                                    C.c_double(1e-5), d["s"], d["y"]))
        if rep < reps["rope_qk"]:
            q = torch.randn(1, HQ, T, HD, generator=g, device=dev).to(bf)
            k = torch.randn(1, HKV, T, HD, generator=g, device=dev).to(bf)
            q_out, k_out = torch.empty_like(q), torch.empty_like(k)
            keep += [q, q_out, k, k_out]
            d.update(q=desc(q), qo=desc(q_out), k=desc(k), ko=desc(k_out))
            kernels["rope_qk"].append(Prepared("sandy_hip_rope_pair", d["q"], d["k"], None, C.c_double(1e4),
                                               C.c_int64(-1), C.c_int32(1), d["qo"], d["ko"]))
        if rep < reps["silu_gate"]:
            gate = torch.randn(T, HID, generator=g, device=dev).to(bf)
            up = torch.randn(T, HID, generator=g, device=dev).to(bf)
            act = torch.empty_like(gate)
            keep += [gate, up, act]
            d.update(gate=desc(gate), up=desc(up), act=desc(act))
            arr = (_lib.SandyTensor * 2)(d["gate"].contents, d["up"].contents)
            bc = (C.c_int32 * 2)(0, 0)
            keep += [arr, bc]
            kernels["silu_gate"].append(Prepared("sandy_hip_elementwise", cnodes, C.c_int32(len(nodes)),
                                                 C.c_uint32(result), arr, bc, C.c_int32(2), d["act"]))
        if rep < reps["paged_decode"]:
            g.manual_seed(2 + 1000 * rep)
            if kv_layout == "interleaved":
                kvpool = torch.randn(DEC_POOL, 2, HKV, DEC_PAGE, HD, generator=g, device=dev).to(bf)
                kpool, vpool = kvpool[:, 0], kvpool[:, 1]
                kcache, vcache = ops.PagedCache.interleaved(kvpool)
                keep.append(kvpool)
            else:
                kpool = torch.randn(DEC_POOL, HKV, DEC_PAGE, HD, generator=g, device=dev).to(bf)
                vpool = torch.randn(DEC_POOL, HKV, DEC_PAGE, HD, generator=g, device=dev).to(bf)
                kcache, vcache = ops.PagedCache(kpool), ops.PagedCache(vpool)
            qd = torch.randn(DEC_B, HQ, 1, HD, generator=g, device=dev).to(bf)
            od = torch.empty_like(qd)
            perm = np.random.default_rng(2 + rep).permutation(DEC_POOL).astype(np.int32)
            table = np.zeros((DEC_B, max_blocks), np.int32)
            off = 0
            for b in range(DEC_B):
                table[b, :nblk[b]] = perm[off:off + nblk[b]]
                off += nblk[b]
            table_t = torch.from_numpy(table).to(dev)
            pos_t = torch.from_numpy(ctx - 1).to(dev)
            kc, vc = kcache.struct(), vcache.struct()
            keep += [kpool, vpool, qd, od, table_t, pos_t, kc, vc]
            d.update({n: desc(t) for n, t in dict(qd=qd, od=od, table=table_t, pos=pos_t).items()})
            kernels["paged_decode"].append(Prepared("sandy_hip_paged_attention", d["qd"], kc, vc, d["table"],
                                                    d["pos"], C.c_int64(0), C.c_double(0.125), d["od"]))
        keep.append(d)
        if rep == 0:
            host = dict(x=x, h=h, w=w, q=q, k=k, gate=gate, up=up, kpool=kpool, vpool=vpool, qd=qd,
                        table=table, ctx=ctx)
    return kernels, bytes_per, keep, host


GEM_B, GEM_HQ, GEM_HKV, GEM_D, GEM_HID, GEM_FF, GEM_VOCAB = 64, 8, 2, 256, 2560, 10240, 262144
GPT2_VOCAB = 50257
FFN, LLAMA_VOCAB = 5632, 32000
MOE_T, MOE_E, MOE_K, MOE_D, MOE_F = 512, 128, 8, 2816, 704


def build_extras(replicas):
    """Config 4 (Gemma decoder layer: paged decode D 256 + norm/GeGLU/softcap
    groups at batch 64), config 5 (MoE block), config 1's greedy argmax, the
    TinyLlama decode projections (dense GEMMs) at the config-3 batch and
    config 2's SiLU gate at the model's FFN width, as prepared kernel calls.
    Reported per kernel; not part of `value`."""
    import numpy as np
    import torch
    from sandyrt_amd import _lib, ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    desc = _lib.desc
    bf = torch.bfloat16
    kernels, keep = {}, []
    # ---- config 4
    r = np.random.default_rng(3)
    ctx = r.integers(1024, 8193, GEM_B).astype(np.int64)
    nblk = (ctx + DEC_PAGE - 1) // DEC_PAGE
    maxb = int(nblk.max())
    pool = int(nblk.sum()) + 64
    names = ["c4_paged_decode", "c4_rms_norm", "c4_geglu", "c4_softcap", "c4_greedy_argmax"]
    for n in names:
        kernels[n] = []
    bytes_per = {
        "c4_paged_decode": int(ctx.sum()) * GEM_HKV * GEM_D * 2 * 2 + 2 * GEM_B * GEM_HQ * GEM_D * 2 + int(nblk.sum()) * 4,
        "c4_rms_norm": 2 * GEM_B * GEM_HID * 2 + GEM_HID * 2,
        "c4_geglu": 3 * GEM_B * GEM_FF * 2,
        "c4_softcap": 2 * GEM_B * GEM_VOCAB * 2,
        "c4_greedy_argmax": GEM_B * GEM_VOCAB * 2 + GEM_B * 10,
    }
    reps = {n: replicas_for(bytes_per[n], replicas) for n in names}
    gnodes, gres = ops.gelu_mul_nodes()
    snodes, sres = ops.softcap_nodes(30.0)
    cg, cs = ops._nodes(gnodes), ops._nodes(snodes)
    bc = (C.c_int32 * 2)(0, 0)
    keep += [cg, cs, bc]
    for rep in range(max(reps.values())):
        g.manual_seed(3 + 1000 * rep)
        if rep < reps["c4_paged_decode"]:
            kpool = torch.randn(pool, GEM_HKV, DEC_PAGE, GEM_D, generator=g, device=dev).to(bf)
            vpool = torch.randn(pool, GEM_HKV, DEC_PAGE, GEM_D, generator=g, device=dev).to(bf)
            qd = torch.randn(GEM_B, GEM_HQ, 1, GEM_D, generator=g, device=dev).to(bf)
            od = torch.empty_like(qd)
            perm = np.random.default_rng(3 + rep).permutation(pool).astype(np.int32)
            table = np.zeros((GEM_B, maxb), np.int32)
            off = 0
            for b in range(GEM_B):
                table[b, :nblk[b]] = perm[off:off + nblk[b]]
                off += nblk[b]
            tt = torch.from_numpy(table).to(dev)
            pt = torch.from_numpy(ctx - 1).to(dev)
            kc, vc = ops.PagedCache(kpool).struct(), ops.PagedCache(vpool).struct()
            d = {k: desc(v) for k, v in dict(qd=qd, od=od, tt=tt, pt=pt).items()}
            keep += [kpool, vpool, qd, od, tt, pt, kc, vc, d]
            kernels["c4_paged_decode"].append(Prepared("sandy_hip_paged_attention", d["qd"], kc, vc, d["tt"], d["pt"],
                                                       C.c_int64(0), C.c_double(1.0), d["od"]))
        if rep < reps["c4_rms_norm"]:
            xg = torch.randn(GEM_B, GEM_HID, generator=g, device=dev).to(bf)
            wg = torch.randn(GEM_HID, generator=g, device=dev).to(bf)
            yg = torch.empty_like(xg)
            d = {k: desc(v) for k, v in dict(xg=xg, wg=wg, yg=yg).items()}
            keep += [xg, wg, yg, d]
            kernels["c4_rms_norm"].append(Prepared("sandy_hip_norm", C.c_int32(0), d["xg"], d["wg"], None,
                                                   C.c_double(1e-6), d["yg"]))
        if rep < reps["c4_geglu"]:
            gate = torch.randn(GEM_B, GEM_FF, generator=g, device=dev).to(bf)
            up = torch.randn(GEM_B, GEM_FF, generator=g, device=dev).to(bf)
            act = torch.empty_like(gate)
            d = {k: desc(v) for k, v in dict(gate=gate, up=up, act=act).items()}
            arr2 = (_lib.SandyTensor * 2)(d["gate"].contents, d["up"].contents)
            keep += [gate, up, act, d, arr2]
            kernels["c4_geglu"].append(Prepared("sandy_hip_elementwise", cg, C.c_int32(len(gnodes)), C.c_uint32(gres),
                                                arr2, bc, C.c_int32(2), d["act"]))
        if rep < max(reps["c4_softcap"], reps["c4_greedy_argmax"]):
            logits = (torch.randn(GEM_B, GEM_VOCAB, generator=g, device=dev) * 20).to(bf)
            capped = torch.empty_like(logits)
            amax_v = torch.empty(GEM_B, 1, dtype=bf, device=dev)
            amax_i = torch.empty(GEM_B, 1, dtype=torch.int64, device=dev)
            d = {k: desc(v) for k, v in dict(logits=logits, capped=capped, amax_v=amax_v, amax_i=amax_i).items()}
            arr1 = (_lib.SandyTensor * 1)(d["logits"].contents)
            keep += [logits, capped, amax_v, amax_i, d, arr1]
            if rep < reps["c4_greedy_argmax"]:
                kernels["c4_greedy_argmax"].append(Prepared("sandy_hip_topk", d["logits"], C.c_int64(1), C.c_int64(-1),
                                                            d["amax_v"], d["amax_i"]))
            if rep < reps["c4_softcap"]:
                kernels["c4_softcap"].append(Prepared("sandy_hip_elementwise", cs, C.c_int32(len(snodes)),
                                                      C.c_uint32(sres), arr1, bc, C.c_int32(1), d["capped"]))
    # ---- config 1: greedy token selection over GPT-2's fp32 vocabulary
    g.manual_seed(1)
    c1_logits = torch.randn(1, GPT2_VOCAB, generator=g, device=dev)
    c1_v = torch.empty(1, 1, device=dev)
    c1_i = torch.empty(1, 1, dtype=torch.int64, device=dev)
    d1 = {k: desc(v) for k, v in dict(l=c1_logits, v=c1_v, i=c1_i).items()}
    keep += [c1_logits, c1_v, c1_i, d1]
    kernels["c1_greedy_argmax"] = [Prepared("sandy_hip_topk", d1["l"], C.c_int64(1), C.c_int64(-1), d1["v"], d1["i"])]
    bytes_per["c1_greedy_argmax"] = GPT2_VOCAB * 4 + 12
    # ---- TinyLlama decode projections at the config-3 batch (32 rows): the
    # dense GEMMs of one decode step (q/k/v and gate/up fused as one weight
    # each) and the lm-head, bf16 weights N(0, 0.02); replicas rotate so the
    # weights stream from HBM
    dense = {"c3_qkv_proj": (HQ * HD + 2 * HKV * HD, HID), "c3_o_proj": (HID, HID),
             "c3_gate_up_proj": (2 * FFN, HID), "c3_down_proj": (HID, FFN), "c3_lm_head": (LLAMA_VOCAB, HID)}
    for name, (n, k) in dense.items():
        kernels[name] = []
        for rep in range(replicas_for(n * k * 2, 1, cap=64)):
            g.manual_seed(7 + 100 * rep)
            xin = torch.randn(DEC_B, k, generator=g, device=dev).to(bf)
            w = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(bf)
            yo = torch.empty(DEC_B, n, dtype=bf, device=dev)
            dd = {kk: desc(v) for kk, v in dict(x=xin, w=w, y=yo).items()}
            keep += [xin, w, yo, dd]
            kernels[name].append(Prepared("sandy_hip_matmul", dd["x"], dd["w"], C.c_int32(0), C.c_int32(1), dd["y"]))
        bytes_per[name] = n * k * 2 + DEC_B * k * 2 + DEC_B * n * 2
    # ---- config 2 SiLU-gate at the model's FFN width (the step above runs it at 2048)
    kernels["c2_silu_gate_ffn"] = []
    snodes, sres = ops.silu_mul_nodes()
    csn = ops._nodes(snodes)
    bc2 = (C.c_int32 * 2)(0, 0)
    keep += [csn, bc2]
    for rep in range(replicas_for(3 * T * FFN * 2, replicas)):
        g.manual_seed(11 + 100 * rep)
        gt = torch.randn(T, FFN, generator=g, device=dev).to(bf)
        ut = torch.randn(T, FFN, generator=g, device=dev).to(bf)
        at = torch.empty_like(gt)
        dd = {kk: desc(v) for kk, v in dict(g=gt, u=ut, a=at).items()}
        arr = (_lib.SandyTensor * 2)(dd["g"].contents, dd["u"].contents)
        keep += [gt, ut, at, dd, arr]
        kernels["c2_silu_gate_ffn"].append(Prepared("sandy_hip_elementwise", csn, C.c_int32(len(snodes)),
                                                    C.c_uint32(sres), arr, bc2, C.c_int32(2), dd["a"]))
    bytes_per["c2_silu_gate_ffn"] = 3 * T * FFN * 2
    # ---- config 2 RoPE from a cos/sin cache (built once per forward pass and
    # shared by q, k and the 22 layers; its build is timed on its own)
    kernels["c2_rope_cache"], kernels["c2_rope_qk_cached"] = [], []
    for rep in range(replicas_for(2 * (HQ + HKV) * T * HD * 2, replicas)):
        g.manual_seed(13 + 100 * rep)
        qq = torch.randn(1, HQ, T, HD, generator=g, device=dev).to(bf)
        kk_ = torch.randn(1, HKV, T, HD, generator=g, device=dev).to(bf)
        qo_, ko_ = torch.empty_like(qq), torch.empty_like(kk_)
        cache = torch.empty(T, HD // 2, 2, dtype=torch.float32, device=dev)
        dd = {kk: desc(v) for kk, v in dict(q=qq, k=kk_, qo=qo_, ko=ko_, c=cache).items()}
        keep += [qq, kk_, qo_, ko_, cache, dd]
        kernels["c2_rope_cache"].append(Prepared("sandy_hip_rope_cache", None, C.c_int64(T), C.c_double(1e4),
                                                 C.c_int64(-1), C.c_int64(HD), C.c_int32(1), dd["c"]))
        kernels["c2_rope_cache"][-1](torch.cuda.current_stream().cuda_stream)
        kernels["c2_rope_qk_cached"].append(Prepared("sandy_hip_rope_pair_cached", dd["q"], dd["k"], dd["c"],
                                                     dd["qo"], dd["ko"]))
    bytes_per["c2_rope_cache"] = T * (HD // 2) * 8
    bytes_per["c2_rope_qk_cached"] = 2 * (HQ + HKV) * T * HD * 2 + T * (HD // 2) * 8
    # ---- plain streams of the config-2 groups' byte counts: the practical
    # ceiling at these sizes (a 1-read/1-write copy of RoPE q+k's bytes, and a
    # 2-read/1-write residual add of SiLU-gate's)
    kernels["c2_copy_rope_bytes"], kernels["c2_add_silu_bytes"] = [], []
    anodes, ares = ops.residual_add_nodes()
    can = ops._nodes(anodes)
    keep += [can]
    for rep in range(replicas_for(2 * (HQ + HKV) * T * HD * 2, replicas)):
        src = torch.empty((HQ + HKV) * T * HD, dtype=bf, device=dev).normal_(generator=g)
        dst = torch.empty_like(src)
        a_ = torch.randn(T, HID, generator=g, device=dev).to(bf)
        b_ = torch.randn(T, HID, generator=g, device=dev).to(bf)
        o_ = torch.empty_like(a_)
        dd = {kk: desc(v) for kk, v in dict(s=src, d=dst, a=a_, b=b_, o=o_).items()}
        arr = (_lib.SandyTensor * 2)(dd["a"].contents, dd["b"].contents)
        keep += [src, dst, a_, b_, o_, dd, arr]
        kernels["c2_copy_rope_bytes"].append(Prepared("sandy_hip_layout_transform", dd["s"], dd["d"], C.c_int32(4)))
        kernels["c2_add_silu_bytes"].append(Prepared("sandy_hip_elementwise", can, C.c_int32(len(anodes)),
                                                     C.c_uint32(ares), arr, bc2, C.c_int32(2), dd["o"]))
    bytes_per["c2_copy_rope_bytes"] = 2 * (HQ + HKV) * T * HD * 2
    bytes_per["c2_add_silu_bytes"] = 3 * T * HID * 2
    # ---- config 5 (one copy: the 1.5 GB of expert weights exceed the cache)
    g.manual_seed(4)
    logits = torch.randn(MOE_T, MOE_E, generator=g, device=dev)
    probs = ops.softmax(logits)
    tw, tid = ops.topk(probs, MOE_K)
    x = torch.randn(MOE_T, MOE_D, generator=g, device=dev).to(bf)
    wgate = (torch.randn(MOE_E, MOE_F, MOE_D, generator=g, device=dev) * 0.02).to(bf)
    wup = (torch.randn(MOE_E, MOE_F, MOE_D, generator=g, device=dev) * 0.02).to(bf)
    wdown = (torch.randn(MOE_E, MOE_D, MOE_F, generator=g, device=dev) * 0.02).to(bf)
    twb = tw.to(bf)
    px, pw, tok, offs = ops.moe_gather(x, tid, twb, MOE_E)
    gate_o = torch.empty(MOE_T * MOE_K, MOE_F, dtype=bf, device=dev)
    up_o, act_o = torch.empty_like(gate_o), torch.empty_like(gate_o)
    down_o = torch.empty(MOE_T * MOE_K, MOE_D, dtype=bf, device=dev)
    comb = torch.empty(MOE_T, MOE_D, dtype=bf, device=dev)
    vals = torch.empty(MOE_T, MOE_K, device=dev)
    idx = torch.empty(MOE_T, MOE_K, dtype=torch.int64, device=dev)
    d = {k: desc(v) for k, v in dict(probs=probs, vals=vals, idx=idx, x=x, tid=tid, twb=twb, px=px, pw=pw, tok=tok,
                                     offs=offs, wgate=wgate, wup=wup, wdown=wdown, gate_o=gate_o, up_o=up_o,
                                     act_o=act_o, down_o=down_o, comb=comb).items()}
    snodes, sres = ops.silu_mul_nodes()
    cs = ops._nodes(snodes)
    arr = (_lib.SandyTensor * 2)(d["gate_o"].contents, d["up_o"].contents)
    bc = (C.c_int32 * 2)(0, 0)
    keep += [logits, probs, tw, tid, x, wgate, wup, wdown, twb, px, pw, tok, offs, gate_o, up_o, act_o, down_o, comb,
             vals, idx, d, cs, arr, bc]
    kernels["c5_topk"] = [Prepared("sandy_hip_topk", d["probs"], C.c_int64(MOE_K), C.c_int64(-1), d["vals"], d["idx"])]
    kernels["c5_moe_gather"] = [Prepared("sandy_hip_moe_gather", d["x"], d["tid"], d["twb"], C.c_int64(MOE_E),
                                         C.c_int64(MOE_K), d["px"], d["pw"], d["tok"], d["offs"])]
    kernels["c5_moe_matmul_gate"] = [Prepared("sandy_hip_moe_matmul", d["px"], d["offs"], d["wgate"], C.c_int32(1),
                                              d["gate_o"])]
    kernels["c5_moe_matmul_up"] = [Prepared("sandy_hip_moe_matmul", d["px"], d["offs"], d["wup"], C.c_int32(1),
                                            d["up_o"])]
    kernels["c5_swiglu"] = [Prepared("sandy_hip_elementwise", cs, C.c_int32(len(snodes)), C.c_uint32(sres), arr, bc,
                                     C.c_int32(2), d["act_o"])]
    kernels["c5_moe_matmul_down"] = [Prepared("sandy_hip_moe_matmul", d["act_o"], d["offs"], d["wdown"],
                                              C.c_int32(1), d["down_o"])]
    kernels["c5_moe_scatter_sum"] = [Prepared("sandy_hip_moe_scatter_sum", d["down_o"], d["pw"], d["tok"], d["comb"])]
    rows = MOE_T * MOE_K
    wbytes = MOE_E * MOE_F * MOE_D * 2
    bytes_per.update({
        "c5_topk": MOE_T * MOE_E * 4 + MOE_T * MOE_K * 12,
        "c5_moe_gather": MOE_T * MOE_D * 2 + rows * MOE_D * 2,
        "c5_moe_matmul_gate": wbytes + rows * MOE_D * 2 + rows * MOE_F * 2,
        "c5_moe_matmul_up": wbytes + rows * MOE_D * 2 + rows * MOE_F * 2,
        "c5_swiglu": 3 * rows * MOE_F * 2,
        "c5_moe_matmul_down": wbytes + rows * MOE_F * 2 + rows * MOE_D * 2,
        "c5_moe_scatter_sum": rows * MOE_D * 2 + MOE_T * MOE_D * 2,
    })
    return kernels, bytes_per, keep


def decode_step_tok_s(batch, contexts, iters=10, seed=2, **decoder_opts):
    """Whole TinyLlama-1.1B greedy decode step (22 layers: projections, RoPE,
    paged append, paged decode attention, SiLU-gated MLP, lm-head, greedy
    token; random bf16 weights, synthetic K/V history of the given context
    lengths, block 16) for `batch` sequences, captured as one HIP graph and
    replayed; returns (us per step, tokens/s, bytes per step)."""
    import torch
    from sandyrt_amd.decode import DecodeConfig, TinyLlamaDecoder, random_weights
    from sandyrt_amd.device import HipDevice
    cfg = DecodeConfig(page_size=DEC_PAGE, max_context=int(max(contexts)) + iters + 64)
    w = random_weights(cfg, seed=seed)
    dev = HipDevice(0)
    dec = TinyLlamaDecoder(dev, cfg, w, batch=batch, **decoder_opts)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    for b, n in enumerate(contexts):
        ks = [torch.randn(1, cfg.kv_heads, int(n), cfg.head_dim, generator=g, device="cuda").to(torch.bfloat16)
              for _ in range(cfg.layers)]
        vs = [torch.randn(1, cfg.kv_heads, int(n), cfg.head_dim, generator=g, device="cuda").to(torch.bfloat16)
              for _ in range(cfg.layers)]
        dec.prefill_cache(ks, vs, seq=b)
    dec.set_token([int(t) for t in range(1, batch + 1)])
    dec.step()  # warm: generated kernels and workspaces exist before capture
    dev.synchronize()
    dec.capture()
    dec.replay()
    dev.synchronize()
    ts = dev.torch_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(ts)
    for _ in range(iters):
        dec.replay()
    ev1.record(ts)
    ev1.synchronize()
    us = ev0.elapsed_time(ev1) / iters * 1e3
    wbytes = sum(v.numel() * v.element_size() for n, v in w.items() if n != "embed") + batch * cfg.hidden * 2
    kv = sum(int(n) + 1 for n in contexts) * cfg.layers * cfg.kv_heads * cfg.head_dim * 2 * 2
    dec.close()
    dev.close()
    del dec, w
    torch.cuda.empty_cache()
    return us, batch / (us * 1e-6), wbytes + kv


def gpt2_config1():
    """BASELINE config 1 on the GPU: GPT-2 small (fp32, random weights
    N(0, 0.02) from numpy default_rng(0)), a 64-token prompt, 32 greedy tokens;
    tokens compared with the CPU chain's committed sequence.  The CPU side
    times the same op chain (the oracle restatement, one core) on a bounded
    sample: an 8-token prompt and 2 single-token steps."""
    import json as _json
    from oracle import oracle as O
    from oracle.gpt2 import GPT2Oracle
    from sandyrt_amd.gpt2 import GPT2Config, GPT2Runner, prompt_ids, random_weights
    cfg = GPT2Config()
    w = random_weights(cfg, seed=0)
    prompt = prompt_ids(cfg, 64, seed=0)
    runner = GPT2Runner(cfg, w, max_seq=128)
    runner.greedy(prompt[:8], 2)  # warm (generated kernels, workspaces)
    runner = GPT2Runner(cfg, w, max_seq=128)
    tokens, t_prompt, t_decode = runner.greedy(prompt, 32)
    golden = os.path.join(ROOT, "tests", "golden", "gpt2_c1_greedy.json")
    match = None
    if os.path.exists(golden):
        match = tokens == _json.load(open(golden))["tokens"]
    if not os.path.exists(O.LIB_PATH):
        O.build()
    kind = "reference" if os.path.exists(O.REF_PATH) else "port"
    cpu = GPT2Oracle(O.Oracle(reference=(kind == "reference")), cfg, w)
    cpu.forward(prompt[:8])
    t0 = time.perf_counter()
    for t in (11, 12):
        cpu.forward([t])
    cpu_tok_s = 2 / (time.perf_counter() - t0)
    return {"prompt_ms": round(t_prompt * 1e3, 2), "decode_tok_s": round(31 / t_decode, 1),
            "tokens_match_cpu": match, "cpu_decode_tok_s": round(cpu_tok_s, 2), "cpu_cores": 1,
            "cpu_kind": kind, **host_cpu_info(),
            "cpu_sample": ("the GPT-2 op chain on the reference's src/core build" if kind == "reference" else
                           "the GPT-2 op chain on the oracle restatement") +
                          ", 2 single-token steps after an 8-token prompt, one thread"}


def host_cpu_info():
    """The host the CPU figures were timed on: CPU model (/proc/cpuinfo, as
    lscpu reports it), logical CPUs of the machine and of this process."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"host_cpu": model, "nproc": os.cpu_count(), "nproc_usable": len(os.sched_getaffinity(0))}


def time_kernels(kernels, iters, stream, torch):
    """Average launch duration of each kernel: `iters` back-to-back launches
    rotating over its replicas are captured once as a HIP graph and replayed,
    timed by HIP events on the replay stream.  Replaying takes the host out
    of the measurement (one ctypes launch costs 4-7 us of host time, longer
    than most of these kernels run); what remains is GPU time, including the
    end-of-kernel drain between consecutive launches, as in a real step."""
    out = {}
    cap = torch.cuda.Stream()
    for name, calls in kernels.items():
        for c in calls:  # warm (compiles hipRTC groups, sizes workspaces)
            c(stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            s_cap = torch.cuda.current_stream().cuda_stream
            for i in range(iters):
                calls[i % len(calls)](s_cap)
        graph.replay()  # warm replay
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        graph.replay()
        ev1.record()
        ev1.synchronize()
        out[name] = ev0.elapsed_time(ev1) / iters * 1e3  # us
        del graph
    return out


def cpu_baseline(host, bytes_per, n_tokens, n_seqs):
    """Time the reference CPU math (or the oracle restatement) on one core."""
    import numpy as np
    from oracle import oracle as O
    from tests.helpers import to_oracle

    kind = "reference" if os.path.exists(O.REF_PATH) else "port"
    if not os.path.exists(O.LIB_PATH):
        O.build()
    cpu = O.Oracle(reference=(kind == "reference"))
    x = to_oracle(host["x"])[:n_tokens]
    h = to_oracle(host["h"])[:n_tokens]
    w = to_oracle(host["w"])
    q = to_oracle(host["q"])[:, :, :n_tokens]
    k = to_oracle(host["k"])[:, :, :n_tokens]
    gate = to_oracle(host["gate"])[:n_tokens]
    up = to_oracle(host["up"])[:n_tokens]
    half = O.f32_to_bf16(np.array(0.5, np.float32))
    one = O.f32_to_bf16(np.array(1.0, np.float32))
    t0 = time.perf_counter()
    s = cpu.binary("add", x, h)                      # reference: __add then __rms_norm
    cpu.rms_norm(s, w, 1e-5)
    cpu.rope(q, 1e4, split_half=True)
    cpu.rope(k, 1e4, split_half=True)
    hx = cpu.binary("mul", half, gate)               # silu lowered to mul/tanh/add/mul, then * up
    t = cpu.unary("tanh", hx)
    a = cpu.binary("add", one, t)
    sg = cpu.binary("mul", hx, a)
    cpu.binary("mul", sg, up)
    t_c2 = (time.perf_counter() - t0) * (T / n_tokens)
    kpool, vpool, table, ctx = to_oracle(host["kpool"]), to_oracle(host["vpool"]), host["table"], host["ctx"]
    qd = to_oracle(host["qd"])
    t_dec = 0.0
    sample_ctx = 0
    mat = O.Oracle()  # CpuDevice.cpp:611-676 restated (the reference build compiles only src/core)
    for b in range(n_seqs):
        c = int(ctx[b])
        # the reference CPU device materialises the paged K/V as dense tensors
        # before every attention (CpuDevice.cpp:611-676): timed with it
        t0 = time.perf_counter()
        kd = mat.paged_to_dense(kpool, table[b], HKV, c, DEC_PAGE, HD)[None]
        vd = mat.paged_to_dense(vpool, table[b], HKV, c, DEC_PAGE, HD)[None]
        cpu.attention(qd[b:b + 1], kd, vd, np.array([c - 1], np.int64), 0, 0.125)
        t_dec += time.perf_counter() - t0
        sample_ctx += c
    t_dec *= float(ctx.sum()) / sample_ctx
    total_bytes = sum(bytes_per.values())
    return {
        "value": round(total_bytes / (t_c2 + t_dec) / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        **host_cpu_info(),
        "sample": (f"config-2 groups on {n_tokens} of {T} tokens and decode attention for {n_seqs} of {DEC_B} "
                   f"sequences (paged->dense K/V materialisation of CpuDevice.cpp:611-676 included, as the reference "
                   f"CPU device runs it before each attention), "
                   f"single thread, scaled linearly to one full step"),
        "step_seconds": round(t_c2 + t_dec, 3),
    }


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (FETCH_SIZE / WRITE_SIZE scaled by an identity copy), or None --
    also when the summary's source stamp is not the stamp of the kernels
    being run (the measurement would describe other code)."""
    from sandyrt_amd.profile_summary import source_stamp, stamp_of
    path = os.path.join(ROOT, "profiles", "hbm_traffic_bench_kernels.md")
    if stamp_of(path) != source_stamp():
        return None
    prefix = {"paged_decode": "paged_decode_units_kernel<64,"}.get(kernel)
    for row in open(path):
        cells = [c.strip().strip("`") for c in row.strip().strip("|").split("|")]
        if prefix and len(cells) == 5 and cells[0].startswith(prefix):
            return int(float(cells[4]))
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the workload shards by rows and by "
              "sequence with no exchange); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    from sandyrt_amd import _lib

    _lib.lib()  # fail loudly if the backend is not built
    torch.cuda.set_device(0)
    if args.gpt2_only:
        print(json.dumps({"metric": "GPT-2 small greedy decode (config 1)", **gpt2_config1()}), flush=True)
        return
    if args.decode_step_only:
        import numpy as np
        ctx = np.random.default_rng(2).integers(512, 4097, DEC_B)
        us, tps, by = decode_step_tok_s(DEC_B, ctx, iters=args.steps)
        print(json.dumps({"metric": "TinyLlama decode step, batch 32, config-3 contexts", "us_per_step": round(us, 1),
                          "tok_s": round(tps, 1), "gbs": round(by / (us * 1e-6) / 1e9, 1)}), flush=True)
        us, tps, by = decode_step_tok_s(1, ctx[:1], iters=args.steps)
        print(json.dumps({"metric": "TinyLlama decode step, batch 1, context %d" % int(ctx[0]), "us_per_step": round(us, 1),
                          "tok_s": round(tps, 1), "gbs": round(by / (us * 1e-6) / 1e9, 1)}), flush=True)
        return
    kernels, bytes_per, keep, host = build_workload(args.replicas, args.kv_layout)
    if args.only:
        kernels = {k: v for k, v in kernels.items() if k in args.only.split(",")}
        bytes_per = {k: v for k, v in bytes_per.items() if k in kernels}
    stream = torch.cuda.current_stream().cuda_stream
    if args.calibrate_copy:
        # 256 MiB identity copy through the generated element-wise kernel
        # (16-byte loads/stores per lane, like every hot kernel here): the
        # rocprofv3 FETCH_SIZE / WRITE_SIZE it reads give the counter scale.
        from sandyrt_amd import ops as _ops
        src = torch.ones(128 << 20, dtype=torch.bfloat16, device="cuda")
        ident = [_ops.ScalarNode(0, _ops.LOAD, 0)]
        for _ in range(4):
            _ops.elementwise(ident, 0, [src])
        torch.cuda.synchronize()
        del src
    per_kernel_us = time_kernels(kernels, args.kernel_iters, stream, torch)

    order = list(kernels)
    reps = args.replicas
    if not args.graph:
        def step(i):
            for n in order:
                calls = kernels[n]
                calls[i % len(calls)](stream)
    else:
        # one HIP graph per replica holding the step's launches (captured
        # after the warm calls above sized every workspace), replayed on the
        # current stream: no host launch gaps between the step's kernels
        graphs = []
        cap = torch.cuda.Stream()
        for r in range(reps):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=cap):
                s_cap = torch.cuda.current_stream().cuda_stream
                for n in order:
                    kernels[n][r % len(kernels[n])](s_cap)
            graphs.append(gr)
        torch.cuda.synchronize()

        def step(i):
            graphs[i % reps].replay()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.steps
    _lib.take_device_errors()

    step_bytes = sum(bytes_per.values())
    value = step_bytes / step_s / 1e9
    if not per_kernel_us:
        per_kernel_us = {"add_rms_norm": float("nan")}
        bytes_per = {"add_rms_norm": 0}
    dominant = max(per_kernel_us, key=per_kernel_us.get)
    achieved = bytes_per[dominant] / (per_kernel_us[dominant] * 1e-6) / 1e9
    traffic = measured_traffic(dominant)
    kern = {n: {"us": round(per_kernel_us[n], 2), "bytes": bytes_per[n],
                "gbs": round(bytes_per[n] / (per_kernel_us[n] * 1e-6) / 1e9, 1),
                "frac": round(bytes_per[n] / (per_kernel_us[n] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)} for n in per_kernel_us}
    line = {
        "metric": "fused-group + paged-decode HBM GB/s (% of 8 TB/s) and decode tok/s, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) (seeds 1 and 2), inputs resident in HBM, rotated over replicas",
        "launch": "hip_graph (one captured step per replica)" if args.graph else "eager",
        "config": {"workload": "config2 TinyLlama fused groups (4096x2048 bf16) + config3 paged decode "
                               "(B32, ctx U[512,4096], 32q/4kv, D64, block 16, pool 32768)",
                   "tokens": T, "hidden": HID, "decode_batch": DEC_B,
                   "replicas": {n: len(v) for n, v in kernels.items()}},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "decode_tok_s": None,
        "kernels": kern,
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "cpu_baseline": None,
    }
    want_extras = not args.no_extras and (not args.only or any(o.startswith(("c1_", "c2_", "c3_", "c4_", "c5_"))
                                                               for o in args.only.split(",")))
    if want_extras:
        ek, eb, ekeep = build_extras(args.replicas)
        if args.only:
            ek = {k: v for k, v in ek.items() if k in args.only.split(",")}
        eus = time_kernels(ek, args.kernel_iters, stream, torch)
        _lib.take_device_errors()
        line["extras"] = {n: {"us": round(eus[n], 2), "bytes": eb[n],
                              "gbs": round(eb[n] / (eus[n] * 1e-6) / 1e9, 1),
                              "frac": round(eb[n] / (eus[n] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)} for n in eus}
        moe_us = sum(v for n, v in eus.items() if n.startswith("c5_"))
        if not args.only:
            line["c1_gpt2_greedy"] = gpt2_config1()
        if not args.only:
            line["extras_summary"] = {
                "c4_decode_tok_s": round(GEM_B / (eus["c4_paged_decode"] * 1e-6), 1),
                "c5_moe_block_us": round(moe_us, 2),
                "c5_moe_block_tok_s": round(MOE_T / (moe_us * 1e-6), 1),
                "c3_projections_us": round(sum(v for n, v in eus.items() if n.startswith("c3_") and n != "c3_lm_head"), 2),
            }
        del ekeep
    if not args.only and not args.no_decode_step:
        # decode tok/s: the whole TinyLlama step, at config 3's batch and
        # contexts, and for one sequence (config 3's first context)
        import numpy as np
        ctx = np.random.default_rng(2).integers(512, 4097, DEC_B)
        us32, tps32, by32 = decode_step_tok_s(DEC_B, ctx)
        us1, tps1, by1 = decode_step_tok_s(1, ctx[:1])
        line["decode_tok_s"] = round(tps32, 1)
        line["decode_step"] = {
            "model": "TinyLlama-1.1B shape (22 layers, d 2048, 32q/4kv, D 64, FFN 5632, vocab 32000), random bf16 "
                     "weights, greedy, block 16, one captured HIP graph per step",
            "batch32_config3_contexts": {"us_per_step": round(us32, 1), "tok_s": round(tps32, 1),
                                         "gbs": round(by32 / (us32 * 1e-6) / 1e9, 1)},
            "batch1_ctx%d" % int(ctx[0]): {"us_per_step": round(us1, 1), "tok_s": round(tps1, 1),
                                           "gbs": round(by1 / (us1 * 1e-6) / 1e9, 1)},
        }
    if not args.no_cpu and not args.only:
        line["cpu_baseline"] = cpu_baseline(host, bytes_per, args.cpu_tokens, args.cpu_seqs)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
