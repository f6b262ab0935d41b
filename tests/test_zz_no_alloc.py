"""The no-allocation paged decode entry point (sandy_hip_paged_attention_noalloc)
against the allocating one (sandy_hip_paged_attention) through the C ABI:
two calls in a row, the second smaller, each equal to the allocating entry
point's output and within tolerance of the oracle (src/core/TensorCalc.cpp:
1167-1314 on the pages materialised as CpuDevice.cpp:611-676 does)."""
import numpy as np
import pytest
import torch

from tests.helpers import assert_close, assert_equal, rng, to_oracle
from tests.test_gpu_attention import make_paged, oracle_paged

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


def _case(ops, oracle, seed, B, hq, hkv, D, ctx, scale):
    r = rng(seed)
    pool = sum((c + 15) // 16 for c in ctx) + 5
    q, kp, vp, table, pos = make_paged(r, B, hq, hkv, D, 16, ctx, pool, torch.bfloat16)
    args = (q, ops.PagedCache(kp), ops.PagedCache(vp), torch.from_numpy(table).cuda(), torch.from_numpy(pos).cuda())
    want_dev = ops.paged_attention(*args, scale=scale)
    out = torch.full_like(q, float("nan"))
    got = ops.paged_attention_noalloc(*args, scale=scale, out=out)
    ops.check_device_errors()
    assert got is out
    assert_equal(got, to_oracle(want_dev), "noalloc vs allocating entry point")
    sel = [0, int(np.argmax(ctx)), B - 1]
    assert_close(got[sel], oracle_paged(oracle, q[sel], kp, vp, table[sel], pos[sel], 0, scale), torch.bfloat16,
                 "noalloc vs oracle")


def test_noalloc_matches_allocating_entry_two_calls(ops, oracle):
    # config-3 geometry with multi-split sequences, then a smaller call that
    # reuses the scratch holding the first call's partials
    _case(ops, oracle, 41, 12, 32, 4, 64, [4096, 1, 700, 3000, 16, 17, 2500, 1025, 513, 4000, 64, 2048], 0.125)
    _case(ops, oracle, 42, 3, 8, 2, 256, [900, 2100, 5], 1.0)


def test_noalloc_rejects_what_does_not_fit(ops):
    from sandyrt_amd._lib import SandyError
    r = rng(43)
    B = 64
    q, kp, vp, table, pos = make_paged(r, B, 16, 1, 256, 16, [16] * B, B + 1, torch.bfloat16)
    big = torch.zeros(B, 65536 // 16, dtype=torch.int32, device="cuda")  # 65536-key tables: partials past 8 MiB
    with pytest.raises(SandyError, match="without allocation needs"):
        ops.paged_attention_noalloc(q, ops.PagedCache(kp), ops.PagedCache(vp), big, torch.from_numpy(pos).cuda())
    f32 = torch.zeros(1, 2, 1, 64, device="cuda")
    pool = torch.zeros(2, 1, 16, 64, device="cuda")
    with pytest.raises(SandyError, match="without allocation takes bf16"):
        ops.paged_attention_noalloc(f32, ops.PagedCache(pool), ops.PagedCache(pool),
                                    torch.zeros(1, 1, dtype=torch.int32, device="cuda"),
                                    torch.zeros(1, dtype=torch.int64, device="cuda"))
