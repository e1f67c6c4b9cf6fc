"""The decode entry point that allocates nothing (mi_decode_static) against
the workspace entry points (mi_decode_plan + mi_decode_run).

Both run the same kernels on the same plan, so the outputs must be identical
bit for bit, on two calls in a row (the second with a smaller batch, so stale
work-list entries of the first call must not leak into it).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from tests.helpers import make_paged_batch, to_dev

pytestmark = pytest.mark.gpu


def _with_workspace(lib, dev, pool, q, ip, ix, lp, hq, hkv, d):
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    s = torch.cuda.current_stream(dev).cuda_stream
    b = q.shape[0]
    assert lib.mi_decode_plan(ws.data_ptr(), ws.numel(), ip.data_ptr(), ix.data_ptr(), lp.data_ptr(), b, hq, hkv,
                              d, 16, 0, s) == 0
    assert lib.mi_decode_run(ws.data_ptr(), ws.numel(), q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(),
                             pool.shape[0], ix.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1), b, hq, hkv,
                             d, 16, 0.0, 0, s) == 0
    return out


def _static(lib, dev, pool, q, ip, ix, lp, hq, hkv, d):
    out = torch.full_like(q, float("nan"))
    s = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.mi_decode_static(q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(), pool.shape[0],
                              ip.data_ptr(), ix.data_ptr(), lp.data_ptr(), out.data_ptr(), out.stride(0),
                              out.stride(1), q.shape[0], hq, hkv, d, 16, 0.0, s)
    assert rc == 0, lib.mi_last_error()
    return out


@pytest.mark.parametrize("hq,hkv,d,big,small", [
    (32, 8, 128, [600, 1000, 37, 260, 129, 17, 800, 333], [64, 9, 500]),   # Mistral-7B heads
    (28, 4, 128, [4000, 300, 1700, 2200], [1, 15]),                         # Qwen2.5-7B, group 7
    (14, 2, 64, [17, 64, 203, 511], [100]),                                  # Qwen2.5-0.5B
])
def test_static_matches_workspace_twice(dev, lib, hq, hkv, d, big, small):
    for k, lens in enumerate((big, small)):
        b = make_paged_batch(lens, hq, hkv, d, seed=40 + k)
        pool, q, ip, ix, lp = to_dev(b, dev)
        want = _with_workspace(lib, dev, pool, q, ip, ix, lp, hq, hkv, d)
        got = _static(lib, dev, pool, q, ip, ix, lp, hq, hkv, d)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {k}: static differs from the workspace path"


def test_static_rejects_a_batch_beyond_its_scratch(dev, lib):
    """A work list over the static array's capacity is an error, not a write past it."""
    hq, hkv, d, bsz = 64, 8, 256, 4096
    q = torch.zeros(bsz, hq, d, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(2, 2, 16, hkv, d, dtype=torch.bfloat16, device=dev)
    ip = torch.zeros(bsz + 1, dtype=torch.int32, device=dev)
    ix = torch.zeros(1, dtype=torch.int32, device=dev)
    lp = torch.ones(bsz, dtype=torch.int32, device=dev)
    rc = lib.mi_decode_static(q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(), 2, ip.data_ptr(),
                              ix.data_ptr(), lp.data_ptr(), q.data_ptr(), q.stride(0), q.stride(1), bsz, hq, hkv, d,
                              16, 0.0, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == -3  # MI_ERR_WORKSPACE
    assert b"static scratch" in lib.mi_last_error()
