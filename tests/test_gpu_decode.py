"""GPU parity: split-K paged decode attention vs the fp32 oracle.

Tolerance (the ``parity`` fixture): max-abs 2e-2 against the fp32 oracle on
bf16 inputs, and max |out - ref| / max(1, |ref|) <= 1.2e-2 -- three bf16
roundings (P, split partials, output) of up to 2^-8 each.  Each case's errors are
printed in the session's parity table.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oatt
from tests.helpers import make_paged_batch, to_dev

pytestmark = pytest.mark.gpu


def _wrapper(dev, ws_mb=128):
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper

    ws = torch.empty(ws_mb << 20, dtype=torch.uint8, device=dev)
    return BatchDecodeWithPagedKVCacheWrapper(ws, kv_layout="NHD")


def _decode(dev, batch, hq, hkv, d, w=None):
    pool, q, ip, ix, lp = to_dev(batch, dev)
    w = w or _wrapper(dev)
    w.plan(ip, ix, lp, hq, hkv, d, 16, pos_encoding_mode="NONE", q_data_type=torch.bfloat16,
           data_type=torch.bfloat16)
    out = w.run(q, pool)
    torch.cuda.synchronize()
    return out.float().cpu()


def _ref(batch):
    return oatt.decode(batch["q"], batch["pool"], batch["indptr"], batch["indices"].tolist(), batch["last"])


def test_config1_qwen05_heads(dev, parity):
    """Qwen2.5-0.5B heads (14/2, d=64), contexts {17, 64, 203, 511}, seed 0."""
    b = make_paged_batch([17, 64, 203, 511], 14, 2, 64, num_pages=128, seed=0)
    parity(_decode(dev, b, 14, 2, 64), _ref(b))


@pytest.mark.parametrize("hq,hkv,d", [
    (32, 8, 128),   # Mistral-7B, group 4
    (28, 4, 128),   # Qwen2.5-7B, group 7 (no padding)
    (64, 8, 128),   # Qwen2.5-72B, group 8
    (14, 2, 64),    # Qwen2.5-0.5B, group 7
    (8, 8, 128),    # group 1
    (12, 4, 64),    # group 3
    (10, 2, 128),   # group 5
    (12, 2, 128),   # group 6
    (4, 2, 64),     # group 2
    (16, 4, 256),   # head_dim 256
    (6, 3, 128),    # odd kv_heads: one-wave workgroups
    (8, 1, 128),    # one KV head (MQA), group 8
    (4, 1, 64),     # one KV head, head_dim 64
])
def test_shapes_ragged(dev, parity, hq, hkv, d):
    # eight requests: the head_dim 64 shapes get two lane groups per unit
    # (the plan aims at two units per CU), the others one
    lens = [1, 15, 16, 17, 33, 100, 257, 700]
    b = make_paged_batch(lens, hq, hkv, d, seed=hq * 7 + d)
    parity(_decode(dev, b, hq, hkv, d), _ref(b))


def test_mistral_b32_ragged(dev, parity):
    """Mistral-7B decode shape: B=32, contexts U[128,1024] + 25, seed 2."""
    g = torch.Generator().manual_seed(2)
    lens = (torch.randint(128, 1025, (32,), generator=g) + 25).tolist()
    b = make_paged_batch(lens, 32, 8, 128, seed=2)
    parity(_decode(dev, b, 32, 8, 128), _ref(b))


@pytest.mark.parametrize("ctx", [4096, 16384])
def test_long_context_many_splits(dev, parity, ctx):
    """One request: the split-K merge across up to 64 splits."""
    b = make_paged_batch([ctx], 28, 4, 128, seed=ctx)
    parity(_decode(dev, b, 28, 4, 128), _ref(b))


@pytest.mark.parametrize("lens", [[16384], [3000, 1, 47, 2049], [33] * 7])
def test_head_dim_64_lane_groups(dev, parity, lens):
    """Head_dim 64 with few requests: two lane groups per unit deal the
    unit's page pairs alternately and merge in LDS.  Long units span several
    64-page id groups; odd pair counts leave one group a masked pair; a
    one-page request gives one group no page at all; ragged sets mix them."""
    b = make_paged_batch(lens, 14, 2, 64, seed=len(lens) * 31 + lens[0])
    parity(_decode(dev, b, 14, 2, 64), _ref(b))


@pytest.mark.parametrize("sm_scale", [0.3, 0.02])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64)])
def test_explicit_softmax_scale(dev, parity, sm_scale, hq, hkv, d):
    """plan(sm_scale=...) replaces 1/sqrt(head_dim): a sharper (0.3) and a
    flatter (0.02) softmax against the oracle at the same scale."""
    lens = [1, 40, 300, 2000]
    b = make_paged_batch(lens, hq, hkv, d, seed=57)
    pool, q, ip, ix, lp = to_dev(b, dev)
    w = _wrapper(dev)
    w.plan(ip, ix, lp, hq, hkv, d, 16, sm_scale=sm_scale)
    out = w.run(q, pool).float().cpu()
    ref = oatt.decode(b["q"], b["pool"], b["indptr"], b["indices"].tolist(), b["last"], sm_scale=sm_scale)
    parity(out, ref)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64)])
def test_large_scores_lazy_rescale(dev, parity, hq, hkv, d):
    """q and K scaled by 6: scores spread over tens of natural
    units, so the running max grows past the lazy-rescale margin (2^8 in the
    exp2 domain) many times within a unit and across splits."""
    lens = [5, 300, 2000, 4100]
    b = make_paged_batch(lens, hq, hkv, d, seed=61)
    b["pool"][:, 0] = (b["pool"][:, 0].float() * 6).to(torch.bfloat16)
    # V / 4 keeps the near one-hot outputs (single V entries) near unit size,
    # where the max-abs bound applies
    b["pool"][:, 1] = (b["pool"][:, 1].float() / 4).to(torch.bfloat16)
    b["q"] = (b["q"].float() * 6).to(torch.bfloat16)
    out = _decode(dev, b, hq, hkv, d)
    assert torch.isfinite(out).all()
    parity(out, _ref(b))


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 2, 64)])
def test_one_long_request_among_short_ones(dev, parity, hq, hkv, d):
    """A 32,768-token request among forty 16-token ones: the plan's uniform
    item length gives the long request well over 64 splits, so its last
    arriver merges them in several rounds of 64."""
    lens = [32768] + [16] * 40
    b = make_paged_batch(lens, hq, hkv, d, seed=63)
    w = _wrapper(dev)
    out = _decode(dev, b, hq, hkv, d, w=w)
    # the plan's first work item (128 bytes after a 256-byte header) is split 0
    # of the long request; word 29 of an item is its split count
    nsplit = int(w._ws[256:384].view(torch.int32)[29])
    assert nsplit > 64
    parity(out, _ref(b))


def test_empty_request_gives_zero(dev, parity):
    b = make_paged_batch([0, 40], 8, 2, 64, seed=5)
    out = _decode(dev, b, 8, 2, 64)
    assert torch.count_nonzero(out[0]) == 0
    parity(out[1], _ref(b)[1])


def test_single_token_returns_v0(dev):
    """kv_len = 1: softmax weight 1 on the only token, so out == V[0] exactly."""
    b = make_paged_batch([1, 1, 1], 32, 8, 128, seed=11)
    out = _decode(dev, b, 32, 8, 128)
    for r in range(3):
        page = int(b["indices"][r])
        v0 = b["pool"][page, 1, 0].float()  # [hkv, d]
        assert torch.equal(out[r], v0.repeat_interleave(4, dim=0))


def test_constant_keys_average_values(dev):
    """Identical keys give uniform weights: out == mean(V) over the context."""
    b = make_paged_batch([48, 130], 16, 4, 128, seed=13)
    b["pool"][:, 0] = b["pool"][0, 0, 0]  # every key row identical
    out = _decode(dev, b, 16, 4, 128)
    from oracle.paging import gather_kv

    for r in range(2):
        _, v = gather_kv(b["pool"], b["indptr"], b["indices"].tolist(), b["last"], r)
        mean = v.float().mean(dim=0).repeat_interleave(4, dim=0)
        assert (out[r] - mean).abs().max().item() < 1e-2


def test_plan_once_run_many_layers(dev, parity):
    """One plan serves several layer pools (the per-step pattern)."""
    lens = [300, 17, 900, 64]
    w = _wrapper(dev)
    batches = [make_paged_batch(lens, 32, 8, 128, seed=100 + i) for i in range(3)]
    # same page table for every layer
    for x in batches[1:]:
        x["indices"], x["indptr"], x["last"] = batches[0]["indices"], batches[0]["indptr"], batches[0]["last"]
    pool0, q0, ip, ix, lp = to_dev(batches[0], dev)
    w.plan(ip, ix, lp, 32, 8, 128, 16)
    for x in batches:
        out = w.run(x["q"].to(dev), x["pool"].to(dev)).float().cpu()
        parity(out, _ref(x))


def test_strided_q_and_out(dev, parity):
    """q as a column slice of a fused projection; out written into a view."""
    lens = [40, 123]
    b = make_paged_batch(lens, 16, 4, 64, seed=21)
    pool, _, ip, ix, lp = to_dev(b, dev)
    big = torch.zeros(len(lens), 24 * 64, dtype=torch.bfloat16, device=dev)
    big[:, :16 * 64] = b["q"].reshape(len(lens), -1).to(dev)
    qv = big[:, :16 * 64].view(len(lens), 16, 64)
    outbuf = torch.zeros(len(lens), 20 * 64, dtype=torch.bfloat16, device=dev)
    ov = outbuf[:, 64:17 * 64].view(len(lens), 16, 64)
    w = _wrapper(dev)
    w.plan(ip, ix, lp, 16, 4, 64, 16)
    w.run(qv, pool, out=ov)
    torch.cuda.synchronize()
    parity(ov.float().cpu(), _ref(b))
    assert torch.count_nonzero(outbuf[:, :64]) == 0


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128), (28, 4, 128)])
def test_head_major_q_and_out_views(dev, parity, hq, hkv, d):
    """q and out as head-major views ([heads, batch, head_dim] storage seen
    as [batch, heads, head_dim]: a head stride of batch * head_dim, larger
    than the row stride)."""
    lens = [40, 123, 1, 700, 16, 33]
    b = make_paged_batch(lens, hq, hkv, d, seed=23)
    pool, q, ip, ix, lp = to_dev(b, dev)
    B = len(lens)
    q_hm = q.transpose(0, 1).contiguous().transpose(0, 1)
    out_hm = torch.full((hq, B, d), float("nan"), dtype=torch.bfloat16, device=dev).transpose(0, 1)
    assert q_hm.stride() == (d, B * d, 1) and out_hm.stride() == q_hm.stride()
    w = _wrapper(dev)
    w.plan(ip, ix, lp, hq, hkv, d, 16)
    w.run(q_hm, pool, out=out_hm)
    torch.cuda.synchronize()
    got = out_hm.float().cpu()
    assert torch.isfinite(got).all()
    parity(got, _ref(b))


def test_graph_replay_after_replan(dev, parity):
    """run() captured once replays correctly after every later plan()."""
    hq, hkv, d = 32, 8, 128
    w = _wrapper(dev)
    cap = 256
    ip = torch.zeros(5, dtype=torch.int32, device=dev)
    ix = torch.zeros(cap, dtype=torch.int32, device=dev)
    lp = torch.ones(4, dtype=torch.int32, device=dev)
    q = torch.zeros(4, hq, d, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(300, 2, 16, hkv, d, dtype=torch.bfloat16, device=dev)
    out = torch.zeros(4, hq, d, dtype=torch.bfloat16, device=dev)
    first = make_paged_batch([16, 16, 16, 16], hq, hkv, d, num_pages=300, seed=1)
    ip.copy_(torch.tensor(first["indptr"], dtype=torch.int32))
    ix[:4].copy_(first["indices"])
    w.plan(ip, ix, lp, hq, hkv, d, 16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w.run(q, pool, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        w.run(q, pool, out=out)
    for seed, lens in [(2, [100, 5, 700, 33]), (3, [1, 1000, 64, 250]), (4, [3000, 1, 2, 17])]:
        b = make_paged_batch(lens, hq, hkv, d, num_pages=300, seed=seed)
        pool.copy_(b["pool"])
        q.copy_(b["q"])
        ip.copy_(torch.tensor(b["indptr"], dtype=torch.int32))
        ix[: b["indices"].numel()].copy_(b["indices"])
        lp.copy_(torch.tensor(b["last"], dtype=torch.int32))
        w.plan(ip, ix, lp, hq, hkv, d, 16)
        graph.replay()
        torch.cuda.synchronize()
        got = out.float().cpu()
        eager = w.run(q, pool).float().cpu()
        assert torch.equal(got, eager)
        parity(got, _ref(b), f"seed {seed}")


def test_rejects_unsupported(dev):
    w = _wrapper(dev)
    ip = torch.tensor([0, 1], dtype=torch.int32, device=dev)
    ix = torch.zeros(1, dtype=torch.int32, device=dev)
    lp = torch.ones(1, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        w.plan(ip, ix, lp, 32, 8, 96, 16)  # head_dim 96 not built
    with pytest.raises(ValueError):
        w.plan(ip, ix, lp, 18, 2, 128, 16)  # group 9
    with pytest.raises(ValueError):
        w.plan(ip, ix, lp, 32, 8, 128, 16, pos_encoding_mode="ROPE_LLAMA")
    with pytest.raises(RuntimeError):
        from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper

        small = BatchDecodeWithPagedKVCacheWrapper(torch.empty(1024, dtype=torch.uint8, device=dev))
        small.plan(ip, ix, lp, 32, 8, 128, 16)


def test_golden_fixture_config1(dev, parity):
    """The kernel against the committed fp32 output of the config-1 case."""
    from safetensors.torch import load_file

    from tests.test_golden import FIX, load_pool

    t = load_file(str(FIX))
    w = _wrapper(dev)
    w.plan(t["indptr"].to(dev), t["page_ids"].to(dev), t["last_page_len"].to(dev), 14, 2, 64, 16)
    out = w.run(t["q"].to(dev), load_pool(t).to(dev)).float().cpu()
    parity(out, t["out_fp32"])


@pytest.mark.parametrize("fill", ["ones", "random", "larger_plan"])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (6, 3, 128)])
def test_work_items_past_the_plan_are_ignored(dev, parity, fill, hq, hkv, d):
    """Every wave of the run reads its first work item before it knows the
    plan's unit count; the items past that count hold whatever the workspace
    held (all bits set, random bytes, or a larger earlier plan's items) and
    must not be used.  A small batch leaves most of the grid past the count."""
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper

    ws = torch.empty(128 << 20, dtype=torch.uint8, device=dev)
    if fill == "ones":
        ws.fill_(0xFF)
    elif fill == "random":
        ws.random_(0, 256, generator=torch.Generator(device=dev).manual_seed(7))
    w = BatchDecodeWithPagedKVCacheWrapper(ws, kv_layout="NHD")
    if fill == "larger_plan":  # its items stay in the workspace past the small plan's
        _decode(dev, make_paged_batch([400] * 40, hq, hkv, d, seed=31), hq, hkv, d, w=w)
    b = make_paged_batch([33, 1, 260], hq, hkv, d, seed=32)
    parity(_decode(dev, b, hq, hkv, d, w=w), _ref(b))


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (6, 3, 128)])
def test_stale_rows_past_the_end_are_not_read(dev, parity, hq, hkv, d):
    """NaN in every pool row past each request's length on its last page."""
    lens = [37, 100, 5, 250, 1000]
    b = make_paged_batch(lens, hq, hkv, d, seed=22)
    pool = b["pool"].clone()
    idx = b["indices"].tolist()
    for r in range(len(lens)):
        hi = b["indptr"][r + 1]
        if b["last"][r] < 16:
            pool[idx[hi - 1], :, b["last"][r]:] = float("nan")
    b = {**b, "pool": pool}
    out = _decode(dev, b, hq, hkv, d)
    assert torch.isfinite(out).all()
    parity(out, _ref(b))


@pytest.mark.parametrize("B,hq,hkv,d,max_ctx", [
    (700, 32, 8, 128, 80),   # units > one resident round: the run's grid-stride rounds
    (1100, 8, 2, 64, 40),    # more requests than the plan's 1024-thread scan takes at once; head_dim 64
                             # with a full round of units, so one lane group per unit
])
def test_large_batches(dev, parity, B, hq, hkv, d, max_ctx):
    g = torch.Generator().manual_seed(B)
    lens = torch.randint(1, max_ctx + 1, (B,), generator=g).tolist()
    b = make_paged_batch(lens, hq, hkv, d, seed=B)
    parity(_decode(dev, b, hq, hkv, d), _ref(b))


@pytest.mark.parametrize("hq,hkv,d,lo,hi", [
    (32, 8, 128, 153, 1049),    # Mistral-7B decode batch: items of 6-7 pages
    (64, 8, 128, 512, 4096),    # Qwen2.5-72B heads: items of 16-29 pages, some past the 24 inline page ids
    (14, 2, 64, 512, 4096),     # Qwen2.5-0.5B heads: head_dim 64, two lane groups merged in LDS
])
def test_repeated_runs_are_bit_identical(dev, parity, hq, hkv, d, lo, hi):
    """Units finish in a different order on every launch and whichever split
    of a request arrives last merges: the output must not depend on which, so
    12 launches of one plan give bit-identical outputs, within the oracle's
    bound.  Items of odd and even page counts, with and without page groups
    past the inline ids, all occur here."""
    g = torch.Generator().manual_seed(hq + lo)
    lens = torch.exp(torch.empty(48).uniform_(math.log(lo), math.log(hi), generator=g)).round().int().tolist()
    b = make_paged_batch(lens, hq, hkv, d, seed=hq + d)
    pool, q, ip, ix, lp = to_dev(b, dev)
    w = _wrapper(dev)
    w.plan(ip, ix, lp, hq, hkv, d, 16)
    outs = [w.run(q, pool).clone() for _ in range(12)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    parity(outs[0].float().cpu(), _ref(b))
