"""GPU parity on the two large workloads.

Qwen2.5-7B (28 Q / 4 KV heads, GQA group 7 run natively, head_dim 128),
random-init bf16, max_batch_size 48, max_seq_len 4096: 64 requests with
prompt lengths log-uniform in [256, 4096] (seed 3) and per-request token
budgets drawn so that requests retire mid-run and the waiting ones are
admitted; 100 engine steps.  Every step's decode page table must equal the
oracle replay of the reference allocator (bit-exact), and the decode
attention of the last layer on the engine's own pool and page table must
match the fp32 oracle at two points of the run.

Qwen2.5-72B (64 Q / 8 KV heads): (a) the kernels at that shape on a pool the
size of one layer's share of the HBM left after 145 GB of weights: 48 decode
requests with contexts log-uniform in [512, 4096] (seed 4) and a ragged
causal prefill of 8 prompts with lengths uniform in [256, 2048], pages from a
seeded permutation of the whole pool, vs the fp32 oracle; (b) the engine with
random-init 72B weights (145 GB) and the page pool sized to the remaining
HBM: 48 requests decode, then 8 new prompts are prefilled in the same step as
the decode of all 56 (prefill then decode, scheduler.py:596-600); page
tables bit-exact vs the oracle replay every step and the last layer's decode
attention vs the fp32 oracle after the interleaved step.

Attention outputs are checked against the fp32 oracle by max-abs error; each
case's measured error is recorded (the session's parity table) against its
bound.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oatt
from oracle import paging as opg

pytestmark = pytest.mark.gpu


def _loguniform(g, n, lo, hi):
    x = torch.rand(n, generator=g, dtype=torch.float64) * (math.log(hi) - math.log(lo)) + math.log(lo)
    return [int(round(math.exp(v))) for v in x.tolist()]


def _decode_vs_oracle(dev, parity, pool, indptr_d, indices_d, last_d, n, hq, hkv, d, seed):
    """Decode attention through the wrapper on (pool, CSR of n rows) vs the
    oracle on the used pages copied to the host."""
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16)
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(indptr_d[: n + 1], indices_d, last_d[:n], hq, hkv, d, 16)
    out = w.run(q.to(dev), pool).float().cpu()
    ip = indptr_d[: n + 1].cpu().tolist()
    ix = indices_d[: ip[-1]].cpu()
    used, local = torch.unique(ix, return_inverse=True)
    pool_cpu = pool.index_select(0, used.to(dev)).cpu()
    ref = oatt.decode(q, pool_cpu, ip, local.tolist(), last_d[:n].cpu().tolist())
    return parity(out, ref, f"decode B={n} seed {seed}")


def _check_step(sch, res):
    dec = res["decode"]
    if dec is None:
        return 0
    n = len(dec["rids"])
    ptr = sch.d_indptr[: n + 1].cpu().tolist()
    assert ptr == dec["indptr"]
    assert sch.d_indices[: ptr[-1]].cpu().tolist() == dec["indices"]
    assert sch.d_last[:n].cpu().tolist() == dec["last_page_len"]
    assert sch.d_pos[:n].cpu().tolist() == dec["positions"]
    return n


def test_config4_qwen7b_b48_retire_and_admit(dev, parity):
    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model

    cfg = PRESETS["qwen2.5-7b"]
    model = Model(cfg, dev, seed=3, max_positions=4096 + 16)
    g = torch.Generator().manual_seed(3)
    n_req = 64
    lens = _loguniform(g, n_req, 256, 4096)
    budgets = torch.randint(8, 121, (n_req,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lens]
    sch = Scheduler(model, max_batch_size=48, max_seq_len=4096, seed=3)
    trace = opg.SchedulerTrace(48, 4096, 16, max_num_pages=sch.kv.max_num_pages)
    reqs = [Request(str(i), p, budgets[i], 0.0) for i, p in enumerate(prompts)]
    for i, r in enumerate(reqs):
        sch.submit(r)
        trace.submit(opg.TraceRequest(i, lens[i], budgets[i]))
    admitted_late = retired = 0
    checks = []
    for step in range(100):
        if not sch.has_work():
            break
        sch.step()
        res = trace.step()
        if step > 0:
            admitted_late += len(res["admitted"])
        retired += len(res["released"])
        n = _check_step(sch, res)
        if step in (30, 80) and n:
            checks.append(_decode_vs_oracle(dev, parity, sch.kv.kv_data[cfg.num_hidden_layers - 1], sch.d_indptr,
                                            sch.d_indices, sch.d_last, n, cfg.num_attention_heads,
                                            cfg.num_key_value_heads, cfg.head_dim, seed=step))
    assert sch.pt.error_word() == 0
    assert admitted_late > 0 and retired > 0
    assert len(checks) == 2
    for r, b in zip(reqs, budgets):
        if r.status.value == "finished":
            assert len(r.generated_tokens) == b or r.current_position >= 4096


def test_config5_qwen72b_shapes_large_pool(dev, parity):
    """Kernels at the 72B head shape; pool pages spread over a 1.5 GB layer pool."""
    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    hq, hkv, d, ps = 64, 8, 128, 16
    num_pages = 24_000                               # 1.57 GB of K/V per layer (80 layers: 126 GB)
    g = torch.Generator().manual_seed(4)
    dec_lens = _loguniform(g, 48, 512, 4096)
    pre_lens = torch.randint(256, 2049, (8,), generator=g).tolist()
    perm = torch.randperm(num_pages - 1, generator=g)
    gd = torch.Generator(device=dev).manual_seed(4)
    pool = torch.randn(num_pages, 2, ps, hkv, d, device=dev, generator=gd).to(torch.bfloat16)

    def csr(lens, start):
        npg = [math.ceil(n / ps) for n in lens]
        ptr = [0]
        for n in npg:
            ptr.append(ptr[-1] + n)
        ix = perm[start: start + ptr[-1]].to(torch.int32)
        last = [n - (p - 1) * ps for n, p in zip(lens, npg)]
        return ptr, ix, last, start + ptr[-1]

    ip, ix, last, used = csr(dec_lens, 0)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    _decode_vs_oracle(dev, parity, pool, i32(ip), ix.to(dev), i32(last), 48, hq, hkv, d, seed=41)

    pip, pix, plast, _ = csr(pre_lens, used)
    qo = [0]
    for n in pre_lens:
        qo.append(qo[-1] + n)
    q = torch.randn(qo[-1], hq, d, generator=g).to(torch.bfloat16)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(i32(qo), i32(pip), pix.to(dev), i32(plast), hq, hkv, d, ps, causal=True)
    out = w.run(q.to(dev), pool).float().cpu()
    pused, plocal = torch.unique(pix, return_inverse=True)
    pool_cpu = pool.index_select(0, pused.to(dev)).cpu()
    ref = oatt.prefill(q, pool_cpu, qo, pip, plocal.tolist(), plast, causal=True)
    parity(out, ref, "prefill 8 prompts")


def test_config5_qwen72b_engine_48_decoding_8_prefilled(dev, parity):
    """Config 5 at its size: 48 requests (prompts log-uniform in [512, 4096],
    admitted 8 per step) decode; then 8 new prompts (U[256, 2048]) are
    prefilled in the same step as the decode of all 56 (prefill then decode,
    scheduler.py:596-600).  Page tables bit-exact vs the oracle replay every
    step; the last layer's decode attention vs the fp32 oracle after the
    interleaved step; every request finishes with its token budget."""
    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model, kv_pool_bytes_per_page

    cfg = PRESETS["qwen2.5-72b"]
    model = Model(cfg, dev, seed=4, max_positions=4096 + 64 + 16)
    torch.cuda.synchronize()
    assert model.weight_bytes() > 140e9
    free, _ = torch.cuda.mem_get_info(dev)
    num_pages = int((free - 24 * 2**30) // kv_pool_bytes_per_page(cfg, 16))   # the rest of the HBM, 24 GiB spare
    assert num_pages > 56 * 260
    g = torch.Generator().manual_seed(4)
    dec_lens = _loguniform(g, 48, 512, 4096)
    pre_lens = torch.randint(256, 2049, (8,), generator=g).tolist()
    lens = dec_lens + pre_lens
    budgets = [14] * 48 + [4] * 8
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lens]
    sch = Scheduler(model, max_batch_size=56, max_seq_len=4096 + 64, num_pages=num_pages, seed=4)
    trace = opg.SchedulerTrace(56, 4096 + 64, 16, max_num_pages=sch.kv.max_num_pages)
    reqs = [Request(str(i), p, budgets[i], 0.0) for i, p in enumerate(prompts)]
    step = 0
    checked = False
    while step < 40 and (step < 8 or sch.has_work()):
        batch = range(8 * step, 8 * step + 8) if step < 6 else range(48, 56) if step == 7 else ()
        for i in batch:
            sch.submit(reqs[i])
            trace.submit(opg.TraceRequest(i, lens[i], budgets[i]))
        sch.step()
        res = trace.step()
        n = _check_step(sch, res)
        if step == 6:
            assert n == 48 and not res["prefill"]
        if step == 7:   # prefill of the 8 new prompts, then decode of all 56, in one step
            assert len(res["prefill"]) == 8 and n == 56
            _decode_vs_oracle(dev, parity, sch.kv.kv_data[cfg.num_hidden_layers - 1], sch.d_indptr, sch.d_indices,
                              sch.d_last, n, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                              seed=72)
            checked = True
        step += 1
    assert checked and not sch.has_work()
    assert sch.pt.error_word() == 0
    assert [len(r.generated_tokens) for r in reqs] == budgets
