"""Benchmark: decode tok/s and decode-attention HBM GB/s, Mistral-7B, B=32, one GPU.

Workload (random-initialised Mistral-7B architecture, bf16): 32 concurrent
requests with prompt lengths uniform in [128, 1024] and random token ids
(seed 2); even requests greedy, odd ones temperature 0.7 / top-p 0.9;
page_size 16; one hipGraph per decode batch size.  All prompts are admitted
and prefilled (one ragged batch) before timing.

A "step" is one full decode step of the 32-request batch: the device
page-table step with the decode plan (one launch), graph replay (32 layers:
GEMMs, RoPE, KV append, split-K paged attention, sampler), the feedback of
the sampled ids and, once per window of ``--decode-window`` steps,
end-of-sequence detection on the GPU and the read-back of the window's ids.
The engine is pipelined: the next window is enqueued before the host waits
for the previous window's ids.  ``value`` is decoded tokens per second over
exactly ``--steps`` timed steps (the last window read back inside the timed
region); ``decode_tok_s_one_step_per_round_trip`` is the same over the next
``--steps`` steps with a read-back after every step.

``roofline`` is measured on the decode step's attention launch, the kernel
the decode path runs per layer (mi_decode_rope_append_run: RoPE of q and k,
the new K/V appended to its slot, split-K paged attention): after the timed
steps, with the CSR of the next decode step (each request's next position
counted, so the launch writes the slot that step writes anyway), the 32
layers' launches (the batch's real page tables and pools, one pool per layer
so nothing is served from the 256 MB Infinity Cache; random qkv rows) are
captured in a hipGraph, replayed ``--attn-iters`` times on the current stream
and bracketed with HIP events; achieved = algorithmic bytes per launch /
average launch time.  Algorithmic bytes per launch (kv_len counts the new
token, whose K/V comes from the qkv row instead of the pool):
sum_b kv_len_b * H_kv * D * 2 (K,V) * 2 B + 2 * B * H_q * D * 2 B (q, out)
+ 4 B * ((B+1) + sum_b npages_b + B) (indptr, indices, last_page_len)
+ B * H_kv * D * 2 * 2 B (new K, V written) + B * D * 2 * 2 B (cos, sin rows).
``decode_attn_alone`` times attention alone (mi_decode_run) on the same CSR
with the first three terms.

``roofline.traffic`` is the HBM bytes per launch that rocprofv3 counted for
this same attention leg (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled
by what the counter reads for a 1 GiB device copy), from
profiles/decode_attn_traffic.json: as counted when the run's mean context is
the one the counters were taken at, otherwise the counted ratio of HBM bytes
to algorithmic bytes times this launch's algorithmic bytes
(``traffic_basis`` says which); null for another model or batch.

``cpu_baseline`` (tok/s, the metric's unit) continues the same B=32 batch on
the host cores through the oracle's model forward: the weights and the used
pages of every layer's pool are copied to the host, then decode steps run in
fp32 torch with the oracle's gather-based paged attention (greedy), median of
up to 8 steps.  The thread count is the CPUs the process may use (affinity,
cgroup quota, OMP_NUM_THREADS), and the counts behind it are reported.
``cpu_baseline_legs`` adds the oracle's attention alone on one layer of the
batch (GB/s).

``decode_attn_other_workloads`` times the same launch (and attention alone
beside it), the same way, on the Qwen2.5-7B (B=48, 28/4 heads) and
Qwen2.5-72B (B=48, 64/8 heads) decode shapes with their log-uniform contexts,
and on the Qwen2.5-0.5B head shape (14/2 heads, head_dim 64) at B=32 with
contexts uniform in [512, 4096] (synthetic pools).

``config1_decode_attn``: the committed config-1 fixture timed on the HIP
kernel and on the CPU oracle, and the kernel's error against the fixture.
``config2_end_to_end``: Qwen2.5-0.5B, 8 requests admitted every 5 steps, 50
greedy tokens each, on the GPU engine and the same schedule on the CPU
through the oracle's model forward.  ``config4_end_to_end``: Qwen2.5-7B,
B<=48, 64 requests retiring and admitted over 100 engine steps.
``config5_end_to_end``: Qwen2.5-72B (145 GB of weights), 48 decoding requests,
then one step that prefills 8 new prompts and decodes all 56.  ``--legs``
selects these legs (main always runs).

``vs_baseline`` is the served aggregate at 32 concurrent requests over the
reference's published 1,532 tok/s at 32 concurrent (README.md:56): the same
measurement on other hardware, random weights and a synthetic tokenizer.

``served`` reproduces the reference's published serving measurement
(README.md:50-70, benchmark.py): the OpenAI-compatible server in a child
process (random weights, synthetic tokenizer) and the streaming client at 2,
20 and 32 concurrent greedy requests, max_tokens 50, 3 runs each: TTFT, T2T
and aggregate tok/s (content chunks / run wall time, prefill included) --
the figures the reference's 1,532 tok/s at 32 concurrent is quoted as.

``path_kernels`` times the other kernels of the path on the same state, each
as repeated launches captured in one hipGraph and replayed between HIP events: the ragged
causal prefill attention of the 32 prompts for one layer (MFMA bound:
flops = sum_b 4 * H_q * D * L_b (L_b + 1) / 2, against 2.5 PFLOP/s bf16) and
of 8 prompts U[256,2048] at the Qwen2.5-72B head shape, the separate
RoPE + KV append of 32 decode rows (into a copy of layer 0's pool; the decode
step folds it into its attention launch), the
prefill-sized appends of the prompts' rows into their pages (HBM bound against
8 TB/s; fused RoPE + append bytes = 2 * T * (H_q + 2 H_kv) * D * 2 B (q, k, v
read and written) + 2 * T * D * 2 B (cos / sin rows) + index ints; plain
append bytes = 2 * 2 * T * H_kv * D * 2 B + index ints) and the sampler for
the 32 rows and for 48 rows of the Qwen vocabulary (152,064) with top-p
(latency bound: microseconds).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_attn_traffic.json"
PUBLISHED_TOKS = 1532.0  # reference README.md:56, H100, 32 concurrent, aggregate tok/s


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_us(fn, iters: int, warm_ms: float = 25.0, reps: int = 3) -> float:
    """GPU microseconds per call of ``fn``: ``iters`` calls captured in one
    hipGraph (so host launch cost is excluded) and replayed on the current
    stream after warm-up calls on a side stream.  The graph is first replayed
    untimed for about ``warm_ms`` of GPU time -- after an idle stretch (the
    CPU legs) the GPU's clocks take a few milliseconds of work to come back
    up, and a kernel timed inside that ramp reads up to ~25 % slow (ragged
    prefill of the 32 bench prompts: 202 -> 163 us over the first 4 ms) --
    then ``reps`` replays are timed between HIP events and the median is
    returned."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    e1.synchronize()
    one_ms = max(e0.elapsed_time(e1), 1e-3)
    for _ in range(min(200, int(warm_ms / one_ms))):
        graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0.record()
        graph.replay()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1) * 1000 / iters)
    return sorted(times)[len(times) // 2]


def path_kernel_times(sch, cfg, reqs, lens, dev) -> dict:
    """The path's other kernels on the bench's real state (see module doc)."""
    import torch

    from minimal_inference_amd.page import rope_append_paged_kv_cache
    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    B = len(reqs)
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    res = {}
    # ragged causal prefill over the prompts' own pages (first ceil(L/16) pages of each request)
    ip = sch.d_indptr[: B + 1].cpu().tolist()
    ix = sch.d_indices[: ip[-1]].cpu()
    pages = [ix[ip[b]: ip[b] + math.ceil(lens[b] / 16)] for b in range(B)]
    p_indptr = torch.tensor([0] + list(torch.tensor([len(x) for x in pages]).cumsum(0).tolist()),
                            dtype=torch.int32, device=dev)
    p_indices = torch.cat(pages).to(dev)
    p_last = torch.tensor([n - (math.ceil(n / 16) - 1) * 16 for n in lens], dtype=torch.int32, device=dev)
    qo = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32, device=dev)
    total = sum(lens)
    q = torch.randn(total, hq, d, device=dev, dtype=torch.bfloat16)
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=dev)
    pw = BatchPrefillWithPagedKVCacheWrapper(ws)
    pw.plan(qo, p_indptr, p_indices, p_last, hq, hkv, d, 16, causal=True, max_total_q=total)
    out = torch.empty_like(q)
    us = time_us(lambda: pw.run(q, sch.kv.kv_data[0], out=out), 20)
    flops = sum(4 * hq * d * (L * (L + 1) // 2) for L in lens)
    res["prefill_attn"] = {"us": round(us, 2), "tflops": round(flops / us / 1e6, 1),
                           "frac_of_2500": round(flops / us / 1e6 / 2500, 4), "query_rows": total}
    # decode-step fused RoPE + append for the batch's rows (writes the next position's slot)
    qkv = torch.randn(B, (hq + 2 * hkv) * d, device=dev, dtype=torch.bfloat16)
    model = sch.model
    pool_copy = sch.kv.kv_data[0].clone()  # the timed appends overwrite cached slots
    us = time_us(lambda: rope_append_paged_kv_cache(qkv, hq, hkv, sch.d_pos[:B], model.cos, model.sin,
                                                    sch.d_batch[:B], sch.d_pos[:B], pool_copy,
                                                    sch.d_indices, sch.d_indptr[: B + 1], sch.d_last[:B]), 200)
    res["rope_append_decode"] = {"us": round(us, 2), "rows": B}
    # prefill-sized appends (HBM bound): the prompts' rows into their own pages, as the ragged
    # prefill writes them -- fused RoPE + append of the qkv rows, and the plain K / V append
    from minimal_inference_amd.page import append_paged_kv_cache

    p_batch = torch.cat([torch.full((n,), b, dtype=torch.int32) for b, n in enumerate(lens)]).to(dev)
    p_pos = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens]).to(dev)
    p_qkv = torch.randn(total, (hq + 2 * hkv) * d, device=dev, dtype=torch.bfloat16)
    p_q = torch.empty(total, hq, d, device=dev, dtype=torch.bfloat16)
    ints = 4 * ((B + 1) + int(p_indices.numel()) + B)
    nbytes = 2 * total * (hq + 2 * hkv) * d * 2 + 2 * total * d * 2 + 4 * 3 * total + ints
    us = time_us(lambda: rope_append_paged_kv_cache(p_qkv, hq, hkv, p_pos, model.cos, model.sin, p_batch, p_pos,
                                                    pool_copy, p_indices, p_indptr, p_last, q_out=p_q), 20)
    res["rope_append_prefill"] = {"us": round(us, 2), "rows": total, "mb": round(nbytes / 1e6, 1),
                                  "gbps": round(nbytes / us / 1e3, 1),
                                  "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBPS, 4)}
    p_k = p_qkv[:, hq * d:(hq + hkv) * d].contiguous().view(total, hkv, d)
    p_v = p_qkv[:, (hq + hkv) * d:].contiguous().view(total, hkv, d)
    nbytes = 2 * 2 * total * hkv * d * 2 + 4 * 2 * total + ints
    us = time_us(lambda: append_paged_kv_cache(p_k, p_v, p_batch, p_pos, pool_copy, p_indices, p_indptr, p_last), 20)
    res["append_prefill"] = {"us": round(us, 2), "rows": total, "mb": round(nbytes / 1e6, 1),
                             "gbps": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBPS, 4)}
    del p_qkv, p_q, p_k, p_v
    # sampler: the batch's settings (half greedy, half T=0.7 / top-p 0.9)
    logits = torch.randn(B, cfg.vocab_size, device=dev, dtype=torch.float32).to(torch.bfloat16)
    smp = sch.sampler
    smp.set_params([r.temperature for r in reqs], [r.top_p for r in reqs])
    us = time_us(lambda: smp.sample(logits, B), 100)
    res["sampler"] = {"us": round(us, 2), "rows": B, "vocab": cfg.vocab_size}
    del logits
    # the sampler at the Qwen vocabulary: 48 rows x 152,064, every row T = 0.7 / top-p 0.9
    from minimal_inference_amd.sampling import Sampler

    big = Sampler(dev, 48, seed=5)
    big.set_params([0.7] * 48, [0.9] * 48)
    logits = torch.randn(48, 152064, device=dev, dtype=torch.float32).mul_(3).to(torch.bfloat16)
    us = time_us(lambda: big.sample(logits, 48), 50)
    res["sampler_qwen_vocab_top_p"] = {"us": round(us, 2), "rows": 48, "vocab": 152064, "top_p": 0.9,
                                       "temperature": 0.7}
    del logits
    res["prefill_attn_qwen72b_8prompts"] = prefill_72b_shape(dev)
    return res


def prefill_72b_shape(dev) -> dict:
    """Ragged causal prefill at the Qwen2.5-72B head shape (64 Q / 8 KV heads,
    head_dim 128): 8 prompts of lengths uniform in [256, 2048] (seed 4), pages
    from a seeded permutation of a pool of 24,000 pages (one layer's share of
    the HBM left after the 145 GB of weights)."""
    import torch

    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    hq, hkv, d, ps, num_pages = 64, 8, 128, 16, 24_000
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(256, 2049, (8,), generator=g).tolist()
    npg = [math.ceil(n / ps) for n in lens]
    perm = torch.randperm(num_pages - 1, generator=g)[: sum(npg)].to(torch.int32)
    pool = torch.empty(num_pages, 2, ps, hkv, d, device=dev, dtype=torch.bfloat16).normal_()
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    ip = [0]
    qo = [0]
    for n, p in zip(lens, npg):
        ip.append(ip[-1] + p)
        qo.append(qo[-1] + n)
    last = [n - (p - 1) * ps for n, p in zip(lens, npg)]
    q = torch.randn(qo[-1], hq, d, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev))
    w.plan(i32(qo), i32(ip), perm.to(dev), i32(last), hq, hkv, d, ps, causal=True, max_total_q=qo[-1])
    us = time_us(lambda: w.run(q, pool, out=out), 10)
    flops = sum(4 * hq * d * (L * (L + 1) // 2) for L in lens)
    del pool
    return {"us": round(us, 2), "tflops": round(flops / us / 1e6, 1), "frac_of_2500": round(flops / us / 1e6 / 2500, 4),
            "query_rows": qo[-1], "prompt_lens": lens}


def served_leg(model: str, concurrency=(2, 20, 32), max_tokens: int = 50, runs: int = 3) -> dict:
    """The reference's serving benchmark (README.md:50-70): the OpenAI server
    (minimal-inference_amd/server.py, random weights of ``model``, synthetic
    tokenizer, max_batch_size 40, max_seq_len 4096, page_size 16) runs in a
    child process; the streaming client sends ``n`` concurrent greedy requests
    of the prompt "Write a short poem about the ocean" with max_tokens 50,
    ``runs`` times per ``n``, and reports mean TTFT, mean T2T and aggregate tok/s."""
    import asyncio
    import socket
    import subprocess
    import tempfile
    import urllib.request

    import yaml

    from minimal_inference_amd.benchmark import run_benchmark

    with socket.socket() as sk:
        sk.bind(("127.0.0.1", 0))
        port = sk.getsockname()[1]
    tmp = Path(tempfile.mkdtemp(prefix="mi_served_"))
    cfg = {"model_preset": model, "device": "cuda", "dtype": "bfloat16", "seed": 0,
           "server": {"host": "127.0.0.1", "port": port},
           "scheduler": {"max_seq_len": 4096, "max_batch_size": 40, "page_size": 16, "decode_window": 1,
                         "pipeline": True, "use_graphs": True}}
    (tmp / "server.yaml").write_text(yaml.safe_dump(cfg))
    logf = open(tmp / "server.log", "w")
    proc = subprocess.Popen([sys.executable, "-u", str(ROOT / "minimal-inference_amd" / "server.py"),
                             "--config", str(tmp / "server.yaml")], stdout=logf, stderr=subprocess.STDOUT)
    url = f"http://127.0.0.1:{port}"
    out = {"server": f"{model} random weights, synthetic byte tokenizer, max_batch_size 40, max_seq_len 4096, "
                     f"page_size 16, one decode step per host round trip, pipelined (each step enqueued before the "
                     f"previous step's ids are read)",
           "prompt": "Write a short poem about the ocean", "max_tokens": max_tokens, "temperature": 0, "runs": runs}
    try:
        t0 = time.time()
        while True:
            if proc.poll() is not None:
                raise RuntimeError(f"server exited with {proc.returncode}")
            try:
                with urllib.request.urlopen(url + "/health", timeout=2) as r:
                    if r.status == 200:
                        break
            except OSError:
                pass
            if time.time() - t0 > 240:
                raise RuntimeError("server did not come up in 240 s")
            time.sleep(0.5)
        log(f"served: server up in {time.time() - t0:.1f}s")
        for n in concurrency:
            res = asyncio.run(run_benchmark(url, prompt=out["prompt"], max_tokens=max_tokens, batch_size=n,
                                            runs=runs, verbose=False))
            out[f"concurrent_{n}"] = {"ttft_ms": round(res["ttft_ms"], 1), "t2t_ms": round(res["t2t_ms"], 2),
                                      "aggregate_tok_s": round(res["aggregate_tok_s"], 1)}
            log(f"served: {n} concurrent: {out[f'concurrent_{n}']}")
    except Exception as e:  # reported in the line, never fatal for the kernel figures
        out["error"] = repr(e)
        logf.flush()
        log("served leg failed: " + repr(e) + "; server log tail:\n" + (tmp / "server.log").read_text()[-2000:])
    finally:
        proc.terminate()
        try:
            proc.wait(30)
        except subprocess.TimeoutExpired:
            proc.kill()
            proc.wait()
        logf.close()
    return out


def decode_attn_bytes(kv_lens, hq, hkv, d) -> int:
    """Algorithmic bytes of one decode-attention launch: every token's K and
    V (bf16), q read and out written, the CSR ints."""
    npages = sum(math.ceil(n / 16) for n in kv_lens)
    B = len(kv_lens)
    return sum(kv_lens) * hkv * d * 2 * 2 + 2 * B * hq * d * 2 + 4 * ((B + 1) + npages + B)


def decode_step_attn_bytes(kv_lens, hq, hkv, d) -> int:
    """Algorithmic bytes of the decode step's attention launch with the RoPE
    and the K/V append folded in (run_rope_append): the attention's bytes --
    the new token's K and V come from the qkv row instead of the pool, the
    same count -- plus the new K and V written to their slots and the cos /
    sin rows read."""
    B = len(kv_lens)
    return decode_attn_bytes(kv_lens, hq, hkv, d) + B * hkv * d * 2 * 2 + B * d * 2 * 2


def decode_attn_configs(dev) -> list:
    """The decode step's attention launch (RoPE + append + attention) on the
    other decode workloads' shapes, and attention alone beside it: 32
    synthetic layer pools (pages from a seeded permutation), one plan, the 32
    launches captured in a graph and replayed between HIP events, as in the
    roofline leg.  Contexts (the new token included) log-uniform as the
    workloads draw them."""
    import torch

    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper
    from minimal_inference_amd.model import precompute_rope

    def loguniform(n, lo, hi, seed):
        g = torch.Generator().manual_seed(seed)
        x = torch.rand(n, generator=g, dtype=torch.float64) * (math.log(hi) - math.log(lo)) + math.log(lo)
        return [int(round(math.exp(v))) for v in x.tolist()], g

    def uniform(n, lo, hi, seed):
        g = torch.Generator().manual_seed(seed)
        return torch.randint(lo, hi + 1, (n,), generator=g).tolist(), g

    out = []
    for name, hq, hkv, d, (lens, g) in [("qwen2.5-7b B=48, contexts log-uniform [256, 4096] seed 3", 28, 4, 128,
                                         loguniform(48, 256, 4096, 3)),
                                        ("qwen2.5-72b B=48, contexts log-uniform [512, 4096] seed 4", 64, 8, 128,
                                         loguniform(48, 512, 4096, 4)),
                                        ("qwen2.5-0.5b head shape (14 Q / 2 KV, head_dim 64) B=32, contexts "
                                         "uniform [512, 4096] seed 1", 14, 2, 64, uniform(32, 512, 4096, 1))]:
        B, L = len(lens), 32
        npg = [math.ceil(n / 16) for n in lens]
        tot = sum(npg)
        perm = torch.randperm(tot + 1, generator=g)[:tot].to(torch.int32).to(dev)
        pools = [torch.randn(tot + 1, 2, 16, hkv, d, device=dev, dtype=torch.bfloat16) for _ in range(L)]
        ip = torch.tensor([0] + torch.tensor(npg).cumsum(0).tolist(), dtype=torch.int32, device=dev)
        lp = torch.tensor([n - (p - 1) * 16 for n, p in zip(lens, npg)], dtype=torch.int32, device=dev)
        qs = [torch.randn(B, hq, d, device=dev, dtype=torch.bfloat16) for _ in range(L)]
        qkvs = [torch.randn(B, (hq + 2 * hkv) * d, device=dev, dtype=torch.bfloat16) for _ in range(L)]
        cos, sin = precompute_rope(d, max(lens) + 1, 1e6, dev, torch.bfloat16)
        outs = [torch.empty_like(q) for q in qs]
        w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev))
        w.plan(ip, perm, lp, hq, hkv, d, 16)
        # the decode step's launch (RoPE + append + attention), then attention alone
        us = time_us(lambda: [w.run_rope_append(qkvs[l], cos, sin, pools[l], out=outs[l]) for l in range(L)], 1) / L
        us_plain = time_us(lambda: [w.run(qs[l], pools[l], out=outs[l]) for l in range(L)], 1) / L
        nbytes = decode_step_attn_bytes(lens, hq, hkv, d)
        pbytes = decode_attn_bytes(lens, hq, hkv, d)
        gbps = nbytes / us / 1e3
        out.append({"workload": name, "us": round(us, 2), "mb": round(nbytes / 1e6, 1), "gbps": round(gbps, 1),
                    "frac": round(gbps / PEAK_HBM_GBPS, 4), "attention_alone_us": round(us_plain, 2),
                    "attention_alone_frac": round(pbytes / us_plain / 1e3 / PEAK_HBM_GBPS, 4)})
        del pools, qs, qkvs, outs
    return out


def measured_traffic(kernel: str, model: str, batch: int, mean_context: float, alg_bytes: float):
    """HBM bytes per attention launch from the committed counter record:
    (bytes, basis), or (None, reason) when the record is for another kernel,
    model or batch.  At the recorded mean context the counted bytes are used as they
    are; at another context (the steps and warm-up counts move it) the counted
    ratio of HBM bytes to algorithmic bytes is applied to this launch's
    algorithmic bytes -- the extra over the algorithmic bytes is the split
    partials' traffic, which scales with the unit count, as K / V does."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None, "no counter record"
    if rec.get("kernel_key") != kernel:
        return None, f"counter record is for another kernel ({rec.get('kernel')})"
    if rec.get("model") != model or rec.get("batch") != batch:
        return None, f"counter record is for {rec.get('model')} B={rec.get('batch')}"
    ratio = float(rec["traffic_bytes"]) / float(rec["alg_bytes"])
    if abs(float(rec["mean_context"]) - mean_context) <= 0.05:
        return float(rec["traffic_bytes"]), f"counted at this workload (mean context {rec['mean_context']})"
    return ratio * alg_bytes, (f"counted ratio {ratio:.4f} x algorithmic bytes (counters taken at mean context "
                               f"{rec['mean_context']}, this run {mean_context})")


# ---------------------------------------------------------------------- CPU legs


def cpu_setup() -> dict:
    """Threads for the CPU legs: the CPUs this process may run on (affinity
    mask, capped by the cgroup CPU quota when one is set), capped by
    OMP_NUM_THREADS when it is set -- on a host shared between GPUs that is
    this GPU's share of the cores.  The counts behind the choice are reported."""
    import torch

    n_os = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = n_os
    quota = None
    try:
        q, per = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, int(q) // int(per))
    except (OSError, ValueError):
        pass
    usable = min(aff, quota) if quota else aff
    omp = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(usable, int(omp)) if omp.isdigit() and int(omp) > 0 else usable
    torch.set_num_threads(threads)
    return {"os_cpu_count": n_os, "affinity_cpus": aff, "cgroup_quota_cpus": quota,
            "omp_num_threads": omp or None, "threads": torch.get_num_threads()}


def median_time(fn, min_runs: int = 10, budget_s: float = 10.0, max_runs: int = 200) -> tuple[float, int]:
    """Median wall seconds of ``fn`` after 3 warm-up calls: at least
    ``min_runs`` runs, more while under ``budget_s`` (at most ``max_runs``)."""
    for _ in range(3):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < max_runs):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times), len(times)


def oracle_weights(model):
    """The GPU model's weights as the oracle's fp32 host tensors (+ its Shape)."""
    import torch

    from oracle import model as om

    cfg = model.cfg
    f = lambda t: None if t is None else t.to("cpu", torch.float32)
    layers = [{"in_norm": f(L.in_norm), "post_norm": f(L.post_norm), "w_qkv": f(L.w_qkv), "b_qkv": f(L.b_qkv),
               "w_o": f(L.w_o), "w_gate_up": f(L.w_gate_up), "w_down": f(L.w_down)} for L in model.layers]
    embed = f(model.embed)
    lm = embed if model.lm_head is model.embed else f(model.lm_head)
    shape = om.Shape(cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                     cfg.intermediate_size, cfg.vocab_size, cfg.rms_norm_eps, cfg.rope_theta)
    return om.Weights(embed, lm, f(model.norm), layers), shape


def _csr(pages: list, lens: list, ps: int = 16):
    ip, ix = [0], []
    for pg, n in zip(pages, lens):
        k = math.ceil(n / ps)
        ix += pg[:k]
        ip.append(ip[-1] + k)
    return ip, ix, [n - (math.ceil(n / ps) - 1) * ps for n in lens]


def cpu_decode_leg(sch, model, reqs, budget_s: float = 20.0, max_steps: int = 8) -> dict:
    """End-to-end decode of the batch on the CPU: the oracle's model forward
    (fp32 math, bf16 pool) continues the GPU batch from its current state --
    the weights and the used pages of every layer's pool are copied to the
    host, each request's next token at its next position, greedy -- one
    decode step at a time, timed per step after one untimed step."""
    import torch

    from oracle import model as om

    B = len(reqs)
    dev = model.device
    ip = sch.d_indptr[: B + 1].cpu().tolist()
    ix = sch.d_indices[: ip[-1]].cpu()
    used = torch.unique(ix)
    local = torch.searchsorted(used, ix).tolist()
    pages = [local[ip[b]: ip[b + 1]] for b in range(B)]
    spare = B * (math.ceil((max_steps + 1) / 16) + 1)
    pools = []
    for kv in sch.kv.kv_data:
        p = torch.zeros(used.numel() + spare, *kv.shape[1:], dtype=kv.dtype)
        p[: used.numel()] = kv.index_select(0, used.to(dev)).cpu()
        pools.append(p)
    w, s = oracle_weights(model)
    nxt = used.numel()
    pos = [r.current_position for r in reqs]
    ids = torch.tensor([r.generated_tokens[-1] for r in reqs])
    times = []
    t_start = time.perf_counter()
    for step in range(max_steps + 1):
        for b in range(B):
            while len(pages[b]) < math.ceil((pos[b] + 1) / 16):
                pages[b].append(nxt)
                nxt += 1
        ind, idx, last = _csr(pages, [p + 1 for p in pos])
        t = time.perf_counter()
        ids = om.decode_step(w, s, ids, torch.tensor(pos), pools, ind, idx, last).argmax(-1)
        if step:
            times.append(time.perf_counter() - t)
        pos = [p + 1 for p in pos]
        if step >= 3 and time.perf_counter() - t_start > budget_s:
            break
    med = statistics.median(times)
    return {"value": round(B / med, 3), "unit": "tok/s", "step_s": round(med, 3), "steps": len(times)}


def cpu_attn_layer_leg(sch, q, alg_bytes: float, budget_s: float = 10.0) -> dict:
    """The oracle's gather-based paged decode attention on layer 0 of the batch."""
    from oracle import attention as oatt

    B = q.shape[0]
    dev = q.device
    import torch

    ip = sch.d_indptr[: B + 1].cpu().tolist()
    ix = sch.d_indices[: ip[-1]].cpu()
    used = torch.unique(ix)
    pool_cpu = sch.kv.kv_data[0].index_select(0, used.to(dev)).cpu()
    ix_local = torch.searchsorted(used, ix).tolist()
    last = sch.d_last[:B].cpu().tolist()
    q_cpu = q.cpu()
    med, n = median_time(lambda: oatt.decode(q_cpu, pool_cpu, ip, ix_local, last), budget_s=budget_s)
    return {"value": round(alg_bytes / med / 1e9, 3), "unit": "GB/s", "ms_per_layer": round(med * 1e3, 2),
            "runs": n}


def c1_leg(dev, with_cpu: bool) -> dict:
    """Config 1 (the committed fixture: Qwen2.5-0.5B head shape, B=4,
    contexts {17, 64, 203, 511}): the oracle on the CPU and the HIP decode
    kernel, both timed, and the kernel's max-abs error against the fixture."""
    import torch
    from safetensors.torch import load_file

    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper

    t = load_file(str(ROOT / "tests" / "golden" / "c1_decode.safetensors"))
    pool = torch.zeros(128, 2, 16, 2, 64, dtype=torch.bfloat16)
    pool[t["page_ids"].long()] = t["pages"]
    ip, ix, last = t["indptr"].tolist(), t["page_ids"].tolist(), t["last_page_len"].tolist()
    lens = [(ip[b + 1] - ip[b] - 1) * 16 + last[b] for b in range(4)]
    alg = sum(lens) * 2 * 64 * 4 + 2 * 4 * 14 * 64 * 2 + 4 * (5 + ip[-1] + 4)
    res = {"workload": "config 1: 14 Q / 2 KV heads, head_dim 64, B=4, contexts " + str(lens), "alg_bytes": alg}
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(16 << 20, dtype=torch.uint8, device=dev))
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    w.plan(i32(ip), i32(ix), i32(last), 14, 2, 64, 16)
    q_d, pool_d = t["q"].to(dev), pool.to(dev)
    out = w.run(q_d, pool_d)
    res["gpu_max_abs_vs_fixture"] = float((out.float().cpu() - t["out_fp32"]).abs().max())
    res["gpu_us"] = round(time_us(lambda: w.run(q_d, pool_d, out=out), 200), 2)
    if with_cpu:
        from oracle import attention as oatt

        med, n = median_time(lambda: oatt.decode(t["q"], pool, ip, ix, last), budget_s=5.0)
        res["cpu_us"] = round(med * 1e6, 1)
        res["cpu_runs"] = n
    return res


def _loguniform(g, n, lo, hi):
    import torch

    x = torch.rand(n, generator=g, dtype=torch.float64) * (math.log(hi) - math.log(lo)) + math.log(lo)
    return [int(round(math.exp(v))) for v in x.tolist()]


def _free_gpu() -> None:
    import gc

    import torch

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def c2_leg(dev, with_cpu: bool) -> dict:
    """Config 2 end to end: Qwen2.5-0.5B (random weights, seed 1), 8 prompts
    of lengths uniform in [32, 256], request i submitted at step 5 i, 50
    greedy tokens each, one engine step per host round trip.  The same
    schedule then runs on the CPU through the oracle's model forward (the same
    weights, fp32 math): batched ragged prefill of the step's admitted
    prompts, then one decode step of every decoding request."""
    import torch

    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model

    cfg = PRESETS["qwen2.5-0.5b"]
    model = Model(cfg, dev, seed=1, max_positions=4096)
    g = torch.Generator().manual_seed(1)
    lens = torch.randint(32, 257, (8,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lens]
    nt = 50

    def run(pipeline: bool):
        sch = Scheduler(model, max_batch_size=8, max_seq_len=1024, seed=1, pipeline=pipeline)
        reqs = [Request(str(i), p, nt, 0.0) for i, p in enumerate(prompts)]
        torch.cuda.synchronize()
        step = toks = 0
        t0 = time.perf_counter()
        while step < 5 * len(reqs) or sch.has_work():
            if step % 5 == 0 and step // 5 < len(reqs):
                sch.submit(reqs[step // 5])
            if sch.has_work():
                toks += len(sch.step())
            step += 1
        toks += len(sch.flush())
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return reqs, {"tokens": toks, "steps": step, "wall_s": round(wall, 3), "tok_s": round(toks / wall, 1)}

    reqs, gpu = run(False)
    piped_reqs, piped = run(True)
    piped["same_tokens"] = [r.generated_tokens for r in piped_reqs] == [r.generated_tokens for r in reqs]
    res = {"workload": "config 2: qwen2.5-0.5b, 8 prompts U[32,256] seed 1, submitted every 5 steps, 50 greedy "
                       "tokens each, one step per host round trip",
           "gpu": gpu,
           "gpu_pipelined": piped}
    if with_cpu:
        w, s = oracle_weights(model)
        cpu = cpu_staggered_run(w, s, prompts, nt)
        ids = cpu.pop("ids")
        # tokens up to the first difference between the GPU's and the CPU's
        # greedy ids (bf16 vs fp32 arithmetic; random weights give close logits)
        same = [next((j for j, (a, b) in enumerate(zip(r.generated_tokens, c)) if a != b),
                     min(len(r.generated_tokens), len(c))) for r, c in zip(reqs, ids)]
        cpu["greedy_ids_common_prefix"] = same
        res["cpu"] = cpu
    return res


def cpu_staggered_run(w, s, prompts, nt: int, every: int = 5, ps: int = 16) -> dict:
    """The config-2 schedule on the CPU through the oracle's model forward:
    request i is admitted at step ``every`` * i and prefilled (ragged causal
    prefill) in that step, then every request still short of ``nt`` tokens
    decodes one token per step (greedy), as the engine orders a step."""
    import torch

    from oracle import model as om

    lens = [len(p) for p in prompts]
    pools = [torch.zeros(sum(math.ceil((n + nt) / ps) for n in lens), 2, ps, s.kv_heads, s.head_dim,
                         dtype=torch.bfloat16) for _ in w.layers]
    pages, nxt = [], 0
    for n in lens:
        k = math.ceil((n + nt) / ps)
        pages.append(list(range(nxt, nxt + k)))
        nxt += k
    gen = [[] for _ in lens]
    active: list[int] = []
    toks = 0
    t_dec = 0.0
    t0 = time.perf_counter()
    step = 0
    while step < every * len(lens) or active:
        if step % every == 0 and step // every < len(lens):
            b = step // every
            ind, idx, last = _csr([pages[b]], [lens[b]], ps)
            logits = om.prefill_step(w, s, torch.tensor(prompts[b]), [0, lens[b]], pools, ind, idx, last, ps)
            gen[b].append(int(logits[0].argmax()))
            toks += 1
            active.append(b)
        dec = [b for b in active if len(gen[b]) < nt]
        if dec:
            td = time.perf_counter()
            pos = [lens[b] + len(gen[b]) - 1 for b in dec]
            ind, idx, last = _csr([pages[b] for b in dec], [p + 1 for p in pos], ps)
            ids = torch.tensor([gen[b][-1] for b in dec])
            nxt_ids = om.decode_step(w, s, ids, torch.tensor(pos), pools, ind, idx, last, ps).argmax(-1).tolist()
            t_dec += time.perf_counter() - td
            for b, t in zip(dec, nxt_ids):
                gen[b].append(t)
            toks += len(dec)
        active = [b for b in active if len(gen[b]) < nt]
        step += 1
    wall = time.perf_counter() - t0
    return {"tokens": toks, "steps": step, "wall_s": round(wall, 3), "tok_s": round(toks / wall, 2),
            "decode_tok_s": round((toks - len(lens)) / t_dec, 2), "kind": "port", "threads": torch.get_num_threads(),
            "what": "oracle model forward (fp32 torch, gather-based paged attention), same weights", "ids": gen}


def c4_leg(dev) -> dict:
    """Config 4 end to end: Qwen2.5-7B (random weights, seed 3),
    max_batch_size 48, max_seq_len 4096; 64 requests with prompt lengths
    log-uniform in [256, 4096] and token budgets uniform in [8, 120] (seed 3)
    so that requests retire and waiting ones are admitted mid-run; 100 engine
    steps, one step per host round trip (greedy)."""
    import torch

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
    reqs = [Request(str(i), p, budgets[i], 0.0) for i, p in enumerate(prompts)]
    for r in reqs:
        sch.submit(r)
    torch.cuda.synchronize()
    toks = retired = admitted_late = 0
    dec_steps = []
    t0 = time.perf_counter()
    for step in range(100):
        if not sch.has_work():
            break
        n_wait, n_active = len(sch.waiting), len(sch.active)
        ts = time.perf_counter()
        emitted = sch.step()  # ends with the host read-back of the step's ids
        dt = time.perf_counter() - ts
        admitted = n_wait - len(sch.waiting)
        retired += n_active + admitted - len(sch.active)
        if step:
            admitted_late += admitted
        toks += len(emitted)
        if admitted == 0:
            dec_steps.append((dt, len(emitted)))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    med = statistics.median(dt for dt, _ in dec_steps) if dec_steps else None
    rows = statistics.median(n for _, n in dec_steps) if dec_steps else None
    # the same 100 steps with the pipelined read-back (each step enqueued
    # before the previous one's ids are read; admissions and retirements
    # read the step in flight first, so the tokens are the same)
    del sch
    _free_gpu()
    psch = Scheduler(model, max_batch_size=48, max_seq_len=4096, seed=3, pipeline=True)
    preqs = [Request(str(i), p, budgets[i], 0.0) for i, p in enumerate(prompts)]
    for r in preqs:
        psch.submit(r)
    torch.cuda.synchronize()
    ptoks = 0
    t0 = time.perf_counter()
    for _ in range(step + 1):
        if not psch.has_work():
            break
        ptoks += len(psch.step())
    ptoks += len(psch.flush())
    torch.cuda.synchronize()
    pwall = time.perf_counter() - t0
    same = [r.generated_tokens[: len(q.generated_tokens)] == q.generated_tokens[: len(r.generated_tokens)]
            for r, q in zip(preqs, reqs)]
    pipelined = {"steps": step + 1, "tokens": ptoks, "wall_s": round(pwall, 3), "tok_s": round(ptoks / pwall, 1),
                 "token_prefixes_agree": all(same)}
    del psch
    return {"workload": "config 4: qwen2.5-7b, B<=48, 64 prompts log-uniform [256,4096] seed 3, budgets U[8,120], "
                        "100 engine steps, one step per host round trip",
            "pipelined": pipelined,
            "steps": step + 1, "tokens": toks, "wall_s": round(wall, 3), "tok_s": round(toks / wall, 1),
            "admitted_late": admitted_late, "retired": retired, "decode_only_steps": len(dec_steps),
            "decode_only_median_ms": round(med * 1e3, 3) if med else None, "decode_only_median_rows": rows,
            "decode_only_tok_s": round(rows / med, 1) if med else None}


def c5_leg(dev) -> dict:
    """Config 5 end to end: Qwen2.5-72B (random weights, seed 4, 145 GB on
    the GPU), the page pool sized to the HBM left (24 GiB kept for
    activations).  48 requests with prompt lengths log-uniform in
    [512, 4096] (seed 4) are admitted 8 per step; then 3 decode steps at
    B=48; then one step that prefills 8 new prompts (lengths uniform in
    [256, 2048]) in one ragged batch and decodes all 56 (prefill then decode,
    as the reference orders a step); then 3 decode steps at B=56.  Greedy, one
    step per host round trip; each step timed on its own."""
    import torch

    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model, kv_pool_bytes_per_page

    cfg = PRESETS["qwen2.5-72b"]
    t_init = time.perf_counter()
    model = Model(cfg, dev, seed=4, max_positions=4096 + 64 + 16)
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t_init
    free, _ = torch.cuda.mem_get_info(dev)
    num_pages = int((free - 24 * 2**30) // kv_pool_bytes_per_page(cfg, 16))
    g = torch.Generator().manual_seed(4)
    dec_lens = _loguniform(g, 48, 512, 4096)
    pre_lens = torch.randint(256, 2049, (8,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in dec_lens + pre_lens]
    sch = Scheduler(model, max_batch_size=56, max_seq_len=4096 + 64, num_pages=num_pages, seed=4)
    reqs = [Request(str(i), p, 64, 0.0) for i, p in enumerate(prompts)]

    def timed_step():
        torch.cuda.synchronize()
        t = time.perf_counter()
        n = len(sch.step())
        torch.cuda.synchronize()
        return time.perf_counter() - t, n

    for k in range(6):
        for r in reqs[8 * k: 8 * k + 8]:
            sch.submit(r)
        timed_step()
    d48 = [timed_step() for _ in range(3)]
    for r in reqs[48:]:
        sch.submit(r)
    mixed_s, mixed_toks = timed_step()
    d56 = [timed_step() for _ in range(3)]
    if any(r.status.value != "decoding" for r in reqs):
        raise RuntimeError("config 5: a request left the decoding state")
    ms48 = statistics.median(t for t, _ in d48)
    ms56 = statistics.median(t for t, _ in d56)
    return {"workload": "config 5: qwen2.5-72b (145 GB random weights), 48 decoding requests with prompts "
                        "log-uniform [512,4096] seed 4, then 8 prompts U[256,2048] prefilled in the same step as "
                        "the decode of all 56",
            "weights_gb": round(model.weight_bytes() / 1e9, 1), "init_s": round(init_s, 1), "pool_pages": num_pages,
            "pool_gb": round(num_pages * kv_pool_bytes_per_page(cfg, 16) / 1e9, 1),
            "decode_b48_ms": round(ms48 * 1e3, 2), "decode_b48_tok_s": round(48 / ms48, 1),
            "prefill8_plus_decode56_ms": round(mixed_s * 1e3, 2), "prefill8_plus_decode56_tokens": mixed_toks,
            "prefill8_query_rows": sum(pre_lens),
            "decode_b56_ms": round(ms56 * 1e3, 2), "decode_b56_tok_s": round(56 / ms56, 1)}


def mistral_leg(args, dev, with_cpu: bool) -> dict:
    """The headline workload: decode tok/s, the decode-attention roofline leg,
    the path's other kernels, the CPU baseline and the one-step-per-round-trip
    decode (see the module docstring).  Returns the fields of the JSON line."""
    import torch

    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model

    cfg = PRESETS[args.model]
    B = args.batch
    # prefill token + first decode step + warmup + two timed legs + CPU-leg headroom
    new_tokens = max(50, 2 + args.warmup + 2 * args.steps + 2)
    g = torch.Generator().manual_seed(args.seed)
    lens = torch.randint(128, 1025, (B,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lens]
    max_seq = 1024 + new_tokens + 16

    log(f"init {args.model} (random weights) on {torch.cuda.get_device_name(0)}")
    t0 = time.time()
    model = Model(cfg, dev, seed=args.seed, max_positions=max_seq + 16)
    torch.cuda.synchronize()
    log(f"weights {model.weight_bytes() / 1e9:.2f} GB in {time.time() - t0:.1f}s; capturing graphs")
    sch = Scheduler(model, max_batch_size=B, max_seq_len=max_seq, seed=args.seed, decode_window=args.decode_window,
                    pipeline=True)
    reqs = [Request(str(i), p, new_tokens, 0.0 if i % 2 == 0 else 0.7, 1.0 if i % 2 == 0 else 0.9)
            for i, p in enumerate(prompts)]
    for r in reqs:
        sch.submit(r)
    t0 = time.time()
    sch.decode_window = 1
    sch.step()  # admit + ragged prefill of all 32 prompts + first decode step
    sch.flush()
    torch.cuda.synchronize()

    def decode_steps(n: int, window: int) -> float:
        """Exactly ``n`` decode steps in windows of ``window`` (the next window
        enqueued before the last one's ids are read), then the last window
        read back; wall seconds."""
        torch.cuda.synchronize()
        t = time.perf_counter()
        first = len(reqs[0].generated_tokens) + sch.in_flight(reqs[0])
        while (done := len(reqs[0].generated_tokens) + sch.in_flight(reqs[0]) - first) < n:
            sch.decode_window = min(window, n - done)
            sch.step()
            if len(reqs[0].generated_tokens) + sch.in_flight(reqs[0]) - first == done:
                raise RuntimeError("no decode progress (requests finished?)")
        sch.flush()
        torch.cuda.synchronize()
        if len(reqs[0].generated_tokens) - first != n:
            raise RuntimeError("decode step count mismatch")
        return time.perf_counter() - t

    log(f"prefill + first decode step {time.time() - t0:.2f}s; warmup {args.warmup} steps")
    decode_steps(args.warmup, args.decode_window)
    n_active = sum(1 for r in reqs if r.status.value == "decoding")
    if n_active != B:
        raise RuntimeError(f"expected {B} decoding requests, have {n_active}")
    log(f"timing {args.steps} decode steps at B={B}, {args.decode_window} steps per host round trip")
    elapsed = decode_steps(args.steps, args.decode_window)
    toks = B * args.steps / elapsed
    ms_step = elapsed * 1000 / args.steps
    log(f"decode: {toks:.0f} tok/s, {ms_step:.3f} ms/step")
    if any(r.status.value != "decoding" for r in reqs):
        raise RuntimeError("a request finished inside the timed steps")

    # ---------------- the decode step's attention launch on the batch's real state
    # The CSR of the next decode step (each request's next position, the new
    # token counted: its pages are allocated here as that step would), so the
    # launch appends into the slot the next step writes anyway.
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    kv_lens = [r.current_position + 1 for r in reqs]
    rows = [(r.slot, r.current_position) for r in reqs]
    sch.pt.step([], rows, B, sch.d_indptr, sch.d_indices, sch.d_last, sch.d_batch, sch.d_pos)
    w = sch.decode_wrapper
    w.plan(sch.d_indptr[: B + 1], sch.d_indices, sch.d_last[:B], hq, hkv, d, 16)
    L = cfg.num_hidden_layers
    qkvs = [torch.randn(B, (hq + 2 * hkv) * d, device=dev, dtype=torch.bfloat16) for _ in range(L)]
    qs = [torch.randn(B, hq, d, device=dev, dtype=torch.bfloat16) for _ in range(L)]
    outs = [torch.empty_like(q) for q in qs]
    alg_bytes = decode_step_attn_bytes(kv_lens, hq, hkv, d)
    plain_bytes = decode_attn_bytes(kv_lens, hq, hkv, d)

    def layer_launches(fused: bool):
        for l in range(L):
            if fused:
                w.run_rope_append(qkvs[l], model.cos, model.sin, sch.kv.kv_data[l], out=outs[l])
            else:
                w.run(qs[l], sch.kv.kv_data[l], out=outs[l])

    def graph_us(fused: bool) -> float:
        """The L launches captured once and replayed, so the events time the
        kernels back to back on the GPU without host launch gaps."""
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                layer_launches(fused)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            layer_launches(fused)
        for _ in range(10):  # ~6 ms of untimed work: clocks at their sustained level
            graph.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.attn_iters):
            graph.replay()
        e1.record(stream)
        e1.synchronize()
        del graph
        return e0.elapsed_time(e1) * 1000 / (args.attn_iters * L)

    attn_us = graph_us(True)
    achieved = alg_bytes / (attn_us * 1e-6) / 1e9
    plain_us = graph_us(False)
    plain_gbps = plain_bytes / (plain_us * 1e-6) / 1e9
    log(f"decode step attention launch (RoPE + append + attention): {attn_us:.2f} us/launch, {achieved:.0f} GB/s "
        f"({100 * achieved / PEAK_HBM_GBPS:.1f}% of {PEAK_HBM_GBPS:.0f}), {alg_bytes / 1e6:.1f} MB/launch; "
        f"attention alone {plain_us:.2f} us, {100 * plain_gbps / PEAK_HBM_GBPS:.1f}%")

    # ---------------- CPU baseline: the oracle continues this batch on the host cores
    cpu = cpu_legs = None
    if with_cpu:
        info = cpu_setup()
        log(f"cpu baseline: {info}")
        mist = cpu_decode_leg(sch, model, reqs)
        cpu = {"value": mist["value"], "unit": "tok/s", "cores": info["threads"], "kind": "port",
               "sample": f"oracle model forward (fp32 torch, gather-based paged attention over the bf16 pool) "
                         f"continuing this {args.model} B={B} batch from its GPU state (weights and used pages "
                         f"copied to the host), greedy, median of {mist['steps']} decode steps after one "
                         f"untimed step: {mist['step_s']} s per step",
               **{k: info[k] for k in ("os_cpu_count", "affinity_cpus", "cgroup_quota_cpus", "omp_num_threads",
                                       "threads")}}
        layer = cpu_attn_layer_leg(sch, qs[0], plain_bytes)
        cpu_legs = {"mistral_attn_one_layer": {**layer, "kind": "port",
                                               "what": "oracle gather-based paged decode attention, layer 0 of "
                                                       "this batch, median after 3 warm-ups"}}
        log(f"cpu baseline: {cpu['value']} tok/s, one layer's attention {layer}")

    path = path_kernel_times(sch, cfg, reqs, lens, dev)
    log(f"path kernels: {path}")

    # the same decode with the ids read back after every step (continues the batch)
    single = decode_steps(args.steps, 1)
    toks_single = B * args.steps / single
    log(f"decode, one step per round trip: {toks_single:.0f} tok/s, {single * 1000 / args.steps:.3f} ms/step")

    mean_ctx = round(sum(kv_lens) / B, 1)
    traffic, basis = measured_traffic("decode_step_attention", args.model, B, mean_ctx, alg_bytes)
    return {
        "value": round(toks, 2), "ms_per_step": round(ms_step, 4),
        "config": {"workload": f"{args.model} decode, B={B}, prompts U[128,1024] seed {args.seed}, "
                               f"half greedy / half T=0.7 top-p 0.9, page_size 16, hipGraph decode, "
                               f"{args.decode_window} decode steps per host round trip",
                   "batch": B, "mean_context": mean_ctx, "decode_window": args.decode_window,
                   "parallelism": "single GPU"},
        "decode_tok_s_one_step_per_round_trip": round(toks_single, 2),
        "decode_attn_kernel": "the decode step's attention launch: RoPE of q and k, the new K/V appended, "
                              "split-K paged attention (mi_decode_rope_append_run, decode_run_kernel<128, 4, 2, 1, "
                              "true>)",
        "decode_attn_us": round(attn_us, 3),
        "decode_attn_gbps": round(achieved, 1),
        "decode_attn_alg_bytes": alg_bytes,
        "decode_attn_alone": {"us": round(plain_us, 3), "gbps": round(plain_gbps, 1), "alg_bytes": plain_bytes,
                              "frac": round(plain_gbps / PEAK_HBM_GBPS, 4),
                              "what": "attention alone on the same CSR (mi_decode_run, q already rotated)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4),
                     "traffic": round(traffic) if traffic is not None else None, "traffic_basis": basis},
        "cpu_baseline": cpu,
        "cpu_baseline_legs": cpu_legs,
        "path_kernels": path,
    }


LEGS = ("main", "served", "c1", "c2", "c4", "c5")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--model", default="mistral-7b")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--attn-iters", type=int, default=20)
    ap.add_argument("--decode-window", type=int, default=8,
                    help="decode steps per host round trip (1 = read the ids back after every step)")
    ap.add_argument("--legs", default=",".join(LEGS),
                    help="comma-separated legs to run: " + ", ".join(LEGS) + " (main is always run)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-served", action="store_true", help="skip the HTTP serving leg")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device-to-device copy (5x): the known-traffic kernel used "
                         "to scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path runs on one MI355X); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        return 2
    legs = {x.strip() for x in args.legs.split(",") if x.strip()} | {"main"}
    unknown = legs - set(LEGS)
    if unknown:
        print(f"unknown legs {sorted(unknown)}; choose from {LEGS}", file=sys.stderr)
        return 2
    if args.no_served:
        legs.discard("served")
    with_cpu = not args.no_cpu_baseline

    import torch

    if args.calibrate_copy:
        n = (1 << 30) // 2
        src = torch.ones(n, dtype=torch.bfloat16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30, "launches": 5}))
        return 0

    from __graft_entry__ import load_package

    load_package()
    dev = torch.device("cuda:0")
    head = mistral_leg(args, dev, with_cpu)
    _free_gpu()
    other_attn = decode_attn_configs(dev)
    log(f"decode attention, other workloads: {other_attn}")
    _free_gpu()
    extra = {}
    if "c1" in legs:
        extra["config1_decode_attn"] = c1_leg(dev, with_cpu)
        log(f"config 1: {extra['config1_decode_attn']}")
    if "c2" in legs:
        extra["config2_end_to_end"] = c2_leg(dev, with_cpu)
        log(f"config 2: {extra['config2_end_to_end']}")
        _free_gpu()

    served = None
    if "served" in legs:
        log("served leg: OpenAI server in a child process + streaming client")
        served = served_leg(args.model)
    if "c4" in legs:
        log("config 4: qwen2.5-7b, 100 engine steps with retire / admit")
        extra["config4_end_to_end"] = c4_leg(dev)
        log(f"config 4: {extra['config4_end_to_end']}")
        _free_gpu()
    if "c5" in legs:
        log("config 5: qwen2.5-72b, 48 decoding + 8 prefilled in one step")
        extra["config5_end_to_end"] = c5_leg(dev)
        log(f"config 5: {extra['config5_end_to_end']}")
        _free_gpu()

    agg32 = (served or {}).get("concurrent_32", {}).get("aggregate_tok_s")
    line = {
        "metric": "decode-attn HBM GB/s (% of peak) + decode tok/s, Mistral-7B B=32",
        "value": head.pop("value"),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(agg32 / PUBLISHED_TOKS, 4) if agg32 else None,
        "vs_baseline_basis": ("served aggregate tok/s at 32 concurrent requests (served.concurrent_32) / the "
                              "reference's published 1,532 (README.md:56, H100, 32 concurrent)") if agg32 else
                             "served leg not run",
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random prompt token ids)",
        **head,
        "decode_attn_other_workloads": other_attn,
        **extra,
        "served": served,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
