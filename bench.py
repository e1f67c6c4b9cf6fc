"""Benchmark: decode tok/s and decode-attention HBM GB/s, Mistral-7B, B=32, one GPU.

Workload (random-initialised Mistral-7B architecture, bf16): 32 concurrent
requests with prompt lengths uniform in [128, 1024] and random token ids
(seed 2); even requests greedy, odd ones temperature 0.7 / top-p 0.9;
page_size 16; one hipGraph per decode batch size.  All prompts are admitted
and prefilled (one ragged batch) before timing.

A "step" is one full decode step of the 32-request batch: device page-table
step, plan(), graph replay (32 layers: GEMMs, RoPE, KV append, split-K paged
attention, sampler), the feedback of the sampled ids and, once per window of
``--decode-window`` steps, end-of-sequence detection on the GPU and the
read-back of the window's ids.  ``value`` is decoded tokens per second over
exactly ``--steps`` timed steps; ``decode_tok_s_one_step_per_round_trip`` is
the same over the next ``--steps`` steps with a read-back after every step.

``roofline`` is measured on the decode-attention kernel alone: after the
timed steps, the 32 layers' attention launches (the batch's real page tables
and pools, one pool per layer so nothing is served from the 256 MB Infinity
Cache) are captured in a hipGraph, replayed ``--attn-iters`` times on the
current stream and bracketed with HIP events; achieved = algorithmic bytes
per launch / average launch time.  Algorithmic bytes per launch:
sum_b kv_len_b * H_kv * D * 2 (K,V) * 2 B + 2 * B * H_q * D * 2 B (q, out)
+ 4 B * ((B+1) + sum_b npages_b + B) (indptr, indices, last_page_len).

``roofline.traffic`` is the HBM bytes per launch that rocprofv3 counted for
this same attention leg (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled
by what the counter reads for a 1 GiB device copy), read from
profiles/decode_attn_traffic.json when that file was measured on this
workload (same model, batch and mean context); otherwise null.

``cpu_baseline`` times the CPU oracle's gather-based attention on one layer of
the same batch.

``decode_attn_other_workloads`` times the same decode-attention kernel, the
same way, on the Qwen2.5-7B (B=48, 28/4 heads) and Qwen2.5-72B (B=48, 64/8
heads) decode shapes with their log-uniform contexts (synthetic pools).

``served`` reproduces the reference's published serving measurement
(README.md:50-70, benchmark.py): the OpenAI-compatible server in a child
process (random weights, synthetic tokenizer) and the streaming client at 2,
20 and 32 concurrent greedy requests, max_tokens 50, 3 runs each: TTFT, T2T
and aggregate tok/s (content chunks / run wall time, prefill included) --
the figures the reference's 1,532 tok/s at 32 concurrent is quoted as.

``path_kernels`` times the other kernels of the path on the same state, each
as repeated launches captured in one hipGraph and replayed between HIP events: the ragged
causal prefill attention of the 32 prompts for one layer (MFMA bound:
flops = sum_b 4 * H_q * D * L_b (L_b + 1) / 2, against 2.5 PFLOP/s bf16), the
decode-step fused RoPE + KV append (into a copy of layer 0's pool), the
prefill-sized appends of the prompts' rows into their pages (HBM bound against
8 TB/s; fused RoPE + append bytes = 2 * T * (H_q + 2 H_kv) * D * 2 B (q, k, v
read and written) + 2 * T * D * 2 B (cos / sin rows) + index ints; plain
append bytes = 2 * 2 * T * H_kv * D * 2 B + index ints) and the sampler for
the 32 rows (latency bound: microseconds).
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


def time_us(fn, iters: int) -> float:
    """Average GPU microseconds per call of ``fn``: ``iters`` calls captured in
    one hipGraph (so host launch cost is excluded), replayed between HIP
    events on the current stream after warm-up calls on a side stream."""
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
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1000 / iters


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
    return res


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
                         "use_graphs": True}}
    (tmp / "server.yaml").write_text(yaml.safe_dump(cfg))
    logf = open(tmp / "server.log", "w")
    proc = subprocess.Popen([sys.executable, "-u", str(ROOT / "minimal-inference_amd" / "server.py"),
                             "--config", str(tmp / "server.yaml")], stdout=logf, stderr=subprocess.STDOUT)
    url = f"http://127.0.0.1:{port}"
    out = {"server": f"{model} random weights, synthetic byte tokenizer, max_batch_size 40, max_seq_len 4096, "
                     f"page_size 16, one decode step per host round trip",
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


def decode_attn_configs(dev) -> list:
    """Decode attention alone on the other decode workloads' shapes: 32
    synthetic layer pools (pages from a seeded permutation), one plan, the 32
    launches captured in a graph and replayed between HIP events, as in the
    roofline leg.  Contexts log-uniform as the workloads draw them."""
    import torch

    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper

    def loguniform(n, lo, hi, seed):
        g = torch.Generator().manual_seed(seed)
        x = torch.rand(n, generator=g, dtype=torch.float64) * (math.log(hi) - math.log(lo)) + math.log(lo)
        return [int(round(math.exp(v))) for v in x.tolist()], g

    out = []
    for name, hq, hkv, d, (lens, g) in [("qwen2.5-7b B=48, contexts log-uniform [256, 4096] seed 3", 28, 4, 128,
                                         loguniform(48, 256, 4096, 3)),
                                        ("qwen2.5-72b B=48, contexts log-uniform [512, 4096] seed 4", 64, 8, 128,
                                         loguniform(48, 512, 4096, 4))]:
        B, L = len(lens), 32
        npg = [math.ceil(n / 16) for n in lens]
        tot = sum(npg)
        perm = torch.randperm(tot + 1, generator=g)[:tot].to(torch.int32).to(dev)
        pools = [torch.randn(tot + 1, 2, 16, hkv, d, device=dev, dtype=torch.bfloat16) for _ in range(L)]
        ip = torch.tensor([0] + torch.tensor(npg).cumsum(0).tolist(), dtype=torch.int32, device=dev)
        lp = torch.tensor([n - (p - 1) * 16 for n, p in zip(lens, npg)], dtype=torch.int32, device=dev)
        qs = [torch.randn(B, hq, d, device=dev, dtype=torch.bfloat16) for _ in range(L)]
        outs = [torch.empty_like(q) for q in qs]
        w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev))
        w.plan(ip, perm, lp, hq, hkv, d, 16)
        us = time_us(lambda: [w.run(qs[l], pools[l], out=outs[l]) for l in range(L)], 1) / L
        nbytes = sum(lens) * hkv * d * 4 + 2 * B * hq * d * 2 + 4 * ((B + 1) + tot + B)
        gbps = nbytes / us / 1e3
        out.append({"workload": name, "us": round(us, 2), "mb": round(nbytes / 1e6, 1), "gbps": round(gbps, 1),
                    "frac": round(gbps / PEAK_HBM_GBPS, 4)})
        del pools, qs, outs
    return out


def measured_traffic(model: str, batch: int, mean_context: float):
    """HBM bytes per attention launch from the committed counter summary, or
    None when it was measured on another workload."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    if rec.get("model") != model or rec.get("batch") != batch:
        return None
    if abs(float(rec.get("mean_context", -1)) - mean_context) > 0.05:
        return None
    return float(rec["traffic_bytes"])


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--model", default="mistral-7b")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--attn-iters", type=int, default=20)
    ap.add_argument("--decode-window", type=int, default=8,
                    help="decode steps per host round trip (1 = read the ids back after every step)")
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
    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model

    dev = torch.device("cuda:0")
    cfg = PRESETS[args.model]
    B = args.batch
    # prefill token + first decode step + warmup + two timed legs, plus slack
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
    sch = Scheduler(model, max_batch_size=B, max_seq_len=max_seq, seed=args.seed, decode_window=args.decode_window)
    reqs = [Request(str(i), p, new_tokens, 0.0 if i % 2 == 0 else 0.7, 1.0 if i % 2 == 0 else 0.9)
            for i, p in enumerate(prompts)]
    for r in reqs:
        sch.submit(r)
    t0 = time.time()
    sch.decode_window = 1
    sch.step()  # admit + ragged prefill of all 32 prompts + first decode step
    torch.cuda.synchronize()
    def decode_steps(n: int, window: int) -> float:
        """Exactly ``n`` decode steps in windows of ``window``; wall seconds."""
        torch.cuda.synchronize()
        t = time.perf_counter()
        done = 0
        while done < n:
            sch.decode_window = min(window, n - done)
            before = len(reqs[0].generated_tokens)
            sch.step()
            if len(reqs[0].generated_tokens) == before:
                raise RuntimeError("no decode progress (requests finished?)")
            done += len(reqs[0].generated_tokens) - before
        torch.cuda.synchronize()
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

    # ---------------- decode-attention kernel on the batch's real state
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    kv_lens = [r.current_position for r in reqs]  # tokens in the cache after the last step
    rows = [(r.slot, r.current_position - 1) for r in reqs]
    # rebuild the CSR for exactly these contexts (no growth: pages already held)
    sch.pt.step([], rows, B, sch.d_indptr, sch.d_indices, sch.d_last, sch.d_batch, sch.d_pos)
    w = sch.decode_wrapper
    w.plan(sch.d_indptr[: B + 1], sch.d_indices, sch.d_last[:B], hq, hkv, d, 16)
    qs = [torch.randn(B, hq, d, device=dev, dtype=torch.bfloat16) for _ in range(cfg.num_hidden_layers)]
    outs = [torch.empty_like(q) for q in qs]
    npages = [math.ceil(n / 16) for n in kv_lens]
    alg_bytes = sum(kv_lens) * hkv * d * 2 * 2 + 2 * B * hq * d * 2 + 4 * ((B + 1) + sum(npages) + B)
    # The 32 launches are captured once and replayed, so the events time the
    # kernels back to back on the GPU without host launch gaps.
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for l in range(cfg.num_hidden_layers):
                w.run(qs[l], sch.kv.kv_data[l], out=outs[l])
    torch.cuda.current_stream().wait_stream(side)
    attn_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(attn_graph):
        for l in range(cfg.num_hidden_layers):
            w.run(qs[l], sch.kv.kv_data[l], out=outs[l])
    attn_graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.attn_iters):
        attn_graph.replay()
    e1.record(stream)
    e1.synchronize()
    launches = args.attn_iters * cfg.num_hidden_layers
    attn_us = e0.elapsed_time(e1) * 1000 / launches
    achieved = alg_bytes / (attn_us * 1e-6) / 1e9
    log(f"decode attention: {attn_us:.2f} us/launch, {achieved:.0f} GB/s "
        f"({100 * achieved / PEAK_HBM_GBPS:.1f}% of {PEAK_HBM_GBPS:.0f}), {alg_bytes / 1e6:.1f} MB/launch")

    path = path_kernel_times(sch, cfg, reqs, lens, dev)
    log(f"path kernels: {path}")
    other_attn = decode_attn_configs(dev)
    log(f"decode attention, other workloads: {other_attn}")

    # ---------------- CPU baseline: the oracle on one layer of the same batch
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import attention as oatt  # CPU checker, timed as the baseline

        torch.set_num_threads(max(1, min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "16")))))
        ip = sch.d_indptr[: B + 1].cpu().tolist()
        ix = sch.d_indices[: ip[-1]].cpu()
        used = torch.unique(ix)
        remap = {int(p): i for i, p in enumerate(used.tolist())}
        pool_cpu = sch.kv.kv_data[0].index_select(0, used.to(dev)).cpu()
        ix_local = [remap[int(p)] for p in ix.tolist()]
        last = sch.d_last[:B].cpu().tolist()
        q_cpu = qs[0].cpu()
        for _ in range(3):
            oatt.decode(q_cpu, pool_cpu, ip, ix_local, last)
        times = []
        t_budget = time.perf_counter()
        while len(times) < 10 or (time.perf_counter() - t_budget < 10 and len(times) < 200):
            t = time.perf_counter()
            oatt.decode(q_cpu, pool_cpu, ip, ix_local, last)
            times.append(time.perf_counter() - t)
            if time.perf_counter() - t_budget > 30:
                break
        med = statistics.median(times)
        cpu = {"value": round(alg_bytes / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"oracle gather-based paged decode attention (fp32 torch) on one Mistral-7B layer of "
                         f"this B={B} batch, median of {len(times)} runs after 3 warm-ups; "
                         f"{med * 1000:.1f} ms per layer"}
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads")

    # the same decode with the ids read back after every step (continues the batch)
    single = decode_steps(args.steps, 1)
    toks_single = B * args.steps / single
    log(f"decode, one step per round trip: {toks_single:.0f} tok/s, {single * 1000 / args.steps:.3f} ms/step")

    served = None
    if not args.no_served:
        log("served leg: OpenAI server in a child process + streaming client")
        served = served_leg(args.model)

    mean_ctx = round(sum(kv_lens) / B, 1)
    traffic = measured_traffic(args.model, B, mean_ctx)
    line = {
        "metric": "decode-attn HBM GB/s (% of peak) + decode tok/s, Mistral-7B B=32",
        "value": round(toks, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(toks / PUBLISHED_TOKS, 4),
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random prompt token ids)",
        "config": {"workload": f"{args.model} decode, B={B}, prompts U[128,1024] seed {args.seed}, "
                               f"half greedy / half T=0.7 top-p 0.9, page_size 16, hipGraph decode, "
                               f"{args.decode_window} decode steps per host round trip",
                   "batch": B, "mean_context": mean_ctx, "decode_window": args.decode_window,
                   "parallelism": "single GPU"},
        "decode_tok_s_one_step_per_round_trip": round(toks_single, 2),
        "decode_attn_us": round(attn_us, 3),
        "decode_attn_gbps": round(achieved, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "path_kernels": path,
        "decode_attn_other_workloads": other_attn,
        "served": served,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
