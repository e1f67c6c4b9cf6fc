"""Streaming latency / throughput client for an OpenAI-compatible server.

Measures what the reference's benchmark.py reports (benchmark.py:23-135,
README.md:51-70): N concurrent streaming chat requests with the same
prompt and ``temperature: 0``, repeated ``--runs`` times.  Per request:
TTFT = first content chunk - request start; T2T = mean interval between
consecutive content chunks (decode only); per run: aggregate tok/s = content
chunks of all requests / wall time of the run.  The summary averages TTFT and
T2T over requests and the aggregate over runs.  A "token" here is a content
chunk, as in the reference (the server sends one chunk per text delta).

    python minimal-inference_amd/benchmark.py --url http://127.0.0.1:8000 --batch-size 32 --runs 3
"""

from __future__ import annotations

import argparse
import asyncio
import json
import time


async def _one(client, endpoint: str, payload: dict, idx: int) -> dict:
    t0 = time.perf_counter()
    stamps: list[float] = []
    parts: list[str] = []
    finish = rid = None
    async with client.stream("POST", endpoint, json=payload) as resp:
        resp.raise_for_status()
        async for line in resp.aiter_lines():
            if not line.startswith("data: "):
                continue
            data = line[len("data: "):].strip()
            if data == "[DONE]":
                break
            try:
                msg = json.loads(data)
            except json.JSONDecodeError:
                continue
            rid = msg.get("id", rid)
            choice = msg["choices"][0]
            text = choice.get("delta", {}).get("content")
            if text:
                stamps.append(time.perf_counter())
                parts.append(text)
            if choice.get("finish_reason"):
                finish = choice["finish_reason"]
    total = time.perf_counter() - t0
    gaps = [b - a for a, b in zip(stamps, stamps[1:])]
    return {"request": idx, "tokens": len(stamps), "ttft_s": (stamps[0] - t0) if stamps else 0.0,
            "t2t_ms": 1000 * sum(gaps) / len(gaps) if gaps else 0.0, "total_s": total, "finish_reason": finish,
            "id": rid, "text": "".join(parts)}


async def run_benchmark(url: str, model: str = "", prompt: str = "Write a short poem about the ocean",
                        max_tokens: int = 100, batch_size: int = 1, runs: int = 3, verbose: bool = True) -> dict:
    import httpx

    endpoint = url.rstrip("/") + "/v1/chat/completions"
    payload = {"model": model, "messages": [{"role": "user", "content": prompt}], "max_tokens": max_tokens,
               "temperature": 0, "stream": True}
    ttft, t2t, agg, per_run = [], [], [], []
    for run in range(runs):
        t0 = time.perf_counter()
        async with httpx.AsyncClient(timeout=120) as client:
            res = await asyncio.gather(*(_one(client, endpoint, payload, i) for i in range(batch_size)))
        wall = time.perf_counter() - t0
        toks = sum(r["tokens"] for r in res)
        agg.append(toks / wall)
        ttft += [r["ttft_s"] for r in res if r["ttft_s"] > 0]
        t2t += [r["t2t_ms"] for r in res if r["t2t_ms"] > 0]
        per_run.append({"tokens": toks, "wall_s": wall, "aggregate_tok_s": toks / wall, "requests": res})
        if verbose:
            for r in res:
                print(f"  run {run + 1} req {r['request']}: {r['tokens']} tokens, TTFT {r['ttft_s'] * 1000:.1f} ms, "
                      f"avg T2T {r['t2t_ms']:.1f} ms, total {r['total_s']:.2f} s")
            print(f"  run {run + 1}: {toks} tokens in {wall:.2f} s ({toks / wall:.1f} tok/s aggregate)")
    out = {"batch_size": batch_size, "runs": runs, "max_tokens": max_tokens,
           "ttft_ms": 1000 * sum(ttft) / len(ttft) if ttft else None,
           "t2t_ms": sum(t2t) / len(t2t) if t2t else None,
           "aggregate_tok_s": sum(agg) / len(agg) if agg else None, "per_run": per_run}
    if verbose:
        print("--- Summary ---")
        if out["ttft_ms"] is not None:
            print(f"  TTFT (time to first token):    avg {out['ttft_ms']:.1f}ms")
        if out["t2t_ms"] is not None:
            print(f"  T2T  (per-request avg):        avg {out['t2t_ms']:.1f}ms "
                  f"({1000 / out['t2t_ms']:.1f} tok/s per stream)")
        if out["aggregate_tok_s"] is not None:
            print(f"  Aggregate throughput:          avg {out['aggregate_tok_s']:.1f} tok/s")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Benchmark TTFT / token-to-token latency of a streaming server")
    ap.add_argument("--url", default="http://127.0.0.1:8000")
    ap.add_argument("--model", default="")
    ap.add_argument("--prompt", default="Write a short poem about the ocean")
    ap.add_argument("--max-tokens", type=int, default=100)
    ap.add_argument("--batch-size", type=int, default=1)
    ap.add_argument("--runs", type=int, default=3)
    ap.add_argument("--json", action="store_true", help="print the summary as one JSON line")
    args = ap.parse_args(argv)
    if not args.json:
        print(f"Benchmarking {args.url} (model={args.model or 'default'})")
        print(f"Prompt: {args.prompt!r}, max_tokens={args.max_tokens}, batch_size={args.batch_size}, "
              f"runs={args.runs}\n")
    res = asyncio.run(run_benchmark(args.url, args.model, args.prompt, args.max_tokens, args.batch_size, args.runs,
                                    verbose=not args.json))
    if args.json:
        print(json.dumps({k: v for k, v in res.items() if k != "per_run"}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
