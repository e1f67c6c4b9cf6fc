"""GPU: fused residual add + RMSNorm and SiLU-gated product vs torch.

Bars: the residual sum x + delta is bit-exact with torch's bf16 add; the
normalised output is within one bf16 rounding of an fp32 evaluation of
rms_norm(x + delta) * w (and of torch's F.rms_norm); SiLU * up is within one
bf16 ulp of torch's F.silu(g) * u.  The model's prefill logits with the fused
kernels agree with the unfused torch ops (relative 2e-2).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _ulp_close(a: torch.Tensor, b: torch.Tensor, ulps: int = 1) -> bool:
    """|a - b| <= ulps bf16 ulps of max(|a|, |b|) elementwise (bf16 inputs)."""
    a32, b32 = a.float(), b.float()
    mag = torch.maximum(a32.abs(), b32.abs())
    ulp = torch.where(mag > 0, torch.pow(2.0, torch.floor(torch.log2(mag)) - 7), torch.zeros_like(mag))
    return bool(((a32 - b32).abs() <= ulps * ulp + 1e-30).all())


@pytest.mark.parametrize("hidden", [896, 3584, 4096, 8192])
@pytest.mark.parametrize("rows", [1, 5, 32, 300])
def test_add_rms_norm(dev, hidden, rows):
    from minimal_inference_amd.dense import add_rms_norm

    g = torch.Generator(device=dev).manual_seed(hidden + rows)
    x = torch.randn(rows, hidden, device=dev, generator=g).to(torch.bfloat16)
    d = (torch.randn(rows, hidden, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, device=dev, generator=g)).to(torch.bfloat16)
    want_x = x + d
    x_run = x.clone()
    h = add_rms_norm(x_run, d, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(x_run, want_x)
    xf = want_x.float()
    ref = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    assert _ulp_close(h, ref.to(torch.bfloat16), 1)
    assert _ulp_close(h, F.rms_norm(want_x, (hidden,), w, 1e-6), 2)


def test_add_rms_norm_modes(dev):
    """No delta (norm only, x untouched); sum only (no norm); strided rows."""
    from minimal_inference_amd.dense import add_rms_norm

    x = torch.randn(7, 1024, device=dev).to(torch.bfloat16)
    w = torch.ones(1024, device=dev, dtype=torch.bfloat16)
    x0 = x.clone()
    h = add_rms_norm(x, None, w, 1e-5, write_x=False)
    torch.cuda.synchronize()
    assert torch.equal(x, x0)
    xf = x.float()
    assert _ulp_close(h, (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16))
    d = torch.randn(7, 1024, device=dev).to(torch.bfloat16)
    assert add_rms_norm(x, d, w, 1e-5, norm=False) is None
    torch.cuda.synchronize()
    assert torch.equal(x, x0 + d)
    big = torch.randn(7, 2048, device=dev).to(torch.bfloat16)
    xv = big[:, 512:1536]                               # row stride 2048
    want = xv + d
    hv = add_rms_norm(xv, d, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(big[:, 512:1536], want)
    wf = want.float()
    assert _ulp_close(hv, (wf * torch.rsqrt(wf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16))


@pytest.mark.parametrize("rows,inter", [(1, 4864), (32, 14336), (300, 18944), (5, 29568)])
def test_silu_mul(dev, rows, inter):
    from minimal_inference_amd.dense import silu_mul

    gu = (torch.randn(rows, 2 * inter, device=dev) * 3).to(torch.bfloat16)
    got = silu_mul(gu)
    g, u = gu.chunk(2, dim=-1)
    want = F.silu(g) * u
    torch.cuda.synchronize()
    assert got.shape == (rows, inter)
    assert _ulp_close(got, want, 1)
    assert (got == want).float().mean().item() > 0.99


def test_rejects_bad_shapes(dev):
    from minimal_inference_amd.dense import add_rms_norm, silu_mul

    with pytest.raises(ValueError):
        add_rms_norm(torch.zeros(2, 12, device=dev, dtype=torch.bfloat16), None,
                     torch.ones(12, device=dev, dtype=torch.bfloat16), 1e-6)     # hidden % 8
    with pytest.raises(ValueError):
        silu_mul(torch.zeros(2, 10, device=dev, dtype=torch.bfloat16))          # intermediate % 8
    with pytest.raises(ValueError):
        add_rms_norm(torch.zeros(2, 16, device=dev, dtype=torch.float32), None,
                     torch.ones(16, device=dev, dtype=torch.bfloat16), 1e-6)     # dtype


def test_model_prefill_logits_fused_vs_unfused(dev):
    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model

    cfg = PRESETS["qwen2.5-0.5b"]
    cfg = type(cfg)(**{**cfg.__dict__, "num_hidden_layers": 6})
    logits = []
    for fused in (True, False):
        model = Model(cfg, dev, seed=5, max_positions=512, fused_dense=fused)
        sch = Scheduler(model, max_batch_size=4, max_seq_len=256, use_graphs=False)
        g = torch.Generator().manual_seed(9)
        for i, n in enumerate([12, 77, 200]):
            sch.submit(Request(str(i), torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist(), 1, 0.0))
        captured = {}
        orig = model.forward

        def spy(*a, **k):
            captured["l"] = orig(*a, **k)
            return captured["l"]

        model.forward = spy
        sch._prefill(sch._admit())
        logits.append(captured["l"].float())
    rel = (logits[0] - logits[1]).abs().max().item() / logits[1].abs().max().item()
    assert rel < 2e-2, rel
