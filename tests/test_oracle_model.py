"""CPU: the oracle's model forward over the paged pool (oracle/model.py).

decode_step, run one token at a time over a paged pool whose pages are a
permutation, must give the same logits as dense_forward -- causal attention
on dense K / V over the whole sequence -- at every position: two independent
formulations of the reference forward (model.py:375-426) that agree only if
the page walk, the slot placement of the appended K / V, RoPE positions and
the GQA head mapping are all right.
"""

from __future__ import annotations

import math

import torch

from oracle import model as om


def _run_paged(w, s, ids, page_size, perm):
    """Decode ids one token at a time from position 0; logits of every step."""
    layers = len(w.layers)
    pools = [torch.zeros(max(perm) + 1, 2, page_size, s.kv_heads, s.head_dim) for _ in range(layers)]
    out = []
    for p in range(ids.shape[0]):
        npages = p // page_size + 1
        pages = perm[:npages]
        last = (p + 1) - (npages - 1) * page_size
        logits = om.decode_step(w, s, ids[p:p + 1], torch.tensor([p]), pools, [0, npages], pages, [last],
                                page_size=page_size)
        out.append(logits[0])
    return torch.stack(out)


def test_paged_decode_steps_equal_the_dense_causal_forward():
    s = om.Shape(hidden=64, heads=6, kv_heads=2, head_dim=16, intermediate=96, vocab=53, theta=10_000.0)
    w = om.random_weights(s, layers=3, seed=7)
    # larger weights than the N(0, 0.02) default so attention is far from uniform
    for L in w.layers:
        L["w_qkv"] *= 20
    ids = torch.randint(0, s.vocab, (23,), generator=torch.Generator().manual_seed(1))
    perm = [5, 2, 9, 0, 7, 3, 8]  # pages in a scrambled order
    paged = _run_paged(w, s, ids, page_size=4, perm=perm)
    dense = om.dense_forward(w, s, ids)
    assert torch.allclose(paged, dense, atol=1e-4, rtol=1e-4), (paged - dense).abs().max()


def test_paged_decode_catches_a_wrong_head_mapping():
    """The same check fails when KV head h % Hkv is read instead of h // group
    (a plausible mistake the dense form does not share)."""
    s = om.Shape(hidden=64, heads=6, kv_heads=2, head_dim=16, intermediate=96, vocab=53, theta=10_000.0)
    w = om.random_weights(s, layers=2, seed=3)
    for L in w.layers:
        L["w_qkv"] *= 20
    ids = torch.randint(0, s.vocab, (9,), generator=torch.Generator().manual_seed(2))
    dense = om.dense_forward(w, s, ids)

    def wrong_mapping(w, s, ids):
        # permute K/V head order within the projection: head h of the group
        # then reads the other KV head
        w2 = om.Weights(w.embed, w.lm_head, w.norm, [dict(L) for L in w.layers])
        d, hq, hkv = s.head_dim, s.heads, s.kv_heads
        for L in w2.layers:
            q, k, v = L["w_qkv"].split([hq * d, hkv * d, hkv * d])
            k = k.view(hkv, d, -1).flip(0).reshape(hkv * d, -1)
            L["w_qkv"] = torch.cat([q, k, v])
            L["b_qkv"] = L["b_qkv"].clone()
        return w2

    paged = _run_paged(wrong_mapping(w, s, ids), s, ids, page_size=4, perm=[1, 0, 2])
    assert not torch.allclose(paged, dense, atol=1e-3, rtol=1e-3)


def test_ragged_prefill_then_decode_equals_the_dense_forward():
    """Two prompts prefilled in one ragged batch (pages interleaved in the
    pool), then two decode steps of both: the last-prompt-token logits and each
    decode step's logits equal the dense causal forward of each sequence."""
    s = om.Shape(hidden=64, heads=6, kv_heads=2, head_dim=16, intermediate=96, vocab=53, theta=10_000.0)
    w = om.random_weights(s, layers=2, seed=11)
    for L in w.layers:
        L["w_qkv"] *= 20
    g = torch.Generator().manual_seed(5)
    seqs = [torch.randint(0, s.vocab, (n,), generator=g) for n in (11, 6)]  # prompt + 2 decoded tokens each
    prompts = [x[:-2] for x in seqs]
    ps = 4
    pages = [[6, 1, 4], [3, 0]]  # request 0: 9 prompt + 2 new tokens in 3 pages; request 1: 4 + 2 in 2
    pools = [torch.zeros(8, 2, ps, s.kv_heads, s.head_dim) for _ in w.layers]
    qo = [0, len(prompts[0]), len(prompts[0]) + len(prompts[1])]

    def csr(lens):
        npg = [math.ceil(n / ps) for n in lens]
        ip = [0, npg[0], npg[0] + npg[1]]
        ix = pages[0][: npg[0]] + pages[1][: npg[1]]
        return ip, ix, [n - (p - 1) * ps for n, p in zip(lens, npg)]

    ip, ix, last = csr([len(p) for p in prompts])
    got = om.prefill_step(w, s, torch.cat(prompts), qo, pools, ip, ix, last, page_size=ps)
    dense = [om.dense_forward(w, s, x) for x in seqs]
    for b in range(2):
        assert torch.allclose(got[b], dense[b][len(prompts[b]) - 1], atol=1e-4, rtol=1e-4)
    for j in range(2):
        pos = [len(p) + j for p in prompts]
        ip, ix, last = csr([p + 1 for p in pos])
        ids = torch.stack([seqs[b][pos[b]] for b in range(2)])
        got = om.decode_step(w, s, ids, torch.tensor(pos), pools, ip, ix, last, page_size=ps)
        for b in range(2):
            assert torch.allclose(got[b], dense[b][pos[b]], atol=1e-4, rtol=1e-4), (j, b)


def test_rms_norm_closed_form():
    x = torch.randn(5, 32, generator=torch.Generator().manual_seed(0), dtype=torch.float64)
    w = torch.rand(32, dtype=torch.float64) + 0.5
    want = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
    assert torch.allclose(om.rms_norm(x.float(), w.float(), 1e-6).double(), want, atol=1e-5)
    c = torch.full((1, 8), 3.0)  # constant row -> the weight (up to eps)
    assert torch.allclose(om.rms_norm(c, torch.ones(8), 0.0), torch.ones(1, 8))


def test_rope_identity_and_rotation():
    d, theta = 8, 10_000.0
    x = torch.randn(3, 2, d, generator=torch.Generator().manual_seed(4))
    assert torch.allclose(om.rope(x, torch.zeros(3, dtype=torch.long), d, theta), x)
    p = 5
    y = om.rope(x, torch.full((3,), p), d, theta)
    for j in range(d // 2):
        ang = p / theta ** (2 * j / d)
        c, sn = math.cos(ang), math.sin(ang)
        a, b = x[..., j], x[..., j + d // 2]
        assert torch.allclose(y[..., j], a * c - b * sn, atol=1e-5)
        assert torch.allclose(y[..., j + d // 2], b * c + a * sn, atol=1e-5)


def test_decode_mistakes_move_logits_beyond_the_engine_bound():
    """The end-to-end logits check of the GPU engine (config 2, bound
    E2E_LOGIT_REL_BOUND on max |engine - oracle| / max |oracle| per step) can
    see decode mistakes: planted here in the oracle's paged decode at the
    Qwen2.5-0.5B shape with its N(0, 0.02) weights, a position off by one
    (RoPE row and append slot) and a new token left out of its own attention
    each move the logits by more than the bound on every step after the
    prompt, while the correct paged decode matches the dense forward."""
    from tests.helpers import E2E_LOGIT_REL_BOUND

    s = om.Shape(896, 14, 2, 64, 4864, 151936)
    w = om.random_weights(s, layers=4, seed=1)
    w.lm_head = w.embed
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, s.vocab, (40,), generator=g)
    gen = torch.randint(0, s.vocab, (6,), generator=g)
    P, ps = prompt.numel(), 16
    dense = om.dense_forward(w, s, torch.cat([prompt, gen]))[P:]

    def paged(shift=0, drop_new=False):
        npg = math.ceil((P + gen.numel() + 2) / ps)
        pools = [torch.zeros(npg, 2, ps, s.kv_heads, s.head_dim, dtype=torch.bfloat16) for _ in w.layers]
        idx = list(range(npg))
        np0 = math.ceil(P / ps)
        om.prefill_step(w, s, prompt, [0, P], pools, [0, np0], idx, [P - (np0 - 1) * ps])
        out = []
        for k in range(gen.numel()):
            pos = P + k
            n = pos + 1 - (1 if drop_new else 0)  # tokens the attention sees
            npages = math.ceil(n / ps)
            out.append(om.decode_step(w, s, gen[k:k + 1], torch.tensor([pos + shift]), pools, [0, npages], idx,
                                      [n - (npages - 1) * ps])[0])
        return torch.stack(out)

    def rel(a):
        return ((a - dense).abs().amax(1) / dense.abs().amax(1))

    assert float(rel(paged()).max()) < 1e-2   # bf16 pool vs fp32 K / V only
    assert float(rel(paged(shift=1)).min()) > E2E_LOGIT_REL_BOUND
    assert float(rel(paged(drop_new=True)).min()) > E2E_LOGIT_REL_BOUND
