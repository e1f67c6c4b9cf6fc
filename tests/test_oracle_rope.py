"""Pins the RoPE oracle (oracle/rope.py) without the kernel.

Checks are chosen so that a plausible mistake fails one of them: a swapped
half or sign (plane-rotation closed form), a wrong frequency index (closed
form at several positions), fp32 kept between the three bf16 ops (explicit
rounding-order evaluation), a wrong table cast (position 0 identity).
"""

from __future__ import annotations

import math

import torch

from oracle import rope


def _rand_rows(t, h, d, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(t, h, d, generator=g).to(torch.bfloat16)


def test_position_zero_is_identity():
    cos, sin = rope.tables(128, 8, 1e6)
    x = _rand_rows(3, 4, 128, 0)
    out = rope.apply(x, cos[[0, 0, 0]], sin[[0, 0, 0]])
    assert torch.equal(out, x)


def test_plane_rotation_closed_form():
    d, theta = 64, 10000.0
    cos, sin = rope.tables(d, 300, theta)
    x = _rand_rows(4, 2, d, 1)
    pos = [1, 17, 123, 299]
    out = rope.apply(x, cos[pos], sin[pos]).double()
    xd = x.double()
    for r, p in enumerate(pos):
        for j in range(d // 2):
            ang = p * (1.0 / theta ** (2 * j / d))
            c, s = math.cos(ang), math.sin(ang)
            a, b = xd[r, :, j], xd[r, :, j + d // 2]
            want_a = a * c - b * s
            want_b = b * c + a * s
            # bf16 tables and three bf16 roundings: a few ulps of |x|
            tol = 0.03 * (a.abs() + b.abs()) + 1e-6
            assert ((out[r, :, j] - want_a).abs() <= tol).all()
            assert ((out[r, :, j + d // 2] - want_b).abs() <= tol).all()


def test_rotations_compose():
    d = 128
    cos, sin = rope.tables(d, 64, 1e6)
    x = _rand_rows(1, 8, d, 2)
    once = rope.apply(x, cos[[30]], sin[[30]]).double()
    twice = rope.apply(rope.apply(x, cos[[10]], sin[[10]]), cos[[20]], sin[[20]]).double()
    assert (once - twice).abs().max().item() < 0.05 * x.double().abs().max().item()
    # and a rotation preserves each pair's norm
    n0 = x.double()[..., :64] ** 2 + x.double()[..., 64:] ** 2
    n1 = once[..., :64] ** 2 + once[..., 64:] ** 2
    assert ((n1 - n0).abs() <= 0.03 * n0 + 1e-4).all()


def test_bf16_rounding_order():
    """out = bf16(bf16(x*c) + bf16(r*s)) element by element, not fp32 fused."""
    d = 128
    cos, sin = rope.tables(d, 2048, 1e6)
    x = _rand_rows(5, 3, d, 3) * 37
    pos = [0, 5, 511, 1024, 2047]
    out = rope.apply(x, cos[pos], sin[pos])
    half = d // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)
    p1 = (x.float() * c.float()).to(torch.bfloat16)
    p2 = (rot.float() * s.float()).to(torch.bfloat16)
    want = (p1.float() + p2.float()).to(torch.bfloat16)
    assert torch.equal(out, want)
    fused = (x.float() * c.float() + rot.float() * s.float()).to(torch.bfloat16)
    assert not torch.equal(out, fused)  # the check above can tell the two apart


def test_rope_append_sequence():
    """rope_append = rotate q / k, then the paging oracle's append."""
    hq, hkv, d, ps = 4, 2, 64, 16
    cos, sin = rope.tables(d, 64, 1e4)
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(3, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    pool = torch.zeros(6, 2, ps, hkv, d, dtype=torch.bfloat16)
    q, out = rope.rope_append(qkv, hq, hkv, [3, 40, 99], cos, sin, pool, [0, 1, 3], [4, 1, 2], [0, 1, 1],
                              [3, 20, 40])
    assert torch.equal(q[1], rope.apply(qkv[1:2, : hq * d].view(1, hq, d), cos[[40]], sin[[40]])[0])
    k0 = rope.apply(qkv[0:1, hq * d: (hq + hkv) * d].view(1, hkv, d), cos[[3]], sin[[3]])[0]
    assert torch.equal(out[4, 0, 3], k0)
    assert torch.equal(out[2, 1, 4], qkv[1, (hq + hkv) * d:].view(hkv, d))  # pos 20 -> page idx 1 -> page 2, slot 4
    assert torch.count_nonzero(out[[0, 3, 5]]) == 0
    # position 99 clamps to the last table row (63) for the rotation
    q2 = rope.apply(qkv[2:3, : hq * d].view(1, hq, d), cos[[63]], sin[[63]])[0]
    assert torch.equal(q[2], q2)
