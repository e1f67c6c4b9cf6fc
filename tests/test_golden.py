"""CPU: the committed config-1 fixture is self-consistent and the oracle reproduces it."""

from __future__ import annotations

from pathlib import Path

import torch
from safetensors.torch import load_file

from oracle import attention as oatt

FIX = Path(__file__).resolve().parent / "golden" / "c1_decode.safetensors"


def load_pool(t):
    pool = torch.zeros(128, 2, 16, 2, 64, dtype=torch.bfloat16)
    pool[t["page_ids"].long()] = t["pages"]
    return pool


def test_fixture_shapes_and_page_table():
    t = load_file(str(FIX))
    assert t["q"].shape == (4, 14, 64) and t["q"].dtype == torch.bfloat16
    assert t["indptr"].tolist() == [0, 2, 6, 19, 51]
    assert t["last_page_len"].tolist() == [1, 16, 11, 15]
    assert len(set(t["page_ids"].tolist())) == 51 and max(t["page_ids"].tolist()) < 128
    assert t["out_fp32"].shape == (4, 14, 64) and t["out_fp32"].dtype == torch.float32


def test_oracle_reproduces_fixture():
    t = load_file(str(FIX))
    got = oatt.decode(t["q"], load_pool(t), t["indptr"].tolist(), t["page_ids"].tolist(),
                      t["last_page_len"].tolist())
    assert torch.equal(got, t["out_fp32"])
