"""Fused batched sampler -- drop-in for the reference's ``sample_batch`` /
``sample`` (scheduler.py:310-343), plus top-p.

``sample_batch(logits [B, S, V], temperatures)`` keeps the reference's
contract: temperatures are rounded to the logits dtype (bf16), rows with
temperature <= 0 are greedy (argmax, first index on ties), the rest draw one
token from softmax(logits / t) in fp32.  One fused kernel per call replaces
softmax + multinomial + argmax + masked index-put; the only host sync is the
final ``.tolist()``, as in the reference.

``Sampler`` is the allocation-free form for graph capture: it owns device
buffers for per-row temperature / top-p, the output ids, the Philox counter
and the kernels' workspace (sized at construction for ``vocab`` when given,
else for the largest vocabulary seen; a workspace that grows is replaced but
kept alive, so a graph captured with the old one never writes into freed
memory), so a captured decode step can include the draw.
"""

from __future__ import annotations

import torch

from . import _lib
from ._util import require_dtype, require_gpu, stream_of

_DEFAULT_SEED = 0x6D69616D64  # "miamd"


class Sampler:
    """Per-device sampler state: rng counter and reusable row buffers."""

    def __init__(self, device: torch.device, max_batch: int, seed: int = _DEFAULT_SEED, vocab: int | None = None):
        self.device = torch.device(device)
        self.max_batch = max_batch
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.rng_offset = torch.zeros(1, dtype=torch.int64, device=self.device)
        self.temperature = torch.zeros(max_batch, dtype=torch.float32, device=self.device)
        self.top_p = torch.ones(max_batch, dtype=torch.float32, device=self.device)
        self.out = torch.zeros(max_batch, dtype=torch.int64, device=self.device)
        self.workspace = torch.zeros(0, dtype=torch.uint8, device=self.device)
        self._retired: list[torch.Tensor] = []  # replaced workspaces a captured graph may still use
        if vocab is not None:
            self._workspace_for(vocab)

    def _workspace_for(self, vocab: int) -> torch.Tensor:
        need = int(_lib.load().mi_sample_workspace_size(self.max_batch, vocab))
        if self.workspace.numel() < need:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"sampler workspace for vocab {vocab} must be sized before graph capture")
            if self.workspace.numel():
                self._retired.append(self.workspace)
            self.workspace = torch.zeros(need, dtype=torch.uint8, device=self.device)  # counters start at zero
        return self.workspace

    def set_params(self, temperatures, top_p=None) -> None:
        """Copy per-row parameters in (asynchronous host->device copies)."""
        n = len(temperatures)
        if n > self.max_batch:
            raise ValueError(f"{n} rows exceed the sampler's max_batch {self.max_batch}")
        t = torch.as_tensor(temperatures, dtype=torch.float32)
        self.temperature[:n].copy_(t, non_blocking=True)
        if top_p is None:
            self.top_p[:n].fill_(1.0)
        else:
            self.top_p[:n].copy_(torch.as_tensor(top_p, dtype=torch.float32), non_blocking=True)

    def sample(self, logits: torch.Tensor, n: int | None = None, out: torch.Tensor | None = None,
               use_top_p: bool = True) -> torch.Tensor:
        """Draw ids for rows 0..n-1 of ``logits`` [B, V] (or [B, 1, V])."""
        if logits.dim() == 3:
            logits = logits[:, -1, :]
        require_gpu("logits", logits)
        require_dtype("logits", logits, torch.bfloat16)
        if logits.dim() != 2 or logits.stride(1) != 1:
            raise ValueError("logits must be [B, V] with a contiguous vocab axis")
        n = logits.shape[0] if n is None else n
        if n > self.max_batch:
            raise ValueError(f"{n} rows exceed the sampler's max_batch {self.max_batch}")
        out = self.out if out is None else out
        ws = self._workspace_for(logits.shape[1])
        _lib.call(
            "mi_sample", logits.data_ptr(), logits.stride(0), n, logits.shape[1],
            self.temperature.data_ptr(), self.top_p.data_ptr() if use_top_p else None,
            self.seed, self.rng_offset.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), stream_of(logits),
        )
        return out[:n]


_samplers: dict[tuple[int, int], Sampler] = {}


def _sampler_for(device: torch.device, batch: int) -> Sampler:
    key = (device.index or 0, batch)
    s = _samplers.get(key)
    if s is None:
        s = Sampler(device, max(batch, 1))
        _samplers[key] = s
    return s


def sample_batch(logits: torch.Tensor, temperatures: list[float], top_p: list[float] | None = None) -> list[int]:
    """Sample one id per row of ``logits`` [B, S, V] (last position)."""
    if logits.dim() != 3:
        raise ValueError(f"logits must be [B, S, V]; got {tuple(logits.shape)}")
    b = logits.shape[0]
    if len(temperatures) != b:
        raise ValueError("one temperature per row is required")
    s = _sampler_for(logits.device, b)
    s.set_params(temperatures, top_p)
    ids = s.sample(logits[:, -1, :], b, use_top_p=top_p is not None)
    return ids.tolist()


def sample(logits: torch.Tensor, temperature: float, top_p: float | None = None) -> int:
    """Single request: logits [1, S, V] -> one id (scheduler.py:310-316)."""
    return sample_batch(logits[:1], [temperature], None if top_p is None else [top_p])[0]
