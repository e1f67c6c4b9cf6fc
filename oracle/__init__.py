"""CPU oracle for the ragged paged-attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's
paged-attention hot path so that the HIP kernels can be checked against it.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only to check results (or as the timed CPU
baseline); the product package never imports it and has no CPU fallback.

Modules:
  paging     -- page pool layout, FIFO page allocator replay, CSR builder,
                KV append (integer / byte exact).
  attention  -- gather-based paged decode and causal prefill attention in fp32.
  sampling   -- greedy argmax, bf16 temperature quantisation, the fp32
                (top-p restricted) sampling distribution.
  rope       -- rotate-half RoPE tables and the bf16 op sequence of the
                reference, and the unfused RoPE-then-append sequence.
  model      -- the model forward over the paged pool in fp32 (one decode
                step, and the dense causal forward that pins it); the CPU
                baseline of the end-to-end decode.

Pinning status per function is recorded in each module's docstring.
"""
