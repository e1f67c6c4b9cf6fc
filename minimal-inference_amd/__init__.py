"""MI355X-native ragged paged-attention path of minimal-inference.

Importable as ``minimal_inference_amd`` (the directory name carries a hyphen;
``load_package()`` in the repository's entry points registers it).

Public surface (mirrors what the reference's model.py / scheduler.py call):
  page.append_paged_kv_cache                        -- model.py:207-216
  decode.BatchDecodeWithPagedKVCacheWrapper         -- scheduler.py:535-539
  prefill.BatchPrefillWithPagedKVCacheWrapper       -- scheduler.py:530-534
  sampling.sample_batch / sample                    -- scheduler.py:310-343
  kv_cache.PagedKVCache / build_csr_metadata        -- scheduler.py:168-302
  kv_cache.DevicePageTable                          -- GPU page table + CSR build
  engine.Scheduler / engine.AttentionBackend        -- scheduler.py:229-259, 477+
  model.Model / model.ModelConfig                   -- model.py:37-435 (dense torch)

All attention, append, sampling and page-table work runs in the HIP library
``libmi_amd.so`` (built by ``build.py``); there is no CPU fallback.
"""

from __future__ import annotations

__all__ = ["lib_path", "load_library"]


def lib_path():
    from ._lib import LIB_PATH

    return LIB_PATH


def load_library():
    """Load the HIP library (raises RuntimeError when it is not built)."""
    from . import _lib

    return _lib.load()
