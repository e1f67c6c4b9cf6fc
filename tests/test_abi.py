"""CPU: the C-ABI library loads and exports every entry point the header declares."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mi_amd.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_path():
    syms = declared_symbols()
    for s in ("mi_paged_kv_append", "mi_decode_plan", "mi_decode_run", "mi_prefill_plan",
              "mi_prefill_run", "mi_sample", "mi_page_table_step", "mi_last_error"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from minimal_inference_amd import _lib

    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in sorted(declared_symbols()) if not hasattr(lib, s)]
    assert not missing, missing


def test_python_prototypes_match_header():
    from minimal_inference_amd import _lib

    assert set(_lib.SIGNATURES) == declared_symbols()


def test_host_only_calls_and_error_reporting():
    """Size queries and argument validation run without touching a GPU."""
    from minimal_inference_amd import _lib

    lib = _lib.load()
    assert lib.mi_version() >= 100
    assert lib.mi_decode_workspace_size(32, 32, 8, 128, 4096) > 0
    assert lib.mi_decode_workspace_size(4, 30, 8, 128, 0) == 0  # 30 % 8 != 0
    assert lib.mi_prefill_workspace_size(8, 4096) > 0
    assert lib.mi_page_table_state_size(1024, 8, 64) > 0
    # invalid arguments are rejected before any launch
    rc = lib.mi_paged_kv_append(None, 0, 0, None, 0, 0, None, None, 1, None, 0, None, None, None,
                                1, 2, 64, 16, None)
    assert rc == _lib.MI_ERR_INVALID
    assert "append" in _lib.last_error()
    rc = lib.mi_decode_plan(None, 0, None, None, None, 1, 32, 8, 96, 16, 0, None)
    assert rc == _lib.MI_ERR_UNSUPPORTED
    rc = lib.mi_decode_plan(None, 0, None, None, None, 1, 32, 8, 128, 16, 0, None)
    assert rc == _lib.MI_ERR_WORKSPACE
    # a run whose work list could not hold one item per request (max_units 4
    # for 8 KV heads) is refused before any launch, like the plan
    import ctypes

    ws = ctypes.create_string_buffer(1 << 20)
    rc = lib.mi_decode_run(ctypes.addressof(ws), 1 << 20, None, 0, 0, None, 0, None, None, 0, 0,
                           2, 32, 8, 128, 16, 0.0, 4, None)
    assert rc == _lib.MI_ERR_WORKSPACE
    assert "room for 4 units" in _lib.last_error()
    # the sampler takes at most 65,535 rows (one workgroup row each in the
    # launch grid's y dimension, one counter line each in the workspace)
    assert lib.mi_sample_workspace_size(65535, 32768) > lib.mi_sample_workspace_size(1, 32768) > 0
    assert lib.mi_sample_workspace_size(65536, 32768) == 0
    rc = lib.mi_sample(None, 32768, 65536, 32768, None, None, 0, None, None, None, 0, None)
    assert rc == _lib.MI_ERR_INVALID
    assert "over 65535 rows" in _lib.last_error()
    # prefill run: out rows must be 16-byte aligned, and a tile's q / out rows
    # must span at most 2^30 elements (its 32-bit buffer offsets); both refused
    # before any launch (the pointers are never dereferenced)
    need = lib.mi_prefill_workspace_size(1, 64)
    pws = ctypes.create_string_buffer(need)
    fake = 1 << 20
    args = dict(q_st=32 * 128, q_sh=128, out=fake, o_st=32 * 128, o_sh=128)

    def prefill_rc(**kw):
        a = {**args, **kw}
        return lib.mi_prefill_run(ctypes.addressof(pws), need, fake, a["q_st"], a["q_sh"], fake, 16, fake, a["out"],
                                  a["o_st"], a["o_sh"], 1, 64, 32, 8, 128, 16, 1, 0.0, None)

    assert prefill_rc(out=fake + 8) == _lib.MI_ERR_INVALID
    assert "16-byte aligned" in _lib.last_error()
    assert prefill_rc(q_sh=1 << 26) == _lib.MI_ERR_INVALID
    assert "2^30" in _lib.last_error()
