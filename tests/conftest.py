"""Shared pytest setup: the ``gpu`` marker, package loading, device fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from __graft_entry__ import load_package  # noqa: E402

load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def lib():
    from minimal_inference_amd import _lib

    return _lib.load()


# (test id, case, max-abs error, scaled error) of every parity check of the session
_PARITY: list[tuple[str, str, float, float]] = []
TOL_ABS = 2e-2      # the path's contract: max-abs against the fp32 oracle
TOL_SCALED = 1.2e-2  # bound on max |out - ref| / max(1, |ref|): three bf16 roundings of u = 2^-8 each


@pytest.fixture
def parity(request):
    """``parity(out, ref, case="")``: compare a bf16 kernel result with the
    fp32 oracle; record the max-abs error and the scaled error
    max |out - ref| / max(1, |ref|) for the end-of-session table; assert
    max-abs <= 2e-2 (the contract) and scaled <= 1.2e-2.

    The kernels round to bf16 (unit roundoff u = 2^-8) up to three times on
    the way to an output: the softmax weights P before the P.V product, a
    split's partial O rows (decode), and the output.  Each rounding moves the
    result by at most u of the magnitude it rounds, so the scaled bound is
    3u = 1.17e-2 rounded up; observed errors are 0.3u to 2.1u (the table).  The
    max-abs error grows with the output's magnitude through the same
    roundings, which is why the tighter bound is on the scaled error."""

    def check(out, ref, case=""):
        e = (out.float() - ref.float()).abs()
        err = float(e.max()) if e.numel() else 0.0
        scaled = float((e / ref.float().abs().clamp(min=1.0)).max()) if e.numel() else 0.0
        _PARITY.append((request.node.nodeid, case, err, scaled))
        assert err <= TOL_ABS, f"{request.node.nodeid} {case}: max-abs {err:.3e} > {TOL_ABS:.0e}"
        assert scaled <= TOL_SCALED, f"{request.node.nodeid} {case}: scaled error {scaled:.3e} > {TOL_SCALED:.1e}"
        return err

    return check


# free-form result lines of tests (error tables and the like), printed at the end
_REPORT: list[tuple[str, str]] = []


@pytest.fixture
def report(request):
    """``report(line)``: keep a result line for the end-of-session summary."""

    def add(line: str):
        _REPORT.append((request.node.nodeid, line))

    return add


def pytest_terminal_summary(terminalreporter):
    tr = terminalreporter
    if _REPORT:
        tr.section("test reports")
        for nodeid, line in _REPORT:
            tr.write_line(f"{nodeid}: {line}")
    if not _PARITY:
        return
    tr.section(f"parity vs the fp32 oracle: max-abs (bound {TOL_ABS:.0e}), scaled (bound {TOL_SCALED:.1e})")
    for nodeid, case, err, scaled in _PARITY:
        tr.write_line(f"abs {err:.3e}  scaled {scaled:.3e} ({100 * scaled / TOL_SCALED:3.0f}% of bound)  "
                      f"{nodeid} {case}".rstrip())
