import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """One line per GPU-vs-oracle output comparison (tests/helpers.py check_close): the
    observed max-abs, cosine and how many elements exceeded 2e-2 (bf16) / 1e-4 (fp32)."""
    from helpers import PARITY_RECORDS
    if not PARITY_RECORDS:
        return
    tr = terminalreporter
    tr.section("parity summary")
    worst = max(r[2] for r in PARITY_RECORDS if r[5] == "bfloat16") if any(
        r[5] == "bfloat16" for r in PARITY_RECORDS) else 0.0
    for label, n, ma, cs, over, dt in PARITY_RECORDS:
        what = "differ" if dt == "bf16-ulp" else "over"
        tr.write_line(f"{label:<60s} {dt:<8s} n={n:<10d} max_abs={ma:.3e} cos={cs:.7f} "
                      f"{what}={over}")
    tr.write_line(f"{len(PARITY_RECORDS)} comparisons; largest bf16 max_abs {worst:.3e}; "
                  f"comparisons with elements above the max-abs bound: "
                  f"{sum(1 for r in PARITY_RECORDS if r[4] > 0 and r[5] != 'bf16-ulp')}")


@pytest.fixture(scope="session")
def oracle():
    from oracle import moe_oracle
    moe_oracle.build()
    return moe_oracle


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no GPU is visible")
    from pisceslx_amd import _lib
    _lib.lib()  # raises if libyvmoe.so is missing: no silent fallback
    return torch.device("cuda:0")
