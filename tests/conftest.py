"""Shared test setup: repo root on sys.path, the `gpu` marker, device fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# The reference's regression cases (pyfiles/run_gqa_regression.py:13-20) plus the
# extra cases committed under tests/golden/ (see tests/golden/make_fixtures.py):
# name, mode, seq_len, seed (None = generator default 20260731), qpos, kv_block_len.
REFERENCE_CASES = (
    ("smoke_len1", "smoke", 1, None, None, 16),
    ("random_len15", "random", 15, 20260815, None, 16),
    ("random_len16", "random", 16, 20260816, None, 16),
    ("random_len17_bp", "random", 17, 20260817, None, 16),
    ("random_len30", "random", 30, 20260805, None, 16),
    ("random_len32_bp", "random", 32, 20260832, None, 16),
    ("smoke_len16_default", "smoke", 16, None, None, 16),
    ("smoke_len30_qpos11", "smoke", 30, None, 11, 16),
    ("random_len30_qpos17", "random", 30, 20260901, 17, 16),
    ("random_len1", "random", 1, 20260902, None, 16),
    ("random_len77_qpos40", "random", 77, 20260903, 40, 16),
    ("random_len130", "random", 130, 20260904, None, 16),
    ("random_len13_blk4", "random", 13, 20260905, None, 4),
)
DEFAULT_SEED = 20260731


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)
