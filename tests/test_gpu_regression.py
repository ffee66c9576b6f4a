"""The reference regression flow end to end on the GPU (tests/regression.py, the
flow of pyfiles/run_gqa_regression.py with the kernel in place of Vivado/XSim)."""
from __future__ import annotations

import pytest

import regression

pytestmark = pytest.mark.gpu


def test_regression_flow(dev, tmp_path, capsys):
    rc = regression.run(tmp_path, in_process=True)
    out = capsys.readouterr().out
    print(out)
    assert rc == 0
    assert "GQA REGRESSION PASSED: 6 datapath cases plus invalid-config rejection" in out
    assert out.count("] PASS") == 7
