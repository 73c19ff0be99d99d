"""CPU checks of the parity summary the GPU tests feed (parity_log via
mla_bar.check_bar): the per-configuration lines, the literal-bar count and
the list of comparisons that needed the |ref| >= 2 exception."""
import numpy as np
import pytest

import mla_bar
import parity_log


@pytest.fixture
def clean_log(monkeypatch):
    monkeypatch.setattr(parity_log, "ATTENTION", [])
    monkeypatch.setattr(parity_log, "EXACT", [])
    return parity_log


def test_summary_lines(clean_log):
    want = np.array([0.5, -1.0, 2.5, 5.0] * 64, np.float32)
    mla_bar.check_bar(want + np.float32(1e-3), want, "small", config="rows16384_b1")
    flip = want.copy()
    flip[3] = 5.03125            # one bf16 ulp above 5.0: over 2e-2, within the exception
    mla_bar.check_bar(flip, want, "flip", config="rows262144_t3_b8")
    parity_log.record_exact("moe_align_b1_b8", "MoE align", 0, 96)
    lines = parity_log.summary_lines()
    text = "\n".join(lines)
    assert "rows16384_b1 attention" in text and "literal bar held by 1" in text
    assert "moe_align_b1_b8 MoE align: 0 of 96 differ" in text
    assert "all attention comparisons: 2; the literal bar (flat max-abs 2e-2, mean-abs 2e-3) held by 1" in text
    assert "[flip]: max-abs 0.03125, 1 of 256 elements over 2e-2, at most 1 bf16 ulp" in text


def test_bar_still_fails_beyond_the_exception(clean_log):
    want = np.array([5.0] * 8, np.float32)
    with pytest.raises(AssertionError):
        mla_bar.check_bar(want + np.float32(0.0625), want, "eight over")   # all 8 over 2e-2: more than max(2, n/1e5)
    with pytest.raises(AssertionError):
        mla_bar.check_bar(want + np.float32(0.03125), want, "one ulp, cap 0", max_ulp=0)
    assert len(parity_log.ATTENTION) == 2 and not any(r["literal"] for r in parity_log.ATTENTION)
