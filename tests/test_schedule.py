"""The attention kernels' tile/phase schedule, replayed on the host by the same
code the GPU runs (ttcd_amd/csrc/schedule.h via ttcd_attn_schedule_coverage):
every (query, key) pair inside a window is folded into that window's output
exactly once, and no pair outside it ever is. This is the brute-force coverage
check for the double-accumulation bug the reference records as a strict xfail
(test/test_fused_dual_attn.py:253-272) and for the narrow-gap segment
(test/test_fused_attn_narrow_gap.py)."""
from __future__ import annotations

import numpy as np
import pytest

from ttcd_amd import _lib


def _coverage(T, dual, a, b, group=2):
    near = np.zeros((T, T), dtype=np.int32)
    far = np.zeros((T, T), dtype=np.int32)
    st = _lib.lib().ttcd_attn_schedule_coverage(T, int(dual), a, b, group, near.ctypes.data,
                                                far.ctypes.data)
    if st != 0:
        raise AssertionError(_lib.lib().ttcd_last_error().decode())
    return near, far


def _band(T, lo, hi):
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    d = i - j
    return ((d >= lo) & (d < hi)).astype(np.int32)


DUAL_CASES = [
    (257, -1, 192), (257, 257, 257), (256, 256, 256), (769, 512, 256), (513, -1, 256),
    (300, 200, 199), (300, 100, 1), (300, 40, 7), (1000, 233, 97), (640, 600, 33),
    (700, 300, 268), (700, 300, 269), (1100, 1000, 999), (64, 64, 1), (1, 1, 1),
    (1300, 1216, 1024), (1300, 560, 512), (900, 4128, 4096), (513, 500, 500),
]


@pytest.mark.parametrize("group", [2, 3])
@pytest.mark.parametrize("T,wt,ws", DUAL_CASES)
def test_dual_schedule_covers_each_pair_once(T, wt, ws, group):
    near, far = _coverage(T, True, ws, wt, group)
    WT = T if wt < 0 else wt
    np.testing.assert_array_equal(near, _band(T, 0, ws))
    np.testing.assert_array_equal(near + far, _band(T, 0, WT))
    np.testing.assert_array_equal(far, _band(T, ws, WT))


@pytest.mark.parametrize("wt,ws", [(4128, 4096), (4160, 4096), (4224, 4096), (1216, 1024),
                                   (8192, 4096), (8192, 7168), (8192, 8064)])
def test_dual_schedule_narrow_gaps_subsampled(wt, ws):
    # The reference's narrow-gap windows (and BASELINE's 7168/8064 gaps) at a T long
    # enough for every tile/boundary pattern to occur.
    T = 8192 + 384
    near, far = _coverage(T, True, ws, wt, 1 + (wt % 2))
    np.testing.assert_array_equal(near, _band(T, 0, ws))
    np.testing.assert_array_equal(far, _band(T, ws, wt))


@pytest.mark.parametrize("T,lo,hi", [(257, 0, 192), (769, 0, 512), (769, 256, 512),
                                     (500, 499, 10**6), (300, 0, 1), (300, 7, 8),
                                     (129, 128, 129), (64, 100, 200), (1000, 97, 233)])
@pytest.mark.parametrize("group", [1, 2])
def test_band_schedule_covers_each_pair_once(T, lo, hi, group):
    near, far = _coverage(T, False, lo, hi, group)
    np.testing.assert_array_equal(near, _band(T, lo, hi))
    assert not far.any()
