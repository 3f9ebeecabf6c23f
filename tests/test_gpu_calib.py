"""The calibration program behind bench.py's roofline.load_only_ceiling
(fasth3inc_amd/csrc/fh3_calib.hip): its gemv mode runs on the GPU and the
bench's own parser reads a time for both GEMV weight sizes, each at or above
what the published 8 TB/s allows (a stream cannot beat the peak)."""
import importlib.util
import os

import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def _bench():
    spec = importlib.util.spec_from_file_location("bench_for_test", os.path.join(H.ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_load_only_ceiling_parses(gpu):
    B = _bench()
    if not os.path.exists(B.CALIB):
        pytest.fail("%s is not built (python -m fasth3inc_amd.build)" % B.CALIB)
    sizes = [14745600] * 3 + [50135040] * 3
    alg = sum(sizes)
    c = B.load_only_ceiling(sizes, alg, 0.075)
    print("ceiling:", c, flush=True)
    assert c and "error" not in c, c
    for b, t in c["best_us_per_launch"].items():
        assert t * 1e-6 >= int(b) / B.HBM_PEAK, (b, t)
    assert 0 < c["frac"] < 1
    assert abs(c["us_per_step"] - sum(c["best_us_per_launch"][str(b)] for b in sizes)) < 0.05
