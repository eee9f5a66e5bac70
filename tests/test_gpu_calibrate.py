"""GPU: the measured cost row re-measured on this device.

tiler_amd.calibrate repeats the work-span sweep (22 (rows, extent) cells x
the sum family's serial, split and tree realizations) and fits
cost = sum over stages (encoder + max(work / P, depth) * step), as the
reference fits its saturated-parallel-fold-steps row
(spikes/program-planning/reduction-dispatch-crossover/README.md:110-140).
The fitted P must agree with the profile's declared row within a factor of
two -- the row is a position on a contour, not a tight constant -- and the
fit must keep its decision accuracy: the serial-or-parallel verdict on at
least 10 of the 12 fit cells and 7 of the 10 held-out cells, a wrong verdict
costing at most 2.5x the best measured strategy.  The misses are near the
crossover.  The largest, about 2x, is one row of 1024, where the staged
serial fold's first load is as long as its chain and the work-span model
has no term for it.
"""
import pytest

from tiler_amd import _lib as L
from tiler_amd import calibrate

pytestmark = pytest.mark.gpu


def test_saturated_parallel_fold_steps_remeasured(ctx):
    declared = L.TargetProfile()
    assert L.lib().tiler_hip_profile_declare(declared) == L.OK
    result = calibrate.calibrate(ctx)
    p = result["saturated_parallel_fold_steps"]
    print(f"[calibrate] P={p:.4g} (declared {declared.saturated_parallel_fold_steps}) "
          f"encoder={result['encoder_seconds']:.3e} s step={result['step_seconds']:.3e} s "
          f"fit {result['fit']} held-out {result['held_out']}", flush=True)
    assert 0.5 <= p / declared.saturated_parallel_fold_steps <= 2.0
    assert result["fit"]["agreed"] >= 10 and result["held_out"]["agreed"] >= 7
    assert max(result["fit"]["worst_penalty"], result["held_out"]["worst_penalty"]) <= 2.5
