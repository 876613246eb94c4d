"""The device's expf, logf and tanhf, as the kernels call them (through
vh_math_probe, same functions and build), against correctly rounded values
over dense sweeps: exp within 1 ulp, log within 2, tanh within 1. With the C
library's bounds (tests/test_oracle_math.py: 1, 1, 2) that bounds every
transcendental the GPU and the oracle evaluate on the same f32 input to 2, 3
and 3 ulp apart, checked here directly as well."""
import numpy as np
import pytest

import oracle as O
from mathsweep import check, inputs, ulps
from parity import dev, fetch, out

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("which,name,dev_bound,cpu_bound", [(0, "expf", 1, 1), (1, "logf", 2, 1),
                                                           (2, "tanhf", 1, 2)])
def test_device_transcendentals_rounding(vh, which, name, dev_bound, cpu_bound):
    print(f"math probe {name}", flush=True)
    x = inputs(which)
    X, Y = dev(vh, x), out(vh, x.shape)
    vh.check(vh.lib.vh_math_probe(which, X.ptr, Y.ptr, x.size, None))
    y = fetch(vh, Y, x.shape)
    check(which, x, y, dev_bound, f"device {name}")
    c = O.math_fn(which, x)
    fin = np.isfinite(y) & np.isfinite(c)
    assert int(ulps(y[fin], c[fin]).max()) <= dev_bound + cpu_bound


def test_math_probe_rejects_bad_arguments(vh):
    X = dev(vh, np.ones(4, np.float32))
    assert vh.lib.vh_math_probe(3, X.ptr, X.ptr, 4, None) == vh.VH_ERR_INVALID
    assert "unknown function" in vh.last_error()
    assert vh.lib.vh_math_probe(0, None, X.ptr, 4, None) == vh.VH_ERR_INVALID
    assert vh.lib.vh_math_probe(0, X.ptr, X.ptr, 0, None) == 0
