"""The C library's expf, logf and tanhf -- what every oracle function calls,
and what the reference's f32 exp / ln / tanh call on Linux -- against
correctly rounded values over dense sweeps: exp and log within 1 ulp, tanh
within 2 (glibc's documented bounds)."""
import numpy as np
import pytest

import oracle as O
from mathsweep import check, inputs


@pytest.mark.parametrize("which,name,bound", [(0, "expf", 1), (1, "logf", 1), (2, "tanhf", 2)])
def test_libm_rounding(which, name, bound):
    x = inputs(which)
    check(which, x, O.math_fn(which, x), bound, f"glibc {name}")
