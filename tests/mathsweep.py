"""Input sweeps and ULP distances for bounding the rounding of expf, logf and
tanhf (the transcendentals the kernels and the oracle call) against correctly
rounded values: the float64 function rounded to f32."""
import numpy as np

FLT_MIN = np.float32(1.1754944e-38)


def ordered(a):
    """f32 -> integers in value order (adjacent floats differ by 1; +0 = -0)."""
    i = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFFFFFF), i)


def ulps(a, b):
    return np.abs(ordered(a) - ordered(b))


def _between(lo, hi, n, rng):
    """n floats evenly spaced in bit pattern over [lo, hi] (one sign) and n
    uniformly random ones."""
    a, b = ordered(np.float32(lo)), ordered(np.float32(hi))
    grid = np.linspace(a, b, n).astype(np.int64)
    rnd = rng.integers(min(a, b), max(a, b) + 1, n)
    o = np.concatenate([grid, rnd])
    return np.where(o < 0, (-o) | 0x80000000, o).astype(np.uint32).view(np.float32)


def inputs(which, n=1 << 20):
    """which = 0 exp, 1 log, 2 tanh: the ranges the kernels feed them and the
    rest of the function's domain, with special values."""
    r = np.random.default_rng(7)
    if which == 0:  # softmax / cross-entropy take exp(x - max), x - max <= 0
        xs = [_between(-0.0, -104.0, n, r), _between(0.0, 88.7, n // 4, r),
              np.float32([0.0, -0.0, -np.inf, np.inf, np.nan, 1e-30, -1e-30, 89.0])]
    elif which == 1:  # cross-entropy's log of a sum of exps (>= 1)
        xs = [_between(1.0, 1e6, n, r), _between(FLT_MIN, 3.4e38, n, r),
              np.float32([1.0, 2.0, np.inf, 0.0, -0.0, -1.0, np.nan, 1e-45])]
    else:  # GELU's inner argument, any real
        xs = [_between(-0.0, -12.0, n, r), _between(0.0, 12.0, n, r), _between(12.0, 3.4e38, n // 16, r),
              np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-30, 9.1, -9.1])]
    return np.concatenate(xs).astype(np.float32)


def correctly_rounded(which, x):
    d = x.astype(np.float64)
    with np.errstate(all="ignore"):
        v = np.exp(d) if which == 0 else np.log(d) if which == 1 else np.tanh(d)
        return v.astype(np.float32)  # past FLT_MAX: inf, as f32 rounding gives


def check(which, x, y, max_ulp, name):
    """y = f(x) as some implementation computes it: NaN, infinities and
    signed zeros where the correctly rounded value has them, normal results
    within max_ulp, subnormal results within one subnormal step (2^-149).
    Returns the largest ULP distance seen on normal results."""
    ref = correctly_rounded(which, x)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(y), nan), f"{name}: NaN mismatch"
    inf = np.isinf(ref)
    assert np.array_equal(y[inf], ref[inf]), f"{name}: infinity mismatch"
    normal = ~nan & ~inf & (np.abs(ref) >= FLT_MIN)
    sub = ~nan & ~inf & ~normal
    u = ulps(y[normal], ref[normal])
    worst = int(u.max())
    assert worst <= max_ulp, f"{name}: {worst} ulp at x = {x[normal][u.argmax()]!r}"
    if sub.any():
        d = np.abs(y[sub].astype(np.float64) - ref[sub].astype(np.float64))
        assert d.max() <= 2.0 ** -149, f"{name}: subnormal result off by {d.max()}"
    return worst
