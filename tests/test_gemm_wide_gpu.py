"""The persistent GEMM's wide tile (256 x 256, kernels/gemm_big.h), which
vh_gemm takes for products whose B is row-contiguous, with at least
VH_GEMMB_WIDE_K (8192) of K in whole k tiles and N >= 256 -- the block step's
lm_head dW ([50260, 768] = dlogits^T ln_f) and the drop-in's lm_head dx and
weight gradients. Both such layouts (kn, mn), edges in M and N, a k tail left
to the tiled kernel, bias / accumulate / alpha epilogues, operands only
4-byte aligned, and the stream-K round with its fix-up (fixed order: the same
bits on a second call); beside them the long-K products the narrow tile keeps
(both operands k-contiguous, or A row-contiguous with B k-contiguous).
Against the oracle, float64 and the f32 error bound of a K-term sum (the
checks of test_gemm_persistent_block_shapes)."""
import pytest

from test_block_ops_gpu import test_gemm_persistent_block_shapes as check_persistent

pytestmark = pytest.mark.gpu

# a_scale 1e-2: a sum of 8192-50260 random-sign products of N(0, 1) x
# N(0, 0.05^2) terms has magnitude ~5 and f32 rounding noise ~1e-5, the bar's
# absolute term; at the scale of the block step's operands (activations times
# ~1e-4 dlogits, as the existing lm_head cases use) the elementwise bar
# compares the products themselves. The unscaled case keeps the check that
# holds at any scale: the f32 error bound of a K-term sum.
#   name, M, N, K, A k-contiguous, B k-contiguous, epilogue, a_scale[, offset]
WIDE_CASES = [
    ("kn, lm_head dx shape, K tail", 512, 768, 50260, True, False, "", 1e-3),
    ("kn, alpha, bases one float off, K tail", 300, 1001, 9000, True, False, "alpha", 1e-2, 1),
    ("kn, edges, bias + residual", 520, 600, 8224, True, False, "bias_acc", 1e-2),
    ("mn, lm_head dW shape [V, D]", 1000, 768, 16384, False, False, "", 1e-2),
    ("mn, lm_head dW^T shape [D, V]", 768, 1000, 16384, False, False, "", 1e-2),
    ("mn, odd M and N, 4-byte aligned", 1001, 777, 8192, False, False, "alpha_acc", 1e-2, 1),
    ("narrow tile: kk, edges, bias + residual", 520, 600, 8224, True, True, "bias_acc", 1e-2),
    ("narrow tile: mk, far-apart B rows", 1024, 768, 8192, False, True, "", 1.0),
]


@pytest.mark.parametrize("case", WIDE_CASES, ids=[c[0] for c in WIDE_CASES])
def test_gemm_persistent_wide_tile(vh, case):
    check_persistent(vh, case)
