"""Host-side pieces of the MLA composition (CPU): the YaRN position tables the
package builds match the oracle's restatement of YaRNRotaryEmbedding."""
import numpy as np
import pytest

from oracle import mla as ol


@pytest.mark.parametrize("s", [1, 64, 2048])
def test_yarn_tables_match_oracle(s):
    """Same formulas; both are fp32, and the angle t * inv_freq reaches ~2047 rad,
    where one ulp of inv_freq moves it by ~1e-4 rad: absolute 2e-4 at s=2048
    (the kernels use the tables rounded to bf16, a 4e-3 step)."""
    from ds_kernels import mla as dm
    cos, sin = dm.yarn_cos_sin(s)
    rc, rs = ol.yarn_cos_sin(s)
    tol = 2e-6 if s <= 64 else 2e-4
    np.testing.assert_allclose(cos.numpy(), rc, rtol=0, atol=tol)
    np.testing.assert_allclose(sin.numpy(), rs, rtol=0, atol=tol)


def test_softmax_scale():
    from ds_kernels import mla as dm
    import torch
    W = dm.MLAWeights(q=torch.zeros(1), kva=torch.zeros(1), kva_norm=torch.zeros(1),
                      kvb=torch.zeros(1), o=torch.zeros(1))
    m = 0.1 * 0.707 * np.log(40.0) + 1.0
    assert abs(W.softmax_scale - 192 ** -0.5 * m * m) < 1e-12
