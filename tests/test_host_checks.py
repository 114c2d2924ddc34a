"""Host-side argument checks of the decomposed-linear wrappers (CPU: every check runs
before any pointer reaches the C ABI)."""

import pytest
import torch

from param_decomp_amd import _lib as L
from param_decomp_amd.decomposed_linear import (BlockedSiteWeights, SiteWeights, blocked_site_forward,
                                                site_forward)


def _site(dt_x=torch.bfloat16, dt_v=torch.bfloat16, dt_u=torch.bfloat16, dt_w=torch.bfloat16, C=8, bad_shape=False):
    T, d_in, d_out = 4, 16, 24
    x = torch.zeros(T, d_in, dtype=dt_x)
    V = torch.zeros(d_in + (8 if bad_shape else 0), C, dtype=dt_v)
    U = torch.zeros(C, d_out, dtype=dt_u)
    W = torch.zeros(d_out, d_in, dtype=dt_w)
    return x, SiteWeights(W, V, U), torch.zeros(T, C), torch.zeros(T)


@pytest.mark.parametrize("which", ["V", "U", "W"])
def test_site_forward_refuses_factor_dtype_mismatch(which):
    kw = {f"dt_{which.lower()}": torch.float32}
    x, w, mask, delta = _site(**kw)
    with pytest.raises(L.PDError, match=f"{which} is torch.float32"):
        site_forward(x, w, mask, delta, None)


def test_site_forward_refuses_shape_mismatch():
    x, w, mask, _ = _site(bad_shape=True)
    with pytest.raises(L.PDError, match="features"):
        site_forward(x, w, mask, None, None)
    x, w, _, _ = _site()
    with pytest.raises(L.PDError, match="mask shape"):
        site_forward(x, w, torch.zeros(4, 9), None, None)


def test_blocked_site_forward_refuses_dtype_and_shape_mismatch():
    E, d_in, d_out, c, T = 3, 8, 16, 4, 5
    x = torch.zeros(T, d_in, dtype=torch.bfloat16)
    V = torch.zeros(E, d_in, c, dtype=torch.bfloat16)
    U = torch.zeros(E, c, d_out, dtype=torch.float32)
    W = torch.zeros(E * d_out, d_in, dtype=torch.bfloat16)
    with pytest.raises(L.PDError, match="U is torch.float32"):
        blocked_site_forward(x, BlockedSiteWeights(W, V, U), torch.zeros(T, E * c), torch.zeros(T), None,
                             "fused_output")
    U = U.to(torch.bfloat16)
    with pytest.raises(L.PDError, match="W has shape"):
        blocked_site_forward(x, BlockedSiteWeights(W[:d_out], V, U), torch.zeros(T, E * c), torch.zeros(T), None,
                             "fused_output")
    with pytest.raises(L.PDError, match="features"):
        blocked_site_forward(x, BlockedSiteWeights(torch.zeros(d_out, E * d_in, dtype=torch.bfloat16), V, U),
                             torch.zeros(T, E * c), None, None, "fused_input")
