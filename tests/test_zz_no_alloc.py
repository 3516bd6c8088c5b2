"""The allocation-free RMSNorm backward (vkh_rmsnorm_backward_noalloc, gain
partials in the library's fixed per-device array) against the allocating
entry point (vkh_rmsnorm_backward) through the C ABI: the same kernels, so the
outputs must be identical bit for bit, on two calls in a row with the second
smaller, with and without the residual and the gain gradient.  Sizes beyond
the array are refused with an error before any launch."""
import numpy as np
import pytest

import oracle as O
from helpers import dev, host, note, rel_l2, zeros

pytestmark = pytest.mark.gpu


def _run(fn, dy, x, w, res, rows, dim, want_dw):
    bdx = zeros(rows * dim)
    bdw = zeros(dim) if want_dw else None
    fn(dev(dy), dev(x), dev(w), bdx, bdw, rows, dim, 1e-6, residual=dev(res) if res is not None else None)
    return host(bdx), (host(bdw) if want_dw else None)


@pytest.mark.parametrize("shapes", [((2048, 1024), (300, 256)), ((4096, 4096), (7, 96))])
def test_rmsnorm_backward_noalloc_matches_allocating_entry_point(shapes):
    import valkyr_amd as v
    from valkyr_amd import kernels as K

    assert v.device_count() > 0
    for i, (rows, dim) in enumerate(shapes):
        note(f"noalloc rmsnorm backward call {i}: rows={rows} dim={dim}")
        x = O.normal(rows * dim, 100 + i)
        w = O.uniform(dim, 110 + i, 0.5, 1.5)
        dy = O.normal(rows * dim, 120 + i)
        res = O.normal(rows * dim, 130 + i) if i == 0 else None
        for want_dw in (False, True):
            dx0, dw0 = _run(K.rmsnorm_backward, dy, x, w, res, rows, dim, want_dw)
            dx1, dw1 = _run(K.rmsnorm_backward_noalloc, dy, x, w, res, rows, dim, want_dw)
            assert np.array_equal(dx0, dx1)
            if want_dw:
                assert np.array_equal(dw0, dw1)
        # and against the oracle (the fp32 bar)
        dx_ref, dw_ref = O.rmsnorm_backward(dy, x, w, 1e-6)
        if res is not None:
            dx_ref = dx_ref + res
        assert rel_l2(dx_ref, dx1) < 1e-5 and rel_l2(dw_ref, dw1) < 1e-5


def test_rmsnorm_backward_noalloc_refuses_oversize():
    import valkyr_amd as v
    from valkyr_amd import kernels as K

    a = zeros(16)
    with pytest.raises(v.VkhError) as e:
        K.rmsnorm_backward_noalloc(a, a, a, a, a, 4, 8192, 1e-6)
    assert e.value.name == "Unsupported"
