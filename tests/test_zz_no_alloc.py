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


def test_rmsnorm_backward_noalloc_allocates_nothing():
    """The entry point's defining property: the library's allocation counter
    (device and pinned allocations and scratch-buffer leases) does not move
    across noalloc calls of different sizes, on the default stream and on a
    second stream, while the allocating entry point moves it on every call."""
    import valkyr_amd as v
    from valkyr_amd import kernels as K
    from valkyr_amd.device import Stream, synchronize

    s2 = Stream()
    calls = []
    for i, (rows, dim) in enumerate([(2048, 1024), (300, 256), (7, 96), (4096, 4096)]):
        x, w = O.normal(rows * dim, 200 + i), O.uniform(dim, 210 + i, 0.5, 1.5)
        dy = O.normal(rows * dim, 220 + i)
        calls.append((rows, dim, dev(dy), dev(x), dev(w), zeros(rows * dim), zeros(dim)))
    synchronize()
    count = v.lib().vkh_allocation_count
    before = count()
    for i, (rows, dim, bdy, bx, bw, bdx, bdw) in enumerate(calls):
        K.rmsnorm_backward_noalloc(bdy, bx, bw, bdx, bdw, rows, dim, 1e-6,
                                   stream=(s2 if i % 2 else None))
    s2.synchronize()
    synchronize()
    after = count()
    note(f"  allocation count {before} -> {after} over {len(calls)} noalloc calls")
    assert after == before
    rows, dim, bdy, bx, bw, bdx, bdw = calls[0]
    K.rmsnorm_backward(bdy, bx, bw, bdx, bdw, rows, dim, 1e-6)
    synchronize()
    assert count() > after  # the counter does see the allocating form


def test_rmsnorm_backward_noalloc_ordered_across_streams():
    """Calls enqueued back to back on two streams, with no host
    synchronisation between them, share the fixed array; each must still see
    its own gain partials (the library orders them with a per-device event)."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import Stream

    rows, dim = 2048, 1024
    note("noalloc rmsnorm backward on two streams sharing the array")
    s1, s2 = Stream(), Stream()
    cases = []
    for seed in (51, 61, 71, 81):
        x, w = O.normal(rows * dim, seed), O.uniform(dim, seed + 1, 0.5, 1.5)
        dy = O.normal(rows * dim, seed + 2)
        cases.append((x, w, dy, O.rmsnorm_backward(dy, x, w, 1e-6)))
    bufs = [(dev(x), dev(w), dev(dy), zeros(rows * dim), zeros(dim)) for x, w, dy, _ in cases]
    for i, (bx, bw, bdy, bdx, bdw) in enumerate(bufs):
        K.rmsnorm_backward_noalloc(bdy, bx, bw, bdx, bdw, rows, dim, 1e-6,
                                   stream=(s1 if i % 2 else s2))
    s1.synchronize()
    s2.synchronize()
    for (x, w, dy, (dx_ref, dw_ref)), (_, _, _, bdx, bdw) in zip(cases, bufs):
        assert rel_l2(dx_ref, host(bdx)) < 1e-5
        assert rel_l2(dw_ref, host(bdw)) < 1e-5
