"""The allocation-free build (dance_vamana_build_resident_noalloc) against
dance_vamana_build_resident through the C ABI: identical graphs, degrees and
medoids on two calls in a row, the second with a smaller input; inputs above
the scratch maximum are rejected before any device work."""
import numpy as np
import pytest

import dance_amd as D

pytestmark = pytest.mark.gpu


def _build(fn, torch, x, R, L, C, steps):
    dev = torch.device("cuda:0")
    xt = torch.from_numpy(x).to(dev)
    n, dim = x.shape
    g = torch.full((n, R), -7, dtype=torch.int32, device=dev)
    d = torch.full((n,), -7, dtype=torch.int32, device=dev)
    code = D.DTYPE_F32 if x.dtype == np.float32 else D.DTYPE_U8
    fn(xt.data_ptr(), code, n, dim, R, L, C, steps, g.data_ptr(), d.data_ptr())
    torch.cuda.synchronize()
    medoid = int(D.lib().gpu_vamana_vnew2_get_last_medoid())
    return g.cpu().numpy().view(np.uint32), d.cpu().numpy().view(np.uint32), medoid


@pytest.mark.parametrize("kind", ["f32", "u8"])
def test_noalloc_equals_resident_twice(kind):
    import torch
    cases = [(100_000, 64, 100, 80, 64), (6_000, 32, 64, 48, 32)]  # second call smaller
    for n, R, L, C, steps in cases:
        if kind == "f32":
            x = D.synth_f32(42, 0, n, 96, 256, 0.3, True)
        else:
            x = D.synth_u8(42, 0, n, 128, 1024, 0.3)
        print(f"[noalloc] {kind} N={n} R={R} L={L} C={C} STEPS={steps}", flush=True)
        gn, dn, mn = _build(D.vamana_build_resident_noalloc, torch, x, R, L, C, steps)
        gr, dr, mr = _build(D.vamana_build_resident, torch, x, R, L, C, steps)
        assert mn == mr
        assert np.array_equal(dn, dr)
        assert np.array_equal(gn, gr)


def test_noalloc_rejects_inputs_beyond_scratch():
    import torch
    n, dim = 400_000, 96
    dev = torch.device("cuda:0")
    xt = torch.zeros((n, dim), dtype=torch.float32, device=dev)
    g = torch.empty((n, 64), dtype=torch.int32, device=dev)
    d = torch.empty((n,), dtype=torch.int32, device=dev)
    rc = D.lib().dance_vamana_build_resident_noalloc(xt.data_ptr(), D.DTYPE_F32, n, dim, 64, 100, 80, 64,
                                                     g.data_ptr(), d.data_ptr())
    assert rc == -1
