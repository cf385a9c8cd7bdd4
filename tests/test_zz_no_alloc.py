"""The allocation-free entry point gphip_refine_logdet_f32_noalloc (no counterpart in the
reference; for callers that cannot allocate device memory) against gphip_refine_logdet_f32,
the entry point it is a variant of, through the C ABI: two calls in a row, the second on a
smaller problem, each bit-identical to the allocating entry point's result (the same kernels on
the same inputs), and the rejection of a table beyond its fixed scratch."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _problem(N, n0, k, nbins, seed):
    import graphgp_hip as G
    rng = np.random.default_rng(seed)
    pts = rng.random((N, 3))
    bins, vals = G.rbf_kernel(1.0, 0.08, 1e-4, 2.0, nbins, jitter=1e-5)
    return G.build_graph(pts, n0, k, bins.astype(np.float32), vals.astype(np.float32))


def _logdet(torch, fn, prob):
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    coords, nbr, bins, vals = d(prob.coords), d(prob.neighbors), d(prob.bins), d(prob.vals)
    out = torch.full((1,), float("nan"), dtype=torch.float32, device="cuda")
    rc = fn(coords.data_ptr(), C.c_float(prob.scale), nbr.data_ptr(), bins.data_ptr(),
            vals.data_ptr(), out.data_ptr(), prob.n0, prob.K, prob.N, len(prob.bins), prob.D,
            None)
    torch.cuda.synchronize()
    return rc, float(out.cpu()[0])


def test_noalloc_matches_allocating_entry_point(gpu):
    from graphgp_hip import _native as nat
    lib = nat.hip()
    big = _problem(20000, 300, 8, 1000, seed=1)
    small = _problem(3000, 100, 5, 600, seed=2)
    for name, prob in (("20000 points, k=8, 1000 bins", big), ("3000 points, k=5, 600 bins", small)):
        _say(f"case noalloc {name}")
        rc, want = _logdet(gpu, lib.gphip_refine_logdet_f32, prob)
        assert rc == 0, lib.ggp_last_error()
        rc, got = _logdet(gpu, lib.gphip_refine_logdet_f32_noalloc, prob)
        assert rc == 0, lib.ggp_last_error()
        _say(f"  noalloc {got!r} vs allocating {want!r}")
        assert np.isfinite(got) and got == want
    # a table beyond the fixed scratch is rejected before any launch
    rc, _ = _logdet(gpu, lib.gphip_refine_logdet_f32_noalloc, _problem(600, 60, 8, 3000, seed=3))
    assert rc == 7 and b"2048" in lib.ggp_last_error()
