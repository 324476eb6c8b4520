import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "nanosaur2-web_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def rel_errors(got, ref):
    """(max|d| / max|ref|, rel-L2) -- rel-L2 is the compare metric of tools/check.js:25-38."""
    import torch

    g = got.detach().double().cpu().reshape(-1)
    r = ref.detach().double().cpu().reshape(-1)
    assert g.numel() == r.numel(), (g.numel(), r.numel())
    assert torch.isfinite(g).all(), "non-finite output"
    d = g - r
    max_rel = (d.abs().max() / r.abs().max().clamp(min=1e-30)).item()
    rel_l2 = (d.norm() / r.norm().clamp(min=1e-30)).item()
    return max_rel, rel_l2


def assert_close(got, ref, tol, what=""):
    max_rel, rel_l2 = rel_errors(got, ref)
    print(f"[parity] {what}: max|d|/max|ref| {max_rel:.3e}  rel-L2 {rel_l2:.3e}  (tol {tol})", flush=True)
    assert max_rel <= tol and rel_l2 <= tol, f"{what}: max_rel {max_rel:.3e} rel_l2 {rel_l2:.3e} > {tol}"


@pytest.fixture(scope="session")
def ns2lib():
    """The HIP library bound on cuda:0 (GPU tests only)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a HIP device")
    import ns2

    lib = ns2.load(0)
    lib.set_stream(torch.cuda.current_stream().cuda_stream)
    return lib
