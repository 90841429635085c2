"""mlg_gemm_noalloc, the entry for callers that cannot allocate: its output against mlg_gemm_ws's
(a Plan with its own workspace) bit for bit, on two calls in a row, the second with a smaller
product, for products whose kernels use scratch (leaf-group roots + fold, the skinny kernels'
completion counters and roots); and the refusal of a product that needs more scratch than the
library's array holds.
"""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"
POISON = -987654.0


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def _noalloc(a, b, scales=None, bias=None, b_type=0, leaf=0):
    from mojolearn_amd import _native
    m, k = a.shape
    n = b.shape[1]
    out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    rc = _native.lib().mlg_gemm_noalloc(out.data_ptr(), a.data_ptr(), b.data_ptr(),
                                        None if scales is None else scales.data_ptr(),
                                        None if bias is None else bias.data_ptr(), m, n, k, 0, 0, b_type, leaf, s)
    _native.check(rc)
    return out


def _with_ws(a, b, scales=None, bias=None, leaf=0):
    from mojolearn_amd import device as D
    plan = D.Plan(a, b, scales=scales, bias=bias, leaf=leaf)
    plan.out.fill_(POISON)
    plan()
    return plan.out


def _pair(rng, kind, size):
    if kind == "skinny_i8":
        m, n, k = {"big": (16, 14336, 4096), "small": (2, 1000, 4096)}[size]
        a = rng.standard_normal((m, k)).astype(np.float32)
        codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        return _t(a), _t(codes), _t(scales), None, 2
    m, n, k = {"big": (512, 512, 512), "small": (150, 170, 8192)}[size]
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    return _t(a), _t(b), None, _t(bias), 0


@pytest.mark.parametrize("kind", ["skinny_i8", "tile_groups"])
def test_noalloc_equals_workspace_entry(kind):
    from mojolearn_amd import device as D
    rng = np.random.default_rng(55)
    for size in ("big", "small"):
        a, b, scales, bias, b_type = _pair(rng, kind, size)
        m, k = a.shape
        n = b.shape[1]
        need = D.workspace_bytes(m, n, k, b_type=b_type, a=a, b=b)
        assert 0 < need <= 32 << 20, need  # the product does use scratch, within the array
        got = _noalloc(a, b, scales, bias, b_type)
        want = _with_ws(a, b, scales, bias)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(got.cpu().numpy()), _bits(want.cpu().numpy())), (kind, size)


def test_noalloc_refuses_a_product_beyond_its_scratch():
    from mojolearn_amd import _native
    from mojolearn_amd import device as D
    # one tile of 17 x 17 cells and 2^20 leaves of one step: 32768 groups of 32 leaves, whose
    # roots need 36 MiB
    m, n, k = 17, 17, 1 << 20
    assert D.workspace_bytes(m, n, k, leaf=1) > 32 << 20
    a = torch.zeros((m, k), dtype=torch.float32, device=DEV)
    b = torch.zeros((k, n), dtype=torch.float32, device=DEV)
    out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
    rc = _native.lib().mlg_gemm_noalloc(out.data_ptr(), a.data_ptr(), b.data_ptr(), None, None, m, n, k, 0, 0, 0, 1,
                                        torch.cuda.current_stream().cuda_stream)
    assert rc != 0
    assert "scratch" in _native.lib().mlg_last_error().decode()
    torch.cuda.synchronize()
    assert np.all(out.cpu().numpy() == np.float32(POISON))  # nothing launched
