"""The caller-workspace entry and the fold stack's reach, on the GPU against the oracle.

* A skinny product's completion counters live in the caller's workspace (the first
  mlg_gemm_counter_bytes bytes), zeroed once when a Plan is made and left zero by every call:
  a Plan captured in a HIP graph on a stream that has never run a product replays correctly,
  and two Plans of one shape on two streams at once each keep their own counters.
* A Plan sizes its workspace for the operands it is given: a view whose storage offset is not
  on the 16-byte grid is repacked into the workspace, not refused.
* Leaf-group roots past 1024 per cell (a ten-slot stack's reach): a skinny product and a tile
  product with a caller leaf of 1 fold 4100, 5000 and 1250 roots per cell, bit for bit.
"""
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


def _skinny(rng, m=2, n=1000, k=4096):
    a = rng.standard_normal((m, k)).astype(np.float32)
    codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    return a, codes, scales


def test_plan_captured_on_a_fresh_stream(oracle):
    from mojolearn_amd import device as D
    rng = np.random.default_rng(101)
    a, codes, scales = _skinny(rng)
    want = oracle.gemm_fast(a, oracle.int8_dequant(codes, scales, 0), 0)
    plan = D.Plan(_t(a), _t(codes), scales=_t(scales))
    assert D.route(2, 1000, 4096, b_type=D.T_I8, a=plan._keep[0], b=plan._keep[1]) >= {"gemv_groups"}
    s = torch.cuda.Stream()  # no product has ever run on it; nothing is called before the capture
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        plan(s)
    for rep in range(3):
        plan.out.fill_(POISON)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(plan.out.cpu().numpy()), _bits(want)), f"replay {rep}"
        D.gemm(_t(a), _t(np.ascontiguousarray(codes[:, :300], dtype=np.float32)))  # eager work between


def test_two_plans_of_one_shape_on_two_streams(oracle):
    from mojolearn_amd import device as D
    rng = np.random.default_rng(102)
    a1, codes, scales = _skinny(rng)
    a2 = rng.standard_normal(a1.shape).astype(np.float32)
    tc, ts = _t(codes), _t(scales)
    p1, p2 = D.Plan(_t(a1), tc, scales=ts), D.Plan(_t(a2), tc, scales=ts)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    wdeq = oracle.int8_dequant(codes, scales, 0)
    w1, w2 = oracle.gemm_fast(a1, wdeq, 0), oracle.gemm_fast(a2, wdeq, 0)
    for rep in range(5):
        p1.out.fill_(POISON)
        p2.out.fill_(POISON)
        torch.cuda.synchronize()
        for _ in range(3):
            p1(s1)
            p2(s2)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(p1.out.cpu().numpy()), _bits(w1)), f"plan 1, round {rep}"
        assert np.array_equal(_bits(p2.out.cpu().numpy()), _bits(w2)), f"plan 2, round {rep}"


@pytest.mark.parametrize("offset", [1, 3])
def test_plan_on_an_offset_view(oracle, offset):
    from mojolearn_amd import device as D
    rng = np.random.default_rng(103 + offset)
    m, n, k = 150, 170, 700
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    store = torch.empty(m * k + offset, dtype=torch.float32, device=DEV)
    view = store[offset:].view(m, k)  # contiguous, base off the 16-byte grid
    view.copy_(_t(a))
    assert "repack" in D.route(m, n, k, a=view, b=None)
    plan = D.Plan(view, _t(b))
    plan.out.fill_(POISON)
    plan()
    torch.cuda.synchronize()
    assert np.array_equal(_bits(plan.out.cpu().numpy()), _bits(oracle.gemm_fast(a, b, 0)))


@pytest.mark.parametrize("shape", [(1, 64, 16400), (2, 70, 20000), (17, 17, 40000)],
                         ids=["gemv-4100-roots", "gemv-5000-roots", "tile-1250-roots"])
def test_roots_past_1024(oracle, shape):
    from mojolearn_amd import device as D
    m, n, k = shape
    rng = np.random.default_rng(k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
    D.gemm(_t(a), _t(b), leaf=1, out=out)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(oracle.gemm(a, b, 0, leaf=1)))
