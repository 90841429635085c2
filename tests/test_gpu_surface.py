"""The host-pointer surface (mojolearn_amd.linalg -> linalg_native_v1 -> gfx950 kernels) against
the reference's verify table: gemm-pinned, gemm-transposed and gemm-bf16 `train` hashes on
all nine fixtures (python/mojolearn/verify_reference/table.json), and the extension ops."""
import numpy as np
import pytest

import verify_lanes as VL

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", VL.FIXTURES)
def test_verify_lanes_through_the_surface(kind):
    from mojolearn_amd import linalg
    print(f"verify lanes {kind}", flush=True)
    X = VL.fixture_x(kind)
    cells = VL.golden()["cells"]
    assert VL.train_hash(VL.lane_gemm_pinned(linalg.matmul, X)) == cells[f"gemm-pinned/{kind}"]["train"]
    assert VL.train_hash(VL.lane_gemm_transposed(linalg.matmul, X)) == cells[f"gemm-transposed/{kind}"]["train"]
    assert VL.train_hash(VL.lane_gemm_bf16(linalg.to_bf16, linalg.matmul_bf16, X)) == \
        cells[f"gemm-bf16/{kind}"]["train"]


def test_surface_out_and_ops(oracle):
    from mojolearn_amd import linalg
    rng = np.random.default_rng(3)
    a = rng.standard_normal((37, 300)).astype(np.float32)
    b = rng.standard_normal((300, 41)).astype(np.float32)
    out = np.full((37, 41), -987654.0, np.float32)
    r = linalg.matmul(a, b, out=out)
    assert r is out
    assert np.array_equal(out.view(np.uint32), oracle.gemm(a, b, 0).view(np.uint32))
    nt = linalg.matmul(a, np.ascontiguousarray(b.T), transpose_b=True)
    tn = linalg.matmul(np.ascontiguousarray(a.T), b, transpose_a=True)
    assert np.array_equal(nt.view(np.uint32), out.view(np.uint32))
    assert np.array_equal(tn.view(np.uint32), out.view(np.uint32))


def test_surface_extensions(oracle):
    from mojolearn_amd import linalg
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 700)).astype(np.float32)
    codes = rng.integers(-127, 128, (700, 90), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, 90).astype(np.float32)
    y = linalg.matmul_int8w(x, codes, scales)
    want = oracle.gemm(x, oracle.int8_dequant(codes, scales, 0), 0)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    w = rng.standard_normal((700, 90)).astype(np.float32)
    bias = rng.standard_normal(90).astype(np.float32)
    y = linalg.linear(x, w, bias)
    assert np.array_equal(y.view(np.uint32), oracle.bias(oracle.gemm(x, w, 0), bias).view(np.uint32))
