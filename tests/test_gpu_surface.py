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


def _device_product(kind, a, b, op, extra=None):
    """The same product through the device-pointer entries, which the parity suite pins."""
    import torch
    from mojolearn_amd import device
    ta = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    tb = torch.from_numpy(np.ascontiguousarray(b)).to("cuda:0")
    if kind == "f32":
        c = device.gemm(ta, tb, op=op)
    elif kind == "bias":
        c = device.gemm(ta, tb, op=op, bias=torch.from_numpy(extra).to("cuda:0"))
    elif kind == "bf16":
        c = device.gemm_bf16w(ta, tb, op=op)
    else:
        c = device.gemm_int8w(ta, tb, torch.from_numpy(extra).to("cuda:0"), op=op)
    torch.cuda.synchronize()
    return c.cpu().numpy()


# (kind, m, n, k, op): A of 16 MB or more is cut into row bands of 256-row multiples
# (2304 x 4096 f32: bands of 1280 + 1024; 3000 x 4096 NT: 1024 + 1024 + 952), OP_TN and
# small products take one band; 512 x 8320 x 512 is 260 tiles, on 256 CUs the whole-rounds +
# grouped-tail split inside the surface's own stream-ordered workspace
BAND_CASES = [("f32", 2304, 640, 4096, 0), ("f32", 3000, 384, 4096, 1), ("f32", 640, 512, 8192, 2),
              ("bias", 2304, 520, 4096, 0), ("bf16", 4100, 256, 2048, 1), ("int8", 2500, 1000, 4096, 0),
              ("f32", 37, 41, 300, 0), ("f32", 512, 8320, 512, 0), ("bias", 512, 8320, 512, 0),
              ("int8", 512, 8320, 512, 1)]


@pytest.mark.parametrize("case", BAND_CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-op{c[4]}" for c in BAND_CASES])
def test_host_bands_equal_device_product(oracle, case):
    from mojolearn_amd import linalg
    kind, m, n, k, op = case
    print(f"host bands {case}", flush=True)
    rng = np.random.default_rng(m + n + k + op)
    a = rng.standard_normal((k, m) if op == 2 else (m, k)).astype(np.float32)
    bshape = (n, k) if op == 1 else (k, n)
    extra = None
    if kind == "bf16":
        b = linalg.to_bf16(rng.standard_normal(bshape).astype(np.float32))
        got = linalg.matmul_bf16(a, b, transpose_a=op == 2, transpose_b=op == 1)
    elif kind == "int8":
        b = rng.integers(-127, 128, bshape, dtype=np.int8)
        extra = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        got = linalg.matmul_int8w(a, b, extra, transpose_b=op == 1)
    elif kind == "bias":
        b = rng.standard_normal(bshape).astype(np.float32)
        extra = rng.standard_normal(n).astype(np.float32)
        got = linalg.linear(a, b, extra, transpose_b=op == 1)
    else:
        b = rng.standard_normal(bshape).astype(np.float32)
        got = linalg.matmul(a, b, transpose_a=op == 2, transpose_b=op == 1)
    want = _device_product(kind, a, b, op, extra)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} words differ, first at {divmod(int(bad[0]), n)}"
    if kind == "f32":
        # rows on both sides of every band edge against the oracle
        rows = sorted({r for e in (1024, 1280, 2048) for r in (e - 1, e) if r < m} | {0, m - 1})
        A = a.T if op == 2 else a
        B = b.T if op == 1 else b
        sub = oracle.gemm(np.ascontiguousarray(A[rows]), np.ascontiguousarray(B), 0)
        assert np.array_equal(got[rows].view(np.uint32), sub.view(np.uint32))


def test_host_out_and_concurrent_callers():
    """A caller-given `out` (pages already resident) and two threads at once: the second caller
    finds the pooled set busy and takes fresh buffers with plain copies; both give the same bits."""
    import threading
    from mojolearn_amd import linalg
    rng = np.random.default_rng(17)
    a = rng.standard_normal((2048, 2048)).astype(np.float32)
    b = rng.standard_normal((2048, 1024)).astype(np.float32)
    want = linalg.matmul(a, b)
    out = np.full_like(want, -1.0)
    assert linalg.matmul(a, b, out=out) is out
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    results, errors = [None] * 4, []

    def one(i):
        try:
            results[i] = linalg.matmul(a, b)
        except Exception as exc:  # noqa: BLE001
            errors.append(exc)

    threads = [threading.Thread(target=one, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for r in results:
        assert np.array_equal(r.view(np.uint32), want.view(np.uint32))


def test_host_staged_conversions(oracle):
    """Conversions large enough for the staged transport (several chunks each way)."""
    from mojolearn_amd import linalg
    rng = np.random.default_rng(23)
    x = rng.standard_normal((3000, 2100)).astype(np.float32)
    bits = linalg.to_bf16(x)
    assert np.array_equal(bits, oracle.bf16_narrow(x))
    assert np.array_equal(linalg.from_bf16(bits).view(np.uint32), oracle.bf16_widen(bits).view(np.uint32))
    codes, exps = linalg.quantize_int8(x)
    oc, oe = oracle.q8_quantize(x)
    assert np.array_equal(codes, oc) and np.array_equal(exps, oe)
    y = linalg.dequantize_int8(codes, exps)
    assert np.array_equal(y.view(np.uint32), oracle.nan_canon(oracle.q8_dequantize(oc, oe)).view(np.uint32))


def test_host_out_aliasing_a():
    """`out` over A's own memory (whole, or starting halfway into it): A is read whole before any
    of C is written, so the product is the one of the original A."""
    from mojolearn_amd import linalg
    rng = np.random.default_rng(29)
    m, k, n = 3072, 3072, 3072
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    want = linalg.matmul(a.copy(), b)
    got = linalg.matmul(a, b, out=a)
    assert got is a and np.array_equal(a.view(np.uint32), want.view(np.uint32))
    m, k, n = 2048, 4096, 1536
    buf = rng.standard_normal(m * k + m * n).astype(np.float32)
    A = buf[:m * k].reshape(m, k)
    B = rng.standard_normal((k, n)).astype(np.float32)
    want = linalg.matmul(A.copy(), B)
    out = buf[m * k // 2:m * k // 2 + m * n].reshape(m, n)
    linalg.matmul(A, B, out=out)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
