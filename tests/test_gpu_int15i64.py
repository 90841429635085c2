"""Profile mojolearn.identical.gemm.int15i64.v1 on gfx950 (plane product on the integer matrix
unit, quantizer, dequantizer) and from_f16 against the CPU oracle, bit for bit
(gemm/IDENTICAL_LOWBIT_CONTRACT.md section 6; gemm/linalg_native.mojo:395-576).  Covers ragged
m/n, k not a multiple of the 64-code slice (repacked planes), misaligned planes, split k, the
contract's bound cases (the code -16383 everywhere at k = 65536; -16257, whose cross term is the
largest), exponent sums past both ends, and the surface's gemm-int15 verify cells."""
import numpy as np
import pytest

import verify_lanes as VL

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _dev():
    from mojolearn_amd import device
    return device


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _bits_equal(got, want, what):
    g = np.ascontiguousarray(got).view(np.uint32).ravel()
    w = np.ascontiguousarray(want).view(np.uint32).ravel()
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} words differ; first at {bad[0]}: "
                           f"got {g[bad[0]]:#010x} want {w[bad[0]]:#010x}")


def _planes(q):
    q = np.asarray(q, np.int64)
    return (q >> 7).astype(np.int8), (q & 127).astype(np.int8)


def _run(oracle, qa, qb, ea, eb, what):
    ah, al = _planes(qa)
    bh, bl = _planes(qb)
    c = _dev().gemm_int15i64(_t(ah), _t(al), _t(ea), _t(bh), _t(bl), _t(eb))
    torch.cuda.synchronize()
    _bits_equal(c.cpu().numpy(), oracle.nan_canon(oracle.q15_gemm(ah, al, ea, bh, bl, eb)), what)


# (1, 4096, 4096), (8, 300, 14336), (33, 47, 65536) and (16, 129, 385) split k;
# k % 64 != 0 takes the repack
SHAPES = [(1, 1, 1), (3, 5, 7), (130, 129, 64), (128, 128, 128), (129, 257, 129), (200, 300, 4097),
          (64, 1000, 520), (512, 512, 512), (1, 4096, 4096), (8, 300, 14336), (33, 47, 65536), (16, 129, 385),
          (2, 77, 1024), (3, 333, 2064), (4, 4096, 4096), (1, 129, 4112), (4, 3, 65536)]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
def test_gemm_int15_vs_oracle(oracle, shape):
    m, n, k = shape
    print(f"int15 gemm {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m * 5 + n * 3 + k)
    qa = rng.integers(-16383, 16384, (m, k))
    qb = rng.integers(-16383, 16384, (n, k))
    qa[0, :] = -16383  # hi = -128 on every lane
    qb[0, :] = -16257  # (hi, lo) = (-128, 127): the largest cross term
    ea = rng.integers(-40, 40, m).astype(np.int32)
    eb = rng.integers(-40, 40, n).astype(np.int32)
    _run(oracle, qa, qb, ea, eb, "int15")


def test_gemm_int15_bounds():
    """k = 65536 with the code -16383 on both operands (HH = -128 * -128 per term, the Int32
    bound), and -16257 on both (MID at its bound): the exact sums, rounded once."""
    from oracle import oracle as O
    k = 65536
    for code in (-16383, -16257, 16383):
        q = np.full((2, k), code, np.int64)
        e0 = np.zeros(2, np.int32)
        ah, al = _planes(q)
        c = _dev().gemm_int15i64(_t(ah), _t(al), _t(e0), _t(ah), _t(al), _t(e0))
        torch.cuda.synchronize()
        want = np.array([code * code * k], np.int64).astype(np.float32)[0]
        assert (c.cpu().numpy() == want).all(), code
        _bits_equal(c.cpu().numpy(), O.q15_gemm(ah, al, e0, ah, al, e0), f"bound {code}")


def test_gemm_int15_exponent_edges(oracle):
    rng = np.random.default_rng(21)
    m, n, k = 70, 90, 300
    qa = rng.integers(-300, 300, (m, k))
    qb = rng.integers(-300, 300, (n, k))
    qa[1] = 0
    ea = rng.integers(-140, 116, m).astype(np.int32)
    eb = rng.integers(-140, 116, n).astype(np.int32)
    _run(oracle, qa, qb, ea, eb, "edges")


@pytest.mark.parametrize("offset", [1, 16])
def test_gemm_int15_misaligned_planes(oracle, offset):
    rng = np.random.default_rng(offset + 7)
    m, n, k = 150, 77, 192
    qa = rng.integers(-16383, 16384, (m, k))
    qb = rng.integers(-16383, 16384, (n, k))
    ea = np.zeros(m, np.int32)
    eb = np.full(n, -5, np.int32)
    planes = []
    for q, rows in ((qa, m), (qb, n)):
        for p in _planes(q):
            buf = torch.zeros(rows * k + 64, dtype=torch.int8, device=DEV)
            t = buf[offset:offset + rows * k].view(rows, k)
            t.copy_(_t(p))
            planes.append(t)
    c = _dev().gemm_int15i64(planes[0], planes[1], _t(ea), planes[2], planes[3], _t(eb))
    torch.cuda.synchronize()
    ah, al = _planes(qa)
    bh, bl = _planes(qb)
    _bits_equal(c.cpu().numpy(), oracle.nan_canon(oracle.q15_gemm(ah, al, ea, bh, bl, eb)), "misaligned")


def _rows15(rng, rows, cols):
    x = (rng.standard_normal((rows, cols)) * np.exp2(rng.uniform(-30, 30, (rows, 1)))).astype(np.float32)
    if rows >= 8:
        x[0] = 0.0
        x[1, ::3] = np.nan
        x[2, 0] = np.inf
        x[3] = (x[3] * np.float32(1e-38)).astype(np.float32)
        x[4] = np.float32(2.0 ** -120) * np.sign(x[4]).astype(np.float32)  # 2^-e infinite
        x[4, ::5] = 0.0
        x[6] = np.ldexp(np.round(rng.standard_normal(cols) * 8192) + 0.5, -3).astype(np.float32)  # ties
    return x


@pytest.mark.parametrize("shape", [(1, 1), (8, 5), (33, 300), (9, 5000), (300, 4096)])
def test_quantize_dequantize_int15_vs_oracle(oracle, shape):
    rows, cols = shape
    print(f"int15 quantize {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    x = _rows15(rng, rows, cols)
    D = _dev()
    hi, lo, exps = D.int15_quantize(_t(x))
    torch.cuda.synchronize()
    wh, wl, we = oracle.q15_quantize(x)
    assert np.array_equal(hi.cpu().numpy(), wh)
    assert np.array_equal(lo.cpu().numpy(), wl)
    assert np.array_equal(exps.cpu().numpy(), we)
    y = D.int15_dequantize(hi, lo, exps)
    torch.cuda.synchronize()
    _bits_equal(y.cpu().numpy(), oracle.nan_canon(oracle.q15_dequantize(wh, wl, we)), "dequantize")
    e2 = rng.integers(-150, 150, rows).astype(np.int32)
    y2 = D.int15_dequantize(hi, lo, _t(e2))
    torch.cuda.synchronize()
    _bits_equal(y2.cpu().numpy(), oracle.nan_canon(oracle.q15_dequantize(wh, wl, e2)), "dequantize edges")


@pytest.mark.parametrize("kind", VL.FIXTURES)
def test_verify_lane_gemm_int15_through_the_surface(kind):
    from mojolearn_amd import linalg
    X = VL.fixture_x(kind)
    lane = VL.lane_gemm_int15(linalg.quantize_int15, linalg.matmul_int15, linalg.dequantize_int15,
                              linalg.INT15_MAX_K, X)
    assert VL.train_hash(lane) == VL.golden()["cells"][f"gemm-int15/{kind}"]["train"]


def test_surface_int15_forms_and_refusals(oracle):
    from mojolearn_amd import linalg
    rng = np.random.default_rng(22)
    a = rng.standard_normal((45, 1000)).astype(np.float32)
    b = rng.standard_normal((70, 1000)).astype(np.float32)
    pa = oracle.q15_quantize(a)
    pb = oracle.q15_quantize(b)
    want = oracle.nan_canon(oracle.q15_gemm(*pa, *pb))
    _bits_equal(linalg.matmul_int15(a, b), want, "f32 operands")
    out = np.full((45, 70), 3.0, np.float32)
    assert linalg.matmul_int15(tuple(pa), tuple(pb), out=out) is out
    _bits_equal(out, want, "planes into out")
    with pytest.raises(TypeError, match="is a tuple of 2"):
        linalg.matmul_int15(pa[:2], b)
    with pytest.raises(ValueError, match="k=65537 is above 65536"):
        linalg.matmul_int15(np.zeros((1, 65537), np.float32), np.zeros((1, 65537), np.float32))


def test_from_f16_all_patterns(oracle):
    """Every float16 pattern through the device entry and the surface: exact, NaN payloads kept."""
    from mojolearn_amd import linalg
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = oracle.f16_widen(bits).view(np.uint32)
    got = _dev().f16_widen(torch.from_numpy(bits.view(np.int16)).to(DEV)).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, want)
    got2 = linalg.from_f16(bits.reshape(256, 256)).view(np.uint32).ravel()
    assert np.array_equal(got2, want)
    got3 = linalg.from_f16(bits.view(np.float16)).view(np.uint32)
    assert np.array_equal(got3, want)
