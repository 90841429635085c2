"""Profile mojolearn.identical.gemm.int8i32.v1 on gfx950 (integer MFMA product, quantizer,
dequantizer) against the CPU oracle, bit for bit (gemm/IDENTICAL_LOWBIT_CONTRACT.md L-3..L-7;
the reference's identical_gemm_int8_into / quantize_rows_int8_device / dequantize_rows_int8_device,
gemm/linalg_native.mojo:258-393).  Covers ragged m/n, k not a multiple of the 16-byte row
chunk or of the 128-code slice, misaligned operand bases (the repack path), exponent sums past
both ends of the float32 range, k at the contract's maximum, and the surface's gemm-int8 verify
cells on all nine fixtures."""
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


# (1, 4096, 4096), (8, 300, 14336), (3, 1000, 1000), (33, 47, 131072) and (16, 129, 385) split k;
# m <= 4 with k a multiple of 16 and aligned rows takes the streaming kernel (the extreme codes of row 0
# reach -127 * 127 * 131072 at k = 131072); m = 5..9 take the tiles with a partial tile of rows.
SHAPES = [(1, 1, 1), (3, 5, 7), (1, 300, 16), (130, 129, 16), (128, 128, 128), (129, 257, 129),
          (200, 300, 4097), (64, 1000, 520), (300, 64, 2048), (33, 47, 131072), (512, 512, 512),
          (1, 4096, 4096), (8, 300, 14336), (3, 1000, 1000), (16, 129, 385), (2, 77, 1024), (3, 333, 2064),
          (4, 14336, 4096), (4, 1, 131072), (1, 129, 4112), (1, 5, 131072), (7, 64, 2048),
          (8, 4096, 4096), (5, 333, 4112), (6, 1, 131072), (8, 7, 16), (9, 70, 2048)]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
def test_gemm_int8i32_vs_oracle(oracle, shape):
    m, n, k = shape
    print(f"int8i32 gemm {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m * 7 + n * 11 + k)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qb = rng.integers(-127, 128, (n, k)).astype(np.int8)
    if k > 1:
        qa[0, :] = 127
        qb[0, :] = -127
    ea = rng.integers(-40, 40, m).astype(np.int32)
    eb = rng.integers(-40, 40, n).astype(np.int32)
    c = _dev().gemm_int8i32(_t(qa), _t(ea), _t(qb), _t(eb))
    torch.cuda.synchronize()
    _bits_equal(c.cpu().numpy(), oracle.nan_canon(oracle.q8_gemm(qa, ea, qb, eb)), "int8i32")


def test_gemm_int8i32_exponent_edges(oracle):
    """Exponent sums above 127 (infinite scale: +-inf, and NaN for a zero sum), below -126
    (+-0), and products that land in the subnormal range (flushed)."""
    rng = np.random.default_rng(9)
    m, n, k = 70, 90, 300
    qa = rng.integers(-3, 4, (m, k)).astype(np.int8)
    qb = rng.integers(-3, 4, (n, k)).astype(np.int8)
    qa[1] = 0
    ea = rng.integers(-140, 140, m).astype(np.int32)
    eb = rng.integers(-140, 140, n).astype(np.int32)
    c = _dev().gemm_int8i32(_t(qa), _t(ea), _t(qb), _t(eb))
    torch.cuda.synchronize()
    _bits_equal(c.cpu().numpy(), oracle.nan_canon(oracle.q8_gemm(qa, ea, qb, eb)), "edges")


@pytest.mark.parametrize("offset", [1, 4, 8])
def test_gemm_int8i32_misaligned_base(oracle, offset):
    """Operand bases off the 16-byte grid take the repack path."""
    rng = np.random.default_rng(offset)
    m, n, k = 150, 77, 160
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qb = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ea = np.zeros(m, np.int32)
    eb = np.full(n, -3, np.int32)
    ba = torch.zeros(m * k + 64, dtype=torch.int8, device=DEV)
    bb = torch.zeros(n * k + 64, dtype=torch.int8, device=DEV)
    ta = ba[offset:offset + m * k].view(m, k)
    tb = bb[offset:offset + n * k].view(n, k)
    ta.copy_(_t(qa))
    tb.copy_(_t(qb))
    c = _dev().gemm_int8i32(ta, _t(ea), tb, _t(eb))
    torch.cuda.synchronize()
    _bits_equal(c.cpu().numpy(), oracle.nan_canon(oracle.q8_gemm(qa, ea, qb, eb)), "misaligned")


def _quant_rows(rng, rows, cols):
    x = (rng.standard_normal((rows, cols)) * np.exp2(rng.uniform(-30, 30, (rows, 1)))).astype(np.float32)
    if rows >= 8:
        x[0] = 0.0
        x[1, ::3] = np.nan
        x[2, 0] = np.inf
        x[3] = (x[3] * np.float32(1e-38)).astype(np.float32)           # subnormal row: flushed to zero
        x[4] = np.float32(2.0 ** -124) * np.sign(x[4]).astype(np.float32)  # absmax below 2^-121
        x[5, 0] = -0.0
        x[6] = np.ldexp(np.round(rng.standard_normal(cols) * 64) + 0.5, -8).astype(np.float32)  # ties
    return x


@pytest.mark.parametrize("shape", [(1, 1), (8, 5), (33, 300), (9, 5000), (300, 4096)])
def test_quantize_dequantize_vs_oracle(oracle, shape):
    rows, cols = shape
    print(f"int8 quantize {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows + cols)
    x = _quant_rows(rng, rows, cols)
    D = _dev()
    codes, exps = D.int8_quantize(_t(x))
    torch.cuda.synchronize()
    wc, we = oracle.q8_quantize(x)
    assert np.array_equal(codes.cpu().numpy(), wc)
    assert np.array_equal(exps.cpu().numpy(), we)
    y = D.int8_dequantize(codes, exps)
    torch.cuda.synchronize()
    _bits_equal(y.cpu().numpy(), oracle.nan_canon(oracle.q8_dequantize(wc, we)), "dequantize")
    e2 = rng.integers(-150, 150, rows).astype(np.int32)  # scales past both ends of the range
    y2 = D.int8_dequantize(codes, _t(e2))
    torch.cuda.synchronize()
    _bits_equal(y2.cpu().numpy(), oracle.nan_canon(oracle.q8_dequantize(wc, e2)), "dequantize edges")


@pytest.mark.parametrize("kind", VL.FIXTURES)
def test_verify_lane_gemm_int8_through_the_surface(kind):
    from mojolearn_amd import linalg
    X = VL.fixture_x(kind)
    lane = VL.lane_gemm_int8(linalg.quantize_int8, linalg.matmul_int8, linalg.dequantize_int8, X)
    assert VL.train_hash(lane) == VL.golden()["cells"][f"gemm-int8/{kind}"]["train"]


def test_surface_matmul_int8_forms(oracle):
    """float32 operands are quantized by the profile's rule; (codes, exponents) pairs are used
    as given; both spellings give the same bits; `out` is written in place."""
    from mojolearn_amd import linalg
    rng = np.random.default_rng(12)
    a = rng.standard_normal((45, 1000)).astype(np.float32)
    b = rng.standard_normal((70, 1000)).astype(np.float32)
    qa, ea = oracle.q8_quantize(a)
    qb, eb = oracle.q8_quantize(b)
    want = oracle.nan_canon(oracle.q8_gemm(qa, ea, qb, eb))
    _bits_equal(linalg.matmul_int8(a, b), want, "f32 operands")
    _bits_equal(linalg.matmul_int8((qa, ea), b), want, "pair and f32")
    out = np.full((45, 70), 5.0, np.float32)
    r = linalg.matmul_int8((qa, ea), (qb, eb), out=out)
    assert r is out
    _bits_equal(out, want, "pairs into out")
    with pytest.raises(ValueError, match="contracted extents differ"):
        linalg.matmul_int8(a, b[:, :999])
    with pytest.raises(ValueError, match=r"a exponents has shape \(44,\), want \(45,\)"):
        linalg.matmul_int8((qa, ea[:44]), b)


@pytest.mark.parametrize("shape", [(1, 4096, 4096), (200, 300, 4097), (8, 300, 1000), (8, 300, 1024)])
def test_gemm_int8i32_ws_in_graph(oracle, shape):
    """The caller-workspace entry (split-k partials, repack) captured in a HIP graph and
    replayed three times, eager work between replays; every replay bit-identical."""
    from mojolearn_amd import _native
    m, n, k = shape
    rng = np.random.default_rng(k)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qb = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ea = rng.integers(-30, 30, m).astype(np.int32)
    eb = rng.integers(-30, 30, n).astype(np.int32)
    want = oracle.nan_canon(oracle.q8_gemm(qa, ea, qb, eb))
    L = _native.lib()
    ta, tb, tea, teb = _t(qa), _t(qb), _t(ea), _t(eb)
    nb = L.mlg_gemm_int8i32_workspace_bytes(ta.data_ptr(), tb.data_ptr(), m, n, k)
    assert nb >= 0
    ws = torch.empty(max(nb, 4), dtype=torch.uint8, device=DEV)
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    s = torch.cuda.Stream()

    def call():
        _native.check(L.mlg_gemm_int8i32_ws(out.data_ptr(), ta.data_ptr(), tea.data_ptr(), tb.data_ptr(),
                                            teb.data_ptr(), m, n, k, ws.data_ptr(), nb, s.cuda_stream))

    with torch.cuda.stream(s):
        call()
    torch.cuda.synchronize()
    _bits_equal(out.cpu().numpy(), want, "eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call()
    for r in range(3):
        out.fill_(-1.0)
        ws.fill_(0x5A)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _bits_equal(out.cpu().numpy(), want, f"replay {r}")
