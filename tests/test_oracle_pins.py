"""Pins of the oracle's seam functions by independent spellings (no GPU).

* `bias` (transformer/impl/llama/modeling_llama.mojo:3979-3989, `add_bias_kernel`: one add per
  cell after the product, ftz(ftz(y) + ftz(b[col]))) against numpy's IEEE float32 add with the
  flush spelled on the integer word, over a million random words (every class: normals,
  subnormals, both zeros, both infinities, NaNs) plus planted cells; and against the oracle's
  other spelling of the same seam, the PLUS_BIAS follower (gemm/checks/gemm_identical.mojo
  :8891-8895).
* `int8_dequant` (this build's per-output-column scale: checks/numerics.mojo:1665-1671 with the
  power of two replaced by an fp32 scale, ftz(f32(code) * ftz(scale[j])), one RNE multiply)
  against numpy's float32 multiply, whole random matrices in both stored layouts (k x n for
  OP_NN/OP_TN, n x k for OP_NT), every int8 code, scales from the workload's range and from
  every word class (subnormal scales flush to a signed zero, tiny ones underflow the product
  into the flush, huge ones overflow it, zeros and infinities make the 0 x inf NaN).
* `host_rows`, the restatement of the reference's fast CPU column
  (gemm/host/gemm_host_rows.mojo): the host card's recorded hashes (20 shapes) and orc_gemm's
  bits on shapes that take both of its paths, every orientation, with accumulators planted to
  pass through subnormals (the deferred flush's redo) and with the redo forced.
"""
import numpy as np
import pytest

import cards

U32, F32 = np.uint32, np.float32


def _ftz(x):
    """The flush on the integer word: exponent field 0 keeps only the sign bit."""
    w = np.ascontiguousarray(x, dtype=F32).view(U32)
    return np.where((w & 0x7F800000) == 0, w & 0x80000000, w).astype(U32).view(F32)


def _canon_words(x):
    w = np.ascontiguousarray(x, dtype=F32).view(U32).copy()
    w[(w & 0x7FFFFFFF) > 0x7F800000] = 0x7FC00000
    return w


def _random_words(rng, shape):
    """Float32 words of every class: uniform random bit patterns (about 0.4 % NaN/inf words and
    0.4 % subnormals), normal magnitudes, subnormals, and the special words."""
    w = rng.integers(0, 1 << 32, size=shape, dtype=np.uint64).astype(U32)
    z = rng.random(shape)
    normal = (rng.standard_normal(shape) * np.exp2(rng.uniform(-20, 20, shape))).astype(F32).view(U32)
    w = np.where(z < 0.5, normal, w)
    sub = rng.integers(1, 0x800000, size=shape).astype(U32) | (rng.integers(0, 2, size=shape).astype(U32) << 31)
    w = np.where((z >= 0.5) & (z < 0.6), sub, w)
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x00800000,
                         0x80800000, 0x007FFFFF, 0x807FFFFF, 0x7F7FFFFF, 0xFF7FFFFF], U32)
    pick = rng.integers(0, specials.size, size=shape)
    w = np.where((z >= 0.6) & (z < 0.66), specials[pick], w)
    return w.view(F32)


def test_bias_against_numpy_words(oracle):
    rng = np.random.default_rng(2026)
    m, n = 1000, 1000
    y = _random_words(rng, (m, n))
    b = _random_words(rng, (n,))
    got = oracle.bias(y, b)
    with np.errstate(invalid="ignore", over="ignore"):
        want = _ftz((_ftz(y) + _ftz(b)[None, :]).astype(F32))
    assert np.array_equal(_canon_words(got), _canon_words(want))
    # NaN exactly where IEEE says (inf - inf, NaN operands), nowhere else
    assert np.array_equal(np.isnan(got), np.isnan(want))
    # the oracle's other spelling of the same seam: the PLUS_BIAS follower
    epi = oracle.epilogue(np.array(y, copy=True), n, m, n, oracle.EPI_PLUS_BIAS, b)
    assert np.array_equal(_canon_words(got), _canon_words(epi))


def test_bias_planted_cells(oracle):
    """Cells whose answer a plausible mistake moves: a subnormal output, subnormal operands,
    signed zeros, inf - inf."""
    f = lambda w: np.array([w], U32).view(F32)[0]  # noqa: E731
    y = np.array([[f(0x00C00000), f(0x00400000), -0.0, 0.0, np.inf, 1.0, 0.0, f(0x007FFFFF)]], F32)
    b = np.array([-f(0x00800000), 1.0, -0.0, -0.0, -np.inf, f(0x80000001), f(0x80000001), f(0x00000001)], F32)
    got = _canon_words(oracle.bias(y, b)).ravel()
    # 1.5*2^-126 - 2^-126 = 2^-127 (subnormal) -> +0; subnormal y flushes: +0 + 1 = 1;
    # -0 + -0 = -0; +0 + -0 = +0; inf - inf = NaN; subnormal bias flushes: 1 + -0 = 1;
    # +0 + flushed -2^-149 = +0 (unflushed: -0); both flushed: +0 (unflushed: 2^-126)
    assert [int(w) for w in got] == [0x00000000, 0x3F800000, 0x80000000, 0x00000000, 0x7FC00000, 0x3F800000,
                                     0x00000000, 0x00000000]


@pytest.mark.parametrize("op", [0, 1])
def test_int8_dequant_against_numpy(oracle, op):
    rng = np.random.default_rng(700 + op)
    k, n = 512, 768
    codes = rng.integers(-128, 128, (k, n) if op == 0 else (n, k), dtype=np.int8)
    codes.flat[:256] = np.arange(-128, 128, dtype=np.int8)  # every code
    f = lambda w: np.array(w, U32).view(F32)  # noqa: E731
    scales = rng.uniform(1e-3, 1e-2, n).astype(F32)
    scales[:64] = _random_words(rng, (64,))  # every word class
    scales[64:80] = f(rng.integers(1, 0x800000, 16).astype(U32))  # subnormal scales
    scales[80:96] = f((rng.integers(1, 8, 16).astype(U32) << 23) | rng.integers(0, 0x800000, 16).astype(U32))
    scales[96:112] = f((rng.integers(248, 255, 16).astype(U32) << 23) | rng.integers(0, 0x800000, 16).astype(U32))
    scales[112:116] = np.array([0.0, -0.0, np.inf, -np.inf], F32)
    got = oracle.int8_dequant(codes, scales, op)
    sc = _ftz(scales)
    with np.errstate(invalid="ignore", over="ignore"):
        prod = codes.astype(F32) * (sc[None, :] if op == 0 else sc[:, None])
    want = _ftz(prod.astype(F32))
    assert np.array_equal(_canon_words(got), _canon_words(want))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    # the cases that pin the flushes: a subnormal scale gives a signed zero, a tiny one a flushed
    # product, a zero code times inf a NaN
    col = (lambda j: got[:, j]) if op == 0 else (lambda j: got[j, :])
    assert np.all((col(64).view(U32) & 0x7FFFFFFF) == 0)
    assert np.isnan(col(114)[(codes[:, 114] if op == 0 else codes[114, :]) == 0]).all()


def test_int8_dequant_layouts_agree(oracle):
    """The OP_NT layout is the transpose of the OP_NN one, word for word."""
    rng = np.random.default_rng(5)
    codes = rng.integers(-127, 128, (300, 200), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, 200).astype(F32)
    nn = oracle.int8_dequant(codes, scales, 0)
    nt = oracle.int8_dequant(np.ascontiguousarray(codes.T), scales, 1)
    assert np.array_equal(nn.view(U32), np.ascontiguousarray(nt.T).view(U32))


@pytest.mark.parametrize("i", range(len(cards.SHAPES)), ids=[s[0] for s in cards.SHAPES])
def test_host_rows_card(oracle, i):
    """The restated fast column reproduces the reference's host card hashes."""
    name, m0, n0, k, op = cards.SHAPES[i]
    m, n = cards.host_capped(m0, n0, k)
    sa, sb = cards.operand_shapes(m, n, k, op)
    a, b = oracle.card_fill(m * k, 11 + i).reshape(sa), oracle.card_fill(n * k, 22 + i).reshape(sb)
    c = oracle.host_rows(a, b, op)
    assert (c.size, oracle.fnv1a64(c)) == cards.parse_card("host_oracle.card")[name + ".out"]


def _planted_subnormal(rng, m, n, k, op):
    """Operands whose accumulators pass through subnormals: in the first half of the rows every
    product lies near 2^-128 (flushed at every step the chain stays a zero; left unflushed it
    sums to a normal number), in the other half such products meet normal ones."""
    A = (rng.standard_normal((m, k)) * np.float32(2.0 ** -70)).astype(F32)
    B = (rng.standard_normal((k, n)) * np.float32(2.0 ** -58)).astype(F32)
    A[m // 2:, 3::7] = rng.standard_normal((m - m // 2, A[:, 3::7].shape[1])).astype(F32) * np.float32(2.0 ** -60)
    a = A if op != 2 else np.ascontiguousarray(A.T)
    b = B if op != 1 else np.ascontiguousarray(B.T)
    return a, b


SHAPES = [(1, 40, 300), (3, 33, 1000), (4, 70, 129), (5, 70, 300), (40, 100, 1000), (64, 96, 4097),
          (9, 31, 129), (70, 65, 128)]


@pytest.mark.parametrize("op", [0, 1, 2])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
def test_host_rows_equals_oracle(oracle, shape, op):
    m, n, k = shape
    rng = np.random.default_rng(m * 31 + n + k + op)
    a, b = _planted_subnormal(rng, m, n, k, op)
    want = _canon_words(oracle.gemm(a, b, op))
    assert np.array_equal(_canon_words(oracle.host_rows(a, b, op)), want)
    assert np.array_equal(_canon_words(oracle.host_rows(a, b, op, force_redo=True)), want)
    # wide exponents with inf/NaN words
    sa, sb = a.shape, b.shape
    a = (rng.standard_normal(sa) * np.exp2(rng.uniform(-140, 60, sa))).astype(F32)
    b = (rng.standard_normal(sb) * np.exp2(rng.uniform(-140, 60, sb))).astype(F32)
    b.flat[::97] = np.inf
    a.flat[::89] = np.nan
    assert np.array_equal(_canon_words(oracle.host_rows(a, b, op)), _canon_words(oracle.gemm(a, b, op)))

