"""Closed forms, invariants and brute force pinning the CPU oracle (no GPU)."""
import numpy as np
import pytest

import kat


def _leaf_rule(k):
    """gemm/contract.mojo:173-214, written from IDENTICAL_FP32_CONTRACT.md section 6."""
    if k <= 0:
        return 1, 0
    if k <= 128:
        return k, 1
    if -(-k // 128) <= 1024:
        return 128, -(-k // 128)
    L = -(-k // 1024)
    return L, -(-k // L)


@pytest.mark.parametrize("k,L,P", [
    (0, 1, 0), (1, 1, 1), (64, 64, 1), (128, 128, 1), (129, 128, 2), (256, 128, 2), (300, 128, 3),
    (517, 128, 5), (1024, 128, 8), (2048, 128, 16), (4096, 128, 32), (4097, 128, 33), (14336, 128, 112),
    (100003, 128, 782), (131072, 128, 1024), (131073, 129, 1017), (1_000_000, 977, 1024),
    (4_000_000, 3907, 1024)])
def test_partition_table(oracle, k, L, P):
    assert _leaf_rule(k) == (L, P)
    assert oracle.leaf_size(k) == L
    assert oracle.leaf_count(k, L) == P


def _count_tree(P):
    """(arithmetic nodes, carries per level) of the contract tree over P leaves."""
    arith, carries, w = 0, [], P
    while w > 1:
        arith += w // 2
        carries.append(w % 2)
        w = w // 2 + w % 2
    return arith, carries


@pytest.mark.parametrize("P", [1, 2, 3, 5, 7, 8, 112, 782, 1024])
def test_tree_shape_invariants(P):
    arith, carries = _count_tree(P)
    assert arith == P - 1                      # exactly P-1 arithmetic nodes
    assert all(c <= 1 for c in carries)        # at most one carry per level
    if P == 5:
        assert sum(carries) == 2
    if P == 7:
        assert sum(carries) == 1


def test_fold_stack_equals_tree(oracle):
    """The register-stack fold (device kernels, fast arm) is the contract's tree, P = 1..2100,
    on partials whose additions do not associate."""
    rng = np.random.default_rng(7)
    for P in range(1, 2101):
        parts = (rng.standard_normal(P) * np.exp2(rng.integers(-30, 30, P))).astype(np.float32)
        t = oracle.fold_tree(parts)
        s = oracle.fold_stack(parts)
        assert t.view(np.uint32) == s.view(np.uint32), P


def test_fold_tree_is_not_stride_or_serial(oracle):
    parts = np.array([2 ** 24, 1, 0, -2 ** 24], np.float32)
    assert oracle.fold_tree(parts).view(np.uint32) == 0            # adjacent: +0.0
    parts = np.array([2 ** 24] + [1] * 7, np.float32)
    assert oracle.fold_tree(parts) == np.float32(2 ** 24 + 6)      # serial would give 2^24


@pytest.mark.parametrize("fx", kat.fixtures(), ids=[f[0] for f in kat.fixtures()])
def test_kat(oracle, fx):
    name, a, b, leaf, want = fx
    c = oracle.nan_canon(oracle.gemm(a.reshape(1, -1), b.reshape(1, -1), oracle.OP_NT, leaf))
    assert c.view(np.uint32)[0, 0] == want, (name, hex(int(c.view(np.uint32)[0, 0])), hex(int(want)))


@pytest.mark.parametrize("op", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 7), (17, 33, 129), (5, 7, 1000), (9, 4, 4097)])
def test_integer_products_are_exact(oracle, op, m, n, k):
    """Small-integer operands keep every step exact, so fp32.v1 equals the integer product."""
    rng = np.random.default_rng(m * 1000 + n * 10 + k + op)
    A = rng.integers(-15, 16, (m, k)).astype(np.float32)
    B = rng.integers(-15, 16, (k, n)).astype(np.float32)
    want = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    a = A if op != 2 else np.ascontiguousarray(A.T)
    b = B if op != 1 else np.ascontiguousarray(B.T)
    for fn in (oracle.gemm, oracle.gemm_fast):
        got = fn(a, b, op)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", range(6))
def test_exact_rational_restatement(oracle, seed):
    """An independent restatement on Fractions (exact fma, explicit RNE to binary32) agrees
    bit for bit on tiny shapes with wide exponents, subnormals and signed zeros."""
    rng = np.random.default_rng(100 + seed)
    m, n, k = 2, 3, [5, 130, 300, 129, 257, 64][seed]
    A = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-70, 20, (m, k)))).astype(np.float32)
    B = (rng.standard_normal((k, n)) * np.exp2(rng.integers(-70, 20, (k, n)))).astype(np.float32)
    A[0, ::7] = np.float32(-0.0)
    B[::5, 1] = (B[::5, 1] * np.float32(1e-38)).astype(np.float32)  # some subnormals
    got = oracle.gemm(A, B, 0)
    for i in range(m):
        for j in range(n):
            want = kat.exact_cell(A[i], B[:, j], k)
            assert got[i, j].view(np.uint32) == np.float32(want).view(np.uint32), (i, j)


def test_bf16_narrow_rules(oracle):
    """L-2: ftz first (every bf16 subnormal narrows to a signed zero: all 254 of them), RNE,
    NaN stays quiet with its sign, overflow rounds to infinity."""
    sub_bits = np.concatenate([np.arange(1, 128), np.arange(0x8001, 0x8080)]).astype(np.uint32) << 16
    sub = sub_bits.view(np.float32)
    assert sub.size == 254
    out = oracle.bf16_narrow(sub)
    assert np.all((out & 0x7FFF) == 0) and np.array_equal(out >> 15, (sub_bits >> 31).astype(np.uint16))
    x = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, np.inf, -np.inf, 3.4e38], np.float32)
    assert list(oracle.bf16_narrow(x)) == [0x3F80, 0x3F82, 0x7F80, 0xFF80, 0x7F80]
    nan = np.array([0xFF800001], np.uint32).view(np.float32)
    assert oracle.bf16_narrow(nan)[0] == 0xFFC0
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(oracle.bf16_widen(bits).view(np.uint32), bits.astype(np.uint32) << 16)


def test_int8_dequant_rule(oracle):
    codes = np.array([[127, -127], [0, -1]], np.int8)
    scales = np.array([np.float32(1e-3), np.array([0x00400000], np.uint32).view(np.float32)[0]], np.float32)
    w = oracle.int8_dequant(codes, scales, 0)
    assert w[0, 0] == np.float32(np.float32(127.0) * np.float32(1e-3))
    assert w[0, 1].view(np.uint32) == 0x80000000  # subnormal scale flushed: -127 * +0 = -0
    assert w[1, 0].view(np.uint32) == 0


def test_nan_canon(oracle):
    w = np.array([0x7F800001, 0xFFC00000, 0x7FFFFFFF, 0x7F800000, 0xFF800000, 0x00000001, 0x80000000],
                 np.uint32)
    got = oracle.nan_canon(w.view(np.float32)).view(np.uint32)
    assert list(got) == [0x7FC00000, 0x7FC00000, 0x7FC00000, 0x7F800000, 0xFF800000, 0x00000001, 0x80000000]


# ---- int8i32.v1 (gemm/IDENTICAL_LOWBIT_CONTRACT.md L-3..L-7), pinned by independent arithmetic:
# exact rationals, numpy's own int->float rounding and ldexp, not the oracle's spelling.

def _ftz32(v):
    v = np.asarray(v, np.float32).copy()
    u = v.view(np.uint32)
    sub = ((u & 0x7F800000) == 0) & ((u & 0x007FFFFF) != 0)
    u[sub] &= 0x80000000
    return v


def test_int8_i32_to_f32_is_round_half_even(oracle):
    """L-5: the split conversion equals one round-to-nearest-even of the integer, which is
    numpy's int64 -> float32 cast; ties at 2^24..2^31 included."""
    rng = np.random.default_rng(5)
    vals = list(rng.integers(-(2 ** 31) + 1, 2 ** 31, 4000))
    for p in range(23, 31):
        for d in (-3, -2, -1, 0, 1, 2, 3):
            vals += [2 ** p + d, -(2 ** p) - d, 2 ** p + 2 ** (p - 23) + d]
    vals += [0, 1, -1, 2 ** 31 - 1, -(2 ** 31) + 1, 16129 * 131072, -16129 * 131072]
    for v in vals:
        want = np.array([v], np.int64).astype(np.float32)[0]
        got = np.float32(oracle.q8_i32_to_f32(int(v)))
        assert got.view(np.uint32) == want.view(np.uint32), v


def test_int8_row_exponent(oracle):
    """L-3: floor(log2 absmax) - 6, by frexp; a zero, subnormal or NaN absmax gives 0."""
    rng = np.random.default_rng(6)
    xs = np.concatenate([np.exp2(np.arange(-126, 128)).astype(np.float32),
                         (rng.uniform(0.5, 1.0, 500) * np.exp2(rng.integers(-125, 128, 500))).astype(np.float32)])
    xs = np.concatenate([xs, np.nextafter(xs, np.float32(0))])
    for x in xs:
        if x < np.finfo(np.float32).tiny:
            continue
        _, e2 = np.frexp(np.float64(x))
        assert oracle.q8_row_exponent(x) == int(e2) - 1 - 6, x
    sub = np.array([0x00000001, 0x007FFFFF], np.uint32).view(np.float32)
    for x in [np.float32(0.0), sub[0], sub[1], np.float32(np.nan)]:
        assert oracle.q8_row_exponent(x) == 0
    assert oracle.q8_row_exponent(np.float32(np.inf)) == 255 - 127 - 6


def test_int8_quantize_rule(oracle):
    """L-4: codes = clamp(round_half_even(x * 2^-e), -127, 127) by exact rationals, with rows
    built to hold exact ties, the 127.5 -> 128 -> 127 clamp, subnormals and a zero row."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    rows = []
    for r in range(40):
        scale = 2.0 ** int(rng.integers(-110, 110))
        halves = rng.integers(-255, 256, 64).astype(np.float64) / 2.0  # ties at every .5
        row = halves * scale / 2 ** 6
        row[0] = 127.75 * scale / 2 ** 6 * (1 if r % 2 else -1)  # absmax in [64, 128) after scaling
        rows.append(row)
    rows.append(rng.standard_normal(64) * 3.0)
    x = np.array(rows, np.float32)
    x[-1, 5] = np.array([0x00000005], np.uint32).view(np.float32)[0]  # flushed to zero
    x = np.concatenate([x, np.zeros((1, 64), np.float32)])
    codes, exps = oracle.q8_quantize(x)
    fx = _ftz32(x)
    for i in range(x.shape[0]):
        absmax = np.max(np.abs(fx[i].astype(np.float64)))
        e = 0 if absmax == 0 else int(np.frexp(absmax)[1]) - 1 - 6
        assert exps[i] == e
        for j in range(x.shape[1]):
            s = Fraction(float(fx[i, j])) * (Fraction(2) ** -e)
            q = max(-127, min(127, round(s)))  # Fraction.__round__ is half-to-even
            assert codes[i, j] == q, (i, j, float(x[i, j]), e)
    assert (codes[-1] == 0).all() and exps[-1] == 0


def test_int8_quantize_specials(oracle):
    """NaN codes to 0 and never wins the absmax; an infinity codes to +-127; a row whose
    absmax is below 2^-121 has an infinite 2^-e: nonzero entries clamp, zeros code to 0."""
    x = np.array([[np.nan, 1.0, -0.5, 0.25],
                  [np.inf, 1.0, -np.inf, 0.0],
                  [2.0 ** -124, -(2.0 ** -125), 0.0, -0.0]], np.float32)
    codes, exps = oracle.q8_quantize(x)
    assert list(exps) == [-6, 122, -130]
    assert list(codes[0]) == [0, 64, -32, 16]
    assert list(codes[1]) == [127, 0, -127, 0]
    assert list(codes[2]) == [127, -127, 0, 0]


def test_int8_dequantize_rule(oracle):
    """L-6: code * 2^e exactly (ldexp), flushed below the normal range; 2^e is infinite above
    127 (so a zero code gives NaN, canonical on the surface) and +0 below -126."""
    rng = np.random.default_rng(8)
    codes = rng.integers(-127, 128, (6, 50)).astype(np.int8)
    codes[:, 0] = 0
    exps = np.array([-140, -133, -20, 0, 100, 121], np.int32)
    got = oracle.q8_dequantize(codes, exps)
    want = _ftz32(np.ldexp(codes.astype(np.float64), exps[:, None].astype(np.int64)).astype(np.float32))
    want[0] = np.where(codes[0] < 0, np.float32(-0.0), np.float32(0.0))  # 2^-140 is +0, sign of code
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    big = oracle.nan_canon(oracle.q8_dequantize(np.array([[0, 3, -3]], np.int8), np.array([128], np.int32)))
    assert list(big.view(np.uint32).ravel()) == [0x7FC00000, 0x7F800000, 0xFF800000]


@pytest.mark.parametrize("m,n,k", [(3, 5, 1), (7, 4, 33), (5, 9, 300), (2, 3, 4097)])
def test_int8_gemm_exact(oracle, m, n, k):
    """L-7: the exact integer dot (numpy int64 matmul) rounded once to float32 and scaled by
    an exact power of two, flushed; exponent sums reach the overflow and underflow edges."""
    rng = np.random.default_rng(m * 1000 + k)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qb = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ea = rng.integers(-70, 70, m).astype(np.int32)
    eb = rng.integers(-70, 70, n).astype(np.int32)
    ea[0], eb[0] = -140, 10
    got = oracle.q8_gemm(qa, ea, qb, eb)
    acc = qa.astype(np.int64) @ qb.astype(np.int64).T
    f = acc.astype(np.float32).astype(np.float64)
    es = ea[:, None].astype(np.int64) + eb[None, :].astype(np.int64)
    want = _ftz32(np.where(es < -126, f * 0.0, np.ldexp(f, es)).astype(np.float32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_int8_gemm_at_max_k(oracle):
    """k = 131072 with every code at +-127: |sum| = 16129 * 2^17 < 2^31, no wrap, one rounding."""
    k = 131072
    qa = np.full((2, k), 127, np.int8)
    qa[1, ::2] = -127
    qb = np.full((2, k), 127, np.int8)
    e0 = np.zeros(2, np.int32)
    got = oracle.q8_gemm(qa, e0, qb, e0)
    full = np.array([16129 * k], np.int64).astype(np.float32)[0]
    assert got[0, 0] == full and got[0, 1] == full and got[1, 0] == 0.0


# ---- int15i64.v1 (contract section 6, W-1..W-7): numpy's own int64 -> float32 rounding, exact
# rationals and integer matmul, none sharing a step with the oracle's spelling.

def test_int15_i64_to_f32_is_round_half_even(oracle):
    """W-6 on the ties and edges the contract plants, random values below and above 2^48 (the
    sticky-bit branch), and the two ends of Int64."""
    rng = np.random.default_rng(15)
    vals = [0, 1, -1, 2 ** 24 + 1, 2 ** 24 + 3, -(2 ** 24 + 1), 2 ** 44, 2 ** 44 - 2 ** 31 + 2 ** 16,
            2 ** 63 - 1, -(2 ** 63)]
    for base in (2 ** 40 + 2 ** 16, 2 ** 40 + 3 * 2 ** 16, 2 ** 48, 2 ** 48 + 2 ** 24, 2 ** 48 + 3 * 2 ** 24):
        vals += [base - 1, base, base + 1, -base + 1, -base, -base - 1]
    for bits in (30, 44, 47, 48, 55, 62):
        vals += [int(v) for v in rng.integers(-(2 ** bits), 2 ** bits, 500, dtype=np.int64)]
    for v in vals:
        want = np.array([v], np.int64).astype(np.float32)[0]
        got = np.float32(oracle.q15_i64_to_f32(v))
        assert got.view(np.uint32) == want.view(np.uint32), v


def test_int15_pieces_cover_every_code(oracle):
    """W-3 on all 32767 codes: a row of the integers themselves has absmax 16383, so e = 0 and
    the codes are the values; hi is the floor quotient, lo the floor remainder."""
    c = np.arange(-16383, 16384, dtype=np.int64)
    hi, lo, e = oracle.q15_quantize(c.astype(np.float32).reshape(1, -1))
    assert e[0] == 0
    assert np.array_equal(hi[0].astype(np.int64), np.floor_divide(c, 128))
    assert np.array_equal(lo[0].astype(np.int64), np.mod(c, 128))
    assert lo.min() >= 0 and hi.min() == -128 and hi.max() == 127
    assert np.array_equal(hi[0].astype(np.int64) * 128 + lo[0], c)


def test_int15_quantize_rule(oracle):
    """W-1/W-2 by exact rationals: e = floor(log2 absmax) - 13, codes clamp(rne(x 2^-e), +-16383),
    with rows built to hold ties and the 16383.5 -> 16384 -> 16383 clamp."""
    from fractions import Fraction
    rng = np.random.default_rng(16)
    rows = []
    for r in range(30):
        scale = 2.0 ** int(rng.integers(-100, 100))
        row = rng.integers(-32767, 32768, 48).astype(np.float64) / 2.0 * scale / 2 ** 13
        row[0] = 16383.5 * scale / 2 ** 13 * (1 if r % 2 else -1)
        rows.append(row)
    x = np.array(rows, np.float32)
    hi, lo, exps = oracle.q15_quantize(x)
    codes = hi.astype(np.int64) * 128 + lo
    for i in range(x.shape[0]):
        absmax = np.max(np.abs(x[i].astype(np.float64)))
        e = int(np.frexp(absmax)[1]) - 1 - 13
        assert exps[i] == e
        for j in range(x.shape[1]):
            q = max(-16383, min(16383, round(Fraction(float(x[i, j])) * Fraction(2) ** -e)))
            assert codes[i, j] == q, (i, j)


def test_int15_quantize_specials(oracle):
    """A NaN codes to 0 before and after the scaling (a zero of a row whose 2^-e is infinite);
    an infinity codes to +-16383 and sets the row exponent from its field (128 - 13)."""
    x = np.array([[np.nan, 1.0, -0.5, 0.0],
                  [np.inf, 1.0, -np.inf, 0.0],
                  [2.0 ** -120, -(2.0 ** -121), 0.0, -0.0]], np.float32)
    hi, lo, exps = oracle.q15_quantize(x)
    codes = hi.astype(np.int64) * 128 + lo
    assert list(exps) == [-13, 115, -133]
    assert list(codes[0]) == [0, 8192, -4096, 0]
    assert list(codes[1]) == [16383, 0, -16383, 0]
    assert list(codes[2]) == [16383, -16383, 0, 0]


@pytest.mark.parametrize("m,n,k", [(3, 5, 1), (6, 4, 200), (4, 7, 4097)])
def test_int15_gemm_exact(oracle, m, n, k):
    """W-5..W-7: the exact integer dot product (numpy int64), rounded once to float32, scaled by
    an exact power of two and flushed; exponent sums past both ends."""
    rng = np.random.default_rng(m * 100 + k)
    qa = rng.integers(-16383, 16384, (m, k)).astype(np.int64)
    qb = rng.integers(-16383, 16384, (n, k)).astype(np.int64)
    ea = rng.integers(-60, 60, m).astype(np.int32)
    eb = rng.integers(-60, 60, n).astype(np.int32)
    ea[0], eb[0] = -140, 10
    planes = lambda q: ((q >> 7).astype(np.int8), (q & 127).astype(np.int8))
    ah, al = planes(qa)
    bh, bl = planes(qb)
    got = oracle.q15_gemm(ah, al, ea, bh, bl, eb)
    f = (qa @ qb.T).astype(np.float32).astype(np.float64)
    es = ea[:, None].astype(np.int64) + eb[None, :].astype(np.int64)
    want = _ftz32(np.where(es < -126, f * 0.0, np.ldexp(f, es)).astype(np.float32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_int15_gemm_at_max_k(oracle):
    """k = 65536 with the code -16383 on both operands (hi = -128): the sum 16383^2 * 2^16 is
    exact in Int64 and rounds once."""
    k = 65536
    ah = np.full((1, k), -128, np.int8)
    al = np.full((1, k), 1, np.int8)
    e0 = np.zeros(1, np.int32)
    got = oracle.q15_gemm(ah, al, e0, ah, al, e0)
    assert got[0, 0] == np.array([16383 * 16383 * k], np.int64).astype(np.float32)[0]


def test_f16_widen_all_patterns(oracle):
    """All 65536 float16 patterns: numbers and infinities equal numpy's exact float16 ->
    float32 conversion; every NaN keeps its sign and payload, quiet bit included as given."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_widen(bits).view(np.uint32)
    f16 = bits.view(np.float16)
    num = ~np.isnan(f16)
    assert np.array_equal(got[num], f16[num].astype(np.float32).view(np.uint32))
    b = bits[~num].astype(np.uint32)
    assert np.array_equal(got[~num], ((b & 0x8000) << 16) | 0x7F800000 | ((b & 0x03FF) << 13))
