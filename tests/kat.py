"""Known-answer fixtures for fp32.v1, each built so that a plausible mistake gives a
different, predicted answer (restating gemm/checks/gemm_oracle_check.mojo F1-F8):

  F1  serial vs split-K           A = [2^24, 1 x k-1], B = 1      split 2^24 + L(P-1), serial 2^24
  F2  partition count             same fixture at L = 64 / 128 / 256
  F3  fused vs unfused            A = [1, a0], B = [-fl(a0 b0), b0]  -> the product's rounding error
  F4a accumulator flush           A = [1.5*2^-126, 2^-126], B = [1, -1] -> +0.0 (not 2^-127)
  F4b operand flush               A = [2^-127], B = [2^20]           -> +0.0 (not 2^-107)
  F5  balanced vs serial fold     partials [2^24, 1 x 7]             -> 2^24 + 6 (serial: 2^24)
  F6  signed zero survives        every leaf -0.0 (2^-126, -1.5*2^-126 at its end) -> -0.0
  F7  odd carry vs +0 padding     F6 at P = 3 and 5                  -> -0.0 (padding: +0.0)
  F8  adjacent vs stride pairing  partials [2^24, 1, +0, -2^24]      -> +0.0 (stride: +1.0)
  inf/NaN                         inf - inf -> NaN word 0x7FC00000; overflow -> +inf

Every fixture is one cell of OP_NT (A is 1 x k, B is 1 x k).
"""
import numpy as np

TWO24 = np.float32(16777216.0)


def f32(bits):
    return np.array([bits], dtype=np.uint32).view(np.float32)[0]


def _hash64(i, f):
    M = (1 << 64) - 1
    h = (i * 0x9E3779B97F4A7C15 + (f + 1) * 0xBF58476D1CE4E5B9) & M
    h ^= h >> 29
    h = (h * 0x94D049BB133111EB) & M
    return h ^ (h >> 32)


def spread_half(i, f):
    """A value in [1, 2) with a 12-bit mantissa (gemm_oracle_check.mojo:561-575)."""
    return np.float32(1.0) + np.float32(_hash64(i, f) & 0xFFF) / np.float32(4096.0)


def _minus_zero_leaves(k, leaf):
    a = np.zeros(k, np.float32)
    for t in range((k + leaf - 1) // leaf):
        e = min((t + 1) * leaf, k)
        a[e - 2] = f32(0x00800000)
        a[e - 1] = -f32(0x00C00000)
    return a


def fixtures():
    """[(name, a[k], b[k], leaf (0 = contract), expected uint32 word)]"""
    out = []
    k = 1024
    a = np.ones(k, np.float32)
    a[0] = TWO24
    b = np.ones(k, np.float32)
    out.append(("F1.split", a, b, 0, (TWO24 + np.float32(128 * 7)).view(np.uint32)))
    out.append(("F1.serial", a, b, k, TWO24.view(np.uint32)))
    out.append(("F2.L64", a, b, 64, (TWO24 + np.float32(64 * 15)).view(np.uint32)))
    out.append(("F2.L256", a, b, 256, (TWO24 + np.float32(256 * 3)).view(np.uint32)))
    n3 = 0
    for t in range(4096):
        a0, b0 = spread_half(t, 0xC0FFEE), spread_half(t, 0xBEEF01)
        q = np.float32(a0 * b0)
        err = float(a0) * float(b0) - float(q)  # exact in float64 (13-bit x 13-bit significands)
        if err == 0.0:
            continue
        e = np.float32(err)
        assert float(e) == err
        out.append((f"F3.{t}", np.array([1.0, a0], np.float32), np.array([-q, b0], np.float32), 0,
                    e.view(np.uint32)))
        n3 += 1
        if n3 == 32:
            break
    out.append(("F4a", np.array([f32(0x00C00000), f32(0x00800000)], np.float32), np.array([1, -1], np.float32), 0,
                np.uint32(0)))
    out.append(("F4b", np.array([f32(0x00400000)], np.float32), np.array([2.0 ** 20], np.float32), 0, np.uint32(0)))
    a = np.zeros(1024, np.float32)
    a[0] = TWO24
    for j in range(1, 8):
        a[128 * j] = 1.0
    out.append(("F5", a, np.ones(1024, np.float32), 0, (TWO24 + np.float32(6)).view(np.uint32)))
    for k in (128, 256, 384, 640, 1000):
        out.append((f"F6.k{k}", _minus_zero_leaves(k, 128 if k > 128 else k), np.ones(k, np.float32), 0,
                    np.uint32(0x80000000)))
    a = np.zeros(512, np.float32)
    a[0], a[128], a[384] = TWO24, 1.0, -TWO24
    out.append(("F8", a, np.ones(512, np.float32), 0, np.uint32(0)))
    inf = np.float32(np.inf)
    out.append(("inf-inf", np.array([inf, 1.0], np.float32), np.array([1.0, -inf], np.float32), 0,
                np.uint32(0x7FC00000)))
    big = np.float32(2.0 ** 127)
    out.append(("overflow", np.array([big, big], np.float32), np.array([2.0, 2.0], np.float32), 0,
                np.uint32(0x7F800000)))
    return out


# ---------------------------------------------------------------------------
# An independent restatement in exact rational arithmetic (tiny shapes only):
# fma(a, b, c) = RNE_float32(a*b + c) computed on Fractions, ftz on words.

from fractions import Fraction  # noqa: E402


def _rne_f32(x):
    """Round a Fraction to the nearest float32 (ties to even), gradual underflow, overflow to inf."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    # x in [2^e, 2^(e+1)); quantum 2^(e-23), but never below 2^-149
    qexp = max(e - 23, -149)
    scaled = x / (Fraction(2) ** qexp)
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = Fraction(n) * Fraction(2) ** qexp
    if v >= Fraction(2) ** 128 - Fraction(2) ** 103:  # rounds to infinity (>= max + half ulp)
        return np.float32(sign * np.inf)
    return np.float32(sign * float(v))


def _ftz(x):
    x = np.float32(x)
    w = x.view(np.uint32)
    if (w & 0x7F800000) == 0 and (w & 0x7FFFFF) != 0:
        return np.array([w & 0x80000000], np.uint32).view(np.float32)[0]
    return x


def _fma(a, b, c):
    """fma on finite float32 values: one rounding of the exact a*b + c."""
    prod = Fraction(float(a)) * Fraction(float(b))
    s = prod + Fraction(float(c))
    if s != 0:
        return _rne_f32(s)
    # an exact zero: -0 only when the product and c are both zeros of negative sign
    prod_neg_zero = prod == 0 and (np.signbit(a) != np.signbit(b))
    return np.float32(-0.0) if (prod_neg_zero and c == 0 and np.signbit(c)) else np.float32(0.0)


def _add(x, y):
    s = Fraction(float(x)) + Fraction(float(y))
    if s != 0:
        return _rne_f32(s)
    return np.float32(-0.0) if (x == 0 and y == 0 and np.signbit(x) and np.signbit(y)) else np.float32(0.0)


def exact_cell(arow, bcol, k, leaf=0):
    """One cell of fp32.v1 on Fractions: leaves, then the level-by-level tree."""
    if leaf <= 0:
        leaf = k if k <= 128 else (128 if (k + 127) // 128 <= 1024 else (k + 1023) // 1024)
    P = (k + leaf - 1) // leaf
    parts = []
    for t in range(P):
        acc = np.float32(0.0)
        for p in range(t * leaf, min((t + 1) * leaf, k)):
            acc = _ftz(_fma(_ftz(arow[p]), _ftz(bcol[p]), acc))
        parts.append(_ftz(acc))
    while len(parts) > 1:
        nxt = [_ftz(_add(_ftz(parts[2 * q]), _ftz(parts[2 * q + 1]))) for q in range(len(parts) // 2)]
        if len(parts) % 2:
            nxt.append(parts[-1])
        parts = nxt
    return _ftz(parts[0]) if parts else np.float32(0.0)
