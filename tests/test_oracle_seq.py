"""The oracle's sequence-executor word (`orc_seq_gemm`, sequence/ops.mojo:518-531) and the
product's followers (`orc_epilogue`, `orc_expf`, `orc_sigmoidf`, `orc_tanhf`; checks/numerics.mojo,
sequence/act_values.mojo), pinned by: the reference's planted special values
(checks/portable_nn_check.mojo:235-245, checks/portable_gelu_check.mojo:690-713), accuracy against
float64 (sigmoid within the reference's 4-ulp bound), an exact-rational restatement of the seeded
chain, the equality of the unseeded word with the one-leaf fp32.v1 word, and the followers' rules
on planted cells."""
import numpy as np
import pytest

import kat as K


def _u(x):
    return np.asarray(x, np.float32).view(np.uint32)


def _f(bits):
    return np.array([bits], np.uint32).view(np.float32)[0]


def _ulp(a, b):
    a = _u(a).astype(np.int64)
    b = _u(b).astype(np.int64)
    a = np.where(a >= 0x80000000, -(a & 0x7FFFFFFF), a)
    b = np.where(b >= 0x80000000, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def _flush64(x):
    x = np.asarray(x, np.float32)
    return np.where(np.abs(x) < np.float32(1.1754943508222875e-38), np.copysign(np.float32(0), x), x)


SIGMOID_PLANTED = [(0x7FC00000, None), (0x00000000, 0x3F000000), (0x80000000, 0x3F000000),
                   (0xFF800000, 0x00000000), (0x7F800000, 0x3F800000), (np.float32(-100.0), 0x00000000),
                   (np.float32(-89.0), 0x00000000), (np.float32(-88.0), 0x00000000),
                   (np.float32(17.0), 0x3F800000), (np.float32(100.0), 0x3F800000)]
TANH_PLANTED = [(0x00000000, 0x00000000), (0x80000000, 0x80000000), (0x7FC00000, None), (0xFFC00000, None),
                (0x7F800000, 0x3F800000), (0xFF800000, 0xBF800000), (0x00400000, 0x00000000),
                (0x80400000, 0x80000000), (0x00000001, 0x00000000), (0x80000001, 0x80000000),
                (0x007FFFFF, 0x00000000), (0x807FFFFF, 0x80000000)]


def _as_f32(x):
    return _f(x) if isinstance(x, int) else np.float32(x)


@pytest.mark.parametrize("x,want", SIGMOID_PLANTED)
def test_sigmoid_planted(oracle, x, want):
    y = np.float32(oracle.lib().orc_sigmoidf(_as_f32(x)))
    if want is None:
        assert np.isnan(y)
    else:
        assert int(_u(y)) == want


@pytest.mark.parametrize("x,want", TANH_PLANTED)
def test_tanh_planted(oracle, x, want):
    y = np.float32(oracle.lib().orc_tanhf(_as_f32(x)))
    if want is None:
        assert np.isnan(y)
    else:
        assert int(_u(y)) == want


def test_expf_sigmoid_tanh_accuracy(oracle):
    rng = np.random.default_rng(5)
    x = rng.uniform(-87.3, 88.7, 1 << 20).astype(np.float32)
    assert _ulp(oracle.fmap(x, 0), _flush64(np.exp(x.astype(np.float64)))).max() <= 1
    xs = (rng.standard_normal(1 << 20) * np.exp2(rng.uniform(-40, 7, 1 << 20))).astype(np.float32)
    for which, ref, bound in ((1, lambda v: 1.0 / (1.0 + np.exp(-v)), 4), (2, np.tanh, 2)):
        y = oracle.fmap(xs, which)
        r = _flush64(ref(xs.astype(np.float64)))
        d = _ulp(y, r)
        d[(r == 0) & (y == 0)] = 0
        assert d.max() <= bound, (which, int(d.max()), xs[d.argmax()])


def test_tanh_branches_and_expf_edges(oracle):
    # the polynomial / exp branch point, the saturation bound, expf's overflow and underflow guards
    for b in (0x3F200000 - 1, 0x3F200000, 0x3F200000 + 1, 0x42317218, 0x42317219):
        x = _f(b)
        y = np.float32(oracle.lib().orc_tanhf(x))
        assert abs(float(y) - np.tanh(float(x))) <= 2 * np.spacing(np.float32(abs(y)))
        assert int(_u(np.float32(oracle.lib().orc_tanhf(-x)))) == int(_u(y)) ^ 0x80000000
    assert np.isinf(oracle.lib().orc_expf(np.float32(88.8)))
    assert oracle.lib().orc_expf(np.float32(-87.4)) == 0.0
    assert oracle.lib().orc_expf(np.float32(0.0)) == 1.0


def _seq_exact(A, B, c0, accumulate):
    m, k = A.shape
    n = B.shape[1]
    out = np.empty((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            acc = K._ftz(c0[i, j]) if accumulate else np.float32(0.0)
            for p in range(k):
                acc = K._ftz(K._fma(K._ftz(A[i, p]), K._ftz(B[p, j]), acc))
            out[i, j] = K._ftz(acc)
    return out


@pytest.mark.parametrize("accumulate", [False, True])
def test_seq_gemm_exact_rational(oracle, accumulate):
    rng = np.random.default_rng(11 + accumulate)
    m, n, k = 3, 4, 37
    A = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-70, 20, (m, k)))).astype(np.float32)
    B = (rng.standard_normal((k, n)) * np.exp2(rng.integers(-70, 20, (k, n)))).astype(np.float32)
    c0 = (rng.standard_normal((m, n)) * 1e3).astype(np.float32)
    c0[0, 0] = _f(0x00000005)  # a subnormal seed flushes to +0
    c = c0.copy()
    oracle.seq_gemm(c.reshape(-1), A.reshape(-1), B.reshape(-1), m, n, k, k, 1, n, 1, n, accumulate)
    assert np.array_equal(_u(c), _u(_seq_exact(A, B, c0, accumulate)))


def test_seq_gemm_strides_and_unseeded_word(oracle):
    """Every stride form gives the same cells; unseeded it is the one-leaf word of fp32.v1."""
    rng = np.random.default_rng(12)
    m, n, k = 7, 9, 300
    A = rng.standard_normal((m, k)).astype(np.float32)
    B = rng.standard_normal((k, n)).astype(np.float32)
    want = oracle.gemm(A, B, 0, leaf=k)
    assert np.array_equal(_u(want), _u(oracle.gemm_serial(A, B)))
    forms = [(A, m, k, k, 1), (np.ascontiguousarray(A.T), k, m, 1, m)]
    bforms = [(B, n, 1), (np.ascontiguousarray(B.T), 1, k)]
    for a_buf, _, _, a_si, a_sp in forms:
        for b_buf, b_sp, b_sj in bforms:
            c = np.full((m, 12), 7.0, np.float32)
            oracle.seq_gemm(c.reshape(-1), a_buf.reshape(-1), b_buf.reshape(-1), m, n, k, a_si, a_sp, b_sp, b_sj,
                            12, False)
            assert np.array_equal(_u(c[:, :n]), _u(want))
            assert (c[:, n:] == 7.0).all()  # cells past n in a row are left alone


def test_epilogue_rules(oracle):
    c = np.array([[1.5, -2.0, _f(0x00000003), np.nan, 0.0, -0.0]], np.float32)
    bias = np.array([0.5, 2.0, 1.0, 1.0, _f(0x80000001), 0.0], np.float32)
    y = oracle.epilogue(c.copy(), 6, 1, 6, oracle.EPI_PLUS_BIAS, bias)
    assert np.array_equal(_u(y[0, :3]), _u([2.0, 0.0, 1.0])) and np.isnan(y[0, 3])
    assert int(_u(y[0, 4])) == 0 and int(_u(y[0, 5])) == 0  # -0 + +0 = +0; 0 + (-0) = +0
    relu = oracle.epilogue(c.copy(), 6, 1, 6, oracle.EPI_BIAS_ACT, bias, oracle.ACT_RELU)
    assert np.array_equal(_u(relu), _u([[2.0, 0.0, 1.0, 0.0, 0.0, 0.0]]))  # NaN is not > 0
    z = np.array([[0.25, 0.0, -0.0, 0.5, 0.9, 0.0]], np.float32)
    d = np.array([[4.0, 3.0, 2.0, 1.0, -1.0, np.nan]], np.float32)
    r = oracle.epilogue(d.copy(), 6, 1, 6, oracle.EPI_ACT_BWD, z, oracle.ACT_RELU)
    assert np.array_equal(_u(r[0, :5]), _u([4.0, 0.0, 0.0, 1.0, -1.0])) and int(_u(r[0, 5])) == 0
    lg = oracle.epilogue(d[:, :5].copy(), 5, 1, 5, oracle.EPI_ACT_BWD, z[:, :5], oracle.ACT_LOGISTIC)
    want = [np.float32(np.float32(dv * zv) * np.float32(1 - zv)) for dv, zv in zip(d[0, :5], z[0, :5])]
    assert np.array_equal(_u(lg[0]), _u(want))
    th = oracle.epilogue(d[:, :5].copy(), 5, 1, 5, oracle.EPI_ACT_BWD, z[:, :5], oracle.ACT_TANH)
    want = [np.float32(dv * np.float32(1 - np.float32(zv * zv))) for dv, zv in zip(d[0, :5], z[0, :5])]
    assert np.array_equal(_u(th[0]), _u(want))
    # identity and softmax codes leave the biased word; logistic/tanh are the maps above
    for code in (oracle.ACT_IDENTITY, oracle.ACT_SOFTMAX):
        y2 = oracle.epilogue(c[:, :3].copy(), 3, 1, 3, oracle.EPI_BIAS_ACT, bias[:3], code)
        assert np.array_equal(_u(y2), _u(y[:, :3]))
    s = oracle.epilogue(c[:, :3].copy(), 3, 1, 3, oracle.EPI_BIAS_ACT, bias[:3], oracle.ACT_LOGISTIC)
    assert np.array_equal(_u(s[0]), _u(oracle.fmap(y[0, :3], 1)))
