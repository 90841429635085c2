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
