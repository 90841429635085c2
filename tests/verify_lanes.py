"""The verify-table fixtures and gemm lanes, restated for the tests.

Fixtures: tools/identity_break.py:1393 (N, D = 20000, 16) and :1414-1485 (`fixture`,
`_hashed_uniform`).  Hashes: `_h` / `_train_hash` (:1355-1382).  Lanes: gemm-pinned
(:2984-2995), gemm-transposed (:5880-5890), gemm-bf16 (:3825-3836), gemm-int8 (:3839-3849),
gemm-int15 (:3852-3879), lowbit-conversions (:4024-4234).  The recorded
`train` hashes are in tests/golden/verify_gemm_cells.json (from
python/mojolearn/verify_reference/table.json).

Each lane takes the three callables it needs, so the same lane runs against the CPU
oracle (tests/test_oracle_golden.py) and against the MI355X surface
(tests/test_gpu_surface.py).
"""
import hashlib
import json
import os

import numpy as np

N, D = 20000, 16
FIXTURES = ["base", "ties", "hashed", "wide", "denormal", "denormal_ftz", "dupes", "odd", "negative"]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "verify_gemm_cells.json")


def golden():
    with open(GOLDEN) as fh:
        return json.load(fh)


def h(*arrays):
    m = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(np.asarray(a))
        m.update(str(a.dtype).encode())
        m.update(str(a.shape).encode())
        m.update(a.tobytes())
    return m.hexdigest()[:16]


def train_hash(parts):
    return h(np.frombuffer("|".join(f"{k}={v}" for k, v in sorted(parts.items())).encode(), dtype=np.uint8))


def _hashed_uniform(n, d, seed):
    ctr = np.arange(n * d, dtype=np.uint64)
    dig = hashlib.sha256(ctr.tobytes() + str(seed).encode()).digest()
    stream = bytearray()
    blk = 0
    while len(stream) < n * d * 4:
        stream += hashlib.sha256(dig + blk.to_bytes(8, "little")).digest()
        blk += 1
    u32 = np.frombuffer(bytes(stream[: n * d * 4]), dtype=np.uint32)
    return (u32.astype(np.float64) / 2**32).astype(np.float32).reshape(n, d)


def fixture_x(kind, n=N, d=D, seed=0):
    rng = np.random.default_rng(seed)
    if kind == "base":
        X = rng.standard_normal((n, d)).astype(np.float32)
    elif kind == "ties":
        X = rng.integers(0, 6, size=(n, d)).astype(np.float32)
    elif kind == "hashed":
        X = (_hashed_uniform(n, d, seed) * 4.0 - 2.0).astype(np.float32)
    elif kind == "wide":
        X = rng.standard_normal((n, d)).astype(np.float32)
        scale = np.logspace(-4, 4, d).astype(np.float32)
        X = (X * scale).astype(np.float32)
    elif kind == "denormal":
        X = rng.standard_normal((n, d)).astype(np.float32)
        X[: n // 4, :3] = (X[: n // 4, :3] * np.float32(1e-40)).astype(np.float32)
    elif kind == "denormal_ftz":
        X = fixture_x("denormal", n, d, seed)
        sub = (X != 0) & (np.abs(X) < np.finfo(np.float32).tiny)
        X = X.copy()
        X[sub] = np.copysign(np.float32(0.0), X[sub])
    elif kind == "dupes":
        X = rng.standard_normal((n, d)).astype(np.float32)
        X[n // 2:] = X[: n - n // 2]
        X[:, d - 2] = np.float32(3.5)
        X[:, d - 1] = np.float32(0.0)
    elif kind == "odd":
        n, d = 12345, 17
        X = rng.standard_normal((n, d)).astype(np.float32)
    elif kind == "negative":
        X = (-np.abs(rng.standard_normal((n, d))) - 2.0).astype(np.float32)
    else:
        raise ValueError(kind)
    return X


def lane_gemm_pinned(matmul, X):
    a = X[:256].T.copy()
    c1 = np.asarray(matmul(a.astype(np.float32), X[:256].astype(np.float32)))
    # X.size < 256 * 4096 for every fixture, so the lane's `wide` product is c1 again
    assert X.size < 256 * 4096
    return dict(small=h(c1), wide=h(c1))


def lane_gemm_transposed(matmul, X):
    a = np.ascontiguousarray(X[:256]).astype(np.float32)
    b = np.ascontiguousarray(X[256:384]).astype(np.float32)
    nt = np.asarray(matmul(a, b, transpose_b=True))
    at = np.ascontiguousarray(X[:256].T).astype(np.float32)
    c = np.ascontiguousarray(X[384:384 + at.shape[0]]).astype(np.float32)
    tn = np.asarray(matmul(at, c, transpose_a=True))
    return dict(nt=h(nt), tn=h(tn))


def lane_gemm_bf16(to_bf16, matmul_bf16, X):
    a = np.ascontiguousarray(X[:256]).astype(np.float32)
    b = np.ascontiguousarray(X[256:256 + 128]).astype(np.float32)
    bb = np.asarray(to_bf16(b))
    c1 = np.asarray(matmul_bf16(a, bb, transpose_b=True))
    c2 = np.asarray(matmul_bf16(np.asarray(to_bf16(a)), bb, transpose_b=True))
    c3 = np.asarray(matmul_bf16(np.ascontiguousarray(a[:64].T), np.asarray(to_bf16(a[64:128]))))
    return dict(nt=h(c1), both=h(c2), nn=h(c3), bits=h(bb))


def lane_gemm_int8(quantize_int8, matmul_int8, dequantize_int8, X):
    """int8i32.v1 on fixture slices: the quantizer's codes and exponents, the product of
    the two quantized operands (a . b^T) and a dequantization."""
    a = np.ascontiguousarray(X[:256]).astype(np.float32)
    b = np.ascontiguousarray(X[256:256 + 128]).astype(np.float32)
    qa, ea = quantize_int8(a)
    qb, eb = quantize_int8(b)
    c = matmul_int8((qa, ea), (qb, eb))
    return dict(codes=h(np.asarray(qa), np.asarray(qb)), exps=h(np.asarray(ea), np.asarray(eb)),
                product=h(np.asarray(c)), dequant=h(np.asarray(dequantize_int8(qb, eb))))


def lane_gemm_int15(quantize_int15, matmul_int15, dequantize_int15, int15_max_k, X):
    """int15i64.v1 on the same slices: the planes and exponents, the product from the planes
    and from the float32 operands (recorded as a number `same`), whether k above the
    profile's maximum is refused by name, and a dequantization."""
    a = np.ascontiguousarray(X[:256]).astype(np.float32)
    b = np.ascontiguousarray(X[256:256 + 128]).astype(np.float32)
    ah, al, ea = quantize_int15(a)
    bh, bl, eb = quantize_int15(b)
    c = np.asarray(matmul_int15((ah, al, ea), (bh, bl, eb)))
    c1 = np.asarray(matmul_int15(a, b))
    same = np.array([int(c.tobytes() == c1.tobytes())], dtype=np.int32)
    wide = np.zeros((1, int15_max_k + 1), dtype=np.float32)
    try:
        matmul_int15(wide, wide)
        refused = False
    except Exception as exc:  # noqa: BLE001 -- the lane records a refusal as a number
        refused = "65536" in str(exc)
    refuses = np.array([int(refused)], dtype=np.int32)
    return dict(planes=h(np.asarray(ah), np.asarray(al), np.asarray(bh), np.asarray(bl)),
                exps=h(np.asarray(ea), np.asarray(eb)), product=h(c), onecall=h(c1), flags=h(same, refuses),
                dequant=h(np.asarray(dequantize_int15(bh, bl, eb))))


LOWBIT_ROWS, LOWBIT_COLS = 64, 16


def lane_lowbit_conversions(lowbit, from_bf16, O, X):
    """The low-bit storage seams as a user reaches them (`pack_one`, `materialize_one`,
    `widen_bf16`, `format_of`, `is_packed`, `linalg.from_bf16`) on a 64 x 16 block of the
    fixture: the stored bytes, their float32 images, the same widening at three ranks, the
    predicates and refusals, and agreement with an independent construction (`O`, the CPU
    oracle, in the place of the harness's pure-Python spelling)."""
    a2 = np.ascontiguousarray(X[:LOWBIT_ROWS, :LOWBIT_COLS]).astype(np.float32)
    bf = lowbit.pack_one(a2, "bfloat16")
    q8 = lowbit.pack_one(a2, "int8")
    f32 = lowbit.pack_one(a2, "float32")
    bits = np.asarray(bf.bits)
    codes, exps = np.asarray(q8.codes), np.asarray(q8.exponents)
    mbf = np.asarray(lowbit.materialize_one(bf))
    mq8 = np.asarray(lowbit.materialize_one(q8))
    w1 = np.asarray(lowbit.widen_bf16(bits.reshape((LOWBIT_ROWS * LOWBIT_COLS,))))
    w3 = np.asarray(lowbit.widen_bf16(bits.reshape((4, LOWBIT_ROWS // 4, LOWBIT_COLS))))
    lin = np.asarray(from_bf16(bits))
    py_bits = O.bf16_narrow(a2)
    py_wide = O.bf16_widen(bits)
    py_codes, py_exps = O.q8_quantize(a2)
    py_deq = O.q8_dequantize(codes, exps)

    def refuses(fn, text):
        try:
            fn()
        except Exception as exc:  # noqa: BLE001 -- a refusal is recorded as a number
            return text in str(exc)
        return False

    flags = np.array([
        lowbit.is_packed(bf), lowbit.is_packed(q8), lowbit.is_packed(a2), lowbit.is_packed(f32),
        lowbit.format_of({"w": bf}) == "bfloat16", lowbit.format_of({"w": q8}) == "int8",
        lowbit.format_of({"w": a2}) == "float32", lowbit.format_of([bf, a2]) == "bfloat16",
        refuses(lambda: lowbit.format_of({"a": bf, "b": q8}), "store a model one way"),
        bf.format == "bfloat16" and tuple(bf.shape) == (LOWBIT_ROWS, LOWBIT_COLS),
        q8.format == "int8" and tuple(q8.shape) == (LOWBIT_ROWS, LOWBIT_COLS),
        refuses(lambda: lowbit.pack_one(a2[:, 0], "bfloat16"), "must be 2-D to pack"),
        refuses(lambda: lowbit.pack_one(a2, "float16"), "unknown format"),
        lin.tobytes() == mbf.tobytes(), w1.tobytes() == mbf.tobytes(), w3.tobytes() == mbf.tobytes(),
        np.asarray(f32).tobytes() == a2.tobytes(),
        py_bits.tobytes() == bits.tobytes(), py_wide.tobytes() == mbf.tobytes(),
        np.asarray(py_codes).tobytes() == codes.tobytes(), np.asarray(py_exps).tobytes() == exps.tobytes(),
        py_deq.tobytes() == mq8.tobytes(),
        False,
    ], dtype=np.int64)
    return dict(bf16_bits=h(bits), int8=h(codes, exps), materialized=h(mbf, mq8), widened=h(w1, w3),
                f32_copy=h(np.asarray(f32)), linalg=h(lin), flags=h(flags))


class OracleConversions:
    """The four conversions the lowbit module calls (`to_bf16`, `from_bf16`, `quantize_int8`,
    `dequantize_int8`), answered by the CPU oracle: installed in place of the module's linalg
    to run the lowbit lane on a machine with no GPU."""

    def __init__(self, O):
        self.O = O

    def to_bf16(self, x):
        return self.O.bf16_narrow(np.ascontiguousarray(x, dtype=np.float32))

    def from_bf16(self, bits):
        return self.O.bf16_widen(bits)

    def quantize_int8(self, x):
        return self.O.q8_quantize(x)

    def dequantize_int8(self, codes, exps):
        return self.O.nan_canon(self.O.q8_dequantize(codes, exps))


class OracleSurface:
    """The three surface calls the lanes need, answered by the CPU oracle."""

    def __init__(self, O):
        self.O = O

    def matmul(self, a, b, transpose_a=False, transpose_b=False, identical=True):
        op = 2 if transpose_a else (1 if transpose_b else 0)
        return self.O.nan_canon(self.O.gemm(a, b, op))

    def to_bf16(self, x):
        return self.O.bf16_narrow(np.ascontiguousarray(x, dtype=np.float32))

    def matmul_bf16(self, a, b, transpose_a=False, transpose_b=False):
        a = np.asarray(a)
        af = self.O.bf16_widen(a) if a.dtype == np.uint16 else a
        return self.matmul(af, self.O.bf16_widen(b), transpose_a, transpose_b)

    def quantize_int8(self, x):
        return self.O.q8_quantize(x)

    def dequantize_int8(self, codes, exps):
        return self.O.nan_canon(self.O.q8_dequantize(codes, exps))

    def matmul_int8(self, a, b):
        qa, ea = a if isinstance(a, tuple) else self.O.q8_quantize(a)
        qb, eb = b if isinstance(b, tuple) else self.O.q8_quantize(b)
        return self.O.nan_canon(self.O.q8_gemm(qa, ea, qb, eb))

    def quantize_int15(self, x):
        return self.O.q15_quantize(x)

    def dequantize_int15(self, hi, lo, exps):
        return self.O.nan_canon(self.O.q15_dequantize(hi, lo, exps))

    def matmul_int15(self, a, b):
        ah, al, ea = a if isinstance(a, tuple) else self.O.q15_quantize(a)
        bh, bl, eb = b if isinstance(b, tuple) else self.O.q15_quantize(b)
        k = np.asarray(ah).shape[1]
        if k > self.O.INT15_MAX_K:
            raise ValueError(f"matmul_int15: k={k} is above {self.O.INT15_MAX_K}")
        return self.O.nan_canon(self.O.q15_gemm(ah, al, ea, bh, bl, eb))
