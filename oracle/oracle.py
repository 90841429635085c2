"""ctypes wrapper of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker.  The product (mojolearn_amd) never calls it.

Each function restates a reference function; the file:line is on the C side
(oracle/gemm_oracle.c).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

OP_NN, OP_NT, OP_TN = 0, 1, 2


def build(sabotage=False):
    """Compile liboracle.so in place (gcc; see oracle/Makefile); with `sabotage`, also the
    planted-mistake variants under oracle/_sabotage/."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    if sabotage:
        build_sabotage()


#: The planted mistakes of gemm_oracle.c (ORC_SABOTAGE = n), by name.
SABOTAGE = {1: "fold_stride_pairs", 2: "fold_pad_zero", 3: "fold_serial", 4: "step_unfused",
            5: "step_flush_before_round", 6: "operands_unflushed", 7: "leaf_from_tile",
            8: "seed_minus_zero", 9: "no_nan_canon", 10: "bias_unflushed", 11: "scale_unflushed",
            12: "accumulator_unflushed", 13: "host_rows_no_redo"}


def sabotage_path(n):
    return os.path.join(_HERE, "_sabotage", f"liboracle_s{n}.so")


def build_sabotage():
    subprocess.run(["make", "-s", "-C", _HERE, "sabotage"], check=True)


class using:
    """Within the block, every function of this module calls the library at `path` (a
    planted-mistake variant) instead of liboracle.so."""

    def __init__(self, path):
        self.path = path

    def __enter__(self):
        global _lib
        self._saved = _lib
        _lib = _configure(ctypes.CDLL(self.path))
        return self

    def __exit__(self, *exc):
        global _lib
        _lib = self._saved
        return False


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = _configure(ctypes.CDLL(_LIB_PATH))
    return _lib


def _configure(L):
    i64, vp, c_int, f32 = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    L.orc_leaf_size.argtypes = [i64]; L.orc_leaf_size.restype = i64
    L.orc_leaf_count.argtypes = [i64, i64]; L.orc_leaf_count.restype = i64
    L.orc_gemm.argtypes = [vp, vp, vp, i64, i64, i64, c_int, i64]; L.orc_gemm.restype = None
    L.orc_gemm_serial.argtypes = [vp, vp, vp, i64, i64, i64, c_int]; L.orc_gemm_serial.restype = None
    L.orc_gemm_fast.argtypes = [vp, vp, vp, i64, i64, i64, c_int, i64, c_int]; L.orc_gemm_fast.restype = None
    L.orc_fold_tree.argtypes = [vp, i64]; L.orc_fold_tree.restype = f32
    L.orc_fold_stack.argtypes = [vp, i64]; L.orc_fold_stack.restype = f32
    L.orc_bias.argtypes = [vp, vp, i64, i64]; L.orc_bias.restype = None
    L.orc_nan_canon.argtypes = [vp, i64]; L.orc_nan_canon.restype = None
    L.orc_bf16_widen.argtypes = [vp, vp, i64]; L.orc_bf16_widen.restype = None
    L.orc_bf16_narrow.argtypes = [vp, vp, i64]; L.orc_bf16_narrow.restype = None
    L.orc_int8_dequant.argtypes = [vp, vp, vp, i64, i64, c_int]; L.orc_int8_dequant.restype = None
    L.orc_fnv1a64.argtypes = [vp, i64]; L.orc_fnv1a64.restype = ctypes.c_uint64
    L.orc_q8_i32_to_f32.argtypes = [ctypes.c_int32]; L.orc_q8_i32_to_f32.restype = f32
    L.orc_q8_row_exponent.argtypes = [f32]; L.orc_q8_row_exponent.restype = c_int
    L.orc_q8_quantize_rows.argtypes = [vp, vp, vp, i64, i64]; L.orc_q8_quantize_rows.restype = None
    L.orc_q8_dequantize_rows.argtypes = [vp, vp, vp, i64, i64]; L.orc_q8_dequantize_rows.restype = None
    L.orc_q8_gemm.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64]; L.orc_q8_gemm.restype = None
    L.orc_q15_i64_to_f32.argtypes = [i64]; L.orc_q15_i64_to_f32.restype = f32
    L.orc_q15_row_exponent.argtypes = [f32]; L.orc_q15_row_exponent.restype = c_int
    L.orc_q15_quantize_rows.argtypes = [vp, vp, vp, vp, i64, i64]; L.orc_q15_quantize_rows.restype = None
    L.orc_q15_dequantize_rows.argtypes = [vp, vp, vp, vp, i64, i64]; L.orc_q15_dequantize_rows.restype = None
    L.orc_q15_gemm.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64]; L.orc_q15_gemm.restype = None
    L.orc_f16_widen.argtypes = [vp, vp, i64]; L.orc_f16_widen.restype = None
    L.orc_card_fill.argtypes = [vp, i64, i64]; L.orc_card_fill.restype = None
    L.orc_ftz.argtypes = [f32]; L.orc_ftz.restype = f32
    L.orc_fma.argtypes = [f32, f32, f32]; L.orc_fma.restype = f32
    L.orc_max_threads.argtypes = []; L.orc_max_threads.restype = c_int
    L.orc_seq_gemm.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i64, i64, i64, c_int]
    L.orc_seq_gemm.restype = None
    L.orc_epilogue.argtypes = [vp, i64, i64, i64, c_int, vp, c_int]; L.orc_epilogue.restype = None
    L.orc_map.argtypes = [vp, vp, i64, c_int]; L.orc_map.restype = None
    for name in ("orc_expf", "orc_sigmoidf", "orc_tanhf"):
        getattr(L, name).argtypes = [f32]
        getattr(L, name).restype = f32
    L.orc_act_value.argtypes = [f32, c_int]; L.orc_act_value.restype = f32
    L.orc_act_bwd_value.argtypes = [f32, f32, c_int]; L.orc_act_bwd_value.restype = f32
    L.orc_host_rows.argtypes = [vp, vp, vp, i64, i64, i64, c_int, c_int, c_int]; L.orc_host_rows.restype = None
    return L


def _p(x):
    return x.ctypes.data_as(ctypes.c_void_p)


def _shape(a, b, op):
    if op == OP_NN:
        (m, k), (kb, n) = a.shape, b.shape
    elif op == OP_NT:
        (m, k), (n, kb) = a.shape, b.shape
    elif op == OP_TN:
        (k, m), (kb, n) = a.shape, b.shape
    else:
        raise ValueError(op)
    assert k == kb, (a.shape, b.shape, op)
    return m, n, k


def _f32c(x):
    x = np.ascontiguousarray(x)
    assert x.dtype == np.float32
    return x


def leaf_size(k):
    return lib().orc_leaf_size(k)


def leaf_count(k, leaf):
    return lib().orc_leaf_count(k, leaf)


def gemm(a, b, op=OP_NN, leaf=0):
    """gemm/host/gemm_oracle.mojo:357-371 `gemm_oracle` (leaf=0), or `gemm_oracle_at_leaf`."""
    a, b = _f32c(a), _f32c(b)
    m, n, k = _shape(a, b, op)
    c = np.empty((m, n), np.float32)
    lib().orc_gemm(_p(c), _p(a), _p(b), m, n, k, op, leaf)
    return c


def gemm_serial(a, b, op=OP_NN):
    """gemm/host/gemm_oracle.mojo:473-524 `gemm_oracle_serial`."""
    a, b = _f32c(a), _f32c(b)
    m, n, k = _shape(a, b, op)
    c = np.empty((m, n), np.float32)
    lib().orc_gemm_serial(_p(c), _p(a), _p(b), m, n, k, op)
    return c


def gemm_fast(a, b, op=OP_NN, leaf=0, threads=0):
    """Same bits as `gemm`, AVX2 + threads (role of gemm/host/gemm_host_rows.mojo)."""
    a, b = _f32c(a), _f32c(b)
    m, n, k = _shape(a, b, op)
    c = np.empty((m, n), np.float32)
    lib().orc_gemm_fast(_p(c), _p(a), _p(b), m, n, k, op, leaf, threads)
    return c


def host_rows(a, b, op=OP_NN, threads=0, force_redo=False):
    """gemm/host/gemm_host_rows.mojo:492-556 `gemm_host_rows_into`: orc_gemm's bits (NaN words
    equal after canonicalization) with the deferred flush and its redo, on `threads` threads."""
    a, b = _f32c(a), _f32c(b)
    m, n, k = _shape(a, b, op)
    c = np.empty((m, n), np.float32)
    lib().orc_host_rows(_p(c), _p(a), _p(b), m, n, k, op, threads, 1 if force_redo else 0)
    return c


def fold_tree(parts):
    buf = np.array(parts, dtype=np.float32, copy=True)
    return np.float32(lib().orc_fold_tree(_p(buf), len(buf)))


def fold_stack(parts):
    buf = np.ascontiguousarray(np.asarray(parts, dtype=np.float32))
    return np.float32(lib().orc_fold_stack(_p(buf), len(buf)))


def bias(y, b):
    y = np.array(y, dtype=np.float32, copy=True)
    b = _f32c(b)
    lib().orc_bias(_p(y), _p(b), y.shape[0], y.shape[1])
    return y


def nan_canon(x):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().orc_nan_canon(_p(x), x.size)
    return x


def bf16_widen(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_bf16_widen(_p(out), _p(bits), bits.size)
    return out


def bf16_narrow(x):
    x = _f32c(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_narrow(_p(out), _p(x), x.size)
    return out


def int8_dequant(codes, scales, op=OP_NN):
    """W_eff = ftz(f32(code) * scale[col]) in the B layout of `op`."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = _f32c(scales)
    if op == OP_NT:
        n, k = codes.shape
    else:
        k, n = codes.shape
    out = np.empty(codes.shape, np.float32)
    lib().orc_int8_dequant(_p(out), _p(codes), _p(scales), n, k, op)
    return out


def fnv1a64(x):
    x = np.ascontiguousarray(x)
    return int(lib().orc_fnv1a64(_p(x), x.nbytes))


def card_fill(count, salt):
    out = np.empty(count, np.float32)
    lib().orc_card_fill(_p(out), count, salt)
    return out


def ftz(x):
    return np.float32(lib().orc_ftz(float(np.float32(x))))


def max_threads():
    return lib().orc_max_threads()


# ---- profile mojolearn.identical.gemm.int8i32.v1 (gemm/IDENTICAL_LOWBIT_CONTRACT.md L-3..L-7)

INT8_MAX_K = 131072


def q8_quantize(x):
    """Per-row power-of-two exponent and int8 codes (L-3, L-4): (codes int8, exponents int32)."""
    x = _f32c(x)
    rows, cols = x.shape
    codes = np.empty((rows, cols), np.int8)
    exps = np.empty(rows, np.int32)
    lib().orc_q8_quantize_rows(_p(codes), _p(exps), _p(x), rows, cols)
    return codes, exps


def q8_dequantize(codes, exps):
    """codes * 2^exponent per row, the pinned dequantization (L-5, L-6)."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    exps = np.ascontiguousarray(exps, dtype=np.int32)
    rows, cols = codes.shape
    out = np.empty((rows, cols), np.float32)
    lib().orc_q8_dequantize_rows(_p(out), _p(codes), _p(exps), rows, cols)
    return out


def q8_gemm(qa, ea, qb, eb):
    """C = qa . qb^T (OP_NT) as int8i32.v1: the exact Int32 sum, pinned to float32, scaled."""
    qa = np.ascontiguousarray(qa, dtype=np.int8)
    qb = np.ascontiguousarray(qb, dtype=np.int8)
    ea = np.ascontiguousarray(ea, dtype=np.int32)
    eb = np.ascontiguousarray(eb, dtype=np.int32)
    (m, k), (n, kb) = qa.shape, qb.shape
    assert k == kb and ea.size == m and eb.size == n
    c = np.empty((m, n), np.float32)
    lib().orc_q8_gemm(_p(c), _p(qa), _p(ea), _p(qb), _p(eb), m, n, k)
    return c


def q8_i32_to_f32(v):
    return lib().orc_q8_i32_to_f32(int(v))


def q8_row_exponent(absmax):
    return lib().orc_q8_row_exponent(float(absmax))


# ---- profile mojolearn.identical.gemm.int15i64.v1 (contract section 6, W-1..W-7)

INT15_MAX_K = 65536


def q15_quantize(x):
    """(hi int8, lo int8, exponents int32): W-1/W-2 codes as W-3 planes, code = hi * 128 + lo."""
    x = _f32c(x)
    rows, cols = x.shape
    hi = np.empty((rows, cols), np.int8)
    lo = np.empty((rows, cols), np.int8)
    exps = np.empty(rows, np.int32)
    lib().orc_q15_quantize_rows(_p(hi), _p(lo), _p(exps), _p(x), rows, cols)
    return hi, lo, exps


def q15_dequantize(hi, lo, exps):
    hi = np.ascontiguousarray(hi, dtype=np.int8)
    lo = np.ascontiguousarray(lo, dtype=np.int8)
    exps = np.ascontiguousarray(exps, dtype=np.int32)
    rows, cols = hi.shape
    out = np.empty((rows, cols), np.float32)
    lib().orc_q15_dequantize_rows(_p(out), _p(hi), _p(lo), _p(exps), rows, cols)
    return out


def q15_gemm(ah, al, ea, bh, bl, eb):
    """C = a . b^T (OP_NT) as int15i64.v1: the exact Int64 sum of code products, W-6, W-7."""
    ah, al, bh, bl = (np.ascontiguousarray(t, dtype=np.int8) for t in (ah, al, bh, bl))
    ea = np.ascontiguousarray(ea, dtype=np.int32)
    eb = np.ascontiguousarray(eb, dtype=np.int32)
    (m, k), (n, kb) = ah.shape, bh.shape
    assert k == kb and al.shape == ah.shape and bl.shape == bh.shape and ea.size == m and eb.size == n
    c = np.empty((m, n), np.float32)
    lib().orc_q15_gemm(_p(c), _p(ah), _p(al), _p(ea), _p(bh), _p(bl), _p(eb), m, n, k)
    return c


def q15_i64_to_f32(v):
    return lib().orc_q15_i64_to_f32(int(v))


def q15_row_exponent(absmax):
    return lib().orc_q15_row_exponent(float(absmax))


def f16_widen(bits):
    """float16 bits (uint16) -> float32, exact, NaN payloads kept (gemm/f16_widen.mojo:12-37)."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.uint32)
    lib().orc_f16_widen(_p(out), _p(bits), bits.size)
    return out.view(np.float32)


# ---- the sequence executor's GEMM word and its followers

EPI_NONE, EPI_PLUS_BIAS, EPI_BIAS_ACT, EPI_ACT_BWD = 0, 3, 4, 5
ACT_IDENTITY, ACT_LOGISTIC, ACT_TANH, ACT_RELU, ACT_SOFTMAX = 0, 1, 2, 3, 4


def seq_gemm(c, a, b, m, n, k, a_si, a_sp, b_sp, b_sj, ldc, accumulate):
    """sequence/ops.mojo:518-531 `op_gemm` on flat float32 buffers, in place on `c`: one whole-k
    chain per cell, seeded by the flushed old C when `accumulate`, else +0."""
    for x in (c, a, b):
        assert x.dtype == np.float32 and x.flags.c_contiguous
    assert c.flags.writeable
    if m > 0 and n > 0:
        assert c.size >= (m - 1) * ldc + n
        assert k == 0 or a.size > (m - 1) * a_si + (k - 1) * a_sp
        assert k == 0 or b.size > (k - 1) * b_sp + (n - 1) * b_sj
    lib().orc_seq_gemm(_p(c), _p(a), _p(b), m, n, k, a_si, a_sp, b_sp, b_sj, ldc, 1 if accumulate else 0)
    return c


def epilogue(c, ldc, m, n, kind, p=None, act=0):
    """The product's followers (gemm/checks/gemm_identical.mojo:8891-8912) in place on `c`."""
    assert c.dtype == np.float32 and c.flags.c_contiguous
    if kind in (EPI_PLUS_BIAS, EPI_BIAS_ACT):
        p = _f32c(p); assert p.size >= n
    elif kind == EPI_ACT_BWD:
        p = _f32c(p); assert p.size >= m * n
    else:
        p = np.zeros(1, np.float32)
    lib().orc_epilogue(_p(c), ldc, m, n, kind, _p(p), act)
    return c


def fmap(x, which):
    """Elementwise expf (0), sigmoidf (1), tanhf (2) or 1/x (3) of the restatements."""
    x = _f32c(x)
    out = np.empty_like(x)
    lib().orc_map(_p(out), _p(x), x.size, which)
    return out


def act_value(z, code):
    return lib().orc_act_value(z, code)


def act_bwd_value(d, z, code):
    return lib().orc_act_bwd_value(d, z, code)
