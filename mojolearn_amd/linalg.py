"""Float32 bit-identical matrix product on MI355X: the surface of `mojolearn.linalg`
for the identical fp32 GEMM path (python/mojolearn/linalg.py, _linalg_impl.py:91-415),
backed by the gfx950 kernels of libmlgemm.so through its C op table.

`matmul` computes ``op(a) @ op(b)`` under the profile ``mojolearn.identical.gemm.fp32.v1``:
k-leaves of `contract_leaf_size(k)` accumulated serially ascending with one FMA per step,
flush-to-zero at every seam, folded by the fixed balanced tree, NaN words canonicalized.
The same names, operation table, refusals and exception types as the reference surface;
argument admission restates bindings/linalg_ops_lowbit_door.mojo:259-416,654-710.

Results are NumPy arrays (``numpy.asarray`` on them is the identity).
"""
import numpy as np

from . import _native

PROFILE_FAMILY = "mojolearn.identical.gemm.fp32"
PROFILE_VERSION = 1
PROFILE = f"{PROFILE_FAMILY}.v{PROFILE_VERSION}"
LOWBIT_PROFILE_VERSION = 1
PROFILE_BF16 = f"mojolearn.identical.gemm.bf16f32.v{LOWBIT_PROFILE_VERSION}"
#: This build's int8-weight extension: int8 codes times one float32 scale per output
#: column, dequantized exactly as ftz(f32(code) * ftz(scale)) and then fp32.v1.
PROFILE_INT8W = "mojolearn.identical.gemm.int8w-colscale-f32.v1"
PROFILE_INT8 = f"mojolearn.identical.gemm.int8i32.v{LOWBIT_PROFILE_VERSION}"
#: Contract L-7: the Int32 sum of k products of codes in [-127, 127] stays exact.
INT8_MAX_K = 131072
INT15_PROFILE_VERSION = 1
PROFILE_INT15 = f"mojolearn.identical.gemm.int15i64.v{INT15_PROFILE_VERSION}"
#: Contract W-4: the shared cross-term accumulator stays exact to k = 66052; a power of two below.
INT15_MAX_K = 65536

OP_NN, OP_NT, OP_TN = 0, 1, 2

# op codes of the native table (gemm/linalg_dispatch.mojo:14-75, + this build's 15, 16)
_LIN_OP_GEMM = 0
_LIN_OP_GEMM_BF16 = 1
_LIN_OP_GEMM_INT8 = 2
_LIN_OP_QUANTIZE_INT8 = 3
_LIN_OP_DEQUANTIZE_INT8 = 4
_LIN_OP_GEMM_INT15 = 5
_LIN_OP_QUANTIZE_INT15 = 6
_LIN_OP_DEQUANTIZE_INT15 = 7
_LIN_OP_FROM_F16 = 10
_LIN_OP_INT15_VERSION = 14
_LIN_OP_TO_BF16 = 8
_LIN_OP_FROM_BF16 = 9
_LIN_OP_MODE = 11
_LIN_OP_PROFILE_VERSION = 12
_LIN_OP_LOWBIT_VERSION = 13
_LIN_OP_GEMM_INT8W = 15
_LIN_OP_GEMM_BIAS = 16


def _shape_text(shape):
    return "(" + ", ".join(str(int(s)) for s in shape) + ("," if len(shape) == 1 else "") + ")"


def _dtype_name(x):
    return str(x.dtype)


def _asarray(x):
    return x if isinstance(x, np.ndarray) else np.asarray(x)


def _operand(x, name):
    """`lin_operand`: a float32 2-D buffer, refused by name otherwise, in C order (a layout
    copy at most, never a cast).  bindings/linalg_ops_lowbit_door.mojo:259-296."""
    v = _asarray(x)
    if v.dtype != np.float32:
        raise TypeError(
            f"mojolearn.linalg: {name} has dtype {_dtype_name(v)}, and only float32 is in this profile "
            f"({PROFILE}; contract section 1 makes FP32 a hard requirement, and section 0.5 excludes FP16, "
            "BF16, TF32 and float64). Refused rather than cast, because a cast from float64 drops mantissa "
            f"bits you may care about. Convert it yourself with np.asarray({name}, dtype=np.float32) if that "
            "is what you want.")
    if v.ndim != 2:
        raise ValueError(
            f"mojolearn.linalg: {name} must be 2-D, got {v.ndim}-D shape {_shape_text(v.shape)}. A vector "
            "product is OP_NT at n == 1 (contract 0.1); pass it as a 2-D array of shape (n, k) or (k, 1).")
    if v.size == 0:
        raise ValueError(
            f"mojolearn.linalg: {name} has shape {_shape_text(v.shape)} and no elements. Contract section 8 "
            "does specify the degenerate shapes (k == 0 writes +0.0 into every cell; m == 0 or n == 0 writes "
            "nothing), but no gate in this tree has run them through the Python surface, so they are refused "
            "here rather than answered unchecked.")
    return np.ascontiguousarray(v)


def _operand_bits(x, name):
    """`lin_operand_bits`: a 2-D uint16 buffer of bf16 bits in C order (door :299-316)."""
    v = _asarray(x)
    if v.dtype != np.uint16:
        raise TypeError(
            f"mojolearn.linalg: {name} has dtype {_dtype_name(v)}; the bf16 profile takes bf16 BITS in a "
            "uint16 buffer, which to_bf16() produces. Refused rather than reinterpreted.")
    if v.ndim != 2:
        raise ValueError(f"mojolearn.linalg: {name} must be 2-D, got {v.ndim}-D")
    if v.size == 0:
        raise ValueError(f"mojolearn.linalg: {name} has no elements")
    return np.ascontiguousarray(v)


def _out(out, m, n, who):
    """`lin_out` (door :327-343): a new float32 (m, n) array, or the caller's, checked."""
    if out is None:
        return np.empty((m, n), dtype=np.float32)
    if not isinstance(out, np.ndarray):
        out = np.asarray(out)
    if out.dtype != np.float32:
        raise TypeError(f"mojolearn.linalg.{who}: out must be float32")
    if out.ndim != 2 or out.shape[0] != m or out.shape[1] != n:
        raise ValueError(f"mojolearn.linalg.{who}: out has shape {_shape_text(out.shape)}, want ({m}, {n})")
    if not out.flags.c_contiguous or not out.flags.writeable:
        raise ValueError(f"mojolearn.linalg.{who}: out must be C-contiguous and writable")
    return out


def _op_and_shape(a, b, transpose_a, transpose_b, who):
    """`_lin_op_and_shape` (door :654-686)."""
    ta, tb = bool(transpose_a), bool(transpose_b)
    if ta and tb:
        raise ValueError(
            f"mojolearn.linalg.{who}: transpose_a and transpose_b together is not one of the contract's three "
            "operations (section 0.1); write (b @ a).T with the flags swapped, in your own source.")
    if ta:
        op, (k, m), (kb, n) = OP_TN, a.shape, b.shape
    elif tb:
        op, (m, k), (n, kb) = OP_NT, a.shape, b.shape
    else:
        op, (m, k), (kb, n) = OP_NN, a.shape, b.shape
    if k != kb:
        raise ValueError(
            f"mojolearn.linalg.{who}: contracted extents differ, a gives k={k} and b gives k={kb} "
            f"(a.shape={_shape_text(a.shape)}, b.shape={_shape_text(b.shape)}, transpose_a={transpose_a}, "
            f"transpose_b={transpose_b})")
    return op, m, n, k


def numeric_mode():
    """'identical': the mode of the loaded binary, read back from it (op 11)."""
    mode = _native.call(_LIN_OP_MODE, [], [])
    if mode != 1:
        raise RuntimeError(f"mojolearn.linalg: the loaded linalg binary reports numeric mode {mode}")
    version = _native.call(_LIN_OP_PROFILE_VERSION, [], [])
    if version != PROFILE_VERSION:
        raise RuntimeError(
            f"mojolearn.linalg: the loaded binary computes profile version {version}, this module "
            f"expects {PROFILE_VERSION} ({PROFILE})")
    return "identical"


def profile():
    """The matrix-product profile this process loaded, as a dict (python/mojolearn/_linalg_impl.py:170-190)."""
    mode = numeric_mode()
    return {
        "profile": PROFILE,
        "profile_family": PROFILE_FAMILY,
        "profile_version": PROFILE_VERSION,
        "lowbit_profile_version": _native.call(_LIN_OP_LOWBIT_VERSION, [], []),
        "numeric_mode": mode,
        "identity_claimed": mode == "identical",
        "dtype": "float32",
        "ops": ["OP_NN", "OP_NT", "OP_TN"],
        "binary": _native.LIB_PATH,
        "abi": _native.lib().mlg_abi_name().decode(),
    }


def require_identical():
    """Raise RuntimeError unless the loaded binary is the identical build."""
    if numeric_mode() != "identical":
        raise RuntimeError("mojolearn.linalg: the identical build is not loaded")


def matmul(a, b, *, transpose_a=False, transpose_b=False, out=None, identical=True):
    """Float32 matrix product ``op(a) @ op(b)`` with the bits of ``mojolearn.identical.gemm.fp32.v1``.

    ===========  ===========  ===========  ========  ========
    transpose_a  transpose_b  C            a.shape   b.shape
    ===========  ===========  ===========  ========  ========
    False        False        ``a @ b``    (m, k)    (k, n)
    False        True         ``a @ b.T``  (m, k)    (n, k)
    True         False        ``a.T @ b``  (k, m)    (k, n)
    ===========  ===========  ===========  ========  ========

    Both True raises ValueError.  Non-float32 operands raise TypeError (never cast).
    NaN output words are 0x7FC00000.  Restates bindings/linalg_ops_lowbit_door.mojo:347-416.
    """
    if identical:
        require_identical()
    else:
        numeric_mode()
    ta, tb = bool(transpose_a), bool(transpose_b)
    if ta and tb:
        raise ValueError(
            f"mojolearn.linalg.matmul: transpose_a=True with transpose_b=True is refused. {PROFILE} has "
            "exactly three operations (contract section 0.1: OP_NN, OP_NT, OP_TN) and a.T @ b.T is not one "
            "of them. This function will not materialize a transpose to fake a fourth. If you want it, write "
            "the identity yourself:\n    np.ascontiguousarray(np.asarray(matmul(b, a)).T)\nwhich is "
            "(b @ a).T == a.T @ b.T, runs as OP_NN, and leaves the extra step visible in your source where "
            "you can price it.")
    op = OP_NN if not ta and not tb else (OP_NT if tb else OP_TN)
    A = _operand(a, "a")
    B = _operand(b, "b")
    m = A.shape[1] if ta else A.shape[0]
    k = A.shape[0] if ta else A.shape[1]
    n = B.shape[0] if tb else B.shape[1]
    kb = B.shape[1] if tb else B.shape[0]
    if k != kb:
        raise ValueError(
            f"mojolearn.linalg.matmul: contracted extents disagree, a gives k={k} and b gives k={kb} "
            f"(a.shape={_shape_text(A.shape)}, b.shape={_shape_text(B.shape)}, transpose_a={ta}, "
            f"transpose_b={tb}). The row-major shapes for each op are in this function's table and in "
            "contract section 0.1.")
    if out is None:
        C = np.empty((m, n), dtype=np.float32)
    else:
        C = out if isinstance(out, np.ndarray) else np.asarray(out)
        if C.dtype != np.float32:
            raise TypeError(
                f"mojolearn.linalg.matmul: out has dtype {C.dtype}, and the profile's output is float32 "
                "(contract section 1). Refused rather than cast on the way out.")
        if C.ndim != 2 or C.shape[0] != m or C.shape[1] != n:
            raise ValueError(f"mojolearn.linalg.matmul: out has shape {_shape_text(C.shape)}, want ({m}, {n})")
        if not C.flags.c_contiguous:
            raise ValueError(
                "mojolearn.linalg.matmul: out must be C-contiguous; the device writes it directly (contract "
                "section 2). A non-contiguous out cannot be written in place, and copying into it afterwards "
                "would make `out` a lie about where the result was produced.")
        if not C.flags.writeable:
            raise ValueError(
                "mojolearn.linalg.matmul: out is read-only, refusing to write to it; the device writes `out` "
                "directly (contract section 2) and a read-only buffer handed to it is memory corruption, not "
                "an exception.")
    _native.call(_LIN_OP_GEMM, [C.ctypes.data, A.ctypes.data, B.ctypes.data], [m, n, k, op])
    return C if out is None else out


def matmul_bf16(a, b, *, transpose_a=False, transpose_b=False, out=None):
    """Matrix product with bfloat16 operands under ``mojolearn.identical.gemm.bf16f32.v1``.

    `b` is bfloat16 bits (uint16, from `to_bf16`); `a` is float32 or bfloat16 bits.  The
    operands are widened exactly and multiplied with `matmul`'s arithmetic, so
    ``matmul(from_bf16(a_bits), from_bf16(b_bits))`` gives the same bits.
    """
    require_identical()
    av = _asarray(a)
    a_bits = av.dtype == np.uint16
    A = _operand_bits(av, "a") if a_bits else _operand(av, "a")
    B = _operand_bits(b, "b")
    op, m, n, k = _op_and_shape(A, B, transpose_a, transpose_b, "matmul_bf16")
    C = _out(out, m, n, "matmul_bf16")
    _native.call(_LIN_OP_GEMM_BF16, [C.ctypes.data, A.ctypes.data, B.ctypes.data], [m, n, k, op, 1 if a_bits else 0])
    return C


def to_bf16(x):
    """float32 -> bfloat16 bits: flush, then round to nearest even (L-2)."""
    v = np.ascontiguousarray(_asarray(x))
    if v.dtype != np.float32:
        raise TypeError(f"mojolearn.linalg.to_bf16: x has dtype {v.dtype}, want float32")
    if v.size == 0:
        raise ValueError("mojolearn.linalg.to_bf16: x has no elements")
    out = np.empty(v.shape, dtype=np.uint16)
    _native.call(_LIN_OP_TO_BF16, [out.ctypes.data, v.ctypes.data], [v.size])
    return out


def from_bf16(bits):
    """bfloat16 bits (uint16) -> float32, exactly (L-1)."""
    v = np.ascontiguousarray(_asarray(bits))
    if v.dtype != np.uint16:
        raise TypeError(f"mojolearn.linalg.from_bf16: bits has dtype {v.dtype}, want uint16")
    if v.size == 0:
        raise ValueError("mojolearn.linalg.from_bf16: bits has no elements")
    out = np.empty(v.shape, dtype=np.float32)
    _native.call(_LIN_OP_FROM_BF16, [out.ctypes.data, v.ctypes.data], [v.size])
    return out


def matmul_int8w(a, codes, scales, *, transpose_b=False, out=None):
    """``a @ W`` with W stored as int8 codes and one float32 scale per output column.

    Extension of this build (profile `PROFILE_INT8W`): ``W[p, j] = ftz(f32(codes[p, j]) *
    ftz(scales[j]))`` -- one RNE multiply -- then fp32.v1.  `codes` is (k, n), or (n, k)
    with ``transpose_b=True`` (the LM's ``W[out, in]`` layout).
    """
    require_identical()
    A = _operand(a, "a")
    Q = _asarray(codes)
    if Q.dtype != np.int8:
        raise TypeError(f"mojolearn.linalg.matmul_int8w: codes has dtype {Q.dtype}, want int8")
    if Q.ndim != 2 or Q.size == 0:
        raise ValueError("mojolearn.linalg.matmul_int8w: codes must be 2-D and non-empty")
    Q = np.ascontiguousarray(Q)
    op, m, n, k = _op_and_shape(A, Q, False, transpose_b, "matmul_int8w")
    S = np.ascontiguousarray(_asarray(scales))
    if S.dtype != np.float32 or S.size != n:
        raise ValueError(f"mojolearn.linalg.matmul_int8w: scales must hold n={n} float32 values")
    C = _out(out, m, n, "matmul_int8w")
    _native.call(_LIN_OP_GEMM_INT8W, [C.ctypes.data, A.ctypes.data, Q.ctypes.data, S.ctypes.data], [m, n, k, op])
    return C


_RESHAPE_HINT = ("Reshape your data either using array.reshape(-1, 1) if your data has a single feature or "
                 "array.reshape(1, -1) if it contains a single sample.")


def _typed(x, dtype, ndim, name):
    """`admit_typed` (bindings/admitted_input_unpack.mojo:1198-1233): `x` as C-order words of
    `dtype` and rank `ndim`, converted by astype's rules when it has another numeric dtype,
    refused when empty."""
    v = _asarray(x)
    if v.dtype.kind not in "biuf":
        raise TypeError(f"mojolearn: {name} has buffer format '{v.dtype.str}', which is not a numeric array")
    if v.ndim != ndim:
        hint = ". " + _RESHAPE_HINT if ndim == 2 and v.ndim < 2 else ""
        raise ValueError(f"mojolearn: {name} must be {ndim}-D, got {v.ndim}-D shape {_shape_text(v.shape)}{hint}")
    if v.size == 0:
        what = "feature(s)" if v.ndim == 2 and v.shape[0] != 0 else "sample(s)"
        shape = _shape_text(v.shape)
        raise ValueError(f"mojolearn: {name} is empty, shape {shape}: Found array with 0 {what} (shape={shape}) "
                         "while a minimum of 1 is required.")
    return np.ascontiguousarray(v, dtype=dtype)


def _quantize(A):
    """`lin_quantize_int8` (bindings/linalg_ops_lowbit_door.mojo:565-575) of an admitted operand."""
    rows, cols = A.shape
    codes = np.empty((rows, cols), dtype=np.int8)
    exps = np.empty((rows,), dtype=np.int32)
    _native.call(_LIN_OP_QUANTIZE_INT8, [codes.ctypes.data, exps.ctypes.data, A.ctypes.data], [rows, cols])
    return codes, exps


def quantize_int8(x):
    """Quantize a 2-D float32 matrix to int8 codes with one power-of-two exponent per row
    (profile ``mojolearn.identical.gemm.int8i32.v1``, contract L-3 and L-4).

    Per row ``e = floor(log2(max |x|)) - 6`` (0 for an all-zero row) and
    ``code = clamp(round_half_even(ftz(x) * 2**-e), -127, 127)``, a NaN coding to 0.
    Returns ``(codes, exponents)``: int8 of `x`'s shape and int32 of shape (rows,), so that
    ``row ~= codes * 2**exponent``.  python/mojolearn/_linalg_impl.py:330-340.
    """
    require_identical()
    return _quantize(_operand(x, "x"))


def dequantize_int8(codes, exponents):
    """float32 ``codes * 2**exponents[row]`` exactly (contract L-6) from `quantize_int8` output.
    bindings/linalg_ops_lowbit_door.mojo:585-601."""
    require_identical()
    Q = _typed(codes, np.int8, 2, "codes")
    E = _typed(exponents, np.int32, 1, "exponents")
    rows, cols = Q.shape
    if E.shape[0] != rows:
        raise ValueError(f"mojolearn.linalg.dequantize_int8: exponents has shape {_shape_text(E.shape)}, "
                         f"want ({rows},)")
    out = np.empty((rows, cols), dtype=np.float32)
    _native.call(_LIN_OP_DEQUANTIZE_INT8, [out.ctypes.data, Q.ctypes.data, E.ctypes.data], [rows, cols])
    return out


def _int8_operand(x, name):
    """`_lin_int8_operand` (door :604-620): a (codes, exponents) pair, or a float32 matrix
    quantized by `quantize_int8`'s rule."""
    if type(x) is tuple and len(x) == 2:
        Q = _typed(x[0], np.int8, 2, name + " codes")
        E = _typed(x[1], np.int32, 1, name + " exponents")
        if E.shape[0] != Q.shape[0]:
            raise ValueError(f"mojolearn.linalg.matmul_int8: {name} exponents has shape {_shape_text(E.shape)}, "
                             f"want ({Q.shape[0]},)")
        return Q, E
    return _quantize(_operand(x, name))


def matmul_int8(a, b, *, out=None):
    """``a @ b.T`` with int8 operands under ``mojolearn.identical.gemm.int8i32.v1`` (OP_NT only).

    Each of `a` (m, k) and `b` (n, k) is a float32 matrix, quantized by `quantize_int8`'s
    rule, or a ``(codes, exponents)`` pair.  ``C[i, j] = ftz(f32(sum_p qa[i, p] qb[j, p]) *
    2**(ea[i] + eb[j]))``: the exact Int32 sum, converted by the contract's pinned split
    (L-5), scaled once.  It is the product of the rounded operands, not the float32
    product.  python/mojolearn/_linalg_impl.py:360-369, door :623-650.
    """
    require_identical()
    qa, ea = _int8_operand(a, "a")
    qb, eb = _int8_operand(b, "b")
    m, k = qa.shape
    n, kb = qb.shape
    if k != kb:
        raise ValueError(f"mojolearn.linalg.matmul_int8: contracted extents differ, a gives k={k} and b gives k={kb}")
    C = _out(out, m, n, "matmul_int8")
    _native.call(_LIN_OP_GEMM_INT8, [C.ctypes.data, qa.ctypes.data, ea.ctypes.data, qb.ctypes.data, eb.ctypes.data],
                 [m, n, k])
    return C


def from_f16(bits):
    """IEEE float16 bits (a uint16 buffer, or a float16 array read as its bits) to float32,
    exact: a subnormal float16 becomes a normal float32, every NaN keeps its sign and payload.
    Any shape.  python/mojolearn/_linalg_impl.py:322-326, door :552-562."""
    require_identical()
    v = _asarray(bits)
    if v.dtype == np.float16:
        v = v.view(np.uint16)
    if v.dtype.kind not in "biuf":
        raise TypeError(f"mojolearn: bits has buffer format '{v.dtype.str}', which is not a numeric array")
    v = np.ascontiguousarray(v, dtype=np.uint16)
    if v.size == 0:
        raise ValueError("mojolearn.linalg.from_f16: bits has no elements")
    out = np.empty(v.shape, dtype=np.float32)
    _native.call(_LIN_OP_FROM_F16, [out.ctypes.data, v.ctypes.data], [v.size])
    return out


def _int15_version():
    """`_int15_binding` (bindings/linalg_ops_lowbit_door.mojo:231-248): the loaded binary's
    fifteen-bit profile version, which must be this module's."""
    version = _native.call(_LIN_OP_INT15_VERSION, [], [])
    if version != INT15_PROFILE_VERSION:
        raise RuntimeError(f"mojolearn.linalg: the loaded extension implements fifteen-bit profile version "
                           f"{version}, this module expects {INT15_PROFILE_VERSION} ({PROFILE_INT15})")


def _quantize15(A):
    """`lin_quantize_int15` (door :713-729) of an admitted operand: (hi, lo, exponents)."""
    rows, cols = A.shape
    hi = np.empty((rows, cols), dtype=np.int8)
    lo = np.empty((rows, cols), dtype=np.int8)
    exps = np.empty((rows,), dtype=np.int32)
    _native.call(_LIN_OP_QUANTIZE_INT15, [hi.ctypes.data, lo.ctypes.data, exps.ctypes.data, A.ctypes.data],
                 [rows, cols])
    return hi, lo, exps


def quantize_int15(x):
    """Quantize a 2-D float32 matrix to fifteen-bit codes stored as two int8 planes
    (profile ``mojolearn.identical.gemm.int15i64.v1``, contract W-1..W-3).

    Per row ``e = floor(log2(absmax)) - 13``; each code is
    ``clamp(round_half_even(x * 2**-e), -16383, 16383)`` (a NaN codes to 0), split as
    ``hi = code >> 7`` and ``lo = code & 127`` so ``code = hi * 128 + lo``.  Returns
    ``(hi, lo, exponents)``.  python/mojolearn/_linalg_impl.py:381-395.
    """
    require_identical()
    _int15_version()
    return _quantize15(_operand(x, "x"))


def _int15_planes(x, name, who):
    """`_lin_int15_planes` (door :739-749)."""
    H = _typed(x[0], np.int8, 2, name + " hi")
    L = _typed(x[1], np.int8, 2, name + " lo")
    E = _typed(x[2], np.int32, 1, name + " exponents")
    if L.shape != H.shape:
        raise ValueError(f"mojolearn.linalg.{who}: {name} lo has shape {_shape_text(L.shape)}, "
                         f"hi has {_shape_text(H.shape)}")
    if E.shape[0] != H.shape[0]:
        raise ValueError(f"mojolearn.linalg.{who}: {name} exponents has shape {_shape_text(E.shape)}, "
                         f"want ({H.shape[0]},)")
    return H, L, E


def dequantize_int15(hi, lo, exponents):
    """float32 ``(hi * 128 + lo) * 2**exponents[row]`` (contract W-6, W-7) from `quantize_int15`
    output.  door :752-774."""
    require_identical()
    _int15_version()
    H, L, E = _int15_planes((hi, lo, exponents), "operand", "dequantize_int15")
    rows, cols = H.shape
    out = np.empty((rows, cols), dtype=np.float32)
    _native.call(_LIN_OP_DEQUANTIZE_INT15, [out.ctypes.data, H.ctypes.data, L.ctypes.data, E.ctypes.data],
                 [rows, cols])
    return out


def _int15_operand(x, name):
    """`_lin_int15_operand` (door :777-792): a (hi, lo, exponents) triple, or a float32 matrix
    quantized by `quantize_int15`'s rule."""
    if type(x) is tuple and len(x) == 3:
        return _int15_planes(x, name, "matmul_int15")
    if type(x) is tuple:
        raise TypeError(f"mojolearn.linalg.matmul_int15: {name} is a tuple of {len(x)}; a fifteen-bit operand "
                        "is (hi, lo, exponents) from quantize_int15, or a float32 matrix")
    return _quantize15(_operand(x, name))


def matmul_int15(a, b, *, out=None):
    """``a @ b.T`` with fifteen-bit operands under ``mojolearn.identical.gemm.int15i64.v1`` (OP_NT).

    Each of `a` (m, k) and `b` (n, k) is a float32 matrix, quantized by `quantize_int15`'s
    rule, or a ``(hi, lo, exponents)`` triple.  The exact integer sum of the code products,
    rounded to nearest even (W-6), scaled by ``2**(ea[i] + eb[j])``.  `k` may be at most
    65536 (`INT15_MAX_K`); larger values raise ValueError.  python/mojolearn/_linalg_impl.py:404-417,
    door :795-840.
    """
    require_identical()
    _int15_version()
    ah, al, ea = _int15_operand(a, "a")
    bh, bl, eb = _int15_operand(b, "b")
    m, k = ah.shape
    n, kb = bh.shape
    if k != kb:
        raise ValueError(f"mojolearn.linalg.matmul_int15: contracted extents differ, a gives k={k} and b gives k={kb}")
    if k > INT15_MAX_K:
        raise ValueError(f"mojolearn.linalg.matmul_int15: k={k} is above {INT15_MAX_K}, the largest contracted "
                         f"extent {PROFILE_INT15} accepts (contract W-4)")
    C = _out(out, m, n, "matmul_int15")
    _native.call(_LIN_OP_GEMM_INT15, [C.ctypes.data, ah.ctypes.data, al.ctypes.data, ea.ctypes.data,
                                      bh.ctypes.data, bl.ctypes.data, eb.ctypes.data], [m, n, k])
    return C


def linear(x, w, bias, *, transpose_b=False, out=None):
    """``Y = ftz(ftz(x @ w) + ftz(bias[j]))``: the product, then the LM's nn.Linear bias
    (transformer/impl/llama/modeling_llama.mojo:3979-3989), fused into the store."""
    require_identical()
    A = _operand(x, "x")
    B = _operand(w, "w")
    op, m, n, k = _op_and_shape(A, B, False, transpose_b, "linear")
    bv = np.ascontiguousarray(_asarray(bias))
    if bv.dtype != np.float32:
        raise TypeError(f"mojolearn.linalg.linear: bias has dtype {bv.dtype}, want float32")
    if bv.size != n:
        raise ValueError(f"mojolearn.linalg.linear: bias must hold n={n} values")
    C = _out(out, m, n, "linear")
    _native.call(_LIN_OP_GEMM_BIAS, [C.ctypes.data, A.ctypes.data, B.ctypes.data, bv.ctypes.data], [m, n, k, op])
    return C


__all__ = ["matmul", "matmul_bf16", "matmul_int8", "matmul_int8w", "linear", "to_bf16", "from_bf16",
           "from_f16", "quantize_int8", "dequantize_int8", "matmul_int15", "quantize_int15", "dequantize_int15",
           "numeric_mode", "profile", "require_identical", "PROFILE", "PROFILE_FAMILY", "PROFILE_VERSION",
           "PROFILE_BF16", "PROFILE_INT8", "PROFILE_INT15", "PROFILE_INT8W", "INT8_MAX_K", "INT15_MAX_K",
           "OP_NN", "OP_NT", "OP_TN"]
