"""Low-bit weight storage with float32 arithmetic: the surface of `mojolearn.lowbit`
(python/mojolearn/lowbit.py:1-186, behaviour of providers/python/lowbit_weight_pyapi_door.mojo).

A 2-D weight can be stored as bfloat16 bits (`BF16Weight`, contract L-2, widened by L-1) or as
int8 codes with one power-of-two exponent per row (`Int8Weight`, L-3/L-4, dequantized by L-6).
Materializing converts back to float32 exactly, so a model built from packed weights computes the
float32 path on the rounded weights.  Every conversion goes through this build's linalg op table
(to_bf16, from_bf16, quantize_int8, dequantize_int8) on the GPU; there is no host fallback.
"""
import numpy as np

from . import linalg as _linalg

FORMATS = ("float32", "bfloat16", "int8")

__all__ = ["FORMATS", "BF16Weight", "Int8Weight", "pack", "unpack", "materialize", "format_of", "is_packed",
           "pack_one", "materialize_one", "widen_bf16"]


def _shape_text(shape):
    return "(" + ", ".join(str(int(s)) for s in shape) + ("," if len(shape) == 1 else "") + ")"


def _empty(name, shape):
    """`low_empty` (bindings/lowbit_weight_run.mojo:9-13)."""
    what = "feature(s)" if len(shape) == 2 and shape[0] != 0 else "sample(s)"
    text = _shape_text(shape)
    raise ValueError(f"mojolearn: {name} is empty, shape {text}: Found array with 0 {what} (shape={text}) "
                     "while a minimum of 1 is required.")


def _admit(value, dtype, rank, name):
    """`low_admit` (lowbit_weight_pyapi_door.mojo:82-98): the exact dtype and rank, else TypeError."""
    v = np.asarray(value)
    ok = v.dtype == dtype and (rank < 0 or v.ndim == rank)
    if not ok:
        if dtype == np.uint16:
            raise TypeError("mojolearn.lowbit.BF16Weight: bits must be a 2-D uint16 array")
        if dtype == np.int8:
            raise TypeError("mojolearn.lowbit.Int8Weight: codes must be a 2-D int8 array")
        raise TypeError("mojolearn.lowbit.Int8Weight: exponents must be int32 of shape (rows,)")
    if v.size == 0:
        _empty(name, v.shape)
    return np.ascontiguousarray(v)


def _exponents(value, rows):
    e = _admit(value, np.int32, 1, "exponents")
    if e.shape[0] != rows:
        raise TypeError("mojolearn.lowbit.Int8Weight: exponents must be int32 of shape (rows,)")
    return e


class BF16Weight:
    """A 2-D weight stored as bfloat16 bits (a 2-D uint16 buffer, e.g. from `linalg.to_bf16`).

    Attributes: ``bits`` (uint16), ``shape``, ``format = 'bfloat16'``.
    """

    format = "bfloat16"

    def __init__(self, bits):
        self.bits = _admit(bits, np.uint16, 2, "bits")
        self.shape = tuple(int(s) for s in self.bits.shape)

    def __repr__(self):
        return f"BF16Weight(shape={self.shape!r})"


class Int8Weight:
    """A 2-D weight stored as int8 codes with one int32 exponent per row:
    ``row = codes * 2**exponent``.  Attributes: ``codes``, ``exponents``, ``shape``,
    ``format = 'int8'``."""

    format = "int8"

    def __init__(self, codes, exponents):
        self.codes = _admit(codes, np.int8, 2, "codes")
        self.exponents = _exponents(exponents, self.codes.shape[0])
        self.shape = tuple(int(s) for s in self.codes.shape)

    def __repr__(self):
        return f"Int8Weight(shape={self.shape!r})"


def _kind(value):
    if type(value) is BF16Weight:
        return 1
    if type(value) is Int8Weight:
        return 2
    return 0


def _format(fmt):
    """`low_format` (door :52-58)."""
    if type(fmt) is not str:
        raise TypeError("mojolearn.lowbit: format must be an exact string")
    if fmt not in FORMATS:
        raise ValueError(f"mojolearn.lowbit: unknown format '{fmt}'; one of ('float32', 'bfloat16', 'int8')")
    return fmt


def _name(name):
    if type(name) is not str:
        raise TypeError("mojolearn.lowbit: tensor names must be exact strings")
    return name


def is_packed(value):
    """Whether `value` is a packed weight (`BF16Weight` or `Int8Weight`)."""
    return _kind(value) != 0


def _values(weights):
    if type(weights) is dict:
        return list(weights.values())
    if type(weights) in (list, tuple):
        return weights
    raise TypeError("mojolearn.lowbit: use a native dict, list or tuple; Python iteration hooks are not supported")


def format_of(weights):
    """The format shared by the packed tensors of `weights` (a dict, list or tuple), or
    ``'float32'`` when none is packed.  Raises ValueError when they mix formats
    (`low_formats`, door :159-170)."""
    kind = 0
    for v in _values(weights):
        cur = _kind(v)
        if cur:
            if kind and cur != kind:
                raise ValueError("mojolearn.lowbit: weights mix formats ['bfloat16', 'int8']; store a model one way")
            kind = cur
    return ("float32", "bfloat16", "int8")[kind]


def widen_bf16(bits):
    """bfloat16 bits of any rank (converted to uint16 by astype's rules) to float32, exactly."""
    v = np.asarray(bits)
    if v.dtype.kind not in "biuf":
        raise TypeError(f"mojolearn: bits has buffer format '{v.dtype.str}', which is not a numeric array")
    v = np.ascontiguousarray(v, dtype=np.uint16)
    if v.size == 0:
        raise ValueError("mojolearn.linalg.from_bf16: bits has no elements")
    return _linalg.from_bf16(v.reshape(-1)).reshape(v.shape)


def materialize_one(value, name="weight"):
    """A packed tensor converted to float32 exactly (`low_materialize`, door :108-125), or any
    other value returned as is."""
    kind = _kind(value)
    if kind == 0:
        return value
    if kind == 1:
        q = _admit(value.bits, np.uint16, 2, name)
        return _linalg.from_bf16(q)
    q = _admit(value.codes, np.int8, 2, name)
    e = _exponents(value.exponents, q.shape[0])
    return _linalg.dequantize_int8(q, e)


def _pack_admitted(v, fmt, name):
    """`low_pack_admitted` (door :128-152)."""
    if v.dtype != np.float32:
        raise TypeError(f"mojolearn.lowbit: {name} has dtype {v.dtype}; pack takes float32")
    if v.ndim != 2:
        raise ValueError(f"mojolearn.lowbit: {name} must be 2-D to pack, got shape {_shape_text(v.shape)}")
    if v.size == 0:
        _empty(name, v.shape)
    a = np.array(v, dtype=np.float32, order="C", copy=True) if fmt == "float32" else np.ascontiguousarray(v)
    if fmt == "float32":
        return a
    if fmt == "bfloat16":
        w = BF16Weight.__new__(BF16Weight)
        w.bits = _linalg.to_bf16(a)
        w.shape = tuple(int(s) for s in a.shape)
        return w
    codes, exps = _linalg.quantize_int8(a)
    w = Int8Weight.__new__(Int8Weight)
    w.codes, w.exponents = codes, exps
    w.shape = tuple(int(s) for s in a.shape)
    return w


def pack_one(value, fmt, name="weight"):
    """Pack one 2-D float32 tensor to `fmt` ('float32' returns a float32 copy); unknown formats and
    non-2-D tensors raise ValueError."""
    fmt = _format(fmt)
    name = _name(name)
    return _pack_admitted(np.asarray(value), fmt, name)


def pack(weights, fmt):
    """Pack every 2-D tensor of a weight dict to `fmt`; other tensors pass through unchanged.
    A tensor already packed in `fmt` is copied, never re-rounded (door :246-300)."""
    fmt = _format(fmt)
    if type(weights) is not dict:
        raise TypeError("mojolearn.lowbit.pack: weights must be a dict keyed by name; Python mapping hooks are "
                        "not supported")
    out = {}
    for key, value in weights.items():
        name = _name(key)
        kind = _kind(value)
        if (kind == 1 and fmt == "bfloat16") or (kind == 2 and fmt == "int8"):
            if kind == 1:
                out[key] = BF16Weight(np.array(value.bits, copy=True))
            else:
                out[key] = Int8Weight(np.array(value.codes, copy=True), np.array(value.exponents, copy=True))
            continue
        if kind:
            value = materialize_one(value, name)
        if type(value) in (list, tuple):
            value = np.asarray(value, dtype=np.float32)
        v = np.asarray(value)
        out[key] = _pack_admitted(v, fmt, name) if fmt != "float32" and v.ndim == 2 else value
    return out


def unpack(weights, what="weights"):
    """Every packed tensor of a weight dict converted to float32 exactly; returns
    ``(dict, format)``.  A value that is not a dict comes back as ``(value, 'float32')``."""
    if type(weights) is not dict:
        return weights, "float32"
    fmt = format_of(weights)
    if fmt == "float32":
        return weights, fmt
    return {k: materialize_one(v, _name(k)) for k, v in weights.items()}, fmt


materialize = unpack
