"""Device-resident entry points on PyTorch-ROCm tensors (torch is plumbing: device memory
and streams).  These are the model-code entries -- the role of the reference's
identical_gemm_into / GemmWorkspace.run (gemm/checks/gemm_identical.mojo:6062-6144,
gemm/neural_dispatch.mojo:468-478) -- enqueued on the current torch stream, no copies.
"""
import torch

from . import _native

OP_NN, OP_NT, OP_TN = 0, 1, 2


def _shape(a, b, op):
    if op == OP_NN:
        (m, k), (kb, n) = a.shape, b.shape
    elif op == OP_NT:
        (m, k), (n, kb) = a.shape, b.shape
    elif op == OP_TN:
        (k, m), (kb, n) = a.shape, b.shape
    else:
        raise ValueError(f"op must be 0 (OP_NN), 1 (OP_NT) or 2 (OP_TN), got {op}")
    if k != kb:
        raise ValueError(f"contracted extents differ: a gives k={k}, b gives k={kb}")
    return m, n, k


def _check(t, name, dtype):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, want {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _stream(t):
    return ctypes_stream(torch.cuda.current_stream(t.device))


def ctypes_stream(s):
    return s.cuda_stream


def _prep_out(out, m, n, ref):
    if out is None:
        return torch.empty((m, n), dtype=torch.float32, device=ref.device)
    _check(out, "out", torch.float32)
    if tuple(out.shape) != (m, n):
        raise ValueError(f"out has shape {tuple(out.shape)}, want ({m}, {n})")
    return out


def _bias(bias, n):
    if bias is None:
        return None
    _check(bias, "bias", torch.float32)
    if bias.numel() != n:
        raise ValueError(f"bias must hold n={n} values")
    return bias.data_ptr()


def gemm(a, b, *, op=OP_NN, bias=None, out=None, leaf=0):
    """C = op(a) . op(b) (fp32.v1), optional fused nn.Linear bias.  float32 tensors."""
    _check(a, "a", torch.float32)
    _check(b, "b", torch.float32)
    m, n, k = _shape(a, b, op)
    c = _prep_out(out, m, n, a)
    with torch.cuda.device(a.device):
        _native.check(_native.lib().mlg_gemm_f32(c.data_ptr(), a.data_ptr(), b.data_ptr(), _bias(bias, n),
                                                 m, n, k, op, leaf, _stream(a)))
    return c


def gemm_bf16w(a, b_bits, *, op=OP_NN, bias=None, out=None, leaf=0):
    """C = op(a) . op(widen(b_bits)); b_bits is a torch.int16/uint16 tensor of bf16 bits
    (a may be float32 or bf16 bits too)."""
    if b_bits.dtype not in (torch.int16, torch.uint16):
        raise TypeError("b_bits must hold bf16 bits as int16/uint16")
    a_bits = a.dtype in (torch.int16, torch.uint16)
    if not a_bits:
        _check(a, "a", torch.float32)
    m, n, k = _shape(a, b_bits, op)
    c = _prep_out(out, m, n, a)
    with torch.cuda.device(a.device):
        _native.check(_native.lib().mlg_gemm_bf16w(c.data_ptr(), a.data_ptr(), b_bits.data_ptr(), _bias(bias, n),
                                                   m, n, k, op, 1 if a_bits else 0, leaf, _stream(a)))
    return c


def gemm_int8w(a, codes, scales, *, op=OP_NN, bias=None, out=None, leaf=0):
    """C = op(a) . W, W[p, j] = ftz(f32(codes[p, j]) * ftz(scales[j])) (int8 codes, one
    float32 scale per output column)."""
    _check(a, "a", torch.float32)
    _check(codes, "codes", torch.int8)
    _check(scales, "scales", torch.float32)
    m, n, k = _shape(a, codes, op)
    if scales.numel() != n:
        raise ValueError(f"scales must hold n={n} values")
    c = _prep_out(out, m, n, a)
    with torch.cuda.device(a.device):
        _native.check(_native.lib().mlg_gemm_int8w(c.data_ptr(), a.data_ptr(), codes.data_ptr(), scales.data_ptr(),
                                                   _bias(bias, n), m, n, k, op, leaf, _stream(a)))
    return c


def bf16_widen(bits):
    out = torch.empty(bits.shape, dtype=torch.float32, device=bits.device)
    with torch.cuda.device(bits.device):
        _native.check(_native.lib().mlg_bf16_widen(out.data_ptr(), bits.data_ptr(), bits.numel(), _stream(bits)))
    return out


def bf16_narrow(x):
    _check(x, "x", torch.float32)
    out = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    with torch.cuda.device(x.device):
        _native.check(_native.lib().mlg_bf16_narrow(out.data_ptr(), x.data_ptr(), x.numel(), _stream(x)))
    return out


def int8_quantize(x):
    """(codes int8, exponents int32) of a float32 (rows, cols) tensor, profile int8i32.v1
    (the reference's quantize_rows_int8_device, gemm/linalg_native.mojo:323-357)."""
    _check(x, "x", torch.float32)
    if x.dim() != 2 or x.numel() == 0:
        raise ValueError("x must be 2-D and non-empty")
    rows, cols = x.shape
    codes = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    exps = torch.empty((rows,), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        _native.check(_native.lib().mlg_int8_quantize(codes.data_ptr(), exps.data_ptr(), x.data_ptr(), rows, cols,
                                                      _stream(x)))
    return codes, exps


def int8_dequantize(codes, exps):
    """float32 ftz(code * 2^exps[row]) (dequantize_rows_int8_device, :359-393)."""
    _check(codes, "codes", torch.int8)
    _check(exps, "exponents", torch.int32)
    if codes.dim() != 2 or codes.numel() == 0 or exps.numel() != codes.shape[0]:
        raise ValueError("codes must be 2-D and non-empty with one exponent per row")
    rows, cols = codes.shape
    out = torch.empty((rows, cols), dtype=torch.float32, device=codes.device)
    with torch.cuda.device(codes.device):
        _native.check(_native.lib().mlg_int8_dequantize(out.data_ptr(), codes.data_ptr(), exps.data_ptr(), rows,
                                                        cols, _stream(codes)))
    return out


def gemm_int8i32(qa, ea, qb, eb, *, out=None):
    """C = qa . qb^T scaled by 2^(ea[i] + eb[j]) (profile int8i32.v1, OP_NT; the reference's
    identical_gemm_int8_into, gemm/linalg_native.mojo:258-321)."""
    _check(qa, "qa", torch.int8)
    _check(qb, "qb", torch.int8)
    _check(ea, "ea", torch.int32)
    _check(eb, "eb", torch.int32)
    m, n, k = _shape(qa, qb, OP_NT)
    if ea.numel() != m or eb.numel() != n:
        raise ValueError("one exponent per row of each operand is required")
    c = _prep_out(out, m, n, qa)
    with torch.cuda.device(qa.device):
        _native.check(_native.lib().mlg_gemm_int8i32(c.data_ptr(), qa.data_ptr(), ea.data_ptr(), qb.data_ptr(),
                                                     eb.data_ptr(), m, n, k, _stream(qa)))
    return c


def f16_widen(bits):
    """float32 of float16 bits (int16/uint16/float16 tensor), exact (gemm/f16_widen.mojo:12-37)."""
    if bits.dtype not in (torch.int16, torch.uint16, torch.float16):
        raise TypeError("bits must hold float16 bits as int16/uint16/float16")
    out = torch.empty(bits.shape, dtype=torch.float32, device=bits.device)
    with torch.cuda.device(bits.device):
        _native.check(_native.lib().mlg_f16_widen(out.data_ptr(), bits.data_ptr(), bits.numel(), _stream(bits)))
    return out


def int15_quantize(x):
    """(hi int8, lo int8, exponents int32) of a float32 (rows, cols) tensor, profile int15i64.v1."""
    _check(x, "x", torch.float32)
    if x.dim() != 2 or x.numel() == 0:
        raise ValueError("x must be 2-D and non-empty")
    rows, cols = x.shape
    hi = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    lo = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    exps = torch.empty((rows,), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        _native.check(_native.lib().mlg_int15_quantize(hi.data_ptr(), lo.data_ptr(), exps.data_ptr(), x.data_ptr(),
                                                       rows, cols, _stream(x)))
    return hi, lo, exps


def int15_dequantize(hi, lo, exps):
    """float32 ftz((hi * 128 + lo) * 2^exps[row])."""
    _check(hi, "hi", torch.int8)
    _check(lo, "lo", torch.int8)
    _check(exps, "exponents", torch.int32)
    if hi.dim() != 2 or hi.numel() == 0 or lo.shape != hi.shape or exps.numel() != hi.shape[0]:
        raise ValueError("hi and lo must be 2-D, non-empty and alike, with one exponent per row")
    rows, cols = hi.shape
    out = torch.empty((rows, cols), dtype=torch.float32, device=hi.device)
    with torch.cuda.device(hi.device):
        _native.check(_native.lib().mlg_int15_dequantize(out.data_ptr(), hi.data_ptr(), lo.data_ptr(), exps.data_ptr(),
                                                         rows, cols, _stream(hi)))
    return out


def gemm_int15i64(ah, al, ea, bh, bl, eb, *, out=None):
    """C = a . b^T of fifteen-bit operands given as planes (profile int15i64.v1, OP_NT)."""
    for t, name in ((ah, "ah"), (al, "al"), (bh, "bh"), (bl, "bl")):
        _check(t, name, torch.int8)
    _check(ea, "ea", torch.int32)
    _check(eb, "eb", torch.int32)
    m, n, k = _shape(ah, bh, OP_NT)
    if al.shape != ah.shape or bl.shape != bh.shape or ea.numel() != m or eb.numel() != n:
        raise ValueError("planes of one operand must agree, with one exponent per row")
    c = _prep_out(out, m, n, ah)
    with torch.cuda.device(ah.device):
        _native.check(_native.lib().mlg_gemm_int15i64(c.data_ptr(), ah.data_ptr(), al.data_ptr(), ea.data_ptr(),
                                                      bh.data_ptr(), bl.data_ptr(), eb.data_ptr(), m, n, k,
                                                      _stream(ah)))
    return c


T_F32, T_BF16, T_I8 = 0, 1, 2


def workspace_bytes(m, n, k, *, op=OP_NN, a_type=T_F32, b_type=T_F32, leaf=0, a=None, b=None):
    """Workspace bytes `gemm_ws` needs for this product on the current device (for the
    operands `a`, `b` when given: a misaligned operand is repacked into the workspace)."""
    pa = a.data_ptr() if a is not None else None
    pb = b.data_ptr() if b is not None else None
    nb = _native.lib().mlg_gemm_workspace_bytes_for(pa, pb, m, n, k, op, a_type, b_type, leaf)
    if nb < 0:
        _native.check(1)
    return nb


#: Bits of `route` (include/mlgemm.h mlg_gemm_route).
ROUTES = {"tile": 1, "fold": 2, "gemv_nn": 4, "gemv_nt": 8, "mfma4": 16, "mfma16": 32, "tail_split": 64,
          "repack": 128, "zero_k": 256, "tile_stack": 512, "gemv_groups": 1024}


def route(m, n, k, *, op=OP_NN, a_type=T_F32, b_type=T_F32, leaf=0, a=None, b=None, num_cus=0):
    """The set of kernel names this product dispatches to (no launch).  With `num_cus` > 0 no
    device is needed; `a`/`b` (tensors or integer addresses) decide the operands' alignment."""
    addr = lambda t: None if t is None else (t if isinstance(t, int) else t.data_ptr())  # noqa: E731
    r = _native.lib().mlg_gemm_route(addr(a), addr(b), m, n, k, op, a_type, b_type, leaf, num_cus)
    if r < 0:
        _native.check(1)
    return {name for name, bit in ROUTES.items() if r & bit}


class Plan:
    """One product's arguments bound once (shapes checked, workspace allocated for these
    operands and zeroed), so that a call is a single C entry with no allocation and no
    synchronization -- capturable in a HIP graph.

    a: float32 (or bf16 bits with b_type=T_BF16), b: float32 / bf16 bits / int8 codes.
    """

    def __init__(self, a, b, *, op=OP_NN, scales=None, bias=None, out=None, leaf=0, b_type=None):
        if b_type is None:
            b_type = {torch.float32: T_F32, torch.int16: T_BF16, torch.uint16: T_BF16, torch.int8: T_I8}[b.dtype]
        a_type = T_BF16 if a.dtype in (torch.int16, torch.uint16) else T_F32
        if a_type == T_F32:
            _check(a, "a", torch.float32)
        m, n, k = _shape(a, b, op)
        if b_type == T_I8:
            _check(scales, "scales", torch.float32)
            if scales.numel() != n:
                raise ValueError(f"scales must hold n={n} values")
        self.out = _prep_out(out, m, n, a)
        nb = workspace_bytes(m, n, k, op=op, a_type=a_type, b_type=b_type, leaf=leaf, a=a, b=b)
        # zeroed once: its completion counters start at zero and every call leaves them so
        self.ws = torch.zeros(max(nb, 4), dtype=torch.uint8, device=a.device)
        self.args = (self.out.data_ptr(), a.data_ptr(), b.data_ptr(),
                     scales.data_ptr() if scales is not None else None, _bias(bias, n), m, n, k, op, a_type, b_type,
                     leaf, self.ws.data_ptr(), nb)
        self._keep = (a, b, scales, bias)
        self._fn = _native.lib().mlg_gemm_ws

    def __call__(self, stream=None):
        s = stream.cuda_stream if stream is not None else torch.cuda.current_stream().cuda_stream
        rc = self._fn(*self.args, s)
        if rc:
            _native.check(rc)
        return self.out


# ---- decode-packed int8 weights (mlg_int8w_pack / mlg_gemv_int8w_packed)

class PackedInt8W:
    """int8 codes[k][n] rearranged once for the decode GEMV: `data` is a 1-D uint8 device tensor
    of mlg_int8w_packed_bytes(k, n) bytes; `k` and `n` are the codes' shape."""

    def __init__(self, data, k, n):
        self.data, self.k, self.n = data, int(k), int(n)

    def __repr__(self):
        return f"PackedInt8W(k={self.k}, n={self.n}, bytes={self.data.numel()})"


def pack_int8w(codes):
    """The decode-packed copy of int8 codes[k][n] (k a positive multiple of 128, at most 1024
    leaves of 128), written on the current stream."""
    _check(codes, "codes", torch.int8)
    if codes.dim() != 2:
        raise ValueError("codes must be 2-D [k, n]")
    k, n = codes.shape
    nb = _native.lib().mlg_int8w_packed_bytes(k, n)
    if nb < 0:
        raise ValueError(f"the decode-packed layout takes k a positive multiple of 128 (at most 1024 leaves), got k={k}")
    data = torch.empty(nb, dtype=torch.uint8, device=codes.device)
    with torch.cuda.device(codes.device):
        _native.check(_native.lib().mlg_int8w_pack(data.data_ptr(), codes.data_ptr(), k, n, _stream(codes)))
    return PackedInt8W(data, k, n)


def _packed_args(x, packed, scales):
    _check(x, "x", torch.float32)
    if not isinstance(packed, PackedInt8W):
        raise TypeError("packed must be a PackedInt8W (from pack_int8w)")
    _check(scales, "scales", torch.float32)
    if x.dim() != 2 or x.shape[1] != packed.k:
        raise ValueError(f"x must be [m, {packed.k}], got {tuple(x.shape)}")
    if scales.numel() != packed.n:
        raise ValueError(f"scales must hold n={packed.n} values")
    m = x.shape[0]
    nb = _native.lib().mlg_gemv_int8w_packed_workspace_bytes(m, packed.n, packed.k)
    if nb < 0:
        raise ValueError(f"the packed decode product takes 1 <= m <= 16, got m={m}")
    return m, nb


def gemv_int8w_packed(x, packed, scales, *, bias=None, out=None):
    """C = x . W_deq (+ bias) from decode-packed weights, 1 <= m <= 16: the bits of
    gemm_int8w(x, codes, scales, bias=bias) on the row-major codes."""
    m, nb = _packed_args(x, packed, scales)
    c = _prep_out(out, m, packed.n, x)
    ws = torch.zeros(max(nb, 4), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        _native.check(_native.lib().mlg_gemv_int8w_packed(c.data_ptr(), x.data_ptr(), packed.data.data_ptr(),
                                                          scales.data_ptr(), _bias(bias, packed.n), m, packed.n,
                                                          packed.k, ws.data_ptr(), nb, _stream(x)))
    return c


class PackedPlan:
    """gemv_int8w_packed's arguments bound once (workspace allocated and zeroed), so that a call
    is a single C entry with no allocation and no synchronization -- capturable in a HIP graph."""

    def __init__(self, x, packed, scales, *, bias=None, out=None):
        m, nb = _packed_args(x, packed, scales)
        self.out = _prep_out(out, m, packed.n, x)
        self.ws = torch.zeros(max(nb, 4), dtype=torch.uint8, device=x.device)
        self.args = (self.out.data_ptr(), x.data_ptr(), packed.data.data_ptr(), scales.data_ptr(),
                     _bias(bias, packed.n), m, packed.n, packed.k, self.ws.data_ptr(), nb)
        self._keep = (x, packed, scales, bias)
        self._fn = _native.lib().mlg_gemv_int8w_packed

    def __call__(self, stream=None):
        s = stream.cuda_stream if stream is not None else torch.cuda.current_stream().cuda_stream
        rc = self._fn(*self.args, s)
        if rc:
            _native.check(rc)
        return self.out


# ---- caller-partition and sequence-executor words on strided views

EPI_NONE, EPI_PLUS_BIAS, EPI_BIAS_ACT, EPI_ACT_BWD = 0, 3, 4, 5
ACT_IDENTITY, ACT_LOGISTIC, ACT_TANH, ACT_RELU, ACT_SOFTMAX = 0, 1, 2, 3, 4


def _view(t, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} has dtype {t.dtype}, want torch.float32")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    return t.stride()


def _views(a, b):
    a_si, a_sp = _view(a, "a")
    b_sp, b_sj = _view(b, "b")
    (m, k), (kb, n) = a.shape, b.shape
    if k != kb:
        raise ValueError(f"contracted extents differ: a gives k={k}, b gives k={kb}")
    return m, n, k, a_si, a_sp, b_sp, b_sj


def _epi_buffer(epi, epi_p, m, n):
    if epi == EPI_NONE:
        return None
    _check(epi_p, "epi_p", torch.float32)
    need = m * n if epi == EPI_ACT_BWD else n
    if epi_p.numel() != need:
        raise ValueError(f"epi_p must hold {need} values for epilogue kind {epi}")
    return epi_p.data_ptr()


def gemm_leaf_ptr(a, b, *, leaf, p_count, out=None, epi=EPI_NONE, epi_p=None, act=ACT_IDENTITY):
    """identical_gemm_leaf_ptr_into / _epi_into (gemm/neural_dispatch.mojo:245-397): C = A_eff . B_eff
    with the caller's partition (leaf, p_count) of k, `a` an (m, k) and `b` a (k, n) view of any
    strides; optional follower `epi` (3 bias, 4 bias + activation `act`, 5 activation derivative
    at `epi_p`, dense (m, n))."""
    m, n, k, a_si, a_sp, b_sp, b_sj = _views(a, b)
    c = _prep_out(out, m, n, a)
    p = _epi_buffer(epi, epi_p, m, n)
    L = _native.lib()
    with torch.cuda.device(a.device):
        if epi == EPI_NONE:
            rc = L.mlg_gemm_leaf_ptr(c.data_ptr(), a.data_ptr(), b.data_ptr(), m, n, k, leaf, p_count,
                                     a_si, a_sp, b_sp, b_sj, _stream(a))
        else:
            rc = L.mlg_gemm_leaf_ptr_epi(c.data_ptr(), a.data_ptr(), b.data_ptr(), m, n, k, leaf, p_count,
                                         a_si, a_sp, b_sp, b_sj, epi, p, act, _stream(a))
        _native.check(rc)
    return c


def seq_gemm(a, b, c, *, accumulate=False):
    """op_gemm (sequence/ops.mojo:518-531) in place on `c`, an (m, n) view with unit column
    stride: one ascending chain over the whole of k per cell, from ftz(old C) when
    `accumulate`, else +0."""
    m, n, k, a_si, a_sp, b_sp, b_sj = _views(a, b)
    ldc, c_sj = _view(c, "c")
    if tuple(c.shape) != (m, n) or (c_sj != 1 and n > 1):
        raise ValueError(f"c must be an ({m}, {n}) view with unit column stride")
    with torch.cuda.device(a.device):
        _native.check(_native.lib().mlg_seq_gemm(c.data_ptr(), a.data_ptr(), b.data_ptr(), m, n, k, a_si, a_sp,
                                                 b_sp, b_sj, ldc, 1 if accumulate else 0, _stream(a)))
    return c


def follow(c, epi, epi_p=None, act=ACT_IDENTITY):
    """The followers alone over the cells of `c` (an (m, n) view, unit column stride)."""
    ldc, c_sj = _view(c, "c")
    m, n = c.shape
    if c_sj != 1 and n > 1:
        raise ValueError("c must have unit column stride")
    p = _epi_buffer(epi, epi_p, m, n)
    with torch.cuda.device(c.device):
        _native.check(_native.lib().mlg_follow(c.data_ptr(), ldc, m, n, epi, p, act, _stream(c)))
    return c
