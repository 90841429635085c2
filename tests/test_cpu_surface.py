"""Host-side checks that need no GPU: the C ABI library loads and exports every symbol
include/mlgemm.h declares, the metadata ops of the op table answer, the error protocol,
the Python surface's refusals (same texts and exception types as the reference door,
bindings/linalg_ops_lowbit_door.mojo:259-416), and the workload generators."""
import ctypes
import os
import re

import numpy as np
import pytest

from mojolearn_amd import _native, linalg
from mojolearn_amd import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "mlgemm.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int64_t|int|const char\*)\s+(\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    L = _native.lib()
    names = _declared()
    assert "linalg_native_v1" in names and "mlg_gemm_f32" in names
    for name in names:
        assert hasattr(L, name), name


def test_stream_read_refuses_before_any_launch():
    """The read-floor entry (bench.py --read-floor) checks its shapes on the host: a missing
    pointer, an unknown pattern, a leaf pattern whose rows are not whole groups of four
    128-row leaves, or a packed pattern whose rows are not whole 32-leaf groups (or whose
    columns are not whole 64-column groups) is refused with a message and launches nothing."""
    L = _native.lib()
    sink = ctypes.c_uint32(0)
    assert L.mlg_stream_read(None, 4096, 14336, 0, ctypes.addressof(sink), None) == 1
    assert b"stream_read" in L.mlg_last_error()
    buf = (ctypes.c_uint8 * 16)()
    assert L.mlg_stream_read(ctypes.addressof(buf), 100, 256, 1, ctypes.addressof(sink), None) == 1
    assert L.mlg_stream_read(ctypes.addressof(buf), 512, 256, 7, ctypes.addressof(sink), None) == 1
    assert L.mlg_stream_read(ctypes.addressof(buf), 2048, 256, 2, ctypes.addressof(sink), None) == 1
    assert L.mlg_stream_read(ctypes.addressof(buf), 4096, 100, 2, ctypes.addressof(sink), None) == 1


def test_int8w_packed_sizes_and_refusals():
    """The decode-packed int8 entries size their buffers on the host (k * 64 * ceil(n / 64)
    packed bytes; a workspace of counters for the 64-column groups, then the roots of 4-leaf
    groups, when there is more than one) and refuse, with a message and before any launch, shapes the layout
    does not take, m past 16, missing buffers, a misaligned packed buffer and a short workspace."""
    L = _native.lib()
    assert L.mlg_int8w_packed_bytes(4096, 14336) == 4096 * 14336
    assert L.mlg_int8w_packed_bytes(4096, 300) == 4096 * 320
    assert L.mlg_int8w_packed_bytes(128, 1) == 128 * 64
    for k, n in ((100, 64), (0, 64), (128, 0), (128 * 1025, 4)):
        assert L.mlg_int8w_packed_bytes(k, n) == -1
    assert L.mlg_gemv_int8w_packed_workspace_bytes(1, 14336, 4096) == (256 + 8 * 14336) * 4
    assert L.mlg_gemv_int8w_packed_counter_bytes(1, 14336, 4096) == 224 * 4
    assert L.mlg_gemv_int8w_packed_workspace_bytes(16, 300, 512) == 0  # 4 leaves: one workgroup
    assert L.mlg_gemv_int8w_packed_workspace_bytes(17, 300, 512) == -1
    assert L.mlg_gemv_int8w_packed_workspace_bytes(1, 300, 500) == -1
    buf = (ctypes.c_uint8 * 64)()
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    assert L.mlg_int8w_pack(base, base, 100, 64, None) == 1
    assert b"mlg_int8w_pack" in L.mlg_last_error()
    assert L.mlg_int8w_pack(None, base, 128, 64, None) == 1
    assert L.mlg_int8w_pack(base + 1, base, 128, 64, None) == 1
    assert b"16-byte" in L.mlg_last_error()
    ok = (base, base, base, base, None, 1, 64, 512)
    assert L.mlg_gemv_int8w_packed(base, base, base, base, None, 17, 64, 512, None, 0, None) == 1
    assert b"m must be" in L.mlg_last_error()
    assert L.mlg_gemv_int8w_packed(base, base, base, base, None, 1, 64, 500, None, 0, None) == 1
    assert L.mlg_gemv_int8w_packed(None, *ok[1:], None, 0, None) == 1
    assert L.mlg_gemv_int8w_packed(base, base, base + 4, base, None, 1, 64, 512, None, 0, None) == 1
    assert b"16-byte" in L.mlg_last_error()
    # 4096 rows are 32 leaves: more than one group, so a workspace is required
    assert L.mlg_gemv_int8w_packed(base, base, base, base, None, 1, 64, 4096, base, 16, None) == 1
    assert b"workspace" in L.mlg_last_error()


def test_metadata_ops():
    assert _native.call(11, [], []) == 1
    assert _native.call(12, [], []) == 1
    assert _native.call(13, [], []) == 1
    assert _native.call(14, [], []) == 1
    assert _native.lib().mlg_abi_name() == b"mojolearn.linalg.v1"
    assert linalg.numeric_mode() == "identical"
    p = linalg.profile()
    assert p["profile"] == "mojolearn.identical.gemm.fp32.v1" and p["identity_claimed"]


def test_capsule_carries_the_one_entry_table():
    """The reference binds its op table as a PyCapsule named "mojolearn.linalg.v1" whose
    pointer is an array of one C function (gemm/linalg_dispatch.mojo:92-102)."""
    cap = _native.capsule()
    get = ctypes.pythonapi.PyCapsule_GetPointer
    get.restype, get.argtypes = ctypes.c_void_p, [ctypes.py_object, ctypes.c_char_p]
    table = ctypes.cast(get(cap, b"mojolearn.linalg.v1"), ctypes.POINTER(ctypes.c_void_p))
    assert table[0] == ctypes.cast(_native.lib().linalg_native_v1, ctypes.c_void_p).value
    entry = ctypes.CFUNCTYPE(ctypes.c_int64, *([ctypes.c_int64] * 9 + [_native.SINK_T]))(table[0])
    r = ctypes.c_int64(0)
    assert entry(12, 0, 0, 0, 0, 0, 0, ctypes.addressof(r), 0, _native.SINK_T(lambda *a: None)) == 0
    assert r.value == 1


def test_op_table_errors_come_through_the_sink_once():
    with pytest.raises(RuntimeError, match="linalg native ABI: unknown operation"):
        _native.call(99, [], [])
    with pytest.raises(RuntimeError, match="metadata takes no descriptors"):
        _native.call(11, [1], [])
    with pytest.raises(RuntimeError, match="invalid gemm address count"):
        _native.call(0, [1, 2], [1, 1, 1, 0])
    with pytest.raises(RuntimeError, match=r"params must contain 4 values \(m, n, k, op\), got 3"):
        _native.call(0, [1, 2, 3], [1, 1, 1])
    with pytest.raises(RuntimeError, match="must all be positive"):
        _native.call(0, [1, 2, 3], [0, 1, 1, 0])
    with pytest.raises(RuntimeError, match="invalid gemm_int15 address count"):
        _native.call(5, [1, 2, 3, 4, 5, 6], [1, 1, 1])
    with pytest.raises(RuntimeError, match=r"gemm_int15: params must contain 3 values \(m, n, k\), got 2"):
        _native.call(5, [1, 2, 3, 4, 5, 6, 7], [1, 1])
    with pytest.raises(RuntimeError, match=r"gemm_int15: k must be at most 65536 \(contract W-4\), got 65537"):
        _native.call(5, [1, 2, 3, 4, 5, 6, 7], [1, 1, 65537])
    with pytest.raises(RuntimeError, match="quantize_int15: rows and cols must be positive, got 2 x 0"):
        _native.call(6, [1, 2, 3, 4], [2, 0])
    with pytest.raises(RuntimeError, match="invalid dequantize_int15 address count"):
        _native.call(7, [1, 2, 3], [2, 2])
    with pytest.raises(RuntimeError, match="from_f16: count must be positive, got 0"):
        _native.call(10, [1, 2], [0])
    with pytest.raises(RuntimeError, match="invalid gemm_int8 address count"):
        _native.call(2, [1, 2, 3, 4], [1, 1, 1])
    with pytest.raises(RuntimeError, match=r"gemm_int8: params must contain 3 values \(m, n, k\), got 4"):
        _native.call(2, [1, 2, 3, 4, 5], [1, 1, 1, 1])
    with pytest.raises(RuntimeError, match="gemm_int8: m, n and k must all be positive, got m=1 n=1 k=0"):
        _native.call(2, [1, 2, 3, 4, 5], [1, 1, 0])
    with pytest.raises(RuntimeError, match=r"gemm_int8: k must be at most 131072 \(contract L-7\), got 131073"):
        _native.call(2, [1, 2, 3, 4, 5], [1, 1, 131073])
    with pytest.raises(RuntimeError, match="quantize_int8: rows and cols must be positive, got 0 x 3"):
        _native.call(3, [1, 2, 3], [0, 3])
    with pytest.raises(RuntimeError, match=r"dequantize_int8: params must contain 2 values \(rows, cols\), got 3"):
        _native.call(4, [1, 2, 3], [1, 2, 3])
    L = _native.lib()
    msgs = []
    sink = _native.SINK_T(lambda ctx, p, n: msgs.append((ctx, ctypes.string_at(p, n))))
    r = ctypes.c_int64(0)
    assert L.linalg_native_v1(12, 0, 0, 0, 0, 0, 1, ctypes.addressof(r), 77, sink) == 1
    assert msgs == [(77, b"linalg native ABI: invalid result or scalar span")]


def test_surface_refusals():
    a = np.ones((4, 3), np.float32)
    with pytest.raises(TypeError, match="only float32 is in this profile"):
        linalg.matmul(a.astype(np.float64), a.T.copy())
    with pytest.raises(ValueError, match="must be 2-D"):
        linalg.matmul(np.ones(3, np.float32), a)
    with pytest.raises(ValueError, match="no elements"):
        linalg.matmul(np.ones((0, 3), np.float32), a)
    with pytest.raises(ValueError, match="transpose_a=True with transpose_b=True is refused"):
        linalg.matmul(a, a, transpose_a=True, transpose_b=True)
    with pytest.raises(ValueError, match="contracted extents disagree"):
        linalg.matmul(a, a)
    with pytest.raises(TypeError, match="out has dtype float64"):
        linalg.matmul(a, a.T.copy(), out=np.empty((4, 4)))
    with pytest.raises(ValueError, match="out has shape"):
        linalg.matmul(a, a.T.copy(), out=np.empty((4, 5), np.float32))
    with pytest.raises(ValueError, match="must be C-contiguous"):
        linalg.matmul(a, a.T.copy(), out=np.empty((4, 8), np.float32)[:, ::2])
    ro = np.empty((4, 4), np.float32)
    ro.flags.writeable = False
    with pytest.raises(ValueError, match="read-only"):
        linalg.matmul(a, a.T.copy(), out=ro)
    with pytest.raises(TypeError, match="bf16 BITS in a uint16 buffer"):
        linalg.matmul_bf16(a, a)
    with pytest.raises(ValueError, match="is not one of the contract's three operations"):
        linalg.matmul_bf16(a, np.ones((3, 4), np.uint16), transpose_a=True, transpose_b=True)


def test_workload_bf16_narrow_matches_oracle(oracle):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(200000) * np.exp2(rng.uniform(-140, 130, 200000))).astype(np.float32)
    specials = np.array([0x7F800001, 0xFFC00001, 0x7F800000, 0x00000001, 0x80000001, 0x7F7FFFFF,
                         0x3F808000, 0x3F818000, 0x00800000], np.uint32).view(np.float32)
    x = np.concatenate([x, specials])
    assert np.array_equal(W.bf16_narrow(x), oracle.bf16_narrow(x))


def test_workload_generators_are_deterministic():
    a, b = W.gemm512()
    assert a.dtype == np.float32 and a.shape == (512, 512) and a.min() >= -1 and a.max() < 1
    x16, codes, scales = W.decode()
    assert codes.dtype == np.int8 and codes.min() >= -127 and scales.min() >= 1e-3 and scales.max() <= 1e-2
    a2, _ = W.gemm512()
    assert np.array_equal(a, a2)


def test_lowbit_containers_and_refusals():
    """The lowbit containers and refusals that run before any conversion
    (python/mojolearn/lowbit.py; providers/python/lowbit_weight_pyapi_door.mojo:52-170)."""
    from mojolearn_amd import lowbit
    bf = lowbit.BF16Weight(np.arange(24, dtype=np.uint16).reshape(6, 4))
    q8 = lowbit.Int8Weight(np.arange(24, dtype=np.int8).reshape(6, 4), np.arange(6, dtype=np.int32) - 3)
    assert bf.shape == (6, 4) and bf.format == "bfloat16" and q8.shape == (6, 4) and q8.format == "int8"
    assert lowbit.is_packed(bf) and lowbit.is_packed(q8) and not lowbit.is_packed(np.ones((2, 2), np.float32))
    assert lowbit.format_of({"w": bf, "n": np.ones(3, np.float32)}) == "bfloat16"
    assert lowbit.format_of((q8,)) == "int8" and lowbit.format_of([]) == "float32"
    with pytest.raises(ValueError, match="store a model one way"):
        lowbit.format_of({"a": bf, "b": q8})
    with pytest.raises(TypeError, match="bits must be a 2-D uint16 array"):
        lowbit.BF16Weight(np.zeros(4, np.uint16))
    with pytest.raises(TypeError, match="codes must be a 2-D int8 array"):
        lowbit.Int8Weight(np.zeros((2, 2), np.uint8), np.zeros(2, np.int32))
    with pytest.raises(TypeError, match="exponents must be int32 of shape"):
        lowbit.Int8Weight(np.zeros((2, 2), np.int8), np.zeros(3, np.int32))
    with pytest.raises(ValueError, match="minimum of 1 is required"):
        lowbit.BF16Weight(np.zeros((0, 4), np.uint16))
    a = np.ones((4, 3), np.float32)
    with pytest.raises(ValueError, match="unknown format 'float16'"):
        lowbit.pack_one(a, "float16")
    with pytest.raises(ValueError, match="must be 2-D to pack, got shape \\(4,\\)"):
        lowbit.pack_one(a[:, 0], "bfloat16")
    with pytest.raises(TypeError, match="pack takes float32"):
        lowbit.pack_one(a.astype(np.float64), "int8")
    with pytest.raises(TypeError, match="must be a dict keyed by name"):
        lowbit.pack([a], "int8")
    with pytest.raises(TypeError, match="format must be an exact string"):
        lowbit.pack({"a": a}, 8)
    # float32 packing copies; non-dicts unpack as themselves; a float32 model unpacks as is
    f = lowbit.pack_one(a, "float32")
    assert f is not a and np.array_equal(f, a)
    assert lowbit.unpack(a) == (a, "float32")
    w = {"a": a}
    assert lowbit.unpack(w) == (w, "float32")


@pytest.mark.parametrize("fmt", ["bfloat16", "int8"])
def test_lowbit_repack_same_format_copies_without_materializing(monkeypatch, fmt):
    from mojolearn_amd import lowbit
    if fmt == "bfloat16":
        original = lowbit.BF16Weight(np.arange(24, dtype=np.uint16).reshape(6, 4))
    else:
        original = lowbit.Int8Weight(np.arange(24, dtype=np.int8).reshape(6, 4), np.arange(6, dtype=np.int32) - 3)
    monkeypatch.setattr(lowbit, "materialize_one", lambda *a, **k: pytest.fail("materialized"))
    copied = lowbit.pack({"w": original}, fmt)["w"]
    assert copied is not original
    if fmt == "bfloat16":
        assert np.array_equal(copied.bits, original.bits) and not np.shares_memory(copied.bits, original.bits)
    else:
        assert np.array_equal(copied.codes, original.codes) and not np.shares_memory(copied.codes, original.codes)
        assert np.array_equal(copied.exponents, original.exponents)
        assert not np.shares_memory(copied.exponents, original.exponents)


def test_route_names_the_kernels_without_a_device():
    """mlg_gemm_route (num_cus > 0: no device needed) for the five workloads and the skinny
    matrix-core shapes: the dispatcher's choices as the design states them."""
    from mojolearn_amd import device as D
    R = lambda *a, **k: D.route(*a, num_cus=256, **k)  # noqa: E731
    assert R(2048, 4096, 4096) == {"tile", "tile_stack"}  # 512 tiles, 32 leaves folded in each tile
    assert R(512, 512, 512) == {"tile", "fold"}  # 16 tiles: 4 leaf groups, then the fold
    assert R(512, 50304, 2048) == {"tile", "tile_stack", "fold", "tail_split"}
    assert R(4096, 11008, 4096, b_type=D.T_BF16) == {"tile", "tile_stack"}
    assert R(1, 14336, 4096, b_type=D.T_I8) == {"gemv_nn", "gemv_groups"}
    assert R(4, 14336, 4096, b_type=D.T_I8) == {"mfma4", "gemv_groups"}
    assert R(16, 14336, 4096, b_type=D.T_I8) == {"mfma16", "gemv_groups"}
    assert R(1, 14336, 4096, op=D.OP_NT) == {"gemv_nt", "gemv_groups"}
    assert R(1, 64, 128) == {"gemv_nn"}  # one leaf group: no cross-workgroup fold
    # whole leaves at m <= 2 take eight leaves a workgroup while the launch keeps a workgroup
    # for every CU: int8 n = 32768 is 256 column groups of 128, k = 1024 is 8 leaves
    assert R(1, 32768, 1024, b_type=D.T_I8) == {"gemv_nn"}
    assert D.route(1, 32768, 1024, b_type=D.T_I8, num_cus=512) == {"gemv_nn", "gemv_groups"}
    assert R(3, 5, 0) == {"zero_k"}
    assert R(16, 64, 4096, a=4) == {"gemv_nn", "gemv_groups"}  # x off the 16-byte grid: the VALU kernel
    assert "repack" in R(64, 64, 100, a=4)


def test_launch_limits_are_refused_with_a_message():
    """Partitions past the fold stack (2^20 roots per cell) or past a tile grid's leaf-group
    column (65535) are refused, never computed wrong (the reference refuses partitions past its
    fold stack, gemm/neural_dispatch.mojo:284-285)."""
    from mojolearn_amd import device as D
    assert D.route(1, 64, 4 * (1 << 20), leaf=1, num_cus=256) == {"gemv_nn", "gemv_groups"}
    with pytest.raises(RuntimeError, match="fold stack"):
        D.route(1, 64, 4 * (1 << 20) + 1, leaf=1, num_cus=256)
    # a tile groups up to 32 leaves: 65535 groups hold 2,097,120 leaves
    assert "fold" in D.route(17, 17, 65535 * 32, leaf=1, num_cus=256)
    with pytest.raises(RuntimeError, match="grid column"):
        D.route(17, 17, 65535 * 32 + 1, leaf=1, num_cus=256)
