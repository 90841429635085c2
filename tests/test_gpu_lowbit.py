"""Low-bit weight storage (mojolearn_amd.lowbit) and the low-bit linalg seams on gfx950: the
lowbit-conversions verify cells on all nine fixtures, pack/unpack containers and repacking
(python/mojolearn/tests/test_lowbit_weights.py:42-94), and the bf16/int8 input forms and
sentinels (python/mojolearn/tests/test_linalg_lowbit.py:52-123), every float compared bit for
bit with the CPU oracle."""
import numpy as np
import pytest

import verify_lanes as VL

pytestmark = pytest.mark.gpu


def _hw(shape, seed, lo=-0.125, hi=0.125):
    rng = np.random.default_rng(seed)
    return (lo + (hi - lo) * rng.random(shape)).astype(np.float32)


def _same(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("kind", VL.FIXTURES)
def test_verify_lane_lowbit_conversions_through_the_surface(oracle, kind):
    from mojolearn_amd import linalg, lowbit
    print(f"lowbit lane {kind}", flush=True)
    X = VL.fixture_x(kind)
    lane = VL.lane_lowbit_conversions(lowbit, linalg.from_bf16, oracle, X)
    assert VL.train_hash(lane) == VL.golden()["cells"][f"lowbit-conversions/{kind}"]["train"]


@pytest.mark.parametrize("fmt", ["bfloat16", "int8"])
def test_pack_unpack_containers_and_repacking(oracle, fmt):
    from mojolearn_amd import lowbit
    print(f"lowbit pack/unpack {fmt}", flush=True)
    w = {"a": _hw((40, 32), 1), "n": _hw((32,), 2), "b": _hw((32, 24), 3)}
    packed = lowbit.pack(w, fmt)
    assert lowbit.format_of(packed) == fmt
    assert lowbit.is_packed(packed["a"]) and not lowbit.is_packed(packed["n"])
    f32, got = lowbit.unpack(packed)
    assert got == fmt and f32["n"] is packed["n"]
    for k in ("a", "b"):
        if fmt == "bfloat16":
            bits = oracle.bf16_narrow(w[k])
            assert np.array_equal(packed[k].bits, bits)
            assert _same(f32[k], oracle.bf16_widen(bits))
        else:
            codes, exps = oracle.q8_quantize(w[k])
            assert np.array_equal(packed[k].codes, codes) and np.array_equal(packed[k].exponents, exps)
            assert _same(f32[k], oracle.q8_dequantize(codes, exps))
    # idempotent: packing the materialized weights again changes nothing
    again = lowbit.pack(f32, fmt)
    for k in ("a", "b"):
        if fmt == "bfloat16":
            assert np.array_equal(again[k].bits, packed[k].bits)
        else:
            assert np.array_equal(again[k].codes, packed[k].codes)
            assert np.array_equal(again[k].exponents, packed[k].exponents)
    # a model stored one way and unpacked to float32 repacks to the other format from the
    # materialized floats
    other = "int8" if fmt == "bfloat16" else "bfloat16"
    cross = lowbit.pack(packed, other)
    assert lowbit.format_of(cross) == other
    want = lowbit.pack(f32, other)
    for k in ("a", "b"):
        assert _same(lowbit.materialize_one(cross[k]), lowbit.materialize_one(want[k]))
    plain = lowbit.pack(packed, "float32")
    assert _same(plain["a"], f32["a"]) and plain["n"] is packed["n"]


def test_linalg_bf16_and_int8_forms():
    from mojolearn_amd import linalg
    x = np.array([[1.25, -2.5], [0.0, 1.0]], np.float32)
    bits = np.asarray(linalg.to_bf16(x))
    assert bits.dtype == np.uint16 and bits.shape == x.shape and bits[0, 0] == 0x3FA0
    wide = np.asarray(linalg.from_bf16(bits))
    assert wide.dtype == np.float32 and wide.shape == x.shape and wide[0, 0] == 1.25
    a = np.array([[1.0, 0.0], [0.0, 1.0]], np.float32)
    b = np.array([[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]], np.float32)
    qa, ea = linalg.quantize_int8(a)
    qb, eb = linalg.quantize_int8(b)
    assert qa.dtype == np.int8 and qa.shape == (2, 2) and ea.dtype == np.int32 and ea.shape == (2,)
    assert qb.shape == (3, 2) and eb.shape == (3,)
    assert qa[0, 0] == 64 and ea[0] == -6
    c1 = linalg.matmul_int8(a, b)
    c2 = linalg.matmul_int8((qa, ea), (qb, eb))
    assert c1.dtype == np.float32 and c1.shape == (2, 3) and _same(c1, c2) and c1[0, 0] == 1.0
    y = linalg.dequantize_int8(qb, eb)
    assert y.shape == (3, 2) and y[0, 0] == 1.0
    for ta, tb, lowbit_a in ((False, True, False), (False, False, False), (True, False, False),
                             (False, True, True)):
        aa = np.array([[1.0, 2.0], [0.0, 1.0]], np.float32)
        bb = np.array([[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]], np.float32)
        if ta:
            aa = np.ascontiguousarray(aa.T)
        if not tb:
            bb = np.ascontiguousarray(bb.T)
        if lowbit_a:
            aa = linalg.to_bf16(aa)
        r = linalg.matmul_bf16(aa, linalg.to_bf16(bb), transpose_a=ta, transpose_b=tb)
        assert r.dtype == np.float32 and r.shape == (2, 3) and r[0, 1] == 2.0 and r[0, 2] == 3.0
