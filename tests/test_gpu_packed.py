"""Decode-packed int8 weights (mlg_int8w_pack, mlg_gemv_int8w_packed), on the GPU.

* The pack kernel's bytes equal a NumPy restatement of the layout (a reshape of the codes to
  [leaf][block][row][group][lane] and a transpose to [block][leaf][group][lane][row], columns
  padded with zero codes), which shares no index arithmetic with the kernel.
* The packed decode product is bit-equal, on poisoned outputs, to the oracle and to the
  row-major product (gemm_int8w) for 1 <= m <= 16, on the VALU kernel (m <= 2, or x off the
  16-byte grid) and the matrix-core one (3 <= m <= 16, both shapes): whole-column workgroups
  (32 leaves, one group), whole-column workgroups with a ragged second group and an odd last
  leaf, 4-leaf groups folded across workgroups, ragged column groups, special x values,
  extreme and subnormal scales, with and without the fused bias; again on a second call
  (counters left zero).
* A PackedPlan captured in a HIP graph on a fresh stream replays correctly with eager work in
  between.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"
POISON = -987654.0


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def packed_layout(codes):
    """The decode-packed bytes of codes[k][n] (k a multiple of 128): each code biased to the
    unsigned byte code + 128 (columns past n hold code 0, byte 128)."""
    k, n = codes.shape
    P, G = k // 128, -(-n // 64)
    pad = np.zeros((k, G * 64), np.int8)
    pad[:, :n] = codes
    a = pad.reshape(P, 8, 16, G, 64).transpose(1, 0, 3, 4, 2)
    return np.ascontiguousarray(a).reshape(-1).view(np.uint8) ^ np.uint8(0x80)


@pytest.mark.parametrize("k,n", [(128, 1), (256, 130), (1152, 257), (4096, 300), (4480, 8196)])
def test_pack_layout(k, n):
    from mojolearn_amd import device as D
    rng = np.random.default_rng(k + n)
    codes = rng.integers(-128, 128, (k, n), dtype=np.int8)
    packed = D.pack_int8w(_t(codes))
    torch.cuda.synchronize()
    got = packed.data.cpu().numpy()
    assert got.size == k * 64 * (-(-n // 64))
    assert np.array_equal(got, packed_layout(codes))


def _x(rng, m, k, special):
    x = (rng.standard_normal((m, k)) * np.exp2(rng.uniform(-20, 20, (m, k)))).astype(np.float32)
    if special:
        flat = x.reshape(-1)
        idx = rng.choice(flat.size, min(flat.size, 64), replace=False)
        vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-42, 3e38], np.float32)
        flat[idx] = vals[np.arange(idx.size) % vals.size]
    return x


# whole-column workgroups where ceil(n / 64) * ceil(k / 4096) >= 192 (on 256 CUs) and m <= 2
# (the VALU kernel) or 3 <= m <= 16 with x on the 16-byte grid (the matrix-core kernel):
# 1x14336x4096, 5x14336x4096, 16x12288x4096 (one group), 1x8196x4480, 8x8196x4480,
# 16x8196x4480, 2x12300x4224 and 3x12300x4224 (a second group of 3 or 1 leaves: an odd last
# leaf run alone); the rest in 4-leaf groups
PACKED_SHAPES = [(1, 14336, 4096), (2, 300, 640), (1, 1, 128), (1, 130, 256), (3, 257, 1024), (4, 1000, 4096),
                 (8, 64, 1152), (16, 129, 1152), (16, 2048, 4096), (1, 8196, 4480), (2, 4096, 8192), (5, 14336, 4096),
                 (16, 12288, 4096), (2, 12300, 4224), (1, 1792, 4096), (1, 64, 384), (4, 14336, 4096),
                 (8, 8196, 4480), (16, 8196, 4480), (3, 12300, 4224), (12, 14336, 4096)]


@pytest.mark.parametrize("shape", PACKED_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in PACKED_SHAPES])
def test_packed_gemv_parity(oracle, shape):
    from mojolearn_amd import device as D
    m, n, k = shape
    rng = np.random.default_rng(m * 31 + n + k)
    special = (m + n) % 2 == 1
    x = _x(rng, m, k, special)
    codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    if special:  # extreme scales: subnormal (flushed on input), zero, huge (past the exact fma
        # form's 2^120: its wave takes the sign-extended dequant), tiny normal, infinite, NaN
        sv = np.array([1e-40, 0.0, 3e37, 1.2e-38, np.inf, -np.inf, np.nan], np.float32)
        scales[: min(n, sv.size)] = sv[: min(n, sv.size)]
    bias = rng.standard_normal(n).astype(np.float32) if k % 256 == 0 else None
    print(f"packed gemv m={m} n={n} k={k} special={special} bias={bias is not None}", flush=True)
    tx, tc, ts = _t(x), _t(codes), _t(scales)
    tb = None if bias is None else _t(bias)
    packed = D.pack_int8w(tc)
    want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0)
    if bias is not None:
        want = oracle.bias(want, bias)
    want = oracle.nan_canon(want)
    for call in range(2):  # a second call: the completion counters were left zero
        out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
        D.gemv_int8w_packed(tx, packed, ts, bias=tb, out=out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        bad = np.flatnonzero(_bits(got) != _bits(want))
        assert bad.size == 0, f"call {call}: {bad.size} words differ, first at {divmod(int(bad[0]), n)}"
    rowmajor = D.gemm_int8w(tx, tc, ts, bias=tb).cpu().numpy()
    assert np.array_equal(_bits(rowmajor), _bits(got))


@pytest.mark.parametrize("m", [1, 4, 16])
def test_packed_gemv_dequant_forms_at_their_boundary(oracle, m):
    """The dequant's fma form (f32(code + 128) * scale - 128 * scale) holds for |scale| < 2^120;
    a wave with any larger scale takes the sign-extended form.  Scales just below and at 2^120
    (products up to 127 * 2^120, finite), the largest and smallest normal floats and ordinary
    ones, in different waves and in one wave together: the bits of the oracle's rn(f32(code) *
    scale) chains either way."""
    from mojolearn_amd import device as D
    k, n = 4096, 12288  # whole-column workgroups (192 groups fill the CUs)
    rng = np.random.default_rng(m + 120)
    x = (rng.standard_normal((m, k)) * 2.0 ** -100).astype(np.float32)  # keeps sums finite
    codes = rng.integers(-128, 128, (k, n), dtype=np.int8)
    edge = np.array([np.nextafter(np.float32(2.0 ** 120), np.float32(0)), np.float32(2.0 ** 120),
                     np.float32(3.4e38), np.float32(1.17549435e-38), np.float32(-2.0 ** 119)], np.float32)
    scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    scales[:64] = edge[np.arange(64) % edge.size]      # one group: every wave of it falls back
    scales[64:128] = edge[0]                           # just below: the fma form
    scales[128:192] = -edge[0]
    scales[200] = edge[1]                              # one lane at 2^120 in an ordinary group
    print(f"packed gemv dequant boundary: m={m} n={n} k={k}", flush=True)
    packed = D.pack_int8w(_t(codes))
    want = oracle.nan_canon(oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0))
    out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
    D.gemv_int8w_packed(_t(x), packed, _t(scales), out=out)
    torch.cuda.synchronize()
    got = oracle.nan_canon(out.cpu().numpy())
    bad = np.flatnonzero(_bits(got) != _bits(want))
    assert bad.size == 0, f"{bad.size} words differ, first at {divmod(int(bad[0]), n)}"


@pytest.mark.parametrize("m,n,k", [(3, 14336, 4096), (8, 300, 1024), (16, 12288, 4096)])
def test_packed_gemv_x_off_the_16_byte_grid(oracle, m, n, k):
    """x at a 4-byte offset: the matrix-core kernel loads x in 16-byte chunks, so these products
    take the VALU kernel (whole columns or 4-leaf groups); the bits are the same."""
    from mojolearn_amd import device as D
    rng = np.random.default_rng(m + n + k + 5)
    x = _x(rng, m, k, True)
    codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    print(f"packed gemv, x off the grid: m={m} n={n} k={k}", flush=True)
    store = torch.empty(m * k + 1, dtype=torch.float32, device=DEV)
    tx = store[1:].view(m, k)
    tx.copy_(_t(x))
    packed = D.pack_int8w(_t(codes))
    want = oracle.nan_canon(oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0))
    out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
    D.gemv_int8w_packed(tx, packed, _t(scales), out=out)
    torch.cuda.synchronize()
    bad = np.flatnonzero(_bits(out.cpu().numpy()) != _bits(want))
    assert bad.size == 0, f"{bad.size} words differ, first at {divmod(int(bad[0]), n)}"


def test_packed_plan_captured_on_a_fresh_stream(oracle):
    from mojolearn_amd import device as D
    rng = np.random.default_rng(303)
    m, n, k = 1, 14336, 4096
    x = rng.standard_normal((m, k)).astype(np.float32)
    codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0)
    packed = D.pack_int8w(_t(codes))
    plan = D.PackedPlan(_t(x), packed, _t(scales))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        plan(s)
    for rep in range(3):
        plan.out.fill_(POISON)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(plan.out.cpu().numpy()), _bits(want)), f"replay {rep}"
        D.gemm(_t(x), _t(np.ascontiguousarray(codes[:, :300], dtype=np.float32)))  # eager work between


def test_packed_refusals():
    from mojolearn_amd import device as D
    codes = torch.zeros((100, 64), dtype=torch.int8, device=DEV)
    with pytest.raises(ValueError, match="multiple of 128"):
        D.pack_int8w(codes)
    packed = D.pack_int8w(torch.zeros((128, 64), dtype=torch.int8, device=DEV))
    scales = torch.ones(64, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError, match="1 <= m <= 16"):
        D.gemv_int8w_packed(torch.zeros((17, 128), dtype=torch.float32, device=DEV), packed, scales)
    with pytest.raises(ValueError, match=r"x must be \[m, 128\]"):
        D.gemv_int8w_packed(torch.zeros((1, 256), dtype=torch.float32, device=DEV), packed, scales)
