"""Parity of the gfx950 kernels (through the C ABI) with the reference, bit for bit.

* the MI325X device card's 20 full-shape rows (hashes recorded by the reference's own device
  kernel, byte-identical to its NVIDIA card) and the host-capped oracle card;
* closed-form fixtures F1-F8, inf/NaN (tests/kat.py);
* the CPU oracle on random shapes: ragged m/n/k, every orientation, wide exponents,
  subnormals, signed zeros, inf/NaN; bf16 and int8 weights; the fused bias; caller leaves;
* the five workloads at their real sizes on row samples (cells are independent of m, so a
  row subset through the oracle is the same bits as the whole product's rows).
"""
import numpy as np
import pytest

import cards
import kat

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _dev():
    from mojolearn_amd import device
    return device


POISON = -987654.0  # gemm/checks/gemm_device_check.mojo:111: a cell left unwritten fails


def gpu_gemm(a, b, op, leaf=0, bias=None):
    D = _dev()
    ta = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    tb = torch.from_numpy(np.ascontiguousarray(b)).to(DEV)
    tbias = None if bias is None else torch.from_numpy(np.ascontiguousarray(bias)).to(DEV)
    m = a.shape[1] if op == 2 else a.shape[0]
    n = b.shape[0] if op == 1 else b.shape[1]
    out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
    c = D.gemm(ta, tb, op=op, leaf=leaf, bias=tbias, out=out)
    torch.cuda.synchronize()
    return c.cpu().numpy()


def words(x):
    return np.ascontiguousarray(x).view(np.uint32)


def assert_bits(got, want, what=""):
    g, w = words(got), words(want)
    bad = np.flatnonzero(g.ravel() != w.ravel())
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {g.size} words differ; first at flat {i}: "
                             f"got {g.ravel()[i]:#010x} want {w.ravel()[i]:#010x}")


def _card_inputs(O, i, m, n, k, op):
    sa, sb = cards.operand_shapes(m, n, k, op)
    return O.card_fill(m * k, 11 + i).reshape(sa), O.card_fill(n * k, 22 + i).reshape(sb)


DEVICE_CARD = cards.parse_card("device_mi325x.card")
HOST_CARD = cards.parse_card("host_oracle.card")


@pytest.mark.parametrize("row", cards.device_rows(), ids=[r[1] for r in cards.device_rows()])
def test_device_card_full_shape(oracle, row):
    """Output hash of the reference's own device run (MI325X card) at the full card shape."""
    i, name, m, n, k, op = row
    print(f"device card {name}: m={m} n={n} k={k} op={op}", flush=True)
    a, b = _card_inputs(oracle, i, m, n, k, op)
    c = gpu_gemm(a, b, op)
    assert (c.size, oracle.fnv1a64(c)) == DEVICE_CARD[name + ".out"], name


@pytest.mark.parametrize("i", range(len(cards.SHAPES)), ids=[s[0] for s in cards.SHAPES])
def test_host_card_capped_shape(oracle, i):
    name, m0, n0, k, op = cards.SHAPES[i]
    m, n = cards.host_capped(m0, n0, k)
    a, b = _card_inputs(oracle, i, m, n, k, op)
    c = gpu_gemm(a, b, op)
    assert (c.size, oracle.fnv1a64(c)) == HOST_CARD[name + ".out"], name


@pytest.mark.parametrize("fx", kat.fixtures(), ids=[f[0] for f in kat.fixtures()])
def test_kat_gpu(fx):
    name, a, b, leaf, want = fx
    c = gpu_gemm(a.reshape(1, -1), b.reshape(1, -1), 1, leaf=leaf)
    assert words(c)[0, 0] == want, (name, hex(int(words(c)[0, 0])), hex(int(want)))


def _values(rng, shape, kind):
    if kind == "normal":
        return rng.standard_normal(shape).astype(np.float32)
    if kind == "wide":  # exponents over most of the range, subnormals, signed zeros
        x = (rng.standard_normal(shape) * np.exp2(rng.uniform(-140, 60, shape))).astype(np.float32)
        z = rng.random(shape)
        x[z < 0.02] = np.float32(0.0)
        x[(z >= 0.02) & (z < 0.04)] = np.float32(-0.0)
        return x
    if kind == "special":  # + a few inf/NaN
        x = _values(rng, shape, "wide")
        z = rng.random(shape)
        x[z < 0.001] = np.float32(np.inf)
        x[(z >= 0.001) & (z < 0.002)] = np.float32(-np.inf)
        x[(z >= 0.002) & (z < 0.0025)] = np.float32(np.nan)
        return x
    raise ValueError(kind)


def _operands(rng, m, n, k, op, kind):
    A = _values(rng, (m, k), kind)
    B = _values(rng, (k, n), kind)
    a = A if op != 2 else np.ascontiguousarray(A.T)
    b = B if op != 1 else np.ascontiguousarray(B.T)
    return a, b


SHAPES = [(1, 1, 1), (5, 7, 3), (17, 33, 129), (130, 129, 300), (128, 128, 128), (257, 255, 517),
          (64, 300, 1024), (3, 1000, 4097), (200, 64, 2048), (4, 5, 100003), (2, 3, 131073), (96, 97, 14336)]


@pytest.mark.parametrize("kind", ["normal", "wide", "special"])
@pytest.mark.parametrize("op", [0, 1, 2])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
def test_random_vs_oracle(oracle, shape, op, kind):
    m, n, k = shape
    rng = np.random.default_rng(m * 7 + n * 13 + k * 17 + op)
    a, b = _operands(rng, m, n, k, op, kind)
    print(f"random {kind} op={op} m={m} n={n} k={k}", flush=True)
    want = oracle.nan_canon(oracle.gemm_fast(a, b, op))
    assert_bits(gpu_gemm(a, b, op), want, f"{shape} op={op} {kind}")


@pytest.mark.parametrize("leaf", [1, 7, 64, 300, 1000])
def test_caller_leaf(oracle, leaf):
    """A caller-given partition (the sequence-executor word is leaf = k, one chain)."""
    rng = np.random.default_rng(leaf)
    m, n, k = 33, 65, 1000
    a, b = _operands(rng, m, n, k, 0, "wide")
    assert_bits(gpu_gemm(a, b, 0, leaf=leaf), oracle.gemm_fast(a, b, 0, leaf=leaf), f"leaf={leaf}")
    serial = gpu_gemm(a, b, 0, leaf=k)
    assert_bits(serial, oracle.gemm_serial(a, b, 0), "serial word")


def test_k_zero_writes_plus_zero():
    D = _dev()
    a = torch.empty((3, 0), dtype=torch.float32, device=DEV)
    b = torch.empty((0, 5), dtype=torch.float32, device=DEV)
    c = torch.full((3, 5), -987654.0, device=DEV)
    D.gemm(a, b, op=0, out=c)
    torch.cuda.synchronize()
    assert np.all(words(c.cpu().numpy()) == 0)


@pytest.mark.parametrize("op", [0, 1])
def test_bias_epilogue(oracle, op):
    rng = np.random.default_rng(11 + op)
    m, n, k = 70, 150, 640
    a, b = _operands(rng, m, n, k, op, "wide")
    bias = _values(rng, (n,), "wide")
    want = oracle.nan_canon(oracle.bias(oracle.gemm_fast(a, b, op), bias))
    assert_bits(gpu_gemm(a, b, op, bias=bias), want, "bias")


@pytest.mark.parametrize("op", [0, 1, 2])
@pytest.mark.parametrize("a_bits", [False, True])
def test_bf16_weights(oracle, op, a_bits):
    D = _dev()
    rng = np.random.default_rng(21 + op)
    m, n, k = 67, 131, 777
    a, b = _operands(rng, m, n, k, op, "wide")
    bb = oracle.bf16_narrow(b)
    aa = oracle.bf16_narrow(a) if a_bits else a
    want = oracle.nan_canon(oracle.gemm_fast(oracle.bf16_widen(aa) if a_bits else aa, oracle.bf16_widen(bb), op))
    ta = torch.from_numpy(aa.view(np.int16) if a_bits else aa).to(DEV)
    c = D.gemm_bf16w(ta, torch.from_numpy(bb.view(np.int16)).to(DEV), op=op)
    torch.cuda.synchronize()
    assert_bits(c.cpu().numpy(), want, "bf16")


@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("m", [1, 4, 16, 100])
def test_int8_weights(oracle, op, m):
    D = _dev()
    rng = np.random.default_rng(31 + op + m)
    n, k = 300, 1100
    a = rng.standard_normal((m, k)).astype(np.float32)
    codes = rng.integers(-127, 128, (k, n) if op == 0 else (n, k), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    want = oracle.nan_canon(oracle.gemm_fast(a, oracle.int8_dequant(codes, scales, op), op))
    c = D.gemm_int8w(torch.from_numpy(a).to(DEV), torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV),
                     op=op)
    torch.cuda.synchronize()
    assert_bits(c.cpu().numpy(), want, "int8")


def test_bf16_conversions(oracle):
    D = _dev()
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    w = D.bf16_widen(torch.from_numpy(bits.view(np.int16)).to(DEV)).cpu().numpy()
    assert_bits(w, oracle.bf16_widen(bits), "widen")
    rng = np.random.default_rng(5)
    x = _values(rng, (100000,), "special")
    n = D.bf16_narrow(torch.from_numpy(x).to(DEV)).cpu().numpy().view(np.uint16)
    assert np.array_equal(n, oracle.bf16_narrow(x))


GEMV_SHAPES = [(1, 1, 1), (1, 255, 129), (2, 256, 128), (7, 257, 1000), (16, 1000, 4096), (1, 4100, 300),
               (3, 4096, 4097), (16, 33, 2048), (1, 14336, 4096), (2, 70, 140000), (5, 300, 515),
               # whole 128-row leaves at m <= 2: one partial group, two full groups and one leaf,
               # three full groups and a partial one, sixteen groups (eight of eight leaves at
               # 256 CUs); eight-leaf groups with a ragged last group and column group
               (2, 300, 640), (1, 1024, 1152), (1, 512, 1664), (2, 4096, 8192), (1, 8196, 4480),
               (2, 8196, 4480)]


@pytest.mark.parametrize("wt", ["f32", "bf16", "i8"])
@pytest.mark.parametrize("shape", GEMV_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in GEMV_SHAPES])
def test_skinny_m(oracle, shape, wt):
    """The skinny-M (decode GEMV) path: a leaf per wave streamed into registers (word loads,
    or element loads when a row is not a multiple of 4 bytes), groups of 4 leaves (8 with
    whole leaves at m <= 2 on a wide launch) folded in LDS, the last-arriving group folding the rest; leaves longer than 128 rows (k > 131072),
    ragged last leaves, ragged last groups."""
    D = _dev()
    m, n, k = shape
    rng = np.random.default_rng(m + n + k)
    x = _values(rng, (m, k), "wide")
    print(f"skinny {wt} m={m} n={n} k={k}", flush=True)
    tx = torch.from_numpy(x).to(DEV)
    if wt == "f32":
        w = _values(rng, (k, n), "wide")
        got = D.gemm(tx, torch.from_numpy(w).to(DEV))
        want = oracle.gemm_fast(x, w, 0)
    elif wt == "bf16":
        wb = oracle.bf16_narrow(_values(rng, (k, n), "wide"))
        got = D.gemm_bf16w(tx, torch.from_numpy(wb.view(np.int16)).to(DEV))
        want = oracle.gemm_fast(x, oracle.bf16_widen(wb), 0)
    else:
        codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        got = D.gemm_int8w(tx, torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV))
        want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0)
    torch.cuda.synchronize()
    assert_bits(got.cpu().numpy(), oracle.nan_canon(want), f"skinny {wt} {shape}")
    # again on the same stream: the completion counters must have been left at zero
    if wt == "i8":
        got2 = D.gemm_int8w(tx, torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV))
        torch.cuda.synchronize()
        assert_bits(got2.cpu().numpy(), oracle.nan_canon(want), "second call")


GEMV_NT_SHAPES = GEMV_SHAPES + [(1, 64, 128), (4, 65, 256), (1, 130, 200)]

# 3 <= m <= 16 with whole 128-row leaves: the matrix-core skinny kernels (4 x 4 shape up to m = 8)
GEMV_MFMA_SHAPES = [(5, 257, 1024), (8, 300, 4096), (12, 64, 512), (16, 1024, 128), (16, 4100, 1024),
                    (9, 1000, 3968), (16, 14336, 4096), (7, 200, 1664), (16, 96, 1152), (2, 300, 1024),
                    (3, 257, 4096), (4, 14336, 4096), (6, 129, 1152), (4, 64, 640)]


# whole 128-row leaves with 3 <= m <= 16 and x off the 16-byte grid: the VALU kernel's straight-line
# leaf with 4, 8 and 16 rows of chains (int8 on 16-bit lanes), which aligned x never reaches
GEMV_OFFGRID_SHAPES = [(3, 300, 1024), (4, 257, 640), (8, 1000, 4096), (16, 129, 1152), (16, 2048, 4096)]


@pytest.mark.parametrize("wt", ["f32", "bf16", "i8"])
@pytest.mark.parametrize("shape", GEMV_OFFGRID_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in GEMV_OFFGRID_SHAPES])
def test_skinny_m_x_off_grid(oracle, shape, wt):
    """x starting one float into its buffer (4-byte but not 16-byte aligned) keeps a whole-leaf
    product with 3 <= m <= 16 off the matrix-core kernels: gemv_nn_kernel's whole-leaf variant
    runs its 4-, 8- or 16-row chains, on poisoned outputs with the fused bias."""
    from mojolearn_amd import device as D
    m, n, k = shape
    rng = np.random.default_rng(m * 7 + n + k)
    x = _values(rng, (m, k), "wide")
    bias = _values(rng, (n,), "wide")
    print(f"skinny off-grid x {wt} m={m} n={n} k={k}", flush=True)
    buf = torch.empty(m * k + 4, dtype=torch.float32, device=DEV)
    tx = buf[1:1 + m * k].view(m, k)
    tx.copy_(torch.from_numpy(x))
    assert tx.data_ptr() % 16 != 0
    tbias = torch.from_numpy(bias).to(DEV)
    out = torch.full((m, n), POISON, dtype=torch.float32, device=DEV)
    if wt == "f32":
        w = _values(rng, (k, n), "wide")
        tw = torch.from_numpy(w).to(DEV)
        D.gemm(tx, tw, bias=tbias, out=out)
        want = oracle.gemm_fast(x, w, 0)
        bt = D.T_F32
    elif wt == "bf16":
        wb = oracle.bf16_narrow(_values(rng, (k, n), "wide"))
        tw = torch.from_numpy(wb.view(np.int16)).to(DEV)
        D.gemm_bf16w(tx, tw, bias=tbias, out=out)
        want = oracle.gemm_fast(x, oracle.bf16_widen(wb), 0)
        bt = D.T_BF16
    else:
        codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        tw = torch.from_numpy(codes).to(DEV)
        D.gemm_int8w(tx, tw, torch.from_numpy(scales).to(DEV), bias=tbias, out=out)
        want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0)
        bt = D.T_I8
    torch.cuda.synchronize()
    assert "gemv_nn" in D.route(m, n, k, b_type=bt, a=tx, b=tw)
    assert_bits(out.cpu().numpy(), oracle.nan_canon(oracle.bias(want, bias)), f"skinny off-grid {wt} {shape}")


@pytest.mark.parametrize("kind", ["wide", "special"])
@pytest.mark.parametrize("wt", ["f32", "bf16", "i8"])
@pytest.mark.parametrize("shape", GEMV_MFMA_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in GEMV_MFMA_SHAPES])
def test_skinny_m_mfma(oracle, shape, wt, kind):
    """3 <= m <= 16, whole leaves: the chains on v_mfma_f32_4x4x1_16b_f32 (m <= 8) or
    v_mfma_f32_16x16x1_4b_f32 (one fma per step per
    cell, input flush by the mode), ragged column groups, one to many leaf groups, subnormal,
    signed-zero, inf and NaN operands, and the fused bias."""
    D = _dev()
    m, n, k = shape
    rng = np.random.default_rng(m * 3 + n + k)
    x = _values(rng, (m, k), kind)
    bias = _values(rng, (n,), "wide")
    print(f"skinny mfma {wt} {kind} m={m} n={n} k={k}", flush=True)
    tx, tbias = torch.from_numpy(x).to(DEV), torch.from_numpy(bias).to(DEV)
    if wt == "f32":
        w = _values(rng, (k, n), kind)
        got = D.gemm(tx, torch.from_numpy(w).to(DEV), bias=tbias)
        want = oracle.gemm_fast(x, w, 0)
    elif wt == "bf16":
        wb = oracle.bf16_narrow(_values(rng, (k, n), kind))
        got = D.gemm_bf16w(tx, torch.from_numpy(wb.view(np.int16)).to(DEV), bias=tbias)
        want = oracle.gemm_fast(x, oracle.bf16_widen(wb), 0)
    else:
        codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        got = D.gemm_int8w(tx, torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV), bias=tbias)
        want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0)
    torch.cuda.synchronize()
    assert_bits(got.cpu().numpy(), oracle.nan_canon(oracle.bias(want, bias)), f"skinny mfma {wt} {shape}")


@pytest.mark.parametrize("wt", ["f32", "bf16", "i8"])
@pytest.mark.parametrize("shape", GEMV_NT_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in GEMV_NT_SHAPES])
def test_skinny_m_nt(oracle, shape, wt):
    """The skinny-M path in the LM layout (OP_NT, W[n][k]): a lane per output column walking
    its own W row, 16-byte loads when rows and leaf starts are 16-byte aligned, element loads
    otherwise; the same leaf groups and fold as OP_NN."""
    D = _dev()
    m, n, k = shape
    rng = np.random.default_rng(m + n + k + 1)
    x = _values(rng, (m, k), "wide")
    print(f"skinny NT {wt} m={m} n={n} k={k}", flush=True)
    tx = torch.from_numpy(x).to(DEV)
    if wt == "f32":
        w = _values(rng, (n, k), "wide")
        got = D.gemm(tx, torch.from_numpy(w).to(DEV), op=D.OP_NT)
        want = oracle.gemm_fast(x, w, oracle.OP_NT)
    elif wt == "bf16":
        wb = oracle.bf16_narrow(_values(rng, (n, k), "wide"))
        got = D.gemm_bf16w(tx, torch.from_numpy(wb.view(np.int16)).to(DEV), op=D.OP_NT)
        want = oracle.gemm_fast(x, oracle.bf16_widen(wb), oracle.OP_NT)
    else:
        codes = rng.integers(-127, 128, (n, k), dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        got = D.gemm_int8w(tx, torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV), op=D.OP_NT)
        want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, oracle.OP_NT), oracle.OP_NT)
    torch.cuda.synchronize()
    assert_bits(got.cpu().numpy(), oracle.nan_canon(want), f"skinny NT {wt} {shape}")


@pytest.mark.parametrize("case", ["skinny_i8", "mfma_groups", "mfma_bias", "mfma_tail_split"])
def test_plan_in_graph_replays(oracle, case):
    """A Plan (caller workspace, no allocation per call) captured in a HIP graph: every replay,
    with eager products and synchronizations between replays, gives the oracle's bits."""
    D = _dev()
    rng = np.random.default_rng(77)
    if case == "skinny_i8":
        m, n, k = 2, 1000, 4096
        a = rng.standard_normal((m, k)).astype(np.float32)
        codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        plan = D.Plan(torch.from_numpy(a).to(DEV), torch.from_numpy(codes).to(DEV),
                      scales=torch.from_numpy(scales).to(DEV))
        want = oracle.gemm_fast(a, oracle.int8_dequant(codes, scales, 0), 0)
    else:
        # the tail split: on 256 CUs, 64 column tiles whole and the last one in leaf groups
        m, n, k = {"mfma_groups": (150, 170, 8192), "mfma_bias": (150, 170, 700),
                   "mfma_tail_split": (512, 8320, 512)}[case]
        a, b = _operands(rng, m, n, k, 0, "wide")
        bias = _values(rng, (n,), "wide") if case in ("mfma_bias", "mfma_tail_split") else None
        plan = D.Plan(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV),
                      bias=None if bias is None else torch.from_numpy(bias).to(DEV))
        want = oracle.gemm_fast(a, b, 0)
        if bias is not None:
            want = oracle.bias(want, bias)
    want = oracle.nan_canon(want)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        plan(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        plan(s)
    for rep in range(3):
        plan.out.fill_(-987654.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_bits(plan.out.cpu().numpy(), want, f"{case} replay {rep}")
        gpu_gemm(*_operands(rng, 33, 40, 300, 0, "normal"), 0)  # eager work between replays


# Products whose tiles fill whole rounds of the CUs and leave a short last round run as two
# column ranges, the tail with its leaves in aligned groups (on 256 CUs: 4 x 65 = 260 tiles, 64
# column tiles whole, the last one grouped).  Every cell against the oracle, bias included.
TAIL = [(0, "f32", 512, 8320, 512, True), (1, "f32", 512, 8300, 384, False), (2, "f32", 512, 8320, 256, True),
        (0, "bf16", 512, 8320, 512, False), (1, "bf16", 512, 8300, 640, True), (0, "i8", 512, 8320, 512, True),
        (1, "i8", 512, 8304, 512, False)]


@pytest.mark.parametrize("case", TAIL, ids=[f"op{o}-{w}-{m}x{n}x{k}{'-bias' if b else ''}" for o, w, m, n, k, b in TAIL])
def test_tail_split_vs_oracle(oracle, case):
    op, wt, m, n, k, with_bias = case
    D = _dev()
    print(f"tail split {case}", flush=True)
    rng = np.random.default_rng(m + n + k + op)
    a, b = _operands(rng, m, n, k, op, "wide")
    bias = _values(rng, (n,), "wide") if with_bias else None
    ta = torch.from_numpy(a).to(DEV)
    tbias = None if bias is None else torch.from_numpy(bias).to(DEV)
    b_type = {"f32": 0, "bf16": 1, "i8": 2}[wt]
    if wt == "f32":
        want = oracle.gemm_fast(a, b, op)
        c = D.gemm(ta, torch.from_numpy(b).to(DEV), op=op, bias=tbias)
    elif wt == "bf16":
        bb = oracle.bf16_narrow(b)
        want = oracle.gemm_fast(a, oracle.bf16_widen(bb), op)
        c = D.gemm_bf16w(ta, torch.from_numpy(bb.view(np.int16)).to(DEV), op=op, bias=tbias)
    else:
        codes = rng.integers(-127, 128, b.shape, dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        want = oracle.gemm_fast(a, oracle.int8_dequant(codes, scales, op), op)
        c = D.gemm_int8w(ta, torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV), op=op,
                         bias=tbias)
    torch.cuda.synchronize()
    if with_bias:
        want = oracle.bias(want, bias)
    assert_bits(c.cpu().numpy(), oracle.nan_canon(want), "tail split")
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        # the grouped tail's roots are the only workspace these in-place products need
        assert D.workspace_bytes(m, n, k, op=op, b_type=b_type) > 0
