"""The sequence executor's word (op_gemm, sequence/ops.mojo:518-531), the caller-partition
product (identical_gemm_leaf_ptr_into, gemm/neural_dispatch.mojo:245-307) and the product's
followers (gemm/checks/gemm_identical.mojo:8884-8912; sequence/act_values.mojo) on gfx950,
against the CPU oracle, bit for bit (NaN compared as 0x7FC00000): every operand view (dense,
transposed, gathered, unaligned), C rows at a stride, accumulate, k = 0, partitions from one leaf
to one step per leaf, and the activations over planted and wide-range values."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _dev():
    from mojolearn_amd import device
    return device


def _same(got, want, what):
    g = np.ascontiguousarray(got, np.float32).view(np.uint32).ravel().copy()
    w = np.ascontiguousarray(want, np.float32).view(np.uint32).ravel().copy()
    for x in (g, w):
        x[(x & 0x7FFFFFFF) > 0x7F800000] = 0x7FC00000
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} words differ; first at {bad[0]}: {g[bad[0]]:#010x} want {w[bad[0]]:#010x}"


def _operand(rng, rows, cols, form, scale=1.0):
    """A (rows, cols) host matrix and a device view of it in the given form."""
    x = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    if form == "dense":
        return x, torch.from_numpy(x).to(DEV)
    if form == "t":  # a transposed view of a (cols, rows) buffer
        return x, torch.from_numpy(np.ascontiguousarray(x.T)).to(DEV).t()
    if form == "gather":  # every other column of a wider buffer
        big = np.zeros((rows, 2 * cols), np.float32)
        big[:, ::2] = x
        return x, torch.from_numpy(big).to(DEV)[:, ::2]
    if form == "offset":  # dense rows starting one element into the buffer (base not 16-byte aligned)
        flat = np.zeros(rows * cols + 1, np.float32)
        flat[1:] = x.ravel()
        return x, torch.from_numpy(flat).to(DEV)[1:].view(rows, cols)
    raise ValueError(form)


FORMS = [("dense", "dense"), ("t", "dense"), ("dense", "t"), ("t", "t"), ("gather", "dense"), ("dense", "gather"),
         ("offset", "offset")]
SHAPES = [(1, 1, 1), (3, 5, 7), (37, 41, 300), (130, 129, 1000), (16, 300, 4097), (200, 64, 64)]


@pytest.mark.parametrize("forms", FORMS, ids=[f"{a}-{b}" for a, b in FORMS])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
@pytest.mark.parametrize("accumulate", [False, True])
def test_seq_word_vs_oracle(oracle, forms, shape, accumulate):
    m, n, k = shape
    print(f"seq word {forms} {shape} acc={accumulate}", flush=True)
    rng = np.random.default_rng(m * 7 + n * 3 + k + accumulate)
    A, ta = _operand(rng, m, k, forms[0])
    B, tb = _operand(rng, k, n, forms[1])
    ldc = n + 3
    c0 = (rng.standard_normal((m, ldc)) * 10).astype(np.float32)
    c0[0, 0] = np.array([5], np.uint32).view(np.float32)[0]  # a subnormal seed
    tc_big = torch.from_numpy(c0).to(DEV)
    _dev().seq_gemm(ta, tb, tc_big[:, :n], accumulate=accumulate)
    torch.cuda.synchronize()
    want = c0.copy()
    oracle.seq_gemm(want.reshape(-1), A.reshape(-1), B.reshape(-1), m, n, k, k, 1, n, 1, ldc, accumulate)
    got = tc_big.cpu().numpy()
    _same(got[:, :n], want[:, :n], "cells")
    _same(got[:, n:], c0[:, n:], "cells past n untouched")


@pytest.mark.parametrize("accumulate", [False, True])
def test_seq_word_k0(accumulate):
    c0 = np.array([[1.5, np.array([7], np.uint32).view(np.float32)[0], -2.0]], np.float32)
    tc = torch.from_numpy(c0).to(DEV)
    a = torch.zeros((1, 0), device=DEV)
    b = torch.zeros((0, 3), device=DEV)
    _dev().seq_gemm(a, b, tc, accumulate=accumulate)
    want = np.array([[1.5, 0.0, -2.0]], np.float32) if accumulate else np.zeros((1, 3), np.float32)
    _same(tc.cpu().numpy(), want, "k = 0")


PARTITIONS = [(64, 96, 1000, 100), (64, 96, 1000, 1000), (33, 17, 200, 1), (129, 130, 777, 64), (5, 300, 4096, 128),
              (256, 256, 4096, 300)]


@pytest.mark.parametrize("case", PARTITIONS, ids=[f"{m}x{n}x{k}-L{L}" for m, n, k, L in PARTITIONS])
@pytest.mark.parametrize("forms", [("dense", "dense"), ("t", "t"), ("gather", "t")], ids=["dense", "tt", "gather-t"])
def test_leaf_partition_vs_oracle(oracle, case, forms):
    m, n, k, L = case
    print(f"leaf ptr {case} {forms}", flush=True)
    rng = np.random.default_rng(m + n + k + L)
    A, ta = _operand(rng, m, k, forms[0])
    B, tb = _operand(rng, k, n, forms[1])
    P = (k + L - 1) // L
    c = _dev().gemm_leaf_ptr(ta, tb, leaf=L, p_count=P)
    torch.cuda.synchronize()
    _same(c.cpu().numpy(), oracle.gemm(A, B, 0, leaf=L), "cells")


def test_leaf_partition_refusals():
    a = torch.zeros((4, 10), device=DEV)
    b = torch.zeros((10, 3), device=DEV)
    for leaf, pc in ((3, 3), (3, 5), (0, 1), (10, 2)):
        with pytest.raises(RuntimeError, match="does not partition k"):
            _dev().gemm_leaf_ptr(a, b, leaf=leaf, p_count=pc)
    with pytest.raises(RuntimeError, match="store epilogue kind"):
        _dev().gemm_leaf_ptr(a, b, leaf=10, p_count=1, epi=1, epi_p=torch.zeros(3, device=DEV))


EPIS = [(3, 0), (4, 0), (4, 1), (4, 2), (4, 3), (4, 4), (5, 1), (5, 2), (5, 3), (5, 0)]


@pytest.mark.parametrize("epi,act", EPIS, ids=[f"epi{e}-act{a}" for e, a in EPIS])
def test_leaf_partition_followers(oracle, epi, act):
    m, n, k, L = 70, 90, 500, 128
    print(f"followers epi={epi} act={act}", flush=True)
    rng = np.random.default_rng(epi * 10 + act)
    A, ta = _operand(rng, m, k, "dense", 0.3)
    B, tb = _operand(rng, k, n, "dense", 0.3)
    p = (rng.standard_normal(n) if epi != 5 else rng.uniform(-1, 1, (m, n))).astype(np.float32)
    if epi == 5:
        p[0, :4] = [0.0, -0.0, 1.0, -1.0]
    c = _dev().gemm_leaf_ptr(ta, tb, leaf=L, p_count=(k + L - 1) // L, epi=epi,
                             epi_p=torch.from_numpy(p.ravel()).to(DEV), act=act)
    torch.cuda.synchronize()
    want = oracle.gemm(A, B, 0, leaf=L)
    oracle.epilogue(want, n, m, n, epi, p.ravel(), act)
    _same(c.cpu().numpy(), want, "cells")


def _wide_values(rng, count):
    x = (rng.standard_normal(count) * np.exp2(rng.uniform(-130, 8, count))).astype(np.float32)
    planted = np.array([0x00000000, 0x80000000, 0x7FC00000, 0xFFC00000, 0x7F800000, 0xFF800000, 0x00400000,
                        0x80400000, 0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF, 0x3F200000, 0x3F1FFFFF,
                        0x42317218, 0x42317219, 0xC2B00000, 0xC2B20000, 0x42B17218, 0x42B17300],
                       np.uint32).view(np.float32)
    extra = np.array([-100.0, -89.0, -88.0, 17.0, 100.0, 0.625, -0.625, 88.72, -87.33, 1e-20, -1e-20], np.float32)
    return np.concatenate([planted, extra, x])


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4])
def test_follower_activations_wide(oracle, act):
    """Kind 4 with a bias of -0.0 applies the activation to the flushed cell itself."""
    rng = np.random.default_rng(40 + act)
    x = _wide_values(rng, 1 << 20)
    n = 1024
    m = (x.size + n - 1) // n
    c = np.zeros(m * n, np.float32)
    c[:x.size] = x
    c = c.reshape(m, n)
    bias = np.full(n, -0.0, np.float32)
    tc = torch.from_numpy(c).to(DEV)
    _dev().follow(tc, 4, torch.from_numpy(bias).to(DEV), act)
    torch.cuda.synchronize()
    want = oracle.epilogue(c.copy(), n, m, n, 4, bias, act)
    _same(tc.cpu().numpy(), want, f"activation {act}")


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_follower_derivatives_wide(oracle, act):
    rng = np.random.default_rng(50 + act)
    d = _wide_values(rng, 1 << 18)
    z = np.concatenate([np.array([0.0, -0.0, 1.0, -1.0, 0.5], np.float32),
                        rng.uniform(-1, 1, d.size - 5).astype(np.float32)])
    z[5:40] = d[:35]  # specials as activations too
    m, n = 1, d.size
    td = torch.from_numpy(d.reshape(m, n).copy()).to(DEV)
    _dev().follow(td, 5, torch.from_numpy(z).to(DEV), act)
    torch.cuda.synchronize()
    want = oracle.epilogue(d.reshape(m, n).copy(), n, m, n, 5, z, act)
    _same(td.cpu().numpy(), want, f"derivative {act}")


LAYOUTS = [(70000, 4, 4, 0), (33, 1028, 1036, 0), (33, 1030, 1036, 0), (33, 1028, 1030, 0), (33, 1028, 1036, 1),
           (5, 3000, 3000, 0)]


@pytest.mark.parametrize("epi,act", [(4, 1), (5, 2), (3, 0)], ids=["bias-logistic", "tanh-bwd", "bias"])
@pytest.mark.parametrize("layout", LAYOUTS, ids=[f"{m}x{n}-ld{ld}-off{o}" for m, n, ld, o in LAYOUTS])
def test_follower_layouts(oracle, layout, epi, act):
    """The followers over views of every layout the launch distinguishes (more rows than one grid
    dimension holds; row strides above n, not a multiple of 4; a base off 16 bytes): every cell
    of the view against the oracle, every word outside it untouched."""
    m, n, ldc, off = layout
    print(f"follower layout {layout} epi={epi} act={act}", flush=True)
    rng = np.random.default_rng(m + n + ldc + off + epi)
    flat = (rng.standard_normal(off + m * ldc) * 4).astype(np.float32)
    p = (rng.standard_normal(n) if epi != 5 else rng.uniform(-1, 1, m * n)).astype(np.float32)
    tflat = torch.from_numpy(flat.copy()).to(DEV)
    view = tflat[off:].view(m, ldc)[:, :n]
    _dev().follow(view, epi, torch.from_numpy(p).to(DEV), act)
    torch.cuda.synchronize()
    want = flat.copy()
    body = np.ascontiguousarray(want[off:])
    oracle.epilogue(body, ldc, m, n, epi, p, act)
    want[off:] = body
    _same(tflat.cpu().numpy(), want, "buffer")


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4])
def test_fused_activation_store_wide(oracle, act):
    """Kind 4 fused into the product's store, on the wide value set: a one-step product
    (A = the values, B = [1]) makes each cell its own flushed value, the bias -0.0 leaves it."""
    rng = np.random.default_rng(60 + act)
    x = _wide_values(rng, 1 << 20)
    a = x.reshape(-1, 1).copy()
    b = np.ones((1, 1), np.float32)
    bias = np.full(1, -0.0, np.float32)
    c = _dev().gemm_leaf_ptr(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV), leaf=1, p_count=1, epi=4,
                             epi_p=torch.from_numpy(bias).to(DEV), act=act)
    torch.cuda.synchronize()
    want = oracle.gemm(a, b, 0, leaf=1)
    oracle.epilogue(want, 1, a.shape[0], 1, 4, bias, act)
    _same(c.cpu().numpy(), want, f"fused activation {act}")


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_fused_derivative_store_wide(oracle, act):
    rng = np.random.default_rng(70 + act)
    d = _wide_values(rng, 1 << 18)
    z = np.concatenate([np.array([0.0, -0.0, 1.0, -1.0, 0.5], np.float32),
                        rng.uniform(-1, 1, d.size - 5).astype(np.float32)])
    z[5:40] = d[:35]
    a = d.reshape(-1, 1).copy()
    b = np.ones((1, 1), np.float32)
    c = _dev().gemm_leaf_ptr(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV), leaf=1, p_count=1, epi=5,
                             epi_p=torch.from_numpy(z).to(DEV), act=act)
    torch.cuda.synchronize()
    want = oracle.gemm(a, b, 0, leaf=1)
    oracle.epilogue(want, 1, a.shape[0], 1, 5, z, act)
    _same(c.cpu().numpy(), want, f"fused derivative {act}")


def test_fused_store_is_one_launch():
    """mlg_gemm_leaf_ptr_epi with an activation follower dispatches the product kernel alone
    (no follower pass) when the leaves fold in one tile."""
    from mojolearn_amd import device as D
    assert D.route(2048, 4096, 4096, leaf=4096, num_cus=256) == {"tile"}
