"""The five workloads at their real sizes on the GPU, bit for bit against the CPU oracle, every
cell of every output.

Each output buffer is first filled with the poison word -987654.0, so a cell no kernel writes
fails.  The oracle's fast arm (AVX2, every host thread) recomputes the whole product: about 1 s
for the prefill and the LM head and 5 s for the SwiGLU projection on 16 host threads.
"""
import numpy as np
import pytest

from mojolearn_amd import workloads as W

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"
POISON = -987654.0


def _rows(m, count=8):
    r = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).choice(m, count - 2, replace=False)]))
    return r


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def _out(m, n):
    return torch.full((m, n), POISON, dtype=torch.float32, device=DEV)


def _same(got, want):
    g, w = _bits(got), _bits(want)
    bad = np.flatnonzero(g.ravel() != w.ravel())
    assert bad.size == 0, (f"{bad.size} of {g.size} words differ; first at flat {bad[0]}: got {g.ravel()[bad[0]]:#010x} "
                           f"want {w.ravel()[bad[0]]:#010x}")


def test_gemm512_whole(oracle):
    from mojolearn_amd import device as D
    a, b = W.gemm512()
    c = D.gemm(_t(a), _t(b), out=_out(512, 512)).cpu().numpy()
    _same(c, oracle.gemm(a, b, 0))


def test_prefill_whole(oracle):
    from mojolearn_amd import device as D
    x, w, bias = W.prefill()
    y = D.gemm(_t(x), _t(w), bias=_t(bias), out=_out(x.shape[0], w.shape[1])).cpu().numpy()
    _same(y, oracle.nan_canon(oracle.bias(oracle.gemm_fast(x, w, 0), bias)))


@pytest.mark.parametrize("m", [1, 4, 16])
def test_decode_whole(oracle, m):
    from mojolearn_amd import device as D
    x16, codes, scales = W.decode()
    x = np.ascontiguousarray(x16[:m])
    y = D.gemm_int8w(_t(x), _t(codes), _t(scales), out=_out(m, codes.shape[1])).cpu().numpy()
    _same(y, oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0))


def test_swiglu_up_whole(oracle):
    from mojolearn_amd import device as D
    x, wbits = W.swiglu_up()
    y = D.gemm_bf16w(_t(x), _t(wbits.view(np.int16)), out=_out(x.shape[0], wbits.shape[1])).cpu().numpy()
    _same(y, oracle.gemm_fast(x, oracle.bf16_widen(wbits), 0))


def test_lm_head_whole(oracle):
    from mojolearn_amd import device as D
    x, w = W.lm_head()
    y = D.gemm(_t(x), _t(w), out=_out(x.shape[0], w.shape[1])).cpu().numpy()
    _same(y, oracle.nan_canon(oracle.gemm_fast(x, w, 0)))
    assert np.isnan(y).any()  # the adversarial magnitudes do produce inf - inf


@pytest.mark.parametrize("m", [1, 16])
def test_decode_column_shards_concatenate_to_the_whole(oracle, m):
    """A column split over 8 GPUs needs no arithmetic exchange: each GPU's N/8 columns (one
    launch each, at the shard's own shape) are the whole product's bits."""
    from mojolearn_amd import device as D
    x16, codes, scales = W.decode()
    x = np.ascontiguousarray(x16[:m])
    tx = _t(x)
    whole = D.gemm_int8w(tx, _t(codes), _t(scales)).cpu().numpy()
    step = codes.shape[1] // 8
    parts = [D.gemm_int8w(tx, _t(codes[:, s:s + step]), _t(scales[s:s + step])).cpu().numpy()
             for s in range(0, codes.shape[1], step)]
    assert np.array_equal(_bits(np.concatenate(parts, axis=1)), _bits(whole))
    want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0)
    assert np.array_equal(_bits(whole), _bits(want))


def test_prefill_column_shards_concatenate_to_the_whole(oracle):
    from mojolearn_amd import device as D
    x, w, bias = W.prefill()
    tx = _t(x)
    whole = D.gemm(tx, _t(w), bias=_t(bias)).cpu().numpy()
    step = w.shape[1] // 8
    parts = [D.gemm(tx, _t(w[:, s:s + step]), bias=_t(bias[s:s + step])).cpu().numpy()
             for s in range(0, w.shape[1], step)]
    assert np.array_equal(_bits(np.concatenate(parts, axis=1)), _bits(whole))
    rows = _rows(x.shape[0])
    want = oracle.nan_canon(oracle.bias(oracle.gemm_fast(x[rows], w[:, :step], 0), bias[:step]))
    assert np.array_equal(_bits(parts[0][rows]), _bits(want))
