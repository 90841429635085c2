"""The five workloads at their real sizes on the GPU, bit for bit against the CPU oracle.

The 512^3 product and the decode GEMVs are checked whole.  For the three large products the
oracle recomputes a sample of rows: a cell depends on its row of X, its column of W and k only
(never on m, the launch or the batch), so a row subset through the oracle is the same bits as
the whole product's rows.  All columns of each sampled row are checked.
"""
import numpy as np
import pytest

from mojolearn_amd import workloads as W

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _rows(m, count=8):
    r = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).choice(m, count - 2, replace=False)]))
    return r


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def test_gemm512_whole(oracle):
    from mojolearn_amd import device as D
    a, b = W.gemm512()
    c = D.gemm(_t(a), _t(b)).cpu().numpy()
    assert np.array_equal(_bits(c), _bits(oracle.gemm(a, b, 0)))


def test_prefill_rows(oracle):
    from mojolearn_amd import device as D
    x, w, bias = W.prefill()
    y = D.gemm(_t(x), _t(w), bias=_t(bias)).cpu().numpy()
    rows = _rows(x.shape[0])
    want = oracle.nan_canon(oracle.bias(oracle.gemm_fast(x[rows], w, 0), bias))
    assert np.array_equal(_bits(y[rows]), _bits(want))


@pytest.mark.parametrize("m", [1, 4, 16])
def test_decode_whole(oracle, m):
    from mojolearn_amd import device as D
    x16, codes, scales = W.decode()
    x = np.ascontiguousarray(x16[:m])
    y = D.gemm_int8w(_t(x), _t(codes), _t(scales)).cpu().numpy()
    want = oracle.gemm_fast(x, oracle.int8_dequant(codes, scales, 0), 0)
    assert np.array_equal(_bits(y), _bits(want))


def test_swiglu_up_rows(oracle):
    from mojolearn_amd import device as D
    x, wbits = W.swiglu_up()
    y = D.gemm_bf16w(_t(x), _t(wbits.view(np.int16))).cpu().numpy()
    rows = _rows(x.shape[0])
    want = oracle.gemm_fast(x[rows], oracle.bf16_widen(wbits), 0)
    assert np.array_equal(_bits(y[rows]), _bits(want))


def test_lm_head_rows(oracle):
    from mojolearn_amd import device as D
    x, w = W.lm_head()
    y = D.gemm(_t(x), _t(w)).cpu().numpy()
    rows = _rows(x.shape[0])
    want = oracle.nan_canon(oracle.gemm_fast(x[rows], w, 0))
    assert np.array_equal(_bits(y[rows]), _bits(want))
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
