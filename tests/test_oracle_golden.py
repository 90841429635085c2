"""The CPU oracle against the reference's own recorded outputs (no GPU).

1. The host-capped oracle card (20 shapes, 16M MACs each) recorded by the reference's
   `gemm_oracle` (bench/results/e1/2026-08-28_131651-runpod-nvidia/lanes/gemm.identical.card):
   every input hash and every output hash, for the scalar oracle and the fast arm.
2. The device card (MI325X, byte-identical to NVIDIA): input hashes of every row, and the
   output hashes of the rows small enough for the CPU suite (the full-shape rows are checked
   against the GPU kernel in tests/test_gpu_parity.py).
3. The verify table's gemm-pinned / gemm-transposed / gemm-bf16 `train` hashes on all nine
   fixtures (python/mojolearn/verify_reference/table.json), including the denormal fixtures.
"""
import numpy as np
import pytest

import cards
import verify_lanes as VL

HOST_CARD = cards.parse_card("host_oracle.card")
DEVICE_CARD = cards.parse_card("device_mi325x.card")


def _inputs(O, i, m, n, k, op):
    sa, sb = cards.operand_shapes(m, n, k, op)
    return O.card_fill(m * k, 11 + i).reshape(sa), O.card_fill(n * k, 22 + i).reshape(sb)


@pytest.mark.parametrize("i", range(len(cards.SHAPES)), ids=[s[0] for s in cards.SHAPES])
def test_host_card_row(oracle, i):
    name, m0, n0, k, op = cards.SHAPES[i]
    m, n = cards.host_capped(m0, n0, k)
    a, b = _inputs(oracle, i, m, n, k, op)
    assert (a.size, oracle.fnv1a64(a)) == HOST_CARD[name + ".in.a"]
    assert (b.size, oracle.fnv1a64(b)) == HOST_CARD[name + ".in.b"]
    c = oracle.gemm(a, b, op)
    assert (c.size, oracle.fnv1a64(c)) == HOST_CARD[name + ".out"]
    cf = oracle.gemm_fast(a, b, op)
    assert np.array_equal(c.view(np.uint32), cf.view(np.uint32))


@pytest.mark.parametrize("row", cards.device_rows(), ids=[r[1] for r in cards.device_rows()])
def test_device_card_row(oracle, row):
    i, name, m, n, k, op = row
    a, b = _inputs(oracle, i, m, n, k, op)
    assert (a.size, oracle.fnv1a64(a)) == DEVICE_CARD[name + ".in.a"]
    assert (b.size, oracle.fnv1a64(b)) == DEVICE_CARD[name + ".in.b"]
    if m * n * k > 300_000_000:
        pytest.skip("full-shape output checked against the GPU kernel (tests/test_gpu_parity.py)")
    c = oracle.gemm_fast(a, b, op)
    assert (c.size, oracle.fnv1a64(c)) == DEVICE_CARD[name + ".out"]


def test_device_card_equals_nvidia_card():
    nv = cards.parse_card("device_nvidia.card")
    assert nv == DEVICE_CARD


@pytest.mark.parametrize("kind", VL.FIXTURES)
def test_verify_fixture_hash(kind):
    X = VL.fixture_x(kind)
    assert VL.h(X) == VL.golden()["fixtures"][kind]


@pytest.mark.parametrize("kind", VL.FIXTURES)
def test_verify_gemm_lanes(oracle, kind):
    X = VL.fixture_x(kind)
    S = VL.OracleSurface(oracle)
    cells = VL.golden()["cells"]
    assert VL.train_hash(VL.lane_gemm_pinned(S.matmul, X)) == cells[f"gemm-pinned/{kind}"]["train"]
    assert VL.train_hash(VL.lane_gemm_transposed(S.matmul, X)) == cells[f"gemm-transposed/{kind}"]["train"]
    assert VL.train_hash(VL.lane_gemm_bf16(S.to_bf16, S.matmul_bf16, X)) == cells[f"gemm-bf16/{kind}"]["train"]
    lane = VL.lane_gemm_int8(S.quantize_int8, S.matmul_int8, S.dequantize_int8, X)
    assert VL.train_hash(lane) == cells[f"gemm-int8/{kind}"]["train"]
    lane = VL.lane_gemm_int15(S.quantize_int15, S.matmul_int15, S.dequantize_int15, oracle.INT15_MAX_K, X)
    assert VL.train_hash(lane) == cells[f"gemm-int15/{kind}"]["train"]


@pytest.mark.parametrize("kind", VL.FIXTURES)
def test_verify_lowbit_conversions_lane(oracle, kind, monkeypatch):
    """The lowbit-conversions cells with the storage module's conversions answered by the oracle:
    pins the module's object logic (predicates, refusals, ranks) and the oracle's conversions."""
    from mojolearn_amd import lowbit
    monkeypatch.setattr(lowbit, "_linalg", VL.OracleConversions(oracle))
    X = VL.fixture_x(kind)
    lane = VL.lane_lowbit_conversions(lowbit, oracle.bf16_widen, oracle, X)
    assert VL.train_hash(lane) == VL.golden()["cells"][f"lowbit-conversions/{kind}"]["train"]
