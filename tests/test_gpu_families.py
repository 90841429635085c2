"""The closed-form fixtures and the smallest-normal boundary words through every kernel family
(tests/families.py), on the GPU through the C ABI, against the oracle, bit for bit -- the
decode-packed int8 product (family `packed`) through its own entry.

Every output is pre-filled with the reference's poison word -987654.0 (gemm/checks/
gemm_device_check.mojo:111,535-556), so a cell a kernel leaves unwritten fails; every case first
asserts, through mlg_gemm_route, that the product does reach the family it is written for
(gemm_device_check.mojo:840-1008 runs its cases through every plan the same way); a planted
fixture cell must also hold its closed-form word (tests/kat.py).
"""
import numpy as np
import pytest

import families as F

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
CASES = F.all_cases()


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _route_name(case):
    return {"tile": "tile", "tile_stack": "tile_stack", "gemv_nn": "gemv_nn", "gemv_nt": "gemv_nt",
            "mfma4": "mfma4", "mfma16": "mfma16"}[case.family]


def run_gpu(case):
    from mojolearn_amd import device as D
    ta, tb = _t(case.a), _t(case.b.view(np.int16) if case.wt == "bf16" else case.b)
    out = torch.full((case.m, case.n), float(F.POISON), dtype=torch.float32, device=DEV)
    bias = None if case.bias is None else _t(case.bias)
    if case.family == "packed":
        D.gemv_int8w_packed(ta, D.pack_int8w(tb), _t(case.scales), bias=bias, out=out)
    elif case.wt == "f32":
        D.gemm(ta, tb, op=case.op, bias=bias, out=out, leaf=case.leaf)
    elif case.wt == "bf16":
        D.gemm_bf16w(ta, tb, op=case.op, bias=bias, out=out, leaf=case.leaf)
    else:
        D.gemm_int8w(ta, tb, _t(case.scales), op=case.op, bias=bias, out=out, leaf=case.leaf)
    torch.cuda.synchronize()
    return ta, tb, out.cpu().numpy()


@pytest.mark.parametrize("case", CASES, ids=[c.id for c in CASES])
def test_family_case(oracle, case):
    from mojolearn_amd import device as D
    print(f"family case {case.id}: m={case.m} n={case.n} k={case.k} op={case.op} wt={case.wt}", flush=True)
    try:
        ta, tb, got = run_gpu(case)
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        route = D.route(case.m, case.n, case.k, op=case.op, b_type=case.b_type, leaf=case.leaf, a=ta, b=tb)
        if case.family == "packed":
            pass  # its own entry, one kernel
        elif case.family != "tile_stack" or cus == 256:
            assert _route_name(case) in route, (case.family, route)
        want = case.want(oracle)
        g, w = got.view(np.uint32), want.view(np.uint32)
        bad = np.flatnonzero(g.ravel() != w.ravel())
        if bad.size:
            i = bad[0]
            raise AssertionError(f"{case.id}: {bad.size} of {g.size} words differ; first at ({i // case.n}, "
                                 f"{i % case.n}): got {g.ravel()[i]:#010x} want {w.ravel()[i]:#010x}")
        for r, c, word in case.plants:
            assert g[r, c] == word, (case.id, r, c, hex(int(g[r, c])), hex(int(word)))
    finally:
        case.release()
