"""The parity gates can fail: each planted mistake of the oracle (oracle/gemm_oracle.c,
ORC_SABOTAGE, built as oracle/_sabotage/liboracle_s<n>.so) moves the answer of at least one of
the GPU family cases (tests/families.py).

Why that shows the GPU gate can fail: tests/test_gpu_families.py requires the kernels' words to
equal the honest oracle's.  A kernel that made one of these mistakes computes what the variant
computes, so on the case named here its words differ from the honest oracle's and that GPU test
fails.  The mistakes are planted in the oracle, on the CPU; no kernel is ever built wrong.  (The
reference shows its gates able to fail with compile-time sabotage of each gate,
gemm/checks/gemm_identical.mojo:213-264, run beside the honest build, pixi.toml:1004-1017.)

Also: the oracle's own pins (tests/test_oracle_pins.py) fail under the mistakes they exist for.
"""
import os
import subprocess

import numpy as np
import pytest

import families as F
import test_oracle_pins as PINS

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_DIR = os.path.join(os.path.dirname(HERE), "oracle")

#: mistakes that change the product's words (13 is orc_host_rows's own, checked below)
PRODUCT_MISTAKES = list(range(1, 13))


@pytest.fixture(scope="module")
def variants(oracle):
    subprocess.run(["make", "-s", "-j8", "-C", ORACLE_DIR, "sabotage"], check=True)
    return {n: oracle.sabotage_path(n) for n in oracle.SABOTAGE}


@pytest.fixture(scope="module")
def cases():
    # the register-stack cases are the families' largest products; the small tile cases reach
    # the same arithmetic
    cs = [c for c in F.all_cases() if c.family != "tile_stack"]
    cs.sort(key=lambda c: c.m * c.n * c.k)
    return cs


def _words(x):
    return np.ascontiguousarray(x).view(np.uint32)


@pytest.mark.parametrize("n", PRODUCT_MISTAKES, ids=lambda n: f"s{n}")
def test_some_family_case_catches(oracle, variants, cases, n):
    caught = None
    for case in cases:
        want = case.want(oracle)
        with oracle.using(variants[n]):
            moved = case.want(oracle)
        case.release()
        if not np.array_equal(_words(want), _words(moved)):
            caught = case
            break
    assert caught is not None, f"planted mistake {n} ({oracle.SABOTAGE[n]}) moves no family case"
    print(f"SABOTAGE s{n} {oracle.SABOTAGE[n]}: first failing case {caught.id} "
          f"(family {caught.family}, {caught.m}x{caught.n}x{caught.k})")


def _fails(oracle, path, fn, *args):
    with oracle.using(path):
        try:
            fn(oracle, *args)
        except AssertionError:
            return True
    return False


def test_bias_pin_catches_unflushed_bias(oracle, variants):
    assert _fails(oracle, variants[10], PINS.test_bias_against_numpy_words)
    assert _fails(oracle, variants[10], PINS.test_bias_planted_cells)


def test_dequant_pin_catches_unflushed_scale(oracle, variants):
    assert _fails(oracle, variants[11], PINS.test_int8_dequant_against_numpy, 0)
    assert _fails(oracle, variants[11], PINS.test_int8_dequant_against_numpy, 1)


def test_host_rows_pin_catches_no_redo(oracle, variants):
    """The fast column's negative control (gemm/host/gemm_host_rows.mojo:84-87): without the
    redo of the deferred flush, the planted-subnormal products differ from orc_gemm."""
    assert _fails(oracle, variants[13], PINS.test_host_rows_equals_oracle, (40, 100, 1000), 0)
    assert _fails(oracle, variants[13], PINS.test_host_rows_equals_oracle, (3, 33, 1000), 1) is False  # m <= 4: no deferral


def test_honest_oracle_passes_the_same_pins(oracle):
    PINS.test_bias_against_numpy_words(oracle)
    PINS.test_int8_dequant_against_numpy(oracle, 0)
    PINS.test_host_rows_equals_oracle(oracle, (40, 100, 1000), 0)


def test_family_plants_hold_on_the_oracle(oracle):
    """Every planted fixture cell of the family cases holds its closed-form word on the oracle
    (the tile_stack copies of these products differ only in their column count)."""
    checked = 0
    for case in F.kat_cases():
        if case.family == "tile_stack":
            continue
        w = _words(case.want(oracle))
        for r, c, word in case.plants:
            assert w[r, c] == word, (case.id, r, c, hex(int(w[r, c])), hex(int(word)))
            checked += 1
        case.release()
    assert checked > 300
