"""The identity-card shape table and card files, restated for the tests.

Shape table: bench/gemm_shapes.mojo:146-275 (names, m, n, k, orientation).  The table
numbers its orientations NT=0, TN=1, NN=2; the contract numbers them NN=0, NT=1, TN=2
(gemm/contract.mojo:252-256).  `bench/gemm_card_main.mojo:314-358` maps one to the
other; the entries below already carry the contract's code.

Inputs of row i: A and B are `card_fill(count, salt)` with salts 11+i and 22+i
(bench/gemm_card_main.mojo:682-692), A holding m*k and B n*k values in the layout of
the row's orientation.  Host cards cap m and n to 16M MACs by halving the larger
(bench/gemm_card_main.mojo:361-378); device cards record the capped counts, from which
m and n are recovered here.
"""
import os

OP_NN, OP_NT, OP_TN = 0, 1, 2
HOST_MAC_BUDGET = 16_000_000

SHAPES = [
    ("gram.32x32x1M", 32, 32, 1_000_000, OP_TN),
    ("gram.32x32x64K", 32, 32, 65_536, OP_TN),
    ("gram.128sq.x100003", 128, 128, 100_003, OP_TN),
    ("ols.step1.16x16x64K", 16, 16, 65_536, OP_TN),
    ("pca.transform.8192x4x4", 8192, 4, 4, OP_NT),
    ("pca.transform.wide.8192x64x128", 8192, 64, 128, OP_NT),
    ("kmeans.dist.4096x64x64", 4096, 64, 64, OP_NT),
    ("ols.predict.gemv.64Kx16", 65536, 1, 16, OP_NT),
    ("llama8b.qkv.t1", 1, 4096, 4096, OP_NT),
    ("llama8b.qkv.t8", 8, 4096, 4096, OP_NT),
    ("llama8b.qkv.t512", 512, 4096, 4096, OP_NT),
    ("llama8b.mlp_up.t1", 1, 14336, 4096, OP_NT),
    ("llama8b.mlp_up.t8", 8, 14336, 4096, OP_NT),
    ("llama8b.mlp_up.t512", 512, 14336, 4096, OP_NT),
    ("llama8b.mlp_down.t1", 1, 4096, 14336, OP_NT),
    ("llama8b.mlp_down.t8", 8, 4096, 14336, OP_NT),
    ("llama8b.mlp_down.t512", 512, 4096, 14336, OP_NT),
    ("llama8b.lm_head.t1", 1, 128256, 4096, OP_NT),
    ("llama8b.lm_head.t8", 8, 128256, 4096, OP_NT),
    ("llama8b.lm_head.t512", 512, 128256, 4096, OP_NT),
]

CARD_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cards")


def host_capped(m, n, k, budget=HOST_MAC_BUDGET):
    """bench/gemm_card_main.mojo:361-378: halve the larger of m, n until m*n*k fits."""
    while m * n * k > budget and (m > 1 or n > 1):
        if n >= m and n > 1:
            n = (n + 1) // 2
        elif m > 1:
            m = (m + 1) // 2
        else:
            break
    return m, n


def parse_card(name):
    """{tag: (count, hash_int)} of a `mojolearn-identity-trace v1` card."""
    out = {}
    with open(os.path.join(CARD_DIR, name)) as fh:
        for line in fh:
            if line.startswith("#") or not line.strip():
                continue
            seq, tag, dtype, count, h = line.rstrip("\n").split("\t")
            assert dtype == "f32"
            out[tag] = (int(count), int(h, 16))
    return out


def device_rows():
    """(index, name, m, n, k, op) of every device-card row, m and n from its counts."""
    card = parse_card("device_mi325x.card")
    rows = []
    for i, (name, m0, n0, k, op) in enumerate(SHAPES):
        ca = card[name + ".in.a"][0]
        co = card[name + ".out"][0]
        m = ca // k
        n = co // m
        assert m * k == ca and m * n == co and card[name + ".in.b"][0] == n * k
        rows.append((i, name, m, n, k, op))
    return rows


def operand_counts(m, n, k, op):
    return m * k, n * k


def operand_shapes(m, n, k, op):
    """Row-major shapes of (A, B) for the contract op."""
    if op == OP_TN:
        return (k, m), (k, n)
    if op == OP_NT:
        return (m, k), (n, k)
    return (m, k), (k, n)
