"""Cases that send the closed-form fixtures and the smallest-normal boundary words through every
kernel family of the product, for tests/test_gpu_families.py (the GPU against the oracle, on
poisoned outputs) and tests/test_sabotage.py (each planted mistake in the oracle moves the
answer of at least one of these cases).

Kernel families (mojolearn_amd/csrc/kernels.hip run_gemm; `route` names them):
  tile        gemm_mfma_kernel, m >= 17 or OP_TN; its leaves split into groups folded by
              fold_groups_kernel when the grid has fewer tiles than CUs (`fold`), or a tile
              folding all its leaves in its own register stack (`tile_stack`) when it has
              at least as many tiles as CUs
  gemv_nn     gemv_nn_kernel, OP_NN with 1 <= m <= 16 float32 rows
  gemv_nt     gemv_nt_kernel, OP_NT with 1 <= m <= 16
  mfma4       gemv_mfma4_nn_kernel, OP_NN, 3 <= m <= 8, leaves of exactly 128 rows
  mfma16      gemv_mfma_nn_kernel, OP_NN, 9 <= m <= 16, leaves of exactly 128 rows

Inputs:
  * the closed-form fixtures F1-F8 and inf/NaN of tests/kat.py (each one cell, a[k] . b[k]),
    planted at (row, column) positions of products with normal filler elsewhere; the planted
    cells must hold the fixture's closed-form word, every cell the oracle's word.  The skinny
    matrix-core kernels need leaves of 128 rows, so there a fixture whose k is not a multiple
    of 128 is padded with zeros to the next multiple (its closed form is then checked only
    through the oracle);
  * the 64 adversarial words of the reference's smallest-normal boundary check
    (gemm/checks/gemm_rtf_boundary_check.mojo:53-64): all 64 x 64 pairs at k = 1 (or as the
    last step of a 128-step leaf whose other steps are zero), pseudo-random draws from the words
    at several k (:247-259 and k in {16, 129, 300, 4097}), the planted products exactly at the
    window's edge 2^-126 - 2^-150 (:313-334), the admitted and mixed controls and the four
    operand kinds of the admission A/B (:261-312), with float32, bf16-stored and int8-stored
    weights (int8 scales drawn from the words: subnormal, tiny, huge).
"""
import numpy as np

import kat

POISON = np.float32(-987654.0)
U32, F32 = np.uint32, np.float32
M64 = (1 << 64) - 1
M32 = (1 << 32) - 1


def boundary_words():
    """gemm/checks/gemm_rtf_boundary_check.mojo:53-64: 22 literal words, then 42 from an LCG."""
    w = [0, 0x80000000, 1, 0x80000001, 0x007fffff, 0x807fffff, 0x00800000, 0x80800000, 0x00800001,
         0x80800001, 0x3f000000, 0xbf000000, 0x3f800000, 0xbf800000, 0x3f800001, 0xbf800001, 0x3f7fffff,
         0xbf7fffff, 0x7f7fffff, 0xff7fffff, 0x4b800001, 0xcb800001]
    seed = 0x9A718BCD
    for _ in range(42):
        seed = (seed * 1664525 + 1013904223) & M32
        w.append(seed & 0xFEFFFFFF)
    return np.array(w, U32).view(F32)


def mix64(x):
    """The splitmix64 finalizer the boundary check draws its word indices with (:67-72)."""
    z = (x + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _mix64_np(x):
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _mix32_np(x):
    x = np.asarray(x, dtype=np.uint64) & np.uint64(M32)
    h = (x * np.uint64(0x9E3779B1)) & np.uint64(M32)
    h ^= h >> np.uint64(15)
    h = (h * np.uint64(0x85EBCA77)) & np.uint64(M32)
    h ^= h >> np.uint64(13)
    h = (h * np.uint64(0xC2B2AE3D)) & np.uint64(M32)
    return h ^ (h >> np.uint64(16))


def kind_words(count, seed, kind):
    """gemm_rtf_boundary_check.mojo:81-101 `_kind_word`: 0 ordinary, 2 mixed, 3 skew's A,
    4 border, 5 sparse."""
    i = np.arange(count, dtype=np.uint64)
    h = _mix32_np(i ^ _mix32_np(np.uint64(seed)))
    h2 = _mix32_np(h ^ np.uint64(0x5BD1E995))
    sign = h & np.uint64(0x80000000)
    mant = h & np.uint64(0x007FFFFF)
    e = np.uint64(119) + h2 % np.uint64(9)
    if kind == 2:
        e = np.where((h2 >> np.uint64(26)) == 0, np.uint64(17) + h2 % np.uint64(10), e)
    elif kind == 3:
        e = np.uint64(2) + h2 % np.uint64(11)
    elif kind == 4:
        e = np.uint64(87) + h2 % np.uint64(7)
    elif kind == 5:
        e = np.where((h2 >> np.uint64(20)) == 0, np.uint64(17) + h2 % np.uint64(10), e)
    return (sign | (e << np.uint64(23)) | mant).astype(U32).view(F32)


def _draw(count, salt_mul, salt_add, s):
    w = boundary_words()
    idx = _mix64_np(np.arange(count, dtype=np.uint64) * np.uint64(salt_mul) + np.uint64(salt_add + s)) % np.uint64(64)
    return w[idx.astype(np.int64)]


# ---------------------------------------------------------------------------------------------
# a case

class Case:
    """One product: C = op(A) . op(B_eff) (+ bias), B_eff the float32 `b`, the bf16 bits `b`
    widened, or the int8 codes `b` times `scales`, in the stored layouts of `op`.  `a` and `b`
    may instead be given by `make`, a function returning (a, b), called on first use (so that
    collecting the cases holds no large operand)."""

    def __init__(self, cid, family, op, a=None, b=None, wt="f32", scales=None, leaf=0, bias=None, plants=(),
                 make=None, shape=None):
        self.id, self.family, self.op = cid, family, op
        self._a, self._b, self._make = a, b, make
        self.wt, self.scales, self.leaf, self.bias = wt, scales, leaf, bias
        self.plants = list(plants)  # (row, col, expected word)
        if shape is not None:
            self.m, self.n, self.k = shape
        elif op == 0:
            (self.m, self.k), self.n = a.shape, b.shape[1]
        elif op == 1:
            (self.m, self.k), self.n = a.shape, b.shape[0]
        else:
            (self.k, self.m), self.n = a.shape, b.shape[1]

    def _load(self):
        if self._a is None:
            self._a, self._b = self._make()

    @property
    def a(self):
        self._load()
        return self._a

    @property
    def b(self):
        self._load()
        return self._b

    def release(self):
        """Drop operands that `make` built (they are rebuilt on the next use)."""
        if self._make is not None:
            self._a = self._b = None

    @property
    def b_type(self):
        return {"f32": 0, "bf16": 1, "i8": 2}[self.wt]

    def b_eff(self, O):
        if self.wt == "f32":
            return self.b
        if self.wt == "bf16":
            return O.bf16_widen(self.b)
        return O.int8_dequant(self.b, self.scales, self.op)

    def want(self, O):
        """The oracle's words (NaN canonicalized, as the product stores them)."""
        y = O.gemm_fast(self.a, self.b_eff(O), self.op, leaf=self.leaf)
        if self.bias is not None:
            y = O.bias(y, self.bias)
        return O.nan_canon(y)


def _filler(rng, shape):
    return rng.standard_normal(shape).astype(F32)


def _stored(A, B, op):
    """A (m x k) and B (k x n) in the stored layouts of `op`."""
    a = A if op != 2 else np.ascontiguousarray(A.T)
    b = B if op != 1 else np.ascontiguousarray(B.T)
    return np.ascontiguousarray(a), np.ascontiguousarray(b)


# Family shapes: (family, op, m, n).  `tile_stack` has as many column tiles as CUs.
def family_shapes(cus=256):
    return [("tile", 0, 24, 128), ("tile", 1, 24, 128), ("tile", 2, 24, 128),
            ("tile_stack", 0, 17, 128 * cus + 1),
            ("gemv_nn", 0, 1, 64), ("gemv_nn", 0, 2, 70), ("gemv_nt", 1, 1, 70), ("gemv_nt", 1, 16, 70),
            ("mfma4", 0, 4, 300), ("mfma16", 0, 16, 300)]


def _kat_groups():
    """kat.fixtures() grouped by (k, leaf)."""
    groups = {}
    for name, a, b, leaf, want in kat.fixtures():
        groups.setdefault((a.size, leaf), []).append((name, a, b, np.uint32(want)))
    return groups


def kat_cases(cus=256):
    out = []
    for (k, leaf), fxs in sorted(_kat_groups().items()):
        P = -(-k // (leaf if leaf > 0 else (k if k <= 128 else 128)))
        for family, op, m, n in family_shapes(cus):
            matrix = family in ("mfma4", "mfma16")
            if matrix and leaf not in (0, 128):
                continue
            if family == "tile_stack" and (P < 2 or leaf != 0):
                continue  # the register stack needs more than one leaf in a tile
            kp = -(-k // 128) * 128 if matrix else k
            padded = kp != k
            for c0 in range(0, len(fxs), m):
                chunk = fxs[c0:c0 + m]
                assert 2 + 4 * (len(chunk) - 1) < n  # one column per fixture
                plants = [(t, 2 + 4 * t, want) for t, (_, _, _, want) in enumerate(chunk)] if not padded else []

                def make(chunk=chunk, seed=k * 131 + c0 + op + m, m=m, n=n, k=k, kp=kp, op=op):
                    rng = np.random.default_rng(seed)
                    A = _filler(rng, (m, kp))
                    B = _filler(rng, (kp, n))
                    for t, (_, fa, fb, _) in enumerate(chunk):
                        col = 2 + 4 * t
                        A[t] = 0.0
                        B[:, col] = 0.0
                        A[t, :k] = fa
                        B[:k, col] = fb
                    return _stored(A, B, op)
                names = ",".join(f[0] for f in chunk) if len(chunk) <= 3 else f"{chunk[0][0]}..{chunk[-1][0]}"
                out.append(Case(f"kat-{family}-op{op}-m{m}-k{k}{'p' + str(kp) if padded else ''}-L{leaf}-{names}",
                                family, op, leaf=leaf, plants=plants, make=make, shape=(m, n, kp)))
    return out


def _weights(rng, wt, B, op, words_scales):
    """The weight operand of kind `wt` from a float32 B (k x n), stored for `op` (OP_TN's B is
    k x n like OP_NN's)."""
    k, n = B.shape
    stored = np.ascontiguousarray(B.T) if op == 1 else B
    if wt == "f32":
        return stored, None
    if wt == "bf16":
        import oracle.oracle as O  # the oracle's L-2 narrowing builds the stored bits
        return O.bf16_narrow(stored), None
    codes = rng.integers(-127, 128, stored.shape, dtype=np.int8)
    return codes, np.ascontiguousarray(words_scales[:n])


def _scale_words(rng, n):
    """int8 column scales drawn from the adversarial words (finite, non-NaN): subnormal scales
    flush, tiny ones flush their products, FLT_MAX-sized ones overflow them."""
    w = boundary_words()
    finite = w[np.isfinite(w)]
    s = finite[rng.integers(0, finite.size, n)]
    s[: min(n, 8)] = np.array([1e-3, 5e-3, 2.0 ** -126, -2.0 ** -126, 2.0 ** -120, 3e38, -1e-2, 0.0],
                              F32)[: min(n, 8)]
    return s.astype(F32)


def boundary_cases(cus=256):
    out = []
    w = boundary_words()
    # all 64 x 64 pairs, k = 1, accumulator +0
    for op in (0, 1, 2):
        A = w.reshape(64, 1).copy()
        B = w.reshape(1, 64).copy()
        a, b = _stored(A, B, op)
        out.append(Case(f"pairs-tile-op{op}", "tile", op, a, b))
    for family, op, m in (("gemv_nn", 0, 16), ("gemv_nt", 1, 16), ("gemv_nn", 0, 1)):
        rows = range(0, 64, m) if m > 1 else range(0, 4)
        for r0 in rows:
            A = w[r0:r0 + m].reshape(m, 1).copy()
            a, b = _stored(A, w.reshape(1, 64).copy(), op)
            out.append(Case(f"pairs-{family}-m{m}-rows{r0}", family, op, a, b))
    # the pair as the last step of a 128-step leaf whose other steps are zero
    for family, m in (("mfma4", 4), ("mfma16", 16)):
        for r0 in range(0, 64, m if m == 16 else 16):
            A = np.zeros((m, 128), F32)
            A[:, 127] = w[r0:r0 + m]
            B = np.zeros((128, 64), F32)
            B[127] = w
            out.append(Case(f"pairs-{family}-rows{r0}", family, 0, A, B))
    # pseudo-random draws from the words
    tile_shapes = [(130, 130, 2), (130, 131, 3), (129, 200, 17), (260, 130, 40), (64, 64, 300), (40, 70, 16),
                   (33, 65, 129), (20, 40, 4097)]
    for s, (m, n, k) in enumerate(tile_shapes):
        A = _draw(m * k, 7, 0, s).reshape(m, k)
        B = _draw(k * n, 13, 1000, s).reshape(k, n)
        for op in (0, 1, 2):
            a, b = _stored(A, B, op)
            out.append(Case(f"draw{s}-tile-op{op}-{m}x{n}x{k}", "tile", op, a, b))
    skinny = [("gemv_nn", 0, m, k) for m in (1, 2, 16) for k in (16, 129, 300, 4097)]
    skinny += [("gemv_nt", 1, m, k) for m in (1, 16) for k in (16, 129, 300, 4097)]
    skinny += [("mfma4", 0, 4, k) for k in (128, 256, 4096)] + [("mfma16", 0, 16, k) for k in (128, 256, 4096)]
    for s, (family, op, m, k) in enumerate(skinny):
        n = 300 if op == 0 else 100
        A = _draw(m * k, 7, 0, 100 + s).reshape(m, k)
        B = _draw(k * n, 13, 1000, 100 + s).reshape(k, n)
        a, b = _stored(A, B, op)
        out.append(Case(f"draw-{family}-m{m}-k{k}", family, op, a, b))
    # the same draws with bf16- and int8-stored weights (the tile kernel and the skinny ones)
    weighted = [("tile", 0, 64, 96, 300), ("tile", 1, 64, 96, 300), ("tile", 0, 40, 70, 4097),
                ("gemv_nn", 0, 1, 300, 4097), ("gemv_nn", 0, 2, 300, 300), ("gemv_nt", 1, 1, 100, 4097),
                ("mfma4", 0, 4, 300, 4096), ("mfma16", 0, 16, 300, 1024)]
    for s, (family, op, m, n, k) in enumerate(weighted):
        rng = np.random.default_rng(900 + s)
        A = _draw(m * k, 7, 0, 200 + s).reshape(m, k)
        B = _draw(k * n, 13, 1000, 200 + s).reshape(k, n)
        a = np.ascontiguousarray(A)
        for wt in ("bf16", "i8"):
            b, scales = _weights(rng, wt, B, op, _scale_words(rng, n))
            out.append(Case(f"draw-{wt}-{family}-op{op}-m{m}-k{k}", family, op, a, b, wt=wt, scales=scales))
    # products exactly at the window's edge: (2 - 2^-23) 2^-64 * 2^-63 = 2^-126 - 2^-150, which
    # rounds to 2^-126 and only then meets the flush (:313-334)
    def planted(m, n, k):
        r, p = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
        A = np.where((r + p) % 7 == 0, np.array([0x1FFFFFFF], U32).view(F32)[0], F32(0.0)).astype(F32)
        p2, c = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
        B = np.where((p2 + 2 * c) % 5 == 0, np.array([0x20000000], U32).view(F32)[0], F32(0.0)).astype(F32)
        return A, B
    A, B = planted(64, 64, 256)
    for op in (0, 1, 2):
        a, b = _stored(A, B, op)
        out.append(Case(f"planted-tile-op{op}", "tile", op, a, b))
    for family, op, m in (("gemv_nn", 0, 1), ("gemv_nt", 1, 16), ("mfma4", 0, 4), ("mfma16", 0, 16)):
        a, b = _stored(np.ascontiguousarray(A[:m]), B, op)
        out.append(Case(f"planted-{family}-m{m}", family, op, a, b))
    # controls: ordinary magnitudes ("admitted") and the mixed windows (:261-297)
    m, n, k = 256, 256, 96
    idx = np.arange(m * k, dtype=np.uint64)
    A = (np.uint64(0x3F000000) | (_mix64_np(idx) & np.uint64(0x80FFFFFF))).astype(U32).view(F32).reshape(m, k)
    idx = np.arange(k * n, dtype=np.uint64)
    B = (np.uint64(0x3F000000) | (_mix64_np(idx + np.uint64(77777)) & np.uint64(0x80FFFFFF))).astype(U32)
    out.append(Case("admitted-tile", "tile", 0, np.ascontiguousarray(A), B.view(F32).reshape(k, n)))
    m, n, k = 192, 160, 640
    i = np.arange(m * k, dtype=np.uint64)
    p = (i % np.uint64(k)).astype(np.int64)
    hi = np.where((p // 16) % 5 == 2, np.uint64(0x0F000000), np.uint64(0x3F000000))
    A = (hi | (_mix64_np(i + np.uint64(555)) & np.uint64(0x80FFFFFF))).astype(U32).view(F32).reshape(m, k)
    i = np.arange(k * n, dtype=np.uint64)
    B = (np.uint64(0x3F000000) | (_mix64_np(i + np.uint64(999)) & np.uint64(0x80FFFFFF))).astype(U32)
    B = B.view(F32).reshape(k, n)
    out.append(Case("mixed-tile", "tile", 0, np.ascontiguousarray(A), B))
    out.append(Case("mixed-mfma16", "mfma16", 0, np.ascontiguousarray(A[:16]), B))
    # the admission A/B's operand kinds (:298-312) at k = 768
    m, n, k = 160, 192, 768
    for kd, kid in enumerate((2, 3, 4, 5)):
        A = kind_words(m * k, 1000 + 7 * kd, kid).reshape(m, k)
        B = kind_words(k * n, 2000 + 7 * kd, 0 if kid == 3 else kid).reshape(k, n)
        name = ("kmixed", "kskew", "kborder", "ksparse")[kd]
        out.append(Case(f"{name}-tile", "tile", 0, np.ascontiguousarray(A), B))
        for family, mm in (("gemv_nn", 1), ("mfma4", 4), ("mfma16", 16)):
            out.append(Case(f"{name}-{family}", family, 0, np.ascontiguousarray(A[:mm]), B))
    return out


def bias_cases():
    """The fused bias on the adversarial words in every family.  Every other column of B and
    the last row of A are zero, so those cells' products are exact +0 and meet the bias words
    (subnormal biases must flush: +0 + -tiny is +0, not -0)."""
    out = []
    w = boundary_words()
    rng = np.random.default_rng(4242)
    for family, op, m, n, k in (("tile", 0, 40, 70, 300), ("tile", 2, 40, 70, 300), ("gemv_nn", 0, 1, 300, 4097),
                                ("gemv_nt", 1, 2, 100, 300), ("mfma4", 0, 4, 300, 1024), ("mfma16", 0, 16, 300, 1024)):
        A = _draw(m * k, 7, 0, 300 + m + k).reshape(m, k)
        B = _draw(k * n, 13, 1000, 300 + m + k).reshape(k, n)
        B[:, 1::2] = 0.0
        if m > 1:
            A[-1] = 0.0
        a, b = _stored(A, B, op)
        bias = w[rng.integers(0, 64, n)].astype(F32)
        bias[1:9:2] = np.array([0x80000001, 0x807FFFFF, 0x00000001, 0x80400000], U32).view(F32)
        out.append(Case(f"bias-{family}-op{op}-m{m}", family, op, a, b, bias=bias))
    return out


def packed_cases(cus=256):
    """The decode-packed int8 product (family `packed`: int8 codes rearranged once, OP_NN, k a
    multiple of 128) on the adversarial words: x drawn from the boundary words, scales from the
    adversarial scale words, in whole-column workgroups (one group, and a second group holding
    one leaf) and in 4-leaf groups; the window's edge planted through the dequant (code 1 times
    the scale 2^-63 is the weight 2^-63); the admission A/B's operand kinds; the fused bias on
    the words."""
    out = []
    whole_n = 192 * 64 * 256 // cus  # ceil(n / 64) >= 3/4 of the CUs: whole-column workgroups
    shapes = [(1, whole_n, 4096), (1, whole_n + 12, 4224), (2, whole_n, 4096), (1, 300, 1024), (2, 300, 384),
              (16, 300, 1024), (4, 200, 4096)]
    for s, (m, n, k) in enumerate(shapes):
        def make(m=m, n=n, k=k, s=s):
            rng = np.random.default_rng(700 + s)
            return _draw(m * k, 7, 0, 400 + s).reshape(m, k), rng.integers(-128, 128, (k, n), dtype=np.int8)
        scales = _scale_words(np.random.default_rng(800 + s), n)
        out.append(Case(f"draw-packed-m{m}-n{n}-k{k}", "packed", 0, wt="i8", scales=scales, make=make,
                        shape=(m, n, k)))
    m, n, k = 1, 300, 256
    r, p = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
    A = np.where((r + p) % 7 == 0, np.array([0x1FFFFFFF], U32).view(F32)[0], F32(0.0)).astype(F32)
    p2, c = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    codes = np.where((p2 + 2 * c) % 5 == 0, 1, 0).astype(np.int8)
    out.append(Case("planted-packed-m1", "packed", 0, np.ascontiguousarray(A), codes, wt="i8",
                    scales=np.full(n, 2.0 ** -63, F32)))
    m, n, k = 16, 160, 768
    for kd, kid in enumerate((2, 3, 4, 5)):
        A = kind_words(m * k, 1000 + 7 * kd, kid).reshape(m, k)
        codes = np.random.default_rng(1500 + kd).integers(-128, 128, (k, n), dtype=np.int8)
        scales = np.random.default_rng(1600 + kd).uniform(1e-3, 1e-2, n).astype(F32)
        name = ("kmixed", "kskew", "kborder", "ksparse")[kd]
        for mm in (1, 16):
            out.append(Case(f"{name}-packed-m{mm}", "packed", 0, np.ascontiguousarray(A[:mm]), codes, wt="i8",
                            scales=scales))
    w = boundary_words()
    rng = np.random.default_rng(4343)
    for m, n, k in ((1, whole_n, 4096), (2, 300, 1024)):
        A = _draw(m * k, 7, 0, 500 + m + k).reshape(m, k)
        codes = rng.integers(-127, 128, (k, n), dtype=np.int8)
        codes[:, 1::2] = 0
        bias = w[rng.integers(0, 64, n)].astype(F32)
        bias[1:9:2] = np.array([0x80000001, 0x807FFFFF, 0x00000001, 0x80400000], U32).view(F32)
        out.append(Case(f"bias-packed-m{m}-n{n}", "packed", 0, np.ascontiguousarray(A), codes, wt="i8",
                        scales=_scale_words(rng, n), bias=bias))
    return out


def all_cases(cus=256):
    return kat_cases(cus) + boundary_cases(cus) + bias_cases() + packed_cases(cus)
