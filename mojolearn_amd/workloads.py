"""The five synthetic workloads the identical-mode GEMM/GEMV is measured and checked on.

Inputs are NumPy PCG64 draws (`numpy.random.default_rng(seed)`), float32 unless stated:

  gemm512     C = A.B, 512^3, A and B uniform[-1, 1) from seed 0 (2*U - 1 in float32)
  prefill     X[2048x4096] ~ N(0,1), W[4096x4096] ~ N(0,0.02), bias[4096] ~ N(0,0.01), seed 1;
              Y = ftz(ftz(X.W) + ftz(bias))  (the LM's nn.Linear)
  decode      X[Mx4096] ~ N(0,1) (the first M rows of one 16-row draw), W int8 codes[4096x14336]
              uniform in [-127,127], per-output-channel scales uniform in [1e-3,1e-2], seed 2;
              W_eff = ftz(f32(code) * ftz(scale[j])), M in {1, 4, 16}
  swiglu_up   X[4096x4096] ~ N(0,1), W = bf16 of N(0,0.02)[4096x11008] (ftz then RNE), seed 3
  lm_head     X[512x2048], W[2048x50304]: magnitudes 10^U(-30,30) with random sign, then 1% of
              positions a random subnormal and another disjoint 1% a signed zero, seed 4

All products are OP_NN in these layouts (X[M x K] . W[K x N]).
"""
import numpy as np

f32 = np.float32


def gemm512():
    rng = np.random.default_rng(0)
    a = (f32(2) * rng.random((512, 512), dtype=f32) - f32(1)).astype(f32)
    b = (f32(2) * rng.random((512, 512), dtype=f32) - f32(1)).astype(f32)
    return a, b


def prefill():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2048, 4096), dtype=f32)
    w = (rng.standard_normal((4096, 4096), dtype=f32) * f32(0.02)).astype(f32)
    bias = (rng.standard_normal(4096, dtype=f32) * f32(0.01)).astype(f32)
    return x, w, bias


def decode():
    """(x16, codes, scales); the M-row workload uses x16[:M]."""
    rng = np.random.default_rng(2)
    x16 = rng.standard_normal((16, 4096), dtype=f32)
    codes = rng.integers(-127, 128, (4096, 14336), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, 14336).astype(f32)
    return x16, codes, scales


def bf16_narrow(x):
    """L-2 (checks/numerics.mojo:1554-1574): ftz, then round to nearest even on the low 16
    bits; a NaN stays a quiet NaN; overflow rounds into the infinity."""
    b = np.ascontiguousarray(x, dtype=f32).view(np.uint32)
    sub = (b & 0x7F800000) == 0
    b = np.where(sub, b & 0x80000000, b).astype(np.uint32)
    nan = ((b & 0x7F800000) == 0x7F800000) & ((b & 0x007FFFFF) != 0)
    lsb = (b >> 16) & 1
    r = ((b.astype(np.uint64) + 0x7FFF + lsb) >> 16).astype(np.uint16)
    return np.where(nan, ((b >> 16) | 0x0040).astype(np.uint16), r)


def swiglu_up():
    """(x, w_bits uint16)"""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4096, 4096), dtype=f32)
    w = (rng.standard_normal((4096, 11008), dtype=f32) * f32(0.02)).astype(f32)
    return x, bf16_narrow(w)


def _adversarial(rng, shape):
    mag = (10.0 ** rng.uniform(-30, 30, shape)).astype(f32)
    sign = rng.choice(np.array([-1, 1], dtype=f32), shape)
    v = (sign * mag).astype(f32)
    u = rng.random(shape)
    sub = u < 0.01
    zero = (u >= 0.01) & (u < 0.02)
    w = v.view(np.uint32)
    ns = int(sub.sum())
    w[sub] = (rng.integers(1, 0x800000, ns, dtype=np.uint32) | (rng.integers(0, 2, ns, dtype=np.uint32) << 31))
    nz = int(zero.sum())
    w[zero] = rng.integers(0, 2, nz, dtype=np.uint32) << 31
    return v


def lm_head():
    rng = np.random.default_rng(4)
    x = _adversarial(rng, (512, 2048))
    w = _adversarial(rng, (2048, 50304))
    return x, w


WORKLOADS = {
    "gemm512": dict(m=512, n=512, k=512),
    "prefill": dict(m=2048, n=4096, k=4096),
    "decode_m1": dict(m=1, n=14336, k=4096),
    "decode_m4": dict(m=4, n=14336, k=4096),
    "decode_m16": dict(m=16, n=14336, k=4096),
    "swiglu_up": dict(m=4096, n=11008, k=4096),
    "lm_head": dict(m=512, n=50304, k=2048),
}
