"""Benchmark of the identical-mode FP32 GEMM/GEMV on one MI355X.

Headline (the JSON line's `value`): the decoder-LM prefill projection, X[2048x4096] . W[4096x4096]
+ bias[4096] under mojolearn.identical.gemm.fp32.v1 (nn.Linear bias fused into the store),
inputs resident in HBM, one product per step, in TFLOP/s (2mnk per step; the bias adds are not
counted).  Beside it: the kernel's roofline fraction (FP32 matrix peak 157.3 TFLOP/s), the
other workloads (--all: 512^3, decode GEMV with an int8 weight at M = 1/4/16 in GB/s, the bf16
SwiGLU up projection, the adversarial LM head, and one GPU's N/8 column shard of the decode GEMV
and of the prefill, each the median of 20 timed runs with the fastest and slowest), the
mismatching words against the CPU oracle over every output cell (the output first filled with a
poison word), and the CPU baseline timed on the host cores: the scalar oracle on one thread on
the reference's host-capped block (the headline `cpu_baseline`) and the reference's fast CPU
column restated on every thread (with --all, both arms on every workload, and the host's CPU).
Just before the headline's timed run its captured graph replays untimed for CLOCK_RAMP_S seconds,
which brings the engine clock to its steady state under this load; the K timed steps are unchanged.
The decode rows and read floors do the same (--decode-ramp seconds; 0 for kernel-trace runs).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--all] [--no-cpu] [--decode-ramp S]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix
HBM_PEAK_GBS = 8000.0


EAGER = False  # --eager: time plain launches instead of graph replays (for counter runs)


def graph_runs(calls, steps, warmup, torch, runs=1, eager=None, ramp_s=0.0, ramp_out=None):
    """Average ms per call of each of `runs` timed runs: `steps` calls (round-robin over `calls`,
    each a Plan) captured in one HIP graph on a private stream, replayed once per run; HIP events
    on the replaying stream.  With EAGER (or `eager`) the same calls are launched one by one on
    that stream, bracketed by its events.  `ramp_s`: untimed replays of the graph for that many
    seconds just before the timed runs (their count appended to `ramp_out`)."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for i in range(max(warmup, len(calls))):
            calls[i % len(calls)](s)
    torch.cuda.synchronize()
    out = []
    if EAGER or eager:
        for _ in range(runs):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            with torch.cuda.stream(s):
                for i in range(steps):
                    calls[i % len(calls)](s)
            e1.record(s)
            e1.synchronize()
            out.append(e0.elapsed_time(e1) / steps)
        return out
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            calls[i % len(calls)](s)
    g.replay()
    torch.cuda.synchronize()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < ramp_s:
        g.replay()
        torch.cuda.synchronize()
        n += 1
    if ramp_out is not None:
        ramp_out.append(n * steps)
    cur = torch.cuda.current_stream()
    for _ in range(runs):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        g.replay()
        e1.record(cur)
        e1.synchronize()
        out.append(e0.elapsed_time(e1) / steps)
    return out


def graph_time(calls, steps, warmup, torch):
    """Average ms per call over one timed run of `steps` calls (graph_runs)."""
    return graph_runs(calls, steps, warmup, torch)[0]


#: seconds of untimed replays of the headline's graph just before its timed run: the engine
#: clock's ramp to its steady state under this load (with 20 timed steps after 5 warmup launches
#: and no ramp the first timed run read 113.5 TFLOP/s, against 123-124 in steady state: the same
#: kernel at a lower clock).
CLOCK_RAMP_S = 1.0
#: the same untimed ramp before each decode row and read floor (set by --decode-ramp): with 100
#: warmup launches of a 12-17 us kernel (1.5 ms) the clock has not settled either (M=4 16.5 us,
#: against 15.6 after 0.75 s of launches).
DECODE_RAMP_S = CLOCK_RAMP_S


def _timed(calls, steps, warmup, torch, runs, eager=None, ramp_s=0.0, ramp_out=None):
    """{"ms": ...} from one run, or with runs > 1 the median run and the fastest and slowest."""
    t = sorted(graph_runs(calls, steps, warmup, torch, runs, eager, ramp_s, ramp_out))
    if runs == 1:
        return {"ms": t[0]}
    return {"ms": float(np.median(t)), "ms_min": t[0], "ms_max": t[-1], "runs": runs}


PREFILL_PROFILE = os.path.join(ROOT, "profiles", "gemm_mfma_kernel_prefill_2048x4096x4096.md")


def profiled_traffic(path=PREFILL_PROFILE):
    """HBM bytes per launch of the prefill kernel as last measured by rocprofv3 (FETCH_SIZE +
    WRITE_SIZE, each scaled by a plain 1 GiB copy), read from the committed summary; None if
    the summary is absent."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


POISON = -987654.0  # an output cell no kernel writes keeps it (gemm/checks/gemm_device_check.mojo:111)


def _rows(m, count=8):
    if m <= count:
        return np.arange(m)
    return np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).choice(m, count - 2, replace=False)]))


def _mismatch(got, want):
    return int(np.count_nonzero(np.ascontiguousarray(got).view(np.uint32) != np.ascontiguousarray(want).view(np.uint32)))


def _t(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def bench_prefill(torch, D, W, O, steps, warmup, check, runs=1, cols=None, ramp=False):
    """The prefill projection; `cols` keeps W's and bias's first columns (one GPU's column
    shard at its real shape); `ramp`: CLOCK_RAMP_S of untimed replays just before the timed run."""
    x, w, bias = W.prefill()
    if cols is not None:
        w, bias = np.ascontiguousarray(w[:, :cols]), np.ascontiguousarray(bias[:cols])
    plan = D.Plan(_t(torch, x), _t(torch, w), bias=_t(torch, bias))
    ramped = []
    res = _timed([plan], steps, warmup, torch, runs, ramp_s=CLOCK_RAMP_S if ramp else 0.0, ramp_out=ramped)
    res["ramp_launches"] = ramped[0] if ramped else 0
    res["out"] = None
    ms = res["ms"]
    m, k = x.shape
    n = w.shape[1]
    res["tflops"] = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    if check:
        # every cell, on an output first filled with the poison word
        plan.out.fill_(POISON)
        plan()
        want = O.nan_canon(O.bias(O.gemm_fast(x, w, 0), bias))
        got = plan.out.cpu().numpy()
        res["mismatched_words"] = _mismatch(got, want)
        res["checked_cells"] = int(m * n)
        res["out"] = got
    return res


def bench_product(torch, D, a, b, steps, warmup, want_fn=None, runs=1):
    """One Plan (a: float32, b: float32 or bf16 bits as uint16) timed as graph replays."""
    tb = _t(torch, b.view(np.int16) if b.dtype == np.uint16 else b)
    plan = D.Plan(_t(torch, a), tb)
    res = _timed([plan], steps, warmup, torch, runs)
    ms = res["ms"]
    m, k = a.shape
    n = b.shape[1]
    res["tflops"] = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    if want_fn is not None:
        plan.out.fill_(POISON)
        plan()
        res["mismatched_words"] = _mismatch(plan.out.cpu().numpy(), want_fn())
        res["checked_cells"] = int(m * n)
    return res


def bench_decode(torch, D, W, O, m, steps, warmup, check, nbuf=8, runs=1, cols=None, wdeq=None, packed=False):
    """int8-weight GEMV; `nbuf` distinct weight buffers rotate so W streams from HBM (8 x 58.7
    MB > the 256 MB Infinity Cache; a column shard rotates enough copies to exceed it too).
    GB/s counts K*N int8 codes + N scales + M*K x + M*N y per call.  `cols` keeps the first
    columns (one GPU's column shard); `wdeq` is the oracle's dequantized W when already made.
    `packed`: each buffer rearranged once, before the timed region, into the decode-packed
    layout (the same bytes for N a multiple of 128) and multiplied by gemv_int8w_packed."""
    x16, codes, scales = W.decode()
    if cols is not None:
        codes, scales = np.ascontiguousarray(codes[:, :cols]), np.ascontiguousarray(scales[:cols])
        nbuf = max(nbuf, -(-(320 << 20) // codes.size))
    x = np.ascontiguousarray(x16[:m])
    tx, ts = _t(torch, x), _t(torch, scales)
    out = torch.empty((m, codes.shape[1]), dtype=torch.float32, device="cuda:0")
    tcodes = [_t(torch, codes)] + [_t(torch, np.roll(codes, i, axis=1)) for i in range(1, nbuf)]
    if packed:
        pw = [D.pack_int8w(tc) for tc in tcodes]
        del tcodes
        plans = [D.PackedPlan(tx, p, ts, out=out) for p in pw]
    else:
        plans = [D.Plan(tx, tc, scales=ts, out=out) for tc in tcodes]
    ramped = []
    res = _timed(plans, max(steps, 2 * nbuf), warmup, torch, runs, ramp_s=DECODE_RAMP_S, ramp_out=ramped)
    res["ramp_launches"] = ramped[0] if ramped else 0
    ms = res["ms"]
    k, n = codes.shape
    nbytes = k * n + 4 * n + 4 * m * k + 4 * m * n
    res.update({"us": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9,
                "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12, "bytes": nbytes})
    if check:
        out.fill_(POISON)
        plans[0]()
        if wdeq is None:
            wdeq = O.int8_dequant(codes, scales, 0)
        want = O.gemm_fast(x, np.ascontiguousarray(wdeq[:, :n]), 0)
        res["mismatched_words"] = _mismatch(out.cpu().numpy(), want)
        res["checked_cells"] = int(m * n)
    return res


def bench_read_floor(torch, steps, warmup, runs, nbuf=8):
    """The memory floors of the decode GEMV's weight stream: a read-only pass over the same
    rotating int8 W[4096x14336] buffers, (linear) in address order with 16-byte loads, (leaf) in
    the row-major decode kernel's own order -- a wave per 128-row leaf and 256-byte strip, every
    leaf of a column streamed at once, as the contract's leaf chains require -- and (packed) in
    the decode-packed product's order: whole-column workgroups of 16 waves, two leaves a wave,
    block s of every leaf read together."""
    from mojolearn_amd import _native
    L = _native.lib()
    k, n = 4096, 14336
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(7)
    bufs = [torch.randint(-127, 128, (k, n), dtype=torch.int8, device="cuda:0", generator=gen) for _ in range(nbuf)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    res = {}
    for pattern, name in ((0, "linear"), (1, "leaf"), (2, "packed")):
        calls = [lambda s, b=b, pattern=pattern: _native.check(
            L.mlg_stream_read(b.data_ptr(), k, n, pattern, sink.data_ptr(), s.cuda_stream)) for b in bufs]
        ramped = []
        r = _timed(calls, max(steps, 2 * nbuf), warmup, torch, runs, ramp_s=DECODE_RAMP_S, ramp_out=ramped)
        r["ramp_launches"] = ramped[0] if ramped else 0
        r.update({"us": r["ms"] * 1e3, "gbs": k * n / (r["ms"] * 1e-3) / 1e9,
                  "hbm_frac": k * n / (r["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, "bytes": k * n})
        res[name] = r
    return res


def _repeat(fn, min_seconds, max_seconds):
    """Call fn until about `min_seconds` have passed; (calls, seconds, last result)."""
    reps, t0 = 0, time.perf_counter()
    while True:
        y = fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or dt * (reps + 1) / reps > max_seconds:
            return reps, dt, y


def cpu_baseline(W, O, gpu_out=None, min_seconds=10.0, max_seconds=30.0):
    """Both CPU arms on the prefill projection, timed on this host.

    Arm (i), the headline: the scalar oracle (orc_gemm: the reference CPU binding's algorithm,
    decomposition/linalg_host_impl.mojo:39-47 -> gemm/host/gemm_oracle.mojo:357-371) on ONE
    thread, on the block the reference's host budget allows (16 M multiply-accumulates: m and n
    halved, k untouched; bench/gemm_card_main.mojo:361-378), + bias, repeated for about
    `min_seconds`; capped.  Its words are compared with the same block of the GPU's output.
    Arm (ii): the reference's fast CPU column (orc_host_rows, gemm/host/gemm_host_rows.mojo,
    deferred flush with redo) on every host thread, the whole product + bias."""
    x, w, bias = W.prefill()
    m, k = x.shape
    n = w.shape[1]
    mm, nn = host_capped(m, n, k)
    xs, ws, bs = np.ascontiguousarray(x[:mm]), np.ascontiguousarray(w[:, :nn]), np.ascontiguousarray(bias[:nn])
    reps, dt, y = _repeat(lambda: O.bias(O.gemm(xs, ws, 0), bs), min_seconds, max_seconds)
    arm1 = {"value": round(2.0 * mm * nn * k * reps / dt / 1e9, 4), "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "capped": True,
            "sample": f"the {mm}x{nn} block of the prefill product (X[:{mm}] . W[:, :{nn}], k = {k}, + bias: the "
                      f"reference's 16M-MAC host cap) x {reps}, oracle/gemm_oracle.c orc_gemm (the scalar "
                      f"gemm_oracle), 1 thread, {dt:.1f} s"}
    if gpu_out is not None:
        arm1["mismatched_words_vs_gpu"] = _mismatch(O.nan_canon(y), gpu_out[:mm, :nn])
    threads = O.max_threads()
    reps, dt, _ = _repeat(lambda: O.bias(O.host_rows(x, w, 0, threads=threads), bias), min_seconds, max_seconds)
    arm2 = {"value": round(2.0 * m * n * k * reps / dt / 1e9, 3), "unit": "GFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"the whole prefill product + bias x {reps}, oracle/gemm_oracle.c orc_host_rows (the "
                      f"reference's gemm_host_rows: AVX2 FMA, deferred flush with redo), {threads} threads, "
                      f"{dt:.1f} s"}
    return arm1, arm2


class _SeqLinear:
    """The sequence executor's linear step (sequence/ops.mojo:485-569, the product word and its
    bias + activation follower, gemm/neural_dispatch.mojo:316-397): one whole-k chain per cell,
    the follower fused into the product's store (one launch)."""

    def __init__(self, torch, D, x, w, bias, act):
        self.D, self.x, self.w, self.bias, self.act = D, x, w, bias, act
        self.out = torch.empty((x.shape[0], w.shape[1]), dtype=torch.float32, device=x.device)

    def __call__(self, stream=None):
        k = self.x.shape[1]
        self.D.gemm_leaf_ptr(self.x, self.w, leaf=k, p_count=1, out=self.out, epi=self.D.EPI_BIAS_ACT,
                             epi_p=self.bias, act=self.act)


class _SeqAccumulate:
    """op_gemm with accumulate: the weight gradient dW += X^T . dY through strided views (X^T is X
    read k-major, no copy), each chain seeded by the flushed old dW."""

    def __init__(self, D, xt, dy, dw):
        self.D, self.xt, self.dy, self.out = D, xt, dy, dw

    def __call__(self, stream=None):
        self.D.seq_gemm(self.xt, self.dy, self.out, accumulate=True)


def bench_seq(torch, D, W, O, steps, warmup, check, runs=1):
    """The sequence-executor word on the prefill operands, eager launches (HIP events on the
    launching stream): the linear step X[2048x4096] . W[4096x4096], bias + ReLU, and the weight
    gradient dW[4096x4096] += X^T . dY[2048x4096].  Sampled rows are checked against the
    oracle's op_gemm and follower."""
    x, w, bias = W.prefill()
    m, k = x.shape
    n = w.shape[1]
    tx, tw, tb = _t(torch, x), _t(torch, w), _t(torch, bias)
    out = {}
    lin = _SeqLinear(torch, D, tx, tw, tb, D.ACT_RELU)
    res = _timed([lin], max(3, steps // 2), max(3, warmup // 4), torch, runs, eager=True)
    res["tflops"] = 2.0 * m * n * k / (res["ms"] * 1e-3) / 1e12
    if check:
        rows = _rows(m)
        xr = np.ascontiguousarray(x[rows])
        want = np.zeros((len(rows), n), np.float32)
        O.seq_gemm(want, xr, w, len(rows), n, k, k, 1, n, 1, n, False)
        O.epilogue(want, n, len(rows), n, O.EPI_BIAS_ACT, bias, O.ACT_RELU)
        res["mismatched_words"] = _mismatch(lin.out.cpu().numpy()[rows], want)
        res["checked_cells"] = int(len(rows) * n)
    out["seq_linear_bias_relu_2048x4096x4096"] = res
    del lin
    dy = np.random.default_rng(5).standard_normal((m, n), dtype=np.float32)
    tdy = _t(torch, dy)
    dw0 = (np.random.default_rng(6).standard_normal((k, n), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    tdw = _t(torch, dw0)
    acc = _SeqAccumulate(D, tx.t(), tdy, tdw)
    if check:
        # one accumulation from a known dW, checked before the timed ones drift it further
        acc()
        rows = _rows(k)
        want = np.ascontiguousarray(dw0[rows])
        xt_rows = np.ascontiguousarray(x[:, rows].T)
        O.seq_gemm(want, xt_rows, dy, len(rows), n, m, m, 1, n, 1, n, True)
        mism = _mismatch(tdw.cpu().numpy()[rows], want)
    res = _timed([acc], max(3, steps // 4), max(3, warmup // 10), torch, runs, eager=True)
    res["tflops"] = 2.0 * k * n * m / (res["ms"] * 1e-3) / 1e12
    if check:
        res["mismatched_words"] = mism
        res["checked_cells"] = int(len(rows) * n)
    out["seq_grad_accumulate_4096x4096x2048"] = res
    return out


#: The reference's fp32.v1 and bf16f32.v1 rows on MI325X (INFERENCE, the median ms of one call and
#: one synchronize per sample; the weights W[n][k] packed once, OP_NT;
#: bench/results/lowbit_units/2026-09-29/TABLE.md:76-89).
LLAMA_ROWS = [("qkv.t1", 1, 4096, 4096, 0.0617, 1.1249), ("qkv.t8", 8, 4096, 4096, 0.0775, 0.1078),
              ("qkv.t512", 512, 4096, 4096, 0.9254, 0.9480), ("mlp_up.t1", 1, 14336, 4096, 0.1631, 1.1905),
              ("mlp_up.t8", 8, 14336, 4096, 0.1677, 0.2920), ("mlp_up.t512", 512, 14336, 4096, 2.3895, 2.5044),
              ("mlp_down.t1", 1, 4096, 14336, 0.1560, 3.9026), ("mlp_down.t8", 8, 4096, 14336, 0.1947, 0.3250),
              ("mlp_down.t512", 512, 4096, 14336, 2.5107, 2.5862), ("lm_head.t1", 1, 128256, 4096, 1.3122, 2.5466),
              ("lm_head.t8", 8, 128256, 4096, 1.2280, 2.4984), ("lm_head.t512", 512, 16032, 4096, 2.7776, 2.9081)]


def bench_llama(torch, D, steps, warmup):
    """The reference's Llama-8B projection rows, fp32 and bf16-stored weights (OP_NT, W[n][k]
    resident, the same buffers every call), device time per product as graph replays; the
    reference's times include one host synchronize per call.  Random weights, made on the device."""
    out = {}
    g = torch.Generator(device="cuda:0")
    g.manual_seed(9)
    for name, m, n, k, ref32, ref16 in LLAMA_ROWS:
        x = torch.randn((m, k), generator=g, device="cuda:0")
        w = torch.randn((n, k), generator=g, device="cuda:0") * 0.02
        row = {}
        for kind, wt, ref in (("fp32", w, ref32), ("bf16w", w.to(torch.bfloat16).view(torch.int16), ref16)):
            plan = D.Plan(x, wt, op=D.OP_NT)
            ms = graph_time([plan], max(3, steps // 2), max(3, warmup // 4), torch)
            row[kind] = {"ms": ms, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12, "reference_mi325x_ms": ref,
                         "speedup_vs_reference": ref / ms}
            del plan
        out[name] = row
        del x, w
    return out


#: The reference's host budget for its scalar oracle arm, in multiply-accumulates
#: (bench/gemm_card_main.mojo:241), and its rule for meeting it (:361-378): halve n (or m, when
#: m > n) until m*n*k fits; k is never touched, so every cell keeps its leaves and tree.
HOST_MAC_BUDGET = 16_000_000


def host_capped(m, n, k):
    while m * n * k > HOST_MAC_BUDGET and (m > 1 or n > 1):
        if n >= m and n > 1:
            n = (n + 1) // 2
        else:
            m = (m + 1) // 2
    return m, n


def host_info():
    """The host's CPU: the threads this process may use and the model name."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count(), "model": model}


def cpu_arms(W, O):
    """Both CPU arms on the five workloads, timed on this host: (i) the scalar oracle (the
    reference's CPU binding's algorithm) on one thread, full size for 512^3 and the decode GEMV,
    capped by the reference's host budget for the three large products; (ii) the reference's fast
    CPU column restated (orc_host_rows: AVX2 FMA, deferred flush with redo) on every host thread,
    full size.  Where an arm ran a capped block, its bits are
    compared with the same block of the fast arm's full output (a cell's arithmetic depends on
    k only, so the block must match word for word)."""
    threads = O.max_threads()
    rows = {}

    def arm(fn, m, n, k):
        t0 = time.perf_counter()
        y = fn()
        dt = time.perf_counter() - t0
        return y, {"shape": [m, n, k], "s": dt, "gflops": 2.0 * m * n * k / dt / 1e9}

    def both(name, a, b, post=None, full=False):
        m, k = a.shape
        n = b.shape[1]
        post = post or (lambda y, cols: y)
        fast, rf = arm(lambda: post(O.host_rows(a, b, 0, threads=threads), n), m, n, k)
        mm, nn = (m, n) if full else host_capped(m, n, k)
        sa, sb = np.ascontiguousarray(a[:mm]), np.ascontiguousarray(b[:, :nn])
        scal, rs = arm(lambda: post(O.gemm(sa, sb, 0), nn), mm, nn, k)
        rs["capped"] = (mm, nn) != (m, n)
        rs["mismatched_words_vs_fast"] = _mismatch(O.nan_canon(scal), O.nan_canon(fast[:mm, :nn]))
        rows[name] = {"scalar_1_thread": rs, "fast_all_threads": rf}

    a, b = W.gemm512()
    both("gemm512", a, b, full=True)
    x, w, bias = W.prefill()
    both("prefill", x, w, post=lambda y, cols: O.bias(y, bias[:cols]))
    x16, codes, scales = W.decode()
    wdeq = O.int8_dequant(codes, scales, 0)
    for m in (1, 4, 16):
        both(f"decode_m{m}", np.ascontiguousarray(x16[:m]), wdeq, full=True)
    x, wb = W.swiglu_up()
    both("swiglu_up", x, O.bf16_widen(wb))
    x, w = W.lm_head()
    both("lm_head", x, w, post=lambda y, cols: O.nan_canon(y))
    return {"host": host_info(), "threads": threads, "rows": rows}


def bench_compare(torch, D, steps, warmup):
    """The rows the reference publishes for this path on MI325X (its own results tree), measured
    the same way here: fp32.v1 512x4096x4096 OP_NT, fp32-weight GEMV 1x14336x4096 (OP_NN and the
    LM layout OP_NT, 235 MB of weights, 4 rotating copies), and the host-pointer surface
    `linalg.matmul` on 4096^3 numpy arrays (upload, product, download, NaN canon), median of 5."""
    from mojolearn_amd import linalg
    rng = np.random.default_rng(7)
    out = {}
    a = rng.standard_normal((512, 4096), dtype=np.float32)
    w = rng.standard_normal((4096, 4096), dtype=np.float32)
    plan = D.Plan(_t(torch, a), _t(torch, w), op=D.OP_NT)
    ms = graph_time([plan], steps, warmup, torch)
    out["nt_512x4096x4096"] = {"ms": ms, "tflops": 2.0 * 512 * 4096 * 4096 / (ms * 1e-3) / 1e12,
                               "reference_mi325x_tflops": 18.6}
    x = rng.standard_normal((1, 4096), dtype=np.float32)
    for name, op, shape in (("gemv_f32_nn_1x14336x4096", D.OP_NN, (4096, 14336)),
                            ("gemv_f32_nt_1x14336x4096", D.OP_NT, (14336, 4096))):
        tx = _t(torch, x)
        ws = [torch.randn(shape, dtype=torch.float32, device="cuda:0") for _ in range(4)]
        o = torch.empty((1, 14336), dtype=torch.float32, device="cuda:0")
        plans = [D.Plan(tx, wi, op=op, out=o) for wi in ws]
        ms = graph_time(plans, max(steps, 8), warmup, torch)
        nbytes = 4 * (4096 * 14336 + 4096 + 14336)
        out[name] = {"ms": ms, "us": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9, "reference_mi325x_gbs": 1440.0}
        del plans, ws
    ha = rng.standard_normal((4096, 4096), dtype=np.float32)
    hb = rng.standard_normal((4096, 4096), dtype=np.float32)
    linalg.matmul(ha, hb)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        linalg.matmul(ha, hb)
        times.append((time.perf_counter() - t0) * 1e3)
    times.sort()
    out["host_matmul_4096"] = {"ms": times[2], "tflops": 2.0 * 4096 ** 3 / (times[2] * 1e-3) / 1e12,
                               "reference_mi325x_ms": 28.2}
    return out


#: The reference's int8i32.v1 rows on MI325X (its integer-MMA arm, best ms of its runs;
#: bench/results/lowbit_amd_tuned/2026-09-29/mi325x/*/lowbit.tsv).
INT8I32_ROWS = [("qkv.t1", 1, 4096, 4096, 0.0480), ("qkv.t8", 8, 4096, 4096, 0.0496),
                ("qkv.t512", 512, 4096, 4096, 0.2644), ("mlp_up.t1", 1, 14336, 4096, 0.0531),
                ("mlp_up.t8", 8, 14336, 4096, 0.0609), ("mlp_up.t512", 512, 14336, 4096, 0.8768),
                ("mlp_down.t1", 1, 4096, 14336, 0.1363), ("mlp_down.t8", 8, 4096, 14336, 0.1406),
                ("mlp_down.t512", 512, 4096, 14336, 0.8387), ("lm_head.t1", 1, 128256, 4096, 0.2742),
                ("lm_head.t8", 8, 128256, 4096, 0.3185), ("lm_head.t512", 512, 16032, 4096, 1.0085)]


class Int8Call:
    """One int8i32.v1 product C = qa . qb^T on device buffers, launched on a given stream."""

    def __init__(self, torch, qa, ea, qb, eb):
        from mojolearn_amd import _native
        self.lib, self.check = _native.lib(), _native.check
        self.qa, self.ea, self.qb, self.eb = qa, ea, qb, eb
        self.m, self.k = qa.shape
        self.n = qb.shape[0]
        self.out = torch.empty((self.m, self.n), dtype=torch.float32, device=qa.device)
        nb = self.lib.mlg_gemm_int8i32_workspace_bytes(qa.data_ptr(), qb.data_ptr(), self.m, self.n, self.k)
        if nb < 0:
            raise RuntimeError(self.lib.mlg_last_error().decode())
        self.nb = nb
        self.ws = torch.empty(max(nb, 4), dtype=torch.uint8, device=qa.device)

    def __call__(self, stream=None):
        import torch
        s = stream if stream is not None else torch.cuda.current_stream()
        self.check(self.lib.mlg_gemm_int8i32_ws(self.out.data_ptr(), self.qa.data_ptr(), self.ea.data_ptr(),
                                                self.qb.data_ptr(), self.eb.data_ptr(), self.m, self.n, self.k,
                                                self.ws.data_ptr(), self.nb, s.cuda_stream))


def bench_int8i32(torch, O, steps, warmup, check):
    """The int8i32.v1 product (integer MFMA) on the reference's Llama-8B rows: codes and row
    exponents resident in HBM, the same buffers every call (as the reference measured them);
    TOP/s counts 2mnk, and the weight codes' GB/s is reported for the skinny rows."""
    rng = np.random.default_rng(11)
    out = {}
    for name, m, n, k, ref_ms in INT8I32_ROWS:
        qa = rng.integers(-127, 128, (m, k), dtype=np.int8)
        qb = rng.integers(-127, 128, (n, k), dtype=np.int8)
        ea = rng.integers(-20, 0, m).astype(np.int32)
        eb = rng.integers(-20, 0, n).astype(np.int32)
        call = Int8Call(torch, _t(torch, qa), _t(torch, ea), _t(torch, qb), _t(torch, eb))
        ms = graph_time([call], steps, warmup, torch)
        row = {"ms": ms, "tops": 2.0 * m * n * k / (ms * 1e-3) / 1e12,
               "weight_gbs": n * k / (ms * 1e-3) / 1e9, "reference_mi325x_ms": ref_ms,
               "speedup_vs_reference": ref_ms / ms}
        if check:
            rows = _rows(m, 4)
            want = O.nan_canon(O.q8_gemm(qa[rows], ea[rows], qb, eb))
            row["mismatched_words"] = _mismatch(call.out.cpu().numpy()[rows], want)
            row["checked_cells"] = int(len(rows) * n)
        out[name] = row
        del call
    return out


#: The reference's int15i64.v1 rows on MI325X (its integer-MMA plan, best ms of its runs;
#: bench/results/lowbit_amd_tuned/2026-09-29/mi325x/*/int15.tsv).
INT15I64_ROWS = [("qkv.t1", 1, 4096, 4096, 0.0799), ("qkv.t8", 8, 4096, 4096, 0.0813),
                 ("qkv.t512", 512, 4096, 4096, 0.5322), ("mlp_up.t1", 1, 14336, 4096, 0.1077),
                 ("mlp_up.t512", 512, 14336, 4096, 1.8390), ("mlp_down.t1", 1, 4096, 14336, 0.2830),
                 ("mlp_down.t512", 512, 4096, 14336, 1.7749), ("lm_head.t1", 1, 128256, 4096, 0.5924),
                 ("lm_head.t512", 512, 16032, 4096, 2.0671)]


class Int15Call:
    """One int15i64.v1 product C = a . b^T on device planes, launched on a given stream."""

    def __init__(self, torch, ah, al, ea, bh, bl, eb):
        from mojolearn_amd import _native
        self.lib, self.check = _native.lib(), _native.check
        self.t = (ah, al, ea, bh, bl, eb)
        self.m, self.k = ah.shape
        self.n = bh.shape[0]
        self.out = torch.empty((self.m, self.n), dtype=torch.float32, device=ah.device)
        nb = self.lib.mlg_gemm_int15i64_workspace_bytes(ah.data_ptr(), al.data_ptr(), bh.data_ptr(), bl.data_ptr(),
                                                        self.m, self.n, self.k)
        if nb < 0:
            raise RuntimeError(self.lib.mlg_last_error().decode())
        self.nb = nb
        self.ws = torch.empty(max(nb, 4), dtype=torch.uint8, device=ah.device)

    def __call__(self, stream=None):
        import torch
        s = stream if stream is not None else torch.cuda.current_stream()
        ah, al, ea, bh, bl, eb = self.t
        self.check(self.lib.mlg_gemm_int15i64_ws(self.out.data_ptr(), ah.data_ptr(), al.data_ptr(), ea.data_ptr(),
                                                 bh.data_ptr(), bl.data_ptr(), eb.data_ptr(), self.m, self.n, self.k,
                                                 self.ws.data_ptr(), self.nb, s.cuda_stream))


def bench_int15i64(torch, O, steps, warmup, check):
    """The int15i64.v1 product (four int8 plane products per step on the integer matrix unit)
    on the reference's Llama-8B rows, planes and exponents resident in HBM."""
    rng = np.random.default_rng(15)
    out = {}
    for name, m, n, k, ref_ms in INT15I64_ROWS:
        qa = rng.integers(-16383, 16384, (m, k))
        qb = rng.integers(-16383, 16384, (n, k))
        ah, al = (qa >> 7).astype(np.int8), (qa & 127).astype(np.int8)
        bh, bl = (qb >> 7).astype(np.int8), (qb & 127).astype(np.int8)
        del qa, qb
        ea = rng.integers(-40, -20, m).astype(np.int32)
        eb = rng.integers(-40, -20, n).astype(np.int32)
        call = Int15Call(torch, *(_t(torch, x) for x in (ah, al, ea, bh, bl, eb)))
        ms = graph_time([call], steps, warmup, torch)
        row = {"ms": ms, "tops": 2.0 * m * n * k / (ms * 1e-3) / 1e12, "reference_mi325x_ms": ref_ms,
               "speedup_vs_reference": ref_ms / ms}
        if check:
            rows = _rows(m, 4)
            want = O.nan_canon(O.q15_gemm(ah[rows], al[rows], ea[rows], bh, bl, eb))
            row["mismatched_words"] = _mismatch(call.out.cpu().numpy()[rows], want)
            row["checked_cells"] = int(len(rows) * n)
        out[name] = row
        del call
    return out


def copy_calibration(torch, nbytes=1 << 30):
    """Three copies of a 1 GiB float32 buffer (torch's elementwise copy kernel): each dispatch
    reads and writes exactly `nbytes`, the yardstick for the FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "dispatches": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 100 untimed steps bring the engine clock to its steady state under this load (with 3, the
    # timed steps ran ~8 % slower while it ramped); 50 timed steps are ~30 ms of product.
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--all", action="store_true", help="also measure the other four workloads")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle comparison")
    ap.add_argument("--eager", action="store_true", help="time eager launches, no HIP graph")
    ap.add_argument("--compare", action="store_true",
                    help="also measure the rows the reference publishes for this path (MI325X)")
    ap.add_argument("--read-floor", action="store_true",
                    help="only time the read-only streams over the decode weight buffers and exit")
    ap.add_argument("--decode-ramp", type=float, default=CLOCK_RAMP_S,
                    help="seconds of untimed graph replays before each decode row and read floor "
                         "(0 for kernel-trace runs: every replay is traced)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (the byte-counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the product shards by output columns with no arithmetic exchange)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        copy_calibration(torch)
        return
    if args.read_floor:
        print(json.dumps({"read_floor": bench_read_floor(torch, args.steps, args.warmup, runs=20)}), flush=True)
        return
    global EAGER, DECODE_RAMP_S
    EAGER = args.eager
    DECODE_RAMP_S = args.decode_ramp

    from mojolearn_amd import device as D
    from mojolearn_amd import workloads as W
    from oracle import oracle as O

    check = not args.no_check
    pre = bench_prefill(torch, D, W, O, args.steps, args.warmup, check, ramp=True)
    gpu_out = pre.pop("out")
    extra = {}
    if args.all:
        # every row: the median of RUNS timed runs (graph replays), with the fastest and slowest
        R = 20
        extra["prefill"] = bench_prefill(torch, D, W, O, args.steps, args.warmup, check, runs=R)
        extra["prefill"].pop("out")
        a, b = W.gemm512()
        extra["gemm512"] = bench_product(torch, D, a, b, args.steps, args.warmup,
                                         want_fn=(lambda: O.gemm(a, b, 0)) if check else None, runs=R)
        x16, codes, scales = W.decode()
        wdeq = O.int8_dequant(codes, scales, 0) if check else None
        del x16, codes, scales
        for m in (1, 4, 16):
            extra[f"decode_m{m}"] = bench_decode(torch, D, W, O, m, args.steps, args.warmup, check, runs=R,
                                                 wdeq=wdeq)
        # the same products on weights rearranged once into the decode-packed layout
        for m in (1, 4, 16):
            extra[f"decode_m{m}_packed"] = bench_decode(torch, D, W, O, m, args.steps, args.warmup, check, runs=R,
                                                        wdeq=wdeq, packed=True)
        x, wb = W.swiglu_up()
        extra["swiglu_up"] = bench_product(
            torch, D, x, wb, max(3, args.steps // 4), max(3, args.warmup // 10),
            want_fn=(lambda: O.gemm_fast(x, O.bf16_widen(wb), 0)) if check else None, runs=R)
        x, w = W.lm_head()
        extra["lm_head"] = bench_product(
            torch, D, x, w, max(3, args.steps // 2), max(3, args.warmup // 4),
            want_fn=(lambda: O.nan_canon(O.gemm_fast(x, w, 0))) if check else None, runs=R)
        del x, w, wb
        # one GPU's share of the two products a column split spreads over 8 GPUs: N/8 columns
        extra["shard_decode_m1_n1792"] = bench_decode(torch, D, W, O, 1, args.steps, args.warmup, check,
                                                      runs=R, cols=14336 // 8, wdeq=wdeq)
        extra["shard_decode_m1_n1792_packed"] = bench_decode(torch, D, W, O, 1, args.steps, args.warmup, check,
                                                             runs=R, cols=14336 // 8, wdeq=wdeq, packed=True)
        extra["shard_prefill_n512"] = bench_prefill(torch, D, W, O, args.steps, args.warmup, check, runs=R,
                                                    cols=4096 // 8)
        extra["shard_prefill_n512"].pop("out")
        del wdeq
        extra.update(bench_seq(torch, D, W, O, args.steps, args.warmup, check, runs=R))

    if args.compare:
        extra["compare"] = bench_compare(torch, D, args.steps, args.warmup)
        extra["int8i32"] = bench_int8i32(torch, O, args.steps, args.warmup, check)
        extra["int15i64"] = bench_int15i64(torch, O, args.steps, args.warmup, check)
        extra["llama_fp32_bf16w"] = bench_llama(torch, D, args.steps, args.warmup)

    line = {
        "metric": "identical-mode FP32 GEMM TFLOP/s & % of peak; GEMV GB/s; 0 mismatched bits",
        "value": round(pre["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "untimed_clock_ramp": {"seconds": CLOCK_RAMP_S, "launches": pre["ramp_launches"]},
        "ms_per_step": round(pre["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (numpy PCG64 seed 1: X~N(0,1), W~N(0,0.02), bias~N(0,0.01))",
        "config": {"workload": "prefill projection X[2048x4096] . W[4096x4096] + bias[4096], "
                               "identical mode (fp32.v1), OP_NN",
                   "m": 2048, "n": 4096, "k": 4096, "parallelism": "none (1 GPU)"},
        "pct_of_peak": round(100.0 * pre["tflops"] / FP32_PEAK_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(pre["tflops"], 3), "peak": FP32_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(pre["tflops"] / FP32_PEAK_TFLOPS, 4),
                     "traffic": profiled_traffic()},
    }
    if check:
        line["mismatched_words"] = pre["mismatched_words"]
        line["checked_cells"] = pre["checked_cells"]
    def _round(v):
        if isinstance(v, dict):
            return {kk: _round(vv) for kk, vv in v.items()}
        return round(v, 4) if isinstance(v, float) else v

    if extra:
        line["workloads"] = _round(extra)
    if not args.no_cpu:
        line["cpu_baseline"], line["cpu_baseline_fast_column"] = cpu_baseline(W, O, gpu_out)
        if args.all:
            line["cpu_arms"] = _round(cpu_arms(W, O))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
