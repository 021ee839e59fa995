"""Benchmark of the matrix-multiplication hot path on one MI355X.

One step = one pass of the d_model-256 byte-LM training-step GEMM set
(T = 4096 tokens, 5 layers x {forward, dX, dW} = 15 GEMMs, 20,937,965,568 FLOP)
on the f16-in/f32-accumulate route, issued as one grouped call
(st_matmul_grouped: the 15 GEMMs are independent here) and replayed from a HIP
graph.  `value` is that set's TFLOP/s; the same set issued in training-step
order (forward one by one, each layer's dW and dX grouped) and one call per
GEMM are reported beside it.  The same JSON line carries the other configurations measured in
the same run (256^3 f32, the tape backward forms, the f32 step set, batched
causal attention, the 125M-key 2-bit kNN scan), a roofline for the dominant
kernel of each headline, and the CPU baseline (the oracle's restatement of the
reference CPU path, one thread) on a bounded sample.

    python bench.py [--steps K] [--warmup W] [--only gemm|knn|all] [--no-cpu]
"""
from __future__ import annotations

import argparse
import contextlib
import hashlib
import itertools
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOP/s + % MFMA peak at d_model-256 step shapes; kNN keys/s + % HBM BW"
PEAK = {"f16": 2500.0, "f32": 157.3, "i8": 5000.0, "hbm_gbs": 8000.0}  # MI355X dense TFLOP/s (i8: TOP/s), HBM GB/s
T_TOKENS = 4096
LAYERS = [("qkv", 256, 768), ("out", 256, 256), ("ffn1", 256, 1024), ("ffn2", 1024, 256), ("head", 256, 256)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


@contextlib.contextmanager
def one_core():
    """Pins this process to one host core for a single-thread CPU baseline."""
    try:
        old = os.sched_getaffinity(0)
        core = min(old)
        os.sched_setaffinity(0, {core})
    except (AttributeError, OSError):
        old = None
    try:
        yield
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)


def host_threads():
    """Threads for the all-cores CPU baselines: this process's CPU share, at most 16 (and at most OMP_NUM_THREADS)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, min(n, 16))


def source_hash(rel):
    """sha256 of a kernel source file: ties a committed rocprof counter summary to the code it measured."""
    with open(os.path.join(ROOT, rel), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def traffic_for(kernel_key, src_rel):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, calibrated) from profiles/traffic.json, or None when that
    summary was taken on a different version of the kernel's source."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    e = t.get(kernel_key)
    if not e or e.get("source_sha256_16") != source_hash(src_rel):
        return None
    return int(e["fetch_bytes"] + e["write_bytes"])


def roofline(kernel, flops, nbytes, ms, traffic=None, route="f16"):
    """Roofline entry for one kernel: the binding roof is the lower of the route's MFMA peak and intensity x HBM
    peak."""
    tflops = flops / ms / 1e9
    gbs = nbytes / ms / 1e6
    peak = PEAK[route]
    ridge = peak * 1e12 / (PEAK["hbm_gbs"] * 1e9)
    if flops / nbytes < ridge:
        r = dict(kernel=kernel, bound="hbm", achieved=round(gbs, 1), peak=PEAK["hbm_gbs"], unit="GB/s",
                 frac=round(gbs / PEAK["hbm_gbs"], 4))
    else:
        r = dict(kernel=kernel, bound="mfma", achieved=round(tflops, 2), peak=peak, unit="TFLOP/s",
                 frac=round(tflops / peak, 4))
    r.update(traffic=traffic, algorithmic_bytes=int(nbytes), flops=int(flops), ms=round(ms, 5),
             tflops=round(tflops, 2), mfma_frac=round(tflops / peak, 4), hbm_gbs=round(gbs, 1),
             roof_tflops=round(min(peak, flops / nbytes * PEAK["hbm_gbs"] / 1e3), 1))
    return r


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


# --------------------------------------------------------------------------- timing helpers

def time_events(fn, reps, stream):
    """Average ms per call of fn() over `reps` calls, HIP events on `stream`."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(reps):
        fn()
    e.record(stream)
    e.synchronize()
    return s.elapsed_time(e) / reps


def time_graph_steps(fn, steps, stream, reps=5, spread=None, warm_s=0.025):
    """The K timed steps captured as ONE HIP graph (each step's calls in full, in order): ms per step, without the
    launch overhead a separate graph per step pays (several us each).  The graph is first replayed untimed for
    about `warm_s` seconds (the device settles at its sustained clocks: the first replays of a cold process read a
    few percent slower), then `reps` times, each replay (exactly K steps) timed on its own between HIP events; the
    median replay is reported (min, max and the untimed replays go into `spread` when given)."""
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(steps):
            fn()
    warm, t0 = 0, time.perf_counter()
    while warm < 200 and (warm < 1 or time.perf_counter() - t0 < warm_s):
        g.replay()
        torch.cuda.synchronize()
        warm += 1
    per = sorted(time_events(g.replay, 1, stream) / steps for _ in range(reps))
    del g
    if spread is not None:
        spread.update(min_ms=round(per[0], 5), max_ms=round(per[-1], 5), replays=reps, untimed_replays=warm)
    return per[len(per) // 2]


def time_graph(fn, steps, warmup, stream):
    """Captures fn() into a HIP graph; returns (ms per replay, graph)."""
    import torch
    fn()  # eager once more so every scratch buffer exists before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ms = time_events(g.replay, steps, stream)
    return ms, g


# --------------------------------------------------------------------------- GEMM step set

# The epilogues the reference's device tape gives each Linear (gpu_step/tape.rs:180-189, 324-347): the forward adds
# the bias (+ ReLU on the first FFN layer, + the residual stream after attention and after the FFN); the backward's
# dW accumulates into the parameter gradients with the bias gradient as column sums of dY.
TAPE_EPI = {"qkv": (False, False), "out": (False, True), "ffn1": (True, False), "ffn2": (False, True),
            "head": (False, False)}  # name -> (relu, residual)


class StepSet:
    """Buffers and the 15 GEMM calls of one d=256 training step (f32 operands in HBM).  With `epilogues`, each
    Linear's weights and bias share one parameter buffer [W, b] and its gradients one [dW, db], and the calls carry
    the device tape's epilogues (TAPE_EPI)."""

    def __init__(self, dev, seed=1, epilogues=False):
        import torch
        import oracle
        self.calls = []
        rng = oracle.Rng(seed)
        T = T_TOKENS
        self.bufs = []
        self.epilogues = epilogues
        extra = 0
        for name, K, N in LAYERS:
            X = torch.from_numpy(rng.gaussian(T * K)).to(dev)
            P = torch.from_numpy(rng.gaussian(K * N + (N if epilogues else 0), 0.02)).to(dev)
            dY = torch.from_numpy(rng.gaussian(T * N)).to(dev)
            Y, dX = (torch.zeros(n, device=dev) for n in (T * N, T * K))
            G = torch.zeros(K * N + (N if epilogues else 0), device=dev)
            R = None
            fwd_epi, dw_epi = None, None
            if epilogues:
                relu, res = TAPE_EPI[name]
                if res:
                    R = torch.from_numpy(rng.gaussian(T * N)).to(dev)
                fwd_epi = dict(bias=(P, K * N), relu=relu, residual=(R, 0) if res else None)
                dw_epi = dict(accumulate=True, col_sum=(K * N, 0))
                # bias read, residual read, dW read for +=, db read and written
                extra += 4 * (N + (T * N if res else 0) + K * N + 2 * N)
            self.bufs.append((X, P, dY, Y, dX, G, R))
            # (label, a, b, out, m, k, n, epilogue)
            self.calls.append((f"{name} fwd", dict(h=X), dict(h=P), dict(h=Y), T, K, N, fwd_epi))
            self.calls.append((f"{name} dX", dict(h=dY), dict(h=P, trans=True), dict(h=dX), T, N, K, None))
            self.calls.append((f"{name} dW", dict(h=X, trans=True), dict(h=dY), dict(h=G), K, T, N, dw_epi))
        self.flops = sum(2 * m * k * n for _, _, _, _, m, k, n, _ in self.calls)
        # Algorithmic bytes: every distinct tensor of the set once (X, W, dY read; Y, dX, dW written).  X, W and dY
        # are each read by two GEMMs; counting them per GEMM (`per_gemm_bytes`) would double them.
        self.bytes = sum(4 * 2 * (T * K + K * N + T * N) for _, K, N in LAYERS) + extra
        self.per_gemm_bytes = sum(4 * (m * k + k * n + m * n) for _, _, _, _, m, k, n, _ in self.calls)

    def call_fn(self, i, use_f16):
        import scratchtape_amd as st
        _, a, b, o, m, k, n, epi = self.calls[i]
        A, B, O = st.MatRef(**a), st.MatRef(**b), st.MatRef(**o)
        E = st.Epilogue(**epi) if epi else None
        return lambda: st.matmul_with(A, B, O, 1, m, k, n, E, use_f16)

    def step_fn(self, use_f16):
        """The 15 GEMMs one call each (the reference's dispatch pattern), in set order."""
        fns = [self.call_fn(i, use_f16) for i in range(len(self.calls))]

        def step():
            for f in fns:
                f()
        return step

    def args(self, i, use_f16):
        import scratchtape_amd as st
        _, a, b, o, m, k, n, epi = self.calls[i]
        return (st.MatRef(**a), st.MatRef(**b), st.MatRef(**o), 1, m, k, n, st.Epilogue(**epi) if epi else None,
                use_f16)

    def grouped_fn(self, use_f16):
        """The 15 GEMMs as one st_matmul_grouped call (they are independent here)."""
        import scratchtape_amd as st
        calls = [self.args(i, use_f16) for i in range(len(self.calls))]
        return lambda: st.matmul_grouped(calls)

    def step_order_fn(self, use_f16):
        """The order a training step can issue them in: the 5 forward GEMMs one by one (each needs the layer
        before), then per layer from the head down one grouped call of its dW and dX (gpu_step/tape.rs:324-347)."""
        import scratchtape_amd as st
        fwd = [self.call_fn(3 * l, use_f16) for l in range(len(LAYERS))]
        bwd = [[self.args(3 * l + 2, use_f16), self.args(3 * l + 1, use_f16)] for l in reversed(range(len(LAYERS)))]

        def step():
            for f in fwd:
                f()
            for pair in bwd:
                st.matmul_grouped(pair)
        return step


def bench_gemm_set(dev, stream, steps, warmup, use_f16):
    """Times the set three ways: one grouped call (the headline), step order (forward one by one, backward
    pairs grouped) and one call per GEMM; each eager (HIP events around the calls), as one HIP graph per step
    replayed `steps` times, and as one HIP graph of all `steps` steps (the headline timing)."""
    import torch
    ss = StepSet(dev)
    modes = {"grouped": ss.grouped_fn(use_f16), "step_order": ss.step_order_fn(use_f16),
             "serial": ss.step_fn(use_f16)}
    times = {}
    with torch.cuda.stream(stream):
        for name, fn in modes.items():
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            eager = time_events(fn, steps, stream)
            graph, _ = time_graph(fn, steps, warmup, stream)
            spread = {}
            steps_ms = time_graph_steps(fn, steps, stream, spread=spread)
            times[name] = dict(eager_ms=round(eager, 5), graph_per_step_ms=round(graph, 5),
                               graph_ms=round(steps_ms, 5), graph_spread=spread,
                               tflops=round(ss.flops / steps_ms / 1e9, 2))
        modes["grouped"]()  # the outputs the parity check reads come from the grouped launch
        torch.cuda.synchronize()
        per_call = []
        for i, (label, _, _, _, m, k, n, _) in enumerate(ss.calls):
            f = ss.call_fn(i, use_f16)
            f()
            ms = time_events(f, 50, stream)
            fl = 2 * m * k * n
            per_call.append(dict(gemm=label, m=m, k=k, n=n, ms=round(ms, 5), tflops=round(fl / ms / 1e9, 2),
                                 gbs=round(4 * (m * k + k * n + m * n) / ms / 1e6, 1)))
    modes["grouped"]()
    torch.cuda.synchronize()
    return ss, times, per_call


def bench_gemm_rotating(dev, stream, steps, use_f16, sets=3):
    """The set as one grouped call per step, but step i working on buffer set i % `sets` (each a full set of the
    step's tensors, 158 MB; together larger than the 256 MB MALL), so a step's operands are not left in the
    device's last-level cache by the step before: the rate with the operands coming from HBM."""
    import torch
    group = [StepSet(dev, seed=100 + i) for i in range(sets)]
    fns = [g.grouped_fn(use_f16) for g in group]
    it = itertools.count()
    with torch.cuda.stream(stream):
        for f in fns:
            f()
        torch.cuda.synchronize()
        spread = {}
        ms = time_graph_steps(lambda: fns[next(it) % sets](), steps, stream, spread=spread)
    flops, nbytes = group[0].flops, group[0].bytes
    del group, fns
    torch.cuda.empty_cache()
    return dict(buffer_sets=sets, bytes_per_set=nbytes, graph_ms=round(ms, 5), graph_spread=spread,
                tflops=round(flops / ms / 1e9, 2), hbm_gbs=round(nbytes / ms / 1e6, 1))


def check_gemm_set(ss, use_f16):
    """Parity of every GEMM of the timed set against the oracle (the bench refuses to report wrong numbers).  Returns
    (max scale-relative error against the oracle on the operands the route multiplies -- f16-rounded for the f16
    route -- and against the oracle on the f32 operands)."""
    import oracle
    errs, errs32 = [], []
    with oracle.threads(host_threads()):
        for label, a, b, o, m, k, n, _ in ss.calls:
            A = a["h"].cpu().numpy()
            B = b["h"].cpu().numpy()
            A = oracle.transpose(A.reshape(k, m)) if a.get("trans") else A.reshape(m, k)
            B = oracle.transpose(B.reshape(n, k)) if b.get("trans") else B.reshape(k, n)
            got = o["h"].cpu().numpy().reshape(m, n)
            want32 = oracle.matmul(A, B)
            errs32.append(float(np.max(np.abs(got - want32)) / np.max(np.abs(want32))))
            if use_f16:
                want = oracle.matmul(oracle.round_f16(A), oracle.round_f16(B))
                errs.append(float(np.max(np.abs(got - want)) / np.max(np.abs(want))))
            else:
                errs.append(errs32[-1])
    return max(errs), max(errs32)


def check_epilogue_set(ss, use_f16=True):
    """Parity of the step set with the tape's epilogues: every output buffer after ONE grouped call from known
    contents (Y, dX zero; the gradient buffers [dW, db] filled with 0.5, so the accumulate and the column sums add to
    them) against oracle.gemm with the same epilogue on the same host buffers.  Returns the largest scale-relative
    errors over the 15 products and over the 5 bias gradients (column sums, in another summation order than the
    oracle's)."""
    import torch
    import oracle
    import scratchtape_amd as st
    for X, P, dY, Y, dX, G, R in ss.bufs:
        Y.zero_()
        dX.zero_()
        G.fill_(0.5)
    st.matmul_grouped([ss.args(i, use_f16) for i in range(len(ss.calls))])
    torch.cuda.synchronize()
    errs, cs_errs = [], []
    with oracle.threads(host_threads()):
        for label, a, b, o, m, k, n, epi in ss.calls:
            ref = lambda d: dict(off=0, stride=0, trans=int(bool(d.get("trans", False))), ld=0, group=1, inner=0)
            out_h = np.zeros(o["h"].numel(), np.float32)
            kw = {}
            if epi:
                if epi.get("bias"):
                    kw["bias"] = (epi["bias"][0].cpu().numpy(), epi["bias"][1])
                if epi.get("residual"):
                    kw["residual"] = (epi["residual"][0].cpu().numpy(), 0)
                kw["relu"] = bool(epi.get("relu", False))
                if epi.get("accumulate"):
                    out_h[:] = 0.5
                    kw["accumulate"] = True
                if epi.get("col_sum"):
                    kw["col_sum"] = epi["col_sum"]
            oracle.gemm(a["h"].cpu().numpy(), ref(a), b["h"].cpu().numpy(), ref(b), out_h, ref(o), 1, m, k, n,
                        f16=use_f16, **kw)
            got = o["h"].cpu().numpy()
            rel = lambda g, w: float(np.max(np.abs(g - w)) / max(float(np.max(np.abs(w))), 1e-30))
            errs.append(rel(got[:m * n], out_h[:m * n]))
            if epi and epi.get("col_sum"):
                cs_errs.append(rel(got[m * n:m * n + n], out_h[m * n:m * n + n]))
    return max(errs), max(cs_errs)


def bench_gemm_tape_epilogues(dev, stream, steps):
    """The C3 f16 set as one grouped call with the device tape's epilogues (TAPE_EPI), graph-timed as the headline,
    and its parity against the oracle."""
    import torch
    ss = StepSet(dev, epilogues=True)
    err, cs_err = check_epilogue_set(ss)
    fn = ss.grouped_fn(True)
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        spread = {}
        ms = time_graph_steps(fn, steps, stream, spread=spread)
    out = dict(graph_ms=round(ms, 5), graph_spread=spread, tflops=round(ss.flops / ms / 1e9, 2),
               algorithmic_bytes=ss.bytes, hbm_gbs=round(ss.bytes / ms / 1e6, 1), parity_max_rel_err=err,
               parity_col_sum_max_rel_err=cs_err,
               epilogues={k: dict(relu=v[0], residual=v[1], bias=True) for k, v in TAPE_EPI.items()},
               dw_epilogue="accumulate + bias gradient as column sums")
    del ss
    torch.cuda.empty_cache()
    return out


def cpu_gemm_baseline(ss, budget_s=10.0):
    """The reference CPU path (NdArray::matmul, with the explicit transposes the tape makes) on full step sets:
    repeated for about `budget_s` seconds (at least 5 sets), one pinned core, median set time reported."""
    import oracle
    host = [(a["h"].cpu().numpy(), b["h"].cpu().numpy(), a.get("trans", False), b.get("trans", False), m, k, n)
            for _, a, b, _, m, k, n, _ in ss.calls]

    def one_set():
        t0 = time.perf_counter()
        for A, B, ta, tb, m, k, n in host:
            A2 = oracle.transpose(A.reshape(k, m)) if ta else A.reshape(m, k)
            B2 = oracle.transpose(B.reshape(n, k)) if tb else B.reshape(k, n)
            oracle.matmul(A2, B2)
        return time.perf_counter() - t0

    with one_core():
        times = [one_set()]
        while len(times) < 5 or sum(times) < budget_s:
            times.append(one_set())
    dt = float(np.median(times))
    # The same restatement with its rows split over every core of this process's share (a restatement, not
    # the reference, whose NdArray::matmul is single-threaded).
    nt = host_threads()
    with oracle.threads(nt):
        mt = [one_set()]
        while len(mt) < 5 or sum(mt) < budget_s / 3:
            mt.append(one_set())
    dtm = float(np.median(mt))
    return dict(value=round(ss.flops / dt / 1e12, 5), unit="TFLOP/s", cores=1, kind="port",
                sample=f"{len(times)} full d=256 step GEMM sets (15 GEMMs, 20.9 GFLOP each; median set time) "
                       "through the oracle's restatement of NdArray::matmul (tensor.rs:248-276) incl. the tape's "
                       "explicit transposes, 1 pinned thread, gcc -O3 -mavx2 -mfma -ffp-contract=off, "
                       f"{cpu_model()}", seconds=round(sum(times), 3),
                all_cores=dict(value=round(ss.flops / dtm / 1e12, 5), unit="TFLOP/s", cores=nt, kind="port",
                               seconds=round(sum(mt), 3),
                               sample=f"{len(mt)} sets, the same restatement with rows split over {nt} OpenMP "
                                      "threads (bit-identical results)"))


# --------------------------------------------------------------------------- smaller GEMM configs

def bench_tape_forms(dev, stream, m, k, n, use_f16, reps=50):
    """C = A·B, dA = dC·Bᵀ, dB = Aᵀ·dC with A [m,k], B [k,n], dC [m,n] uniform [-1,1] (seeded).  `ms` is the time per
    call with `reps` calls replayed as one HIP graph (as every other line), `eager_ms` per call launched eagerly."""
    import torch
    import oracle
    import scratchtape_amd as st
    rng = oracle.Rng(42)
    A, B, dC = (torch.from_numpy(rng.uniform(x)).to(dev) for x in (m * k, k * n, m * n))
    C, dA, dB = (torch.zeros(x, device=dev) for x in (m * n, m * k, k * n))
    forms = {
        "C=A·B": (lambda: st.matmul_with(st.MatRef(A), st.MatRef(B), st.MatRef(C), 1, m, k, n, None, use_f16), m, k, n),
        "dA=dC·Bᵀ": (lambda: st.matmul_with(st.MatRef(dC), st.MatRef(B, trans=True), st.MatRef(dA), 1, m, n, k, None,
                                             use_f16), m, n, k),
        "dB=Aᵀ·dC": (lambda: st.matmul_with(st.MatRef(A, trans=True), st.MatRef(dC), st.MatRef(dB), 1, k, m, n, None,
                                             use_f16), k, m, n),
    }
    out = {}
    with torch.cuda.stream(stream):
        for name, (f, mm, kk, nn) in forms.items():
            f()
            eager = time_events(f, reps, stream)
            ms = time_graph_steps(f, reps, stream)
            out[name] = dict(m=mm, k=kk, n=nn, ms=round(ms, 5), tflops=round(2 * mm * kk * nn / ms / 1e9, 3),
                             eager_ms=round(eager, 5))
    return out


# --------------------------------------------------------------------------- attention

def bench_attention(dev, stream, steps, warmup, use_f16):
    import torch
    import oracle
    from scratchtape_amd import attention
    b, h, t, hd = 32, 4, 128, 64
    d = h * hd
    rng = oracle.Rng(17)
    qkv = rng.gaussian(b * t * 3 * d)
    if use_f16:
        qkv = oracle.round_f16(qkv)
    qkv = torch.from_numpy(qkv).to(dev)
    dctx = torch.from_numpy(rng.gaussian(b * t * d)).to(dev)
    buf = attention.AttnBuffers.empty(b, h, t, hd, dev)
    step = lambda: attention.step(qkv, dctx, buf, b, h, t, hd, use_f16)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step()
        eager_ms = time_events(step, steps, stream)
        per_step_ms, _ = time_graph(step, steps, warmup, stream)
        graph_ms = time_graph_steps(step, steps, stream)
    flops = 6 * b * h * 2 * t * t * hd
    return dict(flops=flops, eager_ms=round(eager_ms, 5), graph_per_step_ms=round(per_step_ms, 5),
                graph_ms=round(graph_ms, 5), tflops=round(flops / graph_ms / 1e9, 3))


def bench_attention_fused(dev, stream, steps, warmup):
    """The same attention step as two fused launches (k_attn_fwd, k_attn_bwd): S and P never leave the chip."""
    import torch
    import oracle
    from scratchtape_amd import attention
    b, h, t, hd = 32, 4, 128, 64
    d = h * hd
    rng = oracle.Rng(17)
    qkv = torch.from_numpy(oracle.round_f16(rng.gaussian(b * t * 3 * d))).to(dev)
    dctx = torch.from_numpy(rng.gaussian(b * t * d)).to(dev)
    buf = attention.FusedBuffers.empty(b, h, t, hd, dev)
    fwd = lambda: attention.fused_forward(qkv, buf, b, h, t, hd)
    bwd = lambda: attention.fused_backward(qkv, dctx, buf, b, h, t, hd)
    step = lambda: attention.fused_step(qkv, dctx, buf, b, h, t, hd)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step()
        eager_ms = time_events(step, steps, stream)
        fwd_ms = time_events(fwd, steps, stream)
        bwd_ms = time_events(bwd, steps, stream)
        per_step_ms, _ = time_graph(step, steps, warmup, stream)
        graph_ms = time_graph_steps(step, steps, stream)
    flops = 6 * b * h * 2 * t * t * hd  # the six products of the unfused step, for comparison
    # Algorithmic bytes: qkv read by both passes, dctx, ctx written then read, lse, dqkv written.
    nbytes = 4 * (2 * b * t * 3 * d + b * t * d + 2 * b * t * d + 2 * b * h * t + b * t * 3 * d)
    return dict(flops=flops, eager_ms=round(eager_ms, 5), graph_per_step_ms=round(per_step_ms, 5),
                graph_ms=round(graph_ms, 5), fwd_ms=round(fwd_ms, 5),
                bwd_ms=round(bwd_ms, 5), tflops=round(flops / graph_ms / 1e9, 3),
                roofline=roofline("k_attn_fwd + k_attn_bwd (fused f16 attention step)", flops, nbytes, graph_ms,
                                  traffic_for("k_attn fused step", "scratchtape_amd/csrc/attn.hip")))


def bench_layer_norm(dev, stream, steps, warmup):
    """LayerNorm forward + backward at the step shape (T = 4096 rows of d_model 256), one parameter set."""
    import torch
    import oracle
    from scratchtape_amd import rows
    n, d = T_TOKENS, 256
    rng = oracle.Rng(29)
    x = torch.from_numpy(rng.gaussian(n * d)).to(dev)
    dy = torch.from_numpy(rng.gaussian(n * d)).to(dev)
    params = torch.from_numpy(np.concatenate([1.0 + 0.1 * rng.gaussian(d), 0.1 * rng.gaussian(d)]).astype(np.float32)).to(dev)
    grads = torch.zeros(2 * d, device=dev)
    dx = torch.empty(n * d, device=dev)
    box = {}

    def fwd():
        box["f"] = rows.layer_norm(x, n, d, params, 0, 1e-5)

    def step():
        fwd()
        rows.layer_norm_backward(dy, x, box["f"], n, d, params, grads, 0, dx, False)

    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step()
        fwd_ms = time_events(fwd, steps, stream)
        per_step_ms, _ = time_graph(step, steps, warmup, stream)
        graph_ms = time_graph_steps(step, steps, stream)
    # Algorithmic bytes: x read and y written (forward); dy and x read, dx written (backward); mean, rstd.
    nbytes = 4 * (5 * n * d + 4 * n)
    return dict(rows=n, d=d, fwd_ms=round(fwd_ms, 5), graph_per_step_ms=round(per_step_ms, 5),
                graph_ms=round(graph_ms, 5),
                roofline=roofline("k_ln_fwd4 + k_ln_bwd4 + k_ln_bwd_sum4", 10 * n * d, nbytes,
                                  graph_ms, traffic_for("k_ln step", "scratchtape_amd/csrc/rows.hip"), route="f32"))


def cpu_attention_baseline(reps=20):
    import oracle
    b, h, t, hd = 32, 4, 128, 64
    rng = oracle.Rng(3)
    q, k, v, do = (rng.gaussian(b * h * t * hd) for _ in range(4))
    times = []
    with one_core():
        for _ in range(reps):
            t0 = time.perf_counter()
            oracle.attention_fwd_bwd(q, k, v, do, b * h, t, hd, hd ** -0.5)
            times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    flops = 6 * b * h * 2 * t * t * hd
    return dict(value=round(flops / dt / 1e12, 5), unit="TFLOP/s", cores=1, kind="port", seconds=round(sum(times), 3),
                sample=f"{reps} full attention fwd+bwd passes (128 chunks of 128x128x64 each; median) through the "
                       "per-chunk loop of tape.rs:73-112 restated in the oracle, 1 pinned thread")


# --------------------------------------------------------------------------- kNN

NQ_CPU = 256  # queries of one batch scored by the CPU baseline (a whole batch, about 4 s of one core)


class KnnBench:
    N, NCELLS, NQ, NPROBE, D = 125_000_000, 12288, 256, 8, 256

    def __init__(self, dev, batches=8, seed=2024):
        import torch
        from scratchtape_amd import knn
        rng = np.random.default_rng(seed)
        sizes = rng.multinomial(self.N, np.full(self.NCELLS, 1.0 / self.NCELLS))
        self.cs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
        self.codes = torch.empty((self.N, self.D // 4), dtype=torch.uint8, device=dev)
        self.scales = torch.empty(self.N, dtype=torch.float32, device=dev)
        t0 = time.perf_counter()
        knn.synth_store_2bit(seed, 0, self.codes, self.scales)
        torch.cuda.synchronize()
        self.gen_s = time.perf_counter() - t0
        self.store = knn.KnnStore2bit(self.codes, self.scales, self.cs)
        self.batches = []
        for _ in range(batches):
            q = rng.standard_normal((self.NQ, self.D)).astype(np.float32)
            p = np.stack([rng.choice(self.NCELLS, self.NPROBE, replace=False) for _ in range(self.NQ)]).astype(np.int32)
            pairs = int(sizes[p].sum())
            distinct = np.unique(p)
            dbytes = int(sizes[distinct].sum()) * (self.D // 4 + 4)
            self.batches.append(dict(q=torch.from_numpy(q).to(dev), p=torch.from_numpy(p).to(dev), qh=q, ph=p,
                                     pairs=pairs, bytes=dbytes))
        self.out = (torch.empty((self.NQ, 128), dtype=torch.int64, device=dev),
                    torch.empty((self.NQ, 128), dtype=torch.float32, device=dev))

    def wide_batch(self, dev, nq=4096, seed=4096):
        """One batch of `nq` queries x 8 probes over the same store (cells shared by ~nq * 8 / 12288 queries each),
        with its own output buffers."""
        import torch
        rng = np.random.default_rng(seed)
        sizes = np.diff(self.cs)
        q = rng.standard_normal((nq, self.D)).astype(np.float32)
        p = np.stack([rng.choice(self.NCELLS, self.NPROBE, replace=False) for _ in range(nq)]).astype(np.int32)
        return dict(q=torch.from_numpy(q).to(dev), p=torch.from_numpy(p).to(dev), qh=q, ph=p,
                    pairs=int(sizes[p].sum()), bytes=int(sizes[np.unique(p)].sum()) * (self.D // 4 + 4),
                    out=(torch.empty((nq, 128), dtype=torch.int64, device=dev),
                         torch.empty((nq, 128), dtype=torch.float32, device=dev)))

    def search(self, i):
        bt = self.batches[i % len(self.batches)]
        return self.store.search_ivf(bt["q"], bt["p"], 128, out=self.out)

    def run(self, stream, steps, warmup):
        import torch
        with torch.cuda.stream(stream):
            for i in range(warmup):
                self.search(i)
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            for i in range(steps):
                self.search(i)
            e.record(stream)
            e.synchronize()
            eager_ms = s.elapsed_time(e) / steps
            # The same eager searches again, queued right behind ~25 ms of untimed ones so that the device is at its
            # sustained clocks (the figure above starts right after the CPU-bound parity check, on an idle device).
            for i in range(max(1, int(25.0 / max(eager_ms, 1e-3)))):
                self.search(i)
            s.record(stream)
            for i in range(steps):
                self.search(i)
            e.record(stream)
            e.synchronize()
            eager_warm_ms = s.elapsed_time(e) / steps
            # The same K searches (batches 0 .. K-1) captured as one HIP graph, as the GEMM lines are timed.
            used, it = [], itertools.count()

            def one():
                i = next(it)
                used.append(i)
                self.search(i)
            spread = {}
            ms = time_graph_steps(one, steps, stream, spread=spread)
        nb = len(self.batches)
        used = used[1:1 + steps]  # the call before the capture is not in the graph
        pairs = np.mean([self.batches[i % nb]["pairs"] for i in used])
        byts = np.mean([self.batches[i % nb]["bytes"] for i in used])
        return ms, pairs, byts, dict(eager_ms=round(eager_ms, 5), eager_warm_ms=round(eager_warm_ms, 5),
                                     graph_spread=spread)

    def check(self, qis=(0, 100, 255), bt=None):
        """Bit-exact top-128 for a few queries of batch 0 (or of `bt`, a wide batch) against the oracle over the
        same stored bytes."""
        import torch
        import oracle
        if bt is None:
            idx, dist = self.search(0)
            bt = self.batches[0]
        else:
            idx, dist = self.store.search_ivf(bt["q"], bt["p"], 128, out=bt["out"])
        idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
        for qi in qis:
            cells = bt["ph"][qi]
            rows = np.concatenate([np.arange(self.cs[c], self.cs[c + 1]) for c in cells])
            sub = np.concatenate([[0], np.cumsum([self.cs[c + 1] - self.cs[c] for c in cells])]).astype(np.int64)
            sel = torch.from_numpy(rows).to(self.codes.device)
            widx, wdist = oracle.knn_search(self.codes[sel].cpu().numpy(), self.scales[sel].cpu().numpy(), sub,
                                            bt["qh"][qi:qi + 1], np.arange(len(cells), dtype=np.int32)[None], 128)
            if not (np.array_equal(idx[qi], rows[widx[0]]) and np.array_equal(dist[qi], wdist[0])):
                return False
        return True

    def cpu_baseline(self, nq=NQ_CPU):
        """The oracle's exact 2-bit scoring + top-128 over the same probed cells, 1 pinned thread."""
        import torch
        import oracle
        bt = self.batches[1]
        total_pairs, dt = 0, 0.0
        for qi in range(nq):
            cells = bt["ph"][qi]
            rows = np.concatenate([np.arange(self.cs[c], self.cs[c + 1]) for c in cells])
            sub = np.concatenate([[0], np.cumsum([self.cs[c + 1] - self.cs[c] for c in cells])]).astype(np.int64)
            sel = torch.from_numpy(rows).to(self.codes.device)
            codes, scales = self.codes[sel].cpu().numpy(), self.scales[sel].cpu().numpy()
            with one_core():
                t0 = time.perf_counter()
                oracle.knn_search(codes, scales, sub, bt["qh"][qi:qi + 1],
                                  np.arange(len(cells), dtype=np.int32)[None], 128)
                dt += time.perf_counter() - t0
            total_pairs += rows.size
        # All cores: up to the whole batch in one call, each query's probed rows gathered as one cell.
        nt = host_threads()
        nqa = min(self.NQ, 16 * nt)
        parts, starts, npairs = [], [0], 0
        for qi in range(nqa):
            cells = bt["ph"][qi]
            rows = np.concatenate([np.arange(self.cs[c], self.cs[c + 1]) for c in cells])
            parts.append(rows)
            starts.append(starts[-1] + rows.size)
            npairs += rows.size
        sel = torch.from_numpy(np.concatenate(parts)).to(self.codes.device)
        codes, scales = self.codes[sel].cpu().numpy(), self.scales[sel].cpu().numpy()
        with oracle.threads(nt):
            t0 = time.perf_counter()
            oracle.knn_search(codes, scales, np.array(starts, np.int64), bt["qh"][:nqa],
                              np.arange(nqa, dtype=np.int32)[:, None], 128)
            dtm = time.perf_counter() - t0
        return dict(value=round(total_pairs / dt / 1e9, 5), unit="G keys/s", cores=1, kind="port",
                    seconds=round(dt, 3),
                    sample=f"{nq} queries x 8 probed cells of the 125M-key store ({total_pairs} pairs), exact 2-bit "
                           "scoring + top-128 by (score, index) in the oracle (C, 1 pinned thread); the reference has "
                           "no CPU quantised scorer",
                    all_cores=dict(value=round(npairs / dtm / 1e9, 5), unit="G keys/s", cores=nt, kind="port",
                                   seconds=round(dtm, 3),
                                   sample=f"{nqa} queries ({npairs} pairs) in one call, queries split over {nt} "
                                          "OpenMP threads"))


class ProbeBench:
    """IVF probe selection at the scan benchmark's batch: 12288 centroids N(0,1), 256 queries, 8 probes each."""
    NLIST, NQ, NPROBE, D = 12288, 256, 8, 256

    def __init__(self, dev, queries, seed=77):
        import torch
        from scratchtape_amd import knn
        g = torch.Generator(device=dev).manual_seed(seed)
        self.cent = torch.randn((self.NLIST, self.D), generator=g, device=dev)
        self.c = knn.Centroids(self.cent)
        self.queries = queries
        self.out = torch.empty((self.NQ, self.NPROBE), dtype=torch.int32, device=dev)
        nct, nqt = -(-self.NLIST // 16), -(-self.NQ // 16)
        # Algorithmic bytes: the centroid store (512 B of digits + 12 B of exponent and norm per cell), the f32
        # queries and the probe ids.  Matrix-core work: 8 k-steps of one 32x32x32 i8 MFMA per (query tile,
        # centroid tile) of 16 vectors each, i.e. the four digit products of every query-centroid dot.
        self.bytes = self.NLIST * (512 + 12) + self.NQ * self.D * 4 + self.NQ * self.NPROBE * 4
        self.ops = nqt * nct * 8 * 2 * 32 * 32 * 32

    def probe(self, i):
        return self.c.probe(self.queries[i % len(self.queries)], self.NPROBE, out=self.out)

    def run(self, stream, steps, warmup):
        import torch
        it = itertools.count()
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                self.probe(next(it))
            torch.cuda.synchronize()
            eager_ms = time_events(lambda: self.probe(next(it)), steps, stream)
            spread = {}
            ms = time_graph_steps(lambda: self.probe(next(it)), steps, stream, spread=spread)
        return ms, dict(eager_ms=round(eager_ms, 5), graph_spread=spread)

    def check(self):
        import oracle
        got = self.probe(0).cpu().numpy()
        return bool(np.array_equal(got, oracle.knn_probe(self.cent.cpu().numpy(), self.queries[0].cpu().numpy(),
                                                         self.NPROBE)))

    def cpu_baseline(self):
        """The oracle's exact probe selection for one whole batch, 1 pinned thread."""
        import oracle
        prep = oracle.knn_centroid_prep(self.cent.cpu().numpy())
        q = self.queries[1].cpu().numpy()
        with one_core():
            t0 = time.perf_counter()
            oracle.knn_probe(None, q, self.NPROBE, prep=prep)
            dt = time.perf_counter() - t0
        return dict(value=round(self.NQ / dt, 1), unit="queries/s", cores=1, kind="port", seconds=round(dt, 3),
                    sample=f"{self.NQ} queries x {self.NLIST} centroids x {self.NPROBE} probes (one batch): exact "
                           "integer distances + top-8 in the oracle (C, 1 pinned thread)")


# --------------------------------------------------------------------------- device ceilings

def device_ceilings(dev, stream):
    """Measured ceilings beside the published peaks every roofline is priced against: the matrix cores with only
    independent MFMA chains in flight (two waves per SIMD, 8 chains each; `mfma_f16` / `mfma_i8` in the 32 x 32
    forms the kernels use, the 16 x 16 forms beside them), a streaming read of 1 GiB (eight workgroups of 4 waves
    per CU, each reading its own slab with sixteen nontemporal 16-byte loads per lane in flight: the fastest read
    shape measured), and the device's CU count and clocks (HIP device attributes)."""
    import ctypes
    import torch
    from scratchtape_amd import _lib
    vals = [ctypes.c_int32() for _ in range(4)]
    _lib.call("st_device_info", *[ctypes.byref(v) for v in vals])
    cus, clk, mclk, bus = (v.value for v in vals)
    out = dict(cus=cus, clock_mhz=clk / 1e3, mem_clock_mhz=mclk / 1e3, mem_bus_bits=bus)
    blocks, iters, chains, waves = 2 * cus, 20000, 8, 4
    sink = torch.zeros(8 * cus, device=dev)
    with torch.cuda.stream(stream):
        for kind, name, per in ((0, "f16_16x16x32", 16384), (3, "f16", 32768), (1, "f32", 2048),
                                (2, "i8_16x16x64", 32768), (4, "i8", 65536)):
            f = lambda: _lib.call("st_peak_mfma", kind, iters, blocks, sink.data_ptr(), stream.cuda_stream)
            f()
            ms = time_events(f, 5, stream)
            out[f"mfma_{name}_tflops_measured"] = round(blocks * waves * chains * iters * per / ms / 1e9, 1)
        buf = torch.empty(1 << 28, dtype=torch.float32, device=dev)
        g = lambda: _lib.call("st_peak_read", buf.data_ptr(), buf.numel() * 4, 8 * cus, sink.data_ptr(),
                              stream.cuda_stream)
        g()
        ms = time_events(g, 10, stream)
        out["hbm_read_gbs_measured"] = round(buf.numel() * 4 / ms / 1e6, 1)
        del buf
    out["published_peaks"] = dict(PEAK)
    return out


# --------------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["all", "gemm", "knn", "gemm_set"], default="all",
                    help="gemm_set: only the headline f16 step set as one grouped call (warm-up, the graph-timed "
                         "steps, parity), one JSON line: the workload its rocprofv3 counter summary is taken on")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run a plain 256 MiB device copy 10 times (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.calib_copy:
        import torch
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes_each_way": src.numel() * 4, "dispatches": 10}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library runs on a single MI355X (asked for --gpus {args.gpus}); "
              "how the path would shard over more is a design note, not a measured run", file=sys.stderr)
        sys.exit(2)

    import torch
    import scratchtape_amd as st
    st.lib()
    dev = torch.device("cuda:0")
    torch.cuda.init()
    stream = torch.cuda.Stream(device=dev)
    prop = torch.cuda.get_device_properties(dev)
    extra = {"device": {"name": prop.name}, "host_cpu": cpu_model(), "nproc": os.cpu_count()}
    result = None

    if args.only == "gemm_set":
        ss = StepSet(dev)
        fn = ss.grouped_fn(True)
        with torch.cuda.stream(stream):
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            ms = time_graph_steps(fn, args.steps, stream)
        err, _ = check_gemm_set(ss, True)
        print(json.dumps(dict(workload="d_model-256 step GEMM set, f16 route, one grouped call", steps=args.steps,
                              ms_per_step=round(ms, 5), tflops=round(ss.flops / ms / 1e9, 2),
                              parity_max_rel_err=err)))
        sys.exit(0 if err <= 1e-5 else 3)

    if args.only in ("all", "gemm"):
        log("[bench] C3 step GEMM set, f16-in/f32-acc")
        ss16, t16, calls16 = bench_gemm_set(dev, stream, args.steps, args.warmup, True)
        err16, err16_f32 = check_gemm_set(ss16, True)
        log(f"[bench] f16 set: {t16}, parity {err16:.2e} (f16-rounded operands), {err16_f32:.2e} (f32 operands)")
        rot16 = bench_gemm_rotating(dev, stream, args.steps, True)
        log(f"[bench] f16 set over rotating buffer sets: {rot16}")
        log("[bench] C3 step GEMM set, f32")
        ss32, t32, calls32 = bench_gemm_set(dev, stream, args.steps, args.warmup, False)
        err32, _ = check_gemm_set(ss32, False)
        log(f"[bench] f32 set: {t32}, parity {err32:.2e}")
        if err16 > 1e-5 or err16_f32 > 2e-3 or err32 > 1e-5:
            log("[bench] PARITY FAILURE: refusing to report")
            sys.exit(3)
        graph16 = t16["grouped"]["graph_ms"]
        value = ss16.flops / graph16 / 1e9
        # The dominant kernel is the grouped launch itself (k_gemm_group16, plus the split-k sum k_sum_group):
        # the set's flops and algorithmic bytes over its time per step with the K timed steps replayed as one
        # HIP graph, from HIP events on its stream.
        roof = roofline("k_gemm_group16 (+ k_sum_group): the 15-GEMM f16 set in one grouped call", ss16.flops,
                        ss16.bytes, graph16,
                        traffic_for("k_gemm_group16 f16 step set", "scratchtape_amd/csrc/gemm_group.hip"))
        extra["c3_f16_set"] = dict(flops=ss16.flops, algorithmic_bytes=ss16.bytes,
                                   per_gemm_bytes=ss16.per_gemm_bytes, graph_ms=graph16,
                                   tflops=round(value, 2), mfma_frac=round(value / PEAK["f16"], 4),
                                   hbm_gbs=round(ss16.bytes / graph16 / 1e6, 1), modes=t16, per_gemm=calls16,
                                   rotating=rot16, parity_max_rel_err=err16, parity_max_rel_err_vs_f32=err16_f32)
        g32 = t32["grouped"]["graph_ms"]
        v32 = ss32.flops / g32 / 1e9
        extra["c3_f32_set"] = dict(graph_ms=g32, tflops=round(v32, 2), mfma_frac=round(v32 / PEAK["f32"], 4),
                                   roofline=roofline("k_gemm_group f32 (+ k_sum_group)", ss32.flops, ss32.bytes, g32,
                                                     route="f32"),
                                   modes=t32, per_gemm=calls32, parity_max_rel_err=err32)
        log("[bench] C3 f16 set with the device tape's epilogues")
        extra["c3_f16_set_tape_epilogues"] = bench_gemm_tape_epilogues(dev, stream, args.steps)
        log(f"[bench] tape-epilogue set: {extra['c3_f16_set_tape_epilogues']}")
        te = extra["c3_f16_set_tape_epilogues"]
        if te["parity_max_rel_err"] > 1e-5 or te["parity_col_sum_max_rel_err"] > 1e-4:
            log("[bench] PARITY FAILURE: refusing to report")
            sys.exit(3)
        log("[bench] C1 / C2 tape forms")
        extra["c1_256cube_f32"] = bench_tape_forms(dev, stream, 256, 256, 256, False)
        extra["c2_backward_f32"] = bench_tape_forms(dev, stream, 4096, 256, 1024, False)
        extra["c2_backward_f16"] = bench_tape_forms(dev, stream, 4096, 256, 1024, True)
        log("[bench] C4 attention")
        extra["c4_attention_f16"] = bench_attention(dev, stream, args.steps, args.warmup, True)
        extra["c4_attention_f32"] = bench_attention(dev, stream, args.steps, args.warmup, False)
        extra["c4_attention_fused_f16"] = bench_attention_fused(dev, stream, args.steps, args.warmup)
        extra["c3_layer_norm"] = bench_layer_norm(dev, stream, args.steps, args.warmup)
        cpu = None
        if not args.no_cpu:
            log("[bench] CPU baselines (oracle, 1 thread)")
            cpu = cpu_gemm_baseline(ss16)
            extra["c4_attention_cpu_baseline"] = cpu_attention_baseline()
        result = dict(metric=METRIC, value=round(value, 3), unit="TFLOP/s", n_gpus=1, steps=args.steps,
                      warmup=args.warmup, ms_per_step=round(graph16, 5), higher_is_better=True, scaling="weak",
                      vs_baseline=None, dtype="f16-in/f32-acc",
                      data="synthetic (seeded nn::Rng restatement: weights N(0,0.02), activations N(0,1))",
                      config=dict(workload="d_model-256 training-step GEMM set: T=4096 tokens, QKV/out/FFN1/FFN2/"
                                           "head forward + dX + dW (15 GEMMs), f32 operands in HBM, f16-in/f32-acc",
                                  global_batch=T_TOKENS, seq_len=128, parallelism="none (1 GPU)"),
                      roofline=roof, cpu_baseline=cpu)
        del ss16, ss32
        torch.cuda.empty_cache()

    if args.only in ("all", "knn"):
        log("[bench] C5 kNN store (125M 2-bit keys)")
        kb = KnnBench(dev)
        ok = kb.check()
        log(f"[bench] kNN store generated in {kb.gen_s:.2f} s; parity {'ok' if ok else 'FAILED'}")
        if not ok:
            log("[bench] PARITY FAILURE: refusing to report")
            sys.exit(3)
        ms, pairs, byts, timing = kb.run(stream, args.steps, args.warmup)
        gbs = byts / ms / 1e6
        knn = dict(ms_per_batch=round(ms, 5), **timing, keys_per_s=round(pairs / ms * 1e3, 1),
                   g_keys_per_s=round(pairs / ms / 1e6, 3), pairs_per_batch=int(pairs),
                   distinct_cell_bytes=int(byts), hbm_gbs=round(gbs, 1), hbm_frac=round(gbs / PEAK["hbm_gbs"], 4),
                   roofline=dict(kernel="k_search (st_knn_search_ivf_2bit: one fused launch)", bound="hbm",
                                 achieved=round(gbs, 1), peak=PEAK["hbm_gbs"], unit="GB/s",
                                 frac=round(gbs / PEAK["hbm_gbs"], 4),
                                 traffic=traffic_for("k_search", "scratchtape_amd/csrc/knn.hip"),
                                 algorithmic_bytes=int(byts)),
                   store_gen_s=round(kb.gen_s, 3))
        if not args.no_cpu:
            knn["cpu_baseline"] = kb.cpu_baseline()
        extra["c5_knn"] = knn
        log("[bench] C5 kNN store, one 4096-query batch")
        wb = kb.wide_batch(dev)
        if not kb.check((0, 1777, 4095), bt=wb):
            log("[bench] PARITY FAILURE (4096-query batch): refusing to report")
            sys.exit(3)
        with torch.cuda.stream(stream):
            for _ in range(args.warmup):
                kb.store.search_ivf(wb["q"], wb["p"], 128, out=wb["out"])
            torch.cuda.synchronize()
            wsteps = max(1, min(args.steps, 5))
            wms = time_graph_steps(lambda: kb.store.search_ivf(wb["q"], wb["p"], 128, out=wb["out"]), wsteps, stream)
        wgbs = wb["bytes"] / wms / 1e6
        extra["c5_knn_4096q"] = dict(ms_per_batch=round(wms, 5), queries=4096, pairs_per_batch=wb["pairs"],
                                     g_keys_per_s=round(wb["pairs"] / wms / 1e6, 3),
                                     distinct_cell_bytes=wb["bytes"], hbm_gbs=round(wgbs, 1),
                                     hbm_frac=round(wgbs / PEAK["hbm_gbs"], 4), steps_per_graph=wsteps,
                                     roofline=dict(kernel="cell-major scan (k_group_* + k_search_cells + "
                                                          "k_merge_parts)", bound="hbm", achieved=round(wgbs, 1),
                                                   peak=PEAK["hbm_gbs"], unit="GB/s",
                                                   frac=round(wgbs / PEAK["hbm_gbs"], 4),
                                                   traffic=traffic_for("k_search cell-major 4096q",
                                                                       "scratchtape_amd/csrc/knn.hip"),
                                                   algorithmic_bytes=int(wb["bytes"])))
        del wb
        log("[bench] C5 probe selection (12288 centroids, 256 queries x 8)")
        pb = ProbeBench(dev, [b["q"] for b in kb.batches])
        pok = pb.check()
        log(f"[bench] probe parity {'ok' if pok else 'FAILED'}")
        if not pok:
            log("[bench] PARITY FAILURE: refusing to report")
            sys.exit(3)
        pms, ptiming = pb.run(stream, args.steps, args.warmup)
        probe = dict(ms_per_batch=round(pms, 5), **ptiming, queries_per_s=round(pb.NQ / pms * 1e3, 1),
                     roofline=roofline("st_knn_probe (k_probe_part + k_probe_merge)", pb.ops,
                                       pb.bytes, pms,
                                       traffic_for("st_knn_probe", "scratchtape_amd/csrc/knn_probe.hip"), route="i8"))
        if not args.no_cpu:
            probe["cpu_baseline"] = pb.cpu_baseline()
        # search_ivf by nprobe: probe selection, then the scan of the selected cells (the store's cells are a
        # uniform assignment, unrelated to these centroids: the timing, not the recall, is the point).
        # Masked exact search (search_tail's use): 256 queries, each over its own window of 81,920 keys
        # (the IVF batch's mean keys per query) at a random place in the 125M-key store.
        rng = np.random.default_rng(7)
        lo = rng.integers(0, kb.N - 81920, (8, kb.NQ))
        lohis = [torch.from_numpy(np.stack([l, l + 81920], 1).astype(np.int64)).to(dev) for l in lo]
        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                kb.store.search_masked(kb.batches[i % 8]["q"], lohis[i % 8], 0, 128, out=kb.out)
            torch.cuda.synchronize()
            it = itertools.count()

            def masked():
                i = next(it)
                kb.store.search_masked(kb.batches[i % 8]["q"], lohis[i % 8], 0, 128, out=kb.out)
            meager = time_events(masked, args.steps, stream)
            mspread = {}
            mms = time_graph_steps(masked, args.steps, stream, spread=mspread)
        mbytes = kb.NQ * 81920 * (kb.D // 4 + 4)
        extra["c5_knn_masked"] = dict(ms_per_batch=round(mms, 5), eager_ms=round(meager, 5), graph_spread=mspread,
                                      g_keys_per_s=round(kb.NQ * 81920 / mms / 1e6, 3),
                                      roofline=dict(kernel="k_search<MASKED> (st_knn_search_masked_2bit)", bound="hbm",
                                                    achieved=round(mbytes / mms / 1e6, 1), peak=PEAK["hbm_gbs"],
                                                    unit="GB/s", frac=round(mbytes / mms / 1e6 / PEAK["hbm_gbs"], 4),
                                                    traffic=traffic_for("k_search masked",
                                                                        "scratchtape_amd/csrc/knn.hip"),
                                                    algorithmic_bytes=int(mbytes)))
        kb.store.centroids = pb.c
        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                kb.store.search_ivf(kb.batches[i % 8]["q"], 8, 128, out=kb.out)
            torch.cuda.synchronize()
            it = itertools.count()
            e2e = time_graph_steps(lambda: kb.store.search_ivf(kb.batches[next(it) % 8]["q"], 8, 128, out=kb.out),
                                   args.steps, stream)
        probe["search_ivf_by_nprobe_ms_per_batch"] = round(e2e, 5)
        extra["c5_knn_probe"] = probe
        del pb
        if result is None:
            result = dict(metric=METRIC, value=knn["g_keys_per_s"], unit="G keys/s", n_gpus=1, steps=args.steps,
                          warmup=args.warmup, ms_per_step=knn["ms_per_batch"], higher_is_better=True,
                          scaling="weak", vs_baseline=None, dtype="u8 codes / int32 dot",
                          data="synthetic (counter-based N(0,1) keys, seeded queries and probes)",
                          config=dict(workload="125M 2-bit keys, 12288 cells, 256 queries x 8 probes, top-128"),
                          roofline=knn["roofline"], cpu_baseline=knn.get("cpu_baseline"))
        del kb
        torch.cuda.empty_cache()

    log("[bench] device ceilings")
    extra["device"].update(device_ceilings(dev, stream))
    result["extra"] = extra
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
