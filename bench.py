"""Benchmark of the quantized matrix-product path on one MI355X.

Headline (`value`): decode tokens/s of the Qwen2-0.5B-shaped step (hidden 896, 24 layers, 14
query / 2 KV heads of 64, FFN 4864, vocabulary 151936 tied embedding/head, Q7b32 weights) for one
token at position 511 over a 511-entry f32 KV cache, every projection through the GPU matrix-vector
kernel, the whole step replayed as one HIP graph. Inputs are synthetic and seeded; everything is
resident in HBM before the timed region.

`roofline` is the matrix-vector kernel's achieved HBM bandwidth over the step's projections: their
algorithmic bytes (weight codes + scales + int8 activations with scales and corrections + f32
outputs) over the kernel's duration, measured with HIP events on the launch stream.

`cpu_baseline` is the oracle (a C restatement of the reference's scalar x86-64 path, column-split
over threads like the reference's team) timed on this host: the decode step at the reference CLI's
default team of min(8, cores - 2) threads, one warm-up then the mean over a bounded number of steps,
the steady-state best of five, and the same on every core; the host's CPU model and count.

Extra fields: the single 4864 x 896 matvec (resident; streamed over 64 copies, one launch each;
all 64 copies as one 311296 x 896 table in one launch), the batched GEMMs (512 x 896 -> 9728,
512 x 4864 -> 896, DiT 4096-row shapes), the packed-int4 14336 x 4096 product (rows 1 and 16)
and the int8 attention at the DiT shape. Every product carries its own CPU baseline (the oracle's
quantization and product, same protocol; the 4096-row shapes on a sample of their rows).
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "fusor-ai_amd")]

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
SIMDS, CLOCK_HZ = 1024, 2.4e9
# The exact product's issue floor on one SIMD, in cycles per 32 x 32 output tile and 32-deep block:
# its int8 MFMA, half an f32 outer product (the scale products of two blocks) and the rescale of 16
# outputs per lane, issued by four waves per SIMD from registers alone (no memory, no LDS), measured
# on MI355X. The matrix cores and the VALU do not overlap on a SIMD (an MFMA wave beside a VALU wave
# takes the sum of their times), so this is the sum of both, not the larger: 203 cycles with the
# scalar backend's convert, multiply and add; 162 with the NEON backend's convert and FMA.
ISSUE_CYCLES_EXACT, ISSUE_CYCLES_FUSED = 203.0, 162.0
METRIC = "int8 qmatvec weight GB/s (% HBM peak); Qwen2-0.5B-shape decode tokens/sec"

Q7B32, Q4B32, T2B128, Q8B32 = 1, 2, 3, 4


def measured_traffic():
    """HBM bytes per launch of the projection pass from the committed counter summary (two
    rocprofv3 --pmc runs, FETCH_SIZE and WRITE_SIZE, scaled by a copy of known size); None when
    the summary is absent."""
    path = os.path.join(ROOT, "profiles", "proj_kernel_qwen2_0.5b_projections_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch = "):
                    return int(line.split("=")[1])
    except OSError:
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_cpu():
    """The host's CPU model, logical CPU count and the CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = nproc
    return model, nproc, usable


def cpu_thread_counts():
    """The reference CLI's default team, min(8, cores - 2) (crates/harness/src/lib.rs:36-44), and
    every core this process may use."""
    _, _, usable = host_cpu()
    return max(1, min(8, usable - 2)), usable


def cpu_protocol(call, calls=3):
    """Milliseconds per call two ways: one warm-up call then the mean of `calls` calls
    (crates/harness/src/bench.rs:8-17), and the steady state of tools/kernel-harness/bench.mjs:29-40
    (iterations doubling until a run takes at least 80 ms, then the best of five runs)."""
    call()
    t0 = time.perf_counter()
    for _ in range(calls):
        call()
    mean_ms = (time.perf_counter() - t0) * 1e3 / calls
    iters = 1
    while True:
        t0 = time.perf_counter()
        for _ in range(iters):
            call()
        if time.perf_counter() - t0 >= 0.08:
            break
        iters *= 2
    best = float("inf")
    for _ in range(5):
        t0 = time.perf_counter()
        for _ in range(iters):
            call()
        best = min(best, time.perf_counter() - t0)
    return mean_ms, best * 1e3 / iters


def cpu_product_baseline(np, dtype, n, k, table_bytes, x, rate, unit, sample):
    """The oracle's product (quantize_rows, then the column- or row-split product of the
    reference's scalar path) on this host at the reference's default team size and on every core;
    `rate(ms)` turns milliseconds per call into the workload's figure."""
    from oracle import oracle as O
    rows = x.shape[0]
    default, every = cpu_thread_counts()
    model, nproc, _ = host_cpu()

    def run(threads):
        def call():
            q, sc, co = O.quantize_rows(x.reshape(-1), dtype)
            O.matmul_threaded(dtype, n, k, table_bytes, q, sc, co, rows, threads=threads)
        mean_ms, best_ms = cpu_protocol(call)
        return {"value": float(f"{rate(best_ms):.4g}"), "mean_ms": round(mean_ms, 3), "best_of_5_ms": round(best_ms, 3)}

    line = {"unit": unit, "cores": default, "kind": "port", "sample": sample, "cpu": model, "nproc": nproc,
            "value_from": "best of 5 (mean of 3 after one warm-up also given)"}
    line.update(run(default))
    line["all_cores"] = dict(run(every), cores=every)
    return line


def synthetic_table(np, dtype, rows, cols, rng):
    """Reference bytes of a [rows, cols] table: i.i.d. codes (Q7b32 levels uniform in [-63, 63],
    Q8b32 in [-127, 127], Q4b32 nibbles, T2b128 ternary codes 0-2 in each two bits) and scales
    uniform in [1e-3, 1e-2]. rows % 4 == 0."""
    assert rows % 4 == 0
    n_codes = rows * cols // {Q4B32: 2, T2B128: 4}.get(dtype, 1)
    if dtype == Q7B32:
        codes = rng.integers(1, 128, n_codes, dtype=np.uint8)
    elif dtype == Q8B32:
        codes = rng.integers(-127, 128, n_codes, dtype=np.int16).astype(np.int8).view(np.uint8)
    elif dtype == T2B128:
        parts = rng.integers(0, 3, (n_codes, 4), dtype=np.uint8)
        codes = (parts[:, 0] | parts[:, 1] << 2 | parts[:, 2] << 4 | parts[:, 3] << 6).astype(np.uint8)
    else:
        codes = rng.integers(0, 256, n_codes, dtype=np.uint8)
    scales = rng.uniform(1e-3, 1e-2, rows * cols // (128 if dtype == T2B128 else 32)).astype(np.float32)
    return np.concatenate([codes, scales.view(np.uint8)])


class Timer:
    """HIP events on the current stream around a callable run `reps` times. With `graph`, the
    calls are captured once into a HIP graph (`reps` launches of `fn`) and the graph is replayed,
    so that the figure is device time rather than the host's launch rate; without a capture (or
    if it fails) the calls are timed as launched."""

    def __init__(self, torch):
        self.torch = torch

    def __call__(self, fn, reps, warmup=3, graph=False):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        run, iters = fn, reps
        if graph:
            try:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for _ in range(reps):
                        fn()
                g.replay()
                torch.cuda.synchronize()
                run, iters = g.replay, 1
            except Exception as e:  # not capturable: time the launches
                log("graph capture failed, timing launches:", e)
                torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            run()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps  # ms


def matvec_bytes(n, k, dtype=Q7B32, residual=False, f32_input=False):
    """Algorithmic bytes of one matrix-vector product: codes + weight scales + activations + outputs."""
    codes = n * k // (2 if dtype == Q4B32 else 1)
    scales = n * k // 32 * 4
    act = k * 4 if f32_input else k + k // 32 * 8
    out = n * 4 * (2 if residual else 1)
    return codes + scales + act + out


def build_decoder(fk, torch, np, exact, seed=0, dtype=Q7B32):
    shape = fk.Shape()
    rng = np.random.default_rng(seed)
    H, F, V = shape.hidden, shape.ffn, shape.vocab
    dims = {"qkv": (shape.qkv(), H), "o": (H, shape.width()), "gate": (F, H), "up": (F, H), "down": (H, F)}
    layers = []
    for _ in range(shape.layers):
        d = {k: fk.Table(fk.Tensor(dtype, list(v), synthetic_table(np, dtype, v[0], v[1], rng))) for k, v in dims.items()}
        d["norm1"] = torch.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)).cuda()
        d["norm2"] = torch.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)).cuda()
        d["qkv_bias"] = torch.from_numpy((0.1 * rng.standard_normal(shape.qkv())).astype(np.float32)).cuda()
        layers.append(d)
    table_bytes = synthetic_table(np, dtype, V, H, rng)
    head = fk.Table(fk.Tensor(dtype, [V, H], table_bytes))
    final = torch.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)).cuda()
    cache_shape = (shape.layers, shape.kv_heads, shape.capacity, shape.head_dim)
    kc = torch.from_numpy(rng.standard_normal(cache_shape).astype(np.float32)).cuda()
    vc = torch.from_numpy(rng.standard_normal(cache_shape).astype(np.float32)).cuda()
    model = fk.Qwen2(shape, dtype, layers, final, head, kc, vc, exact=exact)
    host = {"layers": layers, "head": head, "final": final, "table_bytes": table_bytes, "kc": kc, "vc": vc}
    return shape, model, host


def decode_step_bytes(shape, position, dtype=Q7B32):
    """Algorithmic bytes of one decode step (weights, KV read, activations)."""
    H, F, D = shape.hidden, shape.ffn, shape.head_dim
    per_layer = (matvec_bytes(shape.qkv(), H, dtype) + shape.qkv() * 4 + matvec_bytes(H, shape.width(), dtype, residual=True)
                 + 2 * matvec_bytes(F, H, dtype) + matvec_bytes(H, F, dtype, residual=True))
    kv = 2 * (position + 1) * shape.kv_heads * D * 4
    return shape.layers * (per_layer + kv) + matvec_bytes(shape.vocab, H, dtype)


def time_prefill(fk, torch, np, model, shape, rows, chunk, reps=10):
    """Reader::read of `rows` token rows from position 0 (embedding included), as one HIP graph."""
    ids = torch.from_numpy(np.random.default_rng(7).integers(0, shape.vocab, rows).astype(np.int32)).cuda()
    emb = torch.empty((rows, shape.hidden), dtype=torch.float32, device="cuda")
    nxt = torch.zeros(1, dtype=torch.int32, device="cuda")

    def read():
        model.embed(ids, out=emb)
        model.read(emb, 0, chunk, next_token=nxt)
    ms = Timer(torch)(read, reps, warmup=2, graph=True)
    return {"rows": rows, "chunk": chunk, "ms": round(ms, 4), "rows_per_s": round(rows / ms * 1e3, 1)}


def cpu_prefill_baseline(np, shape, host, rows):
    """The oracle's Reader::read of `rows` rows from position 0 (the reference's scalar path, its
    products column-split over a team of threads), one warm-up then the mean of two reads."""
    from oracle import oracle as O
    layers = []
    for d in host["layers"]:
        layers.append({k: d[k].reference_bytes() for k in ("qkv", "o", "gate", "up", "down")}
                      | {k: d[k].cpu().numpy() for k in ("norm1", "norm2", "qkv_bias")})
    sh = O.Qwen2Shape(hidden=shape.hidden, layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                      head_dim=shape.head_dim, ffn=shape.ffn, vocab=shape.vocab, capacity=shape.capacity,
                      rope_base=shape.rope_base, eps=shape.eps, dtype=O.Q7B32)
    model = O.Qwen2(sh, layers, host["final"].cpu().numpy(), host["table_bytes"])
    kc, vc = host["kc"].cpu().numpy(), host["vc"].cpu().numpy()
    emb = model.embed(np.random.default_rng(7).integers(0, shape.vocab, rows).astype(np.int32))
    default, _ = cpu_thread_counts()
    cpu_model, nproc, _ = host_cpu()
    call = lambda: model.read(kc, vc, emb, 0, rows, threads=default)  # noqa: E731
    call()
    t0 = time.perf_counter()
    for _ in range(2):
        call()
    ms = (time.perf_counter() - t0) * 1e3 / 2
    return {"value": round(rows / ms * 1e3, 2), "unit": "rows/s", "ms": round(ms, 1), "cores": default, "kind": "port",
            "cpu": cpu_model, "nproc": nproc,
            "sample": f"a {rows}-row read from position 0 with the last row's logits, one warm-up then the mean of two"}


def time_decode(fk, torch, model, position, steps, warmup):
    nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
    token = 1234
    model.step(token, position, next_token=nxt)  # eager once: validates the launch sequence
    torch.cuda.synchronize()
    graph = None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            model.step(token, position, next_token=nxt)
        torch.cuda.synchronize()
        run = graph.replay
    except Exception as e:  # capture not available: time eager launches
        log("graph capture failed, timing eager launches:", e)
        graph = None
        run = lambda: model.step(token, position, next_token=nxt)  # noqa: E731
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return ms, graph is not None, int(nxt.item())


def time_matvecs(fk, torch, np, shape, host):
    """The decode step's 121 projections replayed alone, in the step's order over the distinct
    layer tables (about 555 MB per pass, past the 256 MiB Infinity Cache), captured in one graph
    and timed with events. Returns (bytes per pass, ms per pass, launches, per-projection detail);
    the detail times each projection over the 24 layers' tables back to back."""
    H, F = shape.hidden, shape.ffn
    timer = Timer(torch)
    rng = np.random.default_rng(5)
    inputs = {}
    for k in {H, shape.width(), F}:
        q = torch.from_numpy(rng.integers(-127, 128, k, dtype=np.int16).astype(np.int8)).cuda()
        s = torch.from_numpy(rng.uniform(0.001, 0.05, k // 32).astype(np.float32)).cuda()
        c = torch.zeros(k // 32, dtype=torch.int32, device="cuda")
        inputs[k] = fk.Input(quant=fk.Quantized(fk.QuantFormat.Q7b32, q, s, c))
    out = torch.zeros(((max(shape.vocab, F) + 3) // 4 * 4,), dtype=torch.float32, device="cuda")
    order = [("qkv", False), ("o", True), ("gate", False), ("up", False), ("down", True)]
    launches = []
    for ly in host["layers"]:
        for name, residual in order:
            launches.append((name, ly[name].matrix(), residual))
    launches.append(("head", host["head"].matrix(), False))

    def launch(m, residual):
        n = (m.rows + 3) // 4 * 4
        fk.matmul(m, inputs[m.cols], range(0, n), out=out[:n].view(1, n), accumulate=residual)

    def sequence():
        for _, m, residual in launches:
            launch(m, residual)

    total_bytes = sum(matvec_bytes(m.rows, m.cols, residual=r) for _, m, r in launches)
    sequence()
    torch.cuda.synchronize()
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            sequence()
        run = graph.replay
    except Exception as e:
        log("matvec graph capture failed, timing eager launches:", e)
        run = sequence
    total_ms = timer(run, 20)
    detail = {}
    for name, residual in order + [("head", False)]:
        mats = [m for nm, m, _ in launches if nm == name]
        ms = timer(lambda: [launch(m, residual) for m in mats], 10, graph=True) / len(mats)
        b = matvec_bytes(mats[0].rows, mats[0].cols, residual=residual)
        detail[name] = {"n": mats[0].rows, "k": mats[0].cols, "us": round(ms * 1e3, 3), "GB_s": round(b / ms / 1e6, 1)}
    return total_bytes, total_ms, len(launches), detail


def cpu_baseline(np, shape, host, budget_s=10.0):
    """The oracle's decode step on this host (a C restatement of the reference's scalar x86-64
    path, its products column-split over a team of threads like the reference's): at the
    reference CLI's default team, min(8, cores - 2) threads, one warm-up step then the mean over
    as many steps as fit in about `budget_s` seconds (crates/harness/src/bench.rs:8-17), and the
    steady-state best of five runs (tools/kernel-harness/bench.mjs:29-40); the same on every core."""
    from oracle import oracle as O
    layers = []
    for d in host["layers"]:
        layers.append({k: d[k].reference_bytes() for k in ("qkv", "o", "gate", "up", "down")}
                      | {k: d[k].cpu().numpy() for k in ("norm1", "norm2", "qkv_bias")})
    sh = O.Qwen2Shape(hidden=shape.hidden, layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                      head_dim=shape.head_dim, ffn=shape.ffn, vocab=shape.vocab, capacity=shape.capacity,
                      rope_base=shape.rope_base, eps=shape.eps, dtype=O.Q7B32)
    model = O.Qwen2(sh, layers, host["final"].cpu().numpy(), host["table_bytes"])
    kc, vc = host["kc"].cpu().numpy(), host["vc"].cpu().numpy()
    default, every = cpu_thread_counts()
    cpu_model, nproc, _ = host_cpu()

    def measure(threads, budget):
        step = lambda: model.step(kc, vc, 1234, 511, threads=threads)  # noqa: E731
        step()  # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            step()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget or n >= 200:
                break
        iters = 1
        while True:
            t1 = time.perf_counter()
            for _ in range(iters):
                step()
            if time.perf_counter() - t1 >= 0.08:
                break
            iters *= 2
        best = min(timed(step, iters) for _ in range(5)) / iters
        return n, el, {"value": round(n / el, 3), "mean_ms_per_step": round(el * 1e3 / n, 3),
                       "best_of_5_ms_per_step": round(best * 1e3, 3)}

    n, el, line = measure(default, budget_s)
    _, _, every_line = measure(every, budget_s / 2)
    line.update({"unit": "tokens/s", "cores": default, "kind": "port", "cpu": cpu_model, "nproc": nproc,
                 "sample": f"{n} decode steps at position 511 (the full 24-layer step with logits) after one warm-up, "
                           f"{default} threads, {el:.1f} s; value = the mean; C restatement of the reference scalar path",
                 "all_cores": dict(every_line, cores=every)})
    return line


def timed(call, iters):
    t0 = time.perf_counter()
    for _ in range(iters):
        call()
    return time.perf_counter() - t0


def gemm_bound(rows, k, n, ms, fused=False):
    """The attainable time of a batched product: the largest of its int8 MFMA time at the peak, its
    HBM time (Q8b32 codes and scales, f32 rows in, f32 outputs) and its issue floor (the measured
    cycles per 32 x 32 tile and block of the exact or fused rescale with its MFMAs, over every SIMD)."""
    groups = k // 32
    t_mfma = 2.0 * rows * n * k / (INT8_PEAK_TOPS * 1e12)
    t_hbm = (n * k + n * groups * 4 + rows * k * 4 + rows * n * 4) / (HBM_PEAK_GBS * 1e9)
    tile_blocks = ((rows + 31) // 32) * ((n + 31) // 32) * groups
    t_issue = tile_blocks * (ISSUE_CYCLES_FUSED if fused else ISSUE_CYCLES_EXACT) / (SIMDS * CLOCK_HZ)
    attainable = max(t_mfma, t_hbm, t_issue)
    return {"t_mfma_us": round(t_mfma * 1e6, 2), "t_hbm_us": round(t_hbm * 1e6, 2), "t_issue_us": round(t_issue * 1e6, 2),
            "by": ("issue" if attainable == t_issue else "hbm" if attainable == t_hbm else "mfma"),
            "ceiling_frac_int8_peak": round(t_mfma / attainable, 4),
            "frac_attainable": round(attainable * 1e3 / ms, 4)}


def noalloc_product(fk, table, inp, rows, n, out):
    """fg_matmul_noalloc (its scratch a fixed per-device array) over an fk.Input."""
    import ctypes
    from fusor_kernels import _lib
    fi = inp.ffi()
    _lib.check(_lib.lib().fg_matmul_noalloc(table.handle, ctypes.byref(fi), rows, 0, n, None, _lib.ptr(out),
                                            out.stride(0), 0, _lib.stream_handle()))


def extras(fk, torch, np, with_cpu=True):
    """The other workloads: single matvec (resident, streamed over 64 launches, and in one launch
    over all 64 copies), GEMMs, packed int4, int8 attention; each product with its CPU baseline."""
    timer = Timer(torch)
    rng = np.random.default_rng(0)
    res = {}
    # 1. 4864 x 896 Q8b32 (levels in [-127, 127]) and Q7b32, activation f32 quantized in-kernel
    for dtype, name in ((Q8B32, "Q8b32"), (Q7B32, "Q7b32")):
        n, k = 4864, 896
        data = synthetic_table(np, dtype, n, k, rng)
        t = fk.Table(fk.Tensor(dtype, [n, k], data))
        xh = rng.standard_normal(k).astype(np.float32)
        x = torch.from_numpy(xh).cuda()
        out = torch.empty((1, n), dtype=torch.float32, device="cuda")
        m = t.matrix()
        inp_x = fk.Input(f32=x)
        ms = timer(lambda: fk.matmul(m, inp_x, range(0, n), out=out), 200, graph=True)
        b = matvec_bytes(n, k, dtype, f32_input=True)
        entry = {"resident_us": round(ms * 1e3, 3), "resident_GB_s": round(b / ms / 1e6, 1), "bytes": b}
        if dtype == Q8B32:
            # streamed: 64 distinct copies (> 256 MiB Infinity Cache) read in turn, one launch each
            copies = [fk.Table.from_device_bytes(dtype, n, k, torch.from_numpy(data).cuda()) for _ in range(64)]
            mats = [c.matrix() for c in copies]

            def sweep():
                for mm in mats:
                    fk.matmul(mm, inp_x, range(0, n), out=out)
            ms = timer(sweep, 5, graph=True) / len(mats)
            entry.update({"streamed_us": round(ms * 1e3, 3), "streamed_GB_s": round(b / ms / 1e6, 1),
                          "streamed_bytes": 64 * len(data)})
            del copies, mats
            # sustained: the 64 copies' rows as one 311296 x 896 table (314 MB, past the 256 MiB
            # Infinity Cache), streamed by one launch
            big_rows = 64 * n
            big = fk.Table(fk.Tensor(dtype, [big_rows, k], synthetic_table(np, dtype, big_rows, k, rng)))
            big_out = torch.empty((1, big_rows), dtype=torch.float32, device="cuda")
            bm = big.matrix()
            ms = timer(lambda: fk.matmul(bm, inp_x, range(0, big_rows), out=big_out), 20, graph=True)
            bb = matvec_bytes(big_rows, k, dtype, f32_input=True)
            entry.update({"one_launch_311296x896_us": round(ms * 1e3, 3), "one_launch_GB_s": round(bb / ms / 1e6, 1),
                          "one_launch_frac_hbm": round(bb / ms / 1e6 / HBM_PEAK_GBS, 4), "one_launch_bytes": bb})
            del big, bm, big_out
        if with_cpu:
            entry["cpu_baseline"] = cpu_product_baseline(
                np, dtype, n, k, data, xh.reshape(1, k), lambda ms_: b / ms_ / 1e6, "GB/s",
                "the whole 4864 x 896 product, f32 row quantized first")
        res[f"matvec_4864x896_{name}"] = entry
    # 2. GEMMs (Q8b32 weights); the CPU baseline on a sample of rows for the 4096-row shapes
    for label, (rows, k, n, outl, sigma, cpu_rows) in {
            "gemm_512x896x9728": (512, 896, 9728, 0.0, 1.0, 512),
            "gemm_512x4864x896": (512, 4864, 896, 0.0, 1.0, 512),
            "dit_qkv_4096x1152x3456": (4096, 1152, 3456, 0.01, 2.0 ** 0.5, 256),
            "dit_up_4096x1152x4608": (4096, 1152, 4608, 0.01, 2.0 ** 0.5, 256),
            "dit_down_4096x4608x1152": (4096, 4608, 1152, 0.01, 2.0 ** 0.5, 256)}.items():
        data = synthetic_table(np, Q8B32, n, k, rng)
        t = fk.Table(fk.Tensor(Q8B32, [n, k], data))
        xh = (rng.standard_normal((rows, k)) * sigma).astype(np.float32)
        if outl:
            xh[rng.random((rows, k)) < outl] *= 20
        x = torch.from_numpy(xh).cuda()
        m = t.matrix()
        out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        ms_f32 = timer(lambda: fk.matmul(m, fk.Input(f32=x.view(-1)), range(0, n), out=out), 10, graph=True)
        # the same through fg_matmul_noalloc: no per-call workspace (in a graph, fg_matmul's
        # stream-ordered allocation and free are two memory nodes per product)
        inp_x = fk.Input(f32=x.view(-1))
        ms_f32_na = timer(lambda: noalloc_product(fk, t, inp_x, rows, n, out), 10, graph=True)
        qr = fk.QuantizedRows()
        inp = qr.input(m, x.view(-1))
        ms_q = timer(lambda: fk.matmul(m, inp, range(0, n), out=out), 10, graph=True)
        ms_q_na = timer(lambda: noalloc_product(fk, t, inp, rows, n, out), 10, graph=True)
        ms_best = min(ms_q, ms_q_na)
        # the NEON backend's arithmetic (one fused multiply-add per group scaling), its own bits
        ms_fused = timer(lambda: fk.matmul(m, inp, range(0, n), out=out, fused=True), 10, graph=True)
        # the NEON backend's arithmetic from the f32 rows
        ms_fused_f32 = timer(lambda: fk.matmul(m, inp_x, range(0, n), out=out, fused=True), 10, graph=True)
        ops = 2.0 * rows * n * k
        # the headline figure is the configs' own workload: f32 rows, quantized on the way
        entry = {"us": round(ms_f32 * 1e3, 2), "TOPS": round(ops / ms_f32 / 1e9, 1),
                 "frac_int8_peak": round(ops / ms_f32 / 1e9 / INT8_PEAK_TOPS, 4),
                 "TOPS_from": "fg_matmul from f32 rows (quantization included), one HIP graph",
                 "noalloc_us": round(ms_f32_na * 1e3, 2),
                 "prequantized_us": round(ms_q * 1e3, 2), "noalloc_prequantized_us": round(ms_q_na * 1e3, 2),
                 "prequantized_TOPS": round(ops / ms_best / 1e9, 1),
                 "f32_rows_over_prequantized": round(ms_f32 / ms_best, 3),
                 "fused_scale_us": round(ms_fused_f32 * 1e3, 2), "fused_scale_TOPS": round(ops / ms_fused_f32 / 1e9, 1),
                 "fused_scale_frac_int8_peak": round(ops / ms_fused_f32 / 1e9 / INT8_PEAK_TOPS, 4),
                 "fused_scale_prequantized_us": round(ms_fused * 1e3, 2)}
        entry["bound"] = gemm_bound(rows, k, n, ms_f32)
        entry["fused_bound"] = gemm_bound(rows, k, n, ms_fused_f32, fused=True)
        if with_cpu:
            cpu_ops = 2.0 * cpu_rows * n * k
            entry["cpu_baseline"] = cpu_product_baseline(
                np, Q8B32, n, k, data, xh[:cpu_rows], lambda ms_: cpu_ops / ms_ / 1e9, "TOPS",
                f"the first {cpu_rows} of {rows} rows (rows are independent), f32 rows quantized first")
        res[label] = entry
    # 3. packed int4 14336 x 4096, rows 1 and 16: resident (one table, replayed from the 256 MiB
    #    Infinity Cache) and streamed (distinct copies read in turn, more bytes than that cache holds)
    n, k = 14336, 4096
    data = synthetic_table(np, Q4B32, n, k, rng)
    t = fk.Table(fk.Tensor(Q4B32, [n, k], data))
    m = t.matrix()
    copies = [fk.Table.from_device_bytes(Q4B32, n, k, torch.from_numpy(data).cuda()) for _ in range(9)]
    cmats = [c.matrix() for c in copies]
    for rows in (1, 16):
        xh = rng.standard_normal((rows, k)).astype(np.float32)
        x = torch.from_numpy(xh).cuda()
        inp = fk.QuantizedRows().input(m, x.view(-1))
        out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        ms = timer(lambda: fk.matmul(m, inp, range(0, n), out=out), 50, graph=True)
        b = n * k // 2 + n * k // 32 * 4 + rows * (k + k // 32 * 8) + rows * n * 4
        ms_s = timer(lambda: [fk.matmul(cm, inp, range(0, n), out=out) for cm in cmats], 5, graph=True) / len(cmats)
        entry = {"us": round(ms * 1e3, 2), "GB_s": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 4),
                 "bytes": b, "resident": "one table replayed (it fits the 256 MiB Infinity Cache)",
                 "streamed_us": round(ms_s * 1e3, 2), "streamed_GB_s": round(b / ms_s / 1e6, 1),
                 "streamed_frac_hbm": round(b / ms_s / 1e6 / HBM_PEAK_GBS, 4),
                 "streamed": f"{len(cmats)} distinct copies ({len(cmats) * len(data) / 1e6:.0f} MB) read in turn"}
        if with_cpu:
            entry["cpu_baseline"] = cpu_product_baseline(np, Q4B32, n, k, data, xh, lambda ms_: b / ms_ / 1e6, "GB/s",
                                                         f"the whole product, {rows} f32 row(s) quantized first")
        res[f"int4_14336x4096_rows{rows}"] = entry
    del copies, cmats
    # 3b. ternary T2b128 14336 x 4096 (2 bits a weight, a scale per 128), rows 1 and 16, resident and
    #     streamed
    data = synthetic_table(np, T2B128, n, k, rng)
    t = fk.Table(fk.Tensor(T2B128, [n, k], data))
    m = t.matrix()
    copies = [fk.Table.from_device_bytes(T2B128, n, k, torch.from_numpy(data).cuda()) for _ in range(20)]
    cmats = [c.matrix() for c in copies]
    for rows in (1, 16):
        xh = rng.standard_normal((rows, k)).astype(np.float32)
        x = torch.from_numpy(xh).cuda()
        inp = fk.QuantizedRows().input(m, x.view(-1))
        out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        ms = timer(lambda: fk.matmul(m, inp, range(0, n), out=out), 50, graph=True)
        b = n * k // 4 + n * k // 128 * 4 + rows * (k + k // 128 * 8) + rows * n * 4
        ms_s = timer(lambda: [fk.matmul(cm, inp, range(0, n), out=out) for cm in cmats], 5, graph=True) / len(cmats)
        entry = {"us": round(ms * 1e3, 2), "GB_s": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 4),
                 "bytes": b, "resident": "one table replayed (it fits the 256 MiB Infinity Cache)",
                 "streamed_us": round(ms_s * 1e3, 2), "streamed_GB_s": round(b / ms_s / 1e6, 1),
                 "streamed_frac_hbm": round(b / ms_s / 1e6 / HBM_PEAK_GBS, 4),
                 "streamed": f"{len(cmats)} distinct copies ({len(cmats) * len(data) / 1e6:.0f} MB) read in turn"}
        if with_cpu:
            entry["cpu_baseline"] = cpu_product_baseline(np, T2B128, n, k, data, xh, lambda ms_: b / ms_ / 1e6, "GB/s",
                                                         f"the whole product, {rows} f32 row(s) quantized first")
        res[f"t2_14336x4096_rows{rows}"] = entry
    del copies, cmats
    # 3c. the same T2b128 table times 512 rows (prefill-sized: the matrix cores)
    rows, cpu_rows = 512, 16
    xh = rng.standard_normal((rows, k)).astype(np.float32)
    x = torch.from_numpy(xh).cuda()
    inp = fk.QuantizedRows().input(m, x.view(-1))
    out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    ms = timer(lambda: fk.matmul(m, inp, range(0, n), out=out), 20, graph=True)
    ops = 2.0 * rows * n * k
    entry = {"us": round(ms * 1e3, 2), "TOPS": round(ops / ms / 1e9, 1), "frac_int8_peak": round(ops / ms / 1e9 / INT8_PEAK_TOPS, 4)}
    if with_cpu:
        cpu_ops = 2.0 * cpu_rows * n * k
        entry["cpu_baseline"] = cpu_product_baseline(
            np, T2B128, n, k, data, xh[:cpu_rows], lambda ms_: cpu_ops / ms_ / 1e9, "TOPS",
            f"the first {cpu_rows} of {rows} rows (rows are independent), f32 rows quantized first")
    res["t2_512x4096x14336"] = entry
    # 4. int8 attention (attention::attend) at the DiT block's shape: 4096 tokens, 16 heads of 72
    #    read by stride and offset from one fused qkv row, exp_fast
    tokens, heads, hd = 4096, 16, 72
    row = 3 * heads * hd
    qkv = torch.from_numpy(rng.standard_normal((tokens, row)).astype(np.float32)).cuda()
    out = torch.empty((tokens, heads * hd), dtype=torch.float32, device="cuda")
    call = fk.Call(heads, heads, hd, 1, tokens, tokens, fk.Operand(qkv, row, 0), fk.Operand(qkv, row, heads * hd),
                   fk.Operand(qkv, row, 2 * heads * hd), fk.Exponentials.FAST)
    ms = timer(lambda: fk.attend(call, out), 3, warmup=1)
    padded_hd = (hd + 31) // 32 * 32
    ops = 2.0 * heads * tokens * tokens * (padded_hd + hd)  # Q·K over the padded head, P·V
    res["int8_attention_dit_4096x16x72"] = {"ms": round(ms, 3), "int8_TOPS": round(ops / ms / 1e9, 1)}
    del qkv, out
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--exact", action="store_true", help="time the exact-order decoder as the headline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true", help="skip the extra workloads")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run 5 device-to-device copies of this many MiB (the known-size kernel that scales "
                         "the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (--gpus 1 only)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import fusor_kernels as fk
    fk.lib()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    position = 511
    log("building the decoder (synthetic Q7b32 weights)...")
    shape, model, host = build_decoder(fk, torch, np, exact=args.exact)
    ms, graphed, token = time_decode(fk, torch, model, position, args.steps, args.warmup)
    tok_s = 1000.0 / ms
    step_bytes = decode_step_bytes(shape, position)
    log(f"decode: {ms * 1e3:.1f} us/token, {tok_s:.0f} tokens/s, graph={graphed}")
    mv_bytes, mv_ms, mv_launches, mv_detail = time_matvecs(fk, torch, np, shape, host)
    achieved = mv_bytes / mv_ms / 1e6  # GB/s
    log(f"matvec: {mv_launches} launches, {mv_ms * 1e3:.1f} us, {achieved:.0f} GB/s")
    other = {}
    if not args.exact:
        # the same tables and caches, reductions in the reference's order
        ex_model = fk.Qwen2(shape, Q7B32, host["layers"], host["final"], host["head"], host["kc"], host["vc"], exact=True)
        ms_x, _, _ = time_decode(fk, torch, ex_model, position, max(20, args.steps // 4), 5)
        other["exact_order_decode"] = {"ms_per_step": round(ms_x, 4), "tokens_per_s": round(1000.0 / ms_x, 1)}
        # prefill (Reader::read) of 158 rows, the reference's prefill length, in one chunk: the
        # parallel-order model and the exact one (bit-identical to one decode step per row)
        other["prefill_158_rows"] = time_prefill(fk, torch, np, model, shape, 158, 158)
        other["prefill_158_rows"]["exact_order"] = time_prefill(fk, torch, np, ex_model, shape, 158, 158)
        if not args.no_cpu:
            other["prefill_158_rows"]["cpu_baseline"] = cpu_prefill_baseline(np, shape, host, 32)
        del ex_model
        # the same step with Q4b32 tables (the reference's LM layers run Q4b32), parallel order
        _, q4_model, q4_host = build_decoder(fk, torch, np, exact=False, seed=1, dtype=Q4B32)
        ms_4, _, _ = time_decode(fk, torch, q4_model, position, max(20, args.steps // 4), 5)
        b4 = decode_step_bytes(shape, position, Q4B32)
        other["q4b32_decode"] = {"ms_per_step": round(ms_4, 4), "tokens_per_s": round(1000.0 / ms_4, 1),
                                 "step_bytes": b4, "step_GB_s": round(b4 / ms_4 / 1e6, 1)}
        del q4_model, q4_host
    if not args.no_extras:
        log("extra workloads...")
        other.update(extras(fk, torch, np, with_cpu=not args.no_cpu))
    cpu = None
    if not args.no_cpu:
        log("cpu baseline...")
        cpu = cpu_baseline(np, shape, host)
    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random Q7b32 weights, N(0,1) KV cache)",
        "config": {"workload": "Qwen2-0.5B-shape decode step at position 511: hidden 896, 24 layers, 14/2 heads x 64, "
                               "FFN 4864 SwiGLU, tied 151936 x 896 Q7b32 table, 511-entry f32 KV cache",
                   "weights": "Q7b32", "position": position, "graph": graphed,
                   "reductions": "exact order" if args.exact else "parallel",
                   "step_bytes": step_bytes, "step_GB_s": round(step_bytes / ms / 1e6, 1),
                   "greedy_token": token},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "proj_kernel through fg_matmul (the decode step's 121 projections)",
                     "bytes_per_launch": round(mv_bytes / mv_launches), "us_per_launch": round(mv_ms * 1e3 / mv_launches, 3),
                     "by_shape": mv_detail},
        "cpu_baseline": cpu,
    }
    line.update(other)
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["copy_calibration_bytes"] = src.numel() * 4
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
