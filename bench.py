"""Benchmark of the MI355X embedding lookup path (one JSON line on stdout).

Default workload (BASELINE.json's metric, C2-pool): GPUEmbeddingLayer over a
50,000,000 x 128 fp16 table in HBM (values N(0, 0.02)), 262,144 int64 keys per
batch drawn Zipf(alpha=1.05) over the rows with a seeded permutation (the
reference's generator, samples/pytorch/pytorch_samples_common.py:21-47),
fused find-and-pool with Fixed hotness 1024 x 256 bags, Sum, fp16 output,
through the C ABI entry nve_layer_lookup_pooled.  A step is one lookup of one
batch; batches are generated up front and stay resident in HBM.

Reported beside the throughput:
  roofline      algorithmic bytes per launch / the kernel's mean duration
                (HIP events on the lookup stream) against the 8 TB/s HBM peak,
                and the HBM bytes rocprofv3 counts per launch over the same
                time (frac_dram); beside it a plain row-read kernel's rate on
                the same keys and on uniform keys, for comparison;
  host_call_us  host time per call of the module, the torch op and the C ABI;
  cpu_baseline  the product's CPU HostLayer (threaded gather + fp32 pooling,
                restating the reference's) timed on this host's cores on
                whole batches of the same workload, median with p10 / p90,
                at the reference's default worker count and at all cores.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "nv-embedding-cache_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "embedding lookups/sec + achieved HBM GB/s (% peak), fused find-and-pool, 1 GPU"
HBM_PEAK_GBPS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def power_law_keys(torch, n, rows, alpha, gen, perm):
    """translateToPowerLaw(1, rows, alpha, x) then perm[y] (pytorch_samples_common.py:21-47)."""
    x = torch.rand(n, device="cuda", dtype=torch.float64, generator=gen)
    gamma = torch.tensor([1.0 - alpha], device="cuda")  # float32, as the reference
    lo = torch.pow(torch.tensor(1.0, device="cuda"), gamma)
    hi = torch.pow(torch.tensor(float(rows), device="cuda"), gamma)
    y = torch.pow(x * (hi - lo) + lo, 1.0 / gamma)
    y[y >= rows] = rows - 1
    return perm[y.to(torch.int64)]


def cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return model, avail


class HostLayerBaseline:
    """The product's CPU HostLayer (LinearHostTable + HostEmbeddingLayer of
    libnve_amd.so, a restatement of the reference's host_embedding_layer.cpp:
    55-247 -> cpu_gather.hpp:28-80 -> cpu_pooling.hpp:68-150) over a host copy
    of a table, on `threads` worker threads of its own pool."""

    def __init__(self, lib, h_table, rows, row_bytes, dtype, threads):
        L = lib.load()
        self.lib, self.h_table = lib, h_table
        self.pool, self.t, self.layer, self.ctx = (ctypes.c_void_p() for _ in range(4))
        lib.call("nve_thread_pool_create", ctypes.byref(self.pool), f'{{"num_workers": {threads}}}'.encode())
        tc = L.nve_host_table_config_default()
        tc.key_size, tc.max_value_size, tc.value_dtype = 8, row_bytes, dtype
        lib.call("nve_amd_linear_host_table_create", ctypes.byref(self.t), lib.KEY_INT64, ctypes.byref(tc),
                 ctypes.c_void_p(h_table.ctypes.data), rows, 0)
        lc = L.nve_host_embedding_layer_config_default()
        lib.call("nve_host_embedding_layer_create", ctypes.byref(self.layer), lib.KEY_INT64, ctypes.byref(lc),
                 self.t, None)
        lib.call("nve_layer_create_execution_context", self.layer, ctypes.byref(self.ctx), None, None,
                 self.pool, None)

    def pooled(self, keys, out, out_stride, hot, out_dtype):
        self.lib.check(self.lib.load().nve_layer_lookup_pooled(
            self.layer, self.ctx, keys.size, ctypes.c_void_p(keys.ctypes.data), ctypes.c_void_p(out.ctypes.data),
            out_stride, None, self.lib.POOL_SUM, self.lib.SPARSE_FIXED, None, 0, hot, None, 0, out_dtype, None))

    def gather(self, keys, out, out_stride):
        self.lib.check(self.lib.load().nve_layer_lookup(
            self.layer, self.ctx, keys.size, ctypes.c_void_p(keys.ctypes.data), ctypes.c_void_p(out.ctypes.data),
            out_stride, None, None))

    def close(self):
        self.lib.call("nve_context_destroy", self.ctx)
        self.lib.call("nve_layer_destroy", self.layer)
        self.lib.call("nve_table_destroy", self.t)
        self.lib.call("nve_thread_pool_destroy", self.pool)


def time_batches(run, batches, seconds, min_batches=20):
    """3 untimed batches, then batches until `seconds` have passed and at least
    `min_batches` ran; per-batch wall times (s), sorted."""
    for i in range(3):
        run(batches[i % len(batches)])
    times, t0 = [], time.perf_counter()
    while len(times) < min_batches or time.perf_counter() - t0 < seconds:
        b = batches[len(times) % len(batches)]
        t1 = time.perf_counter()
        run(b)
        times.append(time.perf_counter() - t1)
    return sorted(times)


def quantiles(ts):
    n = len(ts)
    return ts[n // 2], ts[max(0, int(0.1 * n))], ts[min(n - 1, int(0.9 * n))]


def cpu_baseline(lib, h_table, rows, row_bytes, dtype, key_batches, run_batch, seconds, what, check):
    """The product HostLayer timed on this host's cores on whole batches of the
    workload: the reference's default worker count max(cores - 2, 1)
    (thread_pool.cpp:112-116) for `value`, and every core beside it; median
    batch time with p10 / p90 (at least 20 batches after 3 warm-up ones).
    After each timing, untimed, one more batch (the first) is run and
    `check()` compares its output with the CPU oracle's restatement of the
    reference HostLayer (bit for bit) or raises."""
    model, avail = cpu_info()
    n = key_batches[0].size
    res = {}
    for label, threads in (("default", max(avail - 2, 1)), ("all_cores", avail)):
        base = HostLayerBaseline(lib, h_table, rows, row_bytes, dtype, threads)
        try:
            ts = time_batches(lambda k: run_batch(base, k), key_batches, seconds)
            run_batch(base, key_batches[0])
            checked = check()
        finally:
            base.close()
        med, p10, p90 = quantiles(ts)
        res[label] = {"threads": threads, "batches": len(ts), "median_ms": round(med * 1e3, 3),
                      "p10_ms": round(p10 * 1e3, 3), "p90_ms": round(p90 * 1e3, 3),
                      "lookups_per_s": round(n / med, 1), "checked": checked}
        log(f"cpu baseline ({label}, {threads} threads): median {med * 1e3:.2f} ms per {n}-key batch "
            f"(p10 {p10 * 1e3:.2f}, p90 {p90 * 1e3:.2f}) = {n / med / 1e6:.1f} M lookups/s")
    d = res["default"]
    return {"value": d["lookups_per_s"], "unit": "lookups/s", "cores": d["threads"], "kind": "port",
            "sample": f"{d['batches']} whole batches of {n} keys ({what}), median batch time, on '{model}' "
                      f"({avail} cores available): the product HostLayer (libnve_amd.so, CPU threads)",
            "median_ms": d["median_ms"], "p10_ms": d["p10_ms"], "p90_ms": d["p90_ms"],
            "checked": d["checked"], "all_cores": res["all_cores"]}


def host_pool_check(h_table, row_bytes, dtype, keys, out, bags, hot):
    """A check for cpu_baseline: `out` (the HostLayer's Fixed-hotness Sum of
    `keys`) equals the oracle's reference HostLayer order (cpu_pooling.hpp:
    68-150) bit for bit.  The oracle is the checker here, not the thing timed."""
    import numpy as np
    from oracle import oracle as O
    from pynve import _lib

    odt = O.F16 if out.dtype == np.float16 else O.F32
    rdt = O.F16 if dtype == _lib.DT_F16 else O.F32
    count = out.shape[1]

    def check():
        ref = O.pool(O.linear_row_ptrs(keys, h_table, row_bytes), rdt, count, O.FIXED, O.SUM, keys.size, None,
                     bags, hot, None, 0, odt, host_order=True)
        if not np.array_equal(out.view(ref.dtype), ref):
            raise SystemExit("bench.py: the CPU HostLayer's output differs from the oracle's reference order")
        return f"all {bags} bags of the first batch bit-exact with the oracle's HostLayer order"
    return check


def read_ceiling(torch, lib, stream, counts):
    """Plain row-read kernel on uniform random 256-byte rows of a 16 GiB buffer
    (far beyond the 256 MB MALL), reading and folding the rows and nothing else.
    Returns {rows_per_launch: (GB/s, us per launch)}."""
    row_bytes = 256
    rows = (16 << 30) // row_bytes
    buf = torch.empty(rows * row_bytes // 2, dtype=torch.int16, device="cuda")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    s = ctypes.c_void_p(stream.cuda_stream)
    res = {}
    for n in counts:
        idx = torch.randint(0, rows, (n,), device="cuda", generator=gen, dtype=torch.int64)
        sink = torch.zeros((n + 127) // 128, dtype=torch.int32, device="cuda")

        fn = lib.load().nve_amd_read_ceiling  # resolved once: the issue loop stays below the kernel time
        args = (ctypes.c_void_p(buf.data_ptr()), row_bytes, ctypes.c_void_p(idx.data_ptr()), n,
                ctypes.c_void_p(sink.data_ptr()), s)

        def launch():
            st = fn(*args)
            if st:
                lib.check(st)

        for _ in range(5):
            launch()
        reps = 100
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        res[n] = ((n * row_bytes + n * 8) / (ms * 1e-3) / 1e9, ms * 1e3)
    del buf
    torch.cuda.empty_cache()
    return res


def host_link_ceiling(torch, lib, stream, host_ptr, rows, row_bytes, counts, reps=20):
    """The same plain row-read kernel (nve_amd_read_ceiling) on uniform random
    rows of a pinned host table (hipHostMalloc, read by the GPU over the host
    link): the host link's random-row read rate.  Returns
    {rows_per_launch: (GB/s, us per launch)}; bytes counted are the rows and
    their 8-byte indices."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    s = ctypes.c_void_p(stream.cuda_stream)
    fn = lib.load().nve_amd_read_ceiling
    res = {}
    for n in counts:
        idx = torch.randint(0, rows, (n,), device="cuda", generator=gen, dtype=torch.int64)
        sink = torch.zeros((n + 127) // 128, dtype=torch.int32, device="cuda")
        args = (ctypes.c_void_p(host_ptr), row_bytes, ctypes.c_void_p(idx.data_ptr()), n,
                ctypes.c_void_p(sink.data_ptr()), s)

        def launch():
            st = fn(*args)
            if st:
                lib.check(st)

        for _ in range(3):
            launch()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        res[n] = ((n * row_bytes + n * 8) / (ms * 1e-3) / 1e9, ms * 1e3)
    return res


def step_spread(torch, stream, step, groups=20, per_group=10):
    """Spread of the step time: `groups` runs of `per_group` back-to-back steps,
    each bracketed by events on `stream` (an event between every single step
    would add its own cost to a step of a few microseconds); median, p10 and
    p90 over the groups of the mean step time, in microseconds."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(groups + 1)]
    evs[0].record(stream)
    for g in range(groups):
        for i in range(per_group):
            step(g * per_group + i)
        evs[g + 1].record(stream)
    torch.cuda.synchronize()
    t = sorted(evs[g].elapsed_time(evs[g + 1]) * 1e3 / per_group for g in range(groups))

    def q(f):
        return round(t[min(groups - 1, int(f * groups))], 3)

    return {"groups": groups, "steps_per_group": per_group, "median_us": q(0.5), "p10_us": q(0.1),
            "p90_us": q(0.9)}


def f16_ulp(torch, x):
    """Spacing of fp16 numbers at |x| (x float64): 2^(floor(log2|x|) - 10), at least 2^-24."""
    _, e = torch.frexp(x)
    return torch.clamp(torch.ldexp(torch.ones_like(x), (e - 11).to(torch.int32)), min=2.0 ** -24)


def check_pooled_bags(torch, table, keys, out, hot):
    """Untimed check of every bag of a Fixed-hotness Sum lookup against
    torch's own gather summed in float64: each fp16 output within one fp16
    ulp of the exact sum, or within 1e-5 of the row's largest magnitude."""
    bags = out.shape[0]
    ref = table[keys].double().view(bags, hot, -1).sum(1)
    got = out.double()
    tol = f16_ulp(torch, ref.half().double()) + 1e-5 * ref.abs().amax(1, keepdim=True)
    bad = ((got - ref).abs() > tol).sum(1)
    if int(bad.sum().item()):
        first = int(torch.nonzero(bad)[0].item())
        raise SystemExit(f"bench.py: pooled bag {first} differs from its float64 sum in {int(bad[first])} elements")
    return bags


def host_call_costs(torch, lib, calls=400):
    """Host time per call of one c2pool-shaped pooled lookup (256 bags x 1024
    keys, CSR offsets, fp16 rows of 128) issued three ways on a 1M-row GPU
    layer: the NVEmbeddingBag module's forward (an inference layer), the
    nve_ops torch op (native, dispatcher to C ABI), and the C ABI called
    through ctypes.  Each way is issued `calls` times without a sync: the host
    time per call is the issue loop's wall time over `calls`; the GPU time per
    call comes from events around the same loop.  A way whose host time
    exceeds its GPU time cannot keep the GPU busy."""
    import pynve.torch  # noqa: F401  (the native ops library)
    from pynve.torch.nve_layers import LayerType, NVEmbeddingBag
    rows, dim, bags, hot = 1_000_000, 128, 256, 1024
    layer = NVEmbeddingBag(rows, dim, torch.float16, LayerType.GPULayer, "sum", optimize_for_training=False)
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    keys = torch.randint(0, rows, (bags * hot,), device="cuda", generator=g)
    offsets = torch.arange(0, bags * hot + 1, hot, device="cuda")
    out = torch.empty((bags, dim), dtype=torch.float16, device="cuda")
    binding = layer.emb_layer
    stream = torch.cuda.current_stream()
    ctx = binding._ctx(stream.cuda_stream)
    look = lib.load().nve_layer_lookup_pooled
    kp, op, ofp = (ctypes.c_void_p(t.data_ptr()) for t in (keys, out, offsets))
    ways = {
        "module_forward": lambda: layer(keys, offsets),
        "torch_op": lambda: torch.ops.nve_ops.embedding_lookup_with_pooling(
            layer.marker_tensor, keys, offsets, None, lib.POOL_SUM, dim, layer.dtype_tag),
        "c_abi_ctypes": lambda: look(binding._layer, ctx, bags * hot, kp, op, dim * 2, None, lib.POOL_SUM,
                                     lib.SPARSE_CSR, ofp, bags + 1, 0, None, lib.DT_UNKNOWN, lib.DT_F16, None),
    }
    res = {}
    with torch.inference_mode():
        for name, fn in ways.items():
            for _ in range(30):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record(stream)
            for _ in range(calls):
                fn()
            t1 = time.perf_counter()
            e1.record(stream)
            torch.cuda.synchronize()
            res[name] = {"host_us": round((t1 - t0) / calls * 1e6, 2),
                         "gpu_us": round(e0.elapsed_time(e1) / calls * 1e3, 2)}
    del layer
    return {"shape": "256 bags x 1024 keys (CSR), fp16 x 128, 1M-row GPU layer", "calls": calls, **res}


def zipf_ceiling(torch, lib, stream, table, row_bytes, batches, launches=100):
    """Plain row-read kernel on the workload's own keys: the random-row read kernel
    fetching row key[i] of the workload's table for every key of a batch
    (same rows, same L2/MALL reuse, no pooling), cycling the batches."""
    sink = torch.zeros((batches[0].numel() + 127) // 128, dtype=torch.int32, device="cuda")
    s = ctypes.c_void_p(stream.cuda_stream)
    n = batches[0].numel()

    fn = lib.load().nve_amd_read_ceiling  # resolved once, arguments built once per batch
    args = [(ctypes.c_void_p(table.data_ptr()), row_bytes, ctypes.c_void_p(b.data_ptr()), n,
             ctypes.c_void_p(sink.data_ptr()), s) for b in batches]

    def launch(i):
        st = fn(*args[i % len(args)])
        if st:
            lib.check(st)

    ms = time_steps(torch, stream, launch, 5, launches)
    return (n * row_bytes + n * 8) / (ms * 1e-3) / 1e9, ms * 1e3


def time_steps(torch, stream, step, warmup, steps):
    """Mean milliseconds per step between HIP events recorded on `stream`."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def fill_rows(torch, rows, width, make_chunk, seed):
    """Device table of rows x width bytes filled chunk by chunk."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    t = torch.empty((rows, width), dtype=torch.uint8, device="cuda")
    chunk = 1 << 22
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        t[r0:r1] = make_chunk(r1 - r0, gen)
    return t


def quant_rows_xi8a(torch, n, gen):
    """int8 U[-127, 127], fp32 scale log-U[1e-3, 1e-1], fp32 offset N(0, 0.01)."""
    q = torch.randint(-127, 128, (n, 256), device="cuda", dtype=torch.int16, generator=gen).to(torch.int8)
    u = torch.rand(n, device="cuda", generator=gen)
    scale = torch.exp(math.log(1e-3) + u * (math.log(1e-1) - math.log(1e-3)))
    off = torch.randn(n, device="cuda", generator=gen) * 0.01
    return torch.cat([q.view(torch.uint8), scale.view(n, 1).view(torch.uint8), off.view(n, 1).view(torch.uint8)], 1)


def quant_rows_e4m3(torch, n, gen):
    """OCP e4m3 codes (NaN codes remapped to 448) and an fp32 scale log-U[1e-3, 1e-1]."""
    q = torch.randint(0, 256, (n, 256), device="cuda", dtype=torch.int16, generator=gen).to(torch.uint8)
    q[(q & 0x7F) == 0x7F] -= 1
    u = torch.rand(n, device="cuda", generator=gen)
    scale = torch.exp(math.log(1e-3) + u * (math.log(1e-1) - math.log(1e-3)))
    return torch.cat([q, scale.view(n, 1).view(torch.uint8)], 1)


def run_workload(args, torch, _lib):
    """Parity-test configurations of BASELINE.json measured the same way
    (not the contract line): c1 (the HostLayer configuration, GPU layer and
    CPU HostLayer side by side), c2 (dedup then gather), c4a / c4b (dequant),
    c5 (26-table jagged weighted mean), c3 (LinearUVM cache over a host
    table) and c2bwd (training backprop of the c2pool lookup)."""
    L = _lib.load()
    stream = torch.cuda.Stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    w = args.workload
    kgen = torch.Generator(device="cuda")
    kgen.manual_seed(1)
    cfg_out = {"workload": w}
    extra = {}
    traffic_key = w  # profiles/traffic.json entry of this run's kernels, if any
    if w == "c1":
        # BASELINE C1, the reference HostLayer configuration: 1,000,000 x 64 fp32
        # N(0, 0.01); 4,096 bags of 8 keys uniform in [0, 1e6); the Fixed-8 Sum
        # (the metric's find-and-pool) and the plain gather, on the GPU layer and
        # on the product HostLayer beside it
        import numpy as np
        rows, dim, bags, hot = 1_000_000, 64, 4096, 8
        nkeys, width = bags * hot, dim * 4
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0)
        table = torch.empty((rows, dim), dtype=torch.float32, device="cuda").normal_(0.0, 0.01, generator=gen)
        batches = [torch.randint(0, rows, (nkeys,), device="cuda", generator=kgen, dtype=torch.int64)
                   for _ in range(args.batches)]
        pooled = torch.empty((bags, dim), dtype=torch.float32, device="cuda")
        gathered = torch.empty((nkeys, dim), dtype=torch.float32, device="cuda")
        lc = L.nve_gpu_embedding_layer_config_default()
        lc.layer_name = b"bench"
        lc.embedding_table = table.data_ptr()
        lc.num_embeddings = rows
        lc.embedding_width_in_bytes = width
        lc.value_dtype = _lib.DT_F32
        layer, ctx = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), None)
        _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(ctx), sp, sp, None, None)
        kp = [ctypes.c_void_p(b.data_ptr()) for b in batches]

        # arguments built once: a ~4 us kernel would otherwise wait on the issue loop
        pooled_args = [(layer, ctx, nkeys, k, ctypes.c_void_p(pooled.data_ptr()), width, None, _lib.POOL_SUM,
                        _lib.SPARSE_FIXED, None, 0, hot, None, _lib.DT_UNKNOWN, _lib.DT_F32, None) for k in kp]
        plain_args = [(layer, ctx, nkeys, k, ctypes.c_void_p(gathered.data_ptr()), width, None, None) for k in kp]
        pooled_fn, plain_fn = L.nve_layer_lookup_pooled, L.nve_layer_lookup

        def step(i):
            st = pooled_fn(*pooled_args[i % len(kp)])
            if st:
                _lib.check(st)

        def plain(i):
            st = plain_fn(*plain_args[i % len(kp)])
            if st:
                _lib.check(st)

        ms_plain = time_steps(torch, stream, plain, args.warmup, args.steps)
        ms = time_steps(torch, stream, step, args.warmup, args.steps)
        extra["step_spread"] = step_spread(torch, stream, step)
        # untimed: the last pooled batch against torch's float64 sums, the gather bitwise
        step(0)
        plain(0)
        torch.cuda.synchronize()
        ref = table[batches[0]].double().view(bags, hot, dim).sum(1)
        if not torch.allclose(pooled.double(), ref, rtol=1e-5, atol=1e-7):
            raise SystemExit("bench.py: c1 pooled output differs from its float64 sums")
        if not torch.equal(gathered, table[batches[0]]):
            raise SystemExit("bench.py: c1 gathered rows differ from the table rows")
        _lib.call("nve_context_wait", ctx)
        _lib.call("nve_context_destroy", ctx)
        _lib.call("nve_layer_destroy", layer)
        alg = nkeys * 8 + nkeys * width + bags * width
        alg_plain = nkeys * 8 + 2 * nkeys * width
        cfg_out.update({"table_rows": rows, "dim": dim, "row_dtype": "f32", "bags": bags, "hotness": hot,
                        "keys": "uniform", "pooling": "sum", "output_dtype": "f32",
                        "plain_gather_ms": round(ms_plain, 6),
                        "plain_gather_lookups_per_s": round(nkeys / (ms_plain * 1e-3), 1),
                        "plain_gather_GBps": round(alg_plain / (ms_plain * 1e-3) / 1e9, 1)})
        kernel = "pool_short_kernel (Fixed 8, one lane group per bag)"
        if not args.no_cpu:
            h_table = table.cpu().numpy().view(np.uint8).reshape(-1)
            h_keys = [b.cpu().numpy() for b in batches[:8]]
            h_pooled = np.empty((bags, dim), np.float32)
            h_gathered = np.empty((nkeys, dim), np.float32)
            extra["cpu_baseline"] = cpu_baseline(
                _lib, h_table, rows, width, _lib.DT_F32, h_keys,
                lambda base, k: base.pooled(k, h_pooled, width, hot, _lib.DT_F32), args.cpu_seconds,
                f"Fixed {hot} x {bags} bags, Sum, fp32",
                host_pool_check(h_table, width, _lib.DT_F32, h_keys[0], h_pooled, bags, hot))
            gb = HostLayerBaseline(_lib, h_table, rows, width, _lib.DT_F32, max(cpu_info()[1] - 2, 1))
            try:
                ts = time_batches(lambda k: gb.gather(k, h_gathered, width), h_keys, args.cpu_seconds / 2)
            finally:
                gb.close()
            med, p10, p90 = quantiles(ts)
            extra["cpu_baseline"]["plain_gather"] = {"median_ms": round(med * 1e3, 3), "p10_ms": round(p10 * 1e3, 3),
                                                     "p90_ms": round(p90 * 1e3, 3),
                                                     "lookups_per_s": round(nkeys / med, 1)}
    elif w in ("c2", "c4a", "c4b"):
        if w == "c2":
            rows, width, nkeys, alpha = 50_000_000, 256, 262144, 1.05
            gen = torch.Generator(device="cuda")
            gen.manual_seed(0)
            table = torch.empty((rows, 128), dtype=torch.float16, device="cuda")
            for r0 in range(0, rows, 1 << 24):
                table[r0:min(rows, r0 + (1 << 24))].normal_(0.0, 0.02, generator=gen)
            vdt, out_w, odt = _lib.DT_F16, 256, _lib.DT_F16
        elif w == "c4a":
            rows, width, nkeys, alpha = 100_000_000, 264, 131072, 1.05
            table = fill_rows(torch, rows, width, lambda n, g: quant_rows_xi8a(torch, n, g), 0)
            vdt, out_w, odt = _lib.DT_XI8A_F32, 512, _lib.DT_F16
        else:
            rows, width, nkeys, alpha = 100_000_000, 260, 131072, 1.05
            table = fill_rows(torch, rows, width, lambda n, g: quant_rows_e4m3(torch, n, g), 0)
            vdt, out_w, odt = _lib.DT_XE4M3_F32, 1024, _lib.DT_F32
        pg = torch.Generator(device="cuda")
        pg.manual_seed(31337)
        perm = torch.randperm(rows, generator=pg, device="cuda", dtype=torch.int64)
        batches = [power_law_keys(torch, nkeys, rows, alpha, kgen, perm) for _ in range(args.batches)]
        del perm
        out = torch.empty((nkeys, out_w), dtype=torch.uint8, device="cuda")
        lc = L.nve_gpu_embedding_layer_config_default()
        lc.layer_name = b"bench"
        lc.embedding_table = table.data_ptr()
        lc.num_embeddings = rows
        lc.embedding_width_in_bytes = width
        lc.value_dtype = vdt
        layer, ctx = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), None)
        _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(ctx), sp, sp, None, None)
        kp = [ctypes.c_void_p(b.data_ptr()) for b in batches]
        op = ctypes.c_void_p(out.data_ptr())
        if w == "c2":
            wsb = ctypes.c_uint64()
            _lib.call("nve_amd_dedup_workspace_size", nkeys, ctypes.byref(wsb))
            ws = torch.empty(int(wsb.value), dtype=torch.uint8, device="cuda")

            def step(i):
                _lib.call("nve_amd_dedup_gather", _lib.KEY_INT64, nkeys, kp[i % len(kp)],
                          ctypes.c_void_p(table.data_ptr()), rows, width, op, width,
                          ctypes.c_void_p(ws.data_ptr()), wsb.value, sp)

            def plain(i):
                _lib.check(L.nve_layer_lookup(layer, ctx, nkeys, kp[i % len(kp)], op, width, None, None))

            ms_plain = time_steps(torch, stream, plain, args.warmup, args.steps)
            cfg_out["plain_gather_ms"] = round(ms_plain, 6)
            alg = nkeys * 8 + nkeys * width + nkeys * width
        else:
            def step(i):
                _lib.check(L.nve_layer_lookup_pooled(layer, ctx, nkeys, kp[i % len(kp)], op, out_w, None,
                                                     _lib.POOL_CONCAT, 0, None, 0, 0, None, 0, odt, None))

            alg = nkeys * 8 + nkeys * width + nkeys * out_w
        ms = time_steps(torch, stream, step, args.warmup, args.steps)
        cfg_out.update({"table_rows": rows, "row_bytes": width, "keys_per_batch": nkeys, "zipf_alpha": alpha})
        _lib.call("nve_context_wait", ctx)
        _lib.call("nve_context_destroy", ctx)
        _lib.call("nve_layer_destroy", layer)
        kernel = ("hash dedup + gather: hash_clear, hash_claim_copy (claims + owners' rows), hash_repeat"
                  if w == "c2" else "gather_realign_kernel (dequant)")
    elif w == "c3":
        # LinearUVM: pinned host table + 32 GiB 8-way HBM cache, warmed by 10
        # batches (auto-insert), then timed pooled lookups whose misses read the
        # host table and are inserted when the heuristic asks for it
        rows, dim, alpha = args.c3_rows, 128, 1.2
        hot = args.c3_hotness
        bags = args.c3_keys // hot
        nkeys = bags * hot
        width = dim * 2
        log(f"c3: pinned host table {rows} x {width} B ({rows * width / 1e9:.1f} GB)")
        # exact-size hipHostMalloc (torch's pinned allocator rounds up to a power of two)
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        hip.hipHostFree.argtypes = [ctypes.c_void_p]
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        host_ptr = ctypes.c_void_p()
        if hip.hipHostMalloc(ctypes.byref(host_ptr), rows * width, 0) != 0:
            raise SystemExit("c3: hipHostMalloc of the host table failed")
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0)
        chunk = 1 << 24
        tmp = torch.empty((chunk, dim), dtype=torch.float16, device="cuda")
        for r0 in range(0, rows, chunk):
            r1 = min(rows, r0 + chunk)
            tmp[:r1 - r0].normal_(0.0, 0.02, generator=gen)
            torch.cuda.synchronize()
            assert hip.hipMemcpy(host_ptr.value + r0 * width, tmp.data_ptr(), (r1 - r0) * width, 2) == 0
        del tmp
        torch.cuda.synchronize()
        if not args.c3_no_touch:
            import numpy as np
            # The table was filled by DMA, so the host has never mapped its pages: the
            # first host read of each page faults (about 11 ms per 1024-row PipelineGather
            # task on this box).  Read one byte per 4 KiB page from host threads first, as
            # a table loaded through host memory would already be.
            t0 = time.perf_counter()
            total = rows * width
            nthreads = max(1, min(16, cpu_info()[1]))
            span = (total + nthreads - 1) // nthreads

            def touch(k):
                b0, b1 = k * span, min(total, (k + 1) * span)
                if b1 <= b0:
                    return 0
                view = np.ctypeslib.as_array((ctypes.c_uint8 * (b1 - b0)).from_address(host_ptr.value + b0))
                return int(view[::4096].sum())  # numpy reductions run without the GIL

            import concurrent.futures as cf
            with cf.ThreadPoolExecutor(nthreads) as ex:
                list(ex.map(touch, range(nthreads)))
            log(f"c3: host pages touched from {nthreads} threads in {time.perf_counter() - t0:.1f} s")
        class _Host:  # the table's address, as the layer config wants it
            def data_ptr(self):
                return host_ptr.value

        host = _Host()
        pg = torch.Generator(device="cuda")
        pg.manual_seed(31337)
        perm = torch.randperm(rows, generator=pg, device="cuda", dtype=torch.int64)
        batches = [power_law_keys(torch, nkeys, rows, alpha, kgen, perm) for _ in range(10 + args.batches)]
        del perm
        tc = L.nve_gpu_table_config_default()
        tc.cache_size = args.c3_cache_gib << 30
        tc.row_size_in_bytes = width
        tc.value_dtype = _lib.DT_F16
        tc.uvm_table = host.data_ptr()
        tc.uvm_num_rows = rows
        tc.kernel_mode_type = args.kernel_mode
        pipe_params = (ctypes.c_uint64 * 2)(1024, 16)  # PipelineGather {task_size, num_aux_streams}
        if args.kernel_mode == 3:
            tc.kernel_mode_value = ctypes.addressof(pipe_params)
        table = ctypes.c_void_p()
        _lib.call("nve_gpu_table_create", ctypes.byref(table), _lib.KEY_INT64, ctypes.byref(tc), None)
        lc = L.nve_linear_uvm_layer_config_default()
        lc.layer_name = b"bench"
        layer, ctx = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), table, None)
        _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(ctx), sp, sp, None, None)
        if args.c3_resident:
            # every row of the backing table resident in the cache, loaded as a cache
            # state (tags and rows written through import_state and the data pointer,
            # as a checkpoint restore would), so that the lookups measure the
            # cache-hit path alone: key k sits in set k % num_sets, way k // num_sets
            ns_ = ctypes.c_int64()
            _lib.call("nve_amd_gpu_table_num_sets", table, ctypes.byref(ns_))
            ns = ns_.value
            if rows > 8 * ns:
                raise SystemExit(f"c3: --c3-resident needs rows <= 8 * num_sets ({8 * ns})")
            # resident keys: row r as key r + offset (--c3-key-offset: keys of more
            # than 32 bits, as hashed ids are), in set key % num_sets; the
            # offset is a multiple of num_sets, so rows keep their set and way
            off = args.c3_key_offset // ns * ns
            idx = torch.arange(rows, dtype=torch.int64, device="cuda")
            slot = (idx % ns) * 8 + idx // ns
            tags = torch.full((ns * 8,), -1, dtype=torch.int64, device="cuda")
            tags[slot] = (idx + off) // ns
            if off:
                batches = [b + off for b in batches]
            data = torch.zeros((ns * 8, dim), dtype=torch.float16, device="cuda")
            for r0 in range(0, rows, 1 << 22):
                r1 = min(rows, r0 + (1 << 22))
                part = torch.empty((r1 - r0, dim), dtype=torch.float16, device="cuda")
                assert hip.hipMemcpy(part.data_ptr(), host_ptr.value + r0 * width, (r1 - r0) * width, 1) == 0
                data[slot[r0:r1]] = part
            torch.cuda.synchronize()
            dptr = ctypes.c_void_p()
            _lib.call("nve_amd_gpu_table_data", table, ctypes.byref(dptr))
            assert hip.hipMemcpy(dptr.value, data.data_ptr(), data.numel() * 2, 3) == 0
            _lib.call("nve_amd_gpu_table_import_state", table, ctypes.c_void_p(tags.data_ptr()), None, None, 0)
            torch.cuda.synchronize()
            del idx, slot, tags, data
            torch.cuda.empty_cache()
        concat = args.c3_concat
        out = torch.empty((nkeys if concat else bags, dim), dtype=torch.float16, device="cuda")
        hr = (ctypes.c_float * 1)()
        kp = [ctypes.c_void_p(b.data_ptr()) for b in batches]
        rates = []

        def lookup(i):
            if concat:  # one row per key (NVEmbedding forward; the reference bench's shape)
                _lib.check(L.nve_layer_lookup(layer, ctx, nkeys, kp[i], ctypes.c_void_p(out.data_ptr()), width,
                                              None, hr))
            else:
                _lib.check(L.nve_layer_lookup_pooled(layer, ctx, nkeys, kp[i], ctypes.c_void_p(out.data_ptr()),
                                                     width, None, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0,
                                                     hot, None, 0, _lib.DT_F16, hr))
            _lib.call("nve_context_wait", ctx)  # joins an auto-insert launched by this lookup
            rates.append(hr[0])

        t0 = time.perf_counter()
        for i in range(10):
            lookup(i)
        log(f"c3: warm-up hit rates {[round(r, 3) for r in rates]} ({time.perf_counter() - t0:.1f} s)")
        rates.clear()
        nt = args.batches
        for i in range(2):  # settle
            lookup(10 + i)
        rates.clear()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(args.steps):
            lookup(10 + (i % nt))
        e1.record(stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps * 1e3
        ms = e0.elapsed_time(e1) / args.steps
        hit = sum(rates) / len(rates)
        log(f"c3: {ms * 1000:.1f} us/step (events), {wall * 1000:.1f} us/step (wall), mean hit rate {hit:.4f}")
        ms_events = ms
        ms = max(ms, wall)  # the step includes a host sync (hit rate) and any insert
        if not args.c3_resident:
            # the host link's random-row read ceiling: the plain read kernel on uniform
            # rows of this same pinned table (far larger than any cache on the way), at
            # about one batch's misses, one batch and four batches of rows per launch
            miss_rows = max(1, int(nkeys * (1 - hit)))
            hl = host_link_ceiling(torch, _lib, stream, host_ptr.value, rows, width,
                                   [miss_rows, nkeys, 4 * nkeys])
            for n_, (g_, us_) in hl.items():
                log(f"c3: host-link random-row read kernel: {g_:.1f} GB/s at {n_} rows/launch ({us_:.1f} us)")
            ceiling = max(g for g, _ in hl.values())
            miss_bytes = miss_rows * width
            # the misses' rate over the step's device time (hits, tags and the
            # hit-rate readback included, so a lower bound on the miss path's rate)
            miss_rate = miss_bytes / (ms_events * 1e-3) / 1e9
            extra["host_link"] = {
                "ceiling_GBps": round(ceiling, 2),
                "read_kernel": {str(n_): {"GBps": round(g_, 2), "us": round(us_, 2)} for n_, (g_, us_) in hl.items()},
                "miss_bytes_per_step": miss_bytes,
                "miss_GBps_over_step": round(miss_rate, 2),
                "frac_of_ceiling": round(miss_rate / ceiling, 4),
                "note": "read kernel = nve_amd_read_ceiling over uniform random 256 B rows of the same "
                        "hipHostMalloc table; the miss rate divides the missed rows' bytes by the whole "
                        "lookup step's device time (events)"}
            log(f"c3: misses {miss_bytes / 1e6:.2f} MB per step at {miss_rate:.1f} GB/s over the step = "
                f"{miss_rate / ceiling:.3f} of the host link's {ceiling:.1f} GB/s read ceiling")
        if args.c3_insert_steps > 0 and not args.c3_resident:
            # the insert behind auto-insert, timed on its own: histogram of a whole
            # batch, replacement, rows copied from the host table (the reference's
            # GpuTable::insert path, gpu_table.cu:579-1046), each call waited for
            tctx = ctypes.c_void_p()
            _lib.call("nve_table_create_execution_context", table, ctypes.byref(tctx), sp, sp, None, None)
            ins = []
            for i in range(args.c3_insert_steps + 1):
                b = batches[(10 + nt + i) % len(batches)]
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                _lib.call("nve_amd_table_insert_from_uvm", table, tctx, nkeys, ctypes.c_void_p(b.data_ptr()))
                _lib.call("nve_context_wait", tctx)
                torch.cuda.synchronize()
                if i:  # the first call sizes its scratch
                    ins.append((time.perf_counter() - t0) * 1e6)
            ins.sort()
            cfg_out["insert_us"] = {"median": round(ins[len(ins) // 2], 1), "min": round(ins[0], 1),
                                    "max": round(ins[-1], 1), "calls": len(ins), "keys_per_call": nkeys}
            log(f"c3: insert of a {nkeys}-key batch: median {ins[len(ins) // 2]:.1f} us over {len(ins)} calls")
            # the insert of a collection of plain lookups: the same histogram and
            # replacement, rows copied from the lookups' output kept in HBM
            # (layer_utils.cpp:187-193, 266-267) instead of read over the host link
            rows_buf = torch.empty((nkeys, width), dtype=torch.uint8, device="cuda")
            ins_rows = []
            for i in range(args.c3_insert_steps + 1):
                b = batches[(20 + nt + i) % len(batches)]
                bp = ctypes.c_void_p(b.data_ptr())
                _lib.call("nve_table_find", table, tctx, nkeys, bp, None, width,
                          ctypes.c_void_p(rows_buf.data_ptr()), None)
                _lib.call("nve_context_wait", tctx)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                _lib.call("nve_table_insert", table, tctx, nkeys, bp, width, width,
                          ctypes.c_void_p(rows_buf.data_ptr()))
                _lib.call("nve_context_wait", tctx)
                torch.cuda.synchronize()
                if i:
                    ins_rows.append((time.perf_counter() - t0) * 1e6)
            _lib.call("nve_context_destroy", tctx)
            # the collection's own cost: one device copy of the batch's output rows
            kept = torch.empty_like(rows_buf)
            cps = []
            for i in range(6):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                kept.copy_(rows_buf)
                e1.record()
                e1.synchronize()
                if i:
                    cps.append(e0.elapsed_time(e1) * 1e3)
            del rows_buf, kept
            ins_rows.sort()
            cps.sort()
            cfg_out["insert_from_lookup_rows_us"] = {
                "median": round(ins_rows[len(ins_rows) // 2], 1), "min": round(ins_rows[0], 1),
                "max": round(ins_rows[-1], 1), "calls": len(ins_rows), "keys_per_call": nkeys,
                "collect_copy_us": round(cps[len(cps) // 2], 1)}
            log(f"c3: insert of a {nkeys}-key batch from lookup rows in HBM: median "
                f"{ins_rows[len(ins_rows) // 2]:.1f} us over {len(ins_rows)} calls; collecting the batch's "
                f"rows (one device copy) {cps[len(cps) // 2]:.1f} us")
        if args.c3_update_steps > 0 and not args.c3_resident:
            # the cache's update and update_accumulate of a whole batch (every key
            # resident) on a cache-only table of the same rows (4 GiB, no backing
            # table to write through to): records of the ways, invalidate, order
            # after the lookups, copy or add the rows, commit
            ucfg = _lib.load().nve_gpu_table_config_default()
            ucfg.cache_size = 4 << 30
            ucfg.row_size_in_bytes = width
            ucfg.value_dtype = _lib.DT_F16
            utab = ctypes.c_void_p()
            _lib.call("nve_gpu_table_create", ctypes.byref(utab), _lib.KEY_INT64, ctypes.byref(ucfg), None)
            uctx = ctypes.c_void_p()
            _lib.call("nve_table_create_execution_context", utab, ctypes.byref(uctx), sp, sp, None, None)
            ukeys = torch.randperm(rows, device="cuda")[:nkeys].to(torch.int64)
            uvals = torch.empty((nkeys, dim), dtype=torch.float16, device="cuda").normal_(0.0, 0.02)
            kp, vp_ = ctypes.c_void_p(ukeys.data_ptr()), ctypes.c_void_p(uvals.data_ptr())
            _lib.call("nve_table_insert", utab, uctx, nkeys, kp, width, width, vp_)
            _lib.call("nve_context_wait", uctx)
            upd = {}
            for name in ("update", "update_accumulate"):
                ts = []
                for i in range(args.c3_update_steps + 1):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    if name == "update":
                        _lib.call("nve_table_update", utab, uctx, nkeys, kp, width, width, vp_)
                    else:
                        _lib.call("nve_table_update_accumulate", utab, uctx, nkeys, kp, width, width, vp_,
                                  _lib.DT_F16)
                    _lib.call("nve_context_wait", uctx)
                    torch.cuda.synchronize()
                    if i:  # the first call sizes its scratch
                        ts.append((time.perf_counter() - t0) * 1e6)
                ts.sort()
                upd[name] = {"median": round(ts[len(ts) // 2], 1), "min": round(ts[0], 1), "calls": len(ts)}
                log(f"c3: cache {name} of a {nkeys}-key batch: median {ts[len(ts) // 2]:.1f} us over {len(ts)} calls")
            upd["table"] = "cache-only GpuTable, 4 GiB, fp16 x 128, every key resident"
            upd["keys_per_call"] = nkeys
            cfg_out["cache_update_us"] = upd
            _lib.call("nve_context_destroy", uctx)
            _lib.call("nve_table_destroy", utab)
            del ukeys, uvals
        # HBM: keys + 8 tags (64 B) per key + cached rows; host link: missed rows
        alg = (nkeys * (8 + 64) + int(nkeys * hit) * width + int(nkeys * (1 - hit)) * width
               + (nkeys if concat else bags) * width)
        cfg_out.update({"host_table_rows": rows, "cache_gib": args.c3_cache_gib, "keys_per_batch": nkeys,
                        "zipf_alpha": alpha, "mean_hit_rate": round(hit, 4),
                        "host_link_bytes_per_step": int(nkeys * (1 - hit)) * width,
                        "lookup": "concat" if concat else f"pooled {bags} x {hot} Sum",
                        "kernel_mode": args.kernel_mode, "resident": bool(args.c3_resident),
                        "host_pages_touched": not args.c3_no_touch,
                        "step": "lookup + hit-rate readback + auto-insert when the heuristic fires"})
        _lib.call("nve_context_destroy", ctx)
        _lib.call("nve_layer_destroy", layer)
        _lib.call("nve_table_destroy", table)
        hip.hipHostFree(host_ptr)
        kernel = ("gather_kernel / SortGather / PipelineGather (cache + host misses)" if concat
                  else "pool_split_kernel (cache + host misses)")
        # HBM counters only for the all-hit case: with misses the kernel is bound by
        # the host link, whose reads the same counters mix in
        traffic_key = "c3_cache_hit" if hit == 1.0 and not concat and args.kernel_mode == 0 else None
    elif w == "c2bwd":
        # training backprop of the headline lookup: the sparse table gradient of
        # 256 bags x 1024 Zipf(1.05) keys (50M-row range) from a 256 x 128 fp16
        # output gradient (dedup, rows and weights per position, run pooling)
        rows, dim, bags, hot, alpha = 50_000_000, 128, 256, 1024, 1.05
        nkeys = bags * hot
        pg = torch.Generator(device="cuda")
        pg.manual_seed(31337)
        perm = torch.randperm(rows, generator=pg, device="cuda", dtype=torch.int64)
        batches = [power_law_keys(torch, nkeys, rows, alpha, kgen, perm) for _ in range(args.batches)]
        del perm
        gg = torch.Generator(device="cuda")
        gg.manual_seed(5)
        grads = torch.randn((bags, dim), device="cuda", generator=gg).to(torch.float16)
        uq = torch.empty(nkeys, dtype=torch.int64, device="cuda")
        gout = torch.empty((nkeys, dim), dtype=torch.float16, device="cuda")
        wsb = ctypes.c_uint64()
        _lib.call("nve_amd_backprop_workspace_size", nkeys, bags, dim, ctypes.byref(wsb))
        ws = torch.empty(int(wsb.value), dtype=torch.uint8, device="cuda")
        nu = ctypes.c_int64()
        kp = [ctypes.c_void_p(b.data_ptr()) for b in batches]
        uniq = []

        def step(i):
            _lib.check(L.nve_amd_pooling_backprop(
                _lib.KEY_INT64, nkeys, kp[i % len(kp)], _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, hot, None,
                _lib.DT_UNKNOWN, ctypes.c_void_p(grads.data_ptr()), _lib.DT_F16, dim,
                ctypes.c_void_p(uq.data_ptr()), ctypes.c_void_p(gout.data_ptr()), ctypes.byref(nu),
                ctypes.c_void_p(ws.data_ptr()), wsb.value, sp))
            uniq.append(nu.value)

        ms = time_steps(torch, stream, step, args.warmup, args.steps)
        u = sum(uniq) // len(uniq)
        # keys + one gradient row read per key position + unique keys and rows written
        alg = nkeys * 8 + nkeys * dim * 2 + u * (8 + dim * 2)
        cfg_out.update({"table_rows": rows, "dim": dim, "bags": bags, "hotness": hot, "zipf_alpha": alpha,
                        "keys_per_batch": nkeys, "mean_unique_keys": u, "pooling": "sum",
                        "grad_dtype": "f16", "step": "one nve_amd_pooling_backprop call (synchronizes)"})
        kernel = "radix dedup (first pass on the raw keys; runs and per-position rows in two launches) + piece_pool_kernel + piece_combine_kernel"
    elif w == "c5":
        T, B, dim = 26, 8192, 128
        cg = torch.Generator()
        cg.manual_seed(4)
        cards = torch.exp(torch.log(torch.tensor(1e3)) + torch.rand(T, generator=cg, dtype=torch.float64)
                          * (torch.log(torch.tensor(4e7)) - torch.log(torch.tensor(1e3)))).long().tolist()
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0)
        tables = []
        for c in cards:
            t = torch.empty((c, dim), dtype=torch.float16, device="cuda")
            for r0 in range(0, c, 1 << 24):
                t[r0:min(c, r0 + (1 << 24))].normal_(0.0, 0.02, generator=gen)
            tables.append(t)
        lg = torch.Generator(device="cuda")
        lg.manual_seed(3)
        wg = torch.Generator(device="cuda")
        wg.manual_seed(2)
        sets = []
        for _ in range(max(2, args.batches // 4)):
            lens = torch.poisson(torch.full((T, B), 20.0, device="cuda"), generator=lg).clamp_(1, 100).long()
            off = torch.zeros(T * B + 1, dtype=torch.int64, device="cuda")
            off[1:] = torch.cumsum(lens.view(-1), 0)
            ks = []
            for t in range(T):
                pg = torch.Generator(device="cuda")
                pg.manual_seed(31337 + t)
                perm = torch.randperm(cards[t], generator=pg, device="cuda", dtype=torch.int64)
                ks.append(power_law_keys(torch, int(lens[t].sum().item()), cards[t], 1.1, kgen, perm))
            keys = torch.cat(ks)
            wts = torch.rand(keys.numel(), device="cuda", generator=wg)
            sets.append((keys, off, wts))
        nkeys = sum(s[0].numel() for s in sets) // len(sets)
        out = torch.empty((B, T, dim), dtype=torch.float32, device="cuda")
        ptrs = (ctypes.c_void_p * T)(*[t.data_ptr() for t in tables])
        rows_arr = (ctypes.c_int64 * T)(*cards)

        def step(i):
            keys, off, wts = sets[i % len(sets)]
            _lib.call("nve_amd_find_and_pool_multi", _lib.KEY_INT64, T, ptrs, rows_arr, dim * 2, _lib.DT_F16, B,
                      keys.numel(), ctypes.c_void_p(keys.data_ptr()), ctypes.c_void_p(off.data_ptr()),
                      ctypes.c_void_p(wts.data_ptr()), _lib.DT_F32, _lib.POOL_WMEAN, _lib.DT_F32,
                      ctypes.c_void_p(out.data_ptr()), sp)

        ms = time_steps(torch, stream, step, args.warmup, args.steps)
        alg = nkeys * (8 + 4 + dim * 2) + (T * B + 1) * 8 + B * T * dim * 4
        cfg_out.update({"tables": T, "cardinalities": cards, "total_rows": sum(cards), "batch": B,
                        "mean_keys_per_batch": nkeys, "pooling": "weighted_mean", "output_dtype": "f32"})
        kernel = "pool_short_kernel (multi-table)"
    else:
        raise SystemExit(f"unknown workload {w}")
    achieved = alg / (ms * 1e-3) / 1e9
    res = {"metric": METRIC, "value": round(nkeys / (ms * 1e-3), 1), "unit": "lookups/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic", "config": cfg_out,
           "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                        "kernel": kernel, "alg_bytes_per_launch": alg}}
    add_traffic(res["roofline"], traffic_key, ms)
    res.update(extra)
    log(f"{w}: {ms * 1000:.2f} us/step, {res['value'] / 1e9:.2f} G lookups/s, {achieved:.0f} GB/s")
    print(json.dumps(res), flush=True)


def add_traffic(roof, workload, ms):
    """HBM bytes per launch of the workload's dominant kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/traffic.json), over this
    run's time per step: the HBM rate net of L2 / MALL reuse."""
    tf = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(tf):
        return
    with open(tf) as f:
        entry = json.load(f).get(workload)
    if not entry:
        return
    roof["traffic"] = entry["traffic_bytes_per_launch"]
    dram = roof["traffic"] / (ms * 1e-3) / 1e9
    roof["achieved_dram"] = round(dram, 1)
    roof["frac_dram"] = round(dram / HBM_PEAK_GBPS, 4)
    roof["traffic_source"] = entry["profile"] + " (rocprofv3 --pmc)"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="c2pool",
                    choices=["c2pool", "c1", "c2", "c2bwd", "c3", "c4a", "c4b", "c5"],
                    help="c2pool (default, the metric's configuration) or a parity configuration")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rows", type=int, default=50_000_000)
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--bags", type=int, default=256)
    ap.add_argument("--hotness", type=int, default=1024)
    ap.add_argument("--alpha", type=float, default=1.05)
    ap.add_argument("--batches", type=int, default=16, help="distinct key batches cycled")
    ap.add_argument("--cpu-seconds", type=float, default=5.0,
                    help="CPU baseline: seconds of batches per thread setting")
    # BASELINE's C3 is 400M rows (102.4 GB pinned) with a 32 GB cache; the GPU
    # boxes pin at most ~64-80 GiB per allocation, so the default keeps the
    # table:cache ratio at 256M rows (65.5 GB) and a 20 GiB cache
    ap.add_argument("--c3-rows", type=int, default=256_000_000, help="c3: host table rows")
    ap.add_argument("--c3-cache-gib", type=int, default=20, help="c3: GPU cache size in GiB")
    ap.add_argument("--c3-concat", action="store_true", help="c3: one row per key instead of pooled bags")
    ap.add_argument("--c3-hotness", type=int, default=1024, choices=[16, 32, 64, 128, 256, 512, 1024],
                    help="c3: keys per pooled bag (262,144 keys per batch in 262,144 / hotness bags)")
    ap.add_argument("--c3-update-steps", type=int, default=5,
                    help="c3: timed update / update_accumulate calls of a whole batch on a cache-only table")
    ap.add_argument("--c3-keys", type=int, default=262144,
                    help="c3: keys per batch (a multiple of --c3-hotness)")
    ap.add_argument("--c3-no-touch", action="store_true",
                    help="c3: leave the DMA-filled host table's pages unmapped on the host")
    ap.add_argument("--c3-insert-steps", type=int, default=5,
                    help="c3: time this many whole-batch inserts from the backing table after the lookups")
    ap.add_argument("--c3-prefill", action="store_true",
                    help="c3: disabled (see --c3-resident)")
    ap.add_argument("--c3-key-offset", type=int, default=0,
                    help="c3 with --c3-resident: add this (rounded down to a multiple of the set count) to "
                         "every key, e.g. 2**40 for keys wider than 32 bits")
    ap.add_argument("--c3-resident", action="store_true",
                    help="c3: every backing row resident in the cache (loaded as a cache state) before the "
                         "lookups: the hit path alone; no inserts or updates are timed")
    ap.add_argument("--kernel-mode", type=int, default=0, choices=[0, 1, 2, 3],
                    help="c3: GPU table lookup mode (0 auto, 1 LookupUVM, 2 SortGather, 3 PipelineGather)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ceiling", action="store_true")
    ap.add_argument("--no-host-calls", action="store_true",
                    help="c2pool: skip the per-call host cost of the module / torch op / C ABI")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run torch's device copy of a 1 GiB buffer 5 times (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.c3_prefill:
        # a run of this mode (insert_from_uvm of 2^20 distinct keys into a 4 GiB
        # cache, then the lookups and the update timings) faulted the GPU and its
        # cause is not found: the mode stays off; --c3-resident measures the hit path
        raise SystemExit("bench.py: --c3-prefill is disabled (it faulted the GPU, cause not found); "
                         "use --c3-resident")

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the lookup path is single-GPU; across GPUs "
              "it would shard the table by rows: local dedup, an all-to-all of unique keys to their "
              "owners, find-and-pool there, an all-to-all of rows back). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from pynve import _lib

    lib = _lib
    _lib.load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "launches": 5}), flush=True)
        return
    if args.workload != "c2pool":
        return run_workload(args, torch, _lib)
    rows, dim, bags, hot = args.rows, args.dim, args.bags, args.hotness
    nkeys = bags * hot
    width = dim * 2

    log(f"table {rows} x {dim} fp16 ({rows * width / 1e9:.1f} GB), {nkeys} keys/batch")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    d_table = torch.empty((rows, dim), dtype=torch.float16, device="cuda")
    chunk = 1 << 24
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        d_table[r0:r1].normal_(0.0, 0.02, generator=gen)
    pgen = torch.Generator(device="cuda")
    pgen.manual_seed(31337)
    perm = torch.randperm(rows, generator=pgen, device="cuda", dtype=torch.int64)
    kgen = torch.Generator(device="cuda")
    kgen.manual_seed(1)
    batches = [power_law_keys(torch, nkeys, rows, args.alpha, kgen, perm) for _ in range(args.batches)]
    del perm
    out = torch.empty((bags, dim), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    uniq = torch.unique(batches[0]).numel()
    log(f"keys ready: {uniq} unique in batch 0 ({100.0 * uniq / nkeys:.1f} %)")

    stream = torch.cuda.Stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    L = _lib.load()
    cfg = L.nve_gpu_embedding_layer_config_default()
    cfg.layer_name = b"bench"
    cfg.embedding_table = d_table.data_ptr()
    cfg.num_embeddings = rows
    cfg.embedding_width_in_bytes = width
    cfg.value_dtype = _lib.DT_F16
    layer, ctx = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(cfg), None)
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(ctx), sp, sp, None, None)
    look = L.nve_layer_lookup_pooled
    kptrs = [ctypes.c_void_p(b.data_ptr()) for b in batches]
    optr = ctypes.c_void_p(out.data_ptr())

    def step(i):
        st = look(layer, ctx, nkeys, kptrs[i % len(kptrs)], optr, width, None, _lib.POOL_SUM,
                  _lib.SPARSE_FIXED, None, 0, hot, None, _lib.DT_UNKNOWN, _lib.DT_F16, None)
        if st:
            _lib.check(st)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    log(f"timed {args.steps} steps: {ms * 1000:.2f} us/step (events), wall {wall * 1e3 / args.steps * 1000:.2f} us/step")
    # untimed: the spread of single steps, then the last batch's output checked on sampled bags
    spread = step_spread(torch, stream, step)
    step(0)
    torch.cuda.synchronize()
    checked = check_pooled_bags(torch, d_table, batches[0], out, hot)
    log(f"step spread {spread}; all {checked} bags match their float64 sums")

    # algorithmic bytes per launch: keys + one stored row per key + pooled output
    alg = nkeys * 8 + nkeys * width + bags * width
    achieved = alg / (ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "pool_split_kernel<F16, G=16, unweighted>", "alg_bytes_per_launch": alg}
    add_traffic(roof, "c2pool", ms)
    result = {"metric": METRIC, "value": round(nkeys / (ms * 1e-3), 1), "unit": "lookups/s",
              "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
              "data": "synthetic",
              "config": {"workload": "C2-pool: GPUEmbeddingLayer fused find-and-pool, fp16 table in HBM",
                         "table_rows": rows, "dim": dim, "row_dtype": "f16", "keys_per_batch": nkeys,
                         "zipf_alpha": args.alpha, "bags": bags, "hotness": hot, "pooling": "sum",
                         "output_dtype": "f16", "accumulate": "f32", "key_batches_cycled": args.batches,
                         "checked_bags": checked},
              "step_spread": spread,
              "roofline": roof}
    if not args.no_ceiling:
        # A plain read kernel (rows read and folded, nothing pooled) on the same
        # keys and table, and on uniform keys over 16 GiB.  It reads the Zipf
        # batch slower than the pool kernel does (10.9 vs 8.3 us, also with 16
        # or 32 rows in flight per lane group or a chunked layout), so it bounds
        # nothing: the physical fraction is frac_dram (counted HBM bytes).
        zc, zus = zipf_ceiling(torch, _lib, stream, d_table, width, batches)
        log(f"read kernel on the workload's own keys and table: {zc:.0f} GB/s ({zus:.1f} us per batch)")
        roof["zipf_read_kernel_GBps"] = round(zc, 1)
        roof["vs_zipf_read_kernel"] = round(achieved / zc, 4)
        # same number of rows per launch as one batch, and 4x that (closer to asymptotic)
        c = read_ceiling(torch, _lib, stream, [nkeys, 4 * nkeys])
        (c1, us1), (c4, us4) = c[nkeys], c[4 * nkeys]
        log(f"uniform random-row read kernel: {c1:.0f} GB/s at {nkeys} rows/launch ({us1:.1f} us), "
            f"{c4:.0f} GB/s at {4 * nkeys} rows/launch ({us4:.1f} us)")
        result["uniform_read_kernel"] = {"GBps": round(c1, 1), "rows_per_launch": nkeys, "us": round(us1, 2),
                                         "GBps_4x_rows": round(c4, 1), "us_4x_rows": round(us4, 2)}
    if not args.no_host_calls:
        hc = host_call_costs(torch, _lib)
        log("host time per call: " + ", ".join(f"{k} {v['host_us']} us (GPU {v['gpu_us']} us)"
                                                for k, v in hc.items() if isinstance(v, dict)))
        result["host_call_us"] = hc
    if not args.no_cpu:
        import numpy as np
        log(f"cpu baseline: copying the table to host ({rows} x {dim} fp16)")
        h_table = d_table.view(torch.int16).cpu().numpy().view(np.uint8).reshape(-1)
        h_keys = [b.cpu().numpy() for b in batches[:4]]
        h_out = np.empty((bags, dim), np.float16)

        def run_batch(base, k):
            base.pooled(k, h_out, width, hot, _lib.DT_F16)

        result["cpu_baseline"] = cpu_baseline(_lib, h_table, rows, width, _lib.DT_F16, h_keys, run_batch,
                                              args.cpu_seconds, f"Fixed {hot} x {bags} bags, Sum, fp16",
                                              host_pool_check(h_table, width, _lib.DT_F16, h_keys[0], h_out,
                                                              bags, hot))
        del h_table
    _lib.call("nve_context_wait", ctx)
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_layer_destroy", layer)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
