#!/usr/bin/env python3
"""bench.py -- throughput of mechta's KV-cache path on one MI355X (libmechta_kv.so through its C ABI).

Headline workload ("cfg2"): one full-attention layer, f16 KV cache holding 65,536 positions,
a 4-token MTP verify step = append of the 4 tokens' K/V rows (RoPE + f32->f16) followed by the 4-token GQA split-K
decode (16 query / 2 KV heads, head_dim 256, causal among the drafts), then 2 drafts rejected: the length is rolled
back by 2 before the next position's appends. The steps go round the model's 10 full-attention layers, each with
its own cache (1.35 GB in all, so the K/V bytes come from HBM, not from the 256 MB last-level cache): step i is the
verify on layer i % 10, and after layer 9 the length is rolled back and the next position starts 2 further. One step
= one layer's append + decode (+ the rollback every 10 steps). Inputs (K/V rows, Q, RoPE tables) are seeded N(0,1)
values already resident in HBM when the timed region starts.

Second figure (configs[2], "cfg3"): causal prefill attention of 512 tokens appended to a cache at 28,000 positions
(28,512 keys), reported as tokens/s, timed after about 60 ms of the same steps (the clock ramps under sustained matrix
work; `warm`). Side figures: cfg1 (configs[0], 1 token at 4,096 positions with the output gate,
µs per step) and cfg4 (configs[3], the 10 layers at 262,144 positions, µs per position and the K+V read rate).

Prints ONE JSON line. value = microseconds per cfg2 step (lower is better). roofline = the decode kernel's achieved
HBM bandwidth (algorithmic K+V bytes it must read / its mean launch duration, from HIP events bracketing each launch
during a second pass of the same K steps). cpu_baseline = the C restatement in oracle/ (test infrastructure, used here
only as the reported CPU baseline) timed on this host's cores on the same cache.
"""
import argparse
import functools
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
F16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the cfg1 / cfg4 side measurements")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 256 MiB device copy kernel (reference for HBM counter scaling)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU work: summarize two rocprofv3 --pmc output directories (FETCH_SIZE, WRITE_SIZE) of a "
                         "--calib-copy run into HBM bytes per dispatch")
    ap.add_argument("--counter-summary", metavar="PMC_DIR",
                    help="no GPU work: mean of every counter per kernel and grid of a rocprofv3 --pmc output directory, "
                         "as a markdown table")
    ap.add_argument("--probe-sweep", action="store_true",
                    help="only the plain-read probe over launch shapes (work-groups, threads, loads in flight, load "
                         "policy, stage order, a tail write), as a markdown table")
    ap.add_argument("--prefill-sweep", action="store_true",
                    help="only the prefill step at contexts of 0 to 100K positions and blocks of 64 to 512, a table")
    ap.add_argument("--context-sweep", action="store_true",
                    help="only the cfg2 step at contexts of 4K to 256K positions, a markdown table")
    ap.add_argument("--flint-only", action="store_true",
                    help="only the Flint KV path's figures (decode and prefill, full and sliding layers), one JSON line")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="only the sustained dense f16 MFMA rate of the part (libmkv_probe.so), one JSON line")
    ap.add_argument("--side-only", action="store_true",
                    help="only the q/k producer and root-file figures of the default line, one JSON line (profiling)")
    ap.add_argument("--token-sweep", action="store_true",
                    help="only plain decodes of 1 to 4 tokens at 65,536 positions, with and without a window start, "
                         "one JSON line")
    ap.add_argument("--cfg5-only", action="store_true",
                    help="only configs[4] (f32 store: snapshot, restore, verify, prefill), as one JSON line (profiling)")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="no GPU work: group a rocprofv3 --kernel-trace csv by kernel and grid (launches, mean, median, "
                         "min, max microseconds) as a markdown table")
    return ap.parse_args()


# HBM bytes per launch of the two kernels at the bench's workloads, from the FETCH_SIZE and WRITE_SIZE counters
# (rocprofv3 --pmc of "bench.py --steps 20 --warmup 2 --no-cpu --no-extra --calib-copy", summarized by --pmc-summary; the
# counters are scaled by what they read for the 256 MiB copy of --calib-copy: FETCH_SIZE x 2.0, WRITE_SIZE x 1.0).
TRAFFIC = {"decode_f16": 142.52e6, "prefill_f16": 163.27e6}


def demangle_nested(raw):
    """The qualified name and integer/bool template arguments of an Itanium-mangled nested name (_ZN...E), the form
    of this library's kernels; rocprofv3 leaves a name mangled when its demangler does not know an argument type
    (_Float16, DF16_). None for any other form."""
    import re
    if not raw.startswith("_ZN"):
        return None
    i, parts, targs = 3, [], ""
    while i < len(raw) and raw[i].isdigit():
        m = re.match(r"\d+", raw[i:])
        n = int(m.group())
        i += len(m.group())
        ident = raw[i:i + n]
        i += n
        if not ident.startswith("_GLOBAL__N"):  # the anonymous namespace
            parts.append(ident)
    if not parts:
        return None
    if raw[i:i + 1] == "I":  # template arguments: literals L<type><value>E
        args, i = [], i + 1
        while raw[i:i + 1] == "L":
            m = re.match(r"L([a-z])(n?\d+)E", raw[i:])
            if not m:
                return None
            t, v = m.groups()
            v = v.replace("n", "-")
            args.append(("true" if v == "1" else "false") if t == "b" else v)
            i += len(m.group())
        if raw[i:i + 1] != "E":
            return None
        targs = "<" + ", ".join(args) + ">"
    return "::".join(parts) + targs


@functools.lru_cache(maxsize=None)
def short_name(raw, width=90):
    """A kernel name of a rocprofv3 csv without namespaces' noise or arguments (mangled names demangled first)."""
    raw = demangle_nested(raw) or raw
    return raw.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:width]


def library_kernel(name):
    """This library's kernels and the probe's (not torch's or the runtime's)."""
    return "mkv" in name or name.startswith("probe_")


def counter_summary(d):
    """Mean value per dispatch of each collected counter, per (kernel, grid) of a rocprofv3 --pmc directory."""
    import csv
    import glob
    import collections
    f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)[0]
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(f)):
        name = short_name(r["Kernel_Name"], 60)
        if not library_kernel(name):
            continue
        per[(name, int(r["Grid_Size"]))][r["Counter_Name"]].append(float(r["Counter_Value"]))
    names = sorted({c for v in per.values() for c in v})
    print("| kernel | grid | dispatches | " + " | ".join(names) + " |")
    print("|---|---|---|" + "---|" * len(names))
    for (name, grid), cs in sorted(per.items()):
        n = max(len(v) for v in cs.values())
        vals = " | ".join(f"{sum(cs[c]) / len(cs[c]):.0f}" if c in cs else "" for c in names)
        print(f"| {name} | {grid} | {n} | {vals} |")


def trace_summary(path):
    """Per (kernel, grid, work-group size) of a rocprofv3 kernel trace: launches and durations in microseconds."""
    import csv
    import collections
    import statistics
    per = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        name = short_name(r["Kernel_Name"])
        if not library_kernel(name):
            continue
        key = (name, r.get("Grid_Size_X", r.get("Grid_Size")), r.get("Workgroup_Size_X", r.get("Workgroup_Size")))
        per[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000)
    print("| kernel | grid threads | wg | launches | mean us | median us | min us | max us |")
    print("|---|---|---|---|---|---|---|---|")
    for (name, grid, wg), v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| {name} | {grid} | {wg} | {len(v)} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} | "
              f"{min(v):.2f} | {max(v):.2f} |")


def pmc_summary(fetch_dir, write_dir):
    """Mean FETCH_SIZE / WRITE_SIZE (KiB) per dispatch of each kernel, scaled to bytes by the 256 MiB copy kernel."""
    import csv
    import glob
    import collections

    def load(d):
        f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)[0]
        per = collections.defaultdict(list)
        for r in csv.DictReader(open(f)):
            per[(r["Kernel_Name"], int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
        return per

    fetch, write = load(fetch_dir), load(write_dir)
    copy_bytes = 256 << 20  # the --calib-copy kernel reads and writes 256 MiB (64M floats, grid 16,777,216)
    cf = [v for (k, g), vs in fetch.items() if g == (64 << 20) // 4 and "elementwise" in k for v in vs]
    cw = [v for (k, g), vs in write.items() if g == (64 << 20) // 4 and "elementwise" in k for v in vs]
    f_scale = copy_bytes / (max(cf) * 1024)
    w_scale = copy_bytes / (max(cw) * 1024)
    print(f"copy kernel (256 MiB read + 256 MiB written): FETCH_SIZE {max(cf):.0f} KiB -> scale {f_scale:.3f}; "
          f"WRITE_SIZE {max(cw):.0f} KiB -> scale {w_scale:.3f}")
    print("| kernel | grid | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | read MB | written MB | HBM MB |")
    print("|---|---|---|---|---|---|---|---|")
    for key in sorted(fetch, key=lambda k: -sum(fetch[k]) / len(fetch[k])):
        name, grid = key
        if "mkv" not in name or key not in write:
            continue
        fk, wk = sum(fetch[key]) / len(fetch[key]), sum(write[key]) / len(write[key])
        rb, wb = fk * 1024 * f_scale / 1e6, wk * 1024 * w_scale / 1e6
        short = short_name(name, 1000).replace("mkv::flint::", "").replace("mkv::", "")[:48]
        print(f"| {short} | {grid} | {len(fetch[key])} | {fk:.1f} | {wk:.1f} | {rb:.2f} | {wb:.2f} | {rb + wb:.2f} |")


def seeded_normal(torch, gen, shape):
    return torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32)


def rope_tabs(torch, mk, p0, p1):
    return torch.tensor([mk.rope_table(p) for p in range(p0, p1)], dtype=torch.float32, device="cuda")


def fill_store(torch, mk, st, layer, n_pos, gen, tabs, chunk=512):
    """Appends n_pos seeded tokens through the library's own append path (tabs: RoPE rows of positions 0..n_pos)."""
    for p0 in range(0, n_pos, chunk):
        m = min(chunk, n_pos - p0)
        st.append(layer, p0, seeded_normal(torch, gen, (m, 2, 256)), seeded_normal(torch, gen, (m, 512)),
                  tabs[p0:p0 + m].contiguous())
    st.sync()


DEC_LAYERS = 10  # full-attention layers of the model


def warm(torch, fn, ms=60.0, min_iters=3):
    """Runs fn until it has kept the GPU busy for about `ms` milliseconds (at least min_iters calls). Sustained
    matrix work ramps the part's clock over about 20 ms: 512-token prefill steps from a cold start, timed in blocks
    of 10, took 303, 280, 267, 254, 248, 242, 239, 238, 237, 237 us per step, and again 254 .. 243 after 0.5 s idle.
    The HBM-bound decode steps do not change with the warm-up (10, 500 or 3,000 steps: 30.2-30.7 us)."""
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while n < min_iters or (time.perf_counter() - t0) * 1e3 < ms:
        fn()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()  # the host runs far ahead of the GPU otherwise
    torch.cuda.synchronize()


_SPIN = {}


def queue_ahead(torch, us=40.0):
    """Queues a spin kernel of about `us` microseconds (torch.cuda._sleep) on the current stream, ahead of a timed
    region's start event: the GPU is then busy while the host submits the region's first launches, so the region
    starts with them already queued instead of counting the host's submission of the first launch (about 8 us on an
    idle GPU, 0.4 us per step at 20 cfg2 steps). Nothing of the timed work moves out of the region."""
    if not hasattr(torch.cuda, "_sleep"):  # a private torch API: without it the region starts on an idle GPU
        return
    if "per_us" not in _SPIN:  # spin cycles per microsecond
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n, t = 200000, 0.0
        for _ in range(2):  # the first launch of the spin kernel is not representative
            torch.cuda.synchronize()
            a.record()
            torch.cuda._sleep(n)
            b.record()
            torch.cuda.synchronize()
            t = a.elapsed_time(b) * 1000
        _SPIN["per_us"] = n / t if t > 1.0 else 0.0  # a spin shorter than 1 us: not calibrated, no spin
    if _SPIN["per_us"] > 0:
        torch.cuda._sleep(max(1000, min(int(_SPIN["per_us"] * us), 4 << 20)))  # at most 4M cycles


def bench_decode(torch, mk, steps, warmup):
    """cfg2 steps over DEC_LAYERS layers, each with its own f16 cache at 65,536 positions (1.35 GB in all, far more
    than the 256 MB last-level cache, so every step streams its layer's K/V from HBM). Step i verifies 4 tokens on
    layer i % DEC_LAYERS; after the last layer of a position the length is rolled back by 2 (2 drafts rejected) and
    the next position starts 2 further, as the model's decode does."""
    N0, NT, L = 65536, 4, DEC_LAYERS
    total = warmup + 3 * steps
    ngroups = (total + L - 1) // L
    ctx = ((N0 + 2 * ngroups + NT + 1023) // 1024) * 1024
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2026)
    st = mk.KvStore(L, ctx, mk.F16)
    tabs0 = rope_tabs(torch, mk, 0, N0)
    for layer in range(L):
        fill_store(torch, mk, st, layer, N0, gen, tabs0)
    del tabs0
    # per-step inputs, resident before timing
    kn = seeded_normal(torch, gen, (total, NT, 2, 256))
    v = seeded_normal(torch, gen, (total, NT, 512))
    q = seeded_normal(torch, gen, (total, NT, 16, 256))
    out = torch.empty((NT, 16, 256), device="cuda")
    gtabs = rope_tabs(torch, mk, N0, N0 + 2 * ngroups + NT + 1)
    kend_sum = 0

    # the C ABI called directly with every step's device pointers taken before timing, so the host issues a step in
    # far less time than the GPU runs it (the Python wrapper's argument checks took about as long as a step)
    import ctypes
    lib, h, P = mk.lib(), st.handle, ctypes.c_void_p
    args = [(i % L, N0 + 2 * (i // L), P(kn[i].data_ptr()), P(v[i].data_ptr()),
             P(gtabs[2 * (i // L) + 1].data_ptr()), P(q[i].data_ptr())) for i in range(total)]
    outp = P(out.data_ptr())

    def step(i):
        nonlocal kend_sum
        layer, pos, a, b, c, d = args[i]
        rc = lib.mkv_append_decode(h, layer, pos + 1, NT, a, b, c, d, 0, 1.0 / 16, outp, None)
        if rc != 0:
            raise mk.MkvError(rc, lib.mkv_last_error().decode())
        kend_sum += pos + NT
        if layer == L - 1:
            st.set_len(pos + 2)  # 2 of the 3 drafts rejected: roll back before the next position's appends

    for i in range(warmup):
        step(i)
    # then about 60 ms more of the same steps (untimed): the part's clocks ramp under sustained work, and the decode
    # kernel of the first few hundred steps measured about 1 us slower than the same launches repeated afterwards.
    # They re-verify the position step `warmup` will take, each round of layers rolled back; the warm-up's own last,
    # partial round of layers is then repeated, so every layer's length is what the W steps left.
    wpos = N0 + 2 * (warmup // L)
    wi = iter(range(10 ** 9))
    wtab = P(gtabs[wpos + 1 - N0].data_ptr())

    def warm_one(i):
        layer = i % L
        _, _, a, b, _, d = args[i % total]
        rc = lib.mkv_append_decode(h, layer, wpos + 1, NT, a, b, wtab, d, 0, 1.0 / 16, outp, None)
        if rc != 0:
            raise mk.MkvError(rc, lib.mkv_last_error().decode())
        if layer == L - 1:
            st.set_len(wpos)

    st.set_len(wpos)
    warm(torch, lambda: warm_one(next(wi)), ms=60.0)
    while True:  # finish the round of layers (every length back at wpos)
        j = next(wi)
        if j % L == 0:
            break
        warm_one(j)
    for i in range(warmup // L * L, warmup):
        step(i)
    torch.cuda.synchronize()
    kend_sum = 0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    queue_ahead(torch)
    t0 = time.perf_counter()
    e0.record()
    for i in range(warmup, warmup + steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)
    kend_mean = kend_sum / steps
    # then every kernel timed by its dispatch (library trace spans): the next K steps once to settle (the first few
    # hundred traced launches of a process measured about 1 us longer per decode launch than the same launches
    # traced again), then the K steps after them, whose spans are the figures
    st.trace(True)
    for i in range(warmup + steps, warmup + 2 * steps):
        step(i)
    st.trace_read()
    st.trace(False)
    kend_sum = 0
    st.trace(True)
    for i in range(warmup + 2 * steps, warmup + 3 * steps):
        step(i)
    spans = st.trace_read()
    st.trace(False)
    kend_mean2 = kend_sum / steps
    # the fused append's share of the decode launch: rounds of the same 4-token verify of every layer at one position,
    # with the append (A) and as a plain decode of the rows A wrote (B), alternating; the first two rounds of each
    # settle the trace, the next AB_ROUNDS are summed
    AB_ROUNDS = 10
    ab = {"A": [0.0, 0], "B": [0.0, 0]}
    for r in range(AB_ROUNDS + 2):
        for leg in ("A", "B"):
            st.trace(True)
            for layer in range(L):
                _, _, a, b, _, d = args[layer]
                if leg == "A":
                    rc = lib.mkv_append_decode(h, layer, wpos + 1, NT, a, b, wtab, d, 0, 1.0 / 16, outp, None)
                else:
                    rc = lib.mkv_decode(h, layer, d, NT, wpos + 1, 0, 1.0 / 16, outp, None)
                if rc != 0:
                    raise mk.MkvError(rc, lib.mkv_last_error().decode())
            sp = st.trace_read()["core"]
            st.trace(False)
            if r >= 2:
                ab[leg][0] += sp[0]
                ab[leg][1] += sp[1]
    # CPU baseline sample: layer 0's first N0 rows plus room for the 4 appended ones
    cache_rows = (st.read_rows(0, mk.K, 0, N0), st.read_rows(0, mk.V, 0, N0))
    last = dict(q=q[total - 1].cpu().numpy(), kn=kn[0].cpu().numpy(), v=v[0].cpu().numpy(),
                tab=gtabs[1:1 + NT].cpu().numpy(), n=N0 - NT + 1)
    st.close()
    return dict(ms=ms, wall=wall, steps=steps, kend=kend_mean, kend2=kend_mean2, spans=spans, ctx=ctx,
                cache=cache_rows, last=last, layers=L, ab=ab)


def bench_prefill(torch, mk, steps, warmup):
    N0, T = 28000, 512
    ctx = ((N0 + T + 1023) // 1024) * 1024
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2027)
    st = mk.KvStore(1, ctx, mk.F16)
    fill_store(torch, mk, st, 0, N0, gen, rope_tabs(torch, mk, 0, N0))
    kn = seeded_normal(torch, gen, (T, 2, 256))
    v = seeded_normal(torch, gen, (T, 512))
    q = seeded_normal(torch, gen, (T, 16, 256)) / 16.0  # pre-scaled by 1/sqrt(256)
    tabs = torch.tensor([mk.rope_table(N0 + t) for t in range(T)], dtype=torch.float32, device="cuda")
    out = torch.empty((T, 16, 256), device="cuda")

    def step():
        st.set_len(N0)
        st.append(0, N0, kn, v, tabs)
        st.prefill(0, q, N0 + 1, scale=1.0, out=out)

    for _ in range(warmup):
        step()
    warm(torch, step)  # the clock's ramp under sustained matrix work (warm's docstring)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    queue_ahead(torch)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    st.trace(True)
    for _ in range(steps):
        step()
    spans = st.trace_read()
    st.trace(False)
    st.close()
    pairs = T * N0 + T * (T + 1) // 2
    flops = 4 * 256 * 16 * pairs
    core_ms = spans["core"][0] / max(spans["core"][1], 1)
    append_ms = spans["kv_write"][0] / max(spans["kv_write"][1], 1)
    merge_ms = spans["merge"][0] / max(spans["merge"][1], 1)
    return dict(ms=ms, tok_s=T / (ms * 1e-3), flops=flops, core_ms=core_ms, core_launches=spans["core"][1] / steps,
                append_ms=append_ms, merge_ms=merge_ms, T=T)


def bench_cfg1(torch, mk, steps):
    """1 query token on an f16 cache of 4096 positions, append + decode + gate, µs per step
    (each step appends at the same position: the same work every step)."""
    N0 = 4096
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2030)
    st = mk.KvStore(1, 8192, mk.F16)
    fill_store(torch, mk, st, 0, N0, gen, rope_tabs(torch, mk, 0, N0))
    kn, v = seeded_normal(torch, gen, (1, 2, 256)), seeded_normal(torch, gen, (1, 512))
    q, gate = seeded_normal(torch, gen, (1, 16, 256)), seeded_normal(torch, gen, (1, 16, 512))
    tab = rope_tabs(torch, mk, N0, N0 + 1)
    out = torch.empty((1, 16, 256), device="cuda")
    # the C ABI called directly (the Python wrapper's checks took longer than the step: 10.9 us of host time per
    # call against 9.1 us on the GPU)
    import ctypes
    lib, h, P = mk.lib(), st.handle, ctypes.c_void_p
    a = [P(x.data_ptr()) for x in (kn, v, tab, q, out, gate)]

    def step():
        rc = lib.mkv_append_decode(h, 0, N0 + 1, 1, a[0], a[1], a[2], a[3], 0, 1.0 / 16, a[4], a[5])
        if rc != 0:
            raise mk.MkvError(rc, lib.mkv_last_error().decode())

    warm(torch, step, ms=30.0)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    queue_ahead(torch)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    st.close()
    return e0.elapsed_time(e1) / steps * 1000


def bench_cfg4(torch, mk, positions):
    """the 10 attention layers at a 262,144-position context, a 4-token verify per layer (the
    store of 5.37 GB), `positions` positions of 10 layer steps each with the rollback of 2 drafts; µs per position
    (all 10 layers) and the K+V read rate."""
    L, ctx, NT = 10, 262144, 4
    pos0 = ctx - 4 - 2 * positions
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2031)
    st = mk.KvStore(L, ctx, mk.F16)
    tabs = rope_tabs(torch, mk, 0, ctx)
    for layer in range(L):
        fill_store(torch, mk, st, layer, pos0, gen, tabs)
    kn, v = seeded_normal(torch, gen, (NT, 2, 256)), seeded_normal(torch, gen, (NT, 512))
    q = seeded_normal(torch, gen, (NT, 16, 256))
    out = torch.empty((NT, 16, 256), device="cuda")

    def position(pos):
        for layer in range(L):
            st.append_decode(layer, pos + 1, kn, v, tabs[pos + 1:pos + 1 + NT], q, out=out)
        st.set_len(pos + 2)

    position(pos0)  # warm-up position
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    queue_ahead(torch)
    e0.record()
    keys = 0
    for i in range(1, positions):
        position(pos0 + 2 * i)
        keys += (pos0 + 2 * i + NT) * L
    e1.record()
    torch.cuda.synchronize()
    st.close()
    us = e0.elapsed_time(e1) / (positions - 1) * 1000
    return us, keys * 2048 / (positions - 1) / (us * 1e-6) / 1e9


def bench_cfg5(torch, mk, reps=3):
    """f32 store, 10 layers x 16,384 positions (671 MB): snapshot to pinned host memory, restore
    into a fresh store, then a 4-token verify per layer, checked bit-identical to the same verify before the
    snapshot. Returns the snapshot and restore rates (host link), the verify's µs per layer, the identity flag, and
    a 512-token prefill on the restored store (prefill_f32 + merge, layers rotated)."""
    L, N0, NT = 10, 16384, 4
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2032)
    tabs = rope_tabs(torch, mk, 0, N0)
    a = mk.KvStore(L, 17408, mk.F32)
    for layer in range(L):
        fill_store(torch, mk, a, layer, N0 - NT + 1, gen, tabs)
    kn, v = seeded_normal(torch, gen, (NT, 2, 256)), seeded_normal(torch, gen, (NT, 512))
    q = seeded_normal(torch, gen, (NT, 16, 256))
    p = N0 - NT + 1
    nb = a.snapshot_bytes(p)
    host = torch.empty(nb, dtype=torch.uint8, pin_memory=True)

    def verify(st):
        outs = []
        for layer in range(L):
            outs.append(st.append_decode(layer, p, kn, v, tabs[p - 1:p - 1 + NT], q))
            st.set_len(p)
        return outs

    before = verify(a)
    a.snapshot(p, host)  # untimed: the process's first device-to-host copy pays a one-time set-up (about 13% slower)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        a.snapshot(p, host)
    t_snap = (time.perf_counter() - t0) / reps
    a.close()
    b = mk.KvStore(L, 17408, mk.F32)
    b.restore(p, host)  # untimed, as the snapshot
    b.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        b.restore(p, host)
        b.sync()
    t_rest = (time.perf_counter() - t0) / reps
    after = verify(b)
    same = all(torch.equal(x, y) for x, y in zip(before, after))
    # the timed verify calls the C ABI directly (a layer's call takes about as long on the GPU as the Python
    # wrapper's checks and output allocation take on the host)
    import ctypes
    lib, P = mk.lib(), ctypes.c_void_p
    tab_v = tabs[p - 1:p - 1 + NT].contiguous()
    out_v = torch.empty((NT, 16, 256), device="cuda")
    va = [P(x.data_ptr()) for x in (kn, v, tab_v, q, out_v)]

    def verify_direct(st):
        h = st.handle
        for layer in range(L):
            rc = lib.mkv_append_decode(h, layer, p, NT, va[0], va[1], va[2], va[3], 0, 1.0 / 16, va[4], None)
            if rc != 0:
                raise mk.MkvError(rc, lib.mkv_last_error().decode())
            lib.mkv_set_len(h, p)

    warm(torch, lambda: verify_direct(b))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    queue_ahead(torch)
    e0.record()
    for _ in range(10):
        verify_direct(b)
    e1.record()
    torch.cuda.synchronize()
    verify_us = e0.elapsed_time(e1) / (10 * L) * 1000
    # the f32 store's prefill (prefill_f32 + merge): a 512-token block ending at the restored length, layers rotated
    q512 = seeded_normal(torch, gen, (512, 16, 256)) / 16
    n512 = p - 511
    it = iter(range(10 ** 9))
    warm(torch, lambda: b.prefill(next(it) % L, q512, n512, scale=1.0))
    queue_ahead(torch)
    e0.record()
    for i in range(10):
        b.prefill(i % L, q512, n512, scale=1.0)
    e1.record()
    torch.cuda.synchronize()
    pf_ms = e0.elapsed_time(e1) / 10
    flops = 4 * 256 * 16 * sum(n512 + t for t in range(512))
    b.close()
    return dict(snapshot_gbps=round(nb / t_snap / 1e9, 2), restore_gbps=round(nb / t_rest / 1e9, 2),
                snapshot_mb=round(nb / 1e6, 1), verify_us_per_layer=round(verify_us, 2), bit_identical=bool(same),
                f32_prefill_512_ms=round(pf_ms, 3), f32_prefill_tflops=round(flops / (pf_ms * 1e-3) / 1e12, 1))


def bench_flint(torch, mk, ctx=32768):
    """The Flint KV path (no BASELINE config names it): one decode token and a 512-token prefill block on full layers
    at `ctx` positions (8 layers rotated, so the K/V come from HBM) and on a sliding layer (1024-row ring, 513-position
    window), f32 cache (the reference's default) and f16. µs per call of mfl_attend (attention + sink merge)."""
    from mechta_amd import flint as mf
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2033)
    res = {}

    def timed(fn, it):
        warm(torch, fn, ms=30.0)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        queue_ahead(torch)
        e0.record()
        for _ in range(it):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / it * 1000

    L = 8
    for fmt, name in ((mk.F32, "f32"), (mk.F16, "f16")):
        st = mf.FlintStore(L + 1, ctx, fmt, sliding=[False] * L + [True])
        k, v = seeded_normal(torch, gen, (512, 4, 128)), seeded_normal(torch, gen, (512, 4, 128))
        for layer in range(L + 1):
            for p0 in range(0, ctx, 512):
                st.append(layer, p0, k, v)
        q1, qb = seeded_normal(torch, gen, (1, 32, 128)), seeded_normal(torch, gen, (512, 32, 128))
        sinks = seeded_normal(torch, gen, (32,))
        o1, ob = torch.empty_like(q1), torch.empty_like(qb)
        i = [0]
        # the C ABI called directly: a one-token call takes less GPU time than the Python wrapper's checks
        import ctypes
        lib, h, P = mf.lib(), st.handle, ctypes.c_void_p
        pq1, pqb, psk, po1, pob = (P(x.data_ptr()) for x in (q1, qb, sinks, o1, ob))

        def attend(layer, pos0, ntok, pq, po):
            rc = lib.mfl_attend(h, layer, pos0, ntok, pq, psk, po)
            if rc != 0:
                raise RuntimeError(f"mfl_attend: {rc}")

        def dec():
            attend(i[0] % L, ctx - 1, 1, pq1, po1)
            i[0] += 1
        us = timed(dec, 50)
        bpe = 4 if fmt == mk.F32 else 2
        res[f"{name}_decode_full_us"] = round(us, 2)
        res[f"{name}_decode_full_gbps"] = round(ctx * 512 * bpe * 2 / (us * 1e-6) / 1e9, 1)
        res[f"{name}_decode_sliding_us"] = round(timed(lambda: attend(L, ctx - 1, 1, pq1, po1), 50), 2)
        us = timed(lambda: attend(0, ctx - 512, 512, pqb, pob), 5)
        flops = 4 * 128 * 32 * sum(ctx - 512 + t + 1 for t in range(512))
        res[f"{name}_prefill_full_us"] = round(us, 1)
        res[f"{name}_prefill_full_tflops"] = round(flops / (us * 1e-6) / 1e12, 1)
        res[f"{name}_prefill_sliding_us"] = round(timed(lambda: attend(L, ctx - 512, 512, pqb, pob), 5), 1)
        st.close()
    res["ctx"] = ctx
    return res


def bench_producer(torch, mk):
    """The q/k producer (mkv_qk_norm_rope: rmsnorm of q and k, rope2 of q) for the cfg2 step's 4 tokens and cfg3's 512,
    called through the C ABI. Bytes per token: qf 32 KB and kb 2 KB read (f32), q 16 KB and k 2 KB written, the table
    row 256 B; the norm weights once."""
    import ctypes
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2040)
    st = mk.KvStore(1, 32768, mk.F16)
    lib, h, P = mk.lib(), st.handle, ctypes.c_void_p
    res = {}
    qw, kw = seeded_normal(torch, gen, (256,)), seeded_normal(torch, gen, (256,))
    # the 512-token calls go round 12 input and output sets (330 MB, more than the 256 MB last-level cache), so their
    # bytes come from HBM
    for name, ntok, pos, it, nset in (("cfg2_4_tokens", 4, 28000, 200, 1), ("cfg3_512_tokens", 512, 28000, 48, 12)):
        sets = []
        for _ in range(nset):
            xs = (seeded_normal(torch, gen, (ntok, 16, 512)), seeded_normal(torch, gen, (ntok, 2, 256)), qw, kw,
                  torch.empty((ntok, 16, 256), device="cuda"), torch.empty((ntok, 2, 256), device="cuda"))
            sets.append((xs, [P(x.data_ptr()) for x in xs]))
        k = [0]

        def f():
            a = sets[k[0] % nset][1]
            k[0] += 1
            rc = lib.mkv_qk_norm_rope(h, pos, ntok, a[0], a[1], a[2], a[3], ctypes.c_float(1e-6), a[4], a[5])
            if rc != 0:
                raise mk.MkvError(rc, lib.mkv_last_error().decode())
        warm(torch, f, ms=20.0)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        queue_ahead(torch)
        e0.record()
        for _ in range(it):
            f()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / it * 1000
        nbytes = ntok * (8192 + 512 + 4096 + 512 + 64) * 4 + 2 * 256 * 4
        res[name] = {"us": round(us, 2), "bytes": nbytes, "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    st.close()
    return res


def bench_root(torch, mk, layers=10, p=8192):
    """A root file of positions [0, p) of a 10-layer f16 store (the reference's MECHTA-ROOT-1 container): save
    (gather to host memory, write path.tmp, rename), the same with the write on the handle's thread (the call's
    return, then the wait), and load, in MB/s of the file's bytes. Written under the system's temporary directory
    and removed afterwards; disk and page cache set the rate, not HBM."""
    import tempfile
    import numpy as np
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2041)
    st = mk.KvStore(layers, p, mk.F16)
    tabs = rope_tabs(torch, mk, 0, p)
    for layer in range(layers):
        fill_store(torch, mk, st, layer, p, gen, tabs)
    tokens = np.arange(p, dtype=np.uint32)
    d = tempfile.mkdtemp(prefix="mkv_root_bench_")
    path = os.path.join(d, "root.bin")
    res = {"p": p, "layers": layers}
    try:
        st.root_save(path, p, tokens)  # once untimed: the first host copy of a process pays a set-up
        t0 = time.perf_counter()
        st.root_save(path, p, tokens)
        t_save = time.perf_counter() - t0
        size = os.path.getsize(path)
        t0 = time.perf_counter()
        st.root_save(path, p, tokens, background=True)
        t_ret = time.perf_counter() - t0
        st.root_wait()
        t_bg = time.perf_counter() - t0
        st.set_len(0)
        t0 = time.perf_counter()
        st.root_load(path)
        t_load = time.perf_counter() - t0
        res.update({"file_mb": round(size / 1e6, 1), "save_mbps": round(size / t_save / 1e6, 1),
                    "background_return_ms": round(t_ret * 1e3, 2), "background_total_ms": round(t_bg * 1e3, 2),
                    "load_mbps": round(size / t_load / 1e6, 1)})
    finally:
        for f in os.listdir(d):
            os.remove(os.path.join(d, f))
        os.rmdir(d)
        st.close()
    return res


def bench_token_counts(torch, mk, n0=65536, layers=6):
    """Plain decodes (mkv_decode, no append) of 1 to 4 tokens at n0 positions, with and without a window start, the
    layers rotated (f16, more bytes than the last-level cache), us per call through the C ABI."""
    import ctypes
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2042)
    st = mk.KvStore(layers, (n0 + 4 + 1023) // 1024 * 1024, mk.F16)
    tabs = rope_tabs(torch, mk, 0, n0)
    for layer in range(layers):
        fill_store(torch, mk, st, layer, n0, gen, tabs)
    lib, h, P = mk.lib(), st.handle, ctypes.c_void_p
    res = {}
    for nt in (1, 2, 3, 4):
        for start in (0, 3000):
            q = seeded_normal(torch, gen, (nt, 16, 256))
            out = torch.empty((nt, 16, 256), device="cuda")
            pq, po = P(q.data_ptr()), P(out.data_ptr())
            i = [0]

            def f():
                rc = lib.mkv_decode(h, i[0] % layers, pq, nt, n0 - nt + 1, start, 1.0 / 16, po, None)
                if rc != 0:
                    raise mk.MkvError(rc, lib.mkv_last_error().decode())
                i[0] += 1
            warm(torch, f, ms=30.0)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            queue_ahead(torch)
            e0.record()
            for _ in range(60):
                f()
            e1.record()
            torch.cuda.synchronize()
            res[f"{nt}_tokens_start_{start}_us"] = round(e0.elapsed_time(e1) / 60 * 1000, 2)
    st.close()
    return {"positions": n0, "layers": layers, **res}


def bench_read_floor(torch, nbytes, nbuf=10, reps=60):
    """A plain streaming read of nbytes by one launch (libmkv_probe.so: 248 work-groups, 64 KB stages dealt round
    robin, non-temporal 16-byte loads, two stages in flight), over nbuf different buffers in turn so that nothing
    comes from the 256 MB last-level cache; durations from the dispatch timestamps, as for the decode kernel."""
    import ctypes
    here = os.path.dirname(os.path.abspath(__file__))
    probe = ctypes.CDLL(os.path.join(here, "mechta_amd", "lib", "libmkv_probe.so"))
    nbytes = (nbytes + 65535) // 65536 * 65536
    bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(nbuf)]
    torch.cuda.synchronize()
    ptrs = (ctypes.c_void_p * nbuf)(*[b.data_ptr() for b in bufs])
    mean, best = ctypes.c_float(), ctypes.c_float()
    rc = probe.mkv_probe_read(ptrs, nbuf, ctypes.c_size_t(nbytes), 248, reps, ctypes.byref(mean), ctypes.byref(best))
    if rc != 0:
        raise RuntimeError(f"mkv_probe_read failed: HIP error {rc}")
    del bufs
    return {"bytes": nbytes, "mean_us": round(mean.value, 2), "best_us": round(best.value, 2),
            "gbps": round(nbytes / (mean.value * 1e-6) / 1e9, 1),
            "what": "one launch of a plain streaming read of the decode launch's K+V bytes (libmkv_probe.so)"}


def context_sweep(torch, mk, steps=100):
    """The cfg2 step (4-token verify with its fused append) at contexts from 4,096 to 262,144 positions, with enough
    layers rotated that the K/V come from HBM (at least 512 MB in all): per context the step's µs, the decode kernel's
    and the merge's µs from the library's dispatch timestamps, and the decode's rate over the K+V it must read.
    Prints a markdown table."""
    print("| positions | layers | step us | decode_f16 us | merge us | K+V MB | decode GB/s | of 8 TB/s |")
    print("|---|---|---|---|---|---|---|---|")
    NT = 4
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2040)
    for n0 in (4096, 8192, 16384, 32768, 65536, 131072, 262140):
        L = max(2, -(-(512 << 20) // (n0 * 2048)))
        ctx = ((n0 + NT + 1023) // 1024) * 1024
        st = mk.KvStore(L, ctx, mk.F16)
        tabs = rope_tabs(torch, mk, 0, n0)
        for layer in range(L):
            fill_store(torch, mk, st, layer, n0, gen, tabs)
        del tabs
        kn, v = seeded_normal(torch, gen, (NT, 2, 256)), seeded_normal(torch, gen, (NT, 512))
        q = seeded_normal(torch, gen, (NT, 16, 256))
        tab = rope_tabs(torch, mk, n0, n0 + NT)
        out = torch.empty((NT, 16, 256), device="cuda")
        i = [0]
        import ctypes
        lib, h, P = mk.lib(), st.handle, ctypes.c_void_p
        a = (P(kn.data_ptr()), P(v.data_ptr()), P(tab.data_ptr()), P(q.data_ptr()))
        op = P(out.data_ptr())

        def step():  # the C ABI called directly, as in bench_decode
            layer = i[0] % L
            rc = lib.mkv_append_decode(h, layer, n0 + 1, NT, *a, 0, 1.0 / 16, op, None)
            if rc != 0:
                raise mk.MkvError(rc, lib.mkv_last_error().decode())
            if layer == L - 1:
                st.set_len(n0)  # every position's drafts rejected: the same work each round
            i[0] += 1

        warm(torch, step, ms=40.0)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        queue_ahead(torch)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / steps * 1000
        for settle in (True, False):  # a settling traced pass, then the recorded one (as bench_decode)
            st.trace(True)
            for _ in range(steps):
                step()
            sp = st.trace_read()
            st.trace(False)
        st.close()
        core = sp["core"][0] / sp["core"][1] * 1000
        merge = sp["merge"][0] / max(1, sp["merge"][1]) * 1000
        mb = (n0 + NT) * 2048 / 1e6
        gbs = mb * 1e3 / core
        print(f"| {n0 + NT} | {L} | {us:.2f} | {core:.2f} | {merge:.2f} | {mb:.1f} | {gbs:.0f} | "
              f"{gbs / HBM_PEAK_GBS:.3f} |", flush=True)


def prefill_sweep(torch, mk):
    """The cfg3 step (a 512-token block appended and prefilled) at contexts of 0 to 100,000 positions and blocks of 64
    to 512 tokens at 28,000 positions, f16 and f32 stores: µs per step, the attention kernel's and the merge's µs from
    the library's trace, and the kernel's TFLOP/s. Prints a markdown table."""
    print("| store | positions before | tokens | step us | kernel us | merge us | kernel TFLOP/s | of 2.5 PFLOP/s |")
    print("|---|---|---|---|---|---|---|---|")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2041)
    for fmt, name in ((mk.F16, "f16"), (mk.F32, "f32")):
        cases = [(0, 512), (2048, 512), (8192, 512), (28000, 512), (100000, 512), (28000, 64), (28000, 128)]
        ctx = 101376
        st = mk.KvStore(1, ctx, fmt)
        for n0, T in cases:
            tabs = rope_tabs(torch, mk, 0, n0 + T)
            kn = seeded_normal(torch, gen, (n0 + T, 2, 256))
            v = seeded_normal(torch, gen, (n0 + T, 512))
            st.set_len(0)
            for p0 in range(0, n0, 512):
                m = min(512, n0 - p0)
                st.append(0, p0, kn[p0:p0 + m], v[p0:p0 + m], tabs[p0:p0 + m])
            q = seeded_normal(torch, gen, (T, 16, 256)) / 16.0

            def step():
                st.set_len(n0)
                st.append(0, n0, kn[n0:n0 + T], v[n0:n0 + T], tabs[n0:n0 + T])
                st.prefill(0, q, n0 + 1, scale=1.0)

            warm(torch, step, ms=40.0)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            queue_ahead(torch)
            e0.record()
            for _ in range(10):
                step()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / 10 * 1000
            st.trace(True)
            for _ in range(10):
                step()
            sp = st.trace_read()
            st.trace(False)
            core = sp["core"][0] / sp["core"][1] * 1000
            merge = sp["merge"][0] / max(1, sp["merge"][1]) * 1000
            tf = 4 * 256 * 16 * sum(n0 + t + 1 for t in range(T)) / (core * 1e-6) / 1e12
            print(f"| {name} | {n0} | {T} | {us:.1f} | {core:.1f} | {merge:.1f} | {tf:.0f} | "
                  f"{tf / F16_MFMA_PEAK_TFLOPS:.3f} |", flush=True)
        st.close()


def bench_mfma_rate(wgs=512, iters=4000, reps=20):
    """The dense f16 rate the matrix units sustain on this part with nothing else to do (libmkv_probe.so: every wave
    runs 8 independent v_mfma_f32_32x32x16_f16 chains from registers, two waves per SIMD), after about 60 ms of the
    same launches (the clock ramps under matrix work): the ceiling the prefill's roofline fraction, taken against the
    published 2.5 PFLOP/s, is read beside."""
    import ctypes
    here = os.path.dirname(os.path.abspath(__file__))
    probe = ctypes.CDLL(os.path.join(here, "mechta_amd", "lib", "libmkv_probe.so"))
    tf, us = ctypes.c_float(), ctypes.c_float()
    rc = probe.mkv_probe_mfma(wgs, iters, reps, ctypes.c_float(60.0), ctypes.byref(tf), ctypes.byref(us))
    if rc != 0:
        raise RuntimeError(f"mkv_probe_mfma failed: HIP error {rc}")
    return {"tflops": round(tf.value, 1), "frac_of_peak": round(tf.value / F16_MFMA_PEAK_TFLOPS, 4),
            "launch_us": round(us.value, 1),
            "what": "dense f16 MFMA chains from registers only, 2 waves per SIMD, after a 60 ms warm-up"}


def bench_launch_floor(torch, nbytes, nbuf=10, reps=200):
    """What two launches back to back cost at least (libmkv_probe.so), for a step of a decode launch reading nbytes
    and a merge launch: the best back-to-back time per launch of a plain streaming read of nbytes (over a few launch
    shapes) plus that of an empty launch of the decode's shape. Microseconds."""
    import ctypes
    here = os.path.dirname(os.path.abspath(__file__))
    probe = ctypes.CDLL(os.path.join(here, "mechta_amd", "lib", "libmkv_probe.so"))
    unit = 512 * 8 * 16  # one 64 KB stage of a 512-thread work-group
    nbytes = (nbytes + unit - 1) // unit * unit
    bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(nbuf)]
    torch.cuda.synchronize()
    ptrs = (ctypes.c_void_p * nbuf)(*[b.data_ptr() for b in bufs])

    def wall(wgs, nb):
        mean, best, w = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        rc = probe.mkv_probe_run(ptrs, nbuf, ctypes.c_size_t(nb), wgs, 512, 2, 1, 1, ctypes.c_size_t(0), reps,
                                 ctypes.byref(mean), ctypes.byref(best), ctypes.byref(w))
        if rc != 0:
            raise RuntimeError(f"mkv_probe_run failed: HIP error {rc}")
        return w.value
    stages = nbytes // unit
    read = min(wall(g, nbytes) for g in sorted({stages, max(1, stages // 2), min(248, stages * 2)}))
    empty = wall(max(1, stages // 2), 0)
    del bufs
    return {"bytes": nbytes, "read_us": round(read, 2), "empty_launch_us": round(empty, 2),
            "floor_us": round(read + empty, 2),
            "what": "back to back: one launch of a plain streaming read of the step's K+V bytes (best of 3 shapes) "
                    "plus one empty launch (libmkv_probe.so)"}


def probe_sweep(torch, nbytes=134348800, nbuf=10, reps=60):
    """The plain-read probe (libmkv_probe.so) over launch shapes, for the bytes of one cfg2 decode launch, over nbuf
    buffers in turn (nothing from the last-level cache). Prints a markdown table: per shape the launch duration from
    the dispatch timestamps (mean, best) and the time per launch back to back."""
    import ctypes
    here = os.path.dirname(os.path.abspath(__file__))
    probe = ctypes.CDLL(os.path.join(here, "mechta_amd", "lib", "libmkv_probe.so"))
    unit = 1024 * 128
    nbytes = (nbytes + unit - 1) // unit * unit
    bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(nbuf)]
    torch.cuda.synchronize()
    ptrs = (ctypes.c_void_p * nbuf)(*[b.data_ptr() for b in bufs])
    # (what, work-groups, threads, depth, non-temporal, round robin (2 + k: skew of k + 1 stages), tail bytes (+ store
    # policy 0..3), bytes)
    shapes = [("empty launch", 248, 512, 2, 1, 1, 0, 0),
              ("default: 248 x 512, 2 stages in flight, nt, round robin", 248, 512, 2, 1, 1, 0, nbytes)]
    shapes += [(f"depth {d}", 248, 512, d, 1, 1, 0, nbytes) for d in (1, 3, 4)]
    shapes += [(f"{w} work-groups", w, 512, 2, 1, 1, 0, nbytes) for w in (124, 186, 256, 496, 512, 1024, 2048)]
    shapes += [("124 work-groups, depth 3", 124, 512, 3, 1, 1, 0, nbytes),
               ("124 x 1024 threads", 124, 1024, 2, 1, 1, 0, nbytes)]
    shapes += [(f"{w} x 256 threads", w, 256, 2, 1, 1, 0, nbytes) for w in (248, 496, 992)]
    shapes += [(f"{w} x 256 threads, depth 4", w, 256, 4, 1, 1, 0, nbytes) for w in (496, 992)]
    shapes += [("248 x 1024 threads", 248, 1024, 2, 1, 1, 0, nbytes),
               ("default load policy", 248, 512, 2, 0, 1, 0, nbytes),
               ("contiguous range per work-group", 248, 512, 2, 1, 0, 0, nbytes),
               ("tail write 33 KB per work-group", 248, 512, 2, 1, 1, 33280, nbytes),
               ("tail write 16 KB per work-group", 248, 512, 2, 1, 1, 16640, nbytes),
               ("tail write 33 KB, sc1 stores", 248, 512, 2, 1, 1, 33280 + 1, nbytes),
               ("tail write 33 KB, nt stores", 248, 512, 2, 1, 1, 33280 + 2, nbytes),
               ("tail write 33 KB, sc0 sc1 stores", 248, 512, 2, 1, 1, 33280 + 3, nbytes),
               ("fused merge: partials 33 KB + barrier per half (wait 1) + merge read", 248, 512, -4, 1, 1, 0, nbytes),
               ("fused merge, wait 20", 248, 512, -5, 1, 1, 0, nbytes),
               ("fused merge: partials only", 248, 512, -1, 1, 1, 0, nbytes),
               ("fused merge: partials + fence + merge read, no counters", 248, 512, -2, 1, 1, 0, nbytes),
               ("fused merge: partials + fence + arrival atomic + merge read", 248, 512, -3, 1, 1, 0, nbytes),
               ("fused merge, sc1 partials, relaxed counters (wait 1)", 248, 512, -6, 1, 1, 0, nbytes),
               ("fused merge, sc1 partials, relaxed counters (wait 8)", 248, 512, -7, 1, 1, 0, nbytes),
               ("fused merge, sc1 partials, arrivals only (no wait)", 248, 512, -8, 1, 1, 0, nbytes),
               ("fused merge, sc1 partials, 8 sub-counters + top", 248, 512, -9, 1, 1, 0, nbytes),
               ("fused merge, sc1 partials, a flag per work-group (epoch)", 248, 512, -10, 1, 1, 0, nbytes),
               ("empty launch, sc1 fused-merge tail only", 248, 512, -6, 1, 1, 0, 0),
               ("empty launch, sc1 tail, 8 sub-counters", 248, 512, -9, 1, 1, 0, 0),
               ("empty launch, sc1 tail, flags", 248, 512, -10, 1, 1, 0, 0),
               ("skew 2: half the work-groups 2 stages more, half 2 fewer", 248, 512, 2, 1, 3, 0, nbytes),
               ("skew 2 + tail write 33 KB", 248, 512, 2, 1, 3, 33280, nbytes),
               ("skew 3 + tail write 33 KB", 248, 512, 2, 1, 4, 33280, nbytes),
               ("half the bytes (67 MB)", 248, 512, 2, 1, 1, 0, nbytes // 2 // unit * unit),
               ("67 MB, 496 x 256 threads", 496, 256, 2, 1, 1, 0, nbytes // 2 // unit * unit),
               ("67 MB, 248 x 256 threads", 248, 256, 2, 1, 1, 0, nbytes // 2 // unit * unit),
               ("67 MB, 248 x 512, depth 1", 248, 512, 1, 1, 1, 0, nbytes // 2 // unit * unit),
               ("67 MB, contiguous range per work-group", 248, 512, 2, 1, 0, 0, nbytes // 2 // unit * unit),
               ("67 MB, 496 x 256, contiguous", 496, 256, 2, 1, 0, 0, nbytes // 2 // unit * unit),
               ("4x the bytes (537 MB, cfg4 per layer)", 248, 512, 2, 1, 1, 0, None)]
    rows = []
    for what, wgs, thr, depth, nt, rr, tail, nb in shapes:
        if nb is None:  # 4x: the buffers hold it only in pairs of 4 consecutive tensors; use one big buffer set
            big = [torch.ones(nbytes, dtype=torch.float32, device="cuda") for _ in range(3)]
            p = (ctypes.c_void_p * 3)(*[b.data_ptr() for b in big])
            nb, pp, nn = nbytes * 4, p, 3
        else:
            big, pp, nn = None, ptrs, nbuf
        mean, best, wall = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        rc = probe.mkv_probe_run(pp, nn, ctypes.c_size_t(nb), wgs, thr, depth, nt, rr, ctypes.c_size_t(tail), reps,
                                 ctypes.byref(mean), ctypes.byref(best), ctypes.byref(wall))
        if rc != 0:
            raise RuntimeError(f"mkv_probe_run failed on {what}: HIP error {rc}")
        del big
        gbs = nb / (mean.value * 1e-6) / 1e9 if nb else 0.0
        rows.append((what, wgs, thr, depth, nb, mean.value, best.value, wall.value, gbs))
        print(f"# {what}: {mean.value:.2f} us", file=sys.stderr, flush=True)
    print("| shape | work-groups | threads | stages in flight | MB | mean us | best us | back-to-back us | GB/s (mean) |")
    print("|---|---|---|---|---|---|---|---|---|")
    for what, wgs, thr, depth, nb, mean, best, wall, gbs in rows:
        print(f"| {what} | {wgs} | {thr} | {depth} | {nb / 1e6:.1f} | {mean:.2f} | {best:.2f} | {wall:.2f} | "
              f"{gbs:.0f} |")


def cpu_baseline(dec, budget_s):
    """The oracle's attn_dmx + append on the bench's own cache, on this host's cores."""
    import numpy as np
    from oracle import oracle as O
    kc = dec["cache"][0].cpu().numpy().view(np.uint16)
    vc = dec["cache"][1].cpu().numpy().view(np.uint16)
    L = dec["last"]
    n = L["n"]
    kcw, vcw = kc.copy(), vc.copy()
    reps, t_att = 0, 0.0
    t_start = time.perf_counter()
    while reps < 50 and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        O.append(0, kcw, vcw, n - 1, L["kn"], L["v"], L["tab"])
        O.attn_dmx(kcw, vcw, L["q"], n)
        t_att += time.perf_counter() - t0
        reps += 1
    us = t_att / reps * 1e6
    return dict(value=round(us, 1), unit="us/step", cores=O.threads(), kind="port",
                sample=f"{reps} cfg2 steps (4-token append + attn_dmx restatement, {n + 3} keys) on the same cache")


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.counter_summary:
        counter_summary(args.counter_summary)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the KV-cache path would "
              f"shard over positions with one small all-gather of split-K partials per step (design only).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import mechta_amd as mk
    mk.lib()
    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(1)
    if args.probe_sweep:
        probe_sweep(torch)
        return
    if args.prefill_sweep:
        prefill_sweep(torch, mk)
        return
    if args.context_sweep:
        context_sweep(torch, mk)
        return
    if args.flint_only:
        r = bench_flint(torch, mk)
        if args.calib_copy:
            src = torch.ones(64 << 20, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(5):
                torch.add(src, 0.0, out=dst)
            torch.cuda.synchronize()
        print(json.dumps({"flint": r}), flush=True)
        return
    if args.mfma_probe:
        print(json.dumps({"mfma_sustained": bench_mfma_rate()}), flush=True)
        return
    if args.side_only:
        print(json.dumps({"producer": bench_producer(torch, mk), "root": bench_root(torch, mk)}), flush=True)
        return
    if args.token_sweep:
        print(json.dumps({"token_sweep": bench_token_counts(torch, mk)}), flush=True)
        return
    if args.cfg5_only:
        r = bench_cfg5(torch, mk)
        if args.calib_copy:
            src = torch.ones(64 << 20, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(5):
                torch.add(src, 0.0, out=dst)
            torch.cuda.synchronize()
        print(json.dumps({"cfg5": r}), flush=True)
        return
    dec = bench_decode(torch, mk, args.steps, args.warmup)
    ms_step = dec["ms"] / dec["steps"]
    bytes_rw = dec["kend"] * 2 * 256 * 2 * 2 + 4 * 2 * 256 * 2 * 2
    core_ms, core_n = dec["spans"]["core"]
    core_avg_ms = core_ms / max(core_n, 1)
    core_bytes = dec["kend2"] * 2 * 256 * 2 * 2
    achieved = core_bytes / (core_avg_ms * 1e-3) / 1e9
    res = {
        "metric": "decode attn+append us/step & HBM GB/s @64K ctx; prefill attn tok/s",
        "value": round(ms_step * 1e3, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) K/V/Q, RoPE tables from rope_table)",
        "config": {"workload": "cfg2: 4-token MTP verify step on one attention layer, f16 KV at 65,536 positions: "
                               "append 4 rows + GQA split-K decode, then 2 drafts rolled back",
                   "q_heads": 16, "kv_heads": 2, "head_dim": 256, "ctx": dec["ctx"], "layers_rotated": dec["layers"],
                   "keys_per_step_mean": round(dec["kend"], 1)},
        "hbm_gbps_step": round(bytes_rw / (ms_step * 1e-3) / 1e9, 1),
        "kernel_ms": {k: round(v[0] / max(v[1], 1), 5) for k, v in dec["spans"].items()},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC["decode_f16"],
                     "kernel": "decode_f16", "bytes_per_launch": int(core_bytes)},
    }
    (a_ms, a_n), (b_ms, b_n) = dec["ab"]["A"], dec["ab"]["B"]
    core_ab_us, core_plain_us = a_ms / max(a_n, 1) * 1e3, b_ms / max(b_n, 1) * 1e3
    # the fused append at cfg2: 4 tokens x (K normed + V inputs in f32, RoPE rows) read, 4 rows of K and V written (f16)
    append_bytes4 = 4 * (2 * 256 * 4 + 512 * 4 + 64 * 4) + 4 * 2 * 2 * 256 * 2
    res["append"] = {"cfg2_fused_4_rows": {"core_with_append_us": round(core_ab_us, 2),
                                           "core_plain_decode_us": round(core_plain_us, 2),
                                           "incremental_us": round(core_ab_us - core_plain_us, 2),
                                           "launches": a_n,
                                           "bytes": append_bytes4}}
    if not args.no_prefill:
        pf = bench_prefill(torch, mk, max(10, args.steps // 5), 5)
        res["prefill_tok_s"] = round(pf["tok_s"], 1)
        res["prefill_ms"] = round(pf["ms"], 4)
        # append_kernel of the 512-token block: f32 K normed, V and RoPE rows read, f16 K and V rows written
        ab = pf["T"] * (2 * 256 * 4 + 512 * 4 + 64 * 4) + pf["T"] * 2 * 2 * 256 * 2
        agbs = ab / (pf["append_ms"] * 1e-3) / 1e9
        res["append"]["cfg3_512_tokens"] = {"us": round(pf["append_ms"] * 1e3, 2), "bytes": ab, "gbps": round(agbs, 1),
                                            "frac": round(agbs / HBM_PEAK_GBS, 4), "kernel": "append_kernel"}
        if pf["core_launches"] == 1:
            tf = pf["flops"] / (pf["core_ms"] * 1e-3) / 1e12
            res["roofline_prefill"] = {"bound": "mfma", "achieved": round(tf, 1), "peak": F16_MFMA_PEAK_TFLOPS,
                                       "unit": "TFLOP/s", "frac": round(tf / F16_MFMA_PEAK_TFLOPS, 4),
                                       "traffic": TRAFFIC["prefill_f16"], "kernel": "prefill_f16"}
    if not args.no_extra:
        res["cfg1_us_per_step"] = round(bench_cfg1(torch, mk, 200), 2)
        res["cfg1_floor"] = bench_launch_floor(torch, 4097 * 2 * 256 * 2 * 2)
        us4, gbs4 = bench_cfg4(torch, mk, 20)
        res["cfg4_us_per_position_10_layers"] = round(us4, 1)
        res["cfg4_kv_read_gbps"] = round(gbs4, 1)
        res["cfg5"] = bench_cfg5(torch, mk)
        res["flint"] = bench_flint(torch, mk)
        res["producer"] = bench_producer(torch, mk)
        res["root"] = bench_root(torch, mk)
        res["hbm_read_floor"] = bench_read_floor(torch, int(core_bytes))
        res["mfma_sustained"] = bench_mfma_rate()
    if args.calib_copy:
        # plain elementwise copy of a known size: its FETCH_SIZE / WRITE_SIZE counters give the scale from counter
        # units to bytes for the KV kernels' counters in the same run
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.add(src, 0.0, out=dst)
        torch.cuda.synchronize()
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(dec, args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
