"""Paged decode benchmark on one MI355X.

Default workload: matched split-KV decode (partition + LSE merge, the two
launches of matched_decode), B=1, Hq=16,
Hkv=4, D=256, page 256, context 2064 (table capacity 2112), bf16 N(0,1)
synthetic Q/K/V, pages in a seeded random physical order, the planner's plan
for the device's CU count.  A step is one operator call (both kernels).  The
timed calls are whole replays of one hipGraph that unrolls 128 calls: K steps
are rounded up to a multiple of 128 (at least one replay) and reported as
calls_timed, so the per-call figure does not depend on K.  The inputs are
resident in device memory; across calls the 8.5 MB of KV stays in the
last-level cache (hot cache, the workload's own setting), and hbm_resident
reports the same call with its KV read from HBM.

Printed: one JSON line with value = achieved algorithmic TB/s of the full call,
a roofline object for the partition kernel (timed alone with HIP events on its
launch stream), the CPU baseline (NumPy restatement of the reference CPU path
on the host cores) and extra measurements (context 528, 1024-token partitions,
the batch-64 bandwidth sweep over a 200 GB page pool).
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "paged-decode-lab_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_TBPS = 8.0            # MI355X HBM3E
UNROLL = 128               # calls per captured graph (reference convention)
PAGE = 256


def progress(msg):
    """One line per finished measurement, on stderr (the JSON line stays alone on stdout)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(lengths, batch, hq, hkv, dim, with_output=True):
    """Bytes the operator must move: K+V rows, Q, output, live table entries, lengths."""
    kv = sum(int(n) for n in lengths) * hkv * dim * 2 * 2
    q = batch * hq * dim * 2
    out = batch * hq * dim * 2 if with_output else 0
    table = sum((int(n) + PAGE - 1) // PAGE for n in lengths) * 4
    return kv + q + out + table + batch * 4


def make_inputs(torch, batch, hq, hkv, dim, capacity, lengths, seed, pool_pages=None):
    """Seeded synthetic inputs; pages scattered over a pool of ``pool_pages`` pages."""
    dev = torch.device("cuda")
    width = (capacity + PAGE - 1) // PAGE
    gen = torch.Generator(device=dev).manual_seed(seed)
    live = [(int(n) + PAGE - 1) // PAGE for n in lengths]
    pool = pool_pages or batch * width
    physical = torch.randperm(pool, device=dev, generator=gen)[: sum(live)]
    table = torch.full((batch, width), -1, dtype=torch.int32, device=dev)
    offset = 0
    for b, n in enumerate(live):
        table[b, :n] = physical[offset:offset + n].to(torch.int32)
        offset += n
    k = torch.empty((pool, PAGE, hkv, dim), dtype=torch.bfloat16, device=dev)
    v = torch.empty_like(k)
    if pool_pages is None:
        k.normal_(generator=gen)
        v.normal_(generator=gen)
    else:  # initialize only the live pages of a large pool
        idx = physical.long()
        for chunk in torch.split(idx, 1024):
            k[chunk] = torch.randn((len(chunk), PAGE, hkv, dim), generator=gen, device=dev,
                                   dtype=torch.bfloat16)
            v[chunk] = torch.randn((len(chunk), PAGE, hkv, dim), generator=gen, device=dev,
                                   dtype=torch.bfloat16)
    q = torch.randn((batch, hq, dim), generator=gen, device=dev, dtype=torch.bfloat16)
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    return q, k, v, table, lens


def timed_calls(calls, unroll=UNROLL):
    """Calls actually timed for a request of ``calls``: whole replays of the ``unroll``-call
    graph, at least one, so the per-call figure never depends on how many were asked for."""
    return unroll * max(1, -(-calls // unroll))


def graph_time_us(torch, fn, calls, unroll=UNROLL, warmup=3):
    """Microseconds per call, timed over ``timed_calls(calls, unroll)`` calls: replays of one
    graph of ``unroll`` calls (the reference convention captures 128), on the replay stream."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(unroll):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    replays = timed_calls(calls, unroll) // unroll
    torch.cuda.synchronize()
    start.record(cur)
    for _ in range(replays):
        graph.replay()
    end.record(cur)
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / (replays * unroll)


def reference_protocol_us(torch, fn, rounds=5, replays=20):
    """Reference convention: 128-call graph, 20 replays, median of 5 rounds; t32 vs t128."""
    from paged_decode.benchmark_protocol import convergence_delta
    t128 = sorted(graph_time_us(torch, fn, replays * 128, 128) for _ in range(rounds))[rounds // 2]
    t32 = sorted(graph_time_us(torch, fn, replays * 32, 32) for _ in range(rounds))[rounds // 2]
    return t128, t32, convergence_delta(t32, t128)


def matched_case(torch, batch, hq, hkv, dim, capacity, lengths, seed, num_splits=0,
                 pool_pages=None):
    from paged_decode.matched_splitkv import (MatchedResources, allocate_matched_resources,
                                              matched_decode)
    from paged_decode.spec import DecodeSpec
    from paged_decode import _native
    spec = DecodeSpec(batch, hq, hkv, dim, capacity)
    res = allocate_matched_resources(spec, "cuda", num_splits=num_splits, fused=True)
    q, k, v, table, lens = make_inputs(torch, batch, hq, hkv, dim, capacity, lengths, seed,
                                       pool_pages)
    plan = res.plan
    scale = dim ** -0.5

    # Default resources (no counters): matched_decode's two launches.
    two_launch = MatchedResources(spec, plan, res.out, res.partials, res.lse)

    def fused():
        matched_decode(q, k, v, table, lens, resources=res)

    def full():
        matched_decode(q, k, v, table, lens, resources=two_launch)

    def partition():
        _native.partition(q, k, v, table, lens, res.partials, res.lse, hkv, plan.splits,
                          plan.tokens_per_split, plan.tile_tokens, scale)

    def merge():
        _native.lse_merge(res.partials, res.lse, res.out, plan.lse_lanes)

    return dict(spec=spec, plan=plan, full=full, fused=fused, partition=partition,
                merge=merge, tensors=(q, k, v, table, lens), res=res, two_launch=two_launch)


def hbm_resident_rate(torch, case, copies=64):
    """The headline call with its KV read from HBM instead of the last-level cache.

    ``copies`` sequences' worth of pages (64 x 9.4 MB = 604 MB, past the 256 MB
    last-level cache and the 8 x 4 MB L2s) are scattered over one pool, and the 128
    calls of the graph cycle through their tables, so a call's pages were last read
    64 calls earlier and have been evicted since.  Returns (us/call, copies, pool MB)."""
    from paged_decode.matched_splitkv import matched_decode
    q, k, v, table, lens = case["tensors"]
    spec, res = case["spec"], case["res"]
    width = spec.table_width
    gen = torch.Generator(device="cuda").manual_seed(7)
    pool = copies * width
    kp = torch.randn((pool, PAGE, spec.num_kv_heads, spec.head_dim), generator=gen,
                     device="cuda", dtype=torch.bfloat16)
    vp = torch.randn_like(kp)
    pages = torch.randperm(pool, generator=gen, device="cuda").to(torch.int32)
    tables = [pages[i * width:(i + 1) * width].view(1, width).contiguous() for i in range(copies)]
    two = case["two_launch"]
    calls = iter(range(1 << 30))

    def call():
        matched_decode(q, kp, vp, tables[next(calls) % copies], lens, resources=two)
    us = graph_time_us(torch, call, UNROLL, unroll=UNROLL, warmup=copies)
    mb = 2 * kp.numel() * 2 / 1e6
    del kp, vp
    torch.cuda.empty_cache()
    return us, copies, mb


def fixed_partition_case(torch, case, part_tokens=1024):
    """The same kernels with fixed ``part_tokens`` partitions (splits = ceil(cap / part))."""
    from paged_decode import _native
    q, k, v, table, lens = case["tensors"]
    spec = case["spec"]
    splits = -(-spec.table_width * PAGE // part_tokens)
    partials = torch.empty((spec.max_batch, spec.num_heads, splits, spec.head_dim),
                           device="cuda", dtype=torch.float32)
    lse = torch.empty((spec.max_batch, spec.num_heads, splits), device="cuda",
                      dtype=torch.float32)
    out = torch.empty((spec.max_batch, spec.num_heads, spec.head_dim), device="cuda",
                      dtype=torch.bfloat16)
    lanes = min(1 << (splits - 1).bit_length(), 32 if spec.head_dim % 128 == 0 else 16)

    def full():
        _native.partition(q, k, v, table, lens, partials, lse, spec.num_kv_heads, splits,
                          part_tokens, 16384 // spec.head_dim, spec.head_dim ** -0.5)
        _native.lse_merge(partials, lse, out, lanes)
    return full, splits


CPU_SNIPPET = r"""
import json, os, sys, time
sys.path.insert(0, {root!r})
import numpy as np
from oracle import reference as R
rng = np.random.default_rng({seed})
lens = np.array({lengths!r}, dtype=np.int32)
batch, hq, hkv, dim, budget = len(lens), {hq}, {hkv}, {dim}, {budget}
width = (max({capacity}, 1) + 255) // 256
table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
bf = lambda x: ((x.view(np.uint32).astype(np.uint64) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
k = bf(rng.normal(size=(batch * width, 256, hkv, dim)).astype(np.float32))
v = bf(rng.normal(size=k.shape).astype(np.float32))
q = bf(rng.normal(size=(batch, hq, dim)).astype(np.float32))
R.streaming_reference(q, k, v, table, lens, split=True)          # warmup
times, t_end = [], time.perf_counter() + budget
while len(times) < 5 or time.perf_counter() < t_end:
    t0 = time.perf_counter()
    R.streaming_reference(q, k, v, table, lens, split=True)
    times.append(time.perf_counter() - t0)
times.sort()
print(json.dumps(dict(us=times[len(times) // 2] * 1e6, calls=len(times))))
"""

# CPU-baseline workloads: name -> (lengths, Hq, Hkv, D, table capacity, seed).
CPU_WORKLOADS = {
    "ctx_2064": ([2064], 16, 4, 256, 2112, 20261105),
    "ctx_528": ([528], 16, 4, 256, 528, 20261105),
    "cpu_reference_b4": ([0, 1, 257, 1000], 8, 2, 128, 1000, 7),
}


def cpu_baseline(workload, threads, budget):
    """Median time of the NumPy restatement of the reference CPU path (split mode) on one
    workload, in a child process limited to ``threads`` BLAS/OpenMP threads."""
    lengths, hq, hkv, dim, capacity, seed = CPU_WORKLOADS[workload]
    env = dict(os.environ)
    env["OPENBLAS_NUM_THREADS"] = str(threads)
    env["OMP_NUM_THREADS"] = str(threads)
    code = CPU_SNIPPET.format(root=ROOT, seed=seed, lengths=list(lengths), hq=hq, hkv=hkv,
                              dim=dim, capacity=capacity, budget=budget)
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=600)
    if res.returncode:
        raise RuntimeError(res.stderr[-2000:])
    return json.loads(res.stdout.strip().splitlines()[-1])


def bandwidth_sweep(torch, seed=64, calls=20):
    """Batch 64, Hq 32, Hkv 8, D 128, lengths U[1, 32768], pages scattered over ~200 GB."""
    import numpy as np
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, 32769, size=64).tolist()
    page_bytes = PAGE * 8 * 128 * 2
    free, _ = torch.cuda.mem_get_info()
    pool_pages = int(100e9 // page_bytes)          # 100 GB of K pages + 100 GB of V pages
    if 2 * pool_pages * page_bytes > 0.9 * free:
        pool_pages = int(0.4 * free // page_bytes)
    case = matched_case(torch, 64, 32, 8, 128, 32768, lengths, seed, pool_pages=pool_pages)
    us = graph_time_us(torch, case["full"], calls, unroll=4, warmup=2)
    part_us = graph_time_us(torch, case["partition"], calls, unroll=4, warmup=1)
    nbytes = algorithmic_bytes(lengths, 64, 32, 8, 128)
    result = dict(workload="bandwidth sweep B=64 Hq=32 Hkv=8 D=128 len~U[1,32768]",
                  pool_gb=round(2 * pool_pages * page_bytes / 1e9, 1),
                  plan=f"{case['plan'].splits}x{case['plan'].tokens_per_split}",
                  algorithmic_bytes=nbytes, us_per_call=round(us, 2),
                  tbps=round(nbytes / us / 1e6, 3), pct_peak=round(100 * nbytes / us / 1e6 / PEAK_TBPS, 1),
                  partition_us=round(part_us, 2),
                  partition_tbps=round(algorithmic_bytes(lengths, 64, 32, 8, 128, False) / part_us / 1e6, 3))
    del case
    torch.cuda.empty_cache()
    return result


def context_sweep(torch, contexts=(8192, 16384, 32768, 49152, 65536, 131072)):
    """D256 GQA 4:1 (Hq 16, Hkv 4), B=1 at longer contexts, planner plan.  The KV of one
    call (33.6 MB at 8192 tokens, 537 MB at 131072) stays partly in the 256 MB last-level
    cache across replays up to about 65536 tokens; ``hbm_*`` gives the same call with its
    tables cycling over page sets of at least 1 GB in total, so that it reads HBM."""
    out = {}
    for ctx in contexts:
        case = matched_case(torch, 1, 16, 4, 256, ctx, [ctx], 11)
        # 128 unrolled calls per graph, as for the headline: a graph replay carries a
        # launch cost of its own that a short unroll would spread over too few calls.
        us = graph_time_us(torch, case["full"], 256, unroll=128)
        fused_us = graph_time_us(torch, case["fused"], 256, unroll=128)
        part_us = graph_time_us(torch, case["partition"], 256, unroll=128)
        nbytes = algorithmic_bytes([ctx], 1, 16, 4, 256)
        pbytes = algorithmic_bytes([ctx], 1, 16, 4, 256, with_output=False)
        p = case["plan"]
        kv_bytes = 2 * ctx * 4 * 256 * 2
        hbm_us, copies, _ = hbm_resident_rate(torch, case, copies=max(2, -(-1_070_000_000 // kv_bytes)))
        out[f"ctx_{ctx}"] = {"plan": f"{p.splits}x{p.tokens_per_split}",
                             "us_per_call": round(us, 2), "tbps": round(nbytes / us / 1e6, 3),
                             "pct_peak": round(100 * nbytes / us / 1e6 / PEAK_TBPS, 1),
                             "fused_us_per_call": round(fused_us, 2),
                             "fused_pct_peak": round(100 * nbytes / fused_us / 1e6 / PEAK_TBPS, 1),
                             "partition_us": round(part_us, 2),
                             "partition_pct_peak": round(100 * pbytes / part_us / 1e6 / PEAK_TBPS, 1),
                             "hbm_us_per_call": round(hbm_us, 2),
                             "hbm_pct_peak": round(100 * nbytes / hbm_us / 1e6 / PEAK_TBPS, 1),
                             "hbm_page_sets": copies}
        del case
        torch.cuda.empty_cache()
    return out


def paged_backend_rates(torch, seed=64):
    """paged_decode backends hip_base (the whole context per sequence and kv head) and
    hip_splitk (fixed 1024-token partitions + m/l/acc merge) on the bandwidth-sweep
    shape and on the edge-coverage shapes (B=128, a quarter of the lengths 0, the rest
    U[1,4096]).  Both run one workgroup per kv head for its whole GQA group (16-head
    slices above 16), so K/V is read once per kv head, as the algorithmic bytes count."""
    import numpy as np
    from paged_decode.runtime import allocate_resources, paged_decode
    from paged_decode.spec import DecodeSpec
    out = {}
    rng = np.random.default_rng(seed)
    c3 = rng.integers(1, 32769, size=64).tolist()
    rng4 = np.random.default_rng(4)
    c4 = [0 if i % 4 == 0 else int(x) for i, x in enumerate(rng4.integers(1, 4097, size=128))]
    shapes = [("bandwidth sweep B=64 Hq=32 Hkv=8 D=128", 64, 32, 8, 128, 32768, c3,
               int(100e9 // (PAGE * 8 * 128 * 2))),
              ("edge coverage B=128 D=64 MHA 16/16", 128, 16, 16, 64, 4096, c4, None),
              ("edge coverage B=128 D=256 GQA 32/4", 128, 32, 4, 256, 4096, c4, None)]
    for name, batch, hq, hkv, dim, cap, lengths, pool in shapes:
        q, k, v, table, lens = make_inputs(torch, batch, hq, hkv, dim, cap, lengths, seed, pool)
        spec = DecodeSpec(batch, hq, hkv, dim, cap)
        nbytes = algorithmic_bytes(lengths, batch, hq, hkv, dim)
        row = {}
        for backend in ("hip_base", "hip_splitk"):
            res = allocate_resources(spec, "cuda", backend)
            fn = lambda: paged_decode(q, k, v, table, lens, resources=res, backend=backend)
            calls = 8 if pool else 64
            us = graph_time_us(torch, fn, calls, unroll=4 if pool else 16, warmup=2)
            row[backend] = {"us_per_call": round(us, 2), "tbps": round(nbytes / us / 1e6, 3),
                            "pct_peak": round(100 * nbytes / us / 1e6 / PEAK_TBPS, 1)}
            del res
        out[name] = row
        del q, k, v, table, lens
        torch.cuda.empty_cache()
    return out


SMALL_BATCH_SHAPES = (
    # name, Hq, Hkv, D, table capacity, context of every sequence
    ("D256 GQA 16/4 ctx 2064", 16, 4, 256, 2112, 2064),
    ("D128 GQA 32/8 ctx 4096", 32, 8, 128, 4096, 4096),
)


def small_batch_backends(torch, batches=(1, 8), seed=20261105):
    """paged_decode hip_base / hip_splitk and matched_decode at small batch: B sequences of
    one context each, on the headline shape (Hq 16, Hkv 4, D 256, ctx 2064) and a D128
    shape (Hq 32, Hkv 8, ctx 4096); hot cache, 128-call graphs."""
    from paged_decode.matched_splitkv import allocate_matched_resources, matched_decode
    from paged_decode.runtime import allocate_resources, paged_decode
    from paged_decode.spec import DecodeSpec
    out = {}
    for name, hq, hkv, dim, cap, ctx in SMALL_BATCH_SHAPES:
        for batch in batches:
            lengths = [ctx] * batch
            q, k, v, table, lens = make_inputs(torch, batch, hq, hkv, dim, cap, lengths, seed)
            spec = DecodeSpec(batch, hq, hkv, dim, cap)
            nbytes = algorithmic_bytes(lengths, batch, hq, hkv, dim)
            row = {}
            for backend in ("hip_base", "hip_splitk", "matched"):
                if backend == "matched":
                    res = allocate_matched_resources(spec, "cuda")
                    fn = lambda: matched_decode(q, k, v, table, lens, resources=res)
                else:
                    res = allocate_resources(spec, "cuda", backend)
                    fn = lambda: paged_decode(q, k, v, table, lens, resources=res,
                                              backend=backend)
                us = graph_time_us(torch, fn, 256, unroll=128)
                row[backend] = {"us_per_call": round(us, 2),
                                "pct_peak": round(100 * nbytes / us / 1e6 / PEAK_TBPS, 1)}
                del res
            out[f"{name} B={batch}"] = row
            progress(f"small batch {name} B={batch}: " + ", ".join(
                f"{b} {r['us_per_call']} us" for b, r in row.items()))
            del q, k, v, table, lens
            torch.cuda.empty_cache()
    return out


def batch_sweep_ctx2064(torch, batches=(8, 16, 32)):
    """The headline shape (Hq 16, Hkv 4, D 256) at B sequences of 2064 tokens, planner plan:
    where the call's share of peak grows with the batch (hot cache)."""
    out = {}
    for batch in batches:
        case = matched_case(torch, batch, 16, 4, 256, 2112, [2064] * batch, 20261105)
        us = graph_time_us(torch, case["full"], 256, unroll=128)
        part_us = graph_time_us(torch, case["partition"], 256, unroll=128)
        nbytes = algorithmic_bytes([2064] * batch, batch, 16, 4, 256)
        pbytes = algorithmic_bytes([2064] * batch, batch, 16, 4, 256, with_output=False)
        p = case["plan"]
        out[f"B_{batch}"] = {"plan": f"{p.splits}x{p.tokens_per_split}",
                             "us_per_call": round(us, 2),
                             "pct_peak": round(100 * nbytes / us / 1e6 / PEAK_TBPS, 1),
                             "partition_us": round(part_us, 2),
                             "partition_pct_peak": round(100 * pbytes / part_us / 1e6 / PEAK_TBPS, 1)}
        del case
        torch.cuda.empty_cache()
    return out


def kv_write_rates(torch, calls=512):
    """KV-cache page writes (pd_store_kv_pages): a 2048-token prefill chunk and one decode
    token, B=1, Hkv=2, D=256 (the end-to-end decoder's full-attention geometry)."""
    from paged_decode.kv_write import write_pages
    out = {}
    for steps in (2048, 1):
        gen = torch.Generator(device="cuda").manual_seed(steps)
        width = 2112 // PAGE + 1
        tables = torch.randperm(width, generator=gen, device="cuda").to(torch.int32).view(1, width)
        key = torch.randn((1, steps, 2, 256), generator=gen, device="cuda").to(torch.bfloat16).transpose(1, 2)
        value = torch.randn((1, steps, 2, 256), generator=gen, device="cuda").to(torch.bfloat16).transpose(1, 2)
        pages = [torch.empty((width, PAGE, 2, 256), device="cuda", dtype=torch.bfloat16) for _ in range(2)]
        positions = torch.arange(steps, device="cuda", dtype=torch.int64)
        us = graph_time_us(torch, lambda: write_pages(key, value, pages[0], pages[1], tables, positions),
                           calls, unroll=128)
        moved = 4 * steps * 2 * 256 * 2  # K and V read, K and V written
        out[f"tokens_{steps}"] = {"us_per_call": round(us, 3), "gbps": round(moved / us / 1e3, 1)}
    return out


def e2e_decoder(torch, output_tokens=64):
    """Random-init 24-layer Qwen3.5-geometry decoder (hidden 2048, full attention Hq 8 /
    Hkv 2 / D 256 every fourth layer, vocab 151936), B=1, greedy decode, one hipGraph per
    step through pd_store_kv_pages + the matched split-KV decode."""
    from paged_decode import hybrid
    model = hybrid.random_init_model(hybrid.decoder_config(), "cuda", 0)
    runner = hybrid.HybridRunner(model=model, backend="hip_matched", mode="graph",
                                 max_context=2048 + output_tokens)
    out = {"workload": "random-init decoder, 24 layers (6 full attention), hidden 2048, vocab 151936, "
                       "bf16 N(0,0.02), B=1, greedy, graph mode"}
    for plen in (512, 2048):
        gen = torch.Generator().manual_seed(plen)
        prompt = [torch.randint(0, 151936, (plen,), generator=gen).tolist()]
        res = runner.generate(prompt, output_tokens=output_tokens, timing=True)
        ms = sorted(res["decode_ms"])
        mean = sum(ms) / len(ms)
        out[f"prompt_{plen}"] = {"decode_steps": len(ms), "step_us_median": round(1000 * ms[len(ms) // 2], 1),
                                 "tokens_per_s": round(1000 / mean, 1)}
    del runner, model
    torch.cuda.empty_cache()
    return out


def committed_traffic(key):
    """HBM bytes per dispatch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)[key]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def profile_launches(torch, which, calls=50):
    """Eager launches for rocprofv3 (kernel trace / PMC counters).

    calibrate: a 256 MiB device copy (known bytes: 256 MiB read + 256 MiB
    written), used to scale FETCH_SIZE / WRITE_SIZE.  headline: partition and
    merge at the headline shape.  sweep: partition and merge of the bandwidth sweep.
    mid: partition and merge at D256 GQA 4:1, B=1, context 32768 (128 splits of 4 tiles,
    walked two per workgroup).
    long: partition and merge at D256 GQA 4:1, B=1, context 131072 (KV from HBM).
    parts: the headline shape with 1024-token partitions (3 splits, 12 workgroups).
    edge: paged_decode's hip_base and hip_splitk on the edge-coverage batches (B=128,
    a quarter of the lengths 0, the rest U[1, 4096]; D 64 MHA 16/16, D 256 GQA 32/4).
    small: paged_decode hip_base and hip_splitk at B=1 on the headline shape (the
    small-batch chunks and their m/l/acc merge).
    decoder: the 24-layer random-init decoder, prompt 512, 16 greedy decode steps as
    hipGraph replays (the kernel mix of one decode step).
    """
    import numpy as np
    src = torch.empty(128 * 1024 * 1024, dtype=torch.bfloat16, device="cuda")
    src.normal_()
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    if "headline" in which:
        case = matched_case(torch, 1, 16, 4, 256, 2112, [2064], 20261105)
        for _ in range(calls):
            case["partition"]()
            case["merge"]()
        torch.cuda.synchronize()
        del case
    if "sweep" in which:
        rng = np.random.default_rng(64)
        lengths = rng.integers(1, 32769, size=64).tolist()
        pool = int(100e9 // (PAGE * 8 * 128 * 2))
        case = matched_case(torch, 64, 32, 8, 128, 32768, lengths, 64, pool_pages=pool)
        for _ in range(3):
            case["partition"]()
            case["merge"]()
        torch.cuda.synchronize()
        del case
    if "parts" in which:
        case = matched_case(torch, 1, 16, 4, 256, 2112, [2064], 20261105)
        full, _ = fixed_partition_case(torch, case)
        for _ in range(calls):
            full()
        torch.cuda.synchronize()
        del case, full
    if "mid" in which:
        # 128 splits of 4 tiles: the partition walks two splits per workgroup.
        case = matched_case(torch, 1, 16, 4, 256, 32768, [32768], 11)
        for _ in range(calls):
            case["partition"]()
            case["merge"]()
        torch.cuda.synchronize()
        del case
    if "small" in which:
        # paged_decode at B=1 on the headline shape: one-workgroup chunks + m/l/acc merge.
        from paged_decode.runtime import allocate_resources, paged_decode
        from paged_decode.spec import DecodeSpec
        q, k, v, table, lens = make_inputs(torch, 1, 16, 4, 256, 2112, [2064], 5)
        for backend in ("hip_base", "hip_splitk"):
            res = allocate_resources(DecodeSpec(1, 16, 4, 256, 2112), "cuda", backend)
            for _ in range(calls):
                paged_decode(q, k, v, table, lens, resources=res, backend=backend)
            torch.cuda.synchronize()
            del res
        del q, k, v, table, lens
    if "long" in which:
        case = matched_case(torch, 1, 16, 4, 256, 131072, [131072], 11)
        for _ in range(10):
            case["partition"]()
            case["merge"]()
        torch.cuda.synchronize()
        del case
    if "edge" in which:
        from paged_decode.runtime import allocate_resources, paged_decode
        from paged_decode.spec import DecodeSpec
        rng4 = np.random.default_rng(4)
        c4 = [0 if i % 4 == 0 else int(x) for i, x in enumerate(rng4.integers(1, 4097, size=128))]
        for hq, hkv, dim in ((16, 16, 64), (32, 4, 256)):
            q, k, v, table, lens = make_inputs(torch, 128, hq, hkv, dim, 4096, c4, 64)
            spec = DecodeSpec(128, hq, hkv, dim, 4096)
            for backend in ("hip_base", "hip_splitk"):
                res = allocate_resources(spec, "cuda", backend)
                for _ in range(10):
                    paged_decode(q, k, v, table, lens, resources=res, backend=backend)
                torch.cuda.synchronize()
                del res
            del q, k, v, table, lens
    if "decoder" in which:
        from paged_decode import hybrid
        model = hybrid.random_init_model(hybrid.decoder_config(), "cuda", 0)
        runner = hybrid.HybridRunner(model=model, backend="hip_matched", mode="graph",
                                     max_context=512 + 16)
        gen = torch.Generator().manual_seed(512)
        runner.generate([torch.randint(0, 151936, (512,), generator=gen).tolist()],
                        output_tokens=16)
        torch.cuda.synchronize()
        del runner, model
    torch.cuda.empty_cache()
    print(json.dumps({"profiled": which}))


AB_WORKLOADS = ("headline", "partitions", "edge_d64", "edge_d256", "sweep", "shape")


def ab_variants_paged(torch, q, k, v, table, lens, spec, backend, libraries):
    """One call per variant of a paged_decode backend (hip_base: pd_base; hip_splitk:
    pd_split_decode, or pd_split_fixed + pd_ml_merge for a build without it) through this
    build ("current") or another one.  All variants share one workspace and output, so
    that they differ in the library only (the placement of a workspace alone moves these
    times by a few percent)."""
    from paged_decode import _native
    from paged_decode.runtime import allocate_resources
    scale = spec.head_dim ** -0.5
    res = allocate_resources(spec, "cuda", backend)
    calls = {}
    for name, library in libraries.items():
        if backend == "hip_base":
            def call(library=library):
                _native.base(q, k, v, table, lens, res.out, spec.num_kv_heads, scale,
                             library=library)
        elif hasattr(library or _native.lib(), "pd_split_decode"):
            def call(library=library):
                _native.split_decode(q, k, v, table, lens, res.maxima, res.denoms, res.accums,
                                     res.out, spec.num_kv_heads, spec.partitions, 1024, scale,
                                     library=library)
        else:
            def call(library=library):
                _native.split_fixed(q, k, v, table, lens, res.maxima, res.denoms, res.accums,
                                    spec.num_kv_heads, spec.partitions, 1024, scale,
                                    library=library)
                _native.ml_merge(res.maxima, res.denoms, res.accums, res.out, spec.max_batch,
                                 library=library)
        calls[name] = call
    return calls, {name: res.out for name in libraries}


def ab_variants_matched(torch, q, k, v, table, lens, spec, splits, part, lanes, libraries,
                        workspace=None):
    """The matched partition + LSE merge with a fixed plan (splits x part tokens) through
    this build or another one; all variants share one workspace (partials, lse, out)."""
    from paged_decode import _native
    scale = spec.head_dim ** -0.5
    if workspace is None:
        shape = (spec.max_batch, spec.num_heads, splits)
        workspace = (torch.empty(shape + (spec.head_dim,), device="cuda"),
                     torch.empty(shape, device="cuda"),
                     torch.empty((spec.max_batch, spec.num_heads, spec.head_dim), device="cuda",
                                 dtype=torch.bfloat16))
    partials, lse, out = workspace
    calls = {}
    for name, library in libraries.items():
        def call(library=library):
            _native.partition(q, k, v, table, lens, partials, lse, spec.num_kv_heads, splits,
                              part, 16384 // spec.head_dim, scale, library=library)
            _native.lse_merge(partials, lse, out, lanes, library=library)

        def decode():
            # pd_matched_decode without counters: one launch for a plan of one split
            _native.matched_decode(q, k, v, table, lens, partials, lse, None, out,
                                   spec.num_kv_heads, splits, part, 16384 // spec.head_dim,
                                   scale)
        calls[name] = decode if name == "decode" else call
    return calls, {name: out for name in libraries}


def ab_report(torch, args):
    """Paired A/B report (paged_decode.evidence) of variants of one workload: each is timed
    as graphs of two unroll counts over shuffled rounds; ratios are per round against the
    first variant, and the outputs of every variant are compared bit for bit with the
    first one's.

    Workloads (--ab-workload):
    * headline: the matched decode, B=--ab-batch, Hq 16 / Hkv 4 / D 256, --ctx tokens,
      planner plan; variants two_launch, fused, noalloc, partition, merge (through
      matched_decode), current or NAME=PATH (pd_partition + pd_lse_merge through this
      or another build of libpaged_decode.so);
    * partitions: the same matched decode with --ab-partition-token splits (the
      reference's 1024 by default);
    * edge_d64 / edge_d256: the edge-coverage batches (B=128, a quarter of the lengths 0,
      the rest U[1, 4096]; D 64 MHA 16/16, D 256 GQA 32/4) through --ab-backend
      (hip_base or hip_splitk);
    * sweep: the bandwidth-sweep batch (B=64, Hq 32 / Hkv 8 / D 128, lengths U[1, 32768],
      pages over a 200 GB pool) through --ab-backend;
    * shape: the matched decode of --ab-shape B,Hq,Hkv,D,ctx (B sequences of ctx tokens),
      planner plan.
    Outside headline the variants are current (this build) or NAME=PATH, and for shape and
    partitions also decode (pd_matched_decode without counters, this build: the
    partition alone for a plan of one split).  Every variant
    of a report uses the same workspace and output buffers (the placement of a workspace
    alone moves these times by a few percent), and each variant's output is copied right
    after its own call for the bit-for-bit comparison."""
    import numpy as np
    from paged_decode import _native, evidence
    from paged_decode.matched_splitkv import matched_decode
    from paged_decode.spec import DecodeSpec
    workload, ctx, batch = args.ab_workload, args.ctx, args.ab_batch
    items = args.ab.split(",")
    libraries = {}
    for item in items:
        if "=" in item:
            name, path = item.split("=", 1)
            libraries[name] = _native.load_library(os.path.abspath(path))
    unrolls, replays = (32, 128), 20
    if workload == "headline":
        case = matched_case(torch, batch, 16, 4, 256, max(2112, ctx), [ctx] * batch, 20261105)
        q, k, v, table, lens = case["tensors"]
        res, plan, scale = case["res"], case["plan"], 256 ** -0.5
        known = {"two_launch": case["full"], "fused": case["fused"],
                 "partition": case["partition"], "merge": case["merge"],
                 "noalloc": lambda: _native.matched_decode_noalloc(
                     q, k, v, table, lens, res.out, 4, plan.splits, plan.tokens_per_split,
                     plan.tile_tokens, scale)}
        # "current" and NAME=PATH variants run the same calls on the same workspace as
        # two_launch, so that they differ in the library only.
        others = dict(libraries, current=None) if "current" in items else libraries
        other, outputs = ab_variants_matched(torch, q, k, v, table, lens, case["spec"],
                                             plan.splits, plan.tokens_per_split,
                                             plan.lse_lanes, others,
                                             workspace=(res.partials, res.lse, res.out))
        variants = {}
        for item in items:
            name = item.split("=", 1)[0]
            if name in others:
                variants[name] = other[name]
            elif item in known:
                variants[item] = known[item]
            else:
                raise SystemExit(f"unknown A/B variant {item!r}; known: {sorted(known)} or "
                                 "NAME=PATH")
        # partition / merge alone leave no output of their own to compare
        outputs = {n: outputs[n] if n in others else
                   (res.out if n in ("two_launch", "fused", "noalloc") else None)
                   for n in variants}
        label = (f"matched decode B={batch} Hq=16 Hkv=4 D=256 ctx {ctx}, plan "
                 f"{plan.splits}x{plan.tokens_per_split}")
    else:
        for item in items:
            if "=" not in item and item not in ("current", "decode"):
                raise SystemExit(f"unknown A/B variant {item!r} for workload {workload}: "
                                 "current, decode (shape and partitions) or NAME=PATH")
            if item == "decode" and workload not in ("shape", "partitions"):
                raise SystemExit("the decode variant is for the shape and partitions workloads")
        libraries = {item.split("=", 1)[0]: libraries.get(item.split("=", 1)[0])
                     for item in items}
        unrolls, replays = (4, 16), 5
        if workload == "shape":
            # --ab-shape B,Hq,Hkv,D,ctx: B sequences of ctx tokens (capacity ctx), planner plan.
            b, hq, hkv, dim, cap = (int(x) for x in args.ab_shape.split(","))
            from paged_decode.splitkv_plan import make_splitkv_plan
            spec = DecodeSpec(b, hq, hkv, dim, cap)
            plan = make_splitkv_plan(spec, torch.cuda.get_device_properties(0)
                                     .multi_processor_count)
            q, k, v, table, lens = make_inputs(torch, b, hq, hkv, dim, cap, [cap] * b, 7)
            variants, outputs = ab_variants_matched(torch, q, k, v, table, lens, spec,
                                                    plan.splits, plan.tokens_per_split,
                                                    plan.lse_lanes, libraries)
            unrolls, replays = (32, 128), 10
            label = (f"matched decode B={b} Hq={hq} Hkv={hkv} D={dim} ctx {cap}, plan "
                     f"{plan.splits}x{plan.tokens_per_split}")
        elif workload == "partitions":
            part = args.ab_partition
            cap = max(2112, ctx)
            spec = DecodeSpec(batch, 16, 4, 256, cap)
            q, k, v, table, lens = make_inputs(torch, batch, 16, 4, 256, cap, [ctx] * batch,
                                               20261105)
            splits = -(-spec.table_width * PAGE // part)
            lanes = min(1 << (splits - 1).bit_length(), 32)
            variants, outputs = ab_variants_matched(torch, q, k, v, table, lens, spec, splits,
                                                    part, lanes, libraries)
            label = (f"matched partition + merge B={batch} Hq=16 Hkv=4 D=256 ctx {ctx}, "
                     f"{splits} partitions of {part} tokens")
        else:
            if workload == "sweep":
                lengths = np.random.default_rng(64).integers(1, 32769, size=64).tolist()
                geometry = (64, 32, 8, 128, 32768)
                pool = int(100e9 // (PAGE * 8 * 128 * 2))
            else:
                rng4 = np.random.default_rng(4)
                lengths = [0 if i % 4 == 0 else int(x)
                           for i, x in enumerate(rng4.integers(1, 4097, size=128))]
                geometry = (128, 16, 16, 64, 4096) if workload == "edge_d64" else \
                    (128, 32, 4, 256, 4096)
                pool = None
            b, hq, hkv, dim, cap = geometry
            q, k, v, table, lens = make_inputs(torch, b, hq, hkv, dim, cap, lengths, 64, pool)
            spec = DecodeSpec(b, hq, hkv, dim, cap)
            if args.ab_backend == "matched":
                from paged_decode.splitkv_plan import make_splitkv_plan
                plan = make_splitkv_plan(spec, torch.cuda.get_device_properties(0)
                                         .multi_processor_count)
                variants, outputs = ab_variants_matched(
                    torch, q, k, v, table, lens, spec, plan.splits, plan.tokens_per_split,
                    plan.lse_lanes, libraries)
            else:
                variants, outputs = ab_variants_paged(torch, q, k, v, table, lens, spec,
                                                      args.ab_backend, libraries)
            label = (f"{args.ab_backend} B={b} Hq={hq} Hkv={hkv} D={dim}, {workload} lengths")
    names = list(variants)
    # Each variant once, its output copied right away (variants may share a buffer).
    identical, first = {}, None
    for n in names:
        variants[n]()
        torch.cuda.synchronize()
        out = None if outputs[n] is None else outputs[n].clone()
        if n == names[0]:
            first = out
        identical[n] = (None if out is None or first is None else
                        bool(torch.equal(out.view(torch.int16), first.view(torch.int16))))
    rows = evidence.paired_timings(torch, variants, rounds=args.ab_rounds, replays=replays,
                                   unrolls=unrolls)
    report = evidence.paired_report(rows, names, names[0], args.ab_rounds, unrolls=unrolls)
    report.update(workload=label, outputs_identical_to_first=identical, rows=rows,
                  environment=benchmark_protocol_fingerprint(torch))
    if args.ab_out:
        evidence.write_json_exclusive(args.ab_out, report)
    top = str(max(unrolls))
    for name, x in report["variants"].items():
        t = x["us_per_call"][top]
        r = x["over_baseline"]
        progress(f"{name}: {t['median']:.3f} us/call (rounds {t['min']:.3f}-{t['max']:.3f}), "
                 f"x{r['median']:.4f} of {names[0]} ({r['min']:.4f}-{r['max']:.4f}), "
                 f"t{min(unrolls)}/t{top}-1 = {x['unroll_relative_delta']:+.4f}, "
                 f"output identical: {identical[name]}")
    print(json.dumps({k: v for k, v in report.items() if k != "rows"}))


# Extra measurements that --section runs on their own.
SECTIONS = {
    "small_batch": small_batch_backends,
    "batch_sweep": batch_sweep_ctx2064,
    "context_sweep": context_sweep,
    "bandwidth_sweep": bandwidth_sweep,
    "paged_backends": paged_backend_rates,
    "kv_write": kv_write_rates,
    "e2e_decoder": e2e_decoder,
}


def benchmark_protocol_fingerprint(torch):
    from paged_decode import benchmark_protocol
    return benchmark_protocol.fingerprint(torch)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2560)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--ctx", type=int, default=2064)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-sweep", action="store_true", help="skip the extra measurements")
    ap.add_argument("--cpu-budget", type=float, default=6.0, help="seconds per CPU run")
    ap.add_argument("--profile", default=None,
                    metavar="headline,sweep,mid,long,parts,edge,small,decoder",
                    help="only make eager launches for rocprofv3 (calibration copy + cases)")
    ap.add_argument("--require-idle-gpu", action="store_true",
                    help="refuse to run (before any GPU work) if amd-smi lists other processes")
    ap.add_argument("--ab", default=None, metavar="V1,V2,...",
                    help="paired A/B report instead of the benchmark: for the headline "
                         "workload two_launch, fused, noalloc, partition, merge; for the others "
                         "current; for all NAME=PATH (the call through another build of "
                         "libpaged_decode.so)")
    ap.add_argument("--ab-rounds", type=int, default=5)
    ap.add_argument("--ab-batch", type=int, default=1,
                    help="sequences of the A/B workload (each of --ctx tokens)")
    ap.add_argument("--ab-out", default=None, help="also write the report to this new JSON file")
    ap.add_argument("--ab-workload", default="headline", choices=AB_WORKLOADS,
                    help="workload of the A/B report (see ab_report)")
    ap.add_argument("--ab-backend", default="hip_base",
                    choices=("hip_base", "hip_splitk", "matched"),
                    help="backend of the edge_d64 / edge_d256 / sweep A/B workloads")
    ap.add_argument("--ab-shape", default="8,32,8,128,4096", metavar="B,Hq,Hkv,D,ctx",
                    help="geometry of the shape A/B workload (matched decode, planner plan)")
    ap.add_argument("--ab-partition", type=int, default=1024,
                    help="partition tokens of the partitions A/B workload")
    ap.add_argument("--section", default=None, metavar="S1,S2,...",
                    help="only these extra measurements, printed as one JSON object: "
                         + ", ".join(SECTIONS))
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the operator has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)

    from paged_decode import benchmark_protocol
    if args.require_idle_gpu:
        benchmark_protocol.require_idle_gpu()
    import torch
    from paged_decode import _native
    _native.lib()
    if args.profile:
        profile_launches(torch, args.profile)
        return
    if args.ab:
        ab_report(torch, args)
        return
    if args.section:
        result = {}
        for name in args.section.split(","):
            if name not in SECTIONS:
                raise SystemExit(f"unknown section {name!r}; known: {', '.join(SECTIONS)}")
            result[name] = SECTIONS[name](torch)
            progress(f"section {name} done")
        print(json.dumps(result))
        return

    ctx, capacity = args.ctx, max(2112, args.ctx)
    case = matched_case(torch, 1, 16, 4, 256, capacity, [ctx], 20261105)
    plan = case["plan"]
    for _ in range(args.warmup):
        case["full"]()
    torch.cuda.synchronize()
    us = graph_time_us(torch, case["full"], args.steps)
    fused_us = graph_time_us(torch, case["fused"], args.steps)
    # The partition and merge alone (the roofline's launch duration): median of five
    # timings, as the reference protocol takes, so that one slow replay does not set it.
    part_us = sorted(graph_time_us(torch, case["partition"], args.steps) for _ in range(5))[2]
    merge_us = sorted(graph_time_us(torch, case["merge"], args.steps) for _ in range(5))[2]
    progress(f"headline: {us:.3f} us/call, partition {part_us:.3f}, merge {merge_us:.3f}, "
             f"fused {fused_us:.3f}")
    nbytes = algorithmic_bytes([ctx], 1, 16, 4, 256)
    part_bytes = algorithmic_bytes([ctx], 1, 16, 4, 256, with_output=False)
    tbps = nbytes / us / 1e6
    part_tbps = part_bytes / part_us / 1e6

    extra = {"us_per_call": round(us, 3), "pct_peak": round(100 * tbps / PEAK_TBPS, 2),
             "calls_timed": timed_calls(args.steps),
             "fused_single_launch_us_per_call": round(fused_us, 3),
             "partition_us": round(part_us, 3), "merge_us": round(merge_us, 3),
             "algorithmic_bytes": nbytes,
             "plan": f"{plan.splits} splits x {plan.tokens_per_split} tokens (sm_count {plan.sm_count})"}
    hbm_us, copies, pool_mb = hbm_resident_rate(torch, case)
    extra["hbm_resident"] = {
        "us_per_call": round(hbm_us, 3), "tbps": round(nbytes / hbm_us / 1e6, 3),
        "pct_peak": round(100 * nbytes / hbm_us / 1e6 / PEAK_TBPS, 2),
        "note": f"same call, tables cycling over {copies} page sets ({pool_mb:.0f} MB pool, past "
                "the 256 MB last-level cache), so the KV comes from HBM"}
    progress(f"hbm-resident: {hbm_us:.3f} us/call")
    if not args.no_sweep:
        t128, t32, delta = reference_protocol_us(torch, case["full"])
        extra["reference_protocol"] = {"us_per_call_unroll128_median5": round(t128, 3),
                                       "us_per_call_unroll32_median5": round(t32, 3),
                                       "convergence_delta": round(delta, 4)}
        fixed, splits = fixed_partition_case(torch, case)
        f_us = graph_time_us(torch, fixed, args.steps)
        extra["partition_1024_tokens"] = {"splits": splits, "us_per_call": round(f_us, 3),
                                          "tbps": round(nbytes / f_us / 1e6, 3)}
        c528 = matched_case(torch, 1, 16, 4, 256, 528, [528], 20261105)
        u528 = graph_time_us(torch, c528["full"], args.steps)
        f528 = graph_time_us(torch, c528["fused"], args.steps)
        b528 = algorithmic_bytes([528], 1, 16, 4, 256)
        extra["ctx_528"] = {"plan": f"{c528['plan'].splits}x{c528['plan'].tokens_per_split}",
                            "us_per_call": round(u528, 3), "tbps": round(b528 / u528 / 1e6, 3),
                            "fused_us_per_call": round(f528, 3)}
        del c528
        progress("reference protocol, 1024-token partitions and context 528 done")
        extra["context_sweep_d256_gqa4"] = context_sweep(torch)
        progress("context sweep: " + ", ".join(f"{k} {v['pct_peak']}%" for k, v in
                                                extra["context_sweep_d256_gqa4"].items()))
        extra["bandwidth_sweep"] = bandwidth_sweep(torch)
        progress(f"bandwidth sweep: {extra['bandwidth_sweep']['us_per_call']} us/call")
        extra["paged_decode_backends"] = paged_backend_rates(torch)
        progress("paged_decode backends done")
        extra["small_batch_backends"] = small_batch_backends(torch)
        extra["batch_sweep_ctx2064_d256_gqa4"] = batch_sweep_ctx2064(torch)
        progress("small-batch backends and the batch sweep at context 2064 done")
        extra["kv_write"] = kv_write_rates(torch)
        progress("kv write done")
        extra["e2e_decoder"] = e2e_decoder(torch)
        progress("e2e decoder done")

    cpu = None
    if not args.no_cpu:
        # The box's CPU share for one GPU is 16 threads, whatever os.cpu_count() reports.
        threads = max(1, min(16, len(os.sched_getaffinity(0))))
        one = cpu_baseline("ctx_2064", 1, args.cpu_budget)
        allc = cpu_baseline("ctx_2064", threads, args.cpu_budget)
        progress(f"cpu baseline: {one['us']:.0f} us (1 thread), {allc['us']:.0f} us (all)")
        best = min((one, 1), (allc, threads), key=lambda x: x[0]["us"])
        others = {}
        for name in ("ctx_528", "cpu_reference_b4"):
            lengths, hq, hkv, dim, _, _ = CPU_WORKLOADS[name]
            nb = algorithmic_bytes(lengths, len(lengths), hq, hkv, dim)
            row = {"workload": f"B={len(lengths)} Hq={hq} Hkv={hkv} D={dim} lengths {lengths}"}
            for label, n in (("one_thread", 1), ("all_threads", threads)):
                r = cpu_baseline(name, n, args.cpu_budget / 2)
                row[f"{label}_us_per_call"] = round(r["us"], 1)
                row[f"{label}_tbps"] = round(nb / r["us"] / 1e6, 6)
            others[name] = row
        progress("cpu baseline of context 528 and the B=4 CPU reference case done")
        cpu = {"value": round(nbytes / best[0]["us"] / 1e6, 6), "unit": "TB/s",
               "cores": best[1], "kind": "port",
               "us_per_call": round(best[0]["us"], 1),
               "one_thread_us_per_call": round(one["us"], 1),
               "all_threads_us_per_call": round(allc["us"], 1),
               "threads_all": threads,
               "host_cpus": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
               "sample": (f"NumPy restatement of the reference CPU path (streaming_reference, "
                          f"1024-token partitions, 64-token tiles, FP32) on the same B=1 Hq=16 Hkv=4 D=256 shape, "
                          f"median of {allc['calls']} calls in ~{args.cpu_budget:.0f} s"),
               "other_workloads": others}

    line = {
        "metric": "paged-decode µs/call + achieved HBM TB/s (% peak), D256 GQA ctx 2064",
        "value": round(tbps, 4), "unit": "TB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1000, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"matched split-KV decode B=1 Hq=16 Hkv=4 D=256 page=256 "
                               f"ctx {ctx} (capacity {capacity}), planner plan, hot cache "
                               "(the KV stays in the last-level cache across calls; "
                               "hbm_resident gives the same call reading HBM)",
                   "global_batch": 1, "seq_len": ctx, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "cache_resident": True,
                     "achieved": round(part_tbps * 1000, 1), "peak": PEAK_TBPS * 1000,
                     "unit": "GB/s", "frac": round(part_tbps / PEAK_TBPS, 4),
                     "traffic": committed_traffic(
                         "matched_tile_kernel<256,4> d256 gqa4 ctx2064"),
                     "traffic_source": "profiles/traffic.json (2.0 x FETCH_SIZE + WRITE_SIZE)",
                     "kernel": "matched_tile_kernel<256,4> (the partition for single-tile splits)",
                     "bytes_per_launch": part_bytes,
                     "us_per_launch": round(part_us, 3)},
        "cpu_baseline": cpu,
        **extra,
        "environment": benchmark_protocol.fingerprint(torch),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
