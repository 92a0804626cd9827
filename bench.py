"""Benchmark: STAR-KV paged decode attention on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

A step is one decode call (one layer) over the whole batch. The headline workload
is the reference metric's configuration: bf16/low-rank codes, batch 64, every
request at 8192 tokens of context, 32 heads x head_dim 128, page size 16, K ranks
per head drawn from {16, 32, 48, 64}, V rank 64, physical pages shuffled. The cache
(1.25 GB) is larger than the 256 MB Infinity Cache, so every step streams it from
HBM. `value` = algorithmic bytes per step / wall time per step (whole call: prep,
decode and merge launches). `roofline.achieved` = the same bytes / the decode
kernel's own average duration (HIP events around that launch, in a second pass of
the same steps). Each workload's warmup runs 60 ms of back-to-back calls after a
first round of 10 (--min-warmup-ms), so that the timed steps see the GPU's settled
clocks. The
3.2-bit kernel at the same shape (three rotating cache copies, 1.3 GB) and the ragged reference
configurations are reported under "extra". `cpu_baseline` times the float64 CPU
oracle on a bounded sample of the same workload on this host.

One JSON line is printed on stdout.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "star-kv-serve_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_PEAK_F16_TFLOPS = 2500.0  # dense fp16/bf16
METRIC = "decode-attn \u00b5s & HBM GB/s (% peak) at bs64\u00d78K; TPOT, tok/s at max sessions"
# HBM bytes per decode-kernel launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
# scaled by the same counters on a copy of known size); written by hand from the runs.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_kernel_hbm_traffic.md")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# Untimed warmup runs at least this long (back-to-back calls). Under sustained load the
# decode kernel's duration moves for about 30 ms: from ~250 us up to ~350 us after a few
# ms, then back down, settling at ~245 us (kernel trace of 400 back-to-back calls). The
# timed steps measure the settled state.
MIN_WARMUP_MS = 60.0


def warm_up(fn, warmup):
    """At least `warmup` untimed calls fn(i), in rounds of 10, continued until the rounds
    after the first (which carries one-time costs: code loading, first-touch of memory)
    have run MIN_WARMUP_MS of back-to-back calls. Returns the number of calls."""
    import torch
    i, t0 = 0, None
    while True:
        fn(i)
        i += 1
        if i % 10:
            continue
        torch.cuda.synchronize()
        now = time.perf_counter()
        if t0 is None:
            t0 = now
        elif i >= warmup and (now - t0) * 1e3 >= MIN_WARMUP_MS:
            return i


def time_steps(fn, steps, warmup):
    """Warmup, then `steps` timed calls bracketed by synchronizes (ms per step, the
    whole call), then `steps` more calls with HIP events around each decode launch
    (decode-kernel ms per call). The events sit in a pass of their own: each record
    holds the stream for a few microseconds, which would count in the whole-call time."""
    import torch
    from starkv_serve import _hip
    warm_up(fn, warmup)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    _hip.profile_begin(steps)
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    kern_ms, calls = _hip.profile_end()
    return ms, kern_ms / max(calls, 1)


def bench_lowrank(lengths, steps, warmup, seed, v_rank=64):
    import torch
    from starkv_serve import workloads as W
    from starkv_serve.kernels.paged_decode import paged_starkv_decode
    dev = torch.device("cuda", 0)
    wl = W.make_lowrank(lengths, num_heads=32, v_rank=v_rank, seed=seed, gen_device=dev).to(dev)
    args = wl.decode_args()
    ms, kern = time_steps(lambda i: paged_starkv_decode(*args), steps, warmup)
    return wl, ms, kern


def bench_quant(lengths, steps, warmup, seed, copies, v_rank=64):
    import torch
    from starkv_serve import workloads as W
    from starkv_serve.kernels.paged_quant import paged_quant_decode
    dev = torch.device("cuda", 0)
    wl = W.make_quant(lengths, num_heads=32, v_rank=v_rank, seed=seed, device=dev, gen_device=dev)
    wl.k_codes = wl.v_codes = None
    torch.cuda.empty_cache()
    caches = [wl.kv_cache] + [wl.kv_cache.clone() for _ in range(copies - 1)]
    base = list(wl.decode_args())

    def step(i):
        base[1] = caches[i % len(caches)]
        return paged_quant_decode(*base)

    ms, kern = time_steps(step, steps, warmup)
    return wl, ms, kern


def bench_stock(n, context, steps, warmup, num_heads=32):
    """Uncompressed bf16 decode attention at the same shape, as the comparator for
    "stock" attention: torch's fused SDPA (flash or memory-efficient kernels only,
    never the unfused math path) over contiguous K/V [n, H, context, 128]. Stock
    paged attention reads the same K/V bytes through a block table, so this
    contiguous read is the more favourable case for the comparator."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(n, num_heads, 1, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(n, num_heads, context, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(n, num_heads, context, 128, generator=g, device="cuda").to(torch.bfloat16)
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            fn = lambda: F.scaled_dot_product_attention(q, k, v)
            warm_up(lambda i: fn(), warmup)
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(steps):
                fn()
            stop.record()
            torch.cuda.synchronize()
    except RuntimeError as e:  # no fused kernel for this shape/device
        return dict(error=str(e)[:200])
    ms = start.elapsed_time(stop) / steps
    b = 2 * k.numel() * 2 + 2 * q.numel() * 2
    return dict(us_per_step=round(ms * 1e3, 2), GBps=round(b / (ms * 1e-3) / 1e9, 1),
                hbm_frac=round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), bytes_per_step=int(b),
                kernel="torch SDPA (flash / memory-efficient), contiguous bf16 K/V, no paging")


def bench_write(n, quant, steps, warmup, seed=1004, layers=24, hidden=4096, num_heads=32, v_rank=64):
    """One layer step of the cache write for n tokens: the fused write_kv (kv_down GEMM +
    scatter / 3.2-bit pack) against the unfused sequence (F.linear, then the scatter or
    pack_kv), rotating over `layers` kv_down matrices (264 MB: more than the Infinity
    Cache, as a model's layers are). Algorithmic bytes per step: kv_down + hidden read,
    the rows written, the slots."""
    import torch
    import torch.nn.functional as F
    from starkv_serve import workloads as W
    from starkv_serve.kernels.kv_write import write_codes, write_kv
    from starkv_serve.kernels.paged_quant import QuantRow, k_tables, pack_kv
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(seed)
    ranks = [W.RANK_CHOICES[i] for i in torch.randint(0, len(W.RANK_CHOICES), (num_heads,), generator=g).tolist()]
    k_width = sum(ranks)  # every rank a multiple of 16
    width = k_width + v_rank
    offsets = torch.tensor([sum(ranks[:h]) for h in range(num_heads)], dtype=torch.int32, device=dev)
    k_ranks = torch.tensor(ranks, dtype=torch.int32, device=dev)
    kv_down = [(torch.randn(width, hidden, device=dev) * hidden ** -0.5).to(torch.bfloat16) for _ in range(layers)]
    x = torch.randn(n, hidden, device=dev).to(torch.bfloat16)
    nb = 4096
    slots = (torch.randperm(nb * 16, device=dev)[:n]).to(torch.int64)
    if quant:
        row = QuantRow(k_width, num_heads, v_rank)
        nouts, _, _ = k_tables(ranks, dev)
        cache = torch.zeros(nb, 16, row.nbytes, dtype=torch.uint8, device=dev)
        row_bytes = row.nbytes
        fused = lambda i: write_kv(x, kv_down[i % layers], cache, slots, k_width, row=row, k_ranks=k_ranks,
                                   k_offsets=offsets, k_nouts=nouts)

        def unfused(i):
            c = F.linear(x, kv_down[i % layers])
            pack_kv(c[:, :k_width], c[:, k_width:], cache, slots, row, k_ranks, offsets, nouts)
    else:
        cache = torch.zeros(nb, 16, width, dtype=torch.bfloat16, device=dev)
        row_bytes = 2 * width
        fused = lambda i: write_kv(x, kv_down[i % layers], cache, slots, k_width)

        def unfused(i):
            c = F.linear(x, kv_down[i % layers])
            write_codes(c[:, :k_width], c[:, k_width:], cache, slots)

    def timed(fn):
        warm_up(fn, warmup)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(steps):
            fn(i)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps * 1e3

    fu, un = timed(fused), timed(unfused)
    by = width * hidden * 2 + n * hidden * 2 + n * row_bytes + n * 8
    return dict(tokens=n, cache="3.2-bit" if quant else "bf16", hidden=hidden, k_width=k_width, v_rank=v_rank,
                fused_us=round(fu, 2), unfused_us=round(un, 2), bytes_per_step=by,
                GBps=round(by / (fu * 1e-6) / 1e9, 1), hbm_frac=round(by / (fu * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))


def measured_traffic(key):
    """HBM bytes per launch for `key` from the committed counter summary, or None."""
    import re
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^%s_hbm_bytes_per_launch:\s*([0-9]+)\s*$" % re.escape(key), text, re.M)
    return int(m.group(1)) if m else None


def copy_probe(gib, reps):
    """A plain device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    n = int(gib * (1 << 30))
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "reps": reps}), flush=True)


def summarize(wl, ms, kern):
    b = wl.bytes_per_step()
    f = wl.flops_per_step()
    return dict(us_per_step=round(ms * 1e3, 2), decode_kernel_us=round(kern * 1e3, 2),
                GBps=round(b / (ms * 1e-3) / 1e9, 1), kernel_GBps=round(b / (kern * 1e-3) / 1e9, 1),
                hbm_frac=round(b / (kern * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                mfma_frac=round(f / (kern * 1e-3) / 1e12 / MFMA_PEAK_F16_TFLOPS, 4),
                bytes_per_step=int(b), flops_per_step=int(f), tokens=wl.tokens, k_width=wl.k_width,
                v_rank=wl.v_rank)


def cpu_baseline(wl, budget_s=12.0):
    """The float64 oracle (numpy) on whole requests of the workload until ~budget_s."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_info

    from oracle import ref
    cores = len(os.sched_getaffinity(0))
    blas = [i.get("num_threads") for i in threadpool_info() if i.get("user_api") == "blas"]
    q = wl.query.float().cpu().numpy()
    bt = wl.block_table.cpu().numpy()
    U = wl.k_up.float().cpu().numpy()
    vq = wl.v_up_by_q.float().cpu().numpy()
    cs = wl.cos_sin_cache.float().cpu().numpy()
    row_bytes = (wl.k_width + wl.v_rank) * wl.kv_cache.element_size()
    done_tokens, done_bytes, t_total, reqs = 0, 0, 0.0, 0
    for b in range(wl.n):
        L = int(wl.lengths[b])
        pages = (L + 15) // 16
        blocks = torch.from_numpy(bt[b, :pages]).long().to(wl.kv_cache.device)
        rows = wl.kv_cache[blocks].float().cpu().numpy()         # [pages, 16, width] of this request
        local_bt = np.arange(pages, dtype=np.int32)[None, :]
        t0 = time.perf_counter()
        ref.lowrank_decode(q[b:b + 1], rows, local_bt, [L], wl.max_seq_len, U, wl.ranks,
                           wl.k_head_offsets.tolist(), wl.k_width, vq, cs, wl.scale)
        t_total += time.perf_counter() - t0
        done_tokens += L
        done_bytes += L * row_bytes
        reqs += 1
        if t_total >= budget_s:
            break
    return dict(value=round(done_bytes / t_total / 1e9, 3), unit="GB/s", cores=blas[0] if blas else cores,
                kind="port",
                sample=f"float64 numpy oracle (oracle/ref.py lowrank_decode) on {reqs} of the {wl.n} requests "
                       f"({done_tokens} tokens, {t_total:.1f} s), GB/s of cache rows attended; "
                       f"host affinity {cores} cores")


def main():
    global MIN_WARMUP_MS
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--min-warmup-ms", type=float, default=MIN_WARMUP_MS,
                    help="each workload's warmup continues until this many ms of back-to-back calls")
    ap.add_argument("--no-extra", action="store_true", help="skip the 3.2-bit and ragged configurations")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["bf16", "quant", "write", "short"], default=None,
                    help="profile runs: time one workload only (bs64 x 8192; short: 64 requests x 16 "
                         "tokens, bf16) and print its summary")
    ap.add_argument("--copy-probe", type=float, default=0.0, metavar="GIB",
                    help="profile runs: only copy GIB GiB device to device 5 times (counter scaling)")
    args = ap.parse_args()
    MIN_WARMUP_MS = args.min_warmup_ms
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (decode shards by request; "
              "each GPU would run this same kernel on its own requests). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    torch.cuda.set_device(0)
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.copy_probe > 0:
        copy_probe(args.copy_probe, 5)
        return

    lengths = [8192] * 64
    if args.only == "write":
        for n_tok in (16, 64):
            for quant in (True, False):
                print(json.dumps(bench_write(n_tok, quant, args.steps, args.warmup)), flush=True)
        return
    if args.only == "short":
        ws_, mss, ks = bench_lowrank([16] * 64, args.steps, args.warmup, seed=1005)
        print(json.dumps(summarize(ws_, mss, ks)), flush=True)
        return
    if args.only == "quant":
        wq, msq, kq = bench_quant(lengths, args.steps, args.warmup, seed=1003, copies=3)
        print(json.dumps(summarize(wq, msq, kq)), flush=True)
        return
    log("headline: bf16 low-rank, 64 x 8192")
    wl, ms, kern = bench_lowrank(lengths, args.steps, args.warmup, seed=1001)
    head = summarize(wl, ms, kern)
    log(json.dumps(head))
    if args.only == "bf16":
        print(json.dumps(head), flush=True)
        return

    extra = {}
    if not args.no_extra:
        from starkv_serve import workloads as W
        log("3.2-bit, 64 x 8192 (3 rotating caches)")
        wq, msq, kq = bench_quant(lengths, args.steps, args.warmup, seed=1003, copies=3)
        extra["quant_bs64x8k"] = summarize(wq, msq, kq)
        extra["quant_bs64x8k"]["hbm_traffic_bytes"] = measured_traffic("quant_bs64x8k")
        log(json.dumps(extra["quant_bs64x8k"]))
        del wq
        torch.cuda.empty_cache()
        log("bf16 low-rank, 64 requests, lengths U[1024, 8192]")
        w1, ms1, k1 = bench_lowrank(W.ragged_lengths(1001), args.steps, args.warmup, seed=1001)
        extra["lowrank_bs64_ragged_1k_8k"] = summarize(w1, ms1, k1)
        log(json.dumps(extra["lowrank_bs64_ragged_1k_8k"]))
        del w1
        torch.cuda.empty_cache()
        log("3.2-bit, 64 requests, lengths U[1024, 8192] (3 rotating caches)")
        w2, ms2, k2 = bench_quant(W.ragged_lengths(1002), args.steps, args.warmup, seed=1002, copies=3)
        extra["quant_bs64_ragged_1k_8k"] = summarize(w2, ms2, k2)
        log(json.dumps(extra["quant_bs64_ragged_1k_8k"]))
        del w2
        torch.cuda.empty_cache()
        for n_tok in (16, 64):
            for quant in (True, False):
                key = f"write_{'quant' if quant else 'bf16'}_n{n_tok}"
                log(f"cache write, {n_tok} tokens, {'3.2-bit' if quant else 'bf16'} (fused vs unfused)")
                extra[key] = bench_write(n_tok, quant, args.steps, args.warmup)
                log(json.dumps(extra[key]))
        torch.cuda.empty_cache()
        log("uncompressed bf16 attention (torch fused SDPA), 64 x 8192")
        stock = bench_stock(64, 8192, args.steps, args.warmup)
        if "us_per_step" in stock:
            stock["starkv_bf16_speedup"] = round(stock["us_per_step"] / head["us_per_step"], 2)
            stock["starkv_quant_speedup"] = round(stock["us_per_step"] / extra["quant_bs64x8k"]["us_per_step"], 2)
        extra["stock_bf16_sdpa_bs64x8k"] = stock
        log(json.dumps(stock))
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(wl)
        log(json.dumps(cpu))

    out = {
        "metric": METRIC,
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) codes and queries, random-init bases, shuffled pages)",
        "config": {"workload": "bf16 low-rank paged decode, one layer, batch 64 x context 8192",
                   "batch": 64, "context": 8192, "num_heads": 32, "head_dim": 128, "page_size": 16,
                   "k_width": wl.k_width, "v_rank": wl.v_rank, "k_ranks": "uniform {16,32,48,64} per head",
                   "decode_us": head["us_per_step"], "min_warmup_ms": MIN_WARMUP_MS},
        "roofline": {"bound": "hbm", "achieved": head["kernel_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["hbm_frac"], "traffic": measured_traffic("bf16_bs64x8k"),
                     "kernel": "lowrank_kernel (bf16 decode)", "kernel_us": head["decode_kernel_us"],
                     "bytes_per_launch": head["bytes_per_step"], "mfma_frac_fp16": head["mfma_frac"]},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
