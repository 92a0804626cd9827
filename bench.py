"""Benchmark: STAR-KV paged decode attention on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

A step is one decode call (one layer) over the whole batch. The headline workload is
the reference metric's configuration: bf16 low-rank codes, batch 64, every request at
8192 tokens of context, 32 heads x head_dim 128, page size 16, K ranks per head drawn
from {16, 32, 48, 64}, V rank 64, physical pages shuffled. The cache (1.25 GB) is
larger than the 256 MB Infinity Cache, so every step streams it from HBM.

Timing, per workload, after W warm-up calls continued until 60 ms of back-to-back calls
have settled the clocks (--min-warmup-ms):
  - `ms_per_step` / `value`: K calls between two synchronizations, one event pair around
    them (the whole call: prep, decode and merge launches), value = algorithmic bytes per
    step / that mean time;
  - `call_us_median`: the median over K more calls of the whole call, from event pairs
    the library records around each call;
  - `decode_kernel_us`: the median over K more calls of the decode kernels alone (the
    roofline figure: `roofline.achieved` = bytes / this time);
  - `call_us_graph`: the call captured once in a HIP graph, K replays back to back (mean;
    no host work between launches, as a serving engine runs uniform decode steps).
Extra workloads: the 3.2-bit kernel at the same shape (three rotating cache copies),
the ragged U[1024, 8192] configurations, batch 1 x 4096, 64 requests x 16 tokens, 16 x
32768 3.2-bit with the fused cache write in each step, the reference checkpoint's shape
(K width 880, V rank 1280 / 1290: the two-pass form), the fused cache write, uncompressed
attention (torch SDPA, this library's paged stock kernel, the 100 %-HBM bound) and the
Llama-2-7B-shaped model (config 4). `cpu_baseline` times the reference's math restated
in fp32 PyTorch (oracle/torch_ref.py) on this host's cores, median of 5 runs after 1.

One JSON line is printed on stdout.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "star-kv-serve_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_PEAK_F16_TFLOPS = 2500.0  # dense fp16/bf16
METRIC = "decode-attn µs & HBM GB/s (% peak) at bs64×8K; TPOT, tok/s at max sessions"
# HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
# the same counters on a copy of known size); written by hand from the runs.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_kernel_hbm_traffic.md")
# K ranks of a 0.75-ratio layer of the reference checkpoint: 880 lanes over 32 heads.
RANKS_880 = [32] * 23 + [16] * 9


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


def time_decode(fn, steps, warmup):
    """Decode calls: warmup; `steps` calls bracketed by synchronizes (mean ms per call, the
    contract figure); `steps` calls with the library's per-call events around the whole
    call (median); `steps` calls with its events around the decode kernels (median). The
    three passes are separate because each event record holds the stream a few
    microseconds."""
    import torch
    from starkv_serve import _hip
    warm_up(fn, warmup)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    stop.record()
    torch.cuda.synchronize()
    mean_ms = start.elapsed_time(stop) / steps
    out = dict(ms=mean_ms)
    for key, whole in (("call_ms", True), ("kern_ms", False)):
        _hip.profile_begin(steps, whole_call=whole)
        for i in range(steps):
            fn(i)
        torch.cuda.synchronize()
        t = _hip.profile_end()
        out[key] = statistics.median(t) if t else float("nan")
    # The same call captured once in a HIP graph and replayed `steps` times back to back
    # (how a serving engine runs uniform decode steps): no host work between the launches.
    # The replays get the same warm-up as the eager calls: the capture leaves the GPU idle,
    # and the clock transient that follows (above) would otherwise fall in the timed ones.
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn(0)
    warm_up(lambda i: g.replay(), warmup)
    start.record()
    for _ in range(steps):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    out["graph_ms"] = start.elapsed_time(stop) / steps
    del g
    return out


def time_events(fn, steps, warmup):
    """Other work (writes, stock attention, write + decode steps): warmup, then `steps`
    calls with an event pair around each; (mean, median) ms per call."""
    import torch
    warm_up(fn, warmup)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        fn(i)
        ev[i][1].record()
    torch.cuda.synchronize()
    t = [a.elapsed_time(b) for a, b in ev]
    return sum(t) / len(t), statistics.median(t)


def decode_args_fp16_cs(wl):
    """The workload's decode arguments with the cos/sin table in fp16, as
    StarKVAttentionImpl.to_device converts it once at load time."""
    from starkv_serve.kernels.paged_decode import cos_sin_for_kernel
    args = list(wl.decode_args())
    args[10] = cos_sin_for_kernel(args[10])
    return args


def bench_lowrank(lengths, steps, warmup, seed, v_rank=64, ranks=None):
    import torch
    from starkv_serve import workloads as W
    from starkv_serve.kernels.paged_decode import paged_starkv_decode
    dev = torch.device("cuda", 0)
    wl = W.make_lowrank(lengths, num_heads=32, v_rank=v_rank, ranks=ranks, seed=seed, gen_device=dev).to(dev)
    args = decode_args_fp16_cs(wl)
    return wl, time_decode(lambda i: paged_starkv_decode(*args), steps, warmup)


def bench_quant(lengths, steps, warmup, seed, copies, v_rank=64, ranks=None):
    import torch
    from starkv_serve import workloads as W
    from starkv_serve.kernels.paged_quant import paged_quant_decode
    dev = torch.device("cuda", 0)
    wl = W.make_quant(lengths, num_heads=32, v_rank=v_rank, ranks=ranks, seed=seed, device=dev, gen_device=dev)
    wl.k_codes = wl.v_codes = None
    torch.cuda.empty_cache()
    caches = [wl.kv_cache] + [wl.kv_cache.clone() for _ in range(copies - 1)]
    base = decode_args_fp16_cs(wl)

    def step(i):
        base[1] = caches[i % len(caches)]
        return paged_quant_decode(*base)

    return wl, time_decode(step, steps, warmup)


def summarize(wl, t):
    b = wl.bytes_per_step()
    f = wl.flops_per_step()
    k = t["kern_ms"]
    return dict(us_per_step=round(t["ms"] * 1e3, 2), call_us_median=round(t["call_ms"] * 1e3, 2),
                call_us_graph=round(t["graph_ms"] * 1e3, 2),
                decode_kernel_us=round(k * 1e3, 2), GBps=round(b / (t["ms"] * 1e-3) / 1e9, 1),
                kernel_GBps=round(b / (k * 1e-3) / 1e9, 1), hbm_frac=round(b / (k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                mfma_frac=round(f / (k * 1e-3) / 1e12 / MFMA_PEAK_F16_TFLOPS, 4), bytes_per_step=int(b),
                flops_per_step=int(f), tokens=wl.tokens, requests=wl.n, k_width=wl.k_width, v_rank=wl.v_rank)


def bench_c3(steps_per_pass, passes, warmup_passes=1, n_req=16, context=32768, hidden=4096, seed=3003):
    """Config 3: 16 requests at context 32768, 3.2-bit, each step writing one token per
    request through the fused write (kv_down GEMM + quantize + scatter) and then decoding
    with the lengths one longer, 32 steps per pass, max_seq_len = the context (a full
    graph's span). Median per step over the timed passes."""
    import torch
    from starkv_serve import checkpoint as ck
    from starkv_serve import workloads as W
    from starkv_serve.kernels.kv_write import write_kv
    from starkv_serve.kernels.paged_quant import paged_quant_decode
    import tempfile
    dev = torch.device("cuda", 0)
    wl = W.make_quant([context] * n_req, num_heads=32, v_rank=64, seed=seed, device=dev, gen_device=dev)
    wl.k_codes = wl.v_codes = None
    torch.cuda.empty_cache()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "fused_weights.pt")
        ck.write_fused_checkpoint(path, 1, 32, 128, hidden, {0: (wl.ranks, wl.v_rank)}, seed=seed + 1)
        w = ck.load_fused_checkpoint(path, 1, 32, 128, dtype=torch.bfloat16, kv_quant=True).layers[0]
    ops = ck.layer_operands(w, 32, dev, torch.bfloat16)
    from starkv_serve.kernels.paged_decode import cos_sin_for_kernel
    cs = cos_sin_for_kernel(wl.cos_sin_cache)
    g = torch.Generator(device=dev).manual_seed(seed + 2)
    hid = torch.randn(steps_per_pass, n_req, hidden, generator=g, device=dev).to(torch.bfloat16)
    qs = torch.randn(steps_per_pass, n_req, 32, 128, generator=g, device=dev).to(torch.bfloat16)
    rows = torch.arange(n_req, device=dev)
    slots_all, lens_all = [], []
    for st in range(steps_per_pass):
        pos = context - steps_per_pass + st
        slots_all.append(wl.block_table[rows, pos // 16].long() * 16 + pos % 16)
        lens_all.append(torch.full((n_req,), pos + 1, dtype=torch.int32, device=dev))

    def step(i):
        st = i % steps_per_pass
        # The write deferred into the decode's first launch, as the attention layer's decode step does.
        write_kv(hid[st], ops.kv_down, wl.kv_cache, slots_all[st], ops.k_width, row=ops.row, k_ranks=ops.k_ranks,
                 k_offsets=ops.k_head_offsets, k_nouts=ops.k_nouts, deferred=True)
        return paged_quant_decode(qs[st], wl.kv_cache, wl.block_table, lens_all[st], context, ops.row, ops.k_up,
                                  ops.head_of_lane, ops.k_tiles, ops.v_up_by_q, cs, wl.scale)

    mean, med = time_events(step, steps_per_pass * passes, steps_per_pass * warmup_passes)
    tok = sum(context - steps_per_pass + st + 1 for st in range(steps_per_pass)) * n_req / steps_per_pass
    dec_bytes = tok * ops.row.nbytes + n_req * 32 * 128 * 4 + ops.k_up.numel() * 2 + ops.v_up_by_q.numel() * 2
    wr_bytes = ops.kv_down.numel() * 2 + n_req * hidden * 2 + n_req * ops.row.nbytes
    b = dec_bytes + wr_bytes
    return dict(requests=n_req, context=context, steps=steps_per_pass * passes, us_per_step=round(mean * 1e3, 2),
                us_per_step_median=round(med * 1e3, 2), bytes_per_step=int(b),
                GBps=round(b / (med * 1e-3) / 1e9, 1), hbm_frac=round(b / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                k_width=ops.k_width, v_rank=ops.v_rank,
                step="fused write (16 tokens: kv_down GEMM inside the decode's first launch, quantize, scatter) "
                     "+ 3.2-bit decode, span 32768")


def bench_stock(n, context, steps, warmup, num_heads=32):
    """Uncompressed bf16 decode attention at the same shape, as the comparator for
    "stock" attention: torch's fused SDPA (flash or memory-efficient kernels only,
    never the unfused math path) over contiguous K/V [n, H, context, 128]. Stock
    paged attention reads the same K/V bytes through a block table, so this
    contiguous read is the more favourable case for the comparator. Also the bound
    of any such kernel: its K/V bytes at 100 % of HBM peak."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(n, num_heads, 1, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(n, num_heads, context, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(n, num_heads, context, 128, generator=g, device="cuda").to(torch.bfloat16)
    b = 2 * k.numel() * 2 + 2 * q.numel() * 2
    res = dict(bytes_per_step=int(b), hbm_bound_us=round(b / (HBM_PEAK_GBS * 1e9) * 1e6, 1))
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            mean, med = time_events(lambda i: F.scaled_dot_product_attention(q, k, v), steps, warmup)
    except RuntimeError as e:  # no fused kernel for this shape/device
        res["error"] = str(e)[:200]
        return res
    res.update(us_per_step=round(mean * 1e3, 2), us_per_step_median=round(med * 1e3, 2),
               GBps=round(b / (med * 1e-3) / 1e9, 1), hbm_frac=round(b / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               kernel="torch SDPA (flash / memory-efficient), contiguous bf16 K/V, no paging")
    # The same K/V through a shuffled block table, with this library's uncompressed paged
    # decode (the kernel of the full layers in the model harness).
    from starkv_serve.kernels.stock_decode import paged_decode_full
    del k, v
    torch.cuda.empty_cache()
    bs, pages = 16, context // 16
    kc = torch.randn(n * pages + 1, bs, num_heads, 128, generator=g, device="cuda", dtype=torch.bfloat16)
    vc = torch.randn(n * pages + 1, bs, num_heads, 128, generator=g, device="cuda", dtype=torch.bfloat16)
    perm = torch.randperm(n * pages, generator=torch.Generator().manual_seed(8)) + 1
    bt = perm.view(n, pages).to(torch.int32).cuda()
    seq = torch.full((n,), context, dtype=torch.int32, device="cuda")
    q3 = q[:, :, 0, :].contiguous()
    pmean, pmed = time_events(lambda i: paged_decode_full(q3, kc, vc, bt, seq, context, 128 ** -0.5), steps, warmup)
    res.update(paged_us_per_step=round(pmean * 1e3, 2), paged_us_per_step_median=round(pmed * 1e3, 2),
               paged_GBps=round(b / (pmed * 1e-3) / 1e9, 1),
               paged_hbm_frac=round(b / (pmed * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               paged_kernel="stock_decode_kernel + stock_merge_kernel, bf16 K/V [blocks, 16, 32, 128], shuffled pages")
    return res


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
        fused = lambda i: write_kv(x, kv_down[i % layers], cache, slots, k_width, row=row, k_ranks=k_ranks,  # noqa: E731
                                   k_offsets=offsets, k_nouts=nouts)

        def unfused(i):
            c = F.linear(x, kv_down[i % layers])
            pack_kv(c[:, :k_width], c[:, k_width:], cache, slots, row, k_ranks, offsets, nouts)
    else:
        cache = torch.zeros(nb, 16, width, dtype=torch.bfloat16, device=dev)
        row_bytes = 2 * width
        fused = lambda i: write_kv(x, kv_down[i % layers], cache, slots, k_width)  # noqa: E731

        def unfused(i):
            c = F.linear(x, kv_down[i % layers])
            write_codes(c[:, :k_width], c[:, k_width:], cache, slots)

    fu = time_events(fused, steps, warmup)[1] * 1e3
    un = time_events(unfused, steps, warmup)[1] * 1e3
    by = width * hidden * 2 + n * hidden * 2 + n * row_bytes + n * 8
    return dict(tokens=n, cache="3.2-bit" if quant else "bf16", hidden=hidden, k_width=k_width, v_rank=v_rank,
                fused_us_median=round(fu, 2), unfused_us_median=round(un, 2), bytes_per_step=by,
                GBps=round(by / (fu * 1e-6) / 1e9, 1), hbm_frac=round(by / (fu * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))


def bench_model(context=16384, steps=32, warm=3, seed=4000, reserve_gb=24.0, modes=("stock", "bf16", "quant"),
                max_sessions=True):
    """Config 4: decode steps of a random-init Llama-2-7B-shaped model (32 layers, 32 heads
    x 128, hidden 4096, MLP 11008, vocab 32000). STAR-KV modes keep layers 0, 1, 2 and 31
    uncompressed and compress the others at the 0.75 ratio (K ranks, multiples of 16, keep
    ~21.5 % of K; V rank, a multiple of 32, ~31.5 % of V: 880 and 1280 here), their factors
    written to a fused checkpoint and read back with load_fused_checkpoint; "stock" keeps
    every layer uncompressed. At concurrency 1 the session's cache comes from its prompt: one
    prefill_step over `context` random tokens (TTFT = its median time over 2 runs after 1;
    compressed layers write their codes and run the dense prefill, full layers write K/V and
    run causal attention), and decoding starts from the prompt's greedy next token. At the
    most sessions the caches hold `context` tokens of synthetic rows (the 3.2-bit rows
    packed from random hidden states through the write path). Each session decodes `steps`
    tokens, one token per session per step. Concurrency 1 and the most
    sessions whose caches fit in the GPU's free memory (less `reserve_gb`). Per mode and
    concurrency: TPOT (median step), tok/s = sessions / TPOT, and attention per step (the
    KV writes and attention of all 32 layers, timed on their own, as bench_serving.py:62-115
    sums them; `max_sessions` False: concurrency 1 only). Each figure twice: with each step
    (or each attention pass) replayed from one HIP graph (`tpot_ms`, `tok_per_s`,
    `attention_us_per_step`: GPU time without host launch
    gaps, the reference's attention figure being summed kernel time) and eager (`*_eager`:
    every launch from the host)."""
    import tempfile
    import torch
    from starkv_serve import checkpoint as ck
    from starkv_serve import model as M
    dev = torch.device("cuda", 0)
    shape = M.LLAMA2_7B
    g = torch.Generator().manual_seed(seed)
    full = (0, 1, 2, shape.num_layers - 1)
    comp = {li: (M.ranks_for_ratio(32, 128, 0.215, 16, g), M.v_rank_for_ratio(32, 128, 0.315, 32))
            for li in range(shape.num_layers) if li not in full}
    # Block-table rows cover every position a step writes: the context, then warm + steps tokens.
    pages = (context + warm + steps + 15) // 16
    assert context + warm + steps <= 16 * pages
    res = dict(model="Llama-2-7B shape, random init", context=context, decode_steps=steps,
               uncompressed_layers=list(full), k_width=sum(next(iter(comp.values()))[0]),
               v_rank=next(iter(comp.values()))[1])

    def run(model, n):
        model.allocate_kv_cache(n * pages + 1)
        gg = torch.Generator(device=dev).manual_seed(seed + n)
        bt = (torch.randperm(n * pages, device=dev, generator=gg) + 1).to(torch.int32).view(n, pages)
        prefill = {}
        if n == 1:  # the session's cache from its prompt
            prompt = torch.randint(0, shape.vocab_size, (context,), device=dev, generator=gg)
            pmd, ppos = M.prefill_metadata(bt, [context], 16)
            times = []
            for i in range(3):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                plog = model.prefill_step(prompt, ppos, pmd)
                b.record()
                torch.cuda.synchronize()
                times.append(a.elapsed_time(b))
            ttft = statistics.median(times[1:])
            prefill = dict(ttft_ms=round(ttft, 2), prefill_tok_per_s=round(context / ttft * 1e3, 1))
            log(f"  prefill of one {context}-token prompt: {ttft:.1f} ms")
        for li, layer in enumerate(model.layers if n > 1 else []):
            c = model.kv_caches[li]
            if not layer.compressed:
                c[0].normal_(generator=gg)
                c[1].normal_(generator=gg)
            elif layer.impl.row is None:
                c.normal_(generator=gg)
            else:  # valid 3.2-bit rows: session 0's context through the write path, copied to the others
                pc = (context + 15) // 16
                pos = torch.arange(context, device=dev)
                slots = bt[0, pos // 16].long() * 16 + pos % 16
                for a in range(0, context, 4096):
                    hid = torch.randn(min(4096, context - a), shape.hidden_size, device=dev, generator=gg)
                    layer.impl.write_from_hidden(hid.to(torch.bfloat16), c, slots[a:a + 4096])
                for sess in range(1, n):
                    c[bt[sess, :pc].long()] = c[bt[0, :pc].long()]
        tokens0 = plog.argmax(-1) if n == 1 else torch.randint(0, shape.vocab_size, (n,), device=dev, generator=gg)
        pos0 = torch.full((n,), context, device=dev, dtype=torch.long)
        torch.cuda.synchronize()

        def timed(fn, count):
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(count)]
            for a, b in ev:
                a.record()
                fn()
                b.record()
            torch.cuda.synchronize()
            return statistics.median([a.elapsed_time(b) for a, b in ev[warm:]])

        # Eager steps: every launch from the host, lengths read on the host.
        st = dict(tokens=tokens0.clone(), pos=pos0.clone())

        def eager_step():
            md = M.decode_metadata(bt, st["pos"], 16, int(context + st["t"]) + 1)
            st["tokens"] = model.decode_step(st["tokens"], st["pos"], md).argmax(-1)
            st["pos"] = st["pos"] + 1
            st["t"] += 1

        st["t"] = 0
        tpot_eager = timed(eager_step, warm + steps)
        # The same steps from one HIP graph per step (decode over the span max_model_len).
        dg = M.DecodeGraph(model, bt, tokens0, pos0)
        tpot = timed(dg.replay, warm + steps)
        del dg
        # Attention per step: the KV writes and attention of the 32 layers, in a graph of
        # their own (their GPU time without host launch gaps), and eager.
        positions = pos0 + warm + steps - 1
        md = M.decode_metadata(bt, positions, 16, int(context + warm + steps))
        hid = torch.randn(n, shape.hidden_size, device=dev, generator=gg).to(torch.bfloat16)
        ins = model.attention_inputs(hid, positions)
        attn_eager = timed(lambda: model.attention_only(hid, ins, md), warm + 5)
        ag = torch.cuda.CUDAGraph()
        with torch.cuda.graph(ag):
            model.attention_only(hid, ins, md, in_graph=True)
        attn = timed(ag.replay, warm + 5)
        del ag
        out = dict(sessions=n, cache_from="prompt prefill" if n == 1 else "synthetic rows", **prefill,
                   tpot_ms=round(tpot, 3), tok_per_s=round(n / tpot * 1e3, 1),
                   attention_us_per_step=round(attn * 1e3, 1), tpot_ms_eager=round(tpot_eager, 3),
                   tok_per_s_eager=round(n / tpot_eager * 1e3, 1), attention_us_per_step_eager=round(attn_eager * 1e3, 1),
                   kv_cache_gb=round(n * pages * 16 * model.cache_bytes_per_token() / 1e9, 2))
        model.kv_caches = []
        torch.cuda.empty_cache()
        return out

    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "fused_weights.pt")
        ck.write_fused_checkpoint(path, shape.num_layers, shape.num_kv_heads, shape.head_dim, shape.hidden_size,
                                  comp, seed=seed)
        for mode in modes:
            try:
                c = None if mode == "stock" else ck.load_fused_checkpoint(
                    path, shape.num_layers, shape.num_kv_heads, shape.head_dim, dtype=torch.bfloat16,
                    kv_quant=mode == "quant")
                model = M.StarKVLlamaForCausalLM(shape, c, max_model_len=16 * pages, device=dev,
                                                 seed=seed + 1, stock=mode == "stock")
                per_tok = model.cache_bytes_per_token()
                free, _ = torch.cuda.mem_get_info()
                n_max = max(1, int((free - reserve_gb * 1e9) // (pages * 16 * per_tok)))
                r = dict(kv_bytes_per_token=per_tok)
                for key, n in (("c1", 1), ("max_sessions", n_max))[:2 if max_sessions else 1]:
                    log(f"config 4 {mode}: {n} sessions x {context}")
                    r[key] = run(model, n)
                    log(json.dumps(r[key]))
                res[mode] = r
                del model
            except RuntimeError as e:  # e.g. out of memory: record it, keep the rest of the bench
                res[mode] = dict(error=str(e)[:300])
            torch.cuda.empty_cache()
    st = res.get("stock", {})
    for mode in ("bf16", "quant"):
        r = res.get(mode, {})
        for key in ("c1", "max_sessions"):
            if key in r and key in st:
                r[key]["tpot_speedup_vs_stock"] = round(st[key]["tpot_ms"] / r[key]["tpot_ms"], 3)
                r[key]["throughput_gain_vs_stock"] = round(r[key]["tok_per_s"] / st[key]["tok_per_s"], 3)
    return res


def bench_prefill(steps, warmup, num_heads=32):
    """Dense causal prefill attention (the attention half of the STAR-KV layer's
    prefill, attention.py:219-251): this library's prefill kernel over fp16 K / V, next
    to torch's fused SDPA (flash or memory-efficient kernels) over the same bf16 q and
    K / V per prompt. Shapes: one 16,384-token prompt (config 4's prompts) and 8 prompts
    of 2,048, 32 heads x 128. FLOPs: the causal half of QK^T and PV, 2 L (L + 1) 128 H."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from starkv_serve.kernels.prefill import prefill_attention
    res = {}
    g = torch.Generator(device="cuda").manual_seed(11)
    for name, lens in (("1x16384", [16384]), ("8x2048", [2048] * 8)):
        T = sum(lens)
        q = torch.randn(T, num_heads, 128, generator=g, device="cuda").to(torch.bfloat16)
        k = torch.randn(T, num_heads, 128, generator=g, device="cuda").to(torch.float16)
        v = torch.randn(T, num_heads, 128, generator=g, device="cuda").to(torch.float16)
        out = torch.empty_like(q)
        flops = sum(2 * L * (L + 1) * 128 * num_heads for L in lens)
        mean, med = time_events(lambda i: prefill_attention(q, k, v, lens, 128 ** -0.5, out=out), steps, warmup)
        r = dict(prompts=len(lens), tokens=T, flops=int(flops), us_median=round(med * 1e3, 1),
                 TFLOPs=round(flops / (med * 1e-3) / 1e12, 1),
                 mfma_frac=round(flops / (med * 1e-3) / 1e12 / MFMA_PEAK_F16_TFLOPS, 4))
        kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)

        def sdpa(i):
            a = 0
            for L in lens:
                qi = q[a:a + L].transpose(0, 1).unsqueeze(0)
                ki = kb[a:a + L].transpose(0, 1).unsqueeze(0)
                vi = vb[a:a + L].transpose(0, 1).unsqueeze(0)
                F.scaled_dot_product_attention(qi, ki, vi, is_causal=True)
                a += L
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                smean, smed = time_events(sdpa, steps, warmup)
            r.update(sdpa_us_median=round(smed * 1e3, 1), sdpa_TFLOPs=round(flops / (smed * 1e-3) / 1e12, 1),
                     speedup_vs_sdpa=round(smed / med, 2))
        except RuntimeError as e:
            r["sdpa_error"] = str(e)[:200]
        res[name] = r
        del q, k, v, kb, vb, out
        torch.cuda.empty_cache()
    return res


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


# ---------------------------------------------------------------------------
# CPU baseline: the reference's math in fp32 PyTorch on this host (oracle/torch_ref.py)
# ---------------------------------------------------------------------------

def _cpu_median(fn, runs=5):
    fn()  # warm-up
    t = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t0)
    return statistics.median(t)


def _cpu_subset(wl, idx):
    """The workload restricted to requests idx, on the CPU (the cache whole)."""
    from starkv_serve import workloads as W
    sub = W.Workload(**{**wl.__dict__})
    for k in ("query", "block_table", "seq_lens"):
        setattr(sub, k, getattr(wl, k)[idx].cpu())
    for k in ("kv_cache", "k_up", "v_up_by_q", "cos_sin_cache"):
        setattr(sub, k, getattr(wl, k).cpu())
    sub.lengths = [wl.lengths[i] for i in idx]
    return sub


def cpu_decode_run(wl):
    """A callable running the fp32 restatement of the workload's decode on the CPU."""
    from oracle import ref, torch_ref
    if wl.quant:
        lay = ref.row_layout(wl.k_width, len(wl.ranks), wl.v_rank)
        return lambda: torch_ref.quant_decode(wl.query, wl.kv_cache, wl.block_table, wl.seq_lens, wl.max_seq_len,
                                              lay, wl.ranks, wl.k_up, wl.v_up_by_q, wl.cos_sin_cache, wl.scale)
    return lambda: torch_ref.lowrank_decode(wl.query, wl.kv_cache, wl.block_table, wl.seq_lens, wl.max_seq_len,
                                            wl.k_up, wl.ranks, wl.k_head_offsets.tolist(), wl.k_width,
                                            wl.v_up_by_q, wl.cos_sin_cache, wl.scale)


def cpu_measure(wl, idx, label):
    import torch
    sub = _cpu_subset(wl, idx)
    t = _cpu_median(cpu_decode_run(sub))
    b = sub.bytes_per_step()
    return dict(value=round(b / t / 1e9, 3), unit="GB/s", seconds_median=round(t, 4), requests=len(idx),
                tokens=sub.tokens, threads=torch.get_num_threads(),
                sample=f"{label}: fp32 PyTorch restatement (oracle/torch_ref.py) on {len(idx)} of the {wl.n} "
                       f"requests ({sub.tokens} tokens), median of 5 runs after 1, GB/s of the same "
                       f"algorithmic bytes")


def cpu_c3_step(n_req=16, context=32768, decode_requests=2, hidden=4096, seed=3003):
    """One config-3 step on the CPU: the 16-token cache write (GEMM, quantize, pack,
    scatter) and the decode of `decode_requests` of the 16 requests."""
    import torch
    from oracle import ref, torch_ref
    from starkv_serve import workloads as W
    wl = W.make_quant([context] * decode_requests, num_heads=32, v_rank=64, seed=seed, device="cpu")
    wl.k_codes = wl.v_codes = None
    lay = ref.row_layout(wl.k_width, 32, wl.v_rank)
    g = torch.Generator().manual_seed(seed + 1)
    kv_down = (torch.randn(wl.k_width + wl.v_rank, hidden, generator=g) * hidden ** -0.5).to(torch.bfloat16)
    hid = torch.randn(n_req, hidden, generator=g).to(torch.bfloat16)
    slots = torch.arange(n_req, dtype=torch.long)
    dec = cpu_decode_run(wl)

    def step():
        torch_ref.write_step(hid, kv_down, wl.k_width, lay, wl.ranks, wl.kv_cache, slots)
        dec()

    t = _cpu_median(step)
    per_req = context * wl.row.nbytes
    return dict(seconds_median=round(t, 3), threads=torch.get_num_threads(),
                GBps=round((decode_requests * per_req + kv_down.numel() * 2) / t / 1e9, 3),
                sample=f"16-token write + decode of {decode_requests} of the 16 requests at {context} tokens, "
                       f"median of 5 runs after 1; the full step would decode 16")


def main():
    global MIN_WARMUP_MS
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--min-warmup-ms", type=float, default=MIN_WARMUP_MS,
                    help="each workload's warmup continues until this many ms of back-to-back calls")
    ap.add_argument("--no-extra", action="store_true", help="skip every workload but the headline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["bf16", "quant", "write", "short", "wide", "wide_quant", "c0", "c3",
                                       "model", "model_c1", "stock", "prefill"],
                    default=None, help="profile runs: time one workload only and print its summary")
    ap.add_argument("--copy-probe", type=float, default=0.0, metavar="GIB",
                    help="profile runs: only copy GIB GiB device to device 5 times (counter scaling)")
    args = ap.parse_args()
    MIN_WARMUP_MS = args.min_warmup_ms
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (decode shards by request; "
              "each GPU would run this same kernel on its own requests). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    torch.cuda.set_device(0)
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.copy_probe > 0:
        copy_probe(args.copy_probe, 5)
        return

    from starkv_serve import workloads as W
    lengths = [8192] * 64
    K, Wm = args.steps, args.warmup
    only = {
        "write": lambda: [bench_write(n, q, K, Wm) for n in (16, 64) for q in (True, False)],
        "short": lambda: summarize(*bench_lowrank([16] * 64, K, Wm, seed=1005)),
        "quant": lambda: summarize(*bench_quant(lengths, K, Wm, seed=1003, copies=3)),
        "wide": lambda: summarize(*bench_lowrank(lengths, K, Wm, seed=1007, v_rank=1280, ranks=RANKS_880)),
        "wide_quant": lambda: summarize(*bench_quant(lengths, K, Wm, seed=1008, copies=3, v_rank=1290,
                                                     ranks=RANKS_880)),
        "c0": lambda: summarize(*bench_lowrank([4096], K, Wm, seed=1000)),
        "c3": lambda: bench_c3(32, 2),
        "model": lambda: bench_model(),
        "model_c1": lambda: bench_model(max_sessions=False),
        "stock": lambda: bench_stock(64, 8192, K, Wm),
        "prefill": lambda: bench_prefill(min(K, 10), min(Wm, 3)),
    }
    if args.only in only:
        print(json.dumps(only[args.only]()), flush=True)
        return
    log("headline: bf16 low-rank, 64 x 8192")
    wl, th = bench_lowrank(lengths, K, Wm, seed=1001)
    head = summarize(wl, th)
    log(json.dumps(head))
    if args.only == "bf16":
        print(json.dumps(head), flush=True)
        return

    extra = {}

    def run(key, what, fn):
        log(what)
        extra[key] = fn()
        log(json.dumps(extra[key]))
        torch.cuda.empty_cache()

    if not args.no_extra:
        run("quant_bs64x8k", "3.2-bit, 64 x 8192 (3 rotating caches)", only["quant"])
        extra["quant_bs64x8k"]["hbm_traffic_bytes"] = measured_traffic("quant_bs64x8k")
        run("lowrank_bs64_ragged_1k_8k", "bf16 low-rank, 64 requests, lengths U[1024, 8192] (config 1)",
            lambda: summarize(*bench_lowrank(W.ragged_lengths(1001), K, Wm, seed=1001)))
        run("quant_bs64_ragged_1k_8k", "3.2-bit, 64 requests, lengths U[1024, 8192] (config 2, 3 rotating caches)",
            lambda: summarize(*bench_quant(W.ragged_lengths(1002), K, Wm, seed=1002, copies=3)))
        run("lowrank_b1x4096", "bf16 low-rank, 1 x 4096 (config 0)", only["c0"])
        run("lowrank_64x16_short", "bf16 low-rank, 64 requests x 16 tokens (host-bound: eager vs graph)",
            only["short"])
        run("quant_bs16x32k_write_decode", "3.2-bit, 16 x 32768, fused write + decode per step (config 3)",
            only["c3"])
        run("lowrank_bs64x8k_w880_v1280", "bf16 low-rank, 64 x 8192, K width 880, V rank 1280 (two-pass)",
            only["wide"])
        run("quant_bs64x8k_w880_v1290", "3.2-bit, 64 x 8192, K width 880, V rank 1290 (two-pass, 3 caches)",
            only["wide_quant"])
        for n_tok in (16, 64):
            for quant in (True, False):
                run(f"write_{'quant' if quant else 'bf16'}_n{n_tok}",
                    f"cache write, {n_tok} tokens, {'3.2-bit' if quant else 'bf16'} (fused vs unfused)",
                    lambda: bench_write(n_tok, quant, K, Wm))
        run("model_llama2_7b_16k", "config 4: Llama-2-7B-shaped decode steps at 16K context", only["model"])
        run("prefill", "dense causal prefill attention (prefill kernel vs torch SDPA)", only["prefill"])
        log("uncompressed bf16 attention (torch fused SDPA), 64 x 8192")
        stock = bench_stock(64, 8192, K, Wm)
        for key, name in (("bf16", head), ("quant", extra["quant_bs64x8k"])):
            if "us_per_step" in stock:
                stock[f"starkv_{key}_speedup_vs_sdpa"] = round(stock["us_per_step"] / name["us_per_step"], 2)
            if "paged_us_per_step" in stock:
                stock[f"starkv_{key}_speedup_vs_paged"] = round(stock["paged_us_per_step"] / name["us_per_step"], 2)
            stock[f"starkv_{key}_speedup_vs_hbm_bound"] = round(stock["hbm_bound_us"] / name["us_per_step"], 2)
        extra["stock_bf16_bs64x8k"] = stock
        log(json.dumps(stock))
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        log(f"cpu baseline ({torch.get_num_threads()} threads)")
        cpu = cpu_measure(wl, list(range(0, 64, 4)), "bf16 64 x 8192")
        cpu.update(cores=torch.get_num_threads(), kind="port")
        log(json.dumps(cpu))
        if not args.no_extra:
            cpu_extra = {}
            w0 = W.make_lowrank([4096], num_heads=32, seed=1000)
            cpu_extra["lowrank_b1x4096"] = cpu_measure(w0, [0], "config 0")
            w1 = W.make_lowrank(W.ragged_lengths(1001), num_heads=32, seed=1001, poison=False)
            cpu_extra["lowrank_bs64_ragged_1k_8k"] = cpu_measure(w1, list(range(0, 64, 4)), "config 1")
            del w1
            w2 = W.make_quant(W.ragged_lengths(1002)[::4], num_heads=32, seed=1002, device="cpu")
            w2.k_codes = w2.v_codes = None
            cpu_extra["quant_bs64_ragged_1k_8k"] = cpu_measure(w2, list(range(16)), "config 2 (16 of its 64 lengths)")
            del w2
            cpu_extra["quant_bs16x32k_write_decode"] = cpu_c3_step()
            extra["cpu_fp32_torch"] = cpu_extra
            log(json.dumps(cpu_extra))

    out = {
        "metric": METRIC,
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(th["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) codes and queries, random-init bases, shuffled pages)",
        "config": {"workload": "bf16 low-rank paged decode, one layer, batch 64 x context 8192",
                   "batch": 64, "context": 8192, "num_heads": 32, "head_dim": 128, "page_size": 16,
                   "k_width": wl.k_width, "v_rank": wl.v_rank, "k_ranks": "uniform {16,32,48,64} per head",
                   "decode_us": head["us_per_step"], "call_us_median": head["call_us_median"],
                   "min_warmup_ms": MIN_WARMUP_MS},
        "roofline": {"bound": "hbm", "achieved": head["kernel_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["hbm_frac"], "traffic": measured_traffic("bf16_bs64x8k"),
                     "kernel": "lowrank_kernel (bf16 decode)", "kernel_us_median": head["decode_kernel_us"],
                     "bytes_per_launch": head["bytes_per_step"], "mfma_frac_fp16": head["mfma_frac"]},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
