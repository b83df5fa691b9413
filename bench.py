"""Benchmark of the paged KV-cache hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

A step is one Mixtral-8x7B-shaped decode step (configuration 2 of the
benchmark set): 32 layers, 64 sequences with context uniform in [512, 4096],
8 KV heads / 32 query heads, head_dim 128, 16-token pages from a seeded
permuted pool.  Per step: the host setup (ensure_pages, device slot mapping,
seq_lens += 1, decode plan with device page-index flattening) and, for each
layer, the KV append of the 64 new tokens followed by paged decode attention
over len + 1 tokens -- the engine's per-layer order (append inside stage 1,
decode in stage 2).  Caches, queries and new K/V rows are resident in HBM
before the timed region starts.

``value`` is the step's algorithmic HBM bytes (decode: every K/V row read once
per KV head + q in + out + page ids; append: rows read + written + slots)
divided by the wall time of the step, so host setup and launch gaps count
against it.  ``roofline`` is the decode-attention launch alone (streaming +
merge kernel, bracketed by HIP events on the stream they run on) against the
8 TB/s HBM3E peak.  ``extra`` carries the other rows of the metric: chunked-
prefill append and gather GB/s (configuration 3), long-context decode GB/s
(configuration 4), swap host-link GB/s with decode slowdown
(configuration 5), continuation-prefill TFLOP/s (the MFMA attention after
the configuration 3 append), the x-packed layout's decode / append GB/s, and
the host-memory policies (layer-wise offload pipeline, swap preemption).  ``cpu_baseline`` times the numpy oracle on one layer of
the same workload on the host cores.

Per-kernel figures (all but the step and configuration 4) are timed after
100 ms of untimed launches of the same call, which bring the clocks to their
steady state.

Other modes used by the profiles (one kernel family each, few launches):
  --mode copy     a plain device copy of known size (FETCH/WRITE calibration)
  --mode decode2  configuration 2 decode with the fused 64-token append, one
                  layer, 10 launches (--separate-append: decode alone)
  --mode decode4  configuration 4 decode only (3 ramp + 3 x 32 timed launches,
                  as in the default run)
  --mode append3  configuration 3 append + gather, one layer, 10 launches each
  --mode prefill3 continuation prefill after the cfg3 append (8 x 2048-token
                  chunks over 2048 and 4096 cached tokens), 10 launches each
  --mode xpacked  vLLM x-packed layout: paged_attention_v2 (1 x 150K and
                  64 x U[512,4096] tokens, MHA 32 x 128 fp16) and
                  reshape_and_cache, 10 launches each
  --mode offload  layer-wise KV offload pipeline (8 layers, 25% of blocks in
                  host memory) and swap preemption of a 4096-token request
  --mode swap5    configuration 5 swap out / swap in of 32 of 128 sequences
                  (16 layers) while the other 96 decode
  --mode bs1      batch-1 latency at the reference's published decode shape
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (no sparsity)
# rocprofv3 FETCH_SIZE/WRITE_SIZE summary of the configuration-2 decode launch
# (calibrated HBM bytes per launch), written from `--mode decode2` runs.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_lds_kernel_cfg2_mixtral_decode.md")


def profiled_traffic():
    """HBM bytes per decode launch measured by the committed counter profile,
    or None when the summary is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="skip configurations 3-5")
    p.add_argument("--separate-append", action="store_true",
                   help="append with reshape_and_cache_flash, then decode (two launches per "
                        "layer) instead of the fused append_and_decode")
    p.add_argument("--mode", default="step",
                   choices=["step", "copy", "decode2", "decode4", "append3", "prefill3",
                            "prefill_power", "xpacked", "offload", "swap5", "bs1"])
    return p.parse_args()


# --------------------------------------------------------------- helpers
def _round_times(torch, fn, reps, rounds=3, warm_s=0.1):
    """Mean event time (s) of ``reps`` back-to-back calls, for each of
    ``rounds`` rounds, after untimed calls that bring the clocks up: at least
    three, and ``warm_s`` seconds of them (a few launches leave an
    MFMA-bound kernel up to 20% slower than its steady state)."""
    t0 = time.perf_counter()
    n = 0
    while n < 3 or time.perf_counter() - t0 < warm_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    ts = []
    for _ in range(rounds):
        e0, e1 = _events(torch)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e-3 / reps)
    return ts


def _timed_rounds(torch, fn, reps, rounds=3):
    """Median over ``rounds`` of the mean event time (s) of ``reps`` calls."""
    ts = _round_times(torch, fn, reps, rounds)
    return sorted(ts)[len(ts) // 2]


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def build_cfg2_cache(torch, seed, num_layers=None):
    from gpu_offloading_amd import workloads
    from gpu_offloading_amd.kv_cache import PagedKVCache

    cfg = workloads.config2(seed=seed)
    sh = cfg.shape
    L = num_layers or sh.num_layers
    B = len(cfg.seq_lens)
    max_len = max(cfg.seq_lens) + cfg.extra["extra_steps"] + 16
    cache = PagedKVCache(L, sh.num_kv_heads, sh.head_dim, max_seqs=B, max_seq_len=max_len,
                         num_qo_heads=sh.num_qo_heads, kv_page_budget=cfg.total_pages,
                         free_page_order=cfg.free_order, device="cuda")
    seqs = list(range(B))
    for s, ln in zip(seqs, cfg.seq_lens):
        cache.ensure_pages(s, (ln + 15) // 16)
    cache.advance(seqs, cfg.seq_lens)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 100)
    for kc, vc in zip(cache.k_cache, cache.v_cache):
        kc.normal_(0.0, 1.0, generator=g)
        vc.normal_(0.0, 1.0, generator=g)
    return cfg, cache, seqs


# ------------------------------------------------------------ main step
def run_step_bench(torch, args):
    from gpu_offloading_amd import workloads

    cfg, cache, seqs = build_cfg2_cache(torch, args.seed)
    sh = cfg.shape
    L, B = sh.num_layers, len(seqs)
    dev = cache.device
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed + 200)
    qs = [torch.randn(B, sh.num_qo_heads, sh.head_dim, device=dev, generator=g).to(torch.bfloat16)
          for _ in range(L)]
    ks = [torch.randn(B, sh.num_kv_heads, sh.head_dim, device=dev, generator=g).to(torch.bfloat16)
          for _ in range(L)]
    vs = [torch.randn(B, sh.num_kv_heads, sh.head_dim, device=dev, generator=g).to(torch.bfloat16)
          for _ in range(L)]
    outs = [torch.empty(B, sh.num_qo_heads, sh.head_dim, dtype=torch.bfloat16, device=dev)
            for _ in range(L)]
    total_steps = args.warmup + args.steps
    if total_steps > cfg.extra["extra_steps"]:
        raise SystemExit(f"warmup + steps must be <= {cfg.extra['extra_steps']} "
                         "(page budget of the configuration)")

    timed = {"on": False, "pairs": [], "bytes": 0, "decode_bytes": []}

    def one_step():
        lens_before = [int(cache._seq_lens_cpu[s]) for s in seqs]
        for s, ln in zip(seqs, lens_before):            # scheduler: ensure_pages
            cache.ensure_pages(s, (ln + 1 + 15) // 16)
        slots = cache.prepare_decode_step(seqs)          # slot map, seq_lens += 1, plan
        lens_after = [ln + 1 for ln in lens_before]
        dbytes = workloads.decode_bytes(lens_after, sh.num_qo_heads, sh.num_kv_heads, sh.head_dim)
        abytes = workloads.append_bytes(B, sh.num_kv_heads, sh.head_dim)
        for layer in range(L):
            if args.separate_append:
                cache.append(layer, ks[layer], vs[layer], slots)
                run = lambda: cache.decode(layer, qs[layer], out=outs[layer])  # noqa: E731
                lbytes = dbytes
            else:
                run = lambda: cache.append_and_decode(  # noqa: E731
                    layer, ks[layer], vs[layer], qs[layer], out=outs[layer])
                lbytes = dbytes + abytes
            # One event pair brackets the step's L decode launches (each
            # recorded event costs the stream a few microseconds, so pairs
            # around single launches overstate them).
            if timed["on"] and layer == 0:
                e0, e1 = _events(torch)
                e0.record()
            run()
            if timed["on"] and layer == L - 1:
                e1.record()
                timed["pairs"].append((e0, e1))
                timed["decode_bytes"].append(lbytes)
        if timed["on"]:
            timed["bytes"] += L * (dbytes + abytes)

    log(f"cfg2: {L} layers, B={B}, pages={cfg.total_pages}, warmup {args.warmup}, steps {args.steps}")
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    timed["on"] = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    step_gbps = timed["bytes"] / (t1 - t0) / 1e9
    durs = [a.elapsed_time(b) / L for a, b in timed["pairs"]]  # ms per launch
    avg_ms = sum(durs) / len(durs)
    avg_bytes = sum(timed["decode_bytes"]) / len(timed["decode_bytes"])
    achieved = avg_bytes / (avg_ms * 1e-3) / 1e9
    sched = cache._decode_wrapper.schedule
    log(f"cfg2: {ms_per_step:.3f} ms/step, step {step_gbps:.1f} GB/s, decode launch "
        f"{avg_ms * 1e3:.1f} us = {achieved:.1f} GB/s ({achieved / HBM_PEAK_GBPS:.1%} of peak); "
        f"segments {sched.num_segments}x{sched.num_head_groups}, max parts {sched.max_partitions}")
    # sanity: the outputs are finite
    assert all(torch.isfinite(o.float()).all().item() for o in outs[:2]), "non-finite decode output"
    res = {
        "ms_per_step": ms_per_step,
        "value": step_gbps,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": profiled_traffic(),
                     "kernel": ("decode_lds_kernel<4, 8> + decode_merge_kernel<128>"
                                + ("" if args.separate_append else
                                   " (the step's 64-token append fused into the streaming "
                                   "kernel: bytes per launch include it)")),
                     "avg_launch_us": avg_ms * 1e3, "algorithmic_bytes_per_launch": avg_bytes,
                     "timing": (f"one event pair around each timed step's {L} back-to-back "
                                "decode launches (streaming + merge kernels and the gaps "
                                "between launches), mean per launch"),
                     "segments": sched.num_segments, "head_groups": sched.num_head_groups,
                     "max_partitions": sched.max_partitions},
    }
    del cache, qs, ks, vs, outs
    torch.cuda.empty_cache()
    return res


# ----------------------------------------------------------- extras
def run_decode2(torch, seed, reps=10, fused=True):
    """Configuration 2 decode attention (len + 1 tokens), one layer; with
    `fused` (the step's default) each launch also appends the step's 64 new
    rows as the requests' last tokens (run_with_append)."""
    from gpu_offloading_amd import workloads

    cfg = workloads.config2(seed=seed)
    sh = cfg.shape
    lens = [ln + 1 for ln in cfg.seq_lens]
    kc, vc, q, w = build_paged(torch, lens, sh.num_kv_heads, sh.head_dim, seed + 3,
                               hq=sh.num_qo_heads)
    out = torch.empty_like(q)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 4)
    nk = torch.randn(len(lens), sh.num_kv_heads, sh.head_dim, device="cuda",
                     generator=g).to(torch.bfloat16)
    nv = torch.randn_like(nk)
    if fused:
        def launch():
            w.run_with_append(q, (kc, vc), nk, nv, out=out)
    else:
        def launch():
            w.run(q, (kc, vc), out=out)
    launch()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(reps):
        launch()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    b = workloads.decode_bytes(lens, sh.num_qo_heads, sh.num_kv_heads, sh.head_dim)
    if fused:
        b += workloads.append_bytes(len(lens), sh.num_kv_heads, sh.head_dim)
    log(f"cfg2 decode: {t * 1e6:.1f} us, {b / t / 1e9:.0f} GB/s, {b} algorithmic bytes")
    print(json.dumps({"mode": "decode2", "us": t * 1e6, "bytes": b, "GBps": b / t / 1e9}),
          flush=True)


def run_cfg3(torch, seed, reps=10, layers=None):
    """Chunked-prefill append of 8 x 2048 tokens per layer into a pool whose
    free list is a random 40% of its blocks, then gather of every sequence."""
    from gpu_offloading_amd import ops, workloads
    from gpu_offloading_amd.allocator import PagePool

    cfg = workloads.config3(seed=seed)
    sh = cfg.shape
    L = layers or sh.num_layers
    pool = PagePool(cfg.total_pages, 8, 2048 // 16, free_order=cfg.free_order)
    bt = torch.full((8, 128), -1, dtype=torch.int32)
    for s in range(8):
        _, pages = pool.alloc(s, 128)
        bt[s] = torch.tensor(pages, dtype=torch.int32)
    pos = torch.arange(2048)
    slots = torch.cat([bt[s, pos // 16].long() * 16 + pos % 16 for s in range(8)]).cuda()
    bt = bt.cuda()
    n = slots.numel()
    shape = (cfg.total_pages, 16, sh.num_kv_heads, sh.head_dim)
    # the PagedKVCache layout: K and V of a page adjacent, one tensor per layer
    kvs = [torch.zeros((shape[0], 2) + tuple(shape[1:]), dtype=torch.bfloat16, device="cuda")
           for _ in range(L)]
    kcs = [t[:, 0] for t in kvs]
    vcs = [t[:, 1] for t in kvs]
    k = [torch.randn(n, sh.num_kv_heads, sh.head_dim, device="cuda").to(torch.bfloat16) for _ in range(2)]
    v = [torch.randn(n, sh.num_kv_heads, sh.head_dim, device="cuda").to(torch.bfloat16) for _ in range(2)]
    ok = torch.empty(n, sh.num_kv_heads, sh.head_dim, dtype=torch.bfloat16, device="cuda")
    ov = torch.empty_like(ok)
    cu = torch.arange(0, 9 * 2048, 2048, dtype=torch.int32, device="cuda")

    def append_all(i):
        for layer in range(L):
            ops.reshape_and_cache_flash(k[i % 2], v[i % 2], kcs[layer], vcs[layer], slots)

    def gather_all():
        for layer in range(L):
            ops.gather_kv(kcs[layer], vcs[layer], bt, cu, 2048, ok, ov)

    append_all(0)
    gather_all()
    torch.cuda.synchronize()
    e = _events(torch)
    e[0].record()
    for i in range(reps):
        append_all(i)
    e[1].record()
    torch.cuda.synchronize()
    t_app = e[0].elapsed_time(e[1]) * 1e-3 / (reps * L)
    e[0].record()
    for _ in range(reps):
        gather_all()
    e[1].record()
    torch.cuda.synchronize()
    t_gat = e[0].elapsed_time(e[1]) * 1e-3 / (reps * L)
    ok_exact = bool(torch.equal(ok, k[(reps - 1) % 2]) and torch.equal(ov, v[(reps - 1) % 2]))
    ab = workloads.append_bytes(n, sh.num_kv_heads, sh.head_dim)
    gb = workloads.gather_bytes([2048] * 8, sh.num_kv_heads, sh.head_dim)
    # What bounds the gather: the same gather over in-order pages (no
    # fragmentation), and the runtime's device copy of the same bytes from
    # the same caches into the same outputs (reads from HBM, writes into
    # outputs that stay in the caches between repetitions).
    bt_inorder = torch.arange(8 * 128, dtype=torch.int32, device="cuda").view(8, 128)
    e[0].record()
    for _ in range(reps):
        for layer in range(L):
            ops.gather_kv(kcs[layer], vcs[layer], bt_inorder, cu, 2048, ok, ov)
    e[1].record()
    torch.cuda.synchronize()
    t_gat_inorder = e[0].elapsed_time(e[1]) * 1e-3 / (reps * L)
    m = ok.numel()                       # the first 512 pages' K and V blocks
    e[0].record()
    for _ in range(reps):
        for layer in range(L):
            flat = kvs[layer].view(-1)
            ok.view(-1).copy_(flat[:m])
            ov.view(-1).copy_(flat[m:2 * m])
    e[1].record()
    torch.cuda.synchronize()
    t_copy = e[0].elapsed_time(e[1]) * 1e-3 / (reps * L)
    res = {"append_GBps": ab / t_app / 1e9, "append_us_per_layer": t_app * 1e6,
           "gather_GBps": gb / t_gat / 1e9, "gather_us_per_layer": t_gat * 1e6,
           "gather_inorder_pages_GBps": gb / t_gat_inorder / 1e9,
           "device_copy_same_bytes_GBps": 2 * ok.numel() * 2 * 2 / t_copy / 1e9,
           "gather_roundtrip_bit_exact": ok_exact, "tokens_per_layer": n}
    log(f"cfg3: append {res['append_GBps']:.0f} GB/s ({t_app * 1e6:.1f} us/layer), gather "
        f"{res['gather_GBps']:.0f} GB/s ({t_gat * 1e6:.1f} us/layer), round trip exact {ok_exact}; "
        f"gather over in-order pages {res['gather_inorder_pages_GBps']:.0f} GB/s, device copy of "
        f"the same bytes {res['device_copy_same_bytes_GBps']:.0f} GB/s")
    del kcs, vcs, k, v, ok, ov
    torch.cuda.empty_cache()
    return res


def build_paged(torch, lens, hkv, d, seed, q_std=1.0, hq=32):
    """Device caches holding sequences `lens` in a seeded permuted pool, plus
    a planned decode wrapper.  K and V are views of one [pages, 2, 16, Hkv, D]
    tensor, the layout PagedKVCache allocates."""
    from gpu_offloading_amd import workloads
    from gpu_offloading_amd.decode import BatchDecodeWithPagedKVCacheWrapper
    import numpy as np

    need = sum((ln + 15) // 16 for ln in lens)
    total = need + 16
    perm = np.asarray(workloads.randperm(total, seed), dtype=np.int32)
    nblk = np.array([(ln + 15) // 16 for ln in lens])
    indptr = np.zeros(len(lens) + 1, np.int32)
    np.cumsum(nblk, out=indptr[1:])
    indices = perm[:need].copy()
    lpl = np.array([ln % 16 or 16 for ln in lens], np.int32)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    kv = torch.empty(total, 2, 16, hkv, d, dtype=torch.bfloat16, device="cuda")
    kc, vc = kv[:, 0], kv[:, 1]
    kc.normal_(0, 1, generator=g)
    vc.normal_(0, 1, generator=g)
    q = (torch.randn(len(lens), hq, d, device="cuda", generator=g) * q_std).to(torch.bfloat16)
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device="cuda"))
    w.plan(torch.from_numpy(indptr), torch.from_numpy(indices).cuda(), torch.from_numpy(lpl),
           num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, page_size=16)
    return kc, vc, q, w


def prefill_flops(q_lens, kv_lens, hq, d, causal=True):
    """Algorithmic FLOPs of prefill attention: 4*D per (query row, head,
    visible key) -- q.k and p.v, multiply + add."""
    total = 0
    for ql, kl in zip(q_lens, kv_lens):
        if causal:
            # query i sees min(kl, i + kl - ql + 1) keys (at least 0)
            vis = sum(max(0, min(kl, i + kl - ql + 1)) for i in range(ql))
        else:
            vis = ql * kl
        total += vis * hq * d * 4
    return total


def _prefill_problem(torch, seed, q_len, kv_len, hq=32, hkv=8, d=128):
    """Eight requests of q_len queries over kv_len cached keys (the chunk's
    own keys last), pages from a seeded permuted pool, planned causal."""
    import numpy as np

    from gpu_offloading_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    q_lens, kv_lens = [q_len] * 8, [kv_len] * 8
    kc, vc, _, w0 = build_paged(torch, kv_lens, hkv, d, seed + 11, hq=hq)
    qo = np.arange(0, 9 * q_len, q_len, dtype=np.int32)
    kvi = np.arange(0, 9 * (kv_len // 16), kv_len // 16, dtype=np.int32)
    lpl = np.full(8, 16, np.int32)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 12)
    q = torch.randn(8 * q_len, hq, d, device="cuda", generator=g).to(torch.bfloat16)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1 << 20, dtype=torch.uint8, device="cuda"))
    w.plan(torch.from_numpy(qo), torch.from_numpy(kvi), w0._indices, torch.from_numpy(lpl),
           num_qo_heads=hq, num_kv_heads=hkv, head_dim_qk=d, page_size=16, causal=True,
           q_data_type=torch.bfloat16)
    out = torch.empty_like(q)
    return (lambda: w.run(q, (kc, vc), out=out)), out, prefill_flops(q_lens, kv_lens, hq, d)


def run_prefill(torch, seed, reps=10):
    """Paged-KV continuation prefill (the attention after the cfg3 append):
    8 requests x 2048-token chunks, Hq=32 / Hkv=8 / D=128, causal, over
    (a) the chunk alone (first chunk) and (b) a 2048-token cached prefix plus
    the chunk (second chunk).  Pages come from a seeded permuted pool."""
    res = {}
    for name, q_len, kv_len in (("first_chunk", 2048, 2048), ("second_chunk", 2048, 4096)):
        fn, out, f = _prefill_problem(torch, seed, q_len, kv_len)
        t = _timed_rounds(torch, fn, reps)
        assert torch.isfinite(out).all().item(), "non-finite prefill output"
        res[name] = {"q_len": q_len, "kv_len": kv_len, "requests": 8, "us": t * 1e6,
                     "TFLOPs": f / t / 1e12, "frac_of_peak": f / t / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                     "algorithmic_flops": f}
        log(f"prefill {name}: 8 x {q_len} queries over {kv_len} keys, {t * 1e6:.1f} us, "
            f"{f / t / 1e12:.1f} TFLOP/s ({f / t / 1e12 / MFMA_BF16_PEAK_TFLOPS:.1%} of bf16 MFMA peak)")
        del fn, out
        torch.cuda.empty_cache()
    return res


def _smi_power_clock():
    """(socket power W, mean GFX clock MHz over the XCDs) from `amd-smi
    metric -p -c`, or (None, None) when the tool is missing."""
    import subprocess

    try:
        txt = subprocess.run(["amd-smi", "metric", "-g", "0", "-p", "-c"], capture_output=True,
                             text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None, None
    power, clocks, section = None, [], ""
    for line in txt.splitlines():
        key, _, val = line.strip().partition(":")
        if not val.strip():
            section = key
            continue
        if key == "SOCKET_POWER":
            power = float(val.split()[0])
        elif key == "CLK" and section.startswith("GFX_"):
            clocks.append(float(val.split()[0]))
    return power, (sum(clocks) / len(clocks) if clocks else None)


def run_prefill_power(torch, seed, seconds=6.0, q_len=2048, kv_len=4096):
    """The (second-chunk) prefill launched back to back for `seconds` while the
    board's socket power and GFX clocks are sampled (amd-smi), and the bf16
    MFMA peak at the sampled clock (1,024 SIMDs x 1,024 FLOP per cycle)."""
    import threading

    fn, out, f = _prefill_problem(torch, seed, q_len, kv_len)
    _round_times(torch, fn, 3, rounds=1, warm_s=0.5)
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.wait(0.5):
            samples.append(_smi_power_clock())

    th = threading.Thread(target=sampler)
    th.start()
    n, t0 = 0, time.perf_counter()
    e0, e1 = _events(torch)
    e0.record()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        n += 20
        torch.cuda.synchronize()
    e1.record()
    torch.cuda.synchronize()
    stop.set()
    th.join()
    t = e0.elapsed_time(e1) * 1e-3 / n
    got = [x for x in samples[1:] if x[0] is not None and x[1] is not None]
    power = sorted(p for p, _ in got)[len(got) // 2] if got else None
    clock = sorted(c for _, c in got)[len(got) // 2] if got else None
    peak = 1024 * 1024 * clock * 1e6 / 1e12 if clock else None
    res = {"launches": n, "us": t * 1e6, "TFLOPs": f / t / 1e12, "samples": len(got),
           "socket_power_W": power, "gfx_clock_MHz": clock, "bf16_peak_at_clock_TFLOPs": peak,
           "frac_of_peak_at_clock": f / t / 1e12 / peak if peak else None}
    log(f"prefill {q_len} over {kv_len} sustained: {t * 1e6:.1f} us, {f / t / 1e12:.1f} TFLOP/s, "
        f"socket {power} W, GFX {clock} MHz")
    return res


def run_xpacked(torch, seed, reps=10):
    """vLLM x-packed layout (the reference's dense sandbox): paged_attention_v2
    at the shape of the reference's GH200 data point -- one 150,000-token
    decode, 32 MHA heads x 128, fp16, 16-token blocks in random order
    (src/dense/include/paged_transformer.py:103-111, 325-332) -- and a 64-
    sequence batch with context U[512, 4096]; reshape_and_cache of a
    16,384-token prefill (whole blocks) and of a 64-token decode step
    (scattered slots)."""
    import numpy as np

    from gpu_offloading_amd import ops

    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 21)
    h, d = 32, 128
    res = {}

    def timed(fn):
        return _timed_rounds(torch, fn, reps)

    rng = np.random.default_rng(seed + 22)
    for name, lens in (("v2_1x150000", [150000]),
                       ("v2_64xU512_4096", rng.integers(512, 4097, 64).tolist())):
        need = sum((n + 15) // 16 for n in lens)
        nb = need + 16
        kc = torch.empty(nb, h, d // 8, 16, 8, dtype=torch.float16, device="cuda")
        vc = torch.empty(nb, h, d, 16, dtype=torch.float16, device="cuda")
        kc.normal_(0, 1, generator=g)
        vc.normal_(0, 1, generator=g)
        perm = torch.randperm(nb, generator=g, device="cuda").to(torch.int32)
        bt = torch.full((len(lens), max((n + 15) // 16 for n in lens)), -1, dtype=torch.int32,
                        device="cuda")
        at = 0
        for b, n in enumerate(lens):
            k = (n + 15) // 16
            bt[b, :k] = perm[at:at + k]
            at += k
        q = torch.randn(len(lens), h, d, device="cuda", generator=g).to(torch.float16)
        sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
        msl = max(lens)
        parts = (msl + 511) // 512
        out = torch.empty_like(q)
        es = torch.empty(len(lens), h, parts, device="cuda")
        ml = torch.empty_like(es)
        tmp = torch.empty(len(lens), h, parts, d, dtype=q.dtype, device="cuda")
        t = timed(lambda: ops.paged_attention_v2(out, es, ml, tmp, q, kc, vc, h, d ** -0.5, bt, sl,
                                                 16, msl, None, "auto", 1.0, 1.0, 0, 0, 0, 0, 0))
        byts = sum(lens) * h * d * 2 * 2 + 2 * len(lens) * h * d * 2
        assert torch.isfinite(out).all().item(), "non-finite v2 output"
        res[name] = {"us": t * 1e6, "GBps": byts / t / 1e9, "frac_of_peak": byts / t / 1e9 / HBM_PEAK_GBPS,
                     "algorithmic_bytes": byts, "seqs": len(lens), "tokens": int(sum(lens))}
        log(f"x-packed {name}: {t * 1e6:.1f} us, {byts / t / 1e9:.0f} GB/s "
            f"({byts / t / 1e9 / HBM_PEAK_GBPS:.1%} of peak)")
        del kc, vc, q, out, es, ml, tmp, bt
        torch.cuda.empty_cache()
    # reshape_and_cache: K/V are views of a packed qkv [N, 3, H, D] (the sandbox's layout)
    n = 16384
    nb = n // 16 + 64
    kc = torch.zeros(nb, h, d // 8, 16, 8, dtype=torch.float16, device="cuda")
    vc = torch.zeros(nb, h, d, 16, dtype=torch.float16, device="cuda")
    qkv = torch.randn(n, 3, h, d, device="cuda", generator=g).to(torch.float16)
    blocks = torch.randperm(nb, generator=g, device="cuda")[: n // 16]
    slots = (blocks.repeat_interleave(16) * 16 + torch.arange(16, device="cuda").repeat(n // 16)).long()
    t = timed(lambda: ops.reshape_and_cache(qkv[:, 1], qkv[:, 2], kc, vc, slots))
    byts = n * (2 * h * d * 2 * 2 + 8)
    res["append_prefill_16384"] = {"us": t * 1e6, "GBps": byts / t / 1e9,
                                   "frac_of_peak": byts / t / 1e9 / HBM_PEAK_GBPS}
    dec = slots[::256][:64].contiguous()
    t64 = timed(lambda: ops.reshape_and_cache(qkv[:64, 1], qkv[:64, 2], kc, vc, dec))
    res["append_decode_64_us"] = t64 * 1e6
    log(f"x-packed reshape_and_cache: 16384 tokens {t * 1e6:.1f} us = {byts / t / 1e9:.0f} GB/s; "
        f"64 scattered tokens {t64 * 1e6:.1f} us")
    del kc, vc, qkv
    torch.cuda.empty_cache()
    return res


def run_offload(torch, seed, steps=3):
    """Host-memory KV policies.  (a) Layer-wise offload of the dense sandbox
    (paged_offload_transformer.py): 8 layers, MHA 32 x 128 fp16, a mixed
    batch of 32 decodes over 2048-token histories + 2 prefills of 512 tokens,
    25% of every sequence's blocks in pinned host memory for layers 1..7,
    staged through two scratchpads by the three-stream pipeline; per step
    each layer appends and runs paged_attention_v2.  Reported: step time,
    the same step all-resident, and the host-link rate of the staging.
    (b) Swap preemption, Mixtral-shaped (32 layers, Hkv 8, D 128, bf16): one
    4096-token request swapped out and back in."""
    from gpu_offloading_amd import hostmem, ops
    from gpu_offloading_amd.kv_cache import PagedKVCache
    from gpu_offloading_amd.offload import KVOffloadPipeline, PagedOffloadKV, SwapPreemption

    res = {}
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 31)
    L, H = 8, 32
    dec, pre = [2048] * 32, [512] * 2
    for ratio in (0.0, 0.25):
        kv = PagedOffloadKV(dec, pre, L, H, 128, ratio, device="cuda", allocation_mode="random",
                            seed=seed + 32)
        kv.key_heap.normal_(0, 1, generator=g)
        kv.val_heap.normal_(0, 1, generator=g)
        for t in kv.k_offload_cpu + kv.v_offload_cpu:
            t.normal_(0, 1)
        pipe = KVOffloadPipeline(kv) if ratio > 0 else None
        T = kv.total_tokens
        ks = [torch.randn(T, H, 128, device="cuda", generator=g).half() for _ in range(L)]
        qs = [torch.randn(len(dec), H, 128, device="cuda", generator=g).half() for _ in range(L)]
        out = torch.empty_like(qs[0])

        def step():
            if pipe:
                pipe.begin_step()
            for layer in range(L):
                if pipe:
                    pipe.before_append(layer)
                ops.reshape_and_cache(ks[layer], ks[layer], kv.key_heap, kv.val_heap,
                                      kv.slot_mapping[layer])
                if pipe:
                    pipe.prefill_done(layer)
                    pipe.before_decode(layer)
                ops.paged_attention_v2(out, kv.exp_sums, kv.max_logits, kv.tmp_output, qs[layer],
                                       kv.key_heap, kv.val_heap, H, 0.0884,
                                       kv.decode_block_table(layer), kv.decode_context_lens, 16,
                                       kv.max_decode_len)
                if pipe:
                    pipe.layer_done(layer)

        step()
        torch.cuda.synchronize()
        if pipe:
            pipe.synchronize()
            pipe.copy_seconds()
            pipe.h2d_bytes = pipe.d2h_bytes = 0
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        if pipe:
            pipe.synchronize()
        wall = (time.perf_counter() - t0) / steps
        r = {"kv_offload_ratio": ratio, "step_ms": wall * 1e3}
        if pipe:
            cs = pipe.copy_seconds()
            # The write-back (D2H) span also holds the gather of the prefill
            # blocks on the D2H stream, beside the compute: a stream span,
            # not a link rate.
            r.update({"h2d_GB_per_step": pipe.h2d_bytes / steps / 1e9,
                      "h2d_GBps": pipe.h2d_bytes / cs["h2d"] / 1e9,
                      "d2h_GB_per_step": pipe.d2h_bytes / steps / 1e9,
                      "d2h_stream_ms_per_step": cs["d2h"] / steps * 1e3,
                      "link_bound_step_ms": cs["h2d"] / steps * 1e3})
        res[f"layer_offload_ratio_{ratio}"] = r
        log(f"offload ratio {ratio}: step {wall * 1e3:.2f} ms" +
            (f", H2D {r['h2d_GB_per_step']:.2f} GB/step at {r['h2d_GBps']:.1f} GB/s "
             f"(copy-stream time {r['link_bound_step_ms']:.2f} ms/step), "
             f"write-back {r['d2h_GB_per_step'] * 1e3:.0f} MB/step in "
             f"{r['d2h_stream_ms_per_step']:.2f} ms of D2H-stream time" if pipe else ""))
        del kv, pipe, ks, qs, out
        torch.cuda.empty_cache()

    cache = PagedKVCache(32, 8, 128, max_seqs=4, max_seq_len=4096 + 64, num_qo_heads=32,
                         kv_page_budget=600, device="cuda", workspace_bytes=1 << 24,
                         staging_bytes=256 << 20)
    cache.ensure_pages(0, 256)
    cache.advance([0], [4096])
    for layer in range(32):
        cache.k_cache[layer].normal_(0, 1, generator=g)
    pre = SwapPreemption(cache)
    cache.reserve_swap()
    snap = cache.k_cache[5][cache.block_table[0, :256].long()].clone()
    # The host image comes from a pool, as an engine would keep one.
    image = hostmem.pinned_empty(32 * 256 * 2 * ops.block_bytes(cache.k_cache[0]))
    torch.cuda.synchronize()
    # One untimed preemption and resume of the same request first (through
    # the same buffer: the first copies of a process pay a one-time set-up),
    # then `cycles` timed ones, the request moving to the next slot each time.
    # Single cycles of this size on these boxes now and then run at 30-34
    # GB/s in one direction (the runtime's copy itself runs slower), so the
    # figure is the median cycle, with every cycle's rate beside it.
    hw = pre.preempt(0, key="warm", host=image)
    cache.synchronize_swaps()
    pre.resume("warm", slot=1)
    cache.synchronize_swaps()
    first = (hw.num_bytes / hw.out_seconds() / 1e9, hw.num_bytes / hw.in_seconds() / 1e9)
    cycles, slot = 8, 1
    t_out, t_in = [], []
    for i in range(cycles):
        h = pre.preempt(slot, key=i, host=image)
        cache.synchronize_swaps()
        t_out.append(h.out_seconds())
        slot = 1 + slot % 3
        pre.resume(i, slot=slot)
        cache.synchronize_swaps()
        t_in.append(h.in_seconds())
    exact = bool(torch.equal(cache.k_cache[5][cache.block_table[slot, :256].long()], snap))
    nb = h.num_bytes
    mo, mi = statistics.median(t_out), statistics.median(t_in)
    res["swap_preemption_4096_tokens"] = {
        "bytes_each_way": nb, "cycles": cycles, "out_ms": mo * 1e3, "in_ms": mi * 1e3,
        "out_GBps": nb / mo / 1e9, "in_GBps": nb / mi / 1e9,
        "out_GBps_per_cycle": [round(nb / t / 1e9, 1) for t in t_out],
        "in_GBps_per_cycle": [round(nb / t / 1e9, 1) for t in t_in],
        "first_cycle_out_in_GBps": [round(first[0], 1), round(first[1], 1)],
        "restored_exact": exact}
    log(f"swap preemption of a 4096-token request (32 layers), median of {cycles} cycles: "
        f"out {mo * 1e3:.1f} ms ({nb / mo / 1e9:.1f} GB/s), in {mi * 1e3:.1f} ms "
        f"({nb / mi / 1e9:.1f} GB/s), restored exact {exact}; per cycle out "
        f"{[round(nb / t / 1e9, 1) for t in t_out]}, in {[round(nb / t / 1e9, 1) for t in t_in]}; "
        f"untimed first cycle {first[0]:.1f} / {first[1]:.1f} GB/s")
    del cache
    torch.cuda.empty_cache()
    return res


def run_small_batch(torch, seed, layers=20, steps=50):
    """Latency at the reference's own decode shape: Mixtral attention (Hkv 8,
    Hq 32, D 128, page 16), batch 1, a 128-token context, 20 layers -- the
    H100 figures it publishes are 90 us of FlashInfer decode per step and a
    9.4 us decode-kernel median (src/MoE/tests/vLLM_comparison/README.md:102,
    src/MoE/pipeline_parallelism.md:144) and 0.258 ms of step setup
    (pipeline_parallelism.md:81).  Reported: the decode launch alone (event
    time per launch over back-to-back launches), one step (setup + 20 fused
    append + decode launches, event time), the same step with its 20
    launches replayed from a HIP graph, and the host time of the step
    setup."""
    from gpu_offloading_amd.kv_cache import PagedKVCache

    cache = PagedKVCache(layers, 8, 128, max_seqs=1, max_seq_len=128 + 2 * steps + 64,
                         num_qo_heads=32, kv_page_budget=64, device="cuda",
                         workspace_bytes=1 << 22, staging_bytes=1 << 20)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 500)
    cache.fill_kv_random(1.0, generator=g)
    cache.ensure_pages(0, 128 // 16)
    cache.advance([0], [128])
    q = torch.randn(1, 32, 128, device="cuda", generator=g).to(torch.bfloat16)
    nk = torch.randn(1, 8, 128, device="cuda", generator=g).to(torch.bfloat16)
    nv = torch.randn_like(nk)
    out = torch.empty_like(q)

    def step():
        cache.ensure_pages(0, (int(cache._seq_lens_cpu[0]) + 1 + 15) // 16)
        t0 = time.perf_counter()
        cache.prepare_decode_step([0])
        setup = time.perf_counter() - t0
        for layer in range(layers):
            cache.append_and_decode(layer, nk, nv, q, out=out)
        return setup

    for _ in range(5):
        step()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    setups = []
    e0.record()
    for _ in range(steps):
        setups.append(step())
    e1.record()
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    t_dec = _timed_rounds(torch, lambda: cache.decode(0, q, out=out), 100)

    # The same steps with the 20 fused launches captured once in a HIP graph
    # and replayed after each step's setup: the kernels read the step's plan,
    # lengths and page ids from the cache's step buffer (decode_graph_key
    # says when a new capture is needed).
    graph, key, captures = None, None, [0]

    def graph_step():
        nonlocal graph, key
        cache.ensure_pages(0, (int(cache._seq_lens_cpu[0]) + 1 + 15) // 16)
        cache.prepare_decode_step([0])
        if cache.decode_graph_key() != key:
            captures[0] += 1
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for layer in range(layers):
                    cache.append_and_decode(layer, nk, nv, q, out=out)
            key = cache.decode_graph_key()
        graph.replay()

    for _ in range(5):
        graph_step()
    torch.cuda.synchronize()
    warm_captures = captures[0]
    e0.record()
    for _ in range(steps):
        graph_step()
    e1.record()
    torch.cuda.synchronize()
    graph_ms = e0.elapsed_time(e1) / steps
    log(f"bs1: graph captures {warm_captures} in warm-up, {captures[0] - warm_captures} timed")
    res = {"decode_launch_us": t_dec * 1e6, "step_ms_20_layers": step_ms,
           "per_layer_us": step_ms * 1e3 / layers,
           "step_ms_20_layers_graph": graph_ms,
           "per_layer_us_graph": graph_ms * 1e3 / layers,
           "step_setup_host_ms": 1e3 * sorted(setups)[len(setups) // 2],
           "shape": "B=1, ctx 128 (+1 per step), Hkv 8, Hq 32, D 128, 20 layers"}
    log(f"bs1: decode launch {res['decode_launch_us']:.1f} us, step {step_ms:.3f} ms for "
        f"{layers} layers ({res['per_layer_us']:.1f} us/layer), setup "
        f"{res['step_setup_host_ms']:.3f} ms host; graph-replayed step {graph_ms:.3f} ms "
        f"({res['per_layer_us_graph']:.1f} us/layer)")
    del cache
    torch.cuda.empty_cache()
    return res


def run_cfg4(torch, seed, reps=32):
    """Configuration 4 (B=16 x 32768-token contexts): three timed rounds of
    `reps` back-to-back launches after a clock ramp of three launches; the
    sustained figure averages every timed launch (power droop included), the
    best round is reported beside it.  `--mode decode4` runs exactly this, so
    its kernel trace covers the same launches."""
    from gpu_offloading_amd import workloads

    cfg = workloads.config4(seed=seed)
    sh = cfg.shape
    kc, vc, q, w = build_paged(torch, cfg.seq_lens, sh.num_kv_heads, sh.head_dim, seed + 5,
                               q_std=cfg.q_std, hq=sh.num_qo_heads)
    out = torch.empty_like(q)
    ts = _round_times(torch, lambda: w.run(q, (kc, vc), out=out), reps, warm_s=0.0)
    t, best = sum(ts) / len(ts), min(ts)
    b = workloads.decode_bytes(cfg.seq_lens, sh.num_qo_heads, sh.num_kv_heads, sh.head_dim)
    # The sustained figure (every launch of every round, power droop
    # included) is the roofline one; the best round is reported beside it.
    res = {"decode_GBps": b / t / 1e9, "decode_us": t * 1e6,
           "frac_of_peak": b / t / 1e9 / HBM_PEAK_GBPS,
           "best_round_GBps": b / best / 1e9, "best_round_us": best * 1e6,
           "best_round_frac_of_peak": b / best / 1e9 / HBM_PEAK_GBPS,
           "timing": (f"sustained: mean over 3 rounds x {reps} back-to-back launches after a "
                      "clock ramp (the roofline figure); best round beside it"),
           "segments": w.schedule.num_segments}
    log(f"cfg4: decode {res['decode_GBps']:.0f} GB/s sustained ({t * 1e6:.1f} us, "
        f"{res['frac_of_peak']:.1%} of peak); best round {res['best_round_GBps']:.0f} GB/s "
        f"({best * 1e6:.1f} us)")
    del kc, vc, q, w, out
    torch.cuda.empty_cache()
    return res


def run_cfg5(torch, seed, decode_steps=6):
    """OLMoE-shaped swap under load: 16 layers, Hkv = Hq = 16, batch 128 at
    2048 tokens; a seeded 25% of the sequences are evicted to pinned host
    memory and restored on the side stream while the other 96 decode."""
    from gpu_offloading_amd import hostmem, workloads
    from gpu_offloading_amd.kv_cache import PagedKVCache

    cfg = workloads.config5(seed=seed)
    sh = cfg.shape
    L, B = sh.num_layers, len(cfg.seq_lens)
    cache = PagedKVCache(L, sh.num_kv_heads, sh.head_dim, max_seqs=B, max_seq_len=2048 + 64,
                         num_qo_heads=sh.num_qo_heads, kv_page_budget=cfg.total_pages,
                         free_page_order=cfg.free_order, device="cuda",
                         staging_bytes=512 << 20)
    cache.reserve_swap()   # staging and streams made before the engine loop
    seqs = list(range(B))
    for s in seqs:
        cache.ensure_pages(s, 2048 // 16)
    cache.advance(seqs, cfg.seq_lens)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 300)
    for kc, vc in zip(cache.k_cache, cache.v_cache):
        kc.normal_(0, 1, generator=g)
        vc.normal_(0, 1, generator=g)
    victims = sorted(workloads.randperm(B, seed + 7)[: B // 4])
    running = [s for s in seqs if s not in set(victims)]
    q = torch.randn(len(running), sh.num_qo_heads, sh.head_dim, device="cuda",
                    generator=g).to(torch.bfloat16)
    out = torch.empty_like(q)

    cache.plan_decode(running)   # the running set and its lengths stay fixed

    def decode_pass():
        for layer in range(L):
            cache.decode(layer, q, out=out)

    # reference snapshot of the victims' rows on every layer (device gathers,
    # 8.6 GB in HBM, compared byte for byte after the restore)
    before = [cache.gather(layer, victims) for layer in range(L)]
    decode_pass()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(decode_steps):
        decode_pass()
    e1.record()
    torch.cuda.synchronize()
    t_alone = e0.elapsed_time(e1) * 1e-3 / decode_steps

    # pinned host buffer allocated up front (hipHostMalloc of 8 GiB is not link time)
    bb = 2 * cache.k_cache[0][0].numel() * cache.k_cache[0].element_size()
    npages = sum(cache.seq_pages(s) for s in victims)
    host = hostmem.pinned_empty(L * npages * bb, "cuda")
    nbytes_est = L * npages * bb
    # One untimed eviction and restore of the same victims first, reported
    # apart from the steady-state figure below.  Without reserve_swap's
    # warm-up of the runtime's copy path the first swaps of a process paid
    # one-time host costs (18-31 / 10-16 / 3 ms to enqueue the first three
    # swap-outs); with it the first is within a few ms of the later ones.
    t0 = time.perf_counter()
    hw = cache.swap_out(victims, host=host)
    first_out_ms = (time.perf_counter() - t0) * 1e3
    cache.synchronize_swaps()
    t0 = time.perf_counter()
    cache.swap_in(hw)
    first_in_ms = (time.perf_counter() - t0) * 1e3
    cache.synchronize_swaps()
    del hw

    def under_swap(start_swap):
        """Start a swap, then enqueue decode passes back to back on the
        current stream (no host waits) for about 1.5x the swap's expected
        time at 50 GB/s; the mean GPU time of the passes that ran entirely
        between the swap's start and end events is the decode time under
        load."""
        n_pass = max(8, int(1.5 * nbytes_est / 50e9 / t_alone))
        t0 = time.perf_counter()
        h_, ev_start, ev_end = start_swap()
        host_ms = (time.perf_counter() - t0) * 1e3
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(n_pass + 1)]
        marks[0].record()
        for i in range(n_pass):
            decode_pass()
            marks[i + 1].record()
        torch.cuda.synchronize()
        ev_end.synchronize()
        w_end = ev_start.elapsed_time(ev_end)
        inside = []
        for i in range(n_pass):
            a, b = ev_start.elapsed_time(marks[i]), ev_start.elapsed_time(marks[i + 1])
            if a >= 0 and b <= w_end:
                inside.append(b - a)
        return h_, (sum(inside) / len(inside) * 1e-3 if inside else None), len(inside), host_ms

    def start_out():
        h_ = cache.swap_out(victims, host=host)
        return h_, h_.out_start, h_.out_event

    h, t_dec_out, n_dec, host_ms_out = under_swap(start_out)
    t_out = h.out_seconds()

    def start_in():
        cache.swap_in(h)
        return h, h.in_start, h.in_event

    _, t_dec_in, n_dec_in, host_ms_in = under_swap(start_in)
    t_in = h.in_seconds()
    exact, layers_checked = True, 0
    for layer in range(L):
        after = cache.gather(layer, victims)
        exact = exact and all(torch.equal(a, b) for a, b in zip(before[layer], after))
        layers_checked += 1
        del after
    nbytes = h.bytes_per_direction
    res = {"swap_out_GBps": nbytes / t_out / 1e9, "swap_in_GBps": nbytes / t_in / 1e9,
           "bytes_each_way": nbytes, "blocks": h.num_blocks * L,
           "decode_ms_alone": t_alone * 1e3,
           "decode_ms_during_swap_out": t_dec_out * 1e3 if n_dec else None,
           "decode_ms_during_swap_in": t_dec_in * 1e3 if n_dec_in else None,
           "decode_steps_during_swap_out": n_dec,
           "decode_steps_during_swap_in": n_dec_in,
           "host_ms_to_enqueue_swap": [round(host_ms_out, 3), round(host_ms_in, 3)],
           "host_ms_to_enqueue_first_swap": [round(first_out_ms, 3), round(first_in_ms, 3)],
           "restored_bit_exact": bool(exact), "layers_checked": layers_checked}
    sl = [x for x in (res["decode_ms_during_swap_out"], res["decode_ms_during_swap_in"]) if x]
    res["decode_slowdown"] = (sum(sl) / len(sl)) / res["decode_ms_alone"] if sl else None
    for k in ("out", "in"):
        x = res[f"decode_ms_during_swap_{k}"]
        res[f"decode_slowdown_{k}"] = x / res["decode_ms_alone"] if x else None
    log(f"cfg5: swap out {res['swap_out_GBps']:.1f} GB/s, in {res['swap_in_GBps']:.1f} GB/s "
        f"({nbytes / 1e9:.2f} GB each way), decode slowdown {res['decode_slowdown']}, "
        f"restored exact {exact} ({layers_checked} layers)")
    cache.synchronize_swaps()
    del cache, q, out, before, h
    torch.cuda.empty_cache()
    return res


def run_link_calibration(torch):
    """The host link's own rate, the roofline of the swap rows: 1 GiB copies
    between a pinned buffer on the GPU's NUMA node (where the node is known)
    and device memory, each way, plus where that buffer was placed."""
    from gpu_offloading_amd import hostmem

    res = hostmem.calibrate_link("cuda")
    log(f"host link: H2D {res['h2d_GBps']:.1f} GB/s, D2H {res['d2h_GBps']:.1f} GB/s "
        f"(GPU NUMA node {res['gpu_numa_node']}, mems allowed {res['mems_allowed']}, "
        f"placement {res['policy']})")
    torch.cuda.empty_cache()
    return res


# ----------------------------------------------------------- CPU baseline
def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _cpu_threads() -> int:
    """Every core this process may run on, capped at the box's CPU share
    (OMP_NUM_THREADS, set to the share on the GPU boxes)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(cap)) if cap.isdigit() and int(cap) > 0 else n


def _time_op(fn, seconds, min_reps=2):
    """Repeat fn for about `seconds` (at least min_reps times); mean seconds."""
    fn()                                     # first touch of the buffers
    t0 = time.perf_counter()
    reps = 0
    while reps < min_reps or time.perf_counter() - t0 < seconds:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def run_cpu_baseline(seed, seconds_per_op=2.5):
    """The reference path's semantics restated in torch on the CPU
    (oracle/torch_cpu.py, pinned to the numpy oracle by tests/test_oracle.py),
    timed on this host with all of its threads, on bounded samples of the
    workloads:
      step    one layer of configuration 2: append of the 64 new rows, then
              fp32 decode of the 64 sequences over len + 1 tokens (the
              metric of `value`, same algorithmic bytes);
      append  configuration 3's 16,384-token chunk into the fragmented pool;
      gather  configuration 3's 8 x 2048 tokens back to contiguous rows;
      swap    one layer of configuration 5: its 25% victim blocks (4096 x
              128 KiB) to a host image and back;
    plus the numpy oracle on one thread over the configuration-2 layer."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    from gpu_offloading_amd import workloads
    from oracle import kv_oracle as orc
    from oracle import torch_cpu as tc

    threads = _cpu_threads()
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed + 900)
    tile = torch.randn(1 << 22, generator=g).to(torch.bfloat16)

    def randn(shape):
        # N(0, 1) bf16 values: a seeded 4M-value block tiled over the tensor
        # (drawing every value would take most of the CPU leg's time)
        t = torch.empty(*shape, dtype=torch.bfloat16)
        flat = t.view(-1)
        n, m = flat.numel(), tile.numel()
        full = n // m
        if full:
            flat[:full * m].view(full, m).copy_(tile.expand(full, m))
        flat[full * m:].copy_(tile[:n - full * m])
        return t

    t_setup = time.perf_counter()
    # -- configuration 2, one layer
    cfg = workloads.config2(seed=seed)
    sh = cfg.shape
    lens = list(cfg.seq_lens)
    B = len(lens)
    pool = orc.FifoPagePool(cfg.total_pages, B, max(lens) // 16 + 8, free_order=cfg.free_order)
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 1 + 15) // 16)
    kc = randn((cfg.total_pages, 16, sh.num_kv_heads, sh.head_dim))
    vc = randn((cfg.total_pages, 16, sh.num_kv_heads, sh.head_dim))
    kn, vn = randn((B, sh.num_kv_heads, sh.head_dim)), randn((B, sh.num_kv_heads, sh.head_dim))
    q = randn((B, sh.num_qo_heads, sh.head_dim))
    lens1 = [ln + 1 for ln in lens]
    slots = torch.from_numpy(orc.slot_mapping(pool.block_table, range(B), lens))
    indptr, lpl = orc.plan_decode(lens1)
    indices = orc.page_indices(pool.block_table, range(B), indptr)
    ip_t, idx_t, lpl_t = (torch.from_numpy(x) for x in (indptr, indices, lpl))
    step_bytes = (workloads.decode_bytes(lens1, sh.num_qo_heads, sh.num_kv_heads, sh.head_dim)
                  + workloads.append_bytes(B, sh.num_kv_heads, sh.head_dim))

    def step():
        tc.reshape_and_cache(kn, vn, kc, vc, slots)
        tc.paged_decode(q, kc, vc, ip_t, idx_t, lpl_t)

    # -- configuration 3
    cfg3 = workloads.config3(seed=seed)
    sh3 = cfg3.shape
    pool3 = orc.FifoPagePool(cfg3.total_pages, 8, 2048 // 16, free_order=cfg3.free_order)
    for s in range(8):
        pool3.ensure_pages(s, 2048 // 16)
    k3c = torch.zeros(cfg3.total_pages, 16, sh3.num_kv_heads, sh3.head_dim, dtype=torch.bfloat16)
    v3c = torch.zeros_like(k3c)
    n3 = 8 * 2048
    k3, v3 = randn((n3, sh3.num_kv_heads, sh3.head_dim)), randn((n3, sh3.num_kv_heads, sh3.head_dim))
    slots3 = torch.from_numpy(orc.slot_mapping(pool3.block_table, np.repeat(np.arange(8), 2048),
                                               np.tile(np.arange(2048), 8)))
    bt3 = torch.from_numpy(pool3.block_table)
    lens3 = [2048] * 8

    # -- configuration 5, one layer
    cfg5 = workloads.config5(seed=seed)
    sh5 = cfg5.shape
    k5c = randn((cfg5.total_pages, 16, sh5.num_kv_heads, sh5.head_dim))
    v5c = randn((cfg5.total_pages, 16, sh5.num_kv_heads, sh5.head_dim))
    victims = torch.tensor(workloads.randperm(cfg5.total_pages, seed + 8)[: cfg5.total_pages // 4],
                           dtype=torch.int32)
    nblk = victims.numel()
    host_img = torch.empty(nblk, 2, sh5.block_bytes, dtype=torch.uint8)
    t_setup = time.perf_counter() - t_setup

    res = {}
    t, reps = _time_op(step, seconds_per_op)
    res["step"] = {"GBps": step_bytes / t / 1e9, "ms": t * 1e3, "reps": reps}
    t, reps = _time_op(lambda: tc.reshape_and_cache(k3, v3, k3c, v3c, slots3), seconds_per_op)
    res["append"] = {"GBps": workloads.append_bytes(n3, sh3.num_kv_heads, sh3.head_dim) / t / 1e9,
                     "ms": t * 1e3, "reps": reps}
    t, reps = _time_op(lambda: tc.gather_kv(k3c, v3c, bt3, lens3), seconds_per_op)
    res["gather"] = {"GBps": workloads.gather_bytes(lens3, sh3.num_kv_heads, sh3.head_dim)
                     / t / 1e9, "ms": t * 1e3, "reps": reps}
    swap_bytes = nblk * 2 * sh5.block_bytes     # bytes each way
    t, reps = _time_op(lambda: tc.gather_blocks(k5c, v5c, victims, out=host_img), seconds_per_op)
    res["swap_out"] = {"GBps": swap_bytes / t / 1e9, "ms": t * 1e3, "reps": reps}
    t, reps = _time_op(lambda: tc.scatter_blocks(host_img, victims, k5c, v5c), seconds_per_op)
    res["swap_in"] = {"GBps": swap_bytes / t / 1e9, "ms": t * 1e3, "reps": reps}

    # numpy oracle, one thread, the configuration-2 layer
    to_u16 = lambda x: x.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    kcn, vcn, knn, vnn, qn = (to_u16(x) for x in (kc, vc, kn, vn, q))
    slots_n = slots.numpy()
    with threadpool_limits(limits=1):
        def np_step():
            orc.reshape_and_cache(knn, vnn, kcn, vcn, slots_n)
            orc.paged_decode(qn, kcn, vcn, indptr, indices, lpl)
        t_np, reps_np = _time_op(np_step, seconds_per_op / 2, min_reps=1)
    torch.set_num_threads(prev_threads)
    total_s = t_setup + sum(v["ms"] * (v["reps"] + 1) for v in res.values()) / 1e3 \
        + t_np * (reps_np + 1)
    log("cpu baseline (torch, %d threads): step %.2f GB/s, append %.2f, gather %.2f, "
        "swap out %.2f / in %.2f GB/s; numpy 1 thread %.2f GB/s; %.1f s"
        % (threads, res["step"]["GBps"], res["append"]["GBps"], res["gather"]["GBps"],
           res["swap_out"]["GBps"], res["swap_in"]["GBps"], step_bytes / t_np / 1e9, total_s))
    return {"value": res["step"]["GBps"], "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": ("torch-CPU restatement of the reference path (oracle/torch_cpu.py), "
                       f"{threads} threads: value = one layer of cfg2 (append 64 rows + fp32 "
                       "decode of 64 seqs over len+1, same algorithmic bytes as `value`); "
                       "ops: cfg3 append/gather of 16,384 tokens, cfg5 swap of one layer's "
                       "4096 victim blocks each way"),
            "ops_GBps": {k: round(v["GBps"], 3) for k, v in res.items()},
            "numpy_oracle_1thread_GBps": step_bytes / t_np / 1e9,
            "seconds": total_s}


# --------------------------------------------------------------- modes
def run_copy_calibration(torch):
    """A plain device-to-device copy of 1 GiB, x5: the FETCH_SIZE /
    WRITE_SIZE calibration for the counter-based traffic figure."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "copy", "bytes_read": n, "bytes_written": n, "launches": 5}), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the paged KV-cache path has no "
              "cross-GPU exchange and this build runs on a single MI355X "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (no CPU fallback)", file=sys.stderr)
        sys.exit(1)
    from gpu_offloading_amd import _lib

    _lib.load()
    torch.cuda.set_device(0)
    if args.mode == "copy":
        run_copy_calibration(torch)
        return
    if args.mode == "decode2":
        run_decode2(torch, args.seed, fused=not args.separate_append)
        return
    if args.mode == "decode4":
        print(json.dumps({"mode": "decode4", **run_cfg4(torch, args.seed)}), flush=True)
        return
    if args.mode == "offload":
        print(json.dumps({"mode": "offload", **run_offload(torch, args.seed)}), flush=True)
        return
    if args.mode == "xpacked":
        print(json.dumps({"mode": "xpacked", **run_xpacked(torch, args.seed)}), flush=True)
        return
    if args.mode == "prefill3":
        print(json.dumps({"mode": "prefill3", **run_prefill(torch, args.seed)}), flush=True)
        return
    if args.mode == "prefill_power":
        print(json.dumps({"mode": "prefill_power", **run_prefill_power(torch, args.seed)}),
              flush=True)
        return
    if args.mode == "bs1":
        print(json.dumps({"mode": "bs1", **run_small_batch(torch, args.seed)}), flush=True)
        return
    if args.mode == "swap5":
        link = run_link_calibration(torch)
        print(json.dumps({"mode": "swap5", "host_link": link, **run_cfg5(torch, args.seed)}),
              flush=True)
        return
    if args.mode == "append3":
        print(json.dumps({"mode": "append3", **run_cfg3(torch, args.seed, layers=1)}), flush=True)
        return

    res = run_step_bench(torch, args)
    extra = {}
    if not args.no_extra:
        extra["cfg3_chunked_prefill"] = run_cfg3(torch, args.seed)
        extra["cfg4_long_context"] = run_cfg4(torch, args.seed)
        link = run_link_calibration(torch)
        extra["host_link"] = link
        extra["cfg5_swap"] = run_cfg5(torch, args.seed)
        for k in ("out", "in"):
            peak = link["d2h_GBps" if k == "out" else "h2d_GBps"]
            extra["cfg5_swap"][f"swap_{k}_frac_of_link"] = round(
                extra["cfg5_swap"][f"swap_{k}_GBps"] / peak, 3)
        extra["f2_continuation_prefill"] = run_prefill(torch, args.seed)
        extra["f2_continuation_prefill"]["second_chunk_sustained"] = run_prefill_power(
            torch, args.seed, seconds=4.0)
        extra["f3_xpacked"] = run_xpacked(torch, args.seed)
        extra["f4_offload"] = run_offload(torch, args.seed)
        extra["bs1_latency"] = run_small_batch(torch, args.seed)
    cpu = None if args.no_cpu else run_cpu_baseline(args.seed)
    line = {
        "metric": "paged decode-attn HBM GB/s (% peak) + KV append/gather/swap GB/s, 1 GPU",
        "value": round(res["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/Q, seeded permuted page pool)",
        "config": {"workload": "cfg2 Mixtral-8x7B-shaped decode step: 32 layers x (append 64 tokens "
                               "+ paged GQA decode), B=64, ctx U[512,4096], Hkv=8, Hq=32, D=128, "
                               "page 16, bf16; value = (decode + append algorithmic bytes) / step "
                               "wall time incl. host setup",
                   "global_batch": 64, "layers": 32, "parallelism": "none (1 GPU)",
                   "append": ("separate reshape_and_cache_flash launch" if args.separate_append
                              else "fused into the decode launch (append_and_decode; cache and "
                                   "output bit-identical to the two calls)")},
        "roofline": res["roofline"],
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
