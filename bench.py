"""Benchmark of the MI355X KV-cache data path (one GPU).

Headline workload (`value`): config 3 of the benchmark plan -- a Qwen3-4B-shape
long-context decode step: 36 layers, 32 query heads, 8 KV heads (GQA 4), head_dim 128,
block_size 16, bf16, batch 16 x 32768-token contexts with random block placement.  One
step = for each layer, append one token per sequence through the slot mapping
(dsp_kv_append), then split-K paged decode attention over the full context
(dsp_paged_decode with its automatic split: on block tables the balanced split-K, every
wave an equal share of the keys, then the log-sum-exp combine).  `value` is decode
attention microseconds per layer.  The same pool is also timed with the fixed 512-token
partitions config 3 names (`c3_fixed512_*`).

Reported beside it on the same JSON line:
  roofline      decode's achieved HBM GB/s = algorithmic bytes per launch (K and V of
                every context token once, plus q, out and the block table) / average
                launch time from HIP events on the launch stream, against 8 TB/s; beside
                it two read ceilings measured in the same run (a streaming read, and the
                decode's access pattern with no arithmetic: dsp_probe_*)
  cpu_baseline  the reference's CPU torch path (gather + repeat_interleave + SDPA) on one
                whole layer of the same workload -- the GPU run's own tensors -- timed on
                this host's cores (median of 5)
  aux           the other configurations, each timed kernel-only with device-resident
                tables: config 2 (decode step), config 4 (copy-on-write fork, suffix
                append, 5-query verify, evict-by-copy), config 5 (gather, map GEMM,
                scatter), a prefill-scale append, skewed decode batches (one long
                context among short ones) with the balanced and the fixed split, and the
                measured streaming-copy ceiling the byte-moving kernels are bounded by.
                The byte movers (copy-on-write, appends, evict, gather, scatter) are timed
                cold -- a 1 GiB fill evicts the L2s and the 256 MB Infinity Cache before
                each call -- with the warm figure beside (`*_warm_GBps`)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-aux]
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

PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0

C3 = dict(layers=36, hq=32, kvh=8, d=128, bs=16, batch=16, ctx=32768)


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def _fill_randn(torch, t, seed: int) -> None:
    g = torch.Generator(device=t.device).manual_seed(seed)
    for i in range(t.shape[0]):
        t[i].normal_(generator=g)


_PROBE = None


def _probe_lib():
    """libdispec_probe.so: the bandwidth probes (bench_probes/dsp_probe.h), measurement
    instruments built beside the product library but not part of it."""
    global _PROBE
    if _PROBE is None:
        import ctypes
        from ctypes import c_int, c_int32, c_int64, c_void_p
        path = os.path.join(ROOT, "bench_probes", "libdispec_probe.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built; run `python -m bench_probes.build` first")
        lib = ctypes.CDLL(path)
        P = c_void_p
        sigs = {"dsp_probe_stream_read": [P, c_int64, c_int32, P, P],
                "dsp_probe_stream_copy": [P, P, c_int64, c_int32, P],
                "dsp_probe_slice_read": [P, P, c_int64, P, c_int64, c_int32, c_int32, c_int32,
                                         c_int32, c_int32, P, P],
                "dsp_probe_gemm_fill": [P, c_int64, c_int64, c_int64, P, c_int64, c_int64,
                                        c_int64, c_int32, P, P],
                "dsp_probe_piece_scatter": [P, P, c_int64, c_int64, P, P],
                "dsp_probe_piece_gather": [P, P, c_int64, c_int64, P, P],
                "dsp_probe_batch_read": [P, P, c_int64, P, c_int64, c_int32, P, P, c_int32,
                                         c_int32, P, P],
                "dsp_probe_piece_fill": [P, c_int64, c_int64, P, P]}
        for name, args in sigs.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = c_int, args
        _PROBE = lib
    return _PROBE


def _time_gpu(torch, fn, iters: int, warmup: int = 2) -> float:
    """Average seconds per call of fn, HIP events on torch's current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = _events(torch)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters / 1e3


_FLUSH = None


def _time_gpu_cold(torch, fn, iters: int, warmup: int = 1) -> float:
    """Average seconds per call of fn with the caches cold: before each call a 1 GiB fill
    evicts the L2s and the 256 MB Infinity Cache (MALL), and HIP events bracket fn alone.
    The fill is enqueued ahead of fn, so the GPU stays busy while the host launches fn."""
    global _FLUSH
    if _FLUSH is None:
        _FLUSH = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
    for _ in range(warmup):
        fn()
    ev = [_events(torch) for _ in range(iters)]
    torch.cuda.synchronize()
    for a, b in ev:
        _FLUSH.fill_(1.0)
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in ev) / iters / 1e3


# ------------------------------------------------------------------------------ config 3
def bench_decode(torch, steps: int, warmup: int, keep_cpu_sample: bool = False) -> dict:
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    from dispec_amd.kv.paged_cache import PagedKVCache

    c = C3
    L, Hq, KVH, D, bs, B, ctx = (c[k] for k in ("layers", "hq", "kvh", "d", "bs", "batch", "ctx"))
    dev = "cuda"
    nb_seq = ctx // bs
    NB = B * nb_seq
    _log(f"config 3: {L}-layer pool of {NB} blocks ({2 * L * NB * bs * KVH * D * 2 / 1e9:.1f} GB)")
    cache = PagedKVCache(L, NB, bs, KVH, D, dtype=torch.bfloat16, device=dev)
    _fill_randn(torch, cache.key, 3001)
    _fill_randn(torch, cache.value, 3002)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3003))
    tables = perm.view(B, nb_seq).to(torch.int32)
    bt = tables.to(dev)
    g = torch.Generator(device=dev).manual_seed(3004)
    q = torch.randn((L, B, Hq, D), generator=g, device=dev).to(torch.bfloat16)
    k_new = torch.randn((L, B, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    v_new = torch.randn((L, B, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    pos = ctx - 1
    wslots = (tables[:, pos // bs].long() * bs + pos % bs).to(dev)
    ctx_lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    out = torch.empty((L, B, Hq, D), dtype=torch.bfloat16, device=dev)
    lib = _lib.lib()
    # automatic split (0): on block tables the balanced split-K, equal key shares per wave
    P = 0
    ws_bytes = max(lib.dsp_paged_decode_workspace_bytes(B, Hq, KVH, D, ctx, p) for p in (0, 512))
    ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=dev)

    def step(ev=None, part=P):
        for layer in range(L):
            cache.write(layer, wslots, k_new[layer], v_new[layer])
            if ev is not None:
                ev[layer][0].record()
            paged_decode_attention_blocks(q[layer], cache.key[layer], cache.value[layer], bt,
                                          ctx_lens, Hq // KVH, block_size=bs, max_ctx=ctx,
                                          partition_tokens=part, out=out[layer], workspace=ws)
            if ev is not None:
                ev[layer][1].record()

    _log(f"config 3: warmup {warmup} steps, balanced split-K")
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    cache.check_errors()
    ev = [list(_events(torch)) for _ in range(L)]
    decode_ms = []
    t0, t1 = _events(torch)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(steps):
        step(ev)
        torch.cuda.synchronize()
        decode_ms.extend(e[0].elapsed_time(e[1]) for e in ev)
    t1.record()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    _log(f"config 3: {steps} steps in {total_ms:.1f} ms")
    alg_bytes = B * ctx * KVH * D * 2 * 2 + 2 * B * Hq * D * 2 + B * nb_seq * 4
    avg_s = statistics.mean(decode_ms) / 1e3
    assert torch.isfinite(out).all()
    # Read ceilings on this GPU, same run: a streaming read of two layers' K (2.15 GB), and
    # the decode's access pattern (one KV head's 256-byte row slice per key, through the
    # block table) over layer 0 with no arithmetic.
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    span = cache.key[0:2]
    probe = _probe_lib()

    def stream_probe():
        _lib.check(probe.dsp_probe_stream_read(span.data_ptr(), span.numel() * 2, 8192,
                                             sink.data_ptr(), stream), "probe")

    def slice_probe(waves):
        _lib.check(probe.dsp_probe_slice_read(cache.key[0].data_ptr(), cache.value[0].data_ptr(),
                                            cache.key.shape[1], bt.data_ptr(), bt.stride(0), bs,
                                            B, KVH, ctx, waves, sink.data_ptr(), stream), "probe")
    stream_s = _time_gpu(torch, stream_probe, 10)
    # best of 256, 512 and 1024 workgroups of 4 waves (one, two and four per CU): the
    # decode's access pattern, 4 heads of each slot row read side by side
    slice_s = min(_time_gpu(torch, lambda: slice_probe(w), 10) for w in (8, 16, 32))
    read_ceiling = span.numel() * 2 / stream_s / 1e9
    pattern_ceiling = B * ctx * KVH * D * 2 * 2 / slice_s / 1e9

    # Config 3 as literally stated (fixed 512-token partitions + LSE combine), same pool.
    fixed_ms = []
    for _ in range(max(1, min(warmup, 3))):
        step(part=512)
    torch.cuda.synchronize()
    for _ in range(steps):
        step(ev, part=512)
        torch.cuda.synchronize()
        fixed_ms.extend(e[0].elapsed_time(e[1]) for e in ev)
    cache.check_errors()
    fixed_s = statistics.mean(fixed_ms) / 1e3
    if keep_cpu_sample:
        # layer 0 exactly as the GPU read it in the last timed step (appended token
        # included): the CPU baseline runs on these same bytes
        res_sample = dict(k=cache.key[0].cpu(), v=cache.value[0].cpu(), q=q[0].cpu(),
                          tables=tables.clone())
    res = dict(us_per_layer=avg_s * 1e6, median_us_per_layer=statistics.median(decode_ms) * 1e3,
               ms_per_step=total_ms / steps, alg_bytes=alg_bytes,
               achieved_gbps=alg_bytes / avg_s / 1e9, split="balanced",
               fixed512_us_per_layer=fixed_s * 1e6,
               fixed512_GBps=alg_bytes / fixed_s / 1e9,
               read_ceiling_GBps=read_ceiling, pattern_ceiling_GBps=pattern_ceiling)
    if keep_cpu_sample:
        res["cpu_sample"] = res_sample
    del cache, q, k_new, v_new, out, ws
    torch.cuda.empty_cache()
    return res


def bench_cpu_baseline(torch, sample) -> dict:
    """The reference's CPU torch path for config 3 (per-sequence gather + repeat_interleave
    + SDPA, ref_torch.decode_repeat_kv_sdpa, in bf16) on one whole layer of the GPU run:
    the same 16 x 32768 block tables, q and K/V bytes the GPU decoded in its last timed
    step, on every host core this process may use.  One warmup, then the median of 5."""
    from oracle import ref_torch

    c = C3
    Hq, KVH, bs, ctx, B = c["hq"], c["kvh"], c["bs"], c["ctx"], c["batch"]
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    kc, vc, q, tables = sample["k"], sample["v"], sample["q"], sample["tables"]
    slot_lists = [(tables[b].long()[:, None] * bs + torch.arange(bs)[None]).reshape(-1)[:ctx]
                  for b in range(B)]
    times = []
    for _ in range(6):
        t = time.perf_counter()
        ref_torch.decode_repeat_kv_sdpa(q, kc, vc, slot_lists, Hq // KVH)
        times.append(time.perf_counter() - t)
    per_layer = statistics.median(times[1:])
    return dict(value=round(per_layer * 1e6, 1), unit="us/layer", cores=cores,
                torch_threads=torch.get_num_threads(), kind="port",
                sample=f"config 3, one whole layer ({B} x {ctx} tokens, the GPU run's own "
                       f"layer-0 tensors), median of 5 after 1 warmup",
                cpu_model=_cpu_model(), transport=_xfer_reference(torch))


def _xfer_reference(torch) -> dict:
    """The reference's TCP handoff (torch.save pickle of CPU copies, bytearray receive,
    torch.load, .to(device): dispec/transport/tcp.py:19-36, 61-70) on the same payload and
    loopback connection as bench_xfer, with the same export and import kernels."""
    import threading

    from oracle import ref_torch
    x = _xfer_setup(torch)

    def step():
        k, v = x["src"].export_contiguous(x["src_ids"], len(x["tokens"]))
        th = threading.Thread(target=ref_torch.tcp_send_pickle,
                              args=(x["a"], x["tokens"], k, v, {"request_id": 1}))
        th.start()
        _, k2, v2, _ = ref_torch.tcp_recv_pickle(x["b"], "cuda")
        th.join()
        x["dst"].import_contiguous(x["dst_ids"], k2, v2)

    t = _xfer_time(torch, step, iters=2)
    x["a"].close()
    x["b"].close()
    res = {"GBps": round(x["payload_bytes"] / t / 1e9, 3), "ms": round(t * 1e3, 1),
           "sample": "one 4096-token, 28-layer payload (470 MB), loopback TCP, median of 2"}
    del x
    torch.cuda.empty_cache()
    return res


def _cpu_model() -> str:
    """`lscpu`'s model name (the /proc/cpuinfo line if lscpu is missing)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ------------------------------------------------------------------------------ config 2
def bench_c2(torch) -> dict:
    """Qwen2.5-1.5B decode step: 28 layers, Hq 12, KVH 2, D 128, B 64, ctx ~U[512, 4096],
    blocks scattered over a pool of 1.25x the tokens; per layer append + decode."""
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    from dispec_amd.kv.paged_cache import PagedKVCache

    L, Hq, KVH, D, bs, B = 28, 12, 2, 128, 16, 64
    dev = "cuda"
    gcpu = torch.Generator().manual_seed(2001)
    ctx = torch.randint(512, 4097, (B,), generator=gcpu)
    need = [-(-int(n) // bs) for n in ctx]
    NB = int(sum(need) * 1.25)
    cache = PagedKVCache(L, NB, bs, KVH, D, device=dev)
    _fill_randn(torch, cache.key, 2002)
    _fill_randn(torch, cache.value, 2003)
    perm = torch.randperm(NB, generator=gcpu).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    bt = cache.block_table(tables)
    ctx_lens = ctx.to(torch.int32).to(dev)
    g = torch.Generator(device=dev).manual_seed(2004)
    q = torch.randn((L, B, Hq, D), generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn((L, B, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn((L, B, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    wslots = torch.tensor([t[(int(n) - 1) // bs] * bs + (int(n) - 1) % bs
                           for t, n in zip(tables, ctx)], device=dev)
    out = torch.empty((L, B, Hq, D), dtype=torch.bfloat16, device=dev)
    max_ctx = int(ctx.max())

    def step():
        for layer in range(L):
            cache.write(layer, wslots, kn[layer], vn[layer])
            paged_decode_attention_blocks(q[layer], cache.key[layer], cache.value[layer], bt,
                                          ctx_lens, Hq // KVH, block_size=bs, max_ctx=max_ctx,
                                          out=out[layer])

    def decode_only():
        for layer in range(L):
            paged_decode_attention_blocks(q[layer], cache.key[layer], cache.value[layer], bt,
                                          ctx_lens, Hq // KVH, block_size=bs, max_ctx=max_ctx,
                                          out=out[layer])

    step_s = _time_gpu(torch, step, 5)
    dec_s = _time_gpu(torch, decode_only, 5) / L
    # the floor of the decode: the same layers' K/V read with no arithmetic, every
    # sequence cut into equal 256-key pieces (dsp_probe_batch_read), same 28-layer loop
    work = torch.tensor([[b, k0] for b, n in enumerate(ctx.tolist()) for k0 in range(0, n, 256)],
                        dtype=torch.int32).to(dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    probe = _probe_lib()
    stream = torch.cuda.current_stream().cuda_stream

    def read_only():
        for layer in range(L):
            _lib.check(probe.dsp_probe_batch_read(
                cache.key[layer].data_ptr(), cache.value[layer].data_ptr(), cache.num_slots,
                bt.data_ptr(), bt.stride(0), bs, ctx_lens.data_ptr(), work.data_ptr(),
                work.shape[0], KVH, sink.data_ptr(), stream), "probe")

    floor_s = _time_gpu(torch, read_only, 5) / L
    # the append at bandwidth scale (BASELINE's append row): every sequence's whole
    # context written as a prefill would write it, through the same block tables -- runs
    # of 16 consecutive slots per randomly placed block -- one launch for the layer
    cslots = torch.cat([cache.context_slots(t, int(n)) for t, n in zip(tables, ctx)])
    n_rows = cslots.numel()
    kp = torch.randn((n_rows, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn((n_rows, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    app_s = _time_gpu_cold(torch, lambda: cache.write(5, cslots, kp, vp), 20)
    app_warm_s = _time_gpu(torch, lambda: cache.write(5, cslots, kp, vp), 20)
    cache.check_errors()
    kv_bytes = int(ctx.sum()) * KVH * D * 2 * 2
    app_bytes = 2 * 2 * n_rows * cache.row_bytes
    res = {"c2_step_us_per_layer": step_s / L * 1e6, "c2_decode_us_per_layer": dec_s * 1e6,
           "c2_decode_GBps": kv_bytes / dec_s / 1e9,
           "c2_read_floor_us_per_layer": floor_s * 1e6,
           "c2_read_floor_GBps": kv_bytes / floor_s / 1e9,
           "c2_append_prefill_rows": n_rows, "c2_append_prefill_us": app_s * 1e6,
           "c2_append_prefill_GBps": app_bytes / app_s / 1e9,
           "c2_append_prefill_warm_GBps": app_bytes / app_warm_s / 1e9}
    # roofline object of the decode launch (balanced kernel + merge) against HBM: the
    # contexts' K and V read once, plus q, out, block table and lengths; traffic from the
    # counter passes in profiles/decode_c2_traffic.md
    alg = kv_bytes + 2 * B * Hq * D * 2 + bt.numel() * 4 + B * 4
    res["c2_decode_roofline"] = {
        "bound": "hbm", "achieved": round(alg / dec_s / 1e9, 1), "peak": PEAK_HBM_GBPS,
        "unit": "GB/s", "frac": round(alg / dec_s / 1e9 / PEAK_HBM_GBPS, 4),
        "traffic": _traffic_per_launch("decode_c2_traffic.md"), "alg_bytes_per_launch": alg}
    del cache, kp, vp
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------ skewed decode batches
def bench_skew(torch) -> dict:
    """Decode batches with uneven contexts (the serving case config 3's uniform batch does
    not show), Qwen3-4B heads (Hq 32, KVH 8, D 128): 'skew' = one 32768-token context beside
    15 of 512; 'mixed' = 32 contexts ~U[16, 2048) with one of 16384.  Timed with the
    automatic split (balanced: equal key shares per wave) and with fixed 1024-token
    partitions over a loop of 16 layers of their own K/V, as a model's step reads them (one
    layer's 165-200 MB would otherwise stay in the 256 MB Infinity Cache between launches);
    per-layer time = loop time / 16, HIP events around the loop."""
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks

    dev, Hq, KVH, D, bs, L = "cuda", 32, 8, 128, 16, 16
    gcpu = torch.Generator().manual_seed(4001)
    mixed = torch.randint(16, 2048, (32,), generator=gcpu).tolist()
    mixed[3] = 16384
    res = {}
    for name, ctxs in (("skew", [32768] + [512] * 15), ("mixed", mixed)):
        B = len(ctxs)
        need = [-(-c // bs) for c in ctxs]
        NB = int(sum(need) * 1.25) + 8
        kc = torch.empty((L, NB * bs, KVH, D), dtype=torch.bfloat16, device=dev)
        vc = torch.empty_like(kc)
        _fill_randn(torch, kc, 4002)
        _fill_randn(torch, vc, 4003)
        perm = torch.randperm(NB, generator=gcpu).tolist()
        bt = torch.zeros((B, max(need)), dtype=torch.int32)
        at = 0
        for i, n in enumerate(need):
            bt[i, :n] = torch.tensor(perm[at:at + n])
            at += n
        bt = bt.to(dev)
        ctx = torch.tensor(ctxs, dtype=torch.int32, device=dev)
        q = torch.randn((B, Hq, D), generator=torch.Generator(device=dev).manual_seed(4004),
                        device=dev).to(torch.bfloat16)
        out = torch.empty_like(q)
        lib = _lib.lib()
        wsb = max(lib.dsp_paged_decode_workspace_bytes(B, Hq, KVH, D, max(ctxs), p)
                  for p in (0, 1024))
        ws = torch.empty(wsb // 4 + 1, dtype=torch.float32, device=dev)
        kv_bytes = sum(ctxs) * KVH * D * 2 * 2
        for label, P in (("balanced", 0), ("fixed1024", 1024)):
            def f():
                for layer in range(L):
                    paged_decode_attention_blocks(q, kc[layer], vc[layer], bt, ctx, Hq // KVH,
                                                  block_size=bs, max_ctx=max(ctxs),
                                                  partition_tokens=P, out=out, workspace=ws)
            us = _time_gpu(torch, f, 5) / L * 1e6
            res[f"{name}_{label}_us"] = us
            res[f"{name}_{label}_GBps"] = kv_bytes / us / 1e3
        del kc, vc
        torch.cuda.empty_cache()
    res.update(_verify_skew(torch))
    return res


def _verify_skew(torch) -> dict:
    """A 5-query verify (Qwen3-1.7B heads: Hq 16, KVH 8, D 128) over one 32768-token context
    beside 15 of 512: the balanced split-K kernel (what ModelRunner picks for such a batch)
    against the fixed key partitions the library sizes from max_ctx; a loop over 16 layers
    of their own K/V, as for the decode batches above."""
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_mq_attention

    dev, Hq, KVH, D, bs, ql, L = "cuda", 16, 8, 128, 16, 5, 16
    ctxs = [32768] + [512] * 15
    B = len(ctxs)
    need = [-(-c // bs) for c in ctxs]
    NB = int(sum(need) * 1.25) + 8
    kc = torch.empty((L, NB * bs, KVH, D), dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    _fill_randn(torch, kc, 4005)
    _fill_randn(torch, vc, 4006)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(4007)).tolist()
    bt = torch.zeros((B, max(need)), dtype=torch.int32)
    at = 0
    for i, n in enumerate(need):
        bt[i, :n] = torch.tensor(perm[at:at + n])
        at += n
    bt = bt.to(dev)
    ctx = torch.tensor(ctxs, dtype=torch.int32, device=dev)
    cu = torch.arange(0, (B + 1) * ql, ql, dtype=torch.int32, device=dev)
    q = torch.randn((B * ql, Hq, D), generator=torch.Generator(device=dev).manual_seed(4008),
                    device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    lib = _lib.lib()
    wsb = max(lib.dsp_paged_mq_workspace_bytes(B, Hq, KVH, D, ql, max(ctxs), p)
              for p in (0, _lib.DSP_SPLIT_BALANCED))
    ws = torch.empty(wsb // 4 + 1, dtype=torch.float32, device=dev)
    kv_bytes = sum(ctxs) * KVH * D * 2 * 2
    res = {}
    for label, bal in (("balanced", True), ("partitioned", False)):
        def f():
            for layer in range(L):
                paged_mq_attention(q, kc[layer], vc[layer], bt, cu, ctx, Hq // KVH,
                                   block_size=bs, max_q_len=ql, max_ctx=max(ctxs), out=out,
                                   workspace=ws, balanced=bal)
        us = _time_gpu(torch, f, 5) / L * 1e6
        res[f"verify_skew_{label}_us"] = us
        res[f"verify_skew_{label}_GBps"] = kv_bytes / us / 1e3
    del kc, vc
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------------------ config 1
def bench_c1(torch) -> dict:
    """Qwen2-0.5B shape, one layer: Hq 14, KVH 2 (G 7), D 64, a 256-block pool, contexts
    {37, 128, 255, 511} plus the token appended this step; append + decode.  Launch-bound:
    the times include the Python wrappers' host work between launches (0.48 MB of K/V)."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    from dispec_amd.kv.paged_cache import PagedKVCache

    Hq, KVH, D, bs, NB = 14, 2, 64, 16, 256
    dev = "cuda"
    lens = [38, 129, 256, 512]
    gcpu = torch.Generator().manual_seed(1001)
    perm = torch.randperm(NB, generator=gcpu).tolist()
    tables, at = [], 0
    for n in lens:
        k = -(-n // bs)
        tables.append(perm[at:at + k])
        at += k
    cache = PagedKVCache(1, NB, bs, KVH, D, device=dev)
    _fill_randn(torch, cache.key, 1002)
    _fill_randn(torch, cache.value, 1003)
    bt = cache.block_table(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(1004)
    q = torch.randn((len(lens), Hq, D), generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn((len(lens), KVH, D), generator=g, device=dev).to(torch.bfloat16)
    slots = torch.tensor([t[(n - 1) // bs] * bs + (n - 1) % bs for t, n in zip(tables, lens)],
                         device=dev)
    out = torch.empty_like(q)

    def step():
        cache.write(0, slots, kn, kn)
        paged_decode_attention_blocks(q, cache.key[0], cache.value[0], bt, ctx, Hq // KVH,
                                      block_size=bs, max_ctx=max(lens), out=out)

    def decode():
        paged_decode_attention_blocks(q, cache.key[0], cache.value[0], bt, ctx, Hq // KVH,
                                      block_size=bs, max_ctx=max(lens), out=out)

    st = _time_gpu(torch, step, 50, warmup=5)
    dec = _time_gpu(torch, decode, 50, warmup=5)
    cache.check_errors()
    kv_bytes = sum(lens) * KVH * D * 2 * 2
    del cache
    return {"c1_step_us": st * 1e6, "c1_decode_us": dec * 1e6,
            "c1_decode_GBps": kv_bytes / dec / 1e9}


def bench_graph(torch) -> dict:
    """Whole-model decode step of the reference's draft model shape (Qwen2.5-0.5B: 24
    layers, hidden 896, Hq 14, KVH 2, D 64, vocab 151936), random-init bf16 weights:
    eager ModelRunner.forward + logits against HipGraphDecoder replays, batch 1 and 16,
    every sequence at 512 tokens of context.  Times are per step, host work included."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from dispec_amd.engine.hip_graph import HipGraphDecoder
    from dispec_amd.engine.model_runner import ModelRunner, SeqMeta
    from dispec_amd.kv.paged_cache import PagedKVCache

    dev, bs, ctx = "cuda", 16, 512
    cfg = Qwen2Config(vocab_size=151936, hidden_size=896, intermediate_size=4864,
                      num_hidden_layers=24, num_attention_heads=14, num_key_value_heads=2,
                      max_position_embeddings=32768, tie_word_embeddings=True)
    torch.manual_seed(2001)
    with torch.device(dev):
        model = Qwen2ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval().requires_grad_(False)
    runner = ModelRunner(model, attn_backend="hip")
    out = {}
    for B in (1, 16):
        W = ctx // bs
        cache = PagedKVCache.for_model(cfg, B * W, bs, torch.bfloat16, dev)
        _fill_randn(torch, cache.key, 2002)
        _fill_randn(torch, cache.value, 2003)
        tables = [list(range(b * W, (b + 1) * W)) for b in range(B)]
        meta = [SeqMeta(t, 1, ctx) for t in tables]
        toks = [7 + b for b in range(B)]
        pos = [ctx - 1] * B
        slots = [t[-1] * bs + bs - 1 for t in tables]
        tt, pt, st = (torch.tensor(x, device=dev) for x in (toks, pos, slots))
        graph = HipGraphDecoder(runner, cache, buckets=(ctx,))
        graph.capture(batch_sizes=(B,))

        def eager():
            runner.logits(runner.forward(tt, pt, st, meta, cache))

        def replay():
            graph.decode_batch(toks, pos, slots, meta)

        e = _time_gpu(torch, eager, 30, warmup=3)
        g = _time_gpu(torch, replay, 30, warmup=3)
        cache.check_errors()
        out[f"graph_b{B}_eager_ms"] = e * 1e3
        out[f"graph_b{B}_replay_ms"] = g * 1e3
        del graph, cache
    return out


# ------------------------------------------------------------------------------ config 4
def bench_c4(torch) -> dict:
    """Qwen3-1.7B shape (28 L, Hq 16, KVH 8, D 128): 32 sequences share a 2050-token
    prefix, fork it copy-on-write (the partial block is copied per sequence), append
    suffixes ~U[64, 512], run a 5-query causal verify over the paged cache (with the shared
    prompt blocks attended once for the batch, and per sequence for comparison) and a
    one-query decode step the same two ways, then evict 10% of the live blocks by copying
    them into a spill pool."""
    from dispec_amd.engine.hip_attn import (decode_workspace, paged_decode_attention_blocks,
                                           paged_mq_attention)
    from dispec_amd.kv.paged_cache import PagedKVCache

    L, Hq, KVH, D, bs, S, prefix, K = 28, 16, 8, 128, 16, 32, 2050, 5
    dev = "cuda"
    gcpu = torch.Generator().manual_seed(4001)
    suffix = torch.randint(64, 513, (S,), generator=gcpu).tolist()
    NB = 1536
    cache = PagedKVCache(L, NB, bs, KVH, D, device=dev)
    mgr = cache.manager
    owner = 1000
    mgr.allocate(owner, prefix)
    g = torch.Generator(device=dev).manual_seed(4002)
    pk = torch.randn((prefix, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    pslots = cache.context_slots(mgr.block_table(owner).block_ids, prefix)
    for layer in range(L):
        cache.write(layer, pslots, pk, pk)
    # copy-on-write fork of the partial last block for every sequence
    pairs = []
    for s in range(S):
        _, p = mgr.cow_fork(owner, s)
        pairs += p
    # every pair copies the prompt's one partial block: copy_blocks routes such a list to the
    # fan-out copy (the id list already on the GPU here, as a captured step would have it)
    assert len({p[0] for p in pairs}) == 1
    dst = torch.tensor([p[1] for p in pairs], dtype=torch.int32, device=dev)
    fork_src = pairs[0][0]
    cow_s = _time_gpu_cold(torch, lambda: cache.copy_block_fanout_device(cache, fork_src, dst),
                           20)
    cow_warm_s = _time_gpu(torch, lambda: cache.copy_block_fanout_device(cache, fork_src, dst),
                           20)
    # HBM bytes the fork moves: each copy's block written, the source block read once per
    # group of 8 copies (the fan-out kernel loads a piece once and stores it 8 times)
    fan = 8
    cow_hbm_bytes = 2 * L * cache.block_bytes * (len(pairs) + -(-len(pairs) // fan))
    # suffix + draft tokens: one append per layer for all 32 sequences
    rows, wslots = [], []
    for s in range(S):
        for _ in range(suffix[s] + K):
            blk, off = mgr.append_token(s)
            wslots.append(blk * bs + off)
        rows.append(suffix[s] + K)
    wslots_t = torch.tensor(wslots, device=dev)
    n = len(wslots)
    kr = torch.randn((n, KVH, D), generator=g, device=dev).to(torch.bfloat16)
    app_s = _time_gpu_cold(torch, lambda: cache.write(3, wslots_t, kr, kr), 20)
    app_warm_s = _time_gpu(torch, lambda: cache.write(3, wslots_t, kr, kr), 20)
    # 5-query verify over ctx = prefix + suffix + 5
    ctx = [prefix + suffix[s] + K for s in range(S)]
    bt = cache.block_table([mgr.block_table(s).block_ids for s in range(S)])
    cu = torch.arange(0, (S + 1) * K, K, dtype=torch.int32, device=dev)
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
    q = torch.randn((L, S * K, Hq, D), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty((L, S * K, Hq, D), dtype=torch.bfloat16, device=dev)
    max_ctx = bt.shape[1] * bs

    # the 128 full prompt blocks are shared by every fork: ModelRunner passes them as a
    # shared prefix (2048 tokens), attended once for the batch; "plain" attends each
    # sequence over its whole context
    shared_tokens = (prefix // bs) * bs // 128 * 128

    def verify(sp):
        for layer in range(L):
            paged_mq_attention(q[layer], cache.key[layer], cache.value[layer], bt, cu, ctx_t,
                               Hq // KVH, block_size=bs, max_q_len=K, max_ctx=max_ctx,
                               out=out[layer], shared_prefix_tokens=sp)

    ver_s = _time_gpu(torch, lambda: verify(shared_tokens), 10) / L
    plain_s = _time_gpu(torch, lambda: verify(0), 10) / L

    # a decode step of the forks (one query row each): shared-prefix multi-query kernel,
    # as ModelRunner routes it, against the per-sequence decode kernel
    cu1 = torch.arange(S + 1, dtype=torch.int32, device=dev)
    q1, out1 = q[:, :S], out[:, :S]
    ws1 = decode_workspace(S, Hq, KVH, D, max_ctx, dev)

    def decode(sp):
        for layer in range(L):
            if sp:
                paged_mq_attention(q1[layer], cache.key[layer], cache.value[layer], bt, cu1,
                                   ctx_t, Hq // KVH, block_size=bs, max_q_len=1,
                                   max_ctx=max_ctx, out=out1[layer], shared_prefix_tokens=sp)
            else:
                paged_decode_attention_blocks(q1[layer], cache.key[layer], cache.value[layer],
                                              bt, ctx_t, Hq // KVH, block_size=bs,
                                              max_ctx=max_ctx, out=out1[layer], workspace=ws1)

    dec_s = _time_gpu(torch, lambda: decode(shared_tokens), 10) / L
    dec_plain_s = _time_gpu(torch, lambda: decode(0), 10) / L
    shared = (prefix // bs) * bs          # full prefix blocks, read by every sequence
    unique_tokens = shared + sum(c - shared for c in ctx)
    logical_tokens = sum(ctx)
    flops = 4 * sum(ctx) * K * Hq * D
    # evict 10% of live blocks by copying them into a spill pool
    live = sorted({b for s in range(S) for b in mgr.block_table(s).block_ids}
                  | set(mgr.block_table(owner).block_ids))
    nev = max(1, len(live) // 10)
    spill = PagedKVCache(L, nev, bs, KVH, D, device=dev)
    esrc = torch.tensor(live[:nev], dtype=torch.int32, device=dev)
    edst = torch.arange(nev, dtype=torch.int32, device=dev)
    ev_s = _time_gpu_cold(torch, lambda: spill.copy_blocks_device(cache, esrc, edst), 20)
    ev_warm_s = _time_gpu(torch, lambda: spill.copy_blocks_device(cache, esrc, edst), 20)
    cache.check_errors()
    spill.check_errors()
    res = {
        "c4_cow_pairs": len(pairs), "c4_cow_us": cow_s * 1e6, "c4_cow_hbm_bytes": cow_hbm_bytes,
        "c4_cow_GBps": cow_hbm_bytes / cow_s / 1e9,
        "c4_cow_warm_GBps": cow_hbm_bytes / cow_warm_s / 1e9,
        "c4_append_rows": n, "c4_append_GBps": 2 * 2 * n * cache.row_bytes / app_s / 1e9,
        "c4_append_warm_GBps": 2 * 2 * n * cache.row_bytes / app_warm_s / 1e9,
        "c4_verify_us_per_layer": ver_s * 1e6,
        "c4_verify_shared_prefix_tokens": shared_tokens,
        "c4_verify_plain_us_per_layer": plain_s * 1e6,
        "c4_verify_unique_GBps": unique_tokens * KVH * D * 4 / ver_s / 1e9,
        "c4_verify_logical_GBps": logical_tokens * KVH * D * 4 / ver_s / 1e9,
        "c4_verify_TFLOPs": flops / ver_s / 1e12,
        "c4_fork_decode_us_per_layer": dec_s * 1e6,
        "c4_fork_decode_plain_us_per_layer": dec_plain_s * 1e6,
        "c4_evict_blocks": nev, "c4_evict_us": ev_s * 1e6,
        "c4_evict_GBps": 2 * 2 * L * nev * cache.block_bytes / ev_s / 1e9,
        "c4_evict_warm_GBps": 2 * 2 * L * nev * cache.block_bytes / ev_warm_s / 1e9,
    }
    # roofline object of the shared-prefix verify launch (attention + merge) against HBM:
    # the unique K/V (shared prompt once, each sequence's own tokens once), q and out;
    # traffic from the counter passes in profiles/verify_c4_traffic.md
    alg = unique_tokens * KVH * D * 4 + 2 * S * K * Hq * D * 2
    res["c4_verify_roofline"] = {
        "bound": "hbm", "achieved": round(alg / ver_s / 1e9, 1), "peak": PEAK_HBM_GBPS,
        "unit": "GB/s", "frac": round(alg / ver_s / 1e9 / PEAK_HBM_GBPS, 4),
        "traffic": _traffic_per_launch("verify_c4_traffic.md", "c4_verify"),
        "alg_bytes_per_launch": alg}
    del cache, spill
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------------------ prefill
def bench_prefill(torch) -> dict:
    """Long query blocks over the paged cache (the 128-row prefill tile): Qwen3-4B heads
    (Hq 32, KVH 8, D 128), blocks of 16 at random places.  `chunk`: 4 sequences whose last
    512 of 4096 tokens are a prefill chunk; `fresh`: 2 sequences of 2048 tokens prefilled
    at once.  FLOPs count the causal keys only (4 * Hq * D per query-key pair).  torch's
    SDPA on contiguous K/V of the same shape is timed beside it for reference."""
    from torch.nn.attention.bias import causal_lower_right

    from dispec_amd.engine.hip_attn import paged_mq_attention
    res = {}
    dev = "cuda"
    for name, B, q_len, ctx in (("chunk", 4, 512, 4096), ("fresh", 2, 2048, 2048)):
        Hq, KVH, D, bs = 32, 8, 128, 16
        nbs = ctx // bs
        NB = B * nbs + 8
        g = torch.Generator(device=dev).manual_seed(6001)
        kc = torch.randn((NB * bs, KVH, D), generator=g, device=dev).to(torch.bfloat16)
        vc = torch.randn((NB * bs, KVH, D), generator=g, device=dev).to(torch.bfloat16)
        perm = torch.randperm(NB, generator=torch.Generator().manual_seed(6002))[:B * nbs]
        bt = perm.view(B, nbs).to(torch.int32).to(dev)
        q = torch.randn((B * q_len, Hq, D), generator=g, device=dev).to(torch.bfloat16)
        cu = torch.arange(0, B + 1, dtype=torch.int32, device=dev) * q_len
        ctx_t = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        out = torch.empty_like(q)
        fn = lambda: paged_mq_attention(q, kc, vc, bt, cu, ctx_t, Hq // KVH,  # noqa: E731
                                        block_size=bs, max_q_len=q_len, max_ctx=ctx, out=out)
        t = _time_gpu(torch, fn, 50, warmup=30)
        keys = q_len * (ctx - q_len) + q_len * (q_len + 1) // 2
        flops = 4 * B * Hq * D * keys
        qq = q.view(B, q_len, Hq, D).transpose(1, 2).contiguous()
        kk = torch.randn((B, Hq, ctx, D), generator=g, device=dev).to(torch.bfloat16)
        vv = torch.randn_like(kk)
        mask = causal_lower_right(q_len, ctx)
        ts = _time_gpu(torch, lambda: torch.nn.functional.scaled_dot_product_attention(
            qq, kk, vv, attn_mask=mask), 50, warmup=10)
        res.update({f"prefill_{name}_us": t * 1e6, f"prefill_{name}_TFLOPs": flops / t / 1e12,
                    f"prefill_{name}_mfma_frac": flops / t / 1e12 / PEAK_BF16_TFLOPS,
                    f"prefill_{name}_torch_sdpa_contiguous_us": ts * 1e6})
        del kc, vc, kk, vv
        torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------------------ transport
def _xfer_setup(torch):
    """One escalation payload of config 5's source model (Qwen3-1.7B: 28 layers, 8 KV heads,
    head_dim 128) for a 4096-token request, exported from a pool with random block
    placement, and a second pool to import it into; a loopback TCP connection."""
    import socket

    from dispec_amd.kv.paged_cache import PagedKVCache
    L, KVH, D, bs, T = 28, 8, 128, 16, 4096
    dev = "cuda"
    nb = T // bs
    src = PagedKVCache(L, nb + 8, bs, KVH, D, device=dev)
    dst = PagedKVCache(L, nb + 8, bs, KVH, D, device=dev)
    _fill_randn(torch, src.key, 5101)
    _fill_randn(torch, src.value, 5102)
    g = torch.Generator().manual_seed(5103)
    src_ids = torch.randperm(nb + 8, generator=g)[:nb].tolist()
    dst_ids = torch.randperm(nb + 8, generator=g)[:nb].tolist()
    tokens = torch.randint(0, 150_000, (T,), generator=g).tolist()
    srv = socket.socket(socket.AF_INET, socket.SOCK_STREAM)
    srv.bind(("127.0.0.1", 0))
    srv.listen(1)
    a = socket.create_connection(srv.getsockname())
    b, _ = srv.accept()
    srv.close()
    for s in (a, b):
        s.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)
    return dict(src=src, dst=dst, src_ids=src_ids, dst_ids=dst_ids, tokens=tokens, a=a, b=b,
                payload_bytes=2 * L * T * KVH * D * 2)


def _xfer_time(torch, step, iters=4) -> float:
    step()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        t = time.perf_counter()
        step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t)
    return statistics.median(times)


def bench_xfer(torch) -> dict:
    """Escalation handoff over TCP (the raw wire format): export (J5a gather) -> TcpTransport.send ->
    loopback socket -> TcpTransport.recv into GPU memory -> import (J5c scatter), sender
    and receiver in two threads of this process.  GB/s = K + V payload bytes / wall time
    of one handoff; the reference's pickle framing is timed in the CPU-baseline leg."""
    import threading

    from dispec_amd.transport.base import KVPayload
    from dispec_amd.transport.tcp import TcpTransport
    x = _xfer_setup(torch)
    tx, rx = TcpTransport(x["a"], "cuda"), TcpTransport(x["b"], "cuda")

    def step():
        p = KVPayload.export(x["src"], x["src_ids"], x["tokens"], request_id=1)
        th = threading.Thread(target=tx.send, args=(p,))
        th.start()
        got = rx.recv()
        th.join()
        got.import_into(x["dst"], x["dst_ids"])

    t = _xfer_time(torch, step)
    ok = torch.equal(x["dst"].export_contiguous(x["dst_ids"], len(x["tokens"]))[0],
                     x["src"].export_contiguous(x["src_ids"], len(x["tokens"]))[0])
    tx.close()
    rx.close()
    res = {"xfer_tcp_payload_MB": x["payload_bytes"] / 1e6, "xfer_tcp_ms": t * 1e3,
           "xfer_tcp_GBps": x["payload_bytes"] / t / 1e9, "xfer_tcp_exact": bool(ok)}
    del x
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------------------ config 5
def bench_c5(torch) -> dict:
    """Gather Qwen3-1.7B paged KV (28 L) of 8 requests x 4096 tokens into contiguous
    buffers, map each of 36 target layers from source layer round(i*27/35) with a bf16
    1024x1024 map (weights ~N(0, 1/1024)) for K and V, scatter into a randomly placed
    Qwen3-4B-layout pool (36 L)."""
    from dispec_amd import _lib
    from dispec_amd.kv.paged_cache import PagedKVCache
    from dispec_amd.kv.transfer import LayerMap

    Ls, Lt, KVH, D, bs, R, T = 28, 36, 8, 128, 16, 8, 4096
    dev = "cuda"
    nb = R * T // bs
    NB = int(nb * 1.25)
    src = PagedKVCache(Ls, NB, bs, KVH, D, device=dev)
    _fill_randn(torch, src.key, 5001)
    _fill_randn(torch, src.value, 5002)
    gcpu = torch.Generator().manual_seed(5003)
    perm = torch.randperm(NB, generator=gcpu)[:nb].view(R, T // bs)
    bt = perm.to(torch.int32).to(dev)
    cu = torch.arange(0, (R + 1) * T, T, dtype=torch.int64, device=dev)
    kbuf = torch.empty((Ls * R * T, KVH, D), dtype=torch.bfloat16, device=dev)
    vbuf = torch.empty_like(kbuf)
    g_s = _time_gpu_cold(torch, lambda: src.gather_into(bt, cu, T, kbuf, vbuf), 10)
    src.check_errors()
    moved = 2 * 2 * Ls * R * T * src.row_bytes
    del src
    torch.cuda.empty_cache()
    # the map: per request b its payload is (Ls, T, KVH, D) at rows Ls*T*b; map over all
    # 8 x 4096 tokens at once by treating the buffer as (R, Ls, T, kv) and the design row
    # of target layer i as source layer round(i*27/35) of every request
    kv = KVH * D
    g = torch.Generator(device=dev).manual_seed(5004)
    maps = []
    for i in range(Lt):
        w = torch.randn((kv, kv), generator=g, device=dev) / 32
        maps.append(LayerMap((int(round(i * 27 / 35)),), torch.zeros(kv, device=dev),
                             weight=w).to(dev, torch.bfloat16))
    mk = torch.empty((Lt * R * T, KVH, D), dtype=torch.bfloat16, device=dev)
    mv = torch.empty_like(mk)

    def run_map():
        # one launch per (target layer, K|V): the 8 requests are the GEMM's batch
        for buf, outb in ((kbuf, mk), (vbuf, mv)):
            ob = outb.view(R, Lt, T, kv)
            for i, m in enumerate(maps):
                m.apply_into(buf, [m.source_layers[0] * T * kv], kv, kv, T, ob[:, i],
                             batch=R, a_batch_stride=Ls * T * kv, c_batch_stride=Lt * T * kv)

    m_s = _time_gpu(torch, run_map, 3, warmup=1)
    flops = 2 * 2 * Lt * R * T * kv * kv
    # the floor of one map launch: its operand stages loaded into LDS with no arithmetic
    # (dsp_probe_gemm_fill: same tiles, same order, same loads)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    probe = _probe_lib()
    stream = torch.cuda.current_stream().cuda_stream

    def fill_probe():
        _lib.check(probe.dsp_probe_gemm_fill(kbuf.data_ptr(), kv, T, Ls * T * kv,
                                             w_probe.data_ptr(), kv, kv, kv, R,
                                             sink.data_ptr(), stream), "probe")
    w_probe = torch.empty((kv, kv), dtype=torch.bfloat16, device=dev).normal_()
    fill_s = _time_gpu(torch, fill_probe, 20)
    # the vendor library on the same problem size (hipBLASLt through torch.matmul): one
    # (8 x 4096, 1024) x (1024, 1024) bf16 product repeated, so its operands stay in the
    # Infinity Cache.  `c5_map_hipblaslt_us` takes the weight as the map kernel does (stored
    # N x K, K contiguous: the transposed view of a contiguous matrix, a plain 2-D product),
    # `_kn_us` as a contiguous K x N matrix; `c5_map_warm_us` is the map kernel on exactly
    # the operands of the first (x, the same N x K weight, no bias, a contiguous output),
    # repeated the same way -- the like-for-like figure beside them (the 72-launch loop
    # above streams a new A from HBM for every launch).
    from dispec_amd.kv.transfer import _gemm
    x_lib = kbuf[:R * T].view(R * T, kv)
    w_lib = w_probe.contiguous()
    out_lib = torch.empty((R * T, kv), dtype=torch.bfloat16, device=dev)
    lib_s = _time_gpu(torch, lambda: torch.matmul(x_lib, w_lib.t()), 20)
    lib_kn_s = _time_gpu(torch, lambda: torch.matmul(x_lib, w_lib), 20)
    warm_s = _time_gpu(torch, lambda: _gemm(x_lib, [0], kv, kv, R * T, w_lib, out_lib), 20)
    # scatter into a 36-layer target pool
    tgt = PagedKVCache(Lt, NB, bs, KVH, D, device=dev)
    perm = torch.randperm(NB, generator=gcpu)[:nb].view(R, T // bs)
    bt2 = perm.to(torch.int32).to(dev)
    s_s = _time_gpu_cold(torch, lambda: tgt.scatter_from(bt2, cu, T, mk, mv), 10)
    tgt.check_errors()

    # the map with the scatter fused into its epilogue: each (target layer, K|V) GEMM
    # writes its rows straight into the target pool's blocks (no 4.8 GB intermediate)
    def run_map_fused():
        for buf, pool in ((kbuf, tgt.key), (vbuf, tgt.value)):
            for i, m in enumerate(maps):
                assert m.apply_to_pool(buf, [m.source_layers[0] * T * kv], kv, kv, T, pool[i],
                                       bt2, bs, None, batch=R, a_batch_stride=Ls * T * kv,
                                       err=tgt._err)

    mf_s = _time_gpu(torch, run_map_fused, 3, warmup=1)
    tgt.check_errors()
    # prefill-scale append of 32768 rows (2 KiB) into random slots of one layer
    n = 32768
    slots = torch.randperm(tgt.num_slots, generator=gcpu)[:n].to(dev)
    kr, vr = mk[:n], mv[:n]
    a_s = _time_gpu_cold(torch, lambda: tgt.write(3, slots, kr, vr), 20)
    a_warm_s = _time_gpu(torch, lambda: tgt.write(3, slots, kr, vr), 20)
    res = {"c5_gather_us": g_s * 1e6, "c5_gather_GBps": moved / g_s / 1e9,
           "c5_map_ms": m_s * 1e3, "c5_map_TFLOPs": flops / m_s / 1e12,
           "c5_map_mfma_frac": flops / m_s / 1e12 / PEAK_BF16_TFLOPS,
           "c5_scatter_us": s_s * 1e6,
           "c5_map_fused_scatter_ms": mf_s * 1e3,
           "c5_map_fused_TFLOPs": flops / mf_s / 1e12,
           "c5_pipeline_ms": (g_s + mf_s) * 1e3,
           "c5_pipeline_unfused_ms": (g_s + m_s + s_s) * 1e3,
           "c5_scatter_GBps": 2 * 2 * Lt * R * T * tgt.row_bytes / s_s / 1e9,
           "append_prefill_GBps": 2 * 2 * n * tgt.row_bytes / a_s / 1e9,
           "append_prefill_warm_GBps": 2 * 2 * n * tgt.row_bytes / a_warm_s / 1e9}
    # roofline objects of the config-5 kernels: gather against HBM (its bytes, read once
    # and written once), the map launch against dense bf16 MFMA; traffic from the counter
    # passes in profiles/byte_movers_c4_c5_traffic.md
    movers = "byte_movers_c4_c5_traffic.md"
    res["c5_gather_roofline"] = {
        "bound": "hbm", "achieved": round(moved / g_s / 1e9, 1), "peak": PEAK_HBM_GBPS,
        "unit": "GB/s", "frac": round(moved / g_s / 1e9 / PEAK_HBM_GBPS, 4),
        "traffic": _traffic_per_launch(movers, "c5_gather"), "alg_bytes_per_launch": moved}
    # the import scatter (destination-block order): every target row read once from the
    # transport buffers and written once into the pool; the owner fill and lookup launches
    # before it are inside the timed call
    scattered = 2 * 2 * Lt * R * T * tgt.row_bytes
    res["c5_scatter_roofline"] = {
        "bound": "hbm", "achieved": round(scattered / s_s / 1e9, 1), "peak": PEAK_HBM_GBPS,
        "unit": "GB/s", "frac": round(scattered / s_s / 1e9 / PEAK_HBM_GBPS, 4),
        "traffic": _traffic_per_launch(movers, "c5_scatter"), "alg_bytes_per_launch": scattered}
    per_launch = m_s / (2 * len(maps))
    res["c5_map_fill_floor_us"] = round(fill_s * 1e6, 2)
    res["c5_map_us_per_launch"] = round(per_launch * 1e6, 2)
    res["c5_map_hipblaslt_us"] = round(lib_s * 1e6, 2)
    res["c5_map_hipblaslt_kn_us"] = round(lib_kn_s * 1e6, 2)
    res["c5_map_warm_us"] = round(warm_s * 1e6, 2)
    res["c5_map_roofline"] = {
        "bound": "mfma", "achieved": round(flops / m_s / 1e12, 1), "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s", "frac": round(flops / m_s / 1e12 / PEAK_BF16_TFLOPS, 4),
        "traffic": _traffic_per_launch(movers, "c5_map"),
        "flops_per_launch": flops / (2 * len(maps)), "us_per_launch": round(per_launch * 1e6, 2)}
    del tgt, kbuf, vbuf, mk, mv
    torch.cuda.empty_cache()
    return res


def bench_copy(torch) -> dict:
    """A plain 1 GiB device-to-device copy (torch's copy kernel): rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE of this dispatch against its known 1 GiB each way gives the
    counters' scale factor."""
    n = 1 << 29
    src = torch.ones(n, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    t = _time_gpu(torch, lambda: dst.copy_(src), 5)
    return {"copy_bytes_each_way": 2 * n, "copy_GBps": 2 * 2 * n / t / 1e9}


def bench_copy_ceiling(torch) -> dict:
    """The ceiling of the byte-moving kernels on this GPU: a 2 GiB streaming copy
    (dsp_probe_stream_copy, non-temporal loads and stores), best of three grid sizes --
    64, 16 and 4 KiB per workgroup, the last two one-shot workgroups -- read + write bytes
    over time; and the same copy with its destinations permuted in 32 KiB blocks, 8 KiB
    blocks and 2 KiB rows (dsp_probe_piece_scatter), the write patterns of scatter / block
    copy, of config 2's prefill-scale append (8 KiB blocks) and of a random-slot append; the
    copy with its sources permuted in 32 KiB blocks (dsp_probe_piece_gather), the transport
    gather's pattern; and stores alone, in order and to random 32 KiB blocks (dsp_probe_piece_fill,
    bytes written over time: the copy-on-write fork reads its one source block from L2 and
    only writes HBM)."""
    from dispec_amd import _lib
    lib = _probe_lib()
    n = 2 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(7)
    stream = torch.cuda.current_stream().cuda_stream
    best = None
    for wgs in (32768, 131072, 524288):
        def f():
            _lib.check(lib.dsp_probe_stream_copy(src.data_ptr(), dst.data_ptr(), n, wgs, stream),
                       "probe")
        t = _time_gpu(torch, f, 10)
        best = t if best is None else min(best, t)
    res = {"copy_ceiling_GBps": 2 * n / best / 1e9}
    # the same copy with its destinations permuted in 32 KiB blocks (the scatter's and the
    # block copy's write pattern) and in 2 KiB rows (the append's); "inorder32k" is that
    # kernel with the identity permutation, the control
    g = torch.Generator(device="cuda").manual_seed(9)
    for name, piece, rand in (("inorder32k", 32768, False), ("block32k", 32768, True),
                              ("block8k", 8192, True), ("row2k", 2048, True)):
        perm = (torch.randperm(n // piece, generator=g, device="cuda") if rand else
                torch.arange(n // piece, device="cuda")).to(torch.int32)

        def f():
            _lib.check(lib.dsp_probe_piece_scatter(src.data_ptr(), dst.data_ptr(), n, piece,
                                                   perm.data_ptr(), stream), "probe")
        res[f"scatter_{name}_ceiling_GBps"] = 2 * n / _time_gpu(torch, f, 10) / 1e9
        if piece == 32768:
            # the same destinations written without reading anything: HBM write bandwidth
            def fill():
                _lib.check(lib.dsp_probe_piece_fill(dst.data_ptr(), n, piece, perm.data_ptr(),
                                                    stream), "probe")
            res[f"write_only_{name}_GBps"] = n / _time_gpu(torch, fill, 10) / 1e9
        if name == "block32k":
            # the same copy read from random 32 KiB blocks and written in order (the gather)
            def gather():
                _lib.check(lib.dsp_probe_piece_gather(src.data_ptr(), dst.data_ptr(), n, piece,
                                                      perm.data_ptr(), stream), "probe")
            res["gather_block32k_ceiling_GBps"] = 2 * n / _time_gpu(torch, gather, 10) / 1e9
        del perm
    del src, dst
    torch.cuda.empty_cache()
    return res


def _traffic_per_launch(profile="decode_c3_traffic.md", key=""):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, each scaled by the copy calibration)
    as measured by the rocprofv3 passes recorded in profiles/<profile>: the line
    `traffic_bytes_per_launch:` (decode: the balanced decode kernel and its combine) or
    `traffic_bytes_per_launch[<key>]:`; None if absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", profile)
    if not os.path.exists(path):
        return None
    tag = f"traffic_bytes_per_launch[{key}]:" if key else "traffic_bytes_per_launch:"
    for line in open(path):
        if line.startswith(tag):
            return int(line[len(tag):].split()[0])
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-aux", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of c1,c2,c4,c5,skew,ceiling,prefill,xfer: run just these auxiliary configs and print "
                         "their numbers (no headline line); 'copy' runs the 1 GiB plain "
                         "device copy that calibrates the FETCH_SIZE / WRITE_SIZE counters; "
                         "'graph' times a whole-model decode step, eager against HIP graph")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the KV data path has no cross-GPU exchange in "
              "this build (it would shard by sequence or KV head); run with --gpus 1",
              file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    configs = (("c1", bench_c1), ("c2", bench_c2), ("c4", bench_c4), ("c5", bench_c5),
               ("skew", bench_skew), ("ceiling", bench_copy_ceiling), ("prefill", bench_prefill),
               ("xfer", bench_xfer), ("copy", bench_copy), ("graph", bench_graph))
    if args.only:
        want = set(args.only.split(","))
        aux = {}
        for name, fn in configs:
            if name in want:
                _log(f"config {name}")
                aux.update(fn(torch))
        print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v)
                          for k, v in aux.items()}), flush=True)
        return 0
    dec = bench_decode(torch, args.steps, args.warmup, keep_cpu_sample=not args.no_cpu_baseline)
    aux = {}
    if not args.no_aux:
        for name, fn in configs[:8]:
            _log(f"config {name}")
            aux.update(fn(torch))
    cpu = None if args.no_cpu_baseline else bench_cpu_baseline(torch, dec.pop("cpu_sample"))
    line = {
        "metric": "paged decode attn us/layer (Qwen3-4B shape, 16 x 32768 ctx)",
        "value": round(dec["us_per_layer"], 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/q, random block placement)",
        "config": {"workload": "config 3: Qwen3-4B-shape long-context decode step",
                   "layers": C3["layers"], "q_heads": C3["hq"], "kv_heads": C3["kvh"],
                   "head_dim": C3["d"], "block_size": C3["bs"], "batch": C3["batch"],
                   "context": C3["ctx"], "split": dec["split"],
                   "step": "per layer: append 1 token/seq + split-K paged decode"},
        "roofline": {"bound": "hbm", "achieved": round(dec["achieved_gbps"], 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(dec["achieved_gbps"] / PEAK_HBM_GBPS, 4),
                     "traffic": _traffic_per_launch(),
                     "kernel": "decode_balanced_kernel + decode_balanced_combine_kernel",
                     "alg_bytes_per_launch": dec["alg_bytes"],
                     "measured_read_ceiling_GBps": round(dec["read_ceiling_GBps"], 1),
                     "measured_decode_pattern_ceiling_GBps": round(dec["pattern_ceiling_GBps"], 1)},
        "decode_GBps": round(dec["achieved_gbps"], 1),
        "c3_fixed512_us_per_layer": round(dec["fixed512_us_per_layer"], 2),
        "c3_fixed512_GBps": round(dec["fixed512_GBps"], 1),
        "aux": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in aux.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
