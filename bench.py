"""Benchmark of the MI355X KV-cache data path (one GPU).

Workload (`value`): config 3 of the benchmark plan -- a Qwen3-4B-shape long-context
decode step: 36 layers, 32 query heads, 8 KV heads (GQA 4), head_dim 128, block_size 16,
bf16, batch 16 x 32768-token contexts with random block placement.  One step = for each
layer, append one token per sequence through the slot mapping (dsp_kv_append) and run
split-K paged decode attention over the full context (dsp_paged_decode, 512-token
partitions, LSE combine).  `value` is decode attention microseconds per layer.

Also reported on the same line:
  roofline      the decode kernel's achieved HBM GB/s (algorithmic bytes / average launch
                time from HIP events on the launch stream) against 8 TB/s
  cpu_baseline  the reference's CPU torch path (gather + repeat_interleave + SDPA) on a
                bounded sample of the same workload, timed on this host
  aux           GB/s of the byte-moving kernels at bandwidth scale: block-table gather of
                8 x 4096 tokens of a 28-layer Qwen3-1.7B-layout pool (config 5), the scatter
                into a 36-layer pool, a prefill-scale append, and copy-on-write block copies

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

C3 = dict(layers=36, hq=32, kvh=8, d=128, bs=16, batch=16, ctx=32768)


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def _fill_randn(torch, t, seed: int) -> None:
    g = torch.Generator(device=t.device).manual_seed(seed)
    for i in range(t.shape[0]):
        t[i].normal_(generator=g)


def bench_decode(torch, steps: int, warmup: int) -> dict:
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    from dispec_amd.kv.paged_cache import PagedKVCache

    c = C3
    L, Hq, KVH, D, bs, B, ctx = (c[k] for k in ("layers", "hq", "kvh", "d", "bs", "batch", "ctx"))
    dev = "cuda"
    nb_seq = ctx // bs
    NB = B * nb_seq
    _log(f"allocating a {L}-layer pool of {NB} blocks "
         f"({2 * L * NB * bs * KVH * D * 2 / 1e9:.1f} GB)")
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
    P = lib.dsp_paged_decode_partition_tokens(B, KVH, D, ctx)
    ws = torch.empty(lib.dsp_paged_decode_workspace_bytes(B, Hq, D, ctx, P) // 4 + 1,
                     dtype=torch.float32, device=dev)

    def step(ev=None):
        for layer in range(L):
            cache.write(layer, wslots, k_new[layer], v_new[layer])
            if ev is not None:
                ev[layer][0].record()
            paged_decode_attention_blocks(q[layer], cache.key[layer], cache.value[layer], bt,
                                          ctx_lens, Hq // KVH, block_size=bs, max_ctx=ctx,
                                          partition_tokens=P, out=out[layer], workspace=ws)
            if ev is not None:
                ev[layer][1].record()

    _log(f"decode: warmup {warmup} steps, partition {P} tokens")
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    cache.check_errors()
    ev = [list(_events(torch)) for _ in range(L)]
    decode_ms = []
    t0, t1 = _events(torch)
    t0.record()
    for i in range(steps):
        step(ev)
        torch.cuda.synchronize()
        decode_ms.extend(e[0].elapsed_time(e[1]) for e in ev)
    t1.record()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    _log(f"decode: {steps} steps in {total_ms:.1f} ms")
    kv_bytes = B * ctx * KVH * D * 2 * 2
    alg_bytes = kv_bytes + 2 * B * Hq * D * 2 + B * nb_seq * 4
    avg_s = statistics.mean(decode_ms) / 1e3
    achieved = alg_bytes / avg_s / 1e9
    # parity spot-check of one layer at full size: shape and finiteness here, the
    # exact checks live in tests/
    assert torch.isfinite(out).all()
    res = dict(
        us_per_layer=avg_s * 1e6, median_us_per_layer=statistics.median(decode_ms) * 1e3,
        ms_per_step=total_ms / steps, alg_bytes=alg_bytes, achieved_gbps=achieved,
        partition_tokens=P)
    del cache, q, k_new, v_new, out, ws
    torch.cuda.empty_cache()
    return res


def bench_cpu_baseline(torch) -> dict:
    """The reference CPU torch path for config 3 on a bounded sample: one layer, 2 of the
    16 sequences (2 x 32768 context), gather + repeat_interleave + SDPA in bf16; the
    per-layer time is scaled by 16/2 to the full batch."""
    from oracle import ref_torch

    c = C3
    Hq, KVH, D, bs, ctx = c["hq"], c["kvh"], c["d"], c["bs"], c["ctx"]
    nseq, B = 2, c["batch"]
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    nb = nseq * ctx // bs
    g = torch.Generator().manual_seed(3101)
    kc = torch.randn((nb * bs, KVH, D), generator=g).to(torch.bfloat16)
    vc = torch.randn((nb * bs, KVH, D), generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=g)
    slot_lists = [(perm[i * (ctx // bs):(i + 1) * (ctx // bs)][:, None] * bs
                   + torch.arange(bs)[None]).reshape(-1) for i in range(nseq)]
    q = torch.randn((nseq, Hq, D), generator=g).to(torch.bfloat16)
    times = []
    for _ in range(3):
        t = time.perf_counter()
        ref_torch.decode_repeat_kv_sdpa(q, kc, vc, slot_lists, Hq // KVH)
        times.append(time.perf_counter() - t)
    per_layer = statistics.median(times[1:]) * (B / nseq)
    return dict(value=per_layer * 1e6, unit="us/layer", cores=torch.get_num_threads(),
                kind="port",
                sample=f"1 layer, {nseq} of {B} sequences x {ctx} tokens, median of "
                       f"{len(times) - 1} after 1 warmup, scaled x{B // nseq}",
                cpu_model=_cpu_model())


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_gpu(torch, fn, iters: int, warmup: int = 2) -> float:
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


def bench_aux(torch) -> dict:
    """GB/s of gather / scatter / append / block copy at bandwidth scale."""
    from dispec_amd.kv.paged_cache import PagedKVCache

    res = {}
    dev = "cuda"
    # config 5: Qwen3-1.7B-layout source pool, 8 requests x 4096 tokens, random blocks
    Ls, Lt, KVH, D, bs, R, T = 28, 36, 8, 128, 16, 8, 4096
    nb = R * T // bs
    NB = int(nb * 1.25)
    src = PagedKVCache(Ls, NB, bs, KVH, D, device=dev)
    _fill_randn(torch, src.key, 3201)
    _fill_randn(torch, src.value, 3202)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3203))[:nb].view(R, T // bs)
    seqs = [(perm[i].tolist(), T) for i in range(R)]
    sec = _time_gpu(torch, lambda: src.export_batch(seqs), 10)
    moved = 2 * 2 * Ls * R * T * src.row_bytes        # read + write, K and V
    res["gather_c5_GBps"] = moved / sec / 1e9
    res["gather_c5_us"] = sec * 1e6
    src.check_errors()
    kbuf, vbuf, cu = src.export_batch(seqs)
    del src, kbuf, vbuf
    torch.cuda.empty_cache()
    # scatter of a 36-layer mapped buffer into a randomly placed Qwen3-4B-layout pool
    tgt = PagedKVCache(Lt, NB, bs, KVH, D, device=dev)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3204))[:nb].view(R, T // bs)
    tables = [perm[i].tolist() for i in range(R)]
    kb = torch.randn((Lt * R * T, KVH, D), device=dev).to(torch.bfloat16)
    vb = torch.randn((Lt * R * T, KVH, D), device=dev).to(torch.bfloat16)
    cu = [i * T for i in range(R + 1)]
    sec = _time_gpu(torch, lambda: tgt.import_batch(tables, kb, vb, cu), 10)
    res["scatter_c5_GBps"] = 2 * 2 * Lt * R * T * tgt.row_bytes / sec / 1e9
    res["scatter_c5_us"] = sec * 1e6
    tgt.check_errors()
    del kb, vb
    # prefill-scale append: 32768 token rows (2 KiB each) into random slots of one layer
    n = 32768
    slots = torch.randperm(tgt.num_slots, generator=torch.Generator().manual_seed(3205))[:n].to(dev)
    kr = torch.randn((n, KVH, D), device=dev).to(torch.bfloat16)
    vr = torch.randn((n, KVH, D), device=dev).to(torch.bfloat16)
    sec = _time_gpu(torch, lambda: tgt.write(3, slots, kr, vr), 20)
    res["append_prefill_GBps"] = 2 * 2 * n * tgt.row_bytes / sec / 1e9
    # decode-step append (16 rows): latency
    sec = _time_gpu(torch, lambda: tgt.write(3, slots[:16], kr[:16], vr[:16]), 50)
    res["append_decode16_us"] = sec * 1e6
    # copy-on-write / evict block copies: 1024 block pairs over 36 layers
    pairs_perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3206))
    src_ids, dst_ids = pairs_perm[:1024].tolist(), pairs_perm[1024:2048].tolist()
    sec = _time_gpu(torch, lambda: tgt.copy_blocks_from(tgt, src_ids, dst_ids), 10)
    res["copy_blocks_GBps"] = 2 * 2 * Lt * 1024 * tgt.block_bytes / sec / 1e9
    tgt.check_errors()
    del tgt
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-aux", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the KV data path has no cross-GPU exchange in "
              "this build (sharding is by sequence or KV head, see the design notes); run "
              "with --gpus 1", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    dec = bench_decode(torch, args.steps, args.warmup)
    aux = {} if args.no_aux else bench_aux(torch)
    cpu = None if args.no_cpu_baseline else bench_cpu_baseline(torch)
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
                   "context": C3["ctx"], "partition_tokens": dec["partition_tokens"],
                   "step": "per layer: append 1 token/seq + split-K paged decode"},
        "roofline": {"bound": "hbm", "achieved": round(dec["achieved_gbps"], 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(dec["achieved_gbps"] / PEAK_HBM_GBPS, 4),
                     "traffic": None, "kernel": "paged_decode_kernel + decode_combine_kernel",
                     "alg_bytes_per_launch": dec["alg_bytes"]},
        "decode_GBps": round(dec["achieved_gbps"], 1),
        "aux": {k: round(v, 2) for k, v in aux.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
