"""Benchmark: int4 KV-residual decode attention at 32K context, batch 8, on one MI355X.

A step is one layer's decode attention over all four loops of the cfg3 workload
(B=8, H=16, D=128, T=32768; int4 residual streams g64, BF16 tail 64; loops 3-4 attend to
the top 10% of keys ranked by the loop-2 logits): dense loop 1, dense loop 2 with
logits, top-k selection, cached-mass sparse loop 3 (which also forms the loop-2
selected aggregate from the rows it reads) and sparse loop 4
(flashloop/engine.py:422-531).  The packed cache is built once on the GPU before timing
(inputs resident in HBM).  Prints one JSON line.

``value`` is the step's algorithmic HBM bytes / step time (GB/s); ``roofline`` reports
the dense loop-2 reader kernel (the dominant kernel) against the 8 TB/s HBM peak, timed
inside the timed steps with HIP events that the library records on the launch stream
immediately around that kernel (fl_profile_dense_reader); ``breakdown`` times each op of
the step (reader + merge, HIP events on the launch stream) over extra steps after the
timed region, with its algorithmic bytes and fraction of peak; ``cpu_baseline`` times
the reference's torch path of the same step (oracle/torch_cpu.py: flashloop_torch's
bf16 attention over the materialised loop caches, top-k mask, mass-scaled sparse
outputs) on torch-CPU with every thread torch is given, on a bounded sample of (b,h)
rows of the same workload (its step repeated for about --cpu-seconds), scaled to the
full step.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "int4 KV-residual decode attn µs/step + HBM GB/s (%peak) at 32K ctx, bs=8"
HBM_PEAK_GBPS = 8000.0
# HBM bytes per launch of the dense reader kernel, from the rocprofv3 counter runs
# (FETCH_SIZE x2.0 calibration against a 1 GiB copy, + WRITE_SIZE) summarised in this
# file, which names its command and the build it was taken on.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "traffic_dense_reader_cfg3.txt")


def traffic_from_profile(kernel_key: str):
    """(bytes per launch, source) of ``kernel_key`` from TRAFFIC_PROFILE, or (None, reason)."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 3 and parts[0] == "traffic_bytes" and parts[1] == kernel_key:
                    build = next((l.split(":", 1)[1].strip() for l in open(TRAFFIC_PROFILE) if l.startswith("build:")),
                                 "unknown")
                    return int(parts[2]), f"{os.path.relpath(TRAFFIC_PROFILE, ROOT)} (counter runs on build {build})"
    except OSError:
        return None, "no counter profile in this tree"
    return None, f"no {kernel_key} line in {os.path.relpath(TRAFFIC_PROFILE, ROOT)}"
CONFIGS = {
    "cfg3": dict(batch=8, heads=16, tokens=32768, seed=3),
    "cfg0": dict(batch=1, heads=16, tokens=2048, seed=0),
    "cfg1": dict(batch=1, heads=16, tokens=8192, seed=1),
    # ragged batch: per-sequence contexts drawn from U[1024, 16384] (seeded)
    "cfg2": dict(batch=32, heads=16, tokens=16384, seed=2, ragged=(1024, 16384)),
    # end-to-end random-init looped decoder, run through FlashLoopEngine
    "cfg4": dict(prompt=8192, new_tokens=256, seed=4),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="cfg3", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-rows", type=int, default=32, help="(b,h) rows of the CPU baseline sample (0 = skip)")
    ap.add_argument("--breakdown-steps", type=int, default=10,
                    help="after the timed region, each op runs this many times back to back between two "
                         "HIP events (its per-op time in the breakdown; 0 = skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU baseline: repeat the sample's step until this much CPU time has run")
    ap.add_argument("--eager", action="store_true", help="cfg4: eager decode launches instead of HIP-graph replay")
    ap.add_argument("--paired-dense", action="store_true",
                    help="cfg3: dense loops 1 and 2 in one pair launch (needs both loops' queries at "
                         "once, which the looped model's loop-by-loop order never provides)")
    ap.add_argument("--no-chain", action="store_true",
                    help="cfg4: residual/norm chains as launches of their own, not inside the next GEMV")
    ap.add_argument("--graph", action="store_true",
                    help="cfg0-cfg3: the metric's timed region replays the step captured once in a HIP "
                         "graph (host launch cost out of the step; the small configs are launch-bound)")
    ap.add_argument("--fraction", type=float, default=0.10)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (a known-size kernel that "
                         "calibrates rocprof FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--pack-reps", type=int, default=0,
                    help="rebuild the packed cache this many more times without masks and as many "
                         "with loop-3/4 masks (30%% / 15%% of tokens), each timed with events over "
                         "the whole build, host set-up included (J1)")
    return ap.parse_args()


def cpu_baseline(sample, fraction: float, seconds: float):
    """Time the reference's torch path of the decode step (oracle/torch_cpu.py) on the
    sampled rows, on torch-CPU with torch's thread count, repeated until ``seconds`` of
    wall time have run.  ``sample``: (q, k_cur, v_cur, keys, values) CPU bf16 tensors.
    Returns (seconds per step of the sample, seconds timed, repetitions, threads)."""
    import torch

    from flashloop_amd.synthetic import SCALING
    from oracle import torch_cpu

    q, kc, vc, keys, values = sample
    torch_cpu.decode_layer_step(q, kc, vc, keys, values, SCALING, fraction)  # warm-up (allocator, threads)
    reps = 0
    t0 = time.perf_counter()
    while True:
        torch_cpu.decode_layer_step(q, kc, vc, keys, values, SCALING, fraction)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= seconds or reps >= 256:
            break
    return dt / reps, dt, reps, torch.get_num_threads()


def cpu_sample(ks, vs, queries, kcur, vcur, rows: int, B: int, H: int, T: int):
    """The first ``rows`` (b,h) rows of the workload as the reference's torch path holds
    them: per loop the materialised bf16 cache (the codec's reconstruction of the packed
    prefix -- built on the GPU, bit-identical to the oracle's -- then the BF16 tail).
    ``T``: the sampled rows' context length (a ragged batch samples rows of its first
    sequence only)."""
    import torch

    from flashloop_amd import CrossLoopKVLayer

    Tall = ks[0].shape[2]
    sub_k = [k.reshape(1, B * H, Tall, 128)[:, :rows, :T].contiguous() for k in ks]
    sub_v = [v.reshape(1, B * H, Tall, 128)[:, :rows, :T].contiguous() for v in vs]
    small = CrossLoopKVLayer.from_prefill(sub_k, sub_v, recon=True)
    tp = small.quantized_tokens
    keys, values = [], []
    for r in range(4):
        rk = small.recon_keys[r].reshape(rows, -1, 128)[:, :tp]
        rv = small.recon_values[r].reshape(rows, -1, 128)[:, :tp]
        keys.append(torch.cat([rk, sub_k[r][0, :, tp:T]], dim=1).cpu())
        values.append(torch.cat([rv, sub_v[r][0, :, tp:T]], dim=1).cpu())
    flat = lambda t: t.reshape(B * H, 1, 128)[:rows].cpu()  # noqa: E731
    out = ([flat(x) for x in queries], [flat(x) for x in kcur], [flat(x) for x in vcur], keys, values)
    del small
    torch.cuda.empty_cache()
    return out


def bench_cfg4(args):
    """Config 4: random-init Ouro-shaped model (24 layers, hidden 2048, 16 heads x 128,
    SwiGLU 5632, vocab 49152, 4 loops), an 8192-token random prompt, greedy generation of
    256 tokens through FlashLoopEngine (token retention 100/100/25/10%, 10% decode keys).
    Reports prefill seconds and decode tokens/s; one JSON line."""
    import torch

    from flashloop_amd import FlashLoopEngine
    from flashloop_amd.model import OuroConfig

    cfg = CONFIGS["cfg4"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    print(f"[bench] cfg4: random-init model on {torch.cuda.get_device_name(0)}", file=sys.stderr, flush=True)
    eng = FlashLoopEngine.from_random_init(OuroConfig(), seed=cfg["seed"], device=dev)
    eng.use_graphs = not args.eager
    eng.fused_chain = not args.no_chain
    g = torch.Generator().manual_seed(cfg["seed"])
    ids = torch.randint(0, eng.model.config.vocab_size, (1, cfg["prompt"]), generator=g).to(dev)
    new = cfg["new_tokens"] if args.steps == 50 else max(2, args.steps)
    # warm-up on a short prompt (library loads, hipBLASLt heuristics)
    eng.generate(ids[:, :640], max_new_tokens=4)
    eng.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = eng.prefill(ids, decode_capacity=new + 64)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    tok = torch.argmax(out.logits, dim=-1, keepdim=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(new - 1):
        tok = torch.argmax(eng.decode(tok).logits, dim=-1, keepdim=True)
    torch.cuda.synchronize()
    decode_s = time.perf_counter() - t0
    receipts = [dict(loop=r.loop, active_rows=r.active_rows) for r in eng.state.prefill_receipts]
    line = {
        "metric": "cfg4 end-to-end greedy decode tokens/s (random-init 24-layer looped decoder, prompt 8192)",
        "value": round((new - 1) / decode_s, 2),
        "unit": "tokens/s",
        "ms_per_token": round(decode_s / (new - 1) * 1e3, 3),
        "prefill_s": round(prefill_s, 4),
        "new_tokens": new,
        "n_gpus": 1,
        "higher_is_better": True,
        "dtype": "bf16 weights / int4 KV",
        "data": "synthetic (random weights, random token ids)",
        "decode_graphs": eng.use_graphs,
        "fused_chain": eng.fused_chain,
        "prefill_receipts": receipts,
        "config": {"workload": "cfg4", "prompt": cfg["prompt"], "layers": eng.model.config.num_hidden_layers,
                   "hidden": eng.model.config.hidden_size},
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the path would shard by (batch, head) rows, with no exchange between GPUs)"}))
        sys.exit(2)
    if args.config == "cfg4":
        bench_cfg4(args)
        return
    import numpy as np
    import torch

    from flashloop_amd import CrossLoopKVLayer, accounting, decode_attention_step
    from flashloop_amd.synthetic import SCALING, decode_workload

    cfg = CONFIGS[args.config]
    B, H, T = cfg["batch"], cfg["heads"], cfg["tokens"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lengths = None
    if "ragged" in cfg:
        from flashloop_amd.synthetic import ragged_lengths

        lengths = ragged_lengths(B, *cfg["ragged"], seed=cfg["seed"])
        T = max(lengths)
    print(f"[bench] building {args.config} workload B={B} H={H} T={T} on {torch.cuda.get_device_name(0)}",
          file=sys.stderr, flush=True)

    w = decode_workload(B, H, T, seed=cfg["seed"], device=dev, lengths=lengths)
    cur = [w.current(r) for r in range(4)]
    queries = [q.contiguous() for q in w.queries]
    ks = [w.keys[r][:, :, :T].contiguous() for r in range(4)]
    vs = [w.values[r][:, :, :T].contiguous() for r in range(4)]
    del w
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    layer = CrossLoopKVLayer.from_prefill(ks, vs, lengths=lengths)
    torch.cuda.synchronize()
    pack_s = time.perf_counter() - t0
    pack_bytes = 8 * H * (B * T if lengths is None else sum(lengths)) * 128 * 2  # bf16 K and V of 4 loops, read once
    pack_reps = {"full": [], "masked": []}
    if args.pack_reps > 0:
        gm = torch.Generator(device=dev).manual_seed(cfg["seed"] + 17)
        m3 = torch.rand(B, T, device=dev, generator=gm) < 0.3
        m4 = m3 & (torch.rand(B, T, device=dev, generator=gm) < 0.5)
        for kind, kw in (("full", {}), ("masked", {"mask_loop3": m3, "mask_loop4": m4})):
            for _ in range(args.pack_reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                extra = CrossLoopKVLayer.from_prefill(ks, vs, lengths=lengths, **kw)
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1)
                packed_rows = [extra.packed_host[r // H] for r in range(B * H)]
                rows = [packed_rows, packed_rows] + [[extra.late_rows_host[s][r // H] for r in range(B * H)]
                                                     for s in range(2)]
                rd, wr = accounting.pack_bytes(packed_rows, rows, sum(extra.packed_host) * 2 if kw else 0)
                pack_reps[kind].append({"build_ms": round(ms, 3), "alg_GB": round((rd + wr) / 1e9, 3),
                                        "alg_TB_per_s_of_build": round((rd + wr) / ms / 1e9, 2)})
                del extra
        del m3, m4
        torch.cuda.empty_cache()
    kcur = [c[0] for c in cur]
    vcur = [c[1] for c in cur]
    sample = None
    if args.cpu_rows > 0:
        # (a ragged batch: rows of its first sequence, at that sequence's length)
        n_rows = min(args.cpu_rows, B * H) if lengths is None else min(args.cpu_rows, H)
        sample = cpu_sample(ks, vs, queries, kcur, vcur, n_rows, B, H, T if lengths is None else lengths[0])
    del ks, vs
    torch.cuda.empty_cache()
    if args.calib_copy_mib > 0:
        src = torch.ones(args.calib_copy_mib * 2**18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def step():
        return decode_attention_step(layer, queries, kcur, vcur, SCALING, args.fraction,
                                     paired_dense=args.paired_dense)

    # the dense reader kernel (the loop-2 launch, or the loops 1+2 pair launch with
    # --paired-dense) is timed by the library: HIP events recorded on the launch stream
    # around that kernel in each timed step (fl_profile_dense_reader; code 4 = the pair)
    from flashloop_amd import _lib

    lib = _lib.load()

    def timed_step(i):
        """One step, op by op (the same launches as ``step``)."""
        if (not args.paired_dense):
            out0, _ = layer.dense_source_attention(0, query=queries[0], current_key=kcur[0], current_value=vcur[0],
                                                   scaling=SCALING, return_logits=False)
            out1, logits, (idx, valid, mass, wts, counts) = layer.dense_source_attention_select(
                1, query=queries[1], current_key=kcur[1], current_value=vcur[1], scaling=SCALING,
                fraction=args.fraction)
        else:
            out0, out1, logits = layer.dense_source_attention_pair(
                queries=queries[:2], current_keys=kcur[:2], current_values=vcur[:2], scaling=SCALING)
            idx, valid, mass, wts, counts = layer.select_decode_keys(logits, args.fraction)
        d2, so = layer.cached_mass_sparse_attention_delta_with_source(
            2, query=queries[2], current_key=kcur[2], current_value=vcur[2], indices=idx, valid=valid,
            source_weights=wts, source_current_value=vcur[1], global_mass=mass, scaling=SCALING, counts=counts)
        d3 = layer.cached_mass_sparse_attention_delta(3, query=queries[3], current_key=kcur[3], current_value=vcur[3],
                                                      indices=idx, valid=valid, source_selected_output=so,
                                                      global_mass=mass, scaling=SCALING, counts=counts)
        return out0, out1, d2, d3

    for _ in range(args.warmup):
        step()
    ref = step()
    torch.cuda.synchronize()
    # the timed region of the metric: K steps with nothing else on the stream
    graph = None
    if args.graph:
        import gc

        side = torch.cuda.Stream()  # default priority
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            timed_step(-1)  # sizes every workspace outside the capture
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        gc.disable()  # no collection may destroy a graph while the stream captures
        try:
            with torch.cuda.graph(graph):
                g_out = timed_step(-1)
        finally:
            gc.enable()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("out0", "out1", "delta2", "delta3"), g_out, (ref.out0, ref.out1, ref.delta2, ref.delta3)):
            if not torch.equal(a, b):
                raise RuntimeError(f"graph replay differs from the eager step in {name}")
    t0 = time.perf_counter()
    for i in range(args.steps):
        if graph is None:
            timed_step(i)
        else:
            graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed / args.steps * 1e3
    # a second timed region of K steps for the roofline: the library records a HIP event
    # pair on the dense reader kernel's own dispatch in every step (hipExtLaunchKernel),
    # kept out of the metric's region all the same.
    _lib.check(lib.fl_profile_dense_reader(1 if (not args.paired_dense) else 4, args.steps), "fl_profile_dense_reader")
    t1 = time.perf_counter()
    for i in range(args.steps):
        timed_step(i)
    torch.cuda.synchronize()
    ms_step_instrumented = (time.perf_counter() - t1) / args.steps * 1e3
    import ctypes

    tot_ms, n_rec = ctypes.c_float(0.0), ctypes.c_int32(0)
    _lib.check(lib.fl_profile_dense_reader_read(ctypes.byref(tot_ms), ctypes.byref(n_rec)), "fl_profile_dense_reader_read")
    _lib.check(lib.fl_profile_dense_reader(1 if (not args.paired_dense) else 4, 0), "fl_profile_dense_reader")
    if n_rec.value != args.steps:
        raise RuntimeError(f"expected {args.steps} profiled loop-2 reader launches, got {n_rec.value}")
    reader_ms = tot_ms.value / n_rec.value

    # algorithmic bytes from the actual selection (read back outside the timed region)
    packed = [layer.packed_host[r // H] for r in range(B * H)]
    tail = [layer.tail_host[r // H] for r in range(B * H)]
    cap = ref.indices.shape[-1]
    idx_h = ref.indices.reshape(B * H, cap).cpu().numpy()
    cnt_h = ref.counts.cpu().numpy()
    stats = accounting.selection_stats(idx_h, cnt_h, packed)
    parts = {
        "dense_loop1": accounting.dense_bytes(packed, tail, 1, False),
        "dense_loop2": accounting.dense_bytes(packed, tail, 2, True),
        "topk": accounting.topk_bytes(packed, tail, cap),
        "sparse_loop3_with_source": accounting.sparse_bytes(stats, cap, 2, with_source=True),
        "sparse_loop4": accounting.sparse_bytes(stats, cap, 3),
    }
    step_bytes = sum(parts.values())
    gbps = step_bytes / (ms_step * 1e-3) / 1e9
    reader_bytes = parts["dense_loop2"] + (0 if (not args.paired_dense) else parts["dense_loop1"])
    reader_gbps = reader_bytes / (reader_ms * 1e-3) / 1e9
    traffic = traffic_from_profile("dense_pair_kernel" if args.paired_dense else "dense_reader_kernel<2,true>") \
        if args.config == "cfg3" else (None, "counter profile taken at cfg3 only")
    finite = all(bool(torch.isfinite(t).all()) for t in (ref.out0, ref.out1, ref.delta2, ref.delta3))

    # per-op breakdown after the timed region: each op of the step (its reader and merge
    # launches) runs `breakdown_steps` times back to back on the step's inputs between two
    # events on the launch stream, so the event overhead is paid once per op, not per run
    breakdown = None
    if args.breakdown_steps > 0:
        idx, valid, mass, wts, counts = layer.select_decode_keys(ref.logits1, args.fraction)
        so = ref.selected_output
        ops = []
        if not args.paired_dense:
            ops.append(("dense_loop1", lambda: layer.dense_source_attention(
                0, query=queries[0], current_key=kcur[0], current_value=vcur[0], scaling=SCALING,
                return_logits=False)))
            ops.append(("dense_loop2+topk", lambda: layer.dense_source_attention_select(
                1, query=queries[1], current_key=kcur[1], current_value=vcur[1], scaling=SCALING,
                fraction=args.fraction)))
        else:
            ops.append(("dense_loop1+2", lambda: layer.dense_source_attention_pair(
                queries=queries[:2], current_keys=kcur[:2], current_values=vcur[:2], scaling=SCALING)))
            ops.append(("topk", lambda: layer.select_decode_keys(ref.logits1, args.fraction)))
        ops.append(("sparse_loop3_with_source", lambda: layer.cached_mass_sparse_attention_delta_with_source(
            2, query=queries[2], current_key=kcur[2], current_value=vcur[2], indices=idx, valid=valid,
            source_weights=wts, source_current_value=vcur[1], global_mass=mass, scaling=SCALING, counts=counts)))
        ops.append(("sparse_loop4", lambda: layer.cached_mass_sparse_attention_delta(
            3, query=queries[3], current_key=kcur[3], current_value=vcur[3], indices=idx, valid=valid,
            source_selected_output=so, global_mass=mass, scaling=SCALING, counts=counts)))
        breakdown = {}
        for name, fn in ops:
            fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            # a spin kernel first keeps the GPU busy while the host enqueues the runs, so the
            # runs execute back to back (their host-side argument handling stays hidden, as
            # it is inside a step)
            torch.cuda._sleep(int(4e6))
            e0.record()
            for _ in range(args.breakdown_steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / args.breakdown_steps * 1e3
            nbytes = parts[name] if name in parts else (
                parts["dense_loop2"] + parts["topk"] if name == "dense_loop2+topk" else parts["dense_loop1"] + parts["dense_loop2"])
            ach = nbytes / (us * 1e-6) / 1e9
            breakdown[name] = {"us": round(us, 2), "algorithmic_bytes": nbytes, "GB_per_s": round(ach, 1),
                               "frac": round(ach / HBM_PEAK_GBPS, 4)}
        breakdown["note"] = (f"each op {args.breakdown_steps} times back to back (queued behind a spin kernel) "
                             "between two events on the launch stream: an op's time holds its reader and merge "
                             "launches (repeats of a sparse op can find part of its 0.3-0.4 GB in the 256 MB memory-side cache); "
                             "per-kernel times are in the rocprof summary")

    cpu = None
    if sample is not None:
        rows = sample[0][0].shape[0]
        print(f"[bench] CPU baseline on {rows} rows", file=sys.stderr, flush=True)
        s_step, dt, reps, threads = cpu_baseline(sample, args.fraction, args.cpu_seconds)
        # scaled by keys: the step's total over the sample's (rows of equal length)
        all_keys = H * (sum(lengths) if lengths is not None else B * T)
        sample_keys = rows * (lengths[0] if lengths is not None else T)
        us_cpu = s_step * all_keys / sample_keys * 1e6
        cpu = {
            "value": round(step_bytes / (us_cpu * 1e-6) / 1e9, 4),
            "unit": "GB/s",
            "us_per_step": round(us_cpu, 1),
            "cores": threads,
            "kind": "port",
            "sample": f"{rows} of {B * H} (b,h) rows of the same workload at full context: flashloop_torch's "
                      f"decode step (oracle/torch_cpu.py: bf16 attention over the materialised caches of all "
                      f"4 loops, top-k mask, mass-scaled sparse outputs) on torch-CPU with {threads} threads, "
                      f"repeated {reps} times ({dt:.1f} s), scaled by the step's keys over the sample's "
                      f"({all_keys}/{sample_keys})",
        }

    line = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "us_per_step": round(ms_step * 1e3, 2),
        "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 codes x fp16 scale/min, f32 accumulate",
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: decode attention of one layer, 4 loops, B={B} H={H} D=128 "
                        + (f"T={T}, " if lengths is None else
                           f"ragged T~U[{cfg['ragged'][0]},{cfg['ragged'][1]}] (seed {cfg['seed']}, max {T}), ")
                        + f"int4 residual streams g64 (fp32 scale/min stored, fp16 copies streamed), BF16 tail {tail[0]}, "
                        f"late loops on top {args.fraction:.0%} keys",
            "batch": B,
            "heads": H,
            "context": T if lengths is None else lengths,
            "fraction": args.fraction,
            "launch": "HIP graph replay" if args.graph else "eager (one host launch per kernel)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": ("dense_reader_kernel<2,true> (loop-2 dense reader)" if (not args.paired_dense)
                       else "dense_pair_kernel (loops 1+2 dense reader, one launch)"),
            "achieved": round(reader_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(reader_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic[0],
            "traffic_source": traffic[1],
            "algorithmic_bytes": reader_bytes,
            "avg_us": round(reader_ms * 1e3, 2),
            "timing": (f"HIP event pair on the kernel's own dispatch (hipExtLaunchKernel, launch stream) in each "
                       f"of {args.steps} steps timed after the metric's region "
                       f"({round(ms_step_instrumented * 1e3, 2)} us/step with the events)"),
        },
        "cpu_baseline": cpu,
        "breakdown_bytes": parts,
        "breakdown": breakdown,
        "pack": {"GB_read_per_s": round(pack_bytes / pack_s / 1e9, 1), "seconds": round(pack_s, 4),
                 "note": "one-off cache build (J1) incl. host setup, not part of the step",
                 **({"repeats": pack_reps} if args.pack_reps > 0 else {})},
        "finite": finite,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
