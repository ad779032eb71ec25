"""Benchmark of the MI355X FlashAttention hot path (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-configs]
                    [--only all|prefill|decode|copy|gqa|loop|d128]

Prints ONE JSON line on stdout (everything else goes to stderr):

* ``value``: causal prefill throughput in TFLOP/s at BASELINE config 3
  (B=1, H=14, S=4096, D=64, fp16 in / fp32 accumulate), K timed steps, one
  ``flashattn_cuda.prefill`` call per step, inputs resident in HBM, FLOPs by
  the reference convention 4*B*H*S^2*D/2 (bench/run_bench.py:102-107).
* ``roofline``: that kernel's achieved TFLOP/s from a HIP event pair around
  the K back-to-back launches of the timed region (on the launch stream),
  against the dense fp16 MFMA peak.
* ``decode``: BASELINE config 5 (ragged B=32, H=14, Lmax=4096) in GB/s of
  algorithmic bytes (valid K/V rows + q + o + seq_lens) against 8 TB/s, with
  the caches rotated over copies larger than the 256 MB MALL.
* ``configs``: every BASELINE config with the reference's timing protocol
  (10 warm-ups, 3 x 30 launches, median; bench/run_bench.py:83-99).
* Every timing starts with ~0.1-0.25 s of untimed launches of the same
  call, which bring the GPU to its sustained clock (an idle MI355X starts
  lower and needs ~50 ms of load to get there).
* ``decode_loop``: tokens/s of the generation step (append_kv + decode) at
  the reference's decode_lines shapes and the config 5 batch, eager and as a
  replayed HIP graph (one step, and eight steps, per graph).
* ``gqa``: grouped-query prefill / decode (2 K/V heads for 14 query heads)
  at the config 3 and 5 shapes, beside the repeat-K/V-then-call path the
  reference's callers use.
* ``cpu_baseline``: the CPU oracle (a numpy restatement of the reference's
  src/attention_cpu.py) timed on this host on a bounded sample of config 3.

The CPU oracle is imported only for that baseline leg.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "flash-attention-cuda_amd"))
sys.path.insert(0, REPO)

MFMA_FP16_PEAK_TFLOPS = 2516.6  # MI355X dense fp16 MFMA (datasheet, no sparsity)
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
SCALE = 0.125
MALL_BYTES = 256 << 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def attention_flops(batch, heads, seq, causal, d=64):
    f = 4.0 * batch * heads * seq * seq * d
    return f * 0.5 if causal else f


def decode_bytes(heads, lens, max_seq, d=64):
    import torch

    lens = torch.clamp(lens.long(), 0, max_seq)
    b = lens.numel()
    return 2 * heads * d * 2 * int(lens.sum()) + 2 * b * heads * d * 2 + 4 * b


def cpu_inputs_prefill(batch, heads, seq, seed=0, d=64):
    import torch

    g = torch.Generator().manual_seed(seed)
    shape = (batch, heads, seq, d)
    return [torch.randn(shape, generator=g, dtype=torch.float32).half() for _ in range(3)]


def cpu_inputs_decode(batch, heads, lmax, seed=0, d=64):
    import torch

    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, lmax + 1, (batch,), generator=g).to(torch.int32)
    q = torch.randn((batch, heads, 1, d), generator=g, dtype=torch.float32).half()
    k = torch.randn((batch, heads, lmax, d), generator=g, dtype=torch.float32).half()
    v = torch.randn((batch, heads, lmax, d), generator=g, dtype=torch.float32).half()
    return q, k, v, lens


def copies_for(nbytes, minimum=1):
    """Number of input copies whose total exceeds 2x the MALL."""
    return max(minimum, math.ceil(2 * MALL_BYTES / max(nbytes, 1)) + 1)


def ref_timeit(fn_list, iters=30, warmup=10):
    """bench/run_bench.py:83-99: median of three means over `iters` launches
    (launch i uses fn_list[i % len(fn_list)] to rotate input copies), after
    the clock warm-up below."""
    import torch

    n = len(fn_list)
    clock_warmup(fn_list, 0.1)
    for i in range(warmup):
        fn_list[i % n]()
    torch.cuda.synchronize()
    samples = []
    for _ in range(3):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(iters):
            fn_list[i % n]()
        end.record()
        torch.cuda.synchronize()
        samples.append(start.elapsed_time(end) / iters)
    return sorted(samples)[1]


def clock_warmup(fn_list, seconds=0.25):
    """Untimed launches for `seconds` before any timing: an idle MI355X
    starts below its sustained engine clock and needs ~50 ms of load to reach
    it (measured: C3 prefill at 73 us in the first 100 launches, 50.5 us from
    ~1200 launches on), so a short fixed warm-up would time the ramp."""
    import torch

    n = len(fn_list)
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(20):
            fn_list[i % n]()
            i += 1
        torch.cuda.synchronize()


def timed_steps(fn_list, steps, warmup):
    """Contract timing: W untimed steps, then exactly K steps between
    synchronisations. A HIP event pair on the launch stream brackets the K
    back-to-back launches: the host submits a launch in 5-9 us, well under
    the kernels' duration, so the stream never drains and the event span
    over K is the kernel's average duration (plus the hardware's
    kernel-to-kernel gap). Events between launches would instead leave the
    stream idle for each record call."""
    import torch

    n = len(fn_list)
    clock_warmup(fn_list)
    for i in range(warmup):
        fn_list[i % n]()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        fn_list[i % n]()
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    return wall_ms / steps, start.elapsed_time(end) / steps


def bench_prefill(fa, batch, heads, seq, causal, protocol="ref", steps=0, warmup=0, d=64):
    import torch

    q, k, v = (t.cuda() for t in cpu_inputs_prefill(batch, heads, seq, d=d))
    n = copies_for(3 * q.numel() * 2) if protocol == "ref" else 1
    sets = [(q, k, v)] + [tuple(t.clone() for t in (q, k, v)) for _ in range(n - 1)]
    scale = d ** -0.5  # 1/sqrt(head_dim): the reference's 0.125 at head_dim 64
    fns = [lambda s=s: fa.prefill(s[0], s[1], s[2], causal, scale) for s in sets]
    torch.cuda.synchronize()
    flops = attention_flops(batch, heads, seq, causal, d)
    if protocol == "ref":
        ms = ref_timeit(fns)
        return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "copies": n}
    step_ms, kern_ms = timed_steps(fns, steps, warmup)
    return {"ms_per_step": step_ms, "kernel_ms": kern_ms, "flops": flops}


def bench_decode(fa, batch, heads, lmax, lens=None, protocol="ref", steps=0, warmup=0, d=64):
    import torch

    q, k, v, rl = cpu_inputs_decode(batch, heads, lmax, d=d)
    if lens is not None:
        rl = torch.tensor(lens, dtype=torch.int32)
    q, k, v, rl = q.cuda(), k.cuda(), v.cuda(), rl.cuda()
    n = copies_for(2 * k.numel() * 2)
    sets = [(q, k, v)] + [tuple(t.clone() for t in (q, k, v)) for _ in range(n - 1)]
    scale = d ** -0.5
    fns = [lambda s=s: fa.decode(s[0], s[1], s[2], rl, scale) for s in sets]
    torch.cuda.synchronize()
    nbytes = decode_bytes(heads, rl.cpu(), lmax, d)
    if protocol == "ref":
        ms = ref_timeit(fns)
        return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "copies": n}
    step_ms, kern_ms = timed_steps(fns, steps, warmup)
    return {"ms_per_step": step_ms, "kernel_ms": kern_ms, "bytes": nbytes, "copies": n,
            "sum_len": int(rl.sum().item())}


def bench_gqa(fa):
    """Grouped-query attention (2 K/V heads for 14 query heads, group 7) at
    the config 3 and config 5 shapes, reference timing protocol: the kernel
    entry points (prefill_gqa / decode_gqa) against what the reference's
    callers do instead, repeat K/V per query head on the device and call
    prefill / decode. Decode GB/s counts the K/V rows read once per K/V
    head."""
    import torch

    rows = []
    kv_heads, heads = 2, 14
    group = heads // kv_heads
    q, k, v = (t.cuda() for t in cpu_inputs_prefill(1, heads, 4096))
    k2, v2 = k[:, ::group].contiguous(), v[:, ::group].contiguous()
    torch.cuda.synchronize()
    flops = attention_flops(1, heads, 4096, True)
    ms = ref_timeit([lambda: fa.prefill_gqa(q, k2, v2, True, SCALE)])
    ms_rep = ref_timeit([lambda: fa.prefill(q, k2.repeat_interleave(group, 1),
                                            v2.repeat_interleave(group, 1), True, SCALE)])
    rows.append({"config": "C3 GQA causal B1 H14 Hkv2 S4096", "ms": ms,
                 "tflops": flops / (ms * 1e-3) / 1e12, "ms_repeat_then_prefill": ms_rep})
    log(f"  {rows[-1]['config']}: {ms * 1e3:.1f} us ({rows[-1]['tflops']:.1f} TFLOP/s); "
        f"repeat + prefill {ms_rep * 1e3:.1f} us")

    qd, kd, vd, rl = cpu_inputs_decode(32, heads, 4096)
    kd, vd = kd[:, ::group].contiguous(), vd[:, ::group].contiguous()
    qd, rl = qd.cuda(), rl.cuda()
    n = copies_for(2 * kd.numel() * 2)
    sets = [(kd.cuda(), vd.cuda())]
    sets += [tuple(t.clone() for t in sets[0]) for _ in range(n - 1)]
    torch.cuda.synchronize()
    nbytes = decode_bytes(kv_heads, rl.cpu(), 4096) + 2 * 32 * (heads - kv_heads) * 64 * 2
    ms = ref_timeit([lambda s=s: fa.decode_gqa(qd, s[0], s[1], rl, SCALE) for s in sets])
    ms_rep = ref_timeit([lambda s=s: fa.decode(qd, s[0].repeat_interleave(group, 1),
                                               s[1].repeat_interleave(group, 1), rl, SCALE)
                         for s in sets])
    rows.append({"config": "C5 GQA ragged decode B32 H14 Hkv2 Lmax4096", "ms": ms,
                 "gbs": nbytes / (ms * 1e-3) / 1e9, "frac_hbm": nbytes / (ms * 1e-3) / 1e9 /
                 HBM_PEAK_GBS, "copies": n, "ms_repeat_then_decode": ms_rep})
    log(f"  {rows[-1]['config']}: {ms * 1e3:.1f} us ({rows[-1]['gbs']:.1f} GB/s); "
        f"repeat + decode {ms_rep * 1e3:.1f} us")
    return rows


def bench_head_dim_128(fa):
    """head_dim 128 (the reference's named next step, README.md:397) at the
    config 3, config 2 (full) and config 5 shapes, reference timing protocol,
    at the standard scale 1/sqrt(128) (the configs' 0.125 is 1/sqrt(64)).
    FLOPs 4 B H S^2 128 (halved when causal); decode bytes count the K/V rows
    read (256 B each per head), q, o and seq_lens."""
    rows = []
    for name, b, h, s, c in [("C3-shape causal B1 H14 S4096 D128", 1, 14, 4096, True),
                             ("C2-shape full B4 H12 S1024 D128", 4, 12, 1024, False)]:
        r = bench_prefill(fa, b, h, s, c, d=128)
        rows.append({"config": name, "ms": r["ms"], "tflops": r["tflops"],
                     "frac_mfma": r["tflops"] / MFMA_FP16_PEAK_TFLOPS})
        log(f"  {name}: {r['ms'] * 1e3:.1f} us, {r['tflops']:.1f} TFLOP/s")
    for name, b, h, lmax, lens in [("C4-shape decode B1 H12 L4096 D128", 1, 12, 4096, [4096]),
                                   ("C5-shape ragged decode B32 H14 Lmax4096 D128", 32, 14,
                                    4096, None)]:
        r = bench_decode(fa, b, h, lmax, lens=lens, d=128)
        rows.append({"config": name, "ms": r["ms"], "gbs": r["gbs"],
                     "frac_hbm": r["gbs"] / HBM_PEAK_GBS, "copies": r["copies"]})
        log(f"  {name}: {r['ms'] * 1e3:.1f} us, {r['gbs']:.1f} GB/s")
    # Grouped queries at head_dim 128 (2 K/V heads for 14 query heads): the
    # matrix-core grouped pass against repeat-then-decode.
    import torch

    kv_heads, heads, group = 2, 14, 7
    qd, kd, vd, rl = cpu_inputs_decode(32, heads, 4096, d=128)
    kd, vd = kd[:, ::group].contiguous(), vd[:, ::group].contiguous()
    qd, rl = qd.cuda(), rl.cuda()
    n = copies_for(2 * kd.numel() * 2)
    sets = [(kd.cuda(), vd.cuda())]
    sets += [tuple(t.clone() for t in sets[0]) for _ in range(n - 1)]
    torch.cuda.synchronize()
    nbytes = decode_bytes(kv_heads, rl.cpu(), 4096, 128) + 2 * 32 * (heads - kv_heads) * 128 * 2
    scale = 128 ** -0.5
    ms = ref_timeit([lambda s=s: fa.decode_gqa(qd, s[0], s[1], rl, scale) for s in sets])
    ms_rep = ref_timeit([lambda s=s: fa.decode(qd, s[0].repeat_interleave(group, 1),
                                               s[1].repeat_interleave(group, 1), rl, scale)
                         for s in sets])
    rows.append({"config": "C5-shape GQA ragged decode B32 H14 Hkv2 Lmax4096 D128", "ms": ms,
                 "gbs": nbytes / (ms * 1e-3) / 1e9,
                 "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "copies": n,
                 "ms_repeat_then_decode": ms_rep})
    log(f"  {rows[-1]['config']}: {ms * 1e3:.1f} us ({rows[-1]['gbs']:.1f} GB/s); "
        f"repeat + decode {ms_rep * 1e3:.1f} us")
    return rows


def bench_decode_loop(fa, steps=64):
    """Token generation: one step = append_kv (the caller's cache write) +
    decode, starting from a context of `ctx` tokens, `steps` tokens per run.
    bench/run_bench.py:183-210 (decode_lines) reports decode tokens/s at
    B=1 H=12 for contexts 128-2048 on a fixed cache; here the same shapes
    (plus the config 5 batch) run the whole step, eagerly (two host calls
    per token) and as one captured HIP graph replayed per token (the lengths
    live on the device, so the step's arguments never change). tokens/s =
    batch x steps / time; `decode_ms` is decode alone on a fixed cache, the
    reference's measurement."""
    import torch

    rows = []
    cases = [(f"B1 H12 ctx {c}", 1, 12, c, None) for c in (128, 256, 512, 1024, 2048)]
    cases.append(("config 5 batch B32 H14 ragged", 32, 14, 4096, "ragged"))
    for name, batch, heads, ctx, kind in cases:
        lmax = ctx + steps + 64
        g = torch.Generator().manual_seed(0)
        if kind == "ragged":
            lens0 = torch.randint(1, ctx + 1, (batch,), generator=g).to(torch.int32)
        else:
            lens0 = torch.full((batch,), ctx, dtype=torch.int32)
        kc0 = torch.randn((batch, heads, lmax, 64), generator=g).half().cuda()
        vc0 = torch.randn((batch, heads, lmax, 64), generator=g).half().cuda()
        qs = torch.randn((steps, batch, heads, 1, 64), generator=g).half().cuda()
        ks = torch.randn((steps, batch, heads, 1, 64), generator=g).half().cuda()
        vs = torch.randn((steps, batch, heads, 1, 64), generator=g).half().cuda()
        lens0 = lens0.cuda()
        torch.cuda.synchronize()

        dec_ms = ref_timeit([lambda: fa.decode(qs[0], kc0, vc0, lens0, SCALE)])

        def eager_run():
            kc, vc, lens = kc0.clone(), vc0.clone(), lens0.clone()
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for t in range(steps):
                fa.append_kv(kc, vc, ks[t], vs[t], lens)
                fa.decode(qs[t], kc, vc, lens, SCALE)
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / steps

        eager_run()
        eager_ms = sorted(eager_run() for _ in range(3))[1]

        kc, vc, lens = kc0.clone(), vc0.clone(), lens0.clone()
        q_in, k_in, v_in = qs[0].clone(), ks[0].clone(), vs[0].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            kw, vw, lw = kc.clone(), vc.clone(), lens.clone()
            fa.append_kv(kw, vw, k_in, v_in, lw)
            fa.decode(q_in, kw, vw, lw, SCALE)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fa.append_kv(kc, vc, k_in, v_in, lens)
            fa.decode(q_in, kc, vc, lens, SCALE)
        torch.cuda.synchronize()

        def graph_run():
            kc.copy_(kc0)
            vc.copy_(vc0)
            lens.copy_(lens0)
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(steps):
                graph.replay()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / steps

        graph_run()
        graph_ms = sorted(graph_run() for _ in range(3))[1]

        # Eight tokens per graph (their q, k, v from the per-token inputs):
        # one replay launches the 16 kernels of eight steps, so the host cost
        # of a replay is shared by eight tokens.
        per_graph = 8
        graph8 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph8):
            for t in range(per_graph):
                fa.append_kv(kc, vc, ks[t], vs[t], lens)
                fa.decode(qs[t], kc, vc, lens, SCALE)
        torch.cuda.synchronize()

        def graph8_run():
            kc.copy_(kc0)
            vc.copy_(vc0)
            lens.copy_(lens0)
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(steps // per_graph):
                graph8.replay()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / (steps // per_graph * per_graph)

        graph8_run()
        graph8_ms = sorted(graph8_run() for _ in range(3))[1]
        rows.append({"config": name, "batch": batch, "heads": heads, "context": ctx,
                     "steps": steps, "decode_ms": dec_ms, "decode_tok_s": batch * 1e3 / dec_ms,
                     "step_ms_eager": eager_ms, "tok_s_eager": batch * 1e3 / eager_ms,
                     "step_ms_graph": graph_ms, "tok_s_graph": batch * 1e3 / graph_ms,
                     "step_ms_graph8": graph8_ms, "tok_s_graph8": batch * 1e3 / graph8_ms})
        log(f"  {name}: decode {dec_ms * 1e3:.1f} us; append + decode step eager "
            f"{eager_ms * 1e3:.1f} us ({batch * 1e3 / eager_ms:,.0f} tok/s), graph "
            f"{graph_ms * 1e3:.1f} us ({batch * 1e3 / graph_ms:,.0f} tok/s), 8 steps per graph "
            f"{graph8_ms * 1e3:.1f} us ({batch * 1e3 / graph8_ms:,.0f} tok/s)")
        del graph, graph8, kc, vc, kc0, vc0
        torch.cuda.empty_cache()
    return rows


def cpu_baseline(budget_s=12.0):
    """The CPU oracle on a bounded sample of config 3: the 14 causal heads of
    B=1, S=4096 one at a time, cycling over them (one warm-up head first)
    until at least `budget_s` seconds of work are done, in TFLOP/s by the same
    causal FLOP convention."""
    import numpy as np

    from oracle import attention as orc

    try:
        from threadpoolctl import threadpool_info

        blas_threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # pragma: no cover
        blas_threads = 1
    q, k, v = (t.numpy().astype(np.float32) for t in cpu_inputs_prefill(1, 14, 4096))
    orc.attention_cpu(q[0, 0], k[0, 0], v[0, 0], SCALE, True)  # warm-up
    t0 = time.perf_counter()
    done = 0
    while True:
        h = done % 14
        orc.attention_cpu(q[0, h], k[0, h], v[0, h], SCALE, True)
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    flops = attention_flops(1, done, 4096, True)
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": int(blas_threads),
        "host_cpus": len(os.sched_getaffinity(0)),
        "kind": "port",
        "sample": f"config 3 (causal S=4096, D=64): {done} head-passes cycling over its "
                  f"14 heads, fp32 numpy restatement of src/attention_cpu.py with a "
                  f"causal mask, {dt:.2f} s after one warm-up head",
        "seconds_per_head": dt / done,
    }


def cpu_per_config(budget_each=1.5):
    """The CPU oracle on every BASELINE config (bounded samples, the same
    inputs recipe as the GPU runs): whole configs where they are cheap (C1,
    C4, C5), else a sample of heads timed for about `budget_each` seconds and
    scaled to the config's head count (C2). Returns one row per config with
    the CPU milliseconds per config and the rate in the config's unit."""
    import numpy as np

    from oracle import attention as orc

    rows = []
    for name, b, h, s, causal in [("C1 causal B1 H12 S128", 1, 12, 128, True),
                                  ("C2 causal B4 H12 S1024", 4, 12, 1024, True),
                                  ("C2 full B4 H12 S1024", 4, 12, 1024, False)]:
        q, k, v = (t.numpy().astype(np.float32) for t in cpu_inputs_prefill(b, h, s))
        qh, kh, vh = (x.reshape(b * h, s, 64) for x in (q, k, v))
        orc.attention_cpu(qh[0], kh[0], vh[0], SCALE, causal)  # warm-up
        t0 = time.perf_counter()
        done = 0
        while done < b * h or time.perf_counter() - t0 < budget_each:
            i = done % (b * h)
            orc.attention_cpu(qh[i], kh[i], vh[i], SCALE, causal)
            done += 1
            if done >= b * h and time.perf_counter() - t0 >= budget_each:
                break
            if done >= 4 * b * h:
                break
        per_head = (time.perf_counter() - t0) / done
        ms = per_head * b * h * 1e3
        rows.append({"config": name, "cpu_ms": ms,
                     "cpu_tflops": attention_flops(b, h, s, causal) / (ms * 1e-3) / 1e12,
                     "sample": f"{done} head-passes"})
    for name, b, h, lmax, lens in [("C4 decode B1 H12 L4096", 1, 12, 4096, [4096]),
                                   ("C5 ragged decode B32 H14 Lmax4096", 32, 14, 4096, None)]:
        import torch

        q, k, v, rl = cpu_inputs_decode(b, h, lmax)
        if lens is not None:
            rl = torch.tensor(lens, dtype=torch.int32)
        qn, kn, vn, ln = (x.numpy() for x in (q.float(), k.float(), v.float(), rl))
        orc.decode(qn, kn, vn, ln, SCALE)  # warm-up
        t0 = time.perf_counter()
        runs = 0
        while runs < 1 or (time.perf_counter() - t0 < budget_each and runs < 20):
            orc.decode(qn, kn, vn, ln, SCALE)
            runs += 1
        ms = (time.perf_counter() - t0) / runs * 1e3
        nbytes = decode_bytes(h, rl, lmax)
        rows.append({"config": name, "cpu_ms": ms, "cpu_gbs": nbytes / (ms * 1e-3) / 1e9,
                     "sample": f"{runs} whole-config runs"})
    return rows


def copy_calibration(steps):
    """A plain 1 GiB device-to-device copy, `steps` times: the known-size
    kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters into HBM
    bytes (it reads and writes exactly 1 GiB per launch)."""
    import torch

    n = 1 << 29  # fp16 elements = 1 GiB
    src = torch.randn(n, device="cuda", dtype=torch.float16)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    step_ms, kern_ms = timed_steps([lambda: dst.copy_(src)], steps, 1)
    nbytes = 2 * src.numel() * 2
    return {"bytes_per_launch": nbytes, "kernel_ms": kern_ms,
            "gbs": nbytes / (kern_ms * 1e-3) / 1e9}


def load_traffic(name):
    """HBM bytes per launch of a workload's main kernel, from the committed
    rocprofv3 report (profiles/<workload>__<kernel>.md, written by
    flash-attention-cuda_amd/profile/profile_rocprof.sh), if present."""
    path = os.path.join(REPO, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path, encoding="utf-8"):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config sweep")
    ap.add_argument("--only", choices=["all", "prefill", "decode", "copy", "gqa", "loop", "d128"],
                    default="all",
                    help="copy: only the 1 GiB copy that calibrates the HBM byte counters; "
                         "gqa: only the grouped-query lines; loop: only the decode loop; "
                         "d128: only the head_dim 128 lines")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py measures one GPU only: this build has no multi-GPU path "
            "(prefill and decode would shard over (batch, head) with no exchange between GPUs). "
            f"Requested --gpus {args.gpus}.")
        sys.exit(2)

    import torch

    import flashattn_cuda as fa

    if not torch.cuda.is_available():
        log("no HIP device visible")
        sys.exit(1)
    props = torch.cuda.get_device_properties(0)
    log(f"device: {props.name} ({props.multi_processor_count} CUs), "
        f"arch {getattr(props, 'gcnArchName', '?')}")

    if args.only == "copy":
        c = copy_calibration(args.steps)
        log(f"1 GiB copy: {c['kernel_ms'] * 1e3:.1f} us, {c['gbs']:.1f} GB/s (read + write)")
        print(json.dumps({"metric": "device copy GB/s (counter calibration)",
                          "value": c["gbs"], "unit": "GB/s", **c}), flush=True)
        return

    if args.only == "loop":
        rows = bench_decode_loop(fa)
        print(json.dumps({"metric": "decode loop tokens/s (append_kv + decode per token)",
                          "value": rows[-1]["tok_s_graph"], "unit": "tokens/s",
                          "decode_loop": rows}), flush=True)
        return

    if args.only == "d128":
        rows = bench_head_dim_128(fa)
        print(json.dumps({"metric": "head_dim 128 prefill TFLOP/s and decode KV GB/s",
                          "value": rows[0]["tflops"], "unit": "TFLOP/s",
                          "head_dim_128": rows}), flush=True)
        return

    if args.only == "gqa":
        rows = bench_gqa(fa)
        print(json.dumps({"metric": "grouped-query prefill TFLOP/s and decode KV GB/s",
                          "value": rows[1]["gbs"], "unit": "GB/s", "gqa": rows}), flush=True)
        return

    result = {
        "metric": "prefill TFLOP/s & %MFMA peak @S=4096; decode KV GB/s & %HBM peak",
        "value": None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "config 3: causal prefill B=1 H=14 S=4096 D=64 "
                               "(fp16 in, fp32 accumulate, fp16 out)",
                   "batch": 1, "heads": 14, "seq_len": 4096, "head_dim": 64,
                   "causal": True, "parallelism": "single GPU"},
    }

    if args.only in ("all", "prefill"):
        log("timing config 3 prefill ...")
        r = bench_prefill(fa, 1, 14, 4096, True, protocol="contract",
                          steps=args.steps, warmup=args.warmup)
        value = r["flops"] / (r["ms_per_step"] * 1e-3) / 1e12
        achieved = r["flops"] / (r["kernel_ms"] * 1e-3) / 1e12
        result["value"] = value
        result["ms_per_step"] = r["ms_per_step"]
        result["roofline"] = {
            "bound": "mfma",
            "kernel": "prefill_kernel<causal=true>",
            "achieved": achieved,
            "peak": MFMA_FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / MFMA_FP16_PEAK_TFLOPS,
            "kernel_ms": r["kernel_ms"],
            "traffic": load_traffic("prefill_c3__prefill_kernel.md"),
        }
        log(f"  {value:.1f} TFLOP/s per step, kernel {achieved:.1f} TFLOP/s "
            f"({100 * achieved / MFMA_FP16_PEAK_TFLOPS:.1f}% of MFMA peak)")

    if args.only in ("all", "decode"):
        log("timing config 5 ragged decode ...")
        d = bench_decode(fa, 32, 14, 4096, protocol="contract", steps=args.steps,
                         warmup=args.warmup)
        gbs_step = d["bytes"] / (d["ms_per_step"] * 1e-3) / 1e9
        gbs_kern = d["bytes"] / (d["kernel_ms"] * 1e-3) / 1e9
        result["decode"] = {
            "workload": "config 5: ragged decode B=32 H=14 Lmax=4096 D=64, lens U[1,4096] seed 0",
            "value": gbs_step,
            "unit": "GB/s",
            "ms_per_step": d["ms_per_step"],
            "sum_len": d["sum_len"],
            "bytes_per_step": d["bytes"],
            "cache_copies_rotated": d["copies"],
            "roofline": {"bound": "hbm", "kernel": "decode_bh_kernel",
                         "achieved": gbs_kern, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs_kern / HBM_PEAK_GBS, "kernel_ms": d["kernel_ms"],
                         "traffic": load_traffic("decode_c5__decode_bh_kernel.md")},
        }
        if args.only == "decode":
            result["value"], result["unit"] = gbs_step, "GB/s"
            result["ms_per_step"] = d["ms_per_step"]
        log(f"  {gbs_step:.1f} GB/s per step ({100 * gbs_kern / HBM_PEAK_GBS:.1f}% of HBM peak)")

    if not args.no_configs and args.only == "all":
        log("reference-protocol sweep over the BASELINE configs ...")
        rows = []
        for name, b, h, s, c in [("C1 causal B1 H12 S128", 1, 12, 128, True),
                                 ("C2 causal B4 H12 S1024", 4, 12, 1024, True),
                                 ("C2 full B4 H12 S1024", 4, 12, 1024, False),
                                 ("C3 causal B1 H14 S4096", 1, 14, 4096, True)]:
            r = bench_prefill(fa, b, h, s, c)
            rows.append({"config": name, "ms": r["ms"], "tflops": r["tflops"],
                         "frac_mfma": r["tflops"] / MFMA_FP16_PEAK_TFLOPS})
            log(f"  {name}: {r['ms'] * 1e3:.1f} us, {r['tflops']:.1f} TFLOP/s")
        for name, b, h, lmax, lens in [("C4 decode B1 H12 L4096", 1, 12, 4096, [4096]),
                                       ("C5 ragged decode B32 H14 Lmax4096", 32, 14, 4096, None)]:
            r = bench_decode(fa, b, h, lmax, lens=lens)
            rows.append({"config": name, "ms": r["ms"], "gbs": r["gbs"],
                         "frac_hbm": r["gbs"] / HBM_PEAK_GBS, "copies": r["copies"]})
            log(f"  {name}: {r['ms'] * 1e3:.1f} us, {r['gbs']:.1f} GB/s")
        result["configs"] = rows
        log("grouped-query attention (no reference counterpart) ...")
        result["gqa"] = bench_gqa(fa)
        log("decode loop: append_kv + decode per token ...")
        result["decode_loop"] = bench_decode_loop(fa)
        log("head_dim 128 (no reference counterpart) ...")
        result["head_dim_128"] = bench_head_dim_128(fa)

    if not args.no_cpu:
        log("CPU baseline (oracle, bounded sample) ...")
        cb = cpu_baseline()
        result["cpu_baseline"] = cb
        log(f"  {cb['value'] * 1e3:.2f} GFLOP/s on {cb['cores']} threads")
        if args.only == "all":
            log("CPU oracle on every config (bounded samples) ...")
            per = cpu_per_config()
            # Config 3 comes from the main baseline sample above.
            per.insert(3, {"config": "C3 causal B1 H14 S4096",
                           "cpu_ms": cb["seconds_per_head"] * 14 * 1e3,
                           "cpu_tflops": cb["value"], "sample": "the cpu_baseline sample"})
            cb["per_config"] = per
            by_name = {r["config"]: r for r in per}
            for row in result.get("configs", []):
                c = by_name.get(row["config"])
                if c:
                    row["cpu_ms"] = c["cpu_ms"]
                    row["gpu_speedup_over_cpu"] = c["cpu_ms"] / row["ms"]
            for r in per:
                log(f"  {r['config']}: {r['cpu_ms']:.2f} ms on the CPU ({r['sample']})")

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
