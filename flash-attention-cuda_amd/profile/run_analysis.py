"""On-box performance analysis: occupancy, rooflines and the decode split study.

    python flash-attention-cuda_amd/profile/run_analysis.py [--out PATH]

Counterpart of bench/run_analysis.py in shrvan30/flash-attention-cuda (main
:284-459): a device table, the kernels' theoretical occupancy from
``occupancy_report()`` (:348-367), a prefill roofline over a set of shapes
(:62-92, :369-395), and the decode split study, fixed 512-row chunks against
the adaptive chunk (:94-140, :397-435). The numbers come from HIP events around
repeated launches and from the occupancy API; the report says which figures
are measured and which are derived. The counter-based evidence (HBM bytes,
MFMA busy, LDS conflicts) comes from rocprofv3 through profile_rocprof.sh.

Peaks are MI355X's published dense figures: 2,516.6 TFLOP/s fp16 MFMA and
8,000 GB/s HBM3E.
"""

from __future__ import annotations

import argparse
import math
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # the package root (flashattn_cuda)

MFMA_PEAK_TFLOPS = 2516.6
HBM_PEAK_GBS = 8000.0
HEAD_DIM = 64
SCALE = 1.0 / math.sqrt(HEAD_DIM)
# Whole-sequence decode threshold of csrc/decode.hip (use_bh_path): caches of
# at most this many rows run one block per (b, h) at any B * H.
BH_SHORT_CACHE = 512

# The reference's shapes (run_analysis.py:375-383, :403, :424-425) plus this
# build's BASELINE configs 2 and 3.
PREFILL_SHAPES = [
    (4, 12, 2048, True),
    (8, 12, 4096, True),
    (8, 12, 4096, False),
    (1, 12, 1024, True),
    (4, 12, 1024, True),
    (4, 12, 1024, False),
    (1, 14, 4096, True),
]
DECODE_STUDY_SHAPES = [(1, 12, 512), (1, 12, 1024), (1, 12, 2048)]
DECODE_SHAPES = [(1, 12, 512), (1, 12, 1024), (1, 12, 2048), (1, 12, 4096), (8, 12, 2048)]


def prefill_model(batch, heads, seq, causal, ms):
    """Derived figures for one prefill timing: FLOPs 4 B H N^2 d (halved for
    causal), minimum traffic (3 reads + 1 write) B H N d 2 bytes."""
    flops = 4.0 * batch * heads * seq * seq * HEAD_DIM * (0.5 if causal else 1.0)
    move_bytes = 4.0 * batch * heads * seq * HEAD_DIM * 2
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = move_bytes / (ms * 1e-3) / 1e9
    return {
        "shape": f"B={batch}, H={heads}, N={seq}, {'causal' if causal else 'full'}",
        "ms": ms,
        "tflops": tflops,
        "pct_mfma": 100.0 * tflops / MFMA_PEAK_TFLOPS,
        "gbs": gbs,
        "pct_hbm": 100.0 * gbs / HBM_PEAK_GBS,
    }


def decode_path(batch, heads, seq, cus):
    """Which decode pass runs (the rule of csrc/decode.hip use_bh_path)."""
    return "whole-sequence" if batch * heads >= cus or seq <= BH_SHORT_CACHE else "split-K + merge"


def decode_model(batch, heads, seq, chunk, path, ms):
    """Derived figures for one decode timing: the cache read once, plus (split
    path only) the partials written by the split pass and read by the merge."""
    splits = -(-seq // chunk)
    units = batch * heads * (splits if path != "whole-sequence" else 1)
    cache_bytes = 2.0 * batch * heads * seq * HEAD_DIM * 2
    ws_bytes = 2.0 * batch * heads * splits * (HEAD_DIM + 2) * 4 if path != "whole-sequence" else 0.0
    gbs = (cache_bytes + ws_bytes) / (ms * 1e-3) / 1e9
    return {
        "shape": f"B={batch}, H={heads}, S={seq}",
        "path": path,
        "chunk": chunk,
        "units": units,
        "ms": ms,
        "gbs": gbs,
        "pct_hbm": 100.0 * gbs / HBM_PEAK_GBS,
    }


def render(device, occupancy, prefill, before, after, adaptive, command):
    """The report as markdown. Pure function of its inputs (tested on the CPU)."""
    out = []
    w = out.append
    w("# On-box performance analysis (MI355X)")
    w("")
    w(f"Made by `{command}` (from the repository root, on the GPU box).")
    w("")
    w("**Measured** here, by a clock or the runtime: kernel wall-clock times (HIP events,")
    w("median of three loops of 30 launches after 0.2 s of untimed launches and 10")
    w("warm-ups, inputs resident in HBM and reused, so small shapes run partly from the")
    w("256 MB MALL); each kernel's registers, LDS and theoretical occupancy")
    w("(`hipOccupancyMaxActiveBlocksPerMultiprocessor`).")
    w("")
    w("**Derived** from those times and the shapes: TFLOP/s, GB/s and the % of peak")
    w("columns, by the FLOP and byte models stated above each table. Achieved HBM bytes,")
    w("MFMA busy and LDS bank conflicts are counter figures: see the rocprofv3 summaries in")
    w("this folder (profile_rocprof.sh).")
    w("")
    w("| | |")
    w("| :-- | :-- |")
    for key, value in device:
        w(f"| {key} | {value} |")
    w("")

    w("## Kernel resources and theoretical occupancy")
    w("")
    w("From `flashattn_cuda.occupancy_report()` at each kernel's launch configuration.")
    w("")
    w("| kernel | threads/block | registers/thread | LDS/block | max blocks/CU | theoretical occupancy |")
    w("| :-- | ---: | ---: | ---: | ---: | ---: |")
    for row in occupancy:
        w(f"| `{row['kernel']}` | {row['threads_per_block']} | {row['registers_per_thread']} | "
          f"{row['shared_bytes_per_block']:,} B | {row['max_active_blocks_per_sm']} | "
          f"{row['theoretical_occupancy'] * 100:.1f}% |")
    w("")
    w("The prefill block is one per CU by design (8 waves, 160 KiB of LDS rings): two waves")
    w("per SIMD, the pairing that lets one wave's MFMAs run under the other's softmax.")
    w("")

    w("## Prefill roofline")
    w("")
    w("`FLOPs = 4 B H N^2 d` (halved for causal); `bytes = (3 reads + 1 write) B H N d 2`;")
    w(f"peaks {MFMA_PEAK_TFLOPS:,.1f} TFLOP/s (dense fp16 MFMA) and {HBM_PEAK_GBS:,.0f} GB/s.")
    w("")
    w("| shape | ms | TFLOP/s | % of MFMA peak | GB/s | % of HBM peak |")
    w("| :-- | ---: | ---: | ---: | ---: | ---: |")
    for r in prefill:
        w(f"| {r['shape']} | {r['ms']:.4f} | {r['tflops']:.1f} | {r['pct_mfma']:.1f}% | "
          f"{r['gbs']:.1f} | {r['pct_hbm']:.2f}% |")
    w("")
    w("Prefill is far from the HBM roofline at every shape (arithmetic intensity N/2 or N")
    w("flop per byte); it is bound by the matrix-core and VALU work of each key tile, and at")
    w("small B * H * N by how many 128-row blocks there are per CU.")
    w("")

    w("## Decode roofline and the split study")
    w("")
    w("`bytes = 2 B H S d 2` for the cache, plus the split partials written by the split")
    w("pass and read by the merge (`2 B H splits (d + 2) 4`) on the split-K path. The")
    w("adaptive chunk is the largest power of two in [128, 1024] that gives at least")
    w("2 x CUs units; caches of at most 512 rows, and batches with B * H >= CUs, run the")
    w("whole-sequence pass (one block per (b, h), no partials) whatever the chunk.")
    w("")
    w("### Fixed 512-row chunks against the adaptive chunk")
    w("")
    w("| shape | chunk before | units | ms | GB/s | chunk after | units | ms | GB/s | speed-up |")
    w("| :-- | ---: | ---: | ---: | ---: | ---: | ---: | ---: | ---: | ---: |")
    for b, a in zip(before, after):
        w(f"| {b['shape']} | {b['chunk']} | {b['units']} | {b['ms']:.4f} | {b['gbs']:.1f} | "
          f"{a['chunk']} | {a['units']} | {a['ms']:.4f} | {a['gbs']:.1f} | "
          f"{b['ms'] / a['ms']:.2f}x |")
    w("")
    w("### Adaptive decode across shapes")
    w("")
    w("| shape | path | chunk | units | ms | GB/s | % of HBM peak |")
    w("| :-- | :-- | ---: | ---: | ---: | ---: | ---: |")
    for r in adaptive:
        w(f"| {r['shape']} | {r['path']} | {r['chunk']} | {r['units']} | {r['ms']:.4f} | "
          f"{r['gbs']:.1f} | {r['pct_hbm']:.1f}% |")
    w("")
    w("At B = 1 the decode step is a few microseconds of launch and memory latency: the")
    w("cache is read at a fraction of the HBM rate because one (b, h) cannot keep enough")
    w("bytes in flight. The ragged B = 32 batch of config 5 is where the pass streams at")
    w("the HBM roofline (bench.py).")
    return "\n".join(out).rstrip() + "\n"


def _timeit(fn, iters=30, warmup=10, clock_s=0.2):
    """Median of three event-timed loops, after `clock_s` seconds of untimed
    launches (the GPU reaches its sustained clock) and `warmup` more."""
    import time

    import torch

    t_end = time.perf_counter() + clock_s
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(3):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn()
        end.record()
        torch.cuda.synchronize()
        samples.append(start.elapsed_time(end) / iters)
    return sorted(samples)[1]


def _prefill_rows(fa):
    import torch

    rows = []
    g = torch.Generator().manual_seed(0)
    for batch, heads, seq, causal in PREFILL_SHAPES:
        shape = (batch, heads, seq, HEAD_DIM)
        q, k, v = (torch.randn(shape, generator=g).half().cuda() for _ in range(3))
        ms = _timeit(lambda: fa.prefill(q, k, v, causal, SCALE))
        rows.append(prefill_model(batch, heads, seq, causal, ms))
        print(f"  prefill {rows[-1]['shape']}: {ms * 1e3:.1f} us", flush=True)
        del q, k, v
    return rows


def _decode_rows(fa, shapes, cus, split=0):
    import torch

    rows = []
    g = torch.Generator().manual_seed(0)
    for batch, heads, seq in shapes:
        q = torch.randn((batch, heads, 1, HEAD_DIM), generator=g).half().cuda()
        k = torch.randn((batch, heads, seq, HEAD_DIM), generator=g).half().cuda()
        v = torch.randn((batch, heads, seq, HEAD_DIM), generator=g).half().cuda()
        lens = torch.full((batch,), seq, dtype=torch.int32).cuda()
        if split:
            chunk = split
            fn = lambda: fa._decode_with_split(q, k, v, lens, SCALE, split)  # noqa: E731
        else:
            chunk = fa.choose_decode_split(seq, batch, heads, 2 * cus)
            fn = lambda: fa.decode(q, k, v, lens, SCALE)  # noqa: E731
        ms = _timeit(fn)
        rows.append(decode_model(batch, heads, seq, chunk, decode_path(batch, heads, seq, cus), ms))
        print(f"  decode {rows[-1]['shape']} chunk {chunk}: {ms * 1e3:.1f} us", flush=True)
        del q, k, v, lens
    return rows


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--out", default=os.path.join("gpurun_out", "analysis.md"))
    args = parser.parse_args(argv)

    import torch

    if not torch.cuda.is_available():
        raise SystemExit("run_analysis.py needs a GPU (an MI355X)")
    import flashattn_cuda as fa

    props = torch.cuda.get_device_properties(0)
    cus = props.multi_processor_count
    device = [
        ("GPU", f"{props.name} ({getattr(props, 'gcnArchName', 'gfx950')})"),
        ("compute units", str(cus)),
        ("HBM", f"{props.total_memory / 2**30:.0f} GiB"),
        ("peaks used", f"{MFMA_PEAK_TFLOPS:,.1f} TFLOP/s fp16 MFMA (dense), "
                       f"{HBM_PEAK_GBS:,.0f} GB/s HBM3E"),
        ("torch", torch.__version__),
        ("decode chunk target", f"2 x CUs = {2 * cus} units"),
    ]
    print("prefill roofline ...", flush=True)
    prefill = _prefill_rows(fa)
    print("decode split study ...", flush=True)
    before = _decode_rows(fa, DECODE_STUDY_SHAPES, cus, split=512)
    after = _decode_rows(fa, DECODE_STUDY_SHAPES, cus)
    adaptive = _decode_rows(fa, DECODE_SHAPES, cus)
    command = "python flash-attention-cuda_amd/profile/run_analysis.py --out " + args.out
    text = render(device, fa.occupancy_report(), prefill, before, after, adaptive, command)
    os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
    with open(args.out, "w", encoding="utf-8") as handle:
        handle.write(text)
    print(f"wrote {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
