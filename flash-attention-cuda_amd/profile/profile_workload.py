"""Single-purpose workloads for the rocprofv3 harness (profile_rocprof.sh).

    python profile_workload.py NAME            # run one workload
    python profile_workload.py occupancy PATH  # write occupancy_report() as JSON
    python profile_workload.py list            # print the workload table as JSON

Each workload builds its inputs on the CPU from a fixed seed (the recipe of
the benchmark), moves them to the GPU (enough copies, rotated call by call,
that their total exceeds twice the 256 MB MALL, as bench.py's per-config
sweep does), runs 0.1 s of untimed launches (the GPU reaches its sustained
clock), then 5 warm-up and ITERS profiled calls. It is
the counterpart of the reference's bench/profile_workload.py (prefill and
decode workloads for its Nsight captures), over this build's BASELINE configs.

WORKLOADS gives, per name, the algorithmic work of ONE call of its main
kernel (FLOPs for prefill, bytes for decode, by the same conventions as
bench.py), which rocprof_extract.py divides by the measured durations.
"""

from __future__ import annotations

import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # the package root (flashattn_cuda)

ITERS = 20
SCALE = 0.125
MALL_BYTES = 256 << 20

# name -> (description, main kernel (short name prefix), unit, work per call)
WORKLOADS = {
    "prefill_c3": ("config 3: causal prefill B=1 H=14 S=4096", "prefill_kernel<64, true",
                   "flop", 4.0 * 14 * 4096 * 4096 * 64 / 2),
    "prefill_c2_causal": ("config 2: causal prefill B=4 H=12 S=1024", "prefill_kernel<64, true",
                          "flop", 4.0 * 4 * 12 * 1024 * 1024 * 64 / 2),
    "prefill_c2_full": ("config 2: full prefill B=4 H=12 S=1024", "prefill_kernel<64, false",
                        "flop", 4.0 * 4 * 12 * 1024 * 1024 * 64),
    "prefill_c3_d128": ("config 3 shape at head_dim 128: causal prefill B=1 H=14 S=4096 D=128, scale 1/sqrt(128)",
                        "prefill_kernel<128, true", "flop", 4.0 * 14 * 4096 * 4096 * 128 / 2),
    "decode_c4": ("config 4: decode B=1 H=12 L=4096 (split-K, merged in the same launch)",
                  "decode_split_fused_kernel",
                  "byte", 2 * 12 * 64 * 2 * 4096 + 2 * 12 * 64 * 2 + 4),
    "decode_c5": ("config 5: ragged decode B=32 H=14 Lmax=4096, lens U[1,4096] seed 0",
                  "decode_bh_kernel", "byte", 2 * 14 * 64 * 2 * 73374 + 2 * 32 * 14 * 64 * 2 + 128),
    "decode_c5_d128": ("config 5 shape at head_dim 128: ragged decode B=32 H=14 Lmax=4096 D=128, scale 1/sqrt(128)",
                       "decode_bh_kernel<128", "byte",
                       2 * 14 * 128 * 2 * 73374 + 2 * 32 * 14 * 128 * 2 + 128),
    "decode_gqa_c5": ("config 5 batch with 2 K/V heads (group 7): grouped decode",
                      "decode_group_kernel", "byte", 2 * 2 * 64 * 2 * 73374 + 2 * 32 * 14 * 64 * 2 + 128),
    "copy_1g": ("1 GiB device copy (byte-counter calibration)", "copyBuffer", "byte",
                2.0 * (1 << 30)),
}


def _clock_warmup(fn, seconds=0.1):
    import torch

    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def _run(fns):
    import torch

    n = len(fns)
    _clock_warmup(fns[0])
    for i in range(5):
        fns[i % n]()
    torch.cuda.synchronize()
    for i in range(ITERS):
        fns[i % n]()
    torch.cuda.synchronize()


def _prefill(batch, heads, seq, causal, d=64):
    import torch

    import flashattn_cuda as fa

    g = torch.Generator().manual_seed(0)
    shape = (batch, heads, seq, d)
    q, k, v = (torch.randn(shape, generator=g).half().cuda() for _ in range(3))
    # Rotate input copies through more than 2x the MALL, as bench.py's
    # per-config sweep (the reference protocol) does.
    n = _copies(3 * q.numel() * 2)
    sets = [(q, k, v)] + [tuple(t.clone() for t in (q, k, v)) for _ in range(n - 1)]
    _run([lambda s=s: fa.prefill(s[0], s[1], s[2], causal, d ** -0.5) for s in sets])


def _decode_inputs(batch, heads, lmax, lens=None, d=64):
    import torch

    g = torch.Generator().manual_seed(0)
    rl = torch.randint(1, lmax + 1, (batch,), generator=g).to(torch.int32)
    if lens is not None:
        rl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn((batch, heads, 1, d), generator=g).half()
    k = torch.randn((batch, heads, lmax, d), generator=g).half()
    v = torch.randn((batch, heads, lmax, d), generator=g).half()
    return q, k, v, rl


def _copies(nbytes):
    return max(1, math.ceil(2 * MALL_BYTES / max(nbytes, 1)) + 1)


def _decode(batch, heads, lmax, lens=None, kv_every=1, d=64):
    import flashattn_cuda as fa

    q, k, v, rl = _decode_inputs(batch, heads, lmax, lens, d)
    call = fa.decode
    if kv_every > 1:  # grouped: keep K/V heads 0, G, 2G, ...
        k, v = k[:, ::kv_every].contiguous(), v[:, ::kv_every].contiguous()
        call = fa.decode_gqa
    q, rl = q.cuda(), rl.cuda()
    n = _copies(2 * k.numel() * 2)  # rotate caches through more than 2x the MALL
    sets = [(k.cuda(), v.cuda()) for _ in range(n)]
    _run([lambda s=s: call(q, s[0], s[1], rl, d ** -0.5) for s in sets])


def _copy():
    import torch

    src = torch.empty(1 << 29, device="cuda", dtype=torch.float16)  # 1 GiB, contents unused
    dst = torch.empty_like(src)
    _run([lambda: dst.copy_(src)])


RUNNERS = {
    "prefill_c3": lambda: _prefill(1, 14, 4096, True),
    "prefill_c2_causal": lambda: _prefill(4, 12, 1024, True),
    "prefill_c2_full": lambda: _prefill(4, 12, 1024, False),
    "prefill_c3_d128": lambda: _prefill(1, 14, 4096, True, d=128),
    "decode_c4": lambda: _decode(1, 12, 4096, lens=[4096]),
    "decode_c5": lambda: _decode(32, 14, 4096),
    "decode_gqa_c5": lambda: _decode(32, 14, 4096, kv_every=7),
    "decode_c5_d128": lambda: _decode(32, 14, 4096, d=128),
    "copy_1g": _copy,
}


def main(argv):
    if len(argv) >= 2 and argv[1] == "list":
        print(json.dumps({k: list(v) for k, v in WORKLOADS.items()}))
        return 0
    if len(argv) == 3 and argv[1] == "occupancy":
        import flashattn_cuda as fa

        with open(argv[2], "w", encoding="utf-8") as handle:
            json.dump(fa.occupancy_report(), handle, indent=1)
        return 0
    if len(argv) != 2 or argv[1] not in RUNNERS:
        print(f"usage: {argv[0]} {{{'|'.join(RUNNERS)}|list|occupancy PATH}}", file=sys.stderr)
        return 2
    RUNNERS[argv[1]]()
    print(f"{argv[1]}: done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
