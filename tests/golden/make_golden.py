"""Write the committed golden fixtures for the prefill / decode path.

    python tests/golden/make_golden.py

The reference ships no golden vectors (its tests draw inputs on the CUDA RNG
at run time), so these fixtures are built here from first principles: the
inputs come from the CPU-seeded recipe (torch.Generator().manual_seed(seed),
fp32 randn cast to fp16) and the expected outputs from an fp64 brute force
written independently of oracle/attention.py -- one query row at a time,
explicit max / exp / sum with math.fsum, no matrix products and no shared
helper. The fixtures pin the oracle (tests/test_oracle.py) and the GPU
kernels (tests/test_parity.py).

Cases (all head_dim 64, scale 1/8 unless stated):
  prefill_{causal,full}_s{1,37,130}   B=1 H=2, ragged lengths around tiles
  prefill_causal_s70_negscale          B=1 H=1, scale -0.3 (sign folding)
  decode_ragged                        B=3 H=2 Lmax=130, lens [1, 63, 130]
  decode_edges                         B=3 H=1 Lmax=8, lens [0, 9, -2]
                                       (empty, clamped to Lmax, negative)
"""

from __future__ import annotations

import math
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
D = 64


def _inputs(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float32).half().numpy() for _ in range(3)]


def _row_attention(qrow, keys, vals, scale):
    """fp64 softmax(q . k_j * scale) v for one query row, keys as a list."""
    if len(keys) == 0:
        return [0.0] * D
    scores = [math.fsum(float(a) * float(b) for a, b in zip(qrow, kj)) * scale for kj in keys]
    mx = max(scores)
    w = [math.exp(s - mx) for s in scores]
    tot = math.fsum(w)
    return [math.fsum(w[j] * float(vals[j][d]) for j in range(len(keys))) / tot for d in range(D)]


def brute_prefill(q, k, v, causal, scale):
    B, H, S, _ = q.shape
    out = np.zeros((B, H, S, D), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            kk = [list(k[b, h, j]) for j in range(S)]
            vv = [list(v[b, h, j]) for j in range(S)]
            for i in range(S):
                n = i + 1 if causal else S
                out[b, h, i] = _row_attention(list(q[b, h, i]), kk[:n], vv[:n], scale)
    return out


def brute_decode(q, k, v, lens, scale):
    B, H, _, _ = q.shape
    lmax = k.shape[2]
    out = np.zeros((B, H, 1, D), dtype=np.float64)
    for b in range(B):
        n = max(0, min(int(lens[b]), lmax))
        for h in range(H):
            kk = [list(k[b, h, j]) for j in range(n)]
            vv = [list(v[b, h, j]) for j in range(n)]
            out[b, h, 0] = _row_attention(list(q[b, h, 0]), kk, vv, scale)
    return out


def main():
    cases = {}
    for causal in (True, False):
        for seq in (1, 37, 130):
            q, k, v = _inputs((1, 2, seq, D), seed=100 + seq)
            name = f"prefill_{'causal' if causal else 'full'}_s{seq}"
            cases[name] = dict(kind="prefill", q=q, k=k, v=v, causal=causal, scale=0.125,
                               out=brute_prefill(q, k, v, causal, 0.125))
    q, k, v = _inputs((1, 1, 70, D), seed=7)
    cases["prefill_causal_s70_negscale"] = dict(kind="prefill", q=q, k=k, v=v, causal=True,
                                                scale=-0.3, out=brute_prefill(q, k, v, True, -0.3))
    q, _, _ = _inputs((3, 2, 1, D), seed=11)
    _, k, v = _inputs((3, 2, 130, D), seed=12)
    lens = np.array([1, 63, 130], dtype=np.int32)
    cases["decode_ragged"] = dict(kind="decode", q=q, k=k, v=v, lens=lens, scale=0.125,
                                  out=brute_decode(q, k, v, lens, 0.125))
    q, _, _ = _inputs((3, 1, 1, D), seed=13)
    _, k, v = _inputs((3, 1, 8, D), seed=14)
    lens = np.array([0, 9, -2], dtype=np.int32)
    cases["decode_edges"] = dict(kind="decode", q=q, k=k, v=v, lens=lens, scale=0.125,
                                 out=brute_decode(q, k, v, lens, 0.125))

    for name, c in cases.items():
        arrays = {key: np.asarray(val) for key, val in c.items()}
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print(name, {key: getattr(val, "shape", val) for key, val in arrays.items() if key != "kind"})


if __name__ == "__main__":
    main()
