"""Seeded random shapes against the oracle: prefill (plain and grouped K/V,
causal and full) and ragged decode (plain and grouped, lengths out of range
included), both head sizes, standard and wide scales.

Each case draws its shape from its own seed, so a failure names a shape that
reproduces. The bar is the fp32-output hook within 2.44e-4 of the oracle and
the fp16 output equal to the round-to-nearest of it, as in test_parity.py.
FA_RANDOM_CASES=<n> runs the first n cases of each kind (default 40) for a
wider sweep with the same seeds.
"""

import math
import os
import random

import numpy as np
import pytest
import torch

import flashattn_cuda
import oracle

pytestmark = pytest.mark.gpu

BOUND = 2.44e-4
N_CASES = int(os.environ.get("FA_RANDOM_CASES", "40"))
SEQS = [1, 2, 31, 63, 64, 65, 127, 128, 129, 200, 255, 256, 257, 300, 511, 512, 513, 700,
        1000, 1023, 1024, 1100]
CACHES = [1, 63, 64, 100, 512, 513, 1000, 2048, 3000]


def _prefill_case(i):
    rng = random.Random(10_000 + i)
    d = rng.choice([64, 128])
    batch, kv_heads, group = rng.randint(1, 2), rng.randint(1, 3), rng.choice([1, 1, 2, 3, 7])
    seq = rng.choice(SEQS)
    while batch * kv_heads * group * seq * seq > 2.5e7 and (batch, kv_heads, group) != (1, 1, 1):
        if batch > 1:
            batch -= 1
        elif kv_heads > 1:
            kv_heads -= 1
        else:
            group = 1
    causal = rng.random() < 0.6
    scale = rng.choice([1 / math.sqrt(d), -1 / math.sqrt(d), 0.05, 0.3])
    return d, batch, kv_heads * group, kv_heads, seq, causal, scale


def _decode_case(i):
    rng = random.Random(20_000 + i)
    d = rng.choice([64, 128])
    batch, kv_heads, group = rng.randint(1, 24), rng.randint(1, 3), rng.choice([1, 1, 2, 7])
    max_seq = rng.choice(CACHES)
    lens = [rng.randint(-2, max_seq + 4) for _ in range(batch)]
    scale = rng.choice([1 / math.sqrt(d), 0.3])
    return d, batch, kv_heads * group, kv_heads, max_seq, lens, scale


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_prefill_shape(i):
    d, batch, heads, kv_heads, seq, causal, scale = _prefill_case(i)
    label = f"prefill case {i}: B{batch} H{heads} Hkv{kv_heads} S{seq} D{d} causal={causal} scale={scale:.4f}"
    print(label, flush=True)
    q, _, _ = oracle.make_prefill_inputs(batch, heads, seq, seed=300 + i, head_dim=d)
    _, k, v = oracle.make_prefill_inputs(batch, kv_heads, seq, seed=400 + i, head_dim=d)
    ref = oracle.prefill_gqa(q.numpy(), k.numpy(), v.numpy(), causal, scale)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    if heads == kv_heads:
        out32 = flashattn_cuda._prefill_fp32(qd, kd, vd, causal, scale)
        out16 = flashattn_cuda.prefill(qd, kd, vd, causal, scale)
    else:
        out32 = flashattn_cuda._prefill_gqa_fp32(qd, kd, vd, causal, scale)
        out16 = flashattn_cuda.prefill_gqa(qd, kd, vd, causal, scale)
    err = float(np.abs(out32.cpu().numpy().astype(np.float64) - ref).max())
    print(f"  fp32-out err {err:.3e}")
    assert err <= BOUND, label
    assert torch.equal(out16.cpu(), out32.half().cpu()), label


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_decode_shape(i):
    d, batch, heads, kv_heads, max_seq, lens, scale = _decode_case(i)
    label = (f"decode case {i}: B{batch} H{heads} Hkv{kv_heads} Lmax{max_seq} D{d} "
             f"scale={scale:.4f} lens[:4]={lens[:4]}")
    print(label, flush=True)
    g = torch.Generator().manual_seed(500 + i)
    q = torch.randn((batch, heads, 1, d), generator=g).half()
    k = torch.randn((batch, kv_heads, max_seq, d), generator=g).half()
    v = torch.randn((batch, kv_heads, max_seq, d), generator=g).half()
    sl = torch.tensor(lens, dtype=torch.int32)
    ref = oracle.decode_gqa(q.numpy(), k.numpy(), v.numpy(), sl.numpy(), scale)
    qd, kd, vd, ld = q.cuda(), k.cuda(), v.cuda(), sl.cuda()
    if heads == kv_heads:
        out32 = flashattn_cuda._decode_fp32(qd, kd, vd, ld, scale)
        out16 = flashattn_cuda.decode(qd, kd, vd, ld, scale)
    else:
        out32 = flashattn_cuda._decode_gqa_fp32(qd, kd, vd, ld, scale)
        out16 = flashattn_cuda.decode_gqa(qd, kd, vd, ld, scale)
    err = float(np.abs(out32.cpu().numpy().astype(np.float64) - ref).max())
    print(f"  fp32-out err {err:.3e}")
    assert err <= BOUND, label
    assert torch.equal(out16.cpu(), out32.half().cpu()), label
