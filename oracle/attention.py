"""CPU oracle for the prefill / decode hot path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker or the timed CPU baseline. The product path (``flashattn_cuda``)
never calls it and has no CPU fallback.

What it restates (paths relative to shrvan30/flash-attention-cuda):

* ``stable_softmax`` / ``attention_cpu``: src/attention_cpu.py:13-27 and
  :29-62 -- numpy fp32, S = (Q @ K.T) * scale, row-max-subtracted softmax,
  O = P @ V. Extended with an optional causal mask (-inf above the
  diagonal, key j visible to query i iff j <= i, as csrc/prefill.cu:268);
  the reference CPU path itself has no mask.
* ``prefill``: the per-(b, h) loop over ``attention_cpu`` -- the oracle role
  of ``sdpa_reference`` in tests/test_correctness.py:29-34 (fp32 maths on
  upcast fp16 inputs).
* ``decode``: tests/test_correctness.py:37-44 (per-sequence attention over
  cache rows [:n]) with the kernel's edge semantics from csrc/decode.cu:69
  (n = min(seq_lens[b], Lmax)) and :155-172 (n <= 0 gives a zero output).
* ``prefill_gqa`` / ``decode_gqa``: grouped-query attention, which the
  reference leaves to its callers (README.md:398, "Kernel-side GQA (stop
  paying the host-side KV repeat)"): K/V carry H_kv heads and query head h
  reads K/V head h // (H // H_kv), the pairing of
  ``repeat_interleave(H // H_kv, dim=1)``; restated as ``prefill`` /
  ``decode`` on the repeated K/V.
* ``kv_append``: the cache write the reference's caller performs before each
  decode step (README.md:9-13: the FlashStack engine writes token t at row
  seq_lens[b]); restated as: for 0 <= seq_lens[b] < Lmax, row seq_lens[b] of
  every K/V head of sequence b takes the new token, then seq_lens[b] += 1.
* ``legacy_attention``: the function the reference's v1 kernels compute
  (src/legacy/naive_attention.cu:45-110, tiled_attention.cu:28-205,
  fused_attention.cu:54-200, launched with scale 1/sqrt(d) by
  :139 / :240 / :213): one (N, 64) fp32 head, no mask -- ``attention_cpu``
  with its default scale.
* ``choose_decode_split``: csrc/decode.cu:183-192 (integer closed form).
* ``attention_flops``: bench/run_bench.py:102-107 (4 B H N^2 d, halved when
  causal). ``decode_bytes``: K and V rows actually read plus q, o, seq_lens.
* Every function above is written for any head size (the shapes carry it);
  head_dim 128, the reference's named next step (README.md:397), is pinned
  like 64 (tests/test_oracle.py).
* ``make_prefill_inputs`` / ``make_decode_inputs``: the deterministic
  CPU-seeded input recipe used by the tests and the benchmark (torch CPU
  generator seeded with 0, fp32 randn cast to fp16, drawn in the order q, k,
  v; ragged lengths drawn first).

How each function is pinned (tests/test_oracle.py): fp64 brute force on tiny
inputs written as explicit loops, torch CPU ``scaled_dot_product_attention``
in fp32, closed forms (constant V rows, scale 0 gives the visible-row mean,
causal row 0 equals V row 0), key-permutation invariance, decode(t) equal to
causal prefill row t, the chooser's pins from tests/test_correctness.py:180-198,
and planted mistakes (wrong mask edge, transposed operand, scale applied
twice) that those checks must reject. The committed fixtures under
tests/golden/ hold inputs and fp64 outputs of an independent brute force.
"""

from __future__ import annotations

import numpy as np

HEAD_DIM = 64
DECODE_SPLIT_MIN = 128
DECODE_SPLIT_MAX = 1024


def stable_softmax(x: np.ndarray) -> np.ndarray:
    """Row softmax with the row max subtracted (src/attention_cpu.py:13-27).

    Works on the last axis; a row may contain -inf entries (masked keys) as
    long as one entry is finite.
    """
    x_max = np.max(x, axis=-1, keepdims=True)
    x_exp = np.exp(x - x_max)
    x_sum = np.sum(x_exp, axis=-1, keepdims=True)
    return x_exp / x_sum


def attention_cpu(Q, K, V, scale=None, causal=False):
    """softmax(Q K^T * scale) V for one head (src/attention_cpu.py:29-62).

    Q: (N, d), K and V: (M, d), all fp32. ``causal`` masks key j for query i
    when j > i + (M - N) (bottom-right aligned; M == N is the prefill case).
    """
    N, d = Q.shape
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    S = (Q @ K.T) * np.float32(scale)
    if causal:
        M = K.shape[0]
        i = np.arange(N)[:, None]
        j = np.arange(M)[None, :]
        S = np.where(j <= i + (M - N), S, np.float32(-np.inf))
    P = stable_softmax(S)
    return P @ V


def prefill(q, k, v, causal: bool, scale: float) -> np.ndarray:
    """[B, H, S, 64] -> [B, H, S, 64] fp32, one ``attention_cpu`` per head."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    B, H, S, D = q.shape
    out = np.empty((B, H, S, D), dtype=np.float32)
    for b in range(B):
        for h in range(H):
            out[b, h] = attention_cpu(q[b, h], k[b, h], v[b, h], scale, causal)
    return out


def decode(q, k_cache, v_cache, seq_lens, scale: float) -> np.ndarray:
    """[B, H, 1, 64] query over [B, H, Lmax, 64] caches -> [B, H, 1, 64] fp32.

    Sequence b attends rows [0, min(seq_lens[b], Lmax)); a sequence with no
    rows gets zeros.
    """
    q = np.asarray(q, dtype=np.float32)
    k_cache = np.asarray(k_cache, dtype=np.float32)
    v_cache = np.asarray(v_cache, dtype=np.float32)
    lens = np.asarray(seq_lens).astype(np.int64)
    B, H, _, D = q.shape
    lmax = k_cache.shape[2]
    out = np.zeros((B, H, 1, D), dtype=np.float32)
    for b in range(B):
        n = int(min(lens[b], lmax))
        if n <= 0:
            continue
        for h in range(H):
            out[b, h] = attention_cpu(q[b, h], k_cache[b, h, :n], v_cache[b, h, :n], scale)
    return out


def legacy_attention(q, k, v) -> np.ndarray:
    """(N, 64) fp32 -> (N, 64) fp32: softmax(q k^T / sqrt(64)) v, no mask.

    The v1 kernels (src/legacy/*_attention.cu) take no scale argument; their
    launchers pass 1 / sqrt(d) (naive_attention.cu:139, tiled_attention.cu:240,
    fused_attention.cu:213).
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    return attention_cpu(q, k, v, scale=None, causal=False)


def repeat_kv(x, heads: int) -> np.ndarray:
    """[B, H_kv, N, 64] -> [B, heads, N, 64]: K/V head g repeated for query
    heads g * G .. g * G + G - 1 (G = heads // H_kv), as repeat_interleave."""
    x = np.asarray(x, dtype=np.float32)
    kv = x.shape[1]
    if kv <= 0 or heads % kv != 0:
        raise ValueError(f"H_kv={kv} must divide H={heads}")
    return np.repeat(x, heads // kv, axis=1)


def prefill_gqa(q, k, v, causal: bool, scale: float) -> np.ndarray:
    """``prefill`` with k, v of shape [B, H_kv, S, 64] (H_kv divides H)."""
    heads = np.asarray(q).shape[1]
    return prefill(q, repeat_kv(k, heads), repeat_kv(v, heads), causal, scale)


def decode_gqa(q, k_cache, v_cache, seq_lens, scale: float) -> np.ndarray:
    """``decode`` with caches of shape [B, H_kv, Lmax, 64] (H_kv divides H)."""
    heads = np.asarray(q).shape[1]
    return decode(q, repeat_kv(k_cache, heads), repeat_kv(v_cache, heads), seq_lens, scale)


def kv_append(k_cache, v_cache, k_new, v_new, seq_lens):
    """Returns (k_cache, v_cache, seq_lens) after appending one token per
    sequence: k_new, v_new are [B, H_kv, 1, 64]; sequences whose length is
    negative or already Lmax are left unchanged. The inputs are not modified."""
    k_cache = np.array(k_cache, copy=True)
    v_cache = np.array(v_cache, copy=True)
    lens = np.array(seq_lens, dtype=np.int32, copy=True)
    lmax = k_cache.shape[2]
    for b in range(lens.shape[0]):
        n = int(lens[b])
        if 0 <= n < lmax:
            k_cache[b, :, n] = np.asarray(k_new)[b, :, 0]
            v_cache[b, :, n] = np.asarray(v_new)[b, :, 0]
            lens[b] = n + 1
    return k_cache, v_cache, lens


def choose_decode_split(max_seq: int, batch: int, heads: int, min_blocks: int) -> int:
    """Largest power-of-two chunk in [128, 1024] reaching ``min_blocks`` blocks."""
    per_split = batch * heads
    split = DECODE_SPLIT_MAX
    while split > DECODE_SPLIT_MIN:
        if per_split * (-(-max_seq // split)) >= min_blocks:
            return split
        split >>= 1
    return DECODE_SPLIT_MIN


def attention_flops(batch: int, heads: int, seq: int, causal: bool, head_dim: int = HEAD_DIM) -> float:
    """4 * B * H * N^2 * d, halved when causal (the reference's convention)."""
    flops = 4.0 * batch * heads * seq * seq * head_dim
    return flops * 0.5 if causal else flops


def decode_bytes(heads: int, seq_lens, max_seq: int, head_dim: int = HEAD_DIM) -> int:
    """HBM bytes one decode call must move: valid K and V rows (fp16), the
    fp16 query and output, and the int32 lengths. Split-K workspace excluded."""
    lens = np.clip(np.asarray(seq_lens, dtype=np.int64), 0, max_seq)
    batch = lens.shape[0]
    kv = 2 * heads * head_dim * 2 * int(lens.sum())
    qo = 2 * batch * heads * head_dim * 2
    return kv + qo + 4 * batch


def make_prefill_inputs(batch: int, heads: int, seq: int, seed: int = 0,
                        head_dim: int = HEAD_DIM):
    """CPU-seeded fp16 q, k, v of shape [B, H, S, head_dim] (torch tensors)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    shape = (batch, heads, seq, head_dim)
    q = torch.randn(shape, generator=g, dtype=torch.float32).half()
    k = torch.randn(shape, generator=g, dtype=torch.float32).half()
    v = torch.randn(shape, generator=g, dtype=torch.float32).half()
    return q, k, v


def make_decode_inputs(batch: int, heads: int, max_seq: int, seed: int = 0, lens=None,
                       head_dim: int = HEAD_DIM):
    """CPU-seeded decode inputs: lengths (uniform in [1, max_seq] unless given,
    drawn first), then q [B, H, 1, D], k_cache, v_cache [B, H, Lmax, D]."""
    import torch

    g = torch.Generator().manual_seed(seed)
    if lens is None:
        lens = torch.randint(1, max_seq + 1, (batch,), generator=g, dtype=torch.int64)
    lens = torch.as_tensor(lens, dtype=torch.int32)
    q = torch.randn((batch, heads, 1, head_dim), generator=g, dtype=torch.float32).half()
    shape = (batch, heads, max_seq, head_dim)
    k = torch.randn(shape, generator=g, dtype=torch.float32).half()
    v = torch.randn(shape, generator=g, dtype=torch.float32).half()
    return q, k, v, lens


def fp16_half_ulp(x: np.ndarray) -> np.ndarray:
    """Half the fp16 spacing at |x| (normal range; 2^-25 below 2^-14)."""
    ax = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(ax, 2.0 ** -14)))
    return 2.0 ** (e - 11)


def fp16_rounding_floor(ref32: np.ndarray) -> float:
    """max |fp16(ref) - ref|: the error any fp16-output kernel shows against an
    fp32 reference even when its pre-rounding result is exact."""
    ref = np.asarray(ref32, dtype=np.float32)
    return float(np.max(np.abs(ref.astype(np.float16).astype(np.float64) - ref.astype(np.float64))))
