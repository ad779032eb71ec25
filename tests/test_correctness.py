"""Correctness of the gfx950 kernels, ported from the reference's contract
(tests/test_correctness.py of shrvan30/flash-attention-cuda, 90 GPU cases).

Same parametrisations, tolerance (2e-3 on fp16 outputs) and error-message
checks. Differences, each deliberate:

* Inputs are drawn on a CPU generator and moved to the device, so every case
  is reproducible on any machine and by the CPU oracle.
* The fp32 reference is an explicit masked softmax on upcast inputs with
  contiguous operands (the reference used fp32 SDPA on the GPU; same maths).
* test_decode_split_choice_targets_the_device is restated for 256 CUs: the
  original asserted blocks >= 2 x SMs for shapes that cannot reach 512
  blocks with chunks >= 128, so here a shape either reaches the target with
  the largest such chunk, or falls back to chunk 128.
"""

import math

import pytest
import torch

import flashattn_cuda

HEAD_DIM = flashattn_cuda.head_dim
SCALE = 1.0 / math.sqrt(HEAD_DIM)
TOL = 2e-3

pytestmark = pytest.mark.gpu


def rand(*shape, seed=None, _state={}):
    if seed is not None:
        _state["g"] = torch.Generator().manual_seed(seed)
    g = _state.setdefault("g", torch.Generator().manual_seed(0))
    return torch.randn(*shape, generator=g, dtype=torch.float32).half().cuda()


def sdpa_reference(q, k, v, causal, scale=SCALE):
    """Prefill oracle: an explicit masked softmax per (b, h) in fp32 on the
    upcast inputs, rounded back to fp16 at the end."""
    out = torch.empty_like(q)
    for b in range(q.shape[0]):
        qf, kf, vf = q[b].float(), k[b].float(), v[b].float()
        s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
        if causal:
            n = q.shape[2]
            mask = torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1)
            s = s.masked_fill(mask, float("-inf"))
        out[b] = torch.matmul(torch.softmax(s, dim=-1), vf).half()
    return out


def decode_reference(q, k_cache, v_cache, seq_lens, scale=SCALE):
    """Decode oracle: each query attends, in fp32, to cache rows [0, len)
    of its own sequence only."""
    out = torch.empty_like(q)
    for b in range(q.shape[0]):
        n = int(seq_lens[b])
        scores = torch.matmul(q[b].float(), k_cache[b, :, :n].float().transpose(-1, -2).contiguous()) * scale
        out[b] = torch.matmul(torch.softmax(scores, dim=-1), v_cache[b, :, :n].float()).half()
    return out


def max_abs_diff(a, b):
    return (a.float() - b.float()).abs().max().item()


# ---------------------------------------------------------------------------
# Prefill
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("heads", [8, 12, 14])
@pytest.mark.parametrize("seq", [128, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_sdpa(batch, heads, seq, causal):
    q = rand(batch, heads, seq, HEAD_DIM, seed=0)
    k = rand(batch, heads, seq, HEAD_DIM)
    v = rand(batch, heads, seq, HEAD_DIM)

    out = flashattn_cuda.prefill(q, k, v, causal, SCALE)
    ref = sdpa_reference(q, k, v, causal)

    assert max_abs_diff(out, ref) <= TOL


@pytest.mark.parametrize("seq", [1, 37, 65, 130, 1023])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_handles_ragged_sequence_lengths(seq, causal):
    """Sequence lengths that leave a partial last tile (ragged tails)."""
    q = rand(2, 5, seq, HEAD_DIM, seed=1)
    k = rand(2, 5, seq, HEAD_DIM)
    v = rand(2, 5, seq, HEAD_DIM)

    out = flashattn_cuda.prefill(q, k, v, causal, SCALE)
    ref = sdpa_reference(q, k, v, causal)

    assert max_abs_diff(out, ref) <= TOL


# ---------------------------------------------------------------------------
# Decode
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("position", [1, 17, 511, 1024, 2047])
def test_decode_matches_causal_prefill_row(position):
    """A decode step at cache length t + 1 sees exactly what causal prefill
    row t sees, so the two outputs agree."""
    batch, heads, seq = 2, 12, 2048
    q = rand(batch, heads, seq, HEAD_DIM, seed=2)
    k = rand(batch, heads, seq, HEAD_DIM)
    v = rand(batch, heads, seq, HEAD_DIM)

    full = flashattn_cuda.prefill(q, k, v, True, SCALE)

    q_step = q[:, :, position : position + 1, :].contiguous()
    seq_lens = torch.full((batch,), position + 1, dtype=torch.int32, device="cuda")
    out = flashattn_cuda.decode(q_step, k, v, seq_lens, SCALE)

    assert max_abs_diff(out, full[:, :, position : position + 1, :]) <= TOL


@pytest.mark.parametrize(
    "seq_lens",
    [
        [1, 2, 512, 4096],
        [513, 1023, 1024, 3000],
        [64, 65, 127, 129],
        [4096, 1, 2048, 7],
    ],
)
def test_decode_ragged_batch(seq_lens):
    """One batch, four different fill levels per cache (1 row to full)."""
    batch, heads, cache = len(seq_lens), 8, 4096
    q = rand(batch, heads, 1, HEAD_DIM, seed=3)
    k_cache = rand(batch, heads, cache, HEAD_DIM)
    v_cache = rand(batch, heads, cache, HEAD_DIM)
    lens = torch.tensor(seq_lens, dtype=torch.int32, device="cuda")

    out = flashattn_cuda.decode(q, k_cache, v_cache, lens, SCALE)
    ref = decode_reference(q, k_cache, v_cache, lens)

    assert max_abs_diff(out, ref) <= TOL


@pytest.mark.parametrize("cache", [1, 63, 512, 513, 2048])
def test_decode_cache_lengths(cache):
    """Cache lengths on both sides of the 512-row path switch (whole-sequence
    kernel below, split-K above), down to a single row."""
    batch, heads = 3, 12
    q = rand(batch, heads, 1, HEAD_DIM, seed=4)
    k_cache = rand(batch, heads, cache, HEAD_DIM)
    v_cache = rand(batch, heads, cache, HEAD_DIM)
    lens = torch.full((batch,), cache, dtype=torch.int32, device="cuda")

    out = flashattn_cuda.decode(q, k_cache, v_cache, lens, SCALE)
    ref = decode_reference(q, k_cache, v_cache, lens)

    assert max_abs_diff(out, ref) <= TOL


@pytest.mark.parametrize("cache", [512, 1024, 2048])
def test_decode_is_invariant_to_split_size(cache):
    """Forcing any chunk size changes only how the work is partitioned: every
    forced result stays within the bound of the reference and close to the
    automatically chunked one."""
    batch, heads = 2, 12
    q = rand(batch, heads, 1, HEAD_DIM, seed=7)
    k_cache = rand(batch, heads, cache, HEAD_DIM)
    v_cache = rand(batch, heads, cache, HEAD_DIM)
    lens = torch.tensor([cache, cache // 2 + 1], dtype=torch.int32, device="cuda")

    chosen = flashattn_cuda.decode(q, k_cache, v_cache, lens, SCALE)
    ref = decode_reference(q, k_cache, v_cache, lens)
    assert max_abs_diff(chosen, ref) <= TOL

    for split in (128, 256, 512, 1024):
        forced = flashattn_cuda._decode_with_split(q, k_cache, v_cache, lens, SCALE, split)
        assert max_abs_diff(forced, ref) <= TOL
        assert max_abs_diff(forced, chosen) <= 1e-3


def test_decode_split_choice_targets_the_device():
    """The automatic chunk gives at least 2 x CUs units whenever some chunk
    can, and is then the coarsest one that does; otherwise the finest."""
    sms = torch.cuda.get_device_properties(0).multi_processor_count
    target = 2 * sms

    for batch, heads, seq in [(1, 12, 2048), (8, 12, 2048), (4, 12, 1024), (32, 14, 4096)]:
        split = flashattn_cuda.choose_decode_split(seq, batch, heads, target)
        assert split in (128, 256, 512, 1024)
        blocks = batch * heads * -(-seq // split)
        if blocks >= target:
            # coarsest qualifying chunk: twice as long would leave too few units
            if split < 1024:
                assert batch * heads * -(-seq // (split * 2)) < target
        else:
            assert split == 128

    # No chunk reaches the target on a small shape: the finest one is used.
    assert flashattn_cuda.choose_decode_split(512, 1, 12, target) == 128


# ---------------------------------------------------------------------------
# Input validation
# ---------------------------------------------------------------------------


def test_prefill_rejects_bad_inputs():
    q = rand(1, 2, 8, HEAD_DIM, seed=5)

    with pytest.raises(RuntimeError, match="must be fp16"):
        flashattn_cuda.prefill(q.float(), q.float(), q.float(), True, SCALE)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        flashattn_cuda.prefill(q.cpu(), q.cpu(), q.cpu(), True, SCALE)
    with pytest.raises(RuntimeError, match="must be 4-D"):
        flashattn_cuda.prefill(q[0], q[0], q[0], True, SCALE)
    with pytest.raises(RuntimeError, match="must be contiguous"):
        flashattn_cuda.prefill(q[:, :, ::2], q, q, True, SCALE)
    with pytest.raises(RuntimeError, match="head_dim"):
        bad = rand(1, 2, 8, 32)
        flashattn_cuda.prefill(bad, bad, bad, True, SCALE)
    with pytest.raises(RuntimeError, match="identical shapes"):
        flashattn_cuda.prefill(q, q[:, :, :4].contiguous(), q, True, SCALE)


def test_decode_rejects_bad_inputs():
    q = rand(1, 2, 1, HEAD_DIM, seed=6)
    cache = rand(1, 2, 8, HEAD_DIM)
    lens = torch.tensor([4], dtype=torch.int32, device="cuda")

    with pytest.raises(RuntimeError, match="exactly one query row"):
        flashattn_cuda.decode(cache, cache, cache, lens, SCALE)
    with pytest.raises(RuntimeError, match="seq_lens must be int32"):
        flashattn_cuda.decode(q, cache, cache, lens.long(), SCALE)
    with pytest.raises(RuntimeError, match="seq_lens must be 1-D"):
        flashattn_cuda.decode(q, cache, cache, lens.repeat(3), SCALE)
    with pytest.raises(RuntimeError, match="identical shapes"):
        flashattn_cuda.decode(q, cache, cache[:, :, :4].contiguous(), lens, SCALE)
