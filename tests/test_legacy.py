"""The reference's v1 single-head kernels: legacy_naive / legacy_tiled /
legacy_fused (csrc/legacy/legacy_ops.cu:10-51, src/legacy/*_attention.cu of
shrvan30/flash-attention-cuda).

They take (N, 64) fp32 q, k, v, compute softmax(q k^T / 8) v with no mask and
return a new (N, 64) fp32 tensor. The oracle is ``oracle.legacy_attention``
(pinned in tests/test_oracle.py); the three variants compute the same
function and must agree with it, and with each other, to fp32 rounding.
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import gpu_available

pytestmark = pytest.mark.gpu

requires_gpu = pytest.mark.skipif(not gpu_available(), reason="HIP device required")

FNS = ("legacy_naive", "legacy_tiled", "legacy_fused")
TOL = 2e-5  # fp32 arithmetic throughout; sums over up to 4096 keys


def _inputs(n, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, 64, generator=g, dtype=torch.float32) * scale for _ in range(3)]


@requires_gpu
@pytest.mark.parametrize("fn", FNS)
@pytest.mark.parametrize("n", [1, 7, 63, 64, 65, 100, 257, 1024, 4096])
def test_legacy_matches_oracle(fn, n):
    import flashattn_cuda as fa

    q, k, v = _inputs(n, seed=n)
    print(f"legacy {fn} n={n}", flush=True)
    out = getattr(fa, fn)(q.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == (n, 64)
    ref = oracle.legacy_attention(q.numpy(), k.numpy(), v.numpy())
    err = np.abs(out.cpu().numpy() - ref).max()
    assert err <= TOL, err


@requires_gpu
def test_legacy_variants_agree_and_survive_large_scores():
    """Scores of several hundred: every variant must subtract a running or
    exact max (an unshifted exp overflows fp32)."""
    import flashattn_cuda as fa

    q, k, v = _inputs(300, seed=3, scale=6.0)
    outs = [getattr(fa, fn)(q.cuda(), k.cuda(), v.cuda()).cpu().numpy() for fn in FNS]
    ref = oracle.legacy_attention(q.numpy(), k.numpy(), v.numpy())
    for o in outs:
        assert np.isfinite(o).all()
        assert np.abs(o - ref).max() <= 1e-4
    assert np.abs(outs[0] - outs[1]).max() <= 1e-4
    assert np.abs(outs[1] - outs[2]).max() <= 1e-4


@requires_gpu
def test_legacy_inputs_not_modified_and_stream_honoured():
    import flashattn_cuda as fa

    q, k, v = (t.cuda() for t in _inputs(130, seed=9))
    copies = [t.clone() for t in (q, k, v)]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = fa.legacy_fused(q, k, v)
    s.synchronize()
    for a, b in zip((q, k, v), copies):
        assert torch.equal(a, b)
    ref = oracle.legacy_attention(*(t.cpu().numpy() for t in (q, k, v)))
    assert np.abs(out.cpu().numpy() - ref).max() <= TOL


@requires_gpu
def test_legacy_empty_input_returns_empty():
    import flashattn_cuda as fa

    z = torch.zeros(0, 64, device="cuda")
    for fn in FNS:
        out = getattr(fa, fn)(z, z, z)
        assert out.shape == (0, 64)


@requires_gpu
def test_legacy_rejects_bad_inputs():
    """legacy_ops.cu:19-35: check order and message texts."""
    import flashattn_cuda as fa

    q = torch.randn(8, 64, device="cuda")
    with pytest.raises(RuntimeError, match="legacy kernels expect CUDA tensors"):
        fa.legacy_naive(q.cpu(), q.cpu(), q.cpu())
    with pytest.raises(RuntimeError, match="legacy kernels are fp32 only"):
        fa.legacy_tiled(q.half(), q.half(), q.half())
    with pytest.raises(RuntimeError, match="legacy kernels expect contiguous tensors"):
        t = torch.randn(64, 8, device="cuda").t()
        fa.legacy_fused(t, t, t)
    with pytest.raises(RuntimeError, match="legacy kernels are single-head"):
        b = q[None]
        fa.legacy_naive(b, b, b)
    with pytest.raises(RuntimeError, match="legacy kernels expect identical q/k/v shapes"):
        fa.legacy_tiled(q, q[:4].contiguous(), q)
    with pytest.raises(RuntimeError, match="legacy kernels expect head_dim == 64"):
        w = torch.randn(8, 32, device="cuda")
        fa.legacy_fused(w, w, w)
