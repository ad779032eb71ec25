"""head_dim 128: prefill, grouped prefill, decode (split-K and whole-sequence
paths), grouped decode and the KV-cache append, against the CPU oracle.

head_dim 128 is the reference's named next step (README.md:230, :397 of
shrvan30/flash-attention-cuda: "Head dimension 128"); it has no reference
kernel, so the oracle (pinned at head_dim 128 in tests/test_oracle.py) is the
only parity anchor. The contract is the head_dim-64 one: the fp32-output
hooks within 2.44e-4 of the fp32 oracle, the fp16 outputs within 2.44e-4 plus
half an fp16 ulp of it and equal to the round-to-nearest of the fp32 result.
"""

import numpy as np
import pytest
import torch

import flashattn_cuda
import oracle
from oracle import attention as orc

pytestmark = pytest.mark.gpu

BOUND = 2.44e-4
SCALE = 0.125
D = 128


def _check(out16, out32, ref, label):
    ref = np.asarray(ref, dtype=np.float64)
    o32 = out32.float().cpu().numpy().astype(np.float64)
    o16 = out16.float().cpu().numpy().astype(np.float64)
    err32 = float(np.abs(o32 - ref).max())
    slack = float((np.abs(o16 - ref) - orc.fp16_half_ulp(ref)).max())
    print(f"[{label}] fp32-out err {err32:.3e} | excess over half-ulp {slack:.3e}", flush=True)
    assert err32 <= BOUND, f"{label}: fp32-output error {err32}"
    assert slack <= BOUND, f"{label}: fp16-output error beyond rounding {slack}"
    assert torch.equal(out16.cpu(), out32.half().cpu()), f"{label}: fp16 != rn(fp32)"


def test_head_dims_attribute():
    assert flashattn_cuda.head_dim == 64
    assert tuple(flashattn_cuda.head_dims) == (64, 128)


PREFILL = [
    # (batch, heads, seq): short rows (plain split-P steps), ragged tails,
    # one and several query tiles, the pipelined main loop.
    (1, 2, 1), (1, 2, 37), (2, 3, 128), (1, 2, 130), (1, 3, 300), (2, 2, 513),
    (1, 2, 1000), (1, 4, 2048),
]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("batch,heads,seq", PREFILL)
def test_prefill_matches_oracle(batch, heads, seq, causal):
    label = f"prefill d128 B{batch} H{heads} S{seq} causal={causal}"
    print(label, flush=True)
    q, k, v = oracle.make_prefill_inputs(batch, heads, seq, seed=seq, head_dim=D)
    ref = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), causal, SCALE)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out16 = flashattn_cuda.prefill(qd, kd, vd, causal, SCALE)
    out32 = flashattn_cuda._prefill_fp32(qd, kd, vd, causal, SCALE)
    torch.cuda.synchronize()
    assert out16.shape == q.shape
    _check(out16, out32, ref, label)


def test_prefill_long_causal_against_fp32_torch():
    """S = 4096 (the config-3 length) at head_dim 128, against torch's fp32
    attention on the same inputs (on the GPU, fp32, explicit softmax)."""
    q, k, v = oracle.make_prefill_inputs(1, 2, 4096, seed=3, head_dim=D)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out32 = flashattn_cuda._prefill_fp32(qd, kd, vd, True, SCALE)
    qf, kf, vf = qd.float(), kd.float(), vd.float()
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * SCALE
    mask = torch.ones(4096, 4096, dtype=torch.bool, device="cuda").triu(1)
    s.masked_fill_(mask, float("-inf"))
    ref = torch.matmul(torch.softmax(s, dim=-1), vf)
    err = (out32 - ref).abs().max().item()
    print(f"prefill d128 S4096 causal fp32 err {err:.3e}", flush=True)
    assert err <= BOUND


@pytest.mark.parametrize("heads,kv_heads,causal", [(4, 1, True), (6, 2, False), (14, 2, True)])
def test_prefill_gqa_matches_oracle(heads, kv_heads, causal):
    g = torch.Generator().manual_seed(heads)
    q = torch.randn(1, heads, 600, D, generator=g).half()
    k = torch.randn(1, kv_heads, 600, D, generator=g).half()
    v = torch.randn(1, kv_heads, 600, D, generator=g).half()
    ref = oracle.prefill_gqa(q.numpy(), k.numpy(), v.numpy(), causal, SCALE)
    out16 = flashattn_cuda.prefill_gqa(q.cuda(), k.cuda(), v.cuda(), causal, SCALE)
    out32 = flashattn_cuda._prefill_gqa_fp32(q.cuda(), k.cuda(), v.cuda(), causal, SCALE)
    _check(out16, out32, ref, f"prefill_gqa d128 H{heads} Hkv{kv_heads} causal={causal}")


DECODE = [
    # (batch, heads, max_seq): split-K path (B*H below the CU count, long
    # caches) and whole-sequence path (short caches, or B*H >= CUs).
    (1, 12, 4096), (2, 8, 3000), (3, 4, 300), (32, 14, 2048),
]


@pytest.mark.parametrize("batch,heads,max_seq", DECODE)
def test_decode_matches_oracle(batch, heads, max_seq):
    label = f"decode d128 B{batch} H{heads} L{max_seq}"
    print(label, flush=True)
    q, k, v, lens = oracle.make_decode_inputs(batch, heads, max_seq, seed=max_seq, head_dim=D)
    ref = oracle.decode(q.numpy(), k.numpy(), v.numpy(), lens.numpy(), SCALE)
    args = (q.cuda(), k.cuda(), v.cuda(), lens.cuda())
    out16 = flashattn_cuda.decode(*args, SCALE)
    out32 = flashattn_cuda._decode_fp32(*args, SCALE)
    _check(out16, out32, ref, label)


def test_decode_split_invariance_and_edges():
    q, k, v, _ = oracle.make_decode_inputs(3, 4, 1000, seed=7, head_dim=D)
    lens = torch.tensor([1000, 0, 1500], dtype=torch.int32)  # full, empty, clamped
    args = (q.cuda(), k.cuda(), v.cuda(), lens.cuda())
    ref = oracle.decode(q.numpy(), k.numpy(), v.numpy(), lens.numpy(), SCALE)
    outs = [flashattn_cuda._decode_fp32(*args, SCALE, split).cpu().numpy()
            for split in (0, 128, 256, 1024)]
    for o in outs:
        assert np.abs(o - ref).max() <= BOUND
        assert np.abs(o - outs[0]).max() <= 1e-5
    assert np.all(outs[0][1] == 0.0)


def test_decode_equals_causal_prefill_rows():
    q, k, v = oracle.make_prefill_inputs(1, 4, 777, seed=11, head_dim=D)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    pre = flashattn_cuda._prefill_fp32(qd, kd, vd, True, SCALE)
    for t in (0, 300, 776):
        lens = torch.tensor([t + 1], dtype=torch.int32, device="cuda")
        dec = flashattn_cuda._decode_fp32(qd[:, :, t:t + 1].contiguous(), kd, vd, lens, SCALE)
        assert (dec[:, :, 0] - pre[:, :, t]).abs().max().item() <= 1e-4


@pytest.mark.parametrize("batch,heads,kv_heads,max_seq", [(2, 8, 2, 1500), (40, 14, 2, 600)])
def test_decode_gqa_matches_oracle(batch, heads, kv_heads, max_seq):
    g = torch.Generator().manual_seed(batch)
    lens = torch.randint(1, max_seq + 1, (batch,), generator=g).int()
    q = torch.randn(batch, heads, 1, D, generator=g).half()
    kc = torch.randn(batch, kv_heads, max_seq, D, generator=g).half()
    vc = torch.randn(batch, kv_heads, max_seq, D, generator=g).half()
    ref = oracle.decode_gqa(q.numpy(), kc.numpy(), vc.numpy(), lens.numpy(), SCALE)
    args = (q.cuda(), kc.cuda(), vc.cuda(), lens.cuda())
    out16 = flashattn_cuda.decode_gqa(*args, SCALE)
    out32 = flashattn_cuda._decode_gqa_fp32(*args, SCALE)
    _check(out16, out32, ref, f"decode_gqa d128 B{batch} H{heads} Hkv{kv_heads} L{max_seq}")


def test_append_kv_then_decode():
    batch, kv_heads, lmax = 3, 2, 64
    g = torch.Generator().manual_seed(21)
    kc = torch.randn(batch, kv_heads, lmax, D, generator=g).half()
    vc = torch.randn(batch, kv_heads, lmax, D, generator=g).half()
    kn = torch.randn(batch, kv_heads, 1, D, generator=g).half()
    vn = torch.randn(batch, kv_heads, 1, D, generator=g).half()
    lens = torch.tensor([5, 63, 64], dtype=torch.int32)
    want_k, want_v, want_l = oracle.kv_append(kc.numpy(), vc.numpy(), kn.numpy(), vn.numpy(),
                                              lens.numpy())
    kd, vd, ld = kc.cuda(), vc.cuda(), lens.cuda()
    flashattn_cuda.append_kv(kd, vd, kn.cuda(), vn.cuda(), ld)
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), want_k)
    assert np.array_equal(vd.cpu().numpy(), want_v)
    assert np.array_equal(ld.cpu().numpy(), want_l)


def test_head_dim_mismatches_are_rejected():
    a = torch.randn(1, 2, 8, D, device="cuda").half()
    b = torch.randn(1, 2, 8, 64, device="cuda").half()
    with pytest.raises(RuntimeError, match="identical shapes"):
        flashattn_cuda.prefill(a, b, b, True, SCALE)
    with pytest.raises(RuntimeError, match="head_dim"):
        flashattn_cuda.prefill_gqa(a, b, b, True, SCALE)
    lens = torch.tensor([4], dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="head_dim"):
        flashattn_cuda.decode(a[:, :, :1].contiguous(), b, b, lens, SCALE)
    bad = torch.randn(1, 2, 8, 96, device="cuda").half()
    with pytest.raises(RuntimeError, match="head_dim"):
        flashattn_cuda.prefill(bad, bad, bad, True, SCALE)


# ---------------------------------------------------------------------------
# The head-size entry points of the C ABI, called directly (ctypes)
# ---------------------------------------------------------------------------


def _capi():
    import ctypes
    import os

    lib = ctypes.CDLL(os.path.join(os.path.dirname(flashattn_cuda.__file__),
                                   "libflashattn_hip.so"))
    lib.fa_last_error.restype = ctypes.c_char_p
    lib.fa_decode_hd_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_prefill_workspace_bytes.restype = ctypes.c_size_t
    return lib


def test_capi_prefill_hd_and_decode_hd_match_python_api():
    import ctypes

    lib = _capi()
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator().manual_seed(31)
    q = torch.randn(2, 6, 300, D, generator=g).half().cuda()
    k = torch.randn(2, 3, 300, D, generator=g).half().cuda()
    v = torch.randn(2, 3, 300, D, generator=g).half().cuda()
    o = torch.empty_like(q)
    # With the workspace the Python API allocates, the C ABI takes the same
    # work split and gives the same bits.
    ws_bytes = lib.fa_prefill_workspace_bytes(2, 6, 300, 1)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    rc = lib.fa_prefill_hd(ptr(q), ptr(k), ptr(v), ptr(o), 0, 2, 6, 3, 300, D, 1,
                           ctypes.c_float(SCALE), ptr(ws), ctypes.c_size_t(ws_bytes), stream)
    assert rc == 0, lib.fa_last_error()
    torch.cuda.synchronize()
    assert torch.equal(o, flashattn_cuda.prefill_gqa(q, k, v, True, SCALE))

    qd = torch.randn(2, 6, 1, D, generator=g).half().cuda()
    lens = torch.tensor([300, 17], dtype=torch.int32, device="cuda")
    for kv_heads, kc, vc in ((3, k, v), (6, q, q)):
        od = torch.empty_like(qd)
        ws_bytes = lib.fa_decode_hd_workspace_bytes(2, 6, kv_heads, 300, D, 0)
        if kv_heads == 6:
            # A 300-row cache takes the whole-sequence kernel: no workspace.
            assert ws_bytes == 0 and lib.fa_last_error() == b""
            ws_ptr = None
        else:
            assert ws_bytes > 0, lib.fa_last_error()
            ws = torch.empty(ws_bytes // 4 + 4, dtype=torch.float32, device="cuda")
            ws_ptr = ptr(ws)
        rc = lib.fa_decode_hd(ptr(qd), ptr(kc), ptr(vc), ptr(lens), ptr(od), 0, 2, 6, kv_heads,
                              300, D, ctypes.c_float(SCALE), 0, ws_ptr,
                              ctypes.c_size_t(ws_bytes), stream)
        assert rc == 0, lib.fa_last_error()
        torch.cuda.synchronize()
        want = (flashattn_cuda.decode_gqa(qd, kc, vc, lens, SCALE) if kv_heads != 6 else
                flashattn_cuda.decode(qd, kc, vc, lens, SCALE))
        assert torch.equal(od, want)
