"""KV-cache append (``append_kv`` / ``fa_kv_append``) and the decode loop it
feeds.

The reference leaves the cache write to its caller (the FlashStack engine
writes token t at row seq_lens[b] before each decode; README.md:9-13). The
checks:

* ``append_kv`` equals the oracle's ``kv_append`` bit for bit (a copy), on
  ragged lengths and the edges it must leave alone (negative, full cache);
* generating token by token (append, then decode over the cache) reproduces
  causal prefill row t (the decode-vs-prefill form of tests:94-110), with and
  without grouped K/V heads;
* one append + decode step captured in a HIP graph and replayed per token
  gives the eager loop's outputs bit for bit, replay after replay, with eager
  work and synchronisations between the replays.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import flashattn_cuda
import oracle

pytestmark = pytest.mark.gpu

SCALE = 0.125
BOUND = 2.44e-4
LIB = os.path.join(os.path.dirname(flashattn_cuda.__file__), "libflashattn_hip.so")


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).half()


def test_append_kv_matches_oracle():
    B, Hkv, L = 6, 3, 40
    kc, vc = _rand((B, Hkv, L, 64), 1), _rand((B, Hkv, L, 64), 2)
    kn, vn = _rand((B, Hkv, 1, 64), 3), _rand((B, Hkv, 1, 64), 4)
    lens = torch.tensor([0, 7, 39, 40, -2, 20], dtype=torch.int32)
    rk, rv, rl = oracle.kv_append(kc.numpy(), vc.numpy(), kn.numpy(), vn.numpy(), lens.numpy())
    kd, vd, ld = kc.cuda(), vc.cuda(), lens.cuda()
    flashattn_cuda.append_kv(kd, vd, kn.cuda(), vn.cuda(), ld)
    torch.cuda.synchronize()
    assert ld.cpu().tolist() == rl.tolist() == [1, 8, 40, 40, -2, 21]
    assert np.array_equal(kd.cpu().numpy(), rk) and np.array_equal(vd.cpu().numpy(), rv)


def test_append_kv_many_heads_and_batches():
    B, Hkv, L = 70, 40, 9  # more (head, K|V, piece) items than threads per block
    kc, vc = _rand((B, Hkv, L, 64), 5), _rand((B, Hkv, L, 64), 6)
    kn, vn = _rand((B, Hkv, 1, 64), 7), _rand((B, Hkv, 1, 64), 8)
    lens = torch.randint(0, L + 1, (B,), generator=torch.Generator().manual_seed(9),
                         dtype=torch.int32)
    rk, rv, rl = oracle.kv_append(kc.numpy(), vc.numpy(), kn.numpy(), vn.numpy(), lens.numpy())
    kd, vd, ld = kc.cuda(), vc.cuda(), lens.cuda()
    flashattn_cuda.append_kv(kd, vd, kn.cuda(), vn.cuda(), ld)
    torch.cuda.synchronize()
    assert np.array_equal(ld.cpu().numpy(), rl)
    assert np.array_equal(kd.cpu().numpy(), rk) and np.array_equal(vd.cpu().numpy(), rv)


def test_append_kv_rejects_bad_shapes():
    kc = torch.zeros(2, 2, 8, 64, dtype=torch.float16, device="cuda")
    k = torch.zeros(2, 2, 1, 64, dtype=torch.float16, device="cuda")
    lens = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="shape \\[B, H_kv, 1, head_dim\\]"):
        flashattn_cuda.append_kv(kc, kc, k[:, :1].contiguous(), k[:, :1].contiguous(), lens)
    with pytest.raises(RuntimeError, match="seq_lens must be int32"):
        flashattn_cuda.append_kv(kc, kc, k, k, lens.long())
    with pytest.raises(RuntimeError, match="seq_lens must be 1-D"):
        flashattn_cuda.append_kv(kc, kc, k, k, lens[:1])
    with pytest.raises(RuntimeError, match="must be fp16"):
        flashattn_cuda.append_kv(kc, kc, k.float(), k, lens)


@pytest.mark.parametrize("batch,heads,kv_heads,prefix,steps", [
    (2, 12, 12, 100, 40),   # plain decode, split-K path
    (24, 14, 14, 300, 20),  # B*H >= CUs: whole-sequence path
    (3, 14, 2, 250, 30),    # grouped queries (crosses 256 rows: split P -> single P)
])
def test_decode_loop_reproduces_causal_prefill(batch, heads, kv_heads, prefix, steps):
    S = prefix + steps
    q = _rand((batch, heads, S, 64), 10).cuda()
    k = _rand((batch, kv_heads, S, 64), 11).cuda()
    v = _rand((batch, kv_heads, S, 64), 12).cuda()
    grouped = kv_heads != heads
    full = (flashattn_cuda._prefill_gqa_fp32 if grouped else flashattn_cuda._prefill_fp32)(
        q, k, v, True, SCALE)
    L = S + 16
    kc = torch.zeros(batch, kv_heads, L, 64, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:, :, :prefix] = k[:, :, :prefix]
    vc[:, :, :prefix] = v[:, :, :prefix]
    lens = torch.full((batch,), prefix, dtype=torch.int32, device="cuda")
    dec = flashattn_cuda._decode_gqa_fp32 if grouped else flashattn_cuda._decode_fp32
    worst = 0.0
    for t in range(prefix, S):
        flashattn_cuda.append_kv(kc, vc, k[:, :, t:t + 1].contiguous(),
                                 v[:, :, t:t + 1].contiguous(), lens)
        o = dec(q[:, :, t:t + 1].contiguous(), kc, vc, lens, SCALE)
        worst = max(worst, (o - full[:, :, t:t + 1]).abs().max().item())
    torch.cuda.synchronize()
    print(f"[decode loop B{batch} H{heads}/{kv_heads} {prefix}+{steps}] "
          f"max |decode - prefill row| = {worst:.3e}", flush=True)
    assert worst <= BOUND
    assert lens.cpu().tolist() == [S] * batch


@pytest.mark.parametrize("kv_heads", [12, 4])
def test_graph_replayed_decode_step_matches_eager_loop(kv_heads):
    """One append + decode step captured once and replayed per token. Every
    replay is checked against the eager loop, with eager launches and
    synchronisations between the replays."""
    B, H, L, prefix, steps = 2, 12, 600, 200, 12
    torch.manual_seed(0)
    qs = _rand((B, H, steps, 64), 20).cuda()
    ks = _rand((B, kv_heads, steps, 64), 21).cuda()
    vs = _rand((B, kv_heads, steps, 64), 22).cuda()
    kc0 = _rand((B, kv_heads, L, 64), 23).cuda()
    vc0 = _rand((B, kv_heads, L, 64), 24).cuda()
    decode = flashattn_cuda.decode if kv_heads == H else flashattn_cuda.decode_gqa

    # Eager reference loop.
    kc, vc = kc0.clone(), vc0.clone()
    lens = torch.full((B,), prefix, dtype=torch.int32, device="cuda")
    eager = []
    for t in range(steps):
        flashattn_cuda.append_kv(kc, vc, ks[:, :, t:t + 1].contiguous(),
                                 vs[:, :, t:t + 1].contiguous(), lens)
        eager.append(decode(qs[:, :, t:t + 1].contiguous(), kc, vc, lens, SCALE).clone())
    torch.cuda.synchronize()

    # Static inputs, one captured step.
    kc, vc = kc0.clone(), vc0.clone()
    lens = torch.full((B,), prefix, dtype=torch.int32, device="cuda")
    q_in = torch.empty(B, H, 1, 64, dtype=torch.float16, device="cuda")
    k_in = torch.empty(B, kv_heads, 1, 64, dtype=torch.float16, device="cuda")
    v_in = torch.empty_like(k_in)
    # Warm-up on a side stream (as torch's graph docs ask) on scratch copies.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kw, vw, lw = kc.clone(), vc.clone(), lens.clone()
        q_in.copy_(qs[:, :, :1]); k_in.copy_(ks[:, :, :1]); v_in.copy_(vs[:, :, :1])
        flashattn_cuda.append_kv(kw, vw, k_in, v_in, lw)
        decode(q_in, kw, vw, lw, SCALE)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        flashattn_cuda.append_kv(kc, vc, k_in, v_in, lens)
        out = decode(q_in, kc, vc, lens, SCALE)
    torch.cuda.synchronize()
    # Capture does not run the step: the caches and lengths are untouched.
    assert lens.cpu().tolist() == [prefix] * B

    for t in range(steps):
        q_in.copy_(qs[:, :, t:t + 1]); k_in.copy_(ks[:, :, t:t + 1]); v_in.copy_(vs[:, :, t:t + 1])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[t]), f"replay {t} differs from the eager step"
        # Unrelated eager work between replays.
        (qs[:, :, :1].float() * 2).sum().item()
    assert lens.cpu().tolist() == [prefix + steps] * B


@pytest.mark.parametrize("kv_heads", [12, 4])
def test_graph_of_several_steps_matches_eager_loop(kv_heads):
    """Four append + decode steps captured in one graph (the decodes share
    one counter slot and run back to back inside it), replayed three times
    with the next four tokens' inputs copied in between: every output equals
    the eager loop's."""
    B, H, L, prefix, per_graph, replays = 2, 12, 600, 200, 4, 3
    steps = per_graph * replays
    qs = _rand((B, H, steps, 64), 40).cuda()
    ks = _rand((B, kv_heads, steps, 64), 41).cuda()
    vs = _rand((B, kv_heads, steps, 64), 42).cuda()
    kc0 = _rand((B, kv_heads, L, 64), 43).cuda()
    vc0 = _rand((B, kv_heads, L, 64), 44).cuda()
    decode = flashattn_cuda.decode if kv_heads == H else flashattn_cuda.decode_gqa

    kc, vc = kc0.clone(), vc0.clone()
    lens = torch.full((B,), prefix, dtype=torch.int32, device="cuda")
    eager = []
    for t in range(steps):
        flashattn_cuda.append_kv(kc, vc, ks[:, :, t:t + 1].contiguous(),
                                 vs[:, :, t:t + 1].contiguous(), lens)
        eager.append(decode(qs[:, :, t:t + 1].contiguous(), kc, vc, lens, SCALE).clone())
    torch.cuda.synchronize()

    kc, vc = kc0.clone(), vc0.clone()
    lens = torch.full((B,), prefix, dtype=torch.int32, device="cuda")
    q_in = [torch.empty(B, H, 1, 64, dtype=torch.float16, device="cuda") for _ in range(per_graph)]
    k_in = [torch.empty(B, kv_heads, 1, 64, dtype=torch.float16, device="cuda")
            for _ in range(per_graph)]
    v_in = [torch.empty_like(k) for k in k_in]

    def load_inputs(r):
        for j in range(per_graph):
            t = r * per_graph + j
            q_in[j].copy_(qs[:, :, t:t + 1]); k_in[j].copy_(ks[:, :, t:t + 1])
            v_in[j].copy_(vs[:, :, t:t + 1])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kw, vw, lw = kc.clone(), vc.clone(), lens.clone()
        load_inputs(0)
        for j in range(per_graph):
            flashattn_cuda.append_kv(kw, vw, k_in[j], v_in[j], lw)
            decode(q_in[j], kw, vw, lw, SCALE)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    outs = []
    with torch.cuda.graph(graph):
        for j in range(per_graph):
            flashattn_cuda.append_kv(kc, vc, k_in[j], v_in[j], lens)
            outs.append(decode(q_in[j], kc, vc, lens, SCALE))
    torch.cuda.synchronize()
    assert lens.cpu().tolist() == [prefix] * B

    for r in range(replays):
        load_inputs(r)
        graph.replay()
        torch.cuda.synchronize()
        for j in range(per_graph):
            assert torch.equal(outs[j], eager[r * per_graph + j]), \
                f"replay {r}, step {j} differs from the eager step"
    assert lens.cpu().tolist() == [prefix + steps] * B


def test_capi_kv_append_matches_python_api():
    lib = ctypes.CDLL(LIB)
    lib.fa_last_error.restype = ctypes.c_char_p
    B, Hkv, L = 3, 2, 50
    kc, vc = _rand((B, Hkv, L, 64), 30).cuda(), _rand((B, Hkv, L, 64), 31).cuda()
    kn, vn = _rand((B, Hkv, 1, 64), 32).cuda(), _rand((B, Hkv, 1, 64), 33).cuda()
    lens = torch.tensor([5, 0, 49], dtype=torch.int32, device="cuda")
    k2, v2, l2 = kc.clone(), vc.clone(), lens.clone()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    rc = lib.fa_kv_append(p(k2), p(v2), p(kn), p(vn), p(l2), B, Hkv, L, stream)
    assert rc == 0, lib.fa_last_error()
    flashattn_cuda.append_kv(kc, vc, kn, vn, lens)
    torch.cuda.synchronize()
    assert torch.equal(k2, kc) and torch.equal(v2, vc) and torch.equal(l2, lens)
    assert lens.cpu().tolist() == [6, 1, 50]
