"""Pin the CPU oracle (oracle/attention.py) before it is trusted as a checker.

Every oracle function is checked against something that does not share its
code: the committed fp64 brute-force fixtures, an fp64 loop written here,
torch's CPU scaled_dot_product_attention, closed forms and invariants. The
last group plants plausible mistakes in copies of the oracle and requires the
same checks to reject them, so the checks are known to have teeth.
"""

import glob
import math
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import attention as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D = 64
SCALE = 0.125


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).half()


def _fixtures():
    return sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---------------------------------------------------------------------------
# Checks (reused by the planted-mistake tests below)
# ---------------------------------------------------------------------------


def check_prefill_fn(prefill_fn, tol=2e-6):
    """Raise AssertionError if `prefill_fn` disagrees with the pins."""
    for path in _fixtures():
        c = _load(path)
        if str(c["kind"]) != "prefill":
            continue
        got = prefill_fn(c["q"], c["k"], c["v"], bool(c["causal"]), float(c["scale"]))
        err = np.abs(got.astype(np.float64) - c["out"]).max()
        assert err <= tol, f"{os.path.basename(path)}: {err}"
    # torch CPU SDPA, fp32, causal and full.
    q, k, v = (_rand((2, 3, 75, D), s) for s in (1, 2, 3))
    for causal in (True, False):
        ref = torch.nn.functional.scaled_dot_product_attention(
            q.float(), k.float(), v.float(), is_causal=causal, scale=SCALE
        ).numpy()
        got = prefill_fn(q.numpy(), k.numpy(), v.numpy(), causal, SCALE)
        assert np.abs(got - ref).max() <= 1e-5


def check_decode_fn(decode_fn, tol=2e-6):
    for path in _fixtures():
        c = _load(path)
        if str(c["kind"]) != "decode":
            continue
        got = decode_fn(c["q"], c["k"], c["v"], c["lens"], float(c["scale"]))
        err = np.abs(got.astype(np.float64) - c["out"]).max()
        assert err <= tol, f"{os.path.basename(path)}: {err}"


# ---------------------------------------------------------------------------
# The oracle against the pins
# ---------------------------------------------------------------------------


def test_golden_fixtures_present():
    names = {os.path.basename(p) for p in _fixtures()}
    assert "prefill_causal_s130.npz" in names and "decode_edges.npz" in names
    assert len(names) == 9


def test_prefill_matches_pins():
    check_prefill_fn(oracle.prefill)


def test_decode_matches_pins():
    check_decode_fn(oracle.decode)


def test_attention_cpu_matches_fp64_loop():
    """attention_cpu (fp32, vectorised) vs an fp64 loop written here."""
    rng = np.random.default_rng(5)
    Q = rng.standard_normal((6, D)).astype(np.float32)
    K = rng.standard_normal((9, D)).astype(np.float32)
    V = rng.standard_normal((9, D)).astype(np.float32)
    for causal in (False, True):
        got = oracle.attention_cpu(Q, K, V, SCALE, causal)
        for i in range(6):
            n = i + 1 + 3 if causal else 9  # bottom-right aligned: M - N = 3
            s = [sum(float(Q[i, d]) * float(K[j, d]) for d in range(D)) * SCALE for j in range(n)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            want = [sum(w[j] * float(V[j, d]) for j in range(n)) / sum(w) for d in range(D)]
            assert np.abs(got[i] - np.array(want)).max() < 2e-6


def test_default_scale_is_inverse_sqrt_d():
    """attention_cpu.py:37-38: scale defaults to 1/sqrt(d)."""
    rng = np.random.default_rng(6)
    Q, K, V = (rng.standard_normal((5, D)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(oracle.attention_cpu(Q, K, V), oracle.attention_cpu(Q, K, V, 0.125), rtol=0, atol=0)


def _legacy_fp64_loop(Q, K, V):
    """softmax(Q K^T / 8) V by explicit fp64 loops (the v1 kernels' function)."""
    out = np.empty(Q.shape, dtype=np.float64)
    for i in range(Q.shape[0]):
        s = [sum(float(Q[i, d]) * float(K[j, d]) for d in range(D)) / 8.0 for j in range(K.shape[0])]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        for d in range(D):
            out[i, d] = sum(w[j] * float(V[j, d]) for j in range(K.shape[0])) / sum(w)
    return out


def test_legacy_attention_matches_fp64_loop():
    """legacy_attention: (N, 64) fp32, scale 1/sqrt(64), no mask
    (src/legacy/*_attention.cu; launchers at naive :139, tiled :240, fused :213)."""
    rng = np.random.default_rng(11)
    Q, K, V = (rng.standard_normal((7, D)).astype(np.float32) for _ in range(3))
    got = oracle.legacy_attention(Q, K, V)
    assert got.dtype == np.float32 and got.shape == (7, D)
    assert np.abs(got - _legacy_fp64_loop(Q, K, V)).max() < 2e-6
    # One row: the output is that value row exactly; equal keys: the mean of V.
    np.testing.assert_array_equal(oracle.legacy_attention(Q[:1], K[:1], V[:1]), V[:1])
    same = np.repeat(K[:1], 5, axis=0)
    np.testing.assert_allclose(oracle.legacy_attention(Q[:2], same, V[:5]),
                               np.repeat(V[:5].mean(0, keepdims=True), 2, 0), atol=1e-6)


@pytest.mark.parametrize("kind", ["scale_1_over_64", "causal", "no_max_shift_overflow"])
def test_planted_legacy_mistakes_are_caught(kind):
    rng = np.random.default_rng(12)
    Q, K, V = (rng.standard_normal((6, D)).astype(np.float32) for _ in range(3))
    if kind == "no_max_shift_overflow":
        Q = Q * 40.0  # scores ~ 300: exp without the max shift overflows
    want = _legacy_fp64_loop(Q, K, V)
    if kind == "scale_1_over_64":
        bad = oracle.attention_cpu(Q, K, V, 1.0 / 64)
    elif kind == "causal":
        bad = oracle.attention_cpu(Q, K, V, None, True)
    else:
        with np.errstate(over="ignore", invalid="ignore"):
            e = np.exp((Q @ K.T) / 8.0)
            bad = (e / e.sum(1, keepdims=True)) @ V
    assert not (np.abs(bad - want).max() < 1e-4)
    assert np.abs(oracle.legacy_attention(Q, K, V) - want).max() < 1e-4


@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_128_prefill_and_decode_match_pins(causal):
    """The oracle at head_dim 128: torch CPU SDPA in fp32 for prefill, an fp64
    loop for one decode row, and decode(t) == causal prefill row t."""
    q, k, v = oracle.make_prefill_inputs(1, 2, 70, seed=4, head_dim=128)
    assert q.shape == (1, 2, 70, 128)
    got = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), causal, SCALE)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.float(), k.float(), v.float(), is_causal=causal, scale=SCALE).numpy()
    assert np.abs(got - ref).max() <= 1e-5
    qd, kd, vd, lens = oracle.make_decode_inputs(2, 1, 9, seed=5, lens=[9, 4], head_dim=128)
    out = oracle.decode(qd.numpy(), kd.numpy(), vd.numpy(), lens.numpy(), SCALE)
    Q, K, V = (t.numpy().astype(np.float64) for t in (qd, kd, vd))
    s = [float(Q[1, 0, 0] @ K[1, 0, j]) * SCALE for j in range(4)]
    w = np.exp(np.array(s) - max(s))
    want = (w[:, None] * V[1, 0, :4]).sum(0) / w.sum()
    assert np.abs(out[1, 0, 0] - want).max() < 2e-6
    if causal:
        dec = oracle.decode(q.numpy()[:, :, 69:70], k.numpy(), v.numpy(),
                            np.array([70]), SCALE)
        assert np.abs(dec[:, :, 0] - got[:, :, 69]).max() < 1e-6


def test_stable_softmax_rows_and_shift_invariance():
    x = np.array([[1.0, 2.0, 3.0], [1000.0, 1001.0, -np.inf]], dtype=np.float32)
    p = oracle.stable_softmax(x)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(p[0], oracle.stable_softmax(x[:1] + 50.0)[0], rtol=1e-6)
    assert p[1, 2] == 0.0
    e = np.exp([-2.0, -1.0, 0.0])
    np.testing.assert_allclose(p[0], e / e.sum(), rtol=1e-6)


@pytest.mark.parametrize("causal", [True, False])
def test_constant_value_rows_give_that_row(causal):
    q, k, _ = (_rand((1, 2, 40, D), s) for s in (7, 8, 9))
    row = _rand((D,), 10)
    v = row.expand(1, 2, 40, D).contiguous()
    out = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), causal, SCALE)
    np.testing.assert_allclose(out, np.broadcast_to(row.float().numpy(), out.shape), atol=2e-6)


def test_scale_zero_gives_visible_mean():
    q, k, v = (_rand((1, 1, 33, D), s) for s in (11, 12, 13))
    out = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), True, 0.0)
    vf = v.float().numpy()[0, 0]
    want = np.cumsum(vf, axis=0) / np.arange(1, 34)[:, None]
    np.testing.assert_allclose(out[0, 0], want, atol=2e-6)
    full = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), False, 0.0)
    np.testing.assert_allclose(full[0, 0], np.broadcast_to(vf.mean(0), (33, D)), atol=2e-6)


def test_causal_row0_is_v_row0():
    q, k, v = (_rand((2, 2, 17, D), s) for s in (14, 15, 16))
    out = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), True, SCALE)
    np.testing.assert_array_equal(out[:, :, 0], v.float().numpy()[:, :, 0])


def test_full_attention_is_key_permutation_invariant():
    q, k, v = (_rand((1, 2, 50, D), s) for s in (17, 18, 19))
    perm = torch.randperm(50, generator=torch.Generator().manual_seed(3))
    a = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), False, SCALE)
    b = oracle.prefill(q.numpy(), k[:, :, perm].numpy(), v[:, :, perm].numpy(), False, SCALE)
    np.testing.assert_allclose(a, b, atol=2e-6)


def test_decode_equals_causal_prefill_row():
    """tests/test_correctness.py:94-110, on the oracle."""
    q, k, v = (_rand((2, 3, 90, D), s) for s in (20, 21, 22))
    full = oracle.prefill(q.numpy(), k.numpy(), v.numpy(), True, SCALE)
    for t in (0, 1, 17, 63, 64, 89):
        lens = np.full((2,), t + 1, dtype=np.int32)
        out = oracle.decode(q[:, :, t : t + 1].numpy(), k.numpy(), v.numpy(), lens, SCALE)
        np.testing.assert_allclose(out[:, :, 0], full[:, :, t], atol=2e-6)


def test_decode_clamps_and_zeroes():
    """decode.cu:69 (len > Lmax clamps) and :155-172 (len <= 0 gives 0)."""
    q = _rand((3, 2, 1, D), 23).numpy()
    k, v = (_rand((3, 2, 12, D), s).numpy() for s in (24, 25))
    out = oracle.decode(q, k, v, np.array([0, 50, -4], dtype=np.int32), SCALE)
    ref = oracle.decode(q, k, v, np.array([0, 12, 0], dtype=np.int32), SCALE)
    np.testing.assert_array_equal(out, ref)
    assert not out[0].any() and not out[2].any()


def test_decode_matches_torch_loop():
    """The reference's own decode oracle form (tests/test_correctness.py:37-44)."""
    q = _rand((3, 4, 1, D), 26)
    k, v = (_rand((3, 4, 200, D), s) for s in (27, 28))
    lens = torch.tensor([200, 1, 77], dtype=torch.int32)
    want = torch.empty(3, 4, 1, D)
    for b in range(3):
        n = int(lens[b])
        s = (q[b].float() @ k[b, :, :n].float().transpose(-1, -2).contiguous()) * SCALE
        want[b] = torch.softmax(s, dim=-1) @ v[b, :, :n].float()
    got = oracle.decode(q.numpy(), k.numpy(), v.numpy(), lens.numpy(), SCALE)
    np.testing.assert_allclose(got, want.numpy(), atol=2e-6)


# ---------------------------------------------------------------------------
# Chooser, FLOP and byte formulas
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("sms", [82, 256, 304])
def test_choose_decode_split_pins(sms):
    """tests/test_correctness.py:180-198, restated so it holds for any CU
    count: either the target is reached and doubling the chunk falls short,
    or the chunk is the 128 fallback."""
    target = 2 * sms
    for batch, heads, seq in [(1, 12, 2048), (8, 12, 2048), (4, 12, 1024), (32, 14, 4096), (1, 12, 4096)]:
        split = oracle.choose_decode_split(seq, batch, heads, target)
        assert split in (128, 256, 512, 1024)
        blocks = batch * heads * -(-seq // split)
        if split > 128:
            assert blocks >= target
        if split < 1024 and blocks >= target:
            assert batch * heads * -(-seq // (split * 2)) < target
        if blocks < target:
            assert split == 128
    assert oracle.choose_decode_split(512, 1, 12, target) == 128


def test_choose_decode_split_reference_asserts_hold_on_3090():
    """On the reference's 82-SM card the original asserts hold verbatim."""
    target = 2 * 82
    for batch, heads, seq in [(1, 12, 2048), (8, 12, 2048), (4, 12, 1024)]:
        split = oracle.choose_decode_split(seq, batch, heads, target)
        assert batch * heads * -(-seq // split) >= target
        if split < 1024:
            assert batch * heads * -(-seq // (split * 2)) < target


def test_choose_decode_split_baseline_configs():
    # MI355X: 256 CUs -> min_blocks 512.
    assert oracle.choose_decode_split(4096, 1, 12, 512) == 128   # C4: 384 blocks, fallback
    assert oracle.choose_decode_split(4096, 32, 14, 512) == 1024  # C5: 1792 blocks
    # analysis.md:113 on the 3090 (164 target): B1 H12 S4096 -> chunk 256.
    assert oracle.choose_decode_split(4096, 1, 12, 164) == 256


def test_flops_and_bytes():
    assert oracle.attention_flops(1, 12, 128, True) == 25_165_824
    assert oracle.attention_flops(1, 14, 4096, True) == 30_064_771_072
    assert oracle.attention_flops(4, 12, 1024, False) == 12_884_901_888
    assert oracle.decode_bytes(12, [4096], 4096) == 12_585_988
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(1, 4097, (32,), generator=g)
    assert int(lens.sum()) == 73_374
    assert oracle.decode_bytes(14, lens.numpy(), 4096) == 263_087_232


def test_fp16_floor_helpers():
    assert orc.fp16_half_ulp(np.array([0.75]))[0] == 2.0 ** -12
    assert orc.fp16_half_ulp(np.array([3.0]))[0] == 2.0 ** -10
    assert orc.fp16_rounding_floor(np.array([1.0, 0.5], dtype=np.float32)) == 0.0


# ---------------------------------------------------------------------------
# Planted mistakes: each mutant must fail the checks above.
# ---------------------------------------------------------------------------


def _mutant_prefill(kind):
    def attn(Q, K, V, scale, causal):
        N, d = Q.shape
        S = (Q @ K.T) * np.float32(scale)
        if kind == "scores_transposed":  # S^T where S was meant
            S = (K @ Q.T) * np.float32(scale)
        if kind == "scale_twice":
            S = S * np.float32(scale)
        if causal:
            i = np.arange(N)[:, None]
            j = np.arange(K.shape[0])[None, :]
            keep = (j < i) | ((i == 0) & (j == 0)) if kind == "mask_edge" else j <= i
            S = np.where(keep, S, np.float32(-np.inf))
        P = orc.stable_softmax(S)
        if kind == "v_rows_reversed":  # wrong key index into V
            return P @ V[::-1]
        if kind == "no_max_shift":
            P = np.exp(S) / np.exp(S).sum(-1, keepdims=True)
            P = P.astype(np.float16).astype(np.float32)
        return P @ V

    def prefill(q, k, v, causal, scale):
        q, k, v = (np.asarray(x, dtype=np.float32) for x in (q, k, v))
        B, H, S, D_ = q.shape
        out = np.empty((B, H, S, D_), dtype=np.float32)
        for b in range(B):
            for h in range(H):
                out[b, h] = attn(q[b, h], k[b, h], v[b, h], scale, causal)
        return out

    return prefill


@pytest.mark.parametrize("kind", ["scale_twice", "mask_edge", "v_rows_reversed", "scores_transposed", "no_max_shift"])
def test_planted_prefill_mistakes_are_caught(kind):
    with pytest.raises(AssertionError):
        check_prefill_fn(_mutant_prefill(kind))


@pytest.mark.parametrize("kind", ["no_clamp", "off_by_one_len"])
def test_planted_decode_mistakes_are_caught(kind):
    def bad_decode(q, k, v, lens, scale):
        lens = np.asarray(lens).astype(np.int64)
        if kind == "off_by_one_len":
            lens = lens - 1
        out = np.zeros((q.shape[0], q.shape[1], 1, D), dtype=np.float32)
        for b in range(q.shape[0]):
            n = int(lens[b]) if kind == "no_clamp" else int(min(lens[b], k.shape[2]))
            if n <= 0:
                continue
            for h in range(q.shape[1]):
                kk = k[b, h, :n].astype(np.float32)
                if kind == "no_clamp" and n > k.shape[2]:
                    kk = np.concatenate([kk, np.zeros((n - kk.shape[0], D), np.float32)])
                vv = v[b, h, : kk.shape[0]].astype(np.float32)
                if vv.shape[0] < kk.shape[0]:
                    vv = np.concatenate([vv, np.zeros((kk.shape[0] - vv.shape[0], D), np.float32)])
                out[b, h] = orc.attention_cpu(q[b, h].astype(np.float32), kk, vv, scale)
        return out

    with pytest.raises(AssertionError):
        check_decode_fn(bad_decode)


# ---------------------------------------------------------------------------
# Grouped-query attention: query head h reads K/V head h // G.
# ---------------------------------------------------------------------------


def _gqa_loop(q, k, v, causal, scale):
    """fp64 brute force written per query head with an explicit K/V index."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    B, H, N, _ = q.shape
    G = H // k.shape[1]
    out = np.zeros(q.shape)
    for b in range(B):
        for h in range(H):
            g = h // G
            for i in range(N):
                n_keys = i + 1 if causal else k.shape[2]
                s = [scale * float(q[b, h, i] @ k[b, g, j]) for j in range(n_keys)]
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                out[b, h, i] = sum(wj * v[b, g, j] for j, wj in enumerate(w)) / sum(w)
    return out


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (6, 1), (6, 3), (3, 3)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_gqa_matches_explicit_head_loop(heads, kv_heads, causal):
    q = _rand((2, heads, 9, 64), 40)
    k = _rand((2, kv_heads, 9, 64), 41)
    v = _rand((2, kv_heads, 9, 64), 42)
    got = oracle.prefill_gqa(q, k, v, causal, 0.125)
    assert np.abs(got - _gqa_loop(q, k, v, causal, 0.125)).max() < 2e-6


def test_gqa_with_one_group_is_plain_attention_and_pairing_is_interleaved():
    q = _rand((1, 6, 7, 64), 43).numpy()
    k = _rand((1, 6, 7, 64), 44).numpy()
    v = _rand((1, 6, 7, 64), 45).numpy()
    assert np.array_equal(oracle.prefill_gqa(q, k, v, True, 0.125), oracle.prefill(q, k, v, True, 0.125))
    # torch's repeat_interleave is the pairing; torch's tile-style repeat
    # (head h reads K/V head h % H_kv) is a planted mistake it must reject.
    k2, v2 = k[:, :2], v[:, :2]
    kt = torch.from_numpy(k2).repeat_interleave(3, dim=1).numpy()
    assert np.array_equal(oracle.repeat_kv(k2, 6), kt)
    tiled = oracle.prefill(q, np.tile(k2, (1, 3, 1, 1)), np.tile(v2, (1, 3, 1, 1)), True, 0.125)
    good = oracle.prefill_gqa(q, k2, v2, True, 0.125)
    assert np.abs(tiled - good).max() > 1e-2
    assert np.abs(good - _gqa_loop(q, k2, v2, True, 0.125)).max() < 2e-6
    with pytest.raises(ValueError):
        oracle.repeat_kv(k[:, :4], 6)


def test_decode_gqa_equals_causal_prefill_gqa_row():
    q = _rand((2, 8, 12, 64), 46)
    k = _rand((2, 2, 12, 64), 47)
    v = _rand((2, 2, 12, 64), 48)
    full = oracle.prefill_gqa(q, k, v, True, 0.125)
    for t in (0, 5, 11):
        lens = np.full(2, t + 1, dtype=np.int32)
        got = oracle.decode_gqa(q[:, :, t : t + 1], k, v, lens, 0.125)
        assert np.abs(got - full[:, :, t : t + 1]).max() < 2e-6
    lens = np.array([0, 30], dtype=np.int32)  # empty, and clamped to the cache
    got = oracle.decode_gqa(q[:, :, 11:12], k, v, lens, 0.125)
    assert not got[0].any()
    assert np.abs(got[1] - full[1, :, 11:12]).max() < 2e-6


# ---------------------------------------------------------------------------
# KV-cache append: the caller step before decode.
# ---------------------------------------------------------------------------


def test_kv_append_writes_row_len_and_advances():
    k = np.zeros((4, 2, 5, 64), np.float16)
    v = np.zeros((4, 2, 5, 64), np.float16)
    kn = _rand((4, 2, 1, 64), 60).numpy()
    vn = _rand((4, 2, 1, 64), 61).numpy()
    lens = np.array([0, 3, 5, -1], np.int32)  # empty, middle, full, negative
    k2, v2, l2 = oracle.kv_append(k, v, kn, vn, lens)
    assert l2.tolist() == [1, 4, 5, -1]
    assert np.array_equal(k2[0, :, 0], kn[0, :, 0]) and np.array_equal(v2[1, :, 3], vn[1, :, 0])
    # Nothing else moved: rows other than the written ones, the full and the
    # negative sequences, and the inputs themselves.
    mask = np.zeros(k.shape, bool)
    mask[0, :, 0] = mask[1, :, 3] = True
    assert not k2[~mask].any() and not v2[~mask].any()
    assert not k.any() and lens.tolist() == [0, 3, 5, -1]


def _incremental_matches_prefill(append_fn, heads, kv_heads):
    S = 9
    q = _rand((2, heads, S, 64), 62).numpy()
    k = _rand((2, kv_heads, S, 64), 63).numpy()
    v = _rand((2, kv_heads, S, 64), 64).numpy()
    full = oracle.prefill_gqa(q, k, v, True, 0.125)
    kc = np.zeros((2, kv_heads, 12, 64), np.float16)
    vc = np.zeros_like(kc)
    lens = np.zeros(2, np.int32)
    for t in range(S):
        kc, vc, lens = append_fn(kc, vc, k[:, :, t : t + 1], v[:, :, t : t + 1], lens)
        out = oracle.decode_gqa(q[:, :, t : t + 1], kc, vc, lens, 0.125)
        assert np.abs(out - full[:, :, t : t + 1]).max() < 2e-6, t


@pytest.mark.parametrize("kind", ["row_after_len", "advance_before_write", "k_into_v"])
def test_planted_kv_append_mistakes_are_caught(kind):
    def bad(kc, vc, kn, vn, lens):
        kc, vc, lens = kc.copy(), vc.copy(), lens.copy()
        for b in range(lens.shape[0]):
            n = int(lens[b])
            row = n + 1 if kind in ("row_after_len", "advance_before_write") else n
            if kind == "advance_before_write":
                row = min(row, kc.shape[2] - 1)
            kc[b, :, row] = kn[b, :, 0]
            vc[b, :, row] = (kn if kind == "k_into_v" else vn)[b, :, 0]
            lens[b] = n + 1
        return kc, vc, lens

    with pytest.raises(AssertionError):
        _incremental_matches_prefill(bad, 6, 2)


@pytest.mark.parametrize("heads,kv_heads", [(3, 3), (6, 2)])
def test_incremental_decode_through_kv_append_equals_causal_prefill(heads, kv_heads):
    """Generating token by token (append, then decode over the cache) gives
    the rows of causal prefill over the whole sequence (tests:94-110 form)."""
    _incremental_matches_prefill(oracle.kv_append, heads, kv_heads)
    S = 9
    q = _rand((2, heads, S, 64), 62).numpy()
    k = _rand((2, kv_heads, S, 64), 63).numpy()
    v = _rand((2, kv_heads, S, 64), 64).numpy()
    full = oracle.prefill_gqa(q, k, v, True, 0.125)
    kc = np.zeros((2, kv_heads, 12, 64), np.float16)
    vc = np.zeros_like(kc)
    lens = np.zeros(2, np.int32)
    for t in range(S):
        kc, vc, lens = oracle.kv_append(kc, vc, k[:, :, t : t + 1], v[:, :, t : t + 1], lens)
        out = oracle.decode_gqa(q[:, :, t : t + 1], kc, vc, lens, 0.125)
        assert np.abs(out - full[:, :, t : t + 1]).max() < 2e-6, t
    assert lens.tolist() == [S, S]
