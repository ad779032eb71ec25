"""fa_decode_hd_noalloc: the decode entry point that takes no workspace.

It has no counterpart in the reference (it serves callers that cannot
allocate device memory). Its split-K partials live in a scratch array the
library holds per device, so the checks are: the result is bit-identical to
fa_decode_hd with a caller-provided workspace (same kernels, same chunking),
on two calls in a row where the second is smaller and finds the first call's
partials still in the scratch; and a shape whose partials exceed the scratch
is refused before anything is launched.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "flash-attention-cuda_amd", "flashattn_cuda", "libflashattn_hip.so")
FA_OK, FA_ERR_WORKSPACE = 0, 2
FA_OUT_F16, FA_OUT_F32 = 0, 1
SCRATCH_BYTES = 8 << 20


@pytest.fixture(scope="module")
def lib():
    dll = ctypes.CDLL(LIB)
    dll.fa_last_error.restype = ctypes.c_char_p
    dll.fa_decode_hd_workspace_bytes.restype = ctypes.c_size_t
    return dll


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _inputs(batch, heads, kv_heads, max_seq, head_dim, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, heads, 1, head_dim, generator=g).half().cuda()
    k = torch.randn(batch, kv_heads, max_seq, head_dim, generator=g).half().cuda()
    v = torch.randn(batch, kv_heads, max_seq, head_dim, generator=g).half().cuda()
    lens = torch.randint(1, max_seq + 1, (batch,), generator=g, dtype=torch.int32)
    lens[0] = max_seq
    return q, k, v, lens.cuda()


def _run(lib, noalloc, q, k, v, lens, out_dtype, kv_heads, scale, split):
    batch, heads, _, head_dim = q.shape
    max_seq = k.shape[2]
    o = torch.empty(q.shape, dtype=torch.float32 if out_dtype == FA_OUT_F32 else torch.float16,
                    device=q.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(lens), _ptr(o), out_dtype, batch, heads, kv_heads,
            max_seq, head_dim, ctypes.c_float(scale), split)
    if noalloc:
        rc = lib.fa_decode_hd_noalloc(*args, stream)
    else:
        need = lib.fa_decode_hd_workspace_bytes(batch, heads, kv_heads, max_seq, head_dim, split)
        assert need > 0, lib.fa_last_error()
        ws = torch.empty(need // 4 + 4, dtype=torch.float32, device=q.device)
        rc = lib.fa_decode_hd(*args, _ptr(ws), ctypes.c_size_t(need), stream)
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    return o


# (batch, heads, kv_heads, max_seq, head_dim, split): both take the split-K
# path (fewer (b, h) pairs than compute units, caches longer than 512 rows);
# the second is smaller and, grouped, uses the matrix-core split pass.
CALLS = [(2, 12, 12, 6000, 128, 0), (1, 8, 2, 1700, 64, 0)]


@pytest.mark.parametrize("out_dtype", [FA_OUT_F16, FA_OUT_F32])
def test_noalloc_decode_equals_workspace_decode_on_two_calls(lib, out_dtype):
    for i, (b, h, hkv, lmax, d, split) in enumerate(CALLS):
        q, k, v, lens = _inputs(b, h, hkv, lmax, d, seed=70 + i)
        scale = d ** -0.5
        assert lib.fa_decode_hd_workspace_bytes(b, h, hkv, lmax, d, split) <= SCRATCH_BYTES
        got = _run(lib, True, q, k, v, lens, out_dtype, hkv, scale, split)
        want = _run(lib, False, q, k, v, lens, out_dtype, hkv, scale, split)
        assert torch.equal(got, want), f"call {i}: max diff {(got.float() - want.float()).abs().max()}"
        # And both are the attention itself (the float64 oracle, 2.44e-4).
        kk = k.cpu().repeat_interleave(h // hkv, dim=1).numpy()
        vv = v.cpu().repeat_interleave(h // hkv, dim=1).numpy()
        ref = oracle.decode(q.cpu().numpy(), kk, vv, lens.cpu().numpy(), scale)
        err = np.abs(got.float().cpu().numpy() - ref).max()
        half_ulp = 0.5 * np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
        bound = 2.44e-4 + (half_ulp.max() if out_dtype == FA_OUT_F16 else 0.0)
        assert err <= bound, f"call {i}: error {err} vs oracle"


def test_noalloc_decode_refuses_shapes_beyond_its_scratch(lib):
    b, h, lmax, d = 1, 200, 1 << 20, 64
    need = lib.fa_decode_hd_workspace_bytes(b, h, h, lmax, d, 0)
    assert need > SCRATCH_BYTES
    q = torch.zeros(b, h, 1, d, dtype=torch.float16, device="cuda")
    kv = torch.zeros(16, dtype=torch.float16, device="cuda")  # never read: refused first
    lens = torch.ones(b, dtype=torch.int32, device="cuda")
    o = torch.empty_like(q)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.fa_decode_hd_noalloc(_ptr(q), _ptr(kv), _ptr(kv), _ptr(lens), _ptr(o), FA_OUT_F16,
                                  b, h, h, lmax, d, ctypes.c_float(0.125), 0, stream)
    assert rc == FA_ERR_WORKSPACE
    assert b"noalloc" in lib.fa_last_error()


_CAPTURE_FIRST_CALL = r"""
import ctypes, sys, torch
lib = ctypes.CDLL(sys.argv[1])
lib.fa_last_error.restype = ctypes.c_char_p
g = torch.Generator().manual_seed(91)
b, h, hkv, lmax, d = 1, 8, 2, 1700, 64
q = torch.randn(b, h, 1, d, generator=g).half().cuda()
k = torch.randn(b, hkv, lmax, d, generator=g).half().cuda()
v = torch.randn(b, hkv, lmax, d, generator=g).half().cuda()
lens = torch.tensor([lmax], dtype=torch.int32).cuda()
o = torch.empty(b, h, 1, d, dtype=torch.float32, device="cuda")
ref = torch.empty_like(o)
P = lambda t: ctypes.c_void_p(t.data_ptr())
def call(out):
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.fa_decode_hd_noalloc(P(q), P(k), P(v), P(lens), P(out), 1, b, h, hkv, lmax, d,
                                    ctypes.c_float(d ** -0.5), 0, s)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = call(o)  # the process's first call into the library
assert rc == 0, lib.fa_last_error()
torch.cuda.synchronize()
for r in range(4):
    o.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert call(ref) == 0, lib.fa_last_error()  # eager work between replays
    torch.cuda.synchronize()
    assert torch.equal(o, ref), f"replay {r}"
print("ok")
"""


def test_noalloc_first_call_inside_graph_capture():
    """A fresh process whose first library call is fa_decode_hd_noalloc
    inside torch.cuda.graph (the scratch array and the counter slot are
    looked up during the capture): every replay equals the eager call."""
    import subprocess
    import sys

    res = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST_CALL, LIB], capture_output=True,
                         text=True, timeout=300)
    print(res.stdout, res.stderr[-2000:])
    assert res.returncode == 0 and "ok" in res.stdout
