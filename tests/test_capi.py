"""CPU-side checks of the C ABI (include/flashattn_hip.h, libflashattn_hip.so).

No test here launches a kernel or touches a device: they cover symbol
export, the pure integer entry points and the argument checks that fail
before any HIP call.
"""

import ctypes
import os
import re

import numpy as np
import pytest

import oracle

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(REPO, "include")
LIB = os.path.join(REPO, "flash-attention-cuda_amd", "flashattn_cuda", "libflashattn_hip.so")

FA_OK, FA_ERR_INVALID_ARGUMENT, FA_ERR_WORKSPACE, FA_ERR_HIP = 0, 1, 2, 3


def declared_functions():
    names = []
    for fn in sorted(os.listdir(HEADER_DIR)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(HEADER_DIR, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(fa_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built; run flash-attention-cuda_amd/build.py")
    dll = ctypes.CDLL(LIB)
    dll.fa_last_error.restype = ctypes.c_char_p
    dll.fa_version.restype = ctypes.c_char_p
    dll.fa_decode_workspace_bytes.restype = ctypes.c_size_t
    dll.fa_decode_gqa_workspace_bytes.restype = ctypes.c_size_t
    dll.fa_prefill_workspace_bytes.restype = ctypes.c_size_t
    return dll


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted(
        [
            "fa_choose_decode_split",
            "fa_decode",
            "fa_decode_gqa",
            "fa_decode_gqa_workspace_bytes",
            "fa_decode_hd",
            "fa_decode_hd_noalloc",
            "fa_decode_hd_workspace_bytes",
            "fa_decode_min_blocks",
            "fa_decode_workspace_bytes",
            "fa_head_dim",
            "fa_kv_append",
            "fa_kv_append_hd",
            "fa_last_error",
            "fa_legacy_attention",
            "fa_occupancy_report",
            "fa_prefill",
            "fa_prefill_gqa",
            "fa_prefill_hd",
            "fa_prefill_plan_units",
            "fa_prefill_workspace_bytes",
            "fa_version",
        ]
    )


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing


def test_head_dim_and_version(lib):
    assert lib.fa_head_dim() == 64
    assert lib.fa_version().decode().startswith("2.0.0")


def test_choose_decode_split_matches_oracle(lib):
    for max_seq in (1, 63, 128, 129, 512, 1000, 2048, 4096, 65536):
        for batch, heads in ((1, 1), (1, 12), (2, 12), (8, 12), (32, 14)):
            for target in (164, 512, 608, 4096):
                assert lib.fa_choose_decode_split(max_seq, batch, heads, target) == \
                    oracle.choose_decode_split(max_seq, batch, heads, target)


def test_decode_workspace_bytes_forced_split(lib):
    # [B, H, n_splits, 64] + [B, H, n_splits, 2] fp32 (decode.cu:215-219).
    assert lib.fa_decode_workspace_bytes(32, 14, 4096, 1024) == 32 * 14 * 4 * 66 * 4
    assert lib.fa_decode_workspace_bytes(1, 12, 4096, 128) == 12 * 32 * 66 * 4
    assert lib.fa_decode_workspace_bytes(1, 12, 4096, 6) == 0  # not a multiple of 4
    assert b"multiple of the warp count" in lib.fa_last_error()
    assert lib.fa_decode_workspace_bytes(0, 12, 4096, 128) == 0


def test_prefill_rejects_bad_arguments_before_any_launch(lib):
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    f = ctypes.c_float
    rc = lib.fa_prefill(None, p, p, p, 0, 1, 1, 8, 1, f(0.125), None, ctypes.c_size_t(0), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"non-NULL" in lib.fa_last_error()
    odd = ctypes.c_void_p(p.value + 2)
    rc = lib.fa_prefill(odd, p, p, p, 0, 1, 1, 8, 1, f(0.125), None, ctypes.c_size_t(0), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"aligned" in lib.fa_last_error()
    rc = lib.fa_prefill(p, p, p, p, 0, 1, 1, 0, 1, f(0.125), None, ctypes.c_size_t(0), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"sequence length must be > 0" in lib.fa_last_error()
    rc = lib.fa_prefill(p, p, p, p, 0, 1, 1, 8, 1, f(float("inf")), None, ctypes.c_size_t(0), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"scale must be finite" in lib.fa_last_error()
    rc = lib.fa_prefill(p, p, p, p, 7, 1, 1, 8, 1, f(0.125), None, ctypes.c_size_t(0), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"out_dtype" in lib.fa_last_error()
    # A workspace that is not 16-byte aligned is refused before anything runs.
    rc = lib.fa_prefill(p, p, p, p, 0, 1, 1, 8, 1, f(0.125), odd, ctypes.c_size_t(32), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"workspace must be" in lib.fa_last_error()


def test_decode_rejects_bad_arguments_before_any_launch(lib):
    buf = ctypes.create_string_buffer(1 << 16)
    p = ctypes.cast(buf, ctypes.c_void_p)
    f = ctypes.c_float
    sz = ctypes.c_size_t
    rc = lib.fa_decode(p, p, p, None, p, 0, 1, 2, 8, f(0.125), 128, p, sz(1 << 16), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"non-NULL" in lib.fa_last_error()
    rc = lib.fa_decode(p, p, p, p, p, 0, 1, 2, 0, f(0.125), 128, p, sz(1 << 16), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"cache length must be in [1, " in lib.fa_last_error()
    rc = lib.fa_decode(p, p, p, p, p, 0, 1, 2, 8, f(0.125), 130, p, sz(1 << 16), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"multiple of the warp count" in lib.fa_last_error()
    rc = lib.fa_decode(p, p, p, p, p, 0, 1, 2, 8, f(0.125), 128, p, sz(16), None)
    assert rc == FA_ERR_WORKSPACE and b"workspace too small" in lib.fa_last_error()
    rc = lib.fa_decode(p, p, p, p, p, 0, 1, 2, 8, f(float("nan")), 128, p, sz(1 << 16), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"scale must be finite" in lib.fa_last_error()


def test_grouped_entry_points_check_the_head_grouping(lib):
    """kv_heads must be in (0, heads] and divide heads; checked before any launch."""
    buf = ctypes.create_string_buffer(1 << 16)
    p = ctypes.cast(buf, ctypes.c_void_p)
    f = ctypes.c_float
    sz = ctypes.c_size_t
    for kv in (0, -2, 3, 16):
        rc = lib.fa_prefill_gqa(p, p, p, p, 0, 1, 8, kv, 8, 1, f(0.125), None, sz(0), None)
        assert rc == FA_ERR_INVALID_ARGUMENT and b"kv_heads must divide heads" in lib.fa_last_error()
        rc = lib.fa_decode_gqa(p, p, p, p, p, 0, 1, 8, kv, 8, f(0.125), 128, p, sz(1 << 16), None)
        assert rc == FA_ERR_INVALID_ARGUMENT and b"kv_heads must divide heads" in lib.fa_last_error()
        assert lib.fa_decode_gqa_workspace_bytes(1, 8, kv, 4096, 128) == 0
    # The other checks are shared with the non-grouped entry points.
    rc = lib.fa_prefill_gqa(p, p, p, p, 0, 1, 8, 2, 0, 1, f(0.125), None, sz(0), None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"sequence length must be > 0" in lib.fa_last_error()
    rc = lib.fa_decode_gqa(p, p, p, p, p, 0, 1, 8, 2, 8, f(0.125), 128, p, sz(16), None)
    assert rc == FA_ERR_WORKSPACE and b"workspace too small" in lib.fa_last_error()


def test_grouped_decode_workspace_holds_one_partial_per_query_head(lib):
    # A forced split: partials are per query head, as without grouping.
    assert lib.fa_decode_gqa_workspace_bytes(32, 14, 2, 4096, 1024) == 32 * 14 * 4 * 66 * 4
    assert lib.fa_decode_gqa_workspace_bytes(32, 14, 14, 4096, 1024) == \
        lib.fa_decode_workspace_bytes(32, 14, 4096, 1024)
    assert lib.fa_decode_gqa_workspace_bytes(1, 12, 4, 4096, 128) == 12 * 32 * 66 * 4


def test_kv_append_rejects_bad_arguments_before_any_launch(lib):
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.cast(buf, ctypes.c_void_p)
    rc = lib.fa_kv_append(p, p, p, None, p, 1, 1, 8, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"non-NULL" in lib.fa_last_error()
    rc = lib.fa_kv_append(p, p, ctypes.c_void_p(p.value + 8), p, p, 1, 1, 8, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"16-byte aligned" in lib.fa_last_error()
    rc = lib.fa_kv_append(p, p, p, p, ctypes.c_void_p(p.value + 2), 1, 1, 8, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"4-byte aligned" in lib.fa_last_error()
    rc = lib.fa_kv_append(p, p, p, p, p, 1, 0, 8, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"must be > 0" in lib.fa_last_error()
    rc = lib.fa_kv_append(p, p, p, p, p, 1, 1, 0, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"cache length must be in [1, " in lib.fa_last_error()


def test_legacy_attention_argument_checks(lib):
    p = ctypes.c_void_p(4096)
    rc = lib.fa_legacy_attention(None, p, p, p, 8, 0, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"non-NULL" in lib.fa_last_error()
    rc = lib.fa_legacy_attention(ctypes.c_void_p(4100), p, p, p, 8, 0, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"16-byte aligned" in lib.fa_last_error()
    rc = lib.fa_legacy_attention(p, p, p, p, 8, 3, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"unknown legacy variant" in lib.fa_last_error()
    rc = lib.fa_legacy_attention(p, p, p, p, -1, 0, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"row count" in lib.fa_last_error()
    # n == 0 computes nothing and launches nothing (no device needed).
    assert lib.fa_legacy_attention(p, p, p, p, 0, 2, None) == FA_OK


def test_head_dim_entry_points_reject_other_sizes(lib):
    p = ctypes.c_void_p(4096)
    rc = lib.fa_prefill_hd(p, p, p, p, 0, 1, 2, 2, 8, 96, 1, ctypes.c_float(0.125), None, 0, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"head_dim must be 64 or 128" in lib.fa_last_error()
    lib.fa_decode_hd_workspace_bytes.restype = ctypes.c_size_t
    assert lib.fa_decode_hd_workspace_bytes(1, 2, 2, 8, 32, 0) == 0
    assert b"head_dim must be 64 or 128" in lib.fa_last_error()
    rc = lib.fa_kv_append_hd(p, p, p, p, p, 1, 1, 8, 256, None)
    assert rc == FA_ERR_INVALID_ARGUMENT and b"head_dim must be 64 or 128" in lib.fa_last_error()
    # The workspace of a forced split grows with head_dim: (D + 2) floats per partial.
    w64 = lib.fa_decode_hd_workspace_bytes(2, 3, 3, 1000, 64, 256)
    w128 = lib.fa_decode_hd_workspace_bytes(2, 3, 3, 1000, 128, 256)
    assert w64 == 2 * 3 * 4 * 66 * 4 and w128 == 2 * 3 * 4 * 130 * 4


def test_python_package_exposes_reference_surface():
    """flashattn_cuda/__init__.py:20-29 of the reference."""
    import flashattn_cuda as fa

    for name in ("prefill", "decode", "head_dim", "occupancy_report", "choose_decode_split",
                 "_decode_with_split", "legacy_naive", "legacy_tiled", "legacy_fused",
                 "prefill_gqa", "decode_gqa", "append_kv"):
        assert hasattr(fa, name), name
    assert fa.head_dim == 64 and fa.__version__ == "2.0.0"
    assert fa.choose_decode_split(512, 1, 12, 512) == 128
    assert fa.choose_decode_split(max_seq=4096, batch=32, heads=14, min_blocks=512) == 1024
    import torch

    x = torch.zeros(4, 64)
    for fn in (fa.legacy_naive, fa.legacy_tiled, fa.legacy_fused):
        with pytest.raises(RuntimeError, match="legacy kernels expect CUDA tensors"):
            fn(x, x, x)


def test_python_rejects_cpu_tensors_without_a_device():
    """'must be a CUDA tensor' (tests/test_correctness.py:213-214) needs no GPU."""
    import torch

    import flashattn_cuda as fa

    q = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        fa.prefill(q, q, q, True, 0.125)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        fa.decode(q[:, :, :1], q, q, torch.tensor([4], dtype=torch.int32), 0.125)
    # The device check comes first (flash_common.h:55-57), so a CPU fp32
    # tensor is reported as "not a CUDA tensor", as in the reference.
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        fa.prefill(q.float(), q.float(), q.float(), True, 0.125)


def test_seq_lens_sum_of_baseline_instance():
    lens = np.asarray(oracle.make_decode_inputs(32, 14, 8, seed=0)[3])
    assert lens.shape == (32,)
