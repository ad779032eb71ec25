"""Batched multi-head causal FlashAttention kernels for head_dim = 64, on MI355X.

Drop-in for the reference package's API (flashattn_cuda/__init__.py:1-31 of
shrvan30/flash-attention-cuda): ``prefill``, ``decode``, ``head_dim``,
``occupancy_report``, ``choose_decode_split`` and the ``_decode_with_split``
benchmark hook, with the same tensor layouts ([B, H, N, 64] fp16 on the
``cuda`` device, which is the HIP device on ROCm) and the same errors.

Added beyond the reference: ``prefill_gqa`` and ``decode_gqa``, the same
kernels for grouped-query attention (k/v or the caches carry H_kv heads, H_kv
dividing H; query head h reads K/V head h // (H // H_kv), as
``k.repeat_interleave(H // H_kv, dim=1)`` would pair them), without
materialising the repeated K/V.

Also added: head_dim 128 (``head_dims == (64, 128)``; ``head_dim`` stays 64,
the reference's value). Every entry point takes the head size from the
tensors, which must agree on it.

Also added: ``append_kv(k_cache, v_cache, k, v, seq_lens)``, the caller's
cache write before a decode step (row ``seq_lens[b]``, then ``seq_lens[b] +=
1``, on the device), so a whole append + decode step can be captured in a
HIP graph and replayed per token.

The v1 ``legacy_naive/tiled/fused`` kernels of the reference (one (N, 64)
fp32 head, no mask, scale 1/8) are there too, with the reference's checks.

There is no fallback: if the compiled extension ``_C`` (and the HIP library
``libflashattn_hip.so`` it links) is missing, importing this package fails.
"""

# The extension links libc10/libtorch, which are only on the loader's path
# once torch itself has been imported (same reason as the reference).
import torch as _torch  # noqa: F401

try:
    from ._C import (  # noqa: F401
        _decode_fp32,
        _decode_gqa_fp32,
        _decode_gqa_with_split,
        _decode_with_split,
        _prefill_fp32,
        _prefill_gqa_fp32,
        append_kv,
        choose_decode_split,
        decode,
        decode_gqa,
        head_dim,
        head_dims,
        legacy_fused,
        legacy_naive,
        legacy_tiled,
        occupancy_report,
        prefill,
        prefill_gqa,
    )
except ImportError as exc:  # pragma: no cover - exercised only when unbuilt
    raise ImportError(
        "flashattn_cuda: the gfx950 extension is not built. Run "
        "`python flash-attention-cuda_amd/build.py` (or __graft_entry__.build()) "
        f"first. Underlying error: {exc}"
    ) from exc


__all__ = [
    "prefill",
    "decode",
    "prefill_gqa",
    "decode_gqa",
    "append_kv",
    "head_dim",
    "head_dims",
    "occupancy_report",
    "choose_decode_split",
    "legacy_naive",
    "legacy_tiled",
    "legacy_fused",
]

__version__ = "2.0.0"
