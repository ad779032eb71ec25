"""CPU tests of the on-box analysis report (flash-attention-cuda_amd/profile/run_analysis.py).

The timings run on the GPU box; these guard the FLOP / byte models, the decode
path rule and the markdown on synthetic rows, as the reference's analysis
script is checked by reading its tables. No GPU needed.
"""

import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "flash-attention-cuda_amd", "profile"))

import run_analysis as ra  # noqa: E402


def test_prefill_model_counts_the_causal_half_and_four_tensors():
    full = ra.prefill_model(1, 1, 1024, False, 1.0)
    causal = ra.prefill_model(1, 1, 1024, True, 1.0)
    # 4 N^2 d flops in 1 ms; the causal count is half of it.
    assert full["tflops"] == pytest.approx(4 * 1024 * 1024 * 64 / 1e-3 / 1e12)
    assert causal["tflops"] == pytest.approx(full["tflops"] / 2)
    # q, k, v read and o written once: 4 N d fp16 values.
    assert full["gbs"] == pytest.approx(4 * 1024 * 64 * 2 / 1e-3 / 1e9)
    assert full["pct_mfma"] == pytest.approx(100 * full["tflops"] / 2516.6)
    assert full["shape"] == "B=1, H=1, N=1024, full"


@pytest.mark.parametrize("batch,heads,seq,cus,path", [
    (1, 12, 4096, 256, "split-K + merge"),
    (1, 12, 512, 256, "whole-sequence"),    # short cache
    (1, 12, 513, 256, "split-K + merge"),
    (32, 14, 4096, 256, "whole-sequence"),  # B * H >= CUs
    (16, 16, 4096, 256, "whole-sequence"),
    (15, 17, 4096, 256, "split-K + merge"),
])
def test_decode_path_rule(batch, heads, seq, cus, path):
    assert ra.decode_path(batch, heads, seq, cus) == path


def test_decode_model_adds_partials_only_on_the_split_path():
    split = ra.decode_model(1, 12, 4096, 128, "split-K + merge", 1.0)
    whole = ra.decode_model(1, 12, 4096, 128, "whole-sequence", 1.0)
    cache = 2 * 12 * 4096 * 64 * 2
    partials = 2 * 12 * 32 * (64 + 2) * 4
    assert whole["gbs"] == pytest.approx(cache / 1e-3 / 1e9)
    assert split["gbs"] == pytest.approx((cache + partials) / 1e-3 / 1e9)
    assert split["units"] == 12 * 32 and whole["units"] == 12


def test_render_writes_every_table():
    occ = [{"kernel": "prefill_kernel<causal=true>", "threads_per_block": 512,
            "registers_per_thread": 240, "shared_bytes_per_block": 163840,
            "max_active_blocks_per_sm": 1, "theoretical_occupancy": 0.25}]
    prefill = [ra.prefill_model(1, 14, 4096, True, 0.0486)]
    before = [ra.decode_model(1, 12, 1024, 512, "split-K + merge", 0.010)]
    after = [ra.decode_model(1, 12, 1024, 128, "split-K + merge", 0.008)]
    text = ra.render([("GPU", "test")], occ, prefill, before, after, after, "cmd --out x")
    assert text.startswith("# On-box performance analysis (MI355X)")
    assert "Made by `cmd --out x`" in text
    assert "| `prefill_kernel<causal=true>` | 512 | 240 | 163,840 B | 1 | 25.0% |" in text
    assert "| B=1, H=14, N=4096, causal | 0.0486 |" in text
    assert "618." in text  # 30.06 GFLOP in 48.6 us
    assert "| B=1, H=12, S=1024 | 512 | 24 | 0.0100 |" in text
    assert "1.25x |" in text
    assert text.endswith("\n") and not text.endswith("\n\n")
