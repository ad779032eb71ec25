"""CPU checks on the gfx950 assembly of the kernels (no GPU needed).

global_to_lds16 (csrc/mfma_tile.h) sets m0, the LDS base of a direct
global->LDS load, from inline asm; the compiler reserves m0 and does not see
that write. These tests fail if anything else in the kernels defines or
reads m0, which would make the loads (or the other user) go wrong silently.
"""

import importlib.util
import os
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_spec = importlib.util.spec_from_file_location(
    "fa_build", os.path.join(REPO, "flash-attention-cuda_amd", "build.py"))
fa_build = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(fa_build)

GOOD = """
prefill_kernel:
\ts_mov_b32 m0, s4
\ts_nop 0
\tglobal_load_lds_dwordx4 v1, s[2:3]
\tv_add_u32_e32 v2, v3, v4 ; m0 in a comment is fine
\ts_mov_b32 m0, s5
\ts_nop 0
\tglobal_load_lds_dwordx4 v[4:5], off
\ts_mov_b32 m0, vcc_lo
\ts_nop 0
\tglobal_load_lds_dwordx4 v6, s[8:9]
"""


def test_m0_checker_accepts_the_load_sequence():
    assert fa_build.m0_problems(GOOD) == []


@pytest.mark.parametrize("planted", [
    "\ts_mov_b32 m0, -1\n\tds_read_b32 v0, v1\n",          # compiler-style m0 write
    "\tv_movrels_b32_e32 v0, v1\n",                       # implicit m0 read
    "\ts_sendmsg sendmsg(MSG_INTERRUPT)\n",               # implicit m0 read
    "\ts_mov_b32 s7, m0\n",                               # m0 read
    "\tglobal_load_lds_dwordx4 v1, off\n",                # load without its m0 write
    "\ts_mov_b32 m0, v0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, off\n",  # not an SGPR
    "\ts_mov_b32 m0, s4\n\tv_add_u32_e32 v1, v2, v3\n\tglobal_load_lds_dwordx4 v1, off\n",
])
def test_m0_checker_flags_other_uses(planted):
    assert fa_build.m0_problems(GOOD + planted)


def test_kernels_touch_m0_only_in_their_global_load_lds_sequences():
    with tempfile.TemporaryDirectory() as tmp:
        units = ["prefill_d64", "prefill_d128", "decode"]
        with ThreadPoolExecutor(max_workers=3) as pool:
            asm = list(pool.map(lambda unit: fa_build.device_assembly(unit, tmp), units))
    for src, text in zip(units, asm):
        assert "global_load_lds_dwordx4" in text, src
        problems = fa_build.m0_problems(text)
        assert not problems, f"{src}: " + "; ".join(problems[:5])
