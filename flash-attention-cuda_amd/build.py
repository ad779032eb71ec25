"""Build the gfx950 HIP library and the Python extension, in-tree.

    python flash-attention-cuda_amd/build.py

Produces, inside flash-attention-cuda_amd/flashattn_cuda/:
  libflashattn_hip.so   the C-ABI library (include/flashattn_hip.h), built by
                        hipcc for gfx950 from csrc/*.hip
  _C.<abi>.so           the pybind11 module `flashattn_cuda._C`
                        (csrc/bindings.cpp, host C++ only), linked to the
                        library above with an $ORIGIN rpath

The reference builds one CUDAExtension through setup.py (setup.py:12-44);
here the HIP kernels are a plain shared library so non-Python hosts can bind
them, and torch is only needed for the thin binding layer.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")
OUT_DIR = os.path.join(PKG_ROOT, "flashattn_cuda")
BUILD_DIR = os.path.join(PKG_ROOT, "_build")

# Compile units: (object name, csrc/ source, extra hipcc flags). prefill.hip
# is built once per head size: the head_dim 64 kernels schedule best with the
# iterative ILP strategy (C3 47.1 -> 46.0 us, C2 causal 20.2 -> 19.0 us, same
# bits), which makes the head_dim 128 full-attention kernel spill (51 -> 77
# us), so that one keeps the default scheduler.
HIP_UNITS = [
    ("runtime", "runtime.hip", []),
    ("prefill_d64", "prefill.hip",
     ["-DFA_PREFILL_D=64", "-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]),
    ("prefill_d128", "prefill.hip", ["-DFA_PREFILL_D=128"]),
    ("decode", "decode.hip", []),
    ("kv_cache", "kv_cache.hip", []),
    ("legacy", "legacy.hip", []),
]
LIB_NAME = "libflashattn_hip.so"
ARCH = os.environ.get("FA_OFFLOAD_ARCH", "gfx950")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed-FP32 VALU forms (v_pk_fma_f32 & co.) are kept out of the device
    # code; the host pass prints a harmless "not a recognized feature" note.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the prefill rescales and reads its O and S
    # accumulators with VALU ops, which cannot address AGPRs directly; the
    # AGPRs hold the MFMA-only source fragments instead.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _hipcc() -> str:
    path = os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(path):
        path = shutil.which("hipcc") or ""
    if not path:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return path


def build_hip_library(jobs: int = 4) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    cmds = []
    for name, src, extra in HIP_UNITS:
        obj = os.path.join(BUILD_DIR, name + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(_run, cmds))
    lib = os.path.join(OUT_DIR, LIB_NAME)
    tmp = lib + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, lib)
    return lib


def build_extension() -> str:
    import torch
    from torch.utils import cpp_extension

    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(OUT_DIR, "_C" + ext_suffix)
    tmp = out + ".tmp"
    torch_lib = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-DTORCH_EXTENSION_NAME=_C",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        *[f"-I{p}" for p in cpp_extension.include_paths()],
        f"-I{ROCM}/include",
        f"-I{sysconfig.get_paths()['include']}",
        f"-I{INCLUDE}",
        os.path.join(CSRC, "bindings.cpp"),
        "-o", tmp,
        f"-L{OUT_DIR}", "-lflashattn_hip",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
        "-ltorch_hip", "-ltorch_python",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


# --- m0 check ------------------------------------------------------------------
# The direct global->LDS loads (global_to_lds16 in csrc/mfma_tile.h) set m0,
# the LDS base of the load, from inline asm. The backend reserves m0 and does
# not see that write, so the kernels stay correct only while nothing else in
# them defines or reads m0. These checks run on the gfx950 assembly.

_M0_IMPLICIT_READERS = ("s_movrel", "v_movrel", "s_sendmsg", "ds_gws", "ds_append",
                        "ds_consume", "v_interp", "ds_read_addtid", "ds_write_addtid",
                        "s_ttracedata", "buffer_load_lds")
# The m0 value is an "s" operand of the asm, so the allocator may place it in
# any SGPR, VCC's halves included.
_M0_WRITE = re.compile(r"s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)$")


def m0_problems(asm: str) -> list:
    """Every instruction in `asm` (AMDGPU assembly) that defines or reads m0
    other than the global_to_lds16 pattern `s_mov_b32 m0, <SGPR>` [s_nop ...]
    `global_load_lds_dwordx4`, and every global_load_lds without that write
    right before it."""
    code = []
    for raw in asm.splitlines():
        ins = raw.split(";", 1)[0].strip()
        if ins and not ins.startswith(".") and not ins.endswith(":"):
            code.append(ins)
    problems = []
    for i, ins in enumerate(code):
        op = ins.split()[0]
        if op.startswith("global_load_lds"):
            j = i - 1
            while j >= 0 and code[j].startswith("s_nop"):
                j -= 1
            if j < 0 or not _M0_WRITE.match(code[j]):
                problems.append(f"global_load_lds without its m0 write: {ins}")
        elif re.search(r"\bm0\b", ins):
            j = i + 1
            while j < len(code) and code[j].startswith("s_nop"):
                j += 1
            if not (_M0_WRITE.match(ins) and j < len(code)
                    and code[j].split()[0].startswith("global_load_lds")):
                problems.append(f"m0 outside a global_load_lds sequence: {ins}")
        elif op.startswith(_M0_IMPLICIT_READERS) or (op.startswith("buffer_load") and " lds" in ins):
            problems.append(f"reads m0 implicitly: {ins}")
    return problems


def device_assembly(unit: str, out_dir: str) -> str:
    """gfx950 assembly of one compile unit (a HIP_UNITS name), built with the
    library's flags."""
    _, src, extra = next(u for u in HIP_UNITS if u[0] == unit)
    out = os.path.join(out_dir, unit + ".s")
    _run([_hipcc(), *HIPCC_FLAGS, *extra, "--cuda-device-only", "-S", os.path.join(CSRC, src),
          "-o", out])
    with open(out, encoding="utf-8") as handle:
        return handle.read()


def build(verbose: bool = True) -> None:
    lib = build_hip_library()
    if verbose:
        print(f"built {os.path.relpath(lib, REPO_ROOT)}")
    ext = build_extension()
    if verbose:
        print(f"built {os.path.relpath(ext, REPO_ROOT)}")


if __name__ == "__main__":
    build()
    sys.exit(0)
