"""Builds libflashgrpo_amd.so from ss-grpo_amd/csrc with hipcc for gfx950.

The library is built in-tree (next to this file) so it travels with the
repository snapshot; objects go to ss-grpo_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB_NAME = "libflashgrpo_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = os.environ.get("FLASHGRPO_AMD_ARCH", "gfx950")

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in device code.
HIP_FLAGS = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *HIP_FLAGS, "-I", CSRC, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


# Sources whose kernels issue register-destination loads as inline assembly; their device
# assembly is checked for uses of a load's registers before it lands (_isa_check).
ASM_CHECKED = {"lm_head.hip": "lm_stream_kernel"}


def _device_asm(src: str) -> str:
    out = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".gfx950.s"))
    cmd = [hipcc(), *HIP_FLAGS, "-I", CSRC, "--cuda-device-only", "-S", src, "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{res.stderr}")
    return out


def check_inline_asm_loads(asm_path: str, name_filter: str) -> int:
    """Raises if any kernel matching name_filter touches an in-flight load's registers."""
    from ._isa_check import check_asm

    with open(asm_path) as f:
        n, hazards = check_asm(f.read(), name_filter)
    if not n:
        raise RuntimeError(f"{asm_path}: no kernel named *{name_filter}* to check")
    if hazards:
        lines = "\n".join(f"  {fn[:60]} line {ln}: {ins} uses {regs}" for fn, ln, ins, regs in hazards[:10])
        raise RuntimeError(f"{asm_path}: {len(hazards)} use(s) of in-flight load registers:\n{lines}")
    return n


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    checked = [s for s in sources if os.path.basename(s) in ASM_CHECKED]
    workers = max(1, min(len(sources) + len(checked), os.cpu_count() or 4, 10))
    with cf.ThreadPoolExecutor(workers) as ex:
        asm_jobs = [ex.submit(_device_asm, s) for s in checked]  # the longest jobs first
        objs = list(ex.map(_compile, sources))
        asms = [j.result() for j in asm_jobs]
    for src, asm in zip(checked, asms):
        n = check_inline_asm_loads(asm, ASM_CHECKED[os.path.basename(src)])
        if verbose:
            print(f"{os.path.basename(src)}: {n} kernels free of early uses of inline-asm load registers")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build()
