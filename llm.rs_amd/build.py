"""Build the llmrs_hip backend: gfx950 code objects and the host library.

Plays the role a build.rs of the Rust crate would: every ``csrc/kernels/*.hip``
becomes ``lib/<name>.hsaco`` (``hipcc --genco --offload-arch=gfx950``), which
the host library loads with ``hipModuleLoad``; ``csrc/host/*.cpp`` becomes
``lib/libllmrs_hip.so`` with the C ABI of ``include/llmrs_hip.h``.

Run: ``python llm.rs_amd/build.py`` (always rebuilds).
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
BUILD = PKG / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

# -ffp-contract=off keeps a*b+c as two roundings, as in the reference (Rust
# never contracts).  Packed FP32 instructions are disabled for all device code.
# MFMA results go to ordinary VGPRs (-amdgpu-mfma-vgpr-form): the prefill
# GEMM's epilogue reads every MFMA result once, and accumulation registers
# would cost a copy instruction per element.
HIP_FLAGS = [
    "--genco", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]
HOST_HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-mf16c",
    "-Wall", "-Wextra", "-Wno-unused-parameter", "-D__HIP_PLATFORM_AMD__",
]


def _run_all(cmds: list[list[str]]) -> None:
    procs = [(c, subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
             for c in cmds]
    failed = []
    for cmd, p in procs:
        out, _ = p.communicate()
        noise = ("unknown target feature", "is not a recognized feature for this target")
        lines = [ln for ln in (out or "").splitlines() if not any(n in ln for n in noise) and ln.strip()]
        if p.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        elif lines:
            sys.stderr.write("\n".join(lines) + "\n")
    if failed:
        msg = "\n\n".join(f"$ {' '.join(c)}\n{o}" for c, o in failed)
        raise RuntimeError(f"llmrs_hip build failed:\n{msg}")


def build(verbose: bool = False) -> Path:
    """Compile every code object and the host library; returns the lib dir."""
    LIB.mkdir(exist_ok=True)
    hipcc = str(ROCM / "bin" / "hipcc")
    cmds = []
    outs = []
    for src in sorted((CSRC / "kernels").glob("*.hip")):
        out = LIB / f"{src.stem}.hsaco"
        tmp = out.with_suffix(".hsaco.tmp")
        cmds.append([hipcc, *HIP_FLAGS, f"-I{CSRC}", "-o", str(tmp), str(src)])
        outs.append((tmp, out))
    # Host sources with device data of their own (csrc/host/*.hip) are
    # compiled by hipcc into objects linked into the host library.
    BUILD.mkdir(exist_ok=True)
    host_objs = []
    obj_cmds = []
    for src in sorted((CSRC / "host").glob("*.hip")):
        obj = BUILD / f"{src.stem}.o"
        obj_cmds.append([hipcc, *HOST_HIP_FLAGS, f"-I{REPO / 'include'}", f"-I{CSRC}", "-c", "-o", str(obj),
                         str(src)])
        host_objs.append(str(obj))
    so = LIB / "libllmrs_hip.so"
    so_tmp = LIB / "libllmrs_hip.so.tmp"
    link = [
        os.environ.get("CXX", "g++"), *HOST_FLAGS, f"-I{ROCM / 'include'}", f"-I{REPO / 'include'}",
        f"-I{CSRC}", "-o", str(so_tmp), *map(str, sorted((CSRC / "host").glob("*.cpp"))), *host_objs,
        f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-ldl", "-lpthread",
    ]
    outs.append((so_tmp, so))
    if verbose:
        for c in cmds + obj_cmds + [link]:
            print("$", " ".join(c))
    _run_all(cmds + obj_cmds)
    _run_all([link])
    for tmp, out in outs:
        tmp.replace(out)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
