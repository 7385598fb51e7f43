"""Build the gfx950 HIP library ``libmxlinear.so`` in-tree with hipcc.

Usage: ``python vllm-mach_amd/build.py`` (also called by ``__graft_entry__.build``).
Each ``csrc/*.hip`` is compiled to an object in parallel, then linked.
"""
from __future__ import annotations

import json
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "libmxlinear.so"
BUILD = HERE / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# per-kernel register, scratch and LDS figures of the last build (compiler remarks)
RESOURCES = BUILD / "kernel_resources.json"

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # codes and scales must be bit-exact: no contraction of separate mul/add
    "-ffp-contract=off",
    # keep the compiler from forming packed-FP32 ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep register staging arrays in VGPRs (the LDS budget belongs to the GEMM tiles)
    "-mllvm", "-disable-promote-alloca-to-lds",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


# per-source additions to FLAGS
FILE_FLAGS: dict[str, list[str]] = {
    "gemm_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # the dense MX wide launches: the iterative ILP schedule
    "gemm_wide_mx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    # the one-row SwiGLU launch: its SiLU arithmetic ahead of the weight stream schedules
    # better for instruction-level parallelism
    "gemm_stream_swiglu.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


_REMARK_FIELDS = {
    "VGPRs": "vgpr", "AGPRs": "agpr", "TotalSGPRs": "sgpr", "ScratchSize [bytes/lane]": "scratch",
    "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill", "LDS Size [bytes/block]": "lds",
    "Occupancy [waves/SIMD]": "occupancy",
}


def parse_resource_remarks(text: str) -> dict[str, dict[str, int]]:
    """Kernel name -> figures from hipcc's ``-Rpass-analysis=kernel-resource-usage`` remarks."""
    kernels: dict[str, dict[str, int]] = {}
    cur = None
    for line in text.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            cur = kernels.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+(?:\[[^\]]*\])?): (\d+) \[", line)
        if m and cur is not None and m.group(1).strip() in _REMARK_FIELDS:
            cur[_REMARK_FIELDS[m.group(1).strip()]] = int(m.group(2))
    return kernels


def _compile(src: Path) -> tuple[Path, dict[str, dict[str, int]]]:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src.name, []), f"-I{BUILD}", "-Rpass-analysis=kernel-resource-usage",
           "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj, parse_resource_remarks(r.stderr)


TORCH_OPS_SRC = CSRC / "torch_ops.cpp"
TORCH_OPS_OUT = HERE / "libmxlinear_torch.so"


def build_torch_ops(verbose: bool = False) -> Path:
    """The torch operator library (host C++ over the C ABI): registers the reference's
    native op names, loadable with ``torch.ops.load_library``."""
    import torch
    import torch.utils.cpp_extension as ext

    inc = ext.include_paths(device_type="cuda") + [str(HERE.parent / "include")]
    libdir = Path(torch.__file__).parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = TORCH_OPS_OUT.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
           "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{d}" for d in inc], str(TORCH_OPS_SRC), "-o", str(tmp),
           f"-L{libdir}", f"-L{HERE}", "-lmxlinear", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip",
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch op library build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, TORCH_OPS_OUT)
    if verbose:
        print(f"built {TORCH_OPS_OUT}")
    return TORCH_OPS_OUT


SILU_GEN = CSRC / "silu_table_gen.cpp"


def generate_silu_table() -> Path:
    """Compile and run the host generator of the SwiGLU activation table: it evaluates
    the device's binary32 SiLU (csrc/silu_math.h) for every bf16 gate of the table's
    range and writes ``_build/silu_table.h``, which the device code includes."""
    exe = BUILD / "silu_table_gen"
    out = BUILD / "silu_table.h"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-ffp-contract=off", "-Wall", f"-I{CSRC}",
           str(SILU_GEN), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"silu_table_gen build failed:\n{r.stdout}\n{r.stderr}")
    r = subprocess.run([str(exe), str(out)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"silu_table_gen failed:\n{r.stdout}\n{r.stderr}")
    return out


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    generate_silu_table()
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        done = list(pool.map(_compile, sources))
    objs = [o for o, _ in done]
    resources: dict[str, dict[str, int]] = {}
    for _, k in done:
        resources.update(k)
    RESOURCES.write_text(json.dumps(resources, indent=1, sort_keys=True))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    build_torch_ops(verbose)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
