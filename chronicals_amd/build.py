"""Build libchronicals_cce.so (HIP, gfx950) in-tree with hipcc.

The library is compiled from ``chronicals_amd/csrc/cce_kernels.hip`` into
``chronicals_amd/lib/libchronicals_cce.so``; the package loads it from there
with ctypes.  Building always recompiles.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
SRC = os.path.join(PKG_DIR, "csrc", "cce_kernels.hip")
HEADER = os.path.join(REPO_DIR, "include", "chronicals_cce.h")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_NAME = "libchronicals_cce.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
# per-kernel register / LDS / spill report of the last build (compiler remarks)
RESOURCES_PATH = os.path.join(LIB_DIR, "libchronicals_cce.resources.txt")
ARCH = "gfx950"


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build chronicals_amd")


def source_hash(paths=(SRC, HEADER)) -> str:
    """SHA-256 (hex) over the files the library is compiled from, in order.
    The build compiles it into the library (cce_source_hash()), so the loader
    can tell a library built from other sources."""
    h = hashlib.sha256()
    for p in paths:
        with open(p, "rb") as f:
            data = f.read()
        h.update(os.path.basename(p).encode() + b"\0" + str(len(data)).encode() + b"\0" + data)
    return h.hexdigest()


def compile_command(out_path: str, src_hash: str = None) -> list:
    return [
        hipcc_path(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # packed fp32 VALU ops stay off (the compiler may not form them)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(REPO_DIR, "include"),
        # bare hex digits (the source stringifies them): no shell quoting involved
        f"-DCCE_SOURCE_HASH={src_hash or source_hash()}",
        # per-kernel resource usage (VGPRs, spills, LDS) as compiler remarks
        "-Rpass-analysis=kernel-resource-usage",
        "-o", out_path,
        SRC,
    ]


def parse_resources(text: str) -> dict:
    """{kernel symbol: {field: int}} from kernel-resource-usage remarks."""
    out, cur = {}, None
    for line in text.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].strip()
        body = body.split(" [-Rpass", 1)[0]
        if body.startswith("Function Name:"):
            cur = out.setdefault(body.split(":", 1)[1].strip(), {})
        elif cur is not None and ":" in body:
            key, val = body.split(":", 1)
            try:
                cur[key.strip()] = int(val.strip().split()[0])
            except ValueError:
                pass
    return out


def build(verbose: bool = False) -> str:
    """Compile the HIP library; returns the path of the built .so."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + f".tmp{os.getpid()}"
    cmd = compile_command(tmp, source_hash())
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    os.replace(tmp, LIB_PATH)
    res = parse_resources(proc.stdout + proc.stderr)
    with open(RESOURCES_PATH, "w") as f:
        for name in sorted(res):
            f.write(name + " " + " ".join(f"{k.replace(' ', '_')}={v}" for k, v in sorted(res[name].items())) + "\n")
    spills = {n: r.get("VGPRs Spill", 0) for n, r in res.items() if r.get("VGPRs Spill", 0)}
    if spills:
        sys.stderr.write(f"warning: kernels spill VGPRs to scratch: {spills}\n")
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
