"""Builds libvdxsampler.so (HIP, gfx950) in-tree with hipcc.

The library is the product: hand-written HIP kernels plus the C ABI declared
in include/vdx_sampler.h.  It is built into vindexllm_amd/lib/ so that it
travels with the source tree.
"""
from __future__ import annotations

import json
import os
import re
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libvdxsampler.so")
SOURCES = ["vdx_api.hip", "vdx_kernels.hip", "vdx_lmhead.hip", "vdx_gguf.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # bit-exact fp32 semantics: no FMA contraction, IEEE denormals,
    # correctly rounded division (HIP's default)
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    # no packed FP32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


RESOURCES = os.path.join(LIBDIR, "kernel_resources.json")


def parse_resource_remarks(text: str) -> dict:
    """Per-kernel register / scratch / occupancy figures from hipcc's
    -Rpass-analysis=kernel-resource-usage remarks."""
    out, cur = {}, None
    fields = {"VGPRs": "vgprs", "TotalSGPRs": "sgprs", "ScratchSize [bytes/lane]": "scratch",
              "Occupancy [waves/SIMD]": "occupancy", "LDS Size [bytes/block]": "lds",
              "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill"}
    for line in text.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([^:]+?): (\S+) \[-Rpass-analysis", line)
        if m and cur is not None and m.group(1) in fields:
            v = m.group(2)
            cur[fields[m.group(1)]] = int(v) if v.isdigit() else v
    return out


def build_library(verbose: bool = False) -> str:
    """Compiles every source for gfx950; always recompiles.  Writes the
    kernels' resource usage (registers, scratch, occupancy) next to the
    library."""
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage",
           "-I", os.path.join(ROOT, "include"), "-o", tmp,
           *[os.path.join(CSRC, s) for s in SOURCES]]
    r = subprocess.run(cmd, cwd=CSRC, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    if verbose:
        print(" ".join(cmd))
    with open(RESOURCES, "w") as f:
        json.dump(parse_resource_remarks(r.stderr), f, indent=1, sort_keys=True)
    os.replace(tmp, LIB)
    return LIB


CPP_TESTBED_SRC = os.path.join(ROOT, "tests", "cpp", "test_sampler_testbed.cpp")
CPP_TESTBED = os.path.join(ROOT, "tests", "cpp", "_build", "test_sampler_testbed")


def build_cpp_testbed(out: str = CPP_TESTBED, rpath: str | None = None) -> str:
    """The C++ host mirror's testbed (include/vdx_sampler.hpp, a port of the
    reference's sampler testbed), linked against the built library; the
    default rpath is relative to the binary, so the tree can move."""
    os.makedirs(os.path.dirname(out), exist_ok=True)
    if rpath is None:
        rpath = "$ORIGIN/" + os.path.relpath(LIBDIR, os.path.dirname(out))
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"), "-o", out, CPP_TESTBED_SRC,
           "-L", LIBDIR, "-lvdxsampler", "-Wl,-rpath," + rpath]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("g++ failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))
