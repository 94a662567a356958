#!/usr/bin/env python3
"""Build the gfx950 code objects and the C-ABI launcher of the entropy engine.

Outputs (in lib/ next to this file):
  <stem>.hsaco                 one raw gfx950 ELF code object per csrc/kernels/<stem>.hip
  entropy_engine_meta.json     every kernel: code object, workgroup size, LDS bytes,
                               register counts -- read from the objects' own
                               AMDGPU metadata notes, checked again at load time
  gemm_{int8,fp8,fp16}_meta.json  CubinEngine-style meta (shared, num_warps,
                               name, BLOCK_M/N/K) for EntropyEngine.from_metadata
  libentropy_engine.so         host launcher (include/entropy_engine.h)

The role of the reference's AOT step (EE/python/compile_kernels.py:11-70,
which dumped Triton cubins + meta JSON) and of its setup.py, for gfx950.
Usage: python build.py [--jobs N] [--only-host]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
KDIR = os.path.join(CSRC, "kernels")
LIB = os.path.join(HERE, "lib")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "--cuda-device-only", "--no-gpu-bundle-output", "-c",
    "-O3", "-std=c++17", "-mcode-object-version=5",
    # packed FP32 VALU ops stay off (hand-written or compiler-formed)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", CSRC, "-I", INCLUDE,
]

# CubinEngine-style meta for the GEMM code object (EE/csrc/generated/*_meta.json schema).
GEMM_TILE = {"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 128}
GEMM_META = {"gemm_int8": "eek_gemm_i8", "gemm_fp8": "eek_gemm_f8", "gemm_fp16": "eek_gemm_f16"}


def _run(cmd, cwd=None):
    p = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _hipcc():
    path = os.path.join(ROCM, "bin", "hipcc")
    return path if os.path.exists(path) else shutil.which("hipcc")


def compile_kernel(stem: str) -> str:
    src = os.path.join(KDIR, stem + ".hip")
    out = os.path.join(LIB, stem + ".hsaco")
    _run([_hipcc(), *HIPCC_FLAGS, src, "-o", out])
    return out


def read_notes(hsaco: str):
    """Kernel descriptors from the code object's AMDGPU metadata note."""
    readelf = os.path.join(ROCM, "llvm", "bin", "llvm-readelf")
    text = _run([readelf, "--notes", hsaco])
    kernels, cur, arg_size = [], None, 0
    for line in text.splitlines():
        m = re.match(r"\s+(?:- )?\.(\w+):\s*(.*)$", line)
        if not m:
            continue
        key, val = m.group(1), m.group(2).strip()
        if key == "args":
            if cur is None:
                cur = {}
            cur["kernarg"] = 0
            continue
        if key == "size":                            # an entry of .args
            arg_size = int(val)
            continue
        if key == "value_kind":                      # explicit arguments only (no hidden ones)
            if val == "by_value" and cur is not None:
                cur["kernarg"] = cur.get("kernarg", 0) + arg_size
            continue
        if key in ("group_segment_fixed_size", "max_flat_workgroup_size", "vgpr_count", "agpr_count",
                   "sgpr_count", "private_segment_fixed_size", "kernarg_segment_size", "name"):
            if cur is None:
                cur = {}
            cur[key] = val if key == "name" else int(val)
            if "name" in cur and "max_flat_workgroup_size" in cur and "group_segment_fixed_size" in cur \
                    and "private_segment_fixed_size" in cur and "vgpr_count" in cur:
                kernels.append(cur)
                cur = None
    return kernels


def build_host() -> str:
    """The launcher (g++) plus ee_noalloc.hip (hipcc, host and device code: the
    device-resident workspace of ee_routed_linear_noalloc) in one library."""
    src = os.path.join(CSRC, "launcher", "ee_launcher.cpp")
    noalloc = os.path.join(CSRC, "launcher", "ee_noalloc.hip")
    out = os.path.join(LIB, "libentropy_engine.so")
    tmp = out + ".tmp"
    obj = os.path.join(LIB, "ee_noalloc.o")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-c", "-O2", "-fPIC", "-std=c++17", "-fvisibility=hidden",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", INCLUDE, "-I", CSRC, noalloc, "-o", obj])
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-fvisibility=hidden", "-Wall", "-Wextra",
          "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", INCLUDE, "-I", CSRC,
          src, obj, "-o", tmp, "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,--no-undefined"])
    os.replace(tmp, out)
    return out


def build(jobs: int = 8, only_host: bool = False, verbose: bool = True) -> str:
    os.makedirs(LIB, exist_ok=True)
    stems = sorted(f[:-4] for f in os.listdir(KDIR) if f.endswith(".hip"))
    if not only_host:
        with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
            list(ex.map(compile_kernel, stems))
        meta = {"format": "entropy-engine-meta/1", "arch": ARCH, "code_objects": {}, "kernels": {}}
        for stem in stems:
            meta["code_objects"][stem] = {"file": stem + ".hsaco"}
            for k in read_notes(os.path.join(LIB, stem + ".hsaco")):
                if k["private_segment_fixed_size"] != 0:
                    raise RuntimeError(f"{k['name']} spills to scratch ({k['private_segment_fixed_size']} B/lane)")
                meta["kernels"][k["name"]] = {
                    "code_object": stem,
                    "block": k["max_flat_workgroup_size"],        # every kernel launches at its bound
                    "lds": k["group_segment_fixed_size"],
                    "max_flat_workgroup_size": k["max_flat_workgroup_size"],
                    "vgpr": k["vgpr_count"], "agpr": k.get("agpr_count", 0), "sgpr": k.get("sgpr_count", 0),
                    # bytes of the kernel's by-value argument block; the launcher checks
                    # it against the size of the struct it passes
                    "kernarg": k.get("kernarg", 0),
                }
                if meta["kernels"][k["name"]]["kernarg"] <= 0:
                    raise RuntimeError(f"{k['name']}: no by-value argument block in the code object's notes")
        for name, kern in GEMM_META.items():
            d = meta["kernels"][kern]
            with open(os.path.join(LIB, name + "_meta.json"), "w") as f:
                json.dump({"shared": d["lds"], "num_warps": d["block"] // 64, "name": kern, **GEMM_TILE}, f, indent=2)
        with open(os.path.join(LIB, "entropy_engine_meta.json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
    so = build_host()
    if verbose:
        print(f"built {len(stems)} code objects + {os.path.relpath(so, ROOT)}")
    return so


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--only-host", action="store_true")
    args = ap.parse_args(argv)
    build(args.jobs, args.only_host)


if __name__ == "__main__":
    sys.exit(main())
