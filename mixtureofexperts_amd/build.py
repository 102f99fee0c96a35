"""Build libmoe_mi355x.so (HIP, gfx950) in-tree with hipcc.

The library is the product: every MoE-layer kernel and the C ABI declared in
include/moe_mi355x.h.  Python, Julia (ccall) or C callers load the same file.
"""
import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libmoe_mi355x.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["moe_api.hip", "moe_route.hip", "moe_gemm.hip", "moe_gemm_bf16.hip", "moe_decode.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-fno-fast-math",
    "-Wall",
    "-Wno-unused-function",
]
# Device pass only: packed fp32 VALU ops stay off (no compiler-generated
# v_pk_*_f32).  clang cannot forward -Xclang through -Xarch_device, so each
# source is compiled in two steps: the device code alone (with this feature)
# into an offload bundle, then the host code, which embeds that bundle.  A
# fixed -cuid per source keeps the two steps' compilation-unit ids equal,
# which makes the result byte-identical to a one-step hipcc compile.
DEVICE_ONLY_FLAGS = [
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE fp32 division / sqrt in device code (routing must be bit-exact)
    "-fhip-fp32-correctly-rounded-divide-sqrt",
]


# The device pass reports each kernel's resources (registers, LDS, private
# "scratch" memory per lane); build_library writes them to RESOURCES_PATH.
# A kernel with scratch keeps a register array in memory (a runtime index
# into it, or spills): the kernels here are written to need none.
RESOURCES_PATH = os.path.join(PKG_DIR, "kernel_resources.json")
_RESOURCE_FIELDS = {"TotalSGPRs": "sgprs", "VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch",
                    "Occupancy [waves/SIMD]": "occupancy", "VGPRs Spill": "vgpr_spill",
                    "LDS Size [bytes/block]": "lds"}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {LIB_NAME} (exit {res.returncode}): {' '.join(cmd)}")
    return res


def parse_resource_remarks(text):
    """{kernel symbol: {sgprs, vgprs, agprs, scratch, occupancy, lds}} from the
    compiler's kernel-resource-usage remarks."""
    import re

    out, name = {}, None
    for line in text.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            out[name] = {}
            continue
        if name is None:
            continue
        for label, key in _RESOURCE_FIELDS.items():
            m = re.search(r"remark:\s+" + re.escape(label) + r": (\d+)", line)
            if m:
                out[name][key] = int(m.group(1))
    return out


def build_library(verbose: bool = False) -> str:
    """Compile the HIP sources (one hipcc process each, in parallel) and link
    them into mixtureofexperts_amd/libmoe_mi355x.so."""
    import concurrent.futures
    import tempfile

    incs = ["-I", os.path.join(REPO_DIR, "include"), "-I", CSRC]

    def compile_one(src, tmpdir):
        stem = os.path.splitext(src)[0]
        path = os.path.join(CSRC, src)
        bundle = os.path.join(tmpdir, stem + ".hipfb")
        obj = os.path.join(tmpdir, stem + ".o")
        cuid = f"-cuid=moe_{stem}"
        dev = _run([HIPCC, *HIP_FLAGS, *DEVICE_ONLY_FLAGS, *incs, cuid, "--cuda-device-only",
                    "-Rpass-analysis=kernel-resource-usage", "-c", path, "-o", bundle], verbose)
        _run([HIPCC, *HIP_FLAGS, *incs, cuid, "--cuda-host-only", "-Xclang", "-fcuda-include-gpubinary", "-Xclang",
              bundle, "-c", path, "-o", obj], verbose)
        return obj, parse_resource_remarks(dev.stderr)

    import json

    with tempfile.TemporaryDirectory(prefix="moe_build_") as tmpdir:
        with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
            done = [f.result() for f in [pool.submit(compile_one, s, tmpdir) for s in SOURCES]]
        objs = [o for o, _ in done]
        tmp = LIB_PATH + ".tmp"
        _run([HIPCC, f"--offload-arch={ARCH}", "-fPIC", "-shared", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    resources = {src: res for src, (_, res) in zip(SOURCES, done)}
    with open(RESOURCES_PATH, "w") as f:
        json.dump(resources, f, indent=1, sort_keys=True)
    scratch = [k for r in resources.values() for k, v in r.items() if v.get("scratch", 0) > 0]
    if scratch:
        sys.stderr.write("warning: kernels with private (scratch) memory: " + ", ".join(scratch) + "\n")
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
