"""Build libdsa_hip.so (the C-ABI HIP library) in-tree for gfx950.

    python -m dsa_triton_ascend_amd.build_lib

Sources under csrc/ are compiled with hipcc in parallel into _build/ at the
repository root and linked into dsa_triton_ascend_amd/libdsa_hip.so.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "libdsa_hip.so")
BUILD_DIR = os.path.join(ROOT, "_build")

SOURCES = [
    "capi.cpp",
    "sfa_fwd.hip",
    "sfa_bwd.hip",
    "li_fwd.hip",
    "kl_bwd.hip",
    "kl_generic.hip",
    "dense_kl.hip",
    "calib.hip",
]

ARCH = os.environ.get("DSA_OFFLOAD_ARCH", "gfx950")


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: set ROCM_PATH")
    return found


def common_flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
        "-Wno-unused-function", "-Wno-unused-variable",
        # packed fp32 VALU forms are kept out of the generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
    ]


# MFMA accumulators in VGPRs: with AGPR-form accumulators the register
# allocator keeps loop-carried accumulators in VGPRs anyway and copies them
# across on every iteration.  Not for sfa_bwd.hip: its D=512 kernel needs the
# AGPR file for its resident fragments, and the VGPR form crashes LLVM's
# AGPR-rewrite pass on it (ROCm 7.2 clang-22).
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]
PER_SOURCE_FLAGS = {
    "sfa_fwd.hip": VGPR_FORM,
    "li_fwd.hip": VGPR_FORM,
}


def _filter(text):
    keep = []
    for line in text.splitlines():
        if "packed-fp32-ops" in line and "not a recognized feature" in line:
            continue
        keep.append(line)
    return "\n".join(keep)


def _compile(src, extra):
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    cmd = ([hipcc()] + lang + common_flags() + PER_SOURCE_FLAGS.get(src, []) + extra
           + ["-c", os.path.join(CSRC, src), "-o", obj])
    r = subprocess.run(cmd, capture_output=True, text=True)
    return src, obj, r.returncode, _filter(r.stdout + r.stderr), cmd


def build(verbose=False, jobs=None, extra_flags=()):
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = jobs or min(8, len(SOURCES))
    objs = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, obj, rc, log, cmd in ex.map(lambda s: _compile(s, list(extra_flags)), SOURCES):
            if rc != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{log}")
            if verbose and log.strip():
                print(log)
            objs.append(obj)
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{_filter(r.stdout + r.stderr)}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
