"""Offline build of the gfx950 code objects and the C-ABI host library.

Outputs (git-ignored, shipped in-tree to the GPU box):
  titan_amd/lib/paged_kv.hsaco      append / gather / page copy / table kernels
  titan_amd/lib/paged_decode_{f32,f16,bf16}.hsaco  split-K decode attention
  titan_amd/lib/paged_prefill.hsaco  MFMA causal chunked prefill
  titan_amd/lib/paged_decode_tiles_{f16,bf16,fp8}.hsaco  token-balanced decode
      (MFMA q.k, optional fused append)
  titan_amd/lib/libengine_hip.so    hipModuleLoad / hipModuleLaunchKernel C-ABI
"""
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

ARCH = "gfx950"
# (output code object, source, extra defines)
KERNELS = [
    ("paged_kv", "paged_kv", []),
    ("paged_decode_f32", "paged_decode", ["-DEH_ONLY_DT=0"]),
    ("paged_decode_f16", "paged_decode", ["-DEH_ONLY_DT=1"]),
    ("paged_decode_bf16", "paged_decode", ["-DEH_ONLY_DT=2"]),
    ("paged_prefill", "paged_prefill", []),
    ("paged_decode_tiles_f16", "paged_decode_tiles", ["-DEH_ONLY_DT=1"]),
    ("paged_decode_tiles_bf16", "paged_decode_tiles", ["-DEH_ONLY_DT=2"]),
    ("paged_decode_tiles_fp8", "paged_decode_tiles", ["-DEH_ONLY_DT=3"]),
]

# Packed-FP32 instructions are disabled for all device code on this pool.
HIP_DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "--genco", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc():
    p = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found")
    return p


def _run_parallel(cmds, verbose):
    procs = []
    for label, cmd in cmds:
        if verbose:
            print("[build]", " ".join(cmd), flush=True)
        procs.append((label, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                   stderr=subprocess.STDOUT, text=True)))
    failed = []
    for label, cmd, p in procs:
        out, _ = p.communicate()
        # hipcc's host pass warns about the device-only target feature: harmless.
        lines = [ln for ln in (out or "").splitlines() if "packed-fp32-ops" not in ln]
        if p.returncode != 0:
            failed.append((label, "\n".join(lines[-40:])))
        elif verbose and lines:
            print("\n".join(lines[-10:]))
    if failed:
        msg = "\n".join(f"--- {lab} ---\n{txt}" for lab, txt in failed)
        raise RuntimeError("build failed:\n" + msg)


def build(verbose=False):
    os.makedirs(LIB, exist_ok=True)
    hipcc = _hipcc()
    cmds = []
    for name, srcname, defs in KERNELS:
        src = os.path.join(CSRC, "kernels", srcname + ".hip")
        out = os.path.join(LIB, name + ".hsaco")
        cmds.append((name, [hipcc, *HIP_DEVICE_FLAGS, *defs, src, "-o", out + ".tmp"]))
    host_out = os.path.join(LIB, "libengine_hip.so")
    cmds.append(("libengine_hip", [
        "g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wno-unused-result",
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
        os.path.join(CSRC, "engine_hip.cpp"), os.path.join(CSRC, "kv_host.cpp"),
        os.path.join(CSRC, "kv_share.cpp"),
        "-o", host_out + ".tmp", f"-L{ROCM}/lib", "-lamdhip64", "-ldl",
        f"-Wl,-rpath,{ROCM}/lib",
    ]))
    _run_parallel(cmds, verbose)
    for name, _, _ in KERNELS:
        out = os.path.join(LIB, name + ".hsaco")
        os.replace(out + ".tmp", out)
    os.replace(host_out + ".tmp", host_out)
    return LIB


def build_oracle(verbose=False):
    """The CPU checker used by tests/ (not part of the product)."""
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["make", "-s", "-C", odir, "-B"], check=True,
                   stdout=None if verbose else subprocess.DEVNULL)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    build_oracle(verbose="-v" in sys.argv)
    print("built", LIB)
