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


HOST_SOURCES = ("engine_hip.cpp", "kv_host.cpp", "kv_share.cpp")
SANITIZE = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=undefined"]


# The one host-library source with device code: the static scratch array of
# eh_append_decode_batched_noalloc (compiled by hipcc, linked by g++).
NOALLOC_SRC = os.path.join(CSRC, "noalloc.hip")
OBJ_DIR = os.path.join(ROOT, "_build", "obj")
NOALLOC_OBJ = os.path.join(OBJ_DIR, "noalloc.o")


def _noalloc_cmd(hipcc):
    return [hipcc, f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-c",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            NOALLOC_SRC, "-o", NOALLOC_OBJ]


def _host_cmd(out, extra=()):
    """g++ line of the C-ABI host library (the hipcc-built noalloc object is
    linked in as is)."""
    return [
        "g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wno-unused-result",
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", *extra,
        *(os.path.join(CSRC, f) for f in HOST_SOURCES), NOALLOC_OBJ,
        "-o", out, f"-L{ROCM}/lib", "-lamdhip64", "-ldl", f"-Wl,-rpath,{ROCM}/lib",
    ]


def build(verbose=False, host_only=False):
    os.makedirs(LIB, exist_ok=True)
    hipcc = _hipcc()
    cmds = []
    kernels = [] if host_only else KERNELS
    for name, srcname, defs in kernels:
        src = os.path.join(CSRC, "kernels", srcname + ".hip")
        out = os.path.join(LIB, name + ".hsaco")
        cmds.append((name, [hipcc, *HIP_DEVICE_FLAGS, *defs, src, "-o", out + ".tmp"]))
    os.makedirs(OBJ_DIR, exist_ok=True)
    _run_parallel([("noalloc", _noalloc_cmd(hipcc))], verbose)
    host_out = os.path.join(LIB, "libengine_hip.so")
    cmds.append(("libengine_hip", _host_cmd(host_out + ".tmp")))
    _run_parallel(cmds, verbose)
    for name, _, _ in kernels:
        out = os.path.join(LIB, name + ".hsaco")
        os.replace(out + ".tmp", out)
    os.replace(host_out + ".tmp", host_out)
    return LIB


def sanitize_check(pytest_args=("-x", "-q", "-m", "not gpu")):
    """Builds the host library (kv_host.cpp, kv_share.cpp, engine_hip.cpp) and
    the CPU oracle with AddressSanitizer + UndefinedBehaviorSanitizer into
    _build/sanitize/ and runs the CPU test suite against those builds (the
    GPU kernels are not involved).  Returns pytest's exit status."""
    out_dir = os.path.join(ROOT, "_build", "sanitize")
    os.makedirs(out_dir, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    _run_parallel([("noalloc", _noalloc_cmd(_hipcc()))], verbose=True)
    host = os.path.join(out_dir, "libengine_hip.so")
    orc = os.path.join(out_dir, "liborc_kv.so")
    _run_parallel([
        ("libengine_hip (sanitized)", _host_cmd(host, SANITIZE)),
        ("liborc_kv (sanitized)", ["gcc", "-O1", "-ffp-contract=off", "-fno-fast-math", "-fPIC",
                                   "-std=c11", "-Wall", "-Wextra", *SANITIZE, "-shared", "-o", orc,
                                   os.path.join(ROOT, "oracle", "kv_oracle.c"), "-lm"]),
    ], verbose=True)
    preload = [subprocess.run(["gcc", f"-print-file-name={n}"], capture_output=True,
                              text=True).stdout.strip() for n in ("libasan.so", "libubsan.so")]
    env = dict(os.environ)
    env.update({
        "TITAN_AMD_HOST_LIB": host, "TITAN_ORACLE_LIB": orc,
        "LD_PRELOAD": " ".join(preload),
        # the interpreter itself is not instrumented: only report errors of
        # the instrumented libraries, not Python's own allocations at exit
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
    })
    cmd = [sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), *pytest_args]
    print("[sanitize]", " ".join(cmd), flush=True)
    return subprocess.run(cmd, env=env, cwd=ROOT).returncode


def build_oracle(verbose=False):
    """The CPU checker used by tests/ (not part of the product)."""
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["make", "-s", "-C", odir, "-B"], check=True,
                   stdout=None if verbose else subprocess.DEVNULL)


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        sys.exit(sanitize_check())
    build(verbose="-v" in sys.argv, host_only="--host" in sys.argv)
    build_oracle(verbose="-v" in sys.argv)
    print("built", LIB)
