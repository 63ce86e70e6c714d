"""Build librlq.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python rust-llama_amd/build.py

Each .hip source compiles to an object under rust-llama_amd/_build/ in
parallel, then hipcc links rust-llama_amd/librlq.so.  Flags:
  --offload-arch=gfx950       MI355X only
  -ffp-contract=off           f32 rounds step by step, as the reference's Rust
  -Xclang -target-feature -Xclang -packed-fp32-ops
                              no packed-f32 instructions are generated
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = ["api.hip", "gemm.hip", "llama.hip", "matvec.hip", "probe.hip", "quantize.hip"]
HOST_SOURCES = ["gguf.cpp"]  # host-only C++ (no device code), built with g++
CXX = os.environ.get("CXX", "g++")
LIB = os.path.join(HERE, "librlq.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(HERE, "csrc"),
]


def _run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is harmless
    noise = ("unknown target feature", "packed-fp32-ops", "warning generated", "warnings generated")
    msg = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if l.strip() and not any(n in l for n in noise))
    return p.returncode, msg


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build (CPU test
# runs only): every flag reaches the host pass alone, the GPU code is built as
# usual; gguf.cpp is built by the same clang so one sanitizer runtime serves
# the process (libclang_rt.asan, preloaded by the oracle Makefile's
# `sanitize` target).
SAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=undefined"]
CLANGXX = "/opt/rocm/llvm/bin/clang++"


def build(verbose=False, sanitize=False):
    out_dir = os.path.join(HERE, "_asan" if sanitize else "_build")
    os.makedirs(out_dir, exist_ok=True)
    objs = [os.path.join(out_dir, s.replace(".hip", ".o")) for s in SOURCES]
    extra = SAN_HOST if sanitize else []
    cmds = [[HIPCC, *FLAGS, *extra, "-c", os.path.join(HERE, "csrc", s), "-o", o] for s, o in zip(SOURCES, objs)]
    host_objs = [os.path.join(out_dir, s.replace(".cpp", ".o")) for s in HOST_SOURCES]
    host_cxx, host_san = (CLANGXX, ["-fsanitize=address,undefined", "-fno-omit-frame-pointer",
                                    "-fno-sanitize-recover=undefined"]) if sanitize else (CXX, [])
    cmds += [[host_cxx, "-O2", "-std=c++17", "-fPIC", "-Wall", *host_san, "-I" + os.path.join(ROOT, "include"),
              "-I" + os.path.join(HERE, "csrc"), "-c", os.path.join(HERE, "csrc", s), "-o", o]
             for s, o in zip(HOST_SOURCES, host_objs)]
    srcs = SOURCES + HOST_SOURCES
    objs = objs + host_objs
    with concurrent.futures.ThreadPoolExecutor(len(cmds)) as ex:
        results = list(ex.map(_run, cmds))
    for (rc, msg), s in zip(results, srcs):
        if msg and (verbose or rc):
            print(f"[{s}]\n{msg}", file=sys.stderr)
        if rc:
            raise RuntimeError(f"hipcc failed on {s}")
    lib = os.path.join(out_dir, "librlq.so") if sanitize else LIB
    tmp = lib + ".tmp"
    link = ["-shared-libsan", *SAN_HOST] if sanitize else []
    rc, msg = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *link, "-o", tmp, *objs])
    if rc:
        raise RuntimeError(f"link failed:\n{msg}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose=True, sanitize="--sanitize" in sys.argv[1:]))
