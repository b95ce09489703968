"""Builds, in-tree:
  libiq.so       the gfx950 HIP kernels + C ABI (include/iq.h), with hipcc;
  libiq_host.so  the C++ host layer (host/iq_host.h: .llmq container,
                 QuantModel, QuantView launchers), over libiq.so.

    python -m infer_amd.build          # or infer_amd.build.build()

The kernels are compiled for gfx950 only, without fast-math and with
-ffp-contract=off (the quantiser must round exactly like src/quant.cpp), and
with packed fp32 ops disabled.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libiq.so")
HOST_LIB = os.path.join(HERE, "libiq_host.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
# flags for host-only C++ that uses the HIP runtime API and include/iq.h
HOST_CXX_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__",
                  "-I" + os.path.join(os.path.dirname(HERE), "include"), "-I" + os.path.join(HERE, "host"),
                  "-I" + os.path.join(ROCM, "include")]
SOURCES = ["iq_abi.hip", "iq_quant.hip", "iq_gemv.hip", "iq_gemm.hip", "iq_chain.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
]


def hipcc():
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found")
    return p


def _run(cmd):
    return subprocess.run(cmd, capture_output=True, text=True)


def build(verbose=False):
    """Compiles every source to an object (in parallel), then links libiq.so."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    cmds = [[hipcc()] + compile_flags + ["-c", src, "-o", obj] for src, obj in zip(srcs, objs)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 4)) as ex:
        results = list(ex.map(_run, cmds))
    msgs = []
    for r in results:
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("hipcc failed building libiq.so")
        # hipcc's host pass warns that it does not know the packed-fp32 feature.
        msgs += [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l]
    tmp = LIB + ".tmp"
    r = _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed linking libiq.so")
    if verbose and msgs:
        sys.stderr.write("\n".join(msgs) + "\n")
    os.replace(tmp, LIB)
    build_host()
    return LIB


def build_host():
    """libiq_host.so: host/iq_host.cpp with g++, linked against libiq.so and
    the HIP runtime (found next to it / in ROCm at run time)."""
    tmp = HOST_LIB + ".tmp"
    cmd = (["g++"] + HOST_CXX_FLAGS + ["-shared", "-o", tmp, os.path.join(HERE, "host", "iq_host.cpp"),
           "-L" + HERE, "-liq", "-L" + os.path.join(ROCM, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    r = _run(cmd)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("g++ failed building libiq_host.so")
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


if __name__ == "__main__":
    print(build(verbose=True))
