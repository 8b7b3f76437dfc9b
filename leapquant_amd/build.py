"""Builds liblq.so (the HIP kernels + C ABI of include/lq.h) in-tree for gfx950, and liblq_probe.so (a streaming-read
probe that bench.py times as the memory system's ceiling; not part of the API).

    python -m leapquant_amd.build          # -> leapquant_amd/_build/liblq.so, liblq_probe.so

hipcc cross-compiles without a GPU.  Every HIP file gets `-Xclang -target-feature -Xclang -packed-fp32-ops` (no
packed FP32 instructions in the device code).
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(OUT, "liblq.so")
SOURCES = ("lq_step.hip", "lq_flush.hip", "lq_dequant.hip", "lq_dense.hip", "lq_noalloc.hip")
PROBE_LIB = os.path.join(OUT, "liblq_probe.so")
PROBE_SOURCES = ("lq_probe.hip",)
ARCH = os.environ.get("LQ_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if p and (os.path.sep not in p or os.path.exists(p)):
            return p
    raise RuntimeError("hipcc not found")


def _compile_one(cc, flags, s, verbose):
    src = os.path.join(CSRC, s)
    obj = os.path.join(OUT, s.replace(".hip", ".o"))
    cmd = [cc] + flags + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on %s:\n%s" % (s, r.stderr))
    if verbose:
        err = "\n".join(x for x in r.stderr.splitlines() if "packed-fp32-ops" not in x)
        if err.strip():
            print(err)
    return obj


def _compile_link(cc, flags, sources, lib, verbose):
    # one hipcc process per source file, run side by side (each is single-threaded)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile_one(cc, flags, s, verbose), sources))
    tmp = lib + ".tmp"
    cmd = [cc, "--offload-arch=%s" % ARCH, "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n%s" % r.stderr)
    os.replace(tmp, lib)


def build(verbose=False):
    os.makedirs(OUT, exist_ok=True)
    cc = hipcc()
    # -amdgpu-atomic-optimizer-strategy=None: every atomic of the library is issued by one lane, so the optimizer's
    # wave-wide rewrite buys nothing, and its result broadcast (a readfirstlane right after the atomic) makes the wave
    # wait for the atomic's return at once -- the flush's schedule take would then hold wave 0 for its round trip
    flags = ["--offload-arch=%s" % ARCH, "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", "-Wno-inline-asm",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]
    _compile_link(cc, flags, SOURCES, LIB, verbose)
    _compile_link(cc, flags, PROBE_SOURCES, PROBE_LIB, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
