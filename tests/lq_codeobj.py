"""Kernel metadata of the built liblq.so (CPU test infrastructure).

The library carries its gfx950 code objects in clang offload bundles (section .hip_fatbin, one bundle per compiled
source file).  `kernels()` unpacks the gfx950 entries of the library built in this tree, reads each code object's AMDGPU
metadata note with llvm-readelf and returns, per kernel, its demangled name, the workgroup size it was compiled for
(.max_flat_workgroup_size, from __launch_bounds__), its static LDS (.group_segment_fixed_size), its private segment
(.private_segment_fixed_size: register spills) and its register counts.

`LAUNCH_BLOCK` states, per kernel family, the workgroup size the library's launch sites use (leapquant_amd/csrc/*.hip),
as a function of the kernel's template arguments.
"""
import os
import re
import struct
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "leapquant_amd", "_build", "liblq.so")
READELF = "/opt/rocm/llvm/bin/llvm-readelf"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
LDS_PER_CU = 160 * 1024                 # gfx950: 160 KiB of LDS per CU (and at most that per workgroup)
VGPRS_PER_SIMD_LANE = 512               # unified VGPR + AGPR file per SIMD lane


def _code_objects(path):
    data = open(path, "rb").read()
    pos = 0
    while True:
        i = data.find(MAGIC, pos)
        if i < 0:
            return
        n = struct.unpack_from("<Q", data, i + 24)[0]
        off = i + 32
        for _ in range(n):
            o, size, tsz = struct.unpack_from("<QQQ", data, off)
            off += 24
            triple = data[off:off + tsz].decode()
            off += tsz
            if "gfx950" in triple:
                yield data[i + o:i + o + size]
        pos = i + 1


def _demangle(names):
    r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True, check=True)
    return r.stdout.splitlines()


def kernels(path=LIB):
    """[{name, mangled, block, lds, scratch, vgpr, agpr}] of every kernel in the library."""
    out = []
    for co in _code_objects(path):
        with tempfile.NamedTemporaryFile(suffix=".co") as f:
            f.write(co)
            f.flush()
            notes = subprocess.run([READELF, "--notes", f.name], capture_output=True, text=True, check=True).stdout
        # one metadata map per kernel: the entries of the amdhsa.kernels list (two-space indent)
        body = notes.split("amdhsa.kernels:", 1)[1] if "amdhsa.kernels:" in notes else ""
        for blk in re.split(r"\n  - ", body)[1:]:
            get = lambda key: re.search(r"\.%s:\s+(\S+)" % key, blk)
            if get("name") is None:                   # a later top-level list (amdhsa.version)
                continue
            name = get("name").group(1)
            out.append(dict(mangled=name, block=int(get("max_flat_workgroup_size").group(1)),
                            lds=int(get("group_segment_fixed_size").group(1)),
                            scratch=int(get("private_segment_fixed_size").group(1)),
                            vgpr=int(get("vgpr_count").group(1)), agpr=int(get("agpr_count").group(1))))
    for k, d in zip(out, _demangle([k["mangled"] for k in out])):
        k["name"] = d
    return out


def _targs(name):
    m = re.search(r"<([^<>]*)>\(", name)
    return [a.strip() for a in m.group(1).split(",")] if m else []


# kernel family -> workgroup size of its launch sites, from the template arguments
LAUNCH_BLOCK = {
    "gdn_step_kernel": lambda t: 128 * int(t[2]),                # <K, V, G, ...>: two waves per value head
    "kda_step_kernel": lambda t: 128,
    "dense_step_kernel": lambda t: 128 * int(t[0]),              # <G, F>
    "conv_update_kernel": lambda t: 256,
    "dequant4_kernel": lambda t: 256,
    "flush_kernel": lambda t: 512,
    "flush4_kernel": lambda t: 256,
    "flush64_kernel": lambda t: 256,
    "quantize_kernel": lambda t: 256,
    "quantize64_kernel": lambda t: 256,
    "dequant_kernel": lambda t: 512,
    "kda_dequant4_kernel": lambda t: 256,
    "lowrank_kernel": lambda t: 512,
}


def family(name):
    m = re.search(r"(\w+_kernel)\b", name)
    return m.group(1) if m else None


def launch_block(k):
    return LAUNCH_BLOCK[family(k["name"])](_targs(k["name"]))
