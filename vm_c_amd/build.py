"""Build the gfx950 attention library and the vm_c C++ host layer in-tree.

    python -m vm_c_amd.build          # -> vm_c_amd/libvmc_attn.so, vm_c_amd/libvm_c_host.so

libvmc_attn.so : the C ABI of include/vmc_attn.h (HIP kernels, gfx950 only).
libvm_c_host.so: namespace vm_c host API (KV block manager, TQConfig,
                 AttentionBackend, kernel entry points) over the C ABI.
"""
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libvmc_attn.so")
HOST_LIB = os.path.join(PKG, "libvm_c_host.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -ffp-contract=off: every fused multiply-add in the kernels is written out
# (the quantizers are bit-exact against their references).  Packed fp32 ops
# are disabled for the device code.  Unaligned-access mode is off so the
# compiler never fuses naturally aligned narrow LDS reads into a wider,
# misaligned one (the LDS serves those with long stalls).
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Xclang", "-target-feature", "-Xclang", "-unaligned-access-mode",
             "-I", os.path.join(ROOT, "include"), "-I", CSRC]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-ffp-contract=off", "-D__HIP_PLATFORM_AMD__",
             "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HOST, "include"),
             "-I", "/opt/rocm/include"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return r


def build_kernels(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(BUILD, os.path.basename(s) + ".o")
        objs.append(o)
        lang = ["-x", "hip"] if s.endswith(".hip") else []
        cmds.append([HIPCC] + HIP_FLAGS + lang + ["-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        for r in ex.map(_run, cmds):
            if verbose and (r.stdout or r.stderr):
                print(r.stdout, r.stderr, file=sys.stderr)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB + ".tmp"] + objs)
    os.replace(LIB + ".tmp", LIB)
    return LIB


def build_host(verbose=False):
    srcs = sorted(glob.glob(os.path.join(HOST, "src", "*.cpp")))
    if not srcs:
        return None
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(BUILD, "host_" + os.path.basename(s) + ".o")
        objs.append(o)
        cmds.append(["g++"] + CXX_FLAGS + ["-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    _run(["g++", "-shared", "-fPIC", "-o", HOST_LIB + ".tmp"] + objs +
         ["-L", PKG, "-lvmc_attn", "-L", "/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(HOST_LIB + ".tmp", HOST_LIB)
    return HOST_LIB


def build(verbose=False):
    lib = build_kernels(verbose)
    host = build_host(verbose)
    return lib, host


if __name__ == "__main__":
    print(build(verbose=True))
