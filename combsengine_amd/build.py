"""Build recipe for the gfx950 library (no cmake/ninja needed).

1. hipcc --genco compiles each csrc/cq_k_*.hip (the device code, split in
   four translation units that compile in parallel) into a gfx950 code
   object, lib/cq_k_*.hsaco.
2. hipcc compiles csrc/cq_scratch.hip (the no-allocation entry point's
   device scratch array and its address lookup) into lib/cq_scratch.o.
3. g++ compiles the host side (C ABI, module loading, quantisers) into
   lib/libcombs_qlinear.so, embedding the code objects with .incbin, links
   cq_scratch.o and the HIP runtime (libamdhip64).

The .so is self-contained: it loads its kernels with hipModuleLoadData at
first use on each device.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
OBJECTS = ("gemv", "gemv1", "gemv2", "gemm")  # csrc/cq_k_<name>.hip -> lib/cq_k_<name>.hsaco
SO = os.path.join(LIBDIR, "libcombs_qlinear.so")

HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17",
               # packed fp32 ops off (the compiler must not emit v_pk_*_f32)
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               # keep MFMA operands/results in VGPRs (no AGPR copies around the
               # fp32 epilogues that scale each superblock's MFMA result)
               "-mllvm", "-amdgpu-mfma-vgpr-form=1"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err)


def build(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    procs = []
    for name in OBJECTS:
        cmd = [os.path.join(ROCM, "bin", "hipcc"), "--genco", *HIPCC_FLAGS,
               os.path.join(CSRC, f"cq_k_{name}.hip"), "-o", os.path.join(LIBDIR, f"cq_k_{name}.hsaco")]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    failed = []
    for cmd, p in procs:
        _, err = p.communicate()
        err = "\n".join(l for l in err.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            failed.append(f"build failed: {' '.join(cmd)}\n{err}")
        elif verbose and err.strip():
            print(err[-4000:])
    if failed:
        raise RuntimeError("\n".join(failed))
    stale = os.path.join(LIBDIR, "cq_gfx950.hsaco")  # the former single code object
    if os.path.exists(stale):
        os.remove(stale)
    # the no-allocation entry point's scratch array (host + device object)
    scratch_o = os.path.join(LIBDIR, "cq_scratch.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), "-c", "-fPIC", *HIPCC_FLAGS, os.path.join(CSRC, "cq_scratch.hip"),
          "-o", scratch_o], verbose)
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-fopenmp", "-Wall",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f'-DCQ_HSACO_DIR="{LIBDIR}"',
          os.path.join(CSRC, "cq_host.cpp"), os.path.join(CSRC, "cq_quantize.cpp"), scratch_o,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", SO], verbose)
    return SO


if __name__ == "__main__":
    build(verbose=True)
