"""Build the gfx950 code objects and the C-ABI host library in-tree.

    python llama.rust_amd/build.py

Outputs (next to this file, git-ignored, shipped with the tree):
  ghip_*.hsaco   one code object per kernel source, loaded with hipModuleLoad
  libghip.so     the C ABI declared in include/ghip.h
  libggml-hip.so the dlopen module declared in include/ggml_hip_reg.h
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

KERNELS = ["ghip_quant", "ghip_gemv", "ghip_wquant", "ghip_gemm", "ghip_fa", "ghip_moe", "ghip_skinny", "ghip_iq", "ghip_dense"]
DEVICE_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    # exact fp32 semantics: products and sums round on their own, fused
    # multiply-adds only where the source calls fmaf()
    "-ffp-contract=off",
    # no packed-fp32 instructions (known to misbehave on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-parameter",
]


def _run(cmd):
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


# MFMA results that the epilogue reads with vector ALU ops stay in VGPRs
# (the AGPR form would add a v_accvgpr_read per element)
EXTRA_FLAGS = {
    "ghip_moe": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "ghip_fa": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "ghip_gemm": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "ghip_skinny": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def build_kernels():
    for k in KERNELS:
        src = os.path.join(CSRC, k + ".hip")
        out = os.path.join(HERE, k + ".hsaco")
        _run([HIPCC, "--genco", *DEVICE_FLAGS, *EXTRA_FLAGS.get(k, []), "-I", CSRC, src, "-o", out])


def build_host():
    """libghip.so: the host library (g++) plus ghip_noalloc.hip (hipcc), whose
    code object carries the fixed scratch array of ghip_mul_mat_noalloc."""
    out = os.path.join(HERE, "libghip.so")
    obj = os.path.join(HERE, "ghip_noalloc.o")
    _run([HIPCC, "-c", "-fPIC", *DEVICE_FLAGS, "-I", CSRC, os.path.join(CSRC, "ghip_noalloc.hip"), "-o", obj])
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wno-unused-result", "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"),
          os.path.join(CSRC, "ghip.cpp"), os.path.join(CSRC, "ghip_gguf.cpp"), obj, "-o", out,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-ldl", "-Wl,-rpath," + os.path.join(ROCM, "lib")])


def build_backend_module():
    """libggml-hip.so: the dlopen module (ggml_backend_score / ggml_backend_init)
    over libghip.so, found next to it at run time."""
    out = os.path.join(HERE, "libggml-hip.so")
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"),
          os.path.join(CSRC, "ghip_backend_reg.cpp"), "-o", out,
          "-L", HERE, "-lghip", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(ROCM, "lib")])


def build():
    build_kernels()
    build_host()
    build_backend_module()


if __name__ == "__main__":
    build()
    sys.exit(0)
