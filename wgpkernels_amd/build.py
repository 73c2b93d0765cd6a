"""Ahead-of-time build of the gfx950 INT8 linear library, written next to its Python layer:

    python -m wgpkernels_amd.build [--library int8] [--arch gfx950] [--output PATH] [--verbose] [--jobs N]

Mirrors the reference's ``python -m wgpkernels.build --hip ...`` (wgpkernels/build.py:73-98): one shared library per
kernel family, a plain C-ABI loaded with ctypes. Only the int8 family and only gfx950 exist here.

Compiler flags that the numerics depend on (the parity tests compare bits with a CPU restatement):
  -ffp-contract=off                            no implicit multiply-add fusion; every fused step is an explicit fmaf
  -fhip-fp32-correctly-rounded-divide-sqrt     IEEE division and square root
  -fno-gpu-flush-denormals-to-zero             denormals kept, as on the CPU
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed FP32 instructions (v_pk_*_f32)
Performance flags:
  -mllvm -amdgpu-mfma-vgpr-form=1              MFMA results in VGPRs (no accvgpr copies before the FP32 epilogue math)
"""
import argparse
import concurrent.futures
import os
import shlex
import shutil
import subprocess
import tempfile
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
DEFAULT_ARCH = "gfx950"
# int8: the product library (include/wq8.h); int8_test: the test-only entry points (include/wq8_test.h), kept out of it
LIBRARIES = {"int8": ["int8/csrc/quantize.hip", "int8/csrc/gemm.hip", "int8/csrc/gemm_bf16.hip", "int8/csrc/gemm_f16.hip",
                      "int8/csrc/fewtoken.hip", "int8/csrc/abi.hip"],
             "int8_test": ["int8/csrc/test_entry.hip"]}
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def rocm_path():
    return Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def library_file(name="int8"):
    return PACKAGE / name.split("_")[0] / f"libwgp_{name}.so"


def _compile(hipcc, source, obj, arch, verbose, include):
    cmd = [str(hipcc), f"--offload-arch={arch}", *HIP_FLAGS, f"-I{include}", "-c", str(source), "-o", str(obj)]
    if verbose:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    cmd += shlex.split(os.environ.get("WGPKERNELS_HIP_FLAGS", ""))
    subprocess.run(cmd, check=True)
    return obj


def build(name="int8", arch=DEFAULT_ARCH, output=None, verbose=False, jobs=None):
    """Compiles every source of the family with hipcc for `arch` and links the shared library; returns its path."""
    if name not in LIBRARIES:
        raise ValueError(f"unknown library {name!r}; this build has {sorted(LIBRARIES)}")
    hipcc = rocm_path() / "bin" / "hipcc"
    target = Path(output or library_file(name)).resolve()
    target.parent.mkdir(parents=True, exist_ok=True)
    sources = [PACKAGE / s for s in LIBRARIES[name]]
    include = sources[0].parent
    with tempfile.TemporaryDirectory(prefix="wgpkernels-amd-build-") as work:
        objs = [Path(work) / (s.stem + ".o") for s in sources]
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs or min(len(sources), 8)) as pool:
            list(pool.map(lambda so: _compile(hipcc, so[0], so[1], arch, verbose, include), zip(sources, objs)))
        built = Path(work) / target.name
        subprocess.run([str(hipcc), f"--offload-arch={arch}", "-shared", "-fPIC", *map(str, objs), "-o", str(built)], check=True)
        shutil.copyfile(built, target)
    return target


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--library", default="int8", choices=sorted(LIBRARIES))
    parser.add_argument("--arch", default=DEFAULT_ARCH)
    parser.add_argument("--output", type=Path, default=None)
    parser.add_argument("--verbose", action="store_true", help="print register and LDS usage per kernel")
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args()
    print(f"Built {build(args.library, args.arch, args.output, args.verbose, args.jobs)}")


if __name__ == "__main__":
    main()
