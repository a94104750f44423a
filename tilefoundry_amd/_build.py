"""Build the native parts in-tree.

Two shared objects, both written next to this file:

* ``libtilefoundry_amd.so`` -- every HIP kernel plus the ``extern "C"`` entry
  points declared in ``include/tilefoundry_amd.h``, compiled by ``hipcc`` for
  gfx950 only;
* ``_C<ext suffix>`` -- the thin PyTorch extension over that C ABI: tensor
  checks, the current HIP stream, status codes raised as Python exceptions.

Run ``python -m tilefoundry_amd._build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJ = ROOT / "_build"
LIB = PKG / "libtilefoundry_amd.so"
EXT = PKG / ("_C" + sysconfig.get_config_var("EXT_SUFFIX"))
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

# gfx950 only. Packed-f32 VALU ops are switched off: the compiler forms them
# from ordinary float code, and the kernels here do not need them.
HIPFLAGS = [
    "-O3", "--offload-arch=gfx950", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(INCLUDE), "-I", str(CSRC),
    "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(
            f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}"
        )


# Per-file code-generation options.
# * MFMA results in the vector registers (-amdgpu-mfma-vgpr-form): the prefill
#   attention keeps its output accumulators and resident Q operands in one
#   wave's register budget without the accumulation-register copies the
#   default form inserts.
# * IEEE mode off with NaNs assumed absent (MLA attention): fmaxf then needs no
#   input quieting, and the DPP max reductions fold into v_max_f32_dpp.
VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
FILE_FLAGS = {
    "prefill.hip": VGPR_MFMA,
    "mla.hip": ["-mno-amdgpu-ieee", "-fno-honor-nans"],
}


def _compile_hip(src: Path) -> Path:
    out = OBJ / (src.name + ".o")
    _run([HIPCC, *HIPFLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(out)])
    return out


def _torch_flags() -> tuple[list[str], list[str]]:
    from torch.utils import cpp_extension as ce  # noqa: PLC0415

    inc = [f"-I{p}" for p in ce.include_paths()]
    inc += [f"-I{sysconfig.get_paths()['include']}", f"-I{ROCM / 'include'}", f"-I{INCLUDE}"]
    libs = [f"-L{p}" for p in ce.library_paths()]
    libs += [f"-Wl,-rpath,{p}" for p in ce.library_paths()]
    libs += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    import torch  # noqa: PLC0415

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    defs = ["-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H"]
    return inc + defs, libs


def _build_ext() -> None:
    cflags, libs = _torch_flags()
    _run([
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-w",
        *cflags, str(CSRC / "torch_ext.cpp"), "-o", str(EXT),
        f"-L{PKG}", "-ltilefoundry_amd", "-Wl,-rpath,$ORIGIN",
        f"-L{ROCM / 'lib'}", "-lamdhip64", *libs,
    ])


def build(verbose: bool = True) -> None:
    """Compile every HIP source and the torch extension; always rebuilds."""
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("abi_*.cpp"))
    jobs = min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile_hip, sources))
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *map(str, objs), "-o", str(LIB),
          f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}"])
    _build_ext()
    if verbose:
        print(f"built {LIB.name} ({len(objs)} objects) and {EXT.name}", file=sys.stderr)


if __name__ == "__main__":
    build()
