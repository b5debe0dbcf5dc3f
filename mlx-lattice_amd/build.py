"""Build the gfx950 library and its Python binding in-tree.

Two artefacts land in ``mlx_lattice_amd/``:

* ``liblattice_hip.so`` — the HIP kernels behind the C ABI of
  ``include/lattice_hip.h`` (hipcc, ``--offload-arch=gfx950``);
* ``_ext.so`` — the native host layer (``native/features``) and its pybind11
  module (``native/bindings``), compiled against torch and linked to the
  library above with an ``$ORIGIN`` rpath.

Run ``python mlx-lattice_amd/build.py`` (or ``__graft_entry__.build()``).
Cross-compiles without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
PKG = HERE / 'mlx_lattice_amd'
CSRC = HERE / 'csrc'
NATIVE = HERE / 'native'
INCLUDE = REPO / 'include'
ARCH = 'gfx950'

HIP_SOURCES = ['scan.hip', 'sort.hip', 'coords.hip', 'conv.hip', 'conv_grad.hip', 'pool.hip', 'quantize.hip']
HOST_SOURCES = [
    'native/features/coordinates/relations.cpp',
    'native/features/convolution/api.cpp',
    'native/features/pooling/pooling.cpp',
    'native/features/quantization/quantization.cpp',
    'native/bindings/module.cpp',
]

# Packed FP32 instructions stay disabled in all device code.
HIP_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
]


def hipcc() -> str:
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    path = Path(rocm) / 'bin' / 'hipcc'
    return str(path) if path.exists() else 'hipcc'


def build_hip_library(verbose: bool = False) -> Path:
    out = PKG / 'liblattice_hip.so'
    tmp = PKG / 'liblattice_hip.so.tmp'
    extra = os.environ.get('LATTICE_HIPCC_FLAGS', '').split()
    cmd = [hipcc(), *HIP_FLAGS, *extra, '-shared', f'-I{INCLUDE}', f'-I{CSRC}',
           *[str(CSRC / s) for s in HIP_SOURCES], '-o', str(tmp)]
    if verbose:
        print(' '.join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


def build_extension(verbose: bool = False) -> Path:
    os.environ.setdefault('PYTORCH_ROCM_ARCH', ARCH)
    from torch.utils import cpp_extension

    build_dir = PKG / '_build'
    if build_dir.exists():
        shutil.rmtree(build_dir)
    build_dir.mkdir(parents=True)
    cpp_extension.load(
        name='_ext',
        sources=[str(HERE / s) for s in HOST_SOURCES],
        extra_include_paths=[str(INCLUDE), str(NATIVE)],
        extra_cflags=['-O2', '-std=c++17', '-D__HIP_PLATFORM_AMD__=1'],
        extra_ldflags=[f'-L{PKG}', '-llattice_hip', r'-Wl,-rpath,\$$ORIGIN', r'-Wl,-rpath,\$$ORIGIN/..'],
        build_directory=str(build_dir),
        with_cuda=True,
        verbose=verbose,
    )
    built = build_dir / '_ext.so'
    target = PKG / '_ext.so'
    shutil.copy2(built, target)
    return target


def build(verbose: bool = False) -> None:
    build_hip_library(verbose)
    build_extension(verbose)


if __name__ == '__main__':
    build(verbose='-v' in sys.argv)
