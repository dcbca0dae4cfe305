"""Compiles the gfx950 kernels and the C ABI into faster-yoco_amd/libyoco_z1.so with hipcc, and the PyTorch operator
layer over that ABI (host code only) into faster-yoco_amd/libyoco_z1_torch.so with the host compiler, in-tree, so
both libraries travel with the source tree.  Numerics flags of the kernels: correctly rounded fp32 division and
square root, fp32 denormals kept, no contraction except explicit FMAs, no fast math; packed-fp32 instructions
disabled."""
import os
import subprocess
import sys

CSRC = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(CSRC)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, 'include')
SOURCES = [os.path.join(CSRC, 'z1_kernels.hip'), os.path.join(CSRC, 'z1_embedding.hip')]
OUTPUT = os.path.join(PKG, 'libyoco_z1.so')
ARCH = os.environ.get('YOCO_Z1_ARCH', 'gfx950')
OPS_SOURCE = os.path.join(CSRC, 'z1_torch_ops.cpp')
OPS_OUTPUT = os.path.join(PKG, 'libyoco_z1_torch.so')

FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-shared',
    '-ffp-contract=off', '-fno-fast-math', '-fhip-fp32-correctly-rounded-divide-sqrt',
    '-fno-gpu-flush-denormals-to-zero',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wall', '-Wno-unused-command-line-argument',
]


def hipcc():
    return os.path.join(os.environ.get('ROCM_PATH', '/opt/rocm'), 'bin', 'hipcc')


def build(output=OUTPUT, extra=(), verbose=False):
    """Compile every source into `output` (written to a temporary name first, then renamed)."""
    tmp = output + '.tmp'
    cmd = [hipcc()] + FLAGS + list(extra) + ['-I', INCLUDE, '-o', tmp] + SOURCES
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown; that line is expected
    noise = [l for l in res.stderr.splitlines() if l.strip() and 'packed-fp32-ops' not in l]
    if res.returncode != 0:
        raise RuntimeError('yoco_z1: hipcc failed:\n' + res.stderr)
    if noise and verbose:
        print('\n'.join(noise), file=sys.stderr)
    os.replace(tmp, output)
    return output


def build_ops(output=OPS_OUTPUT, verbose=False):
    """The torch operator layer: torch's headers and libraries, the C ABI header, ROCm's HIP headers (for torch's
    stream type); the C ABI itself is resolved at run time (z1t_init), not linked."""
    import torch
    from torch.utils import cpp_extension
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    tlib = cpp_extension.library_paths()[0]
    inc = [x for d in cpp_extension.include_paths() for x in ('-I', d)]
    tmp = output + '.tmp'
    cmd = (['g++', '-O2', '-std=c++17', '-fPIC', '-shared', '-Wall', '-Werror',
            f'-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}', '-D__HIP_PLATFORM_AMD__=1',
            '-DUSE_ROCM=1'] + inc + ['-I', os.path.join(rocm, 'include'), '-I', INCLUDE, OPS_SOURCE,
                                     '-L', tlib, '-lc10', '-lc10_hip', '-ltorch_cpu', '-ldl',
                                     f'-Wl,-rpath,{tlib}', '-o', tmp])
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError('yoco_z1: building the operator layer failed:\n' + res.stderr)
    os.replace(tmp, output)
    return output


def build_all(verbose=False):
    return build(verbose=verbose), build_ops(verbose=verbose)


if __name__ == '__main__':
    print(build_all(verbose=True))
