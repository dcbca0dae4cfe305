"""Compiles the gfx950 kernels and the C ABI into faster-yoco_amd/libyoco_z1.so with hipcc (in-tree, so the
library travels with the source tree).  Numerics flags: correctly rounded fp32 division and square root, fp32
denormals kept, no contraction except explicit FMAs, no fast math; packed-fp32 instructions disabled."""
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


if __name__ == '__main__':
    print(build(verbose=True))
