"""CPU-side checks of the C ABI library and the host logic (no kernel launches): every symbol the header
declares is exported, argument errors come back as codes before any device work, and the Python surfaces refuse
CPU tensors instead of falling back."""
import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'yoco_z1.h')


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'^\s*(?:const\s+)?\w+\s*\*?\s*(z1_\w+)\s*\(', text, flags=re.M)))


def test_header_declares_the_abi():
    fns = header_functions()
    assert {'z1_table_create', 'z1_table_destroy', 'z1_owner_sum_bf16', 'z1_grad_sumsq', 'z1_norm_clip',
            'z1_clip_factor', 'z1_adam_cast', 'z1_scale_up', 'z1_cast_bf16', 'z1_strerror'} <= set(fns)


def test_library_exports_every_declared_symbol(pkg):
    from faster_yoco_amd import _lib
    L = _lib.lib()
    for name in header_functions():
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f'{name} has no ctypes signature'


def test_argument_errors_without_device_work(pkg):
    from faster_yoco_amd import _lib
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.z1_table_create(None, -1, 0, ctypes.byref(h)) == -2                  # Z1_E_SIZE
    assert L.z1_table_create(None, 0, 7, ctypes.byref(h)) == -3                   # Z1_E_DTYPE
    assert L.z1_table_create(None, 3, 0, ctypes.byref(h)) == -1                   # Z1_E_NULL
    row = (_lib.Z1Tensor * 1)(_lib.Z1Tensor(None, None, None, None, None, 4))
    assert L.z1_table_create(row, 1, 0, ctypes.byref(h)) == -1                    # row without a gradient
    row = (_lib.Z1Tensor * 1)(_lib.Z1Tensor(16, None, None, None, None, -5))
    assert L.z1_table_create(row, 1, 0, ctypes.byref(h)) == -2
    assert L.z1_owner_sum_bf16(None, 8, 10, 0.125, None, None, None, None) == -1
    nulls = (ctypes.c_void_p * 2)(None, None)
    assert L.z1_owner_sum_bf16(ctypes.cast(nulls, ctypes.c_void_p), 2, 10, 0.5, ctypes.c_void_p(32), None, None,
                               None) == -1
    assert L.z1_scale_up(None, None, None, 0, None) == 0                      # empty: a no-op whatever the pointers
    assert L.z1_cast_bf16(None, None, 0, None) == 0
    arr = (ctypes.c_void_p * 1)(16)
    assert L.z1_owner_sum_bf16(ctypes.cast(arr, ctypes.c_void_p), 0, 10, 1.0, ctypes.c_void_p(32), None, None,
                               None) == -4
    assert L.z1_owner_sum_bf16(ctypes.cast(arr, ctypes.c_void_p), 17, 10, 1.0, ctypes.c_void_p(32), None, None,
                               None) == -4
    assert L.z1_owner_sum_bf16(ctypes.cast(arr, ctypes.c_void_p), 1, -1, 1.0, ctypes.c_void_p(32), None, None,
                               None) == -2
    assert L.z1_adam_cast(None, None, 0, 0, 0, 0, 1, 1, 0, 1, None) == -1
    assert L.z1_grad_sumsq(None, None, None) == -1
    assert L.z1_norm_clip(None, None, 1.0, None, None, None, 1.0, None) == -1
    assert L.z1_clip_factor(None, None, 1.0, None, None, 1.0, None) == -1
    assert L.z1_scale_up(None, None, None, 4, None) == -1
    assert L.z1_cast_bf16(ctypes.c_void_p(16), ctypes.c_void_p(32), -1, None) == -2
    assert L.z1_cast_bf16(None, None, 4, None) == -1
    assert L.z1_table_destroy(None) == 0
    assert L.z1_owner_sum_workspace(-1) == -2
    # one partial per 256-element chunk of a grid that may be shifted by up to 63 elements (to the streams' lines)
    sizes = (0, 1, 193, 194, 256, 257, 449, 450, 513)
    assert [L.z1_owner_sum_waves(n) for n in sizes] == [0, 1, 1, 2, 2, 2, 2, 3, 3]
    assert [L.z1_owner_sum_workspace(n) - 2048 for n in sizes] == [L.z1_owner_sum_waves(n) for n in sizes]
    assert L.z1_owner_sum_waves(-1) == -2
    assert L.z1_owner_sum_bf16_waves(None, 1, 10, 1.0, ctypes.c_void_p(32), None, ctypes.c_void_p(64),
                                     None) == -1                                   # no contributions
    assert L.z1_owner_sum_bf16_waves(ctypes.cast(arr, ctypes.c_void_p), 0, 10, 1.0, ctypes.c_void_p(32), None,
                                     ctypes.c_void_p(64), None) == -4
    assert L.z1_reduce_waves(None, 4, ctypes.c_void_p(64), None) == -1
    assert L.z1_reduce_waves(ctypes.c_void_p(32), 4, None, None) == -1
    assert L.z1_reduce_waves(ctypes.c_void_p(32), -1, ctypes.c_void_p(64), None) == -2
    assert L.z1_grad_norm_clip(None, None, None, 1.0, None, None, None, 1.0, None) == -1
    assert L.z1_grad_update_scalars(None, None, None, None) == -1
    assert L.z1_table_set_grads(None, None, 0, None) == -1
    assert L.z1_table_set_grad_out(None, None, 0, None) == -1
    u = _lib.Z1UpdateScalars()
    assert L.z1_owner_sum_update(ctypes.cast(arr, ctypes.c_void_p), 1, 10, 1.0, ctypes.c_void_p(32), None, None,
                                 ctypes.byref(u), None) == -1                      # no workspace
    assert L.z1_owner_sum_update(ctypes.cast(arr, ctypes.c_void_p), 1, 10, 1.0, ctypes.c_void_p(32), None,
                                 ctypes.c_void_p(64), None, None) == -1            # no scalar outputs struct
    assert L.z1_owner_sum_update(ctypes.cast(arr, ctypes.c_void_p), 0, 10, 1.0, ctypes.c_void_p(32), None,
                                 ctypes.c_void_p(64), ctypes.byref(u), None) == -4
    assert L.z1_table_info(None, None, None, None) == -1
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -99):
        assert L.z1_strerror(code)


def test_python_surfaces_refuse_cpu_tensors(pkg):
    from faster_yoco_amd import fused_adam_cast, ops
    t = torch.zeros(8)
    with pytest.raises(RuntimeError, match='no CPU path'):
        ops.Table([(t, t, t, t, None, 8)], 'cpu')
    fa = fused_adam_cast.FusedAdamCast({})
    with pytest.raises(RuntimeError, match='no CPU path'):
        fa(2048 * 32, None, [[t], [t], [t], [t]], 3e-4, 0.9, 0.95, 1e-8, 1, 1, 1, 0.1)
    nc = torch.zeros(4, 4).t()
    with pytest.raises(RuntimeError, match='expected contiguous fp32 tensors'):
        fa(2048 * 32, None, [[nc], [nc], [nc], [nc]], 3e-4, 0.9, 0.95, 1e-8, 1, 1, 1, 0.1)
    d = torch.zeros(4, dtype=torch.float64)
    with pytest.raises(RuntimeError, match='expected contiguous fp32 tensors'):
        fa(2048 * 32, None, [[d], [d], [d], [d]], 3e-4, 0.9, 0.95, 1e-8, 1, 1, 1, 0.1)
    with pytest.raises(RuntimeError, match='unsupported adam mode'):
        fa(2048 * 32, None, [[t], [t], [t], [t]], 3e-4, 0.9, 0.95, 1e-8, 1, 2, 1, 0.1)
    with pytest.raises(RuntimeError, match='no CPU path'):
        fused_adam_cast.scale_up(torch.zeros(4, dtype=torch.bfloat16), torch.zeros(4), torch.ones(1))


def test_ce_reduce_range_checks(pkg):
    from faster_yoco_amd import ce_reduce
    s = torch.zeros(7 * 10, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match='GPU tensor'):
        ce_reduce.sum_slots(s, torch.zeros(10, dtype=torch.bfloat16), 10, 0, 10, 0, 0.125, 8)


def test_host_bias_corrections_and_scalar_rounding(pkg):
    from faster_yoco_amd import ops
    assert ops.f32(0.1) == float(np.float32(0.1))
    assert ops.f32(1e-8) == float(np.float32(1e-8))
    for step in (1, 2, 1000, 10 ** 6):
        bc = ops.bias_corrections(0.9, 0.95, step)
        assert bc == tuple(float(torch.tensor(1.0 - math.pow(b, step), dtype=torch.float32)) for b in (0.9, 0.95))
    assert ops.bias_corrections(0.9, 0.95, 3, 0) == (1.0, 1.0)


def test_config_shapes(pkg):
    from faster_yoco_amd import configs
    assert configs.numel('c1') == 9_438_208
    assert configs.numel('c2') == 430_662_912 and len(configs.shapes('c2')) == 38
    assert configs.numel('c4') == 3_445_303_296 and len(configs.shapes('c4')) == 304
    assert all(math.prod(s) % 64 == 0 for s in configs.shapes('c2'))       # no alignment gaps at align=64


def test_host_inputs_deterministic(pkg):
    from faster_yoco_amd import configs
    a = configs.host_inputs(1000, 'c5', seed=3)
    b = configs.host_inputs(1000, 'c5', seed=3)
    assert all(np.array_equal(a[k], b[k]) for k in ('g', 'p', 'm', 'v'))
    assert (np.abs(a['g']) == 1e4).sum() == 1


def test_layout_place_params_cpu(pkg):
    from faster_yoco_amd import layout
    ps = [torch.nn.Parameter(torch.randn(s)) for s in [(5, 3), (7,), (2, 2), (11,)]]
    before = [p.detach().clone() for p in ps]
    st = layout.place_params(ps, 2)
    owner, sizes = layout.greedy_partition([15, 7, 4, 11], 2)
    assert st['seg'] == max(sizes) and st['flat'].numel() == 2 * st['seg']
    for p, b, r in zip(ps, before, owner):
        assert torch.equal(p.data, b) and st['owner'][id(p)] == r
        off = (p.data.data_ptr() - st['flat'].data_ptr()) // 4
        assert r * st['seg'] <= off < (r + 1) * st['seg']


def test_header_is_plain_c_and_links(pkg, tmp_path):
    """include/yoco_z1.h compiles as C11 with gcc and a C program links and runs against libyoco_z1.so (argument
    errors only: no device work)."""
    import subprocess
    from faster_yoco_amd import _lib
    libdir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / 'abi_smoke'
    subprocess.run(['gcc', '-std=c11', '-Wall', '-Werror', '-I', os.path.join(ROOT, 'include'),
                    os.path.join(ROOT, 'tests', 'c', 'abi_smoke.c'), '-L', libdir, '-l:libyoco_z1.so',
                    f'-Wl,-rpath,{libdir}', '-o', str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and res.stdout.strip() == 'ok', res.stdout + res.stderr
