"""z1_owner_sum_update_noalloc (the entry point that allocates nothing: its workspace is the library's static device
scratch) against z1_owner_sum_update with a caller workspace, through the C ABI: two calls in a row, the second on a
smaller input, every output bit-identical (the BF16 average, the FP32 sum, norm, grad_norm, factor, the two flags
and the clip metric); the same at Z1_NOALLOC_MAX_N elements, where the whole scratch is in use.  Sizes beyond
Z1_NOALLOC_MAX_N are refused before any device work."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _scalars(lib_mod, dev, sample):
    outs = {k: torch.full((1,), -7.0, device=dev) for k in ('norm', 'grad_norm', 'factor', 'clip')}
    flags = torch.full((2,), 9, dtype=torch.uint8, device=dev)
    u = lib_mod.Z1UpdateScalars(sample.data_ptr(), 8.0, None, 0.5, 1.0, outs['norm'].data_ptr(),
                                outs['grad_norm'].data_ptr(), outs['factor'].data_ptr(), flags.data_ptr(),
                                outs['clip'].data_ptr())
    return u, outs, flags


def _call(pkg, dev, contribs, n, noalloc):
    from faster_yoco_amd import _lib
    L = _lib.lib()
    avg = torch.empty(n, dtype=torch.bfloat16, device=dev)
    fsum = torch.empty(n, dtype=torch.float32, device=dev)
    sample = torch.tensor([16384.0], device=dev)
    u, outs, flags = _scalars(_lib, dev, sample)
    ptrs = (ctypes.c_void_p * len(contribs))(*[c.data_ptr() for c in contribs])
    stream = _lib.stream_handle(dev)
    if noalloc:
        rc = L.z1_owner_sum_update_noalloc(ctypes.cast(ptrs, ctypes.c_void_p), len(contribs), n, 1.0 / len(contribs),
                                           ctypes.c_void_p(avg.data_ptr()), ctypes.c_void_p(fsum.data_ptr()),
                                           ctypes.byref(u), stream)
    else:
        ws = torch.empty(int(L.z1_owner_sum_workspace(n)), dtype=torch.float64, device=dev)
        rc = L.z1_owner_sum_update(ctypes.cast(ptrs, ctypes.c_void_p), len(contribs), n, 1.0 / len(contribs),
                                   ctypes.c_void_p(avg.data_ptr()), ctypes.c_void_p(fsum.data_ptr()),
                                   ctypes.c_void_p(ws.data_ptr()), ctypes.byref(u), stream)
    assert rc == 0, L.z1_strerror(rc)
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy().view(np.uint32).copy() for k, v in outs.items()}
    res['avg'] = avg.view(torch.int16).cpu().numpy()
    res['sum'] = fsum.cpu().numpy().view(np.uint32)
    res['flags'] = flags.cpu().numpy()
    return res


def test_noalloc_owner_sum_update_matches_the_workspace_entry_point(pkg, dev):
    gen = torch.Generator(device='cpu').manual_seed(11)
    n_big, n_small = 1_000_003, 70_001
    contribs = [(torch.randn(n_big, generator=gen) * 1e-2).to(torch.bfloat16).to(dev) for _ in range(8)]
    for n in (n_big, n_small):                    # two calls in a row, the second on a smaller input
        want = _call(pkg, dev, [c[:n] for c in contribs], n, noalloc=False)
        got = _call(pkg, dev, [c[:n] for c in contribs], n, noalloc=True)
        for k in want:
            assert np.array_equal(got[k], want[k]), (n, k)
        assert got['flags'].tolist() == [1, 1]


def test_noalloc_at_its_maximum_size(pkg, dev):
    """Z1_NOALLOC_MAX_N elements: every slot of the scratch in use (the norm's partials, then one per 256-element
    chunk), the same bits as the workspace form."""
    from faster_yoco_amd import _lib
    n = _lib.Z1_NOALLOC_MAX_N
    gen = torch.Generator(device=dev).manual_seed(5)
    contribs = [(torch.randn(n, generator=gen, device=dev) * 1e-2).to(torch.bfloat16) for _ in range(2)]
    want = _call(pkg, dev, contribs, n, noalloc=False)
    got = _call(pkg, dev, contribs, n, noalloc=True)
    for k in want:
        assert np.array_equal(got[k], want[k]), k
    assert got['flags'].tolist() == [1, 1]


def test_noalloc_refuses_sizes_beyond_its_scratch(pkg, dev):
    from faster_yoco_amd import _lib
    L = _lib.lib()
    u = _lib.Z1UpdateScalars()
    one = (ctypes.c_void_p * 1)(16)
    rc = L.z1_owner_sum_update_noalloc(ctypes.cast(one, ctypes.c_void_p), 1, _lib.Z1_NOALLOC_MAX_N + 1, 1.0,
                                       ctypes.c_void_p(32), None, ctypes.byref(u), None)
    assert rc == -8 and b'no-allocation' in L.z1_strerror(rc)
