"""z1_owner_sum_update_noalloc (the entry point that allocates nothing: its workspace is the library's static device
scratch) against z1_owner_sum_update with a caller workspace, through the C ABI: two calls in a row, the second on a
smaller input, every output bit-identical (the BF16 average, the FP32 sum, norm, grad_norm, factor, the two flags
and the clip metric); the same at Z1_NOALLOC_MAX_N elements, where the whole scratch is in use.  Sizes beyond
Z1_NOALLOC_MAX_N are refused before any device work.  In a fresh process whose first call of the entry point is made
under HIP graph capture (where the scratch's address is looked up), the replays match the workspace form, and an
eager call changes neither torch's allocation counters nor the device's free memory."""
import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

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


_CAPTURE_FIRST = textwrap.dedent("""
    import ctypes, sys
    import numpy as np
    import torch
    sys.path.insert(0, {root!r})
    sys.path.insert(0, {tests!r})
    import __graft_entry__
    __graft_entry__.package()
    import test_zz_no_alloc as t
    from faster_yoco_amd import _lib
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    n = 300_007
    gen = torch.Generator(device='cpu').manual_seed(23)
    contribs = [(torch.randn(n, generator=gen) * 1e-2).to(torch.bfloat16).to(dev) for _ in range(8)]
    L = _lib.lib()
    avg = torch.empty(n, dtype=torch.bfloat16, device=dev)
    fsum = torch.empty(n, dtype=torch.float32, device=dev)
    sample = torch.tensor([16384.0], device=dev)
    u, outs, flags = t._scalars(_lib, dev, sample)
    ptrs = (ctypes.c_void_p * 8)(*[c.data_ptr() for c in contribs])

    def call():
        return L.z1_owner_sum_update_noalloc(ctypes.cast(ptrs, ctypes.c_void_p), 8, n, 0.125,
                                             ctypes.c_void_p(avg.data_ptr()), ctypes.c_void_p(fsum.data_ptr()),
                                             ctypes.byref(u), _lib.stream_handle(dev))

    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode='global'):      # the process's first call of the entry point
        rc = call()
    assert rc == 0, L.z1_strerror(rc)
    want = t._call(None, dev, contribs, n, noalloc=False)
    for rep in range(3):
        for x in list(outs.values()) + [avg, fsum]:
            x.fill_(-3.0)
        flags.fill_(7)
        graph.replay()
        torch.cuda.synchronize()
        got = {{k: v.cpu().numpy().view(np.uint32).copy() for k, v in outs.items()}}
        got['avg'] = avg.view(torch.int16).cpu().numpy()
        got['sum'] = fsum.cpu().numpy().view(np.uint32)
        got['flags'] = flags.cpu().numpy()
        for k in want:
            assert np.array_equal(got[k], want[k]), (rep, k)
    torch.cuda.synchronize()
    stats0 = torch.cuda.memory_stats()
    free0 = torch.cuda.mem_get_info()[0]
    assert call() == 0
    torch.cuda.synchronize()
    stats1 = torch.cuda.memory_stats()
    free1 = torch.cuda.mem_get_info()[0]
    for k in ('allocation.all.allocated', 'segment.all.allocated', 'requested_bytes.all.allocated'):
        assert stats0.get(k) == stats1.get(k), k
    assert free0 == free1, (free0, free1)
    print('noalloc capture-first ok')
""")


def test_noalloc_first_call_under_graph_capture(pkg, dev):
    script = _CAPTURE_FIRST.format(root=ROOT, tests=os.path.join(ROOT, 'tests'))
    res = subprocess.run([sys.executable, '-c', script], capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert 'noalloc capture-first ok' in res.stdout
