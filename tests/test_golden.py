"""Committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py from the CPU oracle).

CPU: the oracle still reproduces every fixture bit for bit (a regression pin on the oracle itself).
GPU: the HIP path reproduces them -- owner sum, Adam m / v / master and the BF16 copy bit-exact given the
fixture's clip factor, the norm within 1 fp32 ulp of the fixture's, the clip chain bit-exact given the GPU norm.
"""
import glob
import os

import numpy as np
import pytest
import torch

import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')
FIXTURES = sorted(glob.glob(os.path.join(HERE, '*.npz')))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def hp(f):
    lr, b1, b2, eps, wd, mn = (float(x) for x in f['hp'])
    return dict(lr=lr, beta1=b1, beta2=b2, eps=eps, weight_decay=wd), mn


def test_fixtures_present():
    names = {os.path.basename(p) for p in FIXTURES}
    assert {'c1_mini.npz', 'c2_mini.npz', 'c3_mini.npz', 'c5_mini.npz'} <= names


@pytest.mark.parametrize('path', FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_oracle_reproduces_fixture(path):
    f = load(path)
    h, mn = hp(f)
    if 'contribs' in f:
        avg, s = oracle.owner_sum(list(f['contribs']), want_sum=True)
        assert np.array_equal(avg, f['avg16']) and np.array_equal(s.view(np.uint32), f['sum32'].view(np.uint32))
        g = avg
    else:
        g = f['g']
    nr, gn, fac = oracle.norm_clip(oracle.sumsq(g), 1.0, mn)
    assert (nr, gn, fac) == (f['norm'], f['grad_norm'], f['factor'])
    po, mo, vo, p16 = oracle.adam_cast(g, f['p'], f['m'], f['v'], step=int(f['step']), factor=float(f['factor']), **h)
    for a, b in ((po, f['p_out']), (mo, f['m_out']), (vo, f['v_out'])):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(p16, f['p16_out'])


@pytest.mark.gpu
@pytest.mark.parametrize('path', FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_gpu_reproduces_fixture(pkg, dev, path):
    from faster_yoco_amd import configs, ops
    f = load(path)
    h, mn = hp(f)
    sizes = [int(x) for x in f['sizes']]
    n = sum(sizes)
    part = ops.norm_workspace(dev, n)
    if 'contribs' in f:
        cs = [configs.to_device_bf16(c, dev) for c in f['contribs']]
        g = torch.empty(n, dtype=torch.bfloat16, device=dev)
        ops.owner_sum(cs, g, 1.0 / 8, partials=part)
        torch.cuda.synchronize()
        assert np.array_equal(configs.bf16_bits(g), f['avg16'])
    else:
        g = torch.from_numpy(f['g']).to(dev)
    p = torch.from_numpy(f['p']).to(dev)
    m = torch.from_numpy(f['m']).to(dev)
    v = torch.from_numpy(f['v']).to(dev)
    p16 = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    rows, off = [], 0
    for s in sizes:
        sl = slice(off, off + s)
        rows.append((g[sl], p[sl], m[sl], v[sl], p16[sl], s))
        off += s
    table = ops.Table(rows, dev)
    if 'contribs' not in f:
        ops.grad_sumsq(table, part)
    nr = torch.zeros(1, device=dev)
    gn = torch.zeros(1, device=dev)
    fo = torch.zeros(1, device=dev)
    ops.norm_clip(part, factor=1.0, norm_out=nr, grad_norm_out=gn, factor_out=fo, max_norm=mn)
    torch.cuda.synchronize()
    assert oracle.ulp_diff_f32(np.float32(nr.item()), f['norm']) <= 1
    _, gn_ref, fo_ref = oracle.norm_clip(float(nr.item()) ** 2, 1.0, mn)
    assert np.float32(gn.item()) == gn_ref and np.float32(fo.item()) == fo_ref
    fac = torch.tensor([float(f['factor'])], dtype=torch.float32, device=dev)
    bc1, bc2 = ops.bias_corrections(h['beta1'], h['beta2'], int(f['step']))
    ops.adam_cast(table, fac, h['lr'], h['beta1'], h['beta2'], h['eps'], bc1, bc2, h['weight_decay'], 1)
    torch.cuda.synchronize()
    for t, ref in ((p, f['p_out']), (m, f['m_out']), (v, f['v_out'])):
        assert np.array_equal(t.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(configs.bf16_bits(p16), f['p16_out'])


def _digest_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location('make_fixtures', os.path.join(HERE, 'make_fixtures.py'))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _committed_digest():
    import json
    with open(os.path.join(HERE, 'c1_full_digest.json')) as f:
        return json.load(f)


def test_oracle_reproduces_c1_full_digest(pkg):
    """The full C1 update (9,438,208 params) through the oracle still gives the committed digests."""
    assert _digest_module().c1_full_digest() == _committed_digest()


@pytest.mark.gpu
def test_gpu_c1_full_update_matches_digest(pkg, dev):
    """The full C1 update through the fairseq-shaped optimizer on the GPU: norm, grad_norm and clip factor bits,
    and the sha256 of p, m, v and the BF16 copy, equal to the oracle's committed digest."""
    import hashlib
    from faster_yoco_amd import configs, shard as shard_mod
    d = _committed_digest()
    shapes = [tuple(s) for s in d['shapes']]
    assert shapes == [tuple(s) for s in configs.C1_SHAPES]
    x = configs.host_inputs(d['params'], 'c1', seed=d['seed'])
    sh = shard_mod.FlatShard(shapes, dev)
    start = 0
    for off, n in zip(sh.offsets, sh.numels):
        for name in ('g', 'p', 'm', 'v'):
            getattr(sh, name)[off:off + n].copy_(torch.from_numpy(x[name][start:start + n]))
        start += n
    h = d['hparams']
    opt = shard_mod.Zero1ShardOptimizer(sh, lr=h['lr'], betas=(h['beta1'], h['beta2']), eps=h['eps'],
                                        weight_decay=h['weight_decay'])
    opt.step_count = d['step'] - 1
    gn = opt.clip_grad_norm(d['max_norm'])
    fac = opt._multiply_factor.clone()
    opt.step()
    torch.cuda.synchronize()
    hexbits = lambda t: '0x%08x' % int(t.reshape(-1)[0].view(torch.int32).item() & 0xffffffff)
    assert hexbits(opt._norm) == d['norm_bits']
    assert hexbits(gn) == d['grad_norm_bits']
    assert hexbits(fac) == d['factor_bits']

    def flat(t):
        return torch.cat([t[o:o + n] for o, n in zip(sh.offsets, sh.numels)]).cpu().numpy()

    got = {k: hashlib.sha256(flat(getattr(sh, k)).tobytes()).hexdigest() for k in ('p', 'm', 'v')}
    got['p16'] = hashlib.sha256(flat(sh.p16.view(torch.int16)).tobytes()).hexdigest()
    assert got == d['sha256']


def test_hashed_inputs_match_large_digest_prefixes(pkg):
    """The hashed input generator (NumPy and torch on the CPU, bit for bit alike) still gives the input prefixes the
    large digests were made from."""
    import hashlib
    import json
    from faster_yoco_amd import configs
    with open(os.path.join(HERE, 'large_digests.json')) as f:
        digests = json.load(f)
    for name, d in digests.items():
        P = d['prefix_elements']
        idx = np.arange(P, dtype=np.int64)
        for field, want in d['input_prefix_sha256'].items():
            a = configs.hashed_values(name, field, idx)
            b = configs.hashed_values(name, field, torch.from_numpy(idx)).numpy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name, field)
            if field.startswith('c'):
                a = (a.view(np.uint32) >> 16).astype(np.uint16)
            assert hashlib.sha256(a.tobytes()).hexdigest() == want, (name, field)
