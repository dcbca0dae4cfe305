"""Full-size updates on BASELINE.json's own input distributions, bit-exact on every element: C2 (N(0, 1e-4)
gradients, N(0, 1e-4) m, |N(0, 1e-8)| v, N(0, 0.02) masters, step 1000), C3 (the owner sum of eight N(0, 1e-4)
BF16 contributions first; the clip clamps to 1) and C5 (Student-t(2) x 1e-3 gradients with 0.1% +-1e4 outliers,
clip factor 1.5e-7) on the 430,662,912-parameter shard.  The inputs come from configs.baseline_inputs (seeded
NumPy streams, generated on the host here exactly as tests/golden/make_fixtures.py --baseline generated them for
the CPU oracle) and are copied to the device; tests/golden/baseline_digests.json holds the oracle's results: the bits
of the norm, grad_norm and clip factor, and sha256 of p, m, v, the BF16 copy and (C3) the BF16 average."""
import json
import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_gpu_digests import digest, hexbits  # noqa: E402

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def host_digest(a, n):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(a[:n]).tobytes()).hexdigest()


@pytest.mark.parametrize('name', ['c2', 'c3', 'c5'])
def test_full_size_update_on_baseline_distributions(pkg, dev, name):
    from faster_yoco_amd import configs, shard as shard_mod
    with open(os.path.join(HERE, 'baseline_digests.json')) as f:
        d = json.load(f)[name]
    x = configs.baseline_inputs(name, seed=0)
    P = d['prefix_elements']
    pre = d['input_prefix_sha256']
    for k in ('p', 'm', 'v'):
        assert host_digest(x[k], P) == pre[k], f'input {k}'
    gdt = torch.bfloat16 if name == 'c3' else torch.float32
    sh = shard_mod.FlatShard(configs.shapes(name), dev, grad_dtype=gdt)
    assert sh.total == sh.numel == d['params']           # no alignment gaps: element k sits at position k
    for k in ('p', 'm', 'v'):
        getattr(sh, k).copy_(torch.from_numpy(x.pop(k)))
    if sh.p16 is not None:
        sh.p16.copy_(sh.p)
    contribs = None
    if name == 'c3':
        for r, c in enumerate(x['contribs']):
            assert host_digest(c, P) == pre[f'c{r}'], f'input c{r}'
        contribs = [configs.to_device_bf16(c, dev) for c in x.pop('contribs')]
        sh.g.zero_()
    else:
        assert host_digest(x['g'], P) == pre['g'], 'input g'
        sh.g.copy_(torch.from_numpy(x.pop('g')))
    h = d['hparams']
    opt = shard_mod.Zero1ShardOptimizer(sh, lr=h['lr'], betas=(h['beta1'], h['beta2']), eps=h['eps'],
                                        weight_decay=h['weight_decay'])
    opt.step_count = d['step'] - 1
    if contribs is not None:
        opt.reduce_grads(contribs)
        del contribs
    gn = opt.clip_grad_norm(d['max_norm'])
    fac = opt._multiply_factor.clone()
    opt.step()
    torch.cuda.synchronize()
    assert (hexbits(opt._norm), hexbits(gn), hexbits(fac)) == (d['norm_bits'], d['grad_norm_bits'],
                                                                d['factor_bits'])
    want = d['sha256']
    got = {k: digest(getattr(sh, k)) for k in ('p', 'm', 'v', 'p16')}
    if 'avg16' in want:
        got['avg16'] = digest(sh.g)
    assert got == want
