"""Full-size updates bit-exact on every element: C2, C3 (owner sum of 8 BF16 contributions first) and C5 (values
over 24 binades, 0.1% outliers) on the 430,662,912-parameter shard, and C4 (the unsharded 3,445,303,296-parameter
update, 304 tensors, 62 GB resident), and the same two on YOCO-3B's real tensors (C2R: rank 0's 9-tensor shard
of 443,357,184 parameters under the 8-rank greedy partition; C4R: all 240 tensors), with inputs generated on the
device by
configs.hashed_values -- which NumPy computes bit for bit alike -- checked against tests/golden/large_digests.json,
the CPU oracle's results on the same inputs (tests/golden/make_fixtures.py --large): the bits of the norm,
grad_norm and clip factor, and sha256 of p, m, v, the BF16 copy and (C3) the BF16 average."""
import hashlib
import json
import os

import pytest
import torch

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def digest(t, chunk=1 << 26):
    """sha256 of a flat device tensor's bytes, copied to the host in chunks (bf16 as its 16-bit patterns)."""
    h = hashlib.sha256()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    for i in range(0, t.numel(), chunk):
        h.update(t[i:i + chunk].cpu().numpy().tobytes())
    return h.hexdigest()


def hexbits(t):
    return '0x%08x' % (int(t.reshape(-1)[0].view(torch.int32).item()) & 0xffffffff)


@pytest.mark.parametrize('name', ['c2', 'c3', 'c5', 'c4', 'c2r', 'c4r'])
def test_full_size_update_matches_oracle_digest(pkg, dev, name):
    from faster_yoco_amd import configs, shard as shard_mod
    with open(os.path.join(HERE, 'large_digests.json')) as f:
        d = json.load(f)[name]
    gdt = torch.bfloat16 if name == 'c3' else torch.float32
    sh = shard_mod.FlatShard(configs.shapes(name), dev, grad_dtype=gdt)
    assert sh.total == sh.numel == d['params']           # no alignment gaps: element k sits at position k
    contribs = configs.fill_shard_hashed(sh, name)
    P = d['prefix_elements']
    pre = d['input_prefix_sha256']
    for f in ('p', 'm', 'v'):
        assert digest(getattr(sh, f)[:P]) == pre[f], f'input {f}'
    if contribs is not None:
        for r, c in enumerate(contribs):
            assert digest(c[:P]) == pre[f'c{r}'], f'input c{r}'
    else:
        assert digest(sh.g[:P]) == pre['g'], 'input g'
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
