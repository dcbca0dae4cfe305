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


def test_dropin_fused_adam_cast_full_size_matches_oracle_digest(pkg, dev):
    """The drop-in surface at C2's full size: FusedAdamCast called with amp_C.multi_tensor_adam's signature, as
    fairseq's FusedAdamV2.step calls it (yoco/tasks/fused_adam_cast.py:62-72), over the 38 C2 tensors allocated one
    by one (the reference's per-parameter layout) with BF16 destinations in one flat buffer.  The gradients are
    multiplied by the digest's clip factor first (fp32 products, as the reference's scale pass writes them), so
    p, m, v and the BF16 copy must give C2's digests."""
    import hashlib
    import math
    from faster_yoco_amd import configs
    from faster_yoco_amd.fused_adam_cast import FusedAdamCast
    with open(os.path.join(HERE, 'large_digests.json')) as f:
        d = json.load(f)['c2']
    h = d['hparams']
    factor = torch.tensor([int(d['factor_bits'], 16)], dtype=torch.int64).to(torch.int32).view(torch.float32)
    factor = factor.to(dev)
    shapes = configs.shapes('c2')
    flat16 = torch.empty(d['params'], dtype=torch.bfloat16, device=dev)
    tensors = {f: [] for f in ('g', 'p', 'm', 'v')}
    dest, k = {}, 0
    for s in shapes:
        n = math.prod(s)
        for f in tensors:
            t = torch.empty(n, dtype=torch.float32, device=dev)
            for i in range(0, n, 1 << 25):
                idx = torch.arange(k + i, k + min(n, i + (1 << 25)), dtype=torch.int64, device=dev)
                t[i:i + idx.numel()] = configs.hashed_values('c2', f, idx)
            tensors[f].append(t.view(s))
        tensors['g'][-1].mul_(factor)
        dest[tensors['p'][-1].data_ptr()] = flat16[k:k + n].view(s)
        k += n
    assert k == d['params']
    fa = FusedAdamCast(dest)
    noop = torch.zeros(1, dtype=torch.int32, device=dev)
    fa(2048 * 32, noop, [tensors['g'], tensors['p'], tensors['m'], tensors['v']], h['lr'], h['beta1'], h['beta2'],
       h['eps'], d['step'], 1, 1, h['weight_decay'])
    torch.cuda.synchronize()
    assert len(fa.cast) == len(shapes)
    got = {}
    for f in ('p', 'm', 'v'):
        hs = hashlib.sha256()
        for t in tensors[f]:
            hs.update(t.reshape(-1).cpu().numpy().tobytes())
        got[f] = hs.hexdigest()
    got['p16'] = digest(flat16)
    assert got == {key: d['sha256'][key] for key in ('p', 'm', 'v', 'p16')}


def test_dropin_folded_written_full_size_matches_c3_digest(pkg, dev):
    """The drop-in's default step at full size: zero1_fast.step with the fused Adam hands FusedAdamCast the BF16
    gradients to fold in (times the clip factor) and the FP32 gradient tensors to write, as the reference's scale
    pass would have written them before its Adam (yoco/tasks/zero1_fast.py:175-195, fused_adam_cast.py:75-89).
    On C3's inputs -- the owner sum of the 8 hashed contributions, its norm and clip factor -- over the 38 tensors
    as per-parameter views, p, m, v and the BF16 copy must give C3's digests, and every written FP32 gradient must
    equal torch's fp32 product of the BF16 average and the factor."""
    from faster_yoco_amd import configs, shard as shard_mod
    from faster_yoco_amd.fused_adam_cast import FusedAdamCast
    with open(os.path.join(HERE, 'large_digests.json')) as f:
        d = json.load(f)['c3']
    h = d['hparams']
    sh = shard_mod.FlatShard(configs.shapes('c3'), dev, grad_dtype=torch.bfloat16)
    assert sh.total == sh.numel == d['params']
    contribs = configs.fill_shard_hashed(sh, 'c3')
    opt = shard_mod.Zero1ShardOptimizer(sh, lr=h['lr'], betas=(h['beta1'], h['beta2']), eps=h['eps'],
                                        weight_decay=h['weight_decay'])
    opt.reduce_grads(contribs)
    del contribs
    gn = opt.clip_grad_norm(d['max_norm'])
    fac = opt._multiply_factor.reshape(1).clone()
    torch.cuda.synchronize()
    assert (hexbits(opt._norm), hexbits(gn), hexbits(fac)) == (d['norm_bits'], d['grad_norm_bits'],
                                                                d['factor_bits'])
    ps, ms, vs, g16s, p16s = (sh.views(b) for b in ('p', 'm', 'v', 'g', 'p16'))
    g32s = [torch.full(t.shape, float('nan'), dtype=torch.float32, device=dev) for t in ps]
    fa = FusedAdamCast({p.data_ptr(): q for p, q in zip(ps, p16s)})
    fa.fold, fa.fold_factor, fa.fold_writes = {p.data_ptr(): g for p, g in zip(ps, g16s)}, fac, True
    noop = torch.zeros(1, dtype=torch.int32, device=dev)
    fa(2048 * 32, noop, [g32s, ps, ms, vs], h['lr'], h['beta1'], h['beta2'], h['eps'], d['step'], 1, 1,
       h['weight_decay'])
    torch.cuda.synchronize()
    assert len(fa.cast) == len(ps)
    got = {k: digest(getattr(sh, k)) for k in ('p', 'm', 'v', 'p16')}
    got['avg16'] = digest(sh.g)
    assert got == d['sha256']
    for g16, g32 in zip(g16s, g32s):
        assert torch.equal((g16.float() * fac).view(torch.int32), g32.view(torch.int32))


def test_dropin_ce_sum_slots_full_size_matches_oracle_digest(pkg, dev):
    """The copy-engine path's owner sum at C3's full size through the drop-in of CEReduce._sum
    (yoco/models/decoder/ce_reduce.py:59-74,178-183): rank 3's own contribution in OUT, the seven peers' in the
    slot-major staging buffer (peer k < 3 in slot k, k > 3 in slot k - 1), summed in place in three phases of
    bounds; OUT must then hold C3's BF16 average."""
    from faster_yoco_amd import ce_reduce, configs
    with open(os.path.join(HERE, 'large_digests.json')) as f:
        d = json.load(f)['c3']
    G, R, W = d['params'], 3, 8
    S = torch.empty((W - 1) * G, dtype=torch.bfloat16, device=dev)
    OUT = torch.empty(G, dtype=torch.bfloat16, device=dev)
    for k in range(W):
        dst = OUT if k == R else S[(k if k < R else k - 1) * G:(k if k < R else k - 1) * G + G]
        for i in range(0, G, 1 << 25):
            idx = torch.arange(i, min(G, i + (1 << 25)), dtype=torch.int64, device=dev)
            dst[i:i + idx.numel()] = configs.hashed_values('c3', f'c{k}', idx).to(torch.bfloat16)
    assert digest(OUT[:d['prefix_elements']]) == d['input_prefix_sha256'][f'c{R}']
    for a, b in ((0, 123_456_789), (123_456_789, 123_456_789), (123_456_789, G)):
        ce_reduce.sum_slots(S, OUT, G, a, b, R, 1.0 / W, W)
    torch.cuda.synchronize()
    assert digest(OUT) == d['sha256']['avg16']
