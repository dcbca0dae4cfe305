"""Independent updates on concurrent streams: two shards, each with its own table and workspace, updated for three
steps with every launch of shard A on one stream and of shard B on another (default priority), interleaved by
the host -- the results are bit-identical to the same updates run one after the other on one stream.  One shard
takes the norm path, the other the owner-sum path, so both kinds of launch overlap."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def make(dev, shapes, grad_dtype, seed):
    from faster_yoco_amd import shard as shard_mod
    sh = shard_mod.FlatShard(shapes, dev, grad_dtype=grad_dtype)
    rng = np.random.default_rng(seed)
    n = sh.total
    sh.p.copy_(torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)))
    sh.g.copy_(torch.from_numpy((rng.standard_normal(n) * 3e-3).astype(np.float32)).to(grad_dtype))
    opt = shard_mod.Zero1ShardOptimizer(sh, **HP)
    contribs = None
    if grad_dtype == torch.bfloat16:
        contribs = [torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(dev).to(torch.bfloat16)
                    for _ in range(8)]
    return sh, opt, contribs


def state(sh):
    return {k: getattr(sh, k).clone() for k in ('g', 'p', 'm', 'v', 'p16')}


def restore(sh, opt, snap):
    for k, t in snap.items():
        getattr(sh, k).copy_(t)
    opt.step_count = 0
    opt._multiply_factor = 1.0


def one_update(opt, contribs):
    if contribs is not None:
        opt.reduce_grads(contribs)
    return opt.update(1.0)


def test_two_shards_on_two_streams_match_sequential(pkg, dev):
    from faster_yoco_amd import configs
    a = make(dev, configs.C1_SHAPES, torch.float32, 21)
    b = make(dev, configs.C1_SHAPES, torch.bfloat16, 22)
    snaps = [state(a[0]), state(b[0])]

    # sequential reference on the current stream
    ref_gn = []
    for _ in range(3):
        ref_gn.append([one_update(a[1], a[2]).clone(), one_update(b[1], b[2]).clone()])
    torch.cuda.synchronize()
    ref = [state(a[0]), state(b[0])]

    restore(a[0], a[1], snaps[0])
    restore(b[0], b[1], snaps[1])
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got_gn = []
    for _ in range(3):
        row = []
        for (sh, opt, contribs), s in zip((a, b), streams):
            with torch.cuda.stream(s):
                row.append(one_update(opt, contribs).clone())
        got_gn.append(row)
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for (sh, _, _), r in zip((a, b), ref):
        for k in ('p', 'm', 'v', 'p16'):
            t, e = getattr(sh, k), r[k]
            bits = torch.int16 if t.dtype == torch.bfloat16 else torch.int32
            assert torch.equal(t.view(bits), e.view(bits)), k
    for g_row, r_row in zip(got_gn, ref_gn):
        for g, r in zip(g_row, r_row):
            assert torch.equal(g.view(torch.int32), r.view(torch.int32))
