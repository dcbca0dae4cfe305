"""The step in row ranges with the BF16 exchange pipelined behind it (faster_yoco_amd.exchange; the reference
all-gathers after the whole step, yoco/tasks/zero1_fast.py:224-226).  CPU: the range splitter.  GPU: a step in
ranges is bit-identical to one launch, and every range the side stream sends holds the finished BF16 rows."""
import math

import numpy as np
import pytest
import torch

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


@pytest.mark.parametrize('k', [1, 2, 3, 4, 8, 38, 1000])
def test_even_pieces_cover_every_row_once(pkg, k):
    from faster_yoco_amd import configs, exchange
    for shapes in (configs.shapes('c2'), configs.shapes('c2r'), configs.C1_SHAPES, [(5,)], [(1,)] * 7):
        numels = [math.prod(s) for s in shapes]
        b = exchange.even_pieces(numels, k)
        assert b[0] == 0 and b[-1] == len(numels)
        assert all(x < y for x, y in zip(b, b[1:]))                  # every range holds at least one row
        assert len(b) - 1 <= max(1, min(k, len(numels)))
    numels = [math.prod(s) for s in configs.shapes('c2')]
    sizes = [sum(numels[a:c]) for a, c in zip(*(lambda b: (b, b[1:]))(exchange.even_pieces(numels, 4)))]
    assert max(sizes) < 0.35 * sum(numels)                            # roughly even at the C2 list's granularity


def shard_pair(dev, shapes, seed):
    from faster_yoco_amd import shard as shard_mod
    out = []
    for _ in range(2):
        sh = shard_mod.FlatShard(shapes, dev)
        rng = np.random.default_rng(seed)
        n = sh.total
        sh.p.copy_(torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)))
        sh.m.copy_(torch.from_numpy((rng.standard_normal(n) * 1e-4).astype(np.float32)))
        sh.v.copy_(torch.from_numpy(np.abs(rng.standard_normal(n) * 1e-8).astype(np.float32)))
        sh.g.copy_(torch.from_numpy((rng.standard_normal(n) * 3e-3).astype(np.float32)))
        opt = shard_mod.Zero1ShardOptimizer(sh, **HP)
        opt.step_count = 99
        out.append((sh, opt))
    return out


def bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


SHAPES = [(96, 64), (3, 5), (64,), (0,), (256, 33), (1000,), (7,), (64, 256)]     # an empty row among them


@pytest.mark.gpu
@pytest.mark.parametrize('pieces', [[0, 8], [0, 1, 2, 3, 4, 5, 6, 7, 8], [0, 3, 3, 4, 8], [0, 0, 5, 8]])
def test_step_in_row_ranges_matches_one_launch(pkg, dev, pieces):
    from faster_yoco_amd import exchange
    (sa, oa), (sb, ob) = shard_pair(dev, SHAPES, 1)
    remote = torch.full_like(sb.p16, float('nan'))                 # a peer's flat buffer stand-in
    sent = []

    def send(first, last):
        remote[first:last].copy_(sb.p16[first:last])
        sent.append((first, last))

    px = exchange.PipelinedExchange(sb, pieces, send)
    for _ in range(3):                                             # three steps; the factor clipped on the device
        ga, gb = oa.clip_grad_norm(1.0), ob.clip_grad_norm(1.0)
        oa.step()
        px.step(ob)
    torch.cuda.synchronize()
    assert torch.equal(bits(ga), bits(gb))
    for k in ('p', 'm', 'v', 'p16'):
        assert torch.equal(bits(getattr(sa, k)), bits(getattr(sb, k))), k
    covered = torch.zeros(sb.total, dtype=torch.bool, device=dev)
    for first, last in sent:
        covered[first:last] = True
    for o, n in zip(sb.offsets, sb.numels):
        assert bool(covered[o:o + n].all())
        assert torch.equal(bits(remote[o:o + n]), bits(sb.p16[o:o + n]))
    assert len(sent) == 3 * (len(pieces) - 1)


@pytest.mark.gpu
def test_step_in_row_ranges_rejects_bad_ranges(pkg, dev):
    from faster_yoco_amd import ops, shard as shard_mod
    (sa, oa), _ = shard_pair(dev, SHAPES, 2)
    before = sa.p.clone()
    for bad in ([1, 8], [0, 7], [0, 5, 3, 8]):
        with pytest.raises(RuntimeError, match='pieces'):
            oa.step(pieces=bad)
    assert oa.step_count == 99
    with pytest.raises(RuntimeError, match='outside'):
        ops.adam_cast_rows(sa.table, 0, 9, None, 1e-3, 0.9, 0.95, 1e-8, 1.0, 1.0, 0.0, 1)
    od = shard_mod.Zero1ShardOptimizer(sa, **HP, device_step=True)
    with pytest.raises(RuntimeError, match='device_step'):
        od.step(pieces=[0, 8])
    torch.cuda.synchronize()
    assert torch.equal(bits(sa.p), bits(before))
