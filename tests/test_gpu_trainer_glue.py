"""The trainer's per-update scalar chain (yoco/tasks/trainer_nosync.py:273-289) on the GPU: the one-launch kernel
against the oracle and against the reference's own torch expressions, the deferred NaN/Inf check, and the whole
TrainerUpdate sequence against the separate multiply_grads / clip_grad_norm / step calls."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def torch_chain(nr_t, ss_t, numer, max_norm):
    """The reference's torch ops for the same scalars, on the GPU."""
    denom = torch.where(ss_t > 0, ss_t, torch.ones_like(ss_t))
    factor = 1.0
    factor *= numer / denom
    sq = nr_t.float() ** 2
    norm = sq.sqrt()
    grad_norm = factor * norm
    if max_norm > 0.0:
        factor *= (max_norm / (grad_norm + 1e-6)).clamp_(max=1)
    finite = torch.isfinite(grad_norm).all()
    clip = torch.where(grad_norm > max_norm, grad_norm.new_tensor(100), grad_norm.new_tensor(0))
    return grad_norm, factor, finite, clip


@pytest.mark.parametrize('ss', [16384.0, 0.0, -1.0, 3.0])
@pytest.mark.parametrize('max_norm', [1.0, 1e-3, 0.0])
def test_update_scalars_kernel(pkg, dev, ss, max_norm):
    from faster_yoco_amd import ops
    rng = np.random.default_rng(int(abs(ss)) + 3)
    g = (rng.standard_normal(100_003) * 1e-2).astype(np.float32)
    gt = torch.from_numpy(g).to(dev)
    table = ops.Table([(gt, None, None, None, None, gt.numel())], dev)
    part = ops.norm_workspace(dev)
    ops.grad_sumsq(table, part)
    ss_t = torch.tensor([ss], dtype=torch.float32, device=dev)
    nr, gn, fo, cl = (torch.zeros(1, device=dev) for _ in range(4))
    flags = torch.zeros(2, dtype=torch.uint8, device=dev)
    ops.update_scalars(part, sample_size=ss_t, numer=8, factor=1.0, max_norm=max_norm, norm_out=nr,
                       grad_norm_out=gn, factor_out=fo, flags_out=flags, clip_log_out=cl)
    torch.cuda.synchronize()
    o = oracle.update_scalars(float(nr.item()) ** 2, ss, 8, 1.0, max_norm)
    assert np.float32(gn.item()) == o['grad_norm'] and np.float32(fo.item()) == o['factor']
    assert flags.tolist() == [1, 1]
    if max_norm > 0:
        assert np.float32(cl.item()) == o['clip_log']
    r_gn, r_f, r_finite, r_clip = torch_chain(nr, ss_t, 8, max_norm)
    assert np.float32(r_gn.item()) == np.float32(gn.item())
    assert np.float32(torch.as_tensor(r_f).item()) == np.float32(fo.item())
    if max_norm > 0:
        assert r_clip.item() == cl.item()
    ex = float(np.sqrt(oracle.sumsq(g)))
    assert abs(float(nr.item()) - ex) <= 1e-6 * ex


def build(dev, seed):
    from faster_yoco_amd import configs, shard as shard_mod
    sh = shard_mod.FlatShard(configs.C1_MINI_SHAPES, dev)
    rng = np.random.default_rng(seed)
    sh.p.copy_(torch.from_numpy((rng.standard_normal(sh.total) * 0.02).astype(np.float32)))
    opt = shard_mod.Zero1ShardOptimizer(sh, **HP)
    return sh, opt


def test_trainer_update_equals_separate_calls_and_defers_nan(pkg, dev):
    from faster_yoco_amd import trainer_glue
    sh_a, opt_a = build(dev, 1)
    sh_b, opt_b = build(dev, 1)
    upd = trainer_glue.TrainerUpdate(opt_a, clip_norm=1.0, numer=8)
    rng = np.random.default_rng(2)
    for step in range(4):
        g = torch.from_numpy((rng.standard_normal(sh_a.total) * 3.0).astype(np.float32)).to(dev)
        sh_a.g.copy_(g)
        sh_b.g.copy_(g)
        ss = torch.tensor([2048.0 * (step + 1)], device=dev)
        gn_a, clip_a = upd(ss)
        # the same update through the fairseq-shaped surface, with the reference's factor expression
        opt_b.multiply_grads(8 / torch.where(ss > 0, ss, torch.ones_like(ss)))
        gn_b = opt_b.clip_grad_norm(1.0)
        opt_b.step()
        torch.cuda.synchronize()
        assert gn_a.item() == gn_b.item()
        assert clip_a.item() == (100.0 if gn_b.item() > 1.0 else 0.0)
        for buf in ('p', 'm', 'v', 'p16'):
            assert torch.equal(getattr(sh_a, buf).view(torch.int16), getattr(sh_b, buf).view(torch.int16))
    # a NaN gradient: that update still runs (as in the reference); the next one raises before its step
    sh_a.g[5] = float('nan')
    upd(torch.tensor([2048.0], device=dev))
    with pytest.raises(FloatingPointError, match='gradients are Nan/Inf'):
        upd(torch.tensor([2048.0], device=dev))
    assert torch.isnan(sh_a.p).any()


def test_pending_semantics(pkg, dev):
    from faster_yoco_amd import trainer_glue
    p = trainer_glue.Pending()
    p.check(block=True)                              # not armed: nothing to do
    p.arm(torch.tensor([1, 1], dtype=torch.uint8, device=dev))
    p.check(block=True)
    p.arm(torch.tensor([1, 0], dtype=torch.uint8, device=dev))
    with pytest.raises(FloatingPointError, match='inconsistent between workers'):
        p.check(block=True)
    p.arm(torch.tensor([0, 1], dtype=torch.uint8, device=dev))
    torch.cuda.synchronize()
    with pytest.raises(FloatingPointError, match='Nan/Inf'):
        p.check(block=False)


def test_profiler_regions_carry_the_reference_names(pkg, dev):
    """trainer_nosync.py:268,273,281,288 name the phases for torch's profiler; the same names appear here."""
    from torch.profiler import ProfilerActivity, profile
    from faster_yoco_amd import shard as shard_mod, trainer_glue
    sh16 = shard_mod.FlatShard([(64, 64), (64,)], dev, grad_dtype=torch.bfloat16)
    opt = shard_mod.Zero1ShardOptimizer(sh16, **HP)
    upd = trainer_glue.TrainerUpdate(opt, clip_norm=1.0, numer=8)
    contribs = [torch.zeros(sh16.total, dtype=torch.bfloat16, device=dev) for _ in range(8)]
    with profile(activities=[ProfilerActivity.CPU]) as prof:
        opt.reduce_grads(contribs)
        upd(torch.tensor([2048.0], device=dev))
    torch.cuda.synchronize()
    names = {e.name for e in prof.events()}
    assert {'reduce-grads', 'clip-grads', 'optimizer'} <= names
