"""Parity at the benchmark sizes (C2 431M shard, C3 8-contribution owner reduce, C4 3.45B unsharded, C5 heavy tails).

At these sizes the oracle checks what it can in seconds:
  * Adam / BF16: bit-exact against the oracle on ~1M sampled elements (plus the first and last elements of every
    tensor), using the GPU's own clip factor (Adam is elementwise, so a sample is an exact check of those elements);
  * owner sum (C3): bit-exact on the same samples, from the sampled contributions;
  * norm: within 1 fp32 ulp (and 1e-6 relative) of a float64 sum of squares computed on the device by torch, the
    clip chain bit-exact from the GPU's norm, the norm bit-identical when recomputed, the fused owner-sum norm
    equal to the standalone norm of the same average;
  * run-to-run: the whole update repeated from the same seeded state gives identical integer checksums.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)


def sample_index(shard, k, seed):
    rng = np.random.default_rng(seed)
    parts = []
    for o, n in zip(shard.offsets, shard.numels):
        parts.append(o + np.arange(min(n, 64)))
        parts.append(o + n - 1 - np.arange(min(n, 64)))
    total = shard.numel
    # sample positions proportionally inside the tensors (no alignment gaps)
    pos = np.sort(rng.integers(0, total, k))
    starts = np.cumsum([0] + shard.numels[:-1])
    t = np.searchsorted(starts, pos, side='right') - 1
    parts.append(np.asarray(shard.offsets)[t] + (pos - starts[t]))
    return np.unique(np.concatenate(parts)).astype(np.int64)


def take(t, idx_dev):
    return t.index_select(0, idx_dev).cpu()


def f32bits(t):
    return t.numpy().view(np.uint32) if torch.is_tensor(t) else t.view(np.uint32)


def exact_norm(g, chunk=1 << 27):
    s = torch.zeros((), dtype=torch.float64, device=g.device)
    for i in range(0, g.numel(), chunk):
        x = g[i:i + chunk].double()
        s += torch.dot(x, x)
    return float(torch.sqrt(s).item())


def checksum(*ts):
    out = []
    for t in ts:
        w = t.view(torch.int16).to(torch.int64) if t.dtype == torch.bfloat16 else t.view(torch.int32).to(torch.int64)
        pos = torch.arange(w.numel(), device=w.device, dtype=torch.int64) % 1000003
        out.append((int(w.sum().item()), int((w * pos).sum().item())))
    return out


def build(cfg, grad_dtype=torch.float32, seed=0):
    from faster_yoco_amd import configs, shard as shard_mod
    dev = torch.device('cuda:0')
    sh = shard_mod.FlatShard(configs.shapes(cfg), dev, grad_dtype=grad_dtype)
    contribs = configs.fill_shard(sh, cfg, seed=seed)
    opt = shard_mod.Zero1ShardOptimizer(sh, lr=HP['lr'], betas=(HP['beta1'], HP['beta2']), eps=HP['eps'],
                                        weight_decay=HP['weight_decay'])
    opt.step_count = configs.CONFIGS[cfg]['step'] - 1
    return sh, opt, contribs


def check_update(sh, opt, idx, g_before, p_before, m_before, v_before, g_is_bf16=False, fused_norm=False):
    """One clip + step on the shard; checks norm, chain and sampled Adam outputs."""
    exact = exact_norm(sh.g)
    gn = opt.clip_grad_norm(1.0)
    fac = float(opt._multiply_factor.item())
    nr = np.float32(opt._norm.item())
    assert oracle.ulp_diff_f32(nr, np.float32(exact)) <= 1 and abs(float(nr) - exact) <= 1e-6 * exact
    _, gn_ref, fac_ref = oracle.norm_clip(float(nr) ** 2, 1.0, 1.0)
    assert np.float32(gn.item()) == gn_ref and np.float32(fac) == fac_ref
    opt.step()
    torch.cuda.synchronize()
    idx_dev = torch.from_numpy(idx).to(sh.device)
    g_np = g_before.view(torch.int16).numpy().view(np.uint16) if g_is_bf16 else g_before.numpy()
    po, mo, vo, p16 = oracle.adam_cast(g_np, p_before.numpy(), m_before.numpy(), v_before.numpy(),
                                       step=opt.step_count, factor=fac, **HP)
    assert np.array_equal(f32bits(take(sh.m, idx_dev)), f32bits(mo))
    assert np.array_equal(f32bits(take(sh.v, idx_dev)), f32bits(vo))
    assert np.array_equal(f32bits(take(sh.p, idx_dev)), f32bits(po))
    assert np.array_equal(take(sh.p16, idx_dev).view(torch.int16).numpy().view(np.uint16), p16)
    # the norm recomputed on the unchanged gradient is bit-identical (within 1 ulp when the first one came from
    # the owner sum's fused partials, a different fixed decomposition)
    opt.clip_grad_norm(0.0)
    assert oracle.ulp_diff_f32(np.float32(opt._norm.item()), nr) <= (1 if fused_norm else 0)
    opt._multiply_factor = 1.0
    return fac


@pytest.mark.parametrize('cfg', ['c2', 'c5'])
def test_full_shard_update(pkg, cfg):
    sh, opt, _ = build(cfg)
    idx = sample_index(sh, 1 << 20, seed=1)
    idx_dev = torch.from_numpy(idx).to(sh.device)
    before = [take(t, idx_dev) for t in (sh.g, sh.p, sh.m, sh.v)]
    fac = check_update(sh, opt, idx, *before)
    if cfg == 'c5':
        assert fac < 1e-5                   # heavy tails: the clip is active and strong
    else:
        assert 0.3 < fac < 0.7
    del sh, opt
    torch.cuda.empty_cache()


def test_full_shard_run_to_run_identical(pkg):
    sums = []
    for _ in range(2):
        sh, opt, _ = build('c2', seed=7)
        opt.clip_grad_norm(1.0)
        opt.step()
        torch.cuda.synchronize()
        sums.append(checksum(sh.p, sh.m, sh.v, sh.p16))
        del sh, opt
        torch.cuda.empty_cache()
    assert sums[0] == sums[1]


def test_owner_reduce_full_shard(pkg):
    from faster_yoco_amd import ops
    sh, opt, contribs = build('c3', grad_dtype=torch.bfloat16)
    idx = sample_index(sh, 1 << 20, seed=3)
    idx_dev = torch.from_numpy(idx).to(sh.device)
    c_s = [take(c, idx_dev).view(torch.int16).numpy().view(np.uint16) for c in contribs]
    before = [take(t, idx_dev) for t in (sh.p, sh.m, sh.v)]
    opt.reduce_grads(contribs)
    torch.cuda.synchronize()
    avg_s = take(sh.g, idx_dev)
    assert np.array_equal(avg_s.view(torch.int16).numpy().view(np.uint16), oracle.owner_sum(c_s))
    # the norm fused into the owner sum equals the standalone norm of the same average
    fused = opt._partials[:ops.Z1_NORM_PARTIALS].clone()
    alone = ops.norm_workspace(sh.device)
    ops.grad_sumsq(sh.table, alone)
    n1 = torch.zeros(1, device=sh.device)
    n2 = torch.zeros(1, device=sh.device)
    ops.norm_clip(fused, norm_out=n1)
    ops.norm_clip(alone, norm_out=n2)
    assert oracle.ulp_diff_f32(np.float32(n1.item()), np.float32(n2.item())) <= 1
    fac = check_update(sh, opt, idx, avg_s, *before, g_is_bf16=True, fused_norm=True)
    assert fac == 1.0                       # E|avg| ~ 0.73 < max_norm: the coefficient clamps to 1
    del sh, opt, contribs
    torch.cuda.empty_cache()


def test_unsharded_full_model_update(pkg):
    sh, opt, _ = build('c4')
    assert len(sh.numels) == 304 and sh.numel == 3_445_303_296
    idx = sample_index(sh, 1 << 20, seed=4)
    idx_dev = torch.from_numpy(idx).to(sh.device)
    before = [take(t, idx_dev) for t in (sh.g, sh.p, sh.m, sh.v)]
    fac = check_update(sh, opt, idx, *before)
    assert 0.1 < fac < 0.3
    del sh, opt
    torch.cuda.empty_cache()
