"""Maximum sizes: one tensor of 2^31 + 777 elements, past every 32-bit index.  The norm of a constant gradient
against its closed form (N * 2^-20 exactly in FP64); Adam + BF16 and the owner sum on hashed inputs
(configs.hashed_values) against the oracle on windows at the start, across element 2^31 and at the end; the owner
sum's fused norm against a float64 sum of the average.  About 39 GB of device memory per test."""
import math

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

N = 2 ** 31 + 777
WINDOWS = [(0, 4096), (2 ** 31 - 2048, 2 ** 31 + 512), (N - 4096, N)]     # the middle one across 2^31
HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16) if t.dtype == torch.bfloat16 else \
        t.cpu().numpy().view(np.uint32)


def test_norm_and_adam_on_a_row_past_int32(pkg, dev):
    from faster_yoco_amd import configs, shard as shard_mod
    sh = shard_mod.FlatShard([(N,)], dev)
    opt = shard_mod.Zero1ShardOptimizer(sh, **HP)
    try:
        sh.g.fill_(2.0 ** -10)
        opt.clip_grad_norm(0.0)                                    # no clipping: the norm alone
        torch.cuda.synchronize()
        want = np.float32(math.sqrt(N) * 2.0 ** -10)              # sqrt of the exact sum N * 2^-20
        assert oracle.ulp_diff_f32(np.float32(opt._norm.item()), want) <= 1

        configs.fill_shard_hashed(sh, 'c2')
        opt.step_count = 999
        opt._multiply_factor = 0.5
        opt.step()
        torch.cuda.synchronize()
        for lo, hi in WINDOWS:
            idx = np.arange(lo, hi, dtype=np.int64)
            g, p, m, v = (configs.hashed_values('c2', f, idx) for f in ('g', 'p', 'm', 'v'))
            po, mo, vo, p16 = oracle.adam_cast(g, p, m, v, lr=HP['lr'], beta1=HP['betas'][0], beta2=HP['betas'][1],
                                               eps=HP['eps'], weight_decay=HP['weight_decay'], step=1000, mode=1,
                                               factor=0.5)
            assert np.array_equal(bits(sh.p[lo:hi]), po.view(np.uint32)), (lo, 'p')
            assert np.array_equal(bits(sh.m[lo:hi]), mo.view(np.uint32)), (lo, 'm')
            assert np.array_equal(bits(sh.v[lo:hi]), vo.view(np.uint32)), (lo, 'v')
            assert np.array_equal(bits(sh.p16[lo:hi]), p16), (lo, 'p16')
    finally:
        del sh, opt
        torch.cuda.empty_cache()


def test_owner_sum_past_int32(pkg, dev):
    from faster_yoco_amd import configs, ops
    contribs = [torch.empty(N, dtype=torch.bfloat16, device=dev) for _ in range(8)]
    out = torch.empty(N, dtype=torch.bfloat16, device=dev)
    try:
        for i in range(0, N, 1 << 26):
            idx = torch.arange(i, min(N, i + (1 << 26)), dtype=torch.int64, device=dev)
            for k, c in enumerate(contribs):
                c[i:i + idx.numel()] = configs.hashed_values('c3', f'c{k}', idx).to(torch.bfloat16)
        partials = ops.norm_workspace(dev, N)
        norm = torch.empty(1, dtype=torch.float32, device=dev)
        ops.owner_sum(contribs, out, 0.125, partials=partials)
        ops.norm_clip(partials, norm_out=norm)
        torch.cuda.synchronize()
        for lo, hi in WINDOWS:
            idx = np.arange(lo, hi, dtype=np.int64)
            cs = [(configs.hashed_values('c3', f'c{k}', idx).view(np.uint32) >> 16).astype(np.uint16)
                  for k in range(8)]
            assert np.array_equal(bits(out[lo:hi]), oracle.owner_sum(cs)), lo
        ss = 0.0
        for i in range(0, N, 1 << 27):
            ss += float((out[i:i + (1 << 27)].double() ** 2).sum().item())
        assert abs(float(norm.item()) - math.sqrt(ss)) <= 1e-6 * math.sqrt(ss)
    finally:
        del contribs, out
        torch.cuda.empty_cache()
