"""The drop-in's world > 1 branches -- the all-reduce of n_r^2 in clip_grad_norm (yoco/tasks/zero1_fast.py:150-152)
and the BF16 exchange after the step: the flat-buffer all-gather (:224-226) into placed parameter views or followed
by the copy back into the parameters, or one broadcast per owner segment (YOCO_ZERO1_ALLGATHER off, :227-231) --
with a two-rank world emulated in one process: each rank has its own model copy, its own fairseq / OSS stand-ins
owning its half of the greedy partition, and zero1_fast's torch.distributed calls go to a fake that performs the
exchange between the two ranks' buffers (fp32 addition of two values commutes, so the all-reduced sum does not
depend on the order).  The steps run in two threads, one per rank, and the fake's exchange calls block like
collectives until both ranks have arrived, so each rank's copy back into its parameters follows the exchange.
Checks: both ranks get the same grad_norm and clip factor, equal to the reference's chain on the oracle's per-rank
norms; after both steps every rank holds, at every parameter, the BF16 copy of the oracle's updated master."""
import os
import sys
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from fakes import FakeFairseqOptimizer, FakeFP16Optimizer, FakeOSS  # noqa: E402

pytestmark = pytest.mark.gpu

SHAPES = [(64, 64), (256, 64), (64, 256), (64,), (33, 7), (128,)]
HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
SWITCHES = dict(ENABLED=True, ALLGATHER=True, PARAM_VIEWS=True, REDUCE_OWNER=True, ONE_PASS=True,
                SCALE_KERNEL=True, FUSED_ADAM=True, FOLD_SCALE=True)
EXCHANGES = {                                   # exchange form -> the switches that select it
    'placed_allgather': dict(ALLGATHER=True, PARAM_VIEWS=True, FOLD_SCALE=True),
    'flat_allgather_copy_back': dict(ALLGATHER=True, PARAM_VIEWS=False, FOLD_SCALE=False),
    'broadcast_copy_back': dict(ALLGATHER=False, PARAM_VIEWS=False, FOLD_SCALE=False),
}


class _Done:
    def wait(self):
        return True


class TwoRankDist:
    """The torch.distributed calls zero1_fast makes, for two ranks living in this process (self.cur = the rank
    whose code is running)."""

    def __init__(self):
        self.cur = 0                            # the running rank in the single-threaded phases
        self.tl = threading.local()             # ... and in a rank's own thread
        self.meet = threading.Barrier(2)
        self.mode = 'record'
        self.sq = {}
        self.gather = {}
        self.bcast = {}
        self.calls = []

    def rank(self):
        return getattr(self.tl, 'rank', self.cur)

    def _together(self, exchange):
        """Both ranks arrive, rank 0 performs the exchange for both (its copies go on the one stream after both
        ranks' updates), both leave."""
        self.meet.wait(timeout=60)
        if self.rank() == 0:
            exchange()
        self.meet.wait(timeout=60)

    def is_initialized(self):
        return True

    def get_world_size(self, group=None):
        return 2

    def all_reduce(self, t, group=None):
        if self.mode == 'record':
            self.sq[self.cur] = t.clone()
        else:
            t.add_(self.sq[1 - self.cur])

    def all_gather_into_tensor(self, out, inp, group=None):
        me = self.rank()
        self.calls.append('all_gather')
        seg = inp.numel()
        assert out.numel() == 2 * seg
        assert inp.data_ptr() == out.data_ptr() + me * seg * out.element_size()     # this rank's own slot
        self.gather[me] = out

        def exchange():
            for r in (0, 1):
                src = 1 - r
                self.gather[r][src * seg:(src + 1) * seg].copy_(self.gather[src][src * seg:(src + 1) * seg])
        self._together(exchange)

    def broadcast(self, buf, src, group=None, async_op=False):
        """The k-th broadcast of one rank pairs with the k-th of the other (both walk the owners in order)."""
        me = self.rank()
        self.calls.append('broadcast')
        mine = self.bcast.setdefault(me, [])
        mine.append((buf, src))
        k = len(mine) - 1

        def exchange():
            (b0, s0), (b1, s1) = self.bcast[0][k], self.bcast[1][k]
            assert s0 == s1 == src and b0.numel() == b1.numel()
            bufs = {0: b0, 1: b1}
            bufs[1 - src].copy_(bufs[src])
        self._together(exchange)
        return _Done() if async_op else None


class Model:
    def __init__(self, params):
        self.params = params

    def parameters(self):
        return iter(self.params)


@pytest.mark.parametrize('exchange', sorted(EXCHANGES))
def test_two_rank_clip_and_exchange(pkg, dev, monkeypatch, exchange):
    from faster_yoco_amd import layout, zero1_fast
    fake = TwoRankDist()
    monkeypatch.setattr(zero1_fast, 'dist', fake)
    saved = {k: getattr(zero1_fast, k) for k in SWITCHES}
    placed_before = dict(zero1_fast._PLACED)
    rng = np.random.default_rng(5)
    init = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    owner, _ = layout.greedy_partition([int(np.prod(s)) for s in SHAPES], 2)
    grads16 = [oracle.bf16_rne((rng.standard_normal(s) * 3e-2).astype(np.float32)) for s in SHAPES]
    try:
        zero1_fast.configure(**dict(SWITCHES, **EXCHANGES[exchange]))
        ranks = []
        for r in (0, 1):
            fake.cur = r
            params = [torch.nn.Parameter(torch.from_numpy(x).to(dev).to(torch.bfloat16)) for x in init]
            zero1_fast._PLACED.clear()
            if zero1_fast.PARAM_VIEWS:
                zero1_fast._place_params(Model(params))                   # views of this rank's flat buffer
            opt = FakeFP16Optimizer(params, **HP)
            mine = [p32 for p32, o in zip(opt.fp32_params, owner) if o == r]
            oss = FakeOSS(mine, **HP)                                      # OSS: this rank's partition only
            oss._param_to_rank = {p32: o for p32, o in zip(opt.fp32_params, owner)}
            oss.rank, oss.world_size, oss.group, oss._local_to_global_rank = r, 2, 'group', [0, 1]
            opt.fp32_optimizer = FakeFairseqOptimizer(oss)
            assert zero1_fast._plan(opt).placed == zero1_fast.PARAM_VIEWS  # this rank's placement is captured
            for p, g, o in zip(params, grads16, owner):                   # the owner holds the reduced grads
                p.grad = (torch.from_numpy(g.view(np.int16)).to(dev).view(torch.bfloat16).view(p.shape)
                          if o == r else None)
            ranks.append((params, opt))

        # the all-reduce: record both ranks' n_r^2, then run each rank's clip with its partner's added
        for r, (_, opt) in enumerate(ranks):
            fake.cur = r
            zero1_fast.clip_grad_norm(opt, 1.0)
            opt._multiply_factor = 1.0
        fake.mode = 'sum'
        out = []
        for r, (_, opt) in enumerate(ranks):
            fake.cur = r
            gn = zero1_fast.clip_grad_norm(opt, 1.0)
            out.append((gn.clone(), opt._multiply_factor.clone()))
        torch.cuda.synchronize()
        (gn0, f0), (gn1, f1) = out
        assert torch.equal(gn0.view(torch.int32), gn1.view(torch.int32))
        assert torch.equal(f0.view(torch.int32), f1.view(torch.int32))
        # the reference's chain (zero1_fast.py:150-160) on the oracle's per-rank norms
        sq = np.float32(0.0)
        for r in (0, 1):
            ss = sum(oracle.sumsq(g) for g, o in zip(grads16, owner) if o == r)
            nr = np.float32(oracle.norm_clip(ss, 1.0, 0.0)[0])
            sq = np.float32(sq + np.float32(nr * nr))
        norm = np.float32(np.sqrt(sq))
        gnv = np.float32(gn0.item())
        assert oracle.ulp_diff_f32(gnv, norm) <= 1                      # torch's fp32 sqrt on the device
        o_gn, o_f = oracle.clip_factor(gnv, 1.0, 1.0)                   # the chain from the device's norm
        assert (np.float32(o_gn).view(np.uint32), np.float32(o_f).view(np.uint32)) == \
            (gnv.view(np.uint32), np.float32(f0.item()).view(np.uint32))

        # the steps: each rank updates its half in its own thread, the exchange meets in the middle
        def run(r):
            fake.tl.rank = r
            zero1_fast.step(ranks[r][1])
        with ThreadPoolExecutor(2) as pool:
            for f in [pool.submit(run, r) for r in (0, 1)]:
                f.result(timeout=120)
        torch.cuda.synchronize()
        assert set(fake.calls) == {'all_gather' if zero1_fast.ALLGATHER else 'broadcast'}
        fac = float(f0.item())
        for i, (x, g) in enumerate(zip(init, grads16)):
            x = oracle.bf16_to_f32(oracle.bf16_rne(x))                     # the masters start from the bf16 model
            po, _, _, p16 = oracle.adam_cast(g.reshape(-1), x.reshape(-1), np.zeros(x.size, np.float32),
                                             np.zeros(x.size, np.float32), lr=HP['lr'], beta1=HP['betas'][0],
                                             beta2=HP['betas'][1], eps=HP['eps'], weight_decay=HP['weight_decay'],
                                             step=1, mode=1, factor=fac)
            for r, (params, opt) in enumerate(ranks):
                got = params[i].detach().reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
                assert np.array_equal(got, p16), (r, i, owner[i])
                if owner[i] == r:
                    p32 = opt.fp32_params[i].detach().reshape(-1).cpu().numpy()
                    assert np.array_equal(p32.view(np.uint32), po.view(np.uint32)), (r, i)
    finally:
        for k, v in saved.items():
            setattr(zero1_fast, k, v)
        zero1_fast._PLACED.clear()
        zero1_fast._PLACED.update(placed_before)
