"""The reference's surfaces driven as its trainer drives them, on the GPU, checked against the oracle:
FusedAdamCast through FusedAdamV2.step's multi_tensor_adam call, zero1_fast's clip_grad_norm / step / zero_grad
installed on fairseq's mixin (switch combinations), and CEReduce._sum."""
import os
import sys

import numpy as np
import pytest
import torch

import oracle

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import fakes  # noqa: E402

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
SHAPES = [(96, 64), (256, 33), (3072,), (7,), (64, 256)]


def bits(t):
    a = t.detach().cpu()
    return a.view(torch.int16).numpy().view(np.uint16) if a.dtype == torch.bfloat16 else a.numpy().view(np.uint32)


def bf16_params(dev, seed):
    g = torch.Generator(device='cpu').manual_seed(seed)
    return [torch.nn.Parameter((torch.randn(s, generator=g) * 0.02).to(torch.bfloat16).to(dev)) for s in SHAPES]


def set_grads(params, seed, scale=1e-2):
    g = torch.Generator(device='cpu').manual_seed(seed)
    for p in params:
        p.grad = (torch.randn(p.shape, generator=g) * scale).to(torch.bfloat16).to(p.device)


# ----------------------------------------------------------------------------------------- FusedAdamCast
def test_fused_adam_cast_through_fused_adam_v2(pkg, dev):
    from faster_yoco_amd.fused_adam_cast import FusedAdamCast
    rng = np.random.default_rng(0)
    p32 = [torch.nn.Parameter(torch.from_numpy((rng.standard_normal(s) * 0.02).astype(np.float32)).to(dev))
           for s in SHAPES]
    flat16 = torch.zeros(sum(p.numel() for p in p32), dtype=torch.bfloat16, device=dev)
    views, off = [], 0
    for p in p32:
        views.append(flat16[off:off + p.numel()].view_as(p))
        off += p.numel()
    dest = {p.data_ptr(): v for p, v in zip(p32[:-1], views[:-1])}        # the last master has no bf16 copy
    opt = fakes.FakeFusedAdamV2(p32, lr=HP['lr'], betas=(HP['beta1'], HP['beta2']), eps=HP['eps'],
                                weight_decay=HP['weight_decay'])
    fa = opt.multi_tensor_adam = FusedAdamCast(dest)
    state = [(p.detach().cpu().numpy().ravel().copy(), np.zeros(p.numel(), np.float32),
              np.zeros(p.numel(), np.float32)) for p in p32]
    for step in (1, 2, 3):
        gs = [(rng.standard_normal(p.numel()) * 1e-3).astype(np.float32) for p in p32]
        for p, g in zip(p32, gs):
            p.grad = torch.from_numpy(g.reshape(p.shape)).to(dev)
        opt.step()
        torch.cuda.synchronize()
        assert fa.cast == {p.data_ptr() for p in p32[:-1]}
        fa.cast.clear()
        for i, (p, g) in enumerate(zip(p32, gs)):
            po, mo, vo, p16 = oracle.adam_cast(g, *state[i], step=step, **HP)
            st = opt.state[p]
            assert np.array_equal(bits(p).ravel(), po.view(np.uint32))
            assert np.array_equal(bits(st['exp_avg']).ravel(), mo.view(np.uint32))
            assert np.array_equal(bits(st['exp_avg_sq']).ravel(), vo.view(np.uint32))
            if i < len(p32) - 1:
                assert np.array_equal(bits(views[i]).ravel(), p16)
            state[i] = (po, mo, vo)
    assert not bits(views[-1]).any()                                         # untouched


def test_fused_adam_cast_errors(pkg, dev):
    from faster_yoco_amd.fused_adam_cast import FusedAdamCast
    fa = FusedAdamCast({})
    x = torch.zeros(8, 8, device=dev)
    with pytest.raises(RuntimeError, match='expected contiguous fp32 tensors'):
        fa(0, None, [[x.t()], [x], [x], [x]], 1e-3, 0.9, 0.95, 1e-8, 1, 1, 1, 0.0)
    with pytest.raises(RuntimeError, match='expected contiguous fp32 tensors'):
        fa(0, None, [[x.half()], [x], [x], [x]], 1e-3, 0.9, 0.95, 1e-8, 1, 1, 1, 0.0)
    fa = FusedAdamCast({x.data_ptr(): torch.zeros(64, device=dev)})
    with pytest.raises(RuntimeError, match='bf16 destination'):
        fa(0, None, [[x], [x], [x.clone()], [x.clone()]], 1e-3, 0.9, 0.95, 1e-8, 1, 1, 1, 0.0)
    # a list of masters seen before reuses its plan; the operator still checks every tensor of the call
    fa = FusedAdamCast({})
    m, v = x.clone(), x.clone()
    fa(0, None, [[x.clone()], [x], [m], [v]], 1e-3, 0.9, 0.95, 1e-8, 1, 1, 1, 0.0)
    with pytest.raises(RuntimeError, match='expected contiguous fp32 tensors'):
        fa(0, None, [[x.t()], [x], [m], [v]], 1e-3, 0.9, 0.95, 1e-8, 2, 1, 1, 0.0)
    with pytest.raises(RuntimeError, match='row 0 has 32 elements, the table 64'):
        fa(0, None, [[x.clone()], [x], [m[:4]], [v]], 1e-3, 0.9, 0.95, 1e-8, 2, 1, 1, 0.0)
    fa(0, None, [[], [], [], []], 1e-3, 0.9, 0.95, 1e-8, 2, 1, 1, 0.0)          # empty lists: nothing to do


def test_fused_adam_cast_plans_outlive_the_table_cache(pkg, dev):
    """More table signatures than the table cache holds (5 parameter lists, each with folded and unfolded rows: 10
    tables, the cache keeps 8), cycled twice through FusedAdamCast's plan cache: a plan keeps its tables alive after
    the cache evicted them, and every call matches the oracle bit for bit."""
    from faster_yoco_amd.fused_adam_cast import FusedAdamCast
    fa = FusedAdamCast({})
    factor = torch.full((1,), 0.5, dtype=torch.float32, device=dev)
    rng = np.random.default_rng(17)
    lists = []
    for k in range(5):
        rows = []
        for n in (64 * (k + 1) + 3, 40 + 7 * k):
            g16 = oracle.bf16_rne((rng.standard_normal(n) * 1e-3).astype(np.float32))
            g32 = (rng.standard_normal(n) * 1e-3).astype(np.float32)
            p = (rng.standard_normal(n) * 0.02).astype(np.float32)
            rows.append({'g16': g16, 'g32': g32, 'p': p, 'm': np.zeros(n, np.float32), 'v': np.zeros(n, np.float32),
                         't': [torch.from_numpy(x).to(dev) for x in (g32, p, np.zeros(n, np.float32),
                                                                      np.zeros(n, np.float32))],
                         'g16t': torch.from_numpy(g16.view(np.int16)).to(dev).view(torch.bfloat16)})
        lists.append(rows)
    for rnd in range(2):
        for rows in lists:
            step = rnd + 1
            fa.fold = {rows[0]['t'][1].data_ptr(): rows[0]['g16t']}
            fa.fold_factor, fa.fold_writes = factor, False
            fa(0, None, [[r['t'][k] for r in rows] for k in range(4)], HP['lr'], HP['beta1'], HP['beta2'],
               HP['eps'], step, 1, 1, HP['weight_decay'])
            torch.cuda.synchronize()
            for i, r in enumerate(rows):
                g, f = (r['g16'], 0.5) if i == 0 else (r['g32'], None)
                po, mo, vo, _ = oracle.adam_cast(g, r['p'], r['m'], r['v'], step=step, factor=f, **HP)
                assert np.array_equal(bits(r['t'][1]), po.view(np.uint32)), (rnd, i)
                assert np.array_equal(bits(r['t'][2]), mo.view(np.uint32)), (rnd, i)
                assert np.array_equal(bits(r['t'][3]), vo.view(np.uint32)), (rnd, i)
                r['p'], r['m'], r['v'] = po, mo, vo
    assert fa._tables.builds == 10
    fa.fold, fa.fold_factor = {}, None


# ---------------------------------------------------------------------------------------------- zero1_fast
def expected_update(params, grads16, state, step, factor0, max_norm, reduce_owner):
    """Oracle: norm over all bf16 grads and the clip chain of zero1_fast.py:150-160 (REDUCE_OWNER: via sq and
    sqrt) or :157-160 (grad_norm = factor * norm).  Returns (grad_norm, factor, n_r, None)."""
    ss = sum(oracle.sumsq(g) for g in grads16)
    nr = np.float32(np.sqrt(ss))
    if reduce_owner:
        _, gn, fac = oracle.norm_clip(float(nr) ** 2, factor0, max_norm)
    else:
        gn, fac = oracle.clip_factor(nr, factor0, max_norm)
    return gn, fac, nr, None


@pytest.mark.parametrize('switches', [
    dict(ONE_PASS=True, SCALE_KERNEL=True, FOLD_SCALE=True),
    dict(ONE_PASS=True, SCALE_KERNEL=True, FOLD_SCALE=False),
    dict(ONE_PASS=False, SCALE_KERNEL=False, FOLD_SCALE=False),
    dict(ONE_PASS=True, SCALE_KERNEL=True, FOLD_SCALE=True, ALLGATHER=True),
    dict(ONE_PASS=True, SCALE_KERNEL=True, FOLD_SCALE=False, FUSED_ADAM=False),
], ids=['fold', 'scale_kernel', 'foreach', 'allgather_buffer', 'no_fused_adam'])
@pytest.mark.parametrize('reduce_owner', [False, True], ids=['all_grads', 'reduce_owner'])
def test_zero1_fast_trainer_sequence(pkg, dev, switches, reduce_owner):
    from faster_yoco_amd import zero1_fast
    sw = dict(ENABLED=True, FUSED_ADAM=True, ALLGATHER=False, PARAM_VIEWS=False, REDUCE_OWNER=reduce_owner)
    sw.update(switches)
    zero1_fast.configure(**sw)

    class Mixin(fakes.FakeMixin):
        pass

    zero1_fast._ORIG.clear()
    assert zero1_fast.install(Mixin)

    class Opt(Mixin, fakes.FakeFP16Optimizer):
        pass

    params = bf16_params(dev, 1)
    opt = Opt(params, lr=HP['lr'], betas=(HP['beta1'], HP['beta2']), eps=HP['eps'], weight_decay=HP['weight_decay'])
    state = [(p.detach().float().cpu().numpy().ravel().copy(), np.zeros(p.numel(), np.float32),
              np.zeros(p.numel(), np.float32)) for p in params]
    oss = opt.fp32_optimizer.optimizer
    for step, max_norm in ((1, 1.0), (2, 0.05), (3, 0.0)):
        set_grads(params, 10 + step)
        grads16 = [bits(p.grad).ravel().copy() for p in params]
        # trainer_nosync.py:273-282: multiply_grads(numer / denom) with a device denom, then clip_grad_norm
        denom = torch.tensor(16384.0, device=dev)
        opt.multiply_grads(8 / denom)
        factor0 = np.float32(opt._multiply_factor.item())
        gn = opt.clip_grad_norm(max_norm)
        ftensor = opt._multiply_factor                 # the clipped factor (written in place on device)
        fac_gpu = float(ftensor.item())
        exp_gn, exp_fac, nr, _ = expected_update(params, grads16, state, step, factor0, max_norm, reduce_owner)
        assert gn.dim() == 0 and gn.dtype == torch.float32 and gn.is_cuda
        got_gn = np.float32(gn.item())
        assert abs(float(got_gn) - float(exp_gn)) <= 1e-6 * float(exp_gn) + 1e-30
        if got_gn == exp_gn:                           # same norm bits -> the chain is bit-exact
            assert np.float32(fac_gpu) == exp_fac
        opt.step()
        torch.cuda.synchronize()
        assert opt._multiply_factor == 1.0
        if not sw['FUSED_ADAM']:
            # amp_C's multi_tensor_adam replaced by this build's Adam without BF16 destinations (the step's casts
            # write the BF16 copies)
            from faster_yoco_amd.fused_adam_cast import FusedAdamCast
            assert isinstance(oss.optim.multi_tensor_adam, FusedAdamCast) and oss.optim.multi_tensor_adam.dest == {}
        if not sw.get('FOLD_SCALE'):
            # the masters' FP32 gradients are written as the reference writes them: fp32(float(g16) * factor)
            for i, p32 in enumerate(opt.fp32_params):
                assert np.array_equal(bits(p32.grad).ravel(), oracle.scale_up(grads16[i], fac_gpu).view(np.uint32)), i
        new = [oracle.adam_cast(g, *st_, step=step, factor=fac_gpu, **HP) for g, st_ in zip(grads16, state)]
        for i, p in enumerate(params):
            po, mo, vo, p16 = new[i]
            st = oss.optim.state[opt.fp32_params[i]]
            assert np.array_equal(bits(opt.fp32_params[i]).ravel(), po.view(np.uint32)), i
            assert np.array_equal(bits(st['exp_avg']).ravel(), mo.view(np.uint32)), i
            assert np.array_equal(bits(st['exp_avg_sq']).ravel(), vo.view(np.uint32)), i
            assert np.array_equal(bits(p).ravel(), p16), i
        state = [(po, mo, vo) for po, mo, vo, _ in new]
        opt.zero_grad()
        assert all(p.grad is None for p in params)
    zero1_fast.configure(ENABLED=False)


def test_zero1_fast_default_fold_switch_writes_master_grads(pkg, dev):
    """Under the default YOCO_Z1_FOLD_SCALE (unset: off) the step leaves the reference's observable state: every
    owned master's .grad holds fp32(float(g16) * factor) (zero1_fast.py:175-192) after the step."""
    from faster_yoco_amd import zero1_fast
    default_fold = zero1_fast._switch('YOCO_Z1_FOLD_SCALE')
    assert default_fold is False
    zero1_fast.configure(ENABLED=True, FUSED_ADAM=True, ONE_PASS=True, SCALE_KERNEL=True, ALLGATHER=False,
                         PARAM_VIEWS=False, REDUCE_OWNER=False, FOLD_SCALE=default_fold)

    class Mixin(fakes.FakeMixin):
        pass

    zero1_fast._ORIG.clear()
    assert zero1_fast.install(Mixin)

    class Opt(Mixin, fakes.FakeFP16Optimizer):
        pass

    params = bf16_params(dev, 3)
    opt = Opt(params, lr=HP['lr'], betas=(HP['beta1'], HP['beta2']), eps=HP['eps'], weight_decay=HP['weight_decay'])
    set_grads(params, 31)
    grads16 = [bits(p.grad).ravel().copy() for p in params]
    opt.multiply_grads(8 / torch.tensor(16384.0, device=dev))
    opt.clip_grad_norm(0.05)
    fac = float(opt._multiply_factor.item())
    opt.step()
    torch.cuda.synchronize()
    for i, p32 in enumerate(opt.fp32_params):
        assert np.array_equal(bits(p32.grad).ravel(), oracle.scale_up(grads16[i], fac).view(np.uint32)), i
    zero1_fast.configure(ENABLED=False)


def test_zero1_fast_disabled_falls_back(pkg, dev):
    from faster_yoco_amd import zero1_fast
    zero1_fast.configure(ENABLED=False)

    class Mixin(fakes.FakeMixin):
        pass

    assert not zero1_fast.install(Mixin)
    zero1_fast.configure(ENABLED=True)
    zero1_fast._ORIG.clear()
    zero1_fast.install(Mixin)

    class Opt(Mixin, fakes.FakeFP16Optimizer):
        pass

    opt = Opt(bf16_params(dev, 2))
    opt.fp32_optimizer.optimizer = object()          # not an OSS: the reference falls back to upstream
    with pytest.raises(AssertionError, match='upstream clip_grad_norm reached'):
        opt.clip_grad_norm(1.0)
    zero1_fast.configure(ENABLED=False)


# ------------------------------------------------------------------------------------------------ CEReduce
def test_ce_reduce_sum_installed(pkg, dev):
    from faster_yoco_amd import ce_reduce
    rng = np.random.default_rng(5)
    W, G = 8, 5000
    cls = type('CEReduce', (fakes.FakeCEReduce,), {})
    ce_reduce.install(cls)
    for R in (0, 6):
        S = oracle.bf16_rne((rng.standard_normal((W - 1) * G) * 1e-3).astype(np.float32))
        OUT = oracle.bf16_rne((rng.standard_normal(G) * 1e-3).astype(np.float32))
        bounds = [[0, 1234], [1234, 1234], [1234, G]]
        ce = cls(torch.from_numpy(S.view(np.int16)).to(dev).view(torch.bfloat16),
                 torch.from_numpy(OUT.view(np.int16)).to(dev).view(torch.bfloat16), G, bounds, R, W)
        exp = OUT.copy()
        for ph, (a, b) in enumerate(bounds):
            ce._sum(ph)
            oracle.sum_slots(S, exp, G, a, b, R, 1.0 / W, W)
        torch.cuda.synchronize()
        assert np.array_equal(bits(ce.out), exp)


def test_zero1_fast_measured_switch_set_with_placed_params(pkg, dev):
    """scripts/configs/faster.env's optimizer switches (ZERO1_FAST, ALLGATHER, PARAM_VIEWS, PARAM_ALLREDUCE +
    GRAD_REDUCE_OWNER, Z1_ONE_PASS, Z1_SCALE_KERNEL, FUSED_ADAM) with torch.distributed initialised (gloo, one
    rank): _place_params puts the parameters into the flat BF16 buffer (zero1_fast.py:52-75), _setup checks the
    placement against the OSS partition (:103-118), and the update writes the BF16 copy straight into the placed
    parameters."""
    import torch.distributed as dist
    from faster_yoco_amd import layout, zero1_fast
    if dist.is_initialized():
        pytest.skip('a process group already exists')
    dist.init_process_group('gloo', init_method='tcp://127.0.0.1:29531', rank=0, world_size=1)
    try:
        zero1_fast.configure(ENABLED=True, ALLGATHER=True, PARAM_VIEWS=True, REDUCE_OWNER=True, ONE_PASS=True,
                             SCALE_KERNEL=True, FUSED_ADAM=True, FOLD_SCALE=True)
        zero1_fast._PLACED.clear()
        module = torch.nn.Module()
        for i, p in enumerate(bf16_params(dev, 7)):
            module.register_parameter(f'w{i}', p)
        zero1_fast._place_params(module)
        params = list(module.parameters())
        flat = zero1_fast._PLACED['flat']
        owner, where, seg = layout.segments([p.numel() for p in params], 1)
        assert zero1_fast._PLACED['seg'] == seg
        for p, off in zip(params, where):
            assert p.data_ptr() == flat.data_ptr() + off * 2

        class Mixin(fakes.FakeMixin):
            pass

        zero1_fast._ORIG.clear()
        zero1_fast.install(Mixin)

        class Opt(Mixin, fakes.FakeFP16Optimizer):
            pass

        opt = Opt(params, lr=HP['lr'], betas=(HP['beta1'], HP['beta2']), eps=HP['eps'],
                  weight_decay=HP['weight_decay'])
        state = [(p.detach().float().cpu().numpy().ravel().copy(), np.zeros(p.numel(), np.float32),
                  np.zeros(p.numel(), np.float32)) for p in params]
        for step in (1, 2):
            set_grads(params, 40 + step)
            grads16 = [bits(p.grad).ravel().copy() for p in params]
            opt.multiply_grads(8 / torch.tensor(16384.0, device=dev))
            opt.clip_grad_norm(1.0)
            fac = float(opt._multiply_factor.item())
            opt.step()
            torch.cuda.synchronize()
            assert opt._z1.placed
            for i, p in enumerate(params):
                po, mo, vo, p16 = oracle.adam_cast(grads16[i], *state[i], step=step, factor=fac, **HP)
                assert np.array_equal(bits(p).ravel(), p16), i            # the placed view itself was written
                assert np.array_equal(bits(opt.fp32_params[i]).ravel(), po.view(np.uint32)), i
                state[i] = (po, mo, vo)
            opt.zero_grad()
        # a parameter moved out of its slot is refused, as the reference refuses it
        opt2 = Opt(params)
        params[0].data = params[0].data.clone()
        with pytest.raises(RuntimeError, match='not at its slot'):
            opt2.clip_grad_norm(1.0)
    finally:
        zero1_fast.configure(ENABLED=False, ALLGATHER=False, PARAM_VIEWS=False, REDUCE_OWNER=False)
        zero1_fast._PLACED.clear()
        dist.destroy_process_group()


def test_ce_reduce_phase_norm_feeds_clip_grad_norm(pkg, dev, monkeypatch):
    """The reference's measured switch set with YOCO_CE_REDUCE: CEReduce._sum per phase (two on a side stream, the
    last on the current one, yoco/models/decoder/ce_reduce.py:205-209,227-228), the owned gradients made views of
    CEReduce.out (:232-237), then zero1_fast.clip_grad_norm and step.  The norm comes from the partials the phase
    sums left -- no norm pass over the gradients runs -- and is within one fp32 ulp of the norm pass over the same
    gradients (and 1e-6 of the exact norm); the clip chain, the written FP32 gradients, masters, moments and BF16
    copies match the oracle bit for bit.  Gradients that are not those views (a zero-filled one, or a phase that was
    not summed this update) take the norm pass instead."""
    from faster_yoco_amd import ce_reduce, layout, ops, zero1_fast
    zero1_fast.configure(ENABLED=True, ALLGATHER=True, PARAM_VIEWS=True, REDUCE_OWNER=True, ONE_PASS=True,
                         SCALE_KERNEL=True, FUSED_ADAM=True, FOLD_SCALE=False)
    zero1_fast._PLACED.clear()
    try:
        params = bf16_params(dev, 11)
        zero1_fast._PLACED.update(layout.place_params(params, 1))

        class Mixin(fakes.FakeMixin):
            pass

        zero1_fast._ORIG.clear()
        zero1_fast.install(Mixin)

        class Opt(Mixin, fakes.FakeFP16Optimizer):
            pass

        opt = Opt(params, lr=HP['lr'], betas=(HP['beta1'], HP['beta2']), eps=HP['eps'],
                  weight_decay=HP['weight_decay'])
        numels = [p.numel() for p in params]
        G, W, R = sum(numels), 8, 2
        ends = np.cumsum(numels).tolist()
        bounds = [[0, ends[1]], [ends[1], ends[1]], [ends[1], ends[3]], [ends[3], G]]   # an empty phase too
        cls = ce_reduce.install(type('CEReduce', (fakes.FakeCEReduce,), {}))
        rng = np.random.default_rng(4)
        state = [(p.detach().float().cpu().numpy().ravel().copy(), np.zeros(p.numel(), np.float32),
                  np.zeros(p.numel(), np.float32)) for p in params]
        side = torch.cuda.Stream(device=dev)
        used = {'pass': 0}
        for name in ('grad_sumsq', 'grad_norm_clip'):
            real = getattr(ops, name)

            def counted(*a, _real=real, **k):
                used['pass'] += 1
                return _real(*a, **k)
            monkeypatch.setattr(ops, name, counted)
        two = [[0, ends[3]], [ends[3], G]]              # other phase bounds: the CEReduce's PhaseNorm is made again
        steps = ((1.0, True, bounds), (0.01, True, bounds), (1.0, False, bounds), (1.0, 'stale', bounds),
                 (1.0, True, two))
        for step, (max_norm, fused, bnds) in enumerate(steps, 1):
            S = oracle.bf16_rne((rng.standard_normal((W - 1) * G) * 1e-2).astype(np.float32))
            OUT = oracle.bf16_rne((rng.standard_normal(G) * 1e-2).astype(np.float32))
            if step < 5:
                ce = cls(torch.from_numpy(S.view(np.int16)).to(dev).view(torch.bfloat16),
                         torch.from_numpy(OUT.view(np.int16)).to(dev).view(torch.bfloat16), G, bnds, R, W)
            else:                                  # the same CEReduce and out, new contents and bounds
                ce.staging.copy_(torch.from_numpy(S.view(np.int16)).to(dev).view(torch.bfloat16))
                ce.out.copy_(torch.from_numpy(OUT.view(np.int16)).to(dev).view(torch.bfloat16))
                ce.bounds = bnds
            avg = OUT.copy()
            for a, b in bnds:
                oracle.sum_slots(S, avg, G, a, b, R, 1.0 / W, W)
            cur = torch.cuda.current_stream(dev)
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                for ph in range(len(bnds) - 1):
                    ce._sum(ph)
            if fused != 'stale':
                ce._sum(len(bnds) - 1)
            else:                                  # the last phase summed without its partials: no fused norm
                ce_reduce.sum_slots(ce.staging, ce.out, G, *bnds[-1], R, 1.0 / W, W)
            cur.wait_stream(side)
            off = 0
            for p, n in zip(params, numels):
                p.grad = ce.out[off:off + n].view_as(p)
                off += n
            if fused is False:
                params[1].grad = params[1].grad.clone()          # no longer a view of out
            grads16 = [avg[o - n:o] for o, n in zip(ends, numels)]
            before = used['pass']
            allocs = torch.cuda.memory_stats()['allocation.all.allocated']
            gn = opt.clip_grad_norm(max_norm)
            assert (used['pass'] == before) == (fused is True), step
            fac = float(opt._multiply_factor.item())
            _, exp_gn, exp_fac = oracle.norm_clip(sum(oracle.sumsq(g) for g in grads16), 1.0, max_norm)
            got = np.float32(gn.item())
            assert abs(int(got.view(np.int32)) - int(exp_gn.view(np.int32))) <= 1, (step, got, exp_gn)
            if got == exp_gn:                              # same norm bits -> the chain is bit-exact
                assert np.float32(fac) == exp_fac, step
            opt.step()
            torch.cuda.synchronize()
            if step == 2:                      # a recurring update allocates only the grad_norm it returns
                assert torch.cuda.memory_stats()['allocation.all.allocated'] - allocs == 1
            for i, p in enumerate(params):
                po, mo, vo, p16 = oracle.adam_cast(grads16[i], *state[i], step=step, factor=fac, **HP)
                st = opt.fp32_optimizer.optimizer.optim.state[opt.fp32_params[i]]
                assert np.array_equal(bits(opt.fp32_params[i].grad).ravel(),
                                      oracle.scale_up(grads16[i], fac).view(np.uint32)), (step, i)
                assert np.array_equal(bits(opt.fp32_params[i]).ravel(), po.view(np.uint32)), (step, i)
                assert np.array_equal(bits(st['exp_avg']).ravel(), mo.view(np.uint32)), (step, i)
                assert np.array_equal(bits(st['exp_avg_sq']).ravel(), vo.view(np.uint32)), (step, i)
                assert np.array_equal(bits(p).ravel(), p16), (step, i)
                state[i] = (po, mo, vo)
            opt.zero_grad()
    finally:
        zero1_fast.configure(ENABLED=False, ALLGATHER=False, PARAM_VIEWS=False, REDUCE_OWNER=False)
        zero1_fast._PLACED.clear()
