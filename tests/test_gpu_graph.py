"""The shard update captured in a HIP graph (torch.cuda.graph): norm + clip + Adam + BF16 copy, and the owner-sum
form (owner sum with the fused norm, clip, Adam), each replayed several times from a restored state -- with eager
work and synchronisations between the replays -- and every replay bit-identical to the same update run eagerly.
Likewise the owner's embedding gradient, and the drop-in's FusedAdamCast call (folded BF16 gradients, FP32
gradients written) after one eager call.

The update launches only kernels on the current stream (the tables and the norm workspace are made at set-up, and
nothing in it clears memory with a memset), so it can be captured once per step and replayed; the bias corrections
are kernel arguments rounded on the host, so a graph holds one step's."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def make(dev, shapes, grad_dtype, seed, step):
    from faster_yoco_amd import shard as shard_mod
    sh = shard_mod.FlatShard(shapes, dev, grad_dtype=grad_dtype)
    rng = np.random.default_rng(seed)
    n = sh.total
    sh.p.copy_(torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)))
    sh.m.copy_(torch.from_numpy((rng.standard_normal(n) * 1e-4).astype(np.float32)))
    sh.v.copy_(torch.from_numpy(np.abs(rng.standard_normal(n) * 1e-8).astype(np.float32)))
    g = torch.from_numpy((rng.standard_normal(n) * 3e-3).astype(np.float32))
    sh.g.copy_(g.to(grad_dtype))
    opt = shard_mod.Zero1ShardOptimizer(sh, **HP)
    opt.step_count = step - 1
    return sh, opt


def snapshot(sh):
    return {k: getattr(sh, k).clone() for k in ('g', 'p', 'm', 'v', 'p16')}


def restore(sh, snap):
    for k, t in snap.items():
        getattr(sh, k).copy_(t)


def bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def check_same(sh, ref):
    for k in ('p', 'm', 'v', 'p16'):
        assert torch.equal(bits(getattr(sh, k)), bits(ref[k])), k


def contributions(n, dev, seed):
    rng = np.random.default_rng(seed)
    return [torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(dev).to(torch.bfloat16)
            for _ in range(8)]


@pytest.mark.parametrize('form', ['norm', 'owner_sum'])
def test_update_graph_replays_match_eager(pkg, dev, form):
    from faster_yoco_amd import configs
    step = 7
    gdt = torch.bfloat16 if form == 'owner_sum' else torch.float32
    sh, opt = make(dev, configs.C1_SHAPES, gdt, seed=11, step=step)
    contribs = contributions(sh.total, dev, 12) if form == 'owner_sum' else None
    snap = snapshot(sh)

    def update():
        if contribs is not None:
            opt.reduce_grads(contribs)
        return opt.update(1.0)

    # eager reference of this step
    gn_eager = update().clone()
    torch.cuda.synchronize()
    ref = snapshot(sh)

    # capture the same step (nothing runs during capture), then replay from the restored state
    restore(sh, snap)
    opt.step_count = step - 1
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):                  # captures on torch's capture stream, the current one inside
        gn_graph = update()
    torch.cuda.synchronize()
    assert opt.step_count == step
    for rep in range(3):
        restore(sh, snap)
        junk = torch.randn(1 << 20, device=dev).sum()          # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(gn_graph.reshape(1)), bits(gn_eager.reshape(1))), rep
        check_same(sh, ref)
        del junk
    graph.reset()


def test_device_step_graph_replays_every_step(pkg, dev):
    """With device_step the step counter and bias corrections advance on the device, so one captured update
    replays correctly at every step: each replay (new gradients written between them, as a backward pass would)
    equals the eager update at the next step, with the host-rounded corrections."""
    from faster_yoco_amd import configs, shard as shard_mod
    sh_a, _ = make(dev, configs.C1_MINI_SHAPES, torch.float32, seed=31, step=1)
    sh_b, opt_b = make(dev, configs.C1_MINI_SHAPES, torch.float32, seed=31, step=1)
    opt_a = shard_mod.Zero1ShardOptimizer(sh_a, **HP, device_step=True)
    opt_a.set_step(41)
    opt_b.set_step(41)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gn_graph = opt_a.update(1.0)
    torch.cuda.synchronize()
    rng = np.random.default_rng(32)
    for rep in range(3):
        g = torch.from_numpy((rng.standard_normal(sh_a.total) * 3e-3).astype(np.float32)).to(dev)
        sh_a.g.copy_(g)
        sh_b.g.copy_(g)
        graph.replay()
        gn_eager = opt_b.update(1.0)
        torch.cuda.synchronize()
        assert torch.equal(bits(gn_graph.reshape(1)), bits(gn_eager.reshape(1))), rep
        check_same(sh_a, state(sh_b))
    assert int(opt_a._step_dev.item()) == 44 and opt_b.step_count == 44
    graph.reset()


def state(sh):
    return {k: getattr(sh, k).clone() for k in ('p', 'm', 'v', 'p16')}


def test_device_bias_corrections_equal_host_rounding(pkg, dev):
    """z1_bias_corrections_step's fp32(1 - beta^step), computed in double on the device, equals the host's
    (yoco/tasks/fused_adam_cast.py:58-60) at every step 1..20000 for two beta pairs, and at large steps."""
    from faster_yoco_amd import ops
    for b1, b2 in ((0.9, 0.95), (0.9, 0.999)):
        step = torch.zeros(1, dtype=torch.int64, device=dev)
        bc = torch.empty(2, dtype=torch.float32, device=dev)
        n = 20000
        rec = torch.empty(n, 2, dtype=torch.float32, device=dev)
        for i in range(n):
            ops.bias_corrections_step(step, b1, b2, bc)
            rec[i].copy_(bc)
        got = rec.cpu().numpy()
        want = np.array([ops.bias_corrections(b1, b2, s) for s in range(1, n + 1)], dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (b1, b2)
        assert int(step.item()) == n
        for s in (10 ** 6, 10 ** 7, 2 ** 31, 10 ** 9):
            step.fill_(s - 1)
            ops.bias_corrections_step(step, b1, b2, bc)
            assert tuple(bc.cpu().numpy()) == tuple(np.float32(ops.bias_corrections(b1, b2, s))), s
    step = torch.zeros(1, dtype=torch.int64, device=dev)
    bc = torch.zeros(2, dtype=torch.float32, device=dev)
    ops.bias_corrections_step(step, 0.9, 0.95, bc, bias_correction=0)
    assert bc.tolist() == [1.0, 1.0]


@pytest.mark.parametrize('R,zipf', [(16384, False), (16384, True), (2048, False)])
def test_owner_embedding_grad_graph_replays_match_eager(pkg, dev, R, zipf):
    """The owner's embedding gradient (OwnerEmbeddingGrad: output and workspace made once) captured in a HIP graph
    and replayed on new ids and rows copied into its static inputs, three times with eager work in between: every
    replay bit-identical to the eager call on the same inputs, and to torch's aten + x 1/8 (the reference's
    layer_graphs.py:92-93).  The sort it runs clears nothing with memsets."""
    from faster_yoco_amd import embedding
    D, V = 3072, 100288
    gen = torch.Generator(device='cpu').manual_seed(R + zipf)

    def inputs():
        if zipf:
            z = np.random.default_rng(int(torch.randint(0, 1 << 30, (1,), generator=gen))).zipf(1.2, R) - 1
            ids = torch.from_numpy(np.where(z < V, z, 0).astype(np.int64))
        else:
            ids = torch.randint(0, V, (R,), generator=gen)
        return (torch.randn(R, D, generator=gen) * 1e-2).to(torch.bfloat16).to(dev), ids.to(dev)

    plan = embedding.OwnerEmbeddingGrad(R, D, V, -1, 8, dev)
    g_static, i_static = inputs()
    plan(g_static, i_static)                            # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan(g_static, i_static)
    for _ in range(3):
        g_new, i_new = inputs()
        g_static.copy_(g_new)
        i_static.copy_(i_new)
        graph.replay()
        torch.cuda.synchronize()
        got = plan.out.clone()
        eager = embedding.owner_embedding_grad(g_new, i_new, V, -1, 8)      # eager work between the replays
        aten = torch.ops.aten.embedding_dense_backward(g_new, i_new, V, -1, False).mul_(1.0 / 8)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16))
        assert torch.equal(got.view(torch.int16), aten.view(torch.int16))


def test_dropin_fused_adam_graph_replays_match_eager(pkg, dev):
    """The drop-in's default Adam call -- FusedAdamCast over per-parameter tensors with the BF16 gradients folded in
    and the FP32 gradients written by the same launch -- captured after one eager call (which makes the tables and
    the plan) and replayed three times from a restored state: every replay equals the eager call bit for bit,
    masters, moments, BF16 copies and the written FP32 gradients."""
    from faster_yoco_amd.fused_adam_cast import FusedAdamCast
    shapes = [(96, 64), (3, 1000), (4096,), (7,), (256, 33)]
    gen = torch.Generator(device='cpu').manual_seed(17)
    mk = lambda s, sd: (torch.randn(*s, generator=gen) * sd).to(dev)
    p = [mk(s, 0.02) for s in shapes]
    m = [mk(s, 1e-4) for s in shapes]
    v = [mk(s, 1e-8).abs() for s in shapes]
    g32 = [torch.zeros(s, device=dev) for s in shapes]
    g16 = [mk(s, 1e-2).to(torch.bfloat16) for s in shapes]
    p16 = [torch.zeros(s, dtype=torch.bfloat16, device=dev) for s in shapes]
    fa = FusedAdamCast({a.data_ptr(): b for a, b in zip(p, p16)})
    fa.fold, fa.fold_factor, fa.fold_writes = {a.data_ptr(): b for a, b in zip(p, g16)}, \
        torch.tensor([0.37], device=dev), True
    state = [p, m, v, g32, p16]
    start = [[t.clone() for t in X] for X in state]

    def call():
        fa(2048 * 32, None, [g32, p, m, v], 3e-4, 0.9, 0.95, 1e-8, 5, 1, 1, 0.1)

    def restore_state():
        for X, S in zip(state, start):
            for t, s in zip(X, S):
                t.copy_(s)
    call()                                            # eager: tables, plan, and the reference result
    torch.cuda.synchronize()
    eager = [[t.clone() for t in X] for X in state]
    restore_state()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        restore_state()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for X, E in zip(state, eager):
            for t, e in zip(X, E):
                assert torch.equal(t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32),
                                   e.view(torch.int16) if e.dtype == torch.bfloat16 else e.view(torch.int32))
    assert fa.cast == {a.data_ptr() for a in p}
