"""The custom operators on the GPU: the shard update compiled with torch.compile(fullgraph=True) -- no graph break,
no recompilation across steps -- gives the eager update's bits at every step (under AOT functionalization the
operators may run on copies of the state, which their tables follow); torch.library.opcheck passes for the
operators (schema / mutation annotations, fake tensors, AOT dispatch); and every launch shows up in the profiler as
its operator."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
SHAPES = [(96, 64), (3, 1000), (4096,), (7,), (256, 33)]


def bits(t):
    t = t.detach().cpu()
    return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy().view(np.uint32)


def make_state(dev, grad_dtype, seed):
    from faster_yoco_amd import shard
    sh = shard.FlatShard(SHAPES, dev, grad_dtype=grad_dtype)
    g = torch.Generator(device='cpu').manual_seed(seed)
    n = sh.total
    sh.p.copy_(torch.randn(n, generator=g) * 0.02)
    sh.m.copy_(torch.randn(n, generator=g) * 1e-4)
    sh.v.copy_((torch.randn(n, generator=g) * 1e-8).abs())
    return sh


def update_fn(table):
    ops = torch.ops.yoco_z1

    def update(g, p, m, v, p16, partials, factor, grad_norm, step, bc):
        # norm + clip chain (factor read as 1.0, the clipped factor written), step counter, Adam + BF16
        ops.grad_norm_clip_(table, [g], partials, factor, None, grad_norm, 1.0, 1.0)
        ops.bias_corrections_step_(step, bc, HP['beta1'], HP['beta2'], 1)
        ops.adam_cast_dev_(table, [g], [p], [m], [v], [p16], factor, bc, HP['lr'], HP['beta1'], HP['beta2'],
                           HP['eps'], HP['weight_decay'], 1)
    return update


@pytest.mark.parametrize('grad_dtype', [torch.float32, torch.bfloat16])
def test_compiled_shard_update_matches_eager(pkg, dev, grad_dtype):
    from faster_yoco_amd import ops
    torch._dynamo.reset()
    runs = []
    for compiled in (False, True):
        sh = make_state(dev, grad_dtype, 3)
        partials = ops.norm_workspace(dev)
        factor, grad_norm = torch.zeros(1, device=dev), torch.zeros(1, device=dev)
        step, bc = torch.full((1,), 999, dtype=torch.int64, device=dev), torch.ones(2, device=dev)
        fn = update_fn(sh.table.handle_int)
        if compiled:
            fn = torch.compile(fn, fullgraph=True, backend='aot_eager')
        out = []
        with torch._dynamo.config.patch(error_on_recompile=True):
            for k in range(3):
                gen = torch.Generator(device='cpu').manual_seed(100 + k)
                sh.g.copy_((torch.randn(sh.total, generator=gen) * 1e-2).to(grad_dtype))
                fn(sh.g, sh.p, sh.m, sh.v, sh.p16, partials, factor, grad_norm, step, bc)
                torch.cuda.synchronize()
                out.append([bits(t).copy() for t in (sh.p, sh.m, sh.v, sh.p16, factor, grad_norm, step, bc)])
        runs.append(out)
    for k, (a, b) in enumerate(zip(*runs)):
        for name, x, y in zip(('p', 'm', 'v', 'p16', 'factor', 'grad_norm', 'step', 'bc'), a, b):
            assert np.array_equal(x, y), (k, name)
    assert int(runs[0][-1][6][0]) == 1002                            # three steps counted on the device


def test_opcheck_operators(pkg, dev):
    from faster_yoco_amd import ops
    opcheck = torch.library.opcheck
    Y = torch.ops.yoco_z1
    gen = torch.Generator(device='cpu').manual_seed(7)
    n = 5000
    g = (torch.randn(n, generator=gen) * 1e-2).to(dev)
    p, m = (torch.randn(n, generator=gen) * 0.02).to(dev), (torch.randn(n, generator=gen) * 1e-4).to(dev)
    v, p16 = (torch.randn(n, generator=gen) * 1e-8).abs().to(dev), torch.zeros(n, dtype=torch.bfloat16, device=dev)
    table = ops.Table([(g, p, m, v, p16, n)], dev)
    part = ops.norm_workspace(dev)
    one = lambda: torch.zeros(1, device=dev)
    cases = [
        (Y.grad_sumsq_.default, (table.handle_int, [g], part)),
        (Y.grad_norm_clip_.default, (table.handle_int, [g], part, one(), one(), one(), 1.0, 0.5)),
        (Y.norm_clip_.default, (part, one(), one(), one(), 1.0, 0.5)),
        (Y.clip_factor_.default, (torch.tensor([3.0], device=dev), one(), one(), 1.0, 0.5)),
        (Y.adam_cast_.default, (table.handle_int, [g], [p], [m], [v], [p16], None, 3e-4, 0.9, 0.95, 1e-8, 0.1,
                                0.05, 0.1, 1, 0, 1)),
        (Y.adam_cast_gout_.default, (table.handle_int, [g], [p], [m], [v], [p16], [torch.empty(n, device=dev)],
                                     torch.tensor([0.5], device=dev), 3e-4, 0.9, 0.95, 1e-8, 0.1, 0.05, 0.1, 1, 0,
                                     1)),
        (Y.owner_sum_.default, ([p16, p16.clone()], torch.empty(n, dtype=torch.bfloat16, device=dev), 0.5, None,
                                ops.norm_workspace(dev, n))),
        (Y.scale_up_.default, (p16, torch.empty(n, device=dev), torch.tensor([0.25], device=dev))),
        (Y.cast_bf16_.default, (p, torch.empty(n, dtype=torch.bfloat16, device=dev))),
        (Y.bias_corrections_step_.default, (torch.zeros(1, dtype=torch.int64, device=dev), torch.ones(2, device=dev),
                                            0.9, 0.95, 1)),
    ]
    R, D, V = 4000, 16, 300
    rows = (torch.randn(R, D, generator=gen) * 1e-2).to(torch.bfloat16).to(dev)
    ids = torch.randint(0, V, (R,), generator=gen).to(dev)
    from faster_yoco_amd import embedding
    ws = torch.empty(embedding.workspace_bytes(R, D, V), dtype=torch.uint8, device=dev)
    cases.append((Y.embedding_dense_backward.default, (rows, ids, V, -1, 0.125, 2, ws)))
    for op, args in cases:
        res = opcheck(op, args, test_utils=('test_schema', 'test_faketensor', 'test_aot_dispatch_dynamic'))
        assert all(v == 'SUCCESS' for v in res.values()), (op, res)


def test_profiler_sees_the_operators(pkg, dev):
    sh = make_state(dev, torch.float32, 4)
    from faster_yoco_amd import shard
    opt = shard.Zero1ShardOptimizer(sh)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        opt.clip_grad_norm(1.0)
        opt.step()
        torch.cuda.synchronize()
    names = {e.name for e in prof.events()}
    assert {'yoco_z1::grad_norm_clip_', 'yoco_z1::adam_cast_'} <= names, sorted(n for n in names if 'yoco' in n)


def test_operators_refuse_tensors_off_the_launch_device(pkg, dev):
    """Every auxiliary tensor of a launch (norm workspace, factor and scalar outputs, flags, bias corrections,
    owner-sum workspace, staging, scale/cast operands) must live on the launch's device: each operator raises
    before enqueuing anything, and the state it would have written is untouched.  With one GPU the other device is
    the host; the same check compares device indices between GPUs."""
    from faster_yoco_amd import ops
    Y = torch.ops.yoco_z1
    n = 3000
    gen = torch.Generator(device='cpu').manual_seed(11)
    g = (torch.randn(n, generator=gen) * 1e-2).to(dev)
    p, m = (torch.randn(n, generator=gen) * 0.02).to(dev), (torch.randn(n, generator=gen) * 1e-4).to(dev)
    v, p16 = (torch.randn(n, generator=gen) * 1e-8).abs().to(dev), torch.zeros(n, dtype=torch.bfloat16, device=dev)
    table = ops.Table([(g, p, m, v, p16, n)], dev)
    t = table.handle_int
    part = ops.norm_workspace(dev)
    one = lambda: torch.zeros(1, device=dev)
    host1 = lambda: torch.zeros(1)
    before = [x.clone() for x in (p, m, v, p16)]
    calls = [
        lambda: Y.grad_sumsq_(t, [g], part.cpu()),
        lambda: Y.grad_norm_clip_(t, [g], part, host1(), one(), one(), 1.0, 0.5),
        lambda: Y.norm_clip_(part, one(), host1(), one(), 1.0, None),
        lambda: Y.update_scalars_(part, one(), one(), one(), torch.zeros(2, dtype=torch.uint8), None, None, 1.0,
                                  1.0, None),
        lambda: Y.grad_update_scalars_(t, [g], part, one(), one(), one(), None, host1(), None, 1.0, 1.0, None),
        lambda: Y.clip_factor_(torch.tensor([3.0], device=dev), host1(), one(), 1.0, None),
        lambda: Y.adam_cast_(t, [g], [p], [m], [v], [p16], host1(), 3e-4, 0.9, 0.95, 1e-8, 0.1, 0.05, 0.1, 1, 0, 1),
        lambda: Y.adam_cast_dev_(t, [g], [p], [m], [v], [p16], one(), torch.ones(2), 3e-4, 0.9, 0.95, 1e-8, 0.1, 1),
        lambda: Y.owner_sum_([p16, p16.clone()], torch.empty_like(p16), 0.5, None, ops.norm_workspace(dev, n).cpu()),
        lambda: Y.owner_sum_update_([p16, p16.clone()], torch.empty_like(p16), ops.norm_workspace(dev, n), 0.5, None,
                                    host1(), None, None, None, None, None, 1.0, 1.0, None),
        lambda: Y.sum_slots_(torch.zeros(n, dtype=torch.bfloat16), torch.empty_like(p16), n, 0, n, 0, 0.5, 2),
        lambda: Y.scale_up_(p16, torch.empty(n, device=dev), torch.tensor([0.25])),
        lambda: Y.cast_bf16_(p, torch.empty(n, dtype=torch.bfloat16)),
    ]
    for i, call in enumerate(calls):
        with pytest.raises(RuntimeError):
            call()
        torch.cuda.synchronize()
        for a, b in zip((p, m, v, p16), before):
            assert torch.equal(a, b), f'call {i} changed the state before refusing'
