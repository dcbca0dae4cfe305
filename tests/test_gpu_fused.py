"""The one-call forms against the calls they combine, on the GPU: z1_grad_norm_clip = z1_grad_sumsq +
z1_norm_clip, z1_grad_update_scalars = z1_grad_sumsq + z1_update_scalars_run, z1_owner_sum_update =
z1_owner_sum_bf16 + z1_update_scalars_run (bits of every scalar output, and of the average), called many times in a
row, with two tables interleaved and inputs of changing size.
Rebinding a table's gradients (z1_table_set_grads) is checked against a table made on the new gradients, and the
shard optimizer's update against the oracle when its gradient tensors move between steps.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def f32_bits(t):
    return t.detach().cpu().numpy().view(np.uint32).copy()


def grads_table(pkg, dev, sizes, seed, dtype=torch.float32, scale=1e-2):
    from faster_yoco_amd import ops
    g = torch.Generator(device='cpu').manual_seed(seed)
    gs = [(torch.randn(n, generator=g) * scale).to(dtype).to(dev) for n in sizes]
    return gs, ops.Table([(x, None, None, None, None, x.numel()) for x in gs], dev)


def scalars(dev, k=3):
    return [torch.full((1,), -1.0, device=dev) for _ in range(k)]


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_grad_norm_clip_equals_the_two_launches(pkg, dev, dtype):
    from faster_yoco_amd import ops
    tabs = [grads_table(pkg, dev, [70001, 256 * 37, 100, 0, 12295], 1, dtype),
            grads_table(pkg, dev, [3, 1 << 20, 777], 2, dtype, scale=5.0)]        # clip inactive / active
    part_a, part_b = ops.norm_workspace(dev), ops.norm_workspace(dev)
    for rep in range(12):                                # interleaved tables
        gs, table = tabs[rep % 2]
        fac = [1.0, 0.5, 3.0][rep % 3]
        mn = [1.0, 0.0, 2.5][rep % 3]
        two, one = scalars(dev), scalars(dev)
        ops.grad_sumsq(table, part_a)
        ops.norm_clip(part_a, factor=fac, norm_out=two[0], grad_norm_out=two[1], factor_out=two[2], max_norm=mn)
        ops.grad_norm_clip(table, part_b, factor=fac, norm_out=one[0], grad_norm_out=one[1], factor_out=one[2],
                           max_norm=mn)
        torch.cuda.synchronize()
        assert np.array_equal(f32_bits(part_a[:2048]), f32_bits(part_b[:2048]).view(np.uint32))
        for a, b in zip(two, one):
            assert np.array_equal(f32_bits(a), f32_bits(b)), rep
        ex = float(np.sqrt(sum(oracle.sumsq(x.float().cpu().numpy()) for x in gs)))
        assert abs(float(one[0].item()) - ex) <= 1e-6 * ex
    # a device factor updated in place
    gs, table = tabs[0]
    f_two = torch.tensor([0.25], device=dev)
    f_one = f_two.clone()
    ops.grad_sumsq(table, part_a)
    ops.norm_clip(part_a, factor=f_two, factor_out=f_two, max_norm=1.0)
    ops.grad_norm_clip(table, part_b, factor=f_one, factor_out=f_one, max_norm=1.0)
    torch.cuda.synchronize()
    assert np.array_equal(f32_bits(f_two), f32_bits(f_one))


def test_grad_update_scalars_equals_the_two_launches(pkg, dev):
    from faster_yoco_amd import ops
    gs, table = grads_table(pkg, dev, [4096, 99, 1 << 16], 3)
    part_a, part_b = ops.norm_workspace(dev), ops.norm_workspace(dev)
    for rep, (ss, numer, mn) in enumerate([(16384.0, 8, 1.0), (0.0, 8, 1.0), (-3.0, 1, 0.0), (7.0, 8, 1e-9)]):
        sample = torch.tensor([ss], device=dev)
        outs_a = scalars(dev, 4) + [torch.zeros(2, dtype=torch.uint8, device=dev)]
        outs_b = scalars(dev, 4) + [torch.zeros(2, dtype=torch.uint8, device=dev)]
        for part, outs, fused in ((part_a, outs_a, False), (part_b, outs_b, True)):
            kw = dict(sample_size=sample, numer=numer, factor=1.0, max_norm=mn, norm_out=outs[0],
                      grad_norm_out=outs[1], factor_out=outs[2], clip_log_out=outs[3], flags_out=outs[4])
            if fused:
                ops.grad_update_scalars(table, part, **kw)
            else:
                ops.grad_sumsq(table, part)
                ops.update_scalars(part, **kw)
        torch.cuda.synchronize()
        for a, b in zip(outs_a[:4], outs_b[:4]):
            assert np.array_equal(f32_bits(a), f32_bits(b)), rep
        assert torch.equal(outs_a[4], outs_b[4])


@pytest.mark.parametrize('world', [1, 8, 11])
def test_owner_sum_update_equals_the_two_calls(pkg, dev, world):
    from faster_yoco_amd import ops
    n_max = 300007
    gen = torch.Generator(device='cpu').manual_seed(world)
    contribs = [(torch.randn(n_max, generator=gen) * 1e-2).to(torch.bfloat16).to(dev) for _ in range(world)]
    ws_a, ws_b = ops.norm_workspace(dev, n_max), ops.norm_workspace(dev, n_max)
    for rep, n in enumerate([n_max, n_max, 513, 1, 262144, n_max]):     # shorter inputs reuse the workspace
        cs = [c[:n] for c in contribs]
        avg_a = torch.empty(n, dtype=torch.bfloat16, device=dev)
        avg_b = torch.empty(n, dtype=torch.bfloat16, device=dev)
        sum_b = torch.empty(n, dtype=torch.float32, device=dev)
        a, b = scalars(dev), scalars(dev)
        fac = 0.5 if rep % 2 else 2.0
        ops.owner_sum(cs, avg_a, 1.0 / world, partials=ws_a)
        ops.norm_clip(ws_a, factor=fac, norm_out=a[0], grad_norm_out=a[1], factor_out=a[2], max_norm=0.01)
        ops.owner_sum_update(cs, avg_b, 1.0 / world, ws_b, out_sum=sum_b, factor=fac, norm_out=b[0],
                             grad_norm_out=b[1], factor_out=b[2], max_norm=0.01)
        torch.cuda.synchronize()
        assert torch.equal(avg_a.view(torch.int16), avg_b.view(torch.int16)), (rep, n)
        for x, y in zip(a, b):
            assert np.array_equal(f32_bits(x), f32_bits(y)), (rep, n)
        hc = [c.view(torch.int16).cpu().numpy().view(np.uint16) for c in cs]
        want_avg, want_sum = oracle.owner_sum(hc, scale=1.0 / world, want_sum=True)
        assert np.array_equal(avg_b.view(torch.int16).cpu().numpy().view(np.uint16), want_avg)
        assert np.array_equal(f32_bits(sum_b), want_sum.view(np.uint32))


def test_owner_sum_update_empty_input(pkg, dev):
    from faster_yoco_amd import ops
    out = torch.empty(0, dtype=torch.bfloat16, device=dev)
    ws = ops.norm_workspace(dev, 1)
    s = scalars(dev)
    ops.owner_sum_update([out, out], out, 0.5, ws, factor=0.75, norm_out=s[0], grad_norm_out=s[1], factor_out=s[2],
                         max_norm=1.0)
    torch.cuda.synchronize()
    assert s[0].item() == 0.0 and s[1].item() == 0.0 and s[2].item() == 0.75


def test_set_grads_matches_a_new_table(pkg, dev):
    from faster_yoco_amd import ops
    sizes = [5000, 0, 1 << 14, 33]
    gen = torch.Generator(device='cpu').manual_seed(5)
    ps = [(torch.randn(n, generator=gen) * 0.02).to(dev) for n in sizes]
    ms = [(torch.randn(n, generator=gen) * 1e-4).to(dev) for n in sizes]
    vs = [(torch.randn(n, generator=gen) * 1e-8).abs().to(dev) for n in sizes]
    g1 = [(torch.randn(n, generator=gen) * 1e-3).to(dev) for n in sizes]
    raw = torch.zeros(sum(sizes) + 8, device=dev)          # new gradients, one of them off the vector alignment
    g2, off = [], 1
    for n in sizes:
        g2.append(raw[off:off + n])
        raw[off:off + n].copy_((torch.randn(n, generator=gen) * 1e-3).to(dev))
        off += n
    rows = lambda gs, P, M, V: [(g, p, m, v, None, g.numel()) for g, p, m, v in zip(gs, P, M, V)]
    ta = ops.Table(rows(g1, ps, ms, vs), dev)
    ta.set_grads(g2)
    P2, M2, V2 = ([t.clone() for t in X] for X in (ps, ms, vs))
    tb = ops.Table(rows(g2, P2, M2, V2), dev)
    args = (None, 3e-4, 0.9, 0.95, 1e-8, 0.5, 0.75, 0.1, 1)
    ops.adam_cast(ta, *args)
    ops.adam_cast(tb, *args)
    torch.cuda.synchronize()
    for X, Y in ((ps, P2), (ms, M2), (vs, V2)):
        for a, b in zip(X, Y):
            assert np.array_equal(f32_bits(a), f32_bits(b))
    with pytest.raises(RuntimeError, match='one tensor per table row'):
        ta.set_grads(g2[:-1])


def test_table_cache_rebinds_instead_of_rebuilding(pkg, dev):
    """Gradients reallocated every step (zero_grad drops them): one table build, every step right."""
    from faster_yoco_amd import ops
    cache = ops.TableCache(capacity=2)
    sizes = [4096, 333]
    p = [torch.zeros(n, device=dev) for n in sizes]
    m = [torch.zeros(n, device=dev) for n in sizes]
    v = [torch.zeros(n, device=dev) for n in sizes]
    state = [(np.zeros(n, np.float32),) * 3 for n in sizes]
    keep = []
    for step in range(1, 6):
        gs = [torch.randn(n, device=dev) * 1e-3 for n in sizes]
        keep.append(gs)                                    # distinct addresses every step
        rows = [(g, a, b, c, None, g.numel()) for g, a, b, c in zip(gs, p, m, v)]
        table = cache.get(rows, dev)
        bc1, bc2 = ops.bias_corrections(0.9, 0.95, step)
        ops.adam_cast(table, None, 3e-4, 0.9, 0.95, 1e-8, bc1, bc2, 0.1, 1, tensors=ops.rows_lists(rows))
        torch.cuda.synchronize()
        for i, g in enumerate(gs):
            po, mo, vo, _ = oracle.adam_cast(g.cpu().numpy(), *[x.copy() for x in state[i]], lr=3e-4, beta1=0.9,
                                             beta2=0.95, eps=1e-8, weight_decay=0.1, step=step)
            assert np.array_equal(f32_bits(p[i]), po.view(np.uint32))
            state[i] = (po, mo, vo)
    assert cache.builds == 1


def test_operators_follow_moved_state_tensors(pkg, dev):
    """The operator layer rebinds a table to whichever tensors a call passes: an update on copies of p, m, v (and a
    new gradient, and no BF16 copies) equals the same update on a table made on those copies; the original state is
    left untouched; a call naming an unknown table or tensors of the wrong size raises before any launch."""
    from faster_yoco_amd import ops
    Y = torch.ops.yoco_z1
    sizes = [5000, 0, 1 << 14, 33]
    gen = torch.Generator(device='cpu').manual_seed(9)
    mk = lambda s: [(torch.randn(n, generator=gen) * s).to(dev) for n in sizes]
    g, p, m, v = mk(1e-3), mk(0.02), mk(1e-4), [t.abs() for t in mk(1e-8)]
    p16 = [torch.zeros(n, dtype=torch.bfloat16, device=dev) for n in sizes]
    table = ops.Table([r + (r[0].numel(),) for r in zip(g, p, m, v, p16)], dev)
    keep = [[t.clone() for t in X] for X in (p, m, v, p16)]
    g2 = [t * 2 for t in g]
    P, M, V = ([t.clone() for t in X] for X in (p, m, v))
    args = (None, 3e-4, 0.9, 0.95, 1e-8, 0.5, 0.75, 0.1, 1, 0, len(sizes))
    Y.adam_cast_(table.handle_int, g2, P, M, V, [], *args)           # moved: every stream, BF16 copies off
    P2, M2, V2 = ([t.clone() for t in X] for X in (p, m, v))
    fresh = ops.Table([(a, b, c, d, None, a.numel()) for a, b, c, d in zip(g2, P2, M2, V2)], dev)
    Y.adam_cast_(fresh.handle_int, g2, P2, M2, V2, [], *args)
    torch.cuda.synchronize()
    for X, Z in ((P, P2), (M, M2), (V, V2)):
        for a, b in zip(X, Z):
            assert np.array_equal(f32_bits(a), f32_bits(b))
    for X, K in zip((p, m, v, p16), keep):                            # the tensors the table was made on
        for a, b in zip(X, K):
            assert torch.equal(a, b)
    Y.adam_cast_(table.handle_int, g, p, m, v, p16, *args)            # and back to them
    torch.cuda.synchronize()
    assert not torch.equal(p[0], keep[0][0]) and p16[0].abs().sum() > 0
    with pytest.raises(RuntimeError, match='no live table'):
        Y.adam_cast_(12345, g, p, m, v, p16, *args)
    with pytest.raises(RuntimeError, match='row 0 has 4999 elements, the table 5000'):
        Y.adam_cast_(table.handle_int, [g[0][1:]] + g[1:], p, m, v, p16, *args)
    with pytest.raises(RuntimeError, match='rows \\[0, 9\\) outside'):
        Y.adam_cast_(table.handle_int, g, p, m, v, p16, *args[:-1], 9)


@pytest.mark.parametrize('mode', [1, 0])
def test_adam_writes_the_scaled_gradients(pkg, dev, mode):
    """adam_cast with FP32 gradient outputs (z1_table_set_grad_out): BF16 gradients read times the factor, every
    output row holding fp32(float(g16) * factor) bit for bit as the scale pass writes it, and m / v / master / BF16
    copy as scale pass + Adam give them.  Rows: aligned, an output off the 16-byte alignment (element-wise path), a
    row without an output, an empty row, tails.  A later launch without outputs leaves them untouched."""
    from faster_yoco_amd import ops
    sizes = [5000, 256 * 9, 0, 33, 1 << 14]
    gen = torch.Generator(device='cpu').manual_seed(21 + mode)
    g16 = [(torch.randn(n, generator=gen) * 1e-2).to(torch.bfloat16).to(dev) for n in sizes]
    p = [(torch.randn(n, generator=gen) * 0.02).to(dev) for n in sizes]
    m = [(torch.randn(n, generator=gen) * 1e-4).to(dev) for n in sizes]
    v = [(torch.randn(n, generator=gen) * 1e-8).abs().to(dev) for n in sizes]
    p16 = [torch.zeros(n, dtype=torch.bfloat16, device=dev) for n in sizes]
    raw = torch.full((sum(sizes) + 8,), -7.0, device=dev)
    outs, off = [], 1                                       # row 1's output is 4 bytes off the vector alignment
    for i, n in enumerate(sizes):
        outs.append(torch.empty(0, device=dev) if i == 3 else raw[off:off + n])
        off += n
    outs[0] = torch.full((sizes[0],), -7.0, device=dev)     # row 0: an aligned output of its own
    keep = [(g.view(torch.int16).cpu().numpy().view(np.uint16).copy(), a.cpu().numpy().copy(),
             b.cpu().numpy().copy(), c.cpu().numpy().copy()) for g, a, b, c in zip(g16, p, m, v)]
    factor = torch.tensor([0.37], device=dev)
    fac = float(factor.item())
    table = ops.Table([r + (r[0].numel(),) for r in zip(g16, p, m, v, p16)], dev)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    bc1, bc2 = ops.bias_corrections(hp['beta1'], hp['beta2'], 7)
    ops.adam_cast(table, factor, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2, hp['weight_decay'], mode,
                  g32=outs)
    torch.cuda.synchronize()
    for i, (gb, p0, m0, v0) in enumerate(keep):
        po, mo, vo, p16o = oracle.adam_cast(gb, p0, m0, v0, step=7, mode=mode, factor=fac, **hp)
        assert np.array_equal(f32_bits(p[i]), po.view(np.uint32)), i
        assert np.array_equal(f32_bits(m[i]), mo.view(np.uint32)), i
        assert np.array_equal(f32_bits(v[i]), vo.view(np.uint32)), i
        assert np.array_equal(p16[i].view(torch.int16).cpu().numpy().view(np.uint16), p16o), i
        if i != 3:
            assert np.array_equal(f32_bits(outs[i]), oracle.scale_up(gb, fac).view(np.uint32)), i
    assert raw[0].item() == -7.0 and raw[-1].item() == -7.0       # nothing written outside the outputs
    for o in outs:
        o.fill_(-7.0)
    ops.adam_cast(table, factor, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2, hp['weight_decay'], mode)
    torch.cuda.synchronize()
    assert all(bool((o == -7.0).all()) for o in outs)              # outputs cleared for a launch without them
    with pytest.raises(RuntimeError, match='row 0 has 4999 elements'):
        ops.adam_cast(table, factor, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2, hp['weight_decay'],
                      mode, g32=[outs[0][1:]] + outs[1:])


@pytest.mark.parametrize('nrows', [20, 90])
def test_gradient_outputs_either_side_of_the_row_search(pkg, dev, nrows):
    """BF16 gradients x factor in, FP32 gradients written, over tables whose rows are found by binary search (up to
    64 rows) and from the chunk -> row map (more): each row's output is the one of its own row (rows without an
    output, empty rows and sizes off the chunk among them), bit-exact, and nothing is written outside them."""
    from faster_yoco_amd import ops
    rng = np.random.default_rng(40 + nrows)
    sizes = [0 if i % 13 == 5 else int(n) for i, n in enumerate(rng.integers(1, 2500, nrows))]
    gen = torch.Generator(device='cpu').manual_seed(nrows)
    g16 = [(torch.randn(n, generator=gen) * 1e-2).to(torch.bfloat16).to(dev) for n in sizes]
    p = [(torch.randn(n, generator=gen) * 0.02).to(dev) for n in sizes]
    m = [(torch.randn(n, generator=gen) * 1e-4).to(dev) for n in sizes]
    v = [(torch.randn(n, generator=gen) * 1e-8).abs().to(dev) for n in sizes]
    p16 = [torch.zeros(n, dtype=torch.bfloat16, device=dev) for n in sizes]
    raw = torch.full((sum(sizes) + 2,), -7.0, device=dev)
    outs, off = [], 1
    for i, n in enumerate(sizes):
        outs.append(torch.empty(0, device=dev) if i % 7 == 3 else raw[off:off + n])
        off += n
    keep = [(g.view(torch.int16).cpu().numpy().view(np.uint16).copy(), a.cpu().numpy().copy(),
             b.cpu().numpy().copy(), c.cpu().numpy().copy()) for g, a, b, c in zip(g16, p, m, v)]
    factor = torch.tensor([0.71], device=dev)
    fac = float(factor.item())
    table = ops.Table([r + (r[0].numel(),) for r in zip(g16, p, m, v, p16)], dev)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    bc1, bc2 = ops.bias_corrections(hp['beta1'], hp['beta2'], 4)
    ops.adam_cast(table, factor, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2, hp['weight_decay'], 1,
                  g32=outs)
    torch.cuda.synchronize()
    for i, (gb, p0, m0, v0) in enumerate(keep):
        po, mo, vo, p16o = oracle.adam_cast(gb, p0, m0, v0, step=4, mode=1, factor=fac, **hp)
        assert np.array_equal(f32_bits(p[i]), po.view(np.uint32)), i
        assert np.array_equal(f32_bits(m[i]), mo.view(np.uint32)), i
        assert np.array_equal(f32_bits(v[i]), vo.view(np.uint32)), i
        assert np.array_equal(p16[i].view(torch.int16).cpu().numpy().view(np.uint16), p16o), i
        if i % 7 != 3:
            assert np.array_equal(f32_bits(outs[i]), oracle.scale_up(gb, fac).view(np.uint32)), i
    assert raw[0].item() == -7.0 and raw[-1].item() == -7.0
    for i, n in enumerate(sizes):                        # the rows without an output left their span of raw alone
        if i % 7 == 3 and n:
            o = 1 + sum(sizes[:i])
            assert bool((raw[o:o + n] == -7.0).all()), i
    table.close()


@pytest.mark.parametrize('total', [300_000, 150_000_000])
def test_bf16_norm_pass(pkg, dev, total):
    """The norm pass over BF16 gradients (chunk pairs, one 128-bit load per lane where a pair is whole and aligned,
    the two chunks one after the other elsewhere): rows off the vector alignment, short rows, an empty row and, at
    150M elements, the allocating loads of the MALL-kept part.  Its partials are the same bits on every run, their
    FP64 total is the FP32 pass's over the upcast values and the oracle's sequential sum to 1e-10 (sums of the same
    exact squares in other orders), and the norm is within 1e-6 of the exact one."""
    from faster_yoco_amd import ops
    gen = torch.Generator(device='cpu').manual_seed(total % 1000)
    raw16 = (torch.randn(total + 64, generator=gen) * 1e-2).to(torch.bfloat16).to(dev)
    raw32 = raw16.float()
    cuts = [0, 1, 777, 5001, total // 3, total // 3 + 1, total // 3 + 1, total // 2 + 3, total]
    rows16, rows32 = [], []
    for a, b in zip(cuts, cuts[1:]):
        rows16.append((raw16[a:b], None, None, None, None, b - a))
        rows32.append((raw32[a:b], None, None, None, None, b - a))
    t16 = ops.Table(rows16, dev)
    p16, again, p32 = ops.norm_workspace(dev), ops.norm_workspace(dev), ops.norm_workspace(dev)
    ops.grad_sumsq(t16, p16)
    ops.grad_sumsq(t16, again)
    ops.grad_sumsq(ops.Table(rows32, dev), p32)
    torch.cuda.synchronize()
    assert torch.equal(p16.view(torch.int64), again.view(torch.int64))
    s16, s32 = float(p16.sum()), float(p32.sum())
    seq = oracle.sumsq(raw16[:total].view(torch.int16).cpu().numpy().view(np.uint16))
    assert abs(s16 - s32) <= 1e-10 * s32 and abs(s16 - seq) <= 1e-10 * seq
    exact = float(np.sqrt(seq))
    assert abs(float(np.sqrt(s16)) - exact) <= 1e-6 * exact
