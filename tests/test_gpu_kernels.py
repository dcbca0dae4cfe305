"""GPU parity of the HIP kernels against the CPU oracle on identical seeded inputs (small and C1 sizes).

Bars: owner sum, scale, BF16 copy, Adam m / v / master: bit-exact (NaN compared as NaN); norm: within 1 fp32 ulp
of the correctly rounded exact norm (the stated bar is 1e-6 relative); clip chain: bit-exact given the GPU's norm.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)


def dev_f32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def dev_bf16(h, device):
    return torch.from_numpy(np.ascontiguousarray(h, dtype=np.uint16).view(np.int16)).to(device).view(torch.bfloat16)


def host_bf16(t):
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def host_f32(t):
    return t.detach().cpu().numpy()


def same_f32(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))


def same_bf16(a, b):
    a, b = np.asarray(a, np.uint16), np.asarray(b, np.uint16)
    nan_a = (a & 0x7fff) > 0x7f80
    nan_b = (b & 0x7fff) > 0x7f80
    return np.array_equal(nan_a, nan_b) and np.array_equal(a[~nan_a], b[~nan_a])


def rand_state(n, seed, step1=False, gscale=1e-3):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * gscale).astype(np.float32)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    m = np.zeros(n, np.float32) if step1 else (rng.standard_normal(n) * 1e-4).astype(np.float32)
    v = np.zeros(n, np.float32) if step1 else np.abs(rng.standard_normal(n) * 1e-8).astype(np.float32)
    return g, p, m, v


def run_adam_rows(pkg, dev, rows_np, g_bf16, factor, step, mode=1, with_p16=True, hp=HP, misalign=0):
    """rows_np: list of (g, p, m, v) NumPy arrays; g is uint16 bits when g_bf16.  Runs one table launch and
    returns per row (p, m, v, p16) host arrays.  misalign > 0 shifts every row start by that many elements."""
    from faster_yoco_amd import ops
    keep, rows = [], []
    for g, p, m, v in rows_np:
        n = p.size
        o = misalign
        gt = (dev_bf16(np.concatenate([np.zeros(o, np.uint16), g]), dev) if g_bf16
              else dev_f32(np.concatenate([np.zeros(o, np.float32), g]), dev))[o:]
        pt = dev_f32(np.concatenate([np.zeros(o, np.float32), p]), dev)[o:]
        mt = dev_f32(np.concatenate([np.zeros(o, np.float32), m]), dev)[o:]
        vt = dev_f32(np.concatenate([np.zeros(o, np.float32), v]), dev)[o:]
        p16 = torch.zeros(n + o, dtype=torch.bfloat16, device=dev)[o:] if with_p16 else None
        keep.append((gt, pt, mt, vt, p16))
        rows.append((gt, pt, mt, vt, p16, n))
    table = ops.Table(rows, dev)
    bc1, bc2 = ops.bias_corrections(hp['beta1'], hp['beta2'], step)
    f = None if factor is None else torch.tensor([factor], dtype=torch.float32, device=dev)
    ops.adam_cast(table, f, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2, hp['weight_decay'], mode)
    torch.cuda.synchronize()
    out = [(host_f32(pt), host_f32(mt), host_f32(vt), host_bf16(p16) if p16 is not None else None)
           for _, pt, mt, vt, p16 in keep]
    table.close()
    return out


def check_rows(rows_np, got, g_bf16, factor, step, mode=1, hp=HP):
    for (g, p, m, v), (gp, gm, gv, g16) in zip(rows_np, got):
        po, mo, vo, p16 = oracle.adam_cast(g, p, m, v, lr=hp['lr'], beta1=hp['beta1'], beta2=hp['beta2'],
                                           eps=hp['eps'], weight_decay=hp['weight_decay'], step=step, mode=mode,
                                           factor=factor)
        assert same_f32(gm, mo), 'exp_avg differs'
        assert same_f32(gv, vo), 'exp_avg_sq differs'
        assert same_f32(gp, po), f'master differs in {int(np.sum(gp.view(np.uint32) != po.view(np.uint32)))} places'
        if g16 is not None:
            assert same_bf16(g16, p16), 'bf16 copy differs'


# ---------------------------------------------------------------------------------------------- Adam + BF16
@pytest.mark.parametrize('mode', [1, 0])
@pytest.mark.parametrize('g_bf16', [False, True])
def test_adam_c1_shapes_bit_exact(pkg, dev, mode, g_bf16):
    from faster_yoco_amd import configs
    rows = []
    for i, s in enumerate(configs.C1_SHAPES):
        n = int(np.prod(s))
        g, p, m, v = rand_state(n, 100 + i, step1=True)
        rows.append((oracle.bf16_rne(g) if g_bf16 else g, p, m, v))
    got = run_adam_rows(pkg, dev, rows, g_bf16, factor=0.3255, step=1, mode=mode)
    check_rows(rows, got, g_bf16, 0.3255, 1, mode)


@pytest.mark.parametrize('step', [2, 1000])
def test_adam_nonzero_moments_and_tails(pkg, dev, step):
    # sizes around the chunk and vector widths exercise full chunks, partial chunks and element tails
    sizes = [1, 3, 4, 5, 255, 256, 1023, 4095, 4096, 4097, 8191, 12289, 70001]
    rows = [rand_state(n, 200 + i) for i, n in enumerate(sizes)]
    got = run_adam_rows(pkg, dev, rows, False, factor=None, step=step)
    check_rows(rows, got, False, None, step)


@pytest.mark.parametrize('nrows', [63, 64, 65, 200])
@pytest.mark.parametrize('g_bf16', [False, True])
def test_adam_tables_either_side_of_the_row_search(pkg, dev, nrows, g_bf16):
    """A wave finds its chunk's row by binary search in tables of up to 64 rows and from the chunk -> row map in
    larger ones: rows of random sizes (below one chunk, off the 256-element chunk, several chunks), bit-exact."""
    rng = np.random.default_rng(900 + nrows)
    sizes = rng.integers(1, 3000, nrows)
    rows = []
    for i, n in enumerate(sizes):
        g, p, m, v = rand_state(int(n), 1000 + i)
        rows.append((oracle.bf16_rne(g) if g_bf16 else g, p, m, v))
    got = run_adam_rows(pkg, dev, rows, g_bf16, factor=0.8125, step=12)
    check_rows(rows, got, g_bf16, 0.8125, 12)


def test_adam_misaligned_rows_use_the_element_path(pkg, dev):
    sizes = [4096 * 3, 5000, 17]
    rows = [rand_state(n, 300 + i) for i, n in enumerate(sizes)]
    for off in (1, 2, 3):
        got = run_adam_rows(pkg, dev, rows, False, factor=0.75, step=10, misalign=off)
        check_rows(rows, got, False, 0.75, 10)


def flat_rows(rows_np, g_bf16, dev, with_p16=True):
    """The rows in one allocation per stream, in order and without gaps (the flat shard's layout): the flat
    buffers and per-row views of them."""
    cat = lambda k: np.concatenate([r[k] for r in rows_np])
    G = dev_bf16(cat(0), dev) if g_bf16 else dev_f32(cat(0), dev)
    P, M, V = dev_f32(cat(1), dev), dev_f32(cat(2), dev), dev_f32(cat(3), dev)
    P16 = torch.zeros(P.numel(), dtype=torch.bfloat16, device=dev) if with_p16 else None
    views, off = [], 0
    for r in rows_np:
        n = r[1].size
        sl = slice(off, off + n)
        views.append((G[sl], P[sl], M[sl], V[sl], P16[sl] if with_p16 else None, n))
        off += n
    return (G, P, M, V, P16), views


def host_rows(views):
    return [(host_f32(p), host_f32(m), host_f32(v), host_bf16(p16) if p16 is not None else None)
            for _, p, m, v, p16, _ in views]


@pytest.mark.parametrize('with_p16', [True, False])
@pytest.mark.parametrize('mode', [1, 0])
@pytest.mark.parametrize('g_bf16', [False, True])
def test_adam_contiguous_rows_take_the_flat_launch(pkg, dev, g_bf16, mode, with_p16):
    """Rows that tile one allocation per stream in order (the flat shard) are updated by the launch that walks the
    buffers directly; its chunks straddle the rows' boundaries where sizes are not multiples of 256.  Bit-exact
    against the oracle, as the table walk over the same rows in separate allocations is."""
    from faster_yoco_amd import ops
    sizes = [1000, 333, 4096, 7777, 256, 5, 70001]
    rows = []
    for i, n in enumerate(sizes):
        g, p, m, v = rand_state(n, 500 + i)
        rows.append((oracle.bf16_rne(g) if g_bf16 else g, p, m, v))
    (G, P, M, V, P16), views = flat_rows(rows, g_bf16, dev, with_p16)
    offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]).tolist()
    table = ops.Table.flat(offsets, sizes, G, P, M, V, P16)
    bc1, bc2 = ops.bias_corrections(HP['beta1'], HP['beta2'], 7)
    f = torch.tensor([0.625], dtype=torch.float32, device=dev)
    ops.adam_cast(table, f, HP['lr'], HP['beta1'], HP['beta2'], HP['eps'], bc1, bc2, HP['weight_decay'], mode)
    torch.cuda.synchronize()
    got = host_rows(views)
    check_rows(rows, got, g_bf16, 0.625, 7, mode)
    table.close()
    sep = run_adam_rows(pkg, dev, rows, g_bf16, factor=0.625, step=7, mode=mode, with_p16=with_p16)
    for a, b in zip(got, sep):
        assert all(same_f32(x, y) for x, y in zip(a[:3], b[:3]))
        assert (a[3] is None) == (b[3] is None) and (a[3] is None or same_bf16(a[3], b[3]))


def test_adam_table_rebound_between_flat_and_separate_rows(pkg, dev):
    """One list table bound in turn to views of flat buffers (the launch that walks the buffers), to separately
    allocated tensors (the table walk), and to the flat views again: every update bit-exact against the oracle.
    Whether a launch may walk the buffers directly follows the addresses of each call."""
    from faster_yoco_amd import ops
    sizes = [3000, 1, 4096 + 17, 513]
    rows = [rand_state(n, 600 + i) for i, n in enumerate(sizes)]
    _, views = flat_rows(rows, False, dev)
    sep = [(dev_f32(g, dev), dev_f32(p, dev), dev_f32(m, dev), dev_f32(v, dev),
            torch.zeros(p.size, dtype=torch.bfloat16, device=dev), p.size) for g, p, m, v in rows]
    table = ops.Table(sep, dev)
    bc1, bc2 = ops.bias_corrections(HP['beta1'], HP['beta2'], 3)
    want = rows
    for k, bound in enumerate((views, sep, views)):
        ops.adam_cast(table, None, HP['lr'], HP['beta1'], HP['beta2'], HP['eps'], bc1, bc2, HP['weight_decay'], 1,
                      tensors=ops.rows_lists(bound))
        torch.cuda.synchronize()
        got = host_rows(bound)
        check_rows(want, got, False, None, 3)
        # the next binding's inputs: these outputs (p, m, v) with the same gradients
        want = [(g, gp, gm, gv) for (g, _, _, _), (gp, gm, gv, _) in zip(rows, got)]
        if k < 2:
            nxt = (sep, views)[k]
            for (_, p, m, v, _, _), (gp, gm, gv, _) in zip(nxt, got):
                p.copy_(torch.from_numpy(gp))
                m.copy_(torch.from_numpy(gm))
                v.copy_(torch.from_numpy(gv))
    table.close()


def test_adam_flat_rows_with_gradients_moved_apart(pkg, dev):
    """A table over views of flat buffers whose gradients are then given as separate allocations (the operators
    rebind only the gradient column, as when autograd reallocates gradients): the rows are no longer one allocation
    per stream, so the launch walks the table; then the gradients move into another flat buffer and the launch walks
    the buffers again.  Bit-exact against the oracle each time."""
    from faster_yoco_amd import ops
    sizes = [2048, 777, 4096, 300]
    rows = [rand_state(n, 700 + i) for i, n in enumerate(sizes)]
    (G, _, _, _, _), views = flat_rows(rows, False, dev)
    table = ops.Table(views, dev)
    bc1, bc2 = ops.bias_corrections(HP['beta1'], HP['beta2'], 5)
    G2 = G.clone()
    offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]).tolist()
    want = rows
    for grads in ([v[0] for v in views], [dev_f32(r[0], dev) for r in rows],
                  [G2[o:o + n] for o, n in zip(offsets, sizes)]):
        tensors = (grads, [v[1] for v in views], [v[2] for v in views], [v[3] for v in views],
                   [v[4] for v in views])
        ops.adam_cast(table, None, HP['lr'], HP['beta1'], HP['beta2'], HP['eps'], bc1, bc2, HP['weight_decay'], 1,
                      tensors=tensors)
        torch.cuda.synchronize()
        got = host_rows(views)
        check_rows(want, got, False, None, 5)
        want = [(g, gp, gm, gv) for (g, _, _, _), (gp, gm, gv, _) in zip(rows, got)]
    table.close()


def test_adam_without_bf16_copy_and_special_values(pkg, dev):
    n = 4096 * 2 + 100
    g, p, m, v = rand_state(n, 400)
    g[:8] = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-45, 3e38, -3e38]
    m[8:40] = np.float32(1e-41)            # subnormal moments
    v[8:40] = np.float32(1e-44)
    v[40:48] = 0.0
    g[40:48] = 0.0
    p[48:56] = [0.0, -0.0, 1e-40, -1e-40, 3e38, -3e38, 1.0, -1.0]
    rows = [(g, p, m, v)]
    got = run_adam_rows(pkg, dev, rows, False, factor=None, step=3, with_p16=False)
    check_rows(rows, got, False, None, 3)
    got = run_adam_rows(pkg, dev, rows, False, factor=0.5, step=3, with_p16=True)
    check_rows(rows, got, False, 0.5, 3)


def test_adam_hyperparameter_variants(pkg, dev):
    rows = [rand_state(9000, 500)]
    for hp in (dict(HP, lr=0.0), dict(HP, weight_decay=0.0), dict(HP, beta2=0.999, eps=1e-6),
               dict(HP, lr=1e-2, weight_decay=0.01)):
        for mode in (0, 1):
            got = run_adam_rows(pkg, dev, rows, False, factor=None, step=7, mode=mode, hp=hp)
            check_rows(rows, got, False, None, 7, mode, hp=hp)


def test_adam_runs_twice_identically_and_empty_tables(pkg, dev):
    from faster_yoco_amd import ops
    rows = [rand_state(50000, 600)]
    a = run_adam_rows(pkg, dev, rows, False, factor=0.9, step=5)
    b = run_adam_rows(pkg, dev, rows, False, factor=0.9, step=5)
    assert all(np.array_equal(x.view(np.uint32), y.view(np.uint32)) for x, y in zip(a[0][:3], b[0][:3]))
    t = ops.Table([], dev)
    ops.adam_cast(t, None, 3e-4, 0.9, 0.95, 1e-8, 0.1, 0.05, 0.1, 1)
    z = torch.zeros(0, device=dev)
    t2 = ops.Table([(z, z, z, z, None, 0)], dev)
    ops.adam_cast(t2, None, 3e-4, 0.9, 0.95, 1e-8, 0.1, 0.05, 0.1, 1)
    torch.cuda.synchronize()


# ----------------------------------------------------------------------------------------------------- norm
def gpu_norm(pkg, dev, grads, factor=1.0, max_norm=1.0):
    """grads: list of NumPy arrays (float32 or uint16 bf16 bits).  Returns (n_r, grad_norm, factor_out)."""
    from faster_yoco_amd import ops
    ts = [dev_bf16(g, dev) if g.dtype == np.uint16 else dev_f32(g, dev) for g in grads]
    table = ops.Table([(t, None, None, None, None, t.numel()) for t in ts], dev)
    part = ops.norm_workspace(dev)
    ops.grad_sumsq(table, part)
    nr = torch.zeros(1, device=dev)
    gn = torch.zeros(1, device=dev)
    fo = torch.zeros(1, device=dev)
    ops.norm_clip(part, factor=factor, norm_out=nr, grad_norm_out=gn, factor_out=fo, max_norm=max_norm)
    torch.cuda.synchronize()
    return np.float32(nr.item()), np.float32(gn.item()), np.float32(fo.item())


def exact_norm(grads):
    return float(np.sqrt(sum(oracle.sumsq(g) for g in grads)))


@pytest.mark.parametrize('g_bf16', [False, True])
def test_norm_c1_within_one_ulp_and_clip_chain_bit_exact(pkg, dev, g_bf16):
    from faster_yoco_amd import configs
    grads = []
    for i, s in enumerate(configs.C1_SHAPES):
        g = rand_state(int(np.prod(s)), 700 + i)[0]
        grads.append(oracle.bf16_rne(g) if g_bf16 else g)
    nr, gn, fo = gpu_norm(pkg, dev, grads)
    ex = exact_norm(grads)
    assert oracle.ulp_diff_f32(nr, np.float32(ex)) <= 1 and abs(nr - ex) <= 1e-6 * ex
    _, gn_ref, fo_ref = oracle.norm_clip(float(nr) ** 2, 1.0, 1.0)
    assert gn == gn_ref and fo == fo_ref and fo < 1.0


def test_norm_heavy_tails_deterministic_and_scaling(pkg, dev):
    from faster_yoco_amd import configs
    h = configs.host_inputs(3 * 4096 * 7 + 13, 'c5', seed=5)
    g = h['g']
    grads = [g[:4096], g[4096:4096 * 20], g[4096 * 20:4096 * 20 + 3072], g[4096 * 20 + 3072:]]
    a = gpu_norm(pkg, dev, grads)
    b = gpu_norm(pkg, dev, grads)
    assert a == b                                    # run to run: bit identical
    ex = exact_norm(grads)
    assert abs(a[0] - ex) <= 1e-6 * ex and a[2] < 1e-3
    scaled = [x * np.float32(2.0 ** -7) for x in grads]
    assert gpu_norm(pkg, dev, scaled)[0] == a[0] * np.float32(2.0 ** -7)     # exact power-of-two scaling
    perm = [grads[2], grads[0], grads[3], grads[1]]
    assert abs(gpu_norm(pkg, dev, perm)[0] - ex) <= 1e-6 * ex


@pytest.mark.parametrize('nrows', [300, 511, 512, 513, 1000])
@pytest.mark.parametrize('g_bf16', [False, True])
def test_norm_over_many_rows(pkg, dev, nrows, g_bf16):
    """Tables of nrows device rows around the norm kernel's LDS staging of the rows' first chunks (up to 512; more
    fall back to the search from row 0), plus zero-size rows (absent from the device table), sizes off the
    256-element chunk, and the same rows as views of one buffer at odd offsets (BF16: not 8-byte aligned, the
    element-wise path): within 1 ulp of the exact norm, bit-identical on a second run."""
    from faster_yoco_amd import ops
    rng = np.random.default_rng(nrows + 7 * g_bf16)
    sizes = rng.integers(1, 1200, nrows)                 # nrows device rows
    sizes[rng.choice(nrows, nrows // 10, replace=False)] = 256 * rng.integers(1, 5, nrows // 10)
    sizes = np.insert(sizes, rng.integers(0, nrows + 1, nrows // 10), 0)   # and zero-size rows between them
    grads = []
    for i, n in enumerate(sizes):
        g = (rng.standard_normal(int(n)) * 10.0 ** rng.integers(-6, 1)).astype(np.float32)
        grads.append(oracle.bf16_rne(g) if g_bf16 else g)
    ex = exact_norm([g for g in grads if g.size])
    a = gpu_norm(pkg, dev, grads)
    assert gpu_norm(pkg, dev, grads) == a
    assert oracle.ulp_diff_f32(a[0], np.float32(ex)) <= 1
    # the same gradients as views of one buffer, each starting one element past the last
    flat = np.concatenate([np.zeros(1, grads[0].dtype)] + [np.concatenate([g, np.zeros(1, g.dtype)]) for g in grads])
    buf = dev_bf16(flat, dev) if g_bf16 else dev_f32(flat, dev)
    rows, o = [], 1
    for g in grads:
        rows.append((buf[o:o + g.size], None, None, None, None, g.size))
        o += g.size + 1
    table = ops.Table(rows, dev)
    part = ops.norm_workspace(dev)
    ops.grad_sumsq(table, part)
    nr = torch.zeros(1, device=dev)
    ops.norm_clip(part, norm_out=nr, max_norm=1.0)
    torch.cuda.synchronize()
    assert oracle.ulp_diff_f32(np.float32(nr.item()), np.float32(ex)) <= 1
    table.close()


def test_norm_edge_cases(pkg, dev):
    z = [np.zeros(1000, np.float32)]
    nr, gn, fo = gpu_norm(pkg, dev, z)
    assert nr == 0.0 and gn == 0.0 and fo == 1.0
    nr, gn, fo = gpu_norm(pkg, dev, [np.array([1.0, np.inf], np.float32)])
    assert np.isinf(nr) and fo == 0.0
    nr, gn, fo = gpu_norm(pkg, dev, [np.array([1.0, np.nan], np.float32)])
    assert np.isnan(nr) and np.isnan(fo)
    # max_norm <= 0: no clip, factor passes through
    g = [rand_state(5000, 800)[0]]
    nr, gn, fo = gpu_norm(pkg, dev, g, factor=0.25, max_norm=0.0)
    assert fo == np.float32(0.25) and gn == np.float32(0.25) * nr
    # a device factor tensor
    from faster_yoco_amd import ops
    t = dev_f32(g[0], dev)
    table = ops.Table([(t, None, None, None, None, t.numel())], dev)
    part = ops.norm_workspace(dev)
    ops.grad_sumsq(table, part)
    f = torch.tensor([2.0 ** -11 * 8], device=dev)
    gn_t = torch.zeros(1, device=dev)
    nr_t = torch.zeros(1, device=dev)
    ops.norm_clip(part, factor=f, norm_out=nr_t, grad_norm_out=gn_t, factor_out=f, max_norm=1.0)
    _, gn_ref, fo_ref = oracle.norm_clip(float(nr_t.item()) ** 2, 2.0 ** -11 * 8, 1.0)
    assert np.float32(gn_t.item()) == gn_ref and np.float32(f.item()) == fo_ref
    # the chain entered at a given norm
    gn2 = torch.zeros(1, device=dev)
    fo2 = torch.zeros(1, device=dev)
    ops.clip_factor(torch.tensor([3.5], device=dev), factor=0.5, grad_norm_out=gn2, factor_out=fo2, max_norm=1.0)
    ref = oracle.clip_factor(3.5, 0.5, 1.0)
    assert np.float32(gn2.item()) == ref[0] and np.float32(fo2.item()) == ref[1]


# ------------------------------------------------------------------------------------------------ owner sum
@pytest.mark.parametrize('world', [1, 3, 8, 9, 16])
def test_owner_sum_bit_exact(pkg, dev, world):
    from faster_yoco_amd import ops
    rng = np.random.default_rng(world)
    n = 8 * 4096 + 5
    cs = [oracle.bf16_rne((rng.standard_normal(n) * 1e-4).astype(np.float32)) for _ in range(world)]
    cs[0][:3] = [0x8000, 0x7f80, 0xff80]             # -0, +inf, -inf
    for c in cs:
        c[3] = 0x8000
    avg, s = oracle.owner_sum(cs, want_sum=True)
    ts = [dev_bf16(c, dev) for c in cs]
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    osum = torch.empty(n, dtype=torch.float32, device=dev)
    part = ops.norm_workspace(dev, n)
    ops.owner_sum(ts, out, 1.0 / world, out_sum=osum, partials=part)
    nr = torch.zeros(1, device=dev)
    ops.norm_clip(part, norm_out=nr)
    torch.cuda.synchronize()
    assert same_bf16(host_bf16(out), avg)
    assert same_f32(host_f32(osum), s)
    fin = [c[5:] for c in cs]                       # the norm of the finite part
    ts = [dev_bf16(c, dev) for c in fin]
    out2 = torch.empty(n - 5, dtype=torch.bfloat16, device=dev)
    ops.owner_sum(ts, out2, 1.0 / world, partials=part)
    ops.norm_clip(part, norm_out=nr)
    ex = float(np.sqrt(oracle.sumsq(oracle.owner_sum(fin))))
    assert abs(float(nr.item()) - ex) <= 1e-6 * ex


# sizes at the edges of the owner sum's chunk count (one partial per 256-element chunk of a grid shifted by up to 63
# elements: 193 / 194, 449 / 450 elements need one more chunk), with the streams aligned or 134 bytes into a line
@pytest.mark.parametrize('n', [1, 193, 194, 255, 256, 257, 449, 450, 65536 + 63])
@pytest.mark.parametrize('offset', [0, 67])
def test_owner_sum_at_chunk_count_edges(pkg, dev, n, offset):
    """The average, the fp32 sum and the fused norm against the oracle, at sizes where the last chunk is whole,
    partial or empty for the grid the streams' offset gives."""
    from faster_yoco_amd import ops
    rng = np.random.default_rng(n + offset)
    world = 2
    cs = [(rng.integers(0x3000, 0x4000, n, dtype=np.uint16) | (rng.integers(0, 2, n, dtype=np.uint16) << 15))
          .astype(np.uint16) for _ in range(world)]
    avg, s = oracle.owner_sum(cs, want_sum=True)
    ts = []
    for c in cs:
        buf = torch.zeros(n + 128, dtype=torch.bfloat16, device=dev)
        buf[offset:offset + n].copy_(dev_bf16(c, dev))
        ts.append(buf[offset:offset + n])
    out = torch.zeros(n + 128, dtype=torch.bfloat16, device=dev)[offset:offset + n]
    osum = torch.zeros(n + 128, dtype=torch.float32, device=dev)[offset:offset + n]
    part = ops.norm_workspace(dev, n)
    ops.owner_sum(ts, out, 1.0 / world, out_sum=osum, partials=part)
    nr = torch.zeros(1, device=dev)
    ops.norm_clip(part, norm_out=nr)
    torch.cuda.synchronize()
    assert same_bf16(host_bf16(out), avg)
    assert same_f32(host_f32(osum), s)
    ex = float(np.sqrt(oracle.sumsq(avg)))
    assert abs(float(nr.item()) - ex) <= 1e-6 * ex


def test_owner_sum_in_place_reference_slot_layout(pkg, dev):
    from faster_yoco_amd import ce_reduce
    rng = np.random.default_rng(9)
    W, G = 8, 3 * 4096 + 77
    for R, base, end in ((0, 0, G), (3, 1000, 9001), (7, 5, G - 3), (5, 17, 18)):
        S = oracle.bf16_rne((rng.standard_normal((W - 1) * G) * 1e-3).astype(np.float32))
        OUT = oracle.bf16_rne((rng.standard_normal(G) * 1e-3).astype(np.float32))
        exp = oracle.sum_slots(S, OUT.copy(), G, base, end, R, 1.0 / W, W)
        St, Ot = dev_bf16(S, dev), dev_bf16(OUT, dev)
        ce_reduce.sum_slots(St, Ot, G, base, end, R, 1.0 / W, W)
        torch.cuda.synchronize()
        assert np.array_equal(host_bf16(Ot), exp), (R, base, end)
        assert np.array_equal(host_bf16(St), S)


# element offsets (average, contributions, fp32 sum) of the streams inside 512-byte-aligned allocations
MISALIGNED = {
    'lines_shared_2B': (1, (1, 1, 1, 1), 1),          # every stream 2 bytes into a line: the grid moves by 1
    'lines_shared_134B': (67, (67, 67, 67, 67), 67),  # 6 bytes into the second line of each
    'lines_apart_by_128B': (5, (69, 5, 133, 5), None),
    'words_shared': (1, (5, 1, 9, 13), None),          # same offset within 8-byte words only
    'no_common_word': (1, (2, 1, 1, 1), None),         # element-wise path
    'fp32_sum_off_grid': (1, (1, 1, 1, 1), 0),         # the fp32 sum not 16-byte aligned on the grid: element path
}


@pytest.mark.parametrize('case', sorted(MISALIGNED))
def test_owner_sum_misaligned_ranges(pkg, dev, case):
    """Streams that start off the 16-byte boundaries -- a CEReduce phase starts at any parameter boundary of the
    owner's gradient: the chunk grid follows the offset the streams share (a 128-byte line offset, else an 8-byte
    word offset, else the element-wise path); the average and the fp32 sum stay bit-exact, the fused norm within
    1e-6 of the exact one."""
    from faster_yoco_amd import ops
    oo, co, so = MISALIGNED[case]
    rng = np.random.default_rng(len(case))
    n = 3 * 4096 + 45
    cs = [oracle.bf16_rne((rng.standard_normal(n) * 1e-3).astype(np.float32)) for _ in co]
    avg, s = oracle.owner_sum(cs, want_sum=True)
    ts = []
    for c, off in zip(cs, co):
        buf = torch.zeros(n + 256, dtype=torch.bfloat16, device=dev)
        buf[off:off + n].copy_(dev_bf16(c, dev))
        ts.append(buf[off:off + n])
    out = torch.zeros(n + 256, dtype=torch.bfloat16, device=dev)[oo:oo + n]
    osum = None if so is None else torch.zeros(n + 256, dtype=torch.float32, device=dev)[so:so + n]
    part = ops.norm_workspace(dev, n)
    ops.owner_sum(ts, out, 1.0 / len(cs), out_sum=osum, partials=part)
    nr = torch.zeros(1, device=dev)
    ops.norm_clip(part, norm_out=nr)
    torch.cuda.synchronize()
    assert same_bf16(host_bf16(out), avg)
    if osum is not None:
        assert same_f32(host_f32(osum), s)
    ex = float(np.sqrt(oracle.sumsq(avg)))
    assert abs(float(nr.item()) - ex) <= 1e-6 * ex


def test_sum_slots_phase_partials_give_the_norm_of_the_whole_average(pkg, dev):
    """CEReduce's phases at odd bounds, each summed in place with its norm partials left in its own slice of one
    array (sum_slots' waves), then one fixed-order reduction: the average bit-exact against the oracle, the norm
    within one fp32 ulp of the norm pass over the same BF16 average (and within 1e-6 of the exact norm), and the
    same bits when the phases run again."""
    from faster_yoco_amd import ce_reduce, ops
    rng = np.random.default_rng(21)
    W, R, G = 8, 5, 5 * 4096 + 321
    bounds = [(0, 4099), (4099, 4099), (4099, 12001), (12001, G)]
    S = oracle.bf16_rne((rng.standard_normal((W - 1) * G) * 1e-3).astype(np.float32))
    OUT = oracle.bf16_rne((rng.standard_normal(G) * 1e-3).astype(np.float32))
    exp = OUT.copy()
    counts = [ops.owner_sum_waves(b - a) for a, b in bounds]
    waves = torch.full((sum(counts),), np.nan, dtype=torch.float64, device=dev)
    norms = []
    for rep in range(2):
        St, Ot = dev_bf16(S, dev), dev_bf16(OUT, dev)
        off = 0
        for (a, b), c in zip(bounds, counts):
            ce_reduce.sum_slots(St, Ot, G, a, b, R, 1.0 / W, W, waves=waves[off:off + c])
            if rep == 0:
                oracle.sum_slots(S, exp, G, a, b, R, 1.0 / W, W)
            off += c
        part = ops.norm_workspace(dev)
        ops.reduce_waves(waves, off, part)
        nr = torch.zeros(1, device=dev)
        ops.norm_clip(part, norm_out=nr)
        torch.cuda.synchronize()
        assert np.array_equal(host_bf16(Ot), exp)
        norms.append(np.float32(nr.item()))
    assert norms[0].view(np.uint32) == norms[1].view(np.uint32)
    ex = float(np.sqrt(oracle.sumsq(exp)))
    assert abs(float(norms[0]) - ex) <= 1e-6 * ex
    table = ops.Table([(Ot, None, None, None, None, G)], dev)
    ref = torch.zeros(1, device=dev)
    part = ops.norm_workspace(dev)
    ops.grad_sumsq(table, part)
    ops.norm_clip(part, norm_out=ref)
    torch.cuda.synchronize()
    d = abs(int(np.float32(ref.item()).view(np.int32)) - int(norms[0].view(np.int32)))
    assert d <= 1, (float(ref.item()), float(norms[0]))


# ---------------------------------------------------------------------------------------------- scale / cast
def test_scale_up_and_cast_bit_exact(pkg, dev):
    from faster_yoco_amd import fused_adam_cast, ops
    rng = np.random.default_rng(10)
    for n, off in ((8 * 1000, 0), (8 * 1000 + 3, 0), (777, 1)):
        g16 = oracle.bf16_rne((rng.standard_normal(n + off) * 1e-3).astype(np.float32))
        gt = dev_bf16(g16, dev)[off:]
        out = torch.empty(n + off, dtype=torch.float32, device=dev)[off:]
        f = torch.tensor([0.482], device=dev)
        fused_adam_cast.scale_up(gt, out, f)
        torch.cuda.synchronize()
        assert same_f32(host_f32(out), oracle.scale_up(g16[off:], 0.482))
        p = (rng.standard_normal(n + off) * 0.02).astype(np.float32)
        p[:4] = [np.nan, np.inf, 1e-40, -0.0]
        pt = dev_f32(p, dev)[off:]
        o16 = torch.empty(n + off, dtype=torch.bfloat16, device=dev)[off:]
        ops.cast_bf16(pt, o16)
        torch.cuda.synchronize()
        assert same_bf16(host_bf16(o16), oracle.bf16_rne(p[off:]))
