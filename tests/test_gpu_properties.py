"""Property-based GPU parity (hypothesis): random tensor tables -- row counts, ragged sizes (including 0 and tails),
per-array misalignment, bf16 or fp32 gradients, with or without BF16 copies and FP32 gradient outputs, both Adam
modes, random factors and steps -- random owner sums (world 1..16, odd lengths, offsets), norms of random tables with the clip chain, the
embedding gradient over random ids, widths, padding and scale placements, and the scale / cast passes at random
sizes and offsets; each checked against the oracle (bit-exact; the norm within 1e-6 of the exact value)."""
import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle

pytestmark = pytest.mark.gpu

SETTINGS = settings(max_examples=200, deadline=None, suppress_health_check=list(HealthCheck), derandomize=True)


def place(arr, off, dev, bf16=False):
    """A device copy of arr starting `off` elements into a fresh buffer (to control alignment)."""
    if bf16:
        buf = np.zeros(arr.size + off, np.uint16)
        buf[off:] = arr
        return torch.from_numpy(buf.view(np.int16)).to(dev).view(torch.bfloat16)[off:]
    buf = np.zeros(arr.size + off, np.float32)
    buf[off:] = arr
    return torch.from_numpy(buf).to(dev)[off:]


@SETTINGS
@given(sizes=st.lists(st.integers(0, 9000), min_size=1, max_size=8),
       offs=st.lists(st.integers(0, 7), min_size=5, max_size=5),
       g_bf16=st.booleans(), with_p16=st.booleans(), mode=st.sampled_from([0, 1]),
       factor=st.one_of(st.none(), st.floats(1e-8, 4.0)), step=st.integers(1, 3000),
       cuts=st.lists(st.integers(0, 8), max_size=4), with_gout=st.booleans(), goff=st.integers(0, 7),
       seed=st.integers(0, 2 ** 31 - 1))
def test_adam_random_tables(pkg, dev, sizes, offs, g_bf16, with_p16, mode, factor, step, cuts, with_gout, goff,
                            seed):
    """Adam + BF16 over a random table against the oracle; with `cuts`, as one z1_adam_cast_rows launch per range
    between the cut rows; with FP32 gradient outputs (at a random misalignment), each holding the oracle's scaled
    gradient afterwards."""
    from faster_yoco_amd import ops
    rng = np.random.default_rng(seed)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    rows, keep, ref, outs, want = [], [], [], [], []
    for n in sizes:
        g = (rng.standard_normal(n) * 10.0 ** rng.uniform(-5, 0)).astype(np.float32)
        g = oracle.bf16_rne(g) if g_bf16 else g
        p = (rng.standard_normal(n) * 0.02).astype(np.float32)
        m = (rng.standard_normal(n) * 1e-4).astype(np.float32)
        v = np.abs(rng.standard_normal(n) * 1e-8).astype(np.float32)
        gt = place(g, offs[0], dev, bf16=g_bf16)
        pt, mt, vt = place(p, offs[1], dev), place(m, offs[2], dev), place(v, offs[3], dev)
        p16 = place(np.zeros(n, np.uint16), offs[4], dev, bf16=True) if with_p16 else None
        rows.append((gt, pt, mt, vt, p16, n))
        keep.append((pt, mt, vt, p16))
        ref.append(oracle.adam_cast(g, p, m, v, step=step, mode=mode, factor=factor, **hp))
        outs.append(place(np.full(n, -7.0, np.float32), goff, dev))
        f1 = np.float32(1.0 if factor is None else factor)
        want.append(oracle.scale_up(g, f1) if g_bf16 else (g * f1).astype(np.float32))
    table = ops.Table(rows, dev)
    bc1, bc2 = ops.bias_corrections(hp['beta1'], hp['beta2'], step)
    f = None if factor is None else torch.tensor([factor], dtype=torch.float32, device=dev)
    if cuts:
        bounds = sorted({0, len(sizes)} | {c for c in cuts if c <= len(sizes)})
        for a, b in zip(bounds, bounds[1:]):
            ops.adam_cast_rows(table, a, b, f, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2,
                               hp['weight_decay'], mode, g32=outs if with_gout else None)
    else:
        ops.adam_cast(table, f, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2, hp['weight_decay'], mode,
                      g32=outs if with_gout else None)
    torch.cuda.synchronize()
    for o, w in zip(outs, want):
        got = o.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), w.view(np.uint32) if with_gout else np.full_like(got, -7.0).view(
            np.uint32))
    for (pt, mt, vt, p16), (po, mo, vo, p16o) in zip(keep, ref):
        assert np.array_equal(pt.cpu().numpy().view(np.uint32), po.view(np.uint32))
        assert np.array_equal(mt.cpu().numpy().view(np.uint32), mo.view(np.uint32))
        assert np.array_equal(vt.cpu().numpy().view(np.uint32), vo.view(np.uint32))
        if p16 is not None:
            assert np.array_equal(p16.view(torch.int16).cpu().numpy().view(np.uint16), p16o)
    table.close()


@SETTINGS
@given(world=st.integers(1, 16), n=st.integers(0, 40000), off=st.integers(0, 9), want_sum=st.booleans(),
       seed=st.integers(0, 2 ** 31 - 1))
def test_owner_sum_random(pkg, dev, world, n, off, want_sum, seed):
    from faster_yoco_amd import ops
    rng = np.random.default_rng(seed)
    cs = [oracle.bf16_rne((rng.standard_normal(n) * 10.0 ** rng.uniform(-6, 1)).astype(np.float32))
          for _ in range(world)]
    avg, s = oracle.owner_sum(cs, want_sum=True)
    ts = [place(c, off, dev, bf16=True) for c in cs]
    out = place(np.zeros(n, np.uint16), off, dev, bf16=True)
    osum = place(np.zeros(n, np.float32), off, dev) if want_sum else None
    part = ops.norm_workspace(dev, n)
    ops.owner_sum(ts, out, 1.0 / world, out_sum=osum, partials=part)
    nr = torch.zeros(1, device=dev)
    ops.norm_clip(part, norm_out=nr)
    torch.cuda.synchronize()
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), avg)
    if want_sum:
        assert np.array_equal(osum.cpu().numpy().view(np.uint32), s.view(np.uint32))
    ex = float(np.sqrt(oracle.sumsq(avg)))
    assert abs(float(nr.item()) - ex) <= 1e-6 * ex + 1e-30


@SETTINGS
@given(sizes=st.lists(st.integers(0, 9000), min_size=1, max_size=8),
       offs=st.lists(st.integers(0, 7), min_size=8, max_size=8), g_bf16=st.booleans(),
       mag=st.floats(-6, 2), max_norm=st.sampled_from([0.0, 1e-3, 1.0, 1e6]), factor=st.floats(1e-4, 8.0),
       seed=st.integers(0, 2 ** 31 - 1))
def test_norm_random_tables(pkg, dev, sizes, offs, g_bf16, mag, max_norm, factor, seed):
    """Norm of random tables (misaligned, empty and tail rows, f32 or bf16): within 1e-6 of the exact value; the
    clip chain bit-exact from the GPU's norm."""
    from faster_yoco_amd import ops
    rng = np.random.default_rng(seed)
    rows, hs = [], []
    for i, n in enumerate(sizes):
        g = (rng.standard_normal(n) * 10.0 ** mag).astype(np.float32)
        g = oracle.bf16_rne(g) if g_bf16 else g
        hs.append(g)
        rows.append((place(g, offs[i], dev, bf16=g_bf16), None, None, None, None, n))
    table = ops.Table(rows, dev)
    part = ops.norm_workspace(dev)
    nr, gn, fo = (torch.zeros(1, device=dev) for _ in range(3))
    ops.grad_sumsq(table, part)
    ops.norm_clip(part, factor=factor, norm_out=nr, grad_norm_out=gn, factor_out=fo, max_norm=max_norm)
    torch.cuda.synchronize()
    ex = float(np.sqrt(sum(oracle.sumsq(h) for h in hs)))
    got = float(nr.item())
    assert abs(got - ex) <= 1e-6 * ex + 1e-38
    o_nr, o_gn, o_f = oracle.norm_clip(float(np.float32(got)) ** 2, factor, max_norm)
    assert np.float32(o_nr) == np.float32(got)
    assert np.float32(gn.item()).view(np.uint32) == np.float32(o_gn).view(np.uint32)
    assert np.float32(fo.item()).view(np.uint32) == np.float32(o_f).view(np.uint32)
    table.close()


@SETTINGS
@given(R=st.integers(0, 4000), D=st.integers(1, 72), V=st.integers(1, 300), pad=st.integers(-1, 299),
       mode=st.sampled_from([None, 'after', 'first']), world=st.sampled_from([1, 2, 8, 6]),
       bad=st.integers(0, 20), seed=st.integers(0, 2 ** 31 - 1))
def test_embedding_random(pkg, dev, R, D, V, pad, mode, world, bad, seed):
    """Embedding gradient for random ids (repeats, out-of-range ids, padding), widths (incl. D % 8 != 0) and both
    placements of the 1/world scale: bit-exact against the oracle's restatement of aten's order for the row count
    (the sort path above 3072 rows, chunks of 16 indices up to it)."""
    from faster_yoco_amd import embedding
    rng = np.random.default_rng(seed)
    pad = pad if pad < V else -1
    ids = rng.integers(0, V, R).astype(np.int64)
    if R and bad:
        k = min(bad, R)
        ids[rng.choice(R, k, replace=False)] = rng.choice([-5, -1, V, V + 7], k)
    g16 = oracle.bf16_rne((rng.standard_normal((R, D)) * 1e-2).astype(np.float32))
    scale = None if mode is None else 1.0 / world
    want = oracle.embedding_backward(ids, g16, V, padding_idx=pad, scale=scale, scale_first=(mode == 'first'))
    gt = torch.from_numpy(g16.view(np.int16)).to(dev).view(torch.bfloat16)
    out = embedding.embedding_dense_backward(gt, torch.from_numpy(ids).to(dev), V, pad, False, scale=scale,
                                             scale_first=(mode == 'first'))
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, want)


@SETTINGS
@given(n=st.integers(0, 70000), off=st.integers(0, 9), factor=st.floats(1e-6, 1e3), seed=st.integers(0, 2 ** 31 - 1))
def test_scale_and_cast_random(pkg, dev, n, off, factor, seed):
    """scale_up (bf16 -> fp32 times the factor) and the BF16 cast at random sizes and offsets: bit-exact."""
    from faster_yoco_amd import ops
    rng = np.random.default_rng(seed)
    g16 = oracle.bf16_rne((rng.standard_normal(n) * 1e-2).astype(np.float32))
    p32 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    gt = place(g16, off, dev, bf16=True)
    g32 = place(np.zeros(n, np.float32), (off + 3) % 10, dev)
    f = torch.tensor([factor], dtype=torch.float32, device=dev)
    ops.scale_up(gt, g32, f)
    pt = place(p32, off, dev)
    p16 = place(np.zeros(n, np.uint16), (off + 5) % 10, dev, bf16=True)
    ops.cast_bf16(pt, p16)
    torch.cuda.synchronize()
    assert np.array_equal(g32.cpu().numpy().view(np.uint32), oracle.scale_up(g16, factor).view(np.uint32))
    assert np.array_equal(p16.view(torch.int16).cpu().numpy().view(np.uint16), oracle.bf16_rne(p32))
