"""Property-based GPU parity (hypothesis): random tensor tables -- row counts, ragged sizes (including 0 and tails),
per-array misalignment, bf16 or fp32 gradients, with or without BF16 copies, both Adam modes, random factors and
steps -- and random owner sums (world 1..16, odd lengths, offsets), each checked bit-exact against the oracle."""
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
       seed=st.integers(0, 2 ** 31 - 1))
def test_adam_random_tables(pkg, dev, sizes, offs, g_bf16, with_p16, mode, factor, step, seed):
    from faster_yoco_amd import ops
    rng = np.random.default_rng(seed)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    rows, keep, ref = [], [], []
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
    table = ops.Table(rows, dev)
    bc1, bc2 = ops.bias_corrections(hp['beta1'], hp['beta2'], step)
    f = None if factor is None else torch.tensor([factor], dtype=torch.float32, device=dev)
    ops.adam_cast(table, f, hp['lr'], hp['beta1'], hp['beta2'], hp['eps'], bc1, bc2, hp['weight_decay'], mode)
    torch.cuda.synchronize()
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
