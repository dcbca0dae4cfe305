"""One table shared by calls on several streams, and by eager calls and captured graphs.

A table's device rows are shared by every launch over it, and the operators rebind them to each call's tensors.
These tests make that safe to rely on:
  * two streams: calls alternate between stream A (one set of tensors) and stream B (another set) on one table,
    each call enqueued right after the other; a call on another stream than the table's last one waits, on the
    device, for the work already enqueued there (an event), so no launch reads rows rebound under it;
  * graph capture: a captured call carries its own binding, so every replay updates the tensors it was captured
    with, whatever eager calls bound in between -- including a capture whose tensors the table already held, and
    an eager call after the capture with the captured tensors.
Every result is compared with the CPU oracle, bit for bit (the reference's launches each carry their own pointers,
yoco/tasks/fused_adam_cast.py:68-70, so it has no shared state to race on)."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
SIZES = (4 * 1024 * 1024 + 5, 2 * 1024 * 1024)


def bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


class Set:
    """One set of tensors for the table's rows (g, p, m, v, p16 per row) with its oracle state."""

    def __init__(self, dev, seed):
        rng = np.random.default_rng(seed)
        self.host = []
        self.t = []
        for n in SIZES:
            g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
            p = (rng.standard_normal(n) * 0.02).astype(np.float32)
            m = (rng.standard_normal(n) * 1e-4).astype(np.float32)
            v = np.abs(rng.standard_normal(n) * 1e-8).astype(np.float32)
            self.host.append([g, p, m, v])
            self.t.append([torch.from_numpy(x).to(dev) for x in (g, p, m, v)] +
                          [torch.empty(n, dtype=torch.bfloat16, device=dev)])
        self.steps = 0

    def rows(self):
        return [(r[0], r[1], r[2], r[3], r[4], n) for r, n in zip(self.t, SIZES)]

    def lists(self):
        return [[r[k] for r in self.t] for k in range(5)]

    def expect_step(self):
        self.steps += 1
        for h in self.host:
            po, mo, vo, _ = oracle.adam_cast(h[0], h[1], h[2], h[3], step=7, **HP)
            h[1], h[2], h[3] = po, mo, vo

    def check(self, what):
        for i, (h, r) in enumerate(zip(self.host, self.t)):
            assert np.array_equal(bits(r[1]), h[1].view(np.uint32)), (what, i, 'p')
            assert np.array_equal(bits(r[2]), h[2].view(np.uint32)), (what, i, 'm')
            assert np.array_equal(bits(r[3]), h[3].view(np.uint32)), (what, i, 'v')
            p16 = r[4].view(torch.int16).cpu().numpy().view(np.uint16)
            assert np.array_equal(p16, oracle.bf16_rne(h[1])), (what, i, 'p16')


def adam(table, s):
    from faster_yoco_amd import ops
    bc1, bc2 = ops.bias_corrections(HP['beta1'], HP['beta2'], 7)
    ops.adam_cast(table, None, HP['lr'], HP['beta1'], HP['beta2'], HP['eps'], bc1, bc2, HP['weight_decay'], 1,
                  tensors=s.lists())


def norm_of(table, grads, partials, out):
    from faster_yoco_amd import ops
    ops.grad_sumsq(table, partials, g=grads)
    ops.norm_clip(partials, norm_out=out)


def test_one_table_from_two_streams(pkg, dev):
    from faster_yoco_amd import ops
    x, y = Set(dev, 1), Set(dev, 2)
    cache = ops.TableCache()
    table = cache.get(x.rows(), dev)
    assert cache.get(y.rows(), dev) is table              # same sizes and columns: one table for both sets
    ntab = cache.get([(r[0], None, None, None, None, n) for r, n in zip(x.t, SIZES)], dev)
    a, b = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    parts = {s: ops.norm_workspace(dev) for s in ('a', 'b')}
    norms = {s: torch.zeros(1, device=dev) for s in ('a', 'b')}
    torch.cuda.synchronize()
    for rep in range(3):
        with torch.cuda.stream(a):
            norm_of(ntab, [r[0] for r in x.t], parts['a'], norms['a'])
            adam(table, x)
        with torch.cuda.stream(b):                          # enqueued while stream A's launches may still run
            norm_of(ntab, [r[0] for r in y.t], parts['b'], norms['b'])
            adam(table, y)
        x.expect_step()
        y.expect_step()
        torch.cuda.synchronize()
        x.check(f'A {rep}')
        y.check(f'B {rep}')
        for s, st in (('a', x), ('b', y)):
            ex = float(np.sqrt(sum(oracle.sumsq(h[0]) for h in st.host)))
            assert abs(float(norms[s].item()) - ex) <= 1e-6 * ex, (rep, s)


@pytest.mark.parametrize('captured', ['other_tensors', 'same_tensors'])
def test_captured_call_carries_its_binding(pkg, dev, captured):
    """Eager call (set X) on a side stream, capture (set Y; or X, the tensors the table already holds), eager call
    (set Z), replay, eager call with the captured set, replay: each replay updates the captured set only."""
    from faster_yoco_amd import ops
    x, z = Set(dev, 3), Set(dev, 5)
    y = Set(dev, 4) if captured == 'other_tensors' else x
    cache = ops.TableCache()
    table = cache.get(x.rows(), dev)
    side = torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        adam(table, x)
    x.expect_step()
    torch.cuda.synchronize()
    x.check('eager X on a side stream')
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        adam(table, y)                                     # recorded, not run
    torch.cuda.synchronize()
    x.check('nothing ran during capture')
    adam(table, z)                                         # eager: binds the table to Z
    z.expect_step()
    torch.cuda.synchronize()
    z.check('eager Z')
    graph.replay()
    y.expect_step()
    torch.cuda.synchronize()
    y.check('replay 1')
    z.check('Z untouched by the replay')
    adam(table, y)                                         # eager with the captured tensors
    y.expect_step()
    torch.cuda.synchronize()
    y.check('eager with the captured tensors')
    graph.replay()
    y.expect_step()
    torch.cuda.synchronize()
    y.check('replay 2')
    z.check('Z still untouched')
