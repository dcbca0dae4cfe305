"""Drop-in for the owner-side sum of yoco/models/decoder/ce_reduce.py (the Triton kernel ``_sum_slots``, :59-74,
launched by ``CEReduce._sum``, :178-183) on this build's ``yoco_z1::sum_slots_`` operator.

Only the sum is in scope: the peer transport (CUDA IPC mappings, copy-engine pushes, barriers; :77-104,185-237) stays
the reference's.  ``install(CEReduce)`` replaces ``CEReduce._sum``; ``sum_slots`` takes the Triton kernel's launch
arguments.

The norm of the summed gradients rides along.  Each ``_sum(ph)`` also leaves the FP64 sum of squares of its range's
BF16 average per 256-element chunk (``PhaseNorm``: one array per CEReduce, one slice per phase), which costs 8 bytes
of writes per 256 elements.  When every phase of an update has been summed and the owned gradients handed to
``zero1_fast.clip_grad_norm`` are exactly the views ``CEReduce.finish`` makes of ``out`` (:232-237), clip_grad_norm
reduces those partials (``take_norm_partials``) instead of reading the 2 bytes per element of the average once more,
as the reference's ``clip_grad_norm_`` of the owned gradients does (yoco/tasks/zero1_fast.py:147-151).  The same idea
was screened in the reference as one fused kernel and not adopted (docs/training.md:335).  Either way the norm is the
exact sum of squares of the same BF16 values in FP64, so it is the same to within an fp32 ulp.
"""
import weakref

import torch

from . import ops

__all__ = ['sum_slots', '_sum', 'install', 'PhaseNorm', 'take_norm_partials']

_BY_OUT = weakref.WeakValueDictionary()      # address of a CEReduce's out -> its PhaseNorm
FUSE_NORM = True      # False: _sum leaves no partials and clip_grad_norm reads the gradients again (for comparisons)


def sum_slots(S, OUT, G, BASE, END, R, scale, WORLD, waves=None):
    """OUT[e] = bf16(sum_{k=0..WORLD-1} float(x_k[e]) * scale) for e in [BASE, END), in rank order, where x_R is OUT
    itself (rank R's own gradients) and the peers' contributions sit slot-major in S ([WORLD-1, G]: peer k < R in
    slot k, k > R in slot k-1).  In place in OUT, on the current stream.  waves (float64, nullable): the range's
    norm partials per chunk (``ops.owner_sum_waves(END - BASE)`` of them)."""
    ops.sum_slots(S, OUT, G, BASE, END, R, scale, WORLD, waves=waves)


class PhaseNorm:
    """Norm partials of one CEReduce's phase sums: phase ph writes ``waves[offset[ph]:offset[ph] + count[ph]]``;
    ``summed[ph]`` says whether phase ph has been summed since the partials were last taken.  Made from the
    CEReduce's ``out``, ``G`` and ``bounds``; made again when any of them changes."""

    def __init__(self, ce):
        self.out_ptr = ce.out.data_ptr()
        self.device = ce.out.device
        self.G = int(ce.G)
        self.bounds = tuple((int(a), int(b)) for a, b in ce.bounds)
        self.offset, self.count, m = [], [], 0
        for a, b in self.bounds:
            w = ops.owner_sum_waves(b - a) if b > a else 0
            self.offset.append(m)
            self.count.append(w)
            m += w
        self.m = m
        self.waves = torch.empty(max(m, 1), dtype=torch.float64, device=self.device)
        self.summed = [False] * len(self.bounds)
        spans = sorted((a, b) for a, b in self.bounds if b > a)
        pos = 0
        for a, b in spans:                      # the phases tile [0, G) of out (ce_reduce.py:122-140 builds them so)
            if a != pos:
                break
            pos = b
        self.tiles = pos == self.G

    def matches(self, ce):
        return (ce.out.data_ptr() == self.out_ptr and int(ce.G) == self.G
                and tuple((int(a), int(b)) for a, b in ce.bounds) == self.bounds)

    def ready(self):
        return self.tiles and all(s or a == b for s, (a, b) in zip(self.summed, self.bounds))


def _phase_norm(ce):
    pn = ce.__dict__.get('_z1_norm')
    if pn is None or not pn.matches(ce):
        if pn is not None and _BY_OUT.get(pn.out_ptr) is pn:
            del _BY_OUT[pn.out_ptr]
        pn = PhaseNorm(ce)
        ce._z1_norm = pn
        _BY_OUT[pn.out_ptr] = pn
    return pn


def _sum(self, ph):
    """CEReduce._sum (ce_reduce.py:178-183) on the gfx950 kernel, leaving the phase's norm partials."""
    a, b = self.bounds[ph]
    if b <= a:
        return
    if not FUSE_NORM:
        sum_slots(self.staging, self.out, self.G, a, b, self.rank, 1.0 / self.world, self.world)
        return
    pn = _phase_norm(self)
    o = pn.offset[ph]
    sum_slots(self.staging, self.out, self.G, a, b, self.rank, 1.0 / self.world, self.world,
              waves=pn.waves[o:o + pn.count[ph]])
    # the phases run on CEReduce's sum stream and on the current one, and clip_grad_norm reads the partials on its
    # stream: each use is recorded, so that a PhaseNorm dropped when the bounds change frees its partials only
    # after every stream is past them
    pn.waves.record_stream(torch.cuda.current_stream(self.out.device))
    pn.summed[ph] = True


def take_norm_partials(grads):
    """(waves, m) of the CEReduce whose out the BF16 gradients ``grads`` tile exactly -- every element of [0, G) of
    out in exactly one of them, in any order -- when each of its phases has been summed since the partials were
    last taken; else None.  Taking them marks them used."""
    if not FUSE_NORM or not grads or any(g.dtype != torch.bfloat16 or not g.is_cuda or not g.is_contiguous() for g in grads):
        return None
    spans = sorted((g.data_ptr(), g.numel()) for g in grads if g.numel())
    pn = _BY_OUT.get(spans[0][0]) if spans else None
    if pn is None or not pn.ready() or any(g.device != pn.device for g in grads):
        return None
    pos = pn.out_ptr
    for ptr, n in spans:
        if ptr != pos:
            return None
        pos += 2 * n
    if pos != pn.out_ptr + 2 * pn.G:
        return None
    pn.summed = [False] * len(pn.bounds)
    pn.waves.record_stream(torch.cuda.current_stream(pn.device))       # read by the caller on this stream
    return pn.waves, pn.m


def install(cereduce_cls):
    """Replace the Triton sum of a CEReduce class (from models.decoder.ce_reduce) with this one."""
    cereduce_cls._sum = _sum
    return cereduce_cls
