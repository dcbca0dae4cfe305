"""Drop-in for the owner-side sum of yoco/models/decoder/ce_reduce.py (the Triton kernel ``_sum_slots``, :59-74,
launched by ``CEReduce._sum``, :178-183) on this build's ``yoco_z1::sum_slots_`` operator.

Only the sum is in scope: the peer transport (CUDA IPC mappings, copy-engine pushes, barriers; :77-104,185-237) stays
the reference's.  ``install(CEReduce)`` replaces ``CEReduce._sum``; ``sum_slots`` takes the Triton kernel's launch
arguments.
"""
from . import ops

__all__ = ['sum_slots', '_sum', 'install']


def sum_slots(S, OUT, G, BASE, END, R, scale, WORLD):
    """OUT[e] = bf16(sum_{k=0..WORLD-1} float(x_k[e]) * scale) for e in [BASE, END), in rank order, where x_R is OUT
    itself (rank R's own gradients) and the peers' contributions sit slot-major in S ([WORLD-1, G]: peer k < R in
    slot k, k > R in slot k-1).  In place in OUT, on the current stream."""
    ops.sum_slots(S, OUT, G, BASE, END, R, scale, WORLD)


def _sum(self, ph):
    """CEReduce._sum (ce_reduce.py:178-183) on the gfx950 kernel."""
    a, b = self.bounds[ph]
    if b > a:
        sum_slots(self.staging, self.out, self.G, a, b, self.rank, 1.0 / self.world, self.world)


def install(cereduce_cls):
    """Replace the Triton sum of a CEReduce class (from models.decoder.ce_reduce) with this one."""
    cereduce_cls._sum = _sum
    return cereduce_cls
