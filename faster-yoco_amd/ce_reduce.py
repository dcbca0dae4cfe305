"""Drop-in for the owner-side sum of yoco/models/decoder/ce_reduce.py (the Triton kernel ``_sum_slots``, :59-74,
and its launcher ``CEReduce._sum``, :178-183) on a gfx950 kernel.

Only the sum is in scope: the peer transport (CUDA IPC mappings, copy-engine pushes, barriers; :77-104,185-237) is
the reference's and is left to it.  ``install(CEReduce)`` replaces ``CEReduce._sum``; ``sum_slots`` takes the
Triton kernel's launch arguments.
"""
import torch

from . import ops
from ._lib import Z1_MAX_WORLD

__all__ = ['sum_slots', '_sum', 'install']


def sum_slots(S, OUT, G, BASE, END, R, scale, WORLD):
    """OUT[e] = bf16(sum_{k=0..WORLD-1} float(x_k[e]) * scale) for e in [BASE, END), in rank order, where x_R is OUT
    itself (rank R's own gradients) and the peers' contributions sit slot-major in S ([WORLD-1, G]: peer k < R in
    slot k, k > R in slot k-1).  In place in OUT, on the current stream."""
    for t, name in ((S, 'staging'), (OUT, 'out')):
        if not (torch.is_tensor(t) and t.is_cuda and t.dtype == torch.bfloat16 and t.is_contiguous()):
            raise RuntimeError(f'ce_reduce: {name} must be a contiguous bf16 GPU tensor')
    G, BASE, END, R, WORLD = int(G), int(BASE), int(END), int(R), int(WORLD)
    if not 1 <= WORLD <= Z1_MAX_WORLD or not 0 <= R < WORLD:
        raise RuntimeError(f'ce_reduce: rank {R} / world {WORLD} out of range')
    if not 0 <= BASE <= END <= G or OUT.numel() < G or S.numel() < (WORLD - 1) * G:
        raise RuntimeError(f'ce_reduce: range [{BASE}, {END}) does not fit G={G}, out {OUT.numel()}, '
                           f'staging {S.numel()}')
    if END == BASE:
        return
    es = OUT.element_size()
    s0, o0 = S.data_ptr(), OUT.data_ptr()
    addrs = []
    for k in range(WORLD):
        if k < R:
            addrs.append(s0 + (k * G + BASE) * es)
        elif k == R:
            addrs.append(o0 + BASE * es)
        else:
            addrs.append(s0 + ((k - 1) * G + BASE) * es)
    ops.owner_sum_raw(addrs, END - BASE, o0 + BASE * es, scale, OUT.device)


def _sum(self, ph):
    """CEReduce._sum (ce_reduce.py:178-183) on the gfx950 kernel."""
    a, b = self.bounds[ph]
    if b > a:
        sum_slots(self.staging, self.out, self.G, a, b, self.rank, 1.0 / self.world, self.world)


def install(cereduce_cls):
    """Replace the Triton sum of a CEReduce class (from models.decoder.ce_reduce) with this one."""
    cereduce_cls._sum = _sum
    return cereduce_cls
