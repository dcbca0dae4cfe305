"""Drop-in for yoco/tasks/fused_adam_cast.py on this build's operators: the Adam step that also writes the BF16
copy of each updated master, and the BF16 -> FP32 gradient scale.

``FusedAdamCast`` has the reference's interface (``fused_adam_cast.py:48-72``): it is made from ``dest`` (address of
an fp32 master -> the BF16 tensor to write), called by fairseq's FusedAdamV2.step with amp_C.multi_tensor_adam's
arguments, and collects in ``.cast`` the addresses of the masters whose BF16 copy it wrote.  Internally:
  * all the call's tensors go to one ``torch.ops.yoco_z1.adam_cast_`` launch over a table (cached by the rows'
    sizes, bound to the call's tensors), where the reference launches one Triton kernel per tensor;
  * what a parameter list needs -- its tables, the BF16 destinations found in ``dest``, the masters they belong to
    -- is worked out once per list of masters and set of folded rows (keyed by the masters' addresses and sizes,
    as ``dest`` is keyed by address) and reused while they recur; each call's tensors are still checked, by the
    operator; a table's rows are ordered by their gradients' addresses (the launch starts at the highest, where a
    norm pass over the same gradients, whose table is ordered alike, ends with allocating loads);
  * ``fold`` / ``fold_factor`` (set by zero1_fast.step with the fused Adam) name masters whose BF16 gradient the
    kernel reads times the factor, in place of the FP32 gradient a scale pass would have written first: the same
    products g' = fp32(float(g16) * factor).  With ``fold_writes`` (zero1_fast's default) the kernel also stores
    g' into the FP32 gradient tensors of the call, so they end as the reference's scale pass leaves them, in one
    pass of 32 bytes per element instead of 6 + 30; without it (YOCO_Z1_FOLD_SCALE=1) they are left as they were
    (28 bytes per element).
``scale_up`` keeps ``fused_adam_cast.py:84-89``'s signature.
"""
from collections import OrderedDict

import torch

from . import ops

__all__ = ['FusedAdamCast', 'scale_up']


class FusedAdamCast:
    """amp_C.multi_tensor_adam's call signature, plus the BF16 copy of every master found in ``dest``.  Masters are
    matched by ``data_ptr()``: FusedAdamV2.step hands over ``p.data``, a new tensor object on every call."""

    def __init__(self, dest):
        self.dest = dest                  # master address -> BF16 destination
        self.cast = set()                 # masters whose BF16 copy was written since the caller last cleared it
        self.fold = {}                    # master address -> BF16 gradient read in place of the FP32 one
        self.fold_factor = None           # the 1-element fp32 device factor of the folded gradients
        self.fold_writes = False          # folded rows also write g' into the call's FP32 gradient tensors
        self._tables = ops.TableCache()
        # (masters' (address, size)s, which rows are folded) -> (groups, written addresses); a group is
        # (folded, row indices or None for all rows, table, BF16 destinations)
        self._plans = OrderedDict()

    def __call__(self, chunk_size, noop_flag, tensor_lists, lr, beta1, beta2, eps, step, mode, bias_correction,
                 weight_decay):
        if int(mode) not in (0, 1):
            raise RuntimeError(f'fused_adam_cast: unsupported adam mode {mode}')
        bc1, bc2 = ops.bias_corrections(beta1, beta2, step, bias_correction)
        g, p, m, v = tensor_lists
        if not p:
            return
        key = tuple([(t.data_ptr(), t.numel()) for t in p])
        g16 = [self.fold.get(a) for a, _ in key] if self.fold else None
        folded = None if g16 is None else tuple(x is not None for x in g16)
        if folded is not None and any(folded) and self.fold_factor is None:
            raise RuntimeError('fused_adam_cast: folded gradients without a factor')
        plan = self._plans.get((key, folded))
        if plan is None:
            plan = self._plan(key, folded, tensor_lists, g16)
        groups, written = plan
        for is_folded, idx, table, p16 in groups:
            pick = (lambda lst: lst) if idx is None else (lambda lst: [lst[i] for i in idx])
            gin = pick(g16) if is_folded else pick(g)
            ops.adam_cast(table, self.fold_factor if is_folded else None, lr, beta1, beta2, eps, bc1, bc2,
                          weight_decay, int(mode), tensors=(gin, pick(p), pick(m), pick(v), p16),
                          g32=pick(g) if is_folded and self.fold_writes else None)
        self.cast.update(written)

    def _row(self, g, p, m, v):
        """Checked size and BF16 destination (or None) of one row."""
        if not (g.dtype == p.dtype == m.dtype == v.dtype == torch.float32 and g.is_contiguous()
                and p.is_contiguous() and m.is_contiguous() and v.is_contiguous()):
            raise RuntimeError('fused_adam_cast: expected contiguous fp32 tensors')
        n = p.numel()
        if g.numel() != n or m.numel() != n or v.numel() != n:
            raise RuntimeError('fused_adam_cast: tensor sizes differ within a row')
        d = self.dest.get(p.data_ptr())
        if d is not None and (d.dtype != torch.bfloat16 or not d.is_contiguous() or d.numel() != n):
            raise RuntimeError('fused_adam_cast: the bf16 destination must be a contiguous bf16 view')
        return n, d

    def _plan(self, key, folded, tensor_lists, g16):
        """Groups (rows reading the FP32 gradient / a folded BF16 one: their table and BF16 destinations) and the
        written addresses for a list of masters, checked row by row.  Later calls with the same masters and folded
        rows reuse it; the operators check each call's tensors."""
        rows = {False: [], True: []}
        idx = {False: [], True: []}
        written = []
        for i, (g, p, m, v) in enumerate(zip(*tensor_lists)):
            n, d = self._row(g, p, m, v)
            if d is not None:
                written.append(p.data_ptr())
            f = bool(folded and folded[i])
            if f and (g16[i].dtype != torch.bfloat16 or not g16[i].is_contiguous() or g16[i].numel() != n):
                raise RuntimeError('fused_adam_cast: a folded gradient must be contiguous bf16')
            rows[f].append((g16[i] if f else g, p, m, v, d, n))
            idx[f].append(i)
        groups = []
        for f in (False, True):
            if rows[f]:
                # rows in the order of their gradients' addresses: the launch walks from the last row down, so it
                # starts at the highest gradient address -- where the norm pass over the same gradients (its table
                # ordered alike) read its last 256 MB with allocating loads, still in the MALL -- whatever order
                # the parameters come in (CEReduce lays them out by backward phase, ce_reduce.py:122-140)
                order = sorted(range(len(rows[f])), key=lambda j: rows[f][j][0].data_ptr())
                srows = [rows[f][j] for j in order]
                sidx = [idx[f][j] for j in order]
                table = self._tables.get(srows, srows[0][1].device)
                whole = sidx == list(range(len(key)))
                groups.append((f, None if whole else tuple(sidx), table, ops.rows_lists(srows)[4]))
        plan = (tuple(groups), tuple(written))
        self._plans[(key, folded)] = plan
        while len(self._plans) > 8:
            self._plans.popitem(last=False)
        return plan


def scale_up(g16, g32, factor):
    """Scale pass of yoco/tasks/fused_adam_cast.py:84-89: each BF16 gradient element is widened to fp32 (exact) and
    multiplied by the device scalar ``factor`` (one fp32 element) with one fp32 rounding, written to ``g32``; the
    bits torch's ``mul`` of a bf16 tensor by an fp32 scalar tensor into an fp32 output gives."""
    ops.scale_up(g16, g32, factor)
