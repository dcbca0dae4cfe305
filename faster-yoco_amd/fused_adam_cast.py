"""Drop-in for yoco/tasks/fused_adam_cast.py on this build's operators: the Adam step that also writes the BF16
copy of each updated master, and the BF16 -> FP32 gradient scale.

``FusedAdamCast`` has the reference's interface (``fused_adam_cast.py:48-72``): it is made from ``dest`` (address of
an fp32 master -> the BF16 tensor to write), called by fairseq's FusedAdamV2.step with amp_C.multi_tensor_adam's
arguments, and collects in ``.cast`` the addresses of the masters whose BF16 copy it wrote.  Internally:
  * all the call's tensors go to one ``torch.ops.yoco_z1.adam_cast_`` launch over a table (cached by the rows'
    sizes, bound to the call's tensors), where the reference launches one Triton kernel per tensor;
  * ``fold`` / ``fold_factor`` (set by zero1_fast.step under YOCO_Z1_FOLD_SCALE=1) name masters whose BF16 gradient
    the kernel reads times the factor, in place of the FP32 gradient a scale pass would have written: the same
    products g' = fp32(float(g16) * factor), 6 bytes per element less traffic.
``scale_up`` keeps ``fused_adam_cast.py:84-89``'s signature.
"""
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
        self._tables = ops.TableCache()

    def __call__(self, chunk_size, noop_flag, tensor_lists, lr, beta1, beta2, eps, step, mode, bias_correction,
                 weight_decay):
        if int(mode) not in (0, 1):
            raise RuntimeError(f'fused_adam_cast: unsupported adam mode {mode}')
        bc1, bc2 = ops.bias_corrections(beta1, beta2, step, bias_correction)
        groups = {False: [], True: []}    # rows reading the FP32 gradient / a folded BF16 one
        written = []
        for g, p, m, v in zip(*tensor_lists):
            if not (g.dtype == p.dtype == m.dtype == v.dtype == torch.float32 and g.is_contiguous()
                    and p.is_contiguous() and m.is_contiguous() and v.is_contiguous()):
                raise RuntimeError('fused_adam_cast: expected contiguous fp32 tensors')
            n = p.numel()
            if g.numel() != n or m.numel() != n or v.numel() != n:
                raise RuntimeError('fused_adam_cast: tensor sizes differ within a row')
            key = p.data_ptr()
            d = self.dest.get(key)
            if d is not None:
                if d.dtype != torch.bfloat16 or not d.is_contiguous() or d.numel() != n:
                    raise RuntimeError('fused_adam_cast: the bf16 destination must be a contiguous bf16 view')
                written.append(key)
            g16 = self.fold.get(key)
            if g16 is not None and (g16.dtype != torch.bfloat16 or not g16.is_contiguous() or g16.numel() != n):
                raise RuntimeError('fused_adam_cast: a folded gradient must be contiguous bf16')
            groups[g16 is not None].append((g if g16 is None else g16, p, m, v, d, n))
        if groups[True] and self.fold_factor is None:
            raise RuntimeError('fused_adam_cast: folded gradients without a factor')
        for folded, rows in groups.items():
            if rows:
                table = self._tables.get(rows, rows[0][1].device)
                ops.adam_cast(table, self.fold_factor if folded else None, lr, beta1, beta2, eps, bc1, bc2,
                              weight_decay, int(mode), tensors=ops.rows_lists(rows))
        self.cast.update(written)


def scale_up(g16, g32, factor):
    """g32 = float(g16) * factor (factor: 1-element fp32 tensor) -- the fp32 product of the exactly upcast value, as
    torch.mul(g16, factor, out=g32) computes it."""
    ops.scale_up(g16, g32, factor)
