"""Drop-in for yoco/tasks/fused_adam_cast.py: Adam fused with the BF16 cast of the updated master, and the
BF16 -> FP32 gradient scale, on gfx950 kernels.

``FusedAdamCast`` keeps the reference's interface (``fused_adam_cast.py:48-72``): constructed with ``dest`` (data_ptr
of an fp32 master -> its BF16 view), called with amp_C.multi_tensor_adam's signature by fairseq's
FusedAdamV2.step, recording in ``.cast`` the masters whose BF16 copy it wrote.  Differences, all internal:
  * one multi-tensor launch covers every tensor of the call (tables cached by address), instead of one
    Triton launch per tensor;
  * ``fold`` / ``fold_factor`` (set by zero1_fast.step) let it read a master's BF16 gradient times the factor
    directly, instead of the FP32 gradient a separate scale pass would have written: the same products
    (g' = fp32(float(g16) * factor)), 6 bytes per element less traffic.
``scale_up`` keeps ``fused_adam_cast.py:84-89``'s signature.
"""
import torch

from . import ops

__all__ = ['FusedAdamCast', 'scale_up']


class FusedAdamCast:
    """Callable with amp_C.multi_tensor_adam's signature; dest: data_ptr of an fp32 master -> bf16 tensor to write
    (FusedAdamV2.step passes p.data, a new tensor object each call, so masters are matched by address)."""

    def __init__(self, dest):
        self.dest = dest
        self.cast = set()                 # data_ptrs of masters whose bf16 copy was written since the last clear
        self.fold = {}                    # data_ptr of a master -> bf16 gradient to read instead of its fp32 grad
        self.fold_factor = None           # 1-element fp32 device tensor multiplying the folded gradients
        self._tables = ops.TableCache()

    def __call__(self, chunk_size, noop_flag, tensor_lists, lr, beta1, beta2, eps, step, mode, bias_correction,
                 weight_decay):
        bc1, bc2 = ops.bias_corrections(beta1, beta2, step, bias_correction)
        if int(mode) not in (0, 1):
            raise RuntimeError(f'fused_adam_cast: unsupported adam mode {mode}')
        plain, folded, written = [], [], []
        for g, p, m, v in zip(*tensor_lists):
            if not (g.is_contiguous() and p.is_contiguous() and m.is_contiguous() and v.is_contiguous()
                    and g.dtype == p.dtype == m.dtype == v.dtype == torch.float32):
                raise RuntimeError('fused_adam_cast: expected contiguous fp32 tensors')
            n = p.numel()
            if not (g.numel() == m.numel() == v.numel() == n):
                raise RuntimeError('fused_adam_cast: tensor sizes differ within a row')
            d = self.dest.get(p.data_ptr())
            if d is not None:
                if d.dtype != torch.bfloat16 or not d.is_contiguous() or d.numel() != n:
                    raise RuntimeError('fused_adam_cast: the bf16 destination must be a contiguous bf16 view')
                written.append(p.data_ptr())
            g16 = self.fold.get(p.data_ptr())
            if g16 is not None:
                if g16.dtype != torch.bfloat16 or not g16.is_contiguous() or g16.numel() != n:
                    raise RuntimeError('fused_adam_cast: a folded gradient must be contiguous bf16')
                folded.append((g16, p, m, v, d, n))
            else:
                plain.append((g, p, m, v, d, n))
        if folded and self.fold_factor is None:
            raise RuntimeError('fused_adam_cast: folded gradients without a factor')
        for rows, factor in ((plain, None), (folded, self.fold_factor)):
            if rows:
                table = self._tables.get(rows, rows[0][1].device)
                ops.adam_cast(table, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, int(mode))
        self.cast.update(written)


def scale_up(g16, g32, factor):
    """g32 = float(g16) * factor (factor: 1-element fp32 tensor) -- the fp32 product of the exactly upcast value, as
    torch.mul(g16, factor, out=g32) computes it."""
    ops.scale_up(g16, g32, factor)
