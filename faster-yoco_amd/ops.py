"""The public operations of the path, each a call of a ``torch.ops.yoco_z1`` operator (C++ over the C ABI, loaded by
``library.py``).  Every call enqueues on torch's current stream of the tensors' device and performs no host
synchronisation.  The calls allocate no device memory (tables and workspaces are made at set-up, by
``Table`` / ``TableCache`` / ``norm_workspace``), with one exception: a factor given as a tensor to be read but not
written (``factor_out`` None or another tensor) is copied first -- into ``factor_out`` when one is given, else into a
new tensor -- because the operators write the clipped factor over the one they read.  A Python-number factor and a
device output may be mixed as the reference's fairseq surface mixes them.

``table`` arguments are ``Table`` objects (``kernels.Table``); without explicit tensors an operation runs on the
tensors the table was made with (``Table.bound``).
"""
import torch

from . import kernels, library  # noqa: F401  (library registers the operators)
from ._lib import Z1_NORM_PARTIALS, lib
from .kernels import Table, TableCache, bias_corrections, f32, rows_lists  # noqa: F401

_OPS = torch.ops.yoco_z1


def norm_workspace(device, n=None):
    """Workspace of the norm partials: Z1_NORM_PARTIALS doubles, or (n given) enough for a fused owner sum over n
    elements (its first Z1_NORM_PARTIALS doubles are what norm_clip reads)."""
    size = Z1_NORM_PARTIALS if n is None else int(lib().z1_owner_sum_workspace(int(n)))
    return torch.empty(size, dtype=torch.float64, device=device)


def _bound(table):
    if table.bound is None:
        raise RuntimeError('yoco_z1: the table has no bound tensors; pass them explicitly')
    return table.bound


def _factor_io(factor, factor_out):
    """(in/out factor tensor, factor_value) for an operator from the public (factor, factor_out) pair: factor is a
    Python number or a 1-element fp32 device tensor (read); factor_out (None or a tensor, which may be factor)
    receives the clipped factor."""
    if torch.is_tensor(factor):
        if factor_out is factor:
            return factor, None
        if factor_out is None:
            return factor.clone(), None                  # read only: the chain writes to a copy
        factor_out.copy_(factor)
        return factor_out, None
    return factor_out, f32(1.0 if factor is None else factor)


# ------------------------------------------------------------------------------------------------------- norm
def grad_sumsq(table, partials, g=None):
    _OPS.grad_sumsq_(table.handle_int, _bound(table)[0] if g is None else g, partials)


def norm_clip(partials, factor=1.0, norm_out=None, grad_norm_out=None, factor_out=None, max_norm=0.0):
    """Final fixed-order reduction + the clip chain.  factor: Python number or 1-element fp32 device tensor (read);
    factor_out (nullable, may be `factor`) receives the clipped factor."""
    f, fv = _factor_io(factor, factor_out)
    _OPS.norm_clip_(partials, f, norm_out, grad_norm_out, f32(max_norm), fv)


def grad_norm_clip(table, partials, factor=1.0, norm_out=None, grad_norm_out=None, factor_out=None, max_norm=0.0,
                   g=None):
    """grad_sumsq + norm_clip in one call."""
    f, fv = _factor_io(factor, factor_out)
    _OPS.grad_norm_clip_(table.handle_int, _bound(table)[0] if g is None else g, partials, f, norm_out, grad_norm_out,
                         f32(max_norm), fv)


def update_scalars(partials, sample_size=None, numer=1.0, factor=1.0, max_norm=0.0, norm_out=None,
                   grad_norm_out=None, factor_out=None, flags_out=None, clip_log_out=None):
    """The trainer's per-update scalar chain in one launch: optional sample-size factor, norm + clip chain,
    [finite, consistent] flags (uint8[2]) and the "clip" metric."""
    f, fv = _factor_io(factor, factor_out)
    _OPS.update_scalars_(partials, f, norm_out, grad_norm_out, flags_out, clip_log_out, sample_size, f32(numer),
                         f32(max_norm), fv)


def grad_update_scalars(table, partials, sample_size=None, numer=1.0, factor=1.0, max_norm=0.0, norm_out=None,
                        grad_norm_out=None, factor_out=None, flags_out=None, clip_log_out=None, g=None):
    """grad_sumsq + update_scalars in one call."""
    f, fv = _factor_io(factor, factor_out)
    _OPS.grad_update_scalars_(table.handle_int, _bound(table)[0] if g is None else g, partials, f, norm_out,
                              grad_norm_out, flags_out, clip_log_out, sample_size, f32(numer), f32(max_norm), fv)


def clip_factor(norm, factor=1.0, grad_norm_out=None, factor_out=None, max_norm=0.0):
    """The clip chain entered at `norm` (1-element fp32 device tensor)."""
    f, fv = _factor_io(factor, factor_out)
    _OPS.clip_factor_(norm, f, grad_norm_out, f32(max_norm), fv)


# ------------------------------------------------------------------------------------------------ Adam + BF16
def adam_cast(table, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, mode, tensors=None, g32=None):
    """One multi-tensor Adam + BF16 launch over the table.  factor: 1-element fp32 device tensor or None.
    tensors: (g, p, m, v, p16) lists, by default the table's bound tensors.  g32: FP32 gradient outputs (one per
    row, an empty tensor for none, or the flat buffer): the launch also writes g' = fp32(g * factor) there, the
    master gradient the reference's scale pass writes (yoco/tasks/zero1_fast.py:175-192)."""
    adam_cast_rows(table, 0, table.nrows, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, mode, tensors, g32)


def adam_cast_rows(table, row_begin, row_end, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, mode,
                   tensors=None, g32=None):
    """adam_cast over the table rows [row_begin, row_end) only (indices of the rows the table was built from)."""
    if not 0 <= int(row_begin) <= int(row_end) <= table.nrows:
        raise RuntimeError(f'yoco_z1: rows [{row_begin}, {row_end}) outside the table\'s {table.nrows} rows')
    if table.numel == 0 or row_begin == row_end:
        return                                           # nothing to update (and no tensor to dispatch on)
    g, p, m, v, p16 = _bound(table) if tensors is None else tensors
    args = (factor, f32(lr), f32(beta1), f32(beta2), f32(eps), f32(bc1), f32(bc2), f32(weight_decay), int(mode),
            int(row_begin), int(row_end))
    if g32 is None:
        _OPS.adam_cast_(table.handle_int, g, p, m, v, p16, *args)
    else:
        _OPS.adam_cast_gout_(table.handle_int, g, p, m, v, p16, list(g32), *args)


def adam_cast_dev(table, factor, lr, beta1, beta2, eps, bc, weight_decay, mode, tensors=None):
    """adam_cast with the bias corrections read from bc (2-element fp32 device tensor) when the kernel runs."""
    if table.numel == 0:
        return
    g, p, m, v, p16 = _bound(table) if tensors is None else tensors
    _OPS.adam_cast_dev_(table.handle_int, g, p, m, v, p16, factor, bc, f32(lr), f32(beta1), f32(beta2), f32(eps),
                        f32(weight_decay), int(mode))


def bias_corrections_step(step, beta1, beta2, bc, bias_correction=1):
    """On the device: step += 1, bc = fp32(1 - beta**step) in double (yoco/tasks/fused_adam_cast.py:58-60).
    step: 1-element int64 device tensor; bc: 2-element fp32 device tensor."""
    _OPS.bias_corrections_step_(step, bc, float(beta1), float(beta2), int(bias_correction))


# ------------------------------------------------------------------------------------------------- owner sum
def owner_sum(contribs, out, scale, out_sum=None, partials=None):
    """out[e] = bf16(sum_k float(contribs[k][e]) * scale), k in list order.  contribs: bf16 tensors of
    out.numel() elements each (sum_slots is the form where out holds one rank's own contribution)."""
    _OPS.owner_sum_(list(contribs), out, f32(scale), out_sum, partials)


def owner_sum_update(contribs, out, scale, workspace, out_sum=None, sample_size=None, numer=1.0, factor=1.0,
                     max_norm=0.0, norm_out=None, grad_norm_out=None, factor_out=None, flags_out=None,
                     clip_log_out=None):
    """owner_sum with the fused norm, then the update_scalars chain on its partials, in one call.
    workspace: norm_workspace(device, out.numel())."""
    if workspace is None:
        raise RuntimeError('yoco_z1: owner_sum_update needs its workspace')
    f, fv = _factor_io(factor, factor_out)
    _OPS.owner_sum_update_(list(contribs), out, workspace, f32(scale), out_sum, f, norm_out, grad_norm_out,
                           flags_out, clip_log_out, sample_size, f32(numer), f32(max_norm), fv)


def sum_slots(S, OUT, G, BASE, END, R, scale, WORLD, waves=None):
    """The owner sum in the reference's staging layout, in place (yoco/models/decoder/ce_reduce.py:59-74).  waves
    (float64, at least owner_sum_waves(END - BASE)): the range's norm partials per chunk, for reduce_waves."""
    _OPS.sum_slots_(S, OUT, int(G), int(BASE), int(END), int(R), f32(scale), int(WORLD), waves)


def owner_sum_waves(n):
    """Per-chunk norm partials an owner sum over n elements leaves (sum_slots' waves)."""
    return int(lib().z1_owner_sum_waves(int(n)))


def reduce_waves(waves, m, partials):
    """The first m per-chunk partials of waves, reduced in a fixed order into the norm partials (norm_workspace)
    that norm_clip / update_scalars read."""
    _OPS.reduce_waves_(waves, int(m), partials)


# ------------------------------------------------------------------------------------------------ scale / cast
def scale_up(g16, g32, factor):
    """g32 = float(g16) * factor[0] (yoco/tasks/fused_adam_cast.py:84-89)."""
    _OPS.scale_up_(g16, g32, factor)


def cast_bf16(p32, p16):
    """p16 = bf16(p32), round to nearest even."""
    _OPS.cast_bf16_(p32, p16)
