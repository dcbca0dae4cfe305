"""The path's kernels as PyTorch custom operators (namespace ``yoco_z1``), over the C ABI of libyoco_z1.so.

Each operator declares the tensors it writes (``mutates_args``), has a fake implementation for tracing, and runs
for the CUDA (HIP) dispatch key; its CPU kernel only raises (there is no CPU implementation).  Being operators, the launches are visible to ``torch.compile`` (no graph break; functionalization
may run an operator on copies of its mutable arguments, which the tables follow, see ``kernels.Table.bind``), to
``torch.profiler`` and to ``torch.library.opcheck``.  The reference's Triton launches replaced here are
yoco/tasks/fused_adam_cast.py:68-70,88-89 and yoco/models/decoder/ce_reduce.py:182; the norm and clip chain replace
yoco/tasks/zero1_fast.py:150-160.

Tables are named by ``table`` (``kernels.Table.handle_int``).  Operators over a table take the tensors it covers,
one list per stream: for a flat table one buffer each (g, p, m, v, p16), for a list table one tensor per row; an
empty p16 list means no BF16 copy (an empty tensor in a list table: none for that row).

Argument names avoid ``mode`` (a keyword of torch's functionalization wrapper, which passes operator arguments by
name).  Scalar outputs (factor, norm, grad_norm, clip_log: 1-element fp32; flags: 2 uint8) are optional.  The gradient
factor is read from ``factor`` and overwritten with the clipped one, unless ``factor_value`` is given: then it is the
factor read, and ``factor`` (if given) only receives the result.
"""
from typing import List, Optional

import torch
from torch import Tensor

from . import kernels as K

NS = 'yoco_z1'


def _op(name, mutates):
    return torch.library.custom_op(f'{NS}::{name}', mutates_args=mutates, device_types='cuda')


def _none(*args, **kwargs):
    return None


# ------------------------------------------------------------------------------------------------------- norm
@_op('grad_sumsq_', ('partials',))
def grad_sumsq_(table: int, g: List[Tensor], partials: Tensor) -> None:
    """Z1_NORM_PARTIALS fixed-order FP64 partials of the sum of squares of the table's gradients."""
    K.grad_sumsq(K.table_of(table), g, partials)


@_op('norm_clip_', ('factor', 'norm', 'grad_norm'))
def norm_clip_(partials: Tensor, factor: Optional[Tensor], norm: Optional[Tensor], grad_norm: Optional[Tensor],
               max_norm: float, factor_value: Optional[float]) -> None:
    """Final reduction of the partials + the clip chain of zero1_fast.py:150-160."""
    K.norm_clip(partials, factor, factor_value, norm, grad_norm, max_norm)


@_op('grad_norm_clip_', ('partials', 'factor', 'norm', 'grad_norm'))
def grad_norm_clip_(table: int, g: List[Tensor], partials: Tensor, factor: Optional[Tensor], norm: Optional[Tensor],
                    grad_norm: Optional[Tensor], max_norm: float, factor_value: Optional[float]) -> None:
    """grad_sumsq_ then norm_clip_ in one call."""
    K.grad_norm_clip(K.table_of(table), g, partials, factor, factor_value, norm, grad_norm, max_norm)


@_op('update_scalars_', ('factor', 'norm', 'grad_norm', 'flags', 'clip_log'))
def update_scalars_(partials: Tensor, factor: Optional[Tensor], norm: Optional[Tensor], grad_norm: Optional[Tensor],
                    flags: Optional[Tensor], clip_log: Optional[Tensor], sample_size: Optional[Tensor], numer: float,
                    max_norm: float, factor_value: Optional[float]) -> None:
    """The trainer's scalar chain (trainer_nosync.py:273-286, :194-197): sample-size factor, norm + clip,
    [finite, consistent] flags, "clip" metric."""
    K.update_scalars(partials, factor, factor_value, norm, grad_norm, flags, clip_log, sample_size, numer, max_norm)


@_op('grad_update_scalars_', ('partials', 'factor', 'norm', 'grad_norm', 'flags', 'clip_log'))
def grad_update_scalars_(table: int, g: List[Tensor], partials: Tensor, factor: Optional[Tensor],
                         norm: Optional[Tensor], grad_norm: Optional[Tensor], flags: Optional[Tensor],
                         clip_log: Optional[Tensor], sample_size: Optional[Tensor], numer: float, max_norm: float,
                         factor_value: Optional[float]) -> None:
    """grad_sumsq_ then update_scalars_ in one call."""
    K.grad_update_scalars(K.table_of(table), g, partials, factor, factor_value, norm, grad_norm, flags, clip_log,
                          sample_size, numer, max_norm)


@_op('clip_factor_', ('factor', 'grad_norm'))
def clip_factor_(norm: Tensor, factor: Optional[Tensor], grad_norm: Optional[Tensor], max_norm: float,
                 factor_value: Optional[float]) -> None:
    """The clip chain entered at a given norm (aggregate_norm_fn, zero1_fast.py:153-160)."""
    K.clip_factor(norm, factor, factor_value, grad_norm, max_norm)


# ------------------------------------------------------------------------------------------------ Adam + BF16
@_op('adam_cast_', ('p', 'm', 'v', 'p16'))
def adam_cast_(table: int, g: List[Tensor], p: List[Tensor], m: List[Tensor], v: List[Tensor], p16: List[Tensor],
               factor: Optional[Tensor], lr: float, beta1: float, beta2: float, eps: float, bc1: float, bc2: float,
               weight_decay: float, adam_mode: int, row_begin: int, row_end: int) -> None:
    """Adam + BF16 copy over the table rows [row_begin, row_end) (fused_adam_cast.py:19-45), the gradient factor
    folded into the load (scale_up, :75-89); adam_mode 1 decoupled weight decay, 0 L2."""
    K.adam_cast(K.table_of(table), g, p, m, v, p16, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, adam_mode,
                row_begin, row_end)


@_op('adam_cast_dev_', ('p', 'm', 'v', 'p16'))
def adam_cast_dev_(table: int, g: List[Tensor], p: List[Tensor], m: List[Tensor], v: List[Tensor], p16: List[Tensor],
                   factor: Optional[Tensor], bc: Tensor, lr: float, beta1: float, beta2: float, eps: float,
                   weight_decay: float, adam_mode: int) -> None:
    """adam_cast_ over the whole table with the bias corrections read from device memory (bc: 2 fp32)."""
    K.adam_cast_dev(K.table_of(table), g, p, m, v, p16, factor, lr, beta1, beta2, eps, bc, weight_decay, adam_mode)


@_op('bias_corrections_step_', ('step', 'bc'))
def bias_corrections_step_(step: Tensor, bc: Tensor, beta1: float, beta2: float, bias_correction: int) -> None:
    """On the device: step += 1; bc = fp32(1 - beta**step) in double (fused_adam_cast.py:58-60)."""
    K.bias_corrections_step(step, bc, beta1, beta2, bias_correction)


# ------------------------------------------------------------------------------------------------- owner sum
@_op('owner_sum_', ('out', 'out_sum', 'partials'))
def owner_sum_(contribs: List[Tensor], out: Tensor, scale: float, out_sum: Optional[Tensor],
               partials: Optional[Tensor]) -> None:
    """out = bf16(sum_k float(contribs[k]) * scale) in list order (ce_reduce.py:59-74); with partials, the norm of
    out fused in.  out must not be one of the contributions here (sum_slots_ is the in-place form)."""
    K.owner_sum(contribs, out, scale, out_sum, partials)


@_op('owner_sum_update_', ('out', 'workspace', 'out_sum', 'factor', 'norm', 'grad_norm', 'flags', 'clip_log'))
def owner_sum_update_(contribs: List[Tensor], out: Tensor, workspace: Tensor, scale: float, out_sum: Optional[Tensor],
                      factor: Optional[Tensor], norm: Optional[Tensor], grad_norm: Optional[Tensor],
                      flags: Optional[Tensor], clip_log: Optional[Tensor], sample_size: Optional[Tensor],
                      numer: float, max_norm: float, factor_value: Optional[float]) -> None:
    """owner_sum_ with the fused norm, then update_scalars_ on its partials, in one call."""
    K.owner_sum_update(contribs, out, scale, workspace, out_sum, factor, factor_value, norm, grad_norm, flags,
                       clip_log, sample_size, numer, max_norm)


@_op('sum_slots_', ('out',))
def sum_slots_(staging: Tensor, out: Tensor, G: int, base: int, end: int, rank: int, scale: float,
               world: int) -> None:
    """The owner sum in the reference's staging layout, in place in out[base:end] (ce_reduce.py:59-74,178-183)."""
    K.sum_slots(staging, out, G, base, end, rank, scale, world)


# ------------------------------------------------------------------------------------------------ scale / cast
@_op('scale_up_', ('g32',))
def scale_up_(g16: Tensor, g32: Tensor, factor: Tensor) -> None:
    """g32 = float(g16) * factor[0] (fused_adam_cast.py:75-89)."""
    K.scale_up(g16, g32, factor)


@_op('cast_bf16_', ('p16',))
def cast_bf16_(p32: Tensor, p16: Tensor) -> None:
    """p16 = bf16(p32), round to nearest even (zero1_fast.py:198-209)."""
    K.cast_bf16(p32, p16)


# --------------------------------------------------------------------------------------- embedding gradient
@_op('embedding_dense_backward_out_', ('out', 'workspace'))
def embedding_dense_backward_out_(grad: Tensor, indices: Tensor, num_weights: int, padding_idx: int, scale: float,
                                  scale_mode: int, out: Tensor, workspace: Tensor) -> None:
    """out[V, D] = aten.embedding_dense_backward(grad[R, D], indices[R], V, padding_idx, False) with the reference's
    x 1/world (scale_mode 1: rows first, ce_reduce.py:226-231; 2: after, layer_graphs.py:87-93; 0: none)."""
    K.embedding_backward(grad, indices, num_weights, padding_idx, scale, scale_mode, out, workspace)


@_op('embedding_dense_backward', ('workspace',))
def embedding_dense_backward(grad: Tensor, indices: Tensor, num_weights: int, padding_idx: int, scale: float,
                             scale_mode: int, workspace: Tensor) -> Tensor:
    """The functional form: returns a new bf16 [num_weights, D] tensor."""
    out = torch.empty(num_weights, grad.shape[-1], dtype=torch.bfloat16, device=grad.device)
    K.embedding_backward(grad, indices, num_weights, padding_idx, scale, scale_mode, out, workspace)
    return out


@embedding_dense_backward.register_fake
def _(grad, indices, num_weights, padding_idx, scale, scale_mode, workspace):
    return grad.new_empty((num_weights, grad.shape[-1]), dtype=torch.bfloat16)


for _mutating in (grad_sumsq_, norm_clip_, grad_norm_clip_, update_scalars_, grad_update_scalars_, clip_factor_,
                  adam_cast_, adam_cast_dev_, bias_corrections_step_, owner_sum_, owner_sum_update_, sum_slots_,
                  scale_up_, cast_bf16_, embedding_dense_backward_out_):
    _mutating.register_fake(_none)


def _refuse_cpu(name):
    def refuse(*args, **kwargs):
        raise RuntimeError(f'{NS}::{name}: expected GPU tensors (there is no CPU path)')
    return refuse


for _name in ('grad_sumsq_', 'norm_clip_', 'grad_norm_clip_', 'update_scalars_', 'grad_update_scalars_',
              'clip_factor_', 'adam_cast_', 'adam_cast_dev_', 'bias_corrections_step_', 'owner_sum_',
              'owner_sum_update_', 'sum_slots_', 'scale_up_', 'cast_bf16_', 'embedding_dense_backward_out_',
              'embedding_dense_backward'):
    # CPU tensors reach a kernel that only raises: the operators run on the GPU or not at all
    globals()[_name].register_kernel('cpu', _refuse_cpu(_name))

OPS = ('grad_sumsq_', 'norm_clip_', 'grad_norm_clip_', 'update_scalars_', 'grad_update_scalars_', 'clip_factor_',
       'adam_cast_', 'adam_cast_dev_', 'bias_corrections_step_', 'owner_sum_', 'owner_sum_update_', 'sum_slots_',
       'scale_up_', 'cast_bf16_', 'embedding_dense_backward_out_', 'embedding_dense_backward')
