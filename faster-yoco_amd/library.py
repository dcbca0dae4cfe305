"""The path's kernels as PyTorch operators (namespace ``yoco_z1``).

The operators live in ``libyoco_z1_torch.so`` (``csrc/z1_torch_ops.cpp``): their schemas declare the tensors each
writes (``Tensor(a!)``), their CUDA (HIP) kernels check the arguments, bind the table and call the C ABI of
``libyoco_z1.so`` on torch's current stream, and their CPU kernels only raise (there is no CPU implementation).
This module loads that library, binds it to the C ABI library the process loaded (``_lib.LIB_PATH``), and registers
the operators' fake implementations for tracing.  Being operators, the launches are visible to ``torch.compile`` (no
graph break; functionalization may run an operator on copies of its mutable arguments, which the tables follow), to
``torch.profiler`` and to ``torch.library.opcheck``.  The reference's Triton launches replaced here are
yoco/tasks/fused_adam_cast.py:68-70,88-89 and yoco/models/decoder/ce_reduce.py:182; the norm and clip chain replace
yoco/tasks/zero1_fast.py:150-160.

Host cost: an operator call from Python is torch's dispatch (about 3 us) plus the C++ kernel; the table binding
costs nanoseconds per row.  (A ``torch.library.custom_op`` with Python kernels took about 19 us per call before any
work, plus microseconds per tensor for the checks and binding in Python.)  The operators make no version-counter
bumps of the tensors they write, as the reference's Triton launches make none; none is ever differentiated.

Tables are named by ``table`` (``kernels.Table.handle_int``; ``kernels.Table`` registers each table it creates).
Operators over a table take the tensors it covers, one list per stream: for a flat table one buffer each (g, p, m,
v, p16), for a list table one tensor per row; an empty p16 list means no BF16 copy (an empty tensor in a list table:
none for that row).

Argument names avoid ``mode`` (a keyword of torch's functionalization wrapper, which passes operator arguments by
name).  Scalar outputs (factor, norm, grad_norm, clip_log: 1-element fp32; flags: 2 uint8) are optional.  The gradient
factor is read from ``factor`` and overwritten with the clipped one, unless ``factor_value`` is given: then it is the
factor read, and ``factor`` (if given) only receives the result.
"""
import ctypes
import os

import torch

from . import _lib

NS = 'yoco_z1'
OPS_LIB_NAME = 'libyoco_z1_torch.so'
OPS_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), OPS_LIB_NAME)


def _load():
    """Load the operator library and bind it to the C ABI library (raises RuntimeError when either is missing)."""
    if not os.path.exists(OPS_LIB_PATH):
        raise RuntimeError(f'yoco_z1: operator library {OPS_LIB_PATH} is not built (run __graft_entry__.build())')
    abi = _lib.lib()                                # first: the kernels, bound to torch's HIP runtime
    torch.ops.load_library(OPS_LIB_PATH)
    L = ctypes.CDLL(OPS_LIB_PATH)
    L.z1t_init.argtypes, L.z1t_init.restype = [ctypes.c_char_p], ctypes.c_int
    L.z1t_table_register.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.POINTER(_lib.Z1Tensor), ctypes.POINTER(ctypes.c_int64)]
    L.z1t_table_register.restype = ctypes.c_int
    L.z1t_table_forget.argtypes, L.z1t_table_forget.restype = [ctypes.c_void_p], None
    rc = L.z1t_init(abi._name.encode())
    if rc != 0:
        raise RuntimeError(f'yoco_z1: the operator library could not bind to {abi._name} (code {rc})')
    return L


OPS_LIB = _load()


def _none(*args, **kwargs):
    return None


def _embedding_fake(grad, indices, num_weights, padding_idx, scale, scale_mode, workspace):
    return grad.new_empty((num_weights, grad.shape[-1]), dtype=torch.bfloat16)


OPS = ('grad_sumsq_', 'norm_clip_', 'grad_norm_clip_', 'update_scalars_', 'grad_update_scalars_', 'clip_factor_',
       'adam_cast_', 'adam_cast_gout_', 'adam_cast_dev_', 'bias_corrections_step_', 'owner_sum_', 'owner_sum_update_',
       'sum_slots_', 'reduce_waves_', 'scale_up_', 'cast_bf16_', 'embedding_dense_backward_out_',
       'embedding_dense_backward')

for _name in OPS:
    torch.library.register_fake(f'{NS}::{_name}',
                                _embedding_fake if _name == 'embedding_dense_backward' else _none)
