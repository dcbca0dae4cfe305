"""ctypes binding of ``libyoco_z1.so`` (the C ABI declared in ``include/yoco_z1.h``).

The library is loaded after ``import torch`` so that its HIP calls and code objects bind to the HIP runtime torch
already loaded (both carry the SONAME ``libamdhip64.so.7``): the streams torch hands out are then valid handles for
the library.  There is no fallback: a missing library, a CPU tensor or a failed launch raises ``RuntimeError``.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = 'libyoco_z1.so'
# YOCO_Z1_LIB selects another build of the same C ABI (e.g. an older build, for an A/B timing of two versions)
LIB_PATH = os.environ.get('YOCO_Z1_LIB') or os.path.join(_HERE, LIB_NAME)

Z1_F32 = 0
Z1_BF16 = 1
Z1_MAX_WORLD = 16
Z1_NORM_PARTIALS = 2048
Z1_NOALLOC_MAX_N = 1 << 29

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float


class Z1Tensor(ctypes.Structure):
    """One row of the tensor-offset table (``z1_tensor``)."""
    _fields_ = [('g', _P), ('p', _P), ('m', _P), ('v', _P), ('p16', _P), ('n', _I64)]


class Z1UpdateScalars(ctypes.Structure):
    """``z1_update_scalars``."""
    _fields_ = [('sample_size', _P), ('numer', _F), ('factor_in', _P), ('factor_value', _F), ('max_norm', _F),
                ('norm_out', _P), ('grad_norm_out', _P), ('factor_out', _P), ('flags_out', _P),
                ('clip_log_out', _P)]


# name -> (argtypes, restype); every function the header declares
SIGNATURES = {
    'z1_table_create': ([ctypes.POINTER(Z1Tensor), _I, _I, ctypes.POINTER(_P)], _I),
    'z1_table_destroy': ([_P], _I),
    'z1_table_info': ([_P, ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(_I)], _I),
    'z1_owner_sum_bf16': ([_P, _I, _I64, _F, _P, _P, _P, _P], _I),
    'z1_owner_sum_workspace': ([_I64], _I64),
    'z1_owner_sum_waves': ([_I64], _I64),
    'z1_owner_sum_bf16_waves': ([_P, _I, _I64, _F, _P, _P, _P, _P], _I),
    'z1_reduce_waves': ([_P, _I64, _P, _P], _I),
    'z1_owner_sum_update': ([_P, _I, _I64, _F, _P, _P, _P, ctypes.POINTER(Z1UpdateScalars), _P], _I),
    'z1_owner_sum_update_noalloc': ([_P, _I, _I64, _F, _P, _P, ctypes.POINTER(Z1UpdateScalars), _P], _I),
    'z1_table_set_grads': ([_P, _P, _I, _P], _I),
    'z1_table_rebind': ([_P, ctypes.POINTER(Z1Tensor), _I, _P], _I),
    'z1_table_set_grad_out': ([_P, _P, _I, _P], _I),
    'z1_grad_sumsq': ([_P, _P, _P], _I),
    'z1_grad_norm_clip': ([_P, _P, _P, _F, _P, _P, _P, _F, _P], _I),
    'z1_grad_update_scalars': ([_P, _P, ctypes.POINTER(Z1UpdateScalars), _P], _I),
    'z1_norm_clip': ([_P, _P, _F, _P, _P, _P, _F, _P], _I),
    'z1_clip_factor': ([_P, _P, _F, _P, _P, _F, _P], _I),
    'z1_update_scalars_run': ([_P, ctypes.POINTER(Z1UpdateScalars), _P], _I),
    'z1_adam_cast': ([_P, _P, _F, _F, _F, _F, _F, _F, _F, _I, _P], _I),
    'z1_adam_cast_dev': ([_P, _P, _F, _F, _F, _F, _P, _F, _I, _P], _I),
    'z1_adam_cast_rows': ([_P, _I, _I, _P, _F, _F, _F, _F, _F, _F, _F, _I, _P], _I),
    'z1_bias_corrections_step': ([_P, ctypes.c_double, ctypes.c_double, _I, _P, _P], _I),
    'z1_scale_up': ([_P, _P, _P, _I64, _P], _I),
    'z1_cast_bf16': ([_P, _P, _I64, _P], _I),
    'z1_embedding_backward': ([_P, _P, _I64, _I64, _I64, _I64, _F, _I, _P, _P, _I64, _P], _I),
    'z1_embedding_backward_workspace': ([_I64, _I64, _I64], _I64),
    'z1_strerror': ([_I], ctypes.c_char_p),
}

_LIB = None


def lib():
    """The loaded library; raises RuntimeError when it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f'yoco_z1: native library {LIB_PATH} is not built (run __graft_entry__.build())')
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = L
    return _LIB


def check(rc, what):
    if rc != 0:
        msg = lib().z1_strerror(rc)
        raise RuntimeError(f'yoco_z1: {what} failed: {msg.decode() if msg else "?"} (code {rc})')


def stream_handle(device=None):
    """hipStream_t of torch's current stream on `device`, as a ctypes pointer."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def require_gpu(t, what):
    if not (torch.is_tensor(t) and t.is_cuda):
        raise RuntimeError(f'{what}: expected a GPU tensor (there is no CPU path)')
