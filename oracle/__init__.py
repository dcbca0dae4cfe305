"""CPU oracle for the ZeRO-1 shard update -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import this package, and only as
the checker (or, for bench.py, as the timed CPU baseline).  The product package never imports it.

NumPy wrappers over ``liboracle_z1.so`` (built from ``z1_oracle.c`` by ``oracle/Makefile``).  Each function states
the reference lines it restates; the C file holds the arithmetic.  Pinning: every function here is checked in
``tests/test_oracle_pins.py`` against an independent routine (torch CPU, torch.optim.AdamW, exact rationals,
closed forms or the known YOCO-3B partition).  Parity of the norm's *summation order* against apex's
``multi_tensor_l2norm`` is unpinned (third-party binary, absent); the norm is pinned to the exact value instead.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, 'liboracle_z1.so')
_LIB = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int


def build():
    """Compile the oracle with its Makefile (gcc, IEEE flags)."""
    import subprocess
    subprocess.run(['make', '-s', '-C', _HERE, 'liboracle_z1.so'], check=True)


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_bf16_rne.argtypes = [_F]
        L.oracle_bf16_rne.restype = ctypes.c_uint16
        L.oracle_bf16_rne_array.argtypes = [_P, _P, _I64]
        L.oracle_owner_sum.argtypes = [_P, _I, _I64, _F, _P, _P]
        L.oracle_sum_slots.argtypes = [_P, _P, _I64, _I64, _I64, _I, _F, _I]
        L.oracle_scale_up.argtypes = [_P, _P, _F, _I64]
        L.oracle_sumsq_f32.argtypes = [_P, _I64]
        L.oracle_sumsq_f32.restype = ctypes.c_double
        L.oracle_sumsq_bf16.argtypes = [_P, _I64]
        L.oracle_sumsq_bf16.restype = ctypes.c_double
        L.oracle_norm_clip.argtypes = [ctypes.c_double, _F, _F, _P]
        L.oracle_clip_factor.argtypes = [_F, _F, _F, _P]
        L.oracle_update_scalars.argtypes = [ctypes.c_double, _I, _F, _F, _F, _F, _P]
        L.oracle_bias_corrections.argtypes = [ctypes.c_double, ctypes.c_double, _I64, _I, _P]
        L.oracle_adam_cast.argtypes = [_P, _I, _P, _P, _P, _P, _I64, _F, _I, _F, _F, _F, _F, _F, _F, _F, _I]
        L.oracle_greedy_partition.argtypes = [_P, _I, _I, _P, _P]
        L.oracle_embedding_backward.argtypes = [_P, _P, _I64, _I64, _I64, _I64, _F, _I, _P]
        L.oracle_embedding_backward_chunked.argtypes = [_P, _P, _I64, _I64, _I64, _I64, _F, _I, _I64, _P]
        _LIB = L
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    a = np.ascontiguousarray(a)
    if a.dtype != dtype:
        raise TypeError(f'oracle: expected {dtype}, got {a.dtype}')
    return a


def bf16_rne(x):
    """float32 array -> uint16 bfloat16 bits, round to nearest even (NaN -> 0x7FC0)."""
    x = _c(np.asarray(x, dtype=np.float32), np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_bf16_rne_array(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(h):
    """uint16 bfloat16 bits -> float32 (exact)."""
    h = np.asarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def owner_sum(contribs, scale=None, want_sum=False):
    """ce_reduce.py:59-74 over contributions in rank order.  contribs: list of uint16 (bf16 bits) arrays, equal n.
    Returns avg16 (uint16) or (avg16, fp32 sum)."""
    world = len(contribs)
    cs = [_c(c, np.uint16) for c in contribs]
    n = cs[0].size
    if any(c.size != n for c in cs):
        raise ValueError('oracle: contributions differ in size')
    scale = np.float32(1.0 / world) if scale is None else np.float32(scale)
    ptrs = (ctypes.c_void_p * world)(*[c.ctypes.data for c in cs])
    out = np.empty(n, dtype=np.uint16)
    s = np.empty(n, dtype=np.float32) if want_sum else None
    lib().oracle_owner_sum(ctypes.cast(ptrs, ctypes.c_void_p), world, n, float(scale), _ptr(out),
                           _ptr(s) if want_sum else None)
    return (out, s) if want_sum else out


def sum_slots(S, OUT, G, base, end, R, scale, W):
    """ce_reduce.py:60-74 with the reference's staging layout; OUT (uint16) is updated in place."""
    S = _c(S, np.uint16)
    if OUT.dtype != np.uint16 or not OUT.flags.c_contiguous:
        raise TypeError('oracle: OUT must be contiguous uint16')
    lib().oracle_sum_slots(_ptr(S), _ptr(OUT), G, base, end, R, float(np.float32(scale)), W)
    return OUT


def scale_up(g16, factor):
    """fused_adam_cast.py:75-89: float(g16) * factor in fp32."""
    g16 = _c(g16, np.uint16)
    out = np.empty(g16.shape, dtype=np.float32)
    lib().oracle_scale_up(_ptr(g16), _ptr(out), float(np.float32(factor)), g16.size)
    return out


def sumsq(g):
    """Sequential FP64 sum of squares of the exact values of g (float32 array or uint16 bf16 bits)."""
    g = np.ascontiguousarray(g)
    if g.dtype == np.float32:
        return lib().oracle_sumsq_f32(_ptr(g), g.size)
    if g.dtype == np.uint16:
        return lib().oracle_sumsq_bf16(_ptr(g), g.size)
    raise TypeError(f'oracle: sumsq of {g.dtype}')


def norm_clip(sumsq_value, factor=1.0, max_norm=1.0):
    """zero1_fast.py:150-160 (one owner).  Returns (n_r, grad_norm, new_factor) as np.float32."""
    out = np.empty(3, dtype=np.float32)
    lib().oracle_norm_clip(float(sumsq_value), float(np.float32(factor)), float(np.float32(max_norm)), _ptr(out))
    return out[0], out[1], out[2]


def clip_factor(norm, factor=1.0, max_norm=1.0):
    """zero1_fast.py:155-160 entered at `norm`.  Returns (grad_norm, new_factor) as np.float32."""
    out = np.empty(2, dtype=np.float32)
    lib().oracle_clip_factor(float(np.float32(norm)), float(np.float32(factor)), float(np.float32(max_norm)),
                             _ptr(out))
    return out[0], out[1]


def update_scalars(sumsq_value, sample_size=None, numer=1.0, factor=1.0, max_norm=1.0):
    """trainer_nosync.py:273-285 + zero1_fast.py:150-160 (one owner) + the "clip" metric (:194-197).
    Returns dict(norm, grad_norm, factor, finite, consistent, clip_log) as np.float32 / bool / None."""
    out = np.empty(6, dtype=np.float32)
    lib().oracle_update_scalars(float(sumsq_value), int(sample_size is not None),
                                float(np.float32(0.0 if sample_size is None else sample_size)),
                                float(np.float32(numer)), float(np.float32(factor)), float(np.float32(max_norm)),
                                _ptr(out))
    return dict(norm=out[0], grad_norm=out[1], factor=out[2], finite=bool(out[3]), consistent=bool(out[4]),
                clip_log=None if out[5] < 0 else out[5])


def bias_corrections(beta1, beta2, step, bias_correction=1):
    """fused_adam_cast.py:58-60.  Returns (bc1, bc2) as np.float32."""
    out = np.empty(2, dtype=np.float32)
    lib().oracle_bias_corrections(float(beta1), float(beta2), int(step), int(bias_correction), _ptr(out))
    return out[0], out[1]


def adam_cast(g, p, m, v, *, lr, beta1, beta2, eps, weight_decay, step, mode=1, bias_correction=1, factor=None,
              want_bf16=True):
    """fused_adam_cast.py:19-72 (+ the folded gradient factor of zero1_fast.py:175-192).  Inputs are not modified.
    g: float32 array or uint16 (bf16 bits).  Hyperparameters are Python floats, rounded to fp32 as Triton's scalar
    arguments are.  Returns (p', m', v', p16') with p16' None unless want_bf16."""
    g = np.ascontiguousarray(g)
    if g.dtype not in (np.float32, np.uint16):
        raise TypeError(f'oracle: g dtype {g.dtype}')
    p = _c(p, np.float32).copy()
    m = _c(m, np.float32).copy()
    v = _c(v, np.float32).copy()
    n = p.size
    if not (g.size == m.size == v.size == n):
        raise ValueError('oracle: size mismatch')
    bc1, bc2 = bias_corrections(beta1, beta2, step, bias_correction)
    p16 = np.empty(n, dtype=np.uint16) if want_bf16 else None
    f32 = lambda x: float(np.float32(x))
    lib().oracle_adam_cast(_ptr(g), int(g.dtype == np.uint16), _ptr(p), _ptr(m), _ptr(v),
                           _ptr(p16) if want_bf16 else None, n, f32(1.0 if factor is None else factor),
                           int(factor is not None), f32(lr), f32(beta1), f32(beta2), f32(eps), float(bc1), float(bc2),
                           f32(weight_decay), int(mode))
    return p, m, v, p16


SORT_PATH_MIN_ROWS = 3073         # aten.embedding_dense_backward sorts for more than 3072 indices
FEW_ROWS_CHUNK = 16               # index chunk of its kernel for fewer (torch's ROCm build, MI355X)


def embedding_backward(ids, grad16, num_weights, padding_idx=-1, scale=None, scale_first=False):
    """aten.embedding_dense_backward (+ the reference's optional 1/world) in aten's order for the row count: the
    sort-path order for more than 3072 rows, the chunked order for fewer.  ids: int64 [R]; grad16: uint16 bf16 bits
    [R, D].  Returns uint16 [V, D]."""
    R = np.asarray(grad16).shape[0]
    if R >= SORT_PATH_MIN_ROWS:
        return embedding_backward_sort(ids, grad16, num_weights, padding_idx, scale, scale_first)
    return embedding_backward_chunked(ids, grad16, num_weights, padding_idx, scale, scale_first)


def embedding_backward_sort(ids, grad16, num_weights, padding_idx=-1, scale=None, scale_first=False):
    """aten's sort-path order at any row count (runs of 10 occurrences), see z1_oracle.c."""
    ids = _c(np.asarray(ids, dtype=np.int64), np.int64)
    g = _c(grad16, np.uint16)
    R, D = g.shape
    out = np.empty((num_weights, D), dtype=np.uint16)
    mode = 0 if scale is None else (1 if scale_first else 2)
    lib().oracle_embedding_backward(_ptr(ids), _ptr(g), R, D, num_weights, padding_idx,
                                    float(np.float32(1.0 if scale is None else scale)), mode, _ptr(out))
    return out


def embedding_backward_chunked(ids, grad16, num_weights, padding_idx=-1, scale=None, scale_first=False,
                               chunk=FEW_ROWS_CHUNK):
    """aten's order for few rows at any row count (chunks of `chunk` indices, per-chunk bf16 rounding), see
    z1_oracle.c."""
    ids = _c(np.asarray(ids, dtype=np.int64), np.int64)
    g = _c(grad16, np.uint16)
    R, D = g.shape
    out = np.empty((num_weights, D), dtype=np.uint16)
    mode = 0 if scale is None else (1 if scale_first else 2)
    lib().oracle_embedding_backward_chunked(_ptr(ids), _ptr(g), R, D, num_weights, padding_idx,
                                            float(np.float32(1.0 if scale is None else scale)), mode, int(chunk),
                                            _ptr(out))
    return out


def greedy_partition(numels, world):
    """zero1_fast.py:61-65.  Returns (owner list, per-rank sizes)."""
    nums = np.asarray(numels, dtype=np.int64)
    owner = np.empty(len(nums), dtype=np.int32)
    sizes = np.empty(world, dtype=np.int64)
    lib().oracle_greedy_partition(_ptr(nums), len(nums), world, _ptr(owner), _ptr(sizes))
    return owner.tolist(), sizes.tolist()


def ulp_diff_f32(a, b):
    """Elementwise distance in units in the last place between two float32 arrays (monotone integer mapping)."""
    ai = np.asarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7fffffff), ai)
    bi = np.where(bi < 0, -(bi & 0x7fffffff), bi)
    return np.abs(ai - bi)


__all__ = ['bf16_rne', 'bf16_to_f32', 'owner_sum', 'sum_slots', 'scale_up', 'sumsq', 'norm_clip', 'clip_factor',
           'update_scalars', 'bias_corrections', 'adam_cast', 'embedding_backward', 'greedy_partition',
           'ulp_diff_f32', 'build', 'lib']
