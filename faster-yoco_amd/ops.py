"""Thin torch-tensor wrappers over the C ABI.  Every call enqueues on torch's current stream of the tensors'
device, performs no host synchronisation and no allocation (tables are built once, at set-up)."""
import ctypes
import math
from collections import OrderedDict

import torch

from ._lib import (Z1_BF16, Z1_F32, Z1_MAX_WORLD, Z1_NORM_PARTIALS, Z1Tensor, Z1UpdateScalars, check, lib, ptr,
                   require_gpu, stream_handle)

_GDTYPE = {torch.float32: Z1_F32, torch.bfloat16: Z1_BF16}


def f32(x):
    """Round a Python number to fp32 as a Triton / ctypes fp32 scalar argument receives it (RNE)."""
    return ctypes.c_float(float(x)).value


class Table:
    """Device-resident tensor-offset table over (g, p, m, v, p16) rows.  Holds only addresses: the caller keeps
    the tensors alive and unmoved while the table is used (as the reference's dest map of data_ptrs does,
    yoco/tasks/fused_adam_cast.py:49-50)."""

    def __init__(self, rows, device):
        """rows: sequence of (g, p, m, v, p16, n); tensors or None (p/m/v/p16), all on `device`."""
        self.device = torch.device(device)
        gd = None
        arr = (Z1Tensor * max(1, len(rows)))()
        for i, (g, p, m, v, p16, n) in enumerate(rows):
            if g is None:
                raise RuntimeError('yoco_z1: a table row has no gradient')
            code = _GDTYPE.get(g.dtype)
            if code is None or (gd is not None and code != gd):
                raise RuntimeError(f'yoco_z1: gradients must all be fp32 or all bf16, got {g.dtype}')
            gd = code
            for t in (g, p, m, v, p16):
                if t is not None:
                    require_gpu(t, 'yoco_z1')
                    if t.device != self.device:
                        raise RuntimeError('yoco_z1: table tensors on different devices')
            arr[i] = Z1Tensor(g.data_ptr(), p.data_ptr() if p is not None else None,
                              m.data_ptr() if m is not None else None, v.data_ptr() if v is not None else None,
                              p16.data_ptr() if p16 is not None else None, int(n))
        self.g_dtype = Z1_F32 if gd is None else gd
        self.nrows = len(rows)
        self.sizes = tuple(int(r[5]) for r in rows)
        self.grad_ptrs = tuple(r[0].data_ptr() for r in rows)      # the gradients the device rows point at now
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            check(lib().z1_table_create(arr, len(rows), self.g_dtype, ctypes.byref(h)), 'z1_table_create')
        self._h = h
        numel, nch, nr = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
        check(lib().z1_table_info(h, ctypes.byref(numel), ctypes.byref(nch), ctypes.byref(nr)), 'z1_table_info')
        self.numel, self.nchunks = numel.value, nch.value
        if nr.value != self.nrows:
            raise RuntimeError(f'yoco_z1: the table reports {nr.value} rows, {self.nrows} were given')

    @property
    def handle(self):
        return self._h

    def set_grads(self, grads):
        """Points the rows at new gradient tensors (one per row, same sizes and dtype), enqueued on the current
        stream; nothing is launched when the addresses are the ones the table holds."""
        if len(grads) != self.nrows:
            raise RuntimeError(f'yoco_z1: {len(grads)} gradients for a table of {self.nrows} rows')
        ptrs = []
        for g, n in zip(grads, self.sizes):
            if _GDTYPE.get(g.dtype) != self.g_dtype or g.numel() < n:
                raise RuntimeError('yoco_z1: a rebound gradient differs in dtype or size from its row')
            require_gpu(g, 'yoco_z1')
            if g.device != self.device:
                raise RuntimeError('yoco_z1: a rebound gradient is on another device')
            ptrs.append(g.data_ptr())
        ptrs = tuple(ptrs)
        if ptrs == self.grad_ptrs:
            return
        arr = (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)
        with torch.cuda.device(self.device):
            check(lib().z1_table_set_grads(self._h, ctypes.cast(arr, ctypes.c_void_p), self.nrows,
                                           stream_handle(self.device)), 'z1_table_set_grads')
        self.grad_ptrs = ptrs

    def close(self):
        h, self._h = getattr(self, '_h', None), None
        if h is not None and h.value:
            try:
                with torch.cuda.device(self.device):
                    lib().z1_table_destroy(h)
            except Exception:           # interpreter shutdown: the process frees device memory anyway
                pass

    def __del__(self):
        self.close()


class TableCache:
    """Tables keyed by the parameter / state addresses, sizes and gradient dtype of their rows (bounded, least
    recently used evicted).  Gradient addresses are not part of the key: a hit whose gradients moved (autograd
    allocates new ones after zero_grad drops them) is rebound on the stream (``Table.set_grads``), so steps neither
    allocate nor synchronise with the device.  ``builds`` counts the tables made."""

    def __init__(self, capacity=8):
        self.capacity = capacity
        self._d = OrderedDict()
        self.builds = 0

    def get(self, rows, device):
        key = (str(device),) + tuple((g.dtype, p.data_ptr() if p is not None else 0,
                                      m.data_ptr() if m is not None else 0, v.data_ptr() if v is not None else 0,
                                      p16.data_ptr() if p16 is not None else 0, int(n))
                                     for g, p, m, v, p16, n in rows)
        t = self._d.get(key)
        if t is None:
            t = Table(rows, device)
            self.builds += 1
            self._d[key] = t
            while len(self._d) > self.capacity:
                self._d.popitem(last=False)[1].close()
        else:
            self._d.move_to_end(key)
            t.set_grads([r[0] for r in rows])
        return t

    def clear(self):
        for t in self._d.values():
            t.close()
        self._d.clear()


def norm_workspace(device, n=None):
    """Workspace of the norm partials: Z1_NORM_PARTIALS doubles, or (n given) enough for a fused owner sum over n
    elements (its first Z1_NORM_PARTIALS doubles are what norm_clip reads)."""
    size = Z1_NORM_PARTIALS if n is None else int(lib().z1_owner_sum_workspace(int(n)))
    return torch.empty(size, dtype=torch.float64, device=device)


def _check_partials(partials, what):
    require_gpu(partials, what)
    if partials.dtype != torch.float64 or partials.numel() < Z1_NORM_PARTIALS:
        raise RuntimeError('yoco_z1: norm workspace must hold Z1_NORM_PARTIALS float64')


def grad_sumsq(table, partials):
    _check_partials(partials, 'grad_sumsq')
    with torch.cuda.device(table.device):
        check(lib().z1_grad_sumsq(table.handle, ptr(partials), stream_handle(table.device)), 'z1_grad_sumsq')


def _scalar(t, what):
    if t is None:
        return None
    require_gpu(t, what)
    if t.dtype != torch.float32 or t.numel() != 1:
        raise RuntimeError(f'{what}: expected a 1-element fp32 device tensor')
    return ptr(t)


def _factor_args(factor):
    """(device pointer or None, host value) for a fairseq-style factor: a Python number or a 1-element fp32
    device tensor."""
    if torch.is_tensor(factor):
        return _scalar(factor, 'factor'), 1.0
    return None, f32(1.0 if factor is None else factor)


def norm_clip(partials, factor=1.0, norm_out=None, grad_norm_out=None, factor_out=None, max_norm=0.0):
    """Final fixed-order reduction + the clip chain (include/yoco_z1.h).  factor: Python number or 1-element fp32
    device tensor (read); factor_out (nullable, may be `factor`) receives the clipped factor."""
    require_gpu(partials, 'norm_clip')
    dev = partials.device
    fin, fval = _factor_args(factor)
    with torch.cuda.device(dev):
        check(lib().z1_norm_clip(ptr(partials), fin, fval, _scalar(norm_out, 'norm_clip'),
                                 _scalar(grad_norm_out, 'norm_clip'), _scalar(factor_out, 'norm_clip'), f32(max_norm),
                                 stream_handle(dev)), 'z1_norm_clip')


def clip_factor(norm, factor=1.0, grad_norm_out=None, factor_out=None, max_norm=0.0):
    """The clip chain entered at `norm` (1-element fp32 device tensor)."""
    dev = norm.device
    fin, fval = _factor_args(factor)
    with torch.cuda.device(dev):
        check(lib().z1_clip_factor(_scalar(norm, 'clip_factor'), fin, fval, _scalar(grad_norm_out, 'clip_factor'),
                                   _scalar(factor_out, 'clip_factor'), f32(max_norm), stream_handle(dev)),
              'z1_clip_factor')


def _scalars_struct(what, sample_size=None, numer=1.0, factor=1.0, max_norm=0.0, norm_out=None,
                    grad_norm_out=None, factor_out=None, flags_out=None, clip_log_out=None):
    """z1_update_scalars for the given outputs (each a 1-element fp32 device tensor or None; flags_out 2 uint8)."""
    fin, fval = _factor_args(factor)
    if flags_out is not None:
        require_gpu(flags_out, what)
        if flags_out.dtype not in (torch.uint8, torch.bool) or flags_out.numel() < 2:
            raise RuntimeError(f'{what}: flags_out must hold 2 uint8/bool')
    return Z1UpdateScalars(_scalar(sample_size, what), f32(numer), fin, fval, f32(max_norm),
                           _scalar(norm_out, what), _scalar(grad_norm_out, what), _scalar(factor_out, what),
                           ptr(flags_out), _scalar(clip_log_out, what))


def update_scalars(partials, sample_size=None, numer=1.0, factor=1.0, max_norm=0.0, norm_out=None,
                   grad_norm_out=None, factor_out=None, flags_out=None, clip_log_out=None):
    """The trainer's per-update scalar chain in one launch (include/yoco_z1.h, z1_update_scalars): optional
    sample-size factor, norm + clip chain, [finite, consistent] flags (uint8[2]) and the "clip" metric."""
    require_gpu(partials, 'update_scalars')
    dev = partials.device
    u = _scalars_struct('update_scalars', sample_size, numer, factor, max_norm, norm_out, grad_norm_out, factor_out,
                        flags_out, clip_log_out)
    with torch.cuda.device(dev):
        check(lib().z1_update_scalars_run(ptr(partials), ctypes.byref(u), stream_handle(dev)), 'z1_update_scalars')


def grad_norm_clip(table, partials, factor=1.0, norm_out=None, grad_norm_out=None, factor_out=None, max_norm=0.0):
    """grad_sumsq + norm_clip in one call (the norm kernel, then the one-workgroup final kernel)."""
    _check_partials(partials, 'grad_norm_clip')
    fin, fval = _factor_args(factor)
    with torch.cuda.device(table.device):
        check(lib().z1_grad_norm_clip(table.handle, ptr(partials), fin, fval, _scalar(norm_out, 'grad_norm_clip'),
                                      _scalar(grad_norm_out, 'grad_norm_clip'), _scalar(factor_out, 'grad_norm_clip'),
                                      f32(max_norm), stream_handle(table.device)), 'z1_grad_norm_clip')


def grad_update_scalars(table, partials, sample_size=None, numer=1.0, factor=1.0, max_norm=0.0, norm_out=None,
                        grad_norm_out=None, factor_out=None, flags_out=None, clip_log_out=None):
    """grad_sumsq + update_scalars in one call."""
    _check_partials(partials, 'grad_update_scalars')
    u = _scalars_struct('grad_update_scalars', sample_size, numer, factor, max_norm, norm_out, grad_norm_out,
                        factor_out, flags_out, clip_log_out)
    with torch.cuda.device(table.device):
        check(lib().z1_grad_update_scalars(table.handle, ptr(partials), ctypes.byref(u), stream_handle(table.device)),
              'z1_grad_update_scalars')


def bias_corrections(beta1, beta2, step, bias_correction=1):
    """yoco/tasks/fused_adam_cast.py:58-60: 1 - beta**step in double, rounded once to fp32."""
    if bias_correction == 1:
        return f32(1.0 - math.pow(beta1, step)), f32(1.0 - math.pow(beta2, step))
    return 1.0, 1.0


def adam_cast(table, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, mode):
    """One multi-tensor Adam + BF16 launch over the table.  factor: 1-element fp32 device tensor or None."""
    with torch.cuda.device(table.device):
        check(lib().z1_adam_cast(table.handle, _scalar(factor, 'adam_cast'), f32(lr), f32(beta1), f32(beta2),
                                 f32(eps), f32(bc1), f32(bc2), f32(weight_decay), int(mode),
                                 stream_handle(table.device)), 'z1_adam_cast')


def adam_cast_rows(table, row_begin, row_end, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, mode):
    """adam_cast over the table rows [row_begin, row_end) only (indices of the rows the table was built from)."""
    if not 0 <= int(row_begin) <= int(row_end) <= table.nrows:
        raise RuntimeError(f'yoco_z1: rows [{row_begin}, {row_end}) outside the table\'s {table.nrows} rows')
    with torch.cuda.device(table.device):
        check(lib().z1_adam_cast_rows(table.handle, int(row_begin), int(row_end), _scalar(factor, 'adam_cast_rows'),
                                      f32(lr), f32(beta1), f32(beta2), f32(eps), f32(bc1), f32(bc2),
                                      f32(weight_decay), int(mode), stream_handle(table.device)), 'z1_adam_cast_rows')


def adam_cast_dev(table, factor, lr, beta1, beta2, eps, bc, weight_decay, mode):
    """adam_cast with the bias corrections read from bc (2-element fp32 device tensor) when the kernel runs."""
    require_gpu(bc, 'adam_cast_dev')
    if bc.dtype != torch.float32 or bc.numel() < 2 or not bc.is_contiguous():
        raise RuntimeError('yoco_z1: bias corrections must be a contiguous 2-element fp32 tensor')
    with torch.cuda.device(table.device):
        check(lib().z1_adam_cast_dev(table.handle, _scalar(factor, 'adam_cast_dev'), f32(lr), f32(beta1), f32(beta2),
                                     f32(eps), ptr(bc), f32(weight_decay), int(mode), stream_handle(table.device)),
              'z1_adam_cast_dev')


def bias_corrections_step(step, beta1, beta2, bc, bias_correction=1):
    """On the device: step += 1, bc = fp32(1 - beta**step) in double (yoco/tasks/fused_adam_cast.py:58-60).
    step: 1-element int64 device tensor; bc: 2-element fp32 device tensor."""
    for t in (step, bc):
        require_gpu(t, 'bias_corrections_step')
    if (step.dtype != torch.int64 or step.numel() < 1 or bc.dtype != torch.float32 or bc.numel() < 2
            or not bc.is_contiguous() or step.device != bc.device):
        raise RuntimeError('yoco_z1: bias_corrections_step takes an int64 step and a contiguous 2-element fp32 bc '
                           'on one device')
    with torch.cuda.device(step.device):
        check(lib().z1_bias_corrections_step(ptr(step), float(beta1), float(beta2), int(bias_correction), ptr(bc),
                                             stream_handle(step.device)), 'z1_bias_corrections_step')


def _owner_sum_args(contribs, out, out_sum, workspace):
    """Checked (host pointer array, world) for an owner-sum call."""
    require_gpu(out, 'owner_sum')
    if out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise RuntimeError('yoco_z1: owner_sum output must be a contiguous bf16 tensor')
    world = len(contribs)
    if not 1 <= world <= Z1_MAX_WORLD:
        raise RuntimeError(f'yoco_z1: owner_sum takes 1..{Z1_MAX_WORLD} contributions, got {world}')
    addrs = []
    for c in contribs:
        if isinstance(c, int):
            addrs.append(c)
            continue
        require_gpu(c, 'owner_sum')
        if c.dtype != torch.bfloat16 or not c.is_contiguous() or c.numel() != out.numel() or c.device != out.device:
            raise RuntimeError('yoco_z1: owner_sum contributions must be contiguous bf16 tensors like out')
        addrs.append(c.data_ptr())
    if out_sum is not None:
        require_gpu(out_sum, 'owner_sum')
        if out_sum.dtype != torch.float32 or not out_sum.is_contiguous() or out_sum.numel() != out.numel():
            raise RuntimeError('yoco_z1: owner_sum out_sum must be a contiguous fp32 tensor like out')
    if workspace is not None:
        require_gpu(workspace, 'owner_sum')
        need = int(lib().z1_owner_sum_workspace(out.numel()))
        if workspace.dtype != torch.float64 or workspace.numel() < need or not workspace.is_contiguous():
            raise RuntimeError(f'yoco_z1: the fused-norm workspace must hold {need} float64 '
                               f'(ops.norm_workspace(device, n))')
    return (ctypes.c_void_p * world)(*addrs), world


def owner_sum(contribs, out, scale, out_sum=None, partials=None):
    """out[e] = bf16(sum_k float(contribs[k][e]) * scale), k in list order.  contribs: bf16 tensors (or raw
    device addresses as ints) of out.numel() elements each; out may be one of them."""
    arr, world = _owner_sum_args(contribs, out, out_sum, partials)
    with torch.cuda.device(out.device):
        check(lib().z1_owner_sum_bf16(ctypes.cast(arr, ctypes.c_void_p), world, out.numel(), f32(scale), ptr(out),
                                      ptr(out_sum), ptr(partials), stream_handle(out.device)), 'z1_owner_sum_bf16')


def owner_sum_update(contribs, out, scale, workspace, out_sum=None, sample_size=None, numer=1.0, factor=1.0,
                     max_norm=0.0, norm_out=None, grad_norm_out=None, factor_out=None, flags_out=None,
                     clip_log_out=None):
    """owner_sum with the fused norm, then the update_scalars chain on its partials, in one call
    (z1_owner_sum_update).  workspace: ops.norm_workspace(device, out.numel())."""
    if workspace is None:
        raise RuntimeError('yoco_z1: owner_sum_update needs its workspace')
    arr, world = _owner_sum_args(contribs, out, out_sum, workspace)
    u = _scalars_struct('owner_sum_update', sample_size, numer, factor, max_norm, norm_out, grad_norm_out,
                        factor_out, flags_out, clip_log_out)
    with torch.cuda.device(out.device):
        check(lib().z1_owner_sum_update(ctypes.cast(arr, ctypes.c_void_p), world, out.numel(), f32(scale), ptr(out),
                                        ptr(out_sum), ptr(workspace), ctypes.byref(u), stream_handle(out.device)),
              'z1_owner_sum_update')


def owner_sum_raw(addrs, n, out_addr, scale, device):
    """owner_sum on raw device addresses (the reference's slot layout, yoco/models/decoder/ce_reduce.py:59-74)."""
    arr = (ctypes.c_void_p * len(addrs))(*addrs)
    with torch.cuda.device(device):
        check(lib().z1_owner_sum_bf16(ctypes.cast(arr, ctypes.c_void_p), len(addrs), int(n), f32(scale),
                                      ctypes.c_void_p(out_addr), None, None, stream_handle(device)),
              'z1_owner_sum_bf16')


def scale_up(g16, g32, factor):
    """g32 = float(g16) * factor[0] (yoco/tasks/fused_adam_cast.py:84-89)."""
    for t in (g16, g32, factor):
        require_gpu(t, 'scale_up')
    if g16.dtype != torch.bfloat16 or g32.dtype != torch.float32 or g16.numel() != g32.numel():
        raise RuntimeError('yoco_z1: scale_up expects bf16 -> fp32 of equal size')
    if not (g16.is_contiguous() and g32.is_contiguous()):
        raise RuntimeError('yoco_z1: scale_up expects contiguous tensors')
    with torch.cuda.device(g32.device):
        check(lib().z1_scale_up(ptr(g16), ptr(g32), _scalar(factor.reshape(-1)[:1], 'scale_up'), g16.numel(),
                                stream_handle(g32.device)), 'z1_scale_up')


def cast_bf16(p32, p16):
    """p16 = bf16(p32), round to nearest even."""
    for t in (p32, p16):
        require_gpu(t, 'cast_bf16')
    if p32.dtype != torch.float32 or p16.dtype != torch.bfloat16 or p32.numel() != p16.numel():
        raise RuntimeError('yoco_z1: cast_bf16 expects fp32 -> bf16 of equal size')
    if not (p32.is_contiguous() and p16.is_contiguous()):
        raise RuntimeError('yoco_z1: cast_bf16 expects contiguous tensors')
    with torch.cuda.device(p32.device):
        check(lib().z1_cast_bf16(ptr(p32), ptr(p16), p32.numel(), stream_handle(p32.device)), 'z1_cast_bf16')
