"""The launches behind the PyTorch custom ops (``library.py``): ctypes calls into the C ABI of libyoco_z1.so on
torch tensors, plus the tensor-offset tables.  Every launch is enqueued on torch's current stream of the tensors'
device; nothing here synchronises with the device, and nothing allocates except a table's creation.

A table is a device-resident schedule over rows of given sizes.  It is bound to tensors: ``Table.bind`` points its
rows at the tensors a call passes (a stream-ordered launch, only when the addresses changed), so one table serves
tensors that move -- gradients that autograd reallocates each step, or the copies of the state that torch's
functionalization may hand to an op.  Two forms:

* flat: the rows are slices of flat buffers at fixed element offsets (``FlatShard``); a call passes the flat
  buffers, one per stream (g, p, m, v, p16);
* list: one tensor per row and stream; a BF16 destination may be an empty tensor (no copy for that row).
"""
import ctypes
import math
import weakref
from collections import OrderedDict

import torch

from ._lib import (Z1_BF16, Z1_F32, Z1_MAX_WORLD, Z1_NORM_PARTIALS, Z1Tensor, Z1UpdateScalars, check, lib, ptr,
                   require_gpu, stream_handle)

GDTYPE = {torch.float32: Z1_F32, torch.bfloat16: Z1_BF16}
_TABLES = weakref.WeakValueDictionary()      # handle (int) -> live Table, the tables the operators may name


def f32(x):
    """Round a Python number to fp32 as a Triton / ctypes fp32 scalar argument receives it (RNE)."""
    return ctypes.c_float(float(x)).value


def table_of(handle):
    t = _TABLES.get(int(handle))
    if t is None or t.handle_int == 0:
        raise RuntimeError(f'yoco_z1: no live table with handle {handle:#x}')
    return t


class Table:
    """Device-resident tensor-offset table over rows of fixed sizes.

    ``Table(rows, device)``: list form, rows = sequence of (g, p, m, v, p16, n) with tensors or None (p / m / v /
    p16), bound to those tensors.  ``Table.flat(offsets, numels, g, p, m, v, p16)``: flat form, bound to those
    buffers.  ``bound`` keeps the tensors of that first binding (the default a caller may pass again, as the
    reference's dest map keeps its views, yoco/tasks/fused_adam_cast.py:49-50); whichever tensors a launch names stay
    allocated and unmoved until it has run."""

    def __init__(self, rows, device, _flat=None):
        self.device = torch.device(device)
        if self.device.type == 'cuda' and self.device.index is None:
            self.device = torch.device('cuda', torch.cuda.current_device())
        gd = None
        for (g, p, m, v, p16, n) in rows:
            if g is None:
                raise RuntimeError('yoco_z1: a table row has no gradient')
            code = GDTYPE.get(g.dtype)
            if code is None or (gd is not None and code != gd):
                raise RuntimeError(f'yoco_z1: gradients must all be fp32 or all bf16, got {g.dtype}')
            gd = code
            for t in (g, p, m, v, p16):
                if t is not None:
                    require_gpu(t, 'yoco_z1')
                    if t.device != self.device:
                        raise RuntimeError('yoco_z1: table tensors on different devices')
        self.g_dtype = Z1_F32 if gd is None else gd
        self.nrows = len(rows)
        self.sizes = tuple(int(r[5]) for r in rows)
        self.has_pmv = bool(rows) and all(r[1] is not None and r[2] is not None and r[3] is not None for r in rows)
        self.flat_offsets = _flat                      # element offsets per row (flat form) or None
        arr = self._row_array(rows)
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            check(lib().z1_table_create(arr, self.nrows, self.g_dtype, ctypes.byref(h)), 'z1_table_create')
        self._h = h
        numel, nch, nr = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
        check(lib().z1_table_info(h, ctypes.byref(numel), ctypes.byref(nch), ctypes.byref(nr)), 'z1_table_info')
        self.numel, self.nchunks = numel.value, nch.value
        if nr.value != self.nrows:
            raise RuntimeError(f'yoco_z1: the table reports {nr.value} rows, {self.nrows} were given')
        self._ptrs = self._row_ptrs(rows)
        self.bound = None if _flat is not None else rows_lists(rows)
        _TABLES[self.handle_int] = self

    @classmethod
    def flat(cls, offsets, numels, g, p, m, v, p16):
        """Flat form: row i is elements [offsets[i], offsets[i] + numels[i]) of each buffer (p, m, v, p16 may be
        None; p16 None means no BF16 copy).  Bound to the given buffers."""
        rows = []
        for o, n in zip(offsets, numels):
            sl = slice(int(o), int(o) + int(n))
            rows.append((g[sl], None if p is None else p[sl], None if m is None else m[sl],
                         None if v is None else v[sl], None if p16 is None else p16[sl], int(n)))
        t = cls(rows, g.device, _flat=tuple(int(o) for o in offsets))
        t.bound = ([g], [] if p is None else [p], [] if m is None else [m], [] if v is None else [v],
                   [] if p16 is None else [p16])
        return t

    @property
    def handle(self):
        return self._h

    @property
    def handle_int(self):
        h = getattr(self, '_h', None)
        return 0 if h is None or not h.value else int(h.value)

    # -- binding -------------------------------------------------------------------------------------------------
    @staticmethod
    def _row_array(rows):
        """z1_tensor rows from (g, p, m, v, p16, n): tensors, addresses (int, 0 = none) or None."""
        arr = (Z1Tensor * max(1, len(rows)))()
        for i, r in enumerate(rows):
            addr = [t if isinstance(t, int) else (0 if t is None else t.data_ptr()) for t in r[:5]]
            arr[i] = Z1Tensor(*[a or None for a in addr], int(r[5]))
        return arr

    @staticmethod
    def _row_ptrs(rows):
        return tuple(tuple(0 if t is None else (t if isinstance(t, int) else t.data_ptr()) for t in r[:5])
                     for r in rows)

    def _check(self, t, dtype, what):
        require_gpu(t, what)
        if t.device != self.device:
            raise RuntimeError(f'{what}: a tensor is on another device than its table')
        if t.dtype != dtype or not t.is_contiguous():
            raise RuntimeError(f'{what}: expected contiguous {dtype} tensors')

    def _column(self, lst, k, what):
        """Per-row addresses of stream k (0 g, 1 p, 2 m, 3 v, 4 p16) for the tensors of a call."""
        dtype = ((torch.float32 if self.g_dtype == Z1_F32 else torch.bfloat16), torch.float32, torch.float32,
                 torch.float32, torch.bfloat16)[k]
        if not lst:
            if k != 4:
                raise RuntimeError(f'{what}: a gradient, master or moment list is empty')
            return (0,) * self.nrows                      # no BF16 copies
        if self.flat_offsets is not None:
            if len(lst) != 1:
                raise RuntimeError(f'{what}: a flat table takes one buffer per stream')
            t = lst[0]
            self._check(t, dtype, what)
            need = max((o + n for o, n in zip(self.flat_offsets, self.sizes)), default=0)
            if t.numel() < need:
                raise RuntimeError(f'{what}: a flat buffer holds {t.numel()} elements, the table needs {need}')
            base, es = t.data_ptr(), t.element_size()
            return tuple(base + o * es for o in self.flat_offsets)
        if len(lst) != self.nrows:
            raise RuntimeError(f'{what}: expected one tensor per table row ({self.nrows}), got {len(lst)}')
        col = []
        for i, (t, n) in enumerate(zip(lst, self.sizes)):
            if k == 4 and t.numel() == 0:
                col.append(0)                               # no BF16 copy for this row
                continue
            self._check(t, dtype, what)
            if t.numel() != n:
                raise RuntimeError(f'{what}: row {i} has {t.numel()} elements, the table {n}')
            col.append(t.data_ptr())
        return tuple(col)

    def bind(self, g, p=None, m=None, v=None, p16=None, what='yoco_z1', remember=False):
        """Point the rows at the call's tensors (lists in the table's form; None keeps a stream as bound; an empty
        p16 list means no BF16 copies).  Enqueues a launch on the current stream only when an address changes.
        With remember, they also become ``bound``, the default of later calls (an operator's own binding does not:
        it may be to copies that functionalization made for one call)."""
        if not self.nrows:
            return
        cols = [list(c) for c in zip(*self._ptrs)]
        given = (g, p, m, v, p16)
        for k, lst in enumerate(given):
            if lst is not None:
                cols[k] = list(self._column(list(lst), k, what))
        if self.has_pmv and not all(cols[k][i] for k in (1, 2, 3) for i, n in enumerate(self.sizes) if n):
            raise RuntimeError(f'{what}: the table updates masters and moments; every row needs p, m and v')
        want = tuple(zip(*cols))
        if want != self._ptrs:
            self._rebind(want)
        if remember and self.bound is not None:
            self.bound = tuple(list(lst) if lst is not None else old for lst, old in zip(given, self.bound))

    def _rebind(self, want):
        with torch.cuda.device(self.device):
            if all(a[1:] == b[1:] for a, b in zip(want, self._ptrs)):
                arr = (ctypes.c_void_p * self.nrows)(*[r[0] or None for r in want])
                check(lib().z1_table_set_grads(self._h, ctypes.cast(arr, ctypes.c_void_p), self.nrows,
                                               stream_handle(self.device)), 'z1_table_set_grads')
            else:
                arr = self._row_array([(*r, n) for r, n in zip(want, self.sizes)])
                check(lib().z1_table_rebind(self._h, arr, self.nrows, stream_handle(self.device)),
                      'z1_table_rebind')
        self._ptrs = want

    def set_grads(self, grads):
        """Point the rows' gradients at new tensors (one per row, or the flat buffer), also for later calls that
        name no tensors."""
        self.bind(grads, what='set_grads', remember=True)

    def close(self):
        h, self._h = getattr(self, '_h', None), None
        if h is not None and h.value:
            try:
                _TABLES.pop(int(h.value), None)
                with torch.cuda.device(self.device):
                    lib().z1_table_destroy(h)
            except Exception:           # interpreter shutdown (module state gone): the process frees device memory
                pass

    def __del__(self):
        self.close()


class TableCache:
    """List-form tables keyed by what fixes a schedule -- the device, the gradient dtype, the row sizes and which
    rows carry p / m / v and a BF16 copy -- not by addresses (bounded, least recently used evicted).  The operators
    bind a table to each call's tensors (``Table.bind``: a launch only when addresses moved), so steps whose
    gradients autograd reallocates neither allocate nor synchronise; the cache's tables keep no default tensors,
    so callers pass them (``ops.adam_cast(..., tensors=ops.rows_lists(rows))``, ``ops.grad_sumsq(..., g=grads)``).
    ``builds`` counts the tables made."""

    def __init__(self, capacity=8):
        self.capacity = capacity
        self._d = OrderedDict()
        self.builds = 0

    def get(self, rows, device):
        key = (str(device),) + tuple((g.dtype, p is not None, m is not None, v is not None,
                                      p16 is not None and p16.numel() > 0, int(n)) for g, p, m, v, p16, n in rows)
        t = self._d.get(key)
        if t is None:
            t = Table(rows, device)
            t.bound = None              # no default tensors: every call names its own (and holds no references
            self.builds += 1            # to a step's gradients, so their memory is free for the next step's)
            self._d[key] = t
            while len(self._d) > self.capacity:
                self._d.popitem(last=False)[1].close()
        else:
            self._d.move_to_end(key)
        return t

    def clear(self):
        for t in self._d.values():
            t.close()
        self._d.clear()


def rows_lists(rows):
    """(g, p, m, v, p16) lists of list-form rows (g, p, m, v, p16, n): p, m, v as lists when every row has them
    (else empty), a missing BF16 copy as an empty tensor (an empty list when no row has one)."""
    g = [r[0] for r in rows]
    pmv = [[r[k] for r in rows] if rows and all(r[k] is not None for r in rows) else [] for k in (1, 2, 3)]
    p16 = [] if all(r[4] is None for r in rows) else \
        [r[4] if r[4] is not None else r[0].new_empty(0, dtype=torch.bfloat16) for r in rows]
    return g, pmv[0], pmv[1], pmv[2], p16


# -------------------------------------------------------------------------------------------- scalar outputs
def scalar_ptr(t, what):
    if t is None:
        return None
    require_gpu(t, what)
    if t.dtype != torch.float32 or t.numel() != 1:
        raise RuntimeError(f'{what}: expected a 1-element fp32 device tensor')
    return ptr(t)


def check_partials(partials, what, need=Z1_NORM_PARTIALS):
    require_gpu(partials, what)
    if partials.dtype != torch.float64 or partials.numel() < need or not partials.is_contiguous():
        raise RuntimeError(f'yoco_z1: the norm workspace must hold {need} float64')


def scalars_struct(what, factor, factor_value, norm, grad_norm, flags=None, clip_log=None, sample_size=None,
                   numer=1.0, max_norm=0.0):
    """z1_update_scalars: the factor is read from `factor` (in place) unless factor_value is given (then `factor`,
    if given, only receives the clipped value)."""
    if flags is not None:
        require_gpu(flags, what)
        if flags.dtype not in (torch.uint8, torch.bool) or flags.numel() < 2:
            raise RuntimeError(f'{what}: flags must hold 2 uint8/bool')
    fin = scalar_ptr(factor, what) if factor_value is None else None
    fval = 1.0 if factor_value is None else f32(factor_value)
    return Z1UpdateScalars(scalar_ptr(sample_size, what), f32(numer), fin, fval, f32(max_norm),
                           scalar_ptr(norm, what), scalar_ptr(grad_norm, what), scalar_ptr(factor, what),
                           ptr(flags), scalar_ptr(clip_log, what))


# ---------------------------------------------------------------------------------------------------- launches
def grad_sumsq(table, g, partials):
    check_partials(partials, 'grad_sumsq')
    table.bind(g, what='grad_sumsq')
    with torch.cuda.device(table.device):
        check(lib().z1_grad_sumsq(table.handle, ptr(partials), stream_handle(table.device)), 'z1_grad_sumsq')


def norm_clip(partials, factor, factor_value, norm, grad_norm, max_norm):
    check_partials(partials, 'norm_clip')
    dev = partials.device
    u = scalars_struct('norm_clip', factor, factor_value, norm, grad_norm, max_norm=max_norm)
    with torch.cuda.device(dev):
        check(lib().z1_update_scalars_run(ptr(partials), ctypes.byref(u), stream_handle(dev)), 'z1_norm_clip')


def grad_norm_clip(table, g, partials, factor, factor_value, norm, grad_norm, max_norm):
    check_partials(partials, 'grad_norm_clip')
    table.bind(g, what='grad_norm_clip')
    u = scalars_struct('grad_norm_clip', factor, factor_value, norm, grad_norm, max_norm=max_norm)
    with torch.cuda.device(table.device):
        check(lib().z1_grad_update_scalars(table.handle, ptr(partials), ctypes.byref(u), stream_handle(table.device)),
              'z1_grad_norm_clip')


def update_scalars(partials, factor, factor_value, norm, grad_norm, flags, clip_log, sample_size, numer, max_norm):
    check_partials(partials, 'update_scalars')
    dev = partials.device
    u = scalars_struct('update_scalars', factor, factor_value, norm, grad_norm, flags, clip_log, sample_size, numer,
                       max_norm)
    with torch.cuda.device(dev):
        check(lib().z1_update_scalars_run(ptr(partials), ctypes.byref(u), stream_handle(dev)), 'z1_update_scalars')


def grad_update_scalars(table, g, partials, factor, factor_value, norm, grad_norm, flags, clip_log, sample_size,
                        numer, max_norm):
    check_partials(partials, 'grad_update_scalars')
    table.bind(g, what='grad_update_scalars')
    u = scalars_struct('grad_update_scalars', factor, factor_value, norm, grad_norm, flags, clip_log, sample_size,
                       numer, max_norm)
    with torch.cuda.device(table.device):
        check(lib().z1_grad_update_scalars(table.handle, ptr(partials), ctypes.byref(u), stream_handle(table.device)),
              'z1_grad_update_scalars')


def clip_factor(norm, factor, factor_value, grad_norm, max_norm):
    dev = norm.device
    fin = scalar_ptr(factor, 'clip_factor') if factor_value is None else None
    fval = 1.0 if factor_value is None else f32(factor_value)
    with torch.cuda.device(dev):
        check(lib().z1_clip_factor(scalar_ptr(norm, 'clip_factor'), fin, fval, scalar_ptr(grad_norm, 'clip_factor'),
                                   scalar_ptr(factor, 'clip_factor'), f32(max_norm), stream_handle(dev)),
              'z1_clip_factor')


def bias_corrections(beta1, beta2, step, bias_correction=1):
    """yoco/tasks/fused_adam_cast.py:58-60: 1 - beta**step in double, rounded once to fp32."""
    if bias_correction == 1:
        return f32(1.0 - math.pow(beta1, step)), f32(1.0 - math.pow(beta2, step))
    return 1.0, 1.0


def adam_cast(table, g, p, m, v, p16, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, mode, row_begin, row_end):
    if not table.has_pmv:
        raise RuntimeError('yoco_z1: adam_cast needs a table with p, m and v')
    if not 0 <= int(row_begin) <= int(row_end) <= table.nrows:
        raise RuntimeError(f'yoco_z1: rows [{row_begin}, {row_end}) outside the table\'s {table.nrows} rows')
    table.bind(g, p, m, v, p16, what='adam_cast')
    args = (scalar_ptr(factor, 'adam_cast'), f32(lr), f32(beta1), f32(beta2), f32(eps), f32(bc1), f32(bc2),
            f32(weight_decay), int(mode), stream_handle(table.device))
    with torch.cuda.device(table.device):
        if int(row_begin) == 0 and int(row_end) == table.nrows:
            check(lib().z1_adam_cast(table.handle, *args), 'z1_adam_cast')
        else:
            check(lib().z1_adam_cast_rows(table.handle, int(row_begin), int(row_end), *args), 'z1_adam_cast_rows')


def adam_cast_dev(table, g, p, m, v, p16, factor, lr, beta1, beta2, eps, bc, weight_decay, mode):
    if not table.has_pmv:
        raise RuntimeError('yoco_z1: adam_cast_dev needs a table with p, m and v')
    require_gpu(bc, 'adam_cast_dev')
    if bc.dtype != torch.float32 or bc.numel() < 2 or not bc.is_contiguous():
        raise RuntimeError('yoco_z1: bias corrections must be a contiguous 2-element fp32 tensor')
    table.bind(g, p, m, v, p16, what='adam_cast_dev')
    with torch.cuda.device(table.device):
        check(lib().z1_adam_cast_dev(table.handle, scalar_ptr(factor, 'adam_cast_dev'), f32(lr), f32(beta1),
                                     f32(beta2), f32(eps), ptr(bc), f32(weight_decay), int(mode),
                                     stream_handle(table.device)), 'z1_adam_cast_dev')


def bias_corrections_step(step, bc, beta1, beta2, bias_correction):
    for t in (step, bc):
        require_gpu(t, 'bias_corrections_step')
    if (step.dtype != torch.int64 or step.numel() < 1 or bc.dtype != torch.float32 or bc.numel() < 2
            or not bc.is_contiguous() or step.device != bc.device):
        raise RuntimeError('yoco_z1: bias_corrections_step takes an int64 step and a contiguous 2-element fp32 bc '
                           'on one device')
    with torch.cuda.device(step.device):
        check(lib().z1_bias_corrections_step(ptr(step), float(beta1), float(beta2), int(bias_correction), ptr(bc),
                                             stream_handle(step.device)), 'z1_bias_corrections_step')


def owner_sum_args(contribs, out, out_sum, workspace):
    """Checked (host pointer array, world) for an owner-sum call."""
    require_gpu(out, 'owner_sum')
    if out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise RuntimeError('yoco_z1: owner_sum output must be a contiguous bf16 tensor')
    world = len(contribs)
    if not 1 <= world <= Z1_MAX_WORLD:
        raise RuntimeError(f'yoco_z1: owner_sum takes 1..{Z1_MAX_WORLD} contributions, got {world}')
    for c in contribs:
        require_gpu(c, 'owner_sum')
        if c.dtype != torch.bfloat16 or not c.is_contiguous() or c.numel() != out.numel() or c.device != out.device:
            raise RuntimeError('yoco_z1: owner_sum contributions must be contiguous bf16 tensors like out')
    if out_sum is not None:
        require_gpu(out_sum, 'owner_sum')
        if out_sum.dtype != torch.float32 or not out_sum.is_contiguous() or out_sum.numel() != out.numel():
            raise RuntimeError('yoco_z1: owner_sum out_sum must be a contiguous fp32 tensor like out')
    if workspace is not None:
        check_partials(workspace, 'owner_sum', int(lib().z1_owner_sum_workspace(out.numel())))
    return (ctypes.c_void_p * world)(*[c.data_ptr() for c in contribs]), world


def owner_sum(contribs, out, scale, out_sum, partials):
    arr, world = owner_sum_args(contribs, out, out_sum, partials)
    with torch.cuda.device(out.device):
        check(lib().z1_owner_sum_bf16(ctypes.cast(arr, ctypes.c_void_p), world, out.numel(), f32(scale), ptr(out),
                                      ptr(out_sum), ptr(partials), stream_handle(out.device)), 'z1_owner_sum_bf16')


def owner_sum_update(contribs, out, scale, workspace, out_sum, factor, factor_value, norm, grad_norm, flags, clip_log,
                     sample_size, numer, max_norm):
    if workspace is None:
        raise RuntimeError('yoco_z1: owner_sum_update needs its workspace')
    arr, world = owner_sum_args(contribs, out, out_sum, workspace)
    u = scalars_struct('owner_sum_update', factor, factor_value, norm, grad_norm, flags, clip_log, sample_size, numer,
                       max_norm)
    with torch.cuda.device(out.device):
        check(lib().z1_owner_sum_update(ctypes.cast(arr, ctypes.c_void_p), world, out.numel(), f32(scale), ptr(out),
                                        ptr(out_sum), ptr(workspace), ctypes.byref(u), stream_handle(out.device)),
              'z1_owner_sum_update')


def sum_slots(S, OUT, G, BASE, END, R, scale, WORLD):
    """The owner sum in the reference's staging layout (yoco/models/decoder/ce_reduce.py:59-74): contributions of
    peer k < R in slot k of S, k > R in slot k - 1, rank R's own in OUT, summed in rank order into OUT[BASE:END]."""
    for t, name in ((S, 'staging'), (OUT, 'out')):
        if not (torch.is_tensor(t) and t.is_cuda and t.dtype == torch.bfloat16 and t.is_contiguous()):
            raise RuntimeError(f'ce_reduce: {name} must be a contiguous bf16 GPU tensor')
    if not 1 <= WORLD <= Z1_MAX_WORLD or not 0 <= R < WORLD:
        raise RuntimeError(f'ce_reduce: rank {R} / world {WORLD} out of range')
    if not 0 <= BASE <= END <= G or OUT.numel() < G or S.numel() < (WORLD - 1) * G:
        raise RuntimeError(f'ce_reduce: range [{BASE}, {END}) does not fit G={G}, out {OUT.numel()}, '
                           f'staging {S.numel()}')
    if END == BASE:
        return
    es = OUT.element_size()
    s0, o0 = S.data_ptr(), OUT.data_ptr()
    addrs = [s0 + (k * G + BASE) * es if k < R else (o0 + BASE * es if k == R else s0 + ((k - 1) * G + BASE) * es)
             for k in range(WORLD)]
    arr = (ctypes.c_void_p * WORLD)(*addrs)
    with torch.cuda.device(OUT.device):
        check(lib().z1_owner_sum_bf16(ctypes.cast(arr, ctypes.c_void_p), WORLD, END - BASE, f32(scale),
                                      ctypes.c_void_p(o0 + BASE * es), None, None, stream_handle(OUT.device)),
              'z1_owner_sum_bf16')


def scale_up(g16, g32, factor):
    for t in (g16, g32, factor):
        require_gpu(t, 'scale_up')
    if g16.dtype != torch.bfloat16 or g32.dtype != torch.float32 or g16.numel() != g32.numel():
        raise RuntimeError('yoco_z1: scale_up expects bf16 -> fp32 of equal size')
    if not (g16.is_contiguous() and g32.is_contiguous()):
        raise RuntimeError('yoco_z1: scale_up expects contiguous tensors')
    with torch.cuda.device(g32.device):
        check(lib().z1_scale_up(ptr(g16), ptr(g32), scalar_ptr(factor.reshape(-1)[:1], 'scale_up'), g16.numel(),
                                stream_handle(g32.device)), 'z1_scale_up')


def cast_bf16(p32, p16):
    for t in (p32, p16):
        require_gpu(t, 'cast_bf16')
    if p32.dtype != torch.float32 or p16.dtype != torch.bfloat16 or p32.numel() != p16.numel():
        raise RuntimeError('yoco_z1: cast_bf16 expects fp32 -> bf16 of equal size')
    if not (p32.is_contiguous() and p16.is_contiguous()):
        raise RuntimeError('yoco_z1: cast_bf16 expects contiguous tensors')
    with torch.cuda.device(p32.device):
        check(lib().z1_cast_bf16(ptr(p32), ptr(p16), p32.numel(), stream_handle(p32.device)), 'z1_cast_bf16')


def embedding_workspace_bytes(rows, dim, num_weights):
    n = int(lib().z1_embedding_backward_workspace(int(rows), int(dim), int(num_weights)))
    if n < 0:
        check(n, 'z1_embedding_backward_workspace')
    return n


def embedding_backward(grad, indices, num_weights, padding_idx, scale, scale_mode, out, workspace):
    """out[V, D] (bf16) = aten.embedding_dense_backward(grad, indices, V, padding_idx, False) with the scale; grad
    [R, D] bf16 and indices [R] int64 contiguous, workspace uint8 of at least embedding_workspace_bytes."""
    R, D = grad.shape
    if (out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != num_weights * D
            or out.device != grad.device):
        raise RuntimeError('embedding_dense_backward: out must be a contiguous bf16 [num_weights, D] tensor')
    need = embedding_workspace_bytes(R, D, num_weights)
    if workspace.dtype != torch.uint8 or workspace.numel() < need or workspace.device != grad.device:
        raise RuntimeError(f'embedding_dense_backward: the workspace must hold {need} bytes on the device')
    with torch.cuda.device(grad.device):
        check(lib().z1_embedding_backward(ptr(indices), ptr(grad), R, D, int(num_weights), int(padding_idx),
                                          f32(scale), int(scale_mode), ptr(out), ptr(workspace), workspace.numel(),
                                          stream_handle(grad.device)), 'z1_embedding_backward')
