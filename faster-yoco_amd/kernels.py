"""The tensor-offset tables the operators run over (``library.py``), and host helpers of the launches.

A table is a device-resident schedule over rows of given sizes, made once (``z1_table_create``: a host pass over
the rows, one upload) and registered with the operator layer, which binds it to the tensors each call passes: a
stream-ordered rebind, only when the addresses moved, so one table serves tensors that move -- gradients that
autograd reallocates each step, or the copies of the state that torch's functionalization may hand to an operator.
Two forms:

* flat: the rows are slices of flat buffers at fixed element offsets (``FlatShard``); a call passes the flat
  buffers, one per stream (g, p, m, v, p16);
* list: one tensor per row and stream; a BF16 destination may be an empty tensor (no copy for that row).
"""
import ctypes
import math
from collections import OrderedDict

import torch

from . import library
from ._lib import Z1_BF16, Z1_F32, Z1Tensor, check, lib, require_gpu

GDTYPE = {torch.float32: Z1_F32, torch.bfloat16: Z1_BF16}


def f32(x):
    """Round a Python number to fp32 as a Triton / ctypes fp32 scalar argument receives it (RNE)."""
    return ctypes.c_float(float(x)).value


class Table:
    """Device-resident tensor-offset table over rows of fixed sizes.

    ``Table(rows, device)``: list form, rows = sequence of (g, p, m, v, p16, n) with tensors or None (p / m / v /
    p16), bound to those tensors.  ``Table.flat(offsets, numels, g, p, m, v, p16)``: flat form, bound to those
    buffers.  ``bound`` holds the tensors a call uses when it names none (the first binding, or the gradients of
    ``set_grads``; the reference's dest map keeps its views alike, yoco/tasks/fused_adam_cast.py:49-50); whichever
    tensors a launch names stay allocated and unmoved until it has run."""

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
        offs = None if _flat is None else (ctypes.c_int64 * max(1, self.nrows))(*_flat)
        if library.OPS_LIB.z1t_table_register(h, self.device.index, self.g_dtype, int(self.has_pmv), self.nrows, arr,
                                              offs) != 0:
            lib().z1_table_destroy(h)
            self._h = None
            raise RuntimeError('yoco_z1: the operator layer refused the table')
        self.bound = None if _flat is not None else rows_lists(rows)

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

    @staticmethod
    def _row_array(rows):
        """z1_tensor rows from (g, p, m, v, p16, n): tensors, addresses (int, 0 = none) or None."""
        arr = (Z1Tensor * max(1, len(rows)))()
        for i, r in enumerate(rows):
            addr = [t if isinstance(t, int) else (0 if t is None else t.data_ptr()) for t in r[:5]]
            arr[i] = Z1Tensor(*[a or None for a in addr], int(r[5]))
        return arr

    def _check_grads(self, grads, what):
        """The checks the operators make of a gradient list (one buffer for a flat table, else one per row)."""
        dtype = torch.float32 if self.g_dtype == Z1_F32 else torch.bfloat16
        grads = list(grads)
        if self.flat_offsets is not None:
            need = max((o + n for o, n in zip(self.flat_offsets, self.sizes)), default=0)
            if len(grads) != 1 or grads[0].numel() < need:
                raise RuntimeError(f'{what}: a flat table takes one gradient buffer of at least {need} elements')
        elif len(grads) != self.nrows:
            raise RuntimeError(f'{what}: expected one tensor per table row ({self.nrows}), got {len(grads)}')
        for i, t in enumerate(grads):
            require_gpu(t, what)
            if t.device != self.device or t.dtype != dtype or not t.is_contiguous():
                raise RuntimeError(f'{what}: expected contiguous {dtype} tensors on the table\'s device')
            if self.flat_offsets is None and t.numel() != self.sizes[i]:
                raise RuntimeError(f'{what}: row {i} has {t.numel()} elements, the table {self.sizes[i]}')
        return grads

    def set_grads(self, grads):
        """Make `grads` (one per row, or the flat buffer) the gradients of later calls that name no tensors (the
        device table follows at the next such call)."""
        grads = self._check_grads(grads, 'set_grads')
        if self.bound is None:
            raise RuntimeError('set_grads: this table keeps no default tensors (its callers pass them)')
        self.bound = (grads,) + tuple(self.bound[1:])

    def close(self):
        h, self._h = getattr(self, '_h', None), None
        if h is not None and h.value:
            try:
                library.OPS_LIB.z1t_table_forget(h)
                with torch.cuda.device(self.device):
                    lib().z1_table_destroy(h)
            except Exception:           # interpreter shutdown (module state gone): the process frees device memory
                pass

    def __del__(self):
        self.close()


class TableCache:
    """List-form tables keyed by what fixes a schedule -- the device, the gradient dtype, the row sizes and which
    rows carry p / m / v and a BF16 copy -- not by addresses (bounded, least recently used evicted).  The operators
    bind a table to each call's tensors (a rebind launch only when addresses moved), so steps whose
    gradients autograd reallocates neither allocate nor synchronise; the cache's tables keep no default tensors,
    so callers pass them (``ops.adam_cast(..., tensors=ops.rows_lists(rows))``, ``ops.grad_sumsq(..., g=grads)``).
    An evicted table is only dropped from the cache: a caller that still holds it (``FusedAdamCast``'s plans do)
    keeps using it, and it is freed with its last reference (``Table.__del__``).  ``builds`` counts the tables
    made."""

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
                self._d.popitem(last=False)
        else:
            self._d.move_to_end(key)
        return t

    def clear(self):
        self._d.clear()


def rows_lists(rows):
    """(g, p, m, v, p16) lists of list-form rows (g, p, m, v, p16, n): p, m, v as lists when every row has them
    (else empty), a missing BF16 copy as an empty tensor (an empty list when no row has one)."""
    g = [r[0] for r in rows]
    pmv = [[r[k] for r in rows] if rows and all(r[k] is not None for r in rows) else [] for k in (1, 2, 3)]
    p16 = [] if all(r[4] is None for r in rows) else \
        [r[4] if r[4] is not None else r[0].new_empty(0, dtype=torch.bfloat16) for r in rows]
    return g, pmv[0], pmv[1], pmv[2], p16


def bias_corrections(beta1, beta2, step, bias_correction=1):
    """yoco/tasks/fused_adam_cast.py:58-60: 1 - beta**step in double, rounded once to fp32."""
    if bias_correction == 1:
        return f32(1.0 - math.pow(beta1, step)), f32(1.0 - math.pow(beta2, step))
    return 1.0, 1.0


def embedding_workspace_bytes(rows, dim, num_weights):
    n = int(lib().z1_embedding_backward_workspace(int(rows), int(dim), int(num_weights)))
    if n < 0:
        check(n, 'z1_embedding_backward_workspace')
    return n
