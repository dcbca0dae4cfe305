"""Drop-in for yoco/tasks/zero1_fast.py: the ZeRO-1 fast path of fairseq's FP16Optimizer with the shard's
norm, clip and Adam + BF16 cast on gfx950 kernels.

The same switches select it (read at import, off by default, yoco/tasks/zero1_fast.py:23-44):
    YOCO_ZERO1_FAST, YOCO_ZERO1_ALLGATHER, YOCO_ZERO1_PARAM_VIEWS, YOCO_PARAM_ALLREDUCE + YOCO_GRAD_REDUCE_OWNER,
    YOCO_Z1_ONE_PASS, YOCO_Z1_SCALE_KERNEL, YOCO_FUSED_ADAM, YOCO_CE_ALLGATHER
plus one of this build, YOCO_Z1_FOLD_SCALE (default 1): with the fused Adam installed, the Adam kernel reads each
owned BF16 gradient times the factor itself instead of a scale pass writing the FP32 gradient first (identical
products).  The FP32 masters' ``.grad`` tensors are then not written by the step; set YOCO_Z1_FOLD_SCALE=0 where
something reads them afterwards.

``install(mixin)`` swaps ``clip_grad_norm`` / ``step`` / ``zero_grad`` on fairseq's ``_FP16OptimizerMixin`` (or any
class with its attributes) exactly where the reference does (:252-255); ``install_fairseq()`` does it on the real
fairseq when importable.

The same surface as the reference: ``clip_grad_norm(self, max_norm, aggregate_norm_fn=None) -> Tensor`` (0-d fp32,
on device, no host sync), ``step(self, closure=None, groups=None)``, ``zero_grad(self)``.  The norm is this
build's deterministic FP64-accumulated norm of the owned gradients (the reference calls fairseq's
clip_grad_norm_, i.e. apex multi_tensor_l2norm, whose summation order differs).
"""
import os

import torch
import torch.distributed as dist

from . import layout, ops
from .fused_adam_cast import FusedAdamCast, scale_up


def _env(name, default='0'):
    return os.environ.get(name, default) == '1'


ENABLED = _env('YOCO_ZERO1_FAST')
ALLGATHER = _env('YOCO_ZERO1_ALLGATHER')
PARAM_VIEWS = ALLGATHER and _env('YOCO_ZERO1_PARAM_VIEWS')
REDUCE_OWNER = PARAM_VIEWS and _env('YOCO_PARAM_ALLREDUCE') and _env('YOCO_GRAD_REDUCE_OWNER')
ONE_PASS = _env('YOCO_Z1_ONE_PASS')
CE_ALLGATHER = PARAM_VIEWS and _env('YOCO_CE_ALLGATHER')
FUSED_ADAM = _env('YOCO_FUSED_ADAM')
SCALE_KERNEL = ONE_PASS and _env('YOCO_Z1_SCALE_KERNEL')
FOLD_SCALE = _env('YOCO_Z1_FOLD_SCALE', '1')
_PLACED = {}
_ORIG = {}


def configure(**switches):
    """Set switches programmatically (names as the module constants, e.g. ENABLED=True, FUSED_ADAM=True)."""
    g = globals()
    for k, v in switches.items():
        if k not in ('ENABLED', 'ALLGATHER', 'PARAM_VIEWS', 'REDUCE_OWNER', 'ONE_PASS', 'CE_ALLGATHER', 'FUSED_ADAM',
                     'SCALE_KERNEL', 'FOLD_SCALE'):
            raise KeyError(k)
        g[k] = bool(v)


def _place_params(module):
    """zero1_fast.py:52-75: OSS's greedy partition, every trainable parameter a view of its owner's segment."""
    if not dist.is_initialized():
        return
    params = [p for p in module.parameters() if p.requires_grad]
    if not params or any(not p.is_cuda for p in params):
        return
    _PLACED.update(layout.place_params(params, dist.get_world_size()))


def _oss(self):
    inner = getattr(self.fp32_optimizer, 'optimizer', None)
    if inner is None or not hasattr(inner, 'partition_parameters') or not hasattr(inner, 'optim'):
        return None
    return inner


def _setup(self):
    """zero1_fast.py:85-136: owned pairs, per-owner buckets of the flat BF16 buffer, the fused Adam."""
    st = getattr(self, '_z1', None)
    if st is not None:
        return st
    oss = _oss(self)
    if oss is None or self.has_flat_params or self.scaler is not None:
        self._z1 = False
        return False
    p32s = list(self.fp32_params)
    p16s = list(self.fp16_params)
    if len(p32s) != len(p16s):
        raise RuntimeError('zero1_fast: fp16 and fp32 parameter lists differ in length')
    owner = oss._param_to_rank
    rank, world, group = oss.rank, oss.world_size, oss.group
    pairs = [(p16, p32) for p16, p32 in zip(p16s, p32s) if p16.requires_grad]
    local = [(p16, p32) for p16, p32 in pairs if owner[p32] == rank]
    per = [[(p16, p32) for p16, p32 in pairs if owner[p32] == r] for r in range(world)]
    seg = max(sum(p16.numel() for p16, _ in mine) for mine in per)
    placed = bool(_PLACED) and all(_PLACED['owner'].get(id(p16)) == owner[p32] for p16, p32 in pairs)
    if PARAM_VIEWS and not placed:
        raise RuntimeError('zero1_fast: the placed parameter layout does not match the OSS partition')
    if placed:
        flat, seg = _PLACED['flat'], _PLACED['seg']
    else:
        flat = torch.empty(world * seg, dtype=p16s[0].dtype, device=p16s[0].device) if ALLGATHER else None
    buckets = []
    for r, mine in enumerate(per):
        n = sum(p16.numel() for p16, _ in mine)
        buf = flat[r * seg:r * seg + n] if ALLGATHER else torch.empty(n, dtype=p16s[0].dtype, device=p16s[0].device)
        views, off = [], 0
        for p16, p32 in mine:
            v = buf[off:off + p16.numel()].view_as(p16)
            if placed and v.data_ptr() != p16.data_ptr():
                raise RuntimeError('zero1_fast: a placed parameter is not at its slot')
            views.append((p16, p32, v))
            off += p16.numel()
        buckets.append((r, buf, views))
    oss._broadcast_params = lambda: None          # the fp32 broadcast is replaced by the bf16 exchange
    st = {'local': local, 'buckets': buckets, 'rank': rank, 'world': world, 'group': group,
          'global_ranks': getattr(oss, '_local_to_global_rank', list(range(world))), 'flat': flat, 'seg': seg,
          'placed': placed, 'partials': None, 'tables': ops.TableCache(4)}
    if FUSED_ADAM and hasattr(oss.optim, 'multi_tensor_adam'):
        mine = [b for b in buckets if b[0] == rank]
        dest = {p32.data_ptr(): v for _, _, views in mine for _, p32, v in views if v.is_contiguous()}
        st['fused_adam'] = oss.optim.multi_tensor_adam = FusedAdamCast(dest)
    if CE_ALLGATHER and placed:
        raise RuntimeError('zero1_fast: YOCO_CE_ALLGATHER (CUDA IPC copy-engine exchange) is not part of this build')
    self._z1 = st
    return st


def _norm_table(st, grads):
    dev = grads[0].device
    rows = [(g, None, None, None, None, g.numel()) for g in grads]
    return st['tables'].get(rows, dev), dev


def _factor_arg(self, dev):
    """fairseq's _multiply_factor as the kernels take it: a Python number, or a 1-element fp32 device tensor."""
    f = self._multiply_factor
    if torch.is_tensor(f) and not (f.dtype == torch.float32 and f.is_cuda and f.numel() == 1 and f.device == dev):
        f = f.to(device=dev, dtype=torch.float32).reshape(1)
    return f


def clip_grad_norm(self, max_norm, aggregate_norm_fn=None):
    """zero1_fast.py:139-162."""
    st = _setup(self) if ENABLED else False
    if not st:
        return _ORIG['clip'](self, max_norm, aggregate_norm_fn)
    params = [p for p in self.fp16_params if p.requires_grad]
    for p in ([p16 for p16, _ in st['local']] if REDUCE_OWNER else params):     # only owned grads are used then
        if p.grad is None:
            p.grad = torch.zeros_like(p)
    grads = [p16.grad for p16, _ in st['local']] if REDUCE_OWNER else [p.grad for p in params if p.grad is not None]
    for g in grads:
        if not (g.is_cuda and g.is_contiguous() and g.dtype in (torch.float32, torch.bfloat16)):
            raise RuntimeError('zero1_fast: gradients must be contiguous fp32/bf16 GPU tensors')
    if not grads:
        dev = params[0].device if params else torch.device('cuda')
        grads_dtype = None
    else:
        dev = grads[0].device
        grads_dtype = grads[0].dtype
    if grads and any(g.dtype != grads_dtype for g in grads):
        grads = [g.to(torch.float32) for g in grads]
    if st['partials'] is None:
        st['partials'] = ops.norm_workspace(dev)
    partials = st['partials']
    if grads:
        table, _ = _norm_table(st, grads)
        ops.grad_sumsq(table, partials)
    else:
        partials.zero_()
    factor = _factor_arg(self, dev)
    out = factor if torch.is_tensor(factor) else torch.empty(1, dtype=torch.float32, device=dev)
    grad_norm = torch.empty(1, dtype=torch.float32, device=dev)
    mn = float(max_norm) if max_norm > 0.0 else 0.0
    if REDUCE_OWNER:
        if st['world'] == 1 and aggregate_norm_fn is None:
            # one owner: the all-reduce of sq is the identity; the whole chain runs in one kernel
            ops.norm_clip(partials, factor=factor, grad_norm_out=grad_norm, factor_out=out, max_norm=mn)
        else:
            n_r = torch.empty(1, dtype=torch.float32, device=dev)
            ops.norm_clip(partials, norm_out=n_r)
            sq = n_r.float() ** 2
            if st['world'] > 1:
                dist.all_reduce(sq, group=st['group'])
            norm = sq.sqrt()
            if aggregate_norm_fn is not None:
                norm = aggregate_norm_fn(norm)
            ops.clip_factor(norm.reshape(1).to(torch.float32), factor=factor, grad_norm_out=grad_norm, factor_out=out,
                            max_norm=mn)
    else:
        # every rank holds every gradient: grad_norm = factor * clip_grad_norm_(params, 0, aggregate_norm_fn)
        n = torch.empty(1, dtype=torch.float32, device=dev)
        ops.norm_clip(partials, norm_out=n)
        if aggregate_norm_fn is not None:
            n = aggregate_norm_fn(n).reshape(1).to(torch.float32)
        ops.clip_factor(n, factor=factor, grad_norm_out=grad_norm, factor_out=out, max_norm=mn)
    if max_norm > 0.0 or torch.is_tensor(factor):
        self._multiply_factor = out
    self._needs_sync = False
    return grad_norm.view(())


@torch.no_grad()
def step(self, closure=None, groups=None):
    """zero1_fast.py:165-235 (the exchange after the step only when world > 1)."""
    st = _setup(self) if ENABLED else False
    if not st:
        return _ORIG['step'](self, closure, groups)
    factor = self._multiply_factor
    for p16, p32 in st['local']:
        if p16.grad is None:
            p16.grad = torch.zeros_like(p16)
    g32 = [p32.grad for _, p32 in st['local']]
    fused = st.get('fused_adam')
    dev = g32[0].device if g32 else None
    if g32:
        f1 = (factor.to(device=dev, dtype=torch.float32) if torch.is_tensor(factor)
              else torch.tensor(float(factor), dtype=torch.float32, device=dev)).reshape(1)
        if fused is not None and FOLD_SCALE:
            fold = {}
            for (p16, p32), g in zip(st['local'], g32):
                gg = p16.grad
                if gg.is_contiguous() and gg.dtype == torch.bfloat16 and g.numel() == gg.numel():
                    fold[p32.data_ptr()] = gg
                else:
                    g.copy_(gg)
                    g.mul_(f1)
            fused.fold, fused.fold_factor = fold, f1
        else:
            for (p16, _), g in zip(st['local'], g32):
                if p16.grad.is_contiguous() and g.is_contiguous() and p16.grad.dtype == torch.bfloat16:
                    scale_up(p16.grad, g, f1)
                else:
                    g.copy_(p16.grad)
                    g.mul_(f1)
    self._multiply_factor = 1.0
    self._needs_sync = False
    try:
        self.fp32_optimizer.step(closure, groups=groups)          # the Adam step on this rank's shard (OSS)
    finally:
        if fused is not None:
            fused.fold, fused.fold_factor = {}, None
    rank = st['rank']
    for r, buf, views in st['buckets']:
        if r == rank and fused is not None:
            rest = [(p16, p32, v) for p16, p32, v in views if p32.data_ptr() not in fused.cast]
            for _, p32, v in rest:
                _cast(p32.data, v)
            fused.cast.clear()
        elif r == rank:
            for _, p32, v in views:
                _cast(p32.data, v)
    if st['world'] > 1:
        flat, seg = st['flat'], st['seg']
        if flat is not None:
            dist.all_gather_into_tensor(flat, flat[rank * seg:(rank + 1) * seg], group=st['group'])
        else:
            handles = [dist.broadcast(buf, src=st['global_ranks'][r], group=st['group'], async_op=True)
                       for r, buf, views in st['buckets'] if buf.numel()]
            for h in handles:
                h.wait()
    if not st['placed']:
        for r, buf, views in st['buckets']:
            for p16, p32, v in views:
                if p16.data_ptr() != v.data_ptr():
                    p16.data.copy_(v)


def _cast(p32, v):
    """BF16 copy of a master into its view: the kernel when both are contiguous, torch's RNE copy otherwise."""
    if p32.is_contiguous() and v.is_contiguous() and v.dtype == torch.bfloat16 and p32.dtype == torch.float32:
        ops.cast_bf16(p32.reshape(-1), v.reshape(-1))
    else:
        v.copy_(p32)


def zero_grad(self):
    """zero1_fast.py:238-244."""
    st = _setup(self) if ENABLED else False
    if not st:
        return _ORIG['zero'](self)
    for p in self.fp16_params:
        p.grad = None
    self._needs_sync = False


def install(mixin):
    """Swap the three methods of fairseq's _FP16OptimizerMixin (or a class shaped like it) when ENABLED."""
    if not ENABLED:
        return False
    _ORIG.setdefault('clip', mixin.clip_grad_norm)
    _ORIG.setdefault('step', mixin.step)
    _ORIG.setdefault('zero', mixin.zero_grad)
    mixin.clip_grad_norm = clip_grad_norm
    mixin.step = step
    mixin.zero_grad = zero_grad
    return True


def install_fairseq():
    """install() on fairseq.optim.fp16_optimizer._FP16OptimizerMixin, plus the pre-DDP placement hook when
    PARAM_VIEWS (the reference's layer_graphs hook list), if fairseq and the reference are importable."""
    from fairseq.optim import fp16_optimizer as _f16
    if ENABLED and PARAM_VIEWS:
        from models.decoder import layer_graphs as _lg
        _lg.PRE_DDP_HOOKS.append(_place_params)
        _lg.install_ddp_patch()
    return install(_f16._FP16OptimizerMixin)
