"""Drop-in for yoco/tasks/zero1_fast.py: fairseq's FP16Optimizer under ZeRO-1 (fairscale OSS) with the owned shard's
norm, clip, gradient scale and Adam + BF16 copy on this build's gfx950 operators (``ops`` / ``torch.ops.yoco_z1``).

Switches, read at import like the reference's (yoco/tasks/zero1_fast.py:23-44; off unless set to 1):
    YOCO_ZERO1_FAST, YOCO_ZERO1_ALLGATHER, YOCO_ZERO1_PARAM_VIEWS, YOCO_PARAM_ALLREDUCE + YOCO_GRAD_REDUCE_OWNER,
    YOCO_Z1_ONE_PASS, YOCO_Z1_SCALE_KERNEL, YOCO_FUSED_ADAM, YOCO_CE_ALLGATHER (refused: not part of this build)
plus one of this build, YOCO_Z1_FOLD_SCALE (off by default).  With the fused Adam, the Adam kernel reads each owned
BF16 gradient times the factor itself instead of the FP32 master gradient a scale pass writes first -- the same
products g32 = fp32(g16 * factor).  By default it also writes them into the masters' ``.grad`` tensors, as the
reference's scale pass does (one pass of 32 bytes per element instead of 6 + 30, one launch instead of one per
tensor plus one); with YOCO_Z1_FOLD_SCALE=1 it does not (28 bytes per element), and the masters' ``.grad`` tensors
are left as they were.  Without the fused Adam the scale pass runs as in the reference.

Imported with YOCO_ZERO1_FAST=1 where fairseq is importable, the module installs itself on fairseq's
``_FP16OptimizerMixin`` (``clip_grad_norm`` / ``step`` / ``zero_grad``), adds the parameter placement to the
reference's pre-DDP hooks when YOCO_ZERO1_PARAM_VIEWS=1 and the reference's layer_graphs is importable, and, with
YOCO_CE_REDUCE=1, replaces the reference's ``CEReduce._sum`` -- what yoco/tasks/zero1_fast.py:247-255 does on import.
``install(mixin)`` does the first part on any class shaped like the mixin.

The norm is this build's deterministic FP64-accumulated norm of the gradients (the reference calls fairseq's
clip_grad_norm_, i.e. apex multi_tensor_l2norm, whose summation order differs; both are within 1e-6 of the exact
value).
"""
import os

import torch
import torch.distributed as dist

from . import ce_reduce, layout, ops
from .fused_adam_cast import FusedAdamCast, scale_up


def _switch(name, default='0'):
    return os.environ.get(name, default) == '1'


ENABLED = _switch('YOCO_ZERO1_FAST')
ALLGATHER = _switch('YOCO_ZERO1_ALLGATHER')
PARAM_VIEWS = ALLGATHER and _switch('YOCO_ZERO1_PARAM_VIEWS')
REDUCE_OWNER = PARAM_VIEWS and _switch('YOCO_PARAM_ALLREDUCE') and _switch('YOCO_GRAD_REDUCE_OWNER')
ONE_PASS = _switch('YOCO_Z1_ONE_PASS')
CE_ALLGATHER = PARAM_VIEWS and _switch('YOCO_CE_ALLGATHER')
FUSED_ADAM = _switch('YOCO_FUSED_ADAM')
SCALE_KERNEL = ONE_PASS and _switch('YOCO_Z1_SCALE_KERNEL')
FOLD_SCALE = _switch('YOCO_Z1_FOLD_SCALE')
_SWITCHES = ('ENABLED', 'ALLGATHER', 'PARAM_VIEWS', 'REDUCE_OWNER', 'ONE_PASS', 'CE_ALLGATHER', 'FUSED_ADAM',
             'SCALE_KERNEL', 'FOLD_SCALE')
_PLACED = {}          # the pre-DDP placement: {'flat': bf16 [world * seg], 'seg': int, 'owner': {id(p): rank}}
_ORIG = {}            # the mixin's own methods, for optimizers this path does not cover


def configure(**switches):
    """Set switches programmatically (the module-level names, e.g. ENABLED=True, FUSED_ADAM=True)."""
    for k, v in switches.items():
        if k not in _SWITCHES:
            raise KeyError(k)
        globals()[k] = bool(v)


def _place_params(module):
    """Pre-DDP hook (zero1_fast.py:52-75): OSS's greedy partition over the trainable parameters, each made a view of
    its owner's segment of one flat BF16 buffer, so that the BF16 exchange writes the model directly."""
    if not dist.is_initialized():
        return
    params = [p for p in module.parameters() if p.requires_grad]
    if params and all(p.is_cuda for p in params):
        _PLACED.update(layout.place_params(params, dist.get_world_size()))


class _Plan:
    """One rank's share of the ZeRO-1 update, made on the optimizer's first clip / step / zero_grad
    (zero1_fast.py:85-136 builds the same from the OSS partition): the trainable (BF16, FP32) pairs, their owners,
    every pair's BF16 view in its owner's segment, this rank's pairs, and the fused Adam."""

    def __init__(self, opt, oss):
        p16s, p32s = list(opt.fp16_params), list(opt.fp32_params)
        if len(p16s) != len(p32s):
            raise RuntimeError('zero1_fast: fp16 and fp32 parameter lists differ in length')
        self.rank, self.world, self.group = oss.rank, oss.world_size, oss.group
        self.global_ranks = list(getattr(oss, '_local_to_global_rank', range(self.world)))
        pairs = [(a, b) for a, b in zip(p16s, p32s) if a.requires_grad]
        owners = [oss._param_to_rank[b] for _, b in pairs]
        local, totals, seg = layout.owner_slots([a.numel() for a, _ in pairs], owners, self.world)
        self.placed = bool(_PLACED) and all(_PLACED['owner'].get(id(a)) == r for (a, _), r in zip(pairs, owners))
        if PARAM_VIEWS and not self.placed:
            raise RuntimeError('zero1_fast: the placed parameter layout does not match the OSS partition')
        like = dict(dtype=p16s[0].dtype, device=p16s[0].device) if p16s else {}
        if self.placed:
            self.flat, self.seg = _PLACED['flat'], _PLACED['seg']
        else:
            self.seg = seg
            self.flat = torch.empty(self.world * seg, **like) if ALLGATHER and pairs else None
        if self.flat is not None:
            self.segments = [self.flat[r * self.seg:r * self.seg + totals[r]] for r in range(self.world)]
        else:
            self.segments = [torch.empty(totals[r], **like) for r in range(self.world)]
        self.views = []                               # (p16, p32, its BF16 view in the owner's segment), all pairs
        for (a, b), r, o in zip(pairs, owners, local):
            view = self.segments[r][o:o + a.numel()].view_as(a)
            if self.placed and view.data_ptr() != a.data_ptr():
                raise RuntimeError('zero1_fast: a placed parameter is not at its slot')
            self.views.append((a, b, view))
        self.mine = [t for t, r in zip(self.views, owners) if r == self.rank]
        oss._broadcast_params = lambda: None          # the FP32 broadcast gives way to the BF16 exchange
        self.fused = None
        if FUSED_ADAM and hasattr(oss.optim, 'multi_tensor_adam'):
            self.fused = FusedAdamCast({b.data_ptr(): view for _, b, view in self.mine if view.is_contiguous()})
            oss.optim.multi_tensor_adam = self.fused
        elif hasattr(oss.optim, 'multi_tensor_adam'):
            # without YOCO_FUSED_ADAM the reference leaves FusedAdamV2 on apex's amp_C.multi_tensor_adam
            # (zero1_fast.py:125-129 replace it only with the switch): here the same call, amp_C's signature, runs
            # this build's Adam without BF16 destinations, and the step's casts write every BF16 copy as there
            oss.optim.multi_tensor_adam = FusedAdamCast({})
        if CE_ALLGATHER and self.placed:
            raise RuntimeError('zero1_fast: YOCO_CE_ALLGATHER (CUDA IPC copy-engine exchange) is not part of this build')
        self.partials = None
        self.norm_tables = ops.TableCache(4)
        self.scalars = None                           # device scalars of clip / step: n_r, the factor (see _scalar)

    def scalar(self, k, dev):
        """The plan's k-th 1-element fp32 device scalar (0: the owner's norm n_r, 1: the clipped factor when fairseq's
        factor is a Python number, 2: that number for the step), made once: a step allocates nothing but the
        grad_norm tensor clip_grad_norm returns (a new one each time, as the reference's is)."""
        if self.scalars is None or self.scalars.device != dev:
            self.scalars = torch.zeros(3, dtype=torch.float32, device=dev)
        return self.scalars[k:k + 1]

    def exchange(self):
        """Every owner's BF16 segment to every rank (zero1_fast.py:224-231): one all-gather over the flat buffer, or
        one broadcast per owner."""
        if self.flat is not None:
            mine = self.flat[self.rank * self.seg:(self.rank + 1) * self.seg]
            dist.all_gather_into_tensor(self.flat, mine, group=self.group)
            return
        pending = [dist.broadcast(buf, src=self.global_ranks[r], group=self.group, async_op=True)
                   for r, buf in enumerate(self.segments) if buf.numel()]
        for work in pending:
            work.wait()


def _plan(opt):
    """The optimizer's plan, or None where the reference falls back to fairseq (no OSS shard, flat FP32 params or
    a loss scaler: zero1_fast.py:90-92)."""
    if not ENABLED:
        return None
    plan = opt.__dict__.get('_z1')
    if plan is None:
        inner = getattr(opt.fp32_optimizer, 'optimizer', None)
        covered = (hasattr(inner, 'partition_parameters') and hasattr(inner, 'optim') and not opt.has_flat_params
                   and opt.scaler is None)
        plan = _Plan(opt, inner) if covered else False
        opt._z1 = plan
    return plan or None


def _device_factor(factor, dev, buf=None):
    """fairseq's _multiply_factor as a 1-element fp32 tensor on `dev`: the same tensor when it is one; a Python number
    is filled into `buf` (a fill kernel, no host copy) or a new tensor."""
    if torch.is_tensor(factor):
        if factor.dtype == torch.float32 and factor.device == dev and factor.numel() == 1:
            return factor
        return factor.to(device=dev, dtype=torch.float32).reshape(1)
    if buf is not None:
        return buf.fill_(float(factor))
    return torch.full((1,), float(factor), dtype=torch.float32, device=dev)


def clip_grad_norm(self, max_norm, aggregate_norm_fn=None):
    """zero1_fast.py:139-162: the norm of the gradients (only the owned ones when the reduction goes to owners:
    then the owners' squared norms are summed over the group), grad_norm = factor * norm, and with max_norm > 0
    factor *= min(max_norm / (grad_norm + 1e-6), 1).  Returns grad_norm as a 0-d fp32 device tensor; no host
    synchronisation."""
    plan = _plan(self)
    if plan is None:
        return _ORIG['clip'](self, max_norm, aggregate_norm_fn)
    src = [a for a, _, _ in plan.mine] if REDUCE_OWNER else [a for a in self.fp16_params if a.requires_grad]
    for a in src:
        if a.grad is None:
            a.grad = torch.zeros_like(a)
    grads = [a.grad for a in src]
    if any(not (g.is_cuda and g.is_contiguous() and g.dtype in (torch.float32, torch.bfloat16)) for g in grads):
        raise RuntimeError('zero1_fast: gradients must be contiguous fp32/bf16 GPU tensors')
    if len({g.dtype for g in grads}) > 1:
        grads = [g.float() for g in grads]          # one dtype per table; the fp32 upcast of bf16 is exact
    dev = grads[0].device if grads else (self.fp16_params[0].device if self.fp16_params else torch.device('cuda'))
    if plan.partials is None:
        plan.partials = ops.norm_workspace(dev)
    factor = self._multiply_factor
    if torch.is_tensor(factor):
        factor = _device_factor(factor, dev)
    out = factor if torch.is_tensor(factor) else plan.scalar(1, dev)
    grad_norm = torch.empty(1, dtype=torch.float32, device=dev)        # returned: a new tensor per call
    clip = float(max_norm) if max_norm > 0.0 else 0.0
    # the owned gradients are the average CEReduce's phase sums wrote: their norm partials are already there
    fused = ce_reduce.take_norm_partials(grads) if REDUCE_OWNER else None
    table = None
    if fused is None and grads:
        # rows in the order of the gradients' addresses: the pass reads the last 256 MB of its table with
        # allocating loads, which should be what the fused Adam reads first (it starts at the highest address)
        grads = sorted(grads, key=lambda g: g.data_ptr())
        table = plan.norm_tables.get([(g, None, None, None, None, g.numel()) for g in grads], dev)
    one_owner = REDUCE_OWNER and plan.world == 1 and aggregate_norm_fn is None and (grads or fused)
    if one_owner and fused is not None:
        # one owner: the all-reduce of n_r^2 is the identity, and the kernel's chain is the reference's
        # (sq = n_r^2, norm = sqrt(sq), grad_norm, clip)
        ops.reduce_waves(fused[0], fused[1], plan.partials)
        ops.norm_clip(plan.partials, factor=factor, grad_norm_out=grad_norm, factor_out=out, max_norm=clip)
    elif one_owner:
        ops.grad_norm_clip(table, plan.partials, factor=factor, grad_norm_out=grad_norm, factor_out=out,
                           max_norm=clip, g=grads)                  # norm and clip in one call
    else:
        if fused is not None:
            ops.reduce_waves(fused[0], fused[1], plan.partials)
        elif table is not None:
            ops.grad_sumsq(table, plan.partials, g=grads)
        else:
            plan.partials.zero_()
        n_r = plan.scalar(0, dev)
        ops.norm_clip(plan.partials, norm_out=n_r)              # the owner's (or every rank's) fp32 norm
        if REDUCE_OWNER:
            sq = n_r ** 2                                       # owners' squared norms summed over the group
            if plan.world > 1:
                dist.all_reduce(sq, group=plan.group)
            norm = sq.sqrt()
        else:
            norm = n_r                                          # fairseq's clip_grad_norm_ value itself
        if aggregate_norm_fn is not None:
            norm = aggregate_norm_fn(norm).reshape(1).to(torch.float32)
        ops.clip_factor(norm, factor=factor, grad_norm_out=grad_norm, factor_out=out, max_norm=clip)
    if max_norm > 0.0 or torch.is_tensor(factor):
        self._multiply_factor = out
    self._needs_sync = False
    return grad_norm.view(())


def _cast(p32, view):
    """BF16 copy of a master into its view: the kernel for contiguous tensors, torch's RNE copy otherwise."""
    if p32.is_contiguous() and view.is_contiguous() and p32.dtype == torch.float32 and view.dtype == torch.bfloat16:
        ops.cast_bf16(p32.reshape(-1), view.reshape(-1))
    else:
        view.copy_(p32)


@torch.no_grad()
def step(self, closure=None, groups=None):
    """zero1_fast.py:165-235: the owned masters' FP32 gradients = fp32(BF16 gradient * factor), factor := 1, the
    Adam step on this rank's shard (fairseq -> OSS -> FusedAdamV2, whose multi_tensor_adam is the fused Adam + BF16
    copy), BF16 copies of the owned masters the fused Adam did not write, then every owner's BF16 segment to every
    rank (world > 1) and into the model's parameters (when they are not views of the segments)."""
    plan = _plan(self)
    if plan is None:
        return _ORIG['step'](self, closure, groups)
    for a, b, _ in plan.mine:
        if a.grad is None:
            a.grad = torch.zeros_like(a)
        if b.grad is None:
            b.grad = torch.zeros_like(b)
    if plan.mine:
        dev = plan.mine[0][1].device
        f1 = _device_factor(self._multiply_factor, dev, plan.scalar(2, dev))
        folded = {}
        if plan.fused is not None:
            folded = {b.data_ptr(): a.grad for a, b, _ in plan.mine
                      if a.grad.dtype == torch.bfloat16 and a.grad.is_contiguous() and a.grad.numel() == b.numel()
                      and (FOLD_SCALE or b.grad.is_contiguous())}
        for a, b, _ in plan.mine:
            if b.data_ptr() in folded:
                continue
            if a.grad.dtype == torch.bfloat16 and a.grad.is_contiguous() and b.grad.is_contiguous():
                scale_up(a.grad, b.grad, f1)
            else:
                torch.mul(a.grad, f1, out=b.grad)
        if plan.fused is not None:
            plan.fused.fold, plan.fused.fold_factor, plan.fused.fold_writes = folded, f1, not FOLD_SCALE
    self._multiply_factor = 1.0
    self._needs_sync = False
    try:
        self.fp32_optimizer.step(closure, groups=groups)
    finally:
        if plan.fused is not None:
            plan.fused.fold, plan.fused.fold_factor, plan.fused.fold_writes = {}, None, False
    written = plan.fused.cast if plan.fused is not None else set()
    for _, b, view in plan.mine:
        if b.data_ptr() not in written:
            _cast(b.data, view)
    written.clear()
    if plan.world > 1:
        plan.exchange()
    if not plan.placed:
        for a, _, view in plan.views:
            if a.data_ptr() != view.data_ptr():
                a.data.copy_(view)


def zero_grad(self):
    """zero1_fast.py:238-244: the BF16 gradients are dropped (the FP32 master gradients are overwritten by the next
    step, so they are not cleared)."""
    if _plan(self) is None:
        return _ORIG['zero'](self)
    for a in self.fp16_params:
        a.grad = None
    self._needs_sync = False


def install(mixin):
    """Swap clip_grad_norm / step / zero_grad of fairseq's _FP16OptimizerMixin (or a class shaped like it) when
    ENABLED (zero1_fast.py:252-255).  Returns whether it did."""
    if not ENABLED:
        return False
    for key, name, fn in (('clip', 'clip_grad_norm', clip_grad_norm), ('step', 'step', step),
                          ('zero', 'zero_grad', zero_grad)):
        _ORIG.setdefault(key, getattr(mixin, name))
        setattr(mixin, name, fn)
    return True


def install_reference():
    """What importing yoco/tasks/zero1_fast.py does (:247-255), for whichever of fairseq and the reference's modules
    are importable: the mixin patch, the placement hook (PARAM_VIEWS), and this build's owner sum in CEReduce
    (YOCO_CE_REDUCE=1).  Returns the names of the seams installed."""
    import importlib
    done = []

    def find(name):
        try:
            return importlib.import_module(name)
        except ImportError:
            return None

    f16 = find('fairseq.optim.fp16_optimizer') if ENABLED else None
    if f16 is not None and install(f16._FP16OptimizerMixin):
        done.append('fp16_optimizer')
    lg = find('models.decoder.layer_graphs') if ENABLED and PARAM_VIEWS else None
    if lg is not None and _place_params not in lg.PRE_DDP_HOOKS:
        lg.PRE_DDP_HOOKS.append(_place_params)
        lg.install_ddp_patch()
        done.append('layer_graphs')
    ce = find('models.decoder.ce_reduce') if _switch('YOCO_CE_REDUCE') else None
    if ce is not None:
        ce_reduce.install(ce.CEReduce)
        done.append('ce_reduce')
    return done


def install_fairseq():
    """install() on fairseq's mixin (and the placement hook), raising ImportError where fairseq is missing."""
    import fairseq.optim.fp16_optimizer  # noqa: F401
    return bool(install_reference())


INSTALLED = install_reference() if ENABLED else []
