"""One GPU's ZeRO-1 shard as flat HBM buffers, with the FP16Optimizer-style surface the reference's trainer
drives (``multiply_grads`` / ``clip_grad_norm`` / ``step`` / ``zero_grad``; fairseq ``_FP16OptimizerMixin`` as
patched by yoco/tasks/zero1_fast.py:139-244, called from yoco/tasks/trainer_nosync.py:273-289).

HBM layout (one allocation per stream, every tensor's slice starting on a ``align``-element boundary):
    p    fp32 [N]   master weights            m    fp32 [N]   exp_avg
    v    fp32 [N]   exp_avg_sq                g    fp32 or bf16 [N]   owner gradient (the reduced average)
    p16  bf16 [N]   the parameter copy the model reads
plus a device-resident offset table (one row per tensor) built once.  One optimizer update is three launches: the
norm (fixed-order partials) -> its final reduction + the clip chain (one workgroup) -> Adam + BF16 over the table.
With owner-side contributions (``reduce_grads`` / ``reduce_clip``) the norm is fused into the owner sum.
"""
import math

import torch
from torch.autograd.profiler import record_function

from . import ops


def _numel(shape):
    return int(math.prod(shape)) if len(shape) else 1


class FlatShard:
    """Flat buffers + offset table for a list of tensor shapes (model order)."""

    def __init__(self, shapes, device, grad_dtype=torch.float32, bf16_copy=True, align=64):
        if grad_dtype not in (torch.float32, torch.bfloat16):
            raise RuntimeError('yoco_z1: gradients must be fp32 or bf16')
        if align < 1 or align & (align - 1):
            raise RuntimeError('yoco_z1: align must be a power of two')
        dev = torch.device(device)
        if dev.type == 'cuda' and dev.index is None:
            dev = torch.device('cuda', torch.cuda.current_device())
        self.device = dev
        self.shapes = [tuple(int(d) for d in s) for s in shapes]
        self.numels = [_numel(s) for s in self.shapes]
        self.offsets = []
        off = 0
        for n in self.numels:
            off = (off + align - 1) // align * align
            self.offsets.append(off)
            off += n
        self.total = off
        self.numel = sum(self.numels)
        dev = self.device
        self.p = torch.zeros(self.total, dtype=torch.float32, device=dev)
        self.m = torch.zeros(self.total, dtype=torch.float32, device=dev)
        self.v = torch.zeros(self.total, dtype=torch.float32, device=dev)
        self.g = torch.zeros(self.total, dtype=grad_dtype, device=dev)
        self.p16 = torch.zeros(self.total, dtype=torch.bfloat16, device=dev) if bf16_copy else None
        # flat form: the operators take the five buffers, the table their rows' offsets
        self.table = ops.Table.flat(self.offsets, self.numels, self.g, self.p, self.m, self.v, self.p16)

    def buffers(self):
        """The (g, p, m, v, p16) buffer lists the table's operators take."""
        return self.table.bound

    def row_elements(self, row_begin, row_end):
        """[first, last) positions in the flat buffers spanned by the tensors row_begin .. row_end - 1."""
        if not 0 <= row_begin <= row_end <= len(self.numels):
            raise RuntimeError(f'yoco_z1: rows [{row_begin}, {row_end}) outside the shard')
        if row_begin == row_end:
            return 0, 0
        return self.offsets[row_begin], self.offsets[row_end - 1] + self.numels[row_end - 1]

    def views(self, buf):
        """Per-tensor views of one flat buffer (``'p'``, ``'m'``, ``'v'``, ``'g'`` or ``'p16'``)."""
        b = getattr(self, buf)
        return [b[o:o + n].view(s) for o, n, s in zip(self.offsets, self.numels, self.shapes)]

    def packed(self, buf):
        """The tensors' elements of one buffer, concatenated without the alignment gaps (a copy)."""
        b = getattr(self, buf)
        if self.total == self.numel:
            return b
        return torch.cat([b[o:o + n] for o, n in zip(self.offsets, self.numels)])


class Zero1ShardOptimizer:
    """Mixed-precision Adam over a FlatShard with fairseq's FP16Optimizer surface.

    ``_multiply_factor`` is a Python float or a 1-element fp32 device tensor, as in fairseq; the clip writes it as
    a device tensor and ``step`` resets it to 1.0 (yoco/tasks/zero1_fast.py:158-160,193).  The step counter plays
    FusedAdamV2's ``group['step']``; bias corrections are rounded on the host (fused_adam_cast.py:58-60).
    """

    def __init__(self, shard, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, adam_w_mode=True,
                 bias_correction=True, device_step=False):
        self.shard = shard
        self.lr = float(lr)
        self.betas = (float(betas[0]), float(betas[1]))
        self.eps = float(eps)
        self.weight_decay = float(weight_decay)
        self.mode = 1 if adam_w_mode else 0
        self.bias_correction = 1 if bias_correction else 0
        self.step_count = 0
        self._multiply_factor = 1.0
        self._needs_sync = False
        dev = shard.device
        self._partials = ops.norm_workspace(dev, shard.total if shard.g.dtype == torch.bfloat16 else None)
        self._factor = torch.ones(1, dtype=torch.float32, device=dev)
        self._norm = torch.zeros(1, dtype=torch.float32, device=dev)
        self._partials_ready = False
        # device_step: the step counter and bias corrections live on the device and the step advances there, so
        # an update captured once in a HIP graph replays correctly at every step (step_count counts host calls)
        self.device_step = bool(device_step)
        self._step_dev = torch.zeros(1, dtype=torch.int64, device=dev) if device_step else None
        self._bc = torch.ones(2, dtype=torch.float32, device=dev) if device_step else None

    def _as_device_factor(self, t):
        """A tensor factor as the 1-element fp32 device tensor the kernels read (the same tensor when it is one)."""
        if t.dtype == torch.float32 and t.device == self.shard.device and t.numel() == 1:
            return t
        return t.to(device=self.shard.device, dtype=torch.float32).reshape(1)

    def _clip_factor_args(self):
        """(factor the clip chain reads, tensor it writes the clipped factor to): a tensor factor is updated in
        place, as ``self._multiply_factor *= clip_coef`` on a tensor; a Python factor becomes a device tensor, as in
        the reference (yoco/tasks/zero1_fast.py:158-160)."""
        factor = self._multiply_factor
        if torch.is_tensor(factor):
            factor = self._as_device_factor(factor)
            return factor, factor
        return factor, self._factor

    # -- fairseq surface -------------------------------------------------------------------------------------
    def multiply_grads(self, c):
        """fairseq: ``self._multiply_factor *= c`` (c a number or a device tensor)."""
        self._multiply_factor *= c

    def reduce_grads(self, contribs, scale=None):
        """Owner-side sum of the ranks' BF16 contributions (rank order) into the shard's BF16 gradient, with the
        norm's partials fused in (yoco/models/decoder/ce_reduce.py:59-74,178-183, + the norm of
        zero1_fast.py:150).  contribs: flat bf16 tensors laid out like the shard's gradient buffer."""
        if self.shard.g.dtype != torch.bfloat16:
            raise RuntimeError('yoco_z1: reduce_grads needs a bf16 gradient shard')
        world = len(contribs)
        with record_function('reduce-grads'):        # the reference's profiler region (trainer_nosync.py:268)
            ops.owner_sum(contribs, self.shard.g, 1.0 / world if scale is None else scale, partials=self._partials)
        # the fused partials cover the whole flat buffer; with alignment gaps the norm is taken over the table
        self._partials_ready = self.shard.total == self.shard.numel

    def reduce_clip(self, contribs, max_norm, scale=None, sample_size=None, numer=1.0, flags_out=None,
                    clip_log_out=None):
        """reduce_grads + (the trainer's sample-size factor +) clip_grad_norm(max_norm) as one fused pass: the
        owner sum with the norm fused in, then the scalar chain on its partials (the owner's part of
        yoco/tasks/trainer_nosync.py:268-286).  Returns grad_norm (0-d device tensor), no host sync."""
        if self.shard.g.dtype != torch.bfloat16:
            raise RuntimeError('yoco_z1: reduce_clip needs a bf16 gradient shard')
        world = len(contribs)
        sc = 1.0 / world if scale is None else scale
        factor, out = self._clip_factor_args()
        grad_norm = torch.empty(1, dtype=torch.float32, device=self.shard.device)
        mn = float(max_norm)
        kw = dict(sample_size=sample_size, numer=numer, factor=factor, max_norm=mn if mn > 0.0 else 0.0,
                  norm_out=self._norm, grad_norm_out=grad_norm, factor_out=out, flags_out=flags_out,
                  clip_log_out=clip_log_out)
        with record_function('reduce-grads'):        # the reference's profiler region (trainer_nosync.py:268)
            if self.shard.total == self.shard.numel:
                ops.owner_sum_update(contribs, self.shard.g, sc, self._partials, **kw)
            else:       # alignment gaps: the norm is taken over the table's rows, not the whole flat buffer
                ops.owner_sum(contribs, self.shard.g, sc)
                ops.grad_update_scalars(self.shard.table, self._partials, **kw)
        self._partials_ready = False
        self._multiply_factor = out
        self._needs_sync = False
        return grad_norm.view(())

    def clip_grad_norm(self, max_norm, aggregate_norm_fn=None):
        """zero1_fast.py:139-162 for one owner.  Returns grad_norm as a 0-d fp32 device tensor, no host sync."""
        factor, out = self._clip_factor_args()
        grad_norm = torch.empty(1, dtype=torch.float32, device=self.shard.device)
        mn = float(max_norm)
        if aggregate_norm_fn is None:
            clip = dict(factor=factor, norm_out=self._norm, grad_norm_out=grad_norm, factor_out=out,
                        max_norm=mn if mn > 0.0 else 0.0)
            if self._partials_ready:
                ops.norm_clip(self._partials, **clip)
            else:
                ops.grad_norm_clip(self.shard.table, self._partials, **clip)
        else:
            if not self._partials_ready:
                ops.grad_sumsq(self.shard.table, self._partials)
            ops.norm_clip(self._partials, factor=1.0, norm_out=self._norm)
            norm = (self._norm.float() ** 2).sqrt()
            norm = aggregate_norm_fn(norm).reshape(1).to(torch.float32)
            ops.clip_factor(norm, factor=factor, grad_norm_out=grad_norm, factor_out=out,
                            max_norm=mn if mn > 0.0 else 0.0)
        self._partials_ready = False
        self._multiply_factor = out
        self._needs_sync = False
        return grad_norm.view(())

    def clip_grad_norm_update(self, max_norm, sample_size=None, numer=1.0, flags_out=None, clip_log_out=None):
        """multiply_grads(numer / where(sample_size > 0, sample_size, 1)) + clip_grad_norm(max_norm) in one launch,
        also writing the [finite, consistent] flags and the "clip" metric (yoco/tasks/trainer_nosync.py:273-286,
        :194-197).  sample_size: 1-element fp32 device tensor or None.  Returns grad_norm (0-d device tensor)."""
        factor, out = self._clip_factor_args()
        grad_norm = torch.empty(1, dtype=torch.float32, device=self.shard.device)
        mn = float(max_norm)
        kw = dict(sample_size=sample_size, numer=numer, factor=factor, max_norm=mn if mn > 0.0 else 0.0,
                  norm_out=self._norm, grad_norm_out=grad_norm, factor_out=out, flags_out=flags_out,
                  clip_log_out=clip_log_out)
        if self._partials_ready:
            ops.update_scalars(self._partials, **kw)
        else:
            ops.grad_update_scalars(self.shard.table, self._partials, **kw)
        self._partials_ready = False
        self._multiply_factor = out
        self._needs_sync = False
        return grad_norm.view(())

    def set_step(self, n):
        """The number of steps taken so far (the next step is n + 1), on the host and, with device_step, on the
        device."""
        self.step_count = int(n)
        if self.device_step:
            self._step_dev.fill_(int(n))

    def step(self, closure=None, groups=None, pieces=None, on_piece=None):
        """Adam + BF16 over the shard with the gradient factor folded into the gradient load, then factor := 1.

        pieces (optional): row boundaries [0, r1, ..., nrows]; Adam then runs as one launch per range (the same
        results), and on_piece(row_begin, row_end) is called after each range's launch is enqueued -- e.g. to record
        an event and start sending the finished BF16 rows on another stream, the exchange the reference runs after
        the whole step (yoco/tasks/zero1_fast.py:224-226)."""
        if pieces is not None:              # checked before anything changes
            if self.device_step:
                raise RuntimeError('yoco_z1: a step in pieces takes host-rounded bias corrections (device_step=False)')
            nrows = len(self.shard.numels)
            if list(pieces[:1]) != [0] or pieces[-1] != nrows or any(a > b for a, b in zip(pieces, pieces[1:])):
                raise RuntimeError(f'yoco_z1: pieces must run from 0 to {nrows} in order')
        self.step_count += 1
        bc1, bc2 = ops.bias_corrections(self.betas[0], self.betas[1], self.step_count, self.bias_correction)
        factor = self._multiply_factor
        if torch.is_tensor(factor):
            factor = self._as_device_factor(factor)
        elif float(factor) == 1.0:
            factor = None
        else:
            self._factor.fill_(float(factor))
            factor = self._factor
        if pieces is not None:
            for a, b in zip(pieces, pieces[1:]):
                ops.adam_cast_rows(self.shard.table, a, b, factor, self.lr, self.betas[0], self.betas[1], self.eps,
                                   bc1, bc2, self.weight_decay, self.mode)
                if on_piece is not None:
                    on_piece(a, b)
        elif self.device_step:
            ops.bias_corrections_step(self._step_dev, self.betas[0], self.betas[1], self._bc, self.bias_correction)
            ops.adam_cast_dev(self.shard.table, factor, self.lr, self.betas[0], self.betas[1], self.eps, self._bc,
                              self.weight_decay, self.mode)
        else:
            ops.adam_cast(self.shard.table, factor, self.lr, self.betas[0], self.betas[1], self.eps, bc1, bc2,
                          self.weight_decay, self.mode)
        self._multiply_factor = 1.0
        self._needs_sync = False

    def zero_grad(self):
        """zero1_fast.py:238-244 drops the gradients; the flat gradient is simply overwritten by the next owner
        sum, so nothing runs here."""
        self._needs_sync = False

    # -- one full update ---------------------------------------------------------------------------------------
    def update(self, max_norm=1.0):
        """clip_grad_norm(max_norm) + step(): the timed optimizer update."""
        gn = self.clip_grad_norm(max_norm)
        self.step()
        return gn
