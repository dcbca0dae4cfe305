"""Stand-ins for the third-party objects the reference's hot path is driven through, for where fairseq, fairscale
and apex are not installed (this image): the tests and bench.py drive the drop-in surfaces through them, exactly as
the reference's trainer reaches them.  The product path never uses them.  They carry exactly the attributes
yoco/tasks/zero1_fast.py and fused_adam_cast.py use:

  FakeFusedAdamV2   fairseq's FusedAdamV2.step: one param group, step += 1, lazy fp32 exp_avg / exp_avg_sq,
                    then multi_tensor_applier(self.multi_tensor_adam, noop, [g, p, m, v], lr, beta1, beta2, eps,
                    step, adam_w_mode, bias_correction, weight_decay)  (fused_adam_cast.py:3-10,56-57)
  FakeOSS           fairscale OSS: .optim, ._param_to_rank (keyed by the fp32 tensor), .rank, .world_size,
                    .group, ._local_to_global_rank, partition_parameters(), step() -> optim.step()
  FakeFP16Optimizer fairseq FP16Optimizer: fp16_params, fp32_params (+ fp32 .grad buffers), fp32_optimizer
                    (.optimizer = OSS), has_flat_params, scaler, _multiply_factor, multiply_grads(c)
  FakeCEReduce      the fields CEReduce._sum reads (ce_reduce.py:178-183)
"""
import torch


class FakeFusedAdamV2:
    def __init__(self, params, lr, betas, eps, weight_decay, adam_w_mode=True, bias_correction=True):
        self.param_groups = [dict(params=list(params), lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                                  bias_correction=bias_correction, step=0)]
        self.state = {}
        self.adam_w_mode = 1 if adam_w_mode else 0
        self.multi_tensor_adam = None             # amp_C.multi_tensor_adam; replaced by FusedAdamCast
        self._dummy_overflow_buf = None

    def step(self, closure=None):
        for group in self.param_groups:
            group['step'] += 1
            g32, p32, m32, v32 = [], [], [], []
            for p in group['params']:
                if p.grad is None:
                    continue
                st = self.state.setdefault(p, {})
                if not st:
                    st['exp_avg'] = torch.zeros_like(p.data)
                    st['exp_avg_sq'] = torch.zeros_like(p.data)
                g32.append(p.grad.data)
                p32.append(p.data)
                m32.append(st['exp_avg'])
                v32.append(st['exp_avg_sq'])
            beta1, beta2 = group['betas']
            self.multi_tensor_adam(2048 * 32, self._dummy_overflow_buf, [g32, p32, m32, v32], group['lr'], beta1,
                                   beta2, group['eps'], group['step'], self.adam_w_mode,
                                   1 if group['bias_correction'] else 0, group['weight_decay'])


class FakeOSS:
    def __init__(self, params, **adam):
        self.optim = FakeFusedAdamV2(params, **adam)
        self._param_to_rank = {p: 0 for p in params}
        self.rank, self.world_size, self.group = 0, 1, None
        self._local_to_global_rank = [0]
        self.broadcasts = 0

    def partition_parameters(self):
        return [self.optim.param_groups[0]['params']]

    def _broadcast_params(self):
        self.broadcasts += 1

    def step(self, closure=None):
        self.optim.step(closure)
        self._broadcast_params()


class FakeFairseqOptimizer:
    def __init__(self, oss):
        self.optimizer = oss

    def step(self, closure=None, groups=None):
        self.optimizer.step(closure)


class FakeMixin:
    """Where zero1_fast.install puts clip_grad_norm / step / zero_grad; the originals must not be reached."""

    def clip_grad_norm(self, max_norm, aggregate_norm_fn=None):
        raise AssertionError('upstream clip_grad_norm reached')

    def step(self, closure=None, groups=None):
        raise AssertionError('upstream step reached')

    def zero_grad(self):
        raise AssertionError('upstream zero_grad reached')

    def multiply_grads(self, c):
        self._multiply_factor *= c                # fairseq: factor *= c


class FakeFP16Optimizer(FakeMixin):
    def __init__(self, fp16_params, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1):
        self.fp16_params = list(fp16_params)
        self.fp32_params = []
        for p in self.fp16_params:
            p32 = torch.nn.Parameter(p.detach().float().clone())
            p32.grad = torch.zeros_like(p32)
            self.fp32_params.append(p32)
        oss = FakeOSS(self.fp32_params, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
        self.fp32_optimizer = FakeFairseqOptimizer(oss)
        self.has_flat_params = False
        self.scaler = None
        self._multiply_factor = 1.0
        self._needs_sync = False


class FakeCEReduce:
    def __init__(self, staging, out, G, bounds, rank, world):
        self.staging, self.out, self.G, self.bounds, self.rank, self.world = staging, out, G, bounds, rank, world
