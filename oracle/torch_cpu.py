"""PyTorch-CPU restatement of the reference's optimizer update -- TEST/BASELINE INFRASTRUCTURE ONLY.

Used by bench.py's ``cpu_baseline`` leg (timed on the host cores) and by tests as a tolerance cross-check.  It runs
the reference sequence with torch CPU ops (there is no CPU build of apex's fused kernels):
  1. (owner reduce) FP32 rank-order sum of the BF16 contributions, x 1/world, rounded to BF16
     (yoco/models/decoder/ce_reduce.py:66-74);
  2. per-tensor FP32 L2 norms, then the norm of the stacked norms (fairseq clip_grad_norm_'s structure);
  3. the clip chain of yoco/tasks/zero1_fast.py:150-160;
  4. the gradient factor multiply (zero1_fast.py:189-192: _foreach_mul_);
  5. the Adam expression of yoco/tasks/fused_adam_cast.py:24-45 (decoupled decay, host-rounded bias corrections)
     as _foreach ops, then the BF16 copy.
Step 5 has no FMA on the CPU, so its results match the kernels' to a few ulp, not bit for bit.
"""
import math

import torch


def owner_sum(contribs):
    acc = torch.zeros(contribs[0].numel(), dtype=torch.float32)
    for c in contribs:
        acc.add_(c.float())
    return acc.mul_(1.0 / len(contribs)).to(torch.bfloat16)


def clip_grad_norm(grads, factor=1.0, max_norm=1.0):
    norms = [torch.linalg.vector_norm(g, dtype=torch.float32) for g in grads]
    total = torch.linalg.vector_norm(torch.stack(norms))
    sq = total.float() ** 2
    norm = sq.sqrt()
    grad_norm = factor * norm
    if max_norm > 0.0:
        factor = factor * (max_norm / (grad_norm + 1e-6)).clamp_(max=1)
    return grad_norm, factor


def adam_step(grads, params, exp_avg, exp_avg_sq, p16, *, lr, beta1, beta2, eps, weight_decay, step, factor):
    """One decoupled-decay Adam step over lists of fp32 CPU tensors, in place; p16 receives the BF16 copies."""
    if torch.is_tensor(factor) or factor != 1.0:
        torch._foreach_mul_(grads, factor)
    bc1 = float(torch.tensor(1.0 - math.pow(beta1, step), dtype=torch.float32))
    bc2 = float(torch.tensor(1.0 - math.pow(beta2, step), dtype=torch.float32))
    torch._foreach_mul_(exp_avg, beta1)
    torch._foreach_add_(exp_avg, grads, alpha=1.0 - beta1)
    torch._foreach_mul_(exp_avg_sq, beta2)
    torch._foreach_addcmul_(exp_avg_sq, grads, grads, value=1.0 - beta2)
    denom = torch._foreach_div(exp_avg_sq, bc2)
    torch._foreach_sqrt_(denom)
    torch._foreach_add_(denom, eps)
    upd = torch._foreach_div(exp_avg, bc1)
    torch._foreach_div_(upd, denom)
    torch._foreach_add_(upd, params, alpha=weight_decay)
    torch._foreach_add_(params, upd, alpha=-lr)
    torch._foreach_copy_(p16, params)


def update(grads, params, exp_avg, exp_avg_sq, p16, *, lr, betas, eps, weight_decay, step, max_norm=1.0,
           contribs=None):
    """The whole update; with contribs (lists of per-rank BF16 flat tensors) the gradient is their owner sum first
    and `grads` receives it (fp32 views of the BF16 average, tensor by tensor)."""
    if contribs is not None:
        avg = owner_sum(contribs).float()
        off = 0
        for g in grads:
            g.copy_(avg[off:off + g.numel()].view_as(g))
            off += g.numel()
    grad_norm, factor = clip_grad_norm(grads, 1.0, max_norm)
    adam_step(grads, params, exp_avg, exp_avg_sq, p16, lr=lr, beta1=betas[0], beta2=betas[1], eps=eps,
              weight_decay=weight_decay, step=step, factor=factor)
    return grad_norm
