"""faster-yoco_amd: MI355X-native owner-side ZeRO-1 optimizer update for one GPU's shard.

The directory name is not a Python identifier; the package is imported as ``faster_yoco_amd`` (the repository
root's ``faster_yoco_amd.py`` registers it under that name when the root is on sys.path).

Modules
    library          loads the path's PyTorch operators (torch.ops.yoco_z1.*, C++ over the C ABI) + fake kernels
    ops              the public operations on tensors and tables (each a torch.ops.yoco_z1 call)
    kernels          the tensor-offset tables (made through the C ABI, registered with the operators), helpers
    shard            flat HBM shard + FP16Optimizer-style optimizer (multiply_grads / clip_grad_norm / step)
    fused_adam_cast  drop-in for yoco/tasks/fused_adam_cast.py (FusedAdamCast, scale_up)
    zero1_fast       drop-in for yoco/tasks/zero1_fast.py (clip_grad_norm / step / zero_grad patches, layout)
    ce_reduce        drop-in for the owner-sum kernel of yoco/models/decoder/ce_reduce.py (_sum_slots, _sum)
    embedding        drop-in for the owner's token-embedding gradient (aten embedding_dense_backward + 1/world)
    trainer_glue     the optimizer part of trainer_nosync.train_step: one-launch scalar chain + deferred checks
    exchange         the BF16 exchange pipelined with the step (row ranges, side-stream sends)
    configs          the benchmark/parity workloads (tensor lists and synthetic inputs)
    standins         stand-ins of the fairseq / fairscale objects the drop-in surfaces are driven through where
                     those packages are absent (tests, bench.py); never used by the product path
"""
from . import _lib, library, ops  # noqa: F401

__all__ = ['library', 'ops', 'kernels', 'shard', 'fused_adam_cast', 'zero1_fast', 'ce_reduce', 'configs', 'layout',
           'trainer_glue', 'embedding', 'exchange', 'standins']
