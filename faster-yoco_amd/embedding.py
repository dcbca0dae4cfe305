"""Drop-in for the embedding owner's token-embedding gradient on gfx950 kernels.

The reference forms it on the embedding's owner from every rank's rows with
``torch.ops.aten.embedding_dense_backward`` and scales by 1/world: after the call on the all-gathered rows
(yoco/models/decoder/layer_graphs.py:87-93) or on rows scaled in place first (the copy-engine path,
yoco/models/decoder/ce_reduce.py:226-231).  ``embedding_dense_backward`` keeps aten's signature and summation order
(its sort-based path above 3072 indices, its chunked kernel up to 3072) and fuses the scale; ``owner_embedding_grad`` / ``ce_owner_embedding_grad`` are the two
call sites' forms.
"""
import torch

from . import ops
from ._lib import check, lib, ptr, require_gpu, stream_handle


def workspace_bytes(rows, dim, num_weights):
    n = int(lib().z1_embedding_backward_workspace(int(rows), int(dim), int(num_weights)))
    if n < 0:
        check(n, 'z1_embedding_backward_workspace')
    return n


def embedding_dense_backward(grad, indices, num_weights, padding_idx, scale_grad_by_freq=False, *, scale=None,
                             scale_first=False, out=None):
    """aten.embedding_dense_backward(grad, indices, num_weights, padding_idx, scale_grad_by_freq) for bf16 grad
    rows [R, D] and int64 indices [R]; scale (optional) multiplies the rows before summing (scale_first, with a bf16
    rounding per row element as an in-place bf16 multiply does) or the finished bf16 result.  Returns (or fills)
    a bf16 [num_weights, D] tensor; every row of it is written."""
    require_gpu(grad, 'embedding_dense_backward')
    require_gpu(indices, 'embedding_dense_backward')
    if scale_grad_by_freq:
        raise RuntimeError('embedding_dense_backward: scale_grad_by_freq is not supported (the reference passes False)')
    if grad.dtype != torch.bfloat16:
        raise RuntimeError('embedding_dense_backward: expected bf16 gradient rows')
    D = grad.shape[-1]
    g = grad.reshape(-1, D).contiguous()
    idx = indices.reshape(-1).contiguous()
    if idx.dtype != torch.int64 or idx.numel() != g.shape[0] or idx.device != g.device:
        raise RuntimeError('embedding_dense_backward: indices must be int64, one per gradient row, on its device')
    if out is None:
        out = torch.empty(num_weights, D, dtype=torch.bfloat16, device=g.device)
    elif (out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != num_weights * D
          or out.device != g.device):
        raise RuntimeError('embedding_dense_backward: out must be a contiguous bf16 [num_weights, D] tensor')
    R = g.shape[0]
    ws = torch.empty(workspace_bytes(R, D, num_weights), dtype=torch.uint8, device=g.device)
    mode = 0 if scale is None else (1 if scale_first else 2)
    with torch.cuda.device(g.device):
        check(lib().z1_embedding_backward(ptr(idx), ptr(g), R, D, int(num_weights), int(padding_idx),
                                          ops.f32(1.0 if scale is None else scale), mode, ptr(out), ptr(ws), ws.numel(),
                                          stream_handle(g.device)), 'z1_embedding_backward')
    return out


def owner_embedding_grad(g_all, idx_all, num_weights, padding_idx, world):
    """_OwnerEmbedding.backward on the owner (layer_graphs.py:92-93): aten's sum, then x 1/world in bf16."""
    return embedding_dense_backward(g_all, idx_all, num_weights, padding_idx, False, scale=1.0 / world)


def ce_owner_embedding_grad(grads, ids, num_weights, padding_idx, world):
    """CEReduce.finish on the owner (ce_reduce.py:226-231): rows x 1/world (bf16), then aten's sum.  The staged
    rows are not modified (the reference scales them in place; nothing reads them afterwards)."""
    return embedding_dense_backward(grads, ids, num_weights, padding_idx, False, scale=1.0 / world, scale_first=True)
