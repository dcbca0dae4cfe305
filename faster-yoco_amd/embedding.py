"""Drop-in for the embedding owner's token-embedding gradient on this build's ``yoco_z1::embedding_dense_backward``
operators.

The reference forms it on the embedding's owner from every rank's rows with
``torch.ops.aten.embedding_dense_backward`` and scales by 1/world: after the call on the all-gathered rows
(yoco/models/decoder/layer_graphs.py:87-93) or on rows scaled in place first (the copy-engine path,
yoco/models/decoder/ce_reduce.py:226-231).  ``embedding_dense_backward`` keeps aten's signature and summation order
(its sort-based path above 3072 indices, its chunked kernel up to 3072) and fuses the scale;
``owner_embedding_grad`` / ``ce_owner_embedding_grad`` are the two call sites' forms.

A call allocates nothing but its result: the workspace is cached per device and grown when a larger call needs it
(``workspace``).  ``OwnerEmbeddingGrad`` is the allocation-free form -- output and workspace made once, for a fixed
row count -- which a caller can also capture in a HIP graph.
"""
import torch

from . import kernels, library  # noqa: F401  (library registers the operators)
from ._lib import require_gpu

_OPS = torch.ops.yoco_z1
_WORKSPACES = {}      # device -> uint8 workspace, grown on demand


def workspace_bytes(rows, dim, num_weights):
    return kernels.embedding_workspace_bytes(rows, dim, num_weights)


def workspace(device, rows, dim, num_weights):
    """The cached workspace of `device`, at least large enough for (rows, dim, num_weights)."""
    device = torch.device(device)
    need = workspace_bytes(rows, dim, num_weights)
    ws = _WORKSPACES.get(device)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _WORKSPACES[device] = ws
    return ws


def _args(grad, indices, scale, scale_first):
    require_gpu(grad, 'embedding_dense_backward')
    require_gpu(indices, 'embedding_dense_backward')
    if grad.dtype != torch.bfloat16:
        raise RuntimeError('embedding_dense_backward: expected bf16 gradient rows')
    D = grad.shape[-1]
    g = grad.reshape(-1, D).contiguous()
    idx = indices.reshape(-1).contiguous()
    if idx.dtype != torch.int64 or idx.numel() != g.shape[0] or idx.device != g.device:
        raise RuntimeError('embedding_dense_backward: indices must be int64, one per gradient row, on its device')
    mode = 0 if scale is None else (1 if scale_first else 2)
    return g, idx, kernels.f32(1.0 if scale is None else scale), mode


def embedding_dense_backward(grad, indices, num_weights, padding_idx, scale_grad_by_freq=False, *, scale=None,
                             scale_first=False, out=None):
    """aten.embedding_dense_backward(grad, indices, num_weights, padding_idx, scale_grad_by_freq) for bf16 grad
    rows [R, D] and int64 indices [R]; scale (optional) multiplies the rows before summing (scale_first, with a bf16
    rounding per row element as an in-place bf16 multiply does) or the finished bf16 result.  Returns a new bf16
    [num_weights, D] tensor, or fills `out`; every row of it is written."""
    if scale_grad_by_freq:
        raise RuntimeError('embedding_dense_backward: scale_grad_by_freq is not supported (the reference passes False)')
    g, idx, sc, mode = _args(grad, indices, scale, scale_first)
    ws = workspace(g.device, g.shape[0], g.shape[1], num_weights)
    if out is None:
        return _OPS.embedding_dense_backward(g, idx, int(num_weights), int(padding_idx), sc, mode, ws)
    _OPS.embedding_dense_backward_out_(g, idx, int(num_weights), int(padding_idx), sc, mode, out, ws)
    return out


def owner_embedding_grad(g_all, idx_all, num_weights, padding_idx, world, out=None):
    """_OwnerEmbedding.backward on the owner (layer_graphs.py:92-93): aten's sum, then x 1/world in bf16."""
    return embedding_dense_backward(g_all, idx_all, num_weights, padding_idx, False, scale=1.0 / world, out=out)


def ce_owner_embedding_grad(grads, ids, num_weights, padding_idx, world, out=None):
    """CEReduce.finish on the owner (ce_reduce.py:226-231): rows x 1/world (bf16), then aten's sum.  The staged
    rows are not modified (the reference scales them in place; nothing reads them afterwards)."""
    return embedding_dense_backward(grads, ids, num_weights, padding_idx, False, scale=1.0 / world,
                                    scale_first=True, out=out)


class OwnerEmbeddingGrad:
    """The owner's embedding gradient for a fixed shape, with its output and workspace made once: every call writes
    the same [num_weights, D] tensor and allocates nothing, so it can be captured in a HIP graph.  scale_first
    selects the copy-engine path's order (rows scaled first, ce_reduce.py:226-231), else layer_graphs.py:92-93's."""

    def __init__(self, rows, dim, num_weights, padding_idx, world, device, scale_first=False):
        self.rows, self.dim, self.num_weights = int(rows), int(dim), int(num_weights)
        self.padding_idx = int(padding_idx)
        self.scale = kernels.f32(1.0 / world)
        self.mode = 1 if scale_first else 2
        self.out = torch.empty(self.num_weights, self.dim, dtype=torch.bfloat16, device=device)
        self.ws = torch.empty(workspace_bytes(self.rows, self.dim, self.num_weights), dtype=torch.uint8,
                              device=device)

    def __call__(self, grad, indices):
        g = grad.reshape(-1, self.dim)
        idx = indices.reshape(-1)
        if g.shape[0] != self.rows or idx.numel() != self.rows:
            raise RuntimeError(f'OwnerEmbeddingGrad: made for {self.rows} rows, got {g.shape[0]}')
        if not (g.is_contiguous() and idx.is_contiguous()):
            raise RuntimeError('OwnerEmbeddingGrad: expected contiguous rows and indices')
        _OPS.embedding_dense_backward_out_(g, idx, self.num_weights, self.padding_idx, self.scale, self.mode,
                                           self.out, self.ws)
        return self.out
