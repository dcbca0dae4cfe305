"""Owner partition and flat-buffer layout of the ZeRO-1 shard (yoco/tasks/zero1_fast.py:52-75, 94-121).

The partition is fairscale OSS's greedy rule as the reference replicates it: parameters in model order, each to
the rank with the smallest running total (the first such rank on ties).  Each owner's parameters are contiguous,
in model order, in its segment of one flat buffer of ``world * seg`` elements, ``seg`` = the largest owner total.
"""
import torch


def greedy_partition(numels, world):
    """zero1_fast.py:61-65.  Returns (owner rank per parameter, elements per rank)."""
    if world < 1:
        raise ValueError('layout: world must be >= 1')
    sizes = [0] * world
    owner = []
    for n in numels:
        r = sizes.index(min(sizes))
        owner.append(r)
        sizes[r] += int(n)
    return owner, sizes


def owner_slots(numels, owners, world):
    """Given each parameter's owner: (offset of each parameter inside its owner's segment, model order; elements
    per owner; seg = the largest owner total, the segment length of the flat buffer)."""
    totals = [0] * world
    local = []
    for n, r in zip(numels, owners):
        local.append(totals[r])
        totals[r] += int(n)
    return local, totals, (max(totals) if totals else 0)


def segments(numels, world):
    """Owners, offsets of every parameter in the flat buffer of world * seg elements (zero1_fast.py:66-74), seg."""
    owner, _ = greedy_partition(numels, world)
    local, _, seg = owner_slots(numels, owner, world)
    return owner, [r * seg + o for r, o in zip(owner, local)], seg


def place_params(params, world, device=None):
    """zero1_fast.py:52-75 without the process group: makes every parameter a view of its owner's segment of one
    flat buffer (copying its data), returns {'flat', 'seg', 'owner': {id(p): rank}}."""
    params = [p for p in params if p.requires_grad]
    if not params:
        return {}
    owner, where, seg = segments([p.numel() for p in params], world)
    dev = device if device is not None else params[0].device
    flat = torch.empty(world * seg, dtype=params[0].dtype, device=dev)
    with torch.no_grad():
        for p, off in zip(params, where):
            v = flat[off:off + p.numel()].view_as(p)
            v.copy_(p.data)
            p.data = v
    return {'flat': flat, 'seg': seg, 'owner': {id(p): r for p, r in zip(params, owner)}}


def yoco3b_param_shapes(dim=3072, hidden=8192, layers=26, self_heads=24, attn_heads=24, kv_heads=8, vocab=100288):
    """The 240 trainable tensors of YOCO-3B in module registration order (yoco/models/decoder/yoco.py:51-83,
    127-139,195-207,264-277; gate_retention.py:40-46; cross_attention.py:26-27; feedforward_network.py:24-26;
    rms_norm.py:29-30).  3,445,303,296 elements."""
    shapes = [(vocab, dim), (vocab, dim)]                   # embed_tokens, output_projection
    ffn = [(hidden, dim), (hidden, dim), (dim, hidden)]     # fc1, gate, fc2
    for _ in range(layers // 2):                            # self decoder: gated retention layers
        shapes += [(dim, dim)] * 4 + [(self_heads, dim), (dim, dim)]      # q, k, v, g, gt, out
        shapes += [(dim,)] + ffn + [(dim,)]                 # mixer_layer_norm, ffn, final_layer_norm
    head_dim = dim // attn_heads
    shapes += [(head_dim * kv_heads, dim)] * 2 + [(dim,)]   # cross decoder k_proj, v_proj, kv_layer_norm
    for _ in range(layers // 2):                            # cross-attention layers
        shapes += [(dim, dim), (dim, dim)] + [(dim,)] + ffn + [(dim,)]
    shapes += [(dim,)]                                      # final layer_norm
    return shapes
