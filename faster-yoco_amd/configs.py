"""The five workloads of the benchmark and parity suite: tensor lists, hyperparameters and synthetic inputs.

C1  plumbing: 4 tensors, 9,438,208 params, step 1 from m = v = 0
C2  one GPU's YOCO-3B ZeRO-1 shard: 430,662,912 params in 38 tensors, step 1000
C3  C2 fed by 8 BF16 owner-side contributions summed in rank order (fused owner sum + norm)
C4  the unsharded YOCO-3B update: C2's list x 8 = 304 tensors, 3,445,303,296 params
C5  C2 with heavy-tailed (Student-t nu=2) gradients and 0.1% +-1e4 outliers (clip coefficient << 1)
C2R C2 on the real model's tensors: rank 0's shard of YOCO-3B's 240 tensors under the reference's greedy partition
    over 8 ranks, 443,357,184 params in 9 tensors (the largest of the eight shards, so the one that paces a step)
C4R C4 on the real model's tensors: YOCO-3B's 240 tensors, 3,445,303,296 params

Inputs are synthetic.  GPU inputs come from torch's seeded generator on the device (``fill_shard``); small parity
inputs come from NumPy's seeded PCG64 on the host (``host_inputs``) so the oracle sees the same arrays.
"""
import math
import os

import numpy as np
import torch

from . import layout

HPARAMS = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_norm=1.0)

C1_SHAPES = [(1024, 1024), (4096, 1024), (1024, 4096), (1024,)]
C1_MINI_SHAPES = [(64, 64), (256, 64), (64, 256), (64,)]

DIM, HIDDEN = 3072, 8192


def c2_shapes():
    """38 tensors, 430,662,912 = 3,445,303,296 / 8 params: ([3072,3072], [8192,3072], [3072]) x 12, then
    [3072,3072], then a 1-D tail of 5,952,768 elements."""
    s = [(DIM, DIM), (HIDDEN, DIM), (DIM,)] * 12 + [(DIM, DIM), (5_952_768,)]
    assert sum(math.prod(x) for x in s) == 430_662_912
    return s


def c4_shapes():
    """304 tensors, 3,445,303,296 params."""
    return c2_shapes() * 8


def yoco3b_shapes():
    """YOCO-3B's 240 trainable tensors in model order."""
    return layout.yoco3b_param_shapes()


def yoco3b_rank_shapes(rank=0, world=8):
    """The tensors rank `rank` owns under the greedy partition of YOCO-3B over `world` ranks, in model order."""
    s = yoco3b_shapes()
    owner, _ = layout.greedy_partition([math.prod(x) for x in s], world)
    return [x for x, r in zip(s, owner) if r == rank]


CONFIGS = {
    'c1': dict(shapes=C1_SHAPES, step=1, grad='normal', g_std=1e-3, m_std=0.0, v_std=0.0),
    'c2': dict(shapes=None, step=1000, grad='normal', g_std=1e-4, m_std=1e-4, v_std=1e-8),
    'c3': dict(shapes=None, step=1000, grad='owner8', g_std=1e-4, m_std=1e-4, v_std=1e-8),
    'c4': dict(shapes=None, step=1000, grad='normal', g_std=1e-4, m_std=1e-4, v_std=1e-8),
    'c5': dict(shapes=None, step=1000, grad='student_t', g_std=1e-3, m_std=1e-4, v_std=1e-8),
    'c2r': dict(shapes=None, step=1000, grad='normal', g_std=1e-4, m_std=1e-4, v_std=1e-8),
    'c4r': dict(shapes=None, step=1000, grad='normal', g_std=1e-4, m_std=1e-4, v_std=1e-8),
}


def shapes(name):
    if name == 'c1':
        return list(C1_SHAPES)
    if name in ('c2', 'c3', 'c5'):
        return c2_shapes()
    if name == 'c4':
        return c4_shapes()
    if name == 'c2r':
        return yoco3b_rank_shapes(0)
    if name == 'c4r':
        return yoco3b_shapes()
    raise KeyError(name)


def numel(name):
    return sum(math.prod(s) for s in shapes(name))


# ---------------------------------------------------------------------------------------------------- device
def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _normal_(t, std, gen, chunk=1 << 26):
    for i in range(0, t.numel(), chunk):
        t[i:i + chunk].normal_(0.0, std, generator=gen)
    return t


def student_t2_(t, scale, gen, chunk=1 << 26):
    """t = scale * (2u-1)/sqrt(2u(1-u)), u uniform in (0,1): Student-t with nu = 2 by its closed-form inverse CDF."""
    for i in range(0, t.numel(), chunk):
        u = torch.rand(min(chunk, t.numel() - i), dtype=torch.float64, device=t.device, generator=gen)
        u = u.clamp_(2.0 ** -30, 1.0 - 2.0 ** -30)
        t[i:i + chunk] = ((2.0 * u - 1.0) / torch.sqrt(2.0 * u * (1.0 - u)) * scale).to(t.dtype)
    return t


def outliers_(t, frac, value, gen):
    """Sets round(frac * n) distinct entries to +-value (sign random)."""
    n = t.numel()
    k = int(round(frac * n))
    if k == 0:
        return t
    idx = torch.randperm(n, device=t.device, generator=gen)[:k]
    sign = torch.randint(0, 2, (k,), device=t.device, generator=gen).to(t.dtype) * 2 - 1
    t[idx] = sign * value
    return t


def fill_shard(shard, name, seed=0):
    """Synthetic state for config `name` written into a FlatShard on its device: p ~ N(0, 0.02), m, v and g per
    the config.  Returns the owner-side contributions (list of bf16 flat tensors) for 'c3', else None."""
    cfg = CONFIGS[name]
    gen = _gen(shard.device, seed)
    _normal_(shard.p, 0.02, gen)
    if cfg['m_std'] > 0:
        _normal_(shard.m, cfg['m_std'], gen)
    else:
        shard.m.zero_()
    if cfg['v_std'] > 0:
        _normal_(shard.v, cfg['v_std'], gen).abs_()
    else:
        shard.v.zero_()
    if shard.p16 is not None:
        shard.p16.copy_(shard.p)
    if cfg['grad'] == 'owner8':
        contribs = []
        for r in range(8):
            c = torch.empty(shard.total, dtype=torch.float32, device=shard.device)
            _normal_(c, cfg['g_std'], _gen(shard.device, seed + 1 + r))
            contribs.append(c.to(torch.bfloat16))
            del c
        shard.g.zero_()
        return contribs
    if cfg['grad'] == 'student_t':
        student_t2_(shard.g, cfg['g_std'], gen)
        outliers_(shard.g, 1e-3, 1e4, gen)
    else:
        _normal_(shard.g, cfg['g_std'], gen)
    return None


# ------------------------------------------------------------------------------------------------------ host
def host_inputs(n, name='c1', seed=0):
    """NumPy inputs of n elements for config `name`: dict with g (float32), p, m, v and, for 'c3', 'contribs'
    (8 uint16 bf16 arrays).  Used by the parity tests, where the oracle must see exactly the GPU's inputs."""
    cfg = CONFIGS[name]
    rng = np.random.default_rng(seed)
    out = {'p': (rng.standard_normal(n) * 0.02).astype(np.float32)}
    out['m'] = (rng.standard_normal(n) * cfg['m_std']).astype(np.float32) if cfg['m_std'] > 0 else \
        np.zeros(n, np.float32)
    out['v'] = np.abs(rng.standard_normal(n) * cfg['v_std']).astype(np.float32) if cfg['v_std'] > 0 else \
        np.zeros(n, np.float32)
    if cfg['grad'] == 'student_t':
        u = (rng.integers(0, 1 << 24, n).astype(np.float64) + 0.5) / float(1 << 24)
        g = (2.0 * u - 1.0) / np.sqrt(2.0 * u * (1.0 - u)) * cfg['g_std']
        k = int(round(1e-3 * n))
        if k:
            idx = rng.choice(n, size=k, replace=False)
            g[idx] = np.where(rng.integers(0, 2, k) == 1, 1e4, -1e4)
        out['g'] = g.astype(np.float32)
    else:
        out['g'] = (rng.standard_normal(n) * cfg['g_std']).astype(np.float32)
    if cfg['grad'] == 'owner8':
        contribs = []
        for r in range(8):
            c = (np.random.default_rng(seed + 1 + r).standard_normal(n) * cfg['g_std']).astype(np.float32)
            u = c.view(np.uint32).astype(np.uint64)
            contribs.append(((u + 0x7fff + ((u >> 16) & 1)) >> 16).astype(np.uint16))
        out['contribs'] = contribs
    return out


_BASELINE_FIELDS = {'p': 0, 'm': 1, 'v': 2, 'g': 3, 'outliers': 4}      # contribution r: 16 + r


def baseline_inputs(name, seed=0, pieces=64, threads=None):
    """Full-size NumPy inputs of config `name` with BASELINE.json's distributions -- p ~ N(0, 0.02), the config's
    m ~ N(0, m_std), v = |N(0, v_std)|, g ~ N(0, g_std) (c5: Student-t(2) x 1e-3, drawn as the closed-form inverse of
    its CDF, exactly round(1e-3 n) entries set to +-1e4; c3: eight BF16 contributions ~ N(0, 1e-4), no g) -- as float32
    (contributions as uint16 bf16 bits).  Each field is cut into `pieces` fixed pieces, each drawn from its own PCG64
    stream seeded by (seed, field, piece), so the bits do not depend on `threads` (NumPy releases the GIL while it
    fills and computes, so the pieces run in parallel)."""
    from concurrent.futures import ThreadPoolExecutor
    cfg = CONFIGS[name]
    n = numel(name)
    bounds = [n * k // pieces for k in range(pieces + 1)]

    def rng(fid, k):
        return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, fid, k])))

    def normal(fid, std, out, absolute=False):
        def piece(k):
            lo, hi = bounds[k], bounds[k + 1]
            x = rng(fid, k).standard_normal(hi - lo, dtype=np.float32)
            x *= np.float32(std)
            out[lo:hi] = np.abs(x) if absolute else x
        return [(piece, k) for k in range(pieces)]

    def student(out):
        def piece(k):
            lo, hi = bounds[k], bounds[k + 1]
            u = (rng(_BASELINE_FIELDS['g'], k).integers(0, 1 << 24, hi - lo).astype(np.float64) + 0.5) / float(1 << 24)
            out[lo:hi] = ((2.0 * u - 1.0) / np.sqrt(2.0 * u * (1.0 - u)) * cfg['g_std']).astype(np.float32)
        return [(piece, k) for k in range(pieces)]

    def bf16(fid, std, out):
        def piece(k):
            lo, hi = bounds[k], bounds[k + 1]
            x = rng(fid, k).standard_normal(hi - lo, dtype=np.float32)
            x *= np.float32(std)
            u = x.view(np.uint32)
            out[lo:hi] = ((u + np.uint32(0x7fff) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
        return [(piece, k) for k in range(pieces)]

    out = {f: np.empty(n, np.float32) for f in ('p', 'm', 'v')}
    jobs = normal(0, 0.02, out['p']) + normal(1, cfg['m_std'], out['m']) + normal(2, cfg['v_std'], out['v'], True)
    if cfg['grad'] == 'owner8':
        out['contribs'] = [np.empty(n, np.uint16) for _ in range(8)]
        for r in range(8):
            jobs += bf16(16 + r, cfg['g_std'], out['contribs'][r])
    else:
        out['g'] = np.empty(n, np.float32)
        jobs += student(out['g']) if cfg['grad'] == 'student_t' else normal(3, cfg['g_std'], out['g'])
    with ThreadPoolExecutor(max_workers=threads or min(16, os.cpu_count() or 1)) as ex:
        for f in [ex.submit(fn, k) for fn, k in jobs]:
            f.result()
    if cfg['grad'] == 'student_t':
        k = int(round(1e-3 * n))
        r = rng(_BASELINE_FIELDS['outliers'], 0)
        idx = r.choice(n, size=k, replace=False)
        out['g'][idx] = np.where(r.integers(0, 2, k) == 1, np.float32(1e4), np.float32(-1e4))
    return out


def to_device_bf16(h, device):
    """uint16 bf16 bits (NumPy) -> bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).to(device).view(torch.bfloat16)


def bf16_bits(t):
    """bf16 tensor -> uint16 NumPy bits (host copy)."""
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


# --------------------------------------------------------------------------------------------- hashed inputs
# Inputs that NumPy on the host and torch on the device compute bit for bit alike, so that a full-size update can
# be checked against digests of the CPU oracle's outputs without regenerating the inputs on the host: a 32-bit
# integer hash of (stream, element index) in 64-bit integer arithmetic whose products stay below 2^63, turned
# into floats that are small integers times powers of two (exact in fp32; the BF16 contributions exact in bf16).
_M32 = 0xFFFFFFFF
_STREAM = {'p': 1, 'm': 2, 'v': 3, 'g': 4, 'scale': 5, 'pick': 6, 'sign': 7}   # contribution r: 16 + r
HASHED_CONFIGS = ('c2', 'c3', 'c5', 'c4', 'c2r', 'c4r')


def _mix32(x):
    x = x ^ (x >> 16)
    x = (x * 0x7FEB352D) & _M32
    x = x ^ (x >> 15)
    x = (x * 0x68E31DA5) & _M32
    return x ^ (x >> 16)


def _mix32_u32(x):
    """_mix32 in place on a NumPy uint32 array, whose products wrap modulo 2^32 (the same values, less memory)."""
    x ^= x >> 16
    x *= np.uint32(0x7FEB352D)
    x ^= x >> 15
    x *= np.uint32(0x68E31DA5)
    x ^= x >> 16
    return x


def _hash(idx, stream):
    if isinstance(idx, np.ndarray):
        x = _mix32_u32(idx.astype(np.uint32))              # element indices are below 2^32
        x += np.uint32((stream * 0x9E3779B1) & _M32)
        return _mix32_u32(x).astype(np.int64)
    return _mix32((_mix32(idx) + stream * 0x9E3779B1) & _M32)


class _NP:
    @staticmethod
    def f32(x):
        return x.astype(np.float32)

    @staticmethod
    def pow2(e):                     # 2**-e as float32, exactly, from its bits
        return ((127 - e) << 23).astype(np.int32).view(np.float32)

    where, abs = staticmethod(np.where), staticmethod(np.abs)


class _TORCH:
    @staticmethod
    def f32(x):
        return x.to(torch.float32)

    @staticmethod
    def pow2(e):
        return ((127 - e) << 23).to(torch.int32).view(torch.float32)

    where, abs = staticmethod(torch.where), staticmethod(torch.abs)


def hashed_values(name, field, idx):
    """Values of `field` ('p', 'm', 'v', 'g' or 'c0'..'c7', a BF16 contribution given as fp32) of config `name`
    at the int64 element indices `idx` (a NumPy array or a torch tensor, which decides where it is computed).
    p ~ U[-2^-5, 2^-5), m, g ~ U[-2^-13, 2^-13), v ~ U[0, 2^-27), 24-bit integers times powers of two; c5's g
    spreads each value over 24 binades by a hashed power of two and sets about 0.1% to +-1e4; the c3
    contributions are 8-bit integers times 2^-19 (exact in bf16)."""
    xp = _NP if isinstance(idx, np.ndarray) else _TORCH
    if field.startswith('c'):
        h = _hash(idx, 16 + int(field[1:]))
        return xp.f32((h >> 24) - 128) * np.float32(2.0 ** -19)
    s24 = xp.f32((_hash(idx, _STREAM[field]) >> 8) - (1 << 23))
    if field == 'p':
        return s24 * np.float32(2.0 ** -28)
    if field == 'm':
        return s24 * np.float32(2.0 ** -36)
    if field == 'v':
        return xp.abs(s24) * np.float32(2.0 ** -50)
    if name == 'c5':
        g = s24 * xp.pow2(29 + _hash(idx, _STREAM['scale']) % 24)
        big = xp.where((_hash(idx, _STREAM['sign']) & 1) == 1, np.float32(1e4), np.float32(-1e4))
        return xp.where(_hash(idx, _STREAM['pick']) % 1000 == 0, big, g)
    return s24 * np.float32(2.0 ** -36)


def fill_shard_hashed(shard, name, chunk=1 << 25):
    """The hashed inputs of config `name` written into a FlatShard on its device (element k of the concatenated
    tensor list gets index k; alignment gaps are left alone).  p16 = bf16(p).  Returns the eight BF16
    contributions (flat, laid out like the shard's gradient) for 'c3', else None."""
    dev = shard.device
    fields = ['p', 'm', 'v'] + ([] if name == 'c3' else ['g'])
    contribs = None
    if name == 'c3':
        contribs = [torch.zeros(shard.total, dtype=torch.bfloat16, device=dev) for _ in range(8)]
    k = 0
    for off, n in zip(shard.offsets, shard.numels):
        for i in range(0, n, chunk):
            m = min(chunk, n - i)
            idx = torch.arange(k + i, k + i + m, dtype=torch.int64, device=dev)
            for f in fields:
                getattr(shard, f)[off + i:off + i + m] = hashed_values(name, f, idx).to(getattr(shard, f).dtype)
            if contribs is not None:
                for r in range(8):
                    contribs[r][off + i:off + i + m] = hashed_values(name, f'c{r}', idx).to(torch.bfloat16)
        k += n
    if shard.p16 is not None:
        shard.p16.copy_(shard.p)
    if name == 'c3':
        shard.g.zero_()
    return contribs
