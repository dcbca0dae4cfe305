"""Writes the committed golden fixtures (inputs + oracle outputs) for the parity suite.

    python tests/golden/make_fixtures.py            # the small fixtures and the C1 digest (seconds)
    python tests/golden/make_fixtures.py --large    # large_digests.json: C2, C3, C5, C4 at full size (minutes)
    python tests/golden/make_fixtures.py --baseline # baseline_digests.json: C2, C3, C5 on BASELINE's distributions

Each fixture is an .npz (no pickles) holding the inputs of a small update and the CPU oracle's outputs:
owner-sum average (c3), the norm n_r, grad_norm, the clipped factor, and the Adam outputs p, m, v, p16 computed
with that factor.  c1_full_digest.json holds, for the full C1 update (9,438,208 parameters, seed 0, step 1), the
bits of the norm / grad_norm / factor and the sha256 of the oracle's p, m, v and BF16 outputs, so that a GPU run
can be checked bit for bit at that size without the oracle.  All are produced by this build's oracle
(oracle/z1_oracle.c), not by the reference: the reference ships no vectors for this path.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
MAX_NORM = 1.0

MINI = [(32, 32), (128, 32), (32, 128), (32,), (33, 7)]


def _inputs(n, seed, kind, step1):
    rng = np.random.default_rng(seed)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    m = np.zeros(n, np.float32) if step1 else (rng.standard_normal(n) * 1e-4).astype(np.float32)
    v = np.zeros(n, np.float32) if step1 else np.abs(rng.standard_normal(n) * 1e-8).astype(np.float32)
    if kind == 'student_t':
        u = (rng.integers(0, 1 << 24, n).astype(np.float64) + 0.5) / float(1 << 24)
        g = (2.0 * u - 1.0) / np.sqrt(2.0 * u * (1.0 - u)) * 1e-3
        k = max(1, int(round(1e-3 * n)))
        idx = rng.choice(n, size=k, replace=False)
        g[idx] = np.where(rng.integers(0, 2, k) == 1, 1e4, -1e4)
        g = g.astype(np.float32)
    else:
        g = (rng.standard_normal(n) * (1e-3 if step1 else 1e-4)).astype(np.float32)
    return g, p, m, v


def make(name, shapes, seed, kind='normal', step=1, owner=False):
    sizes = [int(np.prod(s)) for s in shapes]
    n = sum(sizes)
    g, p, m, v = _inputs(n, seed, kind, step == 1)
    out = {'shapes': np.array([list(s) + [0] * (2 - len(s)) for s in shapes], np.int64),
           'sizes': np.array(sizes, np.int64), 'step': np.int64(step), 'p': p, 'm': m, 'v': v,
           'hp': np.array([HP['lr'], HP['beta1'], HP['beta2'], HP['eps'], HP['weight_decay'], MAX_NORM])}
    if owner:
        rng = np.random.default_rng(seed + 100)
        contribs = np.stack([oracle.bf16_rne((rng.standard_normal(n) * 1e-3).astype(np.float32))
                             for _ in range(8)])
        avg16, s = oracle.owner_sum(list(contribs), want_sum=True)
        out.update(contribs=contribs, avg16=avg16, sum32=s)
        gin = avg16
    else:
        out['g'] = g
        gin = g
    ss = oracle.sumsq(gin)
    nr, gn, fac = oracle.norm_clip(ss, 1.0, MAX_NORM)
    po, mo, vo, p16 = oracle.adam_cast(gin, p, m, v, step=step, factor=fac, **HP)
    out.update(norm=np.float32(nr), grad_norm=np.float32(gn), factor=np.float32(fac), p_out=po, m_out=mo, v_out=vo,
               p16_out=p16)
    np.savez_compressed(os.path.join(HERE, f'{name}.npz'), **out)
    return out


def f32_hex(x):
    return '0x%08x' % int(np.float32(x).view(np.uint32))


def sha256(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_full_digest():
    """The full C1 update through the oracle: inputs from the package's seeded generator (configs.host_inputs,
    the one the GPU tests use), clip at 1.0, Adam mode 1 at step 1."""
    import __graft_entry__
    __graft_entry__.package()
    from faster_yoco_amd import configs
    shapes = configs.C1_SHAPES
    n = sum(int(np.prod(s)) for s in shapes)
    x = configs.host_inputs(n, 'c1', seed=0)
    step = configs.CONFIGS['c1']['step']
    nr, gn, fac = oracle.norm_clip(oracle.sumsq(x['g']), 1.0, MAX_NORM)
    po, mo, vo, p16 = oracle.adam_cast(x['g'], x['p'], x['m'], x['v'], step=step, mode=1, factor=fac, **HP)
    return {'config': 'c1', 'seed': 0, 'shapes': [list(s) for s in shapes], 'params': n, 'step': step, 'mode': 1,
            'hparams': HP, 'max_norm': MAX_NORM,
            'norm_bits': f32_hex(nr), 'grad_norm_bits': f32_hex(gn), 'factor_bits': f32_hex(fac),
            'sha256': {'p': sha256(po), 'm': sha256(mo), 'v': sha256(vo), 'p16': sha256(p16)}}


PREFIX = 1 << 20                      # elements of each input whose digest is recorded (input check on the GPU)


def large_digest(name, chunk=1 << 25):
    """The full-size update of config `name` (c2, c3, c5: the 430,662,912-parameter shard; c2r: 443,357,184; c4,
    c4r: 3,445,303,296) on
    the hashed inputs of configs.hashed_values, through the oracle, streamed in chunks of `chunk` elements: pass 1
    sums the squares of the gradient (c3: of the rank-order BF16 average of the eight contributions, x 1/8), the
    chunk sums added in FP64; norm -> clip at 1.0; pass 2 runs Adam mode 1 at step 1000 with the clipped factor and
    feeds sha256 of p, m, v, the BF16 copy (and the BF16 average for c3).  Also records the bits of the norm,
    grad_norm and factor and sha256 of the first PREFIX elements of every input.  Takes minutes."""
    import __graft_entry__
    __graft_entry__.package()
    from faster_yoco_amd import configs
    n = configs.numel(name)
    step = configs.CONFIGS[name]['step']
    gfields = [f'c{r}' for r in range(8)] if name == 'c3' else ['g']

    def values(field, lo, hi, sub=1 << 18):          # pieces small enough for malloc's heap (no page faults)
        a = np.empty(hi - lo, np.float32)
        for s in range(lo, hi, sub):
            e = min(hi, s + sub)
            a[s - lo:e - lo] = configs.hashed_values(name, field, np.arange(s, e, dtype=np.int64))
        return (a.view(np.uint32) >> 16).astype(np.uint16) if field.startswith('c') else a

    def grad(lo, hi):
        if name != 'c3':
            return values('g', lo, hi)
        return oracle.owner_sum([values(f, lo, hi) for f in gfields])

    prefix = {f: sha256(values(f, 0, PREFIX)) for f in ['p', 'm', 'v'] + gfields}
    ss = 0.0
    for lo in range(0, n, chunk):
        ss += oracle.sumsq(grad(lo, min(n, lo + chunk)))
    nr, gn, fac = oracle.norm_clip(ss, 1.0, MAX_NORM)
    hs = {k: hashlib.sha256() for k in (['avg16'] if name == 'c3' else []) + ['p', 'm', 'v', 'p16']}
    for lo in range(0, n, chunk):
        hi = min(n, lo + chunk)
        g = grad(lo, hi)
        po, mo, vo, p16 = oracle.adam_cast(g, values('p', lo, hi), values('m', lo, hi), values('v', lo, hi),
                                           step=step, mode=1, factor=fac, **HP)
        for k, a in (('avg16', g), ('p', po), ('m', mo), ('v', vo), ('p16', p16)):
            if k in hs:
                hs[k].update(np.ascontiguousarray(a).tobytes())
    return {'config': name, 'params': n, 'step': step, 'mode': 1, 'hparams': HP, 'max_norm': MAX_NORM,
            'inputs': 'faster_yoco_amd.configs.hashed_values', 'prefix_elements': PREFIX,
            'norm_bits': f32_hex(nr), 'grad_norm_bits': f32_hex(gn), 'factor_bits': f32_hex(fac),
            'sha256': {k: h.hexdigest() for k, h in hs.items()}, 'input_prefix_sha256': prefix}


def baseline_digest(name):
    """The full-size update of config `name` (c2, c3, c5) on BASELINE.json's own distributions
    (configs.baseline_inputs, seed 0: normals, Student-t with outliers, eight BF16 contributions), through the
    oracle: the norm (c3: of the rank-order BF16 average) -> clip at 1.0 -> Adam mode 1 at the config's step with
    the clipped factor; the bits of norm / grad_norm / factor and sha256 of p, m, v, the BF16 copy (and the BF16
    average for c3), plus sha256 of the first PREFIX elements of every input."""
    import __graft_entry__
    __graft_entry__.package()
    from faster_yoco_amd import configs
    x = configs.baseline_inputs(name, seed=0)
    step = configs.CONFIGS[name]['step']
    g = oracle.owner_sum(x['contribs']) if name == 'c3' else x['g']
    prefix = {f: sha256(x[f][:PREFIX]) for f in ('p', 'm', 'v')}
    if name == 'c3':
        prefix.update({f'c{r}': sha256(c[:PREFIX]) for r, c in enumerate(x['contribs'])})
    else:
        prefix['g'] = sha256(x['g'][:PREFIX])
    nr, gn, fac = oracle.norm_clip(oracle.sumsq(g), 1.0, MAX_NORM)
    po, mo, vo, p16 = oracle.adam_cast(g, x['p'], x['m'], x['v'], step=step, mode=1, factor=fac, **HP)
    digests = {'p': sha256(po), 'm': sha256(mo), 'v': sha256(vo), 'p16': sha256(p16)}
    if name == 'c3':
        digests['avg16'] = sha256(g)
    return {'config': name, 'params': int(g.size), 'step': step, 'mode': 1, 'hparams': HP, 'max_norm': MAX_NORM,
            'inputs': 'faster_yoco_amd.configs.baseline_inputs(name, seed=0)', 'prefix_elements': PREFIX,
            'norm_bits': f32_hex(nr), 'grad_norm_bits': f32_hex(gn), 'factor_bits': f32_hex(fac),
            'sha256': digests, 'input_prefix_sha256': prefix}


def main():
    if '--baseline' in sys.argv[1:]:
        d = {}
        for name in ('c2', 'c3', 'c5'):
            d[name] = baseline_digest(name)
            print('baseline digest of', name, 'done', flush=True)
        with open(os.path.join(HERE, 'baseline_digests.json'), 'w') as f:
            json.dump(d, f, indent=1)
            f.write('\n')
        print('baseline digests written to', HERE)
        return
    if '--large' in sys.argv[1:]:
        # --large [name ...]: (re)computes the named configs (default: all) and keeps the others' entries
        import __graft_entry__
        __graft_entry__.package()
        from faster_yoco_amd import configs
        names = [a for a in sys.argv[1:] if not a.startswith('--')] or list(configs.HASHED_CONFIGS)
        path = os.path.join(HERE, 'large_digests.json')
        d = {}
        if os.path.exists(path):
            with open(path) as f:
                d = json.load(f)
        for name in names:
            d[name] = large_digest(name)
            print('large digest of', name, 'done', flush=True)
        with open(path, 'w') as f:
            json.dump(d, f, indent=1)
            f.write('\n')
        print('large digests written to', HERE)
        return
    with open(os.path.join(HERE, 'c1_full_digest.json'), 'w') as f:
        json.dump(c1_full_digest(), f, indent=1)
        f.write('\n')
    make('c1_mini', MINI, seed=1, step=1)
    make('c2_mini', MINI, seed=2, step=1000)
    make('c3_mini', [(2048,), (3, 333), (64,)], seed=3, step=1000, owner=True)
    make('c5_mini', MINI, seed=5, kind='student_t', step=1000)
    print('fixtures written to', HERE)


if __name__ == '__main__':
    main()
