"""Pins of the CPU oracle (no GPU): each oracle function against an independent routine -- torch CPU running the
reference's own expressions, torch.optim.AdamW, exact rational arithmetic, closed forms, the known YOCO-3B
partition -- chosen so that a dropped term, a swapped operand, a wrong sign or a double rounding fails."""
import math
import os
import sys

import numpy as np
import pytest
import torch

import oracle

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import exact  # noqa: E402

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)


def bits32(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def torch_bf16_bits(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------------------------------------ bf16 rounding
def test_bf16_rne_matches_torch_on_random_bit_patterns():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    x = x[~np.isnan(x)]
    assert np.array_equal(oracle.bf16_rne(x), torch_bf16_bits(x))


def test_bf16_rne_special_values_and_ties():
    specials = [0.0, -0.0, np.inf, -np.inf, 1.0, -1.0, np.finfo(np.float32).max, np.finfo(np.float32).tiny,
                1e-45, -1e-45, 1.17e-38]
    # exact ties: low 16 bits == 0x8000 with even and odd upper halves, and values just above / below a tie
    ties = np.array([0x3f808000, 0x3f818000, 0x3f808001, 0x3f807fff, 0x7f7f8000, 0x00008000, 0x00018000,
                     0x80008000, 0xbf818000], dtype=np.uint32).view(np.float32)
    x = np.concatenate([np.array(specials, np.float32), ties])
    assert np.array_equal(oracle.bf16_rne(x), torch_bf16_bits(x))
    assert oracle.bf16_rne(np.array([np.nan], np.float32))[0] & 0x7fff > 0x7f80       # NaN stays NaN


# ---------------------------------------------------------------------------------------------------- owner sum
@pytest.mark.parametrize('world', [1, 2, 7, 8, 16])
def test_owner_sum_matches_torch_rank_order_adds(world):
    rng = np.random.default_rng(world)
    n = 5001
    cs = [oracle.bf16_rne((rng.standard_normal(n) * 10.0 ** rng.integers(-6, 3)).astype(np.float32))
          for _ in range(world)]
    cs[0][:7] = 0x8000                                   # -0.0 contributions
    for c in cs:
        c[7] = 0x8000                                    # all -0 -> +0 (acc starts at +0)
    avg, s = oracle.owner_sum(cs, want_sum=True)
    acc = torch.zeros(n, dtype=torch.float32)
    for c in cs:
        acc = acc + torch.from_numpy(c.view(np.int16)).view(torch.bfloat16).float()
    ref = (acc * np.float32(1.0 / world)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits32(s), bits32(acc.numpy()))
    assert np.array_equal(avg, ref)
    assert avg[7] == 0x0000


def test_owner_sum_is_order_sensitive_in_rank_order():
    # a case where the fp32 sum depends on order: 1 + 2^-24 + 2^-24 vs 2^-24 + 2^-24 + 1
    a = oracle.bf16_rne(np.array([1.0], np.float32))
    b = oracle.bf16_rne(np.array([2.0 ** -24], np.float32))
    _, s1 = oracle.owner_sum([a, b, b], scale=1.0, want_sum=True)
    _, s2 = oracle.owner_sum([b, b, a], scale=1.0, want_sum=True)
    assert s1[0] == np.float32(1.0) and s2[0] == np.float32(1.0 + 2.0 ** -23)


def test_sum_slots_layout_brute_force():
    rng = np.random.default_rng(3)
    W, G = 8, 37
    for R in (0, 3, 7):
        S = oracle.bf16_rne(rng.standard_normal((W - 1) * G).astype(np.float32))
        OUT = oracle.bf16_rne(rng.standard_normal(G).astype(np.float32))
        base, end = 5, 31
        got = oracle.sum_slots(S, OUT.copy(), G, base, end, R, 1.0 / W, W)
        exp = OUT.copy()
        for e in range(base, end):
            acc = np.float32(0.0)
            for k in range(W):
                x = S[k * G + e] if k < R else OUT[e] if k == R else S[(k - 1) * G + e]
                acc = np.float32(acc + oracle.bf16_to_f32(np.array([x]))[0])
            exp[e] = oracle.bf16_rne(np.array([acc * np.float32(1.0 / W)], np.float32))[0]
        assert np.array_equal(got, exp)
        assert np.array_equal(got[:base], OUT[:base]) and np.array_equal(got[end:], OUT[end:])


# -------------------------------------------------------------------------------------------------- scale_up
def test_scale_up_matches_torch_mul_out():
    rng = np.random.default_rng(4)
    g16 = oracle.bf16_rne((rng.standard_normal(10000) * 1e-3).astype(np.float32))
    for f in (1.0, 0.482, 2.0 ** -11 * 8, 1.5e-7):
        f1 = torch.tensor([f], dtype=torch.float32)
        out = torch.empty(g16.size, dtype=torch.float32)
        torch.mul(torch.from_numpy(g16.view(np.int16)).view(torch.bfloat16), f1, out=out)  # zero1_fast.py:185
        assert np.array_equal(bits32(oracle.scale_up(g16, f)), bits32(out.numpy()))


# ------------------------------------------------------------------------------------------------------ norm
def test_sumsq_against_exactly_rounded_fsum():
    rng = np.random.default_rng(5)
    for scale in (1e-4, 1.0, 1e3):
        g = (rng.standard_normal(20001) * scale).astype(np.float32)
        exact_sum = math.fsum(float(x) * float(x) for x in g)       # squares exact in double, fsum exact
        assert abs(oracle.sumsq(g) - exact_sum) <= 20001 * 2.0 ** -53 * exact_sum
        assert abs(math.sqrt(oracle.sumsq(g)) - math.sqrt(exact_sum)) <= 1e-12 * math.sqrt(exact_sum)


def test_sumsq_bf16_and_power_of_two_scaling():
    rng = np.random.default_rng(6)
    g = rng.standard_normal(4097).astype(np.float32)
    h = oracle.bf16_rne(g)
    assert oracle.sumsq(h) == oracle.sumsq(oracle.bf16_to_f32(h))
    for k in (-20, -3, 5):
        assert oracle.sumsq(g * np.float32(2.0 ** k)) == oracle.sumsq(g) * 4.0 ** k
    # permutation changes the fp64 order only at round-off level
    assert abs(oracle.sumsq(g[::-1].copy()) - oracle.sumsq(g)) <= 1e-13 * oracle.sumsq(g)
    assert oracle.sumsq(np.zeros(0, np.float32)) == 0.0
    assert np.isinf(oracle.sumsq(np.array([1.0, np.inf], np.float32)))
    assert np.isnan(oracle.sumsq(np.array([1.0, np.nan], np.float32)))


def _torch_clip_chain(nr, factor, max_norm):
    """yoco/tasks/zero1_fast.py:150-160 literally, on torch CPU (one owner: the all-reduce is the identity)."""
    n = torch.tensor(nr, dtype=torch.float32)
    sq = n.float() ** 2
    norm = sq.sqrt()
    f = torch.tensor(factor, dtype=torch.float32) if isinstance(factor, torch.Tensor) else factor
    grad_norm = f * norm
    if max_norm > 0.0:
        clip_coef = (max_norm / (grad_norm + 1e-6)).clamp_(max=1)
        f = f * clip_coef
    f = f if isinstance(f, torch.Tensor) else torch.tensor(f, dtype=torch.float32)
    return np.float32(grad_norm.item()), np.float32(f.item())


@pytest.mark.parametrize('factor', [1.0, 2.0 ** -11 * 8, 0.37])
def test_norm_clip_chain_matches_torch_expressions(factor):
    rng = np.random.default_rng(7)
    vals = list(np.float32(10.0 ** rng.uniform(-8, 8, 300))) + [np.float32(0.0), np.float32(1.0),
                                                                 np.float32(0.999999), np.float32(3e19),
                                                                 np.float32(np.inf)]
    for nr in vals:
        for max_norm in (1.0, 0.0, 0.25):
            gn, f = _torch_clip_chain(float(nr), factor, max_norm)
            o_nr, o_gn, o_f = oracle.norm_clip(float(nr) ** 2, factor, max_norm)
            assert o_nr == nr
            assert bits32(o_gn) == bits32(gn) and bits32(o_f) == bits32(f), (nr, max_norm)


def _torch_trainer_scalars(nr, ss, numer, max_norm):
    """yoco/tasks/trainer_nosync.py:273-285 and :194-197 around zero1_fast.py:150-160, literally, on torch CPU."""
    sample_size = torch.tensor(ss, dtype=torch.float32)
    denom = torch.where(sample_size > 0, sample_size, torch.ones_like(sample_size))
    factor = 1.0
    factor *= numer / denom                                   # multiply_grads
    sq = torch.tensor(nr, dtype=torch.float32).float() ** 2
    norm = sq.sqrt()
    grad_norm = factor * norm
    if max_norm > 0.0:
        factor *= (max_norm / (grad_norm + 1e-6)).clamp_(max=1)
    finite = bool(torch.isfinite(grad_norm).all())
    clip = (torch.where(grad_norm > max_norm, grad_norm.new_tensor(100), grad_norm.new_tensor(0)).item()
            if max_norm > 0 else None)
    return np.float32(grad_norm.item()), np.float32(factor.item()), finite, clip


def test_update_scalars_match_trainer_torch_expressions():
    rng = np.random.default_rng(8)
    norms = list(np.float32(10.0 ** rng.uniform(-6, 6, 60))) + [np.float32(0.0), np.float32(np.inf)]
    for nr in norms:
        for ss in (16384.0, 2048.0, 1.0, 0.0, -3.0, 12345.0):
            for numer in (8, 1):
                for max_norm in (1.0, 0.0):
                    gn, f, finite, clip = _torch_trainer_scalars(float(nr), ss, numer, max_norm)
                    o = oracle.update_scalars(float(nr) ** 2, ss, numer, 1.0, max_norm)
                    assert bits32(o['grad_norm']) == bits32(gn) and bits32(o['factor']) == bits32(f)
                    assert o['finite'] == finite and o['consistent']
                    assert o['clip_log'] == clip
    o = oracle.update_scalars(float('nan'), float('nan'), 8, 1.0, 1.0)
    assert not o['finite'] and np.isnan(o['factor'])


def test_norm_clip_nan_propagates():
    o_nr, o_gn, o_f = oracle.norm_clip(float('nan'), 1.0, 1.0)
    assert np.isnan(o_nr) and np.isnan(o_gn) and np.isnan(o_f)
    gn, f = oracle.clip_factor(np.float32(np.inf), 1.0, 1.0)
    assert np.isinf(gn) and f == 0.0


def test_clip_factor_matches_norm_clip():
    for nr in np.float32([1e-3, 0.5, 2.0, 7.25]):
        _, gn1, f1 = oracle.norm_clip(float(nr) ** 2, 0.5, 1.0)
        gn2, f2 = oracle.clip_factor(np.sqrt(np.float32(nr * nr)), 0.5, 1.0)
        assert gn1 == gn2 and f1 == f2


# --------------------------------------------------------------------------------------------------- Adam
@pytest.mark.parametrize('step', [1, 2, 1000])
def test_bias_corrections_match_reference_host_rounding(step):
    for b1, b2 in ((0.9, 0.95), (0.9, 0.999)):
        exp = [float(torch.tensor(1.0 - math.pow(b, step), dtype=torch.float32)) for b in (b1, b2)]
        assert list(map(float, oracle.bias_corrections(b1, b2, step))) == exp
    assert list(map(float, oracle.bias_corrections(0.9, 0.95, 7, bias_correction=0))) == [1.0, 1.0]


def _rand_state(n, seed, step1=False):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * 10.0 ** rng.uniform(-5, -2, n)).astype(np.float32)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    m = np.zeros(n, np.float32) if step1 else (rng.standard_normal(n) * 1e-4).astype(np.float32)
    v = np.zeros(n, np.float32) if step1 else np.abs(rng.standard_normal(n) * 1e-8).astype(np.float32)
    return g, p, m, v


@pytest.mark.parametrize('step', [1, 10, 1000])
def test_adam_matches_torch_adamw(step):
    """torch.optim.AdamW (decoupled decay) is the same update up to rounding: a wrong term, sign, bias
    correction or eps placement fails this by orders of magnitude."""
    n = 4096
    g, p, m, v = _rand_state(n, step, step1=(step == 1))
    pt = torch.nn.Parameter(torch.from_numpy(p.copy()))
    opt = torch.optim.AdamW([pt], lr=HP['lr'], betas=(HP['beta1'], HP['beta2']), eps=HP['eps'],
                            weight_decay=HP['weight_decay'], foreach=False)
    if step > 1:
        opt.state[pt] = {'step': torch.tensor(float(step - 1)), 'exp_avg': torch.from_numpy(m.copy()),
                         'exp_avg_sq': torch.from_numpy(v.copy())}
    pt.grad = torch.from_numpy(g.copy())
    opt.step()
    po, mo, vo, p16 = oracle.adam_cast(g, p, m, v, step=step, **HP)
    st = opt.state[pt]
    b1m = np.abs(np.float32(HP['beta1']) * m) + np.abs(np.float32(0.1) * g)
    assert np.all(np.abs(mo - st['exp_avg'].numpy()) <= 1e-6 * b1m + 1e-30)
    assert np.all(np.abs(vo - st['exp_avg_sq'].numpy()) <= 1e-6 * vo + 1e-37)
    # the masters agree to round-off of the terms (p' can cancel to near zero, so no pure ulp bound)
    assert np.all(np.abs(po.astype(np.float64) - pt.detach().numpy()) <= 1e-6 * (np.abs(p) + HP['lr']))
    assert np.median(oracle.ulp_diff_f32(po, pt.detach().numpy())) <= 1
    assert np.array_equal(p16, torch_bf16_bits(po))


def test_adam_exact_rational_single_rounding():
    """Every fp32 operation of the oracle's Adam, including subnormal moments, against exact rationals rounded
    once (pins FMA placement, IEEE division / square root and the absence of double rounding)."""
    g, p, m, v = _rand_state(160, 11)
    v[:20] = np.float32(1e-42)                         # subnormal second moments
    m[20:40] = np.float32(-3e-41)
    g[40:50] = np.float32(0.0)
    for mode in (0, 1):
        for factor in (None, 0.482):
            po, mo, vo, _ = oracle.adam_cast(g, p, m, v, step=1000, mode=mode, factor=factor, **HP)
            bc1, bc2 = oracle.bias_corrections(HP['beta1'], HP['beta2'], 1000)
            for i in range(len(g)):
                ep, em, ev = exact.adam_elem(g[i], p[i], m[i], v[i], lr=HP['lr'], b1=HP['beta1'], b2=HP['beta2'],
                                             eps=HP['eps'], bc1=bc1, bc2=bc2, wd=HP['weight_decay'], mode=mode,
                                             factor=factor)
                assert bits32(mo[i]) == bits32(em) and bits32(vo[i]) == bits32(ev) and bits32(po[i]) == bits32(ep), \
                    (mode, factor, i)


def test_adam_special_cases():
    g, p, m, v = _rand_state(2048, 12)
    # lr = 0: the master is unchanged bit for bit
    hp = dict(HP, lr=0.0)
    po, mo, vo, p16 = oracle.adam_cast(g, p, m, v, step=5, **hp)
    assert np.array_equal(bits32(po), bits32(p)) and np.array_equal(p16, torch_bf16_bits(p))
    # wd = 0: decoupled (1) and L2 (0) modes coincide
    hp = dict(HP, weight_decay=0.0)
    a = oracle.adam_cast(g, p, m, v, step=5, mode=1, **hp)
    b = oracle.adam_cast(g, p, m, v, step=5, mode=0, **hp)
    assert all(np.array_equal(bits32(x), bits32(y)) for x, y in zip(a[:3], b[:3]))
    # g = m = v = 0, decoupled: pure decay p' = fma(-lr, fp32(wd * p), p)
    z = np.zeros_like(p)
    po, mo, vo, _ = oracle.adam_cast(z, p, z, z, step=1, **HP)
    assert not mo.any() and not vo.any()
    for i in range(0, 2048, 37):
        assert bits32(po[i]) == bits32(exact.fma(-exact.F(HP['lr']), exact.mul(HP['weight_decay'], p[i]), p[i]))
    # step 1 from zero moments with no decay: the update is sign(g) up to eps / |g|
    g1 = (np.sign(g) * np.maximum(np.abs(g), 1e-3)).astype(np.float32)
    po, _, _, _ = oracle.adam_cast(g1, p, z, z, step=1, **dict(HP, weight_decay=0.0))
    upd = (p.astype(np.float64) - po) / np.float32(HP['lr'])
    assert np.all(np.abs(upd - np.sign(g1)) <= 1e-3)


def test_adam_nan_and_inf_propagate():
    g = np.array([np.nan, np.inf, -np.inf, 1e-3], np.float32)
    p = np.full(4, 0.01, np.float32)
    z = np.zeros(4, np.float32)
    po, mo, vo, p16 = oracle.adam_cast(g, p, z, z, step=1, **HP)
    assert np.isnan(po[:3]).all() and np.isnan(mo[0]) and np.isinf(mo[1]) and np.isfinite(po[3])
    assert all((h & 0x7fff) > 0x7f80 for h in p16[:3])


# ------------------------------------------------------------------------------------------------- layout
# per-rank (tensor count, elements) of the greedy partition of YOCO-3B's 240 tensors over 8 ranks, worked out from
# the model code (yoco/models/yoco.py:147-153 dims) and yoco/tasks/zero1_fast.py:61-65's rule
YOCO3B_PARTITION = [(9, 443_357_184), (10, 418_197_504), (40, 428_141_568), (35, 440_573_952),
                    (39, 440_500_224), (32, 428_049_408), (39, 428_000_256), (36, 418_483_200)]


def test_greedy_partition_known_answer(pkg):
    from faster_yoco_amd import layout
    shapes = layout.yoco3b_param_shapes()
    numels = [math.prod(s) for s in shapes]
    assert len(shapes) == 240 and sum(numels) == 3_445_303_296
    owner, sizes = oracle.greedy_partition(numels, 8)
    assert [(owner.count(r), sizes[r]) for r in range(8)] == YOCO3B_PARTITION
    assert layout.greedy_partition(numels, 8) == (owner, sizes)
    rng = np.random.default_rng(13)
    for _ in range(20):
        nums = rng.integers(1, 10_000, rng.integers(1, 60)).tolist()
        w = int(rng.integers(1, 9))
        assert layout.greedy_partition(nums, w) == oracle.greedy_partition(nums, w)


# --------------------------------------------------------------------------------------------- embedding grad
def test_embedding_backward_exact_cases():
    rng = np.random.default_rng(14)
    V, D = 50, 6
    ids = rng.permutation(V)[:30].astype(np.int64)          # no repeats: rows are copied exactly
    g = oracle.bf16_rne(rng.standard_normal((30, D)).astype(np.float32))
    out = oracle.embedding_backward(ids, g, V, padding_idx=int(ids[3]))
    exp = np.zeros((V, D), np.uint16)
    exp[ids] = g
    exp[ids[3]] = 0
    assert np.array_equal(out, exp)
    # small-integer values: every partial and total is exact, so the result is the plain sum in any order
    ids = rng.integers(0, 8, 500).astype(np.int64)
    ids[:5] = [-1, 8, 9, 100, -7]                            # outside [0, V): ignored
    vals = rng.integers(-3, 4, (500, D)).astype(np.float32)
    out = oracle.embedding_backward(ids, oracle.bf16_rne(vals), 8)
    exp = np.zeros((8, D), np.float32)
    np.add.at(exp, ids[5:], vals[5:])
    assert np.array_equal(out, torch_bf16_bits(exp))
    # the 1/world scale: before or after, exact for a power of two
    a = oracle.embedding_backward(ids, oracle.bf16_rne(vals), 8, scale=0.125)
    b = oracle.embedding_backward(ids, oracle.bf16_rne(vals), 8, scale=0.125, scale_first=True)
    assert np.array_equal(a, b) and np.array_equal(a, torch_bf16_bits(exp * 0.125))


def test_embedding_backward_sums_in_runs_of_ten():
    """1 + 2^-8 followed by 18 x 2^-24: added one by one the tiny values are lost (ties to even) and the bf16 result
    is the tie 1 + 2^-8 -> 1.0; summed as aten does (partials over runs of 10 occurrences) the second run keeps
    10 x 2^-24 and the result rounds up to 1 + 2^-7."""
    vals = [1.0, 2.0 ** -8] + [2.0 ** -24] * 18
    g = oracle.bf16_rne(np.array(vals, np.float32).reshape(-1, 1))
    out = oracle.embedding_backward_sort(np.zeros(len(vals), np.int64), g, 1)
    assert out[0, 0] == 0x3F81
    seq = np.float32(0.0)
    for v in vals:
        seq = np.float32(seq + np.float32(v))
    assert torch_bf16_bits(np.array([seq], np.float32))[0] == 0x3F80


def test_embedding_backward_chunks_of_sixteen_below_the_sort_threshold():
    """aten's kernel for at most 3072 indices rounds each chunk's sum to bf16 before adding it to the bf16 row.  On
    one id, rows 1.0, 2^-9, fourteen zeros, 2^-8: chunks of 16 give bf16(1 + 2^-9) = 1.0 (a quarter ulp), then
    bf16(1.0 + 2^-8) = 1.0 (a tie, to even): 0x3F80.  One chunk of 32, and the sort path's runs of 10 (1 + 2^-9, then
    2^-8, summed in fp32), give bf16(1 + 3 * 2^-9) = 1 + 2^-7 (three quarters of an ulp, up): 0x3F81."""
    vals = [1.0, 2.0 ** -9] + [0.0] * 14 + [2.0 ** -8]
    g = oracle.bf16_rne(np.array(vals, np.float32).reshape(-1, 1))
    ids = np.zeros(len(vals), np.int64)
    assert oracle.embedding_backward_chunked(ids, g, 1)[0, 0] == 0x3F80
    assert oracle.embedding_backward_chunked(ids, g, 1, chunk=32)[0, 0] == 0x3F81
    assert oracle.embedding_backward_sort(ids, g, 1)[0, 0] == 0x3F81
    assert oracle.embedding_backward(ids, g, 1)[0, 0] == 0x3F80          # 17 rows: aten's few-rows kernel
    # the dispatch follows aten's threshold: more than 3072 rows take the sort path
    rng = np.random.default_rng(3)
    for R in (3072, 3073):
        ids = rng.integers(0, 5, R).astype(np.int64)
        g = oracle.bf16_rne((rng.standard_normal((R, 3)) * 1e-2).astype(np.float32))
        want = (oracle.embedding_backward_sort if R > 3072 else oracle.embedding_backward_chunked)(ids, g, 5)
        assert np.array_equal(oracle.embedding_backward(ids, g, 5), want)
