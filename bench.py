"""Benchmark of the ZeRO-1 shard optimizer update on one MI355X.

A step is one optimizer update of one GPU's shard with its inputs resident in HBM: the norm -> its final reduction
+ the clip factor -> Adam + BF16 copy (config c3: the owner sum of 8 BF16 contributions with the norm fused in, then
the final reduction + clip factor, then Adam).  Default workload: c2, the 430,662,912-parameter YOCO-3B shard (the configuration the metric is
quoted on).

Prints ONE JSON line: ms per step (the metric), the Adam kernel's roofline from HIP events recorded on the
launch stream, and the PyTorch-CPU restatement's time on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--config c2] [--cpu-sample-tensors T] [--no-cpu-baseline] [--dropin]
                    [--pipeline K] [--no-dropin-step] [--no-side]

With c2 or c3 the line also carries ``dropin_step``: the update at C3's shape through the reference's own seams
(CEReduce._sum per phase, zero1_fast.clip_grad_norm, zero1_fast.step -> FusedAdamCast), timed after the main steps.
"""
import argparse
import contextlib
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PEAK_HBM_GBPS = 8000.0
WORKLOADS = {
    'c1': 'C1 plumbing: 4 fp32 tensors, 9,438,208 params, step 1 (cache-resident; not graded)',
    'c2': 'C2 YOCO-3B ZeRO-1 shard: 430,662,912 params in 38 fp32 tensors, step 1000',
    'c3': 'C3 owner reduce: 8 bf16 contributions of the C2 shard summed in rank order, fused norm, Adam on bf16 g',
    'c4': 'C4 unsharded YOCO-3B: 3,445,303,296 params in 304 fp32 tensors, step 1000',
    'c5': 'C5 C2 with Student-t(2) gradients and 0.1% +-1e4 outliers (clip active)',
    'c2r': 'C2R rank 0 of YOCO-3B\'s 240 real tensors under the greedy 8-rank partition: 443,357,184 params in 9 '
           'fp32 tensors (the largest shard), step 1000',
    'c4r': 'C4R unsharded YOCO-3B on its 240 real tensors: 3,445,303,296 params, step 1000',
}


@contextlib.contextmanager
def gc_paused():
    """Python's cyclic garbage collector held off for a timed loop, as timeit holds it off: a collection pass that
    lands in the loop stops the host for tens of milliseconds, long enough for the GPU to run dry and idle."""
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def algorithmic_bytes(cfg, n):
    """(bytes per step, Adam bytes per launch, Adam bytes per param) from the per-parameter stream sizes."""
    if cfg == 'c3':
        return 46 * n, 28 * n, 28        # owner sum (16 in + 2 out) + Adam with bf16 g (g 2 + p,m,v 12 + 12 + p16 2)
    return 34 * n, 30 * n, 30            # norm (4) + Adam with fp32 g (16 in, 12 out, 2 bf16 out)


def traffic_file(kernel, workload):
    return os.path.join('profiles', f'{kernel}_{workload}_traffic.json')


def load_traffic(kernel, workload):
    """The committed counter summary under profiles/ (rocprofv3 --pmc: the bytes the L2 sends to the data fabric per
    launch, from the read / write request counts by size, which agree with the copy-calibrated FETCH_SIZE +
    WRITE_SIZE; the MALL serves some of them, which these counters cannot see), or None.  Not measured in this run:
    counters need their own profiler runs."""
    path = os.path.join(ROOT, traffic_file(kernel, workload))
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def cpu_baseline(shard, cfg, ntensors, contribs, hp, step, threads):
    """Times the PyTorch-CPU restatement (oracle/torch_cpu.py) on the first `ntensors` tensors of the same shard
    (copied from the GPU buffers), 1 warm-up + the median of the timed runs (at least 5, until ~10 s of timed work,
    at most 25), scaled to the whole shard by parameter count."""
    import torch
    sys.path.insert(0, ROOT)
    from oracle import torch_cpu
    torch.set_num_threads(threads)
    k = min(ntensors, len(shard.numels))
    n_s = sum(shard.numels[:k])
    end = shard.offsets[k - 1] + shard.numels[k - 1]
    host = {b: getattr(shard, b)[:end].cpu() for b in ('p', 'm', 'v')}
    g_host = shard.g[:end].float().cpu() if cfg != 'c3' else None
    c_host = [c[:end].cpu() for c in contribs] if cfg == 'c3' else None

    def views(buf):
        return [buf[o:o + n] for o, n in zip(shard.offsets[:k], shard.numels[:k])]

    times = []
    for it in range(26):           # 1 warm-up, then timed runs until ~10 s of timed work (at least 5, at most 25)
        if it > 5 and sum(times) >= 10.0:
            break
        p, m, v = host['p'].clone(), host['m'].clone(), host['v'].clone()
        g = g_host.clone() if g_host is not None else torch.empty(end, dtype=torch.float32)
        p16 = torch.empty(end, dtype=torch.bfloat16)
        t0 = time.perf_counter()
        torch_cpu.update(views(g), views(p), views(m), views(v), views(p16), lr=hp['lr'], betas=hp['betas'],
                         eps=hp['eps'], weight_decay=hp['weight_decay'], step=step, max_norm=hp['max_norm'],
                         contribs=c_host)
        t1 = time.perf_counter()
        if it:
            times.append(t1 - t0)
    times.sort()
    ms_sample = times[len(times) // 2] * 1e3
    return {'value': round(ms_sample * shard.numel / n_s, 3), 'unit': 'ms per full-shard step (scaled)',
            'cores': threads, 'kind': 'port',
            'sample': f'first {k} tensors of the same {cfg} shard ({n_s:,} of {shard.numel:,} params), '
                      f'median of {len(times)} after 1 warm-up ({sum(times):.1f} s timed) = {ms_sample:.1f} ms, '
                      f'scaled by parameter count; '
                      f'torch {torch.__version__} CPU, os.cpu_count()={os.cpu_count()}'}


def glue_timing(opt, hp, iters=200):
    """Microseconds per update of the trainer's scalar chain (yoco/tasks/trainer_nosync.py:273-286, :194-197 with
    zero1_fast.py:150-160) -- multiply_grads factor, norm -> clip, deferred-check flags, "clip" metric -- run as
    the reference runs it (separate torch ops on the device, flags staged to pinned memory) and as this build runs
    it (one z1_update_scalars launch).  The norm's partials are computed once beforehand; wall clock over `iters`
    back-to-back updates, synchronised at the end."""
    import torch
    from faster_yoco_amd import ops
    dev = opt.shard.device
    ops.grad_sumsq(opt.shard.table, opt._partials)
    nr = torch.zeros(1, device=dev)
    ops.norm_clip(opt._partials, norm_out=nr)
    ss = torch.tensor(16384.0, device=dev)
    host = torch.zeros(2, dtype=torch.bool, pin_memory=True)
    c100, c0 = nr.new_tensor(100), nr.new_tensor(0)
    max_norm = hp['max_norm']

    nr0 = nr.view(())                   # clip_grad_norm_ returns a 0-d tensor

    def reference_ops():
        denom = torch.where(ss > 0, ss, torch.ones_like(ss))
        factor = 1.0
        factor *= 8 / denom
        sq = nr0.float() ** 2
        norm = sq.sqrt()
        grad_norm = factor * norm
        factor *= (max_norm / (grad_norm + 1e-6)).clamp_(max=1)
        flags = torch.stack([torch.isfinite(grad_norm).all(), torch.ones((), dtype=torch.bool, device=dev)])
        host.copy_(flags, non_blocking=True)
        return torch.where(grad_norm > max_norm, c100, c0)

    flags_d = torch.zeros(2, dtype=torch.uint8, device=dev)
    gn, fo, cl = (torch.empty(1, device=dev) for _ in range(3))
    ss1 = ss.reshape(1)

    def fused():
        ops.update_scalars(opt._partials, sample_size=ss1, numer=8, factor=1.0, max_norm=max_norm, norm_out=nr,
                           grad_norm_out=gn, factor_out=fo, flags_out=flags_d, clip_log_out=cl)
        host.copy_(flags_d.view(torch.bool), non_blocking=True)

    out = {}
    for name, fn in (('reference_torch_ops', reference_ops), ('fused_kernel', fused)):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        with gc_paused():
            t0 = time.perf_counter()
            for _ in range(iters):
                fn()
            torch.cuda.synchronize()
            out[name] = round((time.perf_counter() - t0) * 1e6 / iters, 1)
    return out


def dropin_timing(dev, hp, step, reps=10):
    """The drop-in surface at C2's size: FusedAdamCast called with amp_C.multi_tensor_adam's signature (as
    fairseq's FusedAdamV2.step calls it) over the 38 C2 tensors allocated one by one (the reference's
    per-parameter layout, BF16 destinations as views of one flat buffer): with fp32 gradients; after the
    reference's scale pass (one scale_up per tensor writing the fp32 gradients, then Adam reading them); with the
    BF16 gradients folded in and the fp32 gradients written by the same launch (zero1_fast's default); folded
    without writing them (YOCO_Z1_FOLD_SCALE=1).  HIP events on the current stream, ms per call, and the host's
    time per call (wall clock of the enqueues, which the GPU's 2 ms per call keeps from ever waiting)."""
    import torch
    from faster_yoco_amd import configs
    from faster_yoco_amd.fused_adam_cast import FusedAdamCast, scale_up
    shapes = configs.shapes('c2')
    numels = [math.prod(s) for s in shapes]
    flat16 = torch.empty(sum(numels), dtype=torch.bfloat16, device=dev)
    gs, ps, ms, vs, g16s, dest, off = [], [], [], [], [], {}, 0
    for s, n in zip(shapes, numels):
        p = torch.empty(s, device=dev).normal_(0.0, 0.02)
        gs.append(torch.empty(s, device=dev).normal_(0.0, 1e-4))
        ms.append(torch.empty(s, device=dev).normal_(0.0, 1e-4))
        vs.append(torch.empty(s, device=dev).normal_(0.0, 1e-8).abs_())
        g16s.append(gs[-1].to(torch.bfloat16))
        ps.append(p)
        dest[p.data_ptr()] = flat16[off:off + n].view(s)
        off += n
    fa = FusedAdamCast(dest)
    noop = torch.zeros(1, dtype=torch.int32, device=dev)
    factor = torch.full((1,), 0.5, dtype=torch.float32, device=dev)
    out = {'tensors': len(shapes), 'params': sum(numels)}
    adam = lambda: fa(2048 * 32, noop, [gs, ps, ms, vs], hp['lr'], hp['betas'][0], hp['betas'][1], hp['eps'], step,
                      1, 1, hp['weight_decay'])

    def scale_then_adam():
        for g16, g in zip(g16s, gs):
            scale_up(g16, g, factor)
        adam()
    for name, fold, writes in (('fp32_grads_ms', False, False), ('scale_pass_then_adam_ms', None, False),
                               ('folded_bf16_grads_written_ms', True, True), ('folded_bf16_grads_ms', True, False)):
        fa.fold, fa.fold_factor, fa.fold_writes = {}, None, False
        if fold:
            fa.fold, fa.fold_factor = {p.data_ptr(): g for p, g in zip(ps, g16s)}, factor
            fa.fold_writes = writes
        call = scale_then_adam if fold is None else adam
        for _ in range(3):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with gc_paused():
            e0.record()
            t0 = time.perf_counter()
            for _ in range(reps):
                call()
            host = time.perf_counter() - t0
            e1.record()
            torch.cuda.synchronize()
        out[name] = round(e0.elapsed_time(e1) / reps, 4)
        out[name.replace('_ms', '_host_us')] = round(host / reps * 1e6, 1)
        fa.cast.clear()
    fa.fold, fa.fold_factor, fa.fold_writes = {}, None, False
    return out


def dropin_step_timing(dev, hp, step0, steps=20, warmup=5, world=8, rank=3):
    """One update through the reference's own seams at C3's shape, as its trainer runs it with the measured switches
    of scripts/configs/faster.env (ZERO1_FAST, ALLGATHER, PARAM_VIEWS, PARAM_ALLREDUCE + GRAD_REDUCE_OWNER,
    Z1_ONE_PASS, Z1_SCALE_KERNEL, FUSED_ADAM, CE_REDUCE):
      1. CEReduce._sum per phase (this build's, installed on a CEReduce with the reference's slot-major staging:
         8 BF16 contributions of the owner's 430,662,912-element gradient, rank 3's own in ``out``, laid out by
         backward phase as the reference lays it out; phases 0-1 on a side stream and then the last on the
         current one, as CEReduce.push / finish run them, yoco/models/decoder/ce_reduce.py:205-209,227-228), then
         the owned gradients made views of ``out`` (:232-237);
      2. zero1_fast.clip_grad_norm(1.0) (yoco/tasks/zero1_fast.py:139-162);
      3. zero1_fast.step() (:165-235) -> OSS.step -> FusedAdamV2.step -> FusedAdamCast: BF16 gradients folded in
         with the factor, FP32 master gradients written by the same launch;
    over the 38 C3 tensors, with fairseq's per-parameter FP32 masters, gradients and moments, and the BF16
    parameters placed in one flat buffer (fairseq / fairscale stand-ins, faster_yoco_amd.standins).
    Algorithmic bytes: owner sum 18 B/param (8 x 2 in, 2 out) + Adam 32 B/param (BF16 g 2, p / m / v 12 in; p / m / v
    12, BF16 copy 2, FP32 gradient 4 out); the norm reads nothing (the phase sums left its partials).  Timed
    steps chain: rank 3's own slot then holds the previous step's average, the same bytes and launches.  Also timed:
    the same with the norm read again from the gradients (ce_reduce.FUSE_NORM off, +2 B/param: its clip stage is
    the BF16 norm pass over the 38 gradient views plus the clip chain), that norm pass alone (back to back), and the
    phase sums alone, on one stream, with phase bounds on parameter boundaries and with bounds moved off every
    alignment."""
    import torch
    from faster_yoco_amd import ce_reduce, configs, layout, standins, zero1_fast
    shapes = configs.shapes('c3')
    numels = [math.prod(sh) for sh in shapes]
    G = sum(numels)
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)

    def normal(n, std, dtype=torch.float32):
        return (torch.randn(n, generator=gen, device=dev) * std).to(dtype)

    params = [torch.nn.Parameter(normal(n, 0.02, torch.bfloat16).view(sh)) for n, sh in zip(numels, shapes)]
    saved = {k: getattr(zero1_fast, k) for k in zero1_fast._SWITCHES}
    saved_orig, saved_placed = dict(zero1_fast._ORIG), dict(zero1_fast._PLACED)
    zero1_fast.configure(ENABLED=True, ALLGATHER=True, PARAM_VIEWS=True, REDUCE_OWNER=True, ONE_PASS=True,
                         SCALE_KERNEL=True, FUSED_ADAM=True, CE_ALLGATHER=False, FOLD_SCALE=False)
    zero1_fast._PLACED.clear()
    zero1_fast._PLACED.update(layout.place_params(params, 1))

    class Mixin(standins.FakeMixin):
        pass

    class Opt(Mixin, standins.FakeFP16Optimizer):
        pass

    zero1_fast._ORIG.clear()
    zero1_fast.install(Mixin)
    opt = Opt(params, lr=hp['lr'], betas=hp['betas'], eps=hp['eps'], weight_decay=hp['weight_decay'])
    adam = opt.fp32_optimizer.optimizer.optim
    adam.param_groups[0]['step'] = step0 - 1
    for p32, n in zip(opt.fp32_params, numels):
        adam.state[p32] = {'exp_avg': normal(n, 1e-4).view_as(p32),
                           'exp_avg_sq': normal(n, 1e-8).abs_().view_as(p32)}
    staging = normal((world - 1) * G, 1e-4, torch.bfloat16)
    out = normal(G, 1e-4, torch.bfloat16)
    # CEReduce's layout (ce_reduce.py:122-140): the owner's gradients ordered by backward phase, then model order;
    # three phases as layer_graphs.py:207-221 assigns them -- 0: the model's last parameters (output projection,
    # final norm, cross decoder), 1: the middle, 2: the first ones -- here the last, middle and first 12-13 tensors
    phase_of = [2] * 13 + [1] * 13 + [0] * (len(shapes) - 26)
    order = sorted(range(len(shapes)), key=lambda i: (phase_of[i], i))
    where, bounds, off = {}, [[0, 0] for _ in range(3)], 0
    for i in order:
        ph = phase_of[i]
        if bounds[ph][1] == 0:
            bounds[ph] = [off, off]
        where[i] = off
        off += numels[i]
        bounds[ph][1] = off
    cls = ce_reduce.install(type('CEReduce', (standins.FakeCEReduce,), {}))
    ce = cls(staging, out, G, bounds, rank, world)
    views = [out[where[i]:where[i] + n].view(sh) for i, (n, sh) in enumerate(zip(numels, shapes))]
    side = torch.cuda.Stream(device=dev)

    def sums():
        # phases 0 .. n-2 on the side stream, as CEReduce.push launches them during the backward; the last one on
        # the current stream, as finish() does, after them (in the reference the rest of the backward separates
        # them; launched side by side, two owner sums contend and take 1.22 instead of 1.18 ms)
        cur = torch.cuda.current_stream(dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for ph in range(len(ce.bounds) - 1):
                ce._sum(ph)
        cur.wait_stream(side)
        ce._sum(len(ce.bounds) - 1)

    def update(ev=None):
        if ev is not None:
            ev[0].record()
        sums()
        for p, g in zip(params, views):
            p.grad = g
        if ev is not None:
            ev[1].record()
        opt.clip_grad_norm(hp['max_norm'])
        if ev is not None:
            ev[2].record()
        opt.step()
        if ev is not None:
            ev[3].record()
        opt.zero_grad()

    def timed(fn, k):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with gc_paused():
            e0.record()
            t0 = time.perf_counter()
            for _ in range(k):
                fn()
            host = time.perf_counter() - t0
            e1.record()
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / k, host / k

    res = {'tensors': len(shapes), 'params': G, 'world': world, 'rank': rank, 'phases': len(ce.bounds)}
    try:
        for _ in range(warmup):
            update()
        ms, host = timed(update, steps)
        med = lambda xs: sorted(xs)[len(xs) // 2]

        def stages():
            ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(5)]
            for e in ev:
                update(e)
            torch.cuda.synchronize()
            return {'sums_ms': med([e[0].elapsed_time(e[1]) for e in ev]),
                    'clip_ms': med([e[1].elapsed_time(e[2]) for e in ev]),
                    'adam_ms': med([e[2].elapsed_time(e[3]) for e in ev])}
        stage = stages()
        nbytes = 50 * G
        res.update({'ms': round(ms, 4), 'host_us': round(host * 1e6, 1), 'algorithmic_bytes': nbytes,
                    'achieved_GBps': round(nbytes / (ms * 1e-3) / 1e9, 1),
                    'frac_of_peak': round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                    'stage_ms': {k: round(v, 4) for k, v in stage.items()},
                    'adam': {'kernel': 'adam_cast_kernel<1, 1, true>', 'bytes_per_param': 32,
                             'GBps': round(32 * G / (stage['adam_ms'] * 1e-3) / 1e9, 1)},
                    'sums_GBps': round(18 * G / (stage['sums_ms'] * 1e-3) / 1e9, 1)})
        ce_reduce.FUSE_NORM = False
        for _ in range(2):
            update()
        ms_u, _ = timed(update, steps)
        res['norm_read_again_ms'] = round(ms_u, 4)
        res['norm_read_again_stage_ms'] = {k: round(v, 4) for k, v in stages().items()}
        ce_reduce.FUSE_NORM = True
        # that norm pass alone: the BF16 norm over the 38 gradient views (a norm-only table, rows in address order
        # as the clip builds it), 20 launches back to back between two events; in the step it follows the phase
        # sums, whose stores are still draining (its clip stage above)
        from faster_yoco_amd import kernels, ops
        tab = kernels.Table([(v.view(-1), None, None, None, None, v.numel())
                             for v in sorted(views, key=lambda t: t.data_ptr())], dev)
        parts = ops.norm_workspace(dev)

        def norms():
            for _ in range(20):
                ops.grad_sumsq(tab, parts)
        norms()
        us = sorted(timed(norms, 1)[0] * 1e3 / 20 for _ in range(5))[2]
        res['norm_bf16_pass'] = {'kernel': 'sumsq_kernel<1, 128>', 'bytes': 2 * G, 'us_back_to_back': round(us, 1),
                                 'GBps': round(2 * G / (us * 1e-6) / 1e9, 1)}
        del tab

        def phases_one_stream():                                # the kernels alone: no cross-stream waits
            for ph in range(len(ce.bounds)):
                ce._sum(ph)
        phases_one_stream()
        res['sums_aligned_bounds_ms'] = round(timed(phases_one_stream, steps)[0], 4)
        odd = [0, bounds[0][1] + 1, bounds[1][1] + 3, G]        # 2- and 6-byte offsets: no common alignment
        ce.bounds = [[odd[i], odd[i + 1]] for i in range(3)]
        phases_one_stream()
        res['sums_odd_bounds_ms'] = round(timed(phases_one_stream, steps)[0], 4)
    finally:
        ce_reduce.FUSE_NORM = True
        zero1_fast.configure(**saved)
        zero1_fast._ORIG.clear()
        zero1_fast._ORIG.update(saved_orig)
        zero1_fast._PLACED.clear()
        zero1_fast._PLACED.update(saved_placed)
    return res


def pipeline_timing(shard, opt, k, reps=10):
    """Adam in k row ranges of the shard with each finished range's BF16 rows copied out on a second stream
    (faster_yoco_amd.exchange: the exchange the reference runs after the whole step, yoco/tasks/zero1_fast.py:224-226,
    with a copy into a local buffer standing in for a peer's) against one launch and a copy after it.  On one GPU
    the copy competes with Adam for the same HBM, so this measures what splitting costs, not what overlapping with
    xGMI would gain.  HIP events on the current stream (the last one after it waits for the side stream), ms per
    step, steps chained."""
    import torch
    from faster_yoco_amd import exchange
    pieces = exchange.even_pieces(shard.numels, k)
    remote = torch.empty_like(shard.p16)

    def send(first, last):
        remote[first:last].copy_(shard.p16[first:last])

    px = exchange.PipelinedExchange(shard, pieces, send)

    def whole_then_copy():
        opt.step()
        remote.copy_(shard.p16)

    out = {'pieces': len(pieces) - 1, 'rows_per_piece': [b - a for a, b in zip(pieces, pieces[1:])],
           'copy_bytes': 2 * 2 * shard.total}
    for name, fn in (('adam_whole_ms', lambda: opt.step()), ('adam_pieces_ms', lambda: opt.step(pieces=pieces)),
                     ('adam_then_copy_ms', whole_then_copy), ('adam_pipelined_copy_ms', lambda: px.step(opt))):
        for _ in range(2):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with gc_paused():
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
        out[name] = round(e0.elapsed_time(e1) / reps, 4)
    return out


def embedding_timing(dev, reps=20):
    """The embedding owner's gradient at the recipe's size (8 ranks x 2048 token rows of 3072, vocabulary 100,288):
    torch's aten.embedding_dense_backward + x 1/world as the reference runs it, against this build's fused kernel;
    HIP events on the current stream, milliseconds per call.  Uniform ids (the top-level keys) and Zipf(1.2) ids
    (``zipf1_2``: token frequencies as in text, the most frequent id on about 18 % of the rows)."""
    import numpy as np
    import torch
    from faster_yoco_amd import embedding
    R, D, V = 8 * 2048, 3072, 100288
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    uniform = torch.randint(0, V, (R,), device=dev, generator=gen)
    g = (torch.randn(R, D, device=dev, generator=gen) * 1e-2).to(torch.bfloat16)
    rng = np.random.default_rng(0)
    z = rng.zipf(1.2, R) - 1
    zipf = torch.from_numpy(np.where(z < V, z, rng.integers(0, V, R)).astype(np.int64)).to(dev)

    def timed(fn):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with gc_paused():
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) / reps, 4)

    res = {}
    for key, ids in (('uniform', uniform), ('zipf1_2', zipf)):
        r = {'aten_embedding_dense_backward': timed(lambda: torch.ops.aten.embedding_dense_backward(
                 g, ids, V, -1, False).mul_(1.0 / 8)),
             'z1_embedding_backward': timed(lambda: embedding.owner_embedding_grad(g, ids, V, -1, 8)),
             'longest_run': int(torch.bincount(ids, minlength=V).max().item())}
        if key == 'uniform':
            res.update(r)
        else:
            res[key] = r
    res.update(rows=R, dim=D, vocab=V, bytes_written=V * D * 2)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=50)
    ap.add_argument('--warmup', type=int, default=10)
    ap.add_argument('--config', default='c2', choices=sorted(WORKLOADS))
    ap.add_argument('--cpu-sample-tensors', type=int, default=1000)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--pipeline', type=int, default=0, metavar='K',
                    help='also time Adam in K row ranges with each range\'s BF16 rows copied out on a second stream '
                         '(the pipelined exchange; off by default for the same reason as --dropin)')
    ap.add_argument('--dropin', action='store_true',
                    help='also time FusedAdamCast over the 38 C2 tensors allocated one by one (its launches share '
                         'the Adam kernel with the timed steps, so a kernel trace of the default run stays clean)')
    ap.add_argument('--no-dropin-step', action='store_true',
                    help='skip the update through the reference\'s own seams at C3\'s shape (dropin_step)')
    ap.add_argument('--dropin-step-only', action='store_true',
                    help='only time dropin_step (--steps / --warmup apply to it), e.g. for counter runs')
    ap.add_argument('--no-side', action='store_true',
                    help='skip the side measurements (trainer scalar chain, embedding gradient), e.g. for counter runs')
    ap.add_argument('--calibrate-copy', action='store_true',
                    help='only run 5 plain 1 GiB device copies (the reference traffic for rocprofv3 counters)')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py: this build measures one GPU only (the shard update of one ZeRO-1 owner); '
              '--gpus must be 1', file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        a = torch.ones(1 << 28, dtype=torch.float32, device='cuda:0')
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({'calibration': 'torch copy_', 'bytes_read_per_launch': 1 << 30,
                          'bytes_written_per_launch': 1 << 30, 'launches': 5}))
        return
    sys.path.insert(0, ROOT)
    import __graft_entry__
    __graft_entry__.package()
    from faster_yoco_amd import configs, shard as shard_mod

    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    if args.dropin_step_only:
        print(json.dumps({'dropin_step': dropin_step_timing(dev, configs.HPARAMS, configs.CONFIGS['c3']['step'],
                                                            steps=args.steps, warmup=args.warmup)}), flush=True)
        return
    cfg = args.config
    hp = configs.HPARAMS
    gdt = torch.bfloat16 if cfg == 'c3' else torch.float32
    shard = shard_mod.FlatShard(configs.shapes(cfg), dev, grad_dtype=gdt)
    contribs = configs.fill_shard(shard, cfg, seed=0)
    step0 = configs.CONFIGS[cfg]['step']
    opt = shard_mod.Zero1ShardOptimizer(shard, lr=hp['lr'], betas=hp['betas'], eps=hp['eps'],
                                        weight_decay=hp['weight_decay'])
    opt.step_count = step0 - 1
    torch.cuda.synchronize()

    # the CPU baseline copies the pre-update state, so it runs before the GPU steps mutate it
    cpu = None
    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        cpu = cpu_baseline(shard, cfg, args.cpu_sample_tensors, contribs, hp, step0, threads)
        print(f'# cpu baseline done: {cpu["sample"]}', file=sys.stderr, flush=True)

    def one_step(ev=None):
        # a sampled step records three events: before the norm pass, before Adam, after Adam.  Each record leaves
        # the GPU idle for 2.5-5.5 us (a kernel trace of the loop shows no gap at all between the kernels of
        # unsampled steps), so only five steps of the timed region carry them.
        if ev is not None:
            ev[0].record()
        if contribs is not None:
            opt.reduce_clip(contribs, hp['max_norm'])      # owner sum + fused norm, then the clip chain
        else:
            opt.clip_grad_norm(hp['max_norm'])              # norm, then its final reduction + clip chain
        if ev is not None:
            ev[1].record()
        opt.step()
        if ev is not None:
            ev[2].record()

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    every = max(1, args.steps // 5)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(0, args.steps, every)]
    torch.cuda.synchronize()
    with gc_paused():
        t0 = time.perf_counter()
        for i in range(args.steps):
            one_step(events[i // every] if i % every == 0 else None)
        enqueued = time.perf_counter() - t0             # the host's share: every launch of the K steps enqueued
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0

    ms_step = wall * 1e3 / args.steps
    adam_ms = [e[1].elapsed_time(e[2]) for e in events]
    pre_ms = [e[0].elapsed_time(e[1]) for e in events]
    step_ms = sorted(e[0].elapsed_time(e[2]) for e in events)      # GPU time of each sampled step
    adam_avg = sum(adam_ms) / len(adam_ms)
    n = shard.numel
    step_bytes, adam_bytes, adam_bpp = algorithmic_bytes(cfg, n)
    achieved = adam_bytes / (adam_avg * 1e-3) / 1e9
    traffic = load_traffic('adam_cast', cfg)
    mall = traffic['mall_served_bytes_by_design'] if traffic else None
    out = {
        'metric': 'ms per optimizer step (431M-param shard); achieved HBM GB/s vs ~8 TB/s peak',
        'value': round(ms_step, 4),
        'unit': 'ms',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms_step, 4),
        'higher_is_better': False,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'fp32',
        'data': 'synthetic (seeded torch generator on the device; no checkpoint)',
        'config': {'workload': WORKLOADS[cfg], 'config': cfg, 'params': n, 'tensors': len(shard.numels),
                   'grad_dtype': str(gdt).replace('torch.', ''), 'lr': hp['lr'], 'betas': list(hp['betas']),
                   'eps': hp['eps'], 'weight_decay': hp['weight_decay'], 'max_norm': hp['max_norm'],
                   'algorithmic_bytes_per_step': step_bytes},
        'median_step_ms_events': round(step_ms[len(step_ms) // 2], 4),
        'host_us_per_step': round(enqueued * 1e6 / args.steps, 1),
        'event_sampled_steps': len(events),
        'achieved_GBps': round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
        'frac_of_peak': round(step_bytes / (ms_step * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
        'kernel_ms': {'adam_cast': round(adam_avg, 4),
                      ('owner_sum+norm_clip' if cfg == 'c3' else 'norm_clip'):
                          round(sum(pre_ms) / len(pre_ms), 4)},
        'roofline': {'bound': 'hbm', 'kernel': 'adam_flat_kernel', 'achieved': round(achieved, 1),
                     'peak': PEAK_HBM_GBPS, 'unit': 'GB/s', 'frac': round(achieved / PEAK_HBM_GBPS, 4),
                     'traffic': traffic['l2_to_fabric_bytes_per_launch'] if traffic else None,
                     'traffic_counted_at': 'L2 -> data fabric requests (TCC_EA0 read requests by size, 64-byte write '
                                           'requests); MALL hits included: TCC_EA0_RDREQ_DRAM equals TCC_EA0_RDREQ'
                                           if traffic else None,
                     'traffic_source': (traffic_file('adam_cast', cfg) + ' (rocprofv3 --pmc, committed; not measured '
                                        'in this run)') if traffic else None,
                     'mall_served_bytes_by_design': mall,
                     'dram_side_frac_estimate': (round((adam_bytes - mall) / (adam_avg * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)
                                                 if mall is not None else None),
                     'bytes_per_param': adam_bpp, 'params_per_launch': n},
        'cpu_baseline': cpu,
    }
    if not args.no_side:
        out['trainer_scalar_chain_us'] = glue_timing(opt, hp)
        out['owner_embedding_grad_ms'] = embedding_timing(dev)
    if args.dropin:
        out['dropin_multi_tensor_adam'] = dropin_timing(dev, hp, step0)
    if args.pipeline > 0:
        out['pipelined_exchange'] = pipeline_timing(shard, opt, args.pipeline)
    if not args.no_dropin_step and cfg in ('c2', 'c3'):
        del shard, opt, contribs                       # the shard's 15 GB, before the drop-in's own state
        torch.cuda.empty_cache()
        out['dropin_step'] = dropin_step_timing(dev, hp, configs.CONFIGS['c3']['step'])
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
