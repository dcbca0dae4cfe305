/*
 * CPU oracle for the ZeRO-1 shard update -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker.  The product path (faster-yoco_amd/) never calls it.
 *
 * It restates, one IEEE operation at a time, the arithmetic of the reference's hot path:
 *   - owner sum       yoco/models/decoder/ce_reduce.py:59-74   (launch :178-183, scale = 1/world)
 *   - gradient scale  yoco/tasks/fused_adam_cast.py:75-89      (g32 = float(g16) * F[0])
 *   - Adam + BF16     yoco/tasks/fused_adam_cast.py:19-45      (host scalars :56-60)
 *   - norm -> clip    yoco/tasks/zero1_fast.py:139-162          (norm itself: fairseq clip_grad_norm_ / apex
 *                                                                multi_tensor_l2norm, restated as the exact
 *                                                                FP64 sum of squares; apex's order is not pinned)
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math (see oracle/Makefile).  No FMA is formed except where fmaf() is
 * written, division and square root are the IEEE correctly rounded SSE instructions, subnormals are kept.
 *
 * Pins (checked in tests/test_oracle_pins.py): torch CPU's float->bfloat16 conversion, torch CPU fp32 adds in rank
 * order, torch's own tensor/scalar expressions for the clip chain and the trainer's scalar chain, torch.optim.AdamW
 * within a few ulp, closed-form special cases (lr=0, g=0 pure decay, wd=0 mode equality, step-1 sign update), an
 * exact-rational restatement with a single rounding per operation, and for the embedding gradient exact cases plus
 * one only aten's runs-of-10 partial sums get right.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* float -> bfloat16, round to nearest even.  NaN -> 0x7FC0 (NaN payloads are not part of parity). */
uint16_t oracle_bf16_rne(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void oracle_bf16_rne_array(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_bf16_rne(x[i]);
}

/*
 * ce_reduce.py:66-74: acc = 0f; for k in 0..W-1: acc += float(x_k[e]); OUT[e] = bf16(acc * scale).
 * src[k] is contribution k (rank k).  out_sum (nullable) receives the raw FP32 rank-order sum acc.
 */
void oracle_owner_sum(const uint16_t* const* src, int world, int64_t n, float scale, uint16_t* out,
                      float* out_sum) {
    for (int64_t e = 0; e < n; ++e) {
        float acc = 0.0f;
        for (int k = 0; k < world; ++k) acc = acc + bf16_to_f32(src[k][e]);
        if (out_sum) out_sum[e] = acc;
        out[e] = oracle_bf16_rne(acc * scale);
    }
}

/*
 * The reference's slot mapping (ce_reduce.py:60-73): OUT holds rank R's own gradients, S the W-1 peer slots of G
 * elements each (peer s < R in slot s, s > R in slot s-1); elements [base, end) are summed and written to OUT.
 */
void oracle_sum_slots(const uint16_t* S, uint16_t* OUT, int64_t G, int64_t base, int64_t end, int R, float scale,
                      int W) {
    for (int64_t e = base; e < end; ++e) {
        float acc = 0.0f;
        for (int k = 0; k < W; ++k) {
            uint16_t x;
            if (k < R) x = S[(int64_t)k * G + e];
            else if (k == R) x = OUT[e];
            else x = S[(int64_t)(k - 1) * G + e];
            acc = acc + bf16_to_f32(x);
        }
        OUT[e] = oracle_bf16_rne(acc * scale);
    }
}

/* fused_adam_cast.py:78-81: G32 = float(G16) * F[0], one fp32 multiply. */
void oracle_scale_up(const uint16_t* g16, float* g32, float factor, int64_t n) {
    for (int64_t i = 0; i < n; ++i) g32[i] = bf16_to_f32(g16[i]) * factor;
}

/* Exact-as-possible L2 building block: sequential FP64 sum of squares of the (exactly upcast) values. */
double oracle_sumsq_f32(const float* g, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        double d = (double)g[i];
        s = s + d * d;          /* d*d is exact for an fp32-origin d (48 significant bits) */
    }
    return s;
}

double oracle_sumsq_bf16(const uint16_t* g, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        double d = (double)bf16_to_f32(g[i]);
        s = s + d * d;
    }
    return s;
}

/*
 * zero1_fast.py:150-160 with one owner (the all-reduce of sq is the identity):
 *   n_r = fp32 norm of the owned grads            (clip_grad_norm_(owned, 0) returns an fp32 tensor)
 *   sq = n_r ** 2 ; norm = sq.sqrt() ; grad_norm = factor * norm
 *   if max_norm > 0: coef = (max_norm / (grad_norm + 1e-6)).clamp_(max=1) ; factor *= coef
 * `python_float / tensor` is reciprocal(tensor) * python_float in torch, both rounded to fp32; clamp keeps NaN.
 * out[0] = n_r, out[1] = grad_norm, out[2] = the new factor.
 */
void oracle_norm_clip(double sumsq, float factor, float max_norm, float* out) {
    float nr = (float)sqrt(sumsq);
    float sq = nr * nr;
    float norm = sqrtf(sq);
    float gn = factor * norm;
    float f = factor;
    if (max_norm > 0.0f) {
        float t = gn + 1e-6f;
        float coef = (1.0f / t) * max_norm;
        coef = (coef > 1.0f) ? 1.0f : coef;
        f = f * coef;
    }
    out[0] = nr;
    out[1] = gn;
    out[2] = f;
}

/*
 * trainer_nosync.py:273-282 then zero1_fast.py:150-160 (one owner), plus the flags of trainer_nosync.py:285 and the
 * "clip" metric of :194-197.  has_ss: multiply the factor by numer / where(ss > 0, ss, 1) first (torch computes
 * `int / tensor` as reciprocal(tensor) * int).  out: [n_r, grad_norm, factor, finite, consistent, clip_log].
 */
void oracle_update_scalars(double sumsq, int has_ss, float ss, float numer, float factor, float max_norm,
                           float* out) {
    float fac = factor;
    if (has_ss) {
        float denom = (ss > 0.0f) ? ss : 1.0f;
        float c = (1.0f / denom) * numer;
        fac = c * fac;
    }
    float chain[3];
    oracle_norm_clip(sumsq, fac, max_norm, chain);
    out[0] = chain[0];
    out[1] = chain[1];
    out[2] = chain[2];
    out[3] = isfinite(chain[1]) ? 1.0f : 0.0f;
    out[4] = 1.0f;
    out[5] = (max_norm > 0.0f) ? (chain[1] > max_norm ? 100.0f : 0.0f) : -1.0f;
}

/* Same chain entered at `norm` (after sqrt(sq)), for the aggregate_norm_fn path. out[0]=grad_norm, out[1]=factor */
void oracle_clip_factor(float norm, float factor, float max_norm, float* out) {
    float gn = factor * norm;
    float f = factor;
    if (max_norm > 0.0f) {
        float t = gn + 1e-6f;
        float coef = (1.0f / t) * max_norm;
        coef = (coef > 1.0f) ? 1.0f : coef;
        f = f * coef;
    }
    out[0] = gn;
    out[1] = f;
}

/*
 * fused_adam_cast.py:58-60: bc = fp32(1 - pow(double beta, step)) if bias_correction == 1 else 1.0.
 * out[0] = bc1, out[1] = bc2.
 */
void oracle_bias_corrections(double beta1, double beta2, int64_t step, int bias_correction, float* out) {
    if (bias_correction == 1) {
        out[0] = (float)(1.0 - pow(beta1, (double)step));
        out[1] = (float)(1.0 - pow(beta2, (double)step));
    } else {
        out[0] = 1.0f;
        out[1] = 1.0f;
    }
}

/*
 * fused_adam_cast.py:22-45 per element, with the gradient factor of zero1_fast.py:175-192 folded in first
 * (g' = fp32(g * factor), skipped when apply_factor == 0).  `upd + wd*p` (:39) and `p - lr*upd` (:40) are taken as
 * contracted to single-rounding FMAs, as Triton's default fp fusion emits them; :32-33 are explicit FMAs.
 * g_bf16 != 0: g is a bfloat16 array (exact upcast).  p16 may be NULL.
 */
void oracle_adam_cast(const void* g, int g_bf16, float* p, float* m, float* v, uint16_t* p16, int64_t n,
                      float factor, int apply_factor, float lr, float beta1, float beta2, float eps, float bc1,
                      float bc2, float wd, int mode) {
    const float omb1 = 1.0f - beta1;
    const float omb2 = 1.0f - beta2;
    const float* g32 = (const float*)g;
    const uint16_t* g16 = (const uint16_t*)g;
    for (int64_t e = 0; e < n; ++e) {
        float gg = g_bf16 ? bf16_to_f32(g16[e]) : g32[e];
        if (apply_factor) gg = gg * factor;
        float pp = p[e];
        if (mode == 0) gg = fmaf(wd, pp, gg);
        float t1 = omb1 * gg;
        float mm = fmaf(beta1, m[e], t1);
        float t2 = omb2 * gg;
        t2 = t2 * gg;
        float vv = fmaf(beta2, v[e], t2);
        float mh = mm / bc1;
        float vh = vv / bc2;
        float den = sqrtf(vh) + eps;
        float upd = mh / den;
        if (mode == 1) upd = fmaf(wd, pp, upd);
        pp = fmaf(-lr, upd, pp);
        p[e] = pp;
        m[e] = mm;
        v[e] = vv;
        if (p16) p16[e] = oracle_bf16_rne(pp);
    }
}

/*
 * torch.ops.aten.embedding_dense_backward(grad[R x D], ids[R], V, padding_idx, False) as its sort-based GPU path
 * sums (called at yoco/models/decoder/layer_graphs.py:92 and ce_reduce.py:230): for each id t, its occurrences in
 * position order, fp32 partial sums over runs of 10, the partials summed in order, one bf16 rounding; padding rows
 * and ids outside [0, V) give zero rows.  scale_mode 1: each grad element first rounded to bf16(g * scale);
 * 2: the bf16 result multiplied by scale and rounded again.  Brute force over t (test sizes only).
 */
void oracle_embedding_backward(const int64_t* ids, const uint16_t* grad, int64_t R, int64_t D, int64_t V,
                               int64_t padding_idx, float scale, int scale_mode, uint16_t* out) {
    for (int64_t t = 0; t < V; ++t) {
        for (int64_t d = 0; d < D; ++d) {
            float acc = 0.0f, part = 0.0f;
            int64_t k = 0;
            for (int64_t r = 0; r < R; ++r) {
                if (ids[r] != t) continue;
                float x = bf16_to_f32(grad[r * D + d]);
                if (scale_mode == 1) x = bf16_to_f32(oracle_bf16_rne(x * scale));
                part = part + x;
                if (++k == 10) {
                    acc = acc + part;
                    part = 0.0f;
                    k = 0;
                }
            }
            if (k) acc = acc + part;
            uint16_t o = oracle_bf16_rne(acc);
            if (scale_mode == 2) o = oracle_bf16_rne(bf16_to_f32(o) * scale);
            int none = 1;
            for (int64_t r = 0; r < R && none; ++r) none = ids[r] != t;
            out[t * D + d] = (t == padding_idx || none) ? 0 : o;
        }
    }
}

/* The same gradient in the order of aten's kernel for few indices (embedding_dense_backward takes it for at most 3072
 * indices, the sort-based path above otherwise): positions in chunks of `chunk` consecutive indices; per chunk and id
 * the fp32 sum of that id's rows in position order, rounded to bf16 and added to the bf16 row of grad_weight (an fp32
 * add rounded to bf16).  chunk = 16 is what torch's ROCm build does on MI355X (checked against it on the GPU). */
void oracle_embedding_backward_chunked(const int64_t* ids, const uint16_t* grad, int64_t R, int64_t D, int64_t V,
                                       int64_t padding_idx, float scale, int scale_mode, int64_t chunk,
                                       uint16_t* out) {
    for (int64_t t = 0; t < V; ++t) {
        for (int64_t d = 0; d < D; ++d) {
            uint16_t acc = 0;
            int none = 1;
            for (int64_t c0 = 0; c0 < R; c0 += chunk) {
                float part = 0.0f;
                int any = 0;
                for (int64_t r = c0; r < R && r < c0 + chunk; ++r) {
                    if (ids[r] != t) continue;
                    float x = bf16_to_f32(grad[r * D + d]);
                    if (scale_mode == 1) x = bf16_to_f32(oracle_bf16_rne(x * scale));
                    part = part + x;
                    any = 1;
                }
                if (any) {
                    acc = oracle_bf16_rne(bf16_to_f32(acc) + bf16_to_f32(oracle_bf16_rne(part)));
                    none = 0;
                }
            }
            uint16_t o = acc;
            if (scale_mode == 2) o = oracle_bf16_rne(bf16_to_f32(o) * scale);
            out[t * D + d] = (t == padding_idx || none) ? 0 : o;
        }
    }
}

/* zero1_fast.py:61-65: params in order, each to the rank with the smallest running total (first such rank). */
void oracle_greedy_partition(const int64_t* numel, int nparam, int world, int32_t* owner, int64_t* sizes) {
    for (int r = 0; r < world; ++r) sizes[r] = 0;
    for (int i = 0; i < nparam; ++i) {
        int best = 0;
        for (int r = 1; r < world; ++r)
            if (sizes[r] < sizes[best]) best = r;
        owner[i] = best;
        sizes[best] += numel[i];
    }
}
