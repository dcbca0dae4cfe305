/*
 * yoco_z1 -- MI355X (gfx950) kernels for the owner-side, mixed-precision ZeRO-1 optimizer update of one GPU's
 * shard: owner gradient sum, multi-tensor L2 norm + clip factor, fused Adam + BF16 copy.
 *
 * C ABI: plain device pointers and sizes, no framework types.  Every launch is enqueued on the caller's stream
 * (hipStream_t passed as void*; NULL = the null stream) on the caller's current HIP device, with no host
 * synchronisation and no allocation.  The only allocating calls are z1_table_create / z1_table_destroy (set-up).
 *
 * Return value: Z1_OK (0), a negative Z1_E* argument error, or a positive hipError_t from the launch.
 * z1_strerror() turns either into text.
 *
 * Element semantics (the reference's, single rounding per fp32 operation, subnormals kept):
 *   bf16(x)  = round-to-nearest-even of x to bfloat16 (NaN -> a quiet NaN)
 *   g'       = fp32(g * factor)                                 g upcast exactly when bfloat16
 *   m'       = fma(b1, m, fp32((1-b1)*g'))      v' = fma(b2, v, fp32(fp32((1-b2)*g')*g'))
 *   upd      = (m'/bc1) / (sqrt(v'/bc2) + eps)  with IEEE division and square root
 *   mode 1:  upd = fma(wd, p, upd)              mode 0: g' = fma(wd, p, g') before m', v'
 *   p'       = fma(-lr, upd, p)                 p16 = bf16(p')
 */
#ifndef YOCO_Z1_H
#define YOCO_Z1_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    Z1_OK = 0,
    Z1_E_NULL = -1,        /* a required pointer is NULL */
    Z1_E_SIZE = -2,        /* a negative or inconsistent element count */
    Z1_E_DTYPE = -3,       /* unknown gradient dtype code */
    Z1_E_WORLD = -4,       /* world outside 1..Z1_MAX_WORLD */
    Z1_E_MODE = -5,        /* Adam mode other than 0 or 1 */
    Z1_E_WORKSPACE = -6,   /* workspace too small */
    Z1_E_DEVICE = -7,      /* table used on a device other than the one it was created on */
    Z1_E_NOALLOC_MAX = -8, /* input larger than the no-allocation entry point's fixed scratch */
    Z1_E_STATE = -9,       /* a binding launch on the table failed (its device rows may be half rewritten): launches
                              that read what it was rewriting are refused until it is bound again -- the gradients
                              by z1_table_set_grads or z1_table_rebind, the other columns by z1_table_rebind, the
                              FP32 gradient outputs by z1_table_set_grad_out */
};

enum { Z1_F32 = 0, Z1_BF16 = 1 };           /* gradient dtype codes */

#define Z1_MAX_WORLD 16                      /* most contributions one owner-sum call takes */
#define Z1_NORM_PARTIALS 2048                /* doubles in the norm workspace (fixed: the reduction order) */
#define Z1_NOALLOC_MAX_N (1ll << 29)         /* most elements z1_owner_sum_update_noalloc takes */

/* One row of the tensor-offset table.  g is float* (Z1_F32) or uint16_t* bfloat16 bits (Z1_BF16).  For the norm
 * only g and n are read; p, m, v may be NULL there.  p16 may be NULL (no BF16 copy for that tensor). */
typedef struct z1_tensor {
    const void* g;
    float* p;
    float* m;
    float* v;
    uint16_t* p16;
    int64_t n;
} z1_tensor;

typedef struct z1_table z1_table;            /* opaque, device-resident table + chunk schedule */

/* Builds the device copy of `rows` (plain copy of the pointers; rows with n == 0 are dropped) on the current
 * device.  The p, m, v and p16 ranges of different rows must not overlap (each element is updated by exactly one
 * lane; overlapping rows race).  Replaces the per-call tensor-list walk of yoco/tasks/fused_adam_cast.py:62-72 and
 * the bucket/view bookkeeping of yoco/tasks/zero1_fast.py:110-128 with one schedule built at set-up.  When the
 * rows, as last bound (here, z1_table_set_grads or z1_table_rebind), tile one allocation per stream in order and
 * without gaps -- a flat shard -- and no gradient outputs are set, a whole-table Adam launch walks those buffers
 * directly; the values are the same.  Allocates (hipMalloc). */
int z1_table_create(const z1_tensor* rows, int nrows, int g_dtype, z1_table** out);
/* Frees a table (hipFree, which first waits for the device's queued work, so launches already enqueued with the
 * table complete).  Not during stream capture; a captured graph whose launches use the table must not be replayed
 * after it. */
int z1_table_destroy(z1_table* table);
/* Total elements, chunk count and row count of a table (host-side values).  nrows is the count given to
 * z1_table_create, empty rows included: the row indices z1_adam_cast_rows and z1_table_set_grads take. */
int z1_table_info(const z1_table* table, int64_t* numel, int64_t* nchunks, int* nrows);

/* Points the table's rows at new gradient tensors of the same sizes and dtype: g is a HOST array of nrows device
 * pointers, one per row given to z1_table_create (entries of empty rows are ignored and may be NULL).  Enqueued on
 * the stream like a launch (no allocation, no host synchronisation): launches enqueued after it read the new
 * gradients.  For callers whose gradient tensors are reallocated between steps while the parameters and optimizer
 * state stay put (the reference's zero_grad drops every gradient, yoco/tasks/zero1_fast.py:238-244), so that one
 * table made at set-up serves every step.  Rows whose new gradient is not aligned for the vector path take the
 * element-wise path. */
int z1_table_set_grads(z1_table* table, const void* const* g, int nrows, void* stream);

/* Gives the table FP32 gradient outputs: g32 is a HOST array of nrows device float pointers, one per row given to
 * z1_table_create (entries of empty rows are ignored; NULL: no output for that row), or g32 = NULL for none.  The
 * z1_adam_cast, z1_adam_cast_rows and z1_adam_cast_dev launches enqueued after it also store every element's
 * g' = fp32(g * factor), the value the update consumes, to its row's output: the FP32 master gradient that the
 * reference's scale pass writes before its Adam reads it back (yoco/tasks/zero1_fast.py:175-192 with
 * yoco/tasks/fused_adam_cast.py:75-89), here written by the one pass that reads the BF16 gradient (32 bytes per
 * element instead of 6 + 30 over two passes, and one launch instead of one per tensor plus one).  No counterpart in
 * the reference: a fusion of two of its passes with the same values.  Outputs must not overlap any row's p, m, v or
 * p16.  Enqueued on the stream like a launch; no allocation, no host synchronisation. */
int z1_table_set_grad_out(z1_table* table, float* const* g32, int nrows, void* stream);

/* Points every row of the table at new tensors: rows as given to z1_table_create (the same count and the same n per
 * row, else Z1_E_SIZE; p, m, v present wherever the table had them).  Enqueued on the stream like z1_table_set_grads
 * (no allocation, no host synchronisation).  For callers whose tensors move as a whole -- a framework that runs the
 * update on copies of the state, as torch's functionalization may -- so that one table made at set-up follows
 * them. */
int z1_table_rebind(z1_table* table, const z1_tensor* rows, int nrows, void* stream);

/* Owner-side sum (replaces the Triton kernel _sum_slots, yoco/models/decoder/ce_reduce.py:59-74, launched by
 * CEReduce._sum :178-183):
 *   for e in [0,n): acc = 0f; for k = 0..world-1: acc += float(contrib[k][e]); out_avg[e] = bf16(acc * scale)
 * contrib is a HOST array of `world` device pointers (rank order); out_avg may alias one contribution (in place,
 * as OUT does in the reference).  out_sum (nullable) receives acc in fp32.  sumsq_partials (nullable) is a
 * workspace of z1_owner_sum_workspace(n) doubles; when given, the norm of the bf16 average is fused in and its
 * first Z1_NORM_PARTIALS doubles are ready for z1_norm_clip when the call's work completes. */
int z1_owner_sum_bf16(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                      float* out_sum, double* sumsq_partials, void* stream);
/* Doubles the fused-norm workspace of z1_owner_sum_bf16 / z1_owner_sum_update must hold for n elements
 * (negative: error code): Z1_NORM_PARTIALS + z1_owner_sum_waves(n). */
int64_t z1_owner_sum_workspace(int64_t n);
/* Per-chunk norm partials an owner sum over n elements writes (negative: error code).  The chunk grid follows the
 * streams' addresses (boundaries on shared 128-byte lines, else on 8-byte words, so that a range starting anywhere
 * keeps the vector path); this count covers every grid. */
int64_t z1_owner_sum_waves(int64_t n);

/* z1_owner_sum_bf16 with the fused norm left per chunk: waves (z1_owner_sum_waves(n) doubles; nullable: no norm)
 * receives each chunk's FP64 sum of squares of the BF16 average (a fixed decomposition; nothing is reduced).  For a
 * caller that sums a gradient buffer one range at a time -- CEReduce._sum, once per backward phase
 * (yoco/models/decoder/ce_reduce.py:178-183,205-209,227) -- and wants the norm of the whole buffer without reading
 * it again, as yoco/tasks/zero1_fast.py:150 does: the ranges' partials, side by side in one array, go to
 * z1_reduce_waves once.  No counterpart in the reference, whose screen of a norm fused into the sum was not adopted
 * (docs/training.md:335); the values are the same. */
int z1_owner_sum_bf16_waves(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                            float* out_sum, double* waves, void* stream);
/* Fixed-order reduction of m per-chunk partials (z1_owner_sum_bf16_waves) into the Z1_NORM_PARTIALS partials that
 * z1_norm_clip and z1_update_scalars_run read. */
int z1_reduce_waves(const double* waves, int64_t m, double* partials, void* stream);

/* Multi-tensor sum of squares of the table's gradients (the norm of fairseq utils.clip_grad_norm_ ->
 * apex multi_tensor_l2norm, called at yoco/tasks/zero1_fast.py:150,157): per-workgroup FP64 partials over a fixed
 * decomposition into `partials` (Z1_NORM_PARTIALS doubles), no atomics. */
int z1_grad_sumsq(const z1_table* table, double* partials, void* stream);

/* z1_grad_sumsq then z1_norm_clip in one call (the norm kernel and the one-workgroup final kernel, the same bits):
 * the norm + clip of yoco/tasks/zero1_fast.py:150-160 (fairseq utils.clip_grad_norm_ -> apex multi_tensor_l2norm,
 * then the torch scalar ops). */
int z1_grad_norm_clip(const z1_table* table, double* partials, const float* factor_in, float factor_value,
                      float* norm_out, float* grad_norm_out, float* factor_out, float max_norm, void* stream);

/* Fixed-order final reduction of the partials and the clip chain of yoco/tasks/zero1_fast.py:150-160 on device:
 *   n_r = fp32(sqrt(sum)); sq = n_r*n_r; norm = sqrt(sq); grad_norm = factor*norm;
 *   if max_norm > 0: factor *= min(fp32(1/(grad_norm + 1e-6)) * max_norm, 1)   (NaN propagates)
 * The factor is read from factor_in (device fp32 scalar) or, when factor_in is NULL, is factor_value (a host
 * value, e.g. fairseq's Python-float _multiply_factor).  The new factor goes to factor_out (nullable; may equal
 * factor_in).  norm_out / grad_norm_out (device fp32 scalars) are nullable. */
int z1_norm_clip(const double* partials, const float* factor_in, float factor_value, float* norm_out,
                 float* grad_norm_out, float* factor_out, float max_norm, void* stream);

/* The trainer's per-update scalar chain, for callers that also own the trainer step (yoco/tasks/
 * trainer_nosync.py:273-286 with zero1_fast.py:150-160): optional sample-size factor, then the z1_norm_clip chain,
 * the deferred-check flags and fairseq's "clip" logging value, in one launch.  Every output pointer is nullable. */
typedef struct z1_update_scalars {
    const float* sample_size;  /* device fp32 or NULL: factor *= numer / where(ss > 0, ss, 1), computed as torch
                                  computes `int / tensor`: fp32(fp32(1/denom) * numer) */
    float numer;               /* the data-parallel numerator (trainer_nosync.py:274) */
    const float* factor_in;    /* device fp32 factor before the update, or NULL to use factor_value */
    float factor_value;
    float max_norm;            /* clip when > 0 */
    float* norm_out;           /* the fp32 norm of the gradients (clip_grad_norm_'s value) */
    float* grad_norm_out;      /* factor * norm, as returned by clip_grad_norm */
    float* factor_out;         /* the clipped factor (may equal factor_in) */
    uint8_t* flags_out;        /* [isfinite(grad_norm), 1]: the two flags trainer_nosync._Pending.arm stages */
    float* clip_log_out;       /* 100 if grad_norm > max_norm else 0 (written when max_norm > 0) */
} z1_update_scalars;
int z1_update_scalars_run(const double* partials, const z1_update_scalars* u, void* stream);

/* z1_grad_sumsq then z1_update_scalars_run in one call. */
int z1_grad_update_scalars(const z1_table* table, double* partials, const z1_update_scalars* u, void* stream);

/* The owner sum with the norm fused in, then the z1_update_scalars chain, in one call: the owner sum of
 * yoco/models/decoder/ce_reduce.py:59-74, the norm and clip of yoco/tasks/zero1_fast.py:150-160 and optionally the
 * trainer's scalars of yoco/tasks/trainer_nosync.py:273-286 -- z1_owner_sum_bf16 followed by z1_update_scalars_run
 * on its partials (the same launches and bits).  workspace: z1_owner_sum_workspace(n) doubles; its first
 * Z1_NORM_PARTIALS hold the partials afterwards. */
int z1_owner_sum_update(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                        float* out_sum, double* workspace, const z1_update_scalars* u, void* stream);

/* z1_owner_sum_update with its workspace in the library's own fixed device scratch (a static device array of
 * 16.0 MiB per device, held until the process ends): no allocation of any kind, so callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc -- can run the owner sum, norm
 * and clip chain.  No counterpart in the reference.  n is at most Z1_NOALLOC_MAX_N (Z1_E_NOALLOC_MAX beyond; the
 * largest YOCO-3B owner shard is 443,357,184).  Every call on one device shares that device's scratch: calls that
 * overlap in time on one device (several streams, several threads) race.  Each call writes every scratch slot it
 * reads, so nothing carries over from the previous call.  The first call on a device looks up the scratch's
 * address there (hipGetSymbolAddress). */
int z1_owner_sum_update_noalloc(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                                float* out_sum, const z1_update_scalars* u, void* stream);

/* The clip chain entered at `norm` (device fp32), for callers that post-process the norm (aggregate_norm_fn,
 * yoco/tasks/zero1_fast.py:153-160): grad_norm = factor*norm; clip as above.  Factor arguments as above. */
int z1_clip_factor(const float* norm, const float* factor_in, float factor_value, float* grad_norm_out,
                   float* factor_out, float max_norm, void* stream);

/* Fused Adam + BF16 copy over every row of the table in one multi-tensor launch (replaces the per-tensor
 * Triton _adam launches of yoco/tasks/fused_adam_cast.py:19-45,62-72, and folds the gradient factor multiply of
 * yoco/tasks/zero1_fast.py:175-192 / scale_up :75-89 into the gradient load).  factor: device fp32 scalar or NULL
 * (1.0).  lr .. weight_decay are the fp32 kernel scalars; bc1, bc2 as fused_adam_cast.py:58-60 rounds them. */
int z1_adam_cast(const z1_table* table, const float* factor, float lr, float beta1, float beta2, float eps,
                 float bc1, float bc2, float weight_decay, int mode, void* stream);

/* z1_adam_cast with bc1 = bc[0] and bc2 = bc[1] read from device memory when the kernel runs (bc: device float[2],
 * e.g. from z1_bias_corrections_step), so that an update captured once in a HIP graph can be replayed at every
 * step.  No counterpart in the reference, whose host rounds the corrections at each call
 * (yoco/tasks/fused_adam_cast.py:58-60); the values are the same. */
int z1_adam_cast_dev(const z1_table* table, const float* factor, float lr, float beta1, float beta2, float eps,
                     const float* bc, float weight_decay, int mode, void* stream);

/* z1_adam_cast over the rows [row_begin, row_end) of the table only -- indices into the rows array given to
 * z1_table_create, empty rows included (Z1_E_SIZE outside 0 <= row_begin <= row_end <= nrows).  Same kernel and
 * per-element arithmetic, so consecutive ranges that cover the table equal one z1_adam_cast.  For a caller that
 * pipelines the step with the exchange of the finished BF16 rows, which the reference all-gathers after the whole
 * step (yoco/tasks/zero1_fast.py:224-226): after each range it can record an event and start sending that range on
 * another stream. */
int z1_adam_cast_rows(const z1_table* table, int row_begin, int row_end, const float* factor, float lr, float beta1,
                      float beta2, float eps, float bc1, float bc2, float weight_decay, int mode, void* stream);

/* The step counter and bias corrections on the device, for z1_adam_cast_dev: ++*step, then
 * bc[0] = fp32(1 - pow(beta1, *step)), bc[1] = fp32(1 - pow(beta2, *step)) in double (bias_correction != 1:
 * 1, 1) -- yoco/tasks/fused_adam_cast.py:58-60 with FusedAdamV2's group['step'] += 1, on the device.  step: device
 * int64; bc: device float[2]. */
int z1_bias_corrections_step(int64_t* step, double beta1, double beta2, int bias_correction, float* bc,
                             void* stream);

/* g32[i] = fp32(float(g16[i]) * factor[0]) (yoco/tasks/fused_adam_cast.py:75-89). */
int z1_scale_up(const uint16_t* g16, float* g32, const float* factor, int64_t n, void* stream);

/* p16[i] = bf16(p32[i]) (the leftover casts of yoco/tasks/zero1_fast.py:198-209). */
int z1_cast_bf16(const float* p32, uint16_t* p16, int64_t n, void* stream);

/* The embedding owner's token-embedding gradient: out[V x D] (bf16) = torch.ops.aten.embedding_dense_backward(
 * grad[R x D] (bf16), ids[R] (int64), V, padding_idx, False) with the reference's x 1/world
 * (yoco/models/decoder/layer_graphs.py:87-93: scale after, scale_mode 2; yoco/models/decoder/ce_reduce.py:226-231:
 * rows scaled first, scale_mode 1; 0: no scale).  Same order as aten for the row count.  For R > 3072 its
 * sort-based path: each id's occurrences in position order, fp32 partial sums over runs of 10, partials summed in
 * order, one bf16 rounding.  For R <= 3072 its kernel for few indices: chunks of 16 indices, per chunk and id an fp32
 * sum rounded to bf16 and added to the bf16 row.  Every row of
 * out is written (rows without occurrences, padding_idx and ids outside [0, V) give zeros).  workspace: device
 * memory of z1_embedding_backward_workspace(R, D, V) bytes (with D <= 2^24: about 4/7 of R x D x 4 bytes for
 * the fp32 run partials of frequent ids, and R x 16 + V x 4 bytes plus the sort's storage).  */
int z1_embedding_backward(const int64_t* ids, const uint16_t* grad, int64_t R, int64_t D, int64_t V,
                          int64_t padding_idx, float scale, int scale_mode, uint16_t* out, void* workspace,
                          int64_t workspace_bytes, void* stream);
int64_t z1_embedding_backward_workspace(int64_t R, int64_t D, int64_t V);
/* (z1_embedding_backward records no memset into a graph being captured: it sorts with a memset-free sort then.) */

/* Text for a return code (negative: argument errors; positive: hipError_t). */
const char* z1_strerror(int code);

#ifdef __cplusplus
}
#endif

#endif /* YOCO_Z1_H */
