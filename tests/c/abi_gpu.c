/* Plain-C, torch-free consumer of include/yoco_z1.h on the GPU (what a binding from another language does):
 * device buffers from hipMalloc, every call through the C ABI on the null stream, results checked against the CPU
 * oracle's C functions (oracle/z1_oracle.c, test infrastructure) at the parity bars of the Python suite:
 *   1. a 5-row table (tails, a row below one chunk, an empty row, 64-element row alignment): sum of squares ->
 *      norm + clip -> Adam + BF16 copy with the device factor; norm within 1e-6 of the exact one, the clip chain
 *      bit-exact from the GPU's norm, p / m / v / BF16 bit-exact given the GPU's factor; the one-call
 *      z1_grad_norm_clip (three calls in a row) gives the same bits as the two calls.  A second step, on new
 *      gradients bound with z1_table_set_grads (one of them misaligned), runs as two launches over row ranges
 *      bounded by z1_table_info's row count (empty row included), again bit-exact;
 *   2. the owner sum of 8 BF16 contributions with the fused norm: average and FP32 sum bit-exact, norm within
 *      1e-6 of the average's exact norm; the same sum one range at a time with z1_owner_sum_bf16_waves (odd
 *      bounds, an empty range) and the partials reduced once by z1_reduce_waves: the same average and sum bits,
 *      the norm within 1 ulp of the exact one; z1_owner_sum_update (with the clip chain, twice, then on a shorter
 *      input with the same workspace) gives the same bits as z1_owner_sum_bf16 + z1_norm_clip;
 *   3. the embedding gradient (workspace query, ids with repeats, out-of-range ids and padding, x 1/8 after) at
 *      5000 rows (aten's sort-path order) and 1000 rows (its order for few indices): bit-exact;
 *   4. a BF16-gradient table with FP32 gradient outputs (z1_table_set_grad_out; one output off the vector alignment,
 *      one row without): Adam + BF16 bit-exact, every output the oracle's scale_up bit for bit; with the outputs
 *      removed, a second launch leaves them untouched.
 * Built by __graft_entry__.build() with gcc, linked against libyoco_z1.so, the oracle and the HIP runtime, twice:
 * as tests/c/libabi_gpu.so, whose abi_gpu_run() tests/test_gpu_c_abi.py calls in-process, and with -DABI_GPU_MAIN
 * as the standalone program tests/c/abi_gpu.  Returns (exits with) 0 and prints "ok" on success. */
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "yoco_z1.h"

/* oracle/z1_oracle.c */
uint16_t oracle_bf16_rne(float x);
void oracle_scale_up(const uint16_t* g16, float* g32, float factor, int64_t n);
void oracle_owner_sum(const uint16_t* const* src, int world, int64_t n, float scale, uint16_t* out, float* out_sum);
double oracle_sumsq_f32(const float* g, int64_t n);
double oracle_sumsq_bf16(const uint16_t* g, int64_t n);
void oracle_norm_clip(double sumsq, float factor, float max_norm, float* out);
void oracle_bias_corrections(double beta1, double beta2, int64_t step, int bias_correction, float* out);
void oracle_adam_cast(const void* g, int g_bf16, float* p, float* m, float* v, uint16_t* p16, int64_t n,
                      float factor, int apply_factor, float lr, float beta1, float beta2, float eps, float bc1,
                      float bc2, float wd, int mode);
void oracle_embedding_backward(const int64_t* ids, const uint16_t* grad, int64_t R, int64_t D, int64_t V,
                               int64_t padding_idx, float scale, int scale_mode, uint16_t* out);
void oracle_embedding_backward_chunked(const int64_t* ids, const uint16_t* grad, int64_t R, int64_t D, int64_t V,
                                       int64_t padding_idx, float scale, int scale_mode, int64_t chunk,
                                       uint16_t* out);

#define HIP_OK(x)                                                                                   \
    do {                                                                                            \
        hipError_t e_ = (x);                                                                        \
        if (e_ != hipSuccess) {                                                                     \
            fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_));              \
            return 2;                                                                               \
        }                                                                                           \
    } while (0)
#define Z1_OK_(x)                                                                                   \
    do {                                                                                            \
        int r_ = (x);                                                                               \
        if (r_ != Z1_OK) {                                                                          \
            fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, z1_strerror(r_));                    \
            return 3;                                                                               \
        }                                                                                           \
    } while (0)
#define EXPECT(c)                                                                                   \
    do {                                                                                            \
        if (!(c)) {                                                                                 \
            fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #c);                   \
            return 4;                                                                               \
        }                                                                                           \
    } while (0)

static uint64_t rng = 0x9E3779B97F4A7C15ull;

static double unif(void) {                       /* xorshift64*, 53-bit uniform in (0, 1) */
    rng ^= rng >> 12;
    rng ^= rng << 25;
    rng ^= rng >> 27;
    return ((double)((rng * 0x2545F4914F6CDD1Dull) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

static float normal(double sd) {                 /* Box-Muller */
    return (float)(sd * sqrt(-2.0 * log(unif())) * cos(6.283185307179586 * unif()));
}

static uint32_t bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

static int same_f32(const float* a, const float* b, int64_t n) { return memcmp(a, b, (size_t)n * 4) == 0; }

static int table_update(void) {
    enum { R = 5 };
    const int64_t sizes[R] = {70001, 256 * 37, 0, 100, 4096 * 3 + 7};
    int64_t off[R], total = 0;
    for (int i = 0; i < R; ++i) {
        off[i] = total;
        total += (sizes[i] + 63) / 64 * 64;
    }
    float *hg = malloc(total * 4), *hp = malloc(total * 4), *hm = malloc(total * 4), *hv = malloc(total * 4);
    float *op = malloc(total * 4), *om = malloc(total * 4), *ov = malloc(total * 4);
    uint16_t *h16 = malloc(total * 2), *o16 = malloc(total * 2);
    for (int64_t i = 0; i < total; ++i) {
        hg[i] = normal(1e-2);                    /* norm about 3.1 over these ~95K elements: the clip is active */
        hp[i] = normal(0.02);
        hm[i] = normal(1e-4);
        hv[i] = fabsf(normal(1e-8));
    }
    float *dg, *dg2, *dp, *dm, *dv, *ds;
    uint16_t* d16;
    double* dpart;
    HIP_OK(hipMalloc((void**)&dg, total * 4));
    HIP_OK(hipMalloc((void**)&dg2, (total + 1) * 4));
    HIP_OK(hipMalloc((void**)&dp, total * 4));
    HIP_OK(hipMalloc((void**)&dm, total * 4));
    HIP_OK(hipMalloc((void**)&dv, total * 4));
    HIP_OK(hipMalloc((void**)&d16, total * 2));
    HIP_OK(hipMalloc((void**)&ds, 6 * 4));
    HIP_OK(hipMalloc((void**)&dpart, Z1_NORM_PARTIALS * 8));
    HIP_OK(hipMemcpy(dg, hg, total * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dp, hp, total * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dm, hm, total * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dv, hv, total * 4, hipMemcpyHostToDevice));

    z1_tensor rows[R];
    for (int i = 0; i < R; ++i) {
        rows[i].g = dg + off[i];
        rows[i].p = dp + off[i];
        rows[i].m = dm + off[i];
        rows[i].v = dv + off[i];
        rows[i].p16 = d16 + off[i];
        rows[i].n = sizes[i];
    }
    z1_table* t = NULL;
    Z1_OK_(z1_table_create(rows, R, Z1_F32, &t));
    int64_t numel = 0, nch = 0;
    int nr = 0;
    Z1_OK_(z1_table_info(t, &numel, &nch, &nr));
    EXPECT(nr == R && numel == sizes[0] + sizes[1] + sizes[2] + sizes[3] + sizes[4]);   /* the empty row counts */

    const float lr = 3e-4f, b1 = 0.9f, b2 = 0.95f, eps = 1e-8f, wd = 0.1f, max_norm = 1.0f;
    const int64_t step = 1000;
    float bc[2];
    oracle_bias_corrections(0.9, 0.95, step, 1, bc);
    Z1_OK_(z1_grad_sumsq(t, dpart, NULL));
    Z1_OK_(z1_norm_clip(dpart, NULL, 1.0f, ds + 0, ds + 1, ds + 2, max_norm, NULL));
    for (int rep = 0; rep < 3; ++rep) {           /* the one-call form: same bits, every call */
        float one[3];
        HIP_OK(hipMemset(ds + 3, 0, 12));
        Z1_OK_(z1_grad_norm_clip(t, dpart, NULL, 1.0f, ds + 3, ds + 4, ds + 5, max_norm, NULL));
        HIP_OK(hipDeviceSynchronize());
        float two[3];
        HIP_OK(hipMemcpy(two, ds, 12, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(one, ds + 3, 12, hipMemcpyDeviceToHost));
        EXPECT(bits(one[0]) == bits(two[0]) && bits(one[1]) == bits(two[1]) && bits(one[2]) == bits(two[2]));
    }
    Z1_OK_(z1_adam_cast(t, ds + 2, lr, b1, b2, eps, bc[0], bc[1], wd, 1, NULL));
    HIP_OK(hipDeviceSynchronize());
    float sc[3];
    HIP_OK(hipMemcpy(sc, ds, 12, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(op, dp, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(om, dm, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(ov, dv, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(o16, d16, total * 2, hipMemcpyDeviceToHost));

    double ss = 0.0;
    for (int i = 0; i < R; ++i) ss += oracle_sumsq_f32(hg + off[i], sizes[i]);
    const double exact = sqrt(ss);
    EXPECT(fabs((double)sc[0] - exact) <= 1e-6 * exact);
    float chain[3];
    oracle_norm_clip((double)sc[0] * (double)sc[0], 1.0f, max_norm, chain);    /* entered at the GPU's norm */
    EXPECT(bits(chain[0]) == bits(sc[0]) && bits(chain[1]) == bits(sc[1]) && bits(chain[2]) == bits(sc[2]));
    EXPECT(sc[2] < 1.0f);                                                      /* the clip is active */
    for (int i = 0; i < R; ++i) {
        const int64_t o = off[i], n = sizes[i];
        oracle_adam_cast(hg + o, 0, hp + o, hm + o, hv + o, h16 + o, n, sc[2], 1, lr, b1, b2, eps, bc[0], bc[1], wd,
                         1);
        EXPECT(same_f32(op + o, hp + o, n) && same_f32(om + o, hm + o, n) && same_f32(ov + o, hv + o, n));
        EXPECT(memcmp(o16 + o, h16 + o, (size_t)n * 2) == 0);
    }
    /* step 1001 from that state on new gradients (bound with z1_table_set_grads; row 3 one element off the vector
     * alignment) as two launches over row ranges up to z1_table_info's row count, the factor 0.75 */
    int64_t off2[R];
    const void* g2[R];
    for (int i = 0; i < R; ++i) {
        off2[i] = off[i] + (i == 3);
        g2[i] = i == 2 ? NULL : (const void*)(dg2 + off2[i]);  /* the empty row's entry is ignored */
    }
    for (int64_t i = 0; i < total; ++i) hg[i] = normal(1e-2);
    for (int i = 0; i < R; ++i)
        if (sizes[i]) HIP_OK(hipMemcpy(dg2 + off2[i], hg + off[i], sizes[i] * 4, hipMemcpyHostToDevice));
    EXPECT(z1_table_set_grads(t, g2, R - 1, NULL) == Z1_E_SIZE);
    Z1_OK_(z1_table_set_grads(t, g2, R, NULL));
    oracle_bias_corrections(0.9, 0.95, step + 1, 1, bc);
    const float f2 = 0.75f;
    HIP_OK(hipMemcpy(ds + 2, &f2, 4, hipMemcpyHostToDevice));
    EXPECT(z1_adam_cast_rows(t, 3, nr + 1, ds + 2, lr, b1, b2, eps, bc[0], bc[1], wd, 1, NULL) == Z1_E_SIZE);
    Z1_OK_(z1_adam_cast_rows(t, 0, 1, ds + 2, lr, b1, b2, eps, bc[0], bc[1], wd, 1, NULL));
    Z1_OK_(z1_adam_cast_rows(t, 1, nr, ds + 2, lr, b1, b2, eps, bc[0], bc[1], wd, 1, NULL));
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(op, dp, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(om, dm, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(ov, dv, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(o16, d16, total * 2, hipMemcpyDeviceToHost));
    for (int i = 0; i < R; ++i) {
        const int64_t o = off[i], n = sizes[i];
        oracle_adam_cast(hg + o, 0, hp + o, hm + o, hv + o, h16 + o, n, f2, 1, lr, b1, b2, eps, bc[0], bc[1], wd, 1);
        EXPECT(same_f32(op + o, hp + o, n) && same_f32(om + o, hm + o, n) && same_f32(ov + o, hv + o, n));
        EXPECT(memcmp(o16 + o, h16 + o, (size_t)n * 2) == 0);
    }
    Z1_OK_(z1_table_destroy(t));
    HIP_OK(hipFree(dg));
    HIP_OK(hipFree(dg2));
    HIP_OK(hipFree(dp));
    HIP_OK(hipFree(dm));
    HIP_OK(hipFree(dv));
    HIP_OK(hipFree(d16));
    HIP_OK(hipFree(ds));
    HIP_OK(hipFree(dpart));
    free(hg); free(hp); free(hm); free(hv); free(op); free(om); free(ov); free(h16); free(o16);
    return 0;
}

static int owner_sum(void) {
    enum { W = 8 };
    const int64_t n = 100003;                    /* odd: a vector body and an element-wise tail */
    uint16_t* hc[W];
    uint16_t* dc[W];
    for (int k = 0; k < W; ++k) {
        hc[k] = malloc(n * 2);
        for (int64_t i = 0; i < n; ++i) hc[k][i] = oracle_bf16_rne(normal(1e-3));
        HIP_OK(hipMalloc((void**)&dc[k], n * 2));
        HIP_OK(hipMemcpy(dc[k], hc[k], n * 2, hipMemcpyHostToDevice));
    }
    const int64_t nws = z1_owner_sum_workspace(n);
    EXPECT(nws >= Z1_NORM_PARTIALS);
    uint16_t *davg, *havg = malloc(n * 2), *eavg = malloc(n * 2);
    float *dsum, *hsum = malloc(n * 4), *esum = malloc(n * 4), *dnr;
    double* dws;
    HIP_OK(hipMalloc((void**)&davg, n * 2));
    HIP_OK(hipMalloc((void**)&dsum, n * 4));
    HIP_OK(hipMalloc((void**)&dws, nws * 8));
    HIP_OK(hipMalloc((void**)&dnr, 4));
    Z1_OK_(z1_owner_sum_bf16((const uint16_t* const*)dc, W, n, 0.125f, davg, dsum, dws, NULL));
    Z1_OK_(z1_norm_clip(dws, NULL, 1.0f, dnr, NULL, NULL, 0.0f, NULL));
    HIP_OK(hipDeviceSynchronize());
    float nrm;
    HIP_OK(hipMemcpy(havg, davg, n * 2, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hsum, dsum, n * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(&nrm, dnr, 4, hipMemcpyDeviceToHost));
    oracle_owner_sum((const uint16_t* const*)hc, W, n, 0.125f, eavg, esum);
    EXPECT(memcmp(havg, eavg, (size_t)n * 2) == 0);
    EXPECT(same_f32(hsum, esum, n));
    const double exact = sqrt(oracle_sumsq_bf16(eavg, n));
    EXPECT(fabs((double)nrm - exact) <= 1e-6 * exact);
    /* the same sum one range at a time (CEReduce's phases: odd bounds, an empty range), each range's per-chunk norm
     * partials side by side in one array and reduced once: average and FP32 sum bit-exact, the norm within 1 fp32
     * ulp of the correctly rounded exact one */
    {
        const int64_t cut[5] = {0, 30001, 30001, 77777, n};
        int64_t m = 0;
        for (int r = 0; r < 4; ++r) {
            const int64_t w = z1_owner_sum_waves(cut[r + 1] - cut[r]);
            EXPECT(w >= 0);
            m += w;
        }
        double* dwv;
        HIP_OK(hipMalloc((void**)&dwv, (size_t)(m > 0 ? m : 1) * 8));
        HIP_OK(hipMemset(davg, 0, n * 2));
        HIP_OK(hipMemset(dsum, 0, n * 4));
        int64_t off = 0;
        for (int r = 0; r < 4; ++r) {
            const int64_t a = cut[r], len = cut[r + 1] - cut[r];
            const uint16_t* src[W];
            for (int k = 0; k < W; ++k) src[k] = dc[k] + a;
            Z1_OK_(z1_owner_sum_bf16_waves(src, W, len, 0.125f, davg + a, dsum + a, dwv + off, NULL));
            off += z1_owner_sum_waves(len);
        }
        EXPECT(off == m);
        Z1_OK_(z1_reduce_waves(dwv, m, dws, NULL));
        Z1_OK_(z1_norm_clip(dws, NULL, 1.0f, dnr, NULL, NULL, 0.0f, NULL));
        HIP_OK(hipDeviceSynchronize());
        float nrm2;
        HIP_OK(hipMemcpy(havg, davg, n * 2, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(hsum, dsum, n * 4, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(&nrm2, dnr, 4, hipMemcpyDeviceToHost));
        EXPECT(memcmp(havg, eavg, (size_t)n * 2) == 0);
        EXPECT(same_f32(hsum, esum, n));
        const int64_t du = (int64_t)bits(nrm2) - (int64_t)bits((float)exact);
        EXPECT(du >= -1 && du <= 1);
        HIP_OK(hipFree(dwv));
    }
    /* z1_owner_sum_update against z1_owner_sum_bf16 + z1_norm_clip: twice on n, then on a shorter input with the
     * same workspace */
    float* dsc;
    HIP_OK(hipMalloc((void**)&dsc, 6 * 4));
    const int64_t lens[3] = {n, n, 4099};
    for (int rep = 0; rep < 3; ++rep) {
        const int64_t m = lens[rep];
        const float fac = rep == 1 ? 3.0f : 0.5f;
        Z1_OK_(z1_owner_sum_bf16((const uint16_t* const*)dc, W, m, 0.125f, davg, NULL, dws, NULL));
        Z1_OK_(z1_norm_clip(dws, NULL, fac, dsc + 0, dsc + 1, dsc + 2, 1.0f, NULL));
        HIP_OK(hipDeviceSynchronize());
        HIP_OK(hipMemcpy(eavg, davg, m * 2, hipMemcpyDeviceToHost));
        HIP_OK(hipMemset(davg, 0, n * 2));
        z1_update_scalars u;
        memset(&u, 0, sizeof(u));
        u.numer = 1.0f;
        u.factor_value = fac;
        u.max_norm = 1.0f;
        u.norm_out = dsc + 3;
        u.grad_norm_out = dsc + 4;
        u.factor_out = dsc + 5;
        Z1_OK_(z1_owner_sum_update((const uint16_t* const*)dc, W, m, 0.125f, davg, NULL, dws, &u, NULL));
        HIP_OK(hipDeviceSynchronize());
        float sc[6];
        HIP_OK(hipMemcpy(sc, dsc, 24, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(havg, davg, m * 2, hipMemcpyDeviceToHost));
        EXPECT(memcmp(havg, eavg, (size_t)m * 2) == 0);
        EXPECT(bits(sc[0]) == bits(sc[3]) && bits(sc[1]) == bits(sc[4]) && bits(sc[2]) == bits(sc[5]));
    }
    HIP_OK(hipFree(dsc));
    for (int k = 0; k < W; ++k) {
        HIP_OK(hipFree(dc[k]));
        free(hc[k]);
    }
    HIP_OK(hipFree(davg));
    HIP_OK(hipFree(dsum));
    HIP_OK(hipFree(dws));
    HIP_OK(hipFree(dnr));
    free(havg); free(eavg); free(hsum); free(esum);
    return 0;
}

static int embedding_grad(int64_t R) {
    const int64_t D = 40, V = 300, pad = 7;
    int64_t* hid = malloc(R * 8);
    uint16_t *hgr = malloc(R * D * 2), *hout = malloc(V * D * 2), *want = malloc(V * D * 2);
    for (int64_t i = 0; i < R; ++i) {
        const double u = unif();
        hid[i] = (int64_t)(u * u * V);           /* skewed: low ids repeat often, id 0 more than 20 times */
        if (i % 97 == 5) hid[i] = (i % 2) ? -3 : V + 11;      /* outside [0, V): ignored */
    }
    for (int64_t i = 0; i < R * D; ++i) hgr[i] = oracle_bf16_rne(normal(1e-2));
    const int64_t ws = z1_embedding_backward_workspace(R, D, V);
    EXPECT(ws > 0);
    int64_t* did;
    uint16_t *dgr, *dout;
    void* dws;
    HIP_OK(hipMalloc((void**)&did, R * 8));
    HIP_OK(hipMalloc((void**)&dgr, R * D * 2));
    HIP_OK(hipMalloc((void**)&dout, V * D * 2));
    HIP_OK(hipMalloc(&dws, (size_t)ws));
    HIP_OK(hipMemcpy(did, hid, R * 8, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dgr, hgr, R * D * 2, hipMemcpyHostToDevice));
    EXPECT(z1_embedding_backward(did, dgr, R, D, V, pad, 0.125f, 2, dout, dws, ws - 1, NULL) == Z1_E_WORKSPACE);
    Z1_OK_(z1_embedding_backward(did, dgr, R, D, V, pad, 0.125f, 2, dout, dws, ws, NULL));
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(hout, dout, V * D * 2, hipMemcpyDeviceToHost));
    if (R > 3072)
        oracle_embedding_backward(hid, hgr, R, D, V, pad, 0.125f, 2, want);
    else
        oracle_embedding_backward_chunked(hid, hgr, R, D, V, pad, 0.125f, 2, 16, want);
    EXPECT(memcmp(hout, want, (size_t)(V * D * 2)) == 0);
    HIP_OK(hipFree(did));
    HIP_OK(hipFree(dgr));
    HIP_OK(hipFree(dout));
    HIP_OK(hipFree(dws));
    free(hid); free(hgr); free(hout); free(want);
    return 0;
}

static int gradient_outputs(void) {
    enum { R = 3 };
    const int64_t sizes[R] = {4096 + 13, 777, 256 * 5};
    const int64_t off[R] = {0, 4160, 4992};                 /* 64-element aligned rows */
    const int64_t total = 4992 + 256 * 5;
    uint16_t *hg = malloc(total * 2), *h16 = malloc(total * 2), *o16 = malloc(total * 2);
    float *hp = malloc(total * 4), *hm = malloc(total * 4), *hv = malloc(total * 4);
    float *op = malloc(total * 4), *om = malloc(total * 4), *ov = malloc(total * 4);
    float *hout = malloc((total + 1) * 4), *oout = malloc((total + 1) * 4), *ref = malloc(total * 4);
    for (int64_t i = 0; i < total; ++i) {
        hg[i] = oracle_bf16_rne(normal(1e-2));
        hp[i] = normal(0.02);
        hm[i] = normal(1e-4);
        hv[i] = fabsf(normal(1e-8));
    }
    for (int64_t i = 0; i <= total; ++i) hout[i] = -7.0f;
    uint16_t *dg, *d16;
    float *dp, *dm, *dv, *dout, *dfac;
    HIP_OK(hipMalloc((void**)&dg, total * 2));
    HIP_OK(hipMalloc((void**)&d16, total * 2));
    HIP_OK(hipMalloc((void**)&dp, total * 4));
    HIP_OK(hipMalloc((void**)&dm, total * 4));
    HIP_OK(hipMalloc((void**)&dv, total * 4));
    HIP_OK(hipMalloc((void**)&dout, (total + 1) * 4));
    HIP_OK(hipMalloc((void**)&dfac, 4));
    HIP_OK(hipMemcpy(dg, hg, total * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dp, hp, total * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dm, hm, total * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dv, hv, total * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dout, hout, (total + 1) * 4, hipMemcpyHostToDevice));
    const float fac = 0.37f;
    HIP_OK(hipMemcpy(dfac, &fac, 4, hipMemcpyHostToDevice));
    z1_tensor rows[R];
    for (int i = 0; i < R; ++i) {
        rows[i].g = dg + off[i];
        rows[i].p = dp + off[i];
        rows[i].m = dm + off[i];
        rows[i].v = dv + off[i];
        rows[i].p16 = d16 + off[i];
        rows[i].n = sizes[i];
    }
    z1_table* t = NULL;
    Z1_OK_(z1_table_create(rows, R, Z1_BF16, &t));
    /* row 0's output one float past its slot (off the 16-byte alignment: element-wise path), row 1 none */
    float* outs[R] = {dout + off[0] + 1, NULL, dout + off[2]};
    EXPECT(z1_table_set_grad_out(t, outs, R - 1, NULL) == Z1_E_SIZE);
    EXPECT(z1_table_set_grad_out(NULL, outs, R, NULL) == Z1_E_NULL);
    Z1_OK_(z1_table_set_grad_out(t, outs, R, NULL));
    const float lr = 3e-4f, b1 = 0.9f, b2 = 0.95f, eps = 1e-8f, wd = 0.1f;
    float bc[2];
    oracle_bias_corrections(0.9, 0.95, 3, 1, bc);
    Z1_OK_(z1_adam_cast(t, dfac, lr, b1, b2, eps, bc[0], bc[1], wd, 1, NULL));
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(op, dp, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(om, dm, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(ov, dv, total * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(o16, d16, total * 2, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(oout, dout, (total + 1) * 4, hipMemcpyDeviceToHost));
    for (int i = 0; i < R; ++i) {
        const int64_t o = off[i], n = sizes[i];
        oracle_adam_cast(hg + o, 1, hp + o, hm + o, hv + o, h16 + o, n, fac, 1, lr, b1, b2, eps, bc[0], bc[1], wd, 1);
        EXPECT(same_f32(op + o, hp + o, n) && same_f32(om + o, hm + o, n) && same_f32(ov + o, hv + o, n));
        EXPECT(memcmp(o16 + o, h16 + o, (size_t)n * 2) == 0);
        oracle_scale_up(hg + o, ref, fac, n);
        if (i == 0) EXPECT(same_f32(oout + o + 1, ref, n));
        if (i == 2) EXPECT(same_f32(oout + o, ref, n));
    }
    for (int64_t i = off[0] + 1 + sizes[0]; i < off[2]; ++i) EXPECT(bits(oout[i]) == bits(-7.0f));   /* row 1 */
    EXPECT(bits(oout[0]) == bits(-7.0f) && bits(oout[total]) == bits(-7.0f));
    Z1_OK_(z1_table_set_grad_out(t, NULL, 0, NULL));        /* outputs removed: the next launch writes none */
    HIP_OK(hipMemcpy(dout, hout, (total + 1) * 4, hipMemcpyHostToDevice));
    Z1_OK_(z1_adam_cast(t, dfac, lr, b1, b2, eps, bc[0], bc[1], wd, 1, NULL));
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(oout, dout, (total + 1) * 4, hipMemcpyDeviceToHost));
    EXPECT(same_f32(oout, hout, total + 1));
    Z1_OK_(z1_table_destroy(t));
    HIP_OK(hipFree(dg));
    HIP_OK(hipFree(d16));
    HIP_OK(hipFree(dp));
    HIP_OK(hipFree(dm));
    HIP_OK(hipFree(dv));
    HIP_OK(hipFree(dout));
    HIP_OK(hipFree(dfac));
    free(hg); free(h16); free(o16); free(hp); free(hm); free(hv); free(op); free(om); free(ov);
    free(hout); free(oout); free(ref);
    return 0;
}

int abi_gpu_run(void) {
    int rc = table_update();
    if (rc == 0) rc = owner_sum();
    if (rc == 0) rc = embedding_grad(5000);
    if (rc == 0) rc = embedding_grad(1000);
    if (rc == 0) rc = gradient_outputs();
    printf("%s\n", rc ? "FAIL" : "ok");
    fflush(stdout);
    return rc;
}

#ifdef ABI_GPU_MAIN
int main(void) { return abi_gpu_run(); }
#endif
