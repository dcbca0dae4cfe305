// yoco_z1: gfx950 kernels + C ABI for the owner-side ZeRO-1 shard update (declarations: include/yoco_z1.h).
//
// Layout and scheduling
//   * Every multi-tensor kernel walks one device-resident table of rows (g, p, m, v, p16, n) cut into chunks of
//     kChunk = 256 elements (one wave64 x one float4 per lane); row r owns the global chunk range
//     [chunk0_r, chunk0_r + ceil(n_r / kChunk)).  A chunk -> row map (one int32 per chunk) follows the rows in
//     the same device allocation, so a wave finds its row with two scalar loads.
//   * Adam + BF16: one wave per chunk, one wave per workgroup, dispatched by the hardware (grid = chunks).
//     Workgroup b takes the b-th chunk from the end, so the hardware's round-robin dispatch over the 8 XCDs
//     interleaves consecutive chunks over all XCDs, and all of them start on the MALL-resident end of the shard
//     (see the MALL note below); a dynamic LDS reservation the kernel does not touch caps it at 12 resident
//     workgroups per CU.  Measured on MI355X (431M-element shard): 1.93 ms, against 2.03 ms at 16 per CU,
//     2.05 ms when each XCD streams one contiguous eighth (its best cap, 16), 2.52 ms for a persistent grid
//     with a static partition (tail imbalance across CUs/XCDs) and 2.19 ms for 1024-element workgroups; the
//     same kernel with its arithmetic replaced by additions ran at the same speed (the divisions and square
//     roots are hidden under the memory traffic).  A launch covers a chunk range: the whole table, or the
//     chunks of a range of rows (z1_adam_cast_rows), so a step can be cut into launches whose finished rows are
//     sent while the rest runs (2 or 4 ranges of C2 cost nothing measurable, 8 cost 13 us).  When the rows tile
//     one allocation per stream (the flat shard), a whole-table launch walks the buffers directly
//     (adam_flat_kernel, 11 resident workgroups per CU): the same chunks' arithmetic without the two scalar
//     lookups that start each wave, 2.175-2.177 against 2.185-2.188 ms per C2 update.
//   * Each lane moves one 128-bit group per fp32 array (and 64 bits of bf16); a wave instruction covers 1 KiB
//     (fp32) or 512 B (bf16) of contiguous bytes, with nontemporal hints (streams far larger than L2 and MALL).
//     The last, partial chunk of a row (and rows whose pointers are not aligned for the vector path) run an
//     element-wise loop.
//   * The norm uses the same table and a FIXED grid of Z1_NORM_PARTIALS workgroups of 4 waves, split by XCD: the
//     256 workgroups dispatched to one XCD stride through that XCD's eighth of the chunks, 1024 contiguous
//     elements per workgroup step.  FP64 accumulation of the exact squares per lane, a wave64 xor-butterfly and
//     a fixed-order LDS stage: its bits do not depend on timing, on the device's CU count or on the run.
//     Measured 0.25 ms for the 1.72 GB gradient (6.8 TB/s); the grid striding over all chunks (0.27 ms), one
//     wave per chunk with hardware dispatch (0.40 ms), 4-chunk workgroups with hardware dispatch (0.34 ms),
//     2-8 loads in flight per wave (0.28-0.31 ms) and fewer waves (0.35-0.59 ms) were all slower.
//   * MALL reuse between passes: the norm pass reads the last 256 MB of the gradient with ordinary, allocating
//     loads, and Adam walks the chunks from the last one, so its first gradient reads hit the 256 MB MALL
//     (measured 2.05 vs 2.10 ms for Adam on the C2 shard; 128-512 MB kept, or everything, measured the same or
//     slower).
//   * No atomics anywhere; nothing but vector memory instructions write memory.  (The norm's final reduction is a
//     second, one-workgroup launch: folding it into the last workgroup of the norm grid to finish, with an arrival
//     counter, measured 75 us slower per step, because the grid's 2048 workgroups finish together.)
//
// Numerics follow the header: one rounding per fp32 operation, explicit FMAs where the reference has them,
// correctly rounded division and square root (built with -fhip-fp32-correctly-rounded-divide-sqrt, no fast math,
// fp32 denormals kept, no contraction).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <mutex>
#include <new>
#include <vector>

#include "yoco_z1.h"
#include "z1_internal.h"

#pragma clang fp contract(off)

namespace {

// Launch geometry (the measured choices on MI355X; alternatives and their timings are recorded with the design):
constexpr int kWave = 64;
constexpr int kThreads = 256;                                 // FP32 norm and one-workgroup reduction workgroups
constexpr int kAdamWaves = 1;                                 // chunks (one per wave) per Adam workgroup
constexpr int kVec = 4;                                       // fp32 lanes of one 128-bit access
constexpr int kGroups = 1;                                    // 128-bit groups per lane per array and chunk
constexpr int64_t kChunk = (int64_t)kWave * kVec * kGroups;   // elements per chunk: one wave's share
// The norm pass reads the last kMallKeepBytes of the gradient with ordinary, allocating loads, so that they are
// still in the 256 MB MALL when the Adam pass -- which walks the chunks from the end -- reads them again (C2 Adam
// 2.05 against 2.10 ms; 192-272 MB no better).  The owner sum keeps nothing: storing the average's last 224 MB with
// allocating stores for Adam to read back gained nothing (C3 3.048 ms either way; the drop-in step 3.349 ms with
// it, 3.334 ms without).
constexpr int64_t kMallKeepBytes = 256ll << 20;
constexpr int kAdamWgPerCu = 12;                              // resident Adam workgroups per CU (occupancy_lds)
constexpr int kAdamGoutWgPerCu = 11;                          // the same, with FP32 gradient outputs (5 write streams)
constexpr int kAdamFlatWgPerCu = 11;                          // the same, over contiguous flat buffers
constexpr int kOwnerSumWgPerCu = 16;                          // resident owner-sum workgroups per CU
constexpr int kMaxDevices = 64;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Device copy of one table row plus its schedule.  64 bytes: one scalar load brings a whole row.
struct Row {
    const void* g;
    float* p;
    float* m;
    float* v;
    uint16_t* p16;
    int64_t n;
    int64_t chunk0;
    int32_t vec;        // bit 0: g aligned for the vector path; bit 1: p, m, v, p16 aligned as well
    int32_t pmv_aligned;    // p, m, v, p16 aligned for the vector path (vec's bit 1 needs g aligned too)
};
static_assert(sizeof(Row) == 64, "row layout");

enum { kVecG = 1, kVecAll = 2 };

struct AdamK {
    float lr, b1, b2, eps, bc1, bc2, wd, omb1, omb2;
};

// Streams go through the global address space (global_load/global_store, not flat): the pointers come out of a
// table in memory, so the compiler cannot infer the address space by itself.  The big streams carry nontemporal
// hints: they are far larger than L2 and the MALL and are touched once (measured: 2.43 vs 2.10 ms without them).
// The update's big stores go out through st_stream below, which adds the system-scope bits.
#define Z1_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ T ld(const T* p) {
    return __builtin_nontemporal_load((const Z1_GLOBAL T*)p);
}

template <typename T>
__device__ __forceinline__ T ld_keep(const T* p) {       // ordinary load: allocates in L2 and the MALL
    return *(const Z1_GLOBAL T*)p;
}

template <typename T>
__device__ __forceinline__ void st(T* p, T x) {
    __builtin_nontemporal_store(x, (Z1_GLOBAL T*)p);
}

// The update's streaming stores (Adam's p, m, v, BF16 copy and FP32 gradient outputs; the owner sum's average; the
// scale and cast passes) go out as buffer stores whose cache-policy bits mark them system scope as well as
// nontemporal (sc0 sc1 nt; gfx950's store bits: sc0 = 1, nt = 2, sc1 = 16), which the L2 writes through at once
// rather than keeping dirty lines for a later write-back.  Measured against the nontemporal global stores above,
// interleaved on one box: C2 update 2.179 against 2.197-2.228 ms, C3 2.995-3.002 against 3.051-3.053 ms, the drop-in
// step 3.268-3.282 against 3.325-3.329 ms, the scale pass over 430M elements 0.403 against 0.410 ms.  The same stores
// with nt alone, through a buffer, measured like the global ones; the loads marked the same way were slower (C3
// 3.27 ms), and so were the embedding gradient's row stores, which keep nt.  The descriptor covers one wave's chunk
// (word 3 = 0x00020000: the raw 32-bit data format of gfx9 buffer resources), so the offset is the lane's byte offset
// within it.
constexpr int kStreamStorePolicy = 1 | 2 | 16;
__device__ __forceinline__ void st_stream(float* base, int bytes, int off, f4 x) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, x), r, off, 0, kStreamStorePolicy);
}
__device__ __forceinline__ void st_stream(uint16_t* base, int bytes, int off, u2 x) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b64(x, r, off, 0, kStreamStorePolicy);
}

// Chunk of workgroup b: undoes the round-robin dispatch over the 8 XCDs (workgroup b runs on XCD b mod 8), so that
// each XCD streams one contiguous eighth of the chunks.  Used by the scale and cast passes; Adam and the owner sum
// measured faster with the plain b -> b map (consecutive chunks interleaved over the XCDs: C2 update 2.283 vs
// 2.306 ms, C3 3.153 vs 3.225 ms, interleaved A/B runs on one box).
__device__ __forceinline__ int64_t chunk_of_block(int64_t b, int64_t nb) {
    const int64_t x = b & 7, q = b >> 3, Q = nb >> 3, R = nb & 7;
    return x * Q + (x < R ? x : R) + q;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round to nearest even; NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    return ((u & 0x7fffffffu) > 0x7f800000u) ? 0x7fc0u : r;
}

typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

// Two floats -> two bf16 (round to nearest even) with gfx950's packed conversion; matches f32_to_bf16 on every
// non-NaN input, subnormals included (checked against the CPU oracle).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    const bf2 h = __builtin_convertvector(f2{lo, hi}, bf2);
    return __builtin_bit_cast(uint32_t, h);
}

template <int MODE>
__device__ __forceinline__ void adam_elem(float g, float& p, float& m, float& v, const AdamK& k) {
    if (MODE == 0) g = __builtin_fmaf(k.wd, p, g);
    m = __builtin_fmaf(k.b1, m, k.omb1 * g);
    const float t = k.omb2 * g;
    v = __builtin_fmaf(k.b2, v, t * g);
    const float mh = m / k.bc1;
    const float vh = v / k.bc2;
    const float den = __builtin_sqrtf(vh) + k.eps;
    float upd = mh / den;
    if (MODE == 1) upd = __builtin_fmaf(k.wd, p, upd);
    p = __builtin_fmaf(-k.lr, upd, p);
}

// ------------------------------------------------------------------------------------------------ Adam + BF16
template <int GDT>
__device__ __forceinline__ f4 load_g4(const void* g, int64_t i) {
    if (GDT == Z1_F32) return ld(reinterpret_cast<const f4*>(static_cast<const float*>(g) + i));
    const u2 h = ld(reinterpret_cast<const u2*>(static_cast<const uint16_t*>(g) + i));
    return f4{bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y)};
}

template <int GDT>
__device__ __forceinline__ f4 load_g4_keep(const void* g, int64_t i) {
    if (GDT == Z1_F32) return ld_keep(reinterpret_cast<const f4*>(static_cast<const float*>(g) + i));
    const u2 h = ld_keep(reinterpret_cast<const u2*>(static_cast<const uint16_t*>(g) + i));
    return f4{bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y)};
}

template <int GDT>
__device__ __forceinline__ float load_g1(const void* g, int64_t i) {
    if (GDT == Z1_F32) return static_cast<const float*>(g)[i];
    return bf16_to_f32(static_cast<const uint16_t*>(g)[i]);
}

// GOUT: the table carries FP32 gradient outputs (z1_table_set_grad_out): each row's g' = fp32(g * factor), the value
// the update consumes, is also stored to gout[row] (NULL: not for that row) -- the FP32 gradient the reference's
// scale pass writes before its Adam reads it back (yoco/tasks/zero1_fast.py:175-192, fused_adam_cast.py:75-89).
// One chunk of a row: elements [base, base + min(r.n - base, kChunk)) of r; the vector path when the chunk is whole
// and the row's pointers are aligned, else an element-wise loop.
template <int GDT, int MODE, bool GOUT>
__device__ __forceinline__ void adam_chunk(const Row& r, float* go, int64_t base, int lane, float f, const AdamK& k) {
    const int64_t rem = r.n - base;
    if (rem >= kChunk && (r.vec & kVecAll) && (!GOUT || (reinterpret_cast<uintptr_t>(go) & 15) == 0)) {
        f4 g[kGroups], p[kGroups], m[kGroups], v[kGroups];
#pragma unroll
        for (int u = 0; u < kGroups; ++u) {
            const int64_t i = base + (int64_t)(u * kWave + lane) * kVec;
            g[u] = load_g4<GDT>(r.g, i);
            p[u] = ld(reinterpret_cast<const f4*>(r.p + i));
            m[u] = ld(reinterpret_cast<const f4*>(r.m + i));
            v[u] = ld(reinterpret_cast<const f4*>(r.v + i));
        }
#pragma unroll
        for (int u = 0; u < kGroups; ++u) {
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                float pj = p[u][j], mj = m[u][j], vj = v[u][j];
                g[u][j] = g[u][j] * f;
                adam_elem<MODE>(g[u][j], pj, mj, vj, k);
                p[u][j] = pj;
                m[u][j] = mj;
                v[u][j] = vj;
            }
        }
#pragma unroll
        for (int u = 0; u < kGroups; ++u) {
            // lane offsets within the chunk [base, base + kChunk) of each stream
            const int o4 = (u * kWave + lane) * kVec * 4, o2 = (u * kWave + lane) * kVec * 2;
            st_stream(r.p + base, (int)kChunk * 4, o4, p[u]);
            st_stream(r.m + base, (int)kChunk * 4, o4, m[u]);
            st_stream(r.v + base, (int)kChunk * 4, o4, v[u]);
            if (r.p16) {
                const u2 h = u2{pack_bf16(p[u][0], p[u][1]), pack_bf16(p[u][2], p[u][3])};
                st_stream(r.p16 + base, (int)kChunk * 2, o2, h);
            }
            if (GOUT && go) st_stream(go + base, (int)kChunk * 4, o4, g[u]);
        }
    } else {
        const int64_t cnt = rem < kChunk ? rem : kChunk;
        for (int64_t i = base + lane; i < base + cnt; i += kWave) {
            float pj = r.p[i], mj = r.m[i], vj = r.v[i];
            const float gj = load_g1<GDT>(r.g, i) * f;
            if (GOUT && go) go[i] = gj;
            adam_elem<MODE>(gj, pj, mj, vj, k);
            r.p[i] = pj;
            r.m[i] = mj;
            r.v[i] = vj;
            if (r.p16) r.p16[i] = (uint16_t)f32_to_bf16(pj);
        }
    }
}

// A wave of adam_cast_kernel finds its chunk's row by a binary search over the rows' first chunks when the table
// has at most kSearchRows rows (their 64-byte entries stay in the scalar cache: a few cache hits), else from the
// chunk -> row map (one load that mostly misses the scalar cache, then the row).  Measured with 38 rows: C2's 38
// tensors as separate allocations 1.961-1.981 against 1.981-1.989 ms (FP32 gradients), 2.100-2.116 against
// 2.115-2.123 ms (BF16 gradients in, FP32 gradients out); the flat C2 shard walked as a table 1.906-1.915 against
// 1.956-1.974 ms.  A rank's shard holds 9 to 40 tensors.
constexpr int kSearchRows = 64;

template <int GDT, int MODE, bool GOUT>
__global__ __launch_bounds__(kWave * kAdamWaves) void adam_cast_kernel(const Row* __restrict__ rows,
                                                                       const int32_t* __restrict__ chunk_row,
                                                                       int nrows, int64_t chunk_begin, int64_t chunk_end,
                                                                       const float* __restrict__ factor,
                                                                       const float* __restrict__ bc, AdamK k,
                                                                       float* const* __restrict__ gout) {
    const int lane = threadIdx.x & (kWave - 1);
    // chunks [chunk_begin, chunk_end), last chunk first: the end of the gradient is what the pass before left in
    // the MALL.  Consecutive workgroups take consecutive chunks and land on consecutive XCDs.
    const int64_t c = chunk_end - 1 - ((int64_t)blockIdx.x * kAdamWaves +
                                       __builtin_amdgcn_readfirstlane(threadIdx.x / kWave));
    if (c < chunk_begin) return;
    const float f = factor ? *factor : 1.0f;
    if (bc) {                                   // bias corrections from device memory (z1_adam_cast_dev)
        k.bc1 = bc[0];
        k.bc2 = bc[1];
    }
    int32_t ri;
    if (nrows <= kSearchRows) {                 // the last row whose first chunk is <= c
        int lo = 0, hi = nrows - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (rows[mid].chunk0 <= c) lo = mid;
            else hi = mid - 1;
        }
        ri = lo;
    } else {
        ri = chunk_row[c];
    }
    const Row r = rows[ri];
    adam_chunk<GDT, MODE, GOUT>(r, GOUT ? gout[ri] : nullptr, (c - r.chunk0) * kChunk, lane, f, k);
}

// The same update when the table's rows tile one allocation per stream in order, without gaps (the flat shard:
// z1_table marks it contiguous): Adam is element by element, so chunk c of the launch is elements
// [c * kChunk, (c + 1) * kChunk) of the buffers of `w` (the first row's pointers, n = all elements), found without
// the two scalar lookups (chunk -> row map, then the row) that start each wave of adam_cast_kernel.  Last chunk
// first, as there.
template <int GDT, int MODE>
__global__ __launch_bounds__(kWave) void adam_flat_kernel(Row w, int64_t nchunks, const float* __restrict__ factor,
                                                          const float* __restrict__ bc, AdamK k) {
    const int lane = threadIdx.x;
    const int64_t c = nchunks - 1 - (int64_t)blockIdx.x;
    const float f = factor ? *factor : 1.0f;
    if (bc) {
        k.bc1 = bc[0];
        k.bc2 = bc[1];
    }
    adam_chunk<GDT, MODE, false>(w, nullptr, c * kChunk, lane, f, k);
}

// -------------------------------------------------------------------------------------- deterministic norm
// Sum over a workgroup of NT threads, result valid in thread 0: xor butterfly inside each wave64 (a + b == b + a
// exactly, so every lane ends with the same bits), then the wave sums in wave order.
template <int NT = kThreads>
__device__ __forceinline__ double block_sum(double x, double* lds) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = x;
    __syncthreads();
    double s = 0.0;
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 0; w < NT / kWave; ++w) s += lds[w];
    }
    return s;
}

__device__ __forceinline__ double sq64(float x) {
    const double d = (double)x;
    return d * d;                      // exact: 24-bit significand squared
}

// acc + sq64(x) as one fused multiply-add: the square is exact in FP64, so the rounding is the same, in one
// instruction instead of two.  Used where a wave adds a few squares and retires (the owner sum's per-chunk partial:
// C3-shape drop-in update 3.33 against 3.37 ms); the norm pass's long accumulation loop keeps sq64 (its FMA chain
// measured 8 us slower on C2).
__device__ __forceinline__ double add_sq(double acc, float x) {
    const double d = (double)x;
    return __builtin_fma(d, d, acc);
}

// zero1_fast.py:150-160 scalar chain, one owner.
__device__ __forceinline__ void clip_chain(float norm, float fac, float* grad_norm_out, float* factor_out,
                                           float max_norm) {
    const float gn = fac * norm;
    if (grad_norm_out) *grad_norm_out = gn;
    float f = fac;
    if (max_norm > 0.0f) {
        const float t = gn + 1e-6f;
        float coef = (1.0f / t) * max_norm;
        coef = (coef > 1.0f) ? 1.0f : coef;           // clamp(max=1), NaN stays NaN
        f = fac * coef;
    }
    if (factor_out) *factor_out = f;
}

// The Z1_NORM_PARTIALS partials summed in one fixed order (strided per thread, then the workgroup tree); the total
// is valid in thread 0.  Every final reduction of the norm goes through here, so its bits do not depend on which
// kernel runs it.
__device__ __forceinline__ double final_sum(const double* partials, double* lds) {
    double s = 0.0;
    for (int i = threadIdx.x; i < Z1_NORM_PARTIALS; i += kThreads) s += partials[i];
    return block_sum(s, lds);
}

// Thread 0, given the exact sum of squares: the norm / clip chain of zero1_fast.py:150-160, preceded, for the
// trainer's form, by the sample-size factor of trainer_nosync.py:273-279 and followed by the deferred-check flags
// and the "clip" metric (:284-286, :194-197).  With u.sample_size, u.flags_out and u.clip_log_out all NULL this is
// exactly the z1_norm_clip chain.
__device__ __forceinline__ void scalar_tail(double tot, const z1_update_scalars& u) {
    float fac = u.factor_in ? *u.factor_in : u.factor_value;
    if (u.sample_size) {
        // multiply_grads(numer / where(ss > 0, ss, 1)): `int / tensor` is reciprocal(tensor) * int in torch
        const float ss = *u.sample_size;
        const float denom = (ss > 0.0f) ? ss : 1.0f;
        const float c = (1.0f / denom) * u.numer;
        fac = c * fac;
    }
    const float nr = (float)__builtin_sqrt(tot);      // the fp32 norm clip_grad_norm_ returns
    const float sq = nr * nr;                          // .float() ** 2 (all_reduce over one owner: identity)
    const float norm = __builtin_sqrtf(sq);
    if (u.norm_out) *u.norm_out = nr;
    const float gn = fac * norm;
    clip_chain(norm, fac, u.grad_norm_out, u.factor_out, u.max_norm);
    if (u.flags_out) {
        const uint32_t b = __float_as_uint(gn) & 0x7fffffffu;
        u.flags_out[0] = b < 0x7f800000u ? 1 : 0;       // isfinite(grad_norm)
        u.flags_out[1] = 1;                               // one owner: consistent with itself
    }
    if (u.clip_log_out && u.max_norm > 0.0f) *u.clip_log_out = gn > u.max_norm ? 100.0f : 0.0f;
}

// One workgroup: the final reduction and the scalar tail (z1_norm_clip, z1_update_scalars_run).
__global__ __launch_bounds__(kThreads) void scalars_kernel(const double* __restrict__ partials, z1_update_scalars u) {
    __shared__ double lds[kThreads / kWave];
    const double tot = final_sum(partials, lds);
    if (threadIdx.x == 0) scalar_tail(tot, u);
}

// Last row whose first chunk is <= c, searching forward from row t (c only grows within a wave).  The rows table
// is a few KiB and stays in the scalar cache; the chunk -> row map is not read here (it would add ~3% traffic).
__device__ __forceinline__ int advance_row(const Row* __restrict__ rows, int nrows, int t, int64_t c) {
    if (t + 1 >= nrows || rows[t + 1].chunk0 > c) return t;
    int lo = t + 1, hi = nrows - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (rows[mid].chunk0 <= c) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Exact squares of chunk c (row r) added to acc; KEEP selects ordinary loads instead of nontemporal ones.
static_assert(kGroups == 1, "sumsq_chunk reads one 128-bit group per lane");
static_assert(Z1_NORM_PARTIALS % 8 == 0, "the norm grid is split evenly over the 8 XCDs");
template <int GDT, bool KEEP>
__device__ __forceinline__ void sumsq_chunk(const Row& r, int64_t c, int lane, double& acc) {
    const int64_t base = (c - r.chunk0) * kChunk;
    const int64_t rem = r.n - base;
    if (rem >= kChunk && (r.vec & kVecG)) {
        const int64_t i = base + (int64_t)lane * kVec;
        const f4 x = KEEP ? load_g4_keep<GDT>(r.g, i) : load_g4<GDT>(r.g, i);
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc += sq64(x[e]);
    } else {
        const int64_t cnt = rem < kChunk ? rem : kChunk;
        for (int64_t i = base + lane; i < base + cnt; i += kWave) acc += sq64(load_g1<GDT>(r.g, i));
    }
}

// The chunks of one wave below `end` into acc, in order.  FP32: chunks c, c + step, c + 2 step, ... (one 128-bit
// group per lane each).  BF16: runs of kSumsqBf16Span adjacent chunks starting at c, c + step, ...: a run inside one
// row, whole and 16-byte aligned, is kSumsqBf16Span / 2 128-bit loads per lane (8 elements each: the run's
// lane-major order, one 1 KB load of the wave after the other); other runs are their chunks one after the other.
// A BF16 chunk alone gives a wave 512 bytes per load, and the per-chunk latency then bounds the pass (188 us on
// C2's size, 4.6 TB/s, even with two chunks' loads in flight); runs of 2, 4, 8 and 16 chunks measured 143, 135,
// 136 and 143 us.  Either way the order is fixed, so the partials are deterministic.
constexpr int kSumsqBf16Span = 4;
constexpr int kSumsqBf16Threads = 128;                       // 2 waves per norm workgroup for BF16
// r is row t, held in registers until a chunk at or past next0 (row t + 1's first chunk) needs the next row.
template <int GDT, bool KEEP>
__device__ __forceinline__ void sumsq_range(const Row* __restrict__ rows, int nrows, int& t, Row& r, int64_t& next0,
                                            int64_t& c, int64_t end, int64_t step, int lane, double& acc) {
    for (; c < end; c += step) {
        if (c >= next0) {
            t = advance_row(rows, nrows, t, c);
            r = rows[t];
            next0 = t + 1 < nrows ? rows[t + 1].chunk0 : INT64_MAX;
        }
        if (GDT == Z1_BF16) {
            constexpr int S = kSumsqBf16Span, L = kSumsqBf16Span / 2;
            const uint16_t* g = static_cast<const uint16_t*>(r.g) + (c - r.chunk0) * kChunk;
            const bool wide = c + (S - 1) < end && r.n - (c - r.chunk0) * kChunk >= S * kChunk && (r.vec & kVecG) &&
                              (reinterpret_cast<uintptr_t>(g) & 15) == 0;
            if (wide) {
                const u4* q = reinterpret_cast<const u4*>(g) + lane;
                u4 h[L];
#pragma unroll
                for (int u = 0; u < L; ++u) h[u] = KEEP ? ld_keep(q + u * kWave) : ld(q + u * kWave);
#pragma unroll
                for (int u = 0; u < L; ++u) {
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        acc += sq64(bf16_lo(h[u][w]));
                        acc += sq64(bf16_hi(h[u][w]));
                    }
                }
                continue;
            }
            sumsq_chunk<GDT, KEEP>(r, c, lane, acc);
            for (int64_t e = c + 1; e < c + S && e < end; ++e) {
                t = advance_row(rows, nrows, t, e);
                sumsq_chunk<GDT, KEEP>(rows[t], e, lane, acc);
            }
            continue;
        }
        sumsq_chunk<GDT, KEEP>(r, c, lane, acc);
    }
}

// Fixed grid of Z1_NORM_PARTIALS workgroups (a multiple of 8) of NT threads: the 256 workgroups b with b & 7 == x
// cover eighth x of the chunks, wave w of workgroup j taking the runs of `span` chunks that start at
// lo_x + span (j W + w), then every span x 256 W chunks on (W = NT / 64 waves per workgroup; FP32: span 1, W 4,
// 1024 contiguous elements per workgroup step; BF16: span kSumsqBf16Span, W 2, 2048).  Each lane adds its exact
// squares in that fixed order.  Either way one step of an XCD's workgroups spans 1 MB of its eighth (4 waves per
// workgroup for BF16, a 2 MB window, measured 1-3 % slower: 125.1 against 124.4 us back to back over C2's 38
// tensors, 136 against 133.5 us right after the owner sum that wrote them).
// Chunks [keep_from, nchunks) are read with ordinary loads (two loops, so that the two kinds of load stay apart):
// they are where the Adam pass starts (adam_cast_kernel walks the chunks from the last one down), so its first
// gradient reads hit the MALL.
// Each wave's first row comes from the rows' first chunks staged in LDS (tables of up to kSumsqLdsRows rows): one
// load instead of a binary search of dependent scalar loads at the start of every wave.
constexpr int kSumsqLdsRows = 512;
template <int GDT, int NT>
__global__ __launch_bounds__(NT) void sumsq_kernel(const Row* __restrict__ rows, int nrows, int64_t nchunks,
                                                   int64_t keep_from, double* __restrict__ partials) {
    constexpr int W = NT / kWave;
    __shared__ double lds[W];
    __shared__ int64_t first[kSumsqLdsRows];
    const int lane = threadIdx.x & (kWave - 1);
    // workgroup b strides through eighth (b & 7) of the chunks only: the eighth the XCD it is dispatched to
    // (b mod 8) owns, as in chunk_of_block (0.257 vs 0.268 ms on C2, 2.11 vs 2.34 ms on C4 for the whole grid
    // striding over every chunk).  The decomposition depends on b alone, so the partials stay deterministic.
    const int64_t x = blockIdx.x & 7, j = blockIdx.x >> 3;
    const int64_t Q = nchunks >> 3, R = nchunks & 7;
    const int64_t lo = x * Q + (x < R ? x : R), hi = lo + Q + (x < R ? 1 : 0);
    const int64_t nw = (int64_t)(gridDim.x >> 3) * W;
    const int64_t span = GDT == Z1_BF16 ? kSumsqBf16Span : 1;   // chunks a wave takes per step
    const int64_t w0 = lo + span * (j * W + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave));
    int64_t split = keep_from > lo ? (keep_from < hi ? keep_from : hi) : lo;
    split = lo + (split - lo + span - 1) / span * span;   // on the run grid: no run straddles the two loops
    int t = 0;
    if (nrows > 1 && nrows <= kSumsqLdsRows) {            // uniform over the workgroup (kernel arguments)
        for (int i = threadIdx.x; i < nrows; i += NT) first[i] = rows[i].chunk0;
        __syncthreads();
        int a = 0, z = nrows - 1;                         // the last row whose first chunk is <= w0
        while (a < z) {
            const int mid = (a + z + 1) >> 1;
            if (first[mid] <= w0) a = mid;
            else z = mid - 1;
        }
        t = __builtin_amdgcn_readfirstlane(a);
    }
    Row r = {};
    int64_t next0 = 0;                                    // the first chunk loads row t (advance_row from t)
    double acc = 0.0;
    int64_t c = w0;
    sumsq_range<GDT, false>(rows, nrows, t, r, next0, c, split < hi ? split : hi, span * nw, lane, acc);
    sumsq_range<GDT, true>(rows, nrows, t, r, next0, c, hi, span * nw, lane, acc);
    const double s = block_sum<NT>(acc, lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

// The step counter and bias corrections on the device (z1_bias_corrections_step): ++*step; bc = fp32(1 - beta^step)
// computed in double, as yoco/tasks/fused_adam_cast.py:58-60 computes them on the host.
__global__ void bias_step_kernel(int64_t* step, double beta1, double beta2, int bias_correction, float* bc) {
    if (threadIdx.x != 0) return;
    const int64_t s = *step + 1;
    *step = s;
    if (bias_correction == 1) {
        bc[0] = (float)(1.0 - pow(beta1, (double)s));
        bc[1] = (float)(1.0 - pow(beta2, (double)s));
    } else {
        bc[0] = 1.0f;
        bc[1] = 1.0f;
    }
}

__global__ void clip_factor_kernel(const float* __restrict__ norm, const float* factor_in, float factor_value,
                                   float* grad_norm_out, float* factor_out, float max_norm) {
    if (threadIdx.x == 0) clip_chain(*norm, factor_in ? *factor_in : factor_value, grad_norm_out, factor_out, max_norm);
}

// ---------------------------------------------------------------------------------------------- owner sum
struct Srcs {
    const uint16_t* p[Z1_MAX_WORLD];
};

// Owner sum: one wave per chunk of kSumChunk = 256 elements (4 per lane, 8 B per contribution), workgroup b on
// chunk b, dispatched by the hardware round-robin over the XCDs, at most 16 resident workgroups per CU.  Measured
// at C3's size (8 contributions of 430,662,912 elements, throw-away probe of the same kernel): 1.201-1.204 ms at
// 16-20 per CU against 1.221-1.234 ms for 512-element chunks with 16 B per lane at their best caps (10-12),
// 1.38-1.41 ms for 128-element chunks (4 B per lane, 24-40 per CU); this 8-read / 1-write pattern ran at 6.0 TB/s
// with each XCD on one contiguous eighth and 4.5 TB/s for a static grid-stride partition.  W is a compile-time
// constant so that all W loads of a lane are in flight together (a runtime count makes the compiler wait on each
// load before issuing the next).  OUT may alias one source: every element is read before the same lane writes it.
// With wave_partials, lane 0 of each wave writes the FP64 sum of squares of its chunk's rounded averages to a slot
// of its own (a fixed decomposition; the partials are then reduced in a fixed order by reduce_partials_kernel).
// The slot is chunk_of_block of the workgroup, which places the partials of the workgroups one XCD runs next to
// each other, so that XCD's L2 writes them back as whole lines (in chunk order, each partial left its L2 as a
// write request of its own: 54 MB of 32-byte requests at C3's size).
constexpr int kSumVec = 4;                                    // elements per lane and chunk
constexpr int64_t kSumChunk = (int64_t)kWave * kSumVec;
// The chunk grid is shifted by `shift` elements (0..kSumShiftMax): chunk c covers elements [c * kSumChunk - shift,
// (c + 1) * kSumChunk - shift) of the call's range.  The host picks the shift that puts the chunk boundaries on
// 128-byte lines of every stream (else on their 8-byte words), so a range that starts anywhere -- a CEReduce phase
// bound, yoco/models/decoder/ce_reduce.py:178-183 -- keeps the vector path, and no line is shared by two chunks
// (consecutive chunks run on different XCDs, whose L2s would each fetch a shared line).  A call always launches
// owner_sum_waves(n) chunks, enough for any shift; those past the end only write a zero partial.
constexpr int64_t kSumShiftMax = 63;

__device__ __host__ constexpr int64_t owner_sum_waves(int64_t n) {
    return n <= 0 ? 0 : (n + kSumShiftMax + kSumChunk - 1) / kSumChunk;
}

template <int W>
__global__ __launch_bounds__(kWave) void owner_sum_kernel(Srcs s, int64_t n, float scale, uint16_t* out,
                                                          float* out_sum, double* wave_partials, int vec,
                                                          int64_t shift) {
    const int64_t c = (int64_t)blockIdx.x;
    const int64_t e0 = c * kSumChunk + (int64_t)threadIdx.x * kSumVec - shift;
    double acc2 = 0.0;
    if (vec && e0 >= 0 && e0 + kSumVec <= n) {
        u2 x[W];
#pragma unroll
        for (int k = 0; k < W; ++k) x[k] = ld(reinterpret_cast<const u2*>(s.p[k] + e0));
        float a[kSumVec];
#pragma unroll
        for (int j = 0; j < kSumVec; ++j) a[j] = 0.0f;
#pragma unroll
        for (int k = 0; k < W; ++k) {
#pragma unroll
            for (int w = 0; w < kSumVec / 2; ++w) {
                a[2 * w] = a[2 * w] + bf16_lo(x[k][w]);
                a[2 * w + 1] = a[2 * w + 1] + bf16_hi(x[k][w]);
            }
        }
        u2 o;
#pragma unroll
        for (int w = 0; w < kSumVec / 2; ++w) o[w] = pack_bf16(a[2 * w] * scale, a[2 * w + 1] * scale);
        // the chunk's first element (the range's, for a first chunk the shift moves before it): every lane of this
        // path writes [e0, e0 + 4) within [cb, cb + kSumChunk)
        const int64_t cb = c * kSumChunk - shift > 0 ? c * kSumChunk - shift : 0;
        st_stream(out + cb, (int)kSumChunk * 2, (int)(e0 - cb) * 2, o);
        if (out_sum) st_stream(out_sum + cb, (int)kSumChunk * 4, (int)(e0 - cb) * 4, f4{a[0], a[1], a[2], a[3]});
        if (wave_partials) {
#pragma unroll
            for (int w = 0; w < kSumVec / 2; ++w) {
                acc2 = add_sq(acc2, bf16_lo(o[w]));
                acc2 = add_sq(acc2, bf16_hi(o[w]));
            }
        }
    } else {
        const int64_t b = e0 > 0 ? e0 : 0;
        const int64_t e1 = e0 + kSumVec < n ? e0 + kSumVec : n;
        for (int64_t e = b; e < e1; ++e) {
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < W; ++k) a = a + bf16_to_f32(s.p[k][e]);
            const uint32_t o = f32_to_bf16(a * scale);
            out[e] = (uint16_t)o;
            if (out_sum) out_sum[e] = a;
            acc2 = add_sq(acc2, bf16_to_f32((uint16_t)o));
        }
    }
    if (wave_partials) {
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) acc2 += __shfl_xor(acc2, off, kWave);
        if (threadIdx.x == 0) wave_partials[chunk_of_block(blockIdx.x, gridDim.x)] = acc2;
    }
}

// Fixed-order reduction of m per-wave partials into Z1_NORM_PARTIALS: workgroup b sums the contiguous slice
// [b*per, (b+1)*per) (lane-strided, then the fixed workgroup tree).
__global__ __launch_bounds__(kThreads) void reduce_partials_kernel(const double* __restrict__ in, int64_t m,
                                                                   double* __restrict__ out) {
    __shared__ double lds[kThreads / kWave];
    const int64_t per = (m + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per;
    const int64_t hi = lo + per < m ? lo + per : m;
    double acc = 0.0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) acc += in[i];
    const double t = block_sum(acc, lds);
    if (threadIdx.x == 0) out[blockIdx.x] = t;
}

// One launch over every chunk, with the kernel instantiated for the call's contribution count.
template <int W>
void launch_owner_sum(int world, int64_t nchunks, size_t lds, hipStream_t st, const Srcs& s, int64_t n, float scale,
                      uint16_t* out, float* out_sum, double* wave_partials, int vec, int64_t shift) {
    if (world == W) {
        hipLaunchKernelGGL((owner_sum_kernel<W>), dim3((unsigned)nchunks), dim3(kWave), lds, st, s, n, scale, out,
                           out_sum, wave_partials, vec, shift);
    } else if constexpr (W > 1) {
        launch_owner_sum<W - 1>(world, nchunks, lds, st, s, n, scale, out, out_sum, wave_partials, vec, shift);
    }
}

// ------------------------------------------------------------------------------------------ gradient rebinding
// New gradient addresses for up to kBindPerLaunch rows of a table (z1_table_set_grads), passed by value in the
// kernel arguments, so rebinding is stream-ordered and needs neither an allocation nor a host synchronisation.
constexpr int kBindPerLaunch = 128;
struct GradBind {
    const void* g[kBindPerLaunch];
    int32_t row[kBindPerLaunch];
    int32_t count;
    int32_t g_align;
};

__global__ __launch_bounds__(kBindPerLaunch) void set_grads_kernel(Row* rows, GradBind b) {
    const int i = threadIdx.x;
    if (i >= b.count) return;
    Row* r = rows + b.row[i];
    const bool ga = (reinterpret_cast<uintptr_t>(b.g[i]) & (uintptr_t)(b.g_align - 1)) == 0;
    r->g = b.g[i];
    r->vec = ga ? (kVecG | (r->pmv_aligned ? kVecAll : 0)) : 0;
}

// FP32 gradient outputs of up to kBindPerLaunch rows (z1_table_set_grad_out), passed by value like the gradients.
__global__ __launch_bounds__(kBindPerLaunch) void set_grad_out_kernel(float** gout, GradBind b) {
    const int i = threadIdx.x;
    if (i >= b.count) return;
    gout[b.row[i]] = static_cast<float*>(const_cast<void*>(b.g[i]));
}

// All pointers of up to kRebindPerLaunch rows (z1_table_rebind), passed by value like GradBind.
constexpr int kRebindPerLaunch = 64;
struct RowBind {
    const void* g[kRebindPerLaunch];
    float* p[kRebindPerLaunch];
    float* m[kRebindPerLaunch];
    float* v[kRebindPerLaunch];
    uint16_t* p16[kRebindPerLaunch];
    int32_t row[kRebindPerLaunch];
    int32_t count;
    int32_t g_align;
};

__global__ __launch_bounds__(kRebindPerLaunch) void rebind_rows_kernel(Row* rows, RowBind b) {
    const int i = threadIdx.x;
    if (i >= b.count) return;
    Row* r = rows + b.row[i];
    const uintptr_t pmv = reinterpret_cast<uintptr_t>(b.p[i]) | reinterpret_cast<uintptr_t>(b.m[i]) |
                          reinterpret_cast<uintptr_t>(b.v[i]);
    const bool pmv_ok = (pmv & 15) == 0 && (reinterpret_cast<uintptr_t>(b.p16[i]) & 7) == 0;
    const bool ga = (reinterpret_cast<uintptr_t>(b.g[i]) & (uintptr_t)(b.g_align - 1)) == 0;
    r->g = b.g[i];
    r->p = b.p[i];
    r->m = b.m[i];
    r->v = b.v[i];
    r->p16 = b.p16[i];
    r->pmv_aligned = pmv_ok;
    r->vec = ga ? (kVecG | (pmv_ok ? kVecAll : 0)) : 0;
}

// ------------------------------------------------------------------------------------- scale / cast passes
// The scale and cast passes: one wave per kPassChunk-element chunk, dispatched by the hardware with the
// XCD-contiguous map, every load and store instruction of a wave covering one contiguous span (two 4-element
// groups per lane, kPassChunk / 2 elements apart).  A grid-stride loop over the whole array, one 16-byte load in
// flight per wave, reached 3.9 TB/s (scale) and 5.4 TB/s (cast) on 430M elements.
constexpr int64_t kPassChunk = (int64_t)kWave * 8;

__global__ __launch_bounds__(kWave) void scale_up_kernel(const uint16_t* __restrict__ g16, float* __restrict__ g32,
                                                         const float* __restrict__ factor, int64_t n, int vec) {
    const int64_t e0 = chunk_of_block(blockIdx.x, gridDim.x) * kPassChunk;
    const float f = *factor;
    const int lane = threadIdx.x;
    if (vec && e0 + kPassChunk <= n) {
        u2 h[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) h[u] = ld(reinterpret_cast<const u2*>(g16 + e0 + u * (kPassChunk / 2)) + lane);
#pragma unroll
        for (int u = 0; u < 2; ++u)
            st_stream(g32 + e0, (int)kPassChunk * 4, (int)((u * (kPassChunk / 2) + lane * 4) * 4),
                      f4{bf16_lo(h[u].x) * f, bf16_hi(h[u].x) * f, bf16_lo(h[u].y) * f, bf16_hi(h[u].y) * f});
        return;
    }
    const int64_t e1 = e0 + kPassChunk < n ? e0 + kPassChunk : n;
    for (int64_t e = e0 + lane; e < e1; e += kWave) g32[e] = bf16_to_f32(g16[e]) * f;
}

__global__ __launch_bounds__(kWave) void cast_bf16_kernel(const float* __restrict__ p32, uint16_t* __restrict__ p16,
                                                          int64_t n, int vec) {
    const int64_t e0 = chunk_of_block(blockIdx.x, gridDim.x) * kPassChunk;
    const int lane = threadIdx.x;
    if (vec && e0 + kPassChunk <= n) {
        f4 a[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) a[u] = ld(reinterpret_cast<const f4*>(p32 + e0 + u * (kPassChunk / 2)) + lane);
#pragma unroll
        for (int u = 0; u < 2; ++u)
            st_stream(p16 + e0, (int)kPassChunk * 2, (int)((u * (kPassChunk / 2) + lane * 4) * 2),
                      u2{pack_bf16(a[u].x, a[u].y), pack_bf16(a[u].z, a[u].w)});
        return;
    }
    const int64_t e1 = e0 + kPassChunk < n ? e0 + kPassChunk : n;
    for (int64_t e = e0 + lane; e < e1; e += kWave) p16[e] = (uint16_t)f32_to_bf16(p32[e]);
}

// -------------------------------------------------------------------------------------------- host helpers
inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

struct DevInfo {
    int lds_per_cu = -1;       // bytes of LDS per CU; -1: not read yet
};

std::mutex g_mu;
DevInfo g_dev[kMaxDevices];

int current_device(int* dev) {
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return (int)e;
    if (*dev < 0 || *dev >= kMaxDevices) return Z1_E_DEVICE;
    return Z1_OK;
}

// Dynamic LDS a launch reserves (the kernels do not touch it) so that at most `per_cu` of its workgroups are
// resident on one CU: the streaming kernels move HBM faster with fewer requests in flight (MI355X, 160 KiB of LDS
// per CU; C2 update, interleaved A/B runs on one box: Adam 1.93 ms at 11-12 one-wave workgroups per CU, 1.96 at
// 13, 1.99 at 10 and 14, 2.03 at 16, 2.04-2.09 at 20-24, 2.10 at 8, 2.79 at 6; with FP32 gradient outputs, 38
// per-parameter tensors: 2.15-2.17 ms at 11, 2.17-2.19 at 9-10, 2.19-2.23 at 12, 2.27-2.45 at 8 and 14-16; owner
// sum on C3 1.215-1.23 ms at 9-11, 1.23 at 8, 1.42 at 6).  0 when the device does not report its LDS size.
int occupancy_lds(int dev, int per_cu, size_t* bytes) {
    if (dev < 0 || dev >= kMaxDevices || per_cu < 1) return Z1_E_DEVICE;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_dev[dev].lds_per_cu < 0) {
        int v = 0;
        hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev);
        if (e != hipSuccess) return (int)e;
        g_dev[dev].lds_per_cu = v > 0 ? v : 0;
    }
    size_t b = (size_t)g_dev[dev].lds_per_cu / (size_t)per_cu;
    b &= ~(size_t)511;
    *bytes = b > 65536 ? 65536 : b;
    return Z1_OK;
}

inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? Z1_OK : (int)e;
}

}  // namespace

// Scratch of z1_owner_sum_update_noalloc: the norm's Z1_NORM_PARTIALS partials, then one per-wave partial per
// owner-sum chunk, for up to Z1_NOALLOC_MAX_N elements (16.0 MiB; every device the library runs on holds its own copy
// until the process ends).  Host code never passes this name to a kernel: in host code it is a stand-in, not a
// device address.  The address of a device's copy comes from hipGetSymbolAddress, once per device.
constexpr int64_t kNoallocDoubles = Z1_NORM_PARTIALS + owner_sum_waves(Z1_NOALLOC_MAX_N);
static __device__ __align__(256) double scratch[kNoallocDoubles];

namespace {
double* g_scratch_ptr[kMaxDevices];   // device address of `scratch` per device (nullptr: not looked up yet)

// The current device's copy of `scratch`, looked up on the first call on that device with the device current.
int scratch_address(int dev, double** out) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!ptr) return Z1_E_NULL;
        g_scratch_ptr[dev] = static_cast<double*>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return Z1_OK;
}
}  // namespace

struct z1_table {
    Row* rows;            // device, one allocation: the non-empty rows, then nchunks int32 chunk -> row entries
    int32_t* chunk_row;
    std::vector<int64_t> first_chunk;   // host: first chunk of each row given to z1_table_create, + the total
    std::vector<int32_t> dev_row;       // host: device row of each row given to z1_table_create (-1: empty)
    std::vector<int64_t> row_numel;     // host: elements of each row given to z1_table_create
    int nrows;            // rows given to z1_table_create, empty ones included
    int nrows_dev;        // non-empty rows (the device table)
    int g_dtype;
    int device;
    int has_pmv;          // every row has p, m and v
    int gout_rows;        // rows with an FP32 gradient output (z1_table_set_grad_out), as last enqueued
    float** gout;         // device, in the same allocation: the output of each device row (NULL: none)
    int64_t numel;
    int64_t nchunks;
    std::vector<Row> host_rows;   // host copy of the device rows' pointers, kept by rebind / set_grads
    int host_valid;       // 0 once a rebind / set_grads launch failed: the device rows may differ from host_rows
    int g_failed;         // a rebind / set_grads launch failed: the gradient column may be half rewritten; every
                          // launch is refused until a z1_table_set_grads or z1_table_rebind succeeds
    int pmv_failed;       // a rebind launch failed: p, m, v, p16 may be half rewritten; Adam is refused until a
                          // z1_table_rebind succeeds (the norm reads only the gradients)
    int gout_failed;      // a set_grad_out launch failed: Adam is refused until a z1_table_set_grad_out succeeds
    int contig;           // the device rows tile one allocation per stream in order, without gaps (see set_contig)
    Row whole;            // when contig: the first row's pointers, n = numel, the vector flags of the whole
};

namespace z1detail {
int occupancy_lds(int dev, int per_cu, size_t* bytes) { return ::occupancy_lds(dev, per_cu, bytes); }
}  // namespace z1detail

// Whether the table's rows, as the host last bound them, are one flat allocation per stream: row i's g, p, m, v
// (and p16, if any row has one) start where row i - 1's end, every row has p, m and v, and the first row's pointers
// are aligned for the vector path.  Then a whole-table Adam launch walks the buffers directly (adam_flat_kernel).
static void set_contig(z1_table* t) {
    t->contig = 0;
    const std::vector<Row>& h = t->host_rows;
    if (!t->host_valid || h.empty() || !t->has_pmv) return;
    const Row& r0 = h[0];
    const bool with16 = r0.p16 != nullptr;
    const uintptr_t gsz = t->g_dtype == Z1_F32 ? 4 : 2;
    const uintptr_t g0 = reinterpret_cast<uintptr_t>(r0.g), p0 = reinterpret_cast<uintptr_t>(r0.p),
                    m0 = reinterpret_cast<uintptr_t>(r0.m), v0 = reinterpret_cast<uintptr_t>(r0.v),
                    h0 = reinterpret_cast<uintptr_t>(r0.p16);
    if ((g0 & (gsz == 4 ? 15 : 7)) || ((p0 | m0 | v0) & 15) || (h0 & 7)) return;
    uintptr_t off = 0;                                 // elements before row i
    for (const Row& r : h) {
        if ((r.p16 != nullptr) != with16) return;
        if (reinterpret_cast<uintptr_t>(r.g) != g0 + off * gsz || reinterpret_cast<uintptr_t>(r.p) != p0 + off * 4 ||
            reinterpret_cast<uintptr_t>(r.m) != m0 + off * 4 || reinterpret_cast<uintptr_t>(r.v) != v0 + off * 4 ||
            (with16 && reinterpret_cast<uintptr_t>(r.p16) != h0 + off * 2))
            return;
        off += (uintptr_t)r.n;
    }
    t->whole = r0;
    t->whole.n = (int64_t)off;
    t->whole.chunk0 = 0;
    t->whole.pmv_aligned = 1;
    t->whole.vec = kVecG | kVecAll;
    t->contig = 1;
}

extern "C" {

static int table_create(const z1_tensor* rows, int nrows, int g_dtype, z1_table** out);

int z1_table_create(const z1_tensor* rows, int nrows, int g_dtype, z1_table** out) {
    try {
        return table_create(rows, nrows, g_dtype, out);
    } catch (...) {                                     // host allocation failure: no exception crosses the C ABI
        return (int)hipErrorOutOfMemory;
    }
}

static int table_create(const z1_tensor* rows, int nrows, int g_dtype, z1_table** out) {
    if (!out) return Z1_E_NULL;
    *out = nullptr;
    if (nrows < 0) return Z1_E_SIZE;
    if (nrows > 0 && !rows) return Z1_E_NULL;
    if (g_dtype != Z1_F32 && g_dtype != Z1_BF16) return Z1_E_DTYPE;
    const uintptr_t galign = g_dtype == Z1_F32 ? 16 : 8;
    std::vector<Row> h;
    h.reserve(nrows);
    std::vector<int64_t> first((size_t)nrows + 1);
    std::vector<int32_t> dev_row((size_t)nrows, -1);
    std::vector<int64_t> row_numel((size_t)nrows, 0);
    int64_t chunks = 0, numel = 0;
    int has_pmv = 1;
    for (int i = 0; i < nrows; ++i) {
        const z1_tensor& t = rows[i];
        if (t.n < 0 || t.n > (int64_t)INT32_MAX * kChunk) return Z1_E_SIZE;   // also keeps the sums below in range
        first[i] = chunks;
        row_numel[i] = t.n;
        if (t.n == 0) continue;
        if (!t.g) return Z1_E_NULL;
        Row r;
        r.g = t.g;
        r.p = t.p;
        r.m = t.m;
        r.v = t.v;
        r.p16 = t.p16;
        r.n = t.n;
        r.chunk0 = chunks;
        r.pmv_aligned = aligned(t.p, 16) && aligned(t.m, 16) && aligned(t.v, 16) && (!t.p16 || aligned(t.p16, 8));
        r.vec = aligned(t.g, galign) ? (kVecG | (r.pmv_aligned ? kVecAll : 0)) : 0;
        if (!t.p || !t.m || !t.v) has_pmv = 0;
        chunks += (t.n + kChunk - 1) / kChunk;
        numel += t.n;
        if (chunks > INT32_MAX) return Z1_E_SIZE;
        dev_row[i] = (int32_t)h.size();
        h.push_back(r);
    }
    if (chunks > INT32_MAX) return Z1_E_SIZE;          // one workgroup per chunk: grid.x limit
    first[nrows] = chunks;
    int dev = 0;
    int rc = current_device(&dev);
    if (rc) return rc;
    // host image of [rows][chunk -> row][gradient outputs, all NULL], copied in one transfer
    const size_t rows_bytes = sizeof(Row) * h.size();
    const size_t gout_off = (rows_bytes + sizeof(int32_t) * (size_t)chunks + 15) & ~(size_t)15;
    std::vector<unsigned char> img(gout_off + sizeof(float*) * h.size() + 64, 0);
    if (rows_bytes) memcpy(img.data(), h.data(), rows_bytes);
    int32_t* map = reinterpret_cast<int32_t*>(img.data() + rows_bytes);
    for (size_t i = 0; i < h.size(); ++i) {
        const int64_t c1 = i + 1 < h.size() ? h[i + 1].chunk0 : chunks;
        for (int64_t c = h[i].chunk0; c < c1; ++c) map[c] = (int32_t)i;
    }
    z1_table* tb = new (std::nothrow) z1_table();
    if (!tb) return (int)hipErrorOutOfMemory;
    tb->nrows = nrows;
    tb->nrows_dev = (int)h.size();
    tb->g_dtype = g_dtype;
    tb->device = dev;
    tb->has_pmv = has_pmv;
    tb->numel = numel;
    tb->nchunks = chunks;
    tb->first_chunk.swap(first);
    tb->dev_row.swap(dev_row);
    tb->row_numel.swap(row_numel);
    tb->host_rows = h;
    tb->host_valid = 1;
    set_contig(tb);
    tb->rows = nullptr;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&tb->rows), img.size());
    if (e != hipSuccess) {
        delete tb;
        return (int)e;
    }
    tb->chunk_row = reinterpret_cast<int32_t*>(reinterpret_cast<unsigned char*>(tb->rows) + rows_bytes);
    tb->gout = reinterpret_cast<float**>(reinterpret_cast<unsigned char*>(tb->rows) + gout_off);
    tb->gout_rows = 0;
    e = hipMemcpy(tb->rows, img.data(), img.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(tb->rows);
        delete tb;
        return (int)e;
    }
    *out = tb;
    return Z1_OK;
}

static int check_table_device(const z1_table* table, int* dev) {
    int rc = current_device(dev);
    if (rc) return rc;
    return *dev == table->device ? Z1_OK : Z1_E_DEVICE;
}

int z1_table_destroy(z1_table* table) {
    if (!table) return Z1_OK;
    int prev = 0;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess && prev != table->device) e = hipSetDevice(table->device);
    if (e == hipSuccess) e = hipFree(table->rows);
    if (prev != table->device) (void)hipSetDevice(prev);
    delete table;
    return e == hipSuccess ? Z1_OK : (int)e;
}

int z1_table_info(const z1_table* table, int64_t* numel, int64_t* nchunks, int* nrows) {
    if (!table) return Z1_E_NULL;
    if (numel) *numel = table->numel;
    if (nchunks) *nchunks = table->nchunks;
    if (nrows) *nrows = table->nrows;             // the rows given to z1_table_create, empty ones included
    return Z1_OK;
}

int z1_table_rebind(z1_table* table, const z1_tensor* rows, int nrows, void* stream) {
    if (!table || (nrows > 0 && !rows)) return Z1_E_NULL;
    if (nrows != table->nrows) return Z1_E_SIZE;
    int dev = 0;
    int rc = check_table_device(table, &dev);
    if (rc) return rc;
    for (int i = 0; i < nrows; ++i) {                  // the same sizes, and every pointer a launch will follow
        if (rows[i].n != table->row_numel[i]) return Z1_E_SIZE;
        if (table->dev_row[i] < 0) continue;           // an empty row
        if (!rows[i].g) return Z1_E_NULL;
        if (table->has_pmv && (!rows[i].p || !rows[i].m || !rows[i].v)) return Z1_E_NULL;
    }
    RowBind b;
    memset(&b, 0, sizeof(b));
    b.g_align = table->g_dtype == Z1_F32 ? 16 : 8;
    hipStream_t s = static_cast<hipStream_t>(stream);
    table->contig = 0;                                 // until every rebind launch is enqueued
    for (int i = 0; i < nrows; ++i) {
        if (table->dev_row[i] < 0) continue;
        Row& hr = table->host_rows[table->dev_row[i]];
        hr.g = rows[i].g;
        hr.p = rows[i].p;
        hr.m = rows[i].m;
        hr.v = rows[i].v;
        hr.p16 = rows[i].p16;
    }
    for (int i = 0; i < nrows; ++i) {
        if (table->dev_row[i] < 0) continue;
        const int k = b.count;
        b.g[k] = rows[i].g;
        b.p[k] = rows[i].p;
        b.m[k] = rows[i].m;
        b.v[k] = rows[i].v;
        b.p16[k] = rows[i].p16;
        b.row[k] = table->dev_row[i];
        if (++b.count == kRebindPerLaunch) {
            hipLaunchKernelGGL(rebind_rows_kernel, dim3(1), dim3(kRebindPerLaunch), 0, s, table->rows, b);
            rc = launch_status();
            if (rc) {
                table->host_valid = 0;
                table->g_failed = table->pmv_failed = 1;
                return rc;
            }
            b.count = 0;
        }
    }
    if (b.count) {
        hipLaunchKernelGGL(rebind_rows_kernel, dim3(1), dim3(kRebindPerLaunch), 0, s, table->rows, b);
        rc = launch_status();
        if (rc) {
            table->host_valid = 0;
            table->g_failed = table->pmv_failed = 1;
            return rc;
        }
    }
    table->host_valid = 1;                             // every row's pointers as host_rows now holds them
    table->g_failed = table->pmv_failed = 0;
    set_contig(table);
    return Z1_OK;
}

int z1_table_set_grads(z1_table* table, const void* const* g, int nrows, void* stream) {
    if (!table || (nrows > 0 && !g)) return Z1_E_NULL;
    if (nrows != table->nrows) return Z1_E_SIZE;
    int dev = 0;
    int rc = check_table_device(table, &dev);
    if (rc) return rc;
    GradBind b;
    b.count = 0;
    b.g_align = table->g_dtype == Z1_F32 ? 16 : 8;
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < nrows; ++i) {
        if (table->dev_row[i] < 0) continue;
        if (!g[i]) return Z1_E_NULL;
    }
    table->contig = 0;                                 // until every binding launch is enqueued
    for (int i = 0; i < nrows; ++i)
        if (table->dev_row[i] >= 0) table->host_rows[table->dev_row[i]].g = g[i];
    for (int i = 0; i < nrows; ++i) {
        if (table->dev_row[i] < 0) continue;
        b.g[b.count] = g[i];
        b.row[b.count] = table->dev_row[i];
        if (++b.count == kBindPerLaunch) {
            hipLaunchKernelGGL(set_grads_kernel, dim3(1), dim3(kBindPerLaunch), 0, s, table->rows, b);
            rc = launch_status();
            if (rc) {
                table->host_valid = 0;
                table->g_failed = 1;
                return rc;
            }
            b.count = 0;
        }
    }
    if (b.count) {
        hipLaunchKernelGGL(set_grads_kernel, dim3(1), dim3(kBindPerLaunch), 0, s, table->rows, b);
        rc = launch_status();
        if (rc) {
            table->host_valid = 0;
            table->g_failed = 1;
            return rc;
        }
    }
    table->g_failed = 0;                               // every row's gradient rewritten
    set_contig(table);
    return Z1_OK;
}

int z1_table_set_grad_out(z1_table* table, float* const* g32, int nrows, void* stream) {
    if (!table) return Z1_E_NULL;
    if (g32 && nrows != table->nrows) return Z1_E_SIZE;
    int dev = 0;
    int rc = check_table_device(table, &dev);
    if (rc) return rc;
    GradBind b;
    b.count = 0;
    b.g_align = 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int set = 0;
    for (int i = 0; i < table->nrows; ++i) {
        if (table->dev_row[i] < 0) continue;
        float* o = g32 ? g32[i] : nullptr;
        set += o != nullptr;
        b.g[b.count] = o;
        b.row[b.count] = table->dev_row[i];
        if (++b.count == kBindPerLaunch) {
            hipLaunchKernelGGL(set_grad_out_kernel, dim3(1), dim3(kBindPerLaunch), 0, s, table->gout, b);
            rc = launch_status();
            if (rc) {
                table->gout_failed = 1;            // the column may be half rewritten
                return rc;
            }
            b.count = 0;
        }
    }
    if (b.count) {
        hipLaunchKernelGGL(set_grad_out_kernel, dim3(1), dim3(kBindPerLaunch), 0, s, table->gout, b);
        rc = launch_status();
        if (rc) {
            table->gout_failed = 1;
            return rc;
        }
    }
    table->gout_rows = set;
    table->gout_failed = 0;
    return Z1_OK;
}

// First chunk of a table that the norm reads with allocating loads: the last kMallKeepBytes of gradient.
static int64_t keep_from(const z1_table* table) {
    const int64_t chunk_bytes = kChunk * (table->g_dtype == Z1_F32 ? 4 : 2);
    const int64_t keep = kMallKeepBytes / chunk_bytes;
    return table->nchunks > keep ? table->nchunks - keep : 0;
}

// The norm kernel over the table, then, with a tail, the one-workgroup final reduction + scalar chain.  (A single
// launch whose last workgroup to finish runs the tail was measured slower: the 2048 workgroups end together, and
// their device-scope release fences and same-address counter atomics cost 15-35 us at the end of the grid, against
// about 4 us for the second launch.)
static int launch_sumsq(const z1_table* table, double* partials, const z1_update_scalars* tail, void* stream) {
    int dev = 0;
    int rc = check_table_device(table, &dev);
    if (rc) return rc;
    if (table->g_failed) return Z1_E_STATE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t kf = keep_from(table);
    if (table->g_dtype == Z1_F32)
        hipLaunchKernelGGL((sumsq_kernel<Z1_F32, kThreads>), dim3(Z1_NORM_PARTIALS), dim3(kThreads), 0, s,
                           table->rows, table->nrows_dev, table->nchunks, kf, partials);
    else
        hipLaunchKernelGGL((sumsq_kernel<Z1_BF16, kSumsqBf16Threads>), dim3(Z1_NORM_PARTIALS),
                           dim3(kSumsqBf16Threads), 0, s, table->rows, table->nrows_dev, table->nchunks, kf, partials);
    rc = launch_status();
    if (rc || !tail) return rc;
    hipLaunchKernelGGL(scalars_kernel, dim3(1), dim3(kThreads), 0, s, partials, *tail);
    return launch_status();
}

static z1_update_scalars clip_args(const float* factor_in, float factor_value, float* norm_out, float* grad_norm_out,
                                   float* factor_out, float max_norm) {
    z1_update_scalars u;
    memset(&u, 0, sizeof(u));
    u.numer = 1.0f;
    u.factor_in = factor_in;
    u.factor_value = factor_value;
    u.max_norm = max_norm;
    u.norm_out = norm_out;
    u.grad_norm_out = grad_norm_out;
    u.factor_out = factor_out;
    return u;
}

int z1_grad_sumsq(const z1_table* table, double* partials, void* stream) {
    if (!table || !partials) return Z1_E_NULL;
    return launch_sumsq(table, partials, nullptr, stream);
}

int z1_grad_norm_clip(const z1_table* table, double* partials, const float* factor_in, float factor_value,
                      float* norm_out, float* grad_norm_out, float* factor_out, float max_norm, void* stream) {
    if (!table || !partials) return Z1_E_NULL;
    const z1_update_scalars u = clip_args(factor_in, factor_value, norm_out, grad_norm_out, factor_out, max_norm);
    return launch_sumsq(table, partials, &u, stream);
}

int z1_grad_update_scalars(const z1_table* table, double* partials, const z1_update_scalars* u, void* stream) {
    if (!table || !partials || !u) return Z1_E_NULL;
    return launch_sumsq(table, partials, u, stream);
}

int z1_norm_clip(const double* partials, const float* factor_in, float factor_value, float* norm_out,
                 float* grad_norm_out, float* factor_out, float max_norm, void* stream) {
    if (!partials) return Z1_E_NULL;
    hipLaunchKernelGGL(scalars_kernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream), partials,
                       clip_args(factor_in, factor_value, norm_out, grad_norm_out, factor_out, max_norm));
    return launch_status();
}

int z1_update_scalars_run(const double* partials, const z1_update_scalars* u, void* stream) {
    if (!partials || !u) return Z1_E_NULL;
    hipLaunchKernelGGL(scalars_kernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream), partials, *u);
    return launch_status();
}

int z1_clip_factor(const float* norm, const float* factor_in, float factor_value, float* grad_norm_out,
                   float* factor_out, float max_norm, void* stream) {
    if (!norm) return Z1_E_NULL;
    hipLaunchKernelGGL(clip_factor_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), norm, factor_in,
                       factor_value, grad_norm_out, factor_out, max_norm);
    return launch_status();
}

static int adam_launch(const z1_table* table, int64_t chunk_begin, int64_t chunk_end, const float* factor, float lr,
                       float beta1, float beta2, float eps, float bc1, float bc2, const float* bc, float weight_decay,
                       int mode, void* stream) {
    if (!table) return Z1_E_NULL;
    if (mode != 0 && mode != 1) return Z1_E_MODE;
    if (!table->has_pmv) return Z1_E_NULL;
    int dev = 0;
    int rc = check_table_device(table, &dev);
    if (rc) return rc;
    if (table->g_failed || table->pmv_failed || table->gout_failed) return Z1_E_STATE;
    if (chunk_end <= chunk_begin) return Z1_OK;
    AdamK k;
    k.lr = lr;
    k.b1 = beta1;
    k.b2 = beta2;
    k.eps = eps;
    k.bc1 = bc1;
    k.bc2 = bc2;
    k.wd = weight_decay;
    k.omb1 = 1.0f - beta1;
    k.omb2 = 1.0f - beta2;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool gout = table->gout_rows > 0;
    size_t lds = 0;
    if (table->contig && !gout && chunk_begin == 0 && chunk_end == table->nchunks) {   // the whole flat shard
        const int64_t nflat = (table->whole.n + kChunk - 1) / kChunk;
        rc = occupancy_lds(dev, kAdamFlatWgPerCu, &lds);
        if (rc) return rc;
#define Z1_LAUNCH_ADAM_FLAT(GDT, MODE)                                                                        \
    hipLaunchKernelGGL((adam_flat_kernel<GDT, MODE>), dim3((unsigned)nflat), dim3(kWave), lds, s, table->whole, \
                       nflat, factor, bc, k)
        if (table->g_dtype == Z1_F32) {
            if (mode == 1) Z1_LAUNCH_ADAM_FLAT(Z1_F32, 1);
            else Z1_LAUNCH_ADAM_FLAT(Z1_F32, 0);
        } else {
            if (mode == 1) Z1_LAUNCH_ADAM_FLAT(Z1_BF16, 1);
            else Z1_LAUNCH_ADAM_FLAT(Z1_BF16, 0);
        }
#undef Z1_LAUNCH_ADAM_FLAT
        return launch_status();
    }
    const dim3 grid((unsigned)((chunk_end - chunk_begin + kAdamWaves - 1) / kAdamWaves));
    rc = occupancy_lds(dev, gout ? kAdamGoutWgPerCu : kAdamWgPerCu, &lds);
    if (rc) return rc;
#define Z1_LAUNCH_ADAM(GDT, MODE, GOUT)                                                                        \
    hipLaunchKernelGGL((adam_cast_kernel<GDT, MODE, GOUT>), grid, dim3(kWave * kAdamWaves), lds, s, table->rows, \
                       table->chunk_row, table->nrows_dev, chunk_begin, chunk_end, factor, bc, k, table->gout)
#define Z1_LAUNCH_ADAM_MODES(GDT, GOUT)                                                                        \
    if (mode == 1) Z1_LAUNCH_ADAM(GDT, 1, GOUT);                                                              \
    else Z1_LAUNCH_ADAM(GDT, 0, GOUT)
    if (table->g_dtype == Z1_F32) {
        if (gout) { Z1_LAUNCH_ADAM_MODES(Z1_F32, true); }
        else { Z1_LAUNCH_ADAM_MODES(Z1_F32, false); }
    } else {
        if (gout) { Z1_LAUNCH_ADAM_MODES(Z1_BF16, true); }
        else { Z1_LAUNCH_ADAM_MODES(Z1_BF16, false); }
    }
#undef Z1_LAUNCH_ADAM_MODES
#undef Z1_LAUNCH_ADAM
    return launch_status();
}

int z1_adam_cast(const z1_table* table, const float* factor, float lr, float beta1, float beta2, float eps,
                 float bc1, float bc2, float weight_decay, int mode, void* stream) {
    if (!table) return Z1_E_NULL;
    return adam_launch(table, 0, table->nchunks, factor, lr, beta1, beta2, eps, bc1, bc2, nullptr, weight_decay, mode,
                       stream);
}

int z1_adam_cast_rows(const z1_table* table, int row_begin, int row_end, const float* factor, float lr, float beta1,
                      float beta2, float eps, float bc1, float bc2, float weight_decay, int mode, void* stream) {
    if (!table) return Z1_E_NULL;
    const int nrows = (int)table->first_chunk.size() - 1;
    if (row_begin < 0 || row_end < row_begin || row_end > nrows) return Z1_E_SIZE;
    return adam_launch(table, table->first_chunk[row_begin], table->first_chunk[row_end], factor, lr, beta1, beta2,
                       eps, bc1, bc2, nullptr, weight_decay, mode, stream);
}

int z1_adam_cast_dev(const z1_table* table, const float* factor, float lr, float beta1, float beta2, float eps,
                     const float* bc, float weight_decay, int mode, void* stream) {
    if (!table || !bc) return Z1_E_NULL;
    return adam_launch(table, 0, table->nchunks, factor, lr, beta1, beta2, eps, 1.0f, 1.0f, bc, weight_decay, mode,
                       stream);
}

int z1_bias_corrections_step(int64_t* step, double beta1, double beta2, int bias_correction, float* bc,
                             void* stream) {
    if (!step || !bc) return Z1_E_NULL;
    hipLaunchKernelGGL(bias_step_kernel, dim3(1), dim3(kWave), 0, static_cast<hipStream_t>(stream), step, beta1,
                       beta2, bias_correction, bc);
    return launch_status();
}

int64_t z1_owner_sum_waves(int64_t n) {
    if (n < 0) return Z1_E_SIZE;
    return owner_sum_waves(n);
}

int64_t z1_owner_sum_workspace(int64_t n) {
    if (n < 0) return Z1_E_SIZE;
    return Z1_NORM_PARTIALS + owner_sum_waves(n);   // the partials, then one per chunk
}

// Shift of the owner sum's chunk grid (owner_sum_kernel) for these streams, and whether the vector path applies:
// when every bf16 stream lies at the same offset within a 128-byte line as out_avg, the chunk boundaries go on those
// lines; else, when they share the offset within an 8-byte word, on the words; else the element-wise path.  The
// FP32 sum (nullable) must then be 16-byte aligned at the same boundaries.
static int owner_sum_grid(const Srcs& s, int world, const uint16_t* out_avg, const float* out_sum, int64_t* shift) {
    const uintptr_t o = reinterpret_cast<uintptr_t>(out_avg);
    *shift = 0;
    if (o & 1) return 0;
    uintptr_t diff = 0;
    for (int k = 0; k < world; ++k) diff |= reinterpret_cast<uintptr_t>(s.p[k]) - o;
    int64_t sh;
    if ((diff & 127) == 0) sh = (int64_t)((o & 127) >> 1);
    else if ((diff & 7) == 0) sh = (int64_t)((o & 7) >> 1);
    else return 0;
    if (out_sum) {
        const uintptr_t f = reinterpret_cast<uintptr_t>(out_sum);
        if ((f & 3) || (((f >> 2) - (uintptr_t)sh) & 3)) return 0;
    }
    *shift = sh;
    return 1;
}

// The owner sum; with `waves` (owner_sum_waves(n) doubles) each chunk's FP64 norm partial is written there, and with
// a workspace (z1_owner_sum_workspace(n) doubles: the Z1_NORM_PARTIALS partials, then the per-chunk ones) the
// per-chunk partials' fixed-order reduction leaves the Z1_NORM_PARTIALS partials at its start (z1_owner_sum_bf16),
// followed, with a tail, by the one-workgroup final reduction + scalar chain (z1_owner_sum_update).
static int owner_sum(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                     float* out_sum, double* waves, double* workspace, const z1_update_scalars* tail, void* stream) {
    if (!contrib) return Z1_E_NULL;
    if (world < 1 || world > Z1_MAX_WORLD) return Z1_E_WORLD;
    if (n < 0) return Z1_E_SIZE;
    if (n > 0 && !out_avg) return Z1_E_NULL;               // empty inputs may carry NULL data pointers
    Srcs srcs;
    memset(&srcs, 0, sizeof(srcs));
    for (int k = 0; k < world; ++k) {
        if (n > 0 && !contrib[k]) return Z1_E_NULL;
        srcs.p[k] = contrib[k];
    }
    int64_t shift = 0;
    const int vec = owner_sum_grid(srcs, world, out_avg, out_sum, &shift);
    const int64_t nchunks = owner_sum_waves(n);
    if (nchunks > INT32_MAX) return Z1_E_SIZE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    double* wave_partials = workspace ? workspace + Z1_NORM_PARTIALS : waves;
    if (nchunks > 0) {
        int dev = 0;
        size_t lds = 0;
        int rc = current_device(&dev);
        if (rc == Z1_OK) rc = occupancy_lds(dev, kOwnerSumWgPerCu, &lds);
        if (rc) return rc;
        launch_owner_sum<Z1_MAX_WORLD>(world, nchunks, lds, st, srcs, n, scale, out_avg, out_sum, wave_partials, vec,
                                       shift);
        rc = launch_status();
        if (rc) return rc;
    }
    if (!workspace) return Z1_OK;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3(Z1_NORM_PARTIALS), dim3(kThreads), 0, st, wave_partials, nchunks,
                       workspace);
    int rc = launch_status();
    if (rc || !tail) return rc;
    hipLaunchKernelGGL(scalars_kernel, dim3(1), dim3(kThreads), 0, st, workspace, *tail);
    return launch_status();
}

int z1_owner_sum_bf16(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                      float* out_sum, double* sumsq_partials, void* stream) {
    return owner_sum(contrib, world, n, scale, out_avg, out_sum, nullptr, sumsq_partials, nullptr, stream);
}

int z1_owner_sum_bf16_waves(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                            float* out_sum, double* waves, void* stream) {
    return owner_sum(contrib, world, n, scale, out_avg, out_sum, waves, nullptr, nullptr, stream);
}

int z1_reduce_waves(const double* waves, int64_t m, double* partials, void* stream) {
    if (!partials || (m > 0 && !waves)) return Z1_E_NULL;
    if (m < 0) return Z1_E_SIZE;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3(Z1_NORM_PARTIALS), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), waves, m, partials);
    return launch_status();
}

int z1_owner_sum_update(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                        float* out_sum, double* workspace, const z1_update_scalars* u, void* stream) {
    if (!workspace || !u) return Z1_E_NULL;
    return owner_sum(contrib, world, n, scale, out_avg, out_sum, nullptr, workspace, u, stream);
}

int z1_owner_sum_update_noalloc(const uint16_t* const* contrib, int world, int64_t n, float scale, uint16_t* out_avg,
                                float* out_sum, const z1_update_scalars* u, void* stream) {
    if (!u) return Z1_E_NULL;
    if (n < 0) return Z1_E_SIZE;
    if (n > Z1_NOALLOC_MAX_N) return Z1_E_NOALLOC_MAX;
    int dev = 0;
    int rc = current_device(&dev);
    if (rc) return rc;
    double* ws = nullptr;
    rc = scratch_address(dev, &ws);
    if (rc) return rc;
    // every scratch slot this call reads is written by it first (the per-wave partials by the owner sum, the
    // Z1_NORM_PARTIALS partials by their reduction), so nothing needs clearing between calls
    return owner_sum(contrib, world, n, scale, out_avg, out_sum, nullptr, ws, u, stream);
}

int z1_scale_up(const uint16_t* g16, float* g32, const float* factor, int64_t n, void* stream) {
    if (n < 0) return Z1_E_SIZE;
    if (n == 0) return Z1_OK;
    if (!g16 || !g32 || !factor) return Z1_E_NULL;
    const int64_t chunks = (n + kPassChunk - 1) / kPassChunk;
    if (chunks > INT32_MAX) return Z1_E_SIZE;
    const int vec = aligned(g16, 8) && aligned(g32, 16);
    hipLaunchKernelGGL(scale_up_kernel, dim3((unsigned)chunks), dim3(kWave), 0, static_cast<hipStream_t>(stream),
                       g16, g32, factor, n, vec);
    return launch_status();
}

int z1_cast_bf16(const float* p32, uint16_t* p16, int64_t n, void* stream) {
    if (n < 0) return Z1_E_SIZE;
    if (n == 0) return Z1_OK;
    if (!p32 || !p16) return Z1_E_NULL;
    const int64_t chunks = (n + kPassChunk - 1) / kPassChunk;
    if (chunks > INT32_MAX) return Z1_E_SIZE;
    const int vec = aligned(p32, 16) && aligned(p16, 8);
    hipLaunchKernelGGL(cast_bf16_kernel, dim3((unsigned)chunks), dim3(kWave), 0, static_cast<hipStream_t>(stream),
                       p32, p16, n, vec);
    return launch_status();
}

const char* z1_strerror(int code) {
    switch (code) {
        case Z1_OK: return "ok";
        case Z1_E_NULL: return "a required pointer is NULL";
        case Z1_E_SIZE: return "invalid element count";
        case Z1_E_DTYPE: return "unknown gradient dtype";
        case Z1_E_WORLD: return "world outside 1..Z1_MAX_WORLD";
        case Z1_E_MODE: return "Adam mode must be 0 or 1";
        case Z1_E_WORKSPACE: return "workspace too small";
        case Z1_E_DEVICE: return "table used on another device than it was created on";
        case Z1_E_NOALLOC_MAX: return "more than Z1_NOALLOC_MAX_N elements for the no-allocation entry point";
        case Z1_E_STATE: return "a binding launch on this table failed; rebind it before launching over it";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown error";
}

}  // extern "C"
