// yoco_z1: the owner's token-embedding gradient (declarations: include/yoco_z1.h).
//
// Replaces torch.ops.aten.embedding_dense_backward(g_all, ids, V, padding_idx, False) on the embedding's owner,
// followed or preceded by the x 1/world of the reference (yoco/models/decoder/layer_graphs.py:87-93,
// yoco/models/decoder/ce_reduce.py:226-231).  Same summation order as aten's sort-based GPU path (which aten takes
// for more than 3072 indices): occurrences of each token id in stable position order, fp32 partial sums over
// runs of 10 consecutive occurrences, the partials summed in order, one rounding to bf16; padding_idx rows and
// ids outside [0, V) contribute nothing.
//
//   1. keys[i] = id_i (or V when out of range), vals[i] = i;  2. stable radix sort (hipCUB / rocPRIM);
//   3. row_lo[t] = start of id t's run in the sorted keys (one binary search per t, all in parallel);
//   4. one wave per output row t writes the row's sums -- or zeros -- exactly once, 8 bf16 columns per lane, with
//      nontemporal stores (aten zero-fills the whole table and then scatters into it; here every row of the table
//      is written once), for ids with at most kHeavyRows occurrences; the others are listed for
//   5. emb_heavy_kernel, which forms a heavy id's partials of 10 in parallel (16 per workgroup batch) and adds
//      them in order: token frequencies in text are skewed, and one wave walking thousands of occurrences of one
//      id would take milliseconds.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <stdint.h>

#include "yoco_z1.h"
#include "z1_internal.h"

#pragma clang fp contract(off)

namespace {

constexpr int kEmbThreads = 64;                  // one wave per output row
constexpr int kRowsPerPartial = 10;        // aten's NROWS_PER_THREAD
// resident row workgroups per CU, capped with a dynamic LDS reservation the kernel does not use: 0.131 ms per call
// at 9-10 per CU against 0.148 ms at the 32 the waves allow (0.144 at 16, 0.136 at 8, 0.146 at 7, 0.180 at 6)
constexpr int kEmbWgPerCu = 10;
constexpr int kWave = 64;
constexpr int kHeavyRows = 20;             // tokens with more occurrences go to emb_heavy_kernel
constexpr int kHeavyWaves = 16;            // waves of a heavy workgroup: one run partial each per batch
constexpr int kHeavyGrid = 1024;           // heavy workgroups (each loops over the heavy items)

__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t bf16r(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__global__ void emb_keys_kernel(const int64_t* __restrict__ ids, int64_t R, int64_t V, uint32_t* __restrict__ keys,
                                int32_t* __restrict__ vals) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= R) return;
    const int64_t t = ids[i];
    keys[i] = (t >= 0 && t < V) ? (uint32_t)t : (uint32_t)V;
    vals[i] = (int32_t)i;
}

// row_lo[t] = first index of the sorted keys that is >= t, for t in [0, V]: row t's occurrences are
// [row_lo[t], row_lo[t+1]).  One independent binary search per thread (the latency of the searches overlaps).
__global__ void emb_row_ranges_kernel(const uint32_t* __restrict__ sorted, int64_t R, int64_t V,
                                      int32_t* __restrict__ row_lo, int* __restrict__ heavy_count) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t == 0) *heavy_count = 0;               // the rows kernel appends the heavy tokens after this kernel
    if (t > V) return;
    int64_t lo = 0, hi = R;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (sorted[mid] < (uint32_t)t) lo = mid + 1;
        else hi = mid;
    }
    row_lo[t] = (int32_t)lo;
}

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// One gradient element as it enters a partial: scale_mode 1 rounds bf16(g * scale) first (the CE path scales the
// staged rows in place, ce_reduce.py:228).
__device__ __forceinline__ float grad_elem(uint16_t h, float scale, int scale_mode) {
    float v = bf16f(h);
    if (scale_mode == 1) v = bf16f(bf16r(v * scale));
    return v;
}

// The finished fp32 sum to bf16; scale_mode 2 multiplies the bf16 result by scale and rounds again
// (layer_graphs.py:93).
__device__ __forceinline__ uint16_t finish(float acc, float scale, int scale_mode) {
    uint16_t o = bf16r(acc);
    if (scale_mode == 2) o = bf16r(bf16f(o) * scale);
    return o;
}

__device__ __forceinline__ void nt_store(u4* p, u4 x) {
    __builtin_nontemporal_store(x, (__attribute__((address_space(1))) u4*)p);
}

// One wave per output row t (light tokens: at most kHeavyRows occurrences, and empty or padding rows): the row's
// sums -- or zeros -- written once, 8 bf16 columns per lane when vec (D % 8 == 0, 16-byte aligned tables).  Each
// run of up to kRowsPerPartial occurrences has its loads issued together, then is summed in order.  A token with
// more occurrences is appended to heavy_list (its slot from an atomic counter: the order of the list only decides
// which workgroup of emb_heavy_kernel takes it) and its row is left to that kernel.
__global__ __launch_bounds__(kEmbThreads) void emb_rows_kernel(const uint16_t* __restrict__ grad, int64_t D,
                                                               const int32_t* __restrict__ spos,
                                                               const int32_t* __restrict__ row_lo,
                                                               int64_t padding_idx, float scale, int scale_mode,
                                                               int vec, uint16_t* __restrict__ out,
                                                               int* __restrict__ heavy_count,
                                                               int32_t* __restrict__ heavy_list) {
    // row of workgroup b: undoes the round-robin dispatch over the 8 XCDs, so each XCD writes one contiguous
    // eighth of the table (0.148 vs 0.153 ms per call for t = b)
    int64_t t;
    {
        const int64_t b = blockIdx.x, nb = gridDim.x;
        const int64_t x = b & 7, q = b >> 3, Q = nb >> 3, R = nb & 7;
        t = x * Q + (x < R ? x : R) + q;
    }
    const int lane = threadIdx.x;
    uint16_t* orow = out + t * D;
    const int64_t lo = row_lo[t], hi = row_lo[t + 1];
    const bool empty = lo == hi || t == padding_idx;
    if (!empty && hi - lo > kHeavyRows) {
        if (lane == 0) heavy_list[atomicAdd(heavy_count, 1)] = (int32_t)t;
        return;
    }
    if (vec) {
        const int64_t ng = D / 8;
        for (int64_t gi = lane; gi < ng; gi += kEmbThreads) {
            u4 o = u4{0u, 0u, 0u, 0u};
            if (!empty) {
                float acc[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
                for (int64_t j0 = lo; j0 < hi; j0 += kRowsPerPartial) {
                    const int cnt = (int)(j0 + kRowsPerPartial < hi ? kRowsPerPartial : hi - j0);
                    u4 x[kRowsPerPartial];
#pragma unroll
                    for (int u = 0; u < kRowsPerPartial; ++u)
                        if (u < cnt) x[u] = reinterpret_cast<const u4*>(grad + (int64_t)spos[j0 + u] * D)[gi];
                    float part[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) part[k] = 0.0f;
#pragma unroll
                    for (int u = 0; u < kRowsPerPartial; ++u) {
                        if (u < cnt) {
#pragma unroll
                            for (int k = 0; k < 8; ++k)
                                part[k] = part[k] + grad_elem((uint16_t)(x[u][k >> 1] >> ((k & 1) * 16)), scale,
                                                              scale_mode);
                        }
                    }
#pragma unroll
                    for (int k = 0; k < 8; ++k) acc[k] = acc[k] + part[k];
                }
#pragma unroll
                for (int k = 0; k < 8; k += 2)
                    o[k >> 1] = (uint32_t)finish(acc[k], scale, scale_mode) |
                                ((uint32_t)finish(acc[k + 1], scale, scale_mode) << 16);
            }
            // nontemporal: the 616 MB table is written once and not read back here (0.155 vs 0.184 ms per call)
            nt_store(reinterpret_cast<u4*>(orow) + gi, o);
        }
        return;
    }
    for (int64_t d = lane; d < D; d += kEmbThreads) {
        uint16_t o = 0;
        if (!empty) {
            float acc = 0.0f;
            for (int64_t j0 = lo; j0 < hi; j0 += kRowsPerPartial) {
                const int64_t j1 = j0 + kRowsPerPartial < hi ? j0 + kRowsPerPartial : hi;
                float part = 0.0f;
                for (int64_t j = j0; j < j1; ++j) part = part + grad_elem(grad[(int64_t)spos[j] * D + d], scale,
                                                                          scale_mode);
                acc = acc + part;
            }
            o = finish(acc, scale, scale_mode);
        }
        orow[d] = o;
    }
}

// Heavy tokens (more than kHeavyRows occurrences): workgroup g takes the items g, g + G, ... of (heavy token,
// column group) -- 512 columns per group on the vector path, 64 otherwise -- until the count the rows kernel
// left; every workgroup exits.  Per batch, wave w forms the partial of run b + w (its loads issued together,
// summed in order) into LDS, then wave 0 adds the batch's partials to its accumulator in run order: the same
// order as the rows kernel and aten, with the runs of one token computed in parallel.
template <int VEC>
__global__ __launch_bounds__(kWave * kHeavyWaves) void emb_heavy_kernel(const uint16_t* __restrict__ grad, int64_t D,
                                                                         const int32_t* __restrict__ spos,
                                                                         const int32_t* __restrict__ row_lo,
                                                                         float scale, int scale_mode,
                                                                         uint16_t* __restrict__ out,
                                                                         const int* __restrict__ heavy_count,
                                                                         const int32_t* __restrict__ heavy_list) {
    constexpr int kCols = VEC ? 8 : 1;                       // columns per lane
    __shared__ float parts[kHeavyWaves][kWave][kCols];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const int64_t cols_per_item = (int64_t)kWave * kCols;
    const int64_t ncg = (D + cols_per_item - 1) / cols_per_item;
    const int64_t items = (int64_t)(*heavy_count) * ncg;
    for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
        const int64_t t = heavy_list[item / ncg];
        const int64_t c0 = (item % ncg) * cols_per_item + (int64_t)lane * kCols;   // this lane's first column
        const bool valid = c0 < D;                                                 // D % 8 == 0 when VEC
        const int64_t lo = row_lo[t], hi = row_lo[t + 1];
        const int64_t nrun = (hi - lo + kRowsPerPartial - 1) / kRowsPerPartial;
        float acc[kCols];
#pragma unroll
        for (int k = 0; k < kCols; ++k) acc[k] = 0.0f;
        for (int64_t b = 0; b < nrun; b += kHeavyWaves) {
            float part[kCols];
#pragma unroll
            for (int k = 0; k < kCols; ++k) part[k] = 0.0f;
            const int64_t r = b + wave;
            if (r < nrun && valid) {
                const int64_t j0 = lo + r * kRowsPerPartial;
                const int cnt = (int)(j0 + kRowsPerPartial < hi ? kRowsPerPartial : hi - j0);
                if (VEC) {
                    u4 x[kRowsPerPartial];
#pragma unroll
                    for (int u = 0; u < kRowsPerPartial; ++u)
                        if (u < cnt) x[u] = *reinterpret_cast<const u4*>(grad + (int64_t)spos[j0 + u] * D + c0);
#pragma unroll
                    for (int u = 0; u < kRowsPerPartial; ++u) {
                        if (u < cnt) {
#pragma unroll
                            for (int k = 0; k < kCols; ++k)
                                part[k] = part[k] + grad_elem((uint16_t)(x[u][k >> 1] >> ((k & 1) * 16)), scale,
                                                              scale_mode);
                        }
                    }
                } else {
                    uint16_t x[kRowsPerPartial];
#pragma unroll
                    for (int u = 0; u < kRowsPerPartial; ++u)
                        if (u < cnt) x[u] = grad[(int64_t)spos[j0 + u] * D + c0];
#pragma unroll
                    for (int u = 0; u < kRowsPerPartial; ++u)
                        if (u < cnt) part[0] = part[0] + grad_elem(x[u], scale, scale_mode);
                }
            }
#pragma unroll
            for (int k = 0; k < kCols; ++k) parts[wave][lane][k] = part[k];
            __syncthreads();
            if (wave == 0) {
                for (int w = 0; w < kHeavyWaves; ++w) {
                    if (b + w < nrun) {
#pragma unroll
                        for (int k = 0; k < kCols; ++k) acc[k] = acc[k] + parts[w][lane][k];
                    }
                }
            }
            __syncthreads();
        }
        if (wave == 0 && valid) {
            uint16_t* orow = out + t * D + c0;
            if (VEC) {
                u4 o;
#pragma unroll
                for (int k = 0; k < 8; k += 2)
                    o[k >> 1] = (uint32_t)finish(acc[k], scale, scale_mode) |
                                ((uint32_t)finish(acc[k + 1], scale, scale_mode) << 16);
                nt_store(reinterpret_cast<u4*>(orow), o);
            } else {
                orow[0] = finish(acc[0], scale, scale_mode);
            }
        }
    }
}

size_t sort_temp_bytes(int64_t R) {
    size_t bytes = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                             (const int32_t*)nullptr, (int32_t*)nullptr, (int)R, 0, 32);
    return bytes;
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

extern "C" {

// Workspace: keys, positions, sorted keys, sorted positions (R each), row_lo (V + 1), the heavy-token count and
// list (V), then the sort's temporary storage.
int64_t z1_embedding_backward_workspace(int64_t R, int64_t V) {
    if (R < 0 || R > INT32_MAX || V <= 0 || V > INT32_MAX - 1) return Z1_E_SIZE;
    const size_t kb = align256(sizeof(uint32_t) * (size_t)(R > 0 ? R : 1));
    return (int64_t)(4 * kb + align256(sizeof(int32_t) * (size_t)(V + 1)) + 256 +
                     align256(sizeof(int32_t) * (size_t)V) + align256(sort_temp_bytes(R)));
}

int z1_embedding_backward(const int64_t* ids, const uint16_t* grad, int64_t R, int64_t D, int64_t V,
                          int64_t padding_idx, float scale, int scale_mode, uint16_t* out, void* workspace,
                          int64_t workspace_bytes, void* stream) {
    if (!out || !workspace || (R > 0 && (!ids || !grad))) return Z1_E_NULL;
    if (R < 0 || R > INT32_MAX || D <= 0 || V <= 0 || V > INT32_MAX - 1) return Z1_E_SIZE;
    if (scale_mode < 0 || scale_mode > 2) return Z1_E_MODE;
    const int64_t need = z1_embedding_backward_workspace(R, V);
    if (need < 0) return (int)need;
    if (workspace_bytes < need) return Z1_E_WORKSPACE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t kb = align256(sizeof(uint32_t) * (size_t)(R > 0 ? R : 1));
    unsigned char* w = static_cast<unsigned char*>(workspace);
    uint32_t* keys = reinterpret_cast<uint32_t*>(w);
    int32_t* vals = reinterpret_cast<int32_t*>(w + kb);
    uint32_t* skeys = reinterpret_cast<uint32_t*>(w + 2 * kb);
    int32_t* svals = reinterpret_cast<int32_t*>(w + 3 * kb);
    int32_t* row_lo = reinterpret_cast<int32_t*>(w + 4 * kb);
    const size_t rl = align256(sizeof(int32_t) * (size_t)(V + 1));
    int* heavy_count = reinterpret_cast<int*>(w + 4 * kb + rl);
    int32_t* heavy_list = reinterpret_cast<int32_t*>(w + 4 * kb + rl + 256);
    void* temp = w + 4 * kb + rl + 256 + align256(sizeof(int32_t) * (size_t)V);
    hipError_t e = hipSuccess;
    if (R > 0) {
        hipLaunchKernelGGL(emb_keys_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, st, ids, R, V, keys,
                           vals);
        e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        size_t tb = sort_temp_bytes(R);
        int end_bit = 1;
        while (end_bit < 32 && ((uint64_t)V >> end_bit) != 0) ++end_bit;   // keys are <= V
        e = hipcub::DeviceRadixSort::SortPairs(temp, tb, keys, skeys, vals, svals, (int)R, 0, end_bit, st);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(emb_row_ranges_kernel, dim3((unsigned)((V + 1 + 255) / 256)), dim3(256), 0, st, skeys, R, V,
                       row_lo, heavy_count);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    const int vec = (D % 8 == 0) && ((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    int dev = 0;
    e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    size_t lds = 0;
    const int rc = z1detail::occupancy_lds(dev, kEmbWgPerCu, &lds);
    if (rc) return rc;
    hipLaunchKernelGGL(emb_rows_kernel, dim3((unsigned)V), dim3(kEmbThreads), lds, st, grad, D, svals, row_lo,
                       padding_idx, scale, scale_mode, vec, out, heavy_count, heavy_list);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    if (vec)
        hipLaunchKernelGGL(emb_heavy_kernel<1>, dim3(kHeavyGrid), dim3(kWave * kHeavyWaves), 0, st, grad, D, svals,
                           row_lo, scale, scale_mode, out, heavy_count, heavy_list);
    else
        hipLaunchKernelGGL(emb_heavy_kernel<0>, dim3(kHeavyGrid), dim3(kWave * kHeavyWaves), 0, st, grad, D, svals,
                           row_lo, scale, scale_mode, out, heavy_count, heavy_list);
    e = hipGetLastError();
    return e == hipSuccess ? Z1_OK : (int)e;
}

}  // extern "C"
