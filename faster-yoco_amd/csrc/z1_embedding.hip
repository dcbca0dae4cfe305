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
//      is written once).  Measured: 4 rows per 256-thread workgroup instead of one wave per row, no difference.
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
                                      int32_t* __restrict__ row_lo) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
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

// One wave per output row t.  scale_mode 0: none; 1: each gradient element first rounded to bf16(g * scale) (the
// CE path scales the staged rows in place, ce_reduce.py:228); 2: the finished bf16 sum multiplied by scale and
// rounded again (layer_graphs.py:93).  vec: D % 8 == 0 and both tables 16-byte aligned (8 columns per lane).
__global__ __launch_bounds__(kEmbThreads) void emb_rows_kernel(const uint16_t* __restrict__ grad, int64_t D,
                                                               const int32_t* __restrict__ spos,
                                                               const int32_t* __restrict__ row_lo,
                                                               int64_t padding_idx, float scale, int scale_mode,
                                                               int vec, uint16_t* __restrict__ out) {
    // row of workgroup b: undoes the round-robin dispatch over the 8 XCDs, so each XCD writes one contiguous
    // eighth of the table (0.148 vs 0.153 ms per call for t = b)
    int64_t t;
    {
        const int64_t b = blockIdx.x, nb = gridDim.x;
        const int64_t x = b & 7, q = b >> 3, Q = nb >> 3, R = nb & 7;
        t = x * Q + (x < R ? x : R) + q;
    }
    uint16_t* orow = out + t * D;
    const int64_t lo = row_lo[t], hi = row_lo[t + 1];
    const bool empty = lo == hi || t == padding_idx;
    if (vec) {
        const int64_t ng = D / 8;
        for (int64_t gi = threadIdx.x; gi < ng; gi += kEmbThreads) {
            u4 o = u4{0u, 0u, 0u, 0u};
            if (!empty) {
                float acc[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
                for (int64_t j0 = lo; j0 < hi; j0 += kRowsPerPartial) {
                    const int64_t j1 = j0 + kRowsPerPartial < hi ? j0 + kRowsPerPartial : hi;
                    float part[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) part[k] = 0.0f;
                    for (int64_t j = j0; j < j1; ++j) {
                        const u4 x = reinterpret_cast<const u4*>(grad + (int64_t)spos[j] * D)[gi];
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            const uint16_t h = (uint16_t)(x[k >> 1] >> ((k & 1) * 16));
                            float v = bf16f(h);
                            if (scale_mode == 1) v = bf16f(bf16r(v * scale));
                            part[k] = part[k] + v;
                        }
                    }
#pragma unroll
                    for (int k = 0; k < 8; ++k) acc[k] = acc[k] + part[k];
                }
#pragma unroll
                for (int k = 0; k < 8; k += 2) {
                    uint16_t a = bf16r(acc[k]), b = bf16r(acc[k + 1]);
                    if (scale_mode == 2) {
                        a = bf16r(bf16f(a) * scale);
                        b = bf16r(bf16f(b) * scale);
                    }
                    o[k >> 1] = (uint32_t)a | ((uint32_t)b << 16);
                }
            }
            // nontemporal: the 616 MB table is written once and not read back here (0.155 vs 0.184 ms per call)
            __builtin_nontemporal_store(o, (__attribute__((address_space(1))) u4*)(reinterpret_cast<u4*>(orow) + gi));
        }
        return;
    }
    for (int64_t d = threadIdx.x; d < D; d += kEmbThreads) {
        uint16_t o = 0;
        if (!empty) {
            float acc = 0.0f;
            for (int64_t j0 = lo; j0 < hi; j0 += kRowsPerPartial) {
                const int64_t j1 = j0 + kRowsPerPartial < hi ? j0 + kRowsPerPartial : hi;
                float part = 0.0f;
                for (int64_t j = j0; j < j1; ++j) {
                    float v = bf16f(grad[(int64_t)spos[j] * D + d]);
                    if (scale_mode == 1) v = bf16f(bf16r(v * scale));
                    part = part + v;
                }
                acc = acc + part;
            }
            o = bf16r(acc);
            if (scale_mode == 2) o = bf16r(bf16f(o) * scale);
        }
        orow[d] = o;
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

int64_t z1_embedding_backward_workspace(int64_t R, int64_t V) {
    if (R < 0 || R > INT32_MAX || V <= 0 || V > INT32_MAX - 1) return Z1_E_SIZE;
    const size_t kb = align256(sizeof(uint32_t) * (size_t)(R > 0 ? R : 1));
    return (int64_t)(4 * kb + align256(sizeof(int32_t) * (size_t)(V + 1)) + align256(sort_temp_bytes(R)));
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
    void* temp = w + 4 * kb + align256(sizeof(int32_t) * (size_t)(V + 1));
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
                       row_lo);
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
                       padding_idx, scale, scale_mode, vec, out);
    e = hipGetLastError();
    return e == hipSuccess ? Z1_OK : (int)e;
}

}  // extern "C"
