// yoco_z1: the owner's token-embedding gradient (declarations: include/yoco_z1.h).
//
// Replaces torch.ops.aten.embedding_dense_backward(g_all, ids, V, padding_idx, False) on the embedding's owner,
// followed or preceded by the x 1/world of the reference (yoco/models/decoder/layer_graphs.py:87-93,
// yoco/models/decoder/ce_reduce.py:226-231).  Same summation order as aten for the row count.  For more than 3072
// indices aten sorts: occurrences of each token id in stable position order, fp32 partial sums over runs of 10
// consecutive occurrences, the partials summed in order, one rounding to bf16.  For fewer its other kernel walks
// the indices in chunks of 16: per chunk and id an fp32 sum in position order, rounded to bf16 and added to the
// bf16 row (emb_rows_kernel<true>; no heavy passes).  padding_idx rows and ids outside [0, V) contribute nothing.
//
//   1. keys[i] = id_i (or V when out of range), vals[i] = i;  2. stable sort by key: hipCUB's radix sort, or,
//      while the stream is being captured into a HIP graph, rocPRIM's merge sort, which clears nothing with
//      memsets (the radix sort does; both are stable, so the order is the same: 0.136 vs 0.142 ms per call);
//   3. row_lo[t] = start of id t's run in the sorted keys (one binary search per t, all in parallel);
//   4. one wave per output row t writes the row's sums -- or zeros -- exactly once, 8 bf16 columns per lane, with
//      nontemporal stores (aten zero-fills the whole table and then scatters into it; here every row of the table
//      is written once), for ids with at most kHeavyRows occurrences; the others are listed, with a slot range
//      for their runs, for
//   5. emb_heavy_parts_kernel, which forms every run partial of every heavy id in parallel over the whole chip
//      into an fp32 workspace, and
//   6. emb_heavy_chain_kernel, which adds each heavy id's partials in run order per column.  Token frequencies in
//      text are skewed: one wave (or one workgroup) walking thousands of occurrences of one id would take
//      milliseconds.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>
#include <rocprim/device/device_merge_sort.hpp>

#include <stdint.h>

#include "yoco_z1.h"
#include "z1_internal.h"

#pragma clang fp contract(off)

namespace {

constexpr int kEmbThreads = 64;                  // one wave per output row
constexpr int kRowsPerPartial = 10;        // aten's NROWS_PER_THREAD
// aten sorts for more than kSortMinRows - 1 indices; for fewer its kernel walks the indices in chunks of
// kFewRowsChunk (torch's ROCm build; checked bit for bit against it on MI355X)
constexpr int64_t kSortMinRows = 3073;
constexpr int kFewRowsChunk = 16;
// resident row workgroups per CU, capped with a dynamic LDS reservation the kernel does not use: 0.131 ms per call
// at 9-10 per CU against 0.148 ms at the 32 the waves allow (0.144 at 16, 0.136 at 8, 0.146 at 7, 0.180 at 6)
constexpr int kEmbWgPerCu = 10;
constexpr int kWave = 64;
// tokens with more occurrences go to the heavy passes; a heavy token's ceil(n / 10) runs are at most n / 7 for
// n >= 21, so the run slots of all heavy tokens number at most R / 7
constexpr int kHeavyRows = 20;
static_assert(kHeavyRows >= 20, "the run-slot bound R / 7 needs heavy tokens of at least 21 occurrences");
constexpr int kPartsThreads = 256;         // heavy pass 1: one run x column group per wave
constexpr int kPartsGrid = 2048;
constexpr int kChainWaves = 16;            // heavy pass 2: waves that load a batch of partials
constexpr int kChainDepth = 16;            // partials per lane per batch
constexpr int kChainRows = kChainWaves * kChainDepth;
static_assert(kChainRows % 16 == 0, "wave 0 reads a batch 16 rows at a time");
constexpr int kChainGrid = 512;
constexpr int kWaveChainRuns = 32;         // heavy tokens of at most this many runs are chained by one wave
constexpr int64_t kMaxCols = 1 << 24;      // D limit: keeps the workspace size and offsets far from overflow

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
                                      int32_t* __restrict__ row_lo, int* __restrict__ counts) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t == 0) {                               // the rows kernel appends the heavy tokens after this kernel
        counts[0] = 0;
        counts[1] = 0;
        counts[2] = 0;
    }
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
// more occurrences is appended, with the first of its nrun run slots (from counts[1]), to the list of tokens of at
// most kWaveChainRuns runs (heavy_list / heavy_base, count counts[0]) or to that of longer ones (long_list /
// long_base, counts[2]); run_start[slot] = the sorted position of the run's first row.  Its row is left to the heavy
// passes.  The atomics only decide where a token's partials are kept, not how they are summed.
template <bool FEW>
__global__ __launch_bounds__(kEmbThreads) void emb_rows_kernel(const uint16_t* __restrict__ grad, int64_t D,
                                                               const int32_t* __restrict__ spos,
                                                               const int32_t* __restrict__ row_lo,
                                                               int64_t padding_idx, float scale, int scale_mode,
                                                               int vec, uint16_t* __restrict__ out,
                                                               int* __restrict__ counts,
                                                               int32_t* __restrict__ heavy_list,
                                                               int32_t* __restrict__ heavy_base,
                                                               int32_t* __restrict__ long_list,
                                                               int32_t* __restrict__ long_base,
                                                               int32_t* __restrict__ run_start) {
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
    constexpr int chunk = kFewRowsChunk;
    if (!FEW && !empty && hi - lo > kHeavyRows) {
        const int nrun = (int)((hi - lo + kRowsPerPartial - 1) / kRowsPerPartial);
        int base = 0;
        if (lane == 0) {
            const bool wave_chain = nrun <= kWaveChainRuns;
            const int h = atomicAdd(&counts[wave_chain ? 0 : 2], 1);
            base = atomicAdd(&counts[1], nrun);
            (wave_chain ? heavy_list : long_list)[h] = (int32_t)t;
            (wave_chain ? heavy_base : long_base)[h] = base;
        }
        base = __shfl(base, 0);
        for (int k = lane; k < nrun; k += kEmbThreads) run_start[base + k] = (int32_t)(lo + (int64_t)k * kRowsPerPartial);
        return;
    }
    if (vec) {
        const int64_t ng = D / 8;
        for (int64_t gi = lane; gi < ng; gi += kEmbThreads) {
            u4 o = u4{0u, 0u, 0u, 0u};
            if constexpr (FEW) {
              if (!empty) {
                // aten's few-indices order: the id's occurrences grouped by index chunk (positions ascend), each
                // group's fp32 sum rounded to bf16 and added to the bf16 row
                float acc[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
                for (int64_t j0 = lo; j0 < hi;) {
                    const int32_t cid = spos[j0] / chunk;
                    int cnt = 1;
                    while (cnt < kFewRowsChunk && j0 + cnt < hi && spos[j0 + cnt] / chunk == cid) ++cnt;
                    u4 x[kFewRowsChunk];
#pragma unroll
                    for (int u = 0; u < kFewRowsChunk; ++u)
                        if (u < cnt) x[u] = reinterpret_cast<const u4*>(grad + (int64_t)spos[j0 + u] * D)[gi];
                    float part[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) part[k] = 0.0f;
#pragma unroll
                    for (int u = 0; u < kFewRowsChunk; ++u) {
                        if (u < cnt) {
#pragma unroll
                            for (int k = 0; k < 8; ++k)
                                part[k] = part[k] + grad_elem((uint16_t)(x[u][k >> 1] >> ((k & 1) * 16)), scale,
                                                              scale_mode);
                        }
                    }
#pragma unroll
                    for (int k = 0; k < 8; ++k) acc[k] = bf16f(bf16r(acc[k] + bf16f(bf16r(part[k]))));
                    j0 += cnt;
                }
#pragma unroll
                for (int k = 0; k < 8; k += 2)
                    o[k >> 1] = (uint32_t)finish(acc[k], scale, scale_mode) |
                                ((uint32_t)finish(acc[k + 1], scale, scale_mode) << 16);
              }
            } else if (!empty) {
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
        if (FEW && !empty) {
            float acc = 0.0f;
            for (int64_t j0 = lo; j0 < hi;) {
                const int32_t cid = spos[j0] / chunk;
                float part = 0.0f;
                int64_t j = j0;
                for (; j < hi && spos[j] / chunk == cid; ++j)
                    part = part + grad_elem(grad[(int64_t)spos[j] * D + d], scale, scale_mode);
                acc = bf16f(bf16r(acc + bf16f(bf16r(part))));
                j0 = j;
            }
            o = finish(acc, scale, scale_mode);
        } else if (!empty) {
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

// Heavy tokens, pass 1: every run of 10 occurrences of every heavy token, for every column group (512 columns on
// the vector path, 64 otherwise), is one wave's item; the wave sums the run's rows in order (loads issued together)
// and stores the fp32 partial to its run slot of parts (parts[s * D + column]).  The run of slot s starts at sorted
// position run_start[s], and its token is the sorted key there.  Items are spread over the whole
// grid, so one token's thousands of runs are formed in parallel; every wave exits once the items run out.
template <int VEC>
__global__ __launch_bounds__(kPartsThreads) void emb_heavy_parts_kernel(const uint16_t* __restrict__ grad, int64_t D,
                                                                        const int32_t* __restrict__ spos,
                                                                        const uint32_t* __restrict__ skeys,
                                                                        const int32_t* __restrict__ row_lo,
                                                                        const int32_t* __restrict__ run_start,
                                                                        const int* __restrict__ counts, float scale,
                                                                        int scale_mode, float* __restrict__ parts) {
    constexpr int kCols = VEC ? 8 : 1;                       // columns per lane
    constexpr int kWaves = kPartsThreads / kWave;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const int64_t cols_per_item = (int64_t)kWave * kCols;
    const int64_t ncg = (D + cols_per_item - 1) / cols_per_item;
    const int64_t items = (int64_t)counts[1] * ncg;
    for (int64_t item = (int64_t)blockIdx.x * kWaves + wave; item < items; item += (int64_t)gridDim.x * kWaves) {
        const int64_t s = item / ncg;
        const int64_t c0 = (item % ncg) * cols_per_item + (int64_t)lane * kCols;   // D % 8 == 0 when VEC
        if (c0 >= D) continue;
        const int64_t j0 = run_start[s];
        const int64_t hi = row_lo[(int64_t)skeys[j0] + 1];
        const int cnt = (int)(j0 + kRowsPerPartial < hi ? kRowsPerPartial : hi - j0);
        float part[kCols];
#pragma unroll
        for (int k = 0; k < kCols; ++k) part[k] = 0.0f;
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
                        part[k] = part[k] + grad_elem((uint16_t)(x[u][k >> 1] >> ((k & 1) * 16)), scale, scale_mode);
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
        float* dst = parts + s * D + c0;
#pragma unroll
        for (int k = 0; k < kCols; ++k) dst[k] = part[k];
    }
}

// Heavy tokens, pass 2: each (heavy token, 64 columns) is an item, one column per lane, whose partials are added in
// run order -- the order of the rows kernel and of aten -- and rounded to the bf16 row.
//   - tokens of more than kWaveChainRuns runs (long_list): workgroup g takes the items g, g + G, ...; per batch its
//     waves load the token's next kChainRows partials into LDS (kChainDepth loads in flight per lane), then wave 0
//     adds them to its accumulator;
//   - the others (heavy_list): wave w of the grid takes the items w, w + W, ..., loads all of the token's partials
//     at once and adds them in registers, with no barrier.
__global__ __launch_bounds__(kWave * kChainWaves) void emb_heavy_chain_kernel(const float* __restrict__ parts,
                                                                             int64_t D,
                                                                             const int32_t* __restrict__ row_lo,
                                                                             const int32_t* __restrict__ heavy_list,
                                                                             const int32_t* __restrict__ heavy_base,
                                                                             const int32_t* __restrict__ long_list,
                                                                             const int32_t* __restrict__ long_base,
                                                                             const int* __restrict__ counts,
                                                                             float scale, int scale_mode,
                                                                             uint16_t* __restrict__ out) {
    __shared__ float buf[kChainRows][kWave];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const int64_t ncg = (D + kWave - 1) / kWave;
    const int64_t long_items = (int64_t)counts[2] * ncg;
    for (int64_t item = blockIdx.x; item < long_items; item += gridDim.x) {
        const int h = (int)(item / ncg);
        const int64_t col = (item % ncg) * kWave + lane;
        const bool valid = col < D;
        const int64_t t = long_list[h];
        const int64_t nrun = (row_lo[t + 1] - row_lo[t] + kRowsPerPartial - 1) / kRowsPerPartial;
        const float* src = parts + (int64_t)long_base[h] * D + col;
        float acc = 0.0f;
        for (int64_t b = 0; b < nrun; b += kChainRows) {
            float x[kChainDepth];
#pragma unroll
            for (int i = 0; i < kChainDepth; ++i) {
                const int64_t k = b + wave + (int64_t)kChainWaves * i;
                x[i] = (k < nrun && valid) ? src[k * D] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < kChainDepth; ++i) buf[wave + kChainWaves * i][lane] = x[i];
            __syncthreads();
            if (wave == 0) {                                   // LDS reads issued 16 at a time, added in order
                const int n = (int)(nrun - b < kChainRows ? nrun - b : kChainRows);
                for (int k0 = 0; k0 < n; k0 += 16) {
                    float y[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) y[i] = buf[k0 + i][lane];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (k0 + i < n) acc = acc + y[i];
                }
            }
            __syncthreads();
        }
        if (wave == 0 && valid) out[t * D + col] = finish(acc, scale, scale_mode);
    }
    const int64_t items = (int64_t)counts[0] * ncg;
    for (int64_t item = (int64_t)blockIdx.x * kChainWaves + wave; item < items;
         item += (int64_t)gridDim.x * kChainWaves) {
        const int h = (int)(item / ncg);
        const int64_t col = (item % ncg) * kWave + lane;
        if (col >= D) continue;
        const int64_t t = heavy_list[h];
        const int nrun = (int)((row_lo[t + 1] - row_lo[t] + kRowsPerPartial - 1) / kRowsPerPartial);
        const float* src = parts + (int64_t)heavy_base[h] * D + col;
        float x[kWaveChainRuns];
#pragma unroll
        for (int k = 0; k < kWaveChainRuns; ++k) x[k] = k < nrun ? src[(int64_t)k * D] : 0.0f;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < kWaveChainRuns; ++k)
            if (k < nrun) acc = acc + x[k];
        out[t * D + col] = finish(acc, scale, scale_mode);
    }
}

// Stable sort of the (key, position) pairs by key: equal keys keep their position order, which is aten's order.
// end_bit bounds the radix sort's passes (keys are at most V); merge selects the sort that records no memset.
hipError_t sort_pairs(void* temp, size_t& bytes, const uint32_t* keys, uint32_t* skeys, const int32_t* vals,
                      int32_t* svals, int64_t R, int end_bit, bool merge, hipStream_t st) {
    if (merge)
        return rocprim::merge_sort(temp, bytes, keys, skeys, vals, svals, (size_t)R, rocprim::less<uint32_t>(), st);
    return hipcub::DeviceRadixSort::SortPairs(temp, bytes, keys, skeys, vals, svals, (int)R, 0, end_bit, st);
}

size_t sort_temp_bytes(int64_t R) {
    size_t radix = 0, merge = 0;
    (void)sort_pairs(nullptr, radix, nullptr, nullptr, nullptr, nullptr, R, 32, false, 0);
    (void)sort_pairs(nullptr, merge, nullptr, nullptr, nullptr, nullptr, R, 32, true, 0);
    return radix > merge ? radix : merge;
}

// Whether work enqueued on `st` is being captured into a graph (an error reads as not capturing).
bool capturing(hipStream_t st) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &status) == hipSuccess && status != hipStreamCaptureStatusNone;
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace: keys, positions, sorted keys, sorted positions (R each), row_lo (V + 1), the three counters, the two
// lists of heavy tokens and their first run slots (at most R / 21 each), the run starts and the fp32 partials (R / 7
// slots, D each), then the sort's temporary storage.
struct EmbWorkspace {
    uint32_t* keys;
    int32_t* vals;
    uint32_t* skeys;
    int32_t* svals;
    int32_t* row_lo;
    int* counts;
    int32_t* heavy_list;
    int32_t* heavy_base;
    int32_t* long_list;
    int32_t* long_base;
    int32_t* run_start;
    float* parts;
    void* temp;
    size_t temp_bytes;
    size_t total;
};

EmbWorkspace emb_workspace(void* base, int64_t R, int64_t D, int64_t V) {
    EmbWorkspace w{};
    unsigned char* p = static_cast<unsigned char*>(base);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        unsigned char* q = p ? p + off : nullptr;
        off += align256(bytes > 0 ? bytes : 1);
        return q;
    };
    const size_t r = (size_t)R, heavy = (size_t)(R / (kHeavyRows + 1)), slots = (size_t)(R / 7);
    w.keys = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * r));
    w.vals = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * r));
    w.skeys = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * r));
    w.svals = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * r));
    w.row_lo = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * (size_t)(V + 1)));
    w.counts = reinterpret_cast<int*>(take(3 * sizeof(int)));
    w.heavy_list = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * heavy));
    w.heavy_base = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * heavy));
    w.long_list = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * heavy));
    w.long_base = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * heavy));
    w.run_start = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * slots));
    w.parts = reinterpret_cast<float*>(take(sizeof(float) * slots * (size_t)D));
    w.temp_bytes = sort_temp_bytes(R);
    w.temp = take(w.temp_bytes);
    w.total = off;
    return w;
}

}  // namespace

extern "C" {

int64_t z1_embedding_backward_workspace(int64_t R, int64_t D, int64_t V) {
    if (R < 0 || R > INT32_MAX || D <= 0 || D > kMaxCols || V <= 0 || V > INT32_MAX - 1) return Z1_E_SIZE;
    return (int64_t)emb_workspace(nullptr, R, D, V).total;
}

int z1_embedding_backward(const int64_t* ids, const uint16_t* grad, int64_t R, int64_t D, int64_t V,
                          int64_t padding_idx, float scale, int scale_mode, uint16_t* out, void* workspace,
                          int64_t workspace_bytes, void* stream) {
    if (!out || !workspace || (R > 0 && (!ids || !grad))) return Z1_E_NULL;
    if (scale_mode < 0 || scale_mode > 2) return Z1_E_MODE;
    const int64_t need = z1_embedding_backward_workspace(R, D, V);
    if (need < 0) return (int)need;
    if (workspace_bytes < need) return Z1_E_WORKSPACE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const EmbWorkspace w = emb_workspace(workspace, R, D, V);
    hipError_t e = hipSuccess;
    if (R > 0) {
        hipLaunchKernelGGL(emb_keys_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, st, ids, R, V, w.keys,
                           w.vals);
        e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        size_t tb = w.temp_bytes;
        int end_bit = 1;
        while (end_bit < 32 && ((uint64_t)V >> end_bit) != 0) ++end_bit;   // keys are <= V
        e = sort_pairs(w.temp, tb, w.keys, w.skeys, w.vals, w.svals, R, end_bit, capturing(st), st);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(emb_row_ranges_kernel, dim3((unsigned)((V + 1 + 255) / 256)), dim3(256), 0, st, w.skeys, R, V,
                       w.row_lo, w.counts);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    const int vec = (D % 8 == 0) && ((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    int dev = 0;
    e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    size_t lds = 0;
    const int rc = z1detail::occupancy_lds(dev, kEmbWgPerCu, &lds);
    if (rc) return rc;
    if (R < kSortMinRows)   // aten's kernel for few indices: its order, no heavy passes (nothing is listed for them)
        hipLaunchKernelGGL(emb_rows_kernel<true>, dim3((unsigned)V), dim3(kEmbThreads), lds, st, grad, D, w.svals,
                           w.row_lo, padding_idx, scale, scale_mode, vec, out, w.counts, w.heavy_list, w.heavy_base,
                           w.long_list, w.long_base, w.run_start);
    else
        hipLaunchKernelGGL(emb_rows_kernel<false>, dim3((unsigned)V), dim3(kEmbThreads), lds, st, grad, D, w.svals,
                           w.row_lo, padding_idx, scale, scale_mode, vec, out, w.counts, w.heavy_list, w.heavy_base,
                           w.long_list, w.long_base, w.run_start);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    if (vec)
        hipLaunchKernelGGL(emb_heavy_parts_kernel<1>, dim3(kPartsGrid), dim3(kPartsThreads), 0, st, grad, D, w.svals,
                           w.skeys, w.row_lo, w.run_start, w.counts, scale, scale_mode, w.parts);
    else
        hipLaunchKernelGGL(emb_heavy_parts_kernel<0>, dim3(kPartsGrid), dim3(kPartsThreads), 0, st, grad, D, w.svals,
                           w.skeys, w.row_lo, w.run_start, w.counts, scale, scale_mode, w.parts);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(emb_heavy_chain_kernel, dim3(kChainGrid), dim3(kWave * kChainWaves), 0, st, w.parts, D,
                       w.row_lo, w.heavy_list, w.heavy_base, w.long_list, w.long_base, w.counts, scale, scale_mode,
                       out);
    e = hipGetLastError();
    return e == hipSuccess ? Z1_OK : (int)e;
}

}  // extern "C"
