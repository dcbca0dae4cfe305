/*
 * The path's kernels as PyTorch operators, namespace yoco_z1: the schemas, the CUDA (HIP) kernels -- argument checks,
 * table binding and one call of the C ABI of libyoco_z1.so on torch's current stream -- and CPU kernels that only
 * raise (there is no CPU implementation).  Host code only; built with the host compiler against torch's headers into
 * libyoco_z1_torch.so.
 *
 * The C ABI is not linked: z1t_init(path) resolves its functions from the libyoco_z1.so the process has already
 * loaded (the Python side loads it first, so a caller may select another build of the same ABI).
 *
 * Tables: a table (z1_table*, passed to the operators as an int) is registered here by the code that created it
 * (z1t_table_register: row sizes, the flat form's element offsets, the pointers the device copy holds).  An operator
 * over a table receives the tensors of its call, one list per stream (g, p, m, v, p16): one flat buffer each for a
 * flat table, one tensor per row for a list table, an empty p16 list for no BF16 copies.  It computes the rows'
 * addresses, and when they differ from what the device table holds, enqueues z1_table_set_grads (only gradients
 * moved) or z1_table_rebind before the launch.  That is how one table serves gradients that autograd reallocates,
 * and the copies of mutable arguments that torch's functionalization may pass to an operator.
 *
 * The operators replace the reference's Triton launches (yoco/tasks/fused_adam_cast.py:68-70,88-89,
 * yoco/models/decoder/ce_reduce.py:182) and the torch scalar ops of the norm and clip chain
 * (yoco/tasks/zero1_fast.py:150-160, yoco/tasks/trainer_nosync.py:273-286).
 */
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/library.h>

#include <dlfcn.h>

#include <algorithm>
#include <array>
#include <cstdint>
#include <mutex>
#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

#include "yoco_z1.h"

namespace {

using at::Tensor;
using at::TensorList;
using OptTensor = std::optional<Tensor>;

// ------------------------------------------------------------------------------------------ the C ABI, resolved
struct Api {
    decltype(&::z1_table_set_grads) table_set_grads;
    decltype(&::z1_table_rebind) table_rebind;
    decltype(&::z1_table_set_grad_out) table_set_grad_out;
    decltype(&::z1_owner_sum_bf16) owner_sum_bf16;
    decltype(&::z1_owner_sum_workspace) owner_sum_workspace;
    decltype(&::z1_owner_sum_update) owner_sum_update;
    decltype(&::z1_owner_sum_bf16_waves) owner_sum_bf16_waves;
    decltype(&::z1_owner_sum_waves) owner_sum_waves;
    decltype(&::z1_reduce_waves) reduce_waves;
    decltype(&::z1_grad_sumsq) grad_sumsq;
    decltype(&::z1_update_scalars_run) update_scalars_run;
    decltype(&::z1_grad_update_scalars) grad_update_scalars;
    decltype(&::z1_clip_factor) clip_factor;
    decltype(&::z1_adam_cast) adam_cast;
    decltype(&::z1_adam_cast_dev) adam_cast_dev;
    decltype(&::z1_adam_cast_rows) adam_cast_rows;
    decltype(&::z1_bias_corrections_step) bias_corrections_step;
    decltype(&::z1_scale_up) scale_up;
    decltype(&::z1_cast_bf16) cast_bf16;
    decltype(&::z1_embedding_backward) embedding_backward;
    decltype(&::z1_embedding_backward_workspace) embedding_backward_workspace;
    decltype(&::z1_strerror) strerror;
};

Api g_api{};
bool g_api_ok = false;
std::mutex g_mu;   // guards g_api set-up, the table registry and every bind + launch over a table

const Api& api() {
    TORCH_CHECK(g_api_ok, "yoco_z1: the operators are not bound to libyoco_z1.so (import faster_yoco_amd.library)");
    return g_api;
}

void check_rc(int rc, const char* what) {
    if (rc != 0) {
        const char* s = g_api.strerror ? g_api.strerror(rc) : nullptr;
        TORCH_CHECK(false, "yoco_z1: ", what, " failed: ", s ? s : "?", " (code ", rc, ")");
    }
}

void* stream_of(int device) {
    return static_cast<void*>(c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream());
}

c10::Device cuda(int device) { return c10::Device(c10::DeviceType::CUDA, static_cast<c10::DeviceIndex>(device)); }

// ------------------------------------------------------------------------------------------ argument checks
const char* dtype_name(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return "fp32";
        case at::kBFloat16: return "bf16";
        case at::kDouble: return "float64";
        default: return c10::toString(t);
    }
}

void require_gpu(const Tensor& t, const char* what) {
    TORCH_CHECK(t.defined() && t.is_cuda(), what, ": expected a GPU tensor (there is no CPU path)");
}

void* ptr(const OptTensor& t) { return t.has_value() && t->defined() ? t->data_ptr() : nullptr; }

// Every tensor a launch reads or writes must live on the launch's device: a pointer into another GPU's memory would
// reach the kernel unchecked.
void require_on(const Tensor& t, int device, const char* what) {
    require_gpu(t, what);
    TORCH_CHECK(t.device().index() == device, what, ": a tensor is on cuda:", static_cast<int>(t.device().index()),
                ", the launch runs on cuda:", device);
}

float* scalar_ptr(const OptTensor& t, const char* what, int device) {
    if (!t.has_value() || !t->defined()) return nullptr;
    require_on(*t, device, what);
    TORCH_CHECK(t->scalar_type() == at::kFloat && t->numel() == 1, what, ": expected a 1-element fp32 device tensor");
    return static_cast<float*>(t->data_ptr());
}

double* partials_ptr(const Tensor& t, const char* what, int device, int64_t need = Z1_NORM_PARTIALS) {
    require_on(t, device, what);
    TORCH_CHECK(t.scalar_type() == at::kDouble && t.numel() >= need && t.is_contiguous(),
                "yoco_z1: the norm workspace must hold ", need, " float64");
    return static_cast<double*>(t.data_ptr());
}

// z1_update_scalars: the factor is read from `factor` (in place) unless factor_value is given; then `factor`, if
// given, only receives the clipped value.
z1_update_scalars scalars(const char* what, int device, const OptTensor& factor, std::optional<double> factor_value,
                          const OptTensor& norm, const OptTensor& grad_norm, const OptTensor& flags,
                          const OptTensor& clip_log, const OptTensor& sample_size, double numer, double max_norm) {
    uint8_t* fl = nullptr;
    if (flags.has_value() && flags->defined()) {
        require_on(*flags, device, what);
        TORCH_CHECK((flags->scalar_type() == at::kByte || flags->scalar_type() == at::kBool) && flags->numel() >= 2,
                    what, ": flags must hold 2 uint8/bool");
        fl = static_cast<uint8_t*>(flags->data_ptr());
    }
    z1_update_scalars u;
    u.sample_size = scalar_ptr(sample_size, what, device);
    u.numer = static_cast<float>(numer);
    u.factor_in = factor_value.has_value() ? nullptr : scalar_ptr(factor, what, device);
    u.factor_value = factor_value.has_value() ? static_cast<float>(*factor_value) : 1.0f;
    u.max_norm = static_cast<float>(max_norm);
    u.norm_out = scalar_ptr(norm, what, device);
    u.grad_norm_out = scalar_ptr(grad_norm, what, device);
    u.factor_out = scalar_ptr(factor, what, device);
    u.flags_out = fl;
    u.clip_log_out = scalar_ptr(clip_log, what, device);
    return u;
}

// ------------------------------------------------------------------------------------------ tables
using Bound = std::array<uintptr_t, 6>;   // (g, p, m, v, p16, FP32 gradient output) of one row
constexpr uintptr_t kUnknown = ~static_cast<uintptr_t>(0);   // a binding no call can match: rebind at the next call

struct TableState {
    z1_table* h = nullptr;
    int device = 0;
    int gdtype = Z1_F32;
    bool has_pmv = false;
    bool flat = false;
    std::vector<int64_t> sizes;
    std::vector<int64_t> offsets;                    // flat form: element offset of each row in its buffers
    int64_t flat_need = 0;                           // flat form: elements a buffer must hold
    std::vector<Bound> bound;                        // per row, what the device table holds once the launches
                                                     // enqueued so far have run (kUnknown: not known)
    void* last_stream = nullptr;                     // the stream of the table's last eager launch
    hipEvent_t handoff = nullptr;                    // orders a call on another stream after that stream's work
};

std::unordered_map<uintptr_t, TableState> g_tables;

TableState& table_of(int64_t handle) {
    auto it = g_tables.find(static_cast<uintptr_t>(handle));
    TORCH_CHECK(it != g_tables.end(), "yoco_z1: no live table with handle 0x", std::hex, handle);
    return it->second;
}

at::ScalarType column_dtype(const TableState& t, int k) {
    if (k == 0) return t.gdtype == Z1_F32 ? at::kFloat : at::kBFloat16;
    return k == 4 ? at::kBFloat16 : at::kFloat;
}

// Columns that may be left empty: the BF16 copies (4) and the FP32 gradient outputs (5).
bool optional_column(int k) { return k >= 4; }

void check_member(const TableState& t, const Tensor& x, at::ScalarType dt, const char* what) {
    require_gpu(x, what);
    TORCH_CHECK(x.device().index() == t.device, what, ": a tensor is on another device than its table");
    TORCH_CHECK(x.scalar_type() == dt && x.is_contiguous(), what, ": expected contiguous ", dtype_name(dt),
                " tensors");
}

// Per-row addresses of stream k (0 g, 1 p, 2 m, 3 v, 4 p16, 5 FP32 gradient output) for the tensors of a call.
void column(const TableState& t, TensorList lst, int k, const char* what, std::vector<uintptr_t>& col) {
    const size_t nr = t.sizes.size();
    const at::ScalarType dt = column_dtype(t, k);
    col.assign(nr, 0);
    if (lst.empty()) {
        TORCH_CHECK(optional_column(k), what, ": a gradient, master or moment list is empty");
        return;                                       // no BF16 copies / no gradient outputs
    }
    if (t.flat) {
        TORCH_CHECK(lst.size() == 1, what, ": a flat table takes one buffer per stream");
        const Tensor& b = lst[0];
        check_member(t, b, dt, what);
        TORCH_CHECK(b.numel() >= t.flat_need, what, ": a flat buffer holds ", b.numel(), " elements, the table needs ",
                    t.flat_need);
        const uintptr_t base = reinterpret_cast<uintptr_t>(b.data_ptr());
        const size_t es = b.element_size();
        for (size_t i = 0; i < nr; ++i) col[i] = base + static_cast<uintptr_t>(t.offsets[i]) * es;
        return;
    }
    TORCH_CHECK(lst.size() == nr, what, ": expected one tensor per table row (", nr, "), got ", lst.size());
    for (size_t i = 0; i < nr; ++i) {
        const Tensor& x = lst[i];
        if (optional_column(k) && x.numel() == 0) continue;      // none for this row
        check_member(t, x, dt, what);
        TORCH_CHECK(x.numel() == t.sizes[i], what, ": row ", i, " has ", x.numel(), " elements, the table ",
                    t.sizes[i]);
        col[i] = reinterpret_cast<uintptr_t>(x.data_ptr());
    }
}

bool capturing(void* stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(static_cast<hipStream_t>(stream), &st) == hipSuccess &&
           st != hipStreamCaptureStatusNone;
}

void forget_binding(TableState& t) {
    for (Bound& b : t.bound) b.fill(kUnknown);
}

// Orders this call after everything already enqueued on the stream the table was last launched on, when that is
// another stream: the device rows are shared by every launch over the table, and the rebind this call may enqueue
// must not rewrite them under a launch still running there (an event recorded on that stream now, waited for on
// this one; no host synchronisation).  The reference has no such shared state: each of its launches carries its own
// pointers (yoco/tasks/fused_adam_cast.py:68-70).
void order_after_last_stream(TableState& t, void* stream) {
    if (t.last_stream == nullptr || t.last_stream == stream) return;
    hipError_t e = hipSuccess;
    if (!t.handoff) e = hipEventCreateWithFlags(&t.handoff, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(t.handoff, static_cast<hipStream_t>(t.last_stream));
    if (e == hipSuccess) e = hipStreamWaitEvent(static_cast<hipStream_t>(stream), t.handoff, 0);
    TORCH_CHECK(e == hipSuccess, "yoco_z1: ordering a table's call after its previous stream failed: ",
                hipGetErrorString(e));
}

// Points the device table at the call's tensors, enqueuing a rebind on the stream only when an address moved.
// pmv16: the p, m, v, p16 lists, or nullptr to keep their binding; gout: the FP32 gradient outputs (an empty list:
// none), or nullptr to keep them (the norm reads no output).
//
// Under stream capture the call always enqueues the binding of every column it reads (the gradients for the norm;
// every column, and the outputs when given, for Adam), so that each replay of the graph points the table at the
// tensors it was captured with, whatever eager calls did to the table in between; those columns of the recorded
// binding are then forgotten, so the next eager call rebinds them too.  A failed binding launch forgets the whole
// binding (the device rows may be half rewritten).
void bind(TableState& t, TensorList g, const TensorList* pmv16, const TensorList* gout, const char* what,
          void* stream) {
    const size_t nr = t.sizes.size();
    if (nr == 0) return;
    const bool cap = capturing(stream);
    thread_local std::vector<uintptr_t> cols[6];
    column(t, g, 0, what, cols[0]);
    for (int k = 1; k < 6; ++k) {
        const TensorList* given = k < 5 ? (pmv16 ? &pmv16[k - 1] : nullptr) : gout;
        if (given) {
            column(t, *given, k, what, cols[k]);
        } else {                                      // a column this call does not read: left as bound
            cols[k].resize(nr);
            for (size_t i = 0; i < nr; ++i) cols[k][i] = t.bound[i][k];
        }
    }
    if (t.has_pmv && pmv16) {
        for (size_t i = 0; i < nr; ++i)
            TORCH_CHECK(t.sizes[i] == 0 || (cols[1][i] && cols[2][i] && cols[3][i]), what,
                        ": the table updates masters and moments; every row needs p, m and v");
    }
    if (!cap) order_after_last_stream(t, stream);
    bool moved = cap, others = cap && pmv16 != nullptr, outs = cap && gout != nullptr;
    for (size_t i = 0; i < nr; ++i) {
        moved |= cols[0][i] != t.bound[i][0];
        for (int k = 1; k < 5; ++k) others |= cols[k][i] != t.bound[i][k];
        outs |= gout != nullptr && cols[5][i] != t.bound[i][5];
    }
    try {
        if (moved && !others) {
            thread_local std::vector<const void*> gp;
            gp.assign(nr, nullptr);
            for (size_t i = 0; i < nr; ++i) gp[i] = reinterpret_cast<const void*>(cols[0][i]);
            check_rc(api().table_set_grads(t.h, gp.data(), static_cast<int>(nr), stream), "z1_table_set_grads");
        } else if (others) {
            thread_local std::vector<z1_tensor> rows;
            rows.resize(nr);
            for (size_t i = 0; i < nr; ++i) {
                rows[i].g = reinterpret_cast<const void*>(cols[0][i]);
                rows[i].p = reinterpret_cast<float*>(cols[1][i]);
                rows[i].m = reinterpret_cast<float*>(cols[2][i]);
                rows[i].v = reinterpret_cast<float*>(cols[3][i]);
                rows[i].p16 = reinterpret_cast<uint16_t*>(cols[4][i]);
                rows[i].n = t.sizes[i];
            }
            check_rc(api().table_rebind(t.h, rows.data(), static_cast<int>(nr), stream), "z1_table_rebind");
        }
        if (outs) {
            bool any = false;
            thread_local std::vector<float*> op;
            op.assign(nr, nullptr);
            for (size_t i = 0; i < nr; ++i) {
                op[i] = reinterpret_cast<float*>(cols[5][i]);
                any |= op[i] != nullptr;
            }
            check_rc(api().table_set_grad_out(t.h, any ? op.data() : nullptr, static_cast<int>(nr), stream),
                     "z1_table_set_grad_out");
        }
    } catch (...) {
        forget_binding(t);
        throw;
    }
    if (cap) {
        for (size_t i = 0; i < nr; ++i) {
            t.bound[i][0] = kUnknown;
            if (pmv16)
                for (int k = 1; k < 5; ++k) t.bound[i][k] = kUnknown;
            if (gout) t.bound[i][5] = kUnknown;
        }
        return;
    }
    for (size_t i = 0; i < nr; ++i)
        for (int k = 0; k < 5; ++k) t.bound[i][k] = cols[k][i];
    if (gout)
        for (size_t i = 0; i < nr; ++i) t.bound[i][5] = cols[5][i];
    t.last_stream = stream;
}

// A table operator's frame: the registry lock, the table, its device current, torch's current stream there.
struct OnTable {
    std::lock_guard<std::mutex> lock;
    TableState& t;
    c10::DeviceGuard guard;
    void* stream;
    explicit OnTable(int64_t handle)
        : lock(g_mu), t(table_of(handle)), guard(cuda(t.device)), stream(stream_of(t.device)) {}
};

// A tensor operator's frame: `anchor`'s device current, torch's current stream there.
struct OnDevice {
    c10::DeviceGuard guard;
    void* stream;
    explicit OnDevice(const Tensor& anchor)
        : guard(anchor.device()), stream(stream_of(anchor.device().index())) {}
};

// ------------------------------------------------------------------------------------------ norm and clip chain
void grad_sumsq_(int64_t table, TensorList g, const Tensor& partials) {
    OnTable on(table);
    double* part = partials_ptr(partials, "grad_sumsq", on.t.device);
    bind(on.t, g, nullptr, nullptr, "grad_sumsq", on.stream);
    check_rc(api().grad_sumsq(on.t.h, part, on.stream), "z1_grad_sumsq");
}

void norm_clip_(const Tensor& partials, const OptTensor& factor, const OptTensor& norm, const OptTensor& grad_norm,
                double max_norm, std::optional<double> factor_value) {
    require_gpu(partials, "norm_clip");
    OnDevice on(partials);
    const int dev = partials.device().index();
    double* part = partials_ptr(partials, "norm_clip", dev);
    z1_update_scalars u = scalars("norm_clip", dev, factor, factor_value, norm, grad_norm, std::nullopt, std::nullopt,
                                  std::nullopt, 1.0, max_norm);
    check_rc(api().update_scalars_run(part, &u, on.stream), "z1_norm_clip");
}

void grad_norm_clip_(int64_t table, TensorList g, const Tensor& partials, const OptTensor& factor,
                     const OptTensor& norm, const OptTensor& grad_norm, double max_norm,
                     std::optional<double> factor_value) {
    OnTable on(table);
    double* part = partials_ptr(partials, "grad_norm_clip", on.t.device);
    z1_update_scalars u = scalars("grad_norm_clip", on.t.device, factor, factor_value, norm, grad_norm, std::nullopt,
                                  std::nullopt, std::nullopt, 1.0, max_norm);
    bind(on.t, g, nullptr, nullptr, "grad_norm_clip", on.stream);
    check_rc(api().grad_update_scalars(on.t.h, part, &u, on.stream), "z1_grad_norm_clip");
}

void update_scalars_(const Tensor& partials, const OptTensor& factor, const OptTensor& norm,
                     const OptTensor& grad_norm, const OptTensor& flags, const OptTensor& clip_log,
                     const OptTensor& sample_size, double numer, double max_norm,
                     std::optional<double> factor_value) {
    require_gpu(partials, "update_scalars");
    OnDevice on(partials);
    const int dev = partials.device().index();
    double* part = partials_ptr(partials, "update_scalars", dev);
    z1_update_scalars u = scalars("update_scalars", dev, factor, factor_value, norm, grad_norm, flags, clip_log,
                                  sample_size, numer, max_norm);
    check_rc(api().update_scalars_run(part, &u, on.stream), "z1_update_scalars");
}

void grad_update_scalars_(int64_t table, TensorList g, const Tensor& partials, const OptTensor& factor,
                          const OptTensor& norm, const OptTensor& grad_norm, const OptTensor& flags,
                          const OptTensor& clip_log, const OptTensor& sample_size, double numer, double max_norm,
                          std::optional<double> factor_value) {
    OnTable on(table);
    double* part = partials_ptr(partials, "grad_update_scalars", on.t.device);
    z1_update_scalars u = scalars("grad_update_scalars", on.t.device, factor, factor_value, norm, grad_norm, flags,
                                  clip_log, sample_size, numer, max_norm);
    bind(on.t, g, nullptr, nullptr, "grad_update_scalars", on.stream);
    check_rc(api().grad_update_scalars(on.t.h, part, &u, on.stream), "z1_grad_update_scalars");
}

void clip_factor_(const Tensor& norm, const OptTensor& factor, const OptTensor& grad_norm, double max_norm,
                  std::optional<double> factor_value) {
    require_gpu(norm, "clip_factor");
    OnDevice on(norm);
    const int dev = norm.device().index();
    float* nr = scalar_ptr(norm, "clip_factor", dev);
    const float* fin = factor_value.has_value() ? nullptr : scalar_ptr(factor, "clip_factor", dev);
    const float fval = factor_value.has_value() ? static_cast<float>(*factor_value) : 1.0f;
    check_rc(api().clip_factor(nr, fin, fval, scalar_ptr(grad_norm, "clip_factor", dev),
                               scalar_ptr(factor, "clip_factor", dev), static_cast<float>(max_norm), on.stream),
             "z1_clip_factor");
}

// ------------------------------------------------------------------------------------------ Adam + BF16
// Adam + BF16 over rows [row_begin, row_end); with g32 (one FP32 tensor per row, or one flat buffer; an empty
// list: none) the launch also writes each element's g' = fp32(g * factor) there.
void adam_cast_impl(int64_t table, TensorList g, TensorList p, TensorList m, TensorList v, TensorList p16,
                    TensorList g32, const OptTensor& factor, double lr, double beta1, double beta2, double eps,
                    double bc1, double bc2, double weight_decay, int64_t adam_mode, int64_t row_begin,
                    int64_t row_end) {
    OnTable on(table);
    TableState& t = on.t;
    float* fac = scalar_ptr(factor, "adam_cast", t.device);
    TORCH_CHECK(t.has_pmv, "yoco_z1: adam_cast needs a table with p, m and v");
    const int64_t nr = static_cast<int64_t>(t.sizes.size());
    TORCH_CHECK(0 <= row_begin && row_begin <= row_end && row_end <= nr, "yoco_z1: rows [", row_begin, ", ", row_end,
                ") outside the table's ", nr, " rows");
    const TensorList rest[4] = {p, m, v, p16};
    bind(t, g, rest, &g32, "adam_cast", on.stream);
    if (row_begin == 0 && row_end == nr) {
        check_rc(api().adam_cast(t.h, fac, static_cast<float>(lr), static_cast<float>(beta1),
                                 static_cast<float>(beta2), static_cast<float>(eps), static_cast<float>(bc1),
                                 static_cast<float>(bc2), static_cast<float>(weight_decay),
                                 static_cast<int>(adam_mode), on.stream), "z1_adam_cast");
    } else {
        check_rc(api().adam_cast_rows(t.h, static_cast<int>(row_begin), static_cast<int>(row_end), fac,
                                      static_cast<float>(lr), static_cast<float>(beta1), static_cast<float>(beta2),
                                      static_cast<float>(eps), static_cast<float>(bc1), static_cast<float>(bc2),
                                      static_cast<float>(weight_decay), static_cast<int>(adam_mode), on.stream),
                 "z1_adam_cast_rows");
    }
}

void adam_cast_(int64_t table, TensorList g, TensorList p, TensorList m, TensorList v, TensorList p16,
                const OptTensor& factor, double lr, double beta1, double beta2, double eps, double bc1, double bc2,
                double weight_decay, int64_t adam_mode, int64_t row_begin, int64_t row_end) {
    adam_cast_impl(table, g, p, m, v, p16, TensorList(), factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay,
                   adam_mode, row_begin, row_end);
}

void adam_cast_gout_(int64_t table, TensorList g, TensorList p, TensorList m, TensorList v, TensorList p16,
                     TensorList g32, const OptTensor& factor, double lr, double beta1, double beta2, double eps,
                     double bc1, double bc2, double weight_decay, int64_t adam_mode, int64_t row_begin,
                     int64_t row_end) {
    adam_cast_impl(table, g, p, m, v, p16, g32, factor, lr, beta1, beta2, eps, bc1, bc2, weight_decay, adam_mode,
                   row_begin, row_end);
}

void adam_cast_dev_(int64_t table, TensorList g, TensorList p, TensorList m, TensorList v, TensorList p16,
                    const OptTensor& factor, const Tensor& bc, double lr, double beta1, double beta2, double eps,
                    double weight_decay, int64_t adam_mode) {
    OnTable on(table);
    TableState& t = on.t;
    float* fac = scalar_ptr(factor, "adam_cast_dev", t.device);
    require_on(bc, t.device, "adam_cast_dev");
    TORCH_CHECK(bc.scalar_type() == at::kFloat && bc.numel() >= 2 && bc.is_contiguous(),
                "yoco_z1: bias corrections must be a contiguous 2-element fp32 tensor");
    TORCH_CHECK(t.has_pmv, "yoco_z1: adam_cast_dev needs a table with p, m and v");
    const TensorList rest[4] = {p, m, v, p16};
    const TensorList none;
    bind(t, g, rest, &none, "adam_cast_dev", on.stream);
    check_rc(api().adam_cast_dev(t.h, fac, static_cast<float>(lr), static_cast<float>(beta1),
                                 static_cast<float>(beta2), static_cast<float>(eps),
                                 static_cast<const float*>(bc.data_ptr()), static_cast<float>(weight_decay),
                                 static_cast<int>(adam_mode), on.stream), "z1_adam_cast_dev");
}

void bias_corrections_step_(const Tensor& step, const Tensor& bc, double beta1, double beta2,
                            int64_t bias_correction) {
    require_gpu(step, "bias_corrections_step");
    require_gpu(bc, "bias_corrections_step");
    TORCH_CHECK(step.scalar_type() == at::kLong && step.numel() >= 1 && bc.scalar_type() == at::kFloat &&
                bc.numel() >= 2 && bc.is_contiguous() && step.device() == bc.device(),
                "yoco_z1: bias_corrections_step takes an int64 step and a contiguous 2-element fp32 bc on one device");
    OnDevice on(step);
    check_rc(api().bias_corrections_step(static_cast<int64_t*>(step.data_ptr()), beta1, beta2,
                                         static_cast<int>(bias_correction), static_cast<float*>(bc.data_ptr()),
                                         on.stream), "z1_bias_corrections_step");
}

// ------------------------------------------------------------------------------------------ owner sum
// Checked contribution pointers of an owner-sum call (at most Z1_MAX_WORLD).
int contributions(TensorList contribs, const Tensor& out, const OptTensor& out_sum, const uint16_t** ptrs) {
    require_gpu(out, "owner_sum");
    TORCH_CHECK(out.scalar_type() == at::kBFloat16 && out.is_contiguous(),
                "yoco_z1: owner_sum output must be a contiguous bf16 tensor");
    const int world = static_cast<int>(contribs.size());
    TORCH_CHECK(1 <= world && world <= Z1_MAX_WORLD, "yoco_z1: owner_sum takes 1..", Z1_MAX_WORLD,
                " contributions, got ", world);
    for (int k = 0; k < world; ++k) {
        const Tensor& c = contribs[k];
        require_gpu(c, "owner_sum");
        TORCH_CHECK(c.scalar_type() == at::kBFloat16 && c.is_contiguous() && c.numel() == out.numel() &&
                    c.device() == out.device(),
                    "yoco_z1: owner_sum contributions must be contiguous bf16 tensors like out");
        TORCH_CHECK(out.numel() == 0 || c.data_ptr() != out.data_ptr(),
                    "yoco_z1: owner_sum: out must not be one of the contributions (sum_slots_ is the in-place form)");
        ptrs[k] = static_cast<const uint16_t*>(c.data_ptr());
    }
    if (out_sum.has_value() && out_sum->defined()) {
        require_gpu(*out_sum, "owner_sum");
        TORCH_CHECK(out_sum->scalar_type() == at::kFloat && out_sum->is_contiguous() &&
                    out_sum->numel() == out.numel() && out_sum->device() == out.device(),
                    "yoco_z1: owner_sum out_sum must be a contiguous fp32 tensor like out");
    }
    return world;
}

void owner_sum_(TensorList contribs, const Tensor& out, double scale, const OptTensor& out_sum,
                const OptTensor& partials) {
    const uint16_t* ptrs[Z1_MAX_WORLD];
    const int world = contributions(contribs, out, out_sum, ptrs);
    double* part = nullptr;
    if (partials.has_value() && partials->defined())
        part = partials_ptr(*partials, "owner_sum", out.device().index(), api().owner_sum_workspace(out.numel()));
    OnDevice on(out);
    check_rc(api().owner_sum_bf16(ptrs, world, out.numel(), static_cast<float>(scale),
                                  static_cast<uint16_t*>(out.data_ptr()), static_cast<float*>(ptr(out_sum)), part,
                                  on.stream), "z1_owner_sum_bf16");
}

void owner_sum_update_(TensorList contribs, const Tensor& out, const Tensor& workspace, double scale,
                       const OptTensor& out_sum, const OptTensor& factor, const OptTensor& norm,
                       const OptTensor& grad_norm, const OptTensor& flags, const OptTensor& clip_log,
                       const OptTensor& sample_size, double numer, double max_norm,
                       std::optional<double> factor_value) {
    const uint16_t* ptrs[Z1_MAX_WORLD];
    const int world = contributions(contribs, out, out_sum, ptrs);
    const int dev = out.device().index();
    double* ws = partials_ptr(workspace, "owner_sum", dev, api().owner_sum_workspace(out.numel()));
    z1_update_scalars u = scalars("owner_sum_update", dev, factor, factor_value, norm, grad_norm, flags, clip_log,
                                  sample_size, numer, max_norm);
    OnDevice on(out);
    check_rc(api().owner_sum_update(ptrs, world, out.numel(), static_cast<float>(scale),
                                    static_cast<uint16_t*>(out.data_ptr()), static_cast<float*>(ptr(out_sum)), ws, &u,
                                    on.stream), "z1_owner_sum_update");
}

// The owner sum in the reference's staging layout (yoco/models/decoder/ce_reduce.py:59-74): the contribution of
// peer k < rank in slot k of `staging`, of k > rank in slot k - 1, rank's own in `out`, summed in rank order into
// out[base:end].  With `waves` (at least z1_owner_sum_waves(end - base) float64), the norm of the range's average
// is left there per chunk (z1_owner_sum_bf16_waves), for reduce_waves_.
void sum_slots_(const Tensor& staging, const Tensor& out, int64_t G, int64_t base, int64_t end, int64_t rank,
                double scale, int64_t world, const OptTensor& waves) {
    TORCH_CHECK(staging.defined() && staging.is_cuda() && staging.scalar_type() == at::kBFloat16 &&
                staging.is_contiguous(), "ce_reduce: staging must be a contiguous bf16 GPU tensor");
    TORCH_CHECK(out.defined() && out.is_cuda() && out.scalar_type() == at::kBFloat16 && out.is_contiguous(),
                "ce_reduce: out must be a contiguous bf16 GPU tensor");
    TORCH_CHECK(staging.device() == out.device(), "ce_reduce: staging and out must be on one device");
    TORCH_CHECK(1 <= world && world <= Z1_MAX_WORLD && 0 <= rank && rank < world, "ce_reduce: rank ", rank,
                " / world ", world, " out of range");
    TORCH_CHECK(0 <= base && base <= end && end <= G && out.numel() >= G && staging.numel() >= (world - 1) * G,
                "ce_reduce: range [", base, ", ", end, ") does not fit G=", G, ", out ", out.numel(), ", staging ",
                staging.numel());
    double* wp = nullptr;
    if (waves.has_value() && waves->defined())
        wp = partials_ptr(*waves, "sum_slots", out.device().index(), api().owner_sum_waves(end - base));
    if (end == base) return;
    const uint16_t* s0 = static_cast<const uint16_t*>(staging.data_ptr());
    uint16_t* o0 = static_cast<uint16_t*>(out.data_ptr());
    const uint16_t* ptrs[Z1_MAX_WORLD];
    for (int64_t k = 0; k < world; ++k)
        ptrs[k] = k < rank ? s0 + k * G + base : (k == rank ? o0 + base : s0 + (k - 1) * G + base);
    OnDevice on(out);
    check_rc(api().owner_sum_bf16_waves(ptrs, static_cast<int>(world), end - base, static_cast<float>(scale),
                                        o0 + base, nullptr, wp, on.stream), "z1_owner_sum_bf16_waves");
}

// The fixed-order reduction of per-chunk norm partials (the first m of `waves`) into the norm's partials.
void reduce_waves_(const Tensor& waves, int64_t m, const Tensor& partials) {
    require_gpu(partials, "reduce_waves");
    const int dev = partials.device().index();
    TORCH_CHECK(m >= 0, "yoco_z1: reduce_waves: negative count");
    double* wp = partials_ptr(waves, "reduce_waves", dev, m);
    double* part = partials_ptr(partials, "reduce_waves", dev);
    OnDevice on(partials);
    check_rc(api().reduce_waves(wp, m, part, on.stream), "z1_reduce_waves");
}

// ------------------------------------------------------------------------------------------ scale / cast
void scale_up_(const Tensor& g16, const Tensor& g32, const Tensor& factor) {
    require_gpu(g16, "scale_up");
    require_gpu(g32, "scale_up");
    require_gpu(factor, "scale_up");
    TORCH_CHECK(g16.scalar_type() == at::kBFloat16 && g32.scalar_type() == at::kFloat && g16.numel() == g32.numel(),
                "yoco_z1: scale_up expects bf16 -> fp32 of equal size");
    TORCH_CHECK(g16.device() == g32.device() && factor.device() == g32.device(),
                "yoco_z1: scale_up's tensors must be on one device");
    TORCH_CHECK(g16.is_contiguous() && g32.is_contiguous(), "yoco_z1: scale_up expects contiguous tensors");
    TORCH_CHECK(factor.scalar_type() == at::kFloat && factor.numel() >= 1,
                "scale_up: expected a 1-element fp32 device tensor");
    OnDevice on(g32);
    check_rc(api().scale_up(static_cast<const uint16_t*>(g16.data_ptr()), static_cast<float*>(g32.data_ptr()),
                            static_cast<const float*>(factor.data_ptr()), g16.numel(), on.stream), "z1_scale_up");
}

void cast_bf16_(const Tensor& p32, const Tensor& p16) {
    require_gpu(p32, "cast_bf16");
    require_gpu(p16, "cast_bf16");
    TORCH_CHECK(p32.scalar_type() == at::kFloat && p16.scalar_type() == at::kBFloat16 && p32.numel() == p16.numel(),
                "yoco_z1: cast_bf16 expects fp32 -> bf16 of equal size");
    TORCH_CHECK(p32.device() == p16.device(), "yoco_z1: cast_bf16's tensors must be on one device");
    TORCH_CHECK(p32.is_contiguous() && p16.is_contiguous(), "yoco_z1: cast_bf16 expects contiguous tensors");
    OnDevice on(p32);
    check_rc(api().cast_bf16(static_cast<const float*>(p32.data_ptr()), static_cast<uint16_t*>(p16.data_ptr()),
                             p32.numel(), on.stream), "z1_cast_bf16");
}

// ------------------------------------------------------------------------------------------ embedding gradient
void embedding_into(const Tensor& grad, const Tensor& indices, int64_t num_weights, int64_t padding_idx, double scale,
                    int64_t scale_mode, const Tensor& out, const Tensor& workspace) {
    const char* what = "embedding_dense_backward";
    require_gpu(grad, what);
    require_gpu(indices, what);
    TORCH_CHECK(grad.dim() == 2 && grad.scalar_type() == at::kBFloat16 && grad.is_contiguous(), what,
                ": expected contiguous bf16 gradient rows [R, D]");
    const int64_t R = grad.size(0), D = grad.size(1);
    TORCH_CHECK(indices.scalar_type() == at::kLong && indices.is_contiguous() && indices.numel() == R &&
                indices.device() == grad.device(),
                what, ": indices must be int64, one per gradient row, on its device");
    TORCH_CHECK(out.defined() && out.scalar_type() == at::kBFloat16 && out.is_contiguous() &&
                out.numel() == num_weights * D && out.device() == grad.device(),
                what, ": out must be a contiguous bf16 [num_weights, D] tensor");
    const int64_t need = api().embedding_backward_workspace(R, D, num_weights);
    if (need < 0) check_rc(static_cast<int>(need), "z1_embedding_backward_workspace");
    TORCH_CHECK(workspace.defined() && workspace.scalar_type() == at::kByte && workspace.numel() >= need &&
                workspace.device() == grad.device(),
                what, ": the workspace must hold ", need, " bytes on the device");
    OnDevice on(grad);
    check_rc(api().embedding_backward(static_cast<const int64_t*>(indices.data_ptr()),
                                      static_cast<const uint16_t*>(grad.data_ptr()), R, D, num_weights, padding_idx,
                                      static_cast<float>(scale), static_cast<int>(scale_mode),
                                      static_cast<uint16_t*>(out.data_ptr()), workspace.data_ptr(), workspace.numel(),
                                      on.stream), "z1_embedding_backward");
}

void embedding_dense_backward_out_(const Tensor& grad, const Tensor& indices, int64_t num_weights,
                                   int64_t padding_idx, double scale, int64_t scale_mode, const Tensor& out,
                                   const Tensor& workspace) {
    embedding_into(grad, indices, num_weights, padding_idx, scale, scale_mode, out, workspace);
}

Tensor embedding_dense_backward(const Tensor& grad, const Tensor& indices, int64_t num_weights, int64_t padding_idx,
                                double scale, int64_t scale_mode, const Tensor& workspace) {
    require_gpu(grad, "embedding_dense_backward");
    TORCH_CHECK(grad.dim() == 2 && num_weights >= 0, "embedding_dense_backward: expected gradient rows [R, D]");
    Tensor out = at::empty({num_weights, grad.size(1)}, grad.options().dtype(at::kBFloat16));
    embedding_into(grad, indices, num_weights, padding_idx, scale, scale_mode, out, workspace);
    return out;
}

// ------------------------------------------------------------------------------------------ CPU: refuse
void refuse_cpu(const c10::OperatorHandle& op, torch::jit::Stack*) {
    TORCH_CHECK(false, op.schema().name(), ": expected GPU tensors (there is no CPU path)");
}

const char* const kOps[] = {
    "grad_sumsq_", "norm_clip_", "grad_norm_clip_", "update_scalars_", "grad_update_scalars_", "clip_factor_",
    "adam_cast_", "adam_cast_gout_", "adam_cast_dev_", "bias_corrections_step_", "owner_sum_", "owner_sum_update_",
    "sum_slots_", "reduce_waves_", "scale_up_", "cast_bf16_", "embedding_dense_backward_out_",
    "embedding_dense_backward",
};

}  // namespace

TORCH_LIBRARY(yoco_z1, m) {
    m.def("grad_sumsq_(int table, Tensor[] g, Tensor(a2!) partials) -> ()");
    m.def("norm_clip_(Tensor partials, Tensor(a1!)? factor, Tensor(a2!)? norm, Tensor(a3!)? grad_norm, "
          "float max_norm, float? factor_value) -> ()");
    m.def("grad_norm_clip_(int table, Tensor[] g, Tensor(a2!) partials, Tensor(a3!)? factor, Tensor(a4!)? norm, "
          "Tensor(a5!)? grad_norm, float max_norm, float? factor_value) -> ()");
    m.def("update_scalars_(Tensor partials, Tensor(a1!)? factor, Tensor(a2!)? norm, Tensor(a3!)? grad_norm, "
          "Tensor(a4!)? flags, Tensor(a5!)? clip_log, Tensor? sample_size, float numer, float max_norm, "
          "float? factor_value) -> ()");
    m.def("grad_update_scalars_(int table, Tensor[] g, Tensor(a2!) partials, Tensor(a3!)? factor, "
          "Tensor(a4!)? norm, Tensor(a5!)? grad_norm, Tensor(a6!)? flags, Tensor(a7!)? clip_log, "
          "Tensor? sample_size, float numer, float max_norm, float? factor_value) -> ()");
    m.def("clip_factor_(Tensor norm, Tensor(a1!)? factor, Tensor(a2!)? grad_norm, float max_norm, "
          "float? factor_value) -> ()");
    m.def("adam_cast_(int table, Tensor[] g, Tensor(a2!)[] p, Tensor(a3!)[] m, Tensor(a4!)[] v, "
          "Tensor(a5!)[] p16, Tensor? factor, float lr, float beta1, float beta2, float eps, float bc1, float bc2, "
          "float weight_decay, int adam_mode, int row_begin, int row_end) -> ()");
    m.def("adam_cast_gout_(int table, Tensor[] g, Tensor(a2!)[] p, Tensor(a3!)[] m, Tensor(a4!)[] v, "
          "Tensor(a5!)[] p16, Tensor(a6!)[] g32, Tensor? factor, float lr, float beta1, float beta2, float eps, "
          "float bc1, float bc2, float weight_decay, int adam_mode, int row_begin, int row_end) -> ()");
    m.def("adam_cast_dev_(int table, Tensor[] g, Tensor(a2!)[] p, Tensor(a3!)[] m, Tensor(a4!)[] v, "
          "Tensor(a5!)[] p16, Tensor? factor, Tensor bc, float lr, float beta1, float beta2, float eps, "
          "float weight_decay, int adam_mode) -> ()");
    m.def("bias_corrections_step_(Tensor(a0!) step, Tensor(a1!) bc, float beta1, float beta2, "
          "int bias_correction) -> ()");
    m.def("owner_sum_(Tensor[] contribs, Tensor(a1!) out, float scale, Tensor(a3!)? out_sum, "
          "Tensor(a4!)? partials) -> ()");
    m.def("owner_sum_update_(Tensor[] contribs, Tensor(a1!) out, Tensor(a2!) workspace, float scale, "
          "Tensor(a4!)? out_sum, Tensor(a5!)? factor, Tensor(a6!)? norm, Tensor(a7!)? grad_norm, "
          "Tensor(a8!)? flags, Tensor(a9!)? clip_log, Tensor? sample_size, float numer, float max_norm, "
          "float? factor_value) -> ()");
    m.def("sum_slots_(Tensor staging, Tensor(a1!) out, int G, int base, int end, int rank, float scale, "
          "int world, Tensor(a8!)? waves=None) -> ()");
    m.def("reduce_waves_(Tensor waves, int m, Tensor(a2!) partials) -> ()");
    m.def("scale_up_(Tensor g16, Tensor(a1!) g32, Tensor factor) -> ()");
    m.def("cast_bf16_(Tensor p32, Tensor(a1!) p16) -> ()");
    m.def("embedding_dense_backward_out_(Tensor grad, Tensor indices, int num_weights, int padding_idx, "
          "float scale, int scale_mode, Tensor(a6!) out, Tensor(a7!) workspace) -> ()");
    m.def("embedding_dense_backward(Tensor grad, Tensor indices, int num_weights, int padding_idx, float scale, "
          "int scale_mode, Tensor(a6!) workspace) -> Tensor");
}

TORCH_LIBRARY_IMPL(yoco_z1, CUDA, m) {
    m.impl("grad_sumsq_", &grad_sumsq_);
    m.impl("norm_clip_", &norm_clip_);
    m.impl("grad_norm_clip_", &grad_norm_clip_);
    m.impl("update_scalars_", &update_scalars_);
    m.impl("grad_update_scalars_", &grad_update_scalars_);
    m.impl("clip_factor_", &clip_factor_);
    m.impl("adam_cast_", &adam_cast_);
    m.impl("adam_cast_gout_", &adam_cast_gout_);
    m.impl("adam_cast_dev_", &adam_cast_dev_);
    m.impl("bias_corrections_step_", &bias_corrections_step_);
    m.impl("owner_sum_", &owner_sum_);
    m.impl("owner_sum_update_", &owner_sum_update_);
    m.impl("sum_slots_", &sum_slots_);
    m.impl("reduce_waves_", &reduce_waves_);
    m.impl("scale_up_", &scale_up_);
    m.impl("cast_bf16_", &cast_bf16_);
    m.impl("embedding_dense_backward_out_", &embedding_dense_backward_out_);
    m.impl("embedding_dense_backward", &embedding_dense_backward);
}

TORCH_LIBRARY_IMPL(yoco_z1, CPU, m) {
    for (const char* name : kOps) m.impl(name, torch::CppFunction::makeFromBoxedFunction<&refuse_cpu>());
}

// ------------------------------------------------------------------------------------------ host-side set-up
extern "C" {

/* Resolves the C ABI from the already loaded library at `path`: 0, or -1 when it is not loaded, -2 when a function
 * is missing. */
int z1t_init(const char* path) {
    std::lock_guard<std::mutex> lock(g_mu);
    void* h = dlopen(path, RTLD_NOW | RTLD_NOLOAD);
    if (!h) return -1;
    Api a{};
#define Z1T_RESOLVE(field, sym)                                                   \
    a.field = reinterpret_cast<decltype(a.field)>(dlsym(h, #sym));                \
    if (!a.field) return -2;
    Z1T_RESOLVE(table_set_grads, z1_table_set_grads)
    Z1T_RESOLVE(table_rebind, z1_table_rebind)
    Z1T_RESOLVE(table_set_grad_out, z1_table_set_grad_out)
    Z1T_RESOLVE(owner_sum_bf16, z1_owner_sum_bf16)
    Z1T_RESOLVE(owner_sum_workspace, z1_owner_sum_workspace)
    Z1T_RESOLVE(owner_sum_update, z1_owner_sum_update)
    Z1T_RESOLVE(owner_sum_bf16_waves, z1_owner_sum_bf16_waves)
    Z1T_RESOLVE(owner_sum_waves, z1_owner_sum_waves)
    Z1T_RESOLVE(reduce_waves, z1_reduce_waves)
    Z1T_RESOLVE(grad_sumsq, z1_grad_sumsq)
    Z1T_RESOLVE(update_scalars_run, z1_update_scalars_run)
    Z1T_RESOLVE(grad_update_scalars, z1_grad_update_scalars)
    Z1T_RESOLVE(clip_factor, z1_clip_factor)
    Z1T_RESOLVE(adam_cast, z1_adam_cast)
    Z1T_RESOLVE(adam_cast_dev, z1_adam_cast_dev)
    Z1T_RESOLVE(adam_cast_rows, z1_adam_cast_rows)
    Z1T_RESOLVE(bias_corrections_step, z1_bias_corrections_step)
    Z1T_RESOLVE(scale_up, z1_scale_up)
    Z1T_RESOLVE(cast_bf16, z1_cast_bf16)
    Z1T_RESOLVE(embedding_backward, z1_embedding_backward)
    Z1T_RESOLVE(embedding_backward_workspace, z1_embedding_backward_workspace)
    Z1T_RESOLVE(strerror, z1_strerror)
#undef Z1T_RESOLVE
    g_api = a;
    g_api_ok = true;
    return 0;
}

/* Registers a table made by z1_table_create(rows, nrows, g_dtype) on `device`, so that the operators may name it:
 * has_pmv when it updates masters and moments; offsets (nrows element offsets) for the flat form, NULL for the list
 * form; rows as given to z1_table_create (the pointers its device copy holds).  0, or -1 on a bad argument. */
int z1t_table_register(z1_table* table, int device, int g_dtype, int has_pmv, int nrows, const z1_tensor* rows,
                       const int64_t* offsets) {
    if (!table || nrows < 0 || (nrows > 0 && !rows) || (g_dtype != Z1_F32 && g_dtype != Z1_BF16)) return -1;
    TableState t;
    t.h = table;
    t.device = device;
    t.gdtype = g_dtype;
    t.has_pmv = has_pmv != 0;
    t.flat = offsets != nullptr;
    t.sizes.resize(nrows);
    t.bound.resize(nrows);
    for (int i = 0; i < nrows; ++i) {
        if (rows[i].n < 0) return -1;
        t.sizes[i] = rows[i].n;
        t.bound[i] = Bound{reinterpret_cast<uintptr_t>(rows[i].g), reinterpret_cast<uintptr_t>(rows[i].p),
                           reinterpret_cast<uintptr_t>(rows[i].m), reinterpret_cast<uintptr_t>(rows[i].v),
                           reinterpret_cast<uintptr_t>(rows[i].p16), 0};     // no gradient outputs yet
    }
    if (t.flat) {
        t.offsets.assign(offsets, offsets + nrows);
        for (int i = 0; i < nrows; ++i) {
            if (offsets[i] < 0) return -1;
            t.flat_need = std::max(t.flat_need, offsets[i] + t.sizes[i]);
        }
    }
    std::lock_guard<std::mutex> lock(g_mu);
    g_tables[reinterpret_cast<uintptr_t>(table)] = std::move(t);
    return 0;
}

/* Forgets a table (before z1_table_destroy). */
void z1t_table_forget(z1_table* table) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_tables.find(reinterpret_cast<uintptr_t>(table));
    if (it == g_tables.end()) return;
    if (it->second.handoff) (void)hipEventDestroy(it->second.handoff);
    g_tables.erase(it);
}

}  // extern "C"
