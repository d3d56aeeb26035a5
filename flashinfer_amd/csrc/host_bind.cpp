// Native host path of flashinfer_amd.kernel.run (_mi_moe_host): the per-call
// work of the Python wrapper -- the shape and dtype checks of the definition
// (kernel.py:615-625 for the default one), one device, dense layouts, the
// cached workspace of (thread, device, stream), the C-ABI argument block --
// done on the tensors' C++ metadata in one call. Reading one tensor attribute
// from Python costs ~0.2 us and a call reads dozens, which made single-token
// calls host-bound.
//
// run() returns the library's status, or NOT_FAST when the call is not the
// plain case: a tensor that is not dense or not of the definition's dtype and
// shape, a device other than the current one, a scalar that is not a Python
// int / float, T = 0, a stream under graph capture, phase profiling on
// (FIB_PROFILE_PHASES=1), or shapes of no registered definition. The Python
// wrapper then takes its general path, which raises the reference's errors,
// copies non-contiguous tensors and gives captured graphs workspaces of their
// own. Each definition's library is registered (its mi_moe_run and
// mi_moe_workspace_size addresses, keyed by the tensor shapes that select it)
// by the wrapper once it has resolved those shapes.
//
// Built with g++ against torch's headers (no device code here); links c10_hip
// for torch's current stream and the HIP runtime for the capture query.
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <pybind11/pybind11.h>
#include <torch/csrc/autograd/python_variable.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/mi_moe.h"

namespace py = pybind11;

namespace {

constexpr int NOT_FAST = -1;
constexpr int64_t BLK = 128;
constexpr int MAX_DEFS = 32;

typedef int (*RunFn)(const mi_moe_args*, void*);
typedef size_t (*SizeFn)(int64_t);

struct Def {
    int64_t EL, two_i, H, EG;
    RunFn run;
    SizeFn size;
};

// Written under reg_mu, then published by n_defs (release); readers take no lock.
Def defs[MAX_DEFS];
std::atomic<int> n_defs{0};
std::mutex reg_mu;

void register_definition(int64_t EL, int64_t two_i, int64_t H, int64_t EG, uintptr_t run,
                         uintptr_t size) {
    std::lock_guard<std::mutex> g(reg_mu);
    const int n = n_defs.load(std::memory_order_relaxed);
    for (int i = 0; i < n; ++i)
        if (defs[i].EL == EL && defs[i].two_i == two_i && defs[i].H == H && defs[i].EG == EG) {
            if (defs[i].run != reinterpret_cast<RunFn>(run))
                throw std::runtime_error("another library is registered for these shapes");
            return;
        }
    if (n == MAX_DEFS) throw std::runtime_error("too many registered definitions");
    defs[n] = Def{EL, two_i, H, EG, reinterpret_cast<RunFn>(run), reinterpret_cast<SizeFn>(size)};
    n_defs.store(n + 1, std::memory_order_release);
}

const Def* find_def(int64_t EL, int64_t two_i, int64_t H, int64_t EG) {
    const int n = n_defs.load(std::memory_order_acquire);
    for (int i = 0; i < n; ++i)
        if (defs[i].EL == EL && defs[i].two_i == two_i && defs[i].H == H && defs[i].EG == EG)
            return &defs[i];
    return nullptr;
}

// Workspaces cached per thread and (device, stream): calls on one stream from
// two threads would otherwise share one while their kernels interleave. Sizes
// round up to a power of two (at least 1 MiB, exact above 1 GiB) so a slowly
// growing T does not reallocate every call.
// Once the interpreter begins to exit, caches still alive are dropped without
// returning their blocks to torch's allocator, whose own teardown order
// relative to this thread's is not ours to rely on.
struct WsEntry {
    int dev;
    hipStream_t stream;
    at::Tensor ws;
};
std::atomic<bool> exiting{false};
struct WsCache : std::vector<WsEntry> {
    ~WsCache() {
        if (exiting.load())
            for (auto& e : *this) new at::Tensor(std::move(e.ws));
    }
};
thread_local WsCache ws_cache;

at::Tensor& workspace_for(int dev, hipStream_t stream, int64_t nbytes) {
    WsEntry* e = nullptr;
    for (auto& x : ws_cache)
        if (x.dev == dev && x.stream == stream) e = &x;
    if (e && e->ws.numel() >= nbytes) return e->ws;
    int64_t size = std::max<int64_t>(nbytes, 1 << 20);
    if (size < (int64_t(1) << 30)) {
        int64_t p = 1;
        while (p < size) p <<= 1;
        size = p;
    }
    at::Tensor t = at::empty({size}, at::TensorOptions().dtype(at::kByte).device(at::kCUDA, dev));
    if (e) {
        e->ws = std::move(t);
        return e->ws;
    }
    ws_cache.push_back(WsEntry{dev, stream, std::move(t)});
    return ws_cache.back().ws;
}

// The workspace the calling thread holds for (device, stream), or None.
py::object cached_workspace(int dev, uintptr_t stream) {
    for (auto& x : ws_cache)
        if (x.dev == dev && x.stream == reinterpret_cast<hipStream_t>(stream))
            return py::reinterpret_steal<py::object>(THPVariable_Wrap(x.ws));
    return py::none();
}

py::object workspace(int dev, uintptr_t stream, int64_t nbytes) {
    return py::reinterpret_steal<py::object>(
        THPVariable_Wrap(workspace_for(dev, reinterpret_cast<hipStream_t>(stream), nbytes)));
}

bool sizes_are(const at::Tensor& t, std::initializer_list<int64_t> want) {
    if (t.dim() != (int64_t)want.size()) return false;
    int64_t i = 0;
    for (int64_t w : want)
        if (t.size(i++) != w) return false;
    return true;
}

// The tensor behind a Python object, or null when it is not a tensor.
const at::Tensor* tensor_of(py::handle h) {
    if (!THPVariable_Check(h.ptr())) return nullptr;
    return &THPVariable_Unpack(h.ptr());
}

bool dense(const at::Tensor* t, c10::ScalarType dtype, const c10::Device& dev,
           std::initializer_list<int64_t> want) {
    return t && t->scalar_type() == dtype && t->device() == dev && sizes_are(*t, want) &&
           t->is_contiguous();
}

int run(py::handle logits_h, py::handle bias_h, py::handle hs_h, py::handle hss_h, py::handle w1_h,
        py::handle w1s_h, py::handle w2_h, py::handle w2s_h, py::handle offset_h, py::handle rsf_h,
        py::handle out_h) {
    const char* prof = std::getenv("FIB_PROFILE_PHASES");
    if (prof && std::strcmp(prof, "1") == 0) return NOT_FAST;
    const at::Tensor *logits = tensor_of(logits_h), *w1 = tensor_of(w1_h), *out = tensor_of(out_h);
    if (!logits || !w1 || !out || logits->dim() != 2 || w1->dim() != 3 || !out->is_cuda())
        return NOT_FAST;
    const int64_t T = logits->size(0);
    // T = 0 and T past the library's limit take the general path, which
    // returns or raises before any workspace is sized
    if (T == 0 || T > MI_MOE_MAX_TOKENS) return NOT_FAST;
    const Def* d = find_def(w1->size(0), w1->size(1), w1->size(2), logits->size(1));
    if (!d) return NOT_FAST;
    const int64_t H = d->H, I = d->two_i / 2, EL = d->EL, EG = d->EG;

    if (!PyLong_CheckExact(offset_h.ptr())) return NOT_FAST;
    const long long offset = PyLong_AsLongLong(offset_h.ptr());
    if (offset == -1 && PyErr_Occurred()) {
        PyErr_Clear();
        return NOT_FAST;
    }
    double rsf;
    if (PyFloat_CheckExact(rsf_h.ptr())) {
        rsf = PyFloat_AS_DOUBLE(rsf_h.ptr());
    } else if (PyLong_CheckExact(rsf_h.ptr())) {
        rsf = PyLong_AsDouble(rsf_h.ptr());
        if (rsf == -1.0 && PyErr_Occurred()) {
            PyErr_Clear();
            return NOT_FAST;
        }
    } else {
        return NOT_FAST;
    }

    const c10::Device dev = out->device();
    const at::Tensor *bias = tensor_of(bias_h), *hs = tensor_of(hs_h), *hss = tensor_of(hss_h),
                     *w1s = tensor_of(w1s_h), *w2 = tensor_of(w2_h), *w2s = tensor_of(w2s_h);
    if (!bias) return NOT_FAST;
    const bool bias_f32 = bias->scalar_type() == at::kFloat;
    if (!dense(logits, at::kFloat, dev, {T, EG}) ||
        !dense(bias, bias_f32 ? at::kFloat : at::kBFloat16, dev, {EG}) ||
        !dense(hs, at::kFloat8_e4m3fn, dev, {T, H}) ||
        !dense(hss, at::kFloat, dev, {H / BLK, T}) ||
        !dense(w1, at::kFloat8_e4m3fn, dev, {EL, 2 * I, H}) ||
        !dense(w1s, at::kFloat, dev, {EL, 2 * I / BLK, H / BLK}) ||
        !dense(w2, at::kFloat8_e4m3fn, dev, {EL, H, I}) ||
        !dense(w2s, at::kFloat, dev, {EL, H / BLK, I / BLK}) ||
        !dense(out, at::kBFloat16, dev, {T, H}))
        return NOT_FAST;

    const int idx = dev.index();
    if (idx != c10::hip::current_device()) return NOT_FAST;
    hipStream_t stream = c10::hip::getCurrentHIPStream(idx).stream();
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
        return NOT_FAST;
    const at::Tensor& ws = workspace_for(idx, stream, (int64_t)d->size(T));

    mi_moe_args a{};
    a.routing_logits = static_cast<const float*>(logits->data_ptr());
    a.routing_bias = bias->data_ptr();
    a.hidden_states = static_cast<const uint8_t*>(hs->data_ptr());
    a.hidden_states_scale = static_cast<const float*>(hss->data_ptr());
    a.gemm1_weights = static_cast<const uint8_t*>(w1->data_ptr());
    a.gemm1_weights_scale = static_cast<const float*>(w1s->data_ptr());
    a.gemm2_weights = static_cast<const uint8_t*>(w2->data_ptr());
    a.gemm2_weights_scale = static_cast<const float*>(w2s->data_ptr());
    a.local_expert_offset = offset;
    a.routed_scaling_factor = (float)rsf;
    a.output = out->data_ptr();
    a.num_tokens = T;
    a.bias_dtype = bias_f32 ? MI_MOE_DTYPE_F32 : MI_MOE_DTYPE_BF16;
    a.reserved = 0;
    a.workspace = ws.data_ptr();
    a.workspace_bytes = (size_t)ws.numel();
    // The launches run without the GIL (as a ctypes call would); the caller's
    // frame keeps every tensor alive until this returns.
    py::gil_scoped_release nogil;
    return d->run(&a, stream);
}

}  // namespace

PYBIND11_MODULE(_mi_moe_host, m) {
    m.doc() = "Native host path of flashinfer_amd.kernel.run";
    m.attr("NOT_FAST") = NOT_FAST;
    m.def("run", &run, py::arg("routing_logits"), py::arg("routing_bias"),
          py::arg("hidden_states"), py::arg("hidden_states_scale"), py::arg("gemm1_weights"),
          py::arg("gemm1_weights_scale"), py::arg("gemm2_weights"),
          py::arg("gemm2_weights_scale"), py::arg("local_expert_offset"),
          py::arg("routed_scaling_factor"), py::arg("output"),
          "run(11 arguments of kernel.run): the library's status for the plain case, or "
          "NOT_FAST for the general path");
    m.def("register_definition", &register_definition,
          "register_definition(E_local, 2I, H, E_global, mi_moe_run address, "
          "mi_moe_workspace_size address)");
    m.def("workspace", &workspace,
          "workspace(device, stream, nbytes): the calling thread's cached workspace of "
          "(device, stream), grown to at least nbytes");
    py::module_::import("atexit").attr("register")(
        py::cpp_function([]() { exiting.store(true); }));
    m.def("cached_workspace", &cached_workspace,
          "cached_workspace(device, stream): the calling thread's workspace of (device, "
          "stream), or None");
}
