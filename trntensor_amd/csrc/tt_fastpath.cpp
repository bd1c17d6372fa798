// Host fast path for repeated two-operand contractions that run as one GEMM
// launch (e.g. einsum("ap,bp->ab", B[i], B[j]) in a pair loop).
//
// The first call of a contraction is planned in Python; when it runs as a
// single tt_gemm launch on operands in place, its launch parameters are
// recorded here under a key of (subscripts, each operand's sizes, strides,
// dtype and device). A repeat call with the same key is one table lookup,
// one allocation of the output and one call of tt_gemm_packed on torch's
// current stream, with no Python frame in between. The library entry point
// is passed in by address (no link dependency on libtrntensor_hip.so), so the
// status codes map to the same exceptions as the ctypes path: TT_INVALID ->
// ValueError, TT_UNSUPPORTED -> NotImplementedError, others -> RuntimeError.
// Small contractions of contiguous host operands are recorded too: a repeat
// call stages both operands through one pinned buffer and one upload, and
// copies the result back before returning (run_host).
#include <torch/extension.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "trntensor_hip.h"

namespace {

using packed_fn = decltype(&tt_gemm_packed);
using error_fn = decltype(&tt_last_error);
using status_fn = decltype(&tt_status_string);

constexpr int kParams = 15;  // tt_gemm_packed's parameter block

struct Recipe {
    int64_t params[kParams];
    std::vector<int64_t> sizes, strides;  // the output, row-major
    at::ScalarType dtype;
    c10::DeviceIndex device;
    bool swap;  // the output is computed as B^T A^T: operands exchanged
    // Host operands (both contiguous, on the CPU): staged through one pinned
    // buffer and one device buffer, the result copied back before returning.
    bool host = false;
    int64_t a_bytes = 0, b_bytes = 0, out_bytes = 0, b_off = 0;
};

constexpr int64_t kAlign = 256;
// Largest host-operand contraction (both operands plus the output) staged
// here; larger ones are bound by the copies and go through the planned path.
constexpr int64_t kHostMaxBytes = int64_t(4) << 20;

int64_t round_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

void append(std::string& k, const void* p, size_t n) { k.append(static_cast<const char*>(p), n); }

void append_tensor(std::string& k, const at::Tensor& t) {
    const int64_t nd = t.dim();
    append(k, &nd, sizeof nd);
    append(k, t.sizes().data(), nd * sizeof(int64_t));
    append(k, t.strides().data(), nd * sizeof(int64_t));
    const int16_t dt = static_cast<int16_t>(t.scalar_type());
    const int16_t devt = static_cast<int16_t>(t.device().type());
    const int16_t devi = static_cast<int16_t>(t.device().index());
    append(k, &dt, sizeof dt);
    append(k, &devt, sizeof devt);
    append(k, &devi, sizeof devi);
}

std::string make_key(const std::string& sub, const at::Tensor& a, const at::Tensor& b) {
    std::string k;
    k.reserve(sub.size() + 2 * (8 + 8 * 8 + 6) + 1);
    k.append(sub);
    k.push_back('\0');
    append_tensor(k, a);
    append_tensor(k, b);
    return k;
}

class LaunchTable {
   public:
    LaunchTable(int64_t packed, int64_t last_error, int64_t status_string, int64_t max_entries)
        : fn_(reinterpret_cast<packed_fn>(packed)),
          err_(reinterpret_cast<error_fn>(last_error)),
          status_(reinterpret_cast<status_fn>(status_string)),
          max_(max_entries > 0 ? static_cast<size_t>(max_entries) : 1) {
        TORCH_CHECK(fn_ && err_ && status_, "LaunchTable: null library entry point");
    }

    // Record the launch of (sub, a, b): tt_gemm_packed's parameter block, the
    // output's sizes (row-major) and whether the operands are exchanged. The
    // table is cleared when it reaches its bound.
    void add(const std::string& sub, const at::Tensor& a, const at::Tensor& b, const std::vector<int64_t>& params,
             const std::vector<int64_t>& sizes, bool swap) {
        TORCH_CHECK(params.size() == kParams, "LaunchTable.add: ", kParams, " parameters expected");
        TORCH_CHECK(a.device().is_cuda() && b.device() == a.device() && a.scalar_type() == b.scalar_type(),
                    "LaunchTable.add: operands on one device in one dtype expected");
        Recipe r;
        std::memcpy(r.params, params.data(), sizeof r.params);
        r.sizes = sizes;
        r.strides.assign(sizes.size(), 1);
        int64_t acc = 1;
        for (size_t d = sizes.size(); d-- > 0;) {
            r.strides[d] = acc;
            acc *= std::max<int64_t>(sizes[d], 1);
        }
        r.dtype = a.scalar_type();
        r.device = a.device().index();
        r.swap = swap;
        insert(make_key(sub, a, b), std::move(r));
    }

    // Record the launch of (sub, a, b) for contiguous host operands: each call
    // copies both into one pinned buffer, uploads it with one copy, launches
    // on `device` and copies the output back, then waits for the stream.
    // Returns false (nothing recorded) when the operands are not contiguous
    // or the problem is above the staging bound.
    bool add_host(const std::string& sub, const at::Tensor& a, const at::Tensor& b, const std::vector<int64_t>& params,
                  const std::vector<int64_t>& sizes, bool swap, int64_t device) {
        TORCH_CHECK(params.size() == kParams, "LaunchTable.add_host: ", kParams, " parameters expected");
        TORCH_CHECK(a.device().is_cpu() && b.device().is_cpu() && a.scalar_type() == b.scalar_type(),
                    "LaunchTable.add_host: host operands in one dtype expected");
        if (!a.is_contiguous() || !b.is_contiguous()) return false;
        Recipe r;
        std::memcpy(r.params, params.data(), sizeof r.params);
        r.sizes = sizes;
        r.strides.assign(sizes.size(), 1);
        int64_t acc = 1;
        for (size_t d = sizes.size(); d-- > 0;) {
            r.strides[d] = acc;
            acc *= std::max<int64_t>(sizes[d], 1);
        }
        r.dtype = a.scalar_type();
        r.device = static_cast<c10::DeviceIndex>(device);
        r.swap = swap;
        r.host = true;
        const int64_t es = a.element_size();
        r.a_bytes = a.numel() * es;
        r.b_bytes = b.numel() * es;
        r.out_bytes = acc * es;
        r.b_off = round_up(r.a_bytes);
        if (r.b_off + round_up(r.b_bytes) + r.out_bytes > kHostMaxBytes) return false;
        insert(make_key(sub, a, b), std::move(r));
        return true;
    }

    // alpha * (the recorded contraction of a and b), or None when (sub, a, b)
    // has no recorded launch.
    py::object run(const std::string& sub, const at::Tensor& a, const at::Tensor& b, double alpha) {
        const auto it = map_.find(make_key(sub, a, b));
        if (it == map_.end()) return py::none();
        const Recipe& r = it->second;
        if (r.host) return run_host(r, a, b, alpha);
        at::Tensor D = at::empty_strided(r.sizes, r.strides,
                                         at::TensorOptions().dtype(r.dtype).device(c10::DeviceType::CUDA, r.device));
        const at::Tensor& x = r.swap ? b : a;
        const at::Tensor& y = r.swap ? a : b;
        hipStream_t st = c10::hip::getCurrentHIPStream(r.device).stream();
        const int rc = fn_(r.params, alpha, 0.0, x.data_ptr(), y.data_ptr(), nullptr, D.data_ptr(), st);
        if (rc != TT_OK) raise(rc);
        return py::cast(D);
    }

    void clear() { map_.clear(); }
    size_t size() const { return map_.size(); }

   private:
    void insert(std::string key, Recipe&& r) {
        if (map_.size() >= max_) map_.clear();
        map_[std::move(key)] = std::move(r);
    }

    // Host operands: one pinned staging buffer and one device buffer (held by
    // the table, grown on demand up to kHostMaxBytes each) serve every call;
    // each call waits for its stream before returning, so no two calls'
    // copies overlap.
    py::object run_host(const Recipe& r, const at::Tensor& a, const at::Tensor& b, double alpha) {
        const int64_t in_bytes = r.b_off + r.b_bytes;
        const int64_t out_off = round_up(in_bytes);
        const int64_t total = out_off + r.out_bytes;
        if (!pinned_.defined() || pinned_.numel() < total)
            pinned_ = at::empty({total}, at::TensorOptions().dtype(at::kByte).pinned_memory(true));
        if (!dbuf_.defined() || dbuf_.numel() < total || dbuf_.device().index() != r.device)
            dbuf_ = at::empty({total}, at::TensorOptions().dtype(at::kByte).device(c10::DeviceType::CUDA, r.device));
        char* h = static_cast<char*>(pinned_.data_ptr());
        char* d = static_cast<char*>(dbuf_.data_ptr());
        std::memcpy(h, a.data_ptr(), r.a_bytes);
        std::memcpy(h + r.b_off, b.data_ptr(), r.b_bytes);
        c10::hip::HIPGuard guard(r.device);
        hipStream_t st = c10::hip::getCurrentHIPStream(r.device).stream();
        hip_check(hipMemcpyAsync(d, h, in_bytes, hipMemcpyHostToDevice, st), "hipMemcpyAsync (operands)");
        const void* x = r.swap ? d + r.b_off : d;
        const void* y = r.swap ? d : d + r.b_off;
        const int rc = fn_(r.params, alpha, 0.0, x, y, nullptr, d + out_off, st);
        if (rc != TT_OK) raise(rc);
        hip_check(hipMemcpyAsync(h + out_off, d + out_off, r.out_bytes, hipMemcpyDeviceToHost, st),
                  "hipMemcpyAsync (result)");
        hipError_t e;
        {
            py::gil_scoped_release nogil;
            e = hipStreamSynchronize(st);
        }
        hip_check(e, "hipStreamSynchronize");
        at::Tensor D = at::empty_strided(r.sizes, r.strides, at::TensorOptions().dtype(r.dtype));
        std::memcpy(D.data_ptr(), h + out_off, r.out_bytes);
        return py::cast(D);
    }

    static void hip_check(hipError_t e, const char* what) {
        if (e != hipSuccess) {
            PyErr_SetString(PyExc_RuntimeError, (std::string("tt_gemm: ") + what + ": " + hipGetErrorString(e)).c_str());
            throw py::error_already_set();
        }
    }

    [[noreturn]] void raise(int rc) const {
        const char* detail = err_();
        std::string msg = std::string("tt_gemm: ") + (detail && *detail ? detail : status_(rc));
        PyObject* type = rc == TT_INVALID ? PyExc_ValueError
                         : rc == TT_UNSUPPORTED ? PyExc_NotImplementedError
                                                : PyExc_RuntimeError;
        PyErr_SetString(type, msg.c_str());
        throw py::error_already_set();
    }

    packed_fn fn_;
    error_fn err_;
    status_fn status_;
    size_t max_;
    std::unordered_map<std::string, Recipe> map_;
    at::Tensor pinned_, dbuf_;  // host-operand staging
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "Launch table for repeated two-operand contractions (one GEMM launch each)";
    py::class_<LaunchTable>(m, "LaunchTable")
        .def(py::init<int64_t, int64_t, int64_t, int64_t>(), py::arg("packed"), py::arg("last_error"),
             py::arg("status_string"), py::arg("max_entries"))
        .def("add", &LaunchTable::add)
        .def("add_host", &LaunchTable::add_host)
        .def("run", &LaunchTable::run)
        .def("clear", &LaunchTable::clear)
        .def("__len__", &LaunchTable::size);
}
