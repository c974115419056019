// brotensor::Tensor subset over host memory or the kdec context's device
// allocator. Device copies run on the context stream (synchronously where the
// call returns host data or reads a host buffer the caller may free).
#include <brotensor/tensor.h>

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <cstring>

#include "kdec.h"

namespace brotensor {

kdec_ctx* g_ctx = nullptr;  // the runtime context (see init / set_runtime)

namespace {

[[noreturn]] void fail(const std::string& where, const std::string& msg) {
    throw std::runtime_error("brosoundml: " + where + ": " + msg);
}

void hip_ok(hipError_t e, const char* where) {
    if (e != hipSuccess) fail(where, hipGetErrorString(e));
}

hipStream_t stream() { return static_cast<hipStream_t>(kdec_get_stream(runtime())); }

std::shared_ptr<void> alloc(Device dev, std::size_t n) {
    const std::size_t bytes = (n ? n : 1) * sizeof(float);
    if (dev == Device::CPU) {
        void* p = std::calloc(1, bytes);
        if (!p) fail("Tensor", "host allocation failed");
        return std::shared_ptr<void>(p, [](void* q) { std::free(q); });
    }
    kdec_ctx* c = runtime();
    void* p = nullptr;
    if (kdec_malloc(c, bytes, &p) != KDEC_OK) fail("Tensor", kdec_last_error(c));
    return std::shared_ptr<void>(p, [c](void* q) { kdec_free(c, q); });
}

}  // namespace

void init(int device) {
    if (g_ctx) return;
    kdec_ctx* c = nullptr;
    const int rc = kdec_ctx_create(device, &c);
    if (rc != KDEC_OK) fail("brotensor::init", "no usable HIP device (kdec_ctx_create failed)");
    g_ctx = c;
}

kdec_ctx* runtime() {
    if (!g_ctx) init(0);
    return g_ctx;
}

void set_runtime(kdec_ctx* ctx) { g_ctx = ctx; }

}  // namespace brotensor

namespace kdec {
void forget_runtime(kdec_ctx* ctx) {
    if (brotensor::g_ctx == ctx) brotensor::g_ctx = nullptr;
}
}  // namespace kdec

namespace brotensor {

void sync(Device dev) {
    if (dev == Device::HIP && g_ctx) kdec_synchronize(g_ctx);
}

Tensor Tensor::empty_on(Device dev, int rows, int cols, Dtype dt) {
    Tensor t;
    t.rows = rows;
    t.cols = cols;
    t.device = dev;
    t.dtype = dt;
    t.storage = alloc(dev, t.size());
    t.data = t.storage.get();
    return t;
}

Tensor Tensor::zeros_on(Device dev, int rows, int cols, Dtype dt) {
    Tensor t = empty_on(dev, rows, cols, dt);
    if (dev == Device::HIP) {
        if (kdec_fill(runtime(), t.f32(), static_cast<long>(t.size()), 0.0f) != KDEC_OK)
            fail("Tensor::zeros_on", kdec_last_error(runtime()));
    }
    return t;
}

Tensor Tensor::from_host_on(Device dev, const float* src, int rows, int cols) {
    Tensor t = empty_on(dev, rows, cols);
    const std::size_t bytes = t.size() * sizeof(float);
    if (dev == Device::CPU) {
        if (bytes) std::memcpy(t.data, src, bytes);
    } else if (bytes) {
        hip_ok(hipMemcpyAsync(t.data, src, bytes, hipMemcpyHostToDevice, stream()), "Tensor::from_host_on");
        hip_ok(hipStreamSynchronize(stream()), "Tensor::from_host_on");
    }
    return t;
}

Tensor Tensor::mat(int rows, int cols) { return zeros_on(Device::CPU, rows, cols); }

Tensor Tensor::view(Device dev, void* base, int rows, int cols, Dtype dt, long ld) {
    Tensor t;
    t.rows = rows;
    t.cols = cols;
    t.device = dev;
    t.dtype = dt;
    t.data = base;
    t.ld = ld;
    return t;
}

std::vector<float> Tensor::to_host_vector() const {
    std::vector<float> out(size());
    if (out.empty()) return out;
    const long rs = row_stride();
    if (device == Device::CPU) {
        for (int r = 0; r < rows; ++r)
            std::memcpy(out.data() + static_cast<std::size_t>(r) * cols, f32() + r * rs, cols * sizeof(float));
        return out;
    }
    if (contiguous()) {
        hip_ok(hipMemcpyAsync(out.data(), data, out.size() * sizeof(float), hipMemcpyDeviceToHost, stream()),
               "Tensor::to_host_vector");
    } else {
        hip_ok(hipMemcpy2DAsync(out.data(), cols * sizeof(float), data, rs * sizeof(float), cols * sizeof(float),
                                rows, hipMemcpyDeviceToHost, stream()),
               "Tensor::to_host_vector");
    }
    hip_ok(hipStreamSynchronize(stream()), "Tensor::to_host_vector");
    return out;
}

Tensor Tensor::clone() const {
    Tensor t = empty_on(device, rows, cols, dtype);
    if (size() == 0) return t;
    const long rs = row_stride();
    if (device == Device::CPU) {
        for (int r = 0; r < rows; ++r)
            std::memcpy(t.f32() + static_cast<std::size_t>(r) * cols, f32() + r * rs, cols * sizeof(float));
        return t;
    }
    if (kdec_axpby(runtime(), 1.0f, f32(), rs, 0.0f, nullptr, 0, t.f32(), cols, rows, cols) != KDEC_OK)
        fail("Tensor::clone", kdec_last_error(runtime()));
    return t;
}

Tensor Tensor::to(Device dev) const {
    if (dev == device) return clone();
    if (dev == Device::CPU) {
        const std::vector<float> h = to_host_vector();
        return from_host_on(Device::CPU, h.data(), rows, cols);
    }
    if (contiguous()) return from_host_on(dev, f32(), rows, cols);
    return clone().to(dev);
}

float Tensor::operator[](std::size_t i) const {
    if (device != Device::CPU) fail("Tensor::operator[]", "element access needs a CPU tensor");
    const long rs = row_stride();
    return f32()[(i / cols) * rs + i % cols];
}

float& Tensor::operator[](std::size_t i) {
    if (device != Device::CPU) fail("Tensor::operator[]", "element access needs a CPU tensor");
    const long rs = row_stride();
    return f32()[(i / cols) * rs + i % cols];
}

}  // namespace brotensor
