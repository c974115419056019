// The subset of brotensor::Tensor the decoder back half and its tests use
// (rows, cols, device, dtype, data, size(), operator[], clone, to_host_vector,
// to, from_host_on, zeros_on, empty_on, mat, view), backed here by host memory
// or by HIP device memory from the library's stream-ordered allocator.
//
// Copies are shallow (shared storage), as the reference's code relies on
// (kokoro_decoder_backward.cpp:339, 342-343 use clone() for deep copies).
// A tensor's flat element (r, c) lives at data[r * ld + c], ld = cols unless
// the tensor is a strided row view (ld > cols; an extension used to address
// per-utterance slices of a packed buffer without copies).
#pragma once

#include <cstddef>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

struct kdec_ctx;

namespace brotensor {

enum class Device { CPU, HIP };
enum class Dtype { FP32 };

struct Tensor {
    int rows = 0;
    int cols = 0;
    Device device = Device::CPU;
    Dtype dtype = Dtype::FP32;
    void* data = nullptr;
    long ld = 0;  // row stride in elements; 0 means cols
    std::shared_ptr<void> storage;

    std::size_t size() const { return static_cast<std::size_t>(rows) * cols; }
    long row_stride() const { return ld ? ld : cols; }
    bool contiguous() const { return ld == 0 || ld == cols || rows <= 1; }
    float* f32() const { return static_cast<float*>(data); }

    static Tensor empty_on(Device dev, int rows, int cols, Dtype dt = Dtype::FP32);
    static Tensor zeros_on(Device dev, int rows, int cols, Dtype dt = Dtype::FP32);
    static Tensor from_host_on(Device dev, const float* src, int rows, int cols);
    static Tensor mat(int rows, int cols);  // host zeros
    // Non-owning view; the parent must outlive it.
    static Tensor view(Device dev, void* base, int rows, int cols, Dtype dt = Dtype::FP32,
                       long ld = 0);

    std::vector<float> to_host_vector() const;
    Tensor clone() const;
    Tensor to(Device dev) const;

    // Host element access (CPU tensors only, as in the reference's tests).
    float operator[](std::size_t i) const;
    float& operator[](std::size_t i);
};

// Runtime: the HIP context every device tensor and op uses.
void init(int device = 0);
kdec_ctx* runtime();
void set_runtime(kdec_ctx* ctx);  // adopt an externally created context
void sync(Device dev);

}  // namespace brotensor
