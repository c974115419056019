// Raw buffer descriptors for the kernels' bounds-checked loads and stores on
// gfx950.
#pragma once

#include <hip/hip_runtime.h>

namespace kdec {

// Buffer descriptor word 3 for raw 32-bit buffer accesses (DATA_FORMAT = 32).
constexpr int kBufDword3 = 0x00020000;

// Raw buffer descriptor over [base, base + bytes), built from wave-uniform
// (scalar) values: a descriptor the compiler cannot prove uniform would be
// wrapped in a per-lane "waterfall" loop around every buffer access. Loads
// past `bytes` return 0 and stores there are dropped.
__device__ inline __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, int bytes) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(base);
    const unsigned lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(a));
    const unsigned hi = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(a >> 32));
    const int n = __builtin_amdgcn_readfirstlane(bytes);
    void* p = reinterpret_cast<void*>((static_cast<unsigned long long>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(p, static_cast<short>(0), n, kBufDword3);
}

}  // namespace kdec
