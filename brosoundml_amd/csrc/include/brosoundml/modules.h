// Conv1d and Linear with the reference's fields and weight layouts
// (include/brosoundml/modules.h:14-21, 35-46, 67-81): Linear W (out, in),
// b (out, 1); Conv1d W (C_out, (C_in/groups)*k), b (C_out, 1) or empty.
#pragma once

#include <brotensor/tensor.h>

namespace brosoundml {

struct Linear {
    int in_features = 0;
    int out_features = 0;
    brotensor::Tensor W;  // (out, in)
    brotensor::Tensor b;  // (out, 1) — empty when bias is disabled
};

struct Conv1d {
    int in_channels = 0;
    int out_channels = 0;
    int kernel_size = 0;
    int stride = 1;
    int padding = 0;
    int dilation = 1;
    int groups = 1;
    brotensor::Tensor W;  // (out, (in/groups)*kL)
    brotensor::Tensor b;  // (out, 1) — empty when bias is disabled

    // Y:(N, out_channels*L_out). X:(N, in_channels*L) on the HIP device.
    void forward(const brotensor::Tensor& X, int N, int L, brotensor::Tensor& Y) const;
    int out_length(int L) const {
        return (L + 2 * padding - dilation * (kernel_size - 1) - 1) / stride + 1;
    }
};

}  // namespace brosoundml
