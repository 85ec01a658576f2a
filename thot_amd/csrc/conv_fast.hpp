// Specialised conv kernels for the 3x3 / stride-1 shapes (declarations).
#pragma once

#include "common.hpp"

namespace nott {
namespace conv_fast {

bool fwd_applies(const nott_conv2d_desc* d, size_t elem);
bool dgrad_applies(const nott_conv2d_desc* d, size_t elem);
bool wgrad_applies(const nott_conv2d_desc* d, size_t elem);

template <typename T>
int fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu = 0);
template <typename T>
int dgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* w, T* dx);
template <typename T>
int wgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, int accumulate);

}  // namespace conv_fast
}  // namespace nott
