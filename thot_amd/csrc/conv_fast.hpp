// Specialised conv kernels for the 3x3 / stride-1 shapes (declarations).
#pragma once

#include "common.hpp"

namespace nott {
namespace conv_fast {

bool fwd_applies(const nott_conv2d_desc* d, size_t elem);
bool dgrad_applies(const nott_conv2d_desc* d, size_t elem);
// The 3×3 forward that also writes the data gradient's weight slices (one
// prep launch for both layouts), the data gradient from those slices, and
// their element count.  Both need fwd_applies and dgrad_applies.
template <typename T>
int fwd_prep(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu, T* wd);
template <typename T>
int dgrad_prepared(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* wd, T* dx);
int64_t dgrad_prep_elems(const nott_conv2d_desc* d);
bool wgrad_applies(const nott_conv2d_desc* d, size_t elem);

template <typename T>
int fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu = 0);
template <typename T>
int dgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* w, T* dx);
template <typename T>
int wgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, int accumulate);

// LDS-staged implicit GEMM for other NCHW shapes (stride 1 or 2, up to 9
// taps; conv_tap.hip).
bool tap_fwd_applies(nott_ctx ctx, const nott_conv2d_desc* d, size_t elem);
bool tap_dgrad_applies(nott_ctx ctx, const nott_conv2d_desc* d, size_t elem);
template <typename T>
int tap_fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu);
template <typename T>
int tap_dgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* w, T* dx);

// Forward of the 3-channel 7x7 column-stride-2 stem (conv_stem.hip).
bool stem_fwd_applies(nott_ctx ctx, const nott_conv2d_desc* d);
template <typename T>
int stem_fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu);

bool stem_wgrad_applies(nott_ctx ctx, const nott_conv2d_desc* d);
template <typename T>
int stem_wgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, int accumulate);

// bf16 3x3 / stride-1 forward and data gradient with DMA-filled LDS stages
// (conv3x3_dma.hip), in a pass's own terms (cin → cout).  dma_applies is a
// function of the shape only, so a forward can decide which layout the data
// gradient's prepared weights take; dma_prep writes dma_prep_elems elements
// (DGRAD: from the conv weight [cin][cout][3][3] of the pass, flipped).
bool dma_applies(int32_t n, int32_t cin, int32_t h, int32_t w, int32_t cout);
int64_t dma_prep_elems(int32_t cin, int32_t cout);
template <bool DGRAD>
int dma_prep(nott_ctx ctx, const bf16_t* w, bf16_t* wp, int32_t cin, int32_t cout);
// Both: the forward's slices of w (cin → cout) into wf, the data gradient's
// into wd, one launch.
int dma_prep_pair(nott_ctx ctx, const bf16_t* w, bf16_t* wf, bf16_t* wd, int32_t cin, int32_t cout);
int dma_run(nott_ctx ctx, int32_t n, int32_t cin, int32_t h, int32_t w, int32_t cout, const bf16_t* in,
            const bf16_t* wp, const float* bias, bf16_t* out, int relu);

// bf16 3x3 / stride-1 weight gradient with DMA-filled LDS bands
// (conv3x3_dma.hip): writes split partials ws[split][k][c][tap] into the
// context workspace for the ordered reduce; returns the split count.
bool wdma_applies(int32_t n, int32_t c, int32_t h, int32_t w, int32_t k);
int wdma_partials(nott_ctx ctx, int32_t n, int32_t c, int32_t h, int32_t w, int32_t k, const bf16_t* x,
                  const bf16_t* dy, float** ws_out, int32_t* splits_out);

// Widest load (bytes) that keeps every image row's pieces aligned.
int wgrad_load_width(int64_t w, size_t elem);

}  // namespace conv_fast
}  // namespace nott
