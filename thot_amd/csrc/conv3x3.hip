// Specialised 3x3 stride-1 conv kernels (placeholder: none apply yet).
#include "conv_fast.hpp"

namespace nott {
namespace conv_fast {

bool fwd_applies(const nott_conv2d_desc*, size_t) { return false; }
bool dgrad_applies(const nott_conv2d_desc*, size_t) { return false; }
bool wgrad_applies(const nott_conv2d_desc*, size_t) { return false; }

template <typename T>
int fwd(nott_ctx ctx, const nott_conv2d_desc*, const T*, const T*, const float*, T*) {
    return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3 fwd");
}
template <typename T>
int dgrad(nott_ctx ctx, const nott_conv2d_desc*, const T*, const T*, T*) {
    return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3 dgrad");
}
template <typename T>
int wgrad(nott_ctx ctx, const nott_conv2d_desc*, const T*, const T*, float*, int) {
    return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3 wgrad");
}
template int fwd<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, const float*, float*);
template int fwd<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, const float*, bf16_t*);
template int dgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*);
template int dgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, bf16_t*);
template int wgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*, int);
template int wgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, float*, int);

}  // namespace conv_fast
}  // namespace nott
