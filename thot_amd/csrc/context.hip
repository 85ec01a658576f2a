// Context, errors and workspace of libnott_hip.
#include "common.hpp"

#include <cstdlib>

#include <new>

namespace nott {

int fail(nott_ctx ctx, int status, const std::string& msg) {
    if (ctx) ctx->last_error = msg;
    return status;
}

int hip_fail(nott_ctx ctx, hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    return fail(ctx, NOTT_ERR_HIP, m);
}

void* workspace(nott_ctx ctx, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (bytes <= ctx->ws_bytes) return ctx->ws;
    // Geometric growth bounds the retired total by the current arena's size.
    size_t want = (bytes + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
    want = std::max(want, 2 * ctx->ws_bytes);
    void* fresh = nullptr;
    hipError_t e = hipMalloc(&fresh, want);
    if (e != hipSuccess) {
        fail(ctx, NOTT_ERR_ALLOC, std::string("workspace hipMalloc of ") + std::to_string(want) +
                                      " bytes failed: " + hipGetErrorString(e));
        return nullptr;
    }
    if (ctx->ws) {
        ctx->retired.push_back(ctx->ws);
        ctx->retired_bytes += ctx->ws_bytes;
    }
    ctx->ws = fresh;
    ctx->ws_bytes = want;
    return ctx->ws;
}

int launch_status(nott_ctx ctx, const char* kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(ctx, e, kernel);
    return NOTT_OK;
}

}  // namespace nott

extern "C" {

int nott_abi_version(void) { return NOTT_ABI_VERSION; }

const char* nott_status_string(int status) {
    switch (status) {
        case NOTT_OK: return "ok";
        case NOTT_ERR_INVALID_ARG: return "invalid argument";
        case NOTT_ERR_UNSUPPORTED: return "unsupported configuration";
        case NOTT_ERR_HIP: return "HIP runtime error";
        case NOTT_ERR_ALLOC: return "allocation failure";
        case NOTT_ERR_DEVICE: return "device-reported data error";
        default: return "unknown status";
    }
}

int nott_create(int device, nott_ctx* out) {
    if (!out) return NOTT_ERR_INVALID_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return NOTT_ERR_INVALID_ARG;
    nott_ctx c = new (std::nothrow) nott_ctx_s();
    if (!c) return NOTT_ERR_ALLOC;
    c->device = device;
    nott::DeviceScope scope(device);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->num_cu = prop.multiProcessorCount;
    // NOTT_CONV_TAP=0 keeps convolutions off the conv_tap kernels (their
    // column / generic paths run instead), so both implementations can be
    // checked and timed against each other.
    if (const char* e = std::getenv("NOTT_CONV_TAP")) c->conv_tap = (e[0] != '0');
    if (const char* e = std::getenv("NOTT_CONV_DMA")) c->conv_dma = std::atoi(e);
    if (hipMalloc(&c->err_word, sizeof(unsigned long long)) != hipSuccess) {
        delete c;
        return NOTT_ERR_ALLOC;
    }
    if (hipMemset(c->err_word, 0, sizeof(unsigned long long)) != hipSuccess) {
        (void)hipFree(c->err_word);
        delete c;
        return NOTT_ERR_HIP;
    }
    const int st = nott::layernorm_scratch_setup(c);
    if (st != NOTT_OK) {
        (void)hipFree(c->err_word);
        delete c;
        return st;
    }
    *out = c;
    return NOTT_OK;
}

int nott_destroy(nott_ctx ctx) {
    if (!ctx) return NOTT_OK;
    {
        nott::DeviceScope scope(ctx->device);
        (void)hipDeviceSynchronize();
        if (ctx->ws) (void)hipFree(ctx->ws);
        for (void* r : ctx->retired) (void)hipFree(r);
        if (ctx->err_word) (void)hipFree(ctx->err_word);
    }
    delete ctx;
    return NOTT_OK;
}

int nott_set_stream(nott_ctx ctx, void* hip_stream) {
    NOTT_CHECK_CTX(ctx);
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return NOTT_OK;
}

void* nott_get_stream(nott_ctx ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

const char* nott_last_error(nott_ctx ctx) { return ctx ? ctx->last_error.c_str() : "null context"; }

int nott_device_errors(nott_ctx ctx, int64_t* count) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, count != nullptr, "count is null");
    nott::DeviceScope scope(ctx->device);
    unsigned long long h = 0;
    NOTT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    NOTT_HIP(ctx, hipMemcpy(&h, ctx->err_word, sizeof(h), hipMemcpyDeviceToHost));
    NOTT_HIP(ctx, hipMemset(ctx->err_word, 0, sizeof(h)));
    *count = (int64_t)h;
    return NOTT_OK;
}

int nott_workspace_bytes(nott_ctx ctx, int64_t* bytes) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, bytes != nullptr, "bytes is null");
    *bytes = (int64_t)(ctx->ws_bytes + ctx->retired_bytes);
    return NOTT_OK;
}

}  // extern "C"
