// Internal launch interface between the C ABI (abi.cpp) and the kernel
// translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ep {

// Everything that describes one packed weight W[N, K].
struct PackedDesc {
    const uint8_t *packed;
    const void *scale;
    int scale_dtype;
    int64_t ld_scale;
    const void *cb;
    int cb_dtype;
    int levels;
    int group;
    int64_t N, K;
    int bits() const { return levels <= 16 ? 4 : 8; }
};

struct ActDesc {
    const void *ptr;
    int dtype;
    int64_t ld;
};

struct OutDesc {
    void *ptr;
    int dtype;
    int64_t ld;
    int accumulate;
};

// Sets the calling thread's error message; returns `code`.
int set_error(int code, const char *fmt, ...);

// All launchers return EP_OK / a decline code (> 0) / an error (< 0).
int launch_gemv(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                hipStream_t stream);
int launch_gemv_generic(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                        hipStream_t stream);
bool gemv_serves(const PackedDesc &w, const ActDesc &x, int64_t M);

int launch_mfma(const PackedDesc &w, const ActDesc &x, int64_t M, const OutDesc &y,
                void *ws, size_t ws_bytes, hipStream_t stream);
bool mfma_serves(const PackedDesc &w, const ActDesc &x, int64_t M);
size_t mfma_workspace(int64_t M);

int launch_backward(const PackedDesc &w, const ActDesc &gy, const ActDesc &x, int64_t M,
                    const OutDesc &gx, float *grad_cb, float *grad_scale, int64_t ld_gscale,
                    void *ws, size_t ws_bytes, hipStream_t stream);
size_t backward_workspace(int64_t M, int64_t N, int64_t K, int levels, int group);

int launch_unpack(const uint8_t *packed, int64_t n, int levels, uint8_t *idx, hipStream_t stream);
int launch_dequant_tile(const PackedDesc &w, void *out, int out_dtype, int64_t ldo,
                        hipStream_t stream);

// Checks a HIP call; on failure records the error and returns EP_ERR_HIP.
#define EP_HIP_CHECK(expr)                                                                 \
    do {                                                                                   \
        hipError_t _e = (expr);                                                            \
        if (_e != hipSuccess)                                                              \
            return ::ep::set_error(EP_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
    } while (0)

}  // namespace ep
