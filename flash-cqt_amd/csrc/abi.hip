// C-ABI entry points that compose the engines (analysis, synthesis), the
// graph-safe zero fill and the status helpers.
#include "fcqt_fft.hpp"
#include "fcqt_abi_internal.hpp"

namespace fcqt {

__global__ __launch_bounds__(256) void k_fill_zero(float4* __restrict__ p4, long n4, float* __restrict__ tail,
                                                   int ntail) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const long stride = (long)gridDim.x * 256;
    for (long j = i; j < n4; j += stride) p4[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < ntail) tail[i] = 0.0f;
}

}  // namespace fcqt

using namespace fcqt;

extern "C" int fcqt_abi_version(void) { return FCQT_ABI_VERSION; }

extern "C" const char* fcqt_status_string(int status) {
    switch (status) {
        case FCQT_OK: return "ok";
        case FCQT_EARG: return "invalid argument (null pointer, size or layout)";
        case FCQT_EALIGN: return "misaligned pointer";
        case FCQT_ELAUNCH: return "kernel launch failed";
        default: return "unknown status";
    }
}

extern "C" const char* fcqt_last_hip_error(void) { return last_error_buf(); }

extern "C" int fcqt_fill_zero(float* buf, int64_t n, hipStream_t stream) {
    if (!buf || n < 0) return FCQT_EARG;
    if (n == 0) return FCQT_OK;
    if (!aligned(buf, 4)) return FCQT_EALIGN;
    // head up to 16-byte alignment is folded into the tail handling by
    // requiring a 16-byte aligned base for the vector part
    if (!aligned(buf, 16)) return FCQT_EALIGN;
    const long n4 = (long)(n / 4);
    const int ntail = (int)(n - 4 * n4);
    long blocks = (n4 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<float4*>(buf), n4, buf + 4 * n4, ntail);
    return launch_status();
}

extern "C" int fcqt_analysis(const fcqt_tables* tab, const int32_t* route, const float* x, float* coef_re,
                             float* coef_im, int layout, float* xs, float* work, int64_t batch,
                             hipStream_t stream) {
    if (!route || !x || !xs || !work) return FCQT_EARG;
    // validate the band half before launching the FFT half
    if (int e = check_band_args(tab, route, coef_re, coef_im, layout, batch)) return e;
    if (!aligned(xs, 8)) return FCQT_EALIGN;
    if (int e = fcqt_packed_fft_fwd(tab, x, xs, work, batch, stream)) return e;
    return fcqt_route_bands(tab, route, xs, coef_re, coef_im, layout, batch, stream);
}

extern "C" int fcqt_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* ovf,
                              const float* coef_re, const float* coef_im, int layout, float* f,
                              float* work, float* y, int64_t batch, hipStream_t stream) {
    if (!scat || !ovf || !f || !work || !y) return FCQT_EARG;
    // validate the second half before launching the first, so an argument
    // error never leaves F half-written
    if (!tab || !tab->tw_pass || !tab->tw_half || batch < 1 || batch > kMaxBatch) return FCQT_EARG;
    if (!aligned(f, 16) || !aligned(y, 8) || !aligned(work, 8) || !aligned(ovf, 4)) return FCQT_EALIGN;
    if (int e = fcqt_scatter_bands(tab, scat, coef_re, coef_im, layout, f, batch, stream)) return e;
    return fcqt_packed_fft_inv(tab, ovf, f, y, work, batch, stream);
}
