// C-ABI entry points that compose the engines (analysis, synthesis), the
// allocation-free analysis, the graph-safe zero fill and the status helpers.
#include <mutex>

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
        case FCQT_ECAPACITY: return "batch exceeds the static scratch capacity (FCQT_STATIC_MAX_BATCH slices)";
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
    if (batch < kAnalysisChunkMinBatch) {
        if (int e = fcqt_packed_fft_fwd(tab, x, xs, work, batch, stream)) return e;
        return fcqt_route_bands(tab, route, xs, coef_re, coef_im, layout, batch, stream);
    }
    // Large batches run in chunks of kAnalysisChunk slices, all three
    // kernels per chunk, so that a chunk's W and X (0.5 MB per slice) are
    // still in the memory-side cache when its row pass and route read them;
    // over a whole large batch they are not, and the route's gathers wait on
    // HBM. One call against chunks of 128 (stream launches, hipEvents):
    // B = 256 145 against 135 us, 384 261 against 208, 512 372 against 272,
    // 1024 700 against 553; at B = 192 one call was faster (95-97 against
    // 115 us). Slices are independent and every batch form gives the same
    // bits, so the results do not depend on the chunking.
    const int64_t cstride = layout == FCQT_PLANAR ? tab->ncoef : 2 * tab->ncoef;   // floats per coefficient row
    for (int64_t lo = 0; lo < batch; lo += kAnalysisChunk) {
        const int64_t n = batch - lo < kAnalysisChunk ? batch - lo : kAnalysisChunk;
        float* xs_c = xs + lo * 2 * (int64_t)kXStride;
        if (int e = fcqt_packed_fft_fwd(tab, x + lo * (int64_t)kN, xs_c, work + lo * 2 * (int64_t)kL, n, stream))
            return e;
        if (int e = fcqt_route_bands(tab, route, xs_c, coef_re + lo * cstride,
                                     layout == FCQT_PLANAR ? coef_im + lo * cstride : coef_im, layout, n, stream))
            return e;
    }
    return FCQT_OK;
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

extern "C" int fcqt_stream_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* groups,
                                     const int32_t* ovf, const float* coef, float* f, float* work, float* y,
                                     float* tail, float* out, int64_t nsig, int64_t slice, hipStream_t stream) {
    if (!scat || !groups || !ovf || !coef || !f || !work || !y || !tail) return FCQT_EARG;
    if (slice > 0 && !out) return FCQT_EARG;
    // every later step's arguments before the first launch
    if (!tab || !tab->tw_pass || !tab->tw_half || nsig < 1 || nsig > 65535 || slice < 0 || slice > kMaxBatch)
        return FCQT_EARG;
    if (int e = check_band_args(tab, scat, coef, coef, FCQT_INTERLEAVED, nsig)) return e;
    if (!aligned(f, 16) || !aligned(y, 8) || !aligned(work, 8) || !aligned(ovf, 4) || !aligned(groups, 16) ||
        !aligned(tail, 4) || (out && !aligned(out, 4)))
        return FCQT_EALIGN;
    if (int e = fcqt_scatter_bands_sliced(tab, scat, groups, coef, f, nsig, 1, slice, stream)) return e;
    if (int e = fcqt_packed_fft_inv(tab, ovf, f, y, work, nsig, stream)) return e;
    return fcqt_stream_overlap(y, tail, out, nsig, slice, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free analysis. The spectrum X and the four-step intermediate W
// of up to FCQT_STATIC_MAX_BATCH slices live in this file-scope device array
// (every GPU the library runs on holds its own copy until the process ends).
// Both are fully overwritten by every call, so nothing needs clearing. Host
// code never passes the array's name to a kernel: the device address of each
// GPU's copy is looked up once per device (hipGetSymbolAddress, with that
// device current) and that address is passed instead.
namespace fcqt {

constexpr int64_t kStaticXs = (int64_t)FCQT_STATIC_MAX_BATCH * kXStride;   // complex elements of X
constexpr int64_t kStaticWork = (int64_t)FCQT_STATIC_MAX_BATCH * kL;      // complex elements of W
static __device__ __align__(256) float2 scratch[kStaticXs + kStaticWork];

constexpr int kMaxDevices = 64;

// Device address of this GPU's scratch (FCQT_OK), resolved on first use.
static int scratch_address(int device, float2** out) {
    static std::mutex mu;
    static float2* addr[kMaxDevices] = {};
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            std::snprintf(last_error_buf(), 256, "hipGetSymbolAddress: %s (%d)", hipGetErrorString(e), (int)e);
            return FCQT_ELAUNCH;
        }
        addr[device] = static_cast<float2*>(p);
    }
    *out = addr[device];
    return FCQT_OK;
}

}  // namespace fcqt

extern "C" int fcqt_analysis_static(const fcqt_tables* tab, const int32_t* route, const float* x, float* coef_re,
                                    float* coef_im, int layout, int64_t batch, hipStream_t stream) {
    if (!route || !x) return FCQT_EARG;
    if (int e = check_band_args(tab, route, coef_re, coef_im, layout, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    if (batch > FCQT_STATIC_MAX_BATCH) return FCQT_ECAPACITY;
    if (!aligned(x, 8) || !aligned(tab->tw_pass, 8) || !aligned(tab->tw_half, 8)) return FCQT_EALIGN;
    // the scratch of the GPU the launches go to: the stream's device, which
    // must be the current one (hipGetSymbolAddress resolves for it)
    int cur = -1, dev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess) e = stream ? hipStreamGetDevice(stream, &dev) : (dev = cur, hipSuccess);
    if (e != hipSuccess) {
        std::snprintf(last_error_buf(), 256, "%s (%d)", hipGetErrorString(e), (int)e);
        return FCQT_ELAUNCH;
    }
    if (dev != cur || dev < 0 || dev >= kMaxDevices) return FCQT_EARG;
    float2* base = nullptr;
    if (int r = scratch_address(dev, &base)) return r;
    float* xs = reinterpret_cast<float*>(base);
    float* work = reinterpret_cast<float*>(base + kStaticXs);
    if (int r = fcqt_packed_fft_fwd(tab, x, xs, work, batch, stream)) return r;
    return fcqt_route_bands(tab, route, xs, coef_re, coef_im, layout, batch, stream);
}
