// Packed half-length real FFT of 65536-sample slices, forward and inverse.
//
// L = 32768 = 128 x 256 four-step decomposition, n = 256 n1 + n2,
// k = k1 + 128 k2, in two passes over HBM per direction:
//   column pass  for each n2: V = DFT_128 over n1, times W_L^{n2 k1},
//                stored row-major Y[k1][n2] (16 consecutive n2 per workgroup
//                = 128-byte runs)
//   row pass     for each k1: DFT_256 over n2 of Y[k1][:], transposed in LDS
//                and stored at natural index k1 + 128 k2 (16 consecutive k1
//                per workgroup = 128-byte runs).
// Forward: the column pass reads the real slice as complex pairs
// z[n] = x[2n] + i x[2n+1] directly (the pack costs nothing).
// Inverse: the column pass sums each bin's scatter slots (two dense planes
// plus, for the few bins flagged in the table's overflow bitmask, two
// overflow slots) and retangles the half spectrum on load,
//   E = (F[i] + conj F[L-i])/2,  O = (F[i] - conj F[L-i])/2 * conj(W_N^i),
//   W = conj(E + i O),
// the row pass runs the same forward FFT and unpacks on store,
//   y[2k] = Re/L, y[2k+1] = -Im/L.
// Reference semantics: packedfft.cu:100-169 (three radix-32 passes, separate
// retangle/unpack launches and a permuted output order there).
#include "fcqt_fft.hpp"
#include "fcqt_abi_internal.hpp"

namespace fcqt {

constexpr int kColsPerWg = 16;                 // column pass: 16 columns x 128 rows
constexpr int kRowsPerWg = 16;                 // row pass: 16 rows x 256 columns
constexpr int kColWgs = 256 / kColsPerWg;      // 16 workgroups per slice
constexpr int kRowWgs = 128 / kRowsPerWg;      // 8 workgroups per slice

// ------------------------------------------------------------ column pass

// Value of half-spectrum bin i (0 <= i <= L) from its scatter slots.
__device__ __forceinline__ float2 load_bin(const float2* __restrict__ fb, const int* __restrict__ ovf, int i) {
    float2 v = cadd(fb[i], fb[kFStride + i]);
    const unsigned w = (unsigned)ovf[i >> 5];
    const unsigned bit = 1u << (i & 31);
    if (w & bit) {
        int k = ovf[kMaskWords + (i >> 5)] + __popc(w & (bit - 1u));
        k = min(k, kOvfCap - 1);
        const float2* o = fb + 2 * kFStride + 2 * k;
        v = cadd(v, cadd(o[0], o[1]));
    }
    return v;
}

template <bool INVERSE>
__global__ __launch_bounds__(128) void k_col_pass(const float2* __restrict__ in,
                                                  float2* __restrict__ out,
                                                  const float2* __restrict__ twp,
                                                  const float2* __restrict__ twn,
                                                  const int* __restrict__ ovf,
                                                  const float2* __restrict__ tws) {
    using P = Plan<128>;
    __shared__ float2 lds[kColsPerWg * P::US];
    const int b = blockIdx.x / kColWgs;
    const int cg = blockIdx.x - b * kColWgs;
    const int c = threadIdx.x & (kColsPerWg - 1);  // column within the tile
    const int t = threadIdx.x >> 4;                // thread within the column FFT, < 8
    const int n2 = cg * kColsPerWg + c;
    float2 v[16];
    if constexpr (!INVERSE) {
        const float2* xb = in + (long)b * kL;
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = xb[256 * (t + 8 * r) + n2];
    } else {
        const float2* fb = in + (long)b * kFRow;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = 256 * (t + 8 * r) + n2;
            float2 f0 = load_bin(fb, ovf, i);
            float2 f1 = load_bin(fb, ovf, kL - i);
            if (i == 0) {  // bins 0 and L are real for irfft
                f0.y = 0.0f;
                f1.y = 0.0f;
            }
            const float2 e = make_float2(0.5f * (f0.x + f1.x), 0.5f * (f0.y - f1.y));
            const float2 d = make_float2(0.5f * (f0.x - f1.x), 0.5f * (f0.y + f1.y));
            const float2 o = cmulc(d, twn[i]);
            v[r] = make_float2(e.x - o.y, -(e.y + o.x));
        }
    }
    fft_unit<128, -1>(v, lds + c * P::US, t, tws);
    // v[q*8 + r] = V[k1], k1 = t + 8 q + 16 r
    float2* yb = out + (long)b * kL;
#pragma unroll
    for (int q = 0; q < P::QL; ++q) {
#pragma unroll
        for (int r = 0; r < P::RL; ++r) {
            const int k1 = t + 8 * q + 16 * r;
            const int o = k1 * 256 + n2;
            yb[o] = cmul(v[q * P::RL + r], twp[o]);
        }
    }
}

// --------------------------------------------------------------- row pass

template <bool INVERSE>
__global__ __launch_bounds__(256) void k_row_pass(const float2* __restrict__ in,
                                                  float2* __restrict__ out,
                                                  const float2* __restrict__ tws) {
    using P = Plan<256>;
    __shared__ float2 lds[kRowsPerWg * P::US];
    const int b = blockIdx.x / kRowWgs;
    const int rg = blockIdx.x - b * kRowWgs;
    const int rho = threadIdx.x >> 4;   // row within the tile
    const int t = threadIdx.x & 15;     // thread within the row FFT
    const int k1 = rg * kRowsPerWg + rho;
    const float2* yb = in + (long)b * kL + (long)k1 * 256;
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = yb[t + 16 * r];
    float2* s = lds + rho * P::US;
    fft_unit<256, -1>(v, s, t, tws);
    // v[r] = X_row[k2], k2 = t + 16 r ; transpose through LDS so that lanes
    // walk consecutive k1 for the store at k1 + 128 k2.
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) s[pad16(t + 16 * r)] = v[r];
    __syncthreads();
    const int rho2 = threadIdx.x & 15;
    const int kg = threadIdx.x >> 4;
    const float2* s2 = lds + rho2 * P::US;
    const int kk1 = rg * kRowsPerWg + rho2;
    if constexpr (!INVERSE) {
        float2* zb = out + (long)b * kL;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int k2 = kg + 16 * u;
            zb[kk1 + 128 * k2] = s2[pad16(k2)];
        }
    } else {
        constexpr float sc = 1.0f / (float)kL;
        float2* yo = out + (long)b * kL;  // y viewed as [batch][32768] float pairs
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int k2 = kg + 16 * u;
            const float2 w = s2[pad16(k2)];
            yo[kk1 + 128 * k2] = make_float2(w.x * sc, -w.y * sc);
        }
    }
}

}  // namespace fcqt

using namespace fcqt;

extern "C" int fcqt_packed_fft_fwd(const fcqt_tables* tab, const float* x, float* z, float* work,
                                   int64_t batch, hipStream_t stream) {
    if (!tab || !x || !z || !work || batch < 1 || batch > kMaxBatch) return FCQT_EARG;
    if (!tab->tw_pass || !tab->tw_stage) return FCQT_EARG;
    if (!aligned(x, 8) || !aligned(z, 8) || !aligned(work, 8) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_stage, 16))
        return FCQT_EALIGN;
    const auto* tws = reinterpret_cast<const float2*>(tab->tw_stage);
    hipLaunchKernelGGL(k_col_pass<false>, dim3((unsigned)(batch * kColWgs)), dim3(128), 0, stream,
                       reinterpret_cast<const float2*>(x), reinterpret_cast<float2*>(work),
                       reinterpret_cast<const float2*>(tab->tw_pass), nullptr, nullptr, tws);
    if (int e = launch_status()) return e;
    hipLaunchKernelGGL(k_row_pass<false>, dim3((unsigned)(batch * kRowWgs)), dim3(256), 0, stream,
                       reinterpret_cast<const float2*>(work), reinterpret_cast<float2*>(z), tws);
    return launch_status();
}

extern "C" int fcqt_packed_fft_inv(const fcqt_tables* tab, const int32_t* ovf, const float* f, float* y,
                                   float* work, int64_t batch, hipStream_t stream) {
    if (!tab || !ovf || !f || !y || !work || batch < 1 || batch > kMaxBatch) return FCQT_EARG;
    if (!tab->tw_pass || !tab->tw_half || !tab->tw_stage) return FCQT_EARG;
    if (!aligned(f, 16) || !aligned(y, 8) || !aligned(work, 8) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_half, 8) || !aligned(tab->tw_stage, 16) || !aligned(ovf, 4))
        return FCQT_EALIGN;
    const auto* tws = reinterpret_cast<const float2*>(tab->tw_stage);
    hipLaunchKernelGGL(k_col_pass<true>, dim3((unsigned)(batch * kColWgs)), dim3(128), 0, stream,
                       reinterpret_cast<const float2*>(f), reinterpret_cast<float2*>(work),
                       reinterpret_cast<const float2*>(tab->tw_pass),
                       reinterpret_cast<const float2*>(tab->tw_half), reinterpret_cast<const int*>(ovf), tws);
    if (int e = launch_status()) return e;
    hipLaunchKernelGGL(k_row_pass<true>, dim3((unsigned)(batch * kRowWgs)), dim3(256), 0, stream,
                       reinterpret_cast<const float2*>(work), reinterpret_cast<float2*>(y), tws);
    return launch_status();
}
