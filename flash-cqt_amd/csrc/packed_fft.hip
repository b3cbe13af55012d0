// Real FFT of 65536-sample slices (forward: rfft, inverse: irfft) as a packed
// half-length complex FFT, L = 32768 = 128 x 256, four-step decomposition
// n = 256 n1 + n2, k = k1 + 128 k2, two passes over HBM per direction:
//   column pass  for each n2: V = DFT_128 over n1, times W_L^{n2 k1},
//                stored row-major Y[k1][n2]
//   row pass     for each k1: DFT_256 over n2 of Y[k1][:], stored at the
//                natural index k1 + 128 k2.
// Forward: the column pass reads the real slice as complex pairs
// z[n] = x[2n] + i x[2n+1] directly; the row pass pairs every row k1 with its
// mirror row 128 - k1 (rows 0 and 64 are their own mirrors) in one
// workgroup, so it can untangle on the way out:
//   X[k] = cA(k) Z[k] + cB(k) conj Z[L-k],  cA = (1 - i W_N^k)/2, cB = 1 - cA,
// and it writes the real FFT X[0..L] itself (X[L] = Re Z[0] - Im Z[0]).
// Inverse: the column pass pairs every column n2 with its mirror 256 - n2
// (columns 0 and 128 are their own mirrors), stages each bin's value (the sum
// of its scatter slots: two dense slot planes plus, for the bins on the table's
// overflow fold list of this workgroup, two overflow slots) in LDS, and
// retangles there,
//   E = (F[i] + conj F[L-i])/2,  O = (F[i] - conj F[L-i])/2 conj(W_N^i),
//   W = conj(E + i O),
// so every bin is read from memory once; the row pass runs the same forward
// FFT and unpacks on store, y[2k] = Re/L, y[2k+1] = -Im/L.
// Reference semantics: packedfft.cu:100-169 (three radix-32 passes, separate
// retangle/unpack launches and a permuted output order there) and the
// untangle of radix_impl.cuh:27-42, which this engine moves out of the band
// kernels.
#include "fcqt_passes.hpp"
#include "fcqt_abi_internal.hpp"

namespace fcqt {

template <bool SLICED, int CPW>
__global__ __launch_bounds__(8 * CPW) void k_col_fwd(const float2* __restrict__ in, float2* __restrict__ out,
                                                     const float2* __restrict__ twp,
                                                     const float2* __restrict__ tws, const SliceSrc src) {
    constexpr int kWgs = 256 / CPW;               // workgroups per slice
    __shared__ float2 lds[col_lds<CPW>()];
    const int lg = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int b = lg / kWgs;
    col_fwd_tile<SLICED, CPW>(b, lg - b * kWgs, in, out, twp, tws, src, lds);
}

template <int CPW, bool WT>
__global__ __launch_bounds__(8 * CPW) void k_col_inv(const float2* __restrict__ f, float2* __restrict__ out,
                                                     const float2* __restrict__ twp,
                                                     const float2* __restrict__ twn,
                                                     const int* __restrict__ fold,
                                                     const float2* __restrict__ tws) {
    constexpr int kWgs = 256 / CPW;               // workgroups per slice
    __shared__ float2 lds[col_lds<CPW>()];
    const int lg = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int b = lg / kWgs;
    col_inv_tile<CPW, WT>(b, lg - b * kWgs, f, out, twp, twn, fold, tws, lds);
}

template <int RPW>
__global__ __launch_bounds__(16 * RPW) void k_row_fwd(const float2* __restrict__ in, float2* __restrict__ xs,
                                                      const float2* __restrict__ twn,
                                                      const float2* __restrict__ tws) {
    constexpr int kWgs = 128 / RPW;               // workgroups per slice
    __shared__ float2 lds[row_lds<RPW>()];
    const int lg = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int b = lg / kWgs;
    row_fwd_tile<RPW>(b, lg - b * kWgs, in, xs, twn, tws, lds);
}

template <int RPW, bool WT>
__global__ __launch_bounds__(16 * RPW) void k_row_inv(const float2* __restrict__ in, float2* __restrict__ y,
                                                      const float2* __restrict__ tws) {
    constexpr int kWgs = 128 / RPW;               // workgroups per slice
    __shared__ float2 lds[row_lds<RPW>()];
    const int lg = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int b = lg / kWgs;
    row_inv_tile<RPW, WT>(b, lg - b * kWgs, in, y, tws, lds);
}

// Launch helpers: the pass kernels of one direction in the tile shape the
// batch size selects.
template <int CPW, int RPW>
static int launch_fwd_passes(const float2* x, float2* work, float2* xs, const float2* twp, const float2* twh,
                             const float2* tws, const SliceSrc& src, bool sliced, int64_t batch,
                             hipStream_t stream) {
    const dim3 gc((unsigned)(batch * (256 / CPW))), gr((unsigned)(batch * (128 / RPW)));
    if (sliced)
        hipLaunchKernelGGL((k_col_fwd<true, CPW>), gc, dim3(8 * CPW), 0, stream, x, work, twp, tws, src);
    else
        hipLaunchKernelGGL((k_col_fwd<false, CPW>), gc, dim3(8 * CPW), 0, stream, x, work, twp, tws, src);
    if (int e = launch_status()) return e;
    hipLaunchKernelGGL((k_row_fwd<RPW>), gr, dim3(16 * RPW), 0, stream, work, xs, twh, tws);
    return launch_status();
}

static int fwd_passes(const float2* x, float2* work, float2* xs, const float2* twp, const float2* twh,
                      const float2* tws, const SliceSrc& src, bool sliced, int64_t batch, hipStream_t stream) {
    if (batch <= kNarrowMaxBatch)
        return launch_fwd_passes<kColsNarrow, kRowsNarrow>(x, work, xs, twp, twh, tws, src, sliced, batch, stream);
    return launch_fwd_passes<kColsWide, kRowsWide>(x, work, xs, twp, twh, tws, src, sliced, batch, stream);
}

template <int CPW, int RPW, bool WT>
static int launch_inv_passes(const float2* f, float2* work, float2* y, const float2* twp, const float2* twh,
                             const int* ovf, const float2* tws, int64_t batch, hipStream_t stream) {
    hipLaunchKernelGGL((k_col_inv<CPW, WT>), dim3((unsigned)(batch * (256 / CPW))), dim3(8 * CPW), 0, stream, f,
                       work, twp, twh, ovf, tws);
    if (int e = launch_status()) return e;
    hipLaunchKernelGGL((k_row_inv<RPW, WT>), dim3((unsigned)(batch * (128 / RPW))), dim3(16 * RPW), 0, stream, work,
                       y, tws);
    return launch_status();
}

static int inv_passes(const float2* f, float2* work, float2* y, const float2* twp, const float2* twh, const int* ovf,
                      const float2* tws, int64_t batch, hipStream_t stream) {
    if (batch <= kNarrowMaxBatch)
        return launch_inv_passes<kInvColsNarrow, kRowsNarrow, false>(f, work, y, twp, twh, ovf, tws, batch, stream);
    if (batch <= kInvWriteThroughMaxBatch)
        return launch_inv_passes<kInvColsWide, kRowsWide, true>(f, work, y, twp, twh, ovf, tws, batch, stream);
    return launch_inv_passes<kInvColsWide, kRowsWide, false>(f, work, y, twp, twh, ovf, tws, batch, stream);
}

// The inverse row pass with the sliced overlap-add in its store
// (row_inv_ola_tile): the slices of one parity of nsig signals x S slices,
// nper of them per signal; work row sig * S + s, output row sig of `length`.
template <int RPW, bool ODD, bool PAIR>
__global__ __launch_bounds__(16 * RPW) void k_row_inv_ola(const float2* __restrict__ in, float* __restrict__ out,
                                                          const float2* __restrict__ tws, int S, long length,
                                                          int nper) {
    constexpr int kWgs = 128 / RPW;               // workgroups per slice
    __shared__ float2 lds[row_lds<RPW>()];
    const int lg = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int r = lg / kWgs;                      // sig * nper + m: slice s = 2 m + ODD of signal sig
    const int sig = r / nper;
    const int s = 2 * (r - sig * nper) + (ODD ? 1 : 0);
    row_inv_ola_tile<RPW, ODD, PAIR>(sig * S + s, lg - r * kWgs, s, S, length, in, out + (long)sig * length, tws,
                                     lds);
}

// The inverse column pass alone, in the shape inv_passes picks for the batch.
static int col_inv_pass(const float2* f, float2* work, const float2* twp, const float2* twh, const int* ovf,
                        const float2* tws, int64_t batch, hipStream_t stream) {
    if (batch <= kNarrowMaxBatch)
        hipLaunchKernelGGL((k_col_inv<kInvColsNarrow, false>), dim3((unsigned)(batch * (256 / kInvColsNarrow))),
                           dim3(8 * kInvColsNarrow), 0, stream, f, work, twp, twh, ovf, tws);
    else if (batch <= kInvWriteThroughMaxBatch)
        hipLaunchKernelGGL((k_col_inv<kInvColsWide, true>), dim3((unsigned)(batch * (256 / kInvColsWide))),
                           dim3(8 * kInvColsWide), 0, stream, f, work, twp, twh, ovf, tws);
    else
        hipLaunchKernelGGL((k_col_inv<kInvColsWide, false>), dim3((unsigned)(batch * (256 / kInvColsWide))),
                           dim3(8 * kInvColsWide), 0, stream, f, work, twp, twh, ovf, tws);
    return launch_status();
}

// Both parities of the fused row pass: the even slices' launch, then the odd.
template <int RPW, bool PAIR>
static int row_inv_ola_passes(const float2* work, float* out, const float2* tws, int64_t nsig, int64_t S,
                              int64_t length, hipStream_t stream) {
    constexpr int kWgs = 128 / RPW;
    const int64_t even = (S + 1) / 2, odd = S / 2;
    hipLaunchKernelGGL((k_row_inv_ola<RPW, false, PAIR>), dim3((unsigned)(nsig * even * kWgs)), dim3(16 * RPW), 0,
                       stream, work, out, tws, (int)S, (long)length, (int)even);
    if (int e = launch_status()) return e;
    if (odd == 0) return FCQT_OK;
    hipLaunchKernelGGL((k_row_inv_ola<RPW, true, PAIR>), dim3((unsigned)(nsig * odd * kWgs)), dim3(16 * RPW), 0,
                       stream, work, out, tws, (int)S, (long)length, (int)odd);
    return launch_status();
}

}  // namespace fcqt

using namespace fcqt;

extern "C" int fcqt_sliced_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* groups,
                                     const int32_t* ovf, const float* coef, float* f, float* work, float* out,
                                     int64_t nsig, int64_t nslices, int64_t length, hipStream_t stream) {
    if (!scat || !groups || !ovf || !coef || !f || !work || !out) return FCQT_EARG;
    if (nsig < 1 || nslices < 1 || nsig > kMaxBatch || nslices > kMaxBatch || nsig * nslices > kMaxBatch)
        return FCQT_EARG;
    if (length < 1 || length > nslices * 2 * (int64_t)kQuarter) return FCQT_EARG;
    const int64_t batch = nsig * nslices;
    // every step's arguments before the first launch
    if (int e = check_band_args(tab, scat, coef, coef, FCQT_INTERLEAVED, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half || !tab->tw_stage) return FCQT_EARG;
    if (!aligned(f, 16) || !aligned(groups, 16) || !aligned(work, 8) || !aligned(ovf, 4) || !aligned(out, 4) ||
        !aligned(tab->tw_pass, 8) || !aligned(tab->tw_half, 8) || !aligned(tab->tw_stage, 16))
        return FCQT_EALIGN;
    if (int e = fcqt_scatter_bands_sliced(tab, scat, groups, coef, f, nsig, nslices, 0, stream)) return e;
    const auto* tws = reinterpret_cast<const float2*>(tab->tw_stage);
    auto* w2 = reinterpret_cast<float2*>(work);
    if (int e = col_inv_pass(reinterpret_cast<const float2*>(f), w2, reinterpret_cast<const float2*>(tab->tw_pass),
                             reinterpret_cast<const float2*>(tab->tw_half), reinterpret_cast<const int*>(ovf), tws,
                             batch, stream))
        return e;
    const bool pair = length % 2 == 0 && aligned(out, 8);
    if (batch <= kNarrowMaxBatch)
        return pair ? row_inv_ola_passes<kRowsNarrow, true>(w2, out, tws, nsig, nslices, length, stream)
                    : row_inv_ola_passes<kRowsNarrow, false>(w2, out, tws, nsig, nslices, length, stream);
    return pair ? row_inv_ola_passes<kRowsWide, true>(w2, out, tws, nsig, nslices, length, stream)
                : row_inv_ola_passes<kRowsWide, false>(w2, out, tws, nsig, nslices, length, stream);
}

extern "C" int fcqt_packed_fft_fwd(const fcqt_tables* tab, const float* x, float* xs, float* work,
                                   int64_t batch, hipStream_t stream) {
    if (!tab || !x || !xs || !work || batch < 1 || batch > kMaxBatch) return FCQT_EARG;
    if (!tab->tw_pass || !tab->tw_half || !tab->tw_stage) return FCQT_EARG;
    if (!aligned(x, 8) || !aligned(xs, 8) || !aligned(work, 8) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_half, 8) || !aligned(tab->tw_stage, 16))
        return FCQT_EALIGN;
    return fwd_passes(reinterpret_cast<const float2*>(x), reinterpret_cast<float2*>(work),
                      reinterpret_cast<float2*>(xs), reinterpret_cast<const float2*>(tab->tw_pass),
                      reinterpret_cast<const float2*>(tab->tw_half), reinterpret_cast<const float2*>(tab->tw_stage),
                      SliceSrc{nullptr, nullptr, 1, 1, 0, 0, 0, nullptr, 1, 1, 1}, false, batch, stream);
}

extern "C" int fcqt_packed_fft_inv(const fcqt_tables* tab, const int32_t* ovf, const float* f, float* y,
                                   float* work, int64_t batch, hipStream_t stream) {
    if (!tab || !ovf || !f || !y || !work || batch < 1 || batch > kMaxBatch) return FCQT_EARG;
    if (!tab->tw_pass || !tab->tw_half || !tab->tw_stage) return FCQT_EARG;
    if (!aligned(f, 16) || !aligned(y, 8) || !aligned(work, 8) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_half, 8) || !aligned(tab->tw_stage, 16) || !aligned(ovf, 4))
        return FCQT_EALIGN;
    return inv_passes(reinterpret_cast<const float2*>(f), reinterpret_cast<float2*>(work),
                      reinterpret_cast<float2*>(y), reinterpret_cast<const float2*>(tab->tw_pass),
                      reinterpret_cast<const float2*>(tab->tw_half), reinterpret_cast<const int*>(ovf),
                      reinterpret_cast<const float2*>(tab->tw_stage), batch, stream);
}

extern "C" int fcqt_slice_fft_fwd(const fcqt_tables* tab, const float* sig, int64_t sig_len, const float* window,
                                  int64_t nsig, int64_t nslices, int64_t first, int64_t origin, float* xs,
                                  float* work, hipStream_t stream) {
    if (!tab || !sig || !window || !xs || !work || sig_len < 1 || nsig < 1 || nslices < 1) return FCQT_EARG;
    if (first < 0 || first > kMaxBatch || origin < -(int64_t)kN || origin > (int64_t)kN * kMaxBatch)
        return FCQT_EARG;
    if (nsig > kMaxBatch || nslices > kMaxBatch || nsig * nslices > kMaxBatch) return FCQT_EARG;
    if (!tab->tw_pass || !tab->tw_half || !tab->tw_stage) return FCQT_EARG;
    if (!aligned(sig, 4) || !aligned(window, 4) || !aligned(xs, 8) || !aligned(work, 8) ||
        !aligned(tab->tw_pass, 8) || !aligned(tab->tw_half, 8) || !aligned(tab->tw_stage, 16))
        return FCQT_EALIGN;
    const int64_t batch = nsig * nslices;
    // pair loads when every sample pair is aligned and wholly inside or outside the signal
    const int pairs = sig_len >= 2 && sig_len % 2 == 0 && origin % 2 == 0 && aligned(sig, 8) && aligned(window, 8);
    return fwd_passes(nullptr, reinterpret_cast<float2*>(work), reinterpret_cast<float2*>(xs),
                      reinterpret_cast<const float2*>(tab->tw_pass), reinterpret_cast<const float2*>(tab->tw_half),
                      reinterpret_cast<const float2*>(tab->tw_stage),
                      SliceSrc{sig, window, (long)sig_len, (int)nslices, (long)first, (long)origin, pairs, nullptr,
                               (long)sig_len, (long)sig_len, (long)sig_len},
                      true, batch, stream);
}

extern "C" int fcqt_stream_analysis(const fcqt_tables* tab, const int32_t* route, const int32_t* groups,
                                    const float* prev, int64_t prev_stride, const float* next, int64_t next_stride,
                                    const float* window, int64_t nsig, int64_t slice, float* coef, float* xs,
                                    float* work, hipStream_t stream) {
    constexpr long kHop = kN / 2;
    if (!tab || !route || !groups || !prev || !next || !window || !coef || !xs || !work) return FCQT_EARG;
    if (nsig < 1 || nsig > kMaxBatch || slice < 0 || slice > kMaxBatch) return FCQT_EARG;
    if ((nsig > 1 && (prev_stride < kHop || next_stride < kHop)) || prev_stride < 0 || next_stride < 0 ||
        prev_stride > ((int64_t)1 << 40) || next_stride > ((int64_t)1 << 40))
        return FCQT_EARG;
    // the band half first, so an argument error launches nothing
    if (int e = check_band_args(tab, route, coef, coef, FCQT_INTERLEAVED, nsig)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    if (!aligned(prev, 4) || !aligned(next, 4) || !aligned(window, 4) || !aligned(xs, 8) || !aligned(work, 8) ||
        !aligned(groups, 16) || !aligned(tab->tw_pass, 8) || !aligned(tab->tw_half, 8))
        return FCQT_EALIGN;
    // slice `slice` of every signal is [prev row, next row]: the call holds
    // the signal from sample hop (slice - 1) on, N samples per row, the first
    // hop in prev and the rest in next
    const int pairs = aligned(prev, 8) && aligned(next, 8) && aligned(window, 8) && prev_stride % 2 == 0 &&
                      next_stride % 2 == 0;
    if (int e = fwd_passes(nullptr, reinterpret_cast<float2*>(work), reinterpret_cast<float2*>(xs),
                           reinterpret_cast<const float2*>(tab->tw_pass), reinterpret_cast<const float2*>(tab->tw_half),
                           reinterpret_cast<const float2*>(tab->tw_stage),
                           SliceSrc{prev, window, 2 * kHop, 1, (long)slice, kHop * ((long)slice - 1), pairs, next,
                                    (long)prev_stride, (long)next_stride, kHop},
                           true, nsig, stream))
        return e;
    return fcqt_route_bands_sliced(tab, route, groups, xs, coef, nsig, 1, slice, stream);
}

namespace fcqt {
// Overlap-add of rolled slices: out[sig][p] = sum over the (at most two)
// slices s with 0 <= q - 2H s < N, q = p + 2H, of y[sig S + s][jj],
// jj = (q - 2H s - H) mod N in even slices and (q - 2H s + H) mod N in odd
// ones (the reference's roll by +-H, overlap-add and 2H trim).
__global__ __launch_bounds__(256) void k_overlap_add(const float* __restrict__ y, float* __restrict__ out, int S,
                                                     long length) {
    const long p = (long)blockIdx.x * 256 + threadIdx.x;
    const int sig = blockIdx.y;
    if (p >= length) return;
    const long q = p + 2 * kQuarter;
    const long sh = q / (2 * kQuarter);
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const long s = sh - 1 + k;
        if (s >= 0 && s < S) {
            const int j = (int)(q - 2 * kQuarter * s);
            const int jj = (j + ((s & 1) ? kQuarter : kN - kQuarter)) & (kN - 1);
            acc += y[((long)sig * S + s) * kN + jj];
        }
    }
    out[(long)sig * length + p] = acc;
}

// The same sums four samples per thread (16-byte loads and stores), for an
// output whose rows start 16-byte aligned (length % 4 == 0, aligned y and
// out). p = 4 m: the four samples share the hop index, and jj..jj+3 stay
// inside one slice row (jj is a multiple of 4 and N is too). Same additions
// in the same order as k_overlap_add, so the same bits.
__global__ __launch_bounds__(256) void k_overlap_add4(const float4* __restrict__ y, float4* __restrict__ out,
                                                      int S, long length) {
    const long p = 4 * ((long)blockIdx.x * 256 + threadIdx.x);
    const int sig = blockIdx.y;
    if (p >= length) return;
    const long q = p + 2 * kQuarter;
    const long sh = q / (2 * kQuarter);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const long s = sh - 1 + k;
        if (s >= 0 && s < S) {
            const int j = (int)(q - 2 * kQuarter * s);
            const int jj = (j + ((s & 1) ? kQuarter : kN - kQuarter)) & (kN - 1);
            const float4 v = y[(((long)sig * S + s) * kN + jj) / 4];
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
    }
    out[((long)sig * length + p) / 4] = acc;
}
}  // namespace fcqt

namespace fcqt {
// Streamed overlap-add of one inverse slice g per signal (SlicedCQT.stream_bwd):
// with y_r the slice rolled back (y_r[j] = y[(j - H) mod N] for even g,
// y[(j + H) mod N] for odd g), out[p] = tail[p] + y_r[p] and
// tail[p] = y_r[2H + p] for p < 2H; emit = 0 (the first slice) only fills tail.
__global__ __launch_bounds__(256) void k_stream_overlap(const float* __restrict__ y, float* __restrict__ tail,
                                                        float* __restrict__ out, int odd, int emit) {
    const int p = (int)blockIdx.x * 256 + (int)threadIdx.x;   // < 2H: the grid is exact
    const long sig = blockIdx.y;
    const int sh = odd ? kQuarter : kN - kQuarter;
    const float* yr = y + sig * kN;
    float* tr = tail + sig * 2 * kQuarter;
    const float a = yr[(p + sh) & (kN - 1)];
    const float b = yr[(p + 2 * kQuarter + sh) & (kN - 1)];
    if (emit) out[sig * 2 * kQuarter + p] = tr[p] + a;
    tr[p] = b;
}
}  // namespace fcqt

extern "C" int fcqt_stream_overlap(const float* y, float* tail, float* out, int64_t nsig, int64_t slice,
                                   hipStream_t stream) {
    if (!y || !tail || nsig < 1 || nsig > 65535 || slice < 0) return FCQT_EARG;
    if (slice > 0 && !out) return FCQT_EARG;
    if (!aligned(y, 4) || !aligned(tail, 4) || (out && !aligned(out, 4))) return FCQT_EALIGN;
    static_assert((2 * kQuarter) % 256 == 0, "exact grid");
    hipLaunchKernelGGL(k_stream_overlap, dim3((unsigned)(2 * kQuarter / 256), (unsigned)nsig), dim3(256), 0, stream,
                       y, tail, out, (int)(slice & 1), slice > 0 ? 1 : 0);
    return launch_status();
}

extern "C" int fcqt_overlap_add(const float* y, float* out, int64_t nsig, int64_t nslices, int64_t length,
                                hipStream_t stream) {
    if (!y || !out || nsig < 1 || nslices < 1 || length < 1 || nsig > 65535) return FCQT_EARG;
    if (nsig * nslices > kMaxBatch || length > nslices * 2 * (int64_t)kQuarter) return FCQT_EARG;
    if (!aligned(y, 4) || !aligned(out, 4)) return FCQT_EALIGN;
    if (length % 4 == 0 && aligned(y, 16) && aligned(out, 16)) {
        const dim3 grid4((unsigned)((length / 4 + 255) / 256), (unsigned)nsig);
        hipLaunchKernelGGL(k_overlap_add4, grid4, dim3(256), 0, stream, reinterpret_cast<const float4*>(y),
                           reinterpret_cast<float4*>(out), (int)nslices, (long)length);
        return launch_status();
    }
    const dim3 grid((unsigned)((length + 255) / 256), (unsigned)nsig);
    hipLaunchKernelGGL(k_overlap_add, grid, dim3(256), 0, stream, y, out, (int)nslices, (long)length);
    return launch_status();
}
