// Band engines: the fused route + band inverse DFT (analysis, synthesis
// adjoint) and the band DFT + gain + scatter (synthesis, analysis adjoint).
//
// One workgroup of 128 threads (two wave64s) owns one task: up to 2048/M
// consecutive bands of one length M of one slice. Each band is one unit of
// the shared FFT engine (M/16 threads, 16 values each). Tasks come from a
// host-built table {M, first coefficient, band count, first band}; the grid
// is tasks x batch, spread so that each XCD gets a contiguous range of
// (task, slice) pairs (band_place): task-major for small batches (each XCD
// reads few tasks' record rows), slice-major from kBandSliceMajorMinBatch
// slices on (each XCD holds whole slices, the ones whose pass tiles it ran).
//
// Both engines read their per-tap records in kernel order: the table holds,
// for every task, 16 rows of 128 8-byte records, row s giving slot s of each
// thread (the host builds the permutation from the task table). A thread's
// records therefore sit at task * 2048 + s * 128 + thread: the loads depend
// on the task index only, issue before the task record arrives, and every
// load of a wave is one contiguous 512-byte run.
//
// Analysis prologue (slot r of a thread = tap t + T r of its band):
// v = w X[k], conjugated for taps past Nyquist, from the record {k, ±w}:
// X is the real FFT of the slice (the forward row pass already untangled
// the packed spectrum) and w one fp32 weight per tap (window / M for the
// analysis, dual window * 2/N for the synthesis adjoint), stored negated
// for a tap that reads the conjugate (weights are >= 0); taps outside the
// window carry w = 0.
// Synthesis epilogue (slot q RL + r = output t + T q + r OS): the tap stores
// (gr Re D, gi Im D) to its own slot of the half-spectrum buffer F, from the
// record {slot | mode << 30, gr} (plane P0 or P1 at the tap's bin, or an
// overflow slot for bins with more than two taps; mode says how gi follows
// from gr); taps with zero gain are skipped. No atomics: each slot has
// exactly one writer, so the result is bitwise reproducible, and the
// inverse column pass sums a bin's slots on load.
// Reference semantics: radix.cu:46-114, radix_impl.cuh:27-42,100-143.
#include "fcqt_bands.hpp"
#include "fcqt_abi_internal.hpp"

namespace fcqt {

template <int LAYOUT, bool WT, bool SM>
__global__ __launch_bounds__(kBandThreads) void k_route_bands(const float2* __restrict__ xs,
                                                              float* __restrict__ cre,
                                                              float* __restrict__ cim,
                                                              const int2* __restrict__ rec,
                                                              const int4* __restrict__ tasks, int batch,
                                                              long ncoef, const SliceMap sm,
                                                              const float2* __restrict__ tws,
                                                              int ntasks) {
    __shared__ float2 lds[kBandTaskLds];
    int task_id, b;
    decode_task<false, SM>(batch, ntasks, task_id, b);
    route_task<LAYOUT, WT>(task_id, b, xs, cre, cim, rec, tasks, ncoef, sm, tws, lds);
}

template <int LAYOUT, bool WT, bool SM>
__global__ __launch_bounds__(kBandThreads) void k_scatter_bands(const float* __restrict__ cre,
                                                                const float* __restrict__ cim,
                                                                float* __restrict__ f,
                                                                const int2* __restrict__ scat,
                                                                const int4* __restrict__ tasks, int batch,
                                                                long ncoef, const SliceMap sm,
                                                                const float2* __restrict__ tws,
                                                                int ntasks) {
    __shared__ float2 lds[kBandTaskLds];
    int task_id, b;
    decode_task<true, SM>(batch, ntasks, task_id, b);
    scatter_task<LAYOUT, WT>(task_id, b, cre, cim, f, scat, tasks, ncoef, sm, tws, lds);
}

// From this batch size on the band kernels write their outputs through the
// L2 (store_out<true>): measured faster from 4 slices up (B = 4: route 5.14
// against 5.39 us; B = 24: scatter 8.8 against 10.8 us) and slightly slower
// at 1 and 2 slices. Above kBandWriteThroughMaxBatch the round trip's working
// set no longer fits the memory-side cache and plain stores win again
// (slice-major round trips, write-through against plain in both band
// kernels: B = 80 87.1-87.7 against 88.1, B = 96 98.2-98.4 against 98.9-99.6,
// B = 112 130.2-130.4 against 120.6-120.9, B = 128 155.2-155.4 against 143.6,
// B = 192 244.3 against 223.2-223.5, B = 256 336.0 against 314.9-315.1 us).
// The values stored are the same.
constexpr int64_t kBandWriteThroughMinBatch = 4;
constexpr int64_t kBandWriteThroughMaxBatch = 104;

// From this batch size on the band grids run slice-major (band_place):
// measured round trips (stream launches) at B = 64 / 96 / 128 / 192 / 256:
// 74.0-74.3 / 99.1 / 154.5 / 243 / 337 us against 74.4-74.5 / 105.1 / 166.7 /
// 270.4 / 367.9 us task-major; task-major stays faster at B = 16 (35.5
// against 36.9 us). Same results either way.
constexpr int64_t kBandSliceMajorMinBatch = 64;

template <int LAYOUT>
static void launch_route(int64_t ntasks, int64_t batch, hipStream_t stream, const float2* xs, float* cre,
                         float* cim, const int2* rec, const int4* tasks, long ncoef, const SliceMap& sm,
                         const float2* tws) {
    const dim3 grid((unsigned)(ntasks * batch));
    static_assert(kBandWriteThroughMinBatch <= kBandSliceMajorMinBatch &&
                      kBandSliceMajorMinBatch <= kBandWriteThroughMaxBatch,
                  "batch ranges: plain task-major, write-through task-major, write-through slice-major, "
                  "plain slice-major");
    if (batch > kBandWriteThroughMaxBatch)
        hipLaunchKernelGGL((k_route_bands<LAYOUT, false, true>), grid, dim3(kBandThreads), 0, stream, xs, cre, cim,
                           rec, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
    else if (batch >= kBandSliceMajorMinBatch)
        hipLaunchKernelGGL((k_route_bands<LAYOUT, true, true>), grid, dim3(kBandThreads), 0, stream, xs, cre, cim,
                           rec, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
    else if (batch >= kBandWriteThroughMinBatch)
        hipLaunchKernelGGL((k_route_bands<LAYOUT, true, false>), grid, dim3(kBandThreads), 0, stream, xs, cre, cim,
                           rec, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
    else
        hipLaunchKernelGGL((k_route_bands<LAYOUT, false, false>), grid, dim3(kBandThreads), 0, stream, xs, cre, cim,
                           rec, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
}

template <int LAYOUT>
static void launch_scatter(int64_t ntasks, int64_t batch, hipStream_t stream, const float* cre, const float* cim,
                           float* f, const int2* scat, const int4* tasks, long ncoef, const SliceMap& sm,
                           const float2* tws) {
    const dim3 grid((unsigned)(ntasks * batch));
    if (batch > kBandWriteThroughMaxBatch)
        hipLaunchKernelGGL((k_scatter_bands<LAYOUT, false, true>), grid, dim3(kBandThreads), 0, stream, cre, cim, f,
                           scat, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
    else if (batch >= kBandSliceMajorMinBatch)
        hipLaunchKernelGGL((k_scatter_bands<LAYOUT, true, true>), grid, dim3(kBandThreads), 0, stream, cre, cim, f,
                           scat, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
    else if (batch >= kBandWriteThroughMinBatch)
        hipLaunchKernelGGL((k_scatter_bands<LAYOUT, true, false>), grid, dim3(kBandThreads), 0, stream, cre, cim, f,
                           scat, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
    else
        hipLaunchKernelGGL((k_scatter_bands<LAYOUT, false, false>), grid, dim3(kBandThreads), 0, stream, cre, cim, f,
                           scat, tasks, (int)batch, ncoef, sm, tws, (int)ntasks);
}

}  // namespace fcqt

// Checks shared by the band launchers: the record table, the task table,
// the coefficient span the descriptor declares against ncoef (a task table
// reaching past the coefficient row is refused), the layout and alignments.
int fcqt::check_band_args(const fcqt_tables* tab, const int32_t* rec, const float* cre, const float* cim,
                          int layout, int64_t batch) {
    if (!tab || !rec || !cre || batch < 1 || batch > kMaxBatch) return FCQT_EARG;
    if (!tab->tasks || !tab->tw_stage || tab->ntasks < 1 || tab->ncoef < 1) return FCQT_EARG;
    if (tab->coef_span < 1 || tab->coef_span > tab->ncoef) return FCQT_EARG;
    if ((int64_t)tab->ntasks * batch >= (int64_t)1 << 31) return FCQT_EARG;
    if (layout != FCQT_PLANAR && layout != FCQT_INTERLEAVED) return FCQT_EARG;
    if (layout == FCQT_PLANAR && !cim) return FCQT_EARG;
    if (!aligned(rec, 8) || !aligned(tab->tasks, 16) || !aligned(tab->tw_stage, 16)) return FCQT_EALIGN;
    if (layout == FCQT_PLANAR ? (!aligned(cre, 4) || !aligned(cim, 4)) : !aligned(cre, 8)) return FCQT_EALIGN;
    return FCQT_OK;
}

using namespace fcqt;

extern "C" int fcqt_route_bands(const fcqt_tables* tab, const int32_t* route, const float* xs,
                                float* coef_re, float* coef_im, int layout, int64_t batch,
                                hipStream_t stream) {
    if (int e = check_band_args(tab, route, coef_re, coef_im, layout, batch)) return e;
    if (!xs) return FCQT_EARG;
    if (!aligned(xs, 8)) return FCQT_EALIGN;
    const auto* xx = reinterpret_cast<const float2*>(xs);
    const auto* rr = reinterpret_cast<const int2*>(route);
    const auto* tt = reinterpret_cast<const int4*>(tab->tasks);
    const auto* ws = reinterpret_cast<const float2*>(tab->tw_stage);
    if (layout == FCQT_PLANAR)
        launch_route<FCQT_PLANAR>(tab->ntasks, batch, stream, xx, coef_re, coef_im, rr, tt, (long)tab->ncoef,
                                  SliceMap{nullptr, 1, 0}, ws);
    else
        launch_route<FCQT_INTERLEAVED>(tab->ntasks, batch, stream, xx, coef_re, coef_re, rr, tt, (long)tab->ncoef,
                                       SliceMap{nullptr, 1, 0}, ws);
    return launch_status();
}

extern "C" int fcqt_scatter_bands(const fcqt_tables* tab, const int32_t* scat, const float* coef_re,
                                  const float* coef_im, int layout, float* f, int64_t batch,
                                  hipStream_t stream) {
    if (int e = check_band_args(tab, scat, coef_re, coef_im, layout, batch)) return e;
    if (!f) return FCQT_EARG;
    if (!aligned(f, 16)) return FCQT_EALIGN;
    const auto* ss = reinterpret_cast<const int2*>(scat);
    const auto* tt = reinterpret_cast<const int4*>(tab->tasks);
    const auto* ws = reinterpret_cast<const float2*>(tab->tw_stage);
    if (layout == FCQT_PLANAR)
        launch_scatter<FCQT_PLANAR>(tab->ntasks, batch, stream, coef_re, coef_im, f, ss, tt, (long)tab->ncoef,
                                    SliceMap{nullptr, 1, 0}, ws);
    else
        launch_scatter<FCQT_INTERLEAVED>(tab->ntasks, batch, stream, coef_re, coef_re, f, ss, tt, (long)tab->ncoef,
                                         SliceMap{nullptr, 1, 0}, ws);
    return launch_status();
}

extern "C" int fcqt_route_bands_sliced(const fcqt_tables* tab, const int32_t* route, const int32_t* groups,
                                       const float* xs, float* coef, int64_t nsig, int64_t nslices,
                                       int64_t first, hipStream_t stream) {
    if (nsig < 1 || nslices < 1 || nsig > kMaxBatch || nslices > kMaxBatch) return FCQT_EARG;
    if (first < 0 || first > kMaxBatch) return FCQT_EARG;
    const int64_t batch = nsig * nslices;
    if (int e = check_band_args(tab, route, coef, coef, FCQT_INTERLEAVED, batch)) return e;
    if (!xs || !groups) return FCQT_EARG;
    if (!aligned(xs, 8) || !aligned(groups, 16)) return FCQT_EALIGN;
    launch_route<kSliced>(tab->ntasks, batch, stream, reinterpret_cast<const float2*>(xs), coef, coef,
                          reinterpret_cast<const int2*>(route), reinterpret_cast<const int4*>(tab->tasks),
                          (long)tab->ncoef,
                          SliceMap{reinterpret_cast<const int4*>(groups), (int)nslices, (int)first, (long)batch,
                                   (int)nslices, 0, 0},
                          reinterpret_cast<const float2*>(tab->tw_stage));
    return launch_status();
}

extern "C" int fcqt_sliced_analysis(const fcqt_tables* tab, const int32_t* route, const int32_t* groups,
                                    const float* sig, int64_t sig_len, const float* window, int64_t nsig,
                                    int64_t nslices, float* coef, float* xs, float* work, hipStream_t stream) {
    if (!sig || !window || !xs || !work || !groups || sig_len < 1) return FCQT_EARG;
    if (nsig < 1 || nslices < 1 || nsig > kMaxBatch || nslices > kMaxBatch || nsig * nslices > kMaxBatch)
        return FCQT_EARG;
    const int64_t batch = nsig * nslices;
    // the band half first, so an argument error launches nothing (the first
    // chunk's framing pass checks the rest before its launch)
    if (int e = check_band_args(tab, route, coef, coef, FCQT_INTERLEAVED, batch)) return e;
    if (!aligned(xs, 8) || !aligned(groups, 16)) return FCQT_EALIGN;
    // From kAnalysisChunkMinBatch slices on, chunks of about kAnalysisChunk
    // slices (all signals of a range of slices, or ranges of signals one
    // slice each), each framed, transformed and routed in turn so that its
    // W and X are still in the memory-side cache when read (as fcqt_analysis
    // does); a chunk's slices land in the whole call's block layout. The
    // chunks reuse the leading rows of xs and work. Every slice gives the
    // same bits however the call is cut.
    int64_t ns = nsig, cs = nslices;
    if (batch >= kAnalysisChunkMinBatch) {
        ns = nsig < kAnalysisChunk ? nsig : kAnalysisChunk;
        cs = kAnalysisChunk / ns;
        cs = cs < 1 ? 1 : (cs > nslices ? nslices : cs);
    }
    const auto* g4 = reinterpret_cast<const int4*>(groups);
    for (int64_t a = 0; a < nsig; a += ns) {
        const int64_t na = nsig - a < ns ? nsig - a : ns;
        for (int64_t c = 0; c < nslices; c += cs) {
            const int64_t nc = nslices - c < cs ? nslices - c : cs;
            if (int e = fcqt_slice_fft_fwd(tab, sig + a * sig_len, sig_len, window, na, nc, c, 0, xs, work, stream))
                return e;
            launch_route<kSliced>(tab->ntasks, na * nc, stream, reinterpret_cast<const float2*>(xs), coef, coef,
                                  reinterpret_cast<const int2*>(route), reinterpret_cast<const int4*>(tab->tasks),
                                  (long)tab->ncoef,
                                  SliceMap{g4, (int)nc, (int)c, (long)batch, (int)nslices, (int)c, (int)a},
                                  reinterpret_cast<const float2*>(tab->tw_stage));
            if (int e = launch_status()) return e;
        }
    }
    return FCQT_OK;
}

extern "C" int fcqt_scatter_bands_sliced(const fcqt_tables* tab, const int32_t* scat, const int32_t* groups,
                                         const float* coef, float* f, int64_t nsig, int64_t nslices,
                                         int64_t first, hipStream_t stream) {
    if (nsig < 1 || nslices < 1 || nsig > kMaxBatch || nslices > kMaxBatch) return FCQT_EARG;
    if (first < 0 || first > kMaxBatch) return FCQT_EARG;
    const int64_t batch = nsig * nslices;
    if (int e = check_band_args(tab, scat, coef, coef, FCQT_INTERLEAVED, batch)) return e;
    if (!f || !groups) return FCQT_EARG;
    if (!aligned(f, 16) || !aligned(groups, 16)) return FCQT_EALIGN;
    launch_scatter<kSliced>(tab->ntasks, batch, stream, coef, coef, f, reinterpret_cast<const int2*>(scat),
                            reinterpret_cast<const int4*>(tab->tasks), (long)tab->ncoef,
                            SliceMap{reinterpret_cast<const int4*>(groups), (int)nslices, (int)first, (long)batch,
                                     (int)nslices, 0, 0},
                            reinterpret_cast<const float2*>(tab->tw_stage));
    return launch_status();
}
