// Band task bodies (device code) of the route engine (windowed gathers +
// band inverse DFTs) and the scatter engine (band DFTs + gain + slot
// scatter), shared by the band kernels (bands.hip) and the single-launch
// kernels (persist.hip). The engines are described in bands.hip.
#pragma once

#include "fcqt_fft.hpp"
#include "../../include/flashcqt.h"

namespace fcqt {

constexpr int kBandThreads = 128;

// Band units of length M <= FCQT_XLANE_MAX_M exchange between their first
// two stages across lanes (fft_unit_xl) instead of through LDS. 0 in the
// library (the LDS exchange measured faster); the variant library
// libflashcqt_xlane.so is built with 256.
#ifndef FCQT_XLANE_MAX_M
#define FCQT_XLANE_MAX_M 0
#endif

// The unit transform of the band kernels.
template <int M, int SIGN>
__device__ __forceinline__ void band_fft(float2* v, float2* s, int t, const float2* tl, const Tw3<M>& w3) {
    if constexpr (M <= FCQT_XLANE_MAX_M) fft_unit_xl<M, SIGN>(v, t, tl);
    else fft_unit<M, SIGN>(v, s, t, tl, w3);
}
constexpr int kBandPoints = 16 * kBandThreads;  // complex values (and records) per task

constexpr int band_lds(int M) { return (kBandPoints / M) * (M + M / 16 + 1); }
constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int kBandLds = cmax(cmax(cmax(band_lds(32), band_lds(64)), cmax(band_lds(128), band_lds(256))),
                              cmax(cmax(band_lds(512), band_lds(1024)), band_lds(2048)));

// Coefficient addressing. FCQT_PLANAR / FCQT_INTERLEAVED: the engine layout
// [batch][ncoef]. kSliced: the SlicedCQT block layout, interleaved complex.
// The call's batch = nsig * S slices (slice s of signal sig is batch row
// sig * S + s) land in a block layout of NSIG signals x S_out slices
// (rows = NSIG S_out) as its signal sig0 + sig, slice s0 + s: the
// coefficients of group g (first coefficient off_g, bins_g bands of length
// M) form the block [NSIG][bins_g][S_out * M] at rows * off_g, band i's
// slice s at (((sig0 + sig) bins_g + i) S_out + s0 + s) M, and in octave
// groups (roll flag) output m of the band transform sits at (m + M/4) mod M
// in even slices and (m - M/4) mod M in odd slices (the SlicedCQT quarter
// roll; side groups are [NSIG][S_out][1][M] blocks, unrolled). Parity is
// that of the slice's index in its signal, first + s, where first is the
// index of the call's first slice (0 for a whole signal; the chunk's first
// slice; the slice count so far when streaming, with S_out = 1, s0 = 0).
constexpr int kSliced = 2;

struct SliceMap {
    const int4* __restrict__ groups;   // per task {off_g, bins_g, roll, 0}
    int S;                             // slices per signal in this call
    int first;                         // index in the signal of the call's slice 0
    long rows;                         // rows of the block layout (NSIG * S_out)
    int S_out;                         // slices per signal in the block layout
    int s0;                            // layout slice of the call's slice 0
    int sig0;                          // layout signal of the call's signal 0
};

template <int M, int LAYOUT>
__device__ __forceinline__ void unit_coef(const int4 task, const int task_id, const int b, const int u,
                                          const long ncoef, const SliceMap& sm, long& base,
                                          int& shift) {
    if constexpr (LAYOUT == kSliced) {
        const int4 g = sm.groups[task_id];
        const int sig = b / sm.S;
        const int s = b - sig * sm.S;
        const int i = (task.y - g.x) / M + u;
        base = sm.rows * g.x + ((long)((sm.sig0 + sig) * g.y + i) * sm.S_out + sm.s0 + s) * M;
        shift = g.z ? (((sm.first + s) & 1) ? M - M / 4 : M / 4) : 0;
    } else {
        base = (long)b * ncoef + task.y + u * M;
        shift = 0;
    }
}

template <int LAYOUT>
__device__ __forceinline__ float2 load_coef(const float* __restrict__ cre, const float* __restrict__ cim, int i) {
    if constexpr (LAYOUT == FCQT_PLANAR) return make_float2(cre[i], cim[i]);
    else return reinterpret_cast<const float2*>(cre)[i];
}

template <int LAYOUT, bool WT>
__device__ __forceinline__ void store_coef(float* __restrict__ cre, float* __restrict__ cim, int i, float2 v) {
    if constexpr (LAYOUT == FCQT_PLANAR) {
        store_out<WT>(cre + i, v.x);
        store_out<WT>(cim + i, v.y);
    } else {
        store_out<WT>(reinterpret_cast<float2*>(cre) + i, v);
    }
}

// This thread's 16 records of its task (kernel order).
__device__ __forceinline__ void load_records(int2* rv, const int2* __restrict__ rec, int task, int tid) {
    const int2* rr = rec + (long)task * kBandPoints + tid;
#pragma unroll
    for (int s = 0; s < 16; ++s) rv[s] = rr[s * kBandThreads];
}

// Route + band inverse DFTs of one task; stores the coefficients of the
// task's bands (units past the band count compute padding that is never
// stored). The twiddle loads issue before the gathers, so their latency
// hides under the record and gather round trips.
template <int M, int LAYOUT, bool WT>
__device__ __forceinline__ void route_band(const int4 task, const int task_id, const int b,
                                           const int2* rv, const float2* __restrict__ xb,
                                           float* __restrict__ cre, float* __restrict__ cim,
                                           const long ncoef, const SliceMap sm,
                                           const float2* __restrict__ tws, float2* lds, float2* tw2,
                                           const int tid) {
    using P = Plan<M>;
    const int u = tid / P::T;
    const int t = tid - u * P::T;
    Tw2Copy<M, kBandThreads> c2;
    fetch_tw2<M, kBandThreads>(c2, tws, tid);
    Tw3<M> w3;
    load_tw3<M>(w3, tws, t);
    // v = w X[k], conjugated for taps past Nyquist: the record's weight
    // carries the conjugation in its sign bit (weights are >= 0), so
    // v = (|w| Re X, w Im X)
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float2 x = xb[min((unsigned)rv[r].x, (unsigned)kL)];
        const float w = __int_as_float(rv[r].y);
        v[r] = make_float2(fabsf(w) * x.x, w * x.y);
    }
    put_tw2<M, kBandThreads>(tw2, c2, tid);
    band_fft<M, +1>(v, lds + u * P::US, t, tw2, w3);
    if (u < task.z) {
        long ob;
        int shift;
        unit_coef<M, LAYOUT>(task, task_id, b, u, ncoef, sm, ob, shift);   // uniform per unit
        float* orow = cre + (LAYOUT == FCQT_PLANAR ? ob : 2 * ob);
        float* oim = cim + (LAYOUT == FCQT_PLANAR ? ob : 0);
#pragma unroll
        for (int q = 0; q < P::QL; ++q) {
#pragma unroll
            for (int r = 0; r < P::RL; ++r)
                store_coef<LAYOUT, WT>(orow, oim, (t + P::T * q + r * P::OS + shift) & (M - 1), v[q * P::RL + r]);
        }
    }
}

template <int M, int LAYOUT, bool WT>
__device__ __forceinline__ void scatter_band(const int4 task, const int task_id, const int b,
                                             const int2* __restrict__ scat, const float* __restrict__ cre,
                                             const float* __restrict__ cim, float* __restrict__ f,
                                             const long ncoef, const SliceMap sm,
                                             const float2* __restrict__ tws, float2* lds, float2* tw2,
                                             const int tid) {
    using P = Plan<M>;
    const int u = tid / P::T;
    const int t = tid - u * P::T;
    const bool active = u < task.z;
    // coefficients first, then the twiddles, then the records (needed only
    // after the transform)
    long ib;
    int shift;
    unit_coef<M, LAYOUT>(task, task_id, b, active ? u : 0, ncoef, sm, ib, shift);
    const float* cr = cre + (LAYOUT == FCQT_PLANAR ? ib : 2 * ib);
    const float* ci = cim + (LAYOUT == FCQT_PLANAR ? ib : 0);
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = load_coef<LAYOUT>(cr, ci, (t + P::T * r + shift) & (M - 1));
    Tw2Copy<M, kBandThreads> c2;
    fetch_tw2<M, kBandThreads>(c2, tws, tid);
    Tw3<M> w3;
    load_tw3<M>(w3, tws, t);
    int2 rv[16];
    load_records(rv, scat, task_id, tid);
    put_tw2<M, kBandThreads>(tw2, c2, tid);
    band_fft<M, -1>(v, lds + u * P::US, t, tw2, w3);
    if (active) {
        float2* fb = reinterpret_cast<float2*>(f) + (long)b * kFRow;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float gr = __int_as_float(rv[i].y);
            if (gr != 0.0f) {
                const unsigned mode = (unsigned)rv[i].x >> 30;
                const unsigned slot = min((unsigned)rv[i].x & 0x3fffffffu, (unsigned)(kFRow - 1));
                const float gi = mode == 0 ? gr : (mode == 1 ? -gr : 0.0f);
                store_out<WT>(fb + slot, make_float2(gr * v[i].x, gi * v[i].y));
            }
        }
    }
}

// REVERSE: walk each XCD's range from its end (the scatter follows the
// route kernel on the same (task, slice) grid, so it starts with the
// coefficients the route kernel wrote last; measured 0.2-0.9 us per round
// trip at B = 16-120, same results). SLICE_MAJOR: the order band_place
// describes (the launchers choose it by batch size); ntasks is the task
// count of the grid.
template <bool REVERSE, bool SLICE_MAJOR>
__device__ __forceinline__ void decode_task(int batch, int ntasks, int& task, int& b) {
    const int lg = REVERSE ? xcd_remap_reverse((int)blockIdx.x, (int)gridDim.x)
                           : xcd_remap((int)blockIdx.x, (int)gridDim.x);
    band_place(lg, ntasks, batch, SLICE_MAJOR, task, b);
}

// LDS of a band task (float2 elements): the units, then the twiddle block.
constexpr int kBandTaskLds = kBandLds + tw2_len<2048>();

// One band task (task_id, slice b) of the route engine in caller-provided
// LDS; the band kernels and the single-launch analysis (persist.hip) run it.
// WT: write the coefficients through the L2 (store_out), for batches whose
// coefficient output is large.
template <int LAYOUT, bool WT = false>
__device__ __forceinline__ void route_task(const int task_id, const int b, const float2* __restrict__ xs,
                                           float* __restrict__ cre, float* __restrict__ cim,
                                           const int2* __restrict__ rec, const int4* __restrict__ tasks,
                                           const long ncoef, const SliceMap& sm,
                                           const float2* __restrict__ tws, float2* lds,
                                           const int tid = threadIdx.x) {
    float2* tw2 = lds + kBandLds;
    // the records issue first (they need the task index only); the task
    // record then selects the band length, and the gathers follow inside
    int2 rv[16];
    load_records(rv, rec, task_id, tid);
    const float2* xb = xs + (long)b * kXStride;
    const int4 td = tasks[task_id];
    if (td.y < 0 || (long)td.y + (long)td.z * td.x > ncoef) return;   // task outside the coefficient row
#define FCQT_ROUTE(M_) route_band<M_, LAYOUT, WT>(td, task_id, b, rv, xb, cre, cim, ncoef, sm, tws, lds, tw2, tid)
    switch (td.x) {
        case 32: FCQT_ROUTE(32); break;
        case 64: FCQT_ROUTE(64); break;
        case 128: FCQT_ROUTE(128); break;
        case 256: FCQT_ROUTE(256); break;
        case 512: FCQT_ROUTE(512); break;
        case 1024: FCQT_ROUTE(1024); break;
        case 2048: FCQT_ROUTE(2048); break;
        default: break;
    }
#undef FCQT_ROUTE
}


// One band task of the scatter engine in caller-provided LDS (WT: slot
// stores through the L2, as in route_task).
template <int LAYOUT, bool WT = false>
__device__ __forceinline__ void scatter_task(const int task_id, const int b, const float* __restrict__ cre,
                                             const float* __restrict__ cim, float* __restrict__ f,
                                             const int2* __restrict__ scat, const int4* __restrict__ tasks,
                                             const long ncoef, const SliceMap& sm,
                                             const float2* __restrict__ tws, float2* lds,
                                             const int tid = threadIdx.x) {
    float2* tw2 = lds + kBandLds;
    const int4 td = tasks[task_id];
    if (td.y < 0 || (long)td.y + (long)td.z * td.x > ncoef) return;   // task outside the coefficient row
#define FCQT_SCATTER(M_) scatter_band<M_, LAYOUT, WT>(td, task_id, b, scat, cre, cim, f, ncoef, sm, tws, lds, tw2, tid)
    switch (td.x) {
        case 32: FCQT_SCATTER(32); break;
        case 64: FCQT_SCATTER(64); break;
        case 128: FCQT_SCATTER(128); break;
        case 256: FCQT_SCATTER(256); break;
        case 512: FCQT_SCATTER(512); break;
        case 1024: FCQT_SCATTER(1024); break;
        case 2048: FCQT_SCATTER(2048); break;
        default: break;
    }
#undef FCQT_SCATTER
}

}  // namespace fcqt
