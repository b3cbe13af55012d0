// Single-launch directions: each direction of the round trip as one
// ordinary launch whose stages wait for each other slice by slice.
//   analysis   stage 1: column tiles    stage 2: row tiles (untangle)
//              stage 3: band route tasks
//   synthesis  stage 1: band scatter tasks    stage 2: inverse column tiles
//              (slot sums, retangle)          stage 3: inverse row tiles (unpack)
// Every stage runs the same tile and task bodies as the separate kernels
// (fcqt_passes.hpp, fcqt_bands.hpp) in 128-thread workgroups (column tiles of
// 16 columns, row tiles of 8 rows, inverse column tiles of 8 column pairs:
// shapes whose per-slice arithmetic equals the other shapes'), so the results
// equal the six-launch path bit for bit.
//
// Placement and waits. The hardware hands workgroup i to XCD i mod 8 (on
// every partitioning of the chip, workgroups with equal blockIdx mod 8 share
// an XCD and so an L2), and each XCD starts its workgroups in blockIdx order.
// The grid gives all of a slice's workgroups one residue mod 8 and lays out
// each XCD's share as [stage 1 of its slices][stage 2][stage 3]. A stage-2 or
// stage-3 workgroup waits (one lane polls, with sleeps) until its slice's
// previous stage has counted in. The workgroups it waits for started before
// it on the same XCD and wait only on earlier stages, so every wait ends.
// Producer and consumer share an L2, so a wait needs no L2 write-back: the
// producer's stores are in the L2 when its counter moves (each lane waits for
// its stores before the workgroup barrier), and the consumer drops its L1
// before reading. Each stage-1 workgroup marks its XCD in the slice's record
// and each waiting workgroup compares that mark with its own XCD; a mismatch,
// or a wait that outlasts its bound (about two seconds), sets the error word,
// so a broken placement assumption gives an error, never a hang or a silent
// stale read. The last workgroup of a slice's last stage returns the slice's
// record to zero, so the counters are ready for the next call (and for graph
// replays) without a memset.
//
// Measured on MI355X (graphs of 20 calls), against the three launches of the
// same direction: analysis 13.1 / 18.8 / 41.3 / 58.0 us against 11.5 / 17.0 /
// 37.2 / 59.7 us at B = 1 / 16 / 64 / 128; synthesis 15.4 / 28.6 / 50.0 / 72.7
// us against 13.5 / 18.6 / 39.0 / 80.2 us. The cooperative form with two
// grid-wide barriers per direction took 231 / 250 us per direction at B = 64.
// Reference semantics: fwd2_kernel / inv2_kernel, persist2.cu:140-222 (one
// launch per direction; the reference's inverse also zeroes its atomic
// scatter target first, which this engine's slot scatter does not need).
#include "fcqt_passes.hpp"
#include "fcqt_bands.hpp"
#include "fcqt_abi_internal.hpp"

namespace fcqt {

constexpr int kFlowThreads = 128;
constexpr int kFColsPerTile = 16;      // forward column tiles: 8 x 16 threads
constexpr int kFRowsPerTile = 8;       // row tiles: 16 x 8 threads
constexpr int kFInvColsPerTile = 16;   // inverse column tiles (8 pairs): 8 x 16 threads
constexpr int kFColTiles = 256 / kFColsPerTile;
constexpr int kFRowTiles = 128 / kFRowsPerTile;
constexpr int kFInvColTiles = 256 / kFInvColsPerTile;
static_assert(8 * kFColsPerTile == kFlowThreads && 16 * kFRowsPerTile == kFlowThreads &&
                  8 * kFInvColsPerTile == kFlowThreads && kBandThreads == kFlowThreads,
              "every stage runs 128-thread workgroups");
constexpr int kFlowLds = cmax(cmax(col_lds<kFColsPerTile>(), col_lds<kFInvColsPerTile>()),
                              cmax(row_lds<kFRowsPerTile>(), kBandTaskLds));

// A slice's record: FCQT_SYNC_PER_SLICE words; the three stage counters and
// the XCD mask each sit on their own 64-byte line.
constexpr int kSyncStage1 = 0, kSyncStage2 = 16, kSyncStage3 = 32, kSyncXcd = 48;
static_assert(FCQT_SYNC_PER_SLICE == 64, "slice record layout");
constexpr int kWaitPolls = 1 << 22;    // polls of ~1000 cycles of sleep each: about two seconds
constexpr int kXcds = 8;

__device__ __forceinline__ unsigned xcc_id() {
    return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11)) & 15u;   // HW_REG_XCC_ID
}

__device__ __forceinline__ unsigned sync_load(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct FlowArgs {
    const float2* twp;        // pass twiddles
    const float2* twh;        // untangle / retangle twiddles
    const float2* tws;        // stage twiddles
    const int4* tasks;
    const int2* rec;          // route or scatter records
    const int* ovf;           // fold lists (synthesis)
    const float2* x;          // analysis input (float pairs)
    float2* xs;               // spectrum X (analysis)
    float* f;                 // slot buffer F (synthesis)
    float2* work;             // four-step intermediate
    float2* y;                // synthesis output (float pairs)
    float* cre;
    float* cim;
    unsigned* sync;
    long ncoef;
    int ntasks;
    int batch;
};

// This workgroup's stage (1, 2 or 3; 0 past its XCD's share), slice b and
// index t within the stage, for stages of n1, n2, n3 workgroups per slice.
__device__ __forceinline__ int flow_place(int n1, int n2, int n3, int batch, int& b, int& t) {
    const int xcd = (int)(blockIdx.x % kXcds), i = (int)(blockIdx.x / kXcds);
    const int nsl = batch > xcd ? (batch - xcd + kXcds - 1) / kXcds : 0;    // slices xcd, xcd + 8, ...
    int stage, k;
    if (i < nsl * n1) {
        stage = 1, k = i;
    } else if (i < nsl * (n1 + n2)) {
        stage = 2, k = i - nsl * n1;
    } else if (i < nsl * (n1 + n2 + n3)) {
        stage = 3, k = i - nsl * (n1 + n2);
    } else {
        return 0;
    }
    const int n = stage == 1 ? n1 : (stage == 2 ? n2 : n3);
    const int j = k / n;
    t = k - j * n;
    b = xcd + kXcds * j;
    return stage;
}

// After a stage-1 or stage-2 body: this workgroup's stores are in the L2,
// then the slice's counter moves (stage 1 also marks its XCD).
__device__ __forceinline__ void flow_signal(unsigned* rec, int counter, bool mark_xcd) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        if (mark_xcd)
            __hip_atomic_fetch_or(rec + kSyncXcd, 1u << xcc_id(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(rec + counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Before a stage-2 or stage-3 body: wait until `target` workgroups of the
// slice's previous stage have counted in, check that they ran on this XCD,
// then drop this CU's L1 lines (the data comes from the shared L2).
__device__ __forceinline__ void flow_wait(unsigned* rec, int counter, unsigned target, unsigned* err) {
    if (threadIdx.x == 0) {
        int n = 0;
        while (sync_load(rec + counter) < target) {
            __builtin_amdgcn_s_sleep(16);
            if (++n > kWaitPolls) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        if (sync_load(rec + kSyncXcd) != (1u << xcc_id()))
            __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    asm volatile("buffer_inv sc0" ::: "memory");
}

// After a stage-3 body: the slice's last workgroup clears its record.
__device__ __forceinline__ void flow_finish(unsigned* rec, unsigned n3) {
    __syncthreads();
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(rec + kSyncStage3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n3 - 1) {
        __hip_atomic_store(rec + kSyncStage1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(rec + kSyncStage2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(rec + kSyncXcd, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(rec + kSyncStage3, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int LAYOUT>
__global__ __launch_bounds__(kFlowThreads) void k_flow_analysis(const FlowArgs p) {
    __shared__ float2 lds[kFlowLds];
    int b = 0, t = 0;
    const int stage = flow_place(kFColTiles, kFRowTiles, p.ntasks, p.batch, b, t);
    if (stage == 0) return;
    unsigned* rec = p.sync + (long)b * FCQT_SYNC_PER_SLICE;
    unsigned* err = p.sync + (long)p.batch * FCQT_SYNC_PER_SLICE;
    if (stage == 1) {
        col_fwd_tile<false, kFColsPerTile>(b, t, p.x, p.work, p.twp, p.tws, SliceSrc{nullptr, nullptr, 1, 1, 0, 0, 0, nullptr, 1, 1, 1},
                                           lds);
        flow_signal(rec, kSyncStage1, true);
    } else if (stage == 2) {
        flow_wait(rec, kSyncStage1, kFColTiles, err);
        row_fwd_tile<kFRowsPerTile>(b, t, p.work, p.xs, p.twh, p.tws, lds);
        flow_signal(rec, kSyncStage2, false);
    } else {
        flow_wait(rec, kSyncStage2, kFRowTiles, err);
        route_task<LAYOUT, true>(t, b, p.xs, p.cre, p.cim, p.rec, p.tasks, p.ncoef, SliceMap{nullptr, 1, 0},
                                 p.tws, lds);
        flow_finish(rec, (unsigned)p.ntasks);
    }
}

template <int LAYOUT>
__global__ __launch_bounds__(kFlowThreads) void k_flow_synthesis(const FlowArgs p) {
    __shared__ float2 lds[kFlowLds];
    int b = 0, t = 0;
    const int stage = flow_place(p.ntasks, kFInvColTiles, kFRowTiles, p.batch, b, t);
    if (stage == 0) return;
    unsigned* rec = p.sync + (long)b * FCQT_SYNC_PER_SLICE;
    unsigned* err = p.sync + (long)p.batch * FCQT_SYNC_PER_SLICE;
    if (stage == 1) {
        scatter_task<LAYOUT, false>(t, b, p.cre, p.cim, p.f, p.rec, p.tasks, p.ncoef,
                                    SliceMap{nullptr, 1, 0}, p.tws, lds);
        flow_signal(rec, kSyncStage1, true);
    } else if (stage == 2) {
        flow_wait(rec, kSyncStage1, (unsigned)p.ntasks, err);
        col_inv_tile<kFInvColsPerTile, false>(b, t, reinterpret_cast<const float2*>(p.f), p.work, p.twp, p.twh, p.ovf,
                                       p.tws, lds);
        flow_signal(rec, kSyncStage2, false);
    } else {
        flow_wait(rec, kSyncStage2, kFInvColTiles, err);
        row_inv_tile<kFRowsPerTile, false>(b, t, p.work, p.y, p.tws, lds);
        flow_finish(rec, kFRowTiles);
    }
}

// Workgroups of a flow grid: eight residues, each with the stages of the
// largest share of slices.
static dim3 flow_grid(int64_t batch, int per_slice) {
    return dim3((unsigned)(kXcds * ((batch + kXcds - 1) / kXcds) * per_slice));
}

static int check_flow_args(const fcqt_tables* tab, const uint32_t* sync, int64_t batch) {
    if (!sync) return FCQT_EARG;
    if (!aligned(sync, 16)) return FCQT_EALIGN;
    // grid size: 8 ceil(batch / 8) (32 + ntasks) workgroups
    if (((batch + kXcds - 1) / kXcds) * kXcds * (32 + (int64_t)tab->ntasks) >= ((int64_t)1 << 31)) return FCQT_EARG;
    return FCQT_OK;
}

}  // namespace fcqt

using namespace fcqt;

extern "C" int fcqt_persist_analysis(const fcqt_tables* tab, const int32_t* route, const float* x, float* coef_re,
                                     float* coef_im, int layout, float* xs, float* work, uint32_t* sync,
                                     int64_t batch, hipStream_t stream) {
    if (!route || !x || !xs || !work) return FCQT_EARG;
    if (int e = check_band_args(tab, route, coef_re, coef_im, layout, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    if (int e = check_flow_args(tab, sync, batch)) return e;
    if (!aligned(x, 8) || !aligned(xs, 8) || !aligned(work, 8) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_half, 8))
        return FCQT_EALIGN;
    FlowArgs p{};
    p.twp = reinterpret_cast<const float2*>(tab->tw_pass);
    p.twh = reinterpret_cast<const float2*>(tab->tw_half);
    p.tws = reinterpret_cast<const float2*>(tab->tw_stage);
    p.tasks = reinterpret_cast<const int4*>(tab->tasks);
    p.rec = reinterpret_cast<const int2*>(route);
    p.x = reinterpret_cast<const float2*>(x);
    p.xs = reinterpret_cast<float2*>(xs);
    p.work = reinterpret_cast<float2*>(work);
    p.cre = coef_re;
    p.cim = layout == FCQT_PLANAR ? coef_im : coef_re;
    p.sync = sync;
    p.ncoef = (long)tab->ncoef;
    p.ntasks = tab->ntasks;
    p.batch = (int)batch;
    const dim3 grid = flow_grid(batch, kFColTiles + kFRowTiles + tab->ntasks);
    if (layout == FCQT_PLANAR)
        hipLaunchKernelGGL(k_flow_analysis<FCQT_PLANAR>, grid, dim3(kFlowThreads), 0, stream, p);
    else
        hipLaunchKernelGGL(k_flow_analysis<FCQT_INTERLEAVED>, grid, dim3(kFlowThreads), 0, stream, p);
    return launch_status();
}

extern "C" int fcqt_persist_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* ovf,
                                      const float* coef_re, const float* coef_im, int layout, float* f, float* work,
                                      float* y, uint32_t* sync, int64_t batch, hipStream_t stream) {
    if (!scat || !ovf || !f || !work || !y) return FCQT_EARG;
    if (int e = check_band_args(tab, scat, coef_re, coef_im, layout, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    if (int e = check_flow_args(tab, sync, batch)) return e;
    if (!aligned(f, 16) || !aligned(y, 8) || !aligned(work, 8) || !aligned(ovf, 4) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_half, 8))
        return FCQT_EALIGN;
    FlowArgs p{};
    p.twp = reinterpret_cast<const float2*>(tab->tw_pass);
    p.twh = reinterpret_cast<const float2*>(tab->tw_half);
    p.tws = reinterpret_cast<const float2*>(tab->tw_stage);
    p.tasks = reinterpret_cast<const int4*>(tab->tasks);
    p.rec = reinterpret_cast<const int2*>(scat);
    p.ovf = ovf;
    p.f = f;
    p.work = reinterpret_cast<float2*>(work);
    p.y = reinterpret_cast<float2*>(y);
    p.cre = const_cast<float*>(coef_re);
    p.cim = const_cast<float*>(layout == FCQT_PLANAR ? coef_im : coef_re);
    p.sync = sync;
    p.ncoef = (long)tab->ncoef;
    p.ntasks = tab->ntasks;
    p.batch = (int)batch;
    const dim3 grid = flow_grid(batch, tab->ntasks + kFInvColTiles + kFRowTiles);
    if (layout == FCQT_PLANAR)
        hipLaunchKernelGGL(k_flow_synthesis<FCQT_PLANAR>, grid, dim3(kFlowThreads), 0, stream, p);
    else
        hipLaunchKernelGGL(k_flow_synthesis<FCQT_INTERLEAVED>, grid, dim3(kFlowThreads), 0, stream, p);
    return launch_status();
}
