// Single-launch directions: each direction of the round trip as one
// cooperative launch of workgroups resident for the whole transform, with a
// grid-wide barrier where the separate launches had their boundaries.
//   analysis   column tiles -> barrier -> row tiles (untangle) -> barrier ->
//              band route tasks
//   synthesis  band scatter tasks -> barrier -> inverse column tiles
//              (slot sums, retangle) -> barrier -> inverse row tiles (unpack)
// Every phase runs the same tile and task bodies as the separate kernels
// (fcqt_passes.hpp, fcqt_bands.hpp), in 128-thread workgroups (column tiles
// of 16 columns, row tiles of 8 rows, inverse column tiles of 8 column
// pairs: shapes whose per-slice arithmetic equals the other shapes'), so the
// results equal the six-launch path bit for bit. Each workgroup walks its
// phase's tiles with a grid stride and a workgroup barrier between tiles
// (the next tile reuses the LDS).
// Reference semantics: fwd2_kernel / inv2_kernel, persist2.cu:140-222 (one
// cooperative launch per direction, grid syncs between phases); the
// reference's inverse also zeroes its atomic scatter target first, which
// this engine's slot scatter does not need.
#include <mutex>

#include <hip/hip_cooperative_groups.h>

#include "fcqt_passes.hpp"
#include "fcqt_bands.hpp"
#include "fcqt_abi_internal.hpp"

namespace fcqt {

namespace cgs = cooperative_groups;

constexpr int kPersistThreads = 128;
constexpr int kPColsPerTile = 16;      // forward column tiles: 8 x 16 threads
constexpr int kPRowsPerTile = 8;       // row tiles: 16 x 8 threads
constexpr int kPInvColsPerTile = 16;   // inverse column tiles (8 pairs): 8 x 16 threads
constexpr int kPColTiles = 256 / kPColsPerTile;
constexpr int kPRowTiles = 128 / kPRowsPerTile;
constexpr int kPInvColTiles = 256 / kPInvColsPerTile;
static_assert(8 * kPColsPerTile == kPersistThreads && 16 * kPRowsPerTile == kPersistThreads &&
                  8 * kPInvColsPerTile == kPersistThreads && kBandThreads == kPersistThreads,
              "every phase runs 128-thread workgroups");
constexpr int kPersistLds = cmax(cmax(col_lds<kPColsPerTile>(), col_lds<kPInvColsPerTile>()),
                                 cmax(row_lds<kPRowsPerTile>(), kBandTaskLds));

struct PersistArgs {
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
    long ncoef;
    int ntasks;
    int batch;
};

template <int LAYOUT>
__global__ __launch_bounds__(kPersistThreads) void k_persist_analysis(const PersistArgs p) {
    __shared__ float2 lds[kPersistLds];
    cgs::grid_group grid = cgs::this_grid();
    const SliceSrc whole{nullptr, nullptr, 1, 1, 0, 0};
    const int ncol = p.batch * kPColTiles;
    for (int t = blockIdx.x; t < ncol; t += gridDim.x) {
        col_fwd_tile<false, kPColsPerTile>(t / kPColTiles, t % kPColTiles, p.x, p.work, p.twp, p.tws, whole, lds);
        __syncthreads();
    }
    grid.sync();
    const int nrow = p.batch * kPRowTiles;
    for (int t = blockIdx.x; t < nrow; t += gridDim.x) {
        row_fwd_tile<kPRowsPerTile>(t / kPRowTiles, t % kPRowTiles, p.work, p.xs, p.twh, p.tws, lds);
        __syncthreads();
    }
    grid.sync();
    const int nband = p.ntasks * p.batch;
    for (int t = blockIdx.x; t < nband; t += gridDim.x) {
        const int task = t / p.batch;
        route_task<LAYOUT>(task, t - task * p.batch, p.xs, p.cre, p.cim, p.rec, p.tasks, p.batch, p.ncoef,
                           SliceMap{nullptr, 1, 0}, p.tws, lds);
        __syncthreads();
    }
}

template <int LAYOUT>
__global__ __launch_bounds__(kPersistThreads) void k_persist_synthesis(const PersistArgs p) {
    __shared__ float2 lds[kPersistLds];
    cgs::grid_group grid = cgs::this_grid();
    const int nband = p.ntasks * p.batch;
    for (int t = blockIdx.x; t < nband; t += gridDim.x) {
        const int task = t / p.batch;
        scatter_task<LAYOUT>(task, t - task * p.batch, p.cre, p.cim, p.f, p.rec, p.tasks, p.batch, p.ncoef,
                             SliceMap{nullptr, 1, 0}, p.tws, lds);
        __syncthreads();
    }
    grid.sync();
    const int ncol = p.batch * kPInvColTiles;
    const float2* f2 = reinterpret_cast<const float2*>(p.f);
    for (int t = blockIdx.x; t < ncol; t += gridDim.x) {
        col_inv_tile<kPInvColsPerTile>(t / kPInvColTiles, t % kPInvColTiles, f2, p.work, p.twp, p.twh, p.ovf,
                                       p.tws, lds);
        __syncthreads();
    }
    grid.sync();
    const int nrow = p.batch * kPRowTiles;
    for (int t = blockIdx.x; t < nrow; t += gridDim.x) {
        row_inv_tile<kPRowsPerTile>(t / kPRowTiles, t % kPRowTiles, p.work, p.y, p.tws, lds);
        __syncthreads();
    }
}

constexpr int kMaxDevices = 64;

// Workgroups of `kernel` that can be resident at once on the current device
// (cooperative launches must not exceed it), cached per device and kernel.
static int resident_capacity(const void* kernel, int slot, int* out) {
    static std::mutex mu;
    static int cap[kMaxDevices][4] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices)) return FCQT_EARG;
    std::lock_guard<std::mutex> lock(mu);
    if (e == hipSuccess && cap[dev][slot] == 0) {
        int per = 0, cus = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kPersistThreads, 0);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e == hipSuccess) cap[dev][slot] = per * cus;
    }
    if (e != hipSuccess) {
        std::snprintf(last_error_buf(), 256, "%s (%d)", hipGetErrorString(e), (int)e);
        return FCQT_ELAUNCH;
    }
    *out = cap[dev][slot];
    return *out > 0 ? FCQT_OK : FCQT_ELAUNCH;
}

static int cooperative_launch(const void* kernel, int slot, int tasks, const PersistArgs& p, hipStream_t stream) {
    int cap = 0;
    if (int e = resident_capacity(kernel, slot, &cap)) return e;
    const int grid = tasks < cap ? tasks : cap;
    void* args[] = {const_cast<PersistArgs*>(&p)};
    const hipError_t e = hipLaunchCooperativeKernel(kernel, dim3((unsigned)grid), dim3(kPersistThreads), args, 0,
                                                    stream);
    if (e != hipSuccess) {
        std::snprintf(last_error_buf(), 256, "%s (%d)", hipGetErrorString(e), (int)e);
        return FCQT_ELAUNCH;
    }
    return launch_status();
}

static int max3(int a, int b, int c) { return a > b ? (a > c ? a : c) : (b > c ? b : c); }

}  // namespace fcqt

using namespace fcqt;

extern "C" int fcqt_persist_analysis(const fcqt_tables* tab, const int32_t* route, const float* x, float* coef_re,
                                     float* coef_im, int layout, float* xs, float* work, int64_t batch,
                                     hipStream_t stream) {
    if (!route || !x || !xs || !work) return FCQT_EARG;
    if (int e = check_band_args(tab, route, coef_re, coef_im, layout, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    if (batch * (int64_t)tab->ntasks >= ((int64_t)1 << 31) / 2) return FCQT_EARG;
    if (!aligned(x, 8) || !aligned(xs, 8) || !aligned(work, 8) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_half, 8))
        return FCQT_EALIGN;
    PersistArgs p{};
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
    p.ncoef = (long)tab->ncoef;
    p.ntasks = tab->ntasks;
    p.batch = (int)batch;
    const int tasks = max3((int)batch * kPColTiles, (int)batch * kPRowTiles, (int)batch * tab->ntasks);
    if (layout == FCQT_PLANAR)
        return cooperative_launch(reinterpret_cast<const void*>(&k_persist_analysis<FCQT_PLANAR>), 0, tasks, p,
                                  stream);
    return cooperative_launch(reinterpret_cast<const void*>(&k_persist_analysis<FCQT_INTERLEAVED>), 1, tasks, p,
                              stream);
}

extern "C" int fcqt_persist_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* ovf,
                                      const float* coef_re, const float* coef_im, int layout, float* f, float* work,
                                      float* y, int64_t batch, hipStream_t stream) {
    if (!scat || !ovf || !f || !work || !y) return FCQT_EARG;
    if (int e = check_band_args(tab, scat, coef_re, coef_im, layout, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    if (batch * (int64_t)tab->ntasks >= ((int64_t)1 << 31) / 2) return FCQT_EARG;
    if (!aligned(f, 16) || !aligned(y, 8) || !aligned(work, 8) || !aligned(ovf, 4) || !aligned(tab->tw_pass, 8) ||
        !aligned(tab->tw_half, 8))
        return FCQT_EALIGN;
    PersistArgs p{};
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
    p.ncoef = (long)tab->ncoef;
    p.ntasks = tab->ntasks;
    p.batch = (int)batch;
    const int tasks = max3((int)batch * tab->ntasks, (int)batch * kPInvColTiles, (int)batch * kPRowTiles);
    if (layout == FCQT_PLANAR)
        return cooperative_launch(reinterpret_cast<const void*>(&k_persist_synthesis<FCQT_PLANAR>), 2, tasks, p,
                                  stream);
    return cooperative_launch(reinterpret_cast<const void*>(&k_persist_synthesis<FCQT_INTERLEAVED>), 3, tasks, p,
                              stream);
}
