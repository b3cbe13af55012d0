// Single-launch directions: each direction of the round trip as one launch
// of persistent workgroups that take the direction's tasks from per-XCD
// queues.
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
// Queues and order. Queue x holds the slices x, x + 8, x + 16, ... and is
// served only by workgroups that run on XCD x, read from the hardware
// (HW_REG_XCC_ID), so the producer and the consumer of every intermediate
// (W, X; F, W) share one L2 whatever the dispatcher's placement. A
// workgroup takes the next position of its XCD's queue with one atomic
// add; fcqt_flow.hpp maps positions to tasks in a slice-interleaved order
// with lags d1 (stage 2 after stage 1) and d2 (stage 3 after stage 1), so
// a task's dependencies were taken earlier, by running workgroups: every
// wait ends, with any number of workgroups resident. A stage-2 or stage-3
// task waits (one lane polls its slice's counter, with sleeps) for its
// slice's previous stage; the producer's stores reach the shared L2 before
// its counter moves (each lane waits for its stores before the workgroup
// barrier), and the consumer drops its L1 before reading.
//
// Failures become an error word, never a hang or a silent result: a wait
// bounded by the chip's 100 MHz clock (two seconds) sets bit 1 and every
// other wait then stops; the last workgroup to leave sets bit 4 if a queue
// with tasks was never served (no workgroup ran on that XCD). Only when the
// word is zero does that last workgroup return the counters to zero, so a
// stale count can never satisfy a later call's wait; after a nonzero word
// the caller synchronises and zero-fills the whole sync buffer.
//
// Reference semantics: fwd2_kernel / inv2_kernel, persist2.cu:140-222 (one
// launch per direction; the reference's inverse also zeroes its atomic
// scatter target first, which this engine's slot scatter does not need).
#include "fcqt_passes.hpp"
#include "fcqt_bands.hpp"
#include "fcqt_flow.hpp"
#include "fcqt_abi_internal.hpp"

#include <algorithm>

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

// sync buffer: per slice FCQT_SYNC_PER_SLICE words (stage-1 and stage-2
// done counts, each on its own 128-byte line), then the head block of
// FCQT_SYNC_HEAD_WORDS: error word, exit count, one claim counter per queue
// (each on its own 128-byte line).
constexpr int kSyncStage1 = 0, kSyncStage2 = 32;
constexpr int kHeadError = 0, kHeadExit = 32, kHeadClaim = 64;
static_assert(FCQT_SYNC_PER_SLICE == 64 && FCQT_SYNC_HEAD_WORDS == kHeadClaim + 32 * kFlowQueues,
              "sync buffer layout");
constexpr int64_t kWaitTicksDefault = 200000000;   // two seconds of the 100 MHz clock
constexpr unsigned kErrTimeout = 1u, kErrUnserved = 4u;

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
    FlowOrder order;
    uint64_t wait_ticks;      // bound of a stage wait (100 MHz ticks)
#ifdef FCQT_FLOW_TRACE
    unsigned long long* trace;   // fcqt_persist_trace buffer, or null
#endif
};

// Stage trace of the trace build (libflashcqt_flowtrace.so, built with
// FCQT_FLOW_TRACE): lane 0 of each workgroup stamps the chip's 100 MHz
// clock into FCQT_TRACE_TASKS records of FCQT_TRACE_FIELDS uint64 per
// workgroup (blockIdx order). Record i < FCQT_TRACE_TASKS - 1 is the
// workgroup's task i: {stage | slice << 8 | tile << 40, before its claim or
// wait, task ready, body done, counted in}; the last record is {start, XCD,
// left}. The library build records nothing (no code, no cost).
constexpr int kTraceTasks = FCQT_TRACE_TASKS, kTraceFields = FCQT_TRACE_FIELDS;
#ifdef FCQT_FLOW_TRACE
static unsigned long long* g_trace = nullptr;
__device__ __forceinline__ void trace_at(const FlowArgs& p, int i, int f, unsigned long long v) {
    if (p.trace && threadIdx.x == 0 && i < kTraceTasks)
        p.trace[((long)blockIdx.x * kTraceTasks + i) * kTraceFields + f] = v;
}
#else
__device__ __forceinline__ void trace_at(const FlowArgs&, int, int, unsigned long long) {}
#endif
__device__ __forceinline__ unsigned long long clock100() { return __builtin_amdgcn_s_memrealtime(); }

// One lane waits until *c >= target. False when the wait gave up: it ran
// past its bound (error bit set here) or another wait had already failed.
// The error word, one line that every waiting workgroup of the chip would
// read, is looked at only once a wait has lasted kErrPollTicks.
constexpr uint64_t kErrPollTicks = 2000;    // 20 us
__device__ __forceinline__ bool flow_wait(const unsigned* c, unsigned target, unsigned* err, uint64_t bound) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        if (sync_load(c) >= target) return true;
        const uint64_t dt = __builtin_amdgcn_s_memrealtime() - t0;
        if (dt > bound) {
            __hip_atomic_fetch_or(err, kErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        if (dt > kErrPollTicks && sync_load(err)) return false;
        __builtin_amdgcn_s_sleep(4);
    }
}

// Lane 0 takes the next position of this XCD's queue and waits for its
// dependencies; the task (stage 0: the queue is done) goes to every lane
// through LDS. A stage-2/3 task drops this CU's L1 before its body reads.
// The claim is taken one task ahead: lane 0 issues the atomic for the
// position after this one before the body starts, and reads it here at the
// next task (`next`, -1 before the first), so its latency (about as long as
// a load round trip) hides under the body's own loads. A workgroup thus
// holds its next position while it runs a task; every dependency of that
// position still sits at an earlier one, so every wait still ends.
__device__ __forceinline__ int flow_next(const FlowArgs& p, int x, long K, int* sh, long& b, int& t, long& next) {
    unsigned* head = p.sync + (long)p.batch * FCQT_SYNC_PER_SLICE;
    unsigned* claim = head + kHeadClaim + 32 * x;
    if (threadIdx.x == 0) {
        const long j = next >= 0 ? next
                                 : (long)__hip_atomic_fetch_add(claim, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int stage = 0, tt = 0;
        long k = 0;
        const long end = flow_end(p.order, K);
        if (j < end) {
            flow_decode(p.order, K, j, stage, k, tt);
            const long g = x + (long)kFlowQueues * k;
            const unsigned* rec = p.sync + g * FCQT_SYNC_PER_SLICE;
            if (stage == 2) flow_wait(rec + kSyncStage1, (unsigned)p.order.n1, head + kHeadError, p.wait_ticks);
            if (stage == 3) flow_wait(rec + kSyncStage2, (unsigned)p.order.n2, head + kHeadError, p.wait_ticks);
            sh[1] = (int)g;
            sh[2] = tt;
            // the position after this one, in flight during the body
            next = (long)__hip_atomic_fetch_add(claim, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        sh[0] = stage;
    }
    __syncthreads();
    // workgroup-uniform: scalar registers, as blockIdx-derived indices would be
    const int stage = __builtin_amdgcn_readfirstlane(sh[0]);
    b = __builtin_amdgcn_readfirstlane(sh[1]);
    t = __builtin_amdgcn_readfirstlane(sh[2]);
    if (stage >= 2) asm volatile("buffer_inv sc0" ::: "memory");
    return stage;
}

// After a stage-1 or stage-2 body: this workgroup's stores are in the L2,
// then the slice's counter moves. After a stage-3 body: a barrier (the next
// task reuses the LDS).
__device__ __forceinline__ void flow_done(const FlowArgs& p, int stage, long b) {
    if (stage < 3) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (stage < 3 && threadIdx.x == 0)
        __hip_atomic_fetch_add(p.sync + b * FCQT_SYNC_PER_SLICE + (stage == 1 ? kSyncStage1 : kSyncStage2), 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A workgroup leaving: the last one checks that every queue with tasks was
// served and, if the error word is zero, returns every counter to zero.
__device__ __forceinline__ void flow_exit(const FlowArgs& p, int* sh) {
    unsigned* head = p.sync + (long)p.batch * FCQT_SYNC_PER_SLICE;
    if (threadIdx.x == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const unsigned left = __hip_atomic_fetch_add(head + kHeadExit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int clear = 0;
        if (left == gridDim.x - 1) {
            unsigned unserved = 0;
            for (int q = 0; q < kFlowQueues; ++q)
                if ((long)sync_load(head + kHeadClaim + 32 * q) < flow_end(p.order, flow_slices(p.batch, q)))
                    unserved = 1;
            if (unserved)
                __hip_atomic_fetch_or(head + kHeadError, kErrUnserved, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            clear = sync_load(head + kHeadError) == 0u;
        }
        sh[3] = clear;
    }
    __syncthreads();
    if (sh[3]) {
        for (long g = threadIdx.x; g < p.batch; g += kFlowThreads) {
            __hip_atomic_store(p.sync + g * FCQT_SYNC_PER_SLICE + kSyncStage1, 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.sync + g * FCQT_SYNC_PER_SLICE + kSyncStage2, 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        if (threadIdx.x < kFlowQueues)
            __hip_atomic_store(head + kHeadClaim + 32 * threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x == 0)
            __hip_atomic_store(head + kHeadExit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The thread index and the table pointers of one task, made opaque to the
// compiler at every task. Seen as loop invariants, the bodies' thread-index
// address arithmetic (all seven band lengths, both pass shapes) and their
// table loads are hoisted out of the task loop and kept live across it:
// 255-256 VGPRs, a quarter of the occupancy. Recomputed per task they cost
// a few instructions.
template <class T>
__device__ __forceinline__ T* opaque(T* q) {
    asm volatile("" : "+s"(q));
    return q;
}

__device__ __forceinline__ FlowArgs flow_task_args(const FlowArgs& p, int& tid) {
    tid = (int)threadIdx.x;
    asm volatile("" : "+v"(tid));
    FlowArgs q = p;
    q.twp = opaque(p.twp);
    q.twh = opaque(p.twh);
    q.tws = opaque(p.tws);
    q.tasks = opaque(p.tasks);
    q.rec = opaque(p.rec);
    q.ovf = opaque(p.ovf);
    return q;
}

template <int LAYOUT, bool WT>
__global__ __launch_bounds__(kFlowThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_flow_analysis(const FlowArgs p) {
    __shared__ float2 lds[kFlowLds];
    __shared__ int sh[4];
    const int x = (int)(xcc_id() & (kFlowQueues - 1));
    const long K = flow_slices(p.batch, x);
    long next = -1;
    int it = 0;
    trace_at(p, kTraceTasks - 1, 0, clock100());
    trace_at(p, kTraceTasks - 1, 1, (unsigned long long)x);
    for (;;) {
        long b;
        int t;
        trace_at(p, it, 1, clock100());
        const int stage = flow_next(p, x, K, sh, b, t, next);
        trace_at(p, it, 2, clock100());
        if (stage == 0) {
            trace_at(p, kTraceTasks - 1, 2, clock100());
            break;
        }
        trace_at(p, it, 0, (unsigned long long)stage | ((unsigned long long)b << 8) | ((unsigned long long)t << 40));
        int tid;
        const FlowArgs q = flow_task_args(p, tid);
        if (stage == 1) {
            col_fwd_tile<false, kFColsPerTile>((int)b, t, q.x, q.work, q.twp, q.tws,
                                               SliceSrc{nullptr, nullptr, 1, 1, 0, 0, 0, nullptr, 1, 1, 1}, lds, tid);
        } else if (stage == 2) {
            row_fwd_tile<kFRowsPerTile>((int)b, t, q.work, q.xs, q.twh, q.tws, lds, tid);
        } else {
            route_task<LAYOUT, WT>(t, (int)b, q.xs, q.cre, q.cim, q.rec, q.tasks, q.ncoef, SliceMap{nullptr, 1, 0},
                                   q.tws, lds, tid);
        }
        trace_at(p, it, 3, clock100());
        flow_done(p, stage, b);
        trace_at(p, it, 4, clock100());
        ++it;
    }
    flow_exit(p, sh);
}

template <int LAYOUT, bool WT>
__global__ __launch_bounds__(kFlowThreads) void k_flow_synthesis(const FlowArgs p) {
    __shared__ float2 lds[kFlowLds];
    __shared__ int sh[4];
    const int x = (int)(xcc_id() & (kFlowQueues - 1));
    const long K = flow_slices(p.batch, x);
    long next = -1;
    int it = 0;
    trace_at(p, kTraceTasks - 1, 0, clock100());
    trace_at(p, kTraceTasks - 1, 1, (unsigned long long)x);
    for (;;) {
        long b;
        int t;
        trace_at(p, it, 1, clock100());
        const int stage = flow_next(p, x, K, sh, b, t, next);
        trace_at(p, it, 2, clock100());
        if (stage == 0) {
            trace_at(p, kTraceTasks - 1, 2, clock100());
            break;
        }
        trace_at(p, it, 0, (unsigned long long)stage | ((unsigned long long)b << 8) | ((unsigned long long)t << 40));
        int tid;
        const FlowArgs q = flow_task_args(p, tid);
        if (stage == 1) {
            scatter_task<LAYOUT, false>(t, (int)b, q.cre, q.cim, q.f, q.rec, q.tasks, q.ncoef,
                                        SliceMap{nullptr, 1, 0}, q.tws, lds, tid);
        } else if (stage == 2) {
            col_inv_tile<kFInvColsPerTile, false>((int)b, t, reinterpret_cast<const float2*>(q.f), q.work, q.twp,
                                                  q.twh, q.ovf, q.tws, lds, tid);
        } else {
            row_inv_tile<kFRowsPerTile, WT>((int)b, t, q.work, q.y, q.tws, lds, tid);
        }
        trace_at(p, it, 3, clock100());
        flow_done(p, stage, b);
        trace_at(p, it, 4, clock100());
        ++it;
    }
    flow_exit(p, sh);
}

// Workgroups per queue: enough for the largest queue's tasks, at most the
// slots of one XCD: 32 CUs x 8 workgroups for the analysis (LDS-bound; its
// kernel is held to 4 waves per SIMD, 127 VGPRs) and x 6 for the synthesis
// (its loop needs 147 VGPRs, 3 waves per SIMD; held to 128 it spills).
constexpr int kFlowSlotsAnalysis = 256, kFlowSlotsSynthesis = 192;
constexpr int kFlowSlotsPerXcd = kFlowSlotsAnalysis;

static dim3 flow_grid(int64_t batch, const FlowOrder& o, int slots) {
    const int64_t per = std::min<int64_t>(slots, flow_end(o, flow_slices(batch, 0)));
    return dim3((unsigned)(kFlowQueues * std::max<int64_t>(per, 1)));
}

static int check_flow_args(const uint32_t* sync, int64_t batch, const FlowOrder& o) {
    if (!sync) return FCQT_EARG;
    if (!aligned(sync, 16)) return FCQT_EALIGN;
    if (!flow_order_ok(o)) return FCQT_EARG;
    // positions of the largest queue, plus one claim past its end by every
    // workgroup of the grid (whatever XCD each lands on), stay below 2^32
    // (the claim counters are 32-bit)
    if (flow_end(o, flow_slices(batch, 0)) + (int64_t)kFlowQueues * kFlowSlotsPerXcd >= ((int64_t)1 << 32))
        return FCQT_EARG;
    return FCQT_OK;
}

// Settings of fcqt_persist_tune: lags per direction and the wait bound.
// Defaults: the fastest lags of a sweep at B = 1 / 16 / 64 (B = 64 per
// call: analysis 65.0 us at (4, 16) against 68.8 at (2, 4) and 64.9-66.0 at
// (4, 8) to (16, 32); synthesis 60.2 us at (4, 8) against 72.2 at (2, 4),
// 80.7 at (1, 8) and 61.9 at (8, 16); B = 1 and 16 within 0.5 us for all).
static FlowOrder g_order_analysis{kFColTiles, kFRowTiles, 0, 4, 16};
static FlowOrder g_order_synthesis{0, kFInvColTiles, kFRowTiles, 4, 8};
static int64_t g_wait_ticks = kWaitTicksDefault;

}  // namespace fcqt

using namespace fcqt;

extern "C" int fcqt_persist_trace(void* buf, int64_t bytes) {
#ifdef FCQT_FLOW_TRACE
    if (!buf) {
        g_trace = nullptr;
        return FCQT_OK;
    }
    // room for the largest grid either direction launches
    const int64_t need = (int64_t)kFlowQueues * kFlowSlotsPerXcd * kTraceTasks * kTraceFields * 8;
    if (bytes < need || !aligned(buf, 8)) return FCQT_EARG;
    g_trace = static_cast<unsigned long long*>(buf);
    return FCQT_OK;
#else
    (void)buf;
    (void)bytes;
    return FCQT_EARG;   // this build records no trace
#endif
}

extern "C" int fcqt_persist_tune(int direction, int d1, int d2, int64_t wait_ticks) {
    if (direction != 0 && direction != 1) return FCQT_EARG;
    if (d1 < 0 || d2 < d1 || d2 > 64) return FCQT_EARG;
    FlowOrder& o = direction == 0 ? g_order_analysis : g_order_synthesis;
    o.d1 = d1;
    o.d2 = d2;
    if (wait_ticks >= 0) g_wait_ticks = wait_ticks;
    return FCQT_OK;
}

extern "C" int fcqt_persist_analysis(const fcqt_tables* tab, const int32_t* route, const float* x, float* coef_re,
                                     float* coef_im, int layout, float* xs, float* work, uint32_t* sync,
                                     int64_t batch, hipStream_t stream) {
    if (!route || !x || !xs || !work) return FCQT_EARG;
    if (int e = check_band_args(tab, route, coef_re, coef_im, layout, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    FlowOrder o = g_order_analysis;
    o.n3 = tab->ntasks;
    if (int e = check_flow_args(sync, batch, o)) return e;
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
    p.order = o;
    p.wait_ticks = (uint64_t)g_wait_ticks;
#ifdef FCQT_FLOW_TRACE
    p.trace = g_trace;
#endif
    const dim3 grid = flow_grid(batch, o, kFlowSlotsAnalysis);
    // coefficient stores through the L2 from 4 slices up, as the band kernels
    const bool wt = batch >= 4;
    if (layout == FCQT_PLANAR) {
        if (wt) hipLaunchKernelGGL((k_flow_analysis<FCQT_PLANAR, true>), grid, dim3(kFlowThreads), 0, stream, p);
        else hipLaunchKernelGGL((k_flow_analysis<FCQT_PLANAR, false>), grid, dim3(kFlowThreads), 0, stream, p);
    } else {
        if (wt) hipLaunchKernelGGL((k_flow_analysis<FCQT_INTERLEAVED, true>), grid, dim3(kFlowThreads), 0, stream, p);
        else hipLaunchKernelGGL((k_flow_analysis<FCQT_INTERLEAVED, false>), grid, dim3(kFlowThreads), 0, stream, p);
    }
    return launch_status();
}

extern "C" int fcqt_persist_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* ovf,
                                      const float* coef_re, const float* coef_im, int layout, float* f, float* work,
                                      float* y, uint32_t* sync, int64_t batch, hipStream_t stream) {
    if (!scat || !ovf || !f || !work || !y) return FCQT_EARG;
    if (int e = check_band_args(tab, scat, coef_re, coef_im, layout, batch)) return e;
    if (!tab->tw_pass || !tab->tw_half) return FCQT_EARG;
    FlowOrder o = g_order_synthesis;
    o.n1 = tab->ntasks;
    if (int e = check_flow_args(sync, batch, o)) return e;
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
    p.order = o;
    p.wait_ticks = (uint64_t)g_wait_ticks;
#ifdef FCQT_FLOW_TRACE
    p.trace = g_trace;
#endif
    const dim3 grid = flow_grid(batch, o, kFlowSlotsSynthesis);
    // output stores through the L2 at the batches where the wide inverse
    // passes use them
    const bool wt = batch >= 4 && batch <= kInvWriteThroughMaxBatch;
    if (layout == FCQT_PLANAR) {
        if (wt) hipLaunchKernelGGL((k_flow_synthesis<FCQT_PLANAR, true>), grid, dim3(kFlowThreads), 0, stream, p);
        else hipLaunchKernelGGL((k_flow_synthesis<FCQT_PLANAR, false>), grid, dim3(kFlowThreads), 0, stream, p);
    } else {
        if (wt) hipLaunchKernelGGL((k_flow_synthesis<FCQT_INTERLEAVED, true>), grid, dim3(kFlowThreads), 0, stream, p);
        else hipLaunchKernelGGL((k_flow_synthesis<FCQT_INTERLEAVED, false>), grid, dim3(kFlowThreads), 0, stream, p);
    }
    return launch_status();
}
