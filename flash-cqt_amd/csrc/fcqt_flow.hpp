// Task order of the single-launch directions (persist.hip), host and device.
//
// A direction is three stages per slice: n1 stage-1 tasks (dependency
// free), n2 stage-2 tasks (each needs all stage-1 tasks of its slice) and
// n3 stage-3 tasks (each needs all stage-2 tasks of its slice). The slices
// of a batch are split over Q queues, one per XCD: queue x holds the
// slices x, x + Q, x + 2Q, ... (local slice k is slice x + Q k), and the
// workgroups on XCD x (read from the hardware, not from blockIdx) take the
// queue's tasks one at a time in its order, by position j = 0, 1, 2, ...
//
// The order is a sequence of steps. Step s holds, in this order,
//   the n1 stage-1 tasks of local slice s            (if s < K)
//   the n2 stage-2 tasks of local slice s - d1       (if 0 <= s - d1 < K)
//   the n3 stage-3 tasks of local slice s - d2       (if 0 <= s - d2 < K)
// for K local slices and lags 0 <= d1 <= d2, so a slice's stage 2 is taken
// d1 steps after its stage 1 and its stage 3 d2 steps after it: by the time
// a workgroup takes a task, the tasks it waits for were taken about a
// step's worth of tasks times the lag earlier. Positions run over exactly
// K (n1 + n2 + n3) tasks, every task once.
//
// Every task's dependencies sit at earlier positions (d1 >= 0, d2 >= d1,
// and inside a step the stages come in order), so a taken task only ever
// waits for tasks taken before it, by running workgroups: every wait ends,
// whatever the number of workgroups and however many are resident.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define FCQT_HD __host__ __device__ __forceinline__
#else
#define FCQT_HD inline
#endif

namespace fcqt {

constexpr int kFlowQueues = 8;     // one per XCD of an MI355X

struct FlowOrder {
    int n1, n2, n3;   // tasks per slice of stages 1..3
    int d1, d2;       // lags in steps: stage 2 and stage 3 after stage 1
};

FCQT_HD long flow_clamp(long v, long lo, long hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Local slices of queue x for a batch of B slices.
FCQT_HD long flow_slices(long B, int x) { return B > x ? (B - x + kFlowQueues - 1) / kFlowQueues : 0; }

// Position of the first task of step s (0 <= s <= K + d2).
FCQT_HD long flow_step_start(const FlowOrder& o, long K, long s) {
    return o.n1 * flow_clamp(s, 0, K) + o.n2 * flow_clamp(s - o.d1, 0, K) + o.n3 * flow_clamp(s - o.d2, 0, K);
}

// Positions of a queue with K local slices: K (n1 + n2 + n3).
FCQT_HD long flow_end(const FlowOrder& o, long K) { return K * (long)(o.n1 + o.n2 + o.n3); }

// Task at position j (0 <= j < flow_end): stage (1..3), local slice k and
// the task's index t within its stage of that slice.
FCQT_HD void flow_decode(const FlowOrder& o, long K, long j, int& stage, long& k, int& t) {
    // the step s with start(s) <= j < start(s + 1): start is nondecreasing in s
    long lo = 0, hi = K + o.d2;      // start(lo) <= j < start(hi)
    while (hi - lo > 1) {
        const long mid = (lo + hi) / 2;
        if (flow_step_start(o, K, mid) <= j) lo = mid;
        else hi = mid;
    }
    const long s = lo;
    long off = j - flow_step_start(o, K, s);
    if (s < K) {
        if (off < o.n1) {
            stage = 1, k = s, t = (int)off;
            return;
        }
        off -= o.n1;
    }
    if (s - o.d1 >= 0 && s - o.d1 < K) {
        if (off < o.n2) {
            stage = 2, k = s - o.d1, t = (int)off;
            return;
        }
        off -= o.n2;
    }
    stage = 3, k = s - o.d2, t = (int)off;
}

// Checks of an order the launchers accept (the lags keep every
// dependency at an earlier position).
FCQT_HD bool flow_order_ok(const FlowOrder& o) {
    return o.n1 > 0 && o.n2 > 0 && o.n3 > 0 && o.d1 >= 0 && o.d2 >= o.d1 && o.d2 <= 64;
}

}  // namespace fcqt
