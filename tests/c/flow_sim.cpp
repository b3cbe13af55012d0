// Host replay of the single-launch task order (flash-cqt_amd/csrc/fcqt_flow.hpp,
// compiled here without HIP) and of the persistent workgroups' protocol in
// persist.hip, as a discrete-event simulation with random task durations:
//   - every position of every queue decodes to a distinct task, and the
//     positions cover every (stage, slice, tile) of the queue exactly once;
//   - every task's dependencies (all stage-1 tasks of its slice for stage 2,
//     all stage-2 tasks for stage 3) sit at earlier positions;
//   - P workgroups per queue that take positions in order (each claiming
//     its next position when a task starts and holding it while the task
//     runs), wait for their slice's counter and count in when done always
//     finish (no deadlock), never run a task before its dependencies, and
//     leave with the claim counter at end + P (the last-workgroup check of
//     persist.hip).
// Usage: flow_sim  -> prints "ok <cases>" or the first failure, exit 1.
#include <cstdio>
#include <cstdlib>
#include <queue>
#include <random>
#include <vector>

#include "../../flash-cqt_amd/csrc/fcqt_flow.hpp"

using fcqt::FlowOrder;

static int fail(const char* what, long B, const FlowOrder& o, int x, long j) {
    std::printf("FAIL %s B=%ld n=(%d,%d,%d) d=(%d,%d) queue=%d pos=%ld\n", what, B, o.n1, o.n2, o.n3, o.d1, o.d2, x,
                j);
    return 1;
}

// Order properties of one queue.
static int check_order(long B, const FlowOrder& o, int x) {
    const long K = fcqt::flow_slices(B, x);
    const long end = fcqt::flow_end(o, K);
    const int n[4] = {0, o.n1, o.n2, o.n3};
    std::vector<long> pos(3 * K * 256, -1);   // (stage - 1, k, t) -> position; n <= 256
    auto idx = [&](int st, long k, int t) { return ((st - 1) * K + k) * 256 + t; };
    for (long j = 0; j < end; ++j) {
        int st = 0, t = -1;
        long k = -1;
        fcqt::flow_decode(o, K, j, st, k, t);
        if (st < 1 || st > 3 || k < 0 || k >= K || t < 0 || t >= n[st]) return fail("decode range", B, o, x, j);
        long& p = pos[idx(st, k, t)];
        if (p >= 0) return fail("task decoded twice", B, o, x, j);
        p = j;
    }
    for (long k = 0; k < K; ++k)
        for (int st = 1; st <= 3; ++st) {
            long lo = end, hi = -1;
            for (int t = 0; t < n[st]; ++t) {
                const long p = pos[idx(st, k, t)];
                if (p < 0) return fail("task never decoded", B, o, x, k);
                lo = p < lo ? p : lo;
                hi = p > hi ? p : hi;
            }
            if (st > 1) {
                long prev_hi = -1;
                for (int t = 0; t < n[st - 1]; ++t) {
                    const long p = pos[idx(st - 1, k, t)];
                    prev_hi = p > prev_hi ? p : prev_hi;
                }
                if (prev_hi >= lo) return fail("dependency at a later position", B, o, x, k);
            }
        }
    return 0;
}

// Event simulation of P workgroups serving one queue, each taking its
// positions one task ahead as the kernel does: a workgroup's first position
// is claimed when it starts, and the position after each task is claimed
// when that task starts (held while it runs).
static int simulate(long B, const FlowOrder& o, int x, int P, std::mt19937& rng) {
    const long K = fcqt::flow_slices(B, x);
    const long end = fcqt::flow_end(o, K);
    std::vector<int> done1(K, 0), done2(K, 0), done3(K, 0);
    long claim = 0;
    struct Ev {
        double t;
        int wg;
        bool operator<(const Ev& e) const { return t > e.t; }
    };
    std::priority_queue<Ev> ev;
    std::uniform_real_distribution<double> start(0.0, 2.0), dur(0.5, 3.0);
    for (int w = 0; w < P; ++w) ev.push({start(rng), w});
    std::vector<int> st(P, 0);
    std::vector<long> kk(P, -1), held(P, -1);
    std::vector<int> state(P, 0);   // 0: take the held (or a first) position, 1: running, 2: waiting, 3: left
    int left = 0;
    long steps = 0;
    while (!ev.empty()) {
        if (++steps > 50000000) return fail("simulation did not end", B, o, x, claim);
        Ev e = ev.top();
        ev.pop();
        const int w = e.wg;
        if (state[w] == 1) {   // task finished: count in
            if (st[w] == 1) ++done1[kk[w]];
            if (st[w] == 2) ++done2[kk[w]];
            if (st[w] == 3) ++done3[kk[w]];
            state[w] = 0;
        }
        if (state[w] == 0) {   // the held position, or a first claim
            const long j = held[w] >= 0 ? held[w] : claim++;
            held[w] = -1;
            if (j >= end) {
                state[w] = 3;
                ++left;
                continue;
            }
            int s = 0, t = 0;
            long k = 0;
            fcqt::flow_decode(o, K, j, s, k, t);
            st[w] = s, kk[w] = k;
            state[w] = 2;
        }
        if (state[w] == 2) {   // wait for the dependencies, polling
            const bool ready = st[w] == 1 || (st[w] == 2 && done1[kk[w]] == o.n1) ||
                               (st[w] == 3 && done2[kk[w]] == o.n2);
            if (!ready) {
                ev.push({e.t + 0.05, w});
                continue;
            }
            held[w] = claim++;      // the next position, held while this task runs
            state[w] = 1;
            ev.push({e.t + dur(rng), w});
        }
    }
    if (left != P) return fail("a workgroup never left", B, o, x, claim);
    if (claim != end + P) return fail("claim counter not at end + P", B, o, x, claim);
    for (long k = 0; k < K; ++k)
        if (done1[k] != o.n1 || done2[k] != o.n2 || done3[k] != o.n3) return fail("task not run", B, o, x, k);
    return 0;
}

int main() {
    std::mt19937 rng(12345);
    int cases = 0;
    const int nts[][3] = {{16, 16, 68}, {68, 16, 16}, {16, 16, 1}, {1, 1, 1}, {3, 5, 7}};
    const int lags[][2] = {{0, 0}, {0, 1}, {1, 1}, {2, 4}, {2, 3}, {4, 8}, {8, 8}, {0, 16}, {16, 16}, {3, 64}};
    const long batches[] = {1, 2, 5, 7, 8, 9, 16, 17, 64, 65, 130};
    for (auto& n : nts)
        for (auto& d : lags) {
            const FlowOrder o{n[0], n[1], n[2], d[0], d[1]};
            if (!fcqt::flow_order_ok(o)) return fail("order rejected", 0, o, 0, 0);
            for (long B : batches)
                for (int x = 0; x < fcqt::kFlowQueues; ++x) {
                    if (check_order(B, o, x)) return 1;
                    ++cases;
                }
        }
    // the protocol, at a few worker counts (1 = fully serial, more than the
    // tasks, and the kernel's per-XCD slot counts)
    const int workers[] = {1, 3, 37, 192, 256, 600};
    for (auto& n : nts)
        for (auto& d : lags) {
            const FlowOrder o{n[0], n[1], n[2], d[0], d[1]};
            for (long B : {1l, 9l, 64l, 130l})
                for (int P : workers) {
                    if (simulate(B, o, (int)(B % fcqt::kFlowQueues), P, rng)) return 1;
                    ++cases;
                }
        }
    // orders the launchers refuse
    const FlowOrder bad[] = {{16, 16, 68, 2, 1}, {16, 16, 68, -1, 2}, {0, 16, 68, 0, 0}, {16, 16, 68, 0, 65}};
    for (auto& o : bad)
        if (fcqt::flow_order_ok(o)) return fail("bad order accepted", 0, o, 0, 0);
    // a planted mistake must fail: stage 3 of a slice ahead of its stage 2
    // (lags d1 > d2, which the launchers refuse) deadlocks or reads early
    {
        const FlowOrder o{16, 16, 68, 3, 1};
        std::printf("planted: ");
        if (!check_order(64, o, 0) && !simulate(64, o, 0, 1, rng)) {
            std::printf("FAIL planted order passed\n");
            return 1;
        }
    }
    std::printf("ok %d\n", cases);
    return 0;
}
