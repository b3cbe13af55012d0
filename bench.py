#!/usr/bin/env python3
"""Benchmark of the fused factored CQT round trip on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one fused round trip (analysis + synthesis) of a batch of
65536-sample fp32 slices with the input already in device memory. Each batch
size is timed both as hipGraph replays and as plain stream launches (K steps
back to back between two events) and runs in the faster mode: graph replay
carries a fixed per-launch cost on this runtime, stream launches the host's
launch cost. The timed region is exactly K steps at batch 64 (BASELINE
configs[2]); batch 1 (configs[1], sinusoids + noise) and batch 16 are in
"per_batch" with both modes' timings. Beside them, in the same run:
  - the hipFFT-call baseline: the package's pure-torch OctCQT (torch.fft ->
    hipFFT/rocFFT) on the GPU, graph-captured, same inputs;
  - the host-core baseline: the oracle's torch port of the reference
    OctCQT on the box's CPU cores, a bounded sample (cpu_baseline);
  - the SlicedCQT streaming workload in "sliced", with a long
    signal (512 slices) in "sliced.long_signal";
  - the TrainableCQT differentiable step in "training_step".
Per-kernel launch durations are timed with hipEvents on the launch stream
around back-to-back stream launches (graphs of the same launches beside
them); "roofline" reports the dominant kernel's algorithmic bytes per launch
over its duration against 8 TB/s.

Extra modes (for rocprofv3 counter runs): --kernels-only runs a few
launches of every kernel plus a plain copy of known size (the calibration
kernel for FETCH_SIZE / WRITE_SIZE) and prints nothing else; --sliced-only
runs the SlicedCQT workload alone and prints its JSON object;
--sliced-long-only does the same for the long-signal measurement.
"""
import argparse
import json
import math
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "flash-cqt_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

N = 65536
L = N // 2
FS = 44100
METRIC = "CQT round trips/sec (fwd+inv, 65536 samples) at batch 1/16/64; HBM GB/s"
PEAK_GBPS = 8000.0
# algorithmic bytes per slice (fp32; tables excluded, batch invariant)
SLICE_RT_BYTES = 2 * 262144 + 2 * 1063936     # x in, coefficients out, coefficients in, y out
KERNEL_BYTES = {
    "packed_fft": 262144 + 262152,            # x in, X (L+1 bins) out
    "route_bands": 262152 + 1063936,          # X in, coefficients out
    "scatter_bands": 1063936 + 262152,        # coefficients in, half spectrum out
    "packed_ifft": 262152 + 262144,           # half spectrum in, y out
}
KERNEL_LAUNCHES = {"packed_fft": 2, "route_bands": 1, "scatter_bands": 1, "packed_ifft": 2}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def sinusoids(seed=0):
    """8 unit sinusoids, log-uniform 43 Hz..20 kHz, random phase, + N(0, 0.01^2)."""
    rs = np.random.RandomState(seed)
    f = np.exp(rs.uniform(np.log(43.0), np.log(20000.0), 8))
    ph = rs.uniform(0, 2 * np.pi, 8)
    n = np.arange(N)
    x = np.sum(np.sin(2 * np.pi * f[:, None] * n[None, :] / FS + ph[:, None]), 0)
    return (x + 0.01 * rs.standard_normal(N))[None, :].astype(np.float32)


def randn(B, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, N, generator=g, dtype=torch.float32)


def snr_db(ref, got):
    ref = ref.double()
    e = ref.square().sum()
    d = (ref - got.double()).square().sum()
    return float("inf") if float(d) == 0 else float(10 * torch.log10(e / d))


def json_safe(v):
    """Strict JSON: an infinite SNR (bitwise-equal results) becomes the string "inf"."""
    if isinstance(v, dict):
        return {k: json_safe(u) for k, u in v.items()}
    if isinstance(v, (list, tuple)):
        return [json_safe(u) for u in v]
    if isinstance(v, float) and not math.isfinite(v):
        return str(v)
    return v


def capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def median_ms(fn, reps=50, warm=3):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        e.synchronize()
        ts.append(s.elapsed_time(e))
    ts.sort()
    return ts[len(ts) // 2]


def per_step_ms(step, steps=50, warm=5):
    """GPU time per step over `steps` back-to-back steps (event pair)."""
    for _ in range(warm):
        step()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        step()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / steps


def best_mode(graph_step, stream_step):
    """Both launch modes of one step, back to back: (ms, mode, step) of the
    faster, plus both timings. Graph replay carries a fixed per-launch cost on
    this runtime; plain stream launches carry the host's launch cost."""
    tg = min(per_step_ms(graph_step), per_step_ms(graph_step))
    ts = min(per_step_ms(stream_step), per_step_ms(stream_step))
    if tg <= ts:
        return tg, "hipGraph replay", graph_step, {"hipGraph replay": tg, "stream launches": ts}
    return ts, "stream launches", stream_step, {"hipGraph replay": tg, "stream launches": ts}


def replay_matches_eager(g, out, eager, poison, reps=3):
    """Poison what the graph must write, replay, compare with eager; repeat
    with eager work in between."""
    worst = float("inf")
    for r in range(reps):
        for t in poison:
            t.fill_(1e9 if r % 2 == 0 else float("nan"))
        g.replay()
        torch.cuda.synchronize()
        worst = min(worst, snr_db(eager, out))
        _ = torch.randn(4096, device=out.device).sum().item()
    return worst


# ----------------------------------------------------------- baselines

def torch_fft_baseline(cqt_gpu, x):
    """Graph-captured pure-torch OctCQT round trip (hipFFT); eager if the
    replay does not reproduce eager results."""
    fn = lambda: cqt_gpu.bwd(*cqt_gpu.fwd(x))
    with torch.no_grad():
        eager = fn().clone()
        try:
            g, out = capture(fn)
            ok = replay_matches_eager(g, out, eager, [out]) > 100
        except Exception as e:  # capture unsupported by a library call
            log(f"hipFFT baseline capture failed: {e}")
            ok = False
        if ok:
            ms, mode, _, _ = best_mode(g.replay, fn)
            return ms, mode, eager
        return per_step_ms(fn), "stream launches", eager


def sliced_workload(dev):
    """SlicedCQT, batch 8 x 441000 samples (10 s chirp 43 Hz..20 kHz
    + N(0, 0.1^2)), 65536-sample slices at 50% overlap, fwd + bwd. Timed
    graph-replayed with the framing inside the engine's kernels, and beside it
    the same round trip composed of the host framing ops around the same
    engine (the reference's structure)."""
    from flash_cqt import SlicedCQT
    T, n = 10.0, np.arange(441000) / FS
    k = math.log(20000.0 / 43.0)
    sweep = np.sin(2 * np.pi * 43.0 * T / k * (np.exp(n / T * k) - 1.0))
    rs = np.random.RandomState(0)
    x = torch.as_tensor((sweep[None, None, :] + 0.1 * rs.standard_normal((8, 1, n.size)))
                        .astype(np.float32)).to(dev)
    s = SlicedCQT(fs=FS, device=dev)
    fused = lambda: s.bwd(*s.fwd(x), length=x.shape[-1])
    res = {"workload": "configs[4] SlicedCQT batch 8 x 441000 samples, 50% overlap",
           "slices": 8 * s._num_slices(x.shape[-1]), "samples": 8 * x.shape[-1]}
    with torch.no_grad():
        y = fused().clone()
        res["roundtrip_snr_db"] = snr_db(x, y)
        g, out = capture(fused)
        res["replay_vs_eager_db"] = replay_matches_eager(g, out, y, [out])
        ms, mode, _, _ = best_mode(g.replay, fused)
        s.fused_framing = False            # the host-framing composition
        yc = fused().clone()
        gc, _ = capture(fused)
        msc, modec, _, _ = best_mode(gc.replay, fused)
        s.fused_framing = True
        # the configs[4] streaming form: hop-sized chunks in, one slice per
        # step, bounded state (fused calls per slice vs host framing per slice)
        hop = s.hop
        S = s._num_slices(x.shape[-1])
        xp = torch.cat([x, torch.zeros(8, 1, (S - 1) * hop - x.shape[-1], device=dev)], dim=-1)
        chunks = [xp[..., i * hop:(i + 1) * hop] for i in range(S - 1)]

        def stream():
            return torch.cat(list(s.stream_bwd(s.stream_fwd(iter(chunks)))), dim=-1)
        ys = stream()
        res["stream_roundtrip_snr_db"] = snr_db(x, ys[..., :x.shape[-1]])
        res["stream_vs_whole_db"] = snr_db(y, ys[..., :x.shape[-1]])
        mss = per_step_ms(stream, steps=5, warm=1)
        s.fused_framing = False
        mss_host = per_step_ms(stream, steps=2, warm=1)
        s.fused_framing = True
    res.update({"stream_ms": mss, "stream_msamples_per_s": res["samples"] / (mss * 1e-3) / 1e6,
                "stream_host_framing_ms": mss_host, "stream_speedup_vs_host_framing": mss_host / mss})
    res.update({"ms": ms, "launch_mode": mode, "host_framing_launch_mode": modec,
                "msamples_per_s": res["samples"] / (ms * 1e-3) / 1e6,
                "host_framing_ms": msc, "speedup_vs_host_framing": msc / ms,
                "host_framing_vs_fused_db": snr_db(yc, y)})
    log(f"sliced: {ms:.4f} ms  {res['msamples_per_s']:.0f} Msamples/s  rt {res['roundtrip_snr_db']:.1f} dB"
        f"  (host framing {msc:.4f} ms); streamed: {mss:.3f} ms  (host framing {mss_host:.3f} ms)"
        f"  rt {res['stream_roundtrip_snr_db']:.1f} dB")
    return res


def sliced_long(dev):
    """A long signal: SlicedCQT on one signal of 512 slices (16.8 M samples,
    6.3 min at 44.1 kHz), fwd and bwd each timed as the product runs them
    (framing + route in chunks of about 128 slices; overlap-add in the
    inverse row pass) and, in the same run, in their one-call forms (framing
    pass + route over all slices; slice buffer + overlap-add kernel)."""
    from flash_cqt import SlicedCQT
    from flash_cqt import sliced as sl
    s = SlicedCQT(fs=FS, device=dev)
    S = 512
    L = (S - 2) * s.hop + 1000
    assert s._num_slices(L) == S
    x = torch.randn(1, 1, L, generator=torch.Generator().manual_seed(3)).to(dev)
    f = s.cqt.f
    with torch.no_grad():
        bl, sd = s.fwd(x)
        y = s.bwd(bl, sd, length=L)
        res = {"workload": "SlicedCQT, one signal of 512 slices (16.8 M samples)", "slices": S,
               "roundtrip_snr_db": snr_db(x, y)}
        res["fwd_ms"] = per_step_ms(lambda: s.fwd(x), steps=10, warm=2)
        res["bwd_ms"] = per_step_ms(lambda: s.bwd(bl, sd, length=L), steps=10, warm=2)
        ws = s._ws(f, 1, S, x="full")      # the unchunked framing pass needs a row of X per slice
        coef = torch.empty(S * f.ncoef, dtype=torch.complex64, device=dev)
        sig = x.reshape(1, L)

        def fwd_one_call():
            f.slice_fft(sig, s._tw32(), S, ws["X"], ws["W"])
            f.route_bands_sliced(ws["X"], coef, 1, S)
        res["fwd_one_call_ms"] = per_step_ms(fwd_one_call, steps=10, warm=2)
        keep = sl.FUSED_OLA_MIN_SLICES
        sl.FUSED_OLA_MIN_SLICES = 1 << 30          # the slice-buffer synthesis
        try:
            res["bwd_slice_buffer_ms"] = per_step_ms(lambda: s.bwd(bl, sd, length=L), steps=10, warm=2)
        finally:
            sl.FUSED_OLA_MIN_SLICES = keep
    log(f"sliced long signal ({S} slices): fwd {res['fwd_ms']:.3f} ms (one call {res['fwd_one_call_ms']:.3f}),"
        f" bwd {res['bwd_ms']:.3f} ms (slice buffer {res['bwd_slice_buffer_ms']:.3f}),"
        f" rt {res['roundtrip_snr_db']:.1f} dB")
    return res


def training_step(dev, cqt_gpu):
    """TrainableCQT differentiable step at batch 16 (analysis ->
    synthesis -> MSE against a second randn target -> backward), stream
    launches with autograd, beside the same step through the pure-torch
    OctCQT (torch.fft -> hipFFT/rocFFT) with autograd."""
    from flash_cqt.trainable import TrainableCQT
    train = TrainableCQT(cqt_gpu, dev)
    x, tgt = randn(16, 0).to(dev), randn(16, 1).to(dev)
    xg = x.clone().requires_grad_(True)

    def step_with(engine):
        def step():
            xg.grad = None
            y = engine.bwd(*engine.fwd(xg))
            ((y - tgt) ** 2).mean().backward()
        return step

    ours, ref = step_with(train), step_with(cqt_gpu)
    ref()
    g_ref = xg.grad.clone()
    ours()
    res = {"workload": "configs[3] TrainableCQT step, batch 16: fwd -> bwd -> MSE -> backward",
           "grad_snr_db_vs_torch_fft": snr_db(g_ref, xg.grad)}
    ms, ms_ref = per_step_ms(ours, steps=30), per_step_ms(ref, steps=10)
    res.update({"ms": ms, "steps_per_s": 1e3 / ms, "hipfft_baseline_ms": ms_ref, "speedup_vs_hipfft": ms_ref / ms})
    log(f"training step B=16: {ms:.4f} ms  (hipFFT autograd {ms_ref:.4f} ms)  grad {res['grad_snr_db_vs_torch_fft']:.1f} dB")
    return res


def cpu_baseline(batch=64, budget_s=10.0, budget_b1_s=4.0, max_reps=400):
    """The reference OctCQT algorithm (oracle torch port) on the host cores,
    on a bounded sample of the bench's own workload (batch-`batch` round trips
    of the randn input, about budget_s of CPU work), plus batch 1 on the
    configs[1] input and batches 4 and 16 on randn input (short samples).
    torch runs with os.cpu_count() threads (every core the host reports); the
    CPUs this process may run on (affinity) and the cgroup CPU quota are
    reported beside it. The previous thread count is restored."""
    from oracle.torch_port import TorchPortOctCQT
    cores = os.cpu_count() or 1
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        return _cpu_baseline(TorchPortOctCQT(), cores, batch, budget_s, budget_b1_s, max_reps)
    finally:
        torch.set_num_threads(prev_threads)


def host_cpus():
    """CPUs this process may run on, and the cgroup v2 quota in CPUs (None
    if unlimited or unreadable)."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    quota = None
    try:
        q, per = pathlib.Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = int(q) / int(per)
    except (OSError, ValueError):
        pass
    return affinity, quota


def _cpu_baseline(port, cores, batch, budget_s, budget_b1_s, max_reps):

    def timed(x, budget):
        with torch.no_grad():
            y = port.bwd(*port.fwd(x))
            ts = []
            t_end = time.perf_counter() + budget
            while time.perf_counter() < t_end and len(ts) < max_reps:
                t0 = time.perf_counter()
                port.bwd(*port.fwd(x))
                ts.append(time.perf_counter() - t0)
        ts.sort()
        return ts[len(ts) // 2], len(ts), snr_db(x, y)

    med, n, db = timed(randn(batch, 0), budget_s)
    med1, n1, db1 = timed(torch.from_numpy(sinusoids()), budget_b1_s)
    per_batch = {"1": {"round_trips_per_s": 1.0 / med1, "median_ms": med1 * 1e3, "reps": n1},
                 str(batch): {"round_trips_per_s": batch / med, "median_ms": med * 1e3, "reps": n}}
    for b in (4, 16):
        if str(b) not in per_batch:
            mb, nb, _ = timed(randn(b, 0), budget_b1_s / 2)
            per_batch[str(b)] = {"round_trips_per_s": b / mb, "median_ms": mb * 1e3, "reps": nb}
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    affinity, quota = host_cpus()
    return {"value": batch / med, "unit": "slice round trips/s", "cores": cores, "kind": "port",
            "cpu_model": model, "cpus_in_affinity": affinity, "cgroup_cpu_quota": quota,
            "sample": f"{n} batch-{batch} round trips of the bench's randn input (median {med * 1e3:.1f} ms "
                      f"per batch), oracle/torch_port.py, torch CPU {cores} threads (os.cpu_count(); "
                      f"{affinity} CPUs in this process's affinity, cgroup quota {quota} CPUs), {model}",
            "snr_db": db,
            "batch1": {"value": 1.0 / med1, "sample": f"{n1} batch-1 round trips of the configs[1] input "
                                                     f"(median {med1 * 1e3:.2f} ms)", "snr_db": db1},
            "per_batch": per_batch}


# ---------------------------------------------------- single-launch path

def single_launch(f, x, eager):
    """The single-launch directions (one launch of persistent workgroups per
    direction, the reference's persistent pair) at the batch of x,
    stream-launched back to back, and whether they reproduce the six-launch
    round trip bit for bit. The timed calls skip the per-call error check
    (a host synchronization); the error word is read once after them and a
    nonzero word fails the bench."""
    B = x.shape[0]
    step = lambda: f.persist_inv(*f.persist_fwd(x, check=False), check=False)
    with torch.no_grad():
        same = bool(torch.equal(f.persist_inv(*f.persist_fwd(x)), eager))
        ms = min(per_step_ms(step), per_step_ms(step))
    err = f.sync_error(B)
    if err:
        raise RuntimeError(f"single-launch error word {err} at batch {B}")
    return {"ms": ms, "round_trips_per_s": B / (ms * 1e-3), "equal_to_six_launch_bitwise": same,
            "launch_mode": "stream launches", "launches_per_round_trip": 2, "error_word": err}


def launch_floor(f, dev):
    """The per-launch floor on this runtime: the library's smallest kernel (a
    fill of four floats) stream-launched back to back. A round trip is six
    launches, so at batch 1 it takes at least about six of these."""
    from flash_cqt import _native
    tiny = torch.zeros(4, device=dev)
    sh = _native.stream_handle(dev.index)
    ms = min(per_step_ms(lambda: f.lib.fcqt_fill_zero(tiny.data_ptr(), 4, sh), steps=200) for _ in range(3))
    log(f"launch floor: {ms * 1e3:.2f} us per kernel launch (6 per round trip)")
    return {"ms_per_launch": ms, "launches_per_round_trip": 6,
            "kernel": "k_fill_zero of 4 floats, stream-launched back to back"}


def single_launch_workload(f, dev):
    """--single-launch-only: both paths at batches 1, 16, 64 and the
    per-launch floor, for a kernel trace of the single-launch kernels."""
    out = {"launch_floor": launch_floor(f, dev), "per_batch": {}}
    for B in (1, 16, 64):
        x = (torch.from_numpy(sinusoids()) if B == 1 else randn(B, 0)).to(dev)
        fn = lambda x=x: f.bwd(*f.fwd(x))
        with torch.no_grad():
            eager = fn().clone()
        six = min(per_step_ms(fn), per_step_ms(fn))
        r = single_launch(f, x, eager)
        r["six_launch_ms"] = six
        out["per_batch"][str(B)] = r
        log(f"B={B}: six launches {six:.4f} ms, single launch per direction {r['ms']:.4f} ms "
            f"(bitwise equal: {r['equal_to_six_launch_bitwise']})")
    return out


def stage_trace_summary(tr, G, ntrace, nfields):
    """Per-stage figures of one single-launch call's stage trace (the
    fcqt_persist_trace records of its G workgroups): per stage the task
    count, medians / 90th percentiles of claim-or-wait, body and count-in
    times, when the stage's first task was ready and its last done; how
    many task bodies of each stage run, and how many tasks wait after their
    claim, in every 2 us of the call; and when each XCD's last task ended.
    Times in us from the first workgroup's start (100 MHz clock)."""
    a = tr.view(-1, ntrace, nfields)[:G].cpu().numpy().astype(np.int64)
    start = a[:, ntrace - 1, 0]
    t0 = start[start > 0].min()
    rows = []
    for w in range(G):
        for i in range(ntrace - 1):
            info = int(a[w, i, 0])
            if info == 0:
                break
            rows.append((int(a[w, ntrace - 1, 1]), info & 0xff, a[w, i, 1] - t0, a[w, i, 2] - t0, a[w, i, 3] - t0,
                         a[w, i, 4] - t0))
    r = np.array(rows, dtype=np.int64)
    us = lambda v: np.round(v / 100.0, 2)
    out = {"workgroups": int(G), "tasks": len(r), "span_us": float(us(r[:, 5].max())), "stages": {}}
    bins = np.arange(0, r[:, 5].max() + 200, 200)
    for st in (1, 2, 3):
        m = r[r[:, 1] == st]
        if not len(m):
            continue
        cw, body, sig = m[:, 3] - m[:, 2], m[:, 4] - m[:, 3], m[:, 5] - m[:, 4]
        out["stages"][str(st)] = {
            "tasks": len(m),
            "claim_or_wait_us": [float(us(np.median(cw))), float(us(np.percentile(cw, 90)))],
            "body_us": [float(us(np.median(body))), float(us(np.percentile(body, 90)))],
            "count_in_us": [float(us(np.median(sig))), float(us(np.percentile(sig, 90)))],
            "first_ready_us": float(us(m[:, 3].min())), "last_done_us": float(us(m[:, 5].max())),
            "running_per_2us": [int(np.sum((m[:, 3] <= t) & (m[:, 4] > t))) for t in bins],
            "waiting_per_2us": [int(np.sum((m[:, 2] <= t) & (m[:, 3] > t))) for t in bins]}
    out["xcd_end_us"] = [float(us(r[r[:, 0] == x][:, 5].max())) for x in range(8) if np.any(r[:, 0] == x)]
    return out


def single_launch_trace(dev, batches=(1, 16, 64)):
    """--single-launch-trace: one call of each single-launch direction per
    batch size through the trace build of the library
    (libflashcqt_flowtrace.so), with its per-stage timeline; beside it the
    time per call of the library's single-launch and three-launch
    directions (stream-launched back to back, check=False)."""
    from flash_cqt import OctCQT, _native
    from flash_cqt.fused import FusedOctCQT
    cqt_gpu = OctCQT([3, 4, 2], [8, 16, 32], fs=FS, audio_len=N, device=dev)
    f = FusedOctCQT(cqt_gpu, dev)
    ft = FusedOctCQT(cqt_gpu, dev)
    ft.lib = _native.load_variant("flowtrace")
    nt, nf = 32, 6
    tr = torch.zeros(8 * 256 * nt * nf, dtype=torch.int64, device=dev)
    _native.check(ft.lib.fcqt_persist_trace(tr.data_ptr(), tr.numel() * 8), "persist_trace")
    out = {}
    for B in batches:
        x = (torch.from_numpy(sinusoids()) if B == 1 else randn(B, 0)).to(dev)
        with torch.no_grad():
            KR, KI = f.fwd(x)
            k = torch.complex(KR, KI).clone()
            y = f.bwd(KR, KI).clone()
            r = {"ms_per_call": {
                "single_launch_analysis": per_step_ms(lambda: f.persist_fwd(x, check=False)),
                "three_launch_analysis": per_step_ms(lambda: f.fwd(x)),
                "single_launch_synthesis": per_step_ms(lambda: f.persist_inv(KR, KI, check=False)),
                "three_launch_synthesis": per_step_ms(lambda: f.bwd(KR, KI))}}
            if f.sync_error(B):
                raise RuntimeError(f"single-launch error word {f.sync_error(B)} at batch {B}")
            for name, fn in (("analysis", lambda: ft.persist_fwd(x)), ("synthesis", lambda: ft.persist_inv(KR, KI))):
                fn()
                tr.zero_()
                torch.cuda.synchronize()
                res = fn()
                torch.cuda.synchronize()
                same = torch.equal(torch.complex(*res), k) if name == "analysis" else torch.equal(res, y)
                G = int(np.count_nonzero(tr.view(-1, nt, nf)[:, nt - 1, 0].cpu().numpy()))
                r[name] = stage_trace_summary(tr, G, nt, nf)
                r[name]["equal_to_library_bitwise"] = bool(same)
                st = r[name]["stages"]
                log(f"B={B} {name}: span {r[name]['span_us']:.1f} us; " + "; ".join(
                    f"stage {k_}: claim/wait {v['claim_or_wait_us'][0]:.2f} body {v['body_us'][0]:.2f} "
                    f"ready {v['first_ready_us']:.1f}..done {v['last_done_us']:.1f} us" for k_, v in st.items()))
        ms = r["ms_per_call"]
        log(f"B={B}: per call single/three launches: analysis {ms['single_launch_analysis'] * 1e3:.1f} / "
            f"{ms['three_launch_analysis'] * 1e3:.1f} us, synthesis {ms['single_launch_synthesis'] * 1e3:.1f} / "
            f"{ms['three_launch_synthesis'] * 1e3:.1f} us")
        out[str(B)] = r
    _native.check(ft.lib.fcqt_persist_trace(None, 0), "persist_trace")
    return out


# ------------------------------------------------------------ peak memory

def peak_mb(fn):
    """Peak device memory one call allocates beyond what was allocated
    before it, in MB (the reference's recipe, bench/memory_bars.py:24-31)."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    fn()
    torch.cuda.synchronize()
    return (torch.cuda.max_memory_allocated() - base) / 1e6


def peak_memory(cqt_gpu, dev, batches=(1, 8, 16, 32, 64, 128)):
    """Peak MB of one round-trip call per batch size, every buffer the call
    needs allocated inside it (a fresh engine with resident tables: the
    first call of a batch size allocates X, W, F, the coefficient planes
    and the output), beside the hipFFT-call baseline (pure-torch OctCQT)
    measured the same way. The reference publishes 2.6 / 21.1 / 84.4 /
    337.5 MB at batches 1 / 8 / 32 / 128 (bench/figure.py:21-23)."""
    from flash_cqt.fused import FusedOctCQT
    f = FusedOctCQT(cqt_gpu, dev)
    out = {}
    for B in batches:
        x = randn(B, 2).to(dev)
        with torch.no_grad():
            ours = peak_mb(lambda: f.bwd(*f.fwd(x)))
            lib = peak_mb(lambda: cqt_gpu.bwd(*cqt_gpu.fwd(x)))
        out[str(B)] = {"peak_mb": ours, "peak_mb_per_slice": ours / B, "hipfft_baseline_peak_mb": lib}
        f.release_workspace()
    table_mb = sum(f.table_bytes.values()) / 1e6
    log("peak MB per round-trip call: " + "  ".join(f"B={b}: {v['peak_mb']:.1f} (hipFFT {v['hipfft_baseline_peak_mb']:.1f})"
                                                    for b, v in out.items()) + f"; tables resident {table_mb:.1f} MB")
    return {"per_batch": out, "tables_resident_mb": table_mb,
            "method": "torch.cuda.max_memory_allocated minus the allocation before one round-trip call whose "
                      "buffers are all allocated inside it (fresh engine per batch size, tables resident)"}


# ---------------------------------------------------------- kernel timings

def kernel_timings(f, B, reps):
    """Average duration per launch of each engine call at batch B: hipEvents
    on the launch stream around `reps` back-to-back stream launches (median
    of 7 such runs). One untimed call goes first, so the GPU is busy while
    the timed launches are enqueued (each takes far less host time than GPU
    time at B = 64). The same calls as graphs of `reps` launches are reported
    beside it (`ms_per_call_graph`): graph replay adds a fixed cost per
    replay and per node on this runtime."""
    from flash_cqt import _native
    dev = f.dev
    w = f._workspace(B)
    x = randn(B, 1).to(dev)
    kr, ki = w["KR"], w["KI"]          # the engine's own coefficient planes (their placement matters)
    y = torch.empty(B, N, device=dev)
    # each call once through the checked wrappers (buffer sizes, devices),
    # then the same C-ABI calls with cached pointers, so that enqueueing a
    # launch costs the host a few microseconds only
    f.packed_fft(x, w["X"], w["W"])
    f.route_bands(w["X"], kr, ki, _native.PLANAR)
    f.scatter_bands(kr, ki, _native.PLANAR, w["F"])
    f.packed_ifft(w["F"], y, w["W"])
    lib, ct, sh = f.lib, f._ct, _native.stream_handle(dev.index)
    px, pX, pW, pF, py = x.data_ptr(), w["X"].data_ptr(), w["W"].data_ptr(), w["F"].data_ptr(), y.data_ptr()
    pr, pi = kr.data_ptr(), ki.data_ptr()
    t_route, t_scat, t_ovf = f._tp["route"], f._tp["scat"], f._tp["ovf_scat"]
    calls = {
        "packed_fft": lambda: lib.fcqt_packed_fft_fwd(ct, px, pX, pW, B, sh),
        "route_bands": lambda: lib.fcqt_route_bands(ct, t_route, pX, pr, pi, _native.PLANAR, B, sh),
        "scatter_bands": lambda: lib.fcqt_scatter_bands(ct, t_scat, pr, pi, _native.PLANAR, pF, B, sh),
        "packed_ifft": lambda: lib.fcqt_packed_fft_inv(ct, t_ovf, pF, py, pW, B, sh),
    }
    for name, fn in calls.items():
        _native.check(fn(), name)
    # the checked wrappers again for the graph timing: they launch on the
    # current stream, which capture switches
    wrapped = {
        "packed_fft": lambda: f.packed_fft(x, w["X"], w["W"]),
        "route_bands": lambda: f.route_bands(w["X"], kr, ki, _native.PLANAR),
        "scatter_bands": lambda: f.scatter_bands(kr, ki, _native.PLANAR, w["F"]),
        "packed_ifft": lambda: f.packed_ifft(w["F"], y, w["W"]),
    }
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    out = {}
    for name, fn in calls.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ts = []
        bad = 0
        for _ in range(7):
            bad |= fn()
            a.record()
            for _ in range(reps):
                bad |= fn()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b) / reps)
        _native.check(bad, name)
        ts.sort()
        ms = ts[len(ts) // 2]

        def many(fn=wrapped[name]):
            for _ in range(reps):
                fn()
        g, _ = capture(many)
        ms_graph = median_ms(g.replay, reps=10, warm=2) / reps
        per = ms / KERNEL_LAUNCHES[name]
        alg = KERNEL_BYTES[name] * B
        out[name] = {"ms_per_call": ms, "launches": KERNEL_LAUNCHES[name],
                     "ms_per_launch": per, "alg_bytes_per_call": alg,
                     "gbps": alg / (ms * 1e-3) / 1e9, "ms_per_call_graph": ms_graph}
    torch.cuda.synchronize()
    return out


# kernel names in the profiles (the pass kernels in their wide tile shapes
# and the band kernels with write-through stores, which batch 64 runs)
KERNEL_SYMBOL = {"packed_fft": ("k_col_fwd<false,16>", "k_row_fwd<16>"), "route_bands": ("k_route_bands<0,true,true>",),
                 "scatter_bands": ("k_scatter_bands<0,true,true>",), "packed_ifft": ("k_col_inv<32,true>", "k_row_inv<16,true>")}


def measured_traffic(name, B):
    """HBM bytes per launch of a kernel from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE, copy-calibrated), or None."""
    path = ROOT / "profiles" / "hbm_traffic_b64.txt"
    if B != 64 or not path.exists():
        return None
    got = {}
    for ln in path.read_text().splitlines():
        if ln.startswith("TRAFFIC "):
            parts = ln.split()
            got[parts[1]] = float(parts[3].split("=")[1])
    syms = KERNEL_SYMBOL[name]
    if not all(s in got for s in syms):
        return None
    return sum(got[s] for s in syms) / len(syms)


def kernels_only(f, B, reps, band_tasks=None):
    """A few launches of each kernel and one plain copy of known size, for
    rocprofv3 --pmc runs (FETCH_SIZE / WRITE_SIZE calibration). With
    band_tasks = K only the two band kernels run, on the first K tasks."""
    from flash_cqt import _native
    dev = f.dev
    w = f._workspace(B)
    x = randn(B, 1).to(dev)
    kr, ki = w["KR"], w["KI"]          # the engine's own coefficient planes (their placement matters)
    y = torch.empty(B, N, device=dev)
    if band_tasks:
        t, k = leading_tasks(f, ntasks=band_tasks)
        sh = _native.stream_handle(dev.index)
        f.packed_fft(x, w["X"], w["W"])
        for _ in range(reps):
            _native.check(f.lib.fcqt_route_bands(t, f._tp["route"], w["X"].data_ptr(), kr.data_ptr(), ki.data_ptr(),
                                                 _native.PLANAR, B, sh), "route_bands")
            _native.check(f.lib.fcqt_scatter_bands(t, f._tp["scat"], kr.data_ptr(), ki.data_ptr(), _native.PLANAR,
                                                   w["F"].data_ptr(), B, sh), "scatter_bands")
        torch.cuda.synchronize()
        log(f"kernels-only: B={B} reps={reps}; band kernels on the first {k} tasks")
        return
    src = torch.ones(16 * 1024 * 1024, device=dev)      # 64 MiB
    dst = torch.empty_like(src)
    for _ in range(reps):
        f.packed_fft(x, w["X"], w["W"])
        f.route_bands(w["X"], kr, ki, _native.PLANAR)
        f.scatter_bands(kr, ki, _native.PLANAR, w["F"])
        f.packed_ifft(w["F"], y, w["W"])
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"kernels-only: B={B} reps={reps}; copy kernel moves 64 MiB read + 64 MiB write per launch")


def leading_tasks(f, max_m=None, ntasks=None):
    """A copy of the engine's table descriptor whose task table is cut to its
    first tasks: the first `ntasks`, or the leading tasks of band length
    <= max_m. Returns (descriptor, task count)."""
    import ctypes
    from flash_cqt import _native
    if ntasks is None:
        ms = f.tables["tasks"][:, 0].cpu().tolist()
        ntasks = 0
        while ntasks < len(ms) and ms[ntasks] <= max_m:
            ntasks += 1
    t = _native.Tables()
    ctypes.memmove(ctypes.addressof(t), ctypes.addressof(f._ct), ctypes.sizeof(t))
    t.ntasks = ntasks
    return t, ntasks


def band_exchange(f, batches=(16, 64), reps=20):
    """The two stage exchanges of the small band units (M <= 256): the
    library's LDS exchange against the cross-lane (DPP) exchange of the
    variant library libflashcqt_xlane.so. Both band kernels run on the
    leading tasks of M <= 256 only (the tasks the variant changes), on the
    same buffers, hipEvents around `reps` back-to-back launches (median of 7,
    the two libraries alternating), and their coefficients and slot buffers
    are compared bit for bit."""
    from flash_cqt import _native
    dev = f.dev
    libs = {"lds": f.lib, "cross_lane": _native.load_variant("xlane")}
    t, k = leading_tasks(f, max_m=256)
    sh = _native.stream_handle(dev.index)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    out = {"tasks": k, "band_lengths": sorted(set(f.tables["tasks"][:k, 0].cpu().tolist())),
           "duration_source": f"hipEvents around {reps} back-to-back launches, median of 7"}
    for B in batches:
        w = f._workspace(B)
        x = randn(B, 2).to(dev)
        f.packed_fft(x, w["X"], w["W"])
        kr, ki, F = w["KR"], w["KI"], w["F"]
        res, bits = {}, {}
        for name, lib in libs.items():
            calls = {
                "route": lambda lib=lib: lib.fcqt_route_bands(t, f._tp["route"], w["X"].data_ptr(), kr.data_ptr(),
                                                              ki.data_ptr(), _native.PLANAR, B, sh),
                "scatter": lambda lib=lib: lib.fcqt_scatter_bands(t, f._tp["scat"], kr.data_ptr(), ki.data_ptr(),
                                                                  _native.PLANAR, F.data_ptr(), B, sh),
            }
            for cn, fn in calls.items():
                _native.check(fn(), cn)
            torch.cuda.synchronize()
            bits[name] = (kr.clone(), ki.clone(), F.clone())
            for cn, fn in calls.items():
                ts = []
                for _ in range(7):
                    fn()
                    a.record()
                    for _ in range(reps):
                        fn()
                    b.record()
                    b.synchronize()
                    ts.append(a.elapsed_time(b) / reps * 1e3)
                ts.sort()
                res[f"{cn}_{name}_us"] = ts[3]
        res["bitwise_equal"] = all(torch.equal(p, q) for p, q in zip(bits["lds"], bits["cross_lane"]))
        out[str(B)] = res
        log(f"band exchange B={B} ({k} tasks, M <= 256): " + ", ".join(
            f"{key} {val:.2f}" for key, val in res.items() if key.endswith("_us"))
            + f", bitwise equal {res['bitwise_equal']}")
    return out


# ------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-lib-baseline", action="store_true")
    ap.add_argument("--kernels-only", action="store_true")
    ap.add_argument("--sliced-only", action="store_true")
    ap.add_argument("--sliced-long-only", action="store_true")
    ap.add_argument("--no-single-launch", action="store_true",
                    help="skip the single-launch directions (one launch of persistent workgroups each)")
    ap.add_argument("--single-launch-only", action="store_true",
                    help="time only the single-launch directions and the per-launch floor; print their JSON")
    ap.add_argument("--single-launch-trace", action="store_true",
                    help="the single-launch directions' per-stage timeline (trace build of the library) at batches "
                         "1, 16, 64; print its JSON")
    ap.add_argument("--band-tasks", type=int, default=None,
                    help="with --kernels-only: run only the band kernels, on the first K tasks")
    ap.add_argument("--lib-variant", choices=("xlane",), default=None,
                    help="with --kernels-only: launch from a variant library (xlane: cross-lane exchange of the "
                         "band units of M <= 256)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the engine is single-GPU (batch sharding across "
              "GPUs needs no communication and is not exercised here); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    from flash_cqt import OctCQT
    from flash_cqt.fused import FusedOctCQT

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.sliced_only:
        print(json.dumps(json_safe(sliced_workload(dev))), flush=True)
        return
    if args.sliced_long_only:
        print(json.dumps(json_safe(sliced_long(dev))), flush=True)
        return
    if args.single_launch_trace:
        print(json.dumps(json_safe(single_launch_trace(dev))), flush=True)
        return
    cqt_gpu = OctCQT([3, 4, 2], [8, 16, 32], fs=FS, audio_len=N, device=dev)
    f = FusedOctCQT(cqt_gpu, dev)
    if args.single_launch_only:
        print(json.dumps(json_safe(single_launch_workload(f, dev))), flush=True)
        return
    if args.kernels_only:
        if args.lib_variant:
            from flash_cqt import _native
            f.lib = _native.load_variant(args.lib_variant)
        kernels_only(f, args.batch, max(1, args.kernel_reps // 4), args.band_tasks)
        return

    batches = sorted({1, 16, 64, args.batch})
    per_batch = {}
    graphs = {}
    for B in batches:
        x = (torch.from_numpy(sinusoids()) if B == 1 else randn(B, 0)).to(dev)
        w = f._workspace(B)
        fn = lambda x=x: f.bwd(*f.fwd(x))
        with torch.no_grad():
            eager = fn().clone()
            g, out = capture(fn)
            rep_db = replay_matches_eager(g, out, eager, [w["KR"], w["KI"], w["X"], w["W"], w["XO"]])
            rt_rows = min(snr_db(x[b], eager[b]) for b in range(B))
            KR, KI = f.fwd(x)
            ours = torch.complex(KR, KI).clone()
            tb, ts = cqt_gpu.fwd(x)
            ref = torch.cat([c.reshape(B, -1) for c in list(tb) + list(ts)], -1)
            coef_db = snr_db(torch.view_as_real(ref), torch.view_as_real(ours))
        ms, mode, step, modes = best_mode(g.replay, fn)
        graphs[B] = (step, mode)
        per_batch[B] = {"ms": ms, "launch_mode": mode, "ms_by_launch_mode": modes,
                        "round_trips_per_s": B / (ms * 1e-3),
                        "hbm_gbps": B * SLICE_RT_BYTES / (ms * 1e-3) / 1e9,
                        "roundtrip_snr_db_min_row": rt_rows, "coef_snr_db_vs_torch_fft": coef_db,
                        "replay_vs_eager_db": rep_db,
                        "input": "configs[1] sinusoids+noise" if B == 1 else "randn N(0,1) seed 0"}
        if not args.no_single_launch:
            per_batch[B]["single_launch"] = single_launch(f, x, eager)
        if not args.no_lib_baseline:
            bms, bmode, bout = torch_fft_baseline(cqt_gpu, x)
            per_batch[B].update({"hipfft_baseline_ms": bms, "hipfft_baseline_mode": bmode,
                                 "speedup_vs_hipfft": bms / ms,
                                 "hipfft_baseline_roundtrip_snr_db": snr_db(x, bout)})
        log(f"B={B}: {ms:.4f} ms ({mode})  {per_batch[B]['round_trips_per_s']:.0f} rt/s  "
            f"{per_batch[B]['hbm_gbps']:.0f} GB/s  rt {rt_rows:.1f} dB  coef {coef_db:.1f} dB"
            + (f"  single-launch {per_batch[B]['single_launch']['ms']:.4f} ms"
               if "single_launch" in per_batch[B] else "")
            + (f"  hipFFT {per_batch[B]['hipfft_baseline_ms']:.4f} ms ({per_batch[B]['hipfft_baseline_mode']})"
               if not args.no_lib_baseline else ""))

    per_batch[1]["launch_floor"] = launch_floor(f, dev)

    # ---- the timed region: exactly K steps of the batch, in the faster launch mode
    B = args.batch
    step, launch_mode = graphs[B]
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    value = B / (ms_step * 1e-3)
    gbps = B * SLICE_RT_BYTES / (ms_step * 1e-3) / 1e9

    kern = kernel_timings(f, B, args.kernel_reps)
    # per-kernel rates at the other batch of configs[2] (16) too
    for b in (16,):
        if b in per_batch and b != B:
            per_batch[b]["kernels"] = kernel_timings(f, b, args.kernel_reps)
    single = {k: v for k, v in kern.items() if v["launches"] == 1}
    dom = max(single, key=lambda k: single[k]["ms_per_launch"])
    ach = kern[dom]["gbps"]
    traffic = measured_traffic(dom, B)
    roof = {"kernel": dom, "bound": "hbm", "achieved": ach, "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": ach / PEAK_GBPS, "traffic": traffic,
            "traffic_source": "profiles/hbm_traffic_b64.txt (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0)"
            if traffic else None,
            "alg_bytes_per_launch": kern[dom]["alg_bytes_per_call"],
            "ms_per_launch": kern[dom]["ms_per_launch"], "batch": B,
            "duration_source": f"hipEvents on the launch stream around {args.kernel_reps} back-to-back stream "
                               "launches, median of 7 runs",
            "ms_per_launch_graph": kern[dom]["ms_per_call_graph"] / kern[dom]["launches"]}

    # the whole round trip against the same peak: algorithmic bytes of the
    # timed step over its duration, and the HBM traffic the six kernels
    # move per round trip (committed counter summary, batch 64)
    rt_traffic = None
    if B == 64:
        parts = [measured_traffic(k, B) for k in KERNEL_SYMBOL]
        if all(t is not None for t in parts):
            rt_traffic = sum(t * KERNEL_LAUNCHES[k] for t, k in zip(parts, KERNEL_SYMBOL))
    roof_rt = {"bound": "hbm", "achieved": gbps, "peak": PEAK_GBPS, "unit": "GB/s", "frac": gbps / PEAK_GBPS,
               "traffic": rt_traffic, "alg_bytes_per_step": B * SLICE_RT_BYTES, "ms_per_step": ms_step,
               "traffic_source": "sum over the six kernels in profiles/hbm_traffic_b64.txt" if rt_traffic else None}

    sliced = sliced_workload(dev)
    sliced["long_signal"] = sliced_long(dev)
    exchange = band_exchange(f)
    train = training_step(dev, cqt_gpu)
    mem = peak_memory(cqt_gpu, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline(batch=B)

    line = {
        "metric": METRIC, "value": value, "unit": "slice round trips/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"fused fp32 CQT round trip (analysis+synthesis), batch {B} "
                               f"(configs[2]; batch 1 = configs[1] in per_batch), {launch_mode}",
                   "launch_mode": launch_mode,
                   "batch": B, "slice_len": N,
                   "layout": "OctCQT([3,4,2],[8,16,32],fs=44100), 154 bands, 132992 coefficients",
                   "parallelism": "single GPU"},
        "hbm_gbps": gbps, "hbm_frac": gbps / PEAK_GBPS, "wall_s_timed": wall,
        "per_batch": {str(k): v for k, v in per_batch.items()},
        "kernels": kern,
        "sliced": sliced,
        "band_exchange": exchange,
        "training_step": train,
        "table_bytes": f.table_bytes,
        "roofline": roof,
        "roofline_roundtrip": roof_rt,
        "peak_memory": mem,
        "cpu_baseline": cpu,
    }
    print(json.dumps(json_safe(line)), flush=True)


if __name__ == "__main__":
    main()
