/* flashcqt.h -- C ABI of the MI355X (gfx950) fused factored CQT engine.
 *
 * The library (libflashcqt.so, built with hipcc) implements the hot path of
 * the factored constant-Q transform for 65536-sample slices:
 *   analysis   x -> real FFT (packed half-length FFT + untangle) -> windowed
 *              band gathers + band inverse DFTs -> C
 *   synthesis  C -> band DFTs + gain + scatter -> packed inverse FFT -> y
 * and both adjoints by running the same kernels with different tables.
 *
 * Conventions
 *   - Every buffer is device memory allocated by the caller; the library
 *     never allocates or frees (fcqt_analysis_static keeps its workspace in
 *     a static device array of the library instead). Tables are built on
 *     the host (the Python package flash_cqt/tables.py) and uploaded by the
 *     caller (fcqt_tables_upload).
 *   - Complex buffers are interleaved fp32 pairs (re, im), 8-byte aligned.
 *     Record tables (int32 quadruples) must be 16-byte aligned.
 *   - All work is enqueued asynchronously on `stream` (any HIP stream,
 *     including one under hipGraph capture); no call allocates or issues
 *     hipMemset, so every call can be captured into a graph. The one call
 *     that synchronises is the set-up call fcqt_tables_upload.
 *   - Return value: FCQT_OK (0), or an FCQT_E* code. Argument errors are
 *     detected before any HIP call is made.
 *   - Calls that share a workspace must be ordered on one stream.
 *   - Results are deterministic: no result is accumulated with atomics
 *     (every output value has one writer). Atomics appear only as counters
 *     (the single-launch kernels' queues and stage counts) and as
 *     write-through stores of final values. Results are also independent of
 *     the batch size: a slice gives the same bits alone or in any batch
 *     (the launchers pick the FFT passes' tile shape by batch size; every
 *     shape does the same arithmetic per slice).
 *
 * Fixed geometry (the reference's fused path hard-requires it,
 * fused.py:230): N = 65536 real samples per slice, L = N/2 = 32768.
 */
#ifndef FLASHCQT_H
#define FLASHCQT_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FCQT_ABI_VERSION 13

#define FCQT_N 65536          /* real samples per slice */
#define FCQT_L 32768          /* packed complex length */
#define FCQT_FSTRIDE 32832    /* complex elements per half-spectrum plane (>= L+1) */
#define FCQT_OVF_CAP 4096     /* overflow bins (more than two taps) per scatter table */
#define FCQT_FROW 73856       /* complex elements per batch row of F: 2 slot planes of FCQT_FSTRIDE + 2 x FCQT_OVF_CAP */
#define FCQT_OVF_LEN 4096     /* int32 entries of a scatter table's overflow fold lists [8][512] */
#define FCQT_XSTRIDE 32832    /* complex elements per batch row of the real-FFT spectrum X (>= L+1) */
#define FCQT_TW_STAGE_LEN 4064 /* complex elements of the stage twiddle table */
#define FCQT_TW_PASS_LEN 32768 /* complex elements of the pass twiddle table [128][256] */
#define FCQT_TW_HALF_LEN 32768 /* complex elements of the retangle twiddle table W_65536^i */

/* status codes */
#define FCQT_OK 0
#define FCQT_EARG 1      /* null pointer, bad size or bad enum */
#define FCQT_EALIGN 2    /* pointer misaligned for its element type */
#define FCQT_ELAUNCH 3   /* kernel launch failed (HIP error) */
#define FCQT_ECAPACITY 4 /* batch beyond the static scratch capacity of fcqt_analysis_static */

/* coefficient layouts */
#define FCQT_PLANAR 0       /* re and im in two [batch][ncoef] fp32 planes */
#define FCQT_INTERLEAVED 1  /* one [batch][ncoef] complex buffer, pass it as re, im ignored */

/* Host-side descriptor of the uploaded, batch-invariant tables. */
typedef struct fcqt_tables {
    const float*   tw_pass;   /* [128][256] complex, W_32768^(k1*n2) at k1*256+n2 */
    const float*   tw_half;   /* [32768] complex, W_65536^i */
    const float*   tw_stage;  /* [FCQT_TW_STAGE_LEN] complex band/pass stage twiddles */
    const int32_t* tasks;     /* [ntasks][4] band tasks: M, first coefficient, band count, first band */
    int32_t        ntasks;
    int64_t        ncoef;     /* complex coefficients per slice (132992 for [3,4,2]/[8,16,32]) */
    int64_t        coef_span; /* one past the last coefficient any task touches (the task table's
                                 coverage, max of first + count * M); every band launch is refused
                                 with FCQT_EARG unless 1 <= coef_span <= ncoef, and a task whose
                                 coefficients reach past ncoef is skipped by the kernels */
} fcqt_tables;

/* ---- table image, upload and buffer sizes ----
 * The batch-invariant tables come from the host builder
 * (flash-cqt_amd/flash_cqt/tables.py: build() computes them in float64 from
 * the OctCQT bank, image_bytes()/save_image() write them as one flat image);
 * the library does not compute tables. A C or C++ caller loads an image
 * file once, checks it, uploads it and sizes its buffers with the three
 * calls below; no Python is needed at run time. */

#define FCQT_IMAGE_VERSION 1  /* table image format understood by this library */

/* What a checked image holds. */
typedef struct fcqt_image_info {
    int64_t device_bytes;   /* device bytes fcqt_tables_upload needs (the image length) */
    int64_t ncoef;          /* complex coefficients per slice */
    int64_t coef_span;      /* the task table's coverage (== ncoef for a consistent image) */
    int32_t ntasks;         /* band tasks */
    int32_t format;         /* image format version */
} fcqt_image_info;

/* Descriptors of an uploaded image: every table the entry points take. */
typedef struct fcqt_engine_tables {
    fcqt_tables    tab;           /* twiddles, tasks, ncoef, coef_span */
    const int32_t* route;         /* analysis route records */
    const int32_t* route_b;       /* synthesis-adjoint route records */
    const int32_t* scat;          /* synthesis scatter records */
    const int32_t* scat_a;        /* analysis-adjoint scatter records */
    const int32_t* ovf_scat;      /* fold lists of scat */
    const int32_t* ovf_scat_a;    /* fold lists of scat_a */
    const int32_t* slice_groups;  /* SlicedCQT group records */
} fcqt_engine_tables;

/* Check a table image held in host memory, without any HIP call: the
 * header and section table (ids, element sizes, counts, 256-byte aligned
 * offsets inside the image), and every table against the bounds the kernels
 * index with: band lengths and counts of the tasks, their coefficient
 * coverage against ncoef, route bins <= 32768, scatter slots inside an F row
 * and their gain modes, fold-list bins and overflow indices, slice-group
 * records against their tasks. Fills *info (may be NULL) on success.
 * Returns FCQT_OK or FCQT_EARG. No counterpart in the reference, whose
 * tables are device tensors built in Python (fused.py:229-476). */
int fcqt_image_check(const void* image, int64_t len, fcqt_image_info* info);

/* Check the image (as fcqt_image_check), copy it into `dev`, caller-owned
 * device memory of at least info.device_bytes bytes, 256-byte aligned, and
 * fill *out with device pointers into it. The copy is enqueued on `stream`
 * and waited for (hipStreamSynchronize), so the image may be freed on
 * return: a set-up call, not for graph capture. Allocates nothing. */
int fcqt_tables_upload(const void* image, int64_t len, void* dev, int64_t dev_bytes, hipStream_t stream,
                       fcqt_engine_tables* out);

/* Bytes of every caller-allocated buffer at a batch size. */
typedef struct fcqt_sizes {
    int64_t signal;      /* x or y: batch * 65536 fp32 */
    int64_t spectrum;    /* xs: batch * FCQT_XSTRIDE complex */
    int64_t work;        /* work: batch * 32768 complex */
    int64_t scatter;     /* f, one per scatter table: batch * FCQT_FROW complex */
    int64_t coef_plane;  /* one FCQT_PLANAR plane: batch * ncoef fp32 (FCQT_INTERLEAVED: twice this) */
    int64_t tail;        /* fcqt_stream_overlap tail: batch (signals) * 32768 fp32 */
    int64_t sync;        /* single-launch counters: FCQT_SYNC_WORDS(batch) uint32 */
} fcqt_sizes;

/* Fill *out for `batch` slices (tab supplies ncoef). FCQT_EARG on a bad
 * argument or a size that overflows. No counterpart in the reference (its
 * callers size buffers from Python constants, trainable.py:75-110). */
int fcqt_workspace_sizes(const fcqt_tables* tab, int64_t batch, fcqt_sizes* out);

/* ABI version of the loaded library (FCQT_ABI_VERSION). */
int fcqt_abi_version(void);

/* Static text for a status code. */
const char* fcqt_status_string(int status);

/* Text of the last HIP error seen by a launcher on this thread ("" if none). */
const char* fcqt_last_hip_error(void);

/* Real FFT of 65536-sample slices as a packed half-length FFT:
 *   x    [batch][65536] fp32 (8-byte aligned)
 *   xs   [batch][FCQT_XSTRIDE] complex, out: X = rfft(x), bins 0..32768
 *   work [batch][32768] complex scratch
 * Z = FFT_32768(x[0::2] + i x[1::2]) is untangled on the way out,
 * X[k] = cA(k) Z[k] + cB(k) conj Z[L-k]. Replaces the even/odd pack copies
 * (trainable.py:81-82) and fft3 (packedfft.cu:100-126) plus the untangle
 * the reference does per tap (radix_impl.cuh:27-42); two launches. */
int fcqt_packed_fft_fwd(const fcqt_tables* tab, const float* x, float* xs, float* work,
                        int64_t batch, hipStream_t stream);

/* Band tables are in kernel order: for each task, 16 rows of 128 8-byte
 * records (row s = slot s of each of the task's 128 threads), so a table has
 * ntasks * 2048 records. Thread u T + t (T = M/16) works on unit u of the
 * task (band u, units past the task's band count are padding with zero
 * records); its input slot r is tap t + T r of that band, its output slot
 * q RL + r is transform output t + T q + r OS (RL, OS: the last radix and
 * its output stride). The host builder (flash_cqt/tables.py, kernel_taps)
 * makes these tables from per-tap ones.
 *
 * Windowed band gathers + band inverse DFTs: coefficient m of band b is
 *   C_b[m] = sum_j w_j X~[k_j] e^{+2 pi i jm/M_b}
 * where X~ is X, or its conjugate for taps past N/2 (folded to N - k). One
 * record per tap {k, fp32 weight bits}: window/M gives the analysis, dual
 * window * 2/N (halved at bins 0 and L) the synthesis adjoint; taps outside
 * the window have weight 0. The weights are >= 0, and a tap that reads the
 * conjugate stores its weight negated: the kernel forms (|w| Re X, w Im X).
 *   xs      [batch][FCQT_XSTRIDE] complex real-FFT spectrum (fcqt_packed_fft_fwd)
 *   coef    layout FCQT_PLANAR: coef_re, coef_im [batch][ncoef] fp32
 *           layout FCQT_INTERLEAVED: coef_re is [batch][ncoef] complex, coef_im unused
 *   route   [ntasks * 2048][2] int32 route records, kernel order
 * Replaces fwd_bands (radix.cu:46-62). */
int fcqt_route_bands(const fcqt_tables* tab, const int32_t* route, const float* xs,
                     float* coef_re, float* coef_im, int layout,
                     int64_t batch, hipStream_t stream);

/* Band DFTs + per-tap gain + scatter into the half spectrum F:
 *   D_b = DFT_{M_b}(C_b);  slot(j) of F <- (gr_j Re D_b[j], gi_j Im D_b[j])
 * with one 8-byte record {slot | mode << 30, gr} per tap: gi = gr (mode 0),
 * -gr (mode 1) or 0 (mode 2); gr = 0 skips a tap.
 * F holds, per batch row, two dense slot planes of FCQT_FSTRIDE bins
 * (F[bin], F[FCQT_FSTRIDE + bin]) and an overflow area of 2 x FCQT_OVF_CAP
 * slots; a bin's value is the sum of its slots. The
 * table gives every live tap its own slot (no atomics: results are bitwise
 * reproducible), and the set of slots it writes is fixed, so
 *   - f must be zero-filled once when allocated (fcqt_fill_zero),
 *   - a given F buffer must only ever be used with one scatter table.
 * With the synthesis table this is the synthesis front half; with the
 * analysis-adjoint table it is the analysis adjoint front half.
 *   f  [batch][FCQT_FROW] complex, 16-byte aligned
 * Replaces inv_bands (radix.cu:64-91) and adj_bands (radix.cu:93-114). */
int fcqt_scatter_bands(const fcqt_tables* tab, const int32_t* scat /* [ntasks * 2048][2], kernel order */,
                       const float* coef_re, const float* coef_im, int layout,
                       float* f, int64_t batch, hipStream_t stream);

/* Packed inverse real FFT: y = irfft_65536(F[0..32768]) where each bin of F
 * is the sum of its scatter slots (imaginary parts of bins 0 and 32768
 * ignored, as irfft does). F is read only.
 *   ovf  [FCQT_OVF_LEN] int32 overflow fold lists of the scatter table that
 *        filled F: for each of the 8 column workgroups, up to 512 entries
 *        bin | overflow index << 16 (-1 = none)
 *   f    [batch][FCQT_FROW] complex
 *   y    [batch][65536] fp32 out (8-byte aligned)
 *   work [batch][32768] complex scratch
 * Replaces inv_tail (packedfft.cu:233-254); the F memsets of the reference
 * (trainable.py:104-105) are not needed. */
int fcqt_packed_fft_inv(const fcqt_tables* tab, const int32_t* ovf, const float* f, float* y,
                        float* work, int64_t batch, hipStream_t stream);

/* Analysis in one call: fcqt_packed_fft_fwd then fcqt_route_bands.
 * xs is [batch][FCQT_XSTRIDE] and work [batch][32768] complex scratch. From
 * 256 slices on the call runs the three kernels chunk by chunk, 128 slices
 * at a time, so that each chunk's intermediates are still in the
 * memory-side cache when read; the results are the same bits. */
int fcqt_analysis(const fcqt_tables* tab, const int32_t* route, const float* x,
                  float* coef_re, float* coef_im, int layout,
                  float* xs, float* work, int64_t batch, hipStream_t stream);

/* Single-launch directions: the same transforms as fcqt_analysis and
 * fcqt_synthesis (same buffers and rules, same results bit for bit), each
 * as ONE ordinary launch of persistent workgroups. A direction has three
 * stages per slice (analysis: column tiles, row tiles, band tasks;
 * synthesis: band tasks, inverse column tiles, inverse row tiles). The
 * slices are split over one queue per XCD (slice b to queue b mod 8), and
 * the workgroups running on XCD x (as the hardware reports it) take queue
 * x's tasks one at a time, in an order that interleaves the slices' stages
 * with lags (fcqt_persist_tune); a stage-2 or stage-3 task waits, through
 * counters in `sync`, for its slice's previous stage. No grid-wide barrier;
 * every wait is for a task taken earlier, so every wait ends.
 *   sync  uint32 [FCQT_SYNC_WORDS(batch)] (fcqt_sizes.sync bytes), 16-byte
 *         aligned, zero-filled once when allocated (fcqt_fill_zero); a call
 *         that succeeds leaves every word at zero again. Word
 *         batch * FCQT_SYNC_PER_SLICE is an error word: nonzero after a call
 *         means the results are not valid (bit 1: a stage wait outlasted its
 *         bound, about two seconds; bit 4: a queue that had tasks was served
 *         by no workgroup, i.e. no workgroup ran on that XCD, as on a chip
 *         partitioned into fewer XCDs per device). After a nonzero word the
 *         counters are left as they were: the caller synchronises and
 *         zero-fills the whole buffer before the next call.
 *         One sync buffer per stream: calls that overlap on one buffer race.
 * Capturable into a hipGraph like every other entry point (check the error
 * word after replay). Replace the reference's fwd2 / inv2
 * (persist2.cu:140-222, reached through FusedOctCQT.persist_fwd /
 * persist_inv, fused.py:748-778). */
#define FCQT_SYNC_PER_SLICE 64
#define FCQT_SYNC_HEAD_WORDS 320
#define FCQT_SYNC_WORDS(batch) ((int64_t)(batch) * FCQT_SYNC_PER_SLICE + FCQT_SYNC_HEAD_WORDS)
int fcqt_persist_analysis(const fcqt_tables* tab, const int32_t* route, const float* x,
                          float* coef_re, float* coef_im, int layout,
                          float* xs, float* work, uint32_t* sync, int64_t batch, hipStream_t stream);
int fcqt_persist_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* ovf,
                           const float* coef_re, const float* coef_im, int layout,
                           float* f, float* work, float* y, uint32_t* sync, int64_t batch, hipStream_t stream);

/* Process-wide settings of the single-launch kernels, read at each launch
 * (not for use while another host thread launches them). direction 0: the
 * analysis, 1: the synthesis. d1 / d2: the lags, in steps of one slice, of
 * a slice's stage 2 and stage 3 behind its stage 1 in each queue's order
 * (0 <= d1 <= d2 <= 64); wait_ticks: the bound of every stage wait in
 * ticks of the 100 MHz clock (default 200000000, two seconds; a negative
 * value leaves it unchanged). The results do not depend on any of them. No
 * counterpart in the reference (its persistent kernels use grid-stride
 * loops with grid-wide barriers). */
int fcqt_persist_tune(int direction, int d1, int d2, int64_t wait_ticks);

/* Stage trace of the single-launch kernels, in the trace build of the
 * library only (libflashcqt_flowtrace.so, the same sources built with
 * FCQT_FLOW_TRACE; the library itself returns FCQT_EARG and records
 * nothing). Every later single-launch call writes, per workgroup in
 * blockIdx order, FCQT_TRACE_TASKS records of FCQT_TRACE_FIELDS uint64 into
 * `buf` (device memory, zero-filled by the caller): record i of the first
 * FCQT_TRACE_TASKS - 1 is the workgroup's task i, {stage | slice << 8 |
 * tile << 40, 100 MHz clock before its claim or wait, when ready, body
 * done, counted in} (a zero first field ends the list); the last record is
 * {start, XCD, leave}. bytes >= 8 * 256 * FCQT_TRACE_TASKS *
 * FCQT_TRACE_FIELDS * 8 (the largest grid); buf = NULL stops recording.
 * No counterpart in the reference. */
#define FCQT_TRACE_TASKS 32
#define FCQT_TRACE_FIELDS 6
int fcqt_persist_trace(void* buf, int64_t bytes);

/* Allocation-free analysis: fcqt_analysis with the spectrum X and the work
 * buffer taken from a static device array of the library (each GPU holds its
 * own copy, FCQT_STATIC_MAX_BATCH slices = 8.4 MB, until the process ends),
 * so a caller passes only x and the coefficient buffers. It makes no HIP
 * allocation and calls no allocating routine. No counterpart in the
 * reference: it is for callers that cannot allocate (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * results as fcqt_analysis, bit for bit.
 *   batch <= FCQT_STATIC_MAX_BATCH, else FCQT_ECAPACITY (nothing launched)
 *   stream must belong to the current device (the default stream does)
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (unordered streams, other threads) race; order them on one stream. */
#define FCQT_STATIC_MAX_BATCH 16
int fcqt_analysis_static(const fcqt_tables* tab, const int32_t* route, const float* x,
                         float* coef_re, float* coef_im, int layout, int64_t batch, hipStream_t stream);

/* Synthesis in one call: fcqt_scatter_bands then fcqt_packed_fft_inv, with
 * the scatter table `scat` and its overflow map `ovf` (same F rules). */
int fcqt_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* ovf,
                   const float* coef_re, const float* coef_im, int layout,
                   float* f, float* work, float* y, int64_t batch, hipStream_t stream);

/* ---- SlicedCQT framing fused into the engine (same kernels, other I/O) ----
 * nsig signals, each cut into 65536-sample slices at hop N/2; one call
 * handles nslices consecutive slices g = first + s, s < nslices, of every
 * signal (batch row sig * nslices + s); H = N/4. A whole signal is one call
 * with first = 0; streaming (SlicedCQT.stream_fwd/stream_bwd) makes one call
 * per slice with first = the slice's index.
 *
 * Sliced real FFT: slice g of signal sig is x[2H (g - 1) + jj] * window[jj]
 * with jj = (j + H) mod N for even g and (j - H) mod N for odd g, where the
 * call holds the signal from sample `origin` on (x[i] = sig[sig][i - origin]
 * for 0 <= i - origin < sig_len, zero elsewhere): the zero padding,
 * 50%-overlap unfold, Tukey window and quarter roll, read straight from the
 * signal by the column pass. Whole signal: origin = 0; one streamed slice g
 * from a buffer holding its N samples: origin = 2H (g - 1).
 *   sig    [nsig][sig_len] fp32,  window [65536] fp32
 *   xs, work as for fcqt_packed_fft_fwd with batch nsig * nslices
 * Replaces SlicedCQT._slice (sliced.py:106-117) and the per-slice framing of
 * stream_fwd (sliced.py:178-184) + the pack copy and fft3. */
int fcqt_slice_fft_fwd(const fcqt_tables* tab, const float* sig, int64_t sig_len, const float* window,
                       int64_t nsig, int64_t nslices, int64_t first, int64_t origin, float* xs,
                       float* work, hipStream_t stream);

/* Route + band IDFTs storing straight into the SlicedCQT block layout
 * (interleaved complex, nsig * nslices * ncoef values): group g (first
 * coefficient off_g, bins_g bands of length M, per-task table `groups`
 * [ntasks][4] = {off_g, bins_g, roll, 0}) is the block [nsig][bins_g][nslices * M]
 * at nsig * nslices * off_g; in octave groups (roll = 1) band output m of an
 * even slice g goes to (m + M/4) mod M, of an odd slice to (m - M/4) mod M;
 * side groups are [nsig][nslices][1][M] blocks.
 * Replaces fwd_bands + SlicedCQT._arrange(fwd) and the block permute of
 * SlicedCQT.fwd (sliced.py:119-131, 134-146). */
int fcqt_route_bands_sliced(const fcqt_tables* tab, const int32_t* route, const int32_t* groups,
                            const float* xs, float* coef, int64_t nsig, int64_t nslices, int64_t first,
                            hipStream_t stream);

/* The whole-signal sliced analysis in one call: fcqt_slice_fft_fwd (first = 0,
 * origin = 0) then fcqt_route_bands_sliced (first = 0), same arguments and
 * the same block layout and bits. From 256 slices on it runs in chunks of
 * about 128 slices (a range of slices of every signal, or a range of
 * signals), each framed, transformed and routed before the next, so that a
 * chunk's intermediates are still in the memory-side cache when read (xs
 * and work then serve one chunk at a time, in their leading 128 rows).
 *   sig    [nsig][sig_len] fp32,  window [65536] fp32
 *   coef   nsig * nslices * ncoef complex (interleaved)
 *   xs, work as for fcqt_packed_fft_fwd with batch nsig * nslices below 256
 *          slices, and with batch 128 (FCQT_ANALYSIS_CHUNK) from 256 on:
 *          only the leading FCQT_SLICED_ANALYSIS_ROWS(nsig * nslices) rows
 *          are used, so buffers of that many rows suffice
 * Replaces SlicedCQT.fwd's _slice, fwd_bands, _arrange and block permute
 * (sliced.py:106-146) for a whole signal. */
#define FCQT_ANALYSIS_CHUNK 128
#define FCQT_ANALYSIS_CHUNK_MIN_BATCH 256
#define FCQT_SLICED_ANALYSIS_ROWS(batch) \
    ((batch) < FCQT_ANALYSIS_CHUNK_MIN_BATCH ? (int64_t)(batch) : (int64_t)FCQT_ANALYSIS_CHUNK)
int fcqt_sliced_analysis(const fcqt_tables* tab, const int32_t* route, const int32_t* groups,
                         const float* sig, int64_t sig_len, const float* window, int64_t nsig,
                         int64_t nslices, float* coef, float* xs, float* work, hipStream_t stream);

/* Band DFTs + slot scatter reading the same block layout (the inverse
 * arrange). F rules as fcqt_scatter_bands, batch nsig * nslices.
 * Replaces the block permute + SlicedCQT._arrange(bwd) of SlicedCQT.bwd and
 * inv_bands (sliced.py:148-157). */
int fcqt_scatter_bands_sliced(const fcqt_tables* tab, const int32_t* scat, const int32_t* groups,
                              const float* coef, float* f, int64_t nsig, int64_t nslices, int64_t first,
                              hipStream_t stream);

/* The whole-signal sliced synthesis in one call, with the overlap-add in the
 * inverse row pass: fcqt_scatter_bands_sliced (first = 0), the inverse column
 * pass, then the inverse row pass twice, over the even slices (storing into
 * out) and over the odd ones (adding to it), so no [nslices][65536] slice
 * buffer is written or read back. The same output bits as
 * fcqt_scatter_bands_sliced + fcqt_packed_fft_inv + fcqt_overlap_add.
 *   coef   nsig * nslices * ncoef complex, the block layout
 *   f      [nsig * nslices][FCQT_FROW] complex (F rules as fcqt_scatter_bands)
 *   work   [nsig * nslices][32768] complex scratch
 *   out    [nsig][length] fp32, length <= nslices * 32768
 * Replaces SlicedCQT.bwd (sliced.py:148-167) for whole signals. */
int fcqt_sliced_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* groups,
                          const int32_t* ovf, const float* coef, float* f, float* work, float* out,
                          int64_t nsig, int64_t nslices, int64_t length, hipStream_t stream);

/* Overlap-add of the inverse slices (y [nsig * nslices][65536], the output of
 * fcqt_packed_fft_inv): out[sig][p], p < length <= nslices * 2H, sums the
 * slices covering p + 2H after rolling even slices by +H and odd by -H.
 * Replaces the roll, overlap-add and trim of SlicedCQT.bwd (sliced.py:158-166). */
int fcqt_overlap_add(const float* y, float* out, int64_t nsig, int64_t nslices, int64_t length,
                     hipStream_t stream);

/* Streamed overlap-add of one inverse slice g per signal (y [nsig][65536],
 * the output of fcqt_packed_fft_inv for that slice): with the slice rolled
 * back (+H for even g, -H for odd g) into y_r, out[sig][p] = tail[sig][p] +
 * y_r[p] and then tail[sig][p] = y_r[2H + p], p < 2H. For g = 0 only tail is
 * written (out may be NULL). tail [nsig][2H] starts at zero and carries the
 * stream's state between calls.
 * Replaces the roll and half-slice overlap-add of SlicedCQT.stream_bwd
 * (sliced.py:194-209). */
int fcqt_stream_overlap(const float* y, float* tail, float* out, int64_t nsig, int64_t slice,
                        hipStream_t stream);

/* One streamed analysis step: slice `slice` of each of nsig signals, whose
 * 65536 samples are the row of prev (the previous hop of 32768 samples)
 * followed by the row of next (the new hop), framed (window, quarter roll)
 * and transformed as fcqt_slice_fft_fwd does with nslices = 1, first =
 * slice, origin = 32768 (slice - 1) on the concatenated buffer, then routed
 * into the sliced block layout as fcqt_route_bands_sliced with first = slice.
 * The caller passes zeros as prev for slice 0 and as next for the final
 * flush. No concatenated copy is made.
 *   prev, next  nsig rows of 32768 fp32 each, rows prev_stride / next_stride
 *               floats apart (>= 32768 when nsig > 1; a chunk that is a view
 *               into a longer signal is read in place)
 *   coef        nsig * ncoef complex (interleaved)
 *   xs, work    as for fcqt_packed_fft_fwd with batch nsig
 * Replaces the per-slice step of SlicedCQT.stream_fwd (sliced.py:171-192):
 * the concatenation of the carried half slice with the new chunk, _slice,
 * the pack copy, fft3, fwd_bands and _arrange. */
int fcqt_stream_analysis(const fcqt_tables* tab, const int32_t* route, const int32_t* groups,
                         const float* prev, int64_t prev_stride, const float* next, int64_t next_stride,
                         const float* window, int64_t nsig, int64_t slice, float* coef, float* xs,
                         float* work, hipStream_t stream);

/* One streamed synthesis step: fcqt_scatter_bands_sliced (one slice per
 * signal, first = slice), fcqt_packed_fft_inv and fcqt_stream_overlap in one
 * call, with every argument checked before the first launch. out may be NULL
 * for slice 0.
 * Replaces the per-slice step of SlicedCQT.stream_bwd (sliced.py:194-209):
 * _arrange, inv_bands, inv_tail, the roll and the half-slice overlap-add. */
int fcqt_stream_synthesis(const fcqt_tables* tab, const int32_t* scat, const int32_t* groups,
                          const int32_t* ovf, const float* coef, float* f, float* work, float* y,
                          float* tail, float* out, int64_t nsig, int64_t slice, hipStream_t stream);

/* Zero n floats with a fill kernel (graph-capture safe, no hipMemsetAsync). */
int fcqt_fill_zero(float* buf, int64_t n, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHCQT_H */
