// Tile bodies of the packed real-FFT passes (device code), shared by the
// pass kernels (packed_fft.hip) and the single-launch kernels (persist.hip).
// The mathematics and the tile shapes are described in packed_fft.hip.
#pragma once

#include "fcqt_fft.hpp"

namespace fcqt {

// Tile shapes of the four pass kernels. Each kernel comes in a wide shape
// (every tile row reads and writes whole 128-byte lines) and a narrow one
// with half the columns or rows per workgroup and twice the workgroups per
// slice. A small batch has few workgroups per pass (8-16 per slice), so its
// pass time is set by what each workgroup moves; the narrow shapes halve
// that. Large batches fill the chip either way and keep the wide shapes.
//   column pass:          CPW columns x 128 rows, 8 CPW threads
//   row passes:           RPW rows x 256 columns, 16 RPW threads
//   inverse column pass:  CPW/2 columns + their CPW/2 mirrors, 8 CPW threads
constexpr int kColsWide = 16, kColsNarrow = 8;
constexpr int kRowsWide = 16, kRowsNarrow = 8;
constexpr int kInvColsWide = 32, kInvColsNarrow = 16;
// batch sizes up to this one run the narrow shapes
constexpr int64_t kNarrowMaxBatch = 16;
// the fold lists are built for the wide inverse column workgroups
constexpr int kFoldLists = 256 / kInvColsWide;
// the wide inverse passes write through the L2 up to this batch size
constexpr int64_t kInvWriteThroughMaxBatch = 104;

// ------------------------------------------------------------ column pass

// F layout per batch row: two dense slot planes of FSTRIDE bins (plane r
// holds the rank-r tap of each bin), then 2 x OVF_CAP overflow slots. A
// bin's value is plane0 + plane1 (+ its two overflow slots if it has more
// than two contributing taps).
__device__ __forceinline__ float2 dense_bin(const float2* __restrict__ fb, int i) {
    return cadd(fb[i], fb[kFStride + i]);
}

// SlicedCQT framing read by the sliced column pass: batch row sig * S + s is
// slice g = first + s of signal sig, sample j = x[2H (g - 1) + jj] win[jj]
// with jj = (j + H) mod N in even slices g and (j - H) mod N in odd ones
// (H = N/4; samples outside the signal are zero). The call holds the signal
// from sample `origin` on: x[i] = sig[sig][i - origin] for
// 0 <= i - origin < len (a whole signal: first = origin = 0; one streamed
// slice g from a buffer holding exactly its N samples: first = g,
// origin = 2H (g - 1)). This is the zero padding, 50%-overlap unfold, Tukey
// window and quarter roll of the reference SlicedCQT._slice in one read.
struct SliceSrc {
    const float* sig;   // [nsig][stride]: samples [0, split) of each row
    const float* win;   // [N]
    long len;           // samples per row that the call holds
    int S;
    long first;         // index in the signal of the call's slice 0
    long origin;        // signal sample index of sample 0 of the call's rows
    int pairs;          // 1: every sample pair (jj even) is 8-byte aligned and wholly inside or
                        // wholly outside the signal and on one side of split (even len, origin,
                        // strides and split, 8-byte aligned buffers), so it is read with one 8-byte
                        // load (sliced_pair_vec)
    const float* sig2;  // [nsig][stride2]: samples [split, len) of each row (streamed slices:
                        // the previous chunk in sig, the new chunk in sig2); null: sig holds all
    long stride;        // floats between rows of sig
    long stride2;       // floats between rows of sig2
    long split;
};

// Row pointers of a sliced call: sample i of row sig is a[i] for i < split
// and b[i - split] from split on.
struct SliceRow {
    const float* a;
    const float* b;
    long split;
    __device__ __forceinline__ const float* at(long i) const { return i < split ? a + i : b + (i - split); }
};

constexpr int kQuarter = kN / 4;

__device__ __forceinline__ float2 sliced_pair(const SliceSrc& src, const SliceRow& xrow, long s0, int sh, int n) {
    const int jj = (2 * n + sh) & (kN - 1);       // even: the pair (jj, jj + 1) stays inside the slice
    const long i = s0 + jj;
    const long i0 = min(max(i, 0l), src.len - 1), i1 = min(max(i + 1, 0l), src.len - 1);
    const float a = *xrow.at(i0) * ((i >= 0 && i < src.len) ? 1.0f : 0.0f);
    const float c = *xrow.at(i1) * ((i + 1 >= 0 && i + 1 < src.len) ? 1.0f : 0.0f);
    // rounded products (the empty asm keeps them out of the first butterfly's
    // fused multiply-adds): bitwise the windowed slice the reference framing
    // builds before its transform
    float p0 = src.win[jj] * a, p1 = src.win[jj + 1] * c;
    asm volatile("" : "+v"(p0), "+v"(p1));
    return make_float2(p0, p1);
}

// The same pair with src.pairs set: i = s0 + jj is even and len is even, so the
// pair (i, i + 1) lies wholly inside [0, len) or wholly outside, and (split
// even) on one side of split; one 8-byte load at the clamped index (inside
// [0, len - 2], so in bounds) and one of the window pair, zeros outside the
// signal. Same products as sliced_pair.
__device__ __forceinline__ float2 sliced_pair_vec(const SliceSrc& src, const SliceRow& xrow, long s0, int sh,
                                                  int n) {
    const int jj = (2 * n + sh) & (kN - 1);
    const long i = s0 + jj;
    const bool in = i >= 0 && i <= src.len - 2;
    const float2 x = *reinterpret_cast<const float2*>(xrow.at(min(max(i, 0l), src.len - 2)));
    const float2 w = *reinterpret_cast<const float2*>(src.win + jj);
    float p0 = w.x * (in ? x.x : 0.0f), p1 = w.y * (in ? x.y : 0.0f);
    asm volatile("" : "+v"(p0), "+v"(p1));
    return make_float2(p0, p1);
}

// Each pass is a tile body over (slice b, tile index) working in LDS the
// caller provides (the kernels below and the single-launch kernels of
// persist.hip run the same bodies, so both give the same bits): CPW (or RPW)
// units, then the twiddle block. The inverse passes take WT, the store form:
// the wide shapes write through the L2 up to kInvWriteThroughMaxBatch slices
// (store_out<true>: the inverse pair ran 1.4 us faster at batch 64) and plainly
// above, where the round trip's working set outgrows the memory-side cache
// (round trips 119.4-119.8 against 120.6-121.1 us at B = 112, 142.9-143.1
// against 145.9 us at B = 128, 308.4-308.6 against 314.0 us at B = 256; 101
// against 98.2-98.7 us at B = 96). The forward passes and the narrow shapes
// use plain stores: a write-through W
// is no longer in the L2 when the row pass of the same slice reads it on
// the same XCD (its hit rate fell from 0.53 to 0.06, and the round trip
// was 0.4 us slower), and the forward row pass covers each 128-byte line of
// X in two 64-byte halves (write-through wrote 25% more bytes). Same values
// either way.
template <int CPW>
constexpr int col_lds() { return CPW * Plan<128>::US + tw2_len<128>(); }
template <int RPW>
constexpr int row_lds() { return RPW * Plan<256>::US + tw2_len<256>(); }

template <bool SLICED, int CPW>
__device__ __forceinline__ void col_fwd_tile(const int b, const int cg, const float2* __restrict__ in,
                                             float2* __restrict__ out, const float2* __restrict__ twp,
                                             const float2* __restrict__ tws, const SliceSrc& src, float2* lds,
                                             const int tid = threadIdx.x) {
    using P = Plan<128>;
    float2* tw2 = lds + CPW * P::US;
    const int c = tid & (CPW - 1);                // column within the tile
    const int t = tid / CPW;                      // thread within the column FFT, < 8
    const int n2 = cg * CPW + c;
    float2 v[16];
    if constexpr (SLICED) {
        const int sig = b / src.S;
        const int sl = b - sig * src.S;
        const SliceRow xrow{src.sig + (long)sig * src.stride,
                            src.sig2 ? src.sig2 + (long)sig * src.stride2 : src.sig + (long)sig * src.stride + src.split,
                            src.split};
        const long g = src.first + sl;
        const long s0 = 2l * kQuarter * (g - 1) - src.origin;
        const int sh = (g & 1) ? kN - kQuarter : kQuarter;
        if (src.pairs) {
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = sliced_pair_vec(src, xrow, s0, sh, 256 * (t + 8 * r) + n2);
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = sliced_pair(src, xrow, s0, sh, 256 * (t + 8 * r) + n2);
        }
    } else {
        const float2* xb = in + (long)b * kL;
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = xb[256 * (t + 8 * r) + n2];
    }
    // every twiddle this thread needs, in flight with the data
    load_tw2_lds<128>(tw2, tws, tid, 8 * CPW);
    // W_L^{n2 k1}, k1 = t + 8 q + 16 r, from the rows t, 8 and 16 r of the
    // table: W^{n2 t} W^{8 n2 q} W^{16 n2 r} (two roundings more than a table value)
    float2 tb = twp[t * 256 + n2], t8 = twp[8 * 256 + n2];
    float2 t16[8];
    t16[0] = make_float2(1.0f, 0.0f);
#pragma unroll
    for (int r = 1; r < 8; ++r) t16[r] = twp[16 * r * 256 + n2];
    fft_unit<128, -1>(v, lds + c * P::US, t, tw2, Tw3<128>{});
    const float2 tb8 = cmul(tb, t8);
    float2 tp[16];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        tp[r] = r ? cmul(tb, t16[r]) : tb;
        tp[8 + r] = r ? cmul(tb8, t16[r]) : tb8;
    }
    // v[q*8 + r] = V[k1], k1 = t + 8 q + 16 r
    float2* yb = out + (long)b * kL;
#pragma unroll
    for (int q = 0; q < P::QL; ++q) {
#pragma unroll
        for (int r = 0; r < P::RL; ++r) {
            const int k1 = t + 8 * q + 16 * r;
            yb[k1 * 256 + n2] = cmul(v[q * P::RL + r], tp[q * P::RL + r]);
        }
    }
}


// Column of local slot c in inverse column workgroup w with H = CPW / 2
// column pairs: slots 0..H-1 hold columns p = H w .. H w + H - 1, slots
// H..2H-1 their mirrors 256 - p; pair p = 0 is {0, 128} (both
// self-mirrored). Each half is H consecutive columns (whole 128-byte lines
// per tile row in the wide shape, H = 16).
template <int CPW>
__device__ __forceinline__ int inv_col(int w, int c) {
    constexpr int H = CPW / 2;
    const int p = H * w + (c & (H - 1));
    return c < H ? p : (p == 0 ? 128 : 256 - p);
}

template <int CPW, bool WT>
__device__ __forceinline__ void col_inv_tile(const int b, const int w, const float2* __restrict__ f,
                                             float2* __restrict__ out, const float2* __restrict__ twp,
                                             const float2* __restrict__ twn, const int* __restrict__ fold,
                                             const float2* __restrict__ tws, float2* lds,
                                             const int tid = threadIdx.x) {
    using P = Plan<128>;
    constexpr int H = CPW / 2;                    // column pairs per workgroup
    constexpr int kWgs = 256 / CPW;               // workgroups per slice
    constexpr int kThreads = 8 * CPW;
    constexpr int kShare = kWgs / kFoldLists;     // workgroups sharing one fold list
    constexpr int kEnt = kFoldPerWg / kThreads;   // fold-list entries per thread
    static_assert(kShare * kFoldLists == kWgs && kEnt * kThreads == kFoldPerWg, "fold list split");
    // lds: staged bins, then the FFT exchange; then the twiddle block
    float2* tw2 = lds + CPW * P::US;
    const int c = tid & (CPW - 1);
    const int t = tid / CPW;
    const int col = inv_col<CPW>(w, c);
    const float2* fb = f + (long)b * kFRow;
    float2* raw = lds + c * P::US;
    // fold list entries of this thread (bin | overflow index << 16, or -1),
    // from the list of the wide workgroup that contains this one
    int ent[kEnt];
#pragma unroll
    for (int e = 0; e < kEnt; ++e) ent[e] = fold[(w / kShare) * kFoldPerWg + tid + e * kThreads];
    float2 q0[16], q1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        q0[r] = fb[256 * (t + 8 * r) + col];
        q1[r] = fb[kFStride + 256 * (t + 8 * r) + col];
    }
    // retangle and pass twiddles, in flight with the data: W_N^{256 (t + 8 r) + col}
    // = W_N^{256 t + col} W_N^{2048 r} (the second factor is the same for the
    // whole workgroup), one rounding more than a table value
    const float2 tnb = twn[256 * t + col];
    float2 tn[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) tn[r] = twn[2048 * r];
    load_tw2_lds<128>(tw2, tws, tid, kThreads);
    // overflow slot sums of this workgroup's listed bins and their LDS
    // positions (bin L is parked in column 0's pad slot, raw[128] of slot 0)
    float2 oadd[kEnt];
    int opos[kEnt];
#pragma unroll
    for (int e = 0; e < kEnt; ++e) {
        oadd[e] = make_float2(0.0f, 0.0f);
        opos[e] = -1;
        if (ent[e] >= 0) {
            const int bin = ent[e] & 0xffff;
            int pos = -1;
            if (bin >= kL) {
                if (w == 0) pos = 128;
            } else {
                const int cl = bin & 255, n1 = bin >> 8;
                const int pp = cl <= 128 ? (cl == 128 ? 0 : cl) : 256 - cl;
                if (pp / H == w)               // a bin of this workgroup's columns
                    pos = ((cl < 128 ? 0 : H) + (pp & (H - 1))) * P::US + n1;
            }
            if (pos >= 0) {
                const int k = min(ent[e] >> 16, kOvfCap - 1);
                const float2* o = fb + 2 * kFStride + 2 * k;
                oadd[e] = cadd(o[0], o[1]);
                opos[e] = pos;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) raw[t + 8 * r] = cadd(q0[r], q1[r]);
    // bin L is parked in column 0's pad slot raw[128] (column 0 is slot 0 of
    // workgroup 0)
    if (col == 0 && t == 0) raw[128] = dense_bin(fb, kL);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kEnt; ++e)
        if (opos[e] >= 0) lds[opos[e]] = cadd(lds[opos[e]], oadd[e]);   // each listed bin appears once
    __syncthreads();
    if (col == 0 && t == 0) {          // bins 0 and L are real for irfft (after any fold)
        raw[0].y = 0.0f;
        raw[128].y = 0.0f;
    }
    __syncthreads();
    // mirror bin L - i: column 256 - col at row 127 - n1; columns 0 and 128
    // are their own mirrors (column 0 at row 128 - n1, row 128 = bin L)
    const float2* mp = (col == 0 || col == 128) ? raw : lds + (c ^ H) * P::US;
    const int moff = col == 0 ? 128 : 127;
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int n1 = t + 8 * r;
        const float2 f0 = raw[n1];
        const float2 f1 = mp[moff - n1];
        // 2W = conj(S + i D conj(W_N^i)) with S = f0 + conj f1, D = f0 - conj f1;
        // the factor 2 is removed by the 1/(2L) of the unpack
        const float2 sm = make_float2(f0.x + f1.x, f0.y - f1.y);
        const float2 d = make_float2(f0.x - f1.x, f0.y + f1.y);
        const float2 o = cmulc(d, r ? cmul(tnb, tn[r]) : tnb);
        v[r] = make_float2(sm.x - o.y, -(sm.y + o.x));
    }
    const float2 pb = twp[t * 256 + col], p8 = twp[8 * 256 + col];
    float2 p16[8];
    p16[0] = make_float2(1.0f, 0.0f);
#pragma unroll
    for (int r = 1; r < 8; ++r) p16[r] = twp[16 * r * 256 + col];
    __syncthreads();  // staged bins fully consumed before the FFT reuses LDS
    fft_unit<128, -1>(v, lds + c * P::US, t, tw2, Tw3<128>{});
    const float2 pb8 = cmul(pb, p8);
    float2 tp[16];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        tp[r] = r ? cmul(pb, p16[r]) : pb;
        tp[8 + r] = r ? cmul(pb8, p16[r]) : pb8;
    }
    float2* yb = out + (long)b * kL;
#pragma unroll
    for (int q = 0; q < P::QL; ++q) {
#pragma unroll
        for (int r = 0; r < P::RL; ++r) {
            const int k1 = t + 8 * q + 16 * r;
            store_out<WT>(&yb[k1 * 256 + col], cmul(v[q * P::RL + r], tp[q * P::RL + r]));
        }
    }
}


// --------------------------------------------------------------- row pass

// Row of local slot rho in forward row workgroup w with HP = RPW / 2 row
// pairs: slots 0..HP-1 hold rows p = HP w .. HP w + HP - 1, slots
// HP..2HP-1 their mirrors 128 - p; pair p = 0 is {0, 64} (both
// self-mirrored).
template <int RPW>
__device__ __forceinline__ int fwd_row(int w, int rho) {
    constexpr int HP = RPW / 2;
    const int p = HP * w + (rho & (HP - 1));
    return rho < HP ? p : (p == 0 ? 64 : 128 - p);
}

// Row FFTs of one tile of 256-column rows (16 threads per row), results
// left in LDS as Z_row[k2] at lds[rho*US + pad16(k2)] (a barrier follows).
// vhold / shold: a per-thread value and 16 workgroup-uniform values loaded
// before the call that must arrive with the row data (the untangle
// twiddles), so their loads are not deferred past the barriers.
template <bool HOLD>
__device__ __forceinline__ void row_fft_to_lds(const float2* __restrict__ yrow, float2* lds, float2* tw2,
                                               int rho, int t, int nthreads, const float2* __restrict__ tws,
                                               float2* vhold, float2* shold, const int tid) {
    using P = Plan<256>;
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = yrow[t + 16 * r];
    load_tw2_lds<256>(tw2, tws, tid, nthreads);
    if constexpr (HOLD) {
        asm volatile("" : "+v"(vhold->x), "+v"(vhold->y));
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            // the values are workgroup-uniform: held in scalar registers
            // (readfirstlane when the compiler loaded them with vector loads)
            shold[u].x = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(shold[u].x)));
            shold[u].y = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(shold[u].y)));
            asm volatile("" : "+s"(shold[u].x), "+s"(shold[u].y));
        }
    }
    float2* s = lds + rho * P::US;
    fft_unit<256, -1>(v, s, t, tw2, Tw3<256>{});
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) s[pad16(t + 16 * r)] = v[r];
    __syncthreads();
}

template <int RPW>
__device__ __forceinline__ void row_fwd_tile(const int b, const int w, const float2* __restrict__ in,
                                             float2* __restrict__ xs, const float2* __restrict__ twn,
                                             const float2* __restrict__ tws, float2* lds,
                                             const int tid = threadIdx.x) {
    using P = Plan<256>;
    float2* tw2 = lds + RPW * P::US;
    const int rho = tid >> 4;
    const int t = tid & 15;
    // untangle twiddles of this thread's output bins, loaded up front:
    // W_N^{k1 + 128 (kg + 16 u)} = W_N^{k1 + 128 kg} W_N^{2048 u}, the second
    // factor the same for the whole workgroup (one rounding more than a table value)
    const int rho2 = tid & (RPW - 1);             // output lanes walk the tile's rows
    const int kg = tid / RPW;                     // < 16
    const int k1 = fwd_row<RPW>(w, rho2);
    float2 wb = twn[k1 + 128 * kg];
    float2 wu[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) wu[u] = twn[2048 * u];
    row_fft_to_lds<true>(in + (long)b * kL + (long)fwd_row<RPW>(w, rho) * 256, lds, tw2, rho, t, 16 * RPW, tws,
                         &wb, wu, tid);
    // untangle: lanes walk the tile's rows for coalesced stores
    const float2* s = lds + rho2 * P::US;
    // mirror bin L - k: row 128 - k1 at column 255 - k2; rows 0 and 64 are
    // their own mirrors (row 0 at column (256 - k2) mod 256)
    const float2* mp = (k1 == 0 || k1 == 64) ? s : lds + (rho2 ^ (RPW / 2)) * P::US;
    const int mcol = k1 == 0 ? 256 : 255;
    float2* xb = xs + (long)b * kXStride;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int k2 = kg + 16 * u;
        const float2 z = s[pad16(k2)];
        const float2 zm = mp[pad16((mcol - k2) & 255)];
        // X = E + W O,  E = (z + conj zm)/2,  O = (z - conj zm)/(2i),  W = W_N^k
        const float2 sm = make_float2(z.x + zm.x, z.y - zm.y);
        const float2 d = make_float2(z.x - zm.x, z.y + zm.y);
        const float2 wn = u ? cmul(wb, wu[u]) : wb;
        xb[k1 + 128 * k2] = make_float2(0.5f * fmaf(wn.x, d.y, fmaf(wn.y, d.x, sm.x)),
                                        0.5f * fmaf(wn.y, d.y, fmaf(-wn.x, d.x, sm.y)));
    }
    if (w == 0 && tid == 0) {                       // Nyquist bin from Z[0] (row 0, k2 = 0)
        const float2 z0 = lds[pad16(0)];
        xb[kL] = make_float2(z0.x - z0.y, 0.0f);
    }
}


template <int RPW, bool WT>
__device__ __forceinline__ void row_inv_tile(const int b, const int rg, const float2* __restrict__ in,
                                             float2* __restrict__ y, const float2* __restrict__ tws, float2* lds,
                                             const int tid = threadIdx.x) {
    using P = Plan<256>;
    float2* tw2 = lds + RPW * P::US;
    const int rho = tid >> 4;
    const int t = tid & 15;
    row_fft_to_lds<false>(in + (long)b * kL + (long)(rg * RPW + rho) * 256, lds, tw2, rho, t, 16 * RPW, tws,
                          nullptr, nullptr, tid);
    const int rho2 = tid & (RPW - 1);
    const int kg = tid / RPW;
    const float2* s2 = lds + rho2 * P::US;
    const int kk1 = rg * RPW + rho2;
    constexpr float sc = 0.5f / (float)kL;     // 1/L of the inverse, 1/2 of the retangle
    float2* yo = y + (long)b * kL;  // y viewed as [batch][32768] float pairs
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int k2 = kg + 16 * u;
        const float2 w = s2[pad16(k2)];
        store_out<WT>(&yo[kk1 + 128 * k2], make_float2(w.x * sc, -w.y * sc));
    }
}

// The inverse row pass of one slice s of a SlicedCQT signal with the
// overlap-add in its store (whole-signal synthesis; orow is the signal's
// output row of `length` samples). Slice s's samples jj, jj + 1 (jj =
// 2 (kk1 + 128 k2)) go to p, p + 1 with p = 2H (s - 1) + j, j = (jj + H)
// mod N in even slices and (jj - H) mod N in odd ones, where p < length.
// Even slices (one launch) store 0 + v; odd slices (the next launch) add v
// to that, or store 0 + v in their second half when there is no slice
// s + 1. The values are the rounded products k_row_inv stores, so the sums
// are k_overlap_add's (0 + a) + b up to the order of two operands, which
// gives the same bits. PAIR: length even and orow 8-byte aligned, so p and
// p + 1 are both in range or both out, and one 8-byte access serves both.
template <int RPW, bool ODD, bool PAIR>
__device__ __forceinline__ void row_inv_ola_tile(const int b, const int rg, const int s, const int S,
                                                 const long length, const float2* __restrict__ in,
                                                 float* __restrict__ orow, const float2* __restrict__ tws,
                                                 float2* lds, const int tid = threadIdx.x) {
    using P = Plan<256>;
    float2* tw2 = lds + RPW * P::US;
    const int rho = tid >> 4;
    const int t = tid & 15;
    row_fft_to_lds<false>(in + (long)b * kL + (long)(rg * RPW + rho) * 256, lds, tw2, rho, t, 16 * RPW, tws,
                          nullptr, nullptr, tid);
    const int rho2 = tid & (RPW - 1);
    const int kg = tid / RPW;
    const float2* s2 = lds + rho2 * P::US;
    const int kk1 = rg * RPW + rho2;
    constexpr float sc = 0.5f / (float)kL;     // 1/L of the inverse, 1/2 of the retangle
    const long base = 2l * kQuarter * (s - 1);
    const bool last = s + 1 >= S;              // no slice s + 1
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int k2 = kg + 16 * u;
        const float2 w = s2[pad16(k2)];
        const int j = (2 * (kk1 + 128 * k2) + (ODD ? kN - kQuarter : kQuarter)) & (kN - 1);
        const long p = base + j;
        float v0 = w.x * sc, v1 = -w.y * sc;
        asm volatile("" : "+v"(v0), "+v"(v1));    // the rounded products, as k_row_inv stores them
        const bool add = ODD && (j < 2 * kQuarter || !last);
        if constexpr (PAIR) {
            if (p >= 0 && p < length) {
                float2* o = reinterpret_cast<float2*>(orow + p);
                const float2 a = add ? *o : make_float2(0.0f, 0.0f);
                *o = make_float2(a.x + v0, a.y + v1);
            }
        } else {
            if (p >= 0 && p < length) orow[p] = (add ? orow[p] : 0.0f) + v0;
            if (p + 1 >= 0 && p + 1 < length) orow[p + 1] = (add ? orow[p + 1] : 0.0f) + v1;
        }
    }
}

}  // namespace fcqt
