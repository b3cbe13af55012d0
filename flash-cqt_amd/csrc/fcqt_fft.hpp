// Device-side FFT engine shared by every kernel of the fused CQT library.
//
// One "unit" is one transform of length M (a power of two, 32..2048) owned by
// T = M/16 threads of a workgroup; every thread holds 16 complex values in
// registers. The transform is a Stockham auto-sort decomposition
//     M = 16 * R2 [* R3]      (R2 = 16 for M >= 256, else M/16; R3 = M/256)
// whose first stage runs on the values each thread loaded itself (element
// t + T*r of the unit), whose later stages exchange through LDS, and whose
// last stage leaves element  t + T*q + r*(M/RL)  in v[q*RL + r]  (RL = last
// radix), so the caller can store straight to global memory with unit-stride
// lanes. Butterflies are radix 2/4/8/16 codelets on registers; only the
// inter-stage twiddles come from a table (float64-rounded, see
// flash_cqt/tables.py): the second stage reads them from an LDS copy, the
// third forms most of them as products of a few table values (one or two
// roundings more), which keeps the round trip near 130 dB.
//
// LDS layout per unit: element i at i + (i >> 4) (one pad slot every 16
// complex values) and a unit stride of M + M/16 + 1 complex values. With
// 8-byte accesses this keeps 16 consecutive lanes on 16 distinct bank pairs
// for every read/write pattern below, whether consecutive lanes walk one
// unit (band kernels, row passes) or walk across units (column pass).
//
// SIGN = -1 is the forward DFT  X[k] = sum x[n] e^{-2 pi i nk/M},
// SIGN = +1 the unscaled inverse (scales are folded into the tables).
#pragma once

#include <hip/hip_runtime.h>

namespace fcqt {

constexpr int kN = 65536;        // slice length (real samples)
constexpr int kL = 32768;        // packed complex length N/2
constexpr int kFStride = kL + 64;  // complex elements per half-spectrum plane (>= L + 1)
constexpr int kOvfCap = 4096;      // overflow bins (more than two taps) per scatter table
constexpr int kFRow = 2 * kFStride + 2 * kOvfCap;  // complex elements per batch row of F
constexpr int kFoldPerWg = 512;    // overflow fold-list entries per inverse column workgroup
constexpr int kXStride = kL + 64;  // complex elements per row of the rfft spectrum X (>= L + 1)

// ------------------------------------------------------------ complex ops

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }

// a * b
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(fmaf(a.x, b.x, -a.y * b.y), fmaf(a.x, b.y, a.y * b.x));
}
// a * conj(b)
__device__ __forceinline__ float2 cmulc(float2 a, float2 b) {
    return make_float2(fmaf(a.x, b.x, a.y * b.y), fmaf(a.y, b.x, -a.x * b.y));
}
// ------------------------------------------------------------ output stores
// WT = true: a store that writes through this XCD's L2 (a relaxed device-scope
// atomic store, 'sc1'), so the line goes on to the memory-side cache at once
// instead of staying dirty in the L2 until the write-back at the end of the
// kernel, which then no longer sits on the critical path. It pays for
// outputs of many MB that the next kernel reads from other XCDs (or that
// are final): the band kernels from 4 slices up and the wide inverse
// passes. A line written this way is not kept in the writer's L2, so a
// consumer on the same XCD no longer hits it there, and a store covering
// half a 128-byte line costs extra bytes. The values stored are the same
// either way.
template <bool WT>
__device__ __forceinline__ void store_out(float2* p, float2 v) {
    if constexpr (WT) {
        const unsigned long long bits =
            ((unsigned long long)__float_as_uint(v.y) << 32) | (unsigned long long)__float_as_uint(v.x);
        __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), bits, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else {
        *p = v;
    }
}
template <bool WT>
__device__ __forceinline__ void store_out(float* p, float v) {
    if constexpr (WT)
        __hip_atomic_store(reinterpret_cast<unsigned*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

// a * (SIGN i)   i.e. a * e^{SIGN i pi/2}
template <int SIGN>
__device__ __forceinline__ float2 rot4(float2 a) {
    return SIGN < 0 ? make_float2(a.y, -a.x) : make_float2(-a.y, a.x);
}

// cos / sin of e*pi/8 for e = 0..9 (the exponents a 4x4 split of a 16-point
// DFT needs), correctly rounded double literals.
__device__ __forceinline__ constexpr double c16(int e) {
    return e == 0 ? 1.0 : e == 1 ? 0.92387953251128675613 : e == 2 ? 0.70710678118654752440
         : e == 3 ? 0.38268343236508977173 : e == 4 ? 0.0 : e == 5 ? -0.38268343236508977173
         : e == 6 ? -0.70710678118654752440 : e == 7 ? -0.92387953251128675613
         : e == 8 ? -1.0 : -0.92387953251128675613;
}
__device__ __forceinline__ constexpr double s16(int e) {
    return e == 0 ? 0.0 : e == 1 ? 0.38268343236508977173 : e == 2 ? 0.70710678118654752440
         : e == 3 ? 0.92387953251128675613 : e == 4 ? 1.0 : e == 5 ? 0.92387953251128675613
         : e == 6 ? 0.70710678118654752440 : e == 7 ? 0.38268343236508977173
         : e == 8 ? 0.0 : -0.38268343236508977173;
}

// a * W16^E with W16 = e^{SIGN i pi/8}
template <int SIGN, int E>
__device__ __forceinline__ float2 tw16(float2 a) {
    if constexpr (E == 0) {
        return a;
    } else if constexpr (E == 4) {
        return rot4<SIGN>(a);
    } else if constexpr (E == 2 || E == 6) {
        // (c + SIGN i s) with |c| = |s| = 1/sqrt2
        constexpr float h = 0.70710678118654752440f;
        constexpr float sc = E == 2 ? 1.0f : -1.0f;  // sign of cos
        const float re = sc * a.x - (float)SIGN * a.y;
        const float im = sc * a.y + (float)SIGN * a.x;
        return make_float2(re * h, im * h);
    } else {
        constexpr float c = (float)c16(E);
        constexpr float s = (float)(SIGN * s16(E));
        return make_float2(fmaf(a.x, c, -a.y * s), fmaf(a.x, s, a.y * c));
    }
}

// -------------------------------------------------------------- codelets
// All codelets work in place on a[0..R) and leave X[k] in a[k].

template <int SIGN>
__device__ __forceinline__ void dft2(float2* a) {
    const float2 t = a[1];
    a[1] = csub(a[0], t);
    a[0] = cadd(a[0], t);
}

template <int SIGN>
__device__ __forceinline__ void dft4v(float2& a0, float2& a1, float2& a2, float2& a3) {
    const float2 t0 = cadd(a0, a2), t1 = csub(a0, a2);
    const float2 t2 = cadd(a1, a3), t3 = rot4<SIGN>(csub(a1, a3));
    a0 = cadd(t0, t2);
    a2 = csub(t0, t2);
    a1 = cadd(t1, t3);
    a3 = csub(t1, t3);
}

template <int SIGN>
__device__ __forceinline__ void dft4(float2* a) { dft4v<SIGN>(a[0], a[1], a[2], a[3]); }

template <int SIGN>
__device__ __forceinline__ void dft8(float2* a) {
    // even / odd split: E = DFT4(a0,a2,a4,a6), O = DFT4(a1,a3,a5,a7)
    float2 e0 = a[0], e1 = a[2], e2 = a[4], e3 = a[6];
    float2 o0 = a[1], o1 = a[3], o2 = a[5], o3 = a[7];
    dft4v<SIGN>(e0, e1, e2, e3);
    dft4v<SIGN>(o0, o1, o2, o3);
    o1 = tw16<SIGN, 2>(o1);
    o2 = tw16<SIGN, 4>(o2);
    o3 = tw16<SIGN, 6>(o3);
    a[0] = cadd(e0, o0); a[4] = csub(e0, o0);
    a[1] = cadd(e1, o1); a[5] = csub(e1, o1);
    a[2] = cadd(e2, o2); a[6] = csub(e2, o2);
    a[3] = cadd(e3, o3); a[7] = csub(e3, o3);
}

template <int SIGN>
__device__ __forceinline__ void dft16(float2* a) {
    // n = 4 n1 + n2, k = k1 + 4 k2:  X = DFT4_{n2}( W16^{n2 k1} DFT4_{n1}(a) )
    float2 y[16];  // y[n2*4 + k1]
#pragma unroll
    for (int n2 = 0; n2 < 4; ++n2) {
        float2 b0 = a[n2], b1 = a[4 + n2], b2 = a[8 + n2], b3 = a[12 + n2];
        dft4v<SIGN>(b0, b1, b2, b3);
        y[n2 * 4 + 0] = b0; y[n2 * 4 + 1] = b1; y[n2 * 4 + 2] = b2; y[n2 * 4 + 3] = b3;
    }
    y[5] = tw16<SIGN, 1>(y[5]);
    y[6] = tw16<SIGN, 2>(y[6]);
    y[7] = tw16<SIGN, 3>(y[7]);
    y[9] = tw16<SIGN, 2>(y[9]);
    y[10] = tw16<SIGN, 4>(y[10]);
    y[11] = tw16<SIGN, 6>(y[11]);
    y[13] = tw16<SIGN, 3>(y[13]);
    y[14] = tw16<SIGN, 6>(y[14]);
    y[15] = tw16<SIGN, 9>(y[15]);
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) {
        float2 b0 = y[k1], b1 = y[4 + k1], b2 = y[8 + k1], b3 = y[12 + k1];
        dft4v<SIGN>(b0, b1, b2, b3);
        a[k1] = b0; a[k1 + 4] = b1; a[k1 + 8] = b2; a[k1 + 12] = b3;
    }
}

template <int R, int SIGN>
__device__ __forceinline__ void dft(float2* a) {
    if constexpr (R == 2) dft2<SIGN>(a);
    else if constexpr (R == 4) dft4<SIGN>(a);
    else if constexpr (R == 8) dft8<SIGN>(a);
    else dft16<SIGN>(a);
}

// ------------------------------------------------------- stage twiddles
// Table layout (complex, forward sign): for each (NS, R) in the order below,
// entry [r][k] = W_{NS R}^{r k}, r < R, k < NS. The lanes of one load share r
// and hold consecutive k, so every load touches few cache lines. Offsets in
// complex elements.
constexpr int tw_off(int NS, int R) {
    return NS == 16 ? (R == 2 ? 0 : R == 4 ? 32 : R == 8 ? 96 : 224)
                    : (R == 2 ? 480 : R == 4 ? 992 : 2016);
}
constexpr int kTwStageLen = 4064;

// ------------------------------------------------------------ the plan

__device__ __forceinline__ int pad16(int i) { return i + (i >> 4); }

template <int M>
struct Plan {
    static_assert(M >= 32 && M <= 2048 && (M & (M - 1)) == 0, "band length");
    static constexpr int T = M / 16;                     // threads per unit
    static constexpr int R2 = M >= 256 ? 16 : M / 16;    // second radix
    static constexpr int R3 = M > 256 ? M / 256 : 1;     // third radix (1 = none)
    static constexpr int RL = M > 256 ? R3 : R2;         // last radix
    static constexpr int QL = 16 / RL;                   // last-stage butterflies per thread
    static constexpr int OS = M / RL;                    // output stride of r
    static constexpr int US = M + M / 16 + 1;            // LDS stride per unit (complex)
};

// Twiddle sources. The second stage (NS = 16) takes its W_{16 R}^{r k}
// from a copy of its table block in LDS (16 R values, [r][k]): one copy per
// workgroup, and no vector-memory instruction per twiddle. The third stage
// (NS = 256, R <= 8) loads W^k, W^2k and W^4k and forms W^3k, W^5k, W^6k,
// W^7k as products (at most two roundings more than a table value).
template <int M>
constexpr int tw2_len() { return 16 * Plan<M>::R2; }

// Copy the second-stage twiddle block into LDS (tl holds tw2_len<M>()
// values); every thread of the workgroup calls this before its first
// barrier.
template <int M>
__device__ __forceinline__ void load_tw2_lds(float2* tl, const float2* __restrict__ tws, int tid,
                                             int nthreads) {
    constexpr int R = Plan<M>::R2;
    constexpr int N4 = tw2_len<M>() / 2;
    const float4* src = reinterpret_cast<const float4*>(tws + tw_off(16, R));
    float4* dst = reinterpret_cast<float4*>(tl);
    for (int i = tid; i < N4; i += nthreads) dst[i] = src[i];
}

// The same copy in two halves, for a workgroup of NT threads: fetch_tw2
// issues the loads into registers (early, so that their latency hides under
// the data loads), put_tw2 writes them to LDS before the first barrier.
template <int M, int NT>
struct Tw2Copy {
    static constexpr int N4 = tw2_len<M>() / 2;
    static constexpr int PER = (N4 + NT - 1) / NT;
    float4 d[PER];
};

template <int M, int NT>
__device__ __forceinline__ void fetch_tw2(Tw2Copy<M, NT>& c, const float2* __restrict__ tws, int tid) {
    constexpr int N4 = Tw2Copy<M, NT>::N4;
    const float4* src = reinterpret_cast<const float4*>(tws + tw_off(16, Plan<M>::R2));
#pragma unroll
    for (int k = 0; k < Tw2Copy<M, NT>::PER; ++k) c.d[k] = src[min(tid + k * NT, N4 - 1)];
}

template <int M, int NT>
__device__ __forceinline__ void put_tw2(float2* tl, const Tw2Copy<M, NT>& c, int tid) {
    constexpr int N4 = Tw2Copy<M, NT>::N4;
    float4* dst = reinterpret_cast<float4*>(tl);
#pragma unroll
    for (int k = 0; k < Tw2Copy<M, NT>::PER; ++k)
        if (tid + k * NT < N4) dst[tid + k * NT] = c.d[k];
}

// Third-stage bases W^k, W^2k, W^4k (k = j mod 256) of each of a thread's
// 16 / R3 butterflies, loaded with the unit's data so that no table read
// waits behind the transform's barriers.
template <int M>
struct Tw3 {
    static constexpr int R = Plan<M>::R3;
    static constexpr int Q = R > 1 ? 16 / R : 1;
    float2 b[Q][3];
};

template <int M>
__device__ __forceinline__ void load_tw3(Tw3<M>& w3, const float2* __restrict__ tws, int t) {
    constexpr int R = Plan<M>::R3;
    if constexpr (R > 1) {
        static_assert(R == 2 || R == 4 || R == 8, "third-stage radix");
        constexpr int T = M / 16;
        constexpr int Q = Tw3<M>::Q;
        static_assert(T * Q == 256, "butterfly columns k = t + T q stay below 256");
        // k = t + T q: the bases of butterfly q are those of q = 0 times
        // W^{r T q}, the same for the whole workgroup (one rounding more
        // than a table value)
        const float2* blk = tws + tw_off(256, R);
        w3.b[0][0] = blk[256 + t];
        if constexpr (R >= 4) w3.b[0][1] = blk[512 + t];
        if constexpr (R == 8) w3.b[0][2] = blk[1024 + t];
#pragma unroll
        for (int q = 1; q < Q; ++q) {
            w3.b[q][0] = cmul(w3.b[0][0], blk[256 + T * q]);
            if constexpr (R >= 4) w3.b[q][1] = cmul(w3.b[0][1], blk[512 + T * q]);
            if constexpr (R == 8) w3.b[q][2] = cmul(w3.b[0][2], blk[1024 + T * q]);
        }
    }
}

// W^{rk}, r < R, from the bases: W^3k, W^5k, W^6k, W^7k as products (at most
// two roundings more than a table value).
template <int R>
__device__ __forceinline__ void expand_tw3(float2* w, const float2* b) {
    w[0] = make_float2(1.0f, 0.0f);
    w[1] = b[0];
    if constexpr (R >= 4) {
        w[2] = b[1];
        w[3] = cmul(b[0], b[1]);
    }
    if constexpr (R == 8) {
        w[4] = b[2];
        w[5] = cmul(b[0], b[2]);
        w[6] = cmul(b[1], b[2]);
        w[7] = cmul(w[3], b[2]);
    }
}

// One Stockham stage read: butterflies j = t + T q, inputs j + r M/R,
// twiddle W_{NS R}^{r (j mod NS)}, radix-R DFT, results into v[q R + r].
// M/R is a multiple of 16 in every stage that reads LDS, so
// pad16(j + r M/R) = pad16(j) + r (M/R)(17/16): one address per butterfly,
// constant offsets for r (immediate offsets of the LDS instructions).
// tl: the LDS twiddle block for NS = 16; tws: the table for NS = 256.
template <int M, int R, int NS, int SIGN>
__device__ __forceinline__ void stage_read(float2* v, const float2* s, int t, const float2* tl,
                                           const Tw3<M>& w3) {
    constexpr int T = M / 16;
    constexpr int Q = 16 / R;
    constexpr int STRIDE = M / R;
    static_assert(STRIDE % 16 == 0, "padded stride");
    constexpr int PSTRIDE = STRIDE + STRIDE / 16;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int j = t + T * q;
        const float2* sj = s + pad16(j);
        float2 a[R];
#pragma unroll
        for (int r = 0; r < R; ++r) a[r] = sj[r * PSTRIDE];
        if constexpr (NS > 1) {
            float2 w[R];
            if constexpr (NS == 16) {
                const float2* tk = tl + (j & 15);
                w[0] = make_float2(1.0f, 0.0f);
#pragma unroll
                for (int r = 1; r < R; ++r) w[r] = tk[16 * r];
            } else {
                expand_tw3<R>(w, w3.b[q]);
            }
#pragma unroll
            for (int r = 1; r < R; ++r) a[r] = SIGN < 0 ? cmul(a[r], w[r]) : cmulc(a[r], w[r]);
        }
        dft<R, SIGN>(a);
#pragma unroll
        for (int r = 0; r < R; ++r) v[q * R + r] = a[r];
    }
}

// Stockham stage write: butterfly j's result r goes to
// (j / NS) NS R + (j mod NS) + r NS. NS is 1 (R = 16: 16 consecutive slots,
// one pad slot after them) or 16 (pad16(base + 16 r) = pad16(base) + 17 r).
template <int M, int R, int NS>
__device__ __forceinline__ void stage_write(const float2* v, float2* s, int t) {
    constexpr int T = M / 16;
    constexpr int Q = 16 / R;
    static_assert((NS == 1 && R == 16) || NS == 16, "stage write layout");
    constexpr int PS = NS == 1 ? 1 : 17;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int j = t + T * q;
        const int base = (j / NS) * NS * R + (j & (NS - 1));
        float2* sb = s + pad16(base);
#pragma unroll
        for (int r = 0; r < R; ++r) sb[r * PS] = v[q * R + r];
    }
}

// Whole unit transform. Entry: v[r] = x[t + T r]; the unit's LDS region s is
// free to write; tl holds the second-stage twiddle block (load_tw2_lds
// before the call), w3 the third-stage bases (load_tw3). Exit:
// v[q RL + r] = X[t + T q + r OS]; other threads may still read s, so a
// caller that writes s again must barrier first.
// Every thread of the workgroup must call this (it contains barriers).
template <int M, int SIGN>
__device__ __forceinline__ void fft_unit(float2* v, float2* s, int t, const float2* tl, const Tw3<M>& w3) {
    using P = Plan<M>;
    dft16<SIGN>(v);
    stage_write<M, 16, 1>(v, s, t);
    __syncthreads();
    stage_read<M, P::R2, 16, SIGN>(v, s, t, tl, w3);
    if constexpr (P::R3 > 1) {
        __syncthreads();
        stage_write<M, 16, 16>(v, s, t);
        __syncthreads();
        stage_read<M, P::R3, 256, SIGN>(v, s, t, tl, w3);
    }
}

// ------------------------------------- cross-lane (DPP) stage exchange
// An alternative stage-1 -> 2 exchange for units of M <= 256, whose T <= 16
// threads are consecutive, T-aligned lanes of one row of 16 lanes (the band
// kernels' layout). After the radix-16 first stage, thread t holds output
// k1 = t' + T q of its own column in v[T q + t']; the second stage needs, in
// v[T q + r], output k1 = t + T q of thread r. That is a transpose of the
// log2(T) lane bits with the low register bits, done as one butterfly level
// per bit: a DPP read of the partner lane (lane ^ 2^P) and two selects per
// float. The arithmetic is the LDS path's, with the same output layout.
// Measured on MI355X (band kernels restricted to the six tasks of M <= 256,
// 20 launches, B = 16 / 64 / 256): route 4.56 / 5.8-6.0 / 11.7 us against
// 4.00 / 5.2 / 11.2 us with the LDS exchange, scatter 4.85 / 6.0 / 9.05 us
// against 4.25 / 4.93 / 7.8 us; M = 32 and 64 alone: equal or up to 5%
// slower. Each level costs about 64 VALU instructions per thread where the
// LDS exchange issues 16 writes and 16 reads for all levels at once, and the
// band kernels are busier on the VALU than on the LDS, so the library is
// built with the LDS exchange and this one only in the variant library
// (FCQT_XLANE_MAX_M = 256, libflashcqt_xlane.so) that the benchmark and the
// tests compare against it.

// Partner read for lane bit P: lanes with bit P clear read lane + 2^P
// (ABOVE), lanes with bit P set read lane - 2^P, inside rows of 16 lanes.
template <int P, bool ABOVE>
__device__ __forceinline__ float dpp_partner(float x) {
    static_assert(P >= 0 && P < 4, "lane bit inside a row of 16 lanes");
    // quad_perm [1,0,3,2] / [2,3,0,1]; row_shl:4 / row_shr:4; row_ror:8
    constexpr int ctrl = P == 0 ? 0xB1 : P == 1 ? 0x4E : P == 2 ? (ABOVE ? 0x104 : 0x114) : 0x128;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false));
}

// One level: lane l with bit P set exchanges its register i (bit P clear)
// with register i | 2^P of lane l ^ 2^P.
template <int P>
__device__ __forceinline__ void xlane_level(float2* v, int t) {
    const bool hi = (t >> P) & 1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int i = ((k >> P) << (P + 1)) | (k & ((1 << P) - 1));
        const int i2 = i | (1 << P);
        float ax = v[i].x, ay = v[i].y, bx = v[i2].x, by = v[i2].y;
        // selects on values (a select between two elements of v would become
        // a lane-dependent index and push v out of registers)
        asm("" : "+v"(ax), "+v"(ay), "+v"(bx), "+v"(by));
        const float sx = hi ? ax : bx, sy = hi ? ay : by;
        const float ux = dpp_partner<P, true>(sx), uy = dpp_partner<P, true>(sy);
        const float dx = P == 2 ? dpp_partner<P, false>(sx) : ux;
        const float dy = P == 2 ? dpp_partner<P, false>(sy) : uy;
        v[i2].x = hi ? bx : ux;
        v[i2].y = hi ? by : uy;
        v[i].x = hi ? dx : ax;
        v[i].y = hi ? dy : ay;
    }
}

// Unit transform for M <= 256 with the cross-lane exchange; same contract
// as fft_unit (entry v[r] = x[t + T r], exit v[q RL + r] = X[t + T q + r OS]),
// tl holds the second-stage twiddle block. Every thread of the workgroup
// calls this (one barrier: tl is written before the call).
template <int M, int SIGN>
__device__ __forceinline__ void fft_unit_xl(float2* v, int t, const float2* tl) {
    constexpr int T = M / 16;
    static_assert(T >= 2 && T <= 16 && Plan<M>::R3 == 1 && Plan<M>::R2 == T, "cross-lane units");
    dft16<SIGN>(v);
    xlane_level<0>(v, t);
    if constexpr (T >= 4) xlane_level<1>(v, t);
    if constexpr (T >= 8) xlane_level<2>(v, t);
    if constexpr (T >= 16) xlane_level<3>(v, t);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 16 / T; ++q) {
        const float2* tk = tl + ((t + T * q) & 15);
        float2 a[T];
#pragma unroll
        for (int r = 0; r < T; ++r) a[r] = v[q * T + r];
#pragma unroll
        for (int r = 1; r < T; ++r) a[r] = SIGN < 0 ? cmul(a[r], tk[16 * r]) : cmulc(a[r], tk[16 * r]);
        dft<T, SIGN>(a);
#pragma unroll
        for (int r = 0; r < T; ++r) v[q * T + r] = a[r];
    }
}

// Spread consecutive workgroup ids over the 8 XCDs' L2s so that each XCD
// receives a contiguous range of logical ids (the hardware dispatches ids
// round-robin over XCDs). Bijective on [0, G).
__host__ __device__ __forceinline__ int xcd_remap(int lin, int G) {
    const int q = G >> 3, rem = G & 7;
    const int xcd = lin & 7, idx = lin >> 3;
    return xcd < rem ? xcd * (q + 1) + idx : rem * (q + 1) + (xcd - rem) * q + idx;
}

// The same per-XCD ranges walked from their ends: a kernel that reads what
// the previous kernel of the same grid wrote starts with that kernel's
// last (most recently written, still cached) workgroups. Bijective on [0, G).
__host__ __device__ __forceinline__ int xcd_remap_reverse(int lin, int G) {
    const int q = G >> 3, rem = G & 7;
    const int xcd = lin & 7, idx = lin >> 3;
    const int n = xcd < rem ? q + 1 : q;
    const int start = xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q;
    return start + (n - 1 - idx);
}

// Logical band workgroup lg of a grid of ntasks x batch -> (task, slice b).
// Task-major (lg = task * batch + b): each XCD's contiguous range holds a few
// tasks of every slice, so it reads few tasks' record rows. Slice-major
// (lg = b * ntasks + task): each XCD's range holds whole slices, the same
// slices whose pass tiles xcd_remap put on that XCD, so a slice's spectrum
// and slot rows stay with one L2 and the record rows are shared by its
// slices. Bijective on [0, ntasks * batch) either way.
__host__ __device__ __forceinline__ void band_place(int lg, int ntasks, int batch, bool slice_major, int& task,
                                                    int& b) {
    if (slice_major) {
        b = lg / ntasks;
        task = lg - b * ntasks;
    } else {
        task = lg / batch;
        b = lg - task * batch;
    }
}

}  // namespace fcqt
