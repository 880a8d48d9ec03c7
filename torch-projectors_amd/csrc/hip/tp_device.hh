// Device-side building blocks of the gfx950 projector kernels.
//
// Every function here restates one piece of the reference CPU semantics
// (paths relative to the reference repository) with the same IEEE operation
// sequence, so that sample coordinates, stencil indices, Friedel decisions
// and per-tap products are bit-identical to the CPU kernels.  The library is
// compiled with -ffp-contract=off: the compiler forms no FMA anywhere in here;
// the only fused arithmetic is the explicit fmaf of the gradient-sum helpers
// (cubic_w_fast, cubic_dw_fast, cfma), whose outputs carry a relative bar.
//
// Coordinate convention: a sample position is x = (c, r, d) -- x[0] is the
// rfft column (the Hermitian half axis), x[1] the row, x[2] the slice.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "tp_launch.hh"

namespace tp {

template <typename T>
struct alignas(2 * sizeof(T)) Cx {
    T re, im;
};

template <typename T> __device__ __forceinline__ Cx<T> cadd(Cx<T> a, Cx<T> b) { return {a.re + b.re, a.im + b.im}; }
template <typename T> __device__ __forceinline__ Cx<T> csub(Cx<T> a, Cx<T> b) { return {a.re - b.re, a.im - b.im}; }
template <typename T> __device__ __forceinline__ Cx<T> cscale(Cx<T> a, T s) { return {a.re * s, a.im * s}; }
// c10::complex product (torch/headeronly/util/complex.h:229-238): (ac - bd, ad + bc)
template <typename T> __device__ __forceinline__ Cx<T> cmul(Cx<T> a, Cx<T> b) {
    return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}
template <typename T> __device__ __forceinline__ Cx<T> cconj(Cx<T> a) { return {a.re, -a.im}; }

// Volume storage: a reconstruction element is a Cx<S>; it is computed on as a
// Cx<wide_t<S>>.  Complex-half volumes (the opt-in low-precision storage of
// the forward projections) widen each stored value exactly to fp32 on load,
// so every later step is the fp32 path applied to the widened volume.
template <typename S> struct Wide { using type = S; };
template <> struct Wide<__half> { using type = float; };
template <typename S> using wide_t = typename Wide<S>::type;
// Element i of a complex-half volume, widened.  (fp32 / fp64 volumes are read
// with a plain indexed load at each call site: routing them through a helper
// like this one splits the compiler's 8-byte loads and serialises them.)
__device__ __forceinline__ Cx<float> load_widened(const Cx<__half>* p, int64_t i) {
    const Cx<__half> h = p[i];
    return {__half2float(h.re), __half2float(h.im)};
}
template <typename S> constexpr bool kHalfVolume = std::is_same<S, __half>::value;

// floor(x) as an int plus the fraction x - floor(x).  The reference keeps
// floor(x) in int64 (interpolation_kernels.h, projection_utils.h); beyond
// +-2^24 every tap is clamped (gathers) or dropped (scatters) either way, so
// clamping the integer part there keeps its semantics in 32-bit ints.
template <typename T> __device__ __forceinline__ int split(T x, T& frac) {
    const T f = floor(x);
    frac = x - f;
    const T lim = T(16777216.0);
    return (int)(f < -lim ? -lim : (f > lim ? lim : f));
}
// The same without the clamp, for callers whose |x| is bounded by the box.
template <bool CLAMP, typename T> __device__ __forceinline__ int split_as(T x, T& frac) {
    if (CLAMP) return split(x, frac);
    const T f = floor(x);
    frac = x - f;
    return (int)f;
}

// ---------------------------------------------------------------- cubic weights
// Catmull-Rom, a = -0.5 (cubic_kernels.h:25-43, 50-67).  `a` has the real type
// but the literals are double, so the float instantiation evaluates most terms
// in double -- except a*s*s*s, which is a float product -- and rounds once.
// The two pieces, for s = |s| <= 1 and 1 < |s| <= 2.
template <typename T> __host__ __device__ __forceinline__ T cubic_w_in(T s) {
    const T a = -0.5;
    return (a + 2.0) * s * s * s - (a + 3.0) * s * s + 1.0;
}
template <typename T> __host__ __device__ __forceinline__ T cubic_w_out(T s) {
    const T a = -0.5;
    return a * s * s * s - 5.0 * a * s * s + 8.0 * a * s - 4.0 * a;
}
template <typename T> __host__ __device__ __forceinline__ T cubic_w(T s) {
    s = s < T(0) ? -s : s;
    if (s <= 1.0) return cubic_w_in<T>(s);
    if (s <= 2.0) return cubic_w_out<T>(s);
    return 0.0;
}
// cubic_w(f - (j - 1)) of tap j < 4 for a fractional part f in [0, 1] (the tiled kernels, whose
// coordinates are finite), bit for bit: taps 0 and 3 then lie at 1 <= |s| <= 2, taps 1 and 2 at
// |s| <= 1, and at |s| = 1, where the pieces meet, both give +0, so each tap evaluates one piece.
// (tests/cubic_weights_check.hip compares it with cubic_w over every float f in [0, 1].  A NaN f,
// which cubic_w maps to 0, must not reach it.)
template <typename T> __host__ __device__ __forceinline__ T cubic_w_tap(T f, int j) {
    const T s = f - T(j - 1), as = s < T(0) ? -s : s;
    return (j == 1 || j == 2) ? cubic_w_in<T>(as) : cubic_w_out<T>(as);
}
template <typename T> __host__ __device__ __forceinline__ T cubic_dw(T s) {
    const T a = -0.5;
    const T sign = (s < 0) ? -1.0 : 1.0;
    s = s < T(0) ? -s : s;
    if (s <= 1.0) return sign * (3.0 * (a + 2.0) * s * s - 2.0 * (a + 3.0) * s);
    if (s <= 2.0) return sign * (3.0 * a * s * s - 10.0 * a * s + 8.0 * a);
    return 0.0;
}

// Catmull-Rom weight (a = -0.5) of a tap at signed distance s and its derivative d/ds in fp32 with
// fused multiply-adds, from the factored polynomials (1 - |s|)(1 + |s| - 1.5 s^2) for |s| <= 1 and
// -0.5 (|s| - 1)(2 - |s|)^2 for 1 < |s| <= 2 (0 beyond): a few ulps from the true value everywhere,
// so within a few ulps of cubic_w / cubic_dw away from the double root at |s| = 2, where the
// reference's double evaluation carries ~1e-15 absolute error.  For the gradient sums only, whose
// bar is relative (gathered values and scatter taps keep cubic_w's rounding).
__host__ __device__ __forceinline__ float cubic_w_fast(float s) {
    const float a = fabsf(s), t = 2.0f - a;
    const float in = (1.0f - a) * fmaf(a, fmaf(a, -1.5f, 1.0f), 1.0f);
    const float out = -0.5f * (a - 1.0f) * t * t;
    return a <= 1.0f ? in : (a <= 2.0f ? out : 0.0f);
}
__host__ __device__ __forceinline__ float cubic_dw_fast(float s) {
    const float a = fabsf(s);
    const float in = a * fmaf(a, 4.5f, -5.0f);
    const float out = (2.0f - a) * fmaf(a, 1.5f, -2.0f);
    const float d = a <= 1.0f ? in : (a <= 2.0f ? out : 0.0f);
    return s < 0.0f ? -d : d;
}
// acc + a * s with one rounding per component (gradient sums only).
__device__ __forceinline__ Cx<float> cfma(Cx<float> a, float s, Cx<float> acc) {
    return {fmaf(a.re, s, acc.re), fmaf(a.im, s, acc.im)};
}

// ---------------------------------------------------------------- gather taps
// Friedel-aware FFTW-layout fetch with edge replication (fftw_sampling.h:42-76,
// 96-137): c < 0 mirrors all coordinates and conjugates; c is clamped to N/2,
// r and d to [-N/2+1, N/2], negatives wrap by +N.
template <typename S>
__device__ __forceinline__ Cx<wide_t<S>> fetch2(const Cx<S>* __restrict__ rec, int N, int H, int r, int c) {
    const bool cj = c < 0;
    if (cj) { c = -c; r = -r; }
    c = min(c, H - 1);
    r = min(N / 2, max(r, -N / 2 + 1));
    if (r < 0) r += N;
    Cx<wide_t<S>> v;
    if constexpr (kHalfVolume<S>) v = load_widened(rec, r * H + c);
    else v = rec[r * H + c];
    if (cj) v.im = -v.im;
    return v;
}
template <typename S>
__device__ __forceinline__ Cx<wide_t<S>> fetch3(const Cx<S>* __restrict__ rec, int N, int H, int d, int r, int c) {
    const bool cj = c < 0;
    if (cj) { c = -c; r = -r; d = -d; }
    c = min(c, H - 1);
    r = min(N / 2, max(r, -N / 2 + 1));
    d = min(N / 2, max(d, -N / 2 + 1));
    if (r < 0) r += N;
    if (d < 0) d += N;
    Cx<wide_t<S>> v;
    if constexpr (kHalfVolume<S>) v = load_widened(rec, ((int64_t)d * N + r) * H + c);
    else v = rec[((int64_t)d * N + r) * H + c];
    if (cj) v.im = -v.im;
    return v;
}
// Cubic stencils pre-clamp before the Friedel fetch (interpolation_kernels.h:245-255, 331-342).
template <typename S>
__device__ __forceinline__ Cx<wide_t<S>> fetch2_cubic(const Cx<S>* __restrict__ rec, int N, int H, int r, int c) {
    if (abs(c) >= H) c = (c < 0) ? -(H - 1) : (H - 1);
    r = max(-N / 2 + 1, min(r, N / 2));
    return fetch2(rec, N, H, r, c);
}
template <typename S>
__device__ __forceinline__ Cx<wide_t<S>> fetch3_cubic(const Cx<S>* __restrict__ rec, int N, int H, int d, int r,
                                                      int c) {
    if (abs(c) >= H) c = (c < 0) ? -(H - 1) : (H - 1);
    r = max(-N / 2 + 1, min(r, N / 2));
    d = max(-N / 2 + 1, min(d, N / 2));
    return fetch3(rec, N, H, d, r, c);
}

// ---------------------------------------------------------------- interpolation
// Value and, when GRADS, the analytic spatial gradient g[k] = dF/dx[k].
template <typename T> struct Interp {
    Cx<T> v;
    Cx<T> g[3];
};

// Bilinear (interpolation_kernels.h:78-135): lerp along c, then r.
// `fetch(r, c)` returns the tap value the reference's sampler would return for
// integer coordinates (global fetch2, or a staged copy of it in LDS).
template <typename T, bool GRADS, bool CLAMP = true, typename F>
__device__ __forceinline__ Interp<T> lerp2(F&& fetch, T r, T c) {
    T cx, rx;
    const int cf = split_as<CLAMP>(c, cx), rf = split_as<CLAMP>(r, rx);
    const Cx<T> p00 = fetch(rf, cf), p01 = fetch(rf, cf + 1);
    const Cx<T> p10 = fetch(rf + 1, cf), p11 = fetch(rf + 1, cf + 1);
    const Cx<T> p0 = cadd(p00, cscale(csub(p01, p00), cx));
    const Cx<T> p1 = cadd(p10, cscale(csub(p11, p10), cx));
    Interp<T> o;
    o.v = cadd(p0, cscale(csub(p1, p0), rx));
    if (GRADS) {
        o.g[1] = cadd(cscale(csub(p10, p00), T(1 - cx)), cscale(csub(p11, p01), cx));
        o.g[0] = cadd(cscale(csub(p01, p00), T(1 - rx)), cscale(csub(p11, p10), rx));
        o.g[2] = {0, 0};
    }
    return o;
}
template <typename T, bool GRADS, typename S>
__device__ __forceinline__ Interp<T> interp2_linear(const Cx<S>* __restrict__ rec, int N, int H, T r, T c) {
    return lerp2<T, GRADS>([&](int rr, int cc) { return fetch2(rec, N, H, rr, cc); }, r, c);
}

// Bicubic (interpolation_kernels.h:258-322): sum over r then c of (s*wr)*wc.
// `fetch` returns the pre-clamped tap of fetch2_cubic.
template <typename T, bool GRADS, bool CLAMP = true, typename F>
__device__ __forceinline__ Interp<T> cubic2(F&& fetch, T r, T c) {
    T cx, rx;
    const int cf = split_as<CLAMP>(c, cx), rf = split_as<CLAMP>(r, rx);
    T wc[4], dwc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        wc[j] = CLAMP ? cubic_w<T>(cx - T(j - 1)) : cubic_w_tap<T>(cx, j);
        if (GRADS) dwc[j] = cubic_dw<T>(cx - T(j - 1));
    }
    Interp<T> o;
    o.v = {0, 0};
    o.g[0] = o.g[1] = o.g[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const T wr = CLAMP ? cubic_w<T>(rx - T(i - 1)) : cubic_w_tap<T>(rx, i);
        const T dwr = GRADS ? cubic_dw<T>(rx - T(i - 1)) : T(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const Cx<T> s = fetch(rf + i - 1, cf + j - 1);
            o.v = cadd(o.v, cscale(cscale(s, wr), wc[j]));
            if (GRADS) {
                o.g[1] = cadd(o.g[1], cscale(cscale(s, dwr), wc[j]));
                o.g[0] = cadd(o.g[0], cscale(cscale(s, wr), dwc[j]));
            }
        }
    }
    return o;
}
template <typename T, bool GRADS, typename S>
__device__ __forceinline__ Interp<T> interp2_cubic(const Cx<S>* __restrict__ rec, int N, int H, T r, T c) {
    return cubic2<T, GRADS>([&](int rr, int cc) { return fetch2_cubic(rec, N, H, rr, cc); }, r, c);
}

// Trilinear (interpolation_kernels.h:140-228): lerp along c, then r, then d.
// `fetch(d, r, c)` returns the tap value the reference's sampler would return
// for integer coordinates (global fetch3, or a staged copy of it in LDS).
template <typename T, bool GRADS, bool CLAMP = true, typename F>
__device__ __forceinline__ Interp<T> lerp3(F&& fetch, T d, T r, T c) {
    T dx, rx, cx;
    const int df = split_as<CLAMP>(d, dx), rf = split_as<CLAMP>(r, rx), cf = split_as<CLAMP>(c, cx);
    const Cx<T> p000 = fetch(df, rf, cf), p001 = fetch(df, rf, cf + 1);
    const Cx<T> p010 = fetch(df, rf + 1, cf), p011 = fetch(df, rf + 1, cf + 1);
    const Cx<T> p100 = fetch(df + 1, rf, cf), p101 = fetch(df + 1, rf, cf + 1);
    const Cx<T> p110 = fetch(df + 1, rf + 1, cf), p111 = fetch(df + 1, rf + 1, cf + 1);
    const Cx<T> p00 = cadd(p000, cscale(csub(p001, p000), cx));
    const Cx<T> p01 = cadd(p010, cscale(csub(p011, p010), cx));
    const Cx<T> p10 = cadd(p100, cscale(csub(p101, p100), cx));
    const Cx<T> p11 = cadd(p110, cscale(csub(p111, p110), cx));
    const Cx<T> p0 = cadd(p00, cscale(csub(p01, p00), rx));
    const Cx<T> p1 = cadd(p10, cscale(csub(p11, p10), rx));
    Interp<T> o;
    o.v = cadd(p0, cscale(csub(p1, p0), dx));
    if (GRADS) {
        o.g[2] = csub(p1, p0);
        o.g[1] = cadd(cscale(csub(p01, p00), T(1 - dx)), cscale(csub(p11, p10), dx));
        const T a = T(1 - dx) * T(1 - rx), b = T(1 - dx) * rx, e = dx * T(1 - rx), f = dx * rx;
        o.g[0] = cadd(cadd(cadd(cscale(csub(p001, p000), a), cscale(csub(p011, p010), b)),
                           cscale(csub(p101, p100), e)),
                      cscale(csub(p111, p110), f));
    }
    return o;
}
template <typename T, bool GRADS, typename S>
__device__ __forceinline__ Interp<T> interp3_linear(const Cx<S>* __restrict__ rec, int N, int H, T d, T r, T c) {
    return lerp3<T, GRADS>([&](int dd, int rr, int cc) { return fetch3(rec, N, H, dd, rr, cc); }, d, r, c);
}

// Tricubic (interpolation_kernels.h:345-425): sum over d, r, c of ((s*wd)*wr)*wc.
// `fetch` returns the pre-clamped tap of fetch3_cubic.
template <typename T, bool GRADS, bool CLAMP = true, typename F>
__device__ __forceinline__ Interp<T> cubic3(F&& fetch, T d, T r, T c) {
    T dx, rx, cx;
    const int df = split_as<CLAMP>(d, dx), rf = split_as<CLAMP>(r, rx), cf = split_as<CLAMP>(c, cx);
    T wc[4], dwc[4], wr[4], dwr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        wc[j] = CLAMP ? cubic_w<T>(cx - T(j - 1)) : cubic_w_tap<T>(cx, j);
        wr[j] = CLAMP ? cubic_w<T>(rx - T(j - 1)) : cubic_w_tap<T>(rx, j);
        if (GRADS) {
            dwc[j] = cubic_dw<T>(cx - T(j - 1));
            dwr[j] = cubic_dw<T>(rx - T(j - 1));
        }
    }
    Interp<T> o;
    o.v = {0, 0};
    o.g[0] = o.g[1] = o.g[2] = {0, 0};
#pragma unroll 1
    for (int k = 0; k < 4; ++k) {
        const T wd = CLAMP ? cubic_w<T>(dx - T(k - 1)) : cubic_w_tap<T>(dx, k);
        const T dwd = GRADS ? cubic_dw<T>(dx - T(k - 1)) : T(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const Cx<T> s = fetch(df + k - 1, rf + i - 1, cf + j - 1);
                o.v = cadd(o.v, cscale(cscale(cscale(s, wd), wr[i]), wc[j]));
                if (GRADS) {
                    o.g[2] = cadd(o.g[2], cscale(cscale(cscale(s, dwd), wr[i]), wc[j]));
                    o.g[1] = cadd(o.g[1], cscale(cscale(cscale(s, wd), dwr[i]), wc[j]));
                    o.g[0] = cadd(o.g[0], cscale(cscale(cscale(s, wd), wr[i]), dwc[j]));
                }
            }
        }
    }
    return o;
}
template <typename T, bool GRADS, typename S>
__device__ __forceinline__ Interp<T> interp3_cubic(const Cx<S>* __restrict__ rec, int N, int H, T d, T r, T c) {
    return cubic3<T, GRADS>([&](int dd, int rr, int cc) { return fetch3_cubic(rec, N, H, dd, rr, cc); }, d, r, c);
}

template <int DIM, typename T, bool CUBIC, bool GRADS, typename S>
__device__ __forceinline__ Interp<T> interpolate(const Cx<S>* __restrict__ rec, int N, int H, const T* x) {
    if constexpr (DIM == 2) {
        if constexpr (CUBIC) return interp2_cubic<T, GRADS>(rec, N, H, x[1], x[0]);
        else return interp2_linear<T, GRADS>(rec, N, H, x[1], x[0]);
    } else {
        if constexpr (CUBIC) return interp3_cubic<T, GRADS>(rec, N, H, x[2], x[1], x[0]);
        else return interp3_linear<T, GRADS>(rec, N, H, x[2], x[1], x[0]);
    }
}

// ---------------------------------------------------------------- transposed stencil
// Calls tap(d, r, c, wd, wr, wc) for every stencil cell of position x
// (projection_utils.h:172-300); the callee forms ((v*wd)*wr)*wc in 3D and
// (v*wr)*wc in 2D.  Cubic cells whose axis weight is exactly 0 are skipped.
template <int DIM, typename T, bool CUBIC, typename F>
__device__ __forceinline__ void distribute(const T* x, F&& tap) {
    if constexpr (DIM == 2) {
        T rx, cx;
        const int rf = split(x[1], rx), cf = split(x[0], cx);
        if constexpr (!CUBIC) {
            tap(0, rf, cf, T(1), T(1 - rx), T(1 - cx));
            tap(0, rf + 1, cf, T(1), rx, T(1 - cx));
            tap(0, rf, cf + 1, T(1), T(1 - rx), cx);
            tap(0, rf + 1, cf + 1, T(1), rx, cx);
        } else {
            T wc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) wc[j] = cubic_w<T>(cx - T(j - 1));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const T wr = cubic_w<T>(rx - T(i - 1));
                if (wr == T(0)) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (wc[j] == T(0)) continue;
                    tap(0, rf + i - 1, cf + j - 1, T(1), wr, wc[j]);
                }
            }
        }
    } else {
        T dx, rx, cx;
        const int df = split(x[2], dx), rf = split(x[1], rx), cf = split(x[0], cx);
        if constexpr (!CUBIC) {
            tap(df, rf, cf, T(1 - dx), T(1 - rx), T(1 - cx));
            tap(df + 1, rf, cf, dx, T(1 - rx), T(1 - cx));
            tap(df, rf + 1, cf, T(1 - dx), rx, T(1 - cx));
            tap(df + 1, rf + 1, cf, dx, rx, T(1 - cx));
            tap(df, rf, cf + 1, T(1 - dx), T(1 - rx), cx);
            tap(df + 1, rf, cf + 1, dx, T(1 - rx), cx);
            tap(df, rf + 1, cf + 1, T(1 - dx), rx, cx);
            tap(df + 1, rf + 1, cf + 1, dx, rx, cx);
        } else {
            T wc[4], wr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                wc[j] = cubic_w<T>(cx - T(j - 1));
                wr[j] = cubic_w<T>(rx - T(j - 1));
            }
#pragma unroll 1
            for (int k = 0; k < 4; ++k) {
                const T wd = cubic_w<T>(dx - T(k - 1));
                if (wd == T(0)) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (wr[i] == T(0)) continue;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (wc[j] == T(0)) continue;
                        tap(df + k - 1, rf + i - 1, cf + j - 1, wd, wr[i], wc[j]);
                    }
                }
            }
        }
    }
}

template <int DIM, typename T> __device__ __forceinline__ Cx<T> tap_value(Cx<T> v, T wd, T wr, T wc) {
    if constexpr (DIM == 2) return cscale(cscale(v, wr), wc);
    else return cscale(cscale(cscale(v, wd), wr), wc);
}
template <int DIM, typename T> __device__ __forceinline__ T tap_weight(T wd, T wr, T wc) {
    // |((1*wd)*wr)*wc|, the real part of tap_value applied to 1+0i
    T w = DIM == 2 ? T(T(1) * wr) * wc : T(T(T(1) * wd) * wr) * wc;
    return w < T(0) ? -w : w;
}

// Scatter target of a tap (projection_utils.h:336-362, 414-443): Friedel flip
// with conjugation for c < 0, out-of-range taps dropped (-1).  On return
// d, r, c hold the post-flip signed coordinates.
template <int DIM>
__device__ __forceinline__ int64_t scatter_index(int N, int H, int& d, int& r, int& c, bool& cj) {
    cj = c < 0;
    if (cj) { c = -c; r = -r; d = -d; }
    if (c >= H) return -1;
    if (r > N / 2 || r < -N / 2 + 1) return -1;
    if (DIM == 3 && (d > N / 2 || d < -N / 2 + 1)) return -1;
    const int re = r < 0 ? N + r : r;
    if (DIM == 2) return (int64_t)re * H + c;
    const int de = d < 0 ? N + d : d;
    return ((int64_t)de * N + re) * H + c;
}
// Hermitian partner of an x = 0 cell (projection_utils.h:398-405, 481-492),
// or -1 when the cell is its own partner.
template <int DIM>
__device__ __forceinline__ int64_t mirror_index(int N, int H, int d, int r) {
    const int r2 = -r < 0 ? N - r : -r;
    const int re = r < 0 ? N + r : r;
    if (DIM == 2) return r2 == re ? -1 : (int64_t)r2 * H;
    const int d2 = -d < 0 ? N - d : -d;
    const int de = d < 0 ? N + d : d;
    return (r2 == re && d2 == de) ? -1 : ((int64_t)d2 * N + r2) * H;
}

// Weight-gradient tap (backprojection_2d_kernels.cpp:440-451,
// backprojection_2d_to_3d_kernels.cpp:476-492): Friedel flip without
// conjugation, zero outside the box.
template <int DIM, typename T>
__device__ __forceinline__ T weight_tap(const T* __restrict__ g, int N, int H, int d, int r, int c) {
    if (c < 0) { c = -c; r = -r; d = -d; }
    if (c >= H) return T(0);
    if (DIM == 3 && (d > N / 2 || d < -N / 2 + 1)) return T(0);
    if (r > N / 2 || r < -N / 2 + 1) return T(0);
    const int re = r < 0 ? N + r : r;
    if (DIM == 2) return g[(int64_t)re * H + c];
    const int de = d < 0 ? N + d : d;
    return g[((int64_t)de * N + re) * H + c];
}
// Always (bi/tri)linear, also for cubic projections
// (backprojection_2d_kernels.cpp:435-469, backprojection_2d_to_3d_kernels.cpp:466-515).
template <int DIM, typename T>
__device__ __forceinline__ T weight_grad_interp(const T* __restrict__ g, int N, int H, const T* x) {
    if constexpr (DIM == 2) {
        T cx, rx;
        const int cf = split(x[0], cx), rf = split(x[1], rx);
        const T p00 = weight_tap<2>(g, N, H, 0, rf, cf), p01 = weight_tap<2>(g, N, H, 0, rf, cf + 1);
        const T p10 = weight_tap<2>(g, N, H, 0, rf + 1, cf), p11 = weight_tap<2>(g, N, H, 0, rf + 1, cf + 1);
        const T p0 = p00 + (p01 - p00) * cx;
        const T p1 = p10 + (p11 - p10) * cx;
        return p0 + (p1 - p0) * rx;
    } else {
        T cx, rx, dx;
        const int cf = split(x[0], cx), rf = split(x[1], rx), df = split(x[2], dx);
        const T p000 = weight_tap<3>(g, N, H, df, rf, cf), p001 = weight_tap<3>(g, N, H, df, rf, cf + 1);
        const T p010 = weight_tap<3>(g, N, H, df, rf + 1, cf), p011 = weight_tap<3>(g, N, H, df, rf + 1, cf + 1);
        const T p100 = weight_tap<3>(g, N, H, df + 1, rf, cf), p101 = weight_tap<3>(g, N, H, df + 1, rf, cf + 1);
        const T p110 = weight_tap<3>(g, N, H, df + 1, rf + 1, cf);
        const T p111 = weight_tap<3>(g, N, H, df + 1, rf + 1, cf + 1);
        const T p00 = p000 + (p001 - p000) * cx;
        const T p01 = p010 + (p011 - p010) * cx;
        const T p10 = p100 + (p101 - p100) * cx;
        const T p11 = p110 + (p111 - p110) * cx;
        const T p0 = p00 + (p01 - p00) * rx;
        const T p1 = p10 + (p11 - p10) * rx;
        return p0 + (p1 - p0) * dx;
    }
}

// ---------------------------------------------------------------- per-pixel geometry
// Pixel q of a pose's active rectangle (Geom::rr0, rnr, rnc): grid row i and
// column j, or false past the rectangle.
__device__ __forceinline__ bool rect_pixel(const Geom& g, int q, int& i, int& j) {
    if (q >= g.rect) return false;
    const int kr = q / g.rnc;
    j = q - kr * g.rnc;
    const int r = g.rr0 + kr;
    i = r >= 0 ? r : r + g.n;
    return true;
}

// Row index -> signed frequency (projection_utils.h:61-64).
template <typename T> __device__ __forceinline__ T freq_of(int i, int n) { return i <= n / 2 ? T(i) : T(i - n); }
// Radius mask (projection_utils.h:69-76): r^2 + c^2 > cutoff^2 in the real type.
template <typename T> __device__ __forceinline__ bool filtered(T r, T c, T cut2) {
    T s = 0;
    s += r * r;
    s += c * c;
    return s > cut2;
}

// Oversampled, rotated sample position (cpu/2d/projection_2d_kernels.cpp:173-178,
// cpu/3d/projection_3d_to_2d_kernels.cpp:175-188).  The oversampling product
// is formed in double and rounded to the real type; the rotation is evaluated
// left to right without contraction.
template <int DIM, typename T>
__device__ __forceinline__ void rotate(const T* __restrict__ R, T r, T c, double os, T* x, T& sc, T& sr) {
    sc = T(double(c) * os);
    sr = T(double(r) * os);
    if constexpr (DIM == 2) {
        x[1] = R[2] * sc + R[3] * sr;
        x[0] = R[0] * sc + R[1] * sr;
        x[2] = T(0);
    } else {
        const T sd = 0.0;
        x[0] = R[0] * sc + R[1] * sr + R[2] * sd;
        x[1] = R[3] * sc + R[4] * sr + R[5] * sd;
        x[2] = R[6] * sc + R[7] * sr + R[8] * sd;
    }
}

__device__ __forceinline__ void sin_cos(float x, float* s, float* c) { sincosf(x, s, c); }
__device__ __forceinline__ void sin_cos(double x, double* s, double* c) { sincos(x, s, c); }

// Shift phase factor (projection_utils.h:82-94): phase accumulated in the real
// type, scaled by k = -2*pi/n in double, rounded back; factor (cos, sin).
template <typename T> __device__ __forceinline__ Cx<T> phase(T r, T c, T s0, T s1, double k) {
    T ph = 0.0;
    ph += r * s0;
    ph += c * s1;
    ph = T(double(ph) * k);
    Cx<T> f;
    sin_cos(ph, &f.im, &f.re);
    return f;
}

// The same phase angle, evaluated with the hardware sine/cosine: the angle is
// turned into revolutions with an error-free product split (1/2pi = C1 + C2),
// reduced to [-1/2, 1/2] exactly, and fed to v_sin/v_cos.  Differs from the
// library sincosf by the hardware units' few-ulp error only.
__device__ __forceinline__ Cx<float> phase_hw(float r, float c, float s0, float s1, double k) {
    float ph = 0.0f;
    ph += r * s0;
    ph += c * s1;
    ph = float(double(ph) * k);
    constexpr float C1 = 0.15915493667125702f;       // fl(1 / 2pi)
    constexpr float C2 = 6.4206382433e-09f;          // 1 / 2pi - C1
    const float h = ph * C1;
    const float e = fmaf(ph, C1, -h) + ph * C2;      // low part of ph / 2pi
    const float t = (h - rintf(h)) + e;
    return {__builtin_amdgcn_cosf(t), __builtin_amdgcn_sinf(t)};
}

// ---------------------------------------------------------------- pose classes
// A sample of pixel (r, c) lies at x = sc a + sr b, with a and b the first two
// columns of the pose matrix (3D) or its two columns (2D).  The tiled kernels
// enumerate a pose's samples through the plane (3D) or the grid (2D) that a
// and b span, which works for every matrix whose Gram matrix
// G = [[a.a, a.b], [a.b, b.b]] has both eigenvalues (the squared singular
// values) in [kScaleMin^2, kScaleMax^2] (tp_launch.hh): rotations, and scaled
// or sheared matrices such as magnification corrections.  Other matrices
// (degenerate ones, strong scalings) take the per-pixel kernels.  Both
// families evaluate this same predicate, with multiplies and adds only, so
// every pose is handled by exactly one of them.
struct PoseGram {
    float aa, bb, ab;
};
__device__ __forceinline__ PoseGram pose_gram3(const float* __restrict__ R) {
    return {R[0] * R[0] + R[3] * R[3] + R[6] * R[6], R[1] * R[1] + R[4] * R[4] + R[7] * R[7],
            R[0] * R[1] + R[3] * R[4] + R[6] * R[7]};
}
// 2D: row-major 2x2, columns (R[0], R[2]) and (R[1], R[3]).
__device__ __forceinline__ PoseGram pose_gram2(const float* __restrict__ R) {
    return {R[0] * R[0] + R[2] * R[2], R[1] * R[1] + R[3] * R[3], R[0] * R[1] + R[2] * R[3]};
}
// Both eigenvalues of G in [lo, hi]: the characteristic polynomial
// p(t) = t^2 - tr t + det is >= 0 at lo and at hi, and its vertex tr/2 lies
// between them.  (NaN matrices fail every comparison: per-pixel kernels.)
__device__ __forceinline__ bool gram_tiled(PoseGram g) {
    constexpr float lo = kScaleMin * kScaleMin, hi = kScaleMax * kScaleMax;
    const float tr = g.aa + g.bb, det = g.aa * g.bb - g.ab * g.ab;
    const float plo = (lo - tr) * lo + det, phi = (hi - tr) * hi + det;
    return plo >= 0.f && phi >= 0.f && tr >= 2.f * lo && tr <= 2.f * hi;
}
// Columns orthonormal to kRotationTol: a rotation (which gram_tiled accepts
// with a wide margin; testing it first spares rotations the other tests).
__device__ __forceinline__ bool gram_is_rotation(PoseGram g) {
    return fabsf(g.aa - 1.0f) <= kRotationTol && fabsf(g.bb - 1.0f) <= kRotationTol && fabsf(g.ab) <= kRotationTol;
}
// The class test of both kernel families.
__device__ __forceinline__ bool gram_takes_tiles(PoseGram g) { return gram_is_rotation(g) || gram_tiled(g); }
__device__ __forceinline__ bool pose_tiled3(const float* __restrict__ R) { return gram_takes_tiles(pose_gram3(R)); }
__device__ __forceinline__ bool pose_tiled2(const float* __restrict__ R) { return gram_takes_tiles(pose_gram2(R)); }
template <int DIM> __device__ __forceinline__ bool pose_tiled_d(const float* __restrict__ R) {
    if constexpr (DIM == 2) return pose_tiled2(R);
    else return pose_tiled3(R);
}
// Largest singular value of a tiled pose (an upper bound): the root of the
// larger eigenvalue of G, slightly widened.
__device__ __forceinline__ float gram_smax(PoseGram g) {
    const float h = 0.5f * (g.aa - g.bb);
    const float lmax = 0.5f * (g.aa + g.bb) + sqrtf(h * h + g.ab * g.ab);
    return sqrtf(lmax) * 1.000001f;
}

// Dual basis of a tiled pose that is not a rotation: the vectors as, bs with
// sc = as . x and sr = bs . x for every x = sc a + sr b of the pose's plane
// (3D, N = 3) or grid (2D, N = 2), i.e. the rows of G^-1 [a b]^T.  A rotation
// (a and b orthonormal to kRotationTol) uses its columns instead; the bounds
// built on them carry a slack that covers that tolerance.
template <int N>
__device__ __forceinline__ void pose_dual(const float* a, const float* b, PoseGram g, float* as, float* bs) {
    const float inv = __builtin_amdgcn_rcpf(g.aa * g.bb - g.ab * g.ab);  // det >= kScaleMin^4
#pragma unroll
    for (int k = 0; k < N; ++k) {
        as[k] = (g.bb * a[k] - g.ab * b[k]) * inv;
        bs[k] = (g.aa * b[k] - g.ab * a[k]) * inv;
    }
}
__device__ __forceinline__ void pose_dual3(const float* __restrict__ R, PoseGram g, float* as, float* bs) {
    const float a[3] = {R[0], R[3], R[6]}, b[3] = {R[1], R[4], R[7]};
    pose_dual<3>(a, b, g, as, bs);
}
__device__ __forceinline__ void pose_dual2(const float* __restrict__ R, PoseGram g, float* as, float* bs) {
    const float a[2] = {R[0], R[2]}, b[2] = {R[1], R[3]};
    pose_dual<2>(a, b, g, as, bs);
}

// ---------------------------------------------------------------- atomics
__device__ __forceinline__ void atomic_add(float* p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_add(double* p, double v) { unsafeAtomicAdd(p, v); }
template <typename T> __device__ __forceinline__ void atomic_add_cx(Cx<T>* p, Cx<T> v) {
    atomic_add(&p->re, v.re);
    atomic_add(&p->im, v.im);
}

// ---------------------------------------------------------------- block reduction
// Sum `vals[0..K)` over a 256-thread block; the result is valid in thread 0.
template <typename T, int K>
__device__ __forceinline__ void block_sum(T (&vals)[K], T (*lds)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
        T v = vals[k];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        vals[k] = v;
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < K; ++k) lds[wave][k] = vals[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = (blockDim.x + 63) >> 6;
        for (int w = 1; w < nw; ++w) {
#pragma unroll
            for (int k = 0; k < K; ++k) vals[k] += lds[w][k];
        }
    }
    __syncthreads();
}

}  // namespace tp
