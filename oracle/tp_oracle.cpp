// TEST INFRASTRUCTURE — NOT PART OF THE PRODUCT.
//
// CPU restatement of the reference torch-projectors CPU kernels (paths below
// are relative to the reference repository).  It is the parity oracle for the
// HIP library and the "port" CPU baseline of bench.py; only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
//
// Arithmetic is restated operation by operation so that, for the same inputs,
// every sample coordinate, stencil index, Friedel decision and per-tap value
// is bit-identical to the reference (compile with -ffp-contract=off, no
// -ffast-math).  Scatter sums use atomics like the reference, so their
// summation order is as nondeterministic as the reference's for >1 thread.
//
// Entry points mirror include/torch_projectors_hip.h with host pointers,
// `tpo_` instead of `tp_`, and `num_threads` (<=0: OpenMP default) in place
// of the stream.  Outputs are zero-filled first, as the reference allocates
// them with torch::zeros.
//
// Pinning (see tests/test_oracle_golden.py): every function below is checked
// against golden vectors produced by the reference's own compiled CPU
// kernels (tests/golden/), and the sampling/interpolation core additionally
// against closed forms (identity rotation = central slice, impulse volumes,
// partition of unity, the adjoint identity).

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>

namespace {

thread_local std::string g_err;

// ------------------------------------------------------------ complex values
// c10::complex operators (torch/headeronly/util/complex.h:195-238): complex*real
// scales both parts; complex*complex is (ac - bd, ad + bc).
template <typename T>
struct Cx {
    T re, im;
};
template <typename T> inline Cx<T> cadd(Cx<T> a, Cx<T> b) { return {a.re + b.re, a.im + b.im}; }
template <typename T> inline Cx<T> csub(Cx<T> a, Cx<T> b) { return {a.re - b.re, a.im - b.im}; }
template <typename T> inline Cx<T> cscale(Cx<T> a, T s) { return {a.re * s, a.im * s}; }
template <typename T> inline Cx<T> cmul(Cx<T> a, Cx<T> b) {
    return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}
template <typename T> inline Cx<T> cconj(Cx<T> a) { return {a.re, -a.im}; }

template <typename T> inline void atomic_add(T* dst, T v) {
#pragma omp atomic update
    *dst += v;
}
template <typename T> inline void atomic_add_cx(Cx<T>* dst, Cx<T> v) {  // atomic_ops.h:25-34
    atomic_add(&dst->re, v.re);
    atomic_add(&dst->im, v.im);
}
// An accumulated value in the accumulator type (exact widening).
template <typename A, typename T> inline Cx<A> widen(Cx<T> v) { return {A(v.re), A(v.im)}; }

// ------------------------------------------------------------ cubic weights
// cubic_kernels.h:25-43 / 50-67: Catmull-Rom a = -0.5.  `a` is of the real
// type but the literals are double, so for float the polynomial is evaluated
// in double and rounded once on return.
template <typename T> inline T cubic_w(T s) {
    const T a = -0.5;
    s = std::abs(s);
    if (s <= 1.0) return (a + 2.0) * s * s * s - (a + 3.0) * s * s + 1.0;
    if (s <= 2.0) return a * s * s * s - 5.0 * a * s * s + 8.0 * a * s - 4.0 * a;
    return 0.0;
}
template <typename T> inline T cubic_dw(T s) {
    const T a = -0.5;
    T sign = (s < 0) ? -1.0 : 1.0;
    s = std::abs(s);
    if (s <= 1.0) return sign * (3.0 * (a + 2.0) * s * s - 2.0 * (a + 3.0) * s);
    if (s <= 2.0) return sign * (3.0 * a * s * s - 10.0 * a * s + 8.0 * a);
    return 0.0;
}

// ------------------------------------------------------------ sampling
// Friedel-aware FFTW-layout fetch with edge replication (fftw_sampling.h:157-190
// for 2D, :211-251 for 3D).  `rec` points at batch b; N = box, H = N/2+1.
template <typename T>
inline Cx<T> fetch2(const Cx<T>* rec, int64_t N, int64_t H, int64_t r, int64_t c) {
    bool cj = false;
    if (c < 0) { c = -c; r = -r; cj = true; }
    c = std::min(c, H - 1);
    r = std::min(N / 2, std::max(r, -N / 2 + 1));
    if (r < 0) r = N + r;
    r = std::min(r, N - 1);
    Cx<T> v = rec[r * H + c];
    return cj ? cconj(v) : v;
}
template <typename T>
inline Cx<T> fetch3(const Cx<T>* rec, int64_t N, int64_t H, int64_t d, int64_t r, int64_t c) {
    bool cj = false;
    if (c < 0) { c = -c; r = -r; d = -d; cj = true; }
    c = std::min(c, H - 1);
    r = std::min(N / 2, std::max(r, -N / 2 + 1));
    d = std::min(N / 2, std::max(d, -N / 2 + 1));
    if (r < 0) r = N + r;
    if (d < 0) d = N + d;
    r = std::min(r, N - 1);
    d = std::min(d, N - 1);
    Cx<T> v = rec[(d * N + r) * H + c];
    return cj ? cconj(v) : v;
}
// Cubic taps are pre-clamped before the fetch (interpolation_kernels.h:245-255, :331-342).
template <typename T>
inline Cx<T> fetch2_cubic(const Cx<T>* rec, int64_t N, int64_t H, int64_t r, int64_t c) {
    if (std::abs(c) >= H) c = (c < 0) ? -(H - 1) : (H - 1);
    r = std::max(-N / 2 + 1, std::min(r, N / 2));
    return fetch2(rec, N, H, r, c);
}
template <typename T>
inline Cx<T> fetch3_cubic(const Cx<T>* rec, int64_t N, int64_t H, int64_t d, int64_t r, int64_t c) {
    if (std::abs(c) >= H) c = (c < 0) ? -(H - 1) : (H - 1);
    r = std::max(-N / 2 + 1, std::min(r, N / 2));
    d = std::max(-N / 2 + 1, std::min(d, N / 2));
    return fetch3(rec, N, H, d, r, c);
}

// ------------------------------------------------------------ interpolation
// Value plus analytic spatial gradient.  x = (c, r) in 2D, (c, r, d) in 3D;
// g[0] = d/dc, g[1] = d/dr, g[2] = d/dd.
template <typename T> struct Interp {
    Cx<T> v;
    Cx<T> g[3];
};

// interpolation_kernels.h:80-134
template <typename T>
inline Interp<T> interp2_linear(const Cx<T>* rec, int64_t N, int64_t H, T r, T c) {
    const int64_t cf = std::floor(c), rf = std::floor(r);
    const T cx = c - cf, rx = r - rf;
    const Cx<T> p00 = fetch2(rec, N, H, rf, cf), p01 = fetch2(rec, N, H, rf, cf + 1);
    const Cx<T> p10 = fetch2(rec, N, H, rf + 1, cf), p11 = fetch2(rec, N, H, rf + 1, cf + 1);
    const Cx<T> p0 = cadd(p00, cscale(csub(p01, p00), cx));
    const Cx<T> p1 = cadd(p10, cscale(csub(p11, p10), cx));
    Interp<T> o;
    o.v = cadd(p0, cscale(csub(p1, p0), rx));
    o.g[1] = cadd(cscale(csub(p10, p00), T(1 - cx)), cscale(csub(p11, p01), cx));
    o.g[0] = cadd(cscale(csub(p01, p00), T(1 - rx)), cscale(csub(p11, p10), rx));
    o.g[2] = {0, 0};
    return o;
}

// interpolation_kernels.h:258-322 (value accumulates ((s*wr)*wc) in r-major order)
template <typename T>
inline Interp<T> interp2_cubic(const Cx<T>* rec, int64_t N, int64_t H, T r, T c, bool grads) {
    const int64_t cf = std::floor(c), rf = std::floor(r);
    const T cx = c - cf, rx = r - rf;
    Interp<T> o;
    o.v = {0, 0};
    o.g[0] = o.g[1] = o.g[2] = {0, 0};
    for (int i = -1; i <= 2; ++i) {
        const T wr = cubic_w<T>(rx - i);
        const T dwr = grads ? cubic_dw<T>(rx - i) : T(0);
        for (int j = -1; j <= 2; ++j) {
            const Cx<T> s = fetch2_cubic(rec, N, H, rf + i, cf + j);
            const T wc = cubic_w<T>(cx - j);
            o.v = cadd(o.v, cscale(cscale(s, wr), wc));
            if (grads) {
                const T dwc = cubic_dw<T>(cx - j);
                o.g[1] = cadd(o.g[1], cscale(cscale(s, dwr), wc));
                o.g[0] = cadd(o.g[0], cscale(cscale(s, wr), dwc));
            }
        }
    }
    return o;
}

// interpolation_kernels.h:142-227
template <typename T>
inline Interp<T> interp3_linear(const Cx<T>* rec, int64_t N, int64_t H, T d, T r, T c) {
    const int64_t df = std::floor(d), rf = std::floor(r), cf = std::floor(c);
    const T dx = d - df, rx = r - rf, cx = c - cf;
    const Cx<T> p000 = fetch3(rec, N, H, df, rf, cf), p001 = fetch3(rec, N, H, df, rf, cf + 1);
    const Cx<T> p010 = fetch3(rec, N, H, df, rf + 1, cf), p011 = fetch3(rec, N, H, df, rf + 1, cf + 1);
    const Cx<T> p100 = fetch3(rec, N, H, df + 1, rf, cf), p101 = fetch3(rec, N, H, df + 1, rf, cf + 1);
    const Cx<T> p110 = fetch3(rec, N, H, df + 1, rf + 1, cf), p111 = fetch3(rec, N, H, df + 1, rf + 1, cf + 1);
    const Cx<T> p00 = cadd(p000, cscale(csub(p001, p000), cx));
    const Cx<T> p01 = cadd(p010, cscale(csub(p011, p010), cx));
    const Cx<T> p10 = cadd(p100, cscale(csub(p101, p100), cx));
    const Cx<T> p11 = cadd(p110, cscale(csub(p111, p110), cx));
    const Cx<T> p0 = cadd(p00, cscale(csub(p01, p00), rx));
    const Cx<T> p1 = cadd(p10, cscale(csub(p11, p10), rx));
    Interp<T> o;
    o.v = cadd(p0, cscale(csub(p1, p0), dx));
    o.g[2] = csub(p1, p0);
    o.g[1] = cadd(cscale(csub(p01, p00), T(1 - dx)), cscale(csub(p11, p10), dx));
    const T a = T(1 - dx) * T(1 - rx), b = T(1 - dx) * rx, e = dx * T(1 - rx), f = dx * rx;
    o.g[0] = cadd(cadd(cadd(cscale(csub(p001, p000), a), cscale(csub(p011, p010), b)),
                       cscale(csub(p101, p100), e)),
                  cscale(csub(p111, p110), f));
    return o;
}

// interpolation_kernels.h:345-425 (accumulates (((s*wd)*wr)*wc) in d, r, c order)
template <typename T>
inline Interp<T> interp3_cubic(const Cx<T>* rec, int64_t N, int64_t H, T d, T r, T c, bool grads) {
    const int64_t df = std::floor(d), rf = std::floor(r), cf = std::floor(c);
    const T dx = d - df, rx = r - rf, cx = c - cf;
    Interp<T> o;
    o.v = {0, 0};
    o.g[0] = o.g[1] = o.g[2] = {0, 0};
    for (int k = -1; k <= 2; ++k) {
        const T wd = cubic_w<T>(dx - k);
        const T dwd = grads ? cubic_dw<T>(dx - k) : T(0);
        for (int i = -1; i <= 2; ++i) {
            const T wr = cubic_w<T>(rx - i);
            const T dwr = grads ? cubic_dw<T>(rx - i) : T(0);
            for (int j = -1; j <= 2; ++j) {
                const Cx<T> s = fetch3_cubic(rec, N, H, df + k, rf + i, cf + j);
                const T wc = cubic_w<T>(cx - j);
                o.v = cadd(o.v, cscale(cscale(cscale(s, wd), wr), wc));
                if (grads) {
                    const T dwc = cubic_dw<T>(cx - j);
                    o.g[2] = cadd(o.g[2], cscale(cscale(cscale(s, dwd), wr), wc));
                    o.g[1] = cadd(o.g[1], cscale(cscale(cscale(s, wd), dwr), wc));
                    o.g[0] = cadd(o.g[0], cscale(cscale(cscale(s, wd), wr), dwc));
                }
            }
        }
    }
    return o;
}

template <int DIM, typename T>
inline Interp<T> interpolate(const Cx<T>* rec, int64_t N, int64_t H, const T* x, bool cubic, bool grads) {
    if constexpr (DIM == 2) {
        return cubic ? interp2_cubic(rec, N, H, x[1], x[0], grads) : interp2_linear(rec, N, H, x[1], x[0]);
    } else {
        return cubic ? interp3_cubic(rec, N, H, x[2], x[1], x[0], grads)
                     : interp3_linear(rec, N, H, x[2], x[1], x[0]);
    }
}

// ------------------------------------------------------------ scatter
// Transposed interpolation (projection_utils.h:172-300).  Calls
// tap(d, r, c, wd, wr, wc) for each stencil cell in the reference's order;
// the callee forms the product ((v*wd)*wr)*wc (2D: (v*wr)*wc, wd unused).
template <int DIM, typename T, typename F>
inline void distribute(const T* x, bool cubic, F&& tap) {
    if constexpr (DIM == 2) {
        const int64_t rf = std::floor(x[1]), cf = std::floor(x[0]);
        const T rx = x[1] - rf, cx = x[0] - cf;
        if (!cubic) {
            tap(0, rf, cf, T(1), T(1 - rx), T(1 - cx));
            tap(0, rf + 1, cf, T(1), rx, T(1 - cx));
            tap(0, rf, cf + 1, T(1), T(1 - rx), cx);
            tap(0, rf + 1, cf + 1, T(1), rx, cx);
        } else {
            for (int ro = -1; ro <= 2; ++ro) {
                const T wr = cubic_w<T>(rx - ro);
                if (wr == 0.0) continue;
                for (int co = -1; co <= 2; ++co) {
                    const T wc = cubic_w<T>(cx - co);
                    if (wc == 0.0) continue;
                    tap(0, rf + ro, cf + co, T(1), wr, wc);
                }
            }
        }
    } else {
        const int64_t df = std::floor(x[2]), rf = std::floor(x[1]), cf = std::floor(x[0]);
        const T dx = x[2] - df, rx = x[1] - rf, cx = x[0] - cf;
        if (!cubic) {
            tap(df, rf, cf, T(1 - dx), T(1 - rx), T(1 - cx));
            tap(df + 1, rf, cf, dx, T(1 - rx), T(1 - cx));
            tap(df, rf + 1, cf, T(1 - dx), rx, T(1 - cx));
            tap(df + 1, rf + 1, cf, dx, rx, T(1 - cx));
            tap(df, rf, cf + 1, T(1 - dx), T(1 - rx), cx);
            tap(df + 1, rf, cf + 1, dx, T(1 - rx), cx);
            tap(df, rf + 1, cf + 1, T(1 - dx), rx, cx);
            tap(df + 1, rf + 1, cf + 1, dx, rx, cx);
        } else {
            for (int dof = -1; dof <= 2; ++dof) {
                const T wd = cubic_w<T>(dx - dof);
                if (wd == 0.0) continue;
                for (int ro = -1; ro <= 2; ++ro) {
                    const T wr = cubic_w<T>(rx - ro);
                    if (wr == 0.0) continue;
                    for (int co = -1; co <= 2; ++co) {
                        const T wc = cubic_w<T>(cx - co);
                        if (wc == 0.0) continue;
                        tap(df + dof, rf + ro, cf + co, wd, wr, wc);
                    }
                }
            }
        }
    }
}

template <int DIM, typename T> inline Cx<T> tap_value(Cx<T> v, T wd, T wr, T wc) {
    if constexpr (DIM == 2) return cscale(cscale(v, wr), wc);
    else return cscale(cscale(cscale(v, wd), wr), wc);
}

// Friedel-aware, out-of-range-dropping index of a scatter target
// (projection_utils.h:336-362, :414-443).  Returns -1 when dropped.
// `conj` reports a Friedel flip; `d,r` (signed, post-flip) are returned for
// the x = 0 mirror.
template <int DIM>
inline int64_t scatter_index(int64_t N, int64_t H, int64_t& d, int64_t& r, int64_t& c, bool& conj) {
    conj = false;
    if (c < 0) { c = -c; r = -r; d = -d; conj = true; }
    if (c >= H) return -1;
    if (r > N / 2 || r < -N / 2 + 1) return -1;
    if (DIM == 3 && (d > N / 2 || d < -N / 2 + 1)) return -1;
    const int64_t re = r < 0 ? N + r : r;
    const int64_t de = d < 0 ? N + d : d;
    if (re >= N || de >= N) return -1;
    return DIM == 2 ? re * H + c : (de * N + re) * H + c;
}
// Partner cell of an x = 0 entry (projection_utils.h:398-405, :481-492), or -1
// when the entry is its own partner (r, and in 3D d, in {0, N/2}).
template <int DIM>
inline int64_t mirror_index(int64_t N, int64_t H, int64_t d, int64_t r) {
    const int64_t r2 = -r < 0 ? N - r : -r;
    const int64_t d2 = -d < 0 ? N - d : -d;
    const int64_t re = r < 0 ? N + r : r;
    const int64_t de = d < 0 ? N + d : d;
    if (DIM == 2 ? (r2 == re) : (r2 == re && d2 == de)) return -1;
    return DIM == 2 ? r2 * H : (d2 * N + r2) * H;
}

// ------------------------------------------------------------ pose helpers
// Row index -> frequency (projection_utils.h:61-64); radius mask (:69-76).
template <typename T> inline T freq_of(int64_t i, int64_t n) { return i <= n / 2 ? T(i) : T(i - n); }
template <typename T> inline bool filtered(T r, T c, T cut2) {
    T s = 0;
    s += r * r;
    s += c * c;
    return s > cut2;
}

// Rotated sample position x = (c, r[, d]) of frequency (r, c)
// (cpu/2d/projection_2d_kernels.cpp:173-178; cpu/3d/projection_3d_to_2d_kernels.cpp:175-188).
template <int DIM, typename T>
inline void rotate(const T* R, T r, T c, double os, T* x, T* sc_out, T* sr_out) {
    const T sc = c * os;
    const T sr = r * os;
    if constexpr (DIM == 2) {
        x[1] = R[2] * sc + R[3] * sr;
        x[0] = R[0] * sc + R[1] * sr;
    } else {
        const T sd = 0.0;
        x[0] = R[0] * sc + R[1] * sr + R[2] * sd;
        x[1] = R[3] * sc + R[4] * sr + R[5] * sd;
        x[2] = R[6] * sc + R[7] * sr + R[8] * sd;
    }
    *sc_out = sc;
    *sr_out = sr;
}

// Shift phase factor (projection_utils.h:82-94): the accumulated phase is of
// the real type, the scaling by -2*pi/n happens in double and is rounded back.
template <typename T> inline Cx<T> phase(T r, T c, T s0, T s1, T n) {
    T ph = 0.0;
    ph += r * s0;
    ph += c * s1;
    ph *= -2.0 * M_PI / n;
    return {std::cos(ph), std::sin(ph)};
}

// at::parallel_for with an OpenMP backend: one contiguous chunk per thread,
// grain max(1, total/(2*threads)) (projection_utils.h:53-55).
template <typename F> void parallel_for_bp(int64_t total, int num_threads, F&& body) {
    const int nt = num_threads > 0 ? num_threads : omp_get_max_threads();
    const int64_t grain = std::max<int64_t>(1, total / (2 * nt));
#pragma omp parallel num_threads(nt)
    {
        int64_t threads = omp_get_num_threads();
        threads = std::min<int64_t>(threads, (total + grain - 1) / grain);
        const int64_t tid = omp_get_thread_num();
        const int64_t chunk = (total + threads - 1) / std::max<int64_t>(threads, 1);
        const int64_t b0 = tid * chunk;
        if (tid < threads && b0 < total) {
            const int64_t b1 = std::min(total, b0 + chunk);
            for (int64_t bp = b0; bp < b1; ++bp) body(bp);
        }
    }
}

struct Common {
    bool cubic;
    double os;
    int has_cut;
    double cut;
};

template <typename T> inline T cutoff_sq(const Common& cm, int64_t n) {
    const T radius = cm.has_cut ? T(cm.cut) : T(n / 2.0);
    return radius * radius;
}

// ------------------------------------------------------------ forward projection
// cpu/2d/projection_2d_kernels.cpp:96-202, cpu/3d/projection_3d_to_2d_kernels.cpp:97-212
template <int DIM, typename T>
void project_forw(const Common& cm, const Cx<T>* rec, int64_t B, int64_t N, int64_t H, const T* rot, int64_t B_rot,
                  int64_t P, const T* shifts, int64_t B_shift, int64_t n, Cx<T>* out, int nthreads) {
    const int64_t hp = n / 2 + 1;
    const int64_t RS = DIM == 2 ? 4 : 9;
    const int64_t vol = DIM == 2 ? N * H : N * N * H;
    std::memset(out, 0, sizeof(Cx<T>) * B * P * n * hp);
    const T cut2 = cutoff_sq<T>(cm, n);
    parallel_for_bp(B * P, nthreads, [&](int64_t bp) {
        const int64_t b = bp / P, p = bp % P;
        const T* R = rot + ((B_rot == 1 ? 0 : b) * P + p) * RS;
        const T* S = shifts ? shifts + ((B_shift == 1 ? 0 : b) * P + p) * 2 : nullptr;
        const Cx<T>* rb = rec + b * vol;
        for (int64_t i = 0; i < n; ++i) {
            for (int64_t j = 0; j < hp; ++j) {
                const T r = freq_of<T>(i, n), c = T(j);
                if (filtered(r, c, cut2)) continue;
                T x[3], sc, sr;
                rotate<DIM>(R, r, c, cm.os, x, &sc, &sr);
                Cx<T> v = interpolate<DIM>(rb, N, H, x, cm.cubic, false).v;
                if (S) v = cmul(v, phase<T>(r, c, S[0], S[1], T(n)));
                out[((b * P + p) * n + i) * hp + j] = v;
            }
        }
    });
}

// ------------------------------------------------------------ projection backward
// cpu/2d/projection_2d_kernels.cpp:209-375, cpu/3d/projection_3d_to_2d_kernels.cpp:219-402
// A: accumulator type of the reconstruction gradient (T = the reference; double
// for fp32 inputs = the exact sum of the same fp32 tap values, see tpo_*_wide).
template <int DIM, typename T, typename A = T>
void project_back(const Common& cm, const Cx<T>* gproj, int64_t B, int64_t P, int64_t n, int64_t hp,
                  const Cx<T>* rec, int64_t N, int64_t H, const T* rot, int64_t B_rot, const T* shifts,
                  int64_t B_shift, Cx<A>* grec, T* grot, T* gshift, int nthreads) {
    const int64_t RS = DIM == 2 ? 4 : 9;
    const int64_t vol = DIM == 2 ? N * H : N * N * H;
    std::memset(grec, 0, sizeof(Cx<A>) * B * vol);
    if (grot) std::memset(grot, 0, sizeof(T) * B_rot * P * RS);
    if (gshift) std::memset(gshift, 0, sizeof(T) * B_shift * P * 2);
    const T cut2 = cutoff_sq<T>(cm, n);
    parallel_for_bp(B * P, nthreads, [&](int64_t bp) {
        const int64_t b = bp / P, p = bp % P;
        const int64_t rb_idx = B_rot == 1 ? 0 : b, sb_idx = B_shift == 1 ? 0 : b;
        const T* R = rot + (rb_idx * P + p) * RS;
        const T* S = shifts ? shifts + (sb_idx * P + p) * 2 : nullptr;
        const Cx<T>* rb = rec + b * vol;
        Cx<A>* gb = grec + b * vol;
        T lrot[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
        T lsh[2] = {0, 0};
        for (int64_t i = 0; i < n; ++i) {
            for (int64_t j = 0; j < hp; ++j) {
                const T r = freq_of<T>(i, n), c = T(j);
                if (filtered(r, c, cut2)) continue;
                if (j == 0 && i >= n / 2) continue;  // Friedel half of the x = 0 line
                T x[3], sc, sr;
                rotate<DIM>(R, r, c, cm.os, x, &sc, &sr);
                const Cx<T> rec_val = interpolate<DIM>(rb, N, H, x, cm.cubic, false).v;
                const Cx<T> g0 = gproj[((b * P + p) * n + i) * hp + j];
                Cx<T> g = g0;
                if (S) g = cmul(g, phase<T>(-r, -c, S[0], S[1], T(n)));
                distribute<DIM, T>(x, cm.cubic, [&](int64_t d, int64_t rr, int64_t cc, T wd, T wr, T wc) {
                    bool cj;
                    const int64_t idx = scatter_index<DIM>(N, H, d, rr, cc, cj);
                    if (idx < 0) return;
                    const Cx<T> v = tap_value<DIM, T>(g, wd, wr, wc);
                    atomic_add_cx(&gb[idx], widen<A>(cj ? cconj(v) : v));
                });
                if (grot) {
                    const Interp<T> it = interpolate<DIM>(rb, N, H, x, cm.cubic, true);
                    const T s[3] = {sc, sr, T(0.0)};
                    const int rows = DIM;  // row 0 <- d/dc, row 1 <- d/dr, row 2 <- d/dd
                    for (int row = 0; row < rows; ++row)
                        for (int k = 0; k < DIM; ++k)
                            lrot[row * DIM + k] += cmul(g, cconj(cscale(it.g[row], s[k]))).re;
                }
                if (gshift) {
                    Cx<T> mod = rec_val;
                    if (S) mod = cmul(rec_val, phase<T>(r, c, S[0], S[1], T(n)));
                    const Cx<T> kr = {T(0), T(-2.0 * M_PI * r / n)};
                    const Cx<T> kc = {T(0), T(-2.0 * M_PI * c / n)};
                    lsh[0] += cmul(g0, cconj(cmul(kr, mod))).re;
                    lsh[1] += cmul(g0, cconj(cmul(kc, mod))).re;
                }
            }
        }
        if (grot)
            for (int k = 0; k < RS; ++k) atomic_add(&grot[(rb_idx * P + p) * RS + k], lrot[k]);
        if (gshift)
            for (int k = 0; k < 2; ++k) atomic_add(&gshift[(sb_idx * P + p) * 2 + k], lsh[k]);
    });
}

// ------------------------------------------------------------ backprojection
// cpu/2d/backprojection_2d_kernels.cpp:99-282, cpu/3d/backprojection_2d_to_3d_kernels.cpp:98-303
int64_t rec_box(int64_t n, double os) {
    const int64_t raw = static_cast<int64_t>(std::ceil(n * os));
    return raw + (raw % 2);
}

// A: accumulator type of the data and weight volumes (as project_back).
template <int DIM, typename T, typename A = T>
void backproject_forw(const Common& cm, const Cx<T>* proj, int64_t B, int64_t P, int64_t n, int64_t hp,
                      const T* weights, const T* rot, int64_t B_rot, const T* shifts, int64_t B_shift,
                      Cx<A>* data, A* wrec, int nthreads) {
    const int64_t N = rec_box(n, cm.os), H = N / 2 + 1;
    const int64_t RS = DIM == 2 ? 4 : 9;
    const int64_t vol = DIM == 2 ? N * H : N * N * H;
    std::memset(data, 0, sizeof(Cx<A>) * B * vol);
    if (wrec) std::memset(wrec, 0, sizeof(A) * B * vol);
    const T cut2 = cutoff_sq<T>(cm, n);
    parallel_for_bp(B * P, nthreads, [&](int64_t bp) {
        const int64_t b = bp / P, p = bp % P;
        const T* R = rot + ((B_rot == 1 ? 0 : b) * P + p) * RS;
        const T* S = shifts ? shifts + ((B_shift == 1 ? 0 : b) * P + p) * 2 : nullptr;
        Cx<A>* db = data + b * vol;
        A* wb = wrec ? wrec + b * vol : nullptr;
        for (int64_t i = 0; i < n; ++i) {
            for (int64_t j = 0; j < hp; ++j) {
                const T r = freq_of<T>(i, n), c = T(j);
                if (filtered(r, c, cut2)) continue;
                if (j == 0 && i >= n / 2) continue;
                T x[3], sc, sr;
                rotate<DIM>(R, r, c, cm.os, x, &sc, &sr);
                const int64_t pix = ((b * P + p) * n + i) * hp + j;
                Cx<T> v = proj[pix];
                if (S) v = cmul(v, cconj(phase<T>(r, c, S[0], S[1], T(n))));
                // accumulate_*_data: Friedel-aware scatter plus the x = 0 mirror
                // (projection_utils.h:371-406, :451-493)
                distribute<DIM, T>(x, cm.cubic, [&](int64_t d, int64_t rr, int64_t cc, T wd, T wr, T wc) {
                    bool cj;
                    const int64_t idx = scatter_index<DIM>(N, H, d, rr, cc, cj);
                    if (idx < 0) return;
                    const Cx<T> tv = tap_value<DIM, T>(v, wd, wr, wc);
                    const Cx<T> fv = cj ? cconj(tv) : tv;
                    atomic_add_cx(&db[idx], widen<A>(fv));
                    if (cc == 0) {
                        const int64_t m = mirror_index<DIM>(N, H, d, rr);
                        if (m >= 0) atomic_add_cx(&db[m], widen<A>(cconj(fv)));
                    }
                });
                // weight lambda (cpu/2d/backprojection_2d_kernels.cpp:236-264,
                // cpu/3d/backprojection_2d_to_3d_kernels.cpp:245-285): |tap weight|
                // times the pixel weight, same flip (no conj) and mirror.
                if (wb && weights) {
                    const T w = weights[pix];
                    distribute<DIM, T>(x, cm.cubic, [&](int64_t d, int64_t rr, int64_t cc, T wd, T wr, T wc) {
                        const T fw = w * std::abs(tap_value<DIM, T>(Cx<T>{T(1.0), T(0.0)}, wd, wr, wc).re);
                        bool cj;
                        const int64_t idx = scatter_index<DIM>(N, H, d, rr, cc, cj);
                        if (idx < 0) return;
                        atomic_add(&wb[idx], A(fw));
                        if (cc == 0) {
                            const int64_t m = mirror_index<DIM>(N, H, d, rr);
                            if (m >= 0) atomic_add(&wb[m], A(fw));
                        }
                    });
                }
            }
        }
    });
}

// ------------------------------------------------------------ backprojection backward
// cpu/2d/backprojection_2d_kernels.cpp:291-537, cpu/3d/backprojection_2d_to_3d_kernels.cpp:312-590
template <int DIM, typename T>
inline T sample_weight_grad(const T* g, int64_t N, int64_t H, int64_t d, int64_t r, int64_t c) {
    // Friedel flip without conjugation, zero outside (…_2d_kernels.cpp:440-451, …_3d_kernels.cpp:476-492)
    if (c < 0) { c = -c; r = -r; d = -d; }
    if (c >= H) return 0.0;
    if (DIM == 3 && (d > N / 2 || d < -N / 2 + 1)) return 0.0;
    if (r > N / 2 || r < -N / 2 + 1) return 0.0;
    const int64_t de = d < 0 ? N + d : d;
    const int64_t re = r < 0 ? N + r : r;
    if (de >= N || re >= N) return 0.0;
    return DIM == 2 ? g[re * H + c] : g[(de * N + re) * H + c];
}

template <int DIM, typename T>
inline T weight_grad_interp(const T* g, int64_t N, int64_t H, const T* x) {
    if constexpr (DIM == 2) {
        const int64_t cf = std::floor(x[0]), rf = std::floor(x[1]);
        const T cx = x[0] - cf, rx = x[1] - rf;
        const T p00 = sample_weight_grad<2>(g, N, H, 0, rf, cf), p01 = sample_weight_grad<2>(g, N, H, 0, rf, cf + 1);
        const T p10 = sample_weight_grad<2>(g, N, H, 0, rf + 1, cf);
        const T p11 = sample_weight_grad<2>(g, N, H, 0, rf + 1, cf + 1);
        const T p0 = p00 + (p01 - p00) * cx;
        const T p1 = p10 + (p11 - p10) * cx;
        return p0 + (p1 - p0) * rx;
    } else {
        const int64_t cf = std::floor(x[0]), rf = std::floor(x[1]), df = std::floor(x[2]);
        const T cx = x[0] - cf, rx = x[1] - rf, dx = x[2] - df;
        const T p000 = sample_weight_grad<3>(g, N, H, df, rf, cf);
        const T p001 = sample_weight_grad<3>(g, N, H, df, rf, cf + 1);
        const T p010 = sample_weight_grad<3>(g, N, H, df, rf + 1, cf);
        const T p011 = sample_weight_grad<3>(g, N, H, df, rf + 1, cf + 1);
        const T p100 = sample_weight_grad<3>(g, N, H, df + 1, rf, cf);
        const T p101 = sample_weight_grad<3>(g, N, H, df + 1, rf, cf + 1);
        const T p110 = sample_weight_grad<3>(g, N, H, df + 1, rf + 1, cf);
        const T p111 = sample_weight_grad<3>(g, N, H, df + 1, rf + 1, cf + 1);
        const T p00 = p000 + (p001 - p000) * cx;
        const T p01 = p010 + (p011 - p010) * cx;
        const T p10 = p100 + (p101 - p100) * cx;
        const T p11 = p110 + (p111 - p110) * cx;
        const T p0 = p00 + (p01 - p00) * rx;
        const T p1 = p10 + (p11 - p10) * rx;
        return p0 + (p1 - p0) * dx;
    }
}

template <int DIM, typename T>
void backproject_back(const Common& cm, const Cx<T>* gdata, const T* gw, int64_t N, int64_t H, const Cx<T>* proj,
                      int64_t B, int64_t P, int64_t n, int64_t hp, const T* weights, const T* rot, int64_t B_rot,
                      const T* shifts, int64_t B_shift, Cx<T>* gproj, T* gweights, T* grot, T* gshift,
                      int nthreads) {
    const int64_t RS = DIM == 2 ? 4 : 9;
    const int64_t vol = DIM == 2 ? N * H : N * N * H;
    std::memset(gproj, 0, sizeof(Cx<T>) * B * P * n * hp);
    if (gweights) std::memset(gweights, 0, sizeof(T) * B * P * n * hp);
    if (grot) std::memset(grot, 0, sizeof(T) * B_rot * P * RS);
    if (gshift) std::memset(gshift, 0, sizeof(T) * B_shift * P * 2);
    const T cut2 = cutoff_sq<T>(cm, n);
    parallel_for_bp(B * P, nthreads, [&](int64_t bp) {
        const int64_t b = bp / P, p = bp % P;
        const int64_t rb_idx = B_rot == 1 ? 0 : b, sb_idx = B_shift == 1 ? 0 : b;
        const T* R = rot + (rb_idx * P + p) * RS;
        const T* S = shifts ? shifts + (sb_idx * P + p) * 2 : nullptr;
        const Cx<T>* gdb = gdata + b * vol;
        const T* gwb = gw ? gw + b * vol : nullptr;
        T lrot[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
        T lsh[2] = {0, 0};
        for (int64_t i = 0; i < n; ++i) {
            for (int64_t j = 0; j < hp; ++j) {
                const T r = freq_of<T>(i, n), c = T(j);
                if (filtered(r, c, cut2)) continue;
                if (j == 0 && i >= n / 2) continue;
                T x[3], sc, sr;
                rotate<DIM>(R, r, c, cm.os, x, &sc, &sr);
                const int64_t pix = ((b * P + p) * n + i) * hp + j;
                const Cx<T> val = interpolate<DIM>(gdb, N, H, x, cm.cubic, false).v;
                gproj[pix] = S ? cmul(val, phase<T>(r, c, S[0], S[1], T(n))) : val;
                if (gwb && gweights) gweights[pix] = weight_grad_interp<DIM, T>(gwb, N, H, x);
                if (grot) {
                    const Interp<T> it = interpolate<DIM>(gdb, N, H, x, cm.cubic, true);
                    Cx<T> pv = proj[pix];
                    if (S) pv = cmul(pv, cconj(phase<T>(r, c, S[0], S[1], T(n))));
                    const T s[3] = {sc, sr, T(0.0)};
                    for (int row = 0; row < DIM; ++row)
                        for (int k = 0; k < DIM; ++k)
                            lrot[row * DIM + k] += cmul(pv, cconj(cscale(it.g[row], s[k]))).re;
                }
                if (gshift) {
                    const Cx<T> rv = interpolate<DIM>(gdb, N, H, x, cm.cubic, false).v;
                    Cx<T> pv = proj[pix];
                    if (S) pv = cmul(pv, cconj(phase<T>(r, c, S[0], S[1], T(n))));
                    const Cx<T> kr = {T(0), T(-2.0 * M_PI * r / n)};
                    const Cx<T> kc = {T(0), T(-2.0 * M_PI * c / n)};
                    lsh[0] += cmul(pv, cconj(cmul(kr, rv))).re;
                    lsh[1] += cmul(pv, cconj(cmul(kc, rv))).re;
                }
            }
        }
        if (grot)
            for (int k = 0; k < RS; ++k) atomic_add(&grot[(rb_idx * P + p) * RS + k], lrot[k]);
        if (gshift)
            for (int k = 0; k < 2; ++k) atomic_add(&gshift[(sb_idx * P + p) * 2 + k], lsh[k]);
    });
}

// ------------------------------------------------------------ argument checks
bool fail(const std::string& m) {
    g_err = m;
    return false;
}
bool check_common(int dtype, int interp, int64_t B, int64_t B_rot, int64_t P, const void* shifts, int64_t B_shift) {
    if (dtype != 0 && dtype != 1) return fail("dtype must be TP_F32 or TP_F64");
    if (interp != 0 && interp != 1) return fail("Supported interpolation methods: 'linear', 'cubic'");
    if (B < 0 || P < 0) return fail("negative size");
    if (B_rot != B && B_rot != 1) return fail("Batch size of rotations must be 1 or same as reconstruction");
    if (shifts && B_shift != B && B_shift != 1) return fail("Batch size of shifts must be 1 or same as reconstruction");
    return true;
}

}  // namespace

#define DISPATCH_T(dtype, ...)                \
    do {                                      \
        if ((dtype) == 0) {                   \
            using T = float;                  \
            __VA_ARGS__;                      \
        } else {                              \
            using T = double;                 \
            __VA_ARGS__;                      \
        }                                     \
    } while (0)

extern "C" {

const char* tpo_last_error(void) { return g_err.c_str(); }

int64_t tpo_backproject_rec_boxsize(int64_t proj_boxsize, double oversampling) {
    return rec_box(proj_boxsize, oversampling);
}

int tpo_project_2d_forw(int dtype, const void* rec, int64_t B, int64_t N, int64_t H, const void* rot, int64_t B_rot,
                        int64_t P, const void* shifts, int64_t B_shift, int64_t n, int interp, double os,
                        int has_cut, double cut, void* out, int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, project_forw<2, T>(cm, (const Cx<T>*)rec, B, N, H, (const T*)rot, B_rot, P, (const T*)shifts,
                                         B_shift, n, (Cx<T>*)out, nthreads));
    return 0;
}

int tpo_project_3d_to_2d_forw(int dtype, const void* rec, int64_t B, int64_t D, int64_t N, int64_t H,
                              const void* rot, int64_t B_rot, int64_t P, const void* shifts, int64_t B_shift,
                              int64_t n, int interp, double os, int has_cut, double cut, void* out, int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    if (D != N) return fail("reconstruction depth must equal its height"), 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, project_forw<3, T>(cm, (const Cx<T>*)rec, B, N, H, (const T*)rot, B_rot, P, (const T*)shifts,
                                         B_shift, n, (Cx<T>*)out, nthreads));
    return 0;
}

int tpo_project_2d_back(int dtype, const void* gproj, int64_t B, int64_t P, int64_t n, int64_t hp, const void* rec,
                        int64_t N, int64_t H, const void* rot, int64_t B_rot, const void* shifts, int64_t B_shift,
                        int interp, double os, int has_cut, double cut, void* grec, void* grot, void* gshift,
                        int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, project_back<2, T>(cm, (const Cx<T>*)gproj, B, P, n, hp, (const Cx<T>*)rec, N, H,
                                         (const T*)rot, B_rot, (const T*)shifts, B_shift, (Cx<T>*)grec, (T*)grot,
                                         shifts ? (T*)gshift : nullptr, nthreads));
    return 0;
}

int tpo_project_3d_to_2d_back(int dtype, const void* gproj, int64_t B, int64_t P, int64_t n, int64_t hp,
                              const void* rec, int64_t D, int64_t N, int64_t H, const void* rot, int64_t B_rot,
                              const void* shifts, int64_t B_shift, int interp, double os, int has_cut, double cut,
                              void* grec, void* grot, void* gshift, int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    if (D != N) return fail("reconstruction depth must equal its height"), 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, project_back<3, T>(cm, (const Cx<T>*)gproj, B, P, n, hp, (const Cx<T>*)rec, N, H,
                                         (const T*)rot, B_rot, (const T*)shifts, B_shift, (Cx<T>*)grec, (T*)grot,
                                         shifts ? (T*)gshift : nullptr, nthreads));
    return 0;
}

int tpo_backproject_2d_forw(int dtype, const void* proj, int64_t B, int64_t P, int64_t n, int64_t hp,
                            const void* weights, const void* rot, int64_t B_rot, const void* shifts, int64_t B_shift,
                            int interp, double os, int has_cut, double cut, void* data, void* wrec, int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, backproject_forw<2, T>(cm, (const Cx<T>*)proj, B, P, n, hp, (const T*)weights, (const T*)rot,
                                             B_rot, (const T*)shifts, B_shift, (Cx<T>*)data,
                                             (T*)wrec, nthreads));
    return 0;
}

int tpo_backproject_2d_to_3d_forw(int dtype, const void* proj, int64_t B, int64_t P, int64_t n, int64_t hp,
                                  const void* weights, const void* rot, int64_t B_rot, const void* shifts,
                                  int64_t B_shift, int interp, double os, int has_cut, double cut, void* data,
                                  void* wrec, int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, backproject_forw<3, T>(cm, (const Cx<T>*)proj, B, P, n, hp, (const T*)weights, (const T*)rot,
                                             B_rot, (const T*)shifts, B_shift, (Cx<T>*)data,
                                             (T*)wrec, nthreads));
    return 0;
}

int tpo_backproject_2d_back(int dtype, const void* gdata, const void* gw, int64_t N, int64_t H, const void* proj,
                            int64_t B, int64_t P, int64_t n, int64_t hp, const void* weights, const void* rot,
                            int64_t B_rot, const void* shifts, int64_t B_shift, int interp, double os, int has_cut,
                            double cut, void* gproj, void* gweights, void* grot, void* gshift, int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, backproject_back<2, T>(cm, (const Cx<T>*)gdata, (const T*)gw, N, H, (const Cx<T>*)proj, B, P,
                                             n, hp, (const T*)weights, (const T*)rot, B_rot, (const T*)shifts,
                                             B_shift, (Cx<T>*)gproj, weights ? (T*)gweights : nullptr, (T*)grot,
                                             shifts ? (T*)gshift : nullptr, nthreads));
    return 0;
}

int tpo_backproject_2d_to_3d_back(int dtype, const void* gdata, const void* gw, int64_t N, int64_t H,
                                  const void* proj, int64_t B, int64_t P, int64_t n, int64_t hp, const void* weights,
                                  const void* rot, int64_t B_rot, const void* shifts, int64_t B_shift, int interp,
                                  double os, int has_cut, double cut, void* gproj, void* gweights, void* grot,
                                  void* gshift, int nthreads) {
    if (!check_common(dtype, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    DISPATCH_T(dtype, backproject_back<3, T>(cm, (const Cx<T>*)gdata, (const T*)gw, N, H, (const Cx<T>*)proj, B, P,
                                             n, hp, (const T*)weights, (const T*)rot, B_rot, (const T*)shifts,
                                             B_shift, (Cx<T>*)gproj, weights ? (T*)gweights : nullptr, (T*)grot,
                                             shifts ? (T*)gshift : nullptr, nthreads));
    return 0;
}

// The scatters of fp32 inputs summed in double: every sample coordinate,
// stencil decision and fp32 tap value is the reference's, and each cell is the
// exact sum of those values (to double rounding) instead of one fp32 order of
// it.  The reference's fp32 atomics may add in any order, so this is the value
// every order approximates; the tests' per-cell scatter bar is taken against
// it.  Outputs: complex128 / float64 volumes.
int tpo_project_2d_back_wide(const void* gproj, int64_t B, int64_t P, int64_t n, int64_t hp, const void* rec,
                             int64_t N, int64_t H, const void* rot, int64_t B_rot, const void* shifts,
                             int64_t B_shift, int interp, double os, int has_cut, double cut, void* grec,
                             int nthreads) {
    if (!check_common(0, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    project_back<2, float, double>(cm, (const Cx<float>*)gproj, B, P, n, hp, (const Cx<float>*)rec, N, H,
                                   (const float*)rot, B_rot, (const float*)shifts, B_shift, (Cx<double>*)grec,
                                   nullptr, nullptr, nthreads);
    return 0;
}

int tpo_project_3d_to_2d_back_wide(const void* gproj, int64_t B, int64_t P, int64_t n, int64_t hp,
                                   const void* rec, int64_t D, int64_t N, int64_t H, const void* rot, int64_t B_rot,
                                   const void* shifts, int64_t B_shift, int interp, double os, int has_cut,
                                   double cut, void* grec, int nthreads) {
    if (!check_common(0, interp, B, B_rot, P, shifts, B_shift)) return 1;
    if (D != N) return fail("reconstruction depth must equal its height"), 1;
    const Common cm{interp == 1, os, has_cut, cut};
    project_back<3, float, double>(cm, (const Cx<float>*)gproj, B, P, n, hp, (const Cx<float>*)rec, N, H,
                                   (const float*)rot, B_rot, (const float*)shifts, B_shift, (Cx<double>*)grec,
                                   nullptr, nullptr, nthreads);
    return 0;
}

int tpo_backproject_2d_forw_wide(const void* proj, int64_t B, int64_t P, int64_t n, int64_t hp,
                                 const void* weights, const void* rot, int64_t B_rot, const void* shifts,
                                 int64_t B_shift, int interp, double os, int has_cut, double cut, void* data,
                                 void* wrec, int nthreads) {
    if (!check_common(0, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    backproject_forw<2, float, double>(cm, (const Cx<float>*)proj, B, P, n, hp, (const float*)weights,
                                       (const float*)rot, B_rot, (const float*)shifts, B_shift, (Cx<double>*)data,
                                       (double*)wrec, nthreads);
    return 0;
}

int tpo_backproject_2d_to_3d_forw_wide(const void* proj, int64_t B, int64_t P, int64_t n, int64_t hp,
                                       const void* weights, const void* rot, int64_t B_rot, const void* shifts,
                                       int64_t B_shift, int interp, double os, int has_cut, double cut, void* data,
                                       void* wrec, int nthreads) {
    if (!check_common(0, interp, B, B_rot, P, shifts, B_shift)) return 1;
    const Common cm{interp == 1, os, has_cut, cut};
    backproject_forw<3, float, double>(cm, (const Cx<float>*)proj, B, P, n, hp, (const float*)weights,
                                       (const float*)rot, B_rot, (const float*)shifts, B_shift, (Cx<double>*)data,
                                       (double*)wrec, nthreads);
    return 0;
}

}  // extern "C"
