// Backprojection (scatter) and its gradient (gather) for the 2D->2D and
// 2D->3D operators.
//
//   k_backproject_forw  replaces backproject_2d_forw_cpu / backproject_2d_to_3d_forw_cpu
//                       (cpu/2d/backprojection_2d_kernels.cpp:99-282,
//                        cpu/3d/backprojection_2d_to_3d_kernels.cpp:98-303)
//   k_backproject_back  replaces backproject_2d_back_cpu / backproject_2d_to_3d_back_cpu
//                       (cpu/2d/backprojection_2d_kernels.cpp:291-537,
//                        cpu/3d/backprojection_2d_to_3d_kernels.cpp:312-590)
#include "tp_device.hh"
#include "tp_launch.hh"

namespace tp {

namespace {

constexpr double kTwoPi = 6.283185307179586476925286766559;

// One projection pixel: v = proj * conj(phase) is spread over the transposed
// stencil into the data volume, |tap weight| * w into the weight volume,
// Friedel-aware, out-of-range taps dropped, and every x = 0 target also feeds
// its Hermitian partner (projection_utils.h:371-406, 451-493; weight lambdas
// cpu/3d/backprojection_2d_to_3d_kernels.cpp:245-285).
template <int DIM, typename T, bool CUBIC, bool WEIGHTS>
__device__ __forceinline__ void backproject_pixel(const Geom& g, Cx<T> v, T wpix, const T* __restrict__ R,
                                                  const T* __restrict__ S, T r, T c, Cx<T>* __restrict__ db,
                                                  T* __restrict__ wb) {
    T x[3], sc, sr;
    rotate<DIM>(R, r, c, g.os, x, sc, sr);
    if (S) v = cmul(v, cconj(phase<T>(r, c, S[0], S[1], g.phase_k)));
    const int N = g.N, H = g.H;
    distribute<DIM, T, CUBIC>(x, [&](int d, int rr, int cc, T wd, T wr, T wc) {
        bool cj;
        const int64_t idx = scatter_index<DIM>(N, H, d, rr, cc, cj);
        if (idx < 0) return;
        Cx<T> tv = tap_value<DIM, T>(v, wd, wr, wc);
        if (cj) tv.im = -tv.im;
        atomic_add_cx(&db[idx], tv);
        const int64_t m = cc == 0 ? mirror_index<DIM>(N, H, d, rr) : -1;
        if (m >= 0) atomic_add_cx(&db[m], cconj(tv));
        if (WEIGHTS) {
            const T fw = wpix * tap_weight<DIM, T>(wd, wr, wc);
            atomic_add(&wb[idx], fw);
            if (m >= 0) atomic_add(&wb[m], fw);
        }
    });
}

// One lane per projection pixel, float atomics into the volumes.
template <int DIM, typename T, bool CUBIC, bool WEIGHTS>
__global__ __launch_bounds__(kBlock) void k_backproject_forw(Geom g, const Cx<T>* __restrict__ proj,
                                                             const T* __restrict__ weights,
                                                             const T* __restrict__ rot, const T* __restrict__ shifts,
                                                             Cx<T>* __restrict__ data, T* __restrict__ wrec) {
    constexpr int RS = DIM * DIM;
    const T cut2 = T(g.cut2);
    for (int64_t w = blockIdx.x; w < g.work; w += gridDim.x) {
        const int64_t bp = w / g.chunks;
        int i = 0, j = 0;
        if (!rect_pixel(g, int(w - bp * g.chunks) * kBlock + int(threadIdx.x), i, j)) continue;
        const int pix = i * g.hp + j;
        const int64_t b = bp / g.P, p = bp - b * g.P;
        const T r = freq_of<T>(i, g.n), c = T(j);
        if (filtered(r, c, cut2) || (j == 0 && i >= g.n / 2)) continue;
        const T* R = rot + ((g.B_rot == 1 ? 0 : b) * g.P + p) * RS;
        const T* S = shifts ? shifts + ((g.B_shift == 1 ? 0 : b) * g.P + p) * 2 : nullptr;
        const int64_t pidx = bp * g.npix + pix;
        backproject_pixel<DIM, T, CUBIC, WEIGHTS>(g, proj[pidx], WEIGHTS ? weights[pidx] : T(0), R, S, r, c,
                                                  data + b * g.vol, WEIGHTS ? wrec + b * g.vol : nullptr);
    }
}

// The poses of an fp32 backprojection that the tiled kernels do not take (the tiled
// scatter has accumulated the others).  One block per pose.
template <int DIM, bool CUBIC, bool WEIGHTS>
__global__ __launch_bounds__(kBlock) void k_backproject_forw_rest(Geom g, const Cx<float>* __restrict__ proj,
                                                                  const float* __restrict__ weights,
                                                                  const float* __restrict__ rot,
                                                                  const float* __restrict__ shifts,
                                                                  Cx<float>* __restrict__ data,
                                                                  float* __restrict__ wrec) {
    constexpr int RS = DIM * DIM;
    const float cut2 = float(g.cut2);
    for (int64_t bp = blockIdx.x; bp < g.B * g.P; bp += gridDim.x) {
        const int64_t b = bp / g.P, p = bp - b * g.P;
        const float* R = rot + ((g.B_rot == 1 ? 0 : b) * g.P + p) * RS;
        if (pose_tiled_d<DIM>(R)) continue;
        const float* S = shifts ? shifts + ((g.B_shift == 1 ? 0 : b) * g.P + p) * 2 : nullptr;
        for (int q = threadIdx.x; q < g.rect; q += kBlock) {
            int i, j;
            rect_pixel(g, q, i, j);
            const int pix = i * g.hp + j;
            const float r = freq_of<float>(i, g.n), c = float(j);
            if (filtered(r, c, cut2) || (j == 0 && i >= g.n / 2)) continue;
            const int64_t pidx = bp * g.npix + pix;
            backproject_pixel<DIM, float, CUBIC, WEIGHTS>(g, proj[pidx], WEIGHTS ? weights[pidx] : 0.f, R, S, r, c,
                                                          data + b * g.vol, WEIGHTS ? wrec + b * g.vol : nullptr);
        }
    }
}

// Gradient of the backprojection: grad_proj gathers grad_data_rec with the
// forward phase; grad_weights gathers grad_weight_rec (always (bi/tri)linear,
// Friedel flip without conjugation, zero outside); rotation and shift
// gradients pair the conj-phased projection with the spatial derivative /
// value of grad_data_rec (backprojection_2d_to_3d_kernels.cpp:451-567).
// REST (fp32): tiled poses (pose_tiled_d) were computed by the tiled gather
// into zero-filled outputs and are skipped here.
template <int DIM, typename T, bool CUBIC, bool WG, bool ROT, bool SHIFT, bool REST>
__global__ __launch_bounds__(kBlock) void k_backproject_back(Geom g, const Cx<T>* __restrict__ gdata,
                                                             const T* __restrict__ gw, const Cx<T>* __restrict__ proj,
                                                             const T* __restrict__ rot, const T* __restrict__ shifts,
                                                             Cx<T>* __restrict__ gproj, T* __restrict__ gweights,
                                                             T* __restrict__ grot, T* __restrict__ gshift) {
    constexpr int RS = DIM * DIM;
    constexpr int K = RS + 2;
    __shared__ T red[kBlock / 64][K];
    const T cut2 = T(g.cut2);
    // REST: one pose per outer step, skipped at once when it is a tiled pose
    const int64_t outer_n = REST ? g.B * g.P : g.work;
    for (int64_t outer = blockIdx.x; outer < outer_n; outer += gridDim.x) {
      if constexpr (REST) {
        const int64_t b0 = outer / g.P;
        if (pose_tiled_d<DIM>(rot + ((g.B_rot == 1 ? 0 : b0) * g.P + (outer - b0 * g.P)) * RS)) continue;
      }
      for (int ch = 0; ch < (REST ? g.chunks : 1); ++ch) {
        const int64_t w = REST ? outer * g.chunks + ch : outer;
        const int64_t bp = w / g.chunks;
        int i = 0, j = 0;
        const bool in_rect = rect_pixel(g, int(w - bp * g.chunks) * kBlock + int(threadIdx.x), i, j);
        const int pix = i * g.hp + j;
        const int64_t b = bp / g.P, p = bp - b * g.P;
        const int64_t rb = g.B_rot == 1 ? 0 : b, sb = g.B_shift == 1 ? 0 : b;
        T acc[K];
#pragma unroll
        for (int k = 0; k < K; ++k) acc[k] = T(0);
        if (in_rect) {
            const T r = freq_of<T>(i, g.n), c = T(j);
            const int64_t pidx = bp * g.npix + pix;
            Cx<T> out = {0, 0};
            T outw = T(0);
            if (!filtered(r, c, cut2) && !(j == 0 && i >= g.n / 2)) {
                const T* R = rot + (rb * g.P + p) * RS;
                const T* S = shifts ? shifts + (sb * g.P + p) * 2 : nullptr;
                T x[3], sc, sr;
                rotate<DIM>(R, r, c, g.os, x, sc, sr);
                const Interp<T> it = interpolate<DIM, T, CUBIC, ROT>(gdata + b * g.vol, g.N, g.H, x);
                Cx<T> ph = {T(1), T(0)};
                if (S) ph = phase<T>(r, c, S[0], S[1], g.phase_k);
                out = S ? cmul(it.v, ph) : it.v;
                if (WG) outw = weight_grad_interp<DIM, T>(gw + b * g.vol, g.N, g.H, x);
                if (ROT || SHIFT) {
                    Cx<T> pv = proj[pidx];
                    if (S) pv = cmul(pv, cconj(ph));
                    if (ROT) {
                        const T s[3] = {sc, sr, T(0.0)};
#pragma unroll
                        for (int row = 0; row < DIM; ++row)
#pragma unroll
                            for (int k = 0; k < DIM; ++k)
                                acc[row * DIM + k] += cmul(pv, cconj(cscale(it.g[row], s[k]))).re;
                    }
                    if (SHIFT) {
                        const Cx<T> kr = {T(0), T(-kTwoPi * double(r) / double(g.n))};
                        const Cx<T> kc = {T(0), T(-kTwoPi * double(c) / double(g.n))};
                        acc[RS] += cmul(pv, cconj(cmul(kr, it.v))).re;
                        acc[RS + 1] += cmul(pv, cconj(cmul(kc, it.v))).re;
                    }
                }
            }
            gproj[pidx] = out;
            if (gweights) gweights[pidx] = outw;
        }
        if (ROT || SHIFT) {
            block_sum<T, K>(acc, red);
            if (threadIdx.x == 0) {
                if (ROT)
                    for (int k = 0; k < RS; ++k) atomic_add(&grot[(rb * g.P + p) * RS + k], acc[k]);
                if (SHIFT)
                    for (int k = 0; k < 2; ++k) atomic_add(&gshift[(sb * g.P + p) * 2 + k], acc[RS + k]);
            }
        }
      }
    }
}

template <int DIM, typename T, bool CUBIC>
hipError_t forw(const Geom& g, const void* proj, const void* weights, const void* rot, const void* shifts, void* data,
                void* wrec, hipStream_t s) {
    if (weights)
        hipLaunchKernelGGL((k_backproject_forw<DIM, T, CUBIC, true>), dim3(grid_for(g.work)), dim3(kBlock), 0, s, g,
                           (const Cx<T>*)proj, (const T*)weights, (const T*)rot, (const T*)shifts, (Cx<T>*)data,
                           (T*)wrec);
    else
        hipLaunchKernelGGL((k_backproject_forw<DIM, T, CUBIC, false>), dim3(grid_for(g.work)), dim3(kBlock), 0, s,
                           g, (const Cx<T>*)proj, (const T*)nullptr, (const T*)rot, (const T*)shifts, (Cx<T>*)data,
                           (T*)nullptr);
    return hipGetLastError();
}

template <int DIM, bool CUBIC>
hipError_t forw_rest(const Geom& g, const void* proj, const void* weights, const void* rot, const void* shifts,
                     void* data, void* wrec, hipStream_t s) {
    const unsigned grid = grid_for(g.B * g.P);
    if (weights)
        hipLaunchKernelGGL((k_backproject_forw_rest<DIM, CUBIC, true>), dim3(grid), dim3(kBlock), 0, s, g,
                           (const Cx<float>*)proj, (const float*)weights, (const float*)rot, (const float*)shifts,
                           (Cx<float>*)data, (float*)wrec);
    else
        hipLaunchKernelGGL((k_backproject_forw_rest<DIM, CUBIC, false>), dim3(grid), dim3(kBlock), 0, s, g,
                           (const Cx<float>*)proj, (const float*)nullptr, (const float*)rot, (const float*)shifts,
                           (Cx<float>*)data, (float*)nullptr);
    return hipGetLastError();
}

template <int DIM, typename T, bool CUBIC, bool WG, bool ROT, bool SHIFT, bool REST>
hipError_t back8(const Geom& g, const void* gdata, const void* gw, const void* proj, const void* rot,
                 const void* shifts, void* gproj, void* gweights, void* grot, void* gshift, hipStream_t s) {
    const unsigned grid = REST ? grid_for(g.B * g.P) : grid_for(g.work);
    hipLaunchKernelGGL((k_backproject_back<DIM, T, CUBIC, WG, ROT, SHIFT, REST>), dim3(grid), dim3(kBlock), 0,
                       s, g, (const Cx<T>*)gdata, (const T*)gw, (const Cx<T>*)proj, (const T*)rot, (const T*)shifts,
                       (Cx<T>*)gproj, (T*)gweights, (T*)grot, (T*)gshift);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || REST) return e;  // with REST the outputs were zero-filled first
    return launch_zero_outside(sizeof(T) == 4 ? 0 : 1, g, gproj, gweights, s);
}

template <int DIM, typename T, bool CUBIC, bool WG, bool REST>
hipError_t back4(const Geom& g, const void* gdata, const void* gw, const void* proj, const void* rot,
                 const void* shifts, void* gproj, void* gweights, void* grot, void* gshift, hipStream_t s) {
    if (grot && gshift)
        return back8<DIM, T, CUBIC, WG, true, true, REST>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot,
                                                          gshift, s);
    if (grot)
        return back8<DIM, T, CUBIC, WG, true, false, REST>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot,
                                                           gshift, s);
    if (gshift)
        return back8<DIM, T, CUBIC, WG, false, true, REST>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot,
                                                           gshift, s);
    return back8<DIM, T, CUBIC, WG, false, false, REST>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot,
                                                        gshift, s);
}

template <int DIM, typename T, bool CUBIC, bool REST = false>
hipError_t back(const Geom& g, const void* gdata, const void* gw, const void* proj, const void* rot,
                const void* shifts, void* gproj, void* gweights, void* grot, void* gshift, hipStream_t s) {
    if (gw && gweights)
        return back4<DIM, T, CUBIC, true, REST>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift, s);
    return back4<DIM, T, CUBIC, false, REST>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift, s);
}

#define TP_DISPATCH(dim, dt, cubic, FN, ...)                                                  \
    do {                                                                                      \
        if (dim == 2) {                                                                       \
            if (dt == 0) return cubic ? FN<2, float, true>(__VA_ARGS__) : FN<2, float, false>(__VA_ARGS__);    \
            return cubic ? FN<2, double, true>(__VA_ARGS__) : FN<2, double, false>(__VA_ARGS__);               \
        }                                                                                     \
        if (dt == 0) return cubic ? FN<3, float, true>(__VA_ARGS__) : FN<3, float, false>(__VA_ARGS__);        \
        return cubic ? FN<3, double, true>(__VA_ARGS__) : FN<3, double, false>(__VA_ARGS__);                   \
    } while (0)

// Zero fill with 16-byte stores over the aligned body, four per lane per step, on up to 32768
// workgroups.  Plain stores with that grid beat non-temporal ones on 8192 workgroups: c5's 2D
// forward (17 GB of zeros around its gathered discs) 7.01 -> 6.78 ms, backproject_2d_back
// 12.38 -> 12.03 ms (A/B medians; each change alone gave about half of it).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(kBlock) void k_zero(uint32_t* __restrict__ p, int64_t head, int64_t quads,
                                                 int64_t words) {
    const int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    if (t < head) p[t] = 0u;
    u32x4* q = reinterpret_cast<u32x4*>(p + head);
    const u32x4 z = {0u, 0u, 0u, 0u};
    const int64_t step = int64_t(gridDim.x) * kBlock * 4;
    int64_t k = int64_t(blockIdx.x) * kBlock * 4 + threadIdx.x;
    for (; k + 3 * kBlock < quads; k += step) {
#pragma unroll
        for (int u = 0; u < 4; ++u) q[k + u * kBlock] = z;
    }
    for (int u = 0; u < 4; ++u)
        if (k + u * kBlock < quads) q[k + u * kBlock] = z;
    for (int64_t e = head + quads * 4 + t; e < words; e += int64_t(gridDim.x) * kBlock) p[e] = 0u;
}

// Zero elements [lo, hi) of a 4- or 8-byte-element array with 16-byte stores
// over the 16-byte-aligned middle; the threads of one block share the span.
template <typename E>
__device__ __forceinline__ void zero_span(E* __restrict__ p, int64_t lo, int64_t hi) {
    constexpr int V = 16 / sizeof(E);
    const int skip = int(((16 - (reinterpret_cast<uintptr_t>(p + lo) & 15)) & 15) / sizeof(E));
    int64_t a = lo + skip;
    if (a > hi) a = hi;
    const int64_t z = a + (hi - a) / V * V;
    for (int64_t k = lo + threadIdx.x; k < a; k += kBlock) p[k] = E{};
    uint4* q = reinterpret_cast<uint4*>(p + a);
    for (int64_t k = threadIdx.x; k < (z - a) / V; k += kBlock) q[k] = make_uint4(0u, 0u, 0u, 0u);
    for (int64_t k = z + threadIdx.x; k < hi; k += kBlock) p[k] = E{};
}

// Zeros on every pixel outside the active rectangle, one block per pose: the
// rows outside its row range are one contiguous span (rows rmax+1 .. n+rr0-1
// of the grid order), written with 16-byte stores; the columns past the
// rectangle on the rows inside, one wave per row.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_zero_outside(Geom g, Cx<T>* __restrict__ out, T* __restrict__ wout) {
    const int rmax = g.rr0 + g.rnr - 1;
    const int i_lo = rmax + 1, i_hi = g.n + g.rr0;  // grid rows i in [i_lo, i_hi) are outside
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int64_t bp = blockIdx.x; bp < g.B * g.P; bp += gridDim.x) {
        const int64_t base = bp * g.npix;
        if (i_hi > i_lo) {
            constexpr int W = sizeof(Cx<T>) / 8;  // 8-byte words per complex element
            if (out)
                zero_span(reinterpret_cast<uint2*>(out + base), int64_t(i_lo) * g.hp * W, int64_t(i_hi) * g.hp * W);
            if (wout) zero_span(wout + base, int64_t(i_lo) * g.hp, int64_t(i_hi) * g.hp);
        }
        if (g.rnc < g.hp) {
            for (int kr = wave; kr < g.rnr; kr += kBlock / 64) {
                const int r = g.rr0 + kr, i = r >= 0 ? r : r + g.n;
                const int64_t row = base + int64_t(i) * g.hp;
                for (int j = g.rnc + lane; j < g.hp; j += 64) {
                    if (out) out[row + j] = Cx<T>{T(0), T(0)};
                    if (wout) wout[row + j] = T(0);
                }
            }
        }
    }
}

}  // namespace

hipError_t launch_zero_outside(int dt, const Geom& g, void* out, void* wout, hipStream_t s) {
    if (g.rect == g.npix || (!out && !wout) || g.B * g.P == 0) return hipSuccess;
    const unsigned grid = unsigned(g.B * g.P < 65536 ? g.B * g.P : 65536);
    if (dt == 0)
        hipLaunchKernelGGL(k_zero_outside<float>, dim3(grid), dim3(kBlock), 0, s, g, (Cx<float>*)out, (float*)wout);
    else
        hipLaunchKernelGGL(k_zero_outside<double>, dim3(grid), dim3(kBlock), 0, s, g, (Cx<double>*)out,
                           (double*)wout);
    return hipGetLastError();
}

hipError_t launch_zero(void* p, int64_t words, hipStream_t s) {
    if (words <= 0) return hipSuccess;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    int64_t head = int64_t(((16 - (a & 15)) & 15) / 4);
    if (head > words) head = words;
    const int64_t quads = (words - head) / 4;
    int64_t blocks = (quads + kBlock - 1) / kBlock;
    if (blocks < 1) blocks = 1;
    if (blocks > 32768) blocks = 32768;
    hipLaunchKernelGGL(k_zero, dim3(unsigned(blocks)), dim3(kBlock), 0, s, (uint32_t*)p, head, quads, words);
    return hipGetLastError();
}

hipError_t launch_backproject_forw(int dim, int dt, bool cubic, const Geom& g, const void* proj, const void* weights,
                                   const void* rot, const void* shifts, void* data, void* wrec, hipStream_t s,
                                   bool rest_only) {
    if (rest_only && dt == 0) {
        if (dim == 2)
            return cubic ? forw_rest<2, true>(g, proj, weights, rot, shifts, data, wrec, s)
                         : forw_rest<2, false>(g, proj, weights, rot, shifts, data, wrec, s);
        return cubic ? forw_rest<3, true>(g, proj, weights, rot, shifts, data, wrec, s)
                     : forw_rest<3, false>(g, proj, weights, rot, shifts, data, wrec, s);
    }
    TP_DISPATCH(dim, dt, cubic, forw, g, proj, weights, rot, shifts, data, wrec, s);
}

hipError_t launch_backproject_back(int dim, int dt, bool cubic, const Geom& g, const void* gdata, const void* gw,
                                   const void* proj, const void* rot, const void* shifts, void* gproj,
                                   void* gweights, void* grot, void* gshift, hipStream_t s, bool rest_only) {
    if (rest_only && dt == 0) {
        if (dim == 2)
            return cubic ? back<2, float, true, true>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift, s)
                         : back<2, float, false, true>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift, s);
        return cubic ? back<3, float, true, true>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift, s)
                     : back<3, float, false, true>(g, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift, s);
    }
    TP_DISPATCH(dim, dt, cubic, back, g, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift, s);
}

}  // namespace tp
