// Forward projection (gather) and its adjoint/gradient (scatter) for the
// 2D->2D and 3D->2D operators.
//
//   k_project_forw  replaces project_2d_forw_cpu / project_3d_to_2d_forw_cpu
//                   (cpu/2d/projection_2d_kernels.cpp:96-202,
//                    cpu/3d/projection_3d_to_2d_kernels.cpp:97-212)
//   k_project_back  replaces project_2d_back_cpu / project_3d_to_2d_back_cpu
//                   (cpu/2d/projection_2d_kernels.cpp:209-375,
//                    cpu/3d/projection_3d_to_2d_kernels.cpp:219-402)
//
// One lane per output rfft pixel; a 256-lane block covers 256 consecutive
// pixels (row-major i, j) of one pose, so a wavefront walks neighbouring
// columns of neighbouring rows and its taps land on neighbouring volume
// lines.  Blocks loop over (pose, chunk) work items with a grid stride.
#include "tp_device.hh"
#include "tp_launch.hh"

namespace tp {

namespace {

constexpr double kTwoPi = 6.283185307179586476925286766559;

// Value of one active pixel (frequency r, c) of one pose; the volume is
// stored as Cx<VS> (VS = T, or half for a T = float computation).
template <int DIM, typename T, bool CUBIC, typename VS>
__device__ __forceinline__ Cx<T> project_pixel(const Geom& g, const Cx<VS>* __restrict__ recb, const T* __restrict__ R,
                                               const T* __restrict__ S, T r, T c) {
    T x[3], sc, sr;
    rotate<DIM>(R, r, c, g.os, x, sc, sr);
    Cx<T> v = interpolate<DIM, T, CUBIC, false>(recb, g.N, g.H, x).v;
    if (S) v = cmul(v, phase<T>(r, c, S[0], S[1], g.phase_k));
    return v;
}

template <int DIM, typename T, bool CUBIC, typename VS = T>
__global__ __launch_bounds__(kBlock) void k_project_forw(Geom g, const Cx<VS>* __restrict__ rec,
                                                         const T* __restrict__ rot, const T* __restrict__ shifts,
                                                         Cx<T>* __restrict__ out) {
    constexpr int RS = DIM * DIM;
    const T cut2 = T(g.cut2);
    for (int64_t w = blockIdx.x; w < g.work; w += gridDim.x) {
        const int64_t bp = w / g.chunks;
        int i = 0, j = 0;
        if (!rect_pixel(g, int(w - bp * g.chunks) * kBlock + int(threadIdx.x), i, j)) continue;
        const int pix = i * g.hp + j;
        const int64_t b = bp / g.P, p = bp - b * g.P;
        const T r = freq_of<T>(i, g.n), c = T(j);
        Cx<T> v = {0, 0};
        if (!filtered(r, c, cut2)) {
            const T* R = rot + ((g.B_rot == 1 ? 0 : b) * g.P + p) * RS;
            const T* S = shifts ? shifts + ((g.B_shift == 1 ? 0 : b) * g.P + p) * 2 : nullptr;
            v = project_pixel<DIM, T, CUBIC>(g, rec + b * g.vol, R, S, r, c);
        }
        out[bp * g.npix + pix] = v;
    }
}

// Completes the fp32 forward after the tiled kernel, which has written the
// active pixels of tiled poses: zeros on masked pixels, and every pixel of
// the other poses.  One block per pose.  ZEROED: the output was zero-filled
// first, so tiled poses are done.
template <int DIM, bool CUBIC, bool ZEROED, typename VS = float>
__global__ __launch_bounds__(kBlock) void k_project_forw_rest(Geom g, const Cx<VS>* __restrict__ rec,
                                                              const float* __restrict__ rot,
                                                              const float* __restrict__ shifts,
                                                              Cx<float>* __restrict__ out) {
    constexpr int RS = DIM * DIM;
    const float cut2 = float(g.cut2);
    // For a tiled pose only the masked pixels are written.  The mask test r^2 + c^2 > cut2
    // (rounded as the reference rounds it) is monotone in c, so they are the row's tail: the scan
    // starts at an estimate of its first column, sqrt(cut2 - r^2) - 2, once the exact test has
    // passed the column before it (otherwise at 0).  The start depends on the row only, so up to
    // kRestRows rows it is formed once per workgroup for all of its poses.
    constexpr int kRestRows = 1024;
    __shared__ int scan_start[kRestRows];
    auto scan_of = [&](int i) {
        const float r = freq_of<float>(i, g.n);
        int c_scan = 0;
        const float rem = cut2 - r * r;
        if (rem >= 4.f) {  // false for NaN: then every column is tested (none is masked)
            int cs = rem < 1.0e9f ? int(__builtin_amdgcn_sqrtf(rem)) - 2 : g.hp;
            cs = min(g.hp, max(0, cs));
            c_scan = (cs > 0 && filtered(r, float(cs - 1), cut2)) ? 0 : cs;
        }
        return c_scan;
    };
    const bool table = g.n <= kRestRows;
    if (table) {
        for (int i = threadIdx.x; i < g.n; i += kBlock) scan_start[i] = scan_of(i);
        __syncthreads();
    }
    for (int64_t bp = blockIdx.x; bp < g.B * g.P; bp += gridDim.x) {
        const int64_t b = bp / g.P, p = bp - b * g.P;
        const float* R = rot + ((g.B_rot == 1 ? 0 : b) * g.P + p) * RS;
        const float* S = shifts ? shifts + ((g.B_shift == 1 ? 0 : b) * g.P + p) * 2 : nullptr;
        const bool tiled = pose_tiled_d<DIM>(R);
        if (ZEROED && tiled) continue;  // block-uniform
        Cx<float>* outp = out + bp * g.npix;
        // four rows per wave step, 16 lanes along each row (no per-pixel division): most rows'
        // masked tails are short
        constexpr int RL = 16, RW = 64 / RL;
        for (int i0 = (threadIdx.x / 64) * RW; i0 < g.n; i0 += (kBlock / 64) * RW) {
            const int i = i0 + (threadIdx.x % 64) / RL;
            if (i >= g.n) continue;
            const float r = freq_of<float>(i, g.n);
            Cx<float>* row = outp + int64_t(i) * g.hp;
            const int c_scan = tiled ? (table ? scan_start[i] : scan_of(i)) : 0;
            for (int j = c_scan + threadIdx.x % RL; j < g.hp; j += RL) {
                const float c = float(j);
                if (filtered(r, c, cut2)) row[j] = Cx<float>{0.f, 0.f};
                else if (!tiled) row[j] = project_pixel<DIM, float, CUBIC>(g, rec + b * g.vol, R, S, r, c);
            }
        }
    }
}

// Gradient of the forward projection.  The reconstruction gradient is the
// transposed interpolation of g' = g * conj(phase), scattered Friedel-aware
// with out-of-range taps dropped and no x = 0 mirror
// (projection_utils.h:336-362, 414-443).  Rotation and shift gradients are
// per-pose sums, reduced across the block before one atomic per component.
// REST (fp32) 1: the reconstruction gradient of tiled poses comes from the
// tiled scatter; only the other poses are scattered here.  REST 2: the tiled
// kernels also give the rotation/shift gradients of tiled poses, which are
// skipped here entirely.  VS: the volume's storage type (complex half is widened
// exactly to fp32 on load, with T = float).
template <int DIM, typename T, bool CUBIC, bool ROT, bool SHIFT, int REST, typename VS = T>
__global__ __launch_bounds__(kBlock) void k_project_back(Geom g, const Cx<T>* __restrict__ gproj,
                                                         const Cx<VS>* __restrict__ rec, const T* __restrict__ rot,
                                                         const T* __restrict__ shifts, Cx<T>* __restrict__ grec,
                                                         T* __restrict__ grot, T* __restrict__ gshift) {
    constexpr int RS = DIM * DIM;
    constexpr int K = RS + 2;
    __shared__ T red[kBlock / 64][K];
    const T cut2 = T(g.cut2);
    // REST: one pose per outer step, checked once
    const int64_t outer_n = REST != 0 ? g.B * g.P : g.work;
    for (int64_t outer = blockIdx.x; outer < outer_n; outer += gridDim.x) {
      bool scatter = true;
      if constexpr (REST != 0) {
        const int64_t b0 = outer / g.P;
        scatter = !pose_tiled_d<DIM>(rot + ((g.B_rot == 1 ? 0 : b0) * g.P + (outer - b0 * g.P)) * RS);
        if (!scatter && (REST == 2 || (!ROT && !SHIFT))) continue;  // block-uniform
      }
      for (int ch = 0; ch < (REST != 0 ? g.chunks : 1); ++ch) {
        const int64_t w = REST != 0 ? outer * g.chunks + ch : outer;
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
            // masked pixels and the Friedel half of the x = 0 line are skipped
            if (!filtered(r, c, cut2) && !(j == 0 && i >= g.n / 2)) {
                const T* R = rot + (rb * g.P + p) * RS;
                const T* S = shifts ? shifts + (sb * g.P + p) * 2 : nullptr;
                T x[3], sc, sr;
                rotate<DIM>(R, r, c, g.os, x, sc, sr);
                const Cx<T> g0 = gproj[bp * g.npix + pix];
                const Cx<T> gg = S ? cmul(g0, phase<T>(-r, -c, S[0], S[1], g.phase_k)) : g0;
                Cx<T>* gb = grec + b * g.vol;
                const int N = g.N, H = g.H;
                if (scatter)
                    distribute<DIM, T, CUBIC>(x, [&](int d, int rr, int cc, T wd, T wr, T wc) {
                        bool cj;
                        const int64_t idx = scatter_index<DIM>(N, H, d, rr, cc, cj);
                        if (idx < 0) return;
                        Cx<T> v = tap_value<DIM, T>(gg, wd, wr, wc);
                        if (cj) v.im = -v.im;
                        atomic_add_cx(&gb[idx], v);
                    });
                if (ROT || SHIFT) {
                    const Interp<T> it = interpolate<DIM, T, CUBIC, ROT>(rec + b * g.vol, N, H, x);
                    if (ROT) {
                        const T s[3] = {sc, sr, T(0.0)};
#pragma unroll
                        for (int row = 0; row < DIM; ++row)
#pragma unroll
                            for (int k = 0; k < DIM; ++k)
                                acc[row * DIM + k] += cmul(gg, cconj(cscale(it.g[row], s[k]))).re;
                    }
                    if (SHIFT) {
                        const Cx<T> mod = cmul(it.v, phase<T>(r, c, S[0], S[1], g.phase_k));
                        const Cx<T> kr = {T(0), T(-kTwoPi * double(r) / double(g.n))};
                        const Cx<T> kc = {T(0), T(-kTwoPi * double(c) / double(g.n))};
                        acc[RS] += cmul(g0, cconj(cmul(kr, mod))).re;
                        acc[RS + 1] += cmul(g0, cconj(cmul(kc, mod))).re;
                    }
                }
            }
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

template <int DIM, typename T, bool CUBIC, typename VS = T>
hipError_t forw(const Geom& g, const void* rec, const void* rot, const void* shifts, void* out, hipStream_t s) {
    hipLaunchKernelGGL((k_project_forw<DIM, T, CUBIC, VS>), dim3(grid_for(g.work)), dim3(kBlock), 0, s, g,
                       (const Cx<VS>*)rec, (const T*)rot, (const T*)shifts, (Cx<T>*)out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_zero_outside(sizeof(T) == 4 ? 0 : 1, g, out, nullptr, s);
}

template <int DIM, bool CUBIC, typename VS = float>
hipError_t forw_rest(const Geom& g, const void* rec, const void* rot, const void* shifts, void* out, hipStream_t s) {
    // 2D: the C ABI zero-fills the output first (a streaming fill beats per-row masked zeros)
    hipLaunchKernelGGL((k_project_forw_rest<DIM, CUBIC, DIM == 2, VS>), dim3(grid_for(g.B * g.P)), dim3(kBlock), 0,
                       s, g, (const Cx<VS>*)rec, (const float*)rot, (const float*)shifts, (Cx<float>*)out);
    return hipGetLastError();
}

template <int DIM, typename T, bool CUBIC, bool ROT, bool SHIFT, int REST, typename VS>
hipError_t back4(const Geom& g, const void* gproj, const void* rec, const void* rot, const void* shifts, void* grec,
                 void* grot, void* gshift, hipStream_t s) {
    // with REST most (pose, chunk) items are skipped at once: fewer, longer-lived blocks
    const unsigned grid = REST ? grid_for(g.B * g.P) : grid_for(g.work);
    hipLaunchKernelGGL((k_project_back<DIM, T, CUBIC, ROT, SHIFT, REST, VS>), dim3(grid), dim3(kBlock), 0,
                       s, g, (const Cx<T>*)gproj, (const Cx<VS>*)rec, (const T*)rot, (const T*)shifts, (Cx<T>*)grec,
                       (T*)grot, (T*)gshift);
    return hipGetLastError();
}

template <int DIM, typename T, bool CUBIC, int REST = 0, typename VS = T>
hipError_t back(const Geom& g, const void* gproj, const void* rec, const void* rot, const void* shifts, void* grec,
                void* grot, void* gshift, hipStream_t s) {
    if (grot && gshift)
        return back4<DIM, T, CUBIC, true, true, REST, VS>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
    if (grot) return back4<DIM, T, CUBIC, true, false, REST, VS>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
    if (gshift) return back4<DIM, T, CUBIC, false, true, REST, VS>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
    return back4<DIM, T, CUBIC, false, false, REST, VS>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
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

}  // namespace

hipError_t launch_project_forw(int dim, int dt, bool cubic, const Geom& g, const void* rec, const void* rot,
                               const void* shifts, void* out, hipStream_t s, bool rest_only) {
    if (dt == 2) {  // complex-half volume, fp32 arithmetic and output
        if (rest_only) {
            if (dim == 2)
                return cubic ? forw_rest<2, true, __half>(g, rec, rot, shifts, out, s)
                             : forw_rest<2, false, __half>(g, rec, rot, shifts, out, s);
            return cubic ? forw_rest<3, true, __half>(g, rec, rot, shifts, out, s)
                         : forw_rest<3, false, __half>(g, rec, rot, shifts, out, s);
        }
        if (dim == 2)
            return cubic ? forw<2, float, true, __half>(g, rec, rot, shifts, out, s)
                         : forw<2, float, false, __half>(g, rec, rot, shifts, out, s);
        return cubic ? forw<3, float, true, __half>(g, rec, rot, shifts, out, s)
                     : forw<3, float, false, __half>(g, rec, rot, shifts, out, s);
    }
    if (rest_only && dt == 0) {
        if (dim == 2)
            return cubic ? forw_rest<2, true>(g, rec, rot, shifts, out, s)
                         : forw_rest<2, false>(g, rec, rot, shifts, out, s);
        return cubic ? forw_rest<3, true>(g, rec, rot, shifts, out, s) : forw_rest<3, false>(g, rec, rot, shifts, out, s);
    }
    TP_DISPATCH(dim, dt, cubic, forw, g, rec, rot, shifts, out, s);
}

hipError_t launch_project_back(int dim, int dt, bool cubic, const Geom& g, const void* gproj, const void* rec,
                               const void* rot, const void* shifts, void* grec, void* grot, void* gshift,
                               hipStream_t s, int rest) {
    if (dt == 2) {  // complex-half volume, fp32 arithmetic, gradients and outputs
        if (rest != 0) {
            if (dim == 2)
                return cubic ? back<2, float, true, 2, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s)
                             : back<2, float, false, 2, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
            return cubic ? back<3, float, true, 2, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s)
                         : back<3, float, false, 2, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
        }
        if (dim == 2)
            return cubic ? back<2, float, true, 0, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s)
                         : back<2, float, false, 0, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
        return cubic ? back<3, float, true, 0, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s)
                     : back<3, float, false, 0, __half>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
    }
    if (rest != 0 && dt == 0) {
        if (dim == 2)
            return cubic ? back<2, float, true, 2>(g, gproj, rec, rot, shifts, grec, grot, gshift, s)
                         : back<2, float, false, 2>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
        return cubic ? back<3, float, true, 2>(g, gproj, rec, rot, shifts, grec, grot, gshift, s)
                     : back<3, float, false, 2>(g, gproj, rec, rot, shifts, grec, grot, gshift, s);
    }
    TP_DISPATCH(dim, dt, cubic, back, g, gproj, rec, rot, shifts, grec, grot, gshift, s);
}

}  // namespace tp
