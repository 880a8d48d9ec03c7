// Tile-owner scatter for the 2D operators (fp32): backproject_2d_forw and the
// reconstruction gradient of project_2d_back.
//
// The reference spreads each projection pixel's stencil straight into the
// image (cpu/2d/backprojection_2d_kernels.cpp:99-282 with
// projection_utils.h:371-406, 451-493; cpu/2d/projection_2d_kernels.cpp:300-322
// with projection_utils.h:336-362).  A 2D pose covers the whole frequency
// disc, so every cell of an image receives taps from every pose: one float
// atomic per tap into HBM serialises on the same few thousand cells.
//
// Here a workgroup owns a TC x TR tile of the stored half plane, accumulated
// in fp64 LDS, for one range of poses.  Per phase of kChunk2 poses it culls
// the rotations whose sample half-disc reaches the tile (box 1: direct taps,
// c >= 0) or its negation (box 2: taps with c < 0, which the reference
// flips to (-c, -r) and conjugates), then enumerates exactly the samples of
// each such pose whose stencil reaches the box: one lane per (pose, row)
// computes the row's column interval, a wave prefix sum packs the samples of
// KP poses densely onto the lanes.  Partial tiles of the pose ranges are
// added into the zero-filled image with float atomics (once per cell and
// range).  The x = 0 Hermitian completion of the backprojection is applied
// afterwards by k_mirror2_x0.
//
// Poses whose 2x2 matrix has singular values in [kScaleMin, kScaleMax]
// (pose_tiled2: rotations, and scaled or sheared matrices) take this path;
// the per-pixel kernels scatter the others.  Each kernel comes in two
// instantiations: GEN = false takes the rotations, GEN = true (launched
// after it on a small persistent grid that exits at once when the call has
// no such pose) the other tiled matrices.  A sample x = R (sc, sr) of those
// has sc = as . x and sr = bs . x with the dual basis (the rows of R^-1),
// which bounds the rows and the half plane sc >= 0 that reach a box; their
// tiles reach up to kScaleMax times farther out.
#include <type_traits>

#include "tp_device.hh"
#include "tp_launch.hh"
#include "tp_tiled_common.hh"

namespace tp {

namespace {

constexpr int TC = kTile2C, TR = kTile2R, T2 = TC * TR;  // tile edges (cells): c, r
constexpr int kThreads = 256;
constexpr int kRun = 128;         // XCD run length (items)
constexpr int kChunk2 = 512;      // poses culled per phase
constexpr int kInFlight = 2;      // rotations loaded together per lane in the cull
constexpr double kPrivOs = 1.5;   // scatters whose samples are this far apart (os * kScaleMin) use
                                  // wave-private accumulators
static_assert((TC & (TC - 1)) == 0, "tile width must be a power of two");
static_assert(kChunk2 <= 65535, "pose index must fit the list entries");

// Sample position of pixel (r, c), as rotate<2>: x = R (sc, sr).
__device__ __forceinline__ void rotate_pix(const float* __restrict__ R, float r, float c, double os, float* x) {
    const float sc = float(double(c) * os), sr = float(double(r) * os);
    x[0] = R[0] * sc + R[1] * sr;
    x[1] = R[2] * sc + R[3] * sr;
}

// Samples have sc = as . x >= 0: does the box reach that half plane?
__device__ __forceinline__ bool half_plane_hits2(const float* as, const float* lo, const float* hi) {
    const float u = (as[0] >= 0.f ? as[0] * hi[0] : as[0] * lo[0]) + (as[1] >= 0.f ? as[1] * hi[1] : as[1] * lo[1]);
    return u >= 0.f;
}

// Is the pose of this instantiation's class (rotation, or GEN: another tiled
// matrix)?  `as` receives the half-plane vector (column 0, or its dual).
template <bool GEN>
__device__ __forceinline__ bool pose_of_class2(const float* R, float* as) {
    const PoseGram gr = pose_gram2(R);
    if constexpr (GEN) {
        if (gram_is_rotation(gr) || !gram_tiled(gr)) return false;
        float bs[2];
        pose_dual2(R, gr, as, bs);
        return true;
    } else {
        as[0] = R[0];
        as[1] = R[2];
        return gram_is_rotation(gr);
    }
}

// Rows r (sr = r*os = bs . x) whose samples can lie in the box: bs is a
// rotation's column 1, or (GEN) the dual basis vector.
template <bool GEN>
__device__ __forceinline__ void box_rows2(const float* R, const float* lo, const float* hi, const TileSpec2& ts,
                                          int& r0, int& r1) {
    float as[2], bs[2] = {R[1], R[3]};
    if constexpr (GEN) pose_dual2(R, pose_gram2(R), as, bs);
    float vlo = 0.f, vhi = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const float b = bs[k];
        vlo += b >= 0.f ? b * lo[k] : b * hi[k];
        vhi += b >= 0.f ? b * hi[k] : b * lo[k];
    }
    r0 = max(ts.rmin, to_int_clamped(ceilf(vlo * ts.inv_os)));
    r1 = min(ts.rmax, to_int_clamped(floorf(vhi * ts.inv_os)));
}

// Columns c of row r whose sample lies in the box (which carries the slack
// covering rounding), within the pixel grid and (up to one column) the cutoff.
__device__ __forceinline__ void row_span2(const float* R, int r, const float* lo, const float* hi,
                                          const TileSpec2& ts, float cut2, int& c0, int& c1) {
    const float ros = float(r) * ts.os;
    float l = -3.0e38f, h = 3.0e38f;
    bool empty = false;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const float a = R[2 * k], base = ros * R[2 * k + 1];
        const float lk = lo[k] - base, hk = hi[k] - base;  // need a*sc in [lk, hk]
        if (fabsf(a) > 1e-6f) {
            const float ia = __builtin_amdgcn_rcpf(a);
            const float u0 = lk * ia, u1 = hk * ia;
            l = fmaxf(l, a > 0.f ? u0 : u1);
            h = fminf(h, a > 0.f ? u1 : u0);
        } else {
            const float tol = fabsf(a) * ts.smax;
            empty |= lk > tol || hk < -tol;
        }
    }
    c0 = max(0, to_int_clamped(ceilf(l * ts.inv_os - 1e-3f)));
    c1 = min(ts.cmax, to_int_clamped(floorf(h * ts.inv_os + 1e-3f)));
    c1 = empty ? -1 : cap_to_disc(c1, float(r), cut2);
}

// Per-wave copy of the poses of one batch.
struct Slot2 {
    float R[4];
    float s0, s1;
    int p;
};

__device__ __forceinline__ void load_pose2(const float* __restrict__ rotb, const float* __restrict__ shb, int p,
                                           float* R, float* S) {
#pragma unroll
    for (int e = 0; e < 4; ++e) R[e] = rotb[int64_t(p) * 4 + e];
    S[0] = shb ? shb[2 * int64_t(p)] : 0.f;
    S[1] = shb ? shb[2 * int64_t(p) + 1] : 0.f;
}

// Cull poses [pbase, pend) (at most kChunk2) against box 1 and box 2.  Box-1
// survivors fill plist from the front, box-2 survivors from the back.
template <bool GEN>
__device__ __forceinline__ void cull2(const float* __restrict__ rotb, int pend, int pbase, const float* lo1,
                                      const float* hi1, const float* lo2, const float* hi2, unsigned short* plist,
                                      int* pcnt, int& n1, int& n2) {
    static_assert(kChunk2 % kThreads == 0 && (kChunk2 / kThreads) % kInFlight == 0, "cull shape");
    __syncthreads();  // every lane has read the previous counts and lists
    if (threadIdx.x == 0) pcnt[0] = pcnt[1] = 0;
    __syncthreads();
#pragma unroll 1
    for (int q0 = 0; q0 < kChunk2 / kThreads; q0 += kInFlight) {
        float R[kInFlight][4];
#pragma unroll
        for (int q = 0; q < kInFlight; ++q) {
            const int p = min(pbase + int(threadIdx.x) + (q0 + q) * kThreads, pend - 1);
#pragma unroll
            for (int e = 0; e < 4; ++e) R[q][e] = rotb[int64_t(p) * 4 + e];
        }
#pragma unroll
        for (int q = 0; q < kInFlight; ++q) {
            const int p = pbase + int(threadIdx.x) + (q0 + q) * kThreads;
            float as[2];
            if (p >= pend || !pose_of_class2<GEN>(R[q], as)) continue;
            if (half_plane_hits2(as, lo1, hi1)) plist[atomicAdd(&pcnt[0], 1)] = (unsigned short)(p - pbase);
            if (half_plane_hits2(as, lo2, hi2))
                plist[2 * kChunk2 - 1 - atomicAdd(&pcnt[1], 1)] = (unsigned short)(p - pbase);
        }
    }
    __syncthreads();
    n1 = pcnt[0];
    n2 = pcnt[1];
}

// LDS layout of the accumulators: cell (lc, lr) sits at
// lr * TC + ((lc + swizzle2(lr)) mod TC).  Samples stepping along r land two
// rows apart; the rotation by lr / 2 spreads them over different banks (an
// fp64 cell spans two of the 64 four-byte banks).
__device__ __forceinline__ int swizzle2(int lr) { return (lr >> 1) & (TC - 1); }

// Per-pass constants: local cell of tap j on axis a is sgn * floor(x_a) + off[a] + sgn * j
// (sgn = -1 for the flipped taps), valid in [lmin[a], S_a).
struct TapMap2 {
    int sgn;
    int off[2];
    int lmin[2];
};

// Spread one sample over the tile: taps at floor(x) - LOW + j, weights of the
// reference's (bi)linear / Catmull-Rom stencil (projection_utils.h:172-300),
// v * (wr * wc) in fp64 (the reference's (v * wr) * wc in fp32 up to rounding).
template <bool CUBIC, int MODE, bool WEIGHTS>
__device__ __forceinline__ void scatter_sample2(const Geom& g, const Slot2& sd, int rr, int cc, Cx<float> v,
                                                float wpix, bool shifted, bool flip, const TapMap2& tm,
                                                double* acc_re, double* acc_im, double* acc_w) {
    constexpr int K = CUBIC ? 4 : 2;
    const float fr = float(rr), fc = float(cc);
    float x[2];
    rotate_pix(sd.R, fr, fc, g.os, x);
    if (shifted) {
        if (MODE == 0) v = cmul(v, cconj(phase_hw(fr, fc, sd.s0, sd.s1, g.phase_k)));
        else v = cmul(v, phase_hw(-fr, -fc, sd.s0, sd.s1, g.phase_k));
    }
    constexpr int S[2] = {TC, TR};
    int loc[2][K];
    double wt[2][K];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        float f;
        const int fl = split_as<false>(x[a], f);
        const int l0 = (flip ? -fl : fl) + tm.off[a];
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const int l = l0 + tm.sgn * j;
            loc[a][j] = (unsigned)(l - tm.lmin[a]) < (unsigned)(S[a] - tm.lmin[a]) ? l : -1;
            if (CUBIC) wt[a][j] = double(cubic_w_tap<float>(f, j));
        }
        if (!CUBIC) {
            wt[a][1] = double(f);
            wt[a][0] = 1.0 - wt[a][1];
        }
    }
    const double vre = double(v.re), vim = flip ? -double(v.im) : double(v.im), wp = double(wpix);
#pragma unroll
    for (int i = 0; i < K; ++i) {
        if (loc[1][i] < 0) continue;
        const int row = loc[1][i] * TC, rot = swizzle2(loc[1][i]);
#pragma unroll
        for (int j = 0; j < K; ++j) {
            if (loc[0][j] < 0) continue;
            const double w = wt[1][i] * wt[0][j];
            const int li = row + ((loc[0][j] + rot) & (TC - 1));
            atomicAdd(&acc_re[li], vre * w);
            atomicAdd(&acc_im[li], vim * w);
            if (WEIGHTS) atomicAdd(&acc_w[li], wp * (CUBIC ? fabs(w) : w));
        }
    }
}

// The same for a wave-private fp32 accumulator (PRIV): plain read-add-write
// instead of LDS atomics, legal because the 64 lanes of a window hold
// samples of one pose, whose positions are at least os > sqrt(2) apart and so
// lie in distinct cells: the lanes of one tap never share a cell.  A wave's
// LDS operations execute in order; the signal fence keeps the compiler from
// moving one tap's read above the previous tap's write (another lane's tap
// may have written that cell).  The private tile has rows of PS = TC + 1
// cells (the odd stride spreads a column over the banks) and one row more: a
// tap outside the tile goes to that row or to a row's last cell, which are
// never written out, so every tap runs without a test or branch (lanes that
// share those cells only lose garbage).  v * wr is rounded as the reference
// forms it; the product with wc is fused into the fp32 sum (and the weight
// tap wpix * |wr * wc| into its sum as (wpix * |wr|) * |wc|), one rounding per
// tap fewer than the reference's order, far below the per-cell bar, and still
// exactly 0 where every tap weight is.
constexpr int PS = TC + 1, PT = (TR + 1) * PS;  // private tile: row stride, cells
template <bool CUBIC, int MODE, bool WEIGHTS>
__device__ __forceinline__ void scatter_sample2_priv(const Geom& g, const Slot2& sd, int rr, int cc, Cx<float> v,
                                                     float wpix, bool shifted, bool flip, const TapMap2& tm,
                                                     float2* pc, float* pw) {
    constexpr int K = CUBIC ? 4 : 2;
    const float fr = float(rr), fc = float(cc);
    float x[2];
    rotate_pix(sd.R, fr, fc, g.os, x);
    if (shifted) {
        if (MODE == 0) v = cmul(v, cconj(phase_hw(fr, fc, sd.s0, sd.s1, g.phase_k)));
        else v = cmul(v, phase_hw(-fr, -fc, sd.s0, sd.s1, g.phase_k));
    }
    constexpr int S[2] = {TC, TR};
    int loc[2][K];  // column, or row offset, of each tap; the spare cell / row outside the tile
    float wt[2][K];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        float f;
        const int fl = split_as<false>(x[a], f);
        const int l0 = (flip ? -fl : fl) + tm.off[a];
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const int l = l0 + tm.sgn * j;
            const bool in = (unsigned)(l - tm.lmin[a]) < (unsigned)(S[a] - tm.lmin[a]);
            loc[a][j] = a == 0 ? (in ? l : TC) : (in ? l : TR) * PS;
            if (CUBIC) wt[a][j] = cubic_w_tap<float>(f, j);
        }
        if (!CUBIC) {
            wt[a][1] = f;
            wt[a][0] = 1.0f - f;
        }
    }
    const float vre = v.re, vim = flip ? -v.im : v.im;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const float rre = vre * wt[1][i], rim = vim * wt[1][i];
        const float rw = wpix * (CUBIC ? fabsf(wt[1][i]) : wt[1][i]);
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const int li = loc[1][i] + loc[0][j];
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            float2 t = pc[li];
            t.x = fmaf(rre, wt[0][j], t.x);
            t.y = fmaf(rim, wt[0][j], t.y);
            pc[li] = t;
            if (WEIGHTS) pw[li] = fmaf(rw, CUBIC ? fabsf(wt[0][j]) : wt[0][j], pw[li]);
        }
    }
}

// MODE 0: backprojection, v = proj * conj(phase(r, c)), optional weights.
// MODE 1: reconstruction gradient of the projection, v = g * phase(-r, -c).
// dst (and wdst) must be zero-filled: every item adds its partial tile.
// PRIV (one pose per window, KP = 1, os > sqrt(2) with margin): wave-private
// fp32 accumulators without atomics, summed over the waves at write-out;
// otherwise one fp64 accumulator per tile with LDS atomics.
template <bool CUBIC, int MODE, bool WEIGHTS, int KP, bool PRIV, bool GEN>
__global__ __launch_bounds__(kThreads) void k_scatter2_tiled(Geom g, TileSpec2 ts, const Cx<float>* __restrict__ src,
                                                             const float* __restrict__ weights,
                                                             const float* __restrict__ rot,
                                                             const float* __restrict__ shifts,
                                                             Cx<float>* __restrict__ dst, float* __restrict__ wdst,
                                                             CallPoses* __restrict__ cp, int gl) {
    constexpr int SL = CUBIC ? 2 : 1, SH = CUBIC ? 1 : 0;  // stencil reach below / above floor(x)
    constexpr int SLOW = CUBIC ? 1 : 0;                    // first tap at floor(x) - SLOW
    constexpr int RPS = 64 / KP;
    constexpr int NW = kThreads / 64;
    static_assert(!PRIV || KP == 1, "private accumulation needs one pose per window");
    constexpr int TS = PRIV ? 1 : T2, TP = PRIV ? PT : 1;
    __shared__ double acc_re[TS], acc_im[TS];
    __shared__ double acc_w[WEIGHTS ? TS : 1];
    __shared__ float2 pacc[NW][TP];
    __shared__ float pwacc[NW][WEIGHTS ? TP : 1];
    __shared__ unsigned short plist[2 * kChunk2];
    __shared__ int pcnt[2];
    __shared__ Slot2 slots[NW][KP];
    __shared__ int marks[NW][64];
    __shared__ int gen_sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int slot = lane / RPS, jrow = lane % RPS;
    const int N = g.N, H = g.H, half = N / 2;
    // samples lie within |x| <= rho_k: rotations reach rho_unit + 1 (and have nothing to do when
    // the call has none); GEN poses the call's own reach, up to kScaleMax times farther, over
    // the tiles within it (the same rule as the host's for the rotations' and the widest range)
    const int any_rot = GEN ? 1 : call_flag(&cp->any_rot);
    float rho_k = ts.rho_unit + 1.0f;
    int tkr0 = ts.kr0, tnr = ts.nr, tnc = ts.nc;
    if constexpr (GEN) {
        rho_k = fminf(ts.rho, cp->gen_reach);
        if (!(rho_k > 0.f)) return;  // no such pose in this call
        const float reach = fminf(rho_k + 3.0f, float(N));
        tkr0 = max(ts.kr0_2, int(floorf((-reach + float(half - 1)) / float(TR))));
        const int kr1 = min(ts.kr0_2 + ts.nr_2, int(floorf((reach + float(half - 1)) / float(TR))) + 1);
        tnr = max(0, kr1 - tkr0);
        tnc = min(ts.nc_2, int(floorf(reach / float(TC))) + 1);
    }
    const int64_t items = g.B * ts.ksplit * int64_t(tnr) * tnc;
    const float cut2 = float(g.cut2);
    for (Slots<GEN> sl(xcd_per<kRun>(items), slot_counters<GEN>(cp, gl), &gen_sh); sl.ok(); sl.next(&gen_sh)) {
        const int64_t slot_i = sl.s;
        const int64_t w = xcd_item<kRun>(slot_i);
        if (w >= items) continue;
        // items: tile column fastest, then tile row, pose range, batch
        const int kc = int(w % tnc);
        int64_t q = w / tnc;
        const int kr = tkr0 + int(q % tnr);
        q /= tnr;
        const int jr = int(q % ts.ksplit);
        const int64_t b = q / ts.ksplit;
        const int p0 = jr * ts.prange, p1 = min(int(g.P), p0 + ts.prange);
        if (!any_rot) return;  // rotation kernel, no rotation in the call
        // stored cells of this tile, signed coordinates: r in [-N/2+1, N/2], c in [0, N/2]
        const int tc = kc * TC, tr = -half + 1 + kr * TR;
        const int fc0 = -tc - TC + 1, fr0 = -tr - TR + 1;
        const float lo1[2] = {float(tc - SL) - ts.eps, float(tr - SL) - ts.eps};
        const float hi1[2] = {float(tc + TC + SH) + ts.eps, float(tr + TR + SH) + ts.eps};
        const float lo2[2] = {float(fc0 - SL) - ts.eps, float(fr0 - SL) - ts.eps};
        const float hi2[2] = {float(fc0 + TC + SH) + ts.eps, float(fr0 + TR + SH) + ts.eps};
        for (int e = tid; e < T2; e += kThreads) {
            if constexpr (PRIV) {
                const int pe = (e / TC) * PS + e % TC;  // the private tile's cells (not its spare ones)
#pragma unroll
                for (int k = 0; k < NW; ++k) {
                    pacc[k][pe] = float2{0.f, 0.f};
                    if (WEIGHTS) pwacc[k][pe] = 0.f;
                }
            } else {
                acc_re[e] = 0.0;
                acc_im[e] = 0.0;
                if (WEIGHTS) acc_w[e] = 0.0;
            }
        }
        const int64_t rb = g.B_rot == 1 ? 0 : b, sb = g.B_shift == 1 ? 0 : b;
        const float* rotb = rot + rb * g.P * 4;
        const float* shb = shifts ? shifts + sb * g.P * 2 : nullptr;
        const int64_t pose0 = b * g.P;
        // samples lie within |x| <= rho_k; box 2 is box 1 mirrored, so one test serves both
        float dist2 = 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float d = lo1[k] > 0.f ? lo1[k] : (hi1[k] < 0.f ? -hi1[k] : 0.f);
            dist2 += d * d;
        }
        const int pend = dist2 > rho_k * rho_k ? p0 : p1;

        for (int pbase = p0; pbase < pend; pbase += kChunk2) {
            int n1, n2;
            cull2<GEN>(rotb, pend, pbase, lo1, hi1, lo2, hi2, plist, pcnt, n1, n2);
#pragma unroll 1
            for (int pass = 0; pass < 2; ++pass) {
                const int np = pass == 0 ? n1 : n2;
                auto pose_at = [&](int k) { return pbase + int(plist[pass == 0 ? k : 2 * kChunk2 - 1 - k]); };
                float lo[2], hi[2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    lo[k] = pass == 0 ? lo1[k] : lo2[k];
                    hi[k] = pass == 0 ? hi1[k] : hi2[k];
                }
                // direct taps: l = floor(x) - LOW + j - t; flipped: l = -(floor(x) - LOW + j) - t,
                // and at c = 0 a flipped tap must have c < 0 (l >= 1 when t_c = 0)
                TapMap2 tm;
                tm.sgn = pass == 0 ? 1 : -1;
                tm.off[0] = pass == 0 ? -SLOW - tc : SLOW - tc;
                tm.off[1] = pass == 0 ? -SLOW - tr : SLOW - tr;
                tm.lmin[0] = (pass == 1 && tc == 0) ? 1 : 0;
                tm.lmin[1] = 0;
                int base = wave * KP;
                float Rn[4], Sn[2];
                if (base < np) load_pose2(rotb, shb, pose_at(min(base + slot, np - 1)), Rn, Sn);
                for (; base < np; base += NW * KP) {
                    const bool sv = base + slot < np;
                    const int pp = pose_at(min(base + slot, np - 1));
                    float R[4], Sh[2];
#pragma unroll
                    for (int e = 0; e < 4; ++e) R[e] = Rn[e];
                    Sh[0] = Sn[0];
                    Sh[1] = Sn[1];
                    if (base + NW * KP < np)
                        load_pose2(rotb, shb, pose_at(min(base + NW * KP + slot, np - 1)), Rn, Sn);
                    if (jrow == 0 && sv) {
                        Slot2& sd = slots[wave][slot];
#pragma unroll
                        for (int e = 0; e < 4; ++e) sd.R[e] = R[e];
                        sd.s0 = Sh[0];
                        sd.s1 = Sh[1];
                        sd.p = pp;
                    }
                    __builtin_amdgcn_wave_barrier();
                    int r0, r1;
                    box_rows2<GEN>(R, lo, hi, ts, r0, r1);
                    const int nr = sv ? max(0, r1 - r0 + 1) : 0;
                    const int maxnr = wave_max(nr);
                    for (int rbase = 0; rbase < maxnr; rbase += RPS) {
                        const int jj = rbase + jrow;
                        const int r = r0 + jj;
                        int c0 = 0, cnt = 0;
                        if (jj < nr) {
                            int c1;
                            row_span2(R, r, lo, hi, ts, cut2, c0, c1);
                            cnt = max(0, c1 - c0 + 1);
                        }
                        const int incl = dpp_scan_add(cnt);
                        const int excl = incl - cnt;
                        const int total = __builtin_amdgcn_readlane(incl, 63);
                        int carry = 0;
                        // sample e0 + lane of this row block: owner lane, pixel, validity, and its loads
                        auto fetch_sample = [&](int e0, int& rr, int& cc, int& sl, bool& ok, Cx<float>& v,
                                                float& wv) {
                            const int e = e0 + lane;
                            const int lw = window_owner(cnt, excl, e0, carry, marks[wave]);
                            rr = __shfl(r, lw, 64);
                            cc = __shfl(c0, lw, 64) + (e - __shfl(excl, lw, 64));
                            sl = lw / RPS;
                            ok = e < total;
                            const Slot2& sd = slots[wave][sl];
                            ok = ok && !filtered(float(rr), float(cc), cut2) &&
                                 !(cc == 0 && (rr == g.n / 2 || rr < 0));  // Friedel half of x = 0
                            const int i = rr >= 0 ? rr : rr + g.n;
                            const int64_t pidx = (pose0 + sd.p) * int64_t(g.npix) + i * g.hp + cc;
                            v = ok ? src[pidx] : Cx<float>{0.f, 0.f};
                            wv = (WEIGHTS && ok) ? weights[pidx] : 0.f;
                        };
                        int rr, cc, sl;
                        bool ok;
                        Cx<float> v;
                        float wv;
                        fetch_sample(0, rr, cc, sl, ok, v, wv);
                        for (int e0 = 0; e0 < total; e0 += 64) {
                            // the next window's loads are in flight while this one is spread
                            int rr2 = 0, cc2 = 0, sl2 = 0;
                            bool ok2 = false;
                            Cx<float> v2 = {0.f, 0.f};
                            float wv2 = 0.f;
                            if (e0 + 64 < total) fetch_sample(e0 + 64, rr2, cc2, sl2, ok2, v2, wv2);
                            if (ok) {
                                if constexpr (PRIV)
                                    scatter_sample2_priv<CUBIC, MODE, WEIGHTS>(g, slots[wave][sl], rr, cc, v, wv,
                                                                               shifts != nullptr, pass == 1, tm,
                                                                               pacc[wave], pwacc[wave]);
                                else
                                    scatter_sample2<CUBIC, MODE, WEIGHTS>(g, slots[wave][sl], rr, cc, v, wv,
                                                                          shifts != nullptr, pass == 1, tm, acc_re,
                                                                          acc_im, acc_w);
                            }
                            rr = rr2;
                            cc = cc2;
                            sl = sl2;
                            ok = ok2;
                            v = v2;
                            wv = wv2;
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                }
            }
        }

        // add the partial tile into the image (cells past the stored range are dropped taps)
        __syncthreads();
        if (pend > p0) {
            for (int e = tid; e < T2; e += kThreads) {
                const int lc = e % TC, lr = e / TC;
                const int c = tc + lc, r = tr + lr;
                if (c >= H || r > half) continue;
                const int re = r < 0 ? r + N : r;
                const int64_t idx = b * g.vol + int64_t(re) * H + c;
                const int a = (e - lc) + ((lc + swizzle2(lr)) & (TC - 1));
                double vr, vi, vw = 0.0;
                if constexpr (PRIV) {
                    const int pa = lr * PS + lc;
                    vr = vi = 0.0;
#pragma unroll
                    for (int k = 0; k < NW; ++k) {
                        vr += double(pacc[k][pa].x);
                        vi += double(pacc[k][pa].y);
                        if (WEIGHTS) vw += double(pwacc[k][pa]);
                    }
                } else {
                    vr = acc_re[a];
                    vi = acc_im[a];
                    if (WEIGHTS) vw = acc_w[a];
                }
                if (vr != 0.0) atomic_add(&dst[idx].re, float(vr));
                if (vi != 0.0) atomic_add(&dst[idx].im, float(vi));
                if (WEIGHTS && vw != 0.0) atomic_add(&wdst[idx], float(vw));
            }
        }
        __syncthreads();
    }
}

// Hermitian completion of the x = 0 column after an unmirrored accumulation:
// every x = 0 contribution v of the reference is also added, conjugated, at
// the partner cell -r (projection_utils.h:398-405, 481-492), so the final
// value of a cell is A(r) + conj(A(-r)) (weights: A_w(r) + A_w(-r)).  One lane
// per unordered pair; the self-partnered cells r = 0 and r = N/2 are kept.
template <bool WEIGHTS>
__global__ __launch_bounds__(kBlock) void k_mirror2_x0(Geom g, Cx<float>* __restrict__ dst,
                                                       float* __restrict__ wdst) {
    const int N = g.N, H = g.H;
    for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < g.B * N; e += int64_t(gridDim.x) * kBlock) {
        const int64_t b = e / N;
        const int re = int(e - b * N);
        const int rm = re == 0 ? 0 : N - re;
        if (rm <= re) continue;  // self-partnered, or handled by the partner's lane
        const int64_t i0 = b * g.vol + int64_t(re) * H, i1 = b * g.vol + int64_t(rm) * H;
        const Cx<float> a = dst[i0], m = dst[i1];
        dst[i0] = Cx<float>{a.re + m.re, a.im - m.im};
        dst[i1] = Cx<float>{m.re + a.re, m.im - a.im};
        if (WEIGHTS) {
            const float wa = wdst[i0], wm = wdst[i1];
            wdst[i0] = wa + wm;
            wdst[i1] = wm + wa;
        }
    }
}

// Workgroups of a launch of `kernel` over `items`: one per item (rotations), or the persistent
// GEN grid.
template <bool GEN>
unsigned grid2_of(int64_t items, const void* kernel) {
    const int64_t slots = kXcds * xcd_per<kRun>(items);
    if (!GEN) return grid_for(slots);
    const int64_t most = gen_grid(kernel, kThreads);
    return grid_for(slots > most ? most : slots);
}

template <bool CUBIC, int MODE, bool WEIGHTS, int KP, bool PRIV, bool GEN>
hipError_t scatter2_one(const Geom& g, const TileSpec2& ts, const void* src, const void* weights, const void* rot,
                        const void* shifts, void* dst, void* wdst, CallPoses* cp, int gl, hipStream_t s) {
    const int64_t work = g.B * ts.ksplit * (GEN ? int64_t(ts.nr_2) * ts.nc_2 : int64_t(ts.nr) * ts.nc);
    if (work == 0) return hipSuccess;
    const auto k = k_scatter2_tiled<CUBIC, MODE, WEIGHTS, KP, PRIV, GEN>;
    hipLaunchKernelGGL(k, dim3(grid2_of<GEN>(work, (const void*)k)), dim3(kThreads), 0, s, g, ts, (const Cx<float>*)src, (const float*)weights, (const float*)rot,
                       (const float*)shifts, (Cx<float>*)dst, (float*)wdst, cp, gl);
    return hipGetLastError();
}

// Poses per wave batch, and wave-private accumulation: one pose per window keeps a window's
// samples >= os * (smallest singular value) apart (less rounding), beyond sqrt(2) (the diagonal
// of a cell) when that is 1.5 or more.
template <bool CUBIC, int MODE, bool WEIGHTS, bool GEN>
hipError_t scatter2_kp(const Geom& g, const TileSpec2& ts, const void* src, const void* weights, const void* rot,
                       const void* shifts, void* dst, void* wdst, CallPoses* cp, int gl, hipStream_t s) {
    if (g.os * (GEN ? kScaleMin : 1.0) >= kPrivOs)
        return scatter2_one<CUBIC, MODE, WEIGHTS, 1, true, GEN>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    if (ts.kp >= 4) return scatter2_one<CUBIC, MODE, WEIGHTS, 4, false, GEN>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    if (ts.kp == 2) return scatter2_one<CUBIC, MODE, WEIGHTS, 2, false, GEN>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    return scatter2_one<CUBIC, MODE, WEIGHTS, 1, false, GEN>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
}

// Rotations, then the other tiled poses (both add into the zero-filled image), then the
// x = 0 completion of the backprojection.
template <bool CUBIC, int MODE, bool WEIGHTS>
hipError_t scatter2_all(const Geom& g, const TileSpec2& ts, const void* src, const void* weights, const void* rot,
                        const void* shifts, void* dst, void* wdst, CallPoses* cp, int gl, hipStream_t s) {
    hipError_t e = scatter2_kp<CUBIC, MODE, WEIGHTS, false>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    if (e != hipSuccess) return e;
    e = scatter2_kp<CUBIC, MODE, WEIGHTS, true>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    if (e != hipSuccess || MODE != 0) return e;
    int64_t blocks = (g.B * g.N + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) return hipSuccess;
    hipLaunchKernelGGL(k_mirror2_x0<WEIGHTS>, dim3(unsigned(blocks)), dim3(kBlock), 0, s, g, (Cx<float>*)dst,
                       (float*)wdst);
    return hipGetLastError();
}

// ----------------------------------------------------------------------------- gather
// Tile-owner gathers of the 2D operators, over 32 x 32 (c, r) tiles of the
// signed frequency plane (origin ts.gorg, ts.gnt tiles per axis).  A sample is
// computed by the one tile that holds floor(x); the tile plus its stencil halo
// is staged in LDS with exactly the values the reference's sampler returns
// (Friedel conjugation and clamping applied), so the interpolation is
// bit-identical to the per-pixel one.
//
//   GMODE 0  forward projection into `out` (project_2d_forw).
//   GMODE 1  rotation/shift gradients of project_2d_back: `gsrc` holds
//            grad_projections; terms as cpu/2d/projection_2d_kernels.cpp:300-375.
//   GMODE 2  backproject_2d_back: grad_projections (`out`) gathered from
//            grad_data_rec (`rec`), grad_weights (`wout`) bilinearly from
//            grad_weight_rec (`gw`, a second staged tile with the weight-tap
//            rules), and with RS the rotation/shift gradients against the
//            projections `gsrc` (cpu/2d/backprojection_2d_kernels.cpp:420-520).
// In GMODE 1/2 a wave takes one pose at a time (KP = 1) and sums its terms
// before one atomic per gradient component.
constexpr int GC = kGat2, GR = kGat2;
constexpr double kTwoPi2 = 6.283185307179586476925286766559;

// Bicubic value and gradient with the 16 taps reduced along c first (value
// and d/dc weights), then r, with fused multiply-adds and the fp32 weight
// polynomials: the gradient carries the 1e-4 bar.  EXACT_V keeps the value in
// the reference's order and rounding ((s * wr) * wc summed over r then c, with
// its weights, interpolation_kernels.h:258-322) for outputs that are gathers.
template <bool EXACT_V, typename F>
__device__ __forceinline__ Interp<float> cubic2_grads(F&& fetch, float r, float c) {
    float cx, rx;
    const int cf = split_as<false>(c, cx), rf = split_as<false>(r, rx);
    auto w_of = [](float f, int j) { return EXACT_V ? cubic_w_tap<float>(f, j) : cubic_w_fast(f - float(j - 1)); };
    float wc[4], dwc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        wc[j] = w_of(cx, j);
        dwc[j] = cubic_dw_fast(cx - float(j - 1));
    }
    Interp<float> o;
    o.v = o.g[0] = o.g[1] = o.g[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float wr = w_of(rx, i), dwr = cubic_dw_fast(rx - float(i - 1));
        Cx<float> a = {0.f, 0.f}, bc = {0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const Cx<float> t = fetch(rf + i - 1, cf + j - 1);
            if (EXACT_V) o.v = cadd(o.v, cscale(cscale(t, wr), wc[j]));
            a = cfma(t, wc[j], a);
            bc = cfma(t, dwc[j], bc);
        }
        if (!EXACT_V) o.v = cfma(a, wr, o.v);
        o.g[0] = cfma(bc, wr, o.g[0]);
        o.g[1] = cfma(a, dwr, o.g[1]);
    }
    return o;
}

template <bool CUBIC, int KP, int GMODE, bool RS, bool WG, typename VS, bool GEN>
__global__ __launch_bounds__(kThreads) void k_gather2_tiled(Geom g, TileSpec2 ts, const Cx<VS>* __restrict__ rec,
                                                            const float* __restrict__ gw,
                                                            const float* __restrict__ rot,
                                                            const float* __restrict__ shifts,
                                                            Cx<float>* __restrict__ out, float* __restrict__ wout,
                                                            const Cx<float>* __restrict__ gsrc,
                                                            float* __restrict__ grot, float* __restrict__ gshift,
                                                            CallPoses* __restrict__ cp, int gl) {
    static_assert(GMODE == 0 || KP == 1, "the gradient modes sum one pose per wave batch");
    static_assert(GMODE != 2 || std::is_same<VS, float>::value, "complex-half volumes: forward and its gradients only");
    constexpr int LO = CUBIC ? 1 : 0, HI = CUBIC ? 2 : 1, WC = GC + LO + HI, WR = GR + LO + HI, W2 = WC * WR;
    constexpr int WW = (GMODE == 2 && WG) ? (GC + 1) * (GR + 1) : 1;  // bilinear weight taps
    constexpr int RPS = 64 / KP, NW = kThreads / 64, CH = 2048;
    constexpr bool GRADS = GMODE == 1 || (GMODE == 2 && RS);
    __shared__ Cx<float> vt[W2];
    __shared__ float wt[WW];
    __shared__ unsigned short plist[CH];
    __shared__ int pcnt[2];
    __shared__ Slot2 slots[NW][KP];
    __shared__ int marks[NW][64];
    __shared__ int gen_sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int slot = lane / RPS, jrow = lane % RPS;
    const int N = g.N, H = g.H;
    // samples lie within |x| <= rho_k: rotations reach rho_unit + 1 (and have nothing to do when
    // the call has none); GEN poses the call's own reach, up to kScaleMax times farther, on the
    // part of the wide grid that this reach needs
    const int any_rot = GEN ? 1 : call_flag(&cp->any_rot);
    float rho_k = ts.rho_unit + 1.0f;
    int gnt = ts.gnt, gorg = ts.gorg;
    if constexpr (GEN) {
        rho_k = fminf(ts.rho, cp->gen_reach);
        if (!(rho_k > 0.f)) return;  // no such pose in this call
        const int h = half_tiles_for(rho_k, GC, ts.gnt2 / 2);
        gnt = 2 * h;
        gorg = ts.gorg2 + (ts.gnt2 / 2 - h) * GC;
    }
    const int64_t items = g.B * ts.gksplit * int64_t(gnt) * gnt;
    const float cut2 = float(g.cut2);
    for (Slots<GEN> sl(xcd_per<kRun>(items), slot_counters<GEN>(cp, gl), &gen_sh); sl.ok(); sl.next(&gen_sh)) {
        const int64_t slot_i = sl.s;
        const int64_t w = xcd_item<kRun>(slot_i);
        if (w >= items) continue;
        const int kc = int(w % gnt);
        int64_t q = w / gnt;
        const int kr = int(q % gnt);
        q /= gnt;
        const int jr = int(q % ts.gksplit);
        const int64_t b = q / ts.gksplit;
        const int p0 = jr * ts.gprange, p1 = min(int(g.P), p0 + ts.gprange);
        if (!any_rot) return;  // rotation kernel, no rotation in the call
        const int tc = gorg + kc * GC, tr = gorg + kr * GR;
        // samples owned by this tile: floor(x) in [t, t + edge) on both axes (+ slack)
        const float lo[2] = {float(tc) - ts.eps, float(tr) - ts.eps};
        const float hi[2] = {float(tc + GC) + ts.eps, float(tr + GR) + ts.eps};
        float dist2 = 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float d = lo[k] > 0.f ? lo[k] : (hi[k] < 0.f ? -hi[k] : 0.f);
            dist2 += d * d;
        }
        if (dist2 > rho_k * rho_k || p1 <= p0) continue;
        const int64_t rb = g.B_rot == 1 ? 0 : b, sb = g.B_shift == 1 ? 0 : b;
        const float* rotb = rot + rb * g.P * 4;
        const float* shb = shifts ? shifts + sb * g.P * 2 : nullptr;
        const int64_t pose0 = b * g.P;
        auto lds = [&](int r, int c) { return vt[(r - (tr - LO)) * WC + (c - (tc - LO))]; };
        bool loaded = false;
        for (int pbase = p0; pbase < p1; pbase += CH) {
            // cull: rotations whose sample half-disc reaches the tile
            __syncthreads();
            if (tid == 0) pcnt[0] = 0;
            __syncthreads();
            for (int k = tid; k < CH && pbase + k < p1; k += kThreads) {
                float R[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) R[e] = rotb[int64_t(pbase + k) * 4 + e];
                float as[2];
                if (pose_of_class2<GEN>(R, as) && half_plane_hits2(as, lo, hi)) plist[atomicAdd(&pcnt[0], 1)] = k;
            }
            __syncthreads();
            const int np = pcnt[0];
            if (np == 0) continue;
            if (!loaded) {
                const Cx<VS>* recb = rec + b * g.vol;
                for (int e = tid; e < W2; e += kThreads) {
                    const int r = tr - LO + e / WC, c = tc - LO + e % WC;
                    vt[e] = CUBIC ? fetch2_cubic(recb, N, H, r, c) : fetch2(recb, N, H, r, c);
                }
                if constexpr (GMODE == 2 && WG) {
                    const float* gwb = gw + b * g.vol;
                    for (int e = tid; e < WW; e += kThreads)
                        wt[e] = weight_tap<2>(gwb, N, H, 0, tr + e / (GC + 1), tc + e % (GC + 1));
                }
                __syncthreads();
                loaded = true;
            }
            auto pose_at = [&](int k) { return pbase + int(plist[k]); };
            int base = wave * KP;
            float Rn[4], Sn[2];
            if (base < np) load_pose2(rotb, shb, pose_at(min(base + slot, np - 1)), Rn, Sn);
            for (; base < np; base += NW * KP) {
                const bool sv = base + slot < np;
                const int pp = pose_at(min(base + slot, np - 1));
                float R[4], Sh[2];
#pragma unroll
                for (int e = 0; e < 4; ++e) R[e] = Rn[e];
                Sh[0] = Sn[0];
                Sh[1] = Sn[1];
                if (base + NW * KP < np) load_pose2(rotb, shb, pose_at(min(base + NW * KP + slot, np - 1)), Rn, Sn);
                if (jrow == 0 && sv) {
                    Slot2& sd = slots[wave][slot];
#pragma unroll
                    for (int e = 0; e < 4; ++e) sd.R[e] = R[e];
                    sd.s0 = Sh[0];
                    sd.s1 = Sh[1];
                    sd.p = pp;
                }
                __builtin_amdgcn_wave_barrier();
                float acc[6];  // GMODE 1/2: 4 rotation and 2 shift terms of this lane's samples
#pragma unroll
                for (int k = 0; k < 6; ++k) acc[k] = 0.f;
                int r0, r1;
                box_rows2<GEN>(R, lo, hi, ts, r0, r1);
                const int nr = sv ? max(0, r1 - r0 + 1) : 0;
                const int maxnr = wave_max(nr);
                for (int rbase = 0; rbase < maxnr; rbase += RPS) {
                    const int jj = rbase + jrow;
                    const int r = r0 + jj;
                    int c0 = 0, cnt = 0;
                    if (jj < nr) {
                        int c1;
                        row_span2(R, r, lo, hi, ts, cut2, c0, c1);
                        cnt = max(0, c1 - c0 + 1);
                    }
                    const int incl = dpp_scan_add(cnt);
                    const int excl = incl - cnt;
                    const int total = __builtin_amdgcn_readlane(incl, 63);
                    int carry = 0;
                    for (int e0 = 0; e0 < total; e0 += 64) {
                        const int e = e0 + lane;
                        const int lw = window_owner(cnt, excl, e0, carry, marks[wave]);
                        const int rr = __shfl(r, lw, 64);
                        const int cc = __shfl(c0, lw, 64) + (e - __shfl(excl, lw, 64));
                        if (e >= total) continue;
                        // every field of the sample's pose slot is read before the tests, so that the
                        // reads go out together (one LDS round trip) instead of one per test
                        const Slot2& sdl = slots[wave][lw / RPS];
                        Slot2 sd;
#pragma unroll
                        for (int k = 0; k < 4; ++k) sd.R[k] = sdl.R[k];
                        sd.s0 = sdl.s0;
                        sd.s1 = sdl.s1;
                        sd.p = sdl.p;
                        const float fr = float(rr), fc = float(cc);
                        float x[2];
                        rotate_pix(sd.R, fr, fc, g.os, x);
                        const int fxc = int(floorf(x[0])), fxr = int(floorf(x[1]));
                        // outside the cutoff, the Friedel half of the x = 0 line (the backward ops skip
                        // it), or not owned by this tile
                        bool skip = filtered(fr, fc, cut2);
                        if (GMODE != 0) skip |= (cc == 0) & ((rr == g.n / 2) | (rr < 0));
                        skip |= (fxc < tc) | (fxc >= tc + GC) | (fxr < tr) | (fxr >= tr + GR);
                        asm volatile("" ::"v"(sd.s0), "v"(sd.s1), "v"(sd.p));
                        if (skip) continue;
                        const int i = rr >= 0 ? rr : rr + g.n;
                        const int64_t pidx = (pose0 + sd.p) * int64_t(g.npix) + i * g.hp + cc;
                        Interp<float> ip;
                        if constexpr (CUBIC && GRADS) ip = cubic2_grads<GMODE == 2>(lds, x[1], x[0]);
                        else if constexpr (CUBIC) ip = cubic2<float, false, false>(lds, x[1], x[0]);
                        else ip = lerp2<float, GRADS, false>(lds, x[1], x[0]);
                        const Cx<float> ph = shifts ? phase_hw(fr, fc, sd.s0, sd.s1, g.phase_k) : Cx<float>{1.f, 0.f};
                        if constexpr (GMODE == 0) {
                            out[pidx] = shifts ? cmul(ip.v, ph) : ip.v;
                        } else {
                            if constexpr (GMODE == 2) {
                                out[pidx] = shifts ? cmul(ip.v, ph) : ip.v;
                                if constexpr (WG) {
                                    // bilinear as weight_grad_interp<2>
                                    float cx, rx;
                                    const int cf = split_as<false>(x[0], cx), rf = split_as<false>(x[1], rx);
                                    const float* wr0 = &wt[(rf - tr) * (GC + 1) + (cf - tc)];
                                    const float p00 = wr0[0], p01 = wr0[1], p10 = wr0[GC + 1], p11 = wr0[GC + 2];
                                    const float q0 = p00 + (p01 - p00) * cx;
                                    const float q1 = p10 + (p11 - p10) * cx;
                                    wout[pidx] = q0 + (q1 - q0) * rx;
                                }
                            }
                            if constexpr (GRADS) {
                                // project_2d_back pairs g' = g * conj(phase) with dF/dx and g with the
                                // modulated value; backproject_2d_back pairs proj * conj(phase) with both
                                const Cx<float> g0 = gsrc[pidx];
                                const Cx<float> gg = shifts ? cmul(g0, cconj(ph)) : g0;
                                const Cx<float> sv_ = GMODE == 1 ? g0 : gg;
                                const Cx<float> mv = GMODE == 1 ? cmul(ip.v, ph) : ip.v;
                                // Re(gg conj(dF/dx_row * s)) = s Re(gg conj(dF/dx_row)) with s = (c, r) * os, and
                                // Re(sv conj(i k mv)) = k (sv.im mv.re - sv.re mv.im) with k = -2 pi (r, c) / n:
                                // the sums take (c, r) and the constants os and -2 pi / n scale the pose's totals
                                if (grot) {
#pragma unroll
                                    for (int row = 0; row < 2; ++row) {
                                        const float d = fmaf(gg.re, ip.g[row].re, gg.im * ip.g[row].im);
                                        acc[row * 2 + 0] = fmaf(d, fc, acc[row * 2 + 0]);
                                        acc[row * 2 + 1] = fmaf(d, fr, acc[row * 2 + 1]);
                                    }
                                }
                                if (gshift) {
                                    const float cr = fmaf(sv_.im, mv.re, -(sv_.re * mv.im));
                                    acc[4] = fmaf(cr, fr, acc[4]);
                                    acc[5] = fmaf(cr, fc, acc[5]);
                                }
                            }
                        }
                    }
                }
                if constexpr (GRADS) {
                    if (grot) {
                        const float os = float(g.os);
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float t = wave_sum(acc[k]) * os;
                            if (lane == 0 && sv) atomic_add(&grot[(rb * g.P + pp) * 4 + k], t);
                        }
                    }
                    if (gshift) {
                        const float kn = float(-kTwoPi2 / double(g.n));
                        const float t0 = wave_sum(acc[4]) * kn, t1 = wave_sum(acc[5]) * kn;
                        if (lane == 0 && sv) {
                            atomic_add(&gshift[(sb * g.P + pp) * 2], t0);
                            atomic_add(&gshift[(sb * g.P + pp) * 2 + 1], t1);
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        __syncthreads();
    }
}

template <bool CUBIC, int KP, int GMODE, bool RS, bool WG, typename VS = float>
hipError_t gather2_launch(const Geom& g, const TileSpec2& ts, const void* rec, const void* gw, const void* rot,
                          const void* shifts, void* out, void* wout, const void* gsrc, void* grot, void* gshift,
                          CallPoses* cp, int gl, hipStream_t s) {
    // rotations, then the other tiled poses (their samples and gradient terms are their own)
    const int64_t work = g.B * ts.gksplit * int64_t(ts.gnt) * ts.gnt;
    if (work > 0) {
        const auto kr = k_gather2_tiled<CUBIC, KP, GMODE, RS, WG, VS, false>;
        hipLaunchKernelGGL(kr, dim3(grid2_of<false>(work, (const void*)kr)), dim3(kThreads), 0, s, g, ts, (const Cx<VS>*)rec, (const float*)gw, (const float*)rot,
                           (const float*)shifts, (Cx<float>*)out, (float*)wout, (const Cx<float>*)gsrc,
                           (float*)grot, (float*)gshift, cp, gl);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const int64_t work2 = g.B * ts.gksplit * int64_t(ts.gnt2) * ts.gnt2;
    if (work2 == 0) return hipSuccess;
    const auto kg = k_gather2_tiled<CUBIC, KP, GMODE, RS, WG, VS, true>;
    hipLaunchKernelGGL(kg, dim3(grid2_of<true>(work2, (const void*)kg)), dim3(kThreads), 0, s, g, ts, (const Cx<VS>*)rec, (const float*)gw, (const float*)rot,
                       (const float*)shifts, (Cx<float>*)out, (float*)wout, (const Cx<float>*)gsrc, (float*)grot,
                       (float*)gshift, cp, gl);
    return hipGetLastError();
}

template <bool CUBIC, typename VS>
hipError_t gather2_forw(const Geom& g, const TileSpec2& ts, const void* rec, const void* rot, const void* shifts,
                        void* out, CallPoses* cp, int gl, hipStream_t s) {
    if (ts.kp_gather >= 4)
        return gather2_launch<CUBIC, 4, 0, false, false, VS>(g, ts, rec, nullptr, rot, shifts, out, nullptr, nullptr,
                                                             nullptr, nullptr, cp, gl, s);
    if (ts.kp_gather == 2)
        return gather2_launch<CUBIC, 2, 0, false, false, VS>(g, ts, rec, nullptr, rot, shifts, out, nullptr, nullptr,
                                                             nullptr, nullptr, cp, gl, s);
    return gather2_launch<CUBIC, 1, 0, false, false, VS>(g, ts, rec, nullptr, rot, shifts, out, nullptr, nullptr,
                                                         nullptr, nullptr, cp, gl, s);
}

template <bool CUBIC>
hipError_t gather2_modes(int mode, const Geom& g, const TileSpec2& ts, const void* rec, const void* gw,
                         const void* rot, const void* shifts, void* out, void* wout, const void* gsrc, void* grot,
                         void* gshift, CallPoses* cp, int gl, hipStream_t s) {
    if (mode == 0) return gather2_forw<CUBIC, float>(g, ts, rec, rot, shifts, out, cp, gl, s);
    if (mode == 1)
        return gather2_launch<CUBIC, 1, 1, true, false>(g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot, gshift, cp, gl, s);
    const bool rs = grot || gshift;
    if (wout)
        return rs ? gather2_launch<CUBIC, 1, 2, true, true>(g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot,
                                                            gshift, cp, gl, s)
                  : gather2_launch<CUBIC, 1, 2, false, true>(g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot,
                                                             gshift, cp, gl, s);
    return rs ? gather2_launch<CUBIC, 1, 2, true, false>(g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot, gshift, cp, gl, s)
              : gather2_launch<CUBIC, 1, 2, false, false>(g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot,
                                                          gshift, cp, gl, s);
}

}  // namespace

hipError_t launch_gather2_tiled(bool cubic, int mode, const Geom& g, const TileSpec2& ts, const void* rec,
                                const void* gw, const void* rot, const void* shifts, void* out, void* wout,
                                const void* gsrc, void* grot, void* gshift, CallPoses* cp, int gl, hipStream_t s, bool rec_half) {
    if (rec_half) {
        if (mode == 0)
            return cubic ? gather2_forw<true, __half>(g, ts, rec, rot, shifts, out, cp, gl, s)
                         : gather2_forw<false, __half>(g, ts, rec, rot, shifts, out, cp, gl, s);
        if (mode != 1) return hipErrorInvalidValue;
        if (!grot && !gshift) return hipSuccess;
        return cubic ? gather2_launch<true, 1, 1, true, false, __half>(g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot,
                                                                     gshift, cp, gl, s)
                     : gather2_launch<false, 1, 1, true, false, __half>(g, ts, rec, gw, rot, shifts, out, wout, gsrc,
                                                                      grot, gshift, cp, gl, s);
    }
    if (mode == 1 && !grot && !gshift) return hipSuccess;
    return cubic ? gather2_modes<true>(mode, g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot, gshift, cp, gl, s)
                 : gather2_modes<false>(mode, g, ts, rec, gw, rot, shifts, out, wout, gsrc, grot, gshift, cp, gl, s);
}

hipError_t launch_scatter2_tiled(bool cubic, int mode, const Geom& g, const TileSpec2& ts, const void* src,
                                 const void* weights, const void* rot, const void* shifts, void* dst, void* wdst,
                                 CallPoses* cp, int gl, hipStream_t s) {
    if (mode == 0) {
        if (weights)
            return cubic ? scatter2_all<true, 0, true>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s)
                         : scatter2_all<false, 0, true>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
        return cubic ? scatter2_all<true, 0, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s)
                     : scatter2_all<false, 0, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s);
    }
    return cubic ? scatter2_all<true, 1, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s)
                 : scatter2_all<false, 1, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s);
}

}  // namespace tp
