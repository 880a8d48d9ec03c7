// Tile-owner kernels for the 3D operators (fp32).
//
// The reference walks poses and pixels and gathers/scatters each sample's
// stencil straight from/to memory (cpu/3d/projection_3d_to_2d_kernels.cpp:156-209,
// cpu/3d/backprojection_2d_to_3d_kernels.cpp:182-292).  At 2x oversampling
// neighbouring samples are two voxels apart, so every sample touches ~4 fresh
// cache lines, and the scatter is two float atomics per tap into HBM.
//
// Here a workgroup owns a tile of the volume held in LDS and inverts the
// loop: it culls the poses whose slice plane crosses the tile, and for each
// such pose enumerates exactly the grid samples whose stencil reaches the
// tile (one lane per (pose, row) computes the row's column interval, a wave
// prefix sum packs the samples of several poses densely onto the lanes).
// The tiles around the origin are crossed by nearly every pose; they are
// split into pose ranges ("core" work items) that are dispatched first.
//
//   k_forw3_tiled     forward projection.  The tile plus its stencil halo is
//                     staged in LDS holding exactly the value the reference's
//                     sampler returns for each integer coordinate (Friedel
//                     conjugation, clamping and wrapping applied), over the
//                     full signed frequency range, so the interpolation is
//                     bit-identical.  A sample is computed by the one tile
//                     that contains floor(x).
//   k_scatter3_tiled  backprojection (data + weights) and the reconstruction
//                     gradient of the projection backward.  Contributions are
//                     accumulated in fp64 LDS (gfx950's LDS fp32 atomic add
//                     runs at ~0.3 lanes/clk/CU, fp64 at ~7.7) and every
//                     stored cell of the tile is written once with a plain
//                     store: no zero fill and no global atomics, except for
//                     the split core tiles, which add their partial tiles
//                     into a zeroed region.  The Hermitian x = 0 mirror of
//                     the backprojection is applied afterwards by k_mirror_x0.
//
// Poses whose first two matrix columns a, b have singular values in
// [kScaleMin, kScaleMax] take this path (pose_tiled3); the per-pixel kernels
// handle the others and write the masked pixels of the forward.  Each kernel
// comes in two instantiations:
//   GEN = false  rotations (columns orthonormal to kRotationTol), one
//                workgroup per work item over the grid their samples reach
//                (the forward family's: per work item of TileSpec::flist,
//                the tiles within that reach, when the C ABI has the list);
//   GEN = true   the other tiled poses (scaled, anisotropically magnified or
//                sheared matrices), launched after the first on a smaller
//                grid (the forward's: a quarter of the rotation grid's
//                workgroups, each stepping over the slots; the scatter's:
//                persistent, with per-XCD counters).  A per-call pre-pass
//                (k_call_poses) records the largest singular value among
//                such poses; the workgroups exit at once when there is none,
//                so rotation-only calls pay one short launch (and the
//                rotation kernels, when the call has no rotation, exit at
//                their first slot).  A sample x = sc a + sr b of
//                such a pose has sc = as . x and sr = bs . x with the dual
//                basis (as, bs), which bounds the rows and the half plane
//                sc >= 0 that can reach a box; the grid reaches samples up to
//                kScaleMax times farther out.  Scatters add their tiles into
//                the volume.
#include <type_traits>

#include "tp_device.hh"
#include "tp_launch.hh"
#include "tp_tiled_common.hh"

namespace tp {

namespace {

constexpr int L = kTileEdge, LD = kTileEdgeD;  // forward tile edges (voxels): c and r, d
constexpr int SC = kScTC, SR = kScTR, SD = kScTD, S3 = SC * SR * SD;  // scatter tile
constexpr int kForwThreads = 256;     // forward workgroup
constexpr int kScatterThreads = 256;  // scatter workgroup

// Does the slice plane (through the origin, spanned by columns 0 and 1 of R)
// pass within the box [lo, hi] (x-order c, r, d)?
__device__ __forceinline__ bool plane_hits(const float* R, const float* lo, const float* hi) {
    const float n0 = R[3] * R[7] - R[6] * R[4];
    const float n1 = R[6] * R[1] - R[0] * R[7];
    const float n2 = R[0] * R[4] - R[3] * R[1];
    const float m0 = 0.5f * (lo[0] + hi[0]), m1 = 0.5f * (lo[1] + hi[1]), m2 = 0.5f * (lo[2] + hi[2]);
    const float h0 = 0.5f * (hi[0] - lo[0]), h1 = 0.5f * (hi[1] - lo[1]), h2 = 0.5f * (hi[2] - lo[2]);
    return fabsf(n0 * m0 + n1 * m1 + n2 * m2) <= fabsf(n0) * h0 + fabsf(n1) * h1 + fabsf(n2) * h2;
}

// Largest sc = as . x over the box; samples have sc >= 0.
__device__ __forceinline__ bool half_plane_hits(const float* as, const float* hi, const float* lo) {
    float uhi = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) uhi += as[k] >= 0.f ? as[k] * hi[k] : as[k] * lo[k];
    return uhi >= 0.f;
}

// Is the pose of this instantiation's class (rotation, or GEN: another tiled
// matrix)?  `as` receives the half-plane vector (column 0, or its dual).
// `all_rot`: every pose of the call is a rotation (CallPoses), so a rotation
// kernel needs no test.
template <bool GEN>
__device__ __forceinline__ bool pose_of_class(const float* R, float* as, bool all_rot) {
    if constexpr (GEN) {
        const PoseGram gr = pose_gram3(R);
        if (gram_is_rotation(gr) || !gram_tiled(gr)) return false;
        float bs[3];
        pose_dual3(R, gr, as, bs);
        return true;
    } else {
        as[0] = R[0];
        as[1] = R[3];
        as[2] = R[6];
        return all_rot || gram_is_rotation(pose_gram3(R));
    }
}

// Pose of this class whose plane and half plane reach the box.
template <bool GEN>
__device__ __forceinline__ bool pose_hits(const float* R, const float* lo, const float* hi, bool all_rot) {
    float as[3];
    return pose_of_class<GEN>(R, as, all_rot) && plane_hits(R, lo, hi) && half_plane_hits(as, hi, lo);
}

// Rows r (sr = r*os = bs . x) whose samples can lie in the box: bs is a
// rotation's column 1, or (GEN) the dual basis vector.
template <bool GEN>
__device__ __forceinline__ void box_rows(const float* R, const float* lo, const float* hi, const TileSpec& ts,
                                         int& r0, int& r1) {
    float as[3], bs[3] = {R[1], R[4], R[7]};
    if constexpr (GEN) pose_dual3(R, pose_gram3(R), as, bs);
    float vlo = 0.f, vhi = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float b = bs[k];
        vlo += b >= 0.f ? b * lo[k] : b * hi[k];
        vhi += b >= 0.f ? b * hi[k] : b * lo[k];
    }
    r0 = max(ts.rmin, to_int_clamped(ceilf(vlo * ts.inv_os)));
    r1 = min(ts.rmax, to_int_clamped(floorf(vhi * ts.inv_os)));
}

// Columns c of row r whose sample x = c*os*a + r*os*b lies in the box (the
// box already carries the slack that covers rounding), within the pixel grid
// and (up to one column) the cutoff disc.
__device__ __forceinline__ void row_span(const float* R, int r, const float* lo, const float* hi, const TileSpec& ts,
                                         float cut2, int& c0, int& c1) {
    const float ros = float(r) * ts.os;
    float l = -3.0e38f, h = 3.0e38f;
    bool empty = false;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float a = R[3 * k], base = ros * R[3 * k + 1];
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

// Sample position of pixel (r, c): rotate<3> without its R[k][2] * 0 terms.
// Adding that signed zero to the other two terms can only flip the sign of a
// zero coordinate, which floors to the same cell with the same fraction.
// OSX: os is a float value (float(os) == os), so c * os is exact in double and
// float(double(c) * os) is the correctly rounded float product c * float(os).
template <bool OSX>
__device__ __forceinline__ void rotate_slice(const float* __restrict__ R, float r, float c, double os, float* x) {
    const float sc = OSX ? c * float(os) : float(double(c) * os), sr = OSX ? r * float(os) : float(double(r) * os);
    x[0] = R[0] * sc + R[1] * sr;
    x[1] = R[3] * sc + R[4] * sr;
    x[2] = R[6] * sc + R[7] * sr;
}

// rotate_slice on the R6 layout (the same products in the same order).
template <bool OSX>
__device__ __forceinline__ void rotate_slice6(const float* __restrict__ R6, float r, float c, double os, float* x) {
    const float sc = OSX ? c * float(os) : float(double(c) * os), sr = OSX ? r * float(os) : float(double(r) * os);
    x[0] = R6[0] * sc + R6[1] * sr;
    x[1] = R6[2] * sc + R6[3] * sr;
    x[2] = R6[4] * sc + R6[5] * sr;
}
// row_span on the R6 layout.
__device__ __forceinline__ void row_span6(const float* R6, int r, const float* lo, const float* hi,
                                          const TileSpec& ts, float cut2, int& c0, int& c1) {
    const float R[9] = {R6[0], R6[1], 0.f, R6[2], R6[3], 0.f, R6[4], R6[5], 0.f};
    row_span(R, r, lo, hi, ts, cut2, c0, c1);
}

// Per-wave sample queue.  A row block's samples are written once, in
// flattened order, as packed (slot, c, r) entries; windows of 64 lanes then
// read their samples straight from the queue.  Rows hold `cnt` samples from
// column c0 at flattened index `excl`; entries [q0, q0 + QCAP) are written.
// |r| and c are at most n / 2 <= 16383 (use_tiles keeps n <= 32766).
constexpr unsigned kQRowBias = 0x4000u;  // r + bias in bits 0-14, c in bits 15-28, slot in 29-31
__device__ __forceinline__ unsigned q_pack(int r, int c, int slot) {
    return ((unsigned(r) + kQRowBias) & 0x7fffu) | (unsigned(c) << 15) | (unsigned(slot) << 29);
}
__device__ __forceinline__ void q_unpack(unsigned e, int& r, int& c, int& slot) {
    r = int(e & 0x7fffu) - int(kQRowBias);
    c = int((e >> 15) & 0x3fffu);
    slot = int(e >> 29);
}
template <int QCAP>
__device__ __forceinline__ void q_fill(unsigned* q, int r, int c0, int cnt, int excl, int slot, int q0) {
    __builtin_amdgcn_wave_barrier();  // the previous entries have been read
    const int lo = max(excl, q0), hi = min(excl + cnt, q0 + QCAP);
    for (int e = lo; e < hi; ++e) q[e - q0] = q_pack(r, c0 + (e - excl), slot);
    __builtin_amdgcn_wave_barrier();
}
// The same for entries [q0, q0 + room) written after the first `at` entries of the queue.
__device__ __forceinline__ void q_fill_at(unsigned* q, int at, int r, int c0, int cnt, int excl, int slot, int q0,
                                          int room) {
    __builtin_amdgcn_wave_barrier();  // the previous entries have been read
    const int lo = max(excl, q0), hi = min(excl + cnt, q0 + room);
    for (int e = lo; e < hi; ++e) q[at + (e - q0)] = q_pack(r, c0 + (e - excl), slot);
    __builtin_amdgcn_wave_barrier();
}

// Per-wave copy of a pose of a wave batch: columns 0 and 1 of the matrix
// (R6 = R[0], R[1], R[3], R[4], R[6], R[7]: the tiled kernels read no other
// entry), the shifts, the pose's first pixel in the [B, P, n, n/2+1]
// projections, the first row of its samples in the box and the index of that
// row in the batch's flattened row list.  Kernels that carry a partly filled
// sample window into the next batch keep two sets per wave (the current
// batch's and the previous one's, whose samples the carried window may hold).
struct Slot {
    float R6[6];
    float s0, s1;
    int64_t base;
    int r0, start;
};

// The tiled kernels read columns 0 and 1 of a pose only (the slice plane and
// its sample grid); column 2 is not loaded (zero), which cuts the bytes the
// pose culls read per tile by a third.
__device__ __forceinline__ void load_rot(const float* __restrict__ Rg, float* R) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        R[3 * k] = Rg[3 * k];
        R[3 * k + 1] = Rg[3 * k + 1];
        R[3 * k + 2] = 0.f;
    }
}
// Rotation and shift of pose p (shifts may be absent: zeros).
__device__ __forceinline__ void load_pose(const float* __restrict__ rotb, const float* __restrict__ shb, int p,
                                          float* R, float* S) {
    load_rot(rotb + int64_t(p) * 9, R);
    S[0] = shb ? shb[2 * int64_t(p)] : 0.f;
    S[1] = shb ? shb[2 * int64_t(p) + 1] : 0.f;
}

constexpr int kRunForw = 64, kRunScatter = 128;  // measured at the headline
constexpr int kForwFlatKP = 5;  // forward poses per wave batch for poses of up to 16 rows (about 11 rows each)

// Work items: first the core tiles, one item per (batch, tile, pose range),
// then every tile of every batch with all poses (core tiles skipped there).
struct Item {
    int64_t b;
    int kd, kr, kc;
    int p0, p1;
    bool core, skip;
};
__device__ __forceinline__ Item item_of(int64_t w, int64_t B, int P, int nd, int nr, int nc, int d0, int d1, int r0,
                                        int r1, int c0, int c1, int ksplit, int prange) {
    Item it;
    const int cd = d1 - d0, cr = r1 - r0, cc = c1 - c0;
    const int64_t ncore = int64_t(cd) * cr * cc * ksplit;
    it.skip = false;
    if (w < B * ncore) {
        it.core = true;
        it.b = w / ncore;
        int64_t q = w - it.b * ncore;
        const int j = int(q % ksplit);
        q /= ksplit;
        it.kc = c0 + int(q % cc);
        it.kr = r0 + int((q / cc) % cr);
        it.kd = d0 + int(q / (int64_t(cc) * cr));
        it.p0 = j * prange;
        it.p1 = min(P, it.p0 + prange);
    } else {
        it.core = false;
        const int64_t per_b = int64_t(nd) * nr * nc;
        const int64_t q = w - B * ncore;
        it.b = q / per_b;
        const int t = int(q - it.b * per_b);
        it.kc = t % nc;
        it.kr = (t / nc) % nr;
        it.kd = t / (nc * nr);
        it.p0 = 0;
        it.p1 = P;
        it.skip = ksplit > 1 && it.kd >= d0 && it.kd < d1 && it.kr >= r0 && it.kr < r1 && it.kc >= c0 && it.kc < c1;
    }
    return it;
}

// Poses culled per phase: each lane tests kChunk / NT of them, the survivors'
// indices (relative to the phase) go to an LDS list.
constexpr int kCullInFlight = 2;  // rotations loaded together per lane (scatter)
constexpr int kCullInFlightF = 2; // the same, forward
constexpr int kChunk = 1024;      // poses culled per phase

// List entries: pose index relative to the phase, plus which boxes it crosses.
constexpr unsigned kHit1 = 1u << 14, kHit2 = 1u << 15, kPoseMask = kHit1 - 1;
static_assert(kChunk <= int(kPoseMask) + 1, "pose index must fit below the flag bits");

// Cull poses [pbase, pend) (at most CH) against up to two boxes with a
// workgroup of NT lanes; returns the count.
template <int NT, bool TWO, int CH, bool GEN>
__device__ __forceinline__ int cull_chunk(const float* __restrict__ rotb, int pend, int pbase, const float* lo1,
                                          const float* hi1, const float* lo2, const float* hi2,
                                          unsigned short* plist, int* pcount, bool all_rot) {
    __syncthreads();  // every lane has read the previous count and list
    if (threadIdx.x == 0) *pcount = 0;
    __syncthreads();
#pragma unroll 1
    for (int q0 = 0; q0 < CH / NT; q0 += kCullInFlightF) {
        float R[kCullInFlightF][9];
#pragma unroll
        for (int q = 0; q < kCullInFlightF; ++q) {
            const int p = min(pbase + int(threadIdx.x) + (q0 + q) * NT, pend - 1);
            load_rot(rotb + int64_t(p) * 9, R[q]);
        }
#pragma unroll
        for (int q = 0; q < kCullInFlightF; ++q) {
            const int p = pbase + int(threadIdx.x) + (q0 + q) * NT;
            if (p >= pend) continue;
            const bool h1 = pose_hits<GEN>(R[q], lo1, hi1, all_rot),
                       h2 = TWO && pose_hits<GEN>(R[q], lo2, hi2, all_rot);
            if (h1 || h2) plist[atomicAdd(pcount, 1)] = (unsigned short)((p - pbase) | (h1 ? kHit1 : 0) | (h2 ? kHit2 : 0));
        }
    }
    __syncthreads();
    const int np = *pcount;
    return np;
}

// Forward culling of the other tiled poses (GEN) in two stages: a plane test of one pose per lane,
// whose hits gather in the wave's row of `gst` (128 entries), and the class, dual-basis and
// half-plane tests on 64 gathered hits at a time, so only the poses whose plane crosses the box
// pay for the Gram matrix.  List entries as cull_chunk's (box 1 only).
template <int NT, int CH>
__device__ __forceinline__ int cull_chunk_gen(const float* __restrict__ rotb, int pend, int pbase, const float* lo,
                                              const float* hi, unsigned short* plist, int* pcount,
                                              unsigned short* gst) {
    const int lane = threadIdx.x & 63;
    __syncthreads();  // every lane has read the previous count and list
    if (threadIdx.x == 0) *pcount = 0;
    __syncthreads();
    auto classify = [&](int nh) {  // lanes < nh test gathered hit `lane`
        if (lane < nh) {
            const int p = pbase + int(gst[lane]);
            float R[9], as[3];
            load_rot(rotb + int64_t(p) * 9, R);
            if (pose_of_class<true>(R, as, false) && half_plane_hits(as, hi, lo))
                plist[atomicAdd(pcount, 1)] = (unsigned short)((p - pbase) | kHit1);
        }
    };
    int nh = 0;  // gathered hits of this wave
#pragma unroll 1
    for (int q0 = 0; q0 < CH / NT; ++q0) {
        const int p = pbase + int(threadIdx.x) + q0 * NT;
        bool hit = false;
        if (p < pend) {
            float R[9];
            load_rot(rotb + int64_t(p) * 9, R);
            hit = plane_hits(R, lo, hi);
        }
        const uint64_t m = __ballot(hit);
        const int rank = int(__builtin_amdgcn_mbcnt_hi(unsigned(m >> 32), __builtin_amdgcn_mbcnt_lo(unsigned(m), 0u)));
        if (hit) gst[nh + rank] = (unsigned short)(p - pbase);
        nh += __popcll(m);
        __builtin_amdgcn_wave_barrier();
        if (nh >= 64) {
            classify(64);
            __builtin_amdgcn_wave_barrier();
            const unsigned short rest = lane + 64 < nh ? gst[lane + 64] : 0;
            __builtin_amdgcn_wave_barrier();
            if (lane + 64 < nh) gst[lane] = rest;
            nh -= 64;
            __builtin_amdgcn_wave_barrier();
        }
    }
    classify(nh);
    __syncthreads();
    return *pcount;
}

// Scatter culling: candidates [pbase, pend) (at most kChunkSc; poses, or
// positions in the bin list lst as for cull_chunk) against box 1 and box 2
// separately.  Box-1 survivors fill plist from the front, box-2 survivors from
// the back (kChunk entries hold both lists), so each pass batches only poses
// that cross its box.
constexpr int kChunkSc = kChunk / 2;
template <int NT, bool GEN>
__device__ __forceinline__ void cull_chunk_boxes(const float* __restrict__ rotb, int pend, int pbase,
                                                 const float* lo1, const float* hi1, const float* lo2,
                                                 const float* hi2, unsigned short* plist, int* pcnt, int& n1,
                                                 int& n2, bool all_rot, const unsigned short* __restrict__ lst) {
    static_assert(kChunkSc % NT == 0 && (kChunkSc / NT) % kCullInFlight == 0, "cull shape");
    __syncthreads();  // every lane has read the previous counts and lists
    if (threadIdx.x == 0) pcnt[0] = pcnt[1] = 0;
    __syncthreads();
#pragma unroll 1
    for (int q0 = 0; q0 < kChunkSc / NT; q0 += kCullInFlight) {
        float R[kCullInFlight][9];
        int pq[kCullInFlight];
#pragma unroll
        for (int q = 0; q < kCullInFlight; ++q) {
            const int k = min(pbase + int(threadIdx.x) + (q0 + q) * NT, pend - 1);
            pq[q] = lst ? int(lst[k]) : k;
            load_rot(rotb + int64_t(pq[q]) * 9, R[q]);
        }
#pragma unroll
        for (int q = 0; q < kCullInFlight; ++q) {
            const int k = pbase + int(threadIdx.x) + (q0 + q) * NT;
            // box 2 is box 1 negated (bit for bit), which a plane through the origin
            // crosses exactly when it crosses box 1: one plane test serves both
            float as[3];
            if (k >= pend || !pose_of_class<GEN>(R[q], as, all_rot) || !plane_hits(R[q], lo1, hi1)) continue;
            const unsigned short e = lst ? (unsigned short)pq[q] : (unsigned short)(k - pbase);
            if (half_plane_hits(as, hi1, lo1)) plist[atomicAdd(&pcnt[0], 1)] = e;
            if (half_plane_hits(as, hi2, lo2)) plist[kChunk - 1 - atomicAdd(&pcnt[1], 1)] = e;
        }
    }
    __syncthreads();
    n1 = pcnt[0];
    n2 = pcnt[1];
}

// Pose bin of scatter tile (kc, kr, kd) in the grid with bins bg (tiles outside the core): its list
// and count for rotation batch item rb, or lst = nullptr when there are no bins.
__device__ __forceinline__ void tile_bin(const BinGrid& bg, int64_t rb, int64_t P, int kc, int kr, int kd,
                                         const unsigned short*& lst, int& cnt) {
    lst = nullptr;
    cnt = 0;
    if (!bg.list) return;
    const int64_t bi = rb * bg.n + (int64_t(kd >> 1) * bg.nb[1] + (kr >> 1)) * bg.nb[0] + (kc >> 1);
    lst = bg.list + bi * P;
    cnt = bg.count[bi];
}

// ----------------------------------------------------------------------------- forward
// (The forward culls all its poses per tile: its single 2048-pose cull phase measured no faster
// from pose bins, which cost a pre-pass.)
// GMODE 0: forward projection into `out`.
// GMODE 1: rotation and shift gradients of project_3d_to_2d_back for rotation
//          poses (KP = 1): each owned sample's value and spatial gradient
//          from the staged tile, paired with grad_projections `gsrc` as in
//          cpu/3d/projection_3d_to_2d_kernels.cpp:344-379; a wave sums its
//          pose's terms and adds them to grot / gshift (either may be null).
// GMODE 2: backproject_2d_to_3d_back for rotation poses (KP = 1): `rec` is
//          grad_data_rec; grad_projections (`out`) gathered with the value in
//          the reference's order, grad_weights (`wout`, WG) trilinearly from a
//          second staged tile of grad_weight_rec `gw` with the weight-tap rules,
//          and with RS the rotation/shift gradients against the projections
//          `gsrc` (cpu/3d/backprojection_2d_to_3d_kernels.cpp:451-567).
constexpr double kTwoPi = 6.283185307179586476925286766559;

// Tricubic value and spatial gradient for the gradient sums (which carry the
// 1e-4 bar, not bit-identity): the 64 taps are reduced along c first (value
// and d/dc weights), then r, then d, instead of forming the four triple
// products per tap, with fused multiply-adds and the fp32 weight polynomials.
// EXACT_V also forms the value in the reference's order
// (((s * wd) * wr) * wc summed over d, r, c, with its weights) for outputs
// that are gathers.  Weights and taps as cubic3 (interpolation_kernels.h:345-425).
template <bool EXACT_V, typename F>
__device__ __forceinline__ Interp<float> cubic3_grads(F&& fetch, float d, float r, float c) {
    float dx, rx, cx;
    const int df = split_as<false>(d, dx), rf = split_as<false>(r, rx), cf = split_as<false>(c, cx);
    auto w_of = [](float f, int j) { return EXACT_V ? cubic_w_tap<float>(f, j) : cubic_w_fast(f - float(j - 1)); };
    float wc[4], dwc[4], wr[4], dwr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        wc[j] = w_of(cx, j);
        dwc[j] = cubic_dw_fast(cx - float(j - 1));
        wr[j] = w_of(rx, j);
        dwr[j] = cubic_dw_fast(rx - float(j - 1));
    }
    Interp<float> o;
    o.v = o.g[0] = o.g[1] = o.g[2] = {0.f, 0.f};
    Cx<float> ve = {0.f, 0.f};  // EXACT_V: the value in the reference's order
#pragma unroll 1
    for (int k = 0; k < 4; ++k) {
        const float wd = w_of(dx, k), dwd = cubic_dw_fast(dx - float(k - 1));
        Cx<float> pv = {0.f, 0.f}, pc = {0.f, 0.f}, pr = {0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            Cx<float> a = {0.f, 0.f}, bc = {0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const Cx<float> t = fetch(df + k - 1, rf + i - 1, cf + j - 1);
                if (EXACT_V) ve = cadd(ve, cscale(cscale(cscale(t, wd), wr[i]), wc[j]));
                a = cfma(t, wc[j], a);
                bc = cfma(t, dwc[j], bc);
            }
            pv = cfma(a, wr[i], pv);
            pc = cfma(bc, wr[i], pc);
            pr = cfma(a, dwr[i], pr);
        }
        o.v = cfma(pv, wd, o.v);
        o.g[0] = cfma(pc, wd, o.g[0]);
        o.g[1] = cfma(pr, wd, o.g[1]);
        o.g[2] = cfma(pv, dwd, o.g[2]);
    }
    if (EXACT_V) o.v = ve;
    return o;
}

// One sample's terms of the pose gradients: with s = (c, r) * os the rotation term of row k is
// Re(a conj(dF/dx_k * s)) = s Re(a conj(dF/dx_k)), and with k = -2 pi (r, c) / n the shift terms are
// Re(b conj(i k m)) = k (b.im m.re - b.re m.im).  The sums acc[.][3 row + {0, 1}] take (c, r) and
// acc[.][9], acc[.][10] take (r, c); the pose's totals are scaled by os and -2 pi / n once.  With KS
// poses per wave batch a lane keeps one set of sums per pose slot; the sample's terms go to its
// slot's set, the others take 0 (selected, so a non-finite term stays with its own pose).
template <int KS>
__device__ __forceinline__ void grad_terms(const Interp<float>& ip, Cx<float> a, Cx<float> b, Cx<float> m, float fr,
                                           float fc, bool rot, bool shift, int sl, float (*acc)[11]) {
    if (rot) {
#pragma unroll
        for (int row = 0; row < 3; ++row) {
            const float d = fmaf(a.re, ip.g[row].re, a.im * ip.g[row].im);
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const float ds = (KS == 1 || sl == k) ? d : 0.f;
                acc[k][row * 3 + 0] = fmaf(ds, fc, acc[k][row * 3 + 0]);
                acc[k][row * 3 + 1] = fmaf(ds, fr, acc[k][row * 3 + 1]);
            }
        }
    }
    if (shift) {
        const float cr = fmaf(b.im, m.re, -(b.re * m.im));
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const float cs = (KS == 1 || sl == k) ? cr : 0.f;
            acc[k][9] = fmaf(cs, fr, acc[k][9]);
            acc[k][10] = fmaf(cs, fc, acc[k][10]);
        }
    }
}

// Waves per SIMD the forward is compiled for: the linear forward of a complex-half volume fits five
// workgroups per CU in LDS, which its registers must allow too (96 VGPRs, for rotation poses; the
// other poses' instantiation would spill there); the others (1: no target) are limited to four
// workgroups or fewer by LDS or registers anyway.
template <bool CUBIC, int GMODE, typename VS, bool GEN>
constexpr int forw_waves_per_eu() {
    return (!CUBIC && GMODE == 0 && kHalfVolume<VS> && !GEN) ? 5 : 1;
}
template <bool CUBIC, int KP, bool OSX, int GMODE = 0, bool RS = true, bool WG = false, typename VS = float,
          bool GEN = false>
__global__ __launch_bounds__(kForwThreads)
__attribute__((amdgpu_waves_per_eu(forw_waves_per_eu<CUBIC, GMODE, VS, GEN>()))) void k_forw3_tiled(Geom g, TileSpec ts, const Cx<VS>* __restrict__ rec,
                                                        const float* __restrict__ rot,
                                                        const float* __restrict__ shifts,
                                                        Cx<float>* __restrict__ out, CallPoses* __restrict__ cp,
                                                        int gl, const Cx<float>* __restrict__ gsrc = nullptr,
                                                        float* __restrict__ grot = nullptr,
                                                        float* __restrict__ gshift = nullptr,
                                                        const float* __restrict__ gw = nullptr,
                                                        float* __restrict__ wout = nullptr) {
    static_assert(!(GMODE == 1 || (GMODE == 2 && RS)) || KP <= 2,
                  "the gradient modes keep a set of sums per pose of a wave batch");
    static_assert(GMODE != 2 || std::is_same<VS, float>::value, "complex-half volumes: forward and its gradients only");
    constexpr bool GRADS = GMODE == 1 || (GMODE == 2 && RS);
    constexpr int WW = (GMODE == 2 && WG) ? (L + 1) * (L + 1) * (LD + 1) : 1;  // trilinear weight taps
    __shared__ float wt[WW];
    constexpr int LO = CUBIC ? 1 : 0, HI = CUBIC ? 2 : 1, W = L + LO + HI, WD = LD + LO + HI, W3 = W * W * WD;
    // GMODE 0 spreads the rows of a batch's KP poses over the wave's lanes in blocks of 64 (FLAT);
    // the gradient modes keep a set of sums per pose slot and give each pose RPS = 64 / KP lanes
    constexpr bool FLAT = GMODE == 0;
    static_assert(KP >= 1 && KP <= 8, "poses per wave batch (three bits of a queue entry)");
    constexpr int RPS = FLAT ? 64 : 64 / KP;
    constexpr int NT = kForwThreads, NW = NT / 64;
    constexpr int LOADS = (W3 + NT - 1) / NT;
    // the staged tile keeps the volume's storage type: a complex-half volume takes half the LDS
    // (more workgroups per CU) and is widened on each tap read, to the same fp32 values
    __shared__ Cx<VS> vt[W3];
    constexpr int CH = 2 * kChunk;  // poses culled per phase
    static_assert(CH <= int(kPoseMask) + 1, "pose index must fit below the flag bits");
    __shared__ unsigned short plist[CH];
    __shared__ int pcount;
    // sample queue entries per wave (the backprojection backward's second staged tile takes LDS,
    // and a workgroup above 53760 bytes leaves two per CU: LDS is allocated in 1280-byte granules)
    constexpr int QCAP = (GMODE == 2 && WG) ? 192 : 256;
    // CARRY (cubic forward): a wave's last, partly filled window of samples waits for its next
    // batch's samples (a cubic sample's 64 taps make each window costly; 3 % faster), with two
    // pose sets per wave.  The linear forward measured 1 % slower with it: most of its waves take
    // only one or two batches of a tile, and a wave's last batch deposits its window anyway.
    // The sample queues are idle while a phase's poses are culled, so the GEN cull gathers its
    // plane hits (128 per wave) in their memory.
    constexpr bool CARRY = FLAT && CUBIC;
    __shared__ Slot slots[NW][CARRY ? 2 * KP : KP];
    __shared__ union {
        unsigned q[NW][QCAP];
        unsigned short gst[NW][2 * QCAP];
    } qmem;
    auto& queue = qmem.q;
    static_assert(2 * QCAP >= 128, "GEN culling gathers up to 128 plane hits per wave");
    __shared__ unsigned char marks[FLAT ? NW : 1][64];  // FLAT: pose lookup of the batch's rows
    __shared__ int gen_sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // FLAT: lane k < KP holds pose k of the batch; otherwise lane = slot * RPS + row
    const int slot = FLAT ? (lane < KP ? lane : 0) : lane / RPS, jrow = FLAT ? 0 : lane % RPS;
    const bool pose_lane = FLAT ? lane < KP : true;
    // samples lie within |x| <= rho_k: rotations reach rho_unit + 1 (and have nothing to do when
    // the call has none); GEN poses the call's own reach, up to kScaleMax times farther, over
    // the part of the wide grid that this reach needs
    const int any_rot = GEN ? 1 : call_flag(&cp->any_rot);
    const bool all_rot = !GEN && call_flag(&cp->all_rot);
    float rho_k = ts.rho_unit + 1.0f;
    int nt = ts.nt, ntd = ts.ntfd, org = ts.org, orgd = ts.orgd;
    int fc0 = ts.fc0, fc1 = ts.fc1, fd0 = ts.fd0, fd1 = ts.fd1;
    if constexpr (GEN) {
        rho_k = fminf(ts.rho, cp->gen_reach);
        if (!(rho_k > 0.f)) return;  // no such pose in this call
        const int h = half_tiles_for(rho_k, L, ts.nt2 / 2), hd = half_tiles_for(rho_k, LD, ts.ntfd2 / 2);
        const int off = ts.nt2 / 2 - h, offd = ts.ntfd2 / 2 - hd;
        nt = 2 * h;
        ntd = 2 * hd;
        org = ts.org2 + off * L;
        orgd = ts.orgd2 + offd * LD;
        fc0 = min(nt, max(0, ts.fc0_2 - off));
        fc1 = min(nt, max(fc0, ts.fc1_2 - off));
        fd0 = min(ntd, max(0, ts.fd0_2 - offd));
        fd1 = min(ntd, max(fd0, ts.fd1_2 - offd));
    }
    const float rho2 = rho_k * rho_k;
    // core tiles in pose ranges: the rotation kernels' split, or the other poses' (the scatter's)
    const int ksplit = GEN ? ts.ksplit : ts.fksplit, prange = GEN ? ts.prange : ts.fprange;
    int64_t items = g.B * (int64_t(fc1 - fc0) * (fc1 - fc0) * (fd1 - fd0) * ksplit + int64_t(nt) * nt * ntd);
    // rotations: the slots may index the list of the work items in reach (the others' workgroups
    // would only start and leave)
    const int* __restrict__ flist = GEN ? nullptr : ts.flist;
    if (flist) items = ts.fcount;
    const float cut2 = float(g.cut2);
    const int N = g.N, H = g.H;
    // (GEN: the grid holds a quarter of the rotation kernel's slots and steps over the rest)
    for (Slots<false> sl(xcd_per<kRunForw>(items), nullptr, &gen_sh); sl.ok(); sl.next(&gen_sh)) {
        if (!any_rot) return;  // rotation kernel, no rotation in the call (its flags were read above)
        const int64_t slot_i = sl.s;
        const int64_t wi = xcd_item<kRunForw>(slot_i);
        if (wi >= items) continue;
        const int64_t w = flist ? int64_t(flist[wi]) : wi;
        const Item it = item_of(w, g.B, int(g.P), ntd, nt, nt, fd0, fd1, fc0, fc1, fc0, fc1, ksplit, prange);
        if (it.skip) continue;
        const int64_t b = it.b;
        const int tc = org + it.kc * L, tr = org + it.kr * L, td = orgd + it.kd * LD;
        const int p0 = it.p0, p1 = it.p1;
        // samples owned by this tile: floor(x) in [t, t + edge) on every axis (+ slack)
        const float lo[3] = {float(tc) - ts.eps, float(tr) - ts.eps, float(td) - ts.eps};
        const float hi[3] = {float(tc + L) + ts.eps, float(tr + L) + ts.eps, float(td + LD) + ts.eps};
        float dist2 = 0.f;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const float q = lo[k] > 0.f ? lo[k] : (hi[k] < 0.f ? -hi[k] : 0.f);
            dist2 += q * q;
        }
        if (dist2 > rho2) continue;
        const int64_t rb = g.B_rot == 1 ? 0 : b, sb = g.B_shift == 1 ? 0 : b;
        const float* rotb = rot + rb * g.P * 9;
        const Cx<VS>* recb = rec + b * g.vol;
        bool loaded = false;
        for (int pbase = p0; pbase < p1; pbase += CH) {
            const int np = GEN ? cull_chunk_gen<NT, CH>(rotb, p1, pbase, lo, hi, plist, &pcount, qmem.gst[wave])
                               : cull_chunk<NT, false, CH, GEN>(rotb, p1, pbase, lo, hi, lo, hi, plist, &pcount, all_rot);
            if (np == 0) continue;
            auto pose_of = [&](unsigned e) { return pbase + int(e & kPoseMask); };
            if (!loaded) {
                // stage the tile and its halo.  When the staged box lies on one side of c = 0 and
                // needs no clamping, a cell is a plain wrapped load (conjugated from the mirrored
                // cell on the c < 0 side); other boxes go through the reference's sampler rules.
                const int c_lo = tc - LO, c_hi = tc - LO + W - 1, r_lo = tr - LO, r_hi = tr - LO + W - 1,
                          d_lo = td - LO, d_hi = td - LO + WD - 1, hn = N / 2;
                const bool plain_pos = c_lo >= 0 && c_hi <= H - 1 && r_lo >= -hn + 1 && r_hi <= hn &&
                                       d_lo >= -hn + 1 && d_hi <= hn;
                const bool plain_neg = c_hi < 0 && -c_lo <= H - 1 && r_lo >= -hn + 1 && r_hi <= hn - 1 &&
                                       d_lo >= -hn + 1 && d_hi <= hn - 1;
                const bool plain = plain_pos || plain_neg;
                const int sg = plain_neg ? -1 : 1;
                constexpr int STAGE = 8;
#pragma unroll 1
                for (int q0 = 0; q0 < LOADS; q0 += STAGE) {
                    Cx<float> v[STAGE];
#pragma unroll
                    for (int q = 0; q < STAGE; ++q) {
                        const int cell = min(tid + (q0 + q) * NT, W3 - 1);
                        const int lc = cell % W, lr = (cell / W) % W, ld = cell / (W * W);
                        const int d = td - LO + ld, r = tr - LO + lr, c = tc - LO + lc;
                        if (plain) {
                            const int dd = sg * d, rr = sg * r;
                            const int64_t idx = (int64_t(dd < 0 ? dd + N : dd) * N + (rr < 0 ? rr + N : rr)) * H + sg * c;
                            if constexpr (kHalfVolume<VS>) v[q] = load_widened(recb, idx);
                            else v[q] = recb[idx];
                            if (plain_neg) v[q].im = -v[q].im;
                        } else {
                            v[q] = CUBIC ? fetch3_cubic(recb, N, H, d, r, c) : fetch3(recb, N, H, d, r, c);
                        }
                    }
#pragma unroll
                    for (int q = 0; q < STAGE; ++q)
                        if (tid + (q0 + q) * NT < W3) {
                            // a widened half value (or its negation) narrows back exactly
                            if constexpr (kHalfVolume<VS>)
                                vt[tid + (q0 + q) * NT] = Cx<__half>{__float2half(v[q].re), __float2half(v[q].im)};
                            else
                                vt[tid + (q0 + q) * NT] = v[q];
                        }
                }
                if constexpr (GMODE == 2 && WG) {
                    const float* gwb = gw + b * g.vol;
                    for (int e = tid; e < WW; e += NT) {
                        const int lc = e % (L + 1), lr = (e / (L + 1)) % (L + 1), ld = e / ((L + 1) * (L + 1));
                        wt[e] = weight_tap<3>(gwb, N, H, td + ld, tr + lr, tc + lc);
                    }
                }
                __syncthreads();
                loaded = true;
            }
            // wave batches of KP poses; the next batch's rotation and shift load during this one
            int base = wave * KP;
            float Rn[9], Sn[2];
            load_pose(rotb, shifts ? shifts + sb * g.P * 2 : nullptr, pose_of(plist[min(base + slot, np - 1)]), Rn, Sn);
            // CARRY: the wave's queue starts with the mq samples of a partly filled window, the first
            // mprev of them the previous batch's; batch j takes slot set (j mod 2) * KP (buf)
            int mq = 0, mprev = 0, buf = 0;
            for (; base < np; base += NW * KP, buf ^= CARRY ? KP : 0) {
                const bool last = base + NW * KP >= np;
                mprev = mq;
                const bool sv = pose_lane && base + slot < np;
                const int pp = pose_of(plist[min(base + slot, np - 1)]);
                float R[9], Sh[2];
#pragma unroll
                for (int e = 0; e < 9; ++e) R[e] = Rn[e];
                Sh[0] = Sn[0];
                Sh[1] = Sn[1];
                if (base + NW * KP < np)
                    load_pose(rotb, shifts ? shifts + sb * g.P * 2 : nullptr,
                              pose_of(plist[min(base + NW * KP + slot, np - 1)]), Rn, Sn);
                constexpr int KS = GRADS ? KP : 1;
                float acc[KS][11];  // gradient modes: this lane's share of each slot's 9 rotation and 2 shift sums
#pragma unroll
                for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
                    for (int k = 0; k < 11; ++k) acc[s2][k] = 0.f;
                int r0 = 0, r1 = -1;
                if (sv || !FLAT) box_rows<GEN>(R, lo, hi, ts, r0, r1);
                const int nr = sv ? max(0, r1 - r0 + 1) : 0;
                // FLAT: the batch's rows (each pose's in turn) and each pose's first one among them
                const int rincl = FLAT ? dpp_scan_add(nr) : 0;
                const int start = rincl - nr;
                const int rows = FLAT ? __builtin_amdgcn_readlane(rincl, 63) : 0;
                if (jrow == 0 && sv) {
                    Slot& sd = slots[wave][buf + slot];
                    sd.R6[0] = R[0];
                    sd.R6[1] = R[1];
                    sd.R6[2] = R[3];
                    sd.R6[3] = R[4];
                    sd.R6[4] = R[6];
                    sd.R6[5] = R[7];
                    sd.s0 = Sh[0];
                    sd.s1 = Sh[1];
                    sd.base = (b * g.P + pp) * int64_t(g.npix);
                    sd.r0 = r0;
                    sd.start = start;
                }
                __builtin_amdgcn_wave_barrier();
                int pcarry = 0;
                // row blocks: FLAT, 64 rows of the batch at a time; otherwise RPS rows per pose while
                // some pose has rows left
                // (CARRY: a batch without rows still runs one empty block when a window is carried, to
                // deposit it: its samples' slot set is the next batch's)
                for (int rbase = 0; FLAT ? rbase < rows || (CARRY && rbase == 0 && mq > 0) : __ballot(nr > rbase) != 0;
                     rbase += RPS) {
                    int r, c0 = 0, cnt = 0, sk = slot;
                    if constexpr (FLAT) {
                        // row rbase + lane of the batch: its pose (the pose lane whose rows hold it)
                        sk = max(0, window_owner(nr, start, rbase, pcarry, marks[wave]));
                        const int f = rbase + lane;
                        r = 0;
                        if (f < rows) {
                            const Slot& sd = slots[wave][buf + sk];
                            float R6[6];
#pragma unroll
                            for (int e = 0; e < 6; ++e) R6[e] = sd.R6[e];
                            r = sd.r0 + (f - sd.start);
                            int c1;
                            row_span6(R6, r, lo, hi, ts, cut2, c0, c1);
                            cnt = max(0, c1 - c0 + 1);
                        }
                    } else {
                        const int jr = rbase + jrow;
                        r = r0 + jr;
                        if (jr < nr) {
                            int c1;
                            row_span(R, r, lo, hi, ts, cut2, c0, c1);
                            cnt = max(0, c1 - c0 + 1);
                        }
                    }
                    const int incl = dpp_scan_add(cnt);
                    const int excl = incl - cnt;
                    const int total = __builtin_amdgcn_readlane(incl, 63);
                    // queue entry qi: the sample, whose pose is slot `sl` of slot set `sset`
                    auto sample = [&](int qi, int sset) {
                        int rr, cc, sl;
                        q_unpack(queue[wave][qi], rr, cc, sl);
                        // every field of the sample's pose slot is read before the tests, so that the
                        // reads go out together (one LDS round trip) instead of one per test
                        const Slot& sdl = slots[wave][sset + sl];
                        Slot sd;
#pragma unroll
                        for (int e = 0; e < 6; ++e) sd.R6[e] = sdl.R6[e];
                        sd.s0 = sdl.s0;
                        sd.s1 = sdl.s1;
                        sd.base = sdl.base;
                        const float fr = float(rr), fc = float(cc);
                        float x[3];
                        rotate_slice6<OSX>(sd.R6, fr, fc, g.os, x);
                        const int fxc = int(floorf(x[0])), fxr = int(floorf(x[1])), fxd = int(floorf(x[2]));
                        // outside the cutoff, the Friedel half of the x = 0 line (the backward ops skip
                        // it), or not owned by this tile
                        bool skip = filtered(fr, fc, cut2);
                        if (GMODE != 0) skip |= (cc == 0) & ((rr == g.n / 2) | (rr < 0));
                        skip |= (fxc < tc) | (fxc >= tc + L) | (fxr < tr) | (fxr >= tr + L) | (fxd < td) | (fxd >= td + LD);
                        asm volatile("" ::"v"(sd.s0), "v"(sd.s1), "v"(int(sd.base)), "v"(int(sd.base >> 32)));
                        if (skip) return;
                        // staged cell of the tap at floor(x); the interpolation reads its taps at
                        // constant offsets from it (the interpolators split x the same way)
                        const unsigned eb = __umul24(__umul24(unsigned(fxd - (td - LO)), unsigned(W)) + unsigned(fxr - (tr - LO)),
                                                     unsigned(W)) + unsigned(fxc - (tc - LO));
                        auto lds = [&](int d, int r, int c) {
                            const unsigned e = eb + unsigned(((d - fxd) * W + (r - fxr)) * W + (c - fxc));
                            if constexpr (kHalfVolume<VS>) return Cx<float>{__half2float(vt[e].re), __half2float(vt[e].im)};
                            else return vt[e];
                        };
                        // pixel offset in the pose's projection (i, hp < 2^24)
                        const int pix = int(__umul24(unsigned(rr >= 0 ? rr : rr + g.n), unsigned(g.hp))) + cc;
                        if constexpr (GMODE == 0) {
                            Cx<float> v = CUBIC ? cubic3<float, false, false>(lds, x[2], x[1], x[0]).v
                                                : lerp3<float, false, false>(lds, x[2], x[1], x[0]).v;
                            if (shifts) v = cmul(v, phase_hw(fr, fc, sd.s0, sd.s1, g.phase_k));
                            out[sd.base + pix] = v;
                        } else if constexpr (GMODE == 2) {
                            Interp<float> ip;
                            if constexpr (CUBIC && GRADS) ip = cubic3_grads<true>(lds, x[2], x[1], x[0]);
                            else if constexpr (CUBIC) ip = cubic3<float, false, false>(lds, x[2], x[1], x[0]);
                            else ip = lerp3<float, GRADS, false>(lds, x[2], x[1], x[0]);
                            const int64_t pidx = sd.base + pix;
                            const Cx<float> ph = shifts ? phase_hw(fr, fc, sd.s0, sd.s1, g.phase_k)
                                                        : Cx<float>{1.f, 0.f};
                            out[pidx] = shifts ? cmul(ip.v, ph) : ip.v;
                            if constexpr (WG) {
                                // trilinear as weight_grad_interp<3>
                                float cx, rx, dx;
                                const int cf = split_as<false>(x[0], cx), rf = split_as<false>(x[1], rx),
                                          df = split_as<false>(x[2], dx);
                                auto wa = [&](int d, int r, int c) {
                                    return wt[((d - td) * (L + 1) + (r - tr)) * (L + 1) + (c - tc)];
                                };
                                const float p000 = wa(df, rf, cf), p001 = wa(df, rf, cf + 1);
                                const float p010 = wa(df, rf + 1, cf), p011 = wa(df, rf + 1, cf + 1);
                                const float p100 = wa(df + 1, rf, cf), p101 = wa(df + 1, rf, cf + 1);
                                const float p110 = wa(df + 1, rf + 1, cf), p111 = wa(df + 1, rf + 1, cf + 1);
                                const float p00 = p000 + (p001 - p000) * cx;
                                const float p01 = p010 + (p011 - p010) * cx;
                                const float p10 = p100 + (p101 - p100) * cx;
                                const float p11 = p110 + (p111 - p110) * cx;
                                const float p0 = p00 + (p01 - p00) * rx;
                                const float p1 = p10 + (p11 - p10) * rx;
                                wout[pidx] = p0 + (p1 - p0) * dx;
                            }
                            if constexpr (GRADS) {
                                // proj * conj(phase) against dF/dx * s and against -i 2 pi k / n * F
                                // (grad_terms: the sums take (c, r), the pose's totals the constants)
                                Cx<float> pv = gsrc[pidx];
                                if (shifts) pv = cmul(pv, cconj(ph));
                                grad_terms<KS>(ip, pv, pv, ip.v, fr, fc, grot != nullptr, gshift != nullptr, sl, acc);
                            }
                        } else {
                            const Interp<float> ip = CUBIC ? cubic3_grads<false>(lds, x[2], x[1], x[0])
                                                           : lerp3<float, true, false>(lds, x[2], x[1], x[0]);
                            const Cx<float> g0 = gsrc[sd.base + pix];
                            const Cx<float> ph = shifts ? phase_hw(fr, fc, sd.s0, sd.s1, g.phase_k)
                                                        : Cx<float>{1.f, 0.f};
                            // g' = g * phase(-r, -c) = g * conj(phase(r, c)) against dF/dx * s, s = (sc, sr, 0);
                            // g against -i 2 pi k / n * (F * phase)
                            const Cx<float> gg = shifts ? cmul(g0, cconj(ph)) : g0;
                            const Cx<float> mod = shifts ? cmul(ip.v, ph) : ip.v;
                            grad_terms<KS>(ip, gg, g0, mod, fr, fc, grot != nullptr, gshift != nullptr, sl, acc);
                        }
                    };
                    if constexpr (CARRY) {
                        // the batch's last block deposits a partial window if the phase ends here, or if
                        // the window would still hold samples of the previous batch (whose slot set the
                        // next batch takes)
                        const bool flush = rbase + RPS >= rows && (last || (mprev > 0 && mq + total < 64));
                        for (int q0 = 0;;) {
                            // entries [q0, q0 + room) of this block follow the mq carried ones
                            const int room = QCAP - mq;
                            q_fill_at(queue[wave], mq, r, c0, cnt, excl, sk, q0, room);
                            const int n = min(room, total - q0), avail = mq + n;
                            const bool done = q0 + n >= total;
                            const int wend = done && flush ? avail : (avail & ~63);
                            for (int e0 = 0; e0 < wend; e0 += 64)
                                if (e0 + lane < wend) sample(e0 + lane, e0 == 0 && lane < mprev ? buf ^ KP : buf);
                            if (wend > 0) mprev = 0;
                            // a partial window waits at the queue's front
                            const int left = avail - wend;
                            if (wend > 0 && left > 0) {
                                const unsigned e = lane < left ? queue[wave][wend + lane] : 0u;
                                __builtin_amdgcn_wave_barrier();
                                if (lane < left) queue[wave][lane] = e;
                                __builtin_amdgcn_wave_barrier();
                            }
                            mq = left;
                            q0 += n;
                            if (done) break;
                        }
                    } else {
                        for (int q0 = 0; q0 < total; q0 += QCAP) {
                            q_fill<QCAP>(queue[wave], r, c0, cnt, excl, sk, q0);
                            const int m = min(QCAP, total - q0);
                            for (int e0 = 0; e0 < m; e0 += 64)
                                if (e0 + lane < m) sample(e0 + lane, 0);
                        }
                    }
                }
                if constexpr (GRADS) {
                    // each slot's sums (every lane of the wave takes part; the slot's first lane, which
                    // holds its pose, adds them)
#pragma unroll
                    for (int s2 = 0; s2 < KS; ++s2) {
                        const bool mine = lane == s2 * RPS && sv;
                        if (grot) {
                            const float os = float(g.os);
#pragma unroll
                            for (int row = 0; row < 3; ++row)
#pragma unroll
                                for (int k = 0; k < 2; ++k) {
                                    const float t = wave_sum(acc[s2][row * 3 + k]) * os;
                                    if (mine) atomic_add(&grot[(rb * g.P + pp) * 9 + row * 3 + k], t);
                                }
                        }
                        if (gshift) {
                            const float kn = float(-kTwoPi / double(g.n));
                            const float t0 = wave_sum(acc[s2][9]) * kn, t1 = wave_sum(acc[s2][10]) * kn;
                            if (mine) {
                                atomic_add(&gshift[(sb * g.P + pp) * 2], t0);
                                atomic_add(&gshift[(sb * g.P + pp) * 2 + 1], t1);
                            }
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            __syncthreads();
        }
        if (loaded) __syncthreads();
    }
}

// ----------------------------------------------------------------------------- scatter
// Per-sample work of the scatter: one class of the sample's stencil taps,
// spread over the tile's fp64 LDS accumulators.  flip = false takes the direct
// taps (c >= 0), flip = true the taps with c < 0, which the reference moves to
// (-c, -r, -d) and conjugates (projection_utils.h:414-443, 451-493); every
// (sample, tap) pair is thus deposited by exactly one pass.  Taps outside the
// reference's range [-N/2+1, N/2] are dropped there; here they fall outside
// the tile or on cells past the volume edge, which are never written out.
// LDS layout of the scatter accumulators: cell (lc, lr, ld) sits at
// (ld * SR + lr) * SC + ((lc + acc_swizzle(lr, ld)) mod SC).  Rotating each
// row by an amount that changes with lr / 2 and ld spreads the taps of
// samples stepping along r or d over different banks (an fp64 cell spans two
// of the 64 four-byte banks, so without it every cell of a column shares one).
static_assert((SC & (SC - 1)) == 0, "scatter tile width must be a power of two");
__device__ __forceinline__ int acc_swizzle(int lr, int ld) { return ((lr >> 1) + 3 * ld) & (SC - 1); }

// Per-pass constants: local cell of tap j on axis a is sgn * floor(x_a) + off[a] + sgn * j
// (sgn = -1 for the flipped taps), valid in [lmin[a], S_a).
struct TapMap {
    int sgn;
    int off[3];
    int lmin[3];
};

// A sample's row as (batch pose, row) in one word: row + bias in bits 0-15, pose in 16-31.
constexpr unsigned kRowBias = 0x8000u;
__device__ __forceinline__ unsigned kr_pack(int k, int r) { return ((unsigned(r) + kRowBias) & 0xffffu) | (unsigned(k) << 16); }

template <bool CUBIC, int MODE, bool WEIGHTS, bool OSX>
__device__ __forceinline__ void scatter_sample(const Geom& g, const Slot& sd, int rr, int cc, Cx<float> v,
                                               float wpix, bool shifted, bool flip, const TapMap& tm,
                                               double* acc_re, double* acc_im, double* acc_w) {
    constexpr int K = CUBIC ? 4 : 2;  // taps at floor(x) - (CUBIC ? 1 : 0) + j, j < K
    const float fr = float(rr), fc = float(cc);
    float x[3];
    rotate_slice6<OSX>(sd.R6, fr, fc, g.os, x);
    if (shifted) {
        if (MODE == 0) v = cmul(v, cconj(phase_hw(fr, fc, sd.s0, sd.s1, g.phase_k)));
        else v = cmul(v, phase_hw(-fr, -fc, sd.s0, sd.s1, g.phase_k));
    }
    // per axis: local cell of each tap position (or -1 outside the tile) and its weight
    constexpr int S[3] = {SC, SR, SD};
    int loc[3][K];
    double wt[3][K];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
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
    for (int k = 0; k < K; ++k) {
        if (loc[2][k] < 0) continue;
#pragma unroll
        for (int i = 0; i < K; ++i) {
            if (loc[1][i] < 0) continue;
            const double wdr = wt[2][k] * wt[1][i];
            const int row = (loc[2][k] * SR + loc[1][i]) * SC, rot = acc_swizzle(loc[1][i], loc[2][k]);
            // cubic: the value (and weight) times wd * wr once per (d, r) pair, one product per tap
            // after that; linear keeps one weight product per tap (two taps per pair)
            const double pre = CUBIC ? vre * wdr : vre, pim = CUBIC ? vim * wdr : vim,
                         pw = CUBIC ? wp * fabs(wdr) : wp;
#pragma unroll
            for (int j = 0; j < K; ++j) {
                if (loc[0][j] < 0) continue;
                const double w = CUBIC ? wt[0][j] : wdr * wt[0][j];
                const int li = row + ((loc[0][j] + rot) & (SC - 1));
                atomicAdd(&acc_re[li], pre * w);
                atomicAdd(&acc_im[li], pim * w);
                if (WEIGHTS) atomicAdd(&acc_w[li], pw * (CUBIC ? fabs(w) : w));
            }
        }
    }
}

// MODE 0: backprojection, v = proj * conj(phase(r, c)), optional weights.
// MODE 1: reconstruction gradient of the projection, v = g * phase(-r, -c).
template <bool CUBIC, int MODE, bool WEIGHTS, int KP, bool OSX, bool GEN>
__global__ __launch_bounds__(kScatterThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_scatter3_tiled(Geom g, TileSpec ts, const Cx<float>* __restrict__ src,
                                                           const float* __restrict__ weights,
                                                           const float* __restrict__ rot,
                                                           const float* __restrict__ shifts,
                                                           Cx<float>* __restrict__ dst, float* __restrict__ wdst,
                                                           CallPoses* __restrict__ cp, int gl) {
    constexpr int SL = CUBIC ? 2 : 1, SH = CUBIC ? 1 : 0;  // stencil reach below / above floor(x)
    constexpr int SLOW = CUBIC ? 1 : 0;                    // first tap at floor(x) - SLOW
    static_assert(KP >= 1 && KP <= 16, "poses per wave batch");
    constexpr int NT = kScatterThreads, NW = NT / 64;
    __shared__ double acc_re[S3], acc_im[S3];
    __shared__ double acc_w[WEIGHTS ? S3 : 1];
    __shared__ unsigned short plist[kChunk];
    __shared__ int pcnt[2];
    // CARRY (cubic): a row block's last, partial window of samples is not deposited at once but
    // filled up with the following samples, across batches.  At the cubic stencil's ~26 active
    // lanes per tap an LDS atomic instruction costs about as much as with more lanes, so fuller
    // windows take fewer instructions (3-4 % faster).  At the linear stencil's ~37 an
    // instruction's cost grows with its lanes and carried windows measured no faster, so the
    // linear kernels deposit every row block's windows in it.
    constexpr bool CARRY = CUBIC;
    static_assert(!CARRY || KP <= 4, "two pose sets per wave within four workgroups' LDS per CU");
    __shared__ Slot slots[NW][CARRY ? 2 * KP : KP];
    __shared__ unsigned char marks[NW][64];
    __shared__ int gen_sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool pose_lane = lane < KP;  // lane k holds pose k of the wave's batch
    const int N = g.N, H = g.H, half = N / 2;
    const int64_t items = g.B * (int64_t(ts.sd1 - ts.sd0) * (ts.sr1 - ts.sr0) * ts.sc1 * ts.ksplit +
                                 int64_t(ts.ntd) * ts.ntr * ts.ntc);
    const float cut2 = float(g.cut2);
    // samples lie within |x| <= rho_k: rotations reach rho_unit + 1, GEN poses the call's own
    // reach (up to kScaleMax times farther).  Without rotations in the call the rotation kernel
    // does nothing at all and GEN stores every tile it owns; with them GEN adds onto the tiles.
    const int any_rot = call_flag(&cp->any_rot);
    const bool all_rot = !GEN && call_flag(&cp->all_rot);
    float rho_k = ts.rho_unit + 1.0f;
    if constexpr (GEN) {
        rho_k = fminf(ts.rho, cp->gen_reach);
        if (!(rho_k > 0.f)) return;  // no such pose in this call
    }
    for (Slots<GEN> sl(xcd_per<kRunScatter>(items), slot_counters<GEN>(cp, gl), &gen_sh); sl.ok(); sl.next(&gen_sh)) {
        if (!GEN && !any_rot && call_reach(&cp->gen_reach) > 0.f) return;  // GEN stores every tile
        const int64_t slot_i = sl.s;
        const int64_t w = xcd_item<kRunScatter>(slot_i);
        if (w >= items) continue;
        const Item it = item_of(w, g.B, int(g.P), ts.ntd, ts.ntr, ts.ntc, ts.sd0, ts.sd1, ts.sr0, ts.sr1, 0, ts.sc1,
                                ts.ksplit, ts.prange);
        if (it.skip) continue;
        const int64_t b = it.b;
        // stored cells of this tile, signed coordinates: d, r in [-N/2+1, N/2], c in [0, N/2]
        const int tc = it.kc * SC, tr = -half + 1 + it.kr * SR, td = -half + 1 + it.kd * SD;
        // direct taps land here when x is in box 1 (the tile dilated by the stencil);
        // flipped (c < 0) taps when x is in box 2 (the same around the negated tile)
        const int fc0 = -tc - SC + 1, fr0 = -tr - SR + 1, fd0 = -td - SD + 1;
        const float lo1[3] = {float(tc - SL) - ts.eps, float(tr - SL) - ts.eps, float(td - SL) - ts.eps};
        const float hi1[3] = {float(tc + SC + SH) + ts.eps, float(tr + SR + SH) + ts.eps,
                              float(td + SD + SH) + ts.eps};
        const float lo2[3] = {float(fc0 - SL) - ts.eps, float(fr0 - SL) - ts.eps, float(fd0 - SL) - ts.eps};
        const float hi2[3] = {float(fc0 + SC + SH) + ts.eps, float(fr0 + SR + SH) + ts.eps,
                              float(fd0 + SD + SH) + ts.eps};
        static_assert(SL - SH == 1, "box 2 is box 1 negated when the stencil reaches one cell further below");
        const int64_t rb = g.B_rot == 1 ? 0 : b, sb = g.B_shift == 1 ? 0 : b;
        const float* rotb = rot + rb * g.P * 9;
        const int64_t pose0 = b * g.P;
        // samples lie within |x| <= rho_k; box 2 is box 1 mirrored, so one test serves both
        float dist2 = 0.f;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const float q = lo1[k] > 0.f ? lo1[k] : (hi1[k] < 0.f ? -hi1[k] : 0.f);
            dist2 += q * q;
        }
        // (a rotation kernel without rotations in the call only stores zeros)
        const int pend = (dist2 > rho_k * rho_k || (!GEN && !any_rot)) ? it.p0 : it.p1;
        // a tile that no pose can reach stores zeros without its accumulators (about half of the
        // tiles of a volume lie beyond the samples' sphere)
        const bool empty = pend == it.p0;
        if (!empty)
            for (int e = tid; e < S3; e += NT) {
                acc_re[e] = 0.0;
                acc_im[e] = 0.0;
                if (WEIGHTS) acc_w[e] = 0.0;
            }

        const float* shb = shifts ? shifts + sb * g.P * 2 : nullptr;
        bool touched = false;  // GEN: some pose reaches the tile
        // candidates: the tile's pose range, or (outside the core) its bin's poses
        const unsigned short* lst = nullptr;
        int lcnt = 0;
        if (!it.core && pend > it.p0) tile_bin(ts.sbins, rb, g.P, it.kc, it.kr, it.kd, lst, lcnt);
        const int c_begin = lst ? 0 : it.p0, c_end = lst ? lcnt : pend;
        for (int pbase = c_begin; pbase < c_end; pbase += kChunkSc) {
            int n1, n2;
            cull_chunk_boxes<NT, GEN>(rotb, c_end, pbase, lo1, hi1, lo2, hi2, plist, pcnt, n1, n2, all_rot, lst);
            touched |= n1 + n2 > 0;
#pragma unroll 1
            for (int pass = 0; pass < 2; ++pass) {
                const int np = pass == 0 ? n1 : n2;
                // pose of list entry k of this pass (box-2 entries are stored from the back)
                auto pose_at = [&](int k) {
                    const int e = int(plist[pass == 0 ? k : kChunk - 1 - k]);
                    return lst ? e : pbase + e;
                };
                float lo[3], hi[3];
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    lo[k] = pass == 0 ? lo1[k] : lo2[k];
                    hi[k] = pass == 0 ? hi1[k] : hi2[k];
                }
                // direct taps: l = floor(x) - LOW + j - t; flipped: l = -(floor(x) - LOW + j) - t,
                // and at c = 0 a flipped tap must have c < 0 (l >= 1 when t_c = 0)
                TapMap tm;
                tm.sgn = pass == 0 ? 1 : -1;
                tm.off[0] = pass == 0 ? -SLOW - tc : SLOW - tc;
                tm.off[1] = pass == 0 ? -SLOW - tr : SLOW - tr;
                tm.off[2] = pass == 0 ? -SLOW - td : SLOW - td;
                tm.lmin[0] = (pass == 1 && tc == 0) ? 1 : 0;
                tm.lmin[1] = tm.lmin[2] = 0;
                // wave batches of KP poses: lane k < KP holds pose k (the next batch's load in flight
                // during this one), and the batch's rows, all poses' in turn, are spread over the
                // wave's lanes in blocks of 64, so that a lane computes one row's column span
                int base = wave * KP;
                constexpr bool PREFETCH = !CARRY;  // (a carried window takes those registers)
                float Rn[9], Sn[2];
                if (PREFETCH && base < np)
                    load_pose(rotb, shb, pose_at(min(base + (pose_lane ? lane : 0), np - 1)), Rn, Sn);
                // the window being formed: lanes below m hold samples of earlier batches (their
                // row, column, pose slot, validity and loaded value), carried until 64 lanes are
                // filled.  Batch j writes its poses to slot set j mod 2; a window still holding
                // samples of batch j - 1 when batch j ends is deposited then, as is every window
                // at the end of the pass.
                int m = 0, buf = 0;
                unsigned krw = 0;  // the window sample's pose slot and row (kr_pack)
                int cc = 0;
                bool ok = false;
                Cx<float> v = {0.f, 0.f};
                float wv = 0.f;
                for (; base < np; base += NW * KP, buf ^= CARRY ? KP : 0) {
                    const bool last = base + NW * KP >= np;
                    bool prev = m > 0;  // the window holds samples of the previous batch
                    const bool sv = pose_lane && base + lane < np;
                    const int pp = pose_at(min(base + (pose_lane ? lane : 0), np - 1));
                    float R[9], Sh[2];
                    if constexpr (PREFETCH) {
#pragma unroll
                        for (int e = 0; e < 9; ++e) R[e] = Rn[e];
                        Sh[0] = Sn[0];
                        Sh[1] = Sn[1];
                        if (base + NW * KP < np)
                            load_pose(rotb, shb, pose_at(min(base + NW * KP + (pose_lane ? lane : 0), np - 1)), Rn,
                                      Sn);
                    } else {
                        load_pose(rotb, shb, pp, R, Sh);
                    }
                    int r0 = 0, r1 = -1;
                    if (sv) box_rows<GEN>(R, lo, hi, ts, r0, r1);
                    const int nr = sv ? max(0, r1 - r0 + 1) : 0;
                    const int rincl = dpp_scan_add(nr);
                    const int start = rincl - nr;  // the pose's first row in the batch's row list
                    const int rows = __builtin_amdgcn_readlane(rincl, 63);
                    if (sv) {
                        Slot& sd = slots[wave][buf + lane];
                        sd.R6[0] = R[0];
                        sd.R6[1] = R[1];
                        sd.R6[2] = R[3];
                        sd.R6[3] = R[4];
                        sd.R6[4] = R[6];
                        sd.R6[5] = R[7];
                        sd.s0 = Sh[0];
                        sd.s1 = Sh[1];
                        sd.base = (pose0 + pp) * int64_t(g.npix);
                        sd.r0 = r0;
                        sd.start = start;
                    }
                    __builtin_amdgcn_wave_barrier();
                    int pcarry = 0;
                    // (a batch without rows still runs one empty block when a window is carried, to
                    // deposit it: its samples' slots are overwritten by the next batch)
                    for (int rbase = 0; rbase < rows || (CARRY && rbase == 0 && m > 0); rbase += 64) {
                        // row rbase + lane of the batch: its pose (the pose lane whose rows hold it)
                        const int k = max(0, window_owner(nr, start, rbase, pcarry, marks[wave]));
                        const int f = rbase + lane;
                        int c0 = 0, cnt = 0, r = 0;
                        if (f < rows) {
                            const Slot& sd = slots[wave][buf + k];
                            float R6[6];
#pragma unroll
                            for (int e = 0; e < 6; ++e) R6[e] = sd.R6[e];
                            r = sd.r0 + (f - sd.start);
                            int c1;
                            row_span6(R6, r, lo, hi, ts, cut2, c0, c1);
                            cnt = max(0, c1 - c0 + 1);
                        }
                        const unsigned kr = kr_pack(buf + k, r);
                        const int incl = dpp_scan_add(cnt);
                        const int excl = incl - cnt;
                        const int total = __builtin_amdgcn_readlane(incl, 63);
                        const int cx = c0 - excl;  // column of flattened sample e in this row: cx + e
                        // the batch's last block deposits the window if the pass ends here, or if the
                        // window would still hold samples of the previous batch
                        const bool flush = !CARRY || (rbase + 64 >= rows && (last || (prev && m + total < 64)));
                        int carry = 0;
                        // sample e0 + lane of this row block (e < 0: a carried lane): owner lane, pixel,
                        // validity and the element to load (element 0 for lanes without a sample, so
                        // that every load is issued on every path: a load under a branch makes the
                        // compiler wait for it before the previous window's taps).  The owner row's
                        // pose slot and row come from its lane in one word.
                        auto locate = [&](int e0, unsigned& krl, int& rr_, int& cc_, int& sl_, bool& ok_,
                                          int64_t& pidx) {
                            const int e = e0 + lane;
                            const int lw = window_owner(cnt, excl, e0, carry, marks[wave]);
                            cc_ = __shfl(cx, lw, 64) + e;
                            krl = unsigned(__shfl(int(kr), lw, 64));
                            sl_ = int(krl >> 16);
                            rr_ = int(krl & 0xffffu) - int(kRowBias);
                            ok_ = (!CARRY || e >= 0) && e < total;
                            ok_ = ok_ && !filtered(float(rr_), float(cc_), cut2) &&
                                  !(cc_ == 0 && (rr_ == g.n / 2 || rr_ < 0));  // Friedel half of x = 0
                            const int pix = int(__umul24(unsigned(rr_ >= 0 ? rr_ : rr_ + g.n), unsigned(g.hp))) + cc_;
                            pidx = ok_ ? slots[wave][sl_].base + pix : 0;
                        };
                        if constexpr (CARRY) {
                            // the carried lanes stay; the others take samples 0 .. 63 - m of this block.
                            // Full windows are deposited, the last partial one waits unless flushed.
                            int e0 = -m;
                            {
                                unsigned kr2;
                                int rr2, cc2, sl2;
                                bool ok2;
                                int64_t pidx2;
                                locate(e0, kr2, rr2, cc2, sl2, ok2, pidx2);
                                const Cx<float> v2 = src[pidx2];
                                const float wv2 = WEIGHTS ? weights[pidx2] : 0.f;
                                const bool keep = lane < m;
                                krw = keep ? krw : kr2;
                                cc = keep ? cc : cc2;
                                ok = keep ? ok : ok2;
                                v = keep ? v : v2;
                                wv = keep ? wv : wv2;
                            }
                            for (; e0 + 64 <= total || (flush && e0 < total); e0 += 64) {
                                // the next window's loads are in flight while this one is spread
                                unsigned kr2 = 0;
                                int rr2, cc2 = 0, sl2;
                                bool ok2 = false;
                                int64_t pidx2 = 0;
                                if (e0 + 64 < total) locate(e0 + 64, kr2, rr2, cc2, sl2, ok2, pidx2);
                                const Cx<float> v2 = src[pidx2];
                                const float wv2 = WEIGHTS ? weights[pidx2] : 0.f;
                                if (ok)
                                    scatter_sample<CUBIC, MODE, WEIGHTS, OSX>(
                                        g, slots[wave][krw >> 16], int(krw & 0xffffu) - int(kRowBias), cc, v, wv,
                                        shifts != nullptr, pass == 1, tm, acc_re, acc_im, acc_w);
                                krw = kr2;
                                cc = cc2;
                                ok = ok2;
                                v = v2;
                                wv = wv2;
                                prev = false;
                            }
                            m = max(0, total - e0);
                        } else {
                            unsigned krl;
                            int rr, cc_w, sl;
                            bool okw;
                            int64_t pidx;
                            locate(0, krl, rr, cc_w, sl, okw, pidx);
                            Cx<float> vw = src[pidx];
                            float wvw = WEIGHTS ? weights[pidx] : 0.f;
                            for (int e0 = 0; e0 < total; e0 += 64) {
                                // the next window's loads are in flight while this one is spread
                                int rr2 = 0, cc2 = 0, sl2 = 0;
                                bool ok2 = false;
                                int64_t pidx2 = 0;
                                if (e0 + 64 < total) locate(e0 + 64, krl, rr2, cc2, sl2, ok2, pidx2);
                                const Cx<float> v2 = src[pidx2];
                                const float wv2 = WEIGHTS ? weights[pidx2] : 0.f;
                                if (okw)
                                    scatter_sample<CUBIC, MODE, WEIGHTS, OSX>(g, slots[wave][sl], rr, cc_w, vw, wvw,
                                                                         shifts != nullptr, pass == 1, tm, acc_re,
                                                                         acc_im, acc_w);
                                rr = rr2;
                                cc_w = cc2;
                                sl = sl2;
                                okw = ok2;
                                vw = v2;
                                wvw = wv2;
                            }
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                }
            }
            __syncthreads();
        }

        // write every stored cell of the tile once (core pieces add into a zeroed region).  GEN
        // adds onto what the rotation kernel wrote: core pieces with atomics, the other tiles (one
        // workgroup each) by a plain read and write; without rotations in the call it stores them
        if (GEN && !touched && (it.core || any_rot)) continue;
        if (empty && it.core) continue;  // (adds nothing)
        __syncthreads();
        {
            // each lane keeps one (c, r) of the tile and steps along d
            static_assert(NT % (SC * SR) == 0, "write-out lanes keep their column and row");
            const int lc = tid % SC, lr = (tid / SC) % SR;
            const int c = tc + lc, r = tr + lr;
            if (c < H && r <= half) {
                const int64_t row = b * g.vol + int64_t(r < 0 ? r + N : r) * H + c, plane = int64_t(N) * H;
                for (int ld = tid / (SC * SR); ld < SD; ld += NT / (SC * SR)) {
                    const int d = td + ld;
                    if (d > half) break;
                    const int64_t idx = row + (d < 0 ? d + N : d) * plane;
                    const int a = (ld * SR + lr) * SC + ((lc + acc_swizzle(lr, ld)) & (SC - 1));
                    if (it.core) {
                        atomic_add(&dst[idx].re, float(acc_re[a]));
                        atomic_add(&dst[idx].im, float(acc_im[a]));
                        if (WEIGHTS) atomic_add(&wdst[idx], float(acc_w[a]));
                    } else if (GEN && any_rot) {
                        const Cx<float> o = dst[idx];
                        dst[idx] = Cx<float>{o.re + float(acc_re[a]), o.im + float(acc_im[a])};
                        if (WEIGHTS) wdst[idx] += float(acc_w[a]);
                    } else if (empty) {
                        dst[idx] = Cx<float>{0.f, 0.f};
                        if (WEIGHTS) wdst[idx] = 0.f;
                    } else {
                        dst[idx] = Cx<float>{float(acc_re[a]), float(acc_im[a])};
                        if (WEIGHTS) wdst[idx] = float(acc_w[a]);
                    }
                }
            }
        }
        __syncthreads();
    }
}

// Hermitian completion of the x = 0 plane after an unmirrored accumulation:
// every x = 0 contribution v of the reference is also added, conjugated, at
// the partner cell (-d, -r) (projection_utils.h:481-492), so the final value
// of a cell is A(X) + conj(A(mirror X)) (weights: A_w(X) + A_w(mirror X)).
// One lane per unordered pair {X, mirror X}; self-partnered cells are kept.
template <bool WEIGHTS>
__global__ __launch_bounds__(kBlock) void k_mirror_x0(Geom g, Cx<float>* __restrict__ dst,
                                                      float* __restrict__ wdst) {
    const int N = g.N, H = g.H;
    const int64_t plane = int64_t(N) * N;
    for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < g.B * plane;
         e += int64_t(gridDim.x) * kBlock) {
        const int64_t b = e / plane;
        const int q = int(e - b * plane);
        const int de = q / N, re = q - de * N;
        const int dm = de == 0 ? 0 : N - de, rm = re == 0 ? 0 : N - re;
        const int qm = dm * N + rm;
        if (qm <= q) continue;  // self-partnered, or handled by the partner's lane
        const int64_t i0 = b * g.vol + int64_t(q) * H, i1 = b * g.vol + int64_t(qm) * H;
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

// Zero the stored cells of the scatter core tiles, which their pose-range
// pieces then accumulate into with atomics: cells e0, e0 + step, ... (wdst may be null).
__device__ __forceinline__ void zero_core_cells(const Geom& g, const TileSpec& ts, Cx<float>* __restrict__ dst,
                                                float* __restrict__ wdst, int64_t e0, int64_t step) {
    const int N = g.N, H = g.H, half = N / 2;
    const int dd = (ts.sd1 - ts.sd0) * SD, rr = (ts.sr1 - ts.sr0) * SR, cc = ts.sc1 * SC;
    const int64_t cells = int64_t(dd) * rr * cc;
    for (int64_t e = e0; e < g.B * cells; e += step) {
        const int64_t b = e / cells;
        const int64_t q = e - b * cells;
        const int c = int(q % cc), r = -half + 1 + ts.sr0 * SR + int((q / cc) % rr),
                  d = -half + 1 + ts.sd0 * SD + int(q / (int64_t(cc) * rr));
        if (c >= H || r > half || d > half) continue;
        const int re = r < 0 ? r + N : r, de = d < 0 ? d + N : d;
        const int64_t idx = b * g.vol + (int64_t(de) * N + re) * H + c;
        dst[idx] = Cx<float>{0.f, 0.f};
        if (wdst) wdst[idx] = 0.f;
    }
}
template <bool WEIGHTS>
__global__ __launch_bounds__(kBlock) void k_zero_core(Geom g, TileSpec ts, Cx<float>* __restrict__ dst,
                                                      float* __restrict__ wdst) {
    zero_core_cells(g, ts, dst, WEIGHTS ? wdst : nullptr, int64_t(blockIdx.x) * kBlock + threadIdx.x,
                    int64_t(gridDim.x) * kBlock);
}

// Pose bins (launch_pose_bins): one workgroup per rotation batch item, row of bins along c (bins
// differ there only in their c extent) and block of kBinPoses poses, so each pose is loaded once per
// row.  A lane tests its poses against every bin of the row with the tiles' plane test (a bit per
// bin); a wave reserves room for its hits in every bin of the row at once (one atomic instruction,
// a lane per bin, on the bins' counts) and writes them there.  A bin's list is thus in no particular order (the scatter's tiles cull it into
// per-tile lists that are unordered anyway).  A bin box holds every tile box of its 2 x 2 x 2 tiles
// with half a voxel to spare on each side, far beyond the rounding of either plane test, so a pose
// that crosses a tile's box is in its bin.  The counts start at zero (the pose pre-pass clears
// them).  With dst, the workgroups first zero the scatter's core cells (zero_core_cells).
constexpr int kBinThreads = 256, kBinPer = kBinPoses / kBinThreads;
static_assert(kBinPer * kBinThreads == kBinPoses, "bin pre-pass shape");
__global__ __launch_bounds__(kBinThreads) void k_pose_bins(Geom g, const float* __restrict__ rot, BinGrid bg,
                                                           BinBox bb, const CallPoses* __restrict__ cp, TileSpec ts,
                                                           Cx<float>* __restrict__ dst, float* __restrict__ wdst) {
    if (dst)
        zero_core_cells(g, ts, dst, wdst, int64_t(blockIdx.x) * kBinThreads + threadIdx.x,
                        int64_t(gridDim.x) * kBinThreads);
    const int lane = threadIdx.x & 63;
    const int nrow = bg.nb[1] * bg.nb[2];
    const int64_t blocks = (g.P + kBinPoses - 1) / kBinPoses;
    const int64_t w = blockIdx.x / blocks, pb = blockIdx.x - w * blocks;
    const int64_t rb = w / nrow;
    const int row = int(w - rb * nrow);
    const int idx[3] = {0, row % bg.nb[1], row / bg.nb[1]};
    float lo[3], hi[3];
#pragma unroll
    for (int a = 1; a < 3; ++a) {
        lo[a] = bb.org[a] + float(idx[a]) * bb.edge[a] - bb.lo_pad;
        hi[a] = bb.org[a] + float(idx[a] + 1) * bb.edge[a] + bb.hi_pad;
    }
    auto box_c = [&](int i) {
        lo[0] = bb.org[0] + float(i) * bb.edge[0] - bb.lo_pad;
        hi[0] = bb.org[0] + float(i + 1) * bb.edge[0] + bb.hi_pad;
    };
    // bins beyond the reach of the call's tiled poses (rotations, and the others up to their
    // largest singular value) take no pose; a call without tiled poses needs no bins.  Along c
    // (from 0 up) the distance grows, so the reached bins of a row come first.
    const float gen = call_reach(&cp->gen_reach), reach = fmaxf(call_flag(&cp->any_rot) ? bb.reach : 0.f, gen);
    int nreach = 0;
    for (int i = 0; i < bg.nb[0]; ++i) {
        box_c(i);
        float dist2 = 0.f;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const float q = lo[a] > 0.f ? lo[a] : (hi[a] < 0.f ? -hi[a] : 0.f);
            dist2 += q * q;
        }
        if (reach > 0.f && dist2 <= reach * reach) nreach = i + 1;
    }
    if (nreach == 0) return;
    const int P = int(g.P);
    const float* rotb = rot + rb * g.P * 9;
    int p[kBinPer];
    float R[kBinPer][9];
#pragma unroll
    for (int u = 0; u < kBinPer; ++u) {
        p[u] = int(pb) * kBinPoses + u * kBinThreads + int(threadIdx.x);
        load_rot(rotb + int64_t(min(p[u], P - 1)) * 9, R[u]);
    }
    const int64_t bin0 = (rb * nrow + row) * int64_t(bg.nb[0]);
    // the bins of the row in groups of 32, one hit mask bit per bin of the group (a volume of
    // fewer than 2^31 cells has at most 26 bins along c, but the loop does not rely on it)
    for (int i0 = 0; i0 < nreach; i0 += 32) {
        const int ng = min(32, nreach - i0);
        unsigned hits[kBinPer];  // bit i: the pose crosses bin i0 + i
#pragma unroll
        for (int u = 0; u < kBinPer; ++u) hits[u] = 0u;
        for (int i = 0; i < ng; ++i) {
            box_c(i0 + i);
#pragma unroll
            for (int u = 0; u < kBinPer; ++u) hits[u] |= (p[u] < P && plane_hits(R[u], lo, hi)) ? 1u << i : 0u;
        }
        // the wave's hits per bin of the group (lane i: bin i0 + i), then the room in every bin of
        // the group with one atomic instruction (one round trip, not one per bin)
        int room = 0;
        for (int i = 0; i < ng; ++i) {
            int total = 0;
#pragma unroll
            for (int u = 0; u < kBinPer; ++u) total += __popcll(__ballot((hits[u] >> i) & 1u));
            if (lane == i) room = total;
        }
        int first = 0;
        if (lane < ng && room > 0) first = atomicAdd(&bg.count[bin0 + i0 + lane], room);
        for (int i = 0; i < ng; ++i) {
            if (__builtin_amdgcn_readlane(room, i) == 0) continue;
            uint64_t m[kBinPer];
#pragma unroll
            for (int u = 0; u < kBinPer; ++u) m[u] = __ballot((hits[u] >> i) & 1u);
            int base = __builtin_amdgcn_readlane(first, i);
            unsigned short* out = bg.list + (bin0 + i0 + i) * g.P;
#pragma unroll
            for (int u = 0; u < kBinPer; ++u) {
                if ((hits[u] >> i) & 1u) {
                    const int rank = int(__builtin_amdgcn_mbcnt_hi(unsigned(m[u] >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo(unsigned(m[u]), 0u)));
                    out[base + rank] = (unsigned short)p[u];
                }
                base += __popcll(m[u]);
            }
        }
    }
}

// Work items of the rotation kernels' forward tile grid (the unit grid).
int64_t forw_items(const Geom& g, const TileSpec& ts) {
    const int fc = ts.fc1 - ts.fc0, fd = ts.fd1 - ts.fd0;
    return g.B * (int64_t(fc) * fc * fd * ts.fksplit + int64_t(ts.nt) * ts.nt * ts.ntfd);
}
// Workgroups of a launch of `kernel` over `items`: one per item (rotations), or the persistent
// GEN grid (the scatter's).
template <bool GEN, int RUN>
unsigned grid_of(int64_t items, const void* kernel, int threads) {
    const int64_t slots = kXcds * xcd_per<RUN>(items);
    if (!GEN) return grid_for(slots);
    const int64_t most = gen_grid(kernel, threads);
    return grid_for(slots > most ? most : slots);
}

// GEN forward-family grid: a quarter of the rotation kernel's slots (a multiple of kXcds), each
// workgroup stepping over the GEN grid's slots by the grid size.  As many workgroups as the
// rotation kernel's would make a call without such poses pay for their empty launch (about 10 us
// at the headline); a persistent grid (the workgroups that fit on the device at once) balances
// the tiles' uneven work worse: at poses scaled by 1.02 the forward took 0.87 ms with the persistent grid
// and per-XCD counters, 0.77 / 0.74 / 0.74 ms with an eighth / a quarter / half of the rotation
// slots, 0.83 ms with a sixteenth (and 1.29 against 1.69 ms with poses scaled by 1.4).
constexpr int kGenForwShare = 4;
inline unsigned gen_forw_grid(const Geom& g, const TileSpec& ts) {
    const int64_t w = kXcds * xcd_per<kRunForw>(forw_items(g, ts)) / kGenForwShare;
    return grid_for(std::max<int64_t>(kXcds, (w + kXcds - 1) / kXcds * kXcds));
}

// One forward-family kernel (GMODE 0, 1, 2) for rotations, then for the other tiled poses.
template <bool CUBIC, int KP, bool OSX, int GMODE, bool RS, bool WG, typename VS>
hipError_t forw_both(const Geom& g, const TileSpec& ts, const void* rec, const void* rot, const void* shifts,
                     void* out, CallPoses* cp, int gl, const void* gsrc, void* grot, void* gshift, const void* gw,
                     void* wout, hipStream_t s) {
    const auto kr = k_forw3_tiled<CUBIC, KP, OSX, GMODE, RS, WG, VS, false>;
    const auto kg = k_forw3_tiled<CUBIC, KP, OSX, GMODE, RS, WG, VS, true>;
    const int64_t rot_items = ts.flist ? ts.fcount : forw_items(g, ts);
    hipLaunchKernelGGL(kr, dim3(grid_of<false, kRunForw>(rot_items, (const void*)kr, kForwThreads)),
                       dim3(kForwThreads), 0, s, g, ts,
                       (const Cx<VS>*)rec, (const float*)rot, (const float*)shifts, (Cx<float>*)out, cp, gl,
                       (const Cx<float>*)gsrc, (float*)grot, (float*)gshift, (const float*)gw, (float*)wout);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kg, dim3(gen_forw_grid(g, ts)),
                       dim3(kForwThreads), 0, s, g, ts,
                       (const Cx<VS>*)rec, (const float*)rot, (const float*)shifts, (Cx<float>*)out, cp, gl,
                       (const Cx<float>*)gsrc, (float*)grot, (float*)gshift, (const float*)gw, (float*)wout);
    return hipGetLastError();
}

template <bool CUBIC, int MODE, bool WEIGHTS, int KP, bool OSX>
hipError_t scatter_launch(const Geom& g, const TileSpec& ts, const void* src, const void* weights, const void* rot,
                          const void* shifts, void* dst, void* wdst, CallPoses* cp, int gl, hipStream_t s) {
    const int64_t score = int64_t(ts.sd1 - ts.sd0) * (ts.sr1 - ts.sr0) * ts.sc1 * ts.ksplit;
    if (score > 0 && !ts.core_zeroed) {
        const int64_t cells = g.B * int64_t((ts.sd1 - ts.sd0) * SD) * ((ts.sr1 - ts.sr0) * SR) * (ts.sc1 * SC);
        int64_t blocks = (cells + kBlock - 1) / kBlock;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(k_zero_core<WEIGHTS>, dim3(unsigned(blocks)), dim3(kBlock), 0, s, g, ts, (Cx<float>*)dst,
                           (float*)wdst);
        const hipError_t ez = hipGetLastError();
        if (ez != hipSuccess) return ez;
    }
    // rotations write every tile (none: the other tiled poses store them); the other tiled
    // poses add onto them
    const int64_t work = g.B * (score + int64_t(ts.ntd) * ts.ntr * ts.ntc);
    const auto kr = k_scatter3_tiled<CUBIC, MODE, WEIGHTS, KP, OSX, false>;
    const auto kg = k_scatter3_tiled<CUBIC, MODE, WEIGHTS, KP, OSX, true>;
    hipLaunchKernelGGL(kr, dim3(grid_of<false, kRunScatter>(work, (const void*)kr, kScatterThreads)),
                       dim3(kScatterThreads), 0, s, g, ts,
                       (const Cx<float>*)src, (const float*)weights, (const float*)rot, (const float*)shifts,
                       (Cx<float>*)dst, (float*)wdst, cp, gl);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kg, dim3(grid_of<true, kRunScatter>(work, (const void*)kg, kScatterThreads)),
                       dim3(kScatterThreads), 0, s, g, ts,
                       (const Cx<float>*)src, (const float*)weights, (const float*)rot, (const float*)shifts,
                       (Cx<float>*)dst, (float*)wdst, cp, gl);
    e = hipGetLastError();
    if (e != hipSuccess || MODE != 0) return e;
    const int64_t pairs = g.B * int64_t(g.N) * g.N;
    int64_t blocks = (pairs + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_mirror_x0<WEIGHTS>, dim3(unsigned(blocks)), dim3(kBlock), 0, s, g, (Cx<float>*)dst,
                       (float*)wdst);
    return hipGetLastError();
}

template <bool CUBIC, int MODE, bool WEIGHTS, bool OSX>
hipError_t scatter_kp_osx(const Geom& g, const TileSpec& ts, const void* src, const void* weights, const void* rot,
                          const void* shifts, void* dst, void* wdst, CallPoses* cp, int gl, hipStream_t s) {
    // (the cubic stencil carries windows across batches and keeps two pose sets: at most 4 poses)
    if constexpr (!CUBIC)
        if (ts.kp_scatter >= 6)
            return scatter_launch<CUBIC, MODE, WEIGHTS, 6, OSX>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl,
                                                                s);
    if (ts.kp_scatter >= 4)
        return scatter_launch<CUBIC, MODE, WEIGHTS, 4, OSX>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    if (ts.kp_scatter >= 3)
        return scatter_launch<CUBIC, MODE, WEIGHTS, 3, OSX>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    return scatter_launch<CUBIC, MODE, WEIGHTS, 1, OSX>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
}

template <bool CUBIC, int MODE, bool WEIGHTS>
hipError_t scatter_kp(const Geom& g, const TileSpec& ts, const void* src, const void* weights, const void* rot,
                      const void* shifts, void* dst, void* wdst, CallPoses* cp, int gl, hipStream_t s) {
    if (ts.os_exact)
        return scatter_kp_osx<CUBIC, MODE, WEIGHTS, true>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
    return scatter_kp_osx<CUBIC, MODE, WEIGHTS, false>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
}

template <bool CUBIC, bool OSX>
hipError_t bpback_flags(const Geom& g, const TileSpec& ts, const void* gdata, const void* gw, const void* proj,
                        const void* rot, const void* shifts, void* gproj, void* gweights, void* grot, void* gshift,
                        CallPoses* cp, int gl, hipStream_t s) {
    // poses per wave batch: the forward's count, at most two with gradient sums (a set per pose)
    const bool rs = grot || gshift, wg = gw && gweights;
    const int kp = ts.kp_forw >= 4 ? 4 : (ts.kp_forw == 2 ? 2 : 1);
#define TP_BPB(KPV, RSV, WGV)                                                                                   \
    forw_both<CUBIC, KPV, OSX, 2, RSV, WGV, float>(g, ts, gdata, rot, shifts, gproj, cp, gl, proj, grot, gshift, gw, \
                                                   WGV ? gweights : nullptr, s)
    if (rs) {
        if (kp >= 2) return wg ? TP_BPB(2, true, true) : TP_BPB(2, true, false);
        return wg ? TP_BPB(1, true, true) : TP_BPB(1, true, false);
    }
    if (kp == 4) return wg ? TP_BPB(4, false, true) : TP_BPB(4, false, false);
    if (kp == 2) return wg ? TP_BPB(2, false, true) : TP_BPB(2, false, false);
    return wg ? TP_BPB(1, false, true) : TP_BPB(1, false, false);
#undef TP_BPB
}

template <bool CUBIC, bool OSX, typename VS>
hipError_t forw_kp(const Geom& g, const TileSpec& ts, const void* rec, const void* rot, const void* shifts, void* out,
                   CallPoses* cp, int gl, hipStream_t s) {
#define TP_FORW(KPV) \
    forw_both<CUBIC, KPV, OSX, 0, true, false, VS>(g, ts, rec, rot, shifts, out, cp, gl, nullptr, nullptr, nullptr, \
                                                   nullptr, nullptr, s)
    // the forward's batches spread their rows over the lanes: about 64 / (rows of a pose) poses
    if (ts.kp_forw >= 4) return TP_FORW(kForwFlatKP);
    if (ts.kp_forw == 2) return TP_FORW(3);
    return TP_FORW(1);
#undef TP_FORW
}

template <typename VS>
hipError_t forw_store(bool cubic, const Geom& g, const TileSpec& ts, const void* rec, const void* rot,
                      const void* shifts, void* out, CallPoses* cp, int gl, hipStream_t s) {
    if (cubic)
        return ts.os_exact ? forw_kp<true, true, VS>(g, ts, rec, rot, shifts, out, cp, gl, s)
                           : forw_kp<true, false, VS>(g, ts, rec, rot, shifts, out, cp, gl, s);
    return ts.os_exact ? forw_kp<false, true, VS>(g, ts, rec, rot, shifts, out, cp, gl, s)
                       : forw_kp<false, false, VS>(g, ts, rec, rot, shifts, out, cp, gl, s);
}

}  // namespace

int64_t forw_reach_items(const Geom& g, const TileSpec& ts, std::vector<int>& out) {
    const int64_t items = forw_items(g, ts);
    if (items > int64_t(INT32_MAX)) return items;
    // the rotation kernel's test (dist2 > rho2: the tile holds no sample) with a margin, so that
    // every tile the kernel would take is listed whatever the rounding
    const float rho = ts.rho_unit + 1.0f, rho2 = rho * rho * 1.001f + 4.0f;
    auto axis2 = [&](int t, int edge) {  // squared distance of [t, t + edge] (+ slack) from 0
        const float lo = float(t) - ts.eps, hi = float(t + edge) + ts.eps;
        const float q = lo > 0.f ? lo : (hi < 0.f ? -hi : 0.f);
        return q * q;
    };
    // the core pieces (item_of's first items) lie within 40 voxels of the origin: all listed
    const int cd = ts.fd1 - ts.fd0, cc = ts.fc1 - ts.fc0;
    const int64_t ncore = g.B * int64_t(cd) * cc * cc * ts.fksplit;
    for (int64_t w = 0; w < ncore; ++w) out.push_back(int(w));
    // then every tile of each batch item in item_of's order (kd, kr, kc), the core tiles skipped
    // when they are split
    const int nt = ts.nt, nd = ts.ntfd;
    for (int64_t b = 0; b < g.B; ++b)
        for (int kd = 0; kd < nd; ++kd) {
            const float d2 = axis2(ts.orgd + kd * LD, LD);
            for (int kr = 0; kr < nt; ++kr) {
                const float r2 = axis2(ts.org + kr * L, L);
                if (d2 + r2 > rho2) continue;
                const int64_t row = ncore + b * int64_t(nd) * nt * nt + (int64_t(kd) * nt + kr) * nt;
                const bool core_row = ts.fksplit > 1 && kd >= ts.fd0 && kd < ts.fd1 && kr >= ts.fc0 && kr < ts.fc1;
                for (int kc = 0; kc < nt; ++kc) {
                    if (core_row && kc >= ts.fc0 && kc < ts.fc1) continue;
                    if (d2 + r2 + axis2(ts.org + kc * L, L) <= rho2) out.push_back(int(row + kc));
                }
            }
        }
    return items;
}

hipError_t launch_pose_bins(const Geom& g, const void* rot, const BinGrid& bg, const BinBox& bb, const CallPoses* cp,
                            hipStream_t s, const TileSpec& ts, void* dst, void* wdst) {
    const int64_t blocks = g.B_rot * int64_t(bg.nb[1]) * bg.nb[2] * ((g.P + kBinPoses - 1) / kBinPoses);
    if (blocks == 0 || blocks > kBinMaxGroups) return hipErrorInvalidValue;  // make_bins keeps calls within
    hipLaunchKernelGGL(k_pose_bins, dim3(unsigned(blocks)), dim3(kBinThreads), 0, s, g, (const float*)rot, bg, bb, cp,
                       ts, (Cx<float>*)dst, (float*)wdst);
    return hipGetLastError();
}

hipError_t launch_project3_forw_tiled(bool cubic, const Geom& g, const TileSpec& ts, const void* rec,
                                      const void* rot, const void* shifts, void* out, CallPoses* cp, int gl,
                                      hipStream_t s, bool rec_half) {
    if (rec_half) return forw_store<__half>(cubic, g, ts, rec, rot, shifts, out, cp, gl, s);
    return forw_store<float>(cubic, g, ts, rec, rot, shifts, out, cp, gl, s);
}

hipError_t launch_grads3_tiled(bool cubic, const Geom& g, const TileSpec& ts, const void* gproj, const void* rec,
                               const void* rot, const void* shifts, void* grot, void* gshift, CallPoses* cp, int gl,
                               hipStream_t s, bool rec_half) {
    if (!grot && !gshift) return hipSuccess;
#define TP_GRADS(C, O, V) \
    forw_both<C, 2, O, 1, true, false, V>(g, ts, rec, rot, shifts, nullptr, cp, gl, gproj, grot, gshift, nullptr, \
                                          nullptr, s)
    if (rec_half) {
        if (cubic) return ts.os_exact ? TP_GRADS(true, true, __half) : TP_GRADS(true, false, __half);
        return ts.os_exact ? TP_GRADS(false, true, __half) : TP_GRADS(false, false, __half);
    }
    if (cubic) return ts.os_exact ? TP_GRADS(true, true, float) : TP_GRADS(true, false, float);
    return ts.os_exact ? TP_GRADS(false, true, float) : TP_GRADS(false, false, float);
#undef TP_GRADS
}

hipError_t launch_bpback3_tiled(bool cubic, const Geom& g, const TileSpec& ts, const void* gdata, const void* gw,
                                const void* proj, const void* rot, const void* shifts, void* gproj, void* gweights,
                                void* grot, void* gshift, CallPoses* cp, int gl, hipStream_t s) {
    if (cubic)
        return ts.os_exact ? bpback_flags<true, true>(g, ts, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift,
                                                      cp, gl, s)
                           : bpback_flags<true, false>(g, ts, gdata, gw, proj, rot, shifts, gproj, gweights, grot,
                                                       gshift, cp, gl, s);
    return ts.os_exact ? bpback_flags<false, true>(g, ts, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift,
                                                   cp, gl, s)
                       : bpback_flags<false, false>(g, ts, gdata, gw, proj, rot, shifts, gproj, gweights, grot, gshift,
                                                    cp, gl, s);
}

hipError_t launch_scatter3_tiled(bool cubic, int mode, const Geom& g, const TileSpec& ts, const void* src,
                                 const void* weights, const void* rot, const void* shifts, void* dst, void* wdst,
                                 CallPoses* cp, int gl, hipStream_t s) {
    if (mode == 0) {
        if (weights)
            return cubic ? scatter_kp<true, 0, true>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s)
                         : scatter_kp<false, 0, true>(g, ts, src, weights, rot, shifts, dst, wdst, cp, gl, s);
        return cubic ? scatter_kp<true, 0, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s)
                     : scatter_kp<false, 0, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s);
    }
    return cubic ? scatter_kp<true, 1, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s)
                 : scatter_kp<false, 1, false>(g, ts, src, nullptr, rot, shifts, dst, nullptr, cp, gl, s);
}

}  // namespace tp
