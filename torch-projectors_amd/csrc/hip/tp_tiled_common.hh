// Wave-level building blocks shared by the tile-owner kernels (tp_tiled3d.hip,
// tp_tiled2d.hip): DPP scans, the window-owner lookup of compacted sample
// lists, the XCD-aware hand-out of work items, and the reach of a call's
// general poses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tp_device.hh"

namespace tp {
namespace {

__device__ __forceinline__ int to_int_clamped(float v) {
    v = fminf(fmaxf(v, -1.0e8f), 1.0e8f);
    return int(v);
}

// Last column of row r that can lie inside the cutoff disc, applied to a row
// span [c0, c1]: a row beyond the disc (cut2 - r^2 < 0) is empty, otherwise
// the span ends at most one column past the disc (the hardware square root is
// within an ulp, and the +1 covers it).  The cap is an optimisation only:
// every sample is still tested against the mask.  It is skipped when
// cut2 - r^2 is not a finite float below 1e16, so a cutoff of +inf, NaN (which
// masks nothing, as r^2 + c^2 > NaN is false) or beyond any int never reaches
// an undefined float-to-int conversion.
__device__ __forceinline__ int cap_to_disc(int c1, float fr, float cut2) {
    const float rem = cut2 - fr * fr;
    if (rem < 0.f) return -1;
    if (rem < 1.0e16f) return min(c1, int(__builtin_amdgcn_sqrtf(rem)) + 1);
    return c1;
}

// Wave-wide inclusive prefix sum / max with DPP row shifts and broadcasts
// (register-to-register inside the SIMD, no LDS round trip).  Call with
// every lane active.
__device__ __forceinline__ int dpp_scan_add(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}
// Values must be >= 0 (0 is the identity).
__device__ __forceinline__ int dpp_scan_max(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));
    return v;
}
__device__ __forceinline__ int wave_max(int v) { return __builtin_amdgcn_readlane(dpp_scan_max(max(v, 0)), 63); }

// Sum of v over the wave (every lane active), by the same DPP scan.
template <int CTRL, int ROWS> __device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWS, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0x111, 0xf>(v);  // row_shr:1
    v += dpp_f<0x112, 0xf>(v);  // row_shr:2
    v += dpp_f<0x114, 0xf>(v);  // row_shr:4
    v += dpp_f<0x118, 0xf>(v);  // row_shr:8
    v += dpp_f<0x142, 0xa>(v);  // row_bcast:15
    v += dpp_f<0x143, 0xc>(v);  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Row lanes hold `cnt` samples starting at flattened index `excl`.  For the
// window [e0, e0 + 64) every lane gets the row lane owning index e0 + lane:
// rows mark their first index in a per-wave LDS array, a prefix max carries
// the marks forward, and `carry` brings the owner across windows.
__device__ __forceinline__ int window_owner(int cnt, int excl, int e0, int& carry, int* marks) {
    const int lane = threadIdx.x & 63;
    marks[lane] = 0;
    __builtin_amdgcn_wave_barrier();
    if (cnt > 0 && excl >= e0 && excl < e0 + 64) marks[excl - e0] = lane + 1;
    __builtin_amdgcn_wave_barrier();
    const int m = max(dpp_scan_max(marks[lane]), carry);
    carry = __builtin_amdgcn_readlane(m, 63);
    __builtin_amdgcn_wave_barrier();
    return m - 1;
}

// The hardware deals workgroups to the 8 XCDs (each with its own L2) round-
// robin by workgroup id.  Items are handed out in runs of RUN neighbouring
// tiles per XCD (run k of XCD x is item run 8k + x), so an XCD's L2 shares the
// halos and projection rows of a run while the runs stay interleaved over the
// volume for balance.  Slots past the last item do nothing.
constexpr int kXcds = 8;
template <int RUN>
__host__ __device__ inline int64_t xcd_per(int64_t items) {
    const int64_t span = int64_t(kXcds) * RUN;
    return (items + span - 1) / span * RUN;
}
template <int RUN>
__device__ __forceinline__ int64_t xcd_item(int64_t slot) {
    const int64_t x = slot % kXcds, j = slot / kXcds;
    return ((j / RUN) * kXcds + x) * RUN + j % RUN;
}
// Opening scan of the GEN (non-rotation) tiled kernels: the radius their
// samples reach, rho_unit * (largest singular value over the call's tiled
// poses that are not rotations) + 1, or 0 when there is no such pose.  Every
// lane of the NT-lane workgroup takes part; `part` holds NT / 64 ints.
template <int DIM, int NT>
__device__ float general_reach(const float* __restrict__ rot, int64_t poses, float rho_unit, int* part) {
    constexpr int RS = DIM == 2 ? 4 : 9, U = 4;  // U poses per lane in flight
    float m = 0.f;
    for (int64_t p0 = threadIdx.x; p0 < poses; p0 += U * NT) {
        float R[U][RS];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t p = min(p0 + u * NT, poses - 1);
#pragma unroll
            for (int e = 0; e < RS; ++e) R[u][e] = rot[p * RS + e];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const PoseGram gr = DIM == 2 ? pose_gram2(R[u]) : pose_gram3(R[u]);
            if (p0 + u * NT < poses && !gram_is_rotation(gr) && gram_tiled(gr)) m = fmaxf(m, gram_smax(gr));
        }
    }
    // non-negative floats order like their bit patterns as ints
    const int wm = wave_max(__float_as_int(m));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = wm;
    __syncthreads();
    int b = 0;
    for (int w = 0; w < NT / 64; ++w) b = max(b, part[w]);
    __syncthreads();
    const float s = __int_as_float(b);
    return s > 0.f ? rho_unit * s + 1.0f : 0.f;
}

// Workgroups of a GEN kernel's persistent grid (a multiple of kXcds).
constexpr int64_t kGenGrid = 1024;

}  // namespace
}  // namespace tp
