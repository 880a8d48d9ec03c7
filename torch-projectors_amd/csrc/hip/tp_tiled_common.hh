// Wave-level building blocks shared by the tile-owner kernels (tp_tiled3d.hip,
// tp_tiled2d.hip): DPP scans, the window-owner lookup of compacted sample
// lists, the XCD-aware hand-out of work items, and the reach of a call's
// general poses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tp_device.hh"
#include "tp_launch.hh"

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
// rows mark their first index in a per-wave LDS array (int or byte marks: a
// mark is a lane + 1 <= 64), a prefix max carries the marks forward, and
// `carry` brings the owner across windows.
template <typename M>
__device__ __forceinline__ int window_owner(int cnt, int excl, int e0, int& carry, M* marks) {
    const int lane = threadIdx.x & 63;
    marks[lane] = 0;
    __builtin_amdgcn_wave_barrier();
    if (cnt > 0 && excl >= e0 && excl < e0 + 64) marks[excl - e0] = M(lane + 1);
    __builtin_amdgcn_wave_barrier();
    const int m = max(dpp_scan_max(int(marks[lane])), carry);
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
static_assert(kXcds == kXcdCount, "XCD count");

// Slot sequence of a tiled kernel (slots map to work items through xcd_item).
//   GEN = false: slot blockIdx.x, then every gridDim.x-th one (one slot per
//                workgroup when the grid covers every slot, as the rotation
//                kernels' grids do; the GEN forward's grid is a quarter of
//                that and steps).
//   GEN = true:  a persistent grid of the workgroups that fit on the device
//                at once (gen_grid); a workgroup takes batches of kGrab slots
//                of its XCD (blockIdx.x mod kXcds) from that XCD's counter in
//                the call scratch, the next batch in flight while it works on
//                this one, until the XCD's `per` slots are taken.  With one
//                slot per batch an XCD's resident workgroups work on about as
//                many consecutive slots as the rotation kernel's do, so its L2
//                shares their halos and projection rows the same way.
// Every member is called by all lanes of the workgroup (next() synchronises
// them when a new batch is taken); `sh` is one int of LDS.
constexpr int kGrab = 1;
template <bool GEN>
struct Slots {
    int64_t s;       // current slot
    int64_t j, jend;  // GEN: index within the XCD's slots, end of the batch
    int64_t per;      // slots per XCD
    unsigned* ctr;    // GEN: the XCD's counter (batches)
    unsigned nxt;     // GEN, lane 0: the next batch, in flight
    int x;            // GEN: XCD
    __device__ __forceinline__ Slots(int64_t per_xcd, unsigned* counters, int* sh) : per(per_xcd) {
        if constexpr (GEN) {
            x = int(blockIdx.x % kXcds);
            ctr = counters + x;
            if (threadIdx.x == 0) *sh = int(atomicAdd(ctr, 1u));
            __syncthreads();
            j = int64_t(*sh) * kGrab;
            __syncthreads();
            jend = j + kGrab;
            if (threadIdx.x == 0) nxt = atomicAdd(ctr, 1u);
            s = j * kXcds + x;
        } else {
            s = blockIdx.x;
        }
    }
    __device__ __forceinline__ bool ok() const { return GEN ? j < per : s < kXcds * per; }
    __device__ __forceinline__ void next(int* sh) {
        if constexpr (GEN) {
            if (++j == jend) {
                if (threadIdx.x == 0) *sh = int(nxt);
                __syncthreads();
                j = int64_t(*sh) * kGrab;
                __syncthreads();
                jend = j + kGrab;
                if (threadIdx.x == 0 && j < per) nxt = atomicAdd(ctr, 1u);
            }
            s = j * kXcds + x;
        } else {
            s += gridDim.x;
        }
    }
};

// Workgroups of a GEN kernel's persistent grid: as many as are resident on the
// current device at once (occupancy of `kernel` with `threads` lanes times the
// CU count), a multiple of kXcds; kGenGrid when the runtime cannot say.
constexpr int64_t kGenGrid = 1024;
inline int64_t gen_grid(const void* kernel, int threads) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu < 1 ||
        cus < 1)
        return kGenGrid;
    const int64_t g = int64_t(per_cu) * cus / kXcds * kXcds;
    return g >= kXcds ? g : kGenGrid;
}

// Counter set of a kernel of tiled-kernel pair gl (tp_launch.hh: CallPoses).
template <bool GEN>
__device__ __forceinline__ unsigned* slot_counters(CallPoses* cp, int gl) { return cp->next[2 * gl + (GEN ? 1 : 0)]; }
// Fields of the call summary read with a vector load where they are used (a
// scalar load is hoisted to the kernel's start and waited for with the next).
// The pre-pass wrote them in an earlier kernel of the stream, so an L2-cached
// load sees them: a relaxed atomic of workgroup scope is such a load (an agent-
// scope one bypasses the L2 on every workgroup of a one-per-tile grid: a call
// without rotations spent 85 us in each rotation kernel's empty workgroups).
__device__ __forceinline__ int call_flag(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ float call_reach(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Tiles per half axis of a tile grid with edge `edge` centred on the origin
// that holds floor(x) of every sample with |x| <= reach (+ slack below 2).
__device__ __forceinline__ int half_tiles_for(float reach, int edge, int most) {
    return min(most, int(ceilf((reach + 2.0f) / float(edge))));
}

}  // namespace
}  // namespace tp
