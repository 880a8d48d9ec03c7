// Internal interface between the C ABI (tp_capi.hip) and the kernel
// translation units.  Not installed; the public interface is
// include/torch_projectors_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tp {

// Geometry shared by every kernel of one call.  All sizes are validated by
// the C ABI before a launch, so the kernels trust them.
struct Geom {
    int64_t B, P, B_rot, B_shift;  // batch, poses, rotation/shift batch (1 or B)
    int n, hp, npix;               // projection box, n/2+1, n*hp
    int N, H;                      // reconstruction box, N/2+1
    int64_t vol;                   // elements per reconstruction (N*H or N*N*H)
    double os;                     // oversampling
    double phase_k;                // -2*pi/n, in double (projection_utils.h:82-94)
    double cut2;                   // squared radius cutoff, rounded in the real type
    int chunks;                    // 256-pixel blocks per pose
    int64_t work;                  // B*P*chunks
};

constexpr int kBlock = 256;
constexpr int64_t kMaxGrid = int64_t(1) << 22;

inline unsigned grid_for(int64_t work) { return unsigned(work < kMaxGrid ? work : kMaxGrid); }

// Zero `words` 32-bit words at p.
hipError_t launch_zero(void* p, int64_t words, hipStream_t s);

// Kernel launchers; `dim` is 2 or 3, `dt` 0 (fp32) or 1 (fp64).
hipError_t launch_project_forw(int dim, int dt, bool cubic, const Geom& g, const void* rec, const void* rot,
                               const void* shifts, void* out, hipStream_t s);
hipError_t launch_project_back(int dim, int dt, bool cubic, const Geom& g, const void* gproj, const void* rec,
                               const void* rot, const void* shifts, void* grec, void* grot, void* gshift,
                               hipStream_t s);
hipError_t launch_backproject_forw(int dim, int dt, bool cubic, const Geom& g, const void* proj, const void* weights,
                                   const void* rot, const void* shifts, void* data, void* wrec, hipStream_t s);
hipError_t launch_backproject_back(int dim, int dt, bool cubic, const Geom& g, const void* gdata, const void* gw,
                                   const void* proj, const void* rot, const void* shifts, void* gproj,
                                   void* gweights, void* grot, void* gshift, hipStream_t s);

}  // namespace tp
