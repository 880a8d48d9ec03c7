// Per-call reach of the tiled poses (launch_pose_reach, tp_launch.hh).
//
// The tile grids of the tiled kernels are laid out for poses whose singular
// values reach kScaleMax, so that scaled matrices take the tiled path; this
// pre-pass finds the largest singular value among one call's tiled poses, and
// the tiles beyond the radius that the call's samples actually reach do no
// work (for rotations, the same tiles as before the grids were widened).
#include "tp_device.hh"
#include "tp_launch.hh"
#include "tp_tiled_common.hh"

namespace tp {

namespace {

constexpr int kReachThreads = 1024;

template <int DIM>
__global__ __launch_bounds__(kReachThreads) void k_pose_reach(const float* __restrict__ rot, int64_t poses,
                                                              float rho_unit, float* __restrict__ out) {
    constexpr int RS = DIM == 2 ? 4 : 9;
    __shared__ int part[kReachThreads / 64];
    float m = 0.f;  // largest singular value of a tiled pose seen so far (0: none)
    for (int64_t p = threadIdx.x; p < poses; p += kReachThreads) {
        const float* R = rot + p * RS;
        const PoseGram gr = DIM == 2 ? pose_gram2(R) : pose_gram3(R);
        if (gram_takes_tiles(gr)) m = fmaxf(m, gram_smax(gr));
    }
    // non-negative floats order like their bit patterns as ints
    const int wm = wave_max(__float_as_int(m));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = wm;
    __syncthreads();
    if (threadIdx.x == 0) {
        int b = 0;
        for (int w = 0; w < kReachThreads / 64; ++w) b = max(b, part[w]);
        const float s = __int_as_float(b);
        out[0] = s > 0.f ? rho_unit * s + 1.0f : 0.f;
    }
}

}  // namespace

hipError_t launch_pose_reach(int dim, int64_t poses, const void* rot, float rho_unit, float* out, hipStream_t s) {
    if (dim == 2)
        hipLaunchKernelGGL(k_pose_reach<2>, dim3(1), dim3(kReachThreads), 0, s, (const float*)rot, poses, rho_unit,
                           out);
    else
        hipLaunchKernelGGL(k_pose_reach<3>, dim3(1), dim3(kReachThreads), 0, s, (const float*)rot, poses, rho_unit,
                           out);
    return hipGetLastError();
}

}  // namespace tp
