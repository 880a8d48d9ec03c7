// Per-call summary of the poses for the tiled kernels (launch_call_poses,
// tp_launch.hh): whether any pose is a rotation, whether every pose is one,
// and the reach of the other tiled poses (rho_unit times their largest
// singular value, plus a voxel).
// It also clears the work counters of the call's GEN kernels and, for a 3D
// scatter with pose bins, the bins' counts.
#include "tp_device.hh"
#include "tp_launch.hh"
#include "tp_tiled_common.hh"

namespace tp {

namespace {

constexpr int kPoseThreads = 1024;

template <int DIM>
__global__ __launch_bounds__(kPoseThreads) void k_call_poses(const float* __restrict__ rot, int64_t poses,
                                                             float rho_unit, CallPoses* __restrict__ cp,
                                                             int* __restrict__ zero, int64_t nzero) {
    for (int64_t i = threadIdx.x; i < nzero; i += kPoseThreads) zero[i] = 0;
    constexpr int RS = DIM == 2 ? 4 : 9, U = 4;  // U poses per lane in flight
    __shared__ int part[kPoseThreads / 64][3];
    float m = 0.f;  // largest singular value of a tiled pose that is not a rotation (0: none)
    int rot_seen = 0, other_seen = 0;
    for (int64_t p0 = threadIdx.x; p0 < poses; p0 += U * kPoseThreads) {
        float R[U][RS];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t p = min(p0 + u * kPoseThreads, poses - 1);
            // columns 0 and 1 (the Gram matrix needs no more)
#pragma unroll
            for (int e = 0; e < RS; ++e) R[u][e] = (DIM == 3 && e % 3 == 2) ? 0.f : rot[p * RS + e];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (p0 + u * kPoseThreads >= poses) continue;
            const PoseGram gr = DIM == 2 ? pose_gram2(R[u]) : pose_gram3(R[u]);
            if (gram_is_rotation(gr)) {
                rot_seen = 1;
            } else {
                other_seen = 1;
                if (gram_tiled(gr)) m = fmaxf(m, gram_smax(gr));
            }
        }
    }
    // non-negative floats order like their bit patterns as ints
    const int wm = wave_max(__float_as_int(m)), wr = wave_max(rot_seen), wo = wave_max(other_seen);
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6][0] = wm;
        part[threadIdx.x >> 6][1] = wr;
        part[threadIdx.x >> 6][2] = wo;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int b = 0, r = 0, o = 0;
        for (int w = 0; w < kPoseThreads / 64; ++w) {
            b = max(b, part[w][0]);
            r = max(r, part[w][1]);
            o = max(o, part[w][2]);
        }
        const float s = __int_as_float(b);
        cp->any_rot = r;
        cp->all_rot = r && !o;
        cp->gen_reach = s > 0.f ? rho_unit * s + 1.0f : 0.f;
    }
    if (threadIdx.x < 2 * kTiledPairs * kXcdCount) (&cp->next[0][0])[threadIdx.x] = 0u;
}

}  // namespace

hipError_t launch_call_poses(int dim, int64_t poses, const void* rot, float rho_unit, CallPoses* cp, hipStream_t s,
                             int* zero, int64_t nzero) {
    if (dim == 2)
        hipLaunchKernelGGL(k_call_poses<2>, dim3(1), dim3(kPoseThreads), 0, s, (const float*)rot, poses, rho_unit, cp,
                           zero, nzero);
    else
        hipLaunchKernelGGL(k_call_poses<3>, dim3(1), dim3(kPoseThreads), 0, s, (const float*)rot, poses, rho_unit, cp,
                           zero, nzero);
    return hipGetLastError();
}

}  // namespace tp
