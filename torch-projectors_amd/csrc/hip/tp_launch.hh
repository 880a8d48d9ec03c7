// Internal interface between the C ABI (tp_capi.hip) and the kernel
// translation units.  Not installed; the public interface is
// include/torch_projectors_hip.h.
#pragma once

#include <hip/hip_runtime.h>

#include <vector>
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
    // Pixels that can be active (inside the cutoff disc) lie in a rectangle of
    // the grid: row frequencies [rr0, rr0 + rnr), columns [0, rnc).  The
    // per-pixel kernels walk only its rect = rnr * rnc pixels.
    int rr0, rnr, rnc, rect;
    int chunks;                    // 256-pixel blocks of the rectangle per pose
    int64_t work;                  // B*P*chunks
};

// Pose matrices whose first two columns (3D) or two columns (2D) have both
// singular values in [kScaleMin, kScaleMax] take the tiled kernels
// (pose_tiled3 / pose_tiled2): rotations, and scaled or sheared matrices such
// as magnification corrections, up to halving or doubling the sample grid.
// Their bounds use the columns themselves when the columns are orthonormal to
// kRotationTol, the dual basis otherwise (its conditioning is at most
// kScaleMax / kScaleMin = 4).  Degenerate and stronger scalings take the
// per-pixel kernels.
constexpr float kScaleMin = 0.5f, kScaleMax = 2.0f;
constexpr float kRotationTol = 1e-5f;

// Tile-owner enumeration parameters of the fp32 3D kernels (tp_tiled3d.hip).
constexpr int kTileEdge = 16, kTileEdgeD = 12;         // forward tiles: 16 x 16 (c, r) x 12 (d) voxels
constexpr int kScTC = 16, kScTR = 8, kScTD = 12;        // scatter tiles (c, r, d): fp64 accumulators

// Pose bins of the scatter tile grid, filled per call by launch_pose_bins: for each block of
// 2 x 2 x 2 tiles (a bin) and rotation batch item, the poses whose slice plane crosses the bin's
// box, in no particular order (any matrix: the plane is spanned by its first two columns).  The
// scatter's tiles outside the core then cull only their bin's poses instead of all P, in fewer and
// fuller phases.  list == nullptr: no bins (every tile culls all its poses).
constexpr int kBinPoses = 1024;  // poses per workgroup of the bin pre-pass
constexpr int64_t kBinMaxGroups = (int64_t(1) << 24) - 1;  // most workgroups of one bin pre-pass (256 lanes each
                                                          // stay below 2^32 lanes); a larger call gets no bins
struct BinGrid {
    unsigned short* list;  // [B_rot][n][P] pose indices (P < 65536); entries past the count unused
    int* count;            // [B_rot][n]
    int nb[3];             // bins along c, r, d
    int n;                 // nb[0] * nb[1] * nb[2]
};
// Box of bin (i, j, k) on axis a: [org[a] + idx * edge[a] - lo_pad, org[a] + (idx + 1) * edge[a] + hi_pad];
// bins whose box lies beyond `reach` of the origin hold no pose.
struct BinBox {
    float org[3], edge[3];
    float lo_pad, hi_pad, reach;
};
struct TileSpec {
    int nt, org;              // forward: tiles along c and r, and the signed origin of the grid there,
                              // laid out for unit-scale poses (|x| <= rho_unit + 1)
    int fc0, fc1;             // forward core tiles (split by pose range): [fc0, fc1) along c and r
    int ntfd, orgd, fd0, fd1;  // forward: the same along d (tiles of kTileEdgeD)
    int nt2, org2, ntfd2, orgd2;  // forward: the grid that the other tiled poses reach (|x| <= rho)
    int fc0_2, fc1_2, fd0_2, fd1_2;  // and its core tiles (the same voxels as fc0.. fd1)
    int ntd, ntr, ntc;        // scatter: tiles along d, r, c of the stored half volume
    int sd0, sd1, sr0, sr1, sc1;  // scatter core tiles: [sd0, sd1) x [sr0, sr1) x [0, sc1)
    int ksplit, prange;       // pose ranges per core tile, poses per range (the scatters, GEN gathers)
    int fksplit, fprange;     // the same for the rotation forward-family kernels (fc0.. fd1)
    float rho;                // bound on |x| of every active sample of a tiled pose (singular values <= kScaleMax)
    float rho_unit;           // the same for singular values <= 1, less the +1 voxel margin
    float eps;                // slack (voxels) added to every enumeration box
    float os, inv_os;         // oversampling and its inverse
    float smax;               // bound on |c*os| over the pixel grid
    int cmax, rmin, rmax;     // pixel-grid limits of c and r (grid and cutoff)
    // poses per wavefront batch by the rows a pose's box spans: kp_forw 1, 2 or 4 (the forward
    // launches 1, 3 or 5 of them, the gradient modes 1, 2 or 4); kp_scatter 1, 3, 4 or 6 (cubic
    // at most 4)
    int kp_forw, kp_scatter;
    bool os_exact;            // float(os) == os: c * os can be formed in float exactly as in double
    BinGrid sbins;            // pose bins of the scatter tile grid (list null: none)
    // forward: the rotation kernels' work items whose tiles the rotations' samples can reach, in
    // work-item order (forw_reach_items), fcount of them; flist null: every work item of the grid
    // (about half of the headline's tiles lie outside that sphere)
    const int* flist;
    int64_t fcount;
    bool core_zeroed;         // scatter: the bin pre-pass has zeroed the core tiles' cells
};

// The work items of the rotation kernels' forward tile grid (ts's nt, ntfd, core tiles and
// fksplit) whose tiles lie within rho_unit + 1 (and a margin) of the origin, in increasing order,
// appended to `out`; returns the grid's item count.  Host code, for TileSpec::flist.
int64_t forw_reach_items(const Geom& g, const TileSpec& ts, std::vector<int>& out);

// Tile-owner kernels of the fp32 2D operators (tp_tiled2d.hip).
constexpr int kTile2C = 32, kTile2R = 16;  // scatter tile edges (c, r): fp64 accumulators
constexpr int kGat2 = 32;                  // gather tile edge (c and r)
struct TileSpec2 {
    int kr0, nr, nc;        // tiles that rotations' taps reach: rows [kr0, kr0 + nr), columns [0, nc)
    int kr0_2, nr_2, nc_2;  // the same for the other tiled poses
    int ksplit, prange;     // pose ranges per tile, poses per range
    int kp;                 // poses per wavefront batch (1, 2 or 4)
    float rho;              // bound on |x| of every active sample of a tiled pose (singular values <= kScaleMax)
    float rho_unit;         // the same for singular values <= 1, less the +1 cell margin
    float eps;              // slack (cells) added to every enumeration box
    float os, inv_os;       // oversampling and its inverse
    float smax;             // bound on |c*os| over the pixel grid
    int cmax, rmin, rmax;   // pixel-grid limits of c and r (grid and cutoff)
    int gnt, gorg;          // gather: tiles per axis over the signed plane, and its origin (rotations)
    int gnt2, gorg2;        // gather: the same for the other tiled poses
    int gksplit, gprange;   // gather: pose ranges per tile, poses per range
    int kp_gather;          // gather (forward): poses per wavefront batch
};

// Per-call summary of the poses, written into a device scratch area by
// launch_call_poses before the tiled kernels of the call (stream order) and
// read by them: the rotation kernels do nothing when no pose is a rotation,
// the kernels of the other tiled poses (GEN) exit at once when there is no
// such pose, and the persistent kernels take their work from per-XCD
// counters.  A call runs at most kTiledPairs (rotation, GEN) kernel pairs;
// pair `gl` uses counter sets 2 gl (rotations) and 2 gl + 1 (GEN).
constexpr int kXcdCount = 8;    // XCDs of an MI355X (workgroups are dealt to them round-robin)
constexpr int kTiledPairs = 2;
struct CallPoses {
    int any_rot;      // some pose of the call is a rotation
    float gen_reach;  // rho_unit * (largest singular value of the other tiled poses) + 1; 0: none
    int all_rot;      // every pose of the call is a rotation (the rotation kernels skip the class test)
    int pad[13];
    unsigned next[2 * kTiledPairs][kXcdCount];  // batches of slots taken so far (zeroed by the pre-pass)
};
constexpr int kCallScratchBytes = 256;
static_assert(sizeof(CallPoses) <= kCallScratchBytes, "call scratch");

// Fill *cp for the B_rot * P poses at rot (dim 2 or 3), rho_unit = the
// TileSpec/TileSpec2 field of the call; also zero the `nzero` ints at `zero`
// (the call's pose-bin counts, or none).
hipError_t launch_call_poses(int dim, int64_t poses, const void* rot, float rho_unit, CallPoses* cp, hipStream_t s,
                             int* zero = nullptr, int64_t nzero = 0);

// Fill the pose bins bg (list and count allocated by the caller, the counts zeroed by
// launch_call_poses, which has also filled *cp) of the scatter tile grid whose bin boxes bb
// describes, for the B_rot * P poses at rot (bins beyond the reach of the call's tiled poses stay
// empty, bb.reach being the rotations').  With dst, the same workgroups zero the scatter's core
// tiles' cells of dst (and wdst) that ts describes, which the core pieces then add into.
hipError_t launch_pose_bins(const Geom& g, const void* rot, const BinGrid& bg, const BinBox& bb, const CallPoses* cp,
                            hipStream_t s, const TileSpec& ts, void* dst, void* wdst);

constexpr int kBlock = 256;
constexpr int64_t kMaxGrid = int64_t(1) << 22;

inline unsigned grid_for(int64_t work) { return unsigned(work < kMaxGrid ? work : kMaxGrid); }

// Zero `words` 32-bit words at p.
hipError_t launch_zero(void* p, int64_t words, hipStream_t s);
// Zero every pixel outside the active rectangle of [B, P, n, n/2+1] outputs
// (out complex, wout real; either may be null).
hipError_t launch_zero_outside(int dt, const Geom& g, void* out, void* wout, hipStream_t s);

// Kernel launchers; `dim` is 2 or 3, `dt` 0 (fp32) or 1 (fp64); launch_project_forw
// also takes `dt` 2: a complex-half volume with fp32 arithmetic and output.
// `rest_only` (fp32): only masked pixels and the poses that the tiled kernels
// do not take (pose_tiled3 / pose_tiled2).
hipError_t launch_project_forw(int dim, int dt, bool cubic, const Geom& g, const void* rec, const void* rot,
                               const void* shifts, void* out, hipStream_t s, bool rest_only = false);
// `rest` != 0 (fp32): tiled poses are left to the tiled kernels
// entirely (the tiled scatter gives their reconstruction gradient,
// launch_grads3_tiled / launch_gather2_tiled their rotation/shift gradients).
// `dt` 2: a complex-half volume with fp32 arithmetic, gradients and outputs.
hipError_t launch_project_back(int dim, int dt, bool cubic, const Geom& g, const void* gproj, const void* rec,
                               const void* rot, const void* shifts, void* grec, void* grot, void* gshift,
                               hipStream_t s, int rest = 0);
// `rest_only` (fp32 2D and 3D): only the poses that the tiled kernels do not take.
hipError_t launch_backproject_forw(int dim, int dt, bool cubic, const Geom& g, const void* proj, const void* weights,
                                   const void* rot, const void* shifts, void* data, void* wrec, hipStream_t s,
                                   bool rest_only = false);
// fp32 3D tile-owner paths (tiled poses only; the per-pixel kernels with
// `rest_only` complete the other poses and the masked pixels).  Each launches
// the rotation kernel and then the kernel of the other tiled poses, after
// launch_call_poses has filled *cp; `gl` (< kTiledPairs) picks their
// counters, distinct for the kernel pairs of one call.
// `rec_half`: the volume is stored as complex half and widened to fp32 on load.
hipError_t launch_project3_forw_tiled(bool cubic, const Geom& g, const TileSpec& ts, const void* rec,
                                      const void* rot, const void* shifts, void* out, CallPoses* cp, int gl,
                                      hipStream_t s, bool rec_half = false);
// Rotation/shift gradients of project_3d_to_2d_back for tiled poses, added
// into zero-filled grot / gshift (either may be null); `rec_half` as for the forward.
hipError_t launch_grads3_tiled(bool cubic, const Geom& g, const TileSpec& ts, const void* gproj, const void* rec,
                               const void* rot, const void* shifts, void* grot, void* gshift, CallPoses* cp, int gl,
                               hipStream_t s, bool rec_half = false);
// backproject_2d_to_3d_back for tiled poses into zero-filled outputs:
// grad_projections from grad_data_rec, grad_weights from grad_weight_rec (when
// both gw and gweights are given), rotation/shift gradients (either may be null).
hipError_t launch_bpback3_tiled(bool cubic, const Geom& g, const TileSpec& ts, const void* gdata, const void* gw,
                                const void* proj, const void* rot, const void* shifts, void* gproj, void* gweights,
                                void* grot, void* gshift, CallPoses* cp, int gl, hipStream_t s);
// mode 0: backprojection into data (+ weights), with the x = 0 Hermitian completion;
// mode 1: reconstruction gradient of the projection.
hipError_t launch_scatter3_tiled(bool cubic, int mode, const Geom& g, const TileSpec& ts, const void* src,
                                 const void* weights, const void* rot, const void* shifts, void* dst, void* wdst,
                                 CallPoses* cp, int gl, hipStream_t s);

// fp32 2D tile-owner scatter (tiled poses only), into zero-filled dst / wdst.
// mode 0: backprojection with the x = 0 Hermitian completion; mode 1:
// reconstruction gradient of the projection.
hipError_t launch_scatter2_tiled(bool cubic, int mode, const Geom& g, const TileSpec2& ts, const void* src,
                                 const void* weights, const void* rot, const void* shifts, void* dst, void* wdst,
                                 CallPoses* cp, int gl, hipStream_t s);
// fp32 2D tile-owner gathers (tiled poses only; the per-pixel kernels with
// `rest` complete the other poses and the masked pixels).  mode 0: forward
// (rec -> out); mode 1: rotation/shift gradients of project_2d_back (gsrc =
// grad_projections) into zero-filled grot / gshift; mode 2:
// backproject_2d_back (rec = grad_data_rec -> out, gw -> wout, and with gsrc =
// projections the gradients).
// `rec_half` (modes 0 and 1): the volume is stored as complex half and widened to fp32 on load.
hipError_t launch_gather2_tiled(bool cubic, int mode, const Geom& g, const TileSpec2& ts, const void* rec,
                                const void* gw, const void* rot, const void* shifts, void* out, void* wout,
                                const void* gsrc, void* grot, void* gshift, CallPoses* cp, int gl, hipStream_t s,
                                bool rec_half = false);

// Reference preparation (tp_fourier.hip).  Elements are opaque words of
// elem_bytes (2, 4, 8 or 16); `dim` spatial axes (2 or 3) after the batch.
// src [batch, n^dim] -> dst [batch, N^dim] = fftshift(zero-pad at pad_before).
hipError_t launch_fftshift_pad(int elem_bytes, int dim, const void* src, int64_t batch, int64_t n, int64_t N,
                               int64_t pad_before, void* dst, hipStream_t s);
// src [batch, L[0..dim)] -> dst [batch, m[0..dim)] = ifftshift(src)[crop_start : crop_start + m] per axis.
hipError_t launch_ifftshift_crop(int elem_bytes, int dim, const void* src, int64_t batch, const int64_t* L,
                                 const int64_t* m, int64_t crop_start, void* dst, hipStream_t s);
// out = data / (weights + reg) where weights + reg > 0, else 0; `dt` 0 (fp32) or 1 (fp64).
hipError_t launch_normalize(int dt, const void* data, const void* weights, int64_t elems, double reg, void* out,
                            hipStream_t s);

// rfftn / irfftn (norm="forward") of `batch` contiguous N^dim boxes through
// hipFFT (rocFFT), with cached plans; return a hipfftResult (0 = success).
// The inverse overwrites its input.
// fft_forward / fft_inverse return a hipfftResult, or kFftNoPlanUnderCapture: the stream is under
// graph capture and has no plan of this shape yet (making one allocates).
constexpr int kFftNoPlanUnderCapture = -1;
int fft_forward(int dt, int dim, int64_t batch, int64_t N, const void* real, void* spec, hipStream_t s);
int fft_inverse(int dt, int dim, int64_t batch, int64_t N, void* spec, void* real, hipStream_t s);

// `rest_only` (fp32): tiled poses were computed by the tiled gathers into
// zero-filled outputs and are skipped; other poses everything.
hipError_t launch_backproject_back(int dim, int dt, bool cubic, const Geom& g, const void* gdata, const void* gw,
                                   const void* proj, const void* rot, const void* shifts, void* gproj,
                                   void* gweights, void* grot, void* gshift, hipStream_t s, bool rest_only = false);

}  // namespace tp
