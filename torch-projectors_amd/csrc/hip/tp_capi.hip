// C ABI of libtorch_projectors_hip.so (declared in include/torch_projectors_hip.h).
//
// Each entry point validates its arguments with the conditions of the
// reference (validate_projection_inputs, projection_utils.h:23-48, and the
// per-op TORCH_CHECKs), derives the launch geometry, zero-fills the outputs
// that are accumulated, and enqueues the kernels on the caller's stream.
// Nothing is synchronised.  The only memory besides the caller's is a small
// scratch area per (device, stream) that the calls of the tiled kernels use
// (tp::CallPoses: a summary of their poses and work counters), allocated by
// the first such call on that stream and kept for the life of the process;
// tp_project_3d_to_2d_forw_noalloc uses a static device array instead.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../../include/torch_projectors_hip.h"
#include "tp_launch.hh"

namespace {

thread_local std::string g_err;

int fail(const std::string& m) {
    g_err = m;
    return TP_ERR_INVALID;
}

int hip_fail(hipError_t e, const char* what) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return TP_ERR_HIP;
}

constexpr int64_t kInt32Max = 2147483647;

// Shared argument checks; fills the pose part of `g`.
int check_common(int dtype, int interp, int64_t B, int64_t P, int64_t B_rot, const void* shifts, int64_t B_shift,
                 tp::Geom& g) {
    if (dtype != TP_F32 && dtype != TP_F64) return fail("dtype must be TP_F32 or TP_F64");
    if (interp != TP_LINEAR && interp != TP_CUBIC) return fail("Supported interpolation methods: 'linear', 'cubic'");
    if (B < 0 || P < 0) return fail("batch and pose counts must be non-negative");
    if (B_rot != B && B_rot != 1) return fail("Batch size of rotations must be 1 or same as reconstruction");
    if (shifts && B_shift != B && B_shift != 1)
        return fail("Batch size of shifts must be 1 or same as reconstruction");
    g.B = B;
    g.P = P;
    g.B_rot = B_rot;
    g.B_shift = shifts ? B_shift : 1;
    return TP_OK;
}

int set_proj(int64_t n, tp::Geom& g) {
    if (n < 1) return fail("projection box size must be positive");
    const int64_t hp = n / 2 + 1;
    if (n * hp > kInt32Max) return fail("projection too large (n*(n/2+1) must be < 2^31)");
    g.n = int(n);
    g.hp = int(hp);
    g.npix = int(n * hp);
    g.phase_k = -2.0 * M_PI / double(n);
    return TP_OK;
}

int set_rec(int dim, int64_t N, int64_t H, tp::Geom& g) {
    if (N < 2) return fail("reconstruction box size must be at least 2");
    if (H != N / 2 + 1) return fail("reconstruction last dimension must be boxsize/2+1");
    const int64_t vol = dim == 2 ? N * H : N * N * H;
    if (vol > kInt32Max) return fail("reconstruction too large (elements per batch item must be < 2^31)");
    g.N = int(N);
    g.H = int(H);
    g.vol = vol;
    return TP_OK;
}

// Squared cutoff radius, rounded in the real type like the reference
// (cpu/3d/projection_3d_to_2d_kernels.cpp:145-149): default radius n/2.
void set_cut(int dtype, int has_cut, double cut, tp::Geom& g) {
    const double radius = has_cut ? cut : double(g.n) / 2.0;
    if (dtype == TP_F32) {
        const float rf = float(radius);
        const float r2 = rf * rf;
        g.cut2 = double(r2);
    } else {
        g.cut2 = radius * radius;
    }
    // Active rectangle: |r|, c <= floor(sqrt(cut2)) + 2 covers every pixel the
    // mask keeps (r^2 + c^2 <= cut2 in the real type); the whole grid when the
    // radius is not finite or reaches past the grid.
    const int lo = g.n / 2 + 1 - g.n, hi = g.n / 2;
    int cl = hi + 1;
    if (std::isfinite(g.cut2) && g.cut2 < double(hi + 1) * double(hi + 1))
        cl = int(std::floor(std::sqrt(g.cut2))) + 2;
    g.rr0 = std::max(lo, -cl);
    g.rnr = std::min(hi, cl) - g.rr0 + 1;
    g.rnc = std::min(g.hp, cl + 1);
    g.rect = g.rnr * g.rnc;
    g.chunks = (g.rect + tp::kBlock - 1) / tp::kBlock;
    g.work = g.B * g.P * g.chunks;
}

int64_t rec_box(int64_t n, double os) {
    const int64_t raw = static_cast<int64_t>(std::ceil(double(n) * os));
    return raw + (raw % 2);
}

// The fp32 3D operators run the tile-owner kernels for tiled poses (pose_tiled3).
// (Their per-wave sample queues pack a column index into 14 bits: n <= 32766.)
bool use_tiles(int dim, int dtype, double os, int64_t n) {
    return dim == 3 && dtype == TP_F32 && os > 0.0 && std::isfinite(os) && n <= 32766;
}

// Poses per wavefront batch: 64 lanes hold one row of the pose's samples
// each, so a batch takes 64 / rows poses (rows bounded for a box of width w).
int poses_per_batch(double w, double eps, double os) {
    // typical |b_c| + |b_r| + |b_d| of a unit column is about 1.5 (at most sqrt(3));
    // poses with more rows take a second pass over their rows
    const int rows = int(std::floor(1.5 * (w + 2.0 * eps) / os)) + 2;
    return rows <= 16 ? 4 : (rows <= 32 ? 2 : 1);
}

// Poses per wavefront batch of the 3D scatter, whose lanes take the batch's rows (all its poses' in
// turn) in blocks of 64: about 64 / (typical rows of a pose), measured best at 6 for a pose with
// about 10 rows (a 17-voxel box at oversampling 2) and at 4 for the cubic stencil's 19-voxel box;
// poses with more rows share the batch with fewer.  (The cubic kernels take at most 4.)
int scatter_poses_per_batch(double w, double eps, double os) {
    const int rows = int(std::floor(1.5 * (w + 2.0 * eps) / os)) + 2;
    return rows <= 14 ? 6 : (rows <= 21 ? 4 : (rows <= 32 ? 3 : 1));
}

// Poses per range of the forward projection's rotation kernel's core tiles: 2048 at oversampling 2
// and above, fewer as the oversampling (and so the spacing of a pose's samples) shrinks, so that a
// range holds about as many samples: at oversampling 1 a core tile holds four times the samples
// per pose, and unsplit core tiles became the critical path there (the published rows' linear
// batch-1 forward 0.50 -> 0.86 ms at 2048), so it takes 512 like the rest.
int64_t forw_poses_per_range(double os) {
    const double r = 2048.0 * (os / 2.0) * (os / 2.0);
    return r >= 2048.0 ? 2048 : (r <= 512.0 || !(r == r) ? 512 : int64_t(r));
}
// pkf: poses per range of the rotation forward-family kernels' core tiles (forward projections
// take forw_poses_per_range, their backward ops the scatter's 512).
tp::TileSpec tile_spec(const tp::Geom& g, bool cubic, int64_t pkf = 512) {
    constexpr int L = tp::kTileEdge;
    tp::TileSpec ts{};
    // radius bound of the active pixels: the cutoff disc, within the pixel grid
    const double grid_r = std::sqrt(2.0) * double(g.n / 2 + 1);
    double cutr = g.cut2 >= 0.0 ? std::sqrt(g.cut2) : grid_r;
    if (!std::isfinite(cutr) || cutr > grid_r) cutr = grid_r;
    // samples of rotations lie within rho_unit + 1; those of the other tiled poses (singular
    // values up to kScaleMax) within rho, on a second, wider forward grid
    const double rho_unit = g.os * cutr * 1.001;
    const double rho = rho_unit * tp::kScaleMax + 1.0;
    const int half_tiles = int(std::ceil((rho_unit + 3.0) / L));
    ts.nt = 2 * half_tiles;
    ts.org = -half_tiles * L;
    const int half_tiles_d = int(std::ceil((rho_unit + 3.0) / tp::kTileEdgeD));
    ts.ntfd = 2 * half_tiles_d;
    ts.orgd = -half_tiles_d * tp::kTileEdgeD;
    const int half2 = int(std::ceil((rho + 2.0) / L)), half2_d = int(std::ceil((rho + 2.0) / tp::kTileEdgeD));
    ts.nt2 = 2 * half2;
    ts.org2 = -half2 * L;
    ts.ntfd2 = 2 * half2_d;
    ts.orgd2 = -half2_d * tp::kTileEdgeD;
    const int half = g.N / 2;
    ts.ntd = (g.N + tp::kScTD - 1) / tp::kScTD;
    ts.ntr = (g.N + tp::kScTR - 1) / tp::kScTR;
    ts.ntc = (g.H + tp::kScTC - 1) / tp::kScTC;
    // Every random slice plane crosses the tiles around the origin, so those
    // carry up to P poses each; they are split into pose ranges so that no
    // single workgroup holds the critical path.  Core = tiles within `rc`
    // voxels of the origin on every axis.
    const int rc = 40;
    ts.fc0 = std::max(0, (-rc - ts.org) / L);
    ts.fc1 = std::min(ts.nt, (rc - ts.org) / L + 1);
    ts.fd0 = std::max(0, (-rc - ts.orgd) / tp::kTileEdgeD);
    ts.fd1 = std::min(ts.ntfd, (rc - ts.orgd) / tp::kTileEdgeD + 1);
    ts.fc0_2 = std::max(0, (-rc - ts.org2) / L);
    ts.fc1_2 = std::min(ts.nt2, (rc - ts.org2) / L + 1);
    ts.fd0_2 = std::max(0, (-rc - ts.orgd2) / tp::kTileEdgeD);
    ts.fd1_2 = std::min(ts.ntfd2, (rc - ts.orgd2) / tp::kTileEdgeD + 1);
    ts.sd0 = std::max(0, (-rc + half - 1) / tp::kScTD);
    ts.sd1 = std::min(ts.ntd, (rc + half - 1) / tp::kScTD + 1);
    ts.sr0 = std::max(0, (-rc + half - 1) / tp::kScTR);
    ts.sr1 = std::min(ts.ntr, (rc + half - 1) / tp::kScTR + 1);
    ts.sc1 = std::min(ts.ntc, rc / tp::kScTC + 1);
    // poses per range: the scatter's core tiles carry the most work of its grid and split at 512
    // (at 1024 the headline backprojection took 1.41 ms against 1.34; backprojection_ranges
    // lengthens them for calls of more than 2048 poses), as do the kernels of the
    // other tiled poses and the gradient modes (1-4 % slower at 2048); the rotation forward
    // projection's split at pkf (at oversampling 2, c2's forward 0.317 ms at 512 against 0.299 at
    // 2048, the headline's the same)
    const int64_t pk = 512;
    ts.ksplit = int(std::max<int64_t>(1, (g.P + pk - 1) / pk));
    ts.prange = int((g.P + ts.ksplit - 1) / ts.ksplit);
    ts.fksplit = int(std::max<int64_t>(1, (g.P + pkf - 1) / pkf));
    ts.fprange = int((g.P + ts.fksplit - 1) / ts.fksplit);
    if (ts.ksplit == 1)  // nothing to split
        ts.fc1_2 = ts.fc0_2 = ts.fd1_2 = ts.fd0_2 = ts.sd1 = ts.sd0 = ts.sr1 = ts.sr0 = ts.sc1 = 0;
    if (ts.fksplit == 1) ts.fc1 = ts.fc0 = ts.fd1 = ts.fd0 = 0;
    ts.rho = float(rho);
    ts.rho_unit = float(rho_unit);
    ts.os = float(g.os);
    ts.inv_os = float(1.0 / g.os);
    ts.os_exact = double(float(g.os)) == g.os;
    ts.smax = float(g.os * (g.n + 2));
    // Slack of the sample boxes: the row and half-plane bounds of a rotation
    // use its orthonormality (off by at most kRotationTol * |sc, sr| each), those
    // of the other tiled poses their fp32 dual basis (relative error ~1e-6),
    // plus fp32 rounding of the bounds themselves.
    ts.eps = 0.01f + 2.0f * tp::kRotationTol * ts.smax;
    ts.kp_forw = poses_per_batch(L, ts.eps, g.os);
    ts.kp_scatter = scatter_poses_per_batch(tp::kScTC + (cubic ? 3 : 1), ts.eps, g.os);
    const int cl = int(std::floor(cutr)) + 1;
    ts.cmax = std::min(g.n / 2, cl);
    ts.rmin = std::max(g.n / 2 + 1 - g.n, -cl);
    ts.rmax = std::min(g.n / 2, cl);
    return ts;
}

// Pose ranges of the backprojection's core tiles: about four per call, from 512 up to 2048
// poses each (512 for up to 2048 poses, as tile_spec sets them).  With more poses a range of
// 512 left the core's global float atomics the larger cost: c3's shape (8192 poses) took
// 1.369 ms at 512, 1.347 ms at 2048 and 1.372 ms at 1024 poses per range (A/B medians).  The
// reconstruction-gradient scatter keeps 512 (the cubic one was slower with longer ranges).
void backprojection_ranges(const tp::Geom& g, tp::TileSpec& ts) {
    const int64_t pk = std::min<int64_t>(2048, std::max<int64_t>(512, g.P / 4));
    ts.ksplit = int(std::max<int64_t>(1, (g.P + pk - 1) / pk));
    ts.prange = int((g.P + ts.ksplit - 1) / ts.ksplit);
}

// fp32 2D operators take the tile-owner kernels (tp_tiled2d.hip) for tiled poses (pose_tiled2).
bool use_tiles2(int dim, int dtype, double os, int64_t n) {
    return dim == 2 && dtype == TP_F32 && os > 0.0 && std::isfinite(os) && n <= 32766;
}

tp::TileSpec2 tile_spec2(const tp::Geom& g, bool cubic) {
    constexpr int TC = tp::kTile2C, TR = tp::kTile2R;
    tp::TileSpec2 ts{};
    const double grid_r = std::sqrt(2.0) * double(g.n / 2 + 1);
    double cutr = g.cut2 >= 0.0 ? std::sqrt(g.cut2) : grid_r;
    if (!std::isfinite(cutr) || cutr > grid_r) cutr = grid_r;
    // samples of rotations lie within rho_unit + 1, those of the other tiled poses within rho
    const double rho_unit = g.os * cutr * 1.001;
    const double rho = rho_unit * tp::kScaleMax + 1.0;
    // tiles whose cells a tap can reach: |r| and c within the radius plus the stencil
    const int half = g.N / 2;
    const int ntr = (g.N + TR - 1) / TR, ntc = (g.H + TC - 1) / TC;
    auto tiles_within = [&](double radius, int& kr0, int& nr, int& nc) {
        const double reach = std::min(radius + 3.0, double(g.N));
        kr0 = std::max(0, int(std::floor((-reach + half - 1) / TR)));
        const int kr1 = std::min(ntr, int(std::floor((reach + half - 1) / TR)) + 1);
        nr = std::max(0, kr1 - kr0);
        nc = std::min(ntc, int(std::floor(reach / TC)) + 1);
    };
    tiles_within(rho_unit + 1.0, ts.kr0, ts.nr, ts.nc);
    tiles_within(rho, ts.kr0_2, ts.nr_2, ts.nc_2);
    // Every pose reaches every tile of the disc: split the poses into ranges until there are
    // about 65536 work items, keeping >= 128 poses a range.  A workgroup's item is long (all of
    // its range's poses cross its tile), so many short items balance the CUs far better than the
    // partial tiles' extra float atomics cost: c5's backprojection (1360 tiles, 4096 poses)
    // took 13.07 ms at about 4096 items (4 ranges), 11.72 at 8192, 10.18 at 32768 and 10.03
    // at 32 ranges of 128 poses; ranges of 84 poses 10.05, of 43 poses 10.23 ms (A/B medians;
    // its reconstruction gradient 16.50 -> 13.54 ms).
    const int64_t tiles = g.B * int64_t(ts.nr) * ts.nc;
    const int64_t want = tiles > 0 ? (65536 + tiles - 1) / tiles : 1;
    const int64_t most = std::max<int64_t>(1, g.P / 128);
    ts.ksplit = int(std::max<int64_t>(1, std::min(want, most)));
    ts.prange = int((g.P + ts.ksplit - 1) / ts.ksplit);
    ts.rho = float(rho);
    ts.rho_unit = float(rho_unit);
    ts.os = float(g.os);
    ts.inv_os = float(1.0 / g.os);
    ts.smax = float(g.os * (g.n + 2));
    ts.eps = 0.01f + 2.0f * tp::kRotationTol * ts.smax;
    // rows of a pose's samples in one box: at most its diagonal over os, plus the ends
    const double wc = TC + (cubic ? 3 : 1) + 2.0 * ts.eps, wr = TR + (cubic ? 3 : 1) + 2.0 * ts.eps;
    const int rows = int(std::ceil(std::sqrt(wc * wc + wr * wr) / g.os)) + 2;
    ts.kp = rows <= 16 ? 4 : (rows <= 32 ? 2 : 1);
    const int cl = int(std::floor(cutr)) + 1;
    ts.cmax = std::min(g.n / 2, cl);
    ts.rmin = std::max(g.n / 2 + 1 - g.n, -cl);
    ts.rmax = std::min(g.n / 2, cl);
    // gather: square tiles over the signed plane within the radius (+2), and pose ranges
    constexpr int GT = tp::kGat2;
    const int half_g = int(std::ceil((rho_unit + 3.0) / GT)), half_g2 = int(std::ceil((rho + 2.0) / GT));
    ts.gnt = 2 * half_g;
    ts.gorg = -half_g * GT;
    ts.gnt2 = 2 * half_g2;
    ts.gorg2 = -half_g2 * GT;
    // A gather's pose range writes only its own poses' pixels (its pose-gradient atomics are one
    // set per tile and pose whatever the ranges), so its ranges go down to 16 poses: a small call
    // (256 poses over 64 tiles) then fills the GPU, where ranges of at least 128 left it 128 work
    // items.  As for the scatters, about 65536 items balance best: c5's forward took 7.66 ms at
    // about 4096 items, 7.10 at 16384 and 6.93 at 65536 (backproject_2d_back 13.83 -> 12.23,
    // project_2d_back 13.48 -> 12.30 ms; A/B medians); 131072 and 262144 items were 1-2 % and
    // 6-8 % slower than 65536 in all three.
    const int64_t gtiles = g.B * int64_t(ts.gnt) * ts.gnt;
    const int64_t gwant = gtiles > 0 ? (65536 + gtiles - 1) / gtiles : 1;
    const int64_t gmost = std::max<int64_t>(1, g.P / 16);
    ts.gksplit = int(std::max<int64_t>(1, std::min(gwant, gmost)));
    ts.gprange = int((g.P + ts.gksplit - 1) / ts.gksplit);
    const double gw = GT + 2.0 * ts.eps;
    const int grows = int(std::ceil(std::sqrt(2.0) * gw / g.os)) + 2;
    ts.kp_gather = grows <= 16 ? 4 : (grows <= 32 ? 2 : 1);
    return ts;
}

int64_t cx_words(int dtype, int64_t elems) { return elems * (dtype == TP_F32 ? 2 : 4); }
int64_t re_words(int dtype, int64_t elems) { return elems * (dtype == TP_F32 ? 1 : 2); }

int zero(void* p, int64_t words, hipStream_t s) {
    if (!p || words <= 0) return TP_OK;
    const hipError_t e = tp::launch_zero(p, words, s);
    return e == hipSuccess ? TP_OK : hip_fail(e, "zero-fill launch");
}

int need(const void* p, const char* name) {
    if (!p) return fail(std::string(name) + " must not be NULL");
    return TP_OK;
}

#define TP_TRY(expr)                 \
    do {                             \
        const int rc_ = (expr);      \
        if (rc_ != TP_OK) return rc_; \
    } while (0)

int launched(hipError_t e, const char* what) { return e == hipSuccess ? TP_OK : hip_fail(e, what); }

// Scratch of the calls on one (device, stream).  Calls on one stream run in
// order on the GPU, so they share it; `busy` is held while one call enqueues
// its kernels, so that calls from several host threads on one stream do not
// interleave their kernels.
struct StreamScratch {
    tp::CallPoses* p = nullptr;
    std::mutex busy;
    void* bins = nullptr;  // pose-bin workspace of the tiled 3D kernels, grown on demand
    size_t bins_cap = 0;
    // A graph captured on the stream keeps the address of the workspace its calls used, so a
    // workspace that a capture has used is never freed: growing it retires it instead (kept
    // until the process ends; growth is geometric, so these stay a small multiple of the last).
    bool bins_captured = false;
    std::vector<void*> bins_retired;
    // The rotation forward kernels' lists of work items in reach (tp::TileSpec::flist) of the
    // last few geometries; a list that a capture has used is retired in the same way.
    struct ForwList {
        std::vector<int64_t> key;
        int* p = nullptr;
        size_t cap = 0;
        int64_t count = 0;
        bool captured = false;
        uint64_t used = 0;
    };
    ForwList flists[4];
    uint64_t flist_tick = 0;
    std::vector<void*> flist_retired;
};
std::mutex g_scratch_mu;
std::map<std::pair<int, hipStream_t>, std::unique_ptr<StreamScratch>> g_scratch;

// Scratch of tp_project_3d_to_2d_forw_noalloc: the static array `scratch`
// below, one copy per GPU.  Its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and kept in g_noalloc; the
// array's name itself is a host-side stand-in and is never passed to a kernel.
// The calls on one GPU share it: the pose pre-pass of each call rewrites
// every field the kernels read (the flags and the work counters), and calls
// that overlap on the GPU (different streams, no order between them) race.
constexpr int kNoAllocMaxDevices = 64;
constexpr size_t kCallScratchNeed = sizeof(tp::CallPoses);  // the same for every call and input size
struct NoAllocDevice {
    tp::CallPoses* p = nullptr;  // device address of this GPU's `scratch`
    std::mutex busy;             // held while a call enqueues its kernels
};
NoAllocDevice g_noalloc[kNoAllocMaxDevices];
std::mutex g_noalloc_init;

}  // namespace

static __device__ __align__(256) unsigned char scratch[TP_NOALLOC_SCRATCH_BYTES];

namespace {

// The current device's entry of g_noalloc, resolving its address on the first call on that device.
int noalloc_device(NoAllocDevice*& out) {
    if (kCallScratchNeed > TP_NOALLOC_SCRATCH_BYTES)
        return fail("the call needs " + std::to_string(kCallScratchNeed) + " bytes of scratch, more than the " +
                    std::to_string(TP_NOALLOC_SCRATCH_BYTES) + " of the static array");
    int dev = 0;
    TP_TRY(launched(hipGetDevice(&dev), "hipGetDevice"));
    if (dev < 0 || dev >= kNoAllocMaxDevices)
        return fail("the no-allocation entry point supports device indices below " +
                    std::to_string(kNoAllocMaxDevices));
    NoAllocDevice& d = g_noalloc[dev];
    {
        std::lock_guard<std::mutex> lk(g_noalloc_init);
        if (!d.p) {
            void* ptr = nullptr;
            TP_TRY(launched(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
            if (!ptr) return fail("hipGetSymbolAddress(scratch) returned NULL");
            d.p = static_cast<tp::CallPoses*>(ptr);
        }
    }
    out = &d;
    return TP_OK;
}

// The scratch of one call, taken on first use (after the argument checks) and
// held until the call returns, with the `busy` lock of its area.  `static_area`:
// the current GPU's static array (no allocation); otherwise the area of the
// (device, stream), allocated by the first call on that stream.
struct CallScratch {
    tp::CallPoses* p = nullptr;
    std::unique_lock<std::mutex> hold;
    bool static_area = false;
    StreamScratch* area = nullptr;  // the (device, stream) area, when not static_area
    // A pose-bin workspace of `need` bytes on the call's stream, or nullptr: the static area has
    // none, and a failed allocation leaves the call without bins (the kernels then cull every pose).
    // Growing waits for the stream's queued work, which may still read the old workspace; a stream
    // under graph capture can neither wait nor allocate, so there the call goes without bins, and
    // a workspace that a captured call uses is retired rather than freed when it grows later.
    void* bins(size_t need, hipStream_t st) {
        if (static_area || !area) return nullptr;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        const bool capturing = cs != hipStreamCaptureStatusNone;
        if (need > area->bins_cap) {
            if (capturing) return nullptr;
            if (hipStreamSynchronize(st) != hipSuccess) return nullptr;
            if (area->bins) {
                if (area->bins_captured) area->bins_retired.push_back(area->bins);
                else (void)hipFree(area->bins);
            }
            area->bins_captured = false;
            area->bins = nullptr;
            area->bins_cap = 0;
            const size_t cap = need + need / 4;
            if (hipMalloc(&area->bins, cap) != hipSuccess) {
                area->bins = nullptr;
                (void)hipGetLastError();  // clear the allocation error
                return nullptr;
            }
            area->bins_cap = cap;
        }
        if (capturing) area->bins_captured = true;
        return area->bins;
    }
    // The rotation forward kernels' list of work items in reach for the geometry of g and ts
    // (tp::forw_reach_items), or nullptr (the kernels then take every work item of their grid).
    // The area keeps the lists of its last four geometries; another geometry is listed on the host
    // and copied in on the call's stream, which is then synchronised (once per new geometry). A
    // stream under graph capture takes a list that the area holds for its geometry, else none, and
    // a list that a capture has used is retired, never rewritten or freed.
    const int* forw_list(const tp::Geom& g, const tp::TileSpec& ts, hipStream_t st, int64_t& count) {
        if (static_area || !area) return nullptr;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        const bool capturing = cs != hipStreamCaptureStatusNone;
        uint32_t rho_bits = 0, eps_bits = 0;
        std::memcpy(&rho_bits, &ts.rho_unit, 4);
        std::memcpy(&eps_bits, &ts.eps, 4);
        // everything the list depends on (the pose count only through fksplit)
        const std::vector<int64_t> key{g.B, ts.nt, ts.org, ts.ntfd, ts.orgd, ts.fc0, ts.fc1, ts.fd0, ts.fd1,
                                       ts.fksplit, int64_t(rho_bits), int64_t(eps_bits)};
        StreamScratch::ForwList* victim = nullptr;
        for (StreamScratch::ForwList& f : area->flists) {
            if (f.p && f.key == key) {
                f.used = ++area->flist_tick;
                if (capturing) f.captured = true;
                count = f.count;
                return f.p;
            }
            if (!victim || (victim->p && (!f.p || f.used < victim->used))) victim = &f;
        }
        if (capturing) return nullptr;
        std::vector<int> host;
        const int64_t items = tp::forw_reach_items(g, ts, host);
        if (items > int64_t(INT32_MAX) || host.empty()) return nullptr;
        const size_t need = host.size() * sizeof(int);
        // queued work may still read the list that is replaced
        if (hipStreamSynchronize(st) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        StreamScratch::ForwList& f = *victim;
        f.key.clear();
        if (f.p && (f.captured || need > f.cap)) {
            if (f.captured) area->flist_retired.push_back(f.p);
            else (void)hipFree(f.p);
            f.p = nullptr;
            f.cap = 0;
            f.captured = false;
        }
        if (!f.p) {
            const size_t cap = need + need / 4;
            if (hipMalloc(reinterpret_cast<void**>(&f.p), cap) != hipSuccess) {
                f.p = nullptr;
                (void)hipGetLastError();
                return nullptr;
            }
            f.cap = cap;
        }
        if (hipMemcpyAsync(f.p, host.data(), need, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        f.key = key;
        f.count = int64_t(host.size());
        f.used = ++area->flist_tick;
        count = f.count;
        return f.p;
    }
    int get(hipStream_t st) {
        if (p) return TP_OK;
        if (static_area) {
            NoAllocDevice* d = nullptr;
            TP_TRY(noalloc_device(d));
            hold = std::unique_lock<std::mutex>(d->busy);
            p = d->p;
            return TP_OK;
        }
        int dev = 0;
        TP_TRY(launched(hipGetDevice(&dev), "hipGetDevice"));
        StreamScratch* e;
        {
            std::lock_guard<std::mutex> lk(g_scratch_mu);
            std::unique_ptr<StreamScratch>& slot = g_scratch[{dev, st}];
            if (!slot) {
                // the area is allocated by the first call on the stream, which cannot happen under
                // graph capture
                hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
                TP_TRY(launched(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing"));
                if (cs != hipStreamCaptureStatusNone) {
                    g_scratch.erase({dev, st});
                    return fail("the first call on a stream allocates its scratch, which graph capture forbids: "
                                "call once on that stream before capturing, or use "
                                "tp_project_3d_to_2d_forw_noalloc");
                }
                std::unique_ptr<StreamScratch> fresh(new StreamScratch);
                TP_TRY(launched(hipMalloc(reinterpret_cast<void**>(&fresh->p), tp::kCallScratchBytes),
                                "scratch allocation"));
                slot = std::move(fresh);
            }
            e = slot.get();
        }
        hold = std::unique_lock<std::mutex>(e->busy);
        p = e->p;
        area = e;
        return TP_OK;
    }
};

// Summary of the call's poses for its tiled kernels (tp::launch_call_poses), which also clears the
// counts of the pose bins that plan_bins laid out in ts (if any).
int call_poses(int dim, const tp::Geom& g, const void* rot, float rho_unit, CallScratch& sc, hipStream_t s,
               const tp::TileSpec* ts = nullptr) {
    TP_TRY(sc.get(s));
    int* zero = ts && ts->sbins.list ? ts->sbins.count : nullptr;
    const int64_t nzero = zero ? g.B_rot * int64_t(ts->sbins.n) : 0;
    return launched(tp::launch_call_poses(dim, g.B_rot * g.P, rot, rho_unit, sc.p, s, zero, nzero),
                    "pose summary launch");
}

// Pose bins of the tiled 3D scatter's tile grid for this call (tp::BinGrid), in 2 x 2 x 2 tiles:
// plan_bins lays them out in the stream's workspace (ts.sbins; the pose summary then clears their
// counts) and fill_bins fills them after the summary.  None below kBinsMinPoses poses, from 65536
// poses (list entries are 16-bit), beyond kBinsMaxBytes or tp::kBinMaxGroups workgroups of the
// pre-pass, and none without a workspace: the scatter then culls every pose of each tile.
constexpr int64_t kBinsMinPoses = 16;
constexpr size_t kBinsMaxBytes = size_t(1) << 30;
int plan_bins(const tp::Geom& g, tp::TileSpec& ts, CallScratch& sc, hipStream_t s) {
    ts.sbins = tp::BinGrid{};
    TP_TRY(sc.get(s));
    if (g.P < kBinsMinPoses || g.P >= 65536) return TP_OK;
    tp::BinGrid sb{};
    sb.nb[0] = (ts.ntc + 1) / 2;
    sb.nb[1] = (ts.ntr + 1) / 2;
    sb.nb[2] = (ts.ntd + 1) / 2;
    sb.n = sb.nb[0] * sb.nb[1] * sb.nb[2];
    auto align = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t cells = size_t(g.B_rot) * size_t(sb.n);
    const size_t counts = align(cells * sizeof(int)), lists = align(cells * size_t(g.P) * sizeof(unsigned short));
    if (counts + lists > kBinsMaxBytes) return TP_OK;
    if (g.B_rot * int64_t(sb.nb[1]) * sb.nb[2] * ((g.P + tp::kBinPoses - 1) / tp::kBinPoses) > tp::kBinMaxGroups)
        return TP_OK;
    char* w = static_cast<char*>(sc.bins(counts + lists, s));
    if (!w) return TP_OK;
    sb.count = reinterpret_cast<int*>(w);
    sb.list = reinterpret_cast<unsigned short*>(w + counts);
    ts.sbins = sb;
    return TP_OK;
}
// The bins' pre-pass, which also zeroes the core tiles' cells of dst and wdst (dst null: not; the
// scatter then zeroes them itself).
int fill_bins(bool cubic, const tp::Geom& g, tp::TileSpec& ts, const void* rot, void* dst, void* wdst,
              CallScratch& sc, hipStream_t s) {
    ts.core_zeroed = false;
    if (!ts.sbins.list) return TP_OK;
    // a bin's box holds its tiles' box-1 boxes (the tile dilated by the stencil and the slack) with
    // half a voxel to spare
    const float half = float(g.N / 2), pad = 0.5f;
    const float sl = cubic ? 2.f : 1.f, sh = cubic ? 1.f : 0.f;
    const tp::BinBox bb{{0.f, -half + 1.f, -half + 1.f},
                        {2.f * tp::kScTC, 2.f * tp::kScTR, 2.f * tp::kScTD},
                        sl + ts.eps + pad, sh + ts.eps + pad, ts.rho_unit + 1.0f};
    TP_TRY(launched(tp::launch_pose_bins(g, rot, ts.sbins, bb, sc.p, s, ts, dst, wdst), "pose-bin launch"));
    ts.core_zeroed = dst != nullptr;
    return TP_OK;
}

// The rotation forward kernels' work items in reach (tp::TileSpec::flist), when the call's
// (device, stream) area can hold them.
int use_forw_list(const tp::Geom& g, tp::TileSpec& ts, CallScratch& sc, hipStream_t s) {
    TP_TRY(sc.get(s));
    int64_t count = 0;
    ts.flist = sc.forw_list(g, ts, s, count);
    ts.fcount = ts.flist ? count : 0;
    return TP_OK;
}

// TP_F16S: the volume is stored as complex half; it is widened exactly to
// fp32 on load and everything else (poses, arithmetic, projections) is the
// TP_F32 path.
int project_forw(int dim, int dtype, const void* rec, int64_t B, int64_t D, int64_t N, int64_t H, const void* rot,
                 int64_t B_rot, int64_t P, const void* shifts, int64_t B_shift, int64_t n, int interp, double os,
                 int has_cut, double cut, void* out, void* stream, CallScratch& sc) {
    const bool rec_half = dtype == TP_F16S;
    const int dt = rec_half ? TP_F32 : dtype;  // arithmetic and output type
    const int kdt = rec_half ? 2 : dt;         // per-pixel kernels' volume type
    tp::Geom g{};
    if (dtype != TP_F32 && dtype != TP_F64 && !rec_half)
        return fail("dtype must be TP_F32, TP_F64 or (forward projections) TP_F16S");
    TP_TRY(check_common(dt, interp, B, P, B_rot, shifts, B_shift, g));
    if (dim == 3 && D != N) return fail("reconstruction depth must equal its height");
    TP_TRY(set_rec(dim, N, H, g));
    TP_TRY(set_proj(n, g));
    set_cut(dt, has_cut, cut, g);
    g.os = os;
    if (g.work == 0) return TP_OK;
    TP_TRY(need(rec, "reconstruction"));
    TP_TRY(need(rot, "rotations"));
    TP_TRY(need(out, "projections"));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool cubic = interp == TP_CUBIC;
    if (use_tiles(dim, dt, os, n)) {
        tp::TileSpec ts = tile_spec(g, cubic, forw_poses_per_range(os));
        TP_TRY(call_poses(3, g, rot, ts.rho_unit, sc, s));
        TP_TRY(use_forw_list(g, ts, sc, s));
        TP_TRY(launched(tp::launch_project3_forw_tiled(cubic, g, ts, rec, rot, shifts, out, sc.p, 0, s, rec_half),
                        "tiled projection launch"));
        return launched(tp::launch_project_forw(dim, kdt, cubic, g, rec, rot, shifts, out, s, true),
                        "projection launch");
    }
    if (use_tiles2(dim, dt, os, n)) {
        // zero-fill first: the tiled gather writes the active pixels of tiled poses, the
        // rest kernel the other poses
        TP_TRY(zero(out, cx_words(dt, g.B * g.P * int64_t(g.npix)), s));
        const tp::TileSpec2 ts = tile_spec2(g, cubic);
        TP_TRY(call_poses(2, g, rot, ts.rho_unit, sc, s));
        TP_TRY(launched(tp::launch_gather2_tiled(cubic, 0, g, ts, rec, nullptr, rot, shifts, out, nullptr, nullptr,
                                                 nullptr, nullptr, sc.p, 0, s, rec_half),
                        "tiled projection launch"));
        return launched(tp::launch_project_forw(dim, kdt, cubic, g, rec, rot, shifts, out, s, true),
                        "projection launch");
    }
    return launched(tp::launch_project_forw(dim, kdt, cubic, g, rec, rot, shifts, out, s), "projection launch");
}

int project_back(int dim, int dtype, const void* gproj, int64_t B, int64_t P, int64_t n, int64_t hp, const void* rec,
                 int64_t D, int64_t N, int64_t H, const void* rot, int64_t B_rot, const void* shifts,
                 int64_t B_shift, int interp, double os, int has_cut, double cut, void* grec, void* grot,
                 void* gshift, void* stream) {
    // TP_F16S: the reconstruction is stored as complex half, widened exactly to fp32 on load;
    // everything else (gradients of projections, poses and shifts, the outputs) is the TP_F32 path
    const bool rec_half = dtype == TP_F16S;
    if (dtype != TP_F32 && dtype != TP_F64 && !rec_half)
        return fail("dtype must be TP_F32, TP_F64 or (a complex-half reconstruction) TP_F16S");
    if (rec_half) dtype = TP_F32;
    tp::Geom g{};
    TP_TRY(check_common(dtype, interp, B, P, B_rot, shifts, B_shift, g));
    if (dim == 3 && D != N) return fail("reconstruction depth must equal its height");
    if (hp != n / 2 + 1) return fail("grad_projections last dimension must be boxsize/2+1");
    if (gshift && !shifts) return fail("grad_shifts requested without shifts");
    TP_TRY(set_rec(dim, N, H, g));
    TP_TRY(set_proj(n, g));
    set_cut(dtype, has_cut, cut, g);
    g.os = os;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool cubic = interp == TP_CUBIC;
    const bool tiles = use_tiles(dim, dtype, os, n) && g.work > 0;
    const bool tiles2 = use_tiles2(dim, dtype, os, n) && g.work > 0;
    if (g.B > 0) TP_TRY(need(grec, "grad_reconstruction"));
    if (!tiles) TP_TRY(zero(grec, cx_words(dtype, g.B * g.vol), s));
    TP_TRY(zero(grot, re_words(dtype, g.B_rot * g.P * dim * dim), s));
    TP_TRY(zero(gshift, re_words(dtype, g.B_shift * g.P * 2), s));
    if (g.work == 0) return TP_OK;
    TP_TRY(need(gproj, "grad_projections"));
    TP_TRY(need(rec, "reconstruction"));
    TP_TRY(need(rot, "rotations"));
    CallScratch sc;
    if (tiles) {
        tp::TileSpec ts = tile_spec(g, cubic);
        TP_TRY(plan_bins(g, ts, sc, s));
        TP_TRY(call_poses(3, g, rot, ts.rho_unit, sc, s, &ts));
        TP_TRY(fill_bins(cubic, g, ts, rot, grec, nullptr, sc, s));
        TP_TRY(use_forw_list(g, ts, sc, s));
        TP_TRY(launched(tp::launch_scatter3_tiled(cubic, 1, g, ts, gproj, nullptr, rot, shifts, grec, nullptr, sc.p, 0,
                                                  s),
                        "tiled reconstruction-gradient launch"));
        TP_TRY(launched(tp::launch_grads3_tiled(cubic, g, ts, gproj, rec, rot, shifts, grot, gshift, sc.p, 1, s,
                                                rec_half),
                        "tiled rotation/shift-gradient launch"));
    }
    if (tiles2) {
        const tp::TileSpec2 ts = tile_spec2(g, cubic);
        TP_TRY(call_poses(2, g, rot, ts.rho_unit, sc, s));
        TP_TRY(launched(tp::launch_scatter2_tiled(cubic, 1, g, ts, gproj, nullptr, rot, shifts, grec, nullptr, sc.p, 0,
                                                  s),
                        "tiled reconstruction-gradient launch"));
        TP_TRY(launched(tp::launch_gather2_tiled(cubic, 1, g, ts, rec, nullptr, rot, shifts, nullptr, nullptr, gproj,
                                                 grot, gshift, sc.p, 1, s, rec_half),
                        "tiled rotation/shift-gradient launch"));
    }
    return launched(tp::launch_project_back(dim, rec_half ? 2 : dtype, cubic, g, gproj, rec, rot, shifts, grec, grot,
                                            gshift, s, (tiles || tiles2) ? 1 : 0),
                    "projection backward launch");
}

int backproject_forw(int dim, int dtype, const void* proj, int64_t B, int64_t P, int64_t n, int64_t hp,
                     const void* weights, const void* rot, int64_t B_rot, const void* shifts, int64_t B_shift,
                     int interp, double os, int has_cut, double cut, void* data, void* wrec, void* stream) {
    tp::Geom g{};
    TP_TRY(check_common(dtype, interp, B, P, B_rot, shifts, B_shift, g));
    if (hp != n / 2 + 1) return fail("projections last dimension must be boxsize/2+1");
    // with no samples (B * P == 0) an empty weights array may come as NULL; its volume is still zeroed
    if ((weights == nullptr) != (wrec == nullptr) && !(weights == nullptr && B * P == 0))
        return fail("weight_reconstruction must be given exactly when weights are");
    const int64_t N = rec_box(n, os);
    TP_TRY(set_rec(dim, N, N / 2 + 1, g));
    TP_TRY(set_proj(n, g));
    set_cut(dtype, has_cut, cut, g);
    g.os = os;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool cubic = interp == TP_CUBIC;
    const bool tiles = use_tiles(dim, dtype, os, n) && g.work > 0;
    const bool tiles2 = use_tiles2(dim, dtype, os, n) && g.work > 0;
    if (g.B > 0) TP_TRY(need(data, "data_reconstruction"));
    if (!tiles) {
        TP_TRY(zero(data, cx_words(dtype, g.B * g.vol), s));
        TP_TRY(zero(wrec, re_words(dtype, g.B * g.vol), s));
    }
    if (g.work == 0) return TP_OK;
    TP_TRY(need(proj, "projections"));
    TP_TRY(need(rot, "rotations"));
    CallScratch sc;
    if (tiles) {
        tp::TileSpec ts = tile_spec(g, cubic);
        backprojection_ranges(g, ts);
        TP_TRY(plan_bins(g, ts, sc, s));
        TP_TRY(call_poses(3, g, rot, ts.rho_unit, sc, s, &ts));
        TP_TRY(fill_bins(cubic, g, ts, rot, data, weights ? wrec : nullptr, sc, s));
        TP_TRY(launched(tp::launch_scatter3_tiled(cubic, 0, g, ts, proj, weights, rot, shifts, data, wrec, sc.p, 0, s),
                        "tiled backprojection launch"));
    }
    if (tiles2) {
        const tp::TileSpec2 ts = tile_spec2(g, cubic);
        TP_TRY(call_poses(2, g, rot, ts.rho_unit, sc, s));
        TP_TRY(launched(tp::launch_scatter2_tiled(cubic, 0, g, ts, proj, weights, rot, shifts, data, wrec, sc.p, 0, s),
                        "tiled backprojection launch"));
    }
    return launched(
        tp::launch_backproject_forw(dim, dtype, cubic, g, proj, weights, rot, shifts, data, wrec, s, tiles || tiles2),
        "backprojection launch");
}

int backproject_back(int dim, int dtype, const void* gdata, const void* gw, int64_t N, int64_t H, const void* proj,
                     int64_t B, int64_t P, int64_t n, int64_t hp, const void* weights, const void* rot,
                     int64_t B_rot, const void* shifts, int64_t B_shift, int interp, double os, int has_cut,
                     double cut, void* gproj, void* gweights, void* grot, void* gshift, void* stream) {
    tp::Geom g{};
    TP_TRY(check_common(dtype, interp, B, P, B_rot, shifts, B_shift, g));
    if (hp != n / 2 + 1) return fail("projections last dimension must be boxsize/2+1");
    if (gweights && !weights) return fail("grad_weights requested without weights");
    if (gshift && !shifts) return fail("grad_shifts requested without shifts");
    TP_TRY(set_rec(dim, N, H, g));
    TP_TRY(set_proj(n, g));
    set_cut(dtype, has_cut, cut, g);
    g.os = os;
    hipStream_t s = static_cast<hipStream_t>(stream);
    TP_TRY(zero(grot, re_words(dtype, g.B_rot * g.P * dim * dim), s));
    TP_TRY(zero(gshift, re_words(dtype, g.B_shift * g.P * 2), s));
    if (g.work == 0) return TP_OK;
    TP_TRY(need(gdata, "grad_data_rec"));
    TP_TRY(need(proj, "projections"));
    TP_TRY(need(rot, "rotations"));
    TP_TRY(need(gproj, "grad_projections"));
    const bool cubic = interp == TP_CUBIC;
    const bool tiles2 = use_tiles2(dim, dtype, os, n);
    const bool tiles = use_tiles(dim, dtype, os, n);
    if (tiles2 || tiles) {
        // the tiled gathers write the active pixels of tiled poses, the per-pixel kernel the rest
        TP_TRY(zero(gproj, cx_words(dtype, g.B * g.P * int64_t(g.npix)), s));
        TP_TRY(zero(gweights, re_words(dtype, g.B * g.P * int64_t(g.npix)), s));
    }
    CallScratch sc;
    if (tiles) {
        tp::TileSpec ts = tile_spec(g, cubic);
        TP_TRY(call_poses(3, g, rot, ts.rho_unit, sc, s));
        TP_TRY(use_forw_list(g, ts, sc, s));
        TP_TRY(launched(tp::launch_bpback3_tiled(cubic, g, ts, gdata, gw, proj, rot, shifts, gproj, gweights, grot,
                                                 gshift, sc.p, 0, s),
                        "tiled backprojection backward launch"));
    }
    if (tiles2) {
        const tp::TileSpec2 ts = tile_spec2(g, cubic);
        TP_TRY(call_poses(2, g, rot, ts.rho_unit, sc, s));
        TP_TRY(launched(tp::launch_gather2_tiled(cubic, 2, g, ts, gdata, gw, rot, shifts, gproj,
                                                 (gw && gweights) ? gweights : nullptr, proj, grot, gshift, sc.p, 0, s),
                        "tiled backprojection backward launch"));
    }
    return launched(tp::launch_backproject_back(dim, dtype, cubic, g, gdata, gw, proj, rot, shifts, gproj, gweights,
                                                grot, gshift, s, tiles2 || tiles),
                    "backprojection backward launch");
}

}  // namespace

extern "C" {

const char* tp_last_error(void) { return g_err.c_str(); }

int tp_abi_version(void) { return 1; }

int64_t tp_backproject_rec_boxsize(int64_t proj_boxsize, double oversampling) {
    return rec_box(proj_boxsize, oversampling);
}

int tp_project_2d_forw(int dtype, const void* reconstruction, int64_t B, int64_t rec_boxsize,
                       int64_t rec_boxsize_half, const void* rotations, int64_t B_rot, int64_t P, const void* shifts,
                       int64_t B_shift, int64_t proj_boxsize, int interpolation, double oversampling, int has_cutoff,
                       double fourier_radius_cutoff, void* projections, void* stream) {
    g_err.clear();
    CallScratch sc;
    return project_forw(2, dtype, reconstruction, B, rec_boxsize, rec_boxsize, rec_boxsize_half, rotations, B_rot, P,
                        shifts, B_shift, proj_boxsize, interpolation, oversampling, has_cutoff,
                        fourier_radius_cutoff, projections, stream, sc);
}

int tp_project_3d_to_2d_forw(int dtype, const void* reconstruction, int64_t B, int64_t rec_depth,
                             int64_t rec_boxsize, int64_t rec_boxsize_half, const void* rotations, int64_t B_rot,
                             int64_t P, const void* shifts, int64_t B_shift, int64_t proj_boxsize, int interpolation,
                             double oversampling, int has_cutoff, double fourier_radius_cutoff, void* projections,
                             void* stream) {
    g_err.clear();
    CallScratch sc;
    return project_forw(3, dtype, reconstruction, B, rec_depth, rec_boxsize, rec_boxsize_half, rotations, B_rot, P,
                        shifts, B_shift, proj_boxsize, interpolation, oversampling, has_cutoff,
                        fourier_radius_cutoff, projections, stream, sc);
}

int tp_project_3d_to_2d_forw_noalloc(int dtype, const void* reconstruction, int64_t B, int64_t rec_depth,
                                     int64_t rec_boxsize, int64_t rec_boxsize_half, const void* rotations,
                                     int64_t B_rot, int64_t P, const void* shifts, int64_t B_shift,
                                     int64_t proj_boxsize, int interpolation, double oversampling, int has_cutoff,
                                     double fourier_radius_cutoff, void* projections, void* stream) {
    g_err.clear();
    CallScratch sc;
    sc.static_area = true;
    return project_forw(3, dtype, reconstruction, B, rec_depth, rec_boxsize, rec_boxsize_half, rotations, B_rot, P,
                        shifts, B_shift, proj_boxsize, interpolation, oversampling, has_cutoff,
                        fourier_radius_cutoff, projections, stream, sc);
}

int tp_project_2d_back(int dtype, const void* grad_projections, int64_t B, int64_t P, int64_t proj_boxsize,
                       int64_t proj_boxsize_half, const void* reconstruction, int64_t rec_boxsize,
                       int64_t rec_boxsize_half, const void* rotations, int64_t B_rot, const void* shifts,
                       int64_t B_shift, int interpolation, double oversampling, int has_cutoff,
                       double fourier_radius_cutoff, void* grad_reconstruction, void* grad_rotations,
                       void* grad_shifts, void* stream) {
    g_err.clear();
    return project_back(2, dtype, grad_projections, B, P, proj_boxsize, proj_boxsize_half, reconstruction,
                        rec_boxsize, rec_boxsize, rec_boxsize_half, rotations, B_rot, shifts, B_shift, interpolation,
                        oversampling, has_cutoff, fourier_radius_cutoff, grad_reconstruction, grad_rotations,
                        grad_shifts, stream);
}

int tp_project_3d_to_2d_back(int dtype, const void* grad_projections, int64_t B, int64_t P, int64_t proj_boxsize,
                             int64_t proj_boxsize_half, const void* reconstruction, int64_t rec_depth,
                             int64_t rec_boxsize, int64_t rec_boxsize_half, const void* rotations, int64_t B_rot,
                             const void* shifts, int64_t B_shift, int interpolation, double oversampling,
                             int has_cutoff, double fourier_radius_cutoff, void* grad_reconstruction,
                             void* grad_rotations, void* grad_shifts, void* stream) {
    g_err.clear();
    return project_back(3, dtype, grad_projections, B, P, proj_boxsize, proj_boxsize_half, reconstruction, rec_depth,
                        rec_boxsize, rec_boxsize_half, rotations, B_rot, shifts, B_shift, interpolation,
                        oversampling, has_cutoff, fourier_radius_cutoff, grad_reconstruction, grad_rotations,
                        grad_shifts, stream);
}

int tp_backproject_2d_forw(int dtype, const void* projections, int64_t B, int64_t P, int64_t proj_boxsize,
                           int64_t proj_boxsize_half, const void* weights, const void* rotations, int64_t B_rot,
                           const void* shifts, int64_t B_shift, int interpolation, double oversampling,
                           int has_cutoff, double fourier_radius_cutoff, void* data_reconstruction,
                           void* weight_reconstruction, void* stream) {
    g_err.clear();
    return backproject_forw(2, dtype, projections, B, P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot,
                            shifts, B_shift, interpolation, oversampling, has_cutoff, fourier_radius_cutoff,
                            data_reconstruction, weight_reconstruction, stream);
}

int tp_backproject_2d_to_3d_forw(int dtype, const void* projections, int64_t B, int64_t P, int64_t proj_boxsize,
                                 int64_t proj_boxsize_half, const void* weights, const void* rotations,
                                 int64_t B_rot, const void* shifts, int64_t B_shift, int interpolation,
                                 double oversampling, int has_cutoff, double fourier_radius_cutoff,
                                 void* data_reconstruction, void* weight_reconstruction, void* stream) {
    g_err.clear();
    return backproject_forw(3, dtype, projections, B, P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot,
                            shifts, B_shift, interpolation, oversampling, has_cutoff, fourier_radius_cutoff,
                            data_reconstruction, weight_reconstruction, stream);
}

int tp_backproject_2d_back(int dtype, const void* grad_data_rec, const void* grad_weight_rec, int64_t rec_boxsize,
                           int64_t rec_boxsize_half, const void* projections, int64_t B, int64_t P,
                           int64_t proj_boxsize, int64_t proj_boxsize_half, const void* weights,
                           const void* rotations, int64_t B_rot, const void* shifts, int64_t B_shift,
                           int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                           void* grad_projections, void* grad_weights, void* grad_rotations, void* grad_shifts,
                           void* stream) {
    g_err.clear();
    return backproject_back(2, dtype, grad_data_rec, grad_weight_rec, rec_boxsize, rec_boxsize_half, projections, B,
                            P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot, shifts, B_shift,
                            interpolation, oversampling, has_cutoff, fourier_radius_cutoff, grad_projections,
                            grad_weights, grad_rotations, grad_shifts, stream);
}

int tp_backproject_2d_to_3d_back(int dtype, const void* grad_data_rec, const void* grad_weight_rec,
                                 int64_t rec_boxsize, int64_t rec_boxsize_half, const void* projections, int64_t B,
                                 int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half, const void* weights,
                                 const void* rotations, int64_t B_rot, const void* shifts, int64_t B_shift,
                                 int interpolation, double oversampling, int has_cutoff,
                                 double fourier_radius_cutoff, void* grad_projections, void* grad_weights,
                                 void* grad_rotations, void* grad_shifts, void* stream) {
    g_err.clear();
    return backproject_back(3, dtype, grad_data_rec, grad_weight_rec, rec_boxsize, rec_boxsize_half, projections, B,
                            P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot, shifts, B_shift,
                            interpolation, oversampling, has_cutoff, fourier_radius_cutoff, grad_projections,
                            grad_weights, grad_rotations, grad_shifts, stream);
}

/* ---------------------------------------------------------------- reference preparation */

int64_t tp_padded_boxsize(int64_t boxsize, double oversampling) {
    const int64_t raw = static_cast<int64_t>(double(boxsize) * oversampling);
    return raw + (raw % 2);
}

int64_t tp_cropped_boxsize(int64_t boxsize, double oversampling) {
    return static_cast<int64_t>(double(boxsize) / oversampling);
}

int tp_fftshift_pad(int elem_bytes, const void* src, int64_t batch, int dim, int64_t boxsize,
                    int64_t padded_boxsize, int64_t pad_before, void* dst, void* stream) {
    g_err.clear();
    if (elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8 && elem_bytes != 16)
        return fail("elem_bytes must be 2, 4, 8 or 16");
    if (dim != 2 && dim != 3) return fail("dim must be 2 or 3");
    if (batch < 0 || boxsize < 1) return fail("batch must be >= 0 and boxsize >= 1");
    if (padded_boxsize < boxsize || padded_boxsize > (int64_t(1) << 30))
        return fail("padded_boxsize must be in [boxsize, 2^30]");
    if (pad_before < 0 || pad_before > padded_boxsize - boxsize)
        return fail("pad_before must be in [0, padded_boxsize - boxsize]");
    if (batch == 0) return TP_OK;
    TP_TRY(need(src, "src"));
    TP_TRY(need(dst, "dst"));
    return launched(tp::launch_fftshift_pad(elem_bytes, dim, src, batch, boxsize, padded_boxsize, pad_before, dst,
                                            static_cast<hipStream_t>(stream)),
                    "fftshift-pad launch");
}

int tp_ifftshift_crop(int elem_bytes, const void* src, int64_t batch, int dim, int64_t len0, int64_t len1,
                      int64_t len2, int64_t crop_start, int64_t crop_len, void* dst, void* stream) {
    g_err.clear();
    if (elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8 && elem_bytes != 16)
        return fail("elem_bytes must be 2, 4, 8 or 16");
    if (dim != 2 && dim != 3) return fail("dim must be 2 or 3");
    const int64_t L[3] = {len0, len1, dim == 3 ? len2 : 1};
    if (batch < 0 || crop_start < 0 || crop_len < 0) return fail("batch, crop_start and crop_len must be >= 0");
    int64_t m[3] = {1, 1, 1};
    for (int a = 0; a < dim; ++a) {
        if (L[a] < 1 || L[a] > (int64_t(1) << 30)) return fail("axis lengths must be in [1, 2^30]");
        m[a] = std::max<int64_t>(0, std::min(crop_start + crop_len, L[a]) - crop_start);
    }
    if (batch == 0 || m[0] * m[1] * m[2] == 0) return TP_OK;
    TP_TRY(need(src, "src"));
    TP_TRY(need(dst, "dst"));
    return launched(tp::launch_ifftshift_crop(elem_bytes, dim, src, batch, L, m, crop_start, dst,
                                              static_cast<hipStream_t>(stream)),
                    "ifftshift-crop launch");
}

int tp_rfftn(int dtype, int dim, int64_t batch, int64_t boxsize, const void* real, void* spectrum, void* stream) {
    g_err.clear();
    if (dtype != TP_F32 && dtype != TP_F64) return fail("dtype must be TP_F32 or TP_F64");
    if (dim != 2 && dim != 3) return fail("dim must be 2 or 3");
    if (batch < 0 || batch > INT32_MAX || boxsize < 1 || boxsize > INT32_MAX)
        return fail("batch must be in [0, 2^31) and boxsize in [1, 2^31)");
    if (batch == 0) return TP_OK;
    TP_TRY(need(real, "real"));
    TP_TRY(need(spectrum, "spectrum"));
    const int r = tp::fft_forward(dtype, dim, batch, boxsize, real, spectrum, static_cast<hipStream_t>(stream));
    if (r == tp::kFftNoPlanUnderCapture)
        return fail("the first transform of this shape on a stream makes its hipFFT plan, which graph capture "
                    "forbids: run it once on that stream before capturing");
    if (r != 0) {
        g_err = "hipFFT forward transform failed (hipfftResult " + std::to_string(r) + ")";
        return TP_ERR_HIP;
    }
    return TP_OK;
}

int tp_irfftn(int dtype, int dim, int64_t batch, int64_t boxsize, void* spectrum, void* real, void* stream) {
    g_err.clear();
    if (dtype != TP_F32 && dtype != TP_F64) return fail("dtype must be TP_F32 or TP_F64");
    if (dim != 2 && dim != 3) return fail("dim must be 2 or 3");
    if (batch < 0 || batch > INT32_MAX || boxsize < 1 || boxsize > INT32_MAX)
        return fail("batch must be in [0, 2^31) and boxsize in [1, 2^31)");
    if (batch == 0) return TP_OK;
    TP_TRY(need(spectrum, "spectrum"));
    TP_TRY(need(real, "real"));
    const int r = tp::fft_inverse(dtype, dim, batch, boxsize, spectrum, real, static_cast<hipStream_t>(stream));
    if (r == tp::kFftNoPlanUnderCapture)
        return fail("the first transform of this shape on a stream makes its hipFFT plan, which graph capture "
                    "forbids: run it once on that stream before capturing");
    if (r != 0) {
        g_err = "hipFFT inverse transform failed (hipfftResult " + std::to_string(r) + ")";
        return TP_ERR_HIP;
    }
    return TP_OK;
}

int tp_normalize_reconstruction(int dtype, const void* data, const void* weights, int64_t elems, double reg,
                                void* out, void* stream) {
    g_err.clear();
    if (dtype != TP_F32 && dtype != TP_F64) return fail("dtype must be TP_F32 or TP_F64");
    if (elems < 0) return fail("elems must be >= 0");
    if (!std::isfinite(reg)) return fail("reg must be finite");
    if (elems == 0) return TP_OK;
    TP_TRY(need(data, "data"));
    TP_TRY(need(weights, "weights"));
    TP_TRY(need(out, "out"));
    return launched(tp::launch_normalize(dtype, data, weights, elems, reg, out, static_cast<hipStream_t>(stream)),
                    "normalisation launch");
}

}  // extern "C"
