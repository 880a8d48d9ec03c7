// Reference preparation around the projectors: the real-space padding and
// shifting before the forward FFT and after the inverse FFT, and the
// normalisation of a backprojected (data, weight) pair.
//
// The reference does these with PyTorch tensor ops in its helpers
// (tests/test_utils.py:174-247 pad_and_fftshift, :250-293 ifftshift_and_crop;
// README.md:106-143): F.pad, then torch.fft.fftshift (two full passes and an
// intermediate), and ifftshift followed by a slice.  Here each is one pass
// that computes every output element's source index directly:
//
//   k_fftshift_pad    dst = fftshift(zero-pad(src)) over the last DIM axes:
//                     dst[i] = src[((i + N - N/2) mod N) - pad_before] per axis
//                     (zero outside), a cube/square of edge n into edge N.
//   k_ifftshift_crop  dst = ifftshift(src)[crop_start : crop_start + len] per
//                     axis: dst[j] = src[(crop_start + j + L/2) mod L], with L
//                     each axis's own length.
//   k_normalize       out = data / (weight + reg) where weight + reg > 0,
//                     else 0 (component-wise division of the complex value).
//
// Elements are moved as opaque words of 2, 4, 8 or 16 bytes, so any real or
// complex dtype takes the same kernels; the pair of kernels are each other's
// adjoints (fftshift-pad with pad_before = crop_start undoes the crop).
#include <hipfft/hipfft.h>

#include <map>
#include <mutex>
#include <tuple>

#include "tp_device.hh"
#include "tp_launch.hh"

namespace tp {

namespace {

template <int BYTES> struct Word;
template <> struct Word<2> { using T = uint16_t; };
template <> struct Word<4> { using T = uint32_t; };
template <> struct Word<8> { using T = uint2; };
template <> struct Word<16> { using T = uint4; };

// v mod L for 0 <= v < 2L (every index here is an in-range position plus a shift below L).
__device__ __forceinline__ int64_t wrap(int64_t v, int64_t L) { return v >= L ? v - L : v; }
__device__ __forceinline__ int wrap32(int v, int L) { return v >= L ? v - L : v; }

// Rows (the last axis) are spread over threadIdx.y and blocks, the words of
// a row over threadIdx.x.  A word is V consecutive elements (16 bytes when the
// row geometry keeps V-element groups contiguous and aligned, else one
// element), so each group maps to one aligned group of the source row.
template <typename W, int V, int DIM>
__global__ __launch_bounds__(kBlock) void k_fftshift_pad(const W* __restrict__ src, W* __restrict__ dst, int64_t rows,
                                                         int64_t n, int64_t N, int64_t pb) {
    const int64_t sh = N - N / 2;  // fftshift: output i holds input (i + sh) mod N
    const int nw = int(N / V), n32 = int(n), N32 = int(N), sh32 = int(sh), pb32 = int(pb);
    for (int64_t row = int64_t(blockIdx.x) * blockDim.y + threadIdx.y; row < rows;
         row += int64_t(gridDim.x) * blockDim.y) {
        int64_t t = row;
        const int64_t y = t % N;
        t /= N;
        int64_t z = 0;
        if (DIM == 3) {
            z = t % N;
            t /= N;
        }
        const int64_t b = t;
        const int64_t sy = wrap(y + sh, N) - pb, sz = wrap(z + sh, N) - pb;
        const bool in_row = sy >= 0 && sy < n && (DIM == 2 || (sz >= 0 && sz < n));
        const W* s = src + (((b * (DIM == 3 ? n : 1) + (DIM == 3 ? sz : 0)) * n + sy) * n) / V;
        W* d = dst + row * nw;
        for (int w = threadIdx.x; w < nw; w += blockDim.x) {
            const int sx = wrap32(w * V + sh32, N32) - pb32;
            d[w] = (in_row && sx >= 0 && sx < n32) ? s[sx / V] : W{};
        }
    }
}

// The same layout for the crop.  Input axes have lengths L0 ([z] or y), L1,
// L2; the output keeps `m` of each, from crop_start.
template <typename W, int V, int DIM>
__global__ __launch_bounds__(kBlock) void k_ifftshift_crop(const W* __restrict__ src, W* __restrict__ dst,
                                                           int64_t rows, int64_t L0, int64_t L1, int64_t L2,
                                                           int64_t m0, int64_t m1, int64_t m2, int64_t cs) {
    // axes: 2D (y: L0, x: L1); 3D (z: L0, y: L1, x: L2)
    const int64_t Lx = DIM == 3 ? L2 : L1, mx = DIM == 3 ? m2 : m1;
    const int64_t Ly = DIM == 3 ? L1 : L0, my = DIM == 3 ? m1 : m0;
    const int base = int(cs + Lx / 2), Lx32 = int(Lx), mw = int(mx / V);
    for (int64_t row = int64_t(blockIdx.x) * blockDim.y + threadIdx.y; row < rows;
         row += int64_t(gridDim.x) * blockDim.y) {
        int64_t t = row;
        const int64_t y = t % my;
        t /= my;
        int64_t z = 0;
        if (DIM == 3) {
            z = t % m0;
            t /= m0;
        }
        const int64_t b = t;
        const int64_t sy = wrap(cs + y + Ly / 2, Ly);
        const int64_t sz = DIM == 3 ? wrap(cs + z + L0 / 2, L0) : 0;
        const W* s = src + (((b * (DIM == 3 ? L0 : 1) + sz) * Ly + sy) * Lx) / V;
        W* d = dst + row * mw;
        for (int w = threadIdx.x; w < mw; w += blockDim.x) d[w] = s[wrap32(base + w * V, Lx32) / V];
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_normalize(const Cx<T>* data, const T* __restrict__ w, int64_t elems,
                                                      T reg, Cx<T>* out) {  // out may alias data
    for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < elems; e += int64_t(gridDim.x) * kBlock) {
        const T den = w[e] + reg;
        const Cx<T> v = data[e];
        out[e] = den > T(0) ? Cx<T>{v.re / den, v.im / den} : Cx<T>{T(0), T(0)};
    }
}

// Block shape for rows of `words` words: x covers a row (a multiple of 64,
// at most kBlock), y stacks rows up to kBlock threads.
inline dim3 row_block(int64_t words) {
    int bx = 64;
    while (bx < words && bx < kBlock) bx *= 2;
    return dim3(unsigned(bx), unsigned(kBlock / bx));
}

inline bool aligned16(const void* a, const void* b) {
    return ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15u) == 0;
}

template <typename W, int V>
hipError_t pad_launch_w(int dim, const void* src, int64_t rows, int64_t n, int64_t N, int64_t pb, void* dst,
                        hipStream_t s) {
    const dim3 blk = row_block(N / V);
    const unsigned grid = grid_for((rows + blk.y - 1) / blk.y);
    if (dim == 3)
        hipLaunchKernelGGL((k_fftshift_pad<W, V, 3>), dim3(grid), blk, 0, s, (const W*)src, (W*)dst, rows, n, N, pb);
    else
        hipLaunchKernelGGL((k_fftshift_pad<W, V, 2>), dim3(grid), blk, 0, s, (const W*)src, (W*)dst, rows, n, N, pb);
    return hipGetLastError();
}

template <int BYTES>
hipError_t pad_launch(int dim, const void* src, int64_t batch, int64_t n, int64_t N, int64_t pb, void* dst,
                      hipStream_t s) {
    using E = typename Word<BYTES>::T;
    constexpr int V = 16 / BYTES;
    const int64_t rows = batch * N * (dim == 3 ? N : 1);
    if (rows == 0) return hipSuccess;
    // 16-byte words when every V-element group of a row maps to one aligned source group
    if (V > 1 && n % V == 0 && N % V == 0 && pb % V == 0 && (N - N / 2) % V == 0 && aligned16(src, dst))
        return pad_launch_w<uint4, V>(dim, src, rows, n, N, pb, dst, s);
    return pad_launch_w<E, 1>(dim, src, rows, n, N, pb, dst, s);
}

template <typename W, int V>
hipError_t crop_launch_w(int dim, const void* src, int64_t rows, const int64_t* L, const int64_t* m, int64_t cs,
                         void* dst, hipStream_t s) {
    const dim3 blk = row_block(m[dim - 1] / V);
    const unsigned grid = grid_for((rows + blk.y - 1) / blk.y);
    if (dim == 3)
        hipLaunchKernelGGL((k_ifftshift_crop<W, V, 3>), dim3(grid), blk, 0, s, (const W*)src, (W*)dst, rows, L[0],
                           L[1], L[2], m[0], m[1], m[2], cs);
    else
        hipLaunchKernelGGL((k_ifftshift_crop<W, V, 2>), dim3(grid), blk, 0, s, (const W*)src, (W*)dst, rows, L[0],
                           L[1], int64_t(1), m[0], m[1], int64_t(1), cs);
    return hipGetLastError();
}

template <int BYTES>
hipError_t crop_launch(int dim, const void* src, int64_t batch, const int64_t* L, const int64_t* m, int64_t cs,
                       void* dst, hipStream_t s) {
    using E = typename Word<BYTES>::T;
    constexpr int V = 16 / BYTES;
    const int64_t rows = batch * m[0] * (dim == 3 ? m[1] : 1);
    if (rows == 0 || m[dim - 1] == 0) return hipSuccess;
    const int64_t Lx = L[dim - 1], mx = m[dim - 1];
    if (V > 1 && Lx % V == 0 && mx % V == 0 && (cs + Lx / 2) % V == 0 && aligned16(src, dst))
        return crop_launch_w<uint4, V>(dim, src, rows, L, m, cs, dst, s);
    return crop_launch_w<E, 1>(dim, src, rows, L, m, cs, dst, s);
}

}  // namespace

hipError_t launch_fftshift_pad(int elem_bytes, int dim, const void* src, int64_t batch, int64_t n, int64_t N,
                               int64_t pad_before, void* dst, hipStream_t s) {
    switch (elem_bytes) {
        case 2: return pad_launch<2>(dim, src, batch, n, N, pad_before, dst, s);
        case 4: return pad_launch<4>(dim, src, batch, n, N, pad_before, dst, s);
        case 8: return pad_launch<8>(dim, src, batch, n, N, pad_before, dst, s);
        default: return pad_launch<16>(dim, src, batch, n, N, pad_before, dst, s);
    }
}

hipError_t launch_ifftshift_crop(int elem_bytes, int dim, const void* src, int64_t batch, const int64_t* L,
                                 const int64_t* m, int64_t crop_start, void* dst, hipStream_t s) {
    switch (elem_bytes) {
        case 2: return crop_launch<2>(dim, src, batch, L, m, crop_start, dst, s);
        case 4: return crop_launch<4>(dim, src, batch, L, m, crop_start, dst, s);
        case 8: return crop_launch<8>(dim, src, batch, L, m, crop_start, dst, s);
        default: return crop_launch<16>(dim, src, batch, L, m, crop_start, dst, s);
    }
}

// ---------------------------------------------------------------- FFTs (rocFFT through hipFFT)
// Plans are cached per (direction, dtype, dim, edge, batch, device, stream);
// hipFFT allocates each plan's work area once.  Keying on the stream gives
// calls on different streams their own work areas, so transforms that run at
// once on the GPU never share one; calls on one stream run in order.  The
// cache holds at most kMaxPlans plans: the least recently used one is
// destroyed once its last transform has finished (an event recorded after
// each transform; no device-wide synchronisation).  A plan that a graph
// capture used is never destroyed (the graph keeps its work area), and no
// plan is made on a capturing stream (that allocates): such a call fails with
// kFftNoPlanUnderCapture.  The cache lock serialises the enqueues.
namespace {

using PlanKey = std::tuple<int, int, int, int64_t, int64_t, int, hipStream_t>;
struct PlanEntry {
    hipfftHandle h;
    hipEvent_t done;  // recorded after each transform made outside a capture
    uint64_t used;    // tick of the last call
    bool captured;    // used by a call under graph capture: kept until the process ends
};
constexpr size_t kMaxPlans = 32;
std::mutex g_fft_mu;
std::map<PlanKey, PlanEntry> g_plans;
uint64_t g_fft_tick = 0;

hipfftResult evict_oldest_plan() {
    auto old = g_plans.end();
    for (auto it = g_plans.begin(); it != g_plans.end(); ++it)
        if (!it->second.captured && (old == g_plans.end() || it->second.used < old->second.used)) old = it;
    if (old == g_plans.end()) return HIPFFT_SUCCESS;  // every plan is held by a graph: the cache grows
    // its work area may still be in use by its last transform: wait for that one only
    if (hipEventSynchronize(old->second.done) != hipSuccess) return HIPFFT_INTERNAL_ERROR;
    const hipfftResult r = hipfftDestroy(old->second.h);
    (void)hipEventDestroy(old->second.done);
    g_plans.erase(old);
    return r;
}

// The cached plan for a transform on stream s (made on first use); `capturing` tells whether s is
// being captured into a graph.
int plan_for(bool forward, int dt, int dim, int64_t N, int64_t batch, hipStream_t s, PlanEntry*& out,
             bool& capturing) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return HIPFFT_INTERNAL_ERROR;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) return HIPFFT_INTERNAL_ERROR;
    capturing = cs != hipStreamCaptureStatusNone;
    const PlanKey key{forward ? 1 : 0, dt, dim, N, batch, dev, s};
    auto it = g_plans.find(key);
    if (it != g_plans.end()) {
        it->second.used = ++g_fft_tick;
        it->second.captured |= capturing;
        out = &it->second;
        return HIPFFT_SUCCESS;
    }
    if (capturing) return kFftNoPlanUnderCapture;
    if (g_plans.size() >= kMaxPlans) {
        const hipfftResult e = evict_oldest_plan();
        if (e != HIPFFT_SUCCESS) return e;
    }
    hipEvent_t ev;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return HIPFFT_ALLOC_FAILED;
    hipfftHandle h;
    hipfftResult r = hipfftCreate(&h);
    if (r != HIPFFT_SUCCESS) {
        (void)hipEventDestroy(ev);
        return r;
    }
    // norm="forward": the forward transform carries 1/N^dim, the inverse none
    double scale = 1.0;
    if (forward)
        for (int a = 0; a < dim; ++a) scale /= double(N);
    r = hipfftExtPlanScaleFactor(h, scale);
    int n[3] = {int(N), int(N), int(N)};
    const hipfftType type = forward ? (dt == 0 ? HIPFFT_R2C : HIPFFT_D2Z) : (dt == 0 ? HIPFFT_C2R : HIPFFT_Z2D);
    size_t work = 0;
    if (r == HIPFFT_SUCCESS)
        r = hipfftMakePlanMany(h, dim, n, nullptr, 1, 0, nullptr, 1, 0, type, int(batch), &work);
    if (r == HIPFFT_SUCCESS) r = hipfftSetStream(h, s);
    if (r != HIPFFT_SUCCESS) {
        hipfftDestroy(h);
        (void)hipEventDestroy(ev);
        return r;
    }
    out = &g_plans.emplace(key, PlanEntry{h, ev, ++g_fft_tick, false}).first->second;
    return HIPFFT_SUCCESS;
}

// After a transform: outside a capture, mark where its work area is free again.
int transformed(hipfftResult r, const PlanEntry& pe, bool capturing, hipStream_t s) {
    if (r != HIPFFT_SUCCESS || capturing) return int(r);
    return hipEventRecord(pe.done, s) == hipSuccess ? HIPFFT_SUCCESS : HIPFFT_EXEC_FAILED;
}

}  // namespace

int fft_forward(int dt, int dim, int64_t batch, int64_t N, const void* real, void* spec, hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_fft_mu);
    PlanEntry* pe = nullptr;
    bool capturing = false;
    const int r = plan_for(true, dt, dim, N, batch, s, pe, capturing);
    if (r != HIPFFT_SUCCESS) return r;
    // out-of-place real-to-complex transforms leave their input intact
    const hipfftResult e = dt == 0 ? hipfftExecR2C(pe->h, (hipfftReal*)real, (hipfftComplex*)spec)
                                   : hipfftExecD2Z(pe->h, (hipfftDoubleReal*)real, (hipfftDoubleComplex*)spec);
    return transformed(e, *pe, capturing, s);
}

int fft_inverse(int dt, int dim, int64_t batch, int64_t N, void* spec, void* real, hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_fft_mu);
    PlanEntry* pe = nullptr;
    bool capturing = false;
    const int r = plan_for(false, dt, dim, N, batch, s, pe, capturing);
    if (r != HIPFFT_SUCCESS) return r;
    const hipfftResult e = dt == 0 ? hipfftExecC2R(pe->h, (hipfftComplex*)spec, (hipfftReal*)real)
                                   : hipfftExecZ2D(pe->h, (hipfftDoubleComplex*)spec, (hipfftDoubleReal*)real);
    return transformed(e, *pe, capturing, s);
}

hipError_t launch_normalize(int dt, const void* data, const void* weights, int64_t elems, double reg, void* out,
                            hipStream_t s) {
    if (elems == 0) return hipSuccess;
    const unsigned grid = grid_for((elems + kBlock - 1) / kBlock);
    if (dt == 0)
        hipLaunchKernelGGL(k_normalize<float>, dim3(grid), dim3(kBlock), 0, s, (const Cx<float>*)data,
                           (const float*)weights, elems, float(reg), (Cx<float>*)out);
    else
        hipLaunchKernelGGL(k_normalize<double>, dim3(grid), dim3(kBlock), 0, s, (const Cx<double>*)data,
                           (const double*)weights, elems, reg, (Cx<double>*)out);
    return hipGetLastError();
}

}  // namespace tp
