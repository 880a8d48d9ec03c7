// Host-side check of the cubic weight functions of tp_device.hh, built by
// tests/test_cubic_weights_cpu.py with hipcc --cuda-host-only and the library's
// floating-point flags.  For every float f in [0, 1] and tap j < 4:
//   * cubic_w_tap(f, j) must equal cubic_w(f - (j - 1)) bit for bit (float and, on
//     the same f, double);
//   * cubic_w_fast / cubic_dw_fast of s = f - (j - 1) are compared with the
//     piecewise formulas evaluated in double (cubic_w<double> / cubic_dw<double> of
//     the same s): the largest relative error where |exact| >= 1e-6, and the largest
//     absolute error anywhere.
// Prints one line of counts and error maxima.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "tp_device.hh"

namespace {
struct Acc {
    long mism_f = 0, mism_d = 0, n = 0;
    double w_rel = 0, w_abs = 0, dw_rel = 0, dw_abs = 0;
};
template <typename T, typename U> bool same_bits(T a, T b) {
    U x, y;
    std::memcpy(&x, &a, sizeof a);
    std::memcpy(&y, &b, sizeof b);
    return x == y;
}
void track(double got, double exact, double& rel, double& abs_) {
    const double d = std::fabs(got - exact);
    abs_ = std::fmax(abs_, d);
    if (std::fabs(exact) >= 1e-6) rel = std::fmax(rel, d / std::fabs(exact));
}
void run(uint32_t lo, uint32_t hi, Acc& a) {
    for (uint32_t u = lo; u < hi; ++u) {
        float f;
        std::memcpy(&f, &u, 4);
        for (int j = 0; j < 4; ++j) {
            const float s = f - float(j - 1);
            if (!same_bits<float, uint32_t>(tp::cubic_w_tap<float>(f, j), tp::cubic_w<float>(s))) ++a.mism_f;
            const double fd = f;
            if (!same_bits<double, uint64_t>(tp::cubic_w_tap<double>(fd, j), tp::cubic_w<double>(fd - double(j - 1))))
                ++a.mism_d;
            track(tp::cubic_w_fast(s), tp::cubic_w<double>(double(s)), a.w_rel, a.w_abs);
            track(tp::cubic_dw_fast(s), tp::cubic_dw<double>(double(s)), a.dw_rel, a.dw_abs);
        }
        ++a.n;
    }
}
}  // namespace

int main() {
    const uint32_t end = 0x3f800001u;  // bit patterns 0 .. 0x3f800000 are the floats in [0, 1]
    const int nt = 8;
    std::vector<Acc> acc(nt);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t) {
        const uint32_t lo = uint32_t(uint64_t(end) * t / nt), hi = uint32_t(uint64_t(end) * (t + 1) / nt);
        th.emplace_back(run, lo, hi, std::ref(acc[t]));
    }
    for (auto& x : th) x.join();
    Acc s;
    for (const Acc& a : acc) {
        s.mism_f += a.mism_f;
        s.mism_d += a.mism_d;
        s.n += a.n;
        s.w_rel = std::fmax(s.w_rel, a.w_rel);
        s.w_abs = std::fmax(s.w_abs, a.w_abs);
        s.dw_rel = std::fmax(s.dw_rel, a.dw_rel);
        s.dw_abs = std::fmax(s.dw_abs, a.dw_abs);
    }
    std::printf("values %ld tap_mismatch_f32 %ld tap_mismatch_f64 %ld w_fast_rel %.3e w_fast_abs %.3e "
                "dw_fast_rel %.3e dw_fast_abs %.3e\n",
                s.n, s.mism_f, s.mism_d, s.w_rel, s.w_abs, s.dw_rel, s.dw_abs);
    return 0;
}
