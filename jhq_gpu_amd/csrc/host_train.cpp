// host_train.cpp — host-side training math (see host_train.h).
#include "host_train.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <thread>

namespace jhq {

// libstdc++ generate_canonical<float, 24>(mt19937): one draw, float(u)/2^32,
// clamped below 1.
static inline float canonical(std::mt19937& g) {
    const float s = static_cast<float>(static_cast<uint32_t>(g()));
    float r = s / 4294967296.0f;
    if (r >= 1.0f) r = std::nextafter(1.0f, 0.0f);
    return r;
}

// libstdc++ normal_distribution<float>: Marsaglia polar method, y*mult first,
// x*mult cached for the next draw.  The reference instantiates it in a
// -march=native translation unit, where x*x + y*y becomes fma(x, x, y*y).
void normal_fill(uint32_t seed, float* out, int64_t n) {
    std::mt19937 g(seed);
    int64_t i = 0;
    while (i < n) {
        float x, y, r2;
        do {
            x = static_cast<float>(static_cast<double>(2.0f * canonical(g)) - 1.0);
            y = static_cast<float>(static_cast<double>(2.0f * canonical(g)) - 1.0);
            r2 = std::fma(x, x, y * y);
        } while (static_cast<double>(r2) > 1.0 || static_cast<double>(r2) == 0.0);
        const float mult = std::sqrt(-2.0f * std::log(r2) / r2);
        out[i++] = y * mult;
        if (i < n) out[i++] = x * mult;
    }
}

float erfinv_f(float x) {
    if (x >= 1.0f) return std::numeric_limits<float>::infinity();
    if (x <= -1.0f) return -std::numeric_limits<float>::infinity();
    if (x == 0.0f) return 0.0f;
    const float sign = (x > 0.0f) ? 1.0f : -1.0f;
    const float a = std::fabs(x);
    const float kC = 0.147f;
    const float k2Pi = 2.0f / 3.14159265358979f;
    // 1 - a*a, k2Pi/kC + 0.5*ln1 and t*t - ln1/kC are contracted by the
    // reference build.
    const float ln1 = std::log(std::fma(-a, a, 1.0f));
    const float t = std::fma(0.5f, ln1, k2Pi / kC);
    float z = sign * std::sqrt(std::sqrt(std::fma(t, t, -(ln1 / kC))) - t);
    const float err = std::erf(z) - x;
    const float der = (2.0f / std::sqrt(static_cast<float>(M_PI))) * std::exp(-z * z);
    z -= err / der;
    return z;
}

std::vector<float> lloyd_max_c1d(float sigma, int K1D) {
    std::vector<float> c(K1D);
    for (int i = 0; i < K1D; i++) {
        const float q_i = (static_cast<float>(i) + 0.5f) / static_cast<float>(K1D);
        c[i] = sigma * static_cast<float>(M_SQRT2) * erfinv_f(std::fma(2.0f, q_i, -1.0f));
    }
    return c;
}

float estimate_sigma(const float* x, int64_t n, int d) {
    double sum2 = 0.0;
    const int64_t total = n * static_cast<int64_t>(d);
    for (int64_t i = 0; i < total; i++) sum2 += static_cast<double>(x[i]) * static_cast<double>(x[i]);
    return static_cast<float>(std::sqrt(sum2 / (static_cast<double>(n) * d)));
}

int nearest_sorted(const float* arr, int n, float v) {
    if (n == 1) return 0;
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (v < 0.5f * (arr[mid] + arr[mid + 1])) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

// The reference sorts a full copy of the n values only to read Kr quantiles
// (cpu/codebook.cpp:13-20, reused for empty clusters at :46-49).  Order
// statistics are unique values, so selecting just those Kr ranks with
// nth_element gives the same codewords without the O(n log n) sort.
std::vector<float> train_1d_kmeans(const float* vals, int64_t n, int Kr, int max_iter) {
    if (n <= 0 || Kr <= 0) return {};
    if (n < Kr) Kr = static_cast<int>(n);
    const float nf = static_cast<float>(n);
    std::vector<int64_t> qidx(Kr);
    for (int i = 0; i < Kr; i++) {
        int64_t idx = static_cast<int64_t>((static_cast<float>(i) + 0.5f) / static_cast<float>(Kr) * nf);
        qidx[i] = std::min<int64_t>(idx, n - 1);
    }
    std::vector<float> quant(Kr);
    {
        std::vector<float> work(vals, vals + n);
        // ranks ascending; partition successively so each nth_element works on
        // the remaining suffix only.
        std::vector<int> order(Kr);
        for (int i = 0; i < Kr; i++) order[i] = i;
        std::sort(order.begin(), order.end(), [&](int a, int b) { return qidx[a] < qidx[b]; });
        int64_t lo = 0;
        for (int oi = 0; oi < Kr; oi++) {
            const int64_t r = qidx[order[oi]];
            if (r >= lo) {
                std::nth_element(work.begin() + lo, work.begin() + r, work.end());
                lo = r;
            }
            quant[order[oi]] = work[r];
        }
    }
    std::vector<float> c(quant);
    std::vector<double> sum(Kr);
    std::vector<int64_t> cnt(Kr);
    // Assignment is a pure function of (value, codewords): computed in
    // parallel.  The per-cluster double sums stay one sequential pass in index
    // order, so every rounding matches the reference loop.
    std::vector<uint8_t> a8(Kr <= 256 ? static_cast<size_t>(n) : 0);
    std::vector<int32_t> a32(Kr <= 256 ? 0 : static_cast<size_t>(n));
    unsigned nth = std::thread::hardware_concurrency();
    nth = std::max(1u, std::min(nth, 16u));
    if (n < (int64_t)1 << 16) nth = 1;
    for (int iter = 0; iter < max_iter; iter++) {
        std::fill(sum.begin(), sum.end(), 0.0);
        std::fill(cnt.begin(), cnt.end(), 0);
        auto work = [&](int64_t i0, int64_t i1) {
            for (int64_t i = i0; i < i1; i++) {
                const int lo = nearest_sorted(c.data(), Kr, vals[i]);
                if (Kr <= 256) a8[i] = static_cast<uint8_t>(lo);
                else a32[i] = lo;
            }
        };
        if (nth == 1) {
            work(0, n);
        } else {
            std::vector<std::thread> th;
            for (unsigned t = 0; t < nth; t++)
                th.emplace_back(work, n * t / nth, n * (t + 1) / nth);
            for (auto& t : th) t.join();
        }
        if (Kr <= 256) {
            for (int64_t i = 0; i < n; i++) {
                sum[a8[i]] += vals[i];
                cnt[a8[i]]++;
            }
        } else {
            for (int64_t i = 0; i < n; i++) {
                sum[a32[i]] += vals[i];
                cnt[a32[i]]++;
            }
        }
        bool changed = false;
        for (int i = 0; i < Kr; i++) {
            const float new_c = (cnt[i] == 0) ? quant[i]
                                              : static_cast<float>(sum[i] / static_cast<double>(cnt[i]));
            if (new_c != c[i]) { c[i] = new_c; changed = true; }
        }
        std::sort(c.begin(), c.end());
        if (!changed) break;
    }
    return c;
}

std::vector<float> build_rotation(int d, int seed) {
    const int64_t n = d;
    std::vector<float> G(static_cast<size_t>(n * n));
    normal_fill(static_cast<uint32_t>(seed), G.data(), n * n);
    std::vector<double> A(G.begin(), G.end());
    std::vector<double> tau(static_cast<size_t>(n));
    // xGEQR2: column k reflector with beta = -sign(alpha) * ||A(k:n, k)||.
    for (int64_t k = 0; k < n; k++) {
        double* colk = A.data() + k * n;
        const double alpha = colk[k];
        double ss = 0.0;
        for (int64_t i = k + 1; i < n; i++) ss += colk[i] * colk[i];
        if (ss == 0.0) { tau[k] = 0.0; continue; }
        const double nrm = std::sqrt(alpha * alpha + ss);
        const double beta = (alpha >= 0.0) ? -nrm : nrm;
        tau[k] = (beta - alpha) / beta;
        const double scal = 1.0 / (alpha - beta);
        for (int64_t i = k + 1; i < n; i++) colk[i] *= scal;
        colk[k] = beta;
        for (int64_t j = k + 1; j < n; j++) {
            double* colj = A.data() + j * n;
            double w = colj[k];
            for (int64_t i = k + 1; i < n; i++) w += colk[i] * colj[i];
            w *= tau[k];
            colj[k] -= w;
            for (int64_t i = k + 1; i < n; i++) colj[i] -= w * colk[i];
        }
    }
    // xORG2R: Q = H_1 ... H_n applied to the identity, last reflector first.
    for (int64_t i = n - 1; i >= 0; i--) {
        double* coli = A.data() + i * n;
        if (i < n - 1) {
            coli[i] = 1.0;
            for (int64_t j = i + 1; j < n; j++) {
                double* colj = A.data() + j * n;
                double w = 0.0;
                for (int64_t r = i; r < n; r++) w += coli[r] * colj[r];
                w *= tau[i];
                for (int64_t r = i; r < n; r++) colj[r] -= w * coli[r];
            }
            for (int64_t r = i + 1; r < n; r++) coli[r] *= -tau[i];
        }
        coli[i] = 1.0 - tau[i];
        for (int64_t r = 0; r < i; r++) coli[r] = 0.0;
    }
    for (int64_t i = 0; i < n * n; i++) G[i] = static_cast<float>(A[i]);
    return G;
}

}  // namespace jhq
