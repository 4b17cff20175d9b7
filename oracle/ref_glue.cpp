// ref_glue.cpp — extern "C" entry points over the reference's own host code.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile together with the
// reference source file cpu/codebook.cpp (compiled where it lies under the
// reference checkout, with the reference's own host flags -O3 -march=native,
// CMakeLists.txt:25) into oracle/_ref/libjhq_ref.so.  Tests use it to pin the
// C oracle against the real reference implementation.  cpu/jl_transform.cpp
// needs cblas.h and LAPACK, which this image lacks, so it is not built; the
// libstdc++ draws it makes (std::mt19937 + std::normal_distribution<float>,
// cpu/jl_transform.cpp:27-29) are reproduced here with the same flags.
#include "cpu/codebook.h"
#include "cpu/erfinv.h"

#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

extern "C" {

float ref_erfinv(float x) { return erfinv_f(x); }

int ref_c1d(int d, int M, int B, float sigma, float* out) {
    LloydMaxCodebook cb(d, M, B, sigma);
    const std::vector<float>& c = cb.c1d();
    std::memcpy(out, c.data(), c.size() * sizeof(float));
    return (int)c.size();
}

void ref_encode(int d, int M, int B, float sigma, const float* y, int n, uint8_t* codes) {
    LloydMaxCodebook cb(d, M, B, sigma);
    cb.encode(y, codes, n);
}

void ref_flat_lut(int d, int M, int B, float sigma, const float* q, float* lut) {
    LloydMaxCodebook cb(d, M, B, sigma);
    cb.build_flat_lut(q, lut);
}

void ref_build_lut(int d, int M, int B, float sigma, const float* q, float* lut) {
    LloydMaxCodebook cb(d, M, B, sigma);
    cb.build_lut(q, lut);
}

float ref_adc_distance(int d, int M, int B, float sigma, const uint8_t* code, const float* lut) {
    LloydMaxCodebook cb(d, M, B, sigma);
    return cb.adc_distance(code, lut);
}

void ref_reconstruct(int d, int M, int B, float sigma, const uint8_t* code, float* out) {
    LloydMaxCodebook cb(d, M, B, sigma);
    cb.reconstruct(code, out);
}

int ref_train_1d_kmeans(const float* vals, int n, int Kr, int max_iter, float* out) {
    std::vector<float> c = train_1d_kmeans(vals, n, Kr, max_iter);
    std::memcpy(out, c.data(), c.size() * sizeof(float));
    return (int)c.size();
}

void ref_mt19937_fill(int seed, uint32_t* out, int64_t n) {
    std::mt19937 rng(seed);
    for (int64_t i = 0; i < n; i++) out[i] = (uint32_t)rng();
}

void ref_normal_fill(int seed, float* out, int64_t n) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> norm(0.0f, 1.0f);
    for (int64_t i = 0; i < n; i++) out[i] = norm(rng);
}

}  // extern "C"
