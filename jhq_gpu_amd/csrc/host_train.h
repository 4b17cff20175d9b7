// host_train.h — host-side training math of the JHQ engine.
//
// Restates the reference's cpu/ library (lrlorry/JHQ_GPU cpu/jl_transform.cpp,
// cpu/codebook.cpp, cpu/erfinv.h) with the floating-point order pinned: this
// file is compiled with -ffp-contract=off and uses fmaf() exactly where the
// reference's -O3 -march=native build contracts a multiply-add.
#pragma once
#include <cstdint>
#include <vector>

namespace jhq {

// std::mt19937(seed) + libstdc++ std::normal_distribution<float>(0,1) draws
// (cpu/jl_transform.cpp:27-29).
void normal_fill(uint32_t seed, float* out, int64_t n);

// cpu/erfinv.h:7-27
float erfinv_f(float x);

// cpu/codebook.cpp:60-80 — c1d[i] = sigma*sqrt2*erfinv(2(i+1/2)/K1D - 1)
std::vector<float> lloyd_max_c1d(float sigma, int K1D);

// cpu/jl_transform.cpp:73-83
float estimate_sigma(const float* x, int64_t n, int d);

// cpu/codebook.cpp:8-58 — 1-D Lloyd k-means with quantile initialisation.
std::vector<float> train_1d_kmeans(const float* vals, int64_t n, int Kr, int max_iter = 25);

// cpu/jl_transform.cpp:25-56 — Gaussian fill in column-major storage order,
// Householder QR (LAPACK xGEQR2/xORG2R conventions, computed in double).
// Returns Pi in column-major order (JLTransform::pi_data()).
std::vector<float> build_rotation(int d, int seed);

// Nearest codeword by midpoint binary search (v14/encode.cu:6-18).
int nearest_sorted(const float* arr, int n, float v);

}  // namespace jhq
