// AddressSanitizer / UBSan driver (test infrastructure): exercises the C
// oracle (oracle/jhq_oracle.c) and the product's host training code
// (jhq_gpu_amd/csrc/host_train.cpp) on small inputs, including edge cases
// (Kr > n, d = 1, duplicate values, empty lists, k > candidates), so that an
// out-of-bounds access or undefined behaviour in either aborts the run.
// Built and run by tests/test_asan.py with g++ -fsanitize=address,undefined.
#include "../../jhq_gpu_amd/csrc/host_train.h"
extern "C" {
#include "../jhq_oracle.h"
}

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

static int fails = 0;
#define CHECK(c)                                                     \
    do {                                                             \
        if (!(c)) {                                                  \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            fails++;                                                 \
        }                                                            \
    } while (0)

int main() {
    std::mt19937 rng(7);
    std::normal_distribution<float> nd(0.f, 1.f);
    // host training code
    for (int d : {1, 8, 33, 64}) {
        std::vector<float> P = jhq::build_rotation(d, 42);
        CHECK((int)P.size() == d * d);
        std::vector<float> Po((size_t)d * d);
        o_build_rotation(d, 42, Po.data());
        CHECK(std::memcmp(P.data(), Po.data(), P.size() * 4) == 0);
    }
    for (int n : {1, 3, 16, 1000}) {
        std::vector<float> v(n);
        for (auto& x : v) x = nd(rng) * 0.1f;
        if (n == 16) for (auto& x : v) x = 0.25f;  // all equal
        for (int Kr : {1, 2, 16}) {
            std::vector<float> c = jhq::train_1d_kmeans(v.data(), n, Kr);
            std::vector<float> co(Kr);
            const int m = o_train_1d_kmeans(v.data(), n, Kr, 25, co.data());
            CHECK((int)c.size() == m);
            CHECK(std::memcmp(c.data(), co.data(), (size_t)m * 4) == 0);
        }
    }
    for (int K1D : {2, 4, 256}) {
        std::vector<float> c = jhq::lloyd_max_c1d(0.5f, K1D);
        std::vector<float> co(K1D);
        o_lloyd_max_c1d(0.5f, K1D, co.data());
        CHECK(std::memcmp(c.data(), co.data(), (size_t)K1D * 4) == 0);
    }
    // oracle index: train / add / search, with empty lists and k > candidates
    const int d = 32, M = 8, nlist = 16, n = 600, nq = 5;
    std::vector<float> x((size_t)n * d), q((size_t)nq * d);
    for (auto& e : x) e = nd(rng);
    for (auto& e : q) e = nd(rng);
    std::vector<float> P((size_t)d * d), Pc((size_t)d * d);
    o_build_rotation(d, 42, Pc.data());
    for (int j = 0; j < d; j++)
        for (int k = 0; k < d; k++) P[(size_t)j * d + k] = Pc[(size_t)k * d + j];
    std::vector<float> y((size_t)n * d);
    o_set_threads(3);
    o_rotate(P.data(), x.data(), n, d, y.data());
    const float sigma = o_estimate_sigma(x.data(), n, d);
    const int Ds = d / M, bpd = 8 / Ds, K1D = 1 << bpd, Kr = 16, Br = 4, bpv = (d * Br + 7) / 8;
    std::vector<float> c1d(K1D);
    o_lloyd_max_c1d(sigma, K1D, c1d.data());
    std::vector<uint8_t> codes((size_t)n * M), res((size_t)n * bpv);
    std::vector<float> corr(n), rc(Kr);
    o_primary_encode(y.data(), n, d, M, c1d.data(), K1D, codes.data());
    std::vector<float> resid((size_t)n * d);
    for (int i = 0; i < n; i++) {
        std::vector<float> rec(d);
        o_reconstruct(codes.data() + (size_t)i * M, d, M, c1d.data(), K1D, rec.data());
        for (int j = 0; j < d; j++) resid[(size_t)i * d + j] = y[(size_t)i * d + j] - rec[j];
    }
    CHECK(o_train_1d_kmeans(resid.data(), (int64_t)n * d, Kr, 25, rc.data()) == Kr);
    o_residual_encode(y.data(), codes.data(), n, d, M, c1d.data(), K1D, rc.data(), Kr, Br,
                      res.data(), corr.data());
    std::vector<float> cent((size_t)nlist * d), norms(nlist);
    CHECK(o_train_ivf(y.data(), n, d, nlist, 4, cent.data()) == 0);
    // two identical centroids: one list stays empty
    std::memcpy(cent.data() + 15 * d, cent.data() + 14 * d, d * 4);
    o_cent_norms(cent.data(), nlist, d, norms.data());
    std::vector<int32_t> asg(n), offs(nlist + 1), order(n);
    o_assign(y.data(), n, d, cent.data(), norms.data(), nlist, asg.data());
    o_build_lists(asg.data(), n, nlist, offs.data(), order.data());
    CHECK(offs[15] == offs[16]);
    std::vector<uint8_t> lc((size_t)n * M), lr((size_t)n * bpv);
    std::vector<float> lco(n);
    for (int p = 0; p < n; p++) {
        std::memcpy(lc.data() + (size_t)p * M, codes.data() + (size_t)order[p] * M, M);
        std::memcpy(lr.data() + (size_t)p * bpv, res.data() + (size_t)order[p] * bpv, bpv);
        lco[p] = corr[order[p]];
    }
    o_index ix{};
    ix.d = d; ix.M = M; ix.B = 8; ix.Br = Br; ix.Ds = Ds; ix.K1D = K1D; ix.bpd = bpd; ix.Kr = Kr;
    ix.bpv = bpv; ix.nlist = nlist; ix.RC = 1; ix.alpha = 4.0f; ix.ntotal = n;
    ix.P = P.data(); ix.c1d = c1d.data(); ix.res_c1d = rc.data(); ix.cent = cent.data();
    ix.cent_norms = norms.data(); ix.list_offsets = offs.data(); ix.list_ids = order.data();
    ix.list_codes = lc.data(); ix.list_res = lr.data(); ix.list_corr = lco.data();
    for (int nprobe : {1, 3, 16}) {
        for (int k : {1, 10, 200}) {  // 200 * 4 > candidates of one list
            ix.nprobe = nprobe;
            const int ck = o_ck(ix.alpha, k);
            std::vector<float> od((size_t)nq * k), td((size_t)nq * ck);
            std::vector<int32_t> oi((size_t)nq * k), pr((size_t)nq * nprobe), tp((size_t)nq * ck);
            for (int mode : {0, 1}) {
                CHECK(o_search_mode(&ix, q.data(), nullptr, nullptr, nq, k, mode, od.data(),
                                    oi.data(), pr.data(), tp.data(), td.data()) == 0);
                for (int i = 0; i < nq * k; i++) CHECK(oi[i] >= -1 && oi[i] < n);
            }
        }
    }
    std::printf(fails ? "asan driver: %d checks failed\n" : "asan driver ok\n", fails);
    return fails ? 1 : 0;
}
