// jhq_gpu_index.cuh — drop-in for the reference header of the same path
// (lrlorry/JHQ_GPU jhq_v14_streaming_add/jhq_gpu_index.cuh:14-83).
//
// Put this repository's include/ directory ahead of the reference checkout on
// the include path and link with -ljhq_amd: code written against
// jhq_gpu::JHQGpuIndex (e.g. examples/demo_jhq_v14_streaming_add.cu) compiles
// unchanged with g++ or hipcc and runs on the MI355X engine.  The class is a
// header-only forwarder to the C-ABI of jhq.h.
//
// Kept from the reference: the namespace, class and method names, Params with
// the same fields and defaults (:16-36), train / add / search / ntotal / dim
// (:41-47), one add() per index (a second throws std::runtime_error,
// v14/jhq_gpu_index.cu:419-420), the constructor's parameter checks and
// messages (std::invalid_argument, v14/jhq_gpu_index.cu:110-121), search()
// returning row-major [nq x k] dists and labels with (+inf, -1) padding.
// Differences: device failures throw std::runtime_error instead of exiting
// the process (common/cuda_utils.cuh:7-25); the top-ck short list is exact
// (the reference keeps 4 candidates per thread, v14/search.cu:116,153-161).
#pragma once

#include "../jhq.h"

#include <cstdint>
#include <stdexcept>
#include <string>

namespace jhq_gpu {

class JHQGpuIndex {
public:
    struct Params {
        int   M          = 96;
        int   B          = 8;
        int   Br         = 4;
        float alpha      = 4.0f;
        int   nlist      = 1024;
        int   nprobe     = 8;
        int   ivf_iters  = 8;
        int   batch_size = 256;
        int   seed       = 42;
        int   add_batch  = 65536;
        // extension (no reference counterpart): one residual codebook per
        // subspace; 0 = the reference's single codebook
        int   residual_per_subspace = 0;
    };

    JHQGpuIndex(int d, Params p) {
        jhq_params c{p.M,         p.B,          p.Br,   p.alpha,     p.nlist,
                     p.nprobe,    p.ivf_iters,  p.batch_size, p.seed, p.add_batch,
                     p.residual_per_subspace};
        check(jhq_create(d, &c, &h_));
    }
    ~JHQGpuIndex() {
        if (h_) jhq_destroy(h_);
    }
    JHQGpuIndex(const JHQGpuIndex&) = delete;
    JHQGpuIndex& operator=(const JHQGpuIndex&) = delete;
    JHQGpuIndex(JHQGpuIndex&& o) noexcept : h_(o.h_) { o.h_ = nullptr; }
    JHQGpuIndex& operator=(JHQGpuIndex&& o) noexcept {
        if (this != &o) {
            if (h_) jhq_destroy(h_);
            h_ = o.h_;
            o.h_ = nullptr;
        }
        return *this;
    }

    void train(const float* h_x, int n_train) { check(jhq_train(h_, h_x, n_train)); }
    void add(const float* h_x, int n) { check(jhq_add(h_, h_x, n)); }
    void search(const float* h_q, int nq, int k, float* h_dists, int* h_labels) const {
        check(jhq_search(h_, h_q, nq, k, h_dists, reinterpret_cast<int32_t*>(h_labels)));
    }
    int ntotal() const { return static_cast<int>(jhq_ntotal(h_)); }
    int dim() const { return jhq_dim(h_); }

    // ---- extensions (no reference counterpart) ----
    // streaming add: any number of calls, between searches
    void append(const float* h_x, int n) { check(jhq_append(h_, h_x, n)); }
    // byte rows (converted to float32 on the device)
    void train_u8(const uint8_t* h_x, int n) { check(jhq_train_ex(h_, h_x, JHQ_U8, n)); }
    void add_u8(const uint8_t* h_x, int n) { check(jhq_add_ex(h_, h_x, JHQ_U8, n)); }
    void add_i8(const int8_t* h_x, int n) { check(jhq_add_ex(h_, h_x, JHQ_I8, n)); }
    // queries and results in device memory, enqueued on a hipStream_t
    void search_device(const float* d_q, int nq, int k, float* d_dists, int* d_labels,
                       void* stream) const {
        check(jhq_search_device(h_, d_q, nq, k, d_dists, reinterpret_cast<int32_t*>(d_labels),
                                stream));
    }
    void reserve(int k_max) { check(jhq_reserve(h_, k_max)); }
    void set_nprobe(int nprobe) { check(jhq_set_nprobe(h_, nprobe)); }
    void set_alpha(float alpha) { check(jhq_set_alpha(h_, alpha)); }
    void save(const char* path) const { check(jhq_save(h_, path)); }
    static JHQGpuIndex load(const char* path) {
        jhq_index* h = nullptr;
        check(jhq_load(path, &h));
        return JHQGpuIndex(h);
    }

private:
    explicit JHQGpuIndex(jhq_index* h) : h_(h) {}
    static void check(int rc) {
        if (rc == JHQ_OK) return;
        const std::string msg = jhq_last_error();
        if (rc == JHQ_EINVAL) throw std::invalid_argument(msg);
        throw std::runtime_error(msg);
    }
    jhq_index* h_ = nullptr;
};

}  // namespace jhq_gpu
