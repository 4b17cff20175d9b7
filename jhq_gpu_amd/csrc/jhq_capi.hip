// jhq_capi.hip — C-ABI of the JHQ IVF engine: index object, train / add /
// search orchestration over the HIP kernels in kernels.hip.
//
// Mirrors JHQGpuIndex (lrlorry/JHQ_GPU jhq_v14_streaming_add/jhq_gpu_index.cu)
// and search_gpu (jhq_v14_streaming_add/search.cu:388-445); every entry point
// of include/jhq.h cites the reference interface it replaces.
#include "../../include/jhq.h"
#include "host_train.h"
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <new>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

// Progress lines on stderr for long builds, when JHQ_VERBOSE is set.
bool verbose() {
    static const bool v = [] {
        const char* e = std::getenv("JHQ_VERBOSE");
        return e && *e && *e != '0';
    }();
    return v;
}

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define JHQ_HIP(expr)                                                                  \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return fail(e_ == hipErrorOutOfMemory ? JHQ_ENOMEM : JHQ_EDEVICE,          \
                        std::string(#expr) + ": " + hipGetErrorString(e_));            \
    } while (0)

#define JHQ_TRY(expr)            \
    do {                         \
        int rc_ = (expr);        \
        if (rc_ != JHQ_OK) return rc_; \
    } while (0)

// Owning device buffer.
template <class T>
struct DBuf {
    T* p = nullptr;
    size_t n = 0;
    DBuf() = default;
    DBuf(const DBuf&) = delete;
    DBuf& operator=(const DBuf&) = delete;
    ~DBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    // The new buffer is allocated before the old one is freed, so a failed
    // allocation leaves the old buffer (and its contents) in place.
    int alloc(size_t count) {
        if (count == 0) count = 1;
        T* np = nullptr;
        hipError_t e = hipMalloc(reinterpret_cast<void**>(&np), count * sizeof(T));
        if (e != hipSuccess)
            return fail(JHQ_ENOMEM, "hipMalloc of " + std::to_string(count * sizeof(T)) +
                                        " bytes: " + hipGetErrorString(e));
        release();
        p = np;
        n = count;
        return JHQ_OK;
    }
    bool has(size_t count) const { return p && count <= n; }
    int ensure(size_t count) { return has(count) ? JHQ_OK : alloc(count); }
    int upload(const T* h, size_t count) {
        JHQ_TRY(alloc(count));
        JHQ_HIP(hipMemcpy(p, h, count * sizeof(T), hipMemcpyHostToDevice));
        return JHQ_OK;
    }
    // the same into the buffer it already has when that is large enough (n
    // stays its capacity)
    int upload_keep(const T* h, size_t count) {
        JHQ_TRY(ensure(count));
        JHQ_HIP(hipMemcpy(p, h, count * sizeof(T), hipMemcpyHostToDevice));
        return JHQ_OK;
    }
    size_t bytes() const { return p ? n * sizeof(T) : 0; }
};

// Device scratch of an insert (codes, residual codes and corrections of the
// new vectors, their lists, input and rotated batches, sort and scatter
// buffers), kept between inserts so that streaming appends allocate nothing
// once warm; released after an insert whose buffers exceed kInsertKeepBytes.
constexpr size_t kInsertKeepBytes = size_t(256) << 20;
struct InsertScratch {
    DBuf<uint8_t> pc, rc;
    DBuf<float> co;
    DBuf<int32_t> asg;
    DBuf<float> xb[2], yb;
    DBuf<uint8_t> raw[2];
    DBuf<unsigned long long> keys;
    DBuf<unsigned char> oscr;
    DBuf<int32_t> order, slist, sidx;
    DBuf<int4> moves;
    size_t bytes() const {
        return pc.bytes() + rc.bytes() + co.bytes() + asg.bytes() + xb[0].bytes() +
               xb[1].bytes() + yb.bytes() + raw[0].bytes() + raw[1].bytes() + keys.bytes() +
               oscr.bytes() + order.bytes() + slist.bytes() + sidx.bytes() + moves.bytes();
    }
    void release() {
        pc.release(); rc.release(); co.release(); asg.release();
        xb[0].release(); xb[1].release(); yb.release(); raw[0].release(); raw[1].release();
        keys.release(); oscr.release(); order.release(); slist.release(); sidx.release();
        moves.release();
    }
};

constexpr int kSteps = 4;

// Search lanes (workspace, stream, pinned staging) that consecutive batches
// of one call rotate through.  Six are created and the ones on hardware
// queues of their own are used (calibrate_lanes: four with HIP's default
// four queues): each lane's batch is a chain of short, latency-bound
// kernels, and more chains in flight fill the CUs, but two lanes on one
// queue run one after the other (config 2, device-resident: 1.75 M queries/s
// on the four lanes with queues of their own, 1.50 M rotating through all
// six; four lanes created alone landed on two queues, 1.19 M).
#ifndef JHQ_LANES
#define JHQ_LANES 6
#endif
constexpr int kLanes = JHQ_LANES;
static_assert(kLanes >= 1, "at least one lane");

// Consecutive batches of a device search that one lane takes together: their
// query product runs once over all their rows (each split sum is that of the
// batch's own product, the same bits), so the [Pi ; C Pi] operand is read
// once per pair of batches.
#ifndef JHQ_QB_SHARE
#define JHQ_QB_SHARE 2
#endif
constexpr int kQbShare = JHQ_QB_SHARE;
static_assert(kQbShare >= 1, "at least one batch per product");

// Per-batch search buffers (v14/search.cuh:24-46).  The index keeps one set
// per search lane (kLanes): consecutive batches of one device search take the
// lanes in turn, each lane a stream of its own, so one batch's scan overlaps
// the other lanes' query products, plans and re-checks.
struct Workspace {
    DBuf<float> wq, wqrot, wscores, wout_d;
    DBuf<int32_t> wprobes, wgofs, wqtot, wout_i, wpslot;
    DBuf<unsigned long long> wpartial, wtopck, wdump;
    // split sums of the query product
    DBuf<float> wqpart;
    // integer-MFMA pre-scan: quantized queries and the batch's list hash
    DBuf<unsigned char> wmfma;
    // the hash in wmfma is clear for batches of hash_P probes at hash_ws
    // (each batch's re-check clears it for the next; a batch that stopped
    // between its selection and its re-check leaves it unclear)
    bool hash_clear = false;
    int hash_P = 0;
    const unsigned char* hash_ws = nullptr;
};

}  // namespace

struct jhq_index {
    // parameters (v14/jhq_gpu_index.cuh:50-54)
    int d = 0, M = 0, B = 0, Br = 0, Ds = 0, K1D = 0, bpd = 0, Kr = 0, bpv = 0;
    int nlist = 0, nprobe = 0, ivf_iters = 0, batch_size = 0, seed = 0, add_batch = 0;
    int RC = 1;  // residual codebooks: 1 (reference) or M (one per subspace)
    float alpha = 0.f;
    int64_t ntotal = 0;
    bool trained = false;
    bool added = false;
    // set while an insert rewrites the lists; a failed insert leaves it set
    // and searches refuse the index (its device descriptors may be stale)
    bool broken = false;
    int num_cu = 256;
    // searches with k <= res_k (and the current nprobe, alpha, batch_size)
    // run in the preallocated workspace; jhq_reserve raises it
    int res_k = 10;
    // 0: the integer-MFMA pre-scan where it applies (one-bit digits) and its
    // tiles are expected to be mostly full, else the byte-LUT scans; 1: the
    // byte-LUT scans only; 2: the pre-scan wherever it applies
    int scan_kind = 0;
    // the default scan kind's choice of the pre-scan, measured on stored
    // vectors taken as queries; valid for batches of mfma_dec_B queries with
    // mfma_dec_P probes while the index holds 0.8 to 1.25 times mfma_dec_n
    // vectors
    int mfma_dec_B = 0, mfma_dec_P = 0;
    int64_t mfma_dec_n = 0;
    double mfma_dec_cost = 0.0, mfma_dec_cand = 0.0;
    // largest per-query candidate count of the dump scan for dump_P probes
    int dump_P = -1;
    int64_t dump_perq = 0;

    float sigma = 1.f;
    std::vector<float> Pi_cm;  // JLTransform::pi_data() (column-major)
    std::vector<float> P_rm;   // row-major Pi(j,k)
    std::vector<float> c1d, res_c1d, cent, cent_norms;

    // list pool (host mirror of the ListDesc array): list l owns slots
    // [start, start + cap) and holds size candidates
    std::vector<int32_t> l_start, l_cap, l_size;
    int64_t pool_cap = 0, pool_used = 0;

    hipStream_t stream = nullptr;
    // recorded on the caller's stream after every device search; inserts,
    // re-reservations and host searches wait on it
    hipEvent_t done_ev = nullptr;
    bool done_pending = false;
    // inserts and row refreshes end without a host wait: their last work on
    // `stream` is tail_ev; device searches wait for it on the device, and
    // everything that reads or rewrites the lists from the host waits first
    hipEvent_t tail_ev = nullptr;
    bool tail_pending = false;
    // pinned staging of the asynchronous descriptor uploads (two, taken in
    // turn; one is written again once its copy's event has passed) and of
    // the row refresh's first rows
    int4* h_ldesc[2] = {};
    size_t h_ldesc_n[2] = {};
    hipEvent_t ldesc_ev[2] = {};
    bool ldesc_pending[2] = {};
    int ldesc_turn = 0;
    int32_t* h_from = nullptr;
    size_t h_from_n = 0;
    hipEvent_t from_ev = nullptr;
    bool from_pending = false;
    DBuf<float> dP, dc1d, dres_c1d, dcent, dnorms;
    DBuf<int4> dldesc;
    DBuf<int32_t> dlist_ids;
    DBuf<uint8_t> dcodes_t, dres;
    // lane-skewed rows of the primary codes, written when a search plan takes
    // the skewed scan; per list, the block start and row count they hold
    DBuf<uint8_t> dcodes_s;
    bool skew_stale = true;
    std::vector<int32_t> skew_start, skew_rows;
    DBuf<int32_t> dskew_from;
    // row-major rows of the primary codes, kept when the pre-scan can be
    // chosen; per list, the block start and row count they hold
    DBuf<uint8_t> dcodes_r;
    bool rows_stale = true;
    std::vector<int32_t> rows_start, rows_rows;
    DBuf<int32_t> drows_from;
    DBuf<float> dcorr;

    // query GEMM operand [Pi ; centroids * Pi] ((d + nlist) x d): one product
    // gives the rotated query and the centroid dots
    DBuf<float> dqmat;
    // IVF assignment scratch (assign_mfma) and, with JHQ_VERBOSE, the count of
    // rows it re-checked since the insert began (device)
    DBuf<float> dascr;
    DBuf<unsigned long long> drecheck;
    // an insert's scratch, kept between inserts (appends) up to kInsertKeepBytes
    InsertScratch ins;

    // search workspaces; ws[1] and the lane streams serve pipelined batches
    Workspace ws[kLanes];
    hipStream_t lane[kLanes] = {};
    hipEvent_t lane_ev[kLanes + 1] = {};  // fork, then each lane's last batch done
    // the lanes pipelined batches take, in turn: one per hardware queue the
    // lanes landed on (calibrate_lanes)
    int lane_use[kLanes] = {};
    int nlanes = 0;
    // inserts: the two input buffers' copied / consumed events (the copies run
    // on the last lane's stream, idle while an insert runs: a stream of its
    // own would share one of the process's 4 hardware queues with a lane and
    // serialise the lanes' batches)
    hipEvent_t copy_ev[4] = {};
    float* h_q[kLanes] = {};  // pinned staging, one set per lane
    float* h_d[kLanes] = {};
    int32_t* h_i[kLanes] = {};
    size_t h_q_n[kLanes] = {}, h_d_n[kLanes] = {}, h_i_n[kLanes] = {};

    bool timing = false;
    hipEvent_t ev[kSteps + 1] = {};
    double tms[kSteps] = {};
    int64_t tbatches = 0;

    ~jhq_index() {
        for (int l = 0; l < kLanes; l++) {
            if (h_q[l]) (void)hipHostFree(h_q[l]);
            if (h_d[l]) (void)hipHostFree(h_d[l]);
            if (h_i[l]) (void)hipHostFree(h_i[l]);
        }
        if (stream) (void)hipStreamSynchronize(stream);
        for (int t = 0; t < 2; t++) {
            if (h_ldesc[t]) (void)hipHostFree(h_ldesc[t]);
            if (ldesc_ev[t]) (void)hipEventDestroy(ldesc_ev[t]);
        }
        if (h_from) (void)hipHostFree(h_from);
        if (from_ev) (void)hipEventDestroy(from_ev);
        if (tail_ev) (void)hipEventDestroy(tail_ev);
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
        for (auto& e : lane_ev)
            if (e) (void)hipEventDestroy(e);
        for (auto& l : lane)
            if (l) (void)hipStreamDestroy(l);
        if (done_ev) (void)hipEventDestroy(done_ev);
        for (auto& e : copy_ev)
            if (e) (void)hipEventDestroy(e);
        if (stream) (void)hipStreamDestroy(stream);
    }

    int ensure_copy_stream() {
        JHQ_TRY(ensure_lanes());
        if (copy_ev[0]) return JHQ_OK;
        for (auto& e : copy_ev) JHQ_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        return JHQ_OK;
    }

    int ensure_lanes() {
        if (lane[kLanes - 1]) return JHQ_OK;
        for (auto& l : lane) JHQ_HIP(hipStreamCreate(&l));
        for (auto& e : lane_ev) JHQ_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        calibrate_lanes();
        return JHQ_OK;
    }

    // Which lanes run side by side.  HIP gives each stream one of the
    // process's hardware queues (GPU_MAX_HW_QUEUES, 4 by default) and shares
    // a queue between streams beyond those; a queue runs one kernel at a
    // time, so two lanes on one queue run their batches one after the other
    // (with six lanes, two queues carried two lanes each and the other two
    // sat idle half of a search).  A one-wave kernel of fixed length runs on
    // the lanes taken so far and on the next lane at once: if they finish
    // within 1.5 times one kernel's time, the next lane has a queue of its
    // own and is taken.  Any failure leaves every lane in use.
    void calibrate_lanes() {
        nlanes = kLanes;
        for (int l = 0; l < kLanes; l++) lane_use[l] = l;
        if (kLanes < 2) return;
        float* buf = nullptr;
        hipEvent_t e0 = nullptr, e1[kLanes] = {};
        int use[kLanes], n = 1;
        use[0] = 0;
        bool ok = hipMalloc(reinterpret_cast<void**>(&buf), kLanes * sizeof(float)) == hipSuccess &&
                  hipEventCreate(&e0) == hipSuccess;
        for (int l = 0; ok && l < kLanes; l++) ok = hipEventCreate(&e1[l]) == hipSuccess;
        // the span from the first lane's start to the last lane's end
        auto span = [&](const int* ls, int m, float* ms) {
            constexpr int kIters = 200000;  // a few hundred us
            if (hipEventRecord(e0, lane[ls[0]]) != hipSuccess) return false;
            for (int i = 1; i < m; i++)
                if (hipStreamWaitEvent(lane[ls[i]], e0, 0) != hipSuccess) return false;
            for (int i = 0; i < m; i++)
                if (jhq::lane_probe(buf + ls[i], kIters, lane[ls[i]]) != hipSuccess ||
                    hipEventRecord(e1[i], lane[ls[i]]) != hipSuccess)
                    return false;
            *ms = 0.f;
            for (int i = 0; i < m; i++) {
                float t = 0.f;
                if (hipEventSynchronize(e1[i]) != hipSuccess ||
                    hipEventElapsedTime(&t, e0, e1[i]) != hipSuccess)
                    return false;
                *ms = std::max(*ms, t);
            }
            return true;
        };
        float t1 = 0.f, t = 0.f;
        ok = ok && span(use, 1, &t1) && span(use, 1, &t1) && t1 > 0.f;  // the first run loads the kernel
        for (int j = 1; ok && j < kLanes; j++) {
            use[n] = j;
            ok = span(use, n + 1, &t);
            if (ok && t < 1.5f * t1) n++;
        }
        if (ok && n >= 1) {
            nlanes = n;
            for (int i = 0; i < n; i++) lane_use[i] = use[i];
        }
        if (e0) (void)hipEventDestroy(e0);
        for (auto& e : e1)
            if (e) (void)hipEventDestroy(e);
        if (buf) (void)hipFree(buf);
        (void)hipGetLastError();
        if (verbose())
            std::fprintf(stderr, "[jhq] search lanes: %d of %d on queues of their own\n", nlanes,
                         kLanes);
    }

    int ensure_stream() {
        if (stream) return JHQ_OK;
        int ndev = 0;
        if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
            return fail(JHQ_EDEVICE, "no HIP device available");
        int dev = 0;
        JHQ_HIP(hipGetDevice(&dev));
        hipDeviceProp_t prop;
        JHQ_HIP(hipGetDeviceProperties(&prop, dev));
        num_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
        JHQ_HIP(hipStreamCreate(&stream));
        JHQ_HIP(hipEventCreateWithFlags(&done_ev, hipEventDisableTiming));
        JHQ_HIP(hipEventCreateWithFlags(&tail_ev, hipEventDisableTiming));
        JHQ_HIP(hipEventCreateWithFlags(&from_ev, hipEventDisableTiming));
        for (auto& e : ldesc_ev) JHQ_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        return JHQ_OK;
    }

    // Blocks until the last device search has finished with the lists and
    // workspaces.
    int quiesce_searches() {
        if (!done_pending) return JHQ_OK;
        JHQ_HIP(hipEventSynchronize(done_ev));
        done_pending = false;
        return JHQ_OK;
    }

    // Blocks until the last device search and the last insert's (or row
    // refresh's) enqueued work have finished.
    int quiesce() {
        JHQ_TRY(quiesce_searches());
        if (!tail_pending) return JHQ_OK;
        JHQ_HIP(hipEventSynchronize(tail_ev));
        tail_pending = false;
        return JHQ_OK;
    }

    // Marks the work enqueued on `stream` so far as the tail device searches
    // and host accesses wait for.
    int mark_tail() {
        JHQ_HIP(hipEventRecord(tail_ev, stream));
        tail_pending = true;
        return JHQ_OK;
    }
};

namespace {

int ceil_ck(float alpha, int k) {
    const int c = static_cast<int>(std::ceil(alpha * static_cast<float>(k)));
    return std::max(k, c);
}

// Host pinned buffer growth.
template <class T>
int ensure_pinned(T*& p, size_t& cap, size_t n) {
    if (p && cap >= n) return JHQ_OK;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    cap = 0;
    JHQ_HIP(hipHostMalloc(reinterpret_cast<void**>(&p), std::max<size_t>(n, 1) * sizeof(T),
                          hipHostMallocDefault));
    cap = n;
    return JHQ_OK;
}

// assign rows of d_y (device, [n x d]) to the nearest of the index's centroids.
// The list of each row of d_y: on MFMA with the fixed-order re-check where it
// applies (d % 4 == 0), else the fixed-order kernel alone; the same result.
int assign_rows(jhq_index* ix, const float* d_y, int64_t n, int32_t* d_assign,
                DBuf<unsigned long long>& keys) {
    JHQ_TRY(keys.ensure(static_cast<size_t>(n)));
    if (jhq::assign_mfma_ok(ix->d, d_y, ix->dcent.p) && (n + 127) / 128 <= 65535) {
        JHQ_TRY(ix->dascr.ensure(jhq::assign_mfma_scratch_floats(n, ix->d, ix->nlist)));
        JHQ_HIP(jhq::assign_mfma(d_y, n, ix->d, ix->dcent.p, ix->nlist, ix->dnorms.p, d_assign,
                                 ix->dascr.p, ix->dascr.n, keys.p, ix->stream));
        if (verbose() && ix->drecheck.p)
            JHQ_HIP(jhq::assign_mfma_tally(ix->dascr.p, n, ix->drecheck.p, ix->stream));
        return JHQ_OK;
    }
    JHQ_HIP(jhq::fill_u64(keys.p, n, ~0ull, ix->stream));
    JHQ_HIP(jhq::gemm_nt_argmin(d_y, ix->d, ix->dcent.p, ix->d, n, ix->nlist, ix->d, ix->dnorms.p,
                                keys.p, ix->stream));
    JHQ_HIP(jhq::keys_to_assign(keys.p, n, d_assign, ix->stream));
    return JHQ_OK;
}

void compute_norms(jhq_index* ix) {
    ix->cent_norms.assign(ix->nlist, 0.f);
    for (int c = 0; c < ix->nlist; c++) {
        double s = 0.0;
        const float* cc = ix->cent.data() + static_cast<int64_t>(c) * ix->d;
        for (int j = 0; j < ix->d; j++) s += static_cast<double>(cc[j]) * static_cast<double>(cc[j]);
        ix->cent_norms[c] = static_cast<float>(s);
    }
}

int upload_centroids(jhq_index* ix) {
    compute_norms(ix);
    JHQ_TRY(ix->dcent.upload(ix->cent.data(), ix->cent.size()));
    JHQ_TRY(ix->dnorms.upload(ix->cent_norms.data(), ix->cent_norms.size()));
    return JHQ_OK;
}

// dqmat = [Pi ; cent * Pi]: row j < d is Pi's row j, row d + l is centroid l
// taken back to the unrotated space (sum_j cent[l][j] Pi(j, k), a fixed-order
// fmaf chain), so that <q, row d + l> = <c_l, Pi q>.  Only where the
// 64-row MFMA product applies (d % 64 == 0).
int build_query_matrix(jhq_index* ix) {
    const int d = ix->d, nlist = ix->nlist;
    ix->dqmat.release();
    if (!jhq::mfma_q_ok(d, d, d)) return JHQ_OK;
    JHQ_TRY(ix->ensure_stream());
    JHQ_TRY(ix->dqmat.alloc(static_cast<size_t>(d + nlist) * d));
    DBuf<float> dpt;
    JHQ_TRY(dpt.upload(ix->Pi_cm.data(), ix->Pi_cm.size()));  // row k = (Pi(0,k), Pi(1,k), ...)
    JHQ_HIP(hipMemcpyAsync(ix->dqmat.p, ix->dP.p, static_cast<size_t>(d) * d * sizeof(float),
                           hipMemcpyDeviceToDevice, ix->stream));
    JHQ_HIP(jhq::gemm_nt_store(ix->dcent.p, d, dpt.p, d, nlist, d, d,
                               ix->dqmat.p + static_cast<size_t>(d) * d, d, false, ix->stream));
    JHQ_HIP(hipStreamSynchronize(ix->stream));
    return JHQ_OK;
}

// v14/jhq_gpu_index.cu:228-299 — coarse k-means in rotated space, on the
// device: init rows c * n / nlist; each iteration assigns with the current
// centroids and norms, then takes the means (double, ascending rows) or
// reseeds empty lists.  The host copies are read back at the end.
int train_ivf(jhq_index* ix, const float* d_y, int64_t n) {
    const int d = ix->d, nlist = ix->nlist;
    hipStream_t s = ix->stream;
    JHQ_TRY(ix->dcent.alloc(static_cast<size_t>(nlist) * d));
    JHQ_TRY(ix->dnorms.alloc(static_cast<size_t>(nlist)));
    JHQ_HIP(jhq::kmeans_init(d_y, d, n, nlist, ix->dcent.p, s));
    DBuf<int32_t> dasg;
    DBuf<unsigned long long> keys;
    DBuf<unsigned char> scratch;
    JHQ_TRY(dasg.alloc(static_cast<size_t>(n)));
    const size_t sb = jhq::kmeans_scratch_bytes(n, nlist);
    JHQ_TRY(scratch.alloc(sb));
    for (int iter = 0; iter < ix->ivf_iters; iter++) {
        if (verbose())
            std::fprintf(stderr, "[jhq] train: IVF k-means iteration %d/%d (nlist %d, n %lld)\n",
                         iter + 1, ix->ivf_iters, nlist, static_cast<long long>(n));
        JHQ_HIP(jhq::kmeans_norms(ix->dcent.p, d, nlist, ix->dnorms.p, s));
        JHQ_TRY(assign_rows(ix, d_y, n, dasg.p, keys));
        JHQ_HIP(jhq::kmeans_update(dasg.p, d_y, d, n, nlist, iter, ix->dcent.p, scratch.p, sb, s));
    }
    JHQ_HIP(jhq::kmeans_norms(ix->dcent.p, d, nlist, ix->dnorms.p, s));
    ix->cent.resize(static_cast<size_t>(nlist) * d);
    ix->cent_norms.resize(static_cast<size_t>(nlist));
    JHQ_HIP(hipMemcpyAsync(ix->cent.data(), ix->dcent.p, ix->cent.size() * sizeof(float),
                           hipMemcpyDeviceToHost, s));
    JHQ_HIP(hipMemcpyAsync(ix->cent_norms.data(), ix->dnorms.p, ix->cent_norms.size() * sizeof(float),
                           hipMemcpyDeviceToHost, s));
    JHQ_HIP(hipStreamSynchronize(s));
    return JHQ_OK;
}

// A workspace buffer of at least `count` elements: grown when `grow`, else
// it must already be that large (a search outside the reserved shape).
template <class T>
int need(DBuf<T>& b, size_t count, bool grow) {
    if (b.has(count)) return JHQ_OK;
    if (grow) return b.alloc(count);
    return fail(JHQ_ESTATE,
                "the search needs a larger workspace than was reserved; call jhq_reserve() "
                "with this k (after any set_nprobe / set_alpha) before a device search");
}

int ensure_workspace(jhq_index* ix, Workspace& w, int ck, int k, int P, int max_segments,
                     bool grow) {
    const size_t B = static_cast<size_t>(ix->batch_size);
    JHQ_TRY(need(w.wq, B * ix->d, grow));
    JHQ_TRY(need(w.wqrot, B * ix->d, grow));
    JHQ_TRY(need(w.wscores, B * ix->nlist, grow));
    JHQ_TRY(need(w.wprobes, B * P, grow));
    JHQ_TRY(need(w.wgofs, B * (P + 1), grow));
    JHQ_TRY(need(w.wqtot, B, grow));
    JHQ_TRY(need(w.wpartial, static_cast<size_t>(max_segments) * ck, grow));
    JHQ_TRY(need(w.wpslot, static_cast<size_t>(max_segments) * ck, grow));
    JHQ_TRY(need(w.wtopck, B * ck, grow));
    JHQ_TRY(need(w.wout_d, B * k, grow));
    JHQ_TRY(need(w.wout_i, B * k, grow));
    if (ix->dqmat.p) {
        // split sums for kQbShare batches (a device search's lanes run the
        // product once for consecutive batches)
        const size_t pf =
            jhq::mfma_qb_space(ix->batch_size * kQbShare, ix->d + ix->nlist, ix->d);
        if (pf) JHQ_TRY(need(w.wqpart, pf, grow));
    }
    return JHQ_OK;
}

bool skew_eligible(const jhq_index* ix) { return ix->M % 32 == 0 && ix->M <= 128; }

bool rows_wanted(const jhq_index* ix);

// The pre-scan computes 16-query tiles over every probed list; it pays off
// when the queries of a batch share their lists so that the tiles are mostly
// full, and when the byte-LUT scan's work per candidate (M gathers) is large
// against the re-check's (one 4-byte value per candidate, read by the
// query's one workgroup).  Measured: 1M x 1024 (M 128, nlist 4096, batch 64,
// 1.2 rows per pair, 51 K to 200 K candidates per query): 1.5-1.6x the
// byte-LUT scan's QPS at nprobe 16 to 64 and ck 100 to 400; 11M x 768 (M 96,
// batch 128, 237 K candidates per query): 1.39x at ck 400 and 1.30x at
// ck 1000; 10M x 128 uint8 (M 16, 420 K candidates per query, 2.1 rows per
// pair): 11x slower; one query per batch: equal.  Longer short lists than
// 1024 were not measured.
constexpr double kMfmaMaxTileCost = 3.0;
constexpr int kMfmaMinM = 64;
constexpr int kMfmaMaxCk = 1024;

// The row-major code copy serves the pre-scan's re-check: kept where the
// pre-scan can run and the scan kind may choose it.
bool rows_wanted(const jhq_index* ix) {
    return ix->K1D == 2 && ix->Ds == 8 && ix->bpd == 1 && ix->M % 16 == 0 && ix->M <= 128 &&
           (ix->scan_kind == 2 || (ix->scan_kind == 0 && ix->M >= kMfmaMinM));
}

// Rows computed per real (query, candidate) pair for batches of B queries
// with P probes, measured on stored vectors taken as queries: up to 8
// batches of B vectors spread over the index, each decoded from its primary
// code (the rotated-space levels of its digits), their P nearest lists
// selected as a search selects them, and per batch
//   rows = sum over distinct lists of 16 ceil(queries / 16) ceil(size / 16),
//   pairs = sum over probes of ceil(size / 16),
// and the mean candidates per query.
int mfma_measure_cost(jhq_index* ix, int B, int P, double* cost, double* cand) {
    const int64_t n = ix->ntotal;
    const int nb = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(8, n / std::max(B, 1))));
    const int S = static_cast<int>(std::min<int64_t>(static_cast<int64_t>(nb) * B, n));
    const int nlist = ix->nlist, d = ix->d;
    std::vector<int64_t> cpre(nlist + 1, 0);
    for (int l = 0; l < nlist; l++) cpre[l + 1] = cpre[l] + ix->l_size[l];
    std::vector<int4> samp(S);
    for (int i = 0; i < S; i++) {
        // canonical positions spread by a multiplicative hash
        const int64_t pos = static_cast<int64_t>((static_cast<uint64_t>(i) * 2654435761ull +
                                                  12345ull) % static_cast<uint64_t>(n));
        const int l = static_cast<int>(std::upper_bound(cpre.begin(), cpre.end(), pos) -
                                       cpre.begin()) - 1;
        samp[i] = make_int4(ix->l_start[l], ix->l_cap[l], static_cast<int>(pos - cpre[l]), 0);
    }
    DBuf<int4> dsamp;
    DBuf<float> rows, scores;
    DBuf<int32_t> probes, gofs, qtot;
    JHQ_TRY(dsamp.upload(samp.data(), samp.size()));
    JHQ_TRY(rows.alloc(static_cast<size_t>(S) * d));
    JHQ_TRY(scores.alloc(static_cast<size_t>(S) * nlist));
    JHQ_TRY(probes.alloc(static_cast<size_t>(S) * P));
    JHQ_TRY(gofs.alloc(static_cast<size_t>(S) * (P + 1)));
    JHQ_TRY(qtot.alloc(static_cast<size_t>(S)));
    hipStream_t st = ix->stream;
    JHQ_HIP(jhq::decode_rows(dsamp.p, S, ix->dcodes_t.p, ix->M, ix->Ds, ix->K1D, ix->bpd,
                             ix->dc1d.p, rows.p, st));
    JHQ_HIP(jhq::mfma_nt_score(rows.p, d, ix->dcent.p, d, S, nlist, d, ix->dnorms.p, scores.p,
                               nlist, st));
    JHQ_HIP(jhq::select_probes(scores.p, S, nlist, P, ix->dldesc.p, probes.p, gofs.p, qtot.p, st));
    std::vector<int32_t> hp(static_cast<size_t>(S) * P);
    JHQ_HIP(hipMemcpyAsync(hp.data(), probes.p, hp.size() * sizeof(int32_t),
                           hipMemcpyDeviceToHost, st));
    JHQ_HIP(hipStreamSynchronize(st));
    double rows_sum = 0.0, pairs = 0.0, cands = 0.0;
    std::vector<int> cnt(nlist, 0);
    for (int b0 = 0; b0 < S; b0 += B) {
        const int b1 = std::min(S, b0 + B);
        for (int i = b0 * P; i < b1 * P; i++) cnt[hp[i]]++;
        for (int i = b0 * P; i < b1 * P; i++) {
            const int l = hp[i];
            const double tiles = (ix->l_size[l] + jhq::kGroup - 1) / jhq::kGroup;
            pairs += tiles;
            cands += ix->l_size[l];
            if (cnt[l] > 0) {
                rows_sum += 16.0 * ((cnt[l] + 15) / 16) * tiles;
                cnt[l] = 0;  // counted once per batch
            }
        }
    }
    *cost = pairs > 0.0 ? rows_sum / pairs : 1e30;
    *cand = cands / S;
    return JHQ_OK;
}

// Whether a batch of Bq queries (P probes, short list ck) runs the pre-scan.
// measure = false (device searches, plan queries): the cached choice only.
int mfma_choose(jhq_index* ix, int Bq, int P, int ck, bool measure, bool* use) {
    *use = false;
    if (ix->scan_kind == 1 ||
        !jhq::mfma_scan_ok(ix->M, ix->d, ix->Ds, ix->K1D, ix->bpd, Bq, P, ck, ix->RC * ix->Kr))
        return JHQ_OK;
    if (ix->scan_kind == 2) {
        *use = true;
        return JHQ_OK;
    }
    if (ck > kMfmaMaxCk || ix->M < kMfmaMinM)
        return JHQ_OK;
    const int B = ix->batch_size;
    const bool cached = ix->mfma_dec_B == B && ix->mfma_dec_P == P && ix->mfma_dec_n > 0 &&
                        ix->ntotal * 5 >= ix->mfma_dec_n * 4 && ix->ntotal * 4 <= ix->mfma_dec_n * 5;
    if (!cached && measure && ix->ntotal > 0) {
        JHQ_TRY(mfma_measure_cost(ix, B, P, &ix->mfma_dec_cost, &ix->mfma_dec_cand));
        ix->mfma_dec_B = B;
        ix->mfma_dec_P = P;
        ix->mfma_dec_n = ix->ntotal;
        if (verbose())
            std::fprintf(stderr,
                         "[jhq] plan: pre-scan %.2f rows per pair, %.0f candidates per query "
                         "(batch %d, %d probes): %s\n",
                         ix->mfma_dec_cost, ix->mfma_dec_cand, B, P,
                         ix->mfma_dec_cost <= kMfmaMaxTileCost ? "pre-scan" : "byte-LUT scan");
    }
    *use = (cached || (measure && ix->ntotal > 0)) && ix->mfma_dec_cost <= kMfmaMaxTileCost;
    return JHQ_OK;
}

// Brings the skewed copy up to date: rows appended since the last refresh,
// and every row of a list whose block moved (or of every list when the copy
// had to grow).  Synchronous, so any stream may read the copy afterwards.
int refresh_skew(jhq_index* ix) {
    if (!ix->skew_stale) return JHQ_OK;
    const int nl = ix->nlist;
    const size_t need = static_cast<size_t>(jhq::skew_bytes(std::max<int64_t>(ix->pool_cap, 1), ix->M));
    if (ix->dcodes_s.n < need || static_cast<int>(ix->skew_start.size()) != nl) {
        if (ix->dcodes_s.n < need) JHQ_TRY(ix->dcodes_s.alloc(need));
        ix->skew_start.assign(nl, -1);
        ix->skew_rows.assign(nl, 0);
    }
    std::vector<int32_t> from(nl);
    int max_rows = 0;
    for (int l = 0; l < nl; l++) {
        from[l] = ix->skew_start[l] == ix->l_start[l] ? std::min(ix->skew_rows[l], ix->l_size[l]) : 0;
        max_rows = std::max(max_rows, ix->l_size[l] - from[l]);
    }
    if (max_rows > 0) {
        JHQ_TRY(ix->dskew_from.ensure(nl));
        JHQ_HIP(hipMemcpyAsync(ix->dskew_from.p, from.data(), nl * sizeof(int32_t),
                               hipMemcpyHostToDevice, ix->stream));
        JHQ_HIP(jhq::skew_codes(ix->dldesc.p, ix->dskew_from.p, nl, max_rows, ix->dcodes_t.p, ix->M,
                                ix->dcodes_s.p, ix->stream));
        JHQ_HIP(hipStreamSynchronize(ix->stream));
    }
    ix->skew_start = ix->l_start;
    ix->skew_rows = ix->l_size;
    ix->skew_stale = false;
    return JHQ_OK;
}

// Brings the row-major copy up to date: rows a list gained since the last
// refresh (all of a list that moved).
int refresh_rows(jhq_index* ix) {
    if (!ix->rows_stale) return JHQ_OK;
    const int nl = ix->nlist;
    const size_t need = static_cast<size_t>((std::max<int64_t>(ix->pool_cap, 1) + 15) / 16 * 16) *
                        static_cast<size_t>(ix->M);
    if (ix->dcodes_r.n < need || static_cast<int>(ix->rows_start.size()) != nl) {
        // (the old copy may still be read by enqueued work)
        if (ix->dcodes_r.n < need) {
            JHQ_TRY(ix->quiesce());
            JHQ_TRY(ix->dcodes_r.alloc(need));
        }
        ix->rows_start.assign(nl, -1);
        ix->rows_rows.assign(nl, 0);
    }
    std::vector<int32_t> from(nl);
    int max_rows = 0;
    for (int l = 0; l < nl; l++) {
        from[l] = ix->rows_start[l] == ix->l_start[l] ? std::min(ix->rows_rows[l], ix->l_size[l]) : 0;
        max_rows = std::max(max_rows, ix->l_size[l] - from[l]);
    }
    if (max_rows > 0) {
        // enqueued only (from pinned staging): device searches wait for the
        // tail event, host searches run on the same stream or lanes forked
        // from it
        if (ix->from_pending) JHQ_HIP(hipEventSynchronize(ix->from_ev));
        ix->from_pending = false;
        JHQ_TRY(ensure_pinned(ix->h_from, ix->h_from_n, static_cast<size_t>(nl)));
        std::memcpy(ix->h_from, from.data(), nl * sizeof(int32_t));
        JHQ_TRY(ix->drows_from.ensure(nl));
        JHQ_HIP(hipMemcpyAsync(ix->drows_from.p, ix->h_from, nl * sizeof(int32_t),
                               hipMemcpyHostToDevice, ix->stream));
        JHQ_HIP(hipEventRecord(ix->from_ev, ix->stream));
        ix->from_pending = true;
        JHQ_HIP(jhq::row_codes(ix->dldesc.p, ix->drows_from.p, nl, max_rows, ix->dcodes_t.p, ix->M,
                               ix->dcodes_r.p, ix->stream));
        JHQ_TRY(ix->mark_tail());
    }
    ix->rows_start = ix->l_start;
    ix->rows_rows = ix->l_size;
    ix->rows_stale = false;
    return JHQ_OK;
}

struct BatchPlan {
    int ck, P;
    jhq::ScanShape sh;
};

// The plan of a search batch and the workspaces it needs on nws lanes.
// grow = false (device searches): nothing is allocated or refreshed, and a
// shape beyond the reservation fails with JHQ_ESTATE.
int plan_batch(jhq_index* ix, int Bq, int k, BatchPlan* bp, int nws, bool grow) {
    bp->ck = ceil_ck(ix->alpha, k);
    bp->P = std::min(ix->nprobe, ix->nlist);
    bool use_mfma = false;
    JHQ_TRY(mfma_choose(ix, Bq, bp->P, bp->ck, grow, &use_mfma));
    if (!jhq::scan_plan(ix->M, ix->d, bp->P, bp->ck, ix->K1D, Bq, ix->num_cu, &bp->sh,
                        skew_eligible(ix), use_mfma, ix->RC * ix->Kr))
        return fail(JHQ_EINVAL, "M=" + std::to_string(ix->M) + ", ck=" + std::to_string(bp->ck) +
                                    ", batch=" + std::to_string(Bq) +
                                    ": the byte LUT and selection buffers do not fit in LDS");
    if (bp->sh.skew && ix->skew_stale) {
        if (!grow) return fail(JHQ_ESTATE, "the skewed code copy is out of date");
        JHQ_TRY(refresh_skew(ix));
    }
    if (bp->sh.mfma && ix->rows_stale) {
        if (!grow) return fail(JHQ_ESTATE, "the row-major code copy is out of date");
        JHQ_TRY(refresh_rows(ix));
    }
    for (int i = 0; i < nws; i++)
        JHQ_TRY(ensure_workspace(ix, ix->ws[i], bp->ck, k, bp->P, bp->sh.max_segments, grow));
    if (bp->sh.dump || bp->sh.mfma) {
        // a query's candidates are at most the padded sizes of the P largest
        // lists (cached per P; inserts reset the cache)
        if (ix->dump_P != bp->P) {
            std::vector<int32_t> sz(ix->l_size);
            std::partial_sort(sz.begin(), sz.begin() + bp->P, sz.end(), std::greater<int32_t>());
            int64_t per_q = 0;
            for (int i = 0; i < bp->P; i++)
                per_q += (sz[i] + jhq::kGroup - 1) / jhq::kGroup * jhq::kGroup;
            ix->dump_P = bp->P;
            ix->dump_perq = per_q;
        }
        // keys (dump scan) or biased integer distances (MFMA pre-scan)
        // (the pre-scan: u32 slots and one tile minimum per 16 after them)
        // (grown with an eighth to spare: appends lengthen the lists a little
        // at a time, and each reallocation here is one per lane)
        const size_t slots = static_cast<size_t>(Bq) * std::max<int64_t>(ix->dump_perq, 1);
        const size_t words = bp->sh.mfma ? (slots + slots / 16 + 40) / 2 : slots;
        for (int i = 0; i < nws; i++)
            if (!ix->ws[i].wdump.has(words))
                JHQ_TRY(need(ix->ws[i].wdump, grow ? words + words / 8 : words, grow));
        if (bp->sh.mfma)
            for (int i = 0; i < nws; i++)
                JHQ_TRY(need(ix->ws[i].wmfma, jhq::mfma_scan_bytes(Bq, bp->P, ix->M, ix->num_cu),
                             grow));
    }
    return JHQ_OK;
}

// One batch of Bq queries at d_q (device) through the whole pipeline
// (the graph body of v14/search.cu:315-386).  share: the query product of
// share.rows consecutive queries (this batch's first, share.row0 = 0) runs
// once, and the later batches of the group (share.row0 = their first row)
// take their split sums from it; share.rows = 0: the batch's own product.
struct QbShare {
    int rows = 0, row0 = 0;
};
int run_batch(jhq_index* ix, Workspace& w, const float* d_q, int Bq, int k, const BatchPlan& bp,
              float* d_out, int32_t* d_ids, bool want_topck, hipStream_t s,
              QbShare share = QbShare{}) {
    const int d = ix->d;
    if (ix->timing) JHQ_HIP(hipEventRecord(ix->ev[0], s));
    // rotation and centroid dots in one tiled product; its split sums are
    // added by the probe selection where the score row fits in its LDS
    jhq::QbPlan qp{};
    bool sel_qb = false;
    const int qrows = share.rows > 0 ? share.rows : Bq;
    // the pre-scan: the selection also quantizes the queries and lists the
    // batch's (query, probe) pairs in the workspace's list hash
    const int64_t dump_slots = static_cast<int64_t>(w.wdump.n * 2 / 17 * 16);
    jhq::PrescanSel ps{w.wmfma.p, w.wmfma.n, dump_slots, w.wqrot.p, ix->dc1d.p, d, ix->M,
                       ix->batch_size};
    if (bp.sh.mfma) {
        if (!w.hash_clear || w.hash_P != bp.P || w.hash_ws != w.wmfma.p)
            JHQ_HIP(jhq::mfma_hash_clear(ix->batch_size, bp.P, ix->M, w.wmfma.p, w.wmfma.n, s));
        w.hash_clear = false;
        w.hash_P = bp.P;
        w.hash_ws = w.wmfma.p;
    }
    if (ix->dqmat.p) {
        qp = jhq::mfma_qb_plan(qrows, d + ix->nlist, d);
        sel_qb = jhq::select_adds_qb(qp, ix->nlist, d);
        // a shared product leaves its sums split (the selection adds them)
        if (share.rows > 0 && (!sel_qb || share.row0 + Bq > qrows))
            return fail(JHQ_EINVAL, "query product shared where the selection does not add it");
        if (share.row0 == 0)
            JHQ_HIP(jhq::mfma_qb(qp, d_q, d, ix->dqmat.p, d, qrows, d + ix->nlist, d, d,
                                 w.wqrot.p, d, w.wscores.p, ix->nlist, ix->dnorms.p, w.wqpart.p,
                                 w.wqpart.n, s, !sel_qb));
    } else {
        // d not a multiple of 64: the 16-row kernels
        JHQ_HIP(jhq::mfma_nt_store(d_q, d, ix->dP.p, d, Bq, d, d, w.wqrot.p, d, s));
        JHQ_HIP(jhq::mfma_nt_score(w.wqrot.p, d, ix->dcent.p, d, Bq, ix->nlist, d, ix->dnorms.p,
                                   w.wscores.p, ix->nlist, s));
    }
    if (ix->timing) JHQ_HIP(hipEventRecord(ix->ev[1], s));
    const jhq::PrescanSel* psp = bp.sh.mfma ? &ps : nullptr;
    if (sel_qb)
        JHQ_HIP(jhq::select_probes_qb(qp, w.wqpart.p + static_cast<size_t>(share.row0) *
                                                           (d + ix->nlist),
                                      d, w.wqrot.p, d, ix->dnorms.p, Bq, ix->nlist, bp.P,
                                      ix->dldesc.p, w.wprobes.p, w.wgofs.p, w.wqtot.p, s, psp));
    else
        JHQ_HIP(jhq::select_probes(w.wscores.p, Bq, ix->nlist, bp.P, ix->dldesc.p, w.wprobes.p,
                                   w.wgofs.p, w.wqtot.p, s, psp));
    if (ix->timing) JHQ_HIP(hipEventRecord(ix->ev[2], s));
    if (bp.sh.mfma) {
        // the re-check refines short short lists itself
        JHQ_HIP(jhq::mfma_scan(w.wqrot.p, d, ix->Ds, ix->K1D, ix->bpd, ix->dc1d.p, Bq, ix->M,
                               w.wprobes.p, w.wgofs.p, w.wqtot.p, bp.P, ix->dldesc.p,
                               ix->dcodes_t.p,
                               ix->dcodes_r.p, bp.ck, reinterpret_cast<uint32_t*>(w.wdump.p),
                               dump_slots, w.wmfma.p, w.wmfma.n, k, ix->dres_c1d.p, ix->Kr,
                               ix->RC, ix->Br, ix->bpv, ix->dres.p, ix->dcorr.p,
                               ix->dlist_ids.p, d_out, d_ids, want_topck ? w.wtopck.p : nullptr,
                               w.wpartial.p, w.wpslot.p, ix->num_cu, ix->batch_size, s));
        // the re-check clears the hash for the lane's next batch
        w.hash_clear = true;
        if (ix->timing) JHQ_HIP(hipEventRecord(ix->ev[3], s));
        if (!jhq::mfma_fuses_refine(bp.ck))
            JHQ_HIP(jhq::refine_topk(w.wpartial.p, w.wpslot.p, w.wqtot.p, Bq, bp.sh, bp.ck, k,
                                     w.wqrot.p, d, ix->Ds, ix->dres_c1d.p, ix->Kr, ix->RC, ix->Br,
                                     ix->bpv, ix->dldesc.p, ix->nlist, ix->dres.p, ix->dcorr.p,
                                     ix->dlist_ids.p, d_out, d_ids,
                                     want_topck ? w.wtopck.p : nullptr, s));
    } else {
        JHQ_HIP(jhq::scan_topck(w.wqrot.p, d, ix->Ds, ix->K1D, ix->bpd, ix->dc1d.p, Bq, ix->M,
                                w.wprobes.p, w.wgofs.p, w.wqtot.p, bp.P, ix->dldesc.p,
                                ix->dcodes_t.p, bp.ck, bp.sh, w.wpartial.p, w.wpslot.p,
                                w.wdump.p, ix->dcodes_s.p, s));
        if (ix->timing) JHQ_HIP(hipEventRecord(ix->ev[3], s));
        JHQ_HIP(jhq::refine_topk(w.wpartial.p, w.wpslot.p, w.wqtot.p, Bq, bp.sh, bp.ck, k,
                                 w.wqrot.p, d, ix->Ds, ix->dres_c1d.p, ix->Kr, ix->RC, ix->Br,
                                 ix->bpv, ix->dldesc.p, ix->nlist, ix->dres.p, ix->dcorr.p,
                                 ix->dlist_ids.p, d_out, d_ids, want_topck ? w.wtopck.p : nullptr,
                                 s));
    }
    if (ix->timing) {
        JHQ_HIP(hipEventRecord(ix->ev[kSteps], s));
        JHQ_HIP(hipEventSynchronize(ix->ev[kSteps]));
        for (int i = 0; i < kSteps; i++) {
            float ms = 0.f;
            JHQ_HIP(hipEventElapsedTime(&ms, ix->ev[i], ix->ev[i + 1]));
            ix->tms[i] += ms;
        }
        ix->tbatches++;
    }
    return JHQ_OK;
}

int check_searchable(jhq_index* ix, int64_t nq, int k) {
    if (!ix) return fail(JHQ_EINVAL, "null index");
    if (ix->broken)
        return fail(JHQ_ESTATE, "a failed add/append left the index's lists inconsistent");
    if (ix->ntotal == 0) return fail(JHQ_ESTATE, "index is empty");
    if (nq < 0) return fail(JHQ_EINVAL, "nq must be >= 0");
    if (k <= 0) return fail(JHQ_EINVAL, "k must be positive");
    return JHQ_OK;
}

int ensure_host_staging(jhq_index* ix, int l, int Bmax, int k) {
    JHQ_TRY(ensure_pinned(ix->h_q[l], ix->h_q_n[l], static_cast<size_t>(Bmax) * ix->d));
    JHQ_TRY(ensure_pinned(ix->h_d[l], ix->h_d_n[l], static_cast<size_t>(Bmax) * k));
    JHQ_TRY(ensure_pinned(ix->h_i[l], ix->h_i_n[l], static_cast<size_t>(Bmax) * k));
    return JHQ_OK;
}

// The skewed code copy serves only the byte-LUT scan of M % 32 == 0.  A
// device search plans its batches at the index's batch size with its own k
// (k <= res_k), so when the pre-scan is the scan for every such k no device
// search reads the copy: it is then neither built nor refreshed at
// reservation (appends at config 5's shape skip it), and a host search that
// needs it refreshes it itself.
bool skew_needed(jhq_index* ix) {
    if (!skew_eligible(ix)) return false;
    const int P = std::min(ix->nprobe, ix->nlist);
    for (int k = 1; k <= ix->res_k; k++) {
        bool mf = false;
        if (mfma_choose(ix, ix->batch_size, P, ceil_ck(ix->alpha, k), true, &mf) != JHQ_OK || !mf)
            return true;
    }
    return false;
}

// Preallocates everything a search with k <= res_k needs (the reference's
// alloc_workspace at the end of add(), v14/jhq_gpu_index.cu:166-206,531, and
// realloc_ck_buffers, v14/search.cu:294-313): every lane's workspace, stream
// and pinned staging, and an up-to-date skewed code copy.  Called after every
// add / append / load and parameter change, so device searches allocate
// nothing.
int reserve_search(jhq_index* ix) {
    if (ix->ntotal == 0 || !ix->trained) return JHQ_OK;
    // workspaces may be regrown: no device search may be using them (an
    // insert's enqueued tail does not read them; the refreshes below are
    // enqueued behind it)
    JHQ_TRY(ix->quiesce_searches());
    if (ix->skew_stale && skew_needed(ix)) JHQ_TRY(refresh_skew(ix));
    if (rows_wanted(ix) && ix->rows_stale) JHQ_TRY(refresh_rows(ix));
    BatchPlan bp;
    JHQ_TRY(plan_batch(ix, ix->batch_size, ix->res_k, &bp, kLanes, true));
    JHQ_TRY(ix->ensure_lanes());
    for (int l = 0; l < kLanes; l++) JHQ_TRY(ensure_host_staging(ix, l, ix->batch_size, ix->res_k));
    return JHQ_OK;
}

// Host arrays over several batches: the batches rotate through the lanes
// (workspace, pinned staging, stream).  While the other lanes' batches run,
// the host copies a lane's finished results out and its next queries in.
int search_host_pipelined(jhq_index* ix, const float* q, int64_t nq, int k, float* dists,
                          int32_t* ids) {
    const int d = ix->d;
    const int Bmax = ix->batch_size;
    BatchPlan bp;
    JHQ_TRY(plan_batch(ix, Bmax, k, &bp, kLanes, true));
    JHQ_TRY(ix->ensure_lanes());
    for (int l = 0; l < kLanes; l++) JHQ_TRY(ensure_host_staging(ix, l, Bmax, k));
    const int nl = ix->nlanes;
    JHQ_HIP(hipEventRecord(ix->lane_ev[0], ix->stream));
    for (int i = 0; i < nl; i++)
        JHQ_HIP(hipStreamWaitEvent(ix->lane[ix->lane_use[i]], ix->lane_ev[0], 0));
    int64_t pend_q0[kLanes];
    int pend_b[kLanes];
    for (int l = 0; l < kLanes; l++) {
        pend_q0[l] = -1;
        pend_b[l] = 0;
    }
    auto collect = [&](int l) -> int {
        if (pend_q0[l] < 0) return JHQ_OK;
        JHQ_HIP(hipEventSynchronize(ix->lane_ev[1 + l]));
        std::memcpy(dists + pend_q0[l] * k, ix->h_d[l], static_cast<size_t>(pend_b[l]) * k * sizeof(float));
        std::memcpy(ids + pend_q0[l] * k, ix->h_i[l], static_cast<size_t>(pend_b[l]) * k * sizeof(int32_t));
        pend_q0[l] = -1;
        return JHQ_OK;
    };
    int64_t bi = 0;
    for (int64_t q0 = 0; q0 < nq; q0 += Bmax, bi++) {
        const int Bq = static_cast<int>(std::min<int64_t>(Bmax, nq - q0));
        const int l = ix->lane_use[bi % nl];
        Workspace& w = ix->ws[l];
        hipStream_t st = ix->lane[l];
        JHQ_TRY(collect(l));  // the lane's previous batch is done: its buffers are free
        std::memcpy(ix->h_q[l], q + q0 * d, static_cast<size_t>(Bq) * d * sizeof(float));
        JHQ_HIP(hipMemcpyAsync(w.wq.p, ix->h_q[l], static_cast<size_t>(Bq) * d * sizeof(float),
                               hipMemcpyHostToDevice, st));
        JHQ_TRY(run_batch(ix, w, w.wq.p, Bq, k, bp, w.wout_d.p, w.wout_i.p, false, st));
        JHQ_HIP(hipMemcpyAsync(ix->h_d[l], w.wout_d.p, static_cast<size_t>(Bq) * k * sizeof(float),
                               hipMemcpyDeviceToHost, st));
        JHQ_HIP(hipMemcpyAsync(ix->h_i[l], w.wout_i.p, static_cast<size_t>(Bq) * k * sizeof(int32_t),
                               hipMemcpyDeviceToHost, st));
        JHQ_HIP(hipEventRecord(ix->lane_ev[1 + l], st));
        pend_q0[l] = q0;
        pend_b[l] = Bq;
    }
    // the pending batches, oldest first
    for (int j = 0; j < nl; j++) JHQ_TRY(collect(ix->lane_use[(bi + j) % nl]));
    for (int i = 0; i < nl; i++)
        JHQ_HIP(hipStreamWaitEvent(ix->stream, ix->lane_ev[1 + ix->lane_use[i]], 0));
    return JHQ_OK;
}

int search_host(jhq_index* ix, const float* q, int64_t nq, int k, float* dists, int32_t* ids,
                float* q_rot, int32_t* probes, int32_t* topck_pos, float* topck_dist) {
    JHQ_TRY(check_searchable(ix, nq, k));
    if (nq == 0) return JHQ_OK;
    // a device search may still use the workspaces, which a larger k regrows
    JHQ_TRY(ix->quiesce());
    const int d = ix->d;
    const int Bmax = ix->batch_size;
    const bool dbg = (q_rot || probes || topck_pos || topck_dist);
    if (!dbg && !ix->timing && nq > Bmax) return search_host_pipelined(ix, q, nq, k, dists, ids);
    BatchPlan bp;
    JHQ_TRY(plan_batch(ix, Bmax, k, &bp, 1, true));
    JHQ_TRY(ensure_host_staging(ix, 0, Bmax, k));
    std::vector<unsigned long long> tk;
    for (int64_t q0 = 0; q0 < nq; q0 += Bmax) {
        const int Bq = static_cast<int>(std::min<int64_t>(Bmax, nq - q0));
        std::memcpy(ix->h_q[0], q + q0 * d, static_cast<size_t>(Bq) * d * sizeof(float));
        JHQ_HIP(hipMemcpyAsync(ix->ws[0].wq.p, ix->h_q[0], static_cast<size_t>(Bq) * d * sizeof(float),
                               hipMemcpyHostToDevice, ix->stream));
        JHQ_TRY(run_batch(ix, ix->ws[0], ix->ws[0].wq.p, Bq, k, bp, ix->ws[0].wout_d.p,
                          ix->ws[0].wout_i.p, dbg, ix->stream));
        JHQ_HIP(hipMemcpyAsync(ix->h_d[0], ix->ws[0].wout_d.p, static_cast<size_t>(Bq) * k * sizeof(float),
                               hipMemcpyDeviceToHost, ix->stream));
        JHQ_HIP(hipMemcpyAsync(ix->h_i[0], ix->ws[0].wout_i.p, static_cast<size_t>(Bq) * k * sizeof(int32_t),
                               hipMemcpyDeviceToHost, ix->stream));
        JHQ_HIP(hipStreamSynchronize(ix->stream));
        std::memcpy(dists + q0 * k, ix->h_d[0], static_cast<size_t>(Bq) * k * sizeof(float));
        std::memcpy(ids + q0 * k, ix->h_i[0], static_cast<size_t>(Bq) * k * sizeof(int32_t));
        if (q_rot) {
            JHQ_HIP(hipMemcpy(q_rot + q0 * d, ix->ws[0].wqrot.p, static_cast<size_t>(Bq) * d * sizeof(float),
                              hipMemcpyDeviceToHost));
        }
        if (probes) {
            JHQ_HIP(hipMemcpy(probes + q0 * bp.P, ix->ws[0].wprobes.p,
                              static_cast<size_t>(Bq) * bp.P * sizeof(int32_t),
                              hipMemcpyDeviceToHost));
        }
        if (topck_pos || topck_dist) {
            tk.resize(static_cast<size_t>(Bq) * bp.ck);
            JHQ_HIP(hipMemcpy(tk.data(), ix->ws[0].wtopck.p, tk.size() * sizeof(unsigned long long),
                              hipMemcpyDeviceToHost));
            for (size_t i = 0; i < tk.size(); i++) {
                const unsigned long long kk = tk[i];
                const bool empty = (kk == ~0ull);
                const uint32_t hi = static_cast<uint32_t>(kk >> 32);
                uint32_t bits = hi & 0x7fffffffu;
                float f;
                std::memcpy(&f, &bits, 4);
                if (topck_pos) topck_pos[q0 * bp.ck + i] = empty ? -1 : static_cast<int32_t>(kk & 0xffffffffull);
                if (topck_dist) topck_dist[q0 * bp.ck + i] = empty ? INFINITY : f;
            }
        }
    }
    return JHQ_OK;
}

}  // namespace

// Sets the thread-local error message (for entry points in other files).
int jhq_set_error(int code, const char* msg) { return fail(code, msg ? msg : ""); }

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
extern "C" {

const char* jhq_last_error(void) { return g_err.c_str(); }

void jhq_params_default(jhq_params* p) {
    if (!p) return;
    p->M = 96;
    p->B = 8;
    p->Br = 4;
    p->alpha = 4.0f;
    p->nlist = 1024;
    p->nprobe = 8;
    p->ivf_iters = 8;
    p->batch_size = 256;
    p->seed = 42;
    p->add_batch = 65536;
    p->residual_per_subspace = 0;
}

int jhq_create(int d, const jhq_params* p, jhq_index** out) {
    if (!out) return fail(JHQ_EINVAL, "out must not be NULL");
    *out = nullptr;
    if (!p) return fail(JHQ_EINVAL, "params must not be NULL");
    // v14/jhq_gpu_index.cu:110-121, same checks, same order
    if (d <= 0) return fail(JHQ_EINVAL, "d must be positive");
    if (p->M <= 0) return fail(JHQ_EINVAL, "M must be positive");
    if (d % p->M != 0) return fail(JHQ_EINVAL, "d must be divisible by M");
    if (p->B % (d / p->M) != 0) return fail(JHQ_EINVAL, "B must be divisible by Ds = d/M");
    if (p->B > 8) return fail(JHQ_EINVAL, "B must be <= 8");
    if (p->Br != 4 && p->Br != 8) return fail(JHQ_EINVAL, "Br must be 4 or 8");
    if (p->nlist <= 0) return fail(JHQ_EINVAL, "nlist must be positive");
    if (p->nprobe <= 0) return fail(JHQ_EINVAL, "nprobe must be positive");
    if (p->ivf_iters <= 0) return fail(JHQ_EINVAL, "ivf_iters must be positive");
    if (p->batch_size <= 0) return fail(JHQ_EINVAL, "batch_size must be positive");
    if (p->add_batch <= 0) return fail(JHQ_EINVAL, "add_batch must be positive");
    if (!(p->alpha > 0.0f)) return fail(JHQ_EINVAL, "alpha must be positive");
    if (p->B <= 0) return fail(JHQ_EINVAL, "B must be positive");
    if (p->residual_per_subspace != 0 && p->residual_per_subspace != 1)
        return fail(JHQ_EINVAL, "residual_per_subspace must be 0 or 1");
    if (p->residual_per_subspace && p->M * (1 << p->Br) > 8192)
        return fail(JHQ_EINVAL, "per-subspace residual codebooks need M * 2^Br <= 8192");

    jhq_index* ix = new (std::nothrow) jhq_index();
    if (!ix) return fail(JHQ_ENOMEM, "host allocation failed");
    ix->d = d;
    ix->M = p->M;
    ix->B = p->B;
    ix->Br = p->Br;
    ix->nlist = p->nlist;
    ix->nprobe = std::min(p->nprobe, p->nlist);
    ix->ivf_iters = p->ivf_iters;
    ix->batch_size = p->batch_size;
    ix->seed = p->seed;
    ix->add_batch = p->add_batch;
    ix->alpha = p->alpha;
    ix->Ds = d / p->M;
    ix->bpd = p->B / ix->Ds;
    ix->K1D = 1 << ix->bpd;
    ix->Kr = 1 << p->Br;
    ix->bpv = (d * p->Br + 7) / 8;
    ix->RC = p->residual_per_subspace ? p->M : 1;
    ix->l_start.assign(ix->nlist, 0);
    ix->l_cap.assign(ix->nlist, 0);
    ix->l_size.assign(ix->nlist, 0);
    // JLTransform jl_(d, seed): the rotation is built with the index.
    ix->Pi_cm = jhq::build_rotation(d, p->seed);
    ix->P_rm.resize(static_cast<size_t>(d) * d);
    for (int j = 0; j < d; j++)
        for (int k = 0; k < d; k++)
            ix->P_rm[static_cast<size_t>(j) * d + k] = ix->Pi_cm[static_cast<size_t>(k) * d + j];
    *out = ix;
    return JHQ_OK;
}

int jhq_destroy(jhq_index* idx) {
    if (idx) (void)idx->quiesce();
    delete idx;
    return JHQ_OK;
}

int64_t jhq_ntotal(const jhq_index* idx) { return idx ? idx->ntotal : 0; }
int jhq_dim(const jhq_index* idx) { return idx ? idx->d : 0; }

int jhq_set_nprobe(jhq_index* idx, int nprobe) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (nprobe <= 0) return fail(JHQ_EINVAL, "nprobe must be positive");
    JHQ_TRY(idx->quiesce());
    const int prev = idx->nprobe;
    idx->nprobe = std::min(nprobe, idx->nlist);
    const int rc = reserve_search(idx);
    // a failed reservation keeps the setting the workspace was reserved for
    // (buffers only grow, so that reservation still holds)
    if (rc != JHQ_OK) idx->nprobe = prev;
    return rc;
}

int jhq_set_alpha(jhq_index* idx, float alpha) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (!(alpha > 0.0f)) return fail(JHQ_EINVAL, "alpha must be positive");
    JHQ_TRY(idx->quiesce());
    const float prev = idx->alpha;
    idx->alpha = alpha;
    const int rc = reserve_search(idx);
    if (rc != JHQ_OK) idx->alpha = prev;
    return rc;
}

int jhq_reserve(jhq_index* idx, int k_max) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (k_max <= 0) return fail(JHQ_EINVAL, "k_max must be positive");
    const int prev = idx->res_k;
    idx->res_k = std::max(idx->res_k, k_max);
    const int rc = reserve_search(idx);
    if (rc != JHQ_OK) idx->res_k = prev;
    return rc;
}

int jhq_set_scan_kind(jhq_index* idx, int kind) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (kind < 0 || kind > 2) return fail(JHQ_EINVAL, "scan kind must be 0, 1 or 2");
    JHQ_TRY(idx->quiesce());
    const int prev = idx->scan_kind;
    idx->scan_kind = kind;
    const int rc = reserve_search(idx);
    if (rc != JHQ_OK) idx->scan_kind = prev;
    return rc;
}

int jhq_get_dims(const jhq_index* idx, int* Ds, int* K1D, int* bpd, int* Kr, int* bpv) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (Ds) *Ds = idx->Ds;
    if (K1D) *K1D = idx->K1D;
    if (bpd) *bpd = idx->bpd;
    if (Kr) *Kr = idx->Kr;
    if (bpv) *bpv = idx->bpv;
    return JHQ_OK;
}

}  // extern "C"

namespace {

// Host float32 copy of a typed input (dtype 0 float32, 1 uint8, 2 int8).
int host_f32(const void* x, int dtype, int64_t count, std::vector<float>* tmp, const float** out) {
    if (dtype == JHQ_F32) {
        *out = static_cast<const float*>(x);
        return JHQ_OK;
    }
    if (dtype != JHQ_U8 && dtype != JHQ_I8) return fail(JHQ_EINVAL, "unknown dtype");
    tmp->resize(static_cast<size_t>(count));
    if (dtype == JHQ_U8) {
        const uint8_t* u = static_cast<const uint8_t*>(x);
        for (int64_t i = 0; i < count; i++) (*tmp)[i] = static_cast<float>(u[i]);
    } else {
        const int8_t* u = static_cast<const int8_t*>(x);
        for (int64_t i = 0; i < count; i++) (*tmp)[i] = static_cast<float>(u[i]);
    }
    *out = tmp->data();
    return JHQ_OK;
}

size_t dtype_size(int dtype) { return dtype == JHQ_F32 ? 4 : 1; }

// v14/jhq_gpu_index.cu:333-364
int train_impl(jhq_index* ix, const float* x, int64_t n_train) {
    if (n_train <= 0) return fail(JHQ_EINVAL, "n_train must be positive");
    if (n_train < ix->nlist) return fail(JHQ_EINVAL, "n_train must be >= nlist");
    if (n_train * static_cast<int64_t>(ix->d) > INT32_MAX)
        return fail(JHQ_EINVAL, "n_train * d must fit in int (the reference's residual k-means size)");
    if (ix->added || ix->ntotal > 0) return fail(JHQ_ESTATE, "train() after add() is not supported");
    JHQ_TRY(ix->ensure_stream());
    const int d = ix->d, M = ix->M, Ds = ix->Ds;
    ix->sigma = jhq::estimate_sigma(x, n_train, d);
    ix->c1d = jhq::lloyd_max_c1d(ix->sigma, ix->K1D);
    JHQ_TRY(ix->dP.upload(ix->P_rm.data(), ix->P_rm.size()));
    JHQ_TRY(ix->dc1d.upload(ix->c1d.data(), ix->c1d.size()));

    DBuf<float> dx, dy;
    DBuf<uint8_t> dcodes;
    JHQ_TRY(dx.upload(x, static_cast<size_t>(n_train) * d));
    JHQ_TRY(dy.alloc(static_cast<size_t>(n_train) * d));
    JHQ_TRY(dcodes.alloc(static_cast<size_t>(n_train) * M));
    JHQ_HIP(jhq::gemm_nt_store(dx.p, d, ix->dP.p, d, n_train, d, d, dy.p, d, false, ix->stream));
    JHQ_HIP(jhq::encode(dy.p, n_train, d, M, Ds, ix->K1D, ix->bpd, ix->dc1d.p, ix->Kr, 1, ix->Br,
                        ix->bpv, nullptr, dcodes.p, nullptr, nullptr, 1, ix->stream));
    dx.release();
    std::vector<float> h_y(static_cast<size_t>(n_train) * d);
    std::vector<uint8_t> h_codes(static_cast<size_t>(n_train) * M);
    JHQ_HIP(hipMemcpyAsync(h_y.data(), dy.p, h_y.size() * sizeof(float), hipMemcpyDeviceToHost,
                           ix->stream));
    JHQ_HIP(hipMemcpyAsync(h_codes.data(), dcodes.p, h_codes.size(), hipMemcpyDeviceToHost,
                           ix->stream));
    JHQ_HIP(hipStreamSynchronize(ix->stream));

    JHQ_TRY(train_ivf(ix, dy.p, n_train));

    // v14/jhq_gpu_index.cu:302-330 — residual scalars r = y - yhat over the
    // training set.  One codebook over every dimension (the reference), or,
    // with per-subspace codebooks, one 1-D k-means per subspace over that
    // subspace's Ds dimensions.
    const int kmask = ix->K1D - 1;
    auto resid = [&](int64_t i, int j) {
        const int m = j / Ds, k = j - m * Ds;
        return h_y[static_cast<size_t>(i) * d + j] -
               ix->c1d[(h_codes[static_cast<size_t>(i) * M + m] >> (k * ix->bpd)) & kmask];
    };
    if (verbose())
        std::fprintf(stderr, "[jhq] train: %d residual codebook(s) over %lld values each\n", ix->RC,
                     static_cast<long long>(n_train) * (ix->RC == 1 ? d : Ds));
    ix->res_c1d.assign(static_cast<size_t>(ix->RC) * ix->Kr, 0.f);
    std::vector<float> vals;
    for (int cb = 0; cb < ix->RC; cb++) {
        const int j0 = ix->RC == 1 ? 0 : cb * Ds, j1 = ix->RC == 1 ? d : j0 + Ds;
        vals.resize(static_cast<size_t>(n_train) * (j1 - j0));
        size_t t = 0;
        for (int64_t i = 0; i < n_train; i++)
            for (int j = j0; j < j1; j++) vals[t++] = resid(i, j);
        std::vector<float> c = jhq::train_1d_kmeans(vals.data(), static_cast<int64_t>(vals.size()),
                                                    ix->Kr);
        // Kr shrinks only for tiny training sets (train_1d_kmeans clamps Kr to n)
        for (int r = 0; r < ix->Kr; r++)
            ix->res_c1d[static_cast<size_t>(cb) * ix->Kr + r] =
                c.empty() ? 0.f : c[std::min<size_t>(r, c.size() - 1)];
    }
    JHQ_TRY(ix->dres_c1d.upload(ix->res_c1d.data(), ix->res_c1d.size()));
    JHQ_TRY(build_query_matrix(ix));
    ix->trained = true;
    return JHQ_OK;
}

// Uploads the ListDesc array {start, cap, size, cbase} from the host mirror:
// synchronously, or (s given) enqueued on s from pinned staging.
int upload_ldesc(jhq_index* ix, hipStream_t s = nullptr) {
    const size_t nl = static_cast<size_t>(ix->nlist);
    auto fill = [&](int4* h) {
        int64_t cb = 0;
        for (int l = 0; l < ix->nlist; l++) {
            h[l] = make_int4(ix->l_start[l], ix->l_cap[l], ix->l_size[l], static_cast<int>(cb));
            cb += ix->l_size[l];
        }
    };
    if (!s) {
        std::vector<int4> h(nl);
        fill(h.data());
        return ix->dldesc.upload_keep(h.data(), h.size());
    }
    const int t = ix->ldesc_turn;
    ix->ldesc_turn ^= 1;
    if (ix->ldesc_pending[t]) JHQ_HIP(hipEventSynchronize(ix->ldesc_ev[t]));
    ix->ldesc_pending[t] = false;
    JHQ_TRY(ensure_pinned(ix->h_ldesc[t], ix->h_ldesc_n[t], nl));
    fill(ix->h_ldesc[t]);
    JHQ_TRY(ix->dldesc.ensure(nl));
    JHQ_HIP(hipMemcpyAsync(ix->dldesc.p, ix->h_ldesc[t], nl * sizeof(int4), hipMemcpyHostToDevice,
                           s));
    JHQ_HIP(hipEventRecord(ix->ldesc_ev[t], s));
    ix->ldesc_pending[t] = true;
    return JHQ_OK;
}

// The skew scan's copy of the codes (M a multiple of 32, at most 128).
// Grows the device pool to at least `need` slots, keeping every block where
// it is (the old pool is copied to the front of the new one).
int grow_pool(jhq_index* ix, int64_t need) {
    if (need <= ix->pool_cap) return JHQ_OK;
    const int64_t cap = std::max<int64_t>(need, ix->pool_cap + ix->pool_cap / 2);
    const int M = ix->M, bpv = ix->bpv;
    DBuf<uint8_t> nc, nr;
    DBuf<float> nco;
    DBuf<int32_t> ni;
    JHQ_TRY(nc.alloc(static_cast<size_t>(cap) * M + 16));
    JHQ_TRY(nr.alloc(static_cast<size_t>(cap) * bpv));
    JHQ_TRY(nco.alloc(static_cast<size_t>(cap)));
    JHQ_TRY(ni.alloc(static_cast<size_t>(cap)));
    hipStream_t s = ix->stream;
    if (ix->pool_used > 0) {
        const size_t u = static_cast<size_t>(ix->pool_used);
        JHQ_HIP(hipMemcpyAsync(nc.p, ix->dcodes_t.p, u * M, hipMemcpyDeviceToDevice, s));
        JHQ_HIP(hipMemcpyAsync(nr.p, ix->dres.p, u * bpv, hipMemcpyDeviceToDevice, s));
        JHQ_HIP(hipMemcpyAsync(nco.p, ix->dcorr.p, u * sizeof(float), hipMemcpyDeviceToDevice, s));
        JHQ_HIP(hipMemcpyAsync(ni.p, ix->dlist_ids.p, u * sizeof(int32_t), hipMemcpyDeviceToDevice, s));
        JHQ_HIP(hipStreamSynchronize(s));
    }
    std::swap(ix->dcodes_t.p, nc.p);
    std::swap(ix->dcodes_t.n, nc.n);
    std::swap(ix->dres.p, nr.p);
    std::swap(ix->dres.n, nr.n);
    std::swap(ix->dcorr.p, nco.p);
    std::swap(ix->dcorr.n, nco.n);
    std::swap(ix->dlist_ids.p, ni.p);
    std::swap(ix->dlist_ids.n, ni.n);
    ix->pool_cap = cap;
    return JHQ_OK;
}

// Re-packs every list into a new pool: list l gets capacity
// round16(need[l] * 5/4) (need = its size after the pending insert), blocks
// are laid out in list order, dead blocks left by earlier moves are dropped,
// and the pool keeps a quarter of headroom for lists that move later.
int repack_pool(jhq_index* ix, const std::vector<int64_t>& need) {
    const int nlist = ix->nlist, M = ix->M, bpv = ix->bpv;
    std::vector<int32_t> nstart(nlist), ncap(nlist);
    std::vector<int4> moves;
    int64_t pos = 0;
    for (int l = 0; l < nlist; l++) {
        const int64_t want = need[l] > 0 ? need[l] + need[l] / 4 : 0;
        const int64_t cap = (want + jhq::kGroup - 1) / jhq::kGroup * jhq::kGroup;
        if (ix->l_size[l] > 0) {
            moves.push_back(make_int4(ix->l_start[l], ix->l_cap[l], ix->l_size[l], 0));
            moves.push_back(make_int4(static_cast<int>(pos), static_cast<int>(cap), 0, 0));
        }
        nstart[l] = static_cast<int32_t>(pos);
        ncap[l] = static_cast<int32_t>(cap);
        pos += cap;
        if (pos > INT32_MAX) return fail(JHQ_EINVAL, "list pool exceeds int32 slots");
    }
    const int64_t pcap = std::min<int64_t>(std::max<int64_t>(pos + pos / 4, 1), INT32_MAX);
    DBuf<uint8_t> nc, nr;
    DBuf<float> nco;
    DBuf<int32_t> ni;
    JHQ_TRY(nc.alloc(static_cast<size_t>(pcap) * M + 16));
    JHQ_TRY(nr.alloc(static_cast<size_t>(pcap) * bpv));
    JHQ_TRY(nco.alloc(static_cast<size_t>(pcap)));
    JHQ_TRY(ni.alloc(static_cast<size_t>(pcap)));
    hipStream_t s = ix->stream;
    if (!moves.empty()) {
        DBuf<int4> dmoves;
        JHQ_TRY(dmoves.upload(moves.data(), moves.size()));
        JHQ_HIP(jhq::relocate_lists(dmoves.p, static_cast<int>(moves.size() / 2), M, bpv,
                                    ix->dcodes_t.p, nc.p, ix->dres.p, nr.p, ix->dcorr.p, nco.p,
                                    ix->dlist_ids.p, ni.p, s));
        JHQ_HIP(hipStreamSynchronize(s));
    }
    std::swap(ix->dcodes_t.p, nc.p);
    std::swap(ix->dcodes_t.n, nc.n);
    std::swap(ix->dres.p, nr.p);
    std::swap(ix->dres.n, nr.n);
    std::swap(ix->dcorr.p, nco.p);
    std::swap(ix->dcorr.n, nco.n);
    std::swap(ix->dlist_ids.p, ni.p);
    std::swap(ix->dlist_ids.n, ni.n);
    ix->l_start = nstart;
    ix->l_cap = ncap;
    ix->pool_cap = pcap;
    ix->pool_used = pos;
    return JHQ_OK;
}

// Rotates, encodes and assigns n vectors x (host, dtype) in add_batch chunks
// (v14/jhq_gpu_index.cu:438-463), inserts them at the end of their lists
// with ids id_base + i, and grows list blocks as needed.  exact_fit: the
// pool is empty and every list gets capacity round16(size) (the one-shot add
// of the reference); otherwise a list that outgrows its block moves to the
// end of the pool with 1.5 times the capacity, and when the pool has no room
// left for such moves every list is re-packed into a new pool instead.
int insert_impl(jhq_index* ix, const void* x, int dtype, int64_t n, bool exact_fit) {
    JHQ_TRY(ix->ensure_stream());
    // a device search still in flight reads the lists rewritten below
    JHQ_TRY(ix->quiesce());
    ix->skew_stale = true;
    ix->rows_stale = true;
    ix->dump_P = -1;
    const int d = ix->d, M = ix->M, bpv = ix->bpv, nlist = ix->nlist;
    hipStream_t s = ix->stream;
    const int64_t id_base = ix->ntotal;
    if (verbose()) {
        JHQ_TRY(ix->drecheck.ensure(1));
        JHQ_HIP(jhq::fill_u64(ix->drecheck.p, 1, 0ull, s));
    }

    InsertScratch& sc = ix->ins;
    // the scratch goes back to the device after an insert too large to keep
    // (once the enqueued work that reads it is done)
    struct Trim {
        InsertScratch& sc;
        hipStream_t s;
        ~Trim() {
            if (sc.bytes() > kInsertKeepBytes) {
                (void)hipStreamSynchronize(s);
                sc.release();
            }
        }
    } trim{sc, s};
    DBuf<uint8_t>& dpc = sc.pc;
    DBuf<uint8_t>& drc = sc.rc;
    DBuf<float>& dco = sc.co;
    DBuf<int32_t>& dasg = sc.asg;
    JHQ_TRY(dpc.ensure(static_cast<size_t>(n) * M));
    JHQ_TRY(drc.ensure(static_cast<size_t>(n) * bpv));
    JHQ_TRY(dco.ensure(static_cast<size_t>(n)));
    JHQ_TRY(dasg.ensure(static_cast<size_t>(n)));
    {
        const int64_t AB = std::min<int64_t>(ix->add_batch, n);
        DBuf<float>* dxb = sc.xb;
        DBuf<float>& dyb = sc.yb;
        DBuf<uint8_t>* draw = sc.raw;
        DBuf<unsigned long long>& keys = sc.keys;
        for (int i = 0; i < 2 && i * AB < n; i++) {
            JHQ_TRY(dxb[i].ensure(static_cast<size_t>(AB) * d));
            if (dtype != JHQ_F32) JHQ_TRY(draw[i].ensure(static_cast<size_t>(AB) * d));
        }
        JHQ_TRY(dyb.ensure(static_cast<size_t>(AB) * d));
        // the copies run on their own stream a batch ahead of the kernels; an
        // input buffer is refilled once the kernels that read it (two batches
        // back) are done
        JHQ_TRY(ix->ensure_copy_stream());
        // one batch has nothing to overlap: its copy stays on the kernels' stream
        hipStream_t cst = n > AB ? ix->lane[kLanes - 1] : s;
        // on every exit the copy stream is drained before the buffers go
        struct Drain {
            hipStream_t cs;
            ~Drain() { (void)hipStreamSynchronize(cs); }
        } drain{cst};
        struct {
            hipStream_t cs;
            hipEvent_t* copied;
            hipEvent_t* consumed;
        } sy{cst, ix->copy_ev, ix->copy_ev + 2};
        const uint8_t* xb = static_cast<const uint8_t*>(x);
        const size_t es = dtype_size(dtype);
        for (int64_t start = 0, bi = 0; start < n; start += AB, bi++) {
            const int i = static_cast<int>(bi & 1);
            const int64_t nb = std::min(AB, n - start);
            const size_t cnt = static_cast<size_t>(nb) * d;
            if (bi >= 2) JHQ_HIP(hipStreamWaitEvent(sy.cs, sy.consumed[i], 0));
            if (dtype == JHQ_F32) {
                JHQ_HIP(hipMemcpyAsync(dxb[i].p, xb + static_cast<size_t>(start) * d * es,
                                       cnt * sizeof(float), hipMemcpyHostToDevice, sy.cs));
            } else {
                // bytes cross PCIe; float32 conversion on the device
                JHQ_HIP(hipMemcpyAsync(draw[i].p, xb + static_cast<size_t>(start) * d, cnt,
                                       hipMemcpyHostToDevice, sy.cs));
            }
            JHQ_HIP(hipEventRecord(sy.copied[i], sy.cs));
            JHQ_HIP(hipStreamWaitEvent(s, sy.copied[i], 0));
            if (dtype != JHQ_F32)
                JHQ_HIP(jhq::convert_to_f32(draw[i].p, dtype, static_cast<int64_t>(cnt), dxb[i].p, s));
            JHQ_HIP(jhq::gemm_nt_store(dxb[i].p, d, ix->dP.p, d, nb, d, d, dyb.p, d, false, s));
            JHQ_HIP(hipEventRecord(sy.consumed[i], s));
            JHQ_HIP(jhq::encode(dyb.p, nb, d, M, ix->Ds, ix->K1D, ix->bpd, ix->dc1d.p, ix->Kr, ix->RC,
                                ix->Br, bpv, ix->dres_c1d.p, dpc.p + start * M,
                                drc.p + start * bpv, dco.p + start, 3, s));
            JHQ_TRY(assign_rows(ix, dyb.p, nb, dasg.p + start, keys));
            if (verbose() && (bi + 1) % 128 == 0)
                std::fprintf(stderr, "[jhq] add: %lld / %lld vectors enqueued\n",
                             static_cast<long long>(start + nb), static_cast<long long>(n));
        }
    }
    if (verbose() && ix->drecheck.p) {
        JHQ_HIP(hipStreamSynchronize(s));
        unsigned long long rc = 0;
        JHQ_HIP(hipMemcpy(&rc, ix->drecheck.p, sizeof(rc), hipMemcpyDeviceToHost));
        std::fprintf(stderr, "[jhq] add: %llu of %lld rows re-checked by the fixed-order argmin\n",
                     rc, static_cast<long long>(n));
    }
    // stable order by (list, id) of the new vectors (the reference's
    // thrust::sort_by_key, v14/jhq_gpu_index.cu:468-486): keys (list << 32 |
    // vector) radix-sorted on the device; the host reads the list counts only
    DBuf<unsigned char>& oscr = sc.oscr;
    JHQ_TRY(oscr.ensure(jhq::kmeans_scratch_bytes(n, nlist)));
    const unsigned long long* sorted = nullptr;
    const int64_t* first = nullptr;
    JHQ_HIP(jhq::list_order(dasg.p, n, nlist, oscr.p, oscr.n, &sorted, &first, s));
    std::vector<int64_t> firsth(static_cast<size_t>(nlist) + 1);
    JHQ_HIP(hipMemcpyAsync(firsth.data(), first, firsth.size() * sizeof(int64_t),
                           hipMemcpyDeviceToHost, s));
    JHQ_HIP(hipStreamSynchronize(s));
    if (firsth[0] != 0 || firsth[nlist] != n) return fail(JHQ_EDEVICE, "invalid IVF assignment");
    std::vector<int64_t> add(nlist + 1, 0);
    for (int l = 0; l < nlist; l++) add[l + 1] = firsth[l + 1] - firsth[l];
    for (int l = 0; l < nlist; l++) {
        if (static_cast<int64_t>(ix->l_size[l]) + add[l + 1] > INT32_MAX)
            return fail(JHQ_EINVAL, "list size exceeds int32");
    }
    // block placement: from here until the descriptors are uploaded the
    // device lists and the host mirror may disagree
    ix->broken = true;
    std::vector<int4> moves;
    if (exact_fit) {
        int64_t pos = 0;
        for (int l = 0; l < nlist; l++) {
            const int64_t cap = (add[l + 1] + jhq::kGroup - 1) / jhq::kGroup * jhq::kGroup;
            ix->l_start[l] = static_cast<int32_t>(pos);
            ix->l_cap[l] = static_cast<int32_t>(cap);
            pos += cap;
        }
        if (pos > INT32_MAX) return fail(JHQ_EINVAL, "list pool exceeds int32 slots");
        JHQ_TRY(grow_pool(ix, pos));  // empty pool: nothing is copied
        ix->pool_used = pos;
    } else {
        int64_t used = ix->pool_used;
        std::vector<int32_t> nstart(ix->l_start), ncap(ix->l_cap);
        for (int l = 0; l < nlist; l++) {
            const int64_t need = ix->l_size[l] + add[l + 1];
            if (need <= ix->l_cap[l]) continue;
            int64_t cap = std::max<int64_t>(need, ix->l_cap[l] + ix->l_cap[l] / 2);
            cap = std::max<int64_t>(cap, jhq::kGroup);
            cap = (cap + jhq::kGroup - 1) / jhq::kGroup * jhq::kGroup;
            if (ix->l_size[l] > 0) {
                moves.push_back(make_int4(ix->l_start[l], ix->l_cap[l], ix->l_size[l], 0));
                moves.push_back(make_int4(static_cast<int>(used), static_cast<int>(cap), 0, 0));
            }
            nstart[l] = static_cast<int32_t>(used);
            ncap[l] = static_cast<int32_t>(cap);
            used += cap;
        }
        if (used > ix->pool_cap && ix->pool_used > 0) {
            // no room for the moves: re-pack every list instead of growing
            std::vector<int64_t> need(nlist);
            for (int l = 0; l < nlist; l++) need[l] = ix->l_size[l] + add[l + 1];
            JHQ_TRY(repack_pool(ix, need));
            moves.clear();
            nstart = ix->l_start;
            ncap = ix->l_cap;
            used = ix->pool_used;
        }
        if (used > INT32_MAX) return fail(JHQ_EINVAL, "list pool exceeds int32 slots");
        JHQ_TRY(grow_pool(ix, used));  // only an empty pool grows here
        if (!moves.empty()) {
            DBuf<int4>& dmoves = sc.moves;
            JHQ_TRY(dmoves.upload_keep(moves.data(), moves.size()));
            JHQ_HIP(jhq::relocate_lists(dmoves.p, static_cast<int>(moves.size() / 2), M, bpv,
                                        ix->dcodes_t.p, ix->dcodes_t.p, ix->dres.p, ix->dres.p,
                                        ix->dcorr.p, ix->dcorr.p, ix->dlist_ids.p, ix->dlist_ids.p,
                                        s));
            JHQ_HIP(hipStreamSynchronize(s));
        }
        ix->l_start = nstart;
        ix->l_cap = ncap;
        ix->pool_used = used;
    }
    // scatter the new vectors behind each list's current candidates (the
    // descriptors still hold the sizes before the insert)
    {
        JHQ_TRY(upload_ldesc(ix, s));
        DBuf<int32_t>& dorder = sc.order;
        DBuf<int32_t>& dslist = sc.slist;
        DBuf<int32_t>& dsidx = sc.sidx;
        JHQ_TRY(dorder.ensure(static_cast<size_t>(n)));
        JHQ_TRY(dslist.ensure(static_cast<size_t>(n)));
        JHQ_TRY(dsidx.ensure(static_cast<size_t>(n)));
        JHQ_HIP(jhq::scatter_plan(sorted, first, ix->dldesc.p, n, dorder.p, dslist.p, dsidx.p, s));
        JHQ_HIP(jhq::scatter_lists(dorder.p, dslist.p, dsidx.p, n, id_base, ix->dldesc.p, dpc.p,
                                   drc.p, dco.p, M, bpv, ix->dlist_ids.p, ix->dcodes_t.p, ix->dres.p,
                                   ix->dcorr.p, s));
        for (int l = 0; l < nlist; l++) ix->l_size[l] += static_cast<int32_t>(add[l + 1]);
    }
    // the descriptors with the new sizes follow the scatter on s; the host
    // does not wait (device searches wait for the tail event)
    JHQ_TRY(upload_ldesc(ix, s));
    JHQ_TRY(ix->mark_tail());
    ix->ntotal += n;
    ix->broken = false;
    return JHQ_OK;
}

int check_insert(jhq_index* ix, const void* x, int64_t n) {
    if (!ix || !x) return fail(JHQ_EINVAL, "null argument");
    if (!ix->trained) return fail(JHQ_ESTATE, "call train() before add()");
    if (n <= 0) return fail(JHQ_EINVAL, "n must be positive");
    if (ix->ntotal + n > INT32_MAX) return fail(JHQ_EINVAL, "n exceeds int32 ids");
    return JHQ_OK;
}

}  // namespace

extern "C" {

int jhq_train(jhq_index* ix, const float* x, int64_t n_train) {
    return jhq_train_ex(ix, x, JHQ_F32, n_train);
}

int jhq_train_ex(jhq_index* ix, const void* x, int dtype, int64_t n_train) {
    if (!ix || !x) return fail(JHQ_EINVAL, "null argument");
    if (n_train <= 0) return fail(JHQ_EINVAL, "n_train must be positive");
    std::vector<float> tmp;
    const float* xf = nullptr;
    JHQ_TRY(host_f32(x, dtype, n_train * static_cast<int64_t>(ix->d), &tmp, &xf));
    return train_impl(ix, xf, n_train);
}

// v14/jhq_gpu_index.cu:417-532
int jhq_add(jhq_index* ix, const float* x, int64_t n) { return jhq_add_ex(ix, x, JHQ_F32, n); }

int jhq_add_ex(jhq_index* ix, const void* x, int dtype, int64_t n) {
    JHQ_TRY(check_insert(ix, x, n));
    if (dtype != JHQ_F32 && dtype != JHQ_U8 && dtype != JHQ_I8)
        return fail(JHQ_EINVAL, "unknown dtype");
    if (ix->added || ix->ntotal > 0) return fail(JHQ_ESTATE, "only one add() call is supported");
    JHQ_TRY(insert_impl(ix, x, dtype, n, true));
    ix->added = true;
    return reserve_search(ix);
}

int jhq_append(jhq_index* ix, const float* x, int64_t n) {
    return jhq_append_ex(ix, x, JHQ_F32, n);
}

int jhq_append_ex(jhq_index* ix, const void* x, int dtype, int64_t n) {
    JHQ_TRY(check_insert(ix, x, n));
    if (dtype != JHQ_F32 && dtype != JHQ_U8 && dtype != JHQ_I8)
        return fail(JHQ_EINVAL, "unknown dtype");
    JHQ_TRY(insert_impl(ix, x, dtype, n, false));
    ix->added = true;
    return reserve_search(ix);
}

int jhq_search(jhq_index* idx, const float* q, int64_t nq, int k, float* dists, int32_t* ids) {
    if (!q || !dists || !ids) return fail(JHQ_EINVAL, "null argument");
    return search_host(idx, q, nq, k, dists, ids, nullptr, nullptr, nullptr, nullptr);
}

int jhq_search_debug(jhq_index* idx, const float* q, int64_t nq, int k, float* dists,
                     int32_t* ids, float* q_rot, int32_t* probes, int32_t* topck_pos,
                     float* topck_dist) {
    if (!q || !dists || !ids) return fail(JHQ_EINVAL, "null argument");
    return search_host(idx, q, nq, k, dists, ids, q_rot, probes, topck_pos, topck_dist);
}

int jhq_search_device(jhq_index* ix, const float* d_q, int64_t nq, int k, float* d_dists,
                      int32_t* d_ids, void* stream) {
    JHQ_TRY(check_searchable(ix, nq, k));
    if (!d_q || !d_dists || !d_ids) return fail(JHQ_EINVAL, "null argument");
    if (nq == 0) return JHQ_OK;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ix->stream;
    const int Bmax = ix->batch_size;
    // several batches: rotate through the search lanes (workspace and stream
    // each), forked from s and joined back into it (step timing keeps one
    // stream)
    const bool pipe = nq > Bmax && !ix->timing;
    // enqueue-only: the reserved workspace must cover this shape (no
    // allocation, no host synchronisation)
    BatchPlan bp;
    JHQ_TRY(plan_batch(ix, Bmax, k, &bp, pipe ? kLanes : 1, false));
    if (pipe && !ix->lane[kLanes - 1])
        return fail(JHQ_ESTATE, "search lanes are not set up; call jhq_reserve()");
    // ordered after the previous device search (it shares the workspaces),
    // whatever stream that one ran on
    if (ix->done_pending) JHQ_HIP(hipStreamWaitEvent(s, ix->done_ev, 0));
    // and after the last insert's or row refresh's enqueued work
    if (ix->tail_pending) JHQ_HIP(hipStreamWaitEvent(s, ix->tail_ev, 0));
    if (!pipe) {
        for (int64_t q0 = 0; q0 < nq; q0 += Bmax) {
            const int Bq = static_cast<int>(std::min<int64_t>(Bmax, nq - q0));
            JHQ_TRY(run_batch(ix, ix->ws[0], d_q + q0 * ix->d, Bq, k, bp, d_dists + q0 * k,
                              d_ids + q0 * k, false, s));
        }
        JHQ_HIP(hipEventRecord(ix->done_ev, s));
        ix->done_pending = true;
        return JHQ_OK;
    }
    const int nl = ix->nlanes;
    JHQ_HIP(hipEventRecord(ix->lane_ev[0], s));
    for (int i = 0; i < nl; i++)
        JHQ_HIP(hipStreamWaitEvent(ix->lane[ix->lane_use[i]], ix->lane_ev[0], 0));
    // consecutive batches share their lane's query product where the
    // selection adds its split sums
    const int d = ix->d;
    const bool share = kQbShare > 1 && ix->dqmat.p &&
                       jhq::select_adds_qb(jhq::mfma_qb_plan(Bmax * kQbShare, d + ix->nlist, d),
                                           ix->nlist, d);
    int64_t bi = 0;
    for (int64_t q0 = 0; q0 < nq; bi++) {
        const int l = ix->lane_use[bi % nl];
        const int64_t rows = std::min<int64_t>(static_cast<int64_t>(Bmax) * (share ? kQbShare : 1),
                                               nq - q0);
        // one batch alone keeps its own product
        const int srows = rows > Bmax ? static_cast<int>(rows) : 0;
        for (int64_t r0 = 0; r0 < rows; r0 += Bmax) {
            const int Bq = static_cast<int>(std::min<int64_t>(Bmax, rows - r0));
            JHQ_TRY(run_batch(ix, ix->ws[l], d_q + (q0 + r0) * d, Bq, k, bp,
                              d_dists + (q0 + r0) * k, d_ids + (q0 + r0) * k, false, ix->lane[l],
                              QbShare{srows, srows ? static_cast<int>(r0) : 0}));
        }
        q0 += rows;
    }
    for (int i = 0; i < nl; i++) {
        const int l = ix->lane_use[i];
        JHQ_HIP(hipEventRecord(ix->lane_ev[1 + l], ix->lane[l]));
        JHQ_HIP(hipStreamWaitEvent(s, ix->lane_ev[1 + l], 0));
    }
    JHQ_HIP(hipEventRecord(ix->done_ev, s));
    ix->done_pending = true;
    return JHQ_OK;
}

int jhq_get_codebooks(const jhq_index* idx, float* sigma, float* c1d, float* res_c1d, float* P,
                      float* centroids, float* cent_norms) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (sigma) *sigma = idx->sigma;
    if (P) std::memcpy(P, idx->P_rm.data(), idx->P_rm.size() * sizeof(float));
    if ((c1d || res_c1d || centroids || cent_norms) && !idx->trained)
        return fail(JHQ_ESTATE, "index is not trained");
    if (c1d) std::memcpy(c1d, idx->c1d.data(), idx->c1d.size() * sizeof(float));
    if (res_c1d) std::memcpy(res_c1d, idx->res_c1d.data(), idx->res_c1d.size() * sizeof(float));
    if (centroids) std::memcpy(centroids, idx->cent.data(), idx->cent.size() * sizeof(float));
    if (cent_norms) std::memcpy(cent_norms, idx->cent_norms.data(), idx->cent_norms.size() * sizeof(float));
    return JHQ_OK;
}

int jhq_get_lists(const jhq_index* idx, int32_t* offsets, int32_t* ids, uint8_t* codes,
                  uint8_t* res, float* corr) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (!idx->added) return fail(JHQ_ESTATE, "index is empty");
    if (idx->broken)
        return fail(JHQ_ESTATE, "a failed add/append left the index's lists inconsistent");
    // the copies below run on the null stream; a device search may still be
    // in flight on a caller's non-blocking stream
    JHQ_TRY(const_cast<jhq_index*>(idx)->quiesce());
    const int M = idx->M, nlist = idx->nlist, bpv = idx->bpv;
    // canonical order: lists in list order, candidates in insertion order
    std::vector<int64_t> cbase(nlist + 1, 0);
    for (int l = 0; l < nlist; l++) cbase[l + 1] = cbase[l] + idx->l_size[l];
    if (offsets)
        for (int l = 0; l <= nlist; l++) offsets[l] = static_cast<int32_t>(cbase[l]);
    const size_t used = static_cast<size_t>(idx->pool_used);
    if (ids) {
        std::vector<int32_t> t(used);
        JHQ_HIP(hipMemcpy(t.data(), idx->dlist_ids.p, used * sizeof(int32_t), hipMemcpyDeviceToHost));
        for (int l = 0; l < nlist; l++)
            std::memcpy(ids + cbase[l], t.data() + idx->l_start[l], idx->l_size[l] * sizeof(int32_t));
    }
    if (corr) {
        std::vector<float> t(used);
        JHQ_HIP(hipMemcpy(t.data(), idx->dcorr.p, used * sizeof(float), hipMemcpyDeviceToHost));
        for (int l = 0; l < nlist; l++)
            std::memcpy(corr + cbase[l], t.data() + idx->l_start[l], idx->l_size[l] * sizeof(float));
    }
    if (res) {
        std::vector<uint8_t> t(used * bpv);
        JHQ_HIP(hipMemcpy(t.data(), idx->dres.p, t.size(), hipMemcpyDeviceToHost));
        for (int l = 0; l < nlist; l++)
            std::memcpy(res + cbase[l] * bpv, t.data() + static_cast<size_t>(idx->l_start[l]) * bpv,
                        static_cast<size_t>(idx->l_size[l]) * bpv);
    }
    if (codes) {
        std::vector<uint8_t> t(used * M);
        JHQ_HIP(hipMemcpy(t.data(), idx->dcodes_t.p, t.size(), hipMemcpyDeviceToHost));
        for (int l = 0; l < nlist; l++) {
            const int64_t st = idx->l_start[l], cap = idx->l_cap[l], o = cbase[l];
            for (int64_t i = 0; i < idx->l_size[l]; i++)
                for (int m = 0; m < M; m++) codes[(o + i) * M + m] = t[st * M + m * cap + i];
        }
    }
    return JHQ_OK;
}

// ---- index file: params, trained state, lists in canonical order ----------
// Layout (little-endian): "JHQAMD01", u32 version, i32 d, jhq_params fields
// (i32 except alpha f32), u8 trained, u8 added, i64 ntotal, f32 sigma,
// f32 c1d[K1D], f32 res_c1d[RC*Kr], f32 P[d*d] (row-major Pi), f32
// centroids[nlist*d], f32 norms[nlist], i32 sizes[nlist], i32 ids[ntotal],
// u8 codes[ntotal*M], u8 res[ntotal*bpv], f32 corr[ntotal].
}  // extern "C"

namespace {

constexpr char kMagic[8] = {'J', 'H', 'Q', 'A', 'M', 'D', '0', '1'};
constexpr uint32_t kVersion = 1;

struct FileW {
    FILE* f;
    bool ok = true;
    void put(const void* p, size_t n) {
        if (ok && n && std::fwrite(p, 1, n, f) != n) ok = false;
    }
    template <class T>
    void put(const T& v) {
        put(&v, sizeof(T));
    }
};

struct FileR {
    FILE* f;
    bool ok = true;
    void get(void* p, size_t n) {
        if (ok && n && std::fread(p, 1, n, f) != n) ok = false;
    }
    template <class T>
    void get(T& v) {
        get(&v, sizeof(T));
    }
};

}  // namespace

extern "C" {

int jhq_get_params(const jhq_index* idx, jhq_params* out) {
    if (!idx || !out) return fail(JHQ_EINVAL, "null argument");
    out->M = idx->M;
    out->B = idx->B;
    out->Br = idx->Br;
    out->alpha = idx->alpha;
    out->nlist = idx->nlist;
    out->nprobe = idx->nprobe;
    out->ivf_iters = idx->ivf_iters;
    out->batch_size = idx->batch_size;
    out->seed = idx->seed;
    out->add_batch = idx->add_batch;
    out->residual_per_subspace = idx->RC > 1 ? 1 : 0;
    return JHQ_OK;
}

int jhq_save(const jhq_index* idx, const char* path) {
    if (!idx || !path) return fail(JHQ_EINVAL, "null argument");
    if (!idx->trained) return fail(JHQ_ESTATE, "index is not trained");
    const int64_t n = idx->ntotal;
    const int nlist = idx->nlist;
    std::vector<int32_t> offs(nlist + 1), ids(n);
    std::vector<uint8_t> codes(static_cast<size_t>(n) * idx->M), res(static_cast<size_t>(n) * idx->bpv);
    std::vector<float> corr(n);
    if (n > 0) JHQ_TRY(jhq_get_lists(idx, offs.data(), ids.data(), codes.data(), res.data(), corr.data()));
    FILE* f = std::fopen(path, "wb");
    if (!f) return fail(JHQ_EINVAL, std::string("cannot open ") + path + " for writing");
    FileW w{f};
    w.put(kMagic, 8);
    w.put(kVersion);
    w.put(idx->d);
    for (int v : {idx->M, idx->B, idx->Br}) w.put(v);
    w.put(idx->alpha);
    for (int v : {idx->nlist, idx->nprobe, idx->ivf_iters, idx->batch_size, idx->seed,
                  idx->add_batch, idx->RC > 1 ? 1 : 0})
        w.put(v);
    const uint8_t tr = idx->trained ? 1 : 0, ad = idx->added ? 1 : 0;
    w.put(tr);
    w.put(ad);
    w.put(n);
    w.put(idx->sigma);
    w.put(idx->c1d.data(), idx->c1d.size() * sizeof(float));
    w.put(idx->res_c1d.data(), idx->res_c1d.size() * sizeof(float));
    w.put(idx->P_rm.data(), idx->P_rm.size() * sizeof(float));
    w.put(idx->cent.data(), idx->cent.size() * sizeof(float));
    w.put(idx->cent_norms.data(), idx->cent_norms.size() * sizeof(float));
    w.put(idx->l_size.data(), idx->l_size.size() * sizeof(int32_t));
    w.put(ids.data(), ids.size() * sizeof(int32_t));
    w.put(codes.data(), codes.size());
    w.put(res.data(), res.size());
    w.put(corr.data(), corr.size() * sizeof(float));
    const bool closed = std::fclose(f) == 0;
    if (!w.ok || !closed) return fail(JHQ_EINVAL, std::string("write to ") + path + " failed");
    return JHQ_OK;
}

int jhq_load(const char* path, jhq_index** out) {
    if (!path || !out) return fail(JHQ_EINVAL, "null argument");
    *out = nullptr;
    FILE* f = std::fopen(path, "rb");
    if (!f) return fail(JHQ_EINVAL, std::string("cannot open ") + path);
    FileR r{f};
    char magic[8];
    uint32_t ver = 0;
    int d = 0;
    jhq_params p;
    jhq_params_default(&p);
    r.get(magic, 8);
    r.get(ver);
    r.get(d);
    r.get(p.M);
    r.get(p.B);
    r.get(p.Br);
    r.get(p.alpha);
    for (int* v : {&p.nlist, &p.nprobe, &p.ivf_iters, &p.batch_size, &p.seed, &p.add_batch,
                   &p.residual_per_subspace})
        r.get(*v);
    if (!r.ok || std::memcmp(magic, kMagic, 8) != 0 || ver != kVersion) {
        std::fclose(f);
        return fail(JHQ_EINVAL, std::string(path) + " is not a JHQ index file of this version");
    }
    const int nprobe_saved = p.nprobe;
    jhq_index* ix = nullptr;
    int rc = jhq_create(d, &p, &ix);
    if (rc != JHQ_OK) {
        std::fclose(f);
        return rc;
    }
    ix->nprobe = nprobe_saved;
    uint8_t tr = 0, ad = 0;
    int64_t n = 0;
    r.get(tr);
    r.get(ad);
    r.get(n);
    r.get(ix->sigma);
    ix->c1d.resize(ix->K1D);
    ix->res_c1d.resize(static_cast<size_t>(ix->RC) * ix->Kr);
    ix->cent.resize(static_cast<size_t>(ix->nlist) * d);
    ix->cent_norms.resize(ix->nlist);
    std::vector<float> P(static_cast<size_t>(d) * d);
    r.get(ix->c1d.data(), ix->c1d.size() * sizeof(float));
    r.get(ix->res_c1d.data(), ix->res_c1d.size() * sizeof(float));
    r.get(P.data(), P.size() * sizeof(float));
    r.get(ix->cent.data(), ix->cent.size() * sizeof(float));
    r.get(ix->cent_norms.data(), ix->cent_norms.size() * sizeof(float));
    std::vector<int32_t> sizes(ix->nlist), ids;
    r.get(sizes.data(), sizes.size() * sizeof(int32_t));
    const bool ok_n = r.ok && n >= 0 && n <= INT32_MAX;
    int64_t tot = 0;
    bool neg = false;
    for (int32_t v : sizes) {
        tot += v;
        neg |= v < 0;
    }
    if (!ok_n || neg || tot != n || !tr) {
        std::fclose(f);
        delete ix;
        return fail(JHQ_EINVAL, std::string(path) + ": truncated or inconsistent index file");
    }
    ids.resize(n);
    std::vector<uint8_t> codes(static_cast<size_t>(n) * ix->M), res(static_cast<size_t>(n) * ix->bpv);
    std::vector<float> corr(n);
    r.get(ids.data(), ids.size() * sizeof(int32_t));
    r.get(codes.data(), codes.size());
    r.get(res.data(), res.size());
    r.get(corr.data(), corr.size() * sizeof(float));
    std::fclose(f);
    if (!r.ok) {
        delete ix;
        return fail(JHQ_EINVAL, std::string(path) + ": truncated index file");
    }
    // the rotation is rebuilt from the seed at construction; the file's copy
    // must agree (it is the same deterministic computation)
    if (std::memcmp(P.data(), ix->P_rm.data(), P.size() * sizeof(float)) != 0) {
        delete ix;
        return fail(JHQ_EINVAL, std::string(path) + ": stored rotation differs from its seed's");
    }
    auto done = [&](int code) {
        if (code != JHQ_OK) delete ix;
        return code;
    };
    if ((rc = ix->ensure_stream()) != JHQ_OK ||
        (rc = ix->dP.upload(ix->P_rm.data(), ix->P_rm.size())) != JHQ_OK ||
        (rc = ix->dc1d.upload(ix->c1d.data(), ix->c1d.size())) != JHQ_OK ||
        (rc = ix->dres_c1d.upload(ix->res_c1d.data(), ix->res_c1d.size())) != JHQ_OK ||
        (rc = ix->dcent.upload(ix->cent.data(), ix->cent.size())) != JHQ_OK ||
        (rc = ix->dnorms.upload(ix->cent_norms.data(), ix->cent_norms.size())) != JHQ_OK ||
        (rc = build_query_matrix(ix)) != JHQ_OK)
        return done(rc);
    ix->trained = true;
    // compact pool: exact-fit blocks in list order (the one-shot add's layout)
    const int M = ix->M, bpv = ix->bpv, nlist = ix->nlist;
    int64_t pos = 0;
    for (int l = 0; l < nlist; l++) {
        ix->l_start[l] = static_cast<int32_t>(pos);
        ix->l_cap[l] = (sizes[l] + jhq::kGroup - 1) / jhq::kGroup * jhq::kGroup;
        ix->l_size[l] = sizes[l];
        pos += ix->l_cap[l];
    }
    if (pos > INT32_MAX) return done(fail(JHQ_EINVAL, "list pool exceeds int32 slots"));
    if (pos > 0) {
        if ((rc = grow_pool(ix, pos)) != JHQ_OK) return done(rc);
        ix->pool_used = pos;
        std::vector<uint8_t> pc(static_cast<size_t>(pos) * M, 0), pr(static_cast<size_t>(pos) * bpv, 0);
        std::vector<float> pco(static_cast<size_t>(pos), 0.f);
        std::vector<int32_t> pid(static_cast<size_t>(pos), -1);
        int64_t o = 0;
        for (int l = 0; l < nlist; l++) {
            const int64_t st = ix->l_start[l], cap = ix->l_cap[l];
            for (int64_t i = 0; i < sizes[l]; i++, o++) {
                for (int m = 0; m < M; m++) pc[st * M + m * cap + i] = codes[o * M + m];
                std::memcpy(pr.data() + (st + i) * bpv, res.data() + o * bpv, bpv);
                pco[st + i] = corr[o];
                pid[st + i] = ids[o];
            }
        }
        hipStream_t s = ix->stream;
        if (hipMemcpyAsync(ix->dcodes_t.p, pc.data(), pc.size(), hipMemcpyHostToDevice, s) != hipSuccess ||
            hipMemcpyAsync(ix->dres.p, pr.data(), pr.size(), hipMemcpyHostToDevice, s) != hipSuccess ||
            hipMemcpyAsync(ix->dcorr.p, pco.data(), pco.size() * sizeof(float), hipMemcpyHostToDevice,
                           s) != hipSuccess ||
            hipMemcpyAsync(ix->dlist_ids.p, pid.data(), pid.size() * sizeof(int32_t),
                           hipMemcpyHostToDevice, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return done(fail(JHQ_EDEVICE, "index upload failed"));
    }
    rc = upload_ldesc(ix);
    if (rc != JHQ_OK) return done(rc);
    ix->ntotal = n;
    ix->added = ad != 0;
    // The index is whole once its lists are uploaded.  If the search
    // workspace cannot be reserved (out of memory, or a plan that does not fit
    // in LDS), the index is still returned: host searches reserve what they
    // need, device searches fail with JHQ_ESTATE until jhq_reserve succeeds.
    (void)reserve_search(ix);
    *out = ix;
    return JHQ_OK;
}

int jhq_get_plan(const jhq_index* idx, int k, int* scan_kind, int* short_list) {
    if (!idx || k <= 0) return fail(JHQ_EINVAL, "bad argument");
    const int ck = ceil_ck(idx->alpha, k);
    const int P = std::min(idx->nprobe, idx->nlist);
    jhq::ScanShape sh{};
    bool use_mfma = false;
    JHQ_TRY(mfma_choose(const_cast<jhq_index*>(idx), idx->batch_size, P, ck, false, &use_mfma));
    if (!jhq::scan_plan(idx->M, idx->d, P, ck, idx->K1D, idx->batch_size, idx->num_cu, &sh,
                        skew_eligible(idx), use_mfma, idx->RC * idx->Kr))
        return fail(JHQ_EINVAL, "no scan plan fits in LDS");
    if (scan_kind) *scan_kind = sh.mfma ? 4 : sh.dump ? 2 : sh.skew ? 3 : sh.wave ? 1 : 0;
    if (short_list) *short_list = ck;
    return JHQ_OK;
}

int jhq_get_pool(const jhq_index* idx, int64_t* pool_slots, int64_t* pool_capacity) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    if (pool_slots) *pool_slots = idx->pool_used;
    if (pool_capacity) *pool_capacity = idx->pool_cap;
    return JHQ_OK;
}

int jhq_search_ex(jhq_index* idx, const void* q, int dtype, int64_t nq, int k, float* dists,
                  int32_t* ids) {
    if (!idx || !q || !dists || !ids) return fail(JHQ_EINVAL, "null argument");
    if (nq < 0) return fail(JHQ_EINVAL, "nq must be >= 0");
    std::vector<float> tmp;
    const float* qf = nullptr;
    JHQ_TRY(host_f32(q, dtype, nq * static_cast<int64_t>(idx->d), &tmp, &qf));
    return search_host(idx, qf, nq, k, dists, ids, nullptr, nullptr, nullptr, nullptr);
}

int jhq_set_timing(jhq_index* idx, int enable) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    JHQ_TRY(idx->ensure_stream());
    if (enable && !idx->ev[0])
        for (auto& e : idx->ev) JHQ_HIP(hipEventCreate(&e));
    idx->timing = enable != 0;
    for (double& t : idx->tms) t = 0.0;
    idx->tbatches = 0;
    return JHQ_OK;
}

int jhq_get_timing(const jhq_index* idx, double* ms, int n_ms, int64_t* batches) {
    if (!idx) return fail(JHQ_EINVAL, "null index");
    for (int i = 0; i < n_ms && i < kSteps; i++) ms[i] = idx->tms[i];
    if (batches) *batches = idx->tbatches;
    return JHQ_OK;
}

int jhq_k_rotate(const float* d_P, const float* d_x, int64_t n, int d, float* d_y, void* stream) {
    if (!d_P || !d_x || !d_y || n < 0 || d <= 0) return fail(JHQ_EINVAL, "bad argument");
    JHQ_HIP(jhq::gemm_nt_store(d_x, d, d_P, d, n, d, d, d_y, d, n < 1024,
                               static_cast<hipStream_t>(stream)));
    return JHQ_OK;
}

int jhq_k_primary_encode(const float* d_y, uint8_t* d_codes, const float* d_c1d, int64_t n, int d,
                         int M, int Ds, int K1D, int bits_per_dim, void* stream) {
    if (!d_y || !d_codes || !d_c1d || n < 0 || M <= 0 || Ds * M != d || (1 << bits_per_dim) != K1D)
        return fail(JHQ_EINVAL, "bad argument");
    JHQ_HIP(jhq::encode(d_y, n, d, M, Ds, K1D, bits_per_dim, d_c1d, 1, 1, 4, 1, nullptr, d_codes,
                        nullptr, nullptr, 1, static_cast<hipStream_t>(stream)));
    return JHQ_OK;
}

int jhq_k_residual_encode(const float* d_y, const uint8_t* d_primary, uint8_t* d_res_codes,
                          float* d_corrections, const float* d_c1d, const float* d_res_c1d,
                          int64_t n, int d, int M, int Ds, int K1D, int Kr, int Br, int bpv,
                          int bits_per_dim, void* stream) {
    if (!d_y || !d_primary || !d_res_codes || !d_corrections || !d_c1d || !d_res_c1d || n < 0 ||
        M <= 0 || Ds * M != d || (1 << bits_per_dim) != K1D || (Br != 4 && Br != 8) ||
        bpv != (d * Br + 7) / 8 || Kr <= 0 || Kr > (1 << Br))
        return fail(JHQ_EINVAL, "bad argument");
    JHQ_HIP(jhq::encode(d_y, n, d, M, Ds, K1D, bits_per_dim, d_c1d, Kr, 1, Br, bpv, d_res_c1d,
                        const_cast<uint8_t*>(d_primary), d_res_codes, d_corrections, 2,
                        static_cast<hipStream_t>(stream)));
    return JHQ_OK;
}

int jhq_k_assign(const float* d_y, int64_t n, int d, const float* d_cent, const float* d_cent_norms,
                 int nlist, int32_t* d_assign, void* stream) {
    if (!d_y || !d_cent || !d_cent_norms || !d_assign || n < 0 || d <= 0 || nlist <= 0)
        return fail(JHQ_EINVAL, "bad argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    unsigned long long* keys = nullptr;
    JHQ_HIP(hipMallocAsync(reinterpret_cast<void**>(&keys), std::max<int64_t>(n, 1) * 8, s));
    hipError_t e = hipSuccess;
    if (jhq::assign_mfma_ok(d, d_y, d_cent) && (n + 127) / 128 <= 65535) {
        // MFMA scores, fixed-order re-check of near ties: the same lists
        const size_t sf = jhq::assign_mfma_scratch_floats(std::max<int64_t>(n, 1), d, nlist);
        float* scr = nullptr;
        e = hipMallocAsync(reinterpret_cast<void**>(&scr), sf * sizeof(float), s);
        if (e == hipSuccess) {
            e = jhq::assign_mfma(d_y, n, d, d_cent, nlist, d_cent_norms, d_assign, scr, sf, keys, s);
            (void)hipFreeAsync(scr, s);
        }
    } else {
        e = jhq::fill_u64(keys, n, ~0ull, s);
        if (e == hipSuccess) e = jhq::gemm_nt_argmin(d_y, d, d_cent, d, n, nlist, d, d_cent_norms, keys, s);
        if (e == hipSuccess) e = jhq::keys_to_assign(keys, n, d_assign, s);
    }
    (void)hipFreeAsync(keys, s);
    if (e != hipSuccess) return fail(JHQ_EDEVICE, std::string("assign: ") + hipGetErrorString(e));
    return JHQ_OK;
}

int jhq_k_build_lut(const float* d_q_rot, const float* d_c1d, float* d_byte_lut, int B, int d,
                    int M, int Ds, int K1D, int bits_per_dim, void* stream) {
    if (!d_q_rot || !d_c1d || !d_byte_lut || B < 0 || M <= 0 || Ds <= 0 || Ds * M != d ||
        bits_per_dim < 0 || bits_per_dim > 8 || (1 << bits_per_dim) != K1D)
        return fail(JHQ_EINVAL, "bad argument");
    JHQ_HIP(jhq::stage_byte_lut(d_q_rot, d_c1d, d_byte_lut, B, d, M, Ds, K1D, bits_per_dim,
                                static_cast<hipStream_t>(stream)));
    return JHQ_OK;
}

int jhq_k_scan_topck(const float* d_byte_lut, const int32_t* d_probe_ids,
                     const int32_t* d_probe_offsets, const int32_t* d_list_offsets,
                     const uint8_t* d_list_primary_t, const int32_t* d_query_total,
                     float* d_topck_primary, int32_t* d_topck_pos, int B, int nprobe, int M,
                     int64_t N, int ck, void* stream) {
    if (!d_byte_lut || !d_probe_ids || !d_probe_offsets || !d_list_offsets || !d_list_primary_t ||
        !d_query_total || !d_topck_primary || !d_topck_pos || B < 0 || nprobe <= 0 || M <= 0 ||
        N < 0 || N > INT32_MAX || ck <= 0)
        return fail(JHQ_EINVAL, "bad argument");
    hipError_t e = jhq::stage_scan_topck(d_byte_lut, d_probe_ids, d_probe_offsets, d_list_offsets,
                                         d_list_primary_t, d_query_total, d_topck_primary,
                                         d_topck_pos, B, nprobe, M, N, ck,
                                         static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue)
        return fail(JHQ_EINVAL, "nprobe=" + std::to_string(nprobe) + ", ck=" + std::to_string(ck) +
                                    ": the selection state does not fit in LDS");
    JHQ_HIP(e);
    return JHQ_OK;
}

int jhq_k_refine(const float* d_q_rot, const float* d_res_c1d, const int32_t* d_topck_pos,
                 const float* d_topck_primary, const uint8_t* d_list_res, const float* d_list_corr,
                 float* d_comp_dists, int B, int ck, int d, int Kr, int Br, int bpv, void* stream) {
    if (!d_q_rot || !d_res_c1d || !d_topck_pos || !d_topck_primary || !d_list_res ||
        !d_list_corr || !d_comp_dists || B < 0 || ck <= 0 || d <= 0 || (Br != 4 && Br != 8) ||
        Kr <= 0 || Kr > (1 << Br) || bpv != (d * Br + 7) / 8)
        return fail(JHQ_EINVAL, "bad argument");
    JHQ_HIP(jhq::stage_refine(d_q_rot, d_res_c1d, d_topck_pos, d_topck_primary, d_list_res,
                              d_list_corr, d_comp_dists, B, ck, d, Br, bpv,
                              static_cast<hipStream_t>(stream)));
    return JHQ_OK;
}

int jhq_k_final_topk(const float* d_comp_dists, const int32_t* d_topck_pos,
                     const int32_t* d_list_ids, float* d_final_dists, int32_t* d_final_ids, int B,
                     int ck, int k, void* stream) {
    if (!d_comp_dists || !d_topck_pos || !d_list_ids || !d_final_dists || !d_final_ids || B < 0 ||
        ck <= 0 || k <= 0)
        return fail(JHQ_EINVAL, "bad argument");
    hipError_t e = jhq::stage_final_topk(d_comp_dists, d_topck_pos, d_list_ids, d_final_dists,
                                         d_final_ids, B, ck, k, static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue)
        return fail(JHQ_EINVAL, "ck=" + std::to_string(ck) + ", k=" + std::to_string(k) +
                                    ": the selection state does not fit in LDS");
    JHQ_HIP(e);
    return JHQ_OK;
}

int jhq_k_select_probes(const float* d_scores, int B, int nlist, int P,
                        const int32_t* d_list_sizes, int32_t* d_probes, int32_t* d_gofs,
                        int32_t* d_qtot, void* stream) {
    if (!d_scores || !d_list_sizes || !d_probes || !d_gofs || !d_qtot || B <= 0 || nlist <= 0 ||
        P <= 0 || P > nlist)
        return fail(JHQ_EINVAL, "bad argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<int32_t> sizes(nlist);
    JHQ_HIP(hipMemcpyAsync(sizes.data(), d_list_sizes, sizes.size() * 4, hipMemcpyDeviceToHost, s));
    JHQ_HIP(hipStreamSynchronize(s));
    std::vector<int4> h(nlist);
    int64_t cb = 0;
    for (int l = 0; l < nlist; l++) {
        if (sizes[l] < 0) return fail(JHQ_EINVAL, "negative list size");
        h[l] = make_int4(0, sizes[l], sizes[l], static_cast<int>(cb));
        cb += sizes[l];
    }
    DBuf<int4> ld;
    JHQ_TRY(ld.upload(h.data(), h.size()));
    JHQ_HIP(jhq::select_probes(d_scores, B, nlist, P, ld.p, d_probes, d_gofs, d_qtot, s));
    JHQ_HIP(hipStreamSynchronize(s));
    return JHQ_OK;
}

}  // extern "C"
