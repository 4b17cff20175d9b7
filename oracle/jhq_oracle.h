/*
 * jhq_oracle.h — CPU restatement of the lrlorry/JHQ_GPU JHQ IVF path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * in jhq_gpu_amd/: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).  Floating-point order is pinned explicitly:
 * the library is built with -ffp-contract=off and uses fmaf() exactly where the
 * reference's build contracts a multiply-add (nvcc --use_fast_math for device
 * code, gcc -O3 -march=native for cpu/).  The GPU product follows the same
 * order for codes, corrections, LUT entries and primary distances, so those
 * are bit-exact between the two.  The product's query rotation and centroid
 * scores run on fp32 MFMA; o_search_ex takes the product's rotated queries
 * and probe lists so that every later stage is compared bit for bit.
 *
 * Pinning status (what checks each function; see tests/test_oracle_*.py):
 *   o_mt_*               mt19937 known answer (10000th draw of seed 5489) and
 *                        libstdc++ std::mt19937 via oracle/_ref
 *   o_normal_fill        libstdc++ std::normal_distribution<float> via oracle/_ref
 *   o_erfinv_f, o_lloyd_max_c1d
 *                        reference cpu/erfinv.h + cpu/codebook.cpp built into
 *                        oracle/_ref (bit-exact) and scipy ndtri closed form
 *   o_estimate_sigma     numpy float64 closed form
 *   o_train_1d_kmeans    reference cpu/codebook.cpp via oracle/_ref (bit-exact),
 *                        hand-computed cases, Lloyd fixed-point invariant
 *   o_householder_qr     scipy LAPACK sgeqrf/sorgqr goldens, orthogonality, Q·R=G
 *   o_rotate             numpy float64 matmul (tolerance), fmaf-chain order
 *   o_primary_encode, o_residual_encode
 *                        reference LloydMaxCodebook::encode via oracle/_ref,
 *                        brute-force nearest codeword (numpy)
 *   o_flat_lut, o_factored_lut, o_adc_flat
 *                        reference build_flat_lut / build_lut / adc_distance via
 *                        oracle/_ref (bit-exact), closed form (numpy)
 *   o_assign, o_train_ivf
 *                        numpy brute force on tiny inputs
 *   o_select_topk_pairs, o_search
 *                        numpy stable argsort brute force; composite distance
 *                        identity ||q - (yhat + rhat)||^2 + ||q||^2
 *   o_search_mode(1)     (the reference's approximate selection) a
 *                        pure-Python loop transcription of the 256-thread
 *                        block on small cases, and the properties that fix
 *                        it: exact whenever every thread holds at most 4
 *                        candidates; a thread's 5th-best candidate is lost
 */
#ifndef JHQ_ORACLE_H
#define JHQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads for the row-parallel loops (rotation, encode, assignment and
 * search run one vector or query per thread, so results do not depend on
 * the count).  Default 1. */
void o_set_threads(int n);
int  o_get_threads(void);

/* ---- std::mt19937 and std::normal_distribution<float> (libstdc++) ---- */
typedef struct {
    uint32_t mt[624];
    int      idx;
} o_mt19937;

void     o_mt_seed(o_mt19937* g, uint32_t seed);
uint32_t o_mt_next(o_mt19937* g);
/* n draws of normal_distribution<float>(0,1) driven by mt19937(seed). */
void     o_normal_fill(uint32_t seed, float* out, int64_t n);
/* first n raw mt19937 outputs */
void     o_mt_fill(uint32_t seed, uint32_t* out, int64_t n);

/* ---- host train math (cpu/) ---- */
float o_erfinv_f(float x);
void  o_lloyd_max_c1d(float sigma, int K1D, float* c1d);
float o_estimate_sigma(const float* x, int64_t n, int d);
/* returns the number of codewords written (min(Kr, n)) */
int   o_train_1d_kmeans(const float* vals, int64_t n, int Kr, int max_iter, float* out);
/* In-place Householder QR of the d x d column-major matrix A; on return A holds
 * Q (column-major).  Computed in double, LAPACK xGEQR2/xORG2R conventions. */
int   o_householder_qr(int d, float* A);
/* Pi_colmajor as JLTransform::build_rotation leaves it. */
void  o_build_rotation(int d, int seed, float* Pi_colmajor);

/* ---- rotation / encode ---- */
/* y[i][j] = sum_k x[i][k] * P[j][k] as an fmaf chain, k ascending from 0.
 * P is Pi in row-major order (P[j][k] = Pi(j,k)). */
void o_rotate(const float* P, const float* x, int64_t n, int d, float* y);
void o_primary_encode(const float* y, int64_t n, int d, int M, const float* c1d,
                      int K1D, uint8_t* codes);
void o_residual_encode(const float* y, const uint8_t* primary, int64_t n, int d,
                       int M, const float* c1d, int K1D, const float* res_c1d,
                       int Kr, int Br, uint8_t* res_codes, float* corr);
void o_residual_encode_rc(const float* y, const uint8_t* primary, int64_t n, int d,
                          int M, const float* c1d, int K1D, const float* res_c1d,
                          int Kr, int RC, int Br, uint8_t* res_codes, float* corr);
void o_reconstruct(const uint8_t* code, int d, int M, const float* c1d, int K1D,
                   float* out);

/* ---- LUTs and ADC ---- */
void  o_flat_lut(const float* q_rot, int d, int M, const float* c1d, int K1D,
                 float* lut /* [M][256] */);
void  o_factored_lut(const float* q_rot, int d, int M, const float* c1d, int K1D,
                     float* lut /* [M][Ds][K1D] */);
float o_adc_flat(const uint8_t* code, int M, const float* lut);
float o_adc_factored(const uint8_t* code, int d, int M, int K1D, const float* lut);

/* ---- IVF ---- */
void o_cent_norms(const float* cent, int nlist, int d, float* norms);
void o_assign(const float* y, int64_t n, int d, const float* cent,
              const float* norms, int nlist, int32_t* out);
/* k-means in rotated space; returns 0, or -1 if n < nlist */
int  o_train_ivf(const float* y, int64_t n, int d, int nlist, int iters,
                 float* cent /* out [nlist][d] */);

/* ---- selection ---- */
/* Exact top-k of (dist, tag) pairs ordered by (dist, tag) ascending.
 * Unfilled slots get (+inf, -1).  Returns the number of filled slots. */
int  o_select_topk_pairs(const float* dist, const int32_t* tag, int64_t n, int k,
                         float* out_dist, int32_t* out_tag);

/* ---- whole index ---- */
typedef struct {
    int d, M, B, Br, Ds, K1D, bpd, Kr, bpv;
    int nlist, nprobe;
    int RC;                     /* residual codebooks: 1, or M (per subspace) */
    float alpha;
    int64_t ntotal;
    const float*   P;           /* [d][d] row-major Pi(j,k)                 */
    const float*   c1d;         /* [K1D]                                   */
    const float*   res_c1d;     /* [RC][Kr]                                */
    const float*   cent;        /* [nlist][d]                              */
    const float*   cent_norms;  /* [nlist]                                 */
    const int32_t* list_offsets;/* [nlist+1]                               */
    const int32_t* list_ids;    /* [ntotal]  id of each stored position    */
    const uint8_t* list_codes;  /* [ntotal][M] primary codes, list order   */
    const uint8_t* list_res;    /* [ntotal][bpv] residual codes            */
    const float*   list_corr;   /* [ntotal]                                */
} o_index;

/* Per-query search with the reference pipeline; outputs are [nq][k].
 * If dbg_probes != NULL it receives [nq][nprobe] probed list ids;
 * if dbg_topck_pos/dist != NULL they receive [nq][ck] candidates. */
int o_search(const o_index* ix, const float* q, int64_t nq, int k,
             float* out_dist, int32_t* out_ids,
             int32_t* dbg_probes, int32_t* dbg_topck_pos, float* dbg_topck_dist);
/* Stage-wise variant: if q_rot_in != NULL it holds the rotated queries
 * [nq][d] to use instead of rotating q; if probes_in != NULL it holds the
 * probed lists [nq][nprobe] to use instead of selecting them.  The rest of
 * the pipeline is o_search's. */
int o_search_ex(const o_index* ix, const float* q, const float* q_rot_in,
                const int32_t* probes_in, int64_t nq, int k,
                float* out_dist, int32_t* out_ids,
                int32_t* dbg_probes, int32_t* dbg_topck_pos, float* dbg_topck_dist);
/* mode 0: o_search_ex.  mode 1: the same pipeline with the reference's own
 * approximate selection (jhq_v14_streaming_add/search.cu:105-195 per-thread
 * top-4 + block argmin, and :244-291 final block argmin), to measure how
 * often the reference's search differs from exact selection. */
int o_search_mode(const o_index* ix, const float* q, const float* q_rot_in,
                  const int32_t* probes_in, int64_t nq, int k, int mode,
                  float* out_dist, int32_t* out_ids,
                  int32_t* dbg_probes, int32_t* dbg_topck_pos, float* dbg_topck_dist);
/* ck = max(k, ceil(alpha * k)) (jhq_v14_streaming_add/search.cu:408) */
int o_ck(float alpha, int k);

/* Build the IVF list storage exactly like JHQGpuIndex::add: stable order by
 * (list, id).  order[pos] = id, offsets[nlist+1]. */
void o_build_lists(const int32_t* assign, int64_t n, int nlist,
                   int32_t* offsets, int32_t* order);

#ifdef __cplusplus
}
#endif
#endif
