/*
 * jhq.h — C-ABI of the MI355X-native JHQ IVF engine (libjhq_amd.so).
 *
 * Drop-in boundary for the reference's JHQ search path.  Each entry point names
 * the reference interface it replaces (paths relative to the lrlorry/JHQ_GPU
 * checkout; canonical version jhq_v14_streaming_add, abbreviated v14/).
 *
 * Conventions
 *   - Plain pointers and sizes only; no C++ or torch types cross the boundary.
 *   - Every call returns JHQ_OK (0) or an error code; jhq_last_error() gives
 *     a thread-local message.  Nothing calls exit() (the reference's
 *     CUDA_CHECK/CUBLAS_CHECK exit the process, common/cuda_utils.cuh:7-25).
 *   - Host-pointer calls copy inputs in and outputs out before returning.
 *     Calls with a `_device` suffix or a `jhq_k_` prefix take device pointers
 *     and a HIP stream passed as void* (NULL = the index's own stream for
 *     index calls, the null stream for jhq_k_ calls); they are asynchronous
 *     with respect to the host unless stated otherwise.
 *   - An index is not thread-safe: one call at a time per index (the
 *     reference's search() mutates its workspace the same way,
 *     v14/jhq_gpu_index.cuh:73).
 *
 * Results
 *   ids are int32 positions in add() input order (0-based, counted across
 *   add() calls); dists are the reference's composite estimate
 *   ||q - x_hat||^2 + ||q||^2 (v14/search.cu:240 with v14/encode.cu:85).
 *   Rows are sorted ascending by (dist, id); unfilled slots are (+inf, -1)
 *   (v14/search.cu:284-286).
 */
#ifndef JHQ_H
#define JHQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    JHQ_OK = 0,
    JHQ_EINVAL = 1,  /* bad argument     (reference: std::invalid_argument) */
    JHQ_ESTATE = 2,  /* wrong call order (reference: std::runtime_error)    */
    JHQ_EDEVICE = 3, /* HIP runtime / kernel launch failure                 */
    JHQ_ENOMEM = 4   /* device or host allocation failure                   */
};

/* Element types of host input arrays (the _ex entry points). */
enum {
    JHQ_F32 = 0, /* float32                                   */
    JHQ_U8 = 1,  /* uint8, converted to float32 (0..255)      */
    JHQ_I8 = 2   /* int8, converted to float32 (-128..127)    */
};

typedef struct jhq_index jhq_index;

/* JHQGpuIndex::Params (v14/jhq_gpu_index.cuh:16-36), same fields, same
 * defaults (jhq_params_default). */
typedef struct {
    int   M;          /* subspaces; d % M == 0                        */
    int   B;          /* primary bits per subspace; B % (d/M) == 0, <=8 */
    int   Br;         /* residual bits per dimension: 4 or 8           */
    float alpha;      /* short-list factor: ck = max(k, ceil(alpha*k)) */
    int   nlist;      /* IVF lists                                     */
    int   nprobe;     /* lists probed per query (clamped to nlist)     */
    int   ivf_iters;  /* Lloyd iterations of the coarse k-means        */
    int   batch_size; /* queries per search batch                      */
    int   seed;       /* JL rotation seed                              */
    int   add_batch;  /* rows rotated/encoded per add() step           */
    /* Extension (no reference counterpart; the reference trains one residual
     * codebook for all dimensions, v14/jhq_gpu_index.cu:302-330): 1 trains
     * one Kr-word residual codebook per subspace.  Default 0. */
    int   residual_per_subspace;
} jhq_params;

/* Fills the reference defaults: M=96 B=8 Br=4 alpha=4 nlist=1024 nprobe=8
 * ivf_iters=8 batch_size=256 seed=42 add_batch=65536, and
 * residual_per_subspace=0. */
void jhq_params_default(jhq_params* p);

/* JHQGpuIndex::JHQGpuIndex(int d, Params) — v14/jhq_gpu_index.cu:103-131.
 * Validates the parameters exactly like the reference and builds the JL
 * rotation (cpu/jl_transform.cpp:25-56) on the host. */
int jhq_create(int d, const jhq_params* p, jhq_index** out);

/* JHQGpuIndex::~JHQGpuIndex — v14/jhq_gpu_index.cu:133-163. NULL is a no-op. */
int jhq_destroy(jhq_index* idx);

/* JHQGpuIndex::train(const float* h_x, int n_train) —
 * v14/jhq_gpu_index.cu:333-364.  x is host [n_train x d] row-major. */
int jhq_train(jhq_index* idx, const float* x, int64_t n_train);

/* JHQGpuIndex::add(const float* h_x, int n) — v14/jhq_gpu_index.cu:417-532.
 * x is host [n x d].  Like the reference, one add() call per index;
 * a second call fails with JHQ_ESTATE. */
int jhq_add(jhq_index* idx, const float* x, int64_t n);

/* Typed-input variants of train / add (dtype JHQ_F32, JHQ_U8, JHQ_I8).
 * uint8 / int8 rows cross PCIe as bytes and become float32 on the device.
 * The reference reads such data only in its HBlock line
 * (common/bvecs_io.cuh:13-88, common/spacev_io.cuh:23-65). */
int jhq_train_ex(jhq_index* idx, const void* x, int dtype, int64_t n_train);
int jhq_add_ex(jhq_index* idx, const void* x, int dtype, int64_t n);

/* Streaming add (extension; the reference allows one add(),
 * v14/jhq_gpu_index.cu:419-420): rotates, encodes and assigns n more vectors
 * and appends them to their IVF lists, ids continuing from ntotal.  May be
 * called any number of times after train(), before or after add(), and
 * between searches.  A list that outgrows its block moves to the end of the
 * list pool with 1.5 times the capacity; when the pool has no room left for
 * such moves, every list is re-packed into a new pool with a quarter of
 * headroom each (blocks left behind by earlier moves are dropped).  Results
 * are identical to one add() of all vectors in the same order. */
int jhq_append(jhq_index* idx, const float* x, int64_t n);
int jhq_append_ex(jhq_index* idx, const void* x, int dtype, int64_t n);

/* JHQGpuIndex::search(h_q, nq, k, h_dists, h_labels) —
 * v14/jhq_gpu_index.cu:535-552 -> search_gpu, v14/search.cu:388-445.
 * q host [nq x d]; dists/ids host [nq x k].  Over several batches the
 * host copies of one batch overlap the kernels of the next. */
int jhq_search(jhq_index* idx, const float* q, int64_t nq, int k,
               float* dists, int32_t* ids);

/* search() with typed host queries (dtype JHQ_F32, JHQ_U8, JHQ_I8). */
int jhq_search_ex(jhq_index* idx, const void* q, int dtype, int64_t nq, int k,
                  float* dists, int32_t* ids);

/* Same pipeline with queries and results already in device memory
 * (the reference's graph body v14/search.cu:315-386 without the host
 * copies around it).  Returns after the work is enqueued on `stream`:
 * it allocates nothing and does not synchronise with the host.  It runs in
 * the workspace reserved for k <= k_max (jhq_reserve; add(), append(),
 * load() and the setters reserve k_max = 10 at the index's batch_size,
 * nprobe and alpha) and fails with JHQ_ESTATE for a larger k.
 * More than batch_size queries: consecutive batches rotate through the
 * internal search lanes (a workspace and a stream each; of six created, the
 * ones on hardware queues of their own) forked from `stream`
 * and joined back into it, so the call is stream-ordered on `stream` like a
 * single launch; a lane takes two consecutive batches at a time and runs
 * their query product as one launch (each batch's results are those of
 * its own product).  Consecutive device
 * searches are ordered after each other whatever their streams; add,
 * append, host searches, setters and destroy wait for the last one. */
int jhq_search_device(jhq_index* idx, const float* d_q, int64_t nq, int k,
                      float* d_dists, int32_t* d_ids, void* stream);

/* Preallocates the search workspace (every pipeline lane, pinned staging)
 * for searches with k <= k_max at the current batch_size, nprobe and alpha
 * — the reference's alloc_workspace (v14/jhq_gpu_index.cu:166-206, called at
 * the end of add(), :531) with the ck/k capacities realloc_ck_buffers
 * (v14/search.cu:294-313) grows on demand.  k_max only ever grows.  Host
 * searches with a larger k grow the workspace themselves, like the
 * reference; device searches do not. */
int jhq_reserve(jhq_index* idx, int k_max);

/* JHQGpuIndex::ntotal() / dim() — v14/jhq_gpu_index.cuh:46-47 */
int64_t jhq_ntotal(const jhq_index* idx);
int     jhq_dim(const jhq_index* idx);

/* Params.nprobe is fixed at construction in the reference; changing it
 * recaptures the search graph (v14/search.cu:411-418).  This setter does the
 * same for an existing index (clamped to nlist). */
int jhq_set_nprobe(jhq_index* idx, int nprobe);

/* Params.alpha (short-list factor, ck = max(k, ceil(alpha*k)), v14/search.cu:408)
 * is likewise fixed at construction in the reference; this setter changes it
 * for an existing index. */
int jhq_set_alpha(jhq_index* idx, float alpha);

/* Thread-local message of the last failed call on this thread. */
const char* jhq_last_error(void);

/* ---- introspection (copies to host; used by parity tests and tools) ---- */

/* Derived sizes: Ds, K1D, bits_per_dim, Kr, bpv (v14/jhq_gpu_index.cu:123-128). */
int jhq_get_dims(const jhq_index* idx, int* Ds, int* K1D, int* bpd, int* Kr, int* bpv);

/* Trained state: sigma, c1d[K1D], res_c1d[Kr] (or [M][Kr] with
 * residual_per_subspace), P[d*d] (row-major Pi(j,k),
 * i.e. the transpose of JLTransform::pi_data()), centroids[nlist*d],
 * cent_norms[nlist].  Any pointer may be NULL. */
int jhq_get_codebooks(const jhq_index* idx, float* sigma, float* c1d,
                      float* res_c1d, float* P, float* centroids,
                      float* cent_norms);

/* List storage in stored-position order (the reference's list_* arrays,
 * v14/jhq_gpu_index.cuh:67-71): offsets[nlist+1], ids[ntotal],
 * codes[ntotal*M] (row-major primary codes, untransposed), res[ntotal*bpv],
 * corr[ntotal].  Any pointer may be NULL. */
int jhq_get_lists(const jhq_index* idx, int32_t* offsets, int32_t* ids,
                  uint8_t* codes, uint8_t* res, float* corr);

/* Index files (extension; the reference has no serialization).  jhq_save
 * writes the parameters, the trained state and the lists in canonical order;
 * jhq_load creates a new index from such a file (lists re-packed into a
 * compact pool), ready to search and to append to.  Loading checks the magic,
 * the version, the sizes and that the stored rotation equals the one its seed
 * builds. */
int jhq_save(const jhq_index* idx, const char* path);
/* The index's current parameters (nprobe and alpha as last set). */
int jhq_get_params(const jhq_index* idx, jhq_params* out);
int jhq_load(const char* path, jhq_index** out);

/* Which scan a search with this k runs: 0 workgroup-synchronous selection
 * (scan_topck_kernel), 1 wave-level selection (scan_wave_kernel), 2 every
 * distance to a buffer then one selection per query (scan_dump_kernel +
 * select_query_kernel), 3 wave-level selection with lanes skewed across
 * subspaces (scan_skew_kernel), 4 integer-MFMA pre-scan with an exact
 * re-check (mfma_scan_kernel + mfma_recheck_kernel); and the short-list
 * length ck. */
int jhq_get_plan(const jhq_index* idx, int k, int* scan_kind, int* short_list);

/* Scan choice (no counterpart in the reference, whose search always runs its
 * byte-LUT scan).  The integer-MFMA pre-scan applies to one-bit digits (K1D =
 * 2 with Ds = 8), M a multiple of 16 up to 128 and at most 4096 probes per
 * batch.  0 (default): the pre-scan where it applies and the list sizes
 * predict that the queries of a batch share their probed lists (its 16-query
 * tiles mostly full), else the byte-LUT scans; 1: the byte-LUT scans only;
 * 2: the pre-scan wherever it applies.  Results are identical in every
 * case: the pre-scan only decides which candidates get their distance
 * recomputed in the reference's order.  Re-reserves the search workspace
 * like jhq_set_nprobe. */
int jhq_set_scan_kind(jhq_index* idx, int kind);

/* List pool occupancy: slots in use (including padding, headroom and blocks
 * left behind by moves since the last re-pack) and allocated slots. */
int jhq_get_pool(const jhq_index* idx, int64_t* pool_slots, int64_t* pool_capacity);

/* Search that also returns, per query, the rotated query [nq x d] (the
 * fp32 MFMA product the pipeline used), the probed list ids [nq x nprobe]
 * (ascending (score, list)) and the merged top-ck short list [nq x ck] as
 * stored positions and primary distances ((dist, pos) ascending; unfilled =
 * -1 / +inf).  ck = max(k, ceil(alpha*k)).  Any debug pointer may be NULL. */
int jhq_search_debug(jhq_index* idx, const float* q, int64_t nq, int k,
                     float* dists, int32_t* ids, float* q_rot, int32_t* probes,
                     int32_t* topck_pos, float* topck_dist);

/* Per-step device timing (hipEvents around each step, the reference's
 * step list of jhq_v13_step_timing/search.cu:424-491).  When enabled,
 * every search batch records events; jhq_get_timing returns accumulated
 * milliseconds per step and the number of batches:
 *   ms[0] query rotation + centroid scores (one product)  ms[1] select probes
 *   ms[2] byte LUT + ADC scan + top-ck  ms[3] merge + refine + final top-k
 * Events are recorded on the stream the kernels run on. */
int jhq_set_timing(jhq_index* idx, int enable);
int jhq_get_timing(const jhq_index* idx, double* ms, int n_ms, int64_t* batches);

/* ---- kernel-granular entry points (device pointers) ---- */

/* Rotation Y = X * Pi^T as an fmaf chain over k ascending; P row-major
 * Pi(j,k).  Replaces the cuBLAS Sgemm of v14/jhq_gpu_index.cu:444-448 and
 * v14/search.cu:338-339. */
int jhq_k_rotate(const float* d_P, const float* d_x, int64_t n, int d,
                 float* d_y, void* stream);

/* launch_primary_encode — v14/encode.cuh:7-12, kernel v14/encode.cu:20-41. */
int jhq_k_primary_encode(const float* d_y, uint8_t* d_codes, const float* d_c1d,
                         int64_t n, int d, int M, int Ds, int K1D,
                         int bits_per_dim, void* stream);

/* launch_residual_encode — v14/encode.cuh:14-22, kernel v14/encode.cu:43-86. */
int jhq_k_residual_encode(const float* d_y, const uint8_t* d_primary,
                          uint8_t* d_res_codes, float* d_corrections,
                          const float* d_c1d, const float* d_res_c1d,
                          int64_t n, int d, int M, int Ds, int K1D, int Kr,
                          int Br, int bpv, int bits_per_dim, void* stream);

/* assign_on_gpu + assign_from_dots_kernel — v14/jhq_gpu_index.cu:367-393,
 * 23-40: argmin_c ||c||^2 - 2<c,y>, ties to the lowest c, each score the
 * fixed-order fmaf chain (k ascending).  When d % 4 == 0 (and the arrays are
 * 16-byte aligned) the scores are computed on MFMA and every row whose two
 * best scores lie within the summation-order error bound is re-assigned by
 * the fixed-order kernel, so the result is the same bit for bit.  Temporary
 * device memory comes from the stream-ordered allocator on `stream`. */
int jhq_k_assign(const float* d_y, int64_t n, int d, const float* d_cent,
                 const float* d_cent_norms, int nlist, int32_t* d_assign,
                 void* stream);

/* select_probes_kernel — v14/search.cu:13-62: per query the P lists of
 * smallest score (ties to the lower list id), in that order; gofs[b][P+1] is
 * the prefix of ceil(list_size / 16) over the probes and qtot[b] its total.
 * Any nlist (the reference holds a row in shared memory, v14/search.cu:22-33). */
int jhq_k_select_probes(const float* d_scores, int B, int nlist, int P,
                        const int32_t* d_list_sizes, int32_t* d_probes,
                        int32_t* d_gofs, int32_t* d_qtot, void* stream);

/* build_byte_lut_kernel — v14/search.cu:65-91: d_byte_lut[b][m][v] =
 * sum_{k<Ds} (q_rot[b][m*Ds+k] - c1d[(v >> k*bits_per_dim) & (K1D-1)])^2,
 * one fma per k, k ascending ([B][M][256] floats).  The search pipeline
 * builds the same entries in LDS inside its scan. */
int jhq_k_build_lut(const float* d_q_rot, const float* d_c1d, float* d_byte_lut, int B, int d,
                    int M, int Ds, int K1D, int bits_per_dim, void* stream);

/* scan_ivf_coalesced_kernel — v14/search.cu:105-195, same inputs: the byte
 * LUT [B][M][256], probe_ids [B][nprobe], probe_offsets [B][nprobe+1] (the
 * probed lists' sizes as a prefix), list_offsets [nlist+1], the primary codes
 * transposed to [M][N] (v14/jhq_gpu_index.cu:512-517) and query_total [B].
 * dist = sum over m ascending of lut[m][code_m]; per query the ck smallest
 * (dist, position) pairs, ascending, exact (the reference keeps 4 candidates
 * per thread and is approximate, :116,153-161); unfilled = (+inf, -1). */
int jhq_k_scan_topck(const float* d_byte_lut, const int32_t* d_probe_ids,
                     const int32_t* d_probe_offsets, const int32_t* d_list_offsets,
                     const uint8_t* d_list_primary_t, const int32_t* d_query_total,
                     float* d_topck_primary, int32_t* d_topck_pos, int B, int nprobe, int M,
                     int64_t N, int ck, void* stream);

/* build_residual_lut_batched_kernel + residual_refine_batched_kernel —
 * v14/search.cu:198-242: comp[b][c] = (topck_primary + sum over j ascending of
 * (q_rot[b][j] - res_c1d[r_j])^2) + list_corr[pos], r_j the Br-bit residual
 * code of dimension j (Br = 4: even j in the low nibble); pos < 0 -> +inf.
 * The reference's summation order (the search pipeline's fused refine adds 16
 * partial sums instead). */
int jhq_k_refine(const float* d_q_rot, const float* d_res_c1d, const int32_t* d_topck_pos,
                 const float* d_topck_primary, const uint8_t* d_list_res, const float* d_list_corr,
                 float* d_comp_dists, int B, int ck, int d, int Kr, int Br, int bpv, void* stream);

/* batched_topk_final_kernel — v14/search.cu:244-291: per query the k smallest
 * (comp, id) pairs, id = list_ids[pos], ascending by (dist, id)
 * (jhq_v3_ivf/search.cu:242-279); unfilled = (+inf, -1). */
int jhq_k_final_topk(const float* d_comp_dists, const int32_t* d_topck_pos,
                     const int32_t* d_list_ids, float* d_final_dists, int32_t* d_final_ids, int B,
                     int ck, int k, void* stream);

/* jhq_k_assign without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  Same arguments
 * and results as jhq_k_assign, but the per-row keys live in a fixed device
 * array of 2^20 entries (8 MiB per device, held until the process ends), so
 * n is at most 1048576 (larger n fails with JHQ_EINVAL).  Calls on one device
 * share that array, so each call's stream first waits for the previous call's
 * kernels on that device (one event per device).  Under HIP graph capture no
 * such wait is recorded: replays that overlap each other or other calls on
 * one device race on the array. */
int jhq_k_assign_noalloc(const float* d_y, int64_t n, int d, const float* d_cent,
                         const float* d_cent_norms, int nlist, int32_t* d_assign,
                         void* stream);

#ifdef __cplusplus
}
#endif
#endif /* JHQ_H */
