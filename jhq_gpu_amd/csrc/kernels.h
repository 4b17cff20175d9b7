// kernels.h — launchers of the HIP kernels (gfx950).  Internal C++ interface
// between the C-ABI layer (jhq_capi.hip) and the kernels (kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace jhq {

// LDS available to one workgroup on gfx950.
constexpr int kLdsBytes = 160 * 1024;
// Candidates per padded group of the per-list code-major layout.
constexpr int kGroup = 16;

// C[i][j] = sum_k A[i][k] * Bm[j][k] as an fmaf chain, k ascending from 0.
//   store : C[i*ldc + j] = acc
//   score : C[i*ldc + j] = fmaf(-2, acc, norms[j])     (= norms[j] - 2 acc)
//   argmin: keys[i] = min over j of (ord(fmaf(-2, acc, norms[j])) << 32 | j)
//           (keys must be pre-filled with ~0)
hipError_t gemm_nt_store(const float* A, int64_t lda, const float* Bm, int64_t ldb,
                         int64_t n, int m, int d, float* C, int64_t ldc,
                         bool small_rows, hipStream_t s);
hipError_t gemm_nt_score(const float* A, int64_t lda, const float* Bm, int64_t ldb,
                         int64_t n, int m, int d, const float* norms, float* C,
                         int64_t ldc, bool small_rows, hipStream_t s);
hipError_t gemm_nt_argmin(const float* A, int64_t lda, const float* Bm, int64_t ldb,
                          int64_t n, int m, int d, const float* norms,
                          unsigned long long* keys, hipStream_t s);
// EPI argmin over the rows rowidx[0 .. min(n_max, *ndev)) of A (ndev read on
// the device); keys[i] belongs to row rowidx[i].
hipError_t gemm_nt_argmin_rows(const float* A, int64_t lda, const int32_t* rowidx,
                               const int32_t* ndev, int64_t n_max, const float* Bm, int64_t ldb,
                               int m, int d, const float* norms, unsigned long long* keys,
                               hipStream_t s);
// IVF assignment on bf16 MFMA (each float split into two bf16, three
// products per pair) with the fixed-order argmin re-checking every row whose
// two best approximate scores are closer than the error bound
// (assign_mfma.hip); the result equals gemm_nt_argmin's bit for bit.
// scratch: assign_mfma_scratch_floats(n, d, nlist) floats; keys: n u64.
// Enqueue only.
bool assign_mfma_ok(int d, const float* Y, const float* Cm);
size_t assign_mfma_scratch_floats(int64_t n, int d, int nlist);
hipError_t assign_mfma(const float* Y, int64_t n, int d, const float* Cm, int nlist,
                       const float* norms, int32_t* assign, float* scratch,
                       size_t scratch_floats, unsigned long long* keys, hipStream_t s);
// The number of rows the last assign_mfma on this scratch re-checked
// (device int).
const int32_t* assign_mfma_rechecked(const float* scratch, int64_t n);
// *total += that count (on the stream)
hipError_t assign_mfma_tally(const float* scratch, int64_t n, unsigned long long* total,
                             hipStream_t s);
// The same products on fp32 MFMA for the query side (rotation, centroid
// scores); not a fixed summation order, so only distances and near-tie probe
// choices depend on it, never the stored codes.
// Query product against Bm (N rows of K): columns < nrot are stored to C1,
// the others become scores norms[c] - 2 * dot in C2 (column c - nrot).
// fp32 MFMA, 64 rows x 16*C columns x K/nsplit per workgroup, the launch
// sized to the chip.  mfma_q_ok: K % 64 == 0 and lda, ldb multiples of 4 (A
// and Bm must also be 16-byte aligned).  With nsplit > 1 the split sums pass
// through part (part_floats floats, rows of split sp from sp *
// qb_part_stride) and a second kernel adds them in split order, or, with
// reduce false, the caller's select_probes_qb does; launches sharing part
// must not overlap.
bool mfma_q_ok(int K, int64_t lda, int64_t ldb);
struct QbPlan {
    int C, NI, nsplit, ncg, R;
    size_t part_floats;
};
QbPlan mfma_qb_plan(int nb, int N, int K);
// part floats that cover the plan of every nb <= nb_max
size_t mfma_qb_space(int nb_max, int N, int K);
int64_t qb_part_stride(const QbPlan& p, int N);
hipError_t mfma_qb(const QbPlan& p, const float* A, int64_t lda, const float* Bm, int64_t ldb,
                   int nb, int N, int K, int nrot, float* C1, int64_t ld1, float* C2, int64_t ld2,
                   const float* norms, float* part, size_t part_floats, hipStream_t s,
                   bool reduce = true);
hipError_t mfma_nt_store(const float* A, int64_t lda, const float* Bm, int64_t ldb, int nb, int N,
                         int K, float* C, int64_t ldc, hipStream_t s);
hipError_t mfma_nt_score(const float* A, int64_t lda, const float* Bm, int64_t ldb, int nb, int N,
                         int K, const float* norms, float* C, int64_t ldc, hipStream_t s);
// uint8 (dtype 1) / int8 (dtype 2) elements to float32.
hipError_t convert_to_f32(const void* src, int dtype, int64_t n, float* dst, hipStream_t s);
hipError_t fill_u64(unsigned long long* p, int64_t n, unsigned long long v, hipStream_t s);
// One wave spending a fixed time (iters dependent fmaf steps); *out = the chain's value.
hipError_t lane_probe(float* out, int iters, hipStream_t s);
hipError_t keys_to_assign(const unsigned long long* keys, int64_t n, int32_t* assign,
                          hipStream_t s);

// Primary / residual encode.  mode bit 0: compute and write primary codes from
// y; mode bit 1: residual codes + corrections (primary digits from y when bit 0
// is set, else read from `codes`).  res_c1d holds RC codebooks of Kr words:
// RC = 1 (one codebook for every dimension) or RC = M (one per subspace).
hipError_t encode(const float* y, int64_t n, int d, int M, int Ds, int K1D, int bpd,
                  const float* c1d, int Kr, int RC, int Br, int bpv, const float* res_c1d,
                  uint8_t* codes, uint8_t* res, float* corr, int mode, hipStream_t s);

// Coarse k-means on the device (kmeans.hip).  kmeans_init: centroid c =
// row c * n / nlist of y [n x d].  kmeans_update: the means of the rows of
// each list given the assignment asg [n], summed in double in ascending row
// order, an empty list reseeded from row (c * 1103515245 + iter * 12345) % n;
// scratch of kmeans_scratch_bytes(n, nlist) bytes.  kmeans_norms: ||c||^2 in
// double, j ascending.
hipError_t kmeans_init(const float* y, int d, int64_t n, int nlist, float* cent, hipStream_t s);
size_t kmeans_scratch_bytes(int64_t n, int nlist);
hipError_t kmeans_update(const int32_t* asg, const float* y, int d, int64_t n, int nlist, int iter,
                         float* cent, void* scratch, size_t scratch_bytes, hipStream_t s);
hipError_t kmeans_norms(const float* cent, int d, int nlist, float* norms, hipStream_t s);
// keys (asg[i] << 32 | i) sorted ascending into the scratch (same size as
// kmeans_scratch_bytes), and first[l] = index of list l's first sorted key
// (first[nlist] = n); the two pointers point into the scratch.
hipError_t list_order(const int32_t* asg, int64_t n, int nlist, void* scratch, size_t scratch_bytes,
                      const unsigned long long** sorted, const int64_t** first, hipStream_t s);
// From list_order's output: order[p] = vector, slist[p] = its list, sidx[p] =
// ldesc[list].z + its rank in the list (the scatter_lists inputs).
hipError_t scatter_plan(const unsigned long long* sorted, const int64_t* first, const int4* ldesc,
                        int64_t n, int32_t* order, int32_t* slist, int32_t* sidx, hipStream_t s);

// List storage: one pool of padded candidate slots; list l is described by
// int4 {start, cap, size, cbase}: slots [start, start + cap) with cap a
// multiple of kGroup, size candidates, first canonical position cbase
// (lists in list order, candidates in insertion order).  Byte m of candidate
// i is at codes_t[start*M + m*cap + i]; residual codes, corrections and ids
// are indexed by slot.
//
// Scatter: new vector s goes to list slist[s] at index sidx[s]; its id is
// id_base + order[s], order[s] indexing the per-vector inputs pc/rc/co.
// Lane-skewed rows of the primary codes (row[t] = code[(t - i mod 32) mod M]
// for candidate i of each list, the wrapped bytes t < i mod 32 stored as
// code + 1 mod 256), in blocks of 16 slots stored piece by piece (16 bytes of
// each slot's row per piece); skew_bytes(pool_cap, M) bytes.  Rows from[l] ..
// size-1 of list l (from: device [nlist]), max_rows >= the largest
// size - from[l].  M % 32 == 0, M <= 256.
hipError_t skew_codes(const int4* ldesc, const int32_t* from, int nlist, int max_rows,
                      const uint8_t* codes_t, int M, uint8_t* skew, hipStream_t s);
int64_t skew_bytes(int64_t pool_cap, int M);
// Row-major copy of the primary codes (slot p's M bytes at rows[p * M],
// pool_cap * M bytes; M a multiple of 16), rows from[l] .. size-1 of each
// list l (from rounded down to 16).
hipError_t row_codes(const int4* ldesc, const int32_t* from, int nlist, int max_rows,
                     const uint8_t* codes_t, int M, uint8_t* rows, hipStream_t s);
hipError_t scatter_lists(const int32_t* order, const int32_t* slist, const int32_t* sidx,
                         int64_t n, int64_t id_base, const int4* ldesc, const uint8_t* pc,
                         const uint8_t* rc, const float* co, int M, int bpv, int32_t* ids_out,
                         uint8_t* codes_t, uint8_t* res_out, float* corr_out, hipStream_t s);
// Moves list blocks: moves[2r] = {start, cap, size} (source), moves[2r+1] =
// {start, cap} (destination); blocks must not overlap.
hipError_t relocate_lists(const int4* moves, int nmoves, int M, int bpv, const uint8_t* codes_src,
                          uint8_t* codes_dst, const uint8_t* res_src, uint8_t* res_dst,
                          const float* corr_src, float* corr_dst, const int32_t* ids_src,
                          int32_t* ids_dst, hipStream_t s);

// The integer-MFMA pre-scan's share of the probe selection (see mfma_scan):
// its workspace (ws, ws_bytes, laid out for Bcap queries) and dump buffer
// size (dump_slots, as given to mfma_scan), the rotated queries (q_rot
// [B][d]; unused by select_probes_qb, which forms them) and the primary
// codebook c1d; d = 8 M.
struct PrescanSel {
    unsigned char* ws;
    size_t ws_bytes;
    int64_t dump_slots;
    const float* q_rot;
    const float* c1d;
    int d, M, Bcap;
};

// Per query: exact top-P lists by (score, list) from scores[b][nlist];
// writes probes[b][P] (ascending), gofs[b][P+1] (prefix of padded group
// counts) and qtot[b] (= gofs[b][P]).  With ps, also the pre-scan's query
// steps and the batch's (query, probe) pairs in its list hash.
hipError_t select_probes(const float* scores, int B, int nlist, int P, const int4* ldesc,
                         int32_t* probes, int32_t* gofs, int32_t* qtot, hipStream_t s,
                         const PrescanSel* ps = nullptr);
// The same from the split sums of mfma_qb (plan p, launched with reduce
// false, part as given there): each query's workgroup adds its row's splits
// in split order, stores the rotated query (the first nrot columns) to C1
// and selects from the scores norms - 2 dot, held in LDS (no second kernel,
// no score rows in HBM).  select_adds_qb: whether the shape allows it.
bool select_adds_qb(const QbPlan& p, int nlist, int nrot);
hipError_t select_probes_qb(const QbPlan& p, const float* part, int nrot, float* C1, int64_t ld1,
                            const float* norms, int B, int nlist, int P, const int4* ldesc,
                            int32_t* probes, int32_t* gofs, int32_t* qtot, hipStream_t s,
                            const PrescanSel* ps = nullptr);

// rows[i] = the stored vector at column samp[i].z of the list block (start
// samp[i].x, row stride samp[i].y) decoded from its primary code (rotated
// space, one Lloyd-Max level per coordinate)
hipError_t decode_rows(const int4* samp, int S, const uint8_t* codes_t, int M, int Ds, int K1D,
                       int bpd, const float* c1d, float* rows, hipStream_t s);

struct ScanShape {
    int G;             // persistent scan workgroups
    int lds;           // dynamic LDS bytes of the scan kernel
    int max_segments;  // upper bound on top-ck lists per batch (partial rows)
    int wave;          // 0: workgroup-synchronous selection; J: wave selection, 64*J-key buffers
    int nt;            // threads per scan workgroup
    int skew;          // M / 4 when the lane-skewed scan runs (needs the skewed codes)
    int dump;          // 1: every distance to a buffer, then one selection per query (region
                       // = that kernel's LDS); the buffer holds B * (groups of the P largest
                       // lists) * 16 keys
    int region;        // wave selection: bytes of the LUT / merge region
    int ov;            // work plan: virtual groups per query (the cost of a segment)
    int mfma;          // 1: integer-MFMA pre-scan + exact re-check, one segment per query
                       // (B * (groups of the P largest lists) * 16 u32 values in the dump
                       // buffer and mfma_scan_bytes of workspace)
};
// LDS plan of the scan kernel; returns false if the byte LUT and the
// selection buffers do not fit.  rck: residual codebook floats (RC * Kr),
// which the pre-scan's re-check holds for its refine.
bool scan_plan(int M, int d, int P, int ck, int K1D, int B, int target_wg, ScanShape* out,
               bool skew = false, bool mfma = false, int rck = 0);

// Integer-MFMA pre-scan for one-bit digits (K1D = 2, Ds = 8, M a multiple of
// 16 up to 128): per query the distances C + s * I(x) with I exact from int8
// MFMA products over the batch's shared lists, then every candidate that the
// error bound cannot exclude from the exact top-ck is re-checked with the
// reference's arithmetic.  When mfma_fuses_refine(ck), the exact top-ck is
// refined in the same workgroup as refine_topk refines a merged one: out_d /
// out_i [B][k] and (optional) topck_dbg [B][ck] as refine_topk writes them;
// otherwise it goes to partial[query's segment][ck] (one segment per query)
// and the caller runs refine_topk.  dump holds one
// u32 per candidate slot (dump_slots, a multiple of 16, at least B times the
// largest qtot times 16: query b's row starts at b times dump_slots / B
// rounded down to 16) and after them one per 16 slots; ws (256-byte
// aligned) holds mfma_scan_bytes(Bcap, P, M) and is laid out for Bcap
// queries whatever the batch's B.  rows: the
// current row-major copy of the codes (row_codes), which the tiles and the
// re-check read; codes_t: the code-major blocks (the re-check's streamed
// fallback).  rck = RC * Kr.
// The probe selection (select_probes or select_probes_qb with a
// PrescanSel over the same ws and dump) must run first on the same stream:
// it quantizes the queries and lists the batch's (query, probe) pairs in a
// hash of the probed lists in ws, which the tile kernel reads and the
// re-check clears for the next batch.  A new ws, one last used with another
// P, or one a batch left between its selection and its mfma_scan, is
// cleared with mfma_hash_clear (same Bcap, P and M).
bool mfma_scan_ok(int M, int d, int Ds, int K1D, int bpd, int B, int P, int ck, int rck);
hipError_t mfma_hash_clear(int Bcap, int P, int M, unsigned char* ws, size_t ws_bytes,
                           hipStream_t s);
bool mfma_fuses_refine(int ck);
size_t mfma_scan_bytes(int B, int P, int M, int num_cu);
hipError_t mfma_scan(const float* q_rot, int d, int Ds, int K1D, int bpd, const float* c1d, int B,
                     int M, const int32_t* probes, const int32_t* gofs, const int32_t* qtot, int P,
                     const int4* ldesc, const uint8_t* codes_t, const uint8_t* rows, int ck,
                     uint32_t* dump, int64_t dump_slots, unsigned char* ws, size_t ws_bytes,
                     int k, const float* res_c1d, int Kr, int RC, int Br, int bpv,
                     const uint8_t* list_res, const float* list_corr, const int32_t* list_ids,
                     float* out_d, int32_t* out_i, unsigned long long* topck_dbg,
                     unsigned long long* partial, int32_t* partial_slot, int num_cu, int Bcap,
                     hipStream_t s);

// IVF ADC scan + exact top-ck per segment with the byte LUT built in LDS from
// q_rot (v14/search.cu:65-195); partial[segment][ck] keys
// (ord(dist) << 32 | canonical position), unfilled = ~0, and the candidates'
// pool slots in partial_slot[segment][ck].
hipError_t scan_topck(const float* q_rot, int d, int Ds, int K1D, int bpd, const float* c1d,
                      int B, int M, const int32_t* probes, const int32_t* gofs,
                      const int32_t* qtot, int P, const int4* ldesc, const uint8_t* codes_t,
                      int ck, const ScanShape& sh, unsigned long long* partial,
                      int32_t* partial_slot, unsigned long long* dump, const uint8_t* skew, hipStream_t s);

// Per query: merge its segment lists, residual refine, final top-k.
// If topck_dbg != nullptr it receives the merged short list [B][ck] keys.
hipError_t refine_topk(const unsigned long long* partial, const int32_t* partial_slot,
                       const int32_t* qtot, int B, const ScanShape& sh, int ck, int k,
                       const float* q_rot, int d, int Ds, const float* res_c1d, int Kr, int RC,
                       int Br, int bpv, const int4* ldesc, int nlist, const uint8_t* list_res,
                       const float* list_corr, const int32_t* list_ids, float* out_d,
                       int32_t* out_i, unsigned long long* topck_dbg, hipStream_t s);

// Search stages in the reference's data layout (kernel-granular C-ABI):
// byte LUT [B][M][256] (v14/search.cu:65-91); exact top-ck per query over
// [M][N] transposed codes and list_offsets (v14/search.cu:105-195); residual
// refine in the reference's order (v14/search.cu:198-242); exact final top-k
// by (dist, id) (v14/search.cu:244-291).
hipError_t stage_byte_lut(const float* q_rot, const float* c1d, float* lut, int B, int d, int M,
                          int Ds, int K1D, int bpd, hipStream_t s);
hipError_t stage_scan_topck(const float* byte_lut, const int32_t* probe_ids,
                            const int32_t* probe_offsets, const int32_t* list_offsets,
                            const uint8_t* primary_t, const int32_t* query_total, float* out_d,
                            int32_t* out_p, int B, int nprobe, int M, int64_t N, int ck,
                            hipStream_t s);
hipError_t stage_refine(const float* q_rot, const float* res_c1d, const int32_t* topck_pos,
                        const float* topck_primary, const uint8_t* list_res,
                        const float* list_corr, float* comp, int B, int ck, int d, int Br,
                        int bpv, hipStream_t s);
hipError_t stage_final_topk(const float* comp, const int32_t* topck_pos, const int32_t* list_ids,
                            float* out_d, int32_t* out_i, int B, int ck, int k, hipStream_t s);

}  // namespace jhq
