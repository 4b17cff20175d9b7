// kernels.hip — HIP kernels of the JHQ IVF engine for gfx950 (CDNA4).
//
// Compiled with -ffp-contract=off: every fused multiply-add is an explicit
// fmaf() placed where the reference (nvcc --use_fast_math) contracts one, so
// rotations, codes, LUT entries, primary distances and probe scores are
// bit-identical to the CPU restatement of the reference.
//
// Reference path (lrlorry/JHQ_GPU, jhq_v14_streaming_add = v14/):
//   rotation          cuBLAS Sgemm            v14/jhq_gpu_index.cu:444-448, search.cu:338-339
//   centroid scores   cuBLAS Sgemm            v14/search.cu:341-342
//   assignment        assign_from_dots_kernel v14/jhq_gpu_index.cu:23-40
//   encode            primary/residual kernels v14/encode.cu:20-86
//   list build        sort + gather + transpose v14/jhq_gpu_index.cu:468-519
//   probe selection   select_probes_kernel    v14/search.cu:13-62
//   byte LUT          build_byte_lut_kernel   v14/search.cu:65-91
//   ADC scan + top-ck scan_ivf_coalesced_kernel v14/search.cu:105-195
//   refine            residual kernels        v14/search.cu:198-242
//   final top-k       batched_topk_final_kernel v14/search.cu:244-291
// Selection follows the exact (value, tag) order of jhq_v3_ivf/search.cu:22-25.
#include "kernels.h"

#include <hip/hip_runtime.h>
#include <cstdint>

namespace jhq {

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f2ord(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// Block-wide exact selection state (LDS).
struct SelState {
    uint32_t hist[256];
    uint32_t orv;
    uint32_t v0;
    uint32_t prefix;
    uint32_t krem;
    uint32_t eq;
    int cnt;
    int aux;
};

struct SelResult {
    uint32_t mask, prefix, krem;
    bool done;  // true: every element with (v & mask) == prefix is selected
};

// Radix select of the k-th smallest of n u32 values (1 <= k <= n), MSB first
// from the highest bit where the values differ, 8-bit digits, LDS histogram.
// Returns the rule: v selected iff (v & mask) < prefix, or (v & mask) == prefix
// and (done, or the element wins the tie-break among equal values).
template <int NT, class GetV>
__device__ SelResult sel_threshold(GetV getv, int n, uint32_t k, SelState* st) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid == 0) { st->orv = 0u; st->v0 = getv(0); }
    __syncthreads();
    const uint32_t v0 = st->v0;
    uint32_t o = 0u;
    for (int i = tid; i < n; i += NT) o |= getv(i) ^ v0;
    for (int off = 32; off > 0; off >>= 1) o |= __shfl_xor(o, off);
    if (lane == 0 && o) atomicOr(&st->orv, o);
    __syncthreads();
    const uint32_t orv = st->orv;
    SelResult r;
    int shift;
    if (orv == 0u) {
        r.mask = ~0u; r.prefix = v0; shift = 0;
    } else {
        const int hb = 31 - __clz(orv);
        r.mask = (hb >= 31) ? 0u : (~0u << (hb + 1));
        r.prefix = v0 & r.mask;
        shift = hb + 1;
    }
    r.krem = k;
    uint32_t eq = (uint32_t)n;
    r.done = (k == (uint32_t)n);
    while (!r.done && shift > 0) {
        const int lo = shift > 8 ? shift - 8 : 0;
        const uint32_t dm = (shift - lo == 32) ? ~0u : ((1u << (shift - lo)) - 1u);
        for (int i = tid; i < 256; i += NT) st->hist[i] = 0u;
        __syncthreads();
        for (int i = tid; i < n; i += NT) {
            const uint32_t v = getv(i);
            if ((v & r.mask) == r.prefix) atomicAdd(&st->hist[(v >> lo) & dm], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            const uint32_t c0 = st->hist[tid * 4 + 0], c1 = st->hist[tid * 4 + 1];
            const uint32_t c2 = st->hist[tid * 4 + 2], c3 = st->hist[tid * 4 + 3];
            const uint32_t s = c0 + c1 + c2 + c3;
            uint32_t inc = s;
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t t = __shfl_up(inc, off);
                if (lane >= off) inc += t;
            }
            uint32_t base = inc - s;
            const uint32_t cb[4] = {c0, c1, c2, c3};
            for (int j = 0; j < 4; j++) {
                if (base < r.krem && r.krem <= base + cb[j]) {
                    st->prefix = r.prefix | ((uint32_t)(tid * 4 + j) << lo);
                    st->krem = r.krem - base;
                    st->eq = cb[j];
                }
                base += cb[j];
            }
        }
        __syncthreads();
        r.prefix = st->prefix;
        r.krem = st->krem;
        eq = st->eq;
        r.mask |= dm << lo;
        shift = lo;
        r.done = (eq == r.krem);
        __syncthreads();
    }
    return r;
}

// Ballot compaction of pred(i) over i < n into out[], counter st->cnt
// (zeroed here).  Returns the count.
template <int NT, class Pred>
__device__ int sel_compact(Pred pred, int n, int* out, int cap, SelState* st) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid == 0) st->cnt = 0;
    __syncthreads();
    for (int base = 0; base < n; base += NT) {
        const int i = base + tid;
        const bool p = (i < n) && pred(i);
        const unsigned long long bal = __ballot(p);
        int wbase = 0;
        if (lane == 0 && bal) wbase = atomicAdd(&st->cnt, __popcll(bal));
        wbase = __shfl(wbase, 0);
        const int at = wbase + __popcll(bal & ((1ull << lane) - 1ull));
        if (p && at < cap) out[at] = i;
    }
    __syncthreads();
    return st->cnt;
}

// sorted[rank] = idx[a], rank by less() over the m selected (distinct keys).
template <int NT, class Less>
__device__ void rank_sort(const int* idx, int m, int* sorted, Less less) {
    for (int a = threadIdx.x; a < m; a += NT) {
        const int ia = idx[a];
        int r = 0;
        for (int b2 = 0; b2 < m; b2++) r += less(idx[b2], ia) ? 1 : 0;
        if (r < m) sorted[r] = ia;
    }
    __syncthreads();
}

// Exact top-k of n elements by (getv, gett) ascending (gett distinct among
// equal getv).  Writes the k selected element indices, sorted, to sorted[].
// scratch must hold k ints.  Requires 1 <= k <= n.
template <int NT, class GetV, class GetT>
__device__ int block_topk(GetV getv, GetT gett, int n, int k, int* scratch, int* sorted,
                          SelState* st) {
    const SelResult r = sel_threshold<NT>(getv, n, (uint32_t)k, st);
    SelResult t;
    t.mask = 0u; t.prefix = 0u; t.done = true; t.krem = 0u;
    if (!r.done) {
        // ties at the exact threshold value: keep the r.krem smallest tags
        const uint32_t pv = r.prefix;
        t = sel_threshold<NT>([&](int i) { return (getv(i) == pv) ? gett(i) : ~0u; }, n, r.krem,
                              st);
    }
    const bool rdone = r.done;
    const uint32_t rmask = r.mask, rpre = r.prefix, tmask = t.mask, tpre = t.prefix;
    int cnt = sel_compact<NT>(
        [&](int i) {
            const uint32_t v = getv(i) & rmask;
            if (v < rpre) return true;
            if (v != rpre) return false;
            if (rdone) return true;
            return (gett(i) & tmask) <= tpre;
        },
        n, scratch, k, st);
    cnt = cnt < k ? cnt : k;
    // every slot of sorted[] holds a valid element index even if the
    // selection were to come up short
    for (int r = threadIdx.x; r < k; r += NT) sorted[r] = 0;
    __syncthreads();
    rank_sort<NT>(scratch, cnt, sorted, [&](int a, int b2) {
        const uint32_t va = getv(a), vb = getv(b2);
        return va < vb || (va == vb && gett(a) < gett(b2));
    });
    return cnt;
}

// ---------------------------------------------------------------------------
// Fixed-order SIMT GEMM  C = A * Bm^T  (both operands k-contiguous rows)
// ---------------------------------------------------------------------------
enum { EPI_STORE = 0, EPI_SCORE = 1, EPI_ARGMIN = 2 };

template <int BM, int BN, int BK, int TM, int TN, int EPI>
__global__ void __launch_bounds__((BM / TM) * (BN / TN))
gemm_nt_kernel(const float* __restrict__ A, int64_t lda, const float* __restrict__ Bm,
               int64_t ldb, int64_t n, int m, int d, float* __restrict__ C, int64_t ldc,
               const float* __restrict__ norms, unsigned long long* __restrict__ amin) {
    constexpr int TX = BN / TN, TY = BM / TM, NT = TX * TY;
    constexpr int AL = BM * BK / NT, BL = BN * BK / NT;
    static_assert((BM * BK) % NT == 0 && (BN * BK) % NT == 0, "tile/threads mismatch");
    static_assert(TX <= 64 && (TX & (TX - 1)) == 0, "TX must be a power of two <= 64");
    __shared__ __align__(16) float As[2][BK][BM + 4];
    __shared__ __align__(16) float Bs[2][BK][BN + 4];
    const int tid = threadIdx.x;
    const int tx = tid % TX, ty = tid / TX;
    const int64_t row0 = (int64_t)blockIdx.y * BM;
    const int col0 = blockIdx.x * BN;

    float ra[AL], rb[BL];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int e = tid + i * NT, r = e / BK, kk = e % BK;
            const int64_t gr = row0 + r;
            const int gk = k0 + kk;
            ra[i] = (gr < n && gk < d) ? A[gr * lda + gk] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < BL; i++) {
            const int e = tid + i * NT, r = e / BK, kk = e % BK;
            const int gc = col0 + r, gk = k0 + kk;
            rb[i] = (gc < m && gk < d) ? Bm[(int64_t)gc * ldb + gk] : 0.0f;
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int e = tid + i * NT;
            As[buf][e % BK][e / BK] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BL; i++) {
            const int e = tid + i * NT;
            Bs[buf][e % BK][e / BK] = rb[i];
        }
    };
    // thread's rows / cols: groups of 4 interleaved across the tile when
    // TM (TN) is a multiple of 4, contiguous otherwise.
    auto row_of = [&](int i) {
        return (TM % 4 == 0) ? (i / 4) * (TY * 4) + ty * 4 + (i % 4) : ty * TM + i;
    };
    auto col_of = [&](int j) {
        return (TN % 4 == 0) ? (j / 4) * (TX * 4) + tx * 4 + (j % 4) : tx * TN + j;
    };

    float acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = 0.0f;

    const int nk = (d + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int t = 0; t < nk; t++) {
        const int buf = t & 1;
        if (t + 1 < nk) gload((t + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk++) {
            float a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = As[buf][kk][row_of(i)];
#pragma unroll
            for (int j = 0; j < TN; j++) b[j] = Bs[buf][kk][col_of(j)];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        if (t + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    if constexpr (EPI == EPI_ARGMIN) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int64_t gr = row0 + row_of(i);
            unsigned long long best = ~0ull;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int gc = col0 + col_of(j);
                if (gc < m) {
                    const float sc = fmaf(-2.0f, acc[i][j], norms[gc]);
                    const unsigned long long key =
                        ((unsigned long long)f2ord(sc) << 32) | (unsigned long long)(uint32_t)gc;
                    best = key < best ? key : best;
                }
            }
#pragma unroll
            for (int off = TX / 2; off > 0; off >>= 1) {
                const unsigned long long o = __shfl_xor(best, off);
                best = o < best ? o : best;
            }
            if (tx == 0 && gr < n && best != ~0ull) atomicMin(&amin[gr], best);
        }
    } else {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int64_t gr = row0 + row_of(i);
            if (gr >= n) continue;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int gc = col0 + col_of(j);
                if (gc >= m) continue;
                float v = acc[i][j];
                if constexpr (EPI == EPI_SCORE) v = fmaf(-2.0f, v, norms[gc]);
                C[gr * ldc + gc] = v;
            }
        }
    }
}

template <int BM, int BN, int BK, int TM, int TN, int EPI>
static hipError_t launch_gemm(const float* A, int64_t lda, const float* Bm, int64_t ldb,
                              int64_t n, int m, int d, float* C, int64_t ldc, const float* norms,
                              unsigned long long* amin, hipStream_t s) {
    constexpr int NT = (BM / TM) * (BN / TN);
    if (n <= 0 || m <= 0) return hipSuccess;
    // rows go on grid.y; launch in chunks of at most 65535 row tiles.
    const int64_t rows_per_launch = (int64_t)BM * 65535;
    for (int64_t r0 = 0; r0 < n; r0 += rows_per_launch) {
        const int64_t nr = (n - r0) < rows_per_launch ? (n - r0) : rows_per_launch;
        dim3 grid((m + BN - 1) / BN, (unsigned)((nr + BM - 1) / BM));
        hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, BK, TM, TN, EPI>), grid, dim3(NT), 0, s,
                           A + r0 * lda, lda, Bm, ldb, nr, m, d,
                           C ? C + r0 * ldc : nullptr, ldc, norms, amin ? amin + r0 : nullptr);
    }
    return hipGetLastError();
}

hipError_t gemm_nt_store(const float* A, int64_t lda, const float* Bm, int64_t ldb, int64_t n,
                         int m, int d, float* C, int64_t ldc, bool small_rows, hipStream_t s) {
    if (small_rows)
        return launch_gemm<32, 64, 16, 4, 4, EPI_STORE>(A, lda, Bm, ldb, n, m, d, C, ldc, nullptr,
                                                         nullptr, s);
    return launch_gemm<128, 128, 16, 8, 8, EPI_STORE>(A, lda, Bm, ldb, n, m, d, C, ldc, nullptr,
                                                       nullptr, s);
}

hipError_t gemm_nt_score(const float* A, int64_t lda, const float* Bm, int64_t ldb, int64_t n,
                         int m, int d, const float* norms, float* C, int64_t ldc,
                         bool small_rows, hipStream_t s) {
    if (small_rows)
        return launch_gemm<32, 64, 16, 4, 4, EPI_SCORE>(A, lda, Bm, ldb, n, m, d, C, ldc, norms,
                                                         nullptr, s);
    return launch_gemm<128, 128, 16, 8, 8, EPI_SCORE>(A, lda, Bm, ldb, n, m, d, C, ldc, norms,
                                                       nullptr, s);
}

hipError_t gemm_nt_argmin(const float* A, int64_t lda, const float* Bm, int64_t ldb, int64_t n,
                          int m, int d, const float* norms, unsigned long long* keys,
                          hipStream_t s) {
    return launch_gemm<128, 128, 16, 8, 8, EPI_ARGMIN>(A, lda, Bm, ldb, n, m, d, nullptr, 0,
                                                        norms, keys, s);
}

__global__ void fill_u64_kernel(unsigned long long* p, int64_t n, unsigned long long v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

hipError_t fill_u64(unsigned long long* p, int64_t n, unsigned long long v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(fill_u64_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

__global__ void keys_to_assign_kernel(const unsigned long long* keys, int64_t n, int32_t* a) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        a[i] = (int32_t)(uint32_t)(keys[i] & 0xffffffffull);
}

hipError_t keys_to_assign(const unsigned long long* keys, int64_t n, int32_t* assign,
                          hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(keys_to_assign_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, s, keys, n, assign);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Encode: one thread per vector, rows staged through LDS in 32-dim chunks so
// the global reads are coalesced while each thread walks its own vector in
// dimension order (the residual correction is a sequential fmaf chain).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int nearest_mid(const float* mids, int n, float v) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (v < mids[mid]) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

__global__ void __launch_bounds__(256)
encode_kernel(const float* __restrict__ y, int64_t n, int d, int M, int Ds, int K1D, int bpd,
              const float* __restrict__ c1d, int Kr, int Br, int bpv,
              const float* __restrict__ res_c1d, uint8_t* __restrict__ codes,
              uint8_t* __restrict__ res, float* __restrict__ corr, int mode) {
    __shared__ float tile[256][33];
    __shared__ float cval[256], cmid[256], rval[256], rmid[256];
    const int tid = threadIdx.x;
    const int64_t v0 = (int64_t)blockIdx.x * 256;
    const int64_t vid = v0 + tid;
    if (tid < K1D) cval[tid] = c1d[tid];
    if ((mode & 2) && tid < Kr) rval[tid] = res_c1d[tid];
    __syncthreads();
    if (tid + 1 < K1D) cmid[tid] = 0.5f * (cval[tid] + cval[tid + 1]);
    if ((mode & 2) && tid + 1 < Kr) rmid[tid] = 0.5f * (rval[tid] + rval[tid + 1]);
    __syncthreads();
    const bool live = vid < n;
    const int kmask = K1D - 1;
    float dot = 0.0f;
    uint32_t code = 0u, rbyte = 0u;
    for (int c0 = 0; c0 < d; c0 += 32) {
        const int cw = (d - c0) < 32 ? (d - c0) : 32;
        for (int i = 0; i < 32; i++) {
            const int e = tid + i * 256, row = e >> 5, col = e & 31;
            const int64_t gv = v0 + row;
            tile[row][col] = (gv < n && col < cw) ? y[gv * d + c0 + col] : 0.0f;
        }
        __syncthreads();
        if (live) {
            for (int jj = 0; jj < cw; jj++) {
                const int j = c0 + jj;
                const float val = tile[tid][jj];
                const int m = j / Ds, k = j - m * Ds;
                int dig;
                if (mode & 1) {
                    dig = (K1D == 1) ? 0 : nearest_mid(cmid, K1D, val);
                    code |= (uint32_t)dig << (k * bpd);
                    if (k == Ds - 1) {
                        codes[vid * M + m] = (uint8_t)code;
                        code = 0u;
                    }
                } else {
                    dig = (codes[vid * M + m] >> (k * bpd)) & kmask;
                }
                if (mode & 2) {
                    const float yhat = cval[dig];
                    const float r = val - yhat;
                    const int ri = (Kr == 1) ? 0 : nearest_mid(rmid, Kr, r);
                    const float rhat = rval[ri];
                    if (Br == 4) {
                        if ((j & 1) == 0) {
                            rbyte = (uint32_t)(ri & 0x0F);
                        } else {
                            rbyte |= (uint32_t)(ri & 0x0F) << 4;
                            res[vid * bpv + (j >> 1)] = (uint8_t)rbyte;
                        }
                    } else {
                        res[vid * bpv + j] = (uint8_t)ri;
                    }
                    dot = fmaf(yhat, rhat, dot);
                }
            }
        }
        __syncthreads();
    }
    if (live && (mode & 2)) {
        if (Br == 4 && (d & 1)) res[vid * bpv + (d >> 1)] = (uint8_t)rbyte;
        corr[vid] = 2.0f * dot;
    }
}

hipError_t encode(const float* y, int64_t n, int d, int M, int Ds, int K1D, int bpd,
                  const float* c1d, int Kr, int Br, int bpv, const float* res_c1d,
                  uint8_t* codes, uint8_t* res, float* corr, int mode, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (K1D > 256 || Kr > 256 || (32 % Ds) != 0) return hipErrorInvalidValue;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(encode_kernel, dim3((unsigned)blocks), dim3(256), 0, s, y, n, d, M, Ds,
                       K1D, bpd, c1d, Kr, Br, bpv, res_c1d, codes, res, corr, mode);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// List storage scatter.  Primary codes go to a code-major block per list:
// list l occupies padded candidates [padoff[l], padoff[l+1]) and stores byte m
// of candidate i at codes_t[padoff[l]*M + m*npad + i] (npad = multiple of 16),
// so one 32-bit load returns byte m of four consecutive candidates.
// ---------------------------------------------------------------------------
__global__ void scatter_kernel(const int32_t* __restrict__ order, const int32_t* __restrict__ slist,
                               int64_t n, int64_t id_base, const int32_t* __restrict__ list_off,
                               const int32_t* __restrict__ list_padoff,
                               const uint8_t* __restrict__ pc, const uint8_t* __restrict__ rc,
                               const float* __restrict__ co, int M, int bpv,
                               int32_t* __restrict__ ids_out, uint8_t* __restrict__ codes_t,
                               uint8_t* __restrict__ res_out, float* __restrict__ corr_out) {
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const int64_t id = order[s];
    const int l = slist[s];
    const int64_t i = s - list_off[l];
    const int64_t pad0 = list_padoff[l];
    const int64_t npad = list_padoff[l + 1] - pad0;
    ids_out[s] = (int32_t)(id + id_base);
    corr_out[s] = co[id];
    uint8_t* dst = codes_t + pad0 * M + i;
    const uint8_t* src = pc + id * M;
    for (int m = 0; m < M; m++) dst[(int64_t)m * npad] = src[m];
    const uint8_t* rs = rc + id * bpv;
    uint8_t* rd = res_out + s * bpv;
    for (int b2 = 0; b2 < bpv; b2++) rd[b2] = rs[b2];
}

hipError_t scatter_lists(const int32_t* order, const int32_t* slist, int64_t n, int64_t id_base,
                         const int32_t* list_off, const int32_t* list_padoff, const uint8_t* pc,
                         const uint8_t* rc, const float* co, int M, int bpv, int32_t* ids_out,
                         uint8_t* codes_t, uint8_t* res_out, float* corr_out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)blocks), dim3(256), 0, s, order, slist, n,
                       id_base, list_off, list_padoff, pc, rc, co, M, bpv, ids_out, codes_t,
                       res_out, corr_out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Probe selection: exact top-P of (score, list) per query, read straight
// from the score rows (no nlist-sized LDS array, so any nlist works).
// ---------------------------------------------------------------------------
template <int NT>
__global__ void __launch_bounds__(NT)
select_probes_kernel(const float* __restrict__ scores, int nlist, int P,
                     const int32_t* __restrict__ list_padoff, int32_t* __restrict__ probes,
                     int32_t* __restrict__ gofs) {
    extern __shared__ __align__(16) unsigned char smem[];
    int* scratch = (int*)smem;
    int* sorted = scratch + P;
    SelState* st = (SelState*)(sorted + P);
    const int b = blockIdx.x;
    const float* row = scores + (int64_t)b * nlist;
    block_topk<NT>([&](int i) { return f2ord(row[i]); }, [&](int i) { return (uint32_t)i; },
                   nlist, P, scratch, sorted, st);
    for (int r = threadIdx.x; r < P; r += NT) probes[(int64_t)b * P + r] = sorted[r];
    if (threadIdx.x == 0) {
        int acc = 0;
        int32_t* g = gofs + (int64_t)b * (P + 1);
        g[0] = 0;
        for (int r = 0; r < P; r++) {
            const int l = sorted[r];
            acc += (list_padoff[l + 1] - list_padoff[l]) / kGroup;
            g[r + 1] = acc;
        }
    }
}

hipError_t select_probes(const float* scores, int B, int nlist, int P,
                         const int32_t* list_padoff, int32_t* probes, int32_t* gofs,
                         hipStream_t s) {
    constexpr int NT = 256;
    const size_t lds = (size_t)2 * P * sizeof(int) + sizeof(SelState);
    hipLaunchKernelGGL(select_probes_kernel<NT>, dim3(B), dim3(NT), lds, s, scores, nlist, P,
                       list_padoff, probes, gofs);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// IVF ADC scan + exact top-ck.  Workgroup (s, b) scans the s-th slice of the
// padded candidate groups of query b's probed lists.
//   1. byte LUT lut[m][v] built in LDS as a prefix tree over the digits of v
//      (entries sharing low digits share the partial fmaf chain; the chain
//      order per entry is the reference's k = 0..Ds-1);
//   2. each thread takes 4 consecutive candidates of one list: per subspace m
//      one 32-bit coalesced load gives their 4 code bytes, 4 LDS gathers
//      accumulate dist in m order;
//   3. all slice distances stay in LDS; one radix select + rank sort yields
//      the slice's exact top-ck by (dist, pos).
// ---------------------------------------------------------------------------
template <int NT>
__global__ void __launch_bounds__(NT)
scan_topck_kernel(const float* __restrict__ q_rot, int d, int M, int Ds, int K1D, int bpd,
                  const float* __restrict__ c1d, const int32_t* __restrict__ probes,
                  const int32_t* __restrict__ gofs, int P, const int32_t* __restrict__ list_off,
                  const int32_t* __restrict__ list_padoff, const uint8_t* __restrict__ codes_t,
                  int ck, int S, int cap, unsigned long long* __restrict__ partial) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* lut = (float*)smem;
    uint32_t* dbuf = (uint32_t*)(lut + (size_t)M * 256);
    int32_t* sg = (int32_t*)(dbuf + cap);
    int32_t* sprobe = sg + (P + 1);
    float* sq = (float*)(sprobe + P);
    int* scratch = (int*)(sq + d);
    int* sorted = scratch + ck;
    SelState* st = (SelState*)(sorted + ck);
    __shared__ float sc1d[256];

    const int b = blockIdx.y, s = blockIdx.x, tid = threadIdx.x;
    for (int i = tid; i <= P; i += NT) sg[i] = gofs[(int64_t)b * (P + 1) + i];
    for (int i = tid; i < P; i += NT) sprobe[i] = probes[(int64_t)b * P + i];
    for (int i = tid; i < d; i += NT) sq[i] = q_rot[(int64_t)b * d + i];
    for (int i = tid; i < K1D; i += NT) sc1d[i] = c1d[i];
    if (tid == 0) st->aux = 0;
    __syncthreads();
    const int T = sg[P];
    const int g0 = (int)((int64_t)T * s / S), g1 = (int)((int64_t)T * (s + 1) / S);
    unsigned long long* outp = partial + ((int64_t)b * S + s) * ck;
    if (g1 <= g0 || (g1 - g0) * kGroup > cap) {
        for (int i = tid; i < ck; i += NT) outp[i] = ~0ull;
        return;
    }

    // 1. byte LUT, level t of the tree holds the partial sums over digits 0..t
    for (int w = tid; w < M * K1D; w += NT) {
        const int m = w >> bpd, j = w & (K1D - 1);
        const float df = sq[m * Ds] - sc1d[j];
        lut[m * 256 + j] = fmaf(df, df, 0.0f);
    }
    __syncthreads();
    for (int t = 1; t < Ds; t++) {
        const int lw = t * bpd;  // log2 of parents per subspace
        for (int w = tid; w < (M << lw); w += NT) {
            const int m = w >> lw, e = w & ((1 << lw) - 1);
            float* lm = lut + m * 256;
            const float par = lm[e];
            const float qv = sq[m * Ds + t];
            for (int j = 0; j < K1D; j++) {
                const float df = qv - sc1d[j];
                lm[e + (j << lw)] = fmaf(df, df, par);
            }
        }
        __syncthreads();
    }

    // 2. scan
    const int nq4 = (g1 - g0) * 4;
    int nvalid = 0;
    for (int qd = tid; qd < nq4; qd += NT) {
        const int gq = g0 * 4 + qd;
        const int g = gq >> 2, sub = gq & 3;
        int lo = 0, hi = P - 1;  // last p with sg[p] <= g
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (sg[mid] <= g) lo = mid;
            else hi = mid - 1;
        }
        const int l = sprobe[lo];
        const int gi = g - sg[lo];
        const int pad0 = list_padoff[l];
        const int npad = list_padoff[l + 1] - pad0;
        const int nl = list_off[l + 1] - list_off[l];
        const int c0 = gi * kGroup + sub * 4;
        const uint8_t* base = codes_t + (int64_t)pad0 * M + c0;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        int m = 0;
        for (; m + 8 <= M; m += 8) {
            uint32_t w[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                w[u] = *(const uint32_t*)(base + (int64_t)(m + u) * npad);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float* lm = lut + (m + u) * 256;
                a0 += lm[w[u] & 0xffu];
                a1 += lm[(w[u] >> 8) & 0xffu];
                a2 += lm[(w[u] >> 16) & 0xffu];
                a3 += lm[w[u] >> 24];
            }
        }
        for (; m < M; m++) {
            const uint32_t w = *(const uint32_t*)(base + (int64_t)m * npad);
            const float* lm = lut + m * 256;
            a0 += lm[w & 0xffu];
            a1 += lm[(w >> 8) & 0xffu];
            a2 += lm[(w >> 16) & 0xffu];
            a3 += lm[w >> 24];
        }
        uint32_t* db = dbuf + qd * 4;
        db[0] = (c0 + 0 < nl) ? f2ord(a0) : ~0u;
        db[1] = (c0 + 1 < nl) ? f2ord(a1) : ~0u;
        db[2] = (c0 + 2 < nl) ? f2ord(a2) : ~0u;
        db[3] = (c0 + 3 < nl) ? f2ord(a3) : ~0u;
        const int left = nl - c0;
        nvalid += left >= 4 ? 4 : (left > 0 ? left : 0);
    }
    for (int off = 32; off > 0; off >>= 1) nvalid += __shfl_xor(nvalid, off);
    if ((tid & 63) == 0) atomicAdd(&st->aux, nvalid);
    __syncthreads();
    const int nv = st->aux;
    const int ksel = nv < ck ? nv : ck;
    const int nslot = nq4 * 4;

    auto pos_of = [&](int i) -> uint32_t {
        const int gq = g0 * 4 + (i >> 2);
        const int g = gq >> 2;
        int lo = 0, hi = P - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (sg[mid] <= g) lo = mid;
            else hi = mid - 1;
        }
        const int l = sprobe[lo];
        const int cand = (g - sg[lo]) * kGroup + (gq & 3) * 4 + (i & 3);
        return (uint32_t)(list_off[l] + cand);
    };

    // 3. exact top-ck of the slice
    if (ksel > 0) {
        block_topk<NT>([&](int i) { return dbuf[i]; }, pos_of, nslot, ksel, scratch, sorted, st);
    }
    for (int r = tid; r < ck; r += NT) {
        if (r < ksel) {
            const int i = sorted[r];
            outp[r] = ((unsigned long long)dbuf[i] << 32) | (unsigned long long)pos_of(i);
        } else {
            outp[r] = ~0ull;
        }
    }
}

bool scan_plan(int M, int d, int P, int ck, int max_groups_per_query, int B, int target_wg,
               ScanShape* out) {
    const int fixed = M * 256 * 4 + (P + 1) * 4 + P * 4 + d * 4 + 2 * ck * 4 +
                      (int)sizeof(SelState) + 64;
    const int avail = kLdsBytes - 1024 /* static sc1d */ - fixed;
    if (avail < 256 * 4) return false;
    int cap = avail / 4;
    if (cap > 8192) cap = 8192;
    cap = (cap / 64) * 64;
    const int capg = cap / kGroup;
    int S_cap = (max_groups_per_query + capg - 1) / capg;
    int S_par = (target_wg + B - 1) / B;
    int S = S_cap > S_par ? S_cap : S_par;
    if (S < 1) S = 1;
    out->S = S;
    out->cap = cap;
    out->lds = fixed + cap * 4;
    return true;
}

hipError_t scan_topck(const float* q_rot, int B, int d, int M, int Ds, int K1D, int bpd,
                      const float* c1d, const int32_t* probes, const int32_t* gofs, int P,
                      const int32_t* list_off, const int32_t* list_padoff,
                      const uint8_t* codes_t, int ck, const ScanShape& sh,
                      unsigned long long* partial, hipStream_t s) {
    constexpr int NT = 512;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)scan_topck_kernel<NT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           kLdsBytes - 1024);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    dim3 grid(sh.S, B);
    hipLaunchKernelGGL(scan_topck_kernel<NT>, grid, dim3(NT), sh.lds, s, q_rot, d, M, Ds, K1D,
                       bpd, c1d, probes, gofs, P, list_off, list_padoff, codes_t, ck, sh.S,
                       sh.cap, partial);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Merge + residual refine + final top-k, one workgroup per query.
// The residual distance of a candidate is summed by 16 lanes over 16
// contiguous dimension ranges, then added across the lanes in a fixed tree.
// ---------------------------------------------------------------------------
template <int NT>
__global__ void __launch_bounds__(NT)
refine_topk_kernel(const unsigned long long* __restrict__ partial, int S, int ck, int k,
                   const float* __restrict__ q_rot, int d, const float* __restrict__ res_c1d,
                   int Kr, int Br, int bpv, const uint8_t* __restrict__ list_res,
                   const float* __restrict__ list_corr, const int32_t* __restrict__ list_ids,
                   float* __restrict__ out_d, int32_t* __restrict__ out_i,
                   unsigned long long* __restrict__ topck_dbg) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int n = S * ck;
    unsigned long long* keys = (unsigned long long*)smem;
    float* sq = (float*)(keys + n);
    int* scratch = (int*)(sq + d);
    int* sorted = scratch + ck;
    float* cprim = (float*)(sorted + ck);
    int* cpos = (int*)(cprim + ck);
    float* ccomp = (float*)(cpos + ck);
    int* cid = (int*)(ccomp + ck);
    int* fscr = cid + ck;
    int* fsorted = fscr + ck;
    SelState* st = (SelState*)(fsorted + ck);
    __shared__ float rc[256];

    const int b = blockIdx.x, tid = threadIdx.x;
    const unsigned long long* pk = partial + (int64_t)b * n;
    int nv = 0;
    for (int i = tid; i < n; i += NT) {
        const unsigned long long kk = pk[i];
        keys[i] = kk;
        nv += (kk != ~0ull) ? 1 : 0;
    }
    for (int i = tid; i < d; i += NT) sq[i] = q_rot[(int64_t)b * d + i];
    for (int i = tid; i < Kr; i += NT) rc[i] = res_c1d[i];
    if (tid == 0) st->aux = 0;
    __syncthreads();
    for (int off = 32; off > 0; off >>= 1) nv += __shfl_xor(nv, off);
    if ((tid & 63) == 0) atomicAdd(&st->aux, nv);
    __syncthreads();
    const int nvalid = st->aux;
    const int ksel = nvalid < ck ? nvalid : ck;
    if (ksel > 0) {
        block_topk<NT>([&](int i) { return (uint32_t)(keys[i] >> 32); },
                       [&](int i) { return (uint32_t)(keys[i] & 0xffffffffull); }, n, ksel,
                       scratch, sorted, st);
    }
    for (int r = tid; r < ck; r += NT) {
        if (r < ksel) {
            const unsigned long long kk = keys[sorted[r]];
            cprim[r] = ord2f((uint32_t)(kk >> 32));
            cpos[r] = (int)(uint32_t)(kk & 0xffffffffull);
            if (topck_dbg) topck_dbg[(int64_t)b * ck + r] = kk;
        } else if (topck_dbg) {
            topck_dbg[(int64_t)b * ck + r] = ~0ull;
        }
    }
    __syncthreads();

    // residual refine
    const int grp = tid >> 4, l16 = tid & 15;
    constexpr int NG = NT / 16;
    int chk = (d + 15) / 16;
    chk += chk & 1;
    for (int base = 0; base < ksel; base += NG) {
        const int c = base + grp;
        const bool valid = c < ksel;
        float sres = 0.0f;
        int pos = 0;
        if (valid) {
            pos = cpos[c];
            const uint8_t* rcode = list_res + (int64_t)pos * bpv;
            const int j0 = l16 * chk;
            const int j1 = (j0 + chk) < d ? (j0 + chk) : d;
            if (Br == 4) {
                for (int j = j0; j < j1; j += 2) {
                    const uint32_t byte = rcode[j >> 1];
                    const float df0 = sq[j] - rc[byte & 0x0Fu];
                    sres = sres + df0 * df0;
                    if (j + 1 < j1) {
                        const float df1 = sq[j + 1] - rc[byte >> 4];
                        sres = sres + df1 * df1;
                    }
                }
            } else {
                for (int j = j0; j < j1; j++) {
                    const float df = sq[j] - rc[rcode[j]];
                    sres = sres + df * df;
                }
            }
        }
        sres = sres + __shfl_xor(sres, 8);
        sres = sres + __shfl_xor(sres, 4);
        sres = sres + __shfl_xor(sres, 2);
        sres = sres + __shfl_xor(sres, 1);
        if (valid && l16 == 0) {
            ccomp[c] = (cprim[c] + sres) + list_corr[pos];
            cid[c] = list_ids[pos];
        }
    }
    __syncthreads();

    // final top-k by (dist, id)
    const int kf = ksel < k ? ksel : k;
    if (kf > 0) {
        block_topk<NT>([&](int i) { return f2ord(ccomp[i]); }, [&](int i) { return (uint32_t)cid[i]; },
                       ksel, kf, fscr, fsorted, st);
    }
    for (int r = tid; r < k; r += NT) {
        if (r < kf) {
            const int i = fsorted[r];
            out_d[(int64_t)b * k + r] = ccomp[i];
            out_i[(int64_t)b * k + r] = cid[i];
        } else {
            out_d[(int64_t)b * k + r] = __builtin_huge_valf();
            out_i[(int64_t)b * k + r] = -1;
        }
    }
}

hipError_t refine_topk(const unsigned long long* partial, int B, int S, int ck, int k,
                       const float* q_rot, int d, const float* res_c1d, int Kr, int Br, int bpv,
                       const uint8_t* list_res, const float* list_corr, const int32_t* list_ids,
                       float* out_d, int32_t* out_i, unsigned long long* topck_dbg,
                       hipStream_t s) {
    constexpr int NT = 256;
    if (k > ck) return hipErrorInvalidValue;
    const size_t lds = (size_t)S * ck * 8 + (size_t)d * 4 + (size_t)ck * 4 * 8 +
                       sizeof(SelState) + 64;
    if (lds > (size_t)kLdsBytes - 1024) return hipErrorInvalidValue;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)refine_topk_kernel<NT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           kLdsBytes - 1024);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(refine_topk_kernel<NT>, dim3(B), dim3(NT), lds, s, partial, S, ck, k, q_rot,
                       d, res_c1d, Kr, Br, bpv, list_res, list_corr, list_ids, out_d, out_i,
                       topck_dbg);
    return hipGetLastError();
}

}  // namespace jhq
