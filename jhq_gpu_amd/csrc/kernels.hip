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
#include <algorithm>
#include <cstdint>
#include <type_traits>

// Scan workgroup size and code-load pipeline depth (subspaces in flight).
#ifndef JHQ_SCAN_NT
#define JHQ_SCAN_NT 1024
#endif
#ifndef JHQ_SCAN_SU
#define JHQ_SCAN_SU 8
#endif

namespace jhq {

// Phase instrumentation: built with -DJHQ_PHASE_TIMING, thread 0 of each
// workgroup accumulates wall-clock ticks (100 MHz) per phase of the scan,
// probe-selection and refine kernels; jhq_debug_phase_ticks() reads them.
#ifdef JHQ_PHASE_TIMING
constexpr int kPhaseBlocks = 4096, kPhases = 16;
__device__ unsigned long long g_phase[4][kPhaseBlocks][kPhases];
#define JHQ_PHASE_DECL unsigned long long ph_t = wall_clock64(), ph_acc[kPhases] = {0};
#define JHQ_PHASE(i)                                              \
    do {                                                          \
        const unsigned long long ph_n = wall_clock64();           \
        ph_acc[i] += ph_n - ph_t;                                 \
        ph_t = ph_n;                                              \
    } while (0)
#define JHQ_PHASE_FLUSH(kid)                                                         \
    do {                                                                             \
        if (threadIdx.x == 0 && blockIdx.x < kPhaseBlocks)                           \
            for (int ph_i = 0; ph_i < kPhases; ph_i++)                               \
                g_phase[kid][blockIdx.x][ph_i] = ph_acc[ph_i];                       \
    } while (0)
#else
#define JHQ_PHASE_DECL
#define JHQ_PHASE(i) \
    do {             \
    } while (0)
#define JHQ_PHASE_FLUSH(kid) \
    do {                     \
    } while (0)
#endif

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
    uint32_t vmin, vmax;
    uint32_t lo, len_lo, len_hi;
    uint32_t krem;
    uint32_t eq;
    int cnt;
    int aux;
};

struct SelResult {
    uint32_t lo;        // window start
    uint64_t len;       // window length (values lo .. lo+len-1)
    uint32_t krem;      // elements still needed from the window
    bool done;          // true: every element in the window is selected
};

// Adds 1 to hist[bin] for every lane with bin >= 0; the bin shared by the most
// lanes of typical (clustered) data is peeled off with one ballot so that it
// costs one atomic instead of up to 64 serialised ones.
__device__ __forceinline__ void wave_hist_add(uint32_t* hist, int bin) {
    const int lane = threadIdx.x & 63;
    unsigned long long act = __ballot(bin >= 0);
#pragma unroll
    for (int r = 0; r < 2; r++) {
        if (!act) return;
        const int leader = __ffsll((long long)act) - 1;
        const int lb = __shfl(bin, leader);
        const unsigned long long same = __ballot(bin == lb) & act;
        if (lane == leader) atomicAdd(&hist[lb], (uint32_t)__popcll(same));
        act &= ~same;
    }
    if ((act >> lane) & 1ull) atomicAdd(&hist[bin], 1u);
}

// Exact k-th smallest of n u32 values (1 <= k <= number of values != ~0u;
// ~0u marks an empty slot that is never selected).  The first window is the
// actual [min, max] of the values; each pass splits the window into 256
// buckets of width 2^sh counted from its start (a shift, no division),
// histograms the elements inside it and keeps the bucket holding the k-th
// value, so the window narrows 256x per pass whatever the bit patterns.  Returns the rule: v selected iff v < lo, or
// lo <= v < lo+len and (done, or v wins the tie-break among equal values).
template <int NT, class GetV>
__device__ __forceinline__ SelResult sel_threshold(GetV getv, int n, uint32_t k, SelState* st) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid == 0) { st->vmin = ~0u; st->vmax = 0u; }
    __syncthreads();
    uint32_t mn = ~0u, mx = 0u;
    for (int i = tid; i < n; i += NT) {
        const uint32_t v = getv(i);
        if (v != ~0u) { mn = v < mn ? v : mn; mx = v > mx ? v : mx; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t a = __shfl_xor(mn, off), c = __shfl_xor(mx, off);
        mn = a < mn ? a : mn;
        mx = c > mx ? c : mx;
    }
    if (lane == 0) { atomicMin(&st->vmin, mn); atomicMax(&st->vmax, mx); }
    __syncthreads();
    SelResult r;
    r.lo = st->vmin;
    r.len = (st->vmin <= st->vmax) ? (uint64_t)st->vmax - st->vmin + 1ull : 0ull;
    r.krem = k;
    r.done = (r.len == 0ull);
    uint32_t eq = 0;
    while (!r.done && r.len > 1) {
        // 256 buckets of width 2^sh cover the window from its start
        const int sh = (r.len <= 256ull) ? 0 : (64 - __clzll((long long)(r.len - 1ull)) - 8);
        for (int i = tid; i < 256; i += NT) st->hist[i] = 0u;
        __syncthreads();
        const int iters = (n + NT - 1) / NT;
        for (int it = 0; it < iters; it++) {
            const int i = it * NT + tid;
            int bin = -1;
            if (i < n) {
                const uint32_t v = getv(i);
                const uint64_t x = (uint64_t)v - r.lo;
                if (v >= r.lo && x < r.len) bin = (int)(x >> sh);
            }
            wave_hist_add(st->hist, bin);
        }
        __syncthreads();
        if (tid < 64) {
            const uint32_t c0 = st->hist[tid * 4 + 0], c1 = st->hist[tid * 4 + 1];
            const uint32_t c2 = st->hist[tid * 4 + 2], c3 = st->hist[tid * 4 + 3];
            const uint32_t sm = c0 + c1 + c2 + c3;
            uint32_t inc = sm;
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t t = __shfl_up(inc, off);
                if (lane >= off) inc += t;
            }
            uint32_t base = inc - sm;
            const uint32_t cb[4] = {c0, c1, c2, c3};
            for (int j = 0; j < 4; j++) {
                if (base < r.krem && r.krem <= base + cb[j]) {
                    const uint64_t s0 = (uint64_t)(tid * 4 + j) << sh;
                    const uint64_t rest = r.len - s0;
                    const uint64_t nl = rest < (1ull << sh) ? rest : (1ull << sh);
                    st->lo = r.lo + (uint32_t)s0;
                    st->len_lo = (uint32_t)nl;
                    st->len_hi = (uint32_t)(nl >> 32);
                    st->krem = r.krem - base;
                    st->eq = cb[j];
                }
                base += cb[j];
            }
        }
        __syncthreads();
        r.lo = st->lo;
        r.len = ((uint64_t)st->len_hi << 32) | st->len_lo;
        r.krem = st->krem;
        eq = st->eq;
        r.done = (eq == r.krem);
        __syncthreads();
    }
    if (!r.done && r.len == 1) {
        // window is a single value: done iff exactly krem elements hold it
        if (tid == 0) st->eq = 0u;
        __syncthreads();
        uint32_t c = 0;
        for (int i = tid; i < n; i += NT) c += (getv(i) == r.lo) ? 1u : 0u;
        for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off);
        if (lane == 0 && c) atomicAdd(&st->eq, c);
        __syncthreads();
        r.done = (st->eq == r.krem);
        __syncthreads();
    }
    return r;
}

// Ballot compaction of pred(i) over i < n into out[], counter st->cnt
// (zeroed here).  Returns the count.
template <int NT, class Pred>
__device__ __forceinline__ int sel_compact(Pred pred, int n, int* out, int cap, SelState* st) {
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

// Exact top-k of n elements by (getv, gett) ascending (gett distinct among
// equal getv).  Writes the k selected elements' keys (getv << 32 | gett) in
// ascending order to keys[0..k) and returns k.  idx must hold k ints and
// tmp/keys k u64 each (8-byte aligned LDS).  Requires 1 <= k <= the number of
// elements whose value is not ~0u.  gett is evaluated only for elements tied
// at the threshold value and for the k selected elements.
template <int NT, class GetV, class GetT>
__device__ __forceinline__ int block_topk(GetV getv, GetT gett, int n, int k, int* idx, unsigned long long* tmp,
                          unsigned long long* keys, SelState* st,
                          unsigned long long* sub = nullptr) {
#ifdef JHQ_PHASE_TIMING
    unsigned long long t0 = wall_clock64();
#endif
    const SelResult r = sel_threshold<NT>(getv, n, (uint32_t)k, st);
    SelResult t;
    t.lo = 0u; t.len = 0ull; t.done = true; t.krem = 0u;
    if (!r.done) {
        // ties at the single threshold value: keep the r.krem smallest tags
        const uint32_t pv = r.lo;
        t = sel_threshold<NT>(
            [&](int i) {
                const uint32_t v = getv(i);
                if (v != pv) return ~0u;
                return gett(i);
            },
            n, r.krem, st);
    }
    const bool rdone = r.done;
    const uint32_t rlo = r.lo, tlo = t.lo;
    const uint64_t rlen = r.len, tlen = t.len;
    int cnt = sel_compact<NT>(
        [&](int i) {
            const uint32_t v = getv(i);
            if (v == ~0u) return false;
            if (v < rlo) return true;
            if ((uint64_t)(v - rlo) >= rlen) return false;
            if (rdone) return true;
            const uint32_t tg = gett(i);
            return tg < tlo || (uint64_t)(tg - tlo) < tlen;
        },
        n, idx, k, st);
    cnt = cnt < k ? cnt : k;
#ifdef JHQ_PHASE_TIMING
    unsigned long long t2 = wall_clock64();
    if (sub) { sub[0] += t2 - t0; t0 = t2; }
#endif
    for (int a = threadIdx.x; a < cnt; a += NT) {
        const int i = idx[a];
        tmp[a] = ((unsigned long long)getv(i) << 32) | (unsigned long long)gett(i);
    }
    for (int a = threadIdx.x; a < k; a += NT) keys[a] = ~0ull;
    __syncthreads();
    // rank sort of distinct keys; every thread reads tmp[b] in the same order
    // (LDS broadcast)
    for (int a = threadIdx.x; a < cnt; a += NT) {
        const unsigned long long ka = tmp[a];
        int rk = 0;
        for (int b2 = 0; b2 < cnt; b2++) rk += (tmp[b2] < ka) ? 1 : 0;
        if (rk < cnt) keys[rk] = ka;
    }
    __syncthreads();
#ifdef JHQ_PHASE_TIMING
    if (sub) sub[1] += wall_clock64() - t0;
#endif
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

// ---------------------------------------------------------------------------
// Skinny fixed-order GEMM for a query batch: C[b][j] = sum_k A[b][k] Bm[j][k]
// with nb <= a few hundred rows and many columns.  One output column per
// lane, TQ batch rows per wave, 4 waves per workgroup sharing one 64-column
// B tile staged k-major in LDS; A values are LDS broadcasts.  The k loop is
// ascending, so every output is the same fmaf chain as the SIMT tile kernel.
// ---------------------------------------------------------------------------
#ifndef JHQ_SKINNY_BK
#define JHQ_SKINNY_BK 128
#endif
template <int TQ, int EPI>
__global__ void __launch_bounds__(256)
gemm_skinny_kernel(const float* __restrict__ A, int64_t lda, const float* __restrict__ Bm,
                   int64_t ldb, int nb, int m, int d, float* __restrict__ C, int64_t ldc,
                   const float* __restrict__ norms) {
    constexpr int BK = JHQ_SKINNY_BK, QW = 4 * TQ;
    constexpr int BL = 64 * BK / 256;             // B floats per thread per tile
    constexpr int QL = (QW * BK + 255) / 256;     // A floats per thread per tile
    __shared__ float Bs[2][BK][65];
    __shared__ __align__(16) float Qs[2][BK][QW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j0 = blockIdx.x * 64, b0 = blockIdx.y * QW;
    float rb[BL], rq[QL];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < BL; i++) {
            const int e = tid + i * 256, r = e / BK, kk = e % BK;
            const int gj = j0 + r, gk = k0 + kk;
            rb[i] = (gj < m && gk < d) ? Bm[(int64_t)gj * ldb + gk] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < QL; i++) {
            const int e = tid + i * 256, r = e / BK, kk = e % BK;
            const int gb = b0 + r, gk = k0 + kk;
            rq[i] = (e < QW * BK && gb < nb && gk < d) ? A[(int64_t)gb * lda + gk] : 0.0f;
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < BL; i++) {
            const int e = tid + i * 256;
            Bs[buf][e % BK][e / BK] = rb[i];
        }
#pragma unroll
        for (int i = 0; i < QL; i++) {
            const int e = tid + i * 256;
            if (e < QW * BK) Qs[buf][e % BK][e / BK] = rq[i];
        }
    };
    float acc[TQ];
#pragma unroll
    for (int t = 0; t < TQ; t++) acc[t] = 0.0f;
    const int nk = (d + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int t = 0; t < nk; t++) {
        const int buf = t & 1;
        if (t + 1 < nk) gload((t + 1) * BK);
#pragma unroll 16
        for (int kk = 0; kk < BK; kk++) {
            const float bv = Bs[buf][kk][lane];
#pragma unroll
            for (int u = 0; u < TQ; u++) acc[u] = fmaf(Qs[buf][kk][w * TQ + u], bv, acc[u]);
        }
        if (t + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }
    const int j = j0 + lane;
    if (j < m) {
#pragma unroll
        for (int u = 0; u < TQ; u++) {
            const int b = b0 + w * TQ + u;
            if (b < nb) {
                float v = acc[u];
                if constexpr (EPI == EPI_SCORE) v = fmaf(-2.0f, v, norms[j]);
                C[(int64_t)b * ldc + j] = v;
            }
        }
    }
}

template <int EPI>
static hipError_t launch_skinny(const float* A, int64_t lda, const float* Bm, int64_t ldb, int nb,
                                int m, int d, float* C, int64_t ldc, const float* norms,
                                hipStream_t s) {
    // about 2048 waves: TQ = rows per wave, a power of two in [1, 8]
    const int64_t colblocks = (m + 63) / 64;
    int TQ = 1;
    while (TQ < 8 && colblocks * ((nb + TQ - 1) / TQ) > 2048) TQ *= 2;
    dim3 grid((unsigned)colblocks, (unsigned)((nb + 4 * TQ - 1) / (4 * TQ)));
    switch (TQ) {
        case 1: hipLaunchKernelGGL((gemm_skinny_kernel<1, EPI>), grid, dim3(256), 0, s, A, lda, Bm, ldb, nb, m, d, C, ldc, norms); break;
        case 2: hipLaunchKernelGGL((gemm_skinny_kernel<2, EPI>), grid, dim3(256), 0, s, A, lda, Bm, ldb, nb, m, d, C, ldc, norms); break;
        case 4: hipLaunchKernelGGL((gemm_skinny_kernel<4, EPI>), grid, dim3(256), 0, s, A, lda, Bm, ldb, nb, m, d, C, ldc, norms); break;
        default: hipLaunchKernelGGL((gemm_skinny_kernel<8, EPI>), grid, dim3(256), 0, s, A, lda, Bm, ldb, nb, m, d, C, ldc, norms); break;
    }
    return hipGetLastError();
}

hipError_t gemm_nt_store(const float* A, int64_t lda, const float* Bm, int64_t ldb, int64_t n,
                         int m, int d, float* C, int64_t ldc, bool small_rows, hipStream_t s) {
    if (small_rows && n <= 4096)
        return launch_skinny<EPI_STORE>(A, lda, Bm, ldb, (int)n, m, d, C, ldc, nullptr, s);
    return launch_gemm<128, 128, 16, 8, 8, EPI_STORE>(A, lda, Bm, ldb, n, m, d, C, ldc, nullptr,
                                                       nullptr, s);
}

hipError_t gemm_nt_score(const float* A, int64_t lda, const float* Bm, int64_t ldb, int64_t n,
                         int m, int d, const float* norms, float* C, int64_t ldc,
                         bool small_rows, hipStream_t s) {
    if (small_rows && n <= 4096)
        return launch_skinny<EPI_SCORE>(A, lda, Bm, ldb, (int)n, m, d, C, ldc, norms, s);
    return launch_gemm<128, 128, 16, 8, 8, EPI_SCORE>(A, lda, Bm, ldb, n, m, d, C, ldc, norms,
                                                       nullptr, s);
}

hipError_t gemm_nt_argmin(const float* A, int64_t lda, const float* Bm, int64_t ldb, int64_t n,
                          int m, int d, const float* norms, unsigned long long* keys,
                          hipStream_t s) {
    return launch_gemm<128, 128, 16, 8, 8, EPI_ARGMIN>(A, lda, Bm, ldb, n, m, d, nullptr, 0,
                                                        norms, keys, s);
}

// EPI_ARGMIN over listed rows: keys[i] = the smallest
// (f2ord(fmaf(-2, dot, norms[c])) << 32 | c) over the lists c, for the row
// A[rowidx[i]], i < min(n_max, *ndev); each dot the fmaf chain in k order,
// as in gemm_nt_kernel.  The listed rows are few (the near ties of an
// assignment): a workgroup takes 128 lists, one per thread, and steps over
// groups of 8 rows staged in LDS; each list value read feeds the group's 8
// chains, and each row's minimum goes out as one atomic per wave.
constexpr int kArgRows = 8, kArgCols = 128, kArgK = 512, kArgKB = 64;

__global__ void __launch_bounds__(kArgCols)
argmin_rows_kernel(const float* __restrict__ A, int64_t lda, const int32_t* __restrict__ rowidx,
                   const int32_t* __restrict__ ndev, int64_t n_max, const float* __restrict__ Bm,
                   int64_t ldb, int m, int d, const float* __restrict__ norms,
                   unsigned long long* __restrict__ keys) {
    __shared__ __align__(16) float ys[kArgRows][kArgK];
    const int tid = threadIdx.x;
    const int col = blockIdx.x * kArgCols + tid;
    int64_t cnt = *ndev;
    if (cnt > n_max) cnt = n_max;
    const float* brow = Bm + (int64_t)(col < m ? col : 0) * ldb;
    const bool vec = (ldb % 4) == 0 && ((uintptr_t)Bm & 15) == 0;
    for (int64_t g0 = (int64_t)blockIdx.y * kArgRows; g0 < cnt;
         g0 += (int64_t)gridDim.y * kArgRows) {
        const int nr = (cnt - g0) < kArgRows ? (int)(cnt - g0) : kArgRows;
        int64_t rbase[kArgRows];
#pragma unroll
        for (int i = 0; i < kArgRows; i++) rbase[i] = (int64_t)rowidx[g0 + (i < nr ? i : nr - 1)] * lda;
        float acc[kArgRows];
#pragma unroll
        for (int i = 0; i < kArgRows; i++) acc[i] = 0.0f;
        for (int k0 = 0; k0 < d; k0 += kArgK) {
            const int kw = (d - k0) < kArgK ? (d - k0) : kArgK;
            // all of the chunk's loads in flight at once (rows past nr and
            // k past kw read a valid element and store zero)
            constexpr int kPer = kArgRows * kArgK / kArgCols;
            static_assert(kArgK % kArgCols == 0, "a thread's elements stay in one row per k block");
            float v[kPer];
#pragma unroll
            for (int t = 0; t < kPer; t++) {
                const int e = tid + t * kArgCols, i = e / kArgK, kk = e % kArgK;
                const int kc = kk < kw ? kk : kw - 1;
                v[t] = A[rbase[i] + k0 + kc];
            }
            __syncthreads();  // the previous chunk's reads are done
#pragma unroll
            for (int t = 0; t < kPer; t++) {
                const int e = tid + t * kArgCols, i = e / kArgK, kk = e % kArgK;
                ys[i][kk] = (i < nr && kk < kw) ? v[t] : 0.0f;
            }
            __syncthreads();
            if (col < m) {
                int kk = 0;
                if (vec && kw >= kArgKB) {
                    // the list's values kArgKB at a time, the next kArgKB
                    // loading while these feed the chains
                    constexpr int J = kArgKB / 4;
                    const int kend = kw / kArgKB * kArgKB;
                    float4 cur[J], nxt[J];
#pragma unroll
                    for (int j = 0; j < J; j++) cur[j] = *(const float4*)(brow + k0 + 4 * j);
                    for (; kk < kend; kk += kArgKB) {
                        if (kk + kArgKB < kend) {
#pragma unroll
                            for (int j = 0; j < J; j++)
                                nxt[j] = *(const float4*)(brow + k0 + kk + kArgKB + 4 * j);
                        }
#pragma unroll
                        for (int j = 0; j < J; j++) {
                            const float4 b = cur[j];
#pragma unroll
                            for (int i = 0; i < kArgRows; i++) {
                                const float4 a = *(const float4*)&ys[i][kk + 4 * j];
                                acc[i] = fmaf(a.x, b.x, acc[i]);
                                acc[i] = fmaf(a.y, b.y, acc[i]);
                                acc[i] = fmaf(a.z, b.z, acc[i]);
                                acc[i] = fmaf(a.w, b.w, acc[i]);
                            }
                        }
#pragma unroll
                        for (int j = 0; j < J; j++) cur[j] = nxt[j];
                    }
                }
                for (; kk < kw; kk++) {
                    const float b = brow[k0 + kk];
#pragma unroll
                    for (int i = 0; i < kArgRows; i++) acc[i] = fmaf(ys[i][kk], b, acc[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kArgRows; i++) {
            if (i >= nr) break;
            unsigned long long key = ~0ull;
            if (col < m) {
                const float sc = fmaf(-2.0f, acc[i], norms[col]);
                key = ((unsigned long long)f2ord(sc) << 32) | (unsigned long long)(uint32_t)col;
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const unsigned long long o = __shfl_xor(key, off);
                key = o < key ? o : key;
            }
            if ((tid & 63) == 0 && key != ~0ull) atomicMin(&keys[g0 + i], key);
        }
    }
}

hipError_t gemm_nt_argmin_rows(const float* A, int64_t lda, const int32_t* rowidx,
                               const int32_t* ndev, int64_t n_max, const float* Bm, int64_t ldb,
                               int m, int d, const float* norms, unsigned long long* keys,
                               hipStream_t s) {
    if (n_max <= 0 || m <= 0) return hipSuccess;
    // up to 32 workgroup rows step over the groups of rows below the count
    // read on the device
    const int64_t groups = (n_max + kArgRows - 1) / kArgRows;
    dim3 grid((m + kArgCols - 1) / kArgCols, (unsigned)(groups < 32 ? groups : 32));
    hipLaunchKernelGGL(argmin_rows_kernel, grid, dim3(kArgCols), 0, s, A, lda, rowidx, ndev, n_max,
                       Bm, ldb, m, d, norms, keys);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Query-side GEMMs on fp32 MFMA (v_mfma_f32_16x16x4f32):
//   C[b][n] = sum_k A[b][k] * Bm[n][k]      (EPI_STORE: query rotation)
//   C[b][n] = norms[n] - 2 * that           (EPI_SCORE: centroid scores)
// Operand layout of the instruction: lane l supplies A[l%16][k_l] and
// Bm[l%16][k_l] where lane group g = l/16 owns the k values; lane l receives
// D[4*(l/16)+j][l%16], j < 4.  Each k index is assigned to one (lane group,
// step) pair: group g walks its own contiguous quarter of the wave's K slice,
// so each lane streams two contiguous runs (one A row, one Bm row) with
// 128-bit loads.  One wave per 16x16 output tile and K slice; the S waves of a
// workgroup split K and their partial tiles are added in LDS in wave order.
// ---------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));

template <int S, int EPI, bool VEC>
__global__ void __launch_bounds__(64 * S)
mfma_nt_kernel(const float* __restrict__ A, int64_t lda, const float* __restrict__ Bm,
               int64_t ldb, int nb, int N, int K, float* __restrict__ C, int64_t ldc,
               const float* __restrict__ norms) {
    __shared__ v4f red[S > 1 ? (S - 1) * 64 : 1];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int b0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
    const int Ks = (K + S - 1) / S;
    const int kbeg = wv * Ks, kend = min(K, kbeg + Ks);
    const int Kq = (Ks + 3) / 4;  // steps of this wave (every lane issues all of them)
    const int ka = kbeg + g * Kq;
    const int kz = min(kend, ka + Kq);
    const bool arow = (b0 + r) < nb, brow = (n0 + r) < N;
    const float* ap = A + (int64_t)(arow ? b0 + r : 0) * lda;
    const float* bp = Bm + (int64_t)(brow ? n0 + r : 0) * ldb;
    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    if (VEC) {
        // K % (64*S) == 0, rows 16-byte aligned: every lane's run is whole
        // float4s, fetched 4 deep (16 k-steps) with the next 4 in flight
        // rows past the edge read the clamped row 0; they only feed output
        // rows / columns that are never stored, so the loads stay unconditional
        constexpr int D = 4;
        const float4* a4 = (const float4*)(ap + ka);
        const float4* b4 = (const float4*)(bp + ka);
        const int n4 = Kq / 4;
        float4 an[D], bn[D];
#pragma unroll
        for (int u = 0; u < D; u++) {
            an[u] = a4[u];
            bn[u] = b4[u];
        }
        for (int i = 0; i < n4; i += D) {
            float4 ac[D], bc[D];
#pragma unroll
            for (int u = 0; u < D; u++) {
                ac[u] = an[u];
                bc[u] = bn[u];
            }
            if (i + D < n4) {
#pragma unroll
                for (int u = 0; u < D; u++) {
                    an[u] = a4[i + D + u];
                    bn[u] = b4[i + D + u];
                }
            }
#pragma unroll
            for (int u = 0; u < D; u++) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ac[u].x, bc[u].x, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ac[u].y, bc[u].y, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ac[u].z, bc[u].z, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ac[u].w, bc[u].w, acc1, 0, 0, 0);
            }
        }
    } else {
        for (int st = 0; st < Kq; st++) {
            const int k = ka + st;
            const bool ok = k < kz;
            const float av = (arow && ok) ? ap[k] : 0.0f;
            const float bv = (brow && ok) ? bp[k] : 0.0f;
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc0, 0, 0, 0);
        }
    }
    v4f acc = acc0 + acc1;
    if (S > 1) {
        if (wv > 0) red[(wv - 1) * 64 + lane] = acc;
        __syncthreads();
        if (wv > 0) return;
#pragma unroll
        for (int w2 = 0; w2 < S - 1; w2++) acc += red[w2 * 64 + lane];
    }
    const int col = n0 + r;
    if (col >= N) return;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int row = b0 + 4 * g + j;
        if (row < nb) {
            float v = acc[j];
            if (EPI == EPI_SCORE) v = fmaf(-2.0f, v, norms[col]);
            C[(int64_t)row * ldc + col] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Query-side product against Bm = [Pi ; centroids Pi] (the centroids taken
// back to the unrotated space, so the scores need not wait for the rotation):
// C[row][col] = sum_k A[row][k] * Bm[col][k]; columns below nrot are the
// rotated query (stored to C1), the rest centroid scores norms[c] - 2 * dot
// (stored to C2 at column c - nrot).  Requires K % 64 == 0, lda and ldb
// multiples of 4, 16-byte aligned A and Bm.
// ---------------------------------------------------------------------------
bool mfma_q_ok(int K, int64_t lda, int64_t ldb) {
    return K % 64 == 0 && lda % 4 == 0 && ldb % 4 == 0;
}

// The launch is sized to the chip (mfma_qb_plan: about one workgroup per CU
// at D = 1024, nlist 4096, batch 64: C = 5, nsplit = 4, 256 workgroups).
// Workgroup (cg, sp, rb) covers rows 64*rb .. +63, column tiles cg*C .. +C-1
// (16 columns each) and its share sp of K.  Its 4 waves split that share
// again (K in steps of 16, 4 * nsplit * NI = K / 16: wave w of split sp takes
// steps (4*sp + w)*NI .. +NI-1); each wave puts all of its A and Bm float4
// loads in flight up front (NI <= 4 steps) and runs 4*C*4 MFMAs per step
// (4 row tiles x C column tiles, every tile an independent accumulator).
// Lane (r, g) supplies row / column r of a tile and k = 16*step + 4g .. +3,
// one k per MFMA.  The 4 wave sums meet in LDS and are added in wave order.
// With nsplit > 1 the workgroup stores its sums to part[sp] and
// mfma_qb_reduce_kernel (or the probe selection, select_probes_qb) adds the
// nsplit partial rows in split order, so the sum order is fixed.  (A last-arriving-workgroup reduction inside this
// kernel needs device-scope fences, whose L2 write-backs cost more than the
// second launch: 49 against 19 us per batch of 64 at D = 1024, nlist 4096;
// the 8-wave kernel this replaces, 64 rows x 32 columns per wave with K split
// over the waves, took 24 us on 160 workgroups.)
// ---------------------------------------------------------------------------
// Component q of the vector held by the quad lane that quad_perm CTRL
// (k, k, k, k) names: one step of a 4 x 4 transpose across a quad of lanes.
template <int CTRL>
__device__ __forceinline__ float quad_pick(const v4f& x, int q) {
    float b[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        b[e] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x[e]), CTRL, 0xf, 0xf, false));
    return q == 0 ? b[0] : q == 1 ? b[1] : q == 2 ? b[2] : b[3];
}

template <int C, int NI>
__global__ void __launch_bounds__(256)
mfma_qb_kernel(const float* __restrict__ A, int64_t lda, const float* __restrict__ Bm,
               int64_t ldb, int nb, int N, int K, int nrot, float* __restrict__ C1, int64_t ld1,
               float* __restrict__ C2, int64_t ld2, const float* __restrict__ norms, int nsplit,
               v4f* __restrict__ part) {
    constexpr int RT = 4, NT = C * RT;
    extern __shared__ __align__(16) unsigned char smem[];
    v4f* red = reinterpret_cast<v4f*>(smem);  // [4 waves][NT tiles][64 lanes]
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int cg = blockIdx.x, sp = blockIdx.y, rb = blockIdx.z;
    const int b0 = rb * 64, n0 = cg * 16 * C;
    // lane (r, g) reads the float4 at k = 16*step + 4g of its rows: the four
    // k-groups of a row read 64 contiguous bytes per load
    const int ka = (sp * 4 + wv) * NI * 16 + 4 * g;
    float4 av[NI][RT], bv[NI][C];
#pragma unroll
    for (int u = 0; u < NI; u++) {
        const int uu = u;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const int row = b0 + 16 * i + r;
            av[u][i] = ((const float4*)(A + (int64_t)(row < nb ? row : 0) * lda + ka))[4 * uu];
        }
#pragma unroll
        for (int c = 0; c < C; c++) {
            const int col = n0 + 16 * c + r;
            bv[u][c] = ((const float4*)(Bm + (int64_t)(col < N ? col : 0) * ldb + ka))[4 * uu];
        }
    }
    // every load is in flight before the first MFMA (the scheduler would
    // otherwise sink each load to its first use and wait for it there)
    __builtin_amdgcn_sched_barrier(0);
    v4f acc[C][RT];
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int i = 0; i < RT; i++) acc[c][i] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NI; u++) {
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int c = 0; c < C; c++)
#pragma unroll
                for (int i = 0; i < RT; i++) {
                    const float a = e == 0 ? av[u][i].x : e == 1 ? av[u][i].y : e == 2 ? av[u][i].z : av[u][i].w;
                    const float b = e == 0 ? bv[u][c].x : e == 1 ? bv[u][c].y : e == 2 ? bv[u][c].z : bv[u][c].w;
                    acc[c][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c][i], 0, 0, 0);
                }
    }
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int i = 0; i < RT; i++) red[(wv * NT + c * RT + i) * 64 + lane] = acc[c][i];
    __syncthreads();
    // wave w finishes tiles w, w + 4, ...: the four wave sums in wave order
    v4f sum[(NT + 3) / 4];
#pragma unroll
    for (int j = 0; j < (NT + 3) / 4; j++) {
        const int t = wv + 4 * j;
        if (t < NT) {
            v4f v = red[t * 64 + lane];
#pragma unroll
            for (int w2 = 1; w2 < 4; w2++) v += red[(w2 * NT + t) * 64 + lane];
            sum[j] = v;
        }
    }
    if (nsplit > 1) {
        // split sp's rows, row-major: part[sp][row][col] (64 gridDim.z rows
        // per split); mfma_qb_reduce_kernel or the probe selection finishes.
        // A quad of lanes (columns 4a .. 4a+3, rows 4g + e) transposes its
        // 4 x 4 block so that lane q stores row 4g + q, four columns in one
        // 16-byte store (N % 4 == 0; else one float at a time)
        float* mine = reinterpret_cast<float*>(part) + (int64_t)sp * gridDim.z * 64 * N;
        const int q = r & 3;
#pragma unroll
        for (int j = 0; j < (NT + 3) / 4; j++) {
            const int t = wv + 4 * j;
            if (t >= NT) continue;
            const int c = t / RT, i = t % RT;
            if ((N & 3) == 0) {
                // lane kq of the quad holds column 4a + kq, rows 4g + 0..3
                const float4 o = make_float4(quad_pick<0x00>(sum[j], q), quad_pick<0x55>(sum[j], q),
                                             quad_pick<0xAA>(sum[j], q), quad_pick<0xFF>(sum[j], q));
                const int col0 = n0 + 16 * c + (r & ~3);
                if (col0 < N) *(float4*)(mine + (int64_t)(b0 + 16 * i + 4 * g + q) * N + col0) = o;
            } else {
                const int col = n0 + 16 * c + r;
                if (col >= N) continue;
#pragma unroll
                for (int e = 0; e < 4; e++) mine[(int64_t)(b0 + 16 * i + 4 * g + e) * N + col] = sum[j][e];
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < (NT + 3) / 4; j++) {
        const int t = wv + 4 * j;
        if (t >= NT) continue;
        const int c = t / RT, i = t % RT;
        const int col = n0 + 16 * c + r;
        if (col >= N) continue;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int row = b0 + 16 * i + 4 * g + e;
            if (row < nb) {
                const float v = sum[j][e];
                if (col < nrot) C1[(int64_t)row * ld1 + col] = v;
                else C2[(int64_t)row * ld2 + (col - nrot)] = fmaf(-2.0f, v, norms[col - nrot]);
            }
        }
    }
}

// part[sp][row][col] summed over sp in order, then stored like
// mfma_qb_kernel's epilogue; one thread per (row, col), row < nb.
__global__ void __launch_bounds__(256)
mfma_qb_reduce_kernel(const float* __restrict__ part, int64_t pstride, int nsplit, int nb, int N,
                      int nrot, float* __restrict__ C1, int64_t ld1, float* __restrict__ C2,
                      int64_t ld2, const float* __restrict__ norms) {
    const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (x >= (int64_t)nb * N) return;
    const int row = (int)(x / N), col = (int)(x - (int64_t)row * N);
    float v = part[x];
    for (int s2 = 1; s2 < nsplit; s2++) v += part[s2 * pstride + x];
    if (col < nrot) C1[(int64_t)row * ld1 + col] = v;
    else C2[(int64_t)row * ld2 + (col - nrot)] = fmaf(-2.0f, v, norms[col - nrot]);
}

// Floats between two splits' rows in the partial buffer of plan p.
int64_t qb_part_stride(const QbPlan& p, int N) { return (int64_t)p.R * 64 * N; }

QbPlan mfma_qb_plan(int nb, int N, int K) {
    QbPlan p{};
    if (nb <= 0 || N <= 0 || K <= 0 || K % 64 != 0) return p;
    // K / 16 = 4m steps of 16; nsplit = the least divisor of m that leaves
    // at most 4 steps per wave
    const int m = K / 64;
    int s = (m + 3) / 4;
    while (m % s) s++;
    const int T = (N + 15) / 16, R = (nb + 63) / 64;
    int best = 0;
    int64_t best_cost = 0;
    for (int c = 1; c <= 5; c++) {
        // MFMA steps of the busiest CU with one workgroup per CU per round
        const int64_t wg = (int64_t)((T + c - 1) / c) * s * R;
        const int64_t cost = (wg + 255) / 256 * c;
        if (best == 0 || cost <= best_cost) {
            best = c;
            best_cost = cost;
        }
    }
    p.C = best;
    p.nsplit = s;
    p.NI = m / s;
    p.ncg = (T + best - 1) / best;
    p.R = R;
    p.part_floats = s > 1 ? (size_t)s * R * 64 * N : 0;
    return p;
}

size_t mfma_qb_space(int nb_max, int N, int K) {
    // any plan for nb <= nb_max: ncg * C <= T + 4 column tiles, R <= R_max
    const QbPlan p = mfma_qb_plan(nb_max, N, K);
    return p.part_floats;
}

template <int C, int NI>
static hipError_t launch_qb(const QbPlan& p, const float* A, int64_t lda, const float* Bm,
                            int64_t ldb, int nb, int N, int K, int nrot, float* C1, int64_t ld1,
                            float* C2, int64_t ld2, const float* norms, float* part,
                            bool reduce, hipStream_t s) {
    const void* fn = (const void*)mfma_qb_kernel<C, NI>;
    const int lds = 4 * C * 4 * 64 * 16;
    static const hipError_t attr = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((mfma_qb_kernel<C, NI>), dim3(p.ncg, p.nsplit, p.R), dim3(256), lds, s, A, lda,
                       Bm, ldb, nb, N, K, nrot, C1, ld1, C2, ld2, norms, p.nsplit,
                       reinterpret_cast<v4f*>(part));
    if (p.nsplit > 1 && reduce) {
        const int64_t per = (int64_t)nb * N;
        hipLaunchKernelGGL(mfma_qb_reduce_kernel, dim3((unsigned)((per + 255) / 256)), dim3(256), 0,
                           s, part, qb_part_stride(p, N), p.nsplit, nb, N, nrot, C1, ld1, C2, ld2,
                           norms);
    }
    return hipGetLastError();
}

hipError_t mfma_qb(const QbPlan& p, const float* A, int64_t lda, const float* Bm, int64_t ldb,
                   int nb, int N, int K, int nrot, float* C1, int64_t ld1, float* C2, int64_t ld2,
                   const float* norms, float* part, size_t part_floats, hipStream_t s,
                   bool reduce) {
    if (nb <= 0 || N <= 0) return hipSuccess;
    if (!mfma_q_ok(K, lda, ldb) || ((uintptr_t)A & 15) || ((uintptr_t)Bm & 15) ||
        ((uintptr_t)part & 15) || p.C < 1 || p.C > 5 || p.NI < 1 || p.NI > 4 || p.R > 65535 ||
        p.nsplit > 65535 || p.part_floats > part_floats || (p.nsplit > 1 && !part))
        return hipErrorInvalidValue;
#define JHQ_QB(CC)                                                                              \
    switch (p.NI) {                                                                             \
        case 1: return launch_qb<CC, 1>(p, A, lda, Bm, ldb, nb, N, K, nrot, C1, ld1, C2, ld2, norms, part, reduce, s); \
        case 2: return launch_qb<CC, 2>(p, A, lda, Bm, ldb, nb, N, K, nrot, C1, ld1, C2, ld2, norms, part, reduce, s); \
        case 3: return launch_qb<CC, 3>(p, A, lda, Bm, ldb, nb, N, K, nrot, C1, ld1, C2, ld2, norms, part, reduce, s); \
        default: return launch_qb<CC, 4>(p, A, lda, Bm, ldb, nb, N, K, nrot, C1, ld1, C2, ld2, norms, part, reduce, s); \
    }
    switch (p.C) {
        case 1: JHQ_QB(1)
        case 2: JHQ_QB(2)
        case 3: JHQ_QB(3)
        case 4: JHQ_QB(4)
        default: JHQ_QB(5)
    }
#undef JHQ_QB
}

template <int EPI>
static hipError_t launch_mfma(const float* A, int64_t lda, const float* Bm, int64_t ldb, int nb,
                              int N, int K, float* C, int64_t ldc, const float* norms,
                              hipStream_t s) {
    if (nb <= 0 || N <= 0) return hipSuccess;
    const int64_t tiles = (int64_t)((N + 15) / 16) * ((nb + 15) / 16);
    if ((nb + 15) / 16 > 65535) return hipErrorInvalidValue;
    int S = 1;
    while (S < 8 && tiles * S < 2048 && K / (S * 2) >= 64) S *= 2;
    const bool vec = (K % (64 * S) == 0) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                     ((uintptr_t)A % 16 == 0) && ((uintptr_t)Bm % 16 == 0);
    dim3 grid((N + 15) / 16, (nb + 15) / 16);
#define JHQ_MFMA_LAUNCH(SS)                                                                     \
    if (vec)                                                                                  \
        hipLaunchKernelGGL((mfma_nt_kernel<SS, EPI, true>), grid, dim3(64 * SS), 0, s, A, lda, \
                           Bm, ldb, nb, N, K, C, ldc, norms);                                 \
    else                                                                                      \
        hipLaunchKernelGGL((mfma_nt_kernel<SS, EPI, false>), grid, dim3(64 * SS), 0, s, A,     \
                           lda, Bm, ldb, nb, N, K, C, ldc, norms);
    switch (S) {
        case 1: JHQ_MFMA_LAUNCH(1) break;
        case 2: JHQ_MFMA_LAUNCH(2) break;
        case 4: JHQ_MFMA_LAUNCH(4) break;
        default: JHQ_MFMA_LAUNCH(8) break;
    }
#undef JHQ_MFMA_LAUNCH
    return hipGetLastError();
}

hipError_t mfma_nt_store(const float* A, int64_t lda, const float* Bm, int64_t ldb, int nb, int N,
                         int K, float* C, int64_t ldc, hipStream_t s) {
    return launch_mfma<EPI_STORE>(A, lda, Bm, ldb, nb, N, K, C, ldc, nullptr, s);
}

hipError_t mfma_nt_score(const float* A, int64_t lda, const float* Bm, int64_t ldb, int nb, int N,
                         int K, const float* norms, float* C, int64_t ldc, hipStream_t s) {
    return launch_mfma<EPI_SCORE>(A, lda, Bm, ldb, nb, N, K, C, ldc, norms, s);
}

// Stored vectors decoded from their primary codes (rotated space, each
// coordinate its digit's Lloyd-Max level): rows[i] for the candidate at
// column samp[i].z of the list block (start samp[i].x, row stride samp[i].y).
// Used as stand-in queries when estimating how a batch's probes overlap.
__global__ void decode_rows_kernel(const int4* __restrict__ samp, const uint8_t* __restrict__ codes_t,
                                   int M, int Ds, int K1D, int bpd, const float* __restrict__ c1d,
                                   float* __restrict__ rows) {
    const int i = blockIdx.x;
    const int4 sp = samp[i];
    const int d = M * Ds;
    for (int t = threadIdx.x; t < d; t += blockDim.x) {
        const int m = t / Ds, k = t - m * Ds;
        const uint8_t v = codes_t[(int64_t)sp.x * M + (int64_t)m * sp.y + sp.z];
        rows[(int64_t)i * d + t] = c1d[(v >> (k * bpd)) & (K1D - 1)];
    }
}

hipError_t decode_rows(const int4* samp, int S, const uint8_t* codes_t, int M, int Ds, int K1D,
                       int bpd, const float* c1d, float* rows, hipStream_t s) {
    if (S <= 0) return hipSuccess;
    hipLaunchKernelGGL(decode_rows_kernel, dim3(S), dim3(256), 0, s, samp, codes_t, M, Ds, K1D,
                       bpd, c1d, rows);
    return hipGetLastError();
}

// uint8 / int8 vectors converted to float32 on the device (dtype 1 = uint8,
// 2 = int8), 16 elements per thread iteration.
__global__ void convert_kernel(const uint8_t* __restrict__ src, int dtype, int64_t n,
                               float* __restrict__ dst) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = dtype == 1 ? (float)src[i] : (float)(int8_t)src[i];
}

hipError_t convert_to_f32(const void* src, int dtype, int64_t n, float* dst, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (dtype != 1 && dtype != 2) return hipErrorInvalidValue;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(convert_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, s, (const uint8_t*)src, dtype, n, dst);
    return hipGetLastError();
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

// One wave of a fixed-length dependent fmaf chain (the search lanes' queue
// probe): its time is set by the chain, not by the GPU's load.
__global__ void __launch_bounds__(64) lane_probe_kernel(float* out, int iters) {
    float x = (float)threadIdx.x;
    for (int i = 0; i < iters; i++) x = fmaf(x, 0.999999f, 1.0f);
    if (threadIdx.x == 0) *out = x;
}

hipError_t lane_probe(float* out, int iters, hipStream_t s) {
    if (!out || iters < 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(lane_probe_kernel, dim3(1), dim3(64), 0, s, out, iters);
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
// Encode: a workgroup takes kEncV vectors and walks their dimensions in
// chunks of kEncC.  Every thread quantizes dimensions of the chunk (reads of
// consecutive floats of one vector), the digits and residual indices are
// packed into code and residual bytes from LDS, and one lane per vector
// carries that vector's residual correction: a sequential fmaf chain in
// dimension order over the quantized values the chunk left in LDS.
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

constexpr int kEncV = 16, kEncC = 128, kEncT = 256;
constexpr int kEncPer = kEncV * kEncC / kEncT;  // dimensions a thread quantizes per chunk

__global__ void __launch_bounds__(kEncT)
encode_kernel(const float* __restrict__ y, int64_t n, int d, int M, int Ds, int K1D, int bpd,
              const float* __restrict__ c1d, int Kr, int RC, int Br, int bpv,
              const float* __restrict__ res_c1d, uint8_t* __restrict__ codes,
              uint8_t* __restrict__ res, float* __restrict__ corr, int mode) {
    // RC residual codebooks of Kr words: one shared by every dimension (the
    // reference, v14/jhq_gpu_index.cu:302-330) or one per subspace (RC = M)
    __shared__ float cval[256], cmid[256];
    // the chunk's quantized values (yhat, rhat) per vector; the odd row
    // stride puts the chain lanes' reads of one column in distinct banks
    __shared__ float yh[kEncV][kEncC + 1], rh[kEncV][kEncC + 1];
    __shared__ uint8_t dg[kEncV][kEncC], rq[kEncV][kEncC];
    extern __shared__ float rsh[];  // rval[RC*Kr], rmid[RC*Kr]
    float* rval = rsh;
    float* rmid = rsh + RC * Kr;
    const int tid = threadIdx.x;
    const int64_t v0 = (int64_t)blockIdx.x * kEncV;
    const int nv = (n - v0) < kEncV ? (int)(n - v0) : kEncV;
    if (tid < K1D) cval[tid] = c1d[tid];
    if (mode & 2)
        for (int i = tid; i < RC * Kr; i += kEncT) rval[i] = res_c1d[i];
    __syncthreads();
    if (tid + 1 < K1D) cmid[tid] = 0.5f * (cval[tid] + cval[tid + 1]);
    if (mode & 2)
        for (int i = tid; i < RC * Kr; i += kEncT)
            if ((i % Kr) + 1 < Kr) rmid[i] = 0.5f * (rval[i] + rval[i + 1]);
    __syncthreads();
    const int kmask = K1D - 1;
    float dot = 0.0f;  // lane v < nv: vector v0 + v's chain
    for (int c0 = 0; c0 < d; c0 += kEncC) {
        const int cw = (d - c0) < kEncC ? (d - c0) : kEncC;
        float val[kEncPer];
#pragma unroll
        for (int i = 0; i < kEncPer; i++) {
            const int e = tid + i * kEncT, v = e / kEncC, jj = e % kEncC;
            val[i] = (v < nv && jj < cw) ? y[(v0 + v) * d + c0 + jj] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kEncPer; i++) {
            const int e = tid + i * kEncT, v = e / kEncC, jj = e % kEncC;
            if (v >= nv || jj >= cw) continue;
            const int j = c0 + jj;
            const int m = j / Ds, k = j - m * Ds;
            int dig;
            if (mode & 1) dig = (K1D == 1) ? 0 : nearest_mid(cmid, K1D, val[i]);
            else dig = (codes[(v0 + v) * M + m] >> (k * bpd)) & kmask;
            dg[v][jj] = (uint8_t)dig;
            if (mode & 2) {
                const int cb = (RC == 1) ? 0 : m;
                const float yhat = cval[dig];
                const float r = val[i] - yhat;
                const int ri = (Kr == 1) ? 0 : nearest_mid(rmid + cb * Kr, Kr, r);
                rq[v][jj] = (uint8_t)ri;
                yh[v][jj] = yhat;
                rh[v][jj] = rval[cb * Kr + ri];
            }
        }
        __syncthreads();
        if (mode & 1) {
            // whole subspaces of the chunk (c0 is a multiple of Ds, which divides 32)
            const int ms = cw / Ds;
            for (int e = tid; e < kEncV * ms; e += kEncT) {
                const int v = e / ms, mm = e - v * ms;
                if (v >= nv) continue;
                uint32_t code = 0u;
                for (int k = 0; k < Ds; k++) code |= (uint32_t)dg[v][mm * Ds + k] << (k * bpd);
                codes[(v0 + v) * M + c0 / Ds + mm] = (uint8_t)code;
            }
        }
        if (mode & 2) {
            if (Br == 4) {
                // two dimensions a byte, the even one in the low nibble; an odd
                // last dimension alone in the low nibble of the last byte
                const int nb = (cw + 1) >> 1;
                for (int e = tid; e < kEncV * nb; e += kEncT) {
                    const int v = e / nb, b = e - v * nb;
                    if (v >= nv) continue;
                    const uint32_t lo = rq[v][2 * b] & 0x0Fu;
                    const uint32_t hi = (2 * b + 1 < cw) ? (rq[v][2 * b + 1] & 0x0Fu) : 0u;
                    res[(v0 + v) * bpv + (c0 >> 1) + b] = (uint8_t)(lo | (hi << 4));
                }
            } else {
                for (int e = tid; e < kEncV * cw; e += kEncT) {
                    const int v = e / cw, jj = e - v * cw;
                    if (v >= nv) continue;
                    res[(v0 + v) * bpv + c0 + jj] = rq[v][jj];
                }
            }
            if (tid < nv)
                for (int jj = 0; jj < cw; jj++) dot = fmaf(yh[tid][jj], rh[tid][jj], dot);
        }
        __syncthreads();
    }
    if ((mode & 2) && tid < nv) corr[v0 + tid] = 2.0f * dot;
}

hipError_t encode(const float* y, int64_t n, int d, int M, int Ds, int K1D, int bpd,
                  const float* c1d, int Kr, int RC, int Br, int bpv, const float* res_c1d,
                  uint8_t* codes, uint8_t* res, float* corr, int mode, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (K1D > 256 || Kr > 256 || (32 % Ds) != 0 || (RC != 1 && RC != M) || Ds * M != d ||
        ((mode & 2) && Br != 4 && Br != 8))
        return hipErrorInvalidValue;
    const size_t lds = (size_t)2 * RC * Kr * sizeof(float);
    if (lds > 96 * 1024) return hipErrorInvalidValue;
    if (lds > 48 * 1024) {
        static const hipError_t e = hipFuncSetAttribute((const void*)encode_kernel,
                                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                                         96 * 1024);
        if (e != hipSuccess) return e;
    }
    const int64_t blocks = (n + kEncV - 1) / kEncV;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(encode_kernel, dim3((unsigned)blocks), dim3(kEncT), lds, s, y, n, d, M, Ds,
                       K1D, bpd, c1d, Kr, RC, Br, bpv, res_c1d, codes, res, corr, mode);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// List storage.  The lists live in one pool of padded candidate slots; list l
// is described by ListDesc {start, cap, size, cbase} (int4): it owns slots
// [start, start + cap) (cap a multiple of 16) and holds size candidates.
// Primary codes are code-major inside the block: byte m of candidate i is at
// codes_t[start*M + m*cap + i], so one 32-bit load returns byte m of four
// consecutive candidates.  Residual codes, corrections and ids are indexed by
// slot.  cbase is the list's first canonical position (lists in list order,
// candidates in insertion order), the tag the exact selection breaks ties
// with, so results do not depend on where a list's block sits in the pool.
// ---------------------------------------------------------------------------
__global__ void scatter_kernel(const int32_t* __restrict__ order, const int32_t* __restrict__ slist,
                               const int32_t* __restrict__ sidx, int64_t n, int64_t id_base,
                               const int4* __restrict__ ldesc, const uint8_t* __restrict__ pc,
                               const uint8_t* __restrict__ rc, const float* __restrict__ co, int M,
                               int bpv, int32_t* __restrict__ ids_out, uint8_t* __restrict__ codes_t,
                               uint8_t* __restrict__ res_out, float* __restrict__ corr_out) {
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const int64_t id = order[s];
    const int4 L = ldesc[slist[s]];
    const int64_t i = sidx[s];
    const int64_t slot = (int64_t)L.x + i;
    ids_out[slot] = (int32_t)(id + id_base);
    corr_out[slot] = co[id];
    uint8_t* dst = codes_t + (int64_t)L.x * M + i;
    const uint8_t* src = pc + id * M;
    for (int m = 0; m < M; m++) dst[(int64_t)m * L.y] = src[m];
    const uint8_t* rs = rc + id * bpv;
    uint8_t* rd = res_out + slot * bpv;
    for (int b2 = 0; b2 < bpv; b2++) rd[b2] = rs[b2];
}

// ---------------------------------------------------------------------------
// Lane-skewed copy of the primary codes, for the scan that runs each lane a
// fixed number of subspaces behind its neighbours.  Candidate i of a list
// (pool slot p = start + i) gets M bytes
//   row[t] = code[t - s]                 for t >= s = i mod 32,
//   row[t] = (code[M + t - s] + 1) mod 256 for t < s,
// so that at step t the lane holding i reads subspace t - s from row
// position t.  The tail bytes (t < s, read one period later, with the next
// candidate's head bytes) are raised by one LUT row: their LUT address
// (v + 1) * M + t - s is then the head bytes' formula, and code 255 wraps to
// the copy of row 255's last subspaces kept just below the LUT.
// The rows are stored in blocks of 16 slots (list starts and capacities are
// multiples of 16), piece by piece: the 16 bytes row[16q .. 16q+15] of slot p
// are at skew_piece(p, q) = ((p / 16) * (M / 16) + q) * 256 + (p mod 16) * 16,
// so the 64 lanes of a wave reading one piece of their candidates (four
// blocks of 16 consecutive slots) touch four 256-byte runs.
// Rows from[l] .. size-1 of list l are written (with the rest of the first
// block, whose rows are current anyway); one thread per piece, the codes read
// from the code-major blocks (codes_t[start * M + m * cap + i]).
// ---------------------------------------------------------------------------
__host__ __device__ inline int64_t skew_piece(int64_t p, int q, int M) {
    return ((p >> 4) * (M >> 4) + q) * 256 + (p & 15) * 16;
}

__global__ void skew_codes_kernel(const int4* __restrict__ ldesc, const int32_t* __restrict__ from,
                                  const uint8_t* __restrict__ codes_t, int M,
                                  uint8_t* __restrict__ skew) {
    const int4 L = ldesc[blockIdx.x];
    const int q = threadIdx.x >> 4;
    if (q >= M / 16) return;
    // blocks of 16 slots; grid-y strides over the list's blocks
    for (int64_t i = (int64_t)(from[blockIdx.x] & ~15) + (int64_t)blockIdx.y * 16 + (threadIdx.x & 15);
         i < L.z; i += (int64_t)gridDim.y * 16) {
        const uint8_t* src = codes_t + (int64_t)L.x * M + i;
        const int s = (int)(i & 31);
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            w[k] = 0u;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int m = 16 * q + 4 * k + e - s;
                // tail bytes (t < s) hold code + 1 (mod 256)
                const uint32_t inc = m < 0 ? 1u : 0u;
                if (m < 0) m += M;
                w[k] |= ((src[(int64_t)m * L.y] + inc) & 0xffu) << (8 * e);
            }
        }
        *(uint4*)(skew + skew_piece((int64_t)L.x + i, q, M)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

int64_t skew_bytes(int64_t pool_cap, int M) { return (pool_cap + 15) / 16 * 16 * M; }

// Row-major copy of the primary codes: slot p's M bytes at rows[p * M], so
// that one vector's codes are one contiguous run (the pre-scan's re-check
// reads whole rows of a few candidates).  Rows from[l] .. size-1 of list l
// (from rounded down to 16); thread (16-byte piece q, slot i % 16).
__global__ void row_codes_kernel(const int4* __restrict__ ldesc, const int32_t* __restrict__ from,
                                 const uint8_t* __restrict__ codes_t, int M,
                                 uint8_t* __restrict__ rows) {
    const int4 L = ldesc[blockIdx.x];
    const int q = threadIdx.x >> 4;
    if (q >= M / 16) return;
    for (int64_t i = (int64_t)(from[blockIdx.x] & ~15) + (int64_t)blockIdx.y * 16 + (threadIdx.x & 15);
         i < L.z; i += (int64_t)gridDim.y * 16) {
        const uint8_t* src = codes_t + (int64_t)L.x * M + i;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            w[k] = 0u;
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[k] |= (uint32_t)src[(int64_t)(16 * q + 4 * k + e) * L.y] << (8 * e);
        }
        *(uint4*)(rows + ((int64_t)L.x + i) * M + 16 * q) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

hipError_t row_codes(const int4* ldesc, const int32_t* from, int nlist, int max_rows,
                     const uint8_t* codes_t, int M, uint8_t* rows, hipStream_t s) {
    if (nlist <= 0 || max_rows <= 0) return hipSuccess;
    const int64_t gy = std::min<int64_t>(((int64_t)max_rows + 15 + 15) / 16, 65535);
    if (M % 16 != 0 || M > 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(row_codes_kernel, dim3(nlist, (unsigned)gy), dim3(M), 0, s, ldesc, from,
                       codes_t, M, rows);
    return hipGetLastError();
}

hipError_t skew_codes(const int4* ldesc, const int32_t* from, int nlist, int max_rows,
                      const uint8_t* codes_t, int M, uint8_t* skew, hipStream_t s) {
    if (nlist <= 0 || max_rows <= 0) return hipSuccess;
    // one block of threads per 16 slots; from[l] is rounded down to 16
    // (a list of any length: the kernel strides over grid-y)
    const int64_t gy = std::min<int64_t>(((int64_t)max_rows + 15 + 15) / 16, 65535);
    if (M % 32 != 0 || M > 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(skew_codes_kernel, dim3(nlist, (unsigned)gy), dim3(M), 0, s, ldesc, from,
                       codes_t, M, skew);
    return hipGetLastError();
}

hipError_t scatter_lists(const int32_t* order, const int32_t* slist, const int32_t* sidx,
                         int64_t n, int64_t id_base, const int4* ldesc, const uint8_t* pc,
                         const uint8_t* rc, const float* co, int M, int bpv, int32_t* ids_out,
                         uint8_t* codes_t, uint8_t* res_out, float* corr_out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)blocks), dim3(256), 0, s, order, slist, sidx,
                       n, id_base, ldesc, pc, rc, co, M, bpv, ids_out, codes_t, res_out, corr_out);
    return hipGetLastError();
}

// Moves list blocks.  moves[2r] = {start, cap, size} of block r's source,
// moves[2r+1] = {start, cap} of its destination; the size candidates are
// copied and the code-major primary codes re-strided.  Source and
// destination blocks never overlap (destinations lie past every live block,
// or in another pool).
__global__ void relocate_kernel(const int4* __restrict__ moves, int M, int bpv,
                                const uint8_t* __restrict__ codes_src, uint8_t* __restrict__ codes_dst,
                                const uint8_t* __restrict__ res_src, uint8_t* __restrict__ res_dst,
                                const float* __restrict__ corr_src, float* __restrict__ corr_dst,
                                const int32_t* __restrict__ ids_src, int32_t* __restrict__ ids_dst) {
    const int4 fr = moves[blockIdx.x * 2];
    const int4 to = moves[blockIdx.x * 2 + 1];
    const int size = fr.z;
    if (size <= 0) return;
    const uint8_t* cs = codes_src + (int64_t)fr.x * M;
    uint8_t* cd = codes_dst + (int64_t)to.x * M;
    for (int64_t e = threadIdx.x; e < (int64_t)M * size; e += blockDim.x) {
        const int64_t m = e / size, i = e - m * size;
        cd[m * to.y + i] = cs[m * fr.y + i];
    }
    const uint8_t* rs = res_src + (int64_t)fr.x * bpv;
    uint8_t* rd = res_dst + (int64_t)to.x * bpv;
    for (int64_t e = threadIdx.x; e < (int64_t)size * bpv; e += blockDim.x) rd[e] = rs[e];
    for (int i = threadIdx.x; i < size; i += blockDim.x) {
        corr_dst[to.x + i] = corr_src[fr.x + i];
        ids_dst[to.x + i] = ids_src[fr.x + i];
    }
}

hipError_t relocate_lists(const int4* moves, int nmoves, int M, int bpv, const uint8_t* codes_src,
                          uint8_t* codes_dst, const uint8_t* res_src, uint8_t* res_dst,
                          const float* corr_src, float* corr_dst, const int32_t* ids_src,
                          int32_t* ids_dst, hipStream_t s) {
    if (nmoves <= 0) return hipSuccess;
    hipLaunchKernelGGL(relocate_kernel, dim3((unsigned)nmoves), dim3(256), 0, s, moves, M, bpv,
                       codes_src, codes_dst, res_src, res_dst, corr_src, corr_dst, ids_src,
                       ids_dst);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Streaming exact top-k.
//
// The candidates of one selection arrive in rounds: in each round every
// thread of the workgroup supplies CPT (value, tag) pairs (value ~0u = no
// candidate).  The exact top-k by (value, tag) ascending is kept as a short
// list of survivors in LDS:
//   - bound: in the first round each wave contributes its c smallest values
//     (c rounds of wave-min) and the bound is the k-th smallest of that pool,
//     so at least k candidates are <= it; later the bound is the k-th
//     smallest survivor after each prune;
//   - survivors (value <= bound) are appended with one atomic per wave;
//   - when the list passes half its capacity it is pruned to the exact top-k;
//   - if a round does not fit, what fit is pruned, the bound tightens and the
//     rest of the round (still in registers) is appended again.
// Every step is exact: a candidate is dropped only when k kept candidates
// precede it in (value, tag) order.
// ---------------------------------------------------------------------------
template <int NT>
__device__ __forceinline__ void rank_select(const unsigned long long* in, int n, int k,
                                            unsigned long long* out, int* src = nullptr) {
    // Key i's rank = number of keys smaller than it; keys are distinct except
    // for the ~0 padding, which ranks after every key that is written
    // (k <= number of real keys).  tpk lanes share one key, each counting over
    // a contiguous slice of the keys, then add their counts with xor shuffles.
    int tpk = 1;
    while (tpk < 64 && tpk * 2 * n <= NT) tpk *= 2;
    const int part = threadIdx.x & (tpk - 1);
    const int j0 = (int)((int64_t)n * part / tpk), j1 = (int)((int64_t)n * (part + 1) / tpk);
    for (int base = 0; base < n; base += NT / tpk) {
        const int i = base + (int)threadIdx.x / tpk;
        const unsigned long long ki = i < n ? in[i] : ~0ull;
        int r = 0;
#pragma unroll 8
        for (int j = j0; j < j1; j++) r += (in[j] < ki) ? 1 : 0;
        for (int off = tpk >> 1; off > 0; off >>= 1) r += __shfl_xor(r, off);
        if (part == 0 && i < n && r < k) {
            out[r] = ki;
            if (src) src[r] = i;
        }
    }
    __syncthreads();
}

// Exact top-k of n keys in LDS (n >= k, the first k are real) into out[0..k).
// Returns whether src (optional, k ints; may be idx) holds each output key's
// index in `in` (the ranking path, for short inputs).
template <int NT>
__device__ __forceinline__ bool select_keys(const unsigned long long* in, int n, int k,
                                            unsigned long long* out, int* idx,
                                            unsigned long long* tmp, SelState* st,
                                            int* src = nullptr) {
    if ((int64_t)n * n <= (int64_t)NT * 512) {
        rank_select<NT>(in, n, k, out, src);
        return src != nullptr;
    }
    block_topk<NT>([&](int i) { return (uint32_t)(in[i] >> 32); },
                   [&](int i) { return (uint32_t)(in[i] & 0xffffffffull); }, n, k, idx, tmp,
                   out, st);
    return false;
}

// Values each wave contributes to the first-round bound.
__host__ __device__ constexpr int est_per_wave(int k, int nw) {
    return ((k + nw - 1) / nw) * 2 < ((k + nw - 1) / nw) + 8 ? ((k + nw - 1) / nw) * 2
                                                               : ((k + nw - 1) / nw) + 8;
}

struct StreamSel {
    unsigned long long* skeys;  // [scap] survivors
    unsigned long long* kout;   // [k]
    unsigned long long* ktmp;   // [k]
    int* kidx;                  // [k]
    uint32_t* wstat;            // [NT/64 * est_per_wave(k)] per-wave smallest values
    int* ctl;                   // [4]: survivor count, bound, bound valid, estimate
    SelState* st;
    int scap;
};

template <int NT>
__device__ __forceinline__ void stream_begin(const StreamSel& S) {
    if (threadIdx.x == 0) {
        S.ctl[0] = 0;
        S.ctl[1] = (int)~0u;
        S.ctl[2] = 0;
    }
}

// Prunes the survivor list skeys[0..n) to its exact top-k and tightens the
// bound.  Called by every thread; ends with a barrier.
template <int NT>
__device__ __forceinline__ void stream_prune(const StreamSel& S, int n, int k) {
    select_keys<NT>(S.skeys, n, k, S.kout, S.kidx, S.ktmp, S.st);
    for (int i = threadIdx.x; i < k; i += NT) S.skeys[i] = S.kout[i];
    if (threadIdx.x == 0) {
        S.ctl[0] = k;
        S.ctl[1] = (int)min((uint32_t)S.ctl[1], (uint32_t)(S.kout[k - 1] >> 32));
        S.ctl[2] = 1;
    }
    __syncthreads();
}

// One round: o[j] / tg[j] are this thread's values and tags.
template <int NT, int CPT>
__device__ __forceinline__ void stream_round(const StreamSel& S, int k, const uint32_t (&o)[CPT],
                                             const uint32_t (&tg)[CPT],
                                             unsigned long long* stats = nullptr) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t Tcur = (uint32_t)S.ctl[1];
    const bool est = S.ctl[2] == 0;
    if (est) {
        // each wave contributes its c smallest values; the bound is the k-th
        // smallest of the pooled values (>= k values are <= it)
        const int c = est_per_wave(k, NW);
        uint32_t t[CPT];
#pragma unroll
        for (int j = 0; j < CPT; j++) t[j] = o[j];
        for (int it = 0; it < c; it++) {
            uint32_t lm = t[0];
#pragma unroll
            for (int j = 1; j < CPT; j++) lm = min(lm, t[j]);
            uint32_t m = lm;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) m = min(m, (uint32_t)__shfl_xor((int)m, off));
            if (lane == 0) S.wstat[wv * c + it] = m;
            if (m == ~0u) continue;
            const unsigned long long bal = __ballot(lm == m);
            if (lane == __ffsll((long long)bal) - 1) {
                bool hit = false;
#pragma unroll
                for (int j = 0; j < CPT; j++) {
                    if (!hit && t[j] == m) {
                        t[j] = ~0u;
                        hit = true;
                    }
                }
            }
        }
        if (tid == 0) S.ctl[3] = (int)~0u;
    }
    __syncthreads();
    uint32_t T = Tcur;
    if (est) {
        const int c = est_per_wave(k, NW);
        const int npool = NW * c;
        for (int i = tid; i < npool; i += NT) {
            const uint32_t v = S.wstat[i];
            if (v == ~0u) continue;
            int lt = 0, le = 0;
            for (int j = 0; j < npool; j++) {
                const uint32_t u = S.wstat[j];
                lt += (u < v) ? 1 : 0;
                le += (u <= v) ? 1 : 0;
            }
            if (lt < k && k <= le) S.ctl[3] = (int)v;  // the k-th smallest (all writers agree)
        }
        __syncthreads();
        T = min(T, (uint32_t)S.ctl[3]);
        if (tid == 0 && T != ~0u) {
            S.ctl[1] = (int)T;
            S.ctl[2] = 1;
        }
    }
    uint32_t pend = 0u;
#pragma unroll
    for (int j = 0; j < CPT; j++)
        if (o[j] != ~0u && o[j] <= T) pend |= 1u << j;
    for (;;) {
        // append the pending survivors: one atomic per wave
        const int cnt = __popc(pend);
        int incl = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t2 = __shfl_up(incl, off);
            if (lane >= off) incl += t2;
        }
        int wbase = 0;
        if (lane == 63 && incl) wbase = atomicAdd(&S.ctl[0], incl);
        wbase = __shfl(wbase, 63);
        int at = wbase + incl - cnt;
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            if ((pend >> j) & 1u) {
                if (at < S.scap) {
                    S.skeys[at] = ((unsigned long long)o[j] << 32) | tg[j];
                    pend &= ~(1u << j);
                }
                at++;
            }
        }
        __syncthreads();
        const int n_after = S.ctl[0];
#ifdef JHQ_PHASE_TIMING
        if (stats && tid == 0) {
            stats[0] += (n_after > S.scap) ? 1 : 0;
            stats[1] += (n_after <= S.scap && n_after > k && 2 * n_after >= S.scap) ? 1 : 0;
            stats[2] += (unsigned long long)n_after;
        }
#endif
        if (n_after > S.scap) {
            // did not fit: prune what is stored, tighten the bound, retry
            stream_prune<NT>(S, S.scap, k);
            const uint32_t T2 = (uint32_t)S.ctl[1];
#pragma unroll
            for (int j = 0; j < CPT; j++)
                if (((pend >> j) & 1u) && o[j] > T2) pend &= ~(1u << j);
            if (!__syncthreads_or(pend != 0u)) break;
        } else {
            if (n_after > k && 2 * n_after >= S.scap) stream_prune<NT>(S, n_after, k);
            break;
        }
    }
}

// Finishes a selection: S.kout[0..kk) sorted ascending; returns kk.
template <int NT>
__device__ __forceinline__ int stream_end(const StreamSel& S, int k) {
    const int n = S.ctl[0];
    const int kk = min(k, n);
    if (kk > 0) select_keys<NT>(S.skeys, n, kk, S.kout, S.kidx, S.ktmp, S.st);
    return kk;
}

static int stream_scap(int k) { return 4 * k < 512 ? 512 : (4 * k + 63) / 64 * 64; }

__host__ __device__ constexpr size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

// LDS bytes of a StreamSel (rounded to 16 so that what follows stays aligned).
static size_t stream_lds_bytes(int NT, int k) {
    return align16((size_t)stream_scap(k) * 8 + (size_t)k * (8 + 8 + 4) +
                   (size_t)(NT / 64) * est_per_wave(k, NT / 64) * 4 + 16 + sizeof(SelState));
}

// Carves a StreamSel out of LDS at p (16-byte aligned); returns the next
// 16-byte aligned address.
template <int NT>
__device__ unsigned char* stream_carve(unsigned char* p, int k, StreamSel* S) {
    S->scap = (4 * k < 512 ? 512 : (4 * k + 63) / 64 * 64);
    S->skeys = (unsigned long long*)p;
    S->kout = S->skeys + S->scap;
    S->ktmp = S->kout + k;
    S->kidx = (int*)(S->ktmp + k);
    S->wstat = (uint32_t*)(S->kidx + k);
    S->ctl = (int*)(S->wstat + (NT / 64) * est_per_wave(k, NT / 64));
    S->st = (SelState*)(S->ctl + 4);
    const size_t used = (size_t)((unsigned char*)(S->st + 1) - p);
    return p + align16(used);
}

// ---------------------------------------------------------------------------
// Probe selection: exact top-P of (score, list) per query, streamed from the
// score row (no nlist-sized LDS array, so any nlist works).  One workgroup
// per query; writes probes[b][P] ascending, gofs[b][P+1] (prefix of the
// probed lists' padded group counts) and qtot[b] = gofs[b][P].
// ---------------------------------------------------------------------------
constexpr int kProbeFastP = 128;   // largest P served by the two-pass path
constexpr int kProbeU = 8;         // float4 loads in flight per thread
constexpr int kProbeSurv = 1024;   // short-list capacity of the two-pass path

// The r-th smallest (1 <= r <= 64) of the wave's 64 lane values, bit by bit
// from the top with ballots.
__device__ __forceinline__ uint32_t wave_kth_u32(uint32_t v, int r) {
    uint32_t res = 0u;
    unsigned long long cand = ~0ull;
    for (int bit = 31; bit >= 0; bit--) {
        const unsigned long long zeros = cand & __ballot(((v >> bit) & 1u) == 0u);
        const int nz = __popcll(zeros);
        if (r <= nz) {
            cand = zeros;
        } else {
            r -= nz;
            cand &= ~zeros;
            res |= 1u << bit;
        }
    }
    return res;
}

// ---------------------------------------------------------------------------
// Integer-MFMA pre-scan: per-query quantization and the batch's list hash
// (written by the probe selection, read by the tile kernel and re-check).
// ---------------------------------------------------------------------------
struct MfmaQS {
    double s, C, e;
    int all, pad;  // all = 1: re-check every candidate
};

typedef int mfma_v4i __attribute__((ext_vector_type(4)));

// hash slots for BP probes: load factor at most 2/3
static int mfma_hash_size(int BP) { return (3 * BP / 2 + 127) / 64 * 64; }

// A group is one probed list and up to 16 of the queries that probe it: the
// MFMA tiles of 16 candidates over the list's slots (a probed list of nl
// vectors fills ceil(nl / 16) 16-slot groups of each probing query's
// candidate row).  The probe selection inserts every (query, probe) pair of
// the batch into a hash of the probed lists (slot h: the list hk[h], its
// size hz[h], its hc[h] pairs by rank in ql); the tile kernel numbers the
// groups slot by slot and, in a slot, by rank (16 pairs to a group), and
// scan wave v takes tiles [v T / W, (v + 1) T / W).  Query b's candidate row
// starts at slot b * perq of the dump.  The re-check clears hk and hc for
// the next batch.  Workspace pieces, 256-byte aligned, in this order.
struct MfmaWs {
    int8_t* qa;  // [B][2][D]: hi then lo bytes in the lanes' register order
    MfmaQS* qs;  // [B]
    int4* hs;    // [H] slot: (list id or -1 when free, pairs in the slot, list size, -)
    int2* ql;    // [H][B] pair of rank r: (query, dump slot of the list's first candidate)
    int H, B, perq;
};

static size_t mfma_carve(int B, int P, int M, unsigned char* base, MfmaWs* w) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int H = mfma_hash_size(B * P);
    size_t off = 0;
    const size_t o_qa = off;
    off += al((size_t)B * 2 * 8 * M);
    const size_t o_qs = off;
    off += al((size_t)B * sizeof(MfmaQS));
    const size_t o_hs = off;
    off += al((size_t)H * sizeof(int4));
    const size_t o_ql = off;
    off += al((size_t)H * B * sizeof(int2));
    if (w) {
        w->qa = (int8_t*)(base + o_qa);
        w->qs = (MfmaQS*)(base + o_qs);
        w->hs = (int4*)(base + o_hs);
        w->ql = (int2*)(base + o_ql);
        w->H = H;
        w->B = B;
        w->perq = 0;
    }
    return off;
}

constexpr int kMfmaMaxBP = 4096;     // (query, probe) pairs per batch (hash <= 64 slots per tile-kernel thread)

// The batch's pre-scan workspace in ws, carved for Bcap queries (the same
// layout for every batch of the workspace, whose hash the previous batch
// cleared), and the dump stride of a query's candidate row (a multiple of
// 16: B rows fit in dump_slots).
static bool mfma_ws(int B, int Bcap, int P, int M, unsigned char* ws, size_t ws_bytes,
                    int64_t dump_slots, MfmaWs* w) {
    if (!ws || ((uintptr_t)ws & 255) || B < 1 || B > Bcap ||
        mfma_carve(Bcap, P, M, ws, w) > ws_bytes)
        return false;
    const int64_t perq = dump_slots / B / 16 * 16;
    if (perq < 16 || perq > (int64_t)1 << 30) return false;
    w->perq = (int)perq;
    return true;
}

// Block sums / max of three doubles (every thread gets the result).
template <int NT>
__device__ __forceinline__ void block_reduce3(double& a, double& b, double& c, double* red) {
    constexpr int NW = NT / 64;
    for (int off = 32; off > 0; off >>= 1) {
        a += __shfl_xor(a, off);
        b += __shfl_xor(b, off);
        c = fmax(c, __shfl_xor(c, off));
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) {
        red[3 * wv] = a;
        red[3 * wv + 1] = b;
        red[3 * wv + 2] = c;
    }
    __syncthreads();
    a = 0.0;
    b = 0.0;
    c = 0.0;
    for (int w2 = 0; w2 < NW; w2++) {
        a += red[3 * w2];
        b += red[3 * w2 + 1];
        c = fmax(c, red[3 * w2 + 2]);
    }
}

// One (query, probe) pair of the batch into the list hash: the list's slot
// (linear probing; the first pair of a list records its size), then the
// pair at its rank in the slot.  The hash has more slots than the batch has
// pairs, so a free or matching slot is always found; the probe count is
// bounded all the same.
__device__ __forceinline__ void mfma_pair_insert(const MfmaWs& w, int l, int sz, int b, int slot0) {
    int h = (int)(((uint64_t)((uint32_t)l * 2654435761u) * (uint32_t)w.H) >> 32);
    bool found = false;
    for (int tries = 0; tries < w.H && !found; tries++) {
        const int old = atomicCAS(&w.hs[h].x, -1, l);
        if (old == -1) w.hs[h].z = sz;
        if (old == -1 || old == l) found = true;
        else h = h + 1 == w.H ? 0 : h + 1;
    }
    if (!found) return;
    const int r = atomicAdd(&w.hs[h].y, 1);
    if (r < w.B) w.ql[(int64_t)h * w.B + r] = make_int2(b, slot0);
}

// What the probe selection does for the pre-scan: the workspace (with the
// dump stride), the rotated queries (read when the selection does not add
// the product's split sums itself) and the primary codebook.
struct MfSel {
    MfmaWs w;
    const float* q_rot;
    const float* c1d;
    int d, M;
};

// The split sums of the query product (mfma_qb_kernel with nsplit > 1, row
// of query b at part + sp * pstride + b * (nrot + nlist) in split sp): added
// in split order, the rotated query stored to C1, the scores kept in LDS.
// QB = nsplit (0: the scores are read from scores).
struct QbPart {
    const float* part;
    int64_t pstride;
    int nrot;
    float* C1;
    int64_t ld1;
    const float* norms;
};

// MF: for the pre-scan, also quantize the query (mf.w.qa, mf.w.qs) and
// insert its (query, probe) pairs into the batch's list hash.
template <int NT, int QB = 0, bool MF = false>
__global__ void __launch_bounds__(NT)
select_probes_kernel(const float* __restrict__ scores, int nlist, int P,
                     const int4* __restrict__ ldesc, int32_t* __restrict__ probes,
                     int32_t* __restrict__ gofs, int32_t* __restrict__ qtot, QbPart qp,
                     MfSel mf) {
    // Fast path (P <= kProbeFastP), two cheap passes over the row:
    //   1. every thread takes the minimum ord(score) of its share; each wave
    //      finds the ceil(P / waves)-th smallest of its 64 lane minima, and
    //      the bound T is the largest of those, so at least P scores are <= T
    //      (each counted lane minimum is one);
    //   2. every score with ord <= T is appended to a short list as the key
    //      (ord << 32 | list); its exact top P is the row's top P.
    // A short list longer than kProbeSurv (many equal scores) falls back to
    // streaming the row through the exact selector.
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NW = NT / 64;
    StreamSel S;
    unsigned char* tail = stream_carve<NT>(smem, P, &S);
    int* gcnt = (int*)tail;
    unsigned long long* surv = (unsigned long long*)(tail + align16((size_t)P * 4));  // [kProbeSurv]
    uint32_t* wth = (uint32_t*)(surv + kProbeSurv);  // [NW]
    int* scnt = (int*)(wth + NW);                    // [1]
    float* srow = (float*)(scnt + 4);                // [nlist] (QB only)
    float* sqr = srow + (QB ? nlist : 0);             // [d] (QB and MF): the rotated query
    int* gsz = (int*)(sqr + (QB && MF ? mf.d : 0));   // [P] (MF): the probed lists' sizes
    // [3 NW] (MF); aligned by offset from smem, not through an integer
    // address, so its loads stay LDS loads
    double* red = (double*)(smem + ((((unsigned char*)(gsz + (MF ? P : 0)) - smem) + 7) & ~(ptrdiff_t)7));
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float* row = QB ? srow : scores + (int64_t)b * nlist;
    JHQ_PHASE_DECL
    stream_begin<NT>(S);
    if (tid == 0) *scnt = 0;
    if constexpr (QB > 0) {
        // the row's split sums and the centroid norms, every float4 requested
        // before the first is added (nrot and nlist multiples of 4)
        constexpr int U = 5;  // one round at D = 1024, nlist 4096
        const int N4 = (qp.nrot + nlist) >> 2, R4 = qp.nrot >> 2;
        const float4* p4 = (const float4*)(qp.part + (int64_t)b * (qp.nrot + nlist));
        const float4* n4 = (const float4*)qp.norms;
        const int64_t st4 = qp.pstride >> 2;
        for (int i0 = tid; i0 < N4; i0 += U * NT) {
            float4 v[U][QB], nw[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
#pragma unroll
                for (int sp = 0; sp < QB; sp++)
                    v[u][sp] = p4[sp * st4 + min(i0 + u * NT, N4 - 1)];
                // (a clamped index where the float4 is the rotated query's)
                nw[u] = n4[min(max(i0 + u * NT - R4, 0), N4 - R4 - 1)];
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = i0 + u * NT;
                if (i >= N4) continue;
                float4 a = v[u][0];
#pragma unroll
                for (int sp = 1; sp < QB; sp++) {
                    a.x += v[u][sp].x;
                    a.y += v[u][sp].y;
                    a.z += v[u][sp].z;
                    a.w += v[u][sp].w;
                }
                if (i < R4) {
                    ((float4*)(qp.C1 + (int64_t)b * qp.ld1))[i] = a;
                    if constexpr (MF) ((float4*)sqr)[i] = a;
                } else {
                    const float4 nv = nw[u];
                    float4 o;
                    o.x = fmaf(-2.0f, a.x, nv.x);
                    o.y = fmaf(-2.0f, a.y, nv.y);
                    o.z = fmaf(-2.0f, a.z, nv.z);
                    o.w = fmaf(-2.0f, a.w, nv.w);
                    ((float4*)srow)[i - R4] = o;
                }
            }
        }
    }
    __syncthreads();
    JHQ_PHASE(0);
    // the pre-scan's sums over the rotated query (C, the sum and the largest
    // of |dl|), before the selection: after it the query's steps are stored
    // beside the pair inserts
    double qC = 0.0, qA = 0.0, qmx = 0.0;
    if constexpr (MF) {
        const float* qrow = QB ? sqr : mf.q_rot + (int64_t)b * mf.d;
        const double c0 = mf.c1d[0], c1 = mf.c1d[1];
        for (int i = tid; i < mf.d; i += NT) {
            const double q = qrow[i];
            const double t0 = q - c0, t1 = q - c1, dl = t1 * t1 - t0 * t0;
            qC += t0 * t0;
            qA += fabs(dl);
            qmx = fmax(qmx, fabs(dl));
        }
        block_reduce3<NT>(qC, qA, qmx, red);
    }
    int kk = 0;
    bool exact = false;
    if (P <= kProbeFastP) {
        const bool vec = (nlist & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0;
        // visits every score of this thread's share: f(ord, list)
        auto visit = [&](auto f) {
            if (vec) {
                const float4* r4 = reinterpret_cast<const float4*>(row);
                const int n4 = nlist >> 2;
                for (int base = 0; base < n4; base += NT * kProbeU) {
                    float4 v[kProbeU];
#pragma unroll
                    for (int u = 0; u < kProbeU; u++) v[u] = r4[min(base + u * NT + tid, n4 - 1)];
#pragma unroll
                    for (int u = 0; u < kProbeU; u++) {
                        const int i = base + u * NT + tid;
                        if (i < n4) {
                            f(f2ord(v[u].x), 4 * i);
                            f(f2ord(v[u].y), 4 * i + 1);
                            f(f2ord(v[u].z), 4 * i + 2);
                            f(f2ord(v[u].w), 4 * i + 3);
                        }
                    }
                }
            } else {
                for (int base = 0; base < nlist; base += NT * kProbeU * 4) {
                    float v[kProbeU * 4];
#pragma unroll
                    for (int u = 0; u < kProbeU * 4; u++) v[u] = row[min(base + u * NT + tid, nlist - 1)];
#pragma unroll
                    for (int u = 0; u < kProbeU * 4; u++) {
                        const int i = base + u * NT + tid;
                        if (i < nlist) f(f2ord(v[u]), i);
                    }
                }
            }
        };
        uint32_t mn = ~0u;
        visit([&](uint32_t o, int) { mn = o < mn ? o : mn; });
        JHQ_PHASE(1);
        const uint32_t tw = wave_kth_u32(mn, (P + NW - 1) / NW);
        if (lane == 0) wth[wv] = tw;
        __syncthreads();
        uint32_t T = 0u;
#pragma unroll
        for (int w = 0; w < NW; w++) T = wth[w] > T ? wth[w] : T;
        JHQ_PHASE(2);
        visit([&](uint32_t o, int i) {
            if (o <= T) {
                const int at = atomicAdd(scnt, 1);
                if (at < kProbeSurv) surv[at] = ((unsigned long long)o << 32) | (uint32_t)i;
            }
        });
        __syncthreads();
        const int ns = *scnt;
        if (ns <= kProbeSurv) {
            rank_select<NT>(surv, ns, P, S.kout);
            kk = P;
            exact = true;
        }
        JHQ_PHASE(3);
    }
    if (!exact) {
        const int rounds = (nlist + NT * 4 - 1) / (NT * 4);
        for (int r = 0; r < rounds; r++) {
            const int i0 = r * NT * 4 + tid * 4;
            uint32_t o[4], tg[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = i0 + j;
                o[j] = i < nlist ? f2ord(row[i]) : ~0u;
                tg[j] = (uint32_t)i;
            }
            stream_round<NT, 4>(S, P, o, tg);
        }
        kk = stream_end<NT>(S, P);
        JHQ_PHASE(5);
    }
    for (int i = tid; i < P; i += NT) {
        const int l = i < kk ? (int)(uint32_t)(S.kout[i] & 0xffffffffull) : 0;
        probes[(int64_t)b * P + i] = l;
        const int sz = i < kk ? ldesc[l].z : 0;
        gcnt[i] = (sz + kGroup - 1) / kGroup;
        if constexpr (MF) gsz[i] = sz;
    }
    __syncthreads();
    // prefix of the group counts (P is small: one wave); for the pre-scan
    // each probe's pair goes to the list hash with its row offset
    if (tid < 64) {
        int carry = 0;
        int32_t* g = gofs + (int64_t)b * (P + 1);
        if (tid == 0) g[0] = 0;
        for (int base = 0; base < P; base += 64) {
            const int i = base + tid;
            const int v = i < P ? gcnt[i] : 0;
            int incl = v;
            for (int off = 1; off < 64; off <<= 1) {
                const int t = __shfl_up(incl, off);
                if (tid >= off) incl += t;
            }
            if (i < P) g[i + 1] = carry + incl;
            if constexpr (MF) {
                if (i < P && i < kk && gsz[i] > 0)
                    mfma_pair_insert(mf.w, (int)(uint32_t)(S.kout[i] & 0xffffffffull), gsz[i], b,
                                     b * mf.w.perq + (carry + incl - v) * kGroup);
            }
            carry += __shfl(incl, 63);
        }
        if (tid == 0) qtot[b] = carry;
    }
    JHQ_PHASE(7);
    if constexpr (MF) {
        // the query's steps for the pre-scan: dl_k = (q_k - c1)^2 - (q_k -
        // c0)^2 rounded to multiples of s = max |dl| / 32000 (int16 as int8
        // hi and lo halves in the MFMA A-operand layout), C = sum (q_k - c0)^2
        // and the bound's slack e, in double
        const int D = mf.d, NK = mf.M / 8, GS = mf.M / 4;
        const float* qrow = QB ? sqr : mf.q_rot + (int64_t)b * D;
        const double c0 = mf.c1d[0], c1 = mf.c1d[1];
        const double sC = qC, sA = qA, mx = qmx;
        const bool fin = isfinite(sC) && isfinite(sA) && sC + sA < 1e36;
        const double st = fin && mx > 0.0 ? mx / 32000.0 : 1.0;
        int8_t* qa = mf.w.qa + (int64_t)b * 2 * D;
        // waves 1 .. NW-1 (all of them when NW = 1), while wave 0 inserts
        const int x0 = NW > 1 ? tid - 64 : tid, xs = NW > 1 ? NT - 64 : NT;
        for (int x = x0 < 0 ? D / 4 : x0; x < D / 4; x += xs) {
            // dimensions 8 m + k of subspaces m = 4 m4 .. 4 m4 + 3: lane
            // group h = m / GS, dword mm / 4 of that group's subspaces,
            // K-step 2 (mm / 4) + k / 4, register k % 4, byte mm % 4
            const int m4 = x >> 3, k = x & 7, m = 4 * m4, h = m / GS, mm = m % GS;
            uint32_t whi = 0u, wlo = 0u;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const double q = qrow[8 * (m + e) + k];
                const double t0 = q - c0, t1 = q - c1, dl = t1 * t1 - t0 * t0;
                const int iq = fin ? (int)rint(dl / st) : 0;
                const int hi = (iq + 128) >> 8, lo = iq - hi * 256;
                whi |= (uint32_t)(uint8_t)(int8_t)hi << (8 * e);
                wlo |= (uint32_t)(uint8_t)(int8_t)lo << (8 * e);
            }
            const int off = h * NK * 16 + (2 * (mm >> 2) + (k >> 2)) * 16 + (k & 3) * 4;
            *(uint32_t*)(qa + off) = whi;
            *(uint32_t*)(qa + D + off) = wlo;
        }
        if (tid == 0) {
            MfmaQS Q;
            Q.s = st;
            Q.C = sC;
            Q.e = 0.5000001 * st * D + 1e-12 * (sC + sA);
            Q.all = fin ? 0 : 1;
            Q.pad = 0;
            mf.w.qs[b] = Q;
        }
    }
    JHQ_PHASE(8);
    JHQ_PHASE_FLUSH(1);
}

// ---------------------------------------------------------------------------
// Work plan of one search batch, computed identically by the scan and the
// refine kernels.  The batch's padded candidate groups are laid end to end in
// query order; workgroup w of G owns groups [w*T/G, (w+1)*T/G).  The groups of
// one query inside one workgroup's range form a segment, which yields one
// top-ck list.  qpre[b] = first group of query b (qpre[B] = T); spre[b] =
// first segment of query b (spre[B] <= G + B - 1).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wg_of_group(int64_t x, int64_t T, int G) {
    return (int)(((x + 1) * G - 1) / T);
}

// Exclusive prefix over B values f(b) into out[0..B] (out[B] = total).
template <int NT, class F>
__device__ __forceinline__ void block_exclusive_scan(F f, int B, int* out, int* wsum) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int per = (B + NT - 1) / NT;
    const int s0 = min(B, tid * per), s1 = min(B, s0 + per);
    int seg = 0;
    for (int b = s0; b < s1; b++) seg += f(b);
    int inc = seg;
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(inc, off);
        if (lane >= off) inc += t;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    int base = 0;
    for (int j = 0; j < w; j++) base += wsum[j];
    int acc = base + inc - seg;
    for (int b = s0; b < s1; b++) {
        const int v = f(b);
        out[b] = acc;
        acc += v;
    }
    if (tid == NT - 1) out[B] = acc;
    __syncthreads();
}

// Two exclusive prefixes at once: out0 / out1[0..n] of f(i).x / f(i).y
// (one pass, one pair of barriers); wsum: 2 * NT / 64 ints.
template <int NT, class F>
__device__ __forceinline__ void block_exclusive_scan2(F f, int n, int* out0, int* out1, int* wsum) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int per = (n + NT - 1) / NT;
    const int s0 = min(n, tid * per), s1 = min(n, s0 + per);
    int a = 0, c = 0;
    for (int i = s0; i < s1; i++) {
        const int2 v = f(i);
        a += v.x;
        c += v.y;
    }
    int ia = a, ic = c;
    for (int off = 1; off < 64; off <<= 1) {
        const int ta = __shfl_up(ia, off), tc = __shfl_up(ic, off);
        if (lane >= off) {
            ia += ta;
            ic += tc;
        }
    }
    if (lane == 63) {
        wsum[w] = ia;
        wsum[NW + w] = ic;
    }
    __syncthreads();
    int xa = ia - a, xc = ic - c;
    for (int j = 0; j < w; j++) {
        xa += wsum[j];
        xc += wsum[NW + j];
    }
    for (int i = s0; i < s1; i++) {
        const int2 v = f(i);
        out0[i] = xa;
        out1[i] = xc;
        xa += v.x;
        xc += v.y;
    }
    if (tid == NT - 1) {
        out0[n] = xa;
        out1[n] = xc;
    }
    __syncthreads();
}

// Each query's span starts with ov virtual groups, which stand for the cost of
// a segment (its LUT build and merge): a workgroup whose range crosses into a
// new query gets that many fewer real groups.  In these units query b spans
// [qpre[b] + b*ov, qpre[b+1] + (b+1)*ov), its real groups the last qtot[b]
// of them, and T = qpre[B] + B*ov.  Returns the number of workgroups that
// take part: min(G, T).
__device__ __forceinline__ int64_t plan_span(const int* qpre, int b, int ov) {
    return (int64_t)qpre[b] + (int64_t)b * ov;
}

template <int NT>
__device__ __forceinline__ int work_plan(const int32_t* __restrict__ qtot, int B, int Gmax, int ov, int* qpre,
                         int* spre, int* wsum) {
    block_exclusive_scan<NT>([&](int b) { return (int)qtot[b]; }, B, qpre, wsum);
    const int64_t T = plan_span(qpre, B, ov);
    const int G = (int)min<int64_t>(Gmax, T);
    block_exclusive_scan<NT>(
        [&](int b) {
            const int64_t a = plan_span(qpre, b, ov) + ov, e = plan_span(qpre, b + 1, ov);
            if (e <= a) return 0;
            return wg_of_group(e - 1, T, G) - wg_of_group(a, T, G) + 1;
        },
        B, spre, wsum);
    return G;
}

// ---------------------------------------------------------------------------
// Byte LUT of one query in LDS (v14/search.cu:65-91):
//   lut[m][v] = sum_k (q[m*Ds+k] - c1d[digit_k(v)])^2, one fma per k, k
// ascending.  A group of NT/M threads shares subspace m with q[m*Ds..] in
// registers.  For 1-bit digits and Ds = 8 the 16 entries that share the low
// 4 bits share the first 4 steps of their fma chain, so each thread finishes
// one low-nibble prefix and expands the high nibble as a binary tree (34
// fmas for 16 entries instead of 128); every entry is still the same chain.
// TR = 1: layout [v][m] (lut[v*M + m]), plus lut[m - M] = lut[255][m] for the
// last 32 subspaces (the skewed scan reads row 255's tail there).
// TR = 2 (M = 128): the skewed scan's parity layout, lut_parity_index().
// ---------------------------------------------------------------------------
// Parity layout of a 128-subspace LUT for the skewed scan (float index from
// the LUT base; the caller reserves 16 floats below it):
//   odd m:  (v, m) at v*64 + m/2                  (table O, 64 KB)
//   even m: (v, m) at kParE + v*64 + m/2          (table E, after a 64-byte gap)
// Row v of either table is 256 bytes, so a lane's LDS address is one byte
// permute of its code byte (v at bits 8-15, the table at bit 16, a lane
// offset in bits 0-7).  Row 255's entries for m = 128 + d (d = -31 .. -1),
// which a wrapped tail byte (v + 1 = 0) reads one row below row 0, are
// copied to (d - 1) / 2 (odd m, below table O) and kParE + d / 2 (even m, in
// the gap).
constexpr int kParE = (65536 + 64) / 4;
__host__ __device__ constexpr int lut_parity_index(int v, int m) {
    return (m & 1 ? 0 : kParE) + v * 64 + (m >> 1);
}
template <int NT, int TR = 0>
__device__ __forceinline__ void build_lut_lds(const float* sq, int M, int Ds, int K1D, int bpd,
                                              const float* sc1d, float* lut) {
    // one entry of the chosen layout (and its wrapped copy)
    auto put = [&](int v, int m, float x) {
        if (TR == 2) {
            lut[lut_parity_index(v, m)] = x;
            if (v == 255 && m >= 97) {
                const int d = m - 128;
                lut[m & 1 ? (d - 1) / 2 : kParE + d / 2] = x;
            }
        } else if (TR == 1) {
            lut[v * M + m] = x;
            if (v == 255 && m >= M - 32) lut[m - M] = x;
        } else {
            lut[m * 256 + v] = x;
        }
    };
    // threads to subspaces: for [m][v] a group of tpm threads shares m (a
    // wave's writes are runs of consecutive v); for the [v][m] layouts
    // consecutive threads take consecutive m (consecutive banks; threads
    // that share m would write one bank, 64 or 128 words apart)
    const int tid = threadIdx.x;
    const bool mfast = TR != 0 && NT >= M;
    const int tpm = mfast ? NT / M : (NT / M > 0 ? NT / M : 1);
    const int part = mfast ? tid / M : tid % tpm;
    const int kmask = K1D - 1;
    for (int m = mfast ? (part < tpm ? tid % M : M) : tid / tpm; m < M;
         m += mfast ? M : NT / tpm) {
        float qv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) qv[k] = k < Ds ? sq[m * Ds + k] : 0.0f;
        if (K1D == 2 && Ds == 8) {
            const float c0 = sc1d[0], c1 = sc1d[1];
            for (int p = part; p < 16; p += tpm) {
                float s4 = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float df = qv[k] - (((p >> k) & 1) ? c1 : c0);
                    s4 = fmaf(df, df, s4);
                }
                float t[16];
                t[0] = s4;
#pragma unroll
                for (int L = 0; L < 4; L++) {
                    const float d0 = qv[4 + L] - c0, d1 = qv[4 + L] - c1;
#pragma unroll
                    for (int i = (1 << L) - 1; i >= 0; i--) {
                        const float base = t[i];
                        t[i | (1 << L)] = fmaf(d1, d1, base);
                        t[i] = fmaf(d0, d0, base);
                    }
                }
#pragma unroll
                for (int h = 0; h < 16; h++) put(p + 16 * h, m, t[h]);
            }
        } else {
            for (int v = part; v < 256; v += tpm) {
                float sacc = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    if (k < Ds) {
                        const float df = qv[k] - sc1d[(v >> (k * bpd)) & kmask];
                        sacc = fmaf(df, df, sacc);
                    }
                }
                put(v, m, sacc);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// IVF ADC scan + exact top-ck per segment (v14/search.cu:105-195 with the
// exact selection of jhq_v3_ivf/search.cu:189-225).
//   - persistent grid, one workgroup per CU, each owning an equal share of
//     the batch's candidate groups (work_plan);
//   - the query's byte LUT lut[m][v] (v14/search.cu:65-91) is built straight
//     into LDS from q_rot;
//   - each thread takes 4 consecutive candidates of one list: per subspace m
//     one 32-bit coalesced load gives their 4 code bytes (SU loads kept in
//     flight), 4 LDS gathers accumulate dist in m order (v14/search.cu:146-151);
//   - the segment's exact top-ck by (dist, stored position) is kept by the
//     streaming selection above -> partial[segment][ck] keys
//     (ord(dist) << 32 | pos), unfilled = ~0.
// ---------------------------------------------------------------------------
constexpr int kScanCPT = 4;  // candidates per thread per round

template <int NT, int SU>
__global__ void __launch_bounds__(NT)
scan_topck_kernel(const float* __restrict__ q_rot, int d, int Ds, int K1D, int bpd,
                  const float* __restrict__ c1d, int M, const int32_t* __restrict__ probes,
                  const int32_t* __restrict__ gofs, const int32_t* __restrict__ qtot, int B, int P,
                  const int4* __restrict__ ldesc, const uint8_t* __restrict__ codes_t, int ck,
                  unsigned long long* __restrict__ partial, int32_t* __restrict__ partial_slot,
                  int ov) {
    constexpr int CPT = kScanCPT, TPG = kGroup / CPT;  // threads per group of 16
    extern __shared__ __align__(16) unsigned char smem[];
    float* lut = (float*)smem;
    StreamSel S;
    float* sq = (float*)stream_carve<NT>(smem + (size_t)M * 256 * 4, ck, &S);  // [d] query
    int* qpre = (int*)(sq + ((d + 3) & ~3));
    int* spre = qpre + B + 1;
    int32_t* sg = spre + B + 1;     // per probe: group prefix [P+1],
    int32_t* spad0 = sg + P + 1;    // block start, block capacity,
    int32_t* snpad = spad0 + P;     // list size, first canonical position
    int32_t* snl = snpad + P;
    int32_t* soff = snl + P;
    float* sc1d = (float*)(soff + P);
    int* wsum = (int*)(sc1d + K1D);

    const int tid = threadIdx.x, w = blockIdx.x;
    JHQ_PHASE_DECL
    for (int i = tid; i < K1D; i += NT) sc1d[i] = c1d[i];
    const int G = work_plan<NT>(qtot, B, gridDim.x, ov, qpre, spre, wsum);
    const int64_t T = plan_span(qpre, B, ov);
    JHQ_PHASE(0);
    if (w >= G) return;
    const int64_t x0 = T * w / G, x1 = T * (w + 1) / G;
    // first query whose groups reach x0
    int b;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (plan_span(qpre, mid, ov) <= x0) lo = mid;
            else hi = mid - 1;
        }
        b = lo;
    }
    for (; b < B && plan_span(qpre, b, ov) < x1; b++) {
        // the query's real groups, in plan units
        const int64_t qb0 = plan_span(qpre, b, ov) + ov, qb1 = plan_span(qpre, b + 1, ov);
        if (qb1 <= qb0 || qb1 <= x0 || qb0 >= x1) continue;
        const int gA = (int)(max(x0, qb0) - qb0), gB = (int)(min(x1, qb1) - qb0);
        const int seg = spre[b] + (w - wg_of_group(qb0, T, G));
        __syncthreads();
        // probe metadata and the query's rotated vector
        for (int i = tid; i <= P; i += NT) sg[i] = gofs[(int64_t)b * (P + 1) + i];
        for (int i = tid; i < P; i += NT) {
            const int4 L = ldesc[probes[(int64_t)b * P + i]];
            spad0[i] = L.x;
            snpad[i] = L.y;
            snl[i] = L.z;
            soff[i] = L.w;
        }
        for (int i = tid; i < d; i += NT) sq[i] = q_rot[(int64_t)b * d + i];
        stream_begin<NT>(S);
        __syncthreads();
        // byte LUT: lut[m][v] = sum_k (q[m*Ds+k] - c1d[digit_k(v)])^2, fma in k order
        build_lut_lds<NT>(sq, M, Ds, K1D, bpd, sc1d, lut);
        __syncthreads();
        JHQ_PHASE(1);

        const int ntask = (gB - gA) * TPG;
        const int rounds = (ntask + NT - 1) / NT;
        for (int r = 0; r < rounds; r++) {
            const int t = r * NT + tid;
            uint32_t o[CPT], tg[CPT];
#pragma unroll
            for (int j = 0; j < CPT; j++) {
                o[j] = ~0u;
                tg[j] = 0u;
            }
            if (t < ntask) {
                const int g = gA + t / TPG, sub = t % TPG;
                int plo = 0, phi = P - 1;  // last p with sg[p] <= g
                while (plo < phi) {
                    const int mid = (plo + phi + 1) >> 1;
                    if (sg[mid] <= g) plo = mid;
                    else phi = mid - 1;
                }
                const int npad = snpad[plo], nl = snl[plo];
                const int c0 = (g - sg[plo]) * kGroup + sub * CPT;
                const uint8_t* base = codes_t + (int64_t)spad0[plo] * M + c0;
                float a[CPT];
#pragma unroll
                for (int j = 0; j < CPT; j++) a[j] = 0.0f;
                // the next SU subspaces' code words are in flight while the
                // current SU are gathered from the LUT
                const int MS = M - M % SU;
                uint32_t wc[SU], wn[SU];
                if (MS > 0) {
#pragma unroll
                    for (int u = 0; u < SU; u++) wc[u] = *(const uint32_t*)(base + (int64_t)u * npad);
                }
                for (int m = 0; m < MS; m += SU) {
                    if (m + SU < MS) {
#pragma unroll
                        for (int u = 0; u < SU; u++)
                            wn[u] = *(const uint32_t*)(base + (int64_t)(m + SU + u) * npad);
                    }
#pragma unroll
                    for (int u = 0; u < SU; u++) {
                        const float* lm = lut + (m + u) * 256;
                        a[0] += lm[wc[u] & 0xffu];
                        a[1] += lm[(wc[u] >> 8) & 0xffu];
                        a[2] += lm[(wc[u] >> 16) & 0xffu];
                        a[3] += lm[wc[u] >> 24];
                    }
#pragma unroll
                    for (int u = 0; u < SU; u++) wc[u] = wn[u];
                }
                for (int m = MS; m < M; m++) {
                    const uint32_t ww = *(const uint32_t*)(base + (int64_t)m * npad);
                    const float* lm = lut + m * 256;
                    a[0] += lm[ww & 0xffu];
                    a[1] += lm[(ww >> 8) & 0xffu];
                    a[2] += lm[(ww >> 16) & 0xffu];
                    a[3] += lm[ww >> 24];
                }
                const uint32_t p0 = (uint32_t)(soff[plo] + c0);
#pragma unroll
                for (int j = 0; j < CPT; j++) {
                    o[j] = (c0 + j < nl) ? f2ord(a[j]) : ~0u;
                    tg[j] = p0 + (uint32_t)j;
                }
            }
#ifdef JHQ_PHASE_TIMING
            __syncthreads();  // attribute the wait for the slowest wave to the scan
#endif
            JHQ_PHASE(2);
            stream_round<NT, CPT>(S, ck, o, tg,
#ifdef JHQ_PHASE_TIMING
                                  ph_acc + 4
#else
                                  nullptr
#endif
            );
            JHQ_PHASE(3);
        }
        const int kk = stream_end<NT>(S, ck);
        unsigned long long* outp = partial + (int64_t)seg * ck;
        int32_t* outs = partial_slot + (int64_t)seg * ck;
        for (int i = tid; i < ck; i += NT) {
            int32_t slot = -1;
            if (i < kk) {
                // pool slot of the survivor: its probe holds canonical
                // positions [soff, soff + snl) at slots [spad0, ...)
                const int tag = (int)(uint32_t)(S.kout[i] & 0xffffffffull);
                for (int p = 0; p < P; p++)
                    if (tag >= soff[p] && tag - soff[p] < snl[p]) slot = spad0[p] + (tag - soff[p]);
            }
            outp[i] = i < kk ? S.kout[i] : ~0ull;
            outs[i] = slot;
        }
        JHQ_PHASE(3);
    }
    JHQ_PHASE_FLUSH(0);
}

// The r-th smallest (1 <= r <= 64 * C) of the wave's 64 * C values, bit by
// bit from the top with ballots.
template <int C>
__device__ __forceinline__ uint32_t wave_kth_u32(const uint32_t (&v)[C], int r) {
    uint32_t res = 0u;
    unsigned long long cand[C];
#pragma unroll
    for (int j = 0; j < C; j++) cand[j] = ~0ull;
    for (int bit = 31; bit >= 0; bit--) {
        unsigned long long z[C];
        int nz = 0;
#pragma unroll
        for (int j = 0; j < C; j++) {
            z[j] = cand[j] & __ballot(((v[j] >> bit) & 1u) == 0u);
            nz += __popcll(z[j]);
        }
        if (r <= nz) {
#pragma unroll
            for (int j = 0; j < C; j++) cand[j] = z[j];
        } else {
            r -= nz;
#pragma unroll
            for (int j = 0; j < C; j++) cand[j] &= ~z[j];
            res |= 1u << bit;
        }
    }
    return res;
}

// lgkmcnt field of an s_waitcnt immediate (4 bits at bit 8)
__host__ __device__ constexpr int lgkm_imm(int n) { return (n < 15 ? n : 15) << 8; }

template <int CPT> struct CodeWord;
template <> struct CodeWord<1> { using type = uint8_t; };
template <> struct CodeWord<2> { using type = uint16_t; };
template <> struct CodeWord<4> { using type = uint32_t; };

// LDS byte address 4 * (byte J of w): one SDWA shift (src1 selects the byte)
// instead of a bit-field extract and a shift-add.
template <int J>
__device__ __forceinline__ uint32_t byte_x4(uint32_t w) {
    uint32_t a;
    if (J == 0)
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(a) : "v"(w));
    else if (J == 1)
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(a) : "v"(w));
    else if (J == 2)
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(a) : "v"(w));
    else
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(a) : "v"(w));
    return a;
}

// ---------------------------------------------------------------------------
// Wave-level exact selection.  buf[0..n) holds distinct keys
// (value << 32 | tag), n <= 64 * J; keeps the k smallest (k < n), compacted
// to buf[0..k) in no particular order, and returns the k-th smallest key's
// value.  The value is found bit by bit with ballots; among keys equal to it,
// the needed number of smallest tags is found the same way.
// ---------------------------------------------------------------------------
// End of a segment: a bound on its ck-th smallest key value tighter than the
// largest wave bound.  Candidates are the waves' bounds wsum[c] (each wave's
// r-th smallest value, ~0 when it holds fewer than r keys); every wave counts
// its own keys at or below each candidate with ballots, and the smallest
// candidate with at least ck keys of the segment at or below it is returned
// (~0 if none).  cnt: NW + 1 ints of LDS, cnt[c] = 0 and cnt[NW] = ~0 since
// the segment began.  All threads call it after the barrier that follows
// every wave's last buffer write.  Segments with waves that hold fewer than r
// keys otherwise merge every kept key (up to ~1000).
// ---------------------------------------------------------------------------
template <int NT, int J>
__device__ __forceinline__ uint32_t tighter_bound(const unsigned long long* wb, int nw,
                                                  const int* wsum, int ck, int* cnt) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63;
    uint32_t v[J];
    bool ok[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int i = j * 64 + lane;
        ok[j] = i < nw;
        v[j] = ok[j] ? (uint32_t)(wb[i] >> 32) : 0u;
    }
    for (int c = 0; c < NW; c++) {
        const uint32_t t = (uint32_t)wsum[c];
        int m = 0;
#pragma unroll
        for (int j = 0; j < J; j++) m += __popcll(__ballot(ok[j] && v[j] <= t));
        if (lane == 0 && m) atomicAdd(&cnt[c], m);
    }
    __syncthreads();
    if ((int)threadIdx.x < NW && cnt[threadIdx.x] >= ck)
        atomicMin((unsigned int*)&cnt[NW], (uint32_t)wsum[threadIdx.x]);
    __syncthreads();
    return (uint32_t)cnt[NW];
}

// ---------------------------------------------------------------------------
template <int J>
__device__ __forceinline__ uint32_t wave_prune(unsigned long long* buf, int n, int k) {
    const int lane = threadIdx.x & 63;
    const unsigned long long lt = (1ull << lane) - 1ull;
    unsigned long long v[J], valid[J], cand[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int i = j * 64 + lane;
        v[j] = i < n ? buf[i] : ~0ull;
        valid[j] = __ballot(i < n);
        cand[j] = valid[j];
    }
    uint32_t V = 0u;
    int r = k;
    for (int bit = 31; bit >= 0; bit--) {
        unsigned long long z[J];
        int nz = 0;
#pragma unroll
        for (int j = 0; j < J; j++) {
            z[j] = cand[j] & __ballot((((uint32_t)(v[j] >> 32) >> bit) & 1u) == 0u);
            nz += __popcll(z[j]);
        }
        if (r <= nz) {
#pragma unroll
            for (int j = 0; j < J; j++) cand[j] = z[j];
        } else {
            r -= nz;
#pragma unroll
            for (int j = 0; j < J; j++) cand[j] &= ~z[j];
            V |= 1u << bit;
        }
    }
    // cand: the keys whose value is V; the r smallest tags among them stay
    int ceq = 0;
#pragma unroll
    for (int j = 0; j < J; j++) ceq += __popcll(cand[j]);
    uint32_t Tt = ~0u;
    if (ceq > r) {
        Tt = 0u;
        for (int bit = 31; bit >= 0; bit--) {
            unsigned long long z[J];
            int nz = 0;
#pragma unroll
            for (int j = 0; j < J; j++) {
                z[j] = cand[j] & __ballot((((uint32_t)v[j] >> bit) & 1u) == 0u);
                nz += __popcll(z[j]);
            }
            if (r <= nz) {
#pragma unroll
                for (int j = 0; j < J; j++) cand[j] = z[j];
            } else {
                r -= nz;
#pragma unroll
                for (int j = 0; j < J; j++) cand[j] &= ~z[j];
                Tt |= 1u << bit;
            }
        }
    }
    int base = 0;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const uint32_t hi = (uint32_t)(v[j] >> 32), lo = (uint32_t)v[j];
        const bool keep = ((valid[j] >> lane) & 1ull) && (hi < V || (hi == V && lo <= Tt));
        const unsigned long long mk = __ballot(keep);
        if (keep) buf[base + __popcll(mk & lt)] = v[j];
        base += __popcll(mk);
    }
    return V;
}

// ---------------------------------------------------------------------------
// ADC scan with wave-independent selection (same work plan, segments,
// arithmetic and output as scan_topck_kernel).  Inside a segment the waves
// take tasks of 16 groups (64 lanes x 4 candidates) from a counter, with no
// workgroup barrier until the segment ends.  Each wave keeps its candidates
// at or below min(own bound, shared bound) in its own LDS buffer; when the
// buffer has no room for another 64 it is pruned to the wave's exact top-ck,
// whose ck-th value becomes the wave's bound and lowers the shared bound (a
// candidate above it has ck smaller candidates in that wave).  At the
// segment's end every wave prunes to ck, the keys at or below the shared
// bound are gathered where the LUT was, and one exact selection emits the
// segment's top-ck.
// ---------------------------------------------------------------------------
template <int NT, int SU, int J>
__global__ void __launch_bounds__(NT)
scan_wave_kernel(const float* __restrict__ q_rot, int d, int Ds, int K1D, int bpd,
                 const float* __restrict__ c1d, int M, const int32_t* __restrict__ probes,
                 const int32_t* __restrict__ gofs, const int32_t* __restrict__ qtot, int B, int P,
                 const int4* __restrict__ ldesc, const uint8_t* __restrict__ codes_t, int ck,
                 int region_bytes, unsigned long long* __restrict__ partial,
                 int32_t* __restrict__ partial_slot, int ov) {
    // wave buffers of 64 * J keys (ck + 64 <= 64 * J)
    constexpr int NW = NT / 64, wcap = 64 * J;
    extern __shared__ __align__(16) unsigned char smem[];
    float* lut = (float*)smem;                                  // or the merge keys
    unsigned long long* merge = (unsigned long long*)smem;
    unsigned long long* wbuf = (unsigned long long*)(smem + region_bytes);  // [NW][wcap]
    unsigned long long* kout =
        wbuf + max((size_t)NW * wcap, (size_t)((d + 3) & ~3) / 2);  // [ck]
    unsigned long long* ktmp = kout + ck;                       // [ck]
    int* kidx = (int*)(ktmp + ck);                              // [ck]
    SelState* st = (SelState*)(kidx + ((ck + 3) & ~3));
    int* ctl = (int*)(st + 1);                                  // Tg, merge count, task counter
    float* sq = (float*)wbuf;  // the query, needed only until the LUT is built
    int* qpre = ctl + 4;
    int* spre = qpre + B + 1;
    int32_t* sg = spre + B + 1;
    int32_t* spad0 = sg + P + 1;
    int32_t* snpad = spad0 + P;
    int32_t* snl = snpad + P;
    int32_t* soff = snl + P;
    float* sc1d = (float*)(soff + P);
    int* wsum = (int*)(sc1d + K1D);

    const int tid = threadIdx.x, w = blockIdx.x, lane = tid & 63, wv = tid >> 6;
    const unsigned long long lt = (1ull << lane) - 1ull;
    unsigned long long* wb = wbuf + (size_t)wv * wcap;
    JHQ_PHASE_DECL
    for (int i = tid; i < K1D; i += NT) sc1d[i] = c1d[i];
    const int G = work_plan<NT>(qtot, B, gridDim.x, ov, qpre, spre, wsum);
    const int64_t T = plan_span(qpre, B, ov);
    JHQ_PHASE(0);
    if (w >= G) return;
    const int64_t x0 = T * w / G, x1 = T * (w + 1) / G;
    int b;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (plan_span(qpre, mid, ov) <= x0) lo = mid;
            else hi = mid - 1;
        }
        b = lo;
    }
    for (; b < B && plan_span(qpre, b, ov) < x1; b++) {
        // the query's real groups, in plan units
        const int64_t qb0 = plan_span(qpre, b, ov) + ov, qb1 = plan_span(qpre, b + 1, ov);
        if (qb1 <= qb0 || qb1 <= x0 || qb0 >= x1) continue;
        const int gA = (int)(max(x0, qb0) - qb0), gB = (int)(min(x1, qb1) - qb0);
        const int seg = spre[b] + (w - wg_of_group(qb0, T, G));
        __syncthreads();
        for (int i = tid; i <= P; i += NT) sg[i] = gofs[(int64_t)b * (P + 1) + i];
        for (int i = tid; i < P; i += NT) {
            const int4 L = ldesc[probes[(int64_t)b * P + i]];
            spad0[i] = L.x;
            snpad[i] = L.y;
            snl[i] = L.z;
            soff[i] = L.w;
        }
        for (int i = tid; i < d; i += NT) sq[i] = q_rot[(int64_t)b * d + i];
        if (tid == 0) {
            ctl[0] = (int)~0u;  // shared bound
            ctl[1] = 0;         // merge count
            ctl[2] = 0;         // next task
        }
        // the end-of-segment bound's counters (ktmp is free until the merge)
        if (2 * ck >= NW + 1)
            for (int i = tid; i <= NW; i += NT) ((int*)ktmp)[i] = i < NW ? 0 : (int)~0u;
        __syncthreads();
        build_lut_lds<NT>(sq, M, Ds, K1D, bpd, sc1d, lut);
        __syncthreads();
        JHQ_PHASE(1);

        int nw = 0;          // keys in this wave's buffer (wave-uniform)
        uint32_t Tw = ~0u;   // this wave's bound
        // one task: groups [g0, g0 + 64 / (16 / C)), C candidates per lane
        auto task = [&](auto cc, int g0) {
            constexpr int C = decltype(cc)::value, TP = kGroup / C;
            using word_t = typename CodeWord<C>::type;
            const int g = g0 + lane / TP, sub = lane % TP;
            uint32_t o[C], tg[C];
#pragma unroll
            for (int j = 0; j < C; j++) {
                o[j] = ~0u;
                tg[j] = 0u;
            }
            if (g < gB) {
                int plo = 0, phi = P - 1;
                while (plo < phi) {
                    const int mid = (plo + phi + 1) >> 1;
                    if (sg[mid] <= g) plo = mid;
                    else phi = mid - 1;
                }
                const int npad = snpad[plo], nl = snl[plo];
                const int c0 = (g - sg[plo]) * kGroup + sub * C;
                const uint8_t* base = codes_t + (int64_t)spad0[plo] * M + c0;
                float a[C];
#pragma unroll
                for (int j = 0; j < C; j++) a[j] = 0.0f;
                using lds_f = const __attribute__((address_space(3))) float;
                using lds_b = const __attribute__((address_space(3))) char;
                // the pipelined gathers of NGR subspaces (one group of C
                // reads each) from code words cw[]: the reads of the next
                // LA groups are issued before a group's adds, so up to
                // (LA + 1) * C reads stay in flight (the LDS counter tracks
                // 15) instead of one wait per read
                constexpr int GR = C, LA = C == 4 ? 2 : (C == 2 ? 6 : 14);
                static_assert((LA + 1) * GR <= 15, "LDS reads in flight");
                auto gathers = [&](auto ngr, const uint32_t* cw, auto fetchg) {
                    constexpr int NGR = decltype(ngr)::value;
                    float rv[LA + 1][GR];
#pragma unroll
                    for (int k = 0; k < LA && k < NGR; k++) fetchg(k, cw[k], rv[k]);
#pragma unroll
                    for (int k = 0; k < NGR; k++) {
                        if (k + LA < NGR) fetchg(k + LA, cw[k + LA], rv[(k + LA) % (LA + 1)]);
                        __builtin_amdgcn_sched_barrier(0);
                        // groups k + 1 .. k + LA may still be in flight
                        switch (k + LA < NGR ? LA : NGR - 1 - k) {
                            // (immediates clamped to the counter's 4 bits; only
                            // cases up to LA are reached)
                            case 14: __builtin_amdgcn_s_waitcnt(0xc07f | lgkm_imm(14 * GR)); break;
                            case 6: __builtin_amdgcn_s_waitcnt(0xc07f | lgkm_imm(6 * GR)); break;
                            case 5: __builtin_amdgcn_s_waitcnt(0xc07f | lgkm_imm(5 * GR)); break;
                            case 4: __builtin_amdgcn_s_waitcnt(0xc07f | lgkm_imm(4 * GR)); break;
                            case 3: __builtin_amdgcn_s_waitcnt(0xc07f | lgkm_imm(3 * GR)); break;
                            case 2: __builtin_amdgcn_s_waitcnt(0xc07f | lgkm_imm(2 * GR)); break;
                            case 1: __builtin_amdgcn_s_waitcnt(0xc07f | lgkm_imm(1 * GR)); break;
                            default: __builtin_amdgcn_s_waitcnt(0xc07f); break;
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int j = 0; j < C; j++) a[j] += rv[k % (LA + 1)][j];
                        __builtin_amdgcn_sched_barrier(0);
                    }
                };
                if (M == 16) {
                    // config 3's code size: all 16 code words in flight at once,
                    // the subspace offsets immediates, the LUT at LDS address 0
                    // (this kernel has no static LDS; the launch checks it), so
                    // a read's address is one SDWA shift of its code byte
                    uint32_t cw[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) cw[u] = *(const word_t*)(base + (int64_t)u * npad);
                    gathers(std::integral_constant<int, 16>(), cw,
                            [&](int k, uint32_t w, float (&dst)[GR]) {
#pragma unroll
                                for (int j = 0; j < C; j++) {
                                    const uint32_t ad = j == 0 ? byte_x4<0>(w)
                                                      : j == 1 ? byte_x4<1>(w)
                                                      : j == 2 ? byte_x4<2>(w) : byte_x4<3>(w);
                                    dst[j] = *(lds_f*)((lds_b*)(uintptr_t)ad + k * 1024);
                                }
                            });
                } else {
                const int MS = M - M % SU;
                uint32_t wc[SU], wn[SU];
                if (MS > 0) {
#pragma unroll
                    for (int u = 0; u < SU; u++) wc[u] = *(const word_t*)(base + (int64_t)u * npad);
                }
                lds_f* lutl = (lds_f*)lut;
                for (int m = 0; m < MS; m += SU) {
                    if (m + SU < MS) {
#pragma unroll
                        for (int u = 0; u < SU; u++)
                            wn[u] = *(const word_t*)(base + (int64_t)(m + SU + u) * npad);
                    }
                    // the block's gathers, one subspace (C reads) per group
                    lds_f* lb = lutl + m * 256;
                    gathers(std::integral_constant<int, SU>(), wc,
                            [&](int k, uint32_t w, float (&dst)[GR]) {
                                lds_f* lm = lb + k * 256;
#pragma unroll
                                for (int j = 0; j < C; j++) dst[j] = lm[(w >> (8 * j)) & 0xffu];
                            });
#pragma unroll
                    for (int u = 0; u < SU; u++) wc[u] = wn[u];
                }
                for (int m = MS; m < M; m++) {
                    const uint32_t ww = *(const word_t*)(base + (int64_t)m * npad);
                    lds_f* lm = lutl + m * 256;
#pragma unroll
                    for (int j = 0; j < C; j++) a[j] += lm[(ww >> (8 * j)) & 0xffu];
                }
                }
                const uint32_t p0 = (uint32_t)(soff[plo] + c0);
#pragma unroll
                for (int j = 0; j < C; j++) {
                    o[j] = (c0 + j < nl) ? f2ord(a[j]) : ~0u;
                    tg[j] = p0 + (uint32_t)j;
                }
            }
            const uint32_t tgs = (uint32_t)ctl[0];
#pragma unroll
            for (int j = 0; j < C; j++) {
                if (nw + 64 > wcap) {
                    Tw = wave_prune<J>(wb, nw, ck);
                    nw = ck;
                    if (lane == 0) atomicMin((unsigned int*)&ctl[0], Tw);
#ifdef JHQ_PHASE_TIMING
                    if (tid == 0) ph_acc[5] += 1;
#endif
                }
                const bool keep = o[j] != ~0u && o[j] <= min(Tw, tgs);
                const unsigned long long mk = __ballot(keep);
                if (keep) wb[nw + __popcll(mk & lt)] = ((unsigned long long)o[j] << 32) | tg[j];
                nw += __popcll(mk);
            }
        };
        // units of 8 groups: a wave takes two (a 4-candidates-per-lane task)
        // while many remain, then one (2 per lane), so the waves finish close
        // together
        const int nunit = (gB - gA + 7) / 8;
        for (;;) {
            int t = 0, take = 1;
            if (lane == 0) {
                const int done = *(volatile __attribute__((address_space(3))) int*)&ctl[2];
                take = nunit - done > 4 * NW ? 2 : 1;
                t = atomicAdd(&ctl[2], take);
            }
            t = __shfl(t, 0);
            take = __shfl(take, 0);
            if (t >= nunit) break;
            if (take == 2 && t + 1 < nunit) {
                task(std::integral_constant<int, 4>(), gA + t * 8);
            } else {
                task(std::integral_constant<int, 2>(), gA + t * 8);
            }
#ifdef JHQ_PHASE_TIMING
            if (tid == 0) ph_acc[4] += 1;
#endif
        }
        if (nw > ck) {
            Tw = wave_prune<J>(wb, nw, ck);
            nw = ck;
            if (lane == 0) atomicMin((unsigned int*)&ctl[0], Tw);
        }
        JHQ_PHASE(6);
        // a tighter bound for the merge: each wave's r-th smallest value, r =
        // ceil(ck / waves); the largest of them has >= ck values at or below it
        {
            const int r = (ck + NW - 1) / NW;
            uint32_t vals[J];
#pragma unroll
            for (int j = 0; j < J; j++) {
                const int i = j * 64 + lane;
                vals[j] = i < nw ? (uint32_t)(wb[i] >> 32) : ~0u;
            }
            const uint32_t tw = nw >= r ? wave_kth_u32<J>(vals, r) : ~0u;
            if (lane == 0) wsum[wv] = (int)tw;
        }
        __syncthreads();  // every wave's tasks are done: the LUT area is free
        JHQ_PHASE(2);
        uint32_t Tf = (uint32_t)ctl[0];
        {
            uint32_t t3 = 0u;
#pragma unroll
            for (int w2 = 0; w2 < NW; w2++) t3 = max(t3, (uint32_t)wsum[w2]);
            Tf = min(Tf, t3);
        }
        if (2 * ck >= NW + 1) Tf = min(Tf, tighter_bound<NT, J>(wb, nw, wsum, ck, (int*)ktmp));
        for (int i0 = 0; i0 < nw; i0 += 64) {
            const int i = i0 + lane;
            const unsigned long long key = i < nw ? wb[i] : ~0ull;
            const bool keep = i < nw && (uint32_t)(key >> 32) <= Tf;
            const unsigned long long mk = __ballot(keep);
            int at = 0;
            if (lane == 0 && mk) at = atomicAdd(&ctl[1], __popcll(mk));
            at = __shfl(at, 0);
            if (keep) merge[at + __popcll(mk & lt)] = key;
        }
        __syncthreads();
        const int n = ctl[1];
        const int kk = min(ck, n);
        if (kk > 0) select_keys<NT>(merge, n, kk, kout, kidx, ktmp, st);
        __syncthreads();
        unsigned long long* outp = partial + (int64_t)seg * ck;
        int32_t* outs = partial_slot + (int64_t)seg * ck;
        for (int i = tid; i < ck; i += NT) {
            int32_t slot = -1;
            if (i < kk) {
                const int tag = (int)(uint32_t)(kout[i] & 0xffffffffull);
                for (int p = 0; p < P; p++)
                    if (tag >= soff[p] && tag - soff[p] < snl[p]) slot = spad0[p] + (tag - soff[p]);
            }
            outp[i] = i < kk ? kout[i] : ~0ull;
            outs[i] = slot;
        }
#ifdef JHQ_PHASE_TIMING
        if (tid == 0) ph_acc[7] += n;
#endif
        JHQ_PHASE(3);
    }
    JHQ_PHASE_FLUSH(0);
}

// bytes below the skewed scan's LUT: row 255's last 32 subspaces
constexpr int kSkewPad = 128;
// chunks of a code row requested ahead of the one being consumed
#ifndef JHQ_PLAN_OV
#define JHQ_PLAN_OV 40000
#endif
#ifndef JHQ_SKEW_D
#define JHQ_SKEW_D 1
#endif
// probe lookup in registers for up to 64 probes (0: always through LDS)
#ifndef JHQ_SKEW_PREG
#define JHQ_SKEW_PREG 1
#endif
// LUT reads per group of steps, and groups of reads in flight ahead of the adds
#ifndef JHQ_SKEW_GS
#define JHQ_SKEW_GS 4
#endif
#ifndef JHQ_SKEW_LA
#define JHQ_SKEW_LA 2
#endif
// ---------------------------------------------------------------------------
// ADC scan with lanes skewed across subspaces (M a multiple of 32, MW = M/4).
// Random byte-LUT gathers conflict on LDS banks when every lane reads the same
// subspace's table.  Here the LUT is laid out [v][m] (bank = m mod 32) and lane
// l runs s = l mod 32 steps behind step t: at step t it adds subspace t - s of
// its candidate, so the 32 lane classes hit 32 different banks.  Each lane
// still adds its candidate's subspaces in ascending order from 0.0f, exactly
// the unskewed sum:
//   - a period is M steps over one candidate per lane (64 per wave: two
//     32-aligned rows of up to two lists, lanes 0-31 and 32-63); at steps
//     t >= s it adds subspaces 0 .. M-1-s of the current candidate, at steps
//     t < s of the NEXT period subspaces M-s .. M-1 of it, then its sum is
//     final (the lane class of candidate i is i mod 32, so it never changes);
//   - the codes come from the skewed copy (row[t] = code[(t - s) mod M]),
//     streamed in 32-byte chunks; the previous row's first chunk stays in
//     registers for the tails.  Its tail bytes hold code + 1, so a tail read
//     (subspace M + t - s of code v) and a head read (subspace t - s) share
//     one address, lane base + byte * 4M + 4t;
//   - which lanes finish a sum at step t < 32 is a lane mask built on the
//     scalar unit (no per-step compares);
//   - after the last period a drain of up to 31 steps finishes the tails;
//   - at M = 128 the LUT is split by subspace parity into two tables of
//     256-byte rows (lut_parity_index), so a gather's LDS address is one byte
//     permute of the code word and a per-lane constant;
//   - up to 64 probes of a segment live across the wave's lanes, so a task's
//     candidate is found without LDS reads; the next task is taken from the
//     counter a period ahead.
// Work plan, segments, wave selection, merge and output are scan_wave_kernel's.
// ---------------------------------------------------------------------------
template <int NT, int MW, int J>
__global__ void __launch_bounds__(NT)
scan_skew_kernel(const float* __restrict__ q_rot, int d, int Ds, int K1D, int bpd,
                 const float* __restrict__ c1d, const int32_t* __restrict__ probes,
                 const int32_t* __restrict__ gofs, const int32_t* __restrict__ qtot, int B, int P,
                 const int4* __restrict__ ldesc, const uint8_t* __restrict__ skew, int ck,
                 int region_bytes, unsigned long long* __restrict__ partial,
                 int32_t* __restrict__ partial_slot, int ov) {
    constexpr int M = MW * 4, NW = NT / 64, wcap = 64 * J;
    extern __shared__ __align__(16) unsigned char smem[];
    // the LUT ([256][M] after kSkewPad bytes that hold row 255's wrapped tail,
    // or at M = 128 the parity layout after 64 bytes), or the merge keys
    constexpr bool PAR = MW == 32;
    float* lut = (float*)(smem + (PAR ? 64 : kSkewPad));
    unsigned long long* merge = (unsigned long long*)smem;
    unsigned long long* wbuf = (unsigned long long*)(smem + region_bytes);  // [NW][wcap]
    unsigned long long* kout =
        wbuf + max((size_t)NW * wcap, (size_t)((d + 3) & ~3) / 2);  // [ck]
    unsigned long long* ktmp = kout + ck;                       // [ck]
    int* kidx = (int*)(ktmp + ck);                              // [ck]
    SelState* st = (SelState*)(kidx + ((ck + 3) & ~3));
    int* ctl = (int*)(st + 1);                                  // Tg, merge count, task counter
    float* sq = (float*)wbuf;  // the query, needed only until the LUT is built
    int* qpre = ctl + 4;
    int* spre = qpre + B + 1;
    int32_t* sg = spre + B + 1;
    int32_t* spad0 = sg + P + 1;
    int32_t* snpad = spad0 + P;
    int32_t* snl = snpad + P;
    int32_t* soff = snl + P;
    int32_t* sru = soff + P;      // [P+1] first row unit of each probe in the segment
    int32_t* sr0 = sru + P + 1;   // [P] first row of each probe in the segment
    float* sc1d = (float*)(sr0 + P);
    int* wsum = (int*)(sc1d + K1D);

    const int tid = threadIdx.x, w = blockIdx.x, lane = tid & 63, wv = tid >> 6;
    const int s = lane & 31;
    const unsigned long long lt = (1ull << lane) - 1ull;
    unsigned long long* wb = wbuf + (size_t)wv * wcap;
    JHQ_PHASE_DECL
    for (int i = tid; i < K1D; i += NT) sc1d[i] = c1d[i];
    const int G = work_plan<NT>(qtot, B, gridDim.x, ov, qpre, spre, wsum);
    const int64_t T = plan_span(qpre, B, ov);
    JHQ_PHASE(0);
    if (w >= G) return;
    const int64_t x0 = T * w / G, x1 = T * (w + 1) / G;
    int b;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (plan_span(qpre, mid, ov) <= x0) lo = mid;
            else hi = mid - 1;
        }
        b = lo;
    }
    for (; b < B && plan_span(qpre, b, ov) < x1; b++) {
        // the query's real groups, in plan units
        const int64_t qb0 = plan_span(qpre, b, ov) + ov, qb1 = plan_span(qpre, b + 1, ov);
        if (qb1 <= qb0 || qb1 <= x0 || qb0 >= x1) continue;
        const int gA = (int)(max(x0, qb0) - qb0), gB = (int)(min(x1, qb1) - qb0);
        const int seg = spre[b] + (w - wg_of_group(qb0, T, G));
        __syncthreads();
        for (int i = tid; i <= P; i += NT) sg[i] = gofs[(int64_t)b * (P + 1) + i];
        for (int i = tid; i < P; i += NT) {
            const int4 L = ldesc[probes[(int64_t)b * P + i]];
            spad0[i] = L.x;
            snpad[i] = L.y;
            snl[i] = L.z;
            soff[i] = L.w;
        }
        for (int i = tid; i < d; i += NT) sq[i] = q_rot[(int64_t)b * d + i];
        if (tid == 0) {
            ctl[0] = (int)~0u;
            ctl[1] = 0;
            ctl[2] = 0;
        }
        // the end-of-segment bound's counters (ktmp is free until the merge)
        if (2 * ck >= NW + 1)
            for (int i = tid; i <= NW; i += NT) ((int*)ktmp)[i] = i < NW ? 0 : (int)~0u;
        __syncthreads();
        // rows (32 candidates) of each probe that meet the segment's groups
        for (int i = tid; i < P; i += NT) {
            const int lo = max(gA, sg[i]), hi = min(gB, sg[i + 1]);
            sr0[i] = lo < hi ? (lo - sg[i]) >> 1 : 0;
        }
        block_exclusive_scan<NT>(
            [&](int i) {
                const int lo = max(gA, sg[i]), hi = min(gB, sg[i + 1]);
                return lo < hi ? ((hi - sg[i] + 1) >> 1) - ((lo - sg[i]) >> 1) : 0;
            },
            P, sru, wsum);
        build_lut_lds<NT, PAR ? 2 : 1>(sq, M, Ds, K1D, bpd, sc1d, lut);
        __syncthreads();
        JHQ_PHASE(1);

        const int nunit = sru[P];
        const int ntask = (nunit + 1) >> 1;
        int nw = 0;
        uint32_t Tw = ~0u;
        // rows are streamed in chunks of 8 words (32 steps), chunk c + D
        // requested while chunk c is consumed; pw keeps the first chunk of the
        // previous row (its tail steps t < s <= 31 read nothing else).  The
        // steps run in groups of GS: the LUT reads of group g + LA are issued
        // before the adds of group g, so at most (LA + 1) * GS read results
        // are live at a time (the compiler would otherwise issue a whole
        // period's reads first and hold all of them in registers).
        constexpr int C = MW / 8, D = C < JHQ_SKEW_D ? C : JHQ_SKEW_D;
        constexpr int GS = JHQ_SKEW_GS, LA = JHQ_SKEW_LA, NG = M / GS;
        static_assert(LA <= 3 && LA * GS <= 15, "reads in flight exceed the LDS counter");
        uint32_t wr[C + D][8], pw[8], tbm[8];
        // tbm[j]: the bytes of word j (steps 4j .. 4j+3) that are tail steps
        // (t < s) of this lane
#pragma unroll
        for (int j = 0; j < 8; j++) {
            pw[j] = 0u;
            const int nt = min(max(s - 4 * j, 0), 4);
            tbm[j] = nt == 4 ? ~0u : (1u << (8 * nt)) - 1u;
        }
        float acc = 0.0f;
        uint32_t ptag = 0u;
        bool pvalid = false;
        const float* lb = lut - s;  // lane base: lut[v*M + m] = lb[v*M + t] with m = t - s
        // tgs: the workgroup bound ctl[0], read a period early (a stale bound
        // only keeps more keys)
        auto append = [&](bool keep, uint32_t o, uint32_t tg, uint32_t tgs) {
            if (nw + 64 > wcap) {
                Tw = wave_prune<J>(wb, nw, ck);
                nw = ck;
                if (lane == 0) atomicMin((unsigned int*)&ctl[0], Tw);
            }
            keep = keep && o <= min(Tw, tgs);
            const unsigned long long mk = __ballot(keep);
            if (keep) wb[nw + __popcll(mk & lt)] = ((unsigned long long)o << 32) | tg;
            nw += __popcll(mk);
        };
        // the lane's candidate of task t: unit u = 2t + half, row r of probe
        // p, the last probe with sru[p] <= u; i = 32 r + s.  Up to 64 probes
        // live in registers, lane p holding probe p's
        //   sru, A = 32 (sr0 - sru), soff + A, spad0 + A, snl - A, sg + A / 16
        // so that i = A + 32u + s needs no LDS round trip: p by ballot,
        // the rest by readlane.  More probes step forward through LDS from the
        // previous one (a wave's tasks increase).
        const bool preg = JHQ_SKEW_PREG && P <= 64;
        int q_sru = 0x7fffffff, q_T = 0, q_S = 0, q_N = 0, q_G = 0;
        if (preg && lane < P) {
            const int A = 32 * (sr0[lane] - sru[lane]);
            q_sru = sru[lane];
            q_T = soff[lane] + A;
            q_S = spad0[lane] + A;
            q_N = snl[lane] - A;
            q_G = sg[lane] + A / 16;
        }
        int pcur = 0;
        auto locate = [&](int t, bool& valid, uint32_t& tag, int64_t& slot) {
            const int u = 2 * t + (lane >> 5);
            valid = false;
            tag = 0u;
            slot = 0;
            if (preg) {
                const int p0 = __popcll(__ballot(q_sru <= 2 * t)) - 1;
                const int p1 = __popcll(__ballot(q_sru <= 2 * t + 1)) - 1;
                // both halves' values (uniform), then a per-lane select
                const int T0 = __builtin_amdgcn_readlane(q_T, p0), T1 = __builtin_amdgcn_readlane(q_T, p1);
                const int S0 = __builtin_amdgcn_readlane(q_S, p0), S1 = __builtin_amdgcn_readlane(q_S, p1);
                const int N0 = __builtin_amdgcn_readlane(q_N, p0), N1 = __builtin_amdgcn_readlane(q_N, p1);
                const int G0 = __builtin_amdgcn_readlane(q_G, p0), G1 = __builtin_amdgcn_readlane(q_G, p1);
                const bool h = lane >= 32;
                const int T = h ? T1 : T0, S = h ? S1 : S0, N = h ? N1 : N0, G = h ? G1 : G0;
                const int iu = 32 * u + s;
                const int gi = G + 2 * u + (s >> 4);
                valid = t < ntask && u < nunit && iu < N && gi >= gA && gi < gB;
                tag = (uint32_t)(T + iu);
                slot = valid ? (int64_t)S + iu : 0;
            } else if (t < ntask && u < nunit) {
                while (pcur + 1 < P && sru[pcur + 1] <= u) pcur++;
                const int plo = pcur;
                const int r = sr0[plo] + (u - sru[plo]);
                const int i = 32 * r + s;
                const int gi = sg[plo] + (i >> 4);
                valid = i < snl[plo] && gi >= gA && gi < gB;
                tag = (uint32_t)(soff[plo] + i);
                slot = valid ? (int64_t)spad0[plo] + i : 0;
            }
        };
        // tasks from a counter (a fixed wv, wv + NW, ... assignment measured 2%
        // slower: the waves do not advance at the same rate)
        auto grab = [&]() {
            int t = 0;
            if (lane == 0) t = atomicAdd(&ctl[2], 1);
            return __builtin_amdgcn_readfirstlane(t);  // lane 0 is active: every lane is
        };
        // a task taken one period before it is needed: the counter's reply
        // arrives while the period runs (read with readfirstlane a period later)
        auto grab_ahead = [&]() {
            // the counter through an opaque LDS pointer: the atomic optimizer
            // (uniform address) would wait for the reply on the spot
            __attribute__((address_space(3))) int* cp = (__attribute__((address_space(3))) int*)(ctl + 2);
            asm volatile("" : "+v"(cp));
            int t = 0;
            if (lane == 0) t = __hip_atomic_fetch_add(cp, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return t;
        };
        auto load_chunk = [&](int64_t slot, int c, uint32_t (&dst)[8]) {
            // pieces 2c and 2c + 1 of the slot's row
            const uint8_t* rp = skew + skew_piece(slot, 2 * c, M);
            const uint4 a = *(const uint4*)rp, b2 = *(const uint4*)(rp + 256);
            dst[0] = a.x; dst[1] = a.y; dst[2] = a.z; dst[3] = a.w;
            dst[4] = b2.x; dst[5] = b2.y; dst[6] = b2.z; dst[7] = b2.w;
        };
        int t = grab();
        int tahead = grab_ahead();
        bool valid;
        uint32_t tag;
        int64_t slot;
        locate(t, valid, tag, slot);
        if (t < ntask) {
#pragma unroll
            for (int c = 0; c < D; c++) load_chunk(slot, c, wr[c]);
        }
        // tasks come from the counter in increasing order per wave, so when
        // t >= ntask the task taken ahead is past the end too
        while (t < ntask) {
            const int tn = __builtin_amdgcn_readfirstlane(tahead);
            tahead = grab_ahead();
            bool nvalid;
            uint32_t ntag;
            int64_t nslot;
            locate(tn, nvalid, ntag, nslot);
            const uint32_t tgs = *(volatile __attribute__((address_space(3))) uint32_t*)ctl;
            const bool more = tn < ntask;
            float fin = 0.0f;
            // Lane mask of the chunk-0 steps, built on the scalar unit: lanes
            // 32h + s with s == t finish their previous candidate at step t
            // (bits t and 32 + t).  The seed is opaque so the masks are
            // rebuilt each period, not hoisted.
            unsigned long long fseed = 0x100000001ull;
            asm volatile("" : "+s"(fseed));
            // byte offset of the lane's LUT base (opaque: not folded into
            // per-step constants)
            using lds_byte = __attribute__((address_space(3))) const char;
            lds_byte* ph = (lds_byte*)lut - 4 * s;
            asm volatile("" : "+v"(ph));
            // parity layout: at step t the lane reads subspace m = t - s of
            // table O (m odd) or E, at byte (O or E) + v*256 + 2m - 2(m&1) from
            // the LUT base.  With d = t - s and q = d & 1 that is
            //   lutbase + 2t + [byte 2: 1 - q][byte 1: v][byte 0: cq],
            //   cq = 64 (1 - q) + 64 - 2s - 2q   (0 .. 128),
            // where lutbase = smem + 64 and the 64-byte gap before E are folded
            // into cq: one byte permute of the lane constant kp[t & 1] and the
            // code word per step.  A tail byte (v + 1) lands on row v's
            // subspace 128 + d the same way (2 * 128 = 256 bytes = one row).
            uint32_t kp[2];
#pragma unroll
            for (int par = 0; par < 2; par++) {
                const int q = par ^ (s & 1);
                kp[par] = ((uint32_t)(1 - q) << 16) | (uint32_t)(64 * (1 - q) + 64 - 2 * s - 2 * q);
            }
            asm volatile("" : "+v"(kp[0]), "+v"(kp[1]));
            // the permute gives the byte address from smem, which is LDS address 0
            // (this kernel has no static LDS; the launch checks it)
            auto par_read = [&](uint32_t w, int tt) {
                const uint32_t a = __builtin_amdgcn_perm(kp[tt & 1], w, 0x0c060004u | ((uint32_t)(tt & 3) << 8));
                return *(const __attribute__((address_space(3))) float*)((lds_byte*)(uintptr_t)a + 2 * tt);
            };
            // LUT reads of steps GS*g .. GS*g+GS-1.  In chunk 0 a lane with
            // t < s reads the previous candidate's subspace M + t - s, its
            // byte raised by one row: the same address formula
            auto fetch = [&](int g, float (&dst)[GS]) {
#pragma unroll
                for (int i = 0; i < GS; i++) {
                    const int tt = GS * g + i, c = tt >> 5, j = (tt >> 2) & 7, e = tt & 3;
                    if (PAR) {
                        uint32_t w = wr[c][j];
                        // chunk 0: the word's tail bytes from the previous row
                        if (c == 0)
                            asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(w) : "v"(tbm[j]), "v"(pw[j]), "v"(wr[0][j]));
                        dst[i] = par_read(w, tt);
                    } else if (c == 0) {
                        // the word's tail bytes from the previous row, the rest from this one
                        uint32_t w;
                        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(w) : "v"(tbm[j]), "v"(pw[j]), "v"(wr[0][j]));
                        uint32_t v = __builtin_amdgcn_ubfe(w, 8 * e, 8);
                        asm("" : "+v"(v));
                        dst[i] = *(const __attribute__((address_space(3))) float*)(
                            ph + v * (4 * M) + 4 * tt);
                    } else {
                        uint32_t v = __builtin_amdgcn_ubfe(wr[c][j], 8 * e, 8);
                        asm("" : "+v"(v));
                        dst[i] = *(const __attribute__((address_space(3))) float*)(
                            ph + v * (4 * M) + 4 * tt);
                    }
                }
            };
            // adds of steps GS*g .. GS*g+GS-1, in step order; at t == s the
            // previous candidate's sum is final and the current one starts from 0
            auto accum = [&](int g, const float (&src)[GS]) {
#pragma unroll
                for (int i = 0; i < GS; i++) {
                    const int tt = GS * g + i;
                    if (tt < 32) {
                        const bool first = __builtin_amdgcn_inverse_ballot_w64(fseed << tt);
                        fin = first ? acc : fin;
                        acc = first ? 0.0f : acc;
                        // selected here: deferred, the 32 selects keep every step's
                        // sum and lane mask live to the end of the period
                        asm volatile("" : "+v"(fin));
                    }
                    acc += src[i];
                }
            };
            // the reads run LA groups ahead of the adds
            float vq[LA + 1][GS];
#pragma unroll
            for (int g = 0; g < LA; g++) fetch(g, vq[g]);
#pragma unroll
            for (int g = 0; g < NG; g++) {
                if ((g * GS) % 32 == 0) {
                    const int c = g * GS / 32 + D;  // chunk to request
                    if (c < C) load_chunk(slot, c, wr[c]);
                    else if (more) load_chunk(nslot, c - C, wr[c]);
                }
                if (g + LA < NG) fetch(g + LA, vq[(g + LA) % (LA + 1)]);
                // one wait for the group's reads: the reads of the next groups
                // (at most LA * GS) may still be in flight
                __builtin_amdgcn_sched_barrier(0);
                switch (g + LA < NG ? LA : NG - 1 - g) {
                    case 3: __builtin_amdgcn_s_waitcnt(0xc07f | (3 * GS) << 8); break;
                    case 2: __builtin_amdgcn_s_waitcnt(0xc07f | (2 * GS) << 8); break;
                    case 1: __builtin_amdgcn_s_waitcnt(0xc07f | (1 * GS) << 8); break;
                    default: __builtin_amdgcn_s_waitcnt(0xc07f); break;
                }
                __builtin_amdgcn_sched_barrier(0);
                accum(g, vq[g % (LA + 1)]);
                asm volatile("" : "+v"(acc));
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) pw[j] = wr[0][j];
#pragma unroll
            for (int c = 0; c < D; c++)
#pragma unroll
                for (int j = 0; j < 8; j++) wr[c][j] = wr[C + c][j];
            append(pvalid, f2ord(fin), ptag, tgs);
            ptag = tag;
            pvalid = valid;
            tag = ntag;
            valid = nvalid;
            slot = nslot;
            t = tn;
        }
        {
            // drain: the tails of the last candidates
            float fin = acc;
            int sv = s;
            asm volatile("" : "+v"(sv));
#pragma unroll
            for (int j = 0; j < 8; j++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int tt = 4 * j + e;
                    // the tail byte is code + 1: row v - 1, subspace M + tt - s
                    if (tt < sv) {
                        if (PAR) {
                            const int q = (tt & 1) ^ (s & 1);
                            const uint32_t k = ((uint32_t)(1 - q) << 16) |
                                               (uint32_t)(64 * (1 - q) + 64 - 2 * s - 2 * q);
                            const uint32_t a = __builtin_amdgcn_perm(k, pw[j], 0x0c060004u | ((uint32_t)e << 8));
                            acc += *(const __attribute__((address_space(3))) float*)(
                                (const __attribute__((address_space(3))) char*)(uintptr_t)a + 2 * tt);
                        } else {
                            acc += lb[((pw[j] >> (8 * e)) & 0xffu) * M + tt];
                        }
                    }
                    if (tt == sv) fin = acc;
                }
            }
            append(pvalid, f2ord(fin), ptag, *(volatile __attribute__((address_space(3))) uint32_t*)ctl);
        }
        if (nw > ck) {
            Tw = wave_prune<J>(wb, nw, ck);
            nw = ck;
            if (lane == 0) atomicMin((unsigned int*)&ctl[0], Tw);
        }
        {
            const int r = (ck + NW - 1) / NW;
            uint32_t vals[J];
#pragma unroll
            for (int j = 0; j < J; j++) {
                const int i = j * 64 + lane;
                vals[j] = i < nw ? (uint32_t)(wb[i] >> 32) : ~0u;
            }
            const uint32_t tw = nw >= r ? wave_kth_u32<J>(vals, r) : ~0u;
            if (lane == 0) wsum[wv] = (int)tw;
        }
        JHQ_PHASE(6);
        __syncthreads();  // every wave's tasks are done: the LUT area is free
        JHQ_PHASE(2);
        uint32_t Tf = (uint32_t)ctl[0];
        {
            uint32_t t3 = 0u;
#pragma unroll
            for (int w2 = 0; w2 < NW; w2++) t3 = max(t3, (uint32_t)wsum[w2]);
            Tf = min(Tf, t3);
        }
        if (2 * ck >= NW + 1) Tf = min(Tf, tighter_bound<NT, J>(wb, nw, wsum, ck, (int*)ktmp));
        for (int i0 = 0; i0 < nw; i0 += 64) {
            const int i = i0 + lane;
            const unsigned long long key = i < nw ? wb[i] : ~0ull;
            const bool keep = i < nw && (uint32_t)(key >> 32) <= Tf;
            const unsigned long long mk = __ballot(keep);
            int at = 0;
            if (lane == 0 && mk) at = atomicAdd(&ctl[1], __popcll(mk));
            at = __shfl(at, 0);
            if (keep) merge[at + __popcll(mk & lt)] = key;
        }
        __syncthreads();
        const int n = ctl[1];
        const int kk = min(ck, n);
        if (kk > 0) select_keys<NT>(merge, n, kk, kout, kidx, ktmp, st);
        __syncthreads();
        unsigned long long* outp = partial + (int64_t)seg * ck;
        int32_t* outs = partial_slot + (int64_t)seg * ck;
        for (int i = tid; i < ck; i += NT) {
            int32_t slot = -1;
            if (i < kk) {
                const int tag = (int)(uint32_t)(kout[i] & 0xffffffffull);
                for (int p = 0; p < P; p++)
                    if (tag >= soff[p] && tag - soff[p] < snl[p]) slot = spad0[p] + (tag - soff[p]);
            }
            outp[i] = i < kk ? kout[i] : ~0ull;
            outs[i] = slot;
        }
#ifdef JHQ_PHASE_TIMING
        if (tid == 0) ph_acc[7] += n;
#endif
        JHQ_PHASE(3);
    }
    JHQ_PHASE_FLUSH(0);
}

// ---------------------------------------------------------------------------
// Large short lists (ck beyond the wave buffers): the scan writes every
// candidate's key (ord(dist) << 32 | canonical position; ~0 for padding) to
// dump[qpre[b] * 16 + group * 16 + i], and select_query_kernel selects each
// query's exact top-ck from them.  Same work plan, LUT and arithmetic as the
// other scans.
// ---------------------------------------------------------------------------
template <int NT, int SU>
__global__ void __launch_bounds__(NT)
scan_dump_kernel(const float* __restrict__ q_rot, int d, int Ds, int K1D, int bpd,
                 const float* __restrict__ c1d, int M, const int32_t* __restrict__ probes,
                 const int32_t* __restrict__ gofs, const int32_t* __restrict__ qtot, int B, int P,
                 const int4* __restrict__ ldesc, const uint8_t* __restrict__ codes_t,
                 unsigned long long* __restrict__ dump, int ov) {
    constexpr int NW = NT / 64;
    extern __shared__ __align__(16) unsigned char smem[];
    float* lut = (float*)smem;
    int* ctl = (int*)(smem + (size_t)M * 256 * 4);  // task counter
    float* sq = (float*)(ctl + 4);
    int* qpre = (int*)(sq + ((d + 3) & ~3));
    int* spre = qpre + B + 1;
    int32_t* sg = spre + B + 1;
    int32_t* spad0 = sg + P + 1;
    int32_t* snpad = spad0 + P;
    int32_t* snl = snpad + P;
    int32_t* soff = snl + P;
    float* sc1d = (float*)(soff + P);
    int* wsum = (int*)(sc1d + K1D);

    const int tid = threadIdx.x, w = blockIdx.x, lane = tid & 63;
    for (int i = tid; i < K1D; i += NT) sc1d[i] = c1d[i];
    const int G = work_plan<NT>(qtot, B, gridDim.x, ov, qpre, spre, wsum);
    const int64_t T = plan_span(qpre, B, ov);
    if (w >= G) return;
    const int64_t x0 = T * w / G, x1 = T * (w + 1) / G;
    int b;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (plan_span(qpre, mid, ov) <= x0) lo = mid;
            else hi = mid - 1;
        }
        b = lo;
    }
    for (; b < B && plan_span(qpre, b, ov) < x1; b++) {
        // the query's real groups, in plan units
        const int64_t qb0 = plan_span(qpre, b, ov) + ov, qb1 = plan_span(qpre, b + 1, ov);
        if (qb1 <= qb0 || qb1 <= x0 || qb0 >= x1) continue;
        const int gA = (int)(max(x0, qb0) - qb0), gB = (int)(min(x1, qb1) - qb0);
        __syncthreads();
        for (int i = tid; i <= P; i += NT) sg[i] = gofs[(int64_t)b * (P + 1) + i];
        for (int i = tid; i < P; i += NT) {
            const int4 L = ldesc[probes[(int64_t)b * P + i]];
            spad0[i] = L.x;
            snpad[i] = L.y;
            snl[i] = L.z;
            soff[i] = L.w;
        }
        for (int i = tid; i < d; i += NT) sq[i] = q_rot[(int64_t)b * d + i];
        if (tid == 0) ctl[0] = 0;
        __syncthreads();
        build_lut_lds<NT>(sq, M, Ds, K1D, bpd, sc1d, lut);
        __syncthreads();
        unsigned long long* qd = dump + (int64_t)qpre[b] * kGroup;  // real groups of query b
        auto task = [&](auto cc, int g0) {
            constexpr int C = decltype(cc)::value, TP = kGroup / C;
            using word_t = typename CodeWord<C>::type;
            const int g = g0 + lane / TP, sub = lane % TP;
            if (g >= gB) return;
            int plo = 0, phi = P - 1;
            while (plo < phi) {
                const int mid = (plo + phi + 1) >> 1;
                if (sg[mid] <= g) plo = mid;
                else phi = mid - 1;
            }
            const int npad = snpad[plo], nl = snl[plo];
            const int c0 = (g - sg[plo]) * kGroup + sub * C;
            const uint8_t* base = codes_t + (int64_t)spad0[plo] * M + c0;
            float a[C];
#pragma unroll
            for (int j = 0; j < C; j++) a[j] = 0.0f;
            const int MS = M - M % SU;
            uint32_t wc[SU], wn[SU];
            if (MS > 0) {
#pragma unroll
                for (int u = 0; u < SU; u++) wc[u] = *(const word_t*)(base + (int64_t)u * npad);
            }
            for (int m = 0; m < MS; m += SU) {
                if (m + SU < MS) {
#pragma unroll
                    for (int u = 0; u < SU; u++)
                        wn[u] = *(const word_t*)(base + (int64_t)(m + SU + u) * npad);
                }
#pragma unroll
                for (int u = 0; u < SU; u++) {
                    const float* lm = lut + (m + u) * 256;
#pragma unroll
                    for (int j = 0; j < C; j++) a[j] += lm[(wc[u] >> (8 * j)) & 0xffu];
                }
#pragma unroll
                for (int u = 0; u < SU; u++) wc[u] = wn[u];
            }
            for (int m = MS; m < M; m++) {
                const uint32_t ww = *(const word_t*)(base + (int64_t)m * npad);
                const float* lm = lut + m * 256;
#pragma unroll
                for (int j = 0; j < C; j++) a[j] += lm[(ww >> (8 * j)) & 0xffu];
            }
            const uint32_t p0 = (uint32_t)(soff[plo] + c0);
            unsigned long long* out = qd + (int64_t)g * kGroup + sub * C;
#pragma unroll
            for (int j = 0; j < C; j++)
                out[j] = (c0 + j < nl) ? (((unsigned long long)f2ord(a[j]) << 32) | (p0 + j))
                                       : ~0ull;
        };
        const int nunit = (gB - gA + 7) / 8;
        for (;;) {
            int t = 0, take = 1;
            if (lane == 0) {
                const int done = *(volatile int*)&ctl[0];
                take = nunit - done > 4 * NW ? 2 : 1;
                t = atomicAdd(&ctl[0], take);
            }
            t = __shfl(t, 0);
            take = __shfl(take, 0);
            if (t >= nunit) break;
            if (take == 2 && t + 1 < nunit) task(std::integral_constant<int, 4>(), gA + t * 8);
            else task(std::integral_constant<int, 2>(), gA + t * 8);
        }
    }
}

// Exact top-ck of each query's dumped keys (one workgroup per query), written
// as the query's first segment list (sorted, ~0 padded) with pool slots; the
// query's other segment lists are left empty.  Two passes: every thread takes
// the minimum value of its share, the largest of the waves' ceil(ck / waves)-th
// smallest lane minima bounds the ck-th smallest value, the keys at or below
// it are gathered and selected exactly.  Too many (equal values) falls back to
// streaming every key through the exact selector.
constexpr int kDumpSurv = 8192;

template <int NT>
__global__ void __launch_bounds__(NT)
select_query_kernel(const unsigned long long* __restrict__ dump, const int32_t* __restrict__ qtot,
                    int B, int Gmax, int ck, const int32_t* __restrict__ probes, int P,
                    const int4* __restrict__ ldesc, unsigned long long* __restrict__ partial,
                    int32_t* __restrict__ partial_slot, int ov) {
    constexpr int NW = NT / 64;
    extern __shared__ __align__(16) unsigned char smem[];
    StreamSel S;
    unsigned char* p = stream_carve<NT>(smem, ck, &S);
    unsigned long long* surv = (unsigned long long*)p;  // [kDumpSurv]
    int* qpre = (int*)(surv + kDumpSurv);
    int* spre = qpre + B + 1;
    int* wsum = spre + B + 1;                            // [NW]
    int* meta = wsum + NW;                               // [3P]: start, size, first position
    int* scnt = meta + 3 * P;
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const unsigned long long lt = (1ull << lane) - 1ull;
    work_plan<NT>(qtot, B, Gmax, ov, qpre, spre, wsum);
    for (int i = tid; i < P; i += NT) {
        const int4 L = ldesc[probes[(int64_t)b * P + i]];
        meta[3 * i] = L.x;
        meta[3 * i + 1] = L.z;
        meta[3 * i + 2] = L.w;
    }
    if (tid == 0) *scnt = 0;
    stream_begin<NT>(S);
    __syncthreads();
    const int64_t n = (int64_t)(qpre[b + 1] - qpre[b]) * kGroup;
    const unsigned long long* keys = dump + (int64_t)qpre[b] * kGroup;
    uint32_t mn = ~0u;
    for (int64_t i = tid; i < n; i += NT) mn = min(mn, (uint32_t)(keys[i] >> 32));
    const int r = (ck + NW - 1) / NW;
    uint32_t mv[1] = {mn};
    const uint32_t tw = r <= 64 ? wave_kth_u32<1>(mv, r) : ~0u;
    if (lane == 0) wsum[wv] = (int)tw;
    __syncthreads();
    uint32_t T = 0u;
#pragma unroll
    for (int w2 = 0; w2 < NW; w2++) T = max(T, (uint32_t)wsum[w2]);
    for (int64_t i0 = 0; i0 < n; i0 += NT) {
        const int64_t i = i0 + tid;
        const unsigned long long x = i < n ? keys[i] : ~0ull;
        const bool keep = x != ~0ull && (uint32_t)(x >> 32) <= T;
        const unsigned long long mk = __ballot(keep);
        int at = 0;
        if (lane == 0 && mk) at = atomicAdd(scnt, __popcll(mk));
        at = __shfl(at, 0);
        if (keep && at + __popcll(mk & lt) < kDumpSurv) surv[at + __popcll(mk & lt)] = x;
    }
    __syncthreads();
    const int ns = *scnt;
    int kk = 0;
    if (ns <= kDumpSurv) {
        kk = min(ck, ns);
        if (kk > 0) select_keys<NT>(surv, ns, kk, S.kout, S.kidx, S.ktmp, S.st);
    } else {
        for (int64_t r0 = 0; r0 < n; r0 += (int64_t)NT * 4) {
            uint32_t o[4], tg[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int64_t i = r0 + (int64_t)tid * 4 + j;
                const unsigned long long x = i < n ? keys[i] : ~0ull;
                o[j] = (uint32_t)(x >> 32);
                tg[j] = (uint32_t)x;
            }
            stream_round<NT, 4>(S, ck, o, tg);
        }
        kk = stream_end<NT>(S, ck);
    }
    __syncthreads();
    const int s0 = spre[b], s1 = spre[b + 1];
    for (int i = tid; i < ck; i += NT) {
        int32_t slot = -1;
        if (i < kk) {
            const int tag = (int)(uint32_t)(S.kout[i] & 0xffffffffull);
            for (int q = 0; q < P; q++)
                if (tag >= meta[3 * q + 2] && tag - meta[3 * q + 2] < meta[3 * q + 1])
                    slot = meta[3 * q] + (tag - meta[3 * q + 2]);
        }
        partial[(int64_t)s0 * ck + i] = i < kk ? S.kout[i] : ~0ull;
        partial_slot[(int64_t)s0 * ck + i] = slot;
    }
    for (int64_t i = (int64_t)(s0 + 1) * ck + tid; i < (int64_t)s1 * ck; i += NT) {
        partial[i] = ~0ull;
        partial_slot[i] = -1;
    }
}

// Allows `kernel` the LDS left after its static allocation; returns the
// largest dynamic LDS size it may be launched with (0 on failure).
static int static_lds(const void* kernel) {
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, kernel) != hipSuccess) return -1;
    return (int)fa.sharedSizeBytes;
}

static int allow_max_lds(const void* kernel) {
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, kernel) != hipSuccess) return 0;
    const int dyn = kLdsBytes - (int)fa.sharedSizeBytes;
    if (dyn <= 0) return 0;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, dyn) != hipSuccess)
        return 0;
    return dyn;
}

constexpr int kScanNT = JHQ_SCAN_NT;
// 12 waves, three per SIMD: the loop's ~150 registers fit (at most 168 at three
// waves per SIMD) and a third wave hides more of the LDS latency than two (8
// waves: 467 K against 493 K queries/s at config 2; 16 waves spill)
#ifndef JHQ_SKEW_NT
#define JHQ_SKEW_NT 768
#endif
constexpr int kSkewNT = JHQ_SKEW_NT;
// 1024 threads per query: 64 candidates' residuals per round (512: 27.5 us
// against 23.0 us per batch of 64 at config 2)
#ifndef JHQ_REFINE_NT
#define JHQ_REFINE_NT 1024
#endif
constexpr int kRefineNT = JHQ_REFINE_NT;
constexpr int kProbeNT = 512, kProbeSmallNT = 256;
constexpr int kProbeFuseMaxList = 8192;  // score rows the selection holds in LDS


// LDS of the wave-selection scan with wave buffers of 64 * J keys.
static size_t scan_wave_lds(int NT, int M, int d, int P, int ck, int K1D, int B, int J,
                            size_t* region, int lut_pad = 0) {
    const int NW = NT / 64;
    *region = align16(std::max((size_t)lut_pad + (size_t)M * 256 * 4, (size_t)NW * ck * 8));
    // the query vector shares the wave buffers
    const size_t wb = std::max((size_t)NW * 64 * J * 8, (size_t)((d + 3) & ~3) * 4);
    return *region + wb + (size_t)ck * 16 + (size_t)((ck + 3) & ~3) * 4 +
           align16(sizeof(SelState)) + 16 + (size_t)(2 * (B + 1) + (P + 1) + 4 * P) * 4 +
           (size_t)K1D * 4 + NW * 4 + 64;
}

static size_t mfma_recheck_lds(int M, int d, int P, int ck, int K1D, int B, int rck);
bool scan_plan(int M, int d, int P, int ck, int K1D, int B, int target_wg, ScanShape* out,
               bool skew, bool mfma, int rck) {
    out->mfma = 0;
    if (mfma) {
        // integer-MFMA pre-scan and one exact re-check per query: one
        // segment per query (the caller checked mfma_scan_ok)
        out->G = 1;
        out->ov = 0;
        out->max_segments = B;
        out->wave = 0;
        out->skew = 0;
        out->dump = 0;
        out->mfma = 1;
        out->nt = 1024;
        out->lds = (int)mfma_recheck_lds(M, d, P, ck, K1D, B, rck);
        out->region = 0;
        return true;
    }
    out->G = target_wg;
    out->max_segments = target_wg + B;
    // a segment (its LUT build, merge and first loads of a new query's lists)
    // costs about as much as JHQ_PLAN_OV / M groups of the scan: 312 groups at
    // M = 128 (12-wave skewed scan; of 86 / 125 / 172 / 234 / 312 / 390 / 507
    // at config 2 the larger weights run the scan faster, and 312 keeps the
    // alpha = 4 pipeline at its best)
    out->ov = std::max(0, JHQ_PLAN_OV / std::max(M, 1));
    out->skew = 0;
    const int need = ck + 64;
    const int J = need <= 128 ? 2 : need <= 192 ? 3 : need <= 256 ? 4 : need <= 384 ? 6
                : need <= 512 ? 8 : 0;
    out->dump = 0;
    // lanes skewed across subspaces (M a multiple of 32, at most 128), short
    // lists up to 128.  Longer ones take the dump path below: with ck = 400
    // (config 5) the skewed scan's 512-key wave buffers prune too often and
    // it is slower (1124 against 872 us per batch of 128)
    if (J && J <= 3 && skew && M % 32 == 0 && M <= 128) {
        size_t region = 0;
        const size_t lds = scan_wave_lds(kSkewNT, M, d, P, ck, K1D, B, J, &region, kSkewPad) +
                           (size_t)(2 * P + 1) * 4;
        if (lds <= (size_t)kLdsBytes - 1024) {
            out->wave = J;
            out->skew = M / 4;
            out->nt = kSkewNT;
            out->lds = (int)lds;
            out->region = (int)region;
            return true;
        }
    }
    // short lists up to 128: selection inside the scan, 16 waves per workgroup
    if (J && J <= 3) {
        size_t region = 0;
        const size_t lds = scan_wave_lds(kScanNT, M, d, P, ck, K1D, B, J, &region);
        if (lds <= (size_t)kLdsBytes - 1024) {
            out->wave = J;
            out->nt = kScanNT;
            out->lds = (int)lds;
            out->region = (int)region;
            return true;
        }
    }
    // longer ones: every distance to HBM, then one exact selection per query
    {
        const size_t lds = (size_t)M * 256 * 4 + 16 + (size_t)((d + 3) & ~3) * 4 +
                           (size_t)(2 * (B + 1) + (P + 1) + 4 * P) * 4 + (size_t)K1D * 4 +
                           (kScanNT / 64) * 4 + 64;
        const size_t lds2 = stream_lds_bytes(kScanNT, ck) + (size_t)kDumpSurv * 8 +
                            (size_t)(2 * (B + 1)) * 4 + (kScanNT / 64) * 4 + (size_t)P * 12 + 32;
        if (lds <= (size_t)kLdsBytes - 1024 && lds2 <= (size_t)kLdsBytes - 1024) {
            out->dump = 1;
            out->wave = 0;
            out->nt = kScanNT;
            out->lds = (int)lds;
            out->region = (int)lds2;
            return true;
        }
    }
    // 16 waves per workgroup if the LDS allows, else 8 (large ck)
    for (int nt = kScanNT; J && nt >= 512; nt /= 2) {
        size_t region = 0;
        const size_t lds = scan_wave_lds(nt, M, d, P, ck, K1D, B, J, &region);
        if (lds <= (size_t)kLdsBytes - 1024) {
            out->wave = J;
            out->nt = nt;
            out->lds = (int)lds;
            out->region = (int)region;
            return true;
        }
    }
    const size_t lds = (size_t)M * 256 * 4 + stream_lds_bytes(kScanNT, ck) +
                       (size_t)((d + 3) & ~3) * 4 + (size_t)(2 * (B + 1) + (P + 1) + 4 * P) * 4 +
                       (size_t)K1D * 4 + (kScanNT / 64) * 4 + 64;
    if (lds > (size_t)kLdsBytes - 1024) return false;
    out->wave = 0;
    out->nt = kScanNT;
    out->lds = (int)lds;
    out->region = 0;
    return true;
}

template <int NT, int QB = 0, bool MF = false>
static hipError_t launch_select_probes(const float* scores, int B, int nlist, int P,
                                       const int4* ldesc, int32_t* probes, int32_t* gofs,
                                       int32_t* qtot, const QbPart& qp, const MfSel& mf,
                                       hipStream_t s) {
    const size_t lds = stream_lds_bytes(NT, P) + align16((size_t)P * 4) +
                       (size_t)kProbeSurv * 8 + (size_t)(NT / 64) * 4 + 16 +
                       (QB ? (size_t)nlist * 4 + 16 : 0) +
                       (MF ? (size_t)(QB ? mf.d : 0) * 4 + (size_t)P * 4 + 8 +
                                 (size_t)3 * (NT / 64) * 8
                           : 0);
    static const int max_dyn = allow_max_lds((const void*)select_probes_kernel<NT, QB, MF>);
    if ((int)lds > max_dyn) return hipErrorInvalidValue;
    hipLaunchKernelGGL((select_probes_kernel<NT, QB, MF>), dim3(B), dim3(NT), lds, s, scores,
                       nlist, P, ldesc, probes, gofs, qtot, qp, mf);
    return hipGetLastError();
}

// The pre-scan's part of the selection (ps set): its workspace, with the
// dump stride, and the checks the quantization needs.
static hipError_t prescan_sel(const PrescanSel* ps, int B, int P, MfSel* mf) {
    if (!ps) return hipSuccess;
    if (!ps->c1d || ps->d != 8 * ps->M || (int64_t)ps->Bcap * P > kMfmaMaxBP ||
        !mfma_ws(B, ps->Bcap, P, ps->M, ps->ws, ps->ws_bytes, ps->dump_slots, &mf->w))
        return hipErrorInvalidValue;
    mf->q_rot = ps->q_rot;
    mf->c1d = ps->c1d;
    mf->d = ps->d;
    mf->M = ps->M;
    return hipSuccess;
}

hipError_t select_probes(const float* scores, int B, int nlist, int P, const int4* ldesc,
                         int32_t* probes, int32_t* gofs, int32_t* qtot, hipStream_t s,
                         const PrescanSel* ps) {
    // short score rows: 4 waves per query (10.8 against 11.7 us per batch of
    // 64 at nlist 4096 with 8 waves; 16 waves 13.8)
    const QbPart none{};
    MfSel mf{};
    const hipError_t e = prescan_sel(ps, B, P, &mf);
    if (e != hipSuccess) return e;
    if (ps && !ps->q_rot) return hipErrorInvalidValue;
    if (nlist <= 8192)
        return ps ? launch_select_probes<kProbeSmallNT, 0, true>(scores, B, nlist, P, ldesc, probes,
                                                                 gofs, qtot, none, mf, s)
                  : launch_select_probes<kProbeSmallNT>(scores, B, nlist, P, ldesc, probes, gofs,
                                                        qtot, none, mf, s);
    return ps ? launch_select_probes<kProbeNT, 0, true>(scores, B, nlist, P, ldesc, probes, gofs,
                                                        qtot, none, mf, s)
              : launch_select_probes<kProbeNT>(scores, B, nlist, P, ldesc, probes, gofs, qtot, none,
                                               mf, s);
}

bool select_adds_qb(const QbPlan& p, int nlist, int nrot) {
    return p.nsplit >= 2 && p.nsplit <= 4 && nlist <= kProbeFuseMaxList && nlist % 4 == 0 &&
           nrot % 4 == 0;
}

hipError_t select_probes_qb(const QbPlan& p, const float* part, int nrot, float* C1, int64_t ld1,
                            const float* norms, int B, int nlist, int P, const int4* ldesc,
                            int32_t* probes, int32_t* gofs, int32_t* qtot, hipStream_t s,
                            const PrescanSel* ps) {
    if (!select_adds_qb(p, nlist, nrot) || ((uintptr_t)part & 15) || ((uintptr_t)C1 & 15) ||
        ((uintptr_t)norms & 15) || ld1 % 4 != 0 || B > p.R * 64)
        return hipErrorInvalidValue;
    const QbPart qp{part, qb_part_stride(p, nrot + nlist), nrot, C1, ld1, norms};
    MfSel mf{};
    const hipError_t e = prescan_sel(ps, B, P, &mf);
    if (e != hipSuccess) return e;
    if (ps && ps->d != nrot) return hipErrorInvalidValue;
#define JHQ_SELQB(NS)                                                                          \
    return ps ? launch_select_probes<kProbeSmallNT, NS, true>(nullptr, B, nlist, P, ldesc, probes, \
                                                              gofs, qtot, qp, mf, s)           \
              : launch_select_probes<kProbeSmallNT, NS>(nullptr, B, nlist, P, ldesc, probes, gofs, \
                                                        qtot, qp, mf, s);
    switch (p.nsplit) {
        case 2: JHQ_SELQB(2)
        case 3: JHQ_SELQB(3)
        default: JHQ_SELQB(4)
    }
#undef JHQ_SELQB
}

hipError_t scan_topck(const float* q_rot, int d, int Ds, int K1D, int bpd, const float* c1d,
                      int B, int M, const int32_t* probes, const int32_t* gofs,
                      const int32_t* qtot, int P, const int4* ldesc, const uint8_t* codes_t,
                      int ck, const ScanShape& sh, unsigned long long* partial,
                      int32_t* partial_slot, unsigned long long* dump, const uint8_t* skew,
                      hipStream_t s) {
    constexpr int NT = kScanNT, SU = JHQ_SCAN_SU;
    if (Ds > 8 || K1D > 256) return hipErrorInvalidValue;
    if (sh.skew) {
        using KFn = void (*)(const float*, int, int, int, int, const float*, const int32_t*,
                             const int32_t*, const int32_t*, int, int, const int4*,
                             const uint8_t*, int, int, unsigned long long*, int32_t*, int);
        constexpr int NS = kSkewNT;
        static const KFn kf[4][2] = {
            {scan_skew_kernel<NS, 8, 2>, scan_skew_kernel<NS, 8, 3>},
            {scan_skew_kernel<NS, 16, 2>, scan_skew_kernel<NS, 16, 3>},
            {scan_skew_kernel<NS, 24, 2>, scan_skew_kernel<NS, 24, 3>},
            {scan_skew_kernel<NS, 32, 2>, scan_skew_kernel<NS, 32, 3>}};
        static int mx[4][2] = {{-1, -1}, {-1, -1}, {-1, -1}, {-1, -1}};
        const int mi = sh.skew / 8 - 1, ji = sh.wave - 2;
        if (!skew || mi < 0 || mi > 3 || ji < 0 || ji > 1 || sh.skew * 4 != M)
            return hipErrorInvalidValue;
        if (mx[mi][ji] < 0) {
            mx[mi][ji] = allow_max_lds((const void*)kf[mi][ji]);
            // M = 128 addresses its LUT from LDS address 0: no static LDS
            if (mi == 3 && static_lds((const void*)kf[mi][ji]) != 0) mx[mi][ji] = 0;
        }
        if (sh.lds > mx[mi][ji]) return hipErrorInvalidValue;
        hipLaunchKernelGGL(kf[mi][ji], dim3(sh.G), dim3(NS), sh.lds, s, q_rot, d, Ds, K1D, bpd,
                           c1d, probes, gofs, qtot, B, P, ldesc, skew, ck, sh.region, partial,
                           partial_slot, sh.ov);
        return hipGetLastError();
    }
    if (sh.dump) {
        static const int mxd = allow_max_lds((const void*)scan_dump_kernel<NT, SU>);
        static const int mxs = allow_max_lds((const void*)select_query_kernel<NT>);
        if (!dump || sh.lds > mxd || sh.region > mxs) return hipErrorInvalidValue;
        hipLaunchKernelGGL((scan_dump_kernel<NT, SU>), dim3(sh.G), dim3(NT), sh.lds, s, q_rot, d,
                           Ds, K1D, bpd, c1d, M, probes, gofs, qtot, B, P, ldesc, codes_t, dump,
                           sh.ov);
        hipLaunchKernelGGL(select_query_kernel<NT>, dim3(B), dim3(NT), sh.region, s,
                           (const unsigned long long*)dump, qtot, B, sh.G, ck, probes, P, ldesc,
                           partial, partial_slot, sh.ov);
        return hipGetLastError();
    }
    if (sh.wave) {
        using KFn = void (*)(const float*, int, int, int, int, const float*, int, const int32_t*,
                             const int32_t*, const int32_t*, int, int, const int4*, const uint8_t*,
                             int, int, unsigned long long*, int32_t*, int);
        static const KFn kf[2][5] = {
            {scan_wave_kernel<NT, SU, 2>, scan_wave_kernel<NT, SU, 3>, scan_wave_kernel<NT, SU, 4>,
             scan_wave_kernel<NT, SU, 6>, scan_wave_kernel<NT, SU, 8>},
            {scan_wave_kernel<NT / 2, SU, 2>, scan_wave_kernel<NT / 2, SU, 3>,
             scan_wave_kernel<NT / 2, SU, 4>, scan_wave_kernel<NT / 2, SU, 6>,
             scan_wave_kernel<NT / 2, SU, 8>}};
        static int mx[2][5] = {{-1, -1, -1, -1, -1}, {-1, -1, -1, -1, -1}};
        const int ji = sh.wave == 2 ? 0 : sh.wave == 3 ? 1 : sh.wave == 4 ? 2 : sh.wave == 6 ? 3 : 4;
        const int ni = sh.nt == NT ? 0 : 1;
        if (mx[ni][ji] < 0) {
            mx[ni][ji] = allow_max_lds((const void*)kf[ni][ji]);
            // M = 16 addresses its LUT from LDS address 0: no static LDS
            if (static_lds((const void*)kf[ni][ji]) != 0) mx[ni][ji] = 0;
        }
        if (sh.lds > mx[ni][ji]) return hipErrorInvalidValue;
        hipLaunchKernelGGL(kf[ni][ji], dim3(sh.G), dim3(sh.nt), sh.lds, s, q_rot, d, Ds, K1D, bpd,
                           c1d, M, probes, gofs, qtot, B, P, ldesc, codes_t, ck, sh.region,
                           partial, partial_slot, sh.ov);
        return hipGetLastError();
    }
    static const int max_dyn = allow_max_lds((const void*)scan_topck_kernel<NT, SU>);
    if (sh.lds > max_dyn) return hipErrorInvalidValue;
    hipLaunchKernelGGL((scan_topck_kernel<NT, SU>), dim3(sh.G), dim3(NT), sh.lds, s, q_rot, d, Ds,
                       K1D, bpd, c1d, M, probes, gofs, qtot, B, P, ldesc, codes_t, ck, partial,
                       partial_slot, sh.ov);
    return hipGetLastError();
}

// The refine's 8-byte-piece path: 4-bit codes, 16 | d, rows of whole pieces,
// at most 4 pieces per lane (d <= 1024).  Its table of squared differences is
// code-major: the entry of code c and dimension 16 p + e sits at
// c * refine_tab_row(d) + 17 p + e (one pad word per piece; a row is a
// multiple of 64 words, so every code's row starts on bank 0).  Lane l16 of
// candidate group g (the four groups of a wave) takes its pieces l16 + 16 u
// in the order u = g, g + 1, ... (mod its piece count), so at every step the
// wave's 64 reads fall on banks 17 l16 + 16 u + e (mod 64), all distinct
// whatever the codes (reading pieces in the same order in every group put up
// to four lanes on one bank).
__host__ __device__ inline bool refine_pieces(int d, int Br, int bpv) {
    return Br == 4 && d % 16 == 0 && bpv % 8 == 0 && d <= 1024;
}
__host__ __device__ inline int refine_tab_row(int d) { return (d / 16 * 17 + 63) / 64 * 64; }
__host__ __device__ inline int refine_tab_words(int d) { return 16 * refine_tab_row(d); }

// Residual refine and final top-k of one query's exact short list (the
// ksel keys in S.kout, ascending, with their pool slots in kslot):
// topck_dbg (optional) gets the short list, out_d / out_i the k best by
// (refined dist, id), (+inf, -1) past ksel.  Called by the whole workgroup;
// cpos, cprim and fkeys are LDS scratch of ck entries, sq the query (one pad
// word per 32), rc the residual codebooks; tab (optional; refine_tab_words(d)
// floats, used when refine_pieces holds) is LDS scratch for the table of
// squared differences per dimension and code.
template <int NT>
__device__ __forceinline__ void refine_short_list(
    StreamSel& S, int ksel, int ck, int k, int b, const int* kslot, int* cpos, float* cprim,
    unsigned long long* fkeys, const float* sq, const float* rc, int d, int Ds, int Kr, int RC,
    int Br, int bpv, const uint8_t* __restrict__ list_res, const float* __restrict__ list_corr,
    const int32_t* __restrict__ list_ids, float* __restrict__ out_d, int32_t* __restrict__ out_i,
    unsigned long long* __restrict__ topck_dbg, float* tab) {
    const int tid = threadIdx.x;
    // codebook of dimension j: one shared codebook, or that of subspace j / Ds
    int ds_shift = -1;
    if (RC > 1 && (Ds & (Ds - 1)) == 0) ds_shift = __ffs(Ds) - 1;
    auto cbo = [&](int j) -> int {
        if (RC == 1) return 0;
        return (ds_shift >= 0 ? (j >> ds_shift) : (j / Ds)) * Kr;
    };
    const bool pieces = refine_pieces(d, Br, bpv);
    if (!pieces) tab = nullptr;
    const int grp = tid >> 4, l16 = tid & 15;
    constexpr int NG = NT / 16;
    // 4-bit codes in 8-byte pieces of 16 dimensions: lane l16 of a candidate
    // sums its np pieces l16 + 16 up[u], u = 0 .. np-1, up[u] = (u + g) mod np
    // with g = grp mod 4 (a load of the 16 lanes reads 128 contiguous bytes
    // of the candidate); each round's pieces, correction and id are
    // requested while the round before it is summed
    const int npc = d >> 4;
    const int np = pieces && l16 < npc ? (npc - 1 - l16) / 16 + 1 : 0;
    // (u + g) mod np for u < np <= 4, g < 4
    auto upiece = [&](int u) -> int {
        int v = u + (grp & 3);
        if (v >= np) v -= np;
        if (v >= np) v -= np;
        if (v >= np) v -= np;
        return v;
    };
    uint2 pwc[4], pwn[4];
    float pcorr_c = 0.0f, pcorr_n = 0.0f;
    int pid_c = 0, pid_n = 0;
    auto pfetch = [&](int base, uint2 (&w)[4], float& corr, int& id) {
        const int c = base + grp;
        if (c < ksel) {
            const int pos = kslot[c];
            const uint2* rp = (const uint2*)(list_res + (int64_t)pos * bpv) + l16;
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (u < np) w[u] = rp[16 * upiece(u)];
            if (l16 == 0) {
                corr = list_corr[pos];
                id = list_ids[pos];
            }
        }
    };
    const int trow = refine_tab_row(d);
    // the first round's pieces, correction and id are requested before the
    // table is built (kslot is complete on entry)
    if (pieces) pfetch(0, pwc, pcorr_c, pid_c);
    if (tab) {
        // (q_j - codeword c)^2, rounded as the sum below rounds it, at
        // tab[c * trow + (j / 16) * 17 + j % 16]; the query value and the 16
        // codewords of dimension j are read before its 16 stores
        for (int j = tid; j < d; j += NT) {
            const float qj = sq[j + (j >> 5)];
            const float* rj = rc + cbo(j);
            float cv[16];
#pragma unroll
            for (int c = 0; c < 16; c++) cv[c] = rj[c];
            float* tj = tab + (j >> 4) * 17 + (j & 15);
#pragma unroll
            for (int c = 0; c < 16; c++) {
                const float df = qj - cv[c];
                tj[c * trow] = df * df;
            }
        }
    }
    for (int r = tid; r < ck; r += NT) {
        if (r < ksel) {
            const unsigned long long kk = S.kout[r];
            cprim[r] = ord2f((uint32_t)(kk >> 32));
            cpos[r] = kslot[r];
            if (topck_dbg) topck_dbg[(int64_t)b * ck + r] = kk;
        } else if (topck_dbg) {
            topck_dbg[(int64_t)b * ck + r] = ~0ull;
        }
    }
    __syncthreads();

    // residual refine: 16 lanes per candidate, each summing its share of the
    // dimensions, then a fixed xor tree adds the 16 partial sums.
    const int dpc = (Br == 4) ? 32 : 16;  // dimensions per 16-byte chunk
    const bool vec = (bpv % 16) == 0 && (d % dpc) == 0;
    int chk = (d + 15) / 16;
    if (vec) chk = (chk + dpc - 1) / dpc * dpc;
    else chk += chk & 1;
    // the residual distance of one 16-byte chunk (dpc dimensions from jb)
    auto chunk = [&](const uint4& w, int jb, float& sres) {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
        if (Br == 4) {
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
                for (int nb = 0; nb < 8; nb++) {
                    const int jj = jb + q4 * 8 + nb;
                    const float df = sq[jj + (jj >> 5)] - rc[cbo(jj) + ((ww[q4] >> (4 * nb)) & 0x0Fu)];
                    sres = sres + df * df;
                }
        } else {
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
                for (int nb = 0; nb < 4; nb++) {
                    const int jj = jb + q4 * 4 + nb;
                    const float df = sq[jj + (jj >> 5)] - rc[cbo(jj) + ((ww[q4] >> (8 * nb)) & 0xFFu)];
                    sres = sres + df * df;
                }
        }
    };
    if (pieces) {
        uint2(&wc)[4] = pwc;
        uint2(&wn)[4] = pwn;
        float &corr_c = pcorr_c, &corr_n = pcorr_n;
        int &id_c = pid_c, &id_n = pid_n;
        for (int base = 0; base < ksel; base += NG) {
            if (base + NG < ksel) pfetch(base + NG, wn, corr_n, id_n);
            const int c = base + grp;
            const bool valid = c < ksel;
            float sres = 0.0f;
            // l16 opaque per round: the LDS addresses of the pieces'
            // dimensions are formed here instead of being hoisted out of the
            // loop (64 of them would not stay in registers)
            int lv = l16;
            asm volatile("" : "+v"(lv));
            if (valid && tab) {
                // LDS byte addresses: code c's entry is one 24-bit
                // multiply-add from the piece's base
                typedef __attribute__((address_space(3))) const char lds_cchar;
                const uint32_t rowb = 4u * (uint32_t)trow;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (u < np) {
                        lds_cchar* tp = (lds_cchar*)(tab + (lv + 16 * upiece(u)) * 17);
                        const uint32_t ww[2] = {wc[u].x, wc[u].y};
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            const uint32_t c = (ww[e >> 3] >> (4 * (e & 7))) & 15u;
                            sres = sres + *(__attribute__((address_space(3))) const float*)(tp + __umul24(c, rowb) + 4 * e);
                        }
                    }
                }
            } else if (valid) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (u < np) {
                        const int pc = lv + 16 * upiece(u);
                        const uint32_t ww[2] = {wc[u].x, wc[u].y};
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            const int jj = pc * 16 + e;
                            const float df = sq[jj + (jj >> 5)] -
                                             rc[cbo(jj) + ((ww[e >> 3] >> (4 * (e & 7))) & 15u)];
                            sres = sres + df * df;
                        }
                    }
                }
            }
            sres = sres + __shfl_xor(sres, 8);
            sres = sres + __shfl_xor(sres, 4);
            sres = sres + __shfl_xor(sres, 2);
            sres = sres + __shfl_xor(sres, 1);
            if (valid && l16 == 0) {
                const float comp = (cprim[c] + sres) + corr_c;
                fkeys[c] = ((unsigned long long)f2ord(comp) << 32) | (uint32_t)id_c;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) wc[u] = wn[u];
            corr_c = corr_n;
            id_c = id_n;
        }
    } else if (vec && chk / dpc <= 4) {
        // at most 4 chunks per lane: the next round's chunks, correction and
        // id are loaded while this round is summed
        const int j0 = l16 * chk, j1 = (j0 + chk) < d ? (j0 + chk) : d;
        const int nch = j1 > j0 ? (j1 - j0) / dpc : 0;
        uint4 wc[4], wn[4];
        float corr_c = 0.0f, corr_n = 0.0f;
        int id_c = 0, id_n = 0;
        auto fetch = [&](int base, uint4 (&w)[4], float& corr, int& id) {
            const int c = base + grp;
            if (c < ksel) {
                const int pos = cpos[c];
                const uint4* rp = (const uint4*)(list_res + (int64_t)pos * bpv + (j0 * Br) / 8);
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (u < nch) w[u] = rp[u];
                if (l16 == 0) {
                    corr = list_corr[pos];
                    id = list_ids[pos];
                }
            }
        };
        fetch(0, wc, corr_c, id_c);
        for (int base = 0; base < ksel; base += NG) {
            if (base + NG < ksel) fetch(base + NG, wn, corr_n, id_n);
            const int c = base + grp;
            const bool valid = c < ksel;
            float sres = 0.0f;
            // j0 opaque per round: the LDS addresses of the 4 chunks' dimensions
            // are formed here instead of being hoisted out of the loop
            int jv = j0;
            asm volatile("" : "+v"(jv));
            if (valid) {
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (u < nch) chunk(wc[u], jv + u * dpc, sres);
            }
            sres = sres + __shfl_xor(sres, 8);
            sres = sres + __shfl_xor(sres, 4);
            sres = sres + __shfl_xor(sres, 2);
            sres = sres + __shfl_xor(sres, 1);
            if (valid && l16 == 0) {
                const float comp = (cprim[c] + sres) + corr_c;
                fkeys[c] = ((unsigned long long)f2ord(comp) << 32) | (uint32_t)id_c;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) wc[u] = wn[u];
            corr_c = corr_n;
            id_c = id_n;
        }
    } else
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
            if (vec) {
                const uint4* rp = (const uint4*)(rcode + (j0 * Br) / 8);
                const int nch = j1 > j0 ? (j1 - j0) / dpc : 0;
                for (int c4 = 0; c4 < nch; c4 += 4) {
                    uint4 wv[4];
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        if (c4 + u < nch) wv[u] = rp[c4 + u];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        if (c4 + u >= nch) break;
                        chunk(wv[u], j0 + (c4 + u) * dpc, sres);
                    }
                }
            } else if (Br == 4) {
                for (int j = j0; j < j1; j += 2) {
                    const uint32_t byte = rcode[j >> 1];
                    const float df0 = sq[j + (j >> 5)] - rc[cbo(j) + (byte & 0x0Fu)];
                    sres = sres + df0 * df0;
                    if (j + 1 < j1) {
                        const float df1 = sq[(j + 1) + ((j + 1) >> 5)] - rc[cbo(j + 1) + (byte >> 4)];
                        sres = sres + df1 * df1;
                    }
                }
            } else {
                for (int j = j0; j < j1; j++) {
                    const float df = sq[j + (j >> 5)] - rc[cbo(j) + rcode[j]];
                    sres = sres + df * df;
                }
            }
        }
        sres = sres + __shfl_xor(sres, 8);
        sres = sres + __shfl_xor(sres, 4);
        sres = sres + __shfl_xor(sres, 2);
        sres = sres + __shfl_xor(sres, 1);
        if (valid && l16 == 0) {
            const float comp = (cprim[c] + sres) + list_corr[pos];
            fkeys[c] = ((unsigned long long)f2ord(comp) << 32) | (uint32_t)list_ids[pos];
        }
    }
    __syncthreads();

    // final top-k by (dist, id)
    const int kf = ksel < k ? ksel : k;
    if (kf > 0) select_keys<NT>(fkeys, ksel, kf, S.kout, S.kidx, S.ktmp, S.st);
    for (int r = tid; r < k; r += NT) {
        if (r < kf) {
            const unsigned long long kk = S.kout[r];
            out_d[(int64_t)b * k + r] = ord2f((uint32_t)(kk >> 32));
            out_i[(int64_t)b * k + r] = (int32_t)(uint32_t)(kk & 0xffffffffull);
        } else {
            out_d[(int64_t)b * k + r] = __builtin_huge_valf();
            out_i[(int64_t)b * k + r] = -1;
        }
    }
}

// ---------------------------------------------------------------------------
// Merge + residual refine + final top-k, one workgroup per query
// (v14/search.cu:198-291 with the exact selection of jhq_v3_ivf).
// The query's segment lists are merged by the streaming selection; the
// residual distance of a candidate is summed by 16 lanes over 16 contiguous
// dimension ranges, then added across the lanes in a fixed xor tree.
// ---------------------------------------------------------------------------
template <int NT>
__global__ void __launch_bounds__(NT)
refine_topk_kernel(const unsigned long long* __restrict__ partial,
                   const int32_t* __restrict__ partial_slot, const int32_t* __restrict__ qtot,
                   int B, int Gmax, int ck, int k, const float* __restrict__ q_rot, int d, int Ds,
                   const float* __restrict__ res_c1d, int Kr, int RC, int Br, int bpv,
                   const int4* __restrict__ ldesc, int nlist, const uint8_t* __restrict__ list_res,
                   const float* __restrict__ list_corr, const int32_t* __restrict__ list_ids,
                   float* __restrict__ out_d, int32_t* __restrict__ out_i,
                   unsigned long long* __restrict__ topck_dbg, int stage_cap, int ov,
                   int use_tab) {
    extern __shared__ __align__(16) unsigned char smem[];
    StreamSel S;
    unsigned char* p = stream_carve<NT>(smem, ck, &S);
    unsigned long long* fkeys = (unsigned long long*)p;  // [ck] final-candidate keys
    unsigned long long* stage = fkeys + ck;              // [stage_cap] segment lists
    int* sslot = (int*)(stage + stage_cap);              // [stage_cap] their pool slots
    int* kslot = sslot + stage_cap;                      // [ck] slots of the short list
    float* rc = (float*)(kslot + ck);                    // [RC*Kr] residual codebooks
    int* qpre = (int*)(rc + RC * Kr);
    int* spre = qpre + B + 1;
    int* cpos = spre + B + 1;
    float* cprim = (float*)(cpos + ck);
    int* wsum = (int*)(cprim + ck);
    // query staged with one pad word per 32 so that lanes reading 32-dim
    // ranges at a 32-word stride hit distinct banks
    float* sq = (float*)(wsum + NT / 64);
    float* tab = use_tab ? sq + d + d / 32 + 1 : nullptr;  // [refine_tab_words(d)]

    const int b = blockIdx.x, tid = threadIdx.x;
    JHQ_PHASE_DECL
    work_plan<NT>(qtot, B, Gmax, ov, qpre, spre, wsum);
    for (int i = tid; i < d; i += NT) sq[i + (i >> 5)] = q_rot[(int64_t)b * d + i];
    for (int i = tid; i < RC * Kr; i += NT) rc[i] = res_c1d[i];
    const int s0 = spre[b], s1 = spre[b + 1];
    stream_begin<NT>(S);
    __syncthreads();
    JHQ_PHASE(0);

    // merge the query's segment lists into the exact top-ck
    const int nseg = s1 - s0;
    const int nkeys = nseg * ck;
    const unsigned long long* src = partial + (int64_t)s0 * ck;
    int ksel;
    if (nkeys <= stage_cap) {
        // each list is sorted ascending (~0 padded): the rank of key x from
        // list a at index i in the union is i + sum over the other lists of
        // the number of keys below x (keys are distinct)
        const int32_t* srcs = partial_slot + (int64_t)s0 * ck;
        for (int i = tid; i < nkeys; i += NT) {
            stage[i] = src[i];
            sslot[i] = srcs[i];
        }
        if (tid == 0) S.ctl[0] = 0;
        __syncthreads();
        int nv = 0;
        for (int i = tid; i < nkeys; i += NT) nv += stage[i] != ~0ull ? 1 : 0;
        for (int off = 32; off > 0; off >>= 1) nv += __shfl_xor(nv, off);
        if ((tid & 63) == 0 && nv) atomicAdd(&S.ctl[0], nv);
        __syncthreads();
        ksel = min(ck, S.ctl[0]);
        for (int idx = tid; idx < nkeys; idx += NT) {
            const unsigned long long x = stage[idx];
            if (x == ~0ull) continue;
            const int a = idx / ck;
            int r = idx - a * ck;
            for (int bl = 0; bl < nseg && r < ksel; bl++) {
                if (bl == a) continue;
                const unsigned long long* L = stage + bl * ck;
                int lo = 0, hi = ck;  // first index with L[i] >= x
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (L[mid] < x) lo = mid + 1;
                    else hi = mid;
                }
                r += lo;
            }
            if (r < ksel) {
                S.kout[r] = x;
                kslot[r] = sslot[idx];
            }
        }
        __syncthreads();
    } else {
        // many segments: streaming selection, 4 keys per thread per round
        const int rounds = (nkeys + NT * 4 - 1) / (NT * 4);
        for (int r = 0; r < rounds; r++) {
            uint32_t o[4], tg[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = r * NT * 4 + threadIdx.x * 4 + j;
                const unsigned long long kk = i < nkeys ? src[i] : ~0ull;
                o[j] = (uint32_t)(kk >> 32);
                tg[j] = (uint32_t)(kk & 0xffffffffull);
            }
            stream_round<NT, 4>(S, ck, o, tg);
        }
        ksel = stream_end<NT>(S, ck);
        // pool slots of the short list: the list whose canonical range holds
        // the tag (binary search over the list descriptors)
        for (int r = tid; r < ksel; r += NT) {
            const int tag = (int)(uint32_t)(S.kout[r] & 0xffffffffull);
            int lo = 0, hi = nlist - 1;  // last list with cbase <= tag
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (ldesc[mid].w <= tag) lo = mid;
                else hi = mid - 1;
            }
            const int4 L = ldesc[lo];
            kslot[r] = L.x + (tag - L.w);
        }
        __syncthreads();
    }
    JHQ_PHASE(1);
    refine_short_list<NT>(S, ksel, ck, k, b, kslot, cpos, cprim, fkeys, sq, rc, d, Ds, Kr, RC, Br,
                          bpv, list_res, list_corr, list_ids, out_d, out_i, topck_dbg, tab);
    JHQ_PHASE(3);
    JHQ_PHASE_FLUSH(2);
}

hipError_t refine_topk(const unsigned long long* partial, const int32_t* partial_slot,
                       const int32_t* qtot, int B, const ScanShape& sh, int ck, int k,
                       const float* q_rot, int d, int Ds, const float* res_c1d, int Kr, int RC,
                       int Br, int bpv, const int4* ldesc, int nlist, const uint8_t* list_res,
                       const float* list_corr, const int32_t* list_ids, float* out_d,
                       int32_t* out_i, unsigned long long* topck_dbg, hipStream_t s) {
    constexpr int NT = kRefineNT;
    if (k > ck) return hipErrorInvalidValue;
    // the segment lists are staged in LDS for the rank merge when they fit
    // (up to max(4096, 8 ck) keys); more go through the streaming selection,
    // so the stage shrinks to the LDS the rest leaves (long short lists with
    // per-subspace codebooks)
    const size_t rest = stream_lds_bytes(NT, ck) + (size_t)ck * 8 + (size_t)ck * 4 +
                        (size_t)RC * Kr * 4 + (size_t)(2 * (B + 1)) * 4 + (size_t)ck * 4 * 2 +
                        (NT / 64) * 4 + (size_t)(d + d / 32 + 1) * 4 + 32;
    static const int max_dyn = allow_max_lds((const void*)refine_topk_kernel<NT>);
    if ((int)rest > max_dyn) return hipErrorInvalidValue;
    // the table of squared differences halves the refine's LDS reads; it is
    // taken when a stage of 4096 keys still fits beside it
    const size_t tab = refine_pieces(d, Br, bpv) ? (size_t)refine_tab_words(d) * 4 : 0;
    const int use_tab = tab > 0 && rest + tab + (size_t)4096 * 12 <= (size_t)max_dyn;
    const size_t rest_t = rest + (use_tab ? tab : 0);
    const int stage_cap = (int)std::min<size_t>((size_t)std::max(4096, 8 * ck),
                                                ((size_t)max_dyn - rest_t) / 12 / 4 * 4);
    const size_t lds = rest_t + (size_t)stage_cap * (8 + 4);
    hipLaunchKernelGGL(refine_topk_kernel<NT>, dim3(B), dim3(NT), lds, s, partial, partial_slot,
                       qtot, B, sh.G, ck, k, q_rot, d, Ds, res_c1d, Kr, RC, Br, bpv, ldesc, nlist,
                       list_res, list_corr, list_ids, out_d, out_i, topck_dbg, stage_cap,
                       sh.ov, use_tab);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Integer-MFMA pre-scan for one-bit digits (K1D = 2, Ds = 8), with an exact
// re-check.  With one bit per dimension a subspace's LUT entry is affine in
// the bits b_k of its code (v14/search.cu:65-91 computes it as a sum of
// squares over the subspace's dimensions):
//   lut[m][v] = sum_k (q_k - c[b_k])^2 = sum_k (q_k - c0)^2 + sum_k b_k dl_k,
//   dl_k = (q_k - c1)^2 - (q_k - c0)^2,
// so a candidate's ADC distance is a(x) = C + <dl, bits(x)> with
// C = ||q - c0||^2.  Per query, dl is rounded to multiples of a step s
// (|round(dl/s)| <= 32000, split into two int8 halves hi * 256 + lo), and
// I(x) = sum_k b_k round(dl_k / s) is exact in int32: two int8 MFMA products
// per 64 dimensions, for up to 16 queries that probe the same list at once
// (the queries of a batch share most of their probed candidates).
//
// Bound: |C + s I(x) - a(x)| <= e_q = s D / 2 (plus rounding slack), and the
// reference's fp32 distance a_ref(x), a sum of nonnegative rounded terms, is
// within g = (M + 16) 2^-23 of a(x) relatively.  With T the ck-th smallest I
// of the query, at least ck candidates have a_ref <= U = (1 + g)(C + s T +
// e_q), so every candidate in the exact top-ck has
//   I(x) <= ((U / (1 - g)) + e_q - C) / s.
// Those candidates are re-checked: their distances are recomputed in the
// reference's order (each LUT entry's fma chain, then the M entries added in
// m order from 0.0f) and the exact top-ck by (dist, stored position) is
// selected from them, so the result does not depend on the MFMA values.
// Queries with non-finite or huge values re-check every candidate.
// ---------------------------------------------------------------------------
// Tile-kernel waves per CU (on average), by the batch's (query, probe)
// pairs: two (one 4-wave workgroup on every other CU) for at most
// kMfmaFewPairs, else four.  The waves are bound by issue and by their
// start-up load chain, and the CUs left free run the other search lanes'
// kernels beside them.  With the lanes on hardware queues of their own,
// config 2 (1024 pairs) runs at 1.81 M queries/s against 1.75 M with one
// workgroup per CU, 1.77 M with three waves per CU, 1.56 M with one, 1.64 M
// with six, 1.54 M with eight; config 5 (4096 pairs, more tiles per batch)
// at 728 k with four waves per CU against 713 k with two.
constexpr int kMfmaWpcFew = 2, kMfmaWpcMany = 4, kMfmaFewPairs = 2048;
constexpr int kRecheckNT = 1024;
constexpr int kRecheckCap = 2048;   // survivors / members held in LDS
constexpr int kRecheckCHM = 128;    // members per exact-distance round
constexpr int kRecheckLPT = 16;     // 16-byte row loads in flight per thread (whole-row pass)
constexpr int kRecheckQCap = 2048;  // tiles listed for the tile-wise pass 2
constexpr int kRecheckQCap1 = 1536; // tiles listed for the in-register ck-th value
constexpr int kRecheckRegV = 8;     // its values per thread
constexpr int kRecheckTM = 16;      // tile minima per thread in flight (global)
constexpr int kRecheckTR = 32;      // tile minima per thread ranked in registers
constexpr int kRecheckTPL = 4;      // listed tiles' row loads in flight per lane

constexpr int kMfmaPD = 6;  // tiles in flight per wave
// The minimum over each 16-lane row, on every lane of the row: swaps within
// quads, then rotations by 4 and 8 inside the row (DPP operands of v_min, no
// LDS round trips as a shuffle through ds_bpermute would take).
__device__ __forceinline__ uint32_t row16_min_u32(uint32_t v) {
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false));   // quad [1,0,3,2]
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false));   // quad [2,3,0,1]
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false));  // row_ror:4
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false));  // row_ror:8
    return v;
}
// One 16-candidate tile: the lane's code dwords cw (row j of the tile,
// subspaces GS h .. GS h + GS - 1, four to a dword), the bit planes, two
// int8 MFMA chains (hi and lo halves of the query steps), and the biased
// integer distances of rows 4h..4h+3 (rows without a query have d < 0).
template <int M>
__device__ __forceinline__ void mfma_tile(const uint32_t (&cw)[M / 16], int h, int j,
                                          const mfma_v4i (&ahi)[M / 8],
                                          const mfma_v4i (&alo)[M / 8], int cand, int nl,
                                          uint32_t* dump, uint32_t* tmin, int d0, int d1, int d2,
                                          int d3) {
    constexpr int NK = M / 8, ND = M / 16;
    mfma_v4i ah = {0, 0, 0, 0}, alw = {0, 0, 0, 0};
    // code dwords in pairs: one 64-bit shift gives bit plane k of both
    // (bits shifted across the dword boundary land outside the byte mask)
#pragma unroll
    for (int t = 0; t < ND / 2; t++) {
        const uint64_t X = ((uint64_t)cw[2 * t + 1] << 32) | cw[2 * t];
        uint64_t pl[8];
#pragma unroll
        for (int k = 0; k < 8; k++) pl[k] = (X >> k) & 0x0101010101010101ull;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            // step 4t + q: dword 2t + q / 2, bits 4 (q % 2) .. + 3
            const int hi = q >> 1, k0 = 4 * (q & 1);
            mfma_v4i bv;
#pragma unroll
            for (int i = 0; i < 4; i++) bv[i] = (int)(uint32_t)(pl[k0 + i] >> (32 * hi));
            ah = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[4 * t + q], bv, ah, 0, 0, 0);
            alw = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[4 * t + q], bv, alw, 0, 0, 0);
        }
    }
    if constexpr (ND % 2 == 1) {
#pragma unroll
        for (int s = NK - 2; s < NK; s++) {
            const uint32_t x = cw[ND - 1];
            const int k0 = 4 * (s & 1);
            mfma_v4i bv;
            bv[0] = (int)((x >> k0) & 0x01010101u);
            bv[1] = (int)((x >> (k0 + 1)) & 0x01010101u);
            bv[2] = (int)((x >> (k0 + 2)) & 0x01010101u);
            bv[3] = (int)((x >> (k0 + 3)) & 0x01010101u);
            ah = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[s], bv, ah, 0, 0, 0);
            alw = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[s], bv, alw, 0, 0, 0);
        }
    }
    const bool ok = cand < nl;
    const uint32_t v0 = ok ? (uint32_t)(ah[0] * 256 + alw[0]) + 0x80000000u : 0xffffffffu;
    const uint32_t v1 = ok ? (uint32_t)(ah[1] * 256 + alw[1]) + 0x80000000u : 0xffffffffu;
    const uint32_t v2 = ok ? (uint32_t)(ah[2] * 256 + alw[2]) + 0x80000000u : 0xffffffffu;
    const uint32_t v3 = ok ? (uint32_t)(ah[3] * 256 + alw[3]) + 0x80000000u : 0xffffffffu;
    // d0..d3: the rows' dump slots of the tile's first candidate (multiples of 16)
    if (d0 >= 0) dump[d0 + j] = v0;
    if (d1 >= 0) dump[d1 + j] = v1;
    if (d2 >= 0) dump[d2 + j] = v2;
    if (d3 >= 0) dump[d3 + j] = v3;
    // each row's minimum over the tile's 16 candidates (the lanes of one
    // group, one DPP row): the re-check bounds its ck-th smallest value from
    // these
    const uint32_t m0 = row16_min_u32(v0), m1 = row16_min_u32(v1);
    const uint32_t m2 = row16_min_u32(v2), m3 = row16_min_u32(v3);
    if (j == 0) {
        if (d0 >= 0) tmin[d0 / 16] = m0;
        if (d1 >= 0) tmin[d1 / 16] = m1;
        if (d2 >= 0) tmin[d2 / 16] = m2;
        if (d3 >= 0) tmin[d3 / 16] = m3;
    }
}

// Lane l: query row / candidate column l % 16, K group l / 16 (the lane
// layout of v_mfma_i32_16x16x64_i8: A and B bytes of one lane cover the same
// 16 dimensions; result register v of lane l is query row 4 (l / 16) + v,
// candidate l % 16).  Each wave walks its share of the batch's tiles group by
// group (no shared counter).  A tile of 16 candidates is 16 rows of M code
// bytes in the row-major copy; lane (j, h) loads its candidate j's M / 4
// bytes for subspaces GS h .. GS h + GS - 1 straight into registers,
// kMfmaPD tiles ahead (no LDS); bit plane k of a code dword is
// (w >> k) & 0x01010101.
// The lane's code dwords of one tile row from the row-major copy: GS = M / 4
// bytes (ND dwords) at p, as 16-byte loads where GS is a multiple of 16.
template <int M>
__device__ __forceinline__ void mfma_row_load(const uint8_t* p, uint32_t (&cw)[M / 16]) {
    constexpr int ND = M / 16;
    if constexpr ((M / 4) % 16 == 0) {
#pragma unroll
        for (int t = 0; t < ND / 4; t++) {
            const uint4 v = *(const uint4*)(p + 16 * t);
            cw[4 * t] = v.x;
            cw[4 * t + 1] = v.y;
            cw[4 * t + 2] = v.z;
            cw[4 * t + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int t = 0; t < ND; t++) cw[t] = *(const uint32_t*)(p + 4 * t);
    }
}

// Wave wid runs tiles [wid T / W, (wid + 1) T / W) of the batch; each
// workgroup finds where its waves start from the hash of the batch's lists
// (a scan of per-thread slot chunks).  Lane (j, h) holds row j of each tile
// (list slot 16 t + j) for subspaces GS h .. GS h + GS - 1, read straight
// from the row-major copy (a tile's 16 rows are one contiguous run of 16 M
// bytes) into a ring of kMfmaPD tiles in registers.
template <int M>
__global__ void __launch_bounds__(256)
mfma_scan_kernel(MfmaWs w, const int4* __restrict__ ldesc, const uint8_t* __restrict__ rows,
                 uint32_t* __restrict__ dump, uint32_t* __restrict__ tmin) {
    constexpr int NK = M / 8, ND = M / 16, GS = M / 4, D = 8 * M, NT = 256;
    __shared__ int csum[NT + 1], wsm[NT / 64];
    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, h = lane >> 4;
    const int W = gridDim.x * 4, wid = blockIdx.x * 4 + (tid >> 6);
    const int H = w.H;
    JHQ_PHASE_DECL
    // the batch's tiles: thread t sums the slots of its chunk (per slots;
    // per <= 64 since H <= 64 NT), and an exclusive scan of the chunk sums
    // gives csum (csum[NT] = T)
    const int per = (H + NT - 1) / NT;
    const int cs0 = min(H, tid * per), cs1 = min(H, cs0 + per);
    int mine = 0;
    for (int sb = cs0; sb < cs1; sb += 8) {
        int4 rec[8];
#pragma unroll
        for (int u = 0; u < 8; u++) rec[u] = sb + u < cs1 ? w.hs[sb + u] : make_int4(-1, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (rec[u].x >= 0) mine += ((rec[u].y + 15) >> 4) * ((rec[u].z + kGroup - 1) / kGroup);
    }
    int inc = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    if (lane == 63) wsm[tid >> 6] = inc;
    __syncthreads();
    int wbase = 0;
    for (int w2 = 0; w2 < (tid >> 6); w2++) wbase += wsm[w2];
    csum[tid] = wbase + inc - mine;
    if (tid == NT - 1) csum[NT] = wbase + inc;
    __syncthreads();
    const int T = csum[NT];
    JHQ_PHASE(2);
    const int a0 = (int)((int64_t)wid * T / W), a1 = (int)((int64_t)(wid + 1) * T / W);
    int left = a1 - a0;
    if (left <= 0) return;
    // the chunk holding tile a0 (the last with csum <= a0), then its slot:
    // lane l takes slot s0 + l
    int lo = 0, hi = NT - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (csum[mid] <= a0) lo = mid;
        else hi = mid - 1;
    }
    const int s0 = min(H, lo * per), s1 = min(H, s0 + per);
    int tl = 0, nzl = 1;
    // (a clamped load, then the select: no load through a selected pointer)
    int4 rec0 = w.hs[min(s0 + lane, H - 1)];
    if (s0 + lane >= s1) rec0.x = -1;
    if (rec0.x >= 0) {
        nzl = (rec0.z + kGroup - 1) / kGroup;
        tl = ((rec0.y + 15) >> 4) * nzl;
    }
    int tinc = tl;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(tinc, o);
        if (lane >= o) tinc += t;
    }
    const int rel = a0 - csum[lo];
    const unsigned long long fm = __ballot(s0 + lane < s1 && tinc > rel);
    if (fm == 0ull) return;  // not reached: tile a0 lies in chunk lo
    const int fl = __ffsll((long long)fm) - 1;
    int hs = s0 + fl;
    const int rr = rel - __shfl(tinc - tl, fl), nz0 = __shfl(nzl, fl);
    int gt = rr / nz0, off = rr - gt * nz0;
    // the first slot's record is lane fl's (no second load)
    int4 srec = make_int4(__shfl(rec0.x, fl), __shfl(rec0.y, fl), __shfl(rec0.z, fl), 0);
    JHQ_PHASE(3);
    while (left > 0) {
        // the slot's list and the group's 16 pair entries
        const int cnt = srec.y;
        const int r = 16 * gt + j;
        const int2 gqv = r < w.B ? w.ql[(int64_t)hs * w.B + r] : make_int2(0, 0);
        const int4 L = ldesc[srec.x];
        const int nq = min(16, cnt - 16 * gt);
        const int n = min((L.z + kGroup - 1) / kGroup - off, left);
        const int nl = L.z;
        const int4 ga = make_int4(L.x, L.y, L.z, nq);
        // tiles past the run's last reload its last tile (in bounds, unused)
        const uint8_t* base = rows + ((int64_t)ga.x + 16 * off + j) * M + GS * h;
        uint32_t c0[ND], c1[ND], c2[ND], c3[ND], c4[ND], c5[ND];
#define JHQ_MFMA_FETCH(U, K) mfma_row_load<M>(base + (int64_t)16 * M * min((K), n - 1), c##U)
        JHQ_MFMA_FETCH(0, 0);
        JHQ_MFMA_FETCH(1, 1);
        JHQ_MFMA_FETCH(2, 2);
        JHQ_MFMA_FETCH(3, 3);
        JHQ_MFMA_FETCH(4, 4);
        JHQ_MFMA_FETCH(5, 5);
        // query steps of row j (rows past the group's queries take query
        // 0's: their products are never stored), requested with the rows
        mfma_v4i ahi[NK], alo[NK];
        {
            const int b = j < nq ? gqv.x : 0;
            const mfma_v4i* src = (const mfma_v4i*)(w.qa + (int64_t)b * 2 * D + h * NK * 16);
#pragma unroll
            for (int s = 0; s < NK; s++) {
                ahi[s] = src[s];
                alo[s] = src[D / 16 + s];
            }
        }
        // dump offsets of the run's first slot for query rows 4h .. 4h+3
        // (lane r of the wave's first 16 holds row r's entry)
        const int e0 = __shfl(gqv.y, 4 * h + 0), e1 = __shfl(gqv.y, 4 * h + 1);
        const int e2 = __shfl(gqv.y, 4 * h + 2), e3 = __shfl(gqv.y, 4 * h + 3);
        const int d0 = 4 * h + 0 < nq ? e0 + 16 * off : -1;
        const int d1 = 4 * h + 1 < nq ? e1 + 16 * off : -1;
        const int d2 = 4 * h + 2 < nq ? e2 + 16 * off : -1;
        const int d3 = 4 * h + 3 < nq ? e3 + 16 * off : -1;
        const int cbase = 16 * off + j;
        JHQ_PHASE(0);
#ifdef JHQ_PHASE_TIMING
        ph_acc[6] += 1;
        ph_acc[7] += n;
#endif
        // a slot's tile runs, then the slot is refilled kMfmaPD tiles ahead
#define JHQ_MFMA_TILE(U)                                                                    \
    {                                                                                       \
        const int k = k0 + U;                                                               \
        if (k < n)                                                                          \
            mfma_tile<M>(c##U, h, j, ahi, alo, cbase + 16 * k, nl, dump, tmin,              \
                         d0 < 0 ? -1 : d0 + 16 * k, d1 < 0 ? -1 : d1 + 16 * k,              \
                         d2 < 0 ? -1 : d2 + 16 * k, d3 < 0 ? -1 : d3 + 16 * k);             \
        JHQ_MFMA_FETCH(U, k + kMfmaPD);                                                     \
    }
        for (int k0 = 0; k0 < n; k0 += kMfmaPD) {
            JHQ_MFMA_TILE(0)
            JHQ_MFMA_TILE(1)
            JHQ_MFMA_TILE(2)
            JHQ_MFMA_TILE(3)
            JHQ_MFMA_TILE(4)
            JHQ_MFMA_TILE(5)
        }
#undef JHQ_MFMA_TILE
#undef JHQ_MFMA_FETCH
        left -= n;
        off = 0;
        // the next group: the slot's next 16 pairs, else the next occupied
        // slot (64 slots looked at a time, one per lane)
        if (++gt >= (cnt + 15) >> 4 && left > 0) {
            gt = 0;
            int found = -1;
            for (int sb = hs + 1; sb < H && found < 0; sb += 64) {
                const int4 rec = sb + lane < H ? w.hs[sb + lane] : make_int4(-1, 0, 0, 0);
                const unsigned long long oc = __ballot(rec.x >= 0);
                if (oc) {
                    const int fl2 = __ffsll((long long)oc) - 1;
                    found = sb + fl2;
                    srec = make_int4(__shfl(rec.x, fl2), __shfl(rec.y, fl2), __shfl(rec.z, fl2), 0);
                }
            }
            if (found < 0) break;
            hs = found;
        }
        JHQ_PHASE(1);
    }
    JHQ_PHASE_FLUSH(0);
}

// Largest biased I (I + 2^31) a member of the exact top-ck can have, given
// the biased ck-th smallest I of the query (see the bound above).
__device__ __forceinline__ uint32_t mfma_member_bound(const MfmaQS& Q, uint32_t Tb, int M) {
    if (Q.all) return 0xfffffffeu;
    const double g = (double)(M + 16) * 0x1p-23, ab = 1e-30;
    const double I = (double)((int64_t)Tb - 2147483648ll);
    const double U = (1.0 + g) * (Q.C + Q.s * I + Q.e) + ab;
    double R = ((U + ab) / (1.0 - g) + Q.e - Q.C) / Q.s;
    R = R + 1e-9 * fabs(R) + 1.0;
    if (!(R < 2147483646.0)) return 0xfffffffeu;
    if (R < -2147483647.0) return 0u;
    return (uint32_t)((int64_t)floor(R) + 2147483648ll);
}

// The k-th smallest (1 <= k <= n) of n values get(0..n), 8 bits a round:
// an LDS histogram of the values that match the bits found so far, and one
// wave finds the bin that holds the k-th.  hist: 256 ints; c2: 2 ints.
// hist[bin] += 1 for every active lane with match, wave-aggregated: the
// lanes sharing the first pending lane's bin add their count at once (up to
// three bins a call), the rest add one each.  The values of one query mostly
// share their top bytes, and plain atomics on one bin ran one lane at a time.
__device__ __forceinline__ void hist_add_wave(int* hist, uint32_t bin, bool match) {
    const int lane = threadIdx.x & 63;
    unsigned long long pend = __ballot(match);
#pragma unroll
    for (int it = 0; it < 3; it++) {
        if (!pend) return;
        const int first = __ffsll((long long)pend) - 1;
        const uint32_t b0 = (uint32_t)__shfl((int)bin, first);
        const unsigned long long same = __ballot(match && bin == b0) & pend;
        if (lane == first) atomicAdd(&hist[b0], __popcll(same));
        pend &= ~same;
    }
    if ((pend >> lane) & 1ull) atomicAdd(&hist[bin], 1);
}

// (Inlined: as a call it saved its caller's registers to scratch memory, and
// the re-check's tile-minimum bound took 12.5 instead of 8.8 us.)
template <int NT, class Get>
__device__ __forceinline__ uint32_t block_radix_kth(Get get, int n, int k, int* hist, int* c2) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint32_t pre = 0u, msk = 0u;
    int kr = k;
    for (int sh = 24; sh >= 0; sh -= 8) {
        for (int i = tid; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
        for (int i0 = 0; i0 < n; i0 += NT) {
            const int i = i0 + tid;
            const uint32_t v = i < n ? get(i) : 0u;
            hist_add_wave(hist, (v >> sh) & 255u, i < n && (v & msk) == pre);
        }
        __syncthreads();
        if (wv == 0) {
            // lane l holds bins 4l .. 4l+3: inclusive prefix over lanes
            int c[4], t = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                c[e] = hist[4 * lane + e];
                t += c[e];
            }
            int inc = t;
            for (int o = 1; o < 64; o <<= 1) {
                const int x = __shfl_up(inc, o);
                if (lane >= o) inc += x;
            }
            int below = inc - t;
            // the lane whose bins cross kr picks the bin
            if (below < kr && kr <= inc) {
                int e = 0;
                while (below + c[e] < kr) below += c[e++];
                c2[0] = 4 * lane + e;
                c2[1] = below;
            }
        }
        __syncthreads();
        pre |= (uint32_t)c2[0] << sh;
        msk |= 255u << sh;
        kr -= c2[1];
        __syncthreads();
    }
    return pre;
}

// block_radix_kth over a row of n4 * 4 values in global memory: each round
// puts kRecheckLPT 16-byte loads per thread in flight before it counts them
// (a value at a time, each round was a chain of dependent loads: 200 us for
// a 39 K row).
template <int NT>
__device__ __forceinline__ uint32_t block_radix_kth_row(const uint4* __restrict__ row4, int64_t n4,
                                                        int k, int* hist, int* c2) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint32_t pre = 0u, msk = 0u;
    int kr = k;
    for (int sh = 24; sh >= 0; sh -= 8) {
        for (int i = tid; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
        for (int64_t i0 = tid; i0 < n4; i0 += (int64_t)kRecheckLPT * NT) {
            uint4 v4[kRecheckLPT];
#pragma unroll
            for (int u = 0; u < kRecheckLPT; u++) {
                const int64_t i = i0 + (int64_t)u * NT;
                v4[u] = i < n4 ? row4[i] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < kRecheckLPT; u++) {
                const bool ok = i0 + (int64_t)u * NT < n4;
                const uint32_t vv[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
#pragma unroll
                for (int e = 0; e < 4; e++)
                    hist_add_wave(hist, (vv[e] >> sh) & 255u, ok && (vv[e] & msk) == pre);
            }
        }
        __syncthreads();
        if (wv == 0) {
            int c[4], t = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                c[e] = hist[4 * lane + e];
                t += c[e];
            }
            int inc = t;
            for (int o = 1; o < 64; o <<= 1) {
                const int x = __shfl_up(inc, o);
                if (lane >= o) inc += x;
            }
            int below = inc - t;
            if (below < kr && kr <= inc) {
                int e = 0;
                while (below + c[e] < kr) below += c[e++];
                c2[0] = 4 * lane + e;
                c2[1] = below;
            }
        }
        __syncthreads();
        pre |= (uint32_t)c2[0] << sh;
        msk |= 255u << sh;
        kr -= c2[1];
        __syncthreads();
    }
    return pre;
}

// block_radix_kth over n values in global memory (any alignment), with
// kRecheckTM loads per thread in flight per batch.
template <int NT>
__device__ __forceinline__ uint32_t block_radix_kth_glob(const uint32_t* __restrict__ p, int n,
                                                         int k, int* hist, int* c2) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint32_t pre = 0u, msk = 0u;
    int kr = k;
    for (int sh = 24; sh >= 0; sh -= 8) {
        for (int i = tid; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
        for (int i0 = 0; i0 < n; i0 += kRecheckTM * NT) {
            uint32_t v[kRecheckTM];
#pragma unroll
            for (int u = 0; u < kRecheckTM; u++) {
                const int i = i0 + u * NT + tid;
                v[u] = i < n ? p[i] : 0u;
            }
#pragma unroll
            for (int u = 0; u < kRecheckTM; u++)
                hist_add_wave(hist, (v[u] >> sh) & 255u,
                              i0 + u * NT + tid < n && (v[u] & msk) == pre);
        }
        __syncthreads();
        if (wv == 0) {
            int c[4], t = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                c[e] = hist[4 * lane + e];
                t += c[e];
            }
            int inc = t;
            for (int o = 1; o < 64; o <<= 1) {
                const int x = __shfl_up(inc, o);
                if (lane >= o) inc += x;
            }
            int below = inc - t;
            if (below < kr && kr <= inc) {
                int e = 0;
                while (below + c[e] < kr) below += c[e++];
                c2[0] = 4 * lane + e;
                c2[1] = below;
            }
        }
        __syncthreads();
        pre |= (uint32_t)c2[0] << sh;
        msk |= 255u << sh;
        kr -= c2[1];
        __syncthreads();
    }
    return pre;
}

// block_radix_kth over V values per thread held in registers, value u of
// thread t being entry u * NT + t of n (the padding value ~0 counts as a
// value where entries u * NT .. u * NT + NT - 1 are partly real; k must not
// exceed n).
template <int NT, int V>
__device__ __forceinline__ uint32_t block_radix_kth_regs(const uint32_t (&rv)[V], int n, int k,
                                                         int* hist, int* c2) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint32_t pre = 0u, msk = 0u;
    int kr = k;
    for (int sh = 24; sh >= 0; sh -= 8) {
        for (int i = tid; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < V; u++)
            if (u * NT < n) hist_add_wave(hist, (rv[u] >> sh) & 255u, (rv[u] & msk) == pre);
        __syncthreads();
        if (wv == 0) {
            int c[4], t = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                c[e] = hist[4 * lane + e];
                t += c[e];
            }
            int inc = t;
            for (int o = 1; o < 64; o <<= 1) {
                const int x = __shfl_up(inc, o);
                if (lane >= o) inc += x;
            }
            int below = inc - t;
            if (below < kr && kr <= inc) {
                int e = 0;
                while (below + c[e] < kr) below += c[e++];
                c2[0] = 4 * lane + e;
                c2[1] = below;
            }
        }
        __syncthreads();
        pre |= (uint32_t)c2[0] << sh;
        msk |= 255u << sh;
        kr -= c2[1];
        __syncthreads();
    }
    return pre;
}

// Words of the re-check's entry buffer: its [kRecheckCHM][M + 1] entries, or
// more when the refine's short-list arrays (keys, slots, positions and
// primary distances of ck candidates), residual codebooks (rck floats) and
// padded query, which take the place of the survivor buffers and the entry
// buffer once the short list is selected, need the room.
__host__ __device__ inline int recheck_ebuf_words(int M, int ck, int rck, int d, bool fuse) {
    const int refine = 5 * ck + rck + d + d / 32 + 1;   // words, keys counted twice
    const int spare = kRecheckCap * 4;                   // surv, mp and mc, in words
    const int own = kRecheckCHM * (M + 1);
    return fuse && refine - spare > own ? refine - spare : own;
}

// Short lists up to this length are refined inside the re-check; longer ones
// go to refine_topk_kernel (config 2, ck 100: 847 k queries/s with the refine
// inside against 827 k; config 5, ck 400: 193 k with it against 217 k).
constexpr int kMfmaFuseMaxCk = 128;
bool mfma_fuses_refine(int ck) { return ck <= kMfmaFuseMaxCk; }

// One workgroup per query: the ck-th smallest of the query's tile minima
// (written by the scan) bounds the members, one pass over the query's I
// values collects the candidates that can be members, the ck-th smallest I
// among them tightens the bound, the members' distances are recomputed in
// the reference's order, and the exact top-ck by (dist, position) is
// selected.  FUSE: the short list is refined in place (refine_short_list, as
// refine_topk_kernel refines a merged one) and out_d / out_i get the query's
// k best; else it goes to partial[segment][ck] (one segment per query) for
// refine_topk_kernel.
template <int NT, bool FUSE>
__global__ void __launch_bounds__(NT)
mfma_recheck_kernel(const uint32_t* __restrict__ dump, const uint32_t* __restrict__ tmin,
                    MfmaWs w, const int32_t* __restrict__ qtot,
                    const float* __restrict__ q_rot, int d, int Ds, int K1D, int bpd,
                    const float* __restrict__ c1d, int M, const int32_t* __restrict__ probes,
                    const int32_t* __restrict__ gofs, int P, const int4* __restrict__ ldesc,
                    const uint8_t* __restrict__ codes_t, const uint8_t* __restrict__ rows, int ck,
                    int k, const float* __restrict__ res_c1d, int Kr, int RC, int Br, int bpv,
                    const uint8_t* __restrict__ list_res, const float* __restrict__ list_corr,
                    const int32_t* __restrict__ list_ids, float* __restrict__ out_d,
                    int32_t* __restrict__ out_i, unsigned long long* __restrict__ topck_dbg,
                    unsigned long long* __restrict__ partial,
                    int32_t* __restrict__ partial_slot) {
    constexpr int NW = NT / 64;
    extern __shared__ __align__(16) unsigned char smem[];
    StreamSel S;
    unsigned char* p0 = stream_carve<NT>(smem, ck, &S);
    unsigned long long* surv = (unsigned long long*)p0;        // [kRecheckCap]
    int* mp = (int*)(surv + kRecheckCap);                      // [kRecheckCap] member pool slot
    int* mc = mp + kRecheckCap;                                // [kRecheckCap] member tag
    float* ebuf = (float*)(mc + kRecheckCap);                  // [CHM][M + 1] (or more)
    float* sq = ebuf + recheck_ebuf_words(M, ck, RC * Kr, d, FUSE);  // [d]
    float* sc1d = sq + d;                                      // [K1D]
    int* meta = (int*)(sc1d + K1D);                            // [P][4]
    int* sg = meta + 4 * P;                                    // [P + 1]
    int* wsum = sg + P + 1;                                    // [NW]
    int* ctl = wsum + NW;                                      // [4]
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const unsigned long long lt = (1ull << lane) - 1ull;
    JHQ_PHASE_DECL
    // the query's row: first dump slot and tiles (x, z); y, its segment
    // among the queries with candidates, is counted where it is needed.  The
    // workgroups clear the batch's list hash for the next batch on their way
    // out (the tile kernel, its only reader, has finished)
    const int4 qi = make_int4(b * w.perq, 0, qtot[b], 0);
    auto clear_hash = [&]() {
        const int B = gridDim.x, h0 = (int)((int64_t)b * w.H / B);
        const int h1 = (int)((int64_t)(b + 1) * w.H / B);
        for (int h = h0 + tid; h < h1; h += NT) w.hs[h] = make_int4(-1, 0, 0, 0);
    };
    const MfmaQS* qs = w.qs;
    if (qi.z == 0) {
        clear_hash();
        // no candidates: no neighbours (without FUSE, refine sees no segment)
        if (!FUSE) return;
        for (int r = tid; r < k; r += NT) {
            out_d[(int64_t)b * k + r] = __builtin_huge_valf();
            out_i[(int64_t)b * k + r] = -1;
        }
        if (topck_dbg)
            for (int r = tid; r < ck; r += NT) topck_dbg[(int64_t)b * ck + r] = ~0ull;
        return;
    }
    // the probed lists' ids are requested first (their descriptors depend on
    // them), then pass 1's tile minima (when they go through LDS), then the
    // query, codebook and probe table (d <= NT, P < NT): a load waits only
    // for those issued before it, so the descriptors and the LDS stores do
    // not wait for the tile minima
    // (list ids are non-negative: an unsigned index, whose widening does not
    // wait for the load)
    const int prb = tid < P ? probes[(int64_t)b * P + tid] : 0;
    const uint32_t* tm = tmin + qi.x / kGroup;
    const int nt = qi.z;
    const bool tiles_in_lds = nt >= ck && nt <= 2 * kRecheckCap;
    constexpr int TU = (2 * kRecheckCap + NT - 1) / NT;
    uint32_t tv[TU];
    if (tiles_in_lds) {
#pragma unroll
        for (int u = 0; u < TU; u++) tv[u] = tid + u * NT < nt ? tm[tid + u * NT] : ~0u;
    }
    const float qv = tid < d ? q_rot[(int64_t)b * d + tid] : 0.0f;
    const float cv = tid < K1D ? c1d[tid] : 0.0f;
    const int gv = tid <= P ? gofs[(int64_t)b * (P + 1) + tid] : 0;
    // the residual codebooks for the refine, requested now as well
    const float rcv = FUSE && tid < RC * Kr ? res_c1d[tid] : 0.0f;
    const MfmaQS Q = qs[b];
    const int4 Lv = tid < P ? ldesc[(uint32_t)prb] : make_int4(0, 0, 0, 0);
    const int64_t n = (int64_t)qi.z * kGroup;
    const uint32_t* row = dump + qi.x;
    const uint4* row4 = (const uint4*)row;
    const int64_t n4 = n / 4;
    if (tid < d) sq[tid] = qv;
    if (tid < K1D) sc1d[tid] = cv;
    if (tid < P) {
        meta[4 * tid] = Lv.x;
        meta[4 * tid + 1] = Lv.y;
        meta[4 * tid + 2] = Lv.z;
        meta[4 * tid + 3] = Lv.w;
    }
    if (tid <= P) sg[tid] = gv;
    if (tid == 0) ctl[0] = 0;
    stream_begin<NT>(S);
    // pass 1: an upper bound of the ck-th smallest I from the tile minima
    // (each is an I value of its own tile): with a minimum on every lane, a
    // bound from the waves' lane minima; otherwise their exact ck-th
    // smallest, from an LDS copy when they fit there, else from registers or
    // global memory
    uint32_t That = ~0u;
    if (tiles_in_lds) {
        uint32_t* tl = (uint32_t*)mp;  // mp and mc, free until the members
        uint32_t lmin = ~0u;
#pragma unroll
        for (int u = 0; u < TU; u++) {
            if (tid + u * NT < nt) tl[tid + u * NT] = tv[u];
            lmin = min(lmin, tv[u]);
        }
        if (nt >= NT && ck <= 64 * NW) {
            // every lane holds a tile minimum: each wave takes the r-th
            // smallest of its lane minima (r = ceil(ck / waves), so r lanes,
            // r distinct tiles, hold an I at or below it) and the largest of
            // those bounds the ck-th smallest I: no block-wide rounds
            const uint32_t wk = wave_kth_u32(lmin, (ck + NW - 1) / NW);
            if (lane == 0) wsum[wv] = (int)wk;
            __syncthreads();
            That = 0u;
#pragma unroll
            for (int w2 = 0; w2 < NW; w2++) That = max(That, (uint32_t)wsum[w2]);
        } else {
            __syncthreads();
            That = block_radix_kth<NT>([&](int i) { return tl[i]; }, nt, ck, (int*)ebuf, ctl + 2);
        }
    } else if (nt >= ck && nt <= kRecheckTR * NT) {
        // more tile minima than LDS holds (a per-wave bound here leaves
        // thousands of candidates with nprobe 32 over 4096 lists and ck 400):
        // read once into registers, all loads in flight, and ranked there
        uint32_t rv[kRecheckTR];
#pragma unroll
        for (int u = 0; u < kRecheckTR; u++) {
            const int i = u * NT + tid;
            rv[u] = i < nt ? tm[i] : ~0u;
        }
        __syncthreads();
        That = block_radix_kth_regs<NT, kRecheckTR>(rv, nt, ck, (int*)ebuf, ctl + 2);
    } else if (nt >= ck) {
        // more still: read from global memory in each round, the loads
        // batched
        __syncthreads();
        That = block_radix_kth_glob<NT>(tm, nt, ck, (int*)ebuf, ctl + 2);
    } else {
        __syncthreads();
    }
    const uint32_t thr1 = That == ~0u ? 0xfffffffeu : mfma_member_bound(Q, That, M);
    JHQ_PHASE(1);
    // pass 2: the candidates at or below a bound (they include the ck
    // smallest I values and every member), into surv
    auto collect = [&](uint32_t thr) {
        if (tid == 0) ctl[0] = 0;
        __syncthreads();
        for (int64_t i0 = 0; i0 < n4; i0 += kRecheckLPT * NT) {
            uint4 v4[kRecheckLPT];
#pragma unroll
            for (int u = 0; u < kRecheckLPT; u++) {
                const int64_t i = i0 + u * NT + tid;
                v4[u] = i < n4 ? row4[i] : make_uint4(~0u, ~0u, ~0u, ~0u);
            }
#pragma unroll
            for (int u = 0; u < kRecheckLPT; u++) {
                const uint32_t vv[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
                const bool any = __ballot(vv[0] <= thr || vv[1] <= thr || vv[2] <= thr ||
                                          vv[3] <= thr) != 0ull;
                if (!any) continue;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const bool keep = vv[e] <= thr;
                    const unsigned long long mk = __ballot(keep);
                    if (!mk) continue;
                    int at = 0;
                    if (lane == 0) at = atomicAdd(&ctl[0], __popcll(mk));
                    at = __shfl(at, 0);
                    const int pos = at + __popcll(mk & lt);
                    const int64_t i = 4 * (i0 + u * NT + tid) + e;
                    if (keep && pos < kRecheckCap)
                        surv[pos] = ((unsigned long long)vv[e] << 32) | (uint32_t)i;
                }
            }
        }
        __syncthreads();
        return ctl[0];
    };
    // the tiles whose minimum is at or below thr into qlist (at most cap
    // listed; returns the count), tile minima from LDS when they fit there,
    // else from global memory
    auto list_tiles = [&](uint32_t thr, int* qlist, int cap) __attribute__((always_inline)) {
        // (two loops, not one pointer that may point to either memory: a
        // load through such a pointer is a flat load, which every LDS wait
        // then also waits for)
        using lds_u32 = const __attribute__((address_space(3))) uint32_t;
        lds_u32* tl = (lds_u32*)mp;
        if (tid == 0) ctl[1] = 0;
        __syncthreads();
        for (int t0 = 0; t0 < nt; t0 += kRecheckTM * NT) {
            uint32_t mv[kRecheckTM];
            if (tiles_in_lds) {
#pragma unroll
                for (int u = 0; u < kRecheckTM; u++) {
                    const int t = t0 + u * NT + tid;
                    mv[u] = t < nt ? tl[t] : ~0u;
                }
            } else {
#pragma unroll
                for (int u = 0; u < kRecheckTM; u++) {
                    const int t = t0 + u * NT + tid;
                    mv[u] = t < nt ? tm[t] : ~0u;
                }
            }
#pragma unroll
            for (int u = 0; u < kRecheckTM; u++) {
                const int t = t0 + u * NT + tid;
                const bool q = t < nt && mv[u] <= thr;
                const unsigned long long mk = __ballot(q);
                if (!mk) continue;
                int at = 0;
                if (lane == 0) at = atomicAdd(&ctl[1], __popcll(mk));
                at = __shfl(at, 0);
                const int pos = at + __popcll(mk & lt);
                if (q && pos < cap) qlist[pos] = t;
            }
        }
        __syncthreads();
        return ctl[1];
    };
    // only the tiles whose minimum is at or below the bound can hold a
    // candidate at or below it: their 16 values are read (four tiles per
    // wave, kRecheckTPL per lane in flight) instead of the whole row
    auto collect_tiles = [&](uint32_t thr, int& ns_out) {
        int* qlist = (int*)ebuf;  // free until the members' entries
        if (tid == 0) ctl[0] = 0;
        const int nqt = list_tiles(thr, qlist, kRecheckQCap);
        if (nqt > kRecheckQCap) return false;
        for (int i0 = wv * 4; i0 < nqt; i0 += NW * 4 * kRecheckTPL) {
            uint32_t v[kRecheckTPL];
            int ti[kRecheckTPL];
#pragma unroll
            for (int u = 0; u < kRecheckTPL; u++) {
                const int qi2 = i0 + u * NW * 4 + (lane >> 4);
                ti[u] = qi2 < nqt ? qlist[qi2] : -1;
                v[u] = ti[u] >= 0 ? row[(int64_t)ti[u] * kGroup + (lane & 15)] : ~0u;
            }
#pragma unroll
            for (int u = 0; u < kRecheckTPL; u++) {
                const bool keep = v[u] <= thr;
                const unsigned long long mk = __ballot(keep);
                if (!mk) continue;
                int at = 0;
                if (lane == 0) at = atomicAdd(&ctl[0], __popcll(mk));
                at = __shfl(at, 0);
                const int pos = at + __popcll(mk & lt);
                if (keep && pos < kRecheckCap)
                    surv[pos] = ((unsigned long long)v[u] << 32) |
                                (uint32_t)(ti[u] * kGroup + (lane & 15));
            }
        }
        __syncthreads();
        ns_out = ctl[0];
        return true;
    };
    int ns = 0;
    if (!(nt >= ck && collect_tiles(thr1, ns))) ns = collect(thr1);
    uint32_t thr = thr1;
    JHQ_PHASE(12);
#ifdef JHQ_PHASE_TIMING
    ph_acc[14] += (unsigned long long)ns;
#endif
    if (ns > kRecheckCap && n >= ck) {
        // the tile minima left too many candidates: the exact ck-th smallest
        // I, then the pass again.  The ck-th value lies in the tiles whose
        // minimum is at most That (the ck-th smallest minimum): their values
        // (about 16 ck) are radix-selected in registers when they fit, else
        // the whole row is (padding slots hold the largest value)
        bool exact = false;
        int n1 = -1;
        {
            int* qlist = (int*)ebuf + 256;  // after the radix histogram
            n1 = list_tiles(That, qlist, kRecheckQCap1);
            if (n1 <= kRecheckQCap1 && 16 * n1 <= kRecheckRegV * NT) {
                uint32_t rv[kRecheckRegV];
#pragma unroll
                for (int u = 0; u < kRecheckRegV; u++) {
                    const int idx = u * NT + tid;
                    rv[u] = idx < 16 * n1 ? row[(int64_t)qlist[idx >> 4] * kGroup + (idx & 15)]
                                          : ~0u;
                }
                const uint32_t t1 = block_radix_kth_regs<NT, kRecheckRegV>(rv, 16 * n1, ck,
                                                                           (int*)ebuf, ctl + 2);
                thr = min(thr1, mfma_member_bound(Q, t1, M));
                exact = true;
            }
        }
        if (!exact)
            thr = min(thr1, mfma_member_bound(
                                Q, block_radix_kth_row<NT>(row4, n4, ck, (int*)ebuf, ctl + 2), M));
        JHQ_PHASE(13);
#ifdef JHQ_PHASE_TIMING
        ph_acc[15] += (unsigned long long)(n1 + 1);
#endif
        if (!(nt >= ck && collect_tiles(thr, ns))) ns = collect(thr);
    }
    JHQ_PHASE(2);
#ifdef JHQ_PHASE_TIMING
    ph_acc[7] += (unsigned long long)ns;
#endif
    // the exact distance of the candidate in slot i of the query's row
    auto locate = [&](int i, int& pp, int& cc) {
        const int g = i / kGroup;
        int lo = 0, hi = P - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (sg[mid] <= g) lo = mid;
            else hi = mid - 1;
        }
        pp = lo;
        cc = i - sg[lo] * kGroup;
    };
    const int kmask = K1D - 1;
    auto entry = [&](int pp, int cc, int m) {
        const uint8_t v = codes_t[(int64_t)meta[4 * pp] * M + (int64_t)m * meta[4 * pp + 1] + cc];
        float e = 0.0f;
        for (int k = 0; k < Ds; k++) {
            const float df = sq[m * Ds + k] - sc1d[(v >> (k * bpd)) & kmask];
            e = fmaf(df, df, e);
        }
        return e;
    };
    int kk = 0;
    bool by_member = false;
    if (ns <= kRecheckCap) {
        // the ck-th smallest I among the survivors, then the members
        uint32_t thr2 = thr;
        if (ns >= ck) {
            const uint32_t pre = block_radix_kth<NT>(
                [&](int i) { return (uint32_t)(surv[i] >> 32); }, ns, ck, mp, ctl + 2);
            thr2 = min(thr, mfma_member_bound(Q, pre, M));
        }
        JHQ_PHASE(3);
        if (tid == 0) ctl[1] = 0;
        __syncthreads();
        for (int i0 = 0; i0 < ns; i0 += NT) {
            const int i = i0 + tid;
            const bool keep = i < ns && (uint32_t)(surv[i] >> 32) <= thr2;
            const unsigned long long mk = __ballot(keep);
            int at = 0;
            if (lane == 0 && mk) at = atomicAdd(&ctl[1], __popcll(mk));
            at = __shfl(at, 0);
            if (keep) {
                int pp, cc;
                locate((int)(uint32_t)surv[i], pp, cc);
                // the member's pool slot and its tag (canonical position)
                mp[at + __popcll(mk & lt)] = meta[4 * pp] + cc;
                mc[at + __popcll(mk & lt)] = meta[4 * pp + 3] + cc;
            }
        }
        __syncthreads();
        const int nm = ctl[1];
        JHQ_PHASE(4);
#ifdef JHQ_PHASE_TIMING
        ph_acc[6] += (unsigned long long)nm;
#endif
        // member keys replace the survivors in surv.  Thread t computes
        // subspace t % M of members t / M, t / M + NT / M, ... (its query
        // values in registers); every code byte of a round is requested
        // before the first is used, from the row-major copy (a member's M
        // bytes are one run, against M cache lines of the code-major
        // blocks); member rows of the entries are padded to M + 1 words, so
        // both the writes and the in-order sums of a member row are free of
        // bank conflicts
        constexpr int EPT = kRecheckCHM * 128 / NT;  // entries per thread (M <= 128)
        const int me = tid % M, mstep = NT / M;
        float qm[8];
#pragma unroll
        for (int k = 0; k < 8; k++) qm[k] = sq[me * 8 + k];  // Ds == 8
        const float cl0 = sc1d[0], cl1 = sc1d[1];             // K1D == 2, bpd == 1
        for (int c0 = 0; c0 < nm; c0 += kRecheckCHM) {
            const int nc = min(kRecheckCHM, nm - c0);
            // every lane loads (rows past the chunk's end repeat its last
            // member) into a register of its own, so that all EPT loads are
            // in flight before the first wait
            uint32_t cb[EPT];
#pragma unroll
            for (int u = 0; u < EPT; u++) {
                // a member's row is one run: a wave reads 64 of its bytes
                const int jj = min(tid / M + u * mstep, nc - 1);
                cb[u] = rows[(int64_t)mp[c0 + jj] * M + me];
            }
            // one-bit digits (the pre-scan's shape): the level is a select
            // between the two codebook values, not an LDS lookup
#pragma unroll
            for (int u = 0; u < EPT; u++) {
                const int jj = tid / M + u * mstep;
                if (jj < nc) {
                    float e = 0.0f;
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const float df = qm[k] - (((cb[u] >> k) & 1u) ? cl1 : cl0);
                        e = fmaf(df, df, e);
                    }
                    ebuf[jj * (M + 1) + me] = e;
                }
            }
            JHQ_PHASE(8);
            __syncthreads();
            JHQ_PHASE(9);
            if (tid < nc) {
                float acc = 0.0f;
                for (int m = 0; m < M; m++) acc += ebuf[tid * (M + 1) + m];
                surv[c0 + tid] = ((unsigned long long)f2ord(acc) << 32) | (uint32_t)mc[c0 + tid];
            }
            __syncthreads();
        }
        JHQ_PHASE(5);
        kk = min(ck, nm);
        // (S.kidx: each selected member's index, when the ranking path ran)
        if (kk > 0) by_member = select_keys<NT>(surv, nm, kk, S.kout, S.kidx, S.ktmp, S.st, S.kidx);
        JHQ_PHASE(11);
    } else {
        // more survivors than fit (ties at the bound): every candidate at or
        // below it, exact distances one per thread, streamed through the
        // selection
        for (int64_t r0 = 0; r0 < n; r0 += NT) {
            const int64_t i = r0 + tid;
            uint32_t o[1] = {~0u}, tg[1] = {~0u};
            if (i < n && row[i] <= thr) {
                int pp, cc;
                locate((int)i, pp, cc);
                float acc = 0.0f;
                for (int m = 0; m < M; m++) acc += entry(pp, cc, m);
                o[0] = f2ord(acc);
                tg[0] = (uint32_t)(meta[4 * pp + 3] + cc);
            }
            stream_round<NT, 1>(S, ck, o, tg);
        }
        kk = stream_end<NT>(S, ck);
    }
    __syncthreads();
    if (!FUSE) {
        clear_hash();
        // the short list and its pool slots (the probe whose canonical
        // range holds the tag) as the query's one segment: the number of
        // earlier queries with candidates
        int seg = 0;
        for (int i = lane; i < b; i += 64) seg += qtot[i] > 0 ? 1 : 0;
        for (int o = 32; o > 0; o >>= 1) seg += __shfl_xor(seg, o);
        for (int i = tid; i < ck; i += NT) {
            int32_t slot = -1;
            if (i < kk) {
                const int tag = (int)(uint32_t)(S.kout[i] & 0xffffffffull);
                for (int q = 0; q < P; q++)
                    if (tag >= meta[4 * q + 3] && tag - meta[4 * q + 3] < meta[4 * q + 2])
                        slot = meta[4 * q] + (tag - meta[4 * q + 3]);
            }
            partial[(int64_t)seg * ck + i] = i < kk ? S.kout[i] : ~0ull;
            partial_slot[(int64_t)seg * ck + i] = slot;
        }
        JHQ_PHASE(0);
        JHQ_PHASE_FLUSH(3);
        return;
    }
    // the refine's arrays replace the survivor and entry buffers: pool slots
    // of the short list (the probe whose canonical range holds the tag), the
    // residual codebooks, the query with one pad word per 32 and, when the
    // rest of those buffers holds it, the table of squared differences
    unsigned long long* fkeys = (unsigned long long*)p0;
    int* kslot = (int*)(fkeys + ck);
    int* cpos = kslot + ck;
    float* cprim = (float*)(cpos + ck);
    float* rcb = cprim + ck;
    float* sqp = rcb + RC * Kr;
    float* tabp = sqp + d + d / 32 + 1;
    if (tabp + refine_tab_words(d) > sq) tabp = nullptr;
    for (int i = tid; i < kk; i += NT) {
        int32_t slot = -1;
        if (by_member) {
            // the member's pool slot (mp is intact until the refine's table)
            slot = mp[S.kidx[i]];
        } else {
            const int tag = (int)(uint32_t)(S.kout[i] & 0xffffffffull);
            for (int q = 0; q < P; q++)
                if (tag >= meta[4 * q + 3] && tag - meta[4 * q + 3] < meta[4 * q + 2])
                    slot = meta[4 * q] + (tag - meta[4 * q + 3]);
        }
        kslot[i] = slot;
    }
    if (RC * Kr <= NT) {
        if (tid < RC * Kr) rcb[tid] = rcv;
    } else {
        for (int i = tid; i < RC * Kr; i += NT) rcb[i] = res_c1d[i];
    }
    for (int i = tid; i < d; i += NT) sqp[i + (i >> 5)] = sq[i];
    __syncthreads();
    JHQ_PHASE(10);
    refine_short_list<NT>(S, kk, ck, k, b, kslot, cpos, cprim, fkeys, sqp, rcb, d, Ds, Kr, RC, Br,
                          bpv, list_res, list_corr, list_ids, out_d, out_i, topck_dbg, tabp);
    clear_hash();
    JHQ_PHASE(0);
    JHQ_PHASE_FLUSH(3);
}

static size_t mfma_recheck_lds(int M, int d, int P, int ck, int K1D, int B, int rck) {
    return stream_lds_bytes(kRecheckNT, ck) + (size_t)kRecheckCap * (8 + 4 + 4) +
           (size_t)recheck_ebuf_words(M, ck, rck, d, mfma_fuses_refine(ck)) * 4 +
           (size_t)d * 4 + (size_t)K1D * 4 +
           (size_t)(4 * P + P + 1) * 4 + (kRecheckNT / 64) * 4 + 16 + 64;
}

bool mfma_scan_ok(int M, int d, int Ds, int K1D, int bpd, int B, int P, int ck, int rck) {
    if (K1D != 2 || bpd != 1 || Ds != 8 || d != 8 * M) return false;
    if (M % 16 != 0 || M < 16 || M > 128 || d > kRecheckNT || P >= kRecheckNT) return false;
    if (B < 1 || P < 1 || (int64_t)B * P > kMfmaMaxBP || ck < 1 || ck > kRecheckCap) return false;
    return mfma_recheck_lds(M, d, P, ck, K1D, B, rck) <= (size_t)kLdsBytes - 1024;
}

static int mfma_scan_waves(int num_cu, int B, int P) {
#ifdef JHQ_MFMA_WPC
    const int wpc = JHQ_MFMA_WPC;  // a fixed count, for measurements
#else
    const int wpc = (int64_t)B * P <= kMfmaFewPairs ? kMfmaWpcFew : kMfmaWpcMany;
#endif
    return std::max(1, num_cu) * wpc;
}

size_t mfma_scan_bytes(int B, int P, int M, int num_cu) {
    (void)num_cu;
    return mfma_carve(B, P, M, nullptr, nullptr);
}

hipError_t mfma_hash_clear(int Bcap, int P, int M, unsigned char* ws, size_t ws_bytes,
                           hipStream_t s) {
    MfmaWs w;
    if (!ws || ((uintptr_t)ws & 255) || mfma_carve(Bcap, P, M, ws, &w) > ws_bytes)
        return hipErrorInvalidValue;
    // every slot (-1, 0, -1, 0): free, no pairs (its size is set on use)
    return fill_u64((unsigned long long*)w.hs, (int64_t)w.H * 2, 0x00000000ffffffffull, s);
}

hipError_t mfma_scan(const float* q_rot, int d, int Ds, int K1D, int bpd, const float* c1d, int B,
                     int M, const int32_t* probes, const int32_t* gofs, const int32_t* qtot, int P,
                     const int4* ldesc, const uint8_t* codes_t, const uint8_t* rows, int ck,
                     uint32_t* dump, int64_t dump_slots, unsigned char* ws, size_t ws_bytes,
                     int k, const float* res_c1d, int Kr, int RC, int Br, int bpv,
                     const uint8_t* list_res, const float* list_corr, const int32_t* list_ids,
                     float* out_d, int32_t* out_i, unsigned long long* topck_dbg,
                     unsigned long long* partial, int32_t* partial_slot, int num_cu,
                     int Bcap, hipStream_t s) {
    const bool fuse = mfma_fuses_refine(ck);
    if (!mfma_scan_ok(M, d, Ds, K1D, bpd, B, P, ck, RC * Kr) || !dump || !rows ||
        dump_slots % 16 != 0 || k < 1 || k > ck || (!fuse && (!partial || !partial_slot)))
        return hipErrorInvalidValue;
    // tile minima after the candidate slots
    uint32_t* tmin = dump + dump_slots;
    MfmaWs w;
    if ((int64_t)Bcap * P > kMfmaMaxBP || !mfma_ws(B, Bcap, P, M, ws, ws_bytes, dump_slots, &w))
        return hipErrorInvalidValue;
    const int nwaves = mfma_scan_waves(num_cu, B, P);
    using SFn = void (*)(MfmaWs, const int4*, const uint8_t*, uint32_t*, uint32_t*);
    SFn f = M == 16 ? mfma_scan_kernel<16> : M == 32 ? mfma_scan_kernel<32>
          : M == 48 ? mfma_scan_kernel<48> : M == 64 ? mfma_scan_kernel<64>
          : M == 80 ? mfma_scan_kernel<80> : M == 96 ? mfma_scan_kernel<96>
          : M == 112 ? mfma_scan_kernel<112> : mfma_scan_kernel<128>;
    hipLaunchKernelGGL(f, dim3(nwaves / 4), dim3(256), 0, s, w, ldesc, rows, dump, tmin);
    const size_t lr = mfma_recheck_lds(M, d, P, ck, K1D, B, RC * Kr);
    static const int mxf = allow_max_lds((const void*)mfma_recheck_kernel<kRecheckNT, true>);
    static const int mxs = allow_max_lds((const void*)mfma_recheck_kernel<kRecheckNT, false>);
    if ((int)lr > (fuse ? mxf : mxs)) return hipErrorInvalidValue;
    if (fuse)
        hipLaunchKernelGGL((mfma_recheck_kernel<kRecheckNT, true>), dim3(B), dim3(kRecheckNT), lr,
                           s, dump, tmin, w, qtot, q_rot, d, Ds, K1D, bpd, c1d, M, probes,
                           gofs, P, ldesc, codes_t, rows, ck, k, res_c1d, Kr, RC, Br, bpv,
                           list_res, list_corr, list_ids, out_d, out_i, topck_dbg, partial,
                           partial_slot);
    else
        hipLaunchKernelGGL((mfma_recheck_kernel<kRecheckNT, false>), dim3(B), dim3(kRecheckNT), lr,
                           s, dump, tmin, w, qtot, q_rot, d, Ds, K1D, bpd, c1d, M, probes,
                           gofs, P, ldesc, codes_t, rows, ck, k, res_c1d, Kr, RC, Br, bpv,
                           list_res, list_corr, list_ids, out_d, out_i, topck_dbg, partial,
                           partial_slot);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Search stages in the reference's own data layout, for the kernel-granular
// C-ABI (stage-wise parity and callers of the reference's kernels): a global
// byte LUT [B][M][256], primary codes transposed to [M][N] with list_offsets
// (v14/jhq_gpu_index.cu:488-517), per-query probe ids and prefix offsets.
// Every stage follows the reference's arithmetic order; selection is exact
// by (dist, position) and (dist, id) (jhq_v3_ivf/search.cu:22-25).
// ---------------------------------------------------------------------------

// build_byte_lut_kernel (v14/search.cu:65-91): lut[b][m][v] = sum over
// k < Ds of (q[b][m*Ds+k] - c1d[digit_k(v)])^2, one fma per k, k ascending.
__global__ void stage_lut_kernel(const float* __restrict__ q_rot, const float* __restrict__ c1d,
                                 float* __restrict__ lut, int B, int d, int M, int Ds, int K1D,
                                 int bpd) {
    const int64_t total = (int64_t)B * M * 256;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = i / ((int64_t)M * 256);
        const int loc = (int)(i - b * (int64_t)M * 256);
        const int m = loc >> 8, v = loc & 255;
        const float* qm = q_rot + b * d + (int64_t)m * Ds;
        float acc = 0.0f;
        for (int k = 0; k < Ds && k < 8; k++) {
            const float df = qm[k] - c1d[(v >> (k * bpd)) & (K1D - 1)];
            acc = fmaf(df, df, acc);
        }
        lut[i] = acc;
    }
}

// scan_ivf_coalesced_kernel (v14/search.cu:105-195) with exact selection: one
// workgroup per query; candidate t of the probed lists laid end to end (probe
// p holds t in [offs[p], offs[p+1])) is position list_offsets[probe] +
// t - offs[p]; dist = sum over m ascending of lut[m][code_m], the codes read
// from primary_t[m*N + pos] (consecutive threads, consecutive positions).
// The query's top-ck by (dist, pos) goes to out_d / out_p ascending, unfilled
// = (+inf, -1).  LUT_LDS: the query's LUT is copied to LDS first (M <= ~150).
template <int NT, bool LUT_LDS>
__global__ void __launch_bounds__(NT)
stage_scan_kernel(const float* __restrict__ byte_lut, const int32_t* __restrict__ probe_ids,
                  const int32_t* __restrict__ probe_offsets, const int32_t* __restrict__ list_offsets,
                  const uint8_t* __restrict__ primary_t, const int32_t* __restrict__ query_total,
                  float* __restrict__ out_d, int32_t* __restrict__ out_p, int nprobe, int M,
                  int64_t N, int ck) {
    constexpr int CPT = 4;
    extern __shared__ __align__(16) unsigned char smem[];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float* glut = byte_lut + (int64_t)b * M * 256;
    float* llut = (float*)smem;
    StreamSel S;
    int32_t* soff = (int32_t*)stream_carve<NT>(smem + (LUT_LDS ? (size_t)M * 1024 : 0), ck, &S);
    int32_t* sbase = soff + nprobe + 1;
    if (LUT_LDS)
        for (int i = tid; i < M * 256; i += NT) llut[i] = glut[i];
    for (int i = tid; i <= nprobe; i += NT) soff[i] = probe_offsets[(int64_t)b * (nprobe + 1) + i];
    for (int i = tid; i < nprobe; i += NT) sbase[i] = list_offsets[probe_ids[(int64_t)b * nprobe + i]];
    stream_begin<NT>(S);
    __syncthreads();
    const float* L = LUT_LDS ? llut : glut;
    const int total = query_total[b];
    for (int base = 0; base < total; base += NT * CPT) {
        uint32_t o[CPT], tg[CPT];
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int t = base + j * NT + tid;
            o[j] = ~0u;
            tg[j] = 0u;
            if (t < total) {
                int lo = 0, hi = nprobe - 1;  // last probe with offs[p] <= t
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (soff[mid] <= t) lo = mid;
                    else hi = mid - 1;
                }
                const int64_t pos = (int64_t)sbase[lo] + (t - soff[lo]);
                float dist = 0.0f;
                for (int m = 0; m < M; m++) dist += L[m * 256 + primary_t[(int64_t)m * N + pos]];
                o[j] = f2ord(dist);
                tg[j] = (uint32_t)pos;
            }
        }
        stream_round<NT, CPT>(S, ck, o, tg);
    }
    const int kk = stream_end<NT>(S, ck);
    for (int i = tid; i < ck; i += NT) {
        const unsigned long long kv = i < kk ? S.kout[i] : ~0ull;
        out_d[(int64_t)b * ck + i] = i < kk ? ord2f((uint32_t)(kv >> 32)) : __builtin_huge_valf();
        out_p[(int64_t)b * ck + i] = i < kk ? (int32_t)(uint32_t)(kv & 0xffffffffull) : -1;
    }
}

// build_residual_lut_batched_kernel + residual_refine_batched_kernel
// (v14/search.cu:198-242), one thread per short-list entry:
// comp = (primary + sum over j ascending of (q[j] - res_c1d[r_j])^2) + corr[pos]
// with each square rounded before it is added (the reference stores them in a
// LUT first); pos < 0 gives +inf.
__global__ void stage_refine_kernel(const float* __restrict__ q_rot,
                                    const float* __restrict__ res_c1d,
                                    const int32_t* __restrict__ topck_pos,
                                    const float* __restrict__ topck_primary,
                                    const uint8_t* __restrict__ list_res,
                                    const float* __restrict__ list_corr, float* __restrict__ comp,
                                    int B, int ck, int d, int Br, int bpv) {
    const int64_t total = (int64_t)B * ck;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int32_t pos = topck_pos[i];
        if (pos < 0) {
            comp[i] = __builtin_huge_valf();
            continue;
        }
        const float* q = q_rot + (i / ck) * d;
        const uint8_t* rc = list_res + (int64_t)pos * bpv;
        float dres = 0.0f;
        for (int j = 0; j < d; j++) {
            const int ri = (Br == 4) ? ((j & 1) ? (rc[j >> 1] >> 4) : (rc[j >> 1] & 0x0F)) : rc[j];
            const float df = q[j] - res_c1d[ri];
            const float sq = df * df;
            dres = dres + sq;
        }
        comp[i] = (topck_primary[i] + dres) + list_corr[pos];
    }
}

// batched_topk_final_kernel (v14/search.cu:244-291) with exact (dist, id)
// order: per query the k smallest composite distances among entries with
// pos >= 0 and a finite distance, id = list_ids[pos]; unfilled = (+inf, -1).
// Positions within a row are distinct (as the scan emits them).
template <int NT>
__global__ void __launch_bounds__(NT)
stage_final_kernel(const float* __restrict__ comp, const int32_t* __restrict__ topck_pos,
                   const int32_t* __restrict__ list_ids, float* __restrict__ out_d,
                   int32_t* __restrict__ out_i, int ck, int k) {
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned long long* keys = (unsigned long long*)smem;  // [ck]
    unsigned long long* kout = keys + ck;                  // [k]
    unsigned long long* ktmp = kout + k;                   // [k]
    SelState* st = (SelState*)(ktmp + k);
    int* kidx = (int*)(st + 1);                            // [k]
    int* cnt = kidx + k;
    const int b = blockIdx.x, tid = threadIdx.x;
    if (tid == 0) *cnt = 0;
    __syncthreads();
    for (int c = tid; c < ck; c += NT) {
        const int32_t pos = topck_pos[(int64_t)b * ck + c];
        const float dv = comp[(int64_t)b * ck + c];
        if (pos >= 0 && dv < __builtin_huge_valf()) {
            const int at = atomicAdd(cnt, 1);
            keys[at] = ((unsigned long long)f2ord(dv) << 32) | (uint32_t)list_ids[pos];
        }
    }
    __syncthreads();
    const int n = *cnt;
    const int kf = n < k ? n : k;
    if (kf > 0) select_keys<NT>(keys, n, kf, kout, kidx, ktmp, st);
    for (int r = tid; r < k; r += NT) {
        out_d[(int64_t)b * k + r] = r < kf ? ord2f((uint32_t)(kout[r] >> 32)) : __builtin_huge_valf();
        out_i[(int64_t)b * k + r] = r < kf ? (int32_t)(uint32_t)(kout[r] & 0xffffffffull) : -1;
    }
}

static int grid_for(int64_t total, int nt) {
    const int64_t g = (total + nt - 1) / nt;
    return (int)(g < 65536 ? (g > 0 ? g : 1) : 65536);
}

hipError_t stage_byte_lut(const float* q_rot, const float* c1d, float* lut, int B, int d, int M,
                          int Ds, int K1D, int bpd, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    hipLaunchKernelGGL(stage_lut_kernel, dim3(grid_for((int64_t)B * M * 256, 256)), dim3(256), 0,
                       s, q_rot, c1d, lut, B, d, M, Ds, K1D, bpd);
    return hipGetLastError();
}

size_t stage_scan_lds(int M, int nprobe, int ck, bool lut_lds) {
    return (lut_lds ? (size_t)M * 1024 : 0) + stream_lds_bytes(512, ck) + (size_t)(2 * nprobe + 1) * 4;
}

hipError_t stage_scan_topck(const float* byte_lut, const int32_t* probe_ids,
                            const int32_t* probe_offsets, const int32_t* list_offsets,
                            const uint8_t* primary_t, const int32_t* query_total, float* out_d,
                            int32_t* out_p, int B, int nprobe, int M, int64_t N, int ck,
                            hipStream_t s) {
    constexpr int NT = 512;
    if (B <= 0) return hipSuccess;
    static const int mx1 = allow_max_lds((const void*)stage_scan_kernel<NT, true>);
    static const int mx0 = allow_max_lds((const void*)stage_scan_kernel<NT, false>);
    const size_t l1 = stage_scan_lds(M, nprobe, ck, true), l0 = stage_scan_lds(M, nprobe, ck, false);
    if ((int)l1 <= mx1) {
        hipLaunchKernelGGL((stage_scan_kernel<NT, true>), dim3(B), dim3(NT), l1, s, byte_lut,
                           probe_ids, probe_offsets, list_offsets, primary_t, query_total, out_d,
                           out_p, nprobe, M, N, ck);
    } else if ((int)l0 <= mx0) {
        hipLaunchKernelGGL((stage_scan_kernel<NT, false>), dim3(B), dim3(NT), l0, s, byte_lut,
                           probe_ids, probe_offsets, list_offsets, primary_t, query_total, out_d,
                           out_p, nprobe, M, N, ck);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t stage_refine(const float* q_rot, const float* res_c1d, const int32_t* topck_pos,
                        const float* topck_primary, const uint8_t* list_res,
                        const float* list_corr, float* comp, int B, int ck, int d, int Br,
                        int bpv, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    hipLaunchKernelGGL(stage_refine_kernel, dim3(grid_for((int64_t)B * ck, 256)), dim3(256), 0, s,
                       q_rot, res_c1d, topck_pos, topck_primary, list_res, list_corr, comp, B, ck,
                       d, Br, bpv);
    return hipGetLastError();
}

hipError_t stage_final_topk(const float* comp, const int32_t* topck_pos, const int32_t* list_ids,
                            float* out_d, int32_t* out_i, int B, int ck, int k, hipStream_t s) {
    constexpr int NT = 256;
    if (B <= 0) return hipSuccess;
    const size_t lds = (size_t)ck * 8 + (size_t)k * 16 + sizeof(SelState) + (size_t)k * 4 + 16;
    static const int mx = allow_max_lds((const void*)stage_final_kernel<NT>);
    if ((int)lds > mx) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stage_final_kernel<NT>, dim3(B), dim3(NT), lds, s, comp, topck_pos,
                       list_ids, out_d, out_i, ck, k);
    return hipGetLastError();
}

}  // namespace jhq

#ifdef JHQ_PHASE_TIMING
// Copies the phase accumulators [4][4096][8] (ticks of the 100 MHz clock).
extern "C" int jhq_debug_phase_ticks(unsigned long long* out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(jhq::g_phase), sizeof(jhq::g_phase), 0,
                                    hipMemcpyDeviceToHost);
}
#endif
