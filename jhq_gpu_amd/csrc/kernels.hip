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
constexpr int kPhaseBlocks = 4096, kPhases = 8;
__device__ unsigned long long g_phase[3][kPhaseBlocks][kPhases];
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
__device__ SelResult sel_threshold(GetV getv, int n, uint32_t k, SelState* st) {
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

// Exact top-k of n elements by (getv, gett) ascending (gett distinct among
// equal getv).  Writes the k selected elements' keys (getv << 32 | gett) in
// ascending order to keys[0..k) and returns k.  idx must hold k ints and
// tmp/keys k u64 each (8-byte aligned LDS).  Requires 1 <= k <= the number of
// elements whose value is not ~0u.  gett is evaluated only for elements tied
// at the threshold value and for the k selected elements.
template <int NT, class GetV, class GetT>
__device__ int block_topk(GetV getv, GetT gett, int n, int k, int* idx, unsigned long long* tmp,
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
                     int32_t* __restrict__ gofs, int32_t* __restrict__ qtot, bool in_lds) {
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned long long* tmp = (unsigned long long*)smem;
    unsigned long long* sk = tmp + P;
    int* scratch = (int*)(sk + P);
    SelState* st = (SelState*)(scratch + P);
    uint32_t* keys = (uint32_t*)(st + 1);
    const int b = blockIdx.x;
    const float* row = scores + (int64_t)b * nlist;
    JHQ_PHASE_DECL
    if (in_lds) {
        for (int i = threadIdx.x; i < nlist; i += NT) keys[i] = f2ord(row[i]);
        __syncthreads();
        JHQ_PHASE(0);
        block_topk<NT>([&](int i) { return keys[i]; }, [&](int i) { return (uint32_t)i; }, nlist,
                       P, scratch, tmp, sk, st);
    } else {
        block_topk<NT>([&](int i) { return f2ord(row[i]); }, [&](int i) { return (uint32_t)i; },
                       nlist, P, scratch, tmp, sk, st);
    }
    JHQ_PHASE(1);
    for (int r = threadIdx.x; r < P; r += NT) probes[(int64_t)b * P + r] = (int)(uint32_t)sk[r];
    // group counts of the probed lists, gathered in parallel into scratch[]
    for (int r = threadIdx.x; r < P; r += NT) {
        const int l = (int)(uint32_t)sk[r];
        scratch[r] = (list_padoff[l + 1] - list_padoff[l]) / kGroup;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        int32_t* g = gofs + (int64_t)b * (P + 1);
        g[0] = 0;
        for (int r = 0; r < P; r++) {
            acc += scratch[r];
            g[r + 1] = acc;
        }
        qtot[b] = acc;
    }
    JHQ_PHASE(2);
    JHQ_PHASE_FLUSH(1);
}

hipError_t select_probes(const float* scores, int B, int nlist, int P,
                         const int32_t* list_padoff, int32_t* probes, int32_t* gofs,
                         int32_t* qtot, hipStream_t s) {
    constexpr int NT = 256;
    size_t lds = (size_t)P * (8 + 8 + 4) + sizeof(SelState);
    const bool in_lds = lds + (size_t)nlist * 4 <= 64 * 1024;
    if (in_lds) lds += (size_t)nlist * 4;
    hipLaunchKernelGGL(select_probes_kernel<NT>, dim3(B), dim3(NT), lds, s, scores, nlist, P,
                       list_padoff, probes, gofs, qtot, in_lds);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Byte LUT (v14/search.cu:65-91): lut[b][m][v] = sum_k (q[m*Ds+k] - c1d[digit_k(v)])^2
// accumulated with fma in k order.  One workgroup per (m, b), one thread per v.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
byte_lut_kernel(const float* __restrict__ q_rot, int d, int M, int Ds, int K1D, int bpd,
                const float* __restrict__ c1d, float* __restrict__ lut) {
    __shared__ float sq[8];
    __shared__ float sc[256];
    const int m = blockIdx.x, b = blockIdx.y, v = threadIdx.x;
    if (v < Ds) sq[v] = q_rot[(int64_t)b * d + m * Ds + v];
    if (v < K1D) sc[v] = c1d[v];
    __syncthreads();
    float s = 0.0f;
    for (int k = 0; k < Ds; k++) {
        const float df = sq[k] - sc[(v >> (k * bpd)) & (K1D - 1)];
        s = fmaf(df, df, s);
    }
    lut[((int64_t)b * M + m) * 256 + v] = s;
}

hipError_t build_lut(const float* q_rot, int B, int d, int M, int Ds, int K1D, int bpd,
                     const float* c1d, float* lut, hipStream_t s) {
    if (Ds > 8 || K1D > 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(byte_lut_kernel, dim3(M, B), dim3(256), 0, s, q_rot, d, M, Ds, K1D, bpd,
                       c1d, lut);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Chunk plan shared by the scan and merge kernels.  Each query's padded
// candidate groups are cut into chunks of CHg groups, CHg chosen so that the
// batch makes about one chunk per scan workgroup but never more than the
// LDS distance buffer holds.  cpre[b] = first chunk of query b (cpre[B] total).
// ---------------------------------------------------------------------------
template <int NT>
__device__ int chunk_plan(const int32_t* __restrict__ qtot, int B, int capg, int G, int* cpre) {
    // cpre needs B + 2 ints.  Totals gathered in parallel and block-reduced;
    // per-query chunk counts prefix-summed over per-thread segments.
    __shared__ int wsum[NT / 64];
    __shared__ int tot_sh;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (tid == 0) tot_sh = 0;
    __syncthreads();
    int loc = 0;
    for (int b = tid; b < B; b += NT) {
        const int t = qtot[b];
        cpre[b] = t;
        loc += t;
    }
    for (int off = 32; off > 0; off >>= 1) loc += __shfl_xor(loc, off);
    if (lane == 0 && loc) atomicAdd(&tot_sh, loc);
    __syncthreads();
    int chg = (tot_sh + G - 1) / G;
    if (chg < 4) chg = 4;
    if (chg > capg) chg = capg;
    const int per = (B + NT - 1) / NT;
    const int s0 = tid * per, s1 = (s0 + per) < B ? (s0 + per) : B;
    int seg = 0;
    for (int b = s0; b < s1; b++) seg += (cpre[b] + chg - 1) / chg;
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
        const int nch = (cpre[b] + chg - 1) / chg;
        cpre[b] = acc;
        acc += nch;
    }
    if (tid == NT - 1) {
        cpre[B] = acc;
        cpre[B + 1] = chg;
    }
    __syncthreads();
    return cpre[B + 1];
}

// ---------------------------------------------------------------------------
// IVF ADC scan + exact top-ck.  A persistent grid: workgroup w takes the
// contiguous chunk range [w*TC/G, (w+1)*TC/G), so consecutive chunks mostly
// belong to one query and its byte LUT is loaded into LDS once.
//   - each thread takes 4 consecutive candidates of one list: per subspace m
//     one 32-bit coalesced load gives their 4 code bytes (16 loads kept in
//     flight), 4 LDS gathers accumulate dist in m order;
//   - all chunk distances stay in LDS; one radix select + rank sort yields
//     the chunk's exact top-ck by (dist, pos) -> partial[chunk][ck].
// ---------------------------------------------------------------------------
template <int NT, int SU>
__global__ void __launch_bounds__(NT)
scan_topck_kernel(const float* __restrict__ glut, int M, const int32_t* __restrict__ probes,
                  const int32_t* __restrict__ gofs, const int32_t* __restrict__ qtot, int B, int P,
                  const int32_t* __restrict__ list_off, const int32_t* __restrict__ list_padoff,
                  const uint8_t* __restrict__ codes_t, int ck, int cap, int max_chunks,
                  unsigned long long* __restrict__ partial) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* lut = (float*)smem;
    uint32_t* dbuf = (uint32_t*)(lut + (size_t)M * 256);
    unsigned long long* tmpk = (unsigned long long*)(dbuf + cap);  // cap % 64 == 0
    unsigned long long* topk = tmpk + ck;
    int32_t* sg = (int32_t*)(topk + ck);
    int32_t* sprobe = sg + (P + 1);
    int* scratch = (int*)(sprobe + P);
    int* cpre = scratch + ck;
    int32_t* spad0 = cpre + B + 2;  // per probe: padded start, padded size,
    int32_t* snpad = spad0 + P;     // list size, stored-position start
    int32_t* snl = snpad + P;
    int32_t* soff = snl + P;
    SelState* st = (SelState*)(soff + P);

    const int tid = threadIdx.x, G = gridDim.x;
    const int capg = cap / kGroup;
    JHQ_PHASE_DECL
    const int chg = chunk_plan<NT>(qtot, B, capg, G, cpre);
    JHQ_PHASE(0);
    const int TC = cpre[B] < max_chunks ? cpre[B] : max_chunks;
    const int c_begin = (int)((int64_t)TC * blockIdx.x / G);
    const int c_end = (int)((int64_t)TC * (blockIdx.x + 1) / G);
    int cur_b = -1;
    for (int c = c_begin; c < c_end; c++) {
        // query of chunk c: last b with cpre[b] <= c
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (cpre[mid] <= c) lo = mid;
            else hi = mid - 1;
        }
        const int b = lo;
        if (b != cur_b) {
            __syncthreads();
            for (int i = tid; i <= P; i += NT) sg[i] = gofs[(int64_t)b * (P + 1) + i];
            for (int i = tid; i < P; i += NT) {
                const int l = probes[(int64_t)b * P + i];
                sprobe[i] = l;
                const int p0 = list_padoff[l], o0 = list_off[l];
                spad0[i] = p0;
                snpad[i] = list_padoff[l + 1] - p0;
                soff[i] = o0;
                snl[i] = list_off[l + 1] - o0;
            }
            const uint4* src = (const uint4*)(glut + (int64_t)b * M * 256);
            uint4* dst = (uint4*)lut;
            for (int i = tid; i < M * 64; i += NT) dst[i] = src[i];
            cur_b = b;
        }
        if (tid == 0) st->aux = 0;
        __syncthreads();
        JHQ_PHASE(1);
        const int T = sg[P];
        const int g0 = (c - cpre[b]) * chg;
        const int g1 = (g0 + chg) < T ? (g0 + chg) : T;
        unsigned long long* outp = partial + (int64_t)c * ck;

        const int nq4 = (g1 - g0) * 4;
        int nvalid = 0;
        for (int qd = tid; qd < nq4; qd += NT) {
            const int gq = g0 * 4 + qd;
            const int g = gq >> 2, sub = gq & 3;
            int plo = 0, phi = P - 1;  // last p with sg[p] <= g
            while (plo < phi) {
                const int mid = (plo + phi + 1) >> 1;
                if (sg[mid] <= g) plo = mid;
                else phi = mid - 1;
            }
            const int gi = g - sg[plo];
            const int pad0 = spad0[plo];
            const int npad = snpad[plo];
            const int nl = snl[plo];
            const int c0 = gi * kGroup + sub * 4;
            const uint8_t* base = codes_t + (int64_t)pad0 * M + c0;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            // software pipeline: the next SU subspaces' code words are in
            // flight while the current SU are gathered from the LUT
            const int M16 = M & ~(SU - 1);
            uint32_t w[SU], wn[SU];
            if (M16 > 0) {
#pragma unroll
                for (int u = 0; u < SU; u++) w[u] = *(const uint32_t*)(base + (int64_t)u * npad);
            }
            for (int m = 0; m < M16; m += SU) {
                if (m + SU < M16) {
#pragma unroll
                    for (int u = 0; u < SU; u++)
                        wn[u] = *(const uint32_t*)(base + (int64_t)(m + SU + u) * npad);
                }
#pragma unroll
                for (int u = 0; u < SU; u++) {
                    const float* lm = lut + (m + u) * 256;
                    a0 += lm[w[u] & 0xffu];
                    a1 += lm[(w[u] >> 8) & 0xffu];
                    a2 += lm[(w[u] >> 16) & 0xffu];
                    a3 += lm[w[u] >> 24];
                }
#pragma unroll
                for (int u = 0; u < SU; u++) w[u] = wn[u];
            }
            for (int m = M16; m < M; m++) {
                const uint32_t ww = *(const uint32_t*)(base + (int64_t)m * npad);
                const float* lm = lut + m * 256;
                a0 += lm[ww & 0xffu];
                a1 += lm[(ww >> 8) & 0xffu];
                a2 += lm[(ww >> 16) & 0xffu];
                a3 += lm[ww >> 24];
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
        JHQ_PHASE(2);

        auto pos_of = [&](int i) -> uint32_t {
            const int gq = g0 * 4 + (i >> 2);
            const int g = gq >> 2;
            int plo = 0, phi = P - 1;
            while (plo < phi) {
                const int mid = (plo + phi + 1) >> 1;
                if (sg[mid] <= g) plo = mid;
                else phi = mid - 1;
            }
            const int cand = (g - sg[plo]) * kGroup + (gq & 3) * 4 + (i & 3);
            return (uint32_t)(soff[plo] + cand);
        };
        if (ksel > 0)
#ifdef JHQ_PHASE_TIMING
            block_topk<NT>([&](int i) { return dbuf[i]; }, pos_of, nslot, ksel, scratch, tmpk, topk,
                           st, ph_acc + 6);
#else
            block_topk<NT>([&](int i) { return dbuf[i]; }, pos_of, nslot, ksel, scratch, tmpk, topk,
                           st);
#endif
        JHQ_PHASE(3);
        for (int r = tid; r < ck; r += NT) outp[r] = (r < ksel) ? topk[r] : ~0ull;
        JHQ_PHASE(4);
    }
    JHQ_PHASE_FLUSH(0);
}

// Allows `kernel` the LDS left after its static allocation; returns the
// largest dynamic LDS size it may be launched with (0 on failure).
static int allow_max_lds(const void* kernel) {
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, kernel) != hipSuccess) return 0;
    const int dyn = kLdsBytes - (int)fa.sharedSizeBytes;
    if (dyn <= 0) return 0;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, dyn) != hipSuccess)
        return 0;
    return dyn;
}

bool scan_plan(int M, int d, int P, int ck, int max_groups_per_query, int B, int target_wg,
               ScanShape* out) {
    (void)d;
    const int fixed = M * 256 * 4 + 2 * ck * 8 + (P + 1) * 4 + 5 * P * 4 + ck * 4 + (B + 2) * 4 +
                      (int)sizeof(SelState) + 64;
    const int avail = kLdsBytes - 2048 /* static LDS of the kernel */ - fixed;
    if (avail < 1024 * 4) return false;
    int cap = avail / 4;
    if (cap > 16384) cap = 16384;
    cap = (cap / 64) * 64;
    const int capg = cap / kGroup;
    out->G = target_wg;
    out->cap = cap;
    out->lds = fixed + cap * 4;
    // chunks: at most ceil(total/CHg) + B with CHg >= min(capg, ceil(total/G))
    const int64_t per_q_capped = (max_groups_per_query + capg - 1) / capg;
    int64_t mc = (int64_t)B * (per_q_capped + 1);
    if (mc < (int64_t)target_wg + B) mc = (int64_t)target_wg + B;
    out->max_chunks = (int)mc;
    return true;
}

hipError_t scan_topck(const float* glut, int B, int M, const int32_t* probes, const int32_t* gofs,
                      const int32_t* qtot, int P, const int32_t* list_off,
                      const int32_t* list_padoff, const uint8_t* codes_t, int ck,
                      const ScanShape& sh, unsigned long long* partial, hipStream_t s) {
    constexpr int NT = JHQ_SCAN_NT, SU = JHQ_SCAN_SU;
    static const int max_dyn = allow_max_lds((const void*)scan_topck_kernel<NT, SU>);
    if (sh.lds > max_dyn) return hipErrorInvalidValue;
    hipLaunchKernelGGL((scan_topck_kernel<NT, SU>), dim3(sh.G), dim3(NT), sh.lds, s, glut, M, probes,
                       gofs, qtot, B, P, list_off, list_padoff, codes_t, ck, sh.cap,
                       sh.max_chunks, partial);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Merge + residual refine + final top-k, one workgroup per query.
// The residual distance of a candidate is summed by 16 lanes over 16
// contiguous dimension ranges, then added across the lanes in a fixed tree.
// ---------------------------------------------------------------------------
template <int NT>
__global__ void __launch_bounds__(NT)
refine_topk_kernel(const unsigned long long* __restrict__ partial,
                   const int32_t* __restrict__ qtot, int B, int cap, int G, int max_chunks, int mc,
                   int ck, int k, const float* __restrict__ q_rot, int d,
                   const float* __restrict__ res_c1d, int Kr, int Br, int bpv,
                   const uint8_t* __restrict__ list_res, const float* __restrict__ list_corr,
                   const int32_t* __restrict__ list_ids, float* __restrict__ out_d,
                   int32_t* __restrict__ out_i, unsigned long long* __restrict__ topck_dbg) {
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned long long* keys = (unsigned long long*)smem;  // [ck + mc]
    unsigned long long* tmpk = keys + ck + mc;             // [ck]
    unsigned long long* topk = tmpk + ck;                  // [ck]
    // query staged with one pad word per 32 so that lanes reading 32-dim
    // ranges at a 32-word stride hit distinct banks
    float* sq = (float*)(topk + ck);
    int* scratch = (int*)(sq + d + d / 32 + 1);
    float* cprim = (float*)(scratch + ck);
    int* cpos = (int*)(cprim + ck);
    float* ccomp = (float*)(cpos + ck);
    int* cid = (int*)(ccomp + ck);
    int* cpre = cid + ck;
    SelState* st = (SelState*)(cpre + B + 2);
    __shared__ float rc[256];

    const int b = blockIdx.x, tid = threadIdx.x;
    JHQ_PHASE_DECL
    chunk_plan<NT>(qtot, B, cap / kGroup, G, cpre);
    JHQ_PHASE(0);
    for (int i = tid; i < d; i += NT) sq[i + (i >> 5)] = q_rot[(int64_t)b * d + i];
    for (int i = tid; i < Kr; i += NT) rc[i] = res_c1d[i];
    const int cb = cpre[b] < max_chunks ? cpre[b] : max_chunks;
    const int ce = cpre[b + 1] < max_chunks ? cpre[b + 1] : max_chunks;
    const int per_round = mc / ck > 0 ? mc / ck : 1;

    // streaming merge of the query's chunk lists into the exact top-ck
    int cur = 0;
    for (int c0 = cb; c0 < ce; c0 += per_round) {
        const int c1 = (c0 + per_round) < ce ? (c0 + per_round) : ce;
        const int m = (c1 - c0) * ck;
        if (tid == 0) st->aux = 0;
        __syncthreads();
        int nv = 0;
        for (int i = tid; i < m; i += NT) {
            const unsigned long long kk = partial[(int64_t)c0 * ck + i];
            keys[cur + i] = kk;
            nv += (kk != ~0ull) ? 1 : 0;
        }
        for (int off = 32; off > 0; off >>= 1) nv += __shfl_xor(nv, off);
        if ((tid & 63) == 0 && nv) atomicAdd(&st->aux, nv);
        __syncthreads();
        const int n = cur + m;
        const int nvalid = cur + st->aux;
        const int kk = nvalid < ck ? nvalid : ck;
        if (kk > 0) {
            block_topk<NT>([&](int i) { return (uint32_t)(keys[i] >> 32); },
                           [&](int i) { return (uint32_t)(keys[i] & 0xffffffffull); }, n, kk,
                           scratch, tmpk, topk, st);
            for (int r = tid; r < kk; r += NT) keys[r] = topk[r];
        }
        cur = kk;
        __syncthreads();
    }
    const int ksel = cur;
    JHQ_PHASE(1);
    for (int r = tid; r < ck; r += NT) {
        if (r < ksel) {
            const unsigned long long kk = keys[r];
            cprim[r] = ord2f((uint32_t)(kk >> 32));
            cpos[r] = (int)(uint32_t)(kk & 0xffffffffull);
            if (topck_dbg) topck_dbg[(int64_t)b * ck + r] = kk;
        } else if (topck_dbg) {
            topck_dbg[(int64_t)b * ck + r] = ~0ull;
        }
    }
    __syncthreads();

    // residual refine: 16 lanes per candidate, lane l16 sums a contiguous
    // range of dimensions, then a fixed xor tree adds the 16 partial sums.
    const int grp = tid >> 4, l16 = tid & 15;
    constexpr int NG = NT / 16;
    // vector path: each lane's range is whole 16-byte chunks of the code row
    const int dpc = (Br == 4) ? 32 : 16;  // dimensions per 16-byte chunk
    const bool vec = (bpv % 16) == 0 && (d % dpc) == 0;
    int chk = (d + 15) / 16;
    if (vec) chk = (chk + dpc - 1) / dpc * dpc;
    else chk += chk & 1;
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
                        const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                        const int jb = j0 + (c4 + u) * dpc;
                        if (Br == 4) {
#pragma unroll
                            for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
                                for (int nb = 0; nb < 8; nb++) {
                                    const int jj = jb + q4 * 8 + nb;
                                    const float df = sq[jj + (jj >> 5)] - rc[(ww[q4] >> (4 * nb)) & 0x0Fu];
                                    sres = sres + df * df;
                                }
                        } else {
#pragma unroll
                            for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
                                for (int nb = 0; nb < 4; nb++) {
                                    const int jj = jb + q4 * 4 + nb;
                                    const float df = sq[jj + (jj >> 5)] - rc[(ww[q4] >> (8 * nb)) & 0xFFu];
                                    sres = sres + df * df;
                                }
                        }
                    }
                }
            } else if (Br == 4) {
                for (int j = j0; j < j1; j += 2) {
                    const uint32_t byte = rcode[j >> 1];
                    const float df0 = sq[j + (j >> 5)] - rc[byte & 0x0Fu];
                    sres = sres + df0 * df0;
                    if (j + 1 < j1) {
                        const float df1 = sq[(j + 1) + ((j + 1) >> 5)] - rc[byte >> 4];
                        sres = sres + df1 * df1;
                    }
                }
            } else {
                for (int j = j0; j < j1; j++) {
                    const float df = sq[j + (j >> 5)] - rc[rcode[j]];
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

    JHQ_PHASE(2);
    // final top-k by (dist, id)
    const int kf = ksel < k ? ksel : k;
    if (kf > 0) {
        block_topk<NT>([&](int i) { return f2ord(ccomp[i]); }, [&](int i) { return (uint32_t)cid[i]; },
                       ksel, kf, scratch, tmpk, topk, st);
    }
    for (int r = tid; r < k; r += NT) {
        if (r < kf) {
            const unsigned long long kk = topk[r];
            out_d[(int64_t)b * k + r] = ord2f((uint32_t)(kk >> 32));
            out_i[(int64_t)b * k + r] = (int32_t)(uint32_t)(kk & 0xffffffffull);
        } else {
            out_d[(int64_t)b * k + r] = __builtin_huge_valf();
            out_i[(int64_t)b * k + r] = -1;
        }
    }
    JHQ_PHASE(3);
    JHQ_PHASE_FLUSH(2);
}

hipError_t refine_topk(const unsigned long long* partial, const int32_t* qtot, int B,
                       const ScanShape& sh, int ck, int k, const float* q_rot, int d,
                       const float* res_c1d, int Kr, int Br, int bpv, const uint8_t* list_res,
                       const float* list_corr, const int32_t* list_ids, float* out_d,
                       int32_t* out_i, unsigned long long* topck_dbg, hipStream_t s) {
    constexpr int NT = 512;
    if (k > ck || ck > 4 * NT) return hipErrorInvalidValue;
    const int mc = 4096;
    const size_t lds = (size_t)(3 * ck + mc) * 8 + (size_t)(d + d / 32 + 1) * 4 +
                       (size_t)ck * 4 * 5 + (size_t)(B + 2) * 4 + sizeof(SelState) + 64;
    static const int max_dyn = allow_max_lds((const void*)refine_topk_kernel<NT>);
    if ((int)lds > max_dyn) return hipErrorInvalidValue;
    hipLaunchKernelGGL(refine_topk_kernel<NT>, dim3(B), dim3(NT), lds, s, partial, qtot, B, sh.cap,
                       sh.G, sh.max_chunks, mc, ck, k, q_rot, d, res_c1d, Kr, Br, bpv, list_res,
                       list_corr, list_ids, out_d, out_i, topck_dbg);
    return hipGetLastError();
}

}  // namespace jhq

#ifdef JHQ_PHASE_TIMING
// Copies the phase accumulators [3][4096][8] (ticks of the 100 MHz clock).
extern "C" int jhq_debug_phase_ticks(unsigned long long* out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(jhq::g_phase), sizeof(jhq::g_phase), 0,
                                    hipMemcpyDeviceToHost);
}
#endif
