// assign_mfma.hip — IVF assignment on fp32 MFMA with an exact re-check
// (v14/jhq_gpu_index.cu:23-40,367-393: argmin over lists of
// ||c||^2 - 2 <y, c>, ties to the lowest list).
//
// The assignment must equal the fixed-order one (gemm_nt_argmin: each dot an
// fmaf chain in k order, score fmaf(-2, dot, norm), ties to the lowest list)
// bit for bit.  A first pass computes every score on MFMA, whose summation
// order differs, and keeps per row the smallest score s1 (list c1) and the
// second smallest s2.  Both summation orders are within gamma * sum |y_k c_k|
// of the exact dot, so every approximate score is within
//   E = 4 * ((4 (K + 4) + 5) u ||y|| Cmax + 3 u Nmax),   u = 2^-24,
// of its fixed-order value (Cmax = max ||c||, Nmax = max ||c||^2; the factor
// 4 is headroom over the two dot bounds and the final roundings).  If
// s2 - s1 > 2E, list c1 is the unique fixed-order argmin.  Other rows (near
// ties, exact ties, any non-finite score) are listed and re-assigned by the
// fixed-order kernel.
#include "kernels.h"

#include <hip/hip_runtime.h>
#include <cmath>
#include <cstdint>

namespace jhq {

typedef float v4f_a __attribute__((ext_vector_type(4)));

constexpr int kTopBM = 128, kTopBN = 128, kTopBK = 16, kTopLd = kTopBK + 4;

// One workgroup (4 waves) per 128 rows and share of the 128-list tiles
// (blockIdx.y of gridDim.y shares; with more than one, each share's best and
// second best go to their own slots and top2_merge_kernel combines them in
// share order, so a few rows still fill the chip).  Wave w
// covers rows 64*(w>>1) .. +63 and tile columns 64*(w&1) .. +63 as 4 x 4
// tiles of v_mfma_f32_16x16x4_f32.  K advances in chunks of 16 staged in LDS
// (double-buffered, the next chunk's global loads issued before the current
// chunk's MFMAs).  Lane (r, g) supplies k = 16*chunk + 4g + s in instruction
// s of a chunk, so one 16-byte LDS read gives a fragment for 4 instructions.
// Each lane keeps, for each of its 16 rows, the smallest and second smallest
// score over its own columns; the end reduces over the lanes and the two
// column halves.
__global__ void __launch_bounds__(256, 2)
mfma_top2_kernel(const float* __restrict__ Y, int64_t n, int d, const float* __restrict__ Cm,
                 int nlist, const float* __restrict__ norms, int32_t* __restrict__ best,
                 float* __restrict__ s1, float* __restrict__ s2) {
    __shared__ __align__(16) float As[2][kTopBM][kTopLd];
    __shared__ __align__(16) float Bs[2][kTopBN][kTopLd];
    __shared__ float xb[2][kTopBM];
    __shared__ float xs[2][kTopBM];
    __shared__ int xc[2][kTopBM];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, g = lane >> 4, rh = wv >> 1, ch = wv & 1;
    const int64_t r0 = (int64_t)blockIdx.x * kTopBM;
    const int nchunk = (d + kTopBK - 1) / kTopBK;
    const int ntall = (nlist + kTopBN - 1) / kTopBN;
    const int per = (ntall + (int)gridDim.y - 1) / (int)gridDim.y;
    const int tb = (int)blockIdx.y * per, te = min(ntall, tb + per);
    const int ntile = te > tb ? te - tb : 0;
    best += (int64_t)blockIdx.y * n;
    s1 += (int64_t)blockIdx.y * n;
    s2 += (int64_t)blockIdx.y * n;
    // staging: thread t moves rows (t >> 2) and 64 + (t >> 2), k4 = 4 * (t & 3)
    const int lrow = tid >> 2, lk = 4 * (tid & 3);
    float bv[16], sv[16];
    int bc[16];
#pragma unroll
    for (int q = 0; q < 16; q++) {
        bv[q] = INFINITY;
        sv[q] = INFINITY;
        bc[q] = 0x7fffffff;
    }
    auto load_a = [&](int kc, float4 (&ra)[2]) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t row = r0 + lrow + 64 * h;
            const int k = kc * kTopBK + lk;
            ra[h] = (row < n && k < d) ? *(const float4*)(Y + row * d + k)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto load_b = [&](int t, int kc, float4 (&rb)[2]) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int col = t * kTopBN + lrow + 64 * h;
            const int k = kc * kTopBK + lk;
            rb[h] = (col < nlist && k < d) ? *(const float4*)(Cm + (int64_t)col * d + k)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store = [&](int buf, const float4 (&ra)[2], const float4 (&rb)[2]) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            *(float4*)&As[buf][lrow + 64 * h][lk] = ra[h];
            *(float4*)&Bs[buf][lrow + 64 * h][lk] = rb[h];
        }
    };
    const int nsteps = ntile * nchunk;
    float4 ra[2], rb[2];
    if (nsteps > 0) {
        load_a(0, ra);
        load_b(tb, 0, rb);
        store(0, ra, rb);
    }
    __syncthreads();
    v4f_a acc[4][4];
    int step = 0;
    for (int t = tb; t < te; t++) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[i][c] = v4f_a{0.f, 0.f, 0.f, 0.f};
        for (int kc = 0; kc < nchunk; kc++, step++) {
            const int buf = step & 1;
            const bool more = step + 1 < nsteps;
            if (more) {
                const int nkc = kc + 1 < nchunk ? kc + 1 : 0;
                const int nt = kc + 1 < nchunk ? t : t + 1;
                load_a(nkc, ra);
                load_b(nt, nkc, rb);
            }
            float4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) fa[i] = *(const float4*)&As[buf][64 * rh + 16 * i + r][4 * g];
#pragma unroll
            for (int c = 0; c < 4; c++) fb[c] = *(const float4*)&Bs[buf][64 * ch + 16 * c + r][4 * g];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].x, fb[c].x, acc[i][c], 0, 0, 0);
                    acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].y, fb[c].y, acc[i][c], 0, 0, 0);
                    acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].z, fb[c].z, acc[i][c], 0, 0, 0);
                    acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].w, fb[c].w, acc[i][c], 0, 0, 0);
                }
            if (more) store(buf ^ 1, ra, rb);
            __syncthreads();
        }
        // lane (r, g): rows 64*rh + 16*i + 4*g + j, list t*128 + 64*ch + 16*c + r
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int col = t * kTopBN + 64 * ch + 16 * c + r;
            if (col >= nlist) continue;
            const float nc = norms[col];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int q = 4 * i + j;
                    const float v = fmaf(-2.0f, acc[i][c][j], nc);
                    if (v < bv[q]) {
                        sv[q] = bv[q];
                        bv[q] = v;
                        bc[q] = col;
                    } else if (v < sv[q]) {
                        sv[q] = v;
                    }
                }
        }
    }
    // over the 16 lanes r of a lane group (their rows are the same)
#pragma unroll
    for (int q = 0; q < 16; q++) {
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const float ob = __shfl_xor(bv[q], off), os = __shfl_xor(sv[q], off);
            const int oc = __shfl_xor(bc[q], off);
            const bool mine = bv[q] < ob || (bv[q] == ob && bc[q] < oc);
            if (mine) {
                sv[q] = fminf(sv[q], ob);
            } else {
                sv[q] = fminf(os, bv[q]);
                bv[q] = ob;
                bc[q] = oc;
            }
        }
    }
    if (r == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int row = 64 * rh + 16 * i + 4 * g + j;
                xb[ch][row] = bv[4 * i + j];
                xs[ch][row] = sv[4 * i + j];
                xc[ch][row] = bc[4 * i + j];
            }
    }
    __syncthreads();
    if (tid < kTopBM) {
        const int64_t row = r0 + tid;
        if (row < n) {
            const float b0 = xb[0][tid], b1 = xb[1][tid];
            const int c0 = xc[0][tid], c1 = xc[1][tid];
            const bool first = b0 < b1 || (b0 == b1 && c0 < c1);
            best[row] = first ? c0 : c1;
            s1[row] = first ? b0 : b1;
            s2[row] = first ? fminf(xs[0][tid], b1) : fminf(xs[1][tid], b0);
        }
    }
}

// Combines the S shares' (best, list, second) per row in share order (ties to
// the lower list), into share 0's slots.
__global__ void __launch_bounds__(256)
top2_merge_kernel(int64_t n, int S, int32_t* __restrict__ best, float* __restrict__ s1,
                  float* __restrict__ s2) {
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= n) return;
    float b = s1[row], sc = s2[row];
    int c = best[row];
    for (int y = 1; y < S; y++) {
        const float ob = s1[y * n + row], os = s2[y * n + row];
        const int oc = best[y * n + row];
        if (b < ob || (b == ob && c < oc)) {
            sc = fminf(sc, ob);
        } else {
            sc = fminf(os, b);
            b = ob;
            c = oc;
        }
    }
    best[row] = c;
    s1[row] = b;
    s2[row] = sc;
}

// Nmax = max ||c||^2 over the lists (one workgroup); also zeroes the
// re-check count
__global__ void __launch_bounds__(256) max_norm_kernel(const float* __restrict__ norms, int nlist,
                                                       float* __restrict__ out,
                                                       int32_t* __restrict__ cnt) {
    __shared__ float red[256];
    float m = 0.0f;
    for (int c = threadIdx.x; c < nlist; c += 256) m = fmaxf(m, norms[c]);
    red[threadIdx.x] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        out[0] = red[0];
        cnt[0] = 0;
    }
}

// One wave per row: ||y|| in double; accept c1 when the gap clears 2E, else
// append the row to the re-check list.
__global__ void __launch_bounds__(256)
top2_accept_kernel(const float* __restrict__ Y, int64_t n, int d, const int32_t* __restrict__ best,
                   const float* __restrict__ s1, const float* __restrict__ s2,
                   const float* __restrict__ nmax, int32_t* __restrict__ assign,
                   int32_t* __restrict__ recheck, int32_t* __restrict__ nrecheck) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    double ss = 0.0;
    for (int k = lane; k < d; k += 64) {
        const double v = (double)Y[row * d + k];
        ss += v * v;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane != 0) return;
    const double u = 1.0 / 16777216.0;
    const double Nm = (double)nmax[0] * (1.0 + 4.0 * u);
    const double ny = sqrt(ss) * (1.0 + 4.0 * u), cm = sqrt(Nm);
    const double E = 4.0 * ((4.0 * (d + 4) + 5.0) * u * ny * cm + 3.0 * u * Nm);
    const double a = (double)s1[row], b = (double)s2[row];
    // b = +inf (a single list) passes; a non-finite s1 or a NaN goes to the re-check
    const bool ok = isfinite(a) && !isnan(b) && (b - a > 2.0 * E);
    if (ok) {
        assign[row] = best[row];
    } else {
        const int slot = atomicAdd(nrecheck, 1);
        recheck[slot] = (int32_t)row;
    }
}

// assign[recheck[i]] = list of keys[i], i < *cnt
__global__ void __launch_bounds__(256)
recheck_scatter_kernel(const unsigned long long* __restrict__ keys,
                       const int32_t* __restrict__ recheck, const int32_t* __restrict__ cnt,
                       int32_t* __restrict__ assign) {
    const int64_t m = cnt[0];
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < m; i += (int64_t)gridDim.x * 256)
        assign[recheck[i]] = (int32_t)(uint32_t)(keys[i] & 0xffffffffull);
}

__global__ void tally_kernel(const int32_t* __restrict__ cnt, unsigned long long* __restrict__ total) {
    if (threadIdx.x == 0) total[0] += (unsigned long long)cnt[0];
}

hipError_t assign_mfma_tally(const float* scratch, int64_t n, unsigned long long* total,
                             hipStream_t s) {
    hipLaunchKernelGGL(tally_kernel, dim3(1), dim3(64), 0, s, assign_mfma_rechecked(scratch, n),
                       total);
    return hipGetLastError();
}

bool assign_mfma_ok(int d, const float* Y, const float* Cm) {
    return d > 0 && d % 4 == 0 && ((uintptr_t)Y & 15) == 0 && ((uintptr_t)Cm & 15) == 0;
}

// shares of the list tiles: about 512 workgroups when the rows are few
static int top2_shares(int64_t n) {
    const int64_t rb = (n + kTopBM - 1) / kTopBM;
    int64_t s = (512 + rb - 1) / rb;
    return (int)(s < 1 ? 1 : (s > 8 ? 8 : s));
}

size_t assign_mfma_scratch_floats(int64_t n) {
    // best, s1, s2 (one word per row and share), re-check rows, the re-check
    // count, Nmax
    return (size_t)n * (3 * top2_shares(n) + 1) + 64;
}

const int32_t* assign_mfma_rechecked(const float* scratch, int64_t n) {
    return (const int32_t*)(scratch + (size_t)n * (3 * top2_shares(n) + 1));
}

hipError_t assign_mfma(const float* Y, int64_t n, int d, const float* Cm, int nlist,
                       const float* norms, int32_t* assign, float* scratch,
                       size_t scratch_floats, unsigned long long* keys, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (!assign_mfma_ok(d, Y, Cm) || nlist <= 0 || !scratch || !keys ||
        scratch_floats < assign_mfma_scratch_floats(n) || (n + 127) / 128 > 65535)
        return hipErrorInvalidValue;
    const int S = top2_shares(n);
    int32_t* best = (int32_t*)scratch;
    float* s1 = scratch + (size_t)S * n;
    float* s2 = scratch + (size_t)2 * S * n;
    int32_t* recheck = (int32_t*)(scratch + (size_t)3 * S * n);
    int32_t* cnt = (int32_t*)(scratch + (size_t)n * (3 * S + 1));
    float* nmax = (float*)cnt + 16;
    hipLaunchKernelGGL(max_norm_kernel, dim3(1), dim3(256), 0, s, norms, nlist, nmax, cnt);
    hipLaunchKernelGGL(mfma_top2_kernel, dim3((unsigned)((n + kTopBM - 1) / kTopBM), (unsigned)S),
                       dim3(256), 0, s, Y, n, d, Cm, nlist, norms, best, s1, s2);
    if (S > 1)
        hipLaunchKernelGGL(top2_merge_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, n,
                           S, best, s1, s2);
    hipLaunchKernelGGL(top2_accept_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, Y, n, d,
                       best, s1, s2, nmax, assign, recheck, cnt);
    // the fixed-order argmin over the listed rows (their count read on the device)
    hipError_t e = fill_u64(keys, n, ~0ull, s);
    if (e != hipSuccess) return e;
    e = gemm_nt_argmin_rows(Y, d, recheck, cnt, n, Cm, d, nlist, d, norms, keys, s);
    if (e != hipSuccess) return e;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(recheck_scatter_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)),
                       dim3(256), 0, s, keys, recheck, cnt, assign);
    return hipGetLastError();
}

}  // namespace jhq
