// assign_mfma.hip — IVF assignment on bf16 MFMA with an exact re-check
// (v14/jhq_gpu_index.cu:23-40,367-393: argmin over lists of
// ||c||^2 - 2 <y, c>, ties to the lowest list).
//
// The assignment must equal the fixed-order one (gemm_nt_argmin: each dot an
// fmaf chain in k order, score fmaf(-2, dot, norm), ties to the lowest list)
// bit for bit.  A first pass computes every score on MFMA and keeps per row
// the smallest score s1 (list c1) and the second smallest s2.  The pass
// splits each float into two bf16 (hi = bf16(x), lo = bf16(x - hi), so
// |x - hi - lo| <= 2^-16 |x|) and sums hi*hi + hi*lo + lo*hi with three
// bf16 MFMAs per 32 k (the products are exact in fp32).  Against the
// fixed-order dot F, the first pass's dot A differs by at most
//   e_dot = (2u * 1.02 * 33 * 3 * dp/32 + 3.01 * 2^-16 + (d + 4) u) ||y|| Cmax
// (u = 2^-24, dp = d rounded up to 32): at most 33 roundings of at most 2u
// per MFMA over the three product sums, the split's dropped terms
// (hi*E + e*H + r*R <= 3.01 * 2^-16 |y_k c_k|), and the fixed-order chain's
// own rounding.  The scores then differ by at most 2 e_dot plus one rounding
// each; with a factor 2 of headroom and a term for values the MFMA may flush
// as subnormals,
//   E = 2 (2 e_dot + 2u Nmax + 4u ||y|| Cmax) + 6d (2^-126 (||y|| + Cmax) + 2^-149)
// (Cmax = max ||c||, Nmax = max ||c||^2).  If s2 - s1 > 2E, list c1 is the
// unique fixed-order argmin.  Other rows (near ties, exact ties, any
// non-finite score) are listed and re-assigned by the fixed-order kernel.
#include "kernels.h"

#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include <cstdint>

namespace jhq {

typedef __bf16 bf16x8_a __attribute__((ext_vector_type(8)));
typedef float v4f_a __attribute__((ext_vector_type(4)));

// rows (lists) per tile, k per step (one bf16 MFMA), LDS row stride in bf16
// (80 bytes: the 16-byte fragment reads of a 16-row group fall in distinct banks)
constexpr int kTopBM = 128, kTopBN = 128, kTopBK = 32, kTopLd = kTopBK + 8;

__host__ __device__ constexpr int top2_kpad(int d) { return (d + kTopBK - 1) / kTopBK * kTopBK; }

// float -> bf16 bits, round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint32_t bf16_rne(float x) {
    const uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x40u;
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

// hi[r][k] = bf16(x[r][k]), lo[r][k] = bf16(x[r][k] - hi), rows padded with
// zeros to dp (a multiple of 32); one thread per 8 elements of a row
__global__ void __launch_bounds__(256)
split_bf16_kernel(const float* __restrict__ x, int64_t n, int d, int dp,
                  uint4* __restrict__ hi, uint4* __restrict__ lo) {
    const int per = dp / 8;
    const int64_t total = n * per;
    const bool vec = (d % 4) == 0 && ((uintptr_t)x & 15) == 0;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * 256) {
        const int64_t row = e / per;
        const int k0 = (int)(e - row * per) * 8;
        const float* xr = x + row * d;
        float v[8];
        if (vec && k0 + 8 <= d) {
            const float4 a = *(const float4*)(xr + k0), b = *(const float4*)(xr + k0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = (k0 + i < d) ? xr[k0 + i] : 0.0f;
        }
        uint32_t h[8], l[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            h[i] = bf16_rne(v[i]);
            l[i] = bf16_rne(v[i] - __uint_as_float(h[i] << 16));
        }
        hi[e] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                           h[6] | (h[7] << 16));
        lo[e] = make_uint4(l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16),
                           l[6] | (l[7] << 16));
    }
}

// One workgroup (4 waves) per 128 rows and share of the 128-list tiles (S
// shares; with more than one, each share's best and second best go to their
// own slots and top2_merge_kernel combines them in share order, so a few rows
// still fill the chip).  The operands stream from beyond L2 (rows and lists
// are tens of MB), so the workgroups are placed for L2 reuse: workgroups go
// to the 8 XCDs in turn (XCD = block id mod 8), and the S shares of a row
// tile get consecutive slots of one XCD, where they run together and read
// the row tile's k steps from the same L2; the XCD's workgroups of one share
// walk the same list tiles in the same order.  Wave w covers rows
// 64*(w>>1) .. +63 and tile columns 64*(w&1) .. +63 as 4 x 4 tiles of
// v_mfma_f32_16x16x32_bf16, three per tile and k step (hi*hi, hi*lo,
// lo*hi).  K advances in steps of 32 staged in LDS (double-buffered, the next
// step's global loads issued before the current step's MFMAs).  Lane (r, g)
// supplies row (list) r's 8 values k = 32*step + 8g .. +7 of each operand.
// Each lane keeps, for each of its 16 rows, the smallest and second smallest
// score over its own columns; the end reduces over the lanes and the two
// column halves.
__global__ void __launch_bounds__(256, 2)
mfma_top2_kernel(const uint16_t* __restrict__ Yh, const uint16_t* __restrict__ Yl, int64_t n,
                 int dp, const uint16_t* __restrict__ Ch, const uint16_t* __restrict__ Cl,
                 int nlist, const float* __restrict__ norms, int S, int32_t* __restrict__ best,
                 float* __restrict__ s1, float* __restrict__ s2) {
    // [buffer][hi, lo][row][k]; the row exchange at the end reuses the space
    __shared__ __align__(16) uint16_t As[2][2][kTopBM][kTopLd];
    __shared__ __align__(16) uint16_t Bs[2][2][kTopBN][kTopLd];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, g = lane >> 4, rh = wv >> 1, ch = wv & 1;
    // slot j of XCD x: row tile x + 8 (j / S), share j % S
    const int xcd = (int)(blockIdx.x & 7), slot = (int)(blockIdx.x >> 3);
    const int64_t rt = xcd + 8 * (int64_t)(slot / S);
    const int share = slot % S;
    const int64_t r0 = rt * kTopBM;
    if (r0 >= n) return;
    const int nchunk = dp / kTopBK;
    const int ntall = (nlist + kTopBN - 1) / kTopBN;
    const int per = (ntall + S - 1) / S;
    const int tb = share * per, te = min(ntall, tb + per);
    const int ntile = te > tb ? te - tb : 0;
    best += (int64_t)share * n;
    s1 += (int64_t)share * n;
    s2 += (int64_t)share * n;
    // staging: thread t moves rows (t >> 2) and 64 + (t >> 2), 8 values from
    // k = 8 * (t & 3), of hi and lo
    const int lrow = tid >> 2, lk = 8 * (tid & 3);
    float bv[16], sv[16];
    int bc[16];
#pragma unroll
    for (int q = 0; q < 16; q++) {
        bv[q] = INFINITY;
        sv[q] = INFINITY;
        bc[q] = 0x7fffffff;
    }
    // rows past n and lists past nlist read the last valid row (their scores
    // are never kept): plain global loads, no select of an address
    const int64_t ya = min(r0 + lrow, n - 1) * dp + lk, yb = min(r0 + lrow + 64, n - 1) * dp + lk;
    auto cofs = [&](int t, int h) -> int64_t {
        return (int64_t)min(t * kTopBN + lrow + 64 * h, nlist - 1) * dp + lk;
    };
    // next step's operands in registers: rows lrow and lrow + 64, hi and lo
    uint4 a0h, a0l, a1h, a1l, b0h, b0l, b1h, b1l;
    auto load = [&](int t, int kc) {
        const int k = kc * kTopBK;
        a0h = *(const uint4*)(Yh + ya + k);
        a0l = *(const uint4*)(Yl + ya + k);
        a1h = *(const uint4*)(Yh + yb + k);
        a1l = *(const uint4*)(Yl + yb + k);
        const int64_t c0 = cofs(t, 0) + k, c1 = cofs(t, 1) + k;
        b0h = *(const uint4*)(Ch + c0);
        b0l = *(const uint4*)(Cl + c0);
        b1h = *(const uint4*)(Ch + c1);
        b1l = *(const uint4*)(Cl + c1);
    };
    auto store = [&](int buf) {
        *(uint4*)&As[buf][0][lrow][lk] = a0h;
        *(uint4*)&As[buf][1][lrow][lk] = a0l;
        *(uint4*)&As[buf][0][lrow + 64][lk] = a1h;
        *(uint4*)&As[buf][1][lrow + 64][lk] = a1l;
        *(uint4*)&Bs[buf][0][lrow][lk] = b0h;
        *(uint4*)&Bs[buf][1][lrow][lk] = b0l;
        *(uint4*)&Bs[buf][0][lrow + 64][lk] = b1h;
        *(uint4*)&Bs[buf][1][lrow + 64][lk] = b1l;
    };
    const int nsteps = ntile * nchunk;
    if (nsteps > 0) {
        load(tb, 0);
        store(0);
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
                load(nt, nkc);
            }
            bf16x8_a ah[4], al[4], bh[4], bl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ah[i] = *(const bf16x8_a*)&As[buf][0][64 * rh + 16 * i + r][8 * g];
                al[i] = *(const bf16x8_a*)&As[buf][1][64 * rh + 16 * i + r][8 * g];
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                bh[c] = *(const bf16x8_a*)&Bs[buf][0][64 * ch + 16 * c + r][8 * g];
                bl[c] = *(const bf16x8_a*)&Bs[buf][1][64 * ch + 16 * c + r][8 * g];
            }
            // the three product sums in turn, 16 independent tiles apart
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bh[c], acc[i][c], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bl[c], acc[i][c], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bh[c], acc[i][c], 0, 0, 0);
            if (more) store(buf ^ 1);
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
    // the k loop ended with a barrier: the staging space is free
    float (*xb)[kTopBM] = reinterpret_cast<float (*)[kTopBM]>(&As[0][0][0][0]);
    float (*xs)[kTopBM] = xb + 2;
    int (*xc)[kTopBM] = reinterpret_cast<int (*)[kTopBM]>(xb + 4);
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
    const double steps = (double)(top2_kpad(d) / kTopBK);
    const double e_dot = (2.0 * u * 1.02 * 33.0 * 3.0 * steps + 3.01 / 65536.0 + (d + 4.0) * u) *
                         ny * cm;
    const double tiny = 6.0 * d * (ldexp(1.0, -126) * (ny + cm) + ldexp(1.0, -149));
    const double E = 2.0 * (2.0 * e_dot + 2.0 * u * Nm + 4.0 * u * ny * cm) + tiny;
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

// shares of the list tiles: up to 512 workgroups (two per CU) when the rows
// are few
static int top2_shares(int64_t n) {
    const int64_t rb = (n + kTopBM - 1) / kTopBM;
    const int64_t s = 512 / rb;
    return (int)(s < 1 ? 1 : (s > 8 ? 8 : s));
}

// best, s1, s2 (one word per row and share), re-check rows, the re-check
// count, Nmax; then the bf16 halves of the rows and of the lists
static size_t top2_split_offset(int64_t n) {
    return ((size_t)n * (3 * top2_shares(n) + 1) + 64 + 63) / 64 * 64;
}

size_t assign_mfma_scratch_floats(int64_t n, int d, int nlist) {
    // hi and lo of a padded row: dp bf16 each, dp floats together
    return top2_split_offset(n) + ((size_t)n + (size_t)nlist) * (size_t)top2_kpad(d);
}

const int32_t* assign_mfma_rechecked(const float* scratch, int64_t n) {
    return (const int32_t*)(scratch + (size_t)n * (3 * top2_shares(n) + 1));
}

hipError_t assign_mfma(const float* Y, int64_t n, int d, const float* Cm, int nlist,
                       const float* norms, int32_t* assign, float* scratch,
                       size_t scratch_floats, unsigned long long* keys, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (!assign_mfma_ok(d, Y, Cm) || nlist <= 0 || !scratch || !keys ||
        scratch_floats < assign_mfma_scratch_floats(n, d, nlist) || (n + 127) / 128 > 65535)
        return hipErrorInvalidValue;
    const int S = top2_shares(n);
    const int dp = top2_kpad(d);
    uint16_t* yh = (uint16_t*)(scratch + top2_split_offset(n));
    uint16_t* yl = yh + (size_t)n * dp;
    uint16_t* chh = yl + (size_t)n * dp;
    uint16_t* cl = chh + (size_t)nlist * dp;
    {
        const int64_t ry = n * (dp / 8), rc = (int64_t)nlist * (dp / 8);
        hipLaunchKernelGGL(split_bf16_kernel, dim3((unsigned)std::min<int64_t>((ry + 255) / 256, 8192)),
                           dim3(256), 0, s, Y, n, d, dp, (uint4*)yh, (uint4*)yl);
        hipLaunchKernelGGL(split_bf16_kernel, dim3((unsigned)std::min<int64_t>((rc + 255) / 256, 8192)),
                           dim3(256), 0, s, Cm, (int64_t)nlist, d, dp, (uint4*)chh, (uint4*)cl);
    }
    int32_t* best = (int32_t*)scratch;
    float* s1 = scratch + (size_t)S * n;
    float* s2 = scratch + (size_t)2 * S * n;
    int32_t* recheck = (int32_t*)(scratch + (size_t)3 * S * n);
    int32_t* cnt = (int32_t*)(scratch + (size_t)n * (3 * S + 1));
    float* nmax = (float*)cnt + 16;
    hipLaunchKernelGGL(max_norm_kernel, dim3(1), dim3(256), 0, s, norms, nlist, nmax, cnt);
    {
        // 8 XCDs x (row tiles per XCD) x S slots; slots past the last row tile exit
        const int64_t rb = (n + kTopBM - 1) / kTopBM, per_xcd = (rb + 7) / 8;
        hipLaunchKernelGGL(mfma_top2_kernel, dim3((unsigned)(8 * per_xcd * S)), dim3(256), 0, s, yh,
                           yl, n, dp, chh, cl, nlist, norms, S, best, s1, s2);
    }
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
