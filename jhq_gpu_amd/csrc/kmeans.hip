// kmeans.hip — Lloyd iterations of the coarse (IVF) quantizer on the device
// (v14/jhq_gpu_index.cu:228-299, whose means are computed on the host).
//
// The first two steps also order an insert's new vectors by (list, vector)
// (list_order, scatter_plan: the reference's stable sort by list,
// v14/jhq_gpu_index.cu:468-486).
//
// One iteration after the assignment (gemm_nt_argmin):
//   1. keys (list << 32 | sample) sorted ascending: every list's members
//      end up contiguous and in ascending sample order;
//   2. each list's first member by binary search in the sorted keys;
//   3. one workgroup per list sums its members' rows in double, in that
//      order (the reference's host loop adds sample i after sample i-1), and
//      stores the float mean; an empty list takes the reseed row
//      (c * 1103515245 + iter * 12345) mod n;
//   4. the norms ||c||^2 in double, j ascending, like the host twin.
// The sums see the same operands in the same order as the host loop, so the
// centroids are bit-identical to it.
#include "kernels.h"

#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>

namespace jhq {

__global__ void kmeans_init_kernel(const float* __restrict__ y, int d, int64_t n, int nlist,
                                   float* __restrict__ cent) {
    const int c = blockIdx.x;
    const int64_t src = (int64_t)c * n / nlist;
    for (int j = threadIdx.x; j < d; j += blockDim.x) cent[(int64_t)c * d + j] = y[src * d + j];
}

__global__ void kmeans_keys_kernel(const int32_t* __restrict__ asg, int64_t n,
                                   unsigned long long* __restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) keys[i] = ((unsigned long long)(uint32_t)asg[i] << 32) | (uint32_t)i;
}

// first[c] = index of the first sorted key of list c (first[nlist] = n)
__global__ void kmeans_bounds_kernel(const unsigned long long* __restrict__ sorted, int64_t n,
                                     int nlist, int64_t* __restrict__ first) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c > nlist) return;
    const unsigned long long key = (unsigned long long)(uint32_t)c << 32;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (sorted[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    first[c] = lo;
}

__global__ void kmeans_means_kernel(const float* __restrict__ y, int d, int64_t n,
                                    const unsigned long long* __restrict__ sorted,
                                    const int64_t* __restrict__ first, int iter,
                                    float* __restrict__ cent) {
    const int c = blockIdx.x;
    const int64_t o0 = first[c], o1 = first[c + 1];
    float* cc = cent + (int64_t)c * d;
    if (o0 == o1) {
        const int64_t src = ((int64_t)c * 1103515245 + (int64_t)iter * 12345) % n;
        for (int j = threadIdx.x; j < d; j += blockDim.x) cc[j] = y[src * d + j];
        return;
    }
    const double inv = 1.0 / (double)(o1 - o0);
    for (int j = threadIdx.x; j < d; j += blockDim.x) {
        double acc = 0.0;
        int64_t m = o0;
        // rows are loaded 8 ahead of the adds; the adds stay in sample order
        for (; m + 8 <= o1; m += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = y[(int64_t)(uint32_t)sorted[m + u] * d + j];
#pragma unroll
            for (int u = 0; u < 8; u++) acc += (double)v[u];
        }
        for (; m < o1; m++) acc += (double)y[(int64_t)(uint32_t)sorted[m] * d + j];
        cc[j] = (float)(acc * inv);
    }
}

__global__ void kmeans_norms_kernel(const float* __restrict__ cent, int d, int nlist,
                                    float* __restrict__ norms) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= nlist) return;
    const float* cc = cent + (int64_t)c * d;
    double s = 0.0;
    for (int j = 0; j < d; j++) s += (double)cc[j] * (double)cc[j];
    norms[c] = (float)s;
}

hipError_t kmeans_init(const float* y, int d, int64_t n, int nlist, float* cent, hipStream_t s) {
    if (nlist <= 0 || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kmeans_init_kernel, dim3(nlist), dim3(256), 0, s, y, d, n, nlist, cent);
    return hipGetLastError();
}

hipError_t kmeans_norms(const float* cent, int d, int nlist, float* norms, hipStream_t s) {
    if (nlist <= 0) return hipSuccess;
    hipLaunchKernelGGL(kmeans_norms_kernel, dim3((nlist + 255) / 256), dim3(256), 0, s, cent, d,
                       nlist, norms);
    return hipGetLastError();
}

size_t kmeans_scratch_bytes(int64_t n, int nlist) {
    size_t sort_bytes = 0;
    int bits = 1;
    while ((1ll << bits) < (int64_t)nlist) bits++;
    (void)rocprim::radix_sort_keys(nullptr, sort_bytes, (const unsigned long long*)nullptr,
                                   (unsigned long long*)nullptr, (size_t)n, 0u, 32u + bits);
    return ((size_t)n * 8 * 2 + 255) / 256 * 256 + ((size_t)(nlist + 1) * 8 + 255) / 256 * 256 +
           (sort_bytes + 255) / 256 * 256;
}

hipError_t list_order(const int32_t* asg, int64_t n, int nlist, void* scratch, size_t scratch_bytes,
                      const unsigned long long** sorted_out, const int64_t** first_out,
                      hipStream_t s) {
    if (nlist <= 0 || n <= 0 || n > 0x7fffffffll) return hipErrorInvalidValue;
    int bits = 1;
    while ((1ll << bits) < (int64_t)nlist) bits++;
    unsigned char* p = (unsigned char*)scratch;
    unsigned long long* keys = (unsigned long long*)p;
    unsigned long long* sorted = keys + n;
    p += ((size_t)n * 8 * 2 + 255) / 256 * 256;
    int64_t* first = (int64_t*)p;
    p += ((size_t)(nlist + 1) * 8 + 255) / 256 * 256;
    size_t sort_bytes = 0;
    hipError_t e = rocprim::radix_sort_keys(nullptr, sort_bytes, keys, sorted, (size_t)n, 0u,
                                            32u + bits, s);
    if (e != hipSuccess) return e;
    if ((size_t)(p - (unsigned char*)scratch) + sort_bytes > scratch_bytes)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(kmeans_keys_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, asg,
                       n, keys);
    e = rocprim::radix_sort_keys(sort_bytes ? (void*)p : nullptr, sort_bytes, keys, sorted,
                                 (size_t)n, 0u, 32u + bits, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kmeans_bounds_kernel, dim3((nlist + 1 + 255) / 256), dim3(256), 0, s,
                       sorted, n, nlist, first);
    *sorted_out = sorted;
    *first_out = first;
    return hipGetLastError();
}

hipError_t kmeans_update(const int32_t* asg, const float* y, int d, int64_t n, int nlist, int iter,
                         float* cent, void* scratch, size_t scratch_bytes, hipStream_t s) {
    const unsigned long long* sorted = nullptr;
    const int64_t* first = nullptr;
    hipError_t e = list_order(asg, n, nlist, scratch, scratch_bytes, &sorted, &first, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kmeans_means_kernel, dim3(nlist), dim3(256), 0, s, y, d, n, sorted, first,
                       iter, cent);
    return hipGetLastError();
}

// Sorted position p of an insert's new vectors (keys (list << 32 | vector),
// ascending): vector order[p] goes to list slist[p] at index
// ldesc[list].size (the list's size before the insert) + p - first[list].
__global__ void scatter_plan_kernel(const unsigned long long* __restrict__ sorted,
                                    const int64_t* __restrict__ first,
                                    const int4* __restrict__ ldesc, int64_t n,
                                    int32_t* __restrict__ order, int32_t* __restrict__ slist,
                                    int32_t* __restrict__ sidx) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const unsigned long long k = sorted[p];
    const int l = (int)(k >> 32);
    order[p] = (int32_t)(uint32_t)k;
    slist[p] = l;
    sidx[p] = (int32_t)(ldesc[l].z + (p - first[l]));
}

hipError_t scatter_plan(const unsigned long long* sorted, const int64_t* first, const int4* ldesc,
                        int64_t n, int32_t* order, int32_t* slist, int32_t* sidx, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(scatter_plan_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       sorted, first, ldesc, n, order, slist, sidx);
    return hipGetLastError();
}

}  // namespace jhq
