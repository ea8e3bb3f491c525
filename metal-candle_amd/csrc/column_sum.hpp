// Fixed-order column sums of per-block partials, shared by the row kernels
// whose weight gradients are reduced over rows in two stages.
#pragma once

#include "common.hpp"

namespace mc {

// dw[j] = sum_b partial[b][j]. A workgroup owns 32 columns: lane group c
// (8 lanes x 4 adjacent columns) and slice s (32 slices) sum the partial rows
// b = s, s + 32, ... in ascending order, then the 32 slice sums are combined
// in slice order through LDS. The order is fixed, so dw is reproducible;
// 32 independent row walks per column keep enough loads in flight to hide
// the latency (one thread per column walking all rows was latency-bound).
inline constexpr int kSumCols = 32;
template <bool VEC>
__global__ __launch_bounds__(256) void column_sum(int nb, int64_t dim, const float* __restrict__ partial,
                                                  float* __restrict__ out) {
    constexpr int kGroups = kSumCols / 4;       // lanes per slice, 4 columns each
    constexpr int kSlices = 256 / kGroups;      // 32 row slices
    __shared__ float red[kSlices][kSumCols + 1];
    const int g = threadIdx.x % kGroups;
    const int s = threadIdx.x / kGroups;
    const int64_t j0 = (int64_t)blockIdx.x * kSumCols + g * 4;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    if (j0 < dim) {
#pragma unroll 8
        for (int b = s; b < nb; b += kSlices) {
            const float* p = partial + (int64_t)b * dim + j0;
            if constexpr (VEC) {
                const float4 q = *reinterpret_cast<const float4*>(p);
                a[0] += q.x; a[1] += q.y; a[2] += q.z; a[3] += q.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j0 + e < dim) a[e] += p[e];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) red[s][g * 4 + e] = a[e];
    __syncthreads();
    if (threadIdx.x < kSumCols) {
        const int64_t j = (int64_t)blockIdx.x * kSumCols + threadIdx.x;
        float t = red[0][threadIdx.x];
#pragma unroll
        for (int k = 1; k < kSlices; ++k) t += red[k][threadIdx.x];
        if (j < dim) out[j] = t;
    }
}

}  // namespace mc
