// Lloyd k-means over pre-RoPE K or V, one independent problem per (batch, head).
//
// Reference loop (reskv/compression.py:37-53): each iteration assigns every
// token to its nearest centre, then replaces each centre by the mean of its
// members.  K (value_mode = 0) keeps an empty cluster's previous centre and
// carries fp32 centres; V (value_mode = 1) sets an empty cluster to zero and
// rounds centres to fp16 after every update.  The returned ids come from the
// last assignment, i.e. against the centres before the final update.
//
// Assignment uses d(x, c) = |c|^2 - 2 <x, c> (|x|^2 is common to all centres
// of a row), argmin with the lowest index on ties.  Partial sums are reduced
// per workgroup in LDS and then across workgroups in a fixed order, so the
// update is deterministic.
#include "common.h"
#include "../../include/reskv_hip.h"

using namespace reskv;

namespace {

constexpr int kRowsPerBlock = 256;  // one row per lane

__global__ void __launch_bounds__(256) kmeans_assign_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ centers, int32_t* __restrict__ ids,
    float* __restrict__ psum, int* __restrict__ pcnt, int T, int C, int chunks) {
    __shared__ float s_c[kMaxClusters * kDim];
    __shared__ float s_sum[kMaxClusters * kDim];
    __shared__ float s_norm[kMaxClusters];
    __shared__ int s_cnt[kMaxClusters];
    const int chunk = blockIdx.x;
    const long bh = blockIdx.y;
    const float* cb = centers + bh * C * kDim;
    for (int i = threadIdx.x; i < C * kDim; i += blockDim.x) {
        s_c[i] = cb[i];
        s_sum[i] = 0.0f;
    }
    if (threadIdx.x < C) s_cnt[threadIdx.x] = 0;
    __syncthreads();
    if (threadIdx.x < C) {
        float n = 0.0f;
        for (int d = 0; d < kDim; ++d) n = fmaf(s_c[threadIdx.x * kDim + d], s_c[threadIdx.x * kDim + d], n);
        s_norm[threadIdx.x] = n;
    }
    __syncthreads();

    const int t = chunk * kRowsPerBlock + threadIdx.x;
    if (t < T) {
        const uint32_t* row = (const uint32_t*)(x + (bh * T + t) * kDim);
        float xv[kDim];
#pragma unroll
        for (int i = 0; i < kDim / 2; ++i) {
            const uint32_t w = row[i];
            xv[2 * i] = h2f((uint16_t)(w & 0xFFFFu));
            xv[2 * i + 1] = h2f((uint16_t)(w >> 16));
        }
        float best = INFINITY;
        int bid = 0;
        for (int c = 0; c < C; ++c) {
            const float4* cc = (const float4*)(s_c + c * kDim);
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < kDim / 4; ++i) {
                const float4 v = cc[i];
                dot = fmaf(xv[4 * i], v.x, dot);
                dot = fmaf(xv[4 * i + 1], v.y, dot);
                dot = fmaf(xv[4 * i + 2], v.z, dot);
                dot = fmaf(xv[4 * i + 3], v.w, dot);
            }
            const float dist = fmaf(-2.0f, dot, s_norm[c]);
            if (dist < best) {
                best = dist;
                bid = c;
            }
        }
        ids[bh * T + t] = bid;
        atomicAdd(&s_cnt[bid], 1);
#pragma unroll
        for (int d = 0; d < kDim; ++d) atomicAdd(&s_sum[bid * kDim + d], xv[d]);
    }
    __syncthreads();
    float* ps = psum + ((bh * chunks) + chunk) * (long)C * kDim;
    for (int i = threadIdx.x; i < C * kDim; i += blockDim.x) ps[i] = s_sum[i];
    if (threadIdx.x < C) pcnt[(bh * chunks + chunk) * C + threadIdx.x] = s_cnt[threadIdx.x];
}

__global__ void __launch_bounds__(256) kmeans_update_kernel(
    float* __restrict__ centers, const float* __restrict__ psum, const int* __restrict__ pcnt,
    int C, int chunks, int value_mode, uint16_t* __restrict__ out_fp16) {
    const long bh = blockIdx.x;
    for (int i = threadIdx.x; i < C * kDim; i += blockDim.x) {
        const int c = i / kDim;
        float s = 0.0f;
        int n = 0;
        for (int k = 0; k < chunks; ++k) {
            s += psum[((bh * chunks) + k) * (long)C * kDim + i];
            n += pcnt[(bh * chunks + k) * C + c];
        }
        float* cv = centers + bh * C * kDim + i;
        float nv;
        if (value_mode) {
            nv = n > 0 ? h2f(f2h(s / (float)n)) : 0.0f;   // fp16 centres, empty -> 0
        } else {
            nv = n > 0 ? s / (float)n : *cv;              // fp32 centres, empty keeps
        }
        *cv = nv;
        if (out_fp16) out_fp16[bh * C * kDim + i] = f2h(nv);
    }
}

int chunks_for(int T) { return (T + kRowsPerBlock - 1) / kRowsPerBlock; }

}  // namespace

extern "C" int64_t reskv_kmeans_workspace_bytes(int BH, int T, int C) {
    if (BH <= 0 || T <= 0 || C <= 0) return 0;
    const int64_t chunks = chunks_for(T);
    return (int64_t)BH * chunks * C * (kDim * (int64_t)sizeof(float) + (int64_t)sizeof(int)) +
           (int64_t)BH * C * kDim * (int64_t)sizeof(float);
}

extern "C" int reskv_kmeans_assign(const void* x, const float* centers, int32_t* ids, int BH, int T, int C,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(x && centers && ids, "null pointer argument");
    RESKV_REQUIRE(BH > 0 && T > 0, "problem sizes must be positive");
    RESKV_REQUIRE(C >= 1 && C <= kMaxClusters, "centroid count must be in [1, 64]");
    RESKV_REQUIRE(workspace && workspace_bytes >= reskv_kmeans_workspace_bytes(BH, T, C),
                  "k-means workspace too small");
    const int chunks = chunks_for(T);
    float* psum = (float*)workspace + (long)BH * C * kDim;
    int* pcnt = (int*)(psum + (long)BH * chunks * C * kDim);
    hipLaunchKernelGGL(kmeans_assign_kernel, dim3(chunks, BH), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x, centers, ids, psum, pcnt, T, C, chunks);
    return reskv_host::check_launch("kmeans_assign_kernel");
}

extern "C" int reskv_kmeans(const void* x, const float* centers_init, void* centers_out, int32_t* ids,
                            int BH, int T, int C, int iterations, int value_mode, void* workspace,
                            int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(x && centers_init && centers_out && ids, "null pointer argument");
    RESKV_REQUIRE(BH > 0 && T > 0, "problem sizes must be positive");
    RESKV_REQUIRE(C >= 1 && C <= kMaxClusters, "centroid count must be in [1, 64]");
    RESKV_REQUIRE(iterations >= 1, "iterations must be positive");
    RESKV_REQUIRE(workspace && workspace_bytes >= reskv_kmeans_workspace_bytes(BH, T, C),
                  "k-means workspace too small");
    const int chunks = chunks_for(T);
    float* centers = (float*)workspace;
    float* psum = centers + (long)BH * C * kDim;
    int* pcnt = (int*)(psum + (long)BH * chunks * C * kDim);
    hipStream_t st = (hipStream_t)stream;
    if (hipMemcpyAsync(centers, centers_init, (size_t)BH * C * kDim * sizeof(float), hipMemcpyDeviceToDevice, st) !=
        hipSuccess)
        return reskv_host::check_launch("kmeans centre copy");
    for (int it = 0; it < iterations; ++it) {
        hipLaunchKernelGGL(kmeans_assign_kernel, dim3(chunks, BH), dim3(256), 0, st, (const uint16_t*)x, centers,
                           ids, psum, pcnt, T, C, chunks);
        if (reskv_host::check_launch("kmeans_assign_kernel")) return 1;
        hipLaunchKernelGGL(kmeans_update_kernel, dim3(BH), dim3(256), 0, st, centers, psum, pcnt, C, chunks,
                           value_mode, it == iterations - 1 ? (uint16_t*)centers_out : nullptr);
        if (reskv_host::check_launch("kmeans_update_kernel")) return 1;
    }
    return 0;
}
