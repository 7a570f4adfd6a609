// Lloyd k-means over pre-RoPE K or V, one independent problem per (batch, head).
//
// Reference loop (reskv/compression.py:37-53): each iteration assigns every
// token to its nearest centre, then replaces each centre by the mean of its
// members.  K (value_mode = 0) keeps an empty cluster's previous centre and
// carries fp32 centres; V (value_mode = 1) sets an empty cluster to zero and
// rounds centres to fp16 after every update.  The returned ids come from the
// last assignment, i.e. against the centres before the final update.
//
// Assignment (kmeans_assign_kernel): the distance GEMM S = X C^T runs on the
// matrix cores (v_mfma_f32_16x16x16f16).  Tokens are fp16 already; each fp32
// centre is split into fp16 hi + lo parts so that X C^T = X C_hi^T + X C_lo^T
// keeps fp32 accuracy (x * c_hi and x * c_lo are exact in fp32, sums are fp32).
// d(x, c) = |c|^2 - 2 <x, c> (|x|^2 is common to a row); argmin with the lowest
// index on ties is a DPP reduction over the 16 lanes holding a token's
// distances.  Member sums are a second matrix-core product, onehot(ids)^T X,
// with the 16-token tile transposed through LDS: one-hot entries and tokens
// are exact in fp16 and the products accumulate in fp32.  The waves of a
// 128-token chunk are reduced in a fixed order, so sums, counts and centres
// are deterministic.
// Update (kmeans_update_kernel): one workgroup per (head, cluster) reduces the
// chunk partials and writes the new centre.
#include "common.h"
#include "../../include/reskv_hip.h"

using namespace reskv;

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kChunk = 128;          // tokens per assignment workgroup
constexpr int kWaves = 4;
constexpr int kSub = 16;             // tokens per MFMA sub-tile
constexpr int kXPitch = kDim + 4;  // halves per staged token row: 264 bytes puts the 4 row groups on different banks

__device__ __forceinline__ half4_t as_h4(uint2 v) { return __builtin_bit_cast(half4_t, v); }

// (distance, index) minimum with the lower index winning ties
__device__ __forceinline__ void argmin_step(float& d, int& i, float od, int oi) {
    const bool take = od < d || (od == d && oi < i);
    d = take ? od : d;
    i = take ? oi : i;
}
template <int CTRL>
__device__ __forceinline__ void argmin_dpp(float& d, int& i) {
    const float od = dpp<CTRL>(d);
    const int oi = (int)dpp_u<CTRL>((uint32_t)i);
    argmin_step(d, i, od, oi);
}

// One workgroup: tokens [chunk * 128, +128) of problem bh.
// centers fp32 [BH, C, 128]; ids int32 [BH, T]; psum fp32 [BH, chunks, C, 128]
// and pcnt int [BH, chunks, C] (skipped when psum is null).
template <int NB>
__global__ void __launch_bounds__(256) kmeans_assign_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ centers, int32_t* __restrict__ ids,
    float* __restrict__ psum, int* __restrict__ pcnt, int T, int C, int chunks, int split_lo) {
    __shared__ __align__(16) uint16_t s_hi[NB * 16 * kXPitch];  // padded rows: conflict-free operand reads
    __shared__ __align__(16) uint16_t s_lo[NB * 16 * kXPitch];
    __shared__ float s_norm[NB * 16];
    __shared__ float s_sum[kMaxClusters * kDim];  // staged centres, then member sums [C][128]
    __shared__ __align__(16) uint16_t s_x[kWaves][kSub * kXPitch];  // per-wave token tile, padded rows
    __shared__ int s_cnt[kMaxClusters];
    const int chunk = blockIdx.x;
    const long bh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;  // MFMA lane coordinates

    // centres: fp32 rows staged in LDS (in the member-sum buffer) with float4
    // loads, then split into fp16 hi/lo tables; rows >= C are zero and get an
    // infinite distance
    {
        const float4* cb4 = reinterpret_cast<const float4*>(centers + bh * C * kDim);
        float4* st4 = reinterpret_cast<float4*>(s_sum);
        for (int i = tid; i < NB * 16 * kDim / 4; i += 256)
            st4[i] = i < C * kDim / 4 ? cb4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    __syncthreads();
    for (int i = tid; i < NB * 16 * kDim; i += 256) {
        const float v = s_sum[i];
        const uint16_t hb = f2h(v);
        const int o = (i / kDim) * kXPitch + i % kDim;
        s_hi[o] = hb;
        s_lo[o] = split_lo ? f2h(v - h2f(hb)) : (uint16_t)0;
    }
    // |c|^2: 8 threads per centre, 16 channels each, then a fixed-order 8-lane reduction
    for (int c0 = 0; c0 < NB * 16; c0 += 32) {
        const int c = c0 + (tid >> 3), part = tid & 7;
        float n = 0.0f;
        if (c < NB * 16) {
#pragma unroll
            for (int d = 0; d < 16; ++d) {
                const float v = s_sum[c * kDim + 16 * part + d];
                n = fmaf(v, v, n);
            }
        }
        n += __shfl_xor(n, 1);
        n += __shfl_xor(n, 2);
        n += __shfl_xor(n, 4);
        if (part == 0 && c < NB * 16) s_norm[c] = c < C ? n : INFINITY;
    }
    __syncthreads();
    if (tid < kMaxClusters) s_cnt[tid] = 0;
    __syncthreads();

    // B operands come from LDS per use: lane (col, grp) reads centre nb*16 + col,
    // channels 32*grp + 4*s + [0,4) for step s
    float cnorm[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) cnorm[nb] = s_norm[nb * 16 + col];

    float4_t sums[NB][8];  // onehot^T X: rows nb*16 + 4*grp + r, channels db*16 + col
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int db = 0; db < 8; ++db) sums[nb][db] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
    uint16_t* xs = s_x[wave];

    const int base = chunk * kChunk;
    uint4 xn[4];
    auto load_rows = [&](int t0, uint4* dst) {
        const int tok = t0 + col;
        const uint4* src = reinterpret_cast<const uint4*>(x + (bh * T + (tok < T ? tok : t0)) * kDim + 32 * grp);
#pragma unroll
        for (int q = 0; q < 4; ++q) dst[q] = src[q];
    };
    if (base + wave * kSub < T) load_rows(base + wave * kSub, xn);
    for (int sub = wave; sub < kChunk / kSub; sub += kWaves) {
        const int t0 = base + sub * kSub;
        if (t0 >= T) break;
        // A operand rows: token t0 + col, dims [32*grp, 32*grp + 32)
        const int tok = t0 + col;
        const bool valid = tok < T;
        uint4 xr[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) xr[q] = xn[q];
        const int tn = t0 + kWaves * kSub;
        if (sub + kWaves < kChunk / kSub && tn < T) load_rows(tn, xn);
        float4_t acc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            acc[nb] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint2 a = s & 1 ? make_uint2(xr[s >> 1].z, xr[s >> 1].w) : make_uint2(xr[s >> 1].x, xr[s >> 1].y);
                const int off = (nb * 16 + col) * kXPitch + 32 * grp + 4 * s;
                acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    as_h4(a), as_h4(*reinterpret_cast<const uint2*>(s_hi + off)), acc[nb], 0, 0, 0);
                if (split_lo)
                    acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                        as_h4(a), as_h4(*reinterpret_cast<const uint2*>(s_lo + off)), acc[nb], 0, 0, 0);
            }
        }
        // lane (col, grp) holds <x, c> for tokens t0 + 4*grp + r, centres nb*16 + col
        int best_id[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float bd = INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const float d = fmaf(-2.0f, acc[nb][r], cnorm[nb]);
                argmin_step(bd, bi, d, nb * 16 + col);
            }
            argmin_dpp<0xB1>(bd, bi);   // quad xor 1
            argmin_dpp<0x4E>(bd, bi);   // quad xor 2
            argmin_dpp<0x141>(bd, bi);  // row half mirror
            argmin_dpp<0x140>(bd, bi);  // row mirror
            best_id[r] = bi;
        }
        // ids: lane col == r of row grp writes token t0 + 4*grp + r
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + 4 * grp + r;
            if (col == r && t < T) ids[bh * T + t] = best_id[r];
        }
        if (psum != nullptr) {
            // stage the tile: lane (col, grp) writes token col's channels [32*grp, +32)
            uint4* row = reinterpret_cast<uint4*>(xs + col * kXPitch + 32 * grp);
#pragma unroll
            for (int q = 0; q < 4; ++q) row[q] = xr[q];
            wave_sync();
            // A = onehot^T: lane (col, grp) holds [cluster nb*16 + col][tokens 4*grp + i]
            half4_t oh[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool in = (t0 + 4 * grp + i < T) && best_id[i] == nb * 16 + col;
                    oh[nb][i] = in ? (_Float16)1.0f : (_Float16)0.0f;
                }
            }
            // B = X: lane (col, grp) holds [tokens 4*grp + i][channel db*16 + col]
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                half4_t xb;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xb[i] = __builtin_bit_cast(_Float16, xs[(4 * grp + i) * kXPitch + 16 * db + col]);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    sums[nb][db] = __builtin_amdgcn_mfma_f32_16x16x16f16(oh[nb], xb, sums[nb][db], 0, 0, 0);
            }
            // counts: lane col == r of row grp counts token t0 + 4*grp + r
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (col == r && t0 + 4 * grp + r < T) atomicAdd(&s_cnt[best_id[r]], 1);
            wave_sync();  // tile reads done before the next tile is staged
        }
    }
    if (psum == nullptr) return;
    // fixed-order reduction of the four waves' sums into LDS
    for (int w = 0; w < kWaves; ++w) {
        if (wave == w) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int db = 0; db < 8; ++db)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int c = nb * 16 + 4 * grp + r;
                        float* dst = s_sum + c * kDim + db * 16 + col;
                        *dst = (w == 0 ? 0.0f : *dst) + sums[nb][db][r];
                    }
        }
        __syncthreads();
    }
    float* ps = psum + ((bh * chunks) + chunk) * (long)C * kDim;
    for (int i = tid; i < C * kDim; i += 256) ps[i] = s_sum[i];
    if (tid < C) pcnt[(bh * chunks + chunk) * C + tid] = s_cnt[tid];
}

// One workgroup (256 threads: channel x chunk parity) per (cluster, problem);
// the two halves of the chunk sum meet in LDS, in a fixed order.
__global__ void __launch_bounds__(2 * kDim) kmeans_update_kernel(
    float* __restrict__ centers, const float* __restrict__ psum, const int* __restrict__ pcnt, int C,
    int chunks, int value_mode, uint16_t* __restrict__ out_fp16) {
    __shared__ float s_part[kDim];
    __shared__ int s_n[2];
    const int c = blockIdx.x;
    const long bh = blockIdx.y;
    const int d = threadIdx.x & (kDim - 1), par = threadIdx.x >> 7;
    float s = 0.0f;
    int n = 0;
    const float* src = psum + (bh * chunks) * (long)C * kDim + c * kDim + d;
    const int* cnt = pcnt + bh * chunks * C + c;
#pragma unroll 16
    for (int k = par; k < chunks; k += 2) {
        s += src[(long)k * C * kDim];
        n += cnt[k * C];
    }
    if (par == 1) {
        s_part[d] = s;
        if (d == 0) s_n[1] = n;
    }
    __syncthreads();
    if (par == 1) return;
    s += s_part[d];
    n += s_n[1];
    float* cv = centers + (bh * C + c) * kDim + d;
    float nv;
    if (value_mode) {
        nv = n > 0 ? h2f(f2h(s / (float)n)) : 0.0f;  // fp16 centres, empty -> 0
    } else {
        nv = n > 0 ? s / (float)n : *cv;             // fp32 centres, empty keeps
    }
    *cv = nv;
    if (out_fp16) out_fp16[(bh * C + c) * kDim + d] = f2h(nv);
}

int chunks_for(int T) { return (T + kChunk - 1) / kChunk; }

int launch_assign(const void* x, const float* centers, int32_t* ids, float* psum, int* pcnt, int BH, int T, int C,
                  int split_lo, hipStream_t st) {
    const int chunks = chunks_for(T);
    const dim3 grid(chunks, BH);
    const int nb = (C + 15) / 16;
    switch (nb) {
    case 1: hipLaunchKernelGGL(kmeans_assign_kernel<1>, grid, dim3(256), 0, st, (const uint16_t*)x, centers, ids,
                               psum, pcnt, T, C, chunks, split_lo); break;
    case 2: hipLaunchKernelGGL(kmeans_assign_kernel<2>, grid, dim3(256), 0, st, (const uint16_t*)x, centers, ids,
                               psum, pcnt, T, C, chunks, split_lo); break;
    case 3: hipLaunchKernelGGL(kmeans_assign_kernel<3>, grid, dim3(256), 0, st, (const uint16_t*)x, centers, ids,
                               psum, pcnt, T, C, chunks, split_lo); break;
    default: hipLaunchKernelGGL(kmeans_assign_kernel<4>, grid, dim3(256), 0, st, (const uint16_t*)x, centers, ids,
                                psum, pcnt, T, C, chunks, split_lo); break;
    }
    return reskv_host::check_launch("kmeans_assign_kernel");
}

int check_x_alignment(const void* x) {
    RESKV_REQUIRE(((uintptr_t)x & 15u) == 0, "token rows must be 16-byte aligned");
    return 0;
}

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
    (void)workspace;
    (void)workspace_bytes;
    if (check_x_alignment(x)) return 1;
    return launch_assign(x, centers, ids, nullptr, nullptr, BH, T, C, 1, (hipStream_t)stream);
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
    if (check_x_alignment(x)) return 1;
    const int chunks = chunks_for(T);
    float* centers = (float*)workspace;
    float* psum = centers + (long)BH * C * kDim;
    int* pcnt = (int*)(psum + (long)BH * chunks * C * kDim);
    hipStream_t st = (hipStream_t)stream;
    if (hipMemcpyAsync(centers, centers_init, (size_t)BH * C * kDim * sizeof(float), hipMemcpyDeviceToDevice, st) !=
        hipSuccess)
        return reskv_host::check_launch("kmeans centre copy");
    for (int it = 0; it < iterations; ++it) {
        // V centres are fp16 values already: their lo part is zero
        if (launch_assign(x, centers, ids, psum, pcnt, BH, T, C, value_mode ? 0 : 1, st)) return 1;
        hipLaunchKernelGGL(kmeans_update_kernel, dim3(C, BH), dim3(2 * kDim), 0, st, centers, psum, pcnt, C, chunks,
                           value_mode, it == iterations - 1 ? (uint16_t*)centers_out : nullptr);
        if (reskv_host::check_launch("kmeans_update_kernel")) return 1;
    }
    return 0;
}
