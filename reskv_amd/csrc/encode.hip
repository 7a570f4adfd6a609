// Residual encoders: one wavefront per token, lane L owns channels L and L+64.
//
// Every encoder computes r = f32(x) - f32(c[id]) and ranks channels by the
// 15-bit magnitude of fp16(r) with ties going to the lower channel index
// (reskv/csrc/compression.cu:80-118, 184-203, 287-313; reskv/compression.py:75-89).
// The rank key is made unique by appending the inverted channel index, so
// "top-k" is a single threshold on that composite key:
//   ckey(d) = (|fp16(r_d)| bits) << 7 | (127 - d).
// Top-k over all 128 channels uses a 22-step bitwise threshold search on
// wave ballots; top-k inside a 16-channel tile counts larger keys from LDS.
#include "common.h"

using namespace reskv;

namespace {

constexpr int kWavesPerBlock = 4;

struct Residual {
    float r0, r1;     // channels L, L+64
    uint32_t m0, m1;  // |fp16(r)| as 15-bit integers (order == value order)
};

__device__ __forceinline__ Residual load_residual(const uint16_t* __restrict__ keys,
                                                  const uint16_t* __restrict__ cent,
                                                  const int32_t* __restrict__ ids,
                                                  long row, long bh, int C, int lane) {
    int cid = ids[row];
    cid = cid < 0 ? 0 : (cid > C - 1 ? C - 1 : cid);  // compression.cu:83-84
    const uint16_t* x = keys + row * kDim;
    const uint16_t* c = cent + (bh * C + cid) * kDim;
    Residual r;
    r.r0 = h2f(x[lane]) - h2f(c[lane]);
    r.r1 = h2f(x[lane + kHalf]) - h2f(c[lane + kHalf]);
    r.m0 = f2h(r.r0) & 0x7FFFu;
    r.m1 = f2h(r.r1) & 0x7FFFu;
    return r;
}

__device__ __forceinline__ uint32_t ckey(uint32_t mag, int d) { return (mag << 7) | (uint32_t)(127 - d); }

// Threshold tau with exactly k composite keys >= tau (keys are unique).
__device__ __forceinline__ uint32_t topk_threshold(uint32_t k0, uint32_t k1, int k) {
    uint32_t prefix = 0;
#pragma unroll
    for (int bit = 21; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        const int cnt = __builtin_popcountll(ballot(k0 >= cand)) + __builtin_popcountll(ballot(k1 >= cand));
        prefix = cnt >= k ? cand : prefix;
    }
    return prefix;
}

// Number of keys in the lane's 16-channel tile that outrank its own key.
__device__ __forceinline__ int tile_rank(const uint32_t* tile_keys, uint32_t mine) {
    int rank = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) rank += tile_keys[j] > mine ? 1 : 0;
    return rank;
}

__device__ __forceinline__ uint64_t bitrev64(uint64_t v) {
    return ((uint64_t)__builtin_bitreverse32((uint32_t)v) << 32) | __builtin_bitreverse32((uint32_t)(v >> 32));
}

__global__ void __launch_bounds__(256) encode_qtile_kernel(
    const uint16_t* __restrict__ keys, const uint16_t* __restrict__ cent,
    const int32_t* __restrict__ ids, uint16_t* __restrict__ payload, int32_t* __restrict__ meta,
    long rows, int T, int C, int nnz, int struct_index) {
    __shared__ uint32_t s_keys[kWavesPerBlock][kDim];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int per_tile = nnz >> 3;
    for (long row = (long)blockIdx.x * kWavesPerBlock + wave; row < rows;
         row += (long)gridDim.x * kWavesPerBlock) {
        const long bh = row / T;
        const Residual r = load_residual(keys, cent, ids, row, bh, C, lane);
        const uint32_t k0 = ckey(r.m0, lane), k1 = ckey(r.m1, lane + kHalf);
        s_keys[wave][lane] = k0;
        s_keys[wave][lane + kHalf] = k1;
        wave_sync();
        const int tile0 = lane >> 4, bit = lane & 15;
        const bool sel0 = tile_rank(&s_keys[wave][tile0 * 16], k0) < per_tile;
        const bool sel1 = tile_rank(&s_keys[wave][(tile0 + 4) * 16], k1) < per_tile;
        const uint64_t b0 = ballot(sel0), b1 = ballot(sel1);
        const uint32_t below = (1u << bit) - 1u;
        const uint32_t t0 = (uint32_t)(b0 >> (16 * tile0)) & 0xFFFFu;
        const uint32_t t1 = (uint32_t)(b1 >> (16 * tile0)) & 0xFFFFu;
        uint16_t* prow = payload + row * nnz;
        if (sel0) prow[tile0 * per_tile + __builtin_popcount(t0 & below)] = f2h(r.r0);
        if (sel1) prow[(tile0 + 4) * per_tile + __builtin_popcount(t1 & below)] = f2h(r.r1);
        if (lane < 4) {
            // word w = code(tile 2w) | code(tile 2w+1) << 16
            uint32_t word = 0;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int tile = 2 * lane + half;
                const uint64_t b = tile < 4 ? b0 : b1;
                const uint32_t mask = (uint32_t)(b >> (16 * (tile & 3))) & 0xFFFFu;
                uint32_t code = mask;
                if (struct_index) {
                    code = 0;
                    int rank = 0;
                    for (int i = 0; i < 16; ++i)
                        if ((mask >> i) & 1u) code |= (uint32_t)i << (4 * rank++);
                }
                word |= code << (16 * half);
            }
            meta[row * 4 + lane] = (int32_t)word;
        }
        wave_sync();
    }
}

__global__ void __launch_bounds__(256) encode_bitmap_kernel(
    const uint16_t* __restrict__ keys, const uint16_t* __restrict__ cent,
    const int32_t* __restrict__ ids, uint16_t* __restrict__ payload, int64_t* __restrict__ meta,
    long rows, int T, int C, int nnz) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (long row = (long)blockIdx.x * kWavesPerBlock + wave; row < rows;
         row += (long)gridDim.x * kWavesPerBlock) {
        const long bh = row / T;
        const Residual r = load_residual(keys, cent, ids, row, bh, C, lane);
        const uint32_t k0 = ckey(r.m0, lane), k1 = ckey(r.m1, lane + kHalf);
        const uint32_t tau = topk_threshold(k0, k1, nnz);
        const bool sel0 = k0 >= tau, sel1 = k1 >= tau;
        const uint64_t b0 = ballot(sel0), b1 = ballot(sel1);
        uint16_t* prow = payload + row * nnz;
        if (sel0) prow[lanes_below(b0)] = f2h(r.r0);
        if (sel1) prow[__builtin_popcountll(b0) + lanes_below(b1)] = f2h(r.r1);
        // channel d -> bit (63 - d % 64) of word d / 64 (compression.py:87-88)
        if (lane < 2) meta[row * 2 + lane] = (int64_t)bitrev64(lane == 0 ? b0 : b1);
    }
}

template <int BITS>
__global__ void __launch_bounds__(256) encode_multibit_kernel(
    const uint16_t* __restrict__ keys, const uint16_t* __restrict__ cent,
    const int32_t* __restrict__ ids, int32_t* __restrict__ qtiles, uint16_t* __restrict__ qscale,
    long rows, int T, int C, int nnz) {
    constexpr int kPerWord = 32 / BITS;
    constexpr int kQmax = (1 << (BITS - 1)) - 1;
    constexpr int kWords = kDim / kPerWord;
    __shared__ uint8_t s_code[kWavesPerBlock][kDim];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (long row = (long)blockIdx.x * kWavesPerBlock + wave; row < rows;
         row += (long)gridDim.x * kWavesPerBlock) {
        const long bh = row / T;
        const Residual r = load_residual(keys, cent, ids, row, bh, C, lane);
        const uint32_t k0 = ckey(r.m0, lane), k1 = ckey(r.m1, lane + kHalf);
        const uint32_t tau = topk_threshold(k0, k1, nnz);
        const bool sel0 = k0 >= tau, sel1 = k1 >= tau;
        const float amax = wave_max(fmaxf(sel0 ? fabsf(r.r0) : 0.0f, sel1 ? fabsf(r.r1) : 0.0f));
        // fp16(amax / QMAX) with an IEEE fp32 division, fp16(1) for an all-zero residual
        const uint16_t hs = amax > 0.0f ? f2h(amax / (float)kQmax) : f2h(1.0f);
        const float sf = h2f(hs);
        int q0 = (int)rintf(r.r0 / sf), q1 = (int)rintf(r.r1 / sf);
        q0 = q0 < -kQmax ? -kQmax : (q0 > kQmax ? kQmax : q0);
        q1 = q1 < -kQmax ? -kQmax : (q1 > kQmax ? kQmax : q1);
        s_code[wave][lane] = sel0 ? (uint8_t)(q0 & ((1 << BITS) - 1)) : 0;
        s_code[wave][lane + kHalf] = sel1 ? (uint8_t)(q1 & ((1 << BITS) - 1)) : 0;
        wave_sync();
        if (lane < kWords) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < kPerWord; ++i) word |= (uint32_t)s_code[wave][lane * kPerWord + i] << (i * BITS);
            qtiles[row * kWords + lane] = (int32_t)word;
        }
        if (lane == 0) qscale[row] = hs;
        wave_sync();
    }
}

__global__ void __launch_bounds__(256) encode_struct_int4_kernel(
    const uint16_t* __restrict__ keys, const uint16_t* __restrict__ cent,
    const int32_t* __restrict__ ids, int32_t* __restrict__ qpacked, int32_t* __restrict__ qmeta,
    uint16_t* __restrict__ qscale, long rows, int T, int C) {
    __shared__ uint8_t s_nib[kWavesPerBlock][32];
    __shared__ uint8_t s_sel[kWavesPerBlock][32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (long row = (long)blockIdx.x * kWavesPerBlock + wave; row < rows;
         row += (long)gridDim.x * kWavesPerBlock) {
        const long bh = row / T;
        const Residual r = load_residual(keys, cent, ids, row, bh, C, lane);
        // 1 of 4 per subgroup: largest magnitude, lower channel on ties
        const uint32_t sub = (uint32_t)(lane & 3);
        uint32_t c0 = (r.m0 << 2) | (3u - sub), c1 = (r.m1 << 2) | (3u - sub);
        uint32_t x0 = c0, x1 = c1;
        x0 = max(x0, dpp_u<0xB1>(x0));
        x0 = max(x0, dpp_u<0x4E>(x0));
        x1 = max(x1, dpp_u<0xB1>(x1));
        x1 = max(x1, dpp_u<0x4E>(x1));
        const bool sel0 = c0 == x0, sel1 = c1 == x1;
        float v0 = sel0 ? r.r0 : 0.0f, v1 = sel1 ? r.r1 : 0.0f;
        v0 += dpp<0xB1>(v0);
        v0 += dpp<0x4E>(v0);
        v1 += dpp<0xB1>(v1);
        v1 += dpp<0x4E>(v1);
        const float amax = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
        const float s = amax > 0.0f ? amax * (1.0f / 7.0f) : 1.0f;  // compression.cu:224
        int q0 = (int)rintf(v0 / s), q1 = (int)rintf(v1 / s);
        q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
        q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
        const int g0 = lane >> 2, g1 = g0 + 16;  // subgroup indices of channels L, L+64
        if (sel0) {
            s_nib[wave][g0] = (uint8_t)(q0 & 0xF);
            s_sel[wave][g0] = (uint8_t)sub;
        }
        if (sel1) {
            s_nib[wave][g1] = (uint8_t)(q1 & 0xF);
            s_sel[wave][g1] = (uint8_t)sub;
        }
        wave_sync();
        if (lane < 4) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) word |= (uint32_t)s_nib[wave][lane * 8 + i] << (4 * i);
            qpacked[row * 4 + lane] = (int32_t)word;
        } else if (lane < 6) {
            const int w = lane - 4;
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 16; ++i) word |= (uint32_t)s_sel[wave][w * 16 + i] << (2 * i);
            qmeta[row * 2 + w] = (int32_t)word;
        } else if (lane == 6) {
            qscale[row] = f2h(s);
        }
        wave_sync();
    }
}

int grid_for(long rows) {
    long blocks = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
    const long cap = 256L * 64;  // enough resident waves to saturate HBM; loop the rest
    return (int)(blocks < cap ? (blocks < 1 ? 1 : blocks) : cap);
}

int check_common(const void* keys, const void* cent, const void* ids, int B, int H, int T, int C) {
    RESKV_REQUIRE(keys && cent && ids, "null input pointer");
    RESKV_REQUIRE(B > 0 && H > 0 && T > 0, "batch, head and token dimensions must be positive");
    RESKV_REQUIRE(C >= 1 && C <= kMaxClusters, "centroid count must be in [1, 64]");
    return 0;
}

}  // namespace

extern "C" int reskv_compress_fp16(const void* keys, const void* centroids, const int32_t* ids,
                                   void* payload, int32_t* meta, int B, int H, int T, int C,
                                   int nnz, int struct_index, void* stream) {
    if (check_common(keys, centroids, ids, B, H, T, C)) return 1;
    RESKV_REQUIRE(payload && meta, "null output pointer");
    RESKV_REQUIRE(nnz > 0 && nnz < kDim && nnz % 8 == 0,
                  "FP16 tile encoder requires nnz divisible by 8 and < 128");
    RESKV_REQUIRE(!struct_index || nnz == 32, "4:16 index codes require nnz == 32");
    const long rows = (long)B * H * T;
    hipLaunchKernelGGL(encode_qtile_kernel, dim3(grid_for(rows)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)keys, (const uint16_t*)centroids, ids, (uint16_t*)payload, meta,
                       rows, T, C, nnz, struct_index);
    return reskv_host::check_launch("encode_qtile_kernel");
}

extern "C" int reskv_compress_bitmap(const void* keys, const void* centroids, const int32_t* ids,
                                     void* payload, int64_t* meta, int B, int H, int T, int C,
                                     int nnz, void* stream) {
    if (check_common(keys, centroids, ids, B, H, T, C)) return 1;
    RESKV_REQUIRE(payload && meta, "null output pointer");
    RESKV_REQUIRE(nnz > 0 && nnz <= kDim, "nnz must be in [1, 128]");
    const long rows = (long)B * H * T;
    hipLaunchKernelGGL(encode_bitmap_kernel, dim3(grid_for(rows)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)keys, (const uint16_t*)centroids, ids, (uint16_t*)payload, meta,
                       rows, T, C, nnz);
    return reskv_host::check_launch("encode_bitmap_kernel");
}

extern "C" int reskv_compress_quantized(const void* keys, const void* centroids, const int32_t* ids,
                                        int32_t* qtiles, void* qscale, int B, int H, int T, int C,
                                        int nnz, int bits, void* stream) {
    if (check_common(keys, centroids, ids, B, H, T, C)) return 1;
    RESKV_REQUIRE(qtiles && qscale, "null output pointer");
    RESKV_REQUIRE(nnz == 32 || nnz == 64, "quantised encoder requires nnz in {32, 64}");
    RESKV_REQUIRE(bits == 2 || bits == 4, "quantised encoder requires bits in {2, 4}");
    const long rows = (long)B * H * T;
    if (bits == 4)
        hipLaunchKernelGGL(encode_multibit_kernel<4>, dim3(grid_for(rows)), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)keys, (const uint16_t*)centroids, ids, qtiles,
                           (uint16_t*)qscale, rows, T, C, nnz);
    else
        hipLaunchKernelGGL(encode_multibit_kernel<2>, dim3(grid_for(rows)), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)keys, (const uint16_t*)centroids, ids, qtiles,
                           (uint16_t*)qscale, rows, T, C, nnz);
    return reskv_host::check_launch("encode_multibit_kernel");
}

extern "C" int reskv_compress_structured_int4(const void* keys, const void* centroids,
                                              const int32_t* ids, int32_t* qpacked, int32_t* qmeta,
                                              void* qscale, int B, int H, int T, int C, void* stream) {
    if (check_common(keys, centroids, ids, B, H, T, C)) return 1;
    RESKV_REQUIRE(qpacked && qmeta && qscale, "null output pointer");
    const long rows = (long)B * H * T;
    hipLaunchKernelGGL(encode_struct_int4_kernel, dim3(grid_for(rows)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)keys, (const uint16_t*)centroids, ids, qpacked, qmeta,
                       (uint16_t*)qscale, rows, T, C);
    return reskv_host::check_launch("encode_struct_int4_kernel");
}
