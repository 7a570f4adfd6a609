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

// ---------------------------------------------------------------------------
// 4 of 16 per tile (structured 4:16 at 75%): eight lanes per token, lane
// 8 t + j owns 16-channel tile j of token t, so a wave encodes 8 tokens and
// every load and store is a contiguous run of the token's row.
//
// fp16(f32(x) - f32(c)) equals the correctly rounded fp16 difference for every
// pair of finite fp16 values (checked exhaustively), so residuals come from
// packed fp16 subtraction.  Each channel j of the tile gets the unique key
//   (|h| << 5) | ((15 - j) << 1) | sign(h)
// (magnitude first, lower channel on ties, the fp16 bits recoverable from the
// key); a selection network yields the top 4 keys, which are then put in
// channel order.
// ---------------------------------------------------------------------------
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void cx_desc(uint32_t& a, uint32_t& b) {  // a >= b afterwards
    const uint32_t hi = max(a, b), lo = min(a, b);
    a = hi;
    b = lo;
}
__device__ __forceinline__ void sort4_desc(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d) {
    cx_desc(a, b);
    cx_desc(c, d);
    cx_desc(a, c);
    cx_desc(b, d);
    cx_desc(b, c);
}
// a, b: descending lists of 4.  a becomes the descending top 4 of both:
// max(a_i, b_{3-i}) is that set as a bitonic sequence, then a half-cleaner
// merge sorts it.
__device__ __forceinline__ void merge_top4(uint32_t* a, const uint32_t* b) {
    uint32_t c0 = max(a[0], b[3]), c1 = max(a[1], b[2]), c2 = max(a[2], b[1]), c3 = max(a[3], b[0]);
    cx_desc(c0, c2);
    cx_desc(c1, c3);
    cx_desc(c0, c1);
    cx_desc(c2, c3);
    a[0] = c0;
    a[1] = c1;
    a[2] = c2;
    a[3] = c3;
}

__global__ void __launch_bounds__(256) encode_tile4_kernel(
    const uint16_t* __restrict__ keys, const uint16_t* __restrict__ cent,
    const int32_t* __restrict__ ids, uint16_t* __restrict__ payload, int32_t* __restrict__ meta,
    long rows, int T, int C, int struct_index) {
    const int lane = threadIdx.x & 63;
    const long row = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
    const int tile = lane & 7;
    if (row >= rows) return;
    const long bh = row / T;
    int cid = ids[row];
    cid = cid < 0 ? 0 : (cid > C - 1 ? C - 1 : cid);  // compression.cu:83-84
    const uint4* xp = reinterpret_cast<const uint4*>(keys + row * kDim + tile * 16);
    const uint4* cp = reinterpret_cast<const uint4*>(cent + (bh * C + cid) * kDim + tile * 16);
    const uint4 xa = xp[0], xb = xp[1], ca = cp[0], cb = cp[1];
    const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    const uint32_t cw[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
    uint32_t k[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, xw[i]) - __builtin_bit_cast(half2_t, cw[i]));
        const uint32_t lo = h & 0xFFFFu, hi = h >> 16;
        k[2 * i] = ((lo & 0x7FFFu) << 5) | ((uint32_t)(15 - 2 * i) << 1) | (lo >> 15);
        k[2 * i + 1] = ((hi & 0x7FFFu) << 5) | ((uint32_t)(14 - 2 * i) << 1) | (hi >> 15);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) sort4_desc(k[4 * g], k[4 * g + 1], k[4 * g + 2], k[4 * g + 3]);
    merge_top4(k, k + 4);
    merge_top4(k + 8, k + 12);
    // the top 4 of all 16 (unordered), re-keyed by channel: (15 - j) << 16 | fp16 bits
    uint32_t s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = max(k[i], k[11 - i]);
        s[i] = ((t & 0x1Eu) << 15) | ((t & 1u) << 15) | (t >> 5);
    }
    sort4_desc(s[0], s[1], s[2], s[3]);  // ascending channel
    uint2 pw;
    pw.x = (s[0] & 0xFFFFu) | (s[1] << 16);
    pw.y = (s[2] & 0xFFFFu) | (s[3] << 16);
    *reinterpret_cast<uint2*>(payload + row * 32 + tile * 4) = pw;
    uint32_t code = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t j = 15u - (s[i] >> 16);
        code |= struct_index ? j << (4 * i) : 1u << j;
    }
    // word w = code(tile 2w) | code(tile 2w+1) << 16
    const uint32_t other = dpp_u<0xB1>(code);  // quad xor 1: the neighbouring tile
    if ((tile & 1) == 0) meta[row * 4 + (tile >> 1)] = (int32_t)(code | (other << 16));
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

// ---------------------------------------------------------------------------
// Unstructured top-nnz with MSB-first bitmaps, eight lanes per token (lane
// 8 t + j owns channels 16 j .. 16 j + 15 of token t).  The nnz-th largest
// magnitude M comes from a 15-step search over the fp16 magnitude bits; each
// step counts the token's magnitudes below the candidate with packed 16-bit
// subtractions (sign bits gathered into one popcount) and three lane sums.
// Channels above M are kept, and the lowest-indexed channels equal to M fill
// the remainder (ties go to the lower channel, as with the composite key).
// ---------------------------------------------------------------------------
// Number of the lane's 16 magnitudes (packed pairs mp) below cand.
__device__ __forceinline__ int count_below(const uint32_t* mp, uint32_t cand) {
    const uint32_t cc = cand | (cand << 16);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // sign bit of each 16-bit difference: set where the magnitude is below cand
        const uint32_t d0 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2_t, mp[2 * i]) - __builtin_bit_cast(short2_t, cc));
        const uint32_t d1 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2_t, mp[2 * i + 1]) - __builtin_bit_cast(short2_t, cc));
        w[i] = __builtin_amdgcn_perm(d1, d0, 0x07050301u);  // the four high bytes
    }
    const uint32_t g = (w[0] & 0x80808080u) | ((w[1] >> 1) & 0x40404040u) | ((w[2] >> 2) & 0x20202020u) |
                       ((w[3] >> 3) & 0x10101010u);
    return __builtin_popcount(g);
}
// Sum over the 8 lanes of the lane's token (lanes 8t .. 8t+7), in every one of them.
__device__ __forceinline__ int token_sum8(int v) {
    v += (int)dpp_u<0xB1>((uint32_t)v);   // quad xor 1
    v += (int)dpp_u<0x4E>((uint32_t)v);   // quad xor 2
    v += (int)dpp_u<0x141>((uint32_t)v);  // half-row mirror: the other quad of the 8
    return v;
}
// Exclusive prefix sum over the lanes of the token, in channel order.
__device__ __forceinline__ int token_prefix8(int v, int j) {
    int x = v;
#pragma unroll
    for (int sh = 1; sh < 8; sh <<= 1) {
        const int o = __shfl_up(x, sh, 8);
        x += j >= sh ? o : 0;
    }
    return x - v;
}

__global__ void __launch_bounds__(256) encode_bitmap8_kernel(
    const uint16_t* __restrict__ keys, const uint16_t* __restrict__ cent,
    const int32_t* __restrict__ ids, uint16_t* __restrict__ payload, int64_t* __restrict__ meta,
    long rows, int T, int C, int nnz) {
    const int lane = threadIdx.x & 63;
    const long row = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
    const int tile = lane & 7;
    if (row >= rows) return;
    const long bh = row / T;
    int cid = ids[row];
    cid = cid < 0 ? 0 : (cid > C - 1 ? C - 1 : cid);  // compression.cu:83-84
    const uint4* xp = reinterpret_cast<const uint4*>(keys + row * kDim + tile * 16);
    const uint4* cp = reinterpret_cast<const uint4*>(cent + (bh * C + cid) * kDim + tile * 16);
    const uint4 xa = xp[0], xb = xp[1], ca = cp[0], cb = cp[1];
    const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    const uint32_t cw[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
    uint32_t hp[8], mp[8];  // fp16 residual pairs, their magnitudes
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hp[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, xw[i]) - __builtin_bit_cast(half2_t, cw[i]));
        mp[i] = hp[i] & 0x7FFF7FFFu;
    }
    // M = the largest magnitude with at least nnz of the token's magnitudes >= M
    uint32_t m = 0;
#pragma unroll 1
    for (int bit = 14; bit >= 0; --bit) {
        const uint32_t cand = m | (1u << bit);
        const int ge = kDim - token_sum8(count_below(mp, cand));
        m = ge >= nnz ? cand : m;
    }
    // channels above M, channels equal to M
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t v = (mp[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
        gt |= (v > m ? 1u : 0u) << i;
        eq |= (v == m ? 1u : 0u) << i;
    }
    const int need = nnz - token_sum8(__builtin_popcount(gt));  // ties to take, lowest channels first
    int quota = need - token_prefix8(__builtin_popcount(eq), tile);
    quota = quota < 0 ? 0 : quota;
    while (__builtin_popcount(eq) > quota) eq &= ~(0x80000000u >> __builtin_clz(eq));  // drop the highest tie
    const uint32_t sel = gt | eq;
    // payload: the token's kept residuals in channel order
    uint16_t* prow = payload + row * nnz + token_prefix8(__builtin_popcount(sel), tile);
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if ((sel >> i) & 1u) prow[__builtin_popcount(sel & ((1u << i) - 1u))] = (uint16_t)(hp[i >> 1] >> (16 * (i & 1)));
    // channel d -> bit (63 - d % 64) of word d / 64 (compression.py:87-88)
    const uint32_t rev = __builtin_bitreverse32(sel) >> 16;  // channel 16 tile + i -> bit 15 - i
    uint32_t lo = (tile & 1) ? rev : rev << 16, hi = lo;     // 32-bit halves of the tile pair
    lo = (tile & 2) ? lo : 0u;
    hi = (tile & 2) ? 0u : hi;
    lo |= dpp_u<0xB1>(lo);
    hi |= dpp_u<0xB1>(hi);
    lo |= dpp_u<0x4E>(lo);
    hi |= dpp_u<0x4E>(hi);
    if ((tile & 3) == 0) meta[row * 2 + (tile >> 2)] = (int64_t)(((uint64_t)hi << 32) | lo);
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
    if (nnz == 32 && (((uintptr_t)keys | (uintptr_t)centroids) & 15u) == 0 && ((uintptr_t)payload & 7u) == 0) {
        hipLaunchKernelGGL(encode_tile4_kernel, dim3((int)((rows + 31) / 32)), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)keys, (const uint16_t*)centroids, ids, (uint16_t*)payload, meta, rows, T,
                           C, struct_index);
        return reskv_host::check_launch("encode_tile4_kernel");
    }
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
    if ((((uintptr_t)keys | (uintptr_t)centroids) & 15u) == 0) {
        hipLaunchKernelGGL(encode_bitmap8_kernel, dim3((int)((rows + 31) / 32)), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)keys, (const uint16_t*)centroids, ids, (uint16_t*)payload, meta, rows, T,
                           C, nnz);
        return reskv_host::check_launch("encode_bitmap8_kernel");
    }
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
