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

// The tensors one launch encodes: side 0 and, for a layer's K and V in one
// launch, side 1 (grid dimension y for the 4:16 encoder, z for the bitmap
// encoder selects the side).
struct EncSides {
    const uint16_t* x[2];     // tokens fp16 [B*H*T, 128]
    const uint16_t* cent[2];  // centroids fp16 [B*H, C, 128]
    const int32_t* ids[2];    // cluster ids [B*H*T]
    uint16_t* payload[2];
    void* meta[2];
    int C[2];
};

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

__global__ void __launch_bounds__(256) encode_tile4_kernel(EncSides S, long rows, int T, int struct_index) {
    const int side = blockIdx.y;
    const uint16_t* __restrict__ keys = S.x[side];
    const uint16_t* __restrict__ cent = S.cent[side];
    const int32_t* __restrict__ ids = S.ids[side];
    uint16_t* __restrict__ payload = S.payload[side];
    int32_t* __restrict__ meta = static_cast<int32_t*>(S.meta[side]);
    const int C = S.C[side];
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
// Unstructured top-nnz with MSB-first bitmaps, four lanes per token (lane
// 4 t + q owns channels 32 q .. 32 q + 31 of token t; a wave encodes 16
// tokens).  The nnz-th largest 15-bit magnitude M is found bit by bit on byte
// planes: a lane's 32 magnitudes are split into a plane of high bytes (bits
// 14..8) and one of low bytes, four values per dword, byte k of dword i
// holding channel 32 q + 4 i + k.  A search step counts the bytes >= a
// candidate c with two sums of absolute byte differences (v_sad_u8, against
// c and c - 1), four values an instruction; the per-channel flags after each
// phase use ((v | 0x80) - c) & 0x80, set exactly when v >= c (v, c <= 0x80,
// no borrow crosses a byte).  Phases:
//   A: the high seven bits H of M over the high bytes;
//   B: bits 7..1 of M (L) over the low bytes >> 1 of the values whose high
//      byte is H (the others read as 0 and never count: candidates are >= 1),
//      on top of the count of values whose high byte exceeds H;
//   C: bit 0 of M over the values whose high byte is H and low bits 7..1 are L.
// Each step's count is summed over the token's four lanes (one quad) with two
// DPP adds.  Channels above M are kept, and the lowest-indexed channels equal
// to M fill the remainder (ties go to the lower channel, as with the
// composite key).  The kept values are compacted into the wave's LDS rows and
// written to the payload as 16-byte stores.
// ---------------------------------------------------------------------------
constexpr uint32_t kByteTop = 0x80808080u;  // bit 7 of every byte
constexpr uint32_t kByteOne = 0x01010101u;
constexpr int kBitmapTokensPerWave = 16;
constexpr int kBitmapDump = kBitmapTokensPerWave * kDim;  // per-wave LDS halves before the lanes' dump slots

// Sum over the four lanes of the lane's token (one DPP quad), in every one of them.
__device__ __forceinline__ int quad_sum(int v) {
    v += (int)dpp_u<0xB1>((uint32_t)v);  // quad xor 1
    v += (int)dpp_u<0x4E>((uint32_t)v);  // quad xor 2
    return v;
}
// Exclusive prefix sum over the quad, in lane (channel) order.
__device__ __forceinline__ int quad_prefix(int v, int q) {
    int s = v;
    const int a = (int)dpp_u<0x90>((uint32_t)s);  // quad_perm [0,0,1,2]: lane q - 1
    s += q >= 1 ? a : 0;
    const int b = (int)dpp_u<0x44>((uint32_t)s);  // quad_perm [0,1,0,1]: lane q - 2
    s += q >= 2 ? b : 0;
    return s - v;
}
// Bit-7 flags of the bytes of p (each ORed with 0x80 beforehand) that are >= the bytes of c4.
__device__ __forceinline__ uint32_t ge_flags(uint32_t p, uint32_t c4) { return (p - c4) & kByteTop; }
// Twice the number of the lane's 32 plane bytes (7-bit values, bit 7 clear)
// that are >= the bytes of c4 (each 1..127), minus 32: for a byte a,
// |a - c| - |a - (c - 1)| is -1 when a >= c and +1 otherwise, so two sums of
// absolute byte differences (v_sad_u8, four bytes an instruction) give the
// count without per-byte flags.
__device__ __forceinline__ int twice_count_ge_minus(const uint32_t* p, uint32_t c4) {
    uint32_t at = 0, below = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        at = __builtin_amdgcn_sad_u8(p[i], c4, at);
        below = __builtin_amdgcn_sad_u8(p[i], c4 - kByteOne, below);
    }
    return (int)below - (int)at;  // = 2 * count - 32
}
// Largest 7-bit c (as four equal bytes) with base + (token count of plane bytes >= c) >= nnz,
// over planes of 7-bit values.
__device__ __forceinline__ uint32_t search7(const uint32_t* p, int base, int nnz) {
    const int need = 2 * (nnz - base) - 4 * 32;  // 2 * count - 128 over the quad's 128 bytes
    uint32_t c4 = 0;
#pragma unroll
    for (int bit = 6; bit >= 0; --bit) {
        const uint32_t cand = c4 | (kByteOne << bit);
        c4 = quad_sum(twice_count_ge_minus(p, cand)) >= need ? cand : c4;
    }
    return c4;
}
__global__ void __launch_bounds__(256) encode_bitmap4_kernel(EncSides S, int T, int nnz, int bh0) {
    __shared__ __align__(16) uint16_t s_rows[kWavesPerBlock][kBitmapDump + kWave];
    const int side = blockIdx.z;
    const uint16_t* __restrict__ keys = S.x[side];
    const uint16_t* __restrict__ cent = S.cent[side];
    const int32_t* __restrict__ ids = S.ids[side];
    uint16_t* __restrict__ payload = S.payload[side];
    int64_t* __restrict__ meta = static_cast<int64_t*>(S.meta[side]);
    const int C = S.C[side];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3;
    const int t_wave = blockIdx.x * (kWavesPerBlock * kBitmapTokensPerWave) + wave * kBitmapTokensPerWave;
    if (t_wave >= T) return;  // whole waves
    const int t = t_wave + (lane >> 2);
    const bool valid = t < T;  // lanes past T compute on the last token and store nothing
    const long bh = (long)bh0 + blockIdx.y;
    const long row = bh * T + (valid ? t : T - 1);
    int cid = ids[row];
    cid = cid < 0 ? 0 : (cid > C - 1 ? C - 1 : cid);  // compression.cu:83-84
    const uint4* xp = reinterpret_cast<const uint4*>(keys + row * kDim + q * 32);
    const uint4* cp = reinterpret_cast<const uint4*>(cent + (bh * C + cid) * kDim + q * 32);
    uint32_t hp[16];  // fp16 residual pairs (channels 32 q + 2 i, + 1)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 xv = xp[j], cv = cp[j];
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, cw[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            hp[4 * j + k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, xw[k]) - __builtin_bit_cast(half2_t, cw[k]));
    }
    // byte planes of the magnitudes (sign bits dropped): hr = bits 14..8, lb =
    // bits 7..0; hb = hr with bit 7 of every byte set, for the flag tests
    uint32_t hr[8], hb[8], lb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t m0 = hp[2 * i] & 0x7FFF7FFFu, m1 = hp[2 * i + 1] & 0x7FFF7FFFu;
        hr[i] = __builtin_amdgcn_perm(m1, m0, 0x07050301u);
        hb[i] = hr[i] | kByteTop;
        lb[i] = __builtin_amdgcn_perm(m1, m0, 0x06040200u);
    }
    // A: high byte H of M
    const uint32_t h4 = search7(hr, 0, nnz);
    uint32_t gt_h[8], eq_h[8], l7r[8], l7[8];
    int above = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        gt_h[i] = ge_flags(hb[i], h4 + kByteOne);  // H + 1 <= 0x80: no carry between bytes
        eq_h[i] = ge_flags(hb[i], h4) & ~gt_h[i];
        above += __builtin_popcount(gt_h[i]);
        // bits 7..1 of the low byte where the high byte is H, else 0 (bytes of eq_h - (eq_h >> 7) are 0x7F or 0)
        l7r[i] = (lb[i] >> 1) & (eq_h[i] - (eq_h[i] >> 7));
        l7[i] = l7r[i] | kByteTop;
    }
    above = quad_sum(above);
    // B: bits 7..1 of M
    const uint32_t l4 = search7(l7r, above, nnz);
    uint32_t gt_l[8], eq_l[8], one[8];
    int above_l = 0, ones = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        gt_l[i] = ge_flags(l7[i], l4 + kByteOne);            // high byte H, bits 7..1 above L
        eq_l[i] = ge_flags(l7[i], l4) & ~gt_l[i] & eq_h[i];  // high byte H, bits 7..1 equal to L
        one[i] = eq_l[i] & (lb[i] << 7);                      // ... with bit 0 set
        above_l += __builtin_popcount(gt_l[i]);
        ones += __builtin_popcount(one[i]);
    }
    above += quad_sum(above_l);
    ones = quad_sum(ones);
    // C: bit 0 of M
    const bool m_odd = above + ones >= nnz;
    const int need = nnz - (m_odd ? above : above + ones);  // ties to take, lowest channels first
    uint32_t gt[8], eq[8];
    int n_eq = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        gt[i] = gt_h[i] | gt_l[i] | (m_odd ? 0u : one[i]);
        eq[i] = m_odd ? one[i] : eq_l[i] & ~one[i];
        n_eq += __builtin_popcount(eq[i]);
    }
    int quota = need - quad_prefix(n_eq, q);
    quota = quota < 0 ? 0 : quota;
    while (n_eq > quota) {  // drop the highest-channel tie
        int top = 0;
#pragma unroll
        for (int i = 1; i < 8; ++i) top = eq[i] ? i : top;
        uint32_t w = eq[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) w = i == top ? eq[i] : w;
        const uint32_t cleared = w & ~(0x80000000u >> __builtin_clz(w));
#pragma unroll
        for (int i = 0; i < 8; ++i) eq[i] = i == top ? cleared : eq[i];
        --n_eq;
    }
    // kept channels as a 32-bit mask, bit i = channel 32 q + i: the flag bytes
    // (0 or 1 after the shift) of two dwords weighted by 1..128 in one pair of
    // byte dot products give 8 mask bits
    uint32_t sel = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = (gt[2 * j] | eq[2 * j]) >> 7, hi = (gt[2 * j + 1] | eq[2 * j + 1]) >> 7;
        const uint32_t m = __builtin_amdgcn_udot4(lo, 0x08040201u, __builtin_amdgcn_udot4(hi, 0x80402010u, 0u, false),
                                                  false);
        sel |= m << (8 * j);
    }
    // the token keeps exactly nnz channels; the bound check keeps the LDS row
    // writes inside the row regardless
    const int kept = __builtin_popcount(sel);
    const int first = quad_prefix(kept, q);
    if (first + kept > nnz) sel = 0;
    // channel d -> bit (63 - d % 64) of word d / 64 (compression.py:87-88):
    // lane 2w holds the high half of word w, lane 2w + 1 the low half
    const uint32_t rev = __builtin_bitreverse32(sel);
    const uint32_t rev_next = dpp_u<0xB1>(rev);
    if (valid && (q & 1) == 0) meta[row * 2 + (q >> 1)] = (int64_t)(((uint64_t)rev << 32) | rev_next);
    // payload: kept residuals in channel order into the token's LDS row (others
    // to the lane's dump slot), then the wave's rows to HBM
    uint16_t* srow = s_rows[wave];
    uint16_t* my_row = srow + (lane >> 2) * nnz;
    uint16_t* dump = srow + kBitmapDump + lane;
    int rank = first;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int bit = (int)((sel >> i) & 1u);
        uint16_t* dst = bit ? my_row + rank : dump;
        *dst = (uint16_t)(hp[i >> 1] >> (16 * (i & 1)));
        rank += bit;
    }
    wave_sync();
    const int ntok = T - t_wave < kBitmapTokensPerWave ? T - t_wave : kBitmapTokensPerWave;
    uint16_t* grow = payload + (bh * T + t_wave) * (long)nnz;  // the wave's rows are contiguous
    const int halves = ntok * nnz;
    if ((nnz & 7) == 0) {
        const uint4* src = reinterpret_cast<const uint4*>(srow);
        uint4* dst = reinterpret_cast<uint4*>(grow);
        for (int c = lane; c < halves / 8; c += kWave) dst[c] = src[c];
    } else {
        for (int c = lane; c < halves; c += kWave) grow[c] = srow[c];
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

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// 4:16 fast path: nnz 32, 16-byte aligned tokens and centroids, 8-byte aligned payload.
bool tile4_ok(const EncSides& S, int sides, int nnz) {
    bool ok = nnz == 32;
    for (int i = 0; i < sides; ++i)
        ok = ok && aligned16(S.x[i]) && aligned16(S.cent[i]) && ((uintptr_t)S.payload[i] & 7u) == 0;
    return ok;
}
int launch_tile4(const EncSides& S, int sides, int B, int H, int T, int struct_index, hipStream_t st) {
    const long rows = (long)B * H * T;
    hipLaunchKernelGGL(encode_tile4_kernel, dim3((int)((rows + 31) / 32), sides), dim3(256), 0, st, S, rows, T,
                       struct_index);
    return reskv_host::check_launch("encode_tile4_kernel");
}

// bitmap fast path: 16-byte aligned tokens, centroids and payload.
bool bitmap4_ok(const EncSides& S, int sides) {
    bool ok = true;
    for (int i = 0; i < sides; ++i) ok = ok && aligned16(S.x[i]) && aligned16(S.cent[i]) && aligned16(S.payload[i]);
    return ok;
}
int launch_bitmap4(const EncSides& S, int sides, int B, int H, int T, int nnz, hipStream_t st) {
    const int BH = B * H;
    const int per_block = kWavesPerBlock * kBitmapTokensPerWave;
    for (int bh0 = 0; bh0 < BH; bh0 += 65535) {  // grid y covers at most 65535 (batch, head) rows
        const dim3 grid((T + per_block - 1) / per_block, BH - bh0 < 65535 ? BH - bh0 : 65535, sides);
        hipLaunchKernelGGL(encode_bitmap4_kernel, grid, dim3(256), 0, st, S, T, nnz, bh0);
        if (reskv_host::check_launch("encode_bitmap4_kernel")) return 1;
    }
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
    const EncSides S{{(const uint16_t*)keys, nullptr}, {(const uint16_t*)centroids, nullptr}, {ids, nullptr},
                     {(uint16_t*)payload, nullptr}, {meta, nullptr}, {C, 0}};
    if (tile4_ok(S, 1, nnz)) return launch_tile4(S, 1, B, H, T, struct_index, (hipStream_t)stream);
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
    const EncSides S{{(const uint16_t*)keys, nullptr}, {(const uint16_t*)centroids, nullptr}, {ids, nullptr},
                     {(uint16_t*)payload, nullptr}, {meta, nullptr}, {C, 0}};
    if (bitmap4_ok(S, 1)) return launch_bitmap4(S, 1, B, H, T, nnz, (hipStream_t)stream);
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

// A layer's K and V in one launch (grid side dimension); each result equals
// the single-tensor call's.  Inputs that miss the fast path's alignment run
// as two single-tensor calls.
extern "C" int reskv_compress_fp16_kv(const void* k, const void* v, const void* k_centroids,
                                      const void* v_centroids, const int32_t* k_ids, const int32_t* v_ids,
                                      void* k_payload, void* v_payload, int32_t* k_meta, int32_t* v_meta, int B,
                                      int H, int T, int Ck, int Cv, int nnz, int struct_index, void* stream) {
    if (check_common(k, k_centroids, k_ids, B, H, T, Ck) || check_common(v, v_centroids, v_ids, B, H, T, Cv))
        return 1;
    RESKV_REQUIRE(k_payload && v_payload && k_meta && v_meta, "null output pointer");
    const EncSides S{{(const uint16_t*)k, (const uint16_t*)v}, {(const uint16_t*)k_centroids, (const uint16_t*)v_centroids},
                     {k_ids, v_ids}, {(uint16_t*)k_payload, (uint16_t*)v_payload}, {k_meta, v_meta}, {Ck, Cv}};
    if (tile4_ok(S, 2, nnz) && (!struct_index || nnz == 32))
        return launch_tile4(S, 2, B, H, T, struct_index, (hipStream_t)stream);
    if (reskv_compress_fp16(k, k_centroids, k_ids, k_payload, k_meta, B, H, T, Ck, nnz, struct_index, stream))
        return 1;
    return reskv_compress_fp16(v, v_centroids, v_ids, v_payload, v_meta, B, H, T, Cv, nnz, struct_index, stream);
}

extern "C" int reskv_compress_bitmap_kv(const void* k, const void* v, const void* k_centroids,
                                        const void* v_centroids, const int32_t* k_ids, const int32_t* v_ids,
                                        void* k_payload, void* v_payload, int64_t* k_meta, int64_t* v_meta, int B,
                                        int H, int T, int Ck, int Cv, int nnz, void* stream) {
    if (check_common(k, k_centroids, k_ids, B, H, T, Ck) || check_common(v, v_centroids, v_ids, B, H, T, Cv))
        return 1;
    RESKV_REQUIRE(k_payload && v_payload && k_meta && v_meta, "null output pointer");
    RESKV_REQUIRE(nnz > 0 && nnz <= kDim, "nnz must be in [1, 128]");
    const EncSides S{{(const uint16_t*)k, (const uint16_t*)v}, {(const uint16_t*)k_centroids, (const uint16_t*)v_centroids},
                     {k_ids, v_ids}, {(uint16_t*)k_payload, (uint16_t*)v_payload}, {k_meta, v_meta}, {Ck, Cv}};
    if (bitmap4_ok(S, 2)) return launch_bitmap4(S, 2, B, H, T, nnz, (hipStream_t)stream);
    if (reskv_compress_bitmap(k, k_centroids, k_ids, k_payload, k_meta, B, H, T, Ck, nnz, stream)) return 1;
    return reskv_compress_bitmap(v, v_centroids, v_ids, v_payload, v_meta, B, H, T, Cv, nnz, stream);
}
