// Split-K fused decode attention over the compressed K/V cache (gfx950, wave64).
//
// Semantics (reskv/reference.py:59-91, reskv/csrc/cluster_mass.cu:4-11):
//   k_t = c_k[id_k(t)] + r_k(t)            (pre-RoPE key, fp32)
//   s_t = scaling * <rot(q, pos_q), rot(k_t, start + t)>
//   out = sum_t p_t (c_v[id_v(t)] + r_v(t)) / sum_t p_t,  p_t = exp(s_t - m)
// The Value centroids are applied once after the split reduction:
//   sum_t p_t c_v[id_v(t)] = sum_c beta_c c_v[c],  beta_c = sum_{t: id_v(t)=c} p_t.
// RoPE angles are fl32(position * inv_freq[i]) for rotate-half pairs (i, i+64),
// exactly as the reference oracle forms them; each angle is reduced modulo 2*pi
// with a three-part constant and evaluated by the hardware sin/cos.
//
// Partial kernel: one workgroup of 4 waves per (split, kv-head, batch).  A wave
// walks 16-token tiles of its split.  Each tile's raw bytes (ids, metadata,
// payload, scales) are copied with 16-byte buffer loads into the wave's LDS
// stage, prefetching the next tile into registers meanwhile; four lanes decode
// each token (details at the kernel).  Scores, P x V and the cluster mass beta
// run on the matrix cores; the online softmax runs per tile in the log2 domain.
// Merge kernel: one workgroup per (batch, query head) rescales the split
// partials to a common maximum, folds sum_c beta_c c_v[c] and normalises.
#include "common.h"
#include "../../include/reskv_hip.h"

#include <math.h>

#include <mutex>

using namespace reskv;

namespace {

// residual formats as the kernels see them (the two quantised widths split)
// (_W: the same layout with payload rows wider than 128 bytes, i.e. nnz > 64,
// which needs more prefetch registers per lane)
enum DFmt { D_BITMAP = 0, D_TILED, D_STRUCT16, D_SINT4, D_Q4, D_Q2, D_DENSE, D_BITMAP_W, D_TILED_W };

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kTile = 16;      // tokens per wave tile
constexpr int kMaxSplits = 1024;
constexpr int kPartStride = kDim + kMaxClusters + 2;  // cross-wave merge record
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kVPitch = kDim + 8;  // halves per token row of the V transpose tile (16-byte aligned rows; 132, 140 and 144 measured no faster)
constexpr int kCPitch = kDim + 4;  // halves per row of the LDS key-centroid table (66 dwords: 8-byte reads spread over the banks)
constexpr int kRowPad = 8;         // bytes after each staged payload row (34-dword rows for 128-byte payloads)

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// MB: metadata bytes per token; PQ: 16-byte payload pieces per lane and tile
// (the payload rows are staged in LDS, where the decoders gather from them);
// DEPTH: tiles prefetched ahead (two where the registers allow it); SC:
// per-token scale; CENT: centroid + residual.  Every lane loads its token's
// metadata row, cluster id and scale itself, so they need no LDS round trip.
// (Each lane loading only the payload bytes of its own channels straight into
// registers, two to four narrow loads per tensor instead of one 16-byte load
// per lane, measured 3-10% slower for INT2 and 4:16, equal for INT4.)
template <int F> struct Traits;
template <> struct Traits<D_BITMAP> { static constexpr int MB = 16, PQ = 2, DEPTH = 1; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_TILED> { static constexpr int MB = 16, PQ = 2, DEPTH = 1; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_BITMAP_W> { static constexpr int MB = 16, PQ = 4, DEPTH = 1; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_TILED_W> { static constexpr int MB = 16, PQ = 4, DEPTH = 1; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_STRUCT16> { static constexpr int MB = 16, PQ = 1, DEPTH = 1; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_SINT4> { static constexpr int MB = 8, PQ = 1, DEPTH = 2; static constexpr bool SC = true, CENT = true; };
template <> struct Traits<D_Q4> { static constexpr int MB = 0, PQ = 1, DEPTH = 2; static constexpr bool SC = true, CENT = true; };
template <> struct Traits<D_Q2> { static constexpr int MB = 0, PQ = 1, DEPTH = 2; static constexpr bool SC = true, CENT = true; };
template <> struct Traits<D_DENSE> { static constexpr int MB = 0, PQ = 4, DEPTH = 1; static constexpr bool SC = false, CENT = false; };

struct DTensor {
    const uint16_t* cent;     // fp16 [BH, nc, 128] (null for dense)
    const int8_t* ids;        // [BH, T] (null for dense)
    const uint8_t* payload;   // [BH, T, pb bytes]
    const uint8_t* meta;      // [BH, T, MB bytes] or null
    const uint16_t* scale;    // fp16 [BH, T] or null
    int nc, width, pb;        // pb: payload bytes per token, a multiple of 16
    int ts, cs;               // row strides: tokens per (batch, head) row block, centroid rows per table
};

struct DParams {
    const uint16_t* q;
    DTensor k, v;
    const float* inv_freq;
    const float4* rope;  // [position][16][cos x4, sin x4] table, or null (sin/cos evaluated in-kernel)
    int Hq, H, T, start_pos, pos_q, splits;
    float qscale;  // scaling * log2(e): scores come out in the log2 domain
    float one;     // 1.0f, opaque to the compiler: fp16 + fp16 sums as one mixed-precision FMA
    int stage_k, stage_v;  // LDS stage bytes per wave for K and V
    int lut_off, p_off, stage_off;  // LDS byte offsets (region 0 holds centroids / merge records)
    float* pm;
    float* pl;
    float* pd;
    float* pb;
};

// ---------------------------------------------------------------------------
// RoPE sin/cos of an fp32 angle: n = rint(a / 2pi); r = a - n * 2pi with 2pi
// split in three fp32 parts (exact products through FMA); the hardware sin/cos
// then take r / 2pi in revolutions, |r / 2pi| <= 1/2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rope_sincos_fast(float angle, float& s, float& c) {
    constexpr float kInv2Pi = 0.15915493667125702f;
    const float n = __builtin_rintf(angle * kInv2Pi);
    float r = __builtin_fmaf(-n, 6.2831854820251465f, angle);
    r = __builtin_fmaf(-n, -1.7484555314695172e-07f, r);
    r = __builtin_fmaf(-n, -6.8604980400235275e-15f, r);
    const float x = r * kInv2Pi;
    s = __builtin_amdgcn_sinf(x);
    c = __builtin_amdgcn_cosf(x);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// tile staging: global -> registers (prefetch) -> LDS
// ---------------------------------------------------------------------------
// 16-byte LDS accesses issued as two 8-byte halves
__device__ __forceinline__ uint4 lds_ld16(const void* p) {
    const uint2* q = reinterpret_cast<const uint2*>(p);
    const uint2 a = q[0], b = q[1];
    return make_uint4(a.x, a.y, b.x, b.y);
}
__device__ __forceinline__ void lds_st16(void* p, uint4 v) {
    uint2* q = reinterpret_cast<uint2*>(p);
    q[0] = make_uint2(v.x, v.y);
    q[1] = make_uint2(v.z, v.w);
}

__device__ __forceinline__ int clamp_id(int id, int nc) { return id < 0 ? 0 : (id >= nc ? nc - 1 : id); }

template <int F>
struct Prefetch {
    uint4 pay[Traits<F>::PQ];  // payload pieces, staged into LDS
    uint4 meta;  // this lane's token's metadata row (MB = 8: x, y)
    // its cluster id and fp16 scale bits as loaded: kept in their stored
    // widths and widened only where used, so that no conversion next to the
    // load (or at the loop's back edge) makes the prefetch wait for itself
    int8_t id;
    uint16_t sc;
};

// The bytes of one wave's token range [t0, t1) of one tensor as raw buffer
// resources: loads past the range return zero (hardware range check), so a
// partial last tile decodes to zero residuals without masks or zero fills.
constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw buffer, 32-bit data

template <int F>
struct WaveSrc {
    __amdgpu_buffer_rsrc_t pay, meta, ids, scale;
};

template <int F>
__device__ __forceinline__ WaveSrc<F> wave_src(const DTensor& X, long row0, int count) {
    using Tr = Traits<F>;
    WaveSrc<F> w;
    w.pay = __builtin_amdgcn_make_buffer_rsrc((void*)(X.payload + row0 * X.pb), 0, count * X.pb, kBufferWord3);
    w.meta = w.ids = w.scale = w.pay;
    if constexpr (Tr::MB > 0)
        w.meta = __builtin_amdgcn_make_buffer_rsrc((void*)(X.meta + row0 * Tr::MB), 0, count * Tr::MB, kBufferWord3);
    if constexpr (Tr::CENT)
        w.ids = __builtin_amdgcn_make_buffer_rsrc((void*)(X.ids + row0), 0, count, kBufferWord3);
    if constexpr (Tr::SC)
        w.scale = __builtin_amdgcn_make_buffer_rsrc((void*)(X.scale + row0), 0, count * 2, kBufferWord3);
    return w;
}

__device__ __forceinline__ uint4 buf_b128(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint2 buf_b64(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

// Loads the tile starting `off` tokens into the wave's range: the payload rows
// as 16-byte pieces q = lane + 64 i (bytes [16 (q % per_tok), +16) of row
// q / per_tok), and in lane L = 16 g + t token t's metadata row, cluster id
// and scale.
template <int F>
__device__ __forceinline__ void prefetch(const WaveSrc<F>& W, int pb, int off, int lane, Prefetch<F>& P) {
    using Tr = Traits<F>;
    constexpr int kOut = 0x7FFFFFF0;  // an offset past every range: the load returns zero
    const int tok = off + (lane & 15);
    const int per_tok = pb >> 4;
#pragma unroll
    for (int i = 0; i < Tr::PQ; ++i) {
        const int q = lane + kWave * i;
        P.pay[i] = buf_b128(W.pay, q < kTile * per_tok ? off * pb + 16 * q : kOut);
    }
    if constexpr (Tr::MB == 16) {
        P.meta = buf_b128(W.meta, tok * 16);
    } else if constexpr (Tr::MB == 8) {
        const uint2 m = buf_b64(W.meta, tok * 8);
        P.meta = make_uint4(m.x, m.y, 0, 0);
    }
    if constexpr (Tr::CENT) P.id = (int8_t)__builtin_amdgcn_raw_buffer_load_b8(W.ids, tok, 0, 0);
    if constexpr (Tr::SC) P.sc = __builtin_amdgcn_raw_buffer_load_b16(W.scale, tok * 2, 0, 0);
}

// Stage layout (bytes): payload [16][pb + kRowPad] | cluster ids uint8[16]
// (clamped to [0, nc - 1]; the Value ids feed the one-hot operand of the
// cluster mass).  The 8-byte row
// pad staggers consecutive payload rows over the LDS banks (16 lanes read 16
// different rows at similar offsets); rows are 8-byte aligned, so wide stage
// accesses are done as 8-byte halves.
template <int F>
__host__ __device__ constexpr int stage_bytes(int pb) {
    return kTile * (pb + kRowPad) + kTile;
}

// LDS byte offsets of this lane's payload pieces inside the stage, or -1 past
// the tile.  The same for every tile, so computed once.
template <int F>
__device__ __forceinline__ void stage_slots(int pb, int lane, int* slot) {
    const int per_tok = pb >> 4;
#pragma unroll
    for (int i = 0; i < Traits<F>::PQ; ++i) {
        const int q = lane + kWave * i;
        slot[i] = q < kTile * per_tok ? (q / per_tok) * (pb + kRowPad) + (q % per_tok) * 16 : -1;
    }
}

// IDS: also store the tile's clamped cluster ids as bytes.
template <int F, bool IDS>
__device__ __forceinline__ void stage_store(const Prefetch<F>& P, uint8_t* st, int pb, const int* slot, int lane,
                                            int nc) {
    using Tr = Traits<F>;
#pragma unroll
    for (int i = 0; i < Tr::PQ; ++i)
        if (slot[i] >= 0) lds_st16(st + slot[i], P.pay[i]);
    if (IDS && Tr::CENT && lane < kTile) {
        const int cid = clamp_id(P.id, nc);  // compression.cu:83-84
        st[kTile * (pb + kRowPad) + lane] = (uint8_t)cid;
    }
}

template <int F>
struct StageView {
    const uint8_t* st;
    int pp;  // payload row pitch (pb + kRowPad)
    __device__ const uint8_t* row(int t) const { return st + t * pp; }
    __device__ uint32_t ids4(int s) const {  // clamped ids of tokens 4s .. 4s+3, one byte each
        return reinterpret_cast<const uint32_t*>(st + kTile * pp)[s];
    }
};

// The payload dwords of lane (token t, group g) that its decoder reads:
// INT4 words 2g, 2g+1, 8+2g, 9+2g; INT2 words g, 4+g; 4:16 the 8-byte value
// words of tiles g and 4+g; structured INT4 words g/2, 2+g/2.  From the
// staged row.
template <int F>
__device__ __forceinline__ void lane_words(const StageView<F>& S, int t, int g, uint32_t* w) {
    const uint32_t* row = reinterpret_cast<const uint32_t*>(S.row(t));
    if constexpr (F == D_Q4 || F == D_STRUCT16) {
        const uint2 a = *reinterpret_cast<const uint2*>(row + 2 * g);
        const uint2 b = *reinterpret_cast<const uint2*>(row + 8 + 2 * g);
        w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y;
    } else if constexpr (F == D_Q2) {
        w[0] = row[g]; w[1] = row[4 + g];
    } else if constexpr (F == D_SINT4) {
        w[0] = row[g >> 1]; w[1] = row[2 + (g >> 1)];
    }
}

// ---------------------------------------------------------------------------
// residual decoders.  Lane L = 16 g + t owns token t of the tile and channel
// group g: channels 16g..16g+15 (values m = 0..15) and 64+16g..64+16g+15
// (m = 16..31), i.e. the sixteen rotate-half RoPE pairs (m, m + 16).
// FP16 formats yield the residuals as fp16 pairs h[i] = values (2i, 2i+1).
//
// A group's channels are four runs of four.  The kept values of a run are
// consecutive in the payload row, starting at rank `base`; the 8-byte window at
// `base` is fetched with dword reads plus an alignbit, and one v_perm per
// channel pair scatters the window's halves onto the kept channels (zeros
// elsewhere).  The permute selectors depend only on the run's 4-bit keep
// pattern and come from a 16-entry table in LDS (one table for MSB-first
// bitmaps, one for LSB-first tile masks).  The ranks of a lane's runs follow
// from the first one by popcounts of the patterns.
// ---------------------------------------------------------------------------
constexpr int kLutWords = 64;        // [msb|lsb][pattern][lo|hi]
constexpr int kStructLutWords = 160;  // 4:16 tiles: [start rank 0..4][pattern][lo|hi]
constexpr int kQTrigWords = 128;      // cos, then sin, of the query position for the 64 RoPE pairs

// v_perm selector bytes placing window halves on channels 0..3 of a run
// (byte 12 selects zero).  msb: pattern bit 3-j = channel j (bitmaps);
// otherwise bit j = channel j (tile masks).
__host__ __device__ constexpr uint32_t perm_selector(uint32_t v, bool msb, int half) {
    uint32_t sel = 0;
    for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * half + jj;
        const bool kept = msb ? ((v >> (3 - j)) & 1u) : ((v >> j) & 1u);
        const uint32_t rank = msb ? (uint32_t)__builtin_popcount(v >> (4 - j))
                                  : (uint32_t)__builtin_popcount(v & ((1u << j) - 1u));
        const uint32_t b0 = kept ? 2 * rank : 12u, b1 = kept ? 2 * rank + 1 : 12u;
        sel |= (b0 | (b1 << 8)) << (16 * jj);
    }
    return sel;
}

// Selectors for a 4:16 tile: the tile's four values are one 8-byte word, and a
// run whose first kept value has rank `rank` takes bytes 2 (rank + i) of that
// word directly (LSB-first pattern, bit j = channel j).
__host__ __device__ constexpr uint32_t struct_selector(uint32_t v, uint32_t rank, int half) {
    uint32_t sel = 0;
    for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * half + jj;
        const uint32_t pos = rank + (uint32_t)__builtin_popcount(v & ((1u << j) - 1u));
        const bool kept = ((v >> j) & 1u) && pos < 4;
        const uint32_t b0 = kept ? 2 * pos : 12u, b1 = kept ? 2 * pos + 1 : 12u;
        sel |= (b0 | (b1 << 8)) << (16 * jj);
    }
    return sel;
}

__device__ __forceinline__ float half_lo(uint32_t w) { return h2f((uint16_t)(w & 0xFFFFu)); }
__device__ __forceinline__ float half_hi(uint32_t w) { return h2f((uint16_t)(w >> 16)); }
__device__ __forceinline__ int popc(uint32_t v) { return __builtin_popcount(v); }

// Four consecutive runs of a lane's half-group, patterns pat[0..3], the first
// at rank r.  A run's third window dword matters only for a full run at an
// odd rank; the next run then starts four ranks on, so that dword is the next
// run's first one.  Each run therefore reads two dwords and the group one more
// for its last run (36 bytes instead of 48).
__device__ __forceinline__ void runs4_h(const uint8_t* row, int r, const uint32_t* tab, const uint32_t* pat,
                                        uint32_t* out) {
    const uint32_t* base = reinterpret_cast<const uint32_t*>(row);
    int rk[4];
    rk[0] = r;
#pragma unroll
    for (int u = 0; u < 3; ++u) rk[u + 1] = rk[u] + popc(pat[u]);
    uint32_t d0[4], d1[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        d0[u] = base[rk[u] >> 1];
        d1[u] = base[(rk[u] >> 1) + 1];
    }
    const uint32_t dlast = base[(rk[3] >> 1) + 2];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t d2 = u < 3 ? d0[u + 1] : dlast;
        const uint32_t sh = (uint32_t)(rk[u] & 1) * 16u;
        const uint32_t w0 = __builtin_amdgcn_alignbit(d1[u], d0[u], sh);
        const uint32_t w1 = __builtin_amdgcn_alignbit(d2, d1[u], sh);
        const uint2 sel = *reinterpret_cast<const uint2*>(tab + 2 * pat[u]);
        out[2 * u] = __builtin_amdgcn_perm(w1, w0, sel.x);
        out[2 * u + 1] = __builtin_amdgcn_perm(w1, w0, sel.y);
    }
}

// Bits of a bitmap word's channels that come before group g (channel d sits at
// bit 63 - d): bits [64 - 16 g, 63], split into the word's high and low dword.
struct GroupMask {
    uint32_t hi, lo;
};
__device__ __forceinline__ GroupMask group_mask(int g) {
    return {g == 0 ? 0u : (g == 1 ? 0xFFFF0000u : 0xFFFFFFFFu), g == 3 ? 0xFFFF0000u : 0u};
}

template <int F>
constexpr bool kHalfFmt = F == D_BITMAP || F == D_BITMAP_W || F == D_TILED || F == D_TILED_W ||
                          F == D_STRUCT16 || F == D_DENSE;

template <int F>
__device__ __forceinline__ void residual_h(const StageView<F>& S, const Prefetch<F>& R, int t, int g, int width,
                                           GroupMask gm, const uint32_t* lut, uint32_t* h) {
    const uint8_t* row = S.row(t);
    if constexpr (F == D_BITMAP || F == D_BITMAP_W) {
        // words: channels 0..63 in (m.y:m.x), 64..127 in (m.w:m.z), MSB-first
        // (reference.py:22-26); group g's 16 channels are the (g odd ? low : high)
        // half of dword (g < 2 ? high : low), channel 16g + c at field bit 15 - c
        const uint4 m = R.meta;
        const uint32_t sh = (g & 1) ? 0u : 16u;
        const uint32_t f0 = ((g < 2 ? m.y : m.x) >> sh) & 0xFFFFu;
        const uint32_t f1 = ((g < 2 ? m.w : m.z) >> sh) & 0xFFFFu;
        const int r0 = popc(m.y & gm.hi) + popc(m.x & gm.lo);
        const int r1 = popc(m.y) + popc(m.x) + popc(m.w & gm.hi) + popc(m.z & gm.lo);
        uint32_t pa[4], pc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            pa[u] = (f0 >> (12 - 4 * u)) & 15u;
            pc[u] = (f1 >> (12 - 4 * u)) & 15u;
        }
        runs4_h(row, r0, lut, pa, h);
        runs4_h(row, r1, lut, pc, h + 8);
    } else if constexpr (F == D_TILED || F == D_TILED_W || F == D_STRUCT16) {
        // word w = code(tile 2w) | code(tile 2w+1) << 16 (reference.py:36-47);
        // group g covers tiles g and 4 + g
        const uint4 m = R.meta;
        const uint32_t sh = (uint32_t)(g & 1) * 16u;
        uint32_t f0 = ((g < 2 ? m.x : m.y) >> sh) & 0xFFFFu;
        uint32_t f1 = ((g < 2 ? m.z : m.w) >> sh) & 0xFFFFu;
        if constexpr (F == D_STRUCT16) {
            // four ascending in-tile channel indices -> 16-bit mask; the tile's
            // four values are one 8-byte word, and the (rank, pattern) selectors
            // pick each run's values from it
            uint32_t k0 = 0, k1 = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                k0 |= 1u << ((f0 >> (4 * j)) & 15u);
                k1 |= 1u << ((f1 >> (4 * j)) & 15u);
            }
            uint32_t w[4];
            lane_words<F>(S, t, g, w);
            const uint2 pa = make_uint2(w[0], w[1]);  // tile g's four values
            const uint2 pb = make_uint2(w[2], w[3]);  // tile 4 + g's
            const uint32_t* slut = lut + kLutWords;
            int r0 = 0, r1 = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t a = (k0 >> (4 * u)) & 15u, c = (k1 >> (4 * u)) & 15u;
                // ranks stay within 0..4: the mask has at most four bits
                const uint2 sa = *reinterpret_cast<const uint2*>(slut + 2 * (16 * r0 + (int)a));
                const uint2 sb = *reinterpret_cast<const uint2*>(slut + 2 * (16 * r1 + (int)c));
                h[2 * u] = __builtin_amdgcn_perm(pa.y, pa.x, sa.x);
                h[2 * u + 1] = __builtin_amdgcn_perm(pa.y, pa.x, sa.y);
                h[8 + 2 * u] = __builtin_amdgcn_perm(pb.y, pb.x, sb.x);
                h[8 + 2 * u + 1] = __builtin_amdgcn_perm(pb.y, pb.x, sb.y);
                r0 += popc(a);
                r1 += popc(c);
            }
        } else {
            const int per_tile = width >> 3;
            uint32_t pa[4], pc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                pa[u] = (f0 >> (4 * u)) & 15u;
                pc[u] = (f1 >> (4 * u)) & 15u;
            }
            runs4_h(row, g * per_tile, lut + 32, pa, h);
            runs4_h(row, (4 + g) * per_tile, lut + 32, pc, h + 8);
        }
    } else if constexpr (F == D_DENSE) {
        const uint4* r = reinterpret_cast<const uint4*>(row);  // staged rows
        const uint4 a = lds_ld16(r + 2 * g), b = lds_ld16(r + 2 * g + 1), c = lds_ld16(r + 8 + 2 * g),
                    d = lds_ld16(r + 9 + 2 * g);
        const uint32_t v[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) h[i] = v[i];
    }
}

// Structured INT4 residuals in fp32, value m of the lane's channels: 1 of 4
// per subgroup of four channels, 2-bit position, signed nibble code, fp16
// scale (reference.py:27-35); group g holds subgroups 4g..4g+3 (word g/2 of
// the payload row) and 16+4g..16+4g+3 (word 2 + g/2).
template <int F>
__device__ __forceinline__ void residual_f(const StageView<F>& S, const Prefetch<F>& R, int t, int g, float* r) {
    static_assert(F == D_SINT4, "structured INT4 only");
    const float s = h2f(R.sc);
    const uint2 qm = make_uint2(R.meta.x, R.meta.y);
    uint32_t w[2];
    lane_words<F>(S, t, g, w);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int off = 4 * (4 * (g & 1) + u);
        const float vl = (float)(int)__builtin_amdgcn_sbfe((int)w[0], off, 4) * s;
        const float vh = (float)(int)__builtin_amdgcn_sbfe((int)w[1], off, 4) * s;
        const uint32_t sl = (qm.x >> (2 * (4 * g + u))) & 3u, shh = (qm.y >> (2 * (4 * g + u))) & 3u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r[4 * u + j] = (uint32_t)j == sl ? vl : 0.0f;
            r[16 + 4 * u + j] = (uint32_t)j == shh ? vh : 0.0f;
        }
    }
}

// Signed INT4 / INT2 codes of the lane's channel pairs as exact fp16 pairs
// (h[i] = values 2i, 2i + 1), without the scale.  Codes are biased to
// unsigned fields by flipping their sign bits (u = code + 2^(bits-1)).  One
// byte permute copies the pair's byte under an fp16 high byte 0x64 into both
// halves (0x64bb: 1024 + bb, ulp 1); a mask keeps one field per half, which
// then reads 1024 + u * 2^k for the field's bit offset k within the byte; one
// packed fp16 FMA scales by 2^-k and subtracts 1024 / 2^k + 2^(bits-1),
// leaving the code.  Every step is exact.
template <int F>
__device__ __forceinline__ void code_halves(const StageView<F>& S, const Prefetch<F>& R, int t, int g, uint32_t* h) {
    constexpr uint32_t kMagic = 0x64646464u;
    uint32_t lw[4];
    lane_words<F>(S, t, g, lw);
    if constexpr (F == D_Q4) {
        // channel d in word d / 8 at bits 4 (d % 8): pair i of a word is its
        // byte i, low nibble first (reference.py:17-21); words 2g, 2g + 1 hold
        // channels 16g..16g+15 and words 8 + 2g, 9 + 2g channels 64+16g..64+16g+15
        const half2_t mul = {(_Float16)1.0f, (_Float16)0.0625f}, add = {(_Float16)-1032.0f, (_Float16)-72.0f};
        const uint32_t w[4] = {lw[0], lw[1], lw[2], lw[3]};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t x = w[k] ^ 0x88888888u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t d = __builtin_amdgcn_perm(kMagic, x, 0x04000400u + 0x00010001u * (uint32_t)j);
                const half2_t e = __builtin_bit_cast(half2_t, d & 0xFFF0FF0Fu);  // 1024 + u0 | 1024 + 16 u1
                h[4 * k + j] = __builtin_bit_cast(uint32_t, e * mul + add);
            }
        }
    } else {
        // channel d in word d / 16 at bits 2 (d % 16): pair p of a word is its
        // nibble p; word g holds channels 16g..16g+15, word 4 + g 64+16g..
        const half2_t mul_e = {(_Float16)1.0f, (_Float16)0.25f}, add_e = {(_Float16)-1026.0f, (_Float16)-258.0f};
        const half2_t mul_o = {(_Float16)0.0625f, (_Float16)0.015625f}, add_o = {(_Float16)-66.0f, (_Float16)-18.0f};
        const uint32_t w[2] = {lw[0], lw[1]};
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t x = w[k] ^ 0xAAAAAAAAu;
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const uint32_t d = __builtin_amdgcn_perm(kMagic, x, 0x04000400u + 0x00010001u * (uint32_t)(p >> 1));
                // even nibble: fields at bits 0-1 and 2-3 of the byte; odd: 4-5 and 6-7
                const half2_t e = __builtin_bit_cast(half2_t, d & ((p & 1) ? 0xFFC0FF30u : 0xFF0CFF03u));
                h[8 * k + p] = __builtin_bit_cast(uint32_t, (p & 1) ? e * mul_o + add_o : e * mul_e + add_e);
            }
        }
    }
}

// Key values of the lane's 32 channels (pre-RoPE, fp32): centroid + residual.
// fp16 + fp16 (or fp16 + fp32) sums run as one mixed-precision FMA by `one`.
template <int F>
__device__ __forceinline__ void key_values(const StageView<F>& S, const Prefetch<F>& R, int t, int g, int width,
                                           GroupMask gm, const uint32_t* lut, const uint16_t* s_cent, int nc,
                                           float one, float* x) {
    uint32_t c[16];
    if constexpr (Traits<F>::CENT) {
        const int kid = clamp_id(R.id, nc);  // compression.cu:83-84
        const uint4* cr = reinterpret_cast<const uint4*>(s_cent + kid * kCPitch);
        const uint4 a = lds_ld16(cr + 2 * g), b = lds_ld16(cr + 2 * g + 1), d = lds_ld16(cr + 8 + 2 * g), e = lds_ld16(cr + 9 + 2 * g);
        const uint32_t v[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, d.x, d.y, d.z, d.w, e.x, e.y, e.z, e.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) c[i] = v[i];
    }
    if constexpr (kHalfFmt<F>) {
        uint32_t h[16];
        residual_h<F>(S, R, t, g, width, gm, lut, h);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if constexpr (Traits<F>::CENT) {
                x[2 * i] = __builtin_fmaf(half_lo(h[i]), one, half_lo(c[i]));
                x[2 * i + 1] = __builtin_fmaf(half_hi(h[i]), one, half_hi(c[i]));
            } else {
                x[2 * i] = half_lo(h[i]);
                x[2 * i + 1] = half_hi(h[i]);
            }
        }
    } else if constexpr (F == D_Q4 || F == D_Q2) {
        // code * scale + centroid: one mixed-precision FMA per channel
        uint32_t h[16];
        code_halves<F>(S, R, t, g, h);
        const float sc = h2f(R.sc);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            x[2 * i] = __builtin_fmaf(half_lo(h[i]), sc, half_lo(c[i]));
            x[2 * i + 1] = __builtin_fmaf(half_hi(h[i]), sc, half_hi(c[i]));
        }
    } else {
        float r[32];
        residual_f<F>(S, R, t, g, r);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            x[2 * i] = __builtin_fmaf(half_lo(c[i]), one, r[2 * i]);
            x[2 * i + 1] = __builtin_fmaf(half_hi(c[i]), one, r[2 * i + 1]);
        }
    }
}

// Value residuals of the lane's 32 channels as fp16 pairs for the matrix cores.
// FP16 formats hand their payload halves through unchanged.  Quantised codes
// times the fp16 scale are rounded once to fp16: one packed fp16 multiply of
// the exact codes for the unstructured formats, fp32 then a conversion for
// the structured one.  (Folding the Value scale into the softmax weight
// instead, fp16(p * scale) times the exact codes, measured no faster: the
// second weight tile's LDS traffic takes what the multiplies save.)
template <int F>
__device__ __forceinline__ void value_halves(const StageView<F>& S, const Prefetch<F>& R, int t, int g, int width,
                                             GroupMask gm, const uint32_t* lut, uint32_t* h) {
    if constexpr (kHalfFmt<F>) {
        residual_h<F>(S, R, t, g, width, gm, lut, h);
    } else if constexpr (F == D_Q4 || F == D_Q2) {
        uint32_t c[16];
        code_halves<F>(S, R, t, g, c);
        const _Float16 sh = __builtin_bit_cast(_Float16, R.sc);  // the stored fp16 scale
        const half2_t s2 = {sh, sh};
#pragma unroll
        for (int i = 0; i < 16; ++i) h[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, c[i]) * s2);
    } else {
        float r[32];
        residual_f<F>(S, R, t, g, r);
#pragma unroll
        for (int i = 0; i < 16; ++i) h[i] = (uint32_t)f2h(r[2 * i]) | ((uint32_t)f2h(r[2 * i + 1]) << 16);
    }
}

// ---------------------------------------------------------------------------
// cross-lane reductions of the score layout
// ---------------------------------------------------------------------------
__device__ __forceinline__ float swap32_sum(float a, float b) {  // lanes < 32: a + a^32; others: b + b^32
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)f2i(a), (uint32_t)f2i(b), false, false);
    return i2f((int)r[0]) + i2f((int)r[1]);
}
__device__ __forceinline__ float swap16_sum(float a, float b) {  // even rows: a + a^16; odd rows: b + b^16
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)f2i(a), (uint32_t)f2i(b), false, false);
    return i2f((int)r[0]) + i2f((int)r[1]);
}
// Max / sum over the 16 lanes with the same (lane & 3), result in each of them.
__device__ __forceinline__ float head_max(float v) {
    v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
    v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
    auto a = __builtin_amdgcn_permlane32_swap((uint32_t)f2i(v), (uint32_t)f2i(v), false, false);
    v = fmaxf(i2f((int)a[0]), i2f((int)a[1]));
    auto c = __builtin_amdgcn_permlane16_swap((uint32_t)f2i(v), (uint32_t)f2i(v), false, false);
    return fmaxf(i2f((int)c[0]), i2f((int)c[1]));
}
__device__ __forceinline__ float head_sum(float v) {
    v += dpp<0x124>(v);
    v += dpp<0x128>(v);
    v = swap32_sum(v, v);
    return swap16_sum(v, v);
}

// ---------------------------------------------------------------------------
// partial kernel
//
// A wave walks 16-token tiles of its quarter of the split.  Lane L = 16 g + t
// decodes token t, channel group g of K (centroid + residual, RoPE from the
// table) and of V.  Scores run on v_mfma_f32_4x4x1f32: block b (lanes
// 4b..4b+3) multiplies tokens 4(b&3)+i of group b>>2 by query heads j = 0..3
// held in the same lanes, one channel per instruction, 32 instructions per
// tile; two lane swaps then add the four groups, leaving lane L with the
// score of token 4((L>>2)&3) + (L>>4) for head (L&3) (+4 for the second set
// of four heads when G = 8).  The online softmax takes one exponential per
// lane; the weights, rounded to fp16, drive P x V on v_mfma_f32_4x4x4f16
// through a per-wave transpose tile, and the cluster mass beta on the same
// instruction with a one-hot B operand (the tokens' V clusters against
// cluster `lane`), which keeps it in registers.
// ---------------------------------------------------------------------------
// Waves per SIMD the register allocation aims at: three (at most 168 VGPRs)
// for the quantised formats, whose decode needs few registers and gains from
// the third workgroup per CU; two otherwise.
template <int G, int KF, int VF>
constexpr int partial_waves() {
    return (G <= 4 && (KF == D_Q4 || KF == D_Q2) && (VF == D_Q4 || VF == D_Q2)) ? 3 : 1;
}

template <int G, int KF, int VF, bool TAB>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(partial_waves<G, KF, VF>())))
decode_partial_kernel(DParams P) {
    extern __shared__ __align__(16) uint8_t smem[];
    using KT = Traits<KF>;
    using VT = Traits<VF>;
    constexpr int NH = (G + 3) / 4;  // sets of four query heads
    // One-dimensional grid of splits * H * B workgroups.  Workgroups are
    // dispatched to the eight XCDs in turn (linear id w on XCD w % 8), each
    // with its own L2; work items i = (split, head, batch), split-major, are
    // handed out so that each XCD takes one contiguous block of them, i.e.
    // whole splits: its workgroups then read the RoPE table rows of their own
    // share of the positions only, which stays resident in that XCD's L2.
    int split, h, b;
    {
        const int n = (int)gridDim.x, w = (int)blockIdx.x;
        const int x = w & 7, q = n >> 3, r = n & 7;
        const int i = x * q + (x < r ? x : r) + (w >> 3);
        const int pairs = n / P.splits;  // H * B
        split = i / pairs;
        const int pr = i - split * pairs;
        b = pr / P.H;
        h = pr - b * P.H;
    }
    const long bh = (long)b * P.H + h;
    const int s0 = (int)(((long)split * P.T) / P.splits);
    const int s1 = (int)(((long)(split + 1) * P.T) / P.splits);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar registers
    const int t = lane & 15, grp = lane >> 4;  // decode: token of the tile, channel group
    const int hj = lane & 3;                     // query head of this lane within a set
    const int stok = 4 * ((lane >> 2) & 3) + (lane >> 4);  // token of this lane's score
    // this wave's contiguous share of the split
    const int t0 = s0 + (int)(((long)wave * (s1 - s0)) / kWaves);
    const int t1 = s0 + (int)(((long)(wave + 1) * (s1 - s0)) / kWaves);

    uint16_t* s_cent = reinterpret_cast<uint16_t*>(smem);  // region 0: fp16 key centroids [nc][kCPitch]
    uint32_t* s_lut = reinterpret_cast<uint32_t*>(smem + P.lut_off);
    // per wave: fp16 weights [4-token group][head][token] and the V tile [token][kVPitch]
    // per wave: fp16 weights [4-token group][head][token] and the V tile [token][kVPitch]
    uint16_t* my_p = reinterpret_cast<uint16_t*>(smem + P.p_off) + wave * (kTile * G + kTile * kVPitch);
    uint16_t* my_vt = my_p + kTile * G;
    uint8_t* st_k = smem + P.stage_off + wave * (P.stage_k + P.stage_v);
    uint8_t* st_v = st_k + P.stage_k;
    const StageView<KF> SK{st_k, P.k.pb + kRowPad};
    const StageView<VF> SV{st_v, P.v.pb + kRowPad};
    const GroupMask gm = group_mask(grp);

    // The first tiles' loads go out before the set-up work below, which then
    // overlaps their latency.
    const int ntiles = (t1 - t0 + kTile - 1) / kTile;
    const WaveSrc<KF> wk = wave_src<KF>(P.k, bh * P.k.ts + t0, t1 - t0);
    const WaveSrc<VF> wv = wave_src<VF>(P.v, bh * P.v.ts + t0, t1 - t0);
    // Tiles are prefetched kDepth ahead into register buffers used in turn
    // (two for the quantised formats, whose short tiles would otherwise wait
    // on the load latency; one for the others, and for G = 8, whose registers
    // do not allow two).
    constexpr int kDepth = (KT::DEPTH == 2 && VT::DEPTH == 2 && G <= 4) ? 2 : 1;
    Prefetch<KF> pk[kDepth];
    Prefetch<VF> pv[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        pk[d] = Prefetch<KF>{};
        pv[d] = Prefetch<VF>{};
        if (d < ntiles) {
            prefetch<KF>(wk, P.k.pb, d * kTile, lane, pk[d]);
            prefetch<VF>(wv, P.v.pb, d * kTile, lane, pv[d]);
        }
    }

    // cos and sin of the query position, once per workgroup (one pair per
    // thread of the first wave); every lane reads its group's 16 after the
    // barrier below.  The region follows the permute tables and is not
    // written again.
    float* s_qtrig = reinterpret_cast<float*>(s_lut + kLutWords + kStructLutWords);
    if (threadIdx.x < kHalf) {
        float sn, cs;
        rope_sincos_fast(__fmul_rn((float)P.pos_q, P.inv_freq[threadIdx.x]), sn, cs);
        s_qtrig[threadIdx.x] = cs;
        s_qtrig[kHalf + threadIdx.x] = sn;
    }
    if (threadIdx.x < kLutWords) {
        const uint32_t i = threadIdx.x;
        s_lut[i] = perm_selector((i >> 1) & 15u, i < 32, (int)(i & 1));
    } else if (threadIdx.x < kLutWords + kStructLutWords) {
        const uint32_t i = threadIdx.x - kLutWords;
        s_lut[kLutWords + i] = struct_selector((i >> 1) & 15u, i >> 5, (int)(i & 1));
    }

    if constexpr (KT::CENT) {
        const uint4* kc = reinterpret_cast<const uint4*>(P.k.cent + bh * P.k.cs * kDim);
        for (int i = threadIdx.x; i < P.k.nc * (kDim / 8); i += kThreads)
            lds_st16(s_cent + (i >> 4) * kCPitch + 8 * (i & 15), kc[i]);
    }

    // frequencies of this lane's 16 pairs (the keys' angles without a table)
    float fr[16];
    {
        const float4* fq = reinterpret_cast<const float4*>(P.inv_freq + 16 * grp);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 f = fq[u];
            fr[4 * u] = f.x;
            fr[4 * u + 1] = f.y;
            fr[4 * u + 2] = f.z;
            fr[4 * u + 3] = f.w;
        }
    }
    // the query rows of this lane's channels (fp16 pairs), loaded before the
    // barrier; rotated and pre-scaled for heads 4 hs + hj after it
    uint32_t qlo[NH][8], qhi[NH][8];
#pragma unroll
    for (int hs = 0; hs < NH; ++hs) {
        const int g = 4 * hs + hj;
#pragma unroll
        for (int i = 0; i < 8; ++i) qlo[hs][i] = qhi[hs][i] = 0u;
        if (g < G) {
            const uint4* qr = reinterpret_cast<const uint4*>(P.q + ((long)b * P.Hq + (long)h * G + g) * kDim);
            const uint4 a = qr[2 * grp], c = qr[2 * grp + 1], d = qr[8 + 2 * grp], e = qr[9 + 2 * grp];
            const uint32_t vl[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
            const uint32_t vh[8] = {d.x, d.y, d.z, d.w, e.x, e.y, e.z, e.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                qlo[hs][i] = vl[i];
                qhi[hs][i] = vh[i];
            }
        }
    }

    // P x V sums (v_mfma_f32_4x4x4f16, 16 blocks of 4 lanes): lane L
    // accumulates delta[4 hs + i][L + 64 half] in acc[hs][half][i]
    // cluster masses on the same matrix cores: B = one-hot of the tokens' V
    // clusters against cluster `lane`, so lane L accumulates beta[4 hs + i][L] in accb[hs][i]
    float4_t acc[NH][2], accb[NH];
    float m_run[NH], lv[NH];
#pragma unroll
    for (int hs = 0; hs < NH; ++hs) {
        acc[hs][0] = acc[hs][1] = accb[hs] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
        m_run[hs] = -INFINITY;
        lv[hs] = 0.0f;
    }
    int kslot[KT::PQ], vslot[VT::PQ];
    const uint32_t lane_bytes = (uint32_t)lane * 0x01010101u;
    stage_slots<KF>(P.k.pb, lane, kslot);
    stage_slots<VF>(P.v.pb, lane, vslot);
    __syncthreads();

    float qv[NH][32];
    {
        float sn[16], cs[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            cs[m] = s_qtrig[16 * grp + m];
            sn[m] = s_qtrig[kHalf + 16 * grp + m];
        }
#pragma unroll
        for (int hs = 0; hs < NH; ++hs) {
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                const float a = (m & 1) ? half_hi(qlo[hs][m >> 1]) : half_lo(qlo[hs][m >> 1]);
                const float c = (m & 1) ? half_hi(qhi[hs][m >> 1]) : half_lo(qhi[hs][m >> 1]);
                qv[hs][m] = (a * cs[m] - c * sn[m]) * P.qscale;
                qv[hs][16 + m] = (c * cs[m] + a * sn[m]) * P.qscale;
            }
        }
    }

    auto tile_body = [&](int tile, Prefetch<KF>& fk, Prefetch<VF>& fv) {
        const int tb = t0 + tile * kTile;
        const int n = min(kTile, t1 - tb);  // <= 0 for an empty tile
        // The tile's RoPE table rows are requested first: loads complete in
        // order, so the wait for them then does not also wait for the next
        // tiles' prefetch issued below.
        // position of this lane's key token (padded tokens, and all of an
        // empty tile's, reuse the wave's last one: start + t1 - 1)
        const int pos = P.start_pos + tb + min(t, n - 1);
        float4 tr[8];
        if constexpr (TAB) {
            // piece i of group g for position p sits at float4
            // 512 (p / 16) + 64 i + 4 (p % 16) + g: one load instruction reads
            // the tile's 16 positions x 4 groups as at most two contiguous runs
            const float4* trow = P.rope + (long)(pos >> 4) * 512 + 4 * (pos & 15) + grp;
#pragma unroll
            for (int i = 0; i < 8; ++i) tr[i] = trow[64 * i];
        }

        stage_store<KF, false>(fk, st_k, P.k.pb, kslot, lane, P.k.nc);
        stage_store<VF, true>(fv, st_v, P.v.pb, vslot, lane, P.v.nc);
        wave_sync();
        // this tile's per-lane registers (metadata, ids, scales)
        const Prefetch<KF> ck = fk;
        const Prefetch<VF> cv = fv;
        // The loads of tile + kDepth go into the buffer just read.  Issued
        // unconditionally: past the wave's range the buffer loads return zero
        // without touching memory, and a branch here would make the waits that
        // follow count the loads as outstanding on one path only.
        prefetch<KF>(wk, P.k.pb, tb + kDepth * kTile - t0, lane, fk);
        prefetch<VF>(wv, P.v.pb, tb + kDepth * kTile - t0, lane, fv);
        // Wave priority rises through the tile (1: key decode, 2: scores and
        // value decode, 3: softmax and P x V, back to 0 for the next tile's
        // staging), so that of the two waves sharing a SIMD the one further
        // through its tile issues first: the pair drifts into complementary
        // phases, one finishing its matrix-core and softmax tail while the
        // other decodes (measured: 3% at B = 32 50%, 6-9% at 75%, 3-8% for
        // the quantised formats).
        __builtin_amdgcn_s_setprio(1);
        // ---- keys: centroid + residual, rotated ----
        float x[32];
        key_values<KF>(SK, ck, t, grp, P.k.width, gm, s_lut, s_cent, P.k.nc, P.one, x);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float cs4[4], sn4[4];
            if constexpr (TAB) {
                cs4[0] = tr[2 * u].x; cs4[1] = tr[2 * u].y; cs4[2] = tr[2 * u].z; cs4[3] = tr[2 * u].w;
                sn4[0] = tr[2 * u + 1].x; sn4[1] = tr[2 * u + 1].y; sn4[2] = tr[2 * u + 1].z; sn4[3] = tr[2 * u + 1].w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) rope_sincos_fast(__fmul_rn((float)pos, fr[4 * u + j]), sn4[j], cs4[j]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int mi = 4 * u + j;
                const float lo = x[mi], hi = x[16 + mi];
                x[mi] = lo * cs4[j] - hi * sn4[j];
                x[16 + mi] = hi * cs4[j] + lo * sn4[j];
            }
        }

        // ---- scores on the matrix cores, then the sum over the four groups ----
        __builtin_amdgcn_s_setprio(2);
        float sc[NH];
#pragma unroll
        for (int hs = 0; hs < NH; ++hs) {
            // four independent accumulation chains keep dependent MFMAs apart
            float4_t sa = (float4_t){0.0f, 0.0f, 0.0f, 0.0f}, sb = sa, sc4 = sa, sd = sa;
#pragma unroll
            for (int mi = 0; mi < 32; mi += 4) {
                sa = __builtin_amdgcn_mfma_f32_4x4x1f32(x[mi], qv[hs][mi], sa, 0, 0, 0);
                sb = __builtin_amdgcn_mfma_f32_4x4x1f32(x[mi + 1], qv[hs][mi + 1], sb, 0, 0, 0);
                sc4 = __builtin_amdgcn_mfma_f32_4x4x1f32(x[mi + 2], qv[hs][mi + 2], sc4, 0, 0, 0);
                sd = __builtin_amdgcn_mfma_f32_4x4x1f32(x[mi + 3], qv[hs][mi + 3], sd, 0, 0, 0);
            }
            sa += sb;
            sc4 += sd;
            const float u0 = swap32_sum(sa[0] + sc4[0], sa[2] + sc4[2]);
            const float u1 = swap32_sum(sa[1] + sc4[1], sa[3] + sc4[3]);
            sc[hs] = swap16_sum(u0, u1);
        }

        // ---- values: residuals as fp16 into the transpose tile ----
        if constexpr (VF == D_STRUCT16) {
            // 4:16: the row's 32 channels are zeroed and each of the lane's
            // eight kept values is written at the channel its nibble names
            // (tile g: channels 16g + nibble, tile 4 + g: 64 + 16g + nibble;
            // the four values of a tile are one 8-byte word, reference.py:36-47)
            uint16_t* vr = my_vt + t * kVPitch + 16 * grp;
            const uint4 z = make_uint4(0u, 0u, 0u, 0u);
            lds_st16(vr, z);
            lds_st16(vr + 8, z);
            lds_st16(vr + 64, z);
            lds_st16(vr + 72, z);
            const uint32_t sh = (uint32_t)(grp & 1) * 16u;
            const uint32_t c0 = ((grp < 2 ? cv.meta.x : cv.meta.y) >> sh) & 0xFFFFu;
            const uint32_t c1 = ((grp < 2 ? cv.meta.z : cv.meta.w) >> sh) & 0xFFFFu;
            const uint32_t* row = reinterpret_cast<const uint32_t*>(SV.row(t));
            const uint2 pa = *reinterpret_cast<const uint2*>(row + 2 * grp);
            const uint2 pb = *reinterpret_cast<const uint2*>(row + 8 + 2 * grp);
            const uint32_t va[4] = {pa.x, pa.x >> 16, pa.y, pa.y >> 16};
            const uint32_t vb[4] = {pb.x, pb.x >> 16, pb.y, pb.y >> 16};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                vr[(c0 >> (4 * j)) & 15u] = (uint16_t)va[j];
                vr[64 + ((c1 >> (4 * j)) & 15u)] = (uint16_t)vb[j];
            }
        } else {
            uint32_t hv[16];
            value_halves<VF>(SV, cv, t, grp, P.v.width, gm, s_lut, hv);
            uint4* vr = reinterpret_cast<uint4*>(my_vt + t * kVPitch + 16 * grp);
            lds_st16(vr + 0, make_uint4(hv[0], hv[1], hv[2], hv[3]));
            lds_st16(vr + 1, make_uint4(hv[4], hv[5], hv[6], hv[7]));
            lds_st16(vr + 8, make_uint4(hv[8], hv[9], hv[10], hv[11]));
            lds_st16(vr + 9, make_uint4(hv[12], hv[13], hv[14], hv[15]));
        }

        // ---- online softmax over the tile: one exponential per lane ----
        __builtin_amdgcn_s_setprio(3);
        bool grow = false;
        float mnew[NH];
#pragma unroll
        for (int hs = 0; hs < NH; ++hs) {
            const bool ok = stok < n && 4 * hs + hj < G;
            sc[hs] = ok ? sc[hs] : -INFINITY;
            mnew[hs] = fmaxf(m_run[hs], head_max(sc[hs]));
            grow |= mnew[hs] > m_run[hs];
        }
        if (ballot(grow) != 0) {
#pragma unroll
            for (int hs = 0; hs < NH; ++hs) {
                const float alpha = mnew[hs] > m_run[hs] ? exp2_fast(m_run[hs] - mnew[hs]) : 1.0f;
                lv[hs] *= alpha;
                m_run[hs] = mnew[hs];
                // lanes 4q + i hold head i: every lane takes the four factors of its quad
                const float al[4] = {dpp<0x00>(alpha), dpp<0x55>(alpha), dpp<0xAA>(alpha), dpp<0xFF>(alpha)};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[hs][0][i] *= al[i];
                    acc[hs][1][i] *= al[i];
                    accb[hs][i] *= al[i];
                }
            }
        }
#pragma unroll
        for (int hs = 0; hs < NH; ++hs) {
            const int g = 4 * hs + hj;
            const bool ok = stok < n && g < G;
            // the residual sums take the weight in fp16; the normaliser and the
            // cluster mass use the same rounded weight so the average stays consistent
            const uint16_t ph = f2h(ok ? exp2_fast(sc[hs] - m_run[hs]) : 0.0f);
            const float pq = h2f(ph);
            lv[hs] += pq;
            if (g < G) my_p[((((lane >> 2) & 3) * G + g) << 2) + (lane >> 4)] = ph;
        }
        wave_sync();

        // ---- P x V on the matrix cores, four tokens per instruction ----
        {
            const int blk_row = lane & 3;  // A row (query head within the set) of this lane
            // B through transpose reads: lane i of 16-lane row R points at
            // V[4s + i/4][16R + 4(i%4) ..+3] and receives V[4s + r][16R + i], r = 0..3
            const uint16_t* vb = my_vt + ((lane & 15) >> 2) * kVPitch + 16 * (lane >> 4) + 4 * (lane & 3);
#pragma unroll
            for (int s = 0; s < kTile / 4; ++s) {
                const half4_t b0 = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_short4_t*)(vb + 4 * s * kVPitch)));
                const half4_t b1 = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_short4_t*)(vb + 4 * s * kVPitch + 64)));
                half4_t oh = (half4_t){0, 0, 0, 0};
                if constexpr (VT::CENT) {
                    // bytes of x are zero where a token's id equals this lane; ids
                    // and lanes are below 64, so 0x40 - byte keeps bit 6 exactly
                    // there without borrows, and the perms widen those bytes to
                    // fp16 2.0 (0x4000): the mass accumulates twice its value
                    const uint32_t x = SV.ids4(s) ^ lane_bytes;
                    const uint32_t e = (0x40404040u - x) & 0x40404040u;
                    oh = __builtin_bit_cast(half4_t, make_uint2(__builtin_amdgcn_perm(0u, e, 0x010C000Cu),
                                                                __builtin_amdgcn_perm(0u, e, 0x030C020Cu)));
                }
#pragma unroll
                for (int hs = 0; hs < NH; ++hs) {
                    // A: lane 4b + i holds P[head 4 hs + i][tokens 4s + r]
                    const int g = 4 * hs + blk_row;
                    half4_t a = (half4_t){0, 0, 0, 0};
                    if (g < G) a = __builtin_bit_cast(half4_t, *reinterpret_cast<const uint2*>(my_p + ((s * G + g) << 2)));
                    acc[hs][0] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, b0, acc[hs][0], 0, 0, 0);
                    acc[hs][1] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, b1, acc[hs][1], 0, 0, 0);
                    if constexpr (VT::CENT) accb[hs] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, oh, accb[hs], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        wave_sync();  // stage, tile and weight reads done before the next tile overwrites them
    };
    // Whole groups of kDepth tiles, with no branch between the tile bodies: a
    // conditional body makes the load-wait counting conservative at the join,
    // so that a tile would wait for the loads the previous one issued.  A
    // tile past the wave's range (at most kDepth - 1 of them, at the end) is
    // empty: its loads return zero and every one of its tokens is masked.
    for (int tile = 0; tile < ntiles; tile += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) tile_body(tile + d, pk[d], pv[d]);
    }

    // ---- per-head totals, then merge the waves through LDS ----
    float lt[G], mt[G];
#pragma unroll
    for (int hs = 0; hs < NH; ++hs) {
        const float ls = head_sum(lv[hs]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * hs + i < G) {
                lt[4 * hs + i] = readlane(ls, i);
                mt[4 * hs + i] = readlane(m_run[hs], i);
            }
        }
    }
    float bt[G];
#pragma unroll
    for (int g = 0; g < G; ++g) bt[g] = VT::CENT ? 0.5f * accb[g >> 2][g & 3] : 0.0f;  // one-hot entries were 2
    __syncthreads();  // centroid table and stages no longer needed
    float* rec = reinterpret_cast<float*>(smem) + wave * G * kPartStride;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float* e = rec + g * kPartStride;
        e[lane] = acc[g >> 2][0][g & 3];
        e[64 + lane] = acc[g >> 2][1][g & 3];
        e[kDim + lane] = bt[g];
        if (lane == 0) {
            e[kDim + kMaxClusters] = mt[g];
            e[kDim + kMaxClusters + 1] = lt[g];
        }
    }
    __syncthreads();
    for (int g = wave; g < G; g += kWaves) {
        const float* base = reinterpret_cast<const float*>(smem);
        float mx = -INFINITY;
        for (int w = 0; w < kWaves; ++w) {
            const float* e = base + (w * G + g) * kPartStride;
            if (e[kDim + kMaxClusters + 1] > 0.0f) mx = fmaxf(mx, e[kDim + kMaxClusters]);
        }
        float a0 = 0.0f, a1 = 0.0f, ab = 0.0f, al = 0.0f;
        for (int w = 0; w < kWaves; ++w) {
            const float* e = base + (w * G + g) * kPartStride;
            const float lw = e[kDim + kMaxClusters + 1];
            const float f = lw > 0.0f ? exp2_fast(e[kDim + kMaxClusters] - mx) : 0.0f;
            a0 += e[lane] * f;
            a1 += e[lane + 64] * f;
            ab += e[kDim + lane] * f;
            al += lw * f;
        }
        const long slot = ((long)b * P.Hq + (long)h * G + g) * P.splits + split;
        P.pd[slot * kDim + lane] = a0;
        P.pd[slot * kDim + lane + 64] = a1;
        P.pb[slot * kMaxClusters + lane] = ab;
        if (lane == 0) {
            P.pm[slot] = mx;
            P.pl[slot] = al;
        }
    }
}

// One workgroup (256 threads) per (batch, query head) combines the split
// partials (log2 domain).  Every global load is issued before the split
// weights are known, so the kernel waits on memory once: the residual sums are
// read as float4 by 8 groups of 32 threads (split s goes to group s % 8), the
// cluster masses by 16 groups of 16 threads, the first eight (resp. four)
// splits of a thread into registers, and the Value centroids into LDS.  The
// groups are then reduced through LDS and the centroids folded in.
constexpr int kMergeThreads = 256;
constexpr int kMergeRegD = 8;  // residual-sum splits per thread held in registers
constexpr int kMergeRegB = 4;  // cluster-mass splits per thread held in registers
constexpr int kRecentThreads = 128;  // recent tokens per chunk of the joint softmax

// Dense recent tokens joined to a compressed result (Tr may be 0).
struct RecentArgs {
    const uint16_t* q_rope;  // fp16 [B*Hq, 128], rotated query
    const uint16_t* k;       // fp16 rotated keys, rows of rs tokens per (batch, KV head)
    const uint16_t* v;       // fp16 values, same layout
    int Tr, rs;
    float scaling;
};

// Block max / sum over the NT / 64 waves of an NT-thread workgroup (NT = 128
// or 256).
template <int NT>
__device__ __forceinline__ float block_max_nt(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = NT == 128 ? fmaxf(red[0], red[1]) : fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}
template <int NT>
__device__ __forceinline__ float block_sum_nt(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = NT == 128 ? red[0] + red[1] : (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return v;
}

// Chunk-0 operands of the recent join that a kernel may fetch before its
// other work: the rotated query value of thread tid < 128, and half a K row:
// thread tid holds token tid % 128, channels 64 (tid / 128) .. +63.
struct RecentPre {
    uint4 k[kDim / 16];
    float q;
    bool have;
};

__device__ __forceinline__ void recent_prefetch(const RecentArgs& r, const float* scores, long bq, long bh,
                                                RecentPre& pre) {
    const int tid = threadIdx.x;
    const int t = tid & (kRecentThreads - 1), half = tid / kRecentThreads;
    pre.have = scores == nullptr;
    pre.q = 0.0f;
    const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int i = 0; i < kDim / 16; ++i) pre.k[i] = zero;
    if (!pre.have || r.Tr <= 0) return;
    if (tid < kDim) pre.q = h2f(r.q_rope[bq * kDim + tid]);
    if (t < r.Tr) {
        const uint4* kr = reinterpret_cast<const uint4*>(r.k + (bh * r.rs + t) * kDim) + (kDim / 16) * half;
#pragma unroll
        for (int i = 0; i < kDim / 16; ++i) pre.k[i] = kr[i];
    }
}

// Joint softmax (natural-log units) of the compressed result of row bq --
// channel value oc of thread tid < 128, maximum cm, normaliser cl -- with its
// Tr recent tokens, by a 256-thread workgroup.  The tokens are taken in chunks
// of 128: token c0 + j is scored from given fp32 scores, or as a 128-dim dot
// product with the scaled rotated query whose two 64-channel halves threads j
// and j + 128 form; threads 0..127 own channel tid of the weighted value sum;
// chunks combine by online rescaling.  Every sum is written as an explicit
// FMA or rounded product, so the merge_recent kernel and the fused split
// merge, which both call this, agree bit for bit.  `pre` may hold the first
// chunk's query and K halves (recent_prefetch).
template <int NT>
__device__ float recent_join(float oc, float cm, float cl, const RecentArgs& r, const float* scores, long bq,
                             long bh, float* s_q, float* s_p, float* s_red, uint4* s_v, const RecentPre& pre) {
#pragma clang fp contract(off)
    static_assert(NT == 2 * kRecentThreads, "two threads per recent token");
    const int tid = threadIdx.x;
    const bool row = tid < kRecentThreads;
    const int half = tid / kRecentThreads;
    if (scores == nullptr && tid < kDim) s_q[tid] = (pre.have ? pre.q : h2f(r.q_rope[bq * kDim + tid])) * r.scaling;
    __syncthreads();
    float m = -INFINITY, l = 0.0f, acc = 0.0f;  // acc: channel tid
    constexpr int kVPer = kRecentThreads * (kDim / 8) / NT;  // 16-byte pieces of a chunk's V rows per thread
    for (int c0 = 0; c0 < r.Tr; c0 += kRecentThreads) {
        const int t = c0 + tid;
        const bool live = row && t < r.Tr;
        // the chunk's V rows into LDS with 16-byte loads by every thread (one
        // round trip), read from LDS by the weighted sum below
        {
            const int pieces = min(kRecentThreads, r.Tr - c0) * (kDim / 8);
            const uint4* vsrc = reinterpret_cast<const uint4*>(r.v + (bh * r.rs + c0) * kDim);
            uint4 vrow[kVPer];
#pragma unroll
            for (int i = 0; i < kVPer; ++i) {
                const int e = tid + NT * i;
                vrow[i] = e < pieces ? vsrc[e] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int i = 0; i < kVPer; ++i) {
                const int e = tid + NT * i;
                if (e < pieces) s_v[e] = vrow[i];
            }
        }
        float s = -INFINITY;
        if (scores != nullptr) {
            if (live) s = scores[bq * r.Tr + t];
        } else {
            // half a dot product per thread: token c0 + tid % 128, channels 64 half .. +63
            const int th = c0 + (tid & (kRecentThreads - 1));
            uint4 kw[kDim / 16];
            if (pre.have && c0 == 0) {
#pragma unroll
                for (int i = 0; i < kDim / 16; ++i) kw[i] = pre.k[i];
            } else {
                const uint4* kr = reinterpret_cast<const uint4*>(r.k + (bh * r.rs + th) * kDim) + (kDim / 16) * half;
#pragma unroll
                for (int i = 0; i < kDim / 16; ++i) kw[i] = th < r.Tr ? kr[i] : make_uint4(0u, 0u, 0u, 0u);
            }
            const float* q = s_q + (kDim / 2) * half;
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < kDim / 16; ++i) {
                const uint32_t ws[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    d = fmaf(q[8 * i + 2 * j], h2f((uint16_t)(ws[j] & 0xFFFFu)), d);
                    d = fmaf(q[8 * i + 2 * j + 1], h2f((uint16_t)(ws[j] >> 16)), d);
                }
            }
            s_p[tid] = d;
            __syncthreads();
            if (live) s = s_p[tid] + s_p[tid + kRecentThreads];
        }
        const float mn = fmaxf(m, block_max_nt<NT>(s, s_red));  // its barriers also publish s_v (and end the s_p reads)
        const float p = live ? expf(s - mn) : 0.0f;
        if (row) s_p[tid] = p;
        const float ps = block_sum_nt<NT>(p, s_red);  // its barriers also publish s_p
        const float alpha = expf(m - mn);  // 0 for the first chunk (m = -inf, mn finite)
        l = fmaf(l, alpha, ps);
        if (tid < kDim) {
            const int n = min(kRecentThreads, r.Tr - c0);
            const uint16_t* vr = reinterpret_cast<const uint16_t*>(s_v) + tid;
            float a = 0.0f;
            for (int j = 0; j < n; ++j) a = fmaf(s_p[j], h2f(vr[j * kDim]), a);
            acc = fmaf(acc, alpha, a);
        }
        m = mn;
        __syncthreads();  // s_p and s_v reads done before the next chunk writes them
    }
    const float jm = fmaxf(cm, m);
    const float wc = cl > 0.0f ? __fmul_rn(cl, expf(cm - jm)) : 0.0f;
    const float wr = r.Tr > 0 ? expf(m - jm) : 0.0f;
    const float denom = fmaf(l, wr, wc);
    const float inv = denom > 0.0f ? 1.0f / denom : 0.0f;
    return __fmul_rn(fmaf(oc, wc, __fmul_rn(acc, wr)), inv);
}

// LDS of the split merge: the Value centroids, split weights and the two
// group-partial tables are dead once the compressed result is formed, so the
// recent join's staged V rows (128 tokens x 256 B) reuse the same bytes.
constexpr int kMergeVcBytes = kMaxClusters * kDim * 2;
constexpr int kMergeWOff = kMergeVcBytes;
constexpr int kMergeDOff = kMergeWOff + kMaxSplits * 4;
constexpr int kMergeBOff = kMergeDOff + 8 * kDim * 4;
constexpr int kMergeEnd = kMergeBOff + 16 * kMaxClusters * 4;
constexpr int kRecentVBytes = kRecentThreads * kDim * 2;
constexpr int kMergePool = kMergeEnd > kRecentVBytes ? kMergeEnd : kRecentVBytes;

// RECENT: the compressed result, rounded to fp16 as the unfused path stores
// it, is joined with the recent tokens of `rc` before it is written; the
// join's first query and K rows are fetched before the split merge starts.
template <bool RECENT>
__global__ void __launch_bounds__(kMergeThreads) decode_merge_kernel(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ pdelta,
    const float* __restrict__ pbeta, const uint16_t* __restrict__ vcent, int vnc, int vcs, int Hq, int H,
    int splits, uint16_t* __restrict__ out, float* __restrict__ om, float* __restrict__ ol, RecentArgs rc) {
#pragma clang fp contract(off)  // every product and sum as written (FMAs are explicit)
    __shared__ __align__(16) uint8_t s_pool[RECENT ? kMergePool : kMergeEnd];
    uint4* s_vc = reinterpret_cast<uint4*>(s_pool);  // fp16 Value centroids [c][128]
    float* s_w = reinterpret_cast<float*>(s_pool + kMergeWOff);
    float4 (*s_d)[kDim / 4] = reinterpret_cast<float4 (*)[kDim / 4]>(s_pool + kMergeDOff);
    float4 (*s_b)[kMaxClusters / 4] = reinterpret_cast<float4 (*)[kMaxClusters / 4]>(s_pool + kMergeBOff);
    __shared__ float s_red[kMergeThreads / kWave];
    __shared__ float s_beta[kMaxClusters];
    __shared__ float s_q[RECENT ? kDim : 1];
    __shared__ float s_p[RECENT ? 2 * kRecentThreads : 1];
    const long bq = blockIdx.x;  // b * Hq + hq
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = Hq / H;
    const long bh = (bq / Hq) * H + (bq % Hq) / G;
    const float* m_row = pm + bq * splits;
    const float* l_row = pl + bq * splits;
    const int dg = tid >> 5, dq = tid & 31;  // residual sums: split group, channel quad
    const int bg = tid >> 4, bq4 = tid & 15;  // cluster masses: split group, cluster quad
    const float4* dbase = reinterpret_cast<const float4*>(pdelta + (bq * splits) * kDim) + dq;
    const float4* bbase = reinterpret_cast<const float4*>(pbeta + (bq * splits) * kMaxClusters) + bq4;
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    RecentPre pre;
    if constexpr (RECENT) recent_prefetch(rc, nullptr, bq, bh, pre);
    // 0) loads that do not depend on the split weights
    const bool one_pass = splits <= kMergeThreads;  // one split per thread for the maximum and weights
    float m0 = -INFINITY, l0 = 0.0f;
    if (one_pass && tid < splits) {
        m0 = m_row[tid];
        l0 = l_row[tid];
    }
    float4 dv[kMergeRegD], bv[kMergeRegB];
#pragma unroll
    for (int i = 0; i < kMergeRegD; ++i) {
        const int sp = dg + 8 * i;
        dv[i] = sp < splits ? dbase[(long)sp * (kDim / 4)] : zero4;
    }
#pragma unroll
    for (int i = 0; i < kMergeRegB; ++i) {
        const int sp = bg + 16 * i;
        bv[i] = sp < splits ? bbase[(long)sp * (kMaxClusters / 4)] : zero4;
    }
    if (vcent != nullptr) {
        const uint4* vc = reinterpret_cast<const uint4*>(vcent + bh * vcs * kDim);
        for (int i = tid; i < vnc * (kDim / 8); i += kMergeThreads) s_vc[i] = vc[i];
    }

    // 1) common maximum over the non-empty splits
    float mx = one_pass ? (l0 > 0.0f ? m0 : -INFINITY) : -INFINITY;
    if (!one_pass)
        for (int sp = tid; sp < splits; sp += kMergeThreads)
            if (l_row[sp] > 0.0f) mx = fmaxf(mx, m_row[sp]);
    mx = wave_max(mx);
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();

    // 2) split weights and the normaliser
    float lsum = 0.0f;
    if (one_pass) {
        if (tid < splits) {
            const float w = l0 > 0.0f ? exp2_fast(m0 - mx) : 0.0f;
            s_w[tid] = w;
            lsum = __fmul_rn(l0, w);
        }
    } else {
        for (int sp = tid; sp < splits; sp += kMergeThreads) {
            const float lw = l_row[sp];
            const float w = lw > 0.0f ? exp2_fast(m_row[sp] - mx) : 0.0f;
            s_w[sp] = w;
            lsum = fmaf(lw, w, lsum);
        }
    }
    lsum = wave_sum(lsum);
    if (lane == 0) s_red[wave] = lsum;
    __syncthreads();
    lsum = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);

    // 3) weighted residual sums and cluster masses per split group
    {
        float4 acc = zero4;
#pragma unroll
        for (int i = 0; i < kMergeRegD; ++i) {
            const int sp = dg + 8 * i;
            const float w = sp < splits ? s_w[sp] : 0.0f;
            acc.x = fmaf(w, dv[i].x, acc.x);
            acc.y = fmaf(w, dv[i].y, acc.y);
            acc.z = fmaf(w, dv[i].z, acc.z);
            acc.w = fmaf(w, dv[i].w, acc.w);
        }
        for (int sp = dg + 8 * kMergeRegD; sp < splits; sp += 8) {
            const float w = s_w[sp];
            const float4 d = dbase[(long)sp * (kDim / 4)];
            acc.x = fmaf(w, d.x, acc.x);
            acc.y = fmaf(w, d.y, acc.y);
            acc.z = fmaf(w, d.z, acc.z);
            acc.w = fmaf(w, d.w, acc.w);
        }
        s_d[dg][dq] = acc;
        float4 accb = zero4;
#pragma unroll
        for (int i = 0; i < kMergeRegB; ++i) {
            const int sp = bg + 16 * i;
            const float w = sp < splits ? s_w[sp] : 0.0f;
            accb.x = fmaf(w, bv[i].x, accb.x);
            accb.y = fmaf(w, bv[i].y, accb.y);
            accb.z = fmaf(w, bv[i].z, accb.z);
            accb.w = fmaf(w, bv[i].w, accb.w);
        }
        for (int sp = bg + 16 * kMergeRegB; sp < splits; sp += 16) {
            const float w = s_w[sp];
            const float4 d = bbase[(long)sp * (kMaxClusters / 4)];
            accb.x = fmaf(w, d.x, accb.x);
            accb.y = fmaf(w, d.y, accb.y);
            accb.z = fmaf(w, d.z, accb.z);
            accb.w = fmaf(w, d.w, accb.w);
        }
        s_b[bg][bq4] = accb;
    }
    __syncthreads();
    // 4) cluster masses summed over the 16 groups (threads 128..191)
    if (tid >= kDim && tid < kDim + kMaxClusters) {
        const int c = tid - kDim;
        const float* sb = reinterpret_cast<const float*>(s_b);
        float beta = 0.0f;
#pragma unroll
        for (int g2 = 0; g2 < 16; ++g2) beta += sb[g2 * kMaxClusters + c];
        s_beta[c] = beta;
    }
    __syncthreads();
    // 5) fold sum_c beta_c c_v[c] by all threads: channel pair tid % 64 over
    // the centroids c = tid / 64 (mod 4), the four quarters then summed per
    // channel through the (now unused) cluster-mass table
    float* s_f = reinterpret_cast<float*>(s_b);  // [quarter][channel]
    if (vcent != nullptr) {
        const int cp = tid & 63, qq = tid >> 6;
        const uint32_t* vc = reinterpret_cast<const uint32_t*>(s_vc) + cp;
        float f0 = 0.0f, f1 = 0.0f;
        for (int c = qq; c < vnc; c += 4) {
            const uint32_t w = vc[c * (kDim / 2)];
            f0 = fmaf(s_beta[c], h2f((uint16_t)(w & 0xFFFFu)), f0);
            f1 = fmaf(s_beta[c], h2f((uint16_t)(w >> 16)), f1);
        }
        s_f[qq * kDim + 2 * cp] = f0;
        s_f[qq * kDim + 2 * cp + 1] = f1;
        __syncthreads();
    }
    // normalise (threads 0..127: one channel each)
    uint16_t oc = 0;
    if (tid < kDim) {
        const float* sd = reinterpret_cast<const float*>(s_d);
        float acc = 0.0f;
#pragma unroll
        for (int g2 = 0; g2 < 8; ++g2) acc += sd[g2 * kDim + tid];
        if (vcent != nullptr) acc += (s_f[tid] + s_f[kDim + tid]) + (s_f[2 * kDim + tid] + s_f[3 * kDim + tid]);
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        oc = f2h(acc * inv);
        if constexpr (!RECENT) {
            out[bq * kDim + tid] = oc;
            if (tid == 0) {
                if (om) om[bq] = __fmul_rn(mx, kLn2);  // natural-log units, as the reference returns m
                if (ol) ol[bq] = lsum;
            }
        }
    }
    if constexpr (RECENT) {
        // the same rounded product as the m the unfused merge stores (no contraction into cm - jm)
        __syncthreads();  // the centroid fold's LDS reads are done before the join overwrites the pool
        const float r = recent_join<kMergeThreads>(h2f(oc), __fmul_rn(mx, kLn2), lsum, rc, nullptr, bq, bh, s_q, s_p,
                                                   s_red, reinterpret_cast<uint4*>(s_pool), pre);
        if (tid < kDim) out[bq * kDim + tid] = f2h(r);
    }
}

// Joint softmax of a normalised compressed result (m, l) with Tr recent tokens
// whose scaled scores are given (scores != null) or computed from q_rope/k
// (recent_join).  Recent K/V rows of (batch, head) block bh start at token
// bh * rs.  One workgroup per (batch, query head), of the split merge's 256
// threads: both kernels then run the same code for the join (the upper 128
// threads take part in its reductions only).
__global__ void __launch_bounds__(kMergeThreads) merge_recent_kernel(
    const uint16_t* __restrict__ comp_out, const float* __restrict__ comp_m, const float* __restrict__ comp_l,
    const float* __restrict__ scores, const uint16_t* __restrict__ q_rope, const uint16_t* __restrict__ k_recent,
    const uint16_t* __restrict__ v_recent, int Hq, int H, int Tr, int rs, float scaling,
    uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
    __shared__ float s_q[kDim];
    __shared__ float s_p[2 * kRecentThreads];
    __shared__ float s_red[kMergeThreads / kWave];
    __shared__ uint4 s_rv[kRecentThreads * kDim / 8];  // a chunk of recent V rows
    const long bq = blockIdx.x;
    const int tid = threadIdx.x;
    const int G = Hq / H;
    const long b = bq / Hq, hq = bq % Hq;
    const long bh = b * H + hq / G;
    const RecentArgs r{q_rope, k_recent, v_recent, Tr, rs, scaling};
    const float oc = tid < kDim ? h2f(comp_out[bq * kDim + tid]) : 0.0f;
    RecentPre pre;
    recent_prefetch(r, scores, bq, bh, pre);
    const float res = recent_join<kMergeThreads>(oc, comp_m[bq], comp_l[bq], r, scores, bq, bh, s_q, s_p, s_red, s_rv,
                                                 pre);
    if (tid < kDim) out[bq * kDim + tid] = f2h(res);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// The automatic split count fills every CU with as many workgroups as the
// kernel instance keeps resident per CU (two for most formats at their
// register use, three for the quantised ones); each wave keeps at least two
// 16-token tiles so that its next tile's loads overlap the current tile's
// arithmetic.
constexpr int kCUs = 256;            // compute units of an MI355X
constexpr int kMaxGroupsPerCU = 4;   // cap of the automatic split target (and of the workspace bound)

int auto_splits(int B, int H, int T, int per_cu) {
    const long heads = (long)B * H;
    long s = ((long)per_cu * kCUs + heads - 1) / heads;
    const long cap = T / (kWaves * 2 * kTile) > 0 ? T / (kWaves * 2 * kTile) : 1;
    if (s > cap) s = cap;
    if (s > kMaxSplits) s = kMaxSplits;
    return (int)(s < 1 ? 1 : s);
}

// per_cu: workgroups of the kernel instance resident per CU (automatic splits
// fill every CU that many times over).
int resolve_splits(int B, int H, int T, int splits, int per_cu) {
    if (splits > 0) {
        int s = splits < T ? splits : T;
        return s < kMaxSplits ? s : kMaxSplits;
    }
    return auto_splits(B, H, T, per_cu);
}

int64_t workspace_for(int B, int Hq, int S) {
    return (int64_t)B * Hq * S * (2 + kDim + kMaxClusters) * (int64_t)sizeof(float);
}

int dfmt_of(const reskv_ctensor* c) {
    switch (c->format) {
    case RESKV_FMT_BITMAP: return c->width > 64 ? D_BITMAP_W : D_BITMAP;
    case RESKV_FMT_TILED: return c->width > 64 ? D_TILED_W : D_TILED;
    case RESKV_FMT_STRUCT16: return D_STRUCT16;
    case RESKV_FMT_STRUCT_INT4: return D_SINT4;
    default: return c->bits == 4 ? D_Q4 : D_Q2;
    }
}

int payload_bytes(int f, int width) {
    switch (f) {
    case D_BITMAP: case D_TILED: case D_STRUCT16: case D_BITMAP_W: case D_TILED_W: return 2 * width;
    case D_SINT4: return 16;
    case D_Q4: return 64;
    case D_Q2: return 32;
    default: return 2 * kDim;
    }
}

int check_ct(const reskv_ctensor* c, const char* name) {
    RESKV_REQUIRE(c != nullptr, "%s: null tensor descriptor", name);
    RESKV_REQUIRE(c->centroids && c->ids && c->payload, "%s: null pointer", name);
    RESKV_REQUIRE(c->nc >= 1 && c->nc <= kMaxClusters, "%s: centroid count must be in [1, 64]", name);
    switch (c->format) {
    case RESKV_FMT_BITMAP:
        RESKV_REQUIRE(c->meta && c->width >= 8 && c->width <= kDim && c->width % 8 == 0,
                      "%s: bitmap payload width must be a multiple of 8 in [8, 128]", name);
        break;
    case RESKV_FMT_TILED:
        RESKV_REQUIRE(c->meta && c->width % 8 == 0 && c->width >= 8 && c->width < kDim, "%s: bad tiled tensor", name);
        break;
    case RESKV_FMT_STRUCT16:
        RESKV_REQUIRE(c->meta && c->width == 32, "%s: bad 4:16 tensor", name);
        break;
    case RESKV_FMT_STRUCT_INT4:
        RESKV_REQUIRE(c->meta && c->scale && c->width == 4, "%s: bad structured INT4 tensor", name);
        break;
    case RESKV_FMT_QUANT:
        RESKV_REQUIRE(c->scale && (c->bits == 2 || c->bits == 4) && c->width == 4 * c->bits,
                      "%s: bad quantised tensor", name);
        break;
    default:
        RESKV_REQUIRE(false, "%s: unknown residual format %d", name, c->format);
    }
    const uintptr_t align = (uintptr_t)c->payload | (uintptr_t)(c->meta ? c->meta : c->payload) |
                            (uintptr_t)(c->centroids ? c->centroids : c->payload);
    RESKV_REQUIRE((align & 15u) == 0, "%s: payload, metadata and centroids must be 16-byte aligned", name);
    return 0;
}

DTensor to_dt(const reskv_ctensor* c, int f, int T) {
    return DTensor{(const uint16_t*)c->centroids, c->ids, (const uint8_t*)c->payload, (const uint8_t*)c->meta,
                   (const uint16_t*)c->scale, c->nc, c->width, payload_bytes(f, c->width),
                   c->t_stride > 0 ? c->t_stride : T, c->c_stride > 0 ? c->c_stride : c->nc};
}

template <int F>
int stage_of(int pb) { return stage_bytes<F>(pb); }

int stage_bytes_rt(int f, int pb) {
    switch (f) {
    case D_BITMAP: return stage_of<D_BITMAP>(pb);
    case D_TILED: return stage_of<D_TILED>(pb);
    case D_STRUCT16: return stage_of<D_STRUCT16>(pb);
    case D_SINT4: return stage_of<D_SINT4>(pb);
    case D_Q4: return stage_of<D_Q4>(pb);
    case D_Q2: return stage_of<D_Q2>(pb);
    case D_BITMAP_W: return stage_of<D_BITMAP_W>(pb);
    case D_TILED_W: return stage_of<D_TILED_W>(pb);
    default: return stage_of<D_DENSE>(pb);
    }
}

// The partial kernel instance for (K format, V format, GQA ratio, RoPE table).
template <int G, int KF, int VF>
const void* kernel_g(bool tab) {
    return tab ? reinterpret_cast<const void*>(&decode_partial_kernel<G, KF, VF, true>)
               : reinterpret_cast<const void*>(&decode_partial_kernel<G, KF, VF, false>);
}

template <int KF, int VF>
const void* kernel_fmt(int G, bool tab) {
    switch (G) {
    case 1: return kernel_g<1, KF, VF>(tab);
    case 2: return kernel_g<2, KF, VF>(tab);
    case 4: return kernel_g<4, KF, VF>(tab);
    default: return kernel_g<8, KF, VF>(tab);
    }
}

const void* partial_kernel(int kf, int vf, int G, bool tab) {
    if (kf == vf) {
        switch (kf) {
        case D_BITMAP: return kernel_fmt<D_BITMAP, D_BITMAP>(G, tab);
        case D_TILED: return kernel_fmt<D_TILED, D_TILED>(G, tab);
        case D_STRUCT16: return kernel_fmt<D_STRUCT16, D_STRUCT16>(G, tab);
        case D_SINT4: return kernel_fmt<D_SINT4, D_SINT4>(G, tab);
        case D_Q4: return kernel_fmt<D_Q4, D_Q4>(G, tab);
        case D_Q2: return kernel_fmt<D_Q2, D_Q2>(G, tab);
        case D_BITMAP_W: return kernel_fmt<D_BITMAP_W, D_BITMAP_W>(G, tab);
        case D_TILED_W: return kernel_fmt<D_TILED_W, D_TILED_W>(G, tab);
        default: return kernel_fmt<D_DENSE, D_DENSE>(G, tab);
        }
    }
    if (kf == D_Q4 && vf == D_Q2) return kernel_fmt<D_Q4, D_Q2>(G, tab);
    if (kf == D_Q2 && vf == D_Q4) return kernel_fmt<D_Q2, D_Q4>(G, tab);
    return nullptr;
}

// LDS layout of one partial workgroup: centroid table (or the cross-wave merge
// records, whichever is larger), permute tables, per-wave weight and V tiles,
// per-wave K and V stages.
struct PartialLds {
    int lut_off, p_off, stage_off, stage_k, stage_v;
    size_t bytes;
};
PartialLds partial_lds(int kf, const DTensor& k, int vf, const DTensor& v, int G) {
    PartialLds L;
    L.stage_k = stage_bytes_rt(kf, k.pb);
    L.stage_v = stage_bytes_rt(vf, v.pb);
    const int merge_bytes = kWaves * G * kPartStride * 4;
    const int cent_bytes = kf != D_DENSE ? k.nc * kCPitch * 2 : 0;
    L.lut_off = cent_bytes > merge_bytes ? cent_bytes : merge_bytes;
    L.p_off = L.lut_off + (kLutWords + kStructLutWords + kQTrigWords) * 4;
    L.stage_off = L.p_off + kWaves * (kTile * G + kTile * kVPitch) * 2;
    L.bytes = (size_t)L.stage_off + (size_t)kWaves * (L.stage_k + L.stage_v);
    return L;
}

// Workgroups of a partial kernel instance to fill each CU with: the number
// resident at once (its registers and LDS; the instance's LDS limit is set
// first), capped at kMaxGroupsPerCU, at two for the formats that decode runs
// from LDS windows (a third bitmap workgroup per CU measured 2% slower: it adds
// LDS traffic where the quantised formats, which gain 10-13% from it, have
// none), and at two for 4:16 below 33 (batch, head) rows (its one-deep
// prefetch leaves short tiles waiting: 4.6% slower at B = 4 with three).
// Returns 0 on a runtime error.
int groups_per_cu(const void* fn, size_t shm, int kf, long heads) {
    if (shm > 65536 &&
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return 0;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kThreads, shm) != hipSuccess || n < 1) return 0;
    const bool windows = kf == D_BITMAP || kf == D_BITMAP_W || kf == D_TILED || kf == D_TILED_W;
    const int cap = windows || (kf == D_STRUCT16 && heads <= 32) ? 2 : kMaxGroupsPerCU;
    return n < cap ? n : cap;
}

// The split count a decode of these tensors makes (splits <= 0: automatic).
int splits_for(int kf, const DTensor& k, int vf, const DTensor& v, int G, bool tab, int B, int H, int T,
               int splits, int* out) {
    const void* fn = partial_kernel(kf, vf, G, tab);
    RESKV_REQUIRE(fn != nullptr, "K and V residual formats must match (INT4/INT2 may mix)");
    int per_cu = kMaxGroupsPerCU;
    if (splits <= 0) {
        per_cu = groups_per_cu(fn, partial_lds(kf, k, vf, v, G).bytes, kf, (long)B * H);
        RESKV_REQUIRE(per_cu > 0, "decode occupancy query failed: %s", hipGetErrorString(hipGetLastError()));
    }
    *out = resolve_splits(B, H, T, splits, per_cu);
    return 0;
}

int run_decode(const void* q, int kf, const DTensor& k, int vf, const DTensor& v, const float* inv_freq,
               const float* rope, int B, int Hq, int H, int T, int start_pos, int pos_q, float scaling, int splits,
               void* out, float* m, float* l, void* ws, int64_t ws_bytes, void* stream,
               const RecentArgs* recent = nullptr) {
    RESKV_REQUIRE(q && inv_freq && out, "null pointer argument");
    RESKV_REQUIRE(B > 0 && H > 0 && T > 0, "batch, head and token counts must be positive");
    RESKV_REQUIRE(Hq % H == 0, "query heads must be a multiple of KV heads");
    const int G = Hq / H;
    RESKV_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "supported GQA ratios are 1, 2, 4 and 8");
    RESKV_REQUIRE((((uintptr_t)inv_freq | (uintptr_t)q) & 15u) == 0, "q and inv_freq must be 16-byte aligned");
    const void* fn = partial_kernel(kf, vf, G, rope != nullptr);
    RESKV_REQUIRE(fn != nullptr, "K and V residual formats must match (INT4/INT2 may mix)");
    // the smallest split count these sizes can take, checked before any runtime call
    RESKV_REQUIRE(ws != nullptr && ws_bytes >= workspace_for(B, Hq, resolve_splits(B, H, T, splits, 1)),
                  "decode workspace too small");
    const PartialLds L = partial_lds(kf, k, vf, v, G);
    RESKV_REQUIRE(L.bytes <= 160 * 1024, "decode LDS requirement %zu exceeds 160 KiB", L.bytes);
    const int per_cu = groups_per_cu(fn, L.bytes, kf, (long)B * H);  // also sets the instance's LDS limit
    RESKV_REQUIRE(per_cu > 0, "decode occupancy query failed: %s", hipGetErrorString(hipGetLastError()));
    const int S = resolve_splits(B, H, T, splits, per_cu);
    RESKV_REQUIRE(ws != nullptr && ws_bytes >= workspace_for(B, Hq, S), "decode workspace too small");
    DParams p{};
    p.q = (const uint16_t*)q;
    p.k = k;
    p.v = v;
    p.inv_freq = inv_freq;
    p.rope = (const float4*)rope;
    RESKV_REQUIRE(((uintptr_t)rope & 15u) == 0, "RoPE table must be 16-byte aligned");
    p.Hq = Hq;
    p.H = H;
    p.T = T;
    p.start_pos = start_pos;
    p.pos_q = pos_q;
    p.splits = S;
    p.qscale = scaling * kLog2e;
    p.one = 1.0f;
    p.stage_k = L.stage_k;
    p.stage_v = L.stage_v;
    p.lut_off = L.lut_off;
    p.p_off = L.p_off;
    p.stage_off = L.stage_off;
    const bool cent = kf != D_DENSE;
    p.pm = (float*)ws;
    p.pl = p.pm + (long)B * Hq * S;
    p.pd = p.pl + (long)B * Hq * S;
    p.pb = p.pd + (long)B * Hq * S * kDim;
    hipStream_t st = (hipStream_t)stream;
    void* args[] = {&p};
    if (hipLaunchKernel(fn, dim3((unsigned)((long)S * H * B)), dim3(kThreads), args, L.bytes, st) != hipSuccess)
        return reskv_host::check_launch("decode_partial_kernel");
    if (reskv_host::check_launch("decode_partial_kernel")) return 1;
    if (recent != nullptr) {
        hipLaunchKernelGGL(decode_merge_kernel<true>, dim3(B * Hq), dim3(kMergeThreads), 0, st, p.pm, p.pl, p.pd,
                           p.pb, cent ? v.cent : nullptr, v.nc, v.cs, Hq, H, S, (uint16_t*)out, nullptr, nullptr,
                           *recent);
    } else {
        hipLaunchKernelGGL(decode_merge_kernel<false>, dim3(B * Hq), dim3(kMergeThreads), 0, st, p.pm, p.pl, p.pd,
                           p.pb, cent ? v.cent : nullptr, v.nc, v.cs, Hq, H, S, (uint16_t*)out, m, l,
                           RecentArgs{});
    }
    return reskv_host::check_launch("decode_merge_kernel");
}

}  // namespace

extern "C" int64_t reskv_decode_workspace_bytes(int B, int Hq, int H, int T, int splits) {
    if (B <= 0 || Hq <= 0 || H <= 0 || T <= 0) return 0;
    return workspace_for(B, Hq, resolve_splits(B, H, T, splits, kMaxGroupsPerCU));
}

extern "C" int reskv_decode_splits(const reskv_ctensor* k, const reskv_ctensor* v, int rope_table, int B, int Hq,
                                   int H, int T, int splits) {
    if (check_ct(k, "K") || check_ct(v, "V")) return -1;
    if (B <= 0 || H <= 0 || T <= 0 || Hq <= 0 || Hq % H != 0) {
        reskv_host::set_error("batch, head and token counts must be positive, query heads a multiple of KV heads");
        return -1;
    }
    const int kf = dfmt_of(k), vf = dfmt_of(v);
    int s = 0;
    if (splits_for(kf, to_dt(k, kf, T), vf, to_dt(v, vf, T), Hq / H, rope_table != 0, B, H, T, splits, &s)) return -1;
    return s;
}

extern "C" int reskv_decode_rope(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                                 const float* inv_freq, const float* rope_table, int B, int Hq, int H, int T,
                                 int start_pos, int pos_q, float scaling, int splits, void* out, float* m,
                                 float* l, void* workspace, int64_t workspace_bytes, void* stream) {
    if (check_ct(k, "K") || check_ct(v, "V")) return 1;
    RESKV_REQUIRE((k->t_stride == 0 || k->t_stride >= T) && (v->t_stride == 0 || v->t_stride >= T),
                  "token row stride must be 0 or at least T");
    RESKV_REQUIRE((k->c_stride == 0 || k->c_stride >= k->nc) && (v->c_stride == 0 || v->c_stride >= v->nc),
                  "centroid row stride must be 0 or at least nc");
    const int kf = dfmt_of(k), vf = dfmt_of(v);
    return run_decode(q, kf, to_dt(k, kf, T), vf, to_dt(v, vf, T), inv_freq, rope_table, B, Hq, H, T, start_pos,
                      pos_q, scaling, splits, out, m, l, workspace, workspace_bytes, stream);
}

extern "C" int reskv_decode_recent(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                                   const float* inv_freq, const float* rope_table, int B, int Hq, int H, int T,
                                   int start_pos, int pos_q, float scaling, int splits, const void* q_rope,
                                   const void* k_recent, const void* v_recent, int Tr, int r_stride, void* out,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
    if (check_ct(k, "K") || check_ct(v, "V")) return 1;
    RESKV_REQUIRE((k->t_stride == 0 || k->t_stride >= T) && (v->t_stride == 0 || v->t_stride >= T),
                  "token row stride must be 0 or at least T");
    RESKV_REQUIRE((k->c_stride == 0 || k->c_stride >= k->nc) && (v->c_stride == 0 || v->c_stride >= v->nc),
                  "centroid row stride must be 0 or at least nc");
    RESKV_REQUIRE(Tr >= 0, "bad recent-merge sizes");
    const int rs = r_stride > 0 ? r_stride : Tr;
    RESKV_REQUIRE(rs >= Tr, "recent row stride shorter than the window");
    RESKV_REQUIRE(Tr == 0 || (q_rope && k_recent && v_recent), "null recent tensors");
    RESKV_REQUIRE(Tr == 0 || ((((uintptr_t)k_recent | (uintptr_t)v_recent) & 15u) == 0),
                  "recent K and V must be 16-byte aligned");
    const RecentArgs rc{(const uint16_t*)q_rope, (const uint16_t*)k_recent, (const uint16_t*)v_recent, Tr, rs, scaling};
    const int kf = dfmt_of(k), vf = dfmt_of(v);
    return run_decode(q, kf, to_dt(k, kf, T), vf, to_dt(v, vf, T), inv_freq, rope_table, B, Hq, H, T, start_pos,
                      pos_q, scaling, splits, out, nullptr, nullptr, workspace, workspace_bytes, stream, &rc);
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the split-K partial records live in one file-scope
// device array instead of a caller workspace.  Each GPU the library runs on
// holds its own copy until the process ends.  The partial kernel writes every
// record the merge kernel reads, so nothing in it has to start at zero; the
// array keeps the last call's records.  Calls that overlap on one GPU (two
// host threads, or two streams without ordering) race on it.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchBytes = RESKV_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};

// Device address of `scratch` on the current device (its name is only a host
// stand-in).  Looked up once per device; returns null with the error message
// set when the device or the lookup fails.
void* scratch_on_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        reskv_host::set_error("no current HIP device (or device index >= %d)", kMaxDevices);
        return nullptr;
    }
    std::call_once(g_scratch_once[dev], [dev]() {
        void* ptr = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? ptr : nullptr;
    });
    if (g_scratch_ptr[dev] == nullptr) {
        reskv_host::set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                              hipGetErrorString(g_scratch_err[dev]));
        return nullptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int reskv_decode_recent_noalloc(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                                           const float* inv_freq, const float* rope_table, int B, int Hq, int H,
                                           int T, int start_pos, int pos_q, float scaling, int splits,
                                           const void* q_rope, const void* k_recent, const void* v_recent, int Tr,
                                           int r_stride, void* out, void* stream) {
    RESKV_REQUIRE(B > 0 && Hq > 0 && H > 0 && T > 0, "batch, head and token counts must be positive");
    const int64_t need = reskv_decode_workspace_bytes(B, Hq, H, T, splits);
    RESKV_REQUIRE(need <= kNoAllocScratchBytes,
                  "reskv_decode_recent_noalloc: these sizes need %lld bytes of split-K scratch; the "
                  "allocation-free entry point holds %lld (use reskv_decode_recent with a workspace)",
                  (long long)need, (long long)kNoAllocScratchBytes);
    // the array used is the current device's: a stream of another device is rejected
    // (the null stream is the current device's)
    int cur = -1, sdev = -1;
    RESKV_REQUIRE(hipGetDevice(&cur) == hipSuccess, "no current HIP device");
    if (stream == nullptr) sdev = cur;
    else RESKV_REQUIRE(hipStreamGetDevice((hipStream_t)stream, &sdev) == hipSuccess,
                       "reskv_decode_recent_noalloc: cannot query the stream's device");
    RESKV_REQUIRE(sdev == cur,
                  "reskv_decode_recent_noalloc: the stream belongs to device %d but device %d is current; make "
                  "the stream's device current (its scratch array is used)", sdev, cur);
    void* ws = scratch_on_current_device();
    if (ws == nullptr) return 1;
    return reskv_decode_recent(q, k, v, inv_freq, rope_table, B, Hq, H, T, start_pos, pos_q, scaling, splits,
                               q_rope, k_recent, v_recent, Tr, r_stride, out, ws, kNoAllocScratchBytes, stream);
}

extern "C" int reskv_decode(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                            const float* inv_freq, int B, int Hq, int H, int T, int start_pos,
                            int pos_q, float scaling, int splits, void* out, float* m, float* l,
                            void* workspace, int64_t workspace_bytes, void* stream) {
    return reskv_decode_rope(q, k, v, inv_freq, nullptr, B, Hq, H, T, start_pos, pos_q, scaling, splits, out, m, l,
                             workspace, workspace_bytes, stream);
}

extern "C" int reskv_decode_dense(const void* q, const void* k, const void* v, const float* inv_freq,
                                  const float* rope_table, int B, int Hq, int H, int T, int t_stride, int start_pos,
                                  int pos_q, float scaling, int splits, void* out, float* m, float* l,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(k && v, "null K/V pointer");
    RESKV_REQUIRE((((uintptr_t)k | (uintptr_t)v) & 15u) == 0, "K and V must be 16-byte aligned");
    const int ts = t_stride > 0 ? t_stride : T;
    RESKV_REQUIRE(ts >= T, "row stride shorter than the sequence");
    const DTensor kd{nullptr, nullptr, (const uint8_t*)k, nullptr, nullptr, 1, kDim, 2 * kDim, ts, 1};
    const DTensor vd{nullptr, nullptr, (const uint8_t*)v, nullptr, nullptr, 1, kDim, 2 * kDim, ts, 1};
    return run_decode(q, D_DENSE, kd, D_DENSE, vd, inv_freq, rope_table, B, Hq, H, T, start_pos, pos_q, scaling,
                      splits, out, m, l, workspace, workspace_bytes, stream);
}

// Table of cos/sin of the reference's RoPE angles fl32(p * inv_freq[i]) for
// positions [0, count): row p holds, for each i0 = 4*li, cos of pairs i0..i0+3
// then sin of the same pairs (512 bytes per position).
__global__ void __launch_bounds__(256) rope_table_kernel(const float* __restrict__ inv_freq, int count,
                                                         float* __restrict__ table) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;  // (position, pair)
    if (idx >= (long)count * kHalf) return;
    const int pos = (int)(idx / kHalf), pair = (int)(idx % kHalf);
    float sn, cs;
    rope_sincos_fast(__fmul_rn((float)pos, inv_freq[pair]), sn, cs);
    // pair 16 g + 4 u + j: cos in piece 2u, sin in piece 2u + 1 of group g;
    // piece i of group g for position p is float4 512 (p / 16) + 64 i + 4 (p % 16) + g
    const int g = pair >> 4, u = (pair >> 2) & 3, j = pair & 3;
    float* cell = table + 4 * ((long)(pos >> 4) * 512 + 64 * (2 * u) + 4 * (pos & 15) + g) + j;
    cell[0] = cs;
    cell[4 * 64] = sn;
}

extern "C" int reskv_rope_table(const float* inv_freq, int count, float* table, void* stream) {
    RESKV_REQUIRE(inv_freq && table, "null pointer argument");
    RESKV_REQUIRE(count > 0 && count % 16 == 0, "position count must be a positive multiple of 16");
    const long n = (long)count * kHalf;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       inv_freq, count, table);
    return reskv_host::check_launch("rope_table_kernel");
}

extern "C" int reskv_merge_recent_scores(const void* comp_out, const float* comp_m, const float* comp_l,
                                         const float* scores, const void* v_recent, int B, int Hq, int H,
                                         int Tr, void* out, void* stream) {
    RESKV_REQUIRE(comp_out && comp_m && comp_l && out, "null pointer argument");
    RESKV_REQUIRE(B > 0 && H > 0 && Hq % H == 0 && Tr >= 0, "bad recent-merge sizes");
    RESKV_REQUIRE(Tr == 0 || (scores && v_recent), "null recent scores/values");
    RESKV_REQUIRE(Tr == 0 || (((uintptr_t)v_recent) & 15u) == 0, "recent V must be 16-byte aligned");
    hipLaunchKernelGGL(merge_recent_kernel, dim3(B * Hq), dim3(kMergeThreads), 0, (hipStream_t)stream,
                       (const uint16_t*)comp_out, comp_m, comp_l, scores, nullptr, nullptr,
                       (const uint16_t*)v_recent, Hq, H, Tr, Tr, 1.0f, (uint16_t*)out);
    return reskv_host::check_launch("merge_recent_kernel");
}

extern "C" int reskv_merge_recent_qk(const void* comp_out, const float* comp_m, const float* comp_l,
                                     const void* q_rope, const void* k_recent, const void* v_recent, int B,
                                     int Hq, int H, int Tr, int r_stride, float scaling, void* out,
                                     void* stream) {
    RESKV_REQUIRE(comp_out && comp_m && comp_l && out, "null pointer argument");
    RESKV_REQUIRE(B > 0 && H > 0 && Hq % H == 0 && Tr >= 0, "bad recent-merge sizes");
    const int rs = r_stride > 0 ? r_stride : Tr;
    RESKV_REQUIRE(rs >= Tr, "recent row stride shorter than the window");
    RESKV_REQUIRE(Tr == 0 || (q_rope && k_recent && v_recent), "null recent tensors");
    RESKV_REQUIRE(Tr == 0 || ((((uintptr_t)k_recent | (uintptr_t)v_recent) & 15u) == 0),
                  "recent K and V must be 16-byte aligned");
    hipLaunchKernelGGL(merge_recent_kernel, dim3(B * Hq), dim3(kMergeThreads), 0, (hipStream_t)stream,
                       (const uint16_t*)comp_out, comp_m, comp_l, nullptr, (const uint16_t*)q_rope,
                       (const uint16_t*)k_recent, (const uint16_t*)v_recent, Hq, H, Tr, rs, scaling, (uint16_t*)out);
    return reskv_host::check_launch("merge_recent_kernel");
}
