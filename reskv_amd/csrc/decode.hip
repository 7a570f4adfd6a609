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
// payload, scales) are copied with 16-byte loads into the wave's LDS stage,
// prefetching the next tile into registers meanwhile.  Inside a tile the wave
// works on four tokens at a time: lane L = 16 * row + i takes token 4 * step +
// row and channels {4i..4i+3} u {64+4i..64+4i+3} (four RoPE pairs), so a score
// is a 16-lane DPP row sum.  The online softmax runs per tile in the log2
// domain; the cluster mass beta accumulates with LDS atomics.
// Merge kernel: one wave per (batch, query head) rescales the split partials to
// a common maximum, folds sum_c beta_c c_v[c] and normalises.
#include "common.h"
#include "../../include/reskv_hip.h"

#include <math.h>

using namespace reskv;

namespace {

// residual formats as the kernels see them (the two quantised widths split)
// (_W: the same layout with payload rows wider than 128 bytes, i.e. nnz > 64,
// which needs more prefetch registers per lane)
enum DFmt { D_BITMAP = 0, D_TILED, D_STRUCT16, D_SINT4, D_Q4, D_Q2, D_DENSE, D_BITMAP_W, D_TILED_W };

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kTile = 16;      // tokens per wave tile
constexpr int kRows = 4;       // tokens processed together (one per 16-lane row)
constexpr int kSteps = kTile / kRows;
constexpr int kMaxSplits = 1024;
constexpr int kPartStride = kDim + kMaxClusters + 2;  // cross-wave merge record
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kVPitch = kDim + 8;  // halves per token row of the V transpose tile (conflict-free writes)

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

template <int F> struct Traits;
template <> struct Traits<D_BITMAP> { static constexpr int MB = 16, PQ = 2; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_TILED> { static constexpr int MB = 16, PQ = 2; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_BITMAP_W> { static constexpr int MB = 16, PQ = 4; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_TILED_W> { static constexpr int MB = 16, PQ = 4; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_STRUCT16> { static constexpr int MB = 16, PQ = 1; static constexpr bool SC = false, CENT = true; };
template <> struct Traits<D_SINT4> { static constexpr int MB = 8, PQ = 1; static constexpr bool SC = true, CENT = true; };
template <> struct Traits<D_Q4> { static constexpr int MB = 0, PQ = 1; static constexpr bool SC = true, CENT = true; };
template <> struct Traits<D_Q2> { static constexpr int MB = 0, PQ = 1; static constexpr bool SC = true, CENT = true; };
template <> struct Traits<D_DENSE> { static constexpr int MB = 0, PQ = 4; static constexpr bool SC = false, CENT = false; };

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
    const float4* rope;  // [position][16][cos x4, sin x4] table, or null (recurrence in-kernel)
    int Hq, H, T, start_pos, pos_q, splits;
    float qscale;  // scaling * log2(e): scores come out in the log2 domain
    int stage_k, stage_v;  // LDS stage bytes per wave for K and V
    int beta_off, lut_off, p_off, stage_off;  // LDS byte offsets (region 0 holds centroids / merge records)
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
template <int F>
struct Prefetch {
    uint4 pay[Traits<F>::PQ];
    uint4 meta;
    int id;
    float sc;
};

// Loads the raw bytes of tokens [row0, row0 + n) of one tensor (row0 = bh*T + t).
template <int F>
__device__ __forceinline__ void prefetch(const DTensor& X, long row0, int n, int lane, Prefetch<F>& P) {
    using Tr = Traits<F>;
    const int per_tok = X.pb >> 4;
    const int pieces = n * per_tok;
    const uint4* src = reinterpret_cast<const uint4*>(X.payload + row0 * X.pb);
#pragma unroll
    for (int i = 0; i < Tr::PQ; ++i) {
        const int q = lane + kWave * i;
        P.pay[i] = q < pieces ? src[q] : make_uint4(0, 0, 0, 0);
    }
    P.meta = make_uint4(0, 0, 0, 0);
    if constexpr (Tr::MB == 16) {
        if (lane < n) P.meta = reinterpret_cast<const uint4*>(X.meta + row0 * 16)[lane];
    } else if constexpr (Tr::MB == 8) {
        if (lane < n) {
            const uint2 m = reinterpret_cast<const uint2*>(X.meta + row0 * 8)[lane];
            P.meta.x = m.x;
            P.meta.y = m.y;
        }
    }
    P.id = 0;
    if constexpr (Tr::CENT) {
        if (lane < n) P.id = X.ids[row0 + lane];
    }
    P.sc = 0.0f;
    if constexpr (Tr::SC) {
        if (lane < n) P.sc = h2f(X.scale[row0 + lane]);
    }
}

// Stage layout (bytes): payload [16][pb] | meta [16][MB] | ids int32[16] | scale f32[16]
template <int F>
__device__ __forceinline__ void stage_store(const Prefetch<F>& P, uint8_t* st, int pb, int lane) {
    using Tr = Traits<F>;
    const int pieces = kTile * (pb >> 4);
    uint4* pay = reinterpret_cast<uint4*>(st);
#pragma unroll
    for (int i = 0; i < Tr::PQ; ++i) {
        const int q = lane + kWave * i;
        if (q < pieces) pay[q] = P.pay[i];
    }
    uint8_t* meta = st + kTile * pb;
    if (lane < kTile) {
        if constexpr (Tr::MB == 16) reinterpret_cast<uint4*>(meta)[lane] = P.meta;
        if constexpr (Tr::MB == 8) reinterpret_cast<uint2*>(meta)[lane] = make_uint2(P.meta.x, P.meta.y);
        int* ids = reinterpret_cast<int*>(meta + kTile * Tr::MB);
        ids[lane] = P.id;
        reinterpret_cast<float*>(ids + kTile)[lane] = P.sc;
    }
}

template <int F>
__host__ __device__ constexpr int stage_bytes(int pb) {
    return kTile * pb + kTile * Traits<F>::MB + 2 * kTile * 4;
}

// ---------------------------------------------------------------------------
// residual decoders (LDS stage -> 8 fp32 values of this lane's channels)
// r[0..3] = channels 4i..4i+3, r[4..7] = channels 64+4i..64+4i+3
//
// FP16 formats: the kept values of a lane's 4-channel run are consecutive in
// the payload row, starting at rank `base`.  The 8-byte window at `base` is
// fetched with two dword reads plus an alignbit, and one v_perm per channel
// pair scatters the window's halves onto the kept channels (zeros elsewhere).
// The permute selectors depend only on the run's 4-bit keep pattern and come
// from a 16-entry table in LDS (one table for MSB-first bitmaps, one for
// LSB-first tile masks).
// ---------------------------------------------------------------------------
constexpr int kLutWords = 64;  // [msb|lsb][pattern][lo|hi]

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

__device__ __forceinline__ float half_lo(uint32_t w) { return h2f((uint16_t)(w & 0xFFFFu)); }
__device__ __forceinline__ float half_hi(uint32_t w) { return h2f((uint16_t)(w >> 16)); }

// Kept values of one 4-channel run, as fp32: window of the payload row at
// rank `base`, scattered by the pattern's selectors.
__device__ __forceinline__ void expand_run(const uint8_t* row, int base, const uint32_t* lut, uint32_t v,
                                           float* r) {
    const uint32_t* dw = reinterpret_cast<const uint32_t*>(row) + (base >> 1);
    const uint32_t d0 = dw[0], d1 = dw[1], d2 = dw[2];
    const uint32_t sh = (uint32_t)(base & 1) * 16u;
    const uint32_t w0 = __builtin_amdgcn_alignbit(d1, d0, sh);
    const uint32_t w1 = __builtin_amdgcn_alignbit(d2, d1, sh);
    const uint2 sel = *reinterpret_cast<const uint2*>(lut + 2 * v);
    const uint32_t lo = __builtin_amdgcn_perm(w1, w0, sel.x);
    const uint32_t hi = __builtin_amdgcn_perm(w1, w0, sel.y);
    r[0] = half_lo(lo);
    r[1] = half_hi(lo);
    r[2] = half_lo(hi);
    r[3] = half_hi(hi);
}

template <int F>
__device__ __forceinline__ void decode_res(const uint8_t* st, int tok, int pb, int width, int li,
                                           const uint32_t* lut, float* r) {
    using Tr = Traits<F>;
    const uint8_t* payb = st + tok * pb;
    const uint8_t* meta = st + kTile * pb + tok * Tr::MB;
    if constexpr (F == D_BITMAP || F == D_BITMAP_W) {
        // channel d <-> bit (63 - d % 64) of word d / 64; value index = rank (reference.py:22-26)
        const uint4 m = *reinterpret_cast<const uint4*>(meta);
        const uint64_t w0 = (uint64_t)m.x | ((uint64_t)m.y << 32);
        const uint64_t w1 = (uint64_t)m.z | ((uint64_t)m.w << 32);
        const int sh = 60 - 4 * li;
        const uint32_t na = (uint32_t)(w0 >> sh) & 15u, nb = (uint32_t)(w1 >> sh) & 15u;
        // bits above this lane's run: (w >> 1) >> (63 - 4i) keeps every shift below 64
        const int hi = 63 - 4 * li;
        const int ba = li ? __builtin_popcountll((w0 >> 1) >> hi) : 0;
        const int bb = __builtin_popcountll(w0) + (li ? __builtin_popcountll((w1 >> 1) >> hi) : 0);
        expand_run(payb, ba, lut, na, r);
        expand_run(payb, bb, lut, nb, r + 4);
    } else if constexpr (F == D_TILED || F == D_TILED_W || F == D_STRUCT16) {
        // word w = code(tile 2w) | code(tile 2w+1) << 16 (reference.py:36-47)
        const uint4 m = *reinterpret_cast<const uint4*>(meta);
        const uint32_t mw[4] = {m.x, m.y, m.z, m.w};
        const int per_tile = F == D_STRUCT16 ? 4 : (width >> 3);
        const int sub = li & 3;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int tile = (li >> 2) + 4 * half;
            uint32_t code = (mw[tile >> 1] >> (16 * (tile & 1))) & 0xFFFFu;
            if (F == D_STRUCT16) {
                // four ascending in-tile channel indices -> 16-bit mask
                uint32_t mask = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) mask |= 1u << ((code >> (4 * k)) & 15u);
                code = mask;
            }
            const uint32_t nib = (code >> (4 * sub)) & 15u;
            const int base = tile * per_tile + __builtin_popcount(code & ((1u << (4 * sub)) - 1u));
            expand_run(payb, base, lut + 32, nib, r + 4 * half);
        }
    } else if constexpr (F == D_SINT4) {
        // 1 of 4 per subgroup: 2-bit position, signed nibble code, fp16 scale (reference.py:27-35)
        const uint4 qp = *reinterpret_cast<const uint4*>(payb);
        const uint2 qm = *reinterpret_cast<const uint2*>(meta);
        const float s = reinterpret_cast<const float*>(st + kTile * pb + kTile * Tr::MB + kTile * 4)[tok];
        const uint32_t qw[4] = {qp.x, qp.y, qp.z, qp.w};
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int grp = li + 16 * half;
            const uint32_t sel = ((half ? qm.y : qm.x) >> (2 * li)) & 3u;
            const int code = (int)__builtin_amdgcn_sbfe((int)qw[grp >> 3], 4 * (grp & 7), 4);  // typed unsigned
            const float val = (float)code * s;
#pragma unroll
            for (int j = 0; j < 4; ++j) r[4 * half + j] = (uint32_t)j == sel ? val : 0.0f;
        }
    } else if constexpr (F == D_Q4 || F == D_Q2) {
        // signed codes, channel d in word d / (32/bits) at bit (d % (32/bits)) * bits (reference.py:17-21)
        constexpr int bits = F == D_Q4 ? 4 : 2;
        constexpr int per_word = 32 / bits;
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(payb);
        const float s = reinterpret_cast<const float*>(st + kTile * pb + kTile * 4)[tok];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int d0 = 4 * li + 64 * half;
            const int w = (int)qw[d0 / per_word];
            const int off = (d0 % per_word) * bits;
#pragma unroll
            for (int j = 0; j < 4; ++j) r[4 * half + j] = (float)(int)__builtin_amdgcn_sbfe(w, off + j * bits, bits) * s;
        }
    } else {  // dense fp16 rows
        const uint16_t* p16 = reinterpret_cast<const uint16_t*>(payb);
        const uint2 a = *reinterpret_cast<const uint2*>(p16 + 4 * li);
        const uint2 b = *reinterpret_cast<const uint2*>(p16 + 64 + 4 * li);
        r[0] = half_lo(a.x);
        r[1] = half_hi(a.x);
        r[2] = half_lo(a.y);
        r[3] = half_hi(a.y);
        r[4] = half_lo(b.x);
        r[5] = half_hi(b.x);
        r[6] = half_lo(b.y);
        r[7] = half_hi(b.y);
    }
}

// The same residuals as fp16 pairs for the matrix cores: h[0] = channels
// (4i, 4i+1), h[1] = (4i+2, 4i+3), h[2], h[3] = the same of channels 64+4i...
// FP16 formats hand their payload halves through unchanged; quantised codes
// are dequantised in fp32 and rounded once to fp16.
template <int F>
__device__ __forceinline__ void decode_res_h(const uint8_t* st, int tok, int pb, int width, int li,
                                             const uint32_t* lut, uint32_t* h) {
    using Tr = Traits<F>;
    const uint8_t* payb = st + tok * pb;
    const uint8_t* meta = st + kTile * pb + tok * Tr::MB;
    auto run = [&](int base, const uint32_t* tab, uint32_t v, uint32_t* out) {
        const uint32_t* dw = reinterpret_cast<const uint32_t*>(payb) + (base >> 1);
        const uint32_t d0 = dw[0], d1 = dw[1], d2 = dw[2];
        const uint32_t sh = (uint32_t)(base & 1) * 16u;
        const uint32_t w0 = __builtin_amdgcn_alignbit(d1, d0, sh);
        const uint32_t w1 = __builtin_amdgcn_alignbit(d2, d1, sh);
        const uint2 sel = *reinterpret_cast<const uint2*>(tab + 2 * v);
        out[0] = __builtin_amdgcn_perm(w1, w0, sel.x);
        out[1] = __builtin_amdgcn_perm(w1, w0, sel.y);
    };
    if constexpr (F == D_BITMAP || F == D_BITMAP_W) {
        const uint4 m = *reinterpret_cast<const uint4*>(meta);
        const uint64_t w0 = (uint64_t)m.x | ((uint64_t)m.y << 32);
        const uint64_t w1 = (uint64_t)m.z | ((uint64_t)m.w << 32);
        const int sh = 60 - 4 * li;
        const uint32_t na = (uint32_t)(w0 >> sh) & 15u, nb = (uint32_t)(w1 >> sh) & 15u;
        const int hi = 63 - 4 * li;
        const int ba = li ? __builtin_popcountll((w0 >> 1) >> hi) : 0;
        const int bb = __builtin_popcountll(w0) + (li ? __builtin_popcountll((w1 >> 1) >> hi) : 0);
        run(ba, lut, na, h);
        run(bb, lut, nb, h + 2);
    } else if constexpr (F == D_TILED || F == D_TILED_W || F == D_STRUCT16) {
        const uint4 m = *reinterpret_cast<const uint4*>(meta);
        const uint32_t mw[4] = {m.x, m.y, m.z, m.w};
        const int per_tile = F == D_STRUCT16 ? 4 : (width >> 3);
        const int sub = li & 3;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int tile = (li >> 2) + 4 * half;
            uint32_t code = (mw[tile >> 1] >> (16 * (tile & 1))) & 0xFFFFu;
            if (F == D_STRUCT16) {
                uint32_t mask = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) mask |= 1u << ((code >> (4 * k)) & 15u);
                code = mask;
            }
            const uint32_t nib = (code >> (4 * sub)) & 15u;
            const int base = tile * per_tile + __builtin_popcount(code & ((1u << (4 * sub)) - 1u));
            run(base, lut + 32, nib, h + 2 * half);
        }
    } else if constexpr (F == D_DENSE) {
        const uint16_t* p16 = reinterpret_cast<const uint16_t*>(payb);
        const uint2 a = *reinterpret_cast<const uint2*>(p16 + 4 * li);
        const uint2 b = *reinterpret_cast<const uint2*>(p16 + 64 + 4 * li);
        h[0] = a.x;
        h[1] = a.y;
        h[2] = b.x;
        h[3] = b.y;
    } else {
        float r[8];
        decode_res<F>(st, tok, pb, width, li, lut, r);
#pragma unroll
        for (int k = 0; k < 4; ++k) h[k] = (uint32_t)f2h(r[2 * k]) | ((uint32_t)f2h(r[2 * k + 1]) << 16);
    }
}

template <int F>
__device__ __forceinline__ int stage_id(const uint8_t* st, int pb, int tok) {
    return reinterpret_cast<const int*>(st + kTile * pb + kTile * Traits<F>::MB)[tok];
}

__device__ __forceinline__ int clamp_id(int id, int nc) { return id < 0 ? 0 : (id >= nc ? nc - 1 : id); }

__device__ __forceinline__ float rows_max(float v) {
    return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}
// sum over the four rows, result in every lane (lanes i, i+16, i+32, i+48)
__device__ __forceinline__ float cross_rows_sum(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// ---------------------------------------------------------------------------
// RoPE by recurrence.  A lane keeps (C, S) = cos/sin of the exact angle p*f of
// its row's current position p (advanced by 4 positions per step with
// precomputed cos/sin of 4f).  The angle the reference uses is hi = fl32(p*f);
// e = p*f - hi is exact (one FMA), and cos(hi) = C + e*S, sin(hi) = S - e*C to
// well below fp32 resolution (|e| <= ulp(hi)/2, so e^2 is negligible).
// ---------------------------------------------------------------------------
struct Rope {
    float C[4], S[4], c4[4], s4[4];
};

__device__ __forceinline__ void rope_anchor(Rope& R, const float* f, float pos) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float hi = __fmul_rn(pos, f[j]);
        const float e = __builtin_fmaf(pos, f[j], -hi);
        float sn, cs;
        rope_sincos_fast(hi, sn, cs);
        R.C[j] = __builtin_fmaf(-e, sn, cs);
        R.S[j] = __builtin_fmaf(e, cs, sn);
    }
}

// ---------------------------------------------------------------------------
// partial kernel
// ---------------------------------------------------------------------------
template <int G, int KF, int VF, bool TAB>
__global__ void __launch_bounds__(kThreads) decode_partial_kernel(DParams P) {
    extern __shared__ __align__(16) uint8_t smem[];
    using KT = Traits<KF>;
    using VT = Traits<VF>;
    constexpr int NV = kSteps * G;             // softmax values of one row per tile
    constexpr int NVL = (NV + 15) / 16;        // values per lane
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const long bh = (long)b * P.H + h;
    const int s0 = (int)(((long)split * P.T) / P.splits);
    const int s1 = (int)(((long)(split + 1) * P.T) / P.splits);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = lane >> 4, li = lane & 15;
    // this wave's contiguous share of the split
    const int t0 = s0 + (int)(((long)wave * (s1 - s0)) / kWaves);
    const int t1 = s0 + (int)(((long)(wave + 1) * (s1 - s0)) / kWaves);

    float* s_cent = reinterpret_cast<float*>(smem);                          // region 0
    float* my_beta = reinterpret_cast<float*>(smem + P.beta_off) + wave * G * kMaxClusters;
    uint32_t* s_lut = reinterpret_cast<uint32_t*>(smem + P.lut_off);
    // per wave: fp16 weights [step][head][row] and the V tile [token][kVPitch] for the matrix cores
    uint16_t* my_p = reinterpret_cast<uint16_t*>(smem + P.p_off) + wave * (kSteps * G * kRows + kTile * kVPitch);
    uint16_t* my_vt = my_p + kSteps * G * kRows;
    uint8_t* st_k = smem + P.stage_off + wave * (P.stage_k + P.stage_v);
    uint8_t* st_v = st_k + P.stage_k;

    if constexpr (KT::CENT) {
        const uint16_t* kc = P.k.cent + bh * P.k.cs * kDim;
        for (int i = threadIdx.x; i < P.k.nc * kDim; i += kThreads) s_cent[i] = h2f(kc[i]);
#pragma unroll
        for (int g = 0; g < G; ++g) my_beta[g * kMaxClusters + lane] = 0.0f;
    }
    if (threadIdx.x < kLutWords) {
        const uint32_t t = threadIdx.x;
        s_lut[t] = perm_selector((t >> 1) & 15u, t < 32, (int)(t & 1));
    }

    // rotated, pre-scaled query: qa = channels 4i+j, qb = channels 64+4i+j
    const float4 fq = *reinterpret_cast<const float4*>(P.inv_freq + 4 * li);
    const float freq[4] = {fq.x, fq.y, fq.z, fq.w};
    float qa[G][4], qb[G][4];
    Rope R;
    {
        float sn[4], cs[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            rope_sincos_fast(__fmul_rn((float)P.pos_q, freq[j]), sn[j], cs[j]);
            if (!TAB) rope_sincos_fast(4.0f * freq[j], R.s4[j], R.c4[j]);  // 4f is exact in fp32
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint16_t* qr = P.q + ((long)b * P.Hq + (long)h * G + g) * kDim;
            const uint2 ua = *reinterpret_cast<const uint2*>(qr + 4 * li);
            const uint2 ub = *reinterpret_cast<const uint2*>(qr + 64 + 4 * li);
            const float a[4] = {half_lo(ua.x), half_hi(ua.x), half_lo(ua.y), half_hi(ua.y)};
            const float c[4] = {half_lo(ub.x), half_hi(ub.x), half_lo(ub.y), half_hi(ub.y)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qa[g][j] = (a[j] * cs[j] - c[j] * sn[j]) * P.qscale;
                qb[g][j] = (c[j] * cs[j] + a[j] * sn[j]) * P.qscale;
            }
        }
    }

    // this lane's softmax values: v = li + 16k -> (step v / G, head v % G)
    int vs[NVL], vg[NVL];
    bool vown[NVL];
#pragma unroll
    for (int k = 0; k < NVL; ++k) {
        const int v = li + 16 * k;
        vown[k] = v < NV;
        vs[k] = (v % NV) / G;
        vg[k] = (v % NV) % G;
    }

    // residual sums on the matrix cores (v_mfma_f32_4x4x4f16, 16 blocks of 4 lanes):
    // lane L accumulates delta[4*gs + i][L + 64*half] in acc[gs][half][i]
    constexpr int NGS = (G + 3) / 4;
    float4_t acc[NGS][2];
    float m[G], lv[NVL];
#pragma unroll
    for (int gs = 0; gs < NGS; ++gs) acc[gs][0] = acc[gs][1] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < G; ++g) m[g] = -INFINITY;
#pragma unroll
    for (int k = 0; k < NVL; ++k) lv[k] = 0.0f;
    __syncthreads();

    const int ntiles = (t1 - t0 + kTile - 1) / kTile;
    Prefetch<KF> pk;
    Prefetch<VF> pv;
    if (ntiles > 0) {
        const int n = min(kTile, t1 - t0);
        prefetch<KF>(P.k, bh * P.k.ts + t0, n, lane, pk);
        prefetch<VF>(P.v, bh * P.v.ts + t0, n, lane, pv);
    }
    for (int tile = 0; tile < ntiles; ++tile) {
        const int tb = t0 + tile * kTile;
        const int n = min(kTile, t1 - tb);
        stage_store<KF>(pk, st_k, P.k.pb, lane);
        stage_store<VF>(pv, st_v, P.v.pb, lane);
        wave_sync();
        if (tile + 1 < ntiles) {
            const int tb2 = tb + kTile;
            const int n2 = min(kTile, t1 - tb2);
            prefetch<KF>(P.k, bh * P.k.ts + tb2, n2, lane, pk);
            prefetch<VF>(P.v, bh * P.v.ts + tb2, n2, lane, pv);
        }
        if (!TAB && (tile & 7) == 0) rope_anchor(R, freq, (float)(P.start_pos + tb + row));
        // table rows of this lane's four steps: cos/sin of pairs 4i..4i+3 at the row's positions
        float4 tc[kSteps], ts[kSteps];
        if constexpr (TAB) {
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                const float4* tr = P.rope + ((long)(P.start_pos + tb + kRows * s + row) * 16 + li) * 2;
                tc[s] = tr[0];
                ts[s] = tr[1];
            }
        }

        // ---- scores of the tile's 16 tokens (log2 domain) ----
        float sc[G][kSteps];
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const int tok = kRows * s + row;
            float kr[8];
            decode_res<KF>(st_k, tok, P.k.pb, P.k.width, li, s_lut, kr);
            if constexpr (KT::CENT) {
                const int kid = clamp_id(stage_id<KF>(st_k, P.k.pb, tok), P.k.nc);
                const float4 ca = *reinterpret_cast<const float4*>(s_cent + kid * kDim + 4 * li);
                const float4 cb = *reinterpret_cast<const float4*>(s_cent + kid * kDim + 64 + 4 * li);
                kr[0] += ca.x; kr[1] += ca.y; kr[2] += ca.z; kr[3] += ca.w;
                kr[4] += cb.x; kr[5] += cb.y; kr[6] += cb.z; kr[7] += cb.w;
            }
            const float pos = (float)(P.start_pos + tb + tok);
            float xa[4], xb[4];
            if constexpr (TAB) {
                const float cs4[4] = {tc[s].x, tc[s].y, tc[s].z, tc[s].w};
                const float sn4[4] = {ts[s].x, ts[s].y, ts[s].z, ts[s].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    xa[j] = kr[j] * cs4[j] - kr[4 + j] * sn4[j];
                    xb[j] = kr[4 + j] * cs4[j] + kr[j] * sn4[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float hi = __fmul_rn(pos, freq[j]);
                    const float e = __builtin_fmaf(pos, freq[j], -hi);
                    const float cs = __builtin_fmaf(e, R.S[j], R.C[j]);
                    const float sn = __builtin_fmaf(-e, R.C[j], R.S[j]);
                    xa[j] = kr[j] * cs - kr[4 + j] * sn;
                    xb[j] = kr[4 + j] * cs + kr[j] * sn;
                    const float nc = R.C[j] * R.c4[j] - R.S[j] * R.s4[j];
                    R.S[j] = R.S[j] * R.c4[j] + R.C[j] * R.s4[j];
                    R.C[j] = nc;
                }
            }
            const bool valid = tok < n;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float part = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) part = fmaf(qa[g][j], xa[j], fmaf(qb[g][j], xb[j], part));
                const float score = row_sum16(part);
                sc[g][s] = valid ? score : -INFINITY;
            }
        }

        // ---- online softmax over the tile: one exponential per lane value ----
        bool grow = false;
        float mnew[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mx = sc[g][0];
#pragma unroll
            for (int s = 1; s < kSteps; ++s) mx = fmaxf(mx, sc[g][s]);
            mnew[g] = fmaxf(m[g], rows_max(mx));
            grow |= mnew[g] > m[g];
        }
        if (grow) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float alpha = exp2_fast(m[g] - mnew[g]);  // 0 on the first tile
                acc[g >> 2][0][g & 3] *= alpha;
                acc[g >> 2][1][g & 3] *= alpha;
                if constexpr (KT::CENT) my_beta[g * kMaxClusters + lane] *= alpha;
#pragma unroll
                for (int k = 0; k < NVL; ++k) lv[k] = vg[k] == g ? lv[k] * alpha : lv[k];
                m[g] = mnew[g];
            }
        }
#pragma unroll
        for (int k = 0; k < NVL; ++k) {
            float pick = sc[0][0], mg = m[0];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                mg = vg[k] == g ? m[g] : mg;
#pragma unroll
                for (int s = 0; s < kSteps; ++s) pick = (vs[k] == s && vg[k] == g) ? sc[g][s] : pick;
            }
            // the residual sums take the weight in fp16; the normaliser and the
            // cluster mass use the same rounded weight so the average stays consistent
            const uint16_t ph = f2h(exp2_fast(pick - mg));
            const float pk_ = h2f(ph);
            if (vown[k]) {
                lv[k] += pk_;
                my_p[(vs[k] * G + vg[k]) * kRows + row] = ph;
                if constexpr (VT::CENT) {
                    const int vid = clamp_id(stage_id<VF>(st_v, P.v.pb, kRows * vs[k] + row), P.v.nc);
                    atomicAdd(&my_beta[vg[k] * kMaxClusters + vid], pk_);
                }
            }
        }
        wave_sync();

        // ---- values: residuals as fp16 into the transpose tile, then P x V on the matrix cores ----
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const int tok = kRows * s + row;
            uint32_t hv[4];
            decode_res_h<VF>(st_v, tok, P.v.pb, P.v.width, li, s_lut, hv);
            *reinterpret_cast<uint2*>(my_vt + tok * kVPitch + 4 * li) = make_uint2(hv[0], hv[1]);
            *reinterpret_cast<uint2*>(my_vt + tok * kVPitch + 64 + 4 * li) = make_uint2(hv[2], hv[3]);
        }
        wave_sync();
        {
            const int blk_row = lane & 3;  // A row (query head within the set) of this lane
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                // B: lane L holds V[tokens 4s + r, r = 0..3][channel L (+64)]
                half4_t b0, b1;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    b0[r] = __builtin_bit_cast(_Float16, my_vt[(kRows * s + r) * kVPitch + lane]);
                    b1[r] = __builtin_bit_cast(_Float16, my_vt[(kRows * s + r) * kVPitch + 64 + lane]);
                }
#pragma unroll
                for (int gs = 0; gs < NGS; ++gs) {
                    // A: lane 4b + i holds P[head 4*gs + i][tokens 4s + r]
                    const int g = 4 * gs + blk_row;
                    half4_t a = (half4_t){0, 0, 0, 0};
                    if (g < G) a = __builtin_bit_cast(half4_t, *reinterpret_cast<const uint2*>(my_p + (s * G + g) * kRows));
                    acc[gs][0] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, b0, acc[gs][0], 0, 0, 0);
                    acc[gs][1] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, b1, acc[gs][1], 0, 0, 0);
                }
            }
        }
        wave_sync();  // stage and p reads done before the next tile overwrites them
    }

    // ---- fold the four rows, then merge the waves through LDS ----
    float lt[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float ls = 0.0f;
#pragma unroll
        for (int k = 0; k < NVL; ++k) ls += (vown[k] && vg[k] == g) ? lv[k] : 0.0f;
        lt[g] = wave_sum(ls);
    }
    float bt[G];
#pragma unroll
    for (int g = 0; g < G; ++g) bt[g] = KT::CENT ? my_beta[g * kMaxClusters + lane] : 0.0f;
    __syncthreads();  // centroid table and stages no longer needed
    float* rec = reinterpret_cast<float*>(smem) + wave * G * kPartStride;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float* e = rec + g * kPartStride;
        e[lane] = acc[g >> 2][0][g & 3];
        e[64 + lane] = acc[g >> 2][1][g & 3];
        e[kDim + lane] = bt[g];
        if (lane == 0) {
            e[kDim + kMaxClusters] = m[g];
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
// partials (log2 domain).  The residual sums are read as float4 by 8 groups of
// 32 threads (split s goes to group s % 8), the cluster masses by 16 groups of
// 16 threads, so a thread keeps at most S/8 independent loads in flight;
// the groups are then reduced through LDS.
constexpr int kMergeThreads = 256;

__global__ void __launch_bounds__(kMergeThreads) decode_merge_kernel(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ pdelta,
    const float* __restrict__ pbeta, const uint16_t* __restrict__ vcent, int vnc, int vcs, int Hq, int H,
    int splits, uint16_t* __restrict__ out, float* __restrict__ om, float* __restrict__ ol) {
    __shared__ float s_w[kMaxSplits];
    __shared__ float s_red[kMergeThreads / kWave];
    __shared__ float4 s_d[8][kDim / 4];
    __shared__ float4 s_b[16][kMaxClusters / 4];
    const long bq = blockIdx.x;  // b * Hq + hq
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = Hq / H;
    const long bh = (bq / Hq) * H + (bq % Hq) / G;
    const float* m_row = pm + bq * splits;
    const float* l_row = pl + bq * splits;

    // 1) common maximum over the non-empty splits
    float mx = -INFINITY;
    for (int s = tid; s < splits; s += kMergeThreads)
        if (l_row[s] > 0.0f) mx = fmaxf(mx, m_row[s]);
    mx = wave_max(mx);
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();

    // 2) split weights and the normaliser
    float lsum = 0.0f;
    for (int s = tid; s < splits; s += kMergeThreads) {
        const float lw = l_row[s];
        const float w = lw > 0.0f ? exp2_fast(m_row[s] - mx) : 0.0f;
        s_w[s] = w;
        lsum += lw * w;
    }
    lsum = wave_sum(lsum);
    if (lane == 0) s_red[wave] = lsum;
    __syncthreads();
    lsum = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);

    // 3) residual sums: thread = (split group tid / 32, channel quad tid % 32)
    {
        const int grp = tid >> 5, cq = tid & 31;
        const float4* base = reinterpret_cast<const float4*>(pdelta + (bq * splits) * kDim) + cq;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
        for (int s = grp; s < splits; s += 8) {
            const float w = s_w[s];
            const float4 d = base[(long)s * (kDim / 4)];
            acc.x = fmaf(w, d.x, acc.x);
            acc.y = fmaf(w, d.y, acc.y);
            acc.z = fmaf(w, d.z, acc.z);
            acc.w = fmaf(w, d.w, acc.w);
        }
        s_d[grp][cq] = acc;
    }
    // 4) cluster mass: thread = (split group tid / 16, cluster quad tid % 16)
    {
        const int grp = tid >> 4, cq = tid & 15;
        const float4* base = reinterpret_cast<const float4*>(pbeta + (bq * splits) * kMaxClusters) + cq;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
        for (int s = grp; s < splits; s += 16) {
            const float w = s_w[s];
            const float4 d = base[(long)s * (kMaxClusters / 4)];
            acc.x = fmaf(w, d.x, acc.x);
            acc.y = fmaf(w, d.y, acc.y);
            acc.z = fmaf(w, d.z, acc.z);
            acc.w = fmaf(w, d.w, acc.w);
        }
        s_b[grp][cq] = acc;
    }
    __syncthreads();
    // 5) fold sum_c beta_c c_v[c], normalise (threads 0..127: one channel each)
    if (tid < kDim) {
        const float* sd = reinterpret_cast<const float*>(s_d);
        float acc = 0.0f;
#pragma unroll
        for (int g2 = 0; g2 < 8; ++g2) acc += sd[g2 * kDim + tid];
        if (vcent != nullptr) {
            const float* sb = reinterpret_cast<const float*>(s_b);
            const uint16_t* vc = vcent + bh * vcs * kDim + tid;
            for (int c = 0; c < vnc; ++c) {
                float beta = 0.0f;
#pragma unroll
                for (int g2 = 0; g2 < 16; ++g2) beta += sb[g2 * kMaxClusters + c];
                acc = fmaf(beta, h2f(vc[c * kDim]), acc);
            }
        }
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        out[bq * kDim + tid] = f2h(acc * inv);
        if (tid == 0) {
            if (om) om[bq] = mx * kLn2;  // natural-log units, as the reference returns m
            if (ol) ol[bq] = lsum;
        }
    }
}

// Joint softmax of a normalised compressed result (m, l) with Tr recent tokens
// whose scaled scores are given (scores != null) or computed from q_rope/k.
__global__ void __launch_bounds__(64) merge_recent_kernel(
    const uint16_t* __restrict__ comp_out, const float* __restrict__ comp_m, const float* __restrict__ comp_l,
    const float* __restrict__ scores, const uint16_t* __restrict__ q_rope, const uint16_t* __restrict__ k_recent,
    const uint16_t* __restrict__ v_recent, int Hq, int H, int Tr, float scaling, uint16_t* __restrict__ out) {
    const long bq = blockIdx.x;
    const int lane = threadIdx.x;
    const int G = Hq / H;
    const long b = bq / Hq, hq = bq % Hq;
    const long bh = b * H + hq / G;
    float qa = 0.0f, qb = 0.0f;
    if (scores == nullptr) {
        qa = h2f(q_rope[bq * kDim + lane]);
        qb = h2f(q_rope[bq * kDim + lane + 64]);
    }
    float m = -INFINITY, l = 0.0f, a0 = 0.0f, a1 = 0.0f;
    for (int t = 0; t < Tr; ++t) {
        const long vrow = (bh * Tr + t) * kDim;
        float s;
        if (scores != nullptr) {
            s = scores[bq * Tr + t];
        } else {
            s = wave_sum(qa * h2f(k_recent[vrow + lane]) + qb * h2f(k_recent[vrow + lane + 64])) * scaling;
        }
        const float mn = fmaxf(m, s);
        const float alpha = expf(m - mn), p = expf(s - mn);
        l = l * alpha + p;
        a0 = a0 * alpha + p * h2f(v_recent[vrow + lane]);
        a1 = a1 * alpha + p * h2f(v_recent[vrow + lane + 64]);
        m = mn;
    }
    const float cm = comp_m[bq], cl = comp_l[bq];
    const float jm = fmaxf(cm, m);
    const float wc = cl > 0.0f ? cl * expf(cm - jm) : 0.0f;
    const float wr = Tr > 0 ? expf(m - jm) : 0.0f;
    const float denom = wc + l * wr;
    const float inv = denom > 0.0f ? 1.0f / denom : 0.0f;
    out[bq * kDim + lane] = f2h((h2f(comp_out[bq * kDim + lane]) * wc + a0 * wr) * inv);
    out[bq * kDim + lane + 64] = f2h((h2f(comp_out[bq * kDim + lane + 64]) * wc + a1 * wr) * inv);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Two 4-wave workgroups fit a CU at this kernel's register use, so about 512
// workgroups fill the 256 CUs once; each wave keeps at least two 16-token
// tiles so that its next tile's loads overlap the current tile's arithmetic.
int auto_splits(int B, int H, int T) {
    const long heads = (long)B * H;
    long s = (512 + heads - 1) / heads;
    const long cap = T / (kWaves * 2 * kTile) > 0 ? T / (kWaves * 2 * kTile) : 1;
    if (s > cap) s = cap;
    if (s > kMaxSplits) s = kMaxSplits;
    return (int)(s < 1 ? 1 : s);
}

int resolve_splits(int B, int H, int T, int splits) {
    if (splits > 0) {
        int s = splits < T ? splits : T;
        return s < kMaxSplits ? s : kMaxSplits;
    }
    return auto_splits(B, H, T);
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
    const uintptr_t align = (uintptr_t)c->payload | (uintptr_t)(c->meta ? c->meta : c->payload);
    RESKV_REQUIRE((align & 15u) == 0, "%s: payload and metadata must be 16-byte aligned", name);
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

template <int G, int KF, int VF, bool TAB>
int launch_gt(dim3 grid, size_t shm, hipStream_t st, const DParams& p) {
    if (shm > 65536 &&
        hipFuncSetAttribute((const void*)decode_partial_kernel<G, KF, VF, TAB>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return reskv_host::check_launch("decode LDS attribute");
    hipLaunchKernelGGL((decode_partial_kernel<G, KF, VF, TAB>), grid, dim3(kThreads), shm, st, p);
    return reskv_host::check_launch("decode_partial_kernel");
}

template <int G, int KF, int VF>
int launch_g(dim3 grid, size_t shm, hipStream_t st, const DParams& p) {
    return p.rope ? launch_gt<G, KF, VF, true>(grid, shm, st, p) : launch_gt<G, KF, VF, false>(grid, shm, st, p);
}

template <int KF, int VF>
int launch_fmt(int G, dim3 grid, size_t shm, hipStream_t st, const DParams& p) {
    switch (G) {
    case 1: return launch_g<1, KF, VF>(grid, shm, st, p);
    case 2: return launch_g<2, KF, VF>(grid, shm, st, p);
    case 4: return launch_g<4, KF, VF>(grid, shm, st, p);
    default: return launch_g<8, KF, VF>(grid, shm, st, p);
    }
}

int launch_partial(int kf, int vf, int G, dim3 grid, size_t shm, hipStream_t st, const DParams& p) {
    if (kf == vf) {
        switch (kf) {
        case D_BITMAP: return launch_fmt<D_BITMAP, D_BITMAP>(G, grid, shm, st, p);
        case D_TILED: return launch_fmt<D_TILED, D_TILED>(G, grid, shm, st, p);
        case D_STRUCT16: return launch_fmt<D_STRUCT16, D_STRUCT16>(G, grid, shm, st, p);
        case D_SINT4: return launch_fmt<D_SINT4, D_SINT4>(G, grid, shm, st, p);
        case D_Q4: return launch_fmt<D_Q4, D_Q4>(G, grid, shm, st, p);
        case D_Q2: return launch_fmt<D_Q2, D_Q2>(G, grid, shm, st, p);
        case D_BITMAP_W: return launch_fmt<D_BITMAP_W, D_BITMAP_W>(G, grid, shm, st, p);
        case D_TILED_W: return launch_fmt<D_TILED_W, D_TILED_W>(G, grid, shm, st, p);
        default: return launch_fmt<D_DENSE, D_DENSE>(G, grid, shm, st, p);
        }
    }
    if (kf == D_Q4 && vf == D_Q2) return launch_fmt<D_Q4, D_Q2>(G, grid, shm, st, p);
    if (kf == D_Q2 && vf == D_Q4) return launch_fmt<D_Q2, D_Q4>(G, grid, shm, st, p);
    RESKV_REQUIRE(false, "K and V residual formats must match (INT4/INT2 may mix)");
    return 1;
}

int run_decode(const void* q, int kf, const DTensor& k, int vf, const DTensor& v, const float* inv_freq,
               const float* rope, int B, int Hq, int H, int T, int start_pos, int pos_q, float scaling, int splits,
               void* out, float* m, float* l, void* ws, int64_t ws_bytes, void* stream) {
    RESKV_REQUIRE(q && inv_freq && out, "null pointer argument");
    RESKV_REQUIRE(B > 0 && H > 0 && T > 0, "batch, head and token counts must be positive");
    RESKV_REQUIRE(Hq % H == 0, "query heads must be a multiple of KV heads");
    const int G = Hq / H;
    RESKV_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "supported GQA ratios are 1, 2, 4 and 8");
    const int S = resolve_splits(B, H, T, splits);
    RESKV_REQUIRE(ws != nullptr && ws_bytes >= workspace_for(B, Hq, S), "decode workspace too small");
    RESKV_REQUIRE(((uintptr_t)inv_freq & 15u) == 0, "inv_freq must be 16-byte aligned");
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
    p.stage_k = stage_bytes_rt(kf, k.pb);
    p.stage_v = stage_bytes_rt(vf, v.pb);
    const bool cent = kf != D_DENSE;
    const int merge_bytes = kWaves * G * kPartStride * 4;
    const int cent_bytes = cent ? k.nc * kDim * 4 : 0;
    const int region0 = cent_bytes > merge_bytes ? cent_bytes : merge_bytes;
    p.beta_off = region0;
    p.lut_off = p.beta_off + (cent ? kWaves * G * kMaxClusters * 4 : 0);
    p.p_off = p.lut_off + kLutWords * 4;
    p.stage_off = p.p_off + kWaves * (kSteps * G * kRows + kTile * kVPitch) * 2;
    const size_t shm = (size_t)p.stage_off + (size_t)kWaves * (p.stage_k + p.stage_v);
    RESKV_REQUIRE(shm <= 160 * 1024, "decode LDS requirement %zu exceeds 160 KiB", shm);
    p.pm = (float*)ws;
    p.pl = p.pm + (long)B * Hq * S;
    p.pd = p.pl + (long)B * Hq * S;
    p.pb = p.pd + (long)B * Hq * S * kDim;
    hipStream_t st = (hipStream_t)stream;
    if (launch_partial(kf, vf, G, dim3(S, H, B), shm, st, p)) return 1;
    hipLaunchKernelGGL(decode_merge_kernel, dim3(B * Hq), dim3(kMergeThreads), 0, st, p.pm, p.pl, p.pd, p.pb,
                       cent ? v.cent : nullptr, v.nc, v.cs, Hq, H, S, (uint16_t*)out, m, l);
    return reskv_host::check_launch("decode_merge_kernel");
}

}  // namespace

extern "C" int64_t reskv_decode_workspace_bytes(int B, int Hq, int H, int T, int splits) {
    if (B <= 0 || Hq <= 0 || H <= 0 || T <= 0) return 0;
    return workspace_for(B, Hq, resolve_splits(B, H, T, splits));
}

extern "C" int reskv_decode_splits(int B, int Hq, int H, int T, int splits) {
    (void)Hq;
    if (B <= 0 || H <= 0 || T <= 0) return 0;
    return resolve_splits(B, H, T, splits);
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

extern "C" int reskv_decode(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                            const float* inv_freq, int B, int Hq, int H, int T, int start_pos,
                            int pos_q, float scaling, int splits, void* out, float* m, float* l,
                            void* workspace, int64_t workspace_bytes, void* stream) {
    return reskv_decode_rope(q, k, v, inv_freq, nullptr, B, Hq, H, T, start_pos, pos_q, scaling, splits, out, m, l,
                             workspace, workspace_bytes, stream);
}

extern "C" int reskv_decode_dense(const void* q, const void* k, const void* v, const float* inv_freq,
                                  int B, int Hq, int H, int T, int start_pos, int pos_q, float scaling,
                                  int splits, void* out, float* m, float* l, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(k && v, "null K/V pointer");
    RESKV_REQUIRE((((uintptr_t)k | (uintptr_t)v) & 15u) == 0, "K and V must be 16-byte aligned");
    const DTensor kd{nullptr, nullptr, (const uint8_t*)k, nullptr, nullptr, 1, kDim, 2 * kDim, T, 1};
    const DTensor vd{nullptr, nullptr, (const uint8_t*)v, nullptr, nullptr, 1, kDim, 2 * kDim, T, 1};
    return run_decode(q, D_DENSE, kd, D_DENSE, vd, inv_freq, nullptr, B, Hq, H, T, start_pos, pos_q, scaling,
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
    float* row = table + (long)pos * kDim + (pair >> 2) * 8;
    row[pair & 3] = cs;
    row[4 + (pair & 3)] = sn;
}

extern "C" int reskv_rope_table(const float* inv_freq, int count, float* table, void* stream) {
    RESKV_REQUIRE(inv_freq && table, "null pointer argument");
    RESKV_REQUIRE(count > 0, "position count must be positive");
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
    hipLaunchKernelGGL(merge_recent_kernel, dim3(B * Hq), dim3(64), 0, (hipStream_t)stream,
                       (const uint16_t*)comp_out, comp_m, comp_l, scores, nullptr, nullptr,
                       (const uint16_t*)v_recent, Hq, H, Tr, 1.0f, (uint16_t*)out);
    return reskv_host::check_launch("merge_recent_kernel");
}

extern "C" int reskv_merge_recent_qk(const void* comp_out, const float* comp_m, const float* comp_l,
                                     const void* q_rope, const void* k_recent, const void* v_recent, int B,
                                     int Hq, int H, int Tr, float scaling, void* out, void* stream) {
    RESKV_REQUIRE(comp_out && comp_m && comp_l && out, "null pointer argument");
    RESKV_REQUIRE(B > 0 && H > 0 && Hq % H == 0 && Tr >= 0, "bad recent-merge sizes");
    RESKV_REQUIRE(Tr == 0 || (q_rope && k_recent && v_recent), "null recent tensors");
    hipLaunchKernelGGL(merge_recent_kernel, dim3(B * Hq), dim3(64), 0, (hipStream_t)stream,
                       (const uint16_t*)comp_out, comp_m, comp_l, nullptr, (const uint16_t*)q_rope,
                       (const uint16_t*)k_recent, (const uint16_t*)v_recent, Hq, H, Tr, scaling, (uint16_t*)out);
    return reskv_host::check_launch("merge_recent_kernel");
}
