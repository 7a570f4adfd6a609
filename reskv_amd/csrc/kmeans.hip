// Lloyd k-means over pre-RoPE K or V, one independent problem per (batch, head).
//
// Reference loop (reskv/compression.py:37-53): each iteration assigns every
// token to its nearest centre, then replaces each centre by the mean of its
// members.  K (value_mode = 0) keeps an empty cluster's previous centre and
// carries fp32 centres; V (value_mode = 1) sets an empty cluster to zero and
// rounds centres to fp16 after every update.  The returned ids come from the
// last assignment, i.e. against the centres before the final update.
//
// Centre tables (kmeans_prep_kernel, then kmeans_update_kernel every
// iteration): each fp32 centre is split into fp16 hi + lo rows, stored with
// |c|^2, padded to a multiple of 16 rows (padding rows are zero with an
// infinite norm).  They are written once per iteration, so the assignment
// workgroups load ready matrix-core operands instead of rebuilding them.
//
// Assignment (kmeans_assign_kernel): the distance GEMM S^T = C X^T runs on the
// matrix cores (v_mfma_f32_16x16x32f16).  Tokens are fp16 already and
// C X^T = C_hi X^T + C_lo X^T keeps fp32 accuracy (c_hi * x and c_lo * x are
// exact in fp32, sums are fp32).  Each lane holds one token's distances to 4
// centres per 16, so the argmin (lowest index on ties) is a scan in registers
// and two lane swaps across the four lanes sharing the token.  The distance
// follows the rule the reference applies to the tensor:
//   K (compression.py:38, fp32 cdist): |c|^2 - 2 <x, c> in fp32 (|x|^2 is
//     common to a token);
//   V, Lloyd (compression.py:27, 38, fp16 cdist in the mm formulation):
//     fp16(|x|^2_h + |c|^2_h - 2 <x, c>), clamped at zero, square-rooted to
//     fp16; |.|^2_h is the fp16 sum of fp16-rounded squares;
//   V, decode groups (compression.py:61-64):
//     fp16(|x|^2_h + |c|^2_h) - 2 <x, c> in fp32.  Member sums are a second matrix-core
// product, onehot(ids)^T X, whose X operand comes from the wave's 16-token tile
// through LDS transpose reads; the member counts are the same product against
// an all-ones operand.  One-hot entries and tokens are exact in fp16 and the
// products accumulate in fp32.  The waves of a chunk write their sums to
// separate LDS regions that are added in a fixed order, so sums, counts and
// centres are deterministic.
// Update (kmeans_update_kernel): one workgroup per (cluster, problem) reduces
// the chunk partials in a fixed order, writes the new centre and its tables.
#include "common.h"
#include "../../include/reskv_hip.h"

using namespace reskv;

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

constexpr int kWaves = 8;
constexpr int kRegions = 4;  // LDS sum regions: waves w and w + 4 share region w
constexpr int kThreads = kWaves * kWave;
constexpr int kSub = 16;           // tokens per MFMA sub-tile
constexpr int kChunk = 256;        // tokens per assignment workgroup (two sub-tiles per wave)
constexpr int kCUs = 256;          // compute units of an MI355X
constexpr int kXPitch = kDim + 8;  // halves per staged token row (16-byte aligned rows)
constexpr int kRPitch = kDim + 4;  // floats per cluster row of a wave's sum region; column kDim is the count

template <int NB>
constexpr int region_floats() { return NB * 16 * kRPitch; }
template <int NB>
constexpr int smem_bytes() {
    const int loop = kWaves * kSub * kXPitch * 2 + (NB > 2 ? 2 * NB * 16 * kDim * 2 : 0);
    const int reduce = kRegions * region_floats<NB>() * 4;
    return loop > reduce ? loop : reduce;
}

__device__ __forceinline__ half8_t as_h8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

// (distance, index) minimum with the lower index winning ties
__device__ __forceinline__ void argmin_step(float& d, int& i, float od, int oi) {
    const bool take = od < d || (od == d && oi < i);
    d = take ? od : d;
    i = take ? oi : i;
}

// Tables are kept in matrix-core operand order: the 16 x 32 block (centres
// 16 nb + col, channels 32 q + 8 grp + [0, 8)) that lane 16 grp + col of the
// assignment needs for piece q of centre block nb sits at 16-byte slot
// (4 nb + q) * 64 + 16 grp + col, so each operand load is 1 KB contiguous.
__device__ __forceinline__ int operand_slot_half(int c, int d) {
    return (((c >> 4) * 4 + (d >> 5)) * 64 + ((d >> 3) & 3) * 16 + (c & 15)) * 8 + (d & 7);
}

// Centre c of one problem's tables from the fp32 centre v held by threads
// 0..127 (channel = thread).  Every thread of the workgroup calls it (it holds
// a barrier); threads >= 128 pass active = false.  K rows carry an fp16 lo
// part and the fp32 |c|^2; V rows (fp16 centres) carry the fp16 norm of the
// reference's cdist, the fp16 sum of fp16-rounded squares.
__device__ __forceinline__ void store_tables(float v, bool active, bool pad, bool value, int c,
                                             uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                             float* __restrict__ norm, float* s_w) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
    if (active) {
        const uint16_t hb = f2h(v);
        const int o = operand_slot_half(c, t);
        hi[o] = hb;
        lo[o] = value ? (uint16_t)0 : f2h(v - h2f(hb));
        const float sq = value ? h2f(f2h(v * v)) : v * v;  // V: v is fp16, v*v exact in fp32
        const float w = wave_sum(sq);
        if ((t & 63) == 0) s_w[t >> 6] = w;
    }
    __syncthreads();
    if (t == 0) *norm = pad ? INFINITY : (value ? h2f(f2h(s_w[0] + s_w[1])) : s_w[0] + s_w[1]);
}

// Where the problems live: problems [0, split) are rows of tensor 0 and
// [split, BH) rows of tensor 1 (a layer's K and V clustered in one pass);
// problems >= vfrom follow the V rules (fp16 centres, empty -> 0, no lo part).
struct Problems {
    const uint16_t* x[2];  // tokens fp16 [problems, T, 128]
    int32_t* ids[2];       // ids int32 [problems, T]
    uint16_t* out[2];      // final centres fp16 [problems, C, 128]
    int split, vfrom;
    int vgroup;            // V problems assign by the decode-group rule instead of Lloyd's
};
__device__ __forceinline__ int side_of(const Problems& P, long bh) { return bh >= P.split ? 1 : 0; }

// One workgroup (128 threads) per (padded centre row, problem).
__global__ void __launch_bounds__(kDim) kmeans_prep_kernel(const float* __restrict__ centers, uint16_t* __restrict__ thi,
                                                           uint16_t* __restrict__ tlo, float* __restrict__ tnorm, int C,
                                                           int Cp, int vfrom) {
    __shared__ float s_w[2];
    const int c = blockIdx.x;
    const long bh = blockIdx.y;
    const bool pad = c >= C;
    const float v = pad ? 0.0f : centers[(bh * C + c) * kDim + threadIdx.x];
    const long head = bh * Cp * kDim;
    store_tables(v, true, pad, bh >= vfrom, c, thi + head, tlo + head, tnorm + bh * Cp + c, s_w);
}

// Row indices of the initial centres (at most kMaxClusters), passed by value.
struct InitRows {
    int idx[kMaxClusters];
};

// As kmeans_prep_kernel, with the initial centre c of problem bh taken from
// token idx[c] of that problem's rows (fp16, exact in fp32), also written to
// the fp32 centre array.
__global__ void __launch_bounds__(kDim) kmeans_prep_rows_kernel(Problems P, InitRows ir, float* __restrict__ centers,
                                                                uint16_t* __restrict__ thi, uint16_t* __restrict__ tlo,
                                                                float* __restrict__ tnorm, int T, int C, int Cp) {
    __shared__ float s_w[2];
    const int c = blockIdx.x;
    const long bh = blockIdx.y;
    const bool pad = c >= C;
    const int side = side_of(P, bh);
    const long pb = bh - (side ? P.split : 0);
    float v = 0.0f;
    if (!pad) {
        v = h2f(P.x[side][(pb * T + ir.idx[c]) * kDim + threadIdx.x]);
        centers[(bh * C + c) * kDim + threadIdx.x] = v;
    }
    const long head = bh * Cp * kDim;
    store_tables(v, true, pad, bh >= P.vfrom, c, thi + head, tlo + head, tnorm + bh * Cp + c, s_w);
}

// |c|^2 of centre r of a lane's four
__device__ __forceinline__ float cnorm(float4 n, int r) { return r == 0 ? n.x : r == 1 ? n.y : r == 2 ? n.z : n.w; }

// (distance, index) minimum over the four lanes holding one token (lanes
// col + 16 g): every lane ends with the token's nearest centre.
__device__ __forceinline__ void token_argmin(float& bd, int& bi) {
    const auto pd = __builtin_amdgcn_permlane32_swap((uint32_t)f2i(bd), (uint32_t)f2i(bd), false, false);
    const auto pi = __builtin_amdgcn_permlane32_swap((uint32_t)bi, (uint32_t)bi, false, false);
    bd = i2f((int)pd[0]);
    bi = (int)pi[0];
    argmin_step(bd, bi, i2f((int)pd[1]), (int)pi[1]);
    const auto qd = __builtin_amdgcn_permlane16_swap((uint32_t)f2i(bd), (uint32_t)f2i(bd), false, false);
    const auto qi = __builtin_amdgcn_permlane16_swap((uint32_t)bi, (uint32_t)bi, false, false);
    bd = i2f((int)qd[0]);
    bi = (int)qi[0];
    argmin_step(bd, bi, i2f((int)qd[1]), (int)qi[1]);
}
__device__ __forceinline__ float token_min(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap((uint32_t)f2i(v), (uint32_t)f2i(v), false, false);
    v = fminf(i2f((int)a[0]), i2f((int)a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap((uint32_t)f2i(v), (uint32_t)f2i(v), false, false);
    return fminf(i2f((int)b[0]), i2f((int)b[1]));
}
__device__ __forceinline__ int token_min_index(int v) {
    const auto a = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    v = min((int)a[0], (int)a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    return min((int)b[0], (int)b[1]);
}

// fp16 norm of a token as the reference's fp16 cdist forms it: each square
// rounded to fp16, summed in fp32 (this lane's 32 channels, then the four lanes
// of the token; the pairwise sums are commutative, so all four lanes agree),
// rounded to fp16.
__device__ __forceinline__ float token_half_norm(const uint4* xq) {
#pragma clang fp contract(off)
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t w[4] = {xq[q].x, xq[q].y, xq[q].z, xq[q].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = h2f((uint16_t)(w[j] & 0xFFFFu)), b = h2f((uint16_t)(w[j] >> 16));
            acc += h2f(f2h(a * a));  // a * a is exact in fp32; one rounding to fp16
            acc += h2f(f2h(b * b));
        }
    }
    const auto p = __builtin_amdgcn_permlane32_swap((uint32_t)f2i(acc), (uint32_t)f2i(acc), false, false);
    acc = i2f((int)p[0]) + i2f((int)p[1]);
    const auto q = __builtin_amdgcn_permlane16_swap((uint32_t)f2i(acc), (uint32_t)f2i(acc), false, false);
    acc = i2f((int)q[0]) + i2f((int)q[1]);
    return h2f(f2h(acc));
}

// For a non-negative fp16 value d (as float): M^2, with M the midpoint between
// the correctly rounded fp16 square root of d and the next fp16 value above
// it.  An fp16 value e has the same fp16 root as d exactly when d <= e < M^2
// (a root is never exactly a midpoint; M has 12 significant bits, so M^2 is
// exact in fp32).  The hardware root is within one fp16 step after rounding
// and is corrected against the midpoints on both sides.
__device__ __forceinline__ float root_bound_sq(float d) {
#pragma clang fp contract(off)
    const uint16_t sb = f2h(__builtin_sqrtf(d));
    float sv = h2f(sb);
    const float up = h2f((uint16_t)(sb + 1)), dn = sb ? h2f((uint16_t)(sb - 1)) : 0.0f;
    const float mhi = 0.5f * (sv + up), mlo = 0.5f * (sv + dn);
    uint16_t rb = sb;
    if (mhi * mhi < d) rb = (uint16_t)(sb + 1);
    else if (sb && mlo * mlo > d) rb = (uint16_t)(sb - 1);
    if (rb >= 0x7C00u) return INFINITY;  // root is infinite: only d itself qualifies
    sv = h2f(rb);
    const float m = 0.5f * (sv + h2f((uint16_t)(rb + 1)));
    return m * m;
}

// One workgroup: tokens [chunk * kChunk, +kChunk) of problem bh; wave w takes
// sub-tiles w and w + 8 of the chunk, loaded together at the start.
// thi/tlo fp16 [BH, 16 NB, 128] and tnorm fp32 [BH, 16 NB] are the centre
// tables; psum fp32 [BH, chunks, C, 128] and pcnt int [BH, chunks, C] (skipped
// when psum is null).  LO: some problem has fp32 centres (lo tables of the
// others are zero).  REGB: centre operands held in registers (one workgroup per
// CU); otherwise read from LDS, which frees the registers for two workgroups
// per CU (four waves per SIMD: at most 128 VGPRs, requested from the compiler
// with waves_per_eu) when the grid has more workgroups than CUs.  At three
// waves per SIMD only one 8-wave workgroup fits and K+V together at 512
// workgroups took 290 us instead of 245 us.
template <int NB, bool LO, bool REGB>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(REGB ? 1 : 4)))
kmeans_assign_kernel(
    Problems P, const uint16_t* __restrict__ thi, const uint16_t* __restrict__ tlo, const float* __restrict__ tnorm,
    float* __restrict__ psum, int* __restrict__ pcnt, int T, int C, int chunks) {
    constexpr int CP = NB * 16;
    constexpr int SPW = kChunk / (kWaves * kSub);  // sub-tiles per wave
    constexpr bool kRegB = REGB && NB <= 2;
    __shared__ __align__(16) unsigned char smem[smem_bytes<NB>()];
    const int chunk = blockIdx.x;
    const long bh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;  // MFMA lane coordinates
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem) + wave * kSub * kXPitch;
    const int side = side_of(P, bh);
    const long pb = bh - (side ? P.split : 0);
    const uint16_t* __restrict__ x = P.x[side] + pb * T * kDim;
    int32_t* __restrict__ ids = P.ids[side] + pb * T;
    const bool vrule = bh >= P.vfrom;  // workgroup-uniform
    const bool vgroup = P.vgroup != 0;

    // token operand: lane (col, grp) holds token t0 + col, channels 32 q + 8 grp +
    // [0, 8) for piece q, so the four lanes of a token read 64 contiguous bytes;
    // rows past T repeat token t0 (their one-hot entries are 0)
    uint4 xr[SPW][4];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        const int t0 = chunk * kChunk + (wave + kWaves * s) * kSub;
        if (t0 < T) {
            const int tok = t0 + col < T ? t0 + col : t0;
            const uint4* src = reinterpret_cast<const uint4*>(x + (long)tok * kDim + 8 * grp);
#pragma unroll
            for (int q = 0; q < 4; ++q) xr[s][q] = src[4 * q];
        }
    }

    // centre operand: lane (col, grp) holds centre nb*16 + col at the same
    // channels, one contiguous 1 KB wave load per piece (operand-order tables)
    const uint4* ghi = reinterpret_cast<const uint4*>(thi + bh * CP * kDim);
    const uint4* glo = reinterpret_cast<const uint4*>(tlo + bh * CP * kDim);
    uint4 bhi[kRegB ? NB : 1][4], blo[kRegB && LO ? NB : 1][4];
    uint4* sbh = reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(smem) + kWaves * kSub * kXPitch);
    uint4* sbl = sbh + CP * kDim / 8;
    if constexpr (kRegB) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                bhi[nb][q] = ghi[(nb * 4 + q) * 64 + lane];
                if constexpr (LO) blo[nb][q] = glo[(nb * 4 + q) * 64 + lane];
            }
    } else {
        for (int i = tid; i < CP * kDim / 8; i += kThreads) {
            sbh[i] = ghi[i];
            if constexpr (LO) sbl[i] = glo[i];
        }
        __syncthreads();
    }
    auto b_hi = [&](int nb, int q) -> uint4 {
        if constexpr (kRegB) return bhi[nb][q];
        else return sbh[(nb * 4 + q) * 64 + lane];
    };
    auto b_lo = [&](int nb, int q) -> uint4 {
        if constexpr (kRegB) return blo[LO ? nb : 0][q];
        else return sbl[(nb * 4 + q) * 64 + lane];
    };
    // |c|^2 of the centres nb*16 + 4*grp + r whose distances this lane holds
    float4 cn[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) cn[nb] = *reinterpret_cast<const float4*>(tnorm + bh * CP + nb * 16 + 4 * grp);

    float4_t sums[NB][8];  // onehot^T X: rows nb*16 + 4*grp + r, channels db*16 + col
    float4_t cnt[NB];      // onehot^T 1: member counts of rows nb*16 + 4*grp + r
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        cnt[nb] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int db = 0; db < 8; ++db) sums[nb][db] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
    }
    const half4_t ones = (half4_t){(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
    // transpose reads: lane i of 16-lane row g points at token 4g + i/4, channel
    // 16*db + 4*(i%4) and receives tokens 4g + r, channel 16*db + i (r = 0..3)
    const uint16_t* xt = xs + (4 * grp + (col >> 2)) * kXPitch + 4 * (col & 3);

#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        const int t0 = chunk * kChunk + (wave + kWaves * s) * kSub;
        if (t0 >= T) break;
        // S^T = C X^T: lane (col, grp) gets <c, x> for token t0 + col and
        // centres nb*16 + 4*grp + r
        float4_t acc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            acc[nb] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(b_hi(nb, q)), as_h8(xr[s][q]), acc[nb], 0, 0, 0);
                if constexpr (LO)
                    acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(b_lo(nb, q)), as_h8(xr[s][q]), acc[nb], 0, 0, 0);
            }
        }
        int bi;
        if (!vrule) {
            // K: nearest of this lane's centres, scanned in increasing index
            // order (a strict < keeps the lower index on ties), then across the
            // four row groups holding the same token
            float bd = fmaf(-2.0f, acc[0][0], cn[0].x);
            bi = 4 * grp;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (nb == 0 && r == 0) continue;
                    const float d = fmaf(-2.0f, acc[nb][r], cnorm(cn[nb], r));
                    const bool take = d < bd;
                    bd = take ? d : bd;
                    bi = take ? nb * 16 + 4 * grp + r : bi;
                }
            token_argmin(bd, bi);
        } else {
            const float xn = token_half_norm(xr[s]);
            if (vgroup) {
                // decode groups: fp32(fp16(|x|^2 + |c|^2) - 2 <x, c>), lowest index on ties
                float bd = INFINITY;
                bi = 1 << 20;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float e = h2f(f2h(xn + cnorm(cn[nb], r)));
                        const float d = fmaf(-2.0f, acc[nb][r], e);
                        const bool take = d < bd;
                        bd = take ? d : bd;
                        bi = take ? nb * 16 + 4 * grp + r : bi;
                    }
                token_argmin(bd, bi);
            } else {
                // Lloyd: fp16 cdist.  The winner is the lowest index whose fp16
                // root equals the smallest one: with dmin the smallest fp16
                // squared distance and M the midpoint above its fp16 root,
                // that is every d < M^2 (M^2 is exact in fp32), or d == dmin
                // when the root is infinite.
                float d16[NB][4];
                float dmin = INFINITY;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float d = fmaf(-2.0f, acc[nb][r], xn + cnorm(cn[nb], r));
                        d16[nb][r] = fmaxf(h2f(f2h(d)), 0.0f);
                        dmin = fminf(dmin, d16[nb][r]);
                    }
                dmin = token_min(dmin);
                const float thr = root_bound_sq(dmin);
                bi = 1 << 20;
#pragma unroll
                for (int nb = NB - 1; nb >= 0; --nb)
#pragma unroll
                    for (int r = 3; r >= 0; --r)
                        if (d16[nb][r] < thr || d16[nb][r] == dmin) bi = nb * 16 + 4 * grp + r;
                bi = token_min_index(bi);
            }
        }
        // every lane of column col now holds the id of token t0 + col
        if (grp == 0 && t0 + col < T) ids[t0 + col] = bi;
        if (psum != nullptr) {
            // stage the tile: lane (col, grp) writes token col's channels 32 q + 8 grp + [0, 8)
            uint4* row = reinterpret_cast<uint4*>(xs + col * kXPitch + 8 * grp);
#pragma unroll
            for (int q = 0; q < 4; ++q) row[4 * q] = xr[s][q];
            // A = onehot^T: lane (col, grp) holds [cluster nb*16 + col][tokens 4*grp + i],
            // the tokens' ids fetched from the lanes of row 0 that hold them
            int tid4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) tid4[i] = __builtin_amdgcn_ds_bpermute((4 * grp + i) * 4, bi);
            half4_t oh[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool in = (t0 + 4 * grp + i < T) && tid4[i] == nb * 16 + col;
                    oh[nb][i] = in ? (_Float16)1.0f : (_Float16)0.0f;
                }
            }
            wave_sync();
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const half4_t xb = __builtin_bit_cast(
                    half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(xt + 16 * db)));
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    sums[nb][db] = __builtin_amdgcn_mfma_f32_16x16x16f16(oh[nb], xb, sums[nb][db], 0, 0, 0);
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) cnt[nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(oh[nb], ones, cnt[nb], 0, 0, 0);
            wave_sync();  // tile reads done before the next tile is staged
        }
    }
    if (psum == nullptr) return;
    // waves 4..7 write regions 0..3 (the regions reuse the tiles' LDS), waves
    // 0..3 add theirs, then the regions are added in order: a fixed association
    __syncthreads();
    float* reg = reinterpret_cast<float*>(smem) + (wave & (kRegions - 1)) * region_floats<NB>();
    auto region_pass = [&](bool add) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float* dst = reg + (nb * 16 + 4 * grp + r) * kRPitch;
#pragma unroll
                for (int db = 0; db < 8; ++db) dst[db * 16 + col] = (add ? dst[db * 16 + col] : 0.0f) + sums[nb][db][r];
                if (col == 0) dst[kDim] = (add ? dst[kDim] : 0.0f) + cnt[nb][r];
            }
    };
    if (wave >= kRegions) region_pass(false);
    __syncthreads();
    if (wave < kRegions) region_pass(true);
    __syncthreads();
    const float* r0 = reinterpret_cast<const float*>(smem);
    float* ps = psum + ((bh * chunks) + chunk) * (long)C * kDim;
    for (int i = tid; i < C * kDim / 4; i += kThreads) {
        const int o = (i >> 5) * kRPitch + (i & 31) * 4;
        float4 s = *reinterpret_cast<const float4*>(r0 + o);
#pragma unroll
        for (int w = 1; w < kRegions; ++w) {
            const float4 v = *reinterpret_cast<const float4*>(r0 + w * region_floats<NB>() + o);
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        *reinterpret_cast<float4*>(ps + (long)i * 4) = s;
    }
    if (tid < C) {
        float n = r0[tid * kRPitch + kDim];
#pragma unroll
        for (int w = 1; w < kRegions; ++w) n += r0[w * region_floats<NB>() + tid * kRPitch + kDim];
        pcnt[(bh * chunks + chunk) * C + tid] = (int)n;
    }
}

// One workgroup (512 threads: channel x chunk residue mod 4) per (cluster,
// problem); the four parts of the chunk sum meet in LDS and are added in a
// fixed order.  Writes the centre, then either its tables for the next
// assignment (thi non-null) or the fp16 result (thi null).
constexpr int kParts = 4;
__global__ void __launch_bounds__(kParts * kDim) kmeans_update_kernel(
    Problems P, float* __restrict__ centers, const float* __restrict__ psum, const int* __restrict__ pcnt, int C,
    int Cp, int chunks, uint16_t* __restrict__ thi, uint16_t* __restrict__ tlo, float* __restrict__ tnorm) {
    __shared__ float s_part[kParts][kDim];
    __shared__ int s_n[kParts];
    __shared__ float s_w[2];
    const int c = blockIdx.x;
    const long bh = blockIdx.y;
    const int d = threadIdx.x & (kDim - 1), par = threadIdx.x >> 7;
    float s = 0.0f;
    int n = 0;
    const float* src = psum + (bh * chunks) * (long)C * kDim + c * kDim + d;
    const int* cnt = pcnt + bh * chunks * C + c;
#pragma unroll 16
    for (int k = par; k < chunks; k += kParts) {
        s += src[(long)k * C * kDim];
        n += cnt[k * C];
    }
    s_part[par][d] = s;
    if (d == 0) s_n[par] = n;
    __syncthreads();
    s = ((s_part[0][d] + s_part[1][d]) + s_part[2][d]) + s_part[3][d];
    n = s_n[0] + s_n[1] + s_n[2] + s_n[3];
    const bool value_mode = bh >= P.vfrom;
    float nv = 0.0f;
    if (par == 0) {
        float* cv = centers + (bh * C + c) * kDim + d;
        if (value_mode) {
            nv = n > 0 ? h2f(f2h(s / (float)n)) : 0.0f;  // fp16 centres, empty -> 0
        } else {
            nv = n > 0 ? s / (float)n : *cv;             // fp32 centres, empty keeps
        }
        *cv = nv;
        if (thi == nullptr) {
            const int side = side_of(P, bh);
            P.out[side][((bh - (side ? P.split : 0)) * C + c) * kDim + d] = f2h(nv);
        }
    }
    if (thi == nullptr) return;  // uniform over the workgroup
    const long head = bh * Cp * kDim;
    store_tables(nv, par == 0, false, value_mode, c, thi + head, tlo + head, tnorm + bh * Cp + c, s_w);
}

// Workspace: fp32 centres, the fp16 hi/lo tables and norms, chunk partials;
// every array starts on a 256-byte boundary.
struct Layout {
    int Cp, chunks;
    int64_t centers, thi, tlo, tnorm, psum, pcnt, total;
};
Layout layout(int BH, int T, int C) {
    Layout L;
    L.Cp = (C + 15) / 16 * 16;
    L.chunks = (T + kChunk - 1) / kChunk;
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        const int64_t at = off;
        off += (bytes + 255) & ~(int64_t)255;
        return at;
    };
    L.centers = take((int64_t)BH * C * kDim * 4);
    L.thi = take((int64_t)BH * L.Cp * kDim * 2);
    L.tlo = take((int64_t)BH * L.Cp * kDim * 2);
    L.tnorm = take((int64_t)BH * L.Cp * 4);
    L.psum = take((int64_t)BH * L.chunks * C * kDim * 4);
    L.pcnt = take((int64_t)BH * L.chunks * C * 4);
    L.total = off;
    return L;
}

struct Tables {
    uint16_t* hi;
    uint16_t* lo;
    float* norm;
};

template <int NB, bool REGB>
void launch_nb(bool lo, dim3 grid, hipStream_t st, const Problems& P, const Tables& tb, float* psum, int* pcnt, int T,
               int C, int chunks) {
    if (lo)
        hipLaunchKernelGGL((kmeans_assign_kernel<NB, true, REGB>), grid, dim3(kThreads), 0, st, P, tb.hi, tb.lo,
                           tb.norm, psum, pcnt, T, C, chunks);
    else
        hipLaunchKernelGGL((kmeans_assign_kernel<NB, false, REGB>), grid, dim3(kThreads), 0, st, P, tb.hi, tb.lo,
                           tb.norm, psum, pcnt, T, C, chunks);
}

int launch_assign(const Problems& P, const Tables& tb, float* psum, int* pcnt, int BH, int T, int C, const Layout& L,
                  hipStream_t st) {
    const dim3 grid(L.chunks, BH);
    const bool lo = P.vfrom > 0;
    const bool regb = (int64_t)L.chunks * BH <= kCUs;  // one workgroup per CU: registers; more: LDS operands
    switch (L.Cp / 16) {
    case 1:
        if (regb) launch_nb<1, true>(lo, grid, st, P, tb, psum, pcnt, T, C, L.chunks);
        else launch_nb<1, false>(lo, grid, st, P, tb, psum, pcnt, T, C, L.chunks);
        break;
    case 2:
        if (regb) launch_nb<2, true>(lo, grid, st, P, tb, psum, pcnt, T, C, L.chunks);
        else launch_nb<2, false>(lo, grid, st, P, tb, psum, pcnt, T, C, L.chunks);
        break;
    case 3: launch_nb<3, false>(lo, grid, st, P, tb, psum, pcnt, T, C, L.chunks); break;
    default: launch_nb<4, false>(lo, grid, st, P, tb, psum, pcnt, T, C, L.chunks); break;
    }
    return reskv_host::check_launch("kmeans_assign_kernel");
}

int launch_prep(const float* centers, const Tables& tb, int BH, int C, int Cp, int vfrom, hipStream_t st) {
    hipLaunchKernelGGL(kmeans_prep_kernel, dim3(Cp, BH), dim3(kDim), 0, st, centers, tb.hi, tb.lo, tb.norm, C, Cp,
                       vfrom);
    return reskv_host::check_launch("kmeans_prep_kernel");
}

Tables tables_of(void* workspace, const Layout& L) {
    char* w = (char*)workspace;
    return Tables{(uint16_t*)(w + L.thi), (uint16_t*)(w + L.tlo), (float*)(w + L.tnorm)};
}

int check_pointers(const void* x, const void* workspace) {
    RESKV_REQUIRE(((uintptr_t)x & 15u) == 0, "token rows must be 16-byte aligned");
    RESKV_REQUIRE(((uintptr_t)workspace & 255u) == 0, "k-means workspace must be 256-byte aligned");
    return 0;
}

// torch.linspace(0, T - 1, C).long() (reskv/compression.py:35) as torch
// evaluates it in fp32: step = fl32((T - 1) / (C - 1)); index i < C / 2 is
// fl32(i * step), the others fl32((T - 1) - (C - 1 - i) * step) (one rounding
// of the exact value, as torch's fused form), truncated toward zero.
void linspace_rows(int T, int C, int* idx) {
    if (C == 1) {
        idx[0] = 0;
        return;
    }
    const float end = (float)(T - 1);
    const float step = end / (float)(C - 1);
    for (int i = 0; i < C; ++i) {
        const float v = i < C / 2 ? (float)i * step : fmaf(-(float)(C - 1 - i), step, end);
        idx[i] = (int)v;
    }
}

// Lloyd iterations over BH problems; init[side] holds the initial fp32
// centres of the problems in tensor `side`, or both are null: the tokens at
// linspace(0, T - 1, C) of each problem (T >= C).
int run_kmeans(const Problems& P, const float* const init[2], int BH, int T, int C, int iterations, void* workspace,
               hipStream_t st) {
    const Layout L = layout(BH, T, C);
    const Tables tb = tables_of(workspace, L);
    char* w = (char*)workspace;
    float* centers = (float*)(w + L.centers);
    float* psum = (float*)(w + L.psum);
    int* pcnt = (int*)(w + L.pcnt);
    if (init[0] == nullptr && init[1] == nullptr) {
        InitRows ir{};
        linspace_rows(T, C, ir.idx);
        hipLaunchKernelGGL(kmeans_prep_rows_kernel, dim3(L.Cp, BH), dim3(kDim), 0, st, P, ir, centers, tb.hi, tb.lo,
                           tb.norm, T, C, L.Cp);
        if (reskv_host::check_launch("kmeans_prep_rows_kernel")) return 1;
    } else {
        const size_t row = (size_t)C * kDim * sizeof(float);
        for (int side = 0; side < 2; ++side) {
            const int n = side ? BH - P.split : P.split;
            if (n > 0 && hipMemcpyAsync(centers + (side ? (size_t)P.split * C * kDim : 0), init[side], n * row,
                                        hipMemcpyDeviceToDevice, st) != hipSuccess)
                return reskv_host::check_launch("kmeans centre copy");
        }
        if (launch_prep(centers, tb, BH, C, L.Cp, P.vfrom, st)) return 1;
    }
    for (int it = 0; it < iterations; ++it) {
        if (launch_assign(P, tb, psum, pcnt, BH, T, C, L, st)) return 1;
        const bool last = it == iterations - 1;
        hipLaunchKernelGGL(kmeans_update_kernel, dim3(C, BH), dim3(kParts * kDim), 0, st, P, centers, psum, pcnt, C,
                           L.Cp, L.chunks, last ? nullptr : tb.hi, tb.lo, tb.norm);
        if (reskv_host::check_launch("kmeans_update_kernel")) return 1;
    }
    return 0;
}

}  // namespace

extern "C" int64_t reskv_kmeans_workspace_bytes(int BH, int T, int C) {
    if (BH <= 0 || T <= 0 || C <= 0) return 0;
    return layout(BH, T, C).total;
}

extern "C" int reskv_kmeans_assign(const void* x, const float* centers, int32_t* ids, int BH, int T, int C,
                                   int value_mode, void* workspace, int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(x && centers && ids, "null pointer argument");
    RESKV_REQUIRE(BH > 0 && T > 0, "problem sizes must be positive");
    RESKV_REQUIRE(C >= 1 && C <= kMaxClusters, "centroid count must be in [1, 64]");
    RESKV_REQUIRE(value_mode == 0 || value_mode == 1, "value_mode must be 0 (K) or 1 (V)");
    RESKV_REQUIRE(workspace && workspace_bytes >= reskv_kmeans_workspace_bytes(BH, T, C),
                  "k-means workspace too small");
    if (check_pointers(x, workspace)) return 1;
    const Layout L = layout(BH, T, C);
    const Tables tb = tables_of(workspace, L);
    const int vfrom = value_mode ? 0 : BH;
    const Problems P{{(const uint16_t*)x, (const uint16_t*)x}, {ids, ids}, {nullptr, nullptr}, BH, vfrom, 1};
    hipStream_t st = (hipStream_t)stream;
    if (launch_prep(centers, tb, BH, C, L.Cp, vfrom, st)) return 1;
    return launch_assign(P, tb, nullptr, nullptr, BH, T, C, L, st);
}

extern "C" int reskv_linspace_rows(int T, int C, int32_t* rows) {
    RESKV_REQUIRE(rows != nullptr, "null pointer argument");
    RESKV_REQUIRE(C >= 1 && C <= kMaxClusters && T >= C, "need 1 <= C <= 64 and T >= C");
    int idx[kMaxClusters];
    linspace_rows(T, C, idx);
    for (int i = 0; i < C; ++i) rows[i] = idx[i];
    return 0;
}

extern "C" int reskv_kmeans(const void* x, const float* centers_init, void* centers_out, int32_t* ids,
                            int BH, int T, int C, int iterations, int value_mode, void* workspace,
                            int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(x && centers_out && ids, "null pointer argument");
    RESKV_REQUIRE(centers_init || T >= C, "linspace initial centres need T >= C");
    RESKV_REQUIRE(BH > 0 && T > 0, "problem sizes must be positive");
    RESKV_REQUIRE(C >= 1 && C <= kMaxClusters, "centroid count must be in [1, 64]");
    RESKV_REQUIRE(iterations >= 1, "iterations must be positive");
    RESKV_REQUIRE(workspace && workspace_bytes >= reskv_kmeans_workspace_bytes(BH, T, C),
                  "k-means workspace too small");
    if (check_pointers(x, workspace)) return 1;
    const uint16_t* xh = (const uint16_t*)x;
    uint16_t* out = (uint16_t*)centers_out;
    const Problems P{{xh, xh}, {ids, ids}, {out, out}, BH, value_mode ? 0 : BH, 0};
    const float* const init[2] = {centers_init, centers_init};
    return run_kmeans(P, init, BH, T, C, iterations, workspace, (hipStream_t)stream);
}

extern "C" int reskv_kmeans_kv(const void* k, const void* v, const float* init_k, const float* init_v, void* out_k,
                               void* out_v, int32_t* ids_k, int32_t* ids_v, int BH, int T, int C, int iterations,
                               void* workspace, int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(k && v && out_k && out_v && ids_k && ids_v, "null pointer argument");
    RESKV_REQUIRE((init_k == nullptr) == (init_v == nullptr), "give both initial centre arrays or neither");
    RESKV_REQUIRE(init_k || T >= C, "linspace initial centres need T >= C");
    RESKV_REQUIRE(BH > 0 && T > 0, "problem sizes must be positive");
    RESKV_REQUIRE(C >= 1 && C <= kMaxClusters, "centroid count must be in [1, 64]");
    RESKV_REQUIRE(iterations >= 1, "iterations must be positive");
    RESKV_REQUIRE(workspace && workspace_bytes >= reskv_kmeans_workspace_bytes(2 * BH, T, C),
                  "k-means workspace too small");
    if (check_pointers(k, workspace) || check_pointers(v, workspace)) return 1;
    const Problems P{{(const uint16_t*)k, (const uint16_t*)v}, {ids_k, ids_v}, {(uint16_t*)out_k, (uint16_t*)out_v},
                     BH, BH, 0};
    const float* const init[2] = {init_k, init_v};
    return run_kmeans(P, init, 2 * BH, T, C, iterations, workspace, (hipStream_t)stream);
}
