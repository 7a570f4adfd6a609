// Split-K fused decode attention over the compressed K/V cache.
//
// Semantics (reskv/reference.py:59-91, reskv/csrc/cluster_mass.cu:4-11):
//   k_t = c_k[id_k(t)] + r_k(t)            (pre-RoPE key, fp32)
//   s_t = scaling * <rot(q, pos_q), rot(k_t, start + t)>
//   out = sum_t p_t (c_v[id_v(t)] + r_v(t)) / sum_t p_t,  p_t = exp(s_t - m)
// The Value centroids are applied once after the split reduction:
//   sum_t p_t c_v[id_v(t)] = sum_c beta_c c_v[c],  beta_c = sum_{t: id_v(t)=c} p_t.
// RoPE angles are fl32(position * inv_freq[i]) for rotate-half pairs (i, i+64),
// exactly as the reference oracle forms them.
//
// Kernel 1 (partial): one workgroup per (split, kv-head, batch).  Each wave owns
// channels {lane, lane+64} and walks tokens of its split; it keeps an online
// softmax state per query head of the GQA group: running max m, normaliser l,
// unnormalised Value-residual sum delta[128] and cluster mass beta[nc].
// Kernel 2 (merge): one wave per (batch, query head) rescales the split partials
// to a common maximum, folds sum_c beta_c c_v[c] and normalises.
#include "common.h"
#include "../../include/reskv_hip.h"

#include <math.h>

using namespace reskv;

namespace {

constexpr int kFmtDense = 5;  // internal: uncompressed fp16 rows, no centroids
constexpr int kWaves = 4;
constexpr int kMaxSplits = 256;

struct CTensor {
    const uint16_t* cent;
    const int8_t* ids;
    const void* payload;
    const void* meta;
    const uint16_t* scale;
    int nc, fmt, width, bits;
};

__device__ __forceinline__ uint64_t bitrev64(uint64_t v) {
    return ((uint64_t)__builtin_bitreverse32((uint32_t)v) << 32) | __builtin_bitreverse32((uint32_t)(v >> 32));
}

// Residual values of channels `lane` and `lane + 64` of compressed row `row`
// (row = (b * H + h) * T + t, wave-uniform).  Format decoders follow
// reskv/reference.py:12-47.
__device__ __forceinline__ void decode_residual(const CTensor& ct, long row, int lane, float& r0, float& r1) {
    r0 = 0.0f;
    r1 = 0.0f;
    switch (ct.fmt) {
    case RESKV_FMT_BITMAP: {
        // channel d <-> bit (63 - d % 64) of word d / 64; value index = rank
        const uint64_t* mw = (const uint64_t*)ct.meta + row * 2;
        const uint64_t w0 = mw[0], w1 = mw[1];
        const uint64_t v0 = bitrev64(w0), v1 = bitrev64(w1);
        const uint16_t* p = (const uint16_t*)ct.payload + row * ct.width;
        const uint32_t k0 = lanes_below(v0);
        const uint32_t k1 = (uint32_t)__builtin_popcountll(w0) + lanes_below(v1);
        if (((v0 >> lane) & 1ull) && k0 < (uint32_t)ct.width) r0 = h2f(p[k0]);
        if (((v1 >> lane) & 1ull) && k1 < (uint32_t)ct.width) r1 = h2f(p[k1]);
        break;
    }
    case RESKV_FMT_TILED:
    case RESKV_FMT_STRUCT16: {
        // word w = code(tile 2w) | code(tile 2w+1) << 16
        const uint32_t* mw = (const uint32_t*)ct.meta + row * 4;
        const uint16_t* p = (const uint16_t*)ct.payload + row * ct.width;
        const int per_tile = ct.width >> 3;
        const int bit = lane & 15;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int tile = (lane >> 4) + 4 * half;
            const uint32_t code = (mw[tile >> 1] >> (16 * (tile & 1))) & 0xFFFFu;
            int idx = -1;
            if (ct.fmt == RESKV_FMT_TILED) {
                if ((code >> bit) & 1u) idx = tile * per_tile + __builtin_popcount(code & ((1u << bit) - 1u));
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if ((int)((code >> (4 * r)) & 15u) == bit) idx = tile * 4 + r;
            }
            const float val = (idx >= 0 && idx < ct.width) ? h2f(p[idx]) : 0.0f;
            if (half == 0) r0 = val; else r1 = val;
        }
        break;
    }
    case RESKV_FMT_STRUCT_INT4: {
        const uint32_t* qp = (const uint32_t*)ct.payload + row * 4;
        const uint32_t* qm = (const uint32_t*)ct.meta + row * 2;
        const float s = h2f(ct.scale[row]);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int d = lane + 64 * half;
            const int grp = d >> 2;
            const int sel = (int)((qm[grp >> 4] >> (2 * (grp & 15))) & 3u);
            float val = 0.0f;
            if (sel == (d & 3)) {
                const int nib = (int)((qp[grp >> 3] >> (4 * (grp & 7))) & 15u);
                val = (float)((nib ^ 8) - 8) * s;
            }
            if (half == 0) r0 = val; else r1 = val;
        }
        break;
    }
    case RESKV_FMT_QUANT: {
        const uint32_t* qt = (const uint32_t*)ct.payload + row * ct.width;
        const float s = h2f(ct.scale[row]);
        const int bits = ct.bits, per_word = 32 / bits;
        const int sign = 1 << (bits - 1), mask = (1 << bits) - 1;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int d = lane + 64 * half;
            const int code = (int)((qt[d / per_word] >> ((d % per_word) * bits)) & (uint32_t)mask);
            const float val = (float)((code ^ sign) - sign) * s;
            if (half == 0) r0 = val; else r1 = val;
        }
        break;
    }
    default: {  // dense fp16 rows
        const uint16_t* p = (const uint16_t*)ct.payload + row * kDim;
        r0 = h2f(p[lane]);
        r1 = h2f(p[lane + 64]);
        break;
    }
    }
}

__device__ __forceinline__ int clamp_id(int id, int nc) { return id < 0 ? 0 : (id >= nc ? nc - 1 : id); }

template <int G>
__global__ void __launch_bounds__(256) decode_partial_kernel(
    const uint16_t* __restrict__ q, CTensor kt, CTensor vt, const float* __restrict__ inv_freq,
    int Hq, int H, int T, int start_pos, int pos_q, float scaling, int splits,
    float* __restrict__ pm, float* __restrict__ pl, float* __restrict__ pdelta, float* __restrict__ pbeta) {
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const long bh = (long)b * H + h;
    const int t0 = (int)(((long)split * T) / splits);
    const int t1 = (int)(((long)(split + 1) * T) / splits);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    // K centroid table in fp32; reused afterwards for the cross-wave merge.
    __shared__ float s_buf[kMaxClusters * kDim];
    const bool dense = kt.fmt == kFmtDense;
    if (!dense) {
        const uint16_t* kc = kt.cent + bh * kt.nc * kDim;
        for (int i = threadIdx.x; i < kt.nc * kDim; i += blockDim.x) s_buf[i] = h2f(kc[i]);
    }
    __syncthreads();

    const float freq = inv_freq[lane];
    float qa[G], qb[G];
    {
        float s, c;
        rope_sincos((float)pos_q, freq, &s, &c);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint16_t* qr = q + ((long)b * Hq + (long)h * G + g) * kDim;
            const float a = h2f(qr[lane]), bb = h2f(qr[lane + 64]);
            qa[g] = a * c - bb * s;
            qb[g] = bb * c + a * s;
        }
    }

    float m[G], l[G], d0[G], d1[G], beta[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
        d0[g] = d1[g] = beta[g] = 0.0f;
    }

    for (int t = t0 + wave; t < t1; t += kWaves) {
        const long row = bh * T + t;
        float kr0, kr1, vr0, vr1;
        decode_residual(kt, row, lane, kr0, kr1);
        decode_residual(vt, row, lane, vr0, vr1);
        float k0 = kr0, k1 = kr1;
        int vid = -1;
        if (!dense) {
            const int kid = clamp_id(kt.ids[row], kt.nc);
            vid = clamp_id(vt.ids[row], vt.nc);
            k0 += s_buf[kid * kDim + lane];
            k1 += s_buf[kid * kDim + lane + 64];
        }
        float s, c;
        rope_sincos((float)(start_pos + t), freq, &s, &c);
        const float x0 = k0 * c - k1 * s;
        const float x1 = k1 * c + k0 * s;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float score = wave_sum(qa[g] * x0 + qb[g] * x1) * scaling;
            const float mn = fmaxf(m[g], score);
            const float alpha = expf(m[g] - mn);
            const float p = expf(score - mn);
            l[g] = l[g] * alpha + p;
            d0[g] = d0[g] * alpha + p * vr0;
            d1[g] = d1[g] * alpha + p * vr1;
            beta[g] = beta[g] * alpha + (lane == vid ? p : 0.0f);
            m[g] = mn;
        }
    }
    __syncthreads();  // centroid table no longer needed

    // cross-wave merge through LDS: [wave][g][128 delta | 64 beta | m | l]
    constexpr int kStride = kDim + kMaxClusters + 2;
    float* mine = s_buf + (wave * G) * kStride;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float* e = mine + g * kStride;
        e[lane] = d0[g];
        e[lane + 64] = d1[g];
        e[kDim + lane] = beta[g];
        if (lane == 0) {
            e[kDim + kMaxClusters] = m[g];
            e[kDim + kMaxClusters + 1] = l[g];
        }
    }
    __syncthreads();
    for (int g = wave; g < G; g += kWaves) {
        float mx = -INFINITY;
        for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, s_buf[(w * G + g) * kStride + kDim + kMaxClusters]);
        float acc0 = 0.0f, acc1 = 0.0f, accb = 0.0f, accl = 0.0f;
        for (int w = 0; w < kWaves; ++w) {
            const float* e = s_buf + (w * G + g) * kStride;
            const float lw = e[kDim + kMaxClusters + 1];
            const float sc = lw > 0.0f ? expf(e[kDim + kMaxClusters] - mx) : 0.0f;
            acc0 += e[lane] * sc;
            acc1 += e[lane + 64] * sc;
            accb += e[kDim + lane] * sc;
            accl += lw * sc;
        }
        const long slot = ((long)b * Hq + (long)h * G + g) * splits + split;
        pdelta[slot * kDim + lane] = acc0;
        pdelta[slot * kDim + lane + 64] = acc1;
        pbeta[slot * kMaxClusters + lane] = accb;
        if (lane == 0) {
            pm[slot] = mx;
            pl[slot] = accl;
        }
    }
}

// One wave per (batch, query head): combine the split partials.
__global__ void __launch_bounds__(64) decode_merge_kernel(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ pdelta,
    const float* __restrict__ pbeta, const uint16_t* __restrict__ vcent, int vnc, int Hq, int H,
    int splits, uint16_t* __restrict__ out, float* __restrict__ om, float* __restrict__ ol) {
    const long bq = blockIdx.x;  // b * Hq + hq
    const int lane = threadIdx.x;
    const int G = Hq / H;
    const long bh = (bq / Hq) * H + (bq % Hq) / G;
    float mx = -INFINITY;
    for (int s = 0; s < splits; ++s)
        if (pl[bq * splits + s] > 0.0f) mx = fmaxf(mx, pm[bq * splits + s]);
    float acc0 = 0.0f, acc1 = 0.0f, beta = 0.0f, lsum = 0.0f;
    for (int s = 0; s < splits; ++s) {
        const long slot = bq * splits + s;
        const float lw = pl[slot];
        if (!(lw > 0.0f)) continue;
        const float sc = expf(pm[slot] - mx);
        lsum += lw * sc;
        acc0 += pdelta[slot * kDim + lane] * sc;
        acc1 += pdelta[slot * kDim + lane + 64] * sc;
        beta += pbeta[slot * kMaxClusters + lane] * sc;
    }
    if (vcent != nullptr) {
        const uint16_t* vc = vcent + bh * vnc * kDim;
        for (int c = 0; c < vnc; ++c) {
            const float bc = readlane(beta, c);
            acc0 += bc * h2f(vc[c * kDim + lane]);
            acc1 += bc * h2f(vc[c * kDim + lane + 64]);
        }
    }
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    out[bq * kDim + lane] = f2h(acc0 * inv);
    out[bq * kDim + lane + 64] = f2h(acc1 * inv);
    if (lane == 0) {
        if (om) om[bq] = mx;
        if (ol) ol[bq] = lsum;
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

int auto_splits(int B, int H, int T) {
    const long heads = (long)B * H;
    long s = (2048 + heads - 1) / heads;  // ~8 workgroups per CU over 256 CUs
    const long cap = T / 32 > 0 ? T / 32 : 1;
    if (s > cap) s = cap;
    if (s > kMaxSplits) s = kMaxSplits;
    return (int)(s < 1 ? 1 : s);
}

int resolve_splits(int B, int H, int T, int splits) {
    if (splits > 0) return splits < T ? (splits < kMaxSplits ? splits : kMaxSplits) : T;
    return auto_splits(B, H, T);
}

int64_t workspace_for(int B, int Hq, int S) {
    return (int64_t)B * Hq * S * (2 + kDim + kMaxClusters) * (int64_t)sizeof(float);
}

CTensor to_ct(const reskv_ctensor* c) {
    return CTensor{(const uint16_t*)c->centroids, c->ids, c->payload, c->meta,
                   (const uint16_t*)c->scale, c->nc, c->format, c->width, c->bits};
}

int check_ct(const reskv_ctensor* c, const char* name) {
    RESKV_REQUIRE(c != nullptr, "%s: null tensor descriptor", name);
    RESKV_REQUIRE(c->centroids && c->ids && c->payload, "%s: null pointer", name);
    RESKV_REQUIRE(c->nc >= 1 && c->nc <= kMaxClusters, "%s: centroid count must be in [1, 64]", name);
    switch (c->format) {
    case RESKV_FMT_BITMAP:
        RESKV_REQUIRE(c->meta && c->width >= 1 && c->width <= kDim, "%s: bad bitmap tensor", name);
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
    return 0;
}

template <int G>
void launch_partial(dim3 grid, hipStream_t st, const uint16_t* q, const CTensor& k, const CTensor& v,
                    const float* f, int Hq, int H, int T, int start, int pos, float scaling, int S,
                    float* pm, float* pl, float* pd, float* pb) {
    hipLaunchKernelGGL(decode_partial_kernel<G>, grid, dim3(256), 0, st, q, k, v, f, Hq, H, T, start, pos,
                       scaling, S, pm, pl, pd, pb);
}

int run_decode(const void* q, const CTensor& k, const CTensor& v, const uint16_t* vcent, int vnc,
               const float* inv_freq, int B, int Hq, int H, int T, int start_pos, int pos_q,
               float scaling, int splits, void* out, float* m, float* l, void* ws, int64_t ws_bytes,
               void* stream) {
    RESKV_REQUIRE(q && inv_freq && out, "null pointer argument");
    RESKV_REQUIRE(B > 0 && H > 0 && T > 0, "batch, head and token counts must be positive");
    RESKV_REQUIRE(Hq % H == 0, "query heads must be a multiple of KV heads");
    const int G = Hq / H;
    RESKV_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "supported GQA ratios are 1, 2, 4 and 8");
    const int S = resolve_splits(B, H, T, splits);
    RESKV_REQUIRE(ws != nullptr && ws_bytes >= workspace_for(B, Hq, S), "decode workspace too small");
    float* pm = (float*)ws;
    float* pl = pm + (long)B * Hq * S;
    float* pd = pl + (long)B * Hq * S;
    float* pb = pd + (long)B * Hq * S * kDim;
    hipStream_t st = (hipStream_t)stream;
    dim3 grid(S, H, B);
    const uint16_t* qq = (const uint16_t*)q;
    switch (G) {
    case 1: launch_partial<1>(grid, st, qq, k, v, inv_freq, Hq, H, T, start_pos, pos_q, scaling, S, pm, pl, pd, pb); break;
    case 2: launch_partial<2>(grid, st, qq, k, v, inv_freq, Hq, H, T, start_pos, pos_q, scaling, S, pm, pl, pd, pb); break;
    case 4: launch_partial<4>(grid, st, qq, k, v, inv_freq, Hq, H, T, start_pos, pos_q, scaling, S, pm, pl, pd, pb); break;
    default: launch_partial<8>(grid, st, qq, k, v, inv_freq, Hq, H, T, start_pos, pos_q, scaling, S, pm, pl, pd, pb); break;
    }
    if (reskv_host::check_launch("decode_partial_kernel")) return 1;
    hipLaunchKernelGGL(decode_merge_kernel, dim3(B * Hq), dim3(64), 0, st, pm, pl, pd, pb, vcent, vnc, Hq, H, S,
                       (uint16_t*)out, m, l);
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

extern "C" int reskv_decode(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                            const float* inv_freq, int B, int Hq, int H, int T, int start_pos,
                            int pos_q, float scaling, int splits, void* out, float* m, float* l,
                            void* workspace, int64_t workspace_bytes, void* stream) {
    if (check_ct(k, "K") || check_ct(v, "V")) return 1;
    return run_decode(q, to_ct(k), to_ct(v), (const uint16_t*)v->centroids, v->nc, inv_freq, B, Hq, H, T,
                      start_pos, pos_q, scaling, splits, out, m, l, workspace, workspace_bytes, stream);
}

extern "C" int reskv_decode_dense(const void* q, const void* k, const void* v, const float* inv_freq,
                                  int B, int Hq, int H, int T, int start_pos, int pos_q, float scaling,
                                  int splits, void* out, float* m, float* l, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
    RESKV_REQUIRE(k && v, "null K/V pointer");
    const CTensor kd{nullptr, nullptr, k, nullptr, nullptr, 1, kFmtDense, kDim, 16};
    const CTensor vd{nullptr, nullptr, v, nullptr, nullptr, 1, kFmtDense, kDim, 16};
    return run_decode(q, kd, vd, nullptr, 0, inv_freq, B, Hq, H, T, start_pos, pos_q, scaling, splits, out, m, l,
                      workspace, workspace_bytes, stream);
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
