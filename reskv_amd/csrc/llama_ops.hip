// Fused per-layer steps of the end-to-end decode harness (reskv_amd/llama.py):
// RMSNorm, the split / rotate / append of the new token's Q, K and V, and the
// gated activation.  In a batch-16 decode step each replaces a chain of small
// torch kernels (8 for the RMSNorm, about 20 for the rotations, copies and
// appends, 3 for the activation) whose launch gaps cost more than the GEMMs
// around them.  The arithmetic follows the torch formulas step by step (each
// product and sum rounded to fp32, results rounded to fp16 once), so the
// rotations and copies are bit-identical to them; the RMSNorm's sum of squares
// is reduced in a fixed tree order of its own.
#include "common.h"
#include "reskv_llama.h"

using namespace reskv;

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxHidden = 8192;  // 4 uint4 (32 halves) per thread at most

__device__ __forceinline__ float block_sum_256(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup per row; thread i holds the 16-byte chunks i, i + 256, ...
__global__ void __launch_bounds__(kNormThreads) rmsnorm_kernel(const uint4* __restrict__ x,
                                                               const uint4* __restrict__ w, uint4* __restrict__ y,
                                                               int chunks, float inv_n, float eps) {
    __shared__ float red[4];
    const uint4* xr = x + (long)blockIdx.x * chunks;
    uint4* yr = y + (long)blockIdx.x * chunks;
    uint4 xv[kNormMaxHidden / 8 / kNormThreads];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormMaxHidden / 8 / kNormThreads; ++i) {
        const int c = threadIdx.x + i * kNormThreads;
        xv[i] = c < chunks ? xr[c] : make_uint4(0, 0, 0, 0);
        const uint32_t wd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = h2f((uint16_t)(wd[j] & 0xFFFFu)), b = h2f((uint16_t)(wd[j] >> 16));
            ss = __fadd_rn(ss, __fmul_rn(a, a));
            ss = __fadd_rn(ss, __fmul_rn(b, b));
        }
    }
    const float r = rsqrtf(__fadd_rn(__fmul_rn(block_sum_256(ss, red), inv_n), eps));
#pragma unroll
    for (int i = 0; i < kNormMaxHidden / 8 / kNormThreads; ++i) {
        const int c = threadIdx.x + i * kNormThreads;
        if (c >= chunks) break;
        const uint4 wv = w[c];
        const uint32_t xd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w}, wd[4] = {wv.x, wv.y, wv.z, wv.w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float lo = __fmul_rn(__fmul_rn(h2f((uint16_t)(xd[j] & 0xFFFFu)), r), h2f((uint16_t)(wd[j] & 0xFFFFu)));
            const float hi = __fmul_rn(__fmul_rn(h2f((uint16_t)(xd[j] >> 16)), r), h2f((uint16_t)(wd[j] >> 16)));
            o[j] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
        }
        yr[c] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// silu as torch evaluates it for fp16 tensors: x / (1 + exp(-x)) in fp32.
__device__ __forceinline__ float silu_f32(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, expf(-x))); }

// One thread per 8 outputs.
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint4* __restrict__ gu, uint4* __restrict__ out,
                                                       int rows, int chunks) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)rows * chunks) return;
    const long r = idx / chunks, c = idx % chunks;
    const uint4 g = gu[r * 2 * chunks + c], u = gu[r * 2 * chunks + chunks + c];
    const uint32_t gd[4] = {g.x, g.y, g.z, g.w}, ud[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a0 = h2f(f2h(silu_f32(h2f((uint16_t)(gd[j] & 0xFFFFu)))));
        const float a1 = h2f(f2h(silu_f32(h2f((uint16_t)(gd[j] >> 16)))));
        const float lo = __fmul_rn(a0, h2f((uint16_t)(ud[j] & 0xFFFFu)));
        const float hi = __fmul_rn(a1, h2f((uint16_t)(ud[j] >> 16)));
        o[j] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
    }
    out[idx] = make_uint4(o[0], o[1], o[2], o[3]);
}

struct RopeArgs {
    const uint16_t* qkv;
    const float* cos;
    const float* sin;
    const int64_t* pos;
    uint16_t *q, *qr, *k, *kr, *v;
    uint16_t *cache_rot, *cache_raw, *cache_v;
    const int64_t* slot;
    int64_t sb, sh, st;
    int Hq, Hk;
};

// Thread j of a 64-thread row owns channels j and j + 64 (one rotate-half
// pair) of one head: rows 0..Hq-1 are the Q heads, then Hk K heads, then Hk V
// heads of batch row blockIdx.y.
__global__ void __launch_bounds__(256) qkv_rope_kernel(RopeArgs A) {
    const int rows = A.Hq + 2 * A.Hk;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int j = threadIdx.x & 63;
    const long b = blockIdx.y;
    const uint16_t* src = A.qkv + (b * rows + row) * kDim;
    const uint16_t a16 = src[j], b16 = src[j + kHalf];
    if (row >= A.Hq + A.Hk) {  // V: copy and append
        const int hv = row - A.Hq - A.Hk;
        uint16_t* dv = A.v + (b * A.Hk + hv) * kDim;
        dv[j] = a16;
        dv[j + kHalf] = b16;
        if (A.cache_v) {
            uint16_t* cv = A.cache_v + b * A.sb + hv * A.sh + *A.slot * A.st;
            cv[j] = a16;
            cv[j + kHalf] = b16;
        }
        return;
    }
    const long p = *A.pos;
    const float c = A.cos[p * kHalf + j], s = A.sin[p * kHalf + j];
    const float a = h2f(a16), bb = h2f(b16);
    const uint16_t ra = f2h(__fsub_rn(__fmul_rn(a, c), __fmul_rn(bb, s)));
    const uint16_t rb = f2h(__fadd_rn(__fmul_rn(bb, c), __fmul_rn(a, s)));
    if (row < A.Hq) {
        uint16_t* dq = A.q + (b * A.Hq + row) * kDim;
        uint16_t* dr = A.qr + (b * A.Hq + row) * kDim;
        dq[j] = a16;
        dq[j + kHalf] = b16;
        dr[j] = ra;
        dr[j + kHalf] = rb;
        return;
    }
    const int hk = row - A.Hq;
    uint16_t* dk = A.k + (b * A.Hk + hk) * kDim;
    uint16_t* dr = A.kr + (b * A.Hk + hk) * kDim;
    dk[j] = a16;
    dk[j + kHalf] = b16;
    dr[j] = ra;
    dr[j + kHalf] = rb;
    const long at = b * A.sb + hk * A.sh;
    if (A.cache_raw) {
        uint16_t* cr = A.cache_raw + at + *A.slot * A.st;
        cr[j] = a16;
        cr[j + kHalf] = b16;
    }
    if (A.cache_rot) {
        uint16_t* ck = A.cache_rot + at + *A.slot * A.st;
        ck[j] = ra;
        ck[j + kHalf] = rb;
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" int reskv_llama_rmsnorm(const void* x, const void* w, void* y, int rows, int hidden, float eps,
                                   void* stream) {
    RESKV_REQUIRE(x && w && y, "null pointer");
    RESKV_REQUIRE(rows >= 0, "negative row count");
    RESKV_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= kNormMaxHidden,
                  "hidden size %d must be a positive multiple of 8 up to %d", hidden, kNormMaxHidden);
    RESKV_REQUIRE(aligned16(x) && aligned16(w) && aligned16(y), "x, w and y must be 16-byte aligned");
    if (rows == 0) return 0;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, (hipStream_t)stream,
                       (const uint4*)x, (const uint4*)w, (uint4*)y, hidden / 8, 1.0f / (float)hidden, eps);
    return reskv_host::check_launch("rmsnorm_kernel");
}

extern "C" int reskv_llama_silu_mul(const void* gu, void* out, int rows, int ffn, void* stream) {
    RESKV_REQUIRE(gu && out, "null pointer");
    RESKV_REQUIRE(rows >= 0, "negative row count");
    RESKV_REQUIRE(ffn > 0 && ffn % 8 == 0, "ffn size %d must be a positive multiple of 8", ffn);
    RESKV_REQUIRE(aligned16(gu) && aligned16(out), "gu and out must be 16-byte aligned");
    const long n = (long)rows * (ffn / 8);
    if (n == 0) return 0;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)gu, (uint4*)out, rows, ffn / 8);
    return reskv_host::check_launch("silu_mul_kernel");
}

extern "C" int reskv_llama_qkv_rope(const void* qkv, const float* cos, const float* sin, const int64_t* pos, int B,
                                    int Hq, int Hk, void* q, void* qr, void* k, void* kr, void* v, void* cache_rot,
                                    void* cache_raw, void* cache_v, const int64_t* slot, int64_t stride_b,
                                    int64_t stride_h, int64_t stride_t, void* stream) {
    RESKV_REQUIRE(qkv && cos && sin && pos && q && qr && k && kr && v, "null pointer");
    RESKV_REQUIRE(B >= 0 && Hq > 0 && Hk > 0 && Hq % Hk == 0, "bad head counts (Hq %d, Hk %d)", Hq, Hk);
    const bool append = cache_rot || cache_raw || cache_v;
    RESKV_REQUIRE(!append || slot, "a cache append needs the slot pointer");
    RESKV_REQUIRE(!append || (stride_b > 0 && stride_h > 0 && stride_t > 0), "cache strides must be positive");
    if (B == 0) return 0;
    RopeArgs A{(const uint16_t*)qkv, cos, sin, pos, (uint16_t*)q, (uint16_t*)qr, (uint16_t*)k, (uint16_t*)kr,
               (uint16_t*)v, (uint16_t*)cache_rot, (uint16_t*)cache_raw, (uint16_t*)cache_v, slot,
               stride_b, stride_h, stride_t, Hq, Hk};
    const int rows = Hq + 2 * Hk;
    hipLaunchKernelGGL(qkv_rope_kernel, dim3((rows + 3) / 4, B), dim3(256), 0, (hipStream_t)stream, A);
    return reskv_host::check_launch("qkv_rope_kernel");
}
