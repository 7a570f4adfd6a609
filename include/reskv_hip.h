/*
 * ResKV compressed-KV hot path for AMD Instinct MI355X (gfx950): C ABI.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), enqueues its kernels asynchronously on that stream and
 * returns 0 on success.  On failure it returns non-zero and
 * reskv_last_error() describes the problem (thread-local).  No entry point
 * allocates device memory: outputs and scratch are caller-owned (the Python
 * layer allocates them with torch).  Shapes use the reference's names:
 * B batch, H KV heads (H_kv), Hq query heads, T tokens, C centroids, 128 channels.
 *
 * Tensor layouts (all contiguous, row-major):
 *   keys        fp16  [B, H, T, 128]
 *   centroids   fp16  [B, H, C, 128]
 *   ids         int32 [B, H, T] (encoders) / int8 [B*H, T] (decode)
 *   payload     fp16  [B*H, T, nnz] or int32 words (quantised formats)
 *   metadata    int64 [B*H, T, 2] bitmaps | int32 [B*H, T, 4] tile codes |
 *               int32 [B*H, T, 2] 2-bit selections
 *   scale       fp16  [B*H, T]
 */
#ifndef RESKV_HIP_H
#define RESKV_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Thread-local description of the last failure; "" when none. */
const char* reskv_last_error(void);

/* Library ABI version (bumped on any signature, struct or data-layout
 * change, or when entry points are added, here or in reskv_llama.h); 7. */
int reskv_abi_version(void);

/* ------------------------------------------------------------------ *
 * Residual encoders (one call encodes one K or V tensor)
 * ------------------------------------------------------------------ */

/* Tiled / structured-4:16 FP16 encoder.
 * Replaces ext.compress_fp16 (reskv/csrc/compression.cu:423-473, op bound at :509).
 * nnz in {16,..,120} divisible by 8 (64: tiled, 32 with struct_index=1: 4:16).
 * payload fp16 [B,H,T,nnz]; meta int32 [B,H,T,4]. */
int reskv_compress_fp16(const void* keys, const void* centroids, const int32_t* ids,
                        void* payload, int32_t* meta, int B, int H, int T, int C,
                        int nnz, int struct_index, void* stream);

/* Unstructured FP16 encoder (MSB-first int64 bitmaps).
 * Replaces the PyTorch encoder of reskv/compression.py:75-89 (gather, abs,
 * topk/sort, scatter, weighted sum).  payload fp16 [B,H,T,nnz];
 * meta int64 [B,H,T,2]. */
int reskv_compress_bitmap(const void* keys, const void* centroids, const int32_t* ids,
                          void* payload, int64_t* meta, int B, int H, int T, int C,
                          int nnz, void* stream);

/* A layer's K and V through reskv_compress_fp16 / reskv_compress_bitmap in
 * one launch.  Replaces the two _encode calls of compress
 * (reskv/compression.py:166-167), K then V with one plan; each result equals
 * the single-tensor call's.  Ck, Cv: the two centroid counts. */
int reskv_compress_fp16_kv(const void* k, const void* v, const void* k_centroids, const void* v_centroids,
                           const int32_t* k_ids, const int32_t* v_ids, void* k_payload, void* v_payload,
                           int32_t* k_meta, int32_t* v_meta, int B, int H, int T, int Ck, int Cv, int nnz,
                           int struct_index, void* stream);
int reskv_compress_bitmap_kv(const void* k, const void* v, const void* k_centroids, const void* v_centroids,
                             const int32_t* k_ids, const int32_t* v_ids, void* k_payload, void* v_payload,
                             int64_t* k_meta, int64_t* v_meta, int B, int H, int T, int Ck, int Cv, int nnz,
                             void* stream);

/* Unstructured top-nnz + symmetric INT4/INT2 quantiser.
 * Replaces ext.compress_quantized (reskv/csrc/compression.cu:392-421, op at :510).
 * qtiles int32 [B,H,T,4*bits]; qscale fp16 [B,H,T]. */
int reskv_compress_quantized(const void* keys, const void* centroids, const int32_t* ids,
                             int32_t* qtiles, void* qscale, int B, int H, int T, int C,
                             int nnz, int bits, void* stream);

/* Structured 1-of-4 INT4 encoder.
 * Replaces ext.compress_structured_int4 (reskv/csrc/compression.cu:475-504, op at :511).
 * qpacked int32 [B,H,T,4]; qmeta int32 [B,H,T,2]; qscale fp16 [B,H,T]. */
int reskv_compress_structured_int4(const void* keys, const void* centroids,
                                   const int32_t* ids, int32_t* qpacked, int32_t* qmeta,
                                   void* qscale, int B, int H, int T, int C, void* stream);

/* ------------------------------------------------------------------ *
 * K-means (Lloyd) over pre-RoPE K or V, one problem per (batch, head)
 * ------------------------------------------------------------------ */

/* Bytes of scratch reskv_kmeans needs for these sizes. */
int64_t reskv_kmeans_workspace_bytes(int BH, int T, int C);

/* torch.linspace(0, T-1, C).long() as torch evaluates it in fp32 (the
 * initial-centre rows of reskv/compression.py:35); rows int32 [C], host
 * memory.  Needs 1 <= C <= 64 and T >= C. */
int reskv_linspace_rows(int T, int C, int32_t* rows);

/* Lloyd iterations from given initial centres.
 * Replaces the torch loop of reskv/compression.py:37-53 (cdist, argmin,
 * one_hot, bmm).  x fp16 [BH,T,128]; centers_init fp32 [BH,C,128], or null:
 * the tokens at reskv_linspace_rows(T, C) of each problem (compression.py:
 * 34-36; T >= C), gathered on the device; centers_out fp16 [BH,C,128]; ids int32 [BH,T]
 * (from the last assignment).  value_mode=0: K semantics (fp32 distances,
 * empty cluster keeps its centre); 1: V semantics (the fp16 cdist of
 * compression.py:38 -- fp16 norms, fp16 distance, fp16 root, lowest index on
 * ties -- fp16 centres, empty cluster -> 0). */
int reskv_kmeans(const void* x, const float* centers_init, void* centers_out, int32_t* ids,
                 int BH, int T, int C, int iterations, int value_mode, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* A layer's K and V clustered together: the two Lloyd runs of
 * reskv/compression.py:164-165 (cluster(key), cluster(value, value=True)) as
 * one sequence of launches over 2*BH problems, K rules for k and V rules for v.
 * k, v fp16 [BH,T,128]; init_k, init_v fp32 [BH,C,128] (both null: the
 * linspace tokens, as in reskv_kmeans); out_k, out_v fp16
 * [BH,C,128]; ids_k, ids_v int32 [BH,T].  Each result equals the separate
 * reskv_kmeans call's.  workspace: reskv_kmeans_workspace_bytes(2*BH, T, C). */
int reskv_kmeans_kv(const void* k, const void* v, const float* init_k, const float* init_v, void* out_k,
                    void* out_v, int32_t* ids_k, int32_t* ids_v, int BH, int T, int C, int iterations,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* Assignment step only: ids = argmin_c d(x, c) (lowest index on ties).
 * Replaces the assignment of reskv/compression.py:61-69 (_incremental_cluster,
 * one decode group against the shared centroid table).  centers fp32 [BH,C,128]
 * (fp16 values for V).  value_mode=0: K, d = |x - c|^2 in fp32 (cdist, :66);
 * 1: V, d = fp32(fp16(|x|^2 + |c|^2) - 2 x.c) with fp16 norms (:63-64).
 * workspace as for reskv_kmeans. */
int reskv_kmeans_assign(const void* x, const float* centers, int32_t* ids, int BH, int T, int C,
                        int value_mode, void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ *
 * Split-K fused decode attention over the compressed cache
 * ------------------------------------------------------------------ */

/* Residual formats of one compressed tensor. */
enum reskv_format {
    RESKV_FMT_BITMAP = 0,      /* fp16 payload [nnz] + int64[2] MSB-first bitmap   */
    RESKV_FMT_TILED = 1,       /* fp16 payload [nnz] + int32[4] 16-bit tile masks  */
    RESKV_FMT_STRUCT16 = 2,    /* fp16 payload [32]  + int32[4] 4:16 nibble codes  */
    RESKV_FMT_STRUCT_INT4 = 3, /* int32 payload [4]  + int32[2] 2-bit codes + scale */
    RESKV_FMT_QUANT = 4        /* int32 payload [4*bits] signed codes + scale       */
};

/* One compressed tensor as the decode kernels read it.  Rows of (batch, head)
 * bh start at bh * t_stride tokens (and bh * c_stride centroids), so a cache
 * held in preallocated capacity buffers is read in place. */
typedef struct reskv_ctensor {
    const void* centroids;   /* fp16 [B*H, nc, 128] */
    const int8_t* ids;       /* int8 [B*H, T] */
    const void* payload;     /* fp16 or int32 words [B*H, T, width] */
    const void* meta;        /* metadata words or NULL */
    const void* scale;       /* fp16 [B*H, T] or NULL */
    int nc;                  /* centroids per head (1..64) */
    int format;              /* enum reskv_format */
    int width;               /* payload last-dim width (values or words) */
    int bits;                /* 16, 4 or 2 */
    int t_stride;            /* tokens between consecutive (batch, head) rows of
                                ids / payload / meta / scale; 0 means T (dense) */
    int c_stride;            /* centroid rows between consecutive (batch, head)
                                tables; 0 means nc (dense) */
} reskv_ctensor;

/* Bytes of split-K scratch a decode of these sizes needs, for every residual
 * format (the automatic split count depends on the format; this covers the
 * largest); splits<=0 means automatic. */
int64_t reskv_decode_workspace_bytes(int B, int Hq, int H, int T, int splits);

/* Split count a decode of these tensors makes (splits<=0: automatic, filling
 * the 256 CUs with as many workgroups as the format's kernel keeps resident
 * per CU, at least two 16-token tiles per wave; >0: min(splits, T, 1024)).
 * rope_table: non-zero when the call passes a RoPE table.  Returns -1 (and
 * sets reskv_last_error) on bad arguments. */
int reskv_decode_splits(const reskv_ctensor* k, const reskv_ctensor* v, int rope_table, int B, int Hq, int H, int T,
                        int splits);

/* Decode one query token per (batch, query head) against the compressed cache.
 * Replaces the deferred ops ext.decode_fp16 / decode_structured_fp16 /
 * decode_structured_int4 (reskv/csrc/cluster_mass.cu:1177-1459, ops at
 * :1512-1515) and the per-token ops ext.decode_fp16 / decode_int4 /
 * decode_quantized (reskv/csrc/attention.cu:665-835, 1296-1348, ops at
 * :1350-1354).  q fp16 [B*Hq,128] (pre-RoPE); inv_freq fp32 [64];
 * out fp16 [B*Hq,128] (normalised); m, l fp32 [B*Hq] (max score and
 * sum of exp(score - m)); either of m, l may be NULL. */
int reskv_decode(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                 const float* inv_freq, int B, int Hq, int H, int T, int start_pos,
                 int pos_q, float scaling, int splits, void* out, float* m, float* l,
                 void* workspace, int64_t workspace_bytes, void* stream);

/* reskv_decode with a precomputed RoPE table (reskv_rope_table) covering
 * positions [0, start_pos + T): per token the kernel reads cos/sin instead of
 * evaluating them.  rope_table may be NULL (same as reskv_decode).  Replaces the
 * same reference ops as reskv_decode; the table plays the part of the model's
 * rotary cache (positions of compressed tokens never change, so one table
 * serves every layer and decode step). */
int reskv_decode_rope(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                      const float* inv_freq, const float* rope_table, int B, int Hq, int H, int T,
                      int start_pos, int pos_q, float scaling, int splits, void* out, float* m,
                      float* l, void* workspace, int64_t workspace_bytes, void* stream);

/* RoPE table for positions [0, count), count a positive multiple of 16:
 * count * 128 fp32 values in blocks of 16 positions.  For frequency index
 * d = 16 g + 4 u + j (g, u, j < 4), cos(fl32(p * inv_freq[d])) is element j of
 * the float4 at index 512 (p / 16) + 64 (2u) + 4 (p % 16) + g, and the sine
 * the same element of the float4 at 512 (p / 16) + 64 (2u + 1) + 4 (p % 16) + g.
 * (The decode reads, per instruction, one such float4 for 16 consecutive
 * positions and 4 groups: at most two contiguous runs.)  Serves the same
 * role as the rotary cos/sin cache that reskv/models/llama.py reads from the
 * model (position_embeddings). */
int reskv_rope_table(const float* inv_freq, int count, float* table, void* stream);

/* Joint softmax of the compressed result with precomputed fp32 recent scores.
 * Replaces the deferred ext.merge_recent (reskv/csrc/cluster_mass.cu:1461-1508,
 * op at :1515).  comp_out fp16 [B*Hq,128]; comp_m, comp_l fp32 [B*Hq];
 * scores fp32 [B,Hq,Tr]; v_recent fp16 [B,H,Tr,128], 16-byte aligned; out
 * fp16 [B*Hq,128]. */
int reskv_merge_recent_scores(const void* comp_out, const float* comp_m, const float* comp_l,
                              const float* scores, const void* v_recent, int B, int Hq,
                              int H, int Tr, void* out, void* stream);

/* Joint softmax of the compressed result with dense rotated recent tokens.
 * Replaces the per-token ext.merge_recent (reskv/csrc/attention.cu:839-906,
 * op at :1355).  q_rope fp16 [B*Hq,128]; k_recent, v_recent fp16 [B,H,*,128]:
 * the first Tr tokens of rows of r_stride tokens (r_stride<=0: Tr), so that a
 * ring buffer is read in place; k_recent and v_recent 16-byte aligned. */
int reskv_merge_recent_qk(const void* comp_out, const float* comp_m, const float* comp_l,
                          const void* q_rope, const void* k_recent, const void* v_recent,
                          int B, int Hq, int H, int Tr, int r_stride, float scaling, void* out,
                          void* stream);

/* reskv_decode_rope followed by reskv_merge_recent_qk in two kernel launches
 * instead of three: the split merge joins the recent tokens before it writes
 * out (fp16 [B*Hq,128]; the joint m, l are not returned).  The result is
 * bitwise that of the two calls.  The reference runs the same two steps as
 * separate ops (reskv/_attention.py:117-143 after cluster_mass.cu:1177-1296);
 * this entry point serves decode loops, where every launch counts. */
int reskv_decode_recent(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                        const float* inv_freq, const float* rope_table, int B, int Hq, int H, int T,
                        int start_pos, int pos_q, float scaling, int splits, const void* q_rope,
                        const void* k_recent, const void* v_recent, int Tr, int r_stride, void* out,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of device scratch that reskv_decode_recent_noalloc holds per GPU. */
#define RESKV_NOALLOC_SCRATCH_BYTES (8LL << 20)

/* reskv_decode_recent without a workspace argument: it allocates nothing.
 * No counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The split-K partial records go to a file-scope
 * device array of RESKV_NOALLOC_SCRATCH_BYTES (8 MiB) that each GPU holds
 * until the process ends; its address is looked up once per device
 * (hipGetSymbolAddress) on the first call.  Sizes whose partials exceed it
 * (reskv_decode_workspace_bytes(B, Hq, H, T, splits) > 8 MiB; the automatic
 * split count stays below that up to B*Hq = 10,000 rows) are rejected with an
 * error.  The array used is the current device's: `stream` must belong to
 * the current device (the null stream does), otherwise the call is rejected.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * race.  Arguments and result are those of reskv_decode_recent (Tr = 0:
 * plain decode). */
int reskv_decode_recent_noalloc(const void* q, const reskv_ctensor* k, const reskv_ctensor* v,
                                const float* inv_freq, const float* rope_table, int B, int Hq, int H, int T,
                                int start_pos, int pos_q, float scaling, int splits, const void* q_rope,
                                const void* k_recent, const void* v_recent, int Tr, int r_stride, void* out,
                                void* stream);

/* Dense fp16 decode attention (the uncompressed baseline at the same shapes):
 * q fp16 [B*Hq,128] pre-RoPE, k fp16 [B,H,*,128] pre-RoPE, v fp16 [B,H,*,128]:
 * the first T tokens of rows of t_stride tokens (t_stride<=0: T), so that a
 * preallocated cache is read in place.  Same split-K engine and RoPE as
 * reskv_decode_rope (rope_table may be NULL), out fp16 [B*Hq,128]. */
int reskv_decode_dense(const void* q, const void* k, const void* v, const float* inv_freq,
                       const float* rope_table, int B, int Hq, int H, int T, int t_stride, int start_pos,
                       int pos_q, float scaling, int splits, void* out, float* m, float* l,
                       void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RESKV_HIP_H */
