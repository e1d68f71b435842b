/*
 * Token2Tile sparse attention on MI355X (gfx950): the C ABI.
 *
 * Every entry point is destination passing: the caller allocates inputs,
 * outputs and workspaces in device memory and passes plain pointers, sizes
 * and a HIP stream (hipStream_t, passed as void*; NULL = the null stream).
 * Work is enqueued on that stream; nothing synchronises the host.  Each
 * function returns T2T_OK or an error code; t2t_last_error() gives a message
 * for the calling thread's last failure.  Inputs are never modified.
 *
 * Layouts (H heads, N tokens, D = 128 head dim, r = 32 rank, CK = 2048 key
 * clusters, CQ query clusters), all row-major and contiguous:
 *   q, k, v, kp, V_sorted, attn_out, out   [H, N, D]   fp16 or bf16 (dtype)
 *   QU, KU                                 [H, N, r]   fp16
 *   U (Uq / Uk)                            [H, D, r]   fp16
 *   cq                                     [H, CQ, r]  fp16
 *   ck0, ck16, cks                         [H, CK, r]  fp16;  ck2 fp32
 *   gl                                     [H, N, CK]  fp16
 *   labels / perms / rowcnt                [H, N]      int32
 *   counts                                 [H, CQ] or [H, CK] int32
 *   unip (packed union)                    [H, CQ, CK/32] int32, bit c&31
 *                                          of word c>>5 = cluster c
 *   sumv                                   [H, CK, D]  fp16;  lam [H] fp32
 *   lse                                    [H, N] fp32 (log2 units)
 *
 * Reference citations are relative to the Token2Tile source tree
 * (token2tile/operator/...).
 */
#ifndef T2T_HIP_H
#define T2T_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes and data types ------------------------------------- */
#define T2T_OK            0
#define T2T_ERR_ARG       1   /* bad size, pointer or dtype            */
#define T2T_ERR_WORKSPACE 2   /* workspace missing or too small        */
#define T2T_ERR_LAUNCH    3   /* the HIP runtime rejected a launch     */
#define T2T_ERR_UNSUPPORTED 4 /* shape outside the kernels' limits     */

#define T2T_F16  0
#define T2T_BF16 1

/* Message for the calling thread's last non-zero return. */
const char* t2t_last_error(void);
/* ABI version (major * 100 + minor). */
int t2t_abi_version(void);

/* ---- S1 projection --------------------------------------------------- */
/* out[h, n, :] = fp16(x[h, n, :] @ U[h]) with fp32 accumulation; bf16 x is
 * rounded to fp16 first, as the reference backend casts bf16 to fp16.
 * Replaces torch.bmm(q, Uq, out=QU) / torch.bmm(k, Uk, out=KU),
 * operator/deploy_step.py:321-324.  D % 16 == 0, D <= 256, r == 32. */
int t2t_project(const void* x, int x_dtype, const void* U, void* out,
                int H, int N, int D, int r, void* stream);

/* ---- S2 k-means maintenance ------------------------------------------ */
/* Workspace bytes for t2t_kmm_run. */
size_t t2t_kmm_ws_bytes(int H, int N, int CQ, int CK);
/* One warm-started k-means update: query labels over two assignment passes
 * (qlab, cq2, qcounts, qperm), key labels in one pass (klab, kcounts,
 * kperm, ck2 fp32), cluster-ordered V (V_sorted, dtype v_dtype; NULL: not
 * written, for callers that read V through kperm), value sums
 * sumv = fp16(vsum / lam) with lam = max(1, max|vsum| / 32768).  Rows
 * >= N - pin_tail get key label CK - 1.  Deterministic.
 * Replaces kmm_ext.run, kernels/kmeans_maintain/src/main.cpp:20-46
 * (kernels.cu:787-876).  r == 32, 1 <= CQ <= 4096, 1 <= CK <= 4096. */
int t2t_kmm_run(const void* QU, const void* KU, const void* V, int v_dtype,
                const void* cq0, const void* ck0,
                int32_t* qlab, void* cq2, int32_t* klab, float* ck2,
                int32_t* qcounts, int32_t* qperm,
                int32_t* kcounts, int32_t* kperm,
                void* V_sorted, void* sumv, float* lam,
                int H, int N, int CQ, int CK, int pin_tail,
                void* ws, size_t ws_bytes, void* stream);
/* Workspace bytes for the two value-statistics calls. */
size_t t2t_vstats_ws_bytes(int H, int N, int CK);
/* Reuse call: V_sorted = V[kperm] (NULL: not written), sumv, lam from this
 * call's V.
 * Replaces kmm_ext.run_vstats_gather, kmeans_maintain/src/main.cpp:63-78
 * (kernels.cu:900-923). */
int t2t_kmm_run_vstats_gather(const void* V, int v_dtype,
                              const int32_t* kperm, const int32_t* kcounts,
                              void* V_sorted, void* sumv, float* lam,
                              int H, int N, int CK,
                              void* ws, size_t ws_bytes, void* stream);
/* sumv, lam from an already cluster-ordered V_sorted.
 * Replaces kmm_ext.run_vstats, kmeans_maintain/src/main.cpp:48-61. */
int t2t_kmm_run_vstats(const void* V_sorted, int v_dtype,
                       const int32_t* kcounts, void* sumv, float* lam,
                       int H, int N, int CK,
                       void* ws, size_t ws_bytes, void* stream);

/* ---- S3 centroids and scores ----------------------------------------- */
/* ck16 = fp16(ck2); cks = fp16(fp32(ck2 * scale)).
 * Replaces state["ck"] = ck2.half() and cks = (ck2 * scale).half(),
 * operator/deploy_step.py:389,393. Either output may be NULL. */
int t2t_centroid_finalize(const float* ck2, void* ck16, void* cks, float scale,
                          int H, int CK, int r, void* stream);
/* gl[h, n, c] = fp16(QU[h, n] . cks[h, c]) with fp32 accumulation.
 * Replaces torch.bmm(QU, cks^T, out=gl), operator/deploy_step.py:394.
 * r == 32, CK % 256 == 0. */
int t2t_score(const void* QU, const void* cks, void* gl,
              int H, int N, int CK, int r, void* stream);

/* ---- S4 selection and union ------------------------------------------ */
/* Workspace bytes for the selection calls. */
size_t t2t_select_ws_bytes(int H, int N, int CQ);
/* Per query row: the shortest prefix of key clusters, ordered by score
 * descending (fp16 bit order, -0 < +0) then cluster index ascending, whose
 * sizes reach ns (read from device memory, *ns_dev).  unip ORs the
 * selections of the rows qperm[off[t] : off[t] + qcounts[t]] of every query
 * cluster t (off = exclusive scan of qcounts); rowcnt[h, row] = selected
 * keys of that row.  Requires 1 <= ns <= N, N < 524288, CK == 2048.
 * Replaces ext.run_packed, kernels/select_union/src/main.cpp:40-53
 * (kernel.cu:76-97,190-412,447-488,523-537). */
int t2t_select_run_packed(const void* gl, const int32_t* kcounts,
                          const int32_t* qperm, const int32_t* qcounts,
                          const int32_t* ns_dev, int32_t* unip, int32_t* rowcnt,
                          int H, int N, int CQ,
                          void* ws, size_t ws_bytes, void* stream);
/* The split variant: same bitmap (rows are processed in balanced chunks
 * whatever the query cluster sizes); cap >= 1 is validated and recorded.
 * Replaces ext.run_split_packed, select_union/src/main.cpp:55-72. */
int t2t_select_run_split_packed(const void* gl, const int32_t* kcounts,
                                const int32_t* qperm, const int32_t* qcounts,
                                int cap, const int32_t* ns_dev,
                                int32_t* unip, int32_t* rowcnt,
                                int H, int N, int CQ,
                                void* ws, size_t ws_bytes, void* stream);
/* Scoring and selection in one pass (S3 + S4): the scores fp16(QU . cks^T)
 * are computed on chip, with the arithmetic of t2t_score, and never stored;
 * unip and rowcnt are bit-identical to t2t_score followed by
 * t2t_select_run_packed.  Replaces torch.bmm(QU, cks^T, out=gl) +
 * ext.run_packed, operator/deploy_step.py:393-411.  ws as for the selection. */
int t2t_score_select_packed(const void* QU, const void* cks, const int32_t* kcounts,
                            const int32_t* qperm, const int32_t* qcounts,
                            const int32_t* ns_dev, int32_t* unip, int32_t* rowcnt,
                            int H, int N, int CQ, void* ws, size_t ws_bytes, void* stream);
/* Allocation-free t2t_score_select_packed.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It takes no workspace: its scratch (H * (CQ + 1) int32
 * query-cluster offsets) is a static device array of
 * T2T_NOALLOC_SCRATCH_INTS entries per GPU, held until the process ends, and
 * sizes beyond it return T2T_ERR_UNSUPPORTED.  It calls no allocator.  Calls
 * that overlap on one GPU share that array and race.  The stream must belong
 * to the current device (else T2T_ERR_UNSUPPORTED).  Results are
 * bit-identical to t2t_score_select_packed. */
#define T2T_NOALLOC_SCRATCH_INTS 262208   /* 64 heads x (4096 + 1) */
size_t t2t_score_select_noalloc_max_ints(void);
int t2t_score_select_packed_noalloc(const void* QU, const void* cks, const int32_t* kcounts,
                                    const int32_t* qperm, const int32_t* qcounts,
                                    const int32_t* ns_dev, int32_t* unip, int32_t* rowcnt,
                                    int H, int N, int CQ, void* stream);
/* Byte-per-cluster union uni[h, t, c] in {0, 1}, [H, CQ, CK] uint8.
 * Replaces ext.run, select_union/src/main.cpp:5-19 (kernel.cu:414-440). */
int t2t_select_run(const void* gl, const int32_t* kcounts,
                   const int32_t* qperm, const int32_t* qcounts,
                   const int32_t* ns_dev, uint8_t* uni, int32_t* rowcnt,
                   int H, int N, int CQ,
                   void* ws, size_t ws_bytes, void* stream);
/* Sets bit CK-1 of every union word row (pinned context cluster).
 * Replaces operator/deploy_step.py:444-448. */
int t2t_union_or_last(int32_t* unip, int H, int CQ, int CK, void* stream);

/* ---- gather ----------------------------------------------------------- */
/* out[h, i, :] = x[h, perm[h, i], :].  Replaces fast_gather,
 * operator/fast_permute.py:54-56.  D * elem_size % 16 == 0. */
int t2t_fast_gather(const void* x, int dtype, const int32_t* perm, void* out,
                    int H, int N, int D, void* stream);

/* ---- S5/S6 tile attention, residual and merge ------------------------- */
/* int32 elements of a task plan (workspace owned by a structure snapshot).
 * Mirrors plan_workspace_ints, kernels/tile_attn/src/main.cpp:16-22. */
size_t t2t_tile_plan_ints(int H, int N, int CQ);
/* Task plan: key-cluster offsets, union lengths, per-head task list ordered
 * by descending rows x kv_len (ties: lower index first).
 * Replaces the plan kernels, tile_attn/src/kernel.cu:259-378,1123-1130. */
int t2t_tile_plan(const int32_t* qcounts, const int32_t* kcounts,
                  const int32_t* unip, int32_t* plan,
                  int H, int N, int CQ, void* stream);
/* Exact attention of each query cluster over its union (S5).  q in the
 * original order, kp/vp cluster ordered; attn_out [H, N, D] (dtype) and
 * lse [H, N] fp32 in the SORTED query order (position j = qperm order).
 * Empty union: zeros and lse = -inf.  Needs a plan from t2t_tile_plan.
 * Replaces launch_cluster_attn, tile_attn/src/kernel.cu:1101-1138. */
int t2t_tile_attn_exact(const void* q, const void* kp, const void* vp, int dtype,
                        const int32_t* kcounts, const int32_t* unip, const int32_t* qperm,
                        const int32_t* plan, void* attn_out, float* lse,
                        int H, int N, int CQ, void* stream);
/* Bytes of the centroid tile image (cks and transposed sumv in the layout
 * the residual kernel stages into LDS), H x 32 tiles of 22528 bytes. */
size_t t2t_centroid_tiles_bytes(int H);
/* Workspace bytes of t2t_tail_merge (the centroid tile image). */
size_t t2t_tail_merge_ws_bytes(int H);
/* Centroid residual over the clusters outside each query's union and the
 * merge with the exact part under one softmax (S6); attn_out and lse in the
 * SORTED order, out in the ORIGINAL order.  tailw_dev: 0-dim fp32 on device.
 * ws >= t2t_tail_merge_ws_bytes(H).
 * Replaces launch_tail_merge, tile_attn/src/kernel.cu:1478-1495. */
int t2t_tail_merge(const void* attn_out, const float* lse, const void* QU,
                   const void* cks, const void* sumv, const int32_t* kcounts,
                   const int32_t* unip, const int32_t* qlab,
                   const int32_t* qperm, const float* lam, const float* tailw_dev,
                   void* out, int dtype, int H, int N, int CQ,
                   void* ws, size_t ws_bytes, void* stream);
/* The centroid tile image of one call: cks [H, 2048, 32] fp16 and sumv
 * [H, 2048, 128] fp16 -> tiles (t2t_centroid_tiles_bytes(H) bytes).  Part of
 * launch_tail_merge's staging, tile_attn/src/kernel.cu:1172-1250. */
int t2t_centroid_tiles(const void* cks, const void* sumv, void* tiles, int H, void* stream);
/* t2t_tile_attn_exact with the output at the ORIGINAL rows of out (lse still
 * in sorted order), for the residual kernel to merge into in place. */
int t2t_tile_attn_exact_orig(const void* q, const void* kp, const void* vp, int dtype,
                             const int32_t* kcounts, const int32_t* unip, const int32_t* qperm,
                             const int32_t* plan, void* out, float* lse,
                             int H, int N, int CQ, void* stream);
/* t2t_tile_attn_exact_orig with the K gather fused into the kernel's loads:
 * k is [H, N, 128] in the ORIGINAL order and key position p of the cluster
 * order reads row kperm[h, p], so kp = k[kperm] is never stored.  Replaces
 * the fast_gather of deploy_step.py:326,456 together with the attention
 * launch that reads its output (tile_attn/src/kernel.cu:820-1096). */
int t2t_tile_attn_exact_orig_gather(const void* q, const void* k, const int32_t* kperm,
                                    const void* vp, int dtype, const int32_t* kcounts,
                                    const int32_t* unip, const int32_t* qperm, const int32_t* plan,
                                    void* out, float* lse, int H, int N, int CQ, void* stream);
/* t2t_tile_attn_exact_orig_gather with the V gather fused as well: v is
 * [H, N, 128] in the ORIGINAL order and key position p reads row kperm[h, p]
 * of both k and v, so neither kp nor V_sorted is stored.  All tensors are
 * strided [H, N, 128] views as for the strided entry points below (one
 * head's K and V rows must each span under 4 GiB).  Replaces the
 * fast_gather of K and the V_sorted of kmm_ext.run / run_vstats_gather
 * (deploy_step.py:326,456; kmeans_maintain/src/kernels.cu:900-923) together
 * with the attention launch that reads them (tile_attn/src/kernel.cu:820-1096). */
int t2t_tile_attn_exact_orig_gather_kv_strided(
    const void* q, long long q_head_stride, long long q_row_stride, const void* k,
    long long k_head_stride, long long k_row_stride, const void* v, long long v_head_stride,
    long long v_row_stride, const int32_t* kperm, int dtype, const int32_t* kcounts,
    const int32_t* unip, const int32_t* qperm, const int32_t* plan, void* out,
    long long out_head_stride, long long out_row_stride, float* lse, int H, int N, int CQ,
    void* stream);
/* ---- strided variants ---------------------------------------------------
 * No counterpart in the reference: its SGLang backend copies q, k and v from
 * the model's token-major [1, N, H, 128] into head-major [H, N, 128] and the
 * output back (integrations/sglang/backend/t2t_attn.py:1161-1163,1194), four
 * full-size copies per call.  These entry points take the caller's tensors as
 * [H, N, 128] views: row n of head h at base + h * head_stride + n * row_stride
 * (elements; both multiples of 8, row stride >= 128, unit stride along the
 * 128 dims), so a token-major tensor is passed as (head_stride, row_stride) =
 * (128, H * 128).  Results are identical to the contiguous entry points. */
int t2t_project_strided(const void* x, int x_dtype, const void* U, void* out, int H, int N, int D,
                        int r, long long x_head_stride, long long x_row_stride, void* stream);
int t2t_kmm_run_strided(const void* QU, const void* KU, const void* V, int v_dtype,
                        long long v_head_stride, long long v_row_stride, const void* cq0,
                        const void* ck0, int32_t* qlab, void* cq2, int32_t* klab, float* ck2,
                        int32_t* qcounts, int32_t* qperm, int32_t* kcounts, int32_t* kperm,
                        void* V_sorted, void* sumv, float* lam, int H, int N, int CQ, int CK,
                        int pin_tail, void* ws, size_t ws_bytes, void* stream);
int t2t_kmm_run_vstats_gather_strided(const void* V, int v_dtype, long long v_head_stride,
                                      long long v_row_stride, const int32_t* kperm,
                                      const int32_t* kcounts, void* V_sorted, void* sumv,
                                      float* lam, int H, int N, int CK, void* ws,
                                      size_t ws_bytes, void* stream);
int t2t_tile_attn_exact_orig_gather_strided(
    const void* q, long long q_head_stride, long long q_row_stride, const void* k,
    long long k_head_stride, long long k_row_stride, const int32_t* kperm, const void* vp,
    int dtype, const int32_t* kcounts, const int32_t* unip, const int32_t* qperm,
    const int32_t* plan, void* out, long long out_head_stride, long long out_row_stride,
    float* lse, int H, int N, int CQ, void* stream);
int t2t_resid_merge_inplace_strided(void* out, long long out_head_stride, long long out_row_stride,
                                    const float* lse, const void* QU, const void* tiles,
                                    const int32_t* kcounts, const int32_t* unip,
                                    const int32_t* qlab, const int32_t* qperm, const float* lam,
                                    const float* tailw_dev, int dtype, int H, int N, int CQ,
                                    void* stream);

/* Residual + merge into the exact part held at the original rows of out
 * (S6); tiles from t2t_centroid_tiles.  With the two entries above, the
 * steps of t2t_tile_attn_run_planned one launch at a time. */
int t2t_resid_merge_inplace(void* out, const float* lse, const void* QU, const void* tiles,
                            const int32_t* kcounts, const int32_t* unip, const int32_t* qlab,
                            const int32_t* qperm, const float* lam, const float* tailw_dev,
                            int dtype, int H, int N, int CQ, void* stream);
/* Workspace bytes of t2t_tile_attn_run_planned: lse [H, N] fp32 and the
 * centroid tile image. */
size_t t2t_tile_attn_ws_bytes(int H, int N, int dtype);
/* Plan (when rebuild_plan != 0), exact attention, residual and merge in
 * one call: the exact part is written to the original rows of out and the
 * residual kernel merges into them in place.  Replaces
 * tile_attn_ext.run_planned, kernels/tile_attn/src/main.cpp:67-79; ws holds
 * lse and the centroid tiles (the reference allocates attn_out and lse per
 * call). */
int t2t_tile_attn_run_planned(const void* q, const void* kp, const void* vp, int dtype,
                              const int32_t* qcounts, const int32_t* kcounts,
                              const int32_t* unip, const void* QU, const void* cks,
                              const void* sumv, const float* lam,
                              const int32_t* qlab, const int32_t* qperm,
                              const float* tailw_dev, void* out,
                              int32_t* plan, int rebuild_plan,
                              int H, int N, int CQ,
                              void* ws, size_t ws_bytes, void* stream);

/* ---- init_state helpers ----------------------------------------------- */
/* labels[h, n] = nearest centroid of x[h, n] (||x||^2 - 2 x.c + ||c||^2,
 * fp32, lowest index on ties).  Replaces fast_assign,
 * operator/fast_assign.py:79-106.  D % 16 == 0, D <= 128, C <= 4096. */
int t2t_fast_assign(const void* x, const void* c, int32_t* labels,
                    int H, int N, int C, int D, void* stream);
/* Workspace bytes for t2t_det_centroid_update. */
size_t t2t_det_update_ws_bytes(int H, int N, int C);
/* Deterministic centroid update: int64 fixed-point (2^-20) sums per
 * cluster, mean in fp64, cast to fp16 through fp32; empty clusters keep old.
 * Replaces _det_centroid_update, integrations/sglang/backend/t2t_attn.py:242-257. */
int t2t_det_centroid_update(const void* x, const int32_t* labels, const void* old,
                            void* out, int32_t* counts,
                            int H, int N, int C, int D,
                            void* ws, size_t ws_bytes, void* stream);
/* Centroid update with value statistics: labels are grouped by a stable
 * counting sort; per cluster c with n rows, cent[h, c] = fp32 sum of x rows /
 * n (empty: fp32(old[h, c])) and, when v is given, vmean[h, c] = fp32 sum of
 * v rows / max(n, 1); counts[h, c] = n.  The sums run in row order (the
 * reference adds with fp32 atomics in no fixed order), so results agree with
 * it to fp32 rounding and are the same on every call.  x [H, N, D] fp16,
 * D == 32; v [H, N, 128] (v_dtype) or NULL; ws >= t2t_det_update_ws_bytes.
 * Replaces fused_update_vstats, operator/fused_update_vstats.py:72-115. */
int t2t_fused_update_vstats(const void* x, const int32_t* labels, const void* old,
                            const void* v, int v_dtype, float* cent, int32_t* counts,
                            float* vmean, int H, int N, int C, int D, void* ws,
                            size_t ws_bytes, void* stream);
/* G[h] = x[h]^T x[h] / N in fp64 ([H, D, D]); bf16 x is rounded to fp16
 * first.  Replaces the Gram products of online_u,
 * operator/deploy_step.py:135-137. D <= 128.  ws holds the per-split partial
 * products (t2t_gram_ws_bytes); the splits are summed in a fixed order, so the
 * result is the same on every call. */
size_t t2t_gram_ws_bytes(int H, int N, int D);
int t2t_gram(const void* x, int x_dtype, double* G, int H, int N, int D, void* ws,
             size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* T2T_HIP_H */
