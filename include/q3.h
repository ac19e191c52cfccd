/*
 * q3.h -- C ABI of the gfx950 Qwen3 greedy-decode kernels (libq3.so).
 *
 * Every launcher takes device pointers, sizes and the hipStream_t to enqueue
 * on; none allocates, synchronises or reads device memory from the host, so
 * each can be recorded by hipStreamBeginCapture.  Each returns 0 on success or
 * a hipError_t code (hipErrorInvalidValue for arguments that fail the
 * launcher's own checks); q3_error_string() names a code.  BF16 tensors are
 * raw uint16_t bits, row-major, contiguous unless a leading dimension is given.
 *
 * Reference interfaces replaced (file:line in alvinyuwen/starter):
 *   rms_norm            engine/kernels/rmsnorm.py:48   engine/engine.py:75
 *   add_norm            engine/kernels/fused.py:147    engine/engine.py:452
 *   norm_rope           engine/kernels/fused.py:222    engine/engine.py:458
 *   kv_to_cache         engine/kernels/fused.py:620    engine/engine.py:709-718
 *   skinny_linear{,_t,_split}  fused.py:365,441,525    engine/engine.py:431 (_linear)
 *   swiglu              engine/kernels/fused.py:872    engine/engine.py:464
 *   decode_attention{,_gqa,_split}  fused.py:849,712,826  engine/engine.py:720-732
 *   F.embedding / argmax / CUDA graph  engine/engine.py:768,812,833,1029-1065
 */
#ifndef Q3_H
#define Q3_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- x_mode: how the GEMV's input rows are formed -------------------------- */
#define Q3_X_PLAIN 0      /* x as given                                          */
#define Q3_X_NORM 1       /* x = RMSNorm(x, norm_w) computed in the prologue      */
#define Q3_X_EMBED_NORM 2 /* x = RMSNorm(embed[ids], norm_w); embed rows -> resid */

/* ---- epi: what the projection does with its FP32 sums ---------------------- */
#define Q3_EPI_STORE 0        /* y = bf16(acc)                                   */
#define Q3_EPI_RESID 1        /* y = bf16(y + bf16(acc)), y is the residual      */
#define Q3_EPI_SWIGLU 2       /* rows (gate_j, up_j) interleaved: y[j] = bf16(bf16(silu(g))*u) */
#define Q3_EPI_ARGMAX 3       /* per-workgroup (max bf16 logit, lowest index)    */
#define Q3_EPI_STORE_ARGMAX 4 /* both of the above                               */

#define Q3_GEMV_MAX_M 8
#define Q3_GEMV_MAX_NORM_K 4096

const char *q3_error_string(int code);

/* ---- step records of the greedy loop ---------------------------------------
 * A decode step's input token sits at position p = *pos; its logits predict
 * position q = p + 1.  Two optional device tables, indexed by q, let the
 * captured step replay a given token stream (teacher forcing) and record what
 * it computed, with no host copy per step:
 *   feed [npos, B] int64: the token fed at q, or -1 for the greedy choice;
 *   rec  [npos, B, 4] int32: {argmax, max logit, logit of the token fed at q,
 *        token fed at q}; logits as the FP32 bits of the BF16 value.
 * The LM-head argmax epilogues (q3_gemv, q3_skinny_argmax) write the fed
 * token's logit; q3_argmax_finish / q3_argmax_rows write the rest and feed the
 * next step.  The contest judge's replay (QWEN_ENGINE_CONTRACT.md "The
 * quality rule") needs exactly these two logits per position. */

/* Decode projection for M <= 8 rows: y = epi(x' . W^T), x' per x_mode.
 * Replaces _linear (engine.py:431) fused with the input norm (engine.py:790,
 * fused.py:115 add_norm) and the residual / SwiGLU / argmax that follow it.
 * W is [N, K]; K % 8 == 0; x, W 16-byte aligned; ldx % 8 == 0.  Modes:
 * X_EMBED_NORM with EPI_STORE; X_PLAIN with EPI_STORE or EPI_RESID; X_NORM
 * with any epilogue.  EPI_SWIGLU (N % 4 == 0) writes N/2 columns.  EPI_ARGMAX
 * writes part_val/part_idx [q3_gemv_partials(M, N, epi), M] for
 * q3_argmax_finish; with rec != NULL (argmax epilogues only; pos and feed then
 * required) it also writes the fed token's logit into the step record. */
int q3_gemv(int x_mode, const uint16_t *x, int ldx, const int64_t *ids,
            const uint16_t *norm_w, float eps, uint16_t *resid_out,
            const uint16_t *w, int M, int N, int K,
            int epi, uint16_t *y, int ldy, float *part_val, int *part_idx,
            const int64_t *pos, const int64_t *feed, int32_t *rec, int npos, hipStream_t stream);
int q3_gemv_partials(int M, int N, int epi);

/* Dense projection for any M on MFMA: y = epi(x . W^T), epi in {STORE, RESID,
 * SWIGLU}.  Replaces F.linear / cuBLAS in the prompt pass and at decode batches
 * above 64 (engine.py:439,450,803).  With q3_gemm_tiles_wide(M, N) the
 * 256 x 256-tile kernel (eight waves, direct global-to-LDS loads) runs, else
 * 16..128-row tiles.  K % 64 == 0; N % 4 == 0; ldx >= K, ldx % 8 == 0;
 * ldy % 4 == 0 (SWIGLU writes N/2 columns); x, W 16-byte and y 8-byte
 * aligned. */
int q3_gemm(const uint16_t *x, int ldx, const uint16_t *w, int M, int N, int K,
            int epi, uint16_t *y, int ldy, hipStream_t stream);
int q3_gemm_tiles_wide(int M, int N);
/* The same projection split along K on the 256 x 256-tile kernel, for prompts
 * too short to fill the CUs with whole tiles (the residual projections o and
 * down, engine.py:439,450, at 256-4095 tokens): FP32 partials
 * ws [splits, M, N] (splits * M * N floats), summed in split order by
 * q3_add_rmsnorm_partials.  q3_gemm_splits(M, N, K) is the split count where
 * that applies (else 0); q3_gemm_partials takes any splits in
 * 1..min(16, K / 64).  Same operand rules as q3_gemm; ws 16-byte aligned. */
int q3_gemm_splits(int M, int N, int K);
int q3_gemm_partials(const uint16_t *x, int ldx, const uint16_t *w, int M, int N, int K,
                     float *ws, int splits, hipStream_t stream);
/* q3_gemm with a workspace for the split tail of the 256 x 256 tiling: where
 * the tiles' last round on the device's CUs (one tile per CU) is at most half
 * full -- or, at 256+ tokens below q3_gemm_tiles_wide, where all the tiles
 * fill at most half the CUs -- those tiles are split along K and a second
 * kernel sums their FP32 partials in split order and applies the epilogue;
 * the other tiles are q3_gemm's, bit for bit.  ws holds q3_gemm_ws_floats(M, N, K) floats
 * (0: no split tail, and q3_gemm_ws is q3_gemm), 16-byte aligned.  Same
 * operand rules as q3_gemm. */
int q3_gemm_ws_floats(int M, int N, int K);
int q3_gemm_ws(const uint16_t *x, int ldx, const uint16_t *w, int M, int N, int K,
               int epi, uint16_t *y, int ldy, float *ws, hipStream_t stream);

/* act[r, j] = bf16(bf16(silu(g)) * u), (g, u) = gu[r, 2j], gu[r, 2j + 1]:
 * swiglu (fused.py:872; engine.py:464) on interleaved gate/up rows [rows, 2I].
 * I % 8 == 0; gu, act 16-byte aligned. */
int q3_swiglu_rows(const uint16_t *gu, uint16_t *act, int rows, int I, hipStream_t stream);

/* Decode projection for 1..64 rows on MFMA, weights streamed from HBM into
 * MFMA operands: y = epi(x . W^T), epi in {STORE, RESID, SWIGLU}.  Replaces
 * skinny_linear / skinny_linear_split (fused.py:365,525) at batch 9..64.
 * N % 64 == 0, K % 256 == 0.  Narrow N splits K over q3_skinny_splits(M, N, K)
 * workgroup columns; then ws must hold q3_skinny_ws_floats(M, N, K) floats and
 * a fixed-order reduce kernel (same stream) applies the epilogue. */
int q3_skinny(const uint16_t *x, int ldx, const uint16_t *w, int M, int N, int K,
              int epi, uint16_t *y, int ldy, float *ws, hipStream_t stream);
/* q3_skinny on weights repacked by q3_tile16: the same result, but every load
 * instruction reads 1 KB of contiguous weights. */
int q3_skinny_tiled(const uint16_t *x, int ldx, const uint16_t *wt, int M, int N, int K,
                    int epi, uint16_t *y, int ldy, float *ws, hipStream_t stream);
/* q3_skinny_tiled with no workspace argument and no allocation: the split-K
 * partials live in a file-scope device array of q3_skinny_scratch_floats()
 * floats (8 MiB) that each GPU holds for the life of the process.  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under hipGraph capture, serving loops and harnesses that forbid hipMalloc).
 * Same arguments and result, bit for bit, as q3_skinny_tiled; shapes whose
 * q3_skinny_ws_floats(M, N, K) exceeds the array return hipErrorOutOfMemory
 * before any launch.  Every call on one GPU shares that GPU's array (it keeps
 * the last call's partials; each call writes every partial it reads, so
 * nothing needs clearing): calls that overlap on one GPU -- concurrent
 * streams or threads -- race and must be serialised by the caller.  The
 * array's device address is looked up on a device's first call (make that
 * first call outside stream capture). */
int q3_skinny_tiled_noalloc(const uint16_t *x, int ldx, const uint16_t *wt, int M, int N, int K,
                            int epi, uint16_t *y, int ldy, hipStream_t stream);
int q3_skinny_scratch_floats(void);
/* q3_skinny_tiled without an epilogue: the FP32 split partials
 * ws [q3_skinny_splits(M, N, K), M, N] (one split included), for consumers
 * that sum them in split order: q3_add_rmsnorm_partials, q3_attn_decode. */
int q3_skinny_partials(const uint16_t *x, int ldx, const uint16_t *wt, int M, int N, int K,
                       float *ws, hipStream_t stream);
/* LM head + greedy choice for 1..64 rows on tiled weights (shapes with one
 * split, i.e. wide N): per-workgroup maxima of the BF16 logits, lowest index on
 * ties, into part_val/part_idx [N/64, M] for q3_argmax_finish (nparts = N/64);
 * logits [M, ld_logits] are stored too when non-NULL.  engine/engine.py:833. */
int q3_skinny_argmax(const uint16_t *x, int ldx, const uint16_t *wt, int M, int N, int K,
                     uint16_t *logits, int ld_logits, float *part_val, int *part_idx,
                     const int64_t *pos, const int64_t *feed, int32_t *rec, int npos,
                     hipStream_t stream);
/* Repack row-major W [N, K] (N % 16 == 0, K % 32 == 0) into 16-row tiles:
 * element (n, k) goes to ((n/16 * K/32 + k/32) * 64 + (k%32)/8 * 16 + n%16) * 8
 * + k%8, the MFMA A-operand order of one wave.  Setup-time layout change for
 * the weights uploaded at engine init (engine/engine.py:152-175 keeps its fused
 * weights row-major). */
int q3_tile16(const uint16_t *w, int N, int K, uint16_t *out, hipStream_t stream);
int q3_skinny_splits(int M, int N, int K);
int q3_skinny_ws_floats(int M, int N, int K);

/* Row RMSNorm: y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))).  rms_norm
 * (rmsnorm.py:48, engine.py:75).  cols % 8 == 0. */
int q3_rmsnorm(const uint16_t *x, int ldx, const uint16_t *w, uint16_t *y, int ldy,
               int rows, int cols, float eps, hipStream_t stream);

/* resid = bf16(resid + bf16(sum of the split partials ws [splits, rows, cols]
 * in split order)); y = RMSNorm(resid).  A split-K projection's residual
 * epilogue fused with the next add_norm (fused.py:147, 525-550).
 * cols % 8 == 0, cols <= 4096, splits <= 16. */
int q3_add_rmsnorm_partials(const float *ws, int splits, uint16_t *resid, const uint16_t *w,
                            uint16_t *y, int rows, int cols, float eps, hipStream_t stream);

/* sum = bf16(res + delta); y = RMSNorm(sum).  add_norm (fused.py:147).
 * sum_out may equal res (in place). */
int q3_add_rmsnorm(const uint16_t *res, const uint16_t *delta, uint16_t *sum_out,
                   uint16_t *y, const uint16_t *w, int rows, int cols, float eps,
                   hipStream_t stream);

/* resid = embed[ids]; y = RMSNorm(resid).  F.embedding + the first input norm
 * (engine.py:768,790). */
int q3_embed_rmsnorm(const int64_t *ids, const uint16_t *embed, uint16_t *resid,
                     uint16_t *y, const uint16_t *w, int rows, int cols, float eps,
                     hipStream_t stream);

/* Per-head QK RMSNorm + RoPE + KV-cache append for T tokens per sequence at
 * absolute positions start..start+T-1 (start read from *start_pos on the
 * device, plus start_offset).  qkv [B*T, ld_qkv] holds q | k | v;
 * q_out [B*T, Hq, D]; cache_k/v [B, Hkv, capacity, D].
 * norm_rope (fused.py:222) + kv_to_cache (fused.py:620). */
int q3_qk_norm_rope_kv(const uint16_t *qkv, int ld_qkv, const uint16_t *q_norm_w,
                       const uint16_t *k_norm_w, const uint16_t *cos_table,
                       const uint16_t *sin_table, const int64_t *start_pos, int start_offset,
                       uint16_t *q_out, uint16_t *cache_k, uint16_t *cache_v,
                       int B, int T, int Hq, int Hkv, int D, int capacity, float eps,
                       hipStream_t stream);

/* Split-K GQA decode attention for the token at position *pos (one query per
 * sequence), with the q/k RMSNorm + RoPE and the KV append of that token fused
 * in.  qkv [B, ld_qkv] (q | k | v), or, when qkv_part != NULL (qkv unused),
 * the projection's FP32 split partials [qkv_splits, B, ld_qkv] from
 * q3_skinny_partials, summed in split order and rounded to BF16;
 * cache_k/v [B, Hkv, capacity, 128].
 * Writes per-split partials part_acc [B, Hq, splits, 128] (FP32, unnormalised)
 * and part_ml [B, Hq, splits, 2] (running max, sum); q3_attn_merge finishes.
 * With splits == 1 and out != NULL the normalised output out [B, Hq*128]
 * (BF16, what q3_attn_merge would write) is written directly and the partial
 * buffers are unused.  Any splits >= 1 is valid; q3_attn_splits gives the
 * tuned count.  decode_attention_gqa / _split (fused.py:641-846). */
int q3_attn_decode(const uint16_t *qkv, int ld_qkv, const float *qkv_part, int qkv_splits,
                   const uint16_t *q_norm_w,
                   const uint16_t *k_norm_w, const uint16_t *cos_table,
                   const uint16_t *sin_table, const int64_t *pos,
                   uint16_t *cache_k, uint16_t *cache_v, float *part_acc, float *part_ml,
                   uint16_t *out,
                   int B, int Hq, int Hkv, int capacity, int splits, float eps, float scale,
                   hipStream_t stream);
/* Log-sum-exp merge of the splits: out [B, Hq*128] BF16 (fused.py:793-823). */
int q3_attn_merge(const float *part_acc, const float *part_ml, uint16_t *out,
                  int B, int Hq, int splits, hipStream_t stream);
/* Splits q3_attn_decode uses for a cache of `capacity` keys. */
int q3_attn_splits(int B, int Hkv, int capacity);
/* q3_attn_decode + q3_attn_merge in one launch (the same arithmetic, bit for
 * bit): the split units pass their partials to merging workgroups of the same
 * grid as flagged words in xbuf [q3_attn_xbuf_words(B, Hq, splits)] uint32,
 * 16-byte aligned.  A word's flag names (*pos, layer), layer < 64; the caller
 * zeroes xbuf before positions can repeat (a new prompt), so stale words never
 * match.  Applies when q3_attn_fused_grid(B, Hq, Hkv, capacity, splits) > 0 (2..16 splits,
 * a grid that is resident at once).  A merge that waits past 1 s sets *err = 1
 * (err may be NULL) and writes zeros.  Replaces fused.py:729-846 (split + merge
 * launches) with one. */
int q3_attn_decode_fused(const uint16_t *qkv, int ld_qkv, const float *qkv_part, int qkv_splits,
                         const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                         const uint16_t *cos_table, const uint16_t *sin_table, const int64_t *pos,
                         uint16_t *cache_k, uint16_t *cache_v, uint32_t *xbuf, uint16_t *out,
                         int B, int Hq, int Hkv, int capacity, int splits, int layer,
                         float eps, float scale, int *err, hipStream_t stream);
int q3_attn_fused_grid(int B, int Hq, int Hkv, int capacity, int splits);
int q3_attn_xbuf_words(int B, int Hq, int splits);
/* q3_attn_decode with two splits + q3_attn_merge in one launch, where
 * q3_attn_splits keeps one split for 65-128 (sequence, KV head) pairs (B=16 at
 * up to 4096 keys): one eight-wave workgroup per split on every CU; split 1
 * leaves its partial as flagged words in xbuf [q3_attn_xbuf_words(B, Hq, 2)]
 * and split 0 folds it into its own as the merge does.  Same bits as the two
 * launches; xbuf, layer and err as for q3_attn_decode_fused.  Applies when
 * q3_attn_pair_grid(B, Hq, Hkv, capacity) > 0.  Replaces fused.py:641-846
 * (decode_attention_gqa, or split + merge) with one launch. */
int q3_attn_decode_pair(const uint16_t *qkv, int ld_qkv, const float *qkv_part, int qkv_splits,
                        const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                        const uint16_t *cos_table, const uint16_t *sin_table, const int64_t *pos,
                        uint16_t *cache_k, uint16_t *cache_v, uint32_t *xbuf, uint16_t *out,
                        int B, int Hq, int Hkv, int capacity, int layer, float eps, float scale, int *err,
                        hipStream_t stream);
int q3_attn_pair_grid(int B, int Hq, int Hkv, int capacity);

/* The q|k|v projection (q3_gemv with x_mode X_NORM or X_EMBED_NORM and
 * EPI_STORE: x, ldx, ids, norm_w, eps, resid_out and w [N, K] as there, N =
 * (Hq + 2 Hkv) * 128) and q3_attn_decode_fused in one launch, for B = 1-2 rows
 * and K = 2560 or 512.  The projection's outputs go to the attention units as
 * flagged words qkv_x [B, N] uint32 (BF16 payload, the (*pos, layer) flag of
 * xbuf); each unit waits only for its own KV head's rows, with its first key
 * block already in flight.  Bit for bit the same out, cache rows and resid_out
 * as q3_gemv + q3_attn_decode_fused.
 * With w_o != NULL (B = 1, o [K, Hq * 128] with Hq * 128 = 4096 at K = 2560 or
 * 1024 at K = 512) the o projection and its residual join run in the same
 * launch: resid_out [K] += bf16(attention . w_oT), the bits of q3_gemv
 * (X_PLAIN, EPI_RESID); the attention output goes to it as flagged words o_x
 * [Hq * 128] uint32 (16-byte aligned) and out may be NULL.  In X_EMBED_NORM
 * mode the join starts from the embedding row (resid_out is then written once,
 * by the join).  With next_w != NULL (and w_o), the workgroups that wait for
 * the attention bring the first 1 KB of each row of the next launch's weights
 * next_w [next_rows, K] into the L2 of the XCD that will read them -- the
 * launch whose workgroup j reads rows next_group j .. next_group j +
 * next_group - 1 and runs on XCD j % 8 (q3_gemv's gate/up projection at one
 * row: next_group = next_rows / q3_gemv_partials(1, next_rows, Q3_EPI_SWIGLU))
 * -- a cache hint with no effect on results (next_w may be NULL).
 * The caller zeroes qkv_x, xbuf and o_x before positions can repeat (a new
 * prompt); eps is both norms' epsilon.  Applies when q3_qkv_attn_grid(B, Hq,
 * Hkv, capacity, splits, K, w_o != NULL) > 0 (what q3_attn_fused_grid admits,
 * and a grid resident at once).  A wait past 1 s sets *err = 1 (err may be
 * NULL).  Replaces reference engine/engine.py:665-736's first half of _block --
 * _linear(qkv) (:431-450), _norm_rope_pair + KV append (:458-462,
 * fused.py:553-638), _sdpa (:263-280), _linear(o) and the residual add of
 * _add_norm (:452-456) -- with one launch. */
int q3_qkv_attn(int x_mode, const uint16_t *x, int ldx, const int64_t *ids, const uint16_t *norm_w,
                float eps, uint16_t *resid_out, const uint16_t *w, int K, uint32_t *qkv_x,
                const uint16_t *q_norm_w, const uint16_t *k_norm_w, const uint16_t *cos_table,
                const uint16_t *sin_table, const int64_t *pos, uint16_t *cache_k, uint16_t *cache_v,
                uint32_t *xbuf, uint16_t *out, const uint16_t *w_o, uint32_t *o_x, const uint16_t *next_w,
                int next_rows, int next_group, int B, int Hq, int Hkv, int capacity, int splits, int layer,
                float scale, int *err, hipStream_t stream);
int q3_qkv_attn_grid(int B, int Hq, int Hkv, int capacity, int splits, int K, int with_o);

/* q3_qkv_attn at one row with the o projection (X_NORM on resid), preceded in
 * the same launch by the previous layer's down projection and its residual
 * join: resid' = bf16(resid + bf16(act . W_down^T)), the bits q3_gemv
 * (X_PLAIN, EPI_RESID) stores, handed to this layer's norm and o join as
 * flagged words rx [q3_down_rx_words(K)] (zeroed with the other exchange words
 * before positions can repeat).  resid then holds the residual after this
 * layer's o join, as after q3_gemv(down) then q3_qkv_attn.  W_down is [K, I];
 * act [I]; act, W_down, rx, w, norm_w, xbuf, w_o, o_x 16-byte aligned.
 * Applies when q3_down_qkv_attn_grid(Hq, Hkv, capacity, splits, K, I) > 0
 * (the whole grid resident at once).  Replaces engine/engine.py:735's down
 * _linear and the residual add that follows it (:736) together with the next
 * layer's first half of _block (q3_qkv_attn above): one kernel boundary fewer
 * per layer. */
int q3_down_qkv_attn(const uint16_t *act, const uint16_t *w_down, int I, uint32_t *rx, uint16_t *resid,
                     const uint16_t *norm_w, float eps, const uint16_t *w, int K, uint32_t *qkv_x,
                     const uint16_t *q_norm_w, const uint16_t *k_norm_w, const uint16_t *cos_table,
                     const uint16_t *sin_table, const int64_t *pos, uint16_t *cache_k, uint16_t *cache_v,
                     uint32_t *xbuf, const uint16_t *w_o, uint32_t *o_x, const uint16_t *next_w, int next_rows,
                     int next_group, int Hq, int Hkv, int capacity, int splits, int layer, float scale, int *err,
                     hipStream_t stream);
int q3_down_qkv_attn_grid(int Hq, int Hkv, int capacity, int splits, int K, int I);
int q3_down_rx_words(int K);

/* Causal prefill attention: q [B*T, Hq, 128] at positions start..start+T-1
 * against cache keys 0..start+T-1; out [B*T, Hq*128]; q and the caches
 * 16-byte, out 8-byte aligned.  SDPA is_causal / chunk mask
 * (engine.py:263-280,777-787). */
int q3_attn_prefill(const uint16_t *q, const uint16_t *cache_k, const uint16_t *cache_v,
                    uint16_t *out, int B, int T, int start, int Hq, int Hkv,
                    int capacity, float scale, hipStream_t stream);

/* Greedy token from the argmax partials (first index on ties), for each of the
 * B rows: tokens[b] (int64) = the token fed next, i.e. feed[q][b] when feed is
 * given and that entry is >= 0, else the argmax; rec[q][b] is filled when
 * given (the step records above; npos positions).  When pos != NULL, *pos
 * advances by one (the self-feeding graph's advance, engine.py:833-838): every
 * block reads it first and the last block to finish advances it, through
 * *counter (a device int, zero before the first call; not needed for B == 1). */
int q3_argmax_finish(const float *part_val, const int *part_idx, int nparts, int B,
                     int64_t *tokens, int64_t *pos, int *counter, const int64_t *feed,
                     int32_t *rec, int npos, hipStream_t stream);
/* The same over stored BF16 logits rows [B, V] (first index on ties); the fed
 * token's logit is read from the row. */
int q3_argmax_rows(const uint16_t *logits, int ld, int B, int V, int64_t *tokens,
                   int64_t *pos, int *counter, const int64_t *feed, int32_t *rec, int npos,
                   hipStream_t stream);

/* hipGraph capture of everything enqueued on `stream` between begin and end
 * (engine.py:1029-1065). */
int q3_graph_begin(hipStream_t stream);
int q3_graph_end(hipStream_t stream, void **exec_out);
int q3_graph_launch(void *exec, hipStream_t stream);
int q3_graph_destroy(void *exec);

#ifdef __cplusplus
}
#endif

#endif /* Q3_H */
