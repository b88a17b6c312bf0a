/*
 * starter_amd.h - C ABI of the MI355X (gfx950) decode-GEMM hot path.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * enqueues its kernels on the given HIP stream and returns an sk_status code.
 * Nothing here allocates device memory, synchronises the host or depends on
 * host-side pointer values of the data, so every call can be captured into a
 * HIP graph and replayed.  Kernels never abort: a bad argument is reported as a
 * status code before anything is enqueued.
 *
 * Data layout (the reference's tensor layouts, engine/model.py:112-116 and
 * engine/kernels/gemm.py:365-369):
 *   A  [M, K]  bf16 row-major, row stride lda (elements)   - activations
 *   W  [N, K]  bf16 row-major, row stride ldw (elements)   - torch Linear weight
 *   C  [M, N]  bf16 row-major, row stride ldc (elements)   - C = A @ W^T
 * Arithmetic: bf16 inputs, fp32 accumulation, one rounding to bf16 (RNE) at
 * the end, as torch F.linear / the reference's tl.dot + `.to(bf16)` path.
 *
 * Alignment: A, W (and Wg/Wu) must be 16-byte aligned and lda/ldw multiples
 * of 8 elements; K must be a multiple of 32.  M may be 0: nothing is enqueued
 * and the data pointers may then be NULL.
 *
 * Workspace: ops that need device scratch take (ws, ws_bytes); query the size
 * with sk_workspace_bytes() for the same op/shape/config and allocate it once,
 * zero-filled (outside graph capture).  Its first bytes hold arrival counters
 * that let the last workgroup of a tile finish a split-K sum or an argmax in
 * the same kernel; every call leaves them at zero again, so the workspace is
 * reused without clearing.  Calls that share one workspace must not overlap
 * (same stream, or ordered by events).
 */
#ifndef STARTER_AMD_H
#define STARTER_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t sk_bf16; /* raw bfloat16 bits */

typedef enum sk_status {
  SK_OK = 0,
  SK_ERR_NULL = 1,        /* a required pointer is NULL */
  SK_ERR_SHAPE = 2,       /* M/N/K/stride out of the supported range */
  SK_ERR_ALIGN = 3,       /* pointer or stride misaligned for 16-byte loads */
  SK_ERR_WORKSPACE = 4,   /* workspace missing or smaller than required */
  SK_ERR_CONFIG = 5,      /* explicit config invalid for this shape */
  SK_ERR_LAUNCH = 6,      /* the HIP runtime rejected a launch */
  SK_ERR_DEVICE = 7,      /* no usable gfx950 device / runtime query failed */
  SK_ERR_ALIAS = 8,       /* an output overlaps an input it must not alias */
  SK_ERR_SCRATCH = 9      /* sk_gemm_bf16_noalloc: needs more than SK_NOALLOC_SCRATCH_BYTES */
} sk_status;

/* Static device scratch of sk_gemm_bf16_noalloc, per GPU (4 MiB). */
#define SK_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)

typedef enum sk_op {
  SK_OP_GEMM = 0,         /* C = A @ W^T                                  */
  SK_OP_GATEUP = 1,       /* Out = swiglu(A @ Wg^T, A @ Wu^T)             */
  SK_OP_LM_ARGMAX = 2,    /* ids/maxv = argmax_n bf16(A @ W^T)[m, n]      */
  SK_OP_ARGMAX = 3,       /* ids/maxv = argmax over given bf16 logits     */
  SK_OP_RMSNORM_GEMM = 4,       /* SK_OP_GEMM with A = rmsnorm(x + y)      */
  SK_OP_RMSNORM_GATEUP = 5,     /* SK_OP_GATEUP with A = rmsnorm(x + y)    */
  SK_OP_RMSNORM_LM_ARGMAX = 6,  /* SK_OP_LM_ARGMAX with A = rmsnorm(x + y) */
  /* Residual hand-off (a decode step split across kernel boundaries):      */
  SK_OP_RESID_GEMM = 7,         /* r_out = bf16(r + bf16(A @ W^T)), + sums  */
  SK_OP_PRE_GEMM = 8,           /* SK_OP_GEMM on rmsnorm(x) from the sums   */
  SK_OP_PRE_GATEUP = 9,         /* SK_OP_GATEUP on rmsnorm(x) from the sums */
  SK_OP_PRE_LM_ARGMAX = 10      /* SK_OP_LM_ARGMAX on rmsnorm(x) from sums  */
} sk_op;

typedef enum sk_path {
  SK_PATH_AUTO = 0,
  SK_PATH_MFMA = 1,       /* v_mfma_f32_16x16x32_bf16 tiles, 16 weight rows per wave tile */
  SK_PATH_GEMV = 2,       /* VALU v_dot2_f32_bf16, lanes span K, DPP/shuffle lane reduction */
  SK_PATH_MFMA_LDS = 3,   /* MFMA fed from LDS: weight rows loaded 1 KiB-contiguous, transposed in LDS */
  SK_PATH_WIDE = 4        /* up to 128 rows per workgroup: weight tile staged once in LDS for all rows */
} sk_path;

/*
 * Launch configuration.  The reference picks a Triton config per shape at
 * warmup (engine/kernels/gemm.py:381-401, 516-558); here the defaults come
 * from an offline-tuned table (sk_default_config) and an explicit config can
 * be passed to any op (NULL = default) to test or time one candidate.
 *
 *   path   : SK_PATH_MFMA, SK_PATH_MFMA_LDS or SK_PATH_GEMV
 *   waves  : wavefronts per workgroup; they split the workgroup's K slice and
 *            their fp32 partials are summed in LDS in fixed wave order
 *   ku     : K units per wave (MFMA: 32 columns; GEMV: 512 columns; WIDE: 8,
 *            every wave walks its slice in 256-column steps;
 *            MFMA_LDS: 8, 16, 32 or 40, i.e. 256, 512, 1024 or 1280 columns
 *            per wave; all but 512 stream 256-column chunks through an
 *            8-load ring)
 *   rows   : weight rows per workgroup tile (MFMA: 16 or 32; GEMV: 1..8;
 *            MFMA_LDS ring, i.e. ku != 16: any height 1..32, for gate/up
 *            1..48 gate rows and as many up rows, loaded as 16-row slabs
 *            whose rows past the tile are not read, so a height of N / 256
 *            gives every CU one tile; the whole-tile body (ku 16) and the
 *            residual hand-off ops on this path take 16 or 32, gate/up 16;
 *            SK_PATH_WIDE:
 *            1..96 rows, gate/up 1..48, with WN = 2 gate/up 1..32, with
 *            WN = 4 1..128 rows (eight waves 1..128), gate/up 17..64 (eight
 *            waves 17..48); with WN = 4 the residual hand-off producer takes
 *            a multiple of 16 rows and split >= 2, the consumers split 1)
 *   split  : global K splits; >1 writes fp32 partials to the workspace and
 *            the last workgroup to finish a tile sums them in fixed split
 *            order (no floating-point atomics, no second kernel)
 *   grid   : workgroups to launch (0 = derive from the device's CU count)
 *   groups : row groups (0 or 1 = none).  g > 1 (MFMA_LDS with 256- or
 *            1024-column waves, grid > 0 and a multiple of 8) splits the M
 *            rows into g groups of ceil(M / g) rows, each run by its own
 *            `grid` workgroups; the launch interleaves the groups in runs of
 *            8 workgroups, so workgroup b of every group lands on the same
 *            XCD (workgroups are dealt to the 8 XCDs round-robin) and reads
 *            the same weight tiles at about the same time, and that XCD's L2
 *            serves the later groups' reads.  Every group must hold a row.
 *            For M where one group of all rows would need more registers per
 *            wave than a ten-wave workgroup allows (M > 48 at K = 2560).
 *            SK_PATH_WIDE reads it as WN, the groups its waves form along
 *            the tile's weight slabs: 1 (every wave multiplies the whole
 *            tile for its activation tiles) or 2 (eight waves: two groups of
 *            slabs x four groups of activation tiles); 4 selects the body
 *            that stages the activation rows in LDS beside the weight tile
 *            (128-column steps; four waves of 32 activation rows, or eight
 *            whose pairs split each step's K columns).
 *
 * Rows per launch: at most 64 without row groups; with a configuration that
 * splits them into groups (compiled for groups of up to 32 rows), up to 128
 * rows in one launch, so each weight tile leaves HBM once for all of them.
 * A call with more rows runs as several launches of that many rows (64, or
 * 128 when the configuration for 128 rows has groups) plus the remainder,
 * each streaming the weights again (the hand-off ops take one launch's rows).
 * An explicit configuration applies to every launch of a call, the shorter
 * last one included; sk_check_config checks them all.  A shorter last launch
 * with fewer rows than the configuration has groups can give each one (e.g.
 * the one row left of 129) runs with as many groups as hold a row, so the
 * configuration sk_default_config returns for M rows suits every launch.
 */
typedef struct sk_config {
  int32_t path;
  int32_t waves;
  int32_t ku;
  int32_t rows;
  int32_t split;
  int32_t grid;
  int32_t groups;
} sk_config;

/* Library version, (major << 16) | minor. */
int sk_version(void);

/* Static message for a status code. */
const char* sk_strerror(int status);

/* Default launch configuration for op at (M, N, K) on a device with num_cu
 * compute units (pass 0 for the MI355X's 256).  Pure host logic.
 * Replaces the warmup-time pickers pick_matmul / pick_gateup / pick_normed
 * (engine/kernels/gemm.py:516-660). */
int sk_default_config(int op, int M, int N, int K, int num_cu, sk_config* out);

/* Check a config against op/shape limits (tile sizes, LDS, registers).
 * Pure host logic; returns SK_OK or SK_ERR_CONFIG/SK_ERR_SHAPE. */
int sk_check_config(int op, int M, int N, int K, const sk_config* cfg);

/* Workspace bytes op needs at (M, N, K) with cfg (NULL = default config). */
size_t sk_workspace_bytes(int op, int M, int N, int K, const sk_config* cfg);

/* C[M,N] = bf16(A[M,K] @ W[N,K]^T), fp32 accumulation.
 * Replaces SkinnyMatmul.__call__ / _skinny_kernel + _sum_kernel
 * (engine/kernels/gemm.py:349-378, 59-112) and Gemv without gate/up
 * (gemm.py:259-292); the reference's cuBLAS baseline is `a @ w.t()`
 * (gemm.py:527).  Call sites: mm["qkv"], mm["o"], mm["d"], mm["lm"]
 * (engine/model.py:202-210). */
int sk_gemm_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw,
                 sk_bf16* C, int64_t ldc, int M, int N, int K,
                 const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream);

/* sk_gemm_bf16 without a workspace argument: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as sk_gemm_bf16; the split-K arrival
 * counters and partials live in a static device array of
 * SK_NOALLOC_SCRATCH_BYTES (4 MiB) per GPU, held until the process ends.  The
 * call allocates nothing (no hipMalloc/hipFree, no allocating library call);
 * a plan that needs more scratch than that returns SK_ERR_SCRATCH before
 * anything is enqueued.  A split-K call first clears the counters it uses
 * (one small fill kernel).  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race and must
 * be ordered by the caller. */
int sk_gemm_bf16_noalloc(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw,
                         sk_bf16* C, int64_t ldc, int M, int N, int K,
                         const sk_config* cfg, hipStream_t stream);

/* Out[M,I] = bf16(bf16(silu(bf16 g)) * bf16 u), g = A @ Wg^T, u = A @ Wu^T,
 * both fp32-accumulated.  Wg/Wu are the gate and up halves of the fused
 * gate|up weight (engine/model.py:116: wgu[:I], wgu[I:]).
 * Replaces SkinnyGateUp.__call__ / _gateup_kernel + _sum_gateup_kernel +
 * _swiglu_epilogue (engine/kernels/gemm.py:315-346, 124-181, 115-121) and the
 * cuBLAS + swiglu pipeline (gemm.py:569, engine/kernels/swiglu.py:14-33).
 * Call site: mm["gu"] (engine/model.py:207). */
int sk_gateup_swiglu_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* Wg, const sk_bf16* Wu,
                          int64_t ldw, sk_bf16* Out, int64_t ldo, int M, int I, int K,
                          const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream);

/* ids[m] = min{ n : L[m,n] = max_n L[m,n] }, maxv[m] = float(max_n L[m,n]),
 * where L = bf16(A @ W^T) is never written to memory.  Lowest index wins on
 * exact ties, NaN compares above every number (torch.argmax semantics).
 * Replaces `mm["lm"](...)` followed by `logits.argmax(dim=-1)`
 * (engine/model.py:210, 375; engine/engine.py:207, 228) and rank 0 of
 * fast_topk (engine/kernels/topk.py:17-46).  Needs a workspace. */
int sk_lm_argmax_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw,
                      int64_t* ids, float* maxv, int M, int V, int K,
                      const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream);

/* Argmax over materialised bf16 logits L[M,V] (row stride ld, any alignment;
 * 16-byte aligned rows are read with vector loads), same tie and NaN rules as
 * sk_lm_argmax_bf16.  Replaces `logits.argmax(dim=-1)`
 * (engine/engine.py:207) and fast_topk rank 0 (engine/kernels/topk.py:17-37).
 * Needs a workspace (sk_workspace_bytes(SK_OP_ARGMAX, M, V, 0, NULL)). */
int sk_argmax_bf16(const sk_bf16* L, int64_t ld, int M, int V, int64_t* ids, float* maxv,
                   void* ws, size_t ws_bytes, hipStream_t stream);

/* xout = bf16(x + y); out = bf16(w * bf16(xout * rsqrt(mean(xout^2) + eps))).
 * All [M, K] with row stride ld; xout must not overlap x or y; out must not
 * overlap x, y or xout.  Replaces add_rms_norm (engine/kernels/add_rmsnorm.py:
 * 15-43), the unfused prologue of the qkv/gu/lm call sites
 * (engine/model.py:153, 166-170). */
int sk_add_rmsnorm_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w, float eps,
                        sk_bf16* xout, sk_bf16* out, int M, int K, int64_t ld,
                        hipStream_t stream);

/*
 * Residual add + RMSNorm fused in front of a projection: the call sites
 * mm["qkv"](x, y, w_norm, xout, w), mm["gu"](...) and mm["lm"](...)
 * (engine/model.py:202-210, built by pick_normed, engine/kernels/gemm.py:
 * 602-660; prologue _norm_stats/_normed_tile gemm.py:28-56 and
 * _row_rstd/_normed_row gemm.py:184-208).
 *   xout = bf16(x + y)                                  (written, bit-exact)
 *   A    = bf16(w_norm * bf16(xout * rstd)),  rstd = 1/sqrt(mean(xout^2) + eps)
 * then the projection of A exactly as sk_gemm_bf16 / sk_gateup_swiglu_bf16 /
 * sk_lm_argmax_bf16.  x, y and xout are [M, K] with row stride ldx; w_norm is
 * [K].  xout must not overlap x or y, and the outputs must not overlap x, y
 * or xout.  With a one-split GEMV configuration (the M <= 4 default) the
 * prologue runs inside the projection kernel (each workgroup normalises the
 * activation columns it loads; workgroup 0 writes xout); otherwise a separate
 * add+norm kernel writes A into the workspace first (on the MFMA paths every
 * workgroup would redo the whole block's normalisation, which measured slower
 * than the extra launch).  Query the workspace with SK_OP_RMSNORM_* ops.
 */
int sk_rmsnorm_gemm_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w_norm, float eps, sk_bf16* xout,
                         int64_t ldx, const sk_bf16* W, int64_t ldw, sk_bf16* C, int64_t ldc, int M, int N, int K,
                         const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream);

int sk_rmsnorm_gateup_swiglu_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w_norm, float eps,
                                  sk_bf16* xout, int64_t ldx, const sk_bf16* Wg, const sk_bf16* Wu, int64_t ldw,
                                  sk_bf16* Out, int64_t ldo, int M, int I, int K, const sk_config* cfg, void* ws,
                                  size_t ws_bytes, hipStream_t stream);

int sk_rmsnorm_lm_argmax_bf16(const sk_bf16* x, const sk_bf16* y, const sk_bf16* w_norm, float eps, sk_bf16* xout,
                              int64_t ldx, const sk_bf16* W, int64_t ldw, int64_t* ids, float* maxv, int M, int V,
                              int K, const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream);

/* Residual hand-off: the residual add and RMSNorm that sit between two
 * projections of a decoder layer (engine/model.py:202-210: xa = x + y before
 * mm["qkv"], xb = xa + o before mm["gu"], and the final norm before mm["lm"])
 * are split across the producing and the consuming projection kernels, so no
 * separate norm kernel runs between them.  No counterpart in the reference's
 * operator API (its prologue, gemm.py:28-56, recomputes every row's norm in
 * every tile); results follow the same casts:
 *
 * sk_gemm_residual_bf16 (producer, e.g. o_proj / down):
 *   y = bf16(A @ W^T) as sk_gemm_bf16 (not stored);
 *   r_out[m, n] = bf16(r[m, n] + y[m, n])            (bit-exact, the xout of
 *                                                      the reference prologue)
 *   sq[m * sq_ld + g] = sum of r_out[m, n]^2 over n in [16g, 16g+16) (fp32,
 *                       fixed order), sq_ld = ceil(N / 16).
 *   r and r_out are [M, N] with row stride ldr (r_out may equal r; neither may
 *   overlap A).  Query the workspace with SK_OP_RESID_GEMM.
 *
 * sk_rmsnorm_pre_{gemm,gateup_swiglu,lm_argmax}_bf16 (consumer):
 *   rstd[m] = 1/sqrt(sum_g sq[m * (K/16) + g] / K + eps)   (fixed order)
 *   A = bf16(w_norm * bf16(x * rstd))   with x = the producer's r_out
 *   then the projection of A as sk_gemm_bf16 / sk_gateup_swiglu_bf16 /
 *   sk_lm_argmax_bf16.  rstd may differ from a sequential sum's in the last
 *   fp32 bit, which can move rare elements of A by one bf16 ulp (within the
 *   projections' tolerance).  K must be a multiple of 16; the outputs must not
 *   overlap x or sq.  Query the workspace with SK_OP_PRE_* ops.
 *
 * Both run on the ring-streamed LDS-fed MFMA path (a configuration with
 * path 3 and ku 8, or ku 8 / 32 with any split for the producer); cfg NULL or
 * path AUTO picks the tuned configuration when it is such a path, else the
 * first ring configuration that fits.  M <= 128; a consumer holds all of K in
 * one workgroup (12 waves of 256 columns, K <= 3072, at M <= 16; 8 waves,
 * K <= 2048, above), so shapes with no such configuration return
 * SK_ERR_CONFIG (Qwen3-4B's consumers, K = 2560: M <= 16). */
int sk_gemm_residual_bf16(const sk_bf16* A, int64_t lda, const sk_bf16* W, int64_t ldw, const sk_bf16* r,
                          sk_bf16* r_out, int64_t ldr, float* sq, int M, int N, int K, const sk_config* cfg, void* ws,
                          size_t ws_bytes, hipStream_t stream);

int sk_rmsnorm_pre_gemm_bf16(const sk_bf16* x, int64_t ldx, const float* sq, const sk_bf16* w_norm, float eps,
                             const sk_bf16* W, int64_t ldw, sk_bf16* C, int64_t ldc, int M, int N, int K,
                             const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream);

int sk_rmsnorm_pre_gateup_swiglu_bf16(const sk_bf16* x, int64_t ldx, const float* sq, const sk_bf16* w_norm,
                                      float eps, const sk_bf16* Wg, const sk_bf16* Wu, int64_t ldw, sk_bf16* Out,
                                      int64_t ldo, int M, int I, int K, const sk_config* cfg, void* ws,
                                      size_t ws_bytes, hipStream_t stream);

int sk_rmsnorm_pre_lm_argmax_bf16(const sk_bf16* x, int64_t ldx, const float* sq, const sk_bf16* w_norm, float eps,
                                  const sk_bf16* W, int64_t ldw, int64_t* ids, float* maxv, int M, int V, int K,
                                  const sk_config* cfg, void* ws, size_t ws_bytes, hipStream_t stream);

/*
 * Attention side of the decode step (head width D = 128 only).
 *
 * sk_qk_norm_rope_cache_bf16: per-head RMSNorm + rotary embedding + KV-cache
 * write of one QKV projection buffer.  Replaces qk_norm_rope_cache
 * (engine/kernels/rope.py:140-188; cast placement rope.py:17-30):
 *   qkv     [B*T, ld_qkv] bf16, rows (b, t): HQ query heads | HKV key heads | HKV value heads
 *   q_norm_w, k_norm_w [D]; cos, sin [rope_rows, D] bf16 (model.py:85-100 tables)
 *   pos     [B] int32 device array: row (b, t) goes to slot pos[b] + t
 *   depth   NULL: row (b, t) rotates by position pos[b] + t (a chain); else
 *           [T] int32 device array: it rotates by pos[b] + depth[t] (draft-tree
 *           rows, siblings sharing a position; rope.py:94-122, the `depth=`
 *           argument of engine/model.py:204, 369-370)
 *   q_out   [B, HQ, T, D]; k_cache, v_cache [B, HKV, cap, D] (one layer)
 * Rows whose rotary position is outside the table, and key/value rows whose
 * slot is outside [0, cap), are skipped (pos and depth are device data, so the
 * host cannot check them).  No workspace.
 */
int sk_qk_norm_rope_cache_bf16(const sk_bf16* qkv, int64_t ld_qkv, const sk_bf16* q_norm_w, const sk_bf16* k_norm_w,
                               const sk_bf16* cos, const sk_bf16* sin, int rope_rows, const int32_t* pos,
                               const int32_t* depth, sk_bf16* q_out, sk_bf16* k_cache, sk_bf16* v_cache, int B, int T,
                               int HQ, int HKV, int D, int cap, float eps, hipStream_t stream);

/*
 * sk_decode_attention_bf16: split-K grouped-query flash-decoding with a
 * device-side length.  Replaces DecodeAttention (engine/kernels/attention.py:
 * 152-202, kernels 23-149), chain and draft-tree masks:
 *   q      [B, HQ, R, D] bf16; k_cache, v_cache [B, HKV, cap, D] bf16
 *   pos    [B] int32 device array: position of query row 0 of sequence b
 *   tree   NULL: row t sees keys 0 .. pos[b] + t (chain);  else [R] int64
 *          device array of ancestor bit masks: row t sees keys < pos[b] and
 *          key pos[b] + j (j < R) iff bit j of tree[t] is set
 *   out    [B, R, HQ, D] bf16 (rows (b, t) of [B*R, HQ*D])
 *   max_len: the longest sequence the caller will attend over (bounds the
 *            splits; 0 = cap); nsplit: key splits per (b, kv head), 0 = default
 * (HQ/HKV) * R must be at most 64; query rows are processed up to 16 per
 * workgroup (more rows stream the keys once per block of 16).  Scores and softmax
 * statistics in fp32, probabilities rounded to bf16 before the PV product,
 * fp32 accumulation (attention.py:9-11).  Needs a zero-filled workspace of
 * sk_decode_attention_workspace_bytes() bytes when it splits the keys; the
 * last workgroup of each (b, kv head, row block) merges the splits in the
 * same kernel and leaves the workspace counters at zero.
 */
size_t sk_decode_attention_workspace_bytes(int B, int HQ, int HKV, int D, int R, int cap, int max_len, int nsplit);

int sk_decode_attention_bf16(const sk_bf16* q, const sk_bf16* k_cache, const sk_bf16* v_cache, const int32_t* pos,
                             const int64_t* tree, sk_bf16* out, int B, int HQ, int HKV, int D, int R, int cap,
                             int max_len, float scale, int nsplit, void* ws, size_t ws_bytes, hipStream_t stream);

/*
 * sk_decode_attention_rope_bf16: sk_qk_norm_rope_cache_bf16 followed by
 * sk_decode_attention_bf16 (chain mask) in one launch, for the consecutive
 * calls qk_norm_rope_cache(...) and self.attention(q, k_cache, v_cache, pos,
 * out) of engine/model.py's decode layer.  No single reference counterpart.
 * Arguments as in those two calls (qkv rows (b, t), t < R; the query rows go
 * straight to the attention instead of a q buffer).  Each workgroup
 * normalises and rotates its own query rows with the same arithmetic as
 * sk_qk_norm_rope_cache_bf16 (same bits), and each workgroup whose key range
 * holds slot pos[b] + t writes that slot's K and V rows before it reads the
 * cache, so the outputs and the caches equal those of the two calls.  A query
 * row whose slot is outside the rotary table attends with a zero query.
 * Same workspace as sk_decode_attention_bf16 (same plan arguments).  out must
 * not overlap qkv or the caches.
 */
int sk_decode_attention_rope_bf16(const sk_bf16* qkv, int64_t ld_qkv, const sk_bf16* q_norm_w,
                                  const sk_bf16* k_norm_w, const sk_bf16* cos, const sk_bf16* sin, int rope_rows,
                                  float eps, sk_bf16* k_cache, sk_bf16* v_cache, const int32_t* pos, sk_bf16* out,
                                  int B, int HQ, int HKV, int D, int R, int cap, int max_len, float scale,
                                  int nsplit, void* ws, size_t ws_bytes, hipStream_t stream);

/*
 * sk_decode_attention_rope_tree_bf16: the same fused launch for a draft tree,
 * for qk_norm_rope_cache(..., depth=depth) followed by self.attention(q,
 * k_cache, v_cache, pos, out, tree) in the reference's verify forward
 * (engine/model.py:357, 369-370; rope.py:94-122 DEPTH path,
 * attention.py:245-259 masks).  tree [R]: the ancestor bit masks of
 * sk_decode_attention_bf16; depth [R]: row t is written to slot pos[b] + t
 * and rotated by position pos[b] + depth[t].  Both are read at every call
 * (a captured graph follows new trees).  Arguments otherwise as above.
 */
int sk_decode_attention_rope_tree_bf16(const sk_bf16* qkv, int64_t ld_qkv, const sk_bf16* q_norm_w,
                                       const sk_bf16* k_norm_w, const sk_bf16* cos, const sk_bf16* sin,
                                       int rope_rows, float eps, sk_bf16* k_cache, sk_bf16* v_cache,
                                       const int32_t* pos, const int64_t* tree, const int32_t* depth, sk_bf16* out,
                                       int B, int HQ, int HKV, int D, int R, int cap, int max_len, float scale,
                                       int nsplit, void* ws, size_t ws_bytes, hipStream_t stream);

/* Exact argmax plus approximate top-k over bf16 logits L[N, V] (row stride
 * ld) in one pass.  Replaces fast_topk (engine/kernels/topk.py:17-46) with
 * the same algorithm and results: 2048 lanes sweep each row with stride 2048,
 * lane j keeping the first occurrence of the largest value at columns
 * j, j+2048, ...; rank k is the largest remaining lane maximum (lowest column
 * on ties) and removes its lane.  vals [N, K] fp32, idxs [N, K] int32; rank 0
 * is the exact argmax.  1 <= K <= 64.  No workspace. */
int sk_topk_bf16(const sk_bf16* L, int64_t ld, int N, int V, int K, float* vals, int32_t* idxs, hipStream_t stream);

/* Out[M,I] = bf16(bf16(silu(g)) * u) for gu[M, 2I] = [g | u] (row stride ld_gu).
 * Replaces swiglu (engine/kernels/swiglu.py:14-33). */
int sk_swiglu_bf16(const sk_bf16* gu, int64_t ld_gu, sk_bf16* out, int64_t ld_out,
                   int M, int I, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* STARTER_AMD_H */
