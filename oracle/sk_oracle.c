/*
 * sk_oracle.c - CPU restatement of the reference's decode-GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker.
 * The product (libstarter_amd.so) never links or calls it.
 *
 * Every function restates the arithmetic of a reference function, cited per
 * function.  bf16 values are raw uint16 bits; fp32 -> bf16 is round to nearest
 * even with NaN kept quiet, the rounding of torch's `.to(torch.bfloat16)` and
 * Triton's `.to(tl.bfloat16)`.
 *
 * Accumulation order: the reference's contract is "fp32 accumulation, one
 * rounding to bf16" (engine/kernels/gemm.py:87-101; its cuBLAS baseline
 * `a @ w.t()`, gemm.py:527) and its tests fix no summation order (tolerance
 * 0.02*max|ref| + 1e-3, tests/test_kernels.py:111-124).  This file fixes one:
 * eight interleaved fp32 partial sums p[j] = sum_{k = j mod 8} a*w in k order,
 * combined as ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)).  Deterministic, and
 * vectorisable without reassociation.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u; /* NaN -> canonical quiet NaN, as torch */
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float round_bf(float f) { return bf2f(f2bf(f)); }

/* fp32 dot product of two bf16 rows in the fixed 8-lane order above. */
static float dot_bf16(const uint16_t* a, const uint16_t* w, int K) {
  float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int k = 0;
  for (; k + 8 <= K; k += 8)
    for (int j = 0; j < 8; ++j) p[j] += bf2f(a[k + j]) * bf2f(w[k + j]);
  for (int j = 0; k < K; ++k, ++j) p[j] += bf2f(a[k]) * bf2f(w[k]);
  return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}

/* dot_bf16 of one weight row against rows m0..m0+mc-1 of A (mc <= 16), with
 * exactly dot_bf16's operation order per output; the weight row is converted
 * once per 8 columns and shared by the rows (cache reuse only). */
#define DOT_MC 16
static void dot_rows_bf16(const uint16_t* A, int64_t lda, int mc, const uint16_t* w, int K, float* out) {
  float p[DOT_MC][8];
  for (int m = 0; m < mc; ++m)
    for (int j = 0; j < 8; ++j) p[m][j] = 0.0f;
  int k = 0;
  for (; k + 8 <= K; k += 8) {
    float wf[8];
    for (int j = 0; j < 8; ++j) wf[j] = bf2f(w[k + j]);
    for (int m = 0; m < mc; ++m) {
      const uint16_t* a = A + (int64_t)m * lda + k;
      for (int j = 0; j < 8; ++j) p[m][j] += bf2f(a[j]) * wf[j];
    }
  }
  for (int m = 0; m < mc; ++m) {
    const uint16_t* a = A + (int64_t)m * lda;
    for (int kk = k, j = 0; kk < K; ++kk, ++j) p[m][j] += bf2f(a[kk]) * bf2f(w[kk]);
    out[m] = ((p[m][0] + p[m][1]) + (p[m][2] + p[m][3])) + ((p[m][4] + p[m][5]) + (p[m][6] + p[m][7]));
  }
}

/* bf16 round of fp32 value (exported for the tests' rounding checks). */
uint16_t oracle_f32_to_bf16(float f) { return f2bf(f); }

/* C[m,n] fp32 sums (before rounding): the reference's `acc` of
 * _skinny_kernel (gemm.py:87-97) / Gemv (gemm.py:233-244). */
void oracle_gemm_f32(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, float* C, int M, int N, int K,
                     int threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int n = 0; n < N; ++n)
    for (int m0 = 0; m0 < M; m0 += DOT_MC) {
      const int mc = M - m0 < DOT_MC ? M - m0 : DOT_MC;
      float d[DOT_MC];
      dot_rows_bf16(A + (int64_t)m0 * lda, lda, mc, W + (int64_t)n * ldw, K, d);
      for (int m = 0; m < mc; ++m) C[(int64_t)(m0 + m) * N + n] = d[m];
    }
}

/* C = bf16(A @ W^T): SkinnyMatmul (gemm.py:98-99, 104-112) and `a @ w.t()`. */
void oracle_gemm_bf16(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, uint16_t* C, int64_t ldc, int M,
                      int N, int K, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int n = 0; n < N; ++n)
    for (int m0 = 0; m0 < M; m0 += DOT_MC) {
      const int mc = M - m0 < DOT_MC ? M - m0 : DOT_MC;
      float d[DOT_MC];
      dot_rows_bf16(A + (int64_t)m0 * lda, lda, mc, W + (int64_t)n * ldw, K, d);
      for (int m = 0; m < mc; ++m) C[(int64_t)(m0 + m) * ldc + n] = f2bf(d[m]);
    }
}

/* _swiglu_epilogue (gemm.py:115-121) / _swiglu_kernel (swiglu.py:21-24):
 * bf16(g), bf16(u), s = bf16(g / (1 + exp(-g))) in fp32, out = bf16(s * u). */
static inline uint16_t swiglu_bf(float g, float u) {
  const float gb = round_bf(g), ub = round_bf(u);
  const float s = round_bf(gb / (1.0f + expf(-gb)));
  return f2bf(s * ub);
}

uint16_t oracle_swiglu_scalar(uint16_t g, uint16_t u) { return swiglu_bf(bf2f(g), bf2f(u)); }

/* swiglu over gu[M, 2I] = [g | u] (swiglu.py:27-33). */
void oracle_swiglu_bf16(const uint16_t* gu, int64_t ld_gu, uint16_t* out, int64_t ld_out, int M, int I) {
  for (int m = 0; m < M; ++m)
    for (int i = 0; i < I; ++i)
      out[(int64_t)m * ld_out + i] = swiglu_bf(bf2f(gu[(int64_t)m * ld_gu + i]), bf2f(gu[(int64_t)m * ld_gu + I + i]));
}

/* SkinnyGateUp (gemm.py:149-168, 171-181): g and u fp32-accumulated over the
 * gate rows Wg = wgu[0:I] and up rows Wu = wgu[I:2I] (model.py:116), then the
 * SwiGLU epilogue. */
void oracle_gateup_swiglu_bf16(const uint16_t* A, int64_t lda, const uint16_t* Wg, const uint16_t* Wu, int64_t ldw,
                               uint16_t* out, int64_t ldo, int M, int I, int K, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int n = 0; n < I; ++n)
    for (int m0 = 0; m0 < M; m0 += DOT_MC) {
      const int mc = M - m0 < DOT_MC ? M - m0 : DOT_MC;
      float g[DOT_MC], u[DOT_MC];
      dot_rows_bf16(A + (int64_t)m0 * lda, lda, mc, Wg + (int64_t)n * ldw, K, g);
      dot_rows_bf16(A + (int64_t)m0 * lda, lda, mc, Wu + (int64_t)n * ldw, K, u);
      for (int m = 0; m < mc; ++m) out[(int64_t)(m0 + m) * ldo + n] = swiglu_bf(g[m], u[m]);
    }
}

/* add_rms_norm (add_rmsnorm.py:15-29; cast placement rmsnorm.py:34-45):
 * s = bf16(x + y) -> xout; var = sum(s^2) / K; r = 1 / sqrt(var + eps);
 * out = bf16(w * bf16(s * r)).  The reference reduces sum(s^2) with an fp32
 * tree (tl.sum); its result sits within a few fp32 ulps of the exact sum, so
 * the oracle forms the sum exactly in fp64 and rounds it once to fp32 rather
 * than adopting one particular tree order. */
void oracle_add_rmsnorm_bf16(const uint16_t* x, const uint16_t* y, const uint16_t* w, float eps, uint16_t* xout,
                             uint16_t* out, int M, int K, int64_t ld) {
  for (int m = 0; m < M; ++m) {
    const uint16_t* xr = x + (int64_t)m * ld;
    const uint16_t* yr = y + (int64_t)m * ld;
    double sq = 0.0;
    for (int k = 0; k < K; ++k) {
      const uint16_t s = f2bf(bf2f(xr[k]) + bf2f(yr[k]));
      xout[(int64_t)m * ld + k] = s;
      const double sf = (double)bf2f(s);
      sq += sf * sf;
    }
    const float r = 1.0f / sqrtf((float)sq / (float)K + eps);
    for (int k = 0; k < K; ++k) {
      const float sf = bf2f(xout[(int64_t)m * ld + k]);
      out[(int64_t)m * ld + k] = f2bf(bf2f(w[k]) * round_bf(sf * r));
    }
  }
}

/* torch.argmax over bf16 logits (engine.py:207; topk.py:27-34): the first
 * column holding the row maximum; any NaN counts as the maximum (first NaN
 * wins); -0 == +0.  maxv = that value as fp32. */
void oracle_argmax_bf16(const uint16_t* L, int64_t ld, int M, int V, int64_t* ids, float* maxv) {
  for (int m = 0; m < M; ++m) {
    const uint16_t* r = L + (int64_t)m * ld;
    int best = 0;
    float bv = bf2f(r[0]);
    for (int n = 1; n < V && !isnan(bv); ++n) {
      const float v = bf2f(r[n]);
      if (isnan(v) || v > bv) {
        bv = v;
        best = n;
      }
    }
    ids[m] = best;
    maxv[m] = bv;
  }
}

/* lm_head + greedy token: argmax over bf16(A @ W^T) rows (model.py:210 then
 * engine.py:207), without keeping the logits. */
void oracle_lm_argmax_bf16(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, int M, int V, int K,
                           int64_t* ids, float* maxv, int threads) {
  for (int m = 0; m < M; ++m) {
    int64_t best = -1;
    float bv = 0.0f;
    int nan_seen = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
      int64_t lb = -1;
      float lv = 0.0f;
      int ln = 0;
#pragma omp for schedule(static)
      for (int n = 0; n < V; ++n) {
        const float v = bf2f(f2bf(dot_bf16(A + (int64_t)m * lda, W + (int64_t)n * ldw, K)));
        if (ln) continue;
        if (isnan(v)) {
          ln = 1;
          lb = n;
          lv = v;
        } else if (lb < 0 || v > lv) {
          lb = n;
          lv = v;
        }
      }
#pragma omp critical
      {
        if (lb >= 0) {
          if (ln) {
            if (!nan_seen || lb < best) {
              best = lb;
              bv = lv;
              nan_seen = 1;
            }
          } else if (!nan_seen && (best < 0 || lv > bv || (lv == bv && lb < best))) {
            best = lb;
            bv = lv;
          }
        }
      }
    }
    ids[m] = best;
    maxv[m] = bv;
  }
}

/* Per-head RMSNorm + rotary embedding + KV-cache write (engine/kernels/rope.py:
 * 17-30 cast placement, 140-188 layouts):
 *   n = bf16(x * r), r = 1/sqrt(mean(x^2) + eps) (sum of squares formed
 *   exactly, rounded once to fp32); y = bf16(w * n);
 *   o[i]      = bf16(bf16(y[i] * cos[i])           + bf16(-y[i+D/2] * sin[i]))
 *   o[i+D/2]  = bf16(bf16(y[i+D/2] * cos[i+D/2])   + bf16(y[i] * sin[i+D/2]))
 * qkv [B*T, ld] rows (b, t) hold HQ query heads, HKV key heads, HKV value
 * heads of width D; query heads go to q_out [B, HQ, T, D]; key heads
 * (normalised, rotated) and value heads (raw) to the caches [B, HKV, cap, D]
 * at slot pos[b] + t.  The rotary table row is that slot for a chain
 * (depth == NULL), or pos[b] + depth[t] for a draft tree, whose siblings
 * share one absolute position (rope.py:94-122, the DEPTH branch at 108-111). */
static void norm_rope_head(const uint16_t* x, const uint16_t* w, const uint16_t* c, const uint16_t* s, int D,
                           float eps, uint16_t* o) {
  double sq = 0.0;
  for (int i = 0; i < D; ++i) {
    const double v = (double)bf2f(x[i]);
    sq += v * v;
  }
  const float r = 1.0f / sqrtf((float)sq / (float)D + eps);
  const int H = D / 2;
  for (int i = 0; i < H; ++i) {
    const float y1 = round_bf(bf2f(w[i]) * round_bf(bf2f(x[i]) * r));
    const float y2 = round_bf(bf2f(w[i + H]) * round_bf(bf2f(x[i + H]) * r));
    o[i] = f2bf(round_bf(y1 * bf2f(c[i])) + round_bf(-y2 * bf2f(s[i])));
    o[i + H] = f2bf(round_bf(y2 * bf2f(c[i + H])) + round_bf(y1 * bf2f(s[i + H])));
  }
}

void oracle_qk_norm_rope_cache_bf16(const uint16_t* qkv, int64_t ld, const uint16_t* qw, const uint16_t* kw,
                                    const uint16_t* cosT, const uint16_t* sinT, const int32_t* pos, uint16_t* q_out,
                                    uint16_t* k_cache, uint16_t* v_cache, int B, int T, int HQ, int HKV, int D,
                                    int cap, float eps, const int32_t* depth) {
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t) {
      const uint16_t* row = qkv + (int64_t)(b * T + t) * ld;
      const int slot = pos[b] + t;
      const int angle = depth ? pos[b] + depth[t] : slot;
      const uint16_t* c = cosT + (int64_t)angle * D;
      const uint16_t* s = sinT + (int64_t)angle * D;
      for (int h = 0; h < HQ; ++h)
        norm_rope_head(row + (int64_t)h * D, qw, c, s, D, eps, q_out + ((int64_t)(b * HQ + h) * T + t) * D);
      for (int h = 0; h < HKV; ++h) {
        const int64_t cs = ((int64_t)(b * HKV + h) * cap + slot) * D;
        norm_rope_head(row + (int64_t)(HQ + h) * D, kw, c, s, D, eps, k_cache + cs);
        memcpy(v_cache + cs, row + (int64_t)(HQ + HKV + h) * D, (size_t)D * sizeof(uint16_t));
      }
    }
}

/* Decode attention (engine/kernels/attention.py:221-242, SDPA over the valid
 * keys): query row t of sequence b (head h, KV head h / (HQ/HKV)) attends to
 * keys 0 .. pos[b] + t (tree == NULL) or to keys < pos[b] and the draft keys
 * pos[b] + j with bit j of tree[t] set, with scores scale * q.k; softmax and the weighted sum
 * of V are formed in fp64 from the bf16 inputs (exact attention, no bf16
 * probabilities); out [B, R, HQ, D] fp32.  wabs (optional, same shape) gets
 * sum_n p_n |v_n| / sum_n p_n, the scale of the error that rounding the
 * probabilities to bf16 can cause.  OpenMP over (b, h). */
void oracle_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int32_t* pos,
                             const int64_t* tree, float* out, float* wabs, int B, int HQ, int HKV, int D, int R,
                             int cap, float scale, int threads) {
  const int G = HQ / HKV;
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(threads > 0 ? threads : 1)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < HQ; ++h) {
      const int kh = h / G;
      const uint16_t* K = k_cache + (int64_t)(b * HKV + kh) * cap * D;
      const uint16_t* V = v_cache + (int64_t)(b * HKV + kh) * cap * D;
      double* sc = (double*)malloc(sizeof(double) * (size_t)cap);
      double* acc = (double*)malloc(sizeof(double) * (size_t)D * 2);   /* [sum p v | sum p |v|] */
      for (int t = 0; t < R; ++t) {
        const uint16_t* qr = q + ((int64_t)(b * HQ + h) * R + t) * D;
        /* visible keys: 0 .. pos + t (chain), or keys < pos plus the draft
           keys pos + j whose bit j is set in tree[t] (attention.py:229-236) */
        int L = tree ? pos[b] + R : pos[b] + t + 1;
        if (L > cap) L = cap;
        double mx = -INFINITY;
        int any = 0;
        for (int n = 0; n < L; ++n) {
          const int rel = n - pos[b];
          const int vis = !tree || rel < 0 || ((tree[t] >> rel) & 1);
          if (!vis) {
            sc[n] = -INFINITY;
            continue;
          }
          double d = 0.0;
          for (int i = 0; i < D; ++i) d += (double)bf2f(qr[i]) * (double)bf2f(K[(int64_t)n * D + i]);
          sc[n] = d * (double)scale;
          if (sc[n] > mx) mx = sc[n];
          any = 1;
        }
        if (!any) L = 0;
        double den = 0.0;
        for (int i = 0; i < 2 * D; ++i) acc[i] = 0.0;
        for (int n = 0; n < L; ++n) {
          if (sc[n] == -INFINITY) continue;
          const double p = exp(sc[n] - mx);
          den += p;
          for (int i = 0; i < D; ++i) {
            const double v = (double)bf2f(V[(int64_t)n * D + i]);
            acc[i] += p * v;
            acc[D + i] += p * fabs(v);
          }
        }
        const int64_t o0 = ((int64_t)(b * R + t) * HQ + h) * D;
        for (int i = 0; i < D; ++i) {
          out[o0 + i] = L > 0 ? (float)(acc[i] / den) : 0.0f;
          if (wabs) wabs[o0 + i] = L > 0 ? (float)(acc[D + i] / den) : 0.0f;
        }
      }
      free(sc);
      free(acc);
    }
}

/* fast_topk (engine/kernels/topk.py:17-37): 2048 lanes sweep each row with
 * stride 2048 (strictly larger replaces: the first occurrence of a value keeps
 * its lane); rank k = largest remaining lane maximum, lowest column among the
 * lanes holding it; every lane holding that column is then cleared to -inf.
 * vals [N, K] fp32, idxs [N, K] int32. */
void oracle_topk_bf16(const uint16_t* L, int64_t ld, int N, int V, int K, float* vals, int32_t* idxs) {
  enum { LANES = 2048 };
  float best[LANES];
  int bidx[LANES];
  for (int r = 0; r < N; ++r) {
    const uint16_t* x = L + (int64_t)r * ld;
    for (int j = 0; j < LANES; ++j) {
      best[j] = -INFINITY;
      bidx[j] = 0;
    }
    for (int start = 0; start < V; start += LANES)
      for (int j = 0; j < LANES; ++j) {
        const int c = start + j;
        const float v = c < V ? bf2f(x[c]) : -INFINITY;
        if (v > best[j]) {
          best[j] = v;
          bidx[j] = c;
        }
      }
    for (int k = 0; k < K; ++k) {
      float m = -INFINITY;
      for (int j = 0; j < LANES; ++j)
        if (best[j] > m) m = best[j];
      int ci = 0x7FFFFFFF;
      for (int j = 0; j < LANES; ++j)
        if (best[j] == m && bidx[j] < ci) ci = bidx[j];
      vals[(int64_t)r * K + k] = m;
      idxs[(int64_t)r * K + k] = ci;
      for (int j = 0; j < LANES; ++j)
        if (bidx[j] == ci) best[j] = -INFINITY;
    }
  }
}
