// sk_attn.hip - decode attention side of the Qwen3 decode step on gfx950:
//   * per-head RMSNorm + rotary embedding + KV-cache write of the QKV
//     projection (engine/kernels/rope.py:94-188), and
//   * split-K grouped-query flash-decoding over the KV cache with a
//     device-side sequence length (engine/kernels/attention.py:23-202).
// Both are memory-bound: the first touches (HQ + 2*HKV) * D values per row,
// the second streams K and V of every valid position once per KV head.
#include "starter_amd.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include "sk_kernels.hpp"

namespace sk {

constexpr int HEAD_D = 128;   // head width of Qwen3 (the only one compiled)

// K/V blocks a wave keeps in flight beyond the one it processes (1 or 2).
// One: with two the first round of requests of the whole grid (24 MB at
// B = 16, position 1088) was served in no particular order and the last waves
// started late (B = 16 with two key splits: 17.6 us with two blocks ahead,
// 16.9 with one; pure streaming reads of the same 71 MB by 128 workgroups of
// 512 threads: 14.6 us with 8 loads per thread in flight, 19.1 with 16).
#ifndef SK_ATTN_AHEAD
#define SK_ATTN_AHEAD 1
#endif

// ---------------------------------------------------------------------------
// q/k RMSNorm + RoPE + cache write (rope.py:94-188 cast placement):
//   n = bf16(x * rsqrt(mean(x^2) + eps)); y = bf16(w * n)
//   o1 = bf16(bf16(y1 * cos1) + bf16(-y2 * sin1)); o2 = bf16(bf16(y2 * cos2) + bf16(y1 * sin2))
// with (y1, y2) = (y[i], y[i + D/2]).  One wave per head: lane i holds the
// rotation pair (i, i + 64), so the rotation needs no lane exchange.  Workgroup
// (row, head group): 4 waves, heads 4*hg .. 4*hg+3 of projection row (b, t);
// heads < HQ are query heads (to q_out), then HKV key heads (normalised and
// rotated into k_cache at slot pos[b] + t, their value heads copied raw to
// v_cache).  The rotary angle is that of position pos[b] + t (a chain), or of
// pos[b] + depth[t] when depth is given (draft-tree rows, whose siblings share
// one absolute position: rope.py:94-122).  A row whose rotary position is
// outside the table, or a key/value row whose slot is outside [0, cap), is
// skipped.
// ---------------------------------------------------------------------------
struct RopeArgs {
  const uint16_t* qkv;
  int64_t ld_qkv;
  const uint16_t* qw;
  const uint16_t* kw;
  const uint16_t* cos;
  const uint16_t* sin;
  int rope_rows;
  const int32_t* pos;
  const int32_t* depth;   // [T] rotary position offsets, or nullptr (chain: t)
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int T, HQ, HKV, cap;
  float eps;
};

// One wave, one head row src[0..127]: lane i returns the normalised and
// rotated pair (o1, o2) = output dims (i, i + 64).  Shared by the standalone
// kernel and the attention prologue, so both produce the same bits.
__device__ __forceinline__ void rope_head(const uint16_t* src, const uint16_t* w, const uint16_t* cs,
                                          const uint16_t* sn, float eps, int lane, uint16_t& o1, uint16_t& o2) {
  const float x1 = bf2f(src[lane]), x2 = bf2f(src[lane + 64]);
  const float ss = wave_sum(x1 * x1 + x2 * x2);
  const float r = 1.0f / sqrtf(ss / (float)HEAD_D + eps);
  const float y1 = round_bf(bf2f(w[lane]) * round_bf(x1 * r));
  const float y2 = round_bf(bf2f(w[lane + 64]) * round_bf(x2 * r));
  const float c1 = bf2f(cs[lane]), c2 = bf2f(cs[lane + 64]);
  const float s1 = bf2f(sn[lane]), s2 = bf2f(sn[lane + 64]);
  o1 = f2bf(round_bf(y1 * c1) + round_bf(-y2 * s1));
  o2 = f2bf(round_bf(y2 * c2) + round_bf(y1 * s2));
}

__global__ void __launch_bounds__(256) qk_norm_rope_kernel(RopeArgs a) {
  const int row = blockIdx.x;                       // (b, t)
  const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (head >= a.HQ + a.HKV) return;                 // wave-uniform
  const int b = row / a.T, t = row - (row / a.T) * a.T;
  const int p0 = a.pos[b];
  const int slot = p0 + t;
  const int angle = a.depth ? p0 + a.depth[t] : slot;
  if (angle < 0 || angle >= a.rope_rows) return;
  const bool is_q = head < a.HQ;
  if (!is_q && (slot < 0 || slot >= a.cap)) return;
  const uint16_t* src = a.qkv + (int64_t)row * a.ld_qkv + (int64_t)head * HEAD_D;
  uint16_t o1, o2;
  rope_head(src, is_q ? a.qw : a.kw, a.cos + (int64_t)angle * HEAD_D, a.sin + (int64_t)angle * HEAD_D, a.eps, lane,
            o1, o2);
  if (is_q) {
    uint16_t* dst = a.q_out + ((int64_t)(b * a.HQ + head) * a.T + t) * HEAD_D;
    dst[lane] = o1;
    dst[lane + 64] = o2;
  } else {
    const int kh = head - a.HQ;
    const int64_t cslot = ((int64_t)(b * a.HKV + kh) * a.cap + slot) * HEAD_D;
    a.k_cache[cslot + lane] = o1;
    a.k_cache[cslot + lane + 64] = o2;
    const uint16_t* vsrc = a.qkv + (int64_t)row * a.ld_qkv + (int64_t)(a.HQ + a.HKV + kh) * HEAD_D;
    a.v_cache[cslot + lane] = vsrc[lane];
    a.v_cache[cslot + lane + 64] = vsrc[lane + 64];
  }
}

// ---------------------------------------------------------------------------
// Split-K GQA flash-decoding (attention.py:23-149 numerics: scores and
// softmax statistics in fp32, probabilities rounded to bf16 before the PV
// product, fp32 accumulation, one normalisation at the end).
//
// Workgroup (b, kv head, split s): ATTN_WAVES waves stream keys
// [s*split_len, ...) clipped to the row's valid length pos[b] + t + 1, 16 keys
// per wave and block.  The scores of the KV head's query rows (QR = G*R of
// them, the columns of a 16-wide MFMA) come from v_mfma_f32_16x16x32_bf16 with
// the key rows as the A operand; each lane runs the online softmax of its own
// score column (4 keys of one row per block, the row max shared by the row's
// 4 lanes through permlane row swaps), and P.V runs on
// v_mfma_f32_16x16x16_bf16 with the probabilities as they sit in the score
// layout.  The waves' (m, l, acc) are merged in LDS in wave order.
// With several splits, the partial (m, l, acc) goes to the workspace and the
// last workgroup of the (b, kv head) to arrive merges the splits in split
// order (no second kernel).
// ---------------------------------------------------------------------------
struct AttnArgs {
  const uint16_t* q;        // [B, HQ, R, D]
  const uint16_t* k;        // [B, HKV, cap, D]
  const uint16_t* v;
  const int32_t* pos;       // [B]: position of query row 0
  const int64_t* tree;      // [R] ancestor bit masks, or nullptr for the chain (causal) mask
  uint16_t* out;            // [B, R, HQ, D]
  float* part_o;            // [B*HKV, NRB, S, QR, D]
  float* part_ml;           // [B*HKV, NRB, S, QR, 2]
  unsigned* tickets;        // [B*HKV, NRB]
  int HQ, HKV, R, G, cap, S, split_len, NRB;
  float scale;
  // ROPE instances: q rows and the new K/V rows come from the projection
  // buffer (rows (b, t)) through the per-head norm + rotary step.
  const uint16_t* qkv;
  int64_t ld_qkv;
  const uint16_t* qw;
  const uint16_t* kw;
  const uint16_t* cos;
  const uint16_t* sin;
  uint16_t* k_out;          // writable views of k / v
  uint16_t* v_out;
  int rope_rows;
  float eps;
  const int32_t* depth;     // ROPE with TREE: [R] rotary offsets (row t rotates by pos + depth[t])
  int rb_xcd;               // row blocks of one (b, kv head, split) launched 8 apart (one XCD)
};


// Reductions over lanes l, l^16, l^32, l^48 (the four 16-lane rows), by
// row swaps: every lane ends with the same value.
__device__ __forceinline__ float rows4_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int QR, int ATTN_WAVES, bool TREE, bool ROPE = false>
__global__ void __launch_bounds__(64 * ATTN_WAVES) decode_attn_kernel(AttnArgs a) {
  __shared__ float s_m[ATTN_WAVES][QR], s_l[ATTN_WAVES][QR];
  // (rows padded by 8 floats: the lanes of one f32x4 store hold 16 different
  // rows, and 128-float rows put all of them on the same banks)
  __shared__ __attribute__((aligned(16))) float s_acc[ATTN_WAVES][QR][HEAD_D + 8];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int dg = lane & 15, kr = lane >> 4;
  // Workgroup (b, kv head, row block, split): query rows rbk*QR .. +QR-1 of
  // the KV head's G*R rows (row = t*G + g), keys of split s.
  // With rb_xcd, launch position 8i + x runs row block i mod NRB of the
  // (b, kv head, split) unit 8(i / NRB) + x: workgroups are dealt to the 8
  // XCDs round-robin, so the row blocks of one unit run side by side on one
  // XCD and the later ones read the keys from its L2.
  const int S = a.S;
  int bq, s;
  if (a.rb_xcd) {
    const int i = blockIdx.x >> 3, x = blockIdx.x & 7;
    const int unit = 8 * (i / a.NRB) + x;
    s = unit % S;
    bq = (unit / S) * a.NRB + i % a.NRB;
  } else {
    bq = blockIdx.x / S;
    s = blockIdx.x - (blockIdx.x / S) * S;
  }
  const int bk = bq / a.NRB, rbk = bq - (bq / a.NRB) * a.NRB;
  const int b = bk / a.HKV, kh = bk - (bk / a.HKV) * a.HKV;
  const int rows = a.G * a.R;
  const int pos = a.pos[b];
  const int start = s * a.split_len;
  // keys this workgroup may touch: below the longest row's length and the cache
  const int end = min(min(start + a.split_len, pos + a.R), a.cap);

  // Query rows r = t*G + g (head kh*G + g, query row t) as the B operand of
  // v_mfma_f32_16x16x32_bf16: lane l supplies row l%16, dims 32s + 8*(l/16)
  // for K step s (rows >= QR are zero columns).
  const int r16 = lane & 15;
  bf16x8 qb[HEAD_D / 32];
  if constexpr (ROPE) {
    // Query rows through the norm + rotary step (one wave per row), into LDS.
    // Row t rotates by position pos + t (chain) or pos + depth[t] (draft
    // tree); a row whose rotary position is outside the table stays zero.
    __shared__ __attribute__((aligned(16))) uint16_t s_q[QR][HEAD_D];
    const int T = a.R;
    auto rot_of = [&](int t) { return TREE ? pos + a.depth[t] : pos + t; };
    for (int r = wave; r < QR; r += ATTN_WAVES) {   // wave-uniform
      const int gr = rbk * QR + r;
      const int t = gr / a.G, g = gr - (gr / a.G) * a.G;
      const int rot = gr < rows ? rot_of(t) : -1;
      uint16_t o1 = 0, o2 = 0;
      if (rot >= 0 && rot < a.rope_rows)
        rope_head(a.qkv + (int64_t)(b * T + t) * a.ld_qkv + (int64_t)(kh * a.G + g) * HEAD_D, a.qw,
                  a.cos + (int64_t)rot * HEAD_D, a.sin + (int64_t)rot * HEAD_D, a.eps, lane, o1, o2);
      s_q[r][lane] = o1;
      s_q[r][lane + 64] = o2;
    }
    // The new K/V rows of this (b, kv head) are written by every workgroup
    // whose key range holds their slot (the last split also takes slots past
    // the planned length), before any of its K/V loads: the stores are
    // complete (vmcnt 0) before the barrier.  Only those workgroups read
    // these slots, and each reads them after its own stores; several row
    // blocks write the same values, so a read never sees an older row.
    // Row t goes to wave (QR + t) mod ATTN_WAVES, so with fewer query rows
    // than waves the K/V rows run beside the query rows, not after them.
    constexpr int KV_WAVE0 = QR % ATTN_WAVES;
    for (int t = (wave - KV_WAVE0 + ATTN_WAVES) % ATTN_WAVES; t < T; t += ATTN_WAVES) {   // wave-uniform
      const int slot = pos + t, rot = rot_of(t);
      const bool mine = slot >= start && (slot < start + a.split_len || s == S - 1);
      if (mine && slot < a.cap && rot >= 0 && rot < a.rope_rows) {
        const uint16_t* row = a.qkv + (int64_t)(b * T + t) * a.ld_qkv;
        uint16_t o1, o2;
        rope_head(row + (int64_t)(a.HQ + kh) * HEAD_D, a.kw, a.cos + (int64_t)rot * HEAD_D,
                  a.sin + (int64_t)rot * HEAD_D, a.eps, lane, o1, o2);
        const int64_t cs = ((int64_t)bk * a.cap + slot) * HEAD_D;
        a.k_out[cs + lane] = o1;
        a.k_out[cs + lane + 64] = o2;
        const uint16_t* vsrc = row + (int64_t)(a.HQ + a.HKV + kh) * HEAD_D;
        a.v_out[cs + lane] = vsrc[lane];
        a.v_out[cs + lane + 64] = vsrc[lane + 64];
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const bool real = r16 < QR;
#pragma unroll
    for (int st = 0; st < HEAD_D / 32; ++st) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&s_q[min(r16, QR - 1)][32 * st + 8 * kr]);
      qb[st] = __builtin_bit_cast(bf16x8, real ? v : u32x4{0u, 0u, 0u, 0u});
    }
  } else {
    const int gr = rbk * QR + r16;
    const int t = gr / a.G, g = gr - (gr / a.G) * a.G;
    const bool real = r16 < QR && gr < rows;
    const uint16_t* qp =
        a.q + ((int64_t)(b * a.HQ + kh * a.G + min(g, a.G - 1)) * a.R + min(t, a.R - 1)) * HEAD_D + 8 * kr;
#pragma unroll
    for (int st = 0; st < HEAD_D / 32; ++st) {
      const u32x4 v = ld16(qp + 32 * st);
      qb[st] = __builtin_bit_cast(bf16x8, real ? v : u32x4{0u, 0u, 0u, 0u});
    }
  }
  // Lane l owns query row l%16 (its MFMA column) and, in each 16-key block,
  // keys 4*(l/16) .. +3 of that row; the 4 lanes of a row share its running
  // max and keep partial sums.  acc[c][k] = O[row l%16][dim 8*(4*(l/16)+k) + c].
  // Visibility of key n to the row: keys before pos always; key pos + j
  // (j < R) iff j <= t (chain) or bit j of tree[t] is set (draft tree).
  const int my_gr = rbk * QR + r16;
  const bool my_real = r16 < QR && my_gr < rows;
  const int my_t = my_gr / a.G;
  const int row_lim = my_real ? pos + my_t : -1;   // last visible key of the row (chain)
  long long row_tree = 0ll;
  if constexpr (TREE) row_tree = my_real ? (long long)a.tree[min(my_t, a.R - 1)] : 0ll;

  float m = -INFINITY, l = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Wave w processes keys n0 + 16w .. n0 + 16w + 15 of each block of
  // 16 * ATTN_WAVES keys.  K and V are loaded row-contiguously (one load = 4
  // whole 256-byte rows per wave): load j of lane l holds dims 8*(l%16) .. +7
  // of key 4j + l/16 for K and of key 4*(l/16) + j for V.
  //  * Scores: S^T[key][row] = K[16 keys, 128] . Q^T by four MFMAs with K as
  //    the A operand (lane l: key l%16, dims 32s + 8*(l/16)); the wave's K rows
  //    pass through its own LDS tile (rows padded to 288 bytes, so neither the
  //    row writes nor the column reads conflict) into that layout.  Lane l then
  //    holds keys 4*(l/16) + i (i < 4) of query row l%16.
  //  * P.V: lane l's V loads hold keys 4*(l/16) + j, the keys of its scores.
  // The next blocks' rows are loaded while the current one is processed
  // (keys past `end` reload the last valid row and are masked).
  constexpr int KPITCH = 2 * HEAD_D + kRowPad;
  __shared__ __attribute__((aligned(16))) char s_k[ATTN_WAVES][16 * KPITCH];
  char* const ktile = s_k[wave];
  const int64_t kv_row0 = (int64_t)bk * a.cap;
  const int step = 16 * ATTN_WAVES;
  // K and V rows are read once per launch: non-temporal loads keep them from
  // displacing other lines in L2 (17.6 vs 19.1 us at B = 16, position 1088).
  auto load_block = [&](int n0, u32x4* kf, u32x4* vv) {
    const int base = n0 + 16 * wave;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = max(min(base + 4 * j + kr, end - 1), 0);
      kf[j] = ld16_stream(a.k + (kv_row0 + kk) * HEAD_D + 8 * dg);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kv = max(min(base + 4 * kr + j, end - 1), 0);
      vv[j] = ld16_stream(a.v + (kv_row0 + kv) * HEAD_D + 8 * dg);
    }
  };
  // Two blocks in flight beyond the one being processed.  Three buffers with
  // fixed roles rotate through a three-block loop body with a single exit,
  // so no buffer is ever copied (a loop-carried copy makes the compiler wait
  // for the prefetched loads at the end of every iteration).  Blocks past
  // `end` in the last iteration are fully masked; their loads read the last
  // valid row (one cached line).
  // MASKED: the block may hold keys a row must not see; blocks wholly below
  // min(end, pos) need no masks (every real row sees every key below pos, and
  // padding rows are never written out).
  auto process = [&](int n0, const u32x4* kf, const u32x4* vv, auto masked) {
    constexpr bool MASKED = decltype(masked)::value;
    // K rows into the wave's tile and back in the A-operand layout (LDS
    // operations of one wave execute in order; the compiler keeps these
    // accesses in program order since their addresses may alias).
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(ktile + (4 * j + kr) * KPITCH + 16 * dg) = kf[j];
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < HEAD_D / 32; ++st) {
      const u32x4 ka = *reinterpret_cast<const u32x4*>(ktile + r16 * KPITCH + 64 * st + 16 * kr);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka), qb[st], sacc, 0, 0, 0);
    }
    const int key0 = n0 + 16 * wave + 4 * kr;   // keys key0 .. key0+3 of this lane's row
    float sc[4];
    float mx = m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float dot = sacc[j] * a.scale;
      if constexpr (MASKED) {
        const int key = key0 + j;
        bool vis;
        if constexpr (TREE) {
          const int rel = key - pos;
          vis = row_lim >= 0 && (rel < 0 || (rel < a.R && ((row_tree >> rel) & 1ll)));
        } else {
          vis = key <= row_lim;
        }
        sc[j] = (key < end && vis) ? dot : -INFINITY;
      } else {
        sc[j] = dot;
      }
      mx = fmaxf(mx, sc[j]);
    }
    mx = rows4_max(mx);
    const float msafe = mx == -INFINITY ? 0.f : mx;
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = __expf(sc[j] - msafe);
    // Rescale only when some row's max moved (alpha == 1 elsewhere, so the
    // skipped multiplications are exact).
    if (__builtin_amdgcn_ballot_w64(mx != m)) {   // wave-uniform
      const float alpha = __expf(m - msafe);
      l *= alpha;
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] *= alpha;
    }
    l += (p[0] + p[1]) + (p[2] + p[3]);
    m = mx;
    // P.V on MFMA: O^T[dims][rows] += V^T[dims][16 keys] . P^T[16 keys][rows].
    // B = the probabilities as they sit (lane l: row l%16, keys 4*(l/16)+j),
    // rounded to bf16 (RNE) as the reference's tl.dot does; A for dim offset
    // c = V[keys 4*(l/16)+j][8*(l%16) + c], key pairs packed by v_perm.
    const bf16x2 p01 = {(__bf16)p[0], (__bf16)p[1]}, p23 = {(__bf16)p[2], (__bf16)p[3]};
    const s16x4 pb = __builtin_bit_cast(s16x4, u32x2{__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23)});
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t sel = h ? 0x07060302u : 0x05040100u;
        const u32x2 vt = {__builtin_amdgcn_perm(vv[1][c4], vv[0][c4], sel), __builtin_amdgcn_perm(vv[3][c4], vv[2][c4], sel)};
        acc[2 * c4 + h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, vt), pb, acc[2 * c4 + h], 0, 0, 0);
      }
  };
  u32x4 kA[4], vA[4], kB[4], vB[4], kC[4], vC[4];   // the 4 K and 4 V loads of a block
  const int unmasked_end = min(end, pos);   // keys below it need no masks
  // Per wave (uniform): its 16 keys of block nb are nb + 16*wave .. +15.  A
  // wave whose keys all lie at or past `end` skips the block (every score
  // would be masked: p = 0, m and l unchanged, so skipping is exact); one
  // whose keys all lie below `unmasked_end` takes the body without masks.
  auto run = [&](int nb, const u32x4* kf, const u32x4* vv) {
    const int wk = nb + 16 * wave;
    if (wk >= end) return;
    if (wk + 16 <= unmasked_end) process(nb, kf, vv, std::false_type{});
    else process(nb, kf, vv, std::true_type{});
  };
#if SK_ATTN_AHEAD == 1
  // One block in flight beyond the one being processed (two buffers).
  (void)kC;
  (void)vC;
  if (start < end) load_block(start, kA, vA);
  for (int n0 = start; n0 < end; n0 += 2 * step) {
    load_block(n0 + step, kB, vB);
    __builtin_amdgcn_sched_barrier(0);
    run(n0, kA, vA);
    __builtin_amdgcn_sched_barrier(0);
    load_block(n0 + 2 * step, kA, vA);
    __builtin_amdgcn_sched_barrier(0);
    run(n0 + step, kB, vB);
    __builtin_amdgcn_sched_barrier(0);
  }
#else
  if (start < end) {
    load_block(start, kA, vA);
    load_block(start + step, kB, vB);
  }
  // The scheduling fences keep every prefetch ahead of the block it overlaps.
  for (int n0 = start; n0 < end; n0 += 3 * step) {
    load_block(n0 + 2 * step, kC, vC);
    __builtin_amdgcn_sched_barrier(0);
    run(n0, kA, vA);
    __builtin_amdgcn_sched_barrier(0);
    load_block(n0 + 3 * step, kA, vA);
    __builtin_amdgcn_sched_barrier(0);
    run(n0 + step, kB, vB);
    __builtin_amdgcn_sched_barrier(0);
    load_block(n0 + 4 * step, kB, vB);
    __builtin_amdgcn_sched_barrier(0);
    run(n0 + 2 * step, kC, vC);
    __builtin_amdgcn_sched_barrier(0);
  }
#endif

  // Per wave: the row sums of the 4 lanes of each row, then the waves'
  // results merge in LDS in wave order.
  const float lw = rows4_sum(l);
  if (r16 < QR) {
    if (kr == 0) {
      s_m[wave][r16] = m;
      s_l[wave][r16] = lw;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float* dst = &s_acc[wave][r16][8 * (4 * kr + k)];
      *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0][k], acc[1][k], acc[2][k], acc[3][k]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4][k], acc[5][k], acc[6][k], acc[7][k]};
    }
  }
  __syncthreads();
  // Per row: the merged max, each wave's weight and the merged sum (waves in
  // order); then every output of the real rows combines the waves' partial
  // accumulators with those weights.
  __shared__ float s_w[ATTN_WAVES][QR], s_rowM[QR], s_rowL[QR];
  if (threadIdx.x < QR) {
    const int r = threadIdx.x;
    float M = -INFINITY;
#pragma unroll
    for (int wv = 0; wv < ATTN_WAVES; ++wv) M = fmaxf(M, s_m[wv][r]);
    float L = 0.f;
#pragma unroll
    for (int wv = 0; wv < ATTN_WAVES; ++wv) {
      const float w = s_m[wv][r] == -INFINITY ? 0.f : __expf(s_m[wv][r] - M);
      s_w[wv][r] = w;
      L += w * s_l[wv][r];
    }
    s_rowM[r] = M;
    s_rowL[r] = L;
  }
  __syncthreads();
  const bool single = (S == 1);
  const int nreal = min(QR, rows - rbk * QR);   // rows of this block that exist
  for (int idx = threadIdx.x; idx < nreal * HEAD_D; idx += 64 * ATTN_WAVES) {
    const int r = idx / HEAD_D, d = idx - (idx / HEAD_D) * HEAD_D;
    float O = 0.f;
#pragma unroll
    for (int wv = 0; wv < ATTN_WAVES; ++wv) O += s_w[wv][r] * s_acc[wv][r][d];
    const float L = s_rowL[r];
    const int gr = rbk * QR + r;
    const int t = gr / a.G, g = gr - (gr / a.G) * a.G;
    if (single) {
      a.out[((int64_t)(b * a.R + t) * a.HQ + kh * a.G + g) * HEAD_D + d] = f2bf(L > 0.f ? O / L : 0.f);
    } else {
      const int64_t pr = ((int64_t)bq * S + s) * QR + r;
      store_agent(&a.part_o[pr * HEAD_D + d], O);
      if (d == 0) {
        store_agent(&a.part_ml[2 * pr], s_rowM[r]);
        store_agent(&a.part_ml[2 * pr + 1], L);
      }
    }
  }
  if (single) return;

  // Last workgroup of this (b, kv head) merges the splits in split order.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) s_last = take_ticket(&a.tickets[bq], (unsigned)S) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  // Each output loads its splits' (m, l, o) in batches of MB, all loads of a
  // batch issued before any arithmetic (one memory round trip per batch, not
  // one per split); the merge itself runs in split order 0..S-1.
  constexpr int MB = 4;
  for (int idx = threadIdx.x; idx < QR * HEAD_D; idx += 64 * ATTN_WAVES) {
    const int r = idx / HEAD_D, d = idx - (idx / HEAD_D) * HEAD_D;
    const int gr = rbk * QR + r;
    const int t = gr / a.G, g = gr - (gr / a.G) * a.G;
    if (gr >= rows) continue;
    const int64_t pr0 = (int64_t)bq * S * QR + r;   // split sp: pr0 + sp * QR
    float M = -INFINITY;
    for (int s0 = 0; s0 < S; s0 += MB) {
      float ms[MB];
#pragma unroll
      for (int k = 0; k < MB; ++k) ms[k] = load_agent(&a.part_ml[2 * (pr0 + (int64_t)min(s0 + k, S - 1) * QR)]);
#pragma unroll
      for (int k = 0; k < MB; ++k) M = fmaxf(M, ms[k]);   // repeats of split S-1 change nothing
    }
    float L = 0.f, O = 0.f;
    for (int s0 = 0; s0 < S; s0 += MB) {
      float ms[MB], ls[MB], os[MB];
#pragma unroll
      for (int k = 0; k < MB; ++k) {
        const int64_t pr = pr0 + (int64_t)min(s0 + k, S - 1) * QR;
        ms[k] = load_agent(&a.part_ml[2 * pr]);
        ls[k] = load_agent(&a.part_ml[2 * pr + 1]);
        os[k] = load_agent(&a.part_o[pr * HEAD_D + d]);
      }
#pragma unroll
      for (int k = 0; k < MB; ++k) {
        if (s0 + k >= S) break;
        const float w = ms[k] == -INFINITY ? 0.f : __expf(ms[k] - M);
        L += w * ls[k];
        O += w * os[k];
      }
    }
    a.out[((int64_t)(b * a.R + t) * a.HQ + kh * a.G + g) * HEAD_D + d] = f2bf(L > 0.f ? O / L : 0.f);
  }
}

}  // namespace sk

namespace {

constexpr int kAttnMaxRows = 64;   // (HQ/HKV) * R

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
int cdiv(int a, int b) { return (a + b - 1) / b; }
size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Waves per workgroup, 16 keys each per block (at B = 16, ~1.1k keys, one
// split: 8 waves 15.4 us, 4 waves 15.9 us).
constexpr int kAttnWaves = 8;

struct AttnPlan {
  int QR = 0, NRB = 0, S = 0, split_len = 0;
  size_t tickets = 0, part_o = 0, part_ml = 0, need = 0;
};

// Splits: the keys of one (b, kv head) pair are split when B*HKV alone
// leaves most compute units idle, each split a whole number of workgroup
// blocks (16 keys per wave) of the longest sequence the plan will see.
int attn_plan(int B, int HQ, int HKV, int D, int R, int cap, int max_len, int nsplit, AttnPlan* p) {
  if (B < 1 || HKV < 1 || HQ < HKV || HQ % HKV != 0 || R < 1 || cap < 1 || D != sk::HEAD_D) return SK_ERR_SHAPE;
  const int G = HQ / HKV;
  const int rows = G * R;
  if (rows > kAttnMaxRows) return SK_ERR_SHAPE;
  // Query rows per workgroup: up to 16, the columns of the MFMA tiles (the
  // per-lane state does not grow with them); more rows take several row
  // blocks, each streaming the keys once more.  The smaller instances keep
  // less LDS and epilogue work (B = 16, 1088 keys, R = 2: 17.1 us with 8
  // rows, 17.8 us with 16).
  p->QR = rows <= 4 ? 4 : rows <= 8 ? 8 : 16;
  p->NRB = cdiv(rows, p->QR);
  const int work = max_len > 0 && max_len < cap ? max_len : cap;
  const int block = 16 * kAttnWaves;   // keys per workgroup block
  const int blocks = cdiv(work, block);
  int S = nsplit;
  if (S <= 0) {
    // Decode (one query row per sequence): about one workgroup per CU of an
    // MI355X (B = 16, 8 KV heads, 1089 keys: 17.4 us in one split per pair,
    // 16.8 in two; B = 4: 10.9 -> 9.6 us; decode step 5896 -> 5978 tok/s).
    // Verify rows (R > 1, one or more 16-row blocks per pair): about one per
    // two CUs, where a second split cost the 16 x 8 verify pass 10%.
    const long pairs = (long)B * HKV;
    const long target = R == 1 ? 256 : 128;
    S = (int)((target + pairs - 1) / pairs);
    if (S > 32) S = 32;
  }
  if (S > blocks) S = blocks;
  if (S < 1) S = 1;
  p->split_len = cdiv(blocks, S) * block;
  p->S = cdiv(work, p->split_len);
  if (p->S == 1) {
    p->need = 0;
    return SK_OK;
  }
  const size_t pairs = (size_t)B * HKV * p->NRB;
  p->tickets = align256(pairs * sizeof(unsigned));
  p->part_o = pairs * p->S * p->QR * sk::HEAD_D * sizeof(float);
  p->part_ml = pairs * p->S * p->QR * 2 * sizeof(float);
  p->need = p->tickets + align256(p->part_o) + p->part_ml;
  return SK_OK;
}

int attn_launch_status() { return hipGetLastError() == hipSuccess ? SK_OK : SK_ERR_LAUNCH; }

int attn_device_ok() {
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return SK_ERR_DEVICE;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? SK_OK : SK_ERR_DEVICE;
}

}  // namespace

extern "C" {

int sk_qk_norm_rope_cache_bf16(const sk_bf16* qkv, int64_t ld_qkv, const sk_bf16* q_norm_w, const sk_bf16* k_norm_w,
                               const sk_bf16* cos, const sk_bf16* sin, int rope_rows, const int32_t* pos,
                               const int32_t* depth, sk_bf16* q_out, sk_bf16* k_cache, sk_bf16* v_cache, int B, int T,
                               int HQ, int HKV, int D, int cap, float eps, hipStream_t stream) {
  if (B < 0 || T < 0 || HQ < 1 || HKV < 1 || cap < 1 || rope_rows < 1 || D != sk::HEAD_D) return SK_ERR_SHAPE;
  if (ld_qkv < (int64_t)(HQ + 2 * HKV) * D) return SK_ERR_SHAPE;
  if ((long)B * T > 0x7FFFFFFFL) return SK_ERR_SHAPE;
  if (B == 0 || T == 0) return SK_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !pos || !q_out || !k_cache || !v_cache) return SK_ERR_NULL;
  int st = attn_device_ok();
  if (st) return st;
  sk::RopeArgs a;
  a.qkv = qkv;
  a.ld_qkv = ld_qkv;
  a.qw = q_norm_w;
  a.kw = k_norm_w;
  a.cos = cos;
  a.sin = sin;
  a.rope_rows = rope_rows;
  a.pos = pos;
  a.depth = depth;
  a.q_out = q_out;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.T = T;
  a.HQ = HQ;
  a.HKV = HKV;
  a.cap = cap;
  a.eps = eps;
  const unsigned groups = (unsigned)cdiv(HQ + HKV, 4);
  sk::qk_norm_rope_kernel<<<dim3((unsigned)(B * T), groups), dim3(256), 0, stream>>>(a);
  return attn_launch_status();
}

size_t sk_decode_attention_workspace_bytes(int B, int HQ, int HKV, int D, int R, int cap, int max_len, int nsplit) {
  AttnPlan p;
  if (attn_plan(B, HQ, HKV, D, R, cap, max_len, nsplit, &p)) return 0;
  return p.need;
}

}  // extern "C"

namespace {

// Fills the plan-dependent fields of a and launches the instance for
// (QR, tree, rope).
int attn_run(const AttnPlan& p, sk::AttnArgs& a, int B, int HQ, int HKV, int R, int cap, float scale, void* ws,
             bool rope, hipStream_t stream) {
  if (p.need > 0) {
    char* w = static_cast<char*>(ws);
    a.tickets = reinterpret_cast<unsigned*>(w);
    a.part_o = reinterpret_cast<float*>(w + p.tickets);
    a.part_ml = reinterpret_cast<float*>(w + p.tickets + align256(p.part_o));
  }
  a.HQ = HQ;
  a.HKV = HKV;
  a.R = R;
  a.G = HQ / HKV;
  a.cap = cap;
  a.S = p.S;
  a.split_len = p.split_len;
  a.NRB = p.NRB;
  a.rb_xcd = p.NRB > 1 && (B * HKV * p.S) % 8 == 0;
  a.scale = scale;
  const dim3 grid((unsigned)(B * HKV * p.NRB * p.S));
  const dim3 block(64 * kAttnWaves);
  if (rope && a.tree) {
    if (p.QR == 4) sk::decode_attn_kernel<4, kAttnWaves, true, true><<<grid, block, 0, stream>>>(a);
    else if (p.QR == 8) sk::decode_attn_kernel<8, kAttnWaves, true, true><<<grid, block, 0, stream>>>(a);
    else sk::decode_attn_kernel<16, kAttnWaves, true, true><<<grid, block, 0, stream>>>(a);
  } else if (rope) {
    if (p.QR == 4) sk::decode_attn_kernel<4, kAttnWaves, false, true><<<grid, block, 0, stream>>>(a);
    else if (p.QR == 8) sk::decode_attn_kernel<8, kAttnWaves, false, true><<<grid, block, 0, stream>>>(a);
    else sk::decode_attn_kernel<16, kAttnWaves, false, true><<<grid, block, 0, stream>>>(a);
  } else if (a.tree) {
    if (p.QR == 4) sk::decode_attn_kernel<4, kAttnWaves, true><<<grid, block, 0, stream>>>(a);
    else if (p.QR == 8) sk::decode_attn_kernel<8, kAttnWaves, true><<<grid, block, 0, stream>>>(a);
    else sk::decode_attn_kernel<16, kAttnWaves, true><<<grid, block, 0, stream>>>(a);
  } else {
    if (p.QR == 4) sk::decode_attn_kernel<4, kAttnWaves, false><<<grid, block, 0, stream>>>(a);
    else if (p.QR == 8) sk::decode_attn_kernel<8, kAttnWaves, false><<<grid, block, 0, stream>>>(a);
    else sk::decode_attn_kernel<16, kAttnWaves, false><<<grid, block, 0, stream>>>(a);
  }
  return attn_launch_status();
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}

// The fused rotary step + attention of both entry points: tree and depth
// (the draft-tree masks and rotary offsets, both [R]) or both nullptr (chain).
int rope_attention(const sk_bf16* qkv, int64_t ld_qkv, const sk_bf16* q_norm_w, const sk_bf16* k_norm_w,
                   const sk_bf16* cos, const sk_bf16* sin, int rope_rows, float eps, sk_bf16* k_cache,
                   sk_bf16* v_cache, const int32_t* pos, const int64_t* tree, const int32_t* depth, sk_bf16* out,
                   int B, int HQ, int HKV, int D, int R, int cap, int max_len, float scale, int nsplit, void* ws,
                   size_t ws_bytes, hipStream_t stream) {
  if (B < 0) return SK_ERR_SHAPE;
  if (B == 0) return SK_OK;
  AttnPlan p;
  int st = attn_plan(B, HQ, HKV, D, R, cap, max_len, nsplit, &p);
  if (st) return st;
  if (rope_rows < 1 || ld_qkv < (int64_t)(HQ + 2 * HKV) * D || (long)B * R > 0x7FFFFFFFL) return SK_ERR_SHAPE;
  if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !k_cache || !v_cache || !pos || !out) return SK_ERR_NULL;
  if (!aligned16(k_cache) || !aligned16(v_cache)) return SK_ERR_ALIGN;
  if (p.need > 0 && (!ws || ws_bytes < p.need)) return SK_ERR_WORKSPACE;
  // The output is written while the projection rows and the caches are read.
  const size_t out_bytes = (size_t)B * R * HQ * D * 2, cache_bytes = (size_t)B * HKV * cap * D * 2;
  const size_t qkv_bytes = ((size_t)(B * R - 1) * ld_qkv + (size_t)(HQ + 2 * HKV) * D) * 2;
  if (overlaps(out, out_bytes, qkv, qkv_bytes) || overlaps(out, out_bytes, k_cache, cache_bytes) ||
      overlaps(out, out_bytes, v_cache, cache_bytes) || overlaps(k_cache, cache_bytes, v_cache, cache_bytes) ||
      overlaps(k_cache, cache_bytes, qkv, qkv_bytes) || overlaps(v_cache, cache_bytes, qkv, qkv_bytes))
    return SK_ERR_ALIAS;
  st = attn_device_ok();
  if (st) return st;
  sk::AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.k = k_cache;
  a.v = v_cache;
  a.pos = pos;
  a.out = out;
  a.qkv = qkv;
  a.ld_qkv = ld_qkv;
  a.qw = q_norm_w;
  a.kw = k_norm_w;
  a.cos = cos;
  a.sin = sin;
  a.k_out = k_cache;
  a.v_out = v_cache;
  a.rope_rows = rope_rows;
  a.eps = eps;
  a.tree = tree;
  a.depth = depth;
  return attn_run(p, a, B, HQ, HKV, R, cap, scale, ws, true, stream);
}


}  // namespace

extern "C" {

int sk_decode_attention_bf16(const sk_bf16* q, const sk_bf16* k_cache, const sk_bf16* v_cache, const int32_t* pos,
                             const int64_t* tree, sk_bf16* out, int B, int HQ, int HKV, int D, int R, int cap,
                             int max_len, float scale, int nsplit, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (B < 0) return SK_ERR_SHAPE;
  if (B == 0) return SK_OK;
  AttnPlan p;
  int st = attn_plan(B, HQ, HKV, D, R, cap, max_len, nsplit, &p);
  if (st) return st;
  if (!q || !k_cache || !v_cache || !pos || !out) return SK_ERR_NULL;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache)) return SK_ERR_ALIGN;
  if (p.need > 0 && (!ws || ws_bytes < p.need)) return SK_ERR_WORKSPACE;
  st = attn_device_ok();
  if (st) return st;
  sk::AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.pos = pos;
  a.tree = tree;
  a.out = out;
  return attn_run(p, a, B, HQ, HKV, R, cap, scale, ws, false, stream);
}

int sk_decode_attention_rope_bf16(const sk_bf16* qkv, int64_t ld_qkv, const sk_bf16* q_norm_w,
                                  const sk_bf16* k_norm_w, const sk_bf16* cos, const sk_bf16* sin, int rope_rows,
                                  float eps, sk_bf16* k_cache, sk_bf16* v_cache, const int32_t* pos, sk_bf16* out,
                                  int B, int HQ, int HKV, int D, int R, int cap, int max_len, float scale,
                                  int nsplit, void* ws, size_t ws_bytes, hipStream_t stream) {
  return rope_attention(qkv, ld_qkv, q_norm_w, k_norm_w, cos, sin, rope_rows, eps, k_cache, v_cache, pos, nullptr,
                        nullptr, out, B, HQ, HKV, D, R, cap, max_len, scale, nsplit, ws, ws_bytes, stream);
}

int sk_decode_attention_rope_tree_bf16(const sk_bf16* qkv, int64_t ld_qkv, const sk_bf16* q_norm_w,
                                       const sk_bf16* k_norm_w, const sk_bf16* cos, const sk_bf16* sin,
                                       int rope_rows, float eps, sk_bf16* k_cache, sk_bf16* v_cache,
                                       const int32_t* pos, const int64_t* tree, const int32_t* depth, sk_bf16* out,
                                       int B, int HQ, int HKV, int D, int R, int cap, int max_len, float scale,
                                       int nsplit, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (B > 0 && (!tree || !depth)) return SK_ERR_NULL;
  return rope_attention(qkv, ld_qkv, q_norm_w, k_norm_w, cos, sin, rope_rows, eps, k_cache, v_cache, pos, tree,
                        depth, out, B, HQ, HKV, D, R, cap, max_len, scale, nsplit, ws, ws_bytes, stream);
}

}  // extern "C"
