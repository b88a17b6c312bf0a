// sk_wide.hpp - the wide-M body: up to 128 activation rows in one workgroup,
// so every weight tile streams from HBM into a CU once for all of them.
//
// The verify forward of the reference runs its projections at M = B x R rows
// (128 at batch 16; engine/engine.py:451, engine/model.py:359), and its
// skinny GEMM keeps every row in one M tile up to 128 rows so that the
// weights stream exactly once (engine/kernels/gemm.py:300-305).  The ring
// path below 64 rows holds each wave's activation fragments for its own K
// range in registers, which does not scale to 128 rows; this body splits the
// work the other way:
//
//  * A workgroup owns a tile of `tr` weight rows (gate/up: tr gate rows and
//    tr up rows) and one K slice, and walks the slice in 256-column steps.
//  * Each step's weight rows are loaded row-contiguous by all W waves (one
//    load instruction = 512 B of each of two rows, the access pattern of the
//    ring path), written once into one of two LDS buffers (row pitch 544 B:
//    fragment reads are conflict-free) and read back as MFMA A fragments by
//    every wave.
//  * The waves split the activation rows: wave w owns the 16-row activation
//    tiles w, w + W, ... (W = 4: two tiles, W = 8: one), loads their
//    fragments straight from global memory (L2-resident, 16 rows x 64 B per
//    instruction) one step ahead, and keeps the fp32 accumulators of its
//    rows x the tile's weight rows.  No cross-wave reduction is needed.
//  * Weight rows are requested one step ahead (the steps of successive tiles
//    form one sequence, so the next tile's first rows are in flight while
//    this tile finishes).
//  * With WN = 2 the waves also split the tile's weight slabs (two groups of
//    slabs, four groups of activation tiles): each wave then reads half the
//    staged rows from LDS, halving the LDS read traffic per weight byte
//    (LDS, not HBM, bounds the one-group shape at 128 rows).
//  * One barrier per step: a wave writes buffer s & 1 only after every wave
//    passed step s - 1's barrier, i.e. finished the MFMAs of step s - 2 that
//    read that buffer.
//
// Epilogues: bf16 store, SwiGLU (gate and up accumulators sit in the same
// lane), fused argmax (lane candidates folded per row into LDS, then the
// cross-workgroup finish of the other bodies), and fp32 split-K partials
// finished in-kernel by the last workgroup of each tile (splitk_fixup).
#pragma once

#include "sk_kernels.hpp"

namespace sk {

constexpr int kWideChunk = 256;                  // K columns per step
constexpr int kWidePitch = 2 * kWideChunk + kRowPad;  // LDS bytes per staged weight row

// LDS bytes of a wide instance: two weight buffers, then the argmax row bests
// or the split-K ticket flags.
constexpr size_t wide_weight_lds(int NT) { return (size_t)2 * 16 * NT * kWidePitch; }

template <int W, int WN, int NT, int EPI>
__device__ __forceinline__ void wide_body(Args p) {
  constexpr bool GATEUP = EpiTraits<EPI>::gateup;
  constexpr int BASE = EpiTraits<EPI>::base;
  static_assert(!EpiTraits<EPI>::norm && !EpiTraits<EPI>::pre && !EpiTraits<EPI>::resid, "plain epilogues only");
  static_assert(!GATEUP || NT % 2 == 0, "gate/up tiles pair NT/2 gate slabs with NT/2 up slabs");
  static_assert(W == 4 || W == 8, "four or eight waves");
  constexpr int WM = W / WN;                // wave groups along M (WN along the tile's rows)
  constexpr int MTW = 8 / WM;               // activation tiles per wave (128 rows in all)
  constexpr int ROWS = 16 * NT;             // staged weight rows per tile
  constexpr int H = GATEUP ? NT / 2 : NT;   // slabs per half
  static_assert(H % WN == 0, "the slabs (of each half) split evenly over the row groups of waves");
  constexpr int HW = H / WN;                // slabs (of each half) per wave
  constexpr int NL = GATEUP ? 2 * HW : HW;  // slabs a wave multiplies
  constexpr int HROWS = 16 * H;             // output columns a tile can hold (the finish's stride)
  constexpr int UNITS = kWideChunk / 32;    // MFMA K steps per chunk
  constexpr int QPW = ROWS / 2 / W;         // weight load instructions per wave and chunk
  static_assert((ROWS / 2) % W == 0, "weight loads split evenly over the waves");

  extern __shared__ __attribute__((aligned(16))) float lds[];
  char* const wbuf = reinterpret_cast<char*>(lds);
  char* const tail = wbuf + wide_weight_lds(NT);
  unsigned long long* const lds_best = reinterpret_cast<unsigned long long*>(tail);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4, lrow = lane >> 5;
  const int nh = wave % WN, mq = wave / WN;   // this wave's group of slabs, group of activation tiles
  // global slab of local slab k (gate/up: k < HW gate slabs, the rest up slabs)
  auto slab = [&](int k) { return GATEUP && k >= HW ? H + nh * HW + (k - HW) : nh * HW + k; };
  const int M = p.M, TR = p.tr;
  const int S = p.S;
  const int slice = blockIdx.x % (unsigned)S;
  const int rbstep = p.rbstep;
  const int rb0 = blockIdx.x / (unsigned)S;
  const int ntiles = wg_tiles(rb0, rbstep, p.nrb);
  const int nchunks = (p.K + kWideChunk - 1) / kWideChunk;
  const int c_lo = slice * p.slice_units;
  const int c_hi = min(c_lo + p.slice_units, nchunks);
  const uint16_t* const zero16 = reinterpret_cast<const uint16_t*>(kZeroLine);
  if constexpr (BASE == EPI_ARGMAX) {
    for (int i = tid; i < M; i += 64 * W) lds_best[i] = 0ull;   // ordered by the first step's barrier
  }

  // Weight instruction i of this wave: staged row sr = 2*(wave + W*i) + lane/32,
  // 16 bytes at column 8*(lane%32) of the chunk.  Rows past the tile, past N
  // (clamped) or columns past K read the zero line.
  auto w_src = [&](int rb, int c, int i) -> const uint16_t* {
    const int sr = 2 * (wave + W * i) + lrow;
    const int col = c * kWideChunk + 8 * (lane & 31);
    const int half = sr / HROWS, hr = sr - half * HROWS;
    if (col >= p.K || hr >= TR) return zero16;
    const int row = min(rb * TR + hr, p.N - 1);
    return ((GATEUP && half) ? p.W1 : p.W0) + (int64_t)row * p.ldw + col;
  };
  // Activation fragment (tile i of this wave, unit u of chunk c): lane holds
  // A[16*mt + r16][c*256 + 32u + 8*g4 .. +8].  Rows past M repeat row M-1
  // (their MFMA columns are never read); a tile past M or a unit past K reads
  // the zero line.
  auto a_src = [&](int i, int c, int u) -> const uint16_t* {
    const int mt = mq + WM * i;
    const int col = c * kWideChunk + 32 * u + 8 * g4;
    if (16 * mt >= M || col >= p.K) return zero16;
    return p.A + (int64_t)min(16 * mt + r16, M - 1) * p.lda + col;
  };

  // The steps of all the workgroup's tiles form one sequence g = 0 .. G-1
  // (tile g / nsteps, chunk c_lo + g % nsteps), unrolled by D = 2 so that the
  // register slots are compile-time: step g's weight rows sit in slot g % 2
  // and are requested PF = 1 step ahead (across tile boundaries too; two or
  // three steps ahead measured the same at 128 rows), and so are its
  // activation fragments (slot g % 2).
  constexpr int D = 2, PF = 1;
  const int nsteps = max(c_hi - c_lo, 0);
  const int G = ntiles * nsteps;
  auto tile_of = [&](int g) { return rb0 + (g / nsteps) * rbstep; };
  auto chunk_of = [&](int g) { return c_lo + g % nsteps; };

  u32x4 wreg[D][QPW];
  bf16x8 afr[2][MTW][UNITS];
  auto issue_w = [&](auto slot, int g) {
    constexpr int SL = decltype(slot)::value;
    const int rb = tile_of(g), c = chunk_of(g);
#pragma unroll
    for (int i = 0; i < QPW; ++i) wreg[SL][i] = ld16_stream(w_src(rb, c, i));
  };
  auto issue_acts = [&](auto buf, int c) {
    constexpr int B = decltype(buf)::value;
#pragma unroll
    for (int i = 0; i < MTW; ++i)
#pragma unroll
      for (int u = 0; u < UNITS; ++u) afr[B][i][u] = __builtin_bit_cast(bf16x8, ld16(a_src(i, c, u)));
  };
  static_assert(PF >= 1 && PF < D, "prefetch distance within the register slots");
  if (G > 0) issue_w(std::integral_constant<int, 0>{}, 0);
  if constexpr (PF > 1) {
    if (G > 1) issue_w(std::integral_constant<int, 1>{}, 1);
  }
  if constexpr (PF > 2) {
    if (G > 2) issue_w(std::integral_constant<int, 2>{}, 2);
  }
  if (G > 0) issue_acts(std::integral_constant<int, 0>{}, c_lo);

  f32x4 acc[NL][MTW];
  auto zero_acc = [&]() {
#pragma unroll
    for (int nt = 0; nt < NL; ++nt)
#pragma unroll
      for (int i = 0; i < MTW; ++i) acc[nt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  // Tile epilogue.  Lane holds, for activation row m = 16*(mq + WM*i) + r16,
  // the tile's output columns hr = 16*slab(h) + 4*g4 + e (e < 4) of its local
  // slab h (and, for gate/up, the up value of the same column in local slab
  // h + HW).
  auto epilogue = [&](int rb) {
#pragma unroll
    for (int i = 0; i < MTW; ++i) {
      const int m = 16 * (mq + WM * i) + r16;
      unsigned long long key = 0ull;
#pragma unroll
      for (int h = 0; h < HW; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int hr = 16 * slab(h) + 4 * g4 + e;
          const int n = rb * TR + hr;
          const bool ok = m < M && hr < TR && n < p.N;
          if constexpr (BASE == EPI_STORE) {
            if (ok) p.C[(int64_t)m * p.ldc + n] = f2bf(acc[h][i][e]);
          } else if constexpr (BASE == EPI_SWIGLU) {
            if (ok) p.C[(int64_t)m * p.ldc + n] = swiglu_bf(acc[h][i][e], acc[h + HW][i][e]);
          } else if constexpr (BASE == EPI_PART) {
            if (ok) store_agent(&p.part[((int64_t)slice * M + m) * p.N + n], acc[h][i][e]);
          } else if constexpr (BASE == EPI_PART_GU) {
            if (ok) {
              store_agent(&p.part[((int64_t)slice * M + m) * p.N + n], acc[h][i][e]);
              store_agent(&p.part[((int64_t)(S + slice) * M + m) * p.N + n], acc[h + HW][i][e]);
            }
          } else {   // EPI_ARGMAX
            if (ok) {
              const unsigned long long k = argmax_key(f2bf(acc[h][i][e]), n);
              key = k > key ? k : key;
            }
          }
        }
      if constexpr (BASE == EPI_ARGMAX) {
        // the four lanes of row m (g4 = 0..3), then one LDS atomic per row
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
          const unsigned long long o = ((unsigned long long)(uint32_t)__shfl_xor((int)(key >> 32), off) << 32) |
                                       (uint32_t)__shfl_xor((int)(key & 0xFFFFFFFFu), off);
          key = o > key ? o : key;
        }
        if (g4 == 0 && m < M && key) atomicMax(&lds_best[m], key);
      }
    }
  };

  auto step = [&](auto slot, int g) {
    constexpr int SL = decltype(slot)::value;   // g % D
    constexpr int B = SL & 1;                   // g % 2
    char* const wb = wbuf + (g & 1) * (ROWS * kWidePitch);
    // Stage step g's rows, then request step g + PF's into the slot that held
    // step g + PF - D (already staged).
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      const int sr = 2 * (wave + W * i) + lrow;
      *reinterpret_cast<u32x4*>(wb + sr * kWidePitch + 16 * (lane & 31)) = wreg[SL][i];
    }
    if (g + PF < G) issue_w(std::integral_constant<int, (SL + PF) % D>{}, g + PF);
    if (g + 1 < G) issue_acts(std::integral_constant<int, 1 - B>{}, chunk_of(g + 1));
    lds_barrier();
#pragma unroll
    for (int nt = 0; nt < NL; ++nt)
#pragma unroll
      for (int u = 0; u < UNITS; ++u) {
        const bf16x8 wv =
            *reinterpret_cast<const bf16x8*>(wb + (16 * slab(nt) + r16) * kWidePitch + 64 * u + 16 * g4);
#pragma unroll
        for (int i = 0; i < MTW; ++i)
          acc[nt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, afr[B][i][u], acc[nt][i], 0, 0, 0);
      }
    if ((g + 1) % nsteps == 0) {   // the tile's last step
      epilogue(tile_of(g));
      zero_acc();
    }
  };
  static_assert(D == 2, "the loop below is unrolled for two slots");
  for (int g0 = 0; g0 < G; g0 += D) {
    step(std::integral_constant<int, 0>{}, g0);
    if (g0 + 1 < G) step(std::integral_constant<int, 1>{}, g0 + 1);
  }

  if constexpr (BASE == EPI_ARGMAX) {
    lds_barrier();
    argmax_fixup(p, lds_best, reinterpret_cast<int*>(lds_best + M));
  } else if constexpr (BASE == EPI_PART || BASE == EPI_PART_GU) {
    splitk_fixup<HROWS, BASE>(p, ntiles, rb0, reinterpret_cast<int*>(tail));
  }
}

}  // namespace sk
