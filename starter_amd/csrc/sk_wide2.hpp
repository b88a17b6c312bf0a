// sk_wide2.hpp - the wide-M body with both operands staged in LDS: up to 128
// activation rows and a tile of weight rows per workgroup, four or eight
// waves, each multiplying the whole weight tile against 32 activation rows
// (eight waves: two per 32 rows, each on half of every step's K columns).
//
// Why a second wide body: in sk_wide.hpp every wave fetches its activation
// fragments from L2 itself (16 rows x 64 B per instruction) and reads every
// staged weight fragment once per 16 activation rows; at 128 rows those two
// streams, not HBM, set its time.  Here:
//
//  * Each 128-column step stages the tile's weight rows AND the 128
//    activation rows in LDS (one 288-byte row per staged row: fragment reads
//    of 16 consecutive rows are conflict-free), loaded row-contiguous by all
//    four waves (one instruction = 256 B of each of four rows).
//  * Wave w holds the fp32 accumulators of activation tiles 2(w % 4) and
//    2(w % 4) + 1 against every weight slab: per 32-column MFMA step it reads
//    NT weight fragments and two activation fragments for 2 NT MFMAs, i.e.
//    each weight fragment read from LDS feeds two MFMAs and each activation
//    fragment NT.  With eight waves, waves w and w + 4 take the first and the
//    second half of each step's four MFMA steps, and at a tile's end waves
//    4-7 hand their sums to waves 0-3 through LDS: two waves per SIMD hide
//    each other's LDS and MFMA latencies (one wave per SIMD with four waves:
//    gate_up at 128 rows 47.5 us against 36.1 with eight).
//  * Global loads run ahead in a two-slot register ring (the steps of
//    successive tiles form one sequence), LDS is double-buffered with one
//    barrier per step: after step g's barrier a wave issues step g's MFMAs,
//    then stages step g + 1 into the other buffer, which every wave finished
//    reading at step g - 1.
//
// Epilogues and the cross-workgroup finishes are those of sk_wide.hpp: bf16
// store, SwiGLU, fused argmax (per-row LDS bests, then argmax_fixup), split-K
// partials finished in-kernel by the last workgroup of each tile.  The
// residual hand-off runs here too: a producer (split-K partials) finishes
// xout = r + y with the per-row partial sums of squares of xout, and a
// consumer normalises the activation rows as it stages them, with row norms
// from those partial sums.
#pragma once

#include "sk_wide.hpp"

namespace sk {

constexpr int kW2Step = 128;                  // K columns per step
constexpr int kW2Pitch = 2 * kW2Step + kRowPad;   // LDS bytes per staged row
constexpr int kW2Rows = 128;                  // activation rows staged per step (M <= 128)

// LDS bytes of a two-operand wide instance: two buffers of the weight tile's
// 16 NT rows and 128 activation rows; the argmax bests or split-K flags follow.
constexpr size_t wide2_lds(int NT) { return (size_t)2 * (16 * NT + kW2Rows) * kW2Pitch; }

template <int W, int NT, int EPI>
__device__ __forceinline__ void wide2_body(Args p) {
  constexpr bool GATEUP = EpiTraits<EPI>::gateup;
  constexpr int BASE = EpiTraits<EPI>::base;
  constexpr bool PRE = EpiTraits<EPI>::pre;       // consumer: normalise the rows while staging them
  constexpr bool RESID = EpiTraits<EPI>::resid;   // producer: the split-K finish hands the residual on
  static_assert(!EpiTraits<EPI>::norm, "the norm prologue with an add runs on the GEMV path");
  static_assert(!RESID || BASE == EPI_PART, "the residual hand-off follows split-K partials");
  static_assert(!GATEUP || NT % 2 == 0, "gate/up tiles pair NT/2 gate slabs with NT/2 up slabs");
  static_assert(W == 4 || W == 8, "four waves, or eight splitting each step's K units in two");
  constexpr int KH = W / 4;                  // K halves of a step (waves w and w + 4 share tiles)
  constexpr int MTW = 2;                     // 16-row activation tiles per wave
  constexpr int ROWS = 16 * NT;              // staged weight rows
  constexpr int SROWS = ROWS + kW2Rows;      // staged rows per buffer
  constexpr int H = GATEUP ? NT / 2 : NT;    // slabs per half
  constexpr int HROWS = 16 * H;              // output columns a tile can hold (the finish's stride)
  constexpr int UNITS = kW2Step / 32;        // MFMA K steps per step
  constexpr int WLD = ROWS / (4 * W);        // weight load instructions per wave and step
  constexpr int ALD = kW2Rows / (4 * W);     // activation load instructions per wave and step
  static_assert(ROWS % (4 * W) == 0, "weight loads split evenly over the waves");
  constexpr int UW = UNITS / KH;             // MFMA K steps of one wave per step
  // A wave issues step g's MFMAs right after step g's barrier and only then
  // stages step g + 1 (which waits for that step's loads) and requests step
  // g + 3 into the freed register slot: the MFMAs already issued run while
  // the wave waits.  Staging first held every MFMA of the step behind the
  // wait (at 64 rows lm_head + argmax 192 -> 155 us, gate_up 30.1 -> 26.5; at
  // 96 rows 205 -> 180 and 32.9 -> 29.4; at 128 rows within 1-2%).  Two
  // register slots: a third, with each step's loads requested at its start,
  // was slower at every row count (more requests in flight: gate_up at 128
  // rows 38.8 against 34.0 us).
  constexpr int D = 2, PF = 3;

  extern __shared__ __attribute__((aligned(16))) float lds[];
  char* const buf = reinterpret_cast<char*>(lds);
  char* const tail = buf + wide2_lds(NT);
  unsigned long long* const lds_best = reinterpret_cast<unsigned long long*>(tail);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int mw = wave % 4, kh = wave / 4;     // activation tiles 2 mw, 2 mw + 1; K half kh
  const int M = p.M, TR = p.tr;
  const int S = p.S;
  const int slice = blockIdx.x % (unsigned)S;
  const int rbstep = p.rbstep;
  const int rb0 = blockIdx.x / (unsigned)S;
  const int ntiles = wg_tiles(rb0, rbstep, p.nrb);
  // The planner's K units are 256-column chunks; a step is half of one.
  const int nchunks = (p.K + kWideChunk - 1) / kWideChunk;
  const int s_lo = 2 * slice * p.slice_units;
  const int s_hi = min(2 * min((slice + 1) * p.slice_units, nchunks), (p.K + kW2Step - 1) / kW2Step);
  const int nsteps = max(s_hi - s_lo, 0);
  const int G = ntiles * nsteps;
  auto tile_of = [&](int g) { return rb0 + (g / nsteps) * rbstep; };
  auto step_of = [&](int g) { return s_lo + g % nsteps; };
  const uint16_t* const zero16 = reinterpret_cast<const uint16_t*>(kZeroLine);
  if constexpr (BASE == EPI_ARGMAX) {
    for (int i = tid; i < M; i += 64 * W) lds_best[i] = 0ull;   // ordered by the first step's barrier
  }

  // Load instruction i of this wave covers staged rows 4*(wave + W*i) + g4
  // (lane: 16 bytes at column 8*r16 of the step).  The row addresses are
  // formed once (activations) or once per tile (weights); weight rows past
  // the tile or past N (clamped), activation rows past M and columns past K
  // read the zero line.
  const uint16_t* abase[ALD];
  bool aok[ALD];
#pragma unroll
  for (int i = 0; i < ALD; ++i) {
    const int ar = 4 * (wave + W * i) + g4;
    aok[i] = ar < M;
    abase[i] = p.A + (int64_t)min(ar, M - 1) * p.lda + 8 * r16;
  }
  const uint16_t* wbase[WLD];
  bool wok[WLD];
  auto set_tile = [&](int rb) {
#pragma unroll
    for (int i = 0; i < WLD; ++i) {
      const int sr = 4 * (wave + W * i) + g4;
      const int half = sr / HROWS, hr = sr - half * HROWS;
      wok[i] = hr < TR;
      const int row = min(rb * TR + hr, p.N - 1);
      wbase[i] = ((GATEUP && half) ? p.W1 : p.W0) + (int64_t)row * p.ldw + 8 * r16;
    }
  };

  u32x4 wreg[D][WLD];
  u32x4 areg[D][ALD];
  // PRE: the norm weights of the lane's eight columns of the step (the same
  // for every row), requested with the step's rows.
  u32x4 nreg[PRE ? D : 1];
  // Requests are made in step order, so the weight row addresses follow the
  // tile of the step being requested.  Steps past the last (g >= G) request
  // the zero line: the loop below stages and requests without branches, so
  // the compiler's wait for a slot's loads leaves the other slot's in flight
  // (around conditional requests it waited for every load before the next
  // requests, one step of look-ahead instead of two).
  auto issue = [&](auto slot, int g) {
    constexpr int SL = decltype(slot)::value;
    const bool live = g < G;
    const int st = step_of(g);
    if (live && st == s_lo) set_tile(tile_of(g));   // uniform: the first step of a tile
    const int col0 = st * kW2Step;
    const bool colok = live && col0 + 8 * r16 < p.K;
#pragma unroll
    for (int i = 0; i < WLD; ++i) wreg[SL][i] = ld16_stream(wok[i] && colok ? wbase[i] + col0 : zero16);
#pragma unroll
    for (int i = 0; i < ALD; ++i) areg[SL][i] = ld16(aok[i] && colok ? abase[i] + col0 : zero16);
    if constexpr (PRE) nreg[SL] = ld16(colok ? p.NW + col0 + 8 * r16 : zero16);
  };
  // PRE: rstd of each staged activation row of this lane, from the
  // producer's partial sums of squares (K/16 per row, row stride sq_ld): the
  // row's 16 lanes sum every 16th group each, in increasing group order,
  // then a butterfly over the 16 lanes (a fixed order); rows past M sum
  // nothing and are never used.
  float rst[PRE ? ALD : 1];
  auto row_norms = [&]() {
    const int ngrp = p.K >> 4;
    float t[ALD];
#pragma unroll
    for (int i = 0; i < ALD; ++i) t[i] = 0.f;
    for (int g0 = r16; g0 < ngrp; g0 += 16 * 4) {
      float v[ALD][4];
#pragma unroll
      for (int i = 0; i < ALD; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int gi = g0 + 16 * k;
          const int ar = 4 * (wave + W * i) + g4;
          v[i][k] = (aok[i] && gi < ngrp) ? p.SQ[(int64_t)ar * p.sq_ld + gi] : 0.f;
        }
#pragma unroll
      for (int i = 0; i < ALD; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) t[i] += v[i][k];
    }
#pragma unroll
    for (int i = 0; i < ALD; ++i) {
      float u = t[i];
      u += __shfl_xor(u, 1);
      u += __shfl_xor(u, 2);
      u += __shfl_xor(u, 4);
      u += __shfl_xor(u, 8);
      rst[i] = rms_rstd(u, p.K, p.eps);
    }
  };
  auto stage = [&](auto slot, int g) {
    constexpr int SL = decltype(slot)::value;
    char* const sb = buf + (g & 1) * (SROWS * kW2Pitch);
#pragma unroll
    for (int i = 0; i < WLD; ++i)
      *reinterpret_cast<u32x4*>(sb + (4 * (wave + W * i) + g4) * kW2Pitch + 16 * r16) = wreg[SL][i];
    // PRE: A = bf16(w * bf16(x * rstd)) (the cast placement of
    // engine/kernels/gemm.py:28-56); zero lines stay zero
    u32x4 wlo, whi;
    if constexpr (PRE) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        wlo[q] = nreg[SL][q] & 0xFFFFu;
        whi[q] = nreg[SL][q] & 0xFFFF0000u;
      }
    }
#pragma unroll
    for (int i = 0; i < ALD; ++i) {
      u32x4 v = areg[SL][i];
      if constexpr (PRE) v = norm_line_bf16x8(v, wlo, whi, rst[i]);
      *reinterpret_cast<u32x4*>(sb + (ROWS + 4 * (wave + W * i) + g4) * kW2Pitch + 16 * r16) = v;
    }
  };
  if (G > 0) {
    issue(std::integral_constant<int, 0>{}, 0);
    issue(std::integral_constant<int, 1>{}, 1);
    // (the partial sums are requested after the first two steps' rows: the
    // first staging waits for those anyway)
    if constexpr (PRE) row_norms();
    stage(std::integral_constant<int, 0>{}, 0);
    issue(std::integral_constant<int, 0>{}, 2);
  }

  f32x4 acc[NT][MTW];
  auto zero_acc = [&]() {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int i = 0; i < MTW; ++i) acc[nt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  // Tile epilogue.  Lane holds, for activation row m = 16*(MTW*mw + i) + r16,
  // the tile's output columns hr = 16*h + 4*g4 + e (e < 4) of slab h (and,
  // for gate/up, the up value of the same column in slab h + H).
  auto epilogue = [&](int rb) {
#pragma unroll
    for (int i = 0; i < MTW; ++i) {
      const int m = 16 * (MTW * mw + i) + r16;
      unsigned long long key = 0ull;
#pragma unroll
      for (int h = 0; h < H; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int hr = 16 * h + 4 * g4 + e;
          const int n = rb * TR + hr;
          const bool ok = m < M && hr < TR && n < p.N;
          if constexpr (BASE == EPI_STORE) {
            if (ok) p.C[(int64_t)m * p.ldc + n] = f2bf(acc[h][i][e]);
          } else if constexpr (BASE == EPI_SWIGLU) {
            if (ok) p.C[(int64_t)m * p.ldc + n] = swiglu_bf(acc[h][i][e], acc[h + H][i][e]);
          } else if constexpr (BASE == EPI_PART) {
            if (ok) store_agent(&p.part[((int64_t)slice * M + m) * p.N + n], acc[h][i][e]);
          } else if constexpr (BASE == EPI_PART_GU) {
            if (ok) {
              store_agent(&p.part[((int64_t)slice * M + m) * p.N + n], acc[h][i][e]);
              store_agent(&p.part[((int64_t)(S + slice) * M + m) * p.N + n], acc[h + H][i][e]);
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

  // Stores through LDS: the tile's finished values go to LDS in [row][column]
  // order (pitch TP elements), then every thread writes consecutive columns,
  // so a store instruction covers whole lines instead of four 4-byte pieces
  // of sixteen rows (at 128 rows: o_proj's split-K partials 21.0 -> 18.3 us,
  // down 33.4 -> 29.9, the lm_head logits 249 -> 242).  The SwiGLU tile of
  // gate_up too, its products formed from the gate and up accumulators
  // before the LDS write (48-64 rows 2-4% faster than direct stores, 96-128
  // rows within 1%; before the MFMA-first step order it was slower).
  //
  // The argmax tile of the eight-slab, eight-wave instance goes the same way
  // (its per-lane epilogue does not fit the register file beside the
  // pipeline): bf16 values to LDS, then four threads per row scan a quarter
  // of the row's columns each.
  constexpr bool LDS_ARGMAX = BASE == EPI_ARGMAX && W == 8 && NT == 8;
  constexpr bool LDS_OUT =
      BASE == EPI_STORE || BASE == EPI_SWIGLU || BASE == EPI_PART || BASE == EPI_PART_GU || LDS_ARGMAX;
  constexpr bool F32OUT = BASE == EPI_PART || BASE == EPI_PART_GU;
  constexpr int TP = HROWS + (F32OUT ? 4 : 8);
  constexpr int NMAT = BASE == EPI_PART_GU ? 2 : 1;
  static_assert(!LDS_OUT ||
                    (size_t)NMAT * kW2Rows * TP * (F32OUT ? 4 : 2) <= (size_t)SROWS * kW2Pitch,
                "the staged tile fits one step buffer");
  auto write_tile = [&](char* sb) {
#pragma unroll
    for (int i = 0; i < MTW; ++i) {
      const int ml = 16 * (MTW * mw + i) + r16;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const int c = 16 * h + 4 * g4;
        if constexpr (F32OUT) {
          float* const T = reinterpret_cast<float*>(sb);
          *reinterpret_cast<f32x4*>(T + ml * TP + c) = acc[h][i];
          if constexpr (BASE == EPI_PART_GU) *reinterpret_cast<f32x4*>(T + (kW2Rows + ml) * TP + c) = acc[h + H][i];
        } else {
          uint16_t* const T = reinterpret_cast<uint16_t*>(sb);
          uint16_t v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (BASE == EPI_SWIGLU)
              v[e] = swiglu_bf(acc[h][i][e], acc[h + H][i][e]);
            else
              v[e] = f2bf(acc[h][i][e]);
          }
          *reinterpret_cast<u32x2*>(T + ml * TP + c) =
              u32x2{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
        }
      }
    }
  };
  auto store_tile = [&](int rb, const char* sb) {
    for (int idx = tid; idx < M * HROWS; idx += 64 * W) {
      const int m = idx / HROWS, hr = idx - (idx / HROWS) * HROWS;
      const int n = rb * TR + hr;
      if (hr >= TR || n >= p.N) continue;
      if constexpr (F32OUT) {
        const float* const T = reinterpret_cast<const float*>(sb);
        store_agent(&p.part[((int64_t)slice * M + m) * p.N + n], T[m * TP + hr]);
        if constexpr (BASE == EPI_PART_GU)
          store_agent(&p.part[((int64_t)(S + slice) * M + m) * p.N + n], T[(kW2Rows + m) * TP + hr]);
      } else {
        p.C[(int64_t)m * p.ldc + n] = reinterpret_cast<const uint16_t*>(sb)[m * TP + hr];
      }
    }
  };

  auto argmax_tile = [&](int rb, const char* sb) {
    constexpr int QC = HROWS / 4;   // columns per thread
    static_assert(!LDS_ARGMAX || QC % 8 == 0, "16-byte LDS reads");
    const uint16_t* const T = reinterpret_cast<const uint16_t*>(sb);
    // a row's four threads are consecutive lanes, so the loop bound and the
    // exchanges below are uniform over each group of four
    for (int idx = tid; idx < 4 * M; idx += 64 * W) {
      const int m = idx >> 2, q = idx & 3;
      uint32_t bo = 0u;
      int bn = 0;
      // Not unrolled: with all QC columns unrolled the compiler computed every
      // column's bound check up front and held the masks in scalar registers
      // across the step loop (122 of them spilled to vector lanes, which cost
      // the MFMA loop its fragment registers: each fragment read then waited
      // for the one before, lm_head + argmax at 128 rows 212 against 204 us
      // for the logits GEMM of the same loop).
#pragma unroll 1
      for (int v = 0; v < QC / 8; ++v) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(T + m * TP + q * QC + 8 * v);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int hr = q * QC + 8 * v + k;
          const int n = rb * TR + hr;
          const uint32_t o = argmax_ord((uint16_t)(x[k >> 1] >> (16 * (k & 1))));
          if (hr < TR && n < p.N && o > bo) {   // increasing columns: ties keep the lowest
            bo = o;
            bn = n;
          }
        }
      }
      unsigned long long key = bo ? argmax_pack(bo, bn) : 0ull;
#pragma unroll
      for (int off = 1; off <= 2; off <<= 1) {
        const unsigned long long o = ((unsigned long long)(uint32_t)__shfl_xor((int)(key >> 32), off) << 32) |
                                     (uint32_t)__shfl_xor((int)(key & 0xFFFFFFFFu), off);
        key = o > key ? o : key;
      }
      if (q == 0 && key) atomicMax(&lds_best[m], key);
    }
  };

  auto step = [&](auto slot, int g) {
    constexpr int SL = decltype(slot)::value;   // g % D
    char* const sb = buf + (g & 1) * (SROWS * kW2Pitch);
    // Step g's rows are staged (by the previous step or the prologue).  After
    // the barrier every wave has finished step g - 1's reads of the other
    // buffer, so step g + 1 is staged there after this step's MFMAs are
    // issued, and its register slot then takes the loads of step g + 3.
    lds_barrier();
    // (a wave whose 32 activation rows all lie past M has nothing to
    // multiply; step G, run when G is odd, only stages and requests)
    if (g < G && 16 * MTW * mw < M) {
#pragma unroll
      for (int uu = 0; uu < UW; ++uu) {
        const int u = kh * UW + uu;
        bf16x8 af[MTW];
#pragma unroll
        for (int i = 0; i < MTW; ++i)
          af[i] = *reinterpret_cast<const bf16x8*>(sb + (ROWS + 16 * (MTW * mw + i) + r16) * kW2Pitch + 64 * u +
                                                   16 * g4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const bf16x8 wv = *reinterpret_cast<const bf16x8*>(sb + (16 * nt + r16) * kW2Pitch + 64 * u + 16 * g4);
#pragma unroll
          for (int i = 0; i < MTW; ++i)
            acc[nt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, af[i], acc[nt][i], 0, 0, 0);
        }
      }
    }
    stage(std::integral_constant<int, (SL + 1) % D>{}, g + 1);
    issue(std::integral_constant<int, (SL + 1) % D>{}, g + PF);
    if (g < G && (g + 1) % nsteps == 0) {   // the tile's last step
      if constexpr (KH == 2) {
        // Waves 4-7 hand their K half to waves 4 below through this step's
        // buffer: every wave has finished reading it after the barrier, and
        // it is written again only after step g + 1's barrier (staging step
        // g + 2), which waves 0-3 reach only once they have read it.
        float* const red = reinterpret_cast<float*>(sb);
        lds_barrier();
        if (kh == 1) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < MTW; ++i)
              *reinterpret_cast<f32x4*>(red + ((mw * NT + nt) * MTW + i) * 256 + 4 * lane) = acc[nt][i];
        }
        lds_barrier();
        if (kh == 0) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < MTW; ++i)
              acc[nt][i] += *reinterpret_cast<const f32x4*>(red + ((mw * NT + nt) * MTW + i) * 256 + 4 * lane);
        }
      }
      if constexpr (!LDS_OUT) {
        if (kh == 0) epilogue(tile_of(g));
      } else {
        // this step's buffer is free once every wave is past its reads
        // (fragments, or the K-part sums above); it is written again only
        // after step g + 1's barrier
        lds_barrier();
        if (kh == 0) write_tile(sb);
        lds_barrier();
        if constexpr (LDS_ARGMAX)
          argmax_tile(tile_of(g), sb);
        else
          store_tile(tile_of(g), sb);
      }
      zero_acc();
    }
  };
  static_assert(D == 2, "the loop below is unrolled for two slots");
  for (int g0 = 0; g0 < G; g0 += D) {
    step(std::integral_constant<int, 0>{}, g0);
    step(std::integral_constant<int, 1>{}, g0 + 1);
  }

  if constexpr (BASE == EPI_ARGMAX) {
    lds_barrier();
    argmax_fixup(p, lds_best, reinterpret_cast<int*>(lds_best + M));
  } else if constexpr (BASE == EPI_PART || BASE == EPI_PART_GU) {
    splitk_fixup<HROWS, BASE, RESID>(p, ntiles, rb0, reinterpret_cast<int*>(tail));
  }
}

}  // namespace sk
