// sk_kernels.hpp - gfx950 (CDNA4) kernels of the decode-GEMM hot path.
//
// Everything computes C[m, n] = sum_k A[m, k] * W[n, k] with bf16 inputs and
// fp32 accumulation, the contract of the reference's skinny GEMMs
// (engine/kernels/gemm.py:59-101, 124-168, 211-256).  Two inner products are
// provided and chosen per shape by the host table:
//
//  * MFMA path: one wavefront owns a tile of 16 weight rows (two tiles for
//    gate/up) and a range of K in units of 32 columns.  Weight rows are the
//    A operand of v_mfma_f32_16x16x32_bf16 (lane l: row l%16, 8 consecutive
//    columns at 8*(l/16)), so every lane streams 16-byte loads and each
//    16-lane group reads 64 contiguous bytes per row.  The activation rows are
//    the B operand, loaded once per wave and kept in registers for every tile
//    the wave visits.  Rows m >= M are zero lanes, so M = 1..16 costs the same
//    MFMA issue as M = 16 - irrelevant here, the matrix cores run at a few
//    percent of their rate while HBM is saturated.
//
//  * GEMV path: lanes span K (lane l: columns 8l..8l+7 of every 512-column
//    unit), so a wave instruction reads 1 KiB contiguous of one weight row.
//    Products use v_dot2_f32_bf16 (two bf16 products + fp32 add per lane op)
//    and each lane's partial sums are reduced across the wavefront with DPP
//    row operations plus readlane, in a fixed order.
//
// In both paths the waves of a workgroup share a tile and split its K range;
// their fp32 partials meet in LDS and are summed in wave order 0..W-1 by the
// epilogue (double-buffered, one barrier per tile).  A global split over
// workgroups writes fp32 partials that sk_splitk_reduce sums in split order
// 0..S-1.  No floating-point atomics anywhere: results are bitwise
// reproducible run to run.  The lm_head epilogue folds a greedy argmax in,
// using a packed (order key, ~index) 64-bit max that is order independent.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum Epi : int {
  EPI_STORE = 0,      // C = bf16(sum)
  EPI_SWIGLU = 1,     // C = bf16(bf16(silu(bf16 g)) * bf16 u)
  EPI_ARGMAX = 2,     // running (max, lowest index) per row, logits never stored
  EPI_PART = 3,       // fp32 partial of one global K split
  EPI_PART_GU = 4     // fp32 partials of gate and up for one global K split
};

// Kernel arguments, passed by value (one struct keeps the launch ABI simple).
struct Args {
  const uint16_t* A;      // activations [M, K], row stride lda
  const uint16_t* W0;     // weight rows (gate half for gate/up)
  const uint16_t* W1;     // up half for gate/up, else unused
  uint16_t* C;            // bf16 output [M, N], row stride ldc
  float* part;            // split-K partials [S][M][N] (gate/up: [2S][M][N])
  unsigned long long* best;  // argmax partials [gridDim.x][M]
  int64_t lda, ldw, ldc;
  int M, N, K;            // N = output columns (I for gate/up)
  int S;                  // global K splits (gridDim.x % S == 0)
  int slice_units;        // K units per global split
  int ku;                 // K units per wave
  int nrb;                // row blocks (tiles) along N
};

// ---------------------------------------------------------------------------
// bf16 helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// SwiGLU epilogue with the reference's cast placement
// (engine/kernels/gemm.py:115-121, engine/kernels/swiglu.py:23-24):
// bf16(gate), bf16(up), silu in fp32 rounded to bf16, product rounded to bf16.
__device__ __forceinline__ uint16_t swiglu_bf(float g, float u) {
  const float gb = round_bf(g);
  const float ub = round_bf(u);
  const float s = round_bf(gb / (1.0f + expf(-gb)));
  return f2bf(s * ub);
}

// Total order on bf16 values for argmax, packed with the column so that a
// plain unsigned max picks the largest value and, among equal values, the
// lowest column (torch.argmax / engine/kernels/topk.py:27-34).  -0 and +0 are
// equal; any NaN ranks above +inf.  Key 0 means "no candidate".
__device__ __forceinline__ unsigned long long argmax_key(uint16_t h, int n) {
  uint32_t ord;
  if ((h & 0x7FFFu) > 0x7F80u) {
    ord = 0x10001u;                                   // NaN
  } else {
    if (h == 0x8000u) h = 0;                          // -0 -> +0
    ord = (h & 0x8000u) ? (0xFFFFu - h) : (h | 0x8000u);
    ord += 1u;
  }
  return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)n);
}

__device__ __forceinline__ float argmax_key_value(unsigned long long key) {
  const uint32_t ord = (uint32_t)(key >> 32);
  if (ord == 0x10001u) return __uint_as_float(0x7FC00000u);
  const uint32_t o = ord - 1u;
  const uint32_t h = (o >= 0x8000u) ? (o - 0x8000u) : (0xFFFFu - o);
  return bf2f(h);
}

__device__ __forceinline__ int64_t argmax_key_index(unsigned long long key) {
  return (int64_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Weight loads are streamed once per call: mark them non-temporal so they do
// not evict the activations and partials from L2/MALL.
__device__ __forceinline__ u32x4 ld16_stream(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Eight bf16 products summed into acc with four v_dot2_f32_bf16.  The pairs are
// taken as .s01/.s23/.. of a bf16x8 view: hipcc 7.2 folds a per-component
// __builtin_bit_cast(bf16x2, v.y) of a u32x4 back to component 0.
__device__ __forceinline__ float dot8(u32x4 w, u32x4 a, float acc) {
  const bf16x8 wb = __builtin_bit_cast(bf16x8, w), ab = __builtin_bit_cast(bf16x8, a);
  acc = __builtin_amdgcn_fdot2_f32_bf16(wb.s01, ab.s01, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(wb.s23, ab.s23, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(wb.s45, ab.s45, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(wb.s67, ab.s67, acc, false);
  return acc;
}

// Sum over the 64 lanes of a wavefront, result valid in every lane.  Within
// each 16-lane row: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror (each adds the partner lane's value); then the four row sums are
// combined in the fixed order ((r0 + r1) + r2) + r3 through readlane.
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
  int iv = __float_as_int(v);
  int o;
  switch (ctrl_sel) {
    case 0: o = __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false); break;
    case 1: o = __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false); break;
    case 2: o = __builtin_amdgcn_mov_dpp(iv, 0x141, 0xF, 0xF, false); break;
    default: o = __builtin_amdgcn_mov_dpp(iv, 0x140, 0xF, 0xF, false); break;
  }
  return v + __int_as_float(o);
}

__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add(v, 0);
  v = dpp_add(v, 1);
  v = dpp_add(v, 2);
  v = dpp_add(v, 3);
  const int iv = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(iv, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(iv, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(iv, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(iv, 48));
  return ((r0 + r1) + r2) + r3;
}

// ---------------------------------------------------------------------------
// Shared epilogue: the waves' partial tiles sit in LDS as P[w][m][row]
// (ROWS rows per tile); sum them in wave order and finish the tile.
// ---------------------------------------------------------------------------
template <int ROWS, int EPI>
__device__ __forceinline__ void tile_epilogue(const Args& p, const float* P, int nw, int rb, int slice,
                                              unsigned long long* lds_best) {
  const int M = p.M;
  const int tid = threadIdx.x, nthr = blockDim.x;
  if constexpr (EPI == EPI_SWIGLU || EPI == EPI_PART_GU) {
    constexpr int HALF = ROWS / 2;
    const int nout = M * HALF;
    for (int idx = tid; idx < nout; idx += nthr) {
      const int m = idx / HALF, r = idx - (idx / HALF) * HALF;
      float g = 0.f, u = 0.f;
      for (int w = 0; w < nw; ++w) {
        g += P[(w * M + m) * ROWS + r];
        u += P[(w * M + m) * ROWS + r + HALF];
      }
      const int n = rb * HALF + r;
      if (n < p.N) {
        if constexpr (EPI == EPI_SWIGLU) {
          p.C[(int64_t)m * p.ldc + n] = swiglu_bf(g, u);
        } else {
          p.part[((int64_t)slice * M + m) * p.N + n] = g;
          p.part[((int64_t)(p.S + slice) * M + m) * p.N + n] = u;
        }
      }
    }
  } else {
    const int nout = M * ROWS;
    for (int idx = tid; idx < nout; idx += nthr) {
      const int m = idx / ROWS, r = idx - (idx / ROWS) * ROWS;
      float s = 0.f;
      for (int w = 0; w < nw; ++w) s += P[(w * M + m) * ROWS + r];
      const int n = rb * ROWS + r;
      if (n < p.N) {
        if constexpr (EPI == EPI_STORE) {
          p.C[(int64_t)m * p.ldc + n] = f2bf(s);
        } else if constexpr (EPI == EPI_PART) {
          p.part[((int64_t)slice * M + m) * p.N + n] = s;
        } else {  // EPI_ARGMAX
          atomicMax(&lds_best[m], argmax_key(f2bf(s), n));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA path.
//   MT : activation row tiles of 16 (M <= 16*MT)
//   NT : weight row tiles of 16 per workgroup tile (gate/up: 2 = gate + up)
//   KU : compile-time bound on K units (32 columns) per wave
// ---------------------------------------------------------------------------
template <int MT, int NT, int KU, int EPI>
__device__ __forceinline__ void mfma_body(Args p) {
  constexpr bool GATEUP = (EPI == EPI_SWIGLU || EPI == EPI_PART_GU);
  constexpr int ROWS = 16 * NT;                  // partial rows per tile in LDS
  constexpr int WROWS = GATEUP ? 16 : 16 * NT;   // output columns per tile
  static_assert(!GATEUP || NT == 2, "gate/up tiles pair 16 gate rows with 16 up rows");

  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = blockDim.x >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int M = p.M;

  const int S = p.S;
  const int slice = blockIdx.x % S;
  const int rbstep = gridDim.x / S;
  const int units = p.K >> 5;
  const int s_lo = slice * p.slice_units;
  const int s_hi = min(s_lo + p.slice_units, units);
  const int u_lo = s_lo + wave * p.ku;
  const int u_hi = min(u_lo + p.ku, s_hi);
  const int nu = __builtin_amdgcn_readfirstlane(max(0, u_hi - u_lo));
  const int kb = u_lo * 32 + 8 * g4;

  unsigned long long* lds_best = nullptr;
  float* parts = lds;
  const int part_floats = nw * M * ROWS;
  if constexpr (EPI == EPI_ARGMAX) {
    lds_best = reinterpret_cast<unsigned long long*>(lds + 2 * part_floats);
    if (tid < M) lds_best[tid] = 0ull;
  }

  // Activation fragments: lane holds A[16*mt + r16][kb + 32u .. +8].
  bf16x8 af[MT][KU];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r16;
    const uint16_t* ap = p.A + (int64_t)min(m, M - 1) * p.lda + kb;
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (u < nu) v = ld16(ap + 32 * u);
      if (m >= M) v = u32x4{0u, 0u, 0u, 0u};
      af[mt][u] = __builtin_bit_cast(bf16x8, v);
    }
  }

  // Weight row pointers of a tile (rows past N are clamped to N-1: the loads
  // stay in bounds and those columns are never stored).
  auto wrow = [&](int rb, int nt) -> const uint16_t* {
    if constexpr (GATEUP) {
      const int row = min(rb * 16 + r16, p.N - 1);
      return (nt == 0 ? p.W0 : p.W1) + (int64_t)row * p.ldw + kb;
    } else {
      const int row = min(rb * ROWS + 16 * nt + r16, p.N - 1);
      return p.W0 + (int64_t)row * p.ldw + kb;
    }
  };

  u32x4 wf[NT][KU];
  int rb = blockIdx.x / S;
  if (rb < p.nrb) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint16_t* wp = wrow(rb, nt);
#pragma unroll
      for (int u = 0; u < KU; ++u)
        if (u < nu) wf[nt][u] = ld16_stream(wp + 32 * u);
    }
  }

  int buf = 0;
  for (; rb < p.nrb; rb += rbstep) {
    const int rbn = rb + rbstep;
    const bool more = rbn < p.nrb;
    const uint16_t* wpn[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wpn[nt] = wrow(more ? rbn : rb, nt);

    f32x4 acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int u = 0; u < KU; ++u) {
      if (u < nu) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const bf16x8 wv = __builtin_bit_cast(bf16x8, wf[nt][u]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, af[mt][u], acc[nt][mt], 0, 0, 0);
          if (more) wf[nt][u] = ld16_stream(wpn[nt] + 32 * u);
        }
      }
    }

    // Lane holds tile rows 16*nt + 4*g4 + {0..3} for activation row 16*mt + r16.
    float* P = parts + buf * part_floats;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r16;
        if (m < M) *reinterpret_cast<f32x4*>(&P[(wave * M + m) * ROWS + 16 * nt + 4 * g4]) = acc[nt][mt];
      }
    __syncthreads();
    tile_epilogue<ROWS, EPI>(p, P, nw, rb, slice, lds_best);
    buf ^= 1;
    (void)WROWS;
  }

  if constexpr (EPI == EPI_ARGMAX) {
    __syncthreads();
    if (tid < M) p.best[(int64_t)blockIdx.x * M + tid] = lds_best[tid];
  }
}

// ---------------------------------------------------------------------------
// GEMV path (VALU).
//   MR : compile-time bound on activation rows (M <= MR)
//   R  : weight rows per tile (gate/up: R gate rows + R up rows)
//   KU : compile-time bound on K units (512 columns) per wave
// ---------------------------------------------------------------------------
template <int MR, int R, int KU, int EPI>
__device__ __forceinline__ void gemv_body(Args p) {
  constexpr bool GATEUP = (EPI == EPI_SWIGLU || EPI == EPI_PART_GU);
  constexpr int RR = GATEUP ? 2 * R : R;   // partial rows per tile

  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = blockDim.x >> 6;
  const int M = p.M;

  const int S = p.S;
  const int slice = blockIdx.x % S;
  const int rbstep = gridDim.x / S;
  const int units = (p.K + 511) >> 9;
  const int s_lo = slice * p.slice_units;
  const int s_hi = min(s_lo + p.slice_units, units);
  const int u_lo = s_lo + wave * p.ku;
  const int u_hi = min(u_lo + p.ku, s_hi);
  const int nu = __builtin_amdgcn_readfirstlane(max(0, u_hi - u_lo));
  const int kb = u_lo * 512 + 8 * lane;
  const int kend = min(s_hi * 512, p.K);

  unsigned long long* lds_best = nullptr;
  float* parts = lds;
  const int part_floats = nw * M * RR;
  if constexpr (EPI == EPI_ARGMAX) {
    lds_best = reinterpret_cast<unsigned long long*>(lds + 2 * part_floats);
    if (tid < M) lds_best[tid] = 0ull;
  }

  // Activation chunks: lane holds A[m][kb + 512u .. +8] (zero past the slice).
  u32x4 af[MR][KU];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const uint16_t* ap = p.A + (int64_t)min(m, M - 1) * p.lda + kb;
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M && u < nu && kb + 512 * u < kend) v = ld16(ap + 512 * u);
      af[m][u] = v;
    }
  }

  auto wrow = [&](int rb, int rr) -> const uint16_t* {
    if constexpr (GATEUP) {
      const int row = min(rb * R + (rr % R), p.N - 1);
      return (rr < R ? p.W0 : p.W1) + (int64_t)row * p.ldw + kb;
    } else {
      const int row = min(rb * R + rr, p.N - 1);
      return p.W0 + (int64_t)row * p.ldw + kb;
    }
  };

  u32x4 wf[RR][KU];
  int rb = blockIdx.x / S;
  if (rb < p.nrb) {
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) {
      const uint16_t* wp = wrow(rb, rr);
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        wf[rr][u] = u32x4{0u, 0u, 0u, 0u};
        if (u < nu && kb + 512 * u < kend) wf[rr][u] = ld16_stream(wp + 512 * u);
      }
    }
  }

  int buf = 0;
  for (; rb < p.nrb; rb += rbstep) {
    const int rbn = rb + rbstep;
    const bool more = rbn < p.nrb;

    float acc[RR][MR];
#pragma unroll
    for (int rr = 0; rr < RR; ++rr)
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[rr][m] = 0.f;

#pragma unroll
    for (int u = 0; u < KU; ++u) {
      if (u < nu) {
#pragma unroll
        for (int rr = 0; rr < RR; ++rr) {
#pragma unroll
          for (int m = 0; m < MR; ++m) acc[rr][m] = dot8(wf[rr][u], af[m][u], acc[rr][m]);
          if (more) {
            wf[rr][u] = u32x4{0u, 0u, 0u, 0u};
            if (kb + 512 * u < kend) wf[rr][u] = ld16_stream(wrow(rbn, rr) + 512 * u);
          }
        }
      }
    }

    float* P = parts + buf * part_floats;
#pragma unroll
    for (int rr = 0; rr < RR; ++rr)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float s = wave_sum(acc[rr][m]);
        if (m < M && lane == 0) P[(wave * M + m) * RR + rr] = s;
      }
    __syncthreads();
    tile_epilogue<RR, EPI>(p, P, nw, rb, slice, lds_best);
    buf ^= 1;
  }

  if constexpr (EPI == EPI_ARGMAX) {
    __syncthreads();
    if (tid < M) p.best[(int64_t)blockIdx.x * M + tid] = lds_best[tid];
  }
}

// ---------------------------------------------------------------------------
// Global split-K reduction: C = bf16(sum_{s=0..S-1} part[s]) (gate/up: swiglu
// of the two sums), the order of the reference's _sum_kernel /
// _sum_gateup_kernel (engine/kernels/gemm.py:104-112, 171-181).
// ---------------------------------------------------------------------------
template <bool GATEUP>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ C,
                                                            int64_t ldc, int M, int N, int S) {
  const int64_t MN = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += (int64_t)gridDim.x * blockDim.x) {
    float g = 0.f, u = 0.f;
    for (int s = 0; s < S; ++s) {
      g += part[s * MN + i];
      if constexpr (GATEUP) u += part[(S + s) * MN + i];
    }
    const int m = (int)(i / N), n = (int)(i - (int64_t)(i / N) * N);
    C[(int64_t)m * ldc + n] = GATEUP ? swiglu_bf(g, u) : f2bf(g);
  }
}

#ifdef SK_AUX_KERNELS
// Non-template kernels: defined only in the translation unit that launches
// them (sk_abi.hip), so every other unit can include this header.
// Final argmax over G per-workgroup candidates best[g*M + m]; one workgroup
// per row.  The packed-key max is order independent, so any reduction tree
// gives the same (value, lowest index).
__global__ void __launch_bounds__(256) argmax_final_kernel(const unsigned long long* __restrict__ best, int G, int M,
                                                           int64_t* __restrict__ ids, float* __restrict__ maxv) {
  __shared__ unsigned long long red[256];
  const int m = blockIdx.x;
  unsigned long long b = 0ull;
  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    const unsigned long long v = best[(int64_t)g * M + m];
    b = v > b ? v : b;
  }
  red[threadIdx.x] = b;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      const unsigned long long o = red[threadIdx.x + s];
      if (o > red[threadIdx.x]) red[threadIdx.x] = o;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    ids[m] = argmax_key_index(red[0]);
    maxv[m] = argmax_key_value(red[0]);
  }
}

// Argmax over materialised bf16 logits: workgroup (c, m) scans chunk c of row m.
__global__ void __launch_bounds__(256) argmax_partial_kernel(const uint16_t* __restrict__ L, int64_t ld, int M, int V,
                                                             int chunk, int vec, unsigned long long* __restrict__ best) {
  __shared__ unsigned long long red[256];
  const int m = blockIdx.y, c = blockIdx.x;
  const uint16_t* row = L + (int64_t)m * ld;
  const int lo = c * chunk, hi = min(lo + chunk, V);
  unsigned long long b = 0ull;
  // 8-column vector loads over the body when rows are 16-byte aligned
  // (vec: L aligned and ld % 8 == 0; lo is a multiple of chunk, itself of 8),
  // scalar loads for the tail and for unaligned layouts.
  const int vhi = vec ? lo + ((hi - lo) & ~7) : lo;
  for (int k = lo + 8 * threadIdx.x; k < vhi; k += 8 * blockDim.x) {
    const u32x4 v = ld16(row + k);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned long long k0 = argmax_key((uint16_t)(w[j] & 0xFFFFu), k + 2 * j);
      const unsigned long long k1 = argmax_key((uint16_t)(w[j] >> 16), k + 2 * j + 1);
      b = k0 > b ? k0 : b;
      b = k1 > b ? k1 : b;
    }
  }
  for (int k = vhi + threadIdx.x; k < hi; k += blockDim.x) {
    const unsigned long long kk = argmax_key(row[k], k);
    b = kk > b ? kk : b;
  }
  red[threadIdx.x] = b;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      const unsigned long long o = red[threadIdx.x + s];
      if (o > red[threadIdx.x]) red[threadIdx.x] = o;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) best[(int64_t)c * M + m] = red[0];
}

// ---------------------------------------------------------------------------
// Residual add + RMSNorm (engine/kernels/add_rmsnorm.py:15-29 casts):
//   s = bf16(x + y) -> xout;  r = 1/sqrt(sum(s^2)/K + eps) (fp32);
//   out = bf16(w * bf16(s * r)).
// One workgroup of 256 threads per row, 8 columns per thread per chunk.
// ---------------------------------------------------------------------------
constexpr int RMS_THREADS = 256;
constexpr int RMS_MAX_CHUNKS = 8;   // K <= 256 * 8 * 8 = 16384

__global__ void __launch_bounds__(RMS_THREADS) add_rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ y,
                                                                  const uint16_t* __restrict__ w, float eps,
                                                                  uint16_t* __restrict__ xout,
                                                                  uint16_t* __restrict__ out, int K, int64_t ld) {
  __shared__ float wsum[RMS_THREADS / 64];
  const int m = blockIdx.x;
  const uint16_t* xr = x + (int64_t)m * ld;
  const uint16_t* yr = y + (int64_t)m * ld;
  uint16_t* xo = xout + (int64_t)m * ld;
  uint16_t* orow = out + (int64_t)m * ld;
  const int nchunk = K >> 3;
  u32x4 sv[RMS_MAX_CHUNKS];
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < RMS_MAX_CHUNKS; ++j) {
    const int c = threadIdx.x + j * RMS_THREADS;
    sv[j] = u32x4{0u, 0u, 0u, 0u};
    if (c < nchunk) {
      const u32x4 a = ld16(xr + 8 * c), b = ld16(yr + 8 * c);
      const uint32_t aa[4] = {a.x, a.y, a.z, a.w}, bb[4] = {b.x, b.y, b.z, b.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint16_t lo = f2bf(bf2f(aa[q] & 0xFFFFu) + bf2f(bb[q] & 0xFFFFu));
        const uint16_t hi = f2bf(bf2f(aa[q] >> 16) + bf2f(bb[q] >> 16));
        const float flo = bf2f(lo), fhi = bf2f(hi);
        sq += flo * flo;
        sq += fhi * fhi;
        o[q] = (uint32_t)lo | ((uint32_t)hi << 16);
      }
      sv[j] = u32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(xo + 8 * c) = sv[j];
    }
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = sq;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < RMS_THREADS / 64; ++i) tot += wsum[i];
  const float rstd = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
  for (int j = 0; j < RMS_MAX_CHUNKS; ++j) {
    const int c = threadIdx.x + j * RMS_THREADS;
    if (c < nchunk) {
      const u32x4 wv = ld16(w + 8 * c);
      const uint32_t ss[4] = {sv[j].x, sv[j].y, sv[j].z, sv[j].w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint16_t lo = f2bf(bf2f(ww[q] & 0xFFFFu) * round_bf(bf2f(ss[q] & 0xFFFFu) * rstd));
        const uint16_t hi = f2bf(bf2f(ww[q] >> 16) * round_bf(bf2f(ss[q] >> 16) * rstd));
        o[q] = (uint32_t)lo | ((uint32_t)hi << 16);
      }
      *reinterpret_cast<u32x4*>(orow + 8 * c) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

// Unfused SwiGLU over gu = [g | u] (engine/kernels/swiglu.py:14-24).
__global__ void __launch_bounds__(256) swiglu_kernel(const uint16_t* __restrict__ gu, int64_t ld_gu,
                                                     uint16_t* __restrict__ out, int64_t ld_out, int M, int I) {
  const int64_t total = (int64_t)M * I;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(t / I), i = (int)(t - (int64_t)(t / I) * I);
    const float g = bf2f(gu[(int64_t)m * ld_gu + i]);
    const float u = bf2f(gu[(int64_t)m * ld_gu + I + i]);
    out[(int64_t)m * ld_out + i] = swiglu_bf(g, u);
  }
}

#endif  // SK_AUX_KERNELS

}  // namespace sk
