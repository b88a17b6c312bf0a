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
// workgroups writes fp32 partials to a workspace; the last workgroup to
// arrive at a tile sums them in split order 0..S-1 inside the same kernel.
// No floating-point atomics anywhere: results are bitwise reproducible run to
// run.  The lm_head epilogue folds a greedy argmax in, using a packed
// (order key, ~index) 64-bit max that is order independent.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace sk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

enum Epi : int {
  EPI_STORE = 0,      // C = bf16(sum)
  EPI_SWIGLU = 1,     // C = bf16(bf16(silu(bf16 g)) * bf16 u)
  EPI_ARGMAX = 2,     // running (max, lowest index) per row, logits never stored
  EPI_PART = 3,       // fp32 partial of one global K split
  EPI_PART_GU = 4,    // fp32 partials of gate and up for one global K split
  // The first three again, with the residual-add + RMSNorm prologue applied to
  // the activation rows as they are loaded (one global K split only).
  EPI_STORE_NORM = 5,
  EPI_SWIGLU_NORM = 6,
  EPI_ARGMAX_NORM = 7,
  // The first three again, consuming activations the producer of the previous
  // projection already summed (x + y, kept as the residual) and whose per-row
  // sums of squares it left as partials over 16-column groups: the RMSNorm is
  // finished here from those partials (LDS-fed MFMA ring path only).
  EPI_STORE_PRE = 8,
  EPI_SWIGLU_PRE = 9,
  EPI_ARGMAX_PRE = 10,
  // Plain projection (one K split, or split-K partials) whose output y is not
  // stored: the residual xout = bf16(r + bf16(y)) is, with the sums of
  // squares of each 16-column group of xout (the next norm's partials).
  EPI_STORE_RESID = 11,
  EPI_PART_RESID = 12
};

// Kernel arguments, passed by value (one struct keeps the launch ABI simple).
struct Args {
  const uint16_t* A;      // activations [M, K], row stride lda
  const uint16_t* W0;     // weight rows (gate half for gate/up)
  const uint16_t* W1;     // up half for gate/up, else unused
  uint16_t* C;            // bf16 output [M, N], row stride ldc
  float* part;            // split-K partials [S][M][N] (gate/up: [2S][M][N])
  unsigned long long* best;  // argmax: per-row packed best [M]; zero between calls
  unsigned* tickets;      // arrival counters (one per tile, or one for argmax); zero between calls
  int64_t lda, ldw, ldc;
  int M, N, K;            // N = output columns (I for gate/up)
  int S;                  // global K splits (grid % S == 0)
  int slice_units;        // K units per global split
  int ku;                 // K units per wave
  int nrb;                // row blocks (tiles) along N
  int tr;                 // output columns per tile: tile rb covers [rb*tr, rb*tr + tr); at most the
                          // compile-time OUT_ROWS (the ring path takes fewer: the loads of a slab's
                          // rows past tr read the zero line, their MFMA rows are never read)
  int nw;                 // waves per workgroup (blockDim.x / 64)
  int grid;               // workgroups launched (gridDim.x)
  int rbstep;             // grid / S: tile stride of one workgroup
  // Norm prologue (EPI_*_NORM only): A holds x; the GEMM consumes
  // bf16(NW * bf16(s * rstd(s))) with s = bf16(x + Y), and workgroup 0 writes
  // s to XO.  Y and XO share the row stride lda.
  const uint16_t* Y;
  const uint16_t* NW;
  uint16_t* XO;
  float eps;
  // Residual hand-off (EPI_*_PRE consume, EPI_*_RESID produce): R residual in,
  // RO residual out (row stride ldr), SQ per-row partial sums of squares over
  // 16-column groups of RO, row stride sq_ld floats.  The PRE epilogues read
  // SQ and the norm weights NW with eps; their K is the producer's N.
  const uint16_t* R;
  uint16_t* RO;
  int64_t ldr;
  float* SQ;
  int sq_ld;
  // LDS buffers for the waves' fp32 partial tiles on the ring path: 2 (tile
  // j + 1 writes while tile j is reduced), or 1 when two do not fit (one more
  // barrier per tile).  The other bodies always use 2.
  int pbuf;
  // Row groups (ring path only): groups > 1 launches `groups` grids of `grid`
  // workgroups, group g computing rows [g*mrows, min(M, (g+1)*mrows)); the
  // workspace holds one region of counters and partials per group.
  int groups, mrows;
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

// The key's halves on their own: the value's order (1 .. 0x10001) and the
// packing of an order with its column.
__device__ __forceinline__ uint32_t argmax_ord(uint16_t h) { return (uint32_t)(argmax_key(h, 0) >> 32); }
__device__ __forceinline__ unsigned long long argmax_pack(uint32_t ord, int n) {
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

// 128 zero bytes in device memory (never written): the source of loads for
// columns outside K, so that such loads need neither a branch nor a mask on
// the loaded data.
static __device__ __attribute__((aligned(128))) uint32_t kZeroLine[32] = {};

// Padding of every LDS row that holds MFMA fragment data (a lane reads 16
// bytes of row r16 at column byte 64u + 16 g4).  On gfx950 those reads run at
// the full LDS rate when the row pitch in dwords is 8 or 24 mod 32 and at
// ~60% of it when it is 4 mod 32 (measured with eight waves per CU: 288- and
// 544-byte rows 367-382 B/ns per CU like linear reads, 272- and 528-byte rows
// 230-241, 384-byte rows 139), so 256- and 512-byte rows get 32 bytes.
constexpr int kRowPad = 32;

// Data read once per call (weights, K/V cache rows): non-temporal loads, so it
// does not evict the activations and partials from L2/MALL.
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
// Residual add + RMSNorm on packed bf16 (engine/kernels/add_rmsnorm.py:15-29,
// casts as rmsnorm.py:34-45):  s = bf16(x + y);  rstd = 1/sqrt(sum(s^2)/K + eps)
// in fp32;  a = bf16(w * bf16(s * rstd)).
// ---------------------------------------------------------------------------
// s = bf16(x + y) for 8 columns; adds their squares to sq in column order.
__device__ __forceinline__ u32x4 add_bf16x8(u32x4 x, u32x4 y, float& sq) {
  u32x4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint16_t lo = f2bf(bf2f(x[q] & 0xFFFFu) + bf2f(y[q] & 0xFFFFu));
    const uint16_t hi = f2bf(bf2f(x[q] >> 16) + bf2f(y[q] >> 16));
    const float flo = bf2f(lo), fhi = bf2f(hi);
    sq += flo * flo;
    sq += fhi * fhi;
    r[q] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  return r;
}

__device__ __forceinline__ float rms_rstd(float sumsq, int K, float eps) {
  return 1.0f / sqrtf(sumsq / (float)K + eps);
}

// bf16(w * bf16(s * rstd)) for 8 columns.
__device__ __forceinline__ u32x4 norm_bf16x8(u32x4 s, u32x4 w, float rstd) {
  // Re-expand s from its packed bits here: an empty asm hides the packed
  // value's origin, so the compiler does not keep the fp32 copies made when s
  // was formed alive until now (twice the registers).
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t t = s[q];
    asm volatile("" : "+v"(t));
    s[q] = t;
  }
  u32x4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint16_t lo = f2bf(bf2f(w[q] & 0xFFFFu) * round_bf(bf2f(s[q] & 0xFFFFu) * rstd));
    const uint16_t hi = f2bf(bf2f(w[q] >> 16) * round_bf(bf2f(s[q] >> 16) * rstd));
    r[q] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  return r;
}

// The same for 8 columns of one row, with the weights given as bf16 pairs with
// one half zeroed (wlo[q] = (w[2q], 0), whi[q] = (0, w[2q+1])): after the
// first rounding the product w * y comes from v_dot2_f32_bf16 straight off the
// packed bf16 pair; one bf16 x bf16 product plus a zero product is exact in
// fp32, so the result equals the fp32 product rounded once, as above.
__device__ __forceinline__ u32x4 norm_line_bf16x8(u32x4 x, const u32x4& wlo, const u32x4& whi, float rstd) {
  // The pairs are taken as .s01/.s23/.. of a bf16x8 view (see dot8).
  const bf16x8 wl = __builtin_bit_cast(bf16x8, wlo), wh = __builtin_bit_cast(bf16x8, whi);
  const bf16x2 wlp[4] = {wl.s01, wl.s23, wl.s45, wl.s67};
  const bf16x2 whp[4] = {wh.s01, wh.s23, wh.s45, wh.s67};
  u32x4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x2 t = {bf2f(x[q] & 0xFFFFu) * rstd, bf2f(x[q] >> 16) * rstd};
    const bf16x2 yb = __builtin_convertvector(t, bf16x2);   // one v_cvt_pk_bf16_f32 (RNE)
    const f32x2 h = {__builtin_amdgcn_fdot2_f32_bf16(yb, wlp[q], 0.0f, false),
                     __builtin_amdgcn_fdot2_f32_bf16(yb, whp[q], 0.0f, false)};
    r[q] = __builtin_bit_cast(uint32_t, __builtin_convertvector(h, bf16x2));
  }
  return r;
}

// ---------------------------------------------------------------------------
// Shared tile epilogue.  The waves' partial tiles sit in LDS as P[w][m][row]
// (ROWS rows per tile); they are summed in wave order and the finished values
// go to an LDS staging area (or, for argmax, into a per-row running best).
// Nothing here touches global memory: the weight-streaming loop then issues
// only weight loads, so the compiler can keep all of them in flight (global
// stores would share the vmcnt counter with those loads).
// ---------------------------------------------------------------------------
constexpr bool epi_norm(int e) { return e >= EPI_STORE_NORM && e <= EPI_ARGMAX_NORM; }
constexpr bool epi_pre(int e) { return e >= EPI_STORE_PRE && e <= EPI_ARGMAX_PRE; }
constexpr int epi_base(int e) {   // the epilogue proper, without prologue or residual hand-off
  return epi_norm(e) ? e - EPI_STORE_NORM
         : epi_pre(e) ? e - EPI_STORE_PRE
         : e == EPI_STORE_RESID ? EPI_STORE
         : e == EPI_PART_RESID  ? EPI_PART
                                : e;
}
constexpr bool epi_gateup(int e) { return epi_base(e) == EPI_SWIGLU || epi_base(e) == EPI_PART_GU; }

template <int EPI>
struct EpiTraits {
  static constexpr bool norm = epi_norm(EPI);
  static constexpr bool pre = epi_pre(EPI);
  static constexpr bool resid = EPI == EPI_STORE_RESID || EPI == EPI_PART_RESID;
  static constexpr int base = epi_base(EPI);
  static constexpr bool gateup = epi_gateup(EPI);
  // bytes per staged output element (PART_GU stages gate and up fp32 sums)
  static constexpr int stage_bytes = base == EPI_STORE || base == EPI_SWIGLU ? 2 : (base == EPI_PART ? 4 : 8);
};

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum the partials of tile j (output columns rb*OUT_ROWS + r) into staging.
// The partials of (wave w, row m) start at P[(w*M + m) * PST].
template <int ROWS, int EPI, int PST = ROWS>
__device__ __forceinline__ void tile_reduce(const Args& p, const float* P, int nw, int rb, int j, void* stage,
                                            unsigned long long* lds_best) {
  constexpr bool GU = EpiTraits<EPI>::gateup;
  constexpr int OUT_ROWS = GU ? ROWS / 2 : ROWS;
  const int M = p.M;
  const int tid = threadIdx.x, nthr = 64 * p.nw;
  const int nout = M * OUT_ROWS;
  const int TR = p.tr;
  for (int idx = tid; idx < nout; idx += nthr) {
    const int m = idx / OUT_ROWS, r = idx - (idx / OUT_ROWS) * OUT_ROWS;
    if (r >= TR) continue;   // tile rows past tr: nothing to finish
    // Four waves' partials per step are read together (independent LDS loads
    // in flight), then added in wave order 0..nw-1; slots past nw-1 read wave
    // nw-1's slot (in bounds) and are masked to +0.
    float g = 0.f, u = 0.f;
    for (int w0 = 0; w0 < nw; w0 += 4) {
      float pg[4], pu[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ws = min(w0 + i, nw - 1);
        pg[i] = P[(ws * M + m) * PST + r];
        if constexpr (GU) pu[i] = P[(ws * M + m) * PST + r + OUT_ROWS];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t keep = w0 + i < nw ? 0xFFFFFFFFu : 0u;
        g += __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, pg[i]) & keep);
        if constexpr (GU) u += __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, pu[i]) & keep);
      }
    }
    const int sidx = (j * M + m) * OUT_ROWS + r;
    if constexpr (EPI == EPI_STORE) {
      static_cast<uint16_t*>(stage)[sidx] = f2bf(g);
    } else if constexpr (EPI == EPI_SWIGLU) {
      static_cast<uint16_t*>(stage)[sidx] = swiglu_bf(g, u);
    } else if constexpr (EPI == EPI_PART) {
      static_cast<float*>(stage)[sidx] = g;
    } else if constexpr (EPI == EPI_PART_GU) {
      static_cast<float*>(stage)[2 * sidx] = g;
      static_cast<float*>(stage)[2 * sidx + 1] = u;
    } else {   // EPI_ARGMAX
      const int n = rb * TR + r;
      if (n < p.N) atomicMax(&lds_best[m], argmax_key(f2bf(g), n));
    }
  }
}

// Device-coherent (agent scope) accesses for data exchanged between
// workgroups: they bypass the non-coherent per-XCD L2 state (sc1), so no
// full-L2 writeback/invalidate fence is needed around them.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Write the staged outputs of this workgroup's tiles (after the stream).
// Split-K partials are stored device-coherent for the fixup below.
// Residual hand-off for output element (m, n) with bf16 projection value yb
// and residual rb = R[m][n] (resid_in; the split-K finish requests it with the
// partials, so it costs no round trip of its own):
// xout = bf16(r + y) goes to RO and the sum of xout^2 over each 16-column
// group (the 16 consecutive lanes that hold it, added in a fixed butterfly
// order) goes to SQ[m][n / 16].  Every lane of the group must call this;
// ok = false (a column past N) contributes zero and stores nothing.
__device__ __forceinline__ uint16_t resid_in(const Args& p, int m, int n, bool ok) {
  return ok ? p.R[(int64_t)m * p.ldr + n] : (uint16_t)0;
}
__device__ __forceinline__ void resid_out(const Args& p, int m, int n, bool ok, uint16_t yb, uint16_t rb) {
  const float xo = ok ? round_bf(bf2f(rb) + bf2f(yb)) : 0.f;
  if (ok) p.RO[(int64_t)m * p.ldr + n] = f2bf(xo);
  float sq = xo * xo;
  sq += __shfl_xor(sq, 1);
  sq += __shfl_xor(sq, 2);
  sq += __shfl_xor(sq, 4);
  sq += __shfl_xor(sq, 8);
  if ((n & 15) == 0 && ok) p.SQ[(int64_t)m * p.sq_ld + (n >> 4)] = sq;
}

template <int OUT_ROWS, int EPI, bool RESID = false>
__device__ __forceinline__ void flush_stage(const Args& p, const void* stage, int ntiles, int rb0, int slice) {
  static_assert(!RESID || OUT_ROWS % 16 == 0, "16-column groups of one tile");
  const int M = p.M;
  const int total = ntiles * M * OUT_ROWS;
  // Consecutive idx hold consecutive columns of one (tile, row): with OUT_ROWS
  // a multiple of 16, each 16-column group is 16 consecutive lanes of a wave.
  for (int idx = threadIdx.x; idx < total; idx += 64 * p.nw) {
    const int r = idx % OUT_ROWS;
    const int jm = idx / OUT_ROWS;
    const int m = jm % M, j = jm / M;
    // (the residual hand-off runs with tr = OUT_ROWS: 16-column groups of one tile)
    const int n = (rb0 + j * p.rbstep) * p.tr + r;
    if constexpr (RESID) {
      static_assert(EPI == EPI_STORE, "the residual follows a finished projection");
      resid_out(p, m, n, n < p.N, static_cast<const uint16_t*>(stage)[idx], resid_in(p, m, n, n < p.N));
      continue;
    }
    if (r >= p.tr || n >= p.N) continue;
    if constexpr (EPI == EPI_STORE || EPI == EPI_SWIGLU) {
      p.C[(int64_t)m * p.ldc + n] = static_cast<const uint16_t*>(stage)[idx];
    } else if constexpr (EPI == EPI_PART) {
      store_agent(&p.part[((int64_t)slice * M + m) * p.N + n], static_cast<const float*>(stage)[idx]);
    } else if constexpr (EPI == EPI_PART_GU) {
      store_agent(&p.part[((int64_t)slice * M + m) * p.N + n], static_cast<const float*>(stage)[2 * idx]);
      store_agent(&p.part[((int64_t)(p.S + slice) * M + m) * p.N + n], static_cast<const float*>(stage)[2 * idx + 1]);
    }
  }
}

// Cross-workgroup completion without a second kernel.  Every workgroup
// publishes its partial results with device-coherent stores (or, for argmax,
// a device-scope 64-bit atomic max of its packed candidates), waits until they
// are performed, then takes a ticket on an arrival counter.  The workgroup
// that arrives last for a tile (or, for argmax, for the whole grid) reads
// every contribution with device-coherent loads and finishes the output,
// then resets what it used to zero for the next call.  Split-K sums run in
// fixed split order s = 0..S-1 and the key max is order independent, so the
// result never depends on which workgroup arrives last; no workgroup waits.
__device__ __forceinline__ bool take_ticket(unsigned* ticket, unsigned expected) {
  const unsigned old = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool last = (old == expected - 1u);
  if (last) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// Splits whose partials are requested together before the first add: a
// finish costs one memory round trip per batch of splits, not one per split
// and output.
constexpr int kFixupBatch = 4;

template <int OUT_ROWS, int EPI, bool RESID = false>
__device__ __forceinline__ void splitk_fixup(const Args& p, int ntiles, int rb0, int* lds_flags) {
  const int M = p.M, S = p.S;
  const int64_t MN = (int64_t)M * p.N;
  const int nthr = 64 * p.nw;
  __builtin_amdgcn_s_waitcnt(0);   // this thread's partial stores are performed
  __syncthreads();
  // Tickets of up to `cap` tiles per round, one thread per tile so they are
  // taken together (the flags reuse the partials' LDS).
  const int cap = min(2 * p.nw * M * OUT_ROWS, nthr);
  for (int j0 = 0; j0 < ntiles; j0 += cap) {
    const int jn = min(ntiles - j0, cap);
    if ((int)threadIdx.x < jn)
      lds_flags[threadIdx.x] = take_ticket(&p.tickets[rb0 + (j0 + threadIdx.x) * p.rbstep], (unsigned)S) ? 1 : 0;
    __syncthreads();
    for (int j = 0; j < jn; ++j) {
      if (!lds_flags[j]) continue;
      const int rb = rb0 + (j0 + j) * p.rbstep;
      // Every output of the tile is finished by one thread; a thread's outputs
      // (up to 4 per pass) issue all their partial loads before any add.
      for (int base = 0; base < M * OUT_ROWS; base += 4 * nthr) {
        constexpr int NP = EPI == EPI_PART_GU ? 2 : 1;   // gate and up partials
        float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
        int64_t e[4];
        uint16_t rres[4];   // RESID: the residual, requested with the partials
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int idx = min(base + (int)threadIdx.x + i * nthr, M * OUT_ROWS - 1);
          const int m = idx / OUT_ROWS, n = rb * p.tr + idx % OUT_ROWS;
          e[i] = (int64_t)m * p.N + (n < p.N ? n : 0);   // clamped in bounds; stored only if real
          if constexpr (RESID) rres[i] = resid_in(p, m, n, n < p.N);
        }
        // Sums in split order s = 0..S-1, all loads of a batch issued first.
        for (int s0 = 0; s0 < S; s0 += kFixupBatch) {
          float v[NP][4][kFixupBatch];
#pragma unroll
          for (int h = 0; h < NP; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
              for (int k = 0; k < kFixupBatch; ++k)
                v[h][i][k] = load_agent(&p.part[((int64_t)h * S + min(s0 + k, S - 1)) * MN + e[i]]);
#pragma unroll
          for (int k = 0; k < kFixupBatch; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (s0 + k < S) {
                g[i] += v[0][i][k];
                if constexpr (NP == 2) u[i] += v[NP - 1][i][k];
              }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int idx = base + (int)threadIdx.x + i * nthr;
          const int m = idx / OUT_ROWS, r = idx % OUT_ROWS;
          const int n = rb * p.tr + r;
          if constexpr (RESID) {
            // every lane of a 16-column group takes part in the group sum
            // (idx < M*OUT_ROWS is uniform over each 16-lane group)
            static_assert(EPI == EPI_PART && OUT_ROWS % 16 == 0, "residual after split-K partials");
            if (idx < M * OUT_ROWS) resid_out(p, m, n, n < p.N, f2bf(n < p.N ? g[i] : 0.f), rres[i]);
            continue;
          }
          if (idx >= M * OUT_ROWS || r >= p.tr || n >= p.N) continue;
          p.C[(int64_t)m * p.ldc + n] = (EPI == EPI_PART_GU) ? swiglu_bf(g[i], u[i]) : f2bf(g[i]);
        }
      }
    }
    __syncthreads();   // flags are rewritten by the next round
  }
}

// Final argmax: every workgroup folds its per-row best into best[m] with a
// device-scope atomic max; the last to arrive decodes best[m] into ids/maxv
// (passed through p.C as int64* and p.part as float*) and clears best[m].
__device__ __forceinline__ void argmax_fixup(const Args& p, const unsigned long long* lds_best, int* lds_flag) {
  const int M = p.M;
  if ((int)threadIdx.x < M)
    __hip_atomic_fetch_max(&p.best[threadIdx.x], lds_best[threadIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) *lds_flag = take_ticket(&p.tickets[0], (unsigned)p.grid) ? 1 : 0;
  __syncthreads();
  if (!*lds_flag) return;
  if ((int)threadIdx.x < M) {
    const unsigned long long b =
        __hip_atomic_exchange(&p.best[threadIdx.x], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    reinterpret_cast<int64_t*>(p.C)[threadIdx.x] = argmax_key_index(b);
    p.part[threadIdx.x] = argmax_key_value(b);
  }
}

// LDS layout of both kernel families:
//   [partials: 2 buffers x nw x M x ROWS fp32][staging or argmax best]
// Tiles of workgroup b: rb = b/S + j*(gridDim.x/S), j < ntiles.
__device__ __forceinline__ int wg_tiles(int rb0, int rbstep, int nrb) {
  return rb0 < nrb ? (nrb - 1 - rb0) / rbstep + 1 : 0;
}

// Row groups (the grouped entry points only).  Launch position x = 8*i + x8
// runs workgroup b = 8*(i / groups) + x8 of group g = i % groups (the host
// guarantees grid % 8 == 0, so this is a bijection onto groups x grid).  Workgroups are dealt to the 8 XCDs
// round-robin, so workgroup b of every group runs on XCD b % 8, next to its
// siblings, and streams the same weight tiles: the first group's loads fill
// that XCD's L2 and the siblings' hit it.  Each group is an independent GEMM
// on its rows: the pointers move to its rows and to its own region of
// arrival counters and split-K partials.  Returns b.
template <int EPI>
__device__ __forceinline__ unsigned enter_row_group(Args& p) {
  if (p.groups <= 1) return blockIdx.x;
  const int i = blockIdx.x >> 3;
  const int g = i % p.groups;
  const int m0 = g * p.mrows;
  p.A += (int64_t)m0 * p.lda;
  p.M = min(p.mrows, p.M - m0);
  constexpr int BASE = EpiTraits<EPI>::base;
  if constexpr (BASE == EPI_ARGMAX) {
    p.best += m0;
    p.C = reinterpret_cast<uint16_t*>(reinterpret_cast<int64_t*>(p.C) + m0);   // ids
    p.part += m0;                                                             // max logits
    p.tickets += g;
  } else {
    if (p.C) p.C += (int64_t)m0 * p.ldc;
    if constexpr (BASE == EPI_PART || BASE == EPI_PART_GU) {
      p.part += (int64_t)g * (BASE == EPI_PART_GU ? 2 : 1) * p.S * p.mrows * p.N;
      p.tickets += g * p.nrb;
    }
  }
  if constexpr (EpiTraits<EPI>::resid) {
    p.R += (int64_t)m0 * p.ldr;
    p.RO += (int64_t)m0 * p.ldr;
  }
  if constexpr (EpiTraits<EPI>::resid || EpiTraits<EPI>::pre) p.SQ += (int64_t)m0 * p.sq_ld;
  return 8u * (i / p.groups) + (blockIdx.x & 7u);
}

// ---------------------------------------------------------------------------
// MFMA path.
//   MT : activation row tiles of 16 (M <= 16*MT)
//   NT : weight row tiles of 16 per workgroup tile (gate/up: 2 = gate + up)
//   KU : compile-time bound on K units (32 columns) per wave
// The per-tile loop is branch-free: every wave always issues NT*KU weight
// loads (units past the wave's range reload its last unit and meet zero
// activations), and the last tile is peeled so that its iteration issues no
// prefetch.  The compiler can then keep the next tile's NT*KU loads in flight
// while the current tile's MFMAs run.
// ---------------------------------------------------------------------------
template <int MT, int NT, int KU, int EPI>
__device__ __forceinline__ void mfma_body(Args p) {
  constexpr bool GATEUP = EpiTraits<EPI>::gateup;
  constexpr int BASE = EpiTraits<EPI>::base;   // epilogue without the norm prologue
  constexpr bool NORM = EpiTraits<EPI>::norm;
  static_assert(!NORM, "the register-fragment MFMA path has no norm prologue");
  constexpr int ROWS = 16 * NT;                  // partial rows per tile in LDS
  constexpr int OUT_ROWS = GATEUP ? 16 : ROWS;   // output columns per tile
  static_assert(!GATEUP || NT == 2, "gate/up tiles pair 16 gate rows with 16 up rows");

  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = p.nw;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int M = p.M;

  const int S = p.S;
  const int slice = blockIdx.x % S;
  const int rbstep = p.rbstep;
  const int rb0 = blockIdx.x / S;
  const int ntiles = wg_tiles(rb0, rbstep, p.nrb);
  const int units = p.K >> 5;
  const int s_lo = slice * p.slice_units;
  const int s_hi = min(s_lo + p.slice_units, units);
  const int u_lo = s_lo + wave * p.ku;
  const int nu = __builtin_amdgcn_readfirstlane(max(0, min(u_lo + p.ku, s_hi) - u_lo));

  float* parts = lds;
  const int part_floats = nw * M * ROWS;
  void* stage = lds + 2 * part_floats;
  unsigned long long* lds_best = static_cast<unsigned long long*>(stage);
  if constexpr (BASE == EPI_ARGMAX) {
    if (tid < M) lds_best[tid] = 0ull;
  }

  // Column (element) of unit u for this lane; padding units repeat the wave's
  // last unit (always inside the matrix).
  int kcol[KU];
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int uu = min(max(u_lo + min(u, nu - 1), 0), units - 1);
    kcol[u] = uu * 32 + 8 * g4;
  }

  // Weight row base of tile rb (rows past N clamp to N-1: in bounds, unused).
  auto wrow = [&](int rb, int nt) -> const uint16_t* {
    if constexpr (GATEUP) {
      const int row = min(rb * 16 + r16, p.N - 1);
      return (nt == 0 ? p.W0 : p.W1) + (int64_t)row * p.ldw;
    } else {
      const int row = min(rb * ROWS + 16 * nt + r16, p.N - 1);
      return p.W0 + (int64_t)row * p.ldw;
    }
  };

  // First tile's weights, issued before the activations so both latencies overlap.
  u32x4 wf[NT][KU];
  if (ntiles > 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint16_t* wp = wrow(rb0, nt);
#pragma unroll
      for (int u = 0; u < KU; ++u) wf[nt][u] = ld16_stream(wp + kcol[u]);
    }
  }

  // Activation fragments: lane holds A[16*mt + r16][kcol[u] .. +8].  Rows
  // m >= M repeat row M-1: MFMA output column m depends only on activation
  // row m, and those columns are never read, so they need no zeroing (and the
  // loads need no wait before the weight stream).  Padding units (u >= nu,
  // wave-uniform) are zeroed, on the one path that has them.
  bf16x8 af[MT][KU];
  auto load_acts = [&](auto padded) {
    constexpr bool PAD = decltype(padded)::value;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint16_t* ap = p.A + (int64_t)min(16 * mt + r16, M - 1) * p.lda;
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        u32x4 v = ld16(ap + kcol[u]);
        if (PAD && u >= nu) v = u32x4{0u, 0u, 0u, 0u};
        af[mt][u] = __builtin_bit_cast(bf16x8, v);
      }
    }
  };
  if (nu == KU) load_acts(std::false_type{});
  else load_acts(std::true_type{});

  auto tile = [&](int j, auto prefetch) {
    constexpr bool PF = decltype(prefetch)::value;
    const int rb = rb0 + j * rbstep;
    const uint16_t* wpn[NT];
    if constexpr (PF) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wpn[nt] = wrow(rb + rbstep, nt);
    }
    f32x4 acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < KU; ++u) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const bf16x8 wv = __builtin_bit_cast(bf16x8, wf[nt][u]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, af[mt][u], acc[nt][mt], 0, 0, 0);
        if constexpr (PF) wf[nt][u] = ld16_stream(wpn[nt] + kcol[u]);
      }
    }
    // Lane holds tile rows 16*nt + 4*g4 + {0..3} for activation row 16*mt + r16.
    float* P = parts + (j & 1) * part_floats;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r16;
        if (m < M) *reinterpret_cast<f32x4*>(&P[(wave * M + m) * ROWS + 16 * nt + 4 * g4]) = acc[nt][mt];
      }
    lds_barrier();
    tile_reduce<ROWS, BASE>(p, P, nw, rb, j, stage, lds_best);
  };

  int j = 0;
  for (; j + 1 < ntiles; ++j) tile(j, std::integral_constant<bool, true>{});
  if (ntiles > 0) tile(j, std::integral_constant<bool, false>{});
  lds_barrier();
  if constexpr (BASE == EPI_ARGMAX) {
    argmax_fixup(p, lds_best, reinterpret_cast<int*>(lds_best + M));
  } else {
    flush_stage<OUT_ROWS, BASE>(p, stage, ntiles, rb0, slice);
    if constexpr (BASE == EPI_PART || BASE == EPI_PART_GU)
      splitk_fixup<OUT_ROWS, BASE>(p, ntiles, rb0, reinterpret_cast<int*>(parts));
  }
}

// Floats per (wave, row) of the LDS-fed MFMA path's partial tiles in LDS.  A wave
// stores its accumulators as f32x4 per lane, lane (r, g) at row r, column 4g:
// with a row stride of 16 or 32 floats (64 or 128 B) the 16 rows of one store
// fall on the same banks; 4 floats more shift each row by 4 banks (gate_up
// M = 8: 19.05 -> 18.18 us, M = 64: 30.2 -> 28.3 us; lm_head M = 64 -2%).
// Ring path (KW != 512) with one or two activation tiles only: the extra
// address arithmetic tipped a 48-row instance and the whole-tile body's
// two-row-tile instances over their register tiers, and three activation tiles
// or the whole-tile body (lm_head M = 32) gained nothing.
constexpr int lds_part_stride(int MT, int NT, int KW) { return MT <= 2 && KW != 512 ? 16 * NT + 4 : 16 * NT; }

// ---------------------------------------------------------------------------
// MFMA path with LDS-transposed weight rows ("rows through LDS").
//   MT : activation row tiles of 16 (M <= 16*MT)
//   NT : weight row tiles of 16 per workgroup tile (gate/up: 2 = gate + up)
//   KW : K columns per wave (512 or 256): one K chunk per wave per slice
// A wave streams its chunk of every tile row with the GEMV access pattern
// (one load instruction = 1 KiB contiguous of one row for KW = 512, or
// 512 B of each of two rows for KW = 256), writes the rows into a
// wave-private LDS region (row pitch 2*KW + 16 bytes: the 16 rows a
// fragment read touches fall on distinct banks), and reads them back as
// MFMA A fragments (lane: row l%16, 8 columns at 8*(l/16)).  The next tile's
// rows are loaded into registers while the current tile is multiplied.
// ---------------------------------------------------------------------------
template <int MT, int NT, int KW, int EPI>
__device__ __forceinline__ void mfmt_tile_body(Args p) {
  constexpr bool GATEUP = EpiTraits<EPI>::gateup;
  constexpr int BASE = EpiTraits<EPI>::base;   // epilogue without the norm prologue
  static_assert(!EpiTraits<EPI>::norm, "the LDS-fed MFMA path has no norm prologue");
  constexpr int ROWS = 16 * NT;                  // weight rows per tile
  constexpr int OUT_ROWS = GATEUP ? 16 : ROWS;   // output columns per tile
  constexpr int UNITS = KW / 32;                 // MFMA K steps per wave
  constexpr int LPR = KW / 8;                    // lanes per row in a load instruction
  constexpr int RPI = 64 / LPR;                  // rows per load instruction
  constexpr int NLD = ROWS / RPI;                // load instructions per tile (all NT row tiles)
  constexpr int PASSES = KW / 256;               // a 512-column chunk is staged in two halves
  constexpr int PITCH = 2 * 256 + kRowPad;       // LDS bytes per staged row (256 columns)
  static_assert(KW == 512 || KW == 256, "one or two rows per load instruction");
  static_assert(!GATEUP || NT == 2, "gate/up tiles pair 16 gate rows with 16 up rows");

  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = p.nw;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int M = p.M;

  const int S = p.S;
  const int slice = blockIdx.x % S;
  const int rbstep = p.rbstep;
  const int rb0 = blockIdx.x / S;
  const int ntiles = wg_tiles(rb0, rbstep, p.nrb);
  const int chunks = (p.K + KW - 1) / KW;
  const int c_lo = slice * p.slice_units;
  const int c_hi = min(c_lo + p.slice_units, chunks);
  const int chunk = c_lo + wave;                        // this wave's K chunk
  const bool has_chunk = chunk < c_hi;                  // wave-uniform
  const int k0 = min(chunk, chunks - 1) * KW;

  // LDS: [wave-private staging of 16 rows x 256 columns per wave: the NT row
  // tiles (and the two halves of a 512-column chunk) pass through it in
  // turn][partials][staged outputs].
  char* tr = reinterpret_cast<char*>(lds) + wave * (16 * PITCH);
  float* parts = reinterpret_cast<float*>(reinterpret_cast<char*>(lds) + nw * (16 * PITCH));
  constexpr int PST = lds_part_stride(MT, NT, KW);
  const int part_floats = nw * M * PST;
  void* stage = parts + 2 * part_floats;
  unsigned long long* lds_best = static_cast<unsigned long long*>(stage);
  if constexpr (BASE == EPI_ARGMAX) {
    if (tid < M) lds_best[tid] = 0ull;
  }

  // Load instruction i covers tile rows i*RPI + lane/LPR, columns k0 + 8*(lane%LPR).
  const int lrow = lane / LPR;
  const int lcol = min(k0 + 8 * (lane % LPR), p.K - 8);
  auto wsrc = [&](int rb, int i) -> const uint16_t* {
    const int t = i * RPI + lrow;             // row within the tile
    if constexpr (GATEUP) {
      const int row = min(rb * 16 + (t & 15), p.N - 1);
      return (t < 16 ? p.W0 : p.W1) + (int64_t)row * p.ldw + lcol;
    } else {
      const int row = min(rb * ROWS + t, p.N - 1);
      return p.W0 + (int64_t)row * p.ldw + lcol;
    }
  };
  // Staging address of this lane's 16 bytes.  Every staged register holds 256
  // columns of two rows (lanes 0-31: row 2j, lanes 32-63: row 2j+1): a
  // KW = 256 load already has that layout; for KW = 512 (one 512-column row
  // per load) v_permlane32_swap of rows 2j and 2j+1 produces it, one register
  // for columns 0-255 and one for 256-511, so every staging store is
  // unconditional.
  char* const wdst = tr + (lane >> 5) * PITCH + 16 * (lane & 31);
  constexpr int NLD16 = 16 / RPI;                 // load instructions per 16-row tile

  // First tile's weight rows, issued before the activations so that both
  // latencies overlap.
  u32x4 wf[NLD];
  if (ntiles > 0) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) wf[i] = ld16_stream(wsrc(rb0, i));
  }

  // Activation fragments of this chunk: lane holds A[16*mt + r16][k0 + 32u + 8*g4 .. +8].
  // Rows m >= M repeat row M-1 (they only feed MFMA output columns that are
  // never read, so they need no zeroing and no wait); columns >= K and waves
  // without a chunk are zeroed.  When the chunk lies inside K (wave-uniform)
  // the loads share one base address with immediate offsets and need no
  // masking; otherwise each column is clamped in bounds.
  const bool full_chunk = has_chunk && k0 + KW <= p.K;
  bf16x8 af[MT][UNITS];
  auto load_acts = [&](auto full) {
    constexpr bool FULL = decltype(full)::value;
    auto col = [&](int u) { return FULL ? k0 + 8 * g4 + 32 * u : min(k0 + 32 * u + 8 * g4, p.K - 8); };
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r16;
      const int64_t roff = (int64_t)min(m, M - 1) * p.lda;
#pragma unroll
      for (int u = 0; u < UNITS; ++u) {
        const int k = k0 + 32 * u + 8 * g4;
        const bool ok = FULL || (k < p.K && has_chunk);
        u32x4 v = ld16(p.A + roff + col(u));
        if (!ok) v = u32x4{0u, 0u, 0u, 0u};
        af[mt][u] = __builtin_bit_cast(bf16x8, v);
      }
    }
  };
  if (full_chunk) load_acts(std::true_type{});
  else load_acts(std::false_type{});


  auto tile = [&](int j, auto prefetch) {
    constexpr bool PF = decltype(prefetch)::value;
    const int rb = rb0 + j * rbstep;
    f32x4 acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      // Stage this 16-row tile (256 columns per pass) in LDS and read it back
      // as MFMA fragments.  The region is private to the wave and the LDS
      // accesses of one wave execute in order, so no barrier is needed.
      u32x4 half[PASSES][8];   // [pass][row pair]: 256 columns of rows 2j, 2j+1
#pragma unroll
      for (int jp = 0; jp < 8; ++jp) {
        if constexpr (KW == 256) {
          half[0][jp] = wf[nt * NLD16 + jp];
        } else {
          const u32x4 x = wf[nt * NLD16 + 2 * jp], y = wf[nt * NLD16 + 2 * jp + 1];
          u32x4 lo, hi;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const auto r = __builtin_amdgcn_permlane32_swap(x[c], y[c], false, false);
            lo[c] = r[0];
            hi[c] = r[1];
          }
          half[0][jp] = lo;
          half[PASSES - 1][jp] = hi;
        }
      }
      if constexpr (PF) {   // the row registers are free: load the next tile's rows
#pragma unroll
        for (int i = 0; i < NLD16; ++i) wf[nt * NLD16 + i] = ld16_stream(wsrc(rb + rbstep, nt * NLD16 + i));
      }
#pragma unroll
      for (int h = 0; h < PASSES; ++h) {
#pragma unroll
        for (int jp = 0; jp < 8; ++jp) *reinterpret_cast<u32x4*>(wdst + 2 * jp * PITCH) = half[h][jp];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bf16x8 wv = *reinterpret_cast<const bf16x8*>(tr + r16 * PITCH + 64 * u + 16 * g4);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, af[mt][8 * h + u], acc[nt][mt], 0, 0, 0);
        }
      }
    }
    float* P = parts + (j & 1) * part_floats;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r16;
        if (m < M) *reinterpret_cast<f32x4*>(&P[(wave * M + m) * PST + 16 * nt + 4 * g4]) = acc[nt][mt];
      }
    lds_barrier();
    tile_reduce<ROWS, BASE, PST>(p, P, nw, rb, j, stage, lds_best);
  };

  int j = 0;
  for (; j + 1 < ntiles; ++j) tile(j, std::integral_constant<bool, true>{});
  if (ntiles > 0) tile(j, std::integral_constant<bool, false>{});
  lds_barrier();
  if constexpr (BASE == EPI_ARGMAX) {
    argmax_fixup(p, lds_best, reinterpret_cast<int*>(lds_best + M));
  } else {
    flush_stage<OUT_ROWS, BASE>(p, stage, ntiles, rb0, slice);
    if constexpr (BASE == EPI_PART || BASE == EPI_PART_GU)
      splitk_fixup<OUT_ROWS, BASE>(p, ntiles, rb0, reinterpret_cast<int*>(parts));
  }
}

// ---------------------------------------------------------------------------
// Ring-streamed variant of the path above for 256-column slabs.  A wave owns
// KW = 256*CPW columns of the K slice (CPW consecutive 256-column chunks).
// A load instruction reads 512 B of each of two rows (lanes 0-31: row 2q,
// lanes 32-63: row 2q+1), so one 16-row slab of one chunk is 8 instructions.
// The wave keeps exactly one slab of loads in flight in an 8-register ring
// and refills each register as soon as it has been written to the staging
// region, so new loads are issued one at a time while the previous slab is
// multiplied, across chunk, slab and tile boundaries alike; only the last
// slab of the last tile issues nothing.  Slab order within a tile: chunk-
// major, then the NT 16-row groups, so a chunk's activation fragments serve
// NT slabs.  With one chunk per wave the activations are loaded once, before
// the first slab; with several, each chunk's are loaded one chunk ahead into
// registers and turned into fragments when the chunk starts, so waiting for
// them never drains the ring.
// ---------------------------------------------------------------------------
// Weight loads a ring wave keeps in flight (each one 16 bytes per lane, two
// rows of a 16-row slab): a whole slab, except with three 16-row activation
// tiles and one chunk per wave, where half a slab keeps the registers within
// the 12-wave tier (168 per lane): ten waves of 48 rows then cover K = 2560
// without a K split (qkv M = 40: 16.1 -> 11.3 us, gate_up 34.4 -> 24.8 us,
// lm_head 157 -> 129 us).
constexpr int ring_slots(int MT, int CPW) { return MT == 3 && CPW == 1 ? 4 : 8; }


template <int MT, int NT, int CPW, int EPI>
__device__ __forceinline__ void mfmt_ring_body(Args p, unsigned bid) {
  constexpr bool GATEUP = EpiTraits<EPI>::gateup;
  constexpr int BASE = EpiTraits<EPI>::base;
  static_assert(!EpiTraits<EPI>::norm, "the LDS-fed MFMA path has no norm prologue");
  static_assert(!GATEUP || NT % 2 == 0, "gate/up tiles pair NT/2 slabs of gate rows with NT/2 of up rows");
  static_assert(CPW >= 1, "chunks per wave");
  constexpr bool PRE = EpiTraits<EPI>::pre;       // finish the RMSNorm from the producer's partials
  constexpr bool RESID = EpiTraits<EPI>::resid;   // hand the residual and its partials on
  static_assert(!PRE || CPW == 1, "pre-normalised activations are loaded once (one chunk per wave)");
  constexpr int CW = 256;                        // columns per chunk (slab width)
  constexpr int KW = CW * CPW;                   // columns per wave
  constexpr int ROWS = 16 * NT;                  // weight rows per tile
  constexpr int OUT_ROWS = GATEUP ? ROWS / 2 : ROWS;   // staged output columns per tile
  constexpr int UNITS = CW / 32;                 // MFMA K steps per slab
  constexpr int RING = 8;                        // load instructions per 16-row slab
  constexpr int RSLOTS = ring_slots(MT, CPW);    // of which in flight (ring registers)
  constexpr int PITCH = 2 * CW + kRowPad;        // LDS bytes per staged row

  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = p.nw;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int M = p.M;

  const int S = p.S;
  const int slice = bid % (unsigned)S;
  const int rbstep = p.rbstep;
  const int rb0 = bid / (unsigned)S;
  const int ntiles = wg_tiles(rb0, rbstep, p.nrb);
  const int units = (p.K + KW - 1) / KW;
  const int c_lo = slice * p.slice_units;
  const int c_hi = min(c_lo + p.slice_units, units);
  const int unit = c_lo + wave;
  const bool has_unit = unit < c_hi;   // wave-uniform
  const int kw0 = min(unit, units - 1) * KW;

  char* tr = reinterpret_cast<char*>(lds) + wave * (16 * PITCH);
  float* parts = reinterpret_cast<float*>(reinterpret_cast<char*>(lds) + nw * (16 * PITCH));
  constexpr int PST = lds_part_stride(MT, NT, 256 * CPW);
  const int part_floats = nw * M * PST;
  void* stage = parts + p.pbuf * part_floats;
  unsigned long long* lds_best = static_cast<unsigned long long*>(stage);
  if constexpr (BASE == EPI_ARGMAX) {
    if (tid < M) lds_best[tid] = 0ull;
  }

  // Loads are never masked or branched around: a column group past K (or any
  // column of a wave without a K unit) loads 16 zero bytes from kZeroLine
  // instead, for weights and activations alike, so every load is issued
  // unconditionally and nothing forces an early wait.
  const uint16_t* const zero16 = reinterpret_cast<const uint16_t*>(kZeroLine);

  // Activations of chunk c are loaded row-contiguous, like the weights (load
  // q: rows 2q + lane/32 of the 16-row group q/8, 512 B each), staged through
  // this wave's LDS region and read back as MFMA fragments (lane holds
  // A[16*mt + r16][k0 + 32u + 8*g4 .. +8]).  Fragment-order global loads would
  // touch 16 half-used cache lines per instruction; these touch 8 whole ones,
  // which measured 0.5-1.5 us faster per kernel.  Rows m >= M read zeros and
  // only feed MFMA columns that are never read.
  bf16x8 af[MT][UNITS];
  u32x4 araw[8 * MT];
  auto issue_acts = [&](int c) {
    // The chunk's first column is laundered so that later chunks' addresses
    // are computed here, not hoisted out of the tile loop.
    int kc = kw0 + CW * c;
    if constexpr (CPW > 1) asm volatile("" : "+v"(kc));
    const int k = kc + 8 * (lane & 31);
#pragma unroll
    for (int q = 0; q < 8 * MT; ++q) {
      const int row = 2 * q + (lane >> 5);
      araw[q] = ld16((has_unit && k < p.K && row < M) ? p.A + (int64_t)row * p.lda + k : zero16);
    }
  };
  // One wave's LDS accesses execute in order, so the staging region is free
  // here (the previous slab's fragment reads are done) and the next slab's
  // staging stores come after these reads.
  auto stage_acts = [&]() {
    char* const adst = tr + (lane >> 5) * PITCH + 16 * (lane & 31);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int q = 0; q < 8; ++q) *reinterpret_cast<u32x4*>(adst + 2 * q * PITCH) = araw[8 * mt + q];
#pragma unroll
      for (int u = 0; u < UNITS; ++u) af[mt][u] = *reinterpret_cast<const bf16x8*>(tr + r16 * PITCH + 64 * u + 16 * g4);
    }
  };
  // PRE: the producer's partial sums of squares are loaded first (rows
  // wave + nw*i, groups lane + 64*j; the host guarantees M <= 4*nw and
  // K <= 4096), so the row-norm reduction below waits for nothing else.
  constexpr int SQR = PRE ? 4 : 1, SQG = PRE ? 4 : 1;
  float sqv[SQR][SQG];
  if constexpr (PRE) {
    const int ngrp = p.K >> 4;
#pragma unroll
    for (int i = 0; i < SQR; ++i) {
      const float* row = p.SQ + (int64_t)min(wave + nw * i, M - 1) * p.sq_ld;
#pragma unroll
      for (int g = 0; g < SQG; ++g) sqv[i][g] = row[min(lane + 64 * g, ngrp - 1)];
    }
  }
  issue_acts(0);
  // PRE: the norm weights of this lane's 8 columns (the same for every row
  // in the row-contiguous layout), as (w, 0) and (0, w) bf16 pairs.
  u32x4 wlo, whi;
  if constexpr (PRE) {
    const int k = kw0 + 8 * (lane & 31);
    const u32x4 w = ld16((has_unit && k < p.K) ? p.NW + k : zero16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wlo[q] = w[q] & 0xFFFFu;
      whi[q] = w[q] & 0xFFFF0000u;
    }
  }

  // Instruction q of slab (rb, c, nt): rows 2q + lane/32 of the 16-row group nt,
  // 8 columns at kw0 + 256c + 8*(lane%32) (rows clamped in bounds).  Tile rb
  // holds weight rows rb*tr .. rb*tr + tr - 1 (gate/up: that many gate rows in
  // slabs 0..NT/2-1 and up rows in the rest); slab rows past tr load the zero
  // line (one broadcast line, no HBM traffic), so tr need not be a multiple
  // of 16 and the host can give every CU the same number of rows.
  const int lrow = lane >> 5;
  auto col_of = [&](int c) { return kw0 + CW * c + 8 * (lane & 31); };
  auto wsrc_col = [&](int rb, int col, int nt, int q) -> const uint16_t* {
    const int t = 2 * q + lrow;
    if (!(has_unit && col < p.K)) return zero16;
    if constexpr (GATEUP) {
      constexpr int H = NT / 2;
      const int lr = 16 * (nt % H) + t;
      if (lr >= p.tr) return zero16;
      const int row = min(rb * p.tr + lr, p.N - 1);
      return (nt < H ? p.W0 : p.W1) + (int64_t)row * p.ldw + col;
    } else {
      const int lr = 16 * nt + t;
      if (lr >= p.tr) return zero16;
      const int row = min(rb * p.tr + lr, p.N - 1);
      return p.W0 + (int64_t)row * p.ldw + col;
    }
  };
  char* const wdst = tr + lrow * PITCH + 16 * (lane & 31);

  // Issued even by a workgroup without tiles (rows are clamped, so the loads
  // stay in bounds): with a branch here the compiler could no longer count
  // the ring loads behind the activation loads and would wait for all of
  // them before staging the activations.
  u32x4 ring[RSLOTS];
#pragma unroll
  for (int q = 0; q < RSLOTS; ++q) ring[q] = ld16_stream(wsrc_col(rb0, col_of(0), 0, q));
  // PRE: the row norms (the partial sums were the first loads issued), then
  // the first chunk's activations normalised in the row-contiguous layout,
  // A = bf16(w * bf16(x * rstd)) (the cast placement of
  // engine/kernels/gemm.py:28-56), while the first slab is still in flight.
  // rstd of a row: its partial sums lane-strided, then a wave butterfly (a
  // fixed order).
  if constexpr (PRE) {
    __shared__ float s_rstd[64];
    const int ngrp = p.K >> 4;
#pragma unroll
    for (int i = 0; i < SQR; ++i) {
      float t = 0.f;
#pragma unroll
      for (int g = 0; g < SQG; ++g) t += lane + 64 * g < ngrp ? sqv[i][g] : 0.f;
      t = wave_sum(t);
      const int m = wave + nw * i;
      if (lane == 0 && m < M) s_rstd[m] = rms_rstd(t, p.K, p.eps);
    }
    lds_barrier();
    // All row norms are read before any is used (one LDS wait, not one per
    // row pair); row pairs past M hold zeros and are skipped, and when every
    // pair holds a real row the loop carries no per-pair branch.
    float rsv[8 * MT];
#pragma unroll
    for (int q = 0; q < 8 * MT; ++q) rsv[q] = s_rstd[min(2 * q + (lane >> 5), M - 1)];
    if (M > 2 * (8 * MT - 1)) {   // uniform
#pragma unroll
      for (int q = 0; q < 8 * MT; ++q) araw[q] = norm_line_bf16x8(araw[q], wlo, whi, rsv[q]);
    } else {
#pragma unroll
      for (int q = 0; q < 8 * MT; ++q)
        if (2 * q < M) araw[q] = norm_line_bf16x8(araw[q], wlo, whi, rsv[q]);   // uniform
    }
  }
  // The first chunk's activations into fragments (their loads were issued
  // before the ring, so this waits for them alone); with several chunks per
  // wave, the next chunk's loads go out at once and are staged when that
  // chunk starts, one chunk later.
  stage_acts();
  if constexpr (CPW > 1) issue_acts(1);

  auto tile = [&](int j, auto last) {
    constexpr bool LAST = decltype(last)::value;
    const int rb = rb0 + j * rbstep;
    f32x4 acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      if constexpr (CPW > 1) {
        if (c > 0 || j > 0) {
          stage_acts();
          if (!(LAST && c + 1 == CPW)) issue_acts(c + 1 < CPW ? c + 1 : 0);
        }
        __builtin_amdgcn_sched_barrier(0);   // chunks are scheduled one after another
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const bool last_slab = (c + 1 == CPW) && (nt + 1 == NT);
        const int rbn = last_slab ? rb + rbstep : rb;
        const int cn = nt + 1 < NT ? c : (c + 1 < CPW ? c + 1 : 0);
        const int ntn = nt + 1 < NT ? nt + 1 : 0;
        // The refill column is recomputed here (an empty asm hides it from
        // loop-invariant hoisting, which would keep every chunk's addresses
        // live across the tile loop).
        int coln = col_of(cn);
        if constexpr (CPW > 1) asm volatile("" : "+v"(coln));
        // Stage the slab (wave-private region; one wave's LDS accesses execute
        // in order, so the previous slab's fragment reads are done) and refill.
#pragma unroll
        for (int q = 0; q < RING; ++q) {
          // slot q % RSLOTS refills with the load RSLOTS ahead: later in this
          // slab, or in the next one
          const int slot = q % RSLOTS;
          *reinterpret_cast<u32x4*>(wdst + 2 * q * PITCH) = ring[slot];
          if (q + RSLOTS < RING) ring[slot] = ld16_stream(wsrc_col(rb, col_of(c), nt, q + RSLOTS));
          else if (!(LAST && last_slab)) ring[slot] = ld16_stream(wsrc_col(rbn, coln, ntn, q + RSLOTS - RING));
          __builtin_amdgcn_sched_barrier(0);   // keep each refill next to its staging store
        }
#pragma unroll
        for (int u = 0; u < UNITS; ++u) {
          const bf16x8 wv = *reinterpret_cast<const bf16x8*>(tr + r16 * PITCH + 64 * u + 16 * g4);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, af[mt][u], acc[nt][mt], 0, 0, 0);
        }
      }
    }
    float* P = parts + (p.pbuf == 2 ? (j & 1) : 0) * part_floats;
    if (p.pbuf == 1 && j > 0) lds_barrier();   // one buffer: the previous tile's reduction has read it
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r16;
        if (m < M) *reinterpret_cast<f32x4*>(&P[(wave * M + m) * PST + 16 * nt + 4 * g4]) = acc[nt][mt];
      }
    // The barrier keeps the waves of a workgroup on the same tile rows
    // (measured faster than deferring every reduction to the end).
    lds_barrier();
    tile_reduce<ROWS, BASE, PST>(p, P, nw, rb, j, stage, lds_best);
  };

  int j = 0;
  for (; j + 1 < ntiles; ++j) tile(j, std::false_type{});
  if (ntiles > 0) tile(j, std::true_type{});
  lds_barrier();
  if constexpr (BASE == EPI_ARGMAX) {
    argmax_fixup(p, lds_best, reinterpret_cast<int*>(lds_best + M));
  } else if constexpr (BASE == EPI_PART || BASE == EPI_PART_GU) {
    flush_stage<OUT_ROWS, BASE>(p, stage, ntiles, rb0, slice);
    splitk_fixup<OUT_ROWS, BASE, RESID>(p, ntiles, rb0, reinterpret_cast<int*>(parts));
  } else {
    flush_stage<OUT_ROWS, BASE, RESID>(p, stage, ntiles, rb0, slice);
  }
}

template <int MT, int NT, int KW, int EPI>
__device__ __forceinline__ void mfmt_body(Args p) {
  if constexpr (KW == 512) mfmt_tile_body<MT, NT, KW, EPI>(p);
  else mfmt_ring_body<MT, NT, KW / 256, EPI>(p, blockIdx.x);
}

// The ring path with row groups (Args::groups > 1).  A separate entry point,
// so the plain launches carry none of the group arithmetic.
template <int MT, int NT, int KW, int EPI>
__device__ __forceinline__ void mfmt_grouped_body(Args p) {
  static_assert(KW != 512, "row groups run on the ring path");
  const unsigned bid = enter_row_group<EPI>(p);
  mfmt_ring_body<MT, NT, KW / 256, EPI>(p, bid);
}

// ---------------------------------------------------------------------------
// GEMV path (VALU).
//   MR : compile-time bound on activation rows (M <= MR)
//   R  : weight rows per tile (gate/up: R gate rows + R up rows)
//   KU : compile-time bound on K units (512 columns) per wave
// Same loop structure as the MFMA path: branch-free loads, peeled last tile,
// outputs staged in LDS.  Columns past the K slice read a clamped in-bounds
// chunk and meet zero activations.
// ---------------------------------------------------------------------------
template <int MR, int R, int KU, int EPI>
__device__ __forceinline__ void gemv_body(Args p) {
  constexpr bool GATEUP = EpiTraits<EPI>::gateup;
  constexpr int BASE = EpiTraits<EPI>::base;   // epilogue without the norm prologue
  constexpr bool NORM = EpiTraits<EPI>::norm;
  constexpr int RR = GATEUP ? 2 * R : R;   // partial rows per tile
  constexpr int OUT_ROWS = R;

  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = p.nw;
  const int M = p.M;

  const int S = p.S;
  const int slice = blockIdx.x % S;
  const int rbstep = p.rbstep;
  const int rb0 = blockIdx.x / S;
  const int ntiles = wg_tiles(rb0, rbstep, p.nrb);
  const int units = (p.K + 511) >> 9;
  const int s_lo = slice * p.slice_units;
  const int s_hi = min(s_lo + p.slice_units, units);
  const int u_lo = s_lo + wave * p.ku;
  const int nu = __builtin_amdgcn_readfirstlane(max(0, min(u_lo + p.ku, s_hi) - u_lo));
  const int kend = min(s_hi * 512, p.K);

  float* parts = lds;
  const int part_floats = nw * M * RR;
  void* stage = lds + 2 * part_floats;
  unsigned long long* lds_best = static_cast<unsigned long long*>(stage);
  if constexpr (BASE == EPI_ARGMAX) {
    if (tid < M) lds_best[tid] = 0ull;
  }

  // Lane's column of unit u (clamped in bounds) and whether it is real data.
  int kcol[KU];
  bool kok[KU];
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int k = (u_lo + u) * 512 + 8 * lane;
    kok[u] = (u < nu) && (k < kend);
    kcol[u] = min(max(k, 0), p.K - 8);
  }

  auto wrow = [&](int rb, int rr) -> const uint16_t* {
    if constexpr (GATEUP) {
      const int row = min(rb * R + (rr % R), p.N - 1);
      return (rr < R ? p.W0 : p.W1) + (int64_t)row * p.ldw;
    } else {
      const int row = min(rb * R + rr, p.N - 1);
      return p.W0 + (int64_t)row * p.ldw;
    }
  };

  // First tile's weight rows, issued before the activations so both
  // latencies overlap (norm instances: after the prologue, see below).
  u32x4 wf[RR][KU];
  auto load_first_tile = [&]() {
    if (ntiles > 0) {
#pragma unroll
      for (int rr = 0; rr < RR; ++rr) {
        const uint16_t* wp = wrow(rb0, rr);
#pragma unroll
        for (int u = 0; u < KU; ++u) wf[rr][u] = ld16_stream(wp + kcol[u]);
      }
    }
  };
  if constexpr (!NORM) load_first_tile();

  // Activations (and, for norm instances, the residual rows and the norm
  // weights).  Rows m >= M repeat row M-1: their dot products go to partial
  // slots that are never stored.  Padding columns (kok false) are zeroed on
  // the one path that has them (wave-uniform: all of the wave's units real).
  const bool full = (nu == KU) && ((u_lo + KU) * 512 <= kend);
  u32x4 af[MR][KU];
  u32x4 yf[NORM ? MR : 1][NORM ? KU : 1];
  u32x4 nf[NORM ? KU : 1];
  auto load_acts = [&](auto fullc) {
    constexpr bool FULL = decltype(fullc)::value;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const int64_t roff = (int64_t)min(m, M - 1) * p.lda;
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        u32x4 v = ld16(p.A + roff + kcol[u]);
        if (!FULL && !kok[u]) v = u32x4{0u, 0u, 0u, 0u};
        af[m][u] = v;
        if constexpr (NORM) {
          u32x4 yv = ld16(p.Y + roff + kcol[u]);
          if (!FULL && !kok[u]) yv = u32x4{0u, 0u, 0u, 0u};
          yf[m][u] = yv;
        }
      }
    }
    if constexpr (NORM) {
#pragma unroll
      for (int u = 0; u < KU; ++u) nf[u] = ld16(p.NW + kcol[u]);
    }
  };
  if (full) load_acts(std::true_type{});
  else load_acts(std::false_type{});

  if constexpr (NORM) {
    // s = bf16(x + y) replaces x; row sums of squares over the wave (DPP),
    // then over the waves in LDS in wave order (the workgroup covers all of K).
    float sq[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      sq[m] = 0.f;
#pragma unroll
      for (int u = 0; u < KU; ++u) af[m][u] = add_bf16x8(af[m][u], yf[m][u], sq[m]);
      sq[m] = wave_sum(sq[m]);
    }
    float* red = parts + part_floats;   // first written by tile 1, after tile 0's barrier
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) red[wave * M + m] = sq[m];
    }
    lds_barrier();
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float t = 0.f;
      for (int w = 0; w < nw; ++w) t += red[w * M + min(m, M - 1)];
      const float rstd = rms_rstd(t, p.K, p.eps);
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const bool ok = m < M && kok[u];
        if (blockIdx.x == 0 && ok) *reinterpret_cast<u32x4*>(p.XO + (int64_t)m * p.lda + kcol[u]) = af[m][u];
        u32x4 a = norm_bf16x8(af[m][u], nf[u], rstd);
        if (!ok) a = u32x4{0u, 0u, 0u, 0u};
        af[m][u] = a;
      }
    }
  }

  if constexpr (NORM) {
    // Norm instances: the first tile's weight rows after the prologue (not
    // hoisted above it, where they would sit next to its registers).
    __builtin_amdgcn_sched_barrier(0);
    load_first_tile();
  }

  auto tile = [&](int j, auto prefetch) {
    constexpr bool PF = decltype(prefetch)::value;
    const int rb = rb0 + j * rbstep;
    float acc[RR][MR];
#pragma unroll
    for (int rr = 0; rr < RR; ++rr)
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[rr][m] = 0.f;
#pragma unroll
    for (int u = 0; u < KU; ++u) {
#pragma unroll
      for (int rr = 0; rr < RR; ++rr) {
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[rr][m] = dot8(wf[rr][u], af[m][u], acc[rr][m]);
        if constexpr (PF) wf[rr][u] = ld16_stream(wrow(rb + rbstep, rr) + kcol[u]);
      }
    }
    float* P = parts + (j & 1) * part_floats;
#pragma unroll
    for (int rr = 0; rr < RR; ++rr)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float s = wave_sum(acc[rr][m]);
        if (m < M && lane == 0) P[(wave * M + m) * RR + rr] = s;
      }
    lds_barrier();
    tile_reduce<RR, BASE>(p, P, nw, rb, j, stage, lds_best);
  };

  int j = 0;
  for (; j + 1 < ntiles; ++j) tile(j, std::integral_constant<bool, true>{});
  if (ntiles > 0) tile(j, std::integral_constant<bool, false>{});
  lds_barrier();
  if constexpr (BASE == EPI_ARGMAX) {
    argmax_fixup(p, lds_best, reinterpret_cast<int*>(lds_best + M));
  } else {
    flush_stage<OUT_ROWS, BASE>(p, stage, ntiles, rb0, slice);
    if constexpr (BASE == EPI_PART || BASE == EPI_PART_GU)
      splitk_fixup<OUT_ROWS, BASE>(p, ntiles, rb0, reinterpret_cast<int*>(parts));
  }
}

#ifdef SK_AUX_KERNELS
// Non-template kernels: defined only in the translation unit that launches
// them (sk_abi.hip), so every other unit can include this header.
// Argmax over materialised bf16 logits: workgroup (c, m) scans chunk c of row
// m; the last workgroup to arrive reduces every chunk's candidate.  Rows that
// are 16-byte aligned (vec) are read with 8-column vector loads.
constexpr int ARGMAX_THREADS = 256;

__global__ void __launch_bounds__(ARGMAX_THREADS) argmax_kernel(const uint16_t* __restrict__ L, int64_t ld, int M,
                                                                int V, int chunk, int vec,
                                                                unsigned long long* __restrict__ best,
                                                                unsigned* __restrict__ ticket, int64_t* __restrict__ ids,
                                                                float* __restrict__ maxv) {
  __shared__ unsigned long long red[ARGMAX_THREADS];
  __shared__ int flag;
  const int m = blockIdx.y, c = blockIdx.x, tid = threadIdx.x;
  const int chunks = gridDim.x;
  const uint16_t* row = L + (int64_t)m * ld;
  const int lo = c * chunk, hi = min(lo + chunk, V);
  unsigned long long b = 0ull;
  const int vhi = vec ? lo + ((hi - lo) & ~7) : lo;
  for (int k = lo + 8 * tid; k < vhi; k += 8 * ARGMAX_THREADS) {
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
  for (int k = vhi + tid; k < hi; k += ARGMAX_THREADS) {
    const unsigned long long kk = argmax_key(row[k], k);
    b = kk > b ? kk : b;
  }
  red[tid] = b;
  __syncthreads();
  for (int sft = ARGMAX_THREADS / 2; sft > 0; sft >>= 1) {
    if (tid < sft && red[tid + sft] > red[tid]) red[tid] = red[tid + sft];
    __syncthreads();
  }
  if (tid == 0) {
    __hip_atomic_fetch_max(&best[m], red[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    flag = take_ticket(ticket, (unsigned)(chunks * M)) ? 1 : 0;
  }
  __syncthreads();
  if (!flag) return;
  // Last workgroup of the grid: decode every row and clear best[] for the next call.
  for (int mm = tid; mm < M; mm += ARGMAX_THREADS) {
    const unsigned long long bb = __hip_atomic_exchange(&best[mm], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ids[mm] = argmax_key_index(bb);
    maxv[mm] = argmax_key_value(bb);
  }
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
                                                                  uint16_t* __restrict__ out, int K, int64_t ld,
                                                                  int64_t ld_out) {
  __shared__ float wsum[RMS_THREADS / 64];
  const int m = blockIdx.x;
  const uint16_t* xr = x + (int64_t)m * ld;
  const uint16_t* yr = y + (int64_t)m * ld;
  uint16_t* xo = xout + (int64_t)m * ld;
  uint16_t* orow = out + (int64_t)m * ld_out;
  const int nchunk = K >> 3;
  // Every load of the row (x, y and the norm weights) is requested before
  // the first is used: the weights are not left for after the reduction,
  // where they would add a memory round trip to the launch.
  u32x4 sv[RMS_MAX_CHUNKS], xv[RMS_MAX_CHUNKS], yv[RMS_MAX_CHUNKS], wv[RMS_MAX_CHUNKS];
#pragma unroll
  for (int j = 0; j < RMS_MAX_CHUNKS; ++j) {
    const int c = threadIdx.x + j * RMS_THREADS;
    xv[j] = yv[j] = wv[j] = u32x4{0u, 0u, 0u, 0u};
    if (c < nchunk) {
      xv[j] = ld16(xr + 8 * c);
      yv[j] = ld16(yr + 8 * c);
      wv[j] = ld16(w + 8 * c);
    }
  }
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < RMS_MAX_CHUNKS; ++j) {
    const int c = threadIdx.x + j * RMS_THREADS;
    sv[j] = u32x4{0u, 0u, 0u, 0u};
    if (c < nchunk) {
      sv[j] = add_bf16x8(xv[j], yv[j], sq);
      *reinterpret_cast<u32x4*>(xo + 8 * c) = sv[j];
    }
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = sq;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < RMS_THREADS / 64; ++i) tot += wsum[i];
  const float rstd = rms_rstd(tot, K, eps);
#pragma unroll
  for (int j = 0; j < RMS_MAX_CHUNKS; ++j) {
    const int c = threadIdx.x + j * RMS_THREADS;
    if (c < nchunk) *reinterpret_cast<u32x4*>(orow + 8 * c) = norm_bf16x8(sv[j], wv[j], rstd);
  }
}

// Zero n 32-bit words with plain vector stores (clears arrival counters; a
// kernel rather than a memset node, so it also replays from a captured graph).
__global__ void __launch_bounds__(256) clear_words_kernel(unsigned* __restrict__ p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
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
