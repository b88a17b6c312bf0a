// sk_registry.hpp - lookup of the compiled kernel instances.
//
// The kernel templates are instantiated for a fixed set of (row tiles, K-unit
// bound) pairs per epilogue, one translation unit per epilogue
// (sk_inst_mfma.hip / sk_inst_mfmt.hip / sk_inst_gemv.hip built with
// -DSK_EPI=<n>; the norm-prologue epilogues 5..7 exist for the GEMV path only).
// The host planner asks for the smallest instantiated K-unit bound that covers
// a wave's K range; a nullptr answer means "no such instance" and the config
// is rejected with SK_ERR_CONFIG.
#pragma once

#include "sk_kernels.hpp"
#include "sk_wide.hpp"
#include "sk_wide2.hpp"

namespace sk {

typedef void (*KernelFn)(Args);

// K-unit bounds compiled for each path (ascending).
constexpr int kMfmaKU[] = {5, 8, 10, 16, 20};
constexpr int kGemvKU[] = {2, 5, 8, 10};

// Register estimate (VGPR + AGPR per lane) of an instance; decides the
// largest workgroup the instance is compiled for (__launch_bounds__).
// With the norm prologue the residual and norm-weight fragments are live next
// to the activations before the first tile's weights are loaded.
constexpr int mfma_regs(int MT, int NT, int KU) { return 4 * KU * (MT + NT) + 4 * NT * MT + 24; }
constexpr int norm_extra(int act_regs, int weight_regs, int unit_regs) {
  return act_regs + unit_regs > weight_regs ? act_regs + unit_regs - weight_regs : 0;
}
constexpr int gemv_regs(int MR, int RR, int KU, bool norm = false) {
  return 4 * KU * (MR + RR) + RR * MR + 24 + (norm ? norm_extra(4 * KU * MR, 4 * KU * RR, 4 * KU) : 0);
}
// LDS-transposed MFMA.  KW = 512: one chunk's activation units plus a whole
// tile of weight rows in flight (16*NT rows, one row per load instruction).
// Otherwise (ring, KW = 256 * chunks per wave): one 256-column chunk's
// activation units plus the ring (ring_slots loads).
constexpr int mfmt_regs(int MT, int NT, int KW) {
  // tile body: weight tile + fragments + accumulators; ring body: fragments +
  // ring + accumulators, plus, with several chunks, the next chunk's
  // activations and their addresses (measured: about twice the data alone)
  return KW == 512 ? 4 * 16 * MT + 4 * 16 * NT + 4 * NT * MT + 32
                   : 4 * 8 * MT + 4 * ring_slots(MT, KW / 256) + 4 * NT * MT + 32 + (KW > 256 ? 8 * 8 * MT : 0);
}

// Waves per workgroup an instance is compiled for (its __launch_bounds__):
// 16 waves leave 128 VGPRs per lane, 12 waves 168, 8 waves 256, 4 waves 512.
constexpr int max_waves_for_regs(int regs) {
  return regs <= 128 ? 16 : (regs <= 168 ? 12 : (regs <= 256 ? 8 : 4));
}
// Waves per workgroup an LDS-fed MFMA instance is compiled for.  The residual
// hand-off consumers (pre) also hold the norm weights of their chunk and the
// producer's partial sums (48 more registers).
constexpr int mfmt_max_waves(int MT, int NT, int KW, bool pre = false) {
  return max_waves_for_regs(mfmt_regs(MT, NT, KW) + (pre ? 48 : 0));
}

// Waves per workgroup each instance is compiled for.  The estimates above
// decide it, except for the instances listed in sk_tiers.inc: those spilled
// VGPRs at their estimate's tier and are compiled for the largest tier at
// which the compiler reported no spill (waves 0: they spill even with 512
// registers per lane and are not compiled at all).  The list is measured by
// `python -m starter_amd.build --retier`; the regular build fails if any
// instance spills, so a stale list cannot go unnoticed.
enum InstKind { KIND_GEMV = 0, KIND_MFMA = 1, KIND_MFMT = 2 };
struct TierOverride {
  int kind, a, b, c, epi, waves;   // (a, b, c) = the instance's template arguments before EPI
};
#include "sk_tiers.inc"   // constexpr TierOverride kTierOverrides[] = {..., {-1, ...}}

constexpr int estimate_waves(int kind, int a, int b, int c, int epi) {
  return kind == KIND_GEMV
             ? max_waves_for_regs(gemv_regs(a, epi_gateup(epi) ? 2 * b : b, c, epi_norm(epi)))
         : kind == KIND_MFMA ? max_waves_for_regs(mfma_regs(a, b, c))
                             : mfmt_max_waves(a, b, c, epi_pre(epi));
}
constexpr int instance_waves(int kind, int a, int b, int c, int epi) {
  for (const TierOverride& t : kTierOverrides)
    if (t.kind == kind && t.a == a && t.b == b && t.c == c && t.epi == epi) return t.waves;
  return estimate_waves(kind, a, b, c, epi);
}

KernelFn mfma_for_epi0(int MT, int NT, int KU);
KernelFn mfma_for_epi1(int MT, int NT, int KU);
KernelFn mfma_for_epi2(int MT, int NT, int KU);
KernelFn mfma_for_epi3(int MT, int NT, int KU);
KernelFn mfma_for_epi4(int MT, int NT, int KU);
KernelFn mfmt_for_epi0(int MT, int NT, int KW);
KernelFn mfmt_for_epi1(int MT, int NT, int KW);
KernelFn mfmt_for_epi2(int MT, int NT, int KW);
KernelFn mfmt_for_epi3(int MT, int NT, int KW);
KernelFn mfmt_for_epi4(int MT, int NT, int KW);
KernelFn mfmt_for_epi8(int MT, int NT, int KW);
KernelFn mfmt_for_epi9(int MT, int NT, int KW);
KernelFn mfmt_for_epi10(int MT, int NT, int KW);
KernelFn mfmt_for_epi11(int MT, int NT, int KW);
KernelFn mfmt_for_epi12(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi0(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi1(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi2(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi3(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi4(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi8(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi9(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi10(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi11(int MT, int NT, int KW);
KernelFn mfmt_grouped_for_epi12(int MT, int NT, int KW);
KernelFn wide_for_epi0(int W, int WN, int NT);
KernelFn wide_for_epi1(int W, int WN, int NT);
KernelFn wide_for_epi2(int W, int WN, int NT);
KernelFn wide_for_epi3(int W, int WN, int NT);
KernelFn wide_for_epi4(int W, int WN, int NT);
KernelFn wide_for_epi8(int W, int WN, int NT);
KernelFn wide_for_epi9(int W, int WN, int NT);
KernelFn wide_for_epi10(int W, int WN, int NT);
KernelFn wide_for_epi12(int W, int WN, int NT);
KernelFn gemv_for_epi0(int MR, int R, int KU);
KernelFn gemv_for_epi1(int MR, int R, int KU);
KernelFn gemv_for_epi2(int MR, int R, int KU);
KernelFn gemv_for_epi3(int MR, int R, int KU);
KernelFn gemv_for_epi4(int MR, int R, int KU);
KernelFn gemv_for_epi5(int MR, int R, int KU);
KernelFn gemv_for_epi6(int MR, int R, int KU);
KernelFn gemv_for_epi7(int MR, int R, int KU);

inline KernelFn mfma_kernel_for(int epi, int MT, int NT, int KU) {
  switch (epi) {
    case EPI_STORE: return mfma_for_epi0(MT, NT, KU);
    case EPI_SWIGLU: return mfma_for_epi1(MT, NT, KU);
    case EPI_ARGMAX: return mfma_for_epi2(MT, NT, KU);
    case EPI_PART: return mfma_for_epi3(MT, NT, KU);
    case EPI_PART_GU: return mfma_for_epi4(MT, NT, KU);
  }
  return nullptr;
}

inline KernelFn mfmt_kernel_for(int epi, int MT, int NT, int KW) {
  switch (epi) {
    case EPI_STORE: return mfmt_for_epi0(MT, NT, KW);
    case EPI_SWIGLU: return mfmt_for_epi1(MT, NT, KW);
    case EPI_ARGMAX: return mfmt_for_epi2(MT, NT, KW);
    case EPI_PART: return mfmt_for_epi3(MT, NT, KW);
    case EPI_PART_GU: return mfmt_for_epi4(MT, NT, KW);
    case EPI_STORE_PRE: return mfmt_for_epi8(MT, NT, KW);
    case EPI_SWIGLU_PRE: return mfmt_for_epi9(MT, NT, KW);
    case EPI_ARGMAX_PRE: return mfmt_for_epi10(MT, NT, KW);
    case EPI_STORE_RESID: return mfmt_for_epi11(MT, NT, KW);
    case EPI_PART_RESID: return mfmt_for_epi12(MT, NT, KW);
  }
  return nullptr;
}

// Row-group entry points (sk_config::groups > 1); nullptr where none is built.
inline KernelFn mfmt_grouped_kernel_for(int epi, int MT, int NT, int KW) {
  switch (epi) {
    case EPI_STORE: return mfmt_grouped_for_epi0(MT, NT, KW);
    case EPI_SWIGLU: return mfmt_grouped_for_epi1(MT, NT, KW);
    case EPI_ARGMAX: return mfmt_grouped_for_epi2(MT, NT, KW);
    case EPI_PART: return mfmt_grouped_for_epi3(MT, NT, KW);
    case EPI_PART_GU: return mfmt_grouped_for_epi4(MT, NT, KW);
    case EPI_STORE_PRE: return mfmt_grouped_for_epi8(MT, NT, KW);
    case EPI_SWIGLU_PRE: return mfmt_grouped_for_epi9(MT, NT, KW);
    case EPI_ARGMAX_PRE: return mfmt_grouped_for_epi10(MT, NT, KW);
    case EPI_STORE_RESID: return mfmt_grouped_for_epi11(MT, NT, KW);
    case EPI_PART_RESID: return mfmt_grouped_for_epi12(MT, NT, KW);
  }
  return nullptr;
}

// Wide-M instances: W waves (4 or 8) in WN groups along the tile's weight
// slabs, NT 16-row weight slabs per tile.
inline KernelFn wide_kernel_for(int epi, int W, int WN, int NT) {
  switch (epi) {
    case EPI_STORE: return wide_for_epi0(W, WN, NT);
    case EPI_SWIGLU: return wide_for_epi1(W, WN, NT);
    case EPI_ARGMAX: return wide_for_epi2(W, WN, NT);
    case EPI_PART: return wide_for_epi3(W, WN, NT);
    case EPI_PART_GU: return wide_for_epi4(W, WN, NT);
    case EPI_STORE_PRE: return wide_for_epi8(W, WN, NT);
    case EPI_SWIGLU_PRE: return wide_for_epi9(W, WN, NT);
    case EPI_ARGMAX_PRE: return wide_for_epi10(W, WN, NT);
    case EPI_PART_RESID: return wide_for_epi12(W, WN, NT);
  }
  return nullptr;
}

inline KernelFn gemv_kernel_for(int epi, int MR, int R, int KU) {
  switch (epi) {
    case EPI_STORE: return gemv_for_epi0(MR, R, KU);
    case EPI_SWIGLU: return gemv_for_epi1(MR, R, KU);
    case EPI_ARGMAX: return gemv_for_epi2(MR, R, KU);
    case EPI_PART: return gemv_for_epi3(MR, R, KU);
    case EPI_PART_GU: return gemv_for_epi4(MR, R, KU);
    case EPI_STORE_NORM: return gemv_for_epi5(MR, R, KU);
    case EPI_SWIGLU_NORM: return gemv_for_epi6(MR, R, KU);
    case EPI_ARGMAX_NORM: return gemv_for_epi7(MR, R, KU);
  }
  return nullptr;
}

}  // namespace sk
