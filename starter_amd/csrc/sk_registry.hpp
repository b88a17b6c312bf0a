// sk_registry.hpp - lookup of the compiled kernel instances.
//
// The MFMA and GEMV kernel templates are instantiated for a fixed set of
// (row tiles, K-unit bound) pairs per epilogue, one translation unit per
// epilogue (sk_inst_mfma.hip / sk_inst_gemv.hip built with -DSK_EPI=<n>).
// The host planner asks for the smallest instantiated K-unit bound that covers
// a wave's K range; a nullptr answer means "no such instance" and the config
// is rejected with SK_ERR_CONFIG.
#pragma once

#include "sk_kernels.hpp"

namespace sk {

typedef void (*KernelFn)(Args);

// K-unit bounds compiled for each path (ascending).
constexpr int kMfmaKU[] = {5, 8, 10, 16, 20};
constexpr int kGemvKU[] = {2, 5, 8, 10};

// Register estimate (VGPR + AGPR per lane) of an instance; decides the
// largest workgroup the instance is compiled for (__launch_bounds__).
constexpr int mfma_regs(int MT, int NT, int KU) { return 4 * KU * (MT + NT) + 4 * NT * MT + 24; }
constexpr int gemv_regs(int MR, int RR, int KU) { return 4 * KU * (MR + RR) + RR * MR + 24; }
// LDS-transposed MFMA: KW/32 activation units per tile row block plus the
// staged weight rows (KW/512 rows per load instruction).
constexpr int mfmt_regs(int MT, int NT, int KW) { return 4 * (KW / 32) * MT + 4 * (16 * NT * KW / 512) + 4 * NT * MT + 32; }
constexpr int max_waves_for_regs(int regs) { return regs <= 128 ? 16 : (regs <= 256 ? 8 : 4); }

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
KernelFn gemv_for_epi0(int MR, int R, int KU);
KernelFn gemv_for_epi1(int MR, int R, int KU);
KernelFn gemv_for_epi2(int MR, int R, int KU);
KernelFn gemv_for_epi3(int MR, int R, int KU);
KernelFn gemv_for_epi4(int MR, int R, int KU);

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
  }
  return nullptr;
}

}  // namespace sk
