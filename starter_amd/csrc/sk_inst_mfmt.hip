// LDS-transposed MFMA kernel instances for one epilogue (-DSK_EPI=<0..4, 8..12>).
#include "sk_registry.hpp"

#ifndef SK_EPI
#error "build with -DSK_EPI=<epilogue id>"
#endif

#define SK_CAT2(a, b) a##b
#define SK_CAT(a, b) SK_CAT2(a, b)

namespace sk {

template <int MT, int NT, int KW, int EPI>
__global__ void __launch_bounds__(64 * instance_waves(KIND_MFMT, MT, NT, KW, EPI))
mfmt_entry(Args p) {
  mfmt_body<MT, NT, KW, EPI>(p);
}

// Row-group entry points: the same body behind the group decode, compiled for
// the register tier of the plain instance (the decode uses scalar registers).
template <int MT, int NT, int KW, int EPI>
__global__ void __launch_bounds__(64 * instance_waves(KIND_MFMT, MT, NT, KW, EPI))
mfmt_grouped_entry(Args p) {
  mfmt_grouped_body<MT, NT, KW, EPI>(p);
}

// An instance with no spill-free tier is not instantiated.
template <int MT, int NT, int KW, int EPI>
KernelFn mfmt_ptr() {
  if constexpr (instance_waves(KIND_MFMT, MT, NT, KW, EPI) > 0) return &mfmt_entry<MT, NT, KW, EPI>;
  else return nullptr;
}
template <int MT, int NT, int KW, int EPI>
KernelFn mfmt_grouped_ptr() {
  if constexpr (instance_waves(KIND_MFMT, MT, NT, KW, EPI) > 0) return &mfmt_grouped_entry<MT, NT, KW, EPI>;
  else return nullptr;
}

#define SK_C(MT, NT, KW) \
  case MT * 100000 + NT * 1000 + KW: return mfmt_ptr<MT, NT, KW, SK_EPI>();
#define SK_LIST(NT) \
  SK_C(1, NT, 512) SK_C(2, NT, 512) SK_C(1, NT, 256) SK_C(2, NT, 256) SK_C(3, NT, 256) SK_C(4, NT, 256) \
  SK_C(1, NT, 1024) SK_C(2, NT, 1024) SK_C(3, NT, 1024) SK_C(4, NT, 1024)
// Five 256-column chunks per wave (up to 32 rows): K = 9728 in eight waves
// without a global split.
#define SK_LONG_LIST(NT) SK_C(1, NT, 1280) SK_C(2, NT, 1280)

// Gate/up tiles taller than 16 rows (ring path, up to 32 rows of activations):
// two or three 16-row slabs of gate rows and as many of up rows, for tile
// heights such as 38 = 9728 / 256 that give every CU one tile.
#define SK_TALL_GU_LIST \
  SK_C(1, 4, 256) SK_C(2, 4, 256) SK_C(1, 6, 256) SK_C(2, 6, 256)

// Residual hand-off epilogues exist on the ring path only: the consumers
// (EPI 8-10) with one 256-column chunk per wave, the producers (EPI 11-12)
// with one or four.
#define SK_PRE_LIST(NT) SK_C(1, NT, 256) SK_C(2, NT, 256)
#define SK_RESID_LIST(NT) \
  SK_C(1, NT, 256) SK_C(2, NT, 256) SK_C(1, NT, 1024) SK_C(2, NT, 1024) SK_C(1, NT, 1280) SK_C(2, NT, 1280)

// Row groups: groups of up to 32 rows on the ring path, for the plain
// projections and the residual hand-off producers (256- and 1024-column
// waves) and consumers (256-column waves).
#define SK_G(MT, NT, KW) \
  case MT * 100000 + NT * 1000 + KW: return mfmt_grouped_ptr<MT, NT, KW, SK_EPI>();
#define SK_GROUP_LIST(NT) SK_G(1, NT, 256) SK_G(2, NT, 256) SK_G(1, NT, 1024) SK_G(2, NT, 1024)
#define SK_GROUP_PRE_LIST(NT) SK_G(1, NT, 256) SK_G(2, NT, 256)

KernelFn SK_CAT(mfmt_grouped_for_epi, SK_EPI)(int MT, int NT, int KW) {
  switch (MT * 100000 + NT * 1000 + KW) {
#if SK_EPI == 9
    SK_GROUP_PRE_LIST(2)
#elif SK_EPI == 8 || SK_EPI == 10
    SK_GROUP_PRE_LIST(1)
    SK_GROUP_PRE_LIST(2)
#elif SK_EPI == 1 || SK_EPI == 4
    SK_GROUP_LIST(2)
#else
    SK_GROUP_LIST(1)
    SK_GROUP_LIST(2)
#endif
    default: break;
  }
  return nullptr;
}

KernelFn SK_CAT(mfmt_for_epi, SK_EPI)(int MT, int NT, int KW) {
  switch (MT * 100000 + NT * 1000 + KW) {
#if SK_EPI == 9   // gate/up consumer
    SK_PRE_LIST(2)
#elif SK_EPI == 8 || SK_EPI == 10
    SK_PRE_LIST(1)
    SK_PRE_LIST(2)
#elif SK_EPI == 11 || SK_EPI == 12
    SK_RESID_LIST(1)
    SK_RESID_LIST(2)
#elif SK_EPI == 1 || SK_EPI == 4   // gate/up: NT/2 slabs of gate rows + NT/2 of up rows
    SK_LIST(2)
    SK_TALL_GU_LIST
#else
    SK_LIST(1)
    SK_LIST(2)
#if SK_EPI == 0 || SK_EPI == 3
    SK_LONG_LIST(1)
    SK_LONG_LIST(2)
#endif
#endif
    default: break;
  }
  return nullptr;
}

}  // namespace sk
