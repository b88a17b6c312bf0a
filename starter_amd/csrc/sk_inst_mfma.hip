// MFMA kernel instances for one epilogue (built once per -DSK_EPI=<0..4>).
#include "sk_registry.hpp"

#ifndef SK_EPI
#error "build with -DSK_EPI=<epilogue id>"
#endif

#define SK_CAT2(a, b) a##b
#define SK_CAT(a, b) SK_CAT2(a, b)

namespace sk {

template <int MT, int NT, int KU, int EPI>
__global__ void __launch_bounds__(64 * instance_waves(KIND_MFMA, MT, NT, KU, EPI))
mfma_entry(Args p) {
  mfma_body<MT, NT, KU, EPI>(p);
}

// An instance with no spill-free tier is not instantiated.
template <int MT, int NT, int KU, int EPI>
KernelFn mfma_ptr() {
  if constexpr (instance_waves(KIND_MFMA, MT, NT, KU, EPI) > 0) return &mfma_entry<MT, NT, KU, EPI>;
  else return nullptr;
}

#define SK_C(MT, NT, KU) \
  case MT * 10000 + NT * 100 + KU: return mfma_ptr<MT, NT, KU, SK_EPI>();
#define SK_LIST(NT) \
  SK_C(1, NT, 5) SK_C(1, NT, 8) SK_C(1, NT, 10) SK_C(1, NT, 16) SK_C(1, NT, 20) \
  SK_C(2, NT, 5) SK_C(2, NT, 8) SK_C(2, NT, 10) SK_C(2, NT, 16) \
  SK_C(3, NT, 5) SK_C(3, NT, 8) SK_C(3, NT, 10) SK_C(3, NT, 20) \
  SK_C(4, NT, 5) SK_C(4, NT, 8) SK_C(4, NT, 10) SK_C(4, NT, 20)

KernelFn SK_CAT(mfma_for_epi, SK_EPI)(int MT, int NT, int KU) {
  switch (MT * 10000 + NT * 100 + KU) {
#if SK_EPI == 1 || SK_EPI == 4   // gate/up: 16 gate rows + 16 up rows
    SK_LIST(2)
#elif SK_EPI == 3                // split-K partials
    SK_LIST(1)
#else                            // store / argmax
    SK_LIST(1)
    SK_LIST(2)
#endif
    default: break;
  }
  return nullptr;
}

}  // namespace sk
