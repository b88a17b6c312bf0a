// GEMV (VALU dot2) kernel instances for one epilogue (-DSK_EPI=<0..7>).
#include "sk_registry.hpp"

#ifndef SK_EPI
#error "build with -DSK_EPI=<epilogue id>"
#endif

#define SK_CAT2(a, b) a##b
#define SK_CAT(a, b) SK_CAT2(a, b)

namespace sk {

template <int MR, int R, int KU, int EPI>
__global__ void __launch_bounds__(64 * instance_waves(KIND_GEMV, MR, R, KU, EPI))
gemv_entry(Args p) {
  gemv_body<MR, R, KU, EPI>(p);
}

// An instance with no spill-free tier is not instantiated.
template <int MR, int R, int KU, int EPI>
KernelFn gemv_ptr() {
  if constexpr (instance_waves(KIND_GEMV, MR, R, KU, EPI) > 0) return &gemv_entry<MR, R, KU, EPI>;
  else return nullptr;
}

#define SK_C(MR, R, KU) \
  case MR * 10000 + R * 100 + KU: return gemv_ptr<MR, R, KU, SK_EPI>();
#define SK_R(MR, R) SK_C(MR, R, 2) SK_C(MR, R, 5) SK_C(MR, R, 8) SK_C(MR, R, 10)
#define SK_MR(MR) SK_R(MR, 2) SK_R(MR, 4) SK_R(MR, 8)

KernelFn SK_CAT(gemv_for_epi, SK_EPI)(int MR, int R, int KU) {
  switch (MR * 10000 + R * 100 + KU) {
    SK_MR(1) SK_MR(2) SK_MR(4) SK_MR(8)
    default: break;
  }
  return nullptr;
}

}  // namespace sk
