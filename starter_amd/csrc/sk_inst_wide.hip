// Wide-M kernel instances (sk_wide.hpp, sk_wide2.hpp) for one epilogue
// (-DSK_EPI=<0..4, 8..10, 12>).
#include "sk_registry.hpp"

#ifndef SK_EPI
#error "build with -DSK_EPI=<epilogue id>"
#endif

#define SK_CAT2(a, b) a##b
#define SK_CAT(a, b) SK_CAT2(a, b)

namespace sk {

template <int W, int WN, int NT, int EPI>
__global__ void __launch_bounds__(64 * W) wide_entry(Args p) {
  wide_body<W, WN, NT, EPI>(p);
}

// Both operands staged in LDS (sk_wide2.hpp): four or eight waves, keyed as
// WN = 4.
template <int W, int NT, int EPI>
__global__ void __launch_bounds__(64 * W) wide2_entry(Args p) {
  wide2_body<W, NT, EPI>(p);
}

#define SK_W(W, WN, NT) \
  case W * 1000 + WN * 100 + NT: return &wide_entry<W, WN, NT, SK_EPI>;
#define SK_W2(W, NT) \
  case W * 1000 + 4 * 100 + NT: return &wide2_entry<W, NT, SK_EPI>;

// (W waves, WN groups of them along the tile's weight slabs, NT slabs; W = 4,
// WN = 4: the two-operand body)
KernelFn SK_CAT(wide_for_epi, SK_EPI)(int W, int WN, int NT) {
  switch (W * 1000 + WN * 100 + NT) {
#if SK_EPI == 8   // residual hand-off (two-operand body only): consumers, then the producer
    SK_W2(8, 2) SK_W2(8, 4) SK_W2(8, 6)
#elif SK_EPI == 9
    SK_W2(8, 4) SK_W2(8, 6)
#elif SK_EPI == 10
    SK_W2(8, 6) SK_W2(8, 8)
#elif SK_EPI == 12
    SK_W2(8, 2) SK_W2(8, 4)
#elif SK_EPI == 1 || SK_EPI == 4   // gate/up: NT/2 gate slabs + NT/2 up slabs
    SK_W(4, 1, 2) SK_W(4, 1, 4) SK_W(4, 1, 6)
    SK_W(8, 1, 2) SK_W(8, 1, 4) SK_W(8, 1, 6)
    SK_W(8, 2, 4)
    SK_W2(4, 4) SK_W2(4, 6) SK_W2(4, 8) SK_W2(8, 4) SK_W2(8, 6)
#else
    SK_W(4, 1, 2) SK_W(4, 1, 3) SK_W(4, 1, 4) SK_W(4, 1, 5) SK_W(4, 1, 6)
    SK_W(8, 1, 2) SK_W(8, 1, 3) SK_W(8, 1, 4) SK_W(8, 1, 5) SK_W(8, 1, 6)
    SK_W(8, 2, 2) SK_W(8, 2, 4) SK_W(8, 2, 6)
    SK_W2(4, 2) SK_W2(4, 3) SK_W2(4, 4) SK_W2(4, 5) SK_W2(4, 6) SK_W2(4, 8)
    SK_W2(8, 2) SK_W2(8, 4) SK_W2(8, 6) SK_W2(8, 8)
#endif
    default: break;
  }
  return nullptr;
}

}  // namespace sk
